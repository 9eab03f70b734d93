// gemm_tile.h -- the shared MFMA GEMM skeleton of libtkv_hip (gfx950).
//
// C[M,N] = A[M,K] . W[N,K]^T with both operands K-major bytes (int8 codes or
// e4m3 bytes), as the reference's GEMMs index them (matmul.tkv:22,51).
//
// Data movement (per 256- or 512-thread workgroup owning a BM x BN tile):
//  * K advances in BK-byte slices.  Each slice of A (BM rows) and W (BN rows)
//    is copied HBM/L2 -> LDS with global_load_lds_dwordx4 (gfx950 direct-to-
//    LDS DMA, 1 KB per wave instruction, no VGPR staging), into a ring of
//    STAGES slices, so STAGES-1 slices are in flight while MFMA consumes one.
//  * LDS rows hold BK bytes in 16-byte chunks whose position is XOR-swizzled
//    by row: any 16 consecutive rows reading the same logical chunk hit
//    distinct bank groups of gfx950's 64-bank LDS (ds_read_b128 conflict free).
//    The DMA destination is linear per wave, so the swizzle is applied by
//    choosing which global chunk each lane fetches.
//  * Waves are laid out WM x WN; each owns a (BM/WM) x (BN/WN) tile of 32x32
//    MFMA blocks whose fragments are read from LDS.
//  * Workgroups are re-ordered so that each of the 8 XCDs (which take
//    workgroups round-robin) owns a contiguous range of output tiles in
//    row-major tile order: tiles sharing A rows / W columns run on the same
//    XCD and hit its 4 MB L2 instead of re-reading HBM.
// K must be a multiple of BK (launchers pad); rows past M / N are clamped to
// the last valid row when loading and never stored.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tkv {
namespace gemm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr;

template <int BM_, int BN_, int WM_, int WN_, int BK_, int STAGES_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = BK_, STAGES = STAGES_;
    static constexpr int WAVES = WM * WN;
    static constexpr int THREADS = WAVES * 64;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int TM = WTM / 32, TN = WTN / 32;
    static constexpr int CH = BK / 16;            // 16-byte chunks per LDS row
    static constexpr int ROWS_PER_DMA = 64 / CH;  // rows covered by one 1 KB wave DMA
    static constexpr int A_DMA_W = BM / ROWS_PER_DMA / WAVES;
    static constexpr int W_DMA_W = BN / ROWS_PER_DMA / WAVES;
    static constexpr int LPS = A_DMA_W + W_DMA_W;  // DMA instructions per wave per slice
    static constexpr int A_BYTES = BM * BK, W_BYTES = BN * BK;
    static constexpr int STAGE_BYTES = A_BYTES + W_BYTES;
    static constexpr int LDS_BYTES = STAGE_BYTES * STAGES;
    static constexpr int FRAG_DEPTH = BK / 32;  // k-steps of fragments read ahead (all)
    static constexpr int DEFER = 0;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32x32 blocks");
    static_assert(BM % (ROWS_PER_DMA * WAVES) == 0 && BN % (ROWS_PER_DMA * WAVES) == 0,
                  "tile rows must split evenly over wave DMAs");
    static_assert(LDS_BYTES <= 163840, "LDS capacity of a gfx950 workgroup");
    static_assert(LPS * (STAGES - 1) <= 63, "vmcnt range");
};

// Warp-specialised variant: CW = WM x WN consumer waves read LDS, run the
// MFMAs and the epilogue; PW producer waves only issue the operand DMA.
// vmcnt is per wave and retires in issue order, so when one wave issued both
// DMA and output stores, every wait for the next slice also waited for the
// stores issued before it.  With the roles split, the consumers' stores
// drain while the producers keep the ring full, and no consumer ever waits on
// vmcnt for operand data.
template <int BM_, int BN_, int WM_, int WN_, int BK_, int STAGES_, int PW_, int DEFER_ = 0,
          int FD_ = 0, int OCC_ = 1>
struct CfgWS {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = BK_, STAGES = STAGES_;
    static constexpr int CW = WM * WN, PW = PW_;
    static constexpr int WAVES = CW + PW;
    static constexpr int THREADS = WAVES * 64;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int TM = WTM / 32, TN = WTN / 32;
    static constexpr int CH = BK / 16;
    static constexpr int ROWS_PER_DMA = 64 / CH;
    static constexpr int A_BLK = BM / ROWS_PER_DMA, W_BLK = BN / ROWS_PER_DMA;
    static constexpr int LPS = (A_BLK + W_BLK) / PW;  // DMA instructions per producer wave per slice
    static constexpr int A_BYTES = BM * BK, W_BYTES = BN * BK;
    static constexpr int STAGE_BYTES = A_BYTES + W_BYTES;
    static constexpr int LDS_BYTES = STAGE_BYTES * STAGES;
    // DEFER: a tile's output values are stored during the next tile's K
    // slices (spread evenly over them) instead of between tiles; the values
    // wait in registers, paid for by reading fragments fewer k-steps ahead.
    // FD (fragment depth, k-steps read ahead; 0 = automatic) trades registers
    // for LDS latency hiding.
    static constexpr int DEFER = DEFER_;
    static constexpr int FRAG_DEPTH = FD_ ? FD_ : (DEFER ? 2 : BK / 32);
    // OCC workgroups resident per CU: the register budget is set for
    // OCC * WAVES waves over the 4 SIMDs, so that while one workgroup's
    // consumers wait on their output stores the other's run MFMAs.
    static constexpr int OCC = OCC_;
    static constexpr int MIN_WAVES_EU = (OCC * WAVES + 3) / 4;
    static_assert(OCC * LDS_BYTES <= 163840, "OCC workgroups must fit the CU's LDS");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32x32 blocks");
    static_assert(BM % ROWS_PER_DMA == 0 && BN % ROWS_PER_DMA == 0, "rows per DMA block");
    static_assert((A_BLK + W_BLK) % PW == 0, "DMA blocks must split evenly over producers");
    static_assert(LDS_BYTES <= 163840, "LDS capacity of a gfx950 workgroup");
    static_assert(STAGES >= 2 && LPS * (STAGES - 1) <= 63, "vmcnt range");
};

// Chunk swizzle for 64 banks: rows r..r+15 at the same logical chunk map to 16
// distinct (row parity / quad, chunk) bank groups.
template <int CH>
__device__ __forceinline__ int swz(int row) {
    return (row / (16 / CH)) % CH;
}

// s_waitcnt vmcnt(N) leaving lgkmcnt / expcnt alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup barrier without the workgroup-scope memory fence of
// __syncthreads (which would drain every outstanding DMA with vmcnt(0)).
// s_barrier itself does not wait for memory operations: lgkmcnt(0) first
// makes this wave's LDS reads complete, so a slot released by the barrier is
// no longer being read when a producer's DMA refills it.  The "memory"
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Index of the calling wave in its workgroup, as a wave-uniform (scalar)
// value: tile offsets derived from it stay in SGPRs.
__device__ __forceinline__ int wave_id() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Tile order: contiguous tile ranges per XCD (workgroups are dispatched to
// XCDs round-robin by workgroup id).
__device__ __forceinline__ int xcd_tile(int b, int total) {
    constexpr int X = 8;
    const int per = total / X, rem = total % X;
    const int xcd = b % X, j = b / X;
    return xcd < rem ? xcd * (per + 1) + j : rem * (per + 1) + (xcd - rem) * per + j;
}

// Issue the DMA copies of slice `k0` into ring slot `smem`.
template <class C>
__device__ __forceinline__ void issue_slice(const uint8_t* __restrict__ A,
                                            const uint8_t* __restrict__ W, int M, int N, int ldk,
                                            int m0, int n0, int k0, uint8_t* smem, int wave,
                                            int lane) {
    const int lrow = lane / C::CH, lch = lane % C::CH;
#pragma unroll
    for (int d = 0; d < C::A_DMA_W; d++) {
        const int blk = wave * C::A_DMA_W + d;
        const int row = blk * C::ROWS_PER_DMA + lrow;
        const int c = lch ^ swz<C::CH>(row);
        const int gr = m0 + row < M ? m0 + row : M - 1;
        const uint8_t* g = A + (int64_t)gr * ldk + k0 + c * 16;
        __builtin_amdgcn_global_load_lds((const void*)g, (lds_ptr)(smem + blk * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int d = 0; d < C::W_DMA_W; d++) {
        const int blk = wave * C::W_DMA_W + d;
        const int row = blk * C::ROWS_PER_DMA + lrow;
        const int c = lch ^ swz<C::CH>(row);
        const int gr = n0 + row < N ? n0 + row : N - 1;
        const uint8_t* g = W + (int64_t)gr * ldk + k0 + c * 16;
        __builtin_amdgcn_global_load_lds((const void*)g,
                                         (lds_ptr)(smem + C::A_BYTES + blk * 1024), 16, 0, 0);
    }
}

// Producer wave `pw` of a CfgWS workgroup owns DMA blocks d * PW + pw
// (d < LPS) of every slice; block b fills LDS bytes [b * 1024, b * 1024 +
// 1024) of the slot, A blocks first.  WsLane holds, for the current tile, the
// lane's byte offset of each block relative to the tile's first A or W row
// (32-bit: below 256 * 2^17), so issuing a slice costs one scalar base and no
// per-lane address arithmetic.
template <class C>
struct WsLane {
    uint32_t off[C::LPS];
};

template <class C>
__device__ __forceinline__ void ws_lane_offsets(int M, int N, int ldk, int m0, int n0, int pw,
                                                int lane, WsLane<C>& L) {
    const int lrow = lane / C::CH, lch = lane % C::CH;
#pragma unroll
    for (int d = 0; d < C::LPS; d++) {
        const int blk = d * C::PW + pw;
        const bool is_a = blk < C::A_BLK;
        const int row = (is_a ? blk : blk - C::A_BLK) * C::ROWS_PER_DMA + lrow;
        const int c = lch ^ swz<C::CH>(row);
        const int lim = is_a ? M - 1 - m0 : N - 1 - n0;  // rows past the matrix read its last row
        L.off[d] = (uint32_t)(row < lim ? row : lim) * (uint32_t)ldk + (uint32_t)(c * 16);
    }
}

template <class C>
__device__ __forceinline__ void ws_issue(const uint8_t* __restrict__ a_tile,
                                         const uint8_t* __restrict__ w_tile, int k0,
                                         const WsLane<C>& L, uint8_t* slot, int pw) {
#pragma unroll
    for (int d = 0; d < C::LPS; d++) {
        const int blk = d * C::PW + pw;
        const bool is_a = blk < C::A_BLK;
        const uint8_t* base = (is_a ? a_tile : w_tile) + k0;
        uint8_t* dst = slot + (is_a ? blk * 1024 : C::A_BYTES + (blk - C::A_BLK) * 1024);
        __builtin_amdgcn_global_load_lds((const void*)(base + L.off[d]), (lds_ptr)dst, 16, 0, 0);
    }
}

// s_waitcnt vmcnt(n) for a wave-uniform run-time n in [0, 63].
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
    switch (n) {
#define TKV_W(i) case i: wait_vmcnt<i>(); break;
#define TKV_W8(i) TKV_W(i) TKV_W(i + 1) TKV_W(i + 2) TKV_W(i + 3) TKV_W(i + 4) TKV_W(i + 5) \
    TKV_W(i + 6) TKV_W(i + 7)
        TKV_W8(0) TKV_W8(8) TKV_W8(16) TKV_W8(24) TKV_W8(32) TKV_W8(40) TKV_W8(48) TKV_W8(56)
#undef TKV_W8
#undef TKV_W
        default: wait_vmcnt<0>(); break;
    }
}

template <class C>
__device__ __forceinline__ v4i lds_chunk(const uint8_t* base, int row, int ch) {
    return *reinterpret_cast<const v4i*>(base + row * C::BK + ((ch ^ swz<C::CH>(row)) << 4));
}

// Wait until slice `kt` has landed, given how many slices were issued after it.
template <class C, int AHEAD = C::STAGES - 1>
__device__ __forceinline__ void wait_slice(int ahead) {
    if constexpr (AHEAD == 0) {
        wait_vmcnt<0>();
    } else {
        if (ahead >= AHEAD)
            wait_vmcnt<AHEAD * C::LPS>();
        else
            wait_slice<C, AHEAD - 1>(ahead);
    }
}

// Issue the first STAGES-1 slices of a tile (ring slots 0..STAGES-2).
template <class C>
__device__ __forceinline__ void prologue(const uint8_t* __restrict__ A,
                                         const uint8_t* __restrict__ W, int M, int N, int ldk,
                                         int m0, int n0, uint8_t* smem) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nk = ldk / C::BK;
#pragma unroll
    for (int s = 0; s < C::STAGES - 1; s++)
        if (s < nk)
            issue_slice<C>(A, W, M, N, ldk, m0, n0, s * C::BK, smem + s * C::STAGE_BYTES, wave,
                           lane);
}

// Main loop over all K slices of one tile whose prologue has been issued:
// accumulates the wave's TM x TN blocks of 32x32.  One barrier per slice:
// the barrier that publishes slice kt+1 (every wave has waited for its own
// DMAs of it) also certifies that every wave is done reading slice kt, whose
// ring slot the next iteration refills.  Ends right after the last slice's
// MFMAs, with no DMA outstanding.
template <class C, class P>
__device__ __forceinline__ void mainloop(const uint8_t* __restrict__ A,
                                         const uint8_t* __restrict__ W, int M, int N, int ldk,
                                         int m0, int n0, uint8_t* smem,
                                         typename P::Acc (&acc)[C::TM][C::TN]) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int wm = wave / C::WN, wn = wave % C::WN;
    const int nk = ldk / C::BK;
    int a_row[C::TM], w_row[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++) a_row[i] = wm * C::WTM + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < C::TN; j++) w_row[j] = wn * C::WTN + j * 32 + (lane & 31);
    const int khalf = lane >> 5;

    // slice 0 landed (own DMAs) and published (barrier)
    wait_slice<C>((C::STAGES - 2) < (nk - 1) ? (C::STAGES - 2) : (nk - 1));
    barrier();
    for (int kt = 0; kt < nk; kt++) {
        // refill the slot of slice kt-1 (retired by the barrier above)
        const int nxt = kt + C::STAGES - 1;
        if (nxt < nk)
            issue_slice<C>(A, W, M, N, ldk, m0, n0, nxt * C::BK,
                           smem + (nxt % C::STAGES) * C::STAGE_BYTES, wave, lane);
        const uint8_t* sa = smem + (kt % C::STAGES) * C::STAGE_BYTES;
        P::template slice<C>(sa, sa + C::A_BYTES, a_row, w_row, khalf, acc);
        if (kt + 1 < nk) {
            // slices issued after kt+1: up to STAGES-2
            const int last = nxt < nk ? nxt : nk - 1;
            wait_slice<C>(last - (kt + 1));
            barrier();
        }
    }
}

// INT8: v_mfma_i32_32x32x32_i8, 16 K-bytes per lane per 32-K step.
struct PolicyI8 {
    typedef v16i Acc;
    __device__ __forceinline__ static Acc mfma(const v4i& a, const v4i& b, const Acc& c) {
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
    }
    __device__ __forceinline__ static void zero(Acc& a) {
#pragma unroll
        for (int r = 0; r < 16; r++) a[r] = 0;
    }
    // Fragments are read C::FRAG_DEPTH k-steps ahead of the MFMAs that use
    // them, with scheduling barriers between the groups: ds_read returns in
    // order, so each MFMA waits only for its own operands (lgkmcnt(n), n =
    // reads issued after them) while later reads overlap earlier MFMAs.
    // Without the barriers the scheduler sinks every read down to its use and
    // exposes the LDS latency before each MFMA.
    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
        constexpr int KS = C::BK / 32, D = C::FRAG_DEPTH;
        v4i af[KS][C::TM], bf[KS][C::TN];
        auto load = [&](int ks) {
            const int ch = ks * 2 + khalf;
#pragma unroll
            for (int i = 0; i < C::TM; i++) af[ks][i] = lds_chunk<C>(sa, a_row[i], ch);
#pragma unroll
            for (int j = 0; j < C::TN; j++) bf[ks][j] = lds_chunk<C>(sw, w_row[j], ch);
        };
#pragma unroll
        for (int ks = 0; ks < D - 1 && ks < KS; ks++) load(ks);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks + D - 1 < KS) load(ks + D - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks][i], bf[ks][j],
                                                                      acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// PolicyI8 plus the operands' row sums, for QLinearMatMul's zero-point
// corrections: every consumer wave adds the bytes of the A and W fragments it
// holds anyway (v_dot4_i32_i8 against 0x01010101, exact) into per-lane
// partial sums.  acc[i][0].rs: lane l's row a_row[i] (l % 32) over k-half
// l / 32; acc[0][j].cs: likewise for column w_row[j].  Waves sharing rows or
// columns repeat the sums, which keeps every wave's epilogue self-contained.
struct AccQ {
    v16i v;
    int rs, cs;
};

__device__ __forceinline__ int byte_sum4(const v4i& f, int s) {
    s = __builtin_amdgcn_sdot4(f.x, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(f.y, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(f.z, 0x01010101, s, false);
    return __builtin_amdgcn_sdot4(f.w, 0x01010101, s, false);
}

struct PolicyI8Q {
    typedef AccQ Acc;
    __device__ __forceinline__ static Acc mfma(const v4i& a, const v4i& b, const Acc& c) {
        Acc r = c;
        r.v = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c.v, 0, 0, 0);
        return r;
    }
    __device__ __forceinline__ static void zero(Acc& a) {
#pragma unroll
        for (int r = 0; r < 16; r++) a.v[r] = 0;
        a.rs = 0;
        a.cs = 0;
    }
    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
        constexpr int KS = C::BK / 32, D = C::FRAG_DEPTH;
        v4i af[KS][C::TM], bf[KS][C::TN];
        auto load = [&](int ks) {
            const int ch = ks * 2 + khalf;
#pragma unroll
            for (int i = 0; i < C::TM; i++) af[ks][i] = lds_chunk<C>(sa, a_row[i], ch);
#pragma unroll
            for (int j = 0; j < C::TN; j++) bf[ks][j] = lds_chunk<C>(sw, w_row[j], ch);
        };
#pragma unroll
        for (int ks = 0; ks < D - 1 && ks < KS; ks++) load(ks);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks + D - 1 < KS) load(ks + D - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j].v = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks][i], bf[ks][j],
                                                                        acc[i][j].v, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < C::TM; i++) acc[i][0].rs = byte_sum4(af[ks][i], acc[i][0].rs);
#pragma unroll
            for (int j = 0; j < C::TN; j++) acc[0][j].cs = byte_sum4(bf[ks][j], acc[0][j].cs);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// PolicyI8Q with the sums split over the waves that share them, for the
// warp-specialised kernel: wave (wm, wn) adds the A fragment bytes of the
// k-steps with ks % WN == wn and the W fragment bytes of those with
// ks % WM == wm, so every byte of a slice is summed once per workgroup
// instead of WN (A) or WM (W) times (20 dot4 per slice and wave instead of 64
// with cfg 2).  After a tile's last slice each wave stores its partial sums
// in LDS (publish, before that slice's barrier); after the barrier every wave
// adds the partials of its rows and columns (gather), which leaves
// acc[i][0].rs / acc[0][j].cs in PolicyI8Q's form (a lane's value plus that
// of lane ^ 32 is the full sum).  Two LDS areas alternate by tile: tile t's
// area is written again only at tile t + 2's last slice, which a wave reaches
// only after every wave has passed tile t + 1's barriers, i.e. has finished
// reading tile t's sums.
struct PolicyI8QS : PolicyI8Q {
    template <class C>
    static constexpr int share_ints() { return C::BM * C::WN + C::BN * C::WM; }

    template <class C>
    __device__ __forceinline__ static int32_t* share_area() {
        __shared__ __attribute__((aligned(16))) int32_t s_share[2 * share_ints<C>()];
        return s_share;
    }

    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
        constexpr int KS = C::BK / 32, D = C::FRAG_DEPTH;
        const int wave = wave_id();
        const int wm = wave / C::WN, wn = wave % C::WN;
        v4i af[KS][C::TM], bf[KS][C::TN];
        auto load = [&](int ks) {
            const int ch = ks * 2 + khalf;
#pragma unroll
            for (int i = 0; i < C::TM; i++) af[ks][i] = lds_chunk<C>(sa, a_row[i], ch);
#pragma unroll
            for (int j = 0; j < C::TN; j++) bf[ks][j] = lds_chunk<C>(sw, w_row[j], ch);
        };
#pragma unroll
        for (int ks = 0; ks < D - 1 && ks < KS; ks++) load(ks);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks + D - 1 < KS) load(ks + D - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j].v = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks][i], bf[ks][j],
                                                                        acc[i][j].v, 0, 0, 0);
            if (ks % C::WN == wn) {
#pragma unroll
                for (int i = 0; i < C::TM; i++) acc[i][0].rs = byte_sum4(af[ks][i], acc[i][0].rs);
            }
            if (ks % C::WM == wm) {
#pragma unroll
                for (int j = 0; j < C::TN; j++) acc[0][j].cs = byte_sum4(bf[ks][j], acc[0][j].cs);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Area `buf`: row sums [WN][BM] (partial over the k-steps of wave column
    // wn), then column sums [WM][BN] (partial over those of wave row wm).
    template <class C>
    __device__ __forceinline__ static void publish(const Acc (&acc)[C::TM][C::TN], int buf) {
        const int lane = threadIdx.x & 63, wave = wave_id();
        const int wm = wave / C::WN, wn = wave % C::WN;
        int32_t* rs = share_area<C>() + buf * share_ints<C>();
        int32_t* cs = rs + C::BM * C::WN;
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int full = acc[i][0].rs + __shfl_xor(acc[i][0].rs, 32, 64);
            if (lane < 32) rs[wn * C::BM + wm * C::WTM + i * 32 + lane] = full;
        }
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int full = acc[0][j].cs + __shfl_xor(acc[0][j].cs, 32, 64);
            if (lane < 32) cs[wm * C::BN + wn * C::WTN + j * 32 + lane] = full;
        }
    }

    template <class C>
    __device__ __forceinline__ static void gather(Acc (&acc)[C::TM][C::TN], int buf) {
        const int lane = threadIdx.x & 63, wave = wave_id();
        const int wm = wave / C::WN, wn = wave % C::WN;
        const int32_t* rs = share_area<C>() + buf * share_ints<C>();
        const int32_t* cs = rs + C::BM * C::WN;
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int row = wm * C::WTM + i * 32 + (lane & 31);
            int t = 0;
#pragma unroll
            for (int w = 0; w < C::WN; w++) t += rs[w * C::BM + row];
            acc[i][0].rs = lane < 32 ? t : 0;
        }
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int col = wn * C::WTN + j * 32 + (lane & 31);
            int t = 0;
#pragma unroll
            for (int w = 0; w < C::WM; w++) t += cs[w * C::BN + col];
            acc[0][j].cs = lane < 32 ? t : 0;
        }
    }
};

template <class P>
struct shares_sums {
    static constexpr bool value = false;
};
template <>
struct shares_sums<PolicyI8QS> {
    static constexpr bool value = true;
};

// FP8 full rate: v_mfma_scale_f32_32x32x64_f8f6f4 (both operands e4m3,
// E8M0 scales 2^0), 32 K-bytes per lane per 64-K step.  Hardware decode is
// OCP e4m3fn and the dot product is accumulated at reduced precision.
struct PolicyF8 {
    typedef v16f Acc;
    __device__ __forceinline__ static void zero(Acc& a) {
#pragma unroll
        for (int r = 0; r < 16; r++) a[r] = 0.0f;
    }
    static constexpr float kAccScale = 1.0f;
    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
        constexpr int KS = C::BK / 64;
        v4i alo[KS][C::TM], ahi[KS][C::TM], blo[KS][C::TN], bhi[KS][C::TN];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int ch = ks * 4 + khalf * 2;
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
                alo[ks][i] = lds_chunk<C>(sa, a_row[i], ch);
                ahi[ks][i] = lds_chunk<C>(sa, a_row[i], ch + 1);
            }
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                blo[ks][j] = lds_chunk<C>(sw, w_row[j], ch);
                bhi[ks][j] = lds_chunk<C>(sw, w_row[j], ch + 1);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            v8i af[C::TM], bf[C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
                const v4i lo = alo[ks][i], hi = ahi[ks][i];
                af[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const v4i lo = blo[ks][j], hi = bhi[ks][j];
                bf[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        af[i], bf[j], acc[i][j], 0, 0, 0, 127, 0, 127);
        }
    }
};

// Reference e4m3 decode (tv/quantization/types.tkv:193-226) of two bytes to
// two f16, pre-scaled by 2^-8 so that every code is exact in f16:
//   f16 bits (b & 0x7F) << 7 encode OCP(b) * 2^-8 for all codes (normals
//   land on f16 normals, e4m3 subnormals on f16 subnormals); the reference's
//   decoder halves subnormals (its normalisation uses exponent 127-bias-n),
//   so those take one more right shift; 0x7F / 0xFF are +-inf in the
//   reference (its exponent-255 branch ignores the mantissa) -> f16 inf.
// Input: the two bytes in bits [7:0] and [23:16].  Products of two decoded
// values carry 2^-16, which the epilogue removes exactly.
__device__ __forceinline__ uint32_t dec2_f16(uint32_t x) {
    const uint32_t mag = x & 0x007F007Fu;
    uint32_t h = mag << 7;
    // 0x80 in each half whose exponent field is non-zero
    const uint32_t enz = ((x & 0x00780078u) + 0x00780078u) & 0x00800080u;
    const uint32_t keep = __umul24(enz >> 7, 0xFFFFu);
    h = (h & keep) | ((h >> 1) & 0x7FFF7FFFu & ~keep);
    // 0x80 in each half holding 0x7F
    const uint32_t inf = (mag + 0x00010001u) & 0x00800080u;
    const uint32_t isinf = __umul24(inf >> 7, 0xFFFFu);
    h = (h & ~isinf) | (0x7C007C00u & isinf);
    return h | ((x & 0x00800080u) << 8);
}

// f16 operands (pre-decoded e4m3 codes, 2 bytes per element) on
// v_mfma_f32_32x32x16_f16.  A 16-byte LDS chunk holds the 8 halves one lane
// feeds a 32-byte k-step of that MFMA (lane l: row / column l % 32, halves
// 8 (l / 32) .. + 7), the same byte layout as the INT8 MFMA's, so the slice
// is PolicyI8's with the f16 instruction.  kAccScale undoes the decoder's
// 2^-8 pre-scale on both operands.
struct PolicyF16 {
    typedef v16f Acc;
    __device__ __forceinline__ static Acc mfma(const v4i& a, const v4i& b, const Acc& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a),
                                                      __builtin_bit_cast(v8h, b), c, 0, 0, 0);
    }
    __device__ __forceinline__ static void zero(Acc& a) {
#pragma unroll
        for (int r = 0; r < 16; r++) a[r] = 0.0f;
    }
    static constexpr float kAccScale = 65536.0f;
    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
        constexpr int KS = C::BK / 32, D = C::FRAG_DEPTH;
        v4i af[KS][C::TM], bf[KS][C::TN];
        auto load = [&](int ks) {
            const int ch = ks * 2 + khalf;
#pragma unroll
            for (int i = 0; i < C::TM; i++) af[ks][i] = lds_chunk<C>(sa, a_row[i], ch);
#pragma unroll
            for (int j = 0; j < C::TN; j++) bf[ks][j] = lds_chunk<C>(sw, w_row[j], ch);
        };
#pragma unroll
        for (int ks = 0; ks < D - 1 && ks < KS; ks++) load(ks);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks + D - 1 < KS) load(ks + D - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        __builtin_bit_cast(v8h, af[ks][i]), __builtin_bit_cast(v8h, bf[ks][j]),
                        acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

}  // namespace gemm
}  // namespace tkv
