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
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32x32 blocks");
    static_assert(BM % (ROWS_PER_DMA * WAVES) == 0 && BN % (ROWS_PER_DMA * WAVES) == 0,
                  "tile rows must split evenly over wave DMAs");
    static_assert(LDS_BYTES <= 163840, "LDS capacity of a gfx950 workgroup");
    static_assert(LPS * (STAGES - 1) <= 63, "vmcnt range");
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
// __syncthreads (which would drain every outstanding DMA with vmcnt(0));
// the "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

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
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

// Interleave the next step's LDS fragment reads with this step's MFMAs
// (one ds_read after each MFMA while both remain), so LDS latency hides
// behind MFMA execution instead of stalling the pipe at every step.
template <int NMFMA, int NREAD>
__device__ __forceinline__ void interleave_mfma_reads() {
#pragma unroll
    for (int i = 0; i < NMFMA; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (i < NREAD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
#pragma unroll
    for (int i = NMFMA; i < NREAD; i++) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
}

// INT8: v_mfma_i32_32x32x32_i8, 16 K-bytes per lane per 32-K step.
struct PolicyI8 {
    typedef v16i Acc;
    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
        constexpr int KS = C::BK / 32;
        v4i af[2][C::TM], bf[2][C::TN];
#pragma unroll
        for (int i = 0; i < C::TM; i++) af[0][i] = lds_chunk<C>(sa, a_row[i], khalf);
#pragma unroll
        for (int j = 0; j < C::TN; j++) bf[0][j] = lds_chunk<C>(sw, w_row[j], khalf);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int cur = ks & 1, nx = cur ^ 1;
            if (ks + 1 < KS) {
                const int ch = (ks + 1) * 2 + khalf;
#pragma unroll
                for (int i = 0; i < C::TM; i++) af[nx][i] = lds_chunk<C>(sa, a_row[i], ch);
#pragma unroll
                for (int j = 0; j < C::TN; j++) bf[nx][j] = lds_chunk<C>(sw, w_row[j], ch);
            }
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[cur][i], bf[cur][j],
                                                                      acc[i][j], 0, 0, 0);
            if (ks + 1 < KS) interleave_mfma_reads<C::TM * C::TN, C::TM + C::TN>();
        }
    }
};

// FP8 full rate: v_mfma_scale_f32_32x32x64_f8f6f4 (both operands e4m3,
// E8M0 scales 2^0), 32 K-bytes per lane per 64-K step.  Hardware decode is
// OCP e4m3fn and the dot product is accumulated at reduced precision.
struct PolicyF8 {
    typedef v16f Acc;
    static constexpr float kAccScale = 1.0f;
    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
#pragma unroll
        for (int ks = 0; ks < C::BK / 64; ks++) {
            const int ch = ks * 4 + khalf * 2;
            v8i af[C::TM], bf[C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
                v4i lo = lds_chunk<C>(sa, a_row[i], ch), hi = lds_chunk<C>(sa, a_row[i], ch + 1);
                af[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                v4i lo = lds_chunk<C>(sw, w_row[j], ch), hi = lds_chunk<C>(sw, w_row[j], ch + 1);
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

__device__ __forceinline__ v8h dec8_f16(uint32_t lo, uint32_t hi) {
    // bytes b0..b3 of lo then b4..b7 of hi -> 8 f16 in K order
    const uint32_t p0 = dec2_f16(__builtin_amdgcn_perm(0u, lo, 0x0c010c00u));
    const uint32_t p1 = dec2_f16(__builtin_amdgcn_perm(0u, lo, 0x0c030c02u));
    const uint32_t p2 = dec2_f16(__builtin_amdgcn_perm(0u, hi, 0x0c010c00u));
    const uint32_t p3 = dec2_f16(__builtin_amdgcn_perm(0u, hi, 0x0c030c02u));
    return __builtin_bit_cast(v8h, v4i{(int)p0, (int)p1, (int)p2, (int)p3});
}

// FP8 with the reference's products: both operands decoded by the
// reference's decoder into (exact) f16 and multiplied on
// v_mfma_f32_32x32x16_f16, accumulating at f32-class precision.  The f16 MFMA
// runs at half the FP8 rate; this is the drop-in path for matmul_fp8_e4m3.
struct PolicyF8Ref {
    typedef v16f Acc;
    static constexpr float kAccScale = 65536.0f;  // undo the 2^-8 * 2^-8 pre-scale
    template <class C>
    __device__ __forceinline__ static void slice(const uint8_t* sa, const uint8_t* sw,
                                                 const int (&a_row)[C::TM],
                                                 const int (&w_row)[C::TN], int khalf,
                                                 Acc (&acc)[C::TM][C::TN]) {
#pragma unroll
        for (int ks = 0; ks < C::BK / 32; ks++) {
            const int ch = ks * 2 + khalf;  // 16 K-bytes per lane per 32-K step
            v4i af[C::TM], bf[C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; i++) af[i] = lds_chunk<C>(sa, a_row[i], ch);
#pragma unroll
            for (int j = 0; j < C::TN; j++) bf[j] = lds_chunk<C>(sw, w_row[j], ch);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                v8h ah[C::TM], bh[C::TN];
#pragma unroll
                for (int i = 0; i < C::TM; i++)
                    ah[i] = dec8_f16((uint32_t)af[i][2 * h], (uint32_t)af[i][2 * h + 1]);
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    bh[j] = dec8_f16((uint32_t)bf[j][2 * h], (uint32_t)bf[j][2 * h + 1]);
#pragma unroll
                for (int i = 0; i < C::TM; i++)
#pragma unroll
                    for (int j = 0; j < C::TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], acc[i][j],
                                                                           0, 0, 0);
            }
        }
    }
};

}  // namespace gemm
}  // namespace tkv
