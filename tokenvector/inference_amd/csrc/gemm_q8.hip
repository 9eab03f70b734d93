// gemm_q8.hip -- GGUF Q8_0 weights on the INT8 MFMA.  Extension: the
// reference decodes Q8_0 blocks to f32 (_dequant_tensor,
// tv/format/gguf.tkv:284-290) and has no quantized GEMM for them.
//
// A Q8_0 weight [N, K] is K / 32 blocks per row, each an f16 scale d and 32
// int8 codes q (element = d * q).  Unpacked once into codes [N, ldk] (the
// INT8 GEMM's operand layout, rows zero padded to ldk) and group scales f32
// [N, ldk / 32], it multiplies the int8 codes a [M, K] of an activation
// (scale sa per tensor or per token, from the INT8 path's quantizers) as
//   dot_g = sum over the 32 k of block g of a[m, k] q[n, k]   exact INT32
//   acc   = 0;  acc = fma(float(dot_g), d[n, g], acc)  for g = 0, 1, ... in order
//   y     = fl32(fl64(fl64(acc) * sa) + b[n])                 (b = 0 without bias)
// float(dot_g) is exact (|dot_g| <= 32 * 128 * 127 < 2^24), so every group
// adds one rounding, in a fixed order: results do not depend on the launch.
//
// Kernel: 64 x 128 tiles, 4 waves of 32 x 64 (1 x 2 blocks of 32 x 32), three
// workgroups per CU, persistent over tiles in XCD order.  A 2-slot ring of
// 128-deep K slices is filled by LDS DMA (issue_slice); each lane loads its
// own columns' 4 group scales of the next slice (one 16-byte load per
// column block) into registers with that slice's DMA; one barrier per slice.
// (A scale slab filled by DMA beside the operands made the compiler wait
// vmcnt(0) for every slice's DMAs before reading the current slice's scales:
// it could not tell the slab being filled from the one being read.)  A 32-deep k-step
// is one group: one v_mfma_i32_32x32x32_i8 per block into a zero
// accumulator, then per lane 16 conversions and 16 fmas into the f32
// accumulators.  Those two VALU operations per output and group take four
// times the MFMA's time (a wave64 f32 VALU operation issues over 4 cycles and
// packed f32 is not used), so the kernel is VALU-bound near a quarter of the
// INT8 MFMA peak: 2 operations per 32 MACs at 256 CUs x 4 SIMDs x 16 lanes x
// 2.4 GHz give 1.26 POP/s.  Three workgroups per CU (three waves per SIMD)
// let one wave's MFMAs and LDS reads run under the others' VALU work: at
// M = 8192 on the four GPT-2 shapes this measured 47.8 / 17.4 / 62.1 / 56.5
// us against 48.8 / 20.4 / 61.6 / 67.3 with 128 x 128 tiles and two
// workgroups per CU; issuing a group's MFMAs before its VALU work, loading
// the epilogue operands after the K loop, prefetching the next group's
// fragments and 8-wave workgroups all measured within a few percent or
// slower (the 8-wave forms spill).
#include "gemm_kernels.h"

namespace tkv {
namespace gemm {
namespace {

typedef Cfg<64, 128, 2, 2, 128, 2> CfgQ8;  // 48 KB ring (2 slots of 64 + 128 rows x 128 B)
constexpr int kQ8PerCU = 3;                  // resident workgroups per CU
constexpr int kGroupsPerSlice = CfgQ8::BK / 32;
static_assert(kGroupsPerSlice == 4, "one float4 of group scales per column and slice");
static_assert(kQ8PerCU * CfgQ8::LDS_BYTES <= 163840, "LDS of the resident workgroups");

// The 4 group scales of slice kt for the lane's column of each block j
// (tile column w_row[j]); columns past N read column N - 1 (never stored).
template <int TN>
__device__ __forceinline__ void load_scales(const float* __restrict__ gs, int gstride, int N,
                                            int n0, int kt, const int (&w_row)[TN],
                                            float4 (&d4)[TN]) {
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = n0 + w_row[j] < N ? n0 + w_row[j] : N - 1;
        d4[j] = *reinterpret_cast<const float4*>(gs + (int64_t)col * gstride +
                                                 kt * kGroupsPerSlice);
    }
}

// A [M, ldk] and W [N, ldk] int8 (ldk % 128 == 0, rows 16-byte aligned), gs
// f32 [N, ldk / 32] (16-byte aligned); scale_a: sa[0] (ROWS false) or sa[m]
// (ROWS true); bias f32 [N] or null; Y f32 [M, N].  Grid <= tiles.
template <bool ROWS>
__global__ __launch_bounds__(CfgQ8::THREADS, kQ8PerCU) void k_gemm_q8(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ gs,
    int M, int N, int ldk, const float* __restrict__ scale_a, const float* __restrict__ bias,
    float* __restrict__ Y) {
    typedef CfgQ8 C;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS_BYTES];
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5;
    const int tiles_n = (N + C::BN - 1) / C::BN;
    const int tiles = ((M + C::BM - 1) / C::BM) * tiles_n;
    const int nk = ldk / C::BK, gstride = ldk / 32;
    int a_row[C::TM], w_row[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++) a_row[i] = wm * C::WTM + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < C::TN; j++) w_row[j] = wn * C::WTN + j * 32 + (lane & 31);
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    int v = blockIdx.x;
    const int t = xcd_tile(v, tiles);
    int m0 = (t / tiles_n) * C::BM, n0 = (t % tiles_n) * C::BN;
    int slot = 0;
    issue_slice<C>(A, W, M, N, ldk, m0, n0, 0, smem, wave, lane);
    float4 d4[C::TN];
    load_scales(gs, gstride, N, n0, 0, w_row, d4);
    for (;;) {
        float acc[C::TM][C::TN][16];
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
        EpiOperands<C, ROWS> eo;
        load_operands<C, ROWS>(scale_a, 1, nullptr, bias, m0, n0, M, N, eo);
        const int vn = v + (int)gridDim.x;
        const bool more = vn < tiles;
        int m0n = 0, n0n = 0;
        if (more) {
            const int tn = xcd_tile(vn, tiles);
            m0n = (tn / tiles_n) * C::BM;
            n0n = (tn % tiles_n) * C::BN;
        }
        for (int kt = 0; kt < nk; kt++) {
            // this wave's copies of the slice have landed; after the barrier
            // every wave's have, and every wave is done with the other slot
            wait_vmcnt<0>();
            barrier();
            const int nslot = slot ^ 1;
            uint8_t* const nbase = smem + nslot * C::STAGE_BYTES;
            float4 dn[C::TN] = {};
            if (kt + 1 < nk) {
                issue_slice<C>(A, W, M, N, ldk, m0, n0, (kt + 1) * C::BK, nbase, wave, lane);
                load_scales(gs, gstride, N, n0, kt + 1, w_row, dn);
            } else if (more) {
                issue_slice<C>(A, W, M, N, ldk, m0n, n0n, 0, nbase, wave, lane);
                load_scales(gs, gstride, N, n0n, 0, w_row, dn);
            }
            const uint8_t* sa = smem + slot * C::STAGE_BYTES;
            const uint8_t* sw = sa + C::A_BYTES;
#pragma unroll
            for (int g = 0; g < kGroupsPerSlice; g++) {
                v4i af[C::TM], bf[C::TN];
#pragma unroll
                for (int i = 0; i < C::TM; i++) af[i] = lds_chunk<C>(sa, a_row[i], g * 2 + khalf);
#pragma unroll
                for (int j = 0; j < C::TN; j++) bf[j] = lds_chunk<C>(sw, w_row[j], g * 2 + khalf);
#pragma unroll
                for (int i = 0; i < C::TM; i++)
#pragma unroll
                    for (int j = 0; j < C::TN; j++) {
                        const v16i p =
                            __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], zero, 0, 0, 0);
                        const float d = g == 0 ? d4[j].x
                                        : g == 1 ? d4[j].y
                                        : g == 2 ? d4[j].z
                                                 : d4[j].w;
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            acc[i][j][r] = __builtin_fmaf((float)p[r], d, acc[i][j][r]);
                    }
            }
            slot = nslot;
#pragma unroll
            for (int j = 0; j < C::TN; j++) d4[j] = dn[j];
        }
        const EpiOperands<C, ROWS> o = eo.pinned();
        write_tile<C, 0, C::TM * 16>(reinterpret_cast<uint32_t*>(Y), m0, n0, M, N,
                                     [&](int i, int j, int r) {
                                         double y = (double)acc[i][j][r] * (double)o.sa(i, r);
                                         y = y + (double)o.b[j];
                                         return __float_as_uint((float)y);
                                     });
        if (!more) break;
        v = vn;
        m0 = m0n;
        n0 = n0n;
    }
}

// One lane per (row, group) of the unpacked layout.  Group g < kb copies
// block g of row r: its f16 scale through the hardware conversion (exact for
// every code; NaN stays NaN) and its 32 codes as two 16-byte stores.  Groups
// past kb (the zero padding up to ldk) get scale 0.
__global__ __launch_bounds__(256) void k_q8_0_unpack(const uint8_t* __restrict__ raw, int64_t rows,
                                                     int kb, int gstride,
                                                     uint8_t* __restrict__ codes, int64_t ldk,
                                                     float* __restrict__ gs) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * gstride) return;
    const int64_t r = i / gstride;
    const int g = (int)(i - r * gstride);
    if (g >= kb) {
        gs[i] = 0.0f;
        return;
    }
    const uint8_t* __restrict__ p = raw + (r * kb + g) * 34;
    gs[i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(p[0] | (p[1] << 8)));
    uint32_t wv[8];
#pragma unroll
    for (int q = 0; q < 8; q++)
        wv[q] = (uint32_t)p[2 + 4 * q] | (uint32_t)p[3 + 4 * q] << 8 |
                (uint32_t)p[4 + 4 * q] << 16 | (uint32_t)p[5 + 4 * q] << 24;
    uint4* dst = reinterpret_cast<uint4*>(codes + r * ldk + g * 32);
    dst[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    dst[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
}

}  // namespace
}  // namespace gemm

int launch_q8_0_unpack(Ctx* c, const uint8_t* raw, int64_t n, int64_t k, int64_t ldk,
                       uint8_t* codes, float* gs) {
    if (n < 1 || k < 32 || k % 32 != 0 || ldk % 128 != 0 || ldk < k || !raw || !codes ||
        !gs || !aligned(codes, 16))
        return TKV_HIP_UNSUPPORTED;
    const int64_t gstride = ldk / 32, total = n * gstride;
    if (total >= (1ll << 31)) return TKV_HIP_UNSUPPORTED;  // one work-item each, < 2^32 in all
    hipLaunchKernelGGL(gemm::k_q8_0_unpack, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                       c->stream, raw, n, (int)(k / 32), (int)gstride, codes, ldk, gs);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_gemm_q8(Ctx* c, const int8_t* a, const int8_t* w, const float* gs, int64_t m,
                   int64_t n, int64_t ldk, const float* scale_a, int64_t scale_a_stride,
                   const float* bias, float* y) {
    typedef gemm::CfgQ8 C;
    if (m < 1 || n < 1 || ldk < C::BK || ldk % C::BK != 0 || m >= (1ll << 28) ||
        n >= (1ll << 28) || (scale_a_stride != 0 && scale_a_stride != 1) || !scale_a ||
        !aligned(a, 16) || !aligned(w, 16) || !aligned(gs, 16))
        return TKV_HIP_UNSUPPORTED;
    const int64_t tiles = ceil_div(m, C::BM) * ceil_div(n, C::BN);
    if (tiles >= (1ll << 31)) return TKV_HIP_UNSUPPORTED;
    const int64_t resident = (int64_t)c->num_cus * gemm::kQ8PerCU;
    const int64_t grid = tiles < resident ? tiles : resident;
    const uint8_t* ua = reinterpret_cast<const uint8_t*>(a);
    const uint8_t* uw = reinterpret_cast<const uint8_t*>(w);
    if (scale_a_stride)
        hipLaunchKernelGGL(gemm::k_gemm_q8<true>, dim3((unsigned)grid), dim3(C::THREADS), 0,
                           c->stream, ua, uw, gs, (int)m, (int)n, (int)ldk, scale_a, bias, y);
    else
        hipLaunchKernelGGL(gemm::k_gemm_q8<false>, dim3((unsigned)grid), dim3(C::THREADS), 0,
                           c->stream, ua, uw, gs, (int)m, (int)n, (int)ldk, scale_a, bias, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
