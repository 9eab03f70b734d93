// int4.hip -- grouped INT4 weights (tv/quantization/int4.tkv) and the GGUF
// block formats that feed quantized linears (tv/format/gguf.tkv:284-313).
//
//   quantize           one wave per (row, group): max |x| (symmetric) or
//                      min / max (AWQ-asym) by wave reduction, the
//                      reference's scalar f64 arithmetic for scale / zp, then
//                      the group's bytes (an even column and its neighbour,
//                      the pair coded with the scale of group c / group_size
//                      as in the reference).  Unpack: one lane per byte.
//   INT4 GEMM          y = fl32(sum_k x * ((nibble - 8) * scale) + bias) with
//                      f64 accumulation on v_mfma_f64_16x16x4_f64: 64 x 64
//                      tiles (operands straight into MFMA fragments, or
//                      staged in LDS for the act-order gather), K split over
//                      workgroups when the tiles are few; decode batches of
//                      2-32 rows on 16-column MFMA workgroups; one row with
//                      one wave per column.  Every product x * w is exact in
//                      f64 (24 + 4 + 24 bits), so the result differs from the
//                      reference's sequential f64 sum only by the order of
//                      the additions (and, where the group scale is applied
//                      once per group, one fma rounding per group).
//   GGUF blocks        four outputs per lane (one per lane for unaligned
//                      buffers); f16 scales through the hardware conversion
//                      (exact for every finite code).
//
// Codes are packed bytes on the device ([rows, cols / 2], low nibble = even
// column); the host mirrors move the reference's int32-per-byte lists.
#include <algorithm>
#include <cstdlib>

#include "tkv_device.h"
#include "tkv_internal.h"

namespace tkv {

namespace {

constexpr int kI4Block = 256;

// .NET Math.Round (half to even) then the saturating double -> long
// conversion, clamped to [lo, hi].
__device__ __forceinline__ int round_clamp(double v, int lo, int hi) {
    const double r = __builtin_rint(v);
    if (r != r) return lo > 0 ? lo : (hi < 0 ? hi : 0);  // int(NaN) = 0, then clamped
    return r < (double)lo ? lo : (r > (double)hi ? hi : (int)r);
}

// ---------------------------------------------------------------------------
// group parameters (int4.tkv:22-33 symmetric, 96-147 asymmetric)
// ---------------------------------------------------------------------------

// One wave per group, groups grid-strided: the group's parameters, then its
// bytes.  Symmetric: am = max |x| floored at 1e-8, scale = fl32(am / 7) (NaN
// elements never compare greater).  Asym: mn / mx in the reference's scan
// order, which is the NaN-ignoring min / max unless the group's first element
// is NaN (then both stay NaN).
//   Bytes: one lane per column pair (c, c + 1), c even, coded with group
// c / gs (for an odd group size the pair's second column may belong to the
// next group; the reference codes it with this group's scale too), so the
// wave of group g packs the pairs whose even column lies in it.  Symmetric:
// q = clamp(round(x * (1.0 / scale)), -8, 7) + 8 with the f32 scale; asym:
// mn = -zp * scale, q = clamp(round((x - mn) / scale), 0, 15).  OUT32 writes
// the reference's int32-per-byte list.
template <bool ASYM, bool OUT32>
__global__ __launch_bounds__(kI4Block) void k_int4_quantize(const float* __restrict__ src,
                                                            int64_t rows, int64_t cols, int64_t gs,
                                                            float* __restrict__ scales,
                                                            int64_t* __restrict__ zps,
                                                            void* __restrict__ packed) {
    const int64_t ng = cols / gs, groups = rows * ng, half = cols / 2;
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * (kI4Block / 64);
    for (int64_t q = (int64_t)blockIdx.x * (kI4Block / 64) + (threadIdx.x >> 6); q < groups;
         q += waves) {
        const int64_t r = q / ng, g = q - r * ng;
        const float* x = src + r * cols + g * gs;
        float a = 0.0f, mn = __builtin_inff(), mx = -__builtin_inff();
        for (int64_t c = lane; c < gs; c += 64) {
            const float v = x[c];
            if (ASYM) {
                mn = fminf(mn, v);
                mx = fmaxf(mx, v);
            } else {
                a = fmaxf(a, fabsf(v));
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            if (ASYM) {
                mn = fminf(mn, __shfl_xor(mn, o, 64));
                mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            } else {
                a = fmaxf(a, __shfl_xor(a, o, 64));
            }
        }
        // every lane holds the reduced values: each forms the parameters
        float scf;
        int zp = 8;
        if (!ASYM) {
            double am = (double)a;
            if (am < 0.00000001) am = 0.00000001;
            scf = (float)(am / 7.0);
        } else {
            double dmn = (double)mn, dmx = (double)mx;
            if (x[0] != x[0]) dmn = dmx = (double)x[0];
            if (dmx - dmn < 0.00000001) dmx = dmn + 0.00000001;
            double sc = (dmx - dmn) / 15.0;
            zp = round_clamp(-dmn / sc, 0, 15);
            if (zp == 0) {
                if (dmn > 0) {
                    sc = dmx / 15.0;
                    if (sc < 0.00000001) sc = 0.00000001;
                    zp = 0;
                }
            } else if (zp == 15) {
                sc = -dmn / 15.0;
            }
            if (sc < 0.00000001) sc = 0.00000001;
            scf = (float)sc;
        }
        if (lane == 0) {
            scales[q] = scf;
            if (ASYM) zps[q] = zp;
        }
        const double sc = (double)scf;
        const int64_t c_end = (g + 1) * gs;
        for (int64_t c = ((g * gs + 1) & ~(int64_t)1) + 2 * lane; c < c_end; c += 128) {
            const double x0 = (double)src[r * cols + c], x1 = (double)src[r * cols + c + 1];
            int q0, q1;
            if (ASYM) {
                const double mnv = (double)(-zp) * sc;
                q0 = round_clamp((x0 - mnv) / sc, 0, 15);
                q1 = round_clamp((x1 - mnv) / sc, 0, 15);
            } else {
                const double inv = 1.0 / sc;
                q0 = round_clamp(x0 * inv, -8, 7) + 8;
                q1 = round_clamp(x1 * inv, -8, 7) + 8;
            }
            const int b = (q1 << 4) | q0;
            const int64_t i = r * half + c / 2;
            if (OUT32)
                static_cast<int32_t*>(packed)[i] = b;
            else
                static_cast<uint8_t*>(packed)[i] = (uint8_t)b;
        }
    }
}

// dst[c] = fl32(float(nibble - zp) * scale) with zp = 8 (symmetric) or the
// group's zero point; IN32 reads int32-per-byte lists (low 8 bits).
template <bool ASYM, bool IN32>
__global__ __launch_bounds__(kI4Block) void k_int4_unpack(const void* __restrict__ packed,
                                                          int64_t rows, int64_t cols, int64_t gs,
                                                          const float* __restrict__ scales,
                                                          const int64_t* __restrict__ zps,
                                                          float* __restrict__ dst) {
    const int64_t half = cols / 2, total = rows * half, ng = cols / gs;
    const int64_t stride = (int64_t)gridDim.x * kI4Block;
    for (int64_t i = (int64_t)blockIdx.x * kI4Block + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / half, c = (i - r * half) * 2;
        const int64_t gi = r * ng + c / gs;
        const int64_t b = IN32 ? (int64_t) static_cast<const int32_t*>(packed)[i]
                               : (int64_t) static_cast<const uint8_t*>(packed)[i];
        const double sc = (double)scales[gi];
        const int64_t zp = ASYM ? zps[gi] : 8;
        dst[r * cols + c] = (float)((double)((b & 0xF) - zp) * sc);
        dst[r * cols + c + 1] = (float)((double)(((b >> 4) & 0xF) - zp) * sc);
    }
}

// out[r, c] = src[r, perm[c]] (INV: out[r, perm[c]] = src[r, c]).  Entries
// outside [0, cols) gather 0 / are skipped (the host mirror rejects them).
template <bool INV>
__global__ __launch_bounds__(kI4Block) void k_permute_cols(const float* __restrict__ src,
                                                           int64_t rows, int64_t cols,
                                                           const int64_t* __restrict__ perm,
                                                           float* __restrict__ out) {
    const int64_t total = rows * cols, stride = (int64_t)gridDim.x * kI4Block;
    for (int64_t i = (int64_t)blockIdx.x * kI4Block + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / cols, c = i - r * cols;
        const int64_t p = perm[c];
        const bool ok = p >= 0 && p < cols;
        if (INV) {
            if (ok) out[r * cols + p] = src[i];
        } else {
            out[i] = ok ? src[r * cols + p] : 0.0f;
        }
    }
}

// ---------------------------------------------------------------------------
// INT4 GEMM on f64 MFMA (int4.tkv:195-239)
// ---------------------------------------------------------------------------

// Workgroup tile 64 x 64 outputs, four waves of 32 x 32 (2 x 2 blocks of
// v_mfma_f64_16x16x4_f64).  K goes in slices of 32: each slice stages A
// (f32 -> f64, gathered through perm for the act-order form) and the
// dequantized weights w = (nibble - 8) * scale[n, k / gs] (f64, exact) in LDS,
// k-major with a row pitch of 80 doubles: the 4 k-rows one MFMA operand read
// touches then fall into two halves of the 64 banks.  Operand layouts of the
// 16x16x4 f64 MFMA: A lane l = row l % 16, k l / 16; B lane l = k l / 16,
// column l % 16; D lane l, register v holds row l / 16 + 4 v, column l % 16.
constexpr int kGBM = 64, kGBN = 64, kGBK = 32, kGPitch = 80;
typedef double f64x4 __attribute__((ext_vector_type(4)));

// This LDS form serves the act-order gather (PERM) and operands without
// 16-byte rows (K % 8 != 0, gs % 8 != 0 or unaligned bases); the rest takes
// k_matmul_int4_regs below.  The next slice's raw operands are loaded into
// registers before the current slice's MFMAs, so their latency overlaps the
// matrix work.
//   SPLIT (few tiles for the CUs): workgroup z of the grid's third dimension
// takes K range [z kchunk, (z + 1) kchunk) (kchunk a multiple of the slice)
// and writes its f64 partial tile to part[z] ([gridDim.y * 64, gridDim.x *
// 64], every element); k_int4_split_sum then adds the partials in z order.
template <bool PERM, bool SPLIT = false>
__global__ __launch_bounds__(256) void k_matmul_int4_f64(
    const float* __restrict__ A, const uint8_t* __restrict__ Wp, const float* __restrict__ scales,
    const float* __restrict__ bias, const int64_t* __restrict__ perm, float* __restrict__ Y,
    int M, int N, int K, int gs, int kchunk = 0, double* __restrict__ part = nullptr) {
    __shared__ double sA[kGBK][kGPitch];
    __shared__ double sW[kGBK][kGPitch];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kGBM, n0 = blockIdx.x * kGBN;
    const int ng = K / gs, half = K / 2;
    f64x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};
    // staging roles: row / column t / 4, k offset (t % 4) * 8 within the slice
    const int sr = t >> 2, sk = (t & 3) * 8;
    const int gm = m0 + sr, gn = n0 + sr;
    float ra[8], rs[8];
    int rb[4];
    auto fetch = [&](int k0) {
        const int kb = k0 + sk;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int kk = kb + i;
            float x = 0.0f;
            if (gm < M && kk < K) {
                // a perm entry outside [0, K) reads 0 (the host mirror rejects it)
                const int64_t src_k = PERM ? perm[kk] : (int64_t)kk;
                if (src_k >= 0 && src_k < K) x = A[(int64_t)gm * K + src_k];
            }
            ra[i] = x;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kk = kb + 2 * i;  // even
            int bb = 0x88;              // codes 8: w = 0
            float s0 = 0.0f, s1 = 0.0f;
            if (gn < N && kk < K) {
                bb = Wp[(int64_t)gn * half + kk / 2];
                s0 = scales[(int64_t)gn * ng + kk / gs];
                s1 = scales[(int64_t)gn * ng + (kk + 1) / gs];
            }
            rb[i] = bb;
            rs[2 * i] = s0;
            rs[2 * i + 1] = s1;
        }
    };
    const int kbeg = SPLIT ? (int)blockIdx.z * kchunk : 0;
    const int kend = SPLIT ? min(K, kbeg + kchunk) : K;
    fetch(kbeg);
    for (int k0 = kbeg; k0 < kend; k0 += kGBK) {
#pragma unroll
        for (int i = 0; i < 8; i++) sA[sk + i][sr] = (double)ra[i];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            sW[sk + 2 * i][sr] = (double)((rb[i] & 15) - 8) * (double)rs[2 * i];
            sW[sk + 2 * i + 1][sr] = (double)(((rb[i] >> 4) & 15) - 8) * (double)rs[2 * i + 1];
        }
        __syncthreads();
        if (k0 + kGBK < kend) fetch(k0 + kGBK);
#pragma unroll
        for (int kk = 0; kk < kGBK; kk += 4) {
            const int kr = kk + (lane >> 4), l16 = lane & 15;
            const double a0 = sA[kr][wm * 32 + l16], a1 = sA[kr][wm * 32 + 16 + l16];
            const double b0 = sW[kr][wn * 32 + l16], b1 = sW[kr][wn * 32 + 16 + l16];
            acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
    }
    if constexpr (SPLIT) {
        const int64_t nt = (int64_t)gridDim.x * kGBN;
        double* __restrict__ mine = part + (int64_t)blockIdx.z * gridDim.y * kGBM * nt;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int col = n0 + wn * 32 + j * 16 + (lane & 15);
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int row = m0 + wm * 32 + i * 16 + (lane >> 4) + 4 * v;
                    mine[(int64_t)row * nt + col] = acc[i][j][v];
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn * 32 + j * 16 + (lane & 15);
            if (col >= N) continue;
            const double b = bias ? (double)bias[col] : 0.0;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = m0 + wm * 32 + i * 16 + (lane >> 4) + 4 * v;
                if (row < M) Y[(int64_t)row * N + col] = (float)(acc[i][j][v] + b);
            }
        }
}

// Operands with 16-byte rows (K % 8 == 0, gs % 8 == 0, A 16-byte and W 4-byte
// aligned, no perm), without LDS: each wave loads its own operands straight
// into MFMA fragments, as the decode kernel does.  The MFMA's k index is free (both
// operands agree on it), so in slice k0 lane l (row / column l % 16, quad
// q = l / 16) owns k0 + 8 q .. k0 + 8 q + 7 and MFMA step s takes k0 + 8 q + s:
// each lane reads two float4 of its A row and one 32-bit word of its W row
// (8 nibbles, one group scale) per 16 x 16 block.  The products are the LDS
// form's (x as f64 times (nibble - 8) * scale, exact); only the order of the
// f64 additions differs.  No LDS and no barriers: the four waves of a 64 x 64
// tile run independently, and the next slice's operands are loaded before the
// current slice's 32 MFMAs.  Rows past M and columns past N read row M - 1 /
// column N - 1 and are never stored; quads past the end of K read zeros.
template <bool SPLIT, bool FACT = false>
__global__ __launch_bounds__(256) void k_matmul_int4_regs(
    const float* __restrict__ A, const uint8_t* __restrict__ Wp, const float* __restrict__ scales,
    const float* __restrict__ bias, float* __restrict__ Y, int M, int N, int K, int gs,
    int kchunk, double* __restrict__ part) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kGBM, n0 = blockIdx.x * kGBN;
    const int l16 = lane & 15, q = lane >> 4;
    const int half = K / 2, ng = K / gs;
    const float* __restrict__ arow[2];
    const uint8_t* __restrict__ wrow[2];
    const float* __restrict__ srow[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = min(m0 + wm * 32 + i * 16 + l16, M - 1);
        const int c = min(n0 + wn * 32 + i * 16 + l16, N - 1);
        arow[i] = A + (int64_t)r * K;
        wrow[i] = Wp + (int64_t)c * half;
        srow[i] = scales + (int64_t)c * ng;
    }
    f64x4 acc[2][2], accg[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = accg[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};
    const int kbeg = SPLIT ? (int)blockIdx.z * kchunk : 0;
    const int kend = SPLIT ? min(K, kbeg + kchunk) : K;
    struct Buf {
        float4 a[2][2];
        uint32_t w[2];
        float s[2];
    };
    // Loads are issued for every slice, the one past the end included, at
    // addresses clamped into [kbeg, kend): a load under a branch would make
    // the wait before the next MFMAs cover every load in flight (vmcnt counts
    // in issue order), and the prefetch would be lost.  K % 8 == 0 and kend %
    // 8 == 0, so a quad that starts inside [.., kend) ends inside it.
    auto load = [&](Buf& b, int k0) {
        const int kc = min(k0 + 8 * q, kend - 8);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float4* p = reinterpret_cast<const float4*>(arow[i] + kc);
            b.a[i][0] = p[0];
            b.a[i][1] = p[1];
            b.w[i] = *reinterpret_cast<const uint32_t*>(wrow[i] + kc / 2);
            b.s[i] = srow[i][kc / gs];
        }
    };
    // TAIL: the slice runs past kend (K % 32 != 0); quads starting at or past
    // kend count zero
    //   FACT (gs % 32 == 0: a slice lies in one group; unsplit launches
    // only): the B operand is the
    // nibble's integer value, the products x (nibble - 8) (exact) sum into
    // accg over a group, and the group's end adds accg * scale into acc with
    // one fma per output (in the D layout lane l holds column l % 16, whose
    // scale this lane loaded): 16 f64 multiplies per slice fewer.
    auto compute = [&](const Buf& b, bool tail, bool in) {
        double sc[2];
#pragma unroll
        for (int i = 0; i < 2; i++) sc[i] = tail && !in ? 0.0 : (double)b.s[i];
#pragma unroll
        for (int st = 0; st < 8; st++) {
            double x[2], w[2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float4 v = b.a[i][st >> 2];
                const float f = (st & 3) == 0 ? v.x : (st & 3) == 1 ? v.y : (st & 3) == 2 ? v.z : v.w;
                x[i] = tail && !in ? 0.0 : (double)f;
                const double d = (double)((int)((b.w[i] >> (4 * st)) & 15) - 8);
                w[i] = FACT ? d : d * sc[i];
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    if constexpr (FACT)
                        accg[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(x[i], w[j], accg[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(x[i], w[j], acc[i][j], 0, 0, 0);
                }
        }
    };
    auto flush = [&](const Buf& b) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const double sc = (double)b.s[j];
#pragma unroll
            for (int i = 0; i < 2; i++) {
#pragma unroll
                for (int v = 0; v < 4; v++) acc[i][j][v] = __builtin_fma(accg[i][j][v], sc, acc[i][j][v]);
                accg[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};
            }
        }
    };
    auto step = [&](const Buf& b, int k0) {
        if (k0 + kGBK <= kend)
            compute(b, false, true);
        else
            compute(b, true, k0 + 8 * q < kend);
        if constexpr (FACT)
            if ((k0 + kGBK) % gs == 0 || k0 + kGBK >= kend) flush(b);
    };
    Buf b0, b1;
    if (kbeg < kend) {  // K = 0 loads nothing (the launcher also keeps it off this kernel)
        load(b0, kbeg);
        for (int k0 = kbeg;;) {
            load(b1, k0 + kGBK);
            step(b0, k0);
            k0 += kGBK;
            if (k0 >= kend) break;
            load(b0, k0 + kGBK);
            step(b1, k0);
            k0 += kGBK;
            if (k0 >= kend) break;
        }
    }
    if constexpr (SPLIT) {
        const int64_t nt = (int64_t)gridDim.x * kGBN;
        double* __restrict__ mine = part + (int64_t)blockIdx.z * gridDim.y * kGBM * nt;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int col = n0 + wn * 32 + j * 16 + l16;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int row = m0 + wm * 32 + i * 16 + q + 4 * v;
                    mine[(int64_t)row * nt + col] = acc[i][j][v];
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn * 32 + j * 16 + l16;
            if (col >= N) continue;
            const double bb = bias ? (double)bias[col] : 0.0;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = m0 + wm * 32 + i * 16 + q + 4 * v;
                if (row < M) Y[(int64_t)row * N + col] = (float)(acc[i][j][v] + bb);
            }
        }
}

// y[row, col] = fl32((part[0] + part[1] + ... + part[S - 1]) + bias[col]),
// the split partials added in split order (a fixed order: launches repeat
// bit for bit).
__global__ __launch_bounds__(256) void k_int4_split_sum(const double* __restrict__ part, int S,
                                                         int64_t mt, int64_t nt,
                                                         const float* __restrict__ bias,
                                                         float* __restrict__ Y, int M, int N) {
    const int64_t total = (int64_t)M * N;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int64_t row = e / N, col = e - row * N;
        const double* __restrict__ p = part + row * nt + col;
        double acc = p[0];
        for (int s = 1; s < S; s++) acc = acc + p[(int64_t)s * mt * nt];
        const double b = bias ? (double)bias[col] : 0.0;
        Y[e] = (float)(acc + b);
    }
}

// Decode batches (M <= MM <= kGemvRows, MM a power of two): one wave per
// output column streams that
// weight row once; lane l takes bytes l, l + 64, ... (k pairs), every row's
// products are added with f64 FMAs (the products are exact, so each FMA
// rounds like the reference's add), and the 64 lane sums are combined in a
// fixed butterfly order.
constexpr int kGemvRows = 32;

template <int MM, bool PERM>
__global__ __launch_bounds__(256) void k_gemv_int4_f64(
    const float* __restrict__ A, const uint8_t* __restrict__ Wp, const float* __restrict__ scales,
    const float* __restrict__ bias, const int64_t* __restrict__ perm, float* __restrict__ Y,
    int M, int N, int K, int gs) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;  // whole waves
    const int half = K / 2, ng = K / gs;
    const uint8_t* __restrict__ wr = Wp + (int64_t)n * half;
    const float* __restrict__ sr = scales + (int64_t)n * ng;
    double acc[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) acc[m] = 0.0;
    for (int kb = lane; kb < half; kb += 64) {
        const int b = wr[kb], k0 = 2 * kb;
        const double w0 = (double)((b & 15) - 8) * (double)sr[k0 / gs];
        const double w1 = (double)(((b >> 4) & 15) - 8) * (double)sr[(k0 + 1) / gs];
        int64_t c0 = k0, c1 = k0 + 1;
        bool ok0 = true, ok1 = true;
        if (PERM) {
            c0 = perm[k0];
            c1 = perm[k0 + 1];
            ok0 = c0 >= 0 && c0 < K;
            ok1 = c1 >= 0 && c1 < K;
        }
#pragma unroll
        for (int m = 0; m < MM; m++)
            if (m < M) {
                double x0, x1;
                if (PERM) {
                    x0 = ok0 ? (double)A[(int64_t)m * K + c0] : 0.0;
                    x1 = ok1 ? (double)A[(int64_t)m * K + c1] : 0.0;
                } else {  // K even: the pair is one aligned 8-byte load
                    const float2 u = *reinterpret_cast<const float2*>(A + (int64_t)m * K + k0);
                    x0 = (double)u.x;
                    x1 = (double)u.y;
                }
                acc[m] = __builtin_fma(x0, w0, acc[m]);
                acc[m] = __builtin_fma(x1, w1, acc[m]);
            }
    }
    const double bb = bias ? (double)bias[n] : 0.0;
#pragma unroll
    for (int m = 0; m < MM; m++)
        if (m < M) {
            double v = acc[m];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
            if (lane == 0) Y[(int64_t)m * N + n] = (float)(v + bb);
        }
}

// One row (decode at batch 1) with 16-byte rows (K % 8 == 0, gs % 8 == 0, A
// 16-byte and W 4-byte aligned, no perm): one wave per column; at step u lane
// l takes k = 512 u + 8 l .. + 7 (one 32-bit word of nibbles, one group scale,
// two float4 of x), and kRowSteps = ceil(K / 512) steps (at most 6) are
// loaded before any is used, so a column of up to 3072 weights costs one
// memory round trip.  Lanes past K load the last 8-run again (no branch around
// a load) and count zero.  Per lane the products are added in k order, then
// the 64 lane sums pairwise.
template <int kRowSteps>
__global__ __launch_bounds__(256) void k_gemv_int4_row(
    const float* __restrict__ A, const uint8_t* __restrict__ Wp, const float* __restrict__ scales,
    const float* __restrict__ bias, float* __restrict__ Y, int N, int K, int gs) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;  // whole waves
    const int half = K / 2, ng = K / gs;
    const uint8_t* __restrict__ wr = Wp + (int64_t)n * half;
    const float* __restrict__ sr = scales + (int64_t)n * ng;
    double acc = 0.0;
    for (int base = 0; base < K; base += 512 * kRowSteps) {
        uint32_t w[kRowSteps];
        float s[kRowSteps];
        float4 x0[kRowSteps], x1[kRowSteps];
        bool in[kRowSteps];
#pragma unroll
        for (int u = 0; u < kRowSteps; u++) {
            const int kk = base + 512 * u + 8 * lane;
            in[u] = kk < K;
            const int kc = in[u] ? kk : K - 8;
            w[u] = *reinterpret_cast<const uint32_t*>(wr + kc / 2);
            s[u] = sr[kc / gs];
            const float4* p = reinterpret_cast<const float4*>(A + kc);
            x0[u] = p[0];
            x1[u] = p[1];
        }
#pragma unroll
        for (int u = 0; u < kRowSteps; u++) {
            const double sc = (double)s[u];
            const float xs[8] = {x0[u].x, x0[u].y, x0[u].z, x0[u].w,
                                 x1[u].x, x1[u].y, x1[u].z, x1[u].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const double x = in[u] ? (double)xs[e] : 0.0;
                const double wv = (double)((int)((w[u] >> (4 * e)) & 15) - 8) * sc;
                acc = __builtin_fma(x, wv, acc);
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc = acc + __shfl_xor(acc, o, 64);
    if (lane == 0) Y[n] = (float)(acc + (bias ? (double)bias[n] : 0.0));
}

// Decode batches on the f64 MFMA (M <= 16 MB rows, K % 32 == 0, gs % 8 == 0,
// no column permutation).  A workgroup of kDecWaves waves owns 16 output
// columns and one of `splits` contiguous ranges of 32-deep k blocks; its waves
// divide that range again.  Within a k block, lane group g = lane / 16 takes
// k = 32 kb + 8 g + s at MFMA step s (the same permutation of k for A and W,
// so every product x * w still meets its partner): one 16-byte A load per row
// block and one 4-byte weight load (8 nibbles, one scale) per lane cover 8
// steps.  w = (nibble - 8) * scale is formed once per lane and shared by all
// rows through the MFMA, and the activations are read from L2 once per
// 16-column workgroup instead of once per column.
//   The waves' partial sums are added in LDS in wave order.  With splits > 1
// each workgroup writes its partial tile to `part` and counts itself in on
// arrivals[cb]; the workgroup that completes the count adds the splits' tiles
// in split order, adds the bias, stores y and clears the count.  Every output
// is therefore the same fixed-order f64 sum on every run.
//   Ordering without cache maintenance: the tiles are written with agent-scope
// atomic stores and read with agent-scope atomic loads, which gfx950 performs
// at the device coherence point (sc1: not held in, or served from, an XCD's
// L2).  Every wave waits for its own stores to complete (vmcnt(0): an atomic
// store completes once it is performed there) before the workgroup barrier,
// and the arrival add is issued after that barrier; the completing workgroup
// issues its tile loads only after its arrival add has returned.  So every
// tile is in place before any load of it is issued.  A release add with an
// acquire fence would instead write back and invalidate a whole L2 per
// workgroup: measured at ~20 us per call over ~500 workgroups.
//   Each wave's k blocks are a chain of dependent MFMAs per row block, so
// more waves per workgroup shorten every chain: 8 waves against 4 measured
// 5-14% faster on the four GPT-2 shapes at M = 2 .. 32 (attn_out M = 32
// 7.8 -> 6.7 us, mlp_down M = 32 13.5 -> 12.4 us); 12 waves tied with 8 and
// 16 were slower (qkv M = 32 9.5 us).
constexpr int kDecWaves = 8;

// LINES: the workgroup's 16 packed weight rows over its k range are copied
// into LDS first by direct DMA, whole 128-byte lines of 8 rows per 1 KB
// instruction (16-byte chunks XOR-swizzled per row, so the 64 lanes' 4-byte
// reads of one k block hit 64 distinct banks); the loop then loads only the
// activations.  The register form reads 16 bytes of each of 16 rows' lines
// per instruction, one k block ahead.  Needs K % 256 == 0 (rows of whole
// lines); dynamic LDS 2 KB per line of the k range.
__device__ __forceinline__ int int4_swz(int row) { return (row & 7) ^ (row >> 3); }

template <int MB, bool LINES = false>
__global__ __launch_bounds__(kDecWaves * 64) void k_gemv_int4_mfma(
    const float* __restrict__ A, const uint8_t* __restrict__ Wp, const float* __restrict__ scales,
    const float* __restrict__ bias, float* __restrict__ Y, int M, int N, int K, int gs,
    int splits, double* __restrict__ part, unsigned* __restrict__ arrivals) {
    __shared__ double sP[kDecWaves][MB * 16][17];
    __shared__ int s_last;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cb = (int)blockIdx.x / splits, sp = (int)blockIdx.x % splits;
    const int n0 = cb * 16;
    const int g = lane >> 4, l16 = lane & 15;
    const int nkb = K / 32;
    const int lo = (int)((int64_t)nkb * sp / splits), hi = (int)((int64_t)nkb * (sp + 1) / splits);
    const int wlo = lo + (hi - lo) * wave / kDecWaves, whi = lo + (hi - lo) * (wave + 1) / kDecWaves;
    const int half = K / 2, ng = K / gs;
    // rows past M and columns past N read row 0 / column N - 1; they are never stored
    const float* __restrict__ arow[MB];
#pragma unroll
    for (int i = 0; i < MB; i++) {
        const int r = 16 * i + l16;
        arow[i] = A + (int64_t)(r < M ? r : 0) * K + 8 * g;
    }
    const int col = n0 + l16 < N ? n0 + l16 : N - 1;
    const uint8_t* __restrict__ wrow = Wp + (int64_t)col * half + 4 * g;
    const float* __restrict__ srow = scales + (int64_t)col * ng;
    f64x4 acc[MB];
#pragma unroll
    for (int i = 0; i < MB; i++) acc[i] = f64x4{0.0, 0.0, 0.0, 0.0};
    // LINES: lines [p_lo, p_hi) of the k range (8 k blocks each); DMA d = 2
    // (p - p_lo) + h holds rows 8 h .. 8 h + 7, lane 8 rr + q taking chunk
    // q ^ int4_swz(8 h + rr); k block kb of row l16 is chunk kb & 7 of line
    // kb / 8, its dword g the lane's 8 codes
    extern __shared__ __attribute__((aligned(16))) uint8_t s_wl[];
    const int p_lo = lo >> 3;
    if constexpr (LINES) {
        const int nd = 2 * (((hi + 7) >> 3) - p_lo);
        const int rr = lane >> 3, q = lane & 7;
        for (int d = wave; d < nd; d += kDecWaves) {
            const int row = 8 * (d & 1) + rr;
            const int c = n0 + row < N ? n0 + row : N - 1;
            const uint8_t* src = Wp + (int64_t)c * half + (int64_t)(p_lo + (d >> 1)) * 128 +
                                 ((q ^ int4_swz(row)) << 4);
            __builtin_amdgcn_global_load_lds((const void*)src,
                                             (__attribute__((address_space(3))) void*)(s_wl + d * 1024),
                                             16, 0, 0);
        }
        // every wave's DMAs have landed (vmcnt), then a raw barrier publishes
        // them (__syncthreads() would also wait, being a release fence)
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    const int wl_row = ((l16 >> 3) << 10) + ((l16 & 7) << 7) + 4 * g;
    const int wl_swz = int4_swz(l16);
    // each k block's operands are loaded one block ahead, so their latency
    // overlaps the previous block's MFMAs
    float4 an[MB][2];
    uint32_t wn = 0;
    float sn = 0.0f;
    auto fetch = [&](int kb) {
#pragma unroll
        for (int i = 0; i < MB; i++) {
            const float4* p = reinterpret_cast<const float4*>(arow[i] + 32 * kb);
            an[i][0] = p[0];
            an[i][1] = p[1];
        }
        if constexpr (LINES)
            wn = *reinterpret_cast<const uint32_t*>(s_wl + (((kb >> 3) - p_lo) << 11) + wl_row +
                                                    (((kb & 7) ^ wl_swz) << 4));
        else
            wn = *reinterpret_cast<const uint32_t*>(wrow + 16 * kb);
        sn = srow[(32 * kb + 8 * g) / gs];
    };
    if (wlo < whi) fetch(wlo);
    for (int kb = wlo; kb < whi; kb++) {
        float4 a[MB][2];
#pragma unroll
        for (int i = 0; i < MB; i++) {
            a[i][0] = an[i][0];
            a[i][1] = an[i][1];
        }
        const uint32_t w8 = wn;
        const double sc = (double)sn;
        if (kb + 1 < whi) fetch(kb + 1);
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const double b = (double)((int)((w8 >> (4 * s)) & 15) - 8) * sc;
#pragma unroll
            for (int i = 0; i < MB; i++) {
                const float4 q = a[i][s >> 2];
                const float x = (s & 3) == 0 ? q.x : (s & 3) == 1 ? q.y : (s & 3) == 2 ? q.z : q.w;
                acc[i] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)x, b, acc[i], 0, 0, 0);
            }
        }
    }
    // D layout: lane l, register v holds row l / 16 + 4 v, column l % 16
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int v = 0; v < 4; v++) sP[wave][16 * i + g + 4 * v][l16] = acc[i][v];
    __syncthreads();
    constexpr int kT = MB * 16 * 16;  // outputs of the tile
    double sum[(kT + kDecWaves * 64 - 1) / (kDecWaves * 64)];
#pragma unroll
    for (int e = 0; e < (kT + kDecWaves * 64 - 1) / (kDecWaves * 64); e++) {
        const int t = threadIdx.x + e * kDecWaves * 64;
        double v = 0.0;
        if (t < kT) {
            const int r = t / 16, c = t % 16;
            v = sP[0][r][c];
#pragma unroll
            for (int w = 1; w < kDecWaves; w++) v = v + sP[w][r][c];
        }
        sum[e] = v;
    }
    if (splits > 1) {
        double* mine = part + (int64_t)blockIdx.x * kT;
#pragma unroll
        for (int e = 0; e < (kT + kDecWaves * 64 - 1) / (kDecWaves * 64); e++) {
            const int t = threadIdx.x + e * kDecWaves * 64;
            if (t < kT) __hip_atomic_store(mine + t, sum[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0)
            s_last = __hip_atomic_fetch_add(arrivals + cb, 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(splits - 1);
        __syncthreads();
        if (!s_last) return;
        double* tiles = part + (int64_t)cb * splits * kT;
#pragma unroll
        for (int e = 0; e < (kT + kDecWaves * 64 - 1) / (kDecWaves * 64); e++) {
            const int t = threadIdx.x + e * kDecWaves * 64;
            if (t < kT) {
                double v = __hip_atomic_load(tiles + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int q = 1; q < splits; q++)
                    v = v + __hip_atomic_load(tiles + (int64_t)q * kT + t, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                sum[e] = v;
            }
        }
        if (threadIdx.x == 0) __hip_atomic_store(arrivals + cb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int e = 0; e < (kT + kDecWaves * 64 - 1) / (kDecWaves * 64); e++) {
        const int t = threadIdx.x + e * kDecWaves * 64;
        const int r = t / 16, c = n0 + t % 16;
        if (t < kT && r < M && c < N) Y[(int64_t)r * N + c] = (float)(sum[e] + (bias ? (double)bias[c] : 0.0));
    }
}

// ---------------------------------------------------------------------------
// GGUF Q8_0 / Q4_0 / Q4_1 blocks (gguf.tkv:284-313)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float half_at(const uint8_t* p) {
    const unsigned short h = (unsigned short)(p[0] | (p[1] << 8));
    return (float)__builtin_bit_cast(_Float16, h);
}

// One lane per output element of the n / 32 whole blocks; the tail past them
// is 0.  Products of an f16 scale and a small integer are exact in f32;
// Q4_1's d * q - m rounds once.
template <int DT>
__global__ __launch_bounds__(kI4Block) void k_gguf_blocks(const uint8_t* __restrict__ raw,
                                                          int64_t n, float* __restrict__ out) {
    constexpr int STEP = DT == 8 ? 34 : DT == 2 ? 18 : 20;
    const int64_t full = n / 32 * 32, stride = (int64_t)gridDim.x * kI4Block;
    for (int64_t i = (int64_t)blockIdx.x * kI4Block + threadIdx.x; i < n; i += stride) {
        if (i >= full) {
            out[i] = 0.0f;
            continue;
        }
        const uint8_t* p = raw + (i / 32) * STEP;
        const int j = (int)(i & 31);
        const float d = half_at(p);
        float v;
        if (DT == 8) {
            v = d * (float)(int8_t)p[2 + j];
        } else if (DT == 2) {
            const int b = p[2 + (j & 15)];
            v = d * (float)((j < 16 ? (b & 15) : (b >> 4)) - 8);
        } else {
            const int b = p[4 + (j & 15)];
            const double dq = (double)d * (double)(j < 16 ? (b & 15) : (b >> 4));
            v = (float)(dq - (double)half_at(p + 2));
        }
        out[i] = v;
    }
}

// Four outputs per thread and one float4 store (out 16-byte aligned); the
// block's f16 scale and the four codes' bytes come as 16-bit loads: blocks
// are 34 / 18 / 20 bytes, so with raw 2-byte aligned every scale, and every
// run of 4 codes starting at a multiple of 4, sits on an even address.  The
// per-element arithmetic is k_gguf_blocks'.  Elements past the last whole
// block read 0 (a float4 group is either all inside the whole blocks or all
// past them: both bounds are multiples of 4).
__device__ __forceinline__ float half_u16(unsigned short h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

template <int DT>
__global__ __launch_bounds__(kI4Block) void k_gguf_blocks4(const uint8_t* __restrict__ raw,
                                                           int64_t n, float* __restrict__ out) {
    constexpr int STEP = DT == 8 ? 34 : DT == 2 ? 18 : 20;
    const int64_t full = n / 32 * 32, n4 = n / 4, stride = (int64_t)gridDim.x * kI4Block;
    const int64_t tid = (int64_t)blockIdx.x * kI4Block + threadIdx.x;
    for (int64_t t = tid; t < n4; t += stride) {
        const int64_t i = 4 * t;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < full) {
            const uint8_t* p = raw + (i / 32) * STEP;
            const int j0 = (int)(i & 31);
            const float d = half_u16(*reinterpret_cast<const unsigned short*>(p));
            const int off = DT == 8 ? 2 + j0 : (DT == 2 ? 2 : 4) + (j0 & 15);
            const unsigned c01 = *reinterpret_cast<const unsigned short*>(p + off);
            const unsigned c23 = *reinterpret_cast<const unsigned short*>(p + off + 2);
            const unsigned b[4] = {c01 & 255u, c01 >> 8, c23 & 255u, c23 >> 8};
            float v[4];
            if (DT == 8) {
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = d * (float)(int8_t)b[e];
            } else if (DT == 2) {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    v[e] = d * (float)((int)(j0 < 16 ? (b[e] & 15u) : (b[e] >> 4)) - 8);
            } else {
                const double dm = (double)half_u16(*reinterpret_cast<const unsigned short*>(p + 2));
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const double dq = (double)d * (double)(j0 < 16 ? (b[e] & 15u) : (b[e] >> 4));
                    v[e] = (float)(dq - dm);
                }
            }
            o = make_float4(v[0], v[1], v[2], v[3]);
        }
        reinterpret_cast<float4*>(out)[t] = o;
    }
    // the last n % 4 elements lie past the whole blocks (n % 4 <= n % 32)
    for (int64_t j = n4 * 4 + tid; j < n; j += stride) out[j] = 0.0f;
}

unsigned grid_for(Ctx* c, int64_t work) {
    int64_t g = (work + kI4Block - 1) / kI4Block;
    const int64_t cap = (int64_t)c->num_cus * 8;
    if (g > cap) g = cap;
    return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace

int launch_int4_quantize(Ctx* c, const float* src, int64_t rows, int64_t cols, int64_t gs,
                         bool asym, void* packed, bool out32, float* scales, int64_t* zps) {
    const int64_t groups = rows * (cols / gs);
    if (groups <= 0) return TKV_HIP_OK;
    const unsigned gg = grid_for(c, groups * 64);
#define TKV_QUANT4(AS, O32)                                                                   \
    hipLaunchKernelGGL((k_int4_quantize<AS, O32>), dim3(gg), dim3(kI4Block), 0, c->stream, src, \
                       rows, cols, gs, scales, zps, packed)
    if (asym && out32)
        TKV_QUANT4(true, true);
    else if (asym)
        TKV_QUANT4(true, false);
    else if (out32)
        TKV_QUANT4(false, true);
    else
        TKV_QUANT4(false, false);
#undef TKV_QUANT4
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_int4_dequantize(Ctx* c, const void* packed, bool in32, int64_t rows, int64_t cols,
                           int64_t gs, const float* scales, const int64_t* zps, float* dst) {
    const int64_t work = rows * (cols / 2);
    if (work <= 0) return TKV_HIP_OK;
    const unsigned g = grid_for(c, work);
#define TKV_UNPACK(AS, I32)                                                                    \
    hipLaunchKernelGGL((k_int4_unpack<AS, I32>), dim3(g), dim3(kI4Block), 0, c->stream, packed, \
                       rows, cols, gs, scales, zps, dst)
    if (zps && in32)
        TKV_UNPACK(true, true);
    else if (zps)
        TKV_UNPACK(true, false);
    else if (in32)
        TKV_UNPACK(false, true);
    else
        TKV_UNPACK(false, false);
#undef TKV_UNPACK
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_permute_cols(Ctx* c, const float* src, int64_t rows, int64_t cols, const int64_t* perm,
                        bool inverse, float* out) {
    if (rows * cols <= 0) return TKV_HIP_OK;
    const unsigned g = grid_for(c, rows * cols);
    if (inverse)
        hipLaunchKernelGGL(k_permute_cols<true>, dim3(g), dim3(kI4Block), 0, c->stream, src, rows,
                           cols, perm, out);
    else
        hipLaunchKernelGGL(k_permute_cols<false>, dim3(g), dim3(kI4Block), 0, c->stream, src, rows,
                           cols, perm, out);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_matmul_int4(Ctx* c, const float* a, const uint8_t* wp, const float* scales,
                       const float* bias, const int64_t* perm, float* y, int64_t m, int64_t n,
                       int64_t k, int64_t gs) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX || (n + kGBN - 1) / kGBN > INT32_MAX ||
        (m + kGBM - 1) / kGBM > 65535)
        return set_error(TKV_HIP_UNSUPPORTED, "matmul_int4_grouped: sizes beyond the grid");
    // Decode batches of 2..32 rows: 16-column workgroups on the f64 MFMA, K
    // split over workgroups until the grid is about three quarters of the
    // CUs, at least one k block per wave (one counter per column block).  A
    // single row takes the single-row kernel below.  Sweep over the four
    // GPT-2 shapes (us per call, HIP events, M = 1 / 4 / 16 / 32, per-column
    // kernel first): qkv 4.6 / 8.2 / 21.7 / 40.4 against 6.3 / 6.5 / 7.2 /
    // 10.3, mlp_down 8.7 / 20.0 / 55.6 / 108.4 against 9.2 / 9.3 / 10.0 /
    // 13.9 (4-wave workgroups).  With 8-wave workgroups, forced split counts
    // on mlp_down (48 column blocks) at M = 4 / 16 / 32: 4 splits 7.9 / 8.4 /
    // 11.1 us against 8.5 / 8.9 / 12.2 with 3, 9.6 / 10.2 / 13.0 with 8;
    // attn_out (24 k blocks) is capped at 3.
    if (m >= 2 && m <= kGemvRows && !perm && k % 32 == 0 && gs % 8 == 0 && aligned(a, 16) &&
        aligned(wp, 4) && tuned(c, TKV_HIP_TUNE_INT4_GEMV_WAVE) != 1) {
        const int64_t ncb = (n + 15) / 16, nkb = k / 32;
        int64_t splits = 1;
        if (ncb <= kGemvSplitBlocks && 2 * ncb < (int64_t)c->num_cus) {
            splits = ceil_div(3 * (int64_t)c->num_cus, 4 * ncb);
            if (splits > nkb / kDecWaves) splits = nkb / kDecWaves;
            if (splits < 1) splits = 1;
        }
        void* part = nullptr;
        const int mb = m <= 16 ? 1 : 2;
        if (splits > 1)
            TKV_RC_TRY(ctx_workspace(c, 12, (size_t)(ncb * splits) * mb * 256 * sizeof(double), &part));
        const unsigned grid = (unsigned)(ncb * splits);
        // Weight path (K % 256 == 0, 16-byte aligned codes; the context's
        // decode weight-path knob forces either): lines through LDS for two
        // row blocks without a K split, or K >= 2048.  Cold weights, one box,
        // two rounds, registers -> lines: qkv / mlp_up M = 32 9.25 / 9.10 ->
        // 8.76 / 8.64 us, mlp_down M = 16 / 32 9.50 / 11.10 -> 9.26 / 10.76;
        // attn_out (split) and the one-block launches at K = 768 within
        // +-0.1 us, mostly slower through LDS.
        const int64_t knob = tuned(c, TKV_HIP_TUNE_DECODE_DMA);
        const bool lines = k % 256 == 0 && aligned(wp, 16) &&
                           (knob == 1 || (knob < 0 && ((mb == 2 && splits == 1) || k >= 2048)));
        const unsigned lds = lines ? (unsigned)(2048 * (ceil_div(nkb, splits) / 8 + 2)) : 0u;
#define TKV_I4DEC(MBV, L)                                                                          \
    hipLaunchKernelGGL((k_gemv_int4_mfma<MBV, L>), dim3(grid), dim3(kDecWaves * 64), lds,           \
                       c->stream, a, wp, scales, bias, y, (int)m, (int)n, (int)k, (int)gs,          \
                       (int)splits, static_cast<double*>(part), c->gemv_arrivals)
        if (mb == 1) {
            if (lines) TKV_I4DEC(1, true); else TKV_I4DEC(1, false);
        } else {
            if (lines) TKV_I4DEC(2, true); else TKV_I4DEC(2, false);
        }
#undef TKV_I4DEC
        TKV_LAUNCH_CHECK();
        return TKV_HIP_OK;
    }
    // One row: one load step per 512 of K.  Against the per-column kernel
    // below (us per call, GPT-2 shapes): mlp_down (K = 3072) 8.8 -> 4.3-4.5,
    // the K = 768 shapes 4.5-5.4 -> 4.4-5.0.
    if (m == 1 && !perm && k % 8 == 0 && gs % 8 == 0 && aligned(a, 16) && aligned(wp, 4)) {
        const dim3 g((unsigned)((n + 3) / 4));
        switch (std::min<int64_t>(ceil_div(k, (int64_t)512), 6)) {
#define TKV_ROW(S)                                                                                 \
    case S:                                                                                        \
        hipLaunchKernelGGL(k_gemv_int4_row<S>, g, dim3(256), 0, c->stream, a, wp, scales, bias, y, \
                           (int)n, (int)k, (int)gs);                                               \
        break;
            TKV_ROW(1)
            TKV_ROW(2)
            TKV_ROW(3)
            TKV_ROW(4)
            TKV_ROW(5)
            default:
            TKV_ROW(6)
#undef TKV_ROW
        }
        TKV_LAUNCH_CHECK();
        return TKV_HIP_OK;
    }
    if (m <= kGemvRows && (perm || aligned(a, 8))) {
        const unsigned g = (unsigned)((n + 3) / 4);
#define TKV_GEMV(MM)                                                                              \
    if (m <= MM) {                                                                                \
        if (perm)                                                                                 \
            hipLaunchKernelGGL((k_gemv_int4_f64<MM, true>), dim3(g), dim3(256), 0, c->stream, a, \
                               wp, scales, bias, perm, y, (int)m, (int)n, (int)k, (int)gs);       \
        else                                                                                      \
            hipLaunchKernelGGL((k_gemv_int4_f64<MM, false>), dim3(g), dim3(256), 0, c->stream,   \
                               a, wp, scales, bias, perm, y, (int)m, (int)n, (int)k, (int)gs);    \
        TKV_LAUNCH_CHECK();                                                                       \
        return TKV_HIP_OK;                                                                        \
    }
        TKV_GEMV(1)
        TKV_GEMV(2)
        TKV_GEMV(4)
        TKV_GEMV(8)
        TKV_GEMV(16)
        TKV_GEMV(32)
#undef TKV_GEMV
    }
    const dim3 grid((unsigned)((n + kGBN - 1) / kGBN), (unsigned)((m + kGBM - 1) / kGBM));
    const bool vec = !perm && k > 0 && k % 8 == 0 && gs % 8 == 0 && aligned(a, 16) && aligned(wp, 4);
    // K split over workgroups (f64 partial tiles that k_int4_split_sum adds
    // in split order), at least 4 slices per split.  The split forms hold 3
    // workgroups per CU (LDS form 132 VGPRs and 40 KB LDS, register form 138
    // VGPRs), and one workgroup alone on a CU waits on its loads (LDS form:
    // 2.0 us per slice against 0.85 us of MFMA work), so:
    //  - at most one tile per CU: about 3 workgroups per CU, trimmed to a
    //    whole number of workgroups per CU (288 workgroups on 256 CUs ran
    //    mlp_down M = 64 in 27.3 us, 240 in 22.8 us);
    //  - more tiles: the split count minimising rounds of 3 workgroups per CU
    //    times slices per workgroup, +2% per split for the partial traffic.
    // Sweep of forced split counts over the four GPT-2 shapes (group size
    // 128, M = 33 .. 4096, LDS form): this rule is within 1.5% of the best
    // count on average; M = 64 mlp_down 188.9 -> 22.8 us, attn_out 48.6 ->
    // 14.7 us, M = 1024 mlp_down 213.4 -> 120.3 us.
    //   The unsplit group-scaled register form is faster per slice than any
    // split form, so with it a tile count of at least 8 per 32-wide slice of
    // K stays unsplit, unless the tiles overflow the CUs by less than a
    // quarter (then a few CUs would run two tiles while the rest idle).  The
    // same sweep on the current kernels (M = 64 .. 4096) put this within 1.0%
    // of the best count on average, 6.7% at worst (3.3% and 31% without it):
    // qkv M = 768 74.0 -> 64.0 us, M = 3072 250.0 -> 214.5 us, mlp_up M = 256
    // 40.2 -> 33.7 us; mlp_down (96 slices) splits up to 767 tiles.
    const int64_t tiles = (int64_t)grid.x * grid.y, nslices = ceil_div(k, (int64_t)kGBK);
    const int64_t ncu = c->num_cus, smax = nslices / 4;
    const int64_t mt = (int64_t)grid.y * kGBM, nt = (int64_t)grid.x * kGBN;
    const bool fact = vec && gs % 32 == 0;
    const bool fills = tiles <= ncu || tiles % ncu == 0 || tiles % ncu >= ncu / 4;
    int64_t splits = 1;
    if (fact && tiles >= 8 * nslices && fills) {
        splits = 1;
    } else if (smax >= 2 && tiles <= ncu) {
        splits = std::min(ceil_div(3 * ncu, tiles), smax);
        if (tiles * splits > ncu) splits = std::min(splits, tiles * splits / ncu * ncu / tiles);
    } else if (smax >= 2 && tiles < 16 * ncu) {
        double best = 1e300;
        for (int64_t s = 1; s <= std::min<int64_t>(smax, 16); s++) {
            const int64_t q = ceil_div(nslices, s), s2 = ceil_div(nslices, q);
            const double est = (double)ceil_div(tiles * s2, 3 * ncu) * (double)q * (1.0 + 0.02 * s2);
            if (est < best) best = est, splits = s2;
        }
    }
    // partial tiles beyond 256 MiB: fewer splits
    while (splits >= 2 && splits * mt * nt * (int64_t)sizeof(double) > ((int64_t)256 << 20)) splits--;
    if (splits >= 2) {
        const int64_t kchunk = ceil_div(nslices, splits) * kGBK;
        splits = ceil_div(k, kchunk);
        void* part;
        TKV_RC_TRY(ctx_workspace(c, 12, (size_t)(splits * mt * nt) * sizeof(double), &part));
        double* dp = static_cast<double*>(part);
        const dim3 sgrid(grid.x, grid.y, (unsigned)splits);
        if (perm)
            hipLaunchKernelGGL((k_matmul_int4_f64<true, true>), sgrid, dim3(256), 0, c->stream, a,
                               wp, scales, bias, perm, y, (int)m, (int)n, (int)k, (int)gs,
                               (int)kchunk, dp);
        else if (vec)
            hipLaunchKernelGGL((k_matmul_int4_regs<true>), sgrid, dim3(256), 0, c->stream, a, wp,
                               scales, bias, y, (int)m, (int)n, (int)k, (int)gs, (int)kchunk, dp);
        else
            hipLaunchKernelGGL((k_matmul_int4_f64<false, true>), sgrid, dim3(256), 0, c->stream, a,
                               wp, scales, bias, perm, y, (int)m, (int)n, (int)k, (int)gs,
                               (int)kchunk, dp);
        TKV_LAUNCH_CHECK();
        int64_t rblocks = ceil_div(m * n, (int64_t)256);
        if (rblocks > (int64_t)c->num_cus * 8) rblocks = (int64_t)c->num_cus * 8;
        hipLaunchKernelGGL(k_int4_split_sum, dim3((unsigned)rblocks), dim3(256), 0, c->stream, dp,
                           (int)splits, mt, nt, bias, y, (int)m, (int)n);
        TKV_LAUNCH_CHECK();
        return TKV_HIP_OK;
    }
    if (perm)
        hipLaunchKernelGGL((k_matmul_int4_f64<true>), grid, dim3(256), 0, c->stream, a, wp,
                           scales, bias, perm, y, (int)m, (int)n, (int)k, (int)gs);
    // The group-scaled form holds 32 more VGPRs (194: 2 workgroups per CU
    // instead of 3); unsplit it measured 4-6% faster at M = 8192 (qkv 553.6
    // -> 534.3, mlp_down 747.6 -> 704.3 us), split 1-3% slower, so only the
    // unsplit launch takes it.
    else if (fact)
        hipLaunchKernelGGL((k_matmul_int4_regs<false, true>), grid, dim3(256), 0, c->stream, a, wp,
                           scales, bias, y, (int)m, (int)n, (int)k, (int)gs, 0, nullptr);
    else if (vec)
        hipLaunchKernelGGL((k_matmul_int4_regs<false>), grid, dim3(256), 0, c->stream, a, wp,
                           scales, bias, y, (int)m, (int)n, (int)k, (int)gs, 0, nullptr);
    else
        hipLaunchKernelGGL((k_matmul_int4_f64<false>), grid, dim3(256), 0, c->stream, a, wp,
                           scales, bias, perm, y, (int)m, (int)n, (int)k, (int)gs);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_gguf_blocks(Ctx* c, const uint8_t* raw, int64_t n, int dtype, float* out) {
    if (n <= 0) return TKV_HIP_OK;
    // four outputs per thread: 27.7 -> 23.0 us for 28.3 M Q8_0 elements
    // (0.65 -> 0.78 of 8 TB/s)
    if (aligned(raw, 2) && aligned(out, 16)) {
        const unsigned g4 = grid_for(c, n / 4 > 0 ? n / 4 : 1);
        switch (dtype) {
            case 8:
                hipLaunchKernelGGL(k_gguf_blocks4<8>, dim3(g4), dim3(kI4Block), 0, c->stream, raw, n,
                                   out);
                break;
            case 2:
                hipLaunchKernelGGL(k_gguf_blocks4<2>, dim3(g4), dim3(kI4Block), 0, c->stream, raw, n,
                                   out);
                break;
            case 3:
                hipLaunchKernelGGL(k_gguf_blocks4<3>, dim3(g4), dim3(kI4Block), 0, c->stream, raw, n,
                                   out);
                break;
            default:
                return set_error(TKV_HIP_UNSUPPORTED, "gguf: only Q8_0, Q4_0 and Q4_1 blocks");
        }
        TKV_LAUNCH_CHECK();
        return TKV_HIP_OK;
    }
    const unsigned g = grid_for(c, n);
    switch (dtype) {
        case 8:
            hipLaunchKernelGGL(k_gguf_blocks<8>, dim3(g), dim3(kI4Block), 0, c->stream, raw, n, out);
            break;
        case 2:
            hipLaunchKernelGGL(k_gguf_blocks<2>, dim3(g), dim3(kI4Block), 0, c->stream, raw, n, out);
            break;
        case 3:
            hipLaunchKernelGGL(k_gguf_blocks<3>, dim3(g), dim3(kI4Block), 0, c->stream, raw, n, out);
            break;
        default:
            return set_error(TKV_HIP_UNSUPPORTED, "gguf: only Q8_0, Q4_0 and Q4_1 blocks");
    }
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int64_t gguf_block_bytes(int dtype) { return dtype == 8 ? 34 : dtype == 2 ? 18 : dtype == 3 ? 20 : 0; }

}  // namespace tkv
