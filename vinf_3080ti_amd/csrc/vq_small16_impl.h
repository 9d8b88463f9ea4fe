// vq_small16_impl.h -- matvec for a few tokens (1..16: speculative verify, small batches) on f16 MFMA, for the K-quants
// whose sub-block products fit f16 exactly (Q3_K, Q4_K, Q5_K; Q6_K as an f16 rounding plus remainder) and the IQ
// types with signed codes (IQ2_XXS/XS/S, IQ3_XXS; IQ3_S and IQ4_XS as an f16 rounding plus remainder).
//
// Numerics: those of the prefill path (vq_gemm16_impl.h). Each weight element is the integer a = code * sc
// (exact in f16: |a| <= 128 for Q3_K, 945 for Q4_K, 1953 for Q5_K; Q6_K's |(q - 32) * sc| <= 4096 goes in as
// its f16 rounding plus the exact remainder in {-1, 0, 1}, the remainder's b_lo product -- under ~1e-7 of the
// product -- left out), each activation element b = xq * xd * 2^e
// (the CPU path's int8 codes and group scale, one fp32 rounding, 2^e per token and K range) is two f16
// (b_hi + b_lo), and each super-block's C = sum a * (b_hi + b_lo) comes from v_mfma_f32_16x16x32_f16 (exact
// products, fp32 sums) before acc += d * C - 32 * dmin * (m . XS) once per super-block (qwen_cpu.c:581-641
// regrouped per super-block).
//
// Work split: workgroup (128-row block, K range of 512 columns) of 8 waves, one tile each (a persistent walk over
// row tiles with the next tile's slices prefetched measured slower, as did 16 waves, 1024-column ranges and
// weight bytes staged through LDS with 16-byte loads); wave w owns 16 rows and the whole range (two super-blocks), a 16-row x 16-token MFMA tile (tokens beyond ntok are zero lanes). At start each
// wave loads its rows' raw slices of both super-blocks (lane = (row, quarter of the super-block); the slice
// decoders of vq_slices.h), while the workgroup quantizes its slice of the fp32 activations (quantize_group,
// the CPU path's IEEE operations) and splits it into the f16 pair in LDS. Lane (row, q) decodes its quarter into
// 8 MFMA chunks of 8 elements; the B operand of lane (token, q) is the same 8 positions of that token. K ranges
// write partial sums [range][t][r] (scaled back from 2^e) that a second kernel adds in range order
// (deterministic).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_gemm16_impl.h"
#include "vq_qmv.h"
#include "vq_quant.h"
#include "vq_tables.h"

namespace vq {

// IQ types: signed int8 codes (grid magnitude x sign, or the IQ4_NL value) times an integer sub-block scale.
template <int T>
constexpr bool kS16Signed = T == VQ_IQ2_XXS || T == VQ_IQ2_XS || T == VQ_IQ2_S || T == VQ_IQ3_XXS || T == VQ_IQ3_S ||
                            T == VQ_IQ4_XS;
template <int T>
constexpr bool kSmall16 = T == VQ_Q3_K || T == VQ_Q4_K || T == VQ_Q5_K || T == VQ_Q6_K || kS16Signed<T>;
// Types whose element code * scale can exceed f16's exact integers (2048), so it goes in as two exact terms:
// Q6_K (|q - 32| <= 32, sc <= 127), IQ4_XS (|code| <= 127, |ls - 32| <= 32) and IQ3_S (its grid is replaceable:
// any magnitude up to 127, scale up to 31). The fixed IQ2 and IQ3_XXS grids stay below 64 (x 31 <= 1953).
template <int T>
constexpr bool kS16TwoTerm = T == VQ_Q6_K || T == VQ_IQ4_XS || T == VQ_IQ3_S;
// Those types' weight as its f16 rounding plus the remainder a - f16(a) in {-1, 0, 1} (three MFMAs per product,
// the remainder's b_lo product, under ~1e-7 of the product, left out), or as two exact terms (four MFMAs).
#ifndef VQ_S16_RSPLIT
#define VQ_S16_RSPLIT 1
#endif

constexpr int kS16Occ = 2;  // waves per SIMD the register budget is set for
constexpr int kS16Waves = 8, kS16Rows = 16 * kS16Waves, kS16KR = 512, kS16NSB = kS16KR / 256;
constexpr int kS16RowHalves = kS16KR + 8;  // f16 per token row of the activation image (16-byte pad)

// LDS of one workgroup for ntok tokens: b_hi, b_lo [ntok + 1][kS16RowHalves] f16, xs [ntok + 1][2][16] f16 (row
// ntok all zero: the B rows of the MFMA lanes past the last token), codes [ntok][kS16KR] int8, xd [ntok][KR/32]
// fp32, X [ntok][KR/32] int32, token scale [16] fp32.
__host__ __device__ inline size_t s16_lds(int ntok) {
    return static_cast<size_t>(ntok + 1) * (2 * kS16RowHalves * 2 + kS16NSB * 16 * 2) +
           static_cast<size_t>(ntok) * (kS16KR + (kS16KR / 32) * 4 * 2) + 64;
}
inline int s16_ranges(int cols) { return (cols + kS16KR - 1) / kS16KR; }
inline size_t s16_part_bytes(int rows, int cols, int ntok) {
    const int nkr = s16_ranges(cols);
    return nkr > 1 ? (static_cast<size_t>(nkr) * ntok * rows * 4 + 255) / 256 * 256 : 0;
}

// Up to four matrices of one type and width reading the same activations, in one launch: job j owns the row
// tiles [tile0[j], tile0[j + 1]) of the grid and writes out[j] (y, or its partial sums with several K ranges).
constexpr int kS16MaxJobs = 4;
struct S16Jobs {
    const uint8_t *w[kS16MaxJobs];
    float *out[kS16MaxJobs];
    int rows[kS16MaxJobs];
    int tile0[kS16MaxJobs + 1];
    int n;
};

// Eight codes (bytes of c0, c1) times the part's scale, as f16: exact for every type here.
template <int T>
__device__ __forceinline__ void s16_frag(uint32_t c0, uint32_t c1, int isc, g16h8 &a1, g16h8 &a2) {
    const g16h2 k = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    g16h2 v[4] = {g16_pair(c0, 0x04010400u), g16_pair(c0, 0x04030402u), g16_pair(c1, 0x04010400u),
                  g16_pair(c1, 0x04030402u)};  // 1024 + code
    if constexpr (T == VQ_Q4_K || T == VQ_Q5_K || T == VQ_Q2_K) {
        const _Float16 s = static_cast<_Float16>(isc);
        const g16h2 s2 = {s, s};
        const _Float16 nb = static_cast<_Float16>(-1024.0f) * s;  // exact: sc < 64
        const g16h2 n2 = {nb, nb};
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __builtin_elementwise_fma(v[i], s2, n2);  // code * sc in one rounding
        a1 = g16h8{v[0][0], v[0][1], v[1][0], v[1][1], v[2][0], v[2][1], v[3][0], v[3][1]};
    } else if constexpr (T == VQ_Q3_K) {
        const g16h2 off = {static_cast<_Float16>(1028.0f), static_cast<_Float16>(1028.0f)};
        const _Float16 s = static_cast<_Float16>(isc);
        const g16h2 s2 = {s, s};
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (v[i] - off) * s2;  // (code - 4) * (sc - 32): exact, |.| <= 128
        a1 = g16h8{v[0][0], v[0][1], v[1][0], v[1][1], v[2][0], v[2][1], v[3][0], v[3][1]};
    } else if constexpr (kS16Signed<T>) {
        // signed byte c: 1024 + (c ^ 0x80) - 1152 = c, exact; two terms c * 16 (sc >> 4) + c * (sc & 15) where
        // the product can leave f16's exact range (|c| <= 128: each term stays within it)
        const g16h2 off = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
        g16h2 q[4] = {g16_pair(c0 ^ 0x80808080u, 0x04010400u), g16_pair(c0 ^ 0x80808080u, 0x04030402u),
                      g16_pair(c1 ^ 0x80808080u, 0x04010400u), g16_pair(c1 ^ 0x80808080u, 0x04030402u)};
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = q[i] - off;
        if constexpr (kS16TwoTerm<T>) {
            g16h2 w1[4], w2[4];
#if VQ_S16_RSPLIT
            const _Float16 sc = static_cast<_Float16>(isc);
            const g16h2 s2 = {sc, sc};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                w1[i] = q[i] * s2;                                   // f16(c * sc)
                w2[i] = __builtin_elementwise_fma(q[i], s2, -w1[i]);  // c * sc - f16(c * sc) in {-1, 0, 1}: exact
            }
#else
            const _Float16 sh = static_cast<_Float16>(16 * (isc >> 4)), sl = static_cast<_Float16>(isc & 15);
            const g16h2 h2 = {sh, sh}, l2 = {sl, sl};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                w1[i] = q[i] * h2;  // multiple of 16, |.| <= 4096: exact
                w2[i] = q[i] * l2;  // |.| <= 1920: exact
            }
#endif
            a1 = g16h8{w1[0][0], w1[0][1], w1[1][0], w1[1][1], w1[2][0], w1[2][1], w1[3][0], w1[3][1]};
            a2 = g16h8{w2[0][0], w2[0][1], w2[1][0], w2[1][1], w2[2][0], w2[2][1], w2[3][0], w2[3][1]};
        } else {
            const _Float16 sc = static_cast<_Float16>(isc);
            const g16h2 s2 = {sc, sc};
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = q[i] * s2;  // |.| <= 63 * 31: exact
            a1 = g16h8{q[0][0], q[0][1], q[1][0], q[1][1], q[2][0], q[2][1], q[3][0], q[3][1]};
        }
    } else {  // Q6_K: (q - 32) * sc as f16(a) + (a - f16(a)), or as (q - 32) * 16 (sc >> 4) + (q - 32) * (sc & 15)
        const g16h2 off = {static_cast<_Float16>(1056.0f), static_cast<_Float16>(1056.0f)};
        g16h2 w1[4], w2[4];
#if VQ_S16_RSPLIT
        const _Float16 sc = static_cast<_Float16>(isc);
        const g16h2 s2 = {sc, sc};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const g16h2 q = v[i] - off;                       // q - 32, exact
            w1[i] = q * s2;                                   // f16(a)
            w2[i] = __builtin_elementwise_fma(q, s2, -w1[i]);  // a - f16(a), exact
        }
#else
        const _Float16 sh = static_cast<_Float16>(16 * (isc >> 4)), sl = static_cast<_Float16>(isc & 15);
        const g16h2 h2 = {sh, sh}, l2 = {sl, sl};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const g16h2 q = v[i] - off;  // q - 32, exact
            w1[i] = q * h2;              // multiple of 16, |.| <= 4096: exact
            w2[i] = q * l2;              // |.| <= 480: exact
        }
#endif
        a1 = g16h8{w1[0][0], w1[0][1], w1[1][0], w1[1][1], w1[2][0], w1[2][1], w1[3][0], w1[3][1]};
        a2 = g16h8{w2[0][0], w2[0][1], w2[1][0], w2[1][1], w2[2][0], w2[2][1], w2[3][0], w2[3][1]};
    }
    (void)k;
}

__device__ __forceinline__ void s16_opaque(float &v) { asm volatile("" : "+v"(v)); }

// Staged activations (the megakernel's QMV flags, qwen_megakernel.cu:468-551): v = silu(x) * x2 with SILU_MUL, then
// v * (rs[t] * nw[c]) with NORM, rs[t] = 1 / sqrt(mean(v^2) + eps) from s16_rms_kernel, before quantization; ADD
// adds y's previous value to the result (in the K-range sum when there are several ranges). silu(z) = z / (1 +
// e^-z) with the hardware exp2 and reciprocal, as the streaming kernel's staging.
__device__ __forceinline__ float s16_silu(float z) {
    return z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}

// rs[t] = 1 / sqrt(sum_c v[t][c]^2 / cols + eps) of the staged (silu_mul-ed) values: one 256-thread workgroup per
// token, float4 per thread and step, then a fixed-order tree; deterministic.
__global__ __launch_bounds__(256) inline void s16_rms_kernel(const float *__restrict__ x, XStage xs, int cols,
                                                             float *__restrict__ rs) {
    __shared__ float red[256];
    const int t = blockIdx.x;
    const float4 *xr = reinterpret_cast<const float4 *>(x + static_cast<size_t>(t) * cols);
    const float4 *mr = reinterpret_cast<const float4 *>(xs.x2 + static_cast<size_t>(t) * cols);
    const bool silu = (xs.flags & VQ_STAGE_SILU_MUL) != 0;
    float acc = 0.0f;
    for (int i = threadIdx.x; i < cols / 4; i += 256) {
        float4 f = xr[i];
        if (silu) {
            const float4 m = mr[i];
            f = float4{s16_silu(f.x) * m.x, s16_silu(f.y) * m.y, s16_silu(f.z) * m.z, s16_silu(f.w) * m.w};
        }
        acc = fmaf(f.x, f.x, acc);
        acc = fmaf(f.y, f.y, acc);
        acc = fmaf(f.z, f.z, acc);
        acc = fmaf(f.w, f.w, acc);
    }
    red[threadIdx.x] = acc;
    for (int h = 128; h > 0; h >>= 1) {
        __syncthreads();
        if (static_cast<int>(threadIdx.x) < h) red[threadIdx.x] += red[threadIdx.x + h];
    }
    if (threadIdx.x == 0) rs[t] = 1.0f / sqrtf(red[0] / static_cast<float>(cols) + xs.eps);
}

// STG: the staged instance (vq_qmv_staged_ws); the plain one compiles without the staging code (with it, the
// plain batch-8 MLP block measured 95 -> 119 us: the compiler's load scheduling and registers change).
template <int T, bool STG>
__global__ __launch_bounds__(64 * kS16Waves, kS16Occ) void qmv16_kernel(const S16Jobs J, int cols, long row_bytes,
                                                              const float *__restrict__ x, int ntok, const XStage xs,
                                                              const float *__restrict__ rs) {
    using S = Sl<T>;
    constexpr int SPL = S::SPB / 4;  // slices per lane per super-block: a lane owns a quarter of it
    constexpr int NP = S::NP;
    constexpr bool MIN = kHasMin<T>;
    static_assert(SPL * NP * 16 == 64, "a quarter super-block per lane");
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    _Float16 *const xh = reinterpret_cast<_Float16 *>(s_dyn);
    _Float16 *const xl = xh + (ntok + 1) * kS16RowHalves;
    _Float16 *const xsd = xl + (ntok + 1) * kS16RowHalves;                      // [t][sb][16]
    int8_t *const xq = reinterpret_cast<int8_t *>(xsd + (ntok + 1) * kS16NSB * 16);  // [t][KR]
    float *const xdg = reinterpret_cast<float *>(xq + ntok * kS16KR);    // [t][KR/32]
    int *const xsum = reinterpret_cast<int *>(xdg + ntok * (kS16KR / 32));  // [t][KR/32]
    float *const tsc = reinterpret_cast<float *>(xsum + ntok * (kS16KR / 32));  // [16]

    __shared__ uint2 s8[TabSpec<T>::n8 > 0 ? TabSpec<T>::n8 : 1];  // IQ grids (staged before the first barrier)
    __shared__ uint32_t s4[TabSpec<T>::n4 > 0 ? TabSpec<T>::n4 : 1];
    __shared__ uint2 sks[TabSpec<T>::ks ? 128 : 1], ssm[TabSpec<T>::sm ? 256 : 1];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lr = lane & 15, lk = lane >> 4;
    const Tabs tabs = stage_tabs<T>(s8, s4, sks, ssm);
    int jb = 0;
    while (jb + 1 < J.n && static_cast<int>(blockIdx.x) >= J.tile0[jb + 1]) ++jb;
    const uint8_t *const w = J.w[jb];
    float *const out = J.out[jb];
    const int rows = J.rows[jb];
    const int kr = blockIdx.y, k0 = kr * kS16KR;
    const int kw = cols - k0 < kS16KR ? cols - k0 : kS16KR;  // a multiple of 256
    const int nsb = kw >> 8, sbg0 = k0 >> 8;
    const int ngr = kw >> 5;

    // 1. This lane's raw slices of the workgroup's row tile: row 16 wv + lr of it, quarter lk of each super-block
    // of the range (issued first, in flight while the activations are quantized).
    auto load_tile = [&](int tile, typename S::W (&wr)[kS16NSB][SPL]) {
        const int row = min(tile * kS16Rows + 16 * wv + lr, rows - 1);
        const uint8_t *const wrow = w + static_cast<size_t>(row) * row_bytes + static_cast<size_t>(sbg0) * S::UB;
#pragma unroll
        for (int sb = 0; sb < kS16NSB; ++sb)
#pragma unroll
            for (int si = 0; si < SPL; ++si) S::load(wrow + (sb < nsb ? sb : 0) * S::UB, SPL * lk + si, wr[sb][si]);
    };
    // The activation group this thread quantizes (at most one: 16 tokens x KR/32 groups fit the workgroup),
    // loaded before the weights: loads return in order, and waiting for it behind the weight burst would
    // serialize the two.
    static_assert(16 * (kS16KR / 32) <= 64 * kS16Waves, "one activation group per thread");
    const bool has_group = tid < ntok * ngr;
    const int gt = has_group ? tid / ngr : 0, gg = has_group ? tid - gt * ngr : 0;
    float v[32];
    const bool st_silu = STG && (xs.flags & VQ_STAGE_SILU_MUL) != 0, st_norm = STG && (xs.flags & VQ_STAGE_NORM) != 0;
    float m2[32], nwv[32];  // staging inputs, loaded before the weights like x
    if (has_group) {
        const size_t off = static_cast<size_t>(gt) * cols + k0 + 32 * gg;
        const float4 *src = reinterpret_cast<const float4 *>(x + off);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 f = src[q];
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
        if (st_silu) {
            const float4 *s2 = reinterpret_cast<const float4 *>(xs.x2 + off);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 f = s2[q];
                m2[4 * q] = f.x;
                m2[4 * q + 1] = f.y;
                m2[4 * q + 2] = f.z;
                m2[4 * q + 3] = f.w;
            }
        }
        if (st_norm) {
            const float4 *sn = reinterpret_cast<const float4 *>(xs.nw + k0 + 32 * gg);
            const float r = rs[gt];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 f = sn[q];
                nwv[4 * q] = r * f.x;
                nwv[4 * q + 1] = r * f.y;
                nwv[4 * q + 2] = r * f.z;
                nwv[4 * q + 3] = r * f.w;
            }
        }
    }
    const int tile = blockIdx.x - J.tile0[jb];
    typename S::W wr[kS16NSB][SPL];
    load_tile(tile, wr);
    if (has_group && st_silu) {
#pragma unroll
        for (int k = 0; k < 32; ++k) v[k] = s16_silu(v[k]) * m2[k];
    }
    if (has_group && st_norm) {
#pragma unroll
        for (int k = 0; k < 32; ++k) v[k] *= nwv[k];  // v * (rs * nw), as the streaming kernel's staging
    }

    // 2. The activation slice: int8 codes per 32-group (the CPU path's quantize_group), then per token the
    // power of two 2^e with 127 max(xd) 2^e < 2^15, then b = xq * (xd 2^e) split into two f16.
    for (int i = tid; i < kS16KR / 4; i += blockDim.x) {  // the zero token row (8 bytes of b_hi, b_lo each)
        *reinterpret_cast<uint2 *>(xh + ntok * kS16RowHalves + 4 * i) = uint2{0u, 0u};
        *reinterpret_cast<uint2 *>(xl + ntok * kS16RowHalves + 4 * i) = uint2{0u, 0u};
    }
    if (tid < kS16NSB * 16 / 2) reinterpret_cast<uint32_t *>(xsd + ntok * kS16NSB * 16)[tid] = 0u;
    if (has_group) {
        const QGroup qg = quantize_group(v);
        uint4 *dq = reinterpret_cast<uint4 *>(xq + gt * kS16KR + 32 * gg);
        dq[0] = uint4{qg.q[0], qg.q[1], qg.q[2], qg.q[3]};
        dq[1] = uint4{qg.q[4], qg.q[5], qg.q[6], qg.q[7]};
        xdg[gt * (kS16KR / 32) + gg] = qg.d;
        xsum[gt * (kS16KR / 32) + gg] = qg.hs0 + qg.hs1;
    }
    __syncthreads();
    if (tid < ntok) {
        float m = 0.0f;
        for (int g = 0; g < ngr; ++g) m = fmaxf(m, xdg[tid * (kS16KR / 32) + g]);
        int E = 0;
        (void)frexpf(127.0f * m, &E);
        tsc[tid] = m > 0.0f ? ldexpf(1.0f, min(15 - E, 126)) : 1.0f;  // capped: finite for tiny tokens
    }
    __syncthreads();
    for (int i = tid; i < ntok * (kw / 4); i += blockDim.x) {
        const int t = i / (kw / 4), c = 4 * (i - t * (kw / 4));
        const float ds = xdg[t * (kS16KR / 32) + (c >> 5)] * tsc[t];
        const uint32_t q4 = *reinterpret_cast<const uint32_t *>(xq + t * kS16KR + c);
        _Float16 h[4], l[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v = static_cast<float>(static_cast<int8_t>(q4 >> (8 * j))) * ds;
            s16_opaque(v);  // the split of the fp32 product (no contraction into a mixed-precision fma)
            h[j] = static_cast<_Float16>(v);
            l[j] = static_cast<_Float16>(v - static_cast<float>(h[j]));
        }
        *reinterpret_cast<uint2 *>(xh + t * kS16RowHalves + c) = __builtin_bit_cast(uint2, h);
        *reinterpret_cast<uint2 *>(xl + t * kS16RowHalves + c) = __builtin_bit_cast(uint2, l);
    }
    if constexpr (MIN) {
        for (int i = tid; i < ntok * ngr; i += blockDim.x) {
            const int t = i / ngr, g = i - t * ngr;
            float v = static_cast<float>(xsum[t * (kS16KR / 32) + g]) * (xdg[t * (kS16KR / 32) + g] * tsc[t]) * 0.03125f;
            s16_opaque(v);
            const _Float16 hi = static_cast<_Float16>(v);
            xsd[(t * kS16NSB + (g >> 3)) * 16 + (g & 7)] = hi;
            xsd[(t * kS16NSB + (g >> 3)) * 16 + 8 + (g & 7)] = static_cast<_Float16>(v - static_cast<float>(hi));
        }
    }
    __syncthreads();

    // 3. Per super-block: 8 chunks x (b_hi, b_lo) MFMAs (Q6_K: both weight terms), the min MFMA, the scaling.
    // C element j is row 4 lk + j of the wave's 16, token lr.
    const bool tok_ok = lr < ntok;
    const int tb = tok_ok ? lr : ntok;  // the zero row
    const float is = 1.0f / tsc[tok_ok ? lr : 0];
    float *const o = out + (static_cast<size_t>(kr) * ntok + (tok_ok ? lr : 0)) * rows;
    g16f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sb = 0; sb < kS16NSB; ++sb) {
        if (sb >= nsb) break;
        g16f4 C = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int si = 0; si < SPL; ++si) {
            const int sl = SPL * lk + si;
            uint32_t cd[NP][4];
            S::codes(wr[sb][si], sl, tabs, cd);
            int isc[NP];
            S::iscales(wr[sb][si], sl, isc);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                int pg, ph;
                S::part(sl, p, pg, ph);
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    g16h8 a1, a2;
                    s16_frag<T>(cd[p][2 * hf], cd[p][2 * hf + 1], isc[p], a1, a2);
                    // this lane's 8 positions of the chunk: pg, ph, hf of its own slice; the B lanes (token, lk)
                    // of the same lk take the same positions
                    const int e = 256 * sb + 32 * pg + 16 * ph + 8 * hf;
                    g16h8 bh = *reinterpret_cast<const g16h8 *>(xh + tb * kS16RowHalves + e);
                    g16h8 bl = *reinterpret_cast<const g16h8 *>(xl + tb * kS16RowHalves + e);
                    C = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bh, C, 0, 0, 0);
                    C = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bl, C, 0, 0, 0);
                    if constexpr (kS16TwoTerm<T>) {
                        C = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, bh, C, 0, 0, 0);
                        if constexpr (!VQ_S16_RSPLIT) C = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, bl, C, 0, 0, 0);
                    }
                }
            }
        }
        // d (and dmin) of the C rows: row 4 lk + j's values sit in lane 4 lk + j (lk = 0 there).
        const float dmy = S::dmul(wr[sb][0]);
        float dmn = 0.0f;
        if constexpr (MIN) dmn = 32.0f * S::dmin(wr[sb][0]);
        g16f4 cm = {0.f, 0.f, 0.f, 0.f};
        if constexpr (MIN) {
            // A_min: row lr, k = 4 lk .. +4 -> mins of groups 4 (lk & 1) .. +4 (k4_scale_min packing, qwen_cpu.c:54-62)
            const uint32_t hy = wr[sb][0].hd[1], hz = wr[sb][0].hd[2], hw = wr[sb][0].hd[3];
            const uint32_t mw = (lk & 1) ? (((hw >> 4) & 0x0F0F0F0Fu) | ((hz >> 2) & 0x30303030u)) : (hz & 0x3F3F3F3Fu);
            const g16h2 k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
            const g16h2 m01 = g16_pair(mw, 0x04010400u) - k1024, m23 = g16_pair(mw, 0x04030402u) - k1024;
            const g16h4 am = {m01[0], m01[1], m23[0], m23[1]};
            const g16h4 bm = *reinterpret_cast<const g16h4 *>(xsd + (tb * kS16NSB + sb) * 16 + 4 * lk);
            cm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, cm, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float dj = __shfl(dmy, 4 * lk + j, 64);
            const float mj = MIN ? __shfl(dmn, 4 * lk + j, 64) : 0.0f;
            acc[j] = fmaf(dj, C[j], fmaf(-mj, cm[j], acc[j]));
        }
    }

    // 4. Out: rows 16 wv + 4 lk + j of the tile for token lr, back from the token's 2^e (partials of K range kr
    // when the columns span several ranges).
    if (tok_ok) {
        const bool add = STG && (xs.flags & VQ_STAGE_ADD) != 0 && kw == cols;  // one K range: o is y itself
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = tile * kS16Rows + 16 * wv + 4 * lk + j;
            if (r < rows) o[r] = add ? acc[j] * is + o[r] : acc[j] * is;
        }
    }
}

// y = sum of the K ranges' partials, in range order; four outputs per thread (n % 4 == 0), loads four ranges ahead.
__global__ __launch_bounds__(256) inline void s16_sum_kernel(const float *__restrict__ part, int nkr, long n,
                                                            float *__restrict__ y) {
    const long i = (static_cast<long>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const float4 *p = reinterpret_cast<const float4 *>(part + i);
    const long st = n / 4;
    float4 v = p[0];
    int k = 1;
    for (; k + 4 <= nkr; k += 4) {
        const float4 a = p[k * st], b = p[(k + 1) * st], c = p[(k + 2) * st], d = p[(k + 3) * st];
        v.x += a.x, v.y += a.y, v.z += a.z, v.w += a.w;
        v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
        v.x += c.x, v.y += c.y, v.z += c.z, v.w += c.w;
        v.x += d.x, v.y += d.y, v.z += d.z, v.w += d.w;
    }
    for (; k < nkr; ++k) {
        const float4 a = p[k * st];
        v.x += a.x, v.y += a.y, v.z += a.z, v.w += a.w;
    }
    *reinterpret_cast<float4 *>(y + i) = v;
}

// The same, one output per thread (any n).
__global__ __launch_bounds__(256) inline void s16_sum1_kernel(const float *__restrict__ part, int nkr, long n,
                                                             float *__restrict__ y, bool add) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    float v = part[i];
    for (int k = 1; k < nkr; ++k) v += part[static_cast<size_t>(k) * n + i];
    y[i] = add ? v + y[i] : v;
}

// The K-range sums of several jobs in one launch: job j's n[j] outputs (a multiple of 4) are the float4
// elements [e0[j], e0[j + 1]) of the grid; each is summed as s16_sum_kernel does.
struct S16Sum {
    const float *part[kS16MaxJobs];
    float *y[kS16MaxJobs];
    long n[kS16MaxJobs];
    long e0[kS16MaxJobs + 1];
    int jobs;
};
__global__ __launch_bounds__(256) inline void s16_sum_jobs_kernel(S16Sum P, int nkr, bool add) {
    const long e = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (e >= P.e0[P.jobs]) return;
    int jb = 0;
    while (jb + 1 < P.jobs && e >= P.e0[jb + 1]) ++jb;
    const long i = (e - P.e0[jb]) * 4, n = P.n[jb];
    const float4 *p = reinterpret_cast<const float4 *>(P.part[jb] + i);
    const long st = n / 4;
    float4 v = p[0];
    int k = 1;
    for (; k + 4 <= nkr; k += 4) {
        const float4 a = p[k * st], b = p[(k + 1) * st], c = p[(k + 2) * st], d = p[(k + 3) * st];
        v.x += a.x, v.y += a.y, v.z += a.z, v.w += a.w;
        v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
        v.x += c.x, v.y += c.y, v.z += c.z, v.w += c.w;
        v.x += d.x, v.y += d.y, v.z += d.z, v.w += d.w;
    }
    for (; k < nkr; ++k) {
        const float4 a = p[k * st];
        v.x += a.x, v.y += a.y, v.z += a.z, v.w += a.w;
    }
    float4 *const dst = reinterpret_cast<float4 *>(P.y[jb] + i);
    if (add) {  // ADD staging flag: the sum of the ranges plus y's previous value
        const float4 o = *dst;
        v.x += o.x, v.y += o.y, v.z += o.z, v.w += o.w;
    }
    *dst = v;
}

// n <= kS16MaxJobs matrices of type T sharing cols and x: one qmv16 launch over all their row tiles, then one
// launch of K-range sums (several K ranges: `part` holds the sum of s16_part_bytes(rows[j], cols, ntok)).
template <int T>
int launch_small16_group(int n, const uint8_t *const *w, const int *rows, float *const *y, int cols, long rb,
                         const float *x, int ntok, float *part, hipStream_t s, const XStage &xs, float *rs) {
    if constexpr (!kSmall16<T>) {
        (void)n, (void)w, (void)rows, (void)y, (void)cols, (void)rb, (void)x, (void)ntok, (void)part, (void)s;
        (void)xs, (void)rs;
        return static_cast<int>(hipErrorInvalidValue);
    } else {
        if ((xs.flags & VQ_STAGE_NORM) && rs == nullptr) return static_cast<int>(hipErrorInvalidValue);
        if (n < 1 || n > kS16MaxJobs || ntok < 1 || ntok > 16 || cols % 256 != 0)
            return static_cast<int>(hipErrorInvalidValue);
        const int nkr = s16_ranges(cols);
        if (nkr > 1 && part == nullptr) return static_cast<int>(hipErrorInvalidValue);
        S16Jobs J{};
        J.n = n;
        J.tile0[0] = 0;
        uint8_t *pp = reinterpret_cast<uint8_t *>(part);
        for (int k = 0; k < n; ++k) {
            J.w[k] = w[k];
            J.rows[k] = rows[k];
            J.out[k] = nkr > 1 ? reinterpret_cast<float *>(pp) : y[k];
            if (nkr > 1) pp += s16_part_bytes(rows[k], cols, ntok);
            J.tile0[k + 1] = J.tile0[k] + (rows[k] + kS16Rows - 1) / kS16Rows;
        }
        if (xs.flags & VQ_STAGE_NORM) {
            s16_rms_kernel<<<dim3(ntok), dim3(256), 0, s>>>(x, xs, cols, rs);
            const hipError_t e0 = hipGetLastError();
            if (e0 != hipSuccess) return static_cast<int>(e0);
        }
        const bool add = (xs.flags & VQ_STAGE_ADD) != 0;
        const dim3 grid(J.tile0[n], nkr), block(64 * kS16Waves);
        if (xs.flags != 0)
            qmv16_kernel<T, true><<<grid, block, s16_lds(ntok), s>>>(J, cols, rb, x, ntok, xs, rs);
        else
            qmv16_kernel<T, false><<<grid, block, s16_lds(ntok), s>>>(J, cols, rb, x, ntok, xs, rs);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || nkr == 1) return static_cast<int>(e);
        bool vec = true;
        for (int k = 0; k < n; ++k)
            vec = vec && (static_cast<long>(ntok) * rows[k]) % 4 == 0 &&
                  (reinterpret_cast<uintptr_t>(J.out[k]) | reinterpret_cast<uintptr_t>(y[k])) % 16 == 0;
        if (vec) {
            S16Sum P{};
            P.jobs = n;
            P.e0[0] = 0;
            for (int k = 0; k < n; ++k) {
                P.part[k] = J.out[k];
                P.y[k] = y[k];
                P.n[k] = static_cast<long>(ntok) * rows[k];
                P.e0[k + 1] = P.e0[k] + P.n[k] / 4;
            }
            s16_sum_jobs_kernel<<<static_cast<unsigned>((P.e0[n] + 255) / 256), 256, 0, s>>>(P, nkr, add);
        } else {
            for (int k = 0; k < n; ++k) {
                const long m = static_cast<long>(ntok) * rows[k];
                s16_sum1_kernel<<<static_cast<unsigned>((m + 255) / 256), 256, 0, s>>>(J.out[k], nkr, m, y[k], add);
            }
        }
        e = hipGetLastError();
        return e == hipSuccess ? 0 : static_cast<int>(e);
    }
}

template <int T>
int launch_small16(const uint8_t *w, int rows, int cols, long rb, const float *x, int ntok, float *y, float *part,
                   hipStream_t s, const XStage &xs, float *rs) {
    return launch_small16_group<T>(1, &w, &rows, &y, cols, rb, x, ntok, part, s, xs, rs);
}

}  // namespace vq
