// vq_mfma_impl.h -- small-batch quantized matvec on int8 MFMA: y[t][r] = W[r] . x[t] for 2..16 tokens.
//
// The batch-1 streaming kernel (vq_qmv_impl.h) repeats the per-token dot products and scaling in VALU, so
// its cost grows with the token count. Here the dot products run on v_mfma_i32_16x16x32_i8 with the
// tokens' int8 activations as the A operand (16 tokens, zero beyond ntok) and a 16-row block of decoded
// weight codes as the B operand; only the per-(token, row, 32-group) fp32 scaling stays in VALU, where one
// lane owns one row:
//   C[t][r] = sum over the group of x_code[t] * w_code[r]   (exact int32)
//   acc[t]  += C * (sc_r * xd_t) - mn_r * (X_t * xd_t)       (per 16-half for per-16-scale types)
// Same quantized numerics as the matvec (activations from vq_pack_x, codes and scales from the slice
// decoders of vq_slices.h); only the summation order differs.
//
// Work split: wave = one 16-row block x one K range. A workgroup holds R waves on consecutive row blocks
// and one K range (blockIdx.y of S): it stages the tokens' activation image for that range in LDS once.
// Each wave walks its range 256 elements at a time with the raw weight slices of the next steps already
// loaded into registers; a step's slices are decoded into a wave-private LDS tile (signed int8 codes
// [row][k] and scales per row and 16-part) and contracted. With S > 1 every K range writes its partial
// sums to part[s][t][r] and a second kernel adds the S partials in a fixed order (deterministic).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_gemm_impl.h"
#include "vq_gemm16_impl.h"
#include "vq_gemm16n_impl.h"
#include "vq_small16_impl.h"
#include "vq_qmv.h"
#include "vq_tables.h"

namespace vq {

constexpr int kMfmaRowWaves = 4;  // waves (16-row blocks) per workgroup
constexpr int kMfmaPF = 1;        // steps of raw weight slices in flight per wave (besides the one decoded)
constexpr int kMfmaXMax = 48 * 1024;

template <int T>
struct MfmaStep {
    using S = Sl<T>;
    static constexpr int UPS = 256 / (32 * S::UG);          // units per step
    static constexpr int SLJ = 16 * UPS * S::SPB / 64;      // slices per lane per step
    static constexpr int NG = 8;                            // 32-groups per step
    static_assert((16 * UPS * S::SPB) % 64 == 0, "slice split");
};

// Activation image of one K range (kw columns, a multiple of 256) for the ntok tokens: codes [t][kw + 16]
// (t < ntok), then per group g: xd[g][16 tokens], xs[g][2 halves][16 tokens] (xs = X * xd; zero beyond ntok).
struct MfmaX {
    int kw, stride, codes_bytes, xd_off, xs_off, bytes;
    __host__ __device__ MfmaX(int kw_, int ntok)
        : kw(kw_), stride(kw_ + 16), codes_bytes(ntok * (kw_ + 16)), xd_off((ntok * (kw_ + 16) + 15) / 16 * 16),
          xs_off((ntok * (kw_ + 16) + 15) / 16 * 16 + (kw_ / 32) * 16 * 4),
          bytes((ntok * (kw_ + 16) + 15) / 16 * 16 + (kw_ / 32) * 16 * 4 * 3) {}
};

template <int T>
__global__ __launch_bounds__(64 * kMfmaRowWaves) void qmv_mfma_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                                      long row_bytes, const float *__restrict__ x,
                                                                      int ntok, int kw, float *__restrict__ y,
                                                                      float *__restrict__ part) {
    using S = Sl<T>;
    using G = MfmaStep<T>;
    constexpr int NP = S::NP, SPB = S::SPB, UB = S::UB, UG = S::UG, UPS = G::UPS, SLJ = G::SLJ;
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    __shared__ __attribute__((aligned(16))) uint8_t s_codes[kMfmaRowWaves][16 * kGemmRowPad];
    __shared__ float s_sc[kMfmaRowWaves][16][16], s_mn[kMfmaRowWaves][16][16];
    __shared__ uint2 s8[TabSpec<T>::n8 > 0 ? TabSpec<T>::n8 : 1];
    __shared__ uint32_t s4[TabSpec<T>::n4 > 0 ? TabSpec<T>::n4 : 1];
    __shared__ uint2 sks[TabSpec<T>::ks ? 128 : 1];
    __shared__ uint2 ssm[TabSpec<T>::sm ? 256 : 1];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ng = cols >> 5, nu = ng / UG;
    const int k0 = blockIdx.y * kw;                   // first column of this K range
    const int kend = min(k0 + kw, cols);
    const MfmaX xi(kw, ntok);
    const int r0 = (blockIdx.x * kMfmaRowWaves + wv) * 16;
    const Tabs tb = stage_tabs<T>(s8, s4, sks, ssm);

    // This wave's steps: units [u_beg, u_end) of each of its 16 rows.
    const int u_beg = k0 / (32 * UG), u_end = min(kend / (32 * UG), nu);
    const int nsteps = (u_end - u_beg + UPS - 1) / UPS;
    uint8_t *ct = s_codes[wv];
    auto slice_of = [&](int j, int &rl, int &us, int &ss) {
        const int q = lane + 64 * j;
        ss = q % SPB;
        us = (q / SPB) % UPS;
        rl = q / (SPB * UPS);
    };
    typename S::W wr[kMfmaPF + 1][SLJ];
    auto load = [&](int st, typename S::W(&dst)[SLJ]) {
#pragma unroll
        for (int j = 0; j < SLJ; ++j) {
            int rl, us, ss;
            slice_of(j, rl, us, ss);
            const int r = min(r0 + rl, rows - 1);
            const int u = min(u_beg + st * UPS + us, nu - 1);
            S::load(w + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(u) * UB, ss, dst[j]);
        }
    };

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // tokens 4*(lane/16)+j, row lane%16
    const int lr = lane & 15, lk = lane >> 4;
    // The first weight slices are requested before the activation image is staged, so both round trips
    // overlap.
#pragma unroll
    for (int p = 0; p < kMfmaPF; ++p)
        if (p < nsteps) load(p, wr[p]);
    // Activation image of this K range, quantized here from the fp32 input (the CPU path's quantize_group per
    // 32-group, qwen_cpu.c:607-627, as vq_pack_x does): codes, scales, half sums times scale; zero past the
    // matrix's last column and for tokens ntok..15.
    const int ngk = kw >> 5;
    for (int i = tid; i < 16 * ngk; i += blockDim.x) {
        const int t = i / ngk, g = i - t * ngk;
        const int c = k0 + 32 * g;
        u32x4 q0{0u, 0u, 0u, 0u}, q1{0u, 0u, 0u, 0u};
        float xd = 0.0f, x0 = 0.0f, x1 = 0.0f;
        if (t < ntok && c < kend) {
            const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<size_t>(t) * cols + c);
            float v[32];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float4 f = src[k];
                v[4 * k] = f.x;
                v[4 * k + 1] = f.y;
                v[4 * k + 2] = f.z;
                v[4 * k + 3] = f.w;
            }
            const QGroup qg = quantize_group(v);
            q0 = u32x4{qg.q[0], qg.q[1], qg.q[2], qg.q[3]};
            q1 = u32x4{qg.q[4], qg.q[5], qg.q[6], qg.q[7]};
            xd = qg.d;
            x0 = static_cast<float>(qg.hs0) * xd;
            x1 = static_cast<float>(qg.hs1) * xd;
        }
        if (t < ntok) {
            *reinterpret_cast<u32x4 *>(s_dyn + t * xi.stride + 32 * g) = q0;
            *reinterpret_cast<u32x4 *>(s_dyn + t * xi.stride + 32 * g + 16) = q1;
        }
        reinterpret_cast<float *>(s_dyn + xi.xd_off)[g * 16 + t] = xd;
        reinterpret_cast<float *>(s_dyn + xi.xs_off)[(g * 2) * 16 + t] = x0;
        reinterpret_cast<float *>(s_dyn + xi.xs_off)[(g * 2 + 1) * 16 + t] = x1;
    }
    __syncthreads();

    for (int st0 = 0; st0 < nsteps; st0 += kMfmaPF + 1) {
#pragma unroll
        for (int b = 0; b <= kMfmaPF; ++b) {  // ring slot b holds step st0 + b
            const int st = st0 + b;
            if (st >= nsteps) break;
            if (st + kMfmaPF < nsteps) load(st + kMfmaPF, wr[(b + kMfmaPF) % (kMfmaPF + 1)]);
            // Decode step st into the wave's LDS tile.
#pragma unroll
            for (int j = 0; j < SLJ; ++j) {
                int rl, us, ss;
                slice_of(j, rl, us, ss);
                const bool live = u_beg + st * UPS + us < u_end;
                uint32_t cd[NP][4];
                S::codes(wr[b][j], ss, tb, cd);
                float sc[NP], mn[NP];
                S::scales(wr[b][j], ss, sc, mn);
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    int pg, ph;
                    S::part(ss, p, pg, ph);
                    const int gg = us * UG + pg;
                    auto fix = [&](uint32_t c) { return live ? (S::OFF != 0 ? sub_bytes(c, S::OFF) : c) : 0u; };
                    *reinterpret_cast<u32x4 *>(ct + rl * kGemmRowPad + 32 * gg + 16 * ph) =
                        u32x4{fix(cd[p][0]), fix(cd[p][1]), fix(cd[p][2]), fix(cd[p][3])};
                    s_sc[wv][rl][gg * 2 + ph] = live ? sc[p] : 0.0f;
                    s_mn[wv][rl][gg * 2 + ph] = live && kHasMin<T> ? mn[p] : 0.0f;
                }
            }
            // Contract the step's 8 groups.
            const int kst = (u_beg + st * UPS) * UG * 32 - k0;  // step's first column within the K range
#pragma unroll
            for (int gg = 0; gg < 8; ++gg) {
                const long a = lr < ntok ? *reinterpret_cast<const long *>(s_dyn + lr * xi.stride + kst + 32 * gg + 8 * lk) : 0l;
                const long bw = *reinterpret_cast<const long *>(ct + lr * kGemmRowPad + 32 * gg + 8 * lk);
                const int gx = (kst >> 5) + gg;
                const float4 xd4 = *reinterpret_cast<const float4 *>(s_dyn + xi.xd_off + (gx * 16 + 4 * lk) * 4);
                const float xdv[4] = {xd4.x, xd4.y, xd4.z, xd4.w};
                if constexpr (kScalePer32<T>) {
                    const v4i32 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bw, v4i32{0, 0, 0, 0}, 0, 0, 0);
                    const float sc = s_sc[wv][lr][gg * 2];
                    float xsv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    float mn = 0.0f;
                    if constexpr (kHasMin<T>) {
                        mn = s_mn[wv][lr][gg * 2];
                        const float4 a0 = *reinterpret_cast<const float4 *>(s_dyn + xi.xs_off + ((gx * 2) * 16 + 4 * lk) * 4);
                        const float4 a1 = *reinterpret_cast<const float4 *>(s_dyn + xi.xs_off + ((gx * 2 + 1) * 16 + 4 * lk) * 4);
                        xsv[0] = a0.x + a1.x;
                        xsv[1] = a0.y + a1.y;
                        xsv[2] = a0.z + a1.z;
                        xsv[3] = a0.w + a1.w;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float v = fmaf(static_cast<float>(c[j]), sc * xdv[j], acc[j]);
                        if constexpr (kHasMin<T>) v = fmaf(-mn, xsv[j], v);
                        acc[j] = v;
                    }
                } else {
                    const long blo = lk < 2 ? bw : 0l, bhi = lk < 2 ? 0l : bw;
                    const v4i32 c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, blo, v4i32{0, 0, 0, 0}, 0, 0, 0);
                    const v4i32 c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bhi, v4i32{0, 0, 0, 0}, 0, 0, 0);
                    const float sc0 = s_sc[wv][lr][gg * 2], sc1 = s_sc[wv][lr][gg * 2 + 1];
                    float x0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, x1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    float mn0 = 0.0f, mn1 = 0.0f;
                    if constexpr (kHasMin<T>) {
                        mn0 = s_mn[wv][lr][gg * 2];
                        mn1 = s_mn[wv][lr][gg * 2 + 1];
                        const float4 a0 = *reinterpret_cast<const float4 *>(s_dyn + xi.xs_off + ((gx * 2) * 16 + 4 * lk) * 4);
                        const float4 a1 = *reinterpret_cast<const float4 *>(s_dyn + xi.xs_off + ((gx * 2 + 1) * 16 + 4 * lk) * 4);
                        x0[0] = a0.x; x0[1] = a0.y; x0[2] = a0.z; x0[3] = a0.w;
                        x1[0] = a1.x; x1[1] = a1.y; x1[2] = a1.z; x1[3] = a1.w;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float v = fmaf(static_cast<float>(c0[j]), sc0 * xdv[j], acc[j]);
                        v = fmaf(static_cast<float>(c1[j]), sc1 * xdv[j], v);
                        if constexpr (kHasMin<T>) {
                            v = fmaf(-mn0, x0[j], v);
                            v = fmaf(-mn1, x1[j], v);
                        }
                        acc[j] = v;
                    }
                }
            }
        }
    }
    // Row lane%16 of the block, tokens 4*(lane/16)+j.
    const int r = r0 + lr;
    if (r < rows) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = 4 * lk + j;
            if (t < ntok) {
                if (part != nullptr)
                    part[(static_cast<size_t>(blockIdx.y) * ntok + t) * rows + r] = acc[j];
                else
                    y[static_cast<size_t>(t) * rows + r] = acc[j];
            }
        }
    }
}

// y[t][r] = sum over s < nsplit of part[s][t][r], in order s = 0, 1, ...
static __global__ __launch_bounds__(256) void sum_parts_kernel(const float *__restrict__ part, int nsplit, long n,
                                                               float *__restrict__ y) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = part[i];
    for (int s = 1; s < nsplit; ++s) v += part[static_cast<size_t>(s) * n + i];
    y[i] = v;
}

// K ranges for a small-batch launch: enough workgroups to fill the chip, each range a multiple of 256
// columns whose activation image fits the LDS budget.
inline int mfma_splits(int rows, int cols, int ntok) {
    const int row_wgs = (rows + 16 * kMfmaRowWaves - 1) / (16 * kMfmaRowWaves);
    const int steps = (cols + 255) / 256;
    int s = 1;
    while (s < steps && (row_wgs * s < 1024 || MfmaX((steps + s - 1) / s * 256, ntok).bytes > kMfmaXMax)) s *= 2;
    return s > steps ? steps : s;
}

inline size_t mfma_part_bytes(int rows, int cols, int ntok) {
    const int s = mfma_splits(rows, cols, ntok);
    return s > 1 ? static_cast<size_t>(s) * ntok * rows * 4 : 0;
}

template <int T>
int launch_mfma(const uint8_t *w, int rows, int cols, long rb, const float *x, int ntok, float *y, float *part,
                hipStream_t s) {
    if (ntok < 1 || ntok > 16) return static_cast<int>(hipErrorInvalidValue);
    const int steps = (cols + 255) / 256;
    const int ns = mfma_splits(rows, cols, ntok);
    const int kw = (steps + ns - 1) / ns * 256;
    const int nsplit = (cols + kw - 1) / kw;
    const size_t lds = MfmaX(kw, ntok).bytes;
    static const bool raised = [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&qmv_mfma_kernel<T>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        (void)hipGetLastError();
        return true;
    }();
    (void)raised;
    const dim3 grid((rows + 16 * kMfmaRowWaves - 1) / (16 * kMfmaRowWaves), nsplit), block(64 * kMfmaRowWaves);
    float *p = nsplit > 1 ? part : nullptr;
    if (nsplit > 1 && part == nullptr) return static_cast<int>(hipErrorInvalidValue);
    qmv_mfma_kernel<T><<<grid, block, lds, s>>>(w, rows, cols, rb, x, ntok, kw, y, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    if (nsplit > 1) {
        const long n = static_cast<long>(ntok) * rows;
        sum_parts_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(part, nsplit, n, y);
        e = hipGetLastError();
        if (e != hipSuccess) return static_cast<int>(e);
    }
    return 0;
}

}  // namespace vq
