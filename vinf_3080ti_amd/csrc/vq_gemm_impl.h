// vq_gemm_impl.h -- prefill contraction Y[t][r] = W[r] . x[t] for many tokens on CDNA4 int8 MFMA
// (v_mfma_i32_16x16x32_i8), templated on the GGUF type and instantiated by the per-type translation units.
//
// Numerics are the matvec's: the activations are the same int8 codes per 32-group (vq_pack_x), the weights
// the same integer codes (the slice decoders of vq_slices.h, offsets removed so the codes are signed), and
// each 32-group's (or 16-half's) exact int32 partial S is scaled in fp32:
//   y += S * (sc * xd) - mn * (X * xd)
// where sc/mn are the block's decoded scale/min of that row and part, xd the token's group scale and X the
// token's half sum (reference: Cpu_qmv, qwen_cpu.c:581-641, per group; the reference's GPU GEMM
// vinf_qgemm_kernel, qwen_runtime.cu:663-739, rounds x to fp16 instead, which the CPU contract does not
// allow). Only the summation order differs from the matvec.
//
// Work split: a workgroup of 4 waves computes a 64-row x 64-token tile; wave w owns rows 32*(w % 2) ..
// +32 (two 16-row MFMA blocks) and tokens 32*(w / 2) .. +32 (two 16-token blocks). Workgroups that share
// weight rows are adjacent in the grid (token tile = blockIdx.x), so the re-reads of a row block hit L2. The K loop walks 256
// elements at a time: the raw weight slices and activation chunks of step k+1 are loaded into registers
// while step k's MFMAs run, then decoded into LDS (signed int8 codes [row][k], float scales per row and
// 16-element part; activation codes [token][k], group scales and half sums).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_qmv.h"
#include "vq_tables.h"

namespace vq {

constexpr int kGemmBM = 64, kGemmBN = 64, kGemmWaves = 4, kGemmKS = 256;
constexpr int kGemmRowPad = kGemmKS + 8;  // LDS row stride of the code tiles (bytes)

// Parts of one 32-group share one scale (and min): one K=32 MFMA per group. Otherwise the two 16-halves are
// contracted separately (two MFMAs with the other half's codes zeroed).
template <int T>
constexpr bool kScalePer32 = T == VQ_Q4_K || T == VQ_Q5_K || T == VQ_Q8_0 || T == VQ_IQ4_NL || T == VQ_IQ4_XS ||
                             T == VQ_IQ2_XXS || T == VQ_IQ3_S || T == VQ_IQ3_XXS;

typedef int32_t v4i32 __attribute__((ext_vector_type(4)));

// Bytewise c - off for unsigned codes 0..127 (no borrow between bytes).
__device__ __forceinline__ uint32_t sub_bytes(uint32_t c, uint32_t off) {
    return ((c | 0x80808080u) - off * 0x01010101u) ^ 0x80808080u;
}

template <int T>
__global__ __launch_bounds__(64 * kGemmWaves) void qgemm_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                                long row_bytes, const uint8_t *__restrict__ xpack,
                                                                int M, float *__restrict__ y) {
    using S = Sl<T>;
    constexpr int NP = S::NP, SPB = S::SPB, UB = S::UB, UG = S::UG;
    constexpr int UPS = kGemmKS / (32 * UG);           // units per K step
    constexpr int NSL = kGemmBM * UPS * SPB;           // slices per K step
    constexpr int SLT = NSL / (64 * kGemmWaves);       // slices per thread
    constexpr int NG = kGemmKS / 32;                   // 32-groups per K step
    constexpr int XCH = kGemmBN * (kGemmKS / 16) / (64 * kGemmWaves);  // 16-byte x chunks per thread
    static_assert(NSL % (64 * kGemmWaves) == 0, "slice split");

    __shared__ __attribute__((aligned(16))) uint8_t s_codes[kGemmBM * kGemmRowPad];
    __shared__ __attribute__((aligned(16))) uint8_t s_xq[kGemmBN * kGemmRowPad];
    __shared__ float s_sc[kGemmBM][NG * 2], s_mn[kGemmBM][NG * 2];
    __shared__ float s_xd[kGemmBN][NG], s_xs[kGemmBN][NG * 2];
    __shared__ uint2 s8[TabSpec<T>::n8 > 0 ? TabSpec<T>::n8 : 1];
    __shared__ uint32_t s4[TabSpec<T>::n4 > 0 ? TabSpec<T>::n4 : 1];
    __shared__ uint2 sks[TabSpec<T>::ks ? 128 : 1];
    __shared__ uint2 ssm[TabSpec<T>::sm ? 256 : 1];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r0 = blockIdx.y * kGemmBM, t0 = blockIdx.x * kGemmBN;
    const int ng = cols >> 5, nu = ng / UG;
    const int xb = vq_xpack_stride(cols), xh_off = vq_xpack_h_offset(cols);
    const int nsteps = (cols + kGemmKS - 1) / kGemmKS;
    const Tabs tb = stage_tabs<T>(s8, s4, sks, ssm);

    // This thread's decode work per step: slice index i -> (row, unit in step, slice).
    typename S::W wr[SLT];
    u32x4 xr[XCH];
    auto load_step = [&](int k) {
#pragma unroll
        for (int j = 0; j < SLT; ++j) {
            const int i = tid + j * 64 * kGemmWaves;
            const int ss = i % SPB, us = (i / SPB) % UPS, rl = i / (SPB * UPS);
            const int r = min(r0 + rl, rows - 1);
            const int u = min(k * UPS + us, nu - 1);
            S::load(w + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(u) * UB, ss, wr[j]);
        }
#pragma unroll
        for (int j = 0; j < XCH; ++j) {
            const int i = tid + j * 64 * kGemmWaves;
            const int tl = i / (kGemmKS / 16), ch = i % (kGemmKS / 16);
            const int t = min(t0 + tl, M - 1);
            const int c = min(k * kGemmKS + 16 * ch, cols - 16);
            xr[j] = *reinterpret_cast<const u32x4 *>(xpack + static_cast<size_t>(t) * xb + c);
        }
    };
    auto store_step = [&](int k) {
#pragma unroll
        for (int j = 0; j < SLT; ++j) {
            const int i = tid + j * 64 * kGemmWaves;
            const int ss = i % SPB, us = (i / SPB) % UPS, rl = i / (SPB * UPS);
            const bool live = k * UPS + us < nu;
            uint32_t cd[NP][4];
            S::codes(wr[j], ss, tb, cd);
            float sc[NP], mn[NP];
            S::scales(wr[j], ss, sc, mn);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                int pg, ph;
                S::part(ss, p, pg, ph);
                const int gg = us * UG + pg;  // group within the step
                // Codes with an offset (Q3_K, Q6_K) are unsigned 0..127 here: make them signed. The others are
                // already the signed (or small unsigned) int8 values the MFMA takes.
                auto fix = [&](uint32_t c) { return S::OFF != 0 ? sub_bytes(c, S::OFF) : c; };
                u32x4 v;
                v.x = live ? fix(cd[p][0]) : 0u;
                v.y = live ? fix(cd[p][1]) : 0u;
                v.z = live ? fix(cd[p][2]) : 0u;
                v.w = live ? fix(cd[p][3]) : 0u;
                *reinterpret_cast<u32x4 *>(s_codes + rl * kGemmRowPad + 32 * gg + 16 * ph) = v;
                s_sc[rl][gg * 2 + ph] = live ? sc[p] : 0.0f;
                s_mn[rl][gg * 2 + ph] = live && kHasMin<T> ? mn[p] : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < XCH; ++j) {
            const int i = tid + j * 64 * kGemmWaves;
            const int tl = i / (kGemmKS / 16), ch = i % (kGemmKS / 16);
            const bool live = k * kGemmKS + 16 * ch < cols;
            *reinterpret_cast<u32x4 *>(s_xq + tl * kGemmRowPad + 16 * ch) = live ? xr[j] : u32x4{0u, 0u, 0u, 0u};
        }
        for (int i = tid; i < kGemmBN * NG; i += 64 * kGemmWaves) {
            const int tl = i / NG, gg = i % NG;
            const int t = min(t0 + tl, M - 1);
            const int g = k * NG + gg;
            const bool live = g < ng;
            const uint8_t *rec = xpack + static_cast<size_t>(t) * xb;
            const float xd = live ? reinterpret_cast<const float *>(rec + cols)[g] : 0.0f;
            const uint32_t h = live ? reinterpret_cast<const uint32_t *>(rec + xh_off)[g] : 0u;
            s_xd[tl][gg] = xd;
            s_xs[tl][gg * 2] = static_cast<float>(static_cast<int16_t>(h & 0xFFFFu)) * xd;
            s_xs[tl][gg * 2 + 1] = static_cast<float>(static_cast<int16_t>(h >> 16)) * xd;
        }
    };

    constexpr int TB = kGemmBN / 32;  // 16-token blocks per wave
    float acc[2][TB][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < TB; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[a][b][j] = 0.0f;

    const int rw = 32 * (wv & 1), tw = 16 * TB * (wv >> 1);  // this wave's row / token offsets in the tile
    const int lr = lane & 15, lk = lane >> 4;          // MFMA operand row/col and K chunk of this lane

    if (TabSpec<T>::n8 > 0 || TabSpec<T>::n4 > 0) __syncthreads();
    load_step(0);
    for (int k = 0; k < nsteps; ++k) {
        store_step(k);
        __syncthreads();
        if (k + 1 < nsteps) load_step(k + 1);  // in flight during this step's MFMAs
#pragma unroll
        for (int gg = 0; gg < NG; ++gg) {
            long a[2], b[TB];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
                a[rb] = *reinterpret_cast<const long *>(s_codes + (rw + 16 * rb + lr) * kGemmRowPad + 32 * gg + 8 * lk);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
                b[tb] = *reinterpret_cast<const long *>(s_xq + (tw + 16 * tb + lr) * kGemmRowPad + 32 * gg + 8 * lk);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                // C element j of a 16x16 block: row 4*(lane/16) + j, token lane % 16.
                float scr[2][4], mnr[2][4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        scr[h][j] = s_sc[rw + 16 * rb + 4 * lk + j][gg * 2 + h];
                        mnr[h][j] = s_mn[rw + 16 * rb + 4 * lk + j][gg * 2 + h];
                    }
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
                    const int tl = tw + 16 * tb + lr;
                    const float xd = s_xd[tl][gg];
                    if constexpr (kScalePer32<T>) {
                        const v4i32 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[rb], b[tb], v4i32{0, 0, 0, 0}, 0, 0, 0);
                        const float xs = s_xs[tl][gg * 2] + s_xs[tl][gg * 2 + 1];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            float v = fmaf(static_cast<float>(c[j]), scr[0][j] * xd, acc[rb][tb][j]);
                            if constexpr (kHasMin<T>) v = fmaf(-mnr[0][j], xs, v);
                            acc[rb][tb][j] = v;
                        }
                    } else {
                        const long alo = lk < 2 ? a[rb] : 0l, ahi = lk < 2 ? 0l : a[rb];
                        const v4i32 c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(alo, b[tb], v4i32{0, 0, 0, 0}, 0, 0, 0);
                        const v4i32 c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(ahi, b[tb], v4i32{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            float v = fmaf(static_cast<float>(c0[j]), scr[0][j] * xd, acc[rb][tb][j]);
                            v = fmaf(static_cast<float>(c1[j]), scr[1][j] * xd, v);
                            if constexpr (kHasMin<T>) {
                                v = fmaf(-mnr[0][j], s_xs[tl][gg * 2], v);
                                v = fmaf(-mnr[1][j], s_xs[tl][gg * 2 + 1], v);
                            }
                            acc[rb][tb][j] = v;
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    // Write: element j of block (rb, tb) is row r0 + rw + 16 rb + 4 lk + j, token t0 + tw + 16 tb + lr.
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const int t = t0 + tw + 16 * tb + lr;
            if (t >= M) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = r0 + rw + 16 * rb + 4 * lk + j;
                if (r < rows) y[static_cast<size_t>(t) * rows + r] = acc[rb][tb][j];
            }
        }
}

template <int T>
int launch_gemm(const uint8_t *w, int rows, int cols, long rb, const uint8_t *xpack, int M, float *y, hipStream_t s) {
    const dim3 grid((M + kGemmBN - 1) / kGemmBN, (rows + kGemmBM - 1) / kGemmBM), block(64 * kGemmWaves);
    qgemm_kernel<T><<<grid, block, 0, s>>>(w, rows, cols, rb, xpack, M, y);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int>(e);
}

}  // namespace vq
