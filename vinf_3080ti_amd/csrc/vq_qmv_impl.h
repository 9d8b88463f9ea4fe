// vq_qmv_impl.h -- quantized matvec kernels, templated on the GGUF type (one translation unit per type
// instantiates them: vq_t_<type>.hip). Hand-written for CDNA4 (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_qmv.h"
#include "vq_tables.h"

namespace vq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Tuning knobs (compile-time; the defaults are the measured best on MI355X).
#ifndef VQ_KW_MAX
#define VQ_KW_MAX 8  // longest straight-line window of units per lane
#endif
#ifndef VQ_RING_BYTES
#define VQ_RING_BYTES 128  // bytes of raw slice data per lane kept in flight
#endif
#ifndef VQ_PIN
#define VQ_PIN 2  // 0: free scheduling, 1: memory clobber per slot, 2: plus a scheduling barrier
#endif
#ifndef VQ_USE_XL
#define VQ_USE_XL 1  // stage activations in LDS when they fit
#endif
#ifndef VQ_MAX_NT
#define VQ_MAX_NT 8  // tokens per launch compiled (tuning builds may restrict this)
#endif
#ifndef VQ_MAX_WAVES
#define VQ_MAX_WAVES 16  // waves per workgroup
#endif

// Slices kept in flight per lane (ring depth): enough outstanding loads to cover HBM latency within the
// VGPR budget.
template <int T>
constexpr int kUnroll = VQ_RING_BYTES / static_cast<int>(sizeof(typename Sl<T>::W)) < 2
                            ? 2
                            : (VQ_RING_BYTES / static_cast<int>(sizeof(typename Sl<T>::W)) > 8
                                   ? 8
                                   : VQ_RING_BYTES / static_cast<int>(sizeof(typename Sl<T>::W)));

constexpr int kXLdsMax = 48 * 1024;  // NT * vq_xpack_stride(cols) <= this -> activations live in LDS
constexpr int kXStagePieces = 4;     // 16-byte pieces of the activation records each thread stages per pass

// Quantized matvec: y[t][r] = W[r] . x[t] for t < NT.
//
// A workgroup of W waves is split into lane groups of L lanes, one weight row per group. Lane i of a group
// keeps one slice position ss = i % SPB (L is a multiple of SPB) and handles the units u0, u0 + du, ... of
// the row (u0 = i / SPB, du = L / SPB), so consecutive lanes read consecutive bytes and every load
// instruction is coalesced. A window of KW units per lane is straight-line code: slot k + U is loaded
// right after slot k is decoded, so U slices stay in flight, and with no branches inside the window the
// waitcnt pass issues partial vmcnt waits (a loop back-edge or an early exit would make it drain every
// load, or let LLVM sink each load next to its use). Slots past the row end load a clamped unit and are
// dropped with a select. Rows longer than KW units per lane take several windows.
//
// XL: all NT tokens' packed activation records (vq_pack_x) are copied to LDS first, so the per-slice
// activation reads are LDS reads: they neither add L1 traffic nor join the in-order vmcnt queue of the weight
// loads. The staging loads are issued before the first weight loads (vmcnt retires in order: waiting for
// activations issued after the weights would wait for the weights too), then the weight prologue, then
// the activations are written to LDS behind a partial wait.
//
// The group's L partial sums are reduced with cross-lane shuffles; lane 0 of the group writes y.
template <int T, int NT, bool XL, int KW>
__global__ __launch_bounds__(1024) void qmv_slice_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                         long row_bytes, const uint8_t *__restrict__ xpack,
                                                         float *__restrict__ y, int L) {
    using S = Sl<T>;
    constexpr int NP = S::NP;
    constexpr int U = kUnroll<T> < KW ? kUnroll<T> : KW;
    extern __shared__ __attribute__((aligned(16))) uint8_t s_x[];
    __shared__ uint2 s8[TabSpec<T>::n8 > 0 ? TabSpec<T>::n8 : 1];
    __shared__ uint32_t s4[TabSpec<T>::n4 > 0 ? TabSpec<T>::n4 : 1];
    __shared__ uint4 sks[TabSpec<T>::ks ? 128 : 1];
    __shared__ uint4 ssm[TabSpec<T>::sm ? 256 : 1];

    const int ng = cols >> 5;
    const int xb = vq_xpack_stride(cols);
    const int xh_off = vq_xpack_h_offset(cols);
    const int lane = threadIdx.x & 63;
    const int li = lane & (L - 1);
    const int row = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    const int nu = ng / S::UG;
    const int ss = li & (S::SPB - 1);
    const int du = L / S::SPB;
    const int u0 = li / S::SPB;
    const uint8_t *wp = w + static_cast<size_t>(min(row, rows - 1)) * row_bytes;
    auto unit_ptr = [&](int u) { return wp + static_cast<size_t>(min(u, nu - 1)) * S::UB; };

    // Activation staging loads first (first pass of kXStagePieces 16-byte pieces per thread), then the first
    // window's weight prologue, so HBM traffic starts at once and the staging wait does not cover the weights.
    const int npieces = XL ? NT * xb / 16 : 0;
    u32x4 xs_reg[kXStagePieces];
    if constexpr (XL) {
#pragma unroll
        for (int k = 0; k < kXStagePieces; ++k)
            xs_reg[k] = reinterpret_cast<const u32x4 *>(xpack)[min(static_cast<int>(threadIdx.x) + k * static_cast<int>(blockDim.x), npieces - 1)];
    }
    asm volatile("" ::: "memory");
    typename S::W wr[KW];
#pragma unroll
    for (int k = 0; k < U; ++k) S::load(unit_ptr(u0 + k * du), ss, wr[k]);
    asm volatile("" ::: "memory");

    const Tabs tb = stage_tabs<T>(s8, s4, sks, ssm);
    if constexpr (XL) {
#pragma unroll
        for (int k = 0; k < kXStagePieces; ++k) {
            const int i = threadIdx.x + k * blockDim.x;
            if (i < npieces) reinterpret_cast<u32x4 *>(s_x)[i] = xs_reg[k];
        }
        for (int i = threadIdx.x + kXStagePieces * blockDim.x; i < npieces; i += blockDim.x)
            reinterpret_cast<u32x4 *>(s_x)[i] = reinterpret_cast<const u32x4 *>(xpack)[i];
    }
    if constexpr (XL || TabSpec<T>::n8 > 0 || TabSpec<T>::n4 > 0) __syncthreads();
    const uint8_t *xsrc = XL ? s_x : xpack;  // activation records: LDS copy or the global packed buffer

    int pg[NP], ph[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) S::part(ss, p, pg[p], ph[p]);
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;

    for (int wb = 0; wb < nu; wb += KW * du) {
        if (wb > 0) {
#pragma unroll
            for (int k = 0; k < U; ++k) S::load(unit_ptr(wb + u0 + k * du), ss, wr[k]);
        }
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            if (k + U < KW) S::load(unit_ptr(wb + u0 + (k + U) * du), ss, wr[k + U]);
#if VQ_PIN >= 1
            // Pin the load issue point: without a memory clobber LLVM sinks each load next to its use.
            asm volatile("" ::: "memory");
#endif
#if VQ_PIN >= 2
            // Keep the slot's decode here too, so register pressure stays at U slots.
            __builtin_amdgcn_sched_barrier(0);
#endif
            const int u = wb + u0 + k * du;
            const bool valid = u < nu;
            uint32_t c[NP][4];
            S::codes(wr[k], ss, tb, c);
            float sc[NP], mn[NP];
            S::scales(wr[k], ss, sc, mn);
            const int G0 = min(u, nu - 1) * S::UG;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const int G = G0 + pg[p];
                    const uint8_t *xt = xsrc + t * xb;
                    const u32x4 v = *reinterpret_cast<const u32x4 *>(xt + 32 * G + 16 * ph[p]);
                    const float xdv = reinterpret_cast<const float *>(xt + cols)[G];
                    const int X = kNeedsX<T> ? static_cast<int>(static_cast<int16_t>(
                                                   reinterpret_cast<const uint32_t *>(xt + xh_off)[G] >> (16 * ph[p])))
                                             : 0;
                    const uint32_t xv[4] = {v.x, v.y, v.z, v.w};
                    const int Sv = dot16(c[p], xv) - S::OFF * X;
                    float f = static_cast<float>(Sv) * sc[p];
                    if constexpr (kHasMin<T>) f = fmaf(-static_cast<float>(X), mn[p], f);
                    const float nacc = fmaf(f, xdv, acc[t]);
                    acc[t] = valid ? nacc : acc[t];
                }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float v = acc[t];
        for (int off = L >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[t] = v;
    }
    if (li == 0 && row < rows) {
#pragma unroll
        for (int t = 0; t < NT; ++t) y[static_cast<size_t>(t) * rows + row] = acc[t];
    }
}

// ---- test hooks (same decoders as the matvec) -----------------------------------------------------------

template <int T>
__global__ __launch_bounds__(256) void int_partials_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                           long row_bytes, const uint8_t *__restrict__ xpack,
                                                           int ntok, int32_t *__restrict__ part) {
    using S = Sl<T>;
    const int ng = cols >> 5;
    const int nsl = (ng / S::UG) * S::SPB;
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long>(rows) * nsl) return;
    const int r = static_cast<int>(i / nsl), s = static_cast<int>(i - static_cast<long>(r) * nsl);
    const int u = s / S::SPB, ss = s - u * S::SPB;
    const Tabs tb = global_tabs<T>();
    typename S::W wr;
    S::load(w + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(u) * S::UB, ss, wr);
    uint32_t c[S::NP][4];
    S::codes(wr, ss, tb, c);
    for (int t = 0; t < ntok; ++t)
#pragma unroll
        for (int p = 0; p < S::NP; ++p) {
            int gj, h;
            S::part(ss, p, gj, h);
            const int G = u * S::UG + gj;
            const uint8_t *xt = xpack + static_cast<size_t>(t) * vq_xpack_stride(cols);
            const u32x4 v = *reinterpret_cast<const u32x4 *>(xt + 32 * G + 16 * h);
            const uint32_t xv[4] = {v.x, v.y, v.z, v.w};
            const int X = kNeedsX<T> ? static_cast<int>(static_cast<int16_t>(
                                           reinterpret_cast<const uint32_t *>(xt + vq_xpack_h_offset(cols))[G] >> (16 * h)))
                                     : 0;
            part[((static_cast<size_t>(t) * rows + r) * ng + G) * 2 + h] = dot16(c[p], xv) - S::OFF * X;
        }
}

template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ w, int rows, int cols, long row_bytes,
                                                      float *__restrict__ out) {
    using S = Sl<T>;
    const int ng = cols >> 5;
    const int nsl = (ng / S::UG) * S::SPB;
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long>(rows) * nsl) return;
    const int r = static_cast<int>(i / nsl), s = static_cast<int>(i - static_cast<long>(r) * nsl);
    const int u = s / S::SPB, ss = s - u * S::SPB;
    const Tabs tb = global_tabs<T>();
    typename S::W wr;
    S::load(w + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(u) * S::UB, ss, wr);
    uint32_t c[S::NP][4];
    S::codes(wr, ss, tb, c);
    float sc[S::NP], mn[S::NP];
    S::scales(wr, ss, sc, mn);
#pragma unroll
    for (int p = 0; p < S::NP; ++p) {
        int gj, h;
        S::part(ss, p, gj, h);
        float *o = out + static_cast<size_t>(r) * cols + 32 * (u * S::UG + gj) + 16 * h;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int code = static_cast<int>(static_cast<int8_t>(bfe(c[p][k >> 2], 8 * (k & 3), 8))) - S::OFF;
            o[k] = sc[p] * static_cast<float>(code) - mn[p];  // sc*code is exact; one rounding
        }
    }
}

// ---- host side -----------------------------------------------------------------------------------------

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : static_cast<int>(e); }

// Lanes per row: the widest group that still gives every lane >= 3 slices of the row.
inline int lanes_per_row(int nsl) {
    int L = 64;
    while (L > 8 && nsl < 3 * L) L >>= 1;
    return L;
}

// Waves per workgroup: as many as fit 1024 threads while the grid still spreads over all 256 CUs.
inline int waves_per_wg(long lane_groups, int L) {
    const long waves = (lane_groups * L + 63) / 64;
    int W = VQ_MAX_WAVES;
    while (W > 4 && waves / W < 512) W >>= 1;
    return W;
}

template <int T, int N, bool XL>
int launch_window(int KW, dim3 grid, dim3 block, size_t lds, hipStream_t s, const uint8_t *w, int rows, int cols,
                  long rb, const uint8_t *xp, float *yo, int L) {
    if constexpr (N <= 2) {
        switch (KW) {
            case 4: qmv_slice_kernel<T, N, XL, 4><<<grid, block, lds, s>>>(w, rows, cols, rb, xp, yo, L); break;
            case 8: qmv_slice_kernel<T, N, XL, 8><<<grid, block, lds, s>>>(w, rows, cols, rb, xp, yo, L); break;
            case 12: qmv_slice_kernel<T, N, XL, 12><<<grid, block, lds, s>>>(w, rows, cols, rb, xp, yo, L); break;
            default: qmv_slice_kernel<T, N, XL, 16><<<grid, block, lds, s>>>(w, rows, cols, rb, xp, yo, L); break;
        }
    } else {
        (void)KW;
        qmv_slice_kernel<T, N, XL, 8><<<grid, block, lds, s>>>(w, rows, cols, rb, xp, yo, L);
    }
    return hip_status(hipGetLastError());
}

template <int T>
int launch_quant(const uint8_t *w, int rows, int cols, long rb, const uint8_t *xpack, int ntok, float *y,
                 hipStream_t s) {
    using S = Sl<T>;
    const int ng = cols / 32;
    const int nu = ng / S::UG;
    const int L = lanes_per_row(nu * S::SPB);
    const int du = L / S::SPB;
    const int per_lane = (nu + du - 1) / du;
    int KW = per_lane <= 4 ? 4 : per_lane <= 8 ? 8 : per_lane <= 12 ? 12 : 16;
    if (KW > VQ_KW_MAX) KW = VQ_KW_MAX;
    const int W = waves_per_wg(rows, L);
    const int rows_per_wg = W * (64 / L);
    const dim3 grid((rows + rows_per_wg - 1) / rows_per_wg), block(64 * W);
    for (int c = 0; c < ntok; c += 8) {
        const int m = ntok - c < 8 ? ntok - c : 8;
        const uint8_t *xp = xpack + static_cast<size_t>(c) * vq_xpack_stride(cols);
        float *yo = y + static_cast<size_t>(c) * rows;
        const size_t lds = static_cast<size_t>(m) * vq_xpack_stride(cols);
        const bool xl = VQ_USE_XL && lds <= kXLdsMax;
        int st = 0;
        switch (m) {
#define VQ_CASE(N)                                                                                         \
    case N:                                                                                                \
        if constexpr (N <= VQ_MAX_NT)                                                                      \
            st = xl ? launch_window<T, N, true>(KW, grid, block, lds, s, w, rows, cols, rb, xp, yo, L) \
                    : launch_window<T, N, false>(KW, grid, block, 0, s, w, rows, cols, rb, xp, yo, L); \
        else                                                                                               \
            st = hipErrorInvalidValue;                                                                     \
        break;
            VQ_CASE(1) VQ_CASE(2) VQ_CASE(3) VQ_CASE(4) VQ_CASE(5) VQ_CASE(6) VQ_CASE(7) VQ_CASE(8)
#undef VQ_CASE
        }
        if (st) return st;
    }
    return 0;
}

template <int T>
int launch_partials(const uint8_t *w, int rows, int cols, long rb, const uint8_t *xpack, int ntok, int32_t *part,
                    hipStream_t s) {
    using S = Sl<T>;
    const long n = static_cast<long>(rows) * (cols / 32 / S::UG) * S::SPB;
    int_partials_kernel<T><<<(n + 255) / 256, 256, 0, s>>>(w, rows, cols, rb, xpack, ntok, part);
    return hip_status(hipGetLastError());
}

template <int T>
int launch_dequant(const uint8_t *w, int rows, int cols, long rb, float *out, hipStream_t s) {
    using S = Sl<T>;
    const long n = static_cast<long>(rows) * (cols / 32 / S::UG) * S::SPB;
    dequant_kernel<T><<<(n + 255) / 256, 256, 0, s>>>(w, rows, cols, rb, out);
    return hip_status(hipGetLastError());
}

}  // namespace vq

// Explicit instantiation of one type's entry points (used by the per-type translation units).
#define VQ_INSTANTIATE(T)                                                                                       \
    template int vq::launch_quant<T>(const uint8_t *, int, int, long, const uint8_t *, int, float *, hipStream_t); \
    template int vq::launch_partials<T>(const uint8_t *, int, int, long, const uint8_t *, int, int32_t *,          \
                                        hipStream_t);                                                            \
    template int vq::launch_dequant<T>(const uint8_t *, int, int, long, float *, hipStream_t);
