// vq_kernels.hip -- MI355X (gfx950, wave64) quantized-weight matvec hot path and its C ABI.
//
// Kernels (all hand-written for CDNA4):
//   quantize_x_kernel    fp32 activations -> int8 per 32-group + (xd, xs)     [qwen_cpu.c:607-627 rule]
//   qmv_stream_kernel    y[t][r] = W[r] . x[t], raw GGUF blocks streamed row by row through LDS
//   int_partials_kernel  test hook: exact int32 code*xq sums per (t, row, group, half)
//   dequant_kernel       test hook: fp32 dequantization of every element
//   argmax_rows_kernel   row argmax, ties to the lowest index      [qwen_runtime.cu:850-876 semantics]
//
// Data layout in HBM: weights are the GGUF tensor bytes as uploaded (row-major, row_bytes =
// cols/block_size*type_size, rows back to back, >= VQ_TAIL_PAD readable bytes after the last row).
// Activations x[t*cols + c] fp32, outputs y[t*rows + r] fp32 (the reference's token-major layout).
#include <hip/hip_runtime.h>
#include <stdint.h>

#define VQ_GRID_STORAGE static constexpr
#include "vq_iq_grids.h"
#include "vq_common.h"
#include "vq_decode.h"
#include "../../include/vq.h"

namespace {

// ---- codebooks: expanded at compile time from the level-index encoding ------------------------------

template <int N>
struct Tab64 {
    uint64_t v[N];
};
template <int N>
struct Tab32 {
    uint32_t v[N];
};

template <int N>
constexpr Tab64<N> expand_iq2(const uint16_t (&c)[N]) {
    constexpr uint64_t lv[3] = {8, 25, 43};
    Tab64<N> t{};
    for (int e = 0; e < N; ++e) {
        uint64_t x = 0;
        for (int j = 0; j < 8; ++j) x |= lv[(c[e] >> (2 * j)) & 3] << (8 * j);
        t.v[e] = x;
    }
    return t;
}

template <int N>
constexpr Tab32<N> expand_iq3(const uint16_t (&c)[N], bool iq3s) {
    constexpr uint32_t lv[8] = {4, 12, 20, 28, 36, 44, 52, 62};
    Tab32<N> t{};
    for (int e = 0; e < N; ++e) {
        uint32_t x = 0;
        for (int j = 0; j < 4; ++j) {
            const uint32_t k = (c[e] >> (3 * j)) & 7;
            x |= (iq3s ? 2 * k + 1 : lv[k]) << (8 * j);
        }
        t.v[e] = x;
    }
    return t;
}

__device__ const Tab64<256> g_iq2xxs = expand_iq2(vq_iq2xxs_codes);
__device__ const Tab64<512> g_iq2xs = expand_iq2(vq_iq2xs_codes);
__device__ const Tab64<1024> g_iq2s = expand_iq2(vq_iq2s_codes);
__device__ const Tab32<256> g_iq3xxs = expand_iq3(vq_iq3xxs_codes, false);
// IQ3_S grid: replaceable at run time (the reference uploads it at Runtime init, qwen_runtime.cu:1272-1286).
__device__ Tab32<512> g_iq3s = expand_iq3(vq_iq3s_codes, true);

template <int T>
struct GridSpec {
    static constexpr int n64 = T == VQ_IQ2_XXS ? 256 : T == VQ_IQ2_XS ? 512 : T == VQ_IQ2_S ? 1024 : 0;
    static constexpr int n32 = T == VQ_IQ3_XXS ? 256 : T == VQ_IQ3_S ? 512 : 0;
};

__device__ __forceinline__ vq::Grids global_grids() {
    vq::Grids g;
    g.iq2xxs = reinterpret_cast<const uint2 *>(g_iq2xxs.v);
    g.iq2xs = reinterpret_cast<const uint2 *>(g_iq2xs.v);
    g.iq2s = reinterpret_cast<const uint2 *>(g_iq2s.v);
    g.iq3xxs = g_iq3xxs.v;
    g.iq3s = g_iq3s.v;
    return g;
}

// Copy the codebook of type T into LDS (whole workgroup; caller synchronises).
template <int T>
__device__ __forceinline__ vq::Grids stage_grids(uint2 *s64, uint32_t *s32) {
    vq::Grids g = global_grids();
    if constexpr (GridSpec<T>::n64 > 0) {
        const uint2 *src = T == VQ_IQ2_XXS ? g.iq2xxs : T == VQ_IQ2_XS ? g.iq2xs : g.iq2s;
        for (int i = threadIdx.x; i < GridSpec<T>::n64; i += blockDim.x) s64[i] = src[i];
        g.iq2xxs = g.iq2xs = g.iq2s = s64;
    }
    if constexpr (GridSpec<T>::n32 > 0) {
        const uint32_t *src = T == VQ_IQ3_XXS ? g.iq3xxs : g.iq3s;
        for (int i = threadIdx.x; i < GridSpec<T>::n32; i += blockDim.x) s32[i] = src[i];
        g.iq3xxs = g.iq3s = s32;
    }
    return g;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// ---- activation quantizer ------------------------------------------------------------------------------
// One thread per (token, 32-group). Same IEEE operations as the reference CPU quantizer
// (qwen_cpu.c:607-627): amax = max|v|, d = amax/127 (correctly rounded division), id = 1/d,
// q = rint(v*id) (round half to even, as lrintf), xs = d*sum(q).
__global__ __launch_bounds__(256) void quantize_x_kernel(const float *__restrict__ x, int ntok, int cols,
                                                         int8_t *__restrict__ xq, float *__restrict__ xd,
                                                         float *__restrict__ xs) {
    const int ng = cols >> 5;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= ntok * ng) return;
    const int t = i / ng, g = i - t * ng;
    const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<size_t>(t) * cols + 32 * g);
    float v[32];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float4 f = src[k];
        v[4 * k] = f.x;
        v[4 * k + 1] = f.y;
        v[4 * k + 2] = f.z;
        v[4 * k + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(v[k]));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    int sum = 0;
    uint32_t packed[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t p = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int q = static_cast<int>(__builtin_rintf(v[4 * k + b] * id));
            sum += q;
            p |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * b);
        }
        packed[k] = p;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(xq + static_cast<size_t>(t) * cols + 32 * g);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    xd[i] = d;
    xs[i] = d * static_cast<float>(sum);
}

// ---- streaming matvec ----------------------------------------------------------------------------------
// One wave per weight row. The wave copies the row's raw bytes into its private LDS buffer in 16-byte
// lanes (fully coalesced 1 KiB per wave instruction, whatever the block size), then each lane decodes
// one 32-element group at a time from LDS and dots it with the int8 activations of all NT tokens using
// v_dot4_i32_i8. Integer sums per 16-element half are scaled exactly as the reference CPU path does:
// acc += float(S_half) * (scale_half * xd), minus the min terms.
constexpr int kWaves = 4;
constexpr int kChunkBytes = 8192;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int T, int NT>
__device__ __forceinline__ void group_dot(const uint8_t *buf, int off, int j, int G, int cols, int ng,
                                          const vq::Grids &gr, const int8_t *__restrict__ xq,
                                          const float *__restrict__ xd, const float *__restrict__ xs,
                                          const float *__restrict__ xf, float (&acc)[NT]) {
    if constexpr (T == VQ_F32 || T == VQ_F16) {
        float wv[32];
        if constexpr (T == VQ_F32) {
            const float4 *p = reinterpret_cast<const float4 *>(buf + off);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float4 f = p[k];
                wv[4 * k] = f.x;
                wv[4 * k + 1] = f.y;
                wv[4 * k + 2] = f.z;
                wv[4 * k + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const uint32_t h = vq::ld32(buf, off + 4 * k);
                wv[2 * k] = vq::h2f(h);
                wv[2 * k + 1] = vq::h2f(h >> 16);
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 *xp = reinterpret_cast<const float4 *>(xf + static_cast<size_t>(t) * cols + 32 * G);
            float a = acc[t];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float4 f = xp[k];
                a = fmaf(wv[4 * k], f.x, a);
                a = fmaf(wv[4 * k + 1], f.y, a);
                a = fmaf(wv[4 * k + 2], f.z, a);
                a = fmaf(wv[4 * k + 3], f.w, a);
            }
            acc[t] = a;
        }
    } else {
        vq::Group g;
        vq::decode<T>(buf, off, j, gr, g);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint4 *xp = reinterpret_cast<const uint4 *>(xq + static_cast<size_t>(t) * cols + 32 * G);
            const uint4 xa = xp[0], xb = xp[1];
            int s0 = dot4(g.q[0], xa.x, 0);
            s0 = dot4(g.q[1], xa.y, s0);
            s0 = dot4(g.q[2], xa.z, s0);
            s0 = dot4(g.q[3], xa.w, s0);
            int s1 = dot4(g.q[4], xb.x, 0);
            s1 = dot4(g.q[5], xb.y, s1);
            s1 = dot4(g.q[6], xb.z, s1);
            s1 = dot4(g.q[7], xb.w, s1);
            const float d = xd[t * ng + G];
            float a = acc[t];
            a = fmaf(static_cast<float>(s0), g.s0 * d, a);
            a = fmaf(static_cast<float>(s1), g.s1 * d, a);
            if constexpr (T == VQ_Q4_K || T == VQ_Q5_K) a = fmaf(-g.mt, xs[t * ng + G], a);
            if constexpr (T == VQ_Q2_K) {
                int x0 = dot4(0x01010101u, xa.x, 0);
                x0 = dot4(0x01010101u, xa.y, x0);
                x0 = dot4(0x01010101u, xa.z, x0);
                x0 = dot4(0x01010101u, xa.w, x0);
                int x1 = dot4(0x01010101u, xb.x, 0);
                x1 = dot4(0x01010101u, xb.y, x1);
                x1 = dot4(0x01010101u, xb.z, x1);
                x1 = dot4(0x01010101u, xb.w, x1);
                a = fmaf(-static_cast<float>(x0), g.mn0 * d, a);
                a = fmaf(-static_cast<float>(x1), g.mn1 * d, a);
            }
            acc[t] = a;
        }
    }
}

template <int T, int NT>
__global__ __launch_bounds__(64 * kWaves) void qmv_stream_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                                  long row_bytes, const int8_t *__restrict__ xq,
                                                                  const float *__restrict__ xd,
                                                                  const float *__restrict__ xs,
                                                                  const float *__restrict__ xf, float *__restrict__ y) {
    constexpr int UB = VqUnit<T>::bytes, UG = VqUnit<T>::groups;
    constexpr int kUnitsPerChunk = (kChunkBytes - 16) / UB;
    __shared__ __attribute__((aligned(16))) uint8_t s_buf[kWaves][kChunkBytes];
    __shared__ uint2 s_g64[GridSpec<T>::n64 > 0 ? GridSpec<T>::n64 : 1];
    __shared__ uint32_t s_g32[GridSpec<T>::n32 > 0 ? GridSpec<T>::n32 : 1];
    const vq::Grids gr = stage_grids<T>(s_g64, s_g32);
    if constexpr (GridSpec<T>::n64 > 0 || GridSpec<T>::n32 > 0) __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * kWaves + wave;
    if (row >= rows) return;
    const int ng = cols >> 5;
    const int units = ng / UG;
    const uint8_t *rowp = w + static_cast<size_t>(row) * row_bytes;
    uint8_t *buf = s_buf[wave];
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;

    for (int u0 = 0; u0 < units; u0 += kUnitsPerChunk) {
        const int nu = min(kUnitsPerChunk, units - u0);
        const uint8_t *g0 = rowp + static_cast<size_t>(u0) * UB;
        const int lead = static_cast<int>(reinterpret_cast<uintptr_t>(g0) & 15u);
        const u32x4 *src = reinterpret_cast<const u32x4 *>(g0 - lead);
        const int n16 = (lead + nu * UB + 15) >> 4;
        u32x4 tmp[kChunkBytes / 1024];
#pragma unroll
        for (int k = 0; k < kChunkBytes / 1024; ++k) {
            const int i = lane + 64 * k;
            if (i < n16) tmp[k] = __builtin_nontemporal_load(src + i);
        }
#pragma unroll
        for (int k = 0; k < kChunkBytes / 1024; ++k) {
            const int i = lane + 64 * k;
            if (i < n16) reinterpret_cast<u32x4 *>(buf)[i] = tmp[k];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int ngc = nu * UG;
        for (int gi = lane; gi < ngc; gi += 64) {
            const int u = gi / UG, j = gi - u * UG;
            group_dot<T, NT>(buf, lead + u * UB, j, u0 * UG + gi, cols, ng, gr, xq, xd, xs, xf, acc);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float v = wave_sum(acc[t]);
        if (lane == 0) y[static_cast<size_t>(t) * rows + row] = v;
    }
}

// ---- test hooks ------------------------------------------------------------------------------------------

template <int T>
__global__ __launch_bounds__(256) void int_partials_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                           long row_bytes, const int8_t *__restrict__ xq, int ntok,
                                                           int32_t *__restrict__ part) {
    constexpr int UB = VqUnit<T>::bytes, UG = VqUnit<T>::groups;
    const int ng = cols >> 5;
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long>(rows) * ng) return;
    const int r = static_cast<int>(i / ng), G = static_cast<int>(i - static_cast<long>(r) * ng);
    const vq::Grids gr = global_grids();
    vq::Group g;
    vq::decode<T>(w, static_cast<long>(r) * row_bytes + static_cast<long>(G / UG) * UB, G % UG, gr, g);
    for (int t = 0; t < ntok; ++t) {
        const uint4 *xp = reinterpret_cast<const uint4 *>(xq + static_cast<size_t>(t) * cols + 32 * G);
        const uint4 xa = xp[0], xb = xp[1];
        int s0 = dot4(g.q[0], xa.x, 0);
        s0 = dot4(g.q[1], xa.y, s0);
        s0 = dot4(g.q[2], xa.z, s0);
        s0 = dot4(g.q[3], xa.w, s0);
        int s1 = dot4(g.q[4], xb.x, 0);
        s1 = dot4(g.q[5], xb.y, s1);
        s1 = dot4(g.q[6], xb.z, s1);
        s1 = dot4(g.q[7], xb.w, s1);
        int32_t *o = part + ((static_cast<size_t>(t) * rows + r) * ng + G) * 2;
        o[0] = s0;
        o[1] = s1;
    }
}

template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ w, int rows, int cols, long row_bytes,
                                                      float *__restrict__ out) {
    constexpr int UB = VqUnit<T>::bytes, UG = VqUnit<T>::groups;
    const int ng = cols >> 5;
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long>(rows) * ng) return;
    const int r = static_cast<int>(i / ng), G = static_cast<int>(i - static_cast<long>(r) * ng);
    float *o = out + static_cast<size_t>(r) * cols + 32 * G;
    const long off = static_cast<long>(r) * row_bytes + static_cast<long>(G / UG) * UB;
    if constexpr (T == VQ_F32) {
        for (int k = 0; k < 32; ++k) o[k] = __builtin_bit_cast(float, vq::ld32(w, off + 4 * k));
    } else if constexpr (T == VQ_F16) {
        for (int k = 0; k < 32; ++k) o[k] = vq::h2f(vq::ld32u(w, off + 2 * k));
    } else {
        const vq::Grids gr = global_grids();
        vq::Group g;
        vq::decode<T>(w, off, G % UG, gr, g);
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const float code = static_cast<float>(static_cast<int8_t>((g.q[k >> 2] >> (8 * (k & 3))) & 0xFF));
            const float s = k < 16 ? g.s0 : g.s1;
            const float m = T == VQ_Q2_K ? (k < 16 ? g.mn0 : g.mn1) : g.mt;
            o[k] = s * code - m;  // s*code is exact; the subtraction is the only rounding
        }
    }
}

// ---- argmax ------------------------------------------------------------------------------------------------
// One workgroup per row; strict '>' inside each thread's strided scan and lowest index on equal values
// in the tree, so the lowest index of the maximum wins and NaN never does.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float *__restrict__ x, int n, int32_t *__restrict__ out) {
    __shared__ float s_v[1024];
    __shared__ int32_t s_i[1024];
    const float *row = x + static_cast<size_t>(blockIdx.x) * n;
    float bv = -__builtin_inff();
    int32_t bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = row[i];
        if (v > bv) {
            bv = v;
            bi = i;
        }
    }
    s_v[threadIdx.x] = bv;
    s_i[threadIdx.x] = bi;
    __syncthreads();
    for (int stride = blockDim.x / 2; stride > 0; stride >>= 1) {
        if (threadIdx.x < stride) {
            const float ov = s_v[threadIdx.x + stride];
            const int32_t oi = s_i[threadIdx.x + stride];
            if (ov > s_v[threadIdx.x] || (ov == s_v[threadIdx.x] && oi < s_i[threadIdx.x])) {
                s_v[threadIdx.x] = ov;
                s_i[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = s_i[0];
}

// ---- host-side dispatch --------------------------------------------------------------------------------

int hip_status(hipError_t e) { return e == hipSuccess ? VQ_OK : static_cast<int>(e); }

int check_matrix(int type, int rows, int cols) {
    int bs, ts;
    if (!vq_traits(type, &bs, &ts)) return VQ_ERR_TYPE;
    if (rows < 1 || cols < 32 || cols % 32 != 0 || cols % bs != 0) return VQ_ERR_SHAPE;
    return VQ_OK;
}

long row_bytes_of(int type, int cols) {
    int bs, ts;
    vq_traits(type, &bs, &ts);
    return static_cast<long>(cols / bs) * ts;
}

template <typename F>
int dispatch_type(int type, F &&f) {
    switch (type) {
        case VQ_F32: return f(std::integral_constant<int, VQ_F32>{});
        case VQ_F16: return f(std::integral_constant<int, VQ_F16>{});
        case VQ_Q8_0: return f(std::integral_constant<int, VQ_Q8_0>{});
        case VQ_Q2_K: return f(std::integral_constant<int, VQ_Q2_K>{});
        case VQ_Q3_K: return f(std::integral_constant<int, VQ_Q3_K>{});
        case VQ_Q4_K: return f(std::integral_constant<int, VQ_Q4_K>{});
        case VQ_Q5_K: return f(std::integral_constant<int, VQ_Q5_K>{});
        case VQ_Q6_K: return f(std::integral_constant<int, VQ_Q6_K>{});
        case VQ_IQ4_NL: return f(std::integral_constant<int, VQ_IQ4_NL>{});
        case VQ_IQ4_XS: return f(std::integral_constant<int, VQ_IQ4_XS>{});
        case VQ_IQ3_S: return f(std::integral_constant<int, VQ_IQ3_S>{});
        case VQ_IQ2_XXS: return f(std::integral_constant<int, VQ_IQ2_XXS>{});
        case VQ_IQ2_XS: return f(std::integral_constant<int, VQ_IQ2_XS>{});
        case VQ_IQ2_S: return f(std::integral_constant<int, VQ_IQ2_S>{});
        case VQ_IQ3_XXS: return f(std::integral_constant<int, VQ_IQ3_XXS>{});
        default: return VQ_ERR_TYPE;
    }
}

template <int T>
int launch_stream(const uint8_t *w, int rows, int cols, const int8_t *xq, const float *xd, const float *xs,
                  const float *xf, int ntok, float *y, hipStream_t s) {
    const long rb = row_bytes_of(T, cols);
    const int ng = cols / 32;
    const dim3 grid((rows + kWaves - 1) / kWaves), block(64 * kWaves);
    for (int c = 0; c < ntok; c += 8) {
        const int m = ntok - c < 8 ? ntok - c : 8;
        const int8_t *q = xq ? xq + static_cast<size_t>(c) * cols : nullptr;
        const float *d = xd ? xd + static_cast<size_t>(c) * ng : nullptr;
        const float *sm = xs ? xs + static_cast<size_t>(c) * ng : nullptr;
        const float *f = xf ? xf + static_cast<size_t>(c) * cols : nullptr;
        float *yo = y + static_cast<size_t>(c) * rows;
        switch (m) {
#define VQ_CASE(N) \
    case N: qmv_stream_kernel<T, N><<<grid, block, 0, s>>>(w, rows, cols, rb, q, d, sm, f, yo); break;
            VQ_CASE(1) VQ_CASE(2) VQ_CASE(3) VQ_CASE(4) VQ_CASE(5) VQ_CASE(6) VQ_CASE(7) VQ_CASE(8)
#undef VQ_CASE
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_status(e);
    }
    return VQ_OK;
}

size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

}  // namespace

// ---- C ABI -------------------------------------------------------------------------------------------------

extern "C" {

int vq_type_traits(int type, int *block_size, int *type_size) {
    return vq_traits(type, block_size, type_size) ? VQ_OK : VQ_ERR_TYPE;
}

long long vq_row_bytes(int type, int cols) {
    int bs, ts;
    if (!vq_traits(type, &bs, &ts) || cols <= 0 || cols % bs) return -1;
    return static_cast<long long>(cols / bs) * ts;
}

const char *vq_status_string(int status) {
    switch (status) {
        case VQ_OK: return "success";
        case VQ_ERR_TYPE: return "unsupported GGUF tensor type";
        case VQ_ERR_SHAPE: return "invalid shape";
        case VQ_ERR_WORKSPACE: return "workspace too small";
        case VQ_ERR_ARG: return "invalid argument";
        case VQ_ERR_NOT_INIT: return "library not initialised on this device";
        default: return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown error";
    }
}

int vq_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    return hip_status(e);
}

int vq_set_iq3s_grid(const uint8_t *grid) {
    if (grid == nullptr) return VQ_ERR_ARG;
    return hip_status(hipMemcpyToSymbol(HIP_SYMBOL(g_iq3s), grid, 512 * 4, 0, hipMemcpyHostToDevice));
}

size_t vq_qmv_workspace_bytes(int cols, int ntok) {
    if (cols <= 0 || ntok <= 0) return 0;
    const size_t ng = static_cast<size_t>(cols) / 32;
    return align256(static_cast<size_t>(cols) * ntok) + 2 * align256(ng * ntok * sizeof(float));
}

int vq_quantize_x(const float *x, int ntok, int cols, int8_t *xq, float *xd, float *xs, void *stream) {
    if (!x || !xq || !xd || !xs) return VQ_ERR_ARG;
    if (ntok < 1 || cols < 32 || cols % 32) return VQ_ERR_SHAPE;
    const int n = ntok * (cols / 32);
    quantize_x_kernel<<<(n + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(x, ntok, cols, xq, xd, xs);
    return hip_status(hipGetLastError());
}

int vq_qmv_q(int type, const uint8_t *w, int rows, int cols, const int8_t *xq, const float *xd, const float *xs,
             int ntok, float *y, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;  // float weights take fp32 activations (vq_qmv)
    if (!w || !xq || !xd || !xs || !y) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    return dispatch_type(type, [&](auto tc) {
        return launch_stream<decltype(tc)::value>(w, rows, cols, xq, xd, xs, nullptr, ntok, y,
                                                  static_cast<hipStream_t>(stream));
    });
}

int vq_qmv(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, float *y, void *workspace,
           size_t workspace_bytes, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (!w || !x || !y) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (type == VQ_F32 || type == VQ_F16)
        return dispatch_type(type, [&](auto tc) {
            return launch_stream<decltype(tc)::value>(w, rows, cols, nullptr, nullptr, nullptr, x, ntok, y, s);
        });
    if (!workspace || workspace_bytes < vq_qmv_workspace_bytes(cols, ntok)) return VQ_ERR_WORKSPACE;
    const size_t ng = static_cast<size_t>(cols) / 32;
    int8_t *xq = static_cast<int8_t *>(workspace);
    float *xd = reinterpret_cast<float *>(static_cast<char *>(workspace) + align256(static_cast<size_t>(cols) * ntok));
    float *xs = reinterpret_cast<float *>(reinterpret_cast<char *>(xd) + align256(ng * ntok * sizeof(float)));
    st = vq_quantize_x(x, ntok, cols, xq, xd, xs, stream);
    if (st) return st;
    return vq_qmv_q(type, w, rows, cols, xq, xd, xs, ntok, y, stream);
}

int vq_int_partials(int type, const uint8_t *w, int rows, int cols, const int8_t *xq, int ntok, int32_t *part,
                    void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;
    if (!w || !xq || !part) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    const long n = static_cast<long>(rows) * (cols / 32);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return dispatch_type(type, [&](auto tc) {
        constexpr int T = decltype(tc)::value;
        if constexpr (T == VQ_F32 || T == VQ_F16) {
            return VQ_ERR_TYPE;
        } else {
            int_partials_kernel<T><<<(n + 255) / 256, 256, 0, s>>>(w, rows, cols, row_bytes_of(T, cols), xq, ntok, part);
            return hip_status(hipGetLastError());
        }
    });
}

int vq_dequant_rows(int type, const uint8_t *w, int rows, int cols, float *out, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (!w || !out) return VQ_ERR_ARG;
    const long n = static_cast<long>(rows) * (cols / 32);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return dispatch_type(type, [&](auto tc) {
        constexpr int T = decltype(tc)::value;
        dequant_kernel<T><<<(n + 255) / 256, 256, 0, s>>>(w, rows, cols, row_bytes_of(T, cols), out);
        return hip_status(hipGetLastError());
    });
}

int vq_argmax_rows(const float *x, int n, int ntok, int32_t *out, void *stream) {
    if (!x || !out) return VQ_ERR_ARG;
    if (n < 1 || ntok < 1) return VQ_ERR_SHAPE;
    argmax_rows_kernel<<<ntok, 1024, 0, static_cast<hipStream_t>(stream)>>>(x, n, out);
    return hip_status(hipGetLastError());
}

}  // extern "C"
