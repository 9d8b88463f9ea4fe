// vq_api.hip -- MI355X (gfx950, wave64) quantized-weight matvec: the C ABI (include/vq.h) and the
// type-independent kernels.
//
// Kernels here (hand-written for CDNA4):
//   quantize_x_kernel    fp32 activations -> int8 per 32-group + (xd, xs, 16-element sums) [qwen_cpu.c:607-627]
//   qmv_float_kernel     y = W x for F32/F16 weights with fp32 activations                [qwen_cpu.c:345-360]
//   dequant_float_kernel test hook for F32/F16 weights
//   argmax_rows_kernel   row argmax, ties to the lowest index                            [qwen_runtime.cu:850-876]
// The quantized kernels (one translation unit per GGUF type) are in vq_qmv_impl.h / vq_t_<type>.hip.
//
// Data layout in HBM: weights are the GGUF tensor bytes as uploaded (row-major, row_bytes =
// cols/block_size*type_size, rows back to back, >= VQ_TAIL_PAD readable bytes after the last row).
// Activations x[t*cols + c] fp32, outputs y[t*rows + r] fp32 (the reference's token-major layout).
#include <atomic>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include <type_traits>

#include "vq_common.h"
#include "vq_qmv.h"
#include "vq_quant.h"
#include "vq_mfma_impl.h"
#include "../../include/vq.h"

// Every per-type kernel lives in its vq_t_<type>.hip unit; here only declared (no second copy).
VQ_KERNEL_TEMPLATES(extern template, VQ_Q8_0)
VQ_KERNEL_TEMPLATES(extern template, VQ_Q2_K)
VQ_KERNEL_TEMPLATES(extern template, VQ_Q3_K)
VQ_KERNEL_TEMPLATES(extern template, VQ_Q4_K)
VQ_KERNEL_TEMPLATES(extern template, VQ_Q5_K)
VQ_KERNEL_TEMPLATES(extern template, VQ_Q6_K)
VQ_KERNEL_TEMPLATES(extern template, VQ_IQ4_NL)
VQ_KERNEL_TEMPLATES(extern template, VQ_IQ4_XS)
VQ_KERNEL_TEMPLATES(extern template, VQ_IQ3_S)
VQ_KERNEL_TEMPLATES(extern template, VQ_IQ2_XXS)
VQ_KERNEL_TEMPLATES(extern template, VQ_IQ2_XS)
VQ_KERNEL_TEMPLATES(extern template, VQ_IQ2_S)
VQ_KERNEL_TEMPLATES(extern template, VQ_IQ3_XXS)


// ---- static scratch of the no-allocation entry point (vq_qmv_noalloc) -----------------------------------
// One fixed array in device memory per GPU the library runs on, held until the process ends. Host code never
// uses the array's name as an address (on the host it names a stand-in, not device memory): vq_init looks up
// each device's copy with hipGetSymbolAddress and vq_qmv_noalloc passes that pointer to the kernels.
namespace vq {
__device__ __align__(256) uint8_t scratch[VQ_NOALLOC_SCRATCH_BYTES];
}  // namespace vq

namespace {

__device__ __forceinline__ float half_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---- activation quantizer ------------------------------------------------------------------------------
// Eight lanes per (token, 32-group): each lane loads one float4 of the group (coalesced), the group's amax
// is reduced over the eight lanes, and each lane quantizes its four values with the same IEEE operations as
// quantize_group (vq_quant.h): amax = max|v| (exact in any order), d = amax/127, id = 1/d (0 if d == 0),
// q = rint(v*id). The integer sums of the two 16-element halves (lanes 0-3 and 4-7) are exact in any order.
// Outputs go to (xq, xd, xs, xh) with per-token strides, so one kernel writes either the separate arrays of
// vq_quantize_x or the packed activation record of vq_pack_x (layout: vq_xpack_h_offset / vq_xpack_stride in
// vq_common.h).
struct XOut {
    int8_t *xq;
    float *xd, *xs;
    uint32_t *xh;  // (sum of half 0) | (sum of half 1) << 16
    long q_stride, d_stride;  // per-token strides in elements (xs and xh use d_stride)
};

__global__ __launch_bounds__(256) void quantize_x_kernel(const float *__restrict__ x, int ntok, int cols, XOut o) {
    const int ng = cols >> 5;
    const long grp = (static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x) >> 3;
    const int sub = threadIdx.x & 7;
    const bool ok = grp < static_cast<long>(ntok) * ng;
    const long gi = ok ? grp : 0;  // every lane takes part in the shuffles
    const int t = static_cast<int>(gi / ng), g = static_cast<int>(gi - static_cast<long>(t) * ng);
    const float4 f = reinterpret_cast<const float4 *>(x + static_cast<size_t>(t) * cols + 32 * g)[sub];
    float amax = 0.0f;
    amax = fmaxf(amax, fabsf(f.x));
    amax = fmaxf(amax, fabsf(f.y));
    amax = fmaxf(amax, fabsf(f.z));
    amax = fmaxf(amax, fabsf(f.w));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const int q0 = static_cast<int>(__builtin_rintf(f.x * id)), q1 = static_cast<int>(__builtin_rintf(f.y * id));
    const int q2 = static_cast<int>(__builtin_rintf(f.z * id)), q3 = static_cast<int>(__builtin_rintf(f.w * id));
    const uint32_t packed = (static_cast<uint32_t>(q0) & 0xFFu) | ((static_cast<uint32_t>(q1) & 0xFFu) << 8) |
                            ((static_cast<uint32_t>(q2) & 0xFFu) << 16) | (static_cast<uint32_t>(q3) << 24);
    int hs = q0 + q1 + q2 + q3;
    hs += __shfl_xor(hs, 1, 64);
    hs += __shfl_xor(hs, 2, 64);           // lanes 0-3: half 0, lanes 4-7: half 1
    const int hs1 = __shfl_xor(hs, 4, 64);  // lane 0: the other half
    if (!ok) return;
    reinterpret_cast<uint32_t *>(o.xq + t * o.q_stride + 32 * g)[sub] = packed;
    if (sub == 0) {
        o.xd[t * o.d_stride + g] = d;
        if (o.xs) o.xs[t * o.d_stride + g] = d * static_cast<float>(hs + hs1);
        if (o.xh) o.xh[t * o.d_stride + g] = (static_cast<uint32_t>(hs) & 0xFFFFu) | (static_cast<uint32_t>(hs1) << 16);
    }
}

// ---- float weights (F32/F16): one wave per row, fp32 activations, no quantization (qwen_cpu.c:345-360) ---
template <int T, int NT>
__global__ __launch_bounds__(256) void qmv_float_kernel(const uint8_t *__restrict__ w, int rows, int cols, long row_bytes,
                                                        const float *__restrict__ x, float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint8_t *rp = w + static_cast<size_t>(row) * row_bytes;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    for (int c = 4 * lane; c < cols; c += 256) {
        float wv[4];
        if constexpr (T == VQ_F32) {
            const float4 f = *reinterpret_cast<const float4 *>(rp + 4 * static_cast<size_t>(c));
            wv[0] = f.x;
            wv[1] = f.y;
            wv[2] = f.z;
            wv[3] = f.w;
        } else {
            const uint2 h = *reinterpret_cast<const uint2 *>(rp + 2 * static_cast<size_t>(c));
            wv[0] = half_to_float(h.x);
            wv[1] = half_to_float(h.x >> 16);
            wv[2] = half_to_float(h.y);
            wv[3] = half_to_float(h.y >> 16);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 f = *reinterpret_cast<const float4 *>(x + static_cast<size_t>(t) * cols + c);
            acc[t] = fmaf(wv[0], f.x, fmaf(wv[1], f.y, fmaf(wv[2], f.z, fmaf(wv[3], f.w, acc[t]))));
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float v = wave_sum(acc[t]);
        if (lane == 0) y[static_cast<size_t>(t) * rows + row] = v;
    }
}

template <int T>
__global__ __launch_bounds__(256) void dequant_float_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                            long row_bytes, float *__restrict__ out) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long>(rows) * cols) return;
    const long r = i / cols, c = i - r * cols;
    const uint8_t *p = w + r * row_bytes;
    out[i] = T == VQ_F32 ? reinterpret_cast<const float *>(p)[c] : half_to_float(reinterpret_cast<const uint16_t *>(p)[c]);
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

// Calls f(std::integral_constant<int, T>) for a quantized type id.
template <typename F>
int dispatch_quant(int type, F &&f) {
    switch (type) {
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
int launch_float(const uint8_t *w, int rows, int cols, const float *x, int ntok, float *y, hipStream_t s) {
    const long rb = row_bytes_of(T, cols);
    const dim3 grid((rows + 3) / 4), block(256);
    for (int c = 0; c < ntok; c += 8) {
        const int m = ntok - c < 8 ? ntok - c : 8;
        const float *xo = x + static_cast<size_t>(c) * cols;
        float *yo = y + static_cast<size_t>(c) * rows;
        switch (m) {
#define VQ_CASE(N) \
    case N: qmv_float_kernel<T, N><<<grid, block, 0, s>>>(w, rows, cols, rb, xo, yo); break;
            VQ_CASE(1) VQ_CASE(2) VQ_CASE(3) VQ_CASE(4) VQ_CASE(5) VQ_CASE(6) VQ_CASE(7) VQ_CASE(8)
#undef VQ_CASE
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_status(e);
    }
    return VQ_OK;
}

bool misaligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

// ---- f16 prefill path (vq_gemm16_impl.h): activation split and split-K reduction -----------------------------
// The split needs b as the fp32 product and hi + lo as its split: without the barrier the backend rounds the
// product straight to f16 for hi (v_fma_mix) but through fp32 for lo, and at double-rounding ties the pair
// misses b by an f16 ulp of hi (rel-L2 up to 2e-4 on the affected tokens).
__device__ __forceinline__ void opaque(float &v) { asm volatile("" : "+v"(v)); }

// One workgroup per token: b = xq * (xd 2^e) (exact scaling of the fp32 product xq * xd) as f16 hi + lo,
// 2^e the power of two with 127 max(xd) 2^e < 2^15 (every |b| 2^e fits f16); per super-block the mins' terms
// X_g xd_g 2^e / 32 (X_g = the group's code sum, |X_g| <= 32 * 127) likewise; inv = 2^-e.
__global__ __launch_bounds__(256) void gemm_xsplit_kernel(const uint8_t *__restrict__ xpack, int cols,
                                                          _Float16 *__restrict__ bh, _Float16 *__restrict__ bl,
                                                          _Float16 *__restrict__ xs, float *__restrict__ inv,
                                                          int halves) {
    const int t = blockIdx.x, tid = threadIdx.x, ng = cols >> 5;
    const uint8_t *rec = xpack + static_cast<size_t>(t) * vq_xpack_stride(cols);
    const float *xd = reinterpret_cast<const float *>(rec + cols);
    const uint32_t *xh = reinterpret_cast<const uint32_t *>(rec + vq_xpack_h_offset(cols));
    __shared__ float red[4];
    float m = 0.0f;
    for (int g = tid; g < ng; g += 256) m = fmaxf(m, xd[g]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int E = 0;
    (void)frexpf(127.0f * m, &E);  // 127 m < 2^E
    // 2^(15 - E) puts the token's largest |b| just below 2^15; capped at 2^126 so that it and 1/sc stay finite
    // and normal for tokens whose activations are below ~1e-32 (the values then stay below 2^15 instead).
    const float sc = m > 0.0f ? ldexpf(1.0f, min(15 - E, 126)) : 1.0f;
    const size_t base = static_cast<size_t>(t) * cols;
    for (int c = tid; c < cols / 8; c += 256) {
        const float ds = xd[c >> 2] * sc;
        const uint2 q = *reinterpret_cast<const uint2 *>(rec + 8 * c);
        _Float16 h[8], l[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t wd = i < 4 ? q.x : q.y;
            float v = static_cast<float>(static_cast<int8_t>(wd >> (8 * (i & 3)))) * ds;
            opaque(v);
            h[i] = static_cast<_Float16>(v);
            l[i] = static_cast<_Float16>(v - static_cast<float>(h[i]));
        }
        *reinterpret_cast<uint4 *>(bh + base + 8 * c) = __builtin_bit_cast(uint4, h);
        *reinterpret_cast<uint4 *>(bl + base + 8 * c) = __builtin_bit_cast(uint4, l);
    }
    const int nsb = cols >> 8;
    if (halves) {  // Q2_K: the 16 halves' X_h xd 2^e / 32, 16 hi then 16 lo per super-block
        for (int sb = tid; sb < nsb; sb += 256) {
            _Float16 o[32];
#pragma unroll
            for (int hh = 0; hh < 16; ++hh) {
                const int g = 8 * sb + (hh >> 1);
                const uint32_t hx = xh[g];
                const int X = static_cast<int>(static_cast<int16_t>((hh & 1) ? hx >> 16 : hx & 0xFFFFu));
                float v = static_cast<float>(X) * (xd[g] * sc) * 0.03125f;
                opaque(v);
                o[hh] = static_cast<_Float16>(v);
                o[16 + hh] = static_cast<_Float16>(v - static_cast<float>(o[hh]));
            }
            uint4 *dst = reinterpret_cast<uint4 *>(xs + (static_cast<size_t>(t) * nsb + sb) * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = __builtin_bit_cast(uint4, *reinterpret_cast<const _Float16(*)[8]>(o + 8 * i));
        }
        if (tid == 0) inv[t] = 1.0f / sc;
        return;
    }
    for (int sb = tid; sb < nsb; sb += 256) {
        _Float16 o[16];
#pragma unroll
        for (int gg = 0; gg < 8; ++gg) {
            const int g = 8 * sb + gg;
            const uint32_t hx = xh[g];
            const int X = static_cast<int>(static_cast<int16_t>(hx & 0xFFFFu)) + static_cast<int>(static_cast<int16_t>(hx >> 16));
            float v = static_cast<float>(X) * (xd[g] * sc) * 0.03125f;
            opaque(v);
            o[gg] = static_cast<_Float16>(v);
            o[8 + gg] = static_cast<_Float16>(v - static_cast<float>(o[gg]));
        }
        uint4 *dst = reinterpret_cast<uint4 *>(xs + (static_cast<size_t>(t) * nsb + sb) * 16);
        dst[0] = __builtin_bit_cast(uint4, *reinterpret_cast<const _Float16(*)[8]>(o));
        dst[1] = __builtin_bit_cast(uint4, *reinterpret_cast<const _Float16(*)[8]>(o + 8));
    }
    if (tid == 0) inv[t] = 1.0f / sc;
}

// The f16 path: Q2_K..Q6_K, IQ2_XXS/XS/S and IQ3_XXS, with the activation split addressable by the kernels' 32-bit DMA offsets.
bool gemm16_ok(int type, int cols, int M) {
    return (type == VQ_Q2_K || type == VQ_Q3_K || type == VQ_Q4_K || type == VQ_Q5_K || type == VQ_Q6_K ||
            type == VQ_IQ2_XS || type == VQ_IQ2_XXS || type == VQ_IQ2_S || type == VQ_IQ3_XXS) &&
           static_cast<long>(M) * cols < (1L << 30);
}

// Compute units of the current device (256 when there is none: workspace sizes stay computable).
int device_cus() {
    static std::atomic<int> cached[64];  // per device ordinal, 0 = not yet asked
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return 256;
    }
    if (dev >= 0 && dev < 64 && (n = cached[dev].load(std::memory_order_relaxed)) > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) {
        (void)hipGetLastError();
        return 256;
    }
    if (dev >= 0 && dev < 64) cached[dev].store(n, std::memory_order_relaxed);
    return n;
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
        case VQ_ERR_TOO_LARGE: return "needs more than the static scratch of the no-allocation entry point";
        default: return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown error";
    }
}

namespace {
constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices];  // per-device address of vq::scratch, set by vq_init
std::mutex g_scratch_mu;
}  // namespace

int vq_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= kMaxDevices) return VQ_ERR_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(vq::scratch));
        if (e != hipSuccess) return hip_status(e);
        if (p == nullptr) return VQ_ERR_NOT_INIT;
        g_scratch[dev] = p;
    }
    return VQ_OK;
}

int vq_set_iq3s_grid(const uint8_t *grid) {
    if (grid == nullptr) return VQ_ERR_ARG;
    return vq::set_iq3s_grid(grid);
}

size_t vq_xpack_bytes(int cols, int ntok) {
    if (cols <= 0 || ntok <= 0 || cols % 32) return 0;
    return static_cast<size_t>(vq_xpack_stride(cols)) * ntok;
}

// Activations of up to this many columns are quantized inside the matvec (each workgroup quantizes its own
// copy: with one workgroup per CU this beats a separate quantizer launch even for the 17408-wide FFN down
// input, measured on MI355X); wider ones are packed first.
constexpr int kFusedQuantMaxCols = 24576;

size_t vq_qmv_workspace_bytes(int cols, int ntok) {
    return cols > kFusedQuantMaxCols ? vq_xpack_bytes(cols, ntok) : 0;
}

// Small batches (6..16 tokens) take the MFMA matvec when the workspace holds the packed activations and the
// split-K partial sums: from about 6 tokens on it beats the streaming kernel, whose per-token work is VALU
// (measured on MI355X at 17408x5120 and 5120x17408).
constexpr int kMfmaMinTok = 6;
static bool mfma_batch(int type, int ntok) { return type != VQ_F32 && type != VQ_F16 && ntok >= kMfmaMinTok && ntok <= 16; }

// 5..16 tokens of Q3_K..Q6_K and the IQ types but IQ4_NL take the f16-MFMA matvec (vq_small16_impl.h) when the
// workspace holds its K-range partials (none for cols <= 512); below 5 tokens the streaming kernel is faster where it reads the
// weights once (measured on MI355X on the SwiGLU block: 2 tokens 49 vs 91 us, 4 tokens 85 vs 96 us, 8 tokens
// 171 vs 103 us). From 3 tokens on, matrices whose activation image holds fewer tokens than ntok (token_chunk:
// 2 at 17408 columns), which the streaming kernel would read twice or more, go there too.
constexpr int kSmall16MinTok = 5, kSmall16MinTokWide = 3;
static bool small16_batch(int type, int cols, int ntok) {
    return (type == VQ_Q3_K || type == VQ_Q4_K || type == VQ_Q5_K || type == VQ_Q6_K || type == VQ_IQ2_XXS ||
            type == VQ_IQ2_XS || type == VQ_IQ2_S || type == VQ_IQ3_XXS || type == VQ_IQ3_S || type == VQ_IQ4_XS) &&
           cols % 256 == 0 &&
           ntok <= 16 && (ntok >= kSmall16MinTok || (ntok >= kSmall16MinTokWide && ntok > vq::token_chunk(cols)));
}

// The path vq_qmv takes (VQ_PATH_*), given whether a usable (non-NULL, 16-byte aligned) workspace of wsb
// bytes comes with the call.
// Head of the staged small-batch workspace: the per-token RMS scales (16 floats, padded).
constexpr size_t kStagedRsBytes = 256;

static int qmv_route(int type, int rows, int cols, int ntok, bool ws, size_t wsb) {
    if (type == VQ_F32 || type == VQ_F16) return VQ_PATH_STREAM;
    if (small16_batch(type, cols, ntok)) {
        const size_t np = vq::s16_part_bytes(rows, cols, ntok);
        if (np == 0 || (ws && wsb >= np)) return VQ_PATH_MFMA_F16;
    }
    if (mfma_batch(type, ntok)) {
        const size_t np = vq::mfma_part_bytes(rows, cols, ntok);
        if (np == 0 || (ws && wsb >= np)) return VQ_PATH_MFMA_I8;
    }
    return VQ_PATH_STREAM;
}

size_t vq_qmv_workspace_bytes_for(int type, int rows, int cols, int ntok) {
    if (check_matrix(type, rows, cols) || ntok < 1) return 0;
    if (small16_batch(type, cols, ntok)) return vq::s16_part_bytes(rows, cols, ntok);
    if (mfma_batch(type, ntok)) return vq::mfma_part_bytes(rows, cols, ntok);
    return (type == VQ_F32 || type == VQ_F16) ? 0 : vq_qmv_workspace_bytes(cols, ntok);
}

int vq_qmv_path(int type, int rows, int cols, int ntok, size_t workspace_bytes) {
    const int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (ntok < 1) return VQ_ERR_SHAPE;
    return qmv_route(type, rows, cols, ntok, workspace_bytes > 0, workspace_bytes);
}

int vq_quantize_x(const float *x, int ntok, int cols, int8_t *xq, float *xd, float *xs, void *stream) {
    if (!x || !xq || !xd) return VQ_ERR_ARG;
    if (ntok < 1 || cols < 32 || cols % 32) return VQ_ERR_SHAPE;
    const long n = 8L * ntok * (cols / 32);  // eight lanes per group
    const XOut o{xq, xd, xs, nullptr, cols, cols / 32};
    quantize_x_kernel<<<(n + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(x, ntok, cols, o);
    return hip_status(hipGetLastError());
}

int vq_pack_x(const float *x, int ntok, int cols, void *xpack, void *stream) {
    if (!x || !xpack) return VQ_ERR_ARG;
    if (ntok < 1 || cols < 32 || cols % 32) return VQ_ERR_SHAPE;
    const long n = 8L * ntok * (cols / 32);  // eight lanes per group
    const long stride = vq_xpack_stride(cols);
    char *base = static_cast<char *>(xpack);
    const XOut o{reinterpret_cast<int8_t *>(base), reinterpret_cast<float *>(base + cols), nullptr,
                 reinterpret_cast<uint32_t *>(base + vq_xpack_h_offset(cols)), stride, stride / 4};
    quantize_x_kernel<<<(n + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(x, ntok, cols, o);
    return hip_status(hipGetLastError());
}

static_assert(VQ_QMV_ADD == VQ_STAGE_ADD && VQ_QMV_NORM == VQ_STAGE_NORM && VQ_QMV_SILU_MUL == VQ_STAGE_SILU_MUL,
              "public and kernel staging flags agree");

int vq_qmv_staged(int type, const uint8_t *w, int rows, int cols, const float *x, const float *x2,
                  const float *norm_w, float eps, int flags, int ntok, float *y, void *stream) {
    const int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;  // staging feeds the int8 activation path
    if (ntok < 1 || cols > kFusedQuantMaxCols) return VQ_ERR_SHAPE;
    if (flags & ~(VQ_QMV_ADD | VQ_QMV_NORM | VQ_QMV_SILU_MUL)) return VQ_ERR_ARG;
    if (!w || !x || !y || misaligned16(w) || misaligned16(x)) return VQ_ERR_ARG;
    if ((flags & VQ_QMV_SILU_MUL) && (!x2 || misaligned16(x2))) return VQ_ERR_ARG;
    if ((flags & VQ_QMV_NORM) && (!norm_w || misaligned16(norm_w) || !(eps >= 0.0f))) return VQ_ERR_ARG;
    const vq::XStage xs{(flags & VQ_QMV_SILU_MUL) ? x2 : nullptr, (flags & VQ_QMV_NORM) ? norm_w : nullptr, eps,
                        flags};
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_quant_staged<decltype(tc)::value>(w, rows, cols, rb, x, xs, ntok, y, s);
    });
}

size_t vq_qmv_staged_workspace_bytes(int type, int rows, int cols, int ntok) {
    if (check_matrix(type, rows, cols) || ntok < 1 || type == VQ_F32 || type == VQ_F16) return 0;
    if (!small16_batch(type, cols, ntok)) return 0;
    return kStagedRsBytes + vq::s16_part_bytes(rows, cols, ntok);
}

int vq_qmv_staged_ws(int type, const uint8_t *w, int rows, int cols, const float *x, const float *x2,
                     const float *norm_w, float eps, int flags, int ntok, float *y, void *workspace,
                     size_t workspace_bytes, void *stream) {
    const int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;
    if (ntok < 1) return VQ_ERR_SHAPE;
    if (flags & ~(VQ_QMV_ADD | VQ_QMV_NORM | VQ_QMV_SILU_MUL)) return VQ_ERR_ARG;
    if (!w || !x || !y || misaligned16(w) || misaligned16(x)) return VQ_ERR_ARG;
    if ((flags & VQ_QMV_SILU_MUL) && (!x2 || misaligned16(x2))) return VQ_ERR_ARG;
    if ((flags & VQ_QMV_NORM) && (!norm_w || misaligned16(norm_w) || !(eps >= 0.0f))) return VQ_ERR_ARG;
    const size_t need = vq_qmv_staged_workspace_bytes(type, rows, cols, ntok);
    if (need == 0 || !workspace || misaligned16(workspace) || workspace_bytes < need)
        return vq_qmv_staged(type, w, rows, cols, x, x2, norm_w, eps, flags, ntok, y, stream);
    const vq::XStage xs{(flags & VQ_QMV_SILU_MUL) ? x2 : nullptr, (flags & VQ_QMV_NORM) ? norm_w : nullptr, eps,
                        flags};
    float *const rs = static_cast<float *>(workspace);
    float *const part = vq::s16_part_bytes(rows, cols, ntok)
                            ? reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + kStagedRsBytes)
                            : nullptr;
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_small16<decltype(tc)::value>(w, rows, cols, rb, x, ntok, y, part, s, xs, rs);
    });
}

int vq_qmv_packed(int type, const uint8_t *w, int rows, int cols, const void *xpack, int ntok, float *y, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;  // float weights take fp32 activations (vq_qmv)
    if (!w || !xpack || !y || misaligned16(w) || misaligned16(xpack)) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_quant<decltype(tc)::value>(w, rows, cols, rb, xpack, false, ntok, y, s);
    });
}

int vq_qmv(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, float *y, void *workspace,
           size_t workspace_bytes, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (!w || !x || !y || misaligned16(w) || misaligned16(x)) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (type == VQ_F32) return launch_float<VQ_F32>(w, rows, cols, x, ntok, y, s);
    if (type == VQ_F16) return launch_float<VQ_F16>(w, rows, cols, x, ntok, y, s);
    const long rb = row_bytes_of(type, cols);
    const bool ws = workspace && !misaligned16(workspace);
    const int path = qmv_route(type, rows, cols, ntok, ws, workspace_bytes);
    if (path == VQ_PATH_MFMA_F16) {
        float *part = vq::s16_part_bytes(rows, cols, ntok) ? static_cast<float *>(workspace) : nullptr;
        return dispatch_quant(type, [&](auto tc) {
            return vq::launch_small16<decltype(tc)::value>(w, rows, cols, rb, x, ntok, y, part, s);
        });
    }
    if (path == VQ_PATH_MFMA_I8) {
        float *part = vq::mfma_part_bytes(rows, cols, ntok) ? static_cast<float *>(workspace) : nullptr;
        return dispatch_quant(type, [&](auto tc) {
            return vq::launch_mfma<decltype(tc)::value>(w, rows, cols, rb, x, ntok, y, part, s);
        });
    }
    const size_t need = vq_qmv_workspace_bytes(cols, ntok);
    if (need > 0) {
        if (!workspace || workspace_bytes < need || misaligned16(workspace)) return VQ_ERR_WORKSPACE;
        st = vq_pack_x(x, ntok, cols, workspace, stream);
        if (st) return st;
        return vq_qmv_packed(type, w, rows, cols, workspace, ntok, y, stream);
    }
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_quant<decltype(tc)::value>(w, rows, cols, rb, x, true, ntok, y, s);
    });
}

int vq_qmv_noalloc(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, float *y, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (ntok < 1) return VQ_ERR_SHAPE;
    const size_t need = vq_qmv_workspace_bytes_for(type, rows, cols, ntok);
    if (need > VQ_NOALLOC_SCRATCH_BYTES) return VQ_ERR_TOO_LARGE;
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    void *ws = dev >= 0 && dev < kMaxDevices ? g_scratch[dev] : nullptr;  // written once by vq_init
    if (ws == nullptr) return VQ_ERR_NOT_INIT;
    // The same kernels and routing as vq_qmv with a workspace of `need` bytes (none of them needs the scratch
    // cleared first: every byte a kernel reads back was written earlier in the same call).
    return vq_qmv(type, w, rows, cols, x, ntok, y, need ? ws : nullptr, need, stream);
}

static int qmv_group_any(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                         const void *x, bool x_f32, int ntok, void *stream) {
    if (n < 1 || n > VQ_MAX_GROUP || !w || !rows || !y) return VQ_ERR_ARG;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;
    for (int k = 0; k < n; ++k) {
        const int st = check_matrix(type, rows[k], cols);
        if (st) return st;
        if (!w[k] || !y[k] || misaligned16(w[k])) return VQ_ERR_ARG;
    }
    if (!x || misaligned16(x)) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_quant_jobs<decltype(tc)::value>(n, w, rows, y, cols, x, x_f32, ntok, nullptr, nullptr, s);
    });
}

int vq_qmv_group(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                 const void *xpack, int ntok, void *stream) {
    return qmv_group_any(type, n, w, rows, y, cols, xpack, false, ntok, stream);
}

int vq_qmv_group_f32(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                     const float *x, int ntok, void *stream) {
    return qmv_group_any(type, n, w, rows, y, cols, x, true, ntok, stream);
}

// Grouped matvec with vq_qmv's batch routing: 5..16 tokens of Q3_K..Q6_K in one f16-MFMA launch over every
// matrix's row tiles (plus one launch of K-range sums); other MFMA batches matrix by matrix through vq_qmv;
// everything else as vq_qmv_group_f32 (one streaming launch) or, past the in-kernel quantizer's width, vq_qmv.
static bool group_args_ok(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                          const float *x, int ntok, int *st) {
    *st = VQ_OK;
    if (n < 1 || n > VQ_MAX_GROUP || !w || !rows || !y || !x || misaligned16(x)) *st = VQ_ERR_ARG;
    else if (type == VQ_F32 || type == VQ_F16) *st = VQ_ERR_TYPE;
    else if (ntok < 1) *st = VQ_ERR_SHAPE;
    for (int k = 0; *st == VQ_OK && k < n; ++k) {
        *st = check_matrix(type, rows[k], cols);
        if (*st == VQ_OK && (!w[k] || !y[k] || misaligned16(w[k]))) *st = VQ_ERR_ARG;
    }
    return *st == VQ_OK;
}

size_t vq_qmv_group_workspace_bytes(int type, int n, const int *rows, int cols, int ntok) {
    if (n < 1 || n > VQ_MAX_GROUP || !rows || ntok < 1) return 0;
    size_t s16 = 0, most = 0;
    for (int k = 0; k < n; ++k) {
        if (check_matrix(type, rows[k], cols)) return 0;
        s16 += vq::s16_part_bytes(rows[k], cols, ntok);
        const size_t one = vq_qmv_workspace_bytes_for(type, rows[k], cols, ntok);
        most = one > most ? one : most;
    }
    return small16_batch(type, cols, ntok) ? s16 : most;
}

int vq_qmv_group_ws(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                    const float *x, int ntok, void *workspace, size_t workspace_bytes, void *stream) {
    int st;
    if (!group_args_ok(type, n, w, rows, y, cols, x, ntok, &st)) return st;
    const bool ws = workspace && !misaligned16(workspace);
    if (small16_batch(type, cols, ntok)) {
        size_t need = 0;
        for (int k = 0; k < n; ++k) need += vq::s16_part_bytes(rows[k], cols, ntok);
        if (need == 0 || (ws && workspace_bytes >= need)) {
            hipStream_t s = static_cast<hipStream_t>(stream);
            const long rb = row_bytes_of(type, cols);
            float *part = need ? static_cast<float *>(workspace) : nullptr;
            return dispatch_quant(type, [&](auto tc) {
                return vq::launch_small16_group<decltype(tc)::value>(n, w, rows, y, cols, rb, x, ntok, part, s);
            });
        }
    }
    bool each = false;
    for (int k = 0; k < n && !each; ++k)
        each = qmv_route(type, rows[k], cols, ntok, ws, workspace_bytes) != VQ_PATH_STREAM;
    if (!each) {
        const size_t pk = vq_qmv_workspace_bytes(cols, ntok);  // wide inputs: packed once for the group
        if (pk == 0) return vq_qmv_group_f32(type, n, w, rows, y, cols, x, ntok, stream);
        if (!ws || workspace_bytes < pk) return VQ_ERR_WORKSPACE;
        st = vq_pack_x(x, ntok, cols, workspace, stream);
        return st ? st : vq_qmv_group(type, n, w, rows, y, cols, workspace, ntok, stream);
    }
    for (int k = 0; k < n; ++k) {  // in stream order, each call done with the workspace before the next uses it
        st = vq_qmv(type, w[k], rows[k], cols, x, ntok, y[k], workspace, workspace_bytes, stream);
        if (st) return st;
    }
    return VQ_OK;
}

int vq_qmv_group_mixed_f32(int n, const int *types, const uint8_t *const *w, const int *rows, float *const *y,
                           int cols, const float *x, int ntok, void *stream) {
    if (n < 1 || n > VQ_MAX_GROUP || !types || !w || !rows || !y) return VQ_ERR_ARG;
    int main_type = -1;
    bool mixed = false;
    for (int k = 0; k < n; ++k) {
        if (types[k] == VQ_F32 || types[k] == VQ_F16) return VQ_ERR_TYPE;
        const int st = check_matrix(types[k], rows[k], cols);
        if (st) return st;
        if (!w[k] || !y[k] || misaligned16(w[k])) return VQ_ERR_ARG;
        if (types[k] != VQ_Q8_0) {
            if (main_type >= 0 && types[k] != main_type) mixed = true;  // two non-Q8_0 types
            main_type = types[k];
        }
    }
    if (!x || misaligned16(x)) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    if (main_type < 0) main_type = VQ_Q8_0;
    bool q5q6 = mixed;  // Q5_K with Q6_K, nothing else: one launch
    for (int k = 0; k < n; ++k) q5q6 = q5q6 && (types[k] == VQ_Q5_K || types[k] == VQ_Q6_K);
    if (q5q6)
        return vq::launch_mixed2<VQ_Q5_K, VQ_Q6_K>(n, types, w, rows, y, cols, x, ntok, static_cast<hipStream_t>(stream));
    if (mixed) {
        // Other mixes: one grouped launch per type, in order of first appearance.
        bool done[VQ_MAX_GROUP] = {};
        for (int k = 0; k < n; ++k) {
            if (done[k]) continue;
            const uint8_t *wk[VQ_MAX_GROUP];
            int rk[VQ_MAX_GROUP];
            float *yk[VQ_MAX_GROUP];
            int m = 0;
            for (int j = k; j < n; ++j)
                if (!done[j] && types[j] == types[k]) {
                    wk[m] = w[j];
                    rk[m] = rows[j];
                    yk[m] = y[j];
                    ++m;
                    done[j] = true;
                }
            const int st = vq_qmv_group_f32(types[k], m, wk, rk, yk, cols, x, ntok, stream);
            if (st) return st;
        }
        return VQ_OK;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    return dispatch_quant(main_type, [&](auto tc) {
        return vq::launch_mixed_q8<decltype(tc)::value>(n, types, w, rows, y, cols, x, ntok, s);
    });
}

int vq_qgemm(int type, const uint8_t *w, int rows, int cols, const void *xpack, int M, float *y, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;
    if (!w || !xpack || !y || misaligned16(w) || misaligned16(xpack)) return VQ_ERR_ARG;
    if (M < 1) return VQ_ERR_SHAPE;
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *xp = static_cast<const uint8_t *>(xpack);
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_gemm<decltype(tc)::value>(w, rows, cols, rb, xp, M, y, s);
    });
}

size_t vq_qgemm_workspace_bytes_ex(int type, int rows, int cols, int M, int flags) {
    if (check_matrix(type, rows, cols) || M < 1 || !gemm16_ok(type, cols, M) || (flags & ~VQ_GEMM_BATCH_INVARIANT))
        return 0;
    return vq::g16_layout(cols, M, vq::g16_plan(rows, cols, M, device_cus(), flags & VQ_GEMM_BATCH_INVARIANT),
                          type == VQ_Q2_K).total;
}

size_t vq_qgemm_workspace_bytes(int type, int rows, int cols, int M) {
    return vq_qgemm_workspace_bytes_ex(type, rows, cols, M, 0);
}

int vq_qgemm_ws_ex(int type, const uint8_t *w, int rows, int cols, const void *xpack, int M, float *y, void *workspace,
                   size_t workspace_bytes, int flags, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;
    if (flags & ~VQ_GEMM_BATCH_INVARIANT) return VQ_ERR_ARG;
    if (!w || !xpack || !y || misaligned16(w) || misaligned16(xpack)) return VQ_ERR_ARG;
    if (M < 1) return VQ_ERR_SHAPE;
    const bool inv = (flags & VQ_GEMM_BATCH_INVARIANT) != 0;
    const size_t need = vq_qgemm_workspace_bytes_ex(type, rows, cols, M, flags);
    if (need == 0) return vq_qgemm(type, w, rows, cols, xpack, M, y, stream);  // int8 path: full K per tile
    if (!workspace || workspace_bytes < need || misaligned16(workspace)) return VQ_ERR_WORKSPACE;
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int cus = device_cus();
    const vq::G16Ws l = vq::g16_layout(cols, M, vq::g16_plan(rows, cols, M, cus, inv), type == VQ_Q2_K);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    gemm_xsplit_kernel<<<M, 256, 0, s>>>(static_cast<const uint8_t *>(xpack), cols, reinterpret_cast<_Float16 *>(ws + l.bh),
                                         reinterpret_cast<_Float16 *>(ws + l.bl), reinterpret_cast<_Float16 *>(ws + l.xs),
                                         reinterpret_cast<float *>(ws + l.inv), type == VQ_Q2_K ? 1 : 0);
    st = hip_status(hipGetLastError());
    if (st) return st;
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_gemm16<decltype(tc)::value>(w, rows, cols, rb, ws, M, y, cus, s, inv);
    });
}

// Activations of the f16x contraction, one workgroup per token: b_hi = f16(x 2^e) rounded to nearest even, with
// the token's 2^e putting its largest |x| just below 2^15 (capped at 2^126, as for the split above); b_lo is not
// written. xs: per 32-group the fp32 sum of the rounded values (eight per thread in order, then the four threads
// of the group pairwise: a fixed order) times 2^-5, as f16 hi then lo, 8 groups per super-block; halves (Q2_K):
// per 16-element half (two threads), 16 hi then 16 lo per super-block.
__global__ __launch_bounds__(256) void gemm_f16x_split_kernel(const float *__restrict__ x, int cols,
                                                              _Float16 *__restrict__ bh, _Float16 *__restrict__ xs,
                                                              float *__restrict__ inv, int halves) {
    // Rows of up to 256 x KR chunks of 8 values (18432 columns) are read once, into registers; longer rows are
    // read again past that for the conversion.
    constexpr int KR = 9;
    const int t = blockIdx.x, tid = threadIdx.x, nch = cols / 8;
    const float4 *xr = reinterpret_cast<const float4 *>(x + static_cast<size_t>(t) * cols);
    __shared__ float red[4];
    auto amax = [](float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
    float4 r[KR][2];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int c = tid + 256 * k;
        if (c < nch) {
            r[k][0] = xr[2 * c];
            r[k][1] = xr[2 * c + 1];
            m = fmaxf(m, fmaxf(amax(r[k][0]), amax(r[k][1])));
        }
    }
    for (int c = tid + 256 * KR; c < nch; c += 256) m = fmaxf(m, fmaxf(amax(xr[2 * c]), amax(xr[2 * c + 1])));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int E = 0;
    (void)frexpf(m, &E);  // m < 2^E
    const float sc = m > 0.0f ? ldexpf(1.0f, min(15 - E, 126)) : 1.0f;
    const size_t base = static_cast<size_t>(t) * cols;
    const int nsb = cols >> 8;
    // Chunk c (8 values): b_hi, then its group's (or half's) sum. nch is a multiple of 32, so the four threads of a
    // group (consecutive c) are active together.
    auto convert = [&](int c, float4 v0, float4 v1) {
        const float f[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        _Float16 h[8];
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            h[i] = static_cast<_Float16>(f[i] * sc);
            sum += static_cast<float>(h[i]);
        }
        *reinterpret_cast<uint4 *>(bh + base + 8 * c) = __builtin_bit_cast(uint4, h);
        sum += __shfl_xor(sum, 1, 64);
        if (halves) {
            if ((c & 1) == 0) {
                float v = sum * 0.03125f;
                opaque(v);
                const _Float16 hi = static_cast<_Float16>(v);
                _Float16 *const dst = xs + (static_cast<size_t>(t) * nsb + (c >> 5)) * 32 + ((c >> 1) & 15);
                dst[0] = hi;
                dst[16] = static_cast<_Float16>(v - static_cast<float>(hi));
            }
            return;
        }
        sum += __shfl_xor(sum, 2, 64);
        if ((c & 3) == 0) {
            const int g = c >> 2;
            float v = sum * 0.03125f;
            opaque(v);
            const _Float16 hi = static_cast<_Float16>(v);
            _Float16 *const dst = xs + (static_cast<size_t>(t) * nsb + (g >> 3)) * 16 + (g & 7);
            dst[0] = hi;
            dst[8] = static_cast<_Float16>(v - static_cast<float>(hi));
        }
    };
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int c = tid + 256 * k;
        if (c < nch) convert(c, r[k][0], r[k][1]);
    }
    for (int c = tid + 256 * KR; c < nch; c += 256) convert(c, xr[2 * c], xr[2 * c + 1]);
    if (tid == 0) inv[t] = 1.0f / sc;
}

int vq_qgemm_f16x_ws(int type, const uint8_t *w, int rows, int cols, const float *x, int M, float *y, void *workspace,
                     size_t workspace_bytes, int flags, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16 || !gemm16_ok(type, cols, 1)) return VQ_ERR_TYPE;
    if (flags & ~VQ_GEMM_BATCH_INVARIANT) return VQ_ERR_ARG;
    if (!w || !x || !y || misaligned16(w) || misaligned16(x)) return VQ_ERR_ARG;
    if (M < 1) return VQ_ERR_SHAPE;
    const size_t need = vq_qgemm_workspace_bytes_ex(type, rows, cols, M, flags);
    if (need == 0) return VQ_ERR_SHAPE;
    if (!workspace || workspace_bytes < need || misaligned16(workspace)) return VQ_ERR_WORKSPACE;
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool invariant = (flags & VQ_GEMM_BATCH_INVARIANT) != 0;
    const bool halves = type == VQ_Q2_K;
    const vq::G16Ws l = vq::g16_layout(cols, M, vq::g16_plan(rows, cols, M, device_cus(), invariant), halves);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    gemm_f16x_split_kernel<<<M, 256, 0, s>>>(x, cols, reinterpret_cast<_Float16 *>(ws + l.bh),
                                             reinterpret_cast<_Float16 *>(ws + l.xs), reinterpret_cast<float *>(ws + l.inv),
                                             halves ? 1 : 0);
    st = hip_status(hipGetLastError());
    if (st) return st;
    const int cus = device_cus();
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_gemm16<decltype(tc)::value>(w, rows, cols, rb, ws, M, y, cus, s, invariant, true);
    });
}

int vq_qgemm_ws(int type, const uint8_t *w, int rows, int cols, const void *xpack, int M, float *y, void *workspace,
                size_t workspace_bytes, void *stream) {
    return vq_qgemm_ws_ex(type, w, rows, cols, xpack, M, y, workspace, workspace_bytes, 0, stream);
}

size_t vq_lmhead_argmax_workspace_bytes(int type, int rows, int cols, int ntok) {
    if (check_matrix(type, rows, cols) || type == VQ_F32 || type == VQ_F16 || ntok < 1) return 0;
    const long kw = dispatch_quant(type, [&](auto tc) {
        return static_cast<int>(vq::argmax_waves<decltype(tc)::value>(rows, cols, ntok));
    });
    return align256(static_cast<size_t>(ntok) * kw * 8) + vq_qmv_workspace_bytes(cols, ntok);
}

int vq_lmhead_argmax(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, int32_t *out_idx,
                     float *logits, void *workspace, size_t workspace_bytes, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;
    if (!w || !x || !out_idx || misaligned16(w) || misaligned16(x)) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    const size_t need = vq_lmhead_argmax_workspace_bytes(type, rows, cols, ntok);
    if (!workspace || workspace_bytes < need || misaligned16(workspace)) return VQ_ERR_WORKSPACE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto *keys = static_cast<unsigned long long *>(workspace);
    const size_t pack_bytes = vq_qmv_workspace_bytes(cols, ntok);
    const void *xin = x;
    if (pack_bytes > 0) {
        void *xp = static_cast<uint8_t *>(workspace) + (need - pack_bytes);
        st = vq_pack_x(x, ntok, cols, xp, stream);
        if (st) return st;
        xin = xp;
    }
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_quant_jobs<decltype(tc)::value>(1, &w, &rows, &logits, cols, xin, pack_bytes == 0, ntok,
                                                          keys, out_idx, s);
    });
}

int vq_int_partials(int type, const uint8_t *w, int rows, int cols, const void *xpack, int ntok, int32_t *part,
                    void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (type == VQ_F32 || type == VQ_F16) return VQ_ERR_TYPE;
    if (!w || !xpack || !part) return VQ_ERR_ARG;
    if (ntok < 1) return VQ_ERR_SHAPE;
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *xp = static_cast<const uint8_t *>(xpack);
    return dispatch_quant(type, [&](auto tc) {
        return vq::launch_partials<decltype(tc)::value>(w, rows, cols, rb, xp, ntok, part, s);
    });
}
int vq_dequant_rows(int type, const uint8_t *w, int rows, int cols, float *out, void *stream) {
    int st = check_matrix(type, rows, cols);
    if (st) return st;
    if (!w || !out) return VQ_ERR_ARG;
    const long rb = row_bytes_of(type, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (type == VQ_F32 || type == VQ_F16) {
        const long n = static_cast<long>(rows) * cols;
        if (type == VQ_F32)
            dequant_float_kernel<VQ_F32><<<(n + 255) / 256, 256, 0, s>>>(w, rows, cols, rb, out);
        else
            dequant_float_kernel<VQ_F16><<<(n + 255) / 256, 256, 0, s>>>(w, rows, cols, rb, out);
        return hip_status(hipGetLastError());
    }
    return dispatch_quant(type, [&](auto tc) { return vq::launch_dequant<decltype(tc)::value>(w, rows, cols, rb, out, s); });
}

int vq_argmax_rows(const float *x, int n, int ntok, int32_t *out, void *stream) {
    if (!x || !out) return VQ_ERR_ARG;
    if (n < 1 || ntok < 1) return VQ_ERR_SHAPE;
    argmax_rows_kernel<<<ntok, 1024, 0, static_cast<hipStream_t>(stream)>>>(x, n, out);
    return hip_status(hipGetLastError());
}

}  // extern "C"
