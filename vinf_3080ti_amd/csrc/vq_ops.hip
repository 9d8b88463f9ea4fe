// vq_ops.hip -- the runtime's elementwise and normalisation ops around the matvec (the reference runtime's
// rmsnorm_kernel, gated_rmsnorm_kernel, add/silu_mul/sigmoid_mul kernels, qwen_runtime.cu:36-67): HBM-bound
// streams in fp32.
//
// RMS sums: each thread adds its strided elements in order, then a fixed pairwise tree over the 256 threads in
// LDS, so a group's result does not depend on timing. silu / sigmoid use expf and an IEEE division (these
// passes are bound by bytes, not by VALU).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vq.h"

namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float silu_ieee(float z) { return z / (1.0f + expf(-z)); }
__device__ __forceinline__ float sigmoid_ieee(float z) { return 1.0f / (1.0f + expf(-z)); }

// Group g: y = x * rsqrt(mean(x^2) + eps) * w (* silu(z) when z is given). In-place safe (every element is
// read before it is written, by the same thread).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                               const float *__restrict__ z, float *y, int n, float eps) {
    __shared__ float part[kNormThreads];
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    const int tid = threadIdx.x;
    float acc = 0.0f;
    for (int i = tid; i < n; i += kNormThreads) acc = fmaf(x[base + i], x[base + i], acc);
    part[tid] = acc;
    for (int h = kNormThreads / 2; h > 0; h >>= 1) {
        __syncthreads();
        if (tid < h) part[tid] += part[tid + h];
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf(part[0] / static_cast<float>(n) + eps);
    for (int i = tid; i < n; i += kNormThreads) {
        float v = x[base + i] * scale * w[i];
        if (z != nullptr) v *= silu_ieee(z[base + i]);
        y[base + i] = v;
    }
}

// out = a + b (op 0), silu(a) * b (op 1), a * sigmoid(b) (op 2): four elements per thread.
template <int OP>
__device__ __forceinline__ float binop(float a, float b) {
    if constexpr (OP == 0) return a + b;
    else if constexpr (OP == 1) return silu_ieee(a) * b;
    else return a * sigmoid_ieee(b);
}
template <int OP>
__global__ __launch_bounds__(256) void binary_kernel(const float *a, const float *b, float *out, long n) {
    const long i = (static_cast<long>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i + 4 <= n && ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                        reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
        const float4 x = *reinterpret_cast<const float4 *>(a + i), y = *reinterpret_cast<const float4 *>(b + i);
        *reinterpret_cast<float4 *>(out + i) = float4{binop<OP>(x.x, y.x), binop<OP>(x.y, y.y), binop<OP>(x.z, y.z),
                                                      binop<OP>(x.w, y.w)};
    } else {
        for (long k = i; k < i + 4 && k < n; ++k) out[k] = binop<OP>(a[k], b[k]);
    }
}

int status_of(hipError_t e) { return e == hipSuccess ? VQ_OK : static_cast<int>(e); }

}  // namespace

extern "C" {

int vq_rmsnorm(const float *x, const float *w, const float *z, float *y, int n, int groups, float eps, void *stream) {
    if (!x || !w || !y) return VQ_ERR_ARG;
    if (n < 1 || groups < 1 || !(eps >= 0.0f)) return VQ_ERR_SHAPE;
    rmsnorm_kernel<<<groups, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(x, w, z, y, n, eps);
    return status_of(hipGetLastError());
}

int vq_binary(int op, const float *a, const float *b, float *out, long n, void *stream) {
    if (!a || !b || !out) return VQ_ERR_ARG;
    if (op < 0 || op > 2) return VQ_ERR_ARG;
    if (n < 0) return VQ_ERR_SHAPE;
    if (n == 0) return VQ_OK;
    const unsigned blocks = static_cast<unsigned>((n + 1023) / 1024);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (op == 0) binary_kernel<0><<<blocks, 256, 0, s>>>(a, b, out, n);
    else if (op == 1) binary_kernel<1><<<blocks, 256, 0, s>>>(a, b, out, n);
    else binary_kernel<2><<<blocks, 256, 0, s>>>(a, b, out, n);
    return status_of(hipGetLastError());
}

}  // extern "C"
