// vq_qmv.h -- host-side declarations of the per-type quantized kernels (defined in vq_qmv_impl.h and
// instantiated once per GGUF type in vq_t_<type>.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vq {

// Activation image geometry of the streaming kernel.
constexpr int kXLdsMax = 64 * 1024;  // bytes of activation records one launch keeps in LDS
constexpr int kXPad = 16;            // bytes of padding after each 256 codes of the image (bank spread)
// Bytes of one token's activation image (codes padded per 256, then 8 bytes of scales per 32-group).
__host__ __device__ inline int x_image_bytes(int cols) {
    return (((cols / 32 + 7) / 8) * (256 + kXPad) + (cols / 32) * 8 + 15) / 16 * 16;
}
// Activation staging of the fp32-input streaming matvec (the bits of the reference megakernel's QMV flags,
// runtime/instructions.py:179-182): ADD accumulates into y, NORM stages rmsnorm(v) * nw, SILU_MUL stages
// silu(x) * x2.
#define VQ_STAGE_ADD 1
#define VQ_STAGE_NORM 2
#define VQ_STAGE_SILU_MUL 8
struct XStage {
    const float *x2;  // [ntok][cols] second input of SILU_MUL
    const float *nw;  // [cols] RMS norm weights of NORM
    float eps;
    int flags;
};

// Tokens per streaming launch (one weight pass): as many (<= 8) as the activation image budget holds.
inline int token_chunk(int cols) {
    const int chunk = kXLdsMax / x_image_bytes(cols);
    return chunk > 8 ? 8 : chunk < 1 ? 1 : chunk;
}

template <int T>
int launch_quant(const uint8_t *w, int rows, int cols, long row_bytes, const void *x, bool x_f32, int ntok, float *y,
                 hipStream_t s);
// y_j = W_j x for n <= 4 matrices of type T sharing cols and x; optional fused argmax (n == 1): `amax` holds
// [ntok][argmax_waves] keys, amax_out[t] receives the index.
template <int T>
int launch_quant_jobs(int n, const uint8_t *const *w, const int *rows, float *const *y, int cols, const void *x,
                      bool x_f32, int ntok, unsigned long long *amax, int32_t *amax_out, hipStream_t s);
template <int T>
long argmax_waves(int rows, int cols, int ntok);
// y = W v for fp32 activations staged per `xs` (flags VQ_STAGE_*; x2 and nw already offset to token 0).
template <int T>
int launch_quant_staged(const uint8_t *w, int rows, int cols, long row_bytes, const float *x, const XStage &xs,
                        int ntok, float *y, hipStream_t s);
// y_j = W_j x for n <= 4 matrices sharing cols and fp32 x, of type T or Q8_0 (types[j]), in one launch.
constexpr int kMixedMaxTokens = 4;  // tokens per launch of a mixed-type group (more go in several launches)
template <int T>
int launch_mixed_q8(int n, const int *types, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                    const float *x, int ntok, hipStream_t s);
// Jobs of two K-quant types reading one fp32 input in one launch (a full-attention layer's Q5_K q next to its Q6_K
// k and v); instantiated for (Q5_K, Q6_K).
template <int T, int T2>
int launch_mixed2(int n, const int *types, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                  const float *x, int ntok, hipStream_t s);
// Prefill contraction on int8 MFMA: y[t][r] = W[r] . x[t] for t < M, activations packed (vq_pack_x).
template <int T>
int launch_gemm(const uint8_t *w, int rows, int cols, long row_bytes, const uint8_t *xpack, int M, float *y,
                hipStream_t s);
// Prefill contraction on f16 MFMA (Q2_K..Q6_K, IQ2_XXS/XS/S, IQ3_XXS; other types return hipErrorInvalidValue): `ws` holds the split
// activations written by the library's pre-pass and the partial-tile slots (layout g16_layout for
// g16_plan(rows, cols, M, cus, invariant)) and the reduction of split tiles; invariant: the K split depends on the
// matrix only (batch-invariant results); f16x: the activations are b_hi alone, rounded to f16 (Q4_K and Q5_K).
template <int T>
int launch_gemm16(const uint8_t *w, int rows, int cols, long row_bytes, const void *ws, int M, float *y, int cus,
                  hipStream_t s, bool invariant, bool f16x = false);
// Matvec of 1..16 tokens on f16 MFMA (Q3_K, Q4_K, Q5_K, Q6_K; other types return hipErrorInvalidValue), fp32
// activations; `part` holds s16_part_bytes(rows, cols, ntok) bytes (unused when that is 0).
template <int T>
int launch_small16_group(int n, const uint8_t *const *w, const int *rows, float *const *y, int cols, long row_bytes,
                         const float *x, int ntok, float *part, hipStream_t s, const XStage &xs = XStage{},
                         float *rs = nullptr);
template <int T>
int launch_small16(const uint8_t *w, int rows, int cols, long row_bytes, const float *x, int ntok, float *y,
                   float *part, hipStream_t s, const XStage &xs = XStage{}, float *rs = nullptr);
// Small-batch (2..16 tokens) matvec on int8 MFMA over fp32 activations (quantized in the kernel); `part` holds
// mfma_part_bytes(rows, cols, ntok) bytes (unused when that is 0).
template <int T>
int launch_mfma(const uint8_t *w, int rows, int cols, long row_bytes, const float *x, int ntok, float *y,
                float *part, hipStream_t s);
template <int T>
int launch_partials(const uint8_t *w, int rows, int cols, long row_bytes, const uint8_t *xpack, int ntok,
                    int32_t *part, hipStream_t s);
template <int T>
int launch_dequant(const uint8_t *w, int rows, int cols, long row_bytes, float *out, hipStream_t s);

// Replace the IQ3_S codebook used by the IQ3_S kernels (defined in the IQ3_S translation unit).
int set_iq3s_grid(const uint8_t *grid);

}  // namespace vq

// The per-type kernel templates, instantiated once per type by VQ_INSTANTIATE (vq_qmv_impl.h) in
// vq_t_<type>.hip; other translation units that see the definitions declare them extern with
// VQ_KERNEL_TEMPLATES(extern template, T), so each kernel (and each copy of the device tables it reads, e.g.
// the replaceable IQ3_S grid) exists once.
#define VQ_KERNEL_TEMPLATES(KW, T)                                                                                       \
    KW int vq::launch_quant<T>(const uint8_t *, int, int, long, const void *, bool, int, float *, hipStream_t); \
    KW int vq::launch_quant_jobs<T>(int, const uint8_t *const *, const int *, float *const *, int, const void *, \
                                          bool, int, unsigned long long *, int32_t *, hipStream_t);                 \
    KW long vq::argmax_waves<T>(int, int, int);                                                                \
    KW int vq::launch_quant_staged<T>(const uint8_t *, int, int, long, const float *, const vq::XStage &, int, \
                                            float *, hipStream_t);                                                   \
    KW int vq::launch_mixed_q8<T>(int, const int *, const uint8_t *const *, const int *, float *const *, int, \
                                        const float *, int, hipStream_t);                                          \
    KW int vq::launch_gemm<T>(const uint8_t *, int, int, long, const uint8_t *, int, float *, hipStream_t);    \
    KW int vq::launch_gemm16<T>(const uint8_t *, int, int, long, const void *, int, float *, int, hipStream_t, bool, bool); \
    KW int vq::launch_small16_group<T>(int, const uint8_t *const *, const int *, float *const *, int, long,    \
                                             const float *, int, float *, hipStream_t, const vq::XStage &, float *); \
    KW int vq::launch_small16<T>(const uint8_t *, int, int, long, const float *, int, float *, float *,          \
                                       hipStream_t, const vq::XStage &, float *);                                  \
    KW int vq::launch_mfma<T>(const uint8_t *, int, int, long, const float *, int, float *, float *,         \
                                    hipStream_t);                                                                \
    KW int vq::launch_partials<T>(const uint8_t *, int, int, long, const uint8_t *, int, int32_t *,          \
                                        hipStream_t);                                                            \
    KW int vq::launch_dequant<T>(const uint8_t *, int, int, long, float *, hipStream_t);
