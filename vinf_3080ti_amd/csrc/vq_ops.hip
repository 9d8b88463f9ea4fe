// vq_ops.hip -- the runtime's elementwise, normalisation and layout ops around the matvec (the reference
// runtime's rmsnorm, gated_rmsnorm, add / silu_mul / sigmoid_mul, split_gated_q, NeoX rope, kv_append,
// attention, conv_update and gated-delta kernels, qwen_runtime.cu:36-567): fp32, fp16 KV caches allowed.
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

// Gated query: head h's raw row is [query (hd), gate (hd)]; q and gate get the halves.
__global__ __launch_bounds__(256) void split_gated_q_kernel(const float *__restrict__ raw, float *__restrict__ q,
                                                           float *__restrict__ gate, int heads, int hd) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<long>(heads) * hd) return;
    const long h = i / hd, d = i - h * hd;
    q[i] = raw[2 * h * hd + d];
    gate[i] = raw[2 * h * hd + hd + d];
}

// NeoX RoPE in place over dims [0, rot) of each head of token t (position pos0 + t): pair (j, j + rot/2)
// turns by (pos0 + t) * base^(-2j / rot), the angle and its cosine / sine in fp64, the rotation in fp32.
__global__ __launch_bounds__(128) void rope_neox_kernel(float *x, int ntok, int heads, int hd, int rot, int pos0,
                                                        double base) {
    const int half = rot / 2;
    const long i = static_cast<long>(blockIdx.x) * 128 + threadIdx.x;
    if (i >= static_cast<long>(ntok) * heads * half) return;
    const int j = static_cast<int>(i % half);
    const long th = i / half;  // token * heads + head
    const int t = static_cast<int>(th / heads);
    const double ang = static_cast<double>(pos0 + t) * pow(base, -2.0 * j / rot);
    const float c = static_cast<float>(cos(ang)), sn = static_cast<float>(sin(ang));
    float *head = x + th * hd;
    const float a = head[j], b = head[j + half];
    head[j] = a * c - b * sn;
    head[j + half] = b * c + a * sn;
}

// KV append into contiguous caches [kv_head][max_seq][hd] (fp32, or fp16 rounded to nearest): element d of
// head h of token t goes to position pos0 + t.
__device__ __forceinline__ void kv_put(float *c, size_t i, float v) { c[i] = v; }
__device__ __forceinline__ void kv_put(_Float16 *c, size_t i, float v) { c[i] = static_cast<_Float16>(v); }
template <typename C>
__global__ __launch_bounds__(256) void kv_append_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                        C *__restrict__ kc, C *__restrict__ vc, int ntok,
                                                        int kv_heads, int max_seq, int hd, int pos0) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<long>(ntok) * kv_heads * hd) return;
    const long d = i % hd, th = i / hd;
    const long h = th % kv_heads, t = th / kv_heads;
    const size_t dst = (static_cast<size_t>(h) * max_seq + pos0 + t) * hd + d;
    kv_put(kc, dst, k[i]);
    kv_put(vc, dst, v[i]);
}

// GQA attention of query token t, head h (workgroup (h, t), 4 waves): positions [start, end) with end =
// seq_len0 + t (causal) or seq_len0 + ntok - 1 (bidirectional), start = end_q - window when a window is set
// (end_q = seq_len0 + t). Wave w takes the 64-position chunks w, w + 4, ...: lane = position for q . k, an
// online softmax (running max m, sum l, output acc rescaled by e^(m_old - m_new)), lane = output dims for the
// V sum; the four waves' (m, l, acc) are merged in wave order. Caches [kv_head][max_seq][hd], fp32 or fp16.
constexpr int kAttnWaves = 4, kAttnMaxHd = 256;
__device__ __forceinline__ float kv_get(const float *c, size_t i) { return c[i]; }
__device__ __forceinline__ float kv_get(const _Float16 *c, size_t i) { return static_cast<float>(c[i]); }
template <typename C>
__global__ __launch_bounds__(64 * kAttnWaves) void attention_kernel(const float *__restrict__ q, const C *__restrict__ kc,
                                                                    const C *__restrict__ vc, float *__restrict__ out,
                                                                    int heads, int kv_heads, int hd, int max_seq,
                                                                    int seq_len0, int bidirectional, int window) {
    __shared__ float sq[kAttnMaxHd];
    __shared__ float sp[kAttnWaves][64];
    __shared__ float sm[kAttnWaves], sl[kAttnWaves];
    __shared__ float sacc[kAttnWaves][kAttnMaxHd];
    const int h = blockIdx.x, t = blockIdx.y, ntok = gridDim.y;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int qend = seq_len0 + t;
    const int end = bidirectional ? seq_len0 + ntok - 1 : qend;
    const int start = window > 0 && qend > window ? qend - window : 0;
    const int kvh = h / (heads / kv_heads);
    const float scale = 1.0f / sqrtf(static_cast<float>(hd));
    const float *qh = q + (static_cast<size_t>(t) * heads + h) * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) sq[d] = qh[d];
    __syncthreads();
    const size_t hbase = static_cast<size_t>(kvh) * max_seq;
    float m = -INFINITY, l = 0.0f;
    float acc[kAttnMaxHd / 64];
#pragma unroll
    for (int r = 0; r < kAttnMaxHd / 64; ++r) acc[r] = 0.0f;
    for (int p0 = start + 64 * wv; p0 < end; p0 += 64 * kAttnWaves) {
        const int p = p0 + lane;
        float sc = -INFINITY;
        if (p < end) {
            const size_t row = (hbase + p) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot = fmaf(sq[d], kv_get(kc, row + d), dot);
            sc = dot * scale;
        }
        float cm = sc;
        for (int o = 32; o > 0; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o, 64));
        const float mn = fmaxf(m, cm);
        const float pr = p < end ? expf(sc - mn) : 0.0f;
        float ps = pr;
        for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o, 64);
        const float rs = expf(m - mn);  // 0 on the first chunk (m = -inf)
        l = l * rs + ps;
        m = mn;
        sp[wv][lane] = pr;
        __builtin_amdgcn_wave_barrier();
        const int np = end - p0 < 64 ? end - p0 : 64;
#pragma unroll
        for (int r = 0; r < kAttnMaxHd / 64; ++r) {
            const int d = lane + 64 * r;
            if (d < hd) {
                float a = acc[r] * rs;
                for (int j = 0; j < np; ++j) a = fmaf(sp[wv][j], kv_get(vc, (hbase + p0 + j) * hd + d), a);
                acc[r] = a;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0) {
        sm[wv] = m;
        sl[wv] = l;
    }
#pragma unroll
    for (int r = 0; r < kAttnMaxHd / 64; ++r)
        if (lane + 64 * r < hd) sacc[wv][lane + 64 * r] = acc[r];
    __syncthreads();
    if (wv == 0) {
        float M = -INFINITY;
        for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, sm[w]);
        float L = 0.0f, f[kAttnWaves];
        for (int w = 0; w < kAttnWaves; ++w) {
            f[w] = sm[w] == -INFINITY ? 0.0f : expf(sm[w] - M);
            L += sl[w] * f[w];
        }
        float *o = out + (static_cast<size_t>(t) * heads + h) * hd;
        for (int d = lane; d < hd; d += 64) {
            float a = 0.0f;
            for (int w = 0; w < kAttnWaves; ++w) a += sacc[w][d] * f[w];
            o[d] = a / L;
        }
    }
}

// Causal depthwise conv + SiLU through ntok tokens, one thread per channel: the state row [K] holds the last K
// inputs; per token it shifts left, takes x, and out = silu(state . w). snap (optional) receives the state
// after each token but the last, [ntok - 1][channel][K]; the state keeps the final one.
constexpr int kConvMaxK = 8;
__global__ __launch_bounds__(256) void conv_update_kernel(const float *__restrict__ x, float *__restrict__ state,
                                                          const float *__restrict__ w, float *__restrict__ out,
                                                          int channels, int K, int ntok, float *__restrict__ snap) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= channels) return;
    float st[kConvMaxK], wc[kConvMaxK];
#pragma unroll
    for (int k = 0; k < kConvMaxK; ++k) {
        st[k] = k < K ? state[static_cast<size_t>(c) * K + k] : 0.0f;
        wc[k] = k < K ? w[static_cast<size_t>(c) * K + k] : 0.0f;
    }
    for (int t = 0; t < ntok; ++t) {
#pragma unroll
        for (int k = 0; k < kConvMaxK - 1; ++k)
            if (k < K - 1) st[k] = st[k + 1];
        const float xi = x[static_cast<size_t>(t) * channels + c];
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < kConvMaxK; ++k) {
            if (k == K - 1) st[k] = xi;
            if (k < K) acc = fmaf(st[k], wc[k], acc);
        }
        out[static_cast<size_t>(t) * channels + c] = silu_ieee(acc);
        if (snap != nullptr && t < ntok - 1)
            for (int k = 0; k < K; ++k) snap[(static_cast<size_t>(t) * channels + c) * K + k] = st[k];
    }
    for (int k = 0; k < K; ++k) state[static_cast<size_t>(c) * K + k] = st[k];
}

// Gated delta rule through ntok tokens, one workgroup per value head h (state S [kd][vd] of that head): conv
// rows are [q (key_heads kd) | k (key_heads kd) | v (value_heads vd)]; key head kh = h / (vh / kh) (head_order
// 0) or h % kh (1). Per token: q^ = q / (sqrt(|q|^2 + eps) sqrt(kd)), k^ = k / sqrt(|k|^2 + eps) (sums in a fixed
// tree), beta = sigmoid(b), decay = exp(ssm_a softplus(a + dt)); S *= decay; delta = (v - S^T k^) beta;
// S += k^ delta^T; out = S^T q^. Thread j owns state columns j, j + 256, ...; snap: states after each token
// but the last, [ntok - 1][vh][kd][vd].
constexpr int kGdMaxKd = 256;
__global__ __launch_bounds__(256) void gated_delta_kernel(const float *__restrict__ conv, const float *__restrict__ braw,
                                                          const float *__restrict__ araw, const float *__restrict__ ssm_a,
                                                          const float *__restrict__ dt, float *__restrict__ S,
                                                          float *__restrict__ out, int key_heads, int value_heads,
                                                          int kd, int vd, float eps, int head_order, int ntok,
                                                          float *__restrict__ snap) {
    __shared__ float sq[kGdMaxKd], sk[kGdMaxKd], red[2][256];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int kh = head_order == 0 ? h / (value_heads / key_heads) : h % key_heads;
    const size_t cdim = static_cast<size_t>(2) * key_heads * kd + static_cast<size_t>(value_heads) * vd;
    float *const Sh = S + static_cast<size_t>(h) * kd * vd;
    for (int t = 0; t < ntok; ++t) {
        const float *row = conv + static_cast<size_t>(t) * cdim;
        const float *qs = row + static_cast<size_t>(kh) * kd, *ks = row + static_cast<size_t>(key_heads + kh) * kd;
        const float *vs = row + static_cast<size_t>(2) * key_heads * kd + static_cast<size_t>(h) * vd;
        float aq = 0.0f, ak = 0.0f;
        for (int i = tid; i < kd; i += 256) {
            aq = fmaf(qs[i], qs[i], aq);
            ak = fmaf(ks[i], ks[i], ak);
        }
        red[0][tid] = aq;
        red[1][tid] = ak;
        for (int w = 128; w > 0; w >>= 1) {
            __syncthreads();
            if (tid < w) {
                red[0][tid] += red[0][tid + w];
                red[1][tid] += red[1][tid + w];
            }
        }
        __syncthreads();
        const float qscale = 1.0f / (sqrtf(red[0][0] + eps) * sqrtf(static_cast<float>(kd)));
        const float kscale = 1.0f / sqrtf(red[1][0] + eps);
        for (int i = tid; i < kd; i += 256) {
            sq[i] = qs[i] * qscale;
            sk[i] = ks[i] * kscale;
        }
        __syncthreads();
        const float beta = sigmoid_ieee(braw[static_cast<size_t>(t) * value_heads + h]);
        const float xa = araw[static_cast<size_t>(t) * value_heads + h] + dt[h];
        const float sp = xa > 20.0f ? xa : log1pf(expf(xa));
        const float decay = expf(ssm_a[h] * sp);
        float *const sn = snap != nullptr && t < ntok - 1 ? snap + (static_cast<size_t>(t) * value_heads + h) * kd * vd
                                                          : nullptr;
        for (int j = tid; j < vd; j += 256) {
            float mem = 0.0f;
            for (int i = 0; i < kd; ++i) {
                const float v = Sh[static_cast<size_t>(i) * vd + j] * decay;
                Sh[static_cast<size_t>(i) * vd + j] = v;
                mem = fmaf(v, sk[i], mem);
            }
            const float delta = (vs[j] - mem) * beta;
            float o = 0.0f;
            for (int i = 0; i < kd; ++i) {
                const float v = fmaf(sk[i], delta, Sh[static_cast<size_t>(i) * vd + j]);
                Sh[static_cast<size_t>(i) * vd + j] = v;
                o = fmaf(v, sq[i], o);
                if (sn != nullptr) sn[static_cast<size_t>(i) * vd + j] = v;
            }
            out[(static_cast<size_t>(t) * value_heads + h) * vd + j] = o;
        }
        __syncthreads();  // sq / sk / red are rewritten for the next token
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

int vq_split_gated_q(const float *raw, float *q, float *gate, int heads, int hd, void *stream) {
    if (!raw || !q || !gate) return VQ_ERR_ARG;
    if (heads < 1 || hd < 1) return VQ_ERR_SHAPE;
    const long n = static_cast<long>(heads) * hd;
    split_gated_q_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        raw, q, gate, heads, hd);
    return status_of(hipGetLastError());
}

int vq_rope(float *x, int ntok, int heads, int hd, int rot, int pos0, double base, void *stream) {
    if (!x) return VQ_ERR_ARG;
    if (ntok < 1 || heads < 1 || hd < 1 || rot <= 0 || rot % 2 || rot > hd || pos0 < 0 || !(base > 0.0))
        return VQ_ERR_SHAPE;
    const long n = static_cast<long>(ntok) * heads * (rot / 2);
    rope_neox_kernel<<<static_cast<unsigned>((n + 127) / 128), 128, 0, static_cast<hipStream_t>(stream)>>>(
        x, ntok, heads, hd, rot, pos0, base);
    return status_of(hipGetLastError());
}

int vq_kv_append(const float *k, const float *v, void *kc, void *vc, int elem, int ntok, int kv_heads, int max_seq,
                 int hd, int pos0, void *stream) {
    if (!k || !v || !kc || !vc || (elem != 2 && elem != 4)) return VQ_ERR_ARG;
    if (ntok < 1 || kv_heads < 1 || hd < 1 || pos0 < 0 || pos0 + ntok > max_seq) return VQ_ERR_SHAPE;
    const long n = static_cast<long>(ntok) * kv_heads * hd;
    const unsigned blocks = static_cast<unsigned>((n + 255) / 256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (elem == 2)
        kv_append_kernel<_Float16><<<blocks, 256, 0, s>>>(k, v, static_cast<_Float16 *>(kc), static_cast<_Float16 *>(vc),
                                                          ntok, kv_heads, max_seq, hd, pos0);
    else
        kv_append_kernel<float><<<blocks, 256, 0, s>>>(k, v, static_cast<float *>(kc), static_cast<float *>(vc), ntok,
                                                       kv_heads, max_seq, hd, pos0);
    return status_of(hipGetLastError());
}

int vq_attention(const float *q, const void *kc, const void *vc, float *out, int elem, int heads, int kv_heads, int hd,
                 int max_seq, int seq_len, int ntok, int bidirectional, int window, void *stream) {
    if (!q || !kc || !vc || !out || (elem != 2 && elem != 4)) return VQ_ERR_ARG;
    if (kv_heads < 1 || heads < kv_heads || heads % kv_heads || hd < 1 || hd > kAttnMaxHd || ntok < 1 ||
        seq_len < 1 || seq_len + ntok - 1 > max_seq || window < 0)
        return VQ_ERR_SHAPE;
    const dim3 grid(heads, ntok);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (elem == 2)
        attention_kernel<_Float16><<<grid, 64 * kAttnWaves, 0, s>>>(q, static_cast<const _Float16 *>(kc),
                                                                    static_cast<const _Float16 *>(vc), out, heads,
                                                                    kv_heads, hd, max_seq, seq_len, bidirectional, window);
    else
        attention_kernel<float><<<grid, 64 * kAttnWaves, 0, s>>>(q, static_cast<const float *>(kc),
                                                                 static_cast<const float *>(vc), out, heads, kv_heads,
                                                                 hd, max_seq, seq_len, bidirectional, window);
    return status_of(hipGetLastError());
}

int vq_conv_update(const float *x, float *state, const float *w, float *out, int channels, int K, int ntok, float *snap,
                   void *stream) {
    if (!x || !state || !w || !out) return VQ_ERR_ARG;
    if (channels < 1 || K < 1 || K > kConvMaxK || ntok < 1) return VQ_ERR_SHAPE;
    conv_update_kernel<<<static_cast<unsigned>((channels + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        x, state, w, out, channels, K, ntok, snap);
    return status_of(hipGetLastError());
}

int vq_gated_delta(const float *conv, const float *b, const float *a, const float *ssm_a, const float *dt, float *state,
                   float *out, int key_heads, int value_heads, int kd, int vd, float eps, int head_order, int ntok,
                   float *snap, void *stream) {
    if (!conv || !b || !a || !ssm_a || !dt || !state || !out) return VQ_ERR_ARG;
    if (key_heads < 1 || value_heads < key_heads || value_heads % key_heads || kd < 1 || kd > kGdMaxKd || vd < 1 ||
        ntok < 1 || (head_order != 0 && head_order != 1) || !(eps >= 0.0f))
        return VQ_ERR_SHAPE;
    gated_delta_kernel<<<value_heads, 256, 0, static_cast<hipStream_t>(stream)>>>(
        conv, b, a, ssm_a, dt, state, out, key_heads, value_heads, kd, vd, eps, head_order, ntok, snap);
    return status_of(hipGetLastError());
}

}  // extern "C"
