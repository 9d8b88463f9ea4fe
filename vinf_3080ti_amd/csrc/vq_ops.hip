// vq_ops.hip -- the runtime's sequence ops around the matvec: norms and elementwise passes, the gated query
// split, NeoX rope, KV append and GQA attention over contiguous or paged caches, the causal conv update and
// the gated delta rule (the reference runtime's per-op kernels, qwen_runtime.cu:36-567, and its
// multi-sequence forms, qwen_runtime.cu:2333-2600).
//
// One launch per pass. The multi-sequence forms take the pass's segment table by value (each segment is a
// sequence slot, the position of its first row, its row count and the buffer row it starts at): a block finds
// its segment from blockIdx, so a pass of many sequences is still one launch. The single-sequence entry points
// are a one-segment table with contiguous caches.
//
// RMS sums: each thread adds its strided elements in order, then a fixed pairwise tree over the 256 threads in
// LDS, so a group's result does not depend on timing. silu / sigmoid use expf and an IEEE division (these
// passes are bound by bytes, not by VALU).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#include "../../include/vq.h"
#include "vq_lds.h"

namespace {

int status_of(hipError_t e) { return e == hipSuccess ? VQ_OK : static_cast<int>(e); }

// ---- segments and cache addressing ---------------------------------------------------------------------

// A pass's segment table, passed by value in the kernel arguments (1 KB at the maximum).
struct Seg {
    int slot, pos0, rows, row0;
};
struct SegTable {
    int n;
    int total;  // sum of rows (the blocks of a per-row grid)
    Seg s[VQ_MAX_SEGMENTS];
};

// Cross-row lane exchanges of gfx950 without LDS: v_permlane16_swap (rows 0<->1, 2<->3) and v_permlane32_swap (lane
// halves). Called with the same value twice, the pair holds each lane's value and its partner's (lane ^ 16 or
// lane ^ 32) in an order that depends on the lane, so max and (commutative) sums come out bit-identical on both
// partners, as with __shfl_xor.
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_add(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_add(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Global row index g (segments in table order) -> (segment, row within it).
__device__ __forceinline__ const Seg &seg_of_row(const SegTable &T, int g, int &local) {
    int i = 0;
    while (i + 1 < T.n && g >= T.s[i].rows) {
        g -= T.s[i].rows;
        ++i;
    }
    local = g;
    return T.s[i];
}

// KV cache rows: contiguous [kv_head][max_seq][hd] when pt is null, else a page pool
// [page][kv_head][page_size][hd] with the sequence slot's page ids at pt[slot * pps + pos / page_size].
struct KvMap {
    const int32_t *pt;
    int max_seq;  // contiguous caches
    int page, pps, kv_heads;
    __device__ __forceinline__ size_t row(int slot, int kvh, int pos) const {
        if (pt == nullptr) return static_cast<size_t>(kvh) * max_seq + pos;
        const int pg = pt[slot * pps + pos / page];
        return (static_cast<size_t>(pg) * kv_heads + kvh) * page + pos % page;
    }
    // The same with the layout fixed at compile time: no branch around the page-table load, so the compiler can
    // keep the loads that follow in flight (a load under a branch makes it wait for every outstanding load).
    template <bool PAGED>
    __device__ __forceinline__ size_t row_t(int slot, int kvh, int pos) const {
        if constexpr (!PAGED) return static_cast<size_t>(kvh) * max_seq + pos;
        const int pg = pt[slot * pps + pos / page];
        return (static_cast<size_t>(pg) * kv_heads + kvh) * page + pos % page;
    }
};

__device__ __forceinline__ float kv_get(const float *c, size_t i) { return c[i]; }
__device__ __forceinline__ float kv_get(const _Float16 *c, size_t i) { return static_cast<float>(c[i]); }
// Elements i .. i + 3 of a cache as one vector load (the caller checks the alignment), widened to fp32.
__device__ __forceinline__ float4 ld4(const float *c, size_t i) { return *reinterpret_cast<const float4 *>(c + i); }
__device__ __forceinline__ float4 ld4(const _Float16 *c, size_t i) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 a = *reinterpret_cast<const h4 *>(c + i);
    return float4{static_cast<float>(a[0]), static_cast<float>(a[1]), static_cast<float>(a[2]), static_cast<float>(a[3])};
}

// Host side: validate a segment table ([n][4] int32: slot, pos0, rows, row0) into a SegTable.
int make_table(const int32_t *segs, int nseg, SegTable &T, int *rows_spanned) {
    if (segs == nullptr || nseg < 1 || nseg > VQ_MAX_SEGMENTS) return VQ_ERR_ARG;
    T.n = nseg;
    T.total = 0;
    int span = 0;
    for (int i = 0; i < nseg; ++i) {
        const Seg s{segs[4 * i], segs[4 * i + 1], segs[4 * i + 2], segs[4 * i + 3]};
        if (s.slot < 0 || s.pos0 < 0 || s.rows < 1 || s.row0 < 0) return VQ_ERR_SHAPE;
        T.s[i] = s;
        T.total += s.rows;
        span = s.row0 + s.rows > span ? s.row0 + s.rows : span;
    }
    if (rows_spanned) *rows_spanned = span;
    return VQ_OK;
}

SegTable one_segment(int pos0, int rows) {
    SegTable T{};
    T.n = 1;
    T.total = rows;
    T.s[0] = Seg{0, pos0, rows, 0};
    return T;
}

// ---- norms and elementwise -------------------------------------------------------------------------------

constexpr int kNormThreads = 256;

__device__ __forceinline__ float silu_ieee(float z) { return z / (1.0f + expf(-z)); }
__device__ __forceinline__ float sigmoid_ieee(float z) { return 1.0f / (1.0f + expf(-z)); }

// Group g: y = x * rsqrt(mean(x^2) + eps) * w (* silu(z) when z is given). y may be x: every element is read
// before it is written, by the same thread (so x, z and y are not restrict).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float *x, const float *__restrict__ w,
                                                               const float *z, float *y, int n, float eps) {
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

// ---- layout ops ------------------------------------------------------------------------------------------

// Gated query split as a 16-byte copy: quad e of the output (heads * hd / 4 of them) comes from quad
// e + (e / hq) * hq of raw (query half) and hq quads further on (gate half), hq = hd / 4. Needs hd % 4 == 0
// and 16-byte aligned buffers (checked on the host; else the element kernel below).
__global__ __launch_bounds__(256) void split_gated_q4_kernel(const float4 *__restrict__ raw, float4 *__restrict__ q,
                                                             float4 *__restrict__ gate, int hq, long nq) {
    const long e = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (e >= nq) return;
    const long src = e + (e / hq) * hq;
    q[e] = raw[src];
    gate[e] = raw[src + hq];
}
__global__ __launch_bounds__(256) void split_gated_q1_kernel(const float *__restrict__ raw, float *__restrict__ q,
                                                             float *__restrict__ gate, int hd, long n) {
    const long e = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (e >= n) return;
    const long src = e + (e / hd) * hd;
    q[e] = raw[src];
    gate[e] = raw[src + hd];
}

// dst[r] = [a[r] | b[r]], rows of `width` floats.
__global__ __launch_bounds__(256) void concat_rows_kernel(float *__restrict__ dst, const float *__restrict__ a,
                                                          const float *__restrict__ b, int width, long n) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const long r = i / (2 * width), c = i - r * 2 * width;
    dst[i] = c < width ? a[r * width + c] : b[r * width + c - width];
}

// Fill with zeros (a kernel, not hipMemsetAsync, so the op can sit in a captured graph).
__global__ __launch_bounds__(256) void zero_kernel(uint32_t *__restrict__ p, long nwords) {
    for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < nwords; i += static_cast<long>(gridDim.x) * 256)
        p[i] = 0u;
}
__global__ void zero_bytes_kernel(uint8_t *__restrict__ p, int n) {
    if (static_cast<int>(threadIdx.x) < n) p[threadIdx.x] = 0;
}

// ---- rope ------------------------------------------------------------------------------------------------

// NeoX RoPE in place, one workgroup per row (token): the row's rot/2 rotations (angle (pos) * base^(-2j/rot)
// and its cosine / sine in fp64, rounded to fp32) are computed once into LDS and applied to every head, pair
// (x[j], x[j + rot/2]) of each head's first rot dims.
constexpr int kRopeThreads = 128, kRopeMaxHalf = 512;
__global__ __launch_bounds__(kRopeThreads) void rope_kernel(float *x, SegTable T, int heads, int hd, int rot,
                                                            double base) {
    __shared__ float2 cs[kRopeMaxHalf];
    int t;
    const Seg &s = seg_of_row(T, blockIdx.x, t);
    const int half = rot / 2, pos = s.pos0 + t;
    for (int j = threadIdx.x; j < half; j += kRopeThreads) {
        const double ang = static_cast<double>(pos) * pow(base, -2.0 * j / rot);
        cs[j] = float2{static_cast<float>(cos(ang)), static_cast<float>(sin(ang))};
    }
    __syncthreads();
    float *row = x + static_cast<size_t>(s.row0 + t) * heads * hd;
    for (int e = threadIdx.x; e < heads * half; e += kRopeThreads) {
        const int h = e / half, j = e - h * half;
        float *p = row + static_cast<size_t>(h) * hd;
        const float2 c = cs[j];
        const float a = p[j], b = p[j + half];
        p[j] = a * c.x - b * c.y;
        p[j + half] = b * c.x + a * c.y;
    }
}

// ---- KV append -------------------------------------------------------------------------------------------

__device__ __forceinline__ void put4(float *c, size_t i, float4 v) { *reinterpret_cast<float4 *>(c + i) = v; }
__device__ __forceinline__ void put4(_Float16 *c, size_t i, float4 v) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<h4 *>(c + i) = h4{static_cast<_Float16>(v.x), static_cast<_Float16>(v.y),
                                        static_cast<_Float16>(v.z), static_cast<_Float16>(v.w)};
}
__device__ __forceinline__ void put1(float *c, size_t i, float v) { c[i] = v; }
__device__ __forceinline__ void put1(_Float16 *c, size_t i, float v) { c[i] = static_cast<_Float16>(v); }

// One workgroup per row: the row's k, v [kv_heads][hd] go to position pos0 + t of the segment's sequence. Quads
// (VEC = 4, hd % 4 == 0 and aligned buffers) or single values; fp16 caches are written rounded to nearest.
template <typename C, int VEC>
__global__ __launch_bounds__(256) void kv_append_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                        C *__restrict__ kc, C *__restrict__ vc, SegTable T, KvMap M,
                                                        int hd) {
    int t;
    const Seg &s = seg_of_row(T, blockIdx.x, t);
    const int pos = s.pos0 + t, n = M.kv_heads * hd;
    const size_t src = static_cast<size_t>(s.row0 + t) * n;
    for (int e = threadIdx.x * VEC; e < n; e += 256 * VEC) {
        const int kvh = e / hd, d = e - kvh * hd;
        const size_t dst = M.row(s.slot, kvh, pos) * hd + d;
        if constexpr (VEC == 4) {
            put4(kc, dst, *reinterpret_cast<const float4 *>(k + src + e));
            put4(vc, dst, *reinterpret_cast<const float4 *>(v + src + e));
        } else {
            put1(kc, dst, k[src + e]);
            put1(vc, dst, v[src + e]);
        }
    }
}

// ---- attention (decode and verify rows) -------------------------------------------------------------------

// GQA attention of query row t of a segment, head h (workgroup (h, global row), 4 waves). The row sees positions
// [start, end) with end = seq_len0 + t (causal) or seq_len0 + rows - 1 (bidirectional), seq_len0 = pos0 + 1,
// and start = end_q - window when a window is set (end_q = seq_len0 + t). Wave w takes the 64-position chunks
// w, w + 4, ...: lane = position for q . k, an online softmax (running max m, sum l, output acc rescaled by
// e^(m_old - m_new)), lane = output dims for the V sum; the four waves' (m, l, acc) are merged in wave order.
constexpr int kAttnWaves = 4, kAttnMaxHd = 256;
template <typename C>
__global__ __launch_bounds__(64 * kAttnWaves) void attention_kernel(const float *__restrict__ q, const C *__restrict__ kc,
                                                                    const C *__restrict__ vc, float *__restrict__ out,
                                                                    SegTable T, KvMap M, int heads, int hd,
                                                                    int bidirectional, int window) {
    __shared__ float sq[kAttnMaxHd];
    __shared__ float sp[kAttnWaves][64];
    __shared__ float sm[kAttnWaves], sl[kAttnWaves];
    __shared__ float sacc[kAttnWaves][kAttnMaxHd];
    int t;
    const Seg &s = seg_of_row(T, blockIdx.y, t);
    const int h = blockIdx.x;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int seq_len0 = s.pos0 + 1;
    const int qend = seq_len0 + t;
    const int end = bidirectional ? seq_len0 + s.rows - 1 : qend;
    const int start = window > 0 && qend > window ? qend - window : 0;
    const int kvh = h / (heads / M.kv_heads);
    const float scale = 1.0f / sqrtf(static_cast<float>(hd));
    const size_t qrow = (static_cast<size_t>(s.row0 + t) * heads + h) * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) sq[d] = q[qrow + d];
    __syncthreads();
    float m = -INFINITY, l = 0.0f;
    float acc[kAttnMaxHd / 64];
#pragma unroll
    for (int r = 0; r < kAttnMaxHd / 64; ++r) acc[r] = 0.0f;
    for (int p0 = start + 64 * wv; p0 < end; p0 += 64 * kAttnWaves) {
        const int p = p0 + lane;
        float sc = -INFINITY;
        if (p < end) {
            const size_t row = M.row(s.slot, kvh, p) * hd;
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
                for (int j = 0; j < np; ++j) a = fmaf(sp[wv][j], kv_get(vc, M.row(s.slot, kvh, p0 + j) * hd + d), a);
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
        float Mx = -INFINITY;
        for (int w = 0; w < kAttnWaves; ++w) Mx = fmaxf(Mx, sm[w]);
        float L = 0.0f, f[kAttnWaves];
        for (int w = 0; w < kAttnWaves; ++w) {
            f[w] = sm[w] == -INFINITY ? 0.0f : expf(sm[w] - Mx);
            L += sl[w] * f[w];
        }
        float *o = out + qrow;
        for (int d = lane; d < hd; d += 64) {
            float a = 0.0f;
            for (int w = 0; w < kAttnWaves; ++w) a += sacc[w][d] * f[w];
            o[d] = a / L;
        }
    }
}

// ---- attention over many query rows (prompt passes): flash-style on fp32 MFMA ----------------------------------

// A workgroup takes 16 query rows (tokens) of one segment and up to four query heads of one kv head (one wave
// each), so the K/V tiles it stages in LDS serve all of them. Per 16 keys a wave computes S^T = K Q^T (16 keys x
// 16 query rows) with v_mfma_f32_16x16x4f32 over the head dims (Q, pre-scaled by 1/sqrt(hd), stays in registers
// as the B operand for the whole pass), keeps an online softmax per query row (running max m, sum l; the output
// rescaled by e^(m_old - m_new)), and adds O^T += V^T P^T. The accumulator of S^T already holds P^T in the
// layout the second product's B operand needs: its step r takes key 4 g + r in the k slot of lane group g (the
// contraction runs over the keys in that order), so no transpose goes through LDS. fp32 operands and
// accumulation throughout. Visibility rules of attention_kernel.
constexpr int kFaKeys = 32;  // keys per LDS tile
typedef float fa4 __attribute__((ext_vector_type(4)));

// The keys [k_lo, k_hi) of kv head kvh of a sequence, 32 per LDS tile (all four waves stage each tile; fp16 caches
// widened to fp32), against the 16 query vectors a wave holds in qf (query vector col = lane & 15 sees keys
// [qs, qe)). Updates the online softmax (m, l) and the unnormalised output o of the lane's query vector.
// Tile layouts in LDS: K row-major k[key][HD + 4], V transposed vt[dim][kFaKeys + 4]. Both products then read
// their A operand as four consecutive floats per lane (one ds_read_b128 per four MFMAs): the head-dim
// contraction of S^T runs step 4u + v over dims 16 u + 4 g + v in lane group g (the query vector in qf is held
// in the same order), the key contraction of O^T over keys 4 g + r.
constexpr int kFaLdk = kFaKeys + 4;
template <int HD>
struct FaTiles {
    float k[kFaKeys * (HD + 4)];
    float vt[HD * kFaLdk];
    size_t rows[2][kFaKeys];  // cache row of each key of the current / next tile (page-table lookups done once)
};

template <typename C, int HD, bool FAST>
__device__ __forceinline__ void fa_keys(const C *__restrict__ kc, const C *__restrict__ vc, const KvMap &M, int slot,
                                        int kvh, int hd, int k_lo, int k_hi, int qs, int qe, bool wave_on,
                                        const float (&qf)[HD / 4], FaTiles<HD> &tl, float &m, float &l,
                                        fa4 (&o)[HD / 16]) {
    constexpr int LD = HD + 4;
    constexpr int NQ = kFaKeys * (HD / 4) / 256;  // quads of K (and of V) per thread per tile
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    // Cache rows of the keys of a tile (clamped into [.., k_hi)): the first tile's here, each next tile's while
    // the current one is staged, so a paged cache costs one page-table load per key and no serial round trips.
    auto key_row = [&](int p) { return M.row(slot, kvh, p < k_hi ? p : k_hi - 1); };
    if (threadIdx.x < kFaKeys && k_lo < k_hi) tl.rows[0][threadIdx.x] = key_row(k_lo + threadIdx.x);
    for (int k0 = k_lo, cur = 0; k0 < k_hi; k0 += kFaKeys, cur ^= 1) {
        __syncthreads();  // the previous tile is consumed; this tile's rows are visible
        const size_t *rw = tl.rows[cur];
        // K quad i: key i / (HD/4), dims 4 (i % (HD/4)) .. (row-major writes); V quad i: key i % kFaKeys, dims
        // 4 (i / kFaKeys) .. (consecutive lanes write consecutive keys of the transposed tile).
        if constexpr (FAST) {
            // hd % 4 == 0 and aligned caches: every thread's loads of the tile are issued before any is stored
            // (addresses clamped into the tile, values past its edge zeroed afterwards).
            // Two rounds of NQ / 2 quads each keep the staging registers small beside qf and o.
            constexpr int NH = NQ > 1 ? NQ / 2 : 1;
#pragma unroll
            for (int u0 = 0; u0 < NQ; u0 += NH) {
                float4 kq[NH], vq[NH];
#pragma unroll
                for (int u = 0; u < NH; ++u) {
                    const int i = threadIdx.x + 256 * (u0 + u);
                    const int kk = i / (HD / 4), kd = 4 * (i - kk * (HD / 4));
                    const int vk = i % kFaKeys, vd = 4 * (i / kFaKeys);
                    kq[u] = ld4(kc, rw[kk] * hd + (kd < hd ? kd : 0));
                    vq[u] = ld4(vc, rw[vk] * hd + (vd < hd ? vd : 0));
                }
#pragma unroll
                for (int u = 0; u < NH; ++u) {
                    const int i = threadIdx.x + 256 * (u0 + u);
                    const int kk = i / (HD / 4), kd = 4 * (i - kk * (HD / 4));
                    const int vk = i % kFaKeys, vd = 4 * (i / kFaKeys);
                    const float mk = k0 + kk < k_hi && kd < hd ? 1.0f : 0.0f;  // zero past the tile's edge
                    const float mv = k0 + vk < k_hi && vd < hd ? 1.0f : 0.0f;
                    *reinterpret_cast<float4 *>(tl.k + kk * LD + kd) =
                        float4{kq[u].x * mk, kq[u].y * mk, kq[u].z * mk, kq[u].w * mk};
                    tl.vt[(vd + 0) * kFaLdk + vk] = vq[u].x * mv;
                    tl.vt[(vd + 1) * kFaLdk + vk] = vq[u].y * mv;
                    tl.vt[(vd + 2) * kFaLdk + vk] = vq[u].z * mv;
                    tl.vt[(vd + 3) * kFaLdk + vk] = vq[u].w * mv;
                }
            }
        } else {
            for (int i = threadIdx.x; i < kFaKeys * HD; i += blockDim.x) {
                const int kk = i / HD, kd = i - kk * HD;      // K element
                const int vk = i % kFaKeys, vd = i / kFaKeys;  // V element
                const bool okk = k0 + kk < k_hi && kd < hd, okv = k0 + vk < k_hi && vd < hd;
                tl.k[kk * LD + kd] = okk ? kv_get(kc, rw[kk] * hd + kd) : 0.0f;
                tl.vt[vd * kFaLdk + vk] = okv ? kv_get(vc, rw[vk] * hd + vd) : 0.0f;
            }
        }
        if (threadIdx.x < kFaKeys && k0 + kFaKeys < k_hi) tl.rows[cur ^ 1][threadIdx.x] = key_row(k0 + kFaKeys + threadIdx.x);
        __syncthreads();
        if (!wave_on) continue;
#pragma unroll
        for (int sub = 0; sub < kFaKeys / 16; ++sub) {
            const int kb = k0 + 16 * sub;
            if (kb >= k_hi) break;
            // S^T: four independent accumulator chains (one per v of dims 16 u + 4 g + v), added at the end.
            fa4 sc4[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            const float *krow = tl.k + (16 * sub + col) * LD + 4 * grp;
#pragma unroll
            for (int u = 0; u < HD / 16; ++u) {
                const float4 a = *reinterpret_cast<const float4 *>(krow + 16 * u);
                sc4[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, qf[4 * u], sc4[0], 0, 0, 0);
                sc4[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, qf[4 * u + 1], sc4[1], 0, 0, 0);
                sc4[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, qf[4 * u + 2], sc4[2], 0, 0, 0);
                sc4[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, qf[4 * u + 3], sc4[3], 0, 0, 0);
            }
            const fa4 sc = (sc4[0] + sc4[1]) + (sc4[2] + sc4[3]);
            // sc[r]: key kb + 4 grp + r against query vector col
            float v[4], bm = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int p = kb + 4 * grp + r;
                v[r] = p >= qs && p < qe && p < k_hi ? sc[r] : -INFINITY;
                bm = fmaxf(bm, v[r]);
            }
            bm = xor16_max(bm);
            bm = xor32_max(bm);
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.0f : expf(m - mn);  // 0 on the first visible block
            float pr[4], ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[r] = v[r] == -INFINITY ? 0.0f : expf(v[r] - mn);
                ps += pr[r];
            }
            ps = xor16_add(ps);
            ps = xor32_add(ps);
            l = l * alpha + ps;
            m = mn;
            const float *vrow = tl.vt + col * kFaLdk + 16 * sub + 4 * grp;
#pragma unroll
            for (int b = 0; b < HD / 16; ++b) {
                const float4 a = *reinterpret_cast<const float4 *>(vrow + 16 * b * kFaLdk);
                fa4 ob = o[b] * alpha;
                ob = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, pr[0], ob, 0, 0, 0);
                ob = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, pr[1], ob, 0, 0, 0);
                ob = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, pr[2], ob, 0, 0, 0);
                o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, pr[3], ob, 0, 0, 0);
            }
        }
    }
}

// Query vector held in the B-operand order of fa_keys: lane group g keeps dims 16 u + 4 g + v at step 4 u + v,
// times scale.
template <int HD>
__device__ __forceinline__ void fa_load_q(const float *qrow, int hd, float scale, float (&qf)[HD / 4]) {
    const int grp = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int st = 0; st < HD / 4; ++st) {
        const int d = 16 * (st >> 2) + 4 * grp + (st & 3);
        // Clamped address and a multiplied mask rather than a branch: all HD/4 loads are issued before the
        // first wait (guarded loads are each issued and waited for on their own).
        qf[st] = qrow[d < hd ? d : hd - 1] * (d < hd ? scale : 0.0f);
    }
}

// Prompt passes: a workgroup takes 16 query rows (tokens) of one segment and up to four query heads of one kv head
// (one wave each), so the K/V tiles it stages in LDS serve all of them, and walks every key the rows see.
template <typename C, int HD, bool FAST>
__global__ __launch_bounds__(256) void attention_mfma_kernel(const float *__restrict__ q, const C *__restrict__ kc,
                                                             const C *__restrict__ vc, float *__restrict__ out,
                                                             SegTable T, KvMap M, int heads, int hd, int bidirectional,
                                                             int window, int chunks) {
    __shared__ FaTiles<HD> tl;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    int tb = blockIdx.x, si = 0;  // (segment, 16-row tile) of this workgroup
    while (si + 1 < T.n && tb >= (T.s[si].rows + 15) / 16) {
        tb -= (T.s[si].rows + 15) / 16;
        ++si;
    }
    const Seg &s = T.s[si];
    const int G = heads / M.kv_heads;
    const int kvh = blockIdx.y / chunks, gi = (blockIdx.y - kvh * chunks) * 4 + wv;
    const bool wave_on = gi < G;
    const int h = kvh * G + (wave_on ? gi : 0);
    const int t0 = 16 * tb, nq = min(16, s.rows - t0);
    const int seq_len0 = s.pos0 + 1;
    auto q_end = [&](int t) { return bidirectional ? seq_len0 + s.rows - 1 : seq_len0 + t; };
    auto q_start = [&](int t) { return window > 0 && seq_len0 + t > window ? seq_len0 + t - window : 0; };
    const int tq = t0 + min(col, nq - 1);  // this lane's query row (rows past nq repeat the last; not written)
    float qf[HD / 4];
    fa_load_q<HD>(q + (static_cast<size_t>(s.row0 + tq) * heads + h) * hd, hd, 1.0f / sqrtf(static_cast<float>(hd)),
                  qf);
    float m = -INFINITY, l = 0.0f;
    fa4 o[HD / 16];
#pragma unroll
    for (int b = 0; b < HD / 16; ++b) o[b] = fa4{0.f, 0.f, 0.f, 0.f};
    fa_keys<C, HD, FAST>(kc, vc, M, s.slot, kvh, hd, q_start(t0), q_end(t0 + nq - 1), q_start(tq), q_end(tq), wave_on, qf,
                   tl, m, l, o);
    // o[b][r]: head dim 16 b + 4 grp + r of query row tq
    if (wave_on && col < nq) {
        float *orow = out + (static_cast<size_t>(s.row0 + t0 + col) * heads + h) * hd;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int b = 0; b < HD / 16; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 16 * b + 4 * grp + r;
                if (d < hd) orow[d] = o[b][r] * inv;
            }
    }
}

// Decode and verify passes (at most VQ_ATTN_ROW_MAX rows per segment): the keys of a sequence are cut into nch
// chunks, one workgroup per (segment, kv head, chunk, block of 64 query vectors). Query vector j of the block is
// (row j / G, head j % G of the kv head's group): every query head of the group shares the staged K/V. Each
// writes its unnormalised partial output and its (max, sum) to the workspace; attention_merge_kernel combines
// the chunks in chunk order (deterministic).
template <typename C, int HD, bool FAST>
__global__ __launch_bounds__(256) void attention_split_kernel(const float *__restrict__ q, const C *__restrict__ kc,
                                                              const C *__restrict__ vc, float *__restrict__ part,
                                                              float *__restrict__ pml, SegTable T, KvMap M, int heads,
                                                              int hd, int bidirectional, int window, int nch) {
    __shared__ FaTiles<HD> tl;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int c = blockIdx.x % nch, sk_id = blockIdx.x / nch;
    const int kvh = sk_id % M.kv_heads, si = sk_id / M.kv_heads;
    const Seg &s = T.s[si];
    const int G = heads / M.kv_heads;
    const int j = blockIdx.y * 64 + wv * 16 + col;  // query vector of this lane
    const int t = j / G, g = j - t * G;
    const bool valid = t < s.rows;
    const bool wave_on = blockIdx.y * 64 + wv * 16 < s.rows * G;
    const int tq = valid ? t : s.rows - 1, h = kvh * G + (valid ? g : 0);
    const int seq_len0 = s.pos0 + 1;
    const int qe = bidirectional ? seq_len0 + s.rows - 1 : seq_len0 + tq;
    const int qs = window > 0 && seq_len0 + tq > window ? seq_len0 + tq - window : 0;
    const int ctx = seq_len0 + s.rows - 1;                                // keys any row of the segment sees
    const int lo0 = window > 0 && seq_len0 > window ? seq_len0 - window : 0;  // the earliest key any row sees
    const int ch = ((ctx - lo0 + nch - 1) / nch + kFaKeys - 1) / kFaKeys * kFaKeys;
    const int k_lo = lo0 + c * ch, k_hi = min(ctx, k_lo + ch);
    float qf[HD / 4];
    fa_load_q<HD>(q + (static_cast<size_t>(s.row0 + tq) * heads + h) * hd, hd, 1.0f / sqrtf(static_cast<float>(hd)),
                  qf);
    float m = -INFINITY, l = 0.0f;
    fa4 o[HD / 16];
#pragma unroll
    for (int b = 0; b < HD / 16; ++b) o[b] = fa4{0.f, 0.f, 0.f, 0.f};
    fa_keys<C, HD, FAST>(kc, vc, M, s.slot, kvh, hd, k_lo, k_hi, qs, qe, wave_on, qf, tl, m, l, o);
    if (valid) {
        const size_t qv = static_cast<size_t>(s.row0 + t) * heads + h;  // [buffer row][head]
        float *pp = part + (qv * nch + c) * HD;
#pragma unroll
        for (int b = 0; b < HD / 16; ++b)
            *reinterpret_cast<fa4 *>(pp + 16 * b + 4 * grp) = o[b];
        if (grp == 0) {
            pml[(qv * nch + c) * 2] = m;
            pml[(qv * nch + c) * 2 + 1] = l;
        }
    }
}

// ---- fp16 caches on f16 MFMA (v_mfma_f32_16x16x32_f16) --------------------------------------------------------
// The fp32 products of the kernels above become exact f16 products: K and V are fp16 already; each fp32 operand
// that is not (the query, pre-scaled by 1/sqrt(hd) and by a power of two 2^s per query vector that puts its
// largest element near 2^14, and the softmax weights p in [0, 1]) is split into an f16 pair hi + lo with
// hi = f16(x), lo = f16(x - hi), 22 significant bits. Each MFMA adds exact products in fp32, so S and O differ
// from an fp32 evaluation only by the representation error of the pair (2^-22 relative per element) and by
// fp32 rounding of sums; S is scaled back by 2^-s exactly. Per 32 keys a wave issues HD/32 x 2 x 2 MFMAs for S
// and HD/16 x 2 for O (a quarter of the fp32 MFMA count, each at twice the rate).
//
// Operand layout of v_mfma_f32_16x16x32_f16 as used here: lane l = (col c = l & 15, group g = l >> 4) gives row c
// of A and column c of B at the same eight k slots (g, j), j < 8; the result has rows 4 g + r, column c.
//  - S^T (keys x query vectors) of key half h of a 32-key block: A = K rows (key kb + 16 h + c; dims 32 u + 8 g + j,
//    one 16-byte load), B = the query vector c at the same dims; lane (c, g) ends with keys kb + 16 h + 4 g + r.
//  - O^T (dims x query vectors) += V^T P^T: k slot (g, j) is key kb + 4 g + j (j < 4) or kb + 16 + 4 g + j - 4
//    (j >= 4), so B is the lane's own eight softmax weights and A is row 16 b + c of V^T at positions 8 g .. 8 g + 7:
//    V^T is staged per wave in LDS, [dim][32 positions] f16, 16-byte chunks XOR-swizzled by (dim >> 2) & 3
//    (the 16 rows a read instruction touches land on distinct banks).
typedef _Float16 fh8 __attribute__((ext_vector_type(8)));
typedef _Float16 fh4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ fh8 ld_h8(const _Float16 *p) {
    const uint4 v = *reinterpret_cast<const uint4 *>(p);
    return __builtin_bit_cast(fh8, v);
}
__device__ __forceinline__ void split_h(float x, _Float16 &hi, _Float16 &lo) {
    hi = static_cast<_Float16>(x);
    lo = static_cast<_Float16>(x - static_cast<float>(hi));
}
// Position of key k (0..31 of a block) among the 32 k slots of the O^T product.
__device__ __forceinline__ int fa16_pos(int k) { return k < 16 ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3); }
__device__ __forceinline__ int fa16_vt(int d, int pos) { return d * 32 + (((pos >> 3) ^ ((d >> 2) & 3)) << 3) + (pos & 7); }

// The query vector of lane column c (dims 32 u + 8 g .. + 7), loaded raw; fa16_q_split turns it into the B
// operands, times 1/sqrt(hd) * 2^s, and returns 2^-s log2(e): scores leave the S product in base-2 units, so
// the softmax weights are exp2 (v_exp_f32) of their differences, and maxima are converted back (times ln 2) only
// where they leave the kernel. Split in two so that a block's K/V loads can be issued
// between them.
template <int HD>
__device__ __forceinline__ void fa16_q_load(const float *qrow, float4 (&qr)[HD / 16]) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int u = 0; u < HD / 32; ++u) {
        qr[2 * u] = *reinterpret_cast<const float4 *>(qrow + 32 * u + 8 * g);
        qr[2 * u + 1] = *reinterpret_cast<const float4 *>(qrow + 32 * u + 8 * g + 4);
    }
}
template <int HD>
__device__ __forceinline__ float fa16_q_split(const float4 (&qr)[HD / 16], float scale, fh8 (&qh)[HD / 32],
                                              fh8 (&ql)[HD / 32]) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < HD / 16; ++i)
        amax = fmaxf(fmaxf(amax, fmaxf(fabsf(qr[i].x), fabsf(qr[i].y))), fmaxf(fabsf(qr[i].z), fabsf(qr[i].w)));
    amax *= scale;
    amax = xor16_max(amax);
    amax = xor32_max(amax);
    int ex = 0;
    if (amax > 0.0f && amax <= 3.0e38f) frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1)
    // Capped at 2^126 so that the scale and its inverse stay finite for queries below ~1e-34 (their scores are
    // then tiny, as they should be, instead of NaN).
    const int e2 = 14 - ex < 126 ? 14 - ex : 126;
    const float up = ldexpf(1.0f, e2);
#pragma unroll
    for (int u = 0; u < HD / 32; ++u) {
        const float v[8] = {qr[2 * u].x, qr[2 * u].y, qr[2 * u].z, qr[2 * u].w,
                            qr[2 * u + 1].x, qr[2 * u + 1].y, qr[2 * u + 1].z, qr[2 * u + 1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            _Float16 h, l;
            split_h(v[j] * scale * up, h, l);
            qh[u][j] = h;
            ql[u][j] = l;
        }
    }
    return ldexpf(1.0f, -e2) * 1.44269504088896341f;  // S in base-2 units: the softmax uses exp2
}

// The raw K and V of one 32-key block in registers: K as S^T A operands, V as units of four keys x one
// 16-byte chunk (unit lane + 64 it: key quad unit & 7, chunk unit >> 3; the eight key quads of a chunk sit in
// adjacent lanes, which spreads a V^T write instruction over 32 banks instead of 8).
template <int HD>
struct Fa16Raw {
    fh8 ka[2][HD / 32];
    fh8 vv[HD / 64][4];
};

// Issue the loads of block [kb, kb + 32) of kv head kvh (keys at or past k_hi read the last key's row).
template <int HD, bool PAGED>
__device__ __forceinline__ void fa16_issue(const _Float16 *__restrict__ kc, const _Float16 *__restrict__ vc,
                                           const KvMap &M, int slot, int kvh, int kb, int k_hi, Fa16Raw<HD> &rw) {
    constexpr int CR = HD / 8;  // 16-byte chunks per row
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    // Cache rows of the block's keys: lane k < 32 looks up key kb + k, the others read it by shuffle.
    const size_t myrow = M.row_t<PAGED>(slot, kvh, min(kb + (lane & 31), k_hi - 1));
    auto row_of = [&](int k) {
        const uint32_t lo32 = __shfl(static_cast<uint32_t>(myrow), k, 64);
        const uint32_t hi32 = __shfl(static_cast<uint32_t>(myrow >> 32), k, 64);
        return (static_cast<size_t>(hi32) << 32) | lo32;
    };
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const size_t kr = row_of(16 * h + c) * HD + 8 * g;
#pragma unroll
        for (int u = 0; u < HD / 32; ++u) rw.ka[h][u] = ld_h8(kc + kr + 32 * u);
    }
#pragma unroll
    for (int it = 0; it < HD / 64; ++it) {
        const int unit = lane + 64 * it, dc = unit >> 3, qd = unit & 7;
#pragma unroll
        for (int i = 0; i < 4; ++i) rw.vv[it][i] = ld_h8(vc + row_of(4 * qd + i) * HD + 8 * dc);
    }
}

// Online softmax over the S^T values of block [kb, kb + 32) (s[h][r]: key kb + 16 h + 4 g + r, query column c sees
// keys [qs, qe), keys at or past k_hi masked), then O^T += V^T P^T from the block's V^T in LDS (vt, read at rows
// 16 b + c, positions 8 g ..). The caller makes vt visible first.
template <int HD>
__device__ __forceinline__ void fa16_softmax_pv(const fa4 (&s)[2], int kb, int k_hi, int qs, int qe, const _Float16 *vt,
                                                float &m, float &l, fa4 (&o)[HD / 16]) {
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    float v[8], bm = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = kb + 16 * h + 4 * g + r;
            v[4 * h + r] = p >= qs && p < qe && p < k_hi ? s[h][r] : -INFINITY;
            bm = fmaxf(bm, v[4 * h + r]);
        }
    bm = xor16_max(bm);
    bm = xor32_max(bm);
    const float mn = fmaxf(m, bm);
    const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
    fh8 ph, pl;
    float ps = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float p = v[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(v[j] - mn);
        ps += p;
        _Float16 hh, ll;
        split_h(p, hh, ll);
        ph[j] = hh;
        pl[j] = ll;
    }
    ps = xor16_add(ps);
    ps = xor32_add(ps);
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int b = 0; b < HD / 16; ++b) {
        const fh8 a = *reinterpret_cast<const fh8 *>(vt + fa16_vt(16 * b + c, 8 * g));
        fa4 ob = o[b] * alpha;
        ob = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph, ob, 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, ob, 0, 0, 0);
    }
}

// V unit (key quad qd, 16-byte chunk dc) of a block into V^T: eight 8-byte writes (four keys of one dim at
// consecutive positions).
template <int HD>
__device__ __forceinline__ void fa16_put_vt(_Float16 *vt, int qd, int dc, const fh8 (&v4)[4]) {
    const int pos = fa16_pos(4 * qd);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const fh4 w{v4[0][j], v4[1][j], v4[2][j], v4[3][j]};
        *reinterpret_cast<fh4 *>(vt + fa16_vt(8 * dc + j, pos)) = w;
    }
}

// Block kb (loaded in rw) against the wave's 16 query vectors; vt is the wave's own V^T area (HD x 32 f16).
template <int HD>
__device__ __forceinline__ void fa16_consume(const Fa16Raw<HD> &rw, int kb, int k_hi, int qs, int qe,
                                             const fh8 (&qh)[HD / 32], const fh8 (&ql)[HD / 32], float sinv,
                                             _Float16 *vt, float &m, float &l, fa4 (&o)[HD / 16]) {
    constexpr int CR = HD / 8;
    const int lane = threadIdx.x & 63;
    // S^T for both key halves: hi and lo query parts in separate chains.
    fa4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        fa4 a0{0.f, 0.f, 0.f, 0.f}, a1{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < HD / 32; ++u) {
            a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(rw.ka[h][u], qh[u], a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(rw.ka[h][u], ql[u], a1, 0, 0, 0);
        }
        s[h] = (a0 + a1) * sinv;
    }
#pragma unroll
    for (int it = 0; it < HD / 64; ++it) {
        const int unit = lane + 64 * it;
        fa16_put_vt<HD>(vt, unit & 7, unit >> 3, rw.vv[it]);
    }
    // A wave's LDS operations complete in issue order; the fence keeps the compiler from moving the V^T reads
    // above the writes of other lanes.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    fa16_softmax_pv<HD>(s, kb, k_hi, qs, qe, vt, m, l, o);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // every lane has read V^T before the next block's writes
    __builtin_amdgcn_wave_barrier();
}

// Prompt passes on fp16 caches: a workgroup takes 16 query rows of one segment and up to four query heads of one kv
// head (one wave each). Its 256 threads stage each 32-key block once for all four: K row-major [32][HD + 8] f16
// (the S^T A fragments are 16-byte reads, rows 528 bytes apart for HD 256: no two of a read's 16 rows share banks),
// V^T as in the decode kernel; the next two blocks' loads are in flight while one is used.
template <int HD, bool PAGED>
__global__ __launch_bounds__(256) void attention_prompt16_kernel(const float *__restrict__ q,
                                                                 const _Float16 *__restrict__ kc,
                                                                 const _Float16 *__restrict__ vc, float *__restrict__ out,
                                                                 SegTable T, KvMap M, int heads, int bidirectional,
                                                                 int window, int chunks) {
    constexpr int CR = HD / 8, LDK = HD + 8;
    constexpr int KU = 32 * CR / 256;  // K chunks per thread per block
    constexpr int VU = 8 * CR / 256;   // V units per thread per block (HD 64: half the threads take one)
    __shared__ __align__(16) _Float16 ks[32 * LDK];
    __shared__ __align__(16) _Float16 vts[HD * 32];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    int tb = blockIdx.x, si = 0;
    while (si + 1 < T.n && tb >= (T.s[si].rows + 15) / 16) {
        tb -= (T.s[si].rows + 15) / 16;
        ++si;
    }
    const Seg &s = T.s[si];
    const int G = heads / M.kv_heads;
    const int kvh = blockIdx.y / chunks, gi = (blockIdx.y - kvh * chunks) * 4 + wv;
    const bool wave_on = gi < G;
    const int h = kvh * G + (wave_on ? gi : 0);
    const int t0 = 16 * tb, nq = min(16, s.rows - t0);
    const int seq_len0 = s.pos0 + 1;
    auto q_end = [&](int t) { return bidirectional ? seq_len0 + s.rows - 1 : seq_len0 + t; };
    auto q_start = [&](int t) { return window > 0 && seq_len0 + t > window ? seq_len0 + t - window : 0; };
    const int tq = t0 + min(c, nq - 1);  // this lane's query row (rows past nq repeat the last; not written)
    const int qs = q_start(tq), qe = q_end(tq);
    const int k_lo = q_start(t0), k_hi = q_end(t0 + nq - 1);
    float4 qr[HD / 16];
    fa16_q_load<HD>(q + (static_cast<size_t>(s.row0 + tq) * heads + h) * HD, qr);
    // Block loads of this thread: K chunks i = tid + 256 k (key i / CR, chunk i % CR); V unit tid (key quad tid & 7,
    // chunk tid >> 3).
    // Two blocks are in flight ahead of the one being used (register buffers A and B).
    struct Buf {
        fh8 k[KU];
        fh8 v[VU > 0 ? VU : 1][4];
    };
    auto row_of = [&](int key) { return M.row_t<PAGED>(s.slot, kvh, min(key, k_hi - 1)); };
    auto issue = [&](Buf &bf, int kb) {
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int i = threadIdx.x + 256 * k;
            bf.k[k] = ld_h8(kc + row_of(kb + i / CR) * HD + 8 * (i % CR));
        }
#pragma unroll
        for (int k = 0; k < (VU > 0 ? VU : 1); ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < 8 * CR)
#pragma unroll
                for (int j = 0; j < 4; ++j) bf.v[k][j] = ld_h8(vc + row_of(kb + 4 * (i & 7) + j) * HD + 8 * (i >> 3));
        }
    };
    Buf ba, bb;
    if (k_lo < k_hi) issue(ba, k_lo);
    if (k_lo + 32 < k_hi) issue(bb, k_lo + 32);
    fh8 qh[HD / 32], ql[HD / 32];
    const float sinv = fa16_q_split<HD>(qr, 1.0f / sqrtf(static_cast<float>(HD)), qh, ql);
    float m = -INFINITY, l = 0.0f;
    fa4 o[HD / 16];
#pragma unroll
    for (int b = 0; b < HD / 16; ++b) o[b] = fa4{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](Buf &bf, int kb) {
        __syncthreads();  // the previous block is consumed
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int i = threadIdx.x + 256 * k;
            *reinterpret_cast<fh8 *>(ks + (i / CR) * LDK + 8 * (i % CR)) = bf.k[k];
        }
#pragma unroll
        for (int k = 0; k < (VU > 0 ? VU : 1); ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < 8 * CR) fa16_put_vt<HD>(vts, i & 7, i >> 3, bf.v[k]);
        }
        __syncthreads();
        if (kb + 64 < k_hi) issue(bf, kb + 64);
        if (!wave_on) return;
        fa4 sc[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            fa4 a0{0.f, 0.f, 0.f, 0.f}, a1{0.f, 0.f, 0.f, 0.f};
            const _Float16 *kp = ks + (16 * hh + c) * LDK + 8 * g;
#pragma unroll
            for (int u = 0; u < HD / 32; ++u) {
                const fh8 a = *reinterpret_cast<const fh8 *>(kp + 32 * u);
                a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[u], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[u], a1, 0, 0, 0);
            }
            sc[hh] = (a0 + a1) * sinv;
        }
        fa16_softmax_pv<HD>(sc, kb, k_hi, qs, qe, vts, m, l, o);
    };
    for (int kb = k_lo; kb < k_hi; kb += 64) {
        consume(ba, kb);
        if (kb + 32 < k_hi) consume(bb, kb + 32);
    }
    // o[b][r]: head dim 16 b + 4 g + r of query row tq
    if (wave_on && c < nq) {
        float *orow = out + (static_cast<size_t>(s.row0 + t0 + c) * heads + h) * HD;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int b = 0; b < HD / 16; ++b)
            *reinterpret_cast<float4 *>(orow + 16 * b + 4 * g) =
                float4{o[b][0] * inv, o[b][1] * inv, o[b][2] * inv, o[b][3] * inv};
    }
}

// Decode and verify passes on fp16 caches: one workgroup per (segment, kv head, chunk of the keys, group of 16
// query vectors); its four waves take the chunk's 32-key blocks in turn (wave w: blocks w, w + 4, ...) with their
// own online softmax, then combine in wave order through LDS. With one chunk the workgroup writes the output;
// otherwise its unnormalised output and (max, sum) go to the workspace for attention_merge_kernel.
template <int HD, bool PAGED>
__global__ __launch_bounds__(256) void attention_split16_kernel(const float *__restrict__ q,
                                                                const _Float16 *__restrict__ kc,
                                                                const _Float16 *__restrict__ vc, float *__restrict__ part,
                                                                float *__restrict__ pml, float *__restrict__ out,
                                                                SegTable T, KvMap M, int heads, int bidirectional,
                                                                int window, int nch) {
    __shared__ __align__(16) _Float16 vts[4][HD * 32];  // per-wave V^T; reused as the per-wave [16][HD] fp32 output
    __shared__ float sm[4][16], sl[4][16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int ci = blockIdx.x % nch, sk_id = blockIdx.x / nch;
    const int kvh = sk_id % M.kv_heads, si = sk_id / M.kv_heads;
    const Seg &s = T.s[si];
    const int G = heads / M.kv_heads;
    const int j = blockIdx.y * 16 + c;  // query vector of this lane's column
    const int t = j / G, gi = j - t * G;
    const bool valid = t < s.rows;
    const int tq = valid ? t : s.rows - 1, h = kvh * G + (valid ? gi : 0);
    const int seq_len0 = s.pos0 + 1;
    const int qe = bidirectional ? seq_len0 + s.rows - 1 : seq_len0 + tq;
    const int qs = window > 0 && seq_len0 + tq > window ? seq_len0 + tq - window : 0;
    const int ctx = seq_len0 + s.rows - 1;
    const int lo0 = window > 0 && seq_len0 > window ? seq_len0 - window : 0;
    const int ch = ((ctx - lo0 + nch - 1) / nch + kFaKeys - 1) / kFaKeys * kFaKeys;
    const int k_lo = lo0 + ci * ch, k_hi = min(ctx, k_lo + ch);
    float m = -INFINITY, l = 0.0f;
    fa4 o[HD / 16];
#pragma unroll
    for (int b = 0; b < HD / 16; ++b) o[b] = fa4{0.f, 0.f, 0.f, 0.f};
    if (blockIdx.y * 16 < s.rows * G) {  // groups past the segment's query vectors only wait at the barrier
        // The query's loads, then the first block's, in flight together.
        float4 qr[HD / 16];
        fa16_q_load<HD>(q + (static_cast<size_t>(s.row0 + tq) * heads + h) * HD, qr);
        Fa16Raw<HD> rw;
        int kb = k_lo + 32 * wv;
        if (kb < k_hi) fa16_issue<HD, PAGED>(kc, vc, M, s.slot, kvh, kb, k_hi, rw);
        fh8 qh[HD / 32], ql[HD / 32];
        const float sinv = fa16_q_split<HD>(qr, 1.0f / sqrtf(static_cast<float>(HD)), qh, ql);
        for (; kb < k_hi; kb += 128) {
            fa16_consume<HD>(rw, kb, k_hi, qs, qe, qh, ql, sinv, vts[wv], m, l, o);
            if (kb + 128 < k_hi) fa16_issue<HD, PAGED>(kc, vc, M, s.slot, kvh, kb + 128, k_hi, rw);
        }
    }
    // Combine the four waves in wave order: o[b][r] is dim 16 b + 4 g + r of query vector c.
    __syncthreads();
    float *ow = reinterpret_cast<float *>(vts[wv]);  // [16][HD]
#pragma unroll
    for (int b = 0; b < HD / 16; ++b)
        *reinterpret_cast<fa4 *>(ow + c * HD + 16 * b + 4 * g) = o[b];
    if (g == 0) {
        sm[wv][c] = m;
        sl[wv][c] = l;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 16 * (HD / 4); e += 256) {
        const int qc = e / (HD / 4), d4 = 4 * (e - qc * (HD / 4));
        const int jj = blockIdx.y * 16 + qc, tt = jj / G;
        if (tt >= s.rows) continue;
        const int hh = kvh * G + (jj - tt * G);
        const float mx = fmaxf(fmaxf(sm[0][qc], sm[1][qc]), fmaxf(sm[2][qc], sm[3][qc]));
        float L = 0.0f;
        float4 acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = sm[w][qc] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sm[w][qc] - mx);
            L = fmaf(sl[w][qc], f, L);
            const float4 p4 = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(vts[w]) + qc * HD + d4);
            acc.x = fmaf(p4.x, f, acc.x);
            acc.y = fmaf(p4.y, f, acc.y);
            acc.z = fmaf(p4.z, f, acc.z);
            acc.w = fmaf(p4.w, f, acc.w);
        }
        const size_t qv = static_cast<size_t>(s.row0 + tt) * heads + hh;
        if (nch == 1) {
            const float inv = L > 0.0f ? 1.0f / L : 0.0f;
            *reinterpret_cast<float4 *>(out + qv * HD + d4) = float4{acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
        } else {
            *reinterpret_cast<float4 *>(part + (qv * nch + ci) * HD + d4) = acc;
            if (d4 == 0) {
                pml[(qv * nch + ci) * 2] = mx * 0.693147180559945309f;  // natural units for the merge
                pml[(qv * nch + ci) * 2 + 1] = L;
            }
        }
    }
}

// out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, M = max_c m_c; one workgroup of four waves per (row of the
// pass, head): the chunks' maxima through LDS, then wave w adds chunks w, w + 4, ... (lane = four head dims, one
// 16-byte load per chunk) and the four waves' sums are added in wave order (deterministic).
template <int HD>
__global__ __launch_bounds__(256) void attention_merge_kernel(const float *__restrict__ part, const float *__restrict__ pml,
                                                              float *__restrict__ out, SegTable T, int heads, int hd,
                                                              int nch) {
    __shared__ float smx[4];
    __shared__ float4 sacc[4][HD / 4];
    __shared__ float sl[4];
    int t;
    const Seg &s = seg_of_row(T, blockIdx.x / heads, t);
    const int h = blockIdx.x % heads;
    const size_t qv = static_cast<size_t>(s.row0 + t) * heads + h;
    const float *ml = pml + qv * nch * 2;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float mx = -INFINITY;
    for (int c = tid; c < nch; c += 256) mx = fmaxf(mx, ml[2 * c]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) smx[wv] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(smx[0], smx[1]), fmaxf(smx[2], smx[3]));
    float4 acc{0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    if (4 * lane < HD) {
        // Chunks wv, wv + 4, ... in order, four at a time with all their loads in flight.
        for (int c0 = wv; c0 < nch; c0 += 16) {
            float4 p4[4];
            float mc[4], lc[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int c = c0 + 4 * k < nch ? c0 + 4 * k : c0;
                p4[k] = *reinterpret_cast<const float4 *>(part + (qv * nch + c) * HD + 4 * lane);
                mc[k] = ml[2 * c];
                lc[k] = ml[2 * c + 1];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (c0 + 4 * k >= nch) break;
                const float f = mc[k] == -INFINITY ? 0.0f : expf(mc[k] - M);
                L = fmaf(lc[k], f, L);
                acc.x = fmaf(p4[k].x, f, acc.x);
                acc.y = fmaf(p4[k].y, f, acc.y);
                acc.z = fmaf(p4[k].z, f, acc.z);
                acc.w = fmaf(p4[k].w, f, acc.w);
            }
        }
        sacc[wv][lane] = acc;
    }
    if (lane == 0) sl[wv] = L;
    __syncthreads();
    if (wv == 0 && 4 * lane < HD) {
        const float Lt = ((sl[0] + sl[1]) + sl[2]) + sl[3];
        const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
        const float4 a = sacc[0][lane], b = sacc[1][lane], c = sacc[2][lane], d = sacc[3][lane];
        const float r[4] = {((a.x + b.x) + c.x) + d.x, ((a.y + b.y) + c.y) + d.y, ((a.z + b.z) + c.z) + d.z,
                            ((a.w + b.w) + c.w) + d.w};
        float *o = out + qv * hd;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (4 * lane + k < hd) o[4 * lane + k] = r[k] * inv;
    }
}

// Chunks per sequence of a split decode pass: about 512 workgroups for the whole pass, at least 32 keys each.
int split_chunks(const SegTable &T, int kv_heads, int window) {
    int ctx = 1;
    for (int i = 0; i < T.n; ++i) {
        int c = T.s[i].pos0 + T.s[i].rows;
        if (window > 0 && c > window + T.s[i].rows) c = window + T.s[i].rows;
        ctx = c > ctx ? c : ctx;
    }
    const int want = (512 + T.n * kv_heads - 1) / (T.n * kv_heads);
    const int most = (ctx + kFaKeys - 1) / kFaKeys;
    return want < 1 ? 1 : want > most ? most : want;
}
int fa_hd(int hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : 256; }
int max_seg_rows(const SegTable &T) {
    int r = 0;
    for (int i = 0; i < T.n; ++i) r = T.s[i].rows > r ? T.s[i].rows : r;
    return r;
}
// Chunks per sequence of the fp16 decode kernel: one 32-key block per wave where the keys allow it, at most about
// 512 workgroups for the pass.
int split16_chunks(const SegTable &T, int heads, int kv_heads, int window) {
    int ctx = 1;
    for (int i = 0; i < T.n; ++i) {
        int c = T.s[i].pos0 + T.s[i].rows;
        if (window > 0 && c > window + T.s[i].rows) c = window + T.s[i].rows;
        ctx = c > ctx ? c : ctx;
    }
    const int qgroups = (max_seg_rows(T) * (heads / kv_heads) + 15) / 16;
    const int want = ((ctx + kFaKeys - 1) / kFaKeys + 3) / 4;
    const int cap = 512 / (T.n * kv_heads * qgroups);
    return want < 1 ? 1 : want < cap ? want : cap < 1 ? 1 : cap;
}
size_t split_ws_bytes(const SegTable &T, int span_rows, int heads, int kv_heads, int hd, int window) {
    const int n32 = split_chunks(T, kv_heads, window), n16 = split16_chunks(T, heads, kv_heads, window);
    const int nch = n32 > n16 ? n32 : n16;
    return static_cast<size_t>(span_rows) * heads * nch * (fa_hd(hd) + 2) * 4 + 256;
}

// ---- causal conv update ----------------------------------------------------------------------------------

// Depthwise causal conv + SiLU, one thread per (channel, segment), the K-tap window in registers (K a template
// parameter: the shift is register renaming). Per row: window <- [window[1:], x], out = silu(window . w).
// snap (one segment only) gets the window after each row but the last, [rows - 1][channels][K]; the state
// [slot][channels][K] gets the last window unless write_state is 0 (a verification pass leaves it untouched).
template <int K>
__global__ __launch_bounds__(256) void conv_update_kernel(const float *__restrict__ x, float *__restrict__ state,
                                                          const float *__restrict__ w, float *__restrict__ out,
                                                          int channels, SegTable T, float *__restrict__ snap,
                                                          int write_state) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= channels) return;
    const Seg &s = T.s[blockIdx.y];
    float *st = state + (static_cast<size_t>(s.slot) * channels + c) * K;
    float win[K], wc[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        win[k] = st[k];
        wc[k] = w[static_cast<size_t>(c) * K + k];
    }
    const size_t row = static_cast<size_t>(s.row0) * channels + c;
    for (int t = 0; t < s.rows; ++t) {
        const float xi = x[row + static_cast<size_t>(t) * channels];
#pragma unroll
        for (int k = 0; k + 1 < K; ++k) win[k] = win[k + 1];
        win[K - 1] = xi;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) acc = fmaf(win[k], wc[k], acc);
        out[row + static_cast<size_t>(t) * channels] = silu_ieee(acc);
        if (snap != nullptr && t + 1 < s.rows) {
            float *sn = snap + (static_cast<size_t>(t) * channels + c) * K;
#pragma unroll
            for (int k = 0; k < K; ++k) sn[k] = win[k];
        }
    }
    if (write_state) {
#pragma unroll
        for (int k = 0; k < K; ++k) st[k] = win[k];
    }
}

// ---- gated delta rule ------------------------------------------------------------------------------------

// State S [slot][vh][kd][vd] of the gated delta rule, held in VGPRs for the whole pass. A wave owns 8 state
// columns of one value head: lane = (column c = lane & 7, row group g = lane >> 3), and the lane keeps rows
// g*R .. g*R + R - 1 of its column (R = rows per lane, kd <= 8R; rows past kd are zero and never stored). Per
// token every sum over the kd rows is the lane's own R-term chain plus three xor steps over the row groups
// (lanes 8, 16 and 32 apart), so no LDS and no barrier is involved; waves are independent.
//
// Per token (row rr of the segment): q^ = q / (sqrt(|q|^2 + eps) sqrt(kd)), k^ = k / sqrt(|k|^2 + eps),
// beta = sigmoid(b), decay = exp(ssm_a * softplus(a + dt)) with torch's softplus (identity above 20);
// S *= decay; delta = (v - S^T k^) beta; S += k^ delta^T; out = S^T q^. The state is read once and written
// once per pass (fp32, or fp16 widened to fp32 in registers and rounded once when written back).
constexpr int kGdCols = 8, kGdGroups = 64 / kGdCols, kGdMaxKd = 256;

__device__ __forceinline__ float gsum(float v) {  // sum over the 8 row groups of a column (lanes 8, 16, 32 apart)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
    return xor32_add(xor16_add(v));
}
__device__ __forceinline__ float ld_state(const float *p) { return *p; }
__device__ __forceinline__ float ld_state(const _Float16 *p) { return static_cast<float>(*p); }
__device__ __forceinline__ void st_state(float *p, float v) { *p = v; }
__device__ __forceinline__ void st_state(_Float16 *p, float v) { *p = static_cast<_Float16>(v); }

template <int R, typename ST>
__global__ __launch_bounds__(256) void gated_delta_kernel(const float *__restrict__ conv, const float *__restrict__ braw,
                                                          const float *__restrict__ araw, const float *__restrict__ ssm_a,
                                                          const float *__restrict__ dt, ST *__restrict__ state,
                                                          float *__restrict__ out, int key_heads, int value_heads,
                                                          int kd, int vd, float eps, int head_order, SegTable T,
                                                          float *__restrict__ snap, int write_state) {
    const int lane = threadIdx.x & 63;
    const int tiles = (vd + kGdCols - 1) / kGdCols;
    const int wid = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (wid >= value_heads * tiles) return;  // whole waves leave; nothing below synchronises across waves
    const int h = wid / tiles, c0 = (wid - h * tiles) * kGdCols;
    const int c = lane & (kGdCols - 1), g = lane / kGdCols;
    const int col = c0 + c, r0 = g * R;
    const bool col_ok = col < vd;
    const int kh = head_order == 0 ? h / (value_heads / key_heads) : h % key_heads;
    const Seg &s = T.s[blockIdx.y];
    const size_t hstate = static_cast<size_t>(kd) * vd;
    ST *S = state + (static_cast<size_t>(s.slot) * value_heads + h) * hstate;
    const size_t cdim = static_cast<size_t>(2) * key_heads * kd + static_cast<size_t>(value_heads) * vd;

    float st[R];
#pragma unroll
    for (int i = 0; i < R; ++i)
        st[i] = col_ok && r0 + i < kd ? ld_state(S + static_cast<size_t>(r0 + i) * vd + col) : 0.0f;
    const float a_h = ssm_a[h], dt_h = dt[h];
    const float rkd = 1.0f / sqrtf(static_cast<float>(kd));

    for (int t = 0; t < s.rows; ++t) {
        const size_t rr = static_cast<size_t>(s.row0) + t;
        const float *qs = conv + rr * cdim + static_cast<size_t>(kh) * kd;
        const float *ks = qs + static_cast<size_t>(key_heads) * kd;
        float qv[R], kv[R];
        float qq = 0.0f, kk = 0.0f;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const bool ok = r0 + i < kd;
            qv[i] = ok ? qs[r0 + i] : 0.0f;
            kv[i] = ok ? ks[r0 + i] : 0.0f;
            qq = fmaf(qv[i], qv[i], qq);
            kk = fmaf(kv[i], kv[i], kk);
        }
        const float v = col_ok ? conv[rr * cdim + static_cast<size_t>(2) * key_heads * kd + static_cast<size_t>(h) * vd + col]
                               : 0.0f;
        const float beta = sigmoid_ieee(braw[rr * value_heads + h]);
        const float xa = araw[rr * value_heads + h] + dt_h;
        const float decay = expf(a_h * (xa > 20.0f ? xa : log1pf(expf(xa))));
        qq = gsum(qq);
        kk = gsum(kk);
        const float qscale = rkd / sqrtf(qq + eps);
        const float kscale = 1.0f / sqrtf(kk + eps);
        float mem = 0.0f;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            st[i] *= decay;
            mem = fmaf(st[i], kv[i], mem);
        }
        mem = gsum(mem) * kscale;
        const float upd = (v - mem) * beta * kscale;  // S[i] += k[i] * kscale * delta
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            st[i] = fmaf(kv[i], upd, st[i]);
            o = fmaf(st[i], qv[i], o);
        }
        o = gsum(o) * qscale;
        if (g == 0 && col_ok) out[(rr * value_heads + h) * vd + col] = o;
        if (snap != nullptr && t + 1 < s.rows && col_ok) {
            float *sn = snap + (static_cast<size_t>(t) * value_heads + h) * hstate;
#pragma unroll
            for (int i = 0; i < R; ++i)
                if (r0 + i < kd) sn[static_cast<size_t>(r0 + i) * vd + col] = st[i];
        }
    }
    if (write_state && col_ok) {
#pragma unroll
        for (int i = 0; i < R; ++i)
            if (r0 + i < kd) st_state(S + static_cast<size_t>(r0 + i) * vd + col, st[i]);
    }
}

// The same rule with four adjacent state columns per lane (vd % 4 == 0, aligned state): lane = (row group
// g = lane & 7, column quad cq = lane >> 3), a wave owns 32 columns and each row segment it reads or writes is
// 128 bytes (fp32) or 64 bytes (fp16) long instead of 32 or 16. One wave per workgroup, so the 48 x 4 waves of
// the qwen35 shape spread over the CUs. Sums over rows: the lane's R-term chains (one per column) plus three
// DPP steps over the eight row groups, which sit in adjacent lanes (no LDS-path shuffles on the per-token
// recurrence). Every lane of a group ends with the same bits: each step adds the same two values.
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
    int p;
    switch (ctrl_sel) {
        case 0: p = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false); break;   // quad_perm 1,0,3,2
        case 1: p = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false); break;   // quad_perm 2,3,0,1
        default: p = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false); break; // row_half_mirror
    }
    return v + __int_as_float(p);
}
__device__ __forceinline__ float gsum8(float v) { return dpp_add(dpp_add(dpp_add(v, 0), 1), 2); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
__device__ __forceinline__ void st4(_Float16 *p, float4 v) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<h4 *>(p) = h4{static_cast<_Float16>(v.x), static_cast<_Float16>(v.y), static_cast<_Float16>(v.z),
                                    static_cast<_Float16>(v.w)};
}

// The pass walks its tokens in chunks of up to kGdChunk: a chunk's inputs (per token the q and k rows of the head's
// key head and the wave's 32 v columns, a record of 2 kd + 32 floats) reach LDS by DMA, all in flight at once,
// and the recurrence then reads them from LDS, so a pass costs one memory round trip per chunk, not per token.
constexpr int kGdChunk = 16;
constexpr int kGdWaves = 4;  // waves per column tile of the multi-wave form (kd 128 or 256; 2 measured slower)
size_t gd_lds_bytes(int kd, int tc) { return (static_cast<size_t>(tc) * (2 * kd + 32) + 256) * sizeof(float); }

// NW waves share a column tile and split its rows (wave w: rows 8 R w .. 8 R (w + 1) - 1); their partial sums over
// rows meet in LDS and are added in wave order (two barriers per token).
template <int R, typename ST, bool FULL, int NW = 1>  // FULL: kd == 8 R NW, every row of every lane is a state row
__global__ __launch_bounds__(64 * NW) void gated_delta4_kernel(const float *__restrict__ conv, const float *__restrict__ braw,
                                                          const float *__restrict__ araw, const float *__restrict__ ssm_a,
                                                          const float *__restrict__ dt, ST *__restrict__ state,
                                                          float *__restrict__ out, int key_heads, int value_heads,
                                                          int kd, int vd, float eps, int head_order, SegTable T,
                                                          float *__restrict__ snap, int write_state, int tc) {
    extern __shared__ __align__(16) float gd_in[];  // [tc][2 kd + 32] + 1 KB of slack for the last DMA's spare lanes
    __shared__ float4 red_m[NW][8], red_o[NW][8];   // per-wave partial sums of the 8 column quads
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int tiles = (vd + 31) / 32;
    const int h = blockIdx.x / tiles, c0 = (blockIdx.x - h * tiles) * 32;
    const int col = c0 + 4 * (lane >> 3), r0 = (wv * 8 + (lane & 7)) * R;
    const bool col_ok = col < vd;  // vd % 4 == 0: a quad is whole or absent
    const int cc = col_ok ? col : 0;
    const int kh = head_order == 0 ? h / (value_heads / key_heads) : h % key_heads;
    const Seg &s = T.s[blockIdx.y];
    const size_t hstate = static_cast<size_t>(kd) * vd;
    ST *S = state + (static_cast<size_t>(s.slot) * value_heads + h) * hstate;
    const size_t cdim = static_cast<size_t>(2) * key_heads * kd + static_cast<size_t>(value_heads) * vd;
    const float *cbase = conv + static_cast<size_t>(s.row0) * cdim;
    const int rec = 2 * kd + 32, rec4 = rec / 4;
    float4 st[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const bool ok = col_ok && r0 + i < kd;
        const float4 v = ld4(S, static_cast<size_t>(ok ? r0 + i : 0) * vd + cc);
        const float m = ok ? 1.0f : 0.0f;
        st[i] = float4{v.x * m, v.y * m, v.z * m, v.w * m};
    }
    const float a_h = ssm_a[h], dt_h = dt[h];
    const float rkd = 1.0f / sqrtf(static_cast<float>(kd));
    for (int t0 = 0; t0 < s.rows; t0 += tc) {
        const int nt = min(tc, s.rows - t0);
        __syncthreads();  // the previous chunk's records are consumed
        const int units = nt * rec4;
        for (int u0 = 64 * wv; u0 < units; u0 += 64 * NW) {
            const int u = min(u0 + lane, units - 1);
            const int tt = u / rec4, w = 4 * (u - tt * rec4);
            const size_t row = static_cast<size_t>(t0 + tt) * cdim;
            size_t off;
            if (w < kd) off = row + static_cast<size_t>(kh) * kd + w;
            else if (w < 2 * kd) off = row + static_cast<size_t>(key_heads + kh) * kd + (w - kd);
            else off = row + static_cast<size_t>(2) * key_heads * kd + static_cast<size_t>(h) * vd +
                       (c0 + w - 2 * kd < vd ? c0 + w - 2 * kd : 0);
            vq::dma16(cbase, static_cast<uint32_t>(off * sizeof(float)), gd_in + 4 * u0);
        }
        const float bt = lane < nt ? braw[static_cast<size_t>(s.row0 + t0 + lane) * value_heads + h] : 0.0f;
        const float at = lane < nt ? araw[static_cast<size_t>(s.row0 + t0 + lane) * value_heads + h] : 0.0f;
        vq::wait_vm<0>();
        __syncthreads();
        // Everything of a token that does not depend on the state, for all the chunk's tokens at once: lane l
        // holds beta and the decay of token l, and (four lanes per token) the q and k norm scales of token l / 4.
        // The per-token recurrence below then only reads them (v_readlane).
        const float beta_l = sigmoid_ieee(bt);
        const float xa_l = at + dt_h;
        const float decay_l = expf(a_h * (xa_l > 20.0f ? xa_l : log1pf(expf(xa_l))));
        float qsc_l, ksc_l;
        {
            const float4 *rp = reinterpret_cast<const float4 *>(gd_in + min(lane >> 2, nt - 1) * rec);
            float pq = 0.0f, pk = 0.0f;
            for (int f4 = lane & 3; f4 < kd / 4; f4 += 4) {
                const float4 a = rp[f4], b = rp[kd / 4 + f4];
                pq = fmaf(a.x, a.x, fmaf(a.y, a.y, fmaf(a.z, a.z, fmaf(a.w, a.w, pq))));
                pk = fmaf(b.x, b.x, fmaf(b.y, b.y, fmaf(b.z, b.z, fmaf(b.w, b.w, pk))));
            }
            pq = dpp_add(dpp_add(pq, 0), 1);  // the four lanes of a token
            pk = dpp_add(dpp_add(pk, 0), 1);
            qsc_l = rkd / sqrtf(pq + eps);
            ksc_l = 1.0f / sqrtf(pk + eps);
        }
        auto lane_val = [](float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); };
        for (int tt = 0; tt < nt; ++tt) {
            const size_t rr = static_cast<size_t>(s.row0) + t0 + tt;
            const float *rq = gd_in + tt * rec;
            float qv[R], kv[R];
#pragma unroll
            for (int i4 = 0; i4 < R / 4; ++i4) {
                const int r = r0 + 4 * i4;
                const bool ok = FULL || r < kd;  // kd % 4 == 0: a row quad is whole or absent
                const float4 a = *reinterpret_cast<const float4 *>(rq + (ok ? r : 0));
                const float4 b = *reinterpret_cast<const float4 *>(rq + kd + (ok ? r : 0));
                if (FULL) {
                    qv[4 * i4] = a.x, qv[4 * i4 + 1] = a.y, qv[4 * i4 + 2] = a.z, qv[4 * i4 + 3] = a.w;
                    kv[4 * i4] = b.x, kv[4 * i4 + 1] = b.y, kv[4 * i4 + 2] = b.z, kv[4 * i4 + 3] = b.w;
                } else {
                    const float m = ok ? 1.0f : 0.0f;
                    qv[4 * i4] = a.x * m, qv[4 * i4 + 1] = a.y * m, qv[4 * i4 + 2] = a.z * m, qv[4 * i4 + 3] = a.w * m;
                    kv[4 * i4] = b.x * m, kv[4 * i4 + 1] = b.y * m, kv[4 * i4 + 2] = b.z * m, kv[4 * i4 + 3] = b.w * m;
                }
            }
            const float4 v = *reinterpret_cast<const float4 *>(rq + 2 * kd + 4 * (lane >> 3));
            const float beta = lane_val(beta_l, tt), decay = lane_val(decay_l, tt);
            const float qscale = lane_val(qsc_l, 4 * tt), kscale = lane_val(ksc_l, 4 * tt);
            float4 mem{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < R; ++i) {
                st[i] = float4{st[i].x * decay, st[i].y * decay, st[i].z * decay, st[i].w * decay};
                mem.x = fmaf(st[i].x, kv[i], mem.x);
                mem.y = fmaf(st[i].y, kv[i], mem.y);
                mem.z = fmaf(st[i].z, kv[i], mem.z);
                mem.w = fmaf(st[i].w, kv[i], mem.w);
            }
            mem = float4{gsum8(mem.x), gsum8(mem.y), gsum8(mem.z), gsum8(mem.w)};
            if constexpr (NW > 1) {
                if ((lane & 7) == 0) red_m[wv][lane >> 3] = mem;
                __syncthreads();
                mem = red_m[0][lane >> 3];
#pragma unroll
                for (int w = 1; w < NW; ++w) {
                    const float4 p = red_m[w][lane >> 3];
                    mem = float4{mem.x + p.x, mem.y + p.y, mem.z + p.z, mem.w + p.w};
                }
            }
            const float4 upd{(v.x - mem.x * kscale) * beta * kscale, (v.y - mem.y * kscale) * beta * kscale,
                             (v.z - mem.z * kscale) * beta * kscale, (v.w - mem.w * kscale) * beta * kscale};
            float4 o{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < R; ++i) {
                st[i] = float4{fmaf(kv[i], upd.x, st[i].x), fmaf(kv[i], upd.y, st[i].y), fmaf(kv[i], upd.z, st[i].z),
                               fmaf(kv[i], upd.w, st[i].w)};
                o.x = fmaf(st[i].x, qv[i], o.x);
                o.y = fmaf(st[i].y, qv[i], o.y);
                o.z = fmaf(st[i].z, qv[i], o.z);
                o.w = fmaf(st[i].w, qv[i], o.w);
            }
            o = float4{gsum8(o.x), gsum8(o.y), gsum8(o.z), gsum8(o.w)};
            if constexpr (NW > 1) {
                if ((lane & 7) == 0) red_o[wv][lane >> 3] = o;
                __syncthreads();
                o = red_o[0][lane >> 3];
#pragma unroll
                for (int w = 1; w < NW; ++w) {
                    const float4 p = red_o[w][lane >> 3];
                    o = float4{o.x + p.x, o.y + p.y, o.z + p.z, o.w + p.w};
                }
            }
            o = float4{o.x * qscale, o.y * qscale, o.z * qscale, o.w * qscale};
            if (wv == 0 && (lane & 7) == 0 && col_ok) *reinterpret_cast<float4 *>(out + (rr * value_heads + h) * vd + col) = o;
            if (snap != nullptr && t0 + tt + 1 < s.rows && col_ok) {
                float *sn = snap + (static_cast<size_t>(t0 + tt) * value_heads + h) * hstate;
#pragma unroll
                for (int i = 0; i < R; ++i)
                    if (r0 + i < kd) st4(sn + static_cast<size_t>(r0 + i) * vd + col, st[i]);
            }
        }
    }
    if (write_state && col_ok) {
#pragma unroll
        for (int i = 0; i < R; ++i)
            if (r0 + i < kd) st4(S + static_cast<size_t>(r0 + i) * vd + col, st[i]);
    }
}

// ---- host launchers --------------------------------------------------------------------------------------

int launch_rope(float *x, const SegTable &T, int heads, int hd, int rot, double base, hipStream_t s) {
    if (!x) return VQ_ERR_ARG;
    if (heads < 1 || hd < 1 || rot <= 0 || rot % 2 || rot > hd || rot / 2 > kRopeMaxHalf || !(base > 0.0))
        return VQ_ERR_SHAPE;
    rope_kernel<<<T.total, kRopeThreads, 0, s>>>(x, T, heads, hd, rot, base);
    return status_of(hipGetLastError());
}

int launch_kv_append(const float *k, const float *v, void *kc, void *vc, int elem, const SegTable &T, const KvMap &M,
                     int hd, hipStream_t s) {
    if (!k || !v || !kc || !vc || (elem != 2 && elem != 4)) return VQ_ERR_ARG;
    if (M.kv_heads < 1 || hd < 1) return VQ_ERR_SHAPE;
    const bool quad = hd % 4 == 0 && ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15) == 0 &&
                      ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & (elem == 4 ? 15 : 7)) == 0;
    const dim3 grid(T.total);
    if (elem == 2) {
        auto *kh = static_cast<_Float16 *>(kc), *vh = static_cast<_Float16 *>(vc);
        if (quad) kv_append_kernel<_Float16, 4><<<grid, 256, 0, s>>>(k, v, kh, vh, T, M, hd);
        else kv_append_kernel<_Float16, 1><<<grid, 256, 0, s>>>(k, v, kh, vh, T, M, hd);
    } else {
        auto *kf = static_cast<float *>(kc), *vf = static_cast<float *>(vc);
        if (quad) kv_append_kernel<float, 4><<<grid, 256, 0, s>>>(k, v, kf, vf, T, M, hd);
        else kv_append_kernel<float, 1><<<grid, 256, 0, s>>>(k, v, kf, vf, T, M, hd);
    }
    return status_of(hipGetLastError());
}

template <typename C>
bool fa_fast(const C *kc, const C *vc, int hd) {
    return hd % 4 == 0 && ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & (4 * sizeof(C) - 1)) == 0;
}

template <typename C, int HD>
void launch_mfma_hd(bool fast, dim3 grid, hipStream_t s, const float *q, const C *kc, const C *vc, float *out,
                    const SegTable &T, const KvMap &M, int heads, int hd, int bidirectional, int window, int chunks) {
    if (fast)
        attention_mfma_kernel<C, HD, true><<<grid, 256, 0, s>>>(q, kc, vc, out, T, M, heads, hd, bidirectional, window,
                                                               chunks);
    else
        attention_mfma_kernel<C, HD, false><<<grid, 256, 0, s>>>(q, kc, vc, out, T, M, heads, hd, bidirectional, window,
                                                                chunks);
}

template <bool PAGED>
void launch_prompt16(dim3 grid, hipStream_t s, const float *q, const _Float16 *kc, const _Float16 *vc, float *out,
                     const SegTable &T, const KvMap &M, int heads, int hd, int bidirectional, int window, int chunks) {
    if (hd == 64)
        attention_prompt16_kernel<64, PAGED><<<grid, 256, 0, s>>>(q, kc, vc, out, T, M, heads, bidirectional, window, chunks);
    else if (hd == 128)
        attention_prompt16_kernel<128, PAGED><<<grid, 256, 0, s>>>(q, kc, vc, out, T, M, heads, bidirectional, window, chunks);
    else
        attention_prompt16_kernel<256, PAGED><<<grid, 256, 0, s>>>(q, kc, vc, out, T, M, heads, bidirectional, window, chunks);
}

// fp16 caches with hd 64, 128 or 256 and 16-byte aligned q, K, V and out: the f16 MFMA kernels.
bool fa16_ok(const float *q, const void *kc, const void *vc, const float *out, int hd) {
    return (hd == 64 || hd == 128 || hd == 256) &&
           ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc) |
             reinterpret_cast<uintptr_t>(out)) & 15) == 0;
}

template <typename C>
void launch_attention_mfma(const float *q, const C *kc, const C *vc, float *out, const SegTable &T, const KvMap &M,
                           int heads, int hd, int bidirectional, int window, hipStream_t s) {
    int tiles = 0;
    for (int i = 0; i < T.n; ++i) tiles += (T.s[i].rows + 15) / 16;
    const int chunks = (heads / M.kv_heads + 3) / 4;
    const dim3 grid(tiles, M.kv_heads * chunks);
    if constexpr (sizeof(C) == 2) {
        if (fa16_ok(q, kc, vc, out, hd)) {
            if (M.pt != nullptr) launch_prompt16<true>(grid, s, q, kc, vc, out, T, M, heads, hd, bidirectional, window, chunks);
            else launch_prompt16<false>(grid, s, q, kc, vc, out, T, M, heads, hd, bidirectional, window, chunks);
            return;
        }
    }
    const bool fast = fa_fast(kc, vc, hd);
    if (hd <= 64) launch_mfma_hd<C, 64>(fast, grid, s, q, kc, vc, out, T, M, heads, hd, bidirectional, window, chunks);
    else if (hd <= 128) launch_mfma_hd<C, 128>(fast, grid, s, q, kc, vc, out, T, M, heads, hd, bidirectional, window, chunks);
    else launch_mfma_hd<C, 256>(fast, grid, s, q, kc, vc, out, T, M, heads, hd, bidirectional, window, chunks);
}

template <typename C, int HD>
void launch_split_hd(bool fast, dim3 grid, dim3 mgrid, hipStream_t s, const float *q, const C *kc, const C *vc,
                     float *part, float *pml, float *out, const SegTable &T, const KvMap &M, int heads, int hd,
                     int bidirectional, int window, int nch) {
    if (fast)
        attention_split_kernel<C, HD, true><<<grid, 256, 0, s>>>(q, kc, vc, part, pml, T, M, heads, hd, bidirectional,
                                                                window, nch);
    else
        attention_split_kernel<C, HD, false><<<grid, 256, 0, s>>>(q, kc, vc, part, pml, T, M, heads, hd, bidirectional,
                                                                 window, nch);
    attention_merge_kernel<HD><<<mgrid, 256, 0, s>>>(part, pml, out, T, heads, hd, nch);
}


void launch_attention_split16(const float *q, const _Float16 *kc, const _Float16 *vc, float *out, const SegTable &T,
                              const KvMap &M, int heads, int hd, int bidirectional, int window, int span_rows, void *ws,
                              hipStream_t s) {
    const int nch = split16_chunks(T, heads, M.kv_heads, window);
    float *part = static_cast<float *>(ws);
    float *pml = part + static_cast<size_t>(span_rows) * heads * nch * fa_hd(hd);
    const int G = heads / M.kv_heads;
    const dim3 grid(T.n * M.kv_heads * nch, (max_seg_rows(T) * G + 15) / 16);
    auto go = [&](auto paged) {
        constexpr bool P = decltype(paged)::value;
        if (hd == 64)
            attention_split16_kernel<64, P><<<grid, 256, 0, s>>>(q, kc, vc, part, pml, out, T, M, heads, bidirectional, window, nch);
        else if (hd == 128)
            attention_split16_kernel<128, P><<<grid, 256, 0, s>>>(q, kc, vc, part, pml, out, T, M, heads, bidirectional, window, nch);
        else
            attention_split16_kernel<256, P><<<grid, 256, 0, s>>>(q, kc, vc, part, pml, out, T, M, heads, bidirectional, window, nch);
    };
    if (M.pt != nullptr) go(std::true_type{});
    else go(std::false_type{});
    if (nch > 1) {
        const dim3 mgrid(T.total * heads);
        if (hd == 64) attention_merge_kernel<64><<<mgrid, 256, 0, s>>>(part, pml, out, T, heads, hd, nch);
        else if (hd == 128) attention_merge_kernel<128><<<mgrid, 256, 0, s>>>(part, pml, out, T, heads, hd, nch);
        else attention_merge_kernel<256><<<mgrid, 256, 0, s>>>(part, pml, out, T, heads, hd, nch);
    }
}

template <typename C>
void launch_attention_split(const float *q, const C *kc, const C *vc, float *out, const SegTable &T, const KvMap &M,
                            int heads, int hd, int bidirectional, int window, int span_rows, void *ws, hipStream_t s) {
    const int nch = split_chunks(T, M.kv_heads, window);
    const int HD = fa_hd(hd);
    float *part = static_cast<float *>(ws);
    float *pml = part + static_cast<size_t>(span_rows) * heads * nch * HD;
    int max_rows = 0;
    for (int i = 0; i < T.n; ++i) max_rows = T.s[i].rows > max_rows ? T.s[i].rows : max_rows;
    const int G = heads / M.kv_heads;
    const dim3 grid(T.n * M.kv_heads * nch, (max_rows * G + 63) / 64);
    const dim3 mgrid(T.total * heads);
    const bool fast = fa_fast(kc, vc, hd);
    if (HD == 64)
        launch_split_hd<C, 64>(fast, grid, mgrid, s, q, kc, vc, part, pml, out, T, M, heads, hd, bidirectional, window, nch);
    else if (HD == 128)
        launch_split_hd<C, 128>(fast, grid, mgrid, s, q, kc, vc, part, pml, out, T, M, heads, hd, bidirectional, window, nch);
    else
        launch_split_hd<C, 256>(fast, grid, mgrid, s, q, kc, vc, part, pml, out, T, M, heads, hd, bidirectional, window, nch);
}

int launch_attention(const float *q, const void *kc, const void *vc, float *out, int elem, const SegTable &T,
                     const KvMap &M, int heads, int hd, int bidirectional, int window, hipStream_t s,
                     void *ws = nullptr, size_t ws_bytes = 0, int span_rows = 0, bool force_tiled = false) {
    if (!q || !kc || !vc || !out || (elem != 2 && elem != 4)) return VQ_ERR_ARG;
    if (M.kv_heads < 1 || heads < M.kv_heads || heads % M.kv_heads || hd < 1 || hd > kAttnMaxHd || window < 0)
        return VQ_ERR_SHAPE;
    if (ws != nullptr) {  // decode / verify passes with a workspace: the split-context MFMA kernel
        int max_rows = 0;
        for (int i = 0; i < T.n; ++i) max_rows = T.s[i].rows > max_rows ? T.s[i].rows : max_rows;
        if (max_rows <= VQ_ATTN_ROW_MAX) {
            if (ws_bytes < split_ws_bytes(T, span_rows, heads, M.kv_heads, hd, window) ||
                (reinterpret_cast<uintptr_t>(ws) & 15))
                return VQ_ERR_WORKSPACE;
            if (elem == 2 && fa16_ok(q, kc, vc, out, hd))
                launch_attention_split16(q, static_cast<const _Float16 *>(kc), static_cast<const _Float16 *>(vc), out,
                                         T, M, heads, hd, bidirectional, window, span_rows, ws, s);
            else if (elem == 2)
                launch_attention_split(q, static_cast<const _Float16 *>(kc), static_cast<const _Float16 *>(vc), out, T,
                                       M, heads, hd, bidirectional, window, span_rows, ws, s);
            else
                launch_attention_split(q, static_cast<const float *>(kc), static_cast<const float *>(vc), out, T, M,
                                       heads, hd, bidirectional, window, span_rows, ws, s);
            return status_of(hipGetLastError());
        }
    }
    // Passes with a segment of more than VQ_ATTN_ROW_MAX rows (prompt passes): the MFMA kernel reads each K/V
    // tile once per 16 query rows and 4 heads; decode and verify passes: one workgroup per (head, row).
    int max_rows = 0;
    for (int i = 0; i < T.n; ++i) max_rows = T.s[i].rows > max_rows ? T.s[i].rows : max_rows;
    if (max_rows > VQ_ATTN_ROW_MAX || force_tiled) {
        if (elem == 2)
            launch_attention_mfma(q, static_cast<const _Float16 *>(kc), static_cast<const _Float16 *>(vc), out, T, M,
                                  heads, hd, bidirectional, window, s);
        else
            launch_attention_mfma(q, static_cast<const float *>(kc), static_cast<const float *>(vc), out, T, M, heads,
                                  hd, bidirectional, window, s);
        return status_of(hipGetLastError());
    }
    const dim3 grid(heads, T.total);
    if (elem == 2)
        attention_kernel<_Float16><<<grid, 64 * kAttnWaves, 0, s>>>(q, static_cast<const _Float16 *>(kc),
                                                                    static_cast<const _Float16 *>(vc), out, T, M, heads,
                                                                    hd, bidirectional, window);
    else
        attention_kernel<float><<<grid, 64 * kAttnWaves, 0, s>>>(q, static_cast<const float *>(kc),
                                                                 static_cast<const float *>(vc), out, T, M, heads, hd,
                                                                 bidirectional, window);
    return status_of(hipGetLastError());
}

int launch_conv_update(const float *x, float *state, const float *w, float *out, int channels, int K,
                       const SegTable &T, float *snap, int write_state, hipStream_t s) {
    if (!x || !state || !w || !out) return VQ_ERR_ARG;
    if (channels < 1 || K < 1 || K > VQ_CONV_MAX_K) return VQ_ERR_SHAPE;
    if (snap != nullptr && T.n != 1) return VQ_ERR_ARG;
    const dim3 grid((channels + 255) / 256, T.n);
    switch (K) {
#define VQ_CONV_CASE(KK) \
    case KK: conv_update_kernel<KK><<<grid, 256, 0, s>>>(x, state, w, out, channels, T, snap, write_state); break;
        VQ_CONV_CASE(1) VQ_CONV_CASE(2) VQ_CONV_CASE(3) VQ_CONV_CASE(4)
        VQ_CONV_CASE(5) VQ_CONV_CASE(6) VQ_CONV_CASE(7) VQ_CONV_CASE(8)
#undef VQ_CONV_CASE
    }
    return status_of(hipGetLastError());
}

template <typename ST>
void gd_dispatch(int R, dim3 grid, hipStream_t s, const float *conv, const float *b, const float *a, const float *ssm_a,
                 const float *dt, ST *state, float *out, int kh, int vh, int kd, int vd, float eps, int head_order,
                 const SegTable &T, float *snap, int write_state) {
#define VQ_GD_CASE(RR)                                                                                              \
    case RR:                                                                                                        \
        gated_delta_kernel<RR, ST><<<grid, 256, 0, s>>>(conv, b, a, ssm_a, dt, state, out, kh, vh, kd, vd, eps,      \
                                                        head_order, T, snap, write_state);                         \
        break;
    switch (R) { VQ_GD_CASE(4) VQ_GD_CASE(8) VQ_GD_CASE(16) VQ_GD_CASE(32) }
#undef VQ_GD_CASE
}

template <typename ST>
void gd4_dispatch(int R, dim3 grid, hipStream_t s, const float *conv, const float *b, const float *a, const float *ssm_a,
                  const float *dt, ST *state, float *out, int kh, int vh, int kd, int vd, float eps, int head_order,
                  const SegTable &T, float *snap, int write_state) {
    int rows = 1;
    for (int i = 0; i < T.n; ++i) rows = T.s[i].rows > rows ? T.s[i].rows : rows;
    const int tc = rows < kGdChunk ? rows : kGdChunk;
#define VQ_GD_CASE(RR)                                                                                              \
    case RR:                                                                                                        \
        if (kd == 8 * RR)                                                                                           \
            gated_delta4_kernel<RR, ST, true><<<grid, 64, gd_lds_bytes(kd, tc), s>>>(                                \
                conv, b, a, ssm_a, dt, state, out, kh, vh, kd, vd, eps, head_order, T, snap, write_state, tc);      \
        else                                                                                                        \
            gated_delta4_kernel<RR, ST, false><<<grid, 64, gd_lds_bytes(kd, tc), s>>>(                               \
                conv, b, a, ssm_a, dt, state, out, kh, vh, kd, vd, eps, head_order, T, snap, write_state, tc);      \
        break;
    if (kd == 128 || kd == 256) {  // kGdWaves waves per column tile, each 8 R rows: FULL
        const dim3 block(64 * kGdWaves);
        if (kd == 128)
            gated_delta4_kernel<128 / (8 * kGdWaves), ST, true, kGdWaves><<<grid, block, gd_lds_bytes(kd, tc), s>>>(
                conv, b, a, ssm_a, dt, state, out, kh, vh, kd, vd, eps, head_order, T, snap, write_state, tc);
        else
            gated_delta4_kernel<256 / (8 * kGdWaves), ST, true, kGdWaves><<<grid, block, gd_lds_bytes(kd, tc), s>>>(
                conv, b, a, ssm_a, dt, state, out, kh, vh, kd, vd, eps, head_order, T, snap, write_state, tc);
        return;
    }
    switch (R) { VQ_GD_CASE(4) VQ_GD_CASE(8) VQ_GD_CASE(16) VQ_GD_CASE(32) }
#undef VQ_GD_CASE
}

int launch_gated_delta(const float *conv, const float *b, const float *a, const float *ssm_a, const float *dt,
                       void *state, int state_elem, float *out, int kh, int vh, int kd, int vd, float eps,
                       int head_order, const SegTable &T, float *snap, int write_state, hipStream_t s) {
    if (!conv || !b || !a || !ssm_a || !dt || !state || !out || (state_elem != 4 && state_elem != 2)) return VQ_ERR_ARG;
    if (kh < 1 || vh < kh || vh % kh || kd < 1 || kd > kGdMaxKd || vd < 1 || (head_order != 0 && head_order != 1) ||
        !(eps >= 0.0f))
        return VQ_ERR_SHAPE;
    if (snap != nullptr && (T.n != 1 || state_elem != 4)) return VQ_ERR_ARG;
    const int R = kd <= 4 * kGdGroups ? 4 : kd <= 8 * kGdGroups ? 8 : kd <= 16 * kGdGroups ? 16 : 32;
    const uintptr_t align = reinterpret_cast<uintptr_t>(state) | reinterpret_cast<uintptr_t>(conv) |
                            reinterpret_cast<uintptr_t>(out) | (snap ? reinterpret_cast<uintptr_t>(snap) : 0);
    int max_rows = 1;
    for (int i = 0; i < T.n; ++i) max_rows = T.s[i].rows > max_rows ? T.s[i].rows : max_rows;
    const double seg_bytes = static_cast<double>(max_rows) * (2.0 * kh * kd + static_cast<double>(vh) * vd) * 4.0;
    // Column quads: every row offset stays 16-byte aligned; a segment's inputs within 32-bit DMA offsets.
    if (vd % 4 == 0 && kd % 4 == 0 && (align & 15) == 0 && seg_bytes < 4.0e9) {
        const dim3 grid(static_cast<unsigned>(vh * ((vd + 31) / 32)), T.n);
        if (state_elem == 4)
            gd4_dispatch<float>(R, grid, s, conv, b, a, ssm_a, dt, static_cast<float *>(state), out, kh, vh, kd, vd,
                                eps, head_order, T, snap, write_state);
        else
            gd4_dispatch<_Float16>(R, grid, s, conv, b, a, ssm_a, dt, static_cast<_Float16 *>(state), out, kh, vh, kd,
                                   vd, eps, head_order, T, snap, write_state);
        return status_of(hipGetLastError());
    }
    const long waves = static_cast<long>(vh) * ((vd + kGdCols - 1) / kGdCols);
    const dim3 grid(static_cast<unsigned>((waves + 3) / 4), T.n);
    if (state_elem == 4)
        gd_dispatch<float>(R, grid, s, conv, b, a, ssm_a, dt, static_cast<float *>(state), out, kh, vh, kd, vd, eps,
                           head_order, T, snap, write_state);
    else
        gd_dispatch<_Float16>(R, grid, s, conv, b, a, ssm_a, dt, static_cast<_Float16 *>(state), out, kh, vh, kd, vd,
                              eps, head_order, T, snap, write_state);
    return status_of(hipGetLastError());
}

KvMap paged(const int32_t *pt, int page_size, int pps, int kv_heads) { return KvMap{pt, 0, page_size, pps, kv_heads}; }
KvMap contiguous(int max_seq, int kv_heads) { return KvMap{nullptr, max_seq, 1, 1, kv_heads}; }

int check_paging(const int32_t *pt, int page_size, int pps, const SegTable &T) {
    if (pt == nullptr) return VQ_ERR_ARG;
    if (page_size < 1 || pps < 1) return VQ_ERR_SHAPE;
    for (int i = 0; i < T.n; ++i)
        if (static_cast<long>(T.s[i].pos0) + T.s[i].rows > static_cast<long>(page_size) * pps) return VQ_ERR_SHAPE;
    return VQ_OK;
}

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
    hipStream_t s = static_cast<hipStream_t>(stream);
    const long n = static_cast<long>(heads) * hd;
    if (hd % 4 == 0 && ((reinterpret_cast<uintptr_t>(raw) | reinterpret_cast<uintptr_t>(q) |
                         reinterpret_cast<uintptr_t>(gate)) & 15) == 0) {
        const long nq = n / 4;
        split_gated_q4_kernel<<<static_cast<unsigned>((nq + 255) / 256), 256, 0, s>>>(
            reinterpret_cast<const float4 *>(raw), reinterpret_cast<float4 *>(q), reinterpret_cast<float4 *>(gate),
            hd / 4, nq);
    } else {
        split_gated_q1_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(raw, q, gate, hd, n);
    }
    return status_of(hipGetLastError());
}

int vq_concat_rows(float *dst, const float *a, const float *b, int rows, int width, void *stream) {
    if (!dst || !a || !b) return VQ_ERR_ARG;
    if (rows < 0 || width < 0) return VQ_ERR_SHAPE;
    const long n = 2L * rows * width;
    if (n == 0) return VQ_OK;
    concat_rows_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        dst, a, b, width, n);
    return status_of(hipGetLastError());
}

int vq_zero(void *p, size_t nbytes, void *stream) {
    if (!p && nbytes) return VQ_ERR_ARG;
    if (nbytes == 0) return VQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto *b = static_cast<uint8_t *>(p);
    // Unaligned head and tail bytes, aligned words between.
    const size_t head = (4 - (reinterpret_cast<uintptr_t>(b) & 3)) & 3;
    if (nbytes <= head + 3) {
        zero_bytes_kernel<<<1, 64, 0, s>>>(b, static_cast<int>(nbytes));
        return status_of(hipGetLastError());
    }
    if (head) zero_bytes_kernel<<<1, 64, 0, s>>>(b, static_cast<int>(head));
    const size_t words = (nbytes - head) / 4, tail = (nbytes - head) % 4;
    const long blocks = static_cast<long>((words + 255) / 256);
    zero_kernel<<<static_cast<unsigned>(blocks < 4096 ? blocks : 4096), 256, 0, s>>>(
        reinterpret_cast<uint32_t *>(b + head), static_cast<long>(words));
    if (tail) zero_bytes_kernel<<<1, 64, 0, s>>>(b + head + 4 * words, static_cast<int>(tail));
    return status_of(hipGetLastError());
}

int vq_rope(float *x, int ntok, int heads, int hd, int rot, int pos0, double base, void *stream) {
    if (ntok < 1 || pos0 < 0) return VQ_ERR_SHAPE;
    return launch_rope(x, one_segment(pos0, ntok), heads, hd, rot, base, static_cast<hipStream_t>(stream));
}

int vq_rope_seg(float *x, const int32_t *segs, int nseg, int heads, int hd, int rot, double base, void *stream) {
    SegTable T;
    const int st = make_table(segs, nseg, T, nullptr);
    return st != VQ_OK ? st : launch_rope(x, T, heads, hd, rot, base, static_cast<hipStream_t>(stream));
}

int vq_kv_append(const float *k, const float *v, void *kc, void *vc, int elem, int ntok, int kv_heads, int max_seq,
                 int hd, int pos0, void *stream) {
    if (ntok < 1 || kv_heads < 1 || pos0 < 0 || pos0 + ntok > max_seq) return VQ_ERR_SHAPE;
    return launch_kv_append(k, v, kc, vc, elem, one_segment(pos0, ntok), contiguous(max_seq, kv_heads), hd,
                            static_cast<hipStream_t>(stream));
}

int vq_kv_append_seg(const float *k, const float *v, void *kc, void *vc, int elem, const int32_t *segs, int nseg,
                     int kv_heads, int hd, const int32_t *page_table, int page_size, int pages_per_seq, void *stream) {
    SegTable T;
    int st = make_table(segs, nseg, T, nullptr);
    if (st == VQ_OK) st = check_paging(page_table, page_size, pages_per_seq, T);
    if (st != VQ_OK) return st;
    return launch_kv_append(k, v, kc, vc, elem, T, paged(page_table, page_size, pages_per_seq, kv_heads), hd,
                            static_cast<hipStream_t>(stream));
}

int vq_attention(const float *q, const void *kc, const void *vc, float *out, int elem, int heads, int kv_heads, int hd,
                 int max_seq, int seq_len, int ntok, int bidirectional, int window, void *stream) {
    if (kv_heads < 1 || ntok < 1 || seq_len < 1 || seq_len + ntok - 1 > max_seq) return VQ_ERR_SHAPE;
    return launch_attention(q, kc, vc, out, elem, one_segment(seq_len - 1, ntok), contiguous(max_seq, kv_heads), heads,
                            hd, bidirectional, window, static_cast<hipStream_t>(stream));
}

int vq_attention_seg(const float *q, const void *kc, const void *vc, float *out, int elem, const int32_t *segs,
                     int nseg, int heads, int kv_heads, int hd, const int32_t *page_table, int page_size,
                     int pages_per_seq, void *stream) {
    SegTable T;
    int st = make_table(segs, nseg, T, nullptr);
    if (st == VQ_OK) st = check_paging(page_table, page_size, pages_per_seq, T);
    if (st != VQ_OK) return st;
    if (kv_heads < 1) return VQ_ERR_SHAPE;
    return launch_attention(q, kc, vc, out, elem, T, paged(page_table, page_size, pages_per_seq, kv_heads), heads, hd,
                            0, 0, static_cast<hipStream_t>(stream));
}

size_t vq_attention_workspace_bytes(int heads, int kv_heads, int hd, int seq_len, int ntok, int window) {
    if (kv_heads < 1 || heads < kv_heads || heads % kv_heads || hd < 1 || hd > kAttnMaxHd || ntok < 1 || seq_len < 1 ||
        window < 0)
        return 0;
    if (ntok > VQ_ATTN_ROW_MAX) return 0;
    return split_ws_bytes(one_segment(seq_len - 1, ntok), ntok, heads, kv_heads, hd, window);
}

int vq_attention_ws(const float *q, const void *kc, const void *vc, float *out, int elem, int heads, int kv_heads,
                    int hd, int max_seq, int seq_len, int ntok, int bidirectional, int window, void *workspace,
                    size_t workspace_bytes, void *stream) {
    if (kv_heads < 1 || ntok < 1 || seq_len < 1 || seq_len + ntok - 1 > max_seq) return VQ_ERR_SHAPE;
    return launch_attention(q, kc, vc, out, elem, one_segment(seq_len - 1, ntok), contiguous(max_seq, kv_heads), heads,
                            hd, bidirectional, window, static_cast<hipStream_t>(stream), workspace, workspace_bytes,
                            ntok);
}

size_t vq_attention_seg_workspace_bytes(const int32_t *segs, int nseg, int heads, int kv_heads, int hd) {
    SegTable T;
    int span = 0;
    if (make_table(segs, nseg, T, &span) != VQ_OK) return 0;
    if (kv_heads < 1 || heads < kv_heads || heads % kv_heads || hd < 1 || hd > kAttnMaxHd) return 0;
    for (int i = 0; i < T.n; ++i)
        if (T.s[i].rows > VQ_ATTN_ROW_MAX) return 0;
    return split_ws_bytes(T, span, heads, kv_heads, hd, 0);
}

int vq_attention_seg_ws(const float *q, const void *kc, const void *vc, float *out, int elem, const int32_t *segs,
                        int nseg, int heads, int kv_heads, int hd, const int32_t *page_table, int page_size,
                        int pages_per_seq, void *workspace, size_t workspace_bytes, void *stream) {
    SegTable T;
    int span = 0;
    int st = make_table(segs, nseg, T, &span);
    if (st == VQ_OK) st = check_paging(page_table, page_size, pages_per_seq, T);
    if (st != VQ_OK) return st;
    if (kv_heads < 1) return VQ_ERR_SHAPE;
    return launch_attention(q, kc, vc, out, elem, T, paged(page_table, page_size, pages_per_seq, kv_heads), heads, hd,
                            0, 0, static_cast<hipStream_t>(stream), workspace, workspace_bytes, span);
}

int vq_attention_tiled(const float *q, const void *kc, const void *vc, float *out, int elem, int heads, int kv_heads,
                       int hd, int max_seq, int seq_len, int ntok, int bidirectional, int window, void *stream) {
    if (kv_heads < 1 || ntok < 1 || seq_len < 1 || seq_len + ntok - 1 > max_seq) return VQ_ERR_SHAPE;
    return launch_attention(q, kc, vc, out, elem, one_segment(seq_len - 1, ntok), contiguous(max_seq, kv_heads), heads,
                            hd, bidirectional, window, static_cast<hipStream_t>(stream), nullptr, 0, 0, true);
}

int vq_attention_seg_tiled(const float *q, const void *kc, const void *vc, float *out, int elem, const int32_t *segs,
                           int nseg, int heads, int kv_heads, int hd, const int32_t *page_table, int page_size,
                           int pages_per_seq, void *stream) {
    SegTable T;
    int st = make_table(segs, nseg, T, nullptr);
    if (st == VQ_OK) st = check_paging(page_table, page_size, pages_per_seq, T);
    if (st != VQ_OK) return st;
    if (kv_heads < 1) return VQ_ERR_SHAPE;
    return launch_attention(q, kc, vc, out, elem, T, paged(page_table, page_size, pages_per_seq, kv_heads), heads, hd,
                            0, 0, static_cast<hipStream_t>(stream), nullptr, 0, 0, true);
}

int vq_conv_update(const float *x, float *state, const float *w, float *out, int channels, int K, int ntok, float *snap,
                   int write_state, void *stream) {
    if (ntok < 1) return VQ_ERR_SHAPE;
    return launch_conv_update(x, state, w, out, channels, K, one_segment(0, ntok), snap, write_state,
                              static_cast<hipStream_t>(stream));
}

int vq_conv_update_seg(const float *x, float *state, const float *w, float *out, int channels, int K,
                       const int32_t *segs, int nseg, float *snap, int write_state, void *stream) {
    SegTable T;
    const int st = make_table(segs, nseg, T, nullptr);
    return st != VQ_OK ? st
                       : launch_conv_update(x, state, w, out, channels, K, T, snap, write_state,
                                            static_cast<hipStream_t>(stream));
}

int vq_gated_delta(const float *conv, const float *b, const float *a, const float *ssm_a, const float *dt, void *state,
                   int state_elem, float *out, int key_heads, int value_heads, int kd, int vd, float eps,
                   int head_order, int ntok, float *snap, int write_state, void *stream) {
    if (ntok < 1) return VQ_ERR_SHAPE;
    return launch_gated_delta(conv, b, a, ssm_a, dt, state, state_elem, out, key_heads, value_heads, kd, vd, eps,
                              head_order, one_segment(0, ntok), snap, write_state, static_cast<hipStream_t>(stream));
}

int vq_gated_delta_seg(const float *conv, const float *b, const float *a, const float *ssm_a, const float *dt,
                       void *state, int state_elem, float *out, int key_heads, int value_heads, int kd, int vd,
                       float eps, int head_order, const int32_t *segs, int nseg, float *snap, int write_state,
                       void *stream) {
    SegTable T;
    const int st = make_table(segs, nseg, T, nullptr);
    return st != VQ_OK ? st
                       : launch_gated_delta(conv, b, a, ssm_a, dt, state, state_elem, out, key_heads, value_heads, kd,
                                            vd, eps, head_order, T, snap, write_state, static_cast<hipStream_t>(stream));
}

}  // extern "C"
