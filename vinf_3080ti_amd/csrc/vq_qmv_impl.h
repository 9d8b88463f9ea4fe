// vq_qmv_impl.h -- quantized matvec kernels, templated on the GGUF type (one translation unit per type
// instantiates them: vq_t_<type>.hip). Hand-written for CDNA4 (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "vq_qmv.h"
#include "vq_quant.h"
#include "vq_tables.h"

namespace vq {

// Streaming geometry (compile-time; overridable for tuning builds).


// Sum over the 64 lanes with DPP moves (no LDS round trips): pairs, quads, half rows, rows, then rows 1/3
// take row 0/2 (row_bcast:15) and rows 2/3 take lane 31 (row_bcast:31); lane 63 ends with the total.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}
// x in the lanes whose bit of the wave-uniform mask m is set, 0 elsewhere: one v_cndmask on the SGPR pair. Inline
// asm on purpose: written as a select, hipcc turns it into an exec-masked branch around the DPP move that produces
// x, and a DPP move under a partial exec reads 0 from the disabled source lanes.
// The same with bound_ctrl: lanes without a source read 0 (no zeroed old operand needed).
template <int CTRL>
__device__ __forceinline__ float dpp_fz(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float keep_lanes(float x, uint64_t m) {
    float r;
    asm("v_cndmask_b32_e64 %0, 0, %1, %2" : "=v"(r) : "v"(x), "s"(m));
    return r;
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);        // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);        // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);       // row_half_mirror
    v += dpp_f<0x140>(v);       // row_mirror
    v += dpp_f<0x142, 0xA>(v);  // row_bcast:15
    v += dpp_f<0x143, 0xC>(v);  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Per-type stage shape: LPU lanes decode one unit (each takes SPB/LPU of its slices), so a stage is the
// SU = 64/LPU consecutive units of a workgroup's byte range, about 2-7 KB: a wave holds one stage of raw
// bytes in VGPRs while it decodes the previous one.
template <int T>
struct StageShape {
    static constexpr int LPU_DEFAULT =
        (T == VQ_Q8_0 || T == VQ_IQ4_NL || T == VQ_IQ2_XXS || T == VQ_IQ2_XS || T == VQ_IQ2_S || T == VQ_Q3_K) ? 1 : 2;
    static constexpr int LPU = LPU_DEFAULT;
};

// LDS image of the activation records: per token, the int8 codes in blocks of 256 followed by kXPad = 16 bytes
// of padding, then the group scales xd and the half sums xh as in the packed record. Built by DMA from a packed
// record, or by quantizing fp32 activations in the kernel. The pad sets the stride between neighbouring units'
// codes to 68 dwords, so the 16 lanes of one pass of a 16-byte LDS read cover the 64 banks once (with 32 bytes,
// 72 dwords, lanes l and l + 8 shared banks: 2.43 M conflict cycles per Q3_K gate+up launch against 1.73 M, and
// 20.2 against 19.0 µs).
struct XImage {
    int ng, nblk, xq_bytes, bytes;  // bytes: one token's image (16-byte multiple)
    __host__ __device__ explicit XImage(int cols)
        : ng(cols / 32), nblk((cols / 32 + 7) / 8), xq_bytes(((cols / 32 + 7) / 8) * (256 + kXPad)),
          bytes(x_image_bytes(cols)) {}
    __device__ int code_off(int G, int h) const { return __mul24(G >> 3, 256 + kXPad) + (G & 7) * 32 + 16 * h; }
    // Byte of the packed record (vq_xpack_h_offset layout) that LDS image byte o (16-byte aligned) holds,
    // or -1 for padding.
    __device__ int src_of(int o, int cols) const {
        if (o < xq_bytes) {
            const int blk = o / (256 + kXPad), w = o - blk * (256 + kXPad);
            return w < 256 && blk * 256 + w < cols ? blk * 256 + w : -1;
        }
        return cols + (o - xq_bytes);
    }
};

// Waves per workgroup: preferably one 16-wave workgroup per CU for one token, 8 waves for several (their
// activation image takes the LDS that more stage buffers would need); 4 when the image is too wide for that.
template <int NT>
constexpr int wg_waves() {
    return NT == 1 ? 16 : 8;
}
constexpr int kFallbackWaves = 4;

template <int T>
struct Stream {
    using S = Sl<T>;
    static constexpr int LPU = StageShape<T>::LPU;
    static constexpr int SPL = S::SPB / LPU;  // slices per lane
    static constexpr int SU = 64 / LPU;       // units per stage
    // 16-byte chunks one stage's bytes can touch (its units plus the dword the decoders may read past the
    // last unit, from an arbitrary 16-byte phase) and the dwordx4 loads per lane that cover them.
    static constexpr int CMAX = (SU * S::UB + 4 + 15) / 16 + 1;
    static constexpr int NL = (CMAX + 63) / 64;
    static constexpr int STAGE_LDS = NL * 1024;  // one wave's stage buffer
    static_assert(S::SPB % LPU == 0 && NL >= 1 && NL <= 16, "stage geometry");
};

// Partial row sums of one workgroup, at most this many fp32 floats. Two layouts: [stage][lane][token] (one
// part per lane, no reduction inside a stage) when the workgroup's stages fit, else [stage][row of the
// stage][token] (a segmented scan over the lanes gives each row's part of the stage).
constexpr int kSlotFloats = 4096;
// Rows a stage of SU consecutive units can touch when rows have nu units.
__host__ __device__ constexpr int rows_per_stage(int su, int nu) { return (su - 1) / nu + 2; }
// Whether a job of rwg rows per workgroup uses the per-lane layout (one value for the whole job; one token
// only: at several tokens the extra registers of both reductions cost more than the scan).
__host__ __device__ constexpr bool lane_slots(long rwg, int nu, int su, int nt) {
    return nt == 1 && (rwg * nu + su - 1) / su * 64 <= kSlotFloats;
}

// Launches of at most this many tokens of a kSignedGrid type read the pre-signed table (32 KB of LDS; wider
// activation images leave no room for it).
constexpr int kSignedGridMaxTok = 2;
template <int T, int NT>
constexpr bool use_signed_grid() {
    return kSignedGrid<T> && NT <= kSignedGridMaxTok;
}
template <int T, int NT>
constexpr int grid_table_bytes() {
    if constexpr (use_signed_grid<T, NT>()) return 512 * 16 * 4;
    return TabSpec<T>::n8 * 8 + TabSpec<T>::n4 * 4;
}
template <int T, int NT>
__device__ __forceinline__ const uint8_t *grid_table_src() {
    if constexpr (use_signed_grid<T, NT>()) return reinterpret_cast<const uint8_t *>(g_iq3s_sg.v);
    if constexpr (T == VQ_IQ2_XXS) return reinterpret_cast<const uint8_t *>(g_iq2xxs.v);
    if constexpr (T == VQ_IQ2_XS) return reinterpret_cast<const uint8_t *>(g_iq2xs.v);
    if constexpr (T == VQ_IQ2_S) return reinterpret_cast<const uint8_t *>(g_iq2s.v);
    if constexpr (T == VQ_IQ3_XXS) return reinterpret_cast<const uint8_t *>(g_iq3xxs.v);
    if constexpr (T == VQ_IQ3_S) return reinterpret_cast<const uint8_t *>(g_iq3s.v);
    return nullptr;
}

// One launch covers up to kMaxJobs matrices of the same type and width that share the activations (a
// layer's gate/up, q/k/v, ...). Each job's rows are cut into ranges of `rwg` rows, one per workgroup; job j
// owns the workgroups [b0, b0 + ceil(rows / rwg)).
constexpr int kMaxJobs = 4;
struct QJob {
    const uint8_t *w;
    float *y;  // [NT][rows], or null (argmax only)
    int rows, b0;
    int rwg;    // rows per workgroup
    int type;   // GGUF type (a launch may mix its main type with one other, see qmv_stream_kernel)
};
struct QJobs {
    QJob j[kMaxJobs];
    int n;
    int blocks;   // workgroups of the launch
    unsigned long long *amax;  // null, or [NT][blocks] per-workgroup argmax keys (see argmax_key)
};

// Argmax key of a value at row r: larger key = larger value, then lower row. NaN and -inf never win (the
// reference kernel starts from -inf and takes strictly greater values); 0 = no candidate.
__device__ __forceinline__ unsigned long long argmax_key(float v, long r) {
    const uint32_t u = __float_as_uint(v);
    if (v != v || v == -__builtin_huge_valf()) return 0ull;
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(o) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(r));
}

// Timing builds only (-DVQ_STAMPS, never in the shipped library): per-workgroup s_memrealtime stamps, kept in LDS
// until the end (global stores would add to the vmcnt waits the kernel makes) and written out by thread 0 then.
#ifdef VQ_STAMPS
static __device__ unsigned long long g_stamps[8192 * 8];
#define VQ_STAMP_IF(cond, slot)                                                                                \
    do {                                                                                                       \
        if (cond) s_stamp[slot] = __builtin_amdgcn_s_memrealtime();                                            \
    } while (0)
#define VQ_STAMP(slot) VQ_STAMP_IF(threadIdx.x == 0, slot)
#define VQ_STAMP_FLUSH()                                                                                       \
    do {                                                                                                       \
        __syncthreads();                                                                                       \
        if (threadIdx.x < 8) g_stamps[blockIdx.x * 8 + threadIdx.x] = s_stamp[threadIdx.x];                    \
    } while (0)
#define VQ_STAMP_READER(NAME)                                                                                  \
    extern "C" int NAME(void *dst, size_t bytes) {                                                             \
        return static_cast<int>(hipMemcpyFromSymbol(dst, HIP_SYMBOL(vq::g_stamps), bytes, 0, hipMemcpyDeviceToHost)); \
    }
#else
#define VQ_STAMP_IF(cond, slot)
#define VQ_STAMP(slot)
#define VQ_STAMP_FLUSH()
#define VQ_STAMP_READER(NAME)
#endif

// Quantized matvec: y[t][r] = W[r] . x[t] for t < NT.
//
// Workgroup b owns a contiguous range of rows of one job -- a contiguous byte range, since rows are back to
// back and each is a whole number of units (32-element groups for Q8_0/IQ4_NL, 256-element super-blocks
// otherwise) -- cut into stages of SU = 64/LPU units. Its waves take stages from an LDS counter: wave w starts
// with stage w, and each further stage is handed out when a wave asks, so waves that the memory system
// serves faster take more stages and the workgroup's waves finish together (with static shares they finished
// up to 3 us apart within a CU, measured on MI355X). A stage's bytes (16-byte chunks [c0, c1)) arrive in VGPRs
// by NL coalesced nontemporal dwordx4 loads per lane, one stage ahead: a wave requests its next stage before
// it decodes the current one. The landed stage goes to the wave's LDS stage buffer (lane order = byte order)
// and the LPU lanes of each unit decode its slices with the type's slice decoders (weights, activations and
// IQ tables all read from LDS), so the block header is decoded once per 256/LPU elements. A segmented scan
// over the lanes gives each row's part in the stage, kept in an LDS slot per (stage, row); after a barrier the
// workgroup adds each row's parts in stage order and writes y. Which wave decodes a stage does not change any
// sum: results are deterministic.
//
// LDS: [grid table | activation image of the NT tokens | stage buffer per wave | row-part slots]. At start-up
// the waves load the table and the activations (DMA of the packed record, or quantization of fp32 values),
// then request their first stage, and meet at one barrier.
template <int T, int NT, bool XF32, int NW, bool STG = false>
__device__ __forceinline__ void stream_wg(const QJobs &jobs, const int jb, const int cols, const void *__restrict__ xin,
                                          const XStage &xst) {
    using S = Sl<T>;
    using G = Stream<T>;
    constexpr int NP = S::NP, UB = S::UB, LPU = G::LPU, SU = G::SU, NL = G::NL;
    constexpr int TB = grid_table_bytes<T, NT>();
    constexpr bool SG = use_signed_grid<T, NT>();
    extern __shared__ __attribute__((aligned(1024))) uint8_t s_dyn[];
    __shared__ __attribute__((aligned(1024))) uint8_t s_grid[TB > 0 ? TB : 16];
    __shared__ uint2 sks[TabSpec<T>::ks ? 128 : 1];
    __shared__ uint2 ssm[TabSpec<T>::sm ? 256 : 1];
    __shared__ int s_next;                        // next stage to hand out
    __shared__ unsigned long long s_best[NT][NW];  // argmax reduction

#ifdef VQ_STAMPS
    __shared__ unsigned long long s_stamp[8];
#endif
    VQ_STAMP(0);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int nu = (cols >> 5) / S::UG;
    const int xb = vq_xpack_stride(cols);
    const XImage xi(cols);
    const int xreg = (NT * xi.bytes + 1023) & ~1023;
    uint8_t *const sbuf = s_dyn + xreg + wv * G::STAGE_LDS;
    float *const slots = reinterpret_cast<float *>(s_dyn + xreg + NW * G::STAGE_LDS);
    const int rs = rows_per_stage(SU, nu);
    const bool per_lane = lane_slots(jobs.j[jb].rwg, nu, SU, NT);
    const bool add = STG && (xst.flags & VQ_STAGE_ADD) != 0 && jobs.j[jb].y != nullptr;

    // This workgroup's rows and stages (all 32-bit unit indices: a matrix has < 2^31 units).
    const int b = blockIdx.x;
    const uint8_t *const w = jobs.j[jb].w;
    float *const y = jobs.j[jb].y;
    const int rows = jobs.j[jb].rows, rwg = jobs.j[jb].rwg;
    const int R0 = (b - jobs.j[jb].b0) * rwg;
    const int R1 = R0 + rwg < rows ? R0 + rwg : rows;
    const int U0 = R0 * nu, U1 = R1 * nu;
    const int nst = R0 < rows ? (U1 - U0 + SU - 1) / SU : 0;
    // Stage s: 16-byte chunks [c0, c1) with c0 the one holding its first byte and c1 past the one holding the
    // dword after its last unit -- but never past the one holding the matrix's last byte (the weight buffer
    // has 16 readable pad bytes; decoders discard bytes past a block). Lanes past c1 re-read c1 - 1
    // (addresses a lane that does load it also reads: no extra traffic), so every stage issues exactly NL
    // loads.
    const long mend = static_cast<long>(rows) * nu * UB;
    auto load_stage = [&](int s, u32x4 (&R)[NL]) {
        const long ua = U0 + static_cast<long>(s) * SU;
        const long ub = ua + SU < U1 ? ua + SU : U1;
        const long e = ub * UB + 4 < mend ? ub * UB + 4 : mend;
        const long c0 = (ua * UB) >> 4, cl = ((e + 15) >> 4) - 1;
        // Wave-uniform base and limit; per-lane 32-bit chunk offsets.
        const u32x4 *const base = reinterpret_cast<const u32x4 *>(w) + c0;
        const long d = cl - c0;
        const unsigned lim = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(d > 0 ? d : 0)));
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const unsigned c = static_cast<unsigned>(lane + 64 * i);
            R[i] = __builtin_nontemporal_load(base + (c < lim ? c : lim));
        }
    };
    auto store_stage = [&](const u32x4 (&R)[NL]) {
#pragma unroll
        for (int i = 0; i < NL; ++i) reinterpret_cast<u32x4 *>(sbuf)[lane + 64 * i] = R[i];
    };

    // Start-up: table pieces and activations first, alone (waiting for them then waits behind no weight
    // traffic), then the first stage.
    int s = wv < nst ? wv : -1;
    u32x4 RA[NL];
    if constexpr (TB > 0) {
        const uint8_t *src = grid_table_src<T, NT>();
        for (int p = wv; p < TB / 1024; p += NW) dma16(src + p * 1024, lane * 16, s_grid + p * 1024);
    }
    if constexpr (XF32) {
        const float *xf = static_cast<const float *>(xin);
        const bool silu = (xst.flags & VQ_STAGE_SILU_MUL) != 0, norm = (xst.flags & VQ_STAGE_NORM) != 0;
        // Staged activation element i of token t: silu(x) * x2 with SILU_MUL, times rms * nw[i] with NORM
        // (qwen_megakernel.cu:485-551). The RMS sums of squares use the stage buffers, free until the first
        // stage lands: partial[t][k] over groups g = k mod 256 in order, then a fixed pairwise tree.
        float *const nsum = reinterpret_cast<float *>(s_dyn + xreg);
        auto staged = [&](int t, int g, float (&v)[32]) {
            const float4 *src = reinterpret_cast<const float4 *>(xf + static_cast<size_t>(t) * cols + 32 * g);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float4 f = src[k];
                v[4 * k] = f.x;
                v[4 * k + 1] = f.y;
                v[4 * k + 2] = f.z;
                v[4 * k + 3] = f.w;
            }
            if (silu) {
                const float4 *s2 = reinterpret_cast<const float4 *>(xst.x2 + static_cast<size_t>(t) * cols + 32 * g);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 f = s2[k];
                    const float m[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        // silu(z) = z / (1 + e^-z) with the hardware exp2 and reciprocal (~1 ulp each;
                        // v_exp_f32 flushes to 0 / inf at the ends, where silu is 0 or z)
                        const float z = v[4 * k + q];
                        const float e = __builtin_amdgcn_exp2f(-z * 1.4426950408889634f);
                        v[4 * k + q] = z * __builtin_amdgcn_rcpf(1.0f + e) * m[q];
                    }
                }
            }
        };
        bool do_stage = false;  // STG instances only: the plain kernels compile exactly as without staging
        if constexpr (STG) do_stage = (xst.flags & (VQ_STAGE_SILU_MUL | VQ_STAGE_NORM)) != 0;
        if (do_stage) {
            if (norm) {
                for (int i = threadIdx.x; i < NT * 256; i += blockDim.x) {
                    const int t = i >> 8, k = i & 255;
                    float acc = 0.0f;
                    for (int g = k; g < xi.ng; g += 256) {
                        float v[32];
                        staged(t, g, v);
#pragma unroll
                        for (int e = 0; e < 32; ++e) acc = fmaf(v[e], v[e], acc);
                    }
                    nsum[i] = acc;
                }
                for (int h = 128; h > 0; h >>= 1) {
                    __syncthreads();
                    for (int i = threadIdx.x; i < NT * h; i += blockDim.x) {
                        const int t = i / h, k = i - t * h;
                        nsum[t * 256 + k] += nsum[t * 256 + k + h];
                    }
                }
                __syncthreads();
            }
            for (int i = threadIdx.x; i < NT * xi.ng; i += blockDim.x) {
                const int t = i / xi.ng, g = i - t * xi.ng;
                float v[32];
                staged(t, g, v);
                if (norm) {
                    const float rs = 1.0f / sqrtf(nsum[t * 256] / static_cast<float>(cols) + xst.eps);
                    const float4 *nw = reinterpret_cast<const float4 *>(xst.nw + 32 * g);
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const float4 f = nw[k];
                        v[4 * k] *= rs * f.x;
                        v[4 * k + 1] *= rs * f.y;
                        v[4 * k + 2] *= rs * f.z;
                        v[4 * k + 3] *= rs * f.w;
                    }
                }
                const QGroup qg = quantize_group(v);
                uint8_t *img = s_dyn + t * xi.bytes;
                *reinterpret_cast<u32x4 *>(img + xi.code_off(g, 0)) = u32x4{qg.q[0], qg.q[1], qg.q[2], qg.q[3]};
                *reinterpret_cast<u32x4 *>(img + xi.code_off(g, 1)) = u32x4{qg.q[4], qg.q[5], qg.q[6], qg.q[7]};
                reinterpret_cast<float *>(img + xi.xq_bytes)[g] = qg.d;
                reinterpret_cast<uint32_t *>(img + xi.xq_bytes + 4 * xi.ng)[g] = qg.half_sums();
            }
            __syncthreads();  // the RMS sums' LDS is a stage buffer again from here
        } else {
        // Two lanes per (token, group), one 16-element half each: lane pairs read 128 contiguous bytes, so a load
        // instruction touches half as many cache lines as with one lane per group, and the group's amax and the
        // other half's sum come from the partner lane. The IEEE steps are quantize_group's (amax, d = amax/127,
        // id = 1/d, q = rint(v * id)); integer sums do not depend on their order.
        for (int i = threadIdx.x; i < 2 * NT * xi.ng; i += blockDim.x) {
            const int h = i & 1, gi = i >> 1;
            const int t = gi / xi.ng, g = gi - t * xi.ng;
            const float4 *src = reinterpret_cast<const float4 *>(xf + static_cast<size_t>(t) * cols + 32 * g + 16 * h);
            float v[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 f = src[k];
                v[4 * k] = f.x;
                v[4 * k + 1] = f.y;
                v[4 * k + 2] = f.z;
                v[4 * k + 3] = f.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) amax = fmaxf(amax, fabsf(v[k]));
            amax = fmaxf(amax, dpp_f<0xB1>(amax));  // the partner lane (quad_perm [1,0,3,2])
            const float d = amax / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            uint32_t q[4];
            int hs = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t p = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int c = static_cast<int>(__builtin_rintf(v[4 * k + b] * id));
                    hs += c;
                    p |= (static_cast<uint32_t>(c) & 0xFFu) << (8 * b);
                }
                q[k] = p;
            }
            const int hs_other = __builtin_amdgcn_update_dpp(0, hs, 0xB1, 0xF, 0xF, false);
            uint8_t *img = s_dyn + t * xi.bytes;
            *reinterpret_cast<u32x4 *>(img + xi.code_off(g, h)) = u32x4{q[0], q[1], q[2], q[3]};
            if (h == 0) {
                reinterpret_cast<float *>(img + xi.xq_bytes)[g] = d;
                reinterpret_cast<uint32_t *>(img + xi.xq_bytes + 4 * xi.ng)[g] =
                    (static_cast<uint32_t>(hs) & 0xFFFFu) | (static_cast<uint32_t>(hs_other) << 16);
            }
        }
        VQ_STAMP(4);
        VQ_STAMP_IF(threadIdx.x == 128, 5);
        VQ_STAMP_IF(threadIdx.x == 256, 7);
        }
    } else {
        for (int p = wv; p < xreg / 1024; p += NW) {
            const int o = p * 1024 + lane * 16;  // LDS image byte of this lane's chunk
            const int t = o / xi.bytes;
            const int src = t < NT ? xi.src_of(o - t * xi.bytes, cols) : -1;
            dma16(xin, static_cast<uint32_t>(src >= 0 ? t * xb + src : 0), s_dyn + p * 1024);
        }
    }
    wait_vm<0>();
    __builtin_amdgcn_sched_barrier(0);
    // When a minority of the waves fetched activations or tables, those request their first stage only after the
    // start-up barrier: by the time they are done, the other waves' first stages fill the CU's request queue, and
    // issuing a load then stalls the wave until the queue drains (~1-2 us measured), holding every wave at the
    // barrier. (When most waves fetch activations, e.g. a 17408-wide input, requesting late leaves the stream idle
    // through the start-up instead: measured slower.)
    int nact = 0;  // waves with start-up fetches: the first nact
    if constexpr (XF32) nact = STG ? NW : (2 * NT * xi.ng + 63) / 64;
    else nact = xreg / 1024;
    if constexpr (TB > 0) nact = nact > TB / 1024 ? nact : TB / 1024;
    const bool late = wv < nact && 2 * nact <= NW;
    if (s >= 0 && !late) load_stage(s, RA);  // waves without a stage load nothing
    // Stages 0 .. 2 NW - 1 are static: wave w takes w, then w + NW (no ticket round trip before the first
    // decode); tickets hand out the rest.
    const int s2 = wv + NW < nst ? wv + NW : -1;
    if (threadIdx.x == 0) s_next = 2 * NW;
    Tabs tb{};
    if constexpr (SG) {
        tb.sg = reinterpret_cast<const uint32_t *>(s_grid);
    } else {
        if constexpr (TabSpec<T>::n8 > 0) tb.grid8 = reinterpret_cast<const uint2 *>(s_grid);
        if constexpr (TabSpec<T>::n4 > 0) tb.grid4 = reinterpret_cast<const uint32_t *>(s_grid);
    }
    if constexpr (TabSpec<T>::ks) {
        for (int i = threadIdx.x; i < 128; i += blockDim.x) sks[i] = sign_entry(ksigns(i));
        tb.ks128 = sks;
    }
    if constexpr (TabSpec<T>::sm) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) ssm[i] = sign_entry(i);
        tb.sm256 = ssm;
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    VQ_STAMP(1);

    const int ul = lane / LPU;  // unit of this lane within a stage
    const int lj = lane % LPU;  // which of the unit's lanes
    const int ul_bytes = ul * UB;  // this lane's unit within a stage, in bytes past the stage's first unit
    // Lanes 0, LPU nu, 2 LPU nu, ...: shifted by a stage's first row start, the lanes that begin a row.
    uint64_t row_pat = 0;
    for (int p = 0; p < 64; p += LPU * nu) row_pat |= 1ull << p;

    // Decode stage s from the stage buffer; each row's part goes to its slot.
    auto run_stage = [&](int s) {
        const int ua = U0 + s * SU;
        const int nval = U1 - ua < SU ? U1 - ua : SU;  // units in this stage
        const int rf = ua / nu;                          // row of the stage's first unit
        const int col = ua - rf * nu;                    // its unit index within that row
        const bool valid = ul < nval;
        // The stage buffer starts at the 16-byte boundary at or below the stage's first unit.
        const uint8_t *up = sbuf + ((static_cast<unsigned>(ua) * UB) & 15u) + (valid ? ul_bytes : 0);
        // Lanes that start a row (after the stage's first): lane LPU (nu - col) and every LPU nu lanes after it.
        const int p1 = LPU * (nu - col);
        const uint64_t b = p1 < 64 ? row_pat << p1 : 0ull;
        // Row and column unit of this lane's unit: c = col + ul = q*nu + cu, q = the row starts at or below this
        // lane (lane 0 never starts one, so: the bits of b >> 1 below this lane).
        const int c = col + ul;
        const int q = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(b >> 33),
                                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b >> 1), 0)));
        const int cu = c - __mul24(q, nu);
        const int G0 = cu * S::UG;

        float v[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) v[t] = 0.0f;
        // The unit's group scales and half sums of every token.
        float xdu[NT][S::UG];
        int32_t xhu[NT][S::UG];
        if constexpr (kIntScales<T>()) {
            // Every slice decoder's group index is affine in the slice with the lane's own slices lj + LPU k
            // giving the groups of lane 0's slices shifted by one lane constant dg. Accumulators and activation
            // scales are indexed by lane 0's group pg0 (a compile-time index after unrolling: runtime indices
            // into register arrays become compare/select chains), the activation scales read at G0 + dg + pg0.
            static_assert(!kScaledCodes<T>() || LPU == 1, "scaled codes index their shift by the group");
            int dg, dh, d0, h0;
            S::part(lj, 0, dg, dh);
            S::part(0, 0, d0, h0);
            dg -= d0;
            const int Gd = G0 + dg;
            bool used[S::UG];
#pragma unroll
            for (int g = 0; g < S::UG; ++g) used[g] = false;
#pragma unroll
            for (int k = 0; k < G::SPL; ++k)
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    int pg0, ph0;
                    S::part(LPU * k, p, pg0, ph0);
                    used[pg0] = true;
                }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint8_t *xt = s_dyn + t * xi.bytes + xi.xq_bytes;
#pragma unroll
                for (int g = 0; g < S::UG; ++g) {
                    if (!used[g]) continue;
                    xdu[t][g] = reinterpret_cast<const float *>(xt)[Gd + g];
                    if constexpr (kNeedsX<T>) xhu[t][g] = reinterpret_cast<const int32_t *>(xt + 4 * xi.ng)[Gd + g];
                }
            }
            // Integer scales: per (token, group) the exact int32 sum of S * scale (and X * min), then one
            // conversion and fp32 multiply-add per group with the activation scale; the unit's fp32 multipliers
            // (d, dmin) are applied once.
            int gs[NT][S::UG], gm[NT][S::UG];
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int g = 0; g < S::UG; ++g) gs[t][g] = gm[t][g] = 0;
            float dmul = 0.0f, dmn = 0.0f;
#pragma unroll
            for (int k = 0; k < G::SPL; ++k) {
                const int ss = lj + LPU * k;
                typename S::W wr;
                S::load(up, ss, wr);
                uint32_t cd[NP][4];
                if constexpr (kScaledCodes<T>())
                    S::codes_scaled(wr, ss, tb, cd);
                else if constexpr (SG)
                    S::codes_sg(wr, ss, tb, cd);
                else
                    S::codes(wr, ss, tb, cd);
                int isc[NP], imn[NP];
                S::iscales(wr, ss, isc);
                if constexpr (kHasMin<T>) S::imins(wr, ss, imn);
                if (k == 0) {
                    dmul = S::dmul(wr);
                    if constexpr (kHasMin<T>) dmn = S::dmin(wr);
                }
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    int pg, ph, pg0, ph0;
                    S::part(ss, p, pg, ph);
                    S::part(LPU * k, p, pg0, ph0);
                    const int Gi = Gd + pg0;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const uint8_t *xt = s_dyn + t * xi.bytes;
                        const u32x4 xv4 = *reinterpret_cast<const u32x4 *>(xt + xi.code_off(Gi, ph));
                        const int X = kNeedsX<T> ? static_cast<int>(static_cast<int16_t>(
                                                       static_cast<uint32_t>(xhu[t][pg0]) >> (16 * ph)))
                                                 : 0;
                        constexpr int OFFS = S::OFF;
                        int off = OFFS;
                        if constexpr (kScaledCodes<T>()) off = OFFS << S::gsh(pg0);
                        const int Sv = dot4(cd[p][3], xv4.w, dot4(cd[p][2], xv4.z, dot4(cd[p][1], xv4.y,
                                            dot4(cd[p][0], xv4.x, -off * X))));
                        gs[t][pg0] += __mul24(Sv, isc[p]);
                        if constexpr (kHasMin<T>) gm[t][pg0] += __mul24(X, imn[p]);
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float a = 0.0f, m = 0.0f;
#pragma unroll
                for (int g = 0; g < S::UG; ++g) {
                    if (!used[g]) continue;
                    int gsum = gs[t][g];
                    if constexpr (kScaledCodes<T>()) gsum >>= S::gsh(g);  // exact: a multiple of 2^gsh
                    a = fmaf(static_cast<float>(gsum), xdu[t][g], a);
                    if constexpr (kHasMin<T>) m = fmaf(static_cast<float>(gm[t][g]), xdu[t][g], m);
                }
                v[t] = kHasMin<T> ? fmaf(a, dmul, -m * dmn) : a * dmul;
            }
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint8_t *xt = s_dyn + t * xi.bytes + xi.xq_bytes;
#pragma unroll
                for (int g = 0; g < S::UG; ++g) {
                    xdu[t][g] = reinterpret_cast<const float *>(xt)[G0 + g];
                    if constexpr (kNeedsX<T>) xhu[t][g] = reinterpret_cast<const int32_t *>(xt + 4 * xi.ng)[G0 + g];
                }
            }
        }
        if constexpr (!kIntScales<T>()) {
#pragma unroll
            for (int k = 0; k < G::SPL; ++k) {
                const int ss = lj + LPU * k;
                typename S::W wr;
                S::load(up, ss, wr);
                uint32_t cd[NP][4];
                S::codes(wr, ss, tb, cd);
                float sc[NP], mn[NP];
                S::scales(wr, ss, sc, mn);
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    int pg, ph;
                    S::part(ss, p, pg, ph);
                    const int Gi = G0 + pg;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const uint8_t *xt = s_dyn + t * xi.bytes;
                        const u32x4 xv4 = *reinterpret_cast<const u32x4 *>(xt + xi.code_off(Gi, ph));
                        const float xdv = xdu[t][pg];
                        const int X = kNeedsX<T> ? static_cast<int>(static_cast<int16_t>(
                                                       static_cast<uint32_t>(xhu[t][pg]) >> (16 * ph)))
                                                 : 0;
                        const uint32_t xv[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
                        const int Sv = dot16(cd[p], xv) - S::OFF * X;
                        float g = static_cast<float>(Sv) * sc[p];
                        if constexpr (kHasMin<T>) g = fmaf(-static_cast<float>(X), mn[p], g);
                        v[t] = fmaf(g, xdv, v[t]);
                    }
                }
            }
        }
        if (per_lane) {
#pragma unroll
            for (int t = 0; t < NT; ++t) slots[(s * 64 + lane) * NT + t] = v[t];
            return;
        }
        // Segmented inclusive scan over the lanes; segments are the stage's rows (q is non-decreasing in lane
        // order). The last lane of each segment holds that row's part of the stage. DPP moves, no LDS round trips:
        // row_shr 1, 2, 4, 8 scan each 16-lane row, then row_bcast:15 (rows 1, 3 take the last lane of rows 0, 2)
        // and row_bcast:31 (rows 2, 3 take lane 31). A lane adds its source only if no row starts after the
        // source lane and at or before it. Row starts are the same for every lane (lane LPU (nu - col) and every
        // LPU nu lanes after it), so each step's mask of lanes that add is built once in scalar registers:
        // ~(starts smeared over the step's distance). Lanes past the stage's units add garbage among themselves
        // only: sources always lie below a lane.
        const int key = valid ? q : 0x7FFFFFFF;
        {
            const uint64_t s2 = b | (b << 1), s4 = s2 | (s2 << 2), s8 = s4 | (s4 << 4);
            uint64_t w = b;  // a row starts in [16 (lane / 16), lane]
            w |= (w << 1) & 0xFFFEFFFEFFFEFFFEull;
            w |= (w << 2) & 0xFFFCFFFCFFFCFFFCull;
            w |= (w << 4) & 0xFFF0FFF0FFF0FFF0ull;
            w |= (w << 8) & 0xFF00FF00FF00FF00ull;
            const uint32_t bh = static_cast<uint32_t>(b >> 32);  // a row starts in [32, lane]
            const uint64_t vh = bh ? ~0ull << (32 + __builtin_ctz(bh)) : 0ull;
            const uint64_t m1 = ~b, m2 = ~s2, m4 = ~s4, m8 = ~s8, m15 = ~w, m31 = ~vh;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float x = v[t];
                x += keep_lanes(dpp_fz<0x111>(x), m1);        // row_shr:1
                x += keep_lanes(dpp_fz<0x112>(x), m2);        // row_shr:2
                x += keep_lanes(dpp_fz<0x114>(x), m4);        // row_shr:4
                x += keep_lanes(dpp_fz<0x118>(x), m8);        // row_shr:8
                x += keep_lanes(dpp_f<0x142, 0xA>(x), m15);  // row_bcast:15
                x += keep_lanes(dpp_f<0x143, 0xC>(x), m31);  // row_bcast:31
                v[t] = x;
            }
        }
        const int kn = __builtin_amdgcn_update_dpp(-2, key, 0x130, 0xF, 0xF, false);  // wave_shl:1, lane 63 reads -2
        if (valid && kn != key) {
#pragma unroll
            for (int t = 0; t < NT; ++t) slots[(s * rs + q) * NT + t] = v[t];
        }
    };

    // One stage in flight: the next stage's loads are issued before the current one is decoded. Writing RA to
    // LDS waits (compiler-inserted vmcnt) for its loads; the stage buffer is rewritten after the previous
    // stage's LDS reads were issued, and a wave's LDS operations complete in order. The next stage number is
    // asked for one stage ahead, so its LDS round trip hides behind a decode.
    // One lane takes the ticket (a wave-wide atomic would take one per lane); readfirstlane shares it.
    auto take = [&]() { return lane == 0 ? atomicAdd(&s_next, 1) : 0; };
    int ask = s2 >= 0 ? s2 : nst;  // the stage after s (valid in lane 0): the static second stage
    if (s >= 0 && late) load_stage(s, RA);
#ifdef VQ_STAMPS
    bool first_stage = true;
#endif
    while (s >= 0) {
        store_stage(RA);
#ifdef VQ_STAMPS
        VQ_STAMP_IF(first_stage && threadIdx.x == 0, 6);
        first_stage = false;
#endif
        const int sn = __builtin_amdgcn_readfirstlane(ask);
        if (sn < nst) {
            load_stage(sn, RA);
            ask = take();
        }
        run_stage(s);
        s = sn < nst ? sn : -1;
    }
    __syncthreads();
    VQ_STAMP(2);

    // Each row's parts in a fixed order: the row's units are [r*nu - U0, (r+1)*nu - U0) of the range.
    unsigned long long best[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) best[t] = 0ull;
    if (per_lane) {
        // Eight threads per row: thread k adds parts k, k+8, ... of the row's nu*LPU, then three DPP steps.
        const int k = threadIdx.x & 7;
        for (int r0 = R0; r0 < R1; r0 += blockDim.x >> 3) {
            const int r = r0 + static_cast<int>(threadIdx.x >> 3);
            const bool ok = r < R1;
            const int e0 = ok ? (r * nu - U0) * LPU : 0, ne = ok ? nu * LPU : 0;
            float tot[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) tot[t] = 0.0f;
            for (int e = k; e < ne; e += 8) {
#pragma unroll
                for (int t = 0; t < NT; ++t) tot[t] += slots[(e0 + e) * NT + t];
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                // The 8 threads' sums by DPP moves (no LDS round trips): pairs, quads, then the other quad of
                // the half row (row_half_mirror: thread j takes thread 7 - j). Each thread ends with
                // ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)) up to the order of commutative IEEE adds.
                tot[t] += dpp_f<0xB1>(tot[t]);   // quad_perm [1,0,3,2]
                tot[t] += dpp_f<0x4E>(tot[t]);   // quad_perm [2,3,0,1]
                tot[t] += dpp_f<0x141>(tot[t]);  // row_half_mirror
            }
            if (ok && k == 0) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (add) tot[t] += y[static_cast<size_t>(t) * rows + r];
                    if (y != nullptr) y[static_cast<size_t>(t) * rows + r] = tot[t];
                    const unsigned long long key = argmax_key(tot[t], r);
                    best[t] = key > best[t] ? key : best[t];
                }
            }
        }
    }
    for (int r = R0 + static_cast<int>(threadIdx.x); !per_lane && r < R1; r += blockDim.x) {
        const int ua = r * nu - U0, ue = ua + nu - 1;
        const int s0 = ua / SU, s1 = ue / SU;
        float tot[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) tot[t] = 0.0f;
        for (int st = s0; st <= s1; ++st) {
            const int qs = r - (U0 + st * SU) / nu;
#pragma unroll
            for (int t = 0; t < NT; ++t) tot[t] += slots[(st * rs + qs) * NT + t];
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (add) tot[t] += y[static_cast<size_t>(t) * rows + r];
            if (y != nullptr) y[static_cast<size_t>(t) * rows + r] = tot[t];
            const unsigned long long key = argmax_key(tot[t], r);
            best[t] = key > best[t] ? key : best[t];
        }
    }
#ifdef VQ_STAMPS
    __syncthreads();
    VQ_STAMP(3);
    VQ_STAMP_FLUSH();
#endif
    if (jobs.amax != nullptr) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            unsigned long long k = best[t];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const unsigned long long o = __shfl_xor(k, off, 64);
                k = o > k ? o : k;
            }
            if (lane == 0) s_best[t][wv] = k;
        }
        __syncthreads();
        if (threadIdx.x < NT) {
            unsigned long long k = 0ull;
            for (int i = 0; i < NW; ++i) k = s_best[threadIdx.x][i] > k ? s_best[threadIdx.x][i] : k;
            jobs.amax[static_cast<size_t>(threadIdx.x) * jobs.blocks + b] = k;
        }
    }
}

// The kernel: workgroup b runs the body of its job's type. T2 == T for one-type launches; otherwise jobs of
// type T2 (a layer's small tensors, e.g. Q8_0, next to its main matrices) share the launch and its
// activations, and the workgroup size and LDS are the larger of the two types'.
template <int T, int T2, int NT, bool XF32, int NW>
__global__ __launch_bounds__(64 * NW) void qmv_stream_kernel(const QJobs jobs, int cols, const void *__restrict__ xin) {
    const int b = blockIdx.x;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kMaxJobs; ++k) jb = (k < jobs.n && b >= jobs.j[k].b0) ? k : jb;
    if constexpr (T2 != T) {
        if (jobs.j[jb].type == T2) {
            stream_wg<T2, NT, XF32, NW>(jobs, jb, cols, xin, XStage{});
            return;
        }
    }
    stream_wg<T, NT, XF32, NW>(jobs, jb, cols, xin, XStage{});
}
// The same with fp32 activations staged per `xs` (vq_qmv_staged): single-type launches only.
template <int T, int NT, int NW>
__global__ __launch_bounds__(64 * NW) void qmv_staged_kernel(const QJobs jobs, const XStage xs, int cols,
                                                             const float *__restrict__ xin) {
    const int b = blockIdx.x;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kMaxJobs; ++k) jb = (k < jobs.n && b >= jobs.j[k].b0) ? k : jb;
    stream_wg<T, NT, true, NW, true>(jobs, jb, cols, xin, xs);
}

// Final argmax over the per-workgroup keys: one workgroup per token; INT32_MAX when no value qualifies.
static __global__ __launch_bounds__(256) void argmax_keys_kernel(const unsigned long long *__restrict__ keys, int n,
                                                          int32_t *__restrict__ out) {
    __shared__ unsigned long long red[4];
    unsigned long long k = 0ull;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const unsigned long long v = keys[static_cast<size_t>(blockIdx.x) * n + i];
        k = v > k ? v : k;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) k = red[i] > k ? red[i] : k;
        k = red[0] > k ? red[0] : k;
        out[blockIdx.x] = k == 0ull ? 0x7FFFFFFF : static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(k));
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

// Largest dynamic LDS a launch of `kernel` may use: the device's per-workgroup limit minus the kernel's
// static LDS, raised once per kernel (launches above 64 KB need the attribute). 0 if the query fails.
inline int raise_dynamic_lds(const void *kernel) {
    int dev = 0, limit = 0;
    hipFuncAttributes a{};
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&limit, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        hipFuncGetAttributes(&a, kernel) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    const int dyn = limit - static_cast<int>(a.sharedSizeBytes);
    if (dyn <= 0 || hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, dyn) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return dyn;
}

inline size_t static_lds_bytes(const void *kernel) {
    hipFuncAttributes a{};
    if (hipFuncGetAttributes(&a, kernel) != hipSuccess) {
        (void)hipGetLastError();
        return 16 * 1024;
    }
    return a.sharedSizeBytes;
}

// Launch geometry: LDS bytes and resident workgroups on the chip.
// Resident workgroups per CU of a kernel at `lds` dynamic LDS bytes (VGPR, LDS and wave limits, as the
// runtime computes them); 1 if the query fails.
inline int resident_wgs(const void *kernel, int threads, size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess || n < 1) {
        (void)hipGetLastError();
        return 1;
    }
    return n;
}
// Row-part slots (floats) of a workgroup of type TT with rwg rows and N tokens, and the most rows they allow.
template <int TT, int N>
long slot_floats(int cols, long rwg) {
    using G = Stream<TT>;
    const int nu = (cols / 32) / Sl<TT>::UG;
    const long st = (rwg * nu + G::SU - 1) / G::SU;
    return lane_slots(rwg, nu, G::SU, N) ? st * 64 * N : st * rows_per_stage(G::SU, nu) * N;
}
template <int TT, int N>
long max_rwg(int cols) {
    using G = Stream<TT>;
    const int nu = (cols / 32) / Sl<TT>::UG;
    const long max_st = kSlotFloats / (rows_per_stage(G::SU, nu) * N);
    const long r = (max_st * G::SU) / nu;  // whole rows whose stages fit (a row range starts on a row)
    return r > 0 ? r : 1;
}
// Dynamic LDS of a workgroup of type TT with N tokens, NW waves and `slots` row-part slots.
template <int TT, int N, int NW>
size_t stream_lds(int cols, long slots) {
    const int xreg = (N * XImage(cols).bytes + 1023) & ~1023;
    return static_cast<size_t>(xreg) + static_cast<size_t>(NW) * Stream<TT>::STAGE_LDS + 4 * static_cast<size_t>(slots);
}
// Resident workgroups on the chip of qmv_stream_kernel<T, T2, N, *, NW> at `lds` bytes, 0 if the LDS does not
// fit. Both activation forms: the grid must not depend on the form. Cached per LDS size: the occupancy
// queries cost host time on every launch otherwise. (Without a device the queries fail: then 160 KB and one
// workgroup per CU, so that workspace sizes can still be computed.)
template <int T, int T2, int N, int NW>
int resident_chip(size_t lds) {
    static std::mutex mu;
    static std::unordered_map<long, int> cache;
    static const int max_a = raise_dynamic_lds(reinterpret_cast<const void *>(&qmv_stream_kernel<T, T2, N, false, NW>));
    static const int max_b = raise_dynamic_lds(reinterpret_cast<const void *>(&qmv_stream_kernel<T, T2, N, true, NW>));
    const int lim = max_a > 0 && max_b > 0 ? (max_a < max_b ? max_a : max_b) : 160 * 1024;
    if (lds > static_cast<size_t>(lim)) return 0;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(static_cast<long>(lds));
    if (it == cache.end()) {
        const int ra = resident_wgs(reinterpret_cast<const void *>(&qmv_stream_kernel<T, T2, N, false, NW>), 64 * NW, lds);
        const int rb = resident_wgs(reinterpret_cast<const void *>(&qmv_stream_kernel<T, T2, N, true, NW>), 64 * NW, lds);
        it = cache.emplace(static_cast<long>(lds), ra < rb ? ra : rb).first;
    }
    return 256 * it->second;
}

// Work split of one launch: rows per workgroup of each job, workgroups, waves per workgroup (0 blocks if no
// geometry fits). types[k] is T or T2.
struct Plan {
    int rwg[kMaxJobs], b0[kMaxJobs];
    int blocks, nw;
};
template <int T, int T2, int N, int NW>
size_t plan_lds(const int *types, int n, int cols, const int *rwg) {
    size_t lds = 0;
    for (int k = 0; k < n; ++k) {
        const size_t l = types[k] == T2 && T2 != T ? stream_lds<T2, N, NW>(cols, slot_floats<T2, N>(cols, rwg[k]))
                                                   : stream_lds<T, N, NW>(cols, slot_floats<T, N>(cols, rwg[k]));
        lds = l > lds ? l : lds;
    }
    return lds;
}
template <int T, int T2, int N, int NW>
Plan plan_nw(const int *types, const int *rows, int n, int cols) {
    Plan p{};
    int cap[kMaxJobs];
    for (int k = 0; k < n; ++k)
        cap[k] = static_cast<int>(types[k] == T2 && T2 != T ? max_rwg<T2, N>(cols) : max_rwg<T, N>(cols));
    // One round of workgroups, shared out in proportion to each job's bytes (at least one each).
    const int wres = resident_chip<T, T2, N, NW>(plan_lds<T, T2, N, NW>(types, n, cols, cap));
    if (wres == 0) return p;
    double bytes[kMaxJobs], total = 0.0;
    for (int k = 0; k < n; ++k) {
        int bs = 0, ts = 0;
        vq_traits(types[k], &bs, &ts);
        bytes[k] = static_cast<double>(rows[k]) * (cols / bs) * ts;
        total += bytes[k];
    }
    int blocks = 0;
    for (int k = 0; k < n; ++k) {
        long nb = static_cast<long>(wres * bytes[k] / total);
        if (nb < 1) nb = 1;
        long rwg = (rows[k] + nb - 1) / nb;
        if (rwg > cap[k]) rwg = cap[k];
        if (rwg < 1) rwg = 1;
        p.rwg[k] = static_cast<int>(rwg);
        p.b0[k] = blocks;
        blocks += static_cast<int>((rows[k] + rwg - 1) / rwg);
    }
    p.blocks = blocks;
    p.nw = NW;
    return p;
}
template <int T, int T2, int N>
Plan plan_n(const int *types, const int *rows, int n, int cols) {
    const Plan p = plan_nw<T, T2, N, wg_waves<N>()>(types, rows, n, cols);
    return p.blocks > 0 ? p : plan_nw<T, T2, N, kFallbackWaves>(types, rows, n, cols);
}
// Most tokens per launch: 8, or kMixedMaxTokens for mixed-type launches (fewer kernel instantiations).
template <int T, int T2>
constexpr int max_tokens() {
    return T2 == T ? 8 : kMixedMaxTokens;
}
// f(std::integral_constant<int, N>) for N = n_tok clamped to [1, NMAX].
template <int NMAX, typename F>
auto with_tokens(int n_tok, F &&f) {
    if (n_tok <= 1 || NMAX == 1) return f(std::integral_constant<int, 1>{});
    if constexpr (NMAX >= 2) if (n_tok == 2 || NMAX == 2) return f(std::integral_constant<int, 2>{});
    if constexpr (NMAX >= 3) if (n_tok == 3 || NMAX == 3) return f(std::integral_constant<int, 3>{});
    if constexpr (NMAX >= 4) if (n_tok == 4 || NMAX == 4) return f(std::integral_constant<int, 4>{});
    if constexpr (NMAX >= 5) if (n_tok == 5 || NMAX == 5) return f(std::integral_constant<int, 5>{});
    if constexpr (NMAX >= 6) if (n_tok == 6 || NMAX == 6) return f(std::integral_constant<int, 6>{});
    if constexpr (NMAX >= 7) if (n_tok == 7 || NMAX == 7) return f(std::integral_constant<int, 7>{});
    return f(std::integral_constant<int, (NMAX >= 8 ? 8 : NMAX)>{});
}
template <int T, int T2>
Plan plan_launch(const int *types, const int *rows, int n, int cols, int n_tok) {
    return with_tokens<max_tokens<T, T2>()>(n_tok, [&](auto nt) { return plan_n<T, T2, decltype(nt)::value>(types, rows, n, cols); });
}

// One launch of N tokens with the plan's rows per workgroup: the preferred waves per workgroup if the LDS
// holds them, else kFallbackWaves (the rows per workgroup come from the launch's plan, so every token chunk
// splits the rows alike).
template <int T, int T2, int N>
int launch_stream(const QJobs &jobs, const int *types, int cols, const void *xp, bool x_f32, hipStream_t s,
                  const XStage &xs) {
    int rwg[kMaxJobs];
    for (int k = 0; k < jobs.n; ++k) rwg[k] = jobs.j[k].rwg;
    constexpr int NWP = wg_waves<N>(), NWF = kFallbackWaves;
    const dim3 grid(static_cast<unsigned>(jobs.blocks));
    const size_t ldsp = plan_lds<T, T2, N, NWP>(types, jobs.n, cols, rwg);
    if constexpr (T2 == T) {
        // Staged fp32 activations (vq_qmv_staged): their own instances, with the plain kernel's geometry.
        if (x_f32 && xs.flags != 0) {
            static const int raised_p = raise_dynamic_lds(reinterpret_cast<const void *>(&qmv_staged_kernel<T, N, NWP>));
            static const int raised_f = raise_dynamic_lds(reinterpret_cast<const void *>(&qmv_staged_kernel<T, N, NWF>));
            (void)raised_p, (void)raised_f;
            const float *xf = static_cast<const float *>(xp);
            if (resident_chip<T, T2, N, NWP>(ldsp) > 0) {
                qmv_staged_kernel<T, N, NWP><<<grid, dim3(64 * NWP), ldsp, s>>>(jobs, xs, cols, xf);
            } else {
                const size_t ldsf = plan_lds<T, T2, N, NWF>(types, jobs.n, cols, rwg);
                if (resident_chip<T, T2, N, NWF>(ldsf) == 0) return static_cast<int>(hipErrorInvalidConfiguration);
                qmv_staged_kernel<T, N, NWF><<<grid, dim3(64 * NWF), ldsf, s>>>(jobs, xs, cols, xf);
            }
            return hip_status(hipGetLastError());
        }
    }
    if (resident_chip<T, T2, N, NWP>(ldsp) > 0) {
        if (x_f32)
            qmv_stream_kernel<T, T2, N, true, NWP><<<grid, dim3(64 * NWP), ldsp, s>>>(jobs, cols, xp);
        else
            qmv_stream_kernel<T, T2, N, false, NWP><<<grid, dim3(64 * NWP), ldsp, s>>>(jobs, cols, xp);
    } else {
        const size_t ldsf = plan_lds<T, T2, N, NWF>(types, jobs.n, cols, rwg);
        if (resident_chip<T, T2, N, NWF>(ldsf) == 0) return static_cast<int>(hipErrorInvalidConfiguration);
        if (x_f32)
            qmv_stream_kernel<T, T2, N, true, NWF><<<grid, dim3(64 * NWF), ldsf, s>>>(jobs, cols, xp);
        else
            qmv_stream_kernel<T, T2, N, false, NWF><<<grid, dim3(64 * NWF), ldsf, s>>>(jobs, cols, xp);
    }
    return hip_status(hipGetLastError());
}


// Workgroups of a single-job launch (the argmax key count per token).
template <int T>
long argmax_waves(int rows, int cols, int ntok) {
    const int m = ntok < token_chunk(cols) ? ntok : token_chunk(cols);
    const int ty = T;
    return plan_launch<T, T>(&ty, &rows, 1, cols, m).blocks;
}

// y_j = W_j x for the n jobs (types T or T2, same cols), x fp32 (quantized in-kernel) or packed. With `amax`
// ([ntok][argmax_waves] keys, single job), also amax_out[t] = argmax_r y[t][r].
template <int T, int T2>
int launch_jobs(int n, const int *types, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                const void *x, bool x_f32, int ntok, unsigned long long *amax, int32_t *amax_out, hipStream_t s,
                const XStage &xs = XStage{}) {
    if (n < 1 || n > kMaxJobs || (amax && n != 1)) return static_cast<int>(hipErrorInvalidValue);
    // Units per row stay below 2^13 (the kernels' unit-to-row quotient relies on it); the activation image of
    // one token would not fit LDS long before that.
    if (cols >= (1 << 18)) return static_cast<int>(hipErrorInvalidConfiguration);
    const size_t tok_bytes = x_f32 ? static_cast<size_t>(cols) * 4 : static_cast<size_t>(vq_xpack_stride(cols));
    const int chunk = token_chunk(cols) < max_tokens<T, T2>() ? token_chunk(cols) : max_tokens<T, T2>();
    // One split for every token chunk (the first is the widest), so the argmax key layout is the same.
    const Plan pl = plan_launch<T, T2>(types, rows, n, cols, ntok < chunk ? ntok : chunk);
    if (pl.blocks <= 0) return static_cast<int>(hipErrorInvalidConfiguration);
    for (int c = 0; c < ntok; c += chunk) {
        const int m = ntok - c < chunk ? ntok - c : chunk;
        QJobs jobs{};
        jobs.n = n;
        for (int k = 0; k < n; ++k) {
            jobs.j[k].w = w[k];
            jobs.j[k].y = y[k] ? y[k] + static_cast<size_t>(c) * rows[k] : nullptr;
            jobs.j[k].rows = rows[k];
            jobs.j[k].b0 = pl.b0[k];
            jobs.j[k].rwg = pl.rwg[k];
            jobs.j[k].type = types[k];
        }
        jobs.blocks = pl.blocks;
        XStage xsc = xs;
        if (xs.x2 != nullptr) xsc.x2 = xs.x2 + static_cast<size_t>(c) * cols;
        jobs.amax = amax ? amax + static_cast<size_t>(c) * pl.blocks : nullptr;
        const void *xp = static_cast<const uint8_t *>(x) + static_cast<size_t>(c) * tok_bytes;
        const int st = with_tokens<max_tokens<T, T2>()>(m, [&](auto nt) {
            return launch_stream<T, T2, decltype(nt)::value>(jobs, types, cols, xp, x_f32, s, xsc);
        });
        if (st) return st;
    }
    if (amax) {
        argmax_keys_kernel<<<ntok, 256, 0, s>>>(amax, pl.blocks, amax_out);
        return hip_status(hipGetLastError());
    }
    return 0;
}

template <int T>
int launch_quant_jobs(int n, const uint8_t *const *w, const int *rows, float *const *y, int cols, const void *x,
                      bool x_f32, int ntok, unsigned long long *amax, int32_t *amax_out, hipStream_t s) {
    int types[kMaxJobs];
    for (int k = 0; k < kMaxJobs; ++k) types[k] = T;
    return launch_jobs<T, T>(n, types, w, rows, y, cols, x, x_f32, ntok, amax, amax_out, s);
}

// Jobs of type T and Q8_0 in one launch (fp32 activations; token chunks of at most kMixedMaxTokens).
template <int T>
int launch_mixed_q8(int n, const int *types, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                    const float *x, int ntok, hipStream_t s) {
    if constexpr (T == VQ_Q8_0)
        return launch_jobs<T, T>(n, types, w, rows, y, cols, x, true, ntok, nullptr, nullptr, s);
    else
        return launch_jobs<T, VQ_Q8_0>(n, types, w, rows, y, cols, x, true, ntok, nullptr, nullptr, s);
}

template <int T, int T2>
int launch_mixed2(int n, const int *types, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                  const float *x, int ntok, hipStream_t s) {
    return launch_jobs<T, T2>(n, types, w, rows, y, cols, x, true, ntok, nullptr, nullptr, s);
}

template <int T>
int launch_quant_staged(const uint8_t *w, int rows, int cols, long rb, const float *x, const XStage &xs, int ntok,
                        float *y, hipStream_t s) {
    (void)rb;
    const int types[1] = {T};
    return launch_jobs<T, T>(1, types, &w, &rows, &y, cols, x, true, ntok, nullptr, nullptr, s, xs);
}

template <int T>
int launch_quant(const uint8_t *w, int rows, int cols, long rb, const void *x, bool x_f32, int ntok, float *y,
                 hipStream_t s) {
    (void)rb;
    return launch_quant_jobs<T>(1, &w, &rows, &y, cols, x, x_f32, ntok, nullptr, nullptr, s);
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
#define VQ_INSTANTIATE(T) VQ_KERNEL_TEMPLATES(template, T)
