// vq_qmv_impl.h -- quantized matvec kernels, templated on the GGUF type (one translation unit per type
// instantiates them: vq_t_<type>.hip). Hand-written for CDNA4 (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <unordered_map>

#include "vq_qmv.h"
#include "vq_quant.h"
#include "vq_tables.h"

namespace vq {

// Streaming geometry (compile-time; overridable for tuning builds).
#ifndef VQ_X_LDS_MAX
#define VQ_X_LDS_MAX (64 * 1024)  // bytes of activation records one launch keeps in LDS
#endif

// ---- global -> LDS DMA ---------------------------------------------------------------------------------
// The weight stream reaches LDS through global_load_lds_dwordx4 (each lane moves 16 bytes; a wave writes
// 1 KB contiguously at M0), so bytes in flight cost no VGPRs. The DMA is issued from inline asm: the
// compiler then neither counts it nor inserts its own vmcnt(0) before every LDS read, and the kernel waits
// on vmcnt itself (loads retire in order, so "at most N outstanding" means "all but the last N landed").
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void *)p));
}
// 64 lanes x 16 bytes: lane i copies base[voff_i .. +16) to LDS lds + 16 i. base and lds are wave-uniform.
__device__ __forceinline__ void dma16(const void *base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, %0" ::"s"(base), "v"(voff), "s"(lds) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Sum over the 64 lanes with DPP moves (no LDS round trips): pairs, quads, half rows, rows, then rows 1/3
// take row 0/2 (row_bcast:15) and rows 2/3 take lane 31 (row_bcast:31); lane 63 ends with the total.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
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

// Finished row sums one wave keeps in LDS until its end: rows per wave * tokens <= kYSlots.
constexpr int kYSlots = 256;

// Per-type stage shape: LPU lanes decode one unit (each takes SPB/LPU of its slices), so a stage is the
// SU = 64/LPU consecutive units of the wave's stream. LPU is chosen so that a stage spans about 2-7 KB: the
// wave holds two stages of raw bytes in VGPRs (one landing, one in flight), so the stage size sets both the
// bytes a wave keeps in flight and its VGPR cost. Tuning builds override with VQ_LPU / VQ_WAVES.
template <int T>
struct StageShape {
    static constexpr int LPU_DEFAULT =
        (T == VQ_Q8_0 || T == VQ_IQ4_NL || T == VQ_IQ2_XXS || T == VQ_IQ2_XS || T == VQ_IQ2_S || T == VQ_Q3_K) ? 1 : 2;
#ifdef VQ_LPU
    static constexpr int LPU = VQ_LPU < Sl<T>::SPB ? VQ_LPU : Sl<T>::SPB;
#else
    static constexpr int LPU = LPU_DEFAULT;
#endif
#ifdef VQ_WAVES
    static constexpr int NW = VQ_WAVES;
#else
    static constexpr int NW = 4;  // waves per workgroup
#endif
#ifdef VQ_NBUF
    static constexpr int NB = VQ_NBUF;
#else
    static constexpr int NB = 1;
#endif
};

// LDS image of the activation records: per token, the int8 codes in blocks of 256 followed by XPAD bytes
// of padding (so that the codes lanes of neighbouring units read fall in different LDS banks), then the
// group scales xd and the half sums xh as in the packed record. Built by the DMA: LDS chunk i (16 bytes)
// is fetched from the packed record chunk that belongs there.
#ifndef VQ_XPAD
#define VQ_XPAD 32
#endif
struct XImage {
    int ng, nblk, xq_bytes, bytes;  // bytes: one token's image (16-byte multiple)
    __host__ __device__ explicit XImage(int cols)
        : ng(cols / 32), nblk((cols / 32 + 7) / 8), xq_bytes(((cols / 32 + 7) / 8) * (256 + VQ_XPAD)),
          bytes((((cols / 32 + 7) / 8) * (256 + VQ_XPAD) + (cols / 32) * 8 + 15) / 16 * 16) {}
    __device__ int code_off(int G, int h) const { return (G >> 3) * (256 + VQ_XPAD) + (G & 7) * 32 + 16 * h; }
    // Byte of the packed record (vq_xpack_h_offset layout) that LDS image byte o (16-byte aligned) holds,
    // or -1 for padding.
    __device__ int src_of(int o, int cols) const {
        if (o < xq_bytes) {
            const int blk = o / (256 + VQ_XPAD), w = o - blk * (256 + VQ_XPAD);
            return w < 256 && blk * 256 + w < cols ? blk * 256 + w : -1;
        }
        return cols + (o - xq_bytes);
    }
};

template <int T>
struct Stream {
    using S = Sl<T>;
    static constexpr int LPU = StageShape<T>::LPU;
    static constexpr int SPL = S::SPB / LPU;  // slices per lane
    static constexpr int SU = 64 / LPU;       // units per stage
    static constexpr bool BLOCKED = false;    // lane j of a unit takes slices j, j+LPU, ...
    // 16-byte chunks one stage's bytes can touch (its units plus the dword the decoders may read past the
    // last unit, from an arbitrary 16-byte phase) and the dwordx4 loads per lane that cover them.
    static constexpr int CMAX = (SU * S::UB + 4 + 15) / 16 + 1;
    static constexpr int NL = (CMAX + 63) / 64;
    static constexpr int NW = StageShape<T>::NW;
    static constexpr int NB = StageShape<T>::NB;  // stages in flight while one is decoded (1 or 2)
    // Per wave: the stage buffer, then the finished row sums ([NT][rpw] fp32, rpw * NT <= kYSlots). Row sums
    // are written to y once, at the end: a vector store in the stage loop would leave stores and loads
    // pending on the one vmcnt counter, and the compiler then waits for all loads, both buffers included.
    static constexpr int WAVE_LDS = NL * 1024 + 4 * kYSlots;
    static_assert(S::SPB % LPU == 0 && NL >= 1 && NL <= 16, "stage geometry");
};

template <int T>
constexpr int grid_table_bytes() {
    return TabSpec<T>::n8 * 8 + TabSpec<T>::n4 * 4;
}
template <int T>
__device__ __forceinline__ const uint8_t *grid_table_src() {
    if constexpr (T == VQ_IQ2_XXS) return reinterpret_cast<const uint8_t *>(g_iq2xxs.v);
    if constexpr (T == VQ_IQ2_XS) return reinterpret_cast<const uint8_t *>(g_iq2xs.v);
    if constexpr (T == VQ_IQ2_S) return reinterpret_cast<const uint8_t *>(g_iq2s.v);
    if constexpr (T == VQ_IQ3_XXS) return reinterpret_cast<const uint8_t *>(g_iq3xxs.v);
    if constexpr (T == VQ_IQ3_S) return reinterpret_cast<const uint8_t *>(g_iq3s.v);
    return nullptr;
}

// One launch covers up to kMaxJobs matrices of the same type and width that share the activations (a
// layer's gate/up, q/k/v, ...). Job j owns the grid's waves [wave0, wave0 + ceil(rows/rpw)).
constexpr int kMaxJobs = 4;
// Row accumulators per lane on the fast path: a stage of SU units touches at most kRowSlots rows when
// rows have at least SU/(kRowSlots-1) units.
constexpr int kRowSlots = 5;
struct QJob {
    const uint8_t *w;
    float *y;  // [NT][rows], or null (argmax only)
    int rows, rpw, wave0;
};
struct QJobs {
    QJob j[kMaxJobs];
    int n;
    int waves;               // total waves of the grid that own rows
    unsigned long long *amax;  // null, or [NT][waves] per-wave argmax keys (see argmax_key)
};

// Argmax key of a value at row r: larger key = larger value, then lower row. NaN and -inf never win (the
// reference kernel starts from -inf and takes strictly greater values); 0 = no candidate.
__device__ __forceinline__ unsigned long long argmax_key(float v, long r) {
    const uint32_t u = __float_as_uint(v);
    if (v != v || v == -__builtin_huge_valf()) return 0ull;
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(o) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(r));
}

// Quantized matvec: y[t][r] = W[r] . x[t] for t < NT.
//
// Wave g of the grid owns rows [g*rpw, (g+1)*rpw) -- a contiguous byte range, since rows are back to back
// and each row is a whole number of units (32-element groups for Q8_0/IQ4_NL, 256-element super-blocks
// otherwise). It walks that range in stages of SU = 64/LPU units. A stage's bytes (16-byte chunks
// [c0, c1)) arrive in VGPRs by NL coalesced nontemporal dwordx4 loads per lane, two stages ahead: while
// stage s is decoded, the loads of stages s+1 and s+2 are in flight. The landed chunks of stage s are
// written to the wave's LDS stage buffer (lane order = byte order), and the LPU lanes of each unit decode
// its slices with the type's slice decoders (weights, activation records and IQ tables all read from LDS),
// so the block header is decoded once per 256/LPU elements. Rows that end in the stage are summed over the
// wave and written.
//
// LDS: [grid table | activation image of the NT tokens | one stage buffer per wave]. At start-up the waves
// request their share of the table and of the activation image (DMA), then their first two stages, and
// meet at one barrier once the activations are in.
template <int T, int NT, bool FEW, bool XF32>
__global__ __launch_bounds__(64 * Stream<T>::NW) void qmv_stream_kernel(const QJobs jobs, int cols,
                                                                   const void *__restrict__ xin) {
    using S = Sl<T>;
    using G = Stream<T>;
    constexpr int NP = S::NP, UB = S::UB, LPU = G::LPU, SU = G::SU, NL = G::NL;
    constexpr int TB = grid_table_bytes<T>();
    extern __shared__ __attribute__((aligned(1024))) uint8_t s_dyn[];
    __shared__ __attribute__((aligned(1024))) uint8_t s_grid[TB > 0 ? TB : 16];
    __shared__ uint4 sks[TabSpec<T>::ks ? 128 : 1];
    __shared__ uint4 ssm[TabSpec<T>::sm ? 256 : 1];

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    constexpr int NW = G::NW;
    const int nu = (cols >> 5) / S::UG;
    const int xb = vq_xpack_stride(cols);
    const XImage xi(cols);
    const int xreg = (NT * xi.bytes + 1023) & ~1023;
    uint8_t *const sbuf = s_dyn + xreg + wv * G::WAVE_LDS;
    float *const ybuf = reinterpret_cast<float *>(sbuf + NL * 1024);

    // This wave's job, rows and stages.
    const int gw = blockIdx.x * NW + wv;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kMaxJobs; ++k) jb = (k < jobs.n && gw >= jobs.j[k].wave0) ? k : jb;
    const uint8_t *const w = jobs.j[jb].w;
    float *const y = jobs.j[jb].y;
    const int rows = jobs.j[jb].rows, rpw = jobs.j[jb].rpw;
    const long r0 = gw < jobs.waves ? static_cast<long>(gw - jobs.j[jb].wave0) * rpw : rows;
    const long r1 = r0 + rpw < rows ? r0 + rpw : rows;
    const long U0 = r0 * nu, U1 = r1 * nu;
    const int nst = r0 < rows ? static_cast<int>((U1 - U0 + SU - 1) / SU) : 0;
    // Chunks of stage s: [c0, c1) with c0 the chunk of its first byte and c1 past the chunk holding the dword
    // after its last unit -- but never past the chunk holding the matrix's last byte (the weight buffer has
    // 16 readable pad bytes; decoders discard bytes past a block). Lanes past c1 re-read chunk c1 - 1 (the
    // same addresses as a lane that does load it: no extra traffic), so every stage issues exactly NL loads.
    const long mend = static_cast<long>(rows) * nu * UB;
    const u32x4 *const w16 = reinterpret_cast<const u32x4 *>(w);
    auto chunk0 = [&](int s) { return ((U0 + static_cast<long>(s) * SU) * UB) >> 4; };
    auto load_stage = [&](int s, u32x4 (&R)[NL]) {
        const long ua = U0 + static_cast<long>(s) * SU;
        const long ub = ua + SU < U1 ? ua + SU : U1;
        const long e = ub * UB + 4 < mend ? ub * UB + 4 : mend;
        const long c0 = (ua * UB) >> 4, cl = ((e + 15) >> 4) - 1;
        // Wave-uniform base and limit; per-lane 32-bit chunk offsets.
        const u32x4 *const base = w16 + c0;
        const int lim = __builtin_amdgcn_readfirstlane(static_cast<int>(cl - c0));
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const unsigned c = static_cast<unsigned>(lane + 64 * i);
            R[i] = __builtin_nontemporal_load(base + (c < static_cast<unsigned>(lim) ? c : static_cast<unsigned>(lim)));
        }
    };
    auto store_stage = [&](const u32x4 (&R)[NL]) {
#pragma unroll
        for (int i = 0; i < NL; ++i) reinterpret_cast<u32x4 *>(sbuf)[lane + 64 * i] = R[i];
    };

    // Start-up: table and activation pieces (striped over the waves), then the first two stages.
    if constexpr (TB > 0) {
        const uint8_t *src = grid_table_src<T>();
        for (int p = wv; p < TB / 1024; p += NW) dma16(src + p * 1024, lane * 16, lds_addr(s_grid) + p * 1024);
    }
#ifndef VQ_NOXIMG
    if constexpr (!XF32) {
#else
    if constexpr (false) {
#endif
        for (int p = wv; p < xreg / 1024; p += NW) {
            const int o = p * 1024 + lane * 16;  // LDS image byte of this lane's chunk
            const int t = o / xi.bytes;
            const int src = t < NT ? xi.src_of(o - t * xi.bytes, cols) : -1;
            dma16(xin, static_cast<uint32_t>(src >= 0 ? t * xb + src : 0), lds_addr(s_dyn) + p * 1024);
        }
    }
    // Every wave issues exactly NL loads per buffer fill, whatever its stage count (stages past the last
    // re-read the last one, from L2): the compiler's vmcnt bookkeeping then sees the same number of loads
    // in flight on every path and waits for one buffer only.
    const int slast = nst > 0 ? nst - 1 : 0;
    u32x4 RA[NL], RB[G::NB == 2 ? NL : 1];
    load_stage(0, RA);
    if constexpr (G::NB == 2) load_stage(1 < slast ? 1 : slast, RB);
    if constexpr (XF32) {
        // fp32 activations: quantize each 32-group here, straight into the LDS image (the weight stream is
        // already requested, so this overlaps its first round trip).
        const float *x = static_cast<const float *>(xin);
        for (int i = threadIdx.x; i < NT * xi.ng; i += blockDim.x) {
            const int t = i / xi.ng, g = i - t * xi.ng;
            const QGroup qg = quantize_group(x + static_cast<size_t>(t) * cols + 32 * g);
            uint8_t *img = s_dyn + t * xi.bytes;
            *reinterpret_cast<u32x4 *>(img + xi.code_off(g, 0)) = u32x4{qg.q[0], qg.q[1], qg.q[2], qg.q[3]};
            *reinterpret_cast<u32x4 *>(img + xi.code_off(g, 1)) = u32x4{qg.q[4], qg.q[5], qg.q[6], qg.q[7]};
            reinterpret_cast<float *>(img + xi.xq_bytes)[g] = qg.d;
            reinterpret_cast<uint32_t *>(img + xi.xq_bytes + 4 * xi.ng)[g] = qg.half_sums();
        }
    }
    Tabs tb{};
    if constexpr (TabSpec<T>::n8 > 0) tb.grid8 = reinterpret_cast<const uint2 *>(s_grid);
    if constexpr (TabSpec<T>::n4 > 0) tb.grid4 = reinterpret_cast<const uint32_t *>(s_grid);
    if constexpr (TabSpec<T>::ks) {
        for (int i = threadIdx.x; i < 128; i += blockDim.x) sks[i] = sign_entry(ksigns(i));
        tb.ks128 = sks;
    }
    if constexpr (TabSpec<T>::sm) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) ssm[i] = sign_entry(i);
        tb.sm256 = ssm;
    }
    // The DMAs were issued before this wave's stage loads, and loads retire in order: once at most the
    // stage loads are outstanding, the table and activation pieces have landed.
    if constexpr (TB > 0 || !XF32) wait_vm<G::NB * NL>();
    wait_lgkm0();
#ifndef VQ_NOBAR
    __builtin_amdgcn_s_barrier();
#endif
    asm volatile("" ::: "memory");
    if (nst == 0) return;

    const int ul = lane / LPU;  // unit of this lane within a stage
    const int lj = lane % LPU;  // which of the unit's lanes
    const float inv_nu = 1.0f / static_cast<float>(nu);
    long row_a = r0;       // row of the stage's first unit (wave-uniform)
    int col_a = 0;         // its unit index within that row
    long carry_row = -1;   // row whose earlier part is in carry[] (segmented-scan path)
    float carry[NT];
    constexpr int NS = kRowSlots;
    float acc[NS][NT];     // rows row_a .. row_a+NS-1 (FEW path: a stage touches at most NS rows)
    unsigned long long best[NT];  // argmax key of this wave's finished rows (wave-uniform)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        carry[t] = 0.0f;
#pragma unroll
        for (int k = 0; k < NS; ++k) acc[k][t] = 0.0f;
        best[t] = 0ull;
    }

    // Decode stage s from the stage buffer (its chunk c0 at sbuf) and fold it into the row sums.
    auto run_stage = [&](int s) {
        const long ua = U0 + static_cast<long>(s) * SU;
        const int nval = static_cast<int>((U1 - ua < SU ? U1 - ua : SU));  // units in this stage
        const bool valid = ul < nval;
        const uint8_t *up = sbuf + ((ua + (valid ? ul : 0)) * UB - (chunk0(s) << 4));
        // Row and column unit of this lane's unit: c = col_a + ul = q*nu + cu with q small.
        const int c = col_a + ul;
        int q = static_cast<int>(static_cast<float>(c) * inv_nu);
        q = (q + 1) * nu <= c ? q + 1 : q;
        q = q * nu > c ? q - 1 : q;
        const int cu = c - q * nu;
        const int G0 = cu * S::UG;

        float v[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) v[t] = 0.0f;
#ifdef VQ_NODECODE
        v[0] = static_cast<float>(*reinterpret_cast<const uint32_t *>(up + 4 * lj) & 0xFF) * static_cast<float>(G0);
#else
        // The unit's group scales and half sums of every token (two 16-byte LDS reads each).
        float xdu[NT][S::UG];
        int32_t xhu[NT][S::UG];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint8_t *xt = s_dyn + t * xi.bytes + xi.xq_bytes;
#pragma unroll
            for (int g = 0; g < S::UG; ++g) {
                xdu[t][g] = reinterpret_cast<const float *>(xt)[G0 + g];
                if constexpr (kNeedsX<T>) xhu[t][g] = reinterpret_cast<const int32_t *>(xt + 4 * xi.ng)[G0 + g];
            }
        }
        if constexpr (kIntScales<T>()) {
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
                    int pg, ph;
                    S::part(ss, p, pg, ph);
                    const int Gi = G0 + pg;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const uint8_t *xt = s_dyn + t * xi.bytes;
                        const u32x4 xv4 = *reinterpret_cast<const u32x4 *>(xt + xi.code_off(Gi, ph));
                        const int X = kNeedsX<T> ? static_cast<int>(static_cast<int16_t>(
                                                       static_cast<uint32_t>(xhu[t][pg]) >> (16 * ph)))
                                                 : 0;
                        const int Sv = dot4(cd[p][3], xv4.w, dot4(cd[p][2], xv4.z, dot4(cd[p][1], xv4.y,
                                            dot4(cd[p][0], xv4.x, -S::OFF * X))));
                        gs[t][pg] += __mul24(Sv, isc[p]);
                        if constexpr (kHasMin<T>) gm[t][pg] += __mul24(X, imn[p]);
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float a = 0.0f, m = 0.0f;
#pragma unroll
                for (int g = 0; g < S::UG; ++g) {
                    a = fmaf(static_cast<float>(gs[t][g]), xdu[t][g], a);
                    if constexpr (kHasMin<T>) m = fmaf(static_cast<float>(gm[t][g]), xdu[t][g], m);
                }
                v[t] = kHasMin<T> ? fmaf(a, dmul, -m * dmn) : a * dmul;
            }
        } else {
#pragma unroll
        for (int k = 0; k < G::SPL; ++k) {
            const int ss = G::BLOCKED ? lj * G::SPL + k : lj + LPU * k;
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
#endif
        if constexpr (FEW) {
            // Rows have at least SU/(NS-1) units, so this lane's unit is in row row_a + q with q < NS. Rows that
            // end in this stage are summed over the wave and written; the others shift down.
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int k = 0; k < NS; ++k) acc[k][t] += q == k ? v[t] : 0.0f;
            const int done = (col_a + nval) / nu;  // rows completed by this stage (0..NS-1)
#pragma unroll
            for (int k = 0; k < NS - 1; ++k) {
                if (k < done) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const float tot = wave_sum(acc[k][t]);
                        if (lane == 0) ybuf[t * rpw + static_cast<int>(row_a + k - r0)] = tot;
                        const unsigned long long key = argmax_key(tot, row_a + k);
                        best[t] = key > best[t] ? key : best[t];
                    }
                }
            }
            if (done > 0) {
#pragma unroll
                for (int k = 0; k < NS; ++k)
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        float nv = 0.0f;
#pragma unroll
                        for (int d = 1; d < NS; ++d)
                            if (k + d < NS) nv = done == d ? acc[k + d][t] : nv;
                        acc[k][t] = nv;
                    }
            }
            row_a += done;
            col_a += nval - done * nu;
        } else {
            // Segmented inclusive scan over lanes; segments are rows (row ids are non-decreasing in lane order).
            const int rr = valid ? static_cast<int>(row_a + q) : 0x7FFFFFFF;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int rp = __shfl_up(rr, d, 64);
                const bool m = lane >= d && rp == rr;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float vp = __shfl_up(v[t], d, 64);
                    v[t] += m ? vp : 0.0f;
                }
            }
            const int rn = __shfl_down(rr, 1, 64);
            const bool seg_end = valid && (lane == 63 || rn != rr);
            if (rr == carry_row) {
#pragma unroll
                for (int t = 0; t < NT; ++t) v[t] += carry[t];
            }
            const long ub = ua + nval;
            const bool row_done = seg_end && (static_cast<long>(rr) + 1) * nu <= ub;
            if (row_done) {
#pragma unroll
                for (int t = 0; t < NT; ++t) ybuf[t * rpw + static_cast<int>(rr - r0)] = v[t];
            }
            if (jobs.amax != nullptr) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    unsigned long long key = row_done ? argmax_key(v[t], rr) : 0ull;
#pragma unroll
                    for (int off = 32; off > 0; off >>= 1) {
                        const unsigned long long o = __shfl_xor(key, off, 64);
                        key = o > key ? o : key;
                    }
                    best[t] = key > best[t] ? key : best[t];
                }
            }
            // The stage's last row continues into the next stage unless it ends here.
            const int lv = nval * LPU - 1;
            const long last_row = __builtin_amdgcn_readlane(rr, lv);
            if ((last_row + 1) * nu > ub) {
                carry_row = last_row;
#pragma unroll
                for (int t = 0; t < NT; ++t) carry[t] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[t]), lv));
            } else {
                carry_row = -1;
            }
            // Advance the stage origin by SU units.
            col_a += SU;
            if (col_a >= nu) {
                const int adv = col_a / nu;
                row_a += adv;
                col_a -= adv * nu;
            }
        }
    };

    // Two stages in flight: RA holds even stages, RB odd ones. Writing a buffer to LDS waits (compiler-
    // inserted vmcnt) for its own loads only; the stage buffer is rewritten after the previous stage's LDS
    // reads were issued, and a wave's LDS operations complete in order.
    // (No exit from the middle of the pair: a path from there back through the latch would look, to the
    // compiler, like RA's loads being the last ones issued.)
    int s = 0;
    if constexpr (G::NB == 1) {
        // One stage in flight: stage s+1 loads while stage s is decoded.
        for (; s + 1 < nst; ++s) {
            store_stage(RA);
            load_stage(s + 1, RA);
            run_stage(s);
        }
    } else {
    for (; s + 1 < nst; s += 2) {
        store_stage(RA);
        load_stage(s + 2 < slast ? s + 2 : slast, RA);
        run_stage(s);
        store_stage(RB);
        load_stage(s + 3 < slast ? s + 3 : slast, RB);
        run_stage(s + 1);
    }
    }
    if (s < nst) {
        store_stage(RA);
        run_stage(s);
    }
    if (y != nullptr) {
        const int nr = static_cast<int>(r1 - r0);
#pragma unroll
        for (int t = 0; t < NT; ++t)
            for (int i = lane; i < nr; i += 64) y[static_cast<size_t>(t) * rows + r0 + i] = ybuf[t * rpw + i];
    }
    if (jobs.amax != nullptr && lane == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) jobs.amax[static_cast<size_t>(t) * jobs.waves + gw] = best[t];
    }
}

// Final argmax over the per-wave keys: one workgroup per token; INT32_MAX when no value qualifies.
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

// Launch geometry of one grouped matvec: rows per wave so that the waves the chip holds at this LDS
// footprint (160 KB per CU, at most 32 waves per CU) cover all rows of all jobs once.
struct Geometry {
    size_t lds;  // dynamic LDS bytes
    int rpw;
    bool few;
};
// Resident workgroups per CU of a qmv_stream_kernel instantiation at `lds` dynamic LDS bytes (VGPR, LDS and
// wave limits, as the runtime computes them); 1 if the query fails.
inline int resident_wgs(const void *kernel, int threads, size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess || n < 1) {
        (void)hipGetLastError();
        return 1;
    }
    return n;
}
template <int T, int N>
Geometry geometry(long total_rows, int cols) {
    using G = Stream<T>;
    Geometry g;
    const int xreg = (N * XImage(cols).bytes + 1023) & ~1023;
    g.lds = static_cast<size_t>(xreg) + static_cast<size_t>(G::NW) * G::WAVE_LDS;
    g.few = (kRowSlots - 1) * ((cols / 32) / Sl<T>::UG) >= G::SU;
    // Both activation forms of the chosen row path: the grid must not depend on the form. Cached per
    // (few, LDS bytes): the occupancy queries cost host time on every launch otherwise.
    static std::mutex mu;
    static std::unordered_map<long, int> cache;
    const long key = static_cast<long>(g.lds) * 2 + (g.few ? 1 : 0);
    long wg_per_cu;
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = cache.find(key);
        if (it == cache.end()) {
            const void *ka = g.few ? reinterpret_cast<const void *>(&qmv_stream_kernel<T, N, true, false>)
                                   : reinterpret_cast<const void *>(&qmv_stream_kernel<T, N, false, false>);
            const void *kb = g.few ? reinterpret_cast<const void *>(&qmv_stream_kernel<T, N, true, true>)
                                   : reinterpret_cast<const void *>(&qmv_stream_kernel<T, N, false, true>);
            (void)raise_dynamic_lds(ka);
            (void)raise_dynamic_lds(kb);
            const int ra = resident_wgs(ka, 64 * G::NW, g.lds), rb = resident_wgs(kb, 64 * G::NW, g.lds);
            it = cache.emplace(key, ra < rb ? ra : rb).first;
        }
        wg_per_cu = it->second;
    }
#ifdef VQ_WGCAP
    if (wg_per_cu > VQ_WGCAP) wg_per_cu = VQ_WGCAP;
#endif
    const long target = 256 * wg_per_cu * G::NW;
    g.rpw = static_cast<int>((total_rows + target - 1) / target);
    if (g.rpw > kYSlots / N) g.rpw = kYSlots / N;  // more than one round of waves for very tall launches
    return g;
}

// Rows per wave for a launch of n jobs (total rows) with N tokens.
template <int T>
int rows_per_wave(long total_rows, int cols, int n_tok) {
    switch (n_tok) {
        case 1: return geometry<T, 1>(total_rows, cols).rpw;
        case 2: return geometry<T, 2>(total_rows, cols).rpw;
        case 3: return geometry<T, 3>(total_rows, cols).rpw;
        case 4: return geometry<T, 4>(total_rows, cols).rpw;
        case 5: return geometry<T, 5>(total_rows, cols).rpw;
        case 6: return geometry<T, 6>(total_rows, cols).rpw;
        case 7: return geometry<T, 7>(total_rows, cols).rpw;
        default: return geometry<T, 8>(total_rows, cols).rpw;
    }
}

// Fills rpw / wave0 / waves of `jobs` (w, y, rows, n set by the caller); returns the wave count.
inline long plan_jobs(QJobs &jobs, int rpw) {
    long waves = 0;
    for (int k = 0; k < jobs.n; ++k) {
        jobs.j[k].rpw = rpw;
        jobs.j[k].wave0 = static_cast<int>(waves);
        waves += (jobs.j[k].rows + rpw - 1) / rpw;
    }
    jobs.waves = static_cast<int>(waves);
    return waves;
}

template <int T, int N, bool XF32>
int launch_stream(const QJobs &jobs, int cols, const void *xp, hipStream_t s) {
    using G = Stream<T>;
    static const int max_dyn_f = raise_dynamic_lds(reinterpret_cast<const void *>(&qmv_stream_kernel<T, N, true, XF32>));
    static const int max_dyn_s = raise_dynamic_lds(reinterpret_cast<const void *>(&qmv_stream_kernel<T, N, false, XF32>));
    const Geometry g = geometry<T, N>(1, cols);
    if (g.lds > static_cast<size_t>(g.few ? max_dyn_f : max_dyn_s)) return static_cast<int>(hipErrorInvalidConfiguration);
    const dim3 grid(static_cast<unsigned>((jobs.waves + G::NW - 1) / G::NW)), block(64 * G::NW);
    if (g.few)
        qmv_stream_kernel<T, N, true, XF32><<<grid, block, g.lds, s>>>(jobs, cols, xp);
    else
        qmv_stream_kernel<T, N, false, XF32><<<grid, block, g.lds, s>>>(jobs, cols, xp);
    return hip_status(hipGetLastError());
}

// Tokens per launch: as many (<= 8) as the activation image budget holds.
inline int token_chunk(int cols) {
    const int chunk = VQ_X_LDS_MAX / XImage(cols).bytes;
    return chunk > 8 ? 8 : chunk < 1 ? 1 : chunk;
}

// Waves of a single-job launch (the argmax key count per token).
template <int T>
long argmax_waves(int rows, int cols, int ntok) {
    const int m = ntok < token_chunk(cols) ? ntok : token_chunk(cols);
    const int rpw = rows_per_wave<T>(rows, cols, m);
    return (rows + rpw - 1) / rpw;
}

// y_j = W_j x for the n jobs (same type and cols), x fp32 (quantized in-kernel) or packed. With `amax`
// ([ntok][argmax_waves] keys, single job), also amax_out[t] = argmax_r y[t][r].
template <int T>
int launch_quant_jobs(int n, const uint8_t *const *w, const int *rows, float *const *y, int cols, const void *x,
                      bool x_f32, int ntok, unsigned long long *amax, int32_t *amax_out, hipStream_t s) {
    if (n < 1 || n > kMaxJobs || (amax && n != 1)) return static_cast<int>(hipErrorInvalidValue);
    const size_t tok_bytes = x_f32 ? static_cast<size_t>(cols) * 4 : static_cast<size_t>(vq_xpack_stride(cols));
    const int chunk = token_chunk(cols);
    long total = 0;
    for (int k = 0; k < n; ++k) total += rows[k];
    const int rpw = rows_per_wave<T>(total, cols, ntok < chunk ? ntok : chunk);
    long kw = 0;
    for (int c = 0; c < ntok; c += chunk) {
        const int m = ntok - c < chunk ? ntok - c : chunk;
        QJobs jobs{};
        jobs.n = n;
        for (int k = 0; k < n; ++k) {
            jobs.j[k].w = w[k];
            jobs.j[k].y = y[k] ? y[k] + static_cast<size_t>(c) * rows[k] : nullptr;
            jobs.j[k].rows = rows[k];
        }
        kw = plan_jobs(jobs, rpw);
        jobs.amax = amax ? amax + static_cast<size_t>(c) * kw : nullptr;
        const void *xp = static_cast<const uint8_t *>(x) + static_cast<size_t>(c) * tok_bytes;
        int st = 0;
#define VQ_CASE(N)                                                                  \
    case N:                                                                         \
        st = x_f32 ? launch_stream<T, N, true>(jobs, cols, xp, s)                   \
                   : launch_stream<T, N, false>(jobs, cols, xp, s);                 \
        break;
        switch (m) {
            VQ_CASE(1) VQ_CASE(2) VQ_CASE(3) VQ_CASE(4) VQ_CASE(5) VQ_CASE(6) VQ_CASE(7)
            default: VQ_CASE(8)
        }
#undef VQ_CASE
        if (st) return st;
    }
    if (amax) {
        argmax_keys_kernel<<<ntok, 256, 0, s>>>(amax, static_cast<int>(kw), amax_out);
        return hip_status(hipGetLastError());
    }
    return 0;
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
#define VQ_INSTANTIATE(T)                                                                                       \
    template int vq::launch_quant<T>(const uint8_t *, int, int, long, const void *, bool, int, float *, hipStream_t); \
    template int vq::launch_quant_jobs<T>(int, const uint8_t *const *, const int *, float *const *, int, const void *, \
                                          bool, int, unsigned long long *, int32_t *, hipStream_t);                 \
    template long vq::argmax_waves<T>(int, int, int);                                                                \
    template int vq::launch_gemm<T>(const uint8_t *, int, int, long, const uint8_t *, int, float *, hipStream_t);    \
    template int vq::launch_mfma<T>(const uint8_t *, int, int, long, const uint8_t *, int, float *, float *,       \
                                    hipStream_t);                                                                \
    template int vq::launch_partials<T>(const uint8_t *, int, int, long, const uint8_t *, int, int32_t *,          \
                                        hipStream_t);                                                            \
    template int vq::launch_dequant<T>(const uint8_t *, int, int, long, float *, hipStream_t);
