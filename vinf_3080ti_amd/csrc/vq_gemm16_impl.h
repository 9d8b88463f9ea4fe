// vq_gemm16_impl.h -- prefill contraction Y[t][r] = W[r] . x[t] on CDNA4 f16 MFMA (v_mfma_f32_16x16x32_f16) for
// the K-quants with mins whose integer sub-block products are exact in f16 and whose blocks are 16-byte multiples
// (Q4_K, Q5_K). Q2_K, Q3_K, Q6_K, IQ2_XXS/XS/S and IQ3_XXS take qgemm16n_kernel (vq_gemm16n_impl.h) with the
// same plan and workspace.
//
// Numerics. The reference CPU path (Cpu_qmv, qwen_cpu.c:581-641) computes per 32-group
//   y += d * sc * xd * S - dmin * m * xd * X,   S = sum(code * xq) exact, X = sum(xq)
// with xq/xd the int8 activation codes and group scale of vq_pack_x. Here every weight element becomes the
// integer a = code * sc (<= 945 for Q4_K, 1953 for Q5_K: exact in f16), every activation element
// b = xq * xd * 2^e (one fp32 rounding; 2^e per token keeps the token in f16 range) as the f16 pair
// b_hi + b_lo (22 significant bits), and each super-block's
//   C = sum_k a * (b_hi + b_lo)   (MFMA products are exact, fp32 accumulation)
// is applied once per 256 elements: acc += d * C - dmin * sum_g m_g * (X_g xd_g 2^e). Only fp32 rounding of
// sums differs from the CPU path (rel-L2 ~2e-7 against its 1e-5 bar); the int8 path (vq_gemm_impl.h) pays a
// VALU scale per 32-group instead, which caps it near 15 % of MFMA peak.
//
// Work split: a workgroup of 8 waves computes a 256-row x 128-token tile over a range of super-blocks (split
// K when the tiles alone would leave CUs idle; partial tiles are added in a fixed order by the library's
// reduction, so results are deterministic). Wave w owns rows 32 w .. +32 and all 128 tokens: 2 x 8 blocks of 16 x
// 16, so every weight row is decoded by one wave (with 64 x 64 per wave, two waves decoded each row: 3-16 %
// slower by type, at half the B-fragment reads). A K step is 64 elements (a quarter super-block). All global data reaches LDS by
// global_load_lds_dwordx4, two steps ahead, into a ring of three step slots (the step's 32 code bytes of
// every row; the tokens' b_hi/b_lo tile, 16-byte chunks XOR-swizzled by row against bank conflicts) and two
// super-block slots (the first 16/48 bytes of every row's block -- d, dmin, scales, Q5_K's high bits -- and
// the tokens' min terms). Every wave issues the same number of DMAs per step, so one vmcnt wait and one
// barrier per step cover the ring. Each wave decodes its own A fragments (code * scale -> f16 via v_perm_b32
// and v_pk_fma_f16) from the raw bytes: 2 x 16 x 2 v_mfma_f32_16x16x32_f16 per step. A
// super-block's min term is one v_mfma_f32_16x16x16_f16 per block over [m_0..m_7, m_0..m_7] x
// [XS_hi_0..7, XS_lo_0..7].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_qmv.h"
#include "vq_tables.h"

namespace vq {

template <int T>
constexpr bool kGemm16 = T == VQ_Q4_K || T == VQ_Q5_K;

constexpr int kG16BM = 256, kG16BN = 128, kG16KS = 64, kG16Waves = 8, kG16Ring = 3;
// 16-row blocks per wave: 2 (a wave owns 32 rows x all 128 tokens of the tile, so each row is decoded by one
// wave) or 4 (64 rows x 64 tokens: two waves decode every row, half the B-fragment reads).
#ifndef VQ_G16_RB
#define VQ_G16_RB 2
#endif
constexpr int kG16RB = VQ_G16_RB;

typedef _Float16 g16h8 __attribute__((ext_vector_type(8)));
typedef _Float16 g16h4 __attribute__((ext_vector_type(4)));
typedef _Float16 g16h2 __attribute__((ext_vector_type(2)));
typedef float g16f4 __attribute__((ext_vector_type(4)));

// Work split: W workgroups each take an equal contiguous share of the U = tiles x super-blocks work units in
// tile-major order (unit u = tile * nsb + sb; workgroup b owns [b U / W, (b+1) U / W)). A workgroup that covers a
// whole tile writes y; the parts of a tile split between workgroups go to slots [tile][k] (k = the workgroup's
// order among the tile's) that vq_gemm16_reduce adds in slot order (deterministic). Two plans:
//  - default: with more tiles than CUs, W = CUs: each workgroup first takes `rounds` = tiles / CUs whole tiles
//    (units [b rounds nsb, (b+1) rounds nsb), written straight to y), then an equal contiguous share of the
//    remaining tiles' units (stream-K over the last tiles % CUs tiles: only those have parts to add; when they
//    hold fewer units than CUs, stream-K over every unit instead). Else W is the largest multiple of the tile
//    count that fits the CUs (plain split-K). The split depends on M.
//  - batch-invariant: every tile's super-blocks are cut at the same P - 1 boundaries (P = CUs / row tiles,
//    rounded, at most nsb), W = tiles x P. P depends only on the matrix, so a token's result is the same whatever
//    batch it runs in (the reference's contract for its prompt kernels, qwen_runtime.cu:1883-1885), at 10-20 %
//    more time at 512 tokens (more partial tiles to add).
struct G16Plan {
    int tiles, ntt, nrt, nsb, W, per_xcd, maxseg;
    int rounds, t0;  // whole tiles per workgroup; t0 = W rounds tiles taken whole (0: all units shared)
    long U, D;       // units; D = t0 nsb units of the whole tiles
    // Tile order: token-tile major (tile = tt * nrt + rt), so the workgroups of one XCD (consecutive shares) work
    // on one token tile, whose activation tile then stays in that XCD's L2.
    __host__ __device__ int tile_rt(int tile) const { return tile % nrt; }
    __host__ __device__ int tile_tt(int tile) const { return tile / nrt; }
    __host__ __device__ int wg_of(long u) const {  // owner of unit u
        return u < D ? static_cast<int>(u / nsb / rounds) : static_cast<int>(((u - D + 1) * W - 1) / (U - D));
    }
    __host__ __device__ long u0(int b) const { return D + static_cast<long>(b) * (U - D) / W; }  // shared units
    __host__ __device__ long dp0(int b) const { return static_cast<long>(b) * rounds * nsb; }  // whole tiles
    __host__ __device__ long dp1(int b) const { return D ? dp0(b + 1) : 0; }
};
inline G16Plan g16_plan(int rows, int cols, int M, int cus, bool invariant = false) {
    G16Plan p{};
    p.ntt = (M + kG16BN - 1) / kG16BN;
    const int row_tiles = (rows + kG16BM - 1) / kG16BM;
    p.nrt = row_tiles;
    p.tiles = row_tiles * p.ntt;
    p.nsb = cols >> 8;
    p.U = static_cast<long>(p.tiles) * p.nsb;
    p.rounds = 1;
    if (invariant) {
        int P = (cus + row_tiles / 2) / row_tiles;
        P = P < 1 ? 1 : P > p.nsb ? p.nsb : P;
        p.W = p.tiles * P;
        p.per_xcd = (p.W + 7) / 8;
        p.maxseg = P;
        return p;
    }
    // Fewer tiles than CUs: an equal whole number of workgroups per tile (each tile splits at super-block
    // boundaries into that many segments, no workgroup straddles two tiles), unless that leaves more than a
    // tenth of the CUs idle (160 tiles: one workgroup each, 62 % of 256 CUs); then, as for many tiles, one
    // workgroup per CU with stream-K shares, as long as every CU still gets at least one super-block of work.
    if (p.tiles <= cus) {
        const int per = cus / p.tiles < p.nsb ? cus / p.tiles : p.nsb;
        p.W = p.tiles * per;
        if (p.W * 10 < cus * 9 && p.U >= cus) p.W = cus;
    } else {
        p.W = cus;
        const int rem = p.tiles % cus;
        if (rem == 0 || static_cast<long>(rem) * p.nsb >= cus) {
            p.rounds = p.tiles / cus;
            p.t0 = p.rounds * cus;
            p.D = static_cast<long>(p.t0) * p.nsb;
        }
    }
    p.per_xcd = (p.W + 7) / 8;
    const long share = (p.U - p.D) / p.W;  // >= 1 unless every tile is whole
    p.maxseg = share ? static_cast<int>((p.nsb + share - 1) / share + 1) : 1;
    return p;
}

// Workspace layout of the f16 path for M tokens of `cols` columns: b_hi [M][cols] f16, b_lo [M][cols] f16,
// xs [M][cols/256][16] f16 (per super-block: X_g xd_g 2^e / 32 as 8 hi then 8 lo; for Q2_K, whose mins apply per
// 16 elements, [M][cols/256][32]: the 16 halves' X_h xd 2^e / 32 as 16 hi then 16 lo), inv [M] fp32 (2^-e),
// then the partial-tile slots [tiles - t0][maxseg][64 values][512 threads] fp32.
constexpr size_t kG16TileFloats = static_cast<size_t>(kG16BM) * kG16BN;
struct G16Ws {
    size_t bh, bl, xs, inv, part, total;
};
inline G16Ws g16_layout(int cols, int M, const G16Plan &p, bool halves = false) {
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    G16Ws l{};
    const size_t nb = static_cast<size_t>(M) * cols * 2;
    l.bh = 0;
    l.bl = al(nb);
    l.xs = l.bl + al(nb);
    l.inv = l.xs + al(static_cast<size_t>(M) * (cols / 256) * (halves ? 64 : 32));
    l.part = l.inv + al(static_cast<size_t>(M) * 4);
    l.total = l.part + al(static_cast<size_t>(p.tiles - p.t0) * p.maxseg * kG16TileFloats * 4);
    return l;
}

// Two f16 (1024 + c) from bytes of a code word (c < 256): v_perm_b32 puts 0x64 above each byte.
__device__ __forceinline__ g16h2 g16_pair(uint32_t codes, uint32_t sel) {
    return __builtin_bit_cast(g16h2, __builtin_amdgcn_perm(0x64646464u, codes, sel));
}
// Eight codes (bytes of c0, c1, each < 64) times sc as the f16 fragment: (1024 + c) sc - 1024 sc in one rounding
// (v_pk_fma_f16), exact because c sc is.
__device__ __forceinline__ g16h8 g16_frag(uint32_t c0, uint32_t c1, _Float16 sc) {
    const g16h2 s2 = {sc, sc};
    const _Float16 nb = static_cast<_Float16>(-1024.0f) * sc;  // exact: sc < 64
    const g16h2 n2 = {nb, nb};
    const g16h2 p0 = __builtin_elementwise_fma(g16_pair(c0, 0x04010400u), s2, n2);
    const g16h2 p1 = __builtin_elementwise_fma(g16_pair(c0, 0x04030402u), s2, n2);
    const g16h2 p2 = __builtin_elementwise_fma(g16_pair(c1, 0x04010400u), s2, n2);
    const g16h2 p3 = __builtin_elementwise_fma(g16_pair(c1, 0x04030402u), s2, n2);
    return g16h8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// LO: activations as b_hi + b_lo (the int8 path's values, exact); without it b_hi alone (activations rounded to
// f16 under the token's 2^e, the reference's tensor-core numerics): half the activation DMA, LDS and MFMAs.
template <int T, bool LO = true>
struct G16Geo {
    static constexpr int UB = Sl<T>::UB;
    static constexpr int HB = T == VQ_Q5_K ? 48 : 16;          // leading block bytes kept per super-block
    static constexpr int QOFF = T == VQ_Q5_K ? 48 : 16;        // offset of qs in the block
    static constexpr int SB_CHUNKS = kG16BM * HB / 16 + kG16BN * 2;  // 16-byte chunks of a super-block slot
    static constexpr int SB_DMA = SB_CHUNKS / (64 * kG16Waves);      // per wave, first step of a super-block
    static constexpr int NB = LO ? 4 : 2;                            // activation DMAs per wave and step
    static constexpr int NDMA = 1 + NB;                              // per wave, every step
    static constexpr int NDMA_SB = NDMA + SB_DMA;                    // per wave, first step of a super-block
    static constexpr int STEP_BYTES = kG16BM * 32 + (LO ? 2 : 1) * kG16BN * 128;  // codes + b_hi (+ b_lo)
    static constexpr int SB_BYTES = SB_CHUNKS * 16;
    static_assert(SB_CHUNKS % (64 * kG16Waves) == 0, "super-block slot split");
};

template <int T, bool LO>
__global__ __launch_bounds__(64 * kG16Waves) void qgemm16_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                                  long row_bytes, const _Float16 *__restrict__ bh,
                                                                  const _Float16 *__restrict__ bl,
                                                                  const _Float16 *__restrict__ xs,
                                                                  const float *__restrict__ inv, int M, G16Plan pl,
                                                                  float *__restrict__ y, float *__restrict__ part) {
    using G = G16Geo<T, LO>;
    __shared__ __attribute__((aligned(1024))) uint8_t s_step[kG16Ring][G::STEP_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t s_sb[2][G::SB_BYTES];

    // Workgroup id -> share: consecutive ids go round-robin over the 8 XCDs; the ids one XCD receives own
    // consecutive shares, i.e. a contiguous range of tiles: row tiles of one token tile, which share its
    // activations in that XCD's L2 (G16Plan's tile order).
    const int b = blockIdx.x;
    const int v = (b & 7) * pl.per_xcd + (b >> 3);
    if (v >= pl.W) return;
    const int nsb = pl.nsb;
    // The workgroup's whole tiles, then its share of the others.
    long ue = pl.dp1(v), u = pl.dp0(v);
    bool whole = u < ue;
    if (!whole) u = pl.u0(v), ue = pl.u0(v + 1);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    constexpr int RB = kG16RB, TB = 16 / RB;  // 16-row blocks x 16-token blocks of a wave
    const int wr = 16 * RB * (wv % (16 / RB)), wt = 16 * TB * (wv / (16 / RB));
    const int lr = lane & 15, lk = lane >> 4;
    // The share's tile segments: tile t, super-blocks [sb0, sb1).
    while (u < ue) {
    const int tile = static_cast<int>(u / nsb);
    const int sb0 = static_cast<int>(u - static_cast<long>(tile) * nsb);
    const int sb1 = ue - u < nsb - sb0 ? sb0 + static_cast<int>(ue - u) : nsb;
    const int rt = pl.tile_rt(tile), tt = pl.tile_tt(tile);
    const int r0 = rt * kG16BM, t0 = tt * kG16BN;
    const int nsteps = (sb1 - sb0) * 4;
    const uint8_t *const wbase = w + static_cast<size_t>(r0) * row_bytes;  // wave-uniform

    // Lane offsets of the DMAs, fixed for the segment (the step moves only the wave-uniform base, so a copy costs
    // no VALU): the wave's code row piece, its four activation chunks, and its super-block slot chunks.
    uint32_t vo_code, vo_b[G::NB], vo_sb[G::SB_DMA];
    {
        const int row = min(r0 + 32 * wv + (lane >> 1), rows - 1) - r0;
        // The row's two 16-byte halves in swapped order when bit 3 of its tile row is set (rows R and R + 8
        // would read the same LDS banks at the 32-byte row pitch).
        const int rr = 32 * wv + (lane >> 1);
        vo_code = static_cast<uint32_t>(row * row_bytes + G::QOFF + 16 * ((lane & 1) ^ ((rr >> 3) & 1)));
#pragma unroll
        for (int k = 0; k < G::NB; ++k) {
            const int ii = (G::NB * wv + k) & 15;
            const int trow = 8 * ii + (lane >> 3);
            const int tok = min(t0 + trow, M - 1);
            const int c = (lane & 7) ^ ((trow >> 1) & 7);
            vo_b[k] = static_cast<uint32_t>((static_cast<long>(tok) * cols + 8 * c) * 2);
        }
#pragma unroll
        for (int k = 0; k < G::SB_DMA; ++k) {
            const int i = G::SB_DMA * wv + k;
            const int ci = 64 * i + lane;
            constexpr int CH = G::HB / 16, NHC = kG16BM * G::HB / 16;
            if (i * 64 < NHC) {
                const int hrow = min(r0 + ci / CH, rows - 1) - r0;
                vo_sb[k] = static_cast<uint32_t>(hrow * row_bytes + 16 * (ci % CH));
            } else {
                const int cj = ci - NHC;
                const int tok = min(t0 + (cj >> 1), M - 1);
                vo_sb[k] = static_cast<uint32_t>((static_cast<long>(tok) * nsb * 16 + 8 * (cj & 1)) * 2);
            }
        }
    }
    // DMA of step st (j = st % 4 of super-block sb0 + st / 4) into ring slot st % 3 and super-block slot sb & 1.
    // Per wave: codes (rows 32 wv .. +32, two lanes per row), 4 of the 32 KB of b_hi/b_lo (8 tokens per 1 KB,
    // chunk position p of token row r holds chunk p ^ ((r >> 1) & 7): the 16 rows an MFMA fragment reads then
    // hit 16 distinct 16-byte bank groups), and on a super-block's first step SB_DMA KB of its slot.
    auto issue = [&](int st) {
        const int sb = sb0 + (st >> 2), j = st & 3;
        uint8_t *const slot = s_step[st % kG16Ring];
        dma16s(wbase + static_cast<long>(sb) * G::UB + 32 * j, vo_code, slot + 1024 * wv);
        const long kb = (256L * sb + 64 * j) * 2;  // the step's byte offset in a token row of b_hi / b_lo
#pragma unroll
        for (int k = 0; k < G::NB; ++k) {
            const int i = G::NB * wv + k, ii = i & 15;
            dma16s(reinterpret_cast<const uint8_t *>(i < 16 ? bh : bl) + kb, vo_b[k],
                   slot + kG16BM * 32 + (i < 16 ? 0 : kG16BN * 128) + 1024 * ii);
        }
        if (j != 0) return;  // the super-block slot: once, with the super-block's first step
        uint8_t *const sbs = s_sb[sb & 1];
#pragma unroll
        for (int k = 0; k < G::SB_DMA; ++k) {
            const int i = G::SB_DMA * wv + k;
            constexpr int NHC = kG16BM * G::HB / 16;
            if (i * 64 < NHC)
                dma16s(wbase + static_cast<long>(sb) * G::UB, vo_sb[k], sbs + 1024 * i);
            else
                dma16s(reinterpret_cast<const uint8_t *>(xs) + sb * 32, vo_sb[k], sbs + 1024 * i);
        }
    };

    g16f4 acc[RB][TB], C[RB][TB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int q = 0; q < TB; ++q) acc[i][q] = C[i][q] = g16f4{0.f, 0.f, 0.f, 0.f};

    if (nsteps > 0) issue(0);
    if (nsteps > 1) issue(1);
    uint32_t scl[RB] = {}, sch[RB] = {};  // [rb]: 6-bit scales of groups 0..3 / 4..7 of
                                                                      // row wr + 16 rb + lr, one per byte
    const g16h2 k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    for (int st = 0; st < nsteps; ++st) {
        // Step st landed when at most the next step's DMAs are outstanding (loads retire in order).
        if (st + 1 >= nsteps)
            wait_vm<0>();
        else if (((st + 1) & 3) == 0)
            wait_vm<G::NDMA_SB>();
        else
            wait_vm<G::NDMA>();
        __syncthreads();  // step st landed for every wave; step st - 1's slot is free
        if (st + 2 < nsteps) issue(st + 2);
        const int sb = sb0 + (st >> 2), j = st & 3;
        const uint8_t *const slot = s_step[st % kG16Ring];
        const uint8_t *const sbs = s_sb[sb & 1];
        const uint8_t *const sBh = slot + kG16BM * 32, *const sBl = sBh + kG16BN * 128;
        if (j == 0) {
            // The super-block's 6-bit scales, four per dword (the k4_scale_min packing, qwen_cpu.c:54-62):
            // groups 0..3 from scales[0..3], groups 4..7 from scales[8..11] plus the top bits of scales[0..3].
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const uint4 h = *reinterpret_cast<const uint4 *>(sbs + (wr + 16 * rb + lr) * G::HB);
                scl[rb] = h.y & 0x3F3F3F3Fu;
                sch[rb] = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
            }
        }
        // A fragments: rows wr + 16 rb + lr, elements 8 lk .. +8 of groups 2j (c = 0) and 2j + 1 (c = 1).
        const uint32_t ssel = (j & 1) ? 0x04030402u : 0x04010400u;
        g16h8 a[2][RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = wr + 16 * rb + lr;
            const uint32_t sw = j < 2 ? scl[rb] : sch[rb];
            const g16h2 sc = g16_pair(sw, ssel) - k1024;
            const uint2 q = *reinterpret_cast<const uint2 *>(slot + row * 32 + 16 * ((lk >> 1) ^ ((row >> 3) & 1)) + 8 * (lk & 1));
            uint32_t lo0 = q.x & 0x0F0F0F0Fu, lo1 = q.y & 0x0F0F0F0Fu;
            uint32_t hi0 = (q.x >> 4) & 0x0F0F0F0Fu, hi1 = (q.y >> 4) & 0x0F0F0F0Fu;
            if constexpr (T == VQ_Q5_K) {
                const uint2 qh = *reinterpret_cast<const uint2 *>(sbs + row * G::HB + 16 + 8 * lk);
                lo0 |= ((qh.x >> (2 * j)) & 0x01010101u) << 4;
                lo1 |= ((qh.y >> (2 * j)) & 0x01010101u) << 4;
                hi0 |= ((qh.x >> (2 * j + 1)) & 0x01010101u) << 4;
                hi1 |= ((qh.y >> (2 * j + 1)) & 0x01010101u) << 4;
            }
            a[0][rb] = g16_frag(lo0, lo1, sc[0]);
            a[1][rb] = g16_frag(hi0, hi1, sc[1]);
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int h = 0; h < TB / 4; ++h) {  // token blocks four at a time (B fragments' registers)
                g16h8 bhf[4], blf[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = wt + 16 * (4 * h + i) + lr;
                    const int o = r * 128 + (((4 * c + lk) ^ ((r >> 1) & 7)) << 4);
                    bhf[i] = *reinterpret_cast<const g16h8 *>(sBh + o);
                    if constexpr (LO) blf[i] = *reinterpret_cast<const g16h8 *>(sBl + o);
                }
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        g16f4 &cc = C[rb][4 * h + i];
                        cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c][rb], bhf[i], cc, 0, 0, 0);
                        if constexpr (LO) cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c][rb], blf[i], cc, 0, 0, 0);
                    }
            }
        }
        if (j == 3) {
            // Super-block end: acc += d C - 32 dmin (m . XS); C restarts at zero. C element q of a block is row
            // 4 lk + q, token lr.
            const uint8_t *const sxs = sbs + kG16BM * G::HB;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float dq[4], mq[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t hd = *reinterpret_cast<const uint32_t *>(sbs + (wr + 16 * rb + 4 * lk + q) * G::HB);
                    dq[q] = half_to_float(hd);
                    mq[q] = 32.0f * half_to_float(hd >> 16);
                }
                // A_min fragment: row wr + 16 rb + lr, k = 4 lk .. +4 -> mins of groups 4 (lk & 1) .. +4.
                const uint4 h = *reinterpret_cast<const uint4 *>(sbs + (wr + 16 * rb + lr) * G::HB);
                const uint32_t mw = (lk & 1) ? (((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u)) : (h.z & 0x3F3F3F3Fu);
                const g16h2 m01 = g16_pair(mw, 0x04010400u) - k1024, m23 = g16_pair(mw, 0x04030402u) - k1024;
                const g16h4 amin = {m01[0], m01[1], m23[0], m23[1]};
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
                    const g16h4 bm = *reinterpret_cast<const g16h4 *>(sxs + (wt + 16 * tb + lr) * 32 + 8 * lk);
                    const g16f4 cm = __builtin_amdgcn_mfma_f32_16x16x16f16(amin, bm, g16f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[rb][tb][q] = fmaf(dq[q], C[rb][tb][q], fmaf(-mq[q], cm[q], acc[rb][tb][q]));
                    C[rb][tb] = g16f4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    }

    // Output: element q of block (rb, tb) is row r0 + wr + 16 rb + 4 lk + q, token t0 + wt + 16 tb + lr; values
    // leave the 2^e token scale here. A whole tile goes to y (four rows per 16-byte store where rows allow); a
    // part of a tile to its slot, in thread order (coalesced: value i of thread x at [i][x]).
    if (sb0 == 0 && sb1 == nsb) {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const int t = t0 + wt + 16 * tb + lr;
            if (t >= M) continue;
            const float is = inv[t];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int r = r0 + wr + 16 * rb + 4 * lk;
                float *const dst = y + static_cast<size_t>(t) * rows + r;
                if ((rows & 3) == 0 && r + 3 < rows) {
                    *reinterpret_cast<float4 *>(dst) = float4{acc[rb][tb][0] * is, acc[rb][tb][1] * is, acc[rb][tb][2] * is, acc[rb][tb][3] * is};
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (r + q < rows) dst[q] = acc[rb][tb][q] * is;
                }
            }
        }
    } else {
        const int k = v - pl.wg_of(static_cast<long>(tile) * nsb);
        float *const slot = part + (static_cast<size_t>(tile - pl.t0) * pl.maxseg + k) * kG16TileFloats;
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const int t = min(t0 + wt + 16 * tb + lr, M - 1);
            const float is = inv[t];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int q = 0; q < 4; ++q) slot[static_cast<size_t>((rb * TB + tb) * 4 + q) * 512 + tid] = acc[rb][tb][q] * is;
        }
    }
    __syncthreads();  // the ring is reused by the next segment's first DMAs
    u += sb1 - sb0;
    if (whole && u >= ue) whole = false, u = pl.u0(v), ue = pl.u0(v + 1);
    }
}

// Partial tiles: y = the sum of a tile's slots in slot order. Workgroup (tile, block pair (rb, tb)) of 512
// threads, thread x summing the four values the GEMM's thread x held for that pair (independent loads, so the
// slots stream); tiles that one workgroup covered are already in y. RB: the GEMM's 16-row blocks per wave (4: 64
// rows x 64 tokens per wave; 2: 32 rows x 128 tokens).
template <int RB = 4>
__global__ __launch_bounds__(512) void g16_reduce_kernel(const float *__restrict__ part, G16Plan pl, int rows, int M,
                                                         float *__restrict__ y) {
    const int tile = pl.t0 + (blockIdx.x >> 4), pair = blockIdx.x & 15;
    const int k0 = pl.wg_of(static_cast<long>(tile) * pl.nsb), k1 = pl.wg_of(static_cast<long>(tile) * pl.nsb + pl.nsb - 1);
    if (k1 == k0) return;
    constexpr int TB = 16 / RB;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wr = 16 * RB * (wv % (16 / RB)), wt = 16 * TB * (wv / (16 / RB)), lr = lane & 15, lk = lane >> 4;
    const int rb = pair / TB, tb = pair % TB;
    const int rt = pl.tile_rt(tile), tt = pl.tile_tt(tile);
    const int t = tt * kG16BN + wt + 16 * tb + lr, r = rt * kG16BM + wr + 16 * rb + 4 * lk;
    const float *const base = part + static_cast<size_t>(tile - pl.t0) * pl.maxseg * kG16TileFloats +
                              static_cast<size_t>((rb * TB + tb) * 4) * 512 + tid;
    float v4[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k <= k1 - k0; ++k) {
        const float *const sk = base + static_cast<size_t>(k) * kG16TileFloats;
        const float a0 = sk[0], a1 = sk[512], a2 = sk[1024], a3 = sk[1536];
        v4[0] += a0;
        v4[1] += a1;
        v4[2] += a2;
        v4[3] += a3;
    }
    if (t >= M) return;
    float *const dst = y + static_cast<size_t>(t) * rows + r;
    if ((rows & 3) == 0 && r + 3 < rows) {
        *reinterpret_cast<float4 *>(dst) = float4{v4[0], v4[1], v4[2], v4[3]};
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (r + q < rows) dst[q] = v4[q];
    }
}

// Q2_K, Q3_K, Q6_K, IQ2_XXS/XS/S and IQ3_XXS: qgemm16n_kernel (vq_gemm16n_impl.h), same plan, workspace and reduction.
template <int T>
int launch_gemm16n(const uint8_t *w, int rows, int cols, long rb, const void *ws, int M, float *y, int cus,
                   hipStream_t s, bool invariant, bool f16x);

// f16x: b_hi alone holds the activations (rounded to f16).
template <int T>
int launch_gemm16(const uint8_t *w, int rows, int cols, long rb, const void *ws, int M, float *y, int cus,
                  hipStream_t s, bool invariant, bool f16x) {
    if constexpr (T == VQ_Q2_K || T == VQ_Q3_K || T == VQ_Q6_K || T == VQ_IQ2_XS || T == VQ_IQ2_XXS ||
                  T == VQ_IQ2_S || T == VQ_IQ3_XXS) {
        return launch_gemm16n<T>(w, rows, cols, rb, ws, M, y, cus, s, invariant, f16x);
    } else if constexpr (!kGemm16<T>) {
        (void)w, (void)rows, (void)cols, (void)rb, (void)ws, (void)M, (void)y, (void)cus, (void)s, (void)invariant,
            (void)f16x;
        return static_cast<int>(hipErrorInvalidValue);
    } else {
        const G16Plan pl = g16_plan(rows, cols, M, cus, invariant);
        const G16Ws l = g16_layout(cols, M, pl);
        uint8_t *base = static_cast<uint8_t *>(const_cast<void *>(ws));
        float *const part = reinterpret_cast<float *>(base + l.part);
        auto *const kern = f16x ? qgemm16_kernel<T, false> : qgemm16_kernel<T, true>;
        kern<<<dim3(8 * pl.per_xcd), dim3(64 * kG16Waves), 0, s>>>(
            w, rows, cols, rb, reinterpret_cast<const _Float16 *>(base + l.bh),
            reinterpret_cast<const _Float16 *>(base + l.bl), reinterpret_cast<const _Float16 *>(base + l.xs),
            reinterpret_cast<const float *>(base + l.inv), M, pl, y, part);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return static_cast<int>(e);
        if (pl.tiles > pl.t0) g16_reduce_kernel<kG16RB><<<dim3(16 * (pl.tiles - pl.t0)), dim3(512), 0, s>>>(part, pl, rows, M, y);
        e = hipGetLastError();
        return e == hipSuccess ? 0 : static_cast<int>(e);
    }
}

}  // namespace vq
