// vq_gemm16n_impl.h -- prefill contraction on CDNA4 f16 MFMA for Q2_K, Q3_K, Q6_K, IQ2_XXS/XS/S and IQ3_XXS: blocks
// (84, 110, 210, 66, 74, 82 and 98 bytes) only 2- or 4-byte aligned inside a row.
//
// Numerics: those of the Q4_K/Q5_K contraction (vq_gemm16_impl.h). Each weight element is the integer
// a = code * sc: (q3) * (sc - 32), |a| <= 128, for Q3_K; q2 * sc, |a| <= 45, for Q2_K; grid * sign * (2 s + 1),
// |a| <= 43 * 31, for the IQ2 types (d / 8 applied per super-block) and <= 62 * 31 for IQ3_XXS (d / 4); Q6_K's
// (q - 32) * sc (|.| <= 4096, past f16's exact integers) as its f16 rounding p and the exact remainder a - p in
// {-1, 0, 1} (s16_frag), three MFMAs per product: p b_hi + p b_lo + r b_hi (r b_lo, under ~1e-7 of it, left out). Each
// activation element is
// b = xq * xd * 2^e as the f16 pair b_hi + b_lo, and each super-block's C = sum a * (b_hi + b_lo) (exact products,
// fp32 sums) is applied once: acc += d * C, for Q2_K minus 32 dmin (m . XS) with the 16 sub-blocks' mins m and
// XS_h = X_h xd 2^e / 32 (X_h the code sum of 16-element half h; qwen_cpu.c:205-230) as one
// v_mfma_f32_16x16x16_f16 per hi and lo part (qwen_cpu.c:581-641 regrouped per super-block).
//
// Work split, tiles and reduction: those of qgemm16_kernel (G16Plan; 256-row x 128-token tiles, 8 waves of 32
// rows x 128 tokens). Differences:
//  - K order. A step is 64 elements of one super-block, but not 64 consecutive ones: step j = 2n + p takes the
//    elements 128 n + 32 k + 16 p + i (k = 0..3, i = 0..15). The types store element 128 n + 32 k + l as a field
//    of byte l of a 32-byte run (Q6_K: low/high nibble of ql[64 n + 32 (k & 1) + l] and bits 2k of qh[32 n + l];
//    Q3_K: bits 2k of qs[32 n + l] and bit 4n + k of hmask[l]; Q2_K: bits 2k of qs[32 n + l]) and scale it by scale
//    8 n + 2 k + p, so a step needs one 16-byte piece of each run per row (Q6_K: 2 of ql, 1 of qh; Q3_K: 1 of qs,
//    1 of hmask; Q2_K: 1 of qs) and every
//    16-element run of it has one scale. MFMA lane (lr, lk) with chunk c holds k = 2c + (lk >> 1), i = 8 (lk & 1)
//    .. +8; the activation tile of the step is DMA'd in that same permuted order.
//  - Alignment. A piece starts m = (row offset of the block) mod 16 bytes past a 16-byte boundary (m even), so
//    each piece is DMA'd as the 16-byte-aligned pair of chunks covering it (the second one only when m > 0;
//    otherwise the first is fetched twice) and read from LDS as three dwords realigned by v_alignbyte. The scales
//    and d of every row come the same way, once per super-block (Q2_K: two chunk pairs, its 16 scale bytes at the
//    block's start and d, dmin at byte 80; with its XS tile). No read goes past the 16 bytes of padding that
//    follow the tensor.
//  - Two step slots (one step of lead): with three, the chunk pairs and the activation tiles would not fit LDS.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_gemm16_impl.h"
#include "vq_small16_impl.h"

namespace vq {

// LO as for qgemm16_kernel: activations as b_hi + b_lo, or b_hi alone (rounded to f16).
template <int T, bool LO = true>
struct G16N {
    static constexpr bool Q6 = T == VQ_Q6_K, Q2 = T == VQ_Q2_K;
    static constexpr bool IQX = T == VQ_IQ2_XXS;     // scales inside the code pieces
    static constexpr bool IQS = T == VQ_IQ2_S;       // three pieces: grid index bytes, sign bytes, high index bits
    static constexpr bool IQ3X = T == VQ_IQ3_XXS;    // two pieces: grid index bytes, (signs, scale) words
    static constexpr bool IQ = T == VQ_IQ2_XS || IQX || IQS || IQ3X;  // consecutive elements, grid codes, no mins
    static constexpr bool DONLY = IQX || IQ3X;       // scales in the code pieces: the super-block slot holds d only
    static constexpr int UB = Q6 ? 210 : Q2 ? 84 : IQX ? 66 : IQS ? 82 : IQ3X ? 98 : IQ ? 74 : 110;
    static constexpr int NPC = Q6 || IQS ? 3 : Q2 || IQX || T == VQ_IQ2_XS ? 1 : 2;  // 16-byte pieces per row and step
    static constexpr int CPR = 2 * NPC;              // chunks DMA'd per row and step
    static constexpr int SOFF = Q6 ? 192 : Q2 || DONLY ? 0 : IQS ? 74 : IQ ? 66 : 96;  // scales (Q3_K, Q6_K: d
                                                                                         // after them; DONLY: d)
    static constexpr int SLEN = Q6 ? 18 : Q2 ? 16 : DONLY ? 2 : IQ ? 8 : 14;   // bytes from SOFF
    static constexpr int DOFF = Q6 ? 208 : Q2 ? 80 : IQ ? 0 : 108;  // d (Q2_K: then dmin)
    static constexpr int POFF0 = IQ ? 2 : 0;         // the code pieces' offset mod 16 in the block
    static constexpr int SBR = Q2 || (IQ && !DONLY) ? 64 : 32;  // super-block slot bytes per row: chunk pairs
    static constexpr int CODE_BYTES = kG16BM * CPR * 16;
    static constexpr int NB = LO ? 4 : 2;  // activation DMAs per wave and step
    static constexpr int STEP_BYTES = CODE_BYTES + (LO ? 2 : 1) * kG16BN * 128;
    static constexpr int XS_BYTES = Q2 ? kG16BN * 64 : 0;  // the tokens' XS (16 hi, 16 lo f16 each)
    static constexpr int SB_BYTES = kG16BM * SBR + XS_BYTES;
    static constexpr int SB_DMA = SB_BYTES / (1024 * kG16Waves);  // per wave, first step of a super-block
    static constexpr int CODE_DMA = CPR / 2;         // per wave and step: 32 rows x CPR chunks
    static_assert(SB_BYTES % (1024 * kG16Waves) == 0, "super-block slot split");
    // Block offset of piece pc of step (n, p).
    __device__ static int poff(int pc, int n, int p) {
        if constexpr (Q6)
            return pc == 2 ? 128 + 32 * n + 16 * p : 64 * n + 32 * pc + 16 * p;
        else if constexpr (Q2)
            return 16 + 32 * n + 16 * p;
        else if constexpr (IQ3X)  // step j = 2 n + p: qs[16 j .. +16], aux[2 j .. +2]
            return pc == 0 ? 2 + 16 * (2 * n + p) : 66 + 8 * (2 * n + p);
        else if constexpr (IQS)  // step j = 2 n + p: qs[8 j .. +8], signs[8 j .. +8], qh[2 j .. +2]
            return pc == 0 ? 2 + 8 * (2 * n + p) : pc == 1 ? 34 + 8 * (2 * n + p) : 66 + 2 * (2 * n + p);
        else if constexpr (IQ)
            return 2 + 32 * n + 16 * p;  // qs entries 8 j .. 8 j + 7 of step j = 2 n + p
        else
            return pc == 0 ? 32 + 32 * n + 16 * p : 16 * p;
    }
    // Q3_K's two pieces of row R sit in the step slot in swapped order when bit 2 of R is set: with its 64-byte
    // row pitch, rows R and R + 4 would otherwise read the same banks.
    __device__ static int pslot(int pc, int R) { return Q6 || Q2 || IQ ? pc : pc ^ ((R >> 2) & 1); }
    // Super-block element of MFMA chunk q = 4 c + lk of step j (IQ2_XS: in order, 64 j + 8 q).
    __device__ static int bpos(int j, int q) {
        if constexpr (IQ) return 64 * j + 8 * q;
        return 128 * (j >> 1) + 32 * (2 * (q >> 2) + ((q & 3) >> 1)) + 16 * (j & 1) + 8 * (q & 1);
    }
};

// Eight bytes at LDS byte offset `off` (even) of `base` (4-byte aligned): three dwords, realigned.
__device__ __forceinline__ uint2 g16n_read8(const uint8_t *base, int off) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(base + (off & ~3));
    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2], sh = static_cast<uint32_t>(off & 3);
    return uint2{__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh)};
}

template <int T, bool LO>
__global__ __launch_bounds__(64 * kG16Waves) void qgemm16n_kernel(const uint8_t *__restrict__ w, int rows, int cols,
                                                                   long row_bytes, const _Float16 *__restrict__ bh,
                                                                   const _Float16 *__restrict__ bl,
                                                                   const _Float16 *__restrict__ xs,
                                                                   const float *__restrict__ inv, int M, G16Plan pl,
                                                                   float *__restrict__ y, float *__restrict__ part) {
    using G = G16N<T, LO>;
    __shared__ __attribute__((aligned(1024))) uint8_t s_step[2][G::STEP_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t s_sb[2][G::SB_BYTES];
    // IQ2_XS: its grid and sign-selector tables in LDS (the first step's barrier orders them before any read).
    __shared__ uint2 s8[TabSpec<T>::n8 > 0 ? TabSpec<T>::n8 : 1];
    __shared__ uint32_t s4[TabSpec<T>::n4 > 0 ? TabSpec<T>::n4 : 1];
    __shared__ uint2 sks[TabSpec<T>::ks || G::IQ3X ? 128 : 1];
    Tabs tb = stage_tabs<T>(s8, s4, sks, nullptr);
    if constexpr (G::IQ3X) {  // the sign selectors (the streaming kernel decodes IQ3_XXS signs in registers)
        for (int i = threadIdx.x; i < 128; i += blockDim.x) sks[i] = sign_entry(ksigns(i));
        tb.ks128 = sks;
    }

    const int b = blockIdx.x;
    const int v = (b & 7) * pl.per_xcd + (b >> 3);  // XCD-aware share order, as qgemm16_kernel
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
    while (u < ue) {
    const int tile = static_cast<int>(u / nsb);
    const int sb0 = static_cast<int>(u - static_cast<long>(tile) * nsb);
    const int sb1 = ue - u < nsb - sb0 ? sb0 + static_cast<int>(ue - u) : nsb;
    const int rt = pl.tile_rt(tile), tt = pl.tile_tt(tile);
    const int r0 = rt * kG16BM, t0 = tt * kG16BN;
    const int nsteps = (sb1 - sb0) * 4;
    const uint8_t *const wbase = w + static_cast<size_t>(r0) * row_bytes;  // 16-byte aligned (r0 % 256 == 0)
    // Misalignment of tile row R's block sb (the row clamped as the DMA clamps it).
    auto mis = [&](int R, int sb, int off = 0) {
        const int rc = min(r0 + R, rows - 1) - r0;
        return static_cast<int>((static_cast<uint32_t>(rc * row_bytes) + static_cast<uint32_t>(sb * G::UB + off)) & 15u);
    };

    // DMA of step st into step slot st & 1 (and, on a super-block's first step, its scales into slot sb & 1).
    auto issue = [&](int st) {
        const int sb = sb0 + (st >> 2), j = st & 3, n = j >> 1, p = j & 1;
        uint8_t *const slot = s_step[st & 1];
#pragma unroll
        for (int k = 0; k < G::CODE_DMA; ++k) {
            const int ci = 64 * k + lane, rr = 32 * wv + ci / G::CPR, ch = ci % G::CPR;  // slot position of row rr
            const int row = min(r0 + rr, rows - 1) - r0;
            const int pc = G::pslot(ch >> 1, rr);  // the piece stored there (pslot is its own inverse)
            const uint32_t a = static_cast<uint32_t>(row * row_bytes + static_cast<long>(sb) * G::UB + G::poff(pc, n, p));
            const uint32_t off = (a & ~15u) + ((ch & 1) && (a & 15u) ? 16u : 0u);
            dma16(wbase, off, slot + 1024 * (G::CODE_DMA * wv + k));
        }
#pragma unroll
        for (int k = 0; k < G::NB; ++k) {
            const int i = G::NB * wv + k, ii = i & 15;
            const int row = 8 * ii + (lane >> 3);
            const int tok = min(t0 + row, M - 1);
            const int c = (lane & 7) ^ ((row >> 1) & 7);
            const uint32_t off = static_cast<uint32_t>((static_cast<long>(tok) * cols + 256L * sb + G::bpos(j, c)) * 2);
            dma16(i < 16 ? static_cast<const void *>(bh) : static_cast<const void *>(bl), off,
                  slot + G::CODE_BYTES + (i < 16 ? 0 : kG16BN * 128) + 1024 * ii);
        }
        if (j != 0) return;
#pragma unroll
        for (int k = 0; k < G::SB_DMA; ++k) {
            const int ci = 64 * (G::SB_DMA * wv + k) + lane;  // 16-byte chunk of the super-block slot
            uint8_t *const dst = s_sb[sb & 1] + 1024 * (G::SB_DMA * wv + k);
            if (ci < kG16BM * G::SBR / 16) {
                // Row rr's chunk pair(s): Q2_K's second pair holds d and dmin (byte 80, the same misalignment).
                const int rr = ci / (G::SBR / 16), pr = (ci >> 1) & (G::SBR / 32 - 1);
                const int row = min(r0 + rr, rows - 1) - r0;
                const int so = pr ? G::DOFF : G::SOFF, sl = pr ? 4 : G::SLEN;
                const uint32_t a = static_cast<uint32_t>(row * row_bytes + static_cast<long>(sb) * G::UB + so);
                const uint32_t off = (a & ~15u) + ((ci & 1) && (a & 15u) + sl > 16u ? 16u : 0u);
                dma16(wbase, off, dst);
            } else {  // Q2_K: the tokens' XS, 64 bytes each
                const int cj = ci - kG16BM * G::SBR / 16;
                const int tok = min(t0 + (cj >> 2), M - 1);
                const uint32_t off = static_cast<uint32_t>(((static_cast<long>(tok) * nsb + sb) * 32 + 8 * (cj & 3)) * 2);
                dma16(xs, off, dst);
            }
        }
    };

    g16f4 acc[RB][TB], C[RB][TB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int q = 0; q < TB; ++q) acc[i][q] = C[i][q] = g16f4{0.f, 0.f, 0.f, 0.f};

    if (nsteps > 0) issue(0);
    uint32_t scw[RB][2];  // [rb][c]: scales 8n + 4c .. +4 of row wr + 16 rb + lr (Q3_K: 6-bit, unpacked), one per byte
    for (int st = 0; st < nsteps; ++st) {
        wait_vm<0>();
        __syncthreads();  // step st landed for every wave; step st - 1's slot is free
        if (st + 1 < nsteps) issue(st + 1);
        const int sb = sb0 + (st >> 2), j = st & 3, n = j >> 1, p = j & 1;
        const uint8_t *const slot = s_step[st & 1];
        const uint8_t *const sbs = s_sb[sb & 1];
        const uint8_t *const sBh = slot + G::CODE_BYTES, *const sBl = sBh + kG16BN * 128;
        if (G::DONLY ? false : G::IQ ? j == 0 : p == 0) {  // the half's eight scales, on its first step (IQ2_XS: all
                                                           // eight at once; IQ2_XXS: in the code pieces)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int R = wr + 16 * rb + lr, o = R * G::SBR + mis(R, sb, G::SOFF);
                const uint32_t sh = static_cast<uint32_t>(o & 3);
                if constexpr (G::IQ) {  // scales[8]: byte g holds the two 16-element halves of group g
                    const uint2 v = g16n_read8(sbs, o);
                    scw[rb][0] = v.x;
                    scw[rb][1] = v.y;
                } else if constexpr (G::Q2) {  // 4-bit scales in the low nibbles of bytes 8n .. 8n + 7
                    const uint32_t *q = reinterpret_cast<const uint32_t *>(sbs + (o & ~3) + 8 * n);
                    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
                    scw[rb][0] = __builtin_amdgcn_alignbyte(d1, d0, sh) & 0x0F0F0F0Fu;
                    scw[rb][1] = __builtin_amdgcn_alignbyte(d2, d1, sh) & 0x0F0F0F0Fu;
                } else if constexpr (G::Q6) {
                    const uint32_t *q = reinterpret_cast<const uint32_t *>(sbs + (o & ~3) + 8 * n);
                    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
                    scw[rb][0] = __builtin_amdgcn_alignbyte(d1, d0, sh);
                    scw[rb][1] = __builtin_amdgcn_alignbyte(d2, d1, sh);
                } else {  // 6-bit scales: low nibbles in bytes 0..7, high pairs in bytes 8..11 (the k3 packing)
                    const uint32_t *q = reinterpret_cast<const uint32_t *>(sbs + (o & ~3));
                    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2], d3 = q[3];
                    const uint32_t a0 = __builtin_amdgcn_alignbyte(d1, d0, sh), a1 = __builtin_amdgcn_alignbyte(d2, d1, sh),
                                   a2 = __builtin_amdgcn_alignbyte(d3, d2, sh) >> (4 * n);
                    scw[rb][0] = ((a0 >> (4 * n)) & 0x0F0F0F0Fu) | ((a2 & 0x03030303u) << 4);
                    scw[rb][1] = ((a1 >> (4 * n)) & 0x0F0F0F0Fu) | (((a2 >> 2) & 0x03030303u) << 4);
                }
            }
        }
        // A fragments: row R = wr + 16 rb + lr, chunk c: k = 2c + (lk >> 1), elements 8 (lk & 1) .. +8 of the
        // step's 16-element run of k.
        const int hf = 8 * (lk & 1), kl = lk >> 1;
        const uint32_t sbyte = 8u * static_cast<uint32_t>(p + 2 * kl);  // the run's scale: byte p + 2 kl of dword 2n + c
        uint2 ra[RB], rh[RB];  // [rb]: Q6_K ql (run kl) and qh; Q3_K qs and hmask; IQ2_S index and sign bytes
        uint32_t rq2[RB];      // [rb]: IQ2_S high index bits
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int R = wr + 16 * rb + lr;
            if constexpr (G::IQ3X) {  // index bytes 2 lk, 2 lk + 1 of each group; the groups' aux words
                const int rb0 = R * G::CPR * 16, pb = rb0 + mis(R, sb, G::poff(0, n, p)) + 2 * lk;
                ra[rb] = uint2{g16n_read8(slot, pb).x & 0xFFFFu, g16n_read8(slot, pb + 8).x & 0xFFFFu};
                rh[rb] = g16n_read8(slot, rb0 + 32 + mis(R, sb, G::poff(1, n, p)));
            } else if constexpr (G::IQS) {  // the step's 8 index bytes, 8 sign bytes and 2 high-bit bytes
                const int rb0 = R * G::CPR * 16;
                ra[rb] = g16n_read8(slot, rb0 + mis(R, sb, G::poff(0, n, p)));
                rh[rb] = g16n_read8(slot, rb0 + 32 + mis(R, sb, G::poff(1, n, p)));
                rq2[rb] = g16n_read8(slot, rb0 + 64 + mis(R, sb, G::poff(2, n, p))).x;
            } else if constexpr (G::IQX) {  // the two groups' (aux0, aux1): grid bytes, then 4 x 7 sign bits and the scale
                const int pb = R * G::CPR * 16 + mis(R, sb, G::POFF0);
                ra[rb] = g16n_read8(slot, pb);
                rh[rb] = g16n_read8(slot, pb + 8);
            } else if constexpr (G::IQ) {  // entries lk (c = 0) and 4 + lk (c = 1) of the step's eight
                const int pb = R * G::CPR * 16 + mis(R, sb, G::POFF0) + 2 * lk;
                ra[rb] = uint2{g16n_read8(slot, pb).x & 0xFFFFu, g16n_read8(slot, pb + 8).x & 0xFFFFu};
            } else {
                const int base = R * G::CPR * 16 + mis(R, sb) + hf;
                ra[rb] = g16n_read8(slot, base + 32 * G::pslot(G::Q6 ? kl : 0, R));
                if constexpr (!G::Q2) rh[rb] = g16n_read8(slot, base + 32 * G::pslot(G::Q6 ? 2 : 1, R));
            }
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int k = 2 * c + kl;
            g16h8 a1[RB], a2[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const uint32_t sw = scw[rb][c];
                uint32_t c0, c1;
                int isc;
                if constexpr (G::IQ3X) {
                    // Lane lk of group 2 j + c: two 4-magnitude grid entries, 7 sign bits lk of the aux word (with
                    // their parity bit), scale 2 (aux >> 28) + 1 (d / 4 applies at the super-block's end).
                    const uint32_t e = c ? ra[rb].y : ra[rb].x, ax = c ? rh[rb].y : rh[rb].x;
                    const uint2 sel = tb.ks128[(ax >> (7 * lk)) & 127u];
                    c0 = sign4_sel(tb.grid4[e & 255u], sel.x);
                    c1 = sign4_sel(tb.grid4[e >> 8], sel.y);
                    isc = 2 * static_cast<int>(ax >> 28) + 1;
                } else if constexpr (G::IQS) {
                    // Entry lk of group 2 j + c: grid index = its qs byte | 2 bits of the group's qh byte << 8, its
                    // 8 sign bits from the signs byte; the half's scale 2 s + 1.
                    const uint32_t e = 4 * c + lk;
                    const uint32_t idx = ((e < 4 ? ra[rb].x : ra[rb].y) >> (8 * (e & 3)) & 255u) |
                                         (((rq2[rb] >> (8 * c + 2 * lk)) & 3u) << 8);
                    const uint32_t s8 = (e < 4 ? rh[rb].x : rh[rb].y) >> (8 * (e & 3)) & 255u;
                    sign8(tb.grid8[idx], s8, c0, c1);
                    const int grp = 2 * j + c;
                    isc = 2 * static_cast<int>((scw[rb][grp >> 2] >> (8 * (grp & 3) + 4 * kl)) & 15u) + 1;
                } else if constexpr (G::IQX) {
                    // Group 2 j + c: grid index = byte lk of aux0, signs = 7 bits lk of aux1, scale 2 (aux1 >> 28) + 1.
                    const uint2 ax = c ? rh[rb] : ra[rb];
                    const uint2 g = tb.grid8[(ax.x >> (8 * lk)) & 255u], sel = tb.ks128[(ax.y >> (7 * lk)) & 127u];
                    c0 = sign4_sel(g.x, sel.x);
                    c1 = sign4_sel(g.y, sel.y);
                    isc = 2 * static_cast<int>(ax.y >> 28) + 1;
                } else if constexpr (G::IQ) {
                    // Entry e: grid index e & 511 (eight magnitudes), signs from the 7 stored bits e >> 9; the
                    // half's scale 2 s + 1 (d / 8 applies at the super-block's end).
                    const uint32_t e = c ? ra[rb].y : ra[rb].x;
                    const uint2 g = tb.grid8[e & 511u], sel = tb.ks128[e >> 9];
                    c0 = sign4_sel(g.x, sel.x);
                    c1 = sign4_sel(g.y, sel.y);
                    const int grp = 2 * j + c;
                    isc = 2 * static_cast<int>((scw[rb][grp >> 2] >> (8 * (grp & 3) + 4 * kl)) & 15u) + 1;
                } else if constexpr (G::Q2) {
                    c0 = (ra[rb].x >> (2 * k)) & 0x03030303u;
                    c1 = (ra[rb].y >> (2 * k)) & 0x03030303u;
                    isc = static_cast<int>((sw >> sbyte) & 0xFFu);
                } else if constexpr (G::Q6) {
                    c0 = ((ra[rb].x >> (4 * c)) & 0x0F0F0F0Fu) | (((rh[rb].x >> (2 * k)) & 0x03030303u) << 4);
                    c1 = ((ra[rb].y >> (4 * c)) & 0x0F0F0F0Fu) | (((rh[rb].y >> (2 * k)) & 0x03030303u) << 4);
                    isc = static_cast<int>(static_cast<int8_t>(sw >> sbyte));
                } else {
                    const uint32_t hs = static_cast<uint32_t>(4 * n + k);
                    c0 = ((ra[rb].x >> (2 * k)) & 0x03030303u) | (((rh[rb].x >> hs) & 0x01010101u) << 2);
                    c1 = ((ra[rb].y >> (2 * k)) & 0x03030303u) | (((rh[rb].y >> hs) & 0x01010101u) << 2);
                    isc = static_cast<int>((sw >> sbyte) & 0xFFu) - 32;
                }
                s16_frag<T>(c0, c1, isc, a1[rb], a2[rb]);
            }
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
                        cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[rb], bhf[i], cc, 0, 0, 0);
                        if constexpr (LO) cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[rb], blf[i], cc, 0, 0, 0);
                        if constexpr (G::Q6 && LO) {  // b_hi alone: the weight as its f16 rounding p only
                            cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2[rb], bhf[i], cc, 0, 0, 0);
                            if constexpr (LO && !VQ_S16_RSPLIT)
                                cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2[rb], blf[i], cc, 0, 0, 0);
                        }
                    }
            }
        }
        if (j == 3) {
            // Super-block end: acc += d C (Q2_K: - 32 dmin (m . XS)); C element q of a block is row 4 lk + q,
            // token lr.
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float dq[4], mq[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int R = wr + 16 * rb + 4 * lk + q;
                    const int od = G::SBR == 64 ? R * G::SBR + 32 + mis(R, sb, G::DOFF) : R * G::SBR + mis(R, sb, G::SOFF) + G::SLEN - 2;
                    const uint32_t hd = *reinterpret_cast<const uint16_t *>(sbs + od) |
                                        (G::Q2 ? static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(sbs + od + 2)) << 16 : 0u);
                    dq[q] = half_to_float(hd) * (G::IQ3X ? 0.25f : G::IQ ? 0.125f : 1.0f);
                    mq[q] = 32.0f * half_to_float(hd >> 16);
                }
                g16h4 amin = {};
                if constexpr (G::Q2) {
                    // A_min fragment: row wr + 16 rb + lr, k = 4 lk .. +4 -> the mins (high nibbles) of
                    // sub-blocks 4 lk .. 4 lk + 3.
                    const int R = wr + 16 * rb + lr;
                    const uint32_t mw = (g16n_read8(sbs, R * G::SBR + mis(R, sb) + 4 * lk).x >> 4) & 0x0F0F0F0Fu;
                    const g16h2 k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
                    const g16h2 m01 = g16_pair(mw, 0x04010400u) - k1024, m23 = g16_pair(mw, 0x04030402u) - k1024;
                    amin = g16h4{m01[0], m01[1], m23[0], m23[1]};
                }
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
                    if constexpr (G::Q2) {
                        const uint8_t *const sx = sbs + kG16BM * G::SBR + (wt + 16 * tb + lr) * 64 + 8 * lk;
                        const g16h4 bm_hi = *reinterpret_cast<const g16h4 *>(sx);
                        const g16h4 bm_lo = *reinterpret_cast<const g16h4 *>(sx + 32);
                        g16f4 cm = __builtin_amdgcn_mfma_f32_16x16x16f16(amin, bm_hi, g16f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        cm = __builtin_amdgcn_mfma_f32_16x16x16f16(amin, bm_lo, cm, 0, 0, 0);
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc[rb][tb][q] = fmaf(dq[q], C[rb][tb][q], fmaf(-mq[q], cm[q], acc[rb][tb][q]));
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc[rb][tb][q] = fmaf(dq[q], C[rb][tb][q], acc[rb][tb][q]);
                    }
                    C[rb][tb] = g16f4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    }

    // Output, as qgemm16_kernel: a whole tile to y, a part of one to its slot.
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
    __syncthreads();  // the slots are reused by the next segment's first DMAs
    u += sb1 - sb0;
    if (whole && u >= ue) whole = false, u = pl.u0(v), ue = pl.u0(v + 1);
    }
}

template <int T>
int launch_gemm16n(const uint8_t *w, int rows, int cols, long rb, const void *ws, int M, float *y, int cus,
                   hipStream_t s, bool invariant, bool f16x) {
    const G16Plan pl = g16_plan(rows, cols, M, cus, invariant);
    const G16Ws l = g16_layout(cols, M, pl, T == VQ_Q2_K);
    uint8_t *base = static_cast<uint8_t *>(const_cast<void *>(ws));
    float *const part = reinterpret_cast<float *>(base + l.part);
    auto *const kern = f16x ? qgemm16n_kernel<T, false> : qgemm16n_kernel<T, true>;
    kern<<<dim3(8 * pl.per_xcd), dim3(64 * kG16Waves), 0, s>>>(
        w, rows, cols, rb, reinterpret_cast<const _Float16 *>(base + l.bh), reinterpret_cast<const _Float16 *>(base + l.bl),
        reinterpret_cast<const _Float16 *>(base + l.xs), reinterpret_cast<const float *>(base + l.inv), M, pl, y, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    if (pl.tiles > pl.t0) g16_reduce_kernel<kG16RB><<<dim3(16 * (pl.tiles - pl.t0)), dim3(512), 0, s>>>(part, pl, rows, M, y);
    e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int>(e);
}

}  // namespace vq
