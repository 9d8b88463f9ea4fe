// vq_slices.h -- per-type "slice" decoders of the MI355X matvec (hand-written for CDNA4).
//
// A slice is the part of one GGUF super-block a single lane owns: a fixed set of NP "parts", each part
// being 16 consecutive elements (one half of a 32-element group). A lane loads only its slice's bytes
// (plus the block header it needs) with dword/dwordx2/dwordx4 global loads -- unaligned where the block
// size is not a multiple of 4 -- decodes them to packed int8 codes, and produces for every part
//   S  = dot(codes, xq) - OFF * X over the 16 elements (exact int32: the reference's integer partial)
//   sc = fp32 scale of the part (d * sub-block scale), mn = fp32 min coefficient (Q2_K/Q4_K/Q5_K)
// so that part contributes (S * sc - X * mn) * xd to the output, with X = sum of the 16 xq and xd the
// activation scale of the group. This is the reference CPU path's arithmetic
// (/root/reference/engine/csrc/cpu/qwen_cpu.c:125-342) regrouped per 16 elements.
//
// Codes with an offset (Q3_K: lo|hb<<2 - 4, Q6_K: q - 32) are dotted unsigned and corrected with the
// integer X (S = dot(q) - off*X): exact, and cheaper than a bytewise subtract. Sign-coded IQ grids take
// their signs in registers (sign4: a byte permute between the magnitudes and their negation), so the only
// LDS table an IQ slice reads is its grid.
//
// Block layouts: qwen_quant.cuh:151-279 / dequant.py:121-500 (ggml).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_common.h"
#include "vq_lds.h"

namespace vq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---- global -> LDS DMA ---------------------------------------------------------------------------------
// Codebooks in global memory (device tables of the library).
struct Grids {
    const uint2 *iq2xxs;     // 256 entries of 8 magnitudes
    const uint2 *iq2xs;      // 512
    const uint2 *iq2s;       // 1024
    const uint32_t *iq3xxs;  // 256 entries of 4 magnitudes
    const uint32_t *iq3s;    // 512
};

// ggml ksigns_iq2xs[i]: the 7 sign bits plus an even-parity 8th bit.
__device__ __forceinline__ uint32_t ksigns(uint32_t i7) { return i7 | ((__builtin_popcount(i7) & 1u) << 7); }

// LDS tables used by the IQ decoders.
struct Tabs {
    const uint2 *grid8;     // IQ2_XXS / IQ2_XS / IQ2_S magnitudes (8 bytes per entry)
    const uint32_t *grid4;  // IQ3_XXS / IQ3_S magnitudes (4 bytes per entry)
    const uint2 *ks128;     // ggml ksigns (7 bits + parity) -> sign4's permute selectors {bits 0-3, bits 4-7}
    const uint2 *sm256;     // raw 8 sign bits -> the same selectors
    const uint32_t *sg;     // pre-signed grid words (IQ3_S, streaming kernel): [entry][4 sign bits]
};

template <int N>
__device__ __forceinline__ void ldg(const uint8_t *p, uint32_t (&out)[N]) {
    __builtin_memcpy(out, p, 4 * N);
}
__device__ __forceinline__ uint32_t ldg1(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}

// 2-byte-aligned fields (blocks of 34, 18, 66, 74, 82, 98, 110, 210 bytes) are fetched as 4-byte-aligned
// dword spans and re-sliced with v_alignbyte_b32: unaligned multi-dword loads split into many L1 accesses.
// (Pointer arithmetic, not integer casts, so the loads stay global_load and never degrade to flat_load.)
__device__ __forceinline__ uint32_t mis(const uint8_t *p) { return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)) & 3u; }
__device__ __forceinline__ const uint32_t *al4(const uint8_t *p) { return reinterpret_cast<const uint32_t *>(p - mis(p)); }
// A raw span: the N+1 aligned dwords covering N dwords that start at a 2-byte-aligned address, plus that
// address's misalignment. Loading keeps the raw words (so the load has no consumer until the slice is
// decoded, one pipeline trip later); word(i) re-slices on use. (Unaligned LDS dword reads are legal on
// gfx950 but measured slower than aligned reads plus v_alignbyte_b32: the matvec lost 10-35 %.)
template <int N>
struct Span {
    uint32_t t[N + 1];
    uint32_t sh;
    __device__ __forceinline__ uint32_t word(int i) const { return __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh); }
};
template <int N>
__device__ __forceinline__ void ldspan(const uint8_t *p, Span<N> &s) {
    const uint32_t *q = al4(p);
#pragma unroll
    for (int i = 0; i <= N; ++i) s.t[i] = q[i];
    s.sh = mis(p);
}
// A single aligned dword holding byte p and the byte shift to it: lo() = the dword whose low byte is at p
// (bytes past the aligned word read as zero).
struct Lo {
    uint32_t v, sh;
    __device__ __forceinline__ uint32_t lo() const { return v >> (8 * sh); }
};
__device__ __forceinline__ void ldlo(const uint8_t *p, Lo &l) {
    l.v = *al4(p);
    l.sh = mis(p);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}
__device__ __forceinline__ int dot16(const uint32_t (&c)[4], const uint32_t *x) {
    return dot4(c[3], x[3], dot4(c[2], x[2], dot4(c[1], x[1], dot4(c[0], x[0], 0))));
}
__device__ __forceinline__ float half_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}
__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_ubfe(v, off, width);
}
__device__ __forceinline__ uint32_t sgn(uint32_t g, uint32_t m, uint32_t e) { return (g ^ m) + e; }

// Bytes of g (grid magnitudes, every byte >= 1) negated where bit k of s4 (4 sign bits) is set, in registers:
// v_perm_b32 picks byte k of g or of -g, the bytewise negation (~g) + 0x01010101 (carry-free since no byte of
// g is 0). The selector puts bit k at bit 2 of byte k (s4 * 0x00810204 moves bit k to bit 8k + 2 without
// overlap, s4 < 16) over the identity 0x03020100.
// A 32-bit constant in a VGPR. gfx9 VOP3 instructions take no literal and read at most one SGPR, so without this
// the compiler splits (a & m) | (b & ~m) into two VOP2 operations; the asm has no side effects, so the move is
// hoisted out of loops and shared.
__device__ __forceinline__ uint32_t vconst(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
    return r;
}
__device__ __forceinline__ uint32_t sign4(uint32_t g, uint32_t s4) {
    const uint32_t neg = (g ^ 0xFFFFFFFFu) + 0x01010101u;
    const uint32_t sel = (__umul24(s4, 0x00810204u) & vconst(0x04040404u)) | vconst(0x03020100u);
    return __builtin_amdgcn_perm(neg, g, sel);
}
// sign4 with its selector given (a sign table entry).
__device__ __forceinline__ uint32_t sign4_sel(uint32_t g, uint32_t sel) {
    return __builtin_amdgcn_perm((g ^ 0xFFFFFFFFu) + 0x01010101u, g, sel);
}
// ggml's 7 stored sign bits with the even-parity 8th at bit 7 (bits above 7 may be set: callers take bits 0-7).
__device__ __forceinline__ uint32_t ksigns8(uint32_t b7) { return b7 | (__builtin_popcount(b7) << 7); }
// Signs of 8 magnitudes (two words) from 8 sign bits.
__device__ __forceinline__ void sign8(uint2 g, uint32_t s8, uint32_t &lo, uint32_t &hi) {
    lo = sign4(g.x, bfe(s8, 0, 4));
    hi = sign4(g.y, bfe(s8, 4, 4));
}

// IQ4_NL codebook lookup of the four nibbles at bits 4s .. 4s + 3 of each byte of q (s = 0: low nibbles, 1: high
// nibbles): two v_perm_b32 over the 16 table bytes, indexed by the nibbles' low 3 bits, and a third that picks
// per byte by bit 3 (its selector k + 4 bit3 built with one v_bfi_b32).
template <int SH>
__device__ __forceinline__ uint32_t iq4nl4(uint32_t q) {
    constexpr uint32_t t0 = 0xBFAD9881u, t1 = 0xF6EADDCFu, t2 = 0x26190D01u, t3 = 0x71594535u;
    const uint32_t sel = (q >> SH) & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t m = vconst(0x04040404u), b = vconst(0x03020100u);
    const uint32_t pick = (((q >> (SH + 1)) ^ b) & m) ^ b;  // bit 3 of each nibble to bit 2, over k
    return __builtin_amdgcn_perm(hi, lo, pick);
}

// Byte k (runtime) of a 12-byte little-endian field held in three dwords.
__device__ __forceinline__ uint32_t byte12(uint32_t a, uint32_t b, uint32_t c, int k) {
    const uint32_t w = k < 4 ? a : (k < 8 ? b : c);
    return bfe(w, 8 * (k & 3), 8);
}

// Q4_K/Q5_K 6-bit scales and mins of the two groups j = 2p, 2p+1 (k4_scale_min, qwen_cpu.c:54-62), branch-free:
// a/b/c are scales[0..3], [4..7], [8..11]; the pair's bytes sit at byte offset 2*(p & 1) of each. Returns
// sc2/m2 with group 2p in byte 0 and group 2p+1 in byte 1.
__device__ __forceinline__ void k4sm_pair(uint32_t a, uint32_t b, uint32_t c, int p, uint32_t &sc2, uint32_t &m2) {
    const uint32_t sh = 16 * (p & 1);
    const uint32_t A = a >> sh, B = b >> sh, C = c >> sh;
    const uint32_t sc_lo = A & 0x3F3Fu, m_lo = B & 0x3F3Fu;
    const uint32_t sc_hi = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);
    const uint32_t m_hi = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
    sc2 = p >= 2 ? sc_hi : sc_lo;
    m2 = p >= 2 ? m_hi : m_lo;
}
// Byte k of v as float (v_cvt_f32_ubyte{0..3}).
__device__ __forceinline__ float ubyte0(uint32_t v) { return static_cast<float>(v & 0xFFu); }
__device__ __forceinline__ float ubyte1(uint32_t v) { return static_cast<float>((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ubyte2(uint32_t v) { return static_cast<float>((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ubyte3(uint32_t v) { return static_cast<float>(v >> 24); }

template <int T>
struct Sl;

// ---- Q4_K: 144 B = d, dmin, scales[12], qs[128]. Slice s = (pair p, half h): qs[32p+16h .. +16] ->
// parts (group 2p, half h) from low nibbles and (group 2p+1, half h) from high nibbles. 8 slices.
template <>
struct Sl<VQ_Q4_K> {
    static constexpr int SPB = 8, NP = 2, UB = 144, UG = 8;
    struct W {
        uint32_t hd[4], q[4];
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldg(u, w.hd);
        ldg(u + 16 + 16 * s, w.q);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = 2 * (s >> 1) + p;
        h = s & 1;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &, uint32_t (&c)[NP][4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[0][i] = w.q[i] & 0x0F0F0F0Fu;
            c[1][i] = (w.q[i] >> 4) & 0x0F0F0F0Fu;
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int s, float *sc, float *mn) {
        const float d = half_to_float(w.hd[0]), dmin = half_to_float(w.hd[0] >> 16);
        uint32_t sc2, m2;
        k4sm_pair(w.hd[1], w.hd[2], w.hd[3], s >> 1, sc2, m2);
        sc[0] = d * ubyte0(sc2);
        sc[1] = d * ubyte1(sc2);
        mn[0] = dmin * ubyte0(m2);
        mn[1] = dmin * ubyte1(m2);
    }
    // Integer form: part p weighs d * isc[p] and its min dmin * imn[p].
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.hd[0]); }
    static __device__ __forceinline__ float dmin(const W &w) { return half_to_float(w.hd[0] >> 16); }
    static __device__ __forceinline__ void iscales(const W &w, int s, int (&isc)[NP]) {
        uint32_t sc2, m2;
        k4sm_pair(w.hd[1], w.hd[2], w.hd[3], s >> 1, sc2, m2);
        isc[0] = static_cast<int>(sc2 & 0xFFu);
        isc[1] = static_cast<int>((sc2 >> 8) & 0xFFu);
    }
    static __device__ __forceinline__ void imins(const W &w, int s, int (&imn)[NP]) {
        uint32_t sc2, m2;
        k4sm_pair(w.hd[1], w.hd[2], w.hd[3], s >> 1, sc2, m2);
        imn[0] = static_cast<int>(m2 & 0xFFu);
        imn[1] = static_cast<int>((m2 >> 8) & 0xFFu);
    }
};

// ---- Q5_K: 176 B = d, dmin, scales[12], qh[32], qs[128]. Like Q4_K plus qh bit j of element l.
template <>
struct Sl<VQ_Q5_K> {
    static constexpr int SPB = 8, NP = 2, UB = 176, UG = 8;
    struct W {
        uint32_t hd[4], q[4], qh[4];
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldg(u, w.hd);
        ldg(u + 48 + 16 * s, w.q);
        ldg(u + 16 + 16 * (s & 1), w.qh);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = 2 * (s >> 1) + p;
        h = s & 1;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int s, const Tabs &, uint32_t (&c)[NP][4]) {
        const int j = 2 * (s >> 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[0][i] = (w.q[i] & 0x0F0F0F0Fu) | (((w.qh[i] >> j) & 0x01010101u) << 4);
            c[1][i] = ((w.q[i] >> 4) & 0x0F0F0F0Fu) | (((w.qh[i] >> (j + 1)) & 0x01010101u) << 4);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int s, float *sc, float *mn) {
        Sl<VQ_Q4_K>::W t;
#pragma unroll
        for (int i = 0; i < 4; ++i) t.hd[i] = w.hd[i];
        Sl<VQ_Q4_K>::scales(t, s, sc, mn);
    }
    // Integer form (the Q4_K header layout).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.hd[0]); }
    static __device__ __forceinline__ float dmin(const W &w) { return half_to_float(w.hd[0] >> 16); }
    static __device__ __forceinline__ void iscales(const W &w, int s, int (&isc)[NP]) {
        uint32_t sc2, m2;
        k4sm_pair(w.hd[1], w.hd[2], w.hd[3], s >> 1, sc2, m2);
        isc[0] = static_cast<int>(sc2 & 0xFFu);
        isc[1] = static_cast<int>((sc2 >> 8) & 0xFFu);
    }
    static __device__ __forceinline__ void imins(const W &w, int s, int (&imn)[NP]) {
        uint32_t sc2, m2;
        k4sm_pair(w.hd[1], w.hd[2], w.hd[3], s >> 1, sc2, m2);
        imn[0] = static_cast<int>(m2 & 0xFFu);
        imn[1] = static_cast<int>((m2 >> 8) & 0xFFu);
    }
};

// ---- Q6_K: 210 B = ql[128], qh[64], scales[16] (int8), d. Slice s = (chunk c, half hh): elements
// 16hh..16hh+15 of the four groups 4c..4c+3 (quarters q: ql lo/hi nibble of ql[64c + 32(q&1) + l],
// qh bits 2q of qh[32c + l]). 4 slices. Codes q - 32 via S = dot(q) - 32 X.
template <>
struct Sl<VQ_Q6_K> {
    static constexpr int SPB = 4, NP = 4, UB = 210, UG = 8;
    struct W {
        Span<4> a, b, h;
        Span<2> sc;
        Lo d;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        const int c = s >> 1, hh = s & 1;
        ldspan(u + 64 * c + 16 * hh, w.a);
        ldspan(u + 64 * c + 32 + 16 * hh, w.b);
        ldspan(u + 128 + 32 * c + 16 * hh, w.h);
        ldspan(u + 192 + 8 * c, w.sc);
        ldlo(u + 208, w.d);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = 4 * (s >> 1) + p;
        h = s & 1;
    }
    static constexpr int OFF = 32;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &, uint32_t (&c)[NP][4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = w.a.word(i), b = w.b.word(i), h = w.h.word(i);
            c[0][i] = (a & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4);
            c[1][i] = (b & 0x0F0F0F0Fu) | ((h & 0x0C0C0C0Cu) << 2);
            c[2][i] = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
            c[3][i] = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int s, float *sc, float *mn) {
        const float d = half_to_float(w.d.lo());
        const int hh = s & 1;
        const uint32_t sc0 = w.sc.word(0), sc1 = w.sc.word(1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // scales[2(4c+q) + hh] = byte (2q + hh) of the 8 bytes at 192 + 8c
            const uint32_t word = q < 2 ? sc0 : sc1;
            const int v = static_cast<int8_t>(bfe(word, 16 * (q & 1) + 8 * hh, 8));
            sc[q] = d * static_cast<float>(v);
            mn[q] = 0.0f;
        }
    }
    // Integer form: part q weighs d * isc[q] (the signed 8-bit scale).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.d.lo()); }
    static __device__ __forceinline__ void iscales(const W &w, int s, int (&isc)[NP]) {
        const int hh = s & 1;
        const uint32_t sc0 = w.sc.word(0), sc1 = w.sc.word(1);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            isc[q] = __builtin_amdgcn_sbfe(static_cast<int>(q < 2 ? sc0 : sc1), 16 * (q & 1) + 8 * hh, 8);
    }
};

// ---- Q3_K: 110 B = hmask[32], qs[64], scales[12], d. Slice s = (qs half q2, half hh): elements
// 16hh..16hh+15 of groups 4q2..4q2+3; code = lo2 | hb<<2, minus 4 via S = dot - 4X. 4 slices.
template <>
struct Sl<VQ_Q3_K> {
    static constexpr int SPB = 4, NP = 4, UB = 110, UG = 8;
    struct W {
        Span<4> qs, hm, sw;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        const int q2 = s >> 1, hh = s & 1;
        ldspan(u + 32 + 32 * q2 + 16 * hh, w.qs);
        ldspan(u + 16 * hh, w.hm);
        ldspan(u + 96, w.sw);  // scales[12], d, and 2 bytes of the next block (or the tail pad)
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = 4 * (s >> 1) + p;
        h = s & 1;
    }
    static constexpr int OFF = 4;
    static __device__ __forceinline__ void codes(const W &w, int s, const Tabs &, uint32_t (&c)[NP][4]) {
        const int j0 = 4 * (s >> 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t qs = w.qs.word(i), hm = w.hm.word(i);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                // hmask bit j0+p of each byte moved straight to bit 2 (one shift, one mask)
                const int sh = j0 + p - 2;
                const uint32_t hb = (sh >= 0 ? hm >> sh : hm << -sh) & 0x04040404u;
                c[p][i] = ((qs >> (2 * p)) & 0x03030303u) | hb;
            }
        }
    }
    // Streaming form of the codes: part p keeps its 2-bit field in place (bits 2p, 2p+1; part 3 shifted down
    // to bits 4, 5) with the hmask bit just above it, i.e. code << gsh(p) with gsh = 0, 2, 4, 4 -- one shift
    // fewer per word for parts 1 and 2. Values stay <= 112 (positive int8). Every part of group g has
    // p = g & 3, so the caller divides the group's exact integer sum by 2^gsh once.
    static __device__ __forceinline__ constexpr int gsh(int g) { return (g & 3) == 0 ? 0 : (g & 3) == 1 ? 2 : 4; }
    static __device__ __forceinline__ void codes_scaled(const W &w, int s, const Tabs &, uint32_t (&c)[NP][4]) {
        // hmask bit j0 + p goes to bit lb + 2: shifted left by 2, 3, 4, 3 (j0 = 0) or right by 2, 1, 0, 1 (j0 = 4);
        // parts 1 and 3 share their shifted copy.
        const bool lo_half = (s >> 1) == 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t qs = w.qs.word(i), hm = w.hm.word(i);
            const uint32_t h0 = lo_half ? hm << 2 : hm >> 2;
            const uint32_t h13 = lo_half ? hm << 3 : hm >> 1;
            const uint32_t h2 = lo_half ? hm << 4 : hm;
            c[0][i] = (h0 & 0x04040404u) | (qs & 0x03030303u);
            c[1][i] = (h13 & 0x10101010u) | (qs & 0x0C0C0C0Cu);
            c[2][i] = (h2 & 0x40404040u) | (qs & 0x30303030u);
            c[3][i] = ((qs >> 2) & 0x30303030u) | (h13 & 0x40404040u);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int s, float *sc, float *mn) {
        const uint32_t sw[4] = {w.sw.word(0), w.sw.word(1), w.sw.word(2), w.sw.word(3)};
        const float d = half_to_float(sw[3]);
        const int hh = s & 1;
        // k = 2(j0+p) + hh for p = 0..3 spans k0 .. k0+6 step 2, k0 = 8*q2 + hh (q2 = s >> 1):
        // low nibbles: bytes (k & 7) = hh, hh+2, hh+4, hh+6 of scales[0..7], nibble k >> 3 = q2;
        // high 2 bits: byte 8 + (k & 3) = 8 + hh (p even) / 10 + hh (p odd), bit pair k >> 2 = 2q2 + (p >> 1).
        const int q2 = s >> 1;
        const uint32_t lo4 = ((sw[0] >> (8 * hh + 4 * q2)) & 0x000F000Fu) | (((sw[1] >> (8 * hh + 4 * q2)) & 0x000F000Fu) << 8);
        const uint32_t hb = sw[2] >> (8 * hh + 4 * q2);  // bytes 8+hh (bits 0..7) and 10+hh (bits 16..23)
        const uint32_t h01 = ((hb & 0x00030003u) << 4);           // p = 0 (byte 0), p = 1 (byte 2)
        const uint32_t h23 = ((hb >> 2) & 0x00030003u) << 4;      // p = 2, p = 3
        // lo4 bytes: p0 -> byte 0, p1 -> byte 2, p2 -> byte 1, p3 -> byte 3
        const uint32_t v = lo4 | h01 | (h23 << 8);
        sc[0] = d * (ubyte0(v) - 32.0f);
        sc[1] = d * (ubyte2(v) - 32.0f);
        sc[2] = d * (ubyte1(v) - 32.0f);
        sc[3] = d * (ubyte3(v) - 32.0f);
        mn[0] = mn[1] = mn[2] = mn[3] = 0.0f;
    }
    // Integer form of the same scales: part p weighs d * isc[p].
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.sw.word(3)); }
    static __device__ __forceinline__ void iscales(const W &w, int s, int (&isc)[NP]) {
        // Scales 4m..4m+3 as the bytes of one word: low nibbles from scales[0..7] (nibble m >> 1 of bytes
        // 4(m & 1)..), bit pair m of scales[8..11] above them. sc - 32 of a 6-bit sc is the 6-bit two's
        // complement sc ^ 32: bit 1 of every pair is flipped once, and each part takes a signed 6-bit field.
        const uint32_t sw0 = w.sw.word(0), sw1 = w.sw.word(1), hx = w.sw.word(2) ^ 0xAAAAAAAAu;
        const int q2 = s >> 1, hh = s & 1;
        const uint32_t wlo = q2 == 0 ? ((sw0 & 0x0F0F0F0Fu) | ((hx << 4) & 0x30303030u))
                                     : (((sw0 >> 4) & 0x0F0F0F0Fu) | (hx & 0x30303030u));
        const uint32_t whi = q2 == 0 ? ((sw1 & 0x0F0F0F0Fu) | ((hx << 2) & 0x30303030u))
                                     : (((sw1 >> 4) & 0x0F0F0F0Fu) | ((hx >> 2) & 0x30303030u));
        // part p is scale 8 q2 + hh + 2p: byte hh + 2(p & 1) of wlo (p < 2) or whi
        isc[0] = __builtin_amdgcn_sbfe(static_cast<int>(wlo), 8 * hh, 6);
        isc[1] = __builtin_amdgcn_sbfe(static_cast<int>(wlo), 8 * hh + 16, 6);
        isc[2] = __builtin_amdgcn_sbfe(static_cast<int>(whi), 8 * hh, 6);
        isc[3] = __builtin_amdgcn_sbfe(static_cast<int>(whi), 8 * hh + 16, 6);
    }
};

// ---- Q2_K: 84 B = scales[16], qs[64], d, dmin. Slice s = (qs half q2, half hh): elements 16hh.. of
// groups 4q2..4q2+3, code = 2 bits. 4 slices. Mins: - dmin*(s>>4) * X.
template <>
struct Sl<VQ_Q2_K> {
    static constexpr int SPB = 4, NP = 4, UB = 84, UG = 8;
    struct W {
        uint32_t qs[4], sb[2], dd;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        const int q2 = s >> 1, hh = s & 1;
        ldg(u + 16 + 32 * q2 + 16 * hh, w.qs);
        ldg(u + 8 * q2, w.sb);
        w.dd = ldg1(u + 80);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = 4 * (s >> 1) + p;
        h = s & 1;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &, uint32_t (&c)[NP][4]) {
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int i = 0; i < 4; ++i) c[p][i] = (w.qs[i] >> (2 * p)) & 0x03030303u;
    }
    static __device__ __forceinline__ void scales(const W &w, int s, float *sc, float *mn) {
        const float d = half_to_float(w.dd), dmin = half_to_float(w.dd >> 16);
        const int hh = s & 1;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // scales[2(4q2+p) + hh] = byte (2p + hh) of the 8 bytes at 8*q2
            const uint32_t b = bfe(p < 2 ? w.sb[0] : w.sb[1], 16 * (p & 1) + 8 * hh, 8);
            sc[p] = d * static_cast<float>(b & 15);
            mn[p] = dmin * static_cast<float>(b >> 4);
        }
    }
};

// ---- Q8_0: 34 B = d, qs[32]. One slice per block (both halves).
template <>
struct Sl<VQ_Q8_0> {
    static constexpr int SPB = 1, NP = 2, UB = 34, UG = 1;
    struct W {
        Span<9> b;  // d | qs[0..1], qs[2..5], ..., qs[30..31] | 2 bytes past the block
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int, W &w) { ldspan(u, w.b); }
    static __device__ __forceinline__ void part(int, int p, int &g, int &h) {
        g = 0;
        h = p;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &, uint32_t (&c)[NP][4]) {
        uint32_t t[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) t[i] = w.b.word(i);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[0][i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], 2);
            c[1][i] = __builtin_amdgcn_alignbyte(t[i + 5], t[i + 4], 2);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int, float *sc, float *mn) {
        sc[0] = sc[1] = half_to_float(w.b.word(0));
        mn[0] = mn[1] = 0.0f;
    }
};

// ---- IQ4_NL: 18 B = d, qs[16] (low nibbles elements 0-15, high 16-31). One slice per block.
template <>
struct Sl<VQ_IQ4_NL> {
    static constexpr int SPB = 1, NP = 2, UB = 18, UG = 1;
    struct W {
        Span<5> b;  // d | qs[0..1], ..., qs[14..15] | 2 bytes past the block
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int, W &w) { ldspan(u, w.b); }
    static __device__ __forceinline__ void part(int, int p, int &g, int &h) {
        g = 0;
        h = p;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &, uint32_t (&c)[NP][4]) {
        uint32_t t[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) t[i] = w.b.word(i);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = __builtin_amdgcn_alignbyte(t[i + 1], t[i], 2);
            c[0][i] = iq4nl4<0>(q);
            c[1][i] = iq4nl4<4>(q);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int, float *sc, float *mn) {
        sc[0] = sc[1] = half_to_float(w.b.word(0));
        mn[0] = mn[1] = 0.0f;
    }
};

// ---- IQ4_XS: 136 B = d, scales_h (u16), scales_l[4], qs[128]. Slice s = group j (qs[16j..16j+16]).
template <>
struct Sl<VQ_IQ4_XS> {
    static constexpr int SPB = 8, NP = 2, UB = 136, UG = 8;
    struct W {
        uint32_t q[4], hd[2];
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldg(u, w.hd);
        ldg(u + 8 + 16 * s, w.q);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = s;
        h = p;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &, uint32_t (&c)[NP][4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[0][i] = iq4nl4<0>(w.q[i]);
            c[1][i] = iq4nl4<4>(w.q[i]);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int s, float *sc, float *mn) {
        const uint32_t ls = bfe(w.hd[1], 4 * s, 4) | (bfe(w.hd[0], 16 + 2 * s, 2) << 4);
        sc[0] = sc[1] = half_to_float(w.hd[0]) * static_cast<float>(static_cast<int>(ls) - 32);
        mn[0] = mn[1] = 0.0f;
    }
    // Integer form: group s weighs d (ls - 32).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.hd[0]); }
    static __device__ __forceinline__ void iscales(const W &w, int s, int (&isc)[NP]) {
        isc[0] = isc[1] = static_cast<int>(bfe(w.hd[1], 4 * s, 4) | (bfe(w.hd[0], 16 + 2 * s, 2) << 4)) - 32;
    }
};

// ---- IQ2_XXS: 66 B = d, then per group j: aux0 (4 grid indices), aux1 (4 x 7 sign bits, 4-bit scale).
template <>
struct Sl<VQ_IQ2_XXS> {
    static constexpr int SPB = 8, NP = 2, UB = 66, UG = 8;
    struct W {
        Span<2> a;  // aux0 (4 grid indices), aux1 (4 x 7 sign bits, 4-bit scale)
        Lo d;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldlo(u, w.d);
        ldspan(u + 2 + 8 * s, w.a);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = s;
        h = p;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &tb, uint32_t (&cc)[NP][4]) {
        const uint32_t a0 = w.a.word(0), a1 = w.a.word(1);
        // The four grid reads first, so their LDS round trips overlap.
        uint2 g[4];
#pragma unroll
        for (int l = 0; l < 4; ++l) g[l] = tb.grid8[bfe(a0, 8 * l, 8)];
#pragma unroll
        for (int l = 0; l < 4; ++l) {  // the sign selectors of the 7 stored bits (parity included) from LDS
            const uint2 sel = tb.ks128[bfe(a1, 7 * l, 7)];
            cc[l >> 1][2 * (l & 1)] = sign4_sel(g[l].x, sel.x);
            cc[l >> 1][2 * (l & 1) + 1] = sign4_sel(g[l].y, sel.y);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int, float *sc, float *mn) {
        sc[0] = sc[1] = half_to_float(w.d.lo()) * (0.5f + static_cast<float>(w.a.word(1) >> 28)) * 0.25f;
        mn[0] = mn[1] = 0.0f;
    }
    // Integer form: d (0.5 + s) / 4 = (d / 8) (2 s + 1).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.d.lo()) * 0.125f; }
    static __device__ __forceinline__ void iscales(const W &w, int, int (&isc)[NP]) {
        isc[0] = isc[1] = static_cast<int>(2 * (w.a.word(1) >> 28) + 1);
    }
};

// ---- IQ2_XS: 74 B = d, q u16[32] (9-bit grid index, 7 sign bits), scales[8] (nibble per half).
template <>
struct Sl<VQ_IQ2_XS> {
    static constexpr int SPB = 8, NP = 2, UB = 74, UG = 8;
    struct W {
        Span<2> a;
        Lo d, sc;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldlo(u, w.d);
        ldspan(u + 2 + 8 * s, w.a);
        ldlo(u + 66 + s, w.sc);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = s;
        h = p;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &tb, uint32_t (&cc)[NP][4]) {
        const uint32_t a[2] = {w.a.word(0), w.a.word(1)};
        uint2 g[4];  // the four grid reads first, so their LDS round trips overlap
#pragma unroll
        for (int l = 0; l < 4; ++l) g[l] = tb.grid8[bfe(a[l >> 1], 16 * (l & 1), 9)];
#pragma unroll
        for (int l = 0; l < 4; ++l) {  // sign selectors of the 7 stored bits from LDS
            const uint2 sel = tb.ks128[bfe(a[l >> 1], 16 * (l & 1) + 9, 7)];
            cc[l >> 1][2 * (l & 1)] = sign4_sel(g[l].x, sel.x);
            cc[l >> 1][2 * (l & 1) + 1] = sign4_sel(g[l].y, sel.y);
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int, float *sc, float *mn) {
        const float d = half_to_float(w.d.lo());
        const uint32_t b = w.sc.lo();
        sc[0] = d * (0.5f + static_cast<float>(b & 15)) * 0.25f;
        sc[1] = d * (0.5f + static_cast<float>(bfe(b, 4, 4))) * 0.25f;
        mn[0] = mn[1] = 0.0f;
    }
    // Integer form: half h weighs (d / 8) (2 s_h + 1).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.d.lo()) * 0.125f; }
    static __device__ __forceinline__ void iscales(const W &w, int, int (&isc)[NP]) {
        const uint32_t b = w.sc.lo();
        isc[0] = static_cast<int>(2 * (b & 15) + 1);
        isc[1] = static_cast<int>(2 * bfe(b, 4, 4) + 1);
    }
};

// ---- IQ2_S: 82 B = d, qs[32] (grid index low 8 bits), signs[32], qh[8] (2 high index bits each), scales[8].
template <>
struct Sl<VQ_IQ2_S> {
    static constexpr int SPB = 8, NP = 2, UB = 82, UG = 8;
    struct W {
        Span<1> qs, sg;
        Lo qh, sc, d;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldlo(u, w.d);
        ldspan(u + 2 + 4 * s, w.qs);
        ldspan(u + 34 + 4 * s, w.sg);
        ldlo(u + 66 + s, w.qh);
        ldlo(u + 74 + s, w.sc);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = s;
        h = p;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &tb, uint32_t (&cc)[NP][4]) {
        const uint32_t qs = w.qs.word(0), sg = w.sg.word(0), qh = w.qh.lo();
        uint2 g[4];  // the four grid reads first, so their LDS round trips overlap
#pragma unroll
        for (int l = 0; l < 4; ++l) g[l] = tb.grid8[bfe(qs, 8 * l, 8) | (bfe(qh, 2 * l, 2) << 8)];
#pragma unroll
        for (int l = 0; l < 4; ++l)
            sign8(g[l], bfe(sg, 8 * l, 8), cc[l >> 1][2 * (l & 1)], cc[l >> 1][2 * (l & 1) + 1]);
    }
    static __device__ __forceinline__ void scales(const W &w, int, float *sc, float *mn) {
        const float d = half_to_float(w.d.lo());
        const uint32_t b = w.sc.lo();
        sc[0] = d * (0.5f + static_cast<float>(b & 15)) * 0.25f;
        sc[1] = d * (0.5f + static_cast<float>(bfe(b, 4, 4))) * 0.25f;
        mn[0] = mn[1] = 0.0f;
    }
    // Integer form: half h weighs (d / 8) (2 s_h + 1).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.d.lo()) * 0.125f; }
    static __device__ __forceinline__ void iscales(const W &w, int, int (&isc)[NP]) {
        const uint32_t b = w.sc.lo();
        isc[0] = static_cast<int>(2 * (b & 15) + 1);
        isc[1] = static_cast<int>(2 * bfe(b, 4, 4) + 1);
    }
};

// ---- IQ3_XXS: 98 B = d, qs[64] (8 grid indices per group), aux u32[8] (4 x 7 sign bits, 4-bit scale).
template <>
struct Sl<VQ_IQ3_XXS> {
    static constexpr int SPB = 8, NP = 2, UB = 98, UG = 8;
    struct W {
        Span<2> q;
        Span<1> aux;
        Lo d;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldlo(u, w.d);
        ldspan(u + 2 + 8 * s, w.q);
        ldspan(u + 66 + 4 * s, w.aux);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = s;
        h = p;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &tb, uint32_t (&cc)[NP][4]) {
        const uint32_t q[2] = {w.q.word(0), w.q.word(1)};
        const uint32_t aux = w.aux.word(0);
        uint2 g[4];  // the eight grid reads first, so their LDS round trips overlap
#pragma unroll
        for (int l = 0; l < 4; ++l)
            g[l] = uint2{tb.grid4[bfe(q[l >> 1], 16 * (l & 1), 8)], tb.grid4[bfe(q[l >> 1], 16 * (l & 1) + 8, 8)]};
#pragma unroll
        for (int l = 0; l < 4; ++l)  // signs in registers: a table read here measured 4-6 % slower (eight grid reads
                                     // per 8 weights already load the LDS)
            sign8(g[l], ksigns8(bfe(aux, 7 * l, 7)), cc[l >> 1][2 * (l & 1)], cc[l >> 1][2 * (l & 1) + 1]);
    }
    static __device__ __forceinline__ void scales(const W &w, int, float *sc, float *mn) {
        sc[0] = sc[1] = half_to_float(w.d.lo()) * (0.5f + static_cast<float>(w.aux.word(0) >> 28)) * 0.5f;
        mn[0] = mn[1] = 0.0f;
    }
    // Integer form: d (0.5 + s) / 2 = (d / 4) (2 s + 1).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.d.lo()) * 0.25f; }
    static __device__ __forceinline__ void iscales(const W &w, int, int (&isc)[NP]) {
        isc[0] = isc[1] = static_cast<int>(2 * (w.aux.word(0) >> 28) + 1);
    }
};

// ---- IQ3_S: 110 B = d, qs[64], qh[8], signs[32], scales[4]. Slice s = groups 2s and 2s+1 (4 parts).
template <>
struct Sl<VQ_IQ3_S> {
    static constexpr int SPB = 4, NP = 4, UB = 110, UG = 8;
    struct W {
        Span<4> qs;
        Span<2> sg;
        Lo qh, sc, d;
    };
    static __device__ __forceinline__ void load(const uint8_t *u, int s, W &w) {
        ldlo(u, w.d);
        ldspan(u + 2 + 16 * s, w.qs);
        ldspan(u + 74 + 8 * s, w.sg);
        ldlo(u + 66 + 2 * s, w.qh);
        ldlo(u + 106 + s, w.sc);
    }
    static __device__ __forceinline__ void part(int s, int p, int &g, int &h) {
        g = 2 * s + (p >> 1);
        h = p & 1;
    }
    static constexpr int OFF = 0;
    static __device__ __forceinline__ void codes(const W &w, int, const Tabs &tb, uint32_t (&cc)[NP][4]) {
        const uint32_t qh = w.qh.lo();
        uint32_t g[2][8];  // the sixteen grid reads first, so their LDS round trips overlap
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            const uint32_t q[2] = {w.qs.word(2 * gg), w.qs.word(2 * gg + 1)};
#pragma unroll
            for (int l = 0; l < 8; ++l) g[gg][l] = tb.grid4[bfe(q[l >> 2], 8 * (l & 3), 8) | (bfe(qh, 8 * gg + l, 1) << 8)];
        }
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            const uint32_t sg = w.sg.word(gg);
#pragma unroll
            for (int m2 = 0; m2 < 4; ++m2) {  // entries 2*m2, 2*m2+1 of group gg share sign byte m2
                const int l0 = 2 * m2, l1 = 2 * m2 + 1;
                const uint32_t s8 = bfe(sg, 8 * m2, 8);
                cc[2 * gg + (l0 >> 2)][l0 & 3] = sign4(g[gg][l0], s8 & 15u);
                cc[2 * gg + (l1 >> 2)][l1 & 3] = sign4(g[gg][l1], s8 >> 4);
            }
        }
    }
    // Codes from the pre-signed table: word (entry, 4 sign bits) at sg[entry * 16 + bits].
    static __device__ __forceinline__ void codes_sg(const W &w, int, const Tabs &tb, uint32_t (&cc)[NP][4]) {
        const uint32_t qh = w.qh.lo();
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            const uint32_t q[2] = {w.qs.word(2 * gg), w.qs.word(2 * gg + 1)};
            const uint32_t sg = w.sg.word(gg);
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const uint32_t i = bfe(q[l >> 2], 8 * (l & 3), 8) | (bfe(qh, 8 * gg + l, 1) << 8);
                cc[2 * gg + (l >> 2)][l & 3] = tb.sg[(i << 4) | bfe(sg, 4 * l, 4)];
            }
        }
    }
    static __device__ __forceinline__ void scales(const W &w, int, float *sc, float *mn) {
        const float d = half_to_float(w.d.lo());
        const uint32_t b = w.sc.lo();
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            const float v = d * static_cast<float>(1 + 2 * static_cast<int>(bfe(b, 4 * gg, 4)));
            sc[2 * gg] = sc[2 * gg + 1] = v;
            mn[2 * gg] = mn[2 * gg + 1] = 0.0f;
        }
    }
    // Integer form: group gg of the slice weighs d (1 + 2 s_gg).
    static constexpr bool kInt = true;
    static __device__ __forceinline__ float dmul(const W &w) { return half_to_float(w.d.lo()); }
    static __device__ __forceinline__ void iscales(const W &w, int, int (&isc)[NP]) {
        const uint32_t b = w.sc.lo();
        isc[0] = isc[1] = static_cast<int>(1 + 2 * (b & 15));
        isc[2] = isc[3] = static_cast<int>(1 + 2 * bfe(b, 4, 4));
    }
};

// Slice decoders with a pre-signed-table form (Sl<T>::codes_sg, read through Tabs::sg).
template <int T>
constexpr bool kSignedGrid = T == VQ_IQ3_S;

// Types whose float term uses X (the 16-element activation sum) with a min coefficient.
template <int T>
constexpr bool kHasMin = T == VQ_Q2_K || T == VQ_Q4_K || T == VQ_Q5_K;
// Types whose integer partial needs X (offset codes).
template <int T>
constexpr bool kNeedsX = kHasMin<T> || T == VQ_Q3_K || T == VQ_Q6_K;
// Slice decoders that also give their scales as integers (Sl<T>::iscales, with one fp32 multiplier per unit
// Sl<T>::dmul, and for types with mins Sl<T>::imins / Sl<T>::dmin): the matvec then sums S * scale per group
// in int32 and converts once per group.
template <int T>
constexpr bool kIntScales() {
    if constexpr (requires { Sl<T>::kInt; }) return Sl<T>::kInt;
    return false;
}
// Types with a streaming code form scaled by 2^gsh(g) per group (the integer-scale path only).
template <int T>
constexpr bool kScaledCodes() {
    if constexpr (requires { Sl<T>::gsh(0); }) return true;
    return false;
}

}  // namespace vq
