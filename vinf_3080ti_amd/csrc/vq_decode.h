// vq_decode.h -- device-side decoding of one 32-element group of a GGUF quant block into packed int8
// codes plus fp32 scales (hand-written for CDNA4; no CUDA counterpart is translated).
//
// A decoded group is 8 dwords q[0..7] holding the 32 signed int8 codes in element order (byte k of q[i]
// is element 4i+k), one scale per 16-element half (s0 for elements 0-15, s1 for 16-31), and the min
// terms of the types that have them. The value of element e is scale_half * code - min_half exactly in
// fp32; the integer dot of a half with int8 activations is sdot4 over q[0..3] or q[4..7].
//
// Layouts and scale formulas follow the reference decoders: qwen_quant.cuh:151-279 (deq8),
// qwen_cpu.c:125-342 (dot_row_q), dequant.py:121-500.
//
// All byte fields are fetched as aligned dwords from a 4-byte-aligned base plus a byte offset, and
// re-sliced with v_alignbyte_b32, so the odd block sizes (110, 210, 66, ... bytes, only 2-byte aligned)
// never need byte loads. The base may point into LDS or global memory.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_common.h"

namespace vq {

struct Group {
    uint32_t q[8];
    float s0, s1;  // scale of elements 0-15 / 16-31
    float mt;      // Q4_K/Q5_K: dmin*m, multiplies xs = xd*sum(xq)
    float mn0, mn1;  // Q2_K: dmin*(scale>>4) per half, multiplies xd*sum(xq half)
};

// Codebooks as the kernels see them (staged into LDS by each workgroup).
struct Grids {
    const uint2 *iq2xxs;  // 256 entries of 8 magnitudes
    const uint2 *iq2xs;   // 512
    const uint2 *iq2s;    // 1024
    const uint32_t *iq3xxs;  // 256 entries of 4 magnitudes
    const uint32_t *iq3s;    // 512
};

// Dword at a 4-byte-aligned offset.
template <typename Off>
__device__ __forceinline__ uint32_t ld32(const uint8_t *base, Off off) {
    return reinterpret_cast<const uint32_t *>(base)[off >> 2];
}

// Dword at any byte offset: two aligned words re-sliced (branch-free, so lanes whose blocks have
// different alignment do not diverge).
template <typename Off>
__device__ __forceinline__ uint32_t ld32u(const uint8_t *base, Off off) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(base) + (off >> 2);
    return __builtin_amdgcn_alignbyte(w[1], w[0], static_cast<uint32_t>(off) & 3u);
}

__device__ __forceinline__ float h2f(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 0xFFu; }

// Byte k (0..11) of a 12-byte field held in three dwords.
__device__ __forceinline__ uint32_t byte12(const uint32_t s[3], int k) {
    const uint32_t w = k < 4 ? s[0] : (k < 8 ? s[1] : s[2]);
    return byte_of(w, k & 3);
}

// k4_scale_min (qwen_cpu.c:54-62) for group j of a Q4_K/Q5_K super-block.
__device__ __forceinline__ void k4_scale_min(const uint32_t s[3], int j, int &sc, int &m) {
    if (j < 4) {
        sc = byte12(s, j) & 63;
        m = byte12(s, j + 4) & 63;
    } else {
        sc = (byte12(s, j + 4) & 0x0F) | ((byte12(s, j - 4) >> 6) << 4);
        m = (byte12(s, j + 4) >> 4) | ((byte12(s, j) >> 6) << 4);
    }
}

// Bytes of v each minus 32 / minus 4 (every byte of v is in 0..63 / 0..7; no borrow crosses bytes).
__device__ __forceinline__ uint32_t sub32_bytes(uint32_t v) { return (v + 0x60606060u) ^ 0x80808080u; }
__device__ __forceinline__ uint32_t sub4_bytes(uint32_t v) { return (v + 0x7C7C7C7Cu) ^ 0x80808080u; }

// Negate the bytes of g (each <= 0x80) selected by the low 4 bits of s4 (bit k -> byte k).
__device__ __forceinline__ uint32_t apply_signs4(uint32_t g, uint32_t s4) {
    s4 &= 0xFu;
    const uint32_t m = ((s4 * 0x00204081u) & 0x01010101u) * 0xFFu;
    const uint32_t neg = (0x80808080u - g) ^ 0x80808080u;
    return (neg & m) | (g & ~m);
}

// ggml ksigns_iq2xs[i]: the 7 sign bits plus an even-parity 8th bit.
__device__ __forceinline__ uint32_t ksigns(uint32_t i7) { return i7 | ((__builtin_popcount(i7) & 1u) << 7); }

// IQ4_NL codebook lookup of 4 nibble indices (one per byte, 0..15) with v_perm_b32.
__device__ __forceinline__ uint32_t iq4nl4(uint32_t n) {
    // bytes of {-127,-104,-83,-65,-49,-35,-22,-10, 1,13,25,38,53,69,89,113}
    constexpr uint32_t t0 = 0xBFADU << 16 | 0x9881u, t1 = 0xF6EAu << 16 | 0xDDCFu;
    constexpr uint32_t t2 = 0x26190D01u, t3 = 0x71594535u;
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}

// Decode group j (0..groups-1) of the unit at byte offset `off` from `base` (base 4-byte aligned).
template <int T, typename Off>
__device__ __forceinline__ void decode(const uint8_t *base, Off off, int j, const Grids &gr, Group &o) {
    o.mt = 0.0f;
    o.mn0 = o.mn1 = 0.0f;
    if constexpr (T == VQ_Q8_0) {
        const float d = h2f(ld32u(base, off));
#pragma unroll
        for (int i = 0; i < 8; ++i) o.q[i] = ld32u(base, off + 2 + 4 * i);
        o.s0 = o.s1 = d;
    } else if constexpr (T == VQ_IQ4_NL) {
        const uint32_t h = ld32u(base, off);
        const float d = h2f(h);
        uint32_t qs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = ld32u(base, off + 2 + 4 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o.q[i] = iq4nl4(qs[i] & 0x0F0F0F0Fu);
            o.q[4 + i] = iq4nl4((qs[i] >> 4) & 0x0F0F0F0Fu);
        }
        o.s0 = o.s1 = d;
    } else if constexpr (T == VQ_IQ4_XS) {  // 8-byte aligned unit
        const uint32_t w0 = ld32(base, off), w1 = ld32(base, off + 4);
        const float d = h2f(w0);
        const uint32_t sh = w0 >> 16;
        const int ls = ((byte_of(w1, j / 2) >> (4 * (j % 2))) & 15) | (((sh >> (2 * j)) & 3) << 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t qs = ld32(base, off + 8 + 16 * j + 4 * i);
            o.q[i] = iq4nl4(qs & 0x0F0F0F0Fu);
            o.q[4 + i] = iq4nl4((qs >> 4) & 0x0F0F0F0Fu);
        }
        o.s0 = o.s1 = d * static_cast<float>(ls - 32);
    } else if constexpr (T == VQ_Q4_K || T == VQ_Q5_K) {  // 16-byte aligned units
        const uint32_t w0 = ld32(base, off);
        const uint32_t s[3] = {ld32(base, off + 4), ld32(base, off + 8), ld32(base, off + 12)};
        int sc, m;
        k4_scale_min(s, j, sc, m);
        constexpr int qs_off = T == VQ_Q4_K ? 16 : 48;
        const int shift = 4 * (j & 1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t v = (ld32(base, off + qs_off + 32 * (j / 2) + 4 * i) >> shift) & 0x0F0F0F0Fu;
            if constexpr (T == VQ_Q5_K) v |= ((ld32(base, off + 16 + 4 * i) >> j) & 0x01010101u) << 4;
            o.q[i] = v;
        }
        o.s0 = o.s1 = h2f(w0) * static_cast<float>(sc);
        o.mt = h2f(w0 >> 16) * static_cast<float>(m);
    } else if constexpr (T == VQ_Q6_K) {  // ql[128]@0 qh[64]@128 scales[16]@192 d@208
        const int chunk = j / 4, quarter = j % 4;
        const int lsh = quarter >= 2 ? 4 : 0, hsh = 2 * quarter;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = (ld32u(base, off + chunk * 64 + (quarter & 1) * 32 + 4 * i) >> lsh) & 0x0F0F0F0Fu;
            const uint32_t hi = (ld32u(base, off + 128 + chunk * 32 + 4 * i) >> hsh) & 0x03030303u;
            o.q[i] = sub32_bytes(lo | (hi << 4));
        }
        const uint32_t sw = ld32u(base, off + 192 + 2 * j);  // scales[2j], scales[2j+1]
        const float d = h2f(ld32u(base, off + 208));
        o.s0 = d * static_cast<float>(static_cast<int8_t>(sw & 0xFF));
        o.s1 = d * static_cast<float>(static_cast<int8_t>((sw >> 8) & 0xFF));
    } else if constexpr (T == VQ_Q2_K) {  // 4-byte aligned: scales[16]@0 qs[64]@16 d@80 dmin@82
        const int sh = 2 * (j % 4);
#pragma unroll
        for (int i = 0; i < 8; ++i) o.q[i] = (ld32(base, off + 16 + 32 * (j / 4) + 4 * i) >> sh) & 0x03030303u;
        const uint32_t sw = ld32(base, off + 4 * (j / 2)) >> (16 * (j & 1));
        const uint32_t dd = ld32(base, off + 80);
        const float d = h2f(dd), dmin = h2f(dd >> 16);
        o.s0 = d * static_cast<float>(sw & 0x0F);
        o.s1 = d * static_cast<float>((sw >> 8) & 0x0F);
        o.mn0 = dmin * static_cast<float>((sw >> 4) & 0x0F);
        o.mn1 = dmin * static_cast<float>((sw >> 12) & 0x0F);
    } else if constexpr (T == VQ_Q3_K) {  // hmask[32]@0 qs[64]@32 scales[12]@96 d@108
        const int sh = 2 * (j % 4);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = (ld32u(base, off + 32 + 32 * (j / 4) + 4 * i) >> sh) & 0x03030303u;
            const uint32_t hb = (ld32u(base, off + 4 * i) >> j) & 0x01010101u;
            o.q[i] = sub4_bytes(lo | (hb << 2));
        }
        const uint32_t s[3] = {ld32u(base, off + 96), ld32u(base, off + 100), ld32u(base, off + 104)};
        const float d = h2f(ld32u(base, off + 108));
        float sc[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 2 * j + h;
            const int l4 = (byte12(s, k % 8) >> (4 * (k / 8))) & 0x0F;
            const int h2 = (byte12(s, 8 + k % 4) >> (2 * (k / 4))) & 0x03;
            sc[h] = d * static_cast<float>((l4 | (h2 << 4)) - 32);
        }
        o.s0 = sc[0];
        o.s1 = sc[1];
    } else if constexpr (T == VQ_IQ3_S) {  // d@0 qs[64]@2 qh[8]@66 signs[32]@74 scales[4]@106
        const float d = h2f(ld32u(base, off));
        const uint32_t qa = ld32u(base, off + 2 + 8 * j), qb = ld32u(base, off + 6 + 8 * j);
        const uint32_t qh = ld32u(base, off + 66 + j) & 0xFF;
        const uint32_t sg = ld32u(base, off + 74 + 4 * j);
        const uint32_t scb = ld32u(base, off + 106 + j / 2) & 0xFF;
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const uint32_t idx = byte_of(l < 4 ? qa : qb, l & 3) | (((qh >> l) & 1u) << 8);
            o.q[l] = apply_signs4(gr.iq3s[idx], sg >> (4 * l));
        }
        o.s0 = o.s1 = d * static_cast<float>(1 + 2 * static_cast<int>((scb >> (4 * (j % 2))) & 0x0F));
    } else if constexpr (T == VQ_IQ2_XXS) {  // d@0, per group: aux0 aux1 @2+8j
        const float d = h2f(ld32u(base, off));
        const uint32_t aux0 = ld32u(base, off + 2 + 8 * j), aux1 = ld32u(base, off + 6 + 8 * j);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint2 g = gr.iq2xxs[byte_of(aux0, l)];
            const uint32_t sg = ksigns((aux1 >> (7 * l)) & 127u);
            o.q[2 * l] = apply_signs4(g.x, sg);
            o.q[2 * l + 1] = apply_signs4(g.y, sg >> 4);
        }
        o.s0 = o.s1 = d * (0.5f + static_cast<float>(aux1 >> 28)) * 0.25f;
    } else if constexpr (T == VQ_IQ2_XS) {  // d@0 q u16[32]@2 scales[8]@66
        const float d = h2f(ld32u(base, off));
        const uint32_t qa = ld32u(base, off + 2 + 8 * j), qb = ld32u(base, off + 6 + 8 * j);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t q = ((l < 2 ? qa : qb) >> (16 * (l & 1))) & 0xFFFFu;
            const uint2 g = gr.iq2xs[q & 511u];
            const uint32_t sg = ksigns(q >> 9);
            o.q[2 * l] = apply_signs4(g.x, sg);
            o.q[2 * l + 1] = apply_signs4(g.y, sg >> 4);
        }
        const uint32_t sc = ld32u(base, off + 66 + j) & 0xFF;
        o.s0 = d * (0.5f + static_cast<float>(sc & 15)) * 0.25f;
        o.s1 = d * (0.5f + static_cast<float>(sc >> 4)) * 0.25f;
    } else if constexpr (T == VQ_IQ2_S) {  // d@0 qs[32]@2 signs[32]@34 qh[8]@66 scales[8]@74
        const float d = h2f(ld32u(base, off));
        const uint32_t qs = ld32u(base, off + 2 + 4 * j), sg = ld32u(base, off + 34 + 4 * j);
        const uint32_t qh = ld32u(base, off + 66 + j) & 0xFF;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t idx = byte_of(qs, l) | ((qh << (8 - 2 * l)) & 0x300u);
            const uint2 g = gr.iq2s[idx];
            const uint32_t s8 = byte_of(sg, l);
            o.q[2 * l] = apply_signs4(g.x, s8);
            o.q[2 * l + 1] = apply_signs4(g.y, s8 >> 4);
        }
        const uint32_t sc = ld32u(base, off + 74 + j) & 0xFF;
        o.s0 = d * (0.5f + static_cast<float>(sc & 15)) * 0.25f;
        o.s1 = d * (0.5f + static_cast<float>(sc >> 4)) * 0.25f;
    } else if constexpr (T == VQ_IQ3_XXS) {  // d@0 qs[64]@2 aux u32[8]@66
        const float d = h2f(ld32u(base, off));
        const uint32_t qa = ld32u(base, off + 2 + 8 * j), qb = ld32u(base, off + 6 + 8 * j);
        const uint32_t aux = ld32u(base, off + 66 + 4 * j);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t qw = l < 2 ? qa : qb;
            const uint32_t sg = ksigns((aux >> (7 * l)) & 127u);
            o.q[2 * l] = apply_signs4(gr.iq3xxs[byte_of(qw, 2 * (l & 1))], sg);
            o.q[2 * l + 1] = apply_signs4(gr.iq3xxs[byte_of(qw, 2 * (l & 1) + 1)], sg >> 4);
        }
        o.s0 = o.s1 = d * (0.5f + static_cast<float>(aux >> 28)) * 0.5f;
    }
}

}  // namespace vq
