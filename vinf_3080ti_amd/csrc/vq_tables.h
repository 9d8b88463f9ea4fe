// vq_tables.h -- IQ codebooks and sign-mask tables for the device code (included by every kernel TU).
//
// The codebooks are expanded at compile time from the level-index encoding of vq_iq_grids.h (ggml data,
// MIT licence). Each translation unit holds its own read-only copy; the IQ3_S grid, which callers may
// replace at run time (the reference uploads it at Runtime init, qwen_runtime.cu:1272-1286), is only
// read by the IQ3_S translation unit, which also owns its setter.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define VQ_GRID_STORAGE static constexpr
#include "vq_iq_grids.h"
#include "vq_common.h"
#include "vq_slices.h"

namespace vq {

template <int N>
struct Tab64 {
    uint64_t v[N];
};
template <int N>
struct Tab32 {
    uint32_t v[N];
};

template <int N>
constexpr Tab64<N> expand_iq2(const uint16_t (&c)[N]) {
    constexpr uint64_t lv[3] = {8, 25, 43};
    Tab64<N> t{};
    for (int e = 0; e < N; ++e) {
        uint64_t x = 0;
        for (int j = 0; j < 8; ++j) x |= lv[(c[e] >> (2 * j)) & 3] << (8 * j);
        t.v[e] = x;
    }
    return t;
}

template <int N>
constexpr Tab32<N> expand_iq3(const uint16_t (&c)[N], bool iq3s) {
    constexpr uint32_t lv[8] = {4, 12, 20, 28, 36, 44, 52, 62};
    Tab32<N> t{};
    for (int e = 0; e < N; ++e) {
        uint32_t x = 0;
        for (int j = 0; j < 4; ++j) {
            const uint32_t k = (c[e] >> (3 * j)) & 7;
            x |= (iq3s ? 2 * k + 1 : lv[k]) << (8 * j);
        }
        t.v[e] = x;
    }
    return t;
}

static __device__ const Tab64<256> g_iq2xxs = expand_iq2(vq_iq2xxs_codes);
static __device__ const Tab64<512> g_iq2xs = expand_iq2(vq_iq2xs_codes);
static __device__ const Tab64<1024> g_iq2s = expand_iq2(vq_iq2s_codes);
static __device__ const Tab32<256> g_iq3xxs = expand_iq3(vq_iq3xxs_codes, false);
// IQ3_S grid: replaceable at run time (the reference uploads it at Runtime init, qwen_runtime.cu:1272-1286).
static __device__ Tab32<512> g_iq3s = expand_iq3(vq_iq3s_codes, true);

// Pre-signed IQ3_S grid words for the streaming matvec: entry (e, s) is grid entry e with byte k negated where
// bit k of s is set (4 sign bits per 4 weights), [entry 512][signs 16] (32 KB), so one LDS read replaces the
// sign expansion in registers. (For IQ2_XXS the same table, two reads per 8 weights, made LDS the limit: no
// gain, measured.)
constexpr uint32_t signed_word(uint32_t g, uint32_t s4) {
    uint32_t r = 0;
    for (int k = 0; k < 4; ++k) {
        const uint32_t b = (g >> (8 * k)) & 0xFFu;
        r |= (((s4 >> k) & 1u) ? ((0x100u - b) & 0xFFu) : b) << (8 * k);
    }
    return r;
}
template <int N>
constexpr Tab32<N * 16> sign_iq3(const Tab32<N> &g) {
    Tab32<N * 16> t{};
    for (int e = 0; e < N; ++e)
        for (uint32_t s = 0; s < 16; ++s) t.v[e * 16 + s] = signed_word(g.v[e], s);
    return t;
}
// Follows g_iq3s: the IQ3_S grid setter rewrites both.
static __device__ Tab32<512 * 16> g_iq3s_sg = sign_iq3(expand_iq3(vq_iq3s_codes, true));

__device__ __forceinline__ Grids global_grids() {
    Grids g;
    g.iq2xxs = reinterpret_cast<const uint2 *>(g_iq2xxs.v);
    g.iq2xs = reinterpret_cast<const uint2 *>(g_iq2xs.v);
    g.iq2s = reinterpret_cast<const uint2 *>(g_iq2s.v);
    g.iq3xxs = g_iq3xxs.v;
    g.iq3s = g_iq3s.v;
    return g;
}

// ---- LDS tables ----------------------------------------------------------------------------------------
// Sign entry for 8 sign bits b: the v_perm_b32 selectors of sign4 (vq_slices.h) for bits 0-3 (lo) and 4-7 (hi):
// byte k selects byte k of -g (selector k + 4) where bit k is set, else byte k of g.
__host__ __device__ constexpr uint32_t sign_sel4(uint32_t s4) { return ((s4 * 0x00810204u) & 0x04040404u) | 0x03020100u; }
__device__ __forceinline__ uint2 sign_entry(uint32_t b) { return uint2{sign_sel4(b & 15u), sign_sel4((b >> 4) & 15u)}; }

template <int T>
struct TabSpec {
    static constexpr int n8 = T == VQ_IQ2_XXS ? 256 : T == VQ_IQ2_XS ? 512 : T == VQ_IQ2_S ? 1024 : 0;
    static constexpr int n4 = T == VQ_IQ3_XXS ? 256 : T == VQ_IQ3_S ? 512 : 0;
    // Sign bits -> permute selectors, one 8-byte LDS read per 8 weights instead of ~8 VALU (the parity bit and
    // the two selectors): the 7-bit ksigns of IQ2_XXS and IQ2_XS (-6 % and -1 to -3.5 % per launch). Measured
    // slower and not taken: IQ3_XXS (ksigns; +4-6 %) and IQ2_S (raw 8 bits, 256 entries; +3.5 %).
    static constexpr bool ks = T == VQ_IQ2_XXS || T == VQ_IQ2_XS;
    static constexpr bool sm = false;
};

// Workgroup-wide: fill the LDS tables type T needs (caller synchronises afterwards).
template <int T>
__device__ __forceinline__ Tabs stage_tabs(uint2 *s8, uint32_t *s4, uint2 *sks, uint2 *ssm) {
    const Grids g = global_grids();
    Tabs tb{};
    if constexpr (TabSpec<T>::n8 > 0) {
        const uint2 *src = T == VQ_IQ2_XXS ? g.iq2xxs : T == VQ_IQ2_XS ? g.iq2xs : g.iq2s;
        for (int i = threadIdx.x; i < TabSpec<T>::n8; i += blockDim.x) s8[i] = src[i];
        tb.grid8 = s8;
    }
    if constexpr (TabSpec<T>::n4 > 0) {
        const uint32_t *src = T == VQ_IQ3_XXS ? g.iq3xxs : g.iq3s;
        for (int i = threadIdx.x; i < TabSpec<T>::n4; i += blockDim.x) s4[i] = src[i];
        tb.grid4 = s4;
    }
    if constexpr (TabSpec<T>::ks) {
        for (int i = threadIdx.x; i < 128; i += blockDim.x) sks[i] = sign_entry(ksigns(i));
        tb.ks128 = sks;
    }
    if constexpr (TabSpec<T>::sm) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) ssm[i] = sign_entry(i);
        tb.sm256 = ssm;
    }
    return tb;
}

// Global-memory copies of the sign tables for the (non-hot) hook kernels.
struct SignTabs {
    uint2 ks[128], sm[256];
};
constexpr SignTabs make_sign_tabs() {
    SignTabs t{};
    for (uint32_t i = 0; i < 256; ++i) {
        t.sm[i] = uint2{sign_sel4(i & 15u), sign_sel4(i >> 4)};
        if (i < 128) {
            uint32_t par = 0;
            for (int k = 0; k < 7; ++k) par ^= (i >> k) & 1u;
            const uint32_t b = i | (par << 7);
            t.ks[i] = uint2{sign_sel4(b & 15u), sign_sel4(b >> 4)};
        }
    }
    return t;
}
static __device__ const SignTabs g_sign = make_sign_tabs();

template <int T>
__device__ __forceinline__ Tabs global_tabs() {
    const Grids g = global_grids();
    Tabs tb{};
    tb.grid8 = T == VQ_IQ2_XXS ? g.iq2xxs : T == VQ_IQ2_XS ? g.iq2xs : g.iq2s;
    tb.grid4 = T == VQ_IQ3_XXS ? g.iq3xxs : g.iq3s;
    tb.ks128 = g_sign.ks;
    tb.sm256 = g_sign.sm;
    return tb;
}

}  // namespace vq
