// vq_oracle.c -- CPU restatement of the reference's quantized matvec (TEST INFRASTRUCTURE ONLY).
//
// This file is the parity oracle. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
// may load it, and only as the checker (or the timed CPU baseline); the product path never calls it.
//
// What it restates (reference paths relative to /root/reference/engine):
//   * type ids / traits            csrc/cpu/qwen_cpu.c:21-43, src/vinf/gguf/parser.py:65-94
//   * k4 scale/min unpack          csrc/cpu/qwen_cpu.c:54-62
//   * activation quantizer         csrc/cpu/qwen_cpu.c:607-627 (d = amax/127, id = 1/d, q = lrintf(v*id),
//                                  xs = d * sum q), one 32-group at a time
//   * per-type int8 dot + scaling  csrc/cpu/qwen_cpu.c:125-342 (dot_row_q). The reference keeps eight fp32
//                                  accumulators per token (AVX2 lane k covers bytes 4k..4k+3 of a group) and
//                                  reduces them with hsum256 (:72-78); this file reproduces that exact fp32
//                                  operation order so its outputs are bit-identical to the reference CPU path.
//   * float weight path            csrc/cpu/qwen_cpu.c:345-360 (dot_row_f)
//   * row driver                   csrc/cpu/qwen_cpu.c:581-641 (Cpu_qmv), y[t*rows + r], chunks of 8 tokens
//   * dequantization               src/vinf/gguf/dequant.py:121-500, csrc/common/qwen_quant.cuh:151-279
//
// Every group decodes to 32 signed integer codes in element order plus one scale per 16-element half
// (and, for Q2_K/Q4_K/Q5_K, a min term). dequant(e) = scale_half * code - min_half exactly in fp32 (all
// products are exact: fp16 d has 11 significant bits, scales <= 7 bits, codes <= 7 bits).
//
// Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp). fp contraction is off so
// that every fused multiply-add below is an explicit fmaf, matching the reference's _mm256_fmadd_ps sites.
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../vinf_3080ti_amd/csrc/vq_iq_grids.h"

enum {
    VQO_F32 = 0, VQO_F16 = 1, VQO_Q8_0 = 8, VQO_Q2_K = 10, VQO_Q3_K = 11, VQO_Q4_K = 12, VQO_Q5_K = 13,
    VQO_Q6_K = 14, VQO_IQ2_XXS = 16, VQO_IQ2_XS = 17, VQO_IQ3_XXS = 18, VQO_IQ4_NL = 20, VQO_IQ3_S = 21,
    VQO_IQ2_S = 22, VQO_IQ4_XS = 23
};
#define VQO_MAX_TOK 8

int vqo_traits(int type, int *block_size, int *type_size) {
    int bs, ts;
    switch (type) {
        case VQO_F32: bs = 1; ts = 4; break;
        case VQO_F16: bs = 1; ts = 2; break;
        case VQO_Q8_0: bs = 32; ts = 34; break;
        case VQO_Q2_K: bs = 256; ts = 84; break;
        case VQO_Q3_K: bs = 256; ts = 110; break;
        case VQO_Q4_K: bs = 256; ts = 144; break;
        case VQO_Q5_K: bs = 256; ts = 176; break;
        case VQO_Q6_K: bs = 256; ts = 210; break;
        case VQO_IQ4_NL: bs = 32; ts = 18; break;
        case VQO_IQ3_S: bs = 256; ts = 110; break;
        case VQO_IQ4_XS: bs = 256; ts = 136; break;
        case VQO_IQ2_XXS: bs = 256; ts = 66; break;
        case VQO_IQ2_XS: bs = 256; ts = 74; break;
        case VQO_IQ2_S: bs = 256; ts = 82; break;
        case VQO_IQ3_XXS: bs = 256; ts = 98; break;
        default: return 0;
    }
    if (block_size) *block_size = bs;
    if (type_size) *type_size = ts;
    return 1;
}

static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
static const uint8_t kIq2Levels[3] = {8, 25, 43};
static const uint8_t kIq3xxsLevels[8] = {4, 12, 20, 28, 36, 44, 52, 62};

// ---- expanded codebooks (same byte layout as the reference's tables: entry i at [width*i, width*i+width))
static uint8_t g_iq2xxs[256 * 8], g_iq2xs[512 * 8], g_iq2s[1024 * 8], g_iq3xxs[256 * 4], g_iq3s[512 * 4];
static uint8_t g_ksigns[128];
static int g_ready = 0;

static void expand8(const uint16_t *codes, int n, uint8_t *out) {
    for (int e = 0; e < n; ++e)
        for (int j = 0; j < 8; ++j) out[8 * e + j] = kIq2Levels[(codes[e] >> (2 * j)) & 3];
}

static void init_tables(void) {
    if (g_ready) return;
    expand8(vq_iq2xxs_codes, 256, g_iq2xxs);
    expand8(vq_iq2xs_codes, 512, g_iq2xs);
    expand8(vq_iq2s_codes, 1024, g_iq2s);
    for (int e = 0; e < 256; ++e)
        for (int j = 0; j < 4; ++j) g_iq3xxs[4 * e + j] = kIq3xxsLevels[(vq_iq3xxs_codes[e] >> (3 * j)) & 7];
    for (int e = 0; e < 512; ++e)
        for (int j = 0; j < 4; ++j) g_iq3s[4 * e + j] = (uint8_t)(2 * ((vq_iq3s_codes[e] >> (3 * j)) & 7) + 1);
    for (int i = 0; i < 128; ++i) g_ksigns[i] = (uint8_t)(i | ((__builtin_popcount(i) & 1) << 7));
    g_ready = 1;
}

// vqo_table(id, out): copy an expanded codebook. id: 0 iq2xxs (2048 B), 1 iq2xs (4096), 2 iq2s (8192),
// 3 iq3xxs (1024), 4 iq3s (2048), 5 ksigns (128). Returns the byte count, 0 for an unknown id.
int vqo_table(int id, uint8_t *out) {
    init_tables();
    const uint8_t *src;
    int n;
    switch (id) {
        case 0: src = g_iq2xxs; n = sizeof g_iq2xxs; break;
        case 1: src = g_iq2xs; n = sizeof g_iq2xs; break;
        case 2: src = g_iq2s; n = sizeof g_iq2s; break;
        case 3: src = g_iq3xxs; n = sizeof g_iq3xxs; break;
        case 4: src = g_iq3s; n = sizeof g_iq3s; break;
        case 5: src = g_ksigns; n = sizeof g_ksigns; break;
        default: return 0;
    }
    if (out) memcpy(out, src, (size_t)n);
    return n;
}

// IEEE binary16 -> binary32, exact (the reference uses F16C _cvtsh_ss, qwen_cpu.c:48-52).
static float f16(const uint8_t *p) {
    const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    const uint32_t sign = (h & 0x8000u) << 16, exp = (h >> 10) & 0x1F, man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: renormalise
            int e = -1;
            uint32_t m = man;
            do { m <<= 1; ++e; } while ((m & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3FF) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

static void k4_scale_min(const uint8_t *s, int g, int *sc, int *m) {  // qwen_cpu.c:54-62
    if (g < 4) {
        *sc = s[g] & 63;
        *m = s[g + 4] & 63;
    } else {
        *sc = (s[g + 4] & 0x0F) | ((s[g - 4] >> 6) << 4);
        *m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
    }
}

// One decoded 32-element group.
typedef struct {
    int8_t code[32];
    float scale[2];  // per 16-element half (equal for types with one scale per group)
    float mterm;     // Q4_K/Q5_K: dmin*m (multiplies xs); 0 otherwise
    float mn[2];     // Q2_K: dmin*(s>>4) per half (multiplies xd * sum(xq)); 0 otherwise
} Group;

// Decode group g (0-based over the row) of a row of raw blocks.
static void decode_group(int type, const uint8_t *row, int g, Group *o) {
    o->mterm = 0.0f;
    o->mn[0] = o->mn[1] = 0.0f;
    switch (type) {
        case VQO_Q8_0: {  // qwen_cpu.c:147-154
            const uint8_t *blk = row + (size_t)g * 34;
            for (int i = 0; i < 32; ++i) o->code[i] = (int8_t)blk[2 + i];
            o->scale[0] = o->scale[1] = f16(blk);
            break;
        }
        case VQO_IQ4_NL: {  // qwen_cpu.c:155-162, 106-113
            const uint8_t *blk = row + (size_t)g * 18;
            for (int i = 0; i < 16; ++i) {
                o->code[i] = kIq4nl[blk[2 + i] & 15];
                o->code[16 + i] = kIq4nl[blk[2 + i] >> 4];
            }
            o->scale[0] = o->scale[1] = f16(blk);
            break;
        }
        case VQO_IQ4_XS: {  // qwen_cpu.c:163-175
            const uint8_t *blk = row + (size_t)(g / 8) * 136;
            const int j = g % 8;
            const int sh = blk[2] | (blk[3] << 8);
            const int ls = ((blk[4 + j / 2] >> (4 * (j % 2))) & 15) | (((sh >> (2 * j)) & 3) << 4);
            for (int i = 0; i < 16; ++i) {
                o->code[i] = kIq4nl[blk[8 + 16 * j + i] & 15];
                o->code[16 + i] = kIq4nl[blk[8 + 16 * j + i] >> 4];
            }
            o->scale[0] = o->scale[1] = f16(blk) * (float)(ls - 32);
            break;
        }
        case VQO_Q4_K:
        case VQO_Q5_K: {  // qwen_cpu.c:176-199
            const int ts = type == VQO_Q4_K ? 144 : 176;
            const uint8_t *blk = row + (size_t)(g / 8) * ts;
            const int j = g % 8;
            const uint8_t *qs = blk + (type == VQO_Q4_K ? 16 : 48) + 32 * (j / 2);
            int sc, m;
            k4_scale_min(blk + 4, j, &sc, &m);
            for (int i = 0; i < 32; ++i) {
                int q = (qs[i] >> (4 * (j % 2))) & 15;
                if (type == VQO_Q5_K) q |= ((blk[16 + i] >> j) & 1) << 4;
                o->code[i] = (int8_t)q;
            }
            o->scale[0] = o->scale[1] = f16(blk) * (float)sc;
            o->mterm = f16(blk + 2) * (float)m;
            break;
        }
        case VQO_Q6_K: {  // qwen_cpu.c:200-216
            const uint8_t *blk = row + (size_t)(g / 8) * 210;
            const int j = g % 8, chunk = j / 4, quarter = j % 4;
            const uint8_t *ql = blk + chunk * 64 + (quarter % 2) * 32;
            const uint8_t *qh = blk + 128 + chunk * 32;
            for (int i = 0; i < 32; ++i) {
                const int lo = (ql[i] >> (quarter >= 2 ? 4 : 0)) & 15;
                const int hi = (qh[i] >> (2 * quarter)) & 3;
                o->code[i] = (int8_t)((lo | (hi << 4)) - 32);
            }
            const float d = f16(blk + 208);
            o->scale[0] = d * (float)(int8_t)blk[192 + 2 * j];
            o->scale[1] = d * (float)(int8_t)blk[192 + 2 * j + 1];
            break;
        }
        case VQO_Q2_K: {  // qwen_cpu.c:217-238
            const uint8_t *blk = row + (size_t)(g / 8) * 84;
            const int j = g % 8;
            const uint8_t *qs = blk + 16 + 32 * (j / 4);
            for (int i = 0; i < 32; ++i) o->code[i] = (int8_t)((qs[i] >> (2 * (j % 4))) & 3);
            const float d = f16(blk + 80), dmin = f16(blk + 82);
            const uint8_t s0 = blk[2 * j], s1 = blk[2 * j + 1];
            o->scale[0] = d * (float)(s0 & 15);
            o->scale[1] = d * (float)(s1 & 15);
            o->mn[0] = dmin * (float)(s0 >> 4);
            o->mn[1] = dmin * (float)(s1 >> 4);
            break;
        }
        case VQO_Q3_K: {  // qwen_cpu.c:298-319
            const uint8_t *blk = row + (size_t)(g / 8) * 110;
            const int j = g % 8;
            const uint8_t *qs = blk + 32 + 32 * (j / 4);
            const uint8_t *sb = blk + 96;
            for (int i = 0; i < 32; ++i) {
                const int lo = (qs[i] >> (2 * (j % 4))) & 3;
                const int hb = (blk[i] >> j) & 1;
                o->code[i] = (int8_t)((lo | (hb << 2)) - 4);
            }
            const float d = f16(blk + 108);
            for (int h = 0; h < 2; ++h) {
                const int k = 2 * j + h;
                const int l4 = (sb[k % 8] >> (4 * (k / 8))) & 15;
                const int h2 = (sb[8 + k % 4] >> (2 * (k / 4))) & 3;
                o->scale[h] = d * (float)((l4 | (h2 << 4)) - 32);
            }
            break;
        }
        case VQO_IQ3_S: {  // qwen_cpu.c:320-339
            const uint8_t *blk = row + (size_t)(g / 8) * 110;
            const int j = g % 8;
            const uint8_t *qs = blk + 2 + 8 * j;
            const int qh = blk[66 + j];
            const uint32_t sb = rd32(blk + 74 + 4 * j);
            for (int l = 0; l < 8; ++l) {
                const uint8_t *e = g_iq3s + 4 * (qs[l] | (((qh >> l) & 1) << 8));
                for (int i = 0; i < 4; ++i) {
                    const int k = 4 * l + i;
                    o->code[k] = (int8_t)(((sb >> k) & 1) ? -(int)e[i] : (int)e[i]);
                }
            }
            o->scale[0] = o->scale[1] = f16(blk) * (float)(1 + 2 * ((blk[106 + j / 2] >> (4 * (j % 2))) & 15));
            break;
        }
        case VQO_IQ2_XXS:
        case VQO_IQ2_XS:
        case VQO_IQ2_S:
        case VQO_IQ3_XXS: {  // qwen_cpu.c:239-297
            const int ts = type == VQO_IQ2_XXS ? 66 : type == VQO_IQ2_XS ? 74 : type == VQO_IQ2_S ? 82 : 98;
            const uint8_t *blk = row + (size_t)(g / 8) * ts;
            const int ib = g % 8;
            const float d = f16(blk);
            for (int l = 0; l < 4; ++l) {
                uint8_t mag[8];
                int signs;
                if (type == VQO_IQ2_XXS) {
                    const uint32_t aux0 = rd32(blk + 2 + 8 * ib), aux1 = rd32(blk + 6 + 8 * ib);
                    memcpy(mag, g_iq2xxs + 8 * ((aux0 >> (8 * l)) & 0xFF), 8);
                    signs = g_ksigns[(aux1 >> (7 * l)) & 127];
                } else if (type == VQO_IQ2_XS) {
                    const int q = blk[2 + 2 * (4 * ib + l)] | (blk[3 + 2 * (4 * ib + l)] << 8);
                    memcpy(mag, g_iq2xs + 8 * (q & 511), 8);
                    signs = g_ksigns[q >> 9];
                } else if (type == VQO_IQ2_S) {
                    const int qh = blk[66 + ib];
                    memcpy(mag, g_iq2s + 8 * (blk[2 + 4 * ib + l] | ((qh << (8 - 2 * l)) & 0x300)), 8);
                    signs = blk[34 + 4 * ib + l];
                } else {
                    const uint32_t aux = rd32(blk + 66 + 4 * ib);
                    memcpy(mag, g_iq3xxs + 4 * blk[2 + 8 * ib + 2 * l], 4);
                    memcpy(mag + 4, g_iq3xxs + 4 * blk[2 + 8 * ib + 2 * l + 1], 4);
                    signs = g_ksigns[(aux >> (7 * l)) & 127];
                }
                for (int i = 0; i < 8; ++i) o->code[8 * l + i] = (int8_t)(((signs >> i) & 1) ? -(int)mag[i] : (int)mag[i]);
            }
            if (type == VQO_IQ2_XXS) {
                const uint32_t aux1 = rd32(blk + 6 + 8 * ib);
                o->scale[0] = o->scale[1] = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
            } else if (type == VQO_IQ3_XXS) {
                const uint32_t aux = rd32(blk + 66 + 4 * ib);
                o->scale[0] = o->scale[1] = d * (0.5f + (float)(aux >> 28)) * 0.5f;
            } else {
                const uint8_t sc = blk[(type == VQO_IQ2_XS ? 66 : 74) + ib];
                o->scale[0] = d * (0.5f + (float)(sc & 15)) * 0.25f;
                o->scale[1] = d * (0.5f + (float)(sc >> 4)) * 0.25f;
            }
            break;
        }
        default:
            memset(o, 0, sizeof *o);
            break;
    }
}

static int is_quant(int type) { return type != VQO_F32 && type != VQO_F16; }

// ---- dequantization ----------------------------------------------------------------------------------

// out[r*cols + c] = fp32 value of W[r][c]. Returns 0 on success, -1 for an unsupported type or shape.
int vqo_dequant_rows(int type, const uint8_t *w, int rows, int cols, float *out) {
    int bs, ts;
    if (!vqo_traits(type, &bs, &ts) || cols % bs) return -1;
    init_tables();
    const size_t rb = (size_t)(cols / bs) * ts;
    for (int r = 0; r < rows; ++r) {
        const uint8_t *row = w + (size_t)r * rb;
        float *o = out + (size_t)r * cols;
        if (type == VQO_F32) {
            memcpy(o, row, (size_t)cols * 4);
        } else if (type == VQO_F16) {
            for (int c = 0; c < cols; ++c) o[c] = f16(row + 2 * c);
        } else {
            for (int g = 0; g < cols / 32; ++g) {
                Group gr;
                decode_group(type, row, g, &gr);
                for (int i = 0; i < 32; ++i) {
                    const int h = i / 16;
                    const float v = gr.scale[h] * (float)gr.code[i];  // exact
                    const float m = type == VQO_Q2_K ? gr.mn[h] : gr.mterm;
                    o[32 * g + i] = v - m;  // the only rounding (Q2_K/Q4_K/Q5_K)
                }
            }
        }
    }
    return 0;
}

// Integer codes and per-16 scales/mins: codes[r*cols + c], scales/mins[r*(cols/16) + c/16], where
// dequant = scale * code - min exactly. Quantized types only.
int vqo_decode_codes(int type, const uint8_t *w, int rows, int cols, int8_t *codes, float *scales, float *mins) {
    int bs, ts;
    if (!vqo_traits(type, &bs, &ts) || !is_quant(type) || cols % bs) return -1;
    init_tables();
    const size_t rb = (size_t)(cols / bs) * ts;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < cols / 32; ++g) {
            Group gr;
            decode_group(type, w + (size_t)r * rb, g, &gr);
            memcpy(codes + (size_t)r * cols + 32 * g, gr.code, 32);
            for (int h = 0; h < 2; ++h) {
                scales[(size_t)r * (cols / 16) + 2 * g + h] = gr.scale[h];
                mins[(size_t)r * (cols / 16) + 2 * g + h] = type == VQO_Q2_K ? gr.mn[h] : gr.mterm;
            }
        }
    return 0;
}

// ---- activation quantizer (qwen_cpu.c:607-627) -----------------------------------------------------

int vqo_quantize_x(const float *x, int ntok, int cols, int8_t *xq, float *xd, float *xs) {
    if (cols % 32 || ntok < 1) return -1;
    const int ng = cols / 32;
    for (int t = 0; t < ntok; ++t)
        for (int g = 0; g < ng; ++g) {
            const float *v = x + (size_t)t * cols + 32 * g;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
            const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
            int sum = 0;
            for (int i = 0; i < 32; ++i) {
                const int q = (int)lrintf(v[i] * id);
                xq[(size_t)t * cols + 32 * g + i] = (int8_t)q;
                sum += q;
            }
            xd[(size_t)t * ng + g] = d;
            xs[(size_t)t * ng + g] = d * (float)sum;
        }
    return 0;
}

// ---- integer partial sums ----------------------------------------------------------------------------

// part[((t*rows + r)*ng + g)*2 + h] = sum over the 16 elements of half h of group g of code * xq.
int vqo_int_partials(int type, const uint8_t *w, int rows, int cols, const int8_t *xq, int ntok, int32_t *part) {
    int bs, ts;
    if (!vqo_traits(type, &bs, &ts) || !is_quant(type) || cols % bs) return -1;
    init_tables();
    const size_t rb = (size_t)(cols / bs) * ts;
    const int ng = cols / 32;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < ng; ++g) {
            Group gr;
            decode_group(type, w + (size_t)r * rb, g, &gr);
            for (int t = 0; t < ntok; ++t) {
                const int8_t *xv = xq + (size_t)t * cols + 32 * g;
                for (int h = 0; h < 2; ++h) {
                    int32_t s = 0;
                    for (int i = 16 * h; i < 16 * h + 16; ++i) s += (int32_t)gr.code[i] * xv[i];
                    part[(((size_t)t * rows + r) * ng + g) * 2 + h] = s;
                }
            }
        }
    return 0;
}

// ---- matvec in the reference's exact fp32 order ------------------------------------------------------

// Sum of the eight accumulators in hsum256 order (qwen_cpu.c:72-78): ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)).
static float hsum8(const float a[8]) {
    const float v0 = a[0] + a[4], v1 = a[1] + a[5], v2 = a[2] + a[6], v3 = a[3] + a[7];
    return (v0 + v2) + (v1 + v3);
}

// One row, m <= 8 tokens (qwen_cpu.c:125-342).
static void dot_row_q(int type, const uint8_t *row, int cols, const int8_t *xq, const float *xd, const float *xs,
                      int m, float *out) {
    const int ng = cols / 32;
    float acc[VQO_MAX_TOK][8];
    float minsum[VQO_MAX_TOK];
    for (int t = 0; t < m; ++t) {
        for (int k = 0; k < 8; ++k) acc[t][k] = 0.0f;
        minsum[t] = 0.0f;
    }
    for (int g = 0; g < ng; ++g) {
        Group gr;
        decode_group(type, row, g, &gr);
        for (int t = 0; t < m; ++t) {
            const int8_t *xv = xq + (size_t)t * cols + 32 * g;
            const float xdv = xd[(size_t)t * ng + g];
            const float sv[2] = {gr.scale[0] * xdv, gr.scale[1] * xdv};
            for (int k = 0; k < 8; ++k) {
                int32_t s = 0;
                for (int i = 4 * k; i < 4 * k + 4; ++i) s += (int32_t)gr.code[i] * xv[i];
                acc[t][k] = fmaf((float)s, sv[k / 4], acc[t][k]);
            }
            if (type == VQO_Q2_K) {  // acc -= sum(xq) * (dmin*m * xd) per lane (_mm256_fnmadd_ps)
                const float mv[2] = {gr.mn[0] * xdv, gr.mn[1] * xdv};
                for (int k = 0; k < 8; ++k) {
                    int32_t s = 0;
                    for (int i = 4 * k; i < 4 * k + 4; ++i) s += xv[i];
                    acc[t][k] = fmaf(-(float)s, mv[k / 4], acc[t][k]);
                }
            } else if (type == VQO_Q4_K || type == VQO_Q5_K) {  // minsum += dmin*m*xs, contracted by gcc
                minsum[t] = fmaf(gr.mterm, xs[(size_t)t * ng + g], minsum[t]);
            }
        }
    }
    for (int t = 0; t < m; ++t) out[t] = hsum8(acc[t]) - minsum[t];
}

// qwen_cpu.c:345-360: eight accumulators over columns i = 8j + k.
static void dot_row_f(int type, const uint8_t *row, int cols, const float *x, int m, float *out) {
    for (int t = 0; t < m; ++t) {
        const float *xt = x + (size_t)t * cols;
        float acc[8] = {0};
        for (int i = 0; i < cols; i += 8)
            for (int k = 0; k < 8; ++k) {
                const float wv = type == VQO_F32 ? ((const float *)row)[i + k] : f16(row + 2 * (i + k));
                acc[k] = fmaf(wv, xt[i + k], acc[k]);
            }
        out[t] = hsum8(acc);
    }
}

// y[t*rows + r] = W[r] . x[t] (Cpu_qmv, qwen_cpu.c:581-641). threads <= 0: one thread.
// Returns 0, or -1 for an unsupported type, a bad shape, or an allocation failure.
int vqo_qmv(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, float *y, int threads) {
    int bs, ts;
    if (!vqo_traits(type, &bs, &ts) || cols % bs || cols % 32 || ntok < 1 || rows < 1) return -1;
    init_tables();
    const size_t rb = (size_t)(cols / bs) * ts;
    const int nthr = threads > 0 ? threads : 1;
    (void)nthr;
    if (!is_quant(type)) {
#pragma omp parallel for schedule(static) num_threads(nthr)
        for (int r = 0; r < rows; ++r) {
            float out[VQO_MAX_TOK];
            for (int c = 0; c < ntok; c += VQO_MAX_TOK) {
                const int m = ntok - c < VQO_MAX_TOK ? ntok - c : VQO_MAX_TOK;
                dot_row_f(type, w + (size_t)r * rb, cols, x + (size_t)c * cols, m, out);
                for (int k = 0; k < m; ++k) y[(size_t)(c + k) * rows + r] = out[k];
            }
        }
        return 0;
    }
    const int ng = cols / 32;
    int8_t *xq = malloc((size_t)cols * ntok);
    float *xd = malloc(sizeof(float) * (size_t)ng * ntok), *xs = malloc(sizeof(float) * (size_t)ng * ntok);
    if (!xq || !xd || !xs) {
        free(xq);
        free(xd);
        free(xs);
        return -1;
    }
    vqo_quantize_x(x, ntok, cols, xq, xd, xs);
#pragma omp parallel for schedule(static) num_threads(nthr)
    for (int r = 0; r < rows; ++r) {
        float out[VQO_MAX_TOK];
        for (int c = 0; c < ntok; c += VQO_MAX_TOK) {
            const int m = ntok - c < VQO_MAX_TOK ? ntok - c : VQO_MAX_TOK;
            dot_row_q(type, w + (size_t)r * rb, cols, xq + (size_t)c * cols, xd + (size_t)c * ng, xs + (size_t)c * ng, m,
                      out);
            for (int k = 0; k < m; ++k) y[(size_t)(c + k) * rows + r] = out[k];
        }
    }
    free(xq);
    free(xd);
    free(xs);
    return 0;
}

// Row argmax, ties to the lowest index; only values strictly greater than the running best replace it,
// so NaN never wins (qwen_runtime.cu:850-876). All -inf/NaN rows return INT32_MAX like the reference.
int vqo_argmax_rows(const float *x, int n, int ntok, int32_t *out) {
    for (int t = 0; t < ntok; ++t) {
        float bv = -INFINITY;
        int32_t bi = 0x7fffffff;
        for (int i = 0; i < n; ++i)
            if (x[(size_t)t * n + i] > bv) {
                bv = x[(size_t)t * n + i];
                bi = i;
            }
        out[t] = bi;
    }
    return 0;
}
