// vq_common.h -- GGUF quant type ids, block traits and status codes shared by host and device code.
//
// Type ids and (block_size, type_size) pairs are the GGUF/ggml ones the reference uses
// (/root/reference/engine/csrc/common/qwen_quant.cuh:17-58, src/vinf/gguf/parser.py:33-94).
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __HIPCC__
#define VQ_HD __host__ __device__
#else
#define VQ_HD
#endif

enum VqType : int {
    VQ_F32 = 0,
    VQ_F16 = 1,
    VQ_Q8_0 = 8,
    VQ_Q2_K = 10,
    VQ_Q3_K = 11,
    VQ_Q4_K = 12,
    VQ_Q5_K = 13,
    VQ_Q6_K = 14,
    VQ_IQ2_XXS = 16,
    VQ_IQ2_XS = 17,
    VQ_IQ3_XXS = 18,
    VQ_IQ4_NL = 20,
    VQ_IQ3_S = 21,
    VQ_IQ2_S = 22,
    VQ_IQ4_XS = 23,
};

// Status codes returned by every vq_* entry point (0 = success; > 0 = a hipError_t value).
enum VqStatus : int {
    VQ_OK = 0,
    VQ_ERR_TYPE = -1,       // unsupported GGUF type id
    VQ_ERR_SHAPE = -2,      // rows/cols/ntok out of range or not a multiple of the block size / 32
    VQ_ERR_WORKSPACE = -3,  // workspace missing or smaller than the *_workspace_bytes() query
    VQ_ERR_ARG = -4,        // null pointer or otherwise invalid argument
    VQ_ERR_NOT_INIT = -5,   // vq_init() has not run on this device
};

VQ_HD inline bool vq_traits(int type, int *block_size, int *type_size) {
    int bs = 0, ts = 0;
    switch (type) {
        case VQ_F32: bs = 1; ts = 4; break;
        case VQ_F16: bs = 1; ts = 2; break;
        case VQ_Q8_0: bs = 32; ts = 34; break;
        case VQ_Q2_K: bs = 256; ts = 84; break;
        case VQ_Q3_K: bs = 256; ts = 110; break;
        case VQ_Q4_K: bs = 256; ts = 144; break;
        case VQ_Q5_K: bs = 256; ts = 176; break;
        case VQ_Q6_K: bs = 256; ts = 210; break;
        case VQ_IQ4_NL: bs = 32; ts = 18; break;
        case VQ_IQ3_S: bs = 256; ts = 110; break;
        case VQ_IQ4_XS: bs = 256; ts = 136; break;
        case VQ_IQ2_XXS: bs = 256; ts = 66; break;
        case VQ_IQ2_XS: bs = 256; ts = 74; break;
        case VQ_IQ2_S: bs = 256; ts = 82; break;
        case VQ_IQ3_XXS: bs = 256; ts = 98; break;
        default: return false;
    }
    if (block_size) *block_size = bs;
    if (type_size) *type_size = ts;
    return true;
}

// Kernel-side "unit": the bytes covering one 32-element group, or for 256-element super-blocks the whole
// super-block (8 groups). F32/F16 rows are handled as 32-element pseudo-blocks (128 / 64 bytes).
template <int T>
struct VqUnit;
#define VQ_UNIT(T, BYTES, GROUPS) \
    template <>                  \
    struct VqUnit<T> {           \
        static constexpr int bytes = BYTES, groups = GROUPS; \
    };
VQ_UNIT(VQ_F32, 128, 1)
VQ_UNIT(VQ_F16, 64, 1)
VQ_UNIT(VQ_Q8_0, 34, 1)
VQ_UNIT(VQ_IQ4_NL, 18, 1)
VQ_UNIT(VQ_Q2_K, 84, 8)
VQ_UNIT(VQ_Q3_K, 110, 8)
VQ_UNIT(VQ_Q4_K, 144, 8)
VQ_UNIT(VQ_Q5_K, 176, 8)
VQ_UNIT(VQ_Q6_K, 210, 8)
VQ_UNIT(VQ_IQ3_S, 110, 8)
VQ_UNIT(VQ_IQ4_XS, 136, 8)
VQ_UNIT(VQ_IQ2_XXS, 66, 8)
VQ_UNIT(VQ_IQ2_XS, 74, 8)
VQ_UNIT(VQ_IQ2_S, 82, 8)
VQ_UNIT(VQ_IQ3_XXS, 98, 8)
#undef VQ_UNIT

// Packed activation record of one token (written by vq_pack_x, read by the quantized matvec, which copies it
// verbatim into LDS): xq[cols] int8 | xd[cols/32] fp32 | xh[cols/32] u32 (16-element sums of q: half 0 in
// the low 16 bits, half 1 in the high 16 bits, both signed). Tokens are vq_xpack_stride(cols) bytes apart.
VQ_HD constexpr int vq_xpack_h_offset(int cols) { return cols + (cols / 32) * 4; }
VQ_HD constexpr int vq_xpack_stride(int cols) { return (cols + (cols / 32) * 8 + 15) / 16 * 16; }

// Weight buffers handed to the kernels carry at least this many readable bytes past the last block: the
// streaming loads round the end of a row range up to 16 bytes.
#define VQ_TAIL_PAD 16
