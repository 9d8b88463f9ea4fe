// vq_quant.h -- the activation quantizer of one 32-element group, shared by the standalone quantizer
// kernels and the matvec's in-kernel quantization.
//
// Same IEEE operations as the reference CPU quantizer (/root/reference/engine/csrc/cpu/qwen_cpu.c:607-627):
// amax = max|v|, d = amax/127 (correctly rounded division), id = 1/d (0 when d == 0), q = rint(v*id) (round
// half to even, as lrintf), and the integer sums of q over elements 0..15 and 16..31.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vq {

struct QGroup {
    uint32_t q[8];   // 32 int8 codes, little-endian in 8 dwords
    float d;         // scale
    int hs0, hs1;    // sums of the codes of elements 0..15 and 16..31
    __device__ uint32_t half_sums() const {
        return (static_cast<uint32_t>(hs0) & 0xFFFFu) | (static_cast<uint32_t>(hs1) << 16);
    }
};

// v: 32 consecutive fp32 values (registers, or memory 16-byte aligned).
__device__ __forceinline__ QGroup quantize_group(const float *__restrict__ v) {
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(v[k]));
    QGroup g;
    g.d = amax / 127.0f;
    const float id = g.d > 0.0f ? 1.0f / g.d : 0.0f;
    int hs[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t p = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int q = static_cast<int>(__builtin_rintf(v[4 * k + b] * id));
            hs[k >> 2] += q;
            p |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * b);
        }
        g.q[k] = p;
    }
    g.hs0 = hs[0];
    g.hs1 = hs[1];
    return g;
}

}  // namespace vq
