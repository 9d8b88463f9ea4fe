// vq_lds.h -- direct global -> LDS copies (global_load_lds_dwordx4) and the waits that go with them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vq {

// IQ grid tables, packed activation records, the prefill GEMM's tiles and the gated delta rule's inputs reach
// LDS through global_load_lds_dwordx4 (each lane moves 16 bytes; a wave writes 1 KB contiguously at M0). The DMA
// is issued from inline asm, so the compiler does not count it; the kernel waits on vmcnt itself (loads retire
// in order, so "at most N outstanding" means "all but the last N landed").
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void *)p));
}
// 64 lanes x 16 bytes: lane i copies base[voff_i .. +16) to LDS dst + 16 i. base and dst are wave-uniform
// (readfirstlane: values the compiler cannot prove uniform would otherwise reach the "s" operands in VGPRs).
// dst goes to the asm as a pointer operand: the compiler then knows the asm may write that LDS (given only the
// integer address, it treats DMA-filled __shared__ arrays as never written and folds their reads away).
__device__ __forceinline__ void dma16(const void *base, uint32_t voff, void *dst) {
    const uint64_t b = reinterpret_cast<uintptr_t>(base);
    const uint64_t bs = (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)))) << 32) |
                        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xFFFFFFFFu)));
    const uint32_t ls = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_addr(dst))));
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, %0" ::"s"(reinterpret_cast<const void *>(bs)), "v"(voff), "s"(ls),
                 "v"(dst)
                 : "memory", "m0");
}
// The same copy with base and dst in SGPRs (dst still a pointer operand of the asm, see dma16): no VALU per copy
// when the caller's base and dst are already uniform values.
__device__ __forceinline__ void dma16s(const void *base, uint32_t voff, void *dst) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, %0" ::"s"(base), "v"(voff), "s"(lds_addr(dst)), "s"(dst)
                 : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

}  // namespace vq
