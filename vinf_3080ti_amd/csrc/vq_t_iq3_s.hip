// vq_t_iq3_s.hip -- IQ3_S instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

#include <cstring>
#include <vector>

VQ_INSTANTIATE(VQ_IQ3_S)

namespace vq {
int set_iq3s_grid(const uint8_t *grid) {
    const int st = hip_status(hipMemcpyToSymbol(HIP_SYMBOL(g_iq3s), grid, 512 * 4, 0, hipMemcpyHostToDevice));
    if (st) return st;
    // The streaming kernel's pre-signed copy of the grid (entry e, 4 sign bits s: bytes negated mod 256).
    std::vector<uint32_t> sg(512 * 16);
    for (int e = 0; e < 512; ++e) {
        uint32_t g;
        std::memcpy(&g, grid + 4 * e, 4);
        for (uint32_t s4 = 0; s4 < 16; ++s4) sg[e * 16 + s4] = signed_word(g, s4);
    }
    return hip_status(hipMemcpyToSymbol(HIP_SYMBOL(g_iq3s_sg), sg.data(), sg.size() * 4, 0, hipMemcpyHostToDevice));
}
}  // namespace vq
