// vq_t_iq3_s.hip -- IQ3_S instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_IQ3_S)

namespace vq {
int set_iq3s_grid(const uint8_t *grid) {
    return hip_status(hipMemcpyToSymbol(HIP_SYMBOL(g_iq3s), grid, 512 * 4, 0, hipMemcpyHostToDevice));
}
}  // namespace vq
