// vq_t_q8_0.hip -- Q8_0 instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_Q8_0)
