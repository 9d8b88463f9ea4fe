// vq_t_q2_k.hip -- Q2_K instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_Q2_K)
