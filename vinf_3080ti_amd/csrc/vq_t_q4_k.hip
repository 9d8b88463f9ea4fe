// vq_t_q4_k.hip -- Q4_K instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_Q4_K)
VQ_STAMP_READER(vq_stamps_read_q4_k)
