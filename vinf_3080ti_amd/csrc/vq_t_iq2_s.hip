// vq_t_iq2_s.hip -- IQ2_S instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_IQ2_S)
