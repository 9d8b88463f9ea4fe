// vq_t_iq4_xs.hip -- IQ4_XS instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_IQ4_XS)
