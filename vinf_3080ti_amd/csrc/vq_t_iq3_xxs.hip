// vq_t_iq3_xxs.hip -- IQ3_XXS instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_IQ3_XXS)
