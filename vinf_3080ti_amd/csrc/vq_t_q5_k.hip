// vq_t_q5_k.hip -- Q5_K instantiation of the quantized matvec kernels (vq_qmv_impl.h).
#include "vq_qmv_impl.h"
#include "vq_mfma_impl.h"

VQ_INSTANTIATE(VQ_Q5_K)
template int vq::launch_mixed2<VQ_Q5_K, VQ_Q6_K>(int, const int *, const uint8_t *const *, const int *, float *const *,
                                                 int, const float *, int, hipStream_t);
VQ_STAMP_READER(vq_stamps_read_q5_k)
