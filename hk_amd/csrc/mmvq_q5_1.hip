// The decode matvec kernels of Q5_1 (templates in mmvq.hpp).
#define MMVQ_INSTANTIATE
#include "mmvq.hpp"

namespace hkhip {
template mv_kernel_t pick<HKHIP_Q5_1>(int);
template mv_kernel_t mvr_pick<HKHIP_Q5_1>(int, int, int, bool);
template mv_kernel_t mvs_pick<HKHIP_Q5_1>(int, int);
} // namespace hkhip
