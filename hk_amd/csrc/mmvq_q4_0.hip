// The decode matvec kernels of Q4_0 (templates in mmvq.hpp).
#define MMVQ_INSTANTIATE
#include "mmvq.hpp"

namespace hkhip {
template mv_kernel_t pick<HKHIP_Q4_0>(int);
template mv_kernel_t mvr_pick<HKHIP_Q4_0>(int, int, int, bool);
template mv_kernel_t mvs_pick<HKHIP_Q4_0>(int, int);
} // namespace hkhip
