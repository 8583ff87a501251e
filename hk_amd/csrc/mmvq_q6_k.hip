// The decode matvec kernels of Q6_K (templates in mmvq.hpp).
#define MMVQ_INSTANTIATE
#include "mmvq.hpp"

namespace hkhip {
template mv_kernel_t pick<HKHIP_Q6_K>(int);
template mv_kernel_t mvr_pick<HKHIP_Q6_K>(int, int, int, bool);
template mv_kernel_t mvs_pick<HKHIP_Q6_K>(int, int);
} // namespace hkhip
