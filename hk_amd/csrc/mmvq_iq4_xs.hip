// The decode matvec kernels of IQ4_XS (templates in mmvq.hpp).
#define MMVQ_INSTANTIATE
#include "mmvq.hpp"

namespace hkhip {
template mv_kernel_t pick<HKHIP_IQ4_XS>(int);
template mv_kernel_t mvr_pick<HKHIP_IQ4_XS>(int, int, int, bool);
template mv_kernel_t mvs_pick<HKHIP_IQ4_XS>(int, int);
} // namespace hkhip
