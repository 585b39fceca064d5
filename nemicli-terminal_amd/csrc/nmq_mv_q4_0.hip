// Mat-vec kernels of format Q4_0: every (tokens, team width) variant of mv_kernel.
#include "nmq_mv_impl.hpp"

namespace nmq {
template int launch_mv<NMQ_Q4_0>(MvParams, int, int, hipStream_t);
template int launch_moe_down<NMQ_Q4_0>(MvParams, Combine, int, hipStream_t);
template int launch_moe_gu<NMQ_Q4_0>(MvParams, QuantOut, hipStream_t);
template int launch_mvp<NMQ_Q4_0>(MvParams, QuantOut, hipStream_t);
}  // namespace nmq
