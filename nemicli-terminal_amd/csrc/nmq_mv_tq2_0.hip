// Mat-vec kernels of format TQ2_0: every (tokens, team width) variant of mv_kernel.
#include "nmq_mv_impl.hpp"

namespace nmq {
template int launch_mv<NMQ_TQ2_0>(MvParams, int, int, hipStream_t);
template int launch_moe_down<NMQ_TQ2_0>(MvParams, Combine, int, hipStream_t);
template int launch_moe_gu<NMQ_TQ2_0>(MvParams, QuantOut, hipStream_t);
template int launch_mvp<NMQ_TQ2_0>(MvParams, QuantOut, hipStream_t);
}  // namespace nmq
