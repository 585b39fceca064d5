// Mat-vec kernels of format Q6_K: every (tokens, team width) variant of mv_kernel, and the
// fp16 matrix-core kernels for several tokens.
#include "nmq_mv_impl.hpp"

namespace nmq {
template int launch_mv<NMQ_Q6_K>(MvParams, int, int, hipStream_t);
template int launch_moe_down<NMQ_Q6_K>(MvParams, Combine, int, hipStream_t);
template int launch_moe_gu<NMQ_Q6_K>(MvParams, QuantOut, hipStream_t);
template int launch_mvp<NMQ_Q6_K>(MvParams, QuantOut, hipStream_t);
template int launch_mmh<NMQ_Q6_K>(MmhParams, hipStream_t);
}  // namespace nmq
