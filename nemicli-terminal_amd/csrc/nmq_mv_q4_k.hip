// Mat-vec kernels of format Q4_K: every (tokens, team width) variant of mv_kernel, and the
// fp16 matrix-core kernels for several tokens.
#include "nmq_mv_impl.hpp"

namespace nmq {
template int launch_mv<NMQ_Q4_K>(MvParams, int, int, hipStream_t);
template int launch_moe_down<NMQ_Q4_K>(MvParams, Combine, int, hipStream_t);
template int launch_moe_gu<NMQ_Q4_K>(MvParams, QuantOut, hipStream_t);
template int launch_mvp<NMQ_Q4_K>(MvParams, QuantOut, hipStream_t);
template int launch_mmh<NMQ_Q4_K>(MmhParams, hipStream_t);
}  // namespace nmq
