// Mat-vec kernels of format Q6_K: every (tokens, team width) variant of mv_kernel.
#include "nmq_mv_impl.hpp"

namespace nmq {
template int launch_mv<NMQ_Q6_K>(MvParams, int, int, hipStream_t);
}  // namespace nmq
