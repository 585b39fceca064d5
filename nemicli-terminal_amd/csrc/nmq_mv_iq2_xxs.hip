// Mat-vec kernels of format IQ2_XXS: every (tokens, team width) variant of mv_kernel.
#include "nmq_mv_impl.hpp"

namespace nmq {
template int launch_mv<NMQ_IQ2_XXS>(MvParams, int, int, hipStream_t);
template int launch_moe_down<NMQ_IQ2_XXS>(MvParams, Combine, int, hipStream_t);
template int launch_moe_gu<NMQ_IQ2_XXS>(MvParams, QuantOut, hipStream_t);
template int launch_mvp<NMQ_IQ2_XXS>(MvParams, QuantOut, hipStream_t);
}  // namespace nmq
