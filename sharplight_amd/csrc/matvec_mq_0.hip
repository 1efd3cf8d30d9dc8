// Instantiations of the several-token block-format matvec on the bf16 matrix cores for Q4_0, Q8_0, Q4_1, Q5_0, Q5_1
// (a unit of its own so that the formats compile in parallel).
#include "matvec_mq.hpp"

namespace slhip {

int run_mq2_part0(int fmt, const MatvecArgs& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_Q4_0: return mq2_fits<SLHIP_FMT_Q4_0>(a) ? run_mq2<SLHIP_FMT_Q4_0>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    case SLHIP_FMT_Q8_0: return mq2_fits<SLHIP_FMT_Q8_0>(a) ? run_mq2<SLHIP_FMT_Q8_0>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    case SLHIP_FMT_Q4_1: return mq2_fits<SLHIP_FMT_Q4_1>(a) ? run_mq2<SLHIP_FMT_Q4_1>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    case SLHIP_FMT_Q5_0: return mq2_fits<SLHIP_FMT_Q5_0>(a) ? run_mq2<SLHIP_FMT_Q5_0>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    case SLHIP_FMT_Q5_1: return mq2_fits<SLHIP_FMT_Q5_1>(a) ? run_mq2<SLHIP_FMT_Q5_1>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    default: return SLHIP_ERR_UNSUPPORTED;
    }
}

}  // namespace slhip
