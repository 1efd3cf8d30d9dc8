// Instantiations of the several-token block-format matvec on the bf16 matrix cores for Q6_K, Q2_K, Q3_K
// (a unit of its own so that the formats compile in parallel).
#include "matvec_mq.hpp"

namespace slhip {

int run_mq2_part2(int fmt, const MatvecArgs& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_Q6_K: return mq2_fits<SLHIP_FMT_Q6_K>(a) ? run_mq2<SLHIP_FMT_Q6_K>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    case SLHIP_FMT_Q2_K: return mq2_fits<SLHIP_FMT_Q2_K>(a) ? run_mq2<SLHIP_FMT_Q2_K>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    case SLHIP_FMT_Q3_K: return mq2_fits<SLHIP_FMT_Q3_K>(a) ? run_mq2<SLHIP_FMT_Q3_K>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    default: return SLHIP_ERR_UNSUPPORTED;
    }
}

}  // namespace slhip
