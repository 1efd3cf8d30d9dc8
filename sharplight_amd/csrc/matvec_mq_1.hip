// Instantiations of the several-token block-format matvec on the bf16 matrix cores for Q4_K, Q5_K
// (a unit of its own so that the formats compile in parallel).
#include "matvec_mq.hpp"

namespace slhip {

int run_mq2_part1(int fmt, const MatvecArgs& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_Q4_K: return mq2_fits<SLHIP_FMT_Q4_K>(a) ? run_mq2<SLHIP_FMT_Q4_K>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    case SLHIP_FMT_Q5_K: return mq2_fits<SLHIP_FMT_Q5_K>(a) ? run_mq2<SLHIP_FMT_Q5_K>(a, dual, st) : SLHIP_ERR_UNSUPPORTED;
    default: return SLHIP_ERR_UNSUPPORTED;
    }
}

}  // namespace slhip
