// Instantiations of the integer-dot matvec for MXFP4, IQ4_XS, Q6_K weights
// (a unit of its own so that the formats compile in parallel).
#include "matvec_i8.hpp"

namespace slhip {

int run_i8_part2(int fmt, const I8Args& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_MXFP4: return run_i8<SLHIP_FMT_MXFP4>(a, dual, st);
    case SLHIP_FMT_IQ4_XS: return run_i8<SLHIP_FMT_IQ4_XS>(a, dual, st);
    case SLHIP_FMT_Q6_K: return run_i8<SLHIP_FMT_Q6_K>(a, dual, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "matvec_q8: format %d", fmt);
    }
}

}  // namespace slhip
