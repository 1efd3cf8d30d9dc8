// Instantiations of the integer-dot matvec for Q5_0, Q5_1, IQ4_NL weights
// (a unit of its own so that the formats compile in parallel).
#include "matvec_i8.hpp"

namespace slhip {

int run_i8_part1(int fmt, const I8Args& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_Q5_0: return run_i8<SLHIP_FMT_Q5_0>(a, dual, st);
    case SLHIP_FMT_Q5_1: return run_i8<SLHIP_FMT_Q5_1>(a, dual, st);
    case SLHIP_FMT_IQ4_NL: return run_i8<SLHIP_FMT_IQ4_NL>(a, dual, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "matvec_q8: format %d", fmt);
    }
}

}  // namespace slhip
