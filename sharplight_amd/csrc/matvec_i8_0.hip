// Instantiations of the integer-dot matvec for Q8_0, Q4_0, Q4_1 weights
// (a unit of its own so that the formats compile in parallel).
#include "matvec_i8.hpp"

namespace slhip {

int run_i8_part0(int fmt, const I8Args& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_Q8_0: return run_i8<SLHIP_FMT_Q8_0>(a, dual, st);
    case SLHIP_FMT_Q4_0: return run_i8<SLHIP_FMT_Q4_0>(a, dual, st);
    case SLHIP_FMT_Q4_1: return run_i8<SLHIP_FMT_Q4_1>(a, dual, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "matvec_q8: format %d", fmt);
    }
}

}  // namespace slhip
