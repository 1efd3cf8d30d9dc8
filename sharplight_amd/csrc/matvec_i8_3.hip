// Instantiations of the integer-dot matvec for Q4_K, Q5_K weights
// (a unit of its own so that the formats compile in parallel).
#include "matvec_i8.hpp"

namespace slhip {

int run_i8_part3(int fmt, const I8Args& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_Q4_K: return run_i8<SLHIP_FMT_Q4_K>(a, dual, st);
    case SLHIP_FMT_Q5_K: return run_i8<SLHIP_FMT_Q5_K>(a, dual, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "matvec_q8: format %d", fmt);
    }
}

}  // namespace slhip
