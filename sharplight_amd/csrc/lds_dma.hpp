#pragma once
// Direct HBM -> LDS staging shared by the matrix-core matvec kernels.
#include "common.hpp"

namespace slhip {

// global_load_lds of N bytes per lane: lane l's N bytes from base + off land at lds + N l (base and lds
// wave-uniform). Written as inline assembly so that the compiler, which would otherwise treat every later LDS
// read as possibly reading these bytes and wait for the loads (vmcnt(0)) before it -- serializing the next
// stage's loads with this stage's arithmetic -- leaves the wait to the caller: an explicit vmcnt(0) ahead of
// the barrier that publishes the stage. (The compiler's own waits for other loads stay correct: memory
// operations complete in order, so loads it does not count only make its waits longer.)
template <int N>
__device__ __forceinline__ void load_to_lds(const void* base, uint32_t off, void* lds)
{
    static_assert(N == 4 || N == 16, "load width");
    typedef __attribute__((address_space(3))) char lds_char;
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char*)lds)));
    if constexpr (N == 16)
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
}

// Bytes per staged row of the matrix-core kernels (matvec_i8_mfma, matvec_mq2): at least 16 past the row (lds_u64 reads up to 12 bytes beyond
// a piece), a whole number of staging loads, and 32 mod 64 bytes, so that the 16 rows a wave reads at once start
// in 8 different 32-byte bank groups.
// tight: no slack past the row (the caller's array then extends 16 bytes past its last row instead: the bytes
// read past a piece are discarded, so reading the next row's are harmless).
constexpr int stage_pitch(int rb, int ub, bool tight = false)
{
    int p = tight ? rb : rb + 16;
    while (p % ub != 0 || p % 64 != 32) p += 4;
    return p;
}

}  // namespace slhip
