#pragma once
// The integer-dot matvec's 64-value slices (included by matvec_i8.hpp inside namespace slhip, after unit_dot).
//
// A slice is two 32-value units of a row together with the bytes of their block or super-block scales,
// decoded from a few words into two I8Units (codes, multipliers, offsets) with word-wide arithmetic, so that
// each lane decodes only its own scales.
//   * The LDS-staged kernel (matvec_i8) reads each lane's slice out of the row images as words: Q4_K / Q5_K
//     (RegPiece::lds_load: aligned 16-byte reads), Q6_K below three tokens (2-byte aligned super-blocks:
//     aligned words joined by funnel shifts), IQ4_XS in passes of more than four tokens (8-byte reads), and the
//     32-value block formats where that measured ahead (SlicePiece32: two blocks as one run of words).
//   * Q6_K from three tokens and IQ4_XS: the register-piece kernel below loads each lane's slice from HBM
//     straight into registers (unaligned loads: their blocks are only 2- or 8-byte aligned), with no row
//     image in LDS, no LDS store and no per-chunk address arithmetic. A wave takes rows n, n + W, ... (W waves
//     in the grid, sized so that each wave gets the same number of rows), one (row, group of 64 slices) item
//     at a time: the next D - 1 items' loads are in flight while one is computed (D register sets in
//     rotation). The block's quantized activation rows sit in LDS; a row's output is the wave sum of its
//     lanes' unit terms (unit_dot, the same per-unit arithmetic as the LDS-staged kernel).
// Reads of a row's last slice may run up to 12 bytes past it, into the image's 16-byte pad.

typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));

__device__ __forceinline__ uint4 ldw16(const char* p)
{
    const u32x4_a2 v = *reinterpret_cast<const u32x4_a2*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ldw4(const char* p) { return *reinterpret_cast<const u32_a2*>(p); }
__device__ __forceinline__ uint32_t ldw2(const char* p) { return *reinterpret_cast<const uint16_t*>(p); }

__device__ __forceinline__ uint32_t word_of(const uint4& v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; }

// A lane's raw bytes for slice s of a row (NW 16-byte registers) of the super-block formats, and the two units
// they hold with the unit index (32-value units from the row's start) of each; field layouts as in i8_unit.
template <int FMT> struct RegPiece;

// 32-value block formats: slice s is blocks 2 s and 2 s + 1, 2 BB bytes at byte 2 BB s of the row image (4-byte
// aligned for every format but MXFP4), read as one run of words; the fields sit at fixed byte offsets in it.
template <int BB>
struct SliceWords {
    static constexpr int N = (2 * BB + 3) / 4 + 1;  // words read (one spare for the funnel shifts)
    uint32_t w[N];
    // the run starting at byte off of the image (even): aligned reads joined by funnel shifts when off % 4 == 2
    __device__ __forceinline__ void read(const uint32_t* img, int off)
    {
        const uint32_t* q = img + (off >> 2);
        if (BB % 2 == 0) {  // 2 BB s is a multiple of 4
#pragma unroll
            for (int k = 0; k < N; k++) w[k] = q[k];
        } else {
            const uint32_t sh = static_cast<uint32_t>(off & 3) * 8;
            uint32_t d[N + 1];
#pragma unroll
            for (int k = 0; k <= N; k++) d[k] = q[k];
#pragma unroll
            for (int k = 0; k < N; k++) w[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], sh);
        }
    }
    // 4 bytes at byte b of the slice (b a compile-time constant)
    __device__ __forceinline__ uint32_t at(int b) const
    {
        return (b & 3) ? __builtin_amdgcn_alignbit(w[(b >> 2) + 1], w[b >> 2], (b & 3) * 8) : w[b >> 2];
    }
};

// the codes of one 32-value block from its 16 bytes of nibbles q (and, Q5_x, its 32 fifth bits qh), as i8_unit
template <int FMT>
__device__ __forceinline__ void nibble_codes(I8Unit& u, const uint32_t (&q)[4], uint32_t qh)
{
    using F = Fmt<FMT>;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
        if constexpr (F::QH >= 0) {
            lo |= ((((qh >> (4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
            hi |= ((((qh >> (16 + 4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
        }
        if constexpr (FMT == SLHIP_FMT_IQ4_NL) {
            lo = iq4_lookup4(lo);
            hi = iq4_lookup4(hi);
        } else if constexpr (FMT == SLHIP_FMT_MXFP4) {
            lo = fp4_lookup4(lo);
            hi = fp4_lookup4(hi);
        }
        u.c[k] = lo;
        u.c[4 + k] = hi;
    }
}

template <int FMT> struct SlicePiece32 {
    static constexpr int BB = FMT == SLHIP_FMT_MXFP4 ? 17 : Fmt<FMT>::BB;
    using W = SliceWords<BB>;
    // block h (0, 1) of the slice into u
    static __device__ __forceinline__ void block(const W& sw, int h, I8Unit& u)
    {
        const int o = h * BB;
        if constexpr (FMT == SLHIP_FMT_Q8_0) {
            u.a0 = u.a1 = f16_lo(sw.at(o));
            u.b0 = u.b1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) u.c[k] = sw.at(o + 2 + 4 * k);
        } else if constexpr (FMT == SLHIP_FMT_MXFP4) {
            u.a0 = u.a1 = e8m0_half(sw.at(o) & 0xFFu);
            u.b0 = u.b1 = 0.0f;
            const uint32_t q[4] = {sw.at(o + 1), sw.at(o + 5), sw.at(o + 9), sw.at(o + 13)};
            nibble_codes<FMT>(u, q, 0);
        } else {
            using F = Fmt<FMT>;
            const uint32_t h0 = sw.at(o);
            const float d = f16_lo(h0);
            u.a0 = u.a1 = d;
            if constexpr (FMT == SLHIP_FMT_IQ4_NL) u.b0 = u.b1 = 0.0f;
            else if constexpr (F::M) u.b0 = u.b1 = f16_hi(h0);
            else u.b0 = u.b1 = static_cast<float>(F::OFF) * d;
            const uint32_t qh = F::QH >= 0 ? sw.at(o + (F::QH >= 0 ? F::QH : 0)) : 0u;
            const uint32_t q[4] = {sw.at(o + F::QS), sw.at(o + F::QS + 4), sw.at(o + F::QS + 8), sw.at(o + F::QS + 12)};
            nibble_codes<FMT>(u, q, qh);
        }
    }
    static __device__ __forceinline__ void lds_units(const uint32_t* img, int s, I8Unit& u0, I8Unit& u1, int& j0, int& j1)
    {
        W sw;
        sw.read(img, 2 * BB * s);
        block(sw, 0, u0);
        block(sw, 1, u1);
        j0 = 2 * s;
        j1 = j0 + 1;
    }
};

// Q4_K / Q5_K sub-blocks jj, jj + 1 (jj = 2 (p & 1), p = the slice's quarter of its super-block) of the 6-bit
// scales and minimums from the header words (scales[0..3], [4..7], [8..11]): two bytes at a time.
__device__ __forceinline__ void k_scales2(const uint4& h, int p, uint32_t& sc, uint32_t& mn)
{
    const int sh = 16 * (p & 1);
    const uint32_t Y = h.y >> sh, Z = h.z >> sh, W = h.w >> sh;
    if (p >= 2) {
        sc = (W & 0x0F0Fu) | ((Y >> 2) & 0x3030u);
        mn = ((W >> 4) & 0x0F0Fu) | ((Z >> 2) & 0x3030u);
    } else {
        sc = Y & 0x3F3Fu;
        mn = Z & 0x3F3Fu;
    }
}

template <int FMT> struct RegPieceK45 {  // {f16 d, f16 dmin, u8 scales[12], [u8 qh[32]], u8 qs[128]}
    static constexpr bool K5 = FMT == SLHIP_FMT_Q5_K;
    static constexpr int NW = K5 ? 5 : 3;
    // a slice's header and code words from a row image in LDS (super-blocks and their code runs are 16-byte
    // aligned there); with Q5_K, the 32 bytes of fifth bits
    static __device__ __forceinline__ void lds_load(uint4* w, const uint32_t* img, int s)
    {
        const uint4* b = reinterpret_cast<const uint4*>(img) + (K5 ? 11 : 9) * (s >> 2);
        w[0] = b[0];
        const uint4* q = b + (K5 ? 3 : 1) + 2 * (s & 3);
        w[1] = q[0];
        w[2] = q[1];
        if constexpr (K5) {
            w[3] = b[1];
            w[4] = b[2];
        }
    }
    static __device__ __forceinline__ void units(const uint4* w, int s, I8Unit& u0, I8Unit& u1, int& j0, int& j1)
    {
        const int p = s & 3;
        j0 = 2 * s;
        j1 = j0 + 1;
        uint32_t sc, mn;
        k_scales2(w[0], p, sc, mn);
        const float d = f16_lo(w[0].x), dm = f16_hi(w[0].x);
        u0.a0 = u0.a1 = __fmul_rn(d, static_cast<float>(sc & 0xFFu));
        u1.a0 = u1.a1 = __fmul_rn(d, static_cast<float>(sc >> 8));
        u0.b0 = u0.b1 = -__fmul_rn(dm, static_cast<float>(mn & 0xFFu));
        u1.b0 = u1.b1 = -__fmul_rn(dm, static_cast<float>(mn >> 8));
        const int jj = 2 * p;  // sub-block of the super-block (bit of qh)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t q = word_of(w[1 + k / 4], k % 4);
            uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
            if constexpr (K5) {
                const uint32_t qh = word_of(w[3 + k / 4], k % 4);
                lo |= ((qh >> jj) & 0x01010101u) << 4;
                hi |= ((qh >> (jj + 1)) & 0x01010101u) << 4;
            }
            u0.c[k] = lo;
            u1.c[k] = hi;
        }
    }
};
template <> struct RegPiece<SLHIP_FMT_Q4_K> : RegPieceK45<SLHIP_FMT_Q4_K> {};
template <> struct RegPiece<SLHIP_FMT_Q5_K> : RegPieceK45<SLHIP_FMT_Q5_K> {};

template <> struct RegPiece<SLHIP_FMT_IQ4_XS> {  // {f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128]}
    static constexpr int NW = 3;
    // the same words from a row image in LDS (136-byte super-blocks: 8-byte aligned there)
    static __device__ __forceinline__ void lds_load(uint4* w, const uint32_t* img, int s)
    {
        const uint2* b = reinterpret_cast<const uint2*>(img) + 17 * (s >> 2);
        const uint2 h = b[0], q0 = b[1 + 4 * (s & 3)], q1 = b[2 + 4 * (s & 3)], q2 = b[3 + 4 * (s & 3)], q3 = b[4 + 4 * (s & 3)];
        w[0] = make_uint4(h.x, h.y, 0u, 0u);
        w[1] = make_uint4(q0.x, q0.y, q1.x, q1.y);
        w[2] = make_uint4(q2.x, q2.y, q3.x, q3.y);
    }
    static __device__ __forceinline__ void load(uint4* w, const char* row, int s)
    {
        const char* b = row + 136 * (s >> 2);
        w[0].x = ldw4(b);
        w[0].y = ldw4(b + 4);
        w[1] = ldw16(b + 8 + 32 * (s & 3));
        w[2] = ldw16(b + 24 + 32 * (s & 3));
    }
    static __device__ __forceinline__ void units(const uint4* w, int s, I8Unit& u0, I8Unit& u1, int& j0, int& j1)
    {
        const int p = s & 3;
        j0 = 2 * s;
        j1 = j0 + 1;
        const float d = f16_lo(w[0].x);
        const uint32_t sh = (w[0].x >> (16 + 4 * p)) & 0xFu;  // the high bits of sub-blocks 2p and 2p + 1
        const uint32_t sl = (w[0].y >> (8 * p)) & 0xFFu;
        const int ls0 = static_cast<int>((sl & 0xFu) | ((sh & 3u) << 4));
        const int ls1 = static_cast<int>((sl >> 4) | ((sh >> 2) << 4));
        u0.a0 = u0.a1 = __fmul_rn(d, static_cast<float>(ls0 - 32));
        u1.a0 = u1.a1 = __fmul_rn(d, static_cast<float>(ls1 - 32));
        u0.b0 = u0.b1 = u1.b0 = u1.b1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q0 = word_of(w[1], k), q1 = word_of(w[2], k);
            u0.c[k] = iq4_lookup4(q0 & 0x0F0F0F0Fu);
            u0.c[4 + k] = iq4_lookup4((q0 >> 4) & 0x0F0F0F0Fu);
            u1.c[k] = iq4_lookup4(q1 & 0x0F0F0F0Fu);
            u1.c[4 + k] = iq4_lookup4((q1 >> 4) & 0x0F0F0F0Fu);
        }
    }
};

template <> struct RegPiece<SLHIP_FMT_Q6_K> {  // {ql[128], qh[64], i8 scales[16], f16 d}
    // slice quarter p: ql[32 p .. + 31] holds quarters qt = p & 1 (low nibbles) and qt + 2 (high nibbles) of
    // half n = p / 2, whose two high bits are in qh[32 n ..]: units 4 n + qt and 4 n + qt + 2 of the super-block
    static constexpr int NW = 5;
    // the same words from a row image in LDS (210-byte super-blocks: 2-byte aligned there): each run of
    // words as aligned reads joined by funnel shifts (the last super-block's scales read 2 bytes into the
    // image's pad)
    static __device__ __forceinline__ void lds_load(uint4* w, const uint32_t* img, int s)
    {
        const int p = s & 3, n = p >> 1;
        const int o = 210 * (s >> 2);
        auto run8 = [&](int off, uint4& a, uint4& b) {
            const uint32_t* q = img + (off >> 2);
            const uint32_t sh = static_cast<uint32_t>(off & 3) * 8;
            uint32_t d[9];
#pragma unroll
            for (int k = 0; k < 9; k++) d[k] = q[k];
            a = make_uint4(__builtin_amdgcn_alignbit(d[1], d[0], sh), __builtin_amdgcn_alignbit(d[2], d[1], sh),
                           __builtin_amdgcn_alignbit(d[3], d[2], sh), __builtin_amdgcn_alignbit(d[4], d[3], sh));
            b = make_uint4(__builtin_amdgcn_alignbit(d[5], d[4], sh), __builtin_amdgcn_alignbit(d[6], d[5], sh),
                           __builtin_amdgcn_alignbit(d[7], d[6], sh), __builtin_amdgcn_alignbit(d[8], d[7], sh));
        };
        run8(o + 32 * p, w[0], w[1]);
        run8(o + 128 + 32 * n, w[2], w[3]);
        const int so = o + 192 + 8 * n;
        const uint32_t* q = img + (so >> 2);
        const uint32_t sh = static_cast<uint32_t>(so & 3) * 8;
        const uint32_t e0 = q[0], e1 = q[1], e2 = q[2];
        w[4].x = __builtin_amdgcn_alignbit(e1, e0, sh);
        w[4].y = __builtin_amdgcn_alignbit(e2, e1, sh);
        w[4].z = lds_u16(img, o + 208);
    }
    static __device__ __forceinline__ void load(uint4* w, const char* row, int s)
    {
        const int p = s & 3, n = p >> 1;
        const char* b = row + 210 * (s >> 2);
        w[0] = ldw16(b + 32 * p);
        w[1] = ldw16(b + 32 * p + 16);
        w[2] = ldw16(b + 128 + 32 * n);
        w[3] = ldw16(b + 144 + 32 * n);
        w[4].x = ldw4(b + 192 + 8 * n);
        w[4].y = ldw4(b + 196 + 8 * n);
        w[4].z = ldw2(b + 208);
    }
    static __device__ __forceinline__ void units(const uint4* w, int s, I8Unit& u0, I8Unit& u1, int& j0, int& j1)
    {
        const int p = s & 3, n = p >> 1, qt = p & 1;
        j0 = 8 * (s >> 2) + 4 * n + qt;
        j1 = j0 + 2;
        const float d = f16_lo(w[4].z);
        const uint32_t s0 = w[4].x >> (16 * qt), s1 = w[4].y >> (16 * qt);
        u0.a0 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s0 & 0xFFu)));
        u0.a1 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>((s0 >> 8) & 0xFFu)));
        u1.a0 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s1 & 0xFFu)));
        u1.a1 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>((s1 >> 8) & 0xFFu)));
        u0.b0 = -32.0f * u0.a0;
        u0.b1 = -32.0f * u0.a1;
        u1.b0 = -32.0f * u1.a0;
        u1.b1 = -32.0f * u1.a1;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t l = word_of(w[k / 4], k % 4), h = word_of(w[2 + k / 4], k % 4);
            u0.c[k] = (l & 0x0F0F0F0Fu) | (((h >> (2 * qt)) & 0x03030303u) << 4);
            u1.c[k] = ((l >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * qt + 4)) & 0x03030303u) << 4);
        }
    }
};

// Formats whose slices the LDS-staged kernel reads as aligned 16-byte words.
template <int FMT> constexpr bool kLdsPiece = FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K || FMT == SLHIP_FMT_Q6_K || FMT == SLHIP_FMT_IQ4_XS;
// The 32-value block formats by slices in passes of TT tokens: where it measured ahead of the per-unit decode on
// [14336, 4096] gate/up pairs (µs, slices against units: T1 Q4_0 16.5 / 17.8, Q8_0 25.5 / 29.2, Q5_0 19.1 /
// 21.1, IQ4_NL 20.1 / 21.8, MXFP4 21.0 / 21.8; T4 Q8_0 39.2 / 44.8). Elsewhere the slices' registers (~140-160
// against ~120) cost more than the reads they save (Q4_1, Q5_1 at one token; most formats at two or four).
template <int FMT, int TT>
constexpr bool kSlice32 = (TT == 1 && (FMT == SLHIP_FMT_Q8_0 || FMT == SLHIP_FMT_Q4_0 || FMT == SLHIP_FMT_Q5_0 ||
                                       FMT == SLHIP_FMT_IQ4_NL || FMT == SLHIP_FMT_MXFP4)) ||
                          (TT == 4 && FMT == SLHIP_FMT_Q8_0);
// Formats whose LDS-staged decode goes by 64-value slices.
template <int FMT, int TT> constexpr bool kSliceLds = kLdsPiece<FMT> || kSlice32<FMT, TT>;

// A slice's two units from a row image in LDS.
template <int FMT>
__device__ __forceinline__ void slice_units(const uint32_t* img, int s, I8Unit& u0, I8Unit& u1, int& j0, int& j1)
{
    if constexpr (kLdsPiece<FMT>) {
        uint4 w[RegPiece<FMT>::NW];
        RegPiece<FMT>::lds_load(w, img, s);
        RegPiece<FMT>::units(w, s, u0, u1, j0, j1);
    } else {
        SlicePiece32<FMT>::lds_units(img, s, u0, u1, j0, j1);
    }
}

// Formats the register-piece kernel takes (measured against the LDS-staged kernel with per-unit decode on
// [14336, 4096] gate/up pairs at one to four tokens: Q6_K 30.0 / 32.7 / 38.9 us against 30.3 / 35.7 / 49.6,
// IQ4_XS ~10% ahead, also against slices read from the row images; for
// the 32-value block formats the scattered 16-byte pieces cost more L1 accesses than they save, and Q4_K /
// Q5_K run faster as slices of the LDS row images).
template <int FMT> constexpr bool kRegPieceKernel = FMT == SLHIP_FMT_Q6_K || FMT == SLHIP_FMT_IQ4_XS;
// Q6_K below three tokens reads its slices from the LDS row images instead (T1 / T2 29.5 / 32.4 -> 23.4 /
// 30.3 us; at four tokens the register kernel stays ahead, 38.4 against 39.6).
template <int FMT> constexpr int kRegPieceMinT = FMT == SLHIP_FMT_Q6_K ? 3 : 1;

constexpr int kI8RegThreads = 256;

template <int FMT, int TT, bool DUAL, int D>
__global__ __launch_bounds__(kI8RegThreads) void matvec_i8_reg(I8Args a)
{
    using P = RegPiece<FMT>;
    constexpr int R = DUAL ? 2 : 1;
    extern __shared__ uint4 xsm[];
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int K = static_cast<int>(a.K);
    const int xrow = K + K / 2;
    const int ns = K / 64;             // 64-value slices per row
    const int ni = (ns + 63) / 64;     // items (one slice per lane) per row
    {  // the block's TT quantized rows (rows past T repeat row T - 1)
        const int per = xrow / 16;
        for (int u = threadIdx.x; u < TT * per; u += kI8RegThreads) {
            const int t = u / per;
            int64_t tok = a.t0 + t;
            tok = tok < a.T ? tok : a.T - 1;
            xsm[u] = reinterpret_cast<const uint4*>(a.xq + tok * xrow)[u - t * per];
        }
    }
    __syncthreads();
    const char* xs = reinterpret_cast<const char*>(xsm);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * (kI8RegThreads / 64);
    int64_t n = static_cast<int64_t>(blockIdx.x) * (kI8RegThreads / 64) + wave;
    if (n >= a.N) return;  // wave-uniform; no barrier follows

    float ag[TT], au[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) ag[t] = au[t] = 0.0f;

    // loads of item (row, it) into a register set; rows past N read row N - 1 (their results are dropped)
    auto load = [&](uint4 (&w)[R][P::NW], int64_t row, int it) {
        const int64_t rr = row < a.N ? row : a.N - 1;
        int s = it * 64 + lane;
        s = s < ns ? s : ns - 1;
        P::load(w[0], a.wg + rr * a.wrow, s);
        if constexpr (DUAL) P::load(w[1], a.wu + rr * a.wrow, s);
    };
    auto compute = [&](const uint4 (&w)[R][P::NW], int it) {
        const int s0 = it * 64 + lane;
        const bool own = s0 < ns;
        const int s = own ? s0 : ns - 1;
        I8Unit g0, g1, u0, u1;
        int j0, j1;
        P::units(w[0], s, g0, g1, j0, j1);
        if constexpr (DUAL) P::units(w[1], s, u0, u1, j0, j1);
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const char* xt = xs + t * xrow;
            const uint4 x00 = *reinterpret_cast<const uint4*>(xt + 32 * j0);
            const uint4 x01 = *reinterpret_cast<const uint4*>(xt + 32 * j0 + 16);
            const uint4 x10 = *reinterpret_cast<const uint4*>(xt + 32 * j1);
            const uint4 x11 = *reinterpret_cast<const uint4*>(xt + 32 * j1 + 16);
            const float4 sc0 = *reinterpret_cast<const float4*>(xt + K + 16 * j0);
            const float4 sc1 = *reinterpret_cast<const float4*>(xt + K + 16 * j1);
            const float pg = unit_dot<FMT>(g0, x00, x01, sc0) + unit_dot<FMT>(g1, x10, x11, sc1);
            ag[t] += own ? pg : 0.0f;
            if constexpr (DUAL) {
                const float pu = unit_dot<FMT>(u0, x00, x01, sc0) + unit_dot<FMT>(u1, x10, x11, sc1);
                au[t] += own ? pu : 0.0f;
            }
        }
    };
    auto finish = [&](int64_t row) {
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float out = wave_sum(ag[t]);
            if constexpr (DUAL) {
                const float u = wave_sum(au[t]);
                const float g = out;
                const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(g)
                                  : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(g)
                                                                 : activate<SLHIP_ACT_GELU_ERF>(g);
                out = act * u;
            } else if (a.bias) {
                out = out + a.bias[row];
            }
            const int64_t tok = a.t0 + t;
            if (tok < a.T && lane == 0) {
                if (a.yt == SLHIP_F32)
                    static_cast<float*>(a.y)[tok * a.ys + row] = out;
                else
                    static_cast<uint16_t*>(a.y)[tok * a.ys + row] = static_cast<uint16_t>(f32_to_bf16_bits(out));
            }
            ag[t] = au[t] = 0.0f;
        }
    };

    // D register sets in rotation: set k holds item (rn[k], ri[k]); while one is computed the next D - 1
    // items' loads are in flight. Loads past the last item read the clamped row N - 1 (cache hits), so the
    // wait counts stay exact.
    uint4 S[D][R][P::NW];
    int64_t rn[D];
    int ri[D];
    auto next = [&](int k, int from) {
        rn[k] = rn[from];
        ri[k] = ri[from] + 1;
        if (ri[k] == ni) {
            ri[k] = 0;
            rn[k] += stride;
        }
    };
    rn[0] = n;
    ri[0] = 0;
    load(S[0], rn[0], ri[0]);
#pragma unroll
    for (int k = 1; k < D - 1; k++) {
        next(k, k - 1);
        load(S[k], rn[k], ri[k]);
    }
    bool more = true;
    while (more) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            if (more) {
                const int kl = (k + D - 1) % D, kp = (k + D - 2) % D;
                next(kl, kp);
                load(S[kl], rn[kl], ri[kl]);
                compute(S[k], ri[k]);
                if (ri[k] == ni - 1) finish(rn[k]);
                more = rn[(k + 1) % D] < a.N;
            }
        }
    }
}

