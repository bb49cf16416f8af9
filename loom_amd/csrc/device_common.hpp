// device_common.hpp -- device helpers shared by the gfx950 kernels.
//
// All fp64 expressions follow the reference's operation order; the library is
// compiled with -ffp-contract=off so no multiply-add is fused.
#pragma once

#include <math.h>

#include <utility>

#include "lamd.hpp"

#pragma clang fp contract(off)

namespace lamd {

typedef int v4i __attribute__((ext_vector_type(4)));

// Four K-contiguous int8 codes per dword: the tile layout puts column 4d+j of
// a 16-column word at bit 8j+2d, so dword d is one shift and one AND away.
// Word t of a lane with K group g = lane>>4 holds tile columns 64t+16g .. +15.
__device__ __forceinline__ v4i unpack_codes(uint32_t w) {
    v4i b;
    b[0] = (int)(w & 0x03030303u);
    b[1] = (int)((w >> 2) & 0x03030303u);
    b[2] = (int)((w >> 4) & 0x03030303u);
    b[3] = (int)((w >> 6) & 0x03030303u);
    return b;
}

__device__ __forceinline__ uint32_t word_of(const uint4& q, int t) {
    return t == 0 ? q.x : t == 1 ? q.y : t == 2 ? q.z : q.w;
}

// D(16x16 i32) += A(16x64 i8) * B(64x16 i8).  Lane l supplies A row l&15 and B
// column l&15 for the 16-wide K group l>>4 (the same 16 K indices on both
// sides); D element v of lane l is row 4*(l>>4)+v, column l&15.
__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

typedef int v16i __attribute__((ext_vector_type(16)));

// dword 3 of a raw (untyped, unswizzled) gfx9 buffer resource
constexpr int kBufferWord3 = 0x00020000;

// Raw buffer resource over `bytes` bytes: loads at offsets past the end return
// zero without touching memory, which lets a kernel issue a fixed number of
// loads (so the wait counters see a fixed pattern) without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)bytes, kBufferWord3);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Loads of data each launch reads once (decode weights, the LM head table)
// carry the non-temporal hint (`nt`).  Streaming 570 MB of ternary weights in
// one launch, it raised the sustained rate from 5.4 to 6.1 TB/s on MI355X;
// the sc0 bit alone changed nothing.
constexpr int kLoadNT = 2;  // gfx950 buffer cache-policy bits: sc0 1, nt 2, sc1 16

__device__ __forceinline__ uint4 buffer_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kLoadNT));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte loads and stores with the device-scope coherence bit (sc1): the
// cache policy the compiler gives agent-scope relaxed atomic loads and stores
// on gfx950, here on four words at once.  A store goes through to the level
// that every XCD sees; a load reads from that level, not from a line its own
// XCD's L2 may still hold.
constexpr int kCoherentSC1 = 16;

__device__ __forceinline__ u32x4 buffer_load16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCoherentSC1));
}

__device__ __forceinline__ void buffer_store16_sc1(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, kCoherentSC1);
}

__device__ __forceinline__ uint4 load16_nt(const uint4* p) {
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4*)p));
}

__device__ __forceinline__ float4 load16_nt(const float4* p) {
    return __builtin_bit_cast(float4, __builtin_nontemporal_load((const u32x4*)p));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// f(std::integral_constant<int, 0>{}) ... f(...<N - 1>{}): a loop whose index
// is a compile-time constant in every iteration, for bodies the unroller may
// leave rolled (a rolled loop over accumulator blocks indexes them
// dynamically and moves them to scratch memory).
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// 16-byte non-temporal store of four adjacent floats (p 16-byte aligned)
__device__ __forceinline__ void store16_nt(float* p, float a, float b, float c, float d) {
    const f32x4 v = {a, b, c, d};
    __builtin_nontemporal_store(v, (f32x4*)p);
}

// D(32x32 i32) += A(32x32 i8) * B(32x32 i8), twice the int8 rate of the
// 16x16x64 form on gfx950.  Lane l supplies A row l&31 and B column l&31 for
// K half l>>5 (16 bytes each; byte j of A pairs with byte j of B); D element v
// of lane l is row 8*(v>>2) + 4*(l>>5) + (v&3), column l&31.
__device__ __forceinline__ v16i mfma32_i8(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// bitNetQuantizedActivation (poly/bitnet_cpu.go:73-84) with Go's int(float64)
// on amd64 (CVTTSD2SQ): NaN and out-of-range values become INT64_MIN, which
// loom then clamps to -128.
__device__ __forceinline__ int quant_one(double v, double scale) {
    const double r = round(v * scale);
    if (!(r >= -9223372036854775808.0 && r < 9223372036854775808.0)) return -128;
    if (r < -128.0) return -128;
    if (r > 127.0) return 127;
    return (int)r;
}

// quant_one for an fp32 value v with |v| <= amax (s = fp64 127/amax, s32 =
// fp32(s)), decided in fp32 where that is exact.  |v*s| <= 127, and the fp32
// product p32 = fp32(v * s32) is within 2^-23 * 127 < 1.52e-5 of loom's fp64
// product; so when p32 lies farther than 3.1e-5 from every rounding boundary
// k + 1/2, both round to the same integer, the nearest one to p32 (rintf).
// Near a boundary, and for NaN (every comparison fails), the fp64 path
// decides.  (p32 - rintf(p32) and 0.5 - d are exact: Sterbenz.)
__device__ __forceinline__ int quant_f32(float v, float s32, double s) {
    const float p = v * s32;
    const float r = rintf(p);
    const float d = fabsf(p - r);
    if (0.5f - d > 3.1e-5f) {
        const int q = (int)r;
        return q < -128 ? -128 : (q > 127 ? 127 : q);
    }
    return quant_one((double)v, s);
}

// Low bytes of a, b, c, d as bytes 0..3.  v_perm_b32(S0, S1, sel): byte i of
// the result is byte sel_i of the pair {S0:S1} (0..3 from S1, 4..7 from S0),
// and selector 0x0c gives a zero byte.
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
    return lo | (hi << 16);
}

// Sum of the four signed bytes of w plus acc (v_dot4 against 0x01010101).
__device__ __forceinline__ int byte_sum_i8(uint32_t w, int acc) {
    return __builtin_amdgcn_sdot4((int)w, 0x01010101, acc, false);
}

// loom's "a > maxAbs" update: NaN never replaces the running maximum.
__device__ __forceinline__ float max_nan_skip(float m, float a) { return a > m ? a : m; }


// DPP wave reductions (full-rate VALU lane moves instead of LDS-crossbar
// shuffles).  The pattern is fixed: row_shr 1, 2, 4, 8 inside each 16-lane
// row, then row_bcast 15 and 31 across rows; lane 63 ends with the total,
// which readlane broadcasts.  Lanes without a source add the identity.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v, int identity) {
    return __builtin_amdgcn_update_dpp(identity, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v, double identity) {
    const long long b = __double_as_longlong(v), id = __double_as_longlong(identity);
    const int lo = __builtin_amdgcn_update_dpp((int)id, (int)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp((int)(id >> 32), (int)(b >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
constexpr int kDppShr1 = 0x111, kDppShr2 = 0x112, kDppShr4 = 0x114, kDppShr8 = 0x118;
constexpr int kDppBcast15 = 0x142, kDppBcast31 = 0x143;
constexpr int kDppQuadSwap1 = 0xB1;  // quad_perm 1,0,3,2: the value of lane ^ 1

__device__ __forceinline__ double readlane63_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, 63);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// fixed-order fp64 wave sum, broadcast to every lane
__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
    v = v + dpp_d<kDppShr1>(v, 0.0);
    v = v + dpp_d<kDppShr2>(v, 0.0);
    v = v + dpp_d<kDppShr4>(v, 0.0);
    v = v + dpp_d<kDppShr8>(v, 0.0);
    v = v + dpp_d<kDppBcast15>(v, 0.0);
    v = v + dpp_d<kDppBcast31>(v, 0.0);
    return readlane63_d(v);
}

// maximum over the wave of values compared with `>` (NaN never replaces the
// running maximum; lanes without a source compare against -1e9), broadcast
__device__ __forceinline__ double wave_max_f64_dpp(double v) {
#define LAMD_MAXD_STEP(C)                         \
    {                                             \
        const double o = dpp_d<C>(v, -1e9);       \
        v = o > v ? o : v;                        \
    }
    LAMD_MAXD_STEP(kDppShr1)
    LAMD_MAXD_STEP(kDppShr2)
    LAMD_MAXD_STEP(kDppShr4)
    LAMD_MAXD_STEP(kDppShr8)
    LAMD_MAXD_STEP(kDppBcast15)
    LAMD_MAXD_STEP(kDppBcast31)
#undef LAMD_MAXD_STEP
    return readlane63_d(v);
}

__device__ __forceinline__ int wave_sum_i_dpp(int v) {
    v += dpp_i<kDppShr1>(v, 0);
    v += dpp_i<kDppShr2>(v, 0);
    v += dpp_i<kDppShr4>(v, 0);
    v += dpp_i<kDppShr8>(v, 0);
    v += dpp_i<kDppBcast15>(v, 0);
    v += dpp_i<kDppBcast31>(v, 0);
    return __builtin_amdgcn_readlane(v, 63);
}

// max of non-negative floats (NaN never wins): compared as float values
__device__ __forceinline__ float wave_max_dpp(float v) {
    int b = __float_as_int(v);
#define LAMD_MAX_STEP(C)                                                        \
    {                                                                           \
        const float o = __int_as_float(dpp_i<C>(b, 0));                         \
        b = __float_as_int(max_nan_skip(__int_as_float(b), o));                 \
    }
    LAMD_MAX_STEP(kDppShr1)
    LAMD_MAX_STEP(kDppShr2)
    LAMD_MAX_STEP(kDppShr4)
    LAMD_MAX_STEP(kDppShr8)
    LAMD_MAX_STEP(kDppBcast15)
    LAMD_MAX_STEP(kDppBcast31)
#undef LAMD_MAX_STEP
    return __int_as_float(__builtin_amdgcn_readlane(b, 63));
}

// Wave maximum of non-negative floats (NaN never wins) and wave integer sum,
// broadcast to every lane (order-free: the DPP forms above).
__device__ __forceinline__ float wave_max(float v) { return wave_max_dpp(v); }
__device__ __forceinline__ int wave_sum_i(int v) { return wave_sum_i_dpp(v); }

// unsigned maximum over the wave (lanes shifted in from outside a row read 0)
__device__ __forceinline__ unsigned wave_umax_dpp(unsigned v) {
    int b = (int)v;
    b = (int)max((unsigned)b, (unsigned)dpp_i<kDppShr1>(b, 0));
    b = (int)max((unsigned)b, (unsigned)dpp_i<kDppShr2>(b, 0));
    b = (int)max((unsigned)b, (unsigned)dpp_i<kDppShr4>(b, 0));
    b = (int)max((unsigned)b, (unsigned)dpp_i<kDppShr8>(b, 0));
    b = (int)max((unsigned)b, (unsigned)dpp_i<kDppBcast15>(b, 0));
    b = (int)max((unsigned)b, (unsigned)dpp_i<kDppBcast31>(b, 0));
    return (unsigned)__builtin_amdgcn_readlane(b, 63);
}

// s + p[base] + ... + p[base + 15] in index order, the terms past n replaced
// by -0 (s + -0 = s for every s).
__device__ __forceinline__ double add_block16(const double2 (&v)[8], int base, int n, double s) {
    if (base + 16 <= n) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            s = s + v[j].x;
            s = s + v[j].y;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            s = s + (base + 2 * j < n ? v[j].x : -0.0);
            s = s + (base + 2 * j + 1 < n ? v[j].y : -0.0);
        }
    }
    return s;
}

// s + p[0] + p[1] + ... + p[n-1] in index order (one lane; p in LDS, 16-byte
// aligned, C doubles readable, n <= C), two terms per 16-byte read, with the
// reads of four blocks of sixteen terms in flight ahead of the additions
// (reads past n are never added).
template <int C>
__device__ __forceinline__ double chain_add_pairs(const double* p, int n, double s) {
    static_assert(C % 16 == 0, "blocks of sixteen terms");
    const double2* p2 = (const double2*)p;
    constexpr int NB = C / 16, D = NB < 4 ? NB : 4;
    double2 v[D][8];
#pragma unroll
    for (int b = 0; b < D; ++b)
#pragma unroll
        for (int j = 0; j < 8; ++j) v[b][j] = p2[b * 8 + j];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (b * 16 < n) s = add_block16(v[b % D], b * 16, n, s);
        if (b + D < NB) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[b % D][j] = p2[(b + D) * 8 + j];
        }
    }
    return s;
}

// Inclusive prefix sum over the 64 lanes in fp64 (DPP lane moves): row_shr 1,
// 2, 4, 8 scan each 16-lane row, then row_bcast 15 adds row 0's total to row 1
// and row 2's to row 3 (row mask 0xa), and row_bcast 31 adds the first two
// rows' total to rows 2 and 3 (row mask 0xc).  Exact when every partial sum is
// (integers below 2^53).
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_rows_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, ROWS, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, ROWS, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ double wave_scan_f64_dpp(double v) {
    v = v + dpp_rows_d<kDppShr1, 0xf>(v);
    v = v + dpp_rows_d<kDppShr2, 0xf>(v);
    v = v + dpp_rows_d<kDppShr4, 0xf>(v);
    v = v + dpp_rows_d<kDppShr8, 0xf>(v);
    v = v + dpp_rows_d<kDppBcast15, 0xa>(v);
    v = v + dpp_rows_d<kDppBcast31, 0xc>(v);
    return v;
}

// a wave-uniform 64-bit value (e.g. read from LDS) into scalar registers
__device__ __forceinline__ unsigned long long uniform_u64(unsigned long long v) {
    return ((unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
           (unsigned)__builtin_amdgcn_readfirstlane((int)v);
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// The one-lane chain `for (i = 0; i < n; ++i) s = s + t[i];` (t in LDS),
// bit for bit, run by all 64 lanes of a wavefront (uniform control flow; every
// lane returns the result).
//
// While the running sum s stays in one binade [2^E, 2^(E+1)), every rounded
// sum is a multiple of q = 2^(E-52), and for a term 0 <= t < 2^E the rounded
// s + t is s + q * r with r the integer nearest t/q -- unless t/q is a
// half-integer k + 1/2, where round-half-even picks whichever of s + q*k and
// s + q*(k+1) has an even s/q.  A wave therefore takes 64 x C terms per step:
// lane l rounds its C consecutive terms to integers in units of q (scaling by
// a power of two is exact); a tie depends only on the parity of the running
// sum before it, and a tie leaves that sum even, so each lane's block is
// summed for an incoming parity of 0 and the parity each lane actually sees is
// read off three wave ballots (the last lane below with a tie, and the
// parities of the blocks since).  An inclusive prefix sum of the block sums
// (integers below 2^53: exact in fp64) then gives the running sum after each
// block.  The first block whose running sum leaves the binade, or that holds a
// negative, non-finite or too large term, ends the accepted prefix; its terms
// are added one by one with fp64 additions, and the next step starts after it
// in the binade reached.  A running sum of +0 skips to the first non-zero term
// (+0 + t = t); a running sum that is negative, -0, below 2^-967, above 2^977
// or not finite is advanced one term at a time.  Non-negative finite terms
// (squares, exponentials) take the parallel step.
constexpr int kChainC = 4;  // terms per lane and step of ordered_sum_wave

template <int C>
__device__ __forceinline__ double ordered_sum_wave(const double* t, int n, double s) {
    const int lane = threadIdx.x & 63;
    const unsigned long long lt = (1ull << lane) - 1ull;  // lanes below this one
    int base = 0;
    while (base < n) {
        const unsigned long long sb = (unsigned long long)__double_as_longlong(s);
        const int ex = (int)(sb >> 52);  // sign and biased exponent
        if (sb == 0ull) {
            int first = C;
#pragma unroll
            for (int i = C - 1; i >= 0; --i) {
                const int idx = base + lane * C + i;
                if (idx < n && t[idx] != 0.0) first = i;  // (NaN compares unequal)
            }
            const unsigned long long nz = __builtin_amdgcn_ballot_w64(first < C);
            if (nz == 0ull) {
                base += 64 * C;
                continue;
            }
            const int j = __builtin_ctzll(nz);
            const int idx = base + j * C + __builtin_amdgcn_readlane(first, j);
            s = s + t[idx];
            base = idx + 1;
            continue;
        }
        if (ex < 56 || ex > 2000) {
            const int end = min(n, base + 64 * C);
            for (; base < end; ++base) s = s + t[base];
            continue;
        }
        const double scale = __longlong_as_double((long long)(2098 - ex) << 52);  // 1/q
        const double q = __longlong_as_double((long long)(ex - 52) << 52);
        const double su = s * scale;   // s/q: an integer in [2^52, 2^53)
        const double room = 0x1p53 - su;
        double d0 = 0.0, sgn = 0.0;
        int par = 0;  // parity of the running sum: relative until the block's first tie
        bool tied = false, bad = false;
#pragma unroll
        for (int i = 0; i < C; ++i) {
            const int idx = base + lane * C + i;
            const double u = (idx < n ? t[idx] : 0.0) * scale;
            bad |= !(u >= 0.0 && u < 0x1p52);
            const double fl = floor(u);
            const bool tie = u - fl == 0.5;
            const double rn = rint(u);
            const int pf = (int)__double_as_longlong(fl + 0x1p52) & 1;
            const int pr = (int)__double_as_longlong(rn + 0x1p52) & 1;
            const int up = par ^ pf;  // the tie's round-up that leaves the sum even
            if (tie && !tied) sgn = up ? -1.0 : 1.0;  // change for an odd incoming parity
            d0 += tie ? fl + (double)up : rn;
            par = tie ? 0 : (par ^ pr);
            tied |= tie;
        }
        const unsigned long long ht = __builtin_amdgcn_ballot_w64(tied);
        const unsigned long long po = __builtin_amdgcn_ballot_w64(tied && par);
        const unsigned long long fp = __builtin_amdgcn_ballot_w64(!tied && par);
        const unsigned long long below = ht & lt;
        const int b = below ? 63 - __builtin_clzll(below) : -1;
        const unsigned long long since = b >= 0 ? lt & ~((2ull << b) - 1ull) : lt;
        const int p0 = b >= 0 ? (int)(po >> b) & 1 : (int)(sb & 1ull);
        const int pin = p0 ^ (__builtin_popcountll(fp & since) & 1);
        const double psum = wave_scan_f64_dpp(tied && pin ? d0 + sgn : d0);
        const unsigned long long stop = __builtin_amdgcn_ballot_w64(bad || !(psum < room));
        if (stop == 0ull) {
            s = (su + readlane63_d(psum)) * q;
            base += 64 * C;
        } else {
            const int j = __builtin_ctzll(stop);
            s = (su + (j > 0 ? readlane_d(psum, j - 1) : 0.0)) * q;
            const int b0 = base + j * C;
#pragma unroll
            for (int i = 0; i < C; ++i)
                if (b0 + i < n) s = s + t[b0 + i];
            base = b0 + C;
        }
    }
    return s;
}

// Inclusive prefix sum over the lanes of one segment: lane l adds only the
// partial sums of lanes at or above ss (its segment's first lane), so each
// segment is summed on its own (the DPP steps of wave_scan_f64_dpp).
__device__ __forceinline__ double wave_seg_scan_f64(double v, int ss, int lane) {
#define LAMD_SEG_STEP(CTRL, K)                                                    \
    {                                                                             \
        const double o = dpp_rows_d<CTRL, 0xf>(v);                                \
        v = v + (((lane & 15) >= (K) && lane - (K) >= ss) ? o : 0.0);             \
    }
    LAMD_SEG_STEP(kDppShr1, 1)
    LAMD_SEG_STEP(kDppShr2, 2)
    LAMD_SEG_STEP(kDppShr4, 4)
    LAMD_SEG_STEP(kDppShr8, 8)
#undef LAMD_SEG_STEP
    {
        const double o = dpp_rows_d<kDppBcast15, 0xa>(v);  // rows 1 and 3 take lane 15 / 47
        v = v + ((((lane >> 4) & 1) && (lane & ~15) - 1 >= ss) ? o : 0.0);
    }
    {
        const double o = dpp_rows_d<kDppBcast31, 0xc>(v);  // rows 2 and 3 take lane 31
        v = v + ((lane >= 32 && 31 >= ss) ? o : 0.0);
    }
    return v;
}

// LDS of ordered_sum_block for W waves (records at the lane that ends a
// segment).
template <int W>
struct OrderedSumLds {
    double wtot[W];               // plain sum of each wave's terms
    unsigned long long items[W];  // lanes with a record: segment ends and sequential lanes
    unsigned long long seql[W];   // the sequential lanes
    double seg[W * 64];           // a segment's sum (incoming parity even), at its last lane
    double flip[W * 64];          // its change for an odd incoming parity
    int meta[W * 64];             // binade | first lane << 16
    double result;
};

// Terms per lane of ordered_sum_block for n terms over 64W threads: the
// smallest of 1, 3, 5, 11, 15, 17, 27, 33, 63 that covers n (odd, so the lanes'
// blocks start in different LDS banks).  The term array must hold
// 64 * W * ordered_sum_lane_terms(n, W) doubles; ordered_sum_block writes -0
// past the n terms.
__host__ __device__ constexpr int ordered_sum_lane_terms(int n, int w) {
    const int need = (n + 64 * w - 1) / (64 * w);
    return need <= 1 ? 1 : need <= 3 ? 3 : need <= 5 ? 5 : need <= 11 ? 11 : need <= 15 ? 15
         : need <= 17 ? 17 : need <= 27 ? 27 : need <= 33 ? 33 : 63;
}
__host__ __device__ constexpr int ordered_sum_slots(int n, int w) {
    return 64 * w * ordered_sum_lane_terms(n, w);
}

template <int W, int G>
__device__ __forceinline__ double ordered_sum_block_g(double* t, int n, double s0,
                                                     OrderedSumLds<W>& sh) {
    constexpr int U = G < 8 ? G : (G <= 17 ? 8 : 4);  // reads in flight per lane
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const bool active = wave < W;    // waves past W only meet the barriers
    const double* tb = t + tid * G;  // this lane's block (active waves)

    // estimated running sums before and after each lane; an Inf or NaN term
    // shows in the largest exponent field, a negative one in the smallest term
    // (-0 padding is neither)
    double a = 0.0, mn = 0.0, exc = 0.0;
    unsigned hw = 0;
    if (active) {
#pragma unroll(G <= 17 ? 8 : 1)
    for (int i0 = 0; i0 < G; i0 += U) {
        double v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) v[j] = i0 + j < G ? tb[i0 + j] : 0.0;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            if (i0 + j < G) {
                a = a + v[j];
                mn = fmin(mn, v[j]);
                hw = max(hw, (unsigned)((unsigned long long)__double_as_longlong(v[j]) >> 32) & 0x7fffffffu);
            }
        }
    }
    const double inc = wave_scan_f64_dpp(a);
    exc = __shfl_up(inc, 1, 64);
    if (lane == 0) exc = 0.0;
    if (lane == 63) sh.wtot[wave] = inc;
    }
    __syncthreads();
    if (active) {
    double off = s0;
#pragma unroll
    for (int v = 0; v < W - 1; ++v) off = v < wave ? off + sh.wtot[v] : off;
    const double lo = (off + exc) * (1.0 - 0x1p-30);
    const double hi = ((off + exc) + a) * (1.0 + 0x1p-30);
    int e = (int)((unsigned long long)__double_as_longlong(lo) >> 52);  // biased exponent
    const bool sq = !(lo >= 0x1p-960 && hi < 0x1p1000 &&
                      e == (int)((unsigned long long)__double_as_longlong(hi) >> 52) &&
                      hw < 0x7ff00000u && mn >= 0.0);  // non-negative finite terms, one binade
    if (sq) e = 1023;
    const double scale = __longlong_as_double((long long)(2098 - e) << 52);  // 1/q

    // this lane's terms in units of q, for an even incoming parity.  u + 2^52
    // rounds u (0 <= u < 2^52 in a lane that keeps its binade) to the nearest
    // integer, half even; at a half-integer an odd running sum takes the other
    // neighbour u + (u - rn) instead.  The first tie changes the lane's sum by
    // +-1 when the incoming parity is odd (flip).
    double d0 = 0.0;
    unsigned par = 0, tied = 0, flip = 0;
#pragma unroll(G <= 17 ? 8 : 1)
    for (int i0 = 0; i0 < G; i0 += U) {
        double v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) v[j] = i0 + j < G ? tb[i0 + j] : 0.0;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            if (i0 + j < G) {
                const double u = v[j] * scale;
                const double w = u + 0x1p52;
                const double rn = w - 0x1p52;
                const double df = u - rn;  // exact
                const unsigned odd = (unsigned)__double_as_longlong(w) & 1u;
                const unsigned tie = fabs(df) == 0.5 ? 1u : 0u;
                d0 = d0 + ((tie & par) ? u + df : rn);
                const unsigned up = df > 0.0 ? 1u : 0u;
                flip = (tie & ~tied) ? (up ^ par ^ 1u) : flip;  // 1: -1, 0: +1
                tied |= tie;
                par = tie ? 0u : (par ^ odd);
            }
        }
    }
    const double sgn = flip ? -1.0 : 1.0;

    // segments and each lane's incoming parity
    const unsigned long long lt = (1ull << lane) - 1ull, le = lt | (1ull << lane);
    const unsigned long long SQ = __builtin_amdgcn_ballot_w64(sq);
    const int eprev = __shfl_up(e, 1, 64);
    const bool start = !sq && (lane == 0 || ((SQ >> ((lane - 1) & 63)) & 1ull) || eprev != e);
    const unsigned long long SS = __builtin_amdgcn_ballot_w64(start);
    const unsigned long long ht = __builtin_amdgcn_ballot_w64(!sq && tied);
    const unsigned long long po = __builtin_amdgcn_ballot_w64(!sq && tied && par);
    const unsigned long long fp = __builtin_amdgcn_ballot_w64(!sq && !tied && par);
    const int ss = sq ? lane + 1 : 63 - __builtin_clzll((SS & le) | 1ull);
    const int ssc = sq ? lane : ss;
    const unsigned long long inseg = lt & ~((1ull << ssc) - 1ull);  // segment lanes below
    const unsigned long long below = ht & inseg;
    const int b = below ? 63 - __builtin_clzll(below) : -1;       // last tie below
    const unsigned long long since = b >= 0 ? (lt & ~((2ull << b) - 1ull)) : inseg;
    const int p0 = b >= 0 ? (int)((po >> b) & 1ull) : 0;
    const int pin = p0 ^ (__builtin_popcountll(fp & since) & 1);
    const double d = sq ? 0.0 : ((tied && pin) ? d0 + sgn : d0);
    const double dl = (!sq && tied && b < 0) ? (pin ? -sgn : sgn) : 0.0;
    const double psum = wave_seg_scan_f64(d, ss, lane);
    const bool end = !sq && (lane == 63 || (((SS | SQ) >> ((lane + 1) & 63)) & 1ull));
    const unsigned long long SE = __builtin_amdgcn_ballot_w64(end);
    const unsigned long long ft = ht & ~((1ull << ssc) - 1ull) & le;  // ties from the segment start
    const double fl = __shfl(dl, ft ? __builtin_ctzll(ft) : lane, 64);
    if (end) {
        sh.seg[tid] = psum;
        sh.flip[tid] = ft ? fl : 0.0;
        sh.meta[tid] = e | (ss << 16);
    }
    if (lane == 0) {
        sh.items[wave] = SE | SQ;
        sh.seql[wave] = SQ;
    }
    }
    __syncthreads();

    // wave 0 walks the records in order (a failed check ends the walk and
    // the remaining terms go through ordered_sum_wave); the next wave's records
    // are read while the current wave's are walked
    if (wave == 0) {
        double s = s0;
        int rest = -1;
        double segv = sh.seg[lane], flipv = sh.flip[lane];
        int metav = sh.meta[lane];
        unsigned long long itv = sh.items[0], sqv = sh.seql[0];
        for (int w = 0; w < W && rest < 0; ++w) {
            unsigned long long items = uniform_u64(itv);
            const unsigned long long seqm = uniform_u64(sqv);
            const double cseg = segv, cflip = flipv;
            const int cmeta = metav;
            if (w + 1 < W) {
                segv = sh.seg[(w + 1) * 64 + lane];
                flipv = sh.flip[(w + 1) * 64 + lane];
                metav = sh.meta[(w + 1) * 64 + lane];
                itv = sh.items[w + 1];
                sqv = sh.seql[w + 1];
            }
            while (items) {
                const int l = __builtin_ctzll(items);
                items &= items - 1ull;
                const int b0 = (w * 64 + l) * G;
                if ((seqm >> l) & 1ull) {
                    // a sequential lane: its G terms, read U ahead of the additions
                    // (the padding past n is -0, and s + -0 = s for every s)
                    const double* sb = t + b0;
#pragma unroll(G <= 17 ? 8 : 1)
                    for (int i0 = 0; i0 < G; i0 += U) {
                        double v[U];
#pragma unroll
                        for (int j = 0; j < U; ++j) v[j] = i0 + j < G ? sb[i0 + j] : 0.0;
#pragma unroll
                        for (int j = 0; j < U; ++j)
                            if (i0 + j < G) s = s + v[j];
                    }
                    continue;
                }
                const int meta = __builtin_amdgcn_readlane(cmeta, l);
                const int E = meta & 0x7ff;
                const double sc = __longlong_as_double((long long)(2098 - E) << 52);
                const double q = __longlong_as_double((long long)(E - 52) << 52);
                const double seg = readlane_d(cseg, l), fv = readlane_d(cflip, l);
                const double su = s * sc;
                const double D = seg + ((__double_as_longlong(su) & 1ll) ? fv : 0.0);
                const bool ok = (int)((unsigned long long)__double_as_longlong(s) >> 52) == E && D < 0x1p53 - su;
                if (__builtin_expect(!ok, 0)) {
                    rest = (w * 64 + (meta >> 16)) * G;
                    break;
                }
                s = (su + D) * q;
            }
        }
        if (rest >= 0) s = ordered_sum_wave<kChainC>(t + rest, n - rest, s);
        if (lane == 0) sh.result = s;
    }
    __syncthreads();
    return sh.result;
}

// The one-lane chain `for (i = 0; i < n; ++i) s = s + t[i];` (t in LDS), bit
// for bit, formed by the first W waves of the workgroup (every thread of the
// workgroup calls it -- waves past W only meet its four barriers -- and every
// thread gets the result).  t must
// hold ordered_sum_slots(n, W) doubles: the slots past n are set to -0, which
// leaves every sum unchanged.
//
// Thread g takes the G = ordered_sum_lane_terms(n, W) consecutive terms
// [gG, gG + G).  A plain fp64 prefix sum of the lanes' totals estimates the
// running sum before and after each lane (within a relative 1e-12 for
// non-negative terms), which places each lane in the binade [2^E, 2^(E+1))
// its running sum keeps throughout -- with a margin of 2^-30 either side --
// or marks it sequential (a crossing of a power of two, a zero or tiny start,
// a huge end, a negative or non-finite term).  In a binade every rounded sum
// is a multiple of q = 2^(E-52) and s + t rounds to s + q * r with r = t/q
// rounded to the nearest integer, except at a half-integer t/q, whose
// round-half-even result is the candidate that leaves s/q even (see
// ordered_sum_wave).  So a lane sums its r in units of q exactly, taking its
// segment's incoming parity as even; a run of lanes with one binade forms a
// segment whose sum is a segmented prefix sum over the lanes (exact: integers
// below 2^53), where each lane's parity comes from wave ballots, and whose sum
// for an odd incoming parity differs only at its first tie.  Wave 0 then walks
// the records in order: a segment checks that the exact running sum lies in
// its binade with room for the segment's sum and adds it (its parity picks the
// variant); a sequential lane adds its terms with fp64 additions.  A failed
// check (a running sum the estimate misplaced: possible only with negative
// terms) hands the rest of the row, from that segment's first term, to
// ordered_sum_wave.
template <int W>
__device__ __forceinline__ double ordered_sum_block(double* t, int n, double s0,
                                                   OrderedSumLds<W>& sh) {
    static_assert(W >= 2 && W <= 8, "the sum runs on 2 to 8 waves");
    if (n <= 0) return s0;
    const int G = ordered_sum_lane_terms(n, W);
    for (int i = n + (int)threadIdx.x; i < 64 * W * G; i += (int)blockDim.x) t[i] = -0.0;
    __syncthreads();
    switch (G) {
        case 1: return ordered_sum_block_g<W, 1>(t, n, s0, sh);
        case 3: return ordered_sum_block_g<W, 3>(t, n, s0, sh);
        case 5: return ordered_sum_block_g<W, 5>(t, n, s0, sh);
        case 11: return ordered_sum_block_g<W, 11>(t, n, s0, sh);
        case 15: return ordered_sum_block_g<W, 15>(t, n, s0, sh);
        case 17: return ordered_sum_block_g<W, 17>(t, n, s0, sh);
        default: break;
    }
    if constexpr (W <= 4) {  // more than 17 terms per lane (n <= 8064) only below 8 waves
        switch (G) {
            case 27: return ordered_sum_block_g<W, 27>(t, n, s0, sh);
            case 33: return ordered_sum_block_g<W, 33>(t, n, s0, sh);
            default: break;
        }
    }
    if constexpr (W <= 2) return ordered_sum_block_g<W, 63>(t, n, s0, sh);
    return ordered_sum_wave<kChainC>(t, n, s0);  // (not reached for n <= 8064)
}

// Block reductions over blockDim.x threads (a multiple of 64, at most 1024).
__device__ inline float block_max(float v, float* sh) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < nw; ++i) r = max_nan_skip(r, sh[i]);
    __syncthreads();
    return r;
}

__device__ inline int block_sum_i(int v, int* sh) {
    v = wave_sum_i(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    int r = 0;
    for (int i = 0; i < nw; ++i) r += sh[i];
    __syncthreads();
    return r;
}

// loom Activate for float32 (poly/poly.go:167-200).
__device__ inline float activate_f32(float v, int act) {
    switch (act) {
        case 0:
            return v < 0.0f ? 0.0f : v;
        case 1:
            return v * (float)(1.0 / (1.0 + exp(-(double)v)));
        case 2: {
            const double v64 = (double)v;
            return (float)(0.5 * v64 *
                           (1.0 + tanh(sqrt(2.0 / M_PI) * (v64 + 0.044715 * pow(v64, 3.0)))));
        }
        case 3:
            return (float)tanh((double)v);
        case 4:
            return (float)(1.0 / (1.0 + exp(-(double)v)));
        case 5:
            return v < 0.0f ? (float)((double)v * 0.01) : v;
        case 6:
            return v < 0.0f ? 0.0f : v * v;
        default:
            return v;
    }
}

// swigluGateProduct (poly/swiglu.go:37-46).
__device__ __forceinline__ double gate_product(double g, double u, int act) {
    if (act == 6) {
        if (g < 0.0) g = 0.0;
        return (g * g) * u;
    }
    const double sig = 1.0 / (1.0 + exp(-g));
    return (g * sig) * u;
}

// bitNetTernaryMatVecQuantized output scale (poly/bitnet_cpu.go:540-543).
__device__ __forceinline__ double output_scale(float wscale, float amax) {
    const double s = (double)wscale * (double)amax / 127.0;
    return s == 0.0 ? 1.0 : s;
}

// Epilogue parameters shared by every matmul kernel.
struct EpiDev {
    int kind;
    int activation;
    int m, n;
    float scale0, scale1;
    const float* amax;
    const int32_t* xsum;
    const float* bias0;
    const float* bias1;
    const float* residual;
    float* out;
    float* post;
    int ldo;
    int32_t* acc0;
    int32_t* acc1;
};

// Per-token-row constants of the epilogue: loom's output scales of matrix
// 0/1 for the row's amax, and the row's sum(xq).
struct RowScale {
    double os0, os1;
    int xs;
};

__device__ __forceinline__ RowScale row_scale(const EpiDev& e, float am, int xs) {
    RowScale rs;
    rs.os0 = output_scale(e.scale0, am);
    rs.os1 = e.kind == EPI_SWIGLU ? output_scale(e.scale1, am) : 0.0;
    rs.xs = xs;
    return rs;
}

// raw0/raw1: sum(code * xq) of matrix 0/1 for token row i, output n.  Codes
// are weight+1, so acc = raw - sum(xq).  b0/b1 are bias0[n]/bias1[n] and res
// is residual[i*ldo+n], loaded by the caller (read only when those pointers
// are set); callers that batch their loads ahead of their stores use this.
// KIND >= 0 fixes e.kind at compile time (callers that dispatch on it).
template <int KIND = -1>
__device__ __forceinline__ void epilogue_store_pre(const EpiDev& e, int i, int n, int raw0, int raw1,
                                                   double os0, double os1, int xs, float b0, float b1,
                                                   float res) {
    const int kind = KIND >= 0 ? KIND : e.kind;
    const int acc0 = raw0 - xs;
    const size_t o = (size_t)i * e.ldo + n;
    if (e.acc0) e.acc0[(size_t)i * e.n + n] = acc0;
    if (kind == EPI_ACC) return;
    if (kind == EPI_SWIGLU) {
        const int acc1 = raw1 - xs;
        if (e.acc1) e.acc1[(size_t)i * e.n + n] = acc1;
        // g := gate[o] + bias; u := up[o] + bias   (poly/swiglu.go:306-309)
        const double g = (double)acc0 * os0 + (e.bias0 ? (double)b0 : 0.0);
        const double u = (double)acc1 * os1 + (e.bias1 ? (double)b1 : 0.0);
        e.out[o] = (float)gate_product(g, u, e.activation);
        return;
    }
    double d = (double)acc0 * os0;
    if (e.bias0) d = d + (double)b0;
    float v = (float)d;
    if (e.residual) v = v + res;
    e.out[o] = v;
    if (e.post) e.post[o] = activate_f32(v, e.activation);
}

// The epilogue's per-output inputs that come from memory: bias0[n],
// bias1[n] and residual[i*ldo+n] (zero where the pointer is null or the kind
// does not read them).  Kernels load them for all of a round's outputs
// before the round's first store: the vector memory counter is in order, so a
// load issued after a store also waits for that store to complete.
struct EpiIn {
    float b0, b1, res;
};

__device__ __forceinline__ EpiIn epilogue_inputs(const EpiDev& e, int i, int n) {
    EpiIn v;
    v.b0 = e.bias0 ? e.bias0[n] : 0.0f;
    v.b1 = e.kind == EPI_SWIGLU && e.bias1 ? e.bias1[n] : 0.0f;
    v.res = e.kind == EPI_DENSE && e.residual ? e.residual[(size_t)i * e.ldo + n] : 0.0f;
    return v;
}

__device__ __forceinline__ void epilogue_store(const EpiDev& e, int i, int n, int raw0, int raw1,
                                               const RowScale& rs) {
    const EpiIn v = epilogue_inputs(e, i, n);
    epilogue_store_pre(e, i, n, raw0, raw1, rs.os0, rs.os1, rs.xs, v.b0, v.b1, v.res);
}

// Outputs per thread per epilogue round of the small-M kernels.
constexpr int kEpiBatch = 4;

// Arguments of the matmul kernels.
// Workspace of the small-M split kernel (matmul_skinny.hip): int32 output
// accumulators of the row groups and one arrival counter per group, both
// zero between launches (the last workgroup of a group clears them).
constexpr int kSmallSplitInts = 1 << 21;  // 8 MiB
constexpr int kSmallSplitGroups = 2048;
struct SmallSplitWs {
    int32_t* acc = nullptr;
    unsigned* ctr = nullptr;
};
SmallSplitWs small_split_ws(int device);

struct MatArgs {
    const uint4* w0;
    const uint4* w1;
    int ktiles;
    int ntiles;
    const int8_t* xq;  // quantized rows (unfused paths)
    int ldq;
    const float* x;    // fp32 rows (fused-quantization path), ldx = K
    int k;
    int8_t* xq_tap;    // fused path: quantized rows written by workgroup 0 (optional)
    float* amax_tap;
    // norm-fused path: the rows are normalized before the quantization
    const double* x64;  // fp64 rows (NORM_INNER_F64), ldx = K
    const float* nw;    // gain / inner-norm weight (length K), null = ones
    double neps;        // eps of the norm
    void* norm_tap;     // normalized rows (M x K; fp32, fp64 for NORM_INNER_F64), workgroup 0 (optional)
    EpiDev e;
};

}  // namespace lamd
