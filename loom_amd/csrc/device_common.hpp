// device_common.hpp -- device helpers shared by the gfx950 kernels.
//
// All fp64 expressions follow the reference's operation order; the library is
// compiled with -ffp-contract=off so no multiply-add is fused.
#pragma once

#include <math.h>

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

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// loom's "a > maxAbs" update: NaN never replaces the running maximum.
__device__ __forceinline__ float max_nan_skip(float m, float a) { return a > m ? a : m; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max_nan_skip(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

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

// Sum of n fp64 terms in index order (one lane): terms are read from LDS
// sixteen at a time ahead of the dependent additions (each addition waits
// only for its own read: LDS reads return in order).
__device__ __forceinline__ double ordered_sum(const double* t, int n, double s) {
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        double v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = t[i + j];
#pragma unroll
        for (int j = 0; j < 16; ++j) s += v[j];
    }
    for (; i < n; ++i) s += t[i];
    return s;
}

// sum over k in index order of p[k] * (double)v[k * vs] (LDS operands; a
// product, then a sum, each rounded).  Blocks of 16 terms, double-buffered:
// the reads of block b + 1 are issued before the additions of block b (the
// block read after the last full one is clamped to an existing block rather
// than guarded by a branch).
__device__ __forceinline__ double ordered_dot(const double* p, const float* v, int vs, int n, double s) {
    constexpr int B = 16;
    const int nb = n / B;
    if (nb > 0) {
        double a[B], c[B];
        float b[B], d[B];
#pragma unroll
        for (int j = 0; j < B; ++j) {
            a[j] = p[j];
            b[j] = v[j * vs];
        }
        int blk = 0;
        for (; blk + 2 <= nb; blk += 2) {
            const int o1 = (blk + 1) * B, o2 = min(blk + 2, nb - 1) * B;
#pragma unroll
            for (int j = 0; j < B; ++j) {
                c[j] = p[o1 + j];
                d[j] = v[(o1 + j) * vs];
            }
#pragma unroll
            for (int j = 0; j < B; ++j) s += a[j] * (double)b[j];
#pragma unroll
            for (int j = 0; j < B; ++j) {
                a[j] = p[o2 + j];
                b[j] = v[(o2 + j) * vs];
            }
#pragma unroll
            for (int j = 0; j < B; ++j) s += c[j] * (double)d[j];
        }
        if (blk < nb) {
#pragma unroll
            for (int j = 0; j < B; ++j) s += a[j] * (double)b[j];
        }
    }
    for (int i = nb * B; i < n; ++i) s += p[i] * (double)v[i * vs];
    return s;
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

__device__ __forceinline__ void epilogue_store(const EpiDev& e, int i, int n, int raw0, int raw1,
                                               const RowScale& rs) {
    const float b0 = e.bias0 ? e.bias0[n] : 0.0f;
    const float b1 = e.kind == EPI_SWIGLU && e.bias1 ? e.bias1[n] : 0.0f;
    const float res = e.kind == EPI_DENSE && e.residual ? e.residual[(size_t)i * e.ldo + n] : 0.0f;
    epilogue_store_pre(e, i, n, raw0, raw1, rs.os0, rs.os1, rs.xs, b0, b1, res);
}

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
