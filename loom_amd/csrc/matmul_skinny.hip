// matmul_skinny.hip -- ternary matmul for few token rows (decode, M <= 64) and
// the matmul dispatcher.
//
// One workgroup per 16-row weight tile; its WAVES waves split the K tiles and
// merge partial sums with LDS integer adds (order-free, so exact).  Each wave
// issues the 128-bit loads of all its weight tiles first.
//
// FUSEQ (M <= 4, K % 4 == 0): the workgroup quantizes the fp32 rows itself
// while its weight loads are in flight -- row absmax over the whole row, then
// loom's int8 rounding into an LDS copy of the quantized rows -- so a Dense
// forward is one launch.  Every workgroup derives the same amax, xq and sum(xq)
// from the same fp32 row, so all outputs agree with a separate quantization.
#include "device_common.hpp"

namespace lamd {

hipError_t launch_gemm(const MatArgs& p, bool two, int device, hipStream_t s);
bool stream_ok(int m, int k, int n_tiles, bool fused, const Epilogue& epi);
hipError_t launch_stream(const MatArgs& p, bool fuseq, hipStream_t s);

constexpr int kFusedMaxRows = 4;
// 4 < M <= kFusedWaveRows fp32 rows fuse their quantization too, one row per
// wave (MR = kFusedWaveRows selects that prologue).
constexpr int kFusedWaveRows = 8;
// strict norm rows this long form their sum on eight waves (fewer terms per lane)
constexpr int kSumWideCols = 4096;
constexpr int kFusedVec = 16;  // float4 per thread in the fused prologue (max)

// Row of element group idx (4 elements) among M <= MR rows of row4 groups.
template <int MR>
__device__ __forceinline__ int row_of(int idx, int row4) {
    if (MR == 1) return 0;
    return (idx >= row4) + (idx >= 2 * row4) + (idx >= 3 * row4);
}

// NORM: RowNorm applied before the quantization (FUSEQ only).  STRICT sums
// the squares of the (single) row in element order on one lane, from LDS.
// FV: element groups (4 values) per thread.  NTR: adjacent 16-row weight
// tiles per workgroup (the fused prologue's row loads and quantization are
// then shared by NTR tiles; tiles past the last read the last tile and store
// nothing).
template <int NMAT, int MSUB, int WAVES, bool FUSEQ, int NORM = NORM_NONE, int STRICT = 0,
          int FV = kFusedVec, int MR = kFusedMaxRows, int NTR = 1>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2))) void skinny_kernel(MatArgs p) {
    constexpr int T = WAVES * 64;
    constexpr int U = 4 / MSUB;  // K tiles per batch per wave
    extern __shared__ __align__(16) int8_t xq_s[];  // FUSEQ: M rows x ldq (STRICT: k squares first)
    __shared__ int red[NTR][NMAT][MSUB * 16][16];
    constexpr bool RPW = FUSEQ && MR > kFusedMaxRows;  // one row per wave
    static_assert(!RPW || (NORM == NORM_NONE && MR <= WAVES && MSUB == 1), "row-per-wave prologue");
    __shared__ unsigned amax_bits[MR > kFusedMaxRows ? MR : kFusedMaxRows];
    __shared__ int xsum_s[MR > kFusedMaxRows ? MR : kFusedMaxRows];
    __shared__ double nsum[NORM != NORM_NONE ? WAVES : 1][kFusedMaxRows];
    __shared__ float wmax[FUSEQ ? WAVES : 1][kFusedMaxRows];
    __shared__ unsigned wmaxb[FUSEQ ? WAVES : 1][kFusedMaxRows];
    __shared__ int wsum[FUSEQ ? WAVES : 1][kFusedMaxRows];
    const int nt = blockIdx.x * NTR;  // first weight tile of the workgroup
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int M = p.e.m;
    const int ktiles = p.ktiles;
    size_t tile0[NTR];
#pragma unroll
    for (int q = 0; q < NTR; ++q) tile0[q] = (size_t)min(nt + q, p.ntiles - 1) * ktiles * 64 + lane;

    // FUSEQ: the rows (and norm weights) are loaded first, so waiting for them
    // does not also wait for the weight loads queued behind them.
    const int k = p.k;
    const int row4 = k >> 2;            // element groups per row (k % 4 == 0)
    const int n4 = FUSEQ ? M * row4 : 0;
    constexpr bool F64 = NORM == NORM_INNER_F64;
    float4 xv[FUSEQ && !F64 ? FV : 1];
    double xd[F64 ? FV : 1][4];
    float4 gv[NORM != NORM_NONE ? FV : 1];
    // Every slot issues its load; slots past the data read past the end of a
    // buffer resource (zero, no memory traffic).  With no branches around the
    // loads the wait for the rows counts only the weight loads issued after
    // them, which stay in flight through the prologue.
    if (FUSEQ) {
        const uint32_t xb = (uint32_t)n4 * (F64 ? 32u : 16u);
        const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(F64 ? (const void*)p.x64 : (const void*)p.x, xb);
        const __amdgpu_buffer_rsrc_t gr = buffer_rsrc(p.nw, p.nw ? (uint32_t)row4 * 16u : 0u);
        // Plain rows on eight or more waves skip the slots that lie wholly
        // past the rows for the wave (a wave-uniform test; measured at the
        // BitNet-2B down shape, M = 1: 4.95 -> 4.17 us per Dense step; with
        // four waves, or with a norm fused, issuing every slot measured
        // faster).
        constexpr bool kSkipIdle = !RPW && NORM == NORM_NONE && WAVES >= 8;
#pragma unroll
        for (int j = 0; j < FV; ++j) {
            // (one row per wave: lane l takes element groups l + 64 j of row `wave`)
            const int idx = RPW ? wave * row4 + lane + 64 * j : tid + j * T;
            const bool ok = RPW ? wave < M && lane + 64 * j < row4 : idx < n4;
            if (kSkipIdle && j > 0 && __builtin_amdgcn_readfirstlane(wave) * 64 + j * T >= n4) {
                xv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                continue;
            }
            if (F64) {
                const uint32_t o = ok ? (uint32_t)idx * 32u : xb;
                const double2 a = __builtin_bit_cast(double2, buffer_load16(xr, o));
                const double2 b = __builtin_bit_cast(double2, buffer_load16(xr, ok ? o + 16u : xb));
                xd[j][0] = a.x;
                xd[j][1] = a.y;
                xd[j][2] = b.x;
                xd[j][3] = b.y;
            } else {
                xv[j] = __builtin_bit_cast(float4, buffer_load16(xr, ok ? (uint32_t)idx * 16u : xb));
            }
            if (NORM != NORM_NONE) {
                const int c4 = idx - row_of<MR>(idx, row4) * row4;
                gv[j] = p.nw ? __builtin_bit_cast(float4, buffer_load16(gr, ok ? (uint32_t)c4 * 16u : (uint32_t)row4 * 16u))
                             : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            }
        }
    }

    // weights of the first batch
    const uint32_t wbytes = (uint32_t)p.ntiles * (uint32_t)ktiles * 1024u;
    const __amdgpu_buffer_rsrc_t wr0 = buffer_rsrc(p.w0, wbytes);
    const __amdgpu_buffer_rsrc_t wr1 = buffer_rsrc(p.w1, wbytes);
    uint4 wv[NTR][NMAT][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int kt = wave + u * WAVES;
#pragma unroll
        for (int q = 0; q < NTR; ++q) {
            if (FUSEQ) {  // (without a prologue to overlap, skipping the unused loads is cheaper)
                const uint32_t o = kt < ktiles ? (uint32_t)(tile0[q] + (size_t)kt * 64) * 16u : wbytes;
                wv[q][0][u] = buffer_load16_nt(wr0, o);
                if (NMAT == 2) wv[q][NMAT - 1][u] = buffer_load16_nt(wr1, o);
            } else if (kt < ktiles) {
                wv[q][0][u] = load16_nt(p.w0 + tile0[q] + (size_t)kt * 64);
                if (NMAT == 2) wv[q][NMAT - 1][u] = load16_nt(p.w1 + tile0[q] + (size_t)kt * 64);
            }
        }
    }

    // The epilogue inputs of the first output this thread finishes (bias and
    // residual, and for pre-quantized rows the row's amax and sum(xq)) are
    // loaded now, so the epilogue does not start with a memory round trip
    // after the reduction (clamped indices: no branch per lane).  The
    // fused-quantization kernels load them in the epilogue instead: an early
    // residual load measured slower in the norm-fused decode GEMVs (decode
    // 694 -> 678 tokens/s).
    constexpr bool kEarlyIn = !FUSEQ;
    const int tc0 = min((tid % (M * 16)) >> 4, M - 1);
    const int nc0 = min((nt + min(tid / (M * 16), NTR - 1)) * kTileRows + (tid & 15), p.e.n - 1);
    EpiIn in_first{0.0f, 0.0f, 0.0f};
    if (kEarlyIn) in_first = epilogue_inputs(p.e, tc0, nc0);
    float am_first = 0.0f;
    int xs_first = 0;
    if (!FUSEQ) {
        am_first = p.e.amax[tc0];
        xs_first = p.e.xsum[tc0];
    }

    for (int i = tid; i < NTR * NMAT * MSUB * 16 * 16; i += T) (&red[0][0][0][0])[i] = 0;
    if constexpr (RPW) {
        // One row per wave: the row's amax, rounding and sum(xq) are the
        // wave's alone (DPP reductions, no exchange), so the prologue's only
        // workgroup barrier is the last one, before the MFMAs read the LDS
        // copy.  Rounding as below: the largest |x| bit pattern flags a row
        // holding NaN or infinity (loom's NaN-skipping maximum and per-value
        // fp64 rounding for it); finite rows round in fp32 with one exactness
        // test per slot of four values, redoing only the undecided slots.
        if (wave < M) {  // uniform
            const int r = wave;
            unsigned lb = 0u;
#pragma unroll
            for (int j = 0; j < FV; ++j) {
                if (lane + 64 * j < row4) {
                    lb = max(lb, max(max(__float_as_uint(xv[j].x) & 0x7fffffffu, __float_as_uint(xv[j].y) & 0x7fffffffu),
                                     max(__float_as_uint(xv[j].z) & 0x7fffffffu, __float_as_uint(xv[j].w) & 0x7fffffffu)));
                }
            }
            unsigned amb = wave_umax_dpp(lb);
            const bool gen = amb > 0x7f7fffffu;  // (wave-uniform)
            if (gen) {
                float lm = 0.0f;
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    if (lane + 64 * j < row4) {
                        float a = max_nan_skip(0.0f, fabsf(xv[j].x));
                        a = max_nan_skip(a, fabsf(xv[j].y));
                        a = max_nan_skip(a, fabsf(xv[j].z));
                        a = max_nan_skip(a, fabsf(xv[j].w));
                        lm = max_nan_skip(lm, a);
                    }
                }
                amb = __float_as_uint(wave_max_dpp(lm));
            }
            if (lane == 0) amax_bits[r] = amb;  // read after the main loop
            float am = __uint_as_float(amb);
            if (am < 1e-5f) am = 1e-5f;
            uint32_t pk[FV];
            bool undecided[FV];  // slot j holds a value the fp32 test leaves to fp64
            bool any = gen;
#pragma unroll
            for (int j = 0; j < FV; ++j) {
                pk[j] = 0u;
                undecided[j] = gen;
            }
            if (!gen) {
                const float sf = 127.0f / am;  // (fp32 division, correctly rounded)
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    if (lane + 64 * j < row4) {
                        const float p0 = xv[j].x * sf, p1 = xv[j].y * sf, p2 = xv[j].z * sf, p3 = xv[j].w * sf;
                        const float r0 = rintf(p0), r1 = rintf(p1), r2 = rintf(p2), r3 = rintf(p3);
                        const float d = fmaxf(fmaxf(fabsf(p0 - r0), fabsf(p1 - r1)), fmaxf(fabsf(p2 - r2), fabsf(p3 - r3)));
                        undecided[j] = !(0.5f - d > 3.1e-5f);
                        any |= undecided[j];
                        pk[j] = pack4((int)r0, (int)r1, (int)r2, (int)r3);
                    }
                }
            }
            if (any) {  // (per lane) loom's fp64 rounding for the undecided slots
                const double s = 127.0 / (double)am;
                const float s32 = (float)s;
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    if (undecided[j] && lane + 64 * j < row4)
                        pk[j] = pack4(quant_f32(xv[j].x, s32, s), quant_f32(xv[j].y, s32, s),
                                      quant_f32(xv[j].z, s32, s), quant_f32(xv[j].w, s32, s));
                }
            }
            int8_t* qr = xq_s + r * p.ldq;
            int ls = 0;
#pragma unroll
            for (int j = 0; j < FV; ++j) {
                if (lane + 64 * j < row4) {
                    *(uint32_t*)(qr + 4 * (lane + 64 * j)) = pk[j];
                    ls = byte_sum_i8(pk[j], ls);
                }
            }
            for (int c = k + 4 * lane; c < p.ldq; c += 256) *(uint32_t*)(qr + c) = 0u;  // padding
            const int v = wave_sum_i_dpp(ls);
            if (lane == 0) xsum_s[r] = v;  // read after the main loop
        }
        __syncthreads();
        if (blockIdx.x == 0) {
            if (p.xq_tap) {
                for (int i = tid; i < M * k; i += T) p.xq_tap[i] = xq_s[(i / k) * p.ldq + (i % k)];
            }
            if (p.amax_tap && tid < M) {
                float am = __uint_as_float(amax_bits[tid]);
                p.amax_tap[tid] = am < 1e-5f ? 1e-5f : am;
            }
        }
    } else if (FUSEQ) {
        if (NORM != NORM_NONE) {
            // ---- sum of squares per row -----------------------------------
            double tot[MR];
            if (STRICT) {
                // one row: squares to LDS, then their element-order chain
                double* sq = (double*)xq_s;
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    const int idx = tid + j * T;
                    if (idx < n4) {
                        if (F64) {
#pragma unroll
                            for (int c = 0; c < 4; ++c) sq[4 * idx + c] = xd[j][c] * xd[j][c];
                        } else {
                            const double a = xv[j].x, b = xv[j].y, c = xv[j].z, d = xv[j].w;
                            sq[4 * idx] = a * a;
                            sq[4 * idx + 1] = b * b;
                            sq[4 * idx + 2] = c * c;
                            sq[4 * idx + 3] = d * d;
                        }
                    }
                }
                __syncthreads();
                if constexpr (WAVES >= 8 && NMAT == 1) {  // long rows on eight waves, others on four
                    __shared__ union {
                        OrderedSumLds<8> w8;
                        OrderedSumLds<4> w4;
                    } osum;
                    if (k >= kSumWideCols) {
                        tot[0] = ordered_sum_block<8>(sq, k, 0.0, osum.w8);
                    } else {
                        tot[0] = ordered_sum_block<4>(sq, k, 0.0, osum.w4);
                    }
                } else if constexpr (WAVES >= 4) {
                    __shared__ OrderedSumLds<4> osum;
                    tot[0] = ordered_sum_block<4>(sq, k, 0.0, osum);
                } else {
                    tot[0] = ordered_sum_wave<kChainC>(sq, k, 0.0);
                }
#pragma unroll
                for (int rr = 1; rr < MR; ++rr) tot[rr] = 0.0;
            } else {
                double ps[MR];
#pragma unroll
                for (int rr = 0; rr < MR; ++rr) ps[rr] = 0.0;
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    const int idx = tid + j * T;
                    if (idx < n4) {
                        const int row = row_of<MR>(idx, row4);
                        double q = 0.0;
                        if (F64) {
#pragma unroll
                            for (int c = 0; c < 4; ++c) q = q + xd[j][c] * xd[j][c];
                        } else {
                            const double a = xv[j].x, b = xv[j].y, c = xv[j].z, d = xv[j].w;
                            q = a * a;
                            q = q + b * b;
                            q = q + c * c;
                            q = q + d * d;
                        }
#pragma unroll
                        for (int rr = 0; rr < MR; ++rr)
                            if (rr == row) ps[rr] = ps[rr] + q;
                    }
                }
#pragma unroll
                for (int rr = 0; rr < MR; ++rr) {
                    if (rr < M) {
                        const double w = wave_sum_f64_dpp(ps[rr]);
                        if (lane == 0) nsum[wave][rr] = w;
                    }
                }
                __syncthreads();
#pragma unroll
                for (int rr = 0; rr < MR; ++rr) {
                    double t = 0.0;
                    if (rr < M) {
                        t = nsum[0][rr];
                        for (int w = 1; w < WAVES; ++w) t = t + nsum[w][rr];
                    }
                    tot[rr] = t;
                }
            }
            // ---- normalize in registers ------------------------------------
            double f[MR];
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) {
                const double ms = tot[rr] / (double)k + p.neps;
                f[rr] = NORM == NORM_RMS ? sqrt(ms) : 1.0 / sqrt(ms);  // rms, or scale
            }
            if constexpr (NORM == NORM_RMS) {
                // loom's float32((v / rms) * gain), each step in fp64.  With
                // y = 1 / rms (one correctly rounded division per row), p =
                // (v y) g lies within 5 * 2^-53 |p| of loom's fp64 value P
                // (three roundings here, two there); if p - t and p + t, t =
                // |p| 2^-50, round to the same float, so does P (fp64 and
                // fp32 rounding are monotone) and that float is the result.
                // A thread with a value whose bracket holds an fp32 rounding
                // boundary (or is NaN) redoes its values with the divisions.
                double y[MR];
#pragma unroll
                for (int rr = 0; rr < MR; ++rr) y[rr] = 1.0 / f[rr];
                float4 nv[FV];
                bool redo = false;
                auto bracket = [&](float v, double yr, float g) {
                    const double q = ((double)v * yr) * (double)g;
                    const double t = fabs(q) * 0x1p-50;
                    const float lo = (float)(q - t), hi = (float)(q + t);
                    redo |= !(lo == hi);
                    return lo;
                };
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    const int idx = tid + j * T;
                    nv[j] = xv[j];
                    if (idx < n4) {
                        const int row = row_of<MR>(idx, row4);
                        double yr = y[0];
#pragma unroll
                        for (int rr = 1; rr < MR; ++rr)
                            if (rr == row) yr = y[rr];
                        nv[j] = make_float4(bracket(xv[j].x, yr, gv[j].x), bracket(xv[j].y, yr, gv[j].y),
                                            bracket(xv[j].z, yr, gv[j].z), bracket(xv[j].w, yr, gv[j].w));
                    }
                }
                if (redo) {
#pragma unroll
                    for (int j = 0; j < FV; ++j) {
                        const int idx = tid + j * T;
                        if (idx < n4) {
                            const int row = row_of<MR>(idx, row4);
                            double fr = f[0];
#pragma unroll
                            for (int rr = 1; rr < MR; ++rr)
                                if (rr == row) fr = f[rr];
                            nv[j].x = (float)(((double)xv[j].x / fr) * (double)gv[j].x);
                            nv[j].y = (float)(((double)xv[j].y / fr) * (double)gv[j].y);
                            nv[j].z = (float)(((double)xv[j].z / fr) * (double)gv[j].z);
                            nv[j].w = (float)(((double)xv[j].w / fr) * (double)gv[j].w);
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < FV; ++j) xv[j] = nv[j];
            }
#pragma unroll
            for (int j = 0; j < FV; ++j) {
                const int idx = tid + j * T;
                if (NORM != NORM_RMS && idx < n4) {
                    const int row = row_of<MR>(idx, row4);
                    double fr = f[0];
#pragma unroll
                    for (int rr = 1; rr < MR; ++rr)
                        if (rr == row) fr = f[rr];
                    const double g0 = gv[j].x, g1 = gv[j].y, g2 = gv[j].z, g3 = gv[j].w;
                    if (NORM == NORM_INNER_F32) {
                        xv[j].x = (float)((double)xv[j].x * fr * g0);
                        xv[j].y = (float)((double)xv[j].y * fr * g1);
                        xv[j].z = (float)((double)xv[j].z * fr * g2);
                        xv[j].w = (float)((double)xv[j].w * fr * g3);
                    } else {
                        xd[j][0] = xd[j][0] * (fr * g0);
                        xd[j][1] = xd[j][1] * (fr * g1);
                        xd[j][2] = xd[j][2] * (fr * g2);
                        xd[j][3] = xd[j][3] * (fr * g3);
                    }
                }
            }
            if (p.norm_tap && blockIdx.x == 0) {
                // debug tap: the normalized rows as this workgroup quantizes them
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    const int idx = tid + j * T;
                    if (idx < n4) {
                        const int row = row_of<MR>(idx, row4);
                        const size_t at = (size_t)row * k + 4 * (size_t)(idx - row * row4);
                        if (F64) {
                            double* t = (double*)p.norm_tap + at;
                            t[0] = xd[j][0];
                            t[1] = xd[j][1];
                            t[2] = xd[j][2];
                            t[3] = xd[j][3];
                        } else {
                            *(float4*)((float*)p.norm_tap + at) = xv[j];
                        }
                    }
                }
            }
            __syncthreads();
        }
        // bitNetActivationMaxAbs per row (poly/bitnet_cpu.go:45-71).  fp32
        // rows first take the largest |x| bit pattern: the unsigned order of
        // non-negative floats' bits is their value order, and NaN (either
        // sign) sorts above every finite value and infinity, so the same
        // maximum says whether a row holds a value that is not finite.  Such
        // rows (a workgroup-uniform decision) take loom's NaN-skipping
        // maximum in a second pass, as fp64 rows always do.
        unsigned amb[MR];
        bool general = F64;
        if constexpr (!F64) {
            unsigned lb[MR];
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) lb[rr] = 0u;
#pragma unroll
            for (int j = 0; j < FV; ++j) {
                const int idx = tid + j * T;
                if (idx < n4) {
                    const unsigned a = max(max(__float_as_uint(xv[j].x) & 0x7fffffffu, __float_as_uint(xv[j].y) & 0x7fffffffu),
                                           max(__float_as_uint(xv[j].z) & 0x7fffffffu, __float_as_uint(xv[j].w) & 0x7fffffffu));
                    const int row = row_of<MR>(idx, row4);
#pragma unroll
                    for (int rr = 0; rr < MR; ++rr)
                        if (rr == row) lb[rr] = max(lb[rr], a);
                }
            }
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) {
                if (rr < M) {
                    const unsigned wm = wave_umax_dpp(lb[rr]);
                    if (lane == 0) wmaxb[wave][rr] = wm;
                }
            }
            __syncthreads();
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) {
                unsigned m = 0u;
                if (rr < M)
                    for (int w = 0; w < WAVES; ++w) m = max(m, wmaxb[w][rr]);
                amb[rr] = m;
                if (m > 0x7f7fffffu) general = true;  // NaN or infinity in row rr
            }
        }
        if (general) {
            float lm[MR];
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) lm[rr] = 0.0f;
#pragma unroll
            for (int j = 0; j < FV; ++j) {
                const int idx = tid + j * T;
                if (idx < n4) {
                    float a;
                    if (F64) {
                        a = max_nan_skip(0.0f, (float)fabs(xd[j][0]));
                        a = max_nan_skip(a, (float)fabs(xd[j][1]));
                        a = max_nan_skip(a, (float)fabs(xd[j][2]));
                        a = max_nan_skip(a, (float)fabs(xd[j][3]));
                    } else {
                        a = max_nan_skip(0.0f, fabsf(xv[j].x));
                        a = max_nan_skip(a, fabsf(xv[j].y));
                        a = max_nan_skip(a, fabsf(xv[j].z));
                        a = max_nan_skip(a, fabsf(xv[j].w));
                    }
                    const int row = row_of<MR>(idx, row4);
#pragma unroll
                    for (int rr = 0; rr < MR; ++rr)
                        if (rr == row) lm[rr] = max_nan_skip(lm[rr], a);
                }
            }
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) {
                if (rr < M) {
                    const float wm = wave_max_dpp(lm[rr]);
                    if (lane == 0) wmax[wave][rr] = wm;
                }
            }
            __syncthreads();
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) {
                float am = 0.0f;
                if (rr < M) {
                    for (int w = 0; w < WAVES; ++w) am = max_nan_skip(am, wmax[w][rr]);
                }
                amb[rr] = __float_as_uint(am);
            }
        }
        // bitNetQuantizedActivation (poly/bitnet_cpu.go:73-95) into LDS.
        float amc[MR], scf[MR];
#pragma unroll
        for (int rr = 0; rr < MR; ++rr) {
            float am = __uint_as_float(amb[rr]);
            if (tid == rr) amax_bits[rr] = amb[rr];  // read after the main loop
            if (am < 1e-5f) am = 1e-5f;
            amc[rr] = am;
            scf[rr] = rr < M ? 127.0f / am : 0.0f;  // (fp32 division, correctly rounded)
        }
        // loom's fp64 scales 127 / am and their fp32 roundings (formed where a
        // branch needs them, off the fp32 path)
        auto scales64 = [&](double (&sc)[MR], float (&sc32)[MR]) {
#pragma unroll
            for (int rr = 0; rr < MR; ++rr) {
                sc[rr] = rr < M ? 127.0 / (double)amc[rr] : 0.0;
                sc32[rr] = (float)sc[rr];
            }
        };
        int ls[MR];
#pragma unroll
        for (int rr = 0; rr < MR; ++rr) ls[rr] = 0;
        if constexpr (!F64) {
            if (!general) {
                // Finite rows, rounded in fp32 with sf = fl32(127 / am) (an
                // fp32 division, so loom's fp64 scale stays off this path):
                // sf is within 2^-24 + 2^-53 (relative) of loom's scale s, so
                // p = fl32(x sf) is, as in quant_f32, within
                // 127 (2^-23 + 2^-47) < 1.52e-5 of loom's fp64 product x s,
                // and 3.1e-5 from every boundary j + 1/2 decides.  Every
                // |x| <= amax <= am, so |p| < 127.5 and rintf needs no clamp.
                // The test 0.5f - |p - r| > 3.1e-5f holds for all of a
                // thread's values iff it holds for the largest |p - r|
                // (fl(0.5f - d) does not increase with d): one test per thread
                // instead of a branch per value, and a thread with a value
                // nearer a boundary redoes its values with quant_f32 (up to
                // four rows of 640 or fewer float4 a thread: a near-tie in a
                // thread is rare enough that tracking slots cost more).
                float dmax = 0.0f;
                uint32_t pk[FV];
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    const int idx = tid + j * T;
                    pk[j] = 0u;
                    if (idx < n4) {
                        const int row = row_of<MR>(idx, row4);
                        float s32 = scf[0];
#pragma unroll
                        for (int rr = 1; rr < MR; ++rr)
                            if (rr == row) s32 = scf[rr];
                        const float p0 = xv[j].x * s32, p1 = xv[j].y * s32, p2 = xv[j].z * s32, p3 = xv[j].w * s32;
                        const float r0 = rintf(p0), r1 = rintf(p1), r2 = rintf(p2), r3 = rintf(p3);
                        dmax = fmaxf(dmax, fmaxf(fmaxf(fabsf(p0 - r0), fabsf(p1 - r1)),
                                                 fmaxf(fabsf(p2 - r2), fabsf(p3 - r3))));
                        pk[j] = pack4((int)r0, (int)r1, (int)r2, (int)r3);
                    }
                }
                if (!(0.5f - dmax > 3.1e-5f)) {
                    double sc[MR];
                    float sc32[MR];
                    scales64(sc, sc32);
#pragma unroll
                    for (int j = 0; j < FV; ++j) {
                        const int idx = tid + j * T;
                        if (idx < n4) {
                            const int row = row_of<MR>(idx, row4);
                            double s = sc[0];
                            float s32 = sc32[0];
#pragma unroll
                            for (int rr = 1; rr < MR; ++rr)
                                if (rr == row) {
                                    s = sc[rr];
                                    s32 = sc32[rr];
                                }
                            pk[j] = pack4(quant_f32(xv[j].x, s32, s), quant_f32(xv[j].y, s32, s),
                                          quant_f32(xv[j].z, s32, s), quant_f32(xv[j].w, s32, s));
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < FV; ++j) {
                    const int idx = tid + j * T;
                    if (idx < n4) {
                        const int row = row_of<MR>(idx, row4);
                        *(uint32_t*)(xq_s + row * p.ldq + 4 * (idx - row * row4)) = pk[j];
#pragma unroll
                        for (int rr = 0; rr < MR; ++rr)
                            if (rr == row) ls[rr] = byte_sum_i8(pk[j], ls[rr]);
                    }
                }
            }
        }
        if (general) {  // fp64 rows, and fp32 rows with a NaN or infinity
            double sc[MR];
            float sc32[MR];
            scales64(sc, sc32);
#pragma unroll
            for (int j = 0; j < FV; ++j) {
                const int idx = tid + j * T;
                if (idx < n4) {
                    const int row = row_of<MR>(idx, row4);
                    double s = sc[0];
                    float s32 = sc32[0];
#pragma unroll
                    for (int rr = 1; rr < MR; ++rr)
                        if (rr == row) {
                            s = sc[rr];
                            s32 = sc32[rr];
                        }
                    int q0, q1, q2, q3;
                    if (F64) {
                        q0 = quant_one(xd[j][0], s);
                        q1 = quant_one(xd[j][1], s);
                        q2 = quant_one(xd[j][2], s);
                        q3 = quant_one(xd[j][3], s);
                    } else {
                        q0 = quant_f32(xv[j].x, s32, s);
                        q1 = quant_f32(xv[j].y, s32, s);
                        q2 = quant_f32(xv[j].z, s32, s);
                        q3 = quant_f32(xv[j].w, s32, s);
                    }
                    *(uint32_t*)(xq_s + row * p.ldq + 4 * (idx - row * row4)) = pack4(q0, q1, q2, q3);
#pragma unroll
                    for (int rr = 0; rr < MR; ++rr)
                        if (rr == row) ls[rr] += q0 + q1 + q2 + q3;
                }
            }
        }
        // zero the padding columns k .. ldq of every row
        const int pad4 = (p.ldq - k) >> 2;
        for (int i = tid; i < M * pad4; i += T) {
            const int row = i / pad4;
            *(uint32_t*)(xq_s + row * p.ldq + k + 4 * (i - row * pad4)) = 0u;
        }
#pragma unroll
        for (int rr = 0; rr < MR; ++rr) {
            if (rr < M) {
                const int v = wave_sum_i_dpp(ls[rr]);
                if (lane == 0) wsum[wave][rr] = v;
            }
        }
        __syncthreads();
        if (tid < kFusedMaxRows) {
            int t = 0;
            if (tid < M)
                for (int w = 0; w < WAVES; ++w) t += wsum[w][tid];
            xsum_s[tid] = t;  // read after the main loop's barrier
        }
        if (blockIdx.x == 0) {
            if (p.xq_tap) {
                for (int i = tid; i < M * k; i += T) p.xq_tap[i] = xq_s[(i / k) * p.ldq + (i % k)];
            }
            if (p.amax_tap && tid < M) {
                float am = __uint_as_float(amax_bits[tid]);
                p.amax_tap[tid] = am < 1e-5f ? 1e-5f : am;
            }
        }
    }


    v4i acc[NTR][NMAT][MSUB];
#pragma unroll
    for (int q = 0; q < NTR; ++q)
#pragma unroll
        for (int a = 0; a < NMAT; ++a)
#pragma unroll
            for (int ms = 0; ms < MSUB; ++ms) acc[q][a][ms] = v4i{0, 0, 0, 0};

    const int8_t* xbase[MSUB];
    bool xval[MSUB];
    uint32_t xoff[MSUB];  // pre-quantized rows: byte offsets (rows past M read zero)
#pragma unroll
    for (int ms = 0; ms < MSUB; ++ms) {
        const int row = ms * 16 + r;
        xval[ms] = row < M;
        const int rr = xval[ms] ? row : 0;
        xbase[ms] = (FUSEQ ? (const int8_t*)xq_s : p.xq) + (size_t)rr * p.ldq + g * 16;
        xoff[ms] = (uint32_t)row * (uint32_t)p.ldq + (uint32_t)g * 16u;
    }
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(p.xq, FUSEQ ? 0u : (uint32_t)M * (uint32_t)p.ldq);

    for (int kb = wave; kb < ktiles; kb += WAVES * U) {
        // next batch's weights, issued before this batch's MFMAs
        uint4 wn[NTR][NMAT][U];
        const int kn = kb + WAVES * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kn + u * WAVES;
            if (kt < ktiles) {
#pragma unroll
                for (int q = 0; q < NTR; ++q) {
                    wn[q][0][u] = load16_nt(p.w0 + tile0[q] + (size_t)kt * 64);
                    if (NMAT == 2) wn[q][NMAT - 1][u] = load16_nt(p.w1 + tile0[q] + (size_t)kt * 64);
                }
            }
        }
        v4i a[MSUB][U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kb + u * WAVES;
            if (kt < ktiles) {
#pragma unroll
                for (int ms = 0; ms < MSUB; ++ms) {
                    if (FUSEQ) {
                        // rows past M read row 0 of the LDS copy (xbase clamps
                        // them); their sums are never added to the reduction
                        const int8_t* xp = xbase[ms] + (size_t)kt * kTileCols;
#pragma unroll
                        for (int t = 0; t < 4; ++t) a[ms][u][t] = *(const v4i*)(xp + 64 * t);
                    } else {
                        // rows past M fall past the buffer's end: zero, no branch
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            a[ms][u][t] = __builtin_bit_cast(
                                v4i, buffer_load16(xr, xoff[ms] + (uint32_t)kt * kTileCols + 64u * t));
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kb + u * WAVES;
            if (kt < ktiles) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
#pragma unroll
                    for (int q = 0; q < NTR; ++q)
#pragma unroll
                        for (int mat = 0; mat < NMAT; ++mat) {
                            const v4i b = unpack_codes(word_of(wv[q][mat][u], t));
#pragma unroll
                            for (int ms = 0; ms < MSUB; ++ms)
                                acc[q][mat][ms] = mfma_i8(a[ms][u][t], b, acc[q][mat][ms]);
                        }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < NTR; ++q)
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int u = 0; u < U; ++u) wv[q][mat][u] = wn[q][mat][u];
    }

    __syncthreads();
#pragma unroll
    for (int q = 0; q < NTR; ++q)
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int ms = 0; ms < MSUB; ++ms)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int tok = ms * 16 + 4 * g + v;
                    // (rows past M multiplied zero activations: their zero sums go
                    // to rows the epilogue never reads, with no branch)
                    if (!FUSEQ || tok < M) atomicAdd(&red[q][mat][tok][r], acc[q][mat][ms][v]);
                }
    __syncthreads();

    // Rounds of EB (at most two) outputs per thread; a round loads the inputs
    // of all its outputs before its first store (the first round's first
    // output's were loaded at the start).  Output idx: tile idx / (16 M),
    // token (idx mod 16 M) / 16, column idx mod 16.
    constexpr int EPT = (NTR * MSUB * 256 + T - 1) / T;
    constexpr int EB = EPT < 2 ? EPT : 2;
    const int total = NTR * M * 16;
    for (int base = 0; base < total; base += EB * T) {
        int tk[EB], nn[EB], xs[EB], qq[EB];
        float am[EB];
        EpiIn in[EB];
#pragma unroll
        for (int j = 0; j < EB; ++j) {
            const int idx = base + tid + j * T;
            const int q = NTR == 1 ? 0 : idx / (M * 16);
            const int rem = idx - q * (M * 16);
            qq[j] = q;
            tk[j] = rem >> 4;
            nn[j] = (nt + q) * kTileRows + (rem & 15);
            const int tc = min(tk[j], M - 1), nc = min(nn[j], p.e.n - 1);
            const bool first = j == 0 && base == 0;
            if (FUSEQ) {
                const float a = __uint_as_float(amax_bits[tc]);
                am[j] = a < 1e-5f ? 1e-5f : a;
                xs[j] = xsum_s[tc];
            } else if (first) {
                am[j] = am_first;
                xs[j] = xs_first;
            } else {
                am[j] = p.e.amax[tc];
                xs[j] = p.e.xsum[tc];
            }
            in[j] = first && kEarlyIn ? in_first : epilogue_inputs(p.e, tc, nc);
        }
#pragma unroll
        for (int j = 0; j < EB; ++j) {
            const int idx = base + tid + j * T;
            if (idx < total && nt + qq[j] < p.ntiles && nn[j] < p.e.n) {
                const int col = idx & 15;
                const RowScale rs = row_scale(p.e, am[j], xs[j]);
                epilogue_store_pre(p.e, tk[j], nn[j], red[qq[j]][0][tk[j]][col], red[qq[j]][NMAT - 1][tk[j]][col],
                                   rs.os0, rs.os1, rs.xs, in[j].b0, in[j].b1, in[j].res);
            }
        }
    }
}

// ------------------------------------------------------------------------
// skinny_nt: 16 < M <= 64 on pre-quantized rows.  The same per-wave K split
// and 16x16x64 MFMAs as skinny_kernel, but a workgroup owns NT adjacent
// 16-row weight tiles, so the activation operands a wave loads for a K tile
// serve NT tiles.  Every workgroup reads all M rows, and per 256-column K
// tile those are M x 256 bytes against 1 KiB of one tile's weights, so at
// these M the activation bytes pulled into the CUs dominate; they drop by NT.
// ------------------------------------------------------------------------
template <int NMAT, int MSUB, int WAVES, int NT>
__global__ __launch_bounds__(WAVES * 64) void skinny_nt_kernel(MatArgs p) {
    constexpr int T = WAVES * 64;
    constexpr int U = 4 / MSUB;  // K tiles per batch per wave
    __shared__ int red[NT][NMAT][MSUB * 16][16];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int M = p.e.m;
    const int ktiles = p.ktiles;
    const int nt0 = blockIdx.x * NT;
    // tiles past the last one read the last tile and store nothing
    size_t tile0[NT];
#pragma unroll
    for (int q = 0; q < NT; ++q) tile0[q] = (size_t)min(nt0 + q, p.ntiles - 1) * ktiles * 64 + lane;

    uint4 wv[NT][NMAT][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int kt = wave + u * WAVES;
        if (kt < ktiles) {
#pragma unroll
            for (int q = 0; q < NT; ++q) {
                wv[q][0][u] = load16_nt(p.w0 + tile0[q] + (size_t)kt * 64);
                if (NMAT == 2) wv[q][NMAT - 1][u] = load16_nt(p.w1 + tile0[q] + (size_t)kt * 64);
            }
        }
    }
    for (int i = tid; i < NT * NMAT * MSUB * 16 * 16; i += T) (&red[0][0][0][0])[i] = 0;

    v4i acc[NT][NMAT][MSUB];
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
        for (int a = 0; a < NMAT; ++a)
#pragma unroll
            for (int ms = 0; ms < MSUB; ++ms) acc[q][a][ms] = v4i{0, 0, 0, 0};

    uint32_t xoff[MSUB];  // byte offsets of this lane's rows (rows past M read zero)
#pragma unroll
    for (int ms = 0; ms < MSUB; ++ms) xoff[ms] = (uint32_t)(ms * 16 + r) * (uint32_t)p.ldq + (uint32_t)g * 16u;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(p.xq, (uint32_t)M * (uint32_t)p.ldq);

    for (int kb = wave; kb < ktiles; kb += WAVES * U) {
        uint4 wn[NT][NMAT][U];
        const int kn = kb + WAVES * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kn + u * WAVES;
            if (kt < ktiles) {
#pragma unroll
                for (int q = 0; q < NT; ++q) {
                    wn[q][0][u] = load16_nt(p.w0 + tile0[q] + (size_t)kt * 64);
                    if (NMAT == 2) wn[q][NMAT - 1][u] = load16_nt(p.w1 + tile0[q] + (size_t)kt * 64);
                }
            }
        }
        v4i a[MSUB][U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kb + u * WAVES;
            if (kt < ktiles) {
#pragma unroll
                for (int ms = 0; ms < MSUB; ++ms)
#pragma unroll
                    for (int t = 0; t < 4; ++t)  // rows past M fall past the buffer's end: zero, no branch
                        a[ms][u][t] = __builtin_bit_cast(
                            v4i, buffer_load16(xr, xoff[ms] + (uint32_t)kt * kTileCols + 64u * t));
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kb + u * WAVES;
            if (kt < ktiles) {
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int q = 0; q < NT; ++q)
#pragma unroll
                        for (int mat = 0; mat < NMAT; ++mat) {
                            const v4i b = unpack_codes(word_of(wv[q][mat][u], t));
#pragma unroll
                            for (int ms = 0; ms < MSUB; ++ms)
                                acc[q][mat][ms] = mfma_i8(a[ms][u][t], b, acc[q][mat][ms]);
                        }
            }
        }
#pragma unroll
        for (int q = 0; q < NT; ++q)
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int u = 0; u < U; ++u) wv[q][mat][u] = wn[q][mat][u];
    }

    __syncthreads();
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int ms = 0; ms < MSUB; ++ms)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int tok = ms * 16 + 4 * g + v;
                    atomicAdd(&red[q][mat][tok][r], acc[q][mat][ms][v]);  // rows past M add zero
                }
    __syncthreads();

    // Rounds of kEpiBatch outputs per thread: a round loads the amax, sum(xq),
    // bias and residual of all its outputs (clamped indices, no branch per
    // lane) before its first store.
    constexpr int EB = (NT * MSUB * 256 + T - 1) / T < kEpiBatch ? (NT * MSUB * 256 + T - 1) / T : kEpiBatch;
    const int total = NT * M * 16;
    for (int base = 0; base < total; base += EB * T) {
        int tk[EB], nn[EB], qq[EB], xs[EB];
        float am[EB];
        EpiIn in[EB];
#pragma unroll
        for (int j = 0; j < EB; ++j) {
            const int idx = base + tid + j * T;
            const int q = idx / (M * 16);
            const int rem = idx - q * (M * 16);
            qq[j] = q;
            tk[j] = rem >> 4;
            nn[j] = (nt0 + q) * kTileRows + (rem & 15);
            const int tc = min(tk[j], M - 1), nc = min(nn[j], p.e.n - 1);
            am[j] = p.e.amax[tc];
            xs[j] = p.e.xsum[tc];
            in[j] = epilogue_inputs(p.e, tc, nc);
        }
#pragma unroll
        for (int j = 0; j < EB; ++j) {
            const int idx = base + tid + j * T;
            if (idx < total && nt0 + qq[j] < p.ntiles && nn[j] < p.e.n) {
                const int col = nn[j] - (nt0 + qq[j]) * kTileRows;
                const RowScale rs = row_scale(p.e, am[j], xs[j]);
                epilogue_store_pre(p.e, tk[j], nn[j], red[qq[j]][0][tk[j]][col], red[qq[j]][NMAT - 1][tk[j]][col],
                                   rs.os0, rs.os1, rs.xs, in[j].b0, in[j].b1, in[j].res);
            }
        }
    }
}

// ------------------------------------------------------------------------
// small_split: 16 < M <= 64 on pre-quantized rows, one matrix.  What bounds
// these M is not HBM but the activation bytes every workgroup pulls from L2:
// with full K per workgroup each CU reads all M x K int8 rows (442 KB at
// M = 64, K = 6912), and a CU draws only a few tens of GB/s from L2 under
// that load.  So a workgroup owns NT = 4 adjacent 16-row weight tiles and a
// slice of KPS = 4 K tiles: it stages its M x 1 KiB activation slice in LDS
// with row-contiguous 16-byte loads (whole cache lines), its 8 waves take
// one K tile and two row tiles each, and the waves' partial sums meet in
// LDS in a fixed order.  The K slices of a row group then meet through
// device-scope integer atomic adds into the group's accumulators (integer
// sums: exact in any order); the last workgroup to arrive (arrival counter)
// reads the totals, runs the epilogue and sets accumulators and counter back
// to zero for the next launch.  Every partial add has completed (s_waitcnt)
// before its workgroup's arrival is counted, and the last workgroup reads
// only after its own arrival returns: the exchange of the split GEMM.
// ------------------------------------------------------------------------
constexpr int kSmallNT = 4;
constexpr int kSmallKps = 4;
constexpr int kSmallWaves = 8;

struct SmallSplit {
    int S;          // K slices (workgroups per row group)
    int32_t* acc;   // row-group accumulators (S > 1)
    unsigned* ctr;  // arrival counters (S > 1)
};

template <int MSUB>
__global__ __launch_bounds__(kSmallWaves * 64) void small_split_kernel(MatArgs p, SmallSplit ss) {
    constexpr int WAVES = kSmallWaves, T = WAVES * 64, NT = kSmallNT, KPS = kSmallKps;
    constexpr int R = MSUB * 16;          // staged rows (tokens)
    constexpr int PITCH = KPS * 256 + 16;  // bytes per staged row (16-row reads: no bank conflicts)
    constexpr int CH = R * KPS * 16;       // 16-byte chunks staged
    constexpr int CPT = CH / T;
    constexpr int QPW = NT * KPS / WAVES;  // row tiles per wave
    constexpr int EPT = NT * R * 16 / T;   // outputs per thread
    static_assert(CH % T == 0 && (NT * KPS) % WAVES == 0 && (NT * R * 16) % T == 0, "geometry");
    static_assert(NT * KPS * R * 16 * 4 <= R * PITCH, "partial sums fit the staging buffer");
    __shared__ __align__(16) int8_t lds[R * PITCH];  // activation slice, then the waves' partial sums
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int M = p.e.m;
    const int ktiles = p.ktiles;
    const int group = blockIdx.x / ss.S;
    const int slice = blockIdx.x - group * ss.S;
    const int nt0 = group * NT;
    const int kt0 = slice * KPS;

    // activation slice: chunk c is 16 bytes of row c / (16 KPS); a wave reads
    // 1 KiB of one row.  Rows past M and K tiles past the last read zero.
    const uint32_t xbytes = (uint32_t)M * (uint32_t)p.ldq;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(p.xq, xbytes);
    uint4 st[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tid + j * T;
        const int row = c / (KPS * 16), c16 = c % (KPS * 16);
        const bool ok = row < M && kt0 + c16 / 16 < ktiles;
        st[j] = buffer_load16(xr, ok ? (uint32_t)row * (uint32_t)p.ldq + (uint32_t)kt0 * 256u + c16 * 16u : xbytes);
    }
    // weights: wave w takes K tile kt0 + w % KPS of row tiles w / KPS + 2j
    const int ktl = wave % KPS;
    const uint32_t wbytes = (uint32_t)p.ntiles * (uint32_t)ktiles * 1024u;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(p.w0, wbytes);
    uint4 wv[QPW];
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
        const int nt = nt0 + wave / KPS + j * (WAVES / KPS);
        const int kt = kt0 + ktl;
        const bool ok = nt < p.ntiles && kt < ktiles;
        wv[j] = buffer_load16_nt(wr, ok ? (((uint32_t)nt * (uint32_t)ktiles + (uint32_t)kt) * 64u + lane) * 16u : wbytes);
    }
    // the epilogue's per-token amax and sum(xq), loaded while the rest is in
    // flight (clamped, unconditional loads: a branch around a load would make
    // the compiler wait for every load issued before it)
    float am[EPT];
    int xs[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int tok = min(((tid + i * T) % (R * 16)) >> 4, M - 1);
        am[i] = p.e.amax[tok];
        xs[i] = p.e.xsum[tok];
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tid + j * T;
        *(uint4*)&lds[(c / (KPS * 16)) * PITCH + (c % (KPS * 16)) * 16] = st[j];
    }
    __syncthreads();

    v4i acc[QPW][MSUB];
#pragma unroll
    for (int j = 0; j < QPW; ++j)
#pragma unroll
        for (int ms = 0; ms < MSUB; ++ms) acc[j][ms] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        v4i a[MSUB];
#pragma unroll
        for (int ms = 0; ms < MSUB; ++ms)
            a[ms] = *(const v4i*)&lds[(ms * 16 + r) * PITCH + ktl * 256 + 64 * t + 16 * g];
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const v4i b = unpack_codes(word_of(wv[j], t));
#pragma unroll
            for (int ms = 0; ms < MSUB; ++ms) acc[j][ms] = mfma_i8(a[ms], b, acc[j][ms]);
        }
    }
    __syncthreads();  // every wave has read its activations
    // partial sums: part[q][k][tok][col], q = row tile, k = K tile of the slice
    int* part = (int*)lds;
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
        const int q = wave / KPS + j * (WAVES / KPS);
#pragma unroll
        for (int ms = 0; ms < MSUB; ++ms)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                part[((q * KPS + ktl) * R + ms * 16 + 4 * g + v) * 16 + r] = acc[j][ms][v];
    }
    __syncthreads();
    int tot[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid + i * T;
        const int q = e / (R * 16), rem = e % (R * 16);
        int s = 0;
#pragma unroll
        for (int k = 0; k < KPS; ++k) s += part[(q * KPS + k) * R * 16 + rem];
        tot[i] = s;
    }
    if (ss.S > 1) {
        int32_t* gacc = ss.acc + (size_t)group * NT * 64 * 16;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int e = tid + i * T;
            const int q = e / (R * 16), rem = e % (R * 16);
            if ((rem >> 4) < M)
                __hip_atomic_fetch_add(&gacc[q * 64 * 16 + rem], tot[i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            s_last = __hip_atomic_fetch_add(&ss.ctr[group], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (unsigned)(ss.S - 1);
        }
        __syncthreads();
        if (!s_last) return;
        // (rows past M were never added to: zero, read and cleared unconditionally
        // so that no branch serializes the loads)
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int e = tid + i * T;
            const int q = e / (R * 16), rem = e % (R * 16);
            tot[i] = __hip_atomic_load(&gacc[q * 64 * 16 + rem], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int e = tid + i * T;
            const int q = e / (R * 16), rem = e % (R * 16);
            __hip_atomic_store(&gacc[q * 64 * 16 + rem], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // every workgroup of the group has arrived: ready for the next launch
        if (tid == 0) __hip_atomic_store(&ss.ctr[group], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // bias and residual of every output first, then the stores
    EpiIn in[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid + i * T;
        const int q = e / (R * 16), rem = e % (R * 16);
        const int n = (nt0 + q) * kTileRows + (rem & 15);
        in[i] = epilogue_inputs(p.e, min(rem >> 4, M - 1), min(n, p.e.n - 1));
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid + i * T;
        const int q = e / (R * 16), rem = e % (R * 16);
        const int tok = rem >> 4, col = rem & 15;
        const int n = (nt0 + q) * kTileRows + col;
        if (tok < M && nt0 + q < p.ntiles && n < p.e.n) {
            const RowScale rs = row_scale(p.e, am[i], xs[i]);
            epilogue_store_pre(p.e, tok, n, tot[i], tot[i], rs.os0, rs.os1, rs.xs, in[i].b0, in[i].b1, in[i].res);
        }
    }
}

// ------------------------------------------------------------------------
// dispatch
// ------------------------------------------------------------------------

// Split-K width: enough waves for ~2048 in flight over the chip, never more
// waves than K tiles, and at most `cap` (register budget of wide tiles).
static int pick_waves(int ntiles, int ktiles, int cap) {
    const int want = (2048 + ntiles - 1) / ntiles;
    int w = 1;
    while (w < want && w < cap && w < ktiles) w <<= 1;
    return w;
}

// Fused-quantization launch: the fewest float4 slots per thread that hold the
// rows (clamped loads fill the rest), and the one-row prologue for M = 1.
template <int NMAT, int WAVES>
static void launch_fused_w(const MatArgs& p, size_t shm, hipStream_t s) {
    const size_t groups = (size_t)p.e.m * (p.k / 4);
    const dim3 grid(p.ntiles), block(WAVES * 64);
    // One row, one matrix: a workgroup takes two adjacent weight tiles, so
    // the row's loads and quantization serve both, while the paired grid
    // still spans half the CUs (the Dense step at the BitNet-2B up shape,
    // 432 tiles, eight waves: 5.58 -> 5.24 us; at the down shape, 160 tiles,
    // pairs are slower: 4.96 -> 5.72 us).  LOOM_AMD_FUSED_NTR = 1, 2 or 4
    // overrides (tests and tuning; four tiles only with two float4 slots a
    // thread).
    if constexpr (NMAT == 1 && WAVES <= 8) {
        const int ntr = tune_int("LOOM_AMD_FUSED_NTR", ceil_div(p.ntiles, 2) >= 128 ? 2 : 1);
        if (p.e.m == 1 && groups <= (size_t)2 * WAVES * 64 && ntr == 2) {
            hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true, NORM_NONE, 0, 2, 1, 2>),
                               dim3(ceil_div(p.ntiles, 2)), block, shm, s, p);
            return;
        }
        if (p.e.m == 1 && groups <= (size_t)2 * WAVES * 64 && ntr == 4) {
            hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true, NORM_NONE, 0, 2, 1, 4>),
                               dim3(ceil_div(p.ntiles, 4)), block, shm, s, p);
            return;
        }
        if (p.e.m == 1 && groups <= (size_t)4 * WAVES * 64 && ntr == 2) {
            hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true, NORM_NONE, 0, 4, 1, 2>),
                               dim3(ceil_div(p.ntiles, 2)), block, shm, s, p);
            return;
        }
    }
    if (p.e.m == 1 && groups <= (size_t)2 * WAVES * 64) {
        hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true, NORM_NONE, 0, 2, 1>), grid, block, shm, s, p);
    } else if (p.e.m == 1 && groups <= (size_t)4 * WAVES * 64) {
        hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true, NORM_NONE, 0, 4, 1>), grid, block, shm, s, p);
    } else {
        hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true>), grid, block, shm, s, p);
    }
}

// 4 < M <= kFusedWaveRows fused rows: eight waves, one row each, the row's
// element groups in FV slots a lane (10 for K <= 2560, 16 for K <= 4096); two
// weight tiles per workgroup (one matrix) while the paired grid still spans
// half the CUs, as for one row (BitNet-2B up shape, M = 8: 6.0 us per Dense
// step; one tile 7.5, four 7.5; the separate quantization launch took 8.0).
// LOOM_AMD_FUSED_NTR = 1 or 2 overrides.
template <int NMAT, int FV>
static void launch_fused_rows_fv(const MatArgs& p, size_t shm, hipStream_t s) {
    const int ntr = NMAT == 1 ? tune_int("LOOM_AMD_FUSED_NTR", ceil_div(p.ntiles, 2) >= 128 ? 2 : 1) : 1;
    if (NMAT == 1 && ntr == 2) {
        hipLaunchKernelGGL((skinny_kernel<NMAT, 1, 8, true, NORM_NONE, 0, FV, kFusedWaveRows, 2>),
                           dim3(ceil_div(p.ntiles, 2)), dim3(512), shm, s, p);
    } else {
        hipLaunchKernelGGL((skinny_kernel<NMAT, 1, 8, true, NORM_NONE, 0, FV, kFusedWaveRows, 1>),
                           dim3(p.ntiles), dim3(512), shm, s, p);
    }
}

template <int NMAT, int MSUB, bool FUSEQ>
static hipError_t launch_skinny(const MatArgs& p, hipStream_t s) {
    // 1024-thread workgroups leave 128 VGPRs per lane: only the one-matrix kernels fit.
    constexpr int kCap = NMAT == 1 ? 16 : 8;
    if constexpr (FUSEQ) {
        if (p.e.m > kFusedMaxRows) {  // one row per wave (fused_quant_ok: K <= 4096)
            const size_t shm = (size_t)p.e.m * p.ldq;
            if (p.k / 4 <= 10 * 64) {
                launch_fused_rows_fv<NMAT, 10>(p, shm, s);
            } else {
                launch_fused_rows_fv<NMAT, 16>(p, shm, s);
            }
            return hipGetLastError();
        }
    }
    int w = pick_waves(p.ntiles, p.ktiles, kCap);
    if (FUSEQ) {
        // the fused prologue holds M*K/4 float4 over kFusedVec registers per thread
        while (w < kCap && (size_t)p.e.m * p.k > (size_t)4 * kFusedVec * 64 * w) w <<= 1;
    }
    const size_t shm = FUSEQ ? (size_t)p.e.m * p.ldq : 0;
    const dim3 grid(p.ntiles);
    if constexpr (FUSEQ) {
        // One row: the fewest waves, at least four, that hold it in four
        // float4 slots a thread (BitNet-2B shapes, M = 1: the up projection's
        // Dense step 5.15 -> 4.81 us with four waves instead of eight, two
        // waves 7.40; the down projection's 5.61 -> 4.96 us with eight
        // instead of sixteen; the SwiGLU FFN's fused gate|up pair takes the
        // FFN from 19.2 to 17.0 us with four waves instead of eight).
        if (p.e.m == 1) {
            int w1 = 4;
            while (w1 < w && (size_t)p.k / 4 > (size_t)4 * 64 * w1) w1 <<= 1;
            if (w1 < w) w = w1;
        }
    }
    if constexpr (FUSEQ) {
        const int v = tune_int("LOOM_AMD_FUSED_WAVES", 0);  // tuning override (1..16)
        if (v != 0) {
            if (v == 1 || v == 2 || v == 4 || v == 8 || (v == 16 && kCap == 16)) w = v;
            while (w < kCap && (size_t)p.e.m * p.k > (size_t)4 * kFusedVec * 64 * w) w <<= 1;
        }
        static_assert(MSUB == 1, "the fused prologue serves up to 4 rows");
        switch (w) {
            case 1: launch_fused_w<NMAT, 1>(p, shm, s); break;
            case 2: launch_fused_w<NMAT, 2>(p, shm, s); break;
            case 4: launch_fused_w<NMAT, 4>(p, shm, s); break;
            case 8: launch_fused_w<NMAT, 8>(p, shm, s); break;
            default:
                if constexpr (kCap == 16) launch_fused_w<NMAT, 16>(p, shm, s);
                break;
        }
        return hipGetLastError();
    }
    if constexpr (!FUSEQ && NMAT == 1 && MSUB == 1) {
        // Up to 16 pre-quantized rows, one matrix, eight waves: two weight tiles
        // per workgroup share the rows' loads (BitNet-2B up shape: M = 1
        // 4.10 -> 3.91 us, M = 8 4.77 -> 4.43, M = 16 5.59 -> 4.89).
        // LOOM_AMD_SKINNY_NTR = 1 takes one tile (tests and tuning).
        if (w == 8 && tune_int("LOOM_AMD_SKINNY_NTR", 0) != 1) {
            hipLaunchKernelGGL((skinny_kernel<NMAT, MSUB, 8, FUSEQ, NORM_NONE, 0, kFusedVec, kFusedMaxRows, 2>),
                               dim3(ceil_div(p.ntiles, 2)), dim3(512), shm, s, p);
            return hipGetLastError();
        }
    }
    switch (w) {
        case 1:
            hipLaunchKernelGGL((skinny_kernel<NMAT, MSUB, 1, FUSEQ>), grid, dim3(64), shm, s, p);
            break;
        case 2:
            hipLaunchKernelGGL((skinny_kernel<NMAT, MSUB, 2, FUSEQ>), grid, dim3(128), shm, s, p);
            break;
        case 4:
            hipLaunchKernelGGL((skinny_kernel<NMAT, MSUB, 4, FUSEQ>), grid, dim3(256), shm, s, p);
            break;
        case 8:
            hipLaunchKernelGGL((skinny_kernel<NMAT, MSUB, 8, FUSEQ>), grid, dim3(512), shm, s, p);
            break;
        default:
            if constexpr (kCap == 16) {
                hipLaunchKernelGGL((skinny_kernel<NMAT, MSUB, 16, FUSEQ>), grid, dim3(1024), shm, s, p);
            }
            break;
    }
    return hipGetLastError();
}

// 16 < M <= 64 on pre-quantized rows: tiles per workgroup.  Two tiles pay
// for short K with many tiles (measured at M = 17..64: the up shape, K = 2560,
// 13.4 -> 10.9 us at M = 64); with long K (the down shape, 27 K tiles) the
// halved workgroup count lengthens each wave's serial K loop and one tile is
// faster.  LOOM_AMD_SKINNY_NT = 1, 2 or 4 overrides (1 = skinny_kernel).
static int skinny_nt(int ntiles, int ktiles) {
    const int nt = tune_int("LOOM_AMD_SKINNY_NT", 0);
    if (nt == 1 || nt == 2 || nt == 4) return nt;
    return ktiles <= 16 && ntiles >= 256 ? 2 : 1;
}

// At most 8 waves: the NT-tile accumulators leave too few VGPRs for 1024
// threads.
template <int NMAT, int MSUB, int NT>
static hipError_t launch_skinny_nt(const MatArgs& p, hipStream_t s) {
    const int groups = ceil_div(p.ntiles, NT);
    const int w = pick_waves(groups, p.ktiles, 8);
    const dim3 grid(groups);
    switch (w) {
        case 1: hipLaunchKernelGGL((skinny_nt_kernel<NMAT, MSUB, 1, NT>), grid, dim3(64), 0, s, p); break;
        case 2: hipLaunchKernelGGL((skinny_nt_kernel<NMAT, MSUB, 2, NT>), grid, dim3(128), 0, s, p); break;
        case 4: hipLaunchKernelGGL((skinny_nt_kernel<NMAT, MSUB, 4, NT>), grid, dim3(256), 0, s, p); break;
        default: hipLaunchKernelGGL((skinny_nt_kernel<NMAT, MSUB, 8, NT>), grid, dim3(512), 0, s, p); break;
    }
    return hipGetLastError();
}

// small_split_kernel for one matrix when its workspace holds the row groups.
// Its K-slice exchange costs a few microseconds (three device-scope round
// trips), so it pays only where full-K workgroups pull the most activation
// bytes: long K (more than 16 K tiles) and M > 24 (measured at M = 17..64:
// K = 6912 13.8 vs 16.2 us at M = 64, 9.4 vs 9.7 at M = 32; K = 2560 slower
// at every M).  LOOM_AMD_SMALLM = 1 always takes it, 0 never (2: the GEMM
// kernel for every 16 < M <= 64).
template <int MSUB>
static bool launch_small_split(const MatArgs& p, int device, hipStream_t s, hipError_t* e) {
    const int mode = tune_int("LOOM_AMD_SMALLM", -1);
    if (mode == 0 || (mode != 1 && (p.ktiles <= 16 || p.e.m <= 24))) return false;
    const int groups = ceil_div(p.ntiles, kSmallNT);
    const int S = ceil_div(p.ktiles, kSmallKps);
    SmallSplit ss{S, nullptr, nullptr};
    if (S > 1) {
        const SmallSplitWs ws = small_split_ws(device);
        if (!ws.acc || groups > kSmallSplitGroups || (size_t)groups * kSmallNT * 64 * 16 > (size_t)kSmallSplitInts)
            return false;
        ss.acc = ws.acc;
        ss.ctr = ws.ctr;
    }
    hipLaunchKernelGGL((small_split_kernel<MSUB>), dim3(groups * S), dim3(kSmallWaves * 64), 0, s, p, ss);
    *e = hipGetLastError();
    return true;
}

// (four tiles of both SwiGLU matrices do not fit the register file)
// 32 < M <= 64 on one matrix with long K (more than 16 K tiles) or M > 56:
// the GEMM kernel (one 64-token tile: half-width tiles split over K), which
// beats both small-M kernels there (measured, one box: down shape M = 64
// 13.1 -> 10.2 us, M = 48 11.4 -> 10.8, M = 33 11.2 -> 10.5; up shape M = 64
// 9.85 -> 9.0, but M = 48 8.7 -> 9.5, so shorter K keeps the skinny kernels).
template <int NMAT, int MSUB>
static hipError_t launch_small_m(const MatArgs& p, int device, hipStream_t s) {
    hipError_t e = hipSuccess;
    const int mode = tune_int("LOOM_AMD_SMALLM", -1);
    if (mode == 2 || (mode == -1 && NMAT == 1 && MSUB == 4 && (p.ktiles > 16 || p.e.m > 56)))
        return launch_gemm(p, NMAT == 2, device, s);
    if (NMAT == 1 && launch_small_split<MSUB>(p, device, s, &e)) return e;
    const int nt = skinny_nt(p.ntiles, p.ktiles);
    if constexpr (NMAT == 1) {
        if (nt == 4) return launch_skinny_nt<NMAT, MSUB, 4>(p, s);
    }
    if (nt >= 2) return launch_skinny_nt<NMAT, MSUB, 2>(p, s);
    return launch_skinny<NMAT, MSUB, false>(p, s);
}

const char* kernel_variant(int m) {
    if (m <= kFusedWaveRows) return "skinny_m16_fusedq";  // (K <= 4096 from M = 5 on)
    if (m <= 16) return "skinny_m16";
    if (m <= 32) return "skinny_m32";
    if (m <= 56) return "skinny_m64";  // (the GEMM when K exceeds 16 K tiles)
    if (m <= 64) return "gemm_m64";
    return "gemm";  // gemm_lds_kernel (64- or 128-token tiles): 32x32x32 MFMA, split K
}

static MatArgs make_args(const Matrix* w0, const Matrix* w1, int m, const Epilogue& epi) {
    MatArgs p{};
    p.w0 = (const uint4*)w0->tiles;
    p.w1 = (const uint4*)(w1 ? w1->tiles : w0->tiles);
    p.ktiles = w0->ktiles;
    p.ntiles = w0->ntiles;
    p.k = w0->cols;
    EpiDev& e = p.e;
    e.kind = epi.kind;
    e.activation = epi.activation;
    e.m = m;
    e.n = w0->rows;
    e.scale0 = w0->scale;
    e.scale1 = w1 ? w1->scale : w0->scale;
    e.bias0 = epi.bias0;
    e.bias1 = epi.bias1;
    e.residual = epi.residual;
    e.out = epi.out;
    e.post = epi.post;
    e.ldo = epi.ldo > 0 ? epi.ldo : w0->rows;
    e.acc0 = epi.acc0;
    e.acc1 = epi.acc1;
    return p;
}

hipError_t launch_matmul(const Matrix* w0, const Matrix* w1, const QuantAct& a, int m,
                         const Epilogue& epi, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    MatArgs p = make_args(w0, w1, m, epi);
    p.xq = a.xq;
    p.ldq = a.ldq;
    p.e.amax = a.amax;
    p.e.xsum = a.xsum;
    const bool two = epi.kind == EPI_SWIGLU;
    if (!two && stream_ok(m, w0->cols, w0->ntiles, false, epi)) return launch_stream(p, false, s);
    if (m <= 16) return two ? launch_skinny<2, 1, false>(p, s) : launch_skinny<1, 1, false>(p, s);
    if (m <= 32) return two ? launch_small_m<2, 2>(p, w0->device, s) : launch_small_m<1, 2>(p, w0->device, s);
    if (m <= 64) return two ? launch_small_m<2, 4>(p, w0->device, s) : launch_small_m<1, 4>(p, w0->device, s);
    return launch_gemm(p, two, w0->device, s);
}

// The fused prologue holds the M x K rows in registers (kFusedVec float4 per
// thread of a 512-thread workgroup) and their int8 copy in LDS.
bool fused_quant_ok(int m, int k, const float* x) {
    if (m < 1 || k % 4 != 0 || ((uintptr_t)x & 15) != 0) return false;
    if (m <= kFusedMaxRows)
        return (size_t)m * k <= (size_t)4 * kFusedVec * 512 && pad_cols(k) * (size_t)m <= 64 * 1024;
    // one row per wave: a row in at most 16 float4 slots of a wave's lanes
    return m <= kFusedWaveRows && k <= 16 * 64 * 4 && pad_cols(k) * (size_t)m <= 64 * 1024;
}

// ---- norm-fused decode matmuls ------------------------------------------------
// 512-thread workgroups; FV element groups of 4 per thread hold the rows.
constexpr int kNormWaves = 8;
constexpr int kNormThreads = kNormWaves * 64;

// Dynamic LDS of a norm-fused launch: the quantized rows, or in strict mode
// the row's squares padded for ordered_sum_block (four waves, or eight for
// rows of kSumWideCols and more).
static size_t norm_lds(int m, int k, int strict) {
    const size_t q = (size_t)m * pad_cols(k);
    const int slots = max(ordered_sum_slots(k, 4), k >= kSumWideCols ? ordered_sum_slots(k, 8) : 0);
    const size_t sq = strict ? (size_t)slots * 8 : 0;
    return q > sq ? q : sq;
}

bool norm_fused_ok(int m, int k, int strict, bool x16) {
    if (m < 1 || m > kFusedMaxRows || k % 4 != 0 || !x16) return false;
    // rows held in registers: up to 4 element groups per thread (more spills)
    if ((size_t)m * (k / 4) > (size_t)4 * kNormThreads) return false;
    if (strict && m != 1) return false;  // one row of squares in LDS
    return norm_lds(m, k, strict) <= 96 * 1024;
}

template <int NMAT, int NORM, int STRICT, int WAVES, int FV>
static hipError_t launch_norm_t(const MatArgs& p, size_t shm, hipStream_t s) {
    if (p.e.m == 1) {  // one-row prologue (decode)
        hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true, NORM, STRICT, FV, 1>), dim3(p.ntiles),
                           dim3(WAVES * 64), shm, s, p);
    } else {
        hipLaunchKernelGGL((skinny_kernel<NMAT, 1, WAVES, true, NORM, STRICT, FV>), dim3(p.ntiles),
                           dim3(WAVES * 64), shm, s, p);
    }
    return hipGetLastError();
}

// More tiles than CUs: 4-wave workgroups, so two fit a CU and the grid runs in
// one round (8-wave workgroups of the wide kernels fit only one per CU).
template <int NMAT, int NORM, int STRICT>
static hipError_t launch_norm_fv(const MatArgs& p, size_t shm, hipStream_t s) {
    const size_t groups = (size_t)p.e.m * (p.k / 4);
    if (p.ntiles > 256 && groups <= 4 * 256) {
        if (groups <= 2 * 256) return launch_norm_t<NMAT, NORM, STRICT, 4, 2>(p, shm, s);
        // (three slots a thread where they hold the row: the BitNet-2B
        // RMSNorm2 -> gate|up step 7.98 -> 7.68 us fast, 13.90 -> 13.37 strict)
        if (groups <= 3 * 256) return launch_norm_t<NMAT, NORM, STRICT, 4, 3>(p, shm, s);
        return launch_norm_t<NMAT, NORM, STRICT, 4, 4>(p, shm, s);
    }
    if (groups <= 2 * kNormThreads) return launch_norm_t<NMAT, NORM, STRICT, kNormWaves, 2>(p, shm, s);
    return launch_norm_t<NMAT, NORM, STRICT, kNormWaves, 4>(p, shm, s);
}

template <int NMAT, int NORM>
static hipError_t launch_norm_st(const MatArgs& p, int strict, size_t shm, hipStream_t s) {
    return strict ? launch_norm_fv<NMAT, NORM, 1>(p, shm, s) : launch_norm_fv<NMAT, NORM, 0>(p, shm, s);
}

hipError_t launch_matmul_norm(const Matrix* w0, const Matrix* w1, const float* x, const double* x64,
                              int m, int mode, int strict, const float* nw, double eps,
                              const Epilogue& epi, float* amax_tap, hipStream_t s,
                              const NormTaps* taps) {
    if (m <= 0) return hipSuccess;
    const void* rows = mode == NORM_INNER_F64 ? (const void*)x64 : (const void*)x;
    if (!rows || !norm_fused_ok(m, w0->cols, strict, ((uintptr_t)rows & 15) == 0)) {
        return hipErrorInvalidValue;
    }
    if (((uintptr_t)nw & 15) != 0) return hipErrorInvalidValue;
    MatArgs p = make_args(w0, w1, m, epi);
    p.x = x;
    p.x64 = x64;
    p.nw = nw;
    p.neps = eps;
    p.amax_tap = amax_tap;
    if (taps) {
        p.norm_tap = taps->rows;
        p.xq_tap = taps->xq;
        if (taps->amax && !amax_tap) p.amax_tap = taps->amax;
    }
    p.ldq = pad_cols(w0->cols);
    const size_t shm = norm_lds(m, w0->cols, strict);
    const bool two = epi.kind == EPI_SWIGLU;
    switch (mode) {
        case NORM_RMS:
            return two ? launch_norm_st<2, NORM_RMS>(p, strict, shm, s)
                       : launch_norm_st<1, NORM_RMS>(p, strict, shm, s);
        case NORM_INNER_F32:
            if (two) return hipErrorInvalidValue;
            return launch_norm_st<1, NORM_INNER_F32>(p, strict, shm, s);
        case NORM_INNER_F64:
            if (two) return hipErrorInvalidValue;
            return launch_norm_st<1, NORM_INNER_F64>(p, strict, shm, s);
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t launch_matmul_fused(const Matrix* w0, const Matrix* w1, const float* x, int m,
                               const Epilogue& epi, int8_t* xq_tap, float* amax_tap,
                               hipStream_t s) {
    if (m <= 0) return hipSuccess;
    if (!fused_quant_ok(m, w0->cols, x)) return hipErrorInvalidValue;
    MatArgs p = make_args(w0, w1, m, epi);
    p.x = x;
    p.ldq = pad_cols(w0->cols);
    p.xq_tap = xq_tap;
    p.amax_tap = amax_tap;
    if (epi.kind != EPI_SWIGLU && stream_ok(m, w0->cols, w0->ntiles, true, epi)) return launch_stream(p, true, s);
    return epi.kind == EPI_SWIGLU ? launch_skinny<2, 1, true>(p, s) : launch_skinny<1, 1, true>(p, s);
}

}  // namespace lamd
