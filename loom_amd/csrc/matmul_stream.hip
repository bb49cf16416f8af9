// matmul_stream.hip -- ternary GEMV for few token rows over many weight rows,
// streamed at HBM rate.
//
// The skinny kernel gives every 16-row weight tile its own workgroup, whose
// waves split K: right for a few hundred tiles (one launch's worth of
// latency), but with tens of thousands of tiles each workgroup moves only
// ~10 KiB between its launch, its barriers and its epilogue, and the memory
// system idles between workgroups.  Here a fixed grid of waves streams: wave
// w owns 16-row tiles w, w + W, w + 2W, ... (W waves in the grid) and walks
// their 1 KiB K tiles as one flat sequence through a ring of D register
// slots, reissuing each slot's load as soon as its tile is consumed, so D
// tiles are always in flight per wave.  A wave covers all of K for its rows,
// so no partial sums cross waves: when a row tile's last K tile is consumed,
// its lanes finish the 16 outputs (the shared epilogue) and the accumulators
// restart.  The quantized rows (M <= 4) sit in LDS; FUSEQ workgroups
// quantize the fp32 rows themselves first (loom's absmax + int8 rounding,
// poly/bitnet_cpu.go:45-117), once per workgroup.
#include "device_common.hpp"

namespace lamd {

constexpr int kStreamMaxRows = 4;
constexpr int kStreamWaves = 4;   // waves per workgroup
constexpr int kStreamGridWaves = 4096;  // 16 waves per CU on 256 CUs (all resident)
constexpr int kStreamDepth = 12;        // K tiles in flight per wave

template <int D, bool FUSEQ, int FV, int QV>
__global__ __launch_bounds__(kStreamWaves * 64) void stream_kernel(MatArgs p) {
    constexpr int T = kStreamWaves * 64;
    extern __shared__ __align__(16) int8_t xs[];  // M rows x ldq, then 256 zero bytes
    __shared__ float wmax[kStreamWaves][kStreamMaxRows];
    __shared__ int wsum[kStreamWaves][kStreamMaxRows];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.e.m, ktiles = p.ktiles, ntiles = p.ntiles, ldq = p.ldq;
    const int GW = gridDim.x * kStreamWaves;
    const int gw = blockIdx.x * kStreamWaves + wave;
    const int nrt = gw < ntiles ? (ntiles - 1 - gw) / GW + 1 : 0;
    const int total = nrt * ktiles;  // tiles this wave streams

    // ---- the rows: fp32 (FUSEQ) or pre-quantized int8, loads issued first
    const int k = p.k;
    const int row4 = k >> 2;
    const int n4 = FUSEQ ? M * row4 : 0;
    float4 xv[FUSEQ ? FV : 1];
    uint4 qv[FUSEQ ? 1 : QV];
    const int nq16 = FUSEQ ? 0 : M * (ldq >> 4);  // uint4 of the pre-quantized rows
    if (FUSEQ) {
        const uint32_t xb = (uint32_t)n4 * 16u;
        const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(p.x, xb);
#pragma unroll
        for (int j = 0; j < FV; ++j) {
            const int idx = tid + j * T;
            xv[j] = __builtin_bit_cast(float4, buffer_load16(xr, idx < n4 ? (uint32_t)idx * 16u : xb));
        }
    } else {
        // rows are ldq bytes apart in global memory (as in LDS)
        const uint32_t qb = (uint32_t)nq16 * 16u;
        const __amdgpu_buffer_rsrc_t qr = buffer_rsrc(p.xq, qb);
#pragma unroll
        for (int j = 0; j < QV; ++j) {
            const int idx = tid + j * T;
            qv[j] = buffer_load16(qr, idx < nq16 ? (uint32_t)idx * 16u : qb);
        }
    }
    float am_tok[kStreamMaxRows];
    int xs_tok[kStreamMaxRows];
    if (!FUSEQ) {
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t) {
            am_tok[t] = t < M ? p.e.amax[t] : 1.0f;
            xs_tok[t] = t < M ? p.e.xsum[t] : 0;
        }
    }

    // ---- the first D weight tiles
    const uint32_t wbytes = (uint32_t)ntiles * (uint32_t)ktiles * 1024u;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(p.w0, wbytes);
    int lrt = gw, lkt = 0, lf = 0;  // load cursor: row tile, K tile, flat index
    auto next_off = [&]() -> uint32_t {
        const uint32_t o = lf < total ? ((uint32_t)(lrt * ktiles + lkt) * 64u + (uint32_t)lane) * 16u
                                      : wbytes;  // past the end: zero, no traffic
        // (lrt stays below ntiles while lf < total, so the offset fits 32 bits)
        ++lf;
        if (++lkt == ktiles) {
            lkt = 0;
            lrt += GW;
        }
        return o;
    };
    uint4 buf[D];
#pragma unroll
    for (int j = 0; j < D; ++j) buf[j] = buffer_load16_nt(wr, next_off());

    // ---- quantized rows into LDS (+ 256 zero bytes read by the rows past M)
    if (FUSEQ) {
        float lm[kStreamMaxRows];
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t) lm[t] = 0.0f;
#pragma unroll
        for (int j = 0; j < FV; ++j) {
            const int idx = tid + j * T;
            if (idx < n4) {
                float a = max_nan_skip(0.0f, fabsf(xv[j].x));
                a = max_nan_skip(a, fabsf(xv[j].y));
                a = max_nan_skip(a, fabsf(xv[j].z));
                a = max_nan_skip(a, fabsf(xv[j].w));
                const int row = idx / row4;
#pragma unroll
                for (int t = 0; t < kStreamMaxRows; ++t)
                    if (t == row) lm[t] = max_nan_skip(lm[t], a);
            }
        }
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t) {
            if (t < M) {
                const float wm = wave_max_dpp(lm[t]);
                if (lane == 0) wmax[wave][t] = wm;
            }
        }
        __syncthreads();
        double sc[kStreamMaxRows];
        float sc32[kStreamMaxRows];
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t) {
            float am = 0.0f;
            if (t < M)
                for (int w = 0; w < kStreamWaves; ++w) am = max_nan_skip(am, wmax[w][t]);
            if (am < 1e-5f) am = 1e-5f;
            am_tok[t] = am;
            sc[t] = 127.0 / (double)am;
            sc32[t] = (float)sc[t];
        }
        int ls[kStreamMaxRows];
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t) ls[t] = 0;
#pragma unroll
        for (int j = 0; j < FV; ++j) {
            const int idx = tid + j * T;
            if (idx < n4) {
                const int row = idx / row4;
                double s = sc[0];
                float s32 = sc32[0];
#pragma unroll
                for (int t = 1; t < kStreamMaxRows; ++t)
                    if (t == row) {
                        s = sc[t];
                        s32 = sc32[t];
                    }
                const int q0 = quant_f32(xv[j].x, s32, s), q1 = quant_f32(xv[j].y, s32, s);
                const int q2 = quant_f32(xv[j].z, s32, s), q3 = quant_f32(xv[j].w, s32, s);
                *(uint32_t*)(xs + row * ldq + 4 * (idx - row * row4)) = pack4(q0, q1, q2, q3);
#pragma unroll
                for (int t = 0; t < kStreamMaxRows; ++t)
                    if (t == row) ls[t] += q0 + q1 + q2 + q3;
            }
        }
        const int pad4 = (ldq - k) >> 2;
        for (int i = tid; i < M * pad4; i += T) {
            const int row = i / pad4;
            *(uint32_t*)(xs + row * ldq + k + 4 * (i - row * pad4)) = 0u;
        }
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t) {
            if (t < M) {
                const int v = wave_sum_i_dpp(ls[t]);
                if (lane == 0) wsum[wave][t] = v;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < QV; ++j) {
            const int idx = tid + j * T;
            if (idx < nq16) *(uint4*)(xs + (size_t)idx * 16) = qv[j];
        }
    }
    if (tid < 64) *(uint32_t*)(xs + M * ldq + 4 * tid) = 0u;
    __syncthreads();
    if (FUSEQ) {
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t) {
            int s = 0;
            if (t < M)
                for (int w = 0; w < kStreamWaves; ++w) s += wsum[w][t];
            xs_tok[t] = s;
        }
        if (blockIdx.x == 0 && p.amax_tap) {
#pragma unroll
            for (int t = 0; t < kStreamMaxRows; ++t)
                if (tid == t && t < M) p.amax_tap[t] = am_tok[t];
        }
        if (blockIdx.x == 0 && p.xq_tap) {
            for (int i = tid; i < M * k; i += T) p.xq_tap[i] = xs[(i / k) * ldq + (i % k)];
        }
    }
    // epilogue constants of this lane's tokens (4g + v)
    RowScale rs[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int tok = 4 * g + v;
        float am = 1.0f;
        int xsum = 0;
#pragma unroll
        for (int t = 0; t < kStreamMaxRows; ++t)
            if (t == tok) {
                am = am_tok[t];
                xsum = xs_tok[t];
            }
        rs[v] = row_scale(p.e, am, xsum);
    }

    // ---- stream: consume slot j, reissue it D tiles ahead.  A finished row
    // tile parks its accumulators in pend0/pend1 (at most two finish within
    // D tiles while K spans >= D/2 tiles) and its outputs are stored after
    // the unrolled group, which keeps the epilogue out of the unrolled code.
    const int8_t* arow = xs + (r < M ? r * ldq + 16 * g : M * ldq + 16 * g);
    const int astep = r < M ? 256 : 0;  // rows past M read the zero bytes
    v4i acc = v4i{0, 0, 0, 0}, pend0 = acc, pend1 = acc;
    int ckt = 0, crt = gw;
    // The two epilogues with no loads (a load in the epilogue would make the
    // wait counters drain the ring): loom's fp32 output
    // fp32(fp64(acc) * output scale), or the int32 accumulators.
    auto finish = [&](const v4i& a, int rt) {
        const int n = rt * kTileRows + r;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int tok = 4 * g + v;
            if (tok < M && n < p.e.n) {
                const int acc0 = a[v] - rs[v].xs;
                if (p.e.kind == EPI_ACC) {
                    p.e.acc0[(size_t)tok * p.e.n + n] = acc0;
                } else {
                    p.e.out[(size_t)tok * p.e.ldo + n] = (float)((double)acc0 * rs[v].os0);
                }
            }
        }
    };
    // Branch-free steps (a branch around a load makes the wait counters fall
    // back to waiting for every load): the step count is padded to a multiple
    // of D; padded steps read past the end (zeros, no traffic) and belong to
    // row tiles past the last one, which store nothing.
    for (int f0 = 0; f0 < total; f0 += D) {
        int npend = 0, pr0 = 0, pr1 = 0;
#pragma unroll
        for (int j = 0; j < D; ++j) {
            // the slot's load is reissued after its MFMAs read it, so the new
            // load lands in the same registers (no copy at the loop's back
            // edge, which would wait for every load in flight)
            const int8_t* ap = arow + ckt * astep;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const v4i a = *(const v4i*)(ap + 64 * t);
                acc = mfma_i8(a, unpack_codes(word_of(buf[j], t)), acc);
            }
            buf[j] = buffer_load16_nt(wr, next_off());
            if (++ckt == ktiles) {
                if (npend == 0) {
                    pend0 = acc;
                    pr0 = crt;
                } else {
                    pend1 = acc;
                    pr1 = crt;
                }
                ++npend;
                acc = v4i{0, 0, 0, 0};
                ckt = 0;
                crt += GW;
            }
        }
        if (npend > 0) finish(pend0, pr0);
        if (npend > 1) finish(pend1, pr1);
    }
}

// Whether the streaming kernel takes m rows of width k over n_tiles 16-row
// tiles: one matrix with the plain Dense epilogue (no bias, residual,
// activation or accumulator tap) or the accumulators only, m <= 4, the rows'
// int8 copies in LDS (pre-quantized: at most 16 KiB; fused: at most 16 float4
// per thread).
// LOOM_AMD_GEMV_STREAM = 0 / 1 forces the choice (tests take both).
bool stream_ok(int m, int k, int n_tiles, bool fused, const Epilogue& epi) {
    const bool plain = epi.kind == EPI_DENSE && !epi.bias0 && !epi.residual && !epi.post && !epi.acc0;
    const bool acc_only = epi.kind == EPI_ACC && epi.acc0;
    if (!plain && !acc_only) return false;
    const int force = tune_int("LOOM_AMD_GEMV_STREAM", -1);
    if (m < 1 || m > kStreamMaxRows || k % 4 != 0) return false;
    if (ceil_div(k, kTileCols) * 2 < kStreamDepth) return false;  // <= 2 row tiles end per group
    if ((size_t)m * pad_cols(k) > (fused ? (size_t)60 * 1024 - 256 : (size_t)16 * 1024)) return false;
    if (fused && (size_t)m * k > (size_t)16 * 4 * kStreamWaves * 64) return false;
    if (force == 0) return false;
    if (force == 1) return true;
    return n_tiles >= 2 * kStreamGridWaves;
}

// Tuning overrides: LOOM_AMD_STREAM_WAVES (waves in the grid) and
// LOOM_AMD_STREAM_DEPTH (K tiles in flight per wave: 8, 12 or 16).
template <bool FUSEQ, int FV, int QV>
static void launch_stream_t(const MatArgs& p, int grid, size_t shm, hipStream_t s) {
    const int depth = tune_int("LOOM_AMD_STREAM_DEPTH", kStreamDepth);
    const dim3 g(grid), b(kStreamWaves * 64);
    if (depth == 8 && p.ktiles * 2 >= 8) {
        hipLaunchKernelGGL((stream_kernel<8, FUSEQ, FV, QV>), g, b, shm, s, p);
    } else if (depth == 16 && p.ktiles * 2 >= 16) {
        hipLaunchKernelGGL((stream_kernel<16, FUSEQ, FV, QV>), g, b, shm, s, p);
    } else {
        hipLaunchKernelGGL((stream_kernel<kStreamDepth, FUSEQ, FV, QV>), g, b, shm, s, p);
    }
}

hipError_t launch_stream(const MatArgs& p, bool fuseq, hipStream_t s) {
    const int gw = tune_int("LOOM_AMD_STREAM_WAVES", kStreamGridWaves);
    const int cap = gw >= kStreamWaves ? gw : kStreamGridWaves;
    const int waves = p.ntiles < cap ? p.ntiles : cap;
    const int grid = (waves + kStreamWaves - 1) / kStreamWaves;
    const size_t shm = (size_t)p.e.m * p.ldq + 256;
    if (!fuseq) {
        const int nq16 = p.e.m * (p.ldq >> 4);
        constexpr int T = kStreamWaves * 64;
        if (nq16 <= T) {
            launch_stream_t<false, 1, 1>(p, grid, shm, s);
        } else if (nq16 <= 2 * T) {
            launch_stream_t<false, 1, 2>(p, grid, shm, s);
        } else if (nq16 <= 4 * T) {
            launch_stream_t<false, 1, 4>(p, grid, shm, s);
        } else {
            return hipErrorInvalidValue;
        }
    } else {
        const size_t groups = (size_t)p.e.m * (p.k / 4);
        constexpr int T = kStreamWaves * 64;
        if (groups <= 4 * T) {
            launch_stream_t<true, 4, 1>(p, grid, shm, s);
        } else if (groups <= 8 * T) {
            launch_stream_t<true, 8, 1>(p, grid, shm, s);
        } else if (groups <= 16 * T) {
            launch_stream_t<true, 16, 1>(p, grid, shm, s);
        } else {
            return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

}  // namespace lamd
