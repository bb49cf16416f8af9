// quant_norm.hip -- weight repack, activation quantization and the SwiGLU
// inner RMSNorm + requantization (gfx950).
#include <type_traits>

#include "device_common.hpp"

namespace lamd {

// ------------------------------------------------------------------------
// repack: loom row-major Words (poly/bitnet_cpu.go:14-43) -> tile layout
// ------------------------------------------------------------------------

__global__ void repack_tiles_kernel(const uint32_t* __restrict__ words, int rows, int cols,
                                    int row_words, int ktiles, long total,
                                    uint32_t* __restrict__ out) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int t = (int)(idx & 3);
    const int lane = (int)((idx >> 2) & 63);
    const long tile = idx >> 8;
    const int kt = (int)(tile % ktiles);
    const int nt = (int)(tile / ktiles);
    const int n = nt * kTileRows + (lane & 15);
    const int k0 = kt * kTileCols + t * 64 + (lane >> 4) * 16;
    uint32_t src = 0;
    if (n < rows && k0 < cols) {
        src = words[(long)n * row_words + (k0 >> 4)];
        const int valid = cols - k0;
        if (valid < 16) src &= (1u << (2 * valid)) - 1u;
    }
    uint32_t o = 0;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const uint32_t code = (src >> (2 * c)) & 3u;
        o |= code << (8 * (c & 3) + 2 * (c >> 2));
    }
    out[idx] = o;
}

// packMicrosoftOfflineBitNetRowsToU32FromBytes (poly/bitnet_cpu.go:1078-1098):
// byte (pr, c) of the (rows/4) x cols offline matrix holds the 2-bit codes of
// column c for rows lane*(rows/4) + pr, lane = 0..3 (bits 2*lane); code 3
// becomes 1 (a zero weight).  Rows past 4*(rows/4) keep all-zero words.  One
// thread per output word of loom's row-major layout (16 codes per word).
__global__ void ms_offline_to_words_kernel(const uint8_t* __restrict__ packed, int rows, int cols,
                                           int row_words, uint32_t* __restrict__ words) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)rows * row_words) return;
    const int row = (int)(idx / row_words);
    const int w = (int)(idx % row_words);
    const int prs = rows / 4;
    uint32_t word = 0;
    if (prs > 0 && row < 4 * prs) {
        const int lane = row / prs, pr = row % prs;
        const uint8_t* src = packed + (size_t)pr * cols;
        for (int j = 0; j < 16; ++j) {
            const int c = w * 16 + j;
            if (c >= cols) break;
            uint32_t code = (src[c] >> (2 * lane)) & 3u;
            if (code > 2) code = 1;
            word |= code << (2 * j);
        }
    }
    words[idx] = word;
}

hipError_t launch_ms_offline_to_words(const uint8_t* packed, int rows, int cols, uint32_t* words,
                                      hipStream_t s) {
    const int row_words = ceil_div(cols, 16);
    const long total = (long)rows * row_words;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(ms_offline_to_words_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       s, packed, rows, cols, row_words, words);
    return hipGetLastError();
}

hipError_t launch_repack(const uint32_t* words, int rows, int cols, int row_words, Matrix* m,
                         hipStream_t s) {
    const long total = (long)m->ntiles * m->ktiles * kTileWords;
    if (total == 0) return hipSuccess;
    const int threads = 256;
    const long blocks = (total + threads - 1) / threads;
    hipLaunchKernelGGL(repack_tiles_kernel, dim3((unsigned)blocks), dim3(threads), 0, s, words,
                       rows, cols, row_words, m->ktiles, total, m->tiles);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// activation quantization (poly/bitnet_cpu.go:45-117): one workgroup of 256
// threads per token row; every load of the row is issued before the max.
// VPT = values per thread held in registers (k <= 256*VPT); VPT 0 = loop.
// ------------------------------------------------------------------------

template <typename T, int VPT>
__global__ __launch_bounds__(256) void act_quant_kernel(const T* __restrict__ x, int ldx, int k,
                                                        int ldq, int8_t* __restrict__ xq,
                                                        float* __restrict__ amax_out,
                                                        int32_t* __restrict__ xsum_out) {
    __shared__ float shf[4];
    __shared__ int shi[4];
    const int row = blockIdx.x;
    const T* xr = x + (size_t)row * ldx;
    int8_t* qr = xq + (size_t)row * ldq;
    float m = 0.0f;
    int s = 0;
    if (VPT > 0) {
        T v[VPT > 0 ? VPT : 1];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = threadIdx.x + j * 256;
            v[j] = i < k ? xr[i] : (T)0;
        }
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            // float32(|float64(v)|): exact for fp32 input, one rounding for fp64.
            if (threadIdx.x + j * 256 < k) m = max_nan_skip(m, (float)fabs((double)v[j]));
        }
        m = block_max(m, shf);
        if (m < 1e-5f) m = 1e-5f;
        const double scale = 127.0 / (double)m;
        const float scale32 = (float)scale;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = threadIdx.x + j * 256;
            if (i < k) {
                const int q = sizeof(T) == 4 ? quant_f32((float)v[j], scale32, scale)
                                             : quant_one((double)v[j], scale);
                s += q;
                qr[i] = (int8_t)q;
            }
        }
    } else {
        for (int i = threadIdx.x; i < k; i += 256) m = max_nan_skip(m, (float)fabs((double)xr[i]));
        m = block_max(m, shf);
        if (m < 1e-5f) m = 1e-5f;
        const double scale = 127.0 / (double)m;
        for (int i = threadIdx.x; i < k; i += 256) {
            const int q = quant_one((double)xr[i], scale);
            s += q;
            qr[i] = (int8_t)q;
        }
    }
    for (int i = k + threadIdx.x; i < ldq; i += 256) qr[i] = 0;
    s = block_sum_i(s, shi);
    if (threadIdx.x == 0) {
        amax_out[row] = m;
        xsum_out[row] = s;
    }
}

// fp32 rows, 16-byte groups: thread t holds element groups t + 256 j (G4 a
// thread, k <= 1024 G4), 16-byte loads and one 32-bit store of four codes.
// The maximum is taken on |x| bit patterns (unsigned order is value order for
// non-negative floats, and NaN sorts above infinity, so it also flags a row
// holding NaN or infinity: such a row takes loom's NaN-skipping maximum and
// per-value rounding).  Finite rows round in fp32 with sf = fl32(127 / m),
// within 2^-24 + 2^-53 of loom's fp64 scale, so a value's fp32 product is
// within 127 (2^-23 + 2^-47) < 1.52e-5 of loom's fp64 one: one test
// 0.5f - |p - r| > 3.1e-5f per group of four (on their largest |p - r|)
// decides them, and only the undecided groups take quant_f32.  |x| <= m, so
// |p| < 127.5 and rintf needs no clamp.
template <int G4>
__global__ __launch_bounds__(256) void act_quant_rows_kernel(const float* __restrict__ x, int ldx, int k,
                                                             int ldq, int8_t* __restrict__ xq,
                                                             float* __restrict__ amax_out,
                                                             int32_t* __restrict__ xsum_out) {
    __shared__ unsigned shu[4];
    __shared__ float shf[4];
    __shared__ int shi[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k4 = k >> 2;
    const float4* xr = (const float4*)(x + (size_t)row * ldx);
    float4 v[G4];
#pragma unroll
    for (int j = 0; j < G4; ++j) {
        const int g = tid + 256 * j;
        v[j] = g < k4 ? xr[g] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    unsigned lb = 0u;
#pragma unroll
    for (int j = 0; j < G4; ++j)
        lb = max(lb, max(max(__float_as_uint(v[j].x) & 0x7fffffffu, __float_as_uint(v[j].y) & 0x7fffffffu),
                         max(__float_as_uint(v[j].z) & 0x7fffffffu, __float_as_uint(v[j].w) & 0x7fffffffu)));
    lb = wave_umax_dpp(lb);
    if (lane == 0) shu[wave] = lb;
    __syncthreads();
    unsigned mb = max(max(shu[0], shu[1]), max(shu[2], shu[3]));
    const bool gen = mb > 0x7f7fffffu;  // NaN or infinity in the row (uniform)
    float m = __uint_as_float(mb);
    if (gen) {
        float lm = 0.0f;
#pragma unroll
        for (int j = 0; j < G4; ++j) {
            lm = max_nan_skip(lm, fabsf(v[j].x));
            lm = max_nan_skip(lm, fabsf(v[j].y));
            lm = max_nan_skip(lm, fabsf(v[j].z));
            lm = max_nan_skip(lm, fabsf(v[j].w));
        }
        m = block_max(lm, shf);
    }
    if (m < 1e-5f) m = 1e-5f;
    uint32_t pk[G4];
    bool undecided[G4];
    bool any = gen;
#pragma unroll
    for (int j = 0; j < G4; ++j) {
        pk[j] = 0u;
        undecided[j] = gen;
    }
    if (!gen) {
        const float sf = 127.0f / m;  // (fp32 division, correctly rounded)
#pragma unroll
        for (int j = 0; j < G4; ++j) {
            const float p0 = v[j].x * sf, p1 = v[j].y * sf, p2 = v[j].z * sf, p3 = v[j].w * sf;
            const float r0 = rintf(p0), r1 = rintf(p1), r2 = rintf(p2), r3 = rintf(p3);
            const float d = fmaxf(fmaxf(fabsf(p0 - r0), fabsf(p1 - r1)), fmaxf(fabsf(p2 - r2), fabsf(p3 - r3)));
            undecided[j] = !(0.5f - d > 3.1e-5f);
            any |= undecided[j];
            pk[j] = pack4((int)r0, (int)r1, (int)r2, (int)r3);
        }
    }
    if (any) {  // (per thread) loom's fp64 rounding for the undecided groups
        const double scale = 127.0 / (double)m;
        const float scale32 = (float)scale;
#pragma unroll
        for (int j = 0; j < G4; ++j) {
            if (undecided[j])
                pk[j] = pack4(quant_f32(v[j].x, scale32, scale), quant_f32(v[j].y, scale32, scale),
                              quant_f32(v[j].z, scale32, scale), quant_f32(v[j].w, scale32, scale));
        }
    }
    uint32_t* qr = (uint32_t*)(xq + (size_t)row * ldq);
    int sum = 0;
#pragma unroll
    for (int j = 0; j < G4; ++j) {
        const int g = tid + 256 * j;
        if (g < k4) {
            qr[g] = pk[j];
            sum = byte_sum_i8(pk[j], sum);
        }
    }
    for (int g = k4 + tid; g < (ldq >> 2); g += 256) qr[g] = 0u;  // padding columns
    sum = block_sum_i(sum, shi);
    if (tid == 0) {
        amax_out[row] = m;
        xsum_out[row] = sum;
    }
}

template <typename T>
static hipError_t launch_quant_t(const T* x, int ldx, int m, int k, int8_t* xq, int ldq,
                                 float* amax, int32_t* xsum, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    const dim3 g(m), b(256);
    if constexpr (sizeof(T) == 4) {
        // 16-byte rows: the group kernel (measured against act_quant_kernel at
        // the BitNet-2B up shape; its tiers follow the float4 slots a thread)
        const bool v16 = k % 4 == 0 && ldx % 4 == 0 && ldq % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
                         ((uintptr_t)xq & 3) == 0;
        if (v16 && tune_int("LOOM_AMD_QUANT_GROUPS", 1) != 0) {
            if (k <= 1024 * 2) {
                hipLaunchKernelGGL((act_quant_rows_kernel<2>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
                return hipGetLastError();
            }
            if (k <= 1024 * 3) {
                hipLaunchKernelGGL((act_quant_rows_kernel<3>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
                return hipGetLastError();
            }
            if (k <= 1024 * 4) {
                hipLaunchKernelGGL((act_quant_rows_kernel<4>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
                return hipGetLastError();
            }
            if (k <= 1024 * 8) {
                hipLaunchKernelGGL((act_quant_rows_kernel<8>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
                return hipGetLastError();
            }
        }
    }
    if (k <= 256 * 4) {
        hipLaunchKernelGGL((act_quant_kernel<T, 4>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
    } else if (k <= 256 * 8) {
        hipLaunchKernelGGL((act_quant_kernel<T, 8>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
    } else if (k <= 256 * 16) {
        hipLaunchKernelGGL((act_quant_kernel<T, 16>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
    } else if (k <= 256 * 32) {
        hipLaunchKernelGGL((act_quant_kernel<T, 32>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
    } else {
        hipLaunchKernelGGL((act_quant_kernel<T, 0>), g, b, 0, s, x, ldx, k, ldq, xq, amax, xsum);
    }
    return hipGetLastError();
}

hipError_t launch_act_quant(const float* x, int ldx, int m, int k, int8_t* xq, int ldq,
                            float* amax, int32_t* xsum, hipStream_t s) {
    return launch_quant_t<float>(x, ldx, m, k, xq, ldq, amax, xsum, s);
}

hipError_t launch_act_quant_f64(const double* x, int ldx, int m, int k, int8_t* xq, int ldq,
                                float* amax, int32_t* xsum, hipStream_t s) {
    return launch_quant_t<double>(x, ldx, m, k, xq, ldq, amax, xsum, s);
}

// ------------------------------------------------------------------------
// SwiGLU inner RMSNorm + requantization (poly/bitnet_cpu.go:893-913, then
// poly/bitnet_cpu.go:97-106), one 256-thread workgroup per row, in place.
//
// strict: the sum of squares is loom's sequential fp64 chain in column
//   order.  The squares f*f are exact in fp64 (24-bit x 24-bit significands),
//   so all threads form them in parallel into LDS and one lane performs only
//   the ordered additions.
// fast:  thread t sums columns t, t+256, ... then a fixed binary tree; the
//   result is deterministic but rounds differently from the chain, which moves
//   normalized values by at most one fp32 ulp.
// VPT = values per thread in registers (n <= 256*VPT).
// ------------------------------------------------------------------------

template <int STRICT, int VPT>
__global__ __launch_bounds__(256) void norm_quant_kernel(float* __restrict__ h, int ldh, int n,
                                                         const float* __restrict__ weight,
                                                         double eps, int8_t* __restrict__ hq,
                                                         int ldq, float* __restrict__ amax_out,
                                                         int32_t* __restrict__ xsum_out, int keep,
                                                         const double* __restrict__ totals) {
    extern __shared__ double dsh[];  // STRICT: n squares; fast: 256 partial sums
    __shared__ float shf[4];
    __shared__ int shi[4];
    __shared__ double total;
    const int row = blockIdx.x;
    float* hr = h + (size_t)row * ldh;
    float v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        v[j] = i < n ? hr[i] : 0.0f;
    }
    if (STRICT && totals) {
        if (threadIdx.x == 0) total = totals[row];  // the row-chain kernel's ordered sum
        __syncthreads();
    } else if (STRICT) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = threadIdx.x + j * 256;
            if (i < n) {
                const double f = (double)v[j];
                dsh[i] = f * f;
            }
        }
        __syncthreads();
        __shared__ OrderedSumLds<4> osum;
        const double r = ordered_sum_block<4>(dsh, n, 0.0, osum);
        if (threadIdx.x == 0) total = r;
        __syncthreads();
    } else {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const double f = (double)v[j];  // zero past n
            s += f * f;
        }
        // fixed tree: element t adds element t + w for w = 128, 64, ..., 1;
        // the levels below 64 run as lane moves inside wave 0 (same pairs)
        dsh[threadIdx.x] = s;
        __syncthreads();
        if (threadIdx.x < 128) dsh[threadIdx.x] = dsh[threadIdx.x] + dsh[threadIdx.x + 128];
        __syncthreads();
        if (threadIdx.x < 64) {
            double t = dsh[threadIdx.x] + dsh[threadIdx.x + 64];
#pragma unroll
            for (int width = 32; width > 0; width >>= 1) t = t + __shfl_down(t, width, 64);
            if (threadIdx.x == 0) total = t;
        }
        __syncthreads();
    }

    const double scale = 1.0 / sqrt(total / (double)n + eps);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        if (i < n) {
            const double w = weight ? (double)weight[i] : 1.0;
            v[j] = (float)((double)v[j] * scale * w);
            if (keep) hr[i] = v[j];
            m = max_nan_skip(m, fabsf(v[j]));
        }
    }
    m = block_max(m, shf);
    if (m < 1e-5f) m = 1e-5f;
    const double qs = 127.0 / (double)m;
    const float qs32 = (float)qs;
    int s = 0;
    int8_t* qr = hq + (size_t)row * ldq;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        if (i < n) {
            const int q = quant_f32(v[j], qs32, qs);
            s += q;
            qr[i] = (int8_t)q;
        }
    }
    for (int i = n + threadIdx.x; i < ldq; i += 256) qr[i] = 0;
    s = block_sum_i(s, shi);
    if (threadIdx.x == 0) {
        amax_out[row] = m;
        xsum_out[row] = s;
    }
}

// ------------------------------------------------------------------------
// Row norm + requantization, one wave per row (many rows: prefill).  Lane l
// holds columns 256 j + 4 l .. + 3 (16-byte loads and stores, the four int8
// codes as one 32-bit store), i.e. the values of threads 4 l .. 4 l + 3 of
// the one-workgroup-per-row kernels.  Fast mode keeps their tree: each of
// the four partial sums runs over j in order, then the pairs (t, t + w) for
// w = 128 .. 4 are lanes (l, l + w/4) and w = 2, 1 the lane's own partials,
// so the sum is the same bits with no barrier.  The maximum and the code sum
// are order-free.
// ------------------------------------------------------------------------

template <int KIND, int STRICT, int NB>
__global__ __launch_bounds__(256) void row_norm_wave_kernel(RowNormArgs a) {
    using T = typename std::conditional<KIND == kRowInnerF64, double, float>::type;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.m) return;  // wave-uniform
    const int n = a.n;
    const T* xr = (const T*)a.x + (size_t)row * a.ldx;
    T v[NB][4];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int c = 256 * j + 4 * lane;
        if (c < n) {
            if constexpr (KIND == kRowInnerF64) {
                const double2 p0 = *(const double2*)(xr + c), p1 = *(const double2*)(xr + c + 2);
                v[j][0] = p0.x;
                v[j][1] = p0.y;
                v[j][2] = p1.x;
                v[j][3] = p1.y;
            } else {
                const float4 p0 = *(const float4*)(xr + c);
                v[j][0] = p0.x;
                v[j][1] = p0.y;
                v[j][2] = p0.z;
                v[j][3] = p0.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[j][i] = (T)0;
        }
    }
    double total;
    if (STRICT) {
        total = a.totals[row];
    } else {
        double p[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const double f = (double)v[j][i];
                p[i] = p[i] + f * f;
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = p[i] + __shfl_down(p[i], off, 64);
        total = __shfl((p[0] + p[2]) + (p[1] + p[3]), 0, 64);
        // the values again as they were loaded: without this the compiler
        // keeps their fp64 conversions from the sum live for the scaling
        // below, twice the registers (one wave per SIMD at n = 6912)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) __asm__ volatile("" : "+v"(v[j][i]));
    }
    double rms = 0.0, scale = 0.0;
    if (KIND == kRowRms)
        rms = sqrt(total / (double)n + a.eps);
    else
        scale = 1.0 / sqrt(total / (double)n + a.eps);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int c = 256 * j + 4 * lane;
        if (c < n) {
            float4 w4 = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            if (a.w) w4 = *(const float4*)(a.w + c);
            const float wf[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (KIND == kRowRms) {
                    const double normed = (double)v[j][i] / rms;
                    v[j][i] = (float)(normed * (double)wf[i]);
                    m = max_nan_skip(m, fabsf((float)v[j][i]));
                } else if constexpr (KIND == kRowInner) {
                    const double w = a.w ? (double)wf[i] : 1.0;
                    v[j][i] = (float)((double)v[j][i] * scale * w);
                    m = max_nan_skip(m, fabsf((float)v[j][i]));
                } else {
                    const double w = a.w ? (double)wf[i] : 1.0;
                    v[j][i] = v[j][i] * (scale * w);
                    m = max_nan_skip(m, (float)fabs((double)v[j][i]));
                }
            }
            if constexpr (KIND == kRowRms) {
                if (a.yf) *(float4*)(a.yf + (size_t)row * n + c) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
            } else if constexpr (KIND == kRowInner) {
                if (a.yf) *(float4*)(a.yf + (size_t)row * a.ldx + c) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
            } else {
                if (a.keep64) {
                    double* kr = a.keep64 + (size_t)row * a.ldx + c;
                    *(double2*)kr = make_double2(v[j][0], v[j][1]);
                    *(double2*)(kr + 2) = make_double2(v[j][2], v[j][3]);
                }
                if (a.yf)
                    *(float4*)(a.yf + (size_t)row * n + c) =
                        make_float4((float)v[j][0], (float)v[j][1], (float)v[j][2], (float)v[j][3]);
            }
        }
    }
    m = wave_max(m);
    if (m < 1e-5f) m = 1e-5f;
    const double qs = 127.0 / (double)m;
    const float qs32 = (float)qs;
    int sum = 0;
    int8_t* qr = a.xq + (size_t)row * a.ldq;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int c = 256 * j + 4 * lane;
        if (c < a.ldq) {
            int q[4] = {0, 0, 0, 0};
            if (c < n) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (KIND == kRowInnerF64)
                        q[i] = quant_one(v[j][i], qs);
                    else
                        q[i] = quant_f32(v[j][i], qs32, qs);
                    sum += q[i];
                }
            }
            *(uint32_t*)(qr + c) = pack4(q[0], q[1], q[2], q[3]);
        }
    }
    for (int c = 256 * NB + 4 * lane; c < a.ldq; c += 256) *(uint32_t*)(qr + c) = 0u;
    sum = wave_sum_i(sum);
    if (lane == 0) {
        a.amax[row] = m;
        a.xsum[row] = sum;
    }
}

constexpr int kRowWaveMinRows = 1024;

// The kernel instance for nb 256-column blocks: NB of 8, 12, 16, 28 or 32
// (fp64 rows up to 16, the register budget).
template <int KIND, int STRICT>
static void launch_row_norm_nb(int nb, const RowNormArgs& a, hipStream_t s) {
    const dim3 g((a.m + 3) / 4), b(256);
    if (nb <= 8) {
        hipLaunchKernelGGL((row_norm_wave_kernel<KIND, STRICT, 8>), g, b, 0, s, a);
    } else if (nb <= 12) {
        hipLaunchKernelGGL((row_norm_wave_kernel<KIND, STRICT, 12>), g, b, 0, s, a);
    } else if (nb <= 16 || KIND == kRowInnerF64) {
        hipLaunchKernelGGL((row_norm_wave_kernel<KIND, STRICT, 16>), g, b, 0, s, a);
    } else if constexpr (KIND != kRowInnerF64) {
        if (nb <= 28) {
            hipLaunchKernelGGL((row_norm_wave_kernel<KIND, STRICT, 28>), g, b, 0, s, a);
        } else {
            hipLaunchKernelGGL((row_norm_wave_kernel<KIND, STRICT, 32>), g, b, 0, s, a);
        }
    }
}

template <int KIND>
static void launch_row_norm_kind(int strict, int nb, const RowNormArgs& a, hipStream_t s) {
    if (strict)
        launch_row_norm_nb<KIND, 1>(nb, a, s);
    else
        launch_row_norm_nb<KIND, 0>(nb, a, s);
}

bool launch_row_norm_wave(int kind, int strict, const RowNormArgs& a, hipStream_t s, hipError_t* e) {
    if (tune_int("LOOM_AMD_ROWNORM_WAVE", 1) == 0) return false;
    // fewer rows leave too few waves to cover a row's load latency (512 rows
    // of 6912: 20 us against 14 us for the workgroup kernel; 2048 rows: 30
    // against 37 us)
    if (a.m < kRowWaveMinRows || a.n <= 0 || a.n % 4 != 0 || a.ldq % 4 != 0 || a.ldq < a.n) return false;
    if (strict && !a.totals) return false;
    const size_t es = kind == kRowInnerF64 ? 8 : 4;
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(a.x) || ((size_t)a.ldx * es) % 16 != 0 || !al16(a.w) || !al16(a.yf) || !al16(a.keep64) ||
        ((uintptr_t)a.xq & 3) != 0)
        return false;
    const int nb = (a.n + 255) / 256;
    if (nb > (kind == kRowInnerF64 ? 16 : 32)) return false;
    if (kind == kRowRms)
        launch_row_norm_kind<kRowRms>(strict, nb, a, s);
    else if (kind == kRowInner)
        launch_row_norm_kind<kRowInner>(strict, nb, a, s);
    else
        launch_row_norm_kind<kRowInnerF64>(strict, nb, a, s);
    *e = hipGetLastError();
    return true;
}

template <int STRICT>
static hipError_t launch_norm_t(float* h, int ldh, int m, int n, const float* weight, double eps,
                                int8_t* hq, int ldq, float* amax, int32_t* xsum, int keep,
                                const double* totals, hipStream_t s) {
    {
        const RowNormArgs a{h, ldh, m, n, weight, eps, keep ? h : nullptr, nullptr, hq, ldq, amax, xsum, totals};
        hipError_t e = hipSuccess;
        if (launch_row_norm_wave(kRowInner, STRICT, a, s, &e)) return e;
    }
    const size_t shm = STRICT && !totals ? (size_t)ordered_sum_slots(n, 4) * sizeof(double)
                                         : 256 * sizeof(double);
    const dim3 g(m), b(256);
#define LAMD_NQ(VPT)                                                                            \
    hipLaunchKernelGGL((norm_quant_kernel<STRICT, VPT>), g, b, shm, s, h, ldh, n, weight, eps, hq, ldq, \
                       amax, xsum, keep, totals)
    if (n <= 256 * 8) {
        LAMD_NQ(8);
    } else if (n <= 256 * 16) {
        LAMD_NQ(16);
    } else if (n <= 256 * 32) {
        LAMD_NQ(32);
    } else {
        return hipErrorInvalidValue;
    }
#undef LAMD_NQ
    return hipGetLastError();
}

hipError_t launch_norm_quant(float* h, int ldh, int m, int n, const float* weight, double eps,
                             int strict, int8_t* hq, int ldq, float* amax, int32_t* xsum,
                             hipStream_t s, bool keep_rows, double* totals) {
    if (m <= 0) return hipSuccess;
    if (eps <= 0.0) eps = 1e-5;
    if (n > kMaxNormCols) return hipErrorInvalidValue;
    const int keep = keep_rows ? 1 : 0;
    if (!strict) return launch_norm_t<0>(h, ldh, m, n, weight, eps, hq, ldq, amax, xsum, keep, nullptr, s);
    hipError_t e = hipSuccess;
    const bool rows = launch_row_sumsq_f32(h, ldh, m, n, totals, s, &e);
    if (e != hipSuccess) return e;
    return launch_norm_t<1>(h, ldh, m, n, weight, eps, hq, ldq, amax, xsum, keep, rows ? totals : nullptr, s);
}

// One workgroup per row: the row's n terms into LDS, then the index-order
// chain s0 + t[0] + t[1] + ... formed by ordered_sum_wave (64 threads) or
// ordered_sum_block on four waves (256 or 512 threads: the strict norm
// kernels' widths).
template <int W>
__global__ __launch_bounds__(W * 64) void ordered_sum_rows_kernel(const double* __restrict__ terms, int n,
                                                                  double s0, double* __restrict__ out) {
    extern __shared__ double tsh[];
    const double* tr = terms + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += W * 64) tsh[i] = tr[i];
    __syncthreads();
    double r;
    if constexpr (W == 1) {
        r = ordered_sum_wave<kChainC>(tsh, n, s0);
    } else {  // the first four waves form the sum
        __shared__ OrderedSumLds<4> osum;
        r = ordered_sum_block<4>(tsh, n, s0, osum);
    }
    if (threadIdx.x == 0) out[blockIdx.x] = r;
}

hipError_t launch_ordered_sum_rows(const double* terms, int m, int n, double s0, double* out,
                                   int threads, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    if (n <= 0 || n > kMaxStrictNormCols) return hipErrorInvalidValue;
    const size_t shm = (size_t)max(n, ordered_sum_slots(n, threads < 256 ? 1 : 4)) * sizeof(double);
    if (threads == 64) {
        hipLaunchKernelGGL(ordered_sum_rows_kernel<1>, dim3(m), dim3(64), shm, s, terms, n, s0, out);
    } else if (threads == 256) {
        hipLaunchKernelGGL(ordered_sum_rows_kernel<4>, dim3(m), dim3(256), shm, s, terms, n, s0, out);
    } else if (threads == 512) {
        hipLaunchKernelGGL(ordered_sum_rows_kernel<8>, dim3(m), dim3(512), shm, s, terms, n, s0, out);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// y[i] = exp(x[i]) in fp64 with the device exp every kernel of the library
// calls (the attention probabilities, the SwiGLU gate's sigmoid, Activate).
__global__ __launch_bounds__(256) void exp_rows_kernel(const double* __restrict__ x, long n,
                                                       double* __restrict__ y) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = exp(x[i]);
}

hipError_t launch_exp_rows(const double* x, long n, double* y, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const long blocks = std::min<long>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(exp_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, n, y);
    return hipGetLastError();
}

}  // namespace lamd
