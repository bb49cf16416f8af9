// ternary_kernels.hip -- gfx950 kernels of the BitNet b1.58 ternary path.
//
//   repack_tiles      loom Words (poly/bitnet_cpu.go:14-43) -> tile layout (lamd.hpp)
//   act_quant         per-token absmax + int8 quantization (poly/bitnet_cpu.go:45-117)
//   skinny_matmul     M <= 64 token rows: split-K over the waves of a workgroup,
//                     int8 MFMA 16x16x64 with codes unpacked in registers (decode / GEMV)
//   gemm_matmul       M > 64: 128-row x 128-column workgroup tiles on int8 MFMA (prefill)
//   norm_quant        SwiGLU inner RMSNorm + requantization (poly/bitnet_cpu.go:893-913)
//
// Every fp64 expression is evaluated in the reference's operation order with
// contraction disabled (the library is built with -ffp-contract=off), so the
// rescale epilogues are bit-exact against loom's CPU path.
#include "lamd.hpp"

#include <math.h>

#pragma clang fp contract(off)

namespace lamd {

typedef int v4i __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------
// small helpers
// ------------------------------------------------------------------------

__device__ __forceinline__ v4i unpack_codes(uint32_t w) {
    v4i b;
    b[0] = (int)(w & 0x03030303u);
    b[1] = (int)((w >> 2) & 0x03030303u);
    b[2] = (int)((w >> 4) & 0x03030303u);
    b[3] = (int)((w >> 6) & 0x03030303u);
    return b;
}

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Go's int(float64) on amd64 (CVTTSD2SQ): NaN and out-of-range values give
// the integer-indefinite INT64_MIN, which loom then clamps to -128
// (poly/bitnet_cpu.go:73-84).
__device__ __forceinline__ int8_t quant_one(double v, double scale) {
    double r = round(v * scale);
    if (!(r >= -9223372036854775808.0 && r < 9223372036854775808.0)) {
        return (int8_t)-128;
    }
    if (r < -128.0) return (int8_t)-128;
    if (r > 127.0) return (int8_t)127;
    return (int8_t)(int)r;
}

// loom's "a > maxAbs" update: NaN never replaces the running maximum.
__device__ __forceinline__ float max_nan_skip(float m, float a) { return a > m ? a : m; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v = max_nan_skip(v, __shfl_xor(v, off, 64));
    }
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_xor(v, off, 64);
    }
    return v;
}

// Block reductions over blockDim.x threads (multiple of 64, <= 1024).
__device__ float block_max(float v, float* sh) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < nw; ++i) r = max_nan_skip(r, sh[i]);
    __syncthreads();
    return r;
}

__device__ int block_sum_i(int v, int* sh) {
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
__device__ float activate_f32(float v, int act) {
    switch (act) {
        case 0:  // ReLU
            return v < 0.0f ? 0.0f : v;
        case 1:  // SiLU: v * float32(1/(1+exp(-v)))
            return v * (float)(1.0 / (1.0 + exp(-(double)v)));
        case 2: {  // GELU (tanh form)
            double v64 = (double)v;
            return (float)(0.5 * v64 *
                           (1.0 + tanh(sqrt(2.0 / M_PI) * (v64 + 0.044715 * pow(v64, 3.0)))));
        }
        case 3:
            return (float)tanh((double)v);
        case 4:
            return (float)(1.0 / (1.0 + exp(-(double)v)));
        case 5:
            return v < 0.0f ? (float)((double)v * 0.01) : v;
        case 6:  // ReLU2
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
    double sig = 1.0 / (1.0 + exp(-g));
    return (g * sig) * u;
}

// bitNetTernaryMatVecQuantized output scale (poly/bitnet_cpu.go:540-543).
__device__ __forceinline__ double output_scale(float wscale, float amax) {
    double s = (double)wscale * (double)amax / 127.0;
    return s == 0.0 ? 1.0 : s;
}

// ------------------------------------------------------------------------
// repack: loom row-major Words -> tile layout
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
    const int k0 = kt * kTileCols + (lane >> 4) * 64 + t * 16;
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
// activation quantization: one workgroup per token row
// ------------------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(256) void act_quant_kernel(const T* __restrict__ x, int ldx, int k,
                                                        int ldq, int8_t* __restrict__ xq,
                                                        float* __restrict__ amax_out,
                                                        int32_t* __restrict__ xsum_out) {
    __shared__ float shf[16];
    __shared__ int shi[16];
    const int row = blockIdx.x;
    const T* xr = x + (size_t)row * ldx;
    float m = 0.0f;
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        // float32(|float64(v)|): exact for fp32 input, one rounding for fp64.
        m = max_nan_skip(m, (float)fabs((double)xr[i]));
    }
    m = block_max(m, shf);
    if (m < 1e-5f) m = 1e-5f;
    const double scale = 127.0 / (double)m;
    int s = 0;
    int8_t* qr = xq + (size_t)row * ldq;
    for (int i = threadIdx.x; i < ldq; i += blockDim.x) {
        int8_t q = 0;
        if (i < k) {
            q = quant_one((double)xr[i], scale);
            s += q;
        }
        qr[i] = q;
    }
    s = block_sum_i(s, shi);
    if (threadIdx.x == 0) {
        amax_out[row] = m;
        xsum_out[row] = s;
    }
}

hipError_t launch_act_quant(const float* x, int ldx, int m, int k, int8_t* xq, int ldq,
                            float* amax, int32_t* xsum, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    hipLaunchKernelGGL(act_quant_kernel<float>, dim3(m), dim3(256), 0, s, x, ldx, k, ldq, xq,
                       amax, xsum);
    return hipGetLastError();
}

hipError_t launch_act_quant_f64(const double* x, int ldx, int m, int k, int8_t* xq, int ldq,
                                float* amax, int32_t* xsum, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    hipLaunchKernelGGL(act_quant_kernel<double>, dim3(m), dim3(256), 0, s, x, ldx, k, ldq, xq,
                       amax, xsum);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// matmul epilogue
// ------------------------------------------------------------------------

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

// raw0/raw1 are sum(code * xq) of matrix 0/1 for token row i, output n.
__device__ __forceinline__ void epilogue_store(const EpiDev& e, int i, int n, int raw0, int raw1) {
    const int32_t xs = e.xsum[i];
    const float am = e.amax[i];
    const int acc0 = raw0 - xs;
    const size_t o = (size_t)i * e.ldo + n;
    if (e.acc0) e.acc0[(size_t)i * e.n + n] = acc0;
    if (e.kind == EPI_SWIGLU) {
        const int acc1 = raw1 - xs;
        if (e.acc1) e.acc1[(size_t)i * e.n + n] = acc1;
        // g := gate[o] + bias; u := up[o] + bias   (poly/swiglu.go:306-309)
        const double g = (double)acc0 * output_scale(e.scale0, am) +
                         (e.bias0 ? (double)e.bias0[n] : 0.0);
        const double u = (double)acc1 * output_scale(e.scale1, am) +
                         (e.bias1 ? (double)e.bias1[n] : 0.0);
        e.out[o] = (float)gate_product(g, u, e.activation);
        return;
    }
    double d = (double)acc0 * output_scale(e.scale0, am);
    if (e.bias0) d = d + (double)e.bias0[n];
    float v = (float)d;
    if (e.residual) v = v + e.residual[o];
    e.out[o] = v;
    if (e.post) e.post[o] = activate_f32(v, e.activation);
}

// ------------------------------------------------------------------------
// skinny matmul (M <= 16*MSUB): one workgroup per 16-row weight tile,
// K tiles split over WAVES waves, partial sums merged with LDS integer adds
// ------------------------------------------------------------------------

struct MatArgs {
    const uint4* w0;
    const uint4* w1;
    int ktiles;
    int ntiles;
    const int8_t* xq;
    int ldq;
    EpiDev e;
};

template <int NMAT, int MSUB, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void skinny_matmul_kernel(MatArgs p) {
    constexpr int U = 4;  // K tiles in flight per wave
    __shared__ int red[NMAT][MSUB * 16][16];
    const int nt = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int M = p.e.m;

    for (int i = threadIdx.x; i < NMAT * MSUB * 16 * 16; i += WAVES * 64) {
        (&red[0][0][0])[i] = 0;
    }

    v4i acc[NMAT][MSUB];
#pragma unroll
    for (int a = 0; a < NMAT; ++a)
#pragma unroll
        for (int ms = 0; ms < MSUB; ++ms) acc[a][ms] = v4i{0, 0, 0, 0};

    const size_t tile0 = (size_t)nt * p.ktiles * 64 + lane;
    const int8_t* xbase[MSUB];
    bool xval[MSUB];
#pragma unroll
    for (int ms = 0; ms < MSUB; ++ms) {
        const int row = ms * 16 + r;
        xval[ms] = row < M;
        xbase[ms] = p.xq + (size_t)(xval[ms] ? row : 0) * p.ldq + g * 64;
    }

    for (int kb = wave; kb < p.ktiles; kb += WAVES * U) {
        uint4 wv[NMAT][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kb + u * WAVES;
            if (kt < p.ktiles) {
                wv[0][u] = p.w0[tile0 + (size_t)kt * 64];
                if (NMAT == 2) wv[NMAT - 1][u] = p.w1[tile0 + (size_t)kt * 64];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kt = kb + u * WAVES;
            if (kt < p.ktiles) {
                v4i a[MSUB][4];
#pragma unroll
                for (int ms = 0; ms < MSUB; ++ms) {
                    const v4i* xp = (const v4i*)(xbase[ms] + (size_t)kt * kTileCols);
#pragma unroll
                    for (int t = 0; t < 4; ++t) a[ms][t] = xval[ms] ? xp[t] : v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
#pragma unroll
                    for (int mat = 0; mat < NMAT; ++mat) {
                        const uint4 q = wv[mat][u];
                        const uint32_t word = t == 0 ? q.x : t == 1 ? q.y : t == 2 ? q.z : q.w;
                        const v4i b = unpack_codes(word);
#pragma unroll
                        for (int ms = 0; ms < MSUB; ++ms) acc[mat][ms] = mfma_i8(a[ms][t], b, acc[mat][ms]);
                    }
                }
            }
        }
    }

    __syncthreads();
    // D layout of MFMA 16x16: lane l, element v -> A row 4*(l>>4)+v, B column l&15.
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int ms = 0; ms < MSUB; ++ms)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int tok = ms * 16 + 4 * g + v;
                if (tok < M) atomicAdd(&red[mat][tok][r], acc[mat][ms][v]);
            }
    __syncthreads();

    const int outs = M * 16;
    for (int idx = threadIdx.x; idx < outs; idx += WAVES * 64) {
        const int tok = idx >> 4;
        const int col = idx & 15;
        const int n = nt * kTileRows + col;
        if (n < p.e.n) {
            epilogue_store(p.e, tok, n, red[0][tok][col], red[NMAT - 1][tok][col]);
        }
    }
}

// ------------------------------------------------------------------------
// GEMM (M > 64): 256-thread workgroups of 2x2 waves; each wave owns a
// 64-row x (4/NMAT)*16-column block per matrix, K loop over 256-column tiles
// with the next tile's loads issued before the current tile's MFMAs.
// ------------------------------------------------------------------------

template <int NMAT>
__global__ __launch_bounds__(256, 2) void gemm_matmul_kernel(MatArgs p) {
    constexpr int MI = 4;
    constexpr int NJ = 4 / NMAT;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.e.m;

    const int m0 = (blockIdx.y * 2 + wm) * 64;
    const int nt0 = (blockIdx.x * 2 + wn) * NJ;

    const int8_t* arow[MI];
    bool aval[MI];
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int row = m0 + 16 * i + r;
        aval[i] = row < M;
        arow[i] = p.xq + (size_t)(aval[i] ? row : 0) * p.ldq + g * 64;
    }
    const uint4* bptr[NMAT][NJ];
    bool bval[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int nt = nt0 + j;
        bval[j] = nt < p.ntiles;
        const size_t base = (size_t)(bval[j] ? nt : 0) * p.ktiles * 64 + lane;
        bptr[0][j] = p.w0 + base;
        if (NMAT == 2) bptr[NMAT - 1][j] = p.w1 + base;
    }

    v4i acc[NMAT][MI][NJ];
#pragma unroll
    for (int a = 0; a < NMAT; ++a)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[a][i][j] = v4i{0, 0, 0, 0};

    v4i a_cur[MI][4];
    uint4 b_cur[NMAT][NJ];
    auto load_tile = [&](int kt, v4i (&a)[MI][4], uint4 (&b)[NMAT][NJ]) {
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const v4i* xp = (const v4i*)(arow[i] + (size_t)kt * kTileCols);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[i][t] = aval[i] ? xp[t] : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                b[mat][j] = bval[j] ? bptr[mat][j][(size_t)kt * 64] : uint4{0, 0, 0, 0};
    };

    load_tile(0, a_cur, b_cur);
    for (int kt = 0; kt < p.ktiles; ++kt) {
        v4i a_nxt[MI][4];
        uint4 b_nxt[NMAT][NJ];
        if (kt + 1 < p.ktiles) load_tile(kt + 1, a_nxt, b_nxt);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const uint4 q = b_cur[mat][j];
                    const uint32_t word = t == 0 ? q.x : t == 1 ? q.y : t == 2 ? q.z : q.w;
                    const v4i b = unpack_codes(word);
#pragma unroll
                    for (int i = 0; i < MI; ++i) acc[mat][i][j] = mfma_i8(a_cur[i][t], b, acc[mat][i][j]);
                }
        }
        if (kt + 1 < p.ktiles) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int t = 0; t < 4; ++t) a_cur[i][t] = a_nxt[i][t];
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int j = 0; j < NJ; ++j) b_cur[mat][j] = b_nxt[mat][j];
        }
    }

#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int n = (nt0 + j) * kTileRows + r;
            if (n >= p.e.n) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int tok = m0 + 16 * i + 4 * g + v;
                if (tok < M) epilogue_store(p.e, tok, n, acc[0][i][j][v], acc[NMAT - 1][i][j][v]);
            }
        }
}

// ------------------------------------------------------------------------
// dispatch
// ------------------------------------------------------------------------

// Split-K width: enough waves for ~2048 in flight over the chip, never more
// waves than K tiles, and at most `cap` (register budget of wide tiles).
static int pick_waves(int ntiles, int ktiles, int cap) {
    int want = (2048 + ntiles - 1) / ntiles;
    int w = 1;
    while (w < want && w < cap && w < ktiles) w <<= 1;
    return w;
}

template <int NMAT, int MSUB>
static hipError_t launch_skinny(const MatArgs& p, hipStream_t s) {
    // 1024-thread workgroups leave 128 VGPRs per lane: too few for NMAT*MSUB >= 8.
    const int w = pick_waves(p.ntiles, p.ktiles, NMAT * MSUB >= 8 ? 8 : 16);
    const dim3 grid(p.ntiles);
    switch (w) {
        case 1:
            hipLaunchKernelGGL((skinny_matmul_kernel<NMAT, MSUB, 1>), grid, dim3(64), 0, s, p);
            break;
        case 2:
            hipLaunchKernelGGL((skinny_matmul_kernel<NMAT, MSUB, 2>), grid, dim3(128), 0, s, p);
            break;
        case 4:
            hipLaunchKernelGGL((skinny_matmul_kernel<NMAT, MSUB, 4>), grid, dim3(256), 0, s, p);
            break;
        case 8:
            hipLaunchKernelGGL((skinny_matmul_kernel<NMAT, MSUB, 8>), grid, dim3(512), 0, s, p);
            break;
        default:
            if constexpr (NMAT * MSUB < 8) {
                hipLaunchKernelGGL((skinny_matmul_kernel<NMAT, MSUB, 16>), grid, dim3(1024), 0, s, p);
            }
            break;
    }
    return hipGetLastError();
}

const char* kernel_variant(int m) {
    if (m <= 16) return "skinny_m16";
    if (m <= 32) return "skinny_m32";
    if (m <= 64) return "skinny_m64";
    return "gemm_128";
}

hipError_t launch_matmul(const Matrix* w0, const Matrix* w1, const QuantAct& a, int m,
                         const Epilogue& epi, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    MatArgs p;
    p.w0 = (const uint4*)w0->tiles;
    p.w1 = (const uint4*)(w1 ? w1->tiles : w0->tiles);
    p.ktiles = w0->ktiles;
    p.ntiles = w0->ntiles;
    p.xq = a.xq;
    p.ldq = a.ldq;
    EpiDev& e = p.e;
    e.kind = epi.kind;
    e.activation = epi.activation;
    e.m = m;
    e.n = w0->rows;
    e.scale0 = w0->scale;
    e.scale1 = w1 ? w1->scale : w0->scale;
    e.amax = a.amax;
    e.xsum = a.xsum;
    e.bias0 = epi.bias0;
    e.bias1 = epi.bias1;
    e.residual = epi.residual;
    e.out = epi.out;
    e.post = epi.post;
    e.ldo = epi.ldo > 0 ? epi.ldo : w0->rows;
    e.acc0 = epi.acc0;
    e.acc1 = epi.acc1;
    const bool two = epi.kind == EPI_SWIGLU;
    if (m <= 16) return two ? launch_skinny<2, 1>(p, s) : launch_skinny<1, 1>(p, s);
    if (m <= 32) return two ? launch_skinny<2, 2>(p, s) : launch_skinny<1, 2>(p, s);
    if (m <= 64) return two ? launch_skinny<2, 4>(p, s) : launch_skinny<1, 4>(p, s);
    const int nj = two ? 2 : 4;
    const dim3 grid(ceil_div(p.ntiles, 2 * nj), ceil_div(m, 128));
    if (two) {
        hipLaunchKernelGGL(gemm_matmul_kernel<2>, grid, dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL(gemm_matmul_kernel<1>, grid, dim3(256), 0, s, p);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// SwiGLU inner RMSNorm + requantization, one workgroup per row
// ------------------------------------------------------------------------

// strict: the sum of squares is one sequential fp64 chain in column order,
// exactly loom's loop (poly/bitnet_cpu.go:900-905).  fast: each thread sums a
// contiguous chunk, then a fixed binary tree; deterministic, but rounds the
// sum differently, which moves normalized values by at most one fp32 ulp.
template <int STRICT>
__global__ __launch_bounds__(256) void norm_quant_kernel(float* __restrict__ h, int ldh, int n,
                                                         const float* __restrict__ weight,
                                                         double eps, int8_t* __restrict__ hq,
                                                         int ldq, float* __restrict__ amax_out,
                                                         int32_t* __restrict__ xsum_out) {
    extern __shared__ double dsh[];  // STRICT: n floats staged; fast: 256 partial sums
    __shared__ float shf[16];
    __shared__ int shi[16];
    __shared__ double total;
    const int row = blockIdx.x;
    float* hr = h + (size_t)row * ldh;

    if (STRICT) {
        float* stage = (float*)dsh;
        for (int i = threadIdx.x; i < n; i += blockDim.x) stage[i] = hr[i];
        __syncthreads();
        if (threadIdx.x == 0) {
            double s = 0.0;
            for (int i = 0; i < n; ++i) {
                const double f = (double)stage[i];
                s += f * f;
            }
            total = s;
        }
        __syncthreads();
    } else {
        const int chunk = (n + blockDim.x - 1) / blockDim.x;
        const int lo = threadIdx.x * chunk;
        const int hi = min(n, lo + chunk);
        double s = 0.0;
        for (int i = lo; i < hi; ++i) {
            const double f = (double)hr[i];
            s += f * f;
        }
        dsh[threadIdx.x] = s;
        __syncthreads();
        for (int width = blockDim.x >> 1; width > 0; width >>= 1) {
            if (threadIdx.x < width) dsh[threadIdx.x] = dsh[threadIdx.x] + dsh[threadIdx.x + width];
            __syncthreads();
        }
        if (threadIdx.x == 0) total = dsh[0];
        __syncthreads();
    }

    const double scale = 1.0 / sqrt(total / (double)n + eps);
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const double w = weight ? (double)weight[i] : 1.0;
        const float v = (float)((double)hr[i] * scale * w);
        hr[i] = v;
        m = max_nan_skip(m, fabsf(v));
    }
    m = block_max(m, shf);
    if (m < 1e-5f) m = 1e-5f;
    const double qs = 127.0 / (double)m;
    int s = 0;
    int8_t* qr = hq + (size_t)row * ldq;
    for (int i = threadIdx.x; i < ldq; i += blockDim.x) {
        int8_t q = 0;
        if (i < n) {
            q = quant_one((double)hr[i], qs);
            s += q;
        }
        qr[i] = q;
    }
    s = block_sum_i(s, shi);
    if (threadIdx.x == 0) {
        amax_out[row] = m;
        xsum_out[row] = s;
    }
}

hipError_t launch_norm_quant(float* h, int ldh, int m, int n, const float* weight, double eps,
                             int strict, int8_t* hq, int ldq, float* amax, int32_t* xsum,
                             hipStream_t s) {
    if (m <= 0) return hipSuccess;
    if (eps <= 0.0) eps = 1e-5;
    if (strict) {
        const size_t shm = (size_t)n * sizeof(float);
        if (shm > 160 * 1024 - 1024) return hipErrorInvalidValue;
        hipLaunchKernelGGL(norm_quant_kernel<1>, dim3(m), dim3(256), shm, s, h, ldh, n, weight,
                           eps, hq, ldq, amax, xsum);
    } else {
        hipLaunchKernelGGL(norm_quant_kernel<0>, dim3(m), dim3(256), 256 * sizeof(double), s, h,
                           ldh, n, weight, eps, hq, ldq, amax, xsum);
    }
    return hipGetLastError();
}

}  // namespace lamd
