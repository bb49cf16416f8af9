// block.hip -- gfx950 kernels of loom's BitNet decoder block and decode step
// (poly/transformer_forward.go:220-253, poly/mha.go:204-371, poly/norm.go:102-138,
// poly/transformer.go:551-577,635-719, poly/sampling.go:44-55).
//
// Sequential fp64 sums of the reference (RMSNorm, inner norms, softmax) have
// two modes: STRICT reproduces the reference's left-to-right chain (terms are
// formed in parallel, one lane adds them in order); fast uses a fixed-order
// tree (deterministic, last-bit differences only).  The KV position of each
// call is read from device memory so a decode step can be graph-replayed.
#include "block.hpp"
#include "device_common.hpp"

namespace lamd {

// ------------------------------------------------------------------------
// shared: ordered / tree fp64 sum of n terms held in LDS (256 threads)
// ------------------------------------------------------------------------

template <int STRICT>
__device__ __forceinline__ double lds_sum(double* terms, int n, double* scratch256) {
    __shared__ double result;
    __syncthreads();
    if (STRICT) {
        __shared__ OrderedSumLds<4> osum;
        return ordered_sum_block<4>(terms, n, 0.0, osum);
    }
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += terms[i];
    scratch256[threadIdx.x] = s;
    __syncthreads();
    for (int w = blockDim.x >> 1; w > 0; w >>= 1) {
        if (threadIdx.x < w) scratch256[threadIdx.x] = scratch256[threadIdx.x] + scratch256[threadIdx.x + w];
        __syncthreads();
    }
    const double r = scratch256[0];
    __syncthreads();
    return r;
}

// ------------------------------------------------------------------------
// Strict sums of squares of many rows (prefill): one lane per row.  Lane r
// of a wave adds row r's squares in element order -- the reference's
// sequential chain -- so a wave runs 64 chains at the latency of one, where
// the per-row kernels below run one chain per workgroup.  Each lane reads its
// row in 16-byte loads, eight loads a block, the next block in flight while
// the current one is added (the block read after the last full one is
// clamped to an existing block instead of guarded by a branch).  For fp32
// rows the fp64 squares are exact; for fp64 rows each square is rounded
// before its addition, as the reference computes it.
// ------------------------------------------------------------------------
constexpr int kRowChainMinRows = 1024;  // below this the per-row kernels form each row's sum themselves

template <typename T>
__global__ __launch_bounds__(64) void row_sumsq_kernel(const T* __restrict__ x, long ldx, int n, int m,
                                                       double* __restrict__ totals) {
    constexpr int V = 16 / sizeof(T);  // elements per load
    constexpr int G = 8;               // loads per block
    constexpr int E = V * G;           // elements per block
    const int row = blockIdx.x * 64 + threadIdx.x;
    const T* xr = x + (size_t)min(row, m - 1) * ldx;  // lanes past m repeat the last row, store nothing
    double s = 0.0;
    const int nb = n / E;
    auto add = [&](const uint4 (&blk)[G]) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if constexpr (sizeof(T) == 4) {
                const float4 f = __builtin_bit_cast(float4, blk[g]);
                const double a = f.x, b = f.y, c = f.z, d = f.w;
                s = s + a * a;
                s = s + b * b;
                s = s + c * c;
                s = s + d * d;
            } else {
                const double2 f = __builtin_bit_cast(double2, blk[g]);
                s = s + f.x * f.x;
                s = s + f.y * f.y;
            }
        }
    };
    if (nb > 0) {
        const uint4* xv = (const uint4*)xr;
        uint4 a[G], b[G];
#pragma unroll
        for (int g = 0; g < G; ++g) a[g] = xv[g];
        int blk = 0;
        for (; blk + 2 <= nb; blk += 2) {  // a holds block blk
            const uint4* pb = xv + (size_t)(blk + 1) * G;
            const uint4* pa = xv + (size_t)min(blk + 2, nb - 1) * G;
#pragma unroll
            for (int g = 0; g < G; ++g) b[g] = pb[g];
            add(a);
#pragma unroll
            for (int g = 0; g < G; ++g) a[g] = pa[g];
            add(b);
        }
        if (blk < nb) add(a);
    }
    for (int i = nb * E; i < n; ++i) {
        const double f = (double)xr[i];
        s = s + f * f;
    }
    if (row < m) totals[row] = s;
}

// Strict row totals for m rows when the row-chain kernel applies (many rows,
// 16-byte aligned rows); returns false when the caller keeps its own chain.
template <typename T>
static bool launch_row_sumsq(const T* x, long ldx, int m, int n, double* totals, hipStream_t s,
                             hipError_t* e) {
    if (!totals || m < kRowChainMinRows) return false;
    if (((uintptr_t)x & 15) != 0 || ((size_t)ldx * sizeof(T)) % 16 != 0) return false;
    hipLaunchKernelGGL((row_sumsq_kernel<T>), dim3(ceil_div(m, 64)), dim3(64), 0, s, x, ldx, n, m, totals);
    *e = hipGetLastError();
    return true;
}

bool launch_row_sumsq_f32(const float* x, long ldx, int m, int n, double* totals, hipStream_t s,
                          hipError_t* e) {
    return launch_row_sumsq<float>(x, ldx, m, n, totals, s, e);
}

// ------------------------------------------------------------------------
// RMSNorm layer (poly/norm.go:102-138) fused with the following projection's
// int8 quantization (poly/bitnet_cpu.go:45-106): one workgroup per row.
// y = fp32((x / rms) * g), rms = sqrt(sum(x^2)/n + eps).  xq may be null
// (final norm: y only); y may be null (only the quantized row is needed).
// ------------------------------------------------------------------------

template <int STRICT, int VPT>
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const float* __restrict__ x, long ldx, int n,
                                                            const float* __restrict__ gain,
                                                            double eps, float* __restrict__ y,
                                                            int8_t* __restrict__ xq, int ldq,
                                                            float* __restrict__ amax_out,
                                                            int32_t* __restrict__ xsum_out,
                                                            const double* __restrict__ totals) {
    extern __shared__ double sq[];  // STRICT: n squares; fast: 256 partials
    __shared__ double red[256];
    __shared__ float shf[4];
    __shared__ int shi[4];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * ldx;
    float v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        v[j] = i < n ? xr[i] : 0.0f;
    }
    double total;
    if (STRICT && totals) {
        total = totals[row];  // the row-chain kernel's ordered sum
    } else if (STRICT) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = threadIdx.x + j * 256;
            if (i < n) {
                const double f = (double)v[j];
                sq[i] = f * f;  // exact: 24-bit significands
            }
        }
        total = lds_sum<1>(sq, n, red);
    } else {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const double f = (double)v[j];
            s += f * f;
        }
        red[threadIdx.x] = s;
        __syncthreads();
        for (int w = 128; w > 0; w >>= 1) {
            if (threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
            __syncthreads();
        }
        total = red[0];
    }
    const double rms = sqrt(total / (double)n + eps);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        if (i < n) {
            const double normed = (double)v[j] / rms;
            v[j] = (float)(normed * (double)gain[i]);
            if (y) y[(size_t)row * n + i] = v[j];
            m = max_nan_skip(m, fabsf(v[j]));
        }
    }
    if (!xq) return;
    m = block_max(m, shf);
    if (m < 1e-5f) m = 1e-5f;
    const double qs = 127.0 / (double)m;
    const float qs32 = (float)qs;
    int s = 0;
    int8_t* qr = xq + (size_t)row * ldq;
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

template <int STRICT>
static hipError_t launch_rmsnorm_t(const float* x, long ldx, int m, int n, const float* gain,
                                   double eps, float* y, int8_t* xq, int ldq, float* amax,
                                   int32_t* xsum, const double* totals, hipStream_t s) {
    if (xq) {  // (the final norm without quantization keeps the workgroup kernel)
        const RowNormArgs a{x, ldx, m, n, gain, eps, y, nullptr, xq, ldq, amax, xsum, totals};
        hipError_t e = hipSuccess;
        if (launch_row_norm_wave(kRowRms, STRICT, a, s, &e)) return e;
    }
    const size_t shm = STRICT && !totals ? (size_t)ordered_sum_slots(n, 4) * sizeof(double) : 0;
    const dim3 g(m), b(256);
#define LAMD_RMS(VPT)                                                                          \
    hipLaunchKernelGGL((rmsnorm_quant_kernel<STRICT, VPT>), g, b, shm, s, x, ldx, n, gain, eps, y, xq, \
                       ldq, amax, xsum, totals)
    if (n <= 256 * 4) {
        LAMD_RMS(4);
    } else if (n <= 256 * 8) {
        LAMD_RMS(8);
    } else if (n <= 256 * 16) {
        LAMD_RMS(16);
    } else if (n <= 256 * 32) {
        LAMD_RMS(32);
    } else {
        return hipErrorInvalidValue;
    }
#undef LAMD_RMS
    return hipGetLastError();
}

hipError_t launch_rmsnorm_quant(const float* x, long ldx, int m, int n, const float* gain,
                                double eps, int strict, float* y, int8_t* xq, int ldq, float* amax,
                                int32_t* xsum, hipStream_t s, double* totals) {
    if (m <= 0) return hipSuccess;
    if (eps <= 0.0) eps = 1e-6;  // RMSNormForwardPolymorphic default
    if (n > kMaxNormCols || (strict && n > kMaxStrictNormCols)) return hipErrorInvalidValue;
    if (!strict) return launch_rmsnorm_t<0>(x, ldx, m, n, gain, eps, y, xq, ldq, amax, xsum, nullptr, s);
    hipError_t e = hipSuccess;
    const bool rows = launch_row_sumsq<float>(x, ldx, m, n, totals, s, &e);
    if (e != hipSuccess) return e;
    return launch_rmsnorm_t<1>(x, ldx, m, n, gain, eps, y, xq, ldq, amax, xsum, rows ? totals : nullptr, s);
}

// ------------------------------------------------------------------------
// Q/K/V epilogue of the stacked projection (poly/mha.go:258-313).  acc holds
// the int32 accumulators of the stacked [Q; K; V] ternary matrix for `seq`
// token rows (row stride q_dim + 2*kv_dim).  Per token at position pos:
//   Q = fp64(acc)*os_q + bias_q (fp64, kept), rotated in fp64;
//   K = fp32(fp64(acc)*os_k + bias_k), rotated from fp64 back to fp32;
//   V = fp32(fp64(acc)*os_v + bias_v);
// With per-head Q/K norm weights (poly/mha.go:285-290), Q and the fp32 K row
// are normalized per head before the rotation (applyPerHeadRMSNormFloat64 /
// ...Tensor, poly/mha.go:584-646): the head's sum of squares as the
// dimension-order fp64 chain, inv = 1/sqrt(sumSq/hd + eps), x = x*inv*gamma
// (left to right; K rounded back to fp32); a head with rms == 0 is left
// unchanged.
// RoPE rotates the half-split pairs (d, d + hd/2) by pos / theta^(2d/hd).
// K and V go to ring row pos % msl of the row's sequence slot (batch index);
// when one call holds more than msl tokens only the last token of each ring
// row is written (the reference writes them in order, so the last one
// stays).
// ------------------------------------------------------------------------

__device__ __forceinline__ void rope_angle(int pos, int d, int hd, double theta, double* c,
                                           double* sn) {
    const double angle = (double)pos / pow(theta, (double)(2 * d) / (double)hd);
    *c = cos(angle);
    *sn = sin(angle);
}

// Per-head norm of one head (see above).  inv < 0 marks a head the
// reference leaves unchanged (rms == 0); a NaN inv is applied, as there.
struct HeadNorm {
    bool on = false;   // weights present for this projection
    double inv = 0.0;
    double g0 = 1.0, g1 = 1.0;  // gamma of the pair's two dimensions
};

// gamma element of dimension d of head h: gamma[d] when the weights hold one
// head, gamma[h*hd + d] when they hold every head, else 1
__device__ __forceinline__ double qk_gamma(const float* g, int len, int heads, int hd, int h, int d) {
    if (len == hd) return (double)g[d];
    if (len == heads * hd) return (double)g[(size_t)h * hd + d];
    return 1.0;
}

__device__ __forceinline__ double qk_inv_rms(double sum_sq, int hd, double eps) {
    const double rms = sqrt(sum_sq / (double)hd + eps);
    return rms == 0.0 ? -1.0 : 1.0 / rms;
}

__device__ __forceinline__ HeadNorm head_norm(bool on, double inv, const float* g, int len, int heads,
                                              int hd, int h, int d0, int d1) {
    HeadNorm n;
    n.on = on && !(inv < 0.0);
    n.inv = inv;
    if (n.on) {
        n.g0 = qk_gamma(g, len, heads, hd, h, d0);
        n.g1 = qk_gamma(g, len, heads, hd, h, d1);
    }
    return n;
}

// The sequential fp64 sum of squares of one head's Q (fp64 after bias) or K
// (rounded to fp32 first) values, formed by one thread from the accumulators
// (j0: the head's first accumulator index within the projection).
template <bool KROUND>
__device__ __forceinline__ double head_sum_sq(const int32_t* ar, double os, const float* b, int j0, int hd) {
    double s = 0.0;
#pragma unroll 8
    for (int d = 0; d < hd; ++d) {
        double v = (double)ar[j0 + d] * os + (b ? (double)b[j0 + d] : 0.0);
        if (KROUND) v = (double)(float)v;
        s = s + v * v;
    }
    return s;
}

// The three per-element steps, shared with the fused decode attention kernel.
// The *_v forms take the loaded accumulators and biases (b_on: a bias exists).
__device__ __forceinline__ void q_pair_v(int32_t a0, int32_t a1, double os, bool b_on, float b0, float b1,
                                         double c, double sn, double* o0, double* o1,
                                         const HeadNorm& hn = HeadNorm{}) {
    double v0 = (double)a0 * os + (b_on ? (double)b0 : 0.0);
    double v1 = (double)a1 * os + (b_on ? (double)b1 : 0.0);
    if (hn.on) {
        v0 = v0 * hn.inv * hn.g0;
        v1 = v1 * hn.inv * hn.g1;
    }
    *o0 = v0 * c - v1 * sn;
    *o1 = v0 * sn + v1 * c;
}

__device__ __forceinline__ void k_pair_v(int32_t a0, int32_t a1, double os, bool b_on, float b0, float b1,
                                         double c, double sn, float* o0, float* o1,
                                         const HeadNorm& hn = HeadNorm{}) {
    float k0 = (float)((double)a0 * os + (b_on ? (double)b0 : 0.0));
    float k1 = (float)((double)a1 * os + (b_on ? (double)b1 : 0.0));
    if (hn.on) {
        k0 = (float)((double)k0 * hn.inv * hn.g0);
        k1 = (float)((double)k1 * hn.inv * hn.g1);
    }
    const double v0 = (double)k0, v1 = (double)k1;
    *o0 = (float)(v0 * c - v1 * sn);
    *o1 = (float)(v0 * sn + v1 * c);
}

__device__ __forceinline__ float v_val_v(int32_t a, double os, bool b_on, float b) {
    return (float)((double)a * os + (b_on ? (double)b : 0.0));
}

__device__ __forceinline__ void q_pair(const int32_t* ar, double os, const float* bq, int j0, int j1,
                                       double c, double sn, double* o0, double* o1,
                                       const HeadNorm& hn = HeadNorm{}) {
    q_pair_v(ar[j0], ar[j1], os, bq != nullptr, bq ? bq[j0] : 0.0f, bq ? bq[j1] : 0.0f, c, sn, o0, o1,
             hn);
}

// ar points at the K part of the row's accumulators; j0/j1 index into K
__device__ __forceinline__ void k_pair(const int32_t* ar, double os, const float* bk, int j0, int j1,
                                       double c, double sn, float* o0, float* o1,
                                       const HeadNorm& hn = HeadNorm{}) {
    k_pair_v(ar[j0], ar[j1], os, bk != nullptr, bk ? bk[j0] : 0.0f, bk ? bk[j1] : 0.0f, c, sn, o0, o1,
             hn);
}

// ar points at the V part of the row's accumulators
__device__ __forceinline__ float v_val(const int32_t* ar, double os, const float* bv, int j) {
    return v_val_v(ar[j], os, bv != nullptr, bv ? bv[j] : 0.0f);
}

// Workgroups (row, part): the row's hd/2 rotation angles are computed once
// per workgroup into LDS (pos / theta^(2d/hd), cos, sin in fp64: the same
// values for every Q and K head), then its threads stride over the row's Q
// pairs, K pairs and V elements.  Many rows (prefill): one part per row; few
// rows (decode): a row's items spread over several workgroups.
constexpr int kRopeMaxHalf = 128;  // head_dim <= 256

// With per-head norms the workgroup first forms the norm factor of every Q
// and K head of its row (one thread per head, the dimension-order chain) into
// LDS.
__global__ __launch_bounds__(256) void qkv_rope_kernel(
    const int32_t* __restrict__ acc, const float* __restrict__ amax, float sq, float sk, float sv,
    const float* __restrict__ bq, const float* __restrict__ bk, const float* __restrict__ bv, int batch,
    int seq, const int* __restrict__ pos0, int msl, int heads, int kv_heads, int hd, double theta,
    double* __restrict__ q, float* __restrict__ cache_k, float* __restrict__ cache_v, QkNorm qk) {
    __shared__ double rc[kRopeMaxHalf], rs[kRopeMaxHalf];
    __shared__ double inv_s[kQkNormMaxHeads];
    const int half = hd >> 1;
    const int q_dim = heads * hd, kv_dim = kv_heads * hd;
    const int qp = heads * half, kp = kv_heads * half;
    const int per_row = qp + kp + kv_dim;
    const int row = blockIdx.x;  // token row b*seq + s
    const int b = row / seq, s = row % seq;
    const int base = *pos0;
    const int pos = base + s;
    for (int d = threadIdx.x; d < half; d += blockDim.x) rope_angle(pos, d, hd, theta, &rc[d], &rs[d]);
    const int32_t* ar = acc + (size_t)row * (q_dim + 2 * kv_dim);
    const float am = amax[row];
    const double osq = output_scale(sq, am), osk = output_scale(sk, am), osv = output_scale(sv, am);
    const bool qn = qk.q != nullptr, kn = qk.k != nullptr;
    if (qn || kn) {  // uniform
        for (int t = threadIdx.x; t < heads + kv_heads; t += blockDim.x) {
            if (t < heads) {
                if (qn) inv_s[t] = qk_inv_rms(head_sum_sq<false>(ar, osq, bq, t * hd, hd), hd, qk.eps);
            } else if (kn) {
                const int h = t - heads;
                inv_s[t] = qk_inv_rms(head_sum_sq<true>(ar + q_dim, osk, bk, h * hd, hd), hd, qk.eps);
            }
        }
    }
    __syncthreads();
    cache_k += (size_t)b * msl * kv_dim;
    cache_v += (size_t)b * msl * kv_dim;
    const bool latest = pos + msl >= base + seq;
    double* qr = q + (size_t)row * q_dim;
    float* kr = cache_k + (size_t)(pos % msl) * kv_dim;
    float* vr = cache_v + (size_t)(pos % msl) * kv_dim;
    for (int r = threadIdx.x + blockIdx.y * blockDim.x; r < per_row; r += blockDim.x * gridDim.y) {
        if (r < qp) {
            const int h = r / half, d = r % half;
            const int j0 = h * hd + d, j1 = j0 + half;
            const HeadNorm hn = head_norm(qn, qn ? inv_s[h] : 0.0, qk.q, qk.q_len, heads, hd, h, d,
                                          d + half);
            q_pair(ar, osq, bq, j0, j1, rc[d], rs[d], &qr[j0], &qr[j1], hn);
        } else if (r < qp + kp) {
            const int t = r - qp;
            const int h = t / half, d = t % half;
            const int j0 = h * hd + d, j1 = j0 + half;
            const HeadNorm hn = head_norm(kn, kn ? inv_s[heads + h] : 0.0, qk.k, qk.k_len, kv_heads, hd,
                                          h, d, d + half);
            if (latest) k_pair(ar + q_dim, osk, bk, j0, j1, rc[d], rs[d], &kr[j0], &kr[j1], hn);
        } else {
            const int j = r - qp - kp;
            if (latest) vr[j] = v_val(ar + q_dim + kv_dim, osv, bv, j);
        }
    }
}

hipError_t launch_qkv_rope(const int32_t* acc, const float* amax, float sq, float sk, float sv,
                           const float* bq, const float* bk, const float* bv, int batch, int seq,
                           const int* pos0, int msl, int heads, int kv_heads, int hd, double theta,
                           double* q, float* cache_k, float* cache_v, hipStream_t s, const QkNorm& qk) {
    const long rows = (long)batch * seq;
    if (rows <= 0) return hipSuccess;
    if (hd % 2 != 0 || hd / 2 > kRopeMaxHalf) return hipErrorInvalidValue;
    if ((qk.q || qk.k) && heads + kv_heads > kQkNormMaxHeads) return hipErrorInvalidValue;
    if (theta <= 0.0) theta = 10000.0;
    const int per_row = heads * (hd / 2) + kv_heads * (hd / 2) + kv_heads * hd;
    const int parts = rows >= 256 ? 1 : ceil_div(per_row, 256);
    hipLaunchKernelGGL(qkv_rope_kernel, dim3((unsigned)rows, parts), dim3(256), 0, s, acc, amax, sq,
                       sk, sv, bq, bk, bv, batch, seq, pos0, msl, heads, kv_heads, hd, theta, q,
                       cache_k, cache_v, qk);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// Attention (poly/mha.go:316-354).  For query row (b, s) at position pos0+s,
// head h (GQA group kvh = h / (heads / kv_heads)), over positions
// kp = 0..pos0+s of the sequence's ring (row kp; the host keeps every
// position below msl, so no wrap occurs):
//   score_kp = (sum over d in order of q_d * k_kp,d) * (1/sqrt(hd))
//   max from -1e9; p_kp = exp(score_kp - max); expSum = sum over kp in order
//   out_d = (sum over kp in order of p_kp * v_kp,d) / expSum
// STRICT keeps every fp64 sum in that order; fast splits the position sums
// into fixed slices combined in slice order.  The scores of one query live in
// LDS: `span` bounds the positions a launch may see; a query past it gets NaN
// rows (the host checks the span first, so a valid call never does).
//
// Two launch shapes: few query rows (decode) use a scores kernel with one
// wave per 64 positions and a softmax/PV kernel of 1024 threads per head;
// many rows (prefill) use one fused 256-thread workgroup per (head, row).
// ------------------------------------------------------------------------

// Sequential fp64 dot of a K row (fp32) with q (fp64 in LDS), d in order.
// Loads run 16 floats ahead of the chain.
__device__ __forceinline__ double dot_q_k(const double* __restrict__ qs,
                                          const float* __restrict__ kr, int hd) {
    double dot = 0.0;
    int d = 0;
    for (; d + 16 <= hd; d += 16) {
        const float4 a = *(const float4*)(kr + d);
        const float4 b = *(const float4*)(kr + d + 4);
        const float4 c = *(const float4*)(kr + d + 8);
        const float4 e = *(const float4*)(kr + d + 12);
        dot += qs[d] * (double)a.x;
        dot += qs[d + 1] * (double)a.y;
        dot += qs[d + 2] * (double)a.z;
        dot += qs[d + 3] * (double)a.w;
        dot += qs[d + 4] * (double)b.x;
        dot += qs[d + 5] * (double)b.y;
        dot += qs[d + 6] * (double)b.z;
        dot += qs[d + 7] * (double)b.w;
        dot += qs[d + 8] * (double)c.x;
        dot += qs[d + 9] * (double)c.y;
        dot += qs[d + 10] * (double)c.z;
        dot += qs[d + 11] * (double)c.w;
        dot += qs[d + 12] * (double)e.x;
        dot += qs[d + 13] * (double)e.y;
        dot += qs[d + 14] * (double)e.z;
        dot += qs[d + 15] * (double)e.w;
    }
    for (; d < hd; d += 4) {
        const float4 a = *(const float4*)(kr + d);
        dot += qs[d] * (double)a.x;
        dot += qs[d + 1] * (double)a.y;
        dot += qs[d + 2] * (double)a.z;
        dot += qs[d + 3] * (double)a.w;
    }
    return dot;
}

// sum over kp in [k0, k1) in order of p[kp] * v[kp * ld] (v already offset by d);
// eight V loads are issued ahead of the chain.
__device__ __forceinline__ double pv_chain(const double* __restrict__ p, const float* __restrict__ v,
                                           size_t ld, int k0, int k1, double sum) {
    int kp = k0;
    for (; kp + 8 <= k1; kp += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = v[(size_t)(kp + j) * ld];
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += p[kp + j] * (double)t[j];
    }
    for (; kp < k1; ++kp) sum += p[kp] * (double)v[(size_t)kp * ld];
    return sum;
}

// max over [0, L) of LDS values, starting from -1e9 (NaN never wins)
template <int T>
__device__ __forceinline__ double block_max_f64(double v, double* red) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int w = T >> 1; w > 0; w >>= 1) {
        if (threadIdx.x < w) {
            const double o = red[threadIdx.x + w];
            if (o > red[threadIdx.x]) red[threadIdx.x] = o;
        }
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

template <int T>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int w = T >> 1; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

// softmax + PV over p[0..L) (scores in LDS on entry, probabilities after), T threads.
template <int STRICT, int T>
__device__ void softmax_pv(double* p, int L, const float* __restrict__ vbase, size_t ld, int hd,
                           double* red, double* orow) {
    double mx = -1e9;
    for (int kp = threadIdx.x; kp < L; kp += T) {
        const double v = p[kp];
        if (v > mx) mx = v;
    }
    mx = block_max_f64<T>(mx, red);
    for (int kp = threadIdx.x; kp < L; kp += T) p[kp] = exp(p[kp] - mx);
    __syncthreads();
    __shared__ double exp_sum_sh;
    if (STRICT) {
        // value chains on the first hd lanes, the expSum chain on the last wave
        double sum = 0.0;
        if ((int)threadIdx.x < hd) sum = pv_chain(p, vbase + threadIdx.x, ld, 0, L, 0.0);
        if ((int)threadIdx.x == T - 64) {
            double es = 0.0;
            for (int kp = 0; kp < L; ++kp) es += p[kp];
            exp_sum_sh = es;
        }
        __syncthreads();
        if ((int)threadIdx.x < hd) orow[threadIdx.x] = sum / exp_sum_sh;
    } else {
        double es = 0.0;
        for (int kp = threadIdx.x; kp < L; kp += T) es += p[kp];
        es = block_sum_f64<T>(es, red);
        const int slices = T / hd;  // hd <= 256 <= T
        const int d = threadIdx.x % hd, sl = threadIdx.x / hd;
        const int chunk = (L + slices - 1) / slices;
        double sum = 0.0;
        if (sl < slices) {
            const int k0 = min(L, sl * chunk), k1 = min(L, k0 + chunk);
            sum = pv_chain(p, vbase + d, ld, k0, k1, 0.0);
        }
        red[threadIdx.x] = sum;
        __syncthreads();
        if ((int)threadIdx.x < hd) {
            double t = red[threadIdx.x];
            for (int k = 1; k < slices; ++k) t = t + red[k * hd + threadIdx.x];
            orow[threadIdx.x] = t / es;
        }
    }
}

// fused: one workgroup per (head, row); grid (heads, seq, batch)
template <int STRICT>
__global__ __launch_bounds__(256) void attention_kernel(const double* __restrict__ q,
                                                        const float* __restrict__ cache_k,
                                                        const float* __restrict__ cache_v,
                                                        const int* __restrict__ pos0, int msl,
                                                        int span, int heads, int kv_heads, int hd,
                                                        double* __restrict__ out) {
    extern __shared__ double lds[];  // q[hd] then scores[span]
    __shared__ double red[256];
    const int h = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
    const int row = b * gridDim.y + s;
    const int q_dim = heads * hd, kv_dim = kv_heads * hd;
    const int kvh = h / (heads / kv_heads);
    const int L = *pos0 + s + 1;
    double* orow = out + (size_t)row * q_dim + (size_t)h * hd;
    if (L > span) {
        for (int d = threadIdx.x; d < hd; d += 256) orow[d] = __builtin_nan("");
        return;
    }
    const float* kb = cache_k + (size_t)b * msl * kv_dim + (size_t)kvh * hd;
    const float* vb = cache_v + (size_t)b * msl * kv_dim + (size_t)kvh * hd;
    double* qs = lds;
    double* p = lds + ((hd + 1) & ~1);
    const double* qrow = q + (size_t)row * q_dim + (size_t)h * hd;
    for (int d = threadIdx.x; d < hd; d += 256) qs[d] = qrow[d];
    __syncthreads();
    const double scale = 1.0 / sqrt((double)hd);
    for (int kp = threadIdx.x; kp < L; kp += 256) p[kp] = dot_q_k(qs, kb + (size_t)kp * kv_dim, hd) * scale;
    __syncthreads();
    softmax_pv<STRICT, 256>(p, L, vb, kv_dim, hd, red, orow);
}

// ---- prefill path: query tiles -------------------------------------------
// Strict prefill attention.  One workgroup per (head, tile of kTileQ
// consecutive queries, sequence).  K and V chunks of kChunkP positions are
// staged through LDS in fp64 (converted once as they are staged; the next
// chunk is loaded into registers while the current one is used, and the
// barriers between chunks wait for LDS operations only, so those loads stay
// in flight), so each cached row is read once per tile instead of once per
// query.  Pass 1 forms every score of the tile, each lane a 2 x 2 block of
// d-order chains (queries 2 qp, 2 qp + 1 x chunk positions pp, pp + 16),
// reading two dimensions of a Q or K row per 16-byte LDS read (row pitch
// HD + 2: the 16 positions a wave reads at one d fall in distinct banks).
// It keeps each query's maximum and stores the scores in `sc` (rows x heads x
// span).  Pass 2 reads them back, takes p = exp(score - max), adds expSum on
// one lane per query and sum(p * v) on one lane per (four queries, column
// pair or pairs: d = 2l, 2l+1 and 64+2l, 64+2l+1, so a wave's 16-byte value
// reads are contiguous), all in position order; a chunk that every query of
// the tile sees whole is walked position by position for a lane's four
// queries at once (each value read serves four queries), and wave 0 adds the
// expSum chains in the same walk.  Every sum
// therefore has the reference's order and roundings (a product, then a sum,
// each rounded): exact.  Positions past a query's own position are skipped
// (never added).
constexpr int kTileQ = 32;
constexpr int kAttnFastQt = 2;  // 16-query tiles per workgroup of the fast prefill kernel
constexpr int kChunkP = 32;

template <int HD>
struct TileLds {
    static constexpr int QP = HD + 2;  // q row pitch (doubles): the query pairs' rows in distinct banks
    static constexpr int KP = HD + 2;  // K row pitch (doubles): 16 consecutive rows in distinct banks
    static constexpr int PP = kChunkP + 2;  // probability row pitch: 16-byte pairs
    double q[kTileQ * QP];
    union {
        double k[kChunkP * KP];        // pass 1: K chunk, position-major
        double v[kChunkP * HD];        // pass 2: V chunk, position-major
    };
    double p[kTileQ * PP];
    double es[kTileQ];
};

// Workgroup barrier for LDS only: this wave's LDS operations have completed
// (lgkmcnt(0)), then s_barrier.  Unlike __syncthreads it does not wait for
// the wave's outstanding global loads (its release fence would), so a chunk
// prefetched into registers stays in flight across it.  The asm statements
// keep the compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void tile_lds_barrier() {
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
}

// PV over one chunk that every query of the tile sees whole: position by
// position for the lane's four queries (each value read serves all four);
// with ES the lane also adds its expSum query's probabilities (row `pe`) in
// position order.  Each (query, column) chain adds in position order.
template <int HD, bool ES>
__device__ __forceinline__ void tile_pv_whole(const double* __restrict__ pr, const double* __restrict__ pe,
                                              const double* __restrict__ vr, double (&acc)[4][HD / 32],
                                              double& es) {
    constexpr int DB = HD / 32;
    constexpr int PP = kChunkP + 2;
#pragma unroll 2
    for (int kk = 0; kk < kChunkP; kk += 2) {
        double2 pk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pk[i] = *(const double2*)(pr + i * PP + kk);
        if constexpr (ES) {
            const double2 e = *(const double2*)(pe + kk);
            es += e.x;
            es += e.y;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            double v[DB];
            const double2 va = *(const double2*)(vr + (kk + u) * HD);
            v[0] = va.x;
            v[1] = va.y;
            if constexpr (DB == 4) {
                const double2 vc = *(const double2*)(vr + (kk + u) * HD + 64);
                v[2] = vc.x;
                v[3] = vc.y;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const double pv = u ? pk[i].y : pk[i].x;
#pragma unroll
                for (int j = 0; j < DB; ++j) acc[i][j] = acc[i][j] + pv * v[j];
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(256) void attn_tile_kernel(const double* __restrict__ q,
                                                        const float* __restrict__ cache_k,
                                                        const float* __restrict__ cache_v,
                                                        const int* __restrict__ pos0, int msl,
                                                        int span, int heads, int kv_heads, int seq,
                                                        double* __restrict__ sc_all,
                                                        double* __restrict__ out) {
    using Lds = TileLds<HD>;
    constexpr int QP = Lds::QP, KP = Lds::KP, PP = Lds::PP;
    constexpr int DB = HD / 32;                       // value columns per PV lane
    constexpr int F4 = kChunkP * HD / 4 / 256;        // float4 per thread per chunk
    static_assert(F4 >= 1 && kChunkP * HD == F4 * 4 * 256, "chunk geometry");
    static_assert(DB == 2 || DB == 4, "head_dim 64 or 128");
    __shared__ __align__(16) Lds sm;
    const int tid = threadIdx.x;
    const int h = blockIdx.x;
    const int tile = gridDim.y - 1 - blockIdx.y;  // longest tiles first
    const int b = blockIdx.z;
    const int s0 = tile * kTileQ;
    const int nq = min(kTileQ, seq - s0);
    const int base = *pos0;
    const int q_dim = heads * HD, kv_dim = kv_heads * HD;
    const int kvh = h / (heads / kv_heads);
    const size_t row0 = (size_t)b * seq + s0;
    if (base + s0 + nq > span) {
        for (int i = tid; i < nq * HD; i += 256)
            out[(row0 + i / HD) * q_dim + (size_t)h * HD + i % HD] = __builtin_nan("");
        return;
    }
    const int nch = (base + s0 + nq + kChunkP - 1) / kChunkP;
    const float* kb = cache_k + (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    const float* vb = cache_v + (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    for (int i = tid; i < kTileQ * HD; i += 256) {
        const int qi = i / HD;
        sm.q[qi * QP + i % HD] = qi < nq ? q[(row0 + qi) * q_dim + (size_t)h * HD + i % HD] : 0.0;
    }
    // chunk loads: branch-free (rows clamped into the ring); thread t takes
    // float4 (t + 256 j): position e / HD, columns e % HD .. +3
    float4 rk[F4];
#define LAMD_TILE_LOAD(SRC, C)                                                      \
    _Pragma("unroll") for (int j = 0; j < F4; ++j) {                                \
        const int e = (tid + j * 256) * 4;                                          \
        const int k = min((C) * kChunkP + e / HD, msl - 1);                         \
        rk[j] = *(const float4*)((SRC) + (size_t)k * kv_dim + e % HD);              \
    }
    // score lanes: queries qa = 2*qp, qa+1 x chunk positions pp, pp+16; their
    // scores live at sca[k], sca[sc_next + k] (rows qa, qa+1 of the tile)
    const int qp = tid >> 4, pp = tid & 15;
    const int qa = 2 * qp;
    const int lim_a = base + s0 + qa;  // last position query qa sees
    const double scale = 1.0 / sqrt((double)HD);
    // rows past the tile's last query (a partial tile) neither store nor use
    // scores; their reads are clamped onto the last query's row
    const bool w0 = qa < nq, w1 = qa + 1 < nq;
    double* sca = sc_all + ((row0 + min(qa, nq - 1)) * heads + h) * (size_t)span;
    const size_t sc_next = w1 ? (size_t)heads * span : 0;  // row qa+1

    // ---- pass 1: scores and maxima ---------------------------------------
    double m0 = -1e9, m1 = -1e9;
    LAMD_TILE_LOAD(kb, 0)
    __syncthreads();  // Q rows staged
    for (int c = 0; c < nch; ++c) {
#pragma unroll
        for (int j = 0; j < F4; ++j) {  // K chunk: k[position][d]
            const int e = (tid + j * 256) * 4;
            double* d = &sm.k[(e / HD) * KP + e % HD];
            *(double2*)d = make_double2((double)rk[j].x, (double)rk[j].y);
            *(double2*)(d + 2) = make_double2((double)rk[j].z, (double)rk[j].w);
        }
        LAMD_TILE_LOAD(kb, c + 1)  // prefetch (clamped past the last chunk)
        tile_lds_barrier();        // chunk c staged
        double d00 = 0.0, d01 = 0.0, d10 = 0.0, d11 = 0.0;
        const double* q0 = &sm.q[qa * QP];
        const double* q1 = q0 + QP;
        const double* k0 = &sm.k[pp * KP];
        const double* k1 = k0 + 16 * KP;
#pragma unroll 8
        for (int d = 0; d < HD; d += 2) {
            const double2 a0 = *(const double2*)(q0 + d), a1 = *(const double2*)(q1 + d);
            const double2 b0 = *(const double2*)(k0 + d), b1 = *(const double2*)(k1 + d);
            d00 += a0.x * b0.x;
            d01 += a0.x * b1.x;
            d10 += a1.x * b0.x;
            d11 += a1.x * b1.x;
            d00 += a0.y * b0.y;
            d01 += a0.y * b1.y;
            d10 += a1.y * b0.y;
            d11 += a1.y * b1.y;
        }
        const double s00 = d00 * scale, s01 = d01 * scale, s10 = d10 * scale, s11 = d11 * scale;
        const int k = c * kChunkP + pp;  // positions k and k + 16
        if (k < span) {
            if (w0) sca[k] = s00;
            if (w1) sca[sc_next + k] = s10;
        }
        if (k + 16 < span) {
            if (w0) sca[k + 16] = s01;
            if (w1) sca[sc_next + k + 16] = s11;
        }
        if (k <= lim_a && s00 > m0) m0 = s00;
        if (k + 16 <= lim_a && s01 > m0) m0 = s01;
        if (k <= lim_a + 1 && s10 > m1) m1 = s10;
        if (k + 16 <= lim_a + 1 && s11 > m1) m1 = s11;
        tile_lds_barrier();  // chunk c read before chunk c + 1 overwrites it
    }
    // maximum over the 16 lanes of each query pair (order-free)
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
        const double o0 = __shfl_xor(m0, off, 16), o1 = __shfl_xor(m1, off, 16);
        m0 = o0 > m0 ? o0 : m0;
        m1 = o1 > m1 ? o1 : m1;
    }
    // ---- pass 2: probabilities, expSum, PV --------------------------------
    // PV lanes: queries 4*pq .. +3; columns 2*dl, 2*dl+1 (and 64 + those
    // when HD = 128)
    const int pq = tid >> 5, dl = tid & 31;
    double acc[4][DB];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < DB; ++j) acc[i][j] = 0.0;
    double es = 0.0;  // lane tid < kTileQ: query tid
    // this lane's four scores of chunk c (clamped past the end; surplus unused)
    double sv00, sv01, sv10, sv11;
    auto load_scores = [&](int c) {
        const int k = min(c, nch - 1) * kChunkP + pp;
        const int k0c = min(k, span - 1), k1c = min(k + 16, span - 1);
        sv00 = sca[k0c];
        sv01 = sca[k1c];
        sv10 = sca[sc_next + k0c];
        sv11 = sca[sc_next + k1c];
    };
    // the stored scores are read back by the lanes that wrote them; the full
    // barrier also orders those stores before the loads
    __syncthreads();
    LAMD_TILE_LOAD(vb, 0)
    load_scores(0);
    // every query of the tile sees every position of chunks before this one
    const int whole_ch = (base + s0 + 1) / kChunkP;
    const double* pe = &sm.p[min(tid, kTileQ - 1) * PP];  // expSum row (wave 0)
    for (int c = 0; c < nch; ++c) {
#pragma unroll
        for (int j = 0; j < F4; ++j) {  // V chunk, row-major: v[position][d]
            const int e = (tid + j * 256) * 4;
            double* d = &sm.v[(e / HD) * HD + e % HD];
            *(double2*)d = make_double2((double)rk[j].x, (double)rk[j].y);
            *(double2*)(d + 2) = make_double2((double)rk[j].z, (double)rk[j].w);
        }
        const int k = c * kChunkP + pp;
        sm.p[qa * PP + pp] = k <= lim_a ? exp(sv00 - m0) : 0.0;
        sm.p[qa * PP + pp + 16] = k + 16 <= lim_a ? exp(sv01 - m0) : 0.0;
        sm.p[(qa + 1) * PP + pp] = k <= lim_a + 1 ? exp(sv10 - m1) : 0.0;
        sm.p[(qa + 1) * PP + pp + 16] = k + 16 <= lim_a + 1 ? exp(sv11 - m1) : 0.0;
        LAMD_TILE_LOAD(vb, c + 1)  // next V chunk
        load_scores(c + 1);
        tile_lds_barrier();  // chunk c's values and probabilities staged
        const int kc = c * kChunkP;
        const double* vr = &sm.v[2 * dl];
        if (c < whole_ch) {  // wave-uniform
            if (tid < 64)
                tile_pv_whole<HD, true>(&sm.p[4 * pq * PP], pe, vr, acc, es);
            else
                tile_pv_whole<HD, false>(&sm.p[4 * pq * PP], pe, vr, acc, es);
        } else {
            if (tid < kTileQ) {
                const int lim = base + s0 + tid;
                for (int kk = 0; kk < kChunkP; kk += 2) {
                    const double2 pk = *(const double2*)(pe + kk);
                    if (kc + kk <= lim) es += pk.x;
                    if (kc + kk + 1 <= lim) es += pk.y;
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int qi = 4 * pq + i;
                const int n = min(kChunkP, base + s0 + qi + 1 - kc);  // valid positions of this chunk
                for (int kk = 0; kk < n; ++kk) {
                    const double pk = sm.p[qi * PP + kk];
                    double v[DB];
                    const double2 va = *(const double2*)(vr + kk * HD);
                    v[0] = va.x;
                    v[1] = va.y;
                    if constexpr (DB == 4) {
                        const double2 vc = *(const double2*)(vr + kk * HD + 64);
                        v[2] = vc.x;
                        v[3] = vc.y;
                    }
#pragma unroll
                    for (int j = 0; j < DB; ++j) acc[i][j] = acc[i][j] + pk * v[j];
                }
            }
        }
        tile_lds_barrier();  // chunk c's reads done before chunk c + 1 is staged
    }
#undef LAMD_TILE_LOAD
    if (tid < kTileQ) sm.es[tid] = es;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int qi = 4 * pq + i;
        if (qi < nq) {
            const double e = sm.es[qi];
#pragma unroll
            for (int j = 0; j < DB; ++j)
                out[(row0 + qi) * q_dim + (size_t)h * HD + 64 * (j >> 1) + 2 * dl + (j & 1)] = acc[i][j] / e;
        }
    }
}

// ---- prefill path, fast mode: fp64 MFMA tiles -------------------------------
// Same tiling and two passes as attn_tile_kernel, with the score and value
// sums on v_mfma_f64_16x16x4f64 (lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; element v of lane l is D[4v + l/16][l%16]).  Each MFMA adds
// four products at once, so the d-order and position-order chains become
// 4-wide blocks: fast mode only.  Masked positions enter the value MFMAs with
// p = 0 (the cached rows they meet are finite).  The Q fragments stay in
// registers for the whole tile.  4 waves: for the scores, wave w owns query
// tile w/2 and position tile w%2 of a 32 x 32 block; for the values, query
// tile w/2 and HD/32 tiles of 16 value columns.
typedef double v4d __attribute__((ext_vector_type(4)));

// One-pass fast prefill attention (fast mode).  The two-pass kernel below
// keeps every score in a workspace between its passes (rows x heads x span
// fp64: 2.7 GB per layer at 8 x 2048 tokens); this one keeps a running row
// maximum instead (online softmax).  Each wave owns 16 queries of one head and
// computes, per 32-position chunk, the transposed scores S^T = K Q^T on the
// fp64 matrix cores: lane (lr, lg) then holds query lr's scores at positions
// 16 kt + 4 v + lg, which is exactly the B operand layout of O^T = V^T P^T.
// So the probabilities never leave registers, a query's running maximum and
// sum live in the four lanes that share lr (two shuffles per chunk), and the
// output rows are rescaled lane-locally by exp(old max - new max) when the
// maximum grows.  The HPW heads of a workgroup share one KV head: every chunk
// of K and V is staged once (converted to fp64) for all four waves.  The sums
// differ in order from loom's sequential ones (a fixed order: deterministic),
// within 1e-12 of the row scale.
template <int HD, int HPW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_flash_mfma_kernel(
    const double* __restrict__ q, const float* __restrict__ cache_k,
    const float* __restrict__ cache_v, const int* __restrict__ pos0, int msl, int span, int heads,
    int kv_heads, int seq, double* __restrict__ out) {
    constexpr int TQ = 16 * (4 / HPW);  // queries per workgroup
    constexpr int NM = HD / 4;          // k-steps of a score tile
    constexpr int NT = HD / 16;         // output tiles of 16 head columns
    constexpr int F2 = kChunkP * HD / 2 / 256;  // float2 loads per thread and operand
    static_assert(HPW == 1 || HPW == 2 || HPW == 4, "heads per workgroup");
    static_assert(F2 >= 1 && kChunkP * HD == F2 * 2 * 256, "chunk geometry");
    // K rows KP doubles apart (16 rows x 4 columns per read: 2*KP = 4 mod 64
    // banks), V rows VP (4 rows x 16 columns: 2*VP = 32 mod 64): both reads
    // are conflict-free per half wave.
    constexpr int KP = HD + 2, VP = HD + 16;
    __shared__ double kd[kChunkP * KP];
    __shared__ double vd[kChunkP * VP];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int h = blockIdx.x * HPW + wave % HPW;
    const int tile = gridDim.y - 1 - blockIdx.y;  // long rows first
    const int b = blockIdx.z;
    const int s0 = tile * TQ;
    const int nq = min(TQ, seq - s0);
    const int base = *pos0;
    const int q_dim = heads * HD, kv_dim = kv_heads * HD;
    const int kvh = blockIdx.x * HPW / (heads / kv_heads);
    const size_t row0 = (size_t)b * seq + s0;
    if (base + s0 + nq > span) {
        for (int i = tid; i < nq * HD * HPW; i += 256)
            out[(row0 + i / (HD * HPW)) * q_dim + (size_t)blockIdx.x * HPW * HD + i % (HD * HPW)] =
                __builtin_nan("");
        return;
    }
    const int nch = (base + s0 + nq + kChunkP - 1) / kChunkP;
    const float* kb = cache_k + (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    const float* vb = cache_v + (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    // staging: consecutive lanes take consecutive column pairs of a row, so
    // the fp64 pairs they write to LDS are consecutive 16-byte words
    float2 rk[F2], rv[F2];
    auto load = [&](int c) {
#pragma unroll
        for (int j = 0; j < F2; ++j) {
            const int e = (tid + j * 256) * 2;
            const size_t off = (size_t)min(c * kChunkP + e / HD, msl - 1) * kv_dim + e % HD;
            rk[j] = *(const float2*)(kb + off);
            rv[j] = *(const float2*)(vb + off);
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int j = 0; j < F2; ++j) {
            const int e = (tid + j * 256) * 2;
            double* dk = &kd[(e / HD) * KP + e % HD];
            double* dv = &vd[(e / HD) * VP + e % HD];
            dk[0] = (double)rk[j].x;
            dk[1] = (double)rk[j].y;
            dv[0] = (double)rv[j].x;
            dv[1] = (double)rv[j].y;
        }
    };
    const int qi = 16 * (wave / HPW) + lr;  // this lane's query in the tile
    const int qpos = base + s0 + qi;
    // B operand of S^T: Q^T[4 m + lg][lr] = Q[query lr][4 m + lg]
    double qa[NM];
    {
        const double* src = q + (row0 + min(qi, nq - 1)) * q_dim + (size_t)h * HD + lg;
#pragma unroll
        for (int m = 0; m < NM; ++m) qa[m] = qi < nq ? src[4 * m] : 0.0;
    }
    const double scale = 1.0 / sqrt((double)HD);
    double mrun = -1e9;  // running maximum of query qi's scores
    double lsum = 0.0;   // this lane's share of their exponential sum
    v4d o[NT];           // o[t][v] = O[query qi][16 t + 4 v + lg]
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = v4d{0.0, 0.0, 0.0, 0.0};
    load(0);
    for (int c = 0; c < nch; ++c) {
        __syncthreads();  // the previous chunk's reads of kd and vd are done
        store();
        load(c + 1);  // in flight during this chunk's products
        __syncthreads();
        v4d sa[2] = {v4d{0.0, 0.0, 0.0, 0.0}, v4d{0.0, 0.0, 0.0, 0.0}};
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const double ak = kd[(16 * kt + lr) * KP + 4 * m + lg];
                sa[kt] = __builtin_amdgcn_mfma_f64_16x16x4f64(ak, qa[m], sa[kt], 0, 0, 0);
            }
        // sa[kt][v] = S[query qi][position c*32 + 16 kt + 4 v + lg]
        double sv[2][4];
        bool ok[2][4];
        double cm = -1e9;  // NaN never wins
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                ok[kt][v] = c * kChunkP + 16 * kt + 4 * v + lg <= qpos;
                sv[kt][v] = sa[kt][v] * scale;
                if (ok[kt][v] && sv[kt][v] > cm) cm = sv[kt][v];
            }
        {
            double t = __shfl_xor(cm, 16);
            cm = t > cm ? t : cm;
            t = __shfl_xor(cm, 32);
            cm = t > cm ? t : cm;
        }
        if (cm > mrun) {
            const double alpha = exp(mrun - cm);
            lsum *= alpha;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) o[t][v] *= alpha;
            mrun = cm;
        }
        double p[2][4];  // exp(-inf) = 0 at masked positions: no branch
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                p[kt][v] = exp(ok[kt][v] ? sv[kt][v] - mrun : -__builtin_inf());
                lsum += p[kt][v];
            }
        // O^T += V^T P^T: A = V[position 16 kt + 4 m + lg][16 t + lr], B = p[kt][m]
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const double av = vd[(16 * kt + 4 * m + lg) * VP + 16 * t + lr];
                    o[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(av, p[kt][m], o[t], 0, 0, 0);
                }
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (qi < nq) {
        double* orow = out + (row0 + qi) * q_dim + (size_t)h * HD;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) orow[16 * t + 4 * v + lg] = o[t][v] / lsum;
    }
}

template <int HD, int QT>
__global__ __launch_bounds__(256) void attn_tile_mfma_kernel(const double* __restrict__ q,
                                                             const float* __restrict__ cache_k,
                                                             const float* __restrict__ cache_v,
                                                             const int* __restrict__ pos0, int msl,
                                                             int span, int heads, int kv_heads,
                                                             int seq, double* __restrict__ sc_all,
                                                             double* __restrict__ out) {
    // QT 16-query tiles per workgroup; WPQ waves share one query tile: for
    // the scores each takes KTW of the chunk's two 16-position tiles, for the
    // values DT of the HD/16 value tiles.
    constexpr int TQ = 16 * QT;
    constexpr int WPQ = 4 / QT;
    constexpr int KTW = 2 / WPQ;
    constexpr int NM = HD / 4;         // score MFMAs along d
    constexpr int DT = HD / 16 / WPQ;  // value tiles (16 columns) per wave
    constexpr int F4 = kChunkP * HD / 4 / 256;
    static_assert(QT == 2 || QT == 4, "32 or 64 queries per workgroup");
    static_assert(F4 >= 1 && kChunkP * HD == F4 * 4 * 256, "chunk geometry");
    // The K or V chunk, converted to fp64 once as it is staged.  K rows are
    // KP doubles apart (pass 1 reads 16 rows x 4 columns: 2*KP = 4 mod 64
    // banks), V rows VP (pass 2 reads 4 rows x 16 columns: 2*VP = 32 mod 64),
    // so both read patterns fill the banks without conflicts.
    constexpr int KP = HD + 2, VP = HD + 16;
    __shared__ double kvd[kChunkP * VP];
    __shared__ double pt[TQ][kChunkP + 1];
    __shared__ double red[WPQ * TQ];  // the waves' row maxima, later the expSums
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int h = blockIdx.x;
    const int tile = gridDim.y - 1 - blockIdx.y;
    const int b = blockIdx.z;
    const int s0 = tile * TQ;
    const int nq = min(TQ, seq - s0);
    const int base = *pos0;
    const int q_dim = heads * HD, kv_dim = kv_heads * HD;
    const int kvh = h / (heads / kv_heads);
    const size_t row0 = (size_t)b * seq + s0;
    if (base + s0 + nq > span) {
        for (int i = tid; i < nq * HD; i += 256)
            out[(row0 + i / HD) * q_dim + (size_t)h * HD + i % HD] = __builtin_nan("");
        return;
    }
    const int nch = (base + s0 + nq + kChunkP - 1) / kChunkP;
    const float* kb = cache_k + (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    const float* vb = cache_v + (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    float4 rk[F4];
    auto load = [&](const float* src, int c) {
#pragma unroll
        for (int j = 0; j < F4; ++j) {
            const int e = (tid + j * 256) * 4;
            const int k = min(c * kChunkP + e / HD, msl - 1);
            rk[j] = *(const float4*)(src + (size_t)k * kv_dim + e % HD);
        }
    };
    auto store = [&](int pitch) {
#pragma unroll
        for (int j = 0; j < F4; ++j) {
            const int e = (tid + j * 256) * 4;
            double* d = &kvd[(e / HD) * pitch + e % HD];
            d[0] = (double)rk[j].x;
            d[1] = (double)rk[j].y;
            d[2] = (double)rk[j].z;
            d[3] = (double)rk[j].w;
        }
    };
    const int qt = wave / WPQ, slot = wave % WPQ, kt0 = slot * KTW;
    // Q fragment: Q[16 qt + lr][4 m + lg]
    double qa[NM];
    {
        const int qr = 16 * qt + lr;
        const double* src = q + (row0 + min(qr, nq - 1)) * q_dim + (size_t)h * HD + lg;
#pragma unroll
        for (int m = 0; m < NM; ++m) qa[m] = qr < nq ? src[4 * m] : 0.0;
    }
    const double scale = 1.0 / sqrt((double)HD);
    // this lane's score slots: rows qi(v) = 16 qt + 4 v + lg, positions 16 kt + lr
    double* scr[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int qi = 16 * qt + 4 * v + lg;
        scr[v] = sc_all + ((row0 + min(qi, nq - 1)) * heads + h) * (size_t)span;
    }

    // ---- pass 1 ---------------------------------------------------------------
    double mv[4] = {-1e9, -1e9, -1e9, -1e9};
    load(kb, 0);
    for (int c = 0; c < nch; ++c) {
        __syncthreads();
        store(KP);
        load(kb, c + 1);
        __syncthreads();
        v4d acc[KTW];
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) acc[kk] = v4d{0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int kk = 0; kk < KTW; ++kk) {
                const double bk = kvd[(16 * (kt0 + kk) + lr) * KP + 4 * m + lg];
                acc[kk] = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[m], bk, acc[kk], 0, 0, 0);
            }
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) {
            const int k = c * kChunkP + 16 * (kt0 + kk) + lr;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int qi = 16 * qt + 4 * v + lg;
                const double sv = acc[kk][v] * scale;
                if (qi < nq && k < span) scr[v][k] = sv;
                if (k <= base + s0 + qi && sv > mv[v]) mv[v] = sv;
            }
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            const double o = __shfl_xor(mv[v], off, 16);
            mv[v] = o > mv[v] ? o : mv[v];
        }
        if (lr == 0) red[slot * TQ + 16 * qt + 4 * v + lg] = mv[v];
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int qi = 16 * qt + 4 * v + lg;
        double mm = red[qi];
#pragma unroll
        for (int w = 1; w < WPQ; ++w) mm = red[w * TQ + qi] > mm ? red[w * TQ + qi] : mm;
        mv[v] = mm;
    }

    // ---- pass 2 ---------------------------------------------------------------
    v4d o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = v4d{0.0, 0.0, 0.0, 0.0};
    double es = 0.0;  // lane tid < TQ: query tid
    double sv[KTW][4];
    auto load_scores = [&](int c) {
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) {
            const int k = min(min(c, nch - 1) * kChunkP + 16 * (kt0 + kk) + lr, span - 1);
#pragma unroll
            for (int v = 0; v < 4; ++v) sv[kk][v] = scr[v][k];
        }
    };
    load(vb, 0);
    load_scores(0);
    const int dt0 = slot * DT;
    for (int c = 0; c < nch; ++c) {
        __syncthreads();  // previous chunk's values and probabilities read (and the maxima)
        store(VP);        // V chunk c
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) {
            const int k = c * kChunkP + 16 * (kt0 + kk) + lr;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int qi = 16 * qt + 4 * v + lg;
                pt[qi][16 * (kt0 + kk) + lr] = k <= base + s0 + qi ? exp(sv[kk][v] - mv[v]) : 0.0;
            }
        }
        load(vb, c + 1);
        load_scores(c + 1);
        __syncthreads();
        if (tid < TQ) {
#pragma unroll 8
            for (int kk = 0; kk < kChunkP; ++kk) es += pt[tid][kk];
        }
#pragma unroll
        for (int m = 0; m < kChunkP / 4; ++m) {
            const double a = pt[16 * qt + lr][4 * m + lg];
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const double bv = kvd[(4 * m + lg) * VP + 16 * (dt0 + t) + lr];
                o[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, bv, o[t], 0, 0, 0);
            }
        }
    }
    if (tid < TQ) red[tid] = es;
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int qi = 16 * qt + 4 * v + lg;
        if (qi < nq) {
            const double e = red[qi];
            double* orow = out + (row0 + qi) * q_dim + (size_t)h * HD;
#pragma unroll
            for (int t = 0; t < DT; ++t) orow[16 * (dt0 + t) + lr] = o[t][v] / e;
        }
    }
}

// ---- decode path (few query rows) ----------------------------------------
// Scratch layout per (row, head): scores[span], chunk maxima cmax[nchunk]
// (64 positions per chunk on the strict path, 32 on the fast GQA path), and
// for the fast path the chunk-local partial sums part[nchunk][hd] and partial
// expSums pes[nchunk].

struct DecodeScratch {
    double* scores;  // rows x heads x span
    double* cmax;    // rows x heads x nchunk
    double* part;    // rows x heads x nchunk x hd
    double* pes;     // rows x heads x nchunk
};

__host__ __device__ inline int attn_nchunk(int span) { return (span + 63) / 64; }

// ---- fast decode attention for head_dim 64 / 128 ------------------------------
// Part 1: one workgroup per (KV head, 32-position chunk, row) serves every
// query head of the KV head's group (GQA), so each K/V row is read once.  Wave
// w takes group member w (w+4, ...).  Scores: two lanes per position, four
// interleaved chains over half the head each, (c0+c1)+(c2+c3), lo + hi.  Then
// the chunk maximum m_c, p = exp(s - m_c), the chunk's expSum and sum(p * v)
// (even and odd positions in two chains).
// ROPE (one token per sequence, seq == 1): the Q/K/V epilogue of the stacked
// projection runs here instead of in qkv_rope_kernel, with the same steps
// (q_pair / k_pair / v_val): each workgroup rotates the Q of its heads, and the
// workgroup whose chunk holds the new position writes that position's K and V
// to the cache (and uses them from LDS).  No other workgroup reads that row.
constexpr int kGqaChunk = 32;
__host__ __device__ inline int attn_nchunk32(int span) { return (span + kGqaChunk - 1) / kGqaChunk; }

struct RopeArgs {
    const int32_t* acc;  // stacked [Q; K; V] accumulators, row stride q_dim + 2 kv_dim
    const float* amax;
    float sq, sk, sv;
    const float* bq;
    const float* bk;
    const float* bv;
    double theta;
    double* q_tap;  // debug tap: Q rows after bias and RoPE (rows x q_dim), written by chunk 0
    QkNorm qk;      // per-head Q/K norms (the QKN kernels only)
};

// The norm factor of one head from its squares in LDS (sq[0..hd)): every lane
// forms the dimension-order chain itself (the same address for all lanes).
template <int HD>
__device__ __forceinline__ double lds_head_inv(const double* sq, double eps) {
    double s = 0.0;
#pragma unroll 16
    for (int d = 0; d < HD; ++d) s = s + sq[d];
    return qk_inv_rms(s, HD, eps);
}

// strict part 1: the scores of one 64-position chunk for every query head of
// one KV head, and each head's chunk maximum.  The chunk's K rows are copied
// to LDS with coalesced loads (pitch HD + 2 floats: the lanes' row reads fall
// in different banks); wave w serves group members w, w + 4, ...; lane i owns
// position k0 + i and forms q . k in dimension order, one rounded product and
// one rounded sum per dimension (the reference's `dot += q[d] * k[d]`), then
// scales it by 1 / sqrt(hd).  ROPE (one token per sequence): Q comes from the
// stacked projection accumulators by the Q/K/V epilogue steps of
// qkv_rope_kernel (each lane computes the rotation angle of its own pair), and
// the workgroup whose chunk holds the new position writes that position's K
// and V rows to the cache and takes the K row into LDS itself.  No other
// workgroup reads that row.  QKN: the per-head Q/K norms run before the
// rotation (each head's squares staged in LDS, the chain formed by every lane
// of the head's wave).  grid (kv_heads, nchunk, rows), 256 threads.
template <int HD, bool ROPE, bool QKN = false>
__global__ __launch_bounds__(256) void attn_scores_gqa_kernel(const double* __restrict__ q,
                                                              float* cache_k, float* cache_v,
                                                              const int* __restrict__ pos0, int msl,
                                                              int span, int heads, int kv_heads,
                                                              int seq, DecodeScratch sc, RopeArgs ra) {
    constexpr int CH = 64;
    constexpr int KP = HD + 2;       // LDS row pitch (floats)
    constexpr int PR4 = HD / 4;      // float4 per K row
    constexpr int NK = CH * PR4 / 256;
    constexpr int HALF = HD / 2;
    constexpr int NA = (HALF + 63) / 64;  // rotation pairs per lane
    static_assert(NK * 256 == CH * PR4, "chunk geometry");
    __shared__ __align__(16) float ks[CH * KP];
    __shared__ double qs[4][HD];
    __shared__ double nsq[QKN ? 4 : 1][QKN ? HD : 1];  // one head's squares per wave
    const int kvh = blockIdx.x, chunk = blockIdx.y, row = blockIdx.z;
    const int G = heads / kv_heads;
    const int b = row / seq, s = row % seq;
    const int pos = *pos0 + s;
    const int L = min(pos + 1, span);
    const int k0 = chunk * CH;
    if (k0 >= L) return;  // uniform over the workgroup
    const int nchunk = attn_nchunk(span);
    const int q_dim = heads * HD, kv_dim = kv_heads * HD;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const size_t cb = (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    // the chunk's K rows (rows past the length are read but never scored)
    float4 kreg[NK];
#pragma unroll
    for (int j = 0; j < NK; ++j) {
        const int i = tid + j * 256;
        const int r = i / PR4, c4 = (i % PR4) * 4;
        kreg[j] = load16_nt((const float4*)(cache_k + cb + (size_t)min(k0 + r, msl - 1) * kv_dim + c4));
    }
    const int32_t* ar = ROPE ? ra.acc + (size_t)row * (q_dim + 2 * kv_dim) : nullptr;
    const bool newrow = ROPE && k0 <= pos && pos < k0 + CH;
    double rcos[NA], rsin[NA];
    double osq = 0.0;
    if (ROPE) {
        const float am = ra.amax[row];
        osq = output_scale(ra.sq, am);
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const int d = lane + 64 * a;
            rcos[a] = rsin[a] = 0.0;
            if (d < HALF) rope_angle(pos, d, HD, ra.theta, &rcos[a], &rsin[a]);
        }
        double kinv = 0.0;
        if (QKN && newrow && ra.qk.k) {  // uniform: the new K row's squares, then its norm factor
            const double osk = output_scale(ra.sk, am);
            for (int d = tid; d < HD; d += 256) {
                const int j = q_dim + kvh * HD + d;
                const double v = (double)(float)((double)ar[j] * osk + (ra.bk ? (double)ra.bk[j - q_dim] : 0.0));
                nsq[0][d] = v * v;
            }
            __syncthreads();
            kinv = lds_head_inv<HD>(nsq[0], ra.qk.eps);
            __syncthreads();  // nsq is reused by the Q rounds
        }
        if (newrow && wave == 0) {
            // the new position's K pairs (lane d: d, d + HD/2) and V values
            const double osk = output_scale(ra.sk, am), osv = output_scale(ra.sv, am);
            float* krow = cache_k + (size_t)b * msl * kv_dim + (size_t)(pos % msl) * kv_dim + kvh * HD;
            float* vrow = cache_v + (size_t)b * msl * kv_dim + (size_t)(pos % msl) * kv_dim + kvh * HD;
            float* kl = ks + (pos - k0) * KP;
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                const int d = lane + 64 * a;
                if (d < HALF) {
                    float o0, o1;
                    const HeadNorm hn = head_norm(QKN && ra.qk.k != nullptr, kinv, ra.qk.k, ra.qk.k_len,
                                                  kv_heads, HD, kvh, d, d + HALF);
                    k_pair(ar + q_dim, osk, ra.bk, kvh * HD + d, kvh * HD + d + HALF, rcos[a], rsin[a],
                           &o0, &o1, hn);
                    krow[d] = o0;
                    krow[d + HALF] = o1;
                    kl[d] = o0;
                    kl[d + HALF] = o1;
                }
            }
            for (int d = lane; d < HD; d += 64) vrow[d] = v_val(ar + q_dim + kv_dim, osv, ra.bv, kvh * HD + d);
        }
    }
#pragma unroll
    for (int j = 0; j < NK; ++j) {
        const int i = tid + j * 256;
        const int r = i / PR4, c4 = (i % PR4) * 4;
        if (!(newrow && k0 + r == pos)) {
            float* kl = ks + r * KP + c4;
            *(float2*)kl = make_float2(kreg[j].x, kreg[j].y);
            *(float2*)(kl + 2) = make_float2(kreg[j].z, kreg[j].w);
        }
    }
    const size_t rh0 = (size_t)row * heads;
    const float* kr = ks + lane * KP;
    const int kp = k0 + lane;
    // rounds of four group members (uniform: every wave meets each barrier)
    for (int m0 = 0; m0 < G; m0 += 4) {
        const int member = m0 + wave;
        const int h = kvh * G + member;
        double qinv = 0.0;
        if (QKN && ra.qk.q) {  // uniform: the head's squares, then its norm factor
            if (member < G) {
                for (int d = lane; d < HD; d += 64) {
                    const int j = h * HD + d;
                    const double v = (double)ar[j] * osq + (ra.bq ? (double)ra.bq[j] : 0.0);
                    nsq[wave][d] = v * v;
                }
            }
            __syncthreads();
            if (member < G) qinv = lds_head_inv<HD>(nsq[wave], ra.qk.eps);
        }
        if (member < G) {
            if (ROPE) {
#pragma unroll
                for (int a = 0; a < NA; ++a) {
                    const int d = lane + 64 * a;
                    if (d < HALF) {
                        double o0, o1;
                        const HeadNorm hn = head_norm(QKN && ra.qk.q != nullptr, qinv, ra.qk.q, ra.qk.q_len,
                                                      heads, HD, h, d, d + HALF);
                        q_pair(ar, osq, ra.bq, h * HD + d, h * HD + d + HALF, rcos[a], rsin[a], &o0, &o1,
                               hn);
                        qs[wave][d] = o0;
                        qs[wave][d + HALF] = o1;
                        if (ra.q_tap && chunk == 0) {
                            double* qt = ra.q_tap + (size_t)row * q_dim + (size_t)h * HD;
                            qt[d] = o0;
                            qt[d + HALF] = o1;
                        }
                    }
                }
            } else {
                const double* qr = q + (size_t)row * q_dim + (size_t)h * HD;
                for (int d = lane; d < HD; d += 64) qs[wave][d] = qr[d];
            }
        }
        __syncthreads();  // K rows (first round) and this round's Q in LDS
        if (member < G) {
            double dot = 0.0;
#pragma unroll 8
            for (int d = 0; d < HD; d += 2) {
                const float2 kk = *(const float2*)(kr + d);
                dot += qs[wave][d] * (double)kk.x;
                dot += qs[wave][d + 1] * (double)kk.y;
            }
            const size_t rh = rh0 + h;
            double m = -1e9;
            if (kp < L) {
                const double v = dot * (1.0 / sqrt((double)HD));
                sc.scores[rh * span + kp] = v;
                m = v;
            }
            // chunk maximum (exact in any order; NaN never wins)
            for (int off = 32; off > 0; off >>= 1) {
                const double o = __shfl_xor(m, off, 64);
                m = o > m ? o : m;
            }
            if (lane == 0) sc.cmax[rh * nchunk + chunk] = m;
        }
        __syncthreads();  // this round's Q reads are done before the next round's writes
    }
}

// QKN (with ROPE): the per-head Q/K norms run before the rotation, as in
// attn_scores_gqa_kernel.
template <int HD, bool ROPE, bool QKN = false>
__global__ __launch_bounds__(256) void attn_gqa_kernel(const double* __restrict__ q, float* cache_k,
                                                       float* cache_v, const int* __restrict__ pos0,
                                                       int msl, int span, int heads, int kv_heads,
                                                       int seq, DecodeScratch sc, RopeArgs ra) {
    constexpr int CH = kGqaChunk;
    constexpr int DH = HD / 2;   // score dims per lane
    constexpr int DP = HD / 64;  // output dims per lane
    constexpr int KP = HD + 4;   // padded LDS row (floats)
    constexpr int PR4 = HD / 4;
    // K rows: the two dimension halves a position's lane pair reads start 32
    // banks apart (half offset KHO = 32 mod 64 words) and rows 4 banks apart
    // (KPK = 4 mod 64), so the 16 lanes of one 128-bit LDS read pass (eight
    // positions, both halves) hit 64 distinct banks
    constexpr int KHO = (HD / 2) % 64 == 0 ? HD / 2 + 32 : HD / 2;
    constexpr int KPK = ((KHO + HD / 2 + 63) / 64) * 64 + 4;
    __shared__ __align__(16) float ks[CH * KPK];
    __shared__ __align__(16) float vs[CH * KP];
    __shared__ double qs[4][HD];
    __shared__ double ps[4][CH];
    __shared__ double rc[ROPE ? HD / 2 : 1], rsn[ROPE ? HD / 2 : 1];
    __shared__ double nsq[QKN ? 4 : 1][QKN ? HD : 1];  // one head's squares per wave
    const int kvh = blockIdx.x, chunk = blockIdx.y, row = blockIdx.z;
    const int G = heads / kv_heads;
    const int b = row / seq, s = row % seq;
    const int pos = *pos0 + s;
    const int L = min(pos + 1, span);
    const int k0 = chunk * CH;
    if (k0 >= L) return;  // uniform
    const int n = min(CH, L - k0);
    const int nchunk = attn_nchunk32(span);
    const int q_dim = heads * HD, kv_dim = kv_heads * HD;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // K and V rows of the chunk -> registers (V rows past the length as zeros:
    // their cache slots may hold anything, and 0 * NaN would poison the sums)
    const size_t cb = (size_t)b * msl * kv_dim + (size_t)kvh * HD;
    constexpr int NKV = CH * PR4 / 256;
    static_assert(NKV * 256 == CH * PR4, "chunk geometry");
    float4 kreg[NKV], vreg[NKV];
#pragma unroll
    for (int j = 0; j < NKV; ++j) {
        const int i = tid + j * 256;
        const int r = i / PR4, c4 = (i % PR4) * 4;
        const size_t o = cb + (size_t)min(k0 + r, msl - 1) * kv_dim + c4;
        kreg[j] = load16_nt((const float4*)(cache_k + o));
        vreg[j] = load16_nt((const float4*)(cache_v + o));
    }
    // ROPE: the projection operands this workgroup needs are loaded with the
    // K/V rows, and the angles computed while both are in flight: Q of the
    // first group member per wave (lane d < HD/2: pair d, d + HD/2), and, in
    // the workgroup whose chunk holds the new position, its K pair and V value
    const int32_t* ar = ROPE ? ra.acc + (size_t)row * (q_dim + 2 * kv_dim) : nullptr;
    const bool newrow = ROPE && k0 <= pos && pos < k0 + CH;
    int32_t qa0 = 0, qa1 = 0, ka0 = 0, ka1 = 0, va = 0;
    float qb0 = 0.0f, qb1 = 0.0f, kb0 = 0.0f, kb1 = 0.0f, vbv = 0.0f;
    float am = 0.0f;
    if (ROPE) {
        am = ra.amax[row];
        const int h0 = kvh * G + wave;
        if (wave < G && lane < HD / 2) {
            const int j0 = h0 * HD + lane, j1 = j0 + HD / 2;
            qa0 = ar[j0];
            qa1 = ar[j1];
            if (ra.bq) {
                qb0 = ra.bq[j0];
                qb1 = ra.bq[j1];
            }
        }
        if (newrow) {
            if (tid < HD / 2) {
                const int j0 = kvh * HD + tid, j1 = j0 + HD / 2;
                ka0 = ar[q_dim + j0];
                ka1 = ar[q_dim + j1];
                if (ra.bk) {
                    kb0 = ra.bk[j0];
                    kb1 = ra.bk[j1];
                }
            }
            if (tid < HD) {
                const int j = kvh * HD + tid;
                va = ar[q_dim + kv_dim + j];
                if (ra.bv) vbv = ra.bv[j];
            }
        }
        if (tid < HD / 2) rope_angle(pos, tid, HD, ra.theta, &rc[tid], &rsn[tid]);
    }
#pragma unroll
    for (int j = 0; j < NKV; ++j) {
        const int i = tid + j * 256;
        const int r = i / PR4, c4 = (i % PR4) * 4;
        *(float4*)&ks[r * KPK + (c4 < HD / 2 ? c4 : c4 - HD / 2 + KHO)] = kreg[j];
        *(float4*)&vs[r * KP + c4] = r >= n ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : vreg[j];
    }
    if (ROPE) {
        double kinv = 0.0;
        if (QKN && newrow && ra.qk.k) {  // uniform: the new K row's squares, then its norm factor
            const double osk = output_scale(ra.sk, am);
            if (tid < HD / 2) {
                const double v0 = (double)(float)((double)ka0 * osk + (ra.bk ? (double)kb0 : 0.0));
                const double v1 = (double)(float)((double)ka1 * osk + (ra.bk ? (double)kb1 : 0.0));
                nsq[0][tid] = v0 * v0;
                nsq[0][tid + HD / 2] = v1 * v1;
            }
            __syncthreads();
            kinv = lds_head_inv<HD>(nsq[0], ra.qk.eps);
        }
        __syncthreads();  // angles; the chunk's K/V rows in LDS; nsq reads done
        if (newrow) {
            const int rr = pos - k0;
            float* krow = cache_k + (size_t)b * msl * kv_dim + (size_t)(pos % msl) * kv_dim;
            float* vrow = cache_v + (size_t)b * msl * kv_dim + (size_t)(pos % msl) * kv_dim;
            if (tid < HD / 2) {
                const int j0 = kvh * HD + tid, j1 = j0 + HD / 2;
                float o0, o1;
                const HeadNorm hn = head_norm(QKN && ra.qk.k != nullptr, kinv, ra.qk.k, ra.qk.k_len, kv_heads,
                                              HD, kvh, tid, tid + HD / 2);
                k_pair_v(ka0, ka1, output_scale(ra.sk, am), ra.bk != nullptr, kb0, kb1, rc[tid], rsn[tid],
                         &o0, &o1, hn);
                ks[rr * KPK + tid] = o0;
                ks[rr * KPK + tid + KHO] = o1;
                krow[j0] = o0;
                krow[j1] = o1;
            }
            if (tid < HD) {
                const int j = kvh * HD + tid;
                const float v = v_val_v(va, output_scale(ra.sv, am), ra.bv != nullptr, vbv);
                vs[rr * KP + tid] = v;
                vrow[j] = v;
            }
        }
    }
    const int pl = lane >> 1, half = lane & 1;
    const double inv_sqrt = 1.0 / sqrt((double)HD);
    for (int g0 = 0; g0 < G; g0 += 4) {
        const int g = g0 + wave;
        const bool act = g < G;
        const int h = kvh * G + g;
        const size_t rh = (size_t)row * heads + h;
        double qinv = 0.0;
        if (QKN && ra.qk.q) {  // uniform: the head's squares, then its norm factor
            if (act) {
                const double os = output_scale(ra.sq, am);
                for (int d = lane; d < HD; d += 64) {
                    const int j = h * HD + d;
                    const double v = (double)ar[j] * os + (ra.bq ? (double)ra.bq[j] : 0.0);
                    nsq[wave][d] = v * v;
                }
            }
            __syncthreads();
            if (act) qinv = lds_head_inv<HD>(nsq[wave], ra.qk.eps);
        }
        if (act) {
            if (ROPE) {
                const double os = output_scale(ra.sq, am);
                double* qt = ra.q_tap && chunk == 0 ? ra.q_tap + (size_t)row * q_dim + (size_t)h * HD : nullptr;
                if (g0 == 0) {  // operands loaded with the K/V rows
                    if (lane < HD / 2) {
                        double o0, o1;
                        const HeadNorm hn = head_norm(QKN && ra.qk.q != nullptr, qinv, ra.qk.q, ra.qk.q_len,
                                                      heads, HD, h, lane, lane + HD / 2);
                        q_pair_v(qa0, qa1, os, ra.bq != nullptr, qb0, qb1, rc[lane], rsn[lane], &o0, &o1, hn);
                        qs[wave][lane] = o0;
                        qs[wave][lane + HD / 2] = o1;
                        if (qt) {
                            qt[lane] = o0;
                            qt[lane + HD / 2] = o1;
                        }
                    }
                } else {
                    for (int d = lane; d < HD / 2; d += 64) {
                        const int j0 = h * HD + d, j1 = j0 + HD / 2;
                        double o0, o1;
                        const HeadNorm hn = head_norm(QKN && ra.qk.q != nullptr, qinv, ra.qk.q, ra.qk.q_len,
                                                      heads, HD, h, d, d + HD / 2);
                        q_pair(ar, os, ra.bq, j0, j1, rc[d], rsn[d], &o0, &o1, hn);
                        qs[wave][d] = o0;
                        qs[wave][d + HD / 2] = o1;
                        if (qt) {
                            qt[d] = o0;
                            qt[d + HD / 2] = o1;
                        }
                    }
                }
            } else {
                for (int d = lane; d < HD; d += 64) qs[wave][d] = q[(size_t)row * q_dim + (size_t)h * HD + d];
            }
        }
        __syncthreads();
        double mc = -1e9, es = 0.0;
        if (act) {
            const float* kr = &ks[pl * KPK + half * KHO];
            const double* qq = &qs[wave][half * DH];
            double c0 = 0.0, c1 = 0.0, c2 = 0.0, c3 = 0.0;
#pragma unroll
            for (int d = 0; d < DH; d += 4) {
                const float4 k4 = *(const float4*)(kr + d);
                c0 = fma(qq[d], (double)k4.x, c0);
                c1 = fma(qq[d + 1], (double)k4.y, c1);
                c2 = fma(qq[d + 2], (double)k4.z, c2);
                c3 = fma(qq[d + 3], (double)k4.w, c3);
            }
            // (DPP lane moves instead of LDS-crossbar shuffles: the pair
            // exchange is quad_perm 1,0,3,2; the maximum and expSum the fixed
            // row_shr / row_bcast pattern, lane 63 holding the result)
            const double part = (c0 + c1) + (c2 + c3);
            const double oth = dpp_d<kDppQuadSwap1>(part, 0.0);
            const double dot = half ? oth + part : part + oth;
            const double scv = dot * inv_sqrt;
            const bool valid = pl < n;
            double m = valid ? (scv > -1e9 ? scv : -1e9) : -1e9;  // NaN never wins
            m = wave_max_f64_dpp(m);
            mc = m;
            const double pr = valid ? exp(scv - mc) : 0.0;
            if (half == 0) ps[wave][pl] = pr;
            es = wave_sum_f64_dpp(half == 0 ? pr : 0.0);
        }
        __syncthreads();
        if (act) {
            double a0[DP], a1[DP];
#pragma unroll
            for (int i = 0; i < DP; ++i) a0[i] = a1[i] = 0.0;
#pragma unroll 4
            for (int pp = 0; pp < CH; pp += 2) {
                const double p0 = ps[wave][pp], p1 = ps[wave][pp + 1];
#pragma unroll
                for (int i = 0; i < DP; ++i) {
                    a0[i] = fma(p0, (double)vs[pp * KP + lane * DP + i], a0[i]);
                    a1[i] = fma(p1, (double)vs[(pp + 1) * KP + lane * DP + i], a1[i]);
                }
            }
            double* dst = sc.part + (rh * nchunk + chunk) * HD + lane * DP;
#pragma unroll
            for (int i = 0; i < DP; ++i) dst[i] = a0[i] + a1[i];
            if (lane == 0) {
                sc.cmax[rh * nchunk + chunk] = mc;
                sc.pes[rh * nchunk + chunk] = es;
            }
        }
        __syncthreads();  // qs / ps are rewritten by the next group member
    }
}

// Part 2: grid (heads, HD/32, rows), 256 threads: 8 threads per output dim,
// thread j of a dim adds the chunks c = j (mod 8) rescaled by exp(m_c - M)
// (M the overall maximum, the reference's M), then the 8 partial sums combine
// as ((t0+t1)+(t2+t3))+((t4+t5)+(t6+t7)); expSum the same way over pes.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine32_kernel(const int* __restrict__ pos0, int span,
                                                             int heads, int seq, DecodeScratch sc,
                                                             double* __restrict__ out) {
    constexpr int kMaxChunks = (kMaxAttnSpan + kGqaChunk - 1) / kGqaChunk;
    __shared__ double facs[kMaxChunks];
    __shared__ double wm[4];
    const int h = blockIdx.x, dg = blockIdx.y, row = blockIdx.z;
    const int s = row % seq;
    const int Lt = *pos0 + s + 1;
    const int L = min(Lt, span);
    const int nca = (L + kGqaChunk - 1) / kGqaChunk;
    const int nchunk = attn_nchunk32(span);
    const size_t rh = (size_t)row * heads + h;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = tid & 7, d = dg * 32 + (tid >> 3);
    const double* pb = sc.part + rh * nchunk * HD + d;
    // the partial sums of the first two groups of 64 chunks do not depend on
    // the maximum: they load while it is formed
    double pv[2][8], pe[2][8];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = 64 * gi + 8 * u + j;
            pv[gi][u] = c < nca ? pb[(size_t)c * HD] : 0.0;
            pe[gi][u] = c < nca ? sc.pes[rh * nchunk + c] : 0.0;
        }
    double M = -1e9;
    for (int c = tid; c < nca; c += 256) {
        const double v = sc.cmax[rh * nchunk + c];
        M = v > M ? v : M;
    }
    M = wave_max_f64_dpp(M);
    if (lane == 0) wm[wave] = M;
    __syncthreads();
    M = wm[0];
    for (int w = 1; w < 4; ++w) M = wm[w] > M ? wm[w] : M;
    for (int c = tid; c < nca; c += 256) facs[c] = exp(sc.cmax[rh * nchunk + c] - M);
    __syncthreads();
    double t = 0.0, e = 0.0;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = 64 * gi + 8 * u + j;
            if (c < nca) {
                t = fma(pv[gi][u], facs[c], t);
                e = fma(pe[gi][u], facs[c], e);
            }
        }
    for (int c0 = 128; c0 < nca; c0 += 64) {
        double w[8], we[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + 8 * u + j;
            w[u] = c < nca ? pb[(size_t)c * HD] : 0.0;
            we[u] = c < nca ? sc.pes[rh * nchunk + c] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + 8 * u + j;
            if (c < nca) {
                t = fma(w[u], facs[c], t);
                e = fma(we[u], facs[c], e);
            }
        }
    }
    // fixed tree over the 8 threads of the dim (consecutive lanes), as DPP
    // row shifts: lane j = 7 ends with ((t7+t6)+(t5+t4))+((t3+t2)+(t1+t0)),
    // the bits of ((t0+t1)+(t2+t3))+((t4+t5)+(t6+t7)) (every node commutes)
    t = t + dpp_d<kDppShr1>(t, 0.0);
    e = e + dpp_d<kDppShr1>(e, 0.0);
    t = t + dpp_d<kDppShr2>(t, 0.0);
    e = e + dpp_d<kDppShr2>(e, 0.0);
    t = t + dpp_d<kDppShr4>(t, 0.0);
    e = e + dpp_d<kDppShr4>(e, 0.0);
    if (j == 7) {
        double* orow = out + (size_t)row * heads * HD + (size_t)h * HD;
        orow[d] = Lt > span ? __builtin_nan("") : t / e;
    }
}

// fast decode attention, part 1: one workgroup per (head, 64-position chunk,
// row).  Scores: four lanes per position, each a d-order chain over a quarter
// of the head, combined as (q0 + q1) + (q2 + q3).  Then the chunk maximum m_c,
// p = exp(score - m_c), the chunk's expSum and its sum(p * v) per column.
// The combine kernel rescales each chunk by exp(m_c - M) (M the overall
// maximum, the same M the reference uses) and adds the chunks in order.
// grid (heads, nchunk, rows), 256 threads.
__global__ __launch_bounds__(256) void attn_chunk_kernel(const double* __restrict__ q,
                                                         const float* __restrict__ cache_k,
                                                         const float* __restrict__ cache_v,
                                                         const int* __restrict__ pos0, int msl,
                                                         int span, int heads, int kv_heads, int hd,
                                                         int seq, DecodeScratch sc) {
    extern __shared__ float vs[];  // V rows of the chunk: 64 x (hd + 4)
    __shared__ double qs[256];
    __shared__ double ps[64];
    __shared__ double red[256];
    __shared__ double wmx[4];
    const int h = blockIdx.x, chunk = blockIdx.y, row = blockIdx.z;
    const int b = row / seq, s = row % seq;
    const int kvh = h / (heads / kv_heads);
    const int q_dim = heads * hd, kv_dim = kv_heads * hd;
    const int L = min(*pos0 + s + 1, span);
    const int k0 = chunk * 64;
    if (k0 >= L) return;
    const int n = min(64, L - k0);
    const int nchunk = attn_nchunk(span);
    const size_t rh = (size_t)row * heads + h;
    const int tid = threadIdx.x;
    // V rows of the chunk -> LDS (loads in flight during the scores)
    const float* vb = cache_v + (size_t)b * msl * kv_dim + (size_t)kvh * hd;
    const int per_row4 = hd / 4;
    for (int i = tid; i < 64 * per_row4; i += 256) {
        const int r = i / per_row4, c4 = (i % per_row4) * 4;
        *(float4*)&vs[r * (hd + 4) + c4] = *(const float4*)(vb + (size_t)min(k0 + r, msl - 1) * kv_dim + c4);
    }
    const double* qr = q + (size_t)row * q_dim + (size_t)h * hd;
    for (int d = tid; d < hd; d += 256) qs[d] = qr[d];
    __syncthreads();
    // scores
    const int pl = tid >> 2, part = tid & 3;  // position in the chunk, quarter of d
    const int kp = k0 + pl;
    const int dq = hd / 4, d0 = part * dq;
    double dot = 0.0;
    {
        const float* kr = cache_k + (size_t)b * msl * kv_dim + (size_t)min(kp, msl - 1) * kv_dim +
                          (size_t)kvh * hd + d0;
        if ((dq & 3) == 0) {
            for (int d = 0; d < dq; d += 4) {
                const float4 k4 = *(const float4*)(kr + d);
                dot = fma(qs[d0 + d], (double)k4.x, dot);
                dot = fma(qs[d0 + d + 1], (double)k4.y, dot);
                dot = fma(qs[d0 + d + 2], (double)k4.z, dot);
                dot = fma(qs[d0 + d + 3], (double)k4.w, dot);
            }
        } else {
            for (int d = 0; d < dq; ++d) dot = fma(qs[d0 + d], (double)kr[d], dot);
        }
    }
    const double o1 = __shfl_xor(dot, 1, 64);
    const double pair = (part & 1) ? o1 + dot : dot + o1;  // q0+q1 (lanes 0,1), q2+q3 (lanes 2,3)
    const double o2 = __shfl_xor(pair, 2, 64);
    const double tot = (part & 2) ? o2 + pair : pair + o2;
    const double sc_v = tot * (1.0 / sqrt((double)hd));
    const bool valid = pl < n;
    // chunk maximum (-1e9 start, NaN never wins)
    double m = valid ? (sc_v > -1e9 ? sc_v : -1e9) : -1e9;
    for (int off = 32; off > 0; off >>= 1) {
        const double o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if ((tid & 63) == 0) wmx[tid >> 6] = m;
    __syncthreads();
    double mc = wmx[0];
    for (int w = 1; w < 4; ++w) mc = wmx[w] > mc ? wmx[w] : mc;
    if (part == 0) ps[pl] = valid ? exp(sc_v - mc) : 0.0;
    __syncthreads();
    if (tid < 64) {
        double e = ps[tid];
        for (int off = 32; off > 0; off >>= 1) e = e + __shfl_down(e, off, 64);
        if (tid == 0) {
            sc.pes[rh * nchunk + chunk] = e;
            sc.cmax[rh * nchunk + chunk] = mc;
        }
    }
    // partial PV: (256 / hd) slices of the chunk per column, combined in order
    const int slices = 256 / hd;
    const int d = tid % hd, sl = tid / hd;
    const int per = (n + slices - 1) / slices;
    double sum = 0.0;
    if (sl < slices) {
        const int a0 = min(n, sl * per), a1 = min(n, a0 + per);
        for (int k = a0; k < a1; ++k) sum = fma(ps[k], (double)vs[k * (hd + 4) + d], sum);
    }
    red[tid] = sum;
    __syncthreads();
    if (tid < hd) {
        double t = red[tid];
        for (int k = 1; k < slices; ++k) t = t + red[k * hd + tid];
        sc.part[(rh * nchunk + chunk) * hd + tid] = t;
    }
}

// fast part 2: combine the chunk partials in chunk order, each rescaled by
// exp(m_c - M); grid (heads, rows)
__global__ __launch_bounds__(256) void attn_combine_kernel(const int* __restrict__ pos0, int span,
                                                           int heads, int hd, int seq,
                                                           DecodeScratch sc,
                                                           double* __restrict__ out) {
    __shared__ double fac[kMaxAttnSpan / 64 + 1];
    __shared__ double es_sh;
    const int h = blockIdx.x, row = blockIdx.y;
    const int s = row % seq;
    const int L = *pos0 + s + 1;
    const int q_dim = heads * hd;
    double* orow = out + (size_t)row * q_dim + (size_t)h * hd;
    if (L > span) {
        for (int d = threadIdx.x; d < hd; d += 256) orow[d] = __builtin_nan("");
        return;
    }
    const int nc = (L + 63) / 64, nchunk = attn_nchunk(span);
    const size_t rh = (size_t)row * heads + h;
    if (threadIdx.x < 64) {
        double M = -1e9;
        for (int c = threadIdx.x; c < nc; c += 64) {
            const double v = sc.cmax[rh * nchunk + c];
            M = v > M ? v : M;
        }
        for (int off = 32; off > 0; off >>= 1) {
            const double o = __shfl_xor(M, off, 64);
            M = o > M ? o : M;
        }
        for (int c = threadIdx.x; c < nc; c += 64) fac[c] = exp(sc.cmax[rh * nchunk + c] - M);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double es = 0.0;
        for (int c = 0; c < nc; ++c) es = fma(sc.pes[rh * nchunk + c], fac[c], es);
        es_sh = es;
    }
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += 256) {
        double t = 0.0;
        for (int c0 = 0; c0 < nc; c0 += 8) {
            double v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = c0 + i < nc ? sc.part[(rh * nchunk + c0 + i) * hd + d] : 0.0;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (c0 + i < nc) t = fma(v[i], fac[c0 + i], t);
        }
        orow[d] = t / es_sh;
    }
}

// strict part 2: one workgroup per (head, group of DG value columns, row).
// The probabilities p[k] = exp(score[k] - max) are formed here: the maximum
// over the chunk maxima (every wave forms it), then one probability per thread
// and 256-position chunk into an LDS ring two chunks deep.  Lane d <= DG of
// wave 0 adds column d of the products p[k] * v[k][d] in position order (the
// reference's `sum += p * v`, a product then a sum, each rounded); column DG
// holds p itself, whose chain is expSum.  Chunks of C = 4096 / DG positions:
// each of the 256 threads of waves 1-4 loads its 16 values of a chunk (and
// the scores it turns into probabilities: C / 256) kChainDepth chunks ahead,
// forms its products in registers and writes them to one of two LDS product
// buffers, transposed so that a chain lane reads two positions per 16-byte
// load; wave 0 only adds: chunk c while the other waves write the products of
// chunk c + 1 and the probabilities of chunk c + 2.  The loads are
// branch-free (indices clamped into the ring and the score row; surplus
// values are never added).  grid (heads * HD / DG, rows), 320 threads.
constexpr int kChainDepth = 4;
constexpr int kChainCols = 16;
constexpr int kChainThreads = 320;  // wave 0: the chains; waves 1-4: loads, probabilities, products

template <int HD, int DG>
__global__ __launch_bounds__(kChainThreads) void attn_chain_kernel(const float* __restrict__ cache_v,
                                                         const int* __restrict__ pos0, int msl,
                                                         int span, int heads, int kv_heads,
                                                         int seq, DecodeScratch sc,
                                                         double* __restrict__ out) {
    constexpr int C = 4096 / DG;  // positions per chunk
    constexpr int CP = C + 2;     // row pitch (16-byte aligned rows, lanes' reads in different banks)
    static_assert(C * DG == 4096 && C % 256 == 0 && C <= 512 && HD % DG == 0 && DG % 4 == 0,
                  "chunk geometry");
    constexpr int PT = C / 256;   // probabilities per thread and chunk
    __shared__ __align__(16) double prod[2][DG + 1][CP];
    __shared__ double pr_sh[2][C];
    const int h = blockIdx.x / (HD / DG), dg = blockIdx.x % (HD / DG), row = blockIdx.y;
    const int b = row / seq, s = row % seq;
    const int kvh = h / (heads / kv_heads);
    const int q_dim = heads * HD, kv_dim = kv_heads * HD;
    const int tid = threadIdx.x, lane = tid & 63;
    const int pt = tid - 64;        // product thread index (waves 1-4)
    const bool maker = tid >= 64;   // waves 1-4 (wave-uniform)
    const int L = *pos0 + s + 1;
    double* orow = out + (size_t)row * q_dim + (size_t)h * HD + dg * DG;
    if (L > span) {
        if (tid < DG) orow[tid] = __builtin_nan("");
        return;
    }
    const int nch = (L + C - 1) / C;
    const float* vb = cache_v + (size_t)b * msl * kv_dim + (size_t)kvh * HD + dg * DG;
    const size_t rh = (size_t)row * heads + h;
    const double* sr = sc.scores + rh * span;

    // staging registers of the chunks in flight (named scalars filled by
    // macros: arrays of them, indexed in loops, were kept in scratch memory).
    // Thread tid holds the float4s at elements 4(tid + 256 I) of the chunk's
    // C x DG values (position e / DG, column e % DG) and the scores of
    // positions tid + 256 q.
    float4 r0_0, r0_1, r0_2, r0_3, r1_0, r1_1, r1_2, r1_3;
    float4 r2_0, r2_1, r2_2, r2_3, r3_0, r3_1, r3_2, r3_3;
    double pt0[PT], pt1[PT], pt2[PT], pt3[PT];
#define LAMD_CHAIN_LD(U, I, CC)                                                   \
    {                                                                             \
        const int e = (pt + (I) * 256) * 4; /* element of the C x DG chunk */     \
        const int k = (CC) * C + e / DG;                                          \
        r##U##_##I = *(const float4*)(vb + (size_t)min(k, msl - 1) * kv_dim + e % DG); \
    }
#define LAMD_CHAIN_ISSUE(U, CH)                                                   \
    {                                                                             \
        const int cc = min((CH), nch - 1);                                        \
        LAMD_CHAIN_LD(U, 0, cc) LAMD_CHAIN_LD(U, 1, cc)                           \
        LAMD_CHAIN_LD(U, 2, cc) LAMD_CHAIN_LD(U, 3, cc)                           \
        _Pragma("unroll") for (int q = 0; q < PT; ++q)                            \
            pt##U[q] = sr[min(cc * C + pt + 256 * q, span - 1)];                 \
    }
#define LAMD_CHAIN_EXP(U, BUF)                                                    \
    {                                                                             \
        _Pragma("unroll") for (int q = 0; q < PT; ++q)                            \
            pr_sh[BUF][pt + 256 * q] = exp(pt##U[q] - mx);                       \
    }
#define LAMD_CHAIN_PR(U, I, BUF)                                                  \
    {                                                                             \
        const int e = (pt + (I) * 256) * 4;                                      \
        const int k = e / DG, d = e % DG;                                         \
        const double p = pr_sh[BUF][k];                                           \
        prod[BUF][d][k] = p * (double)r##U##_##I.x;                               \
        prod[BUF][d + 1][k] = p * (double)r##U##_##I.y;                           \
        prod[BUF][d + 2][k] = p * (double)r##U##_##I.z;                           \
        prod[BUF][d + 3][k] = p * (double)r##U##_##I.w;                           \
    }
#define LAMD_CHAIN_PRODUCTS(U, BUF)                                               \
    {                                                                             \
        LAMD_CHAIN_PR(U, 0, BUF) LAMD_CHAIN_PR(U, 1, BUF)                         \
        LAMD_CHAIN_PR(U, 2, BUF) LAMD_CHAIN_PR(U, 3, BUF)                         \
        _Pragma("unroll") for (int q = 0; q < PT; ++q)                            \
            prod[BUF][DG][pt + 256 * q] = pr_sh[BUF][pt + 256 * q];             \
    }
    if (maker) {
        LAMD_CHAIN_ISSUE(0, 0)
        LAMD_CHAIN_ISSUE(1, 1)
        LAMD_CHAIN_ISSUE(2, 2)
        LAMD_CHAIN_ISSUE(3, 3)
    }
    // maximum over the chunk maxima of the 64-position score chunks with
    // data: -1e9 start, NaN never wins (each wave forms the same value)
    double mx = -1e9;
    {
        const double* cm = sc.cmax + rh * attn_nchunk(span);
        const int nc = (L + 63) / 64;
        for (int c = lane; c < nc; c += 64) {
            const double v = cm[c];
            mx = v > mx ? v : mx;
        }
        for (int off = 32; off > 0; off >>= 1) {
            const double o = __shfl_xor(mx, off, 64);
            mx = o > mx ? o : mx;
        }
    }
    if (maker) {
        LAMD_CHAIN_EXP(0, 0)
        LAMD_CHAIN_EXP(1, 1)
    }
    __syncthreads();
    if (maker) {
        LAMD_CHAIN_PRODUCTS(0, 0)
        LAMD_CHAIN_ISSUE(0, kChainDepth)
    }
    __syncthreads();

    double sum = 0.0;  // column tid's chain (tid <= DG)
    // step for chunk c = c0 + U: waves 1-4 write the products of chunk c + 1
    // (staging set U + 1) to buffer (c + 1) & 1 and refill that set, and the
    // probabilities of chunk c + 2 (set UE) to ring slot c & 1, while wave 0
    // adds chunk c from buffer c & 1 (all parities are compile-time: c0 is a
    // multiple of four).  Products, probabilities and loads run for every
    // chunk's step, for chunks past the last one too (clamped indices; no
    // chain reads them), so the loads of the next three chunks stay in flight
    // across each wait.
#define LAMD_CHAIN_STEP(U, UN, UE)                                                \
    {                                                                             \
        const int c = c0 + (U);                                                   \
        if (c >= nch) break;                                                      \
        if (maker) {                                                               \
            LAMD_CHAIN_PRODUCTS(UN, ((U) + 1) & 1)                                \
            LAMD_CHAIN_EXP(UE, (U) & 1)                                           \
            LAMD_CHAIN_ISSUE(UN, c + 1 + kChainDepth)                             \
        }                                                                         \
        if (c < nch && tid <= DG) {                                               \
            const double* pc = prod[(U) & 1][tid];                                \
            const int n = min(C, L - c * C);                                      \
            sum = chain_add_pairs<C>(pc, n, sum);                                 \
        }                                                                         \
        __syncthreads();                                                          \
    }
    static_assert(kChainDepth == 4, "the loop below expands four chunk steps");
    for (int c0 = 0; c0 < nch; c0 += kChainDepth) {
        LAMD_CHAIN_STEP(0, 1, 2)
        LAMD_CHAIN_STEP(1, 2, 3)
        LAMD_CHAIN_STEP(2, 3, 0)
        LAMD_CHAIN_STEP(3, 0, 1)
    }
#undef LAMD_CHAIN_STEP
#undef LAMD_CHAIN_PRODUCTS
#undef LAMD_CHAIN_PR
#undef LAMD_CHAIN_EXP
#undef LAMD_CHAIN_ISSUE
#undef LAMD_CHAIN_LD
    __shared__ double es_sh;
    if (tid == DG) es_sh = sum;
    __syncthreads();
    if (tid < DG) orow[tid] = sum / es_sh;
}

// LDS bytes of one fused attention workgroup for `span` positions.
size_t attention_lds_bytes(int hd, int span) {
    return ((size_t)((hd + 1) & ~1) + (size_t)span) * sizeof(double);
}

// Fast prefill attention: 0 picks per call (the two-pass kernel for up to
// kAutoTwoPassRows rows when the one-pass grid has fewer workgroups than the
// chip has CUs: at one BitNet-2B sequence of 512 the block took 209.5 against
// 229.6 us), 1 the one-pass kernel always, 2 or 4 the two-pass kernel with
// that many 16-query tiles per workgroup.
constexpr int kAutoTwoPassRows = 1024;
constexpr int kAutoTwoPassGrid = 256;

int attention_fast_two_pass_qt() {
    const int qt = tune_int("LOOM_AMD_ATTN_QT", 0);
    return qt == 1 || qt == 2 || qt == 4 ? qt : 0;
}

size_t attention_scratch_bytes(int rows, int heads, int hd, int span, int strict, int fast_qt) {
    // prefill tiles of the strict and two-pass fast kernels: every score of
    // every row (rows x heads x span fp64); the one-pass kernel needs none
    if (rows > kSplitMaxRows) {
        if (hd != 64 && hd != 128) return 0;
        if (!strict && fast_qt == 1) return 0;
        if (!strict && fast_qt == 0) rows = rows < kAutoTwoPassRows ? rows : kAutoTwoPassRows;
        return (size_t)rows * heads * span * 8;
    }
    // (room for 32-position chunks; the 64-position kernels use a prefix of each region)
    const size_t rh = (size_t)rows * heads;
    const size_t nc = attn_nchunk32(span);
    return rh * ((size_t)span + nc + nc * hd + nc) * sizeof(double);
}

static DecodeScratch decode_scratch(double* base, int rows, int heads, int hd, int span) {
    const size_t rh = (size_t)rows * heads;
    const size_t nc = attn_nchunk32(span);
    DecodeScratch sc;
    sc.scores = base;
    sc.cmax = sc.scores + rh * span;
    sc.part = sc.cmax + rh * nc;
    sc.pes = sc.part + rh * nc * hd;
    return sc;
}

// Strict decode attention: scores (with the Q/K/V epilogue when ra.acc is
// set), then probabilities with the value and expSum chains.
static hipError_t launch_strict_decode(const double* q, float* cache_k, float* cache_v,
                                       const int* pos0, int msl, int span, int heads, int kv_heads,
                                       int hd, int seq, int rows, const DecodeScratch& sc,
                                       const RopeArgs& ra, double* out, hipStream_t s) {
    const int nc = attn_nchunk(span);
    const dim3 gs(kv_heads, nc, rows), t(256);
    constexpr int DG = kChainCols;
#define LAMD_SCORES(HDV)                                                                          \
    {                                                                                             \
        if (ra.acc && (ra.qk.q || ra.qk.k))                                                       \
            hipLaunchKernelGGL((attn_scores_gqa_kernel<HDV, true, true>), gs, t, 0, s, q, cache_k,  \
                               cache_v, pos0, msl, span, heads, kv_heads, seq, sc, ra);           \
        else if (ra.acc)                                                                          \
            hipLaunchKernelGGL((attn_scores_gqa_kernel<HDV, true>), gs, t, 0, s, q, cache_k, cache_v, \
                               pos0, msl, span, heads, kv_heads, seq, sc, ra);                    \
        else                                                                                      \
            hipLaunchKernelGGL((attn_scores_gqa_kernel<HDV, false>), gs, t, 0, s, q, cache_k,       \
                               cache_v, pos0, msl, span, heads, kv_heads, seq, sc, ra);           \
    }
#define LAMD_CHAIN(HDV)                                                                              \
    hipLaunchKernelGGL((attn_chain_kernel<HDV, DG>), dim3(heads * (HDV / DG), rows), dim3(kChainThreads), 0, \
                       s, cache_v, pos0, msl, span, heads, kv_heads, seq, sc, out)
    switch (hd) {
        case 32: LAMD_SCORES(32); break;
        case 64: LAMD_SCORES(64); break;
        case 128: LAMD_SCORES(128); break;
        default: LAMD_SCORES(256); break;
    }
    switch (hd) {
        case 32: LAMD_CHAIN(32); break;
        case 64: LAMD_CHAIN(64); break;
        case 128: LAMD_CHAIN(128); break;
        default: LAMD_CHAIN(256); break;
    }
#undef LAMD_CHAIN
#undef LAMD_SCORES
    return hipGetLastError();
}

bool attention_rope_ok(int seq, int hd, int strict, int span) {
    if (seq != 1 || span > kMaxAttnSpan) return false;
    return strict ? (hd == 32 || hd == 64 || hd == 128 || hd == 256) : (hd == 64 || hd == 128);
}

hipError_t launch_attention_rope(const int32_t* acc, const float* amax, float sq, float sk, float sv,
                                 const float* bq, const float* bk, const float* bv, double theta,
                                 int batch, const int* pos0, int msl, int span, int heads,
                                 int kv_heads, int hd, int strict, float* cache_k, float* cache_v,
                                 double* scratch, double* out, hipStream_t s, double* q_tap,
                                 const QkNorm& qk) {
    if (batch <= 0) return hipSuccess;
    if (!attention_rope_ok(1, hd, strict, span) || span > msl || !scratch || !acc)
        return hipErrorInvalidValue;
    if (kv_heads <= 0 || heads % kv_heads != 0 || batch > kSplitMaxRows) return hipErrorInvalidValue;
    if (theta <= 0.0) theta = 10000.0;
    const DecodeScratch sc = decode_scratch(scratch, batch, heads, hd, span);
    const RopeArgs ra{acc, amax, sq, sk, sv, bq, bk, bv, theta, q_tap, qk};
    const bool qkn = qk.q || qk.k;
    if (strict) {
        return launch_strict_decode(nullptr, cache_k, cache_v, pos0, msl, span, heads, kv_heads, hd, 1,
                                    batch, sc, ra, out, s);
    }
    const dim3 g(kv_heads, attn_nchunk32(span), batch), gc(heads, hd / 32, batch);
    if (hd == 128) {
        if (qkn)
            hipLaunchKernelGGL((attn_gqa_kernel<128, true, true>), g, dim3(256), 0, s, nullptr, cache_k,
                               cache_v, pos0, msl, span, heads, kv_heads, 1, sc, ra);
        else
            hipLaunchKernelGGL((attn_gqa_kernel<128, true>), g, dim3(256), 0, s, nullptr, cache_k, cache_v,
                               pos0, msl, span, heads, kv_heads, 1, sc, ra);
        hipLaunchKernelGGL(attn_combine32_kernel<128>, gc, dim3(256), 0, s, pos0, span, heads, 1, sc, out);
    } else {
        if (qkn)
            hipLaunchKernelGGL((attn_gqa_kernel<64, true, true>), g, dim3(256), 0, s, nullptr, cache_k,
                               cache_v, pos0, msl, span, heads, kv_heads, 1, sc, ra);
        else
            hipLaunchKernelGGL((attn_gqa_kernel<64, true>), g, dim3(256), 0, s, nullptr, cache_k, cache_v,
                               pos0, msl, span, heads, kv_heads, 1, sc, ra);
        hipLaunchKernelGGL(attn_combine32_kernel<64>, gc, dim3(256), 0, s, pos0, span, heads, 1, sc, out);
    }
    return hipGetLastError();
}

hipError_t launch_attention(const double* q, const float* cache_k, const float* cache_v,
                            int batch, int seq, const int* pos0, int msl, int span, int heads,
                            int kv_heads, int hd, int strict, int fast_qt, double* scratch,
                            double* out, hipStream_t s) {
    if (seq <= 0 || batch <= 0) return hipSuccess;
    if (hd % 4 != 0 || hd > 256 || kv_heads <= 0 || heads % kv_heads != 0) return hipErrorInvalidValue;
    if (span > kMaxAttnSpan || span > msl) return hipErrorInvalidValue;
    const int rows = batch * seq;
    const bool chain_hd = hd == 32 || hd == 64 || hd == 128 || hd == 256;
    if (rows <= kSplitMaxRows && (!strict || chain_hd)) {
        if (!scratch) return hipErrorInvalidValue;
        const DecodeScratch sc = decode_scratch(scratch, rows, heads, hd, span);
        const int nc = attn_nchunk(span);
        if (!strict && (hd == 64 || hd == 128)) {
            const dim3 g(kv_heads, attn_nchunk32(span), rows), gc(heads, hd / 32, rows);
            const RopeArgs none{};
            float* ck = const_cast<float*>(cache_k);  // read only without ROPE
            float* cv = const_cast<float*>(cache_v);
            if (hd == 128) {
                hipLaunchKernelGGL((attn_gqa_kernel<128, false>), g, dim3(256), 0, s, q, ck, cv, pos0,
                                   msl, span, heads, kv_heads, seq, sc, none);
                hipLaunchKernelGGL(attn_combine32_kernel<128>, gc, dim3(256), 0, s, pos0, span, heads,
                                   seq, sc, out);
            } else {
                hipLaunchKernelGGL((attn_gqa_kernel<64, false>), g, dim3(256), 0, s, q, ck, cv, pos0,
                                   msl, span, heads, kv_heads, seq, sc, none);
                hipLaunchKernelGGL(attn_combine32_kernel<64>, gc, dim3(256), 0, s, pos0, span, heads,
                                   seq, sc, out);
            }
        } else if (!strict) {
            hipLaunchKernelGGL(attn_chunk_kernel, dim3(heads, nc, rows), dim3(256),
                               (size_t)64 * (hd + 4) * sizeof(float), s, q, cache_k, cache_v, pos0,
                               msl, span, heads, kv_heads, hd, seq, sc);
            hipLaunchKernelGGL(attn_combine_kernel, dim3(heads, rows), dim3(256), 0, s, pos0, span,
                               heads, hd, seq, sc, out);
        } else {
            const RopeArgs none{};
            return launch_strict_decode(q, const_cast<float*>(cache_k), const_cast<float*>(cache_v),
                                        pos0, msl, span, heads, kv_heads, hd, seq, rows, sc, none, out,
                                        s);
        }
        return hipGetLastError();
    }
    if (hd == 64 || hd == 128) {
        // one-pass grid: heads sharing one KV head go to one workgroup, up to four
        const int group = heads / kv_heads;
        const int hpw = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
        const dim3 gridh(heads / hpw, ceil_div(seq, 64 / hpw), batch);
        int qt = fast_qt == 2 || fast_qt == 4 ? fast_qt : 0;
        if (fast_qt == 0 && (long)gridh.x * gridh.y * gridh.z < kAutoTwoPassGrid && rows <= kAutoTwoPassRows &&
            scratch && span % 2 == 0)
            qt = 2;  // too few one-pass workgroups to fill the chip
        if (!strict && qt == 0) {
#define LAMD_FLASH(HDV, HPWV)                                                                    \
    hipLaunchKernelGGL((attn_flash_mfma_kernel<HDV, HPWV>), gridh, dim3(256), 0, s, q, cache_k, \
                       cache_v, pos0, msl, span, heads, kv_heads, seq, out)
            if (hd == 128) {
                if (hpw == 4) LAMD_FLASH(128, 4);
                else if (hpw == 2) LAMD_FLASH(128, 2);
                else LAMD_FLASH(128, 1);
            } else {
                if (hpw == 4) LAMD_FLASH(64, 4);
                else if (hpw == 2) LAMD_FLASH(64, 2);
                else LAMD_FLASH(64, 1);
            }
#undef LAMD_FLASH
            return hipGetLastError();
        }
        if (!scratch || span % 2 != 0) return hipErrorInvalidValue;
        const dim3 grid(heads, ceil_div(seq, kTileQ), batch);
#define LAMD_TILE(HDV)                                                                             \
    hipLaunchKernelGGL((attn_tile_kernel<HDV>), grid, dim3(256), 0, s, q, cache_k, cache_v, pos0,    \
                       msl, span, heads, kv_heads, seq, scratch, out)
        const dim3 gridf(heads, ceil_div(seq, 16 * (qt ? qt : 2)), batch);
#define LAMD_FAST(HDV, QTV)                                                                          \
    hipLaunchKernelGGL((attn_tile_mfma_kernel<HDV, QTV>), gridf, dim3(256), 0, s, q, cache_k, cache_v, \
                       pos0, msl, span, heads, kv_heads, seq, scratch, out)
        if (hd == 128) {
            if (strict) {
                LAMD_TILE(128);
            } else if (qt == 4) {
                LAMD_FAST(128, 4);
            } else {
                LAMD_FAST(128, 2);
            }
        } else {
            if (strict) {
                LAMD_TILE(64);
            } else if (qt == 4) {
                LAMD_FAST(64, 4);
            } else {
                LAMD_FAST(64, 2);
            }
        }
#undef LAMD_FAST
#undef LAMD_TILE
        return hipGetLastError();
    }
    const size_t shm = attention_lds_bytes(hd, span);
    if (shm > kMaxAttnLds) return hipErrorInvalidValue;
    const dim3 grid(heads, seq, batch);
    if (strict) {
        hipLaunchKernelGGL(attention_kernel<1>, grid, dim3(256), shm, s, q, cache_k, cache_v, pos0,
                           msl, span, heads, kv_heads, hd, out);
    } else {
        hipLaunchKernelGGL(attention_kernel<0>, grid, dim3(256), shm, s, q, cache_k, cache_v, pos0,
                           msl, span, heads, kv_heads, hd, out);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// MHA inner norm on fp64 rows (bitNetRMSNormFloat64Weighted,
// poly/bitnet_cpu.go:868-887: data *= scale*w) + fp64 requantization
// (bitNetQuantizeActivationFloat64, poly/bitnet_cpu.go:59-71,108-117).
// pre (optional) receives fp32(normalized), loom's MHA preAct.
// ------------------------------------------------------------------------

template <int STRICT, int VPT>
__global__ __launch_bounds__(256) void norm_quant_f64_kernel(double* __restrict__ a, int n,
                                                             const float* __restrict__ weight,
                                                             double eps, float* __restrict__ pre,
                                                             int8_t* __restrict__ xq, int ldq,
                                                             float* __restrict__ amax_out,
                                                             int32_t* __restrict__ xsum_out, int keep,
                                                             const double* __restrict__ totals) {
    extern __shared__ double sq[];
    __shared__ double red[256];
    __shared__ float shf[4];
    __shared__ int shi[4];
    const int row = blockIdx.x;
    double* ar = a + (size_t)row * n;
    double v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        v[j] = i < n ? ar[i] : 0.0;
    }
    double total;
    if (STRICT && totals) {
        total = totals[row];  // the row-chain kernel's ordered sum
    } else if (STRICT) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = threadIdx.x + j * 256;
            if (i < n) sq[i] = v[j] * v[j];
        }
        total = lds_sum<1>(sq, n, red);
    } else {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < VPT; ++j) s += v[j] * v[j];
        red[threadIdx.x] = s;
        __syncthreads();
        for (int w = 128; w > 0; w >>= 1) {
            if (threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
            __syncthreads();
        }
        total = red[0];
    }
    const double scale = 1.0 / sqrt(total / (double)n + eps);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        if (i < n) {
            const double w = weight ? (double)weight[i] : 1.0;
            v[j] = v[j] * (scale * w);
            if (keep) ar[i] = v[j];
            if (pre) pre[(size_t)row * n + i] = (float)v[j];
            m = max_nan_skip(m, (float)fabs(v[j]));
        }
    }
    m = block_max(m, shf);
    if (m < 1e-5f) m = 1e-5f;
    const double qs = 127.0 / (double)m;
    int s = 0;
    int8_t* qr = xq + (size_t)row * ldq;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int i = threadIdx.x + j * 256;
        if (i < n) {
            const int q = quant_one(v[j], qs);
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

template <int STRICT>
static hipError_t launch_norm_f64_t(double* a, int m, int n, const float* w, double eps, float* pre,
                                    int8_t* xq, int ldq, float* amax, int32_t* xsum, int keep,
                                    const double* totals, hipStream_t s) {
    {
        const RowNormArgs ra{a, n, m, n, w, eps, pre, keep ? a : nullptr, xq, ldq, amax, xsum, totals};
        hipError_t e = hipSuccess;
        if (launch_row_norm_wave(kRowInnerF64, STRICT, ra, s, &e)) return e;
    }
    const size_t shm = STRICT && !totals ? (size_t)ordered_sum_slots(n, 4) * sizeof(double) : 0;
    const dim3 g(m), b(256);
#define LAMD_NF64(VPT)                                                                          \
    hipLaunchKernelGGL((norm_quant_f64_kernel<STRICT, VPT>), g, b, shm, s, a, n, w, eps, pre, xq, ldq, \
                       amax, xsum, keep, totals)
    if (n <= 256 * 4) {
        LAMD_NF64(4);
    } else if (n <= 256 * 8) {
        LAMD_NF64(8);
    } else if (n <= 256 * 16) {
        LAMD_NF64(16);
    } else if (n <= 256 * 32) {
        LAMD_NF64(32);
    } else {
        return hipErrorInvalidValue;
    }
#undef LAMD_NF64
    return hipGetLastError();
}

hipError_t launch_norm_quant_f64(double* a, int m, int n, const float* w, double eps, int strict,
                                 float* pre, int8_t* xq, int ldq, float* amax, int32_t* xsum,
                                 hipStream_t s, bool keep_rows, double* totals) {
    if (m <= 0) return hipSuccess;
    if (eps <= 0.0) eps = 1e-5;  // bitNetRMSNormFloat64Weighted default
    if (n > kMaxNormCols || (strict && n > kMaxStrictNormCols)) return hipErrorInvalidValue;
    const int keep = keep_rows ? 1 : 0;
    if (!strict) return launch_norm_f64_t<0>(a, m, n, w, eps, pre, xq, ldq, amax, xsum, keep, nullptr, s);
    hipError_t e = hipSuccess;
    const bool rows = launch_row_sumsq<double>(a, n, m, n, totals, s, &e);
    if (e != hipSuccess) return e;
    return launch_norm_f64_t<1>(a, m, n, w, eps, pre, xq, ldq, amax, xsum, keep, rows ? totals : nullptr, s);
}

// ------------------------------------------------------------------------
// embeddings (poly/transformer.go:551-577): rows of the fp32 table; an id
// outside the table gives a zero row.
// ------------------------------------------------------------------------

__global__ void embed_kernel(const float* __restrict__ table, int vocab, int hidden,
                             const int* __restrict__ tokens, int cap, const int* __restrict__ pos0,
                             int batch, int seq, float* __restrict__ out) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)batch * seq * hidden) return;
    const int r = (int)(idx / hidden);  // token row b*seq + s
    const int c = (int)(idx % hidden);
    const int b = r / seq, s = r % seq;
    const int p = (pos0 ? *pos0 : 0) + s;
    const int id = p < cap ? tokens[(size_t)b * cap + p] : -1;
    out[idx] = (id >= 0 && id < vocab) ? table[(size_t)id * hidden + c] : 0.0f;
}

hipError_t launch_embed(const float* table, int vocab, int hidden, const int* tokens, int cap,
                        const int* pos0, int batch, int seq, float* out, hipStream_t s) {
    const long total = (long)batch * seq * hidden;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, table,
                       vocab, hidden, tokens, cap, pos0, batch, seq, out);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// fp32 LM head, logits[r][v] = fp32(sum_d fp64(x[r][d]) * fp64(table[v][d])),
// in either of loom's two orders (applyFP32LMHeadRows,
// poly/transformer.go:664-719):
//  - DOTTILE (SIMD forward on; amd64 DotTile, poly/simd/avx2_amd64.s:14-79,
//    which every architecture's DotTile matches): eight fp64 lane partials
//    p_l over the 8-column chunks in chunk order, then
//    ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)) + 0, then the n%8 tail in order;
//  - sequential (SIMD forward off, poly/transformer.go:681-687, = dotTileGo,
//    poly/simd/dot.go:14-21): one fp64 chain, sum += x[d]*w[d] in order.
// The product of two fp32 values is exact in fp64, so an FMA rounds exactly
// as the separate multiply and add do.  Each thread owns one logit (the
// eight DotTile partials are eight independent chains of that thread): a
// workgroup covers 256 logits and stages 64-column slabs of its 256 table
// rows through LDS (16 threads read one 256-byte row segment), the next
// slab's loads in flight while the current one is summed.  The row pitch of
// 65 floats keeps the per-thread column reads and the staging stores free of
// bank conflicts.  A slab is a whole number of 8-column chunks, so the n%8
// tail always lies in the last slab.
// ------------------------------------------------------------------------

constexpr int kHeadLogits = 256;
constexpr int kHeadSlab = 64;

template <bool VEC, bool DOTTILE>
__global__ __launch_bounds__(256) void lm_head_kernel(const float* __restrict__ table, int vocab,
                                                      int hidden, const float* __restrict__ x,
                                                      float* __restrict__ logits) {
    __shared__ float slab[kHeadLogits][kHeadSlab + 1];
    extern __shared__ float xs[];  // hidden
    const int tid = threadIdx.x;
    const int v0 = blockIdx.x * kHeadLogits;
    x += (size_t)blockIdx.y * hidden;
    logits += (size_t)blockIdx.y * vocab;
    for (int i = tid; i < hidden; i += 256) xs[i] = x[i];
    constexpr int C4N = kHeadSlab / 4;           // threads per row segment
    constexpr int NL = kHeadLogits * C4N / 256;  // float4 loads per thread per slab
    const int lcol = (tid % C4N) * 4;
    const float* srow[NL];
#pragma unroll
    for (int it = 0; it < NL; ++it) {
        srow[it] = table + (size_t)min(v0 + tid / C4N + it * (256 / C4N), vocab - 1) * hidden;
    }
    // Loads past the last column are clamped and never stored.  Every slab
    // but the last issues the next slab's loads with no branch around them (a
    // branch would make the compiler wait for them at once); the staging
    // registers are a plain unrolled array (no lambda captures it, so it stays
    // in VGPRs).
#define LAMD_HEAD_LOAD(C0)                                                             \
    _Pragma("unroll") for (int it = 0; it < NL; ++it) {                              \
        const int c = (C0) + lcol;                                                   \
        if (VEC) {                                                                   \
            nx[it] = load16_nt((const float4*)(srow[it] + min(c, hidden - 4)));      \
        } else {                                                                     \
            nx[it] = make_float4(srow[it][min(c, hidden - 1)],                       \
                                 srow[it][min(c + 1, hidden - 1)],                   \
                                 srow[it][min(c + 2, hidden - 1)],                   \
                                 srow[it][min(c + 3, hidden - 1)]);                  \
        }                                                                            \
    }
#define LAMD_HEAD_STORE(W)                                                             \
    _Pragma("unroll") for (int it = 0; it < NL; ++it) {                              \
        float* d = &slab[tid / C4N + it * (256 / C4N)][lcol];                        \
        if (lcol < (W)) d[0] = nx[it].x;                                             \
        if (lcol + 1 < (W)) d[1] = nx[it].y;                                         \
        if (lcol + 2 < (W)) d[2] = nx[it].z;                                         \
        if (lcol + 3 < (W)) d[3] = nx[it].w;                                         \
    }
    // one 8-column chunk at slab column K into the lane partials (DOTTILE) or
    // the single chain
#define LAMD_HEAD_CHUNK(C0, K)                                                         \
    _Pragma("unroll") for (int j = 0; j < 8; ++j) {                                  \
        const double prod_x = (double)xs[(C0) + (K) + j];                            \
        const double prod_w = (double)slab[tid][(K) + j];                            \
        if (DOTTILE) {                                                               \
            pl[j] = fma(prod_x, prod_w, pl[j]);                                      \
        } else {                                                                     \
            pl[0] = fma(prod_x, prod_w, pl[0]);                                      \
        }                                                                            \
    }
    float4 nx[NL];
    double pl[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pl[j] = 0.0;
    const int nsl = (hidden + kHeadSlab - 1) / kHeadSlab;
    LAMD_HEAD_LOAD(0)
    for (int i = 0; i + 1 < nsl; ++i) {
        const int c0 = i * kHeadSlab;
        __syncthreads();  // the previous slab is summed (and xs is written)
        LAMD_HEAD_STORE(kHeadSlab)
        LAMD_HEAD_LOAD(c0 + kHeadSlab)
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kHeadSlab; k += 8) LAMD_HEAD_CHUNK(c0, k)
    }
    const int c0 = (nsl - 1) * kHeadSlab;
    const int width = hidden - c0;
    const int wfull = DOTTILE ? (width / 8) * 8 : 0;  // whole chunks of the last slab
    __syncthreads();
    LAMD_HEAD_STORE(width)
    __syncthreads();
    for (int k = 0; k < wfull; k += 8) LAMD_HEAD_CHUNK(c0, k)
#undef LAMD_HEAD_LOAD
#undef LAMD_HEAD_STORE
#undef LAMD_HEAD_CHUNK
    double r = pl[0];
    if (DOTTILE) r = (((pl[0] + pl[4]) + (pl[2] + pl[6])) + ((pl[1] + pl[5]) + (pl[3] + pl[7]))) + 0.0;
    for (int c = wfull; c < width; ++c) r = fma((double)xs[c0 + c], (double)slab[tid][c], r);
    if (v0 + tid < vocab) logits[v0 + tid] = (float)r;
}

template <bool DOTTILE>
static hipError_t launch_head(const float* table, int vocab, int hidden, const float* x, int rows,
                              float* logits, hipStream_t s) {
    if (vocab <= 0 || hidden <= 0 || rows <= 0) return hipSuccess;
    const size_t shm = (size_t)hidden * sizeof(float);
    if (shm > 64 * 1024) return hipErrorInvalidValue;
    const dim3 g((unsigned)ceil_div(vocab, kHeadLogits), rows), b(256);
    if (hidden % 4 == 0 && ((uintptr_t)table & 15) == 0) {
        hipLaunchKernelGGL((lm_head_kernel<true, DOTTILE>), g, b, shm, s, table, vocab, hidden, x,
                           logits);
    } else {
        hipLaunchKernelGGL((lm_head_kernel<false, DOTTILE>), g, b, shm, s, table, vocab, hidden, x,
                           logits);
    }
    return hipGetLastError();
}

hipError_t launch_lm_head(const float* table, int vocab, int hidden, const float* x, int rows,
                          float* logits, hipStream_t s) {
    return launch_head<true>(table, vocab, hidden, x, rows, logits, s);
}

hipError_t launch_lm_head_seq(const float* table, int vocab, int hidden, const float* x, int rows,
                              float* logits, hipStream_t s) {
    return launch_head<false>(table, vocab, hidden, x, rows, logits, s);
}

// ------------------------------------------------------------------------
// greedy SampleTopK (poly/sampling.go:44-55): first strict maximum.  Equal to
// the smallest index holding the largest non-NaN value, except that a NaN at
// index 0 is never replaced.  One 1024-thread workgroup.
// ------------------------------------------------------------------------

// (value, index) order of the greedy pick: larger value first, then the
// smaller index; NaN never wins.
__device__ __forceinline__ bool beats(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// stage 1: partial argmax of `chunk` consecutive logits per workgroup
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits, int n,
                                                             int chunk, float2* __restrict__ part) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const float* lg = logits + (size_t)blockIdx.y * n;
    const int i0 = blockIdx.x * chunk, i1 = min(n, i0 + chunk);
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = i0 + threadIdx.x; i < i1; i += 256) {
        const float v = lg[i];
        if (beats(v, i, best, idx)) {
            best = v;
            idx = i;
        }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w && beats(bv[threadIdx.x + w], bi[threadIdx.x + w], bv[threadIdx.x], bi[threadIdx.x])) {
            bv[threadIdx.x] = bv[threadIdx.x + w];
            bi[threadIdx.x] = bi[threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        part[(size_t)blockIdx.y * gridDim.x + blockIdx.x] = make_float2(bv[0], __int_as_float(bi[0]));
    }
}

// stage 2: combine the partials of one row and store the token
// (lkey, when set: the screened head's threshold, cleared for the next pick)
__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ logits, int n,
                                                          const float2* __restrict__ part, int parts,
                                                          int* __restrict__ tokens, int cap,
                                                          const int* __restrict__ pos0, int offset,
                                                          unsigned long long* __restrict__ lkey) {
    const float2* pr = part + (size_t)blockIdx.x * parts;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int j = threadIdx.x; j < parts; j += 64) {
        const float2 e = pr[j];
        const int i = __float_as_int(e.y);
        if (beats(e.x, i, best, idx)) {
            best = e.x;
            idx = i;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_down(best, off, 64);
        const int oi = __shfl_down(idx, off, 64);
        if (beats(ov, oi, best, idx)) {
            best = ov;
            idx = oi;
        }
    }
    if (threadIdx.x == 0) {
        const float first = logits[(size_t)blockIdx.x * n];
        int r = idx;
        if (first != first || r == 0x7fffffff) r = 0;  // NaN at 0, or nothing comparable
        const int p = (pos0 ? *pos0 : 0) + offset;
        if (p < cap) tokens[(size_t)blockIdx.x * cap + p] = r;
        if (lkey) *lkey = 0ull;
    }
}

int argmax_parts(int n) { return min(kArgmaxMaxParts, max(1, ceil_div(n, 4096))); }

hipError_t launch_argmax(const float* logits, int n, int rows, float2* part, int* tokens, int cap,
                         const int* pos0, int offset, hipStream_t s) {
    if (n <= 0 || rows <= 0) return hipErrorInvalidValue;
    const int parts = argmax_parts(n);
    const int chunk = ceil_div(n, parts);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts, rows), dim3(256), 0, s, logits, n, chunk, part);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, s, logits, n, part, parts, tokens,
                       cap, pos0, offset, nullptr);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// Greedy token of the fp32 LM head for one row, by screening.  Greedy
// decoding needs the argmax of the logits, not every logit.  An int8 copy of
// the table (per vocab row v a scale s_v = max_j |w_vj| / 127 and codes
// q_vj = round(w_vj / s_v), so |w_vj - s_v q_vj| <= s_v (1/2 + 2^-14)) gives
// for every row, reading a quarter of the bytes,
//   A_v = s_v * sum_j x_j q_vj   (one fp32 multiply-add chain per row, then an fp64 product)
// and, with X1 = sum_j |x_j|, the bound |F_v - A_v| <= B_v on loom's logit
// F_v = fp32(fp64 sum of x_j w_vj in its order):
//   B_v = s_v X1 (1/2 + 2^-14 + 127 (g32 + g64)) + 2^-24 (|A_v| + s_v X1)
//         + 2^-150, widened by 2^-20,
// which covers the codes' rounding, the fp32 and fp64 summation errors
// (g_p = n 2^-p / (1 - n 2^-p), n = hidden + 64; |q| <= 127 and
// |w| <= 127.01 s) and the final rounding to fp32.  Every row with
// A_v + B_v >= L, where L = max_u (A_u - B_u), is a candidate: the greedy pick
// g is one, since A_g + B_g >= F_g >= F_u >= A_u - B_u for every row u, and so
// is every row tying with it.  So are row 0 (the greedy rule reads logit 0)
// and every row whose scale, sum or bound is not finite or reaches 2^127 (a
// non-finite entry makes its scale NaN; its logit may be non-finite or
// overflow; such rows stay out of L).  The candidates' logits are computed
// exactly as lm_head_kernel computes them, from the fp32 table, and the
// greedy pick over them is the pick over all logits.  Only the candidates'
// logits are written; a caller that wants every logit runs lm_head_kernel.
// L crosses the grid as a monotone 64-bit key (device-scope atomic maximum);
// the final pick clears it for the next call.
// ------------------------------------------------------------------------

// order-preserving key of a non-NaN double (0 is below every key: "none")
__device__ __forceinline__ unsigned long long lm_order_key(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
__device__ __forceinline__ double lm_key_value(unsigned long long k) {
    if (k == 0ull) return -INFINITY;
    const unsigned long long b = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
    return __longlong_as_double((long long)b);
}

// one workgroup per vocab row: the row's scale (NaN when an entry is not
// finite) and codes
__global__ __launch_bounds__(256) void lm_quant_rows_kernel(const float* __restrict__ w, int hidden,
                                                            int8_t* __restrict__ q, float* __restrict__ scale) {
    __shared__ float red[4];
    __shared__ int bad[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* row = w + (size_t)blockIdx.x * hidden;
    float m = 0.0f;
    int nf = 0;
    for (int j = tid; j < hidden; j += 256) {
        const float v = row[j];
        nf |= !(fabsf(v) <= 3.4028235e38f);  // NaN or Inf
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max(m);
    nf = wave_sum_i(nf);
    if (lane == 0) {
        red[wave] = m;
        bad[wave] = nf;
    }
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    nf = bad[0] | bad[1] | bad[2] | bad[3];
    const float s = m / 127.0f;
    // a scale below the normal range rounds too coarsely for the bound: such a
    // row (and one with a non-finite entry) gets scale NaN, i.e. is always a
    // candidate
    const bool bad_row = nf || (m > 0.0f && s < 1.17549435e-38f);
    // interleaved layout: 16-column group t of row v at byte
    // ((v / 64 * (hidden / 16) + t) * 64 + v % 64) * 16
    const int v = blockIdx.x;
    int8_t* qb = q + ((size_t)(v >> 6) * (hidden / 16) * 64 + (v & 63)) * 16;
    for (int j = tid; j < hidden; j += 256) {
        const float r = (bad_row || s == 0.0f) ? 0.0f : rintf(row[j] / s);
        qb[(size_t)(j >> 4) * 1024 + (j & 15)] = (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
    }
    if (tid == 0) scale[v] = bad_row ? __builtin_nanf("") : s;
}

size_t lm_screen_code_bytes(int vocab, int hidden) { return (size_t)ceil_div(vocab, 64) * 64 * hidden; }

hipError_t launch_lm_quant_rows(const float* w, int vocab, int hidden, int8_t* q, float* scale, hipStream_t s) {
    if (vocab <= 0 || hidden <= 0) return hipSuccess;
    hipLaunchKernelGGL(lm_quant_rows_kernel, dim3(vocab), dim3(256), 0, s, w, hidden, q, scale);
    return hipGetLastError();
}

constexpr int kScreenMaxHidden = 2816;  // the pick's x and four staged rows within 64 KB of LDS
constexpr int kScreenBlocks = 1024;
constexpr int kPickRows = 256;          // vocab rows per workgroup of the pick

bool lm_screen_ok(int hidden) { return hidden > 0 && hidden % 16 == 0 && hidden <= kScreenMaxHidden; }
int lm_screen_parts(int vocab) { return ceil_div(vocab, kPickRows); }

// wave maximum of doubles (no NaN), -inf where no lane has a value
__device__ __forceinline__ double wave_max_f64_ninf(double v) {
#define LAMD_MAXSTEP(C)                                   \
    {                                                     \
        const double o = dpp_d<C>(v, -INFINITY);          \
        v = o > v ? o : v;                                \
    }
    LAMD_MAXSTEP(kDppShr1) LAMD_MAXSTEP(kDppShr2) LAMD_MAXSTEP(kDppShr4) LAMD_MAXSTEP(kDppShr8)
    LAMD_MAXSTEP(kDppBcast15) LAMD_MAXSTEP(kDppBcast31)
#undef LAMD_MAXSTEP
    return readlane63_d(v);
}

// A wave per 64 vocab rows, lane l owning row 64 * blk + l: in the interleaved
// code layout the wave's 16-byte loads of one 16-column group cover 1 KB
// contiguously, and every lane reads the same x values from LDS (broadcast),
// so no sum crosses lanes.  A row past the vocabulary (the last block's
// padding) is summed but never stored.
__global__ __launch_bounds__(256) void lm_screen_kernel(const uint4* __restrict__ qt, const float* __restrict__ scale,
                                                        int vocab, int hidden, const float* __restrict__ x, double k1,
                                                        double* __restrict__ hi,
                                                        unsigned long long* __restrict__ lkey) {
    extern __shared__ float xs[];  // hidden
    __shared__ double wl[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int T = hidden / 16;
    for (int i = tid; i < hidden / 4; i += 256) ((float4*)xs)[i] = ((const float4*)x)[i];
    __syncthreads();
    double x1 = 0.0;
    for (int i = lane; i < hidden; i += 64) x1 += fabs((double)xs[i]);
    x1 = wave_sum_f64_dpp(x1);
    double best = -INFINITY;  // largest A - B of this wave's finite rows
    const int nblk = (vocab + 63) / 64;
    for (int blk = blockIdx.x * 4 + wave; blk < nblk; blk += gridDim.x * 4) {  // wave-uniform
        const uint4* src = qt + (size_t)blk * T * 64 + lane;
        float a = 0.0f;
#pragma unroll 8
        for (int t = 0; t < T; ++t) {
            const uint4 w = load16_nt(src + (size_t)t * 64);
            const float4* xt = (const float4*)(xs + 16 * t);
            const float4 xa[4] = {xt[0], xt[1], xt[2], xt[3]};
            const unsigned c[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a = fmaf(xa[e].x, (float)(int8_t)(c[e]), a);
                a = fmaf(xa[e].y, (float)(int8_t)(c[e] >> 8), a);
                a = fmaf(xa[e].z, (float)(int8_t)(c[e] >> 16), a);
                a = fmaf(xa[e].w, (float)(int8_t)(c[e] >> 24), a);
            }
        }
        const int v = blk * 64 + lane;
        if (v < vocab) {
            const double s = (double)scale[v];
            const double A = s * (double)a;
            const double sx = s * x1;
            const double B = (k1 * sx + 0x1p-24 * (fabs(A) + sx) + 0x1p-150) * (1.0 + 0x1p-20);
            const bool ok = fabs(A) + B < 0x1p127;  // false for NaN and Inf too
            if (ok) best = A - B > best ? A - B : best;
            hi[v] = ok ? A + B : INFINITY;
        }
    }
    best = wave_max_f64_ninf(best);
    if (lane == 0) wl[wave] = best;
    __syncthreads();
    if (tid == 0) {
        double m = wl[0];
        for (int w = 1; w < 4; ++w) m = wl[w] > m ? wl[w] : m;
        if (m > -INFINITY) __hip_atomic_fetch_max(lkey, lm_order_key(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// kPickRows rows per workgroup: the candidates among them, their exact
// logits and the workgroup's greedy pick into part[blockIdx.x].  A wave takes
// one candidate at a time: it stages the candidate's fp32 row in its own LDS
// region (16-byte loads, one round trip), then lanes 0-7 run the eight
// DotTile chains (or lane 0 the sequential chain) from LDS.
template <bool DOTTILE>
__global__ __launch_bounds__(256) void lm_pick_kernel(const float* __restrict__ table, int vocab, int hidden,
                                                      const float* __restrict__ x, const double* __restrict__ hi,
                                                      const unsigned long long* __restrict__ lkey,
                                                      float* __restrict__ logits, float2* __restrict__ part) {
    extern __shared__ float xs[];  // x, then one row region per wave: 5 x hidden
    __shared__ int cand[kPickRows];
    __shared__ int ncand;
    __shared__ double pp[4][8];
    __shared__ float bv[256];
    __shared__ int bi[256];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid == 0) ncand = 0;
    const int h4 = hidden / 4;
    for (int i = tid; i < h4; i += 256) ((float4*)xs)[i] = ((const float4*)x)[i];  // (loads with hi[v])
    __syncthreads();
    const double L = lm_key_value(*lkey);
    const int v = blockIdx.x * kPickRows + tid;
    if (v < vocab && (v == 0 || hi[v] >= L)) cand[atomicAdd(&ncand, 1)] = v;
    __syncthreads();
    const int nc = ncand;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    if (nc > 0) {  // uniform
        float* rw = xs + (size_t)(1 + wave) * hidden;
        for (int ci = wave; ci < nc; ci += 4) {  // wave-uniform
            const int vv = cand[ci];
            const float4* src = (const float4*)(table + (size_t)vv * hidden);
            for (int i = lane; i < h4; i += 64) ((float4*)rw)[i] = src[i];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // the wave's row stores are done before its lanes read
            __builtin_amdgcn_wave_barrier();
            double r = 0.0;
            if constexpr (DOTTILE) {
                const int nk = hidden / 8;
                if (lane < 8) {
                    double p = 0.0;
#pragma unroll 16
                    for (int k = 0; k < nk; ++k) p = fma((double)xs[8 * k + lane], (double)rw[8 * k + lane], p);
                    pp[wave][lane] = p;
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);
                __builtin_amdgcn_wave_barrier();
                if (lane == 0) {
                    r = (((pp[wave][0] + pp[wave][4]) + (pp[wave][2] + pp[wave][6])) +
                         ((pp[wave][1] + pp[wave][5]) + (pp[wave][3] + pp[wave][7]))) + 0.0;
                    for (int c = 8 * nk; c < hidden; ++c) r = fma((double)xs[c], (double)rw[c], r);
                }
            } else if (lane == 0) {
#pragma unroll 8
                for (int c = 0; c < hidden; ++c) r = fma((double)xs[c], (double)rw[c], r);
            }
            if (lane == 0) {
                const float f = (float)r;
                logits[vv] = f;
                if (beats(f, vv, best, bidx)) {
                    best = f;
                    bidx = vv;
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();  // the region and pp are rewritten by the next candidate
        }
    }
    bv[tid] = best;
    bi[tid] = bidx;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w && beats(bv[tid + w], bi[tid + w], bv[tid], bi[tid])) {
            bv[tid] = bv[tid + w];
            bi[tid] = bi[tid + w];
        }
        __syncthreads();
    }
    if (tid == 0) part[blockIdx.x] = make_float2(bv[0], __int_as_float(bi[0]));
}

hipError_t launch_lm_greedy_screened(const float* table, const int8_t* table_q, const float* scale, int vocab,
                                     int hidden, const float* x, int sequential, double* hi,
                                     unsigned long long* lkey, float* logits, float2* part, int* tokens, int cap,
                                     const int* pos0, int offset, hipStream_t s) {
    if (vocab <= 0 || !lm_screen_ok(hidden) || ((uintptr_t)table_q & 15) != 0) return hipErrorInvalidValue;
    const double n = (double)hidden + 64.0;
    const double g32 = n * 0x1p-24 / (1.0 - n * 0x1p-24);
    const double g64 = n * 0x1p-53 / (1.0 - n * 0x1p-53);
    const double k1 = 0.5 + 0x1p-14 + 127.0 * (g32 + g64) * (1.0 + 0x1p-10);
    const int blocks = min(kScreenBlocks, ceil_div(ceil_div(vocab, 64), 4));
    hipLaunchKernelGGL(lm_screen_kernel, dim3(blocks), dim3(256), (size_t)hidden * sizeof(float), s,
                       (const uint4*)table_q, scale, vocab, hidden, x, k1, hi, lkey);
    const int parts = lm_screen_parts(vocab);
    const size_t shm = (size_t)5 * hidden * sizeof(float);  // x and four staged rows
    if (sequential)
        hipLaunchKernelGGL(lm_pick_kernel<false>, dim3(parts), dim3(256), shm, s, table, vocab, hidden, x, hi, lkey,
                           logits, part);
    else
        hipLaunchKernelGGL(lm_pick_kernel<true>, dim3(parts), dim3(256), shm, s, table, vocab, hidden, x, hi, lkey,
                           logits, part);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, s, logits, vocab, part, parts, tokens, cap, pos0,
                       offset, lkey);
    return hipGetLastError();
}

// position bookkeeping on the device (graph-replayable)
__global__ void set_int_kernel(int* p, int v) { *p = v; }
__global__ void add_int_kernel(int* p, int v) { *p += v; }

hipError_t launch_set_int(int* p, int v, hipStream_t s) {
    hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, s, p, v);
    return hipGetLastError();
}

hipError_t launch_add_int(int* p, int v, hipStream_t s) {
    hipLaunchKernelGGL(add_int_kernel, dim3(1), dim3(1), 0, s, p, v);
    return hipGetLastError();
}

}  // namespace lamd
