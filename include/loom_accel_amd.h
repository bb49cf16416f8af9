/*
 * loom_accel_amd.h -- device-resident extension of libloom_accel_amd.so.
 *
 * loom's v2 plugin ABI (loom_accel.h) moves fp32 host buffers per call,
 * which costs two PCIe copies per layer.  These extra symbols keep weights,
 * activations and intermediates in HBM so a caller (loom's cgo glue, or the
 * Python host mirror in loom_amd/) can chain layers without host round trips.
 * They do not change LOOM_ACCEL_API_VERSION: loom's loader only resolves the
 * v2 symbols and ignores these.
 *
 * Conventions:
 *   - every pointer named x, out, pre, post, residual, bias, inner_norm, h_out,
 *     xq, amax, xsum, acc* or hq is DEVICE memory on the matrix's device;
 *   - stream is a hipStream_t (NULL = the legacy default stream); calls are
 *     asynchronous on it unless stated otherwise;
 *   - return 0 on success, -1 on failure with loom_amd_last_error() set;
 *   - the library keeps one scratch arena per device for quantized
 *     activations; calls that overlap on one device (two host threads, or
 *     two streams) race on it and must be serialized by the caller.
 *
 * Activation ids are loom's ActivationType (poly/poly.go:89-98):
 * 0 ReLU, 1 SiLU, 2 GELU, 3 Tanh, 4 Sigmoid, 5 LeakyReLU, 6 ReLU2, -1 Linear.
 */
#ifndef LOOM_ACCEL_AMD_H
#define LOOM_ACCEL_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct loom_amd_matrix loom_amd_matrix;

/* Inner-norm summation order of the SwiGLU / row-norm entry points. */
#define LOOM_AMD_NORM_STRICT 1 /* loom's sequential fp64 sum: bit-exact */
#define LOOM_AMD_NORM_FAST 0   /* parallel fixed-order fp64 sum: <= 1 fp32 ulp */

/* Message of the last failing loom_amd_* call on the calling thread. */
const char* loom_amd_last_error(void);

/* Number of visible gfx950 devices (0 when none). */
int loom_amd_device_count(void);

/* Kernel family the matmul dispatcher uses for m token rows
 * ("skinny_m16_fusedq" -- quantization fused into the matmul launch when the
 * fp32 rows allow it --, "skinny_m16", "skinny_m32", "skinny_m64", "gemm"). */
const char* loom_amd_kernel_variant(int m);

/* ---- weights --------------------------------------------------------- */

/* Upload loom BitNetTernaryMatrix words (host, row-major, 16 codes per u32,
 * poly/bitnet_cpu.go:14-43) and repack them once into the gfx950 tile
 * layout.  Synchronous.  Replaces GetBitNetTernaryMatrix's packed cache
 * (poly/bitnet_cpu.go:312-355) on the GPU side. */
int loom_amd_matrix_create(int device, const uint32_t* words, size_t n_words, int rows,
                           int cols, int row_words, float scale, loom_amd_matrix** out);

/* Same, from one .entity BITNET_TERNARY blob (poly/entity_bitnet.go:38-88)
 * in host memory; *consumed receives the blob's byte length. */
int loom_amd_matrix_from_entity_blob(int device, const void* blob, size_t len,
                                     loom_amd_matrix** out, size_t* consumed);

void loom_amd_matrix_release(loom_amd_matrix* m);

int loom_amd_matrix_shape(const loom_amd_matrix* m, int* rows, int* cols, float* scale,
                          size_t* device_bytes);

/* Device pointer of the repacked tiles (read-only; for inspection). */
const void* loom_amd_matrix_tiles(const loom_amd_matrix* m);

/* ---- stages ---------------------------------------------------------- */

/* bitNetQuantizeActivationNumeric per row (poly/bitnet_cpu.go:45-106):
 * x m*k fp32 -> xq (m rows of ldq bytes, zero padded past k; ldq >= k and
 * a multiple of 256), amax (m), xsum = sum(xq) per row (m). */
int loom_amd_quantize_rows(const float* x, int m, int k, int8_t* xq, int ldq, float* amax,
                           int32_t* xsum, void* stream);

/* bitNetQuantizeActivationFloat64 per row (poly/bitnet_cpu.go:59-71,108-117). */
int loom_amd_quantize_rows_f64(const double* x, int m, int k, int8_t* xq, int ldq,
                               float* amax, int32_t* xsum, void* stream);

/* bitNetTernaryMatVecQuantized for m rows at once (poly/bitnet_cpu.go:536-546):
 * out[i][n] = fp32(fp64(acc) * (fp64(scale)*fp64(amax[i]))/127), and
 * acc (optional, m*n int32) = sum_k xq[i][k] * w[n][k]. */
int loom_amd_ternary_matmul(const loom_amd_matrix* w, const int8_t* xq, int ldq,
                            const float* amax, const int32_t* xsum, int m, float* out,
                            int32_t* acc, void* stream);

/* bitNetRMSNormTensorRowWeighted + requantization of m rows of n fp32, in
 * place on h (poly/bitnet_cpu.go:893-913, then 97-106).  weight NULL = 1. */
int loom_amd_norm_quant_rows(float* h, int m, int n, const float* weight, double eps,
                             int norm_mode, int8_t* hq, int ldq, float* amax, int32_t* xsum,
                             void* stream);

/* ---- layers ---------------------------------------------------------- */

typedef struct loom_amd_dense_taps {
    int8_t* xq;   /* m*k, optional */
    float* amax;  /* m, optional */
    int32_t* acc; /* m*n, optional */
} loom_amd_dense_taps;

/* DenseForwardPackedTernaryCPU (poly/dense.go:66-101) for m token rows:
 * pre = fp32(matvec), post = Activate(pre) (optional), and, when residual
 * is given, pre = fp32(pre + residual) as loom's Tensor.Add
 * (poly/poly.go:481-494) would add it afterwards. */
int loom_amd_dense_forward(const loom_amd_matrix* w, const float* x, int m, int activation,
                           float* pre, float* post, const float* residual,
                           const loom_amd_dense_taps* taps, void* stream);

typedef struct loom_amd_swiglu_taps {
    int8_t* xq;        /* m*hidden */
    float* amax;       /* m */
    int32_t* acc_gate; /* m*inter */
    int32_t* acc_up;   /* m*inter */
    int8_t* hq;        /* m*inter, requantized normalized rows */
    float* hamax;      /* m */
    int32_t* acc_down; /* m*hidden */
} loom_amd_swiglu_taps;

/* SwiGLUForwardPackedTernaryCPU (poly/swiglu.go:270-322) for m token rows:
 * gate/up share one quantization of x; h = fp32(gateprod(g, u)); inner
 * RMSNorm (eps <= 0 -> 1e-5, inner_norm NULL -> weight 1); requantize;
 * down; out = fp32(down + bias) [+ residual in fp32].
 * bias: NULL or device [gate inter | up inter | down hidden] fp32.
 * h_out: optional m*inter fp32, loom's preAct (normalized rows). */
int loom_amd_swiglu_forward(const loom_amd_matrix* gate, const loom_amd_matrix* up,
                            const loom_amd_matrix* down, const float* bias,
                            const float* inner_norm, double eps, int activation,
                            int norm_mode, const float* x, int m, float* out,
                            const float* residual, float* h_out,
                            const loom_amd_swiglu_taps* taps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOOM_ACCEL_AMD_H */
