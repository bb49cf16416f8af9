/*
 * bitnet_oracle.c -- CPU restatement of loom's BitNet b1.58 CPU path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.
 * Nothing in libloom_accel_amd.so links, loads or calls this code.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).  fp
 * contraction is off so every fp64 expression rounds after each operation,
 * the way Go's amd64 compiler (GOAMD64=v1, no FMA fusion) evaluates the
 * reference's source.
 *
 * Citations: paths relative to the loom v0.83.0 tree.
 */
#define _GNU_SOURCE
#include "bitnet_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Go conversion semantics                                             */
/* ------------------------------------------------------------------ */

/* Go's int(float64) on amd64 compiles to CVTTSD2SQ: NaN and values outside
 * the int64 range produce the "integer indefinite" 0x8000000000000000.
 * Inputs here are already integral (math.Round output). */
static int64_t go_int_from_f64(double r) {
    if (isnan(r) || r >= 9223372036854775808.0 || r < -9223372036854775808.0) {
        return INT64_MIN;
    }
    return (int64_t)r;
}

/* ------------------------------------------------------------------ */
/* Activation quantization                                             */
/* ------------------------------------------------------------------ */

/* bitNetActivationMaxAbs (poly/bitnet_cpu.go:45-57): max of float32(|float64(v)|),
 * floored at float32(1e-5).  NaN never wins the strict '>' comparison. */
float orc_act_maxabs_f32(const float* x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = (float)fabs((double)x[i]);
        if (a > m) {
            m = a;
        }
    }
    if (m < 1e-5f) {
        return 1e-5f;
    }
    return m;
}

/* bitNetActivationMaxAbsFloat64 (poly/bitnet_cpu.go:59-71): |v| in fp64 rounded to fp32. */
float orc_act_maxabs_f64(const double* x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = (float)fabs(x[i]);
        if (a > m) {
            m = a;
        }
    }
    if (m < 1e-5f) {
        return 1e-5f;
    }
    return m;
}

/* bitNetQuantizedActivation / ...Float64 (poly/bitnet_cpu.go:73-95):
 * scale = 127/float64(amax) (fp64 divide), q = round_half_away(v*scale)
 * (fp64 multiply), clamp to [-128,127].  NaN -> int64 indefinite -> -128. */
int8_t orc_quant_value_act(double v, float amax) {
    double scale = 127.0 / (double)amax;
    int64_t q = go_int_from_f64(round(v * scale));
    if (q < -128) {
        q = -128;
    }
    if (q > 127) {
        q = 127;
    }
    return (int8_t)q;
}

/* bitNetQuantizeActivationNumeric (poly/bitnet_cpu.go:97-106). */
float orc_quant_act_f32(const float* x, int n, int8_t* q) {
    float amax = orc_act_maxabs_f32(x, n);
    for (int i = 0; i < n; i++) {
        q[i] = orc_quant_value_act((double)x[i], amax);
    }
    return amax;
}

/* bitNetQuantizeActivationFloat64 (poly/bitnet_cpu.go:108-117). */
float orc_quant_act_f64(const double* x, int n, int8_t* q) {
    float amax = orc_act_maxabs_f64(x, n);
    for (int i = 0; i < n; i++) {
        q[i] = orc_quant_value_act(x[i], amax);
    }
    return amax;
}

/* ------------------------------------------------------------------ */
/* Weight quantization and packing                                     */
/* ------------------------------------------------------------------ */

/* bitNetTernaryScale (poly/bitnet_cpu.go:119-132): absmean, fp64 sequential sum. */
float orc_ternary_scale(const float* w, long n) {
    if (n == 0) {
        return 1.0f;
    }
    double sum_abs = 0.0;
    for (long i = 0; i < n; i++) {
        sum_abs += fabs((double)w[i]);
    }
    float scale = (float)(sum_abs / (double)n);
    if (scale == 0.0f) {
        return 1.0f;
    }
    return scale;
}

/* bitNetQuantValue (poly/bitnet_cpu.go:134-146): v/scale is an fp32 divide,
 * rounded half away from zero in fp64, clamped to {-1,0,1}, stored as uint8(int8). */
uint8_t orc_quant_value(float v, float scale) {
    if (scale == 0.0f) {
        scale = 1.0f;
    }
    float ratio = v / scale;
    int64_t q = go_int_from_f64(round((double)ratio));
    if (q > 1) {
        q = 1;
    }
    if (q < -1) {
        q = -1;
    }
    return (uint8_t)(int8_t)q;
}

/* ternaryStorageToCode (poly/bitnet_cpu.go:498-507): -1 -> 0, +1 -> 2, else 1. */
uint8_t orc_storage_to_code(uint8_t v) {
    switch ((int8_t)v) {
        case -1:
            return 0;
        case 1:
            return 2;
        default:
            return 1;
    }
}

/* packTernaryRowsToU32 (poly/bitnet_cpu.go:964-977): row-major, 16 codes per
 * u32, code of column c at bits 2*(c%16) of word c/16. */
void orc_pack_ternary_rows(const uint8_t* native, int rows, int cols, uint32_t* words) {
    int row_words = (cols + 15) / 16;
    memset(words, 0, (size_t)rows * (size_t)row_words * sizeof(uint32_t));
    for (int r = 0; r < rows; r++) {
        const uint8_t* src = native + (size_t)r * (size_t)cols;
        uint32_t* dst = words + (size_t)r * (size_t)row_words;
        for (int c = 0; c < cols; c++) {
            uint32_t code = orc_storage_to_code(src[c]);
            dst[c / 16] |= code << ((c % 16) * 2);
        }
    }
}

/* packFloat32AsBitNetTernaryMatrix (poly/bitnet_cpu.go:934-962), including the
 * alreadyTernary quirk: a master whose every value is within 1e-6 of {-1,0,1}
 * is packed at scale 1.  Returns the scale; words sized rows*ceil(cols/16). */
float orc_pack_float32(const float* w, int rows, int cols, uint32_t* words) {
    long total = (long)rows * (long)cols;
    float scale = orc_ternary_scale(w, total);
    uint8_t* raw = (uint8_t*)malloc((size_t)total);
    int already_ternary = 1;
    for (long i = 0; i < total; i++) {
        float v = w[i];
        if (!(fabs((double)v) < 1e-6 || fabs((double)(v - 1.0f)) < 1e-6 ||
              fabs((double)(v + 1.0f)) < 1e-6)) {
            already_ternary = 0;
        }
        raw[i] = orc_quant_value(v, scale);
    }
    if (already_ternary) {
        scale = 1.0f;
        for (long i = 0; i < total; i++) {
            raw[i] = orc_quant_value(w[i], 1.0f);
        }
    }
    orc_pack_ternary_rows(raw, rows, cols, words);
    free(raw);
    return scale;
}

/* packMicrosoftOfflineBitNetRowsToU32FromBytes (poly/bitnet_cpu.go:1078-1098):
 * byte (pr, c) holds 4 codes; lane l -> row l*(rows/4)+pr; code 3 -> 1. */
void orc_pack_ms_offline_bytes(const uint8_t* packed, int rows, int cols, uint32_t* words) {
    int row_words = (cols + 15) / 16;
    int packed_rows = rows / 4;
    memset(words, 0, (size_t)rows * (size_t)row_words * sizeof(uint32_t));
    for (int pr = 0; pr < packed_rows; pr++) {
        for (int c = 0; c < cols; c++) {
            uint8_t b = packed[(size_t)pr * (size_t)cols + (size_t)c];
            for (int lane = 0; lane < 4; lane++) {
                uint32_t code = (uint32_t)((b >> (lane * 2)) & 0x03);
                if (code > 2) {
                    code = 1;
                }
                int row = lane * packed_rows + pr;
                words[(size_t)row * (size_t)row_words + (size_t)(c / 16)] |= code << ((c % 16) * 2);
            }
        }
    }
}

/* packMicrosoftOfflineBitNetRowsToU32FromFloatU8Slots (poly/bitnet_cpu.go:1056-1076). */
void orc_pack_ms_offline_float_slots(const float* packed, int rows, int cols, uint32_t* words) {
    size_t n = (size_t)(rows / 4) * (size_t)cols;
    uint8_t* bytes = (uint8_t*)malloc(n ? n : 1);
    for (size_t i = 0; i < n; i++) {
        bytes[i] = (uint8_t)(int64_t)packed[i];
    }
    orc_pack_ms_offline_bytes(bytes, rows, cols, words);
    free(bytes);
}

/* ------------------------------------------------------------------ */
/* Matvec kernels                                                      */
/* ------------------------------------------------------------------ */

/* bitNetTernaryMatVecQuantized rescale (poly/bitnet_cpu.go:536-546):
 * (float64(scale)*float64(amax))/127, 0 -> 1. */
double orc_output_scale(float weight_scale, float amax) {
    double s = (double)weight_scale * (double)amax / 127.0;
    if (s == 0.0) {
        s = 1.0;
    }
    return s;
}

/* bitNetTernaryWordDot16 (poly/bitnet_cpu.go:810-845). */
int32_t orc_word_dot16(uint32_t word, const int8_t* xq) {
    int32_t sum = 0;
    for (int i = 0; i < 16; i++) {
        int32_t code = (int32_t)((word >> (2 * i)) & 0x03u);
        sum += (int32_t)xq[i] * (code - 1);
    }
    return sum;
}

/* bitNetTernaryWordDotTail (poly/bitnet_cpu.go:847-854). */
int32_t orc_word_dot_tail(uint32_t word, const int8_t* xq, int n) {
    int32_t sum = 0;
    for (int i = 0; i < n; i++) {
        int32_t code = (int32_t)((word >> (2 * i)) & 0x03u);
        sum += (int32_t)xq[i] * (code - 1);
    }
    return sum;
}

/* bitNetRunRows partition (poly/bitnet_cpu.go:780-808): single worker when
 * rows*cols < 262144 or rows < 4, else min(workers, rows) contiguous chunks of
 * ceil(rows/workers) rows. */
void orc_run_rows_plan(int rows, int cols, int workers, int* n_chunks, int* chunk) {
    long work = (long)rows * (long)cols;
    if (work < 262144 || rows < 4 || workers <= 1) {
        *n_chunks = 1;
        *chunk = rows;
        return;
    }
    if (workers > rows) {
        workers = rows;
    }
    int c = (rows + workers - 1) / workers;
    *chunk = c;
    *n_chunks = (rows + c - 1) / c;
}

/* bitNetTernaryMatVecInt8Scalar (poly/bitnet_cpu.go:752-776). */
void orc_matvec_scalar(const uint32_t* words, int rows, int cols, int row_words,
                       const int8_t* xq, double output_scale, double* out,
                       int32_t* acc_out) {
    if (row_words <= 0) {
        row_words = (cols + 15) / 16;
    }
    int full_words = cols / 16;
    int tail_cols = cols % 16;
    for (int r = 0; r < rows; r++) {
        const uint32_t* w = words + (size_t)r * (size_t)row_words;
        int32_t sum = 0;
        int x_off = 0;
        for (int i = 0; i < full_words; i++) {
            sum += orc_word_dot16(w[i], xq + x_off);
            x_off += 16;
        }
        if (tail_cols > 0) {
            sum += orc_word_dot_tail(w[full_words], xq + x_off, tail_cols);
        }
        if (acc_out) {
            acc_out[r] = sum;
        }
        out[r] = (double)sum * output_scale;
    }
}

/* ensureBitNetCodes row stride (poly/bitnet_cpu.go:717). */
int orc_codes_stride(int cols) {
    return ((cols + 31) / 32) * 32;
}

/* ensureBitNetCodes (poly/bitnet_cpu.go:700-729): one unsigned code byte per
 * weight, rows zero-padded to a multiple of 32. */
void orc_ensure_codes(const uint32_t* words, int rows, int cols, int row_words,
                      uint8_t* codes) {
    if (row_words <= 0) {
        row_words = (cols + 15) / 16;
    }
    int stride = orc_codes_stride(cols);
    memset(codes, 0, (size_t)rows * (size_t)stride);
    for (int r = 0; r < rows; r++) {
        const uint32_t* w = words + (size_t)r * (size_t)row_words;
        uint8_t* dst = codes + (size_t)r * (size_t)stride;
        for (int c = 0; c < cols; c++) {
            dst[c] = (uint8_t)((w[c / 16] >> ((c % 16) * 2)) & 0x03u);
        }
    }
}

/* bitNetTernaryCodeRowDotGo (poly/simd/bitnet_ternary.go:18-24). */
int32_t orc_code_row_dot_go(const uint8_t* codes, const int8_t* acts, int n_bytes) {
    int32_t sum = 0;
    for (int i = 0; i < n_bytes; i++) {
        sum += (int32_t)codes[i] * (int32_t)acts[i];
    }
    return sum;
}

/* AVX2 MAD row dot (poly/simd/bitnet_ternary_amd64.s:7-39): per 32 bytes,
 * u8*s8 pair sums to i16 (no saturation: |code*act| <= 384), widen with a
 * multiply-add against ones to i32 lanes, accumulate, then fold 8 lanes.
 * Bytes past the last whole 32-byte chunk are ignored, as in the asm. */
__attribute__((target("avx2")))
int32_t orc_code_row_dot_avx2(const uint8_t* codes, const int8_t* acts, int n_bytes) {
    __m256i acc = _mm256_setzero_si256();
    const __m256i ones = _mm256_set1_epi16(1);
    int chunks = n_bytes >> 5;
    for (int i = 0; i < chunks; i++) {
        __m256i c = _mm256_loadu_si256((const __m256i*)(codes + 32 * i));
        __m256i a = _mm256_loadu_si256((const __m256i*)(acts + 32 * i));
        __m256i p16 = _mm256_maddubs_epi16(c, a);
        __m256i p32 = _mm256_madd_epi16(p16, ones);
        acc = _mm256_add_epi32(acc, p32);
    }
    __m128i lo = _mm256_castsi256_si128(acc);
    __m128i hi = _mm256_extracti128_si256(acc, 1);
    __m128i s = _mm_add_epi32(lo, hi);
    s = _mm_hadd_epi32(s, s);
    s = _mm_hadd_epi32(s, s);
    return _mm_cvtsi128_si32(s);
}

int orc_simd_available(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") ? 1 : 0;
}

/* bitNetTernaryMatVecInt8Simd (poly/bitnet_cpu.go:733-750) with the
 * bitNetRunRows fan-out (poly/bitnet_cpu.go:780-808):
 * out = float64(raw - sum(xq)) * outputScale. */
void orc_matvec_simd(const uint8_t* codes, int rows, int cols, const int8_t* xq,
                     double output_scale, double* out, int32_t* acc_out,
                     int workers) {
    int stride = orc_codes_stride(cols);
    int8_t* acts = (int8_t*)calloc((size_t)stride, 1);
    memcpy(acts, xq, (size_t)cols);
    int32_t act_sum = 0;
    for (int i = 0; i < cols; i++) {
        act_sum += (int32_t)xq[i];
    }
    int use_avx2 = orc_simd_available();
    int n_chunks = 1;
    int chunk = rows;
    orc_run_rows_plan(rows, cols, workers, &n_chunks, &chunk);
#pragma omp parallel for num_threads(n_chunks) schedule(static, 1) if (n_chunks > 1)
    for (int ci = 0; ci < n_chunks; ci++) {
        int start = ci * chunk;
        int end = start + chunk;
        if (end > rows) {
            end = rows;
        }
        for (int r = start; r < end; r++) {
            const uint8_t* row = codes + (size_t)r * (size_t)stride;
            int32_t raw = use_avx2 ? orc_code_row_dot_avx2(row, acts, stride)
                                   : orc_code_row_dot_go(row, acts, stride);
            int32_t acc = raw - act_sum;
            if (acc_out) {
                acc_out[r] = acc;
            }
            out[r] = (double)acc * output_scale;
        }
    }
    free(acts);
}

/* ------------------------------------------------------------------ */
/* Layer forwards                                                      */
/* ------------------------------------------------------------------ */

/* Activate for T=float32 (poly/poly.go:167-200). */
float orc_activate_f32(float v, int activation) {
    switch (activation) {
        case ORC_ACT_RELU:
            return v < 0.0f ? 0.0f : v;
        case ORC_ACT_SILU:
            return v * (float)(1.0 / (1.0 + exp(-(double)v)));
        case ORC_ACT_GELU: {
            double v64 = (double)v;
            return (float)(0.5 * v64 *
                           (1.0 + tanh(sqrt(2.0 / M_PI) * (v64 + 0.044715 * pow(v64, 3)))));
        }
        case ORC_ACT_TANH:
            return (float)tanh((double)v);
        case ORC_ACT_SIGMOID:
            return (float)(1.0 / (1.0 + exp(-(double)v)));
        case ORC_ACT_LEAKY_RELU:
            return v < 0.0f ? (float)((double)v * 0.01) : v;
        case ORC_ACT_RELU2:
            return v < 0.0f ? 0.0f : v * v;
        default:
            return v;
    }
}

static void matvec_quantized(const orc_matrix* w, const int8_t* xq, float amax, int simd,
                             int workers, double* out, int32_t* acc_out) {
    double os = orc_output_scale(w->scale, amax);
    if (simd && w->codes) {
        orc_matvec_simd(w->codes, w->rows, w->cols, xq, os, out, acc_out, workers);
    } else {
        orc_matvec_scalar(w->words, w->rows, w->cols, w->row_words, xq, os, out, acc_out);
    }
}

/* DenseForwardPackedTernaryCPU (poly/dense.go:66-101): rows of the batch are
 * processed one by one: quantize, ternary matvec, fp64 -> fp32, Activate. */
void orc_dense_forward(const orc_matrix* w, const float* in, int m, int activation,
                       int simd, int workers, float* pre, float* post,
                       int8_t* xq_out, float* amax_out, int32_t* acc_out) {
    int k = w->cols;
    int n = w->rows;
    double* tmp = (double*)malloc((size_t)n * sizeof(double));
    int8_t* xq = (int8_t*)malloc((size_t)k);
    for (int b = 0; b < m; b++) {
        const float* row = in + (size_t)b * (size_t)k;
        float amax = orc_quant_act_f32(row, k, xq);
        matvec_quantized(w, xq, amax, simd, workers, tmp,
                         acc_out ? acc_out + (size_t)b * (size_t)n : NULL);
        if (xq_out) {
            memcpy(xq_out + (size_t)b * (size_t)k, xq, (size_t)k);
        }
        if (amax_out) {
            amax_out[b] = amax;
        }
        for (int o = 0; o < n; o++) {
            float v = (float)tmp[o];
            if (pre) {
                pre[(size_t)b * (size_t)n + o] = v;
            }
            if (post) {
                post[(size_t)b * (size_t)n + o] = orc_activate_f32(v, activation);
            }
        }
    }
    free(xq);
    free(tmp);
}

/* swigluGateProduct (poly/swiglu.go:37-46): ReLU^2 gate when activation is
 * ReLU2 (6), SiLU otherwise: (g*sigma(g))*u with sigma = 1/(1+exp(-g)). */
double orc_swiglu_gate_product(double g, double u, int activation) {
    if (activation == ORC_ACT_RELU2) {
        if (g < 0.0) {
            g = 0.0;
        }
        return (g * g) * u;
    }
    double sig = 1.0 / (1.0 + exp(-g));
    return (g * sig) * u;
}

/* bitNetRMSNormTensorRowWeighted for T=float32 (poly/bitnet_cpu.go:893-913):
 * scale = 1/sqrt(sum(f*f)/n + eps) with a sequential fp64 sum,
 * data[i] = fp32((float64(v)*scale)*w), w = 1 past the weight slice. */
void orc_bitnet_rmsnorm_row_f32(float* data, int n, const float* weight, double eps) {
    if (n == 0) {
        return;
    }
    if (eps <= 0.0) {
        eps = 1e-5;
    }
    double sum_sq = 0.0;
    for (int i = 0; i < n; i++) {
        double f = (double)data[i];
        sum_sq += f * f;
    }
    double scale = 1.0 / sqrt(sum_sq / (double)n + eps);
    for (int i = 0; i < n; i++) {
        double w = weight ? (double)weight[i] : 1.0;
        data[i] = (float)((double)data[i] * scale * w);
    }
}

/* bitNetRMSNormFloat64Weighted (poly/bitnet_cpu.go:868-887): data[i] *= scale*w
 * (note: scale*w is formed first, unlike the fp32-row helper above). */
void orc_bitnet_rmsnorm_f64(double* data, int n, const float* weight, double eps) {
    if (n == 0) {
        return;
    }
    if (eps <= 0.0) {
        eps = 1e-5;
    }
    double sum_sq = 0.0;
    for (int i = 0; i < n; i++) {
        sum_sq += data[i] * data[i];
    }
    double scale = 1.0 / sqrt(sum_sq / (double)n + eps);
    for (int i = 0; i < n; i++) {
        double w = weight ? (double)weight[i] : 1.0;
        data[i] *= scale * w;
    }
}

/* Stage of the MHA output projection (poly/mha.go:362-368) and the SwiGLU
 * down projection (poly/swiglu.go:316-320) from given int8 rows: per row s,
 * out = fp32(bitNetTernaryMatVecQuantized(xq[s], amax[s]) + bias), the bias
 * (0 when NULL) added in fp64 as both sites add it. */
void orc_dense_quantized(const orc_matrix* w, const int8_t* xq, const float* amax, int m,
                         const float* bias, int simd, int workers, float* out) {
    double* t = (double*)malloc((size_t)w->rows * sizeof(double));
    for (int s = 0; s < m; s++) {
        matvec_quantized(w, xq + (size_t)s * w->cols, amax[s], simd, workers, t, NULL);
        for (int i = 0; i < w->rows; i++) {
            out[(size_t)s * w->rows + i] = (float)(t[i] + (bias ? (double)bias[i] : 0.0));
        }
    }
    free(t);
}

/* Gate/up stage of SwiGLUForwardPackedTernaryCPU (poly/swiglu.go:303-312)
 * from given int8 rows: h = fp32(swigluGateProduct(g + bias_g, u + bias_u)),
 * bias = [gate inter | up inter] or NULL. */
void orc_swiglu_gate_rows(const orc_matrix* gate, const orc_matrix* up, const float* bias,
                          int activation, const int8_t* xq, const float* amax, int m, int simd,
                          int workers, float* h) {
    const int inter = gate->rows;
    double* g = (double*)malloc((size_t)inter * sizeof(double));
    double* u = (double*)malloc((size_t)inter * sizeof(double));
    for (int s = 0; s < m; s++) {
        const int8_t* row = xq + (size_t)s * gate->cols;
        matvec_quantized(gate, row, amax[s], simd, workers, g, NULL);
        matvec_quantized(up, row, amax[s], simd, workers, u, NULL);
        for (int o = 0; o < inter; o++) {
            double gv = g[o] + (bias ? (double)bias[o] : 0.0);
            double uv = u[o] + (bias ? (double)bias[inter + o] : 0.0);
            h[(size_t)s * inter + o] = (float)orc_swiglu_gate_product(gv, uv, activation);
        }
    }
    free(u);
    free(g);
}

/* SwiGLUForwardPackedTernaryCPU (poly/swiglu.go:270-322). */
void orc_swiglu_forward(const orc_matrix* gate, const orc_matrix* up,
                        const orc_matrix* down, const float* bias,
                        const float* inner_norm, double eps, int activation,
                        const float* in, int m, int simd, int workers,
                        float* out, float* h_out,
                        int8_t* xq_out, float* amax_out,
                        int8_t* hq_out, float* hamax_out,
                        int32_t* acc_gate, int32_t* acc_up, int32_t* acc_down) {
    int hidden = gate->cols;
    int inter = gate->rows;
    double* g = (double*)malloc((size_t)inter * sizeof(double));
    double* u = (double*)malloc((size_t)inter * sizeof(double));
    double* d = (double*)malloc((size_t)hidden * sizeof(double));
    int8_t* xq = (int8_t*)malloc((size_t)hidden);
    int8_t* hq = (int8_t*)malloc((size_t)inter);
    float* h = (float*)malloc((size_t)inter * sizeof(float));
    const float* bias_g = bias ? bias : NULL;
    const float* bias_u = bias ? bias + inter : NULL;
    const float* bias_d = bias ? bias + 2 * inter : NULL;
    for (int s = 0; s < m; s++) {
        const float* row = in + (size_t)s * (size_t)hidden;
        float amax = orc_quant_act_f32(row, hidden, xq);
        matvec_quantized(gate, xq, amax, simd, workers, g,
                         acc_gate ? acc_gate + (size_t)s * (size_t)inter : NULL);
        matvec_quantized(up, xq, amax, simd, workers, u,
                         acc_up ? acc_up + (size_t)s * (size_t)inter : NULL);
        if (xq_out) {
            memcpy(xq_out + (size_t)s * (size_t)hidden, xq, (size_t)hidden);
        }
        if (amax_out) {
            amax_out[s] = amax;
        }
        for (int o = 0; o < inter; o++) {
            double gv = g[o] + (bias_g ? (double)bias_g[o] : 0.0);
            double uv = u[o] + (bias_u ? (double)bias_u[o] : 0.0);
            h[o] = (float)orc_swiglu_gate_product(gv, uv, activation);
        }
        orc_bitnet_rmsnorm_row_f32(h, inter, inner_norm, eps);
        if (h_out) {
            memcpy(h_out + (size_t)s * (size_t)inter, h, (size_t)inter * sizeof(float));
        }
        float hamax = orc_quant_act_f32(h, inter, hq);
        if (hq_out) {
            memcpy(hq_out + (size_t)s * (size_t)inter, hq, (size_t)inter);
        }
        if (hamax_out) {
            hamax_out[s] = hamax;
        }
        matvec_quantized(down, hq, hamax, simd, workers, d,
                         acc_down ? acc_down + (size_t)s * (size_t)hidden : NULL);
        for (int i = 0; i < hidden; i++) {
            out[(size_t)s * (size_t)hidden + i] =
                (float)(d[i] + (bias_d ? (double)bias_d[i] : 0.0));
        }
    }
    free(h);
    free(hq);
    free(xq);
    free(d);
    free(u);
    free(g);
}

/* RMSNormForwardPolymorphic (poly/norm.go:102-138). */
void orc_rmsnorm_forward(const float* x, int rows, int n, const float* gain,
                         double eps, float* y, float* rms_out) {
    if (eps <= 0.0) {
        eps = 1e-6;
    }
    for (int b = 0; b < rows; b++) {
        const float* row = x + (size_t)b * (size_t)n;
        double sum_sq = 0.0;
        for (int i = 0; i < n; i++) {
            double v = (double)row[i];
            sum_sq += v * v;
        }
        double rms = sqrt(sum_sq / (double)n + eps);
        if (rms_out) {
            rms_out[b] = (float)rms;
        }
        for (int i = 0; i < n; i++) {
            double normed = (double)row[i] / rms;
            y[(size_t)b * (size_t)n + i] = (float)(normed * (double)gain[i]);
        }
    }
}

/* ------------------------------------------------------------------ */
/* .entity BITNET_TERNARY blob                                         */
/* ------------------------------------------------------------------ */

static void put_u32(uint8_t* p, uint32_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
    p[2] = (uint8_t)(v >> 16);
    p[3] = (uint8_t)(v >> 24);
}

static uint32_t get_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}

size_t orc_entity_blob_bytes(int n_words) {
    return 24 + (size_t)n_words * 4;
}

/* encodeEntityBitNetTernaryBlob (poly/entity_bitnet.go:38-55): LE header
 * [rows][cols][offset][scale bits][rowWords][nWords] then the words. */
size_t orc_entity_encode(int rows, int cols, int offset, float scale, int row_words,
                         const uint32_t* words, int n_words, uint8_t* raw) {
    uint32_t sbits;
    memcpy(&sbits, &scale, 4);
    put_u32(raw + 0, (uint32_t)rows);
    put_u32(raw + 4, (uint32_t)cols);
    put_u32(raw + 8, (uint32_t)offset);
    put_u32(raw + 12, sbits);
    put_u32(raw + 16, (uint32_t)row_words);
    put_u32(raw + 20, (uint32_t)n_words);
    for (int i = 0; i < n_words; i++) {
        put_u32(raw + 24 + 4 * (size_t)i, words[i]);
    }
    return orc_entity_blob_bytes(n_words);
}

/* decodeEntityBitNetTernaryBlob header (poly/entity_bitnet.go:57-88);
 * rowWords <= 0 defaults to ceil(cols/16). */
int orc_entity_decode_header(const uint8_t* raw, size_t len, int* rows, int* cols,
                             int* offset, float* scale, int* row_words, int* n_words) {
    if (len < 24) {
        return -1;
    }
    *rows = (int)get_u32(raw + 0);
    *cols = (int)get_u32(raw + 4);
    *offset = (int)get_u32(raw + 8);
    uint32_t sbits = get_u32(raw + 12);
    memcpy(scale, &sbits, 4);
    *row_words = (int)get_u32(raw + 16);
    *n_words = (int)get_u32(raw + 20);
    if (len < 24 + (size_t)(uint32_t)*n_words * 4) {
        return -2;
    }
    if (*row_words <= 0) {
        *row_words = (*cols + 15) / 16;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Deterministic inputs                                                */
/* ------------------------------------------------------------------ */

/* deterministicWeights (poly/tests/bitnet_cpu_test.go:10-20). */
void orc_deterministic_weights(float* out, int n) {
    for (int i = 0; i < n; i++) {
        float v = (float)((i % 11) - 5) * 0.13f;
        if (i % 7 == 0) {
            v *= -0.5f;
        }
        out[i] = v;
    }
}

/* SplitMix64 (Steele, Lea, Flood 2014). */
uint64_t orc_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double unit_open(uint64_t* st) {
    /* (0, 1]: 53 random bits, never zero so log() is finite. */
    return ((double)(orc_splitmix64(st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

/* x ~ N(0,1) by fp64 Box-Muller, rounded to fp32. */
void orc_fill_normal_f32(float* out, long n, uint64_t seed) {
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (long i = 0; i < n; i += 2) {
        double u1 = unit_open(&st);
        double u2 = unit_open(&st);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2));
        if (i + 1 < n) {
            out[i + 1] = (float)(r * sin(two_pi * u2));
        }
    }
}

/* Ternary storage values (uint8(int8) of {-1,0,1}), 2 bits per draw:
 * 00,01 -> 0 (P=.5), 10 -> +1, 11 -> -1 (P=.25 each). */
void orc_fill_ternary_codes(uint8_t* native, long n, uint64_t seed) {
    uint64_t st = seed;
    uint64_t bits = 0;
    int left = 0;
    for (long i = 0; i < n; i++) {
        if (left == 0) {
            bits = orc_splitmix64(&st);
            left = 32;
        }
        unsigned t = (unsigned)(bits & 3u);
        bits >>= 2;
        left--;
        native[i] = t < 2 ? 0 : (t == 2 ? 1 : (uint8_t)0xFF);
    }
}

void orc_fill_uniform_f32(float* out, long n, float lo, float hi, uint64_t seed) {
    uint64_t st = seed;
    for (long i = 0; i < n; i++) {
        double u = (double)(orc_splitmix64(&st) >> 11) * (1.0 / 9007199254740992.0);
        out[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
    }
}

/* ------------------------------------------------------------------ */
/* Attention, decoder block, LM head                                   */
/* ------------------------------------------------------------------ */

/* bitNetRMSNormFloat64Weighted + bitNetQuantizeActivationFloat64 are above. */

/* Attention of MHAForwardPackedTernaryCPU (poly/mha.go:316-354) for `seq`
 * queries at positions seq_base + s over the ring caches (row kp % msl):
 * fp64 dot over d in order times 1/sqrt(hd), running max from -1e9,
 * exp(score - max), expSum in position order, out[d] = sum in position order
 * of p*V / expSum.  GQA group of head h: h / (heads / kv_heads). */
void orc_attention(const double* Q, const float* cache_k, const float* cache_v, int seq,
                   int seq_base, int msl, int heads, int kv_heads, int hd, double* attn) {
    const int q_dim = heads * hd, kv_dim = kv_heads * hd;
    const int per_kv = heads / kv_heads;
    const double scale = 1.0 / sqrt((double)hd);
    /* (query, head) pairs are independent: threads split the pairs, and each
     * pair runs the reference's loops unchanged, so the results do not depend
     * on the thread count */
#pragma omp parallel
    {
        double* scores = (double*)malloc((size_t)(seq_base + seq) * sizeof(double));
#pragma omp for schedule(dynamic, 1)
        for (long sh = 0; sh < (long)seq * heads; sh++) {
            const int s = (int)(sh / heads), h = (int)(sh % heads);
            const int total = seq_base + s;
            const int kvh = h / per_kv;
            double max_score = -1e9;
            for (int kp = 0; kp <= total; kp++) {
                const float* kr = cache_k + (size_t)(kp % msl) * kv_dim + (size_t)kvh * hd;
                const double* qr = Q + (size_t)s * q_dim + (size_t)h * hd;
                double dot = 0.0;
                for (int d = 0; d < hd; d++) dot += qr[d] * (double)kr[d];
                double score = dot * scale;
                scores[kp] = score;
                if (score > max_score) max_score = score;
            }
            double exp_sum = 0.0;
            for (int kp = 0; kp <= total; kp++) {
                scores[kp] = exp(scores[kp] - max_score);
                exp_sum += scores[kp];
            }
            for (int d = 0; d < hd; d++) {
                double sum = 0.0;
                for (int kp = 0; kp <= total; kp++) {
                    sum += scores[kp] * (double)cache_v[(size_t)(kp % msl) * kv_dim + (size_t)kvh * hd + d];
                }
                attn[(size_t)s * q_dim + (size_t)h * hd + d] = sum / exp_sum;
            }
        }
        free(scores);
    }
}

/* The attention of MHAForwardPackedTernaryCPU (poly/mha.go:316-354) in two
 * stages on either side of math.Exp, so that a device's chains can be
 * checked bit for bit given the device's own exp.  Only the listed rows
 * rows[0..nrows) of Q are evaluated (row s sits at position seq_base + s).
 * Layout of args / probs: for each listed row i, for each head h, the
 * positions 0..seq_base+rows[i]; orc_attention_span gives the length.
 *
 * Stage 1 (poly/mha.go:324-337): every score is the dimension-order chain
 * dot += Q*K, then dot*scale; the maximum runs from -1e9 over positions in
 * order; args = score - max.
 * Stage 2 (poly/mha.go:339-352): p = probs (the caller's exp of args);
 * expSum += p in position order; each column's sum += p*V in position
 * order; out = sum / expSum. */
long orc_attention_span(const int* rows, int nrows, int seq_base, int heads) {
    long n = 0;
    for (int i = 0; i < nrows; i++) n += (long)heads * (seq_base + rows[i] + 1);
    return n;
}

static long attn_span_offset(const int* rows, int i, int seq_base, int heads) {
    return orc_attention_span(rows, i, seq_base, heads);
}

void orc_attention_args(const double* Q, const float* cache_k, const int* rows, int nrows,
                        int seq_base, int msl, int heads, int kv_heads, int hd, double* args) {
    const int q_dim = heads * hd, kv_dim = kv_heads * hd;
    const int per_kv = heads / kv_heads;
    const double scale = 1.0 / sqrt((double)hd);
#pragma omp parallel for schedule(dynamic, 1)
    for (long ih = 0; ih < (long)nrows * heads; ih++) {
        const int i = (int)(ih / heads), h = (int)(ih % heads);
        const int s = rows[i], total = seq_base + s;
        const int kvh = h / per_kv;
        double* a = args + attn_span_offset(rows, i, seq_base, heads) + (long)h * (total + 1);
        const double* qr = Q + (size_t)s * q_dim + (size_t)h * hd;
        double max_score = -1e9;
        for (int kp = 0; kp <= total; kp++) {
            const float* kr = cache_k + (size_t)(kp % msl) * kv_dim + (size_t)kvh * hd;
            double dot = 0.0;
            for (int d = 0; d < hd; d++) dot += qr[d] * (double)kr[d];
            const double score = dot * scale;
            a[kp] = score;
            if (score > max_score) max_score = score;
        }
        for (int kp = 0; kp <= total; kp++) a[kp] = a[kp] - max_score;
    }
}

void orc_attention_chains(const double* probs, const float* cache_v, const int* rows, int nrows,
                          int seq_base, int msl, int heads, int kv_heads, int hd, double* attn) {
    const int q_dim = heads * hd, kv_dim = kv_heads * hd;
    const int per_kv = heads / kv_heads;
#pragma omp parallel for schedule(dynamic, 1)
    for (long ih = 0; ih < (long)nrows * heads; ih++) {
        const int i = (int)(ih / heads), h = (int)(ih % heads);
        const int total = seq_base + rows[i];
        const int kvh = h / per_kv;
        const double* p = probs + attn_span_offset(rows, i, seq_base, heads) + (long)h * (total + 1);
        double exp_sum = 0.0;
        for (int kp = 0; kp <= total; kp++) exp_sum += p[kp];
        for (int d = 0; d < hd; d++) {
            double sum = 0.0;
            for (int kp = 0; kp <= total; kp++) {
                sum += p[kp] * (double)cache_v[(size_t)(kp % msl) * kv_dim + (size_t)kvh * hd + d];
            }
            attn[(size_t)i * q_dim + (size_t)h * hd + d] = sum / exp_sum;
        }
    }
}

/* The host C library's exp, elementwise (the exp that orc_attention calls). */
void orc_exp_rows(const double* x, long n, double* y) {
    for (long i = 0; i < n; i++) y[i] = exp(x[i]);
}

/* Output stage of MHAForwardPackedTernaryCPU (poly/mha.go:356-368): per row,
 * bitNetRMSNormFloat64Weighted in place, fp64 requantization, O matvec,
 * pre = fp32(normalized row), post = fp32(O + bias).  attn is modified. */
void orc_attn_out(const orc_matrix* o, const float* bias_o, const float* inner_norm, double eps,
                  double* attn, int seq, int q_dim, int simd, int workers, float* pre,
                  float* post) {
    const int d_model = o->rows;
    double* to = (double*)malloc((size_t)d_model * sizeof(double));
    int8_t* aq = (int8_t*)malloc((size_t)q_dim);
    for (int s = 0; s < seq; s++) {
        double* ar = attn + (size_t)s * q_dim;
        orc_bitnet_rmsnorm_f64(ar, q_dim, inner_norm, eps);
        float amax = orc_quant_act_f64(ar, q_dim, aq);
        matvec_quantized(o, aq, amax, simd, workers, to, NULL);
        for (int i = 0; i < d_model; i++) {
            if (pre) pre[(size_t)s * d_model + i] = (float)ar[i];
            post[(size_t)s * d_model + i] = (float)(to[i] + (bias_o ? (double)bias_o[i] : 0.0));
        }
    }
    free(aq);
    free(to);
}

/* mhaQKNormEpsilon (poly/mha.go:19-24): the layer's RMSNormEps when set,
 * else 1e-6 (the inner norm's own default is 1e-5, poly/bitnet_cpu.go:868-874). */
double orc_qk_norm_eps(double layer_eps) {
    return layer_eps > 0 ? layer_eps : 1e-6;
}

/* The gamma element of dimension d of head h: gamma[d] when the weights hold
 * one head, gamma[h*hd + d] when they hold every head, else 1 (both
 * applyPerHeadRMSNorm variants, poly/mha.go:605-611, 634-640). */
static double per_head_gamma(const float* gamma, int gamma_len, int heads, int hd, int h, int d) {
    if (gamma_len == hd) return (double)gamma[d];
    if (gamma_len == heads * hd) return (double)gamma[(size_t)h * hd + d];
    return 1.0;
}

/* applyPerHeadRMSNormFloat64 (poly/mha.go:584-614): per head, the sequential
 * fp64 sum of squares, rms = sqrt(sumSq/hd + eps) (eps <= 0 -> 1e-6), a head
 * with rms == 0 left unchanged, then x = x * (1/rms) * gamma, left to right. */
void orc_per_head_rmsnorm_f64(double* data, const float* gamma, int gamma_len, int heads,
                              int hd, double eps) {
    if (heads <= 0 || hd <= 0) return;
    if (eps <= 0) eps = 1e-6;
    for (int h = 0; h < heads; h++) {
        double* x = data + (size_t)h * hd;
        double sum_sq = 0.0;
        for (int i = 0; i < hd; i++) sum_sq += x[i] * x[i];
        const double rms = sqrt(sum_sq / (double)hd + eps);
        if (rms == 0) continue;
        const double inv = 1.0 / rms;
        for (int d = 0; d < hd; d++) {
            x[d] = x[d] * inv * per_head_gamma(gamma, gamma_len, heads, hd, h, d);
        }
    }
}

/* applyPerHeadRMSNormTensor for T = float32 (poly/mha.go:616-646): the same
 * on fp32 values widened to fp64, each result rounded back to fp32. */
void orc_per_head_rmsnorm_f32(float* data, const float* gamma, int gamma_len, int heads, int hd,
                              double eps) {
    if (heads <= 0 || hd <= 0) return;
    if (eps <= 0) eps = 1e-6;
    for (int h = 0; h < heads; h++) {
        float* x = data + (size_t)h * hd;
        double sum_sq = 0.0;
        for (int i = 0; i < hd; i++) {
            const double v = (double)x[i];
            sum_sq += v * v;
        }
        const double rms = sqrt(sum_sq / (double)hd + eps);
        if (rms == 0) continue;
        const double inv = 1.0 / rms;
        for (int d = 0; d < hd; d++) {
            x[d] = (float)((double)x[d] * inv * per_head_gamma(gamma, gamma_len, heads, hd, h, d));
        }
    }
}

/* MHAForwardPackedTernaryCPU (poly/mha.go:204-371) for one batch row of
 * `seq` tokens, with the optional per-head Q/K norms of poly/mha.go:285-290.
 * The KV cache is a ring of msl rows (pos % msl), prepared as
 * mhaPrepareKVForForward does (poly/mha_layout.go:62-70): a pass that is not
 * a warm single-token step resets kv_offset to 0. */
void orc_mha_project(orc_mha* L, const float* in, int seq, int seq_base, int simd, int workers,
                     double* Q) {
    const int d_model = L->d_model;
    const int heads = L->num_heads;
    const int kv_heads = L->num_kv_heads > 0 ? L->num_kv_heads : heads;
    const int hd = L->head_dim;
    const int q_dim = heads * hd;
    const int kv_dim = kv_heads * hd;
    const int msl = L->msl > 0 ? L->msl : 512;
    double* tq = (double*)malloc((size_t)q_dim * sizeof(double));
    double* tk = (double*)malloc((size_t)kv_dim * sizeof(double));
    double* tv = (double*)malloc((size_t)kv_dim * sizeof(double));
    int8_t* xq = (int8_t*)malloc((size_t)d_model);
    const double theta = L->theta > 0 ? L->theta : 10000.0;
    const int half = hd / 2;
    for (int s = 0; s < seq; s++) {
        const int pos = seq_base + s;
        const float* row = in + (size_t)s * d_model;
        float* krow = L->cache_k + (size_t)(pos % msl) * kv_dim;
        float* vrow = L->cache_v + (size_t)(pos % msl) * kv_dim;
        float amax = orc_quant_act_f32(row, d_model, xq);
        matvec_quantized(L->q, xq, amax, simd, workers, tq, NULL);
        for (int i = 0; i < q_dim; i++) {
            Q[(size_t)s * q_dim + i] = tq[i] + (L->bias_q ? (double)L->bias_q[i] : 0.0);
        }
        matvec_quantized(L->k, xq, amax, simd, workers, tk, NULL);
        matvec_quantized(L->v, xq, amax, simd, workers, tv, NULL);
        for (int i = 0; i < kv_dim; i++) {
            krow[i] = (float)(tk[i] + (L->bias_k ? (double)L->bias_k[i] : 0.0));
            vrow[i] = (float)(tv[i] + (L->bias_v ? (double)L->bias_v[i] : 0.0));
        }
        if (L->q_norm_len > 0) {
            orc_per_head_rmsnorm_f64(Q + (size_t)s * q_dim, L->q_norm, L->q_norm_len, heads, hd,
                                     orc_qk_norm_eps(L->eps));
        }
        if (L->k_norm_len > 0) {
            orc_per_head_rmsnorm_f32(krow, L->k_norm, L->k_norm_len, kv_heads, hd,
                                     orc_qk_norm_eps(L->eps));
        }
        for (int h = 0; h < heads; h++) {
            for (int d = 0; d < half; d++) {
                double angle = (double)pos / pow(theta, (double)(2 * d) / (double)hd);
                double c = cos(angle), sv = sin(angle);
                size_t off = (size_t)s * q_dim + (size_t)h * hd + d;
                double v0 = Q[off], v1 = Q[off + half];
                Q[off] = v0 * c - v1 * sv;
                Q[off + half] = v0 * sv + v1 * c;
            }
        }
        for (int h = 0; h < kv_heads; h++) {
            for (int d = 0; d < half; d++) {
                double angle = (double)pos / pow(theta, (double)(2 * d) / (double)hd);
                double c = cos(angle), sv = sin(angle);
                int off = h * hd + d;
                double v0 = (double)krow[off], v1 = (double)krow[off + half];
                krow[off] = (float)(v0 * c - v1 * sv);
                krow[off + half] = (float)(v0 * sv + v1 * c);
            }
        }
    }
    free(xq);
    free(tv);
    free(tk);
    free(tq);
}

void orc_mha_forward(orc_mha* L, const float* in, int seq, int simd, int workers,
                     float* pre, float* post, double* q_out, double* attn_out) {
    const int heads = L->num_heads;
    const int kv_heads = L->num_kv_heads > 0 ? L->num_kv_heads : heads;
    const int hd = L->head_dim;
    const int q_dim = heads * hd;
    const int kv_dim = kv_heads * hd;
    const int msl = L->msl > 0 ? L->msl : 512;
    const int incremental = (seq == 1 && L->kv_offset > 0);
    if (!incremental) {
        memset(L->cache_k, 0, (size_t)msl * kv_dim * sizeof(float));
        memset(L->cache_v, 0, (size_t)msl * kv_dim * sizeof(float));
        L->kv_offset = 0;
    }
    const int seq_base = L->kv_offset;
    double* Q = (double*)malloc((size_t)seq * q_dim * sizeof(double));
    orc_mha_project(L, in, seq, seq_base, simd, workers, Q);
    if (q_out) memcpy(q_out, Q, (size_t)seq * q_dim * sizeof(double));
    double* attn = (double*)malloc((size_t)seq * q_dim * sizeof(double));
    orc_attention(Q, L->cache_k, L->cache_v, seq, seq_base, msl, heads, kv_heads, hd, attn);
    if (attn_out) memcpy(attn_out, attn, (size_t)seq * q_dim * sizeof(double));
    orc_attn_out(L->o, L->bias_o, L->inner_norm, L->eps, attn, seq, q_dim, simd, workers, pre,
                 post);
    L->kv_offset = seq_base + seq;
    free(attn);
    free(Q);
}

/* One decoder block (poly/transformer_forward.go:228-245) on seq rows of x,
 * in place: x += MHA(RMSNorm1(x)); x += SwiGLU(RMSNorm2(x)).  Tensor.Add is an
 * fp32 add (poly/poly.go:481-494). */
void orc_block_forward(orc_block* B, float* x, int seq, int simd, int workers) {
    const int n = B->hidden;
    const size_t cnt = (size_t)seq * n;
    float* y = (float*)malloc(cnt * sizeof(float));
    float* o = (float*)malloc(cnt * sizeof(float));
    orc_rmsnorm_forward(x, seq, n, B->norm1, B->norm_eps, y, NULL);
    orc_mha_forward(&B->mha, y, seq, simd, workers, NULL, o, NULL, NULL);
    for (size_t i = 0; i < cnt; i++) x[i] = o[i] + x[i];
    orc_rmsnorm_forward(x, seq, n, B->norm2, B->norm_eps, y, NULL);
    const int inter = B->gate->rows;
    float* h = (float*)malloc((size_t)seq * inter * sizeof(float));
    orc_swiglu_forward(B->gate, B->up, B->down, NULL, B->ffn_inner_norm, B->ffn_eps,
                       B->ffn_activation, y, seq, simd, workers, o, h, NULL, NULL, NULL, NULL,
                       NULL, NULL, NULL);
    for (size_t i = 0; i < cnt; i++) x[i] = o[i] + x[i];
    free(h);
    free(o);
    free(y);
}

/* applyFP32LMHeadRows, SIMD off (poly/transformer.go:683-689): sequential fp64. */
void orc_lm_head_seq(const float* hidden, const float* lm, int vocab, int h, float* logits) {
#pragma omp parallel for schedule(static)
    for (int v = 0; v < vocab; v++) {
        const float* w = lm + (size_t)v * h;
        double sum = 0.0;
        for (int d = 0; d < h; d++) sum += (double)hidden[d] * (double)w[d];
        logits[v] = (float)sum;
    }
}

/* DotTile with SIMD on amd64 (poly/simd/avx2_amd64.s:14-79): eight strided
 * fp64 partials p_l = sum over 8-element chunks of x[8c+l]*w[8c+l] (the
 * products are exact in fp64, so the FMAs equal multiply-then-add), reduced
 * as ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)), plus prev, then the n%8 tail
 * added in order. */
double orc_dot_tile(const float* x, const float* w, int n, double prev) {
    double p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        for (int l = 0; l < 8; l++) p[l] += (double)x[i + l] * (double)w[i + l];
    }
    double x0 = p[0] + p[4], x1 = p[1] + p[5];
    double x2 = p[2] + p[6], x3 = p[3] + p[7];
    double t0 = x0 + x2, t1 = x1 + x3;
    double r = (t0 + t1) + prev;
    for (; i < n; i++) r += (double)x[i] * (double)w[i];
    return r;
}

/* applyFP32LMHeadRows with UseSimdForward (poly/transformer.go:679-681). */
void orc_lm_head_dottile(const float* hidden, const float* lm, int vocab, int h, float* logits) {
#pragma omp parallel for schedule(static)
    for (int v = 0; v < vocab; v++) {
        logits[v] = (float)orc_dot_tile(hidden, lm + (size_t)v * h, h, 0.0);
    }
}

/* SampleTopK greedy branch (poly/sampling.go:44-55): first strict maximum. */
int orc_argmax_first(const float* logits, int n) {
    int idx = 0;
    float best = logits[0];
    for (int i = 0; i < n; i++) {
        if (logits[i] > best) {
            best = logits[i];
            idx = i;
        }
    }
    return idx;
}
