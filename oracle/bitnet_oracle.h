/*
 * bitnet_oracle.h -- CPU restatement of loom's BitNet b1.58 CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the
 * timed CPU baseline ("port" of loom's bitnet_simd path).  It is loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, and by
 * nothing else: libloom_accel_amd.so never links or calls it.
 *
 * Every function cites the reference file:line it restates
 * (paths relative to the loom v0.83.0 tree).
 *
 * Parity pinning (what checks each function, see tests/test_oracle_*.py):
 *   orc_act_maxabs_*, orc_quant_act_*   pinned: KAT tail 3x17 brute force,
 *                                       closed-form edge cases (zero row,
 *                                       1e-5 floor, +-amax -> +-127, NaN).
 *   orc_ternary_scale, orc_quant_value,
 *   orc_pack_float32                    pinned: absmean KAT {-0.2,-0.8,0.1,0.8}
 *                                       -> 0.475 / {0,-1,0,1}; alreadyTernary
 *                                       quirk (native unit scale).
 *   orc_pack_ms_offline_*               pinned: 8x2 microsoft offline KAT,
 *                                       bytes vs float-slot equality.
 *   orc_matvec_scalar / orc_matvec_simd pinned: 8x2 KAT, tail brute force,
 *                                       SIMD == scalar bit-identical sweep.
 *   orc_dense_forward                   pinned: packed vs dequantized fp32
 *                                       dense within 5e-3 (reference test).
 *   orc_entity_encode / decode          pinned: blob round trip KAT.
 *   orc_swiglu_forward                  partially pinned: integer stages by the
 *                                       matvec pins; the fp64 exp() in the
 *                                       gate is glibc exp, not Go math.Exp
 *                                       (parity unpinned at the last ulp).
 *   orc_rmsnorm_forward                 pinned by closed forms (constant row,
 *                                       unit weights) -- IEEE basic ops only.
 */
#ifndef LOOM_BITNET_ORACLE_H
#define LOOM_BITNET_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* loom ActivationType values (poly/poly.go:89-98). */
enum {
    ORC_ACT_RELU = 0,
    ORC_ACT_SILU = 1,
    ORC_ACT_GELU = 2,
    ORC_ACT_TANH = 3,
    ORC_ACT_SIGMOID = 4,
    ORC_ACT_LEAKY_RELU = 5,
    ORC_ACT_RELU2 = 6,
    ORC_ACT_LINEAR = -1
};

/* ---- activation quantization (poly/bitnet_cpu.go:45-117) ---- */
float orc_act_maxabs_f32(const float* x, int n);
float orc_act_maxabs_f64(const double* x, int n);
int8_t orc_quant_value_act(double v, float amax);
float orc_quant_act_f32(const float* x, int n, int8_t* q);
float orc_quant_act_f64(const double* x, int n, int8_t* q);

/* ---- weight quantization + packing (poly/bitnet_cpu.go:119-146,498-512,918-977) ---- */
float orc_ternary_scale(const float* w, long n);
uint8_t orc_quant_value(float v, float scale);
uint8_t orc_storage_to_code(uint8_t v);
void orc_pack_ternary_rows(const uint8_t* native, int rows, int cols, uint32_t* words);
float orc_pack_float32(const float* w, int rows, int cols, uint32_t* words);
void orc_pack_ms_offline_bytes(const uint8_t* packed, int rows, int cols, uint32_t* words);
void orc_pack_ms_offline_float_slots(const float* packed, int rows, int cols, uint32_t* words);

/* ---- matvec kernels (poly/bitnet_cpu.go:536-566,700-854; poly/simd/bitnet_ternary*.go/.s) ---- */
double orc_output_scale(float weight_scale, float amax);
int32_t orc_word_dot16(uint32_t word, const int8_t* xq);
int32_t orc_word_dot_tail(uint32_t word, const int8_t* xq, int n);
void orc_matvec_scalar(const uint32_t* words, int rows, int cols, int row_words,
                       const int8_t* xq, double output_scale, double* out,
                       int32_t* acc_out);
int orc_codes_stride(int cols);
void orc_ensure_codes(const uint32_t* words, int rows, int cols, int row_words,
                      uint8_t* codes);
int32_t orc_code_row_dot_go(const uint8_t* codes, const int8_t* acts, int n_bytes);
int32_t orc_code_row_dot_avx2(const uint8_t* codes, const int8_t* acts, int n_bytes);
int orc_simd_available(void);
void orc_matvec_simd(const uint8_t* codes, int rows, int cols, const int8_t* xq,
                     double output_scale, double* out, int32_t* acc_out,
                     int workers);
void orc_run_rows_plan(int rows, int cols, int workers, int* n_chunks, int* chunk);

/* ---- layer forwards (poly/dense.go:66-101; poly/swiglu.go:37-46,270-322) ---- */
typedef struct orc_matrix {
    int rows;
    int cols;
    int row_words;
    float scale;
    const uint32_t* words;
    const uint8_t* codes; /* optional byte-code cache (orc_ensure_codes), row stride orc_codes_stride(cols) */
} orc_matrix;

/* simd: 1 -> byte-code AVX2 path (bitnet_simd on), 0 -> scalar path.
 * workers: goroutine fan-out width for bitNetRunRows (GOMAXPROCS).
 * xq_out (M*cols), amax_out (M), acc_out (M*rows, raw signed dot) optional. */
void orc_dense_forward(const orc_matrix* w, const float* in, int m, int activation,
                       int simd, int workers, float* pre, float* post,
                       int8_t* xq_out, float* amax_out, int32_t* acc_out);

float orc_activate_f32(float v, int activation);
double orc_swiglu_gate_product(double g, double u, int activation);
void orc_bitnet_rmsnorm_row_f32(float* data, int n, const float* weight, double eps);
void orc_bitnet_rmsnorm_f64(double* data, int n, const float* weight, double eps);

/* gate/up: rows=inter, cols=hidden; down: rows=hidden, cols=inter.
 * bias: NULL or 2*inter+hidden values laid out as [gate | up | down].
 * inner_norm: NULL (weight 1) or inter values.  eps<=0 -> 1e-5.
 * h_out (M*inter) receives the normalized pre-activation like loom's preAct. */
void orc_swiglu_forward(const orc_matrix* gate, const orc_matrix* up,
                        const orc_matrix* down, const float* bias,
                        const float* inner_norm, double eps, int activation,
                        const float* in, int m, int simd, int workers,
                        float* out, float* h_out,
                        int8_t* xq_out, float* amax_out,
                        int8_t* hq_out, float* hamax_out,
                        int32_t* acc_gate, int32_t* acc_up, int32_t* acc_down);

/* RMSNorm layer (poly/norm.go:102-138): y = fp32((x/rms)*g). eps<=0 -> 1e-6. */
void orc_rmsnorm_forward(const float* x, int rows, int n, const float* gain,
                         double eps, float* y, float* rms_out);

/* ---- attention, decoder block, LM head (poly/mha.go:204-371,
 *      poly/transformer_forward.go:220-253, poly/transformer.go:635-719,
 *      poly/simd/avx2_amd64.s:14-79, poly/sampling.go:44-55) ---- */
typedef struct orc_mha {
    int d_model, num_heads, num_kv_heads, head_dim, msl;
    double theta;              /* RoPE base; <= 0 -> 10000 */
    double eps;                /* inner RMSNorm eps; <= 0 -> 1e-5 */
    const orc_matrix *q, *k, *v, *o;
    const float *bias_q, *bias_k, *bias_v, *bias_o; /* NULL -> 0 */
    const float* inner_norm;   /* NULL -> weight 1 */
    float* cache_k;            /* msl * kv_dim, caller-owned */
    float* cache_v;
    int kv_offset;             /* tokens already cached (in/out) */
    /* per-head Q / K RMSNorm weights (QNormWeight / KNormWeight); a length of
     * 0 applies no norm (poly/mha.go:285-290), eps from mhaQKNormEpsilon */
    const float* q_norm;
    int q_norm_len;
    const float* k_norm;
    int k_norm_len;
} orc_mha;

void orc_attention(const double* Q, const float* cache_k, const float* cache_v, int seq,
                   int seq_base, int msl, int heads, int kv_heads, int hd, double* attn);
long orc_attention_span(const int* rows, int nrows, int seq_base, int heads);
void orc_attention_args(const double* Q, const float* cache_k, const int* rows, int nrows,
                        int seq_base, int msl, int heads, int kv_heads, int hd, double* args);
void orc_attention_chains(const double* probs, const float* cache_v, const int* rows, int nrows,
                          int seq_base, int msl, int heads, int kv_heads, int hd, double* attn);
void orc_exp_rows(const double* x, long n, double* y);
void orc_attn_out(const orc_matrix* o, const float* bias_o, const float* inner_norm, double eps,
                  double* attn, int seq, int q_dim, int simd, int workers, float* pre,
                  float* post);
/* Projection stage of MHAForwardPackedTernaryCPU (poly/mha.go:262-314) for
 * `seq` rows at positions seq_base + s: shared quantization, Q (fp64 + bias),
 * K/V rows (fp32 + bias) into the ring caches, RoPE on Q and the cached K.
 * Q receives seq x q_dim; kv_offset is not changed. */
void orc_per_head_rmsnorm_f64(double* data, const float* gamma, int gamma_len, int heads,
                              int hd, double eps);
void orc_per_head_rmsnorm_f32(float* data, const float* gamma, int gamma_len, int heads, int hd,
                              double eps);
double orc_qk_norm_eps(double layer_eps);
void orc_mha_project(orc_mha* L, const float* in, int seq, int seq_base, int simd, int workers,
                     double* Q);
void orc_mha_forward(orc_mha* L, const float* in, int seq, int simd, int workers,
                     float* pre, float* post, double* q_out, double* attn_out);

/* Stages from given int8 rows (for stage-wise checks): the output / down
 * projection with its fp64 bias add, and the SwiGLU gate product rows. */
void orc_dense_quantized(const orc_matrix* w, const int8_t* xq, const float* amax, int m,
                         const float* bias, int simd, int workers, float* out);
void orc_swiglu_gate_rows(const orc_matrix* gate, const orc_matrix* up, const float* bias,
                          int activation, const int8_t* xq, const float* amax, int m, int simd,
                          int workers, float* h);

typedef struct orc_block {
    int hidden;
    const float* norm1;
    const float* norm2;
    double norm_eps;           /* RMSNorm layers; <= 0 -> 1e-6 */
    orc_mha mha;
    const orc_matrix *gate, *up, *down;
    const float* ffn_inner_norm;
    double ffn_eps;
    int ffn_activation;
} orc_block;

void orc_block_forward(orc_block* B, float* x, int seq, int simd, int workers);
void orc_lm_head_seq(const float* hidden, const float* lm, int vocab, int h, float* logits);
double orc_dot_tile(const float* x, const float* w, int n, double prev);
void orc_lm_head_dottile(const float* hidden, const float* lm, int vocab, int h, float* logits);
int orc_argmax_first(const float* logits, int n);

/* ---- .entity BITNET_TERNARY blob codec (poly/entity_bitnet.go:38-88) ---- */
size_t orc_entity_blob_bytes(int n_words);
size_t orc_entity_encode(int rows, int cols, int offset, float scale, int row_words,
                         const uint32_t* words, int n_words, uint8_t* raw);
/* returns 0 on success, -1 short, -2 truncated. */
int orc_entity_decode_header(const uint8_t* raw, size_t len, int* rows, int* cols,
                             int* offset, float* scale, int* row_words, int* n_words);

/* ---- deterministic inputs ---- */
void orc_deterministic_weights(float* out, int n);
uint64_t orc_splitmix64(uint64_t* state);
void orc_fill_normal_f32(float* out, long n, uint64_t seed);
void orc_fill_ternary_codes(uint8_t* native, long n, uint64_t seed);
void orc_fill_uniform_f32(float* out, long n, float lo, float hi, uint64_t seed);

#ifdef __cplusplus
}
#endif

#endif
