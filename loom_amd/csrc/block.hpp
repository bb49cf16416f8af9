// block.hpp -- launchers of the decoder-block and decode-step kernels (block.hip).
//
// Device positions: every kernel that depends on the KV position reads it from
// an int in device memory (pos0), so a captured decode step replays unchanged
// while the position advances on the device.
#pragma once

#include "lamd.hpp"

namespace lamd {

constexpr size_t kMaxAttnLds = 60 * 1024;  // dynamic LDS of one attention workgroup (q row + scores)
constexpr int kMaxAttnSpan = 7424;         // positions: (60 KiB / 8) - 256

// RMSNormForwardPolymorphic (poly/norm.go:102-138) on m rows of n, optionally
// followed by the int8 quantization of the normalized row.  y and xq may each
// be null.  eps <= 0 selects the reference default 1e-6.
// x rows are ldx floats apart; y rows are dense (n).  totals (optional, m
// doubles of workspace): in strict mode with many rows, the rows' ordered sums
// of squares are formed one lane per row first (row_sumsq_kernel).
hipError_t launch_rmsnorm_quant(const float* x, long ldx, int m, int n, const float* gain,
                                double eps, int strict, float* y, int8_t* xq, int ldq, float* amax,
                                int32_t* xsum, hipStream_t s, double* totals = nullptr);

// Per-head Q/K RMSNorm weights (QNormWeight / KNormWeight of loom's MHA,
// applyPerHeadRMSNorm*, poly/mha.go:584-646), device pointers: q (k) null
// applies no norm to Q (K); *_len is the weights' length (head_dim: shared by
// the heads, heads*head_dim: one block per head, any other: unit weights);
// eps as mhaQKNormEpsilon (poly/mha.go:19-24).  At most kQkNormMaxHeads Q and
// K heads together.
constexpr int kQkNormMaxHeads = 512;
struct QkNorm {
    const float* q = nullptr;
    int q_len = 0;
    const float* k = nullptr;
    int k_len = 0;
    double eps = 1e-6;
};

// Rescale + bias (+ per-head Q/K norms) + RoPE of the stacked Q/K/V
// accumulators (batch*seq rows of q_dim + 2*kv_dim int32): Q rows to q (fp64,
// rows x q_dim), K/V rows into the fp32 ring caches (batch slots of msl x
// kv_dim) at positions *pos0 + s.
hipError_t launch_qkv_rope(const int32_t* acc, const float* amax, float sq, float sk, float sv,
                           const float* bq, const float* bk, const float* bv, int batch, int seq,
                           const int* pos0, int msl, int heads, int kv_heads, int hd, double theta,
                           double* q, float* cache_k, float* cache_v, hipStream_t s,
                           const QkNorm& qk = QkNorm{});

// Causal attention of batch x seq queries at positions *pos0 + s over each
// sequence's ring cache.  span >= *pos0 + seq must hold (LDS holds span
// scores) and span <= msl.  Up to kSplitMaxRows query rows take the split
// decode path, which needs `scratch` (attention_scratch_bytes).
constexpr int kSplitMaxRows = 16;
size_t attention_lds_bytes(int hd, int span);
// fast_qt: 0 selects the one-pass fast prefill kernel (no score workspace),
// 2 or 4 the two-pass kernel with that many 16-query tiles per workgroup.
size_t attention_scratch_bytes(int rows, int heads, int hd, int span, int strict, int fast_qt);
// LOOM_AMD_ATTN_QT = 2 or 4 asks for the two-pass fast prefill kernel; 0 otherwise.
int attention_fast_two_pass_qt();
// Decode (one token per sequence; head_dim 64/128 fast, 32/64/128/256
// strict): the Q/K/V epilogue of qkv_rope fused into the attention launch
// (writes the new K/V to the caches, never materializes Q).
bool attention_rope_ok(int seq, int hd, int strict, int span);
hipError_t launch_attention_rope(const int32_t* acc, const float* amax, float sq, float sk, float sv,
                                 const float* bq, const float* bk, const float* bv, double theta,
                                 int batch, const int* pos0, int msl, int span, int heads,
                                 int kv_heads, int hd, int strict, float* cache_k, float* cache_v,
                                 double* scratch, double* out, hipStream_t s,
                                 double* q_tap = nullptr, const QkNorm& qk = QkNorm{});
hipError_t launch_attention(const double* q, const float* cache_k, const float* cache_v,
                            int batch, int seq, const int* pos0, int msl, int span, int heads,
                            int kv_heads, int hd, int strict, int fast_qt, double* scratch, double* out,
                            hipStream_t s);

// MHA inner norm on fp64 rows in place (data *= scale*w; skipped when
// keep_rows is false) + fp64 requantization.  pre (optional) receives fp32 of
// the normalized rows.  eps <= 0 selects 1e-5.  totals: as for
// launch_rmsnorm_quant.
hipError_t launch_norm_quant_f64(double* a, int m, int n, const float* w, double eps, int strict,
                                 float* pre, int8_t* xq, int ldq, float* amax, int32_t* xsum,
                                 hipStream_t s, bool keep_rows = true, double* totals = nullptr);

// Embedding rows of batch x seq tokens: row (b, s) takes the id at
// tokens[b*cap + *pos0 + s] (pos0 null = 0); ids outside the table give zero
// rows (poly/transformer.go:563-577).
hipError_t launch_embed(const float* table, int vocab, int hidden, const int* tokens, int cap,
                        const int* pos0, int batch, int seq, float* out, hipStream_t s);

// fp32 LM head over `rows` hidden rows (row stride hidden) in loom's amd64
// DotTile order; logits rows are vocab apart.
hipError_t launch_lm_head(const float* table, int vocab, int hidden, const float* x, int rows,
                          float* logits, hipStream_t s);
// The same logits in loom's scalar order (one sequential fp64 sum per logit).
hipError_t launch_lm_head_seq(const float* table, int vocab, int hidden, const float* x, int rows,
                              float* logits, hipStream_t s);

// Greedy sampling per logits row b: first strict maximum (index 0 when
// logits[0] is NaN), written to tokens[b*cap + *pos0 + offset] when < cap.
// Two launches; `part` holds rows x argmax_parts(n) partial results.
constexpr int kArgmaxMaxParts = 64;
int argmax_parts(int n);
hipError_t launch_argmax(const float* logits, int n, int rows, float2* part, int* tokens, int cap,
                         const int* pos0, int offset, hipStream_t s);

// Greedy token of the fp32 LM head for ONE row by screening with an int8 copy
// of the table (launch_lm_quant_rows: per-row scale and codes) and exact
// logits for the candidates only (hidden a multiple of 16, at most 2816:
// lm_screen_ok).  hi holds vocab doubles, part lm_screen_parts(vocab)
// entries; *lkey must be 0 before the first call (each call leaves it 0).
// Writes the token as launch_argmax does; only the candidates' logits are
// written.
bool lm_screen_ok(int hidden);
int lm_screen_parts(int vocab);
// q holds lm_screen_code_bytes(vocab, hidden) bytes (rows in blocks of 64,
// interleaved by 16-column group)
size_t lm_screen_code_bytes(int vocab, int hidden);
hipError_t launch_lm_quant_rows(const float* w, int vocab, int hidden, int8_t* q, float* scale, hipStream_t s);
hipError_t launch_lm_greedy_screened(const float* table, const int8_t* table_q, const float* scale, int vocab,
                                     int hidden, const float* x, int sequential, double* hi,
                                     unsigned long long* lkey, float* logits, float2* part, int* tokens, int cap,
                                     const int* pos0, int offset, hipStream_t s);

hipError_t launch_set_int(int* p, int v, hipStream_t s);
hipError_t launch_add_int(int* p, int v, hipStream_t s);

}  // namespace lamd
