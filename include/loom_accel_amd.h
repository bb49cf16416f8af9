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

/* Summation order of the fp32 LM head (both bit-exact with loom). */
#define LOOM_AMD_LM_DOTTILE 0    /* SIMD forward on: simd.DotTile's eight-lane order */
#define LOOM_AMD_LM_SEQUENTIAL 1 /* SIMD forward off: one sequential fp64 sum per logit */

/* Message of the last failing loom_amd_* call on the calling thread. */
const char* loom_amd_last_error(void);

/* Number of visible gfx950 devices (0 when none). */
int loom_amd_device_count(void);

/* Kernel family the matmul dispatcher uses for m token rows
 * ("skinny_m16_fusedq" -- quantization fused into the matmul launch when the
 * fp32 rows allow it: m <= 4, or m <= 8 with k <= 4096 --, "skinny_m16",
 * "skinny_m32", "skinny_m64", "gemm_m64", "gemm"). */
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

/* Same, from Microsoft's offline BitNet U8 layout (HF checkpoints): packed is
 * (rows/4) x cols bytes in host memory, byte (pr, c) holding the codes of
 * rows lane*(rows/4) + pr for lane 0..3; scale is the checkpoint's
 * weight_scale.  Replaces packMicrosoftOfflineBitNetRowsToU32FromBytes
 * (poly/bitnet_cpu.go:1078-1098) followed by the repack.  Synchronous. */
int loom_amd_matrix_from_ms_offline(int device, const uint8_t* packed, int rows, int cols,
                                    float scale, loom_amd_matrix** out);

/* Same, from an fp32 master (host, rows x cols, row-major), packed as loom's
 * packFloat32AsBitNetTernaryMatrix does (poly/bitnet_cpu.go:934-962): scale =
 * fp32(sequential fp64 sum of |w| / n) (0 -> 1), code = clamp(round(fp64(w /
 * scale)), -1, 1) with the fp32 division of bitNetQuantValue
 * (poly/bitnet_cpu.go:119-146); a master whose every weight is within 1e-6 of
 * -1, 0 or 1 is packed at scale 1.  *scale_out (optional) receives the scale.
 * Synchronous. */
int loom_amd_matrix_from_float32(int device, const float* master, int rows, int cols,
                                 loom_amd_matrix** out, float* scale_out);

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

/* The reference's sequential fp64 sum, out[i] = s0 + t[i][0] + t[i][1] + ...
 * in index order with one rounding per addition, for m rows of n terms
 * (n <= 8064; device pointers), one workgroup of `threads` (64, 256 or 512:
 * the widths the strict norm kernels use) per row.  Every strict-mode sum of
 * squares is this chain (e.g. the sum of squares of
 * bitNetRMSNormTensorRowWeighted, poly/bitnet_cpu.go:901-905); the entry
 * point has no counterpart of its own in the reference: it exposes the
 * library's exact parallel forms of the chain so that callers and tests can
 * check them against a plain sequential sum. */
int loom_amd_ordered_sum_rows(const double* terms, int m, int n, double s0, double* out,
                              int threads, void* stream);

/* Re-reads the LOOM_AMD_* tuning variables (the tuning table of the
 * library's documentation), which the library otherwise reads once, when it
 * first plans a launch.  No counterpart in the reference: for tuning runs and
 * tests that change the variables within one process.  Must not run while
 * another thread launches work through the library.  Returns 0. */
int loom_amd_reload_tuning(void);

/* y[i] = exp(x[i]) for n fp64 values (device pointers), with the device exp
 * that every kernel of the library calls: the attention probabilities
 * exp(score - max) of MHAForwardPackedTernaryCPU (poly/mha.go:339-342), the
 * SwiGLU gate's sigmoid (poly/swiglu.go:37-46) and Activate
 * (poly/poly.go:167-200), all math.Exp in the reference.  No counterpart of
 * its own in the reference: it lets callers and tests evaluate the
 * reference's exp-free chains around the device's exp, e.g. strict
 * attention bit for bit. */
int loom_amd_exp_rows(const double* x, long n, double* y, void* stream);

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

/* loom_amd_dense_forward that allocates nothing.  No counterpart in loom: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Quantized
 * rows are staged in a fixed 8 MiB device array per GPU instead of the
 * growable scratch arena: m * (256*ceil(k/256) + 8) plus alignment must fit
 * 8 MiB (larger calls fail with a message; rows the matmul quantizes itself,
 * up to four, or eight for k <= 4096, need no staging).
 * Every call on one GPU shares that array: calls overlapping on one GPU race
 * and must be serialized by the caller.  Like every direct loom_amd_* call,
 * it also shares the GPU's split-K partial sums and arrival counters with
 * the other entry points and with plugin infers on that GPU (which hold a
 * per-device lock the direct calls do not take): a direct call must not
 * overlap a plugin infer or another direct call on the same GPU.  Same
 * outputs as loom_amd_dense_forward, without taps. */
int loom_amd_dense_forward_noalloc(const loom_amd_matrix* w, const float* x, int m,
                                   int activation, float* pre, float* post,
                                   const float* residual, void* stream);

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

/* ---- decoder block (poly/transformer_forward.go:228-245) -------------- */

typedef struct loom_amd_block loom_amd_block;

/* Shape and numerics of one BitNet decoder block:
 *   x += O(InnerNorm(Attention(RoPE(Q,K,V)(RMSNorm1(x)))))
 *   x += SwiGLU(RMSNorm2(x))
 * Sequential fp64 sums of the reference (RMSNorms, inner norms, softmax
 * sums) follow norm_mode: STRICT adds in the reference's order; FAST uses a
 * fixed parallel order.  exp/pow/sin/cos are the device libm's (within 1 ulp
 * of the host's, not bit-identical). */
typedef struct loom_amd_block_desc {
    int hidden;         /* d_model */
    int num_heads;
    int num_kv_heads;   /* 0 = num_heads; must divide num_heads */
    int head_dim;       /* multiple of 4, <= 256 */
    int intermediate;   /* SwiGLU width */
    int max_seq_len;    /* KV ring rows, loom MaxSeqLen (0 = 512), at most 7424; a call
                           whose positions would pass it is refused (loom wraps the ring) */
    int max_batch;      /* independent sequences per call (0 = 1) */
    double rope_theta;  /* 0 = 10000 */
    double norm_eps;    /* RMSNorm1/2 eps (<= 0: 1e-6, poly/norm.go:104) */
    double attn_eps;    /* the MHA layer's RMSNormEps: inner norm eps (<= 0: 1e-5);
                           per-head Q/K norm eps (<= 0: 1e-6, mhaQKNormEpsilon) */
    double ffn_eps;     /* SwiGLU inner norm eps (<= 0: 1e-5) */
    int ffn_activation; /* gate activation: 1 SiLU, 6 ReLU2 */
    int norm_mode;      /* LOOM_AMD_NORM_STRICT or LOOM_AMD_NORM_FAST */
} loom_amd_block_desc;

/* Weights of one block.  Matrices are copied into the block at create time
 * (the caller may release them afterwards); the float arrays are HOST
 * memory, copied at create time. */
typedef struct loom_amd_block_weights {
    const loom_amd_matrix* q;    /* q_dim x hidden */
    const loom_amd_matrix* k;    /* kv_dim x hidden */
    const loom_amd_matrix* v;    /* kv_dim x hidden */
    const loom_amd_matrix* o;    /* hidden x q_dim */
    const loom_amd_matrix* gate; /* intermediate x hidden */
    const loom_amd_matrix* up;   /* intermediate x hidden */
    const loom_amd_matrix* down; /* hidden x intermediate */
    const float* norm1;           /* hidden */
    const float* norm2;           /* hidden */
    const float* attn_inner_norm; /* q_dim, NULL = ones */
    const float* ffn_inner_norm;  /* intermediate, NULL = ones */
    const float* bias_q;          /* q_dim, optional */
    const float* bias_k;          /* kv_dim, optional */
    const float* bias_v;          /* kv_dim, optional */
    const float* bias_o;          /* hidden, optional */
    /* per-head Q / K RMSNorm weights, loom's QNormWeight / KNormWeight
     * (poly/mha.go:285-290, 584-646), applied before RoPE when the length
     * is > 0: head_dim (shared by every head), heads*head_dim (one block per
     * head) or any other length (unit weights, as loom) */
    const float* q_norm;
    int q_norm_len;
    const float* k_norm;
    int k_norm_len;
} loom_amd_block_weights;

/* Optional device copies of block intermediates (rows = batch*seq), every
 * field optional.  Requesting taps does not change which kernels run: each
 * stage writes its tap from the kernel that computes it. */
typedef struct loom_amd_block_taps {
    float* y1;         /* rows x hidden: RMSNorm1 output */
    double* q;         /* rows x q_dim: Q after bias and RoPE */
    double* attn;      /* rows x q_dim: attention output before the inner norm */
    float* mid;        /* rows x hidden: x after the attention residual */
    int8_t* xq1;       /* rows x hidden: int8 RMSNorm1 rows (Q/K/V input) */
    float* amax1;      /* rows: their activation absmax (floored at 1e-5) */
    double* attn_norm; /* rows x q_dim: attention after the MHA inner norm */
    int8_t* aq;        /* rows x q_dim: its int8 rows (O projection input) */
    float* aamax;      /* rows */
    float* y2;         /* rows x hidden: RMSNorm2 output */
    int8_t* xq2;       /* rows x hidden: its int8 rows (gate/up input) */
    float* amax2;      /* rows */
    float* h;          /* rows x intermediate: gate product before the inner norm */
    float* hn;         /* rows x intermediate: after the SwiGLU inner norm (loom's preAct) */
    int8_t* hq;        /* rows x intermediate: its int8 rows (down input) */
    float* hamax;      /* rows */
} loom_amd_block_taps;

/* Build a block on device: stacks Q|K|V into one projection, allocates the
 * KV ring caches (max_batch x max_seq_len x kv_dim fp32, K and V) and the
 * device position.  Synchronous. */
int loom_amd_block_create(int device, const loom_amd_block_desc* desc,
                          const loom_amd_block_weights* w, loom_amd_block** out);
void loom_amd_block_release(loom_amd_block* b);

/* One block forward on x (DEVICE, batch x seq x hidden fp32, in place).
 * KV rule of mhaPrepareKVForForward (poly/mha_layout.go:62-70): a call with
 * seq == 1 on a warm cache continues at the current position; any other
 * call restarts at position 0.  Each of the batch sequences has its own KV
 * cache; all of them advance together, so a single-token call on a warm
 * cache must carry the batch that filled it (another batch is refused).
 * loom's own 3-D batch semantics -- the batch's sequences share one KV
 * timeline from position 0 (poly/mha.go:251-371) -- are this call with
 * batch = 1 and seq = batch * seq over the same rows.  Replaces the block loop body of
 * forwardOnCPUNormal (poly/transformer_forward.go:228-245) for BitNet layers
 * (MHAForwardPackedTernaryCPU, poly/mha.go:204-371, and
 * SwiGLUForwardPackedTernaryCPU, poly/bitnet_cpu.go:915-1002).  May grow the
 * block's workspace (synchronizing the stream) when rows exceed earlier calls. */
int loom_amd_block_forward(loom_amd_block* b, float* x, int batch, int seq,
                           const loom_amd_block_taps* taps, void* stream);

/* Current KV position (loom KVOffset) as the host tracks it. */
int loom_amd_block_kv_offset(const loom_amd_block* b);

/* Device pointers of the K and V ring of one sequence slot (max_seq_len x kv_dim). */
int loom_amd_block_kv_cache(const loom_amd_block* b, int slot, const float** k,
                            const float** v);

/* ---- LM head and greedy sampling -------------------------------------- */

/* fp32 LM head (applyFP32LMHeadRows with SIMD on amd64,
 * poly/transformer.go:673-720): logits[r][v] = DotTile(x[r], table[v]) with
 * loom's eight-lane fp64 order (poly/simd/avx2_amd64.s:14-79).  table is
 * vocab x hidden, x rows x hidden, logits rows x vocab (all DEVICE). */
int loom_amd_lm_head(const float* table, int vocab, int hidden, const float* x, int rows,
                     float* logits, void* stream);

/* The same head with SIMD forward off (applyFP32LMHeadRows' scalar loop,
 * poly/transformer.go:681-687, = dotTileGo, poly/simd/dot.go:14-21):
 * logits[r][v] = fp32(sum over d in order of fp64(x[r][d]) * fp64(table[v][d])). */
int loom_amd_lm_head_sequential(const float* table, int vocab, int hidden, const float* x,
                                int rows, float* logits, void* stream);

/* Greedy SampleTopK (k <= 1, poly/sampling.go:44-55) per row: the first
 * index of the largest logit, 0 when logits[r][0] is NaN.  ids (DEVICE) gets
 * one int32 per row. */
int loom_amd_greedy_sample(const float* logits, int n, int rows, int32_t* ids, void* stream);

/* ---- transformer decode (poly/transformer.go:330-520) ---------------- */

typedef struct loom_amd_model loom_amd_model;

typedef struct loom_amd_model_desc {
    loom_amd_block_desc block; /* every layer has this shape */
    int num_layers;
    int vocab;
    double final_norm_eps; /* <= 0: 1e-6 */
    int max_tokens;        /* tokens per sequence the model can hold (prompt + generated) */
    int max_prefill;       /* largest prompt length per call (0 = max_tokens) */
    int lm_head_order;     /* fp32 head: LOOM_AMD_LM_DOTTILE (Network.UseSimdForward on
                              amd64/arm64) or LOOM_AMD_LM_SEQUENTIAL (SIMD forward off) */
} loom_amd_model_desc;

/* Build a model: layers[num_layers] as for loom_amd_block_create, fp32
 * embeddings (HOST, vocab x hidden), final RMSNorm gain (HOST, hidden, NULL =
 * no final norm) and fp32 LM head (HOST, vocab x hidden, NULL = tied to the
 * embeddings, BitNet's weight tying).  A tied head runs in fp32, summed in
 * desc->lm_head_order (poly/transformer.go:664-719).  An untied head of a model whose layers
 * are ternary is what loom ternarizes (usePackedTernaryLMHead,
 * poly/transformer.go:721-755): it is packed once here as
 * loom_amd_matrix_from_float32 does and applied as the ternary matvec with
 * per-token int8 activations, logits fp32(fp64 result).  All layers share one
 * device position. */
int loom_amd_model_create(int device, const loom_amd_model_desc* desc,
                          const loom_amd_block_weights* layers, const float* embeddings,
                          const float* final_norm, const float* lm_head, loom_amd_model** out);
void loom_amd_model_release(loom_amd_model* m);

/* Prefill: restart every sequence with batch x n prompt ids (HOST), run the
 * stack, the final norm and the LM head on each sequence's last row, and
 * pick the next token greedily (SampleTopK with k<=1, poly/sampling.go:44-55).
 * The ids are copied out of the caller's memory before the call returns.
 * logits (DEVICE, batch x vocab) is optional. */
int loom_amd_model_prefill(loom_amd_model* m, const int32_t* ids, int batch, int n,
                           float* logits, void* stream);

/* `steps` greedy decode steps: each feeds every sequence's newest token at
 * the current position, runs the stack, the LM head and the argmax, and
 * appends the result.  use_graph != 0 replays one captured HIP graph per
 * step (positions live on the device).  logits (DEVICE, batch x vocab) is
 * optional and holds the last step's logits. */
int loom_amd_model_decode(loom_amd_model* m, int steps, int use_graph, float* logits,
                          void* stream);

/* Copy the tokens of every sequence (HOST, batch x count: prompt then
 * generated ids).  Waits for stream; `out` holds the ids when the call
 * returns.  count = current position + 1. */
int loom_amd_model_tokens(const loom_amd_model* m, int32_t* out, int count, void* stream);

/* Current position (tokens fed through the stack per sequence). */
int loom_amd_model_position(const loom_amd_model* m);

/* Final hidden rows of the last call (DEVICE, batch x hidden: each
 * sequence's last row after the final norm). */
const float* loom_amd_model_last_hidden(const loom_amd_model* m);

#ifdef __cplusplus
}
#endif

#endif /* LOOM_ACCEL_AMD_H */
