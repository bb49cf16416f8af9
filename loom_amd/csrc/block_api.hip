// block_api.hip -- loom_amd_block_* and loom_amd_model_* entry points
// (include/loom_accel_amd.h): one BitNet decoder block, and the greedy
// decode loop of a stack of them, device-resident end to end.
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "api_util.hpp"
#include "block.hpp"
#include "lamd.hpp"
#include "loom_accel_amd.h"

namespace lamd {

// Device state of one block.  Every buffer is owned by the block.
struct BlockDev {
    int device = 0;
    int hidden = 0, heads = 0, kv_heads = 0, hd = 0, inter = 0, msl = 0, max_batch = 1;
    int q_dim = 0, kv_dim = 0;
    double theta = 10000.0, norm_eps = 0.0, attn_eps = 0.0, ffn_eps = 0.0;
    int activation = 1, strict = 1;
    int attn_qt = 0;  // fast prefill attention kernel (attention_fast_two_pass_qt at creation)
    bool fuse_rope = true;  // decode: Q/K/V epilogue inside the attention launch
    bool fuse_norm = true;  // decode: row norms inside the consuming matmul
    Matrix qkv, o, gate, up, down;  // tiles point into `weights`
    float sq = 1.0f, sk = 1.0f, sv = 1.0f;
    float *norm1 = nullptr, *norm2 = nullptr, *attn_norm = nullptr, *ffn_norm = nullptr;
    float *bq = nullptr, *bk = nullptr, *bv = nullptr, *bo = nullptr;
    QkNorm qk;  // per-head Q/K norms (device weights; none when null)
    float *cache_k = nullptr, *cache_v = nullptr;  // max_batch x msl x kv_dim
    void* weights = nullptr;
    void* params = nullptr;
    void* caches = nullptr;

    int span() const { return msl; }
    size_t cache_slot() const { return (size_t)msl * kv_dim; }
};

// Per-call intermediates for `rows` token rows.
struct Workspace {
    void* base = nullptr;
    size_t bytes = 0;
    int rows = 0;
    int8_t* xq = nullptr;  // rows x pad(hidden)
    float* amax = nullptr;
    int32_t* xsum = nullptr;
    int32_t* acc = nullptr;  // rows x (q_dim + 2 kv_dim)
    double* q = nullptr;     // rows x q_dim
    double* attn = nullptr;  // rows x q_dim
    double* scores = nullptr;  // attention scratch (decode: partial results; prefill: scores)
    int8_t* aq = nullptr;    // rows x pad(q_dim)
    float* amax2 = nullptr;
    int32_t* xsum2 = nullptr;
    float* h = nullptr;      // rows x inter
    int8_t* hq = nullptr;    // rows x pad(inter)
    float* amax3 = nullptr;
    int32_t* xsum3 = nullptr;
    double* totals = nullptr;  // rows x fp64: strict ordered sums of squares (many rows)
};

static size_t workspace_layout(const BlockDev& B, int rows, Workspace* W, char* base) {
    Layout L;
    const size_t r = (size_t)rows;
    const size_t o_xq = L.take(r * pad_cols(B.hidden));
    const size_t o_am = L.take(r * 4);
    const size_t o_xs = L.take(r * 4);
    const size_t o_acc = L.take(r * (B.q_dim + 2 * B.kv_dim) * 4);
    const size_t o_q = L.take(r * B.q_dim * 8);
    const size_t o_at = L.take(r * B.q_dim * 8);
    const size_t sc_small = attention_scratch_bytes(rows < kSplitMaxRows ? rows : kSplitMaxRows,
                                                    B.heads, B.hd, B.span(), B.strict, B.attn_qt);
    const size_t sc_big = attention_scratch_bytes(rows, B.heads, B.hd, B.span(), B.strict, B.attn_qt);
    const size_t o_sc = L.take(sc_small > sc_big ? sc_small : sc_big);
    const size_t o_aq = L.take(r * pad_cols(B.q_dim));
    const size_t o_am2 = L.take(r * 4);
    const size_t o_xs2 = L.take(r * 4);
    const size_t o_h = L.take(r * B.inter * 4);
    const size_t o_hq = L.take(r * pad_cols(B.inter));
    const size_t o_am3 = L.take(r * 4);
    const size_t o_xs3 = L.take(r * 4);
    const size_t o_tot = L.take(r * 8);
    if (W && base) {
        W->base = base;
        W->bytes = L.off;
        W->rows = rows;
        W->xq = (int8_t*)(base + o_xq);
        W->amax = (float*)(base + o_am);
        W->xsum = (int32_t*)(base + o_xs);
        W->acc = (int32_t*)(base + o_acc);
        W->q = (double*)(base + o_q);
        W->attn = (double*)(base + o_at);
        W->scores = (double*)(base + o_sc);
        W->aq = (int8_t*)(base + o_aq);
        W->amax2 = (float*)(base + o_am2);
        W->xsum2 = (int32_t*)(base + o_xs2);
        W->h = (float*)(base + o_h);
        W->hq = (int8_t*)(base + o_hq);
        W->amax3 = (float*)(base + o_am3);
        W->xsum3 = (int32_t*)(base + o_xs3);
        W->totals = (double*)(base + o_tot);
    }
    return L.off;
}

static void free_workspace(Workspace* W) {
    if (W->base) (void)hipFree(W->base);
    *W = Workspace{};
}

static int alloc_workspace(const BlockDev& B, int rows, Workspace* W) {
    const size_t bytes = workspace_layout(B, rows, nullptr, nullptr);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail_hip("block workspace", e);
    workspace_layout(B, rows, W, (char*)p);
    return 0;
}

static void free_block(BlockDev* B) {
    if (B->weights) (void)hipFree(B->weights);
    if (B->params) (void)hipFree(B->params);
    if (B->caches) (void)hipFree(B->caches);
    B->weights = B->params = B->caches = nullptr;
}

static int check_desc(const loom_amd_block_desc* d) {
    if (!d) return fail("block desc is null");
    if (d->hidden <= 0 || d->num_heads <= 0 || d->head_dim <= 0 || d->intermediate <= 0) {
        return fail("block desc: hidden, num_heads, head_dim and intermediate must be positive");
    }
    const int kvh = d->num_kv_heads > 0 ? d->num_kv_heads : d->num_heads;
    if (d->num_heads % kvh != 0) return fail("block desc: num_kv_heads must divide num_heads");
    if (d->head_dim % 4 != 0 || d->head_dim > 256) {
        return fail("block desc: head_dim must be a multiple of 4 and at most 256");
    }
    const int msl = d->max_seq_len > 0 ? d->max_seq_len : 512;
    if (msl > kMaxAttnSpan) {
        return fail("block desc: max_seq_len is limited to " + std::to_string(kMaxAttnSpan));
    }
    if (d->max_batch < 0) return fail("block desc: max_batch must be >= 0");
    const int strict = d->norm_mode == LOOM_AMD_NORM_STRICT;
    const int q_dim = d->num_heads * d->head_dim;
    const int widest = d->hidden > q_dim ? (d->hidden > d->intermediate ? d->hidden : d->intermediate)
                                         : (q_dim > d->intermediate ? q_dim : d->intermediate);
    if (widest > kMaxNormCols || (strict && widest > kMaxStrictNormCols)) {
        return fail("block desc: normalized widths are limited to 8192 (strict: 8064)");
    }
    if ((q_dim % kTileRows) != 0 || ((kvh * d->head_dim) % kTileRows) != 0) {
        return fail("block desc: q_dim and kv_dim must be multiples of 16");
    }
    return 0;
}

static int expect_shape(const loom_amd_matrix* w, const char* name, int rows, int cols, int dev) {
    if (w == nullptr || w->m.tiles == nullptr) return fail(std::string(name) + " matrix is null");
    if (w->m.rows != rows || w->m.cols != cols) {
        return fail(std::string(name) + " matrix is " + std::to_string(w->m.rows) + "x" +
                    std::to_string(w->m.cols) + ", want " + std::to_string(rows) + "x" +
                    std::to_string(cols));
    }
    if (w->m.device != dev) return fail(std::string(name) + " matrix is on another device");
    return 0;
}

// Builds the device state of one block (synchronous).
static int build_block(int device, const loom_amd_block_desc* d, const loom_amd_block_weights* w,
                       BlockDev* B) {
    if (check_desc(d)) return -1;
    if (!w) return fail("block weights are null");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        return fail("device " + std::to_string(device) + " is not visible");
    }
    if (!is_gfx950(device)) return fail("device is not gfx950");
    B->device = device;
    B->hidden = d->hidden;
    B->heads = d->num_heads;
    B->kv_heads = d->num_kv_heads > 0 ? d->num_kv_heads : d->num_heads;
    B->hd = d->head_dim;
    B->inter = d->intermediate;
    B->msl = d->max_seq_len > 0 ? d->max_seq_len : 512;
    B->max_batch = d->max_batch > 0 ? d->max_batch : 1;
    B->q_dim = B->heads * B->hd;
    B->kv_dim = B->kv_heads * B->hd;
    B->theta = d->rope_theta > 0 ? d->rope_theta : 10000.0;
    B->norm_eps = d->norm_eps;
    B->attn_eps = d->attn_eps;
    B->ffn_eps = d->ffn_eps;
    B->activation = d->ffn_activation;
    B->strict = d->norm_mode == LOOM_AMD_NORM_STRICT;
    B->attn_qt = attention_fast_two_pass_qt();
    // LOOM_AMD_UNFUSED_ROPE=1 keeps the separate Q/K/V epilogue launch in
    // decode (the tests compare both paths)
    B->fuse_rope = tune_int("LOOM_AMD_UNFUSED_ROPE", 0) != 1;
    // LOOM_AMD_UNFUSED_NORM=1 keeps the separate norm launches in decode
    B->fuse_norm = tune_int("LOOM_AMD_UNFUSED_NORM", 0) != 1;
    const int H = B->hidden;
    if (expect_shape(w->q, "q", B->q_dim, H, device) || expect_shape(w->k, "k", B->kv_dim, H, device) ||
        expect_shape(w->v, "v", B->kv_dim, H, device) || expect_shape(w->o, "o", H, B->q_dim, device) ||
        expect_shape(w->gate, "gate", B->inter, H, device) ||
        expect_shape(w->up, "up", B->inter, H, device) ||
        expect_shape(w->down, "down", H, B->inter, device)) {
        return -1;
    }
    if (!w->norm1 || !w->norm2) return fail("norm1 and norm2 gains are required");
    if (w->q_norm_len < 0 || w->k_norm_len < 0 || (w->q_norm_len > 0 && !w->q_norm) ||
        (w->k_norm_len > 0 && !w->k_norm)) {
        return fail("block weights: per-head norm weights and lengths disagree");
    }
    if ((w->q_norm_len > 0 || w->k_norm_len > 0) && B->heads + B->kv_heads > kQkNormMaxHeads) {
        return fail("block desc: per-head Q/K norms support at most " + std::to_string(kQkNormMaxHeads) +
                    " Q and K heads together");
    }
    DeviceGuard guard(device);

    // weights: stacked [Q; K; V] then O, gate, up, down, each 256-byte aligned
    Layout L;
    const size_t o_qkv = L.take(w->q->m.bytes() + w->k->m.bytes() + w->v->m.bytes());
    const size_t o_o = L.take(w->o->m.bytes());
    const size_t o_g = L.take(w->gate->m.bytes());
    const size_t o_u = L.take(w->up->m.bytes());
    const size_t o_d = L.take(w->down->m.bytes());
    hipError_t e = hipMalloc(&B->weights, L.off);
    if (e != hipSuccess) return fail_hip("block weights", e);
    char* wb = (char*)B->weights;
    size_t at = o_qkv;
    for (const loom_amd_matrix* m : {w->q, w->k, w->v}) {
        if (e == hipSuccess) e = hipMemcpy(wb + at, m->m.tiles, m->m.bytes(), hipMemcpyDeviceToDevice);
        at += m->m.bytes();
    }
    auto place = [&](Matrix* dst, const loom_amd_matrix* src, size_t off) {
        *dst = src->m;
        dst->tiles = (uint32_t*)(wb + off);
        if (e == hipSuccess) e = hipMemcpy(dst->tiles, src->m.tiles, src->m.bytes(), hipMemcpyDeviceToDevice);
    };
    place(&B->o, w->o, o_o);
    place(&B->gate, w->gate, o_g);
    place(&B->up, w->up, o_u);
    place(&B->down, w->down, o_d);
    B->qkv = w->q->m;
    B->qkv.rows = B->q_dim + 2 * B->kv_dim;
    B->qkv.ntiles = B->qkv.rows / kTileRows;
    B->qkv.tiles = (uint32_t*)(wb + o_qkv);
    B->qkv.scale = 1.0f;  // EPI_ACC: the Q/K/V scales are applied by qkv_rope
    B->sq = w->q->m.scale;
    B->sk = w->k->m.scale;
    B->sv = w->v->m.scale;
    if (e != hipSuccess) {
        free_block(B);
        return fail_hip("block weight copy", e);
    }

    // small fp32 parameters
    Layout P;
    const size_t p_n1 = P.take((size_t)H * 4);
    const size_t p_n2 = P.take((size_t)H * 4);
    const size_t p_an = P.take(w->attn_inner_norm ? (size_t)B->q_dim * 4 : 0);
    const size_t p_fn = P.take(w->ffn_inner_norm ? (size_t)B->inter * 4 : 0);
    const size_t p_bq = P.take(w->bias_q ? (size_t)B->q_dim * 4 : 0);
    const size_t p_bk = P.take(w->bias_k ? (size_t)B->kv_dim * 4 : 0);
    const size_t p_bv = P.take(w->bias_v ? (size_t)B->kv_dim * 4 : 0);
    const size_t p_bo = P.take(w->bias_o ? (size_t)H * 4 : 0);
    const size_t p_qn = P.take((size_t)(w->q_norm_len > 0 ? w->q_norm_len : 0) * 4);
    const size_t p_kn = P.take((size_t)(w->k_norm_len > 0 ? w->k_norm_len : 0) * 4);
    e = hipMalloc(&B->params, P.off);
    if (e != hipSuccess) {
        free_block(B);
        return fail_hip("block parameters", e);
    }
    char* pb = (char*)B->params;
    auto up = [&](float** dst, const float* src, size_t off, size_t n) {
        if (!src) return;
        *dst = (float*)(pb + off);
        if (e == hipSuccess) e = hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice);
    };
    up(&B->norm1, w->norm1, p_n1, H);
    up(&B->norm2, w->norm2, p_n2, H);
    up(&B->attn_norm, w->attn_inner_norm, p_an, B->q_dim);
    up(&B->ffn_norm, w->ffn_inner_norm, p_fn, B->inter);
    up(&B->bq, w->bias_q, p_bq, B->q_dim);
    up(&B->bk, w->bias_k, p_bk, B->kv_dim);
    up(&B->bv, w->bias_v, p_bv, B->kv_dim);
    up(&B->bo, w->bias_o, p_bo, H);
    // QNormWeight / KNormWeight apply when non-empty (poly/mha.go:285-290),
    // with eps from mhaQKNormEpsilon (poly/mha.go:19-24)
    float* qn = nullptr;
    float* kn = nullptr;
    if (w->q_norm_len > 0) up(&qn, w->q_norm, p_qn, (size_t)w->q_norm_len);
    if (w->k_norm_len > 0) up(&kn, w->k_norm, p_kn, (size_t)w->k_norm_len);
    B->qk.q = qn;
    B->qk.q_len = w->q_norm_len;
    B->qk.k = kn;
    B->qk.k_len = w->k_norm_len;
    B->qk.eps = d->attn_eps > 0 ? d->attn_eps : 1e-6;

    // KV rings, zeroed like a fresh loom cache
    const size_t cache_bytes = (size_t)B->max_batch * B->cache_slot() * 4;
    if (e == hipSuccess) e = hipMalloc(&B->caches, 2 * cache_bytes);
    if (e == hipSuccess) e = hipMemset(B->caches, 0, 2 * cache_bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_block(B);
        return fail_hip("block parameters", e);
    }
    B->cache_k = (float*)B->caches;
    B->cache_v = (float*)((char*)B->caches + cache_bytes);
    return 0;
}

static hipError_t tap_copy(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (!dst) return hipSuccess;
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s);
}

// int8 rows of a padded workspace (ld bytes apart) into a dense tap (n bytes apart).
static hipError_t tap_rows(int8_t* dst, const int8_t* src, int ld, int n, int rows, hipStream_t s) {
    if (!dst) return hipSuccess;
    return hipMemcpy2DAsync(dst, (size_t)n, src, (size_t)ld, (size_t)n, rows, hipMemcpyDeviceToDevice, s);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Enqueues one block forward on x (rows = batch*seq) at device position *pos.
// Few rows take the decode path: each row norm runs inside the matmul that
// consumes it (launch_matmul_norm).  Taps never change the path: every stage
// writes its tap from the kernel that computes it (workgroup 0 of a
// norm-fused matmul, the chunk-0 workgroups of the fused decode attention) or
// by a copy of the workspace it leaves behind.
static int block_forward_dev(const BlockDev& B, const Workspace& W, float* x, int batch, int seq,
                             const int* pos, const loom_amd_block_taps* taps, hipStream_t s) {
    const int R = batch * seq;
    const int ldh = pad_cols(B.hidden), ldqd = pad_cols(B.q_dim), ldi = pad_cols(B.inter);
    const double rms_eps = B.norm_eps > 0 ? B.norm_eps : 1e-6;   // RMSNormForwardPolymorphic
    const double attn_eps = B.attn_eps > 0 ? B.attn_eps : 1e-5;  // bitNetRMSNormFloat64Weighted
    const double ffn_eps = B.ffn_eps > 0 ? B.ffn_eps : 1e-5;     // bitNetRMSNormTensorRowWeighted
    const loom_amd_block_taps none{};
    const loom_amd_block_taps& T = taps ? *taps : none;
    const bool fuse = B.fuse_norm && aligned16(x);
    hipError_t e;
#define TAP(call)                                                  \
    do {                                                           \
        if ((e = (call)) != hipSuccess) return fail_hip("block taps", e); \
    } while (0)
    // x := x + MHA(RMSNorm1(x))
    {
        Epilogue ep;
        ep.kind = EPI_ACC;
        ep.acc0 = W.acc;
        if (fuse && norm_fused_ok(R, B.hidden, B.strict, true)) {
            NormTaps nt;
            nt.rows = T.y1;
            nt.xq = T.xq1;
            e = launch_matmul_norm(&B.qkv, nullptr, x, nullptr, R, NORM_RMS, B.strict, B.norm1,
                                   rms_eps, ep, W.amax, s, &nt);
            if (e != hipSuccess) return fail_hip("block rmsnorm1 + qkv projection", e);
        } else {
            e = launch_rmsnorm_quant(x, B.hidden, R, B.hidden, B.norm1, rms_eps, B.strict, T.y1,
                                     W.xq, ldh, W.amax, W.xsum, s, W.totals);
            if (e != hipSuccess) return fail_hip("block rmsnorm1", e);
            TAP(tap_rows(T.xq1, W.xq, ldh, B.hidden, R, s));
            QuantAct a{W.xq, ldh, W.amax, W.xsum};
            e = launch_matmul(&B.qkv, nullptr, a, R, ep, s);
            if (e != hipSuccess) return fail_hip("block qkv projection", e);
        }
        TAP(tap_copy(T.amax1, W.amax, (size_t)R * 4, s));
    }
    if (B.fuse_rope && batch <= kSplitMaxRows && attention_rope_ok(seq, B.hd, B.strict, B.span())) {
        // decode: the Q/K/V epilogue runs inside the attention launch
        e = launch_attention_rope(W.acc, W.amax, B.sq, B.sk, B.sv, B.bq, B.bk, B.bv, B.theta, batch, pos,
                                  B.msl, B.span(), B.heads, B.kv_heads, B.hd, B.strict, B.cache_k,
                                  B.cache_v,
                                  W.scores, W.attn, s, T.q, B.qk);
        if (e != hipSuccess) return fail_hip("block attention", e);
    } else {
        e = launch_qkv_rope(W.acc, W.amax, B.sq, B.sk, B.sv, B.bq, B.bk, B.bv, batch, seq, pos, B.msl,
                            B.heads, B.kv_heads, B.hd, B.theta, W.q, B.cache_k, B.cache_v, s, B.qk);
        if (e != hipSuccess) return fail_hip("block qkv rope", e);
        TAP(tap_copy(T.q, W.q, (size_t)R * B.q_dim * 8, s));
        e = launch_attention(W.q, B.cache_k, B.cache_v, batch, seq, pos, B.msl, B.span(), B.heads,
                             B.kv_heads, B.hd, B.strict, B.attn_qt, W.scores, W.attn, s);
        if (e != hipSuccess) return fail_hip("block attention", e);
    }
    TAP(tap_copy(T.attn, W.attn, (size_t)R * B.q_dim * 8, s));
    {
        Epilogue ep;
        ep.kind = EPI_DENSE;
        ep.bias0 = B.bo;
        ep.residual = x;
        ep.out = x;
        ep.ldo = B.hidden;
        if (fuse && norm_fused_ok(R, B.q_dim, B.strict, true)) {
            NormTaps nt;
            nt.rows = T.attn_norm;
            nt.xq = T.aq;
            nt.amax = T.aamax;
            e = launch_matmul_norm(&B.o, nullptr, nullptr, W.attn, R, NORM_INNER_F64, B.strict,
                                   B.attn_norm, attn_eps, ep, nullptr, s, &nt);
            if (e != hipSuccess) return fail_hip("block attention inner norm + o projection", e);
        } else {
            // (only the int8 rows feed the O projection: the normalized fp64
            // rows are written back only for the tap)
            e = launch_norm_quant_f64(W.attn, R, B.q_dim, B.attn_norm, attn_eps, B.strict, nullptr,
                                      W.aq, ldqd, W.amax2, W.xsum2, s, T.attn_norm != nullptr,
                                      W.totals);
            if (e != hipSuccess) return fail_hip("block attention inner norm", e);
            TAP(tap_copy(T.attn_norm, W.attn, (size_t)R * B.q_dim * 8, s));
            TAP(tap_rows(T.aq, W.aq, ldqd, B.q_dim, R, s));
            TAP(tap_copy(T.aamax, W.amax2, (size_t)R * 4, s));
            QuantAct a{W.aq, ldqd, W.amax2, W.xsum2};
            e = launch_matmul(&B.o, nullptr, a, R, ep, s);
            if (e != hipSuccess) return fail_hip("block o projection", e);
        }
    }
    TAP(tap_copy(T.mid, x, (size_t)R * B.hidden * 4, s));
    // x := x + SwiGLU(RMSNorm2(x))
    {
        Epilogue ep;
        ep.kind = EPI_SWIGLU;
        ep.activation = B.activation;
        ep.out = W.h;
        ep.ldo = B.inter;
        if (fuse && norm_fused_ok(R, B.hidden, B.strict, true)) {
            NormTaps nt;
            nt.rows = T.y2;
            nt.xq = T.xq2;
            nt.amax = T.amax2;
            e = launch_matmul_norm(&B.gate, &B.up, x, nullptr, R, NORM_RMS, B.strict, B.norm2,
                                   rms_eps, ep, nullptr, s, &nt);
            if (e != hipSuccess) return fail_hip("block rmsnorm2 + gate/up", e);
        } else {
            e = launch_rmsnorm_quant(x, B.hidden, R, B.hidden, B.norm2, rms_eps, B.strict, T.y2,
                                     W.xq, ldh, W.amax, W.xsum, s, W.totals);
            if (e != hipSuccess) return fail_hip("block rmsnorm2", e);
            TAP(tap_rows(T.xq2, W.xq, ldh, B.hidden, R, s));
            TAP(tap_copy(T.amax2, W.amax, (size_t)R * 4, s));
            QuantAct a{W.xq, ldh, W.amax, W.xsum};
            e = launch_matmul(&B.gate, &B.up, a, R, ep, s);
            if (e != hipSuccess) return fail_hip("block gate/up", e);
        }
    }
    TAP(tap_copy(T.h, W.h, (size_t)R * B.inter * 4, s));
    {
        Epilogue ep;
        ep.kind = EPI_DENSE;
        ep.residual = x;
        ep.out = x;
        ep.ldo = B.hidden;
        if (fuse && norm_fused_ok(R, B.inter, B.strict, true)) {
            NormTaps nt;
            nt.rows = T.hn;
            nt.xq = T.hq;
            nt.amax = T.hamax;
            e = launch_matmul_norm(&B.down, nullptr, W.h, nullptr, R, NORM_INNER_F32, B.strict,
                                   B.ffn_norm, ffn_eps, ep, nullptr, s, &nt);
            if (e != hipSuccess) return fail_hip("block ffn inner norm + down", e);
        } else {
            // (only the int8 rows feed the down projection; the normalized
            // rows are written back only for the tap)
            e = launch_norm_quant(W.h, B.inter, R, B.inter, B.ffn_norm, ffn_eps, B.strict, W.hq, ldi,
                                  W.amax3, W.xsum3, s, T.hn != nullptr, W.totals);
            if (e != hipSuccess) return fail_hip("block ffn inner norm", e);
            TAP(tap_copy(T.hn, W.h, (size_t)R * B.inter * 4, s));
            TAP(tap_rows(T.hq, W.hq, ldi, B.inter, R, s));
            TAP(tap_copy(T.hamax, W.amax3, (size_t)R * 4, s));
            QuantAct a{W.hq, ldi, W.amax3, W.xsum3};
            e = launch_matmul(&B.down, nullptr, a, R, ep, s);
            if (e != hipSuccess) return fail_hip("block down", e);
        }
    }
#undef TAP
    return 0;
}

// Host-side position rule of mhaPrepareKVForForward: continue only for a
// single-token call on a warm cache.
static int next_base(int shadow, int seq) { return (seq == 1 && shadow > 0) ? shadow : 0; }

}  // namespace lamd

using namespace lamd;

struct loom_amd_block {
    BlockDev dev;
    Workspace ws;
    int* pos = nullptr;  // device
    int shadow = 0;      // host copy of the KV position
    int warm_batch = 0;  // sequences the warm cache holds (batch of the calls that filled it)
};

struct loom_amd_model {
    int device = 0;
    int layers_n = 0, vocab = 0, hidden = 0, max_tokens = 0, max_prefill = 0;
    double final_eps = 0.0;
    int strict = 1;
    int lm_sequential = 0;  // fp32 head in loom's scalar order (SIMD forward off)
    std::vector<BlockDev> layers;
    Workspace ws;
    float* embeddings = nullptr;
    float* lm_head = nullptr;     // fp32 head: == embeddings when tied
    loom_amd_matrix* lm_ternary = nullptr;  // untied head of a ternary model (loom packs it)
    float* final_norm = nullptr;  // null: no final norm
    float* x = nullptr;           // max_batch*max_prefill x hidden
    float* fin = nullptr;         // max_batch x hidden
    float* logits = nullptr;      // max_batch x vocab
    int* tokens = nullptr;        // max_batch x max_tokens
    float2* argmax_part = nullptr;  // max_batch x kArgmaxMaxParts
    // screened greedy head (fp32 table, one row): int8 codes and per-row
    // scales of the table, each row's upper bound, the threshold key and
    // per-workgroup picks
    int8_t* lm_q = nullptr;       // vocab x hidden
    float* lm_qscale = nullptr;   // vocab
    double* screen_hi = nullptr;  // vocab
    unsigned long long* screen_key = nullptr;
    float2* screen_part = nullptr;  // lm_screen_parts(vocab)
    bool head_screened = false;   // the last head left only the candidates' logits
    int* pos = nullptr;           // device position shared by every layer
    void* misc = nullptr;
    // Pinned staging for the ids that cross the boundary (prompt upload,
    // token read-back): copies from pageable memory need not have finished
    // when the call that queued them returns.  ids_sent marks the last upload
    // out of it, so neither the next upload nor a read-back overwrites it early.
    int32_t* host_ids = nullptr;  // max_batch x max_tokens
    hipEvent_t ids_sent = nullptr;
    int batch = 0;                // batch of the current sequences
    int shadow = 0;               // host copy of the position
    hipStream_t own = nullptr;
    hipGraphExec_t graph = nullptr;
    int graph_batch = 0;
};

extern "C" {

int loom_amd_block_create(int device, const loom_amd_block_desc* desc,
                          const loom_amd_block_weights* w, loom_amd_block** out) {
    if (!out) return fail("out is null");
    *out = nullptr;
    auto* b = new loom_amd_block();
    if (build_block(device, desc, w, &b->dev)) {
        delete b;
        return -1;
    }
    DeviceGuard guard(device);
    hipError_t e = hipMalloc(&b->pos, sizeof(int));
    if (e == hipSuccess) e = hipMemset(b->pos, 0, sizeof(int));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_block(&b->dev);
        if (b->pos) (void)hipFree(b->pos);
        delete b;
        return fail_hip("block position", e);
    }
    *out = b;
    return 0;
}

void loom_amd_block_release(loom_amd_block* b) {
    if (!b) return;
    DeviceGuard guard(b->dev.device);
    (void)hipDeviceSynchronize();
    free_workspace(&b->ws);
    free_block(&b->dev);
    if (b->pos) (void)hipFree(b->pos);
    delete b;
}

int loom_amd_block_forward(loom_amd_block* b, float* x, int batch, int seq,
                           const loom_amd_block_taps* taps, void* stream) {
    if (!b) return fail("block is null");
    if (!x) return fail("x is null");
    if (batch <= 0 || seq <= 0) return fail("batch and seq must be positive");
    const BlockDev& B = b->dev;
    if (batch > B.max_batch) {
        return fail("batch " + std::to_string(batch) + " > max_batch " + std::to_string(B.max_batch));
    }
    const int base = next_base(b->shadow, seq);
    if (base > 0 && batch != b->warm_batch) {
        // each sequence owns a ring: a single-token call with another batch
        // would read slots the warm cache never filled
        return fail("single-token call of batch " + std::to_string(batch) +
                    " on a warm cache of batch " + std::to_string(b->warm_batch) +
                    ": continue with the same batch or restart with a longer call");
    }
    if (base + seq > B.span()) {
        return fail("positions " + std::to_string(base) + ".." + std::to_string(base + seq - 1) +
                    " pass max_seq_len " + std::to_string(B.msl));
    }
    DeviceGuard guard(B.device);
    hipStream_t s = (hipStream_t)stream;
    const int rows = batch * seq;
    if (b->ws.rows < rows) {
        hipError_t e = hipDeviceSynchronize();  // queued calls may still use the old workspace
        if (e != hipSuccess) return fail_hip("block workspace", e);
        free_workspace(&b->ws);
        if (alloc_workspace(B, rows, &b->ws)) return -1;
    }
    hipError_t e = hipSuccess;
    if (base == 0) e = launch_set_int(b->pos, 0, s);
    if (e != hipSuccess) return fail_hip("block position", e);
    if (block_forward_dev(B, b->ws, x, batch, seq, b->pos, taps, s)) return -1;
    e = launch_add_int(b->pos, seq, s);
    if (e != hipSuccess) return fail_hip("block position", e);
    b->shadow = base + seq;
    b->warm_batch = batch;
    return 0;
}

int loom_amd_block_kv_offset(const loom_amd_block* b) { return b ? b->shadow : -1; }

int loom_amd_block_kv_cache(const loom_amd_block* b, int slot, const float** k, const float** v) {
    if (!b) return fail("block is null");
    if (slot < 0 || slot >= b->dev.max_batch) return fail("slot out of range");
    if (k) *k = b->dev.cache_k + (size_t)slot * b->dev.cache_slot();
    if (v) *v = b->dev.cache_v + (size_t)slot * b->dev.cache_slot();
    return 0;
}

int loom_amd_lm_head(const float* table, int vocab, int hidden, const float* x, int rows,
                     float* logits, void* stream) {
    if (!table || !x || !logits) return fail("null buffer");
    if (vocab <= 0 || hidden <= 0 || rows < 0) return fail("bad shape");
    if ((size_t)hidden * 4 > 64 * 1024) return fail("hidden is limited to 16384");
    if (rows == 0) return 0;
    hipError_t e = launch_lm_head(table, vocab, hidden, x, rows, logits, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("lm_head", e);
}

int loom_amd_lm_head_sequential(const float* table, int vocab, int hidden, const float* x,
                                int rows, float* logits, void* stream) {
    if (!table || !x || !logits) return fail("null buffer");
    if (vocab <= 0 || hidden <= 0 || rows < 0) return fail("bad shape");
    if ((size_t)hidden * 4 > 64 * 1024) return fail("hidden is limited to 16384");
    if (rows == 0) return 0;
    hipError_t e = launch_lm_head_seq(table, vocab, hidden, x, rows, logits, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("lm_head_sequential", e);
}

int loom_amd_greedy_sample(const float* logits, int n, int rows, int32_t* ids, void* stream) {
    if (!logits || !ids) return fail("null buffer");
    if (n <= 0 || rows < 0) return fail("bad shape");
    if (rows == 0) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail("no current device");
    std::string err;
    void* part = scratch(dev, (size_t)rows * kArgmaxMaxParts * sizeof(float2), &err);
    if (!part) return fail(err);
    hipError_t e = launch_argmax(logits, n, rows, (float2*)part, ids, 1, nullptr, 0, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("greedy_sample", e);
}

// ---- model -----------------------------------------------------------------

static void free_model(loom_amd_model* m) {
    DeviceGuard guard(m->device);
    (void)hipDeviceSynchronize();
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    for (auto& L : m->layers) free_block(&L);
    free_workspace(&m->ws);
    if (m->misc) (void)hipFree(m->misc);
    if (m->host_ids) (void)hipHostFree(m->host_ids);
    if (m->ids_sent) (void)hipEventDestroy(m->ids_sent);
    if (m->own) (void)hipStreamDestroy(m->own);
    if (m->lm_ternary) loom_amd_matrix_release(m->lm_ternary);
    delete m;
}

int loom_amd_model_create(int device, const loom_amd_model_desc* desc,
                          const loom_amd_block_weights* layers, const float* embeddings,
                          const float* final_norm, const float* lm_head, loom_amd_model** out) {
    if (!out) return fail("out is null");
    *out = nullptr;
    if (!desc) return fail("model desc is null");
    if (desc->num_layers < 0 || desc->vocab <= 0) return fail("model desc: bad layer count or vocab");
    if (desc->num_layers > 0 && !layers) return fail("layers are null");
    if (desc->lm_head_order != LOOM_AMD_LM_DOTTILE && desc->lm_head_order != LOOM_AMD_LM_SEQUENTIAL)
        return fail("model desc: lm_head_order must be LOOM_AMD_LM_DOTTILE or LOOM_AMD_LM_SEQUENTIAL");
    if (!embeddings) return fail("embeddings are null");
    if (check_desc(&desc->block)) return -1;
    const loom_amd_block_desc& bd = desc->block;
    const int msl = bd.max_seq_len > 0 ? bd.max_seq_len : 512;
    const int max_tokens = desc->max_tokens > 0 ? desc->max_tokens : msl + 1;
    const int max_prefill = desc->max_prefill > 0 ? desc->max_prefill : (max_tokens < msl ? max_tokens : msl);
    const int max_batch = bd.max_batch > 0 ? bd.max_batch : 1;
    const int H = bd.hidden;
    if ((size_t)H * 4 > 64 * 1024) return fail("model: hidden is limited to 16384 for the LM head");
    auto* m = new loom_amd_model();
    m->device = device;
    m->layers_n = desc->num_layers;
    m->vocab = desc->vocab;
    m->hidden = H;
    m->max_tokens = max_tokens;
    m->max_prefill = max_prefill;
    m->final_eps = desc->final_norm_eps;
    m->strict = bd.norm_mode == LOOM_AMD_NORM_STRICT;
    m->lm_sequential = desc->lm_head_order == LOOM_AMD_LM_SEQUENTIAL;
    m->layers.resize(desc->num_layers);
    for (int i = 0; i < desc->num_layers; ++i) {
        if (build_block(device, &bd, &layers[i], &m->layers[i])) {
            const std::string msg = "layer " + std::to_string(i) + ": " + g_amd_error;
            free_model(m);
            return fail(msg);
        }
    }
    DeviceGuard guard(device);
    Layout L;
    const size_t o_emb = L.take((size_t)desc->vocab * H * 4);
    // usePackedTernaryLMHead (poly/transformer.go:721-734): an untied head of
    // a model with ternary layers is packed and applied as a ternary matvec
    const bool ternary_head = lm_head && desc->num_layers > 0;
    const bool fp32_head = lm_head && !ternary_head;
    const size_t o_lm = L.take(fp32_head ? (size_t)desc->vocab * H * 4 : 0);
    const size_t o_fn = L.take(final_norm ? (size_t)H * 4 : 0);
    const size_t o_x = L.take((size_t)max_batch * max_prefill * H * 4);
    const size_t o_fin = L.take((size_t)max_batch * H * 4);
    const size_t o_lg = L.take((size_t)max_batch * desc->vocab * 4);
    const size_t o_tok = L.take((size_t)max_batch * max_tokens * 4);
    const size_t o_part = L.take((size_t)max_batch * kArgmaxMaxParts * sizeof(float2));
    // ternary_head: the packed matrix replaces the fp32 head
    const bool screen = !ternary_head && lm_screen_ok(H);
    const size_t o_hb = L.take(screen ? lm_screen_code_bytes(desc->vocab, H) : 0);
    const size_t o_qs = L.take(screen ? (size_t)desc->vocab * 4 : 0);
    const size_t o_hi = L.take(screen ? (size_t)desc->vocab * 8 : 0);
    const size_t o_key = L.take(screen ? 8 : 0);
    const size_t o_sp = L.take(screen ? (size_t)lm_screen_parts(desc->vocab) * sizeof(float2) : 0);
    const size_t o_pos = L.take(4);
    hipError_t e = hipMalloc(&m->misc, L.off);
    if (e != hipSuccess) {
        free_model(m);
        return fail_hip("model buffers", e);
    }
    char* base = (char*)m->misc;
    m->embeddings = (float*)(base + o_emb);
    m->lm_head = fp32_head ? (float*)(base + o_lm) : m->embeddings;
    m->final_norm = final_norm ? (float*)(base + o_fn) : nullptr;
    m->x = (float*)(base + o_x);
    m->fin = (float*)(base + o_fin);
    m->logits = (float*)(base + o_lg);
    m->tokens = (int*)(base + o_tok);
    m->argmax_part = (float2*)(base + o_part);
    if (screen) {
        m->lm_q = (int8_t*)(base + o_hb);
        m->lm_qscale = (float*)(base + o_qs);
        m->screen_hi = (double*)(base + o_hi);
        m->screen_key = (unsigned long long*)(base + o_key);
        m->screen_part = (float2*)(base + o_sp);
    }
    m->pos = (int*)(base + o_pos);
    e = hipMemcpy(m->embeddings, embeddings, (size_t)desc->vocab * H * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess && fp32_head) {
        e = hipMemcpy(m->lm_head, lm_head, (size_t)desc->vocab * H * 4, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess && final_norm) {
        e = hipMemcpy(m->final_norm, final_norm, (size_t)H * 4, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) e = hipMemset(m->tokens, 0, (size_t)max_batch * max_tokens * 4);
    if (e == hipSuccess) e = hipMemset(m->pos, 0, sizeof(int));
    if (e == hipSuccess && screen) e = hipMemset(m->screen_key, 0, 8);
    if (e == hipSuccess && screen) e = hipMemset(m->lm_q, 0, lm_screen_code_bytes(desc->vocab, H));  // block padding
    if (e == hipSuccess && screen) e = launch_lm_quant_rows(m->lm_head, desc->vocab, H, m->lm_q, m->lm_qscale, nullptr);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&m->own, hipStreamNonBlocking);
    if (e == hipSuccess) {
        e = hipHostMalloc((void**)&m->host_ids, (size_t)max_batch * max_tokens * 4,
                          hipHostMallocDefault);
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&m->ids_sent, hipEventDisableTiming);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_model(m);
        return fail_hip("model upload", e);
    }
    if (ternary_head &&
        loom_amd_matrix_from_float32(device, lm_head, desc->vocab, H, &m->lm_ternary, nullptr)) {
        const std::string msg = "model LM head: " + g_amd_error;
        free_model(m);
        return fail(msg);
    }
    if (desc->num_layers > 0 && alloc_workspace(m->layers[0], max_batch * max_prefill, &m->ws)) {
        free_model(m);
        return -1;
    }
    *out = m;
    return 0;
}

void loom_amd_model_release(loom_amd_model* m) {
    if (m) free_model(m);
}

// Final norm + LM head + argmax of each sequence's last row (row stride ld
// floats between sequences), writing the token at *pos + offset.
static int model_head(loom_amd_model* m, const float* last, long ld, int batch, int offset,
                      hipStream_t s) {
    hipError_t e;
    const float* h = last;
    if (m->final_norm) {
        e = launch_rmsnorm_quant(last, ld, batch, m->hidden, m->final_norm, m->final_eps, m->strict,
                                 m->fin, nullptr, 0, nullptr, nullptr, s);
        if (e != hipSuccess) return fail_hip("model final norm", e);
    } else {
        e = hipSuccess;
        for (int b = 0; b < batch && e == hipSuccess; ++b) {
            e = hipMemcpyAsync(m->fin + (size_t)b * m->hidden, last + (size_t)b * ld,
                               (size_t)m->hidden * 4, hipMemcpyDeviceToDevice, s);
        }
        if (e != hipSuccess) return fail_hip("model last rows", e);
    }
    h = m->fin;
    if (m->lm_ternary) {
        // applyPackedTernaryLMHead (poly/transformer.go:736-755): per-row int8
        // quantization, ternary matvec, logits = fp32(fp64 result)
        Epilogue epi;
        epi.kind = EPI_DENSE;
        epi.out = m->logits;
        epi.ldo = m->vocab;
        const Matrix& W = m->lm_ternary->m;
        if (fused_quant_ok(batch, m->hidden, h)) {
            e = launch_matmul_fused(&W, nullptr, h, batch, epi, nullptr, nullptr, s);
        } else {
            const Workspace& ws = m->ws;
            const int ldq = pad_cols(m->hidden);
            e = launch_act_quant(h, m->hidden, batch, m->hidden, ws.xq, ldq, ws.amax, ws.xsum, s);
            if (e == hipSuccess) {
                QuantAct a{ws.xq, ldq, ws.amax, ws.xsum};
                e = launch_matmul(&W, nullptr, a, batch, epi, s);
            }
        }
        if (e != hipSuccess) return fail_hip("model ternary lm head", e);
    } else if (m->lm_q && tune_int("LOOM_AMD_LM_SCREEN", 1) != 0) {
        // greedy pick from an int8 screening pass and the candidates' exact
        // logits, one row after the other (the bounds and the threshold are
        // per row; every call leaves the threshold cleared)
        for (int b = 0; b < batch; ++b) {
            e = launch_lm_greedy_screened(m->lm_head, m->lm_q, m->lm_qscale, m->vocab, m->hidden,
                                          h + (size_t)b * m->hidden, m->lm_sequential, m->screen_hi,
                                          m->screen_key, m->logits + (size_t)b * m->vocab, m->screen_part,
                                          m->tokens + (size_t)b * m->max_tokens, m->max_tokens, m->pos, offset, s);
            if (e != hipSuccess) return fail_hip("model screened lm head", e);
        }
        m->head_screened = true;
        return 0;
    } else {
        e = m->lm_sequential
                ? launch_lm_head_seq(m->lm_head, m->vocab, m->hidden, h, batch, m->logits, s)
                : launch_lm_head(m->lm_head, m->vocab, m->hidden, h, batch, m->logits, s);
        if (e != hipSuccess) return fail_hip("model lm head", e);
    }
    m->head_screened = false;
    e = launch_argmax(m->logits, m->vocab, batch, m->argmax_part, m->tokens, m->max_tokens, m->pos,
                      offset, s);
    if (e != hipSuccess) return fail_hip("model argmax", e);
    return 0;
}

// every logit of the last head call (the screened head leaves only its
// candidates' logits): the full fp32 head over the final rows still in fin
static hipError_t model_full_logits(loom_amd_model* m, int batch, hipStream_t s) {
    if (!m->head_screened) return hipSuccess;
    return m->lm_sequential ? launch_lm_head_seq(m->lm_head, m->vocab, m->hidden, m->fin, batch, m->logits, s)
                            : launch_lm_head(m->lm_head, m->vocab, m->hidden, m->fin, batch, m->logits, s);
}

int loom_amd_model_prefill(loom_amd_model* m, const int32_t* ids, int batch, int n,
                           float* logits, void* stream) {
    if (!m) return fail("model is null");
    if (!ids) return fail("ids are null");
    const int max_batch = m->layers_n > 0 ? m->layers[0].max_batch : 1;
    if (batch <= 0 || batch > max_batch) return fail("batch out of range (max_batch " + std::to_string(max_batch) + ")");
    if (n <= 0 || n > m->max_prefill) return fail("prompt length out of range (max_prefill " + std::to_string(m->max_prefill) + ")");
    if (n >= m->max_tokens) return fail("prompt leaves no room for a generated token (max_tokens)");
    if (m->layers_n > 0 && n > m->layers[0].span()) return fail("prompt longer than max_seq_len");
    DeviceGuard guard(m->device);
    hipStream_t s = (hipStream_t)stream;
    // the previous upload out of host_ids must have left it before it is refilled
    hipError_t e = hipEventSynchronize(m->ids_sent);
    if (e == hipSuccess) {
        memcpy(m->host_ids, ids, (size_t)batch * n * 4);
        e = launch_set_int(m->pos, 0, s);
    }
    if (e == hipSuccess) {
        e = hipMemcpy2DAsync(m->tokens, (size_t)m->max_tokens * 4, m->host_ids, (size_t)n * 4,
                             (size_t)n * 4, batch, hipMemcpyHostToDevice, s);
    }
    if (e == hipSuccess) e = hipEventRecord(m->ids_sent, s);
    if (e == hipSuccess) {
        e = launch_embed(m->embeddings, m->vocab, m->hidden, m->tokens, m->max_tokens, m->pos, batch,
                         n, m->x, s);
    }
    if (e != hipSuccess) return fail_hip("model prefill", e);
    for (int i = 0; i < m->layers_n; ++i) {
        if (block_forward_dev(m->layers[i], m->ws, m->x, batch, n, m->pos, nullptr, s)) {
            return fail("layer " + std::to_string(i) + ": " + g_amd_error);
        }
    }
    if (model_head(m, m->x + (size_t)(n - 1) * m->hidden, (long)n * m->hidden, batch, n, s)) return -1;
    e = launch_add_int(m->pos, n, s);
    if (e == hipSuccess && logits) e = model_full_logits(m, batch, s);
    if (e == hipSuccess && logits) {
        e = hipMemcpyAsync(logits, m->logits, (size_t)batch * m->vocab * 4, hipMemcpyDeviceToDevice, s);
    }
    if (e != hipSuccess) return fail_hip("model prefill", e);
    m->batch = batch;
    m->shadow = n;
    return 0;
}

// One decode step on stream s (graph-capturable: kernels only).
static int decode_step(loom_amd_model* m, hipStream_t s) {
    const int batch = m->batch;
    hipError_t e = launch_embed(m->embeddings, m->vocab, m->hidden, m->tokens, m->max_tokens, m->pos,
                                batch, 1, m->x, s);
    if (e != hipSuccess) return fail_hip("model embed", e);
    for (int i = 0; i < m->layers_n; ++i) {
        if (block_forward_dev(m->layers[i], m->ws, m->x, batch, 1, m->pos, nullptr, s)) {
            return fail("layer " + std::to_string(i) + ": " + g_amd_error);
        }
    }
    if (model_head(m, m->x, m->hidden, batch, 1, s)) return -1;
    e = launch_add_int(m->pos, 1, s);
    if (e != hipSuccess) return fail_hip("model position", e);
    return 0;
}

int loom_amd_model_decode(loom_amd_model* m, int steps, int use_graph, float* logits,
                          void* stream) {
    if (!m) return fail("model is null");
    if (steps < 0) return fail("steps must be >= 0");
    if (m->batch <= 0 || m->shadow <= 0) return fail("decode needs a prefill first");
    const int limit_seq = m->layers_n > 0 ? m->layers[0].span() : m->max_tokens;
    if (m->shadow + steps > limit_seq || m->shadow + steps >= m->max_tokens) {
        return fail("decode would pass max_seq_len or max_tokens");
    }
    if (steps == 0) return 0;
    DeviceGuard guard(m->device);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    if (use_graph) {
        // captured on the model's own (idle) stream, replayed on the caller's
        // stream: the step graphs stay in one queue with the caller's work
        hipStream_t cs = m->own;
        if (!m->graph || m->graph_batch != m->batch) {
            if (m->graph) {
                (void)hipGraphExecDestroy(m->graph);
                m->graph = nullptr;
            }
            hipGraph_t g = nullptr;
            e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
            if (e != hipSuccess) return fail_hip("model decode capture", e);
            const int rc = decode_step(m, cs);
            hipError_t ec = hipStreamEndCapture(cs, &g);
            if (rc || ec != hipSuccess) {
                if (g) (void)hipGraphDestroy(g);
                return rc ? -1 : fail_hip("model decode capture", ec);
            }
            e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e != hipSuccess) {
                m->graph = nullptr;
                return fail_hip("model decode instantiate", e);
            }
            m->graph_batch = m->batch;
        }
        for (int i = 0; i < steps && e == hipSuccess; ++i) e = hipGraphLaunch(m->graph, s);
        if (e != hipSuccess) return fail_hip("model decode replay", e);
    } else {
        for (int i = 0; i < steps; ++i) {
            if (decode_step(m, s)) return -1;
        }
    }
    if (logits) {
        e = model_full_logits(m, m->batch, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(logits, m->logits, (size_t)m->batch * m->vocab * 4, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return fail_hip("model logits", e);
    }
    m->shadow += steps;
    return 0;
}

int loom_amd_model_tokens(const loom_amd_model* m, int32_t* out, int count, void* stream) {
    if (!m) return fail("model is null");
    if (!out) return fail("out is null");
    if (count <= 0 || count > m->max_tokens) return fail("count out of range");
    DeviceGuard guard(m->device);
    hipStream_t s = (hipStream_t)stream;
    const int rows = m->batch > 0 ? m->batch : 1;
    // through the pinned buffer: the copy has landed once the stream is idle
    hipError_t e = hipEventSynchronize(m->ids_sent);
    if (e == hipSuccess) {
        e = hipMemcpy2DAsync(m->host_ids, (size_t)count * 4, m->tokens, (size_t)m->max_tokens * 4,
                             (size_t)count * 4, rows, hipMemcpyDeviceToHost, s);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail_hip("model tokens", e);
    memcpy(out, m->host_ids, (size_t)rows * count * 4);
    return 0;
}

int loom_amd_model_position(const loom_amd_model* m) { return m ? m->shadow : -1; }

const float* loom_amd_model_last_hidden(const loom_amd_model* m) { return m ? m->fin : nullptr; }

}  // extern "C"
