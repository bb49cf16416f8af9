"""BASELINE configs 3 and 4 at their real sizes, against the CPU oracle.

Config 3 (poly/transformer.go:434-485 Generate, poly/mha.go:316-354
attention over the whole cache, poly/transformer.go:664-719 LM head): a
BitNet-2B block after a 2048-token prompt, single-token steps checked stage
by stage over a 2048+ position cache, and models with vocab 128256 (two
layers after a 2048-token prompt; all 30 layers after a 64-token prompt) whose
graph-replayed decode steps give the oracle's logits (both of loom's LM-head
orders) and argmax tokens, their hidden rows equal to the same blocks chained
stage-checked.

Config 4 (batch 8 x 2048, M = 16384 rows per ternary GEMM): the GEMM's int32
accumulators and fp32 outputs at M = 16384 on both FFN shapes, and one
BitNet-2B block over 8 sequences of 2048 tokens with two sequences checked
stage by stage (loom's batch semantics restated per sequence: each sequence
equals a batch-1 run, poly/mha.go:256-258).

Bars: those of tests/stages.py.  Rows past the Q/K/V projection are checked on
a sample that covers every 64-row tile boundary class (first, last, the rows
around 32/64/512/1024/2048-row borders); the K/V caches and Q are checked on
every row.  Citations are relative to the loom v0.83.0 tree.
"""
import numpy as np
import pytest

from tests.stages import (ACT_SILU, Shape, Weights, check_stages, run_block_case, to_dev)

pytestmark = pytest.mark.gpu

PROMPT = 2048
CONFIG3 = Shape(2560, 20, 5, 128, 6912, PROMPT + 16)
VOCAB = 128256


def sample_rows(seq):
    base = [0, 1, 2, 15, 16, 31, 32, 33, 63, 64, 65, 127, 128, 255, 256, 511, 512, 513, 777,
            1023, 1024, 1025, 1500, 1983, 2015, 2016, 2017, 2046, 2047]
    return sorted({r for r in base if r < seq} | {seq - 1})


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from loom_amd import _lib
    assert _lib.lib().loom_amd_device_count() >= 1, "no gfx950 device visible to the library"
    return torch


@pytest.fixture(scope="module")
def tf(torch_dev):
    from loom_amd import transformer
    return transformer


# ---------------------------------------------------------------- config 3
@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_config3_block_prefill_2048_then_decode(orc, torch_dev, tf, norm):
    # One BitNet-2B block: a 2048-token prefill (sampled rows past the
    # projection), then 10 single-token steps over the 2048+ position cache:
    # fast mode's GQA chunk attention + combine over 65 chunks, strict mode's
    # ordered value chains; every step checked stage by stage.
    w = Weights(orc, CONFIG3, seed=3001, act=ACT_SILU, bias=True)
    run_block_case(orc, torch_dev, tf, w, [PROMPT] + [1] * 10, seed=3100,
                   strict=norm == "strict", rows_for=lambda seq: sample_rows(seq) if seq > 1 else None)


class _Model:
    def __init__(self, orc, layers, seed):
        self.layers = [Weights(orc, CONFIG3, seed + 100 * i, act=ACT_SILU) for i in range(layers)]
        # (numpy's generator: the oracle's Box-Muller takes ~30 s for 328 M values)
        rng = np.random.default_rng(seed + 7)
        self.emb = rng.standard_normal(VOCAB * CONFIG3.hidden, dtype=np.float32) * np.float32(0.02)
        self.fn = orc.uniform_f32(CONFIG3.hidden, 0.5, 1.5, seed + 8)

    def gpu(self, tf, norm, simd_forward=True):
        cfg = self.layers[0].cfg(tf, norm=norm)
        return tf.Transformer(cfg, [w.gpu(tf) for w in self.layers], self.emb, self.fn, vocab=VOCAB,
                              final_norm_eps=1e-6, max_tokens=PROMPT + 12, max_prefill=PROMPT,
                              simd_forward=simd_forward)


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_config3_model_graph_decode(orc, torch_dev, tf, norm):
    # Two BitNet-2B layers, vocab 128256 (tied fp32 head, DotTile order),
    # a 2048-token prompt, then 8 graph-replayed decode steps.  Each step's
    # logits equal the oracle's LM head of the model's final hidden row and
    # the token its argmax; the hidden rows equal the same two blocks chained
    # (fed the embeddings of the prompt and of each generated token), every
    # block call checked stage by stage, then the oracle's final RMSNorm.
    torch = torch_dev
    M = _Model(orc, 2, seed=3201)
    model = M.gpu(tf, norm)
    rng = np.random.default_rng(32)
    prompt = rng.integers(0, VOCAB, PROMPT).astype(np.int32)
    table = M.emb.reshape(VOCAB, CONFIG3.hidden)
    logits = model.prefill(prompt, logits=True).cpu().numpy()[0]
    hid = model.last_hidden().cpu().numpy()[0]
    assert logits.tobytes() == orc.lm_head(hid, M.emb, simd=True).tobytes()
    assert model.tokens()[0, PROMPT] == orc.argmax_first(logits)
    hids = [hid]
    for step in range(8):
        lg = model.decode(1, use_graph=True, logits=True).cpu().numpy()[0]
        h = model.last_hidden().cpu().numpy()[0]
        assert lg.tobytes() == orc.lm_head(h, M.emb, simd=True).tobytes(), f"step {step} logits"
        assert model.tokens()[0, PROMPT + 1 + step] == orc.argmax_first(lg), f"step {step} token"
        hids.append(h)
    toks = model.tokens()[0]
    assert np.array_equal(toks[:PROMPT], prompt)
    model.release()
    # the same blocks chained, stage-checked, give the model's hidden rows
    strict = norm == "strict"
    blocks = [tf.BitNetBlock(w.cfg(tf, norm), w.gpu(tf)) for w in M.layers]
    refs = [w.oracle_mha(orc) for w in M.layers]
    x = table[toks[:PROMPT]].copy()
    base = 0
    for call in range(9):
        for li, (blk, w) in enumerate(zip(blocks, M.layers)):
            xd = to_dev(torch, x)
            _, t = blk.forward(xd, taps=True)
            torch.cuda.synchronize()
            out = xd.cpu().numpy()
            ck, cv = (a.cpu().numpy() for a in blk.kv_cache(0))
            print(f"  chain call {call} layer {li}: rows={x.shape[0]} base={base}", flush=True)
            check_stages(orc, w, refs[li], x, t.numpy(), out, ck, cv, base, strict,
                         sample_rows(x.shape[0]) if x.shape[0] > 1 else None)
            x = out
        fin = orc.rmsnorm_forward(x[-1:], M.fn, 1e-6)[0]
        assert fin.tobytes() == hids[call].tobytes(), f"final hidden of call {call}"
        base += x.shape[0]
        x = table[toks[PROMPT + call]][None].copy()
    for b in blocks:
        b.release()


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_config3_model_30_layers(orc, torch_dev, tf, norm):
    # config 3's full depth: 30 BitNet-2B layers, vocab 128256 (tied fp32
    # head), a 64-token prompt and 8 graph-replayed decode steps.  Each step's
    # logits equal the oracle's LM head of the model's final hidden row and
    # its token their argmax; the final hidden rows equal the same 30 blocks
    # chained (prompt and generated tokens fed in), every block call checked
    # stage by stage, then the oracle's final RMSNorm.
    torch = torch_dev
    L, P = 30, 64
    shape = Shape(2560, 20, 5, 128, 6912, P + 16)
    layers = [Weights(orc, shape, 3501 + 100 * i, act=ACT_SILU) for i in range(L)]
    rng = np.random.default_rng(3507)
    emb = rng.standard_normal(VOCAB * shape.hidden, dtype=np.float32) * np.float32(0.02)
    fn = orc.uniform_f32(shape.hidden, 0.5, 1.5, 3508)
    table = emb.reshape(VOCAB, shape.hidden)
    model = tf.Transformer(layers[0].cfg(tf, norm=norm), [w.gpu(tf) for w in layers], emb, fn,
                           vocab=VOCAB, final_norm_eps=1e-6, max_tokens=P + 12, max_prefill=P)
    prompt = rng.integers(0, VOCAB, P).astype(np.int32)
    lg = model.prefill(prompt, logits=True).cpu().numpy()[0]
    hids = [model.last_hidden().cpu().numpy()[0]]
    assert lg.tobytes() == orc.lm_head(hids[0], emb, simd=True).tobytes()
    assert model.tokens()[0, P] == orc.argmax_first(lg)
    for step in range(8):
        lg = model.decode(1, use_graph=True, logits=True).cpu().numpy()[0]
        h = model.last_hidden().cpu().numpy()[0]
        assert lg.tobytes() == orc.lm_head(h, emb, simd=True).tobytes(), f"step {step} logits"
        assert model.tokens()[0, P + 1 + step] == orc.argmax_first(lg), f"step {step} token"
        hids.append(h)
    toks = model.tokens()[0]
    model.release()
    blocks = [tf.BitNetBlock(w.cfg(tf, norm), w.gpu(tf)) for w in layers]
    refs = [w.oracle_mha(orc) for w in layers]
    x = table[toks[:P]].copy()
    base = 0
    for call in range(9):
        print(f"  chain call {call}: rows={x.shape[0]} base={base}", flush=True)
        for li, (blk, w) in enumerate(zip(blocks, layers)):
            xd = to_dev(torch, x)
            _, t = blk.forward(xd, taps=True)
            torch.cuda.synchronize()
            out = xd.cpu().numpy()
            ck, cv = (a.cpu().numpy() for a in blk.kv_cache(0))
            check_stages(orc, w, refs[li], x, t.numpy(), out, ck, cv, base, norm == "strict")
            x = out
        fin = orc.rmsnorm_forward(x[-1:], fn, 1e-6)[0]
        assert fin.tobytes() == hids[call].tobytes(), f"final hidden of call {call}"
        base += x.shape[0]
        x = table[toks[P + call]][None].copy()
    for b in blocks:
        b.release()


def test_config3_model_sequential_lm_head(orc, torch_dev, tf):
    # Network.UseSimdForward off (poly/transformer.go:681-687): the tied head
    # sums each of the 128256 logits in order, in prefill and in the captured
    # decode step; one BitNet-2B layer, a 2048-token prompt, 8 steps.
    M = _Model(orc, 1, seed=3301)
    model = M.gpu(tf, "fast", simd_forward=False)
    rng = np.random.default_rng(33)
    prompt = rng.integers(0, VOCAB, PROMPT).astype(np.int32)
    lg = model.prefill(prompt, logits=True).cpu().numpy()[0]
    h = model.last_hidden().cpu().numpy()[0]
    assert lg.tobytes() == orc.lm_head(h, M.emb, simd=False).tobytes()
    for step in range(8):
        lg = model.decode(1, use_graph=True, logits=True).cpu().numpy()[0]
        h = model.last_hidden().cpu().numpy()[0]
        assert lg.tobytes() == orc.lm_head(h, M.emb, simd=False).tobytes(), f"step {step}"
        assert model.tokens()[0, PROMPT + 1 + step] == orc.argmax_first(lg)
    model.release()


def test_config3_lm_head_full_vocab_both_orders(orc, torch_dev, tf):
    # the LM head kernels at vocab 128256 x 2560 on several rows: DotTile and
    # sequential orders bit-exact, greedy pick = oracle argmax
    torch = torch_dev
    table = np.random.default_rng(3401).standard_normal(VOCAB * 2560, dtype=np.float32) * np.float32(0.02)
    rows = np.stack([orc.normal_f32(2560, 3402 + r) for r in range(3)])
    dt, dx = to_dev(torch, table.reshape(VOCAB, 2560)), to_dev(torch, rows)
    got = tf.lm_head(dt, dx).cpu().numpy()
    seq = tf.lm_head_sequential(dt, dx).cpu().numpy()
    ids = tf.greedy_sample(to_dev(torch, got)).cpu().numpy()
    for r in range(3):
        want = orc.lm_head(rows[r], table, simd=True)
        assert got[r].tobytes() == want.tobytes()
        assert seq[r].tobytes() == orc.lm_head(rows[r], table, simd=False).tobytes()
        assert ids[r] == orc.argmax_first(want)


# ---------------------------------------------------------------- config 4
@pytest.mark.parametrize("shape", ["up", "down"])
def test_config4_gemm_m16384(orc, torch_dev, shape):
    # M = 16384 rows (config 4's rows per ternary GEMM): int32 accumulators of
    # every row and column against an exact integer product (fp32 matmul of
    # integers: every partial sum is an integer below 2^24, so each fp32
    # operation is exact in any order), and the fp32 outputs of sampled rows
    # against the oracle's Dense forward bit for bit.
    from loom_amd import bitnet as bn
    torch = torch_dev
    n, k = (6912, 2560) if shape == "up" else (2560, 6912)
    M = 16384
    assert 127 * k < 2 ** 24
    m = orc.random_matrix(n, k, seed=4001 if shape == "up" else 4002)
    x = np.random.default_rng(4010).standard_normal((M, k), dtype=np.float32)
    w = bn.TernaryMatrix.from_words(m.words, n, k, m.scale)
    xd = to_dev(torch, x)
    q = bn.quantize_activation(xd)
    out, acc = bn.ternary_matvec_quantized(w, q, want_acc=True)
    torch.cuda.synchronize()
    xq = q.unpadded().cpu().numpy()
    rows = sample_rows(M) + [4095, 4096, 8191, 8192, 12287, 12288, 16320, 16383]
    xq_ref, am_ref = orc.quant_rows(x[rows])
    assert np.array_equal(xq[rows], xq_ref) and q.amax.cpu().numpy()[rows].tobytes() == am_ref.tobytes()
    # the decoded ternary weights (codes 0/1/2 -> -1/0/+1) as fp32
    codes = m.ensure_codes().reshape(n, -1)[:, :k].astype(np.float32) - 1.0
    acc_np = acc.cpu().numpy()
    for r0 in range(0, M, 2048):
        want = xq[r0:r0 + 2048].astype(np.float32) @ codes.T
        assert np.array_equal(acc_np[r0:r0 + 2048], want.astype(np.int32)), f"rows {r0}.."
    ref = orc.dense_forward(m, x[rows], simd=True)
    assert np.array_equal(acc_np[rows], ref.acc)
    assert out.cpu().numpy()[rows].tobytes() == ref.pre.tobytes()


@pytest.mark.parametrize("norm", ["fast", "strict"])
def test_config4_block_batch8_2048(orc, torch_dev, tf, norm):
    # One BitNet-2B block over 8 sequences x 2048 tokens (M = 16384 rows per
    # projection; the fast mode's fp64-MFMA prefill attention at 2048).
    # Sequences 0 and 5 are checked stage by stage, each against its own
    # oracle MHA (the batch is 8 independent sequences); the others must
    # equal the first by construction of the same kernels, so their K/V
    # caches are checked against the oracle's projection too.
    torch = torch_dev
    sh = CONFIG3
    w = Weights(orc, sh, seed=4101, act=ACT_SILU)
    blk = tf.BitNetBlock(w.cfg(tf, norm, max_batch=8), w.gpu(tf))
    x_in = np.stack([orc.normal_f32(PROMPT * sh.hidden, 4200 + b).reshape(PROMPT, sh.hidden)
                     for b in range(8)])
    xd = to_dev(torch, x_in)
    _, t = blk.forward(xd, taps=True)
    torch.cuda.synchronize()
    out = xd.cpu().numpy()
    T = t.numpy()
    for b in (0, 5):
        Tb = {k: v[b * PROMPT:(b + 1) * PROMPT] for k, v in T.items()}
        ck, cv = (a.cpu().numpy() for a in blk.kv_cache(b))
        print(f"  sequence {b}", flush=True)
        check_stages(orc, w, w.oracle_mha(orc), x_in[b], Tb, out[b], ck, cv, 0,
                     strict=norm == "strict", rows=sample_rows(PROMPT))
    for b in (1, 7):
        mha = w.oracle_mha(orc)
        mha.project(T["y1"][b * PROMPT:(b + 1) * PROMPT], 0)
        ck, cv = (a.cpu().numpy() for a in blk.kv_cache(b))
        assert np.array_equal(cv[:PROMPT], mha.cache_v.reshape(sh.msl, sh.kv_dim)[:PROMPT])
    blk.release()
