"""Parity of the gfx950 decoder block and decode loop against the CPU oracle
(loom's MHAForwardPackedTernaryCPU / forwardOnCPUNormal / Generate restated).

Every block call is checked stage by stage, each stage fed the GPU's own
input to it (tests/stages.py states the bar of each stage).  Taps do not
change which kernels run, so the decode rows are checked on the norm-fused
matmuls and the fused decode attention that production runs; the staged
kernels are checked by forcing them (LOOM_AMD_UNFUSED_NORM /
LOOM_AMD_UNFUSED_ROPE).  The LM head is bit-exact in both of loom's orders
and the greedy token is the oracle's argmax of the GPU logits.
Citations are relative to the loom v0.83.0 tree.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from tests.stages import (ACT_RELU2, ACT_SILU, BITNET_2B, SMALL, Shape, Weights, check_stages,  # noqa: F401
                          run_block_case, to_dev, ulp_diff_f32)


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


@pytest.mark.parametrize("seqs", [[1], [5], [9, 1, 1, 1], [64], [37, 1], [17]])
def test_block_stages_small(orc, torch_dev, tf, seqs):
    w = Weights(orc, SMALL, seed=101)
    run_block_case(orc, torch_dev, tf, w, seqs, seed=900)


def test_block_stages_bias_and_silu(orc, torch_dev, tf):
    # MHA biases (poly/mha.go:273-282) and the SiLU gate
    w = Weights(orc, SMALL, seed=131, act=ACT_SILU, bias=True)
    run_block_case(orc, torch_dev, tf, w, [7, 1, 1], seed=910)


def test_block_stages_mha_no_gqa(orc, torch_dev, tf):
    # num_kv_heads == num_heads, head_dim 32
    sh = Shape(128, 4, 4, 32, 256, 32)
    w = Weights(orc, sh, seed=141)
    run_block_case(orc, torch_dev, tf, w, [6, 1], seed=920)


@pytest.mark.parametrize("seqs", [[12, 1], [40, 1]])
def test_block_stages_fast_norm(orc, torch_dev, tf, seqs):
    # fast mode: tree / chunked sums, fused multiply-adds in the prefill tiles
    w = Weights(orc, SMALL, seed=151)
    run_block_case(orc, torch_dev, tf, w, seqs, seed=930, strict=False)


def test_block_fast_prefill_bitnet_2b(orc, torch_dev, tf):
    # fast prefill tiles at the BitNet-2B head size (128)
    w = Weights(orc, BITNET_2B, seed=155)
    run_block_case(orc, torch_dev, tf, w, [70, 1], seed=935, strict=False)


@pytest.mark.parametrize("norm", ["fast", "strict"])
def test_block_repeatable(orc, torch_dev, tf, norm):
    # The same prefill (every GEMM shape of the block, K-stage tails included)
    # and decode step, many times back to back: every output byte and every
    # cached K/V row must repeat.  A race between waves or launches shows up
    # here as a rare difference.
    torch = torch_dev
    # 700 rows: the down projection (K = 6912, an odd number of K stages) runs
    # unsplit, so its one-stage tail meets the epilogue
    sh = Shape(2560, 20, 5, 128, 6912, 768)
    w = Weights(orc, sh, seed=181, act=ACT_SILU)
    blk = tf.BitNetBlock(w.cfg(tf, norm), w.gpu(tf))
    xp = to_dev(torch, orc.normal_f32(700 * sh.hidden, 960).reshape(700, sh.hidden))
    x1 = to_dev(torch, orc.normal_f32(sh.hidden, 961).reshape(1, sh.hidden))
    ref = None
    for rep in range(40 if norm == "fast" else 10):
        a, b = xp.clone(), x1.clone()
        blk.forward(a)
        blk.forward(b)
        ck, cv = blk.kv_cache(0)
        got = (a.clone(), b.clone(), ck.clone(), cv.clone())
        if ref is None:
            ref = got
            continue
        for name, g, r in zip(("prefill", "decode", "K cache", "V cache"), got, ref):
            assert torch.equal(g, r), f"repetition {rep}: {name} differs"
    blk.release()


def test_block_stages_bitnet_2b_shape(orc, torch_dev, tf):
    # config 2's block shape: hidden 2560, 20 heads / 5 KV heads x 128, FFN 6912
    w = Weights(orc, BITNET_2B, seed=161)
    run_block_case(orc, torch_dev, tf, w, [16, 1, 1], seed=940)


def test_block_bitnet_2b_seq512(orc, torch_dev, tf):
    # config 2 at its full length: seq 512, batch 1 (stage-wise, strict)
    w = Weights(orc, BITNET_2B, seed=171)
    run_block_case(orc, torch_dev, tf, w, [512], seed=950)


def test_block_end_to_end_tolerance(orc, torch_dev, tf):
    # Whole block vs the oracle's own chain, each fed only the block input
    # (not a parity bar: the stage-wise tests are).  Only libm last bits
    # (pow/cos/sin in RoPE, exp in the softmax) differ, so almost every element
    # is identical; a moved int8 code changes a row by about one quantization
    # step.
    torch = torch_dev
    w = Weights(orc, SMALL, seed=181)
    blk = tf.BitNetBlock(w.cfg(tf), w.gpu(tf))
    ref = w.oracle_block(orc)
    for i, seq in enumerate([10, 1, 1]):
        x_in = orc.normal_f32(seq * SMALL.hidden, 960 + i).reshape(seq, SMALL.hidden)
        x = to_dev(torch, x_in)
        blk.forward(x)
        got = x.cpu().numpy()
        want = ref.forward(x_in)
        eq = np.mean(got == want)
        err = np.abs(got - want).max() / np.abs(want).max()
        print(f"  call {i}: identical {eq:.4f}, max rel err {err:.2e}", flush=True)
        assert eq > 0.95 and err < 1e-2
    blk.release()


def test_block_batch_equals_separate_sequences(orc, torch_dev, tf):
    # batch sequences each own a KV cache: a batch-3 call equals three batch-1
    # calls, prefill and decode, bit for bit.
    torch = torch_dev
    w = Weights(orc, SMALL, seed=191)
    gw = w.gpu(tf)
    big = tf.BitNetBlock(w.cfg(tf, max_batch=3), gw)
    singles = [tf.BitNetBlock(w.cfg(tf), gw) for _ in range(3)]
    for step, seq in enumerate([8, 1, 1]):
        xs = [orc.normal_f32(seq * SMALL.hidden, 1000 + 10 * step + b).reshape(seq, SMALL.hidden)
              for b in range(3)]
        xb = to_dev(torch, np.stack(xs))
        big.forward(xb)
        for b in range(3):
            xi = to_dev(torch, xs[b])
            singles[b].forward(xi)
            assert np.array_equal(xb[b].cpu().numpy(), xi.cpu().numpy())
    for b in range(3):
        kb, vb = (t.cpu().numpy() for t in big.kv_cache(b))
        ks, vs = (t.cpu().numpy() for t in singles[b].kv_cache(0))
        assert np.array_equal(kb[:10], ks[:10]) and np.array_equal(vb[:10], vs[:10])


def test_block_prefill_resets_cache(orc, torch_dev, tf):
    # mhaPrepareKVForForward: any call that is not a warm single-token step
    # restarts at position 0 (same outputs again).
    torch = torch_dev
    w = Weights(orc, SMALL, seed=201)
    blk = tf.BitNetBlock(w.cfg(tf), w.gpu(tf))
    x_in = orc.normal_f32(4 * SMALL.hidden, 1100).reshape(4, SMALL.hidden)
    a = to_dev(torch, x_in)
    blk.forward(a)
    blk.forward(to_dev(torch, x_in[:1]))
    assert blk.kv_offset == 5
    b = to_dev(torch, x_in)
    blk.forward(b)
    assert blk.kv_offset == 4
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_block_refuses_positions_past_ring(orc, torch_dev, tf):
    from loom_amd._lib import AMDError
    torch = torch_dev
    w = Weights(orc, SMALL, seed=211)
    blk = tf.BitNetBlock(w.cfg(tf), w.gpu(tf))
    with pytest.raises(AMDError, match="max_seq_len"):
        blk.forward(to_dev(torch, np.zeros((SMALL.msl + 1, SMALL.hidden), np.float32)))
    with pytest.raises(AMDError, match="max_batch"):
        blk.forward(to_dev(torch, np.zeros((2, 3, SMALL.hidden), np.float32)))


def test_block_refuses_decode_batch_other_than_warm_cache(orc, torch_dev, tf):
    # each sequence owns a KV ring: a single-token call continuing a warm
    # cache must have the batch that filled it (a wider batch would read slots
    # no call wrote); a longer call restarts every sequence at position 0
    from loom_amd._lib import AMDError
    torch = torch_dev
    w = Weights(orc, SMALL, seed=213)
    blk = tf.BitNetBlock(w.cfg(tf, max_batch=2), w.gpu(tf))
    x4 = orc.normal_f32(4 * SMALL.hidden, 1110).reshape(1, 4, SMALL.hidden)
    blk.forward(to_dev(torch, x4))
    with pytest.raises(AMDError, match="warm cache of batch 1"):
        blk.forward(to_dev(torch, np.zeros((2, 1, SMALL.hidden), np.float32)))
    assert blk.kv_offset == 4
    blk.forward(to_dev(torch, x4[:, :1]))  # same batch continues
    assert blk.kv_offset == 5
    blk.forward(to_dev(torch, np.concatenate([x4, x4])))  # batch 2 restarts
    assert blk.kv_offset == 4
    blk.forward(to_dev(torch, np.zeros((2, 1, SMALL.hidden), np.float32)))
    assert blk.kv_offset == 5
    with pytest.raises(AMDError, match="warm cache of batch 2"):
        blk.forward(to_dev(torch, np.zeros((1, 1, SMALL.hidden), np.float32)))
    blk.release()


@pytest.mark.parametrize("hd,seq", [(128, 300), (64, 200)])
def test_fast_prefill_attention_kernels_agree(orc, torch_dev, tf, tuning, hd, seq):
    # the two-pass fast prefill kernel with 32 or 64 queries per workgroup
    # sums in the same order: identical bytes for the block output and its K/V
    # caches, ragged last query tile included.  The one-pass kernel (running
    # maximum; LOOM_AMD_ATTN_QT=1 forces it) sums in another fixed order: its
    # attention rows are within the fast bar (1e-12 of the row scale) of the
    # two-pass rows, and its K/V caches are the same bytes.  Unset, a grid this
    # small takes the two-pass kernel: the same bytes as "2".
    torch = torch_dev
    sh = Shape(hd * 4, 4, 2, hd, 512, 512)
    w = Weights(orc, sh, seed=451)
    x = orc.normal_f32(seq * sh.hidden, seed=452).reshape(seq, sh.hidden)
    outs, attn, kv = [], [], []
    for qt in ("2", "4", "1", ""):
        tuning("LOOM_AMD_ATTN_QT", qt)
        blk = tf.BitNetBlock(w.cfg(tf, norm="fast"), w.gpu(tf))
        xd = to_dev(torch, x)
        _, T = blk.forward(xd, taps=True)
        torch.cuda.synchronize()
        outs.append(xd.cpu().numpy().tobytes())
        attn.append(T.numpy()["attn"])
        kv.append(b"".join(c.cpu().numpy().tobytes() for c in blk.kv_cache()))
        blk.release()
    assert outs[0] == outs[1] == outs[3] and kv[0] == kv[1] == kv[2] == kv[3]
    assert np.array_equal(attn[0], attn[1]) and np.array_equal(attn[0], attn[3])
    scale = np.abs(attn[0]).max(axis=-1, keepdims=True)
    assert np.all(np.abs(attn[2] - attn[0]) <= 1e-12 * scale)
    assert not np.array_equal(attn[2], attn[0])  # (the one-pass kernel did run)


# ---------------------------------------------------------------- model / decode loop
class Model:
    def __init__(self, orc, sh: Shape, layers: int, vocab: int, seed: int):
        self.sh, self.vocab = sh, vocab
        self.layers = [Weights(orc, sh, seed + 100 * i) for i in range(layers)]
        self.emb = orc.normal_f32(vocab * sh.hidden, seed + 7) * np.float32(0.5)
        self.fn = orc.uniform_f32(sh.hidden, 0.5, 1.5, seed + 8)

    def gpu(self, tf, max_tokens, max_batch=1, norm="strict"):
        cfg = self.layers[0].cfg(tf, norm=norm, max_batch=max_batch)
        return tf.Transformer(cfg, [w.gpu(tf) for w in self.layers], self.emb, self.fn,
                              vocab=self.vocab, final_norm_eps=1e-6, max_tokens=max_tokens)


def test_model_prefill_head_and_greedy_token(orc, torch_dev, tf):
    torch = torch_dev
    sh = SMALL
    M = Model(orc, sh, layers=2, vocab=1000, seed=301)
    model = M.gpu(tf, max_tokens=40)
    ids = (np.arange(12) * 37 + 5) % 1000
    logits = model.prefill(ids, logits=True).cpu().numpy()[0]
    hid = model.last_hidden().cpu().numpy()[0]
    # stack plumbing: embeddings -> the same blocks one by one -> final norm
    blocks = [tf.BitNetBlock(w.cfg(tf), w.gpu(tf)) for w in M.layers]
    x = to_dev(torch, M.emb.reshape(1000, sh.hidden)[ids])
    for b in blocks:
        b.forward(x)
    last = x.cpu().numpy()[-1:]
    assert np.array_equal(hid, orc.rmsnorm_forward(last, M.fn, 1e-6)[0])
    # LM head in DotTile order (poly/transformer.go:679-681) and greedy pick
    table = M.emb
    assert np.array_equal(logits, orc.lm_head(hid, table, simd=True))
    toks = model.tokens()[0]
    assert np.array_equal(toks[:12], ids)
    assert toks[12] == orc.argmax_first(logits)
    # close to the oracle's own full chain (libm last bits only)
    ref_x = M.emb.reshape(1000, sh.hidden)[ids].copy()
    for w in M.layers:
        ref_x = w.oracle_block(orc).forward(ref_x)
    ref_logits = orc.lm_head(orc.rmsnorm_forward(ref_x[-1:], M.fn, 1e-6)[0], table, simd=True)
    err = np.abs(ref_logits - logits).max() / np.abs(ref_logits).max()
    print(f"  prefill logits vs oracle chain: max rel err {err:.2e}", flush=True)
    assert err < 1e-2


def test_model_decode_graph_matches_eager(orc, torch_dev, tf):
    torch = torch_dev
    M = Model(orc, SMALL, layers=2, vocab=1000, seed=401)
    model = M.gpu(tf, max_tokens=48)
    prompt = (np.arange(9) * 101 + 3) % 1000
    model.prefill(prompt)
    model.decode(4, use_graph=True)  # capture, then replay after a new prefill
    model.prefill(prompt)
    lg_graph = model.decode(20, use_graph=True, logits=True).cpu().numpy()
    t_graph = model.tokens()
    assert model.position == 29
    assert t_graph.min() >= 0 and t_graph.max() < 1000
    model.prefill(prompt)
    lg_eager = model.decode(20, use_graph=False, logits=True).cpu().numpy()
    t_eager = model.tokens()
    assert np.array_equal(t_graph, t_eager)
    assert np.array_equal(lg_graph, lg_eager)
    # each decode step: LM head of the final hidden row, then argmax
    hid = model.last_hidden().cpu().numpy()[0]
    assert np.array_equal(lg_eager[0], orc.lm_head(hid, M.emb, simd=True))
    assert t_eager[0, 29] == orc.argmax_first(lg_eager[0])
    # graph replays continue from where eager steps stopped
    model.decode(3, use_graph=True)
    assert model.position == 32


def _screen_table(orc, case, vocab, hidden):
    """LM-head tables around the screened head's cases: (table, query row id)."""
    rng = np.random.default_rng(7)
    e = (rng.standard_normal((vocab, hidden)) * 0.5).astype(np.float32)
    q = np.abs(e[11]) + np.float32(0.25)  # positive entries
    e[11] = q
    if case == "below_code":
        # three rows whose int8 codes and scales are the query's: the exact logits order them
        e[100] = q * np.float32(1 + 2.0 ** -20)
        e[2000] = q * np.float32(1 + 2.0 ** -19)
    elif case == "ties":
        for r in (700, 300, 2500):
            e[r] = q * np.float32(1.5)
    elif case == "zero_query":
        e[11] = 0.0
    elif case == "nan_at_0":
        e[0, 3] = np.nan
        e[40] = q * np.float32(2)
    elif case == "nan_and_inf":
        e[5, 9] = np.nan
        e[7, 20] = np.inf
    elif case == "overflow":
        e[9] = np.float32(3e37)
    elif case == "tiny_rows":
        # with the final norm -1 the query is -1 in every column: every row of
        # positive entries has a negative logit, an all-zero row gives -0 and a
        # row of negative subnormals (its scale would round coarsely) leads
        e[:] = np.abs(e)
        e[11] = 1.0
        e[13] = np.float32(-1e-41)
        e[14] = 0.0
    elif case == "near_max":
        # many rows within the screening bound of the maximum
        e[1000:1400] = q * np.float32(1.2) + (rng.standard_normal((400, hidden)) * 1e-4).astype(np.float32)
    return e, 11


@pytest.mark.parametrize("case", ["random", "below_code", "ties", "zero_query", "nan_at_0", "nan_and_inf",
                                  "overflow", "tiny_rows", "near_max", "sequential", "final_norm"])
def test_model_screened_greedy_head(orc, torch_dev, tf, case, tuning):
    # One row's greedy token comes from an int8 screening pass and the exact
    # logits of its candidates; LOOM_AMD_LM_SCREEN=0 runs the full fp32 head.
    # Same token in both, equal to the oracle's pick over every logit, on
    # tables built around the bound: rows equal below the codes' precision,
    # exact ties, an all-zero query (every row a candidate), NaN at row 0 and
    # elsewhere, an Inf entry, a logit that overflows fp32, subnormal and zero
    # rows, 400 rows near the maximum; loom's sequential order; a final norm.
    vocab, hidden = 3000, 256
    table, qid = _screen_table(orc, "random" if case in ("sequential", "final_norm") else case, vocab, hidden)
    cfg = tf.BlockConfig(hidden, 4, 2, 64, 512, max_seq_len=64, norm="fast")
    fn = orc.uniform_f32(hidden, 0.5, 1.5, 91) if case == "final_norm" else None
    if case == "tiny_rows":
        fn = np.full(hidden, -1.0, np.float32)
    model = tf.Transformer(cfg, [], table, fn, vocab=vocab, final_norm_eps=1e-6, max_tokens=8,
                           simd_forward=case != "sequential")
    picks = []
    for screen in (None, "0"):
        tuning("LOOM_AMD_LM_SCREEN", screen)
        lg = model.prefill([3, qid], logits=True).cpu().numpy()[0]
        tok_lg = int(model.tokens()[0, 2])
        model.prefill([3, qid])
        picks.append((int(model.tokens()[0, 2]), tok_lg, lg))
    tuning("LOOM_AMD_LM_SCREEN", None)
    (t_s, t_s2, lg_s), (t_f, t_f2, lg_f) = picks
    want = orc.argmax_first(lg_f)
    print(f"  {case}: screened {t_s}, full {t_f}, oracle {want}", flush=True)
    assert lg_s.tobytes() == lg_f.tobytes()  # logits asked for are every logit, both ways
    assert t_s == t_s2 == t_f == t_f2 == want
    if case == "ties":
        assert want == 300
    if case == "below_code":
        assert want == 2000
    if case in ("zero_query", "nan_at_0"):
        assert want == 0
    if case == "overflow":
        assert want == 9
    if case == "tiny_rows":
        assert want == 13
    model.release()


@pytest.mark.parametrize("batch", [1, 2])
def test_model_screened_head_decode(orc, torch_dev, tf, tuning, batch):
    # 40 graph-replayed decode steps of a two-layer model, one or two
    # sequences (the screened head runs row after row): the screened head's
    # tokens equal the full head's (each model captures its graph under its
    # own setting)
    M = Model(orc, SMALL, layers=2, vocab=1000, seed=411)
    prompt = (np.arange(7) * 53 + 1) % 1000
    if batch == 2:
        prompt = np.stack([prompt, (np.arange(7) * 31 + 5) % 1000])
    toks = []
    for screen in (None, "0"):
        tuning("LOOM_AMD_LM_SCREEN", screen)
        model = M.gpu(tf, max_tokens=64, max_batch=batch, norm="fast")
        model.prefill(prompt)
        model.decode(40, use_graph=True)
        toks.append(model.tokens())
        model.release()
    tuning("LOOM_AMD_LM_SCREEN", None)
    assert np.array_equal(toks[0], toks[1])


def test_model_decode_step_equals_block_chain(orc, torch_dev, tf):
    # one decode step == embedding of the newest token through the same
    # blocks (warm caches), final norm, LM head
    torch = torch_dev
    sh = SMALL
    M = Model(orc, sh, layers=2, vocab=500, seed=501)
    model = M.gpu(tf, max_tokens=32)
    prompt = (np.arange(6) * 13 + 1) % 500
    model.prefill(prompt)
    model.decode(2, use_graph=True)
    toks = model.tokens()[0]
    blocks = [tf.BitNetBlock(w.cfg(tf), w.gpu(tf)) for w in M.layers]
    table = M.emb.reshape(500, sh.hidden)
    x = to_dev(torch, table[prompt])
    for b in blocks:
        b.forward(x)
    for step in range(2):
        x = to_dev(torch, table[toks[6 + step]][None])
        for b in blocks:
            b.forward(x)
    hid = orc.rmsnorm_forward(x.cpu().numpy(), M.fn, 1e-6)[0]
    assert np.array_equal(model.last_hidden().cpu().numpy()[0], hid)
    assert toks[8] == orc.argmax_first(orc.lm_head(hid, M.emb, simd=True))


def test_model_batch_generate_equals_single(orc, torch_dev, tf):
    M = Model(orc, SMALL, layers=1, vocab=700, seed=601)
    prompts = np.stack([(np.arange(7) * (17 + b) + b) % 700 for b in range(3)])
    big = M.gpu(tf, max_tokens=24, max_batch=3)
    got = big.generate(prompts, 10)
    for b in range(3):
        one = M.gpu(tf, max_tokens=24)
        assert np.array_equal(got[b], one.generate(prompts[b], 10)[0])


def test_model_refuses_bad_calls(orc, torch_dev, tf):
    from loom_amd._lib import AMDError
    M = Model(orc, SMALL, layers=1, vocab=300, seed=701)
    model = M.gpu(tf, max_tokens=16)
    with pytest.raises(AMDError, match="prefill first"):
        model.decode(1)
    with pytest.raises(AMDError, match="prompt"):
        model.prefill(np.zeros(16, np.int32))
    model.prefill(np.zeros(10, np.int32))
    with pytest.raises(AMDError, match="max_tokens"):
        model.decode(6)
    # ids outside the table embed as zero rows (poly/transformer.go:568-571)
    model.prefill(np.array([5, 299, 300, -1, 1 << 30], np.int32))
    model.decode(1)


# ---------------------------------------------------------------- LM head / sampling
@pytest.mark.parametrize("vocab,hidden", [(1, 8), (33, 7), (100, 64), (257, 100), (1000, 2560),
                                          (70, 2567), (5000, 320)])
def test_lm_head_dottile_order(orc, torch_dev, tf, vocab, hidden):
    # applyFP32LMHeadRows with SIMD (poly/transformer.go:679-681): DotTile's
    # eight-lane order (poly/simd/avx2_amd64.s), bit-exact; several rows.
    torch = torch_dev
    table = orc.normal_f32(vocab * hidden, 17 + hidden) * np.float32(0.05)
    rows = [orc.normal_f32(hidden, 29 + r) for r in range(3)]
    got = tf.lm_head(to_dev(torch, table.reshape(vocab, hidden)), to_dev(torch, np.stack(rows)))
    got = got.cpu().numpy()
    for r, x in enumerate(rows):
        assert np.array_equal(got[r], orc.lm_head(x, table, simd=True)), (vocab, hidden, r)


@pytest.mark.parametrize("vocab,hidden", [(1, 8), (33, 7), (100, 64), (257, 100), (1000, 2560),
                                          (70, 2567), (5000, 320), (600, 65)])
def test_lm_head_sequential_order(orc, torch_dev, tf, vocab, hidden):
    # applyFP32LMHeadRows with SIMD forward off (poly/transformer.go:681-687):
    # one sequential fp64 sum per logit, bit-exact; several rows, widths that
    # end mid-slab, and a last row where the sequential and DotTile orders
    # give 0 and 1 (products 2^60, 1, -2^60).
    torch = torch_dev
    table = orc.normal_f32(vocab * hidden, 19 + hidden) * np.float32(0.05)
    rows = [orc.normal_f32(hidden, 31 + r) for r in range(3)]
    if hidden >= 3:
        t = table.reshape(vocab, hidden)
        t[-1] = 0.0
        t[-1, :3] = [2.0 ** 30, 2.0 ** -30, -(2.0 ** 30)]
        rows.append(np.full(hidden, 2.0 ** 30, np.float32))
    dt, dx = to_dev(torch, table.reshape(vocab, hidden)), to_dev(torch, np.stack(rows))
    got = tf.lm_head_sequential(dt, dx).cpu().numpy()
    for r, x in enumerate(rows):
        assert np.array_equal(got[r], orc.lm_head(x, table, simd=False)), (vocab, hidden, r)
    if hidden >= 3:
        assert got[-1, -1] == 0.0
    if hidden >= 8:  # narrower rows are all DotTile tail, summed in order
        assert tf.lm_head(dt, dx).cpu().numpy()[-1, -1] == 1.0


def test_greedy_sample_semantics(orc, torch_dev, tf):
    # SampleTopK greedy (poly/sampling.go:44-55): first strict maximum; NaN
    # never wins; a NaN at index 0 is never replaced.  Rows long enough to
    # span several partial ranges, with ties placed across range borders.
    torch = torch_dev
    n = 128256
    rows = []
    base = orc.normal_f32(n, 5)
    rows.append(base.copy())
    r = base.copy(); r[4007] = 9.0; r[4008] = 9.0; r[100000] = 9.0; rows.append(r)   # tie across ranges
    r = base.copy(); r[0] = np.nan; r[77] = 50.0; rows.append(r)                     # NaN at 0
    r = base.copy(); r[5] = np.nan; r[n - 1] = 50.0; rows.append(r)                 # NaN elsewhere, max last
    r = np.full(n, -np.inf, np.float32); rows.append(r)                              # all -inf
    r = np.full(n, np.nan, np.float32); r[3] = 1.0; r[0] = 0.5; rows.append(r)
    r = np.full(n, 2.0, np.float32); rows.append(r)                                  # all equal
    x = np.stack(rows)
    ids = tf.greedy_sample(to_dev(torch, x)).cpu().numpy()
    want = [orc.argmax_first(row) for row in rows]
    assert ids.tolist() == want
    assert want[1] == 4007 and want[2] == 0 and want[3] == n - 1 and want[4] == 0
    for m in (1, 2, 4095, 4096, 4097, 70000):
        row = orc.normal_f32(m, m)
        got = tf.greedy_sample(to_dev(torch, row[None])).cpu().numpy()[0]
        assert got == orc.argmax_first(row), m


# ---------------------------------------------------------------- per-head Q/K norms
# MHAForwardPackedTernaryCPU normalizes Q (fp64) and the fp32 K cache row per
# head before RoPE when QNormWeight / KNormWeight are set (poly/mha.go:285-290,
# 584-646).  The stage checks pin them bit for bit at position 0 (rotation the
# identity) and within the RoPE bar elsewhere; the prefill runs qkv_rope_kernel,
# the single-token calls the fused decode attention (strict: the scores kernel,
# fast: the GQA chunk kernel).
@pytest.mark.parametrize("norm", ["strict", "fast"])
@pytest.mark.parametrize("qk", ["shared", "per_head"])
def test_block_stages_qk_norm(orc, torch_dev, tf, norm, qk):
    w = Weights(orc, SMALL, seed=191, qk=qk)
    run_block_case(orc, torch_dev, tf, w, [9, 1, 1], seed=1910, strict=norm == "strict")


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_block_stages_qk_norm_default_eps_bias_odd_length(orc, torch_dev, tf, norm):
    # RMSNormEps unset: Q/K eps 1e-6 (mhaQKNormEpsilon), inner norm 1e-5; a Q
    # norm of another length than head_dim / q_dim applies unit weights; biases
    w = Weights(orc, SMALL, seed=193, act=ACT_SILU, bias=True, qk="odd", attn_eps=0.0)
    run_block_case(orc, torch_dev, tf, w, [5, 1, 1], seed=1930, strict=norm == "strict")


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_block_stages_qk_norm_bitnet_2b_shape(orc, torch_dev, tf, norm):
    w = Weights(orc, BITNET_2B, seed=195, qk="per_head")
    run_block_case(orc, torch_dev, tf, w, [70, 1, 1], seed=1950, strict=norm == "strict")


def test_block_stages_qk_norm_head_dims(orc, torch_dev, tf):
    # strict decode scores kernels at head_dim 32 and 256
    for i, sh in enumerate([Shape(128, 4, 4, 32, 256, 48), Shape(512, 4, 2, 256, 512, 48)]):
        w = Weights(orc, sh, seed=197 + i, qk="shared")
        run_block_case(orc, torch_dev, tf, w, [6, 1, 1], seed=1970 + 10 * i)


@pytest.mark.parametrize("shape,norm", [("small", "fast"), ("bitnet2b", "fast"),
                                        ("small", "strict"), ("bitnet2b", "strict")])
def test_decode_qk_norm_fused_equals_separate(orc, torch_dev, tf, shape, norm, tuning):
    # the norms inside the fused decode attention equal qkv_rope_kernel's
    # (LOOM_AMD_UNFUSED_ROPE=1), outputs and caches bit for bit, batch 2
    torch = torch_dev
    sh = {"small": SMALL, "bitnet2b": BITNET_2B}[shape]
    w = Weights(orc, sh, seed=1261, bias=True, qk="per_head")
    gw = w.gpu(tf)
    fused = tf.BitNetBlock(w.cfg(tf, norm, max_batch=2), gw)
    tuning("LOOM_AMD_UNFUSED_ROPE", "1")
    plain = tf.BitNetBlock(w.cfg(tf, norm, max_batch=2), gw)
    tuning("LOOM_AMD_UNFUSED_ROPE", None)
    for i, seq in enumerate([min(62, sh.msl - 8), 1, 1, 1]):
        x_in = orc.normal_f32(2 * seq * sh.hidden, 1500 + i).reshape(2, seq, sh.hidden)
        a = to_dev(torch, x_in.reshape(2 * seq, sh.hidden)).reshape(2, seq, sh.hidden)
        b = a.clone()
        fused.forward(a)
        plain.forward(b)
        torch.cuda.synchronize()
        assert a.cpu().numpy().tobytes() == b.cpu().numpy().tobytes(), f"call {i}"
        for slot in (0, 1):
            for t_a, t_b in zip(fused.kv_cache(slot), plain.kv_cache(slot)):
                assert t_a.cpu().numpy().tobytes() == t_b.cpu().numpy().tobytes(), f"cache call {i}"
    fused.release()
    plain.release()


@pytest.mark.parametrize("shape,norm", [("small", "fast"), ("bitnet2b", "fast"),
                                        ("small", "strict"), ("bitnet2b", "strict"),
                                        ("mha32", "strict")])
def test_decode_rope_fused_attention(orc, torch_dev, tf, shape, norm, tuning):
    # Single-token decode runs the Q/K/V epilogue (RoPE, K/V cache write)
    # inside the attention launch (fast: the GQA chunk kernel; strict: the
    # scores kernel); with LOOM_AMD_UNFUSED_ROPE=1 a block keeps the separate
    # epilogue kernel.  Same steps, so outputs and caches agree bit for bit,
    # over batch 2 and several positions (past one 64-position chunk).
    torch = torch_dev
    sh = {"small": SMALL, "bitnet2b": BITNET_2B, "mha32": Shape(128, 4, 4, 32, 256, 128)}[shape]
    w = Weights(orc, sh, seed=1251, bias=True)
    gw = w.gpu(tf)
    fused = tf.BitNetBlock(w.cfg(tf, norm, max_batch=2), gw)
    tuning("LOOM_AMD_UNFUSED_ROPE", "1")
    plain = tf.BitNetBlock(w.cfg(tf, norm, max_batch=2), gw)
    tuning("LOOM_AMD_UNFUSED_ROPE", None)
    for i, seq in enumerate([min(62, sh.msl - 8), 1, 1, 1, 1]):
        x_in = orc.normal_f32(2 * seq * sh.hidden, 1400 + i).reshape(2, seq, sh.hidden)
        a = to_dev(torch, x_in.reshape(2 * seq, sh.hidden)).reshape(2, seq, sh.hidden)
        b = a.clone()
        fused.forward(a)
        plain.forward(b)
        torch.cuda.synchronize()
        assert a.cpu().numpy().tobytes() == b.cpu().numpy().tobytes(), f"call {i}"
        for slot in (0, 1):
            for t_a, t_b in zip(fused.kv_cache(slot), plain.kv_cache(slot)):
                assert t_a.cpu().numpy().tobytes() == t_b.cpu().numpy().tobytes(), f"cache call {i}"
    fused.release()
    plain.release()


@pytest.mark.parametrize("shape,norm", [("small", "strict"), ("small", "fast"),
                                        ("bitnet2b", "strict"), ("bitnet2b", "fast")])
def test_block_decode_norm_fused_and_staged(orc, torch_dev, tf, shape, norm, tuning):
    # A decode row is normalized inside each matmul that consumes it (RMSNorm1
    # -> QKV, attention inner norm -> O, RMSNorm2 -> gate/up, FFN inner norm
    # -> down); LOOM_AMD_UNFUSED_NORM=1 keeps the separate norm launches.  Both
    # paths are checked stage by stage against the oracle; strict sums are
    # the same ordered chains in both, so their outputs are also equal byte
    # for byte.
    torch = torch_dev
    sh = SMALL if shape == "small" else BITNET_2B
    w = Weights(orc, sh, seed=1201, act=ACT_SILU)
    gw = w.gpu(tf)
    fused = tf.BitNetBlock(w.cfg(tf, norm), gw)
    tuning("LOOM_AMD_UNFUSED_NORM", "1")
    staged = tf.BitNetBlock(w.cfg(tf, norm), gw)
    tuning("LOOM_AMD_UNFUSED_NORM", None)
    refs = {"fused": w.oracle_mha(orc), "staged": w.oracle_mha(orc)}
    base = 0
    for i, seq in enumerate([6, 1, 1, 1]):
        x_in = orc.normal_f32(seq * sh.hidden, 1300 + i).reshape(seq, sh.hidden)
        outs = {}
        for name, blk in (("fused", fused), ("staged", staged)):
            x = to_dev(torch, x_in)
            _, t = blk.forward(x, taps=True)
            torch.cuda.synchronize()
            ck, cv = (a.cpu().numpy() for a in blk.kv_cache(0))
            outs[name] = x.cpu().numpy()
            print(f"  call {i} ({name}): seq={seq} base={base}", flush=True)
            check_stages(orc, w, refs[name], x_in, t.numpy(), outs[name], ck, cv, base,
                         strict=norm == "strict")
        if norm == "strict":
            assert outs["fused"].tobytes() == outs["staged"].tobytes(), f"call {i}"
        base += seq
    fused.release()
    staged.release()


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_decode_rmsnorm_rounding_tie(orc, torch_dev, tf, norm):
    # The norm-fused decode matmul forms loom's float32((v / rms) * gain) from
    # one reciprocal per row and takes the divisions for any value within
    # 2^-50 (relative) of an fp32 rounding boundary.  This row makes rms
    # exactly 1 (127 ones, two values 1 + 2^-12, zeros: every partial sum of
    # squares is exact in any order, and eps tops the mean up to 1), so v =
    # 1 + 2^-12 with gain 1 + 2^-12 gives 1 + 2^-11 + 2^-24, a tie (to even:
    # 1 + 2^-11), while gain 1 + 2^-11 gives a product that is an fp32 value.
    torch = torch_dev
    sh = SMALL
    w = Weights(orc, sh, seed=1401, act=ACT_SILU)
    e = np.float32(1.0 + 2.0 ** -12)
    w.n1 = np.ones(sh.hidden, np.float32)
    w.n1[5] = e
    w.n1[77] = np.float32(1.0 + 2.0 ** -11)
    x = np.zeros((1, sh.hidden), np.float32)
    x[0, 128:255] = 1.0
    x[0, 5] = e
    x[0, 77] = e
    tot = 127.0 + 2 * float(e) ** 2
    eps = 1.0 - tot / sh.hidden
    assert tot / sh.hidden + eps == 1.0
    cfg = tf.BlockConfig(sh.hidden, sh.heads, sh.kv, sh.hd, sh.inter, max_seq_len=sh.msl, max_batch=1,
                         rope_theta=sh.theta, norm_eps=eps, attn_eps=1e-5, ffn_eps=1e-5,
                         ffn_activation=ACT_SILU, norm=norm)
    blk = tf.BitNetBlock(cfg, w.gpu(tf))
    _, t = blk.forward(to_dev(torch, x), taps=True)
    torch.cuda.synchronize()
    T = t.numpy()
    want = orc.rmsnorm_forward(x, w.n1, eps)
    assert want[0, 5] == np.float32(1.0 + 2.0 ** -11)
    assert T["y1"].tobytes() == want.tobytes()
    q_ref, a_ref = orc.quant_rows(T["y1"])
    assert np.array_equal(T["xq1"], q_ref) and T["amax1"].tobytes() == a_ref.tobytes()
    blk.release()


@pytest.mark.parametrize("norm", ["strict", "fast"])
@pytest.mark.parametrize("seq", [5, 1030])
def test_prefill_rmsnorm_rounding_tie(orc, torch_dev, tf, norm, seq):
    # The prefill RMSNorm kernels (one workgroup per row below 1024 rows, one
    # wave per row from 1024) on loom's float32((v / rms) * gain) at an exact
    # fp32 tie: row 0 is the tie row of the decode test (rms exactly 1), the
    # other rows are random.
    torch = torch_dev
    sh = Shape(256, 4, 2, 64, 512, 1100)
    w = Weights(orc, sh, seed=1402, act=ACT_SILU)
    e = np.float32(1.0 + 2.0 ** -12)
    w.n1 = orc.uniform_f32(sh.hidden, 0.5, 1.5, 1403)
    w.n1[5] = e
    x = orc.normal_f32(seq * sh.hidden, 1404).reshape(seq, sh.hidden)
    x[0] = 0.0
    x[0, 128:255] = 1.0
    x[0, 5] = e
    x[0, 77] = e
    tot = 127.0 + 2 * float(e) ** 2
    eps = 1.0 - tot / sh.hidden
    cfg = tf.BlockConfig(sh.hidden, sh.heads, sh.kv, sh.hd, sh.inter, max_seq_len=sh.msl, max_batch=1,
                         rope_theta=sh.theta, norm_eps=eps, attn_eps=1e-5, ffn_eps=1e-5,
                         ffn_activation=ACT_SILU, norm=norm)
    blk = tf.BitNetBlock(cfg, w.gpu(tf))
    _, t = blk.forward(to_dev(torch, x), taps=True)
    torch.cuda.synchronize()
    T = t.numpy()
    want = orc.rmsnorm_forward(x, w.n1, eps)
    assert want[0, 5] == np.float32(1.0 + 2.0 ** -11)
    y1 = T["y1"]
    assert y1[0].tobytes() == want[0].tobytes()
    if norm == "strict":
        assert y1.tobytes() == want.tobytes()
    else:
        assert ulp_diff_f32(y1, want).max() <= 1
    q_ref, a_ref = orc.quant_rows(y1)
    assert np.array_equal(T["xq1"], q_ref) and T["amax1"].tobytes() == a_ref.tobytes()
    blk.release()


@pytest.mark.parametrize("norm,seq", [("fast", 300), ("fast", 1100), ("strict", 1100)])
def test_prefill_row_norms_one_wave_equal_workgroup(orc, torch_dev, tf, tuning, norm, seq):
    # The prefill row norms (RMSNorm1 and 2, the MHA fp64 inner norm, the
    # SwiGLU inner norm) run one wave per row: fast mode in the same summation
    # tree as the one-workgroup-per-row kernels, strict mode with 1024 or more
    # rows on the rows' ordered sums.  LOOM_AMD_ROWNORM_WAVE=0 keeps the
    # workgroup kernels; every tap and the block output must be the same bytes.
    torch = torch_dev
    sh = Shape(2560, 20, 5, 128, 6912, 1152)
    w = Weights(orc, sh, seed=1401, act=ACT_SILU)
    gw = w.gpu(tf)
    x_in = orc.normal_f32(seq * sh.hidden, 1402).reshape(seq, sh.hidden)
    outs = {}
    for mode in ("wave", "workgroup"):
        tuning("LOOM_AMD_ROWNORM_WAVE", None if mode == "wave" else "0")
        blk = tf.BitNetBlock(w.cfg(tf, norm), gw)
        x = to_dev(torch, x_in)
        _, t = blk.forward(x, taps=True)
        torch.cuda.synchronize()
        outs[mode] = (x.cpu().numpy(), t.numpy())
        blk.release()
    a, b = outs["wave"], outs["workgroup"]
    for f in tf.BlockTaps.FIELDS:
        assert a[1][f].tobytes() == b[1][f].tobytes(), f
    assert a[0].tobytes() == b[0].tobytes(), "block output"


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_block_shared_timeline_is_loom_batch(orc, torch_dev, tf, norm):
    # loom's [batch, seq, hidden] call (poly/mha.go:251-371): one KV timeline
    # from position 0 shared by the batch's sequences -- the oracle's literal
    # batch loop equals its call on the rows concatenated (pinned in
    # tests/test_oracle_attention.py), so the shared-timeline call is checked
    # stage by stage as one sequence of batch*seq rows; a warm single-token
    # step then continues the timeline
    torch = torch_dev
    B, S = 3, 7
    sh = SMALL
    w = Weights(orc, sh, seed=1501, act=ACT_SILU)
    blk = tf.BitNetBlock(w.cfg(tf, norm), w.gpu(tf))
    mha_ref = w.oracle_mha(orc)
    x_in = orc.normal_f32(B * S * sh.hidden, 1502).reshape(B, S, sh.hidden)
    x = to_dev(torch, x_in)
    _, t = blk.forward(x, taps=True, shared_timeline=True)
    torch.cuda.synchronize()
    assert blk.kv_offset == B * S
    ck, cv = (a.cpu().numpy() for a in blk.kv_cache(0))
    check_stages(orc, w, mha_ref, x_in.reshape(B * S, sh.hidden), t.numpy(),
                 x.cpu().numpy().reshape(B * S, sh.hidden), ck, cv, 0, strict=norm == "strict")
    x1_in = orc.normal_f32(sh.hidden, 1503).reshape(1, sh.hidden)
    x1 = to_dev(torch, x1_in)
    _, t1 = blk.forward(x1, taps=True)
    torch.cuda.synchronize()
    assert blk.kv_offset == B * S + 1
    ck, cv = (a.cpu().numpy() for a in blk.kv_cache(0))
    check_stages(orc, w, mha_ref, x1_in, t1.numpy(), x1.cpu().numpy(), ck, cv, B * S,
                 strict=norm == "strict")
    blk.release()


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_block_decode_many_positions(orc, torch_dev, tf, norm):
    # single-token steps after a prefill, across decode-attention chunk
    # borders (32-position chunks in fast mode), checked stage by stage
    w = Weights(orc, BITNET_2B, seed=1211, act=ACT_SILU, bias=True)
    run_block_case(orc, torch_dev, tf, w, [31] + [1] * 5 + [1] * 30, seed=1220,
                   strict=norm == "strict")


# ---------------------------------------------------------------- untied (ternary) LM head
def _tiles(tf, bn_mat):
    from loom_amd import _lib
    import ctypes as C
    rows, cols, scale, nbytes = C.c_int(), C.c_int(), C.c_float(), C.c_size_t()
    _lib.lib().loom_amd_matrix_shape(bn_mat.handle, C.byref(rows), C.byref(cols), C.byref(scale),
                                     C.byref(nbytes))
    p = _lib.lib().loom_amd_matrix_tiles(bn_mat.handle)
    t = tf._clone_device(p, (nbytes.value // 4,), 0, "<i4")
    return t.cpu().numpy(), scale.value


@pytest.mark.parametrize("case", ["kat", "normal", "ternary", "specials", "ragged"])
def test_matrix_from_float32_matches_packer(orc, torch_dev, tf, case):
    # loom_amd_matrix_from_float32 packs as packFloat32AsBitNetTernaryMatrix
    # (poly/bitnet_cpu.go:934-962): the same words (hence the same device
    # tiles) and the same scale as the oracle's packer.
    from loom_amd import bitnet as bn
    rng = np.random.default_rng(5)
    if case == "kat":  # poly/tests/bitnet_cpu_test.go:134-153
        rows, cols = 1, 4
        w = np.array([-0.2, -0.8, 0.1, 0.8], np.float32)
    elif case == "normal":
        rows, cols = 96, 640
        w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    elif case == "ternary":  # every weight within 1e-6 of -1, 0, 1: scale 1
        rows, cols = 32, 256
        w = rng.integers(-1, 2, rows * cols).astype(np.float32)
        w += (rng.standard_normal(rows * cols) * 1e-7).astype(np.float32)
    elif case == "specials":  # NaN and out-of-range values become code -1
        rows, cols = 16, 256
        w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
        w[3], w[17], w[40], w[41] = np.nan, np.inf, -np.inf, np.float32(3e38)
    else:
        rows, cols = 33, 65
        w = rng.standard_normal(rows * cols).astype(np.float32)
    ref = orc.pack_float32(w, rows, cols)
    got = bn.TernaryMatrix.from_float32(w, rows, cols)
    want = bn.TernaryMatrix.from_words(ref.words, rows, cols, ref.scale)
    tg, sg = _tiles(tf, got)
    tw, sw = _tiles(tf, want)
    assert np.float32(sg).tobytes() == np.float32(ref.scale).tobytes(), (sg, ref.scale)
    assert np.array_equal(tg, tw)
    if case == "kat":
        assert np.float32(sg) == np.float32(0.475)
    if case == "ternary":
        assert sg == 1.0


@pytest.mark.parametrize("batch", [1, 5])
def test_model_untied_ternary_lm_head(orc, torch_dev, tf, batch):
    # An untied head of a ternary model is what loom ternarizes
    # (usePackedTernaryLMHead / applyPackedTernaryLMHead,
    # poly/transformer.go:721-755): logits = fp32 of the ternary matvec of the
    # final hidden with per-row int8 activations, bit for bit; 5 rows take the
    # separate quantization launch, 1 row the fused one.
    sh = SMALL
    vocab = 700
    M = Model(orc, sh, layers=2, vocab=vocab, seed=331)
    head = orc.normal_f32(vocab * sh.hidden, 339) * np.float32(0.05)
    cfg = M.layers[0].cfg(tf, norm="strict", max_batch=batch)
    model = tf.Transformer(cfg, [w.gpu(tf) for w in M.layers], M.emb, M.fn, lm_head=head,
                           vocab=vocab, final_norm_eps=1e-6, max_tokens=40)
    ids = np.stack([(np.arange(10) * (31 + 2 * b) + 3 * b) % vocab for b in range(batch)])
    logits = model.prefill(ids, logits=True).cpu().numpy()
    hid = model.last_hidden().cpu().numpy()
    packed = orc.pack_float32(head, vocab, sh.hidden)
    ref = orc.dense_forward(packed, hid, simd=True)
    assert logits.tobytes() == ref.pre.tobytes()
    toks = model.tokens()
    for b in range(batch):
        assert toks[b, 10] == orc.argmax_first(logits[b])
    # decode steps take the same head inside the captured step graph
    step_logits = model.decode(3, use_graph=True, logits=True).cpu().numpy()
    hid = model.last_hidden().cpu().numpy()
    assert step_logits.tobytes() == orc.dense_forward(packed, hid, simd=True).pre.tobytes()
    model.release()


def test_model_sequential_lm_head(orc, torch_dev, tf):
    # Network.UseSimdForward off: the tied fp32 head sums each logit in
    # order (poly/transformer.go:681-687), in prefill and in the captured
    # decode step.
    sh = SMALL
    vocab = 900
    M = Model(orc, sh, layers=2, vocab=vocab, seed=351)
    cfg = M.layers[0].cfg(tf, norm="strict", max_batch=2)
    model = tf.Transformer(cfg, [w.gpu(tf) for w in M.layers], M.emb, M.fn, vocab=vocab,
                           final_norm_eps=1e-6, max_tokens=40, simd_forward=False)
    ids = np.stack([(np.arange(9) * 29 + 1) % vocab, (np.arange(9) * 41 + 7) % vocab])
    logits = model.prefill(ids, logits=True).cpu().numpy()
    hid = model.last_hidden().cpu().numpy()
    for b in range(2):
        assert logits[b].tobytes() == orc.lm_head(hid[b], M.emb, simd=False).tobytes()
        assert model.tokens()[b, 9] == orc.argmax_first(logits[b])
    step_logits = model.decode(3, use_graph=True, logits=True).cpu().numpy()
    hid = model.last_hidden().cpu().numpy()
    for b in range(2):
        assert step_logits[b].tobytes() == orc.lm_head(hid[b], M.emb, simd=False).tobytes()
    model.release()
