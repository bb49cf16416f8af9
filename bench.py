"""Benchmark of the BitNet b1.58 ternary hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-sweep] [--cpu-seconds S]

Headline (BASELINE.json metric, config 1 at M=1 on the up/gate shape, which is
config 0's GEMV): one step = one DenseForwardPackedTernary pass (activation
quantization + ternary GEMV + fp64 rescale epilogue) of one token row through
a K=2560 -> N=6912 ternary matrix.  Steps rotate over R distinct weight copies
(R * 4.42 MB >= 2 x the 256 MB Infinity Cache) so every step streams its
weights from HBM.  value = algorithmic bytes per step / time per step, with
bytes = N*ceil(K/16)*4 + 4*M*(K+N) (packed weights + fp32 in + fp32 out).

Also reported: the dominant kernel's roofline (per-launch time from HIP events
on the launch stream), the config-1 sweep (M in {1,8,64,512,4096} on both FFN
shapes, plus M=16384, config 4's rows per GEMM: GB/s for M <= 8, int8 TOPS for
M >= 64), the fused SwiGLU FFN, the
config-2 decoder block (seq 512), the config-3 greedy decode (30 layers, vocab
128256, 2048-token prompt, 256 tokens; tok/s) and the config-4 prefill (batch
8 x 2048; tok/s and int8 TOPS of the ternary projections), and the CPU
baseline: the oracle's restatement of loom's bitnet_simd path (AVX2 byte
codes, row fan-out over the host cores) on a bounded sample of config 0.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA, TOPS
MALL_BYTES = 256 << 20
METRIC = ("ternary GEMV GB/s (%HBM peak); decode tok/s + prefill int8 TOPS at BitNet-2B shape")

SUSTAIN_COPIES = 128  # stacked up-shape matrices of the sustained figure (566 MB)

UP = (6912, 2560)    # (N, K) of up/gate
DOWN = (2560, 6912)  # (N, K) of down


def pmc_traffic():
    """HBM bytes per launch of the GEMV kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs of this same workload (profiles/
    gemv_m1_up_pmc.md: counters scaled by a copy kernel of known size)."""
    path = os.path.join(ROOT, "profiles", "gemv_m1_up_pmc.json")
    try:
        with open(path) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def traced_step():
    """The timed kernel's figures from the committed rocprofv3 kernel trace of
    this same command (profiles/gemv_m1_up_trace.json): average dispatch
    duration over the timed launches, and their span (first start to last end)
    per launch, which the tracer's own per-dispatch work lengthens."""
    path = os.path.join(ROOT, "profiles", "gemv_m1_up_trace.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * ((k + 15) // 16) * 4 + 4 * m * (k + n)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_cores() -> int:
    """Worker threads of the CPU baseline: every core the process may run on
    (Go's GOMAXPROCS default), at most 16, the GPU box's host share."""
    return max(1, min(cpu_nproc(), 16))


def cpu_nproc() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_host_fields(cores: int) -> dict:
    return {"cores": cores, "nproc": cpu_nproc(), "os_cpu_count": os.cpu_count(),
            "cpu_model": cpu_model()}


class Timer:
    """HIP-event timing on the stream every loom_amd launch uses (torch's current
    stream).  Steps are captured into HIP graphs and the graphs are replayed,
    so the measurement is the device's back-to-back throughput, not the Python
    launch rate.

    Rotating runs (rotate=R > 1: call i uses weight copy i % R) capture one
    graph of all R calls, whatever `steps` is, and time ceil(steps / R) replays
    of it: the timed region always covers whole rotations (at least `steps`
    calls, every copy read), and the mean is over the calls actually run
    (`last_launches`).  Before the timed region the
    full graph runs once untimed, so copy i was last read R - i calls earlier:
    the copies read after it (>= 2 x MALL of bytes for the first R - 58) have
    evicted it from the MALL and the L2s, while the address translations stay
    warm, as they are for a model whose weights are read once per token.
    Inside the timed region a copy is read again only after the other R - 1
    copies, so every call streams its weights from HBM."""

    def __init__(self, torch):
        self.torch = torch
        self.last_working_set = 0  # distinct copies the last rotating timed region read
        self.last_launches = 0  # calls the last timed region ran

    def _capture(self, fn, first: int, count: int):
        graph = self.torch.cuda.CUDAGraph()
        with self.torch.cuda.graph(graph):
            for i in range(first, first + count):
                fn(i)
        return graph

    def run(self, fn, steps: int, warmup: int, per_graph: int = 64, rotate: int = 0) -> float:
        """Mean ms per call over `steps` calls (after `warmup` calls); rotating
        runs round `steps` up to whole rotations."""
        torch = self.torch
        steps = max(1, steps)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(max(1, warmup)):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        if rotate > 1:
            # whole rotations only: the timed region reads every copy, so its
            # working set is all R copies whatever `steps` is
            per_graph = rotate
            full, rest = -(-steps // rotate), 0
        else:
            per_graph = max(1, min(per_graph, steps))
            full, rest = divmod(steps, per_graph)
        graph = self._capture(fn, 0, per_graph) if full else None
        tail = self._capture(fn, 0, rest) if rest else None
        for g in (tail, graph):
            if g is not None:
                g.replay()  # untimed: uploads the graphs; the full rotation runs last
        launches = full * per_graph + rest
        self.last_launches = launches
        if rotate > 1:
            self.last_working_set = rotate
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(full):
            graph.replay()
        if tail is not None:
            tail.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / launches  # ms per call

    def run_big(self, fn, reps: int) -> float:
        """Mean ms per call of `reps` back-to-back calls that each stream more
        than 2 x MALL (so each call's first bytes were evicted by the previous
        call's last ones), after one untimed call."""
        torch = self.torch
        fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps


def make_matrix(orc, n, k, seed):
    return orc.random_matrix(n, k, seed=seed)


def random_ternary_words(rng, rows: int, cols: int):
    """loom BitNetTernaryMatrix words with P(0)=.5, P(+1)=P(-1)=.25: each 2-bit
    field f of a uniform word maps to code 01 (zero) for f<2, 10 (+1) for f=2,
    00 (-1) for f=3 (codes 0/1/2 = -1/0/+1, poly/bitnet_cpu.go:498-507)."""
    import numpy as np
    rw = (cols + 15) // 16
    w = rng.integers(0, 1 << 32, size=rows * rw, dtype=np.uint64).astype(np.uint32)
    lo = w & np.uint32(0x55555555)
    hi = (w >> np.uint32(1)) & np.uint32(0x55555555)
    code = ((hi & ~lo & np.uint32(0x55555555)) << np.uint32(1)) | (~hi & np.uint32(0x55555555))
    if cols % 16:
        keep = np.uint32((1 << (2 * (cols % 16))) - 1)
        code.reshape(rows, rw)[:, -1] &= keep
    return code


BITNET_2B = dict(hidden=2560, heads=20, kv_heads=5, head_dim=128, inter=6912, vocab=128256,
                 layers=30, theta=500000.0)


def ternary_ops_per_token(c) -> float:
    """2 x (ternary weights per layer) x layers: int8 ops of the projections."""
    h, q, kv, f = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]
    per_layer = h * (q + 2 * kv) + q * h + 3 * h * f
    return 2.0 * per_layer * c["layers"]


def decode_bytes_per_token(c, ctx: float) -> float:
    """HBM bytes one decode step must read: packed ternary weights, the LM
    head's int8 screening copy (codes and per-row scales: the greedy head reads
    the fp32 rows of its candidates only, about a hundred rows here, which
    are not counted), the K and V rows of `ctx` cached positions, the norm
    vectors."""
    h, q, kv, f = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]
    packed = (q + 2 * kv) * ((h + 15) // 16) * 4 + h * ((q + 15) // 16) * 4 \
        + 2 * f * ((h + 15) // 16) * 4 + h * ((f + 15) // 16) * 4
    norms = (2 * h + q + f) * 4
    return c["layers"] * (packed + norms + 2 * kv * 4 * ctx) + c["vocab"] * (h + 4)


def cpu_decode_sample(c, cores, log):
    """Bounded CPU sample of config 3 on the oracle (loom's bitnet_simd path
    restated): one decode step of one layer at context 2048 with a synthetic
    KV cache (the step's cost does not depend on the cached values), times 30
    layers, plus one fp32 LM head in DotTile order."""
    import numpy as np

    from oracle import oracle as orc
    h, q_dim, kv_dim, inter = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]
    ctx = 2048
    mats = [orc.random_matrix(r, k, 0x900 + i) for i, (r, k) in
            enumerate([(q_dim, h), (kv_dim, h), (kv_dim, h), (h, q_dim), (inter, h), (inter, h), (h, inter)])]
    mha = orc.MHA(*mats[:4], c["heads"], c["kv_heads"], c["head_dim"], ctx + 64, theta=c["theta"],
                  eps=1e-5, inner_norm=orc.uniform_f32(q_dim, 0.5, 1.5, 1))
    mha.cache_k[:] = orc.normal_f32(mha.cache_k.size, 2)
    mha.cache_v[:] = orc.normal_f32(mha.cache_v.size, 3)
    blk = orc.Block(mha, orc.uniform_f32(h, 0.5, 1.5, 4), orc.uniform_f32(h, 0.5, 1.5, 5), *mats[4:],
                    orc.uniform_f32(inter, 0.5, 1.5, 6), norm_eps=1e-5, ffn_eps=1e-5, ffn_activation=1)
    x = orc.normal_f32(h, 7).reshape(1, h)
    steps = 3
    t0 = time.perf_counter()
    for i in range(steps):
        mha.c.kv_offset = ctx + i
        blk.c.mha.kv_offset = ctx + i
        blk.forward(x, workers=cores)
    layer_s = (time.perf_counter() - t0) / steps
    table = orc.normal_f32(c["vocab"] * h, 8)
    t0 = time.perf_counter()
    orc.lm_head(x[0], table, simd=True)
    lm_s = time.perf_counter() - t0
    step_s = layer_s * c["layers"] + lm_s
    log(f"cpu decode sample: layer step {layer_s * 1e3:.1f} ms, LM head {lm_s * 1e3:.1f} ms")
    return {"value": round(1.0 / step_s, 3), "unit": "tok/s", **cpu_host_fields(cores), "kind": "port",
            "sample": f"one decode step of one BitNet-2B layer at context {ctx} (synthetic KV), "
                      f"{steps} runs, x{c['layers']} layers, + one fp32 LM head "
                      f"({layer_s * 1e3:.1f} ms/layer, {lm_s * 1e3:.1f} ms LM head)"}


def cpu_block_sample(c, cores, seq, log):
    """Config 2 on the oracle: one block forward over `seq` tokens."""
    from oracle import oracle as orc
    h, q_dim, kv_dim, inter = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]
    mats = [orc.random_matrix(r, k, 0xA00 + i) for i, (r, k) in
            enumerate([(q_dim, h), (kv_dim, h), (kv_dim, h), (h, q_dim), (inter, h), (inter, h), (h, inter)])]
    mha = orc.MHA(*mats[:4], c["heads"], c["kv_heads"], c["head_dim"], 512, theta=c["theta"], eps=1e-5,
                  inner_norm=orc.uniform_f32(q_dim, 0.5, 1.5, 1))
    blk = orc.Block(mha, orc.uniform_f32(h, 0.5, 1.5, 4), orc.uniform_f32(h, 0.5, 1.5, 5), *mats[4:],
                    orc.uniform_f32(inter, 0.5, 1.5, 6), norm_eps=1e-5, ffn_eps=1e-5, ffn_activation=1)
    x = orc.normal_f32(seq * h, 9).reshape(seq, h)
    t0 = time.perf_counter()
    blk.forward(x, workers=cores)
    s = time.perf_counter() - t0
    log(f"cpu block seq{seq}: {s:.2f} s")
    return {"value": round(seq / s, 1), "unit": "tokens/s", **cpu_host_fields(cores), "kind": "port",
            "sample": f"one config-2 block forward over {seq} tokens ({s:.2f} s)"}


def cpu_sweep_sample(orc, cores, ms, log):
    """Config 1 on the oracle: DenseForwardPackedTernaryCPU over M rows, each
    row a full bitNetRunRows fan-out GEMV, rows one after another
    (poly/dense.go:83-99), on both FFN shapes."""
    import numpy as np
    rows = []
    for shape_name, (nn, kk), seed in (("up_gate", UP, 0xB17), ("down", DOWN, 0xD0)):
        m = orc.random_matrix(nn, kk, seed)
        m.ensure_codes()
        for M in ms:
            x = orc.normal_f32(M * kk, seed=M).reshape(M, kk)
            orc.dense_forward(m, x[:1], simd=True, workers=cores)
            t0 = time.perf_counter()
            orc.dense_forward(m, x, simd=True, workers=cores)
            dt = time.perf_counter() - t0
            by = gemv_bytes(M, nn, kk)
            rows.append({"shape": shape_name, "M": M, "ms": round(dt * 1e3, 3),
                         "GBs": round(by / dt / 1e9, 3),
                         "GOPS": round(2.0 * M * kk * nn / dt / 1e9, 2)})
            log(f"cpu sweep {rows[-1]}")
    del np
    return {"runs": rows, "unit": "ms per DenseForward of M rows", **cpu_host_fields(cores),
            "kind": "port",
            "sample": "each (shape, M) once after one warm row; M rows serial, each fanned out "
                      "over the cores as loom's bitNetRunRows does"}


def cpu_prefill_slice(c, cores, log, seq=64):
    """Config 4 on the oracle, bounded: one BitNet-2B layer's block forward
    over a 64-token prefill slice (fresh cache), scaled to 30 layers."""
    from oracle import oracle as orc
    h, q_dim, kv_dim, inter = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]
    mats = [orc.random_matrix(r, k, 0xB00 + i) for i, (r, k) in
            enumerate([(q_dim, h), (kv_dim, h), (kv_dim, h), (h, q_dim), (inter, h), (inter, h), (h, inter)])]
    mha = orc.MHA(*mats[:4], c["heads"], c["kv_heads"], c["head_dim"], 2048, theta=c["theta"],
                  eps=1e-5, inner_norm=orc.uniform_f32(q_dim, 0.5, 1.5, 1))
    blk = orc.Block(mha, orc.uniform_f32(h, 0.5, 1.5, 4), orc.uniform_f32(h, 0.5, 1.5, 5), *mats[4:],
                    orc.uniform_f32(inter, 0.5, 1.5, 6), norm_eps=1e-5, ffn_eps=1e-5, ffn_activation=1)
    x = orc.normal_f32(seq * h, 11).reshape(seq, h)
    t0 = time.perf_counter()
    blk.forward(x, workers=cores)
    layer_s = time.perf_counter() - t0
    tok_s = seq / (layer_s * c["layers"])
    log(f"cpu prefill slice: {seq} tokens, one layer {layer_s:.2f} s")
    return {"value": round(tok_s, 2), "unit": "tokens/s", **cpu_host_fields(cores), "kind": "port",
            "sample": f"one BitNet-2B layer over a {seq}-token prefill slice ({layer_s:.2f} s), "
                      f"x{c['layers']} layers (config 4's prefill is 8 x 2048 tokens; the "
                      "slice's per-token cost is the rate)"}


def bench_model(args, torch, timer, log):
    """Configs 2-4 on a random-init BitNet-2B-shape model."""
    import numpy as np

    from loom_amd import transformer as tf
    from loom_amd.bitnet import TernaryMatrix

    c = dict(BITNET_2B)
    c["layers"] = args.model_layers
    h, q_dim, kv_dim, inter = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]
    prompt, gen, batch = 2048, 256, 8
    msl = prompt + gen
    rng = np.random.default_rng(2025)
    t0 = time.perf_counter()

    def mat(rows, cols):
        return TernaryMatrix.from_words(random_ternary_words(rng, rows, cols), rows, cols,
                                        float(rng.uniform(0.01, 0.03)))

    def layer():
        return tf.BlockWeights(
            mat(q_dim, h), mat(kv_dim, h), mat(kv_dim, h), mat(h, q_dim), mat(inter, h),
            mat(inter, h), mat(h, inter),
            rng.uniform(0.5, 1.5, h).astype(np.float32), rng.uniform(0.5, 1.5, h).astype(np.float32),
            rng.uniform(0.5, 1.5, q_dim).astype(np.float32),
            rng.uniform(0.5, 1.5, inter).astype(np.float32))

    out = {}
    # ---- config 2: one block, seq 512, batch 1 -------------------------------
    w0 = layer()
    blocks = {}
    for norm in ("strict", "fast"):
        cfg = tf.BlockConfig(h, c["heads"], c["kv_heads"], c["head_dim"], inter, max_seq_len=512,
                             rope_theta=c["theta"], norm_eps=1e-5, ffn_activation=1, norm=norm)
        blocks[norm] = tf.BitNetBlock(cfg, w0)
    x512 = torch.from_numpy(rng.standard_normal((512, h), dtype=np.float32)).cuda()
    xs = x512.clone()
    blk_res = []
    for norm, blk in blocks.items():
        def fwd(i, blk=blk):
            xs.copy_(x512)
            blk.forward(xs)
        steps = 10
        ms = timer.run(fwd, steps, 2, per_graph=5)
        ops = ternary_ops_per_token(dict(c, layers=1)) * 512
        blk_res.append({"norm": norm, "ms": round(ms, 3), "tok_s": round(512 / (ms * 1e-3), 1),
                        "int8_TOPS_projections": round(ops / (ms * 1e-3) / 1e12, 2)})
        log(f"config2 block seq512 {blk_res[-1]}")
        blk.release()
    if args.cpu_seconds > 0:
        out["cpu_block_seq512"] = cpu_block_sample(c, cpu_cores(), 512, log)
    out["block_seq512"] = {"config": "config2 BitNet-2B block (hidden 2560, 20/5 heads x 128, "
                                     "FFN 6912 SiLU-gated), seq 512, batch 1, fp32 norms, fp64 "
                                     "attention", "runs": blk_res}

    # ---- configs 3 and 4: the full stack ---------------------------------------
    layers = [w0] + [layer() for _ in range(c["layers"] - 1)]
    emb = rng.standard_normal((c["vocab"], h), dtype=np.float32) * np.float32(0.02)
    fnorm = rng.uniform(0.5, 1.5, h).astype(np.float32)
    log(f"model weights generated in {time.perf_counter() - t0:.1f}s")
    res3, res4 = [], []
    # one prompt (and one config-4 batch) for both norm modes, so their tokens compare
    ids1 = rng.integers(0, c["vocab"], size=(1, prompt)).astype(np.int32)
    ids8 = rng.integers(0, c["vocab"], size=(batch, prompt)).astype(np.int32)
    gen_tokens = {}
    for norm in args.model_norms.split(","):
        cfg = tf.BlockConfig(h, c["heads"], c["kv_heads"], c["head_dim"], inter, max_seq_len=msl,
                             max_batch=batch, rope_theta=c["theta"], norm_eps=1e-5,
                             ffn_activation=1, norm=norm)
        t1 = time.perf_counter()
        model = tf.Transformer(cfg, layers, emb, fnorm, vocab=c["vocab"], final_norm_eps=1e-5,
                               max_tokens=msl + 1, max_prefill=prompt)
        log(f"model ({norm}) on device in {time.perf_counter() - t1:.1f}s")
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # config 3: prefill 2048, then 256 greedy tokens through the captured step
        model.prefill(ids1)
        model.decode(4, use_graph=True)  # capture + upload the step graph
        torch.cuda.synchronize()
        ev0.record()
        model.prefill(ids1)
        ev1.record()
        torch.cuda.synchronize()
        t_pre1 = ev0.elapsed_time(ev1)
        ev0.record()
        model.decode(gen, use_graph=True)
        ev1.record()
        torch.cuda.synchronize()
        t_dec = ev0.elapsed_time(ev1)
        toks = model.tokens()
        gen_tokens[norm] = toks[0, prompt + 1:prompt + 1 + gen].copy()
        tok_s = gen / (t_dec * 1e-3)
        gbs = decode_bytes_per_token(c, prompt + gen / 2) * tok_s / 1e9
        res3.append({"norm": norm, "decode_tok_s": round(tok_s, 2),
                     "hbm_GBs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                     "ms_per_token": round(t_dec / gen, 4), "prefill_ms": round(t_pre1, 2),
                     "prefill_tok_s": round(prompt / (t_pre1 * 1e-3), 1),
                     "last_tokens": toks[0, -4:].tolist()})
        log(f"config3 decode {res3[-1]}")
        # config 4: batch 8 x 2048 prefill
        model.prefill(ids8)
        torch.cuda.synchronize()
        reps = 2
        ev0.record()
        for _ in range(reps):
            model.prefill(ids8)
        ev1.record()
        torch.cuda.synchronize()
        t4 = ev0.elapsed_time(ev1) / reps
        ntok = batch * prompt
        res4.append({"norm": norm, "ms": round(t4, 2), "tok_s": round(ntok / (t4 * 1e-3), 1),
                     "int8_TOPS_projections": round(ternary_ops_per_token(c) * ntok / (t4 * 1e-3) / 1e12, 2)})
        log(f"config4 prefill {res4[-1]}")
        model.release()
    if args.cpu_seconds > 0:
        out["cpu_decode"] = cpu_decode_sample(c, cpu_cores(), log)
        out["cpu_prefill_slice"] = cpu_prefill_slice(c, cpu_cores(), log)
    out["decode"] = {"config": f"config3: {c['layers']} layers, vocab {c['vocab']}, tied fp32 "
                               f"LM head, greedy, {prompt}-token random prompt, {gen} tokens, "
                               "one HIP graph per token, positions on device; the same prompt "
                               "for both norm modes",
                     "runs": res3}
    if "fast" in gen_tokens and "strict" in gen_tokens:
        # greedy tokens of the two summation modes, position by position: they
        # agree until a near-tie of two logits flips (then the sequences part)
        same = gen_tokens["fast"] == gen_tokens["strict"]
        first = int(np.argmin(same)) if not same.all() else len(same)
        out["decode"]["fast_strict_tokens"] = {"equal": int(same.sum()), "of": int(same.size),
                                               "first_difference_at": first}
    out["prefill"] = {"config": f"config4: batch {batch} x {prompt} random ids, M={batch * prompt} "
                                "rows per ternary GEMM, KV cache per sequence",
                      "runs": res4}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--sweep-m", default="1,8,64,512,4096,16384",
                    help="token rows of the config-1 sweep (16384: config 4's rows per GEMM)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-model", action="store_true", help="skip configs 2-4")
    ap.add_argument("--model-layers", type=int, default=30)
    ap.add_argument("--model-norms", default="fast,strict")
    ap.add_argument("--no-sustained", dest="sustained", action="store_false",
                    help="skip the single-launch sustained-bandwidth figure")
    ap.add_argument("--calibrate-copy", type=int, default=0,
                    help="also run 4 device copies of this many MiB (PMC byte-counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the ternary layers shard by output rows; see DESIGN.md). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from loom_amd import _lib, bitnet as bn
    from oracle import oracle as orc

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    _lib.lib()
    torch.cuda.set_device(0)
    timer = Timer(torch)
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")

    # ---------------- weights: R rotating copies of each FFN shape -------------
    n, k = UP
    per = n * ((k + 15) // 16) * 4
    rot = max(2, -(-2 * MALL_BYTES // per))  # >= 2 x MALL
    host_up = make_matrix(orc, n, k, seed=0xB17)
    ups = [bn.TernaryMatrix.from_words(host_up.words, n, k, host_up.scale) for _ in range(rot)]
    host_dn = make_matrix(orc, DOWN[0], DOWN[1], seed=0xD0)
    dns = [bn.TernaryMatrix.from_words(host_dn.words, DOWN[0], DOWN[1], host_dn.scale)
           for _ in range(rot)]
    log(f"weights: {rot} rotating copies x 2 shapes, {rot * per * 2 / 1e6:.0f} MB resident")

    # ---------------- headline: dense forward M=1 on the up shape ---------------
    x1 = torch.from_numpy(orc.normal_f32(k, seed=1).reshape(1, k)).cuda()
    out1 = torch.empty((1, n), dtype=torch.float32, device="cuda")
    b1 = gemv_bytes(1, n, k)

    def step_dense(i):
        bn.dense_forward_packed_ternary(ups[i % rot], x1, out=out1)

    ms_step = timer.run(step_dense, args.steps, args.warmup, rotate=rot)
    copies_read = timer.last_working_set
    launches_timed = timer.last_launches
    working_set = copies_read * per + 4 * (k + n)
    value = b1 / (ms_step * 1e-3) / 1e9
    log(f"dense M=1 up: {ms_step * 1e3:.2f} us/step, {value:.0f} GB/s "
        f"(timed region read {copies_read} copies, {working_set / 1e6:.0f} MB)")

    # the GEMV alone on pre-quantized activations (the step's kernel without
    # its quantization prologue)
    q1 = bn.quantize_activation(x1)

    def step_gemv(i):
        bn.ternary_matvec_quantized(ups[i % rot], q1)

    ms_kernel = timer.run(step_gemv, args.steps, args.warmup, rotate=rot)
    log(f"gemv kernel M=1 up (pre-quantized): {ms_kernel * 1e3:.2f} us/launch, "
        f"{b1 / (ms_kernel * 1e-3) / 1e9:.0f} GB/s")

    # latency floor of one launch that streams this many bytes: a device copy
    # of the packed weights' size, rotating over as many buffers (HBM-resident)
    srcs = [torch.empty(per // 4, dtype=torch.float32, device="cuda").fill_(1.0) for _ in range(rot)]
    dst = torch.empty_like(srcs[0])
    ms_copy = timer.run(lambda i: dst.copy_(srcs[i % rot]), args.steps, args.warmup, rotate=rot)
    del srcs, dst
    log(f"device copy of {per} B: {ms_copy * 1e3:.2f} us/launch")

    # sustained rate of the same kernels without the per-launch floor: one
    # launch over a stacked matrix of SUSTAIN_COPIES up-shape matrices (N =
    # 6912 x copies rows, >= 2 x MALL), launched back to back
    sustained = None
    if args.sustained:
        big_n = n * SUSTAIN_COPIES
        words = np.tile(host_up.words.reshape(n, -1), (SUSTAIN_COPIES, 1)).reshape(-1)
        bigs = [bn.TernaryMatrix.from_words(words, big_n, k, host_up.scale) for _ in range(2)]
        del words
        big_bytes = gemv_bytes(1, big_n, k)
        ob = torch.empty((1, big_n), dtype=torch.float32, device="cuda")
        # two such matrices alternate: each launch's weights were last read
        # 570 MB (> 2 x MALL) earlier
        t_big_f = timer.run(lambda i: bn.dense_forward_packed_ternary(bigs[i % 2], x1, out=ob), 10, 2,
                            rotate=2)
        t_big_k = timer.run(lambda i: bn.ternary_matvec_quantized(bigs[i % 2], q1), 10, 2, rotate=2)
        sustained = {
            "bytes_per_launch": big_bytes, "rows": big_n, "K": k,
            "us_fused": round(t_big_f * 1e3, 2), "us_kernel": round(t_big_k * 1e3, 2),
            "GBs_fused": round(big_bytes / (t_big_f * 1e-3) / 1e9, 1),
            "GBs_kernel": round(big_bytes / (t_big_k * 1e-3) / 1e9, 1),
            "frac": round(big_bytes / (t_big_f * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "frac_kernel": round(big_bytes / (t_big_k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel": "stream_kernel (persistent streaming GEMV: the dispatcher's choice for "
                      ">= 4096 16-row tiles)",
            "note": f"one launch over {SUSTAIN_COPIES} stacked up-shape matrices "
                    f"({big_bytes / 1e6:.0f} MB, > 2 x MALL); two such matrices alternate over "
                    "10 timed launches",
        }
        log(f"sustained: {sustained}")
        for b in bigs:
            b.release()
        del ob

    achieved = b1 / (ms_step * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xternary->int32, fp64 rescale, fp32 io",
        "data": "synthetic: seeded ternary weights P(0)=.5, x~N(0,1); step i reads weight copy "
                f"i % {rot} ({rot} HBM-resident copies, {rot * per / 1e6:.0f} MB); the timed "
                f"region runs whole rotations ({launches_timed} launches for --steps "
                f"{args.steps}, every copy read) after an untimed one, so each timed step's "
                "weights come from HBM; ms_per_step is the mean over the launches run",
        "working_set_bytes": working_set,
        "launches_timed": launches_timed,
        "config": {"workload": "config1 ternary GEMV M=1 K=2560 N=6912 (= config0 shape), "
                               "DenseForwardPackedTernary: act-quant + GEMV + epilogue",
                   "M": 1, "K": k, "N": n, "rotating_copies": rot,
                   "kernel": _lib.lib().loom_amd_kernel_variant(1).decode()},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": pmc_traffic(),
                     "kernel": "skinny_kernel<1,1,4,true,0,0,4,1,2> (fused act-quant + ternary "
                               "GEMV + epilogue; four waves, two 16-row weight tiles per workgroup: "
                               "the step's only launch)",
                     "us_per_launch": round(ms_step * 1e3, 3), "bytes_per_launch": b1,
                     "us_prequantized_kernel": round(ms_kernel * 1e3, 3),
                     "GBs_prequantized_kernel": round(b1 / (ms_kernel * 1e-3) / 1e9, 1),
                     "copy_floor_us": round(ms_copy * 1e3, 3),
                     "copy_floor_note": f"torch device copy of {per} B (read + write) per launch, "
                                        f"same rotation: the per-launch latency floor at this size",
                     "sustained": sustained},
    }
    tr = traced_step()
    if tr:
        # frac from the profile's per-dispatch duration, next to the one from
        # this run's HIP events (`frac`, the line's figure)
        us = tr["us_per_dispatch"]
        result["roofline"]["traced"] = {
            "us_per_dispatch": us, "frac": round(b1 / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "us_span_per_launch": tr["us_span_per_launch"],
            "us_per_step_hip_events_traced": tr["us_per_step_hip_events_traced"],
            "source": "profiles/gemv_m1_up_kernel_trace.md (rocprofv3 --kernel-trace of this command)"}

    # ---------------- config-1 sweep ----------------------------------------------
    if not args.no_sweep:
        sweep = []
        for shape_name, (nn, kk), mats in (("up_gate", UP, ups), ("down", DOWN, dns)):
            for M in (int(v) for v in args.sweep_m.split(",") if v):
                x = torch.from_numpy(orc.normal_f32(M * kk, seed=M).reshape(M, kk)).cuda()
                q = bn.quantize_activation(x)
                o = torch.empty((M, nn), dtype=torch.float32, device="cuda")
                steps = max(20, min(args.steps, int(2e5 / M)))
                nm = len(mats) if M <= 64 else 1
                t_k = timer.run(lambda i: bn.ternary_matvec_quantized(mats[i % nm], q),
                                steps, max(5, steps // 10), per_graph=16, rotate=nm)
                t_d = timer.run(lambda i: bn.dense_forward_packed_ternary(mats[i % nm], x, out=o),
                                steps, max(5, steps // 10), per_graph=16, rotate=nm)
                ent = {"shape": shape_name, "M": M, "K": kk, "N": nn,
                       "kernel": _lib.lib().loom_amd_kernel_variant(M).decode(),
                       "us_kernel": round(t_k * 1e3, 3), "us_dense": round(t_d * 1e3, 3)}
                by = gemv_bytes(M, nn, kk)
                ops = 2.0 * M * kk * nn
                ent["GBs_kernel"] = round(by / (t_k * 1e-3) / 1e9, 1)
                ent["TOPS_kernel"] = round(ops / (t_k * 1e-3) / 1e12, 2)
                if M <= 8:
                    ent["frac_hbm"] = round(ent["GBs_kernel"] / HBM_PEAK_GBS, 4)
                else:
                    ent["frac_int8"] = round(ent["TOPS_kernel"] / INT8_PEAK_TOPS, 4)
                sweep.append(ent)
                log(f"sweep {ent}")
        result["sweep"] = sweep

        # fused SwiGLU FFN (gate|up -> SiLU -> inner norm -> requant -> down)
        ffn = []
        g0, u0, d0 = ups[0], ups[1], dns[0]
        for M in (1, 64, 512):
            x = torch.from_numpy(orc.normal_f32(M * 2560, seed=7 + M).reshape(M, 2560)).cuda()
            for norm in ("strict", "fast"):
                steps = max(10, min(500, int(5e4 / M)))
                t = timer.run(lambda i: bn.swiglu_forward_packed_ternary(g0, u0, d0, x, norm=norm),
                              steps, max(3, steps // 10), per_graph=8)
                ffn.append({"M": M, "norm": norm, "us": round(t * 1e3, 2),
                            "TOPS": round(3 * 2.0 * M * 2560 * 6912 / (t * 1e-3) / 1e12, 2)})
                log(f"swiglu {ffn[-1]}")
        result["swiglu_ffn"] = ffn

    # ---------------- configs 2-4: block, decode loop, batched prefill ------------
    if not args.no_model:
        result.update(bench_model(args, torch, timer, log))

    # ---------------- copy kernel of known size (PMC calibration runs) ---------------
    if args.calibrate_copy > 0:
        nbytes = int(args.calibrate_copy) << 20
        src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = nbytes
        log(f"calibration: 4 device copies of {nbytes} B")

    # ---------------- CPU baseline (oracle port of loom's bitnet_simd path) -------
    if args.cpu_seconds <= 0:
        print(json.dumps(result), flush=True)
        return 0
    cores = cpu_cores()
    xs = orc.normal_f32(k, seed=1).reshape(1, k)
    host_up.ensure_codes()
    orc.dense_forward(host_up, xs, simd=True, workers=cores)  # warm the codes / threads
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < args.cpu_seconds:
        orc.dense_forward(host_up, xs, simd=True, workers=cores)
        reps += 1
    cpu_s = (time.perf_counter() - t0) / reps
    result["cpu_baseline"] = {
        "value": round(b1 / cpu_s / 1e9, 3), "unit": "GB/s", **cpu_host_fields(cores), "kind": "port",
        "sample": f"config0 GEMV M=1 K=2560 N=6912 repeated {reps}x over {args.cpu_seconds:.0f}s "
                  f"({cpu_s * 1e3:.3f} ms/GEMV; AVX2 byte-code path, bitNetRunRows fan-out)",
        "simd": "avx2" if orc.simd_available() else "scalar",
    }
    log(f"cpu baseline {result['cpu_baseline']}")
    if not args.no_sweep:
        result["cpu_sweep"] = cpu_sweep_sample(orc, cores, [1, 8, 64, 512, 4096], log)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
