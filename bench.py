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
shapes: GB/s for M <= 8, int8 TOPS for M >= 64), the fused SwiGLU FFN, and the
CPU baseline: the oracle's restatement of loom's bitnet_simd path (AVX2 byte
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

UP = (6912, 2560)    # (N, K) of up/gate
DOWN = (2560, 6912)  # (N, K) of down


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * ((k + 15) // 16) * 4 + 4 * m * (k + n)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_cores() -> int:
    try:
        c = len(os.sched_getaffinity(0))
    except AttributeError:
        c = os.cpu_count() or 1
    return max(1, min(c, 16))  # the GPU box's host share is 16 cores


class Timer:
    """HIP-event timing on the stream every loom_amd launch uses (torch's current
    stream).  Steps are captured into a HIP graph of `per_graph` consecutive
    calls and the graph is replayed, so the measurement is the device's
    back-to-back throughput, not the Python launch rate."""

    def __init__(self, torch):
        self.torch = torch

    def _capture(self, fn, first: int, count: int):
        graph = self.torch.cuda.CUDAGraph()
        with self.torch.cuda.graph(graph):
            for i in range(first, first + count):
                fn(i)
        return graph

    def run(self, fn, steps: int, warmup: int, per_graph: int = 64) -> float:
        """Mean ms per call over exactly `steps` calls (after `warmup` calls)."""
        torch = self.torch
        per_graph = max(1, min(per_graph, steps))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(max(1, warmup)):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        full, rest = divmod(steps, per_graph)
        graph = self._capture(fn, 0, per_graph) if full else None
        tail = self._capture(fn, full * per_graph, rest) if rest else None
        for g in (graph, tail):
            if g is not None:
                g.replay()  # untimed: first replay uploads the graph
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
        return start.elapsed_time(end) / steps  # ms per call


def make_matrix(orc, n, k, seed):
    return orc.random_matrix(n, k, seed=seed)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
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

    def step_dense(i):
        bn.dense_forward_packed_ternary(ups[i % rot], x1, out=out1)

    ms_step = timer.run(step_dense, args.steps, args.warmup, per_graph=rot)
    b1 = gemv_bytes(1, n, k)
    value = b1 / (ms_step * 1e-3) / 1e9
    log(f"dense M=1 up: {ms_step * 1e3:.2f} us/step, {value:.0f} GB/s")

    # dominant kernel alone (pre-quantized activations): per-launch duration
    q1 = bn.quantize_activation(x1)

    def step_gemv(i):
        bn.ternary_matvec_quantized(ups[i % rot], q1)

    ms_kernel = timer.run(step_gemv, args.steps, args.warmup, per_graph=rot)
    achieved = b1 / (ms_kernel * 1e-3) / 1e9
    log(f"gemv kernel M=1 up: {ms_kernel * 1e3:.2f} us/launch, {achieved:.0f} GB/s")

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
        "data": "synthetic: seeded ternary weights P(0)=.5, x~N(0,1); weights rotate over "
                f"{rot} HBM-resident copies",
        "config": {"workload": "config1 ternary GEMV M=1 K=2560 N=6912 (= config0 shape), "
                               "DenseForwardPackedTernary: act-quant + GEMV + epilogue",
                   "M": 1, "K": k, "N": n, "rotating_copies": rot,
                   "kernel": _lib.lib().loom_amd_kernel_variant(1).decode()},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "skinny_matmul_kernel<1,1,8> (ternary GEMV)",
                     "us_per_launch": round(ms_kernel * 1e3, 3), "bytes_per_launch": b1},
    }

    # ---------------- config-1 sweep ----------------------------------------------
    if not args.no_sweep:
        sweep = []
        for shape_name, (nn, kk), mats in (("up_gate", UP, ups), ("down", DOWN, dns)):
            for M in (1, 8, 64, 512, 4096):
                x = torch.from_numpy(orc.normal_f32(M * kk, seed=M).reshape(M, kk)).cuda()
                q = bn.quantize_activation(x)
                o = torch.empty((M, nn), dtype=torch.float32, device="cuda")
                steps = max(20, min(args.steps, int(2e5 / M)))
                nm = len(mats) if M <= 64 else 1
                t_k = timer.run(lambda i: bn.ternary_matvec_quantized(mats[i % nm], q),
                                steps, max(5, steps // 10), per_graph=min(nm, 64) if nm > 1 else 16)
                t_d = timer.run(lambda i: bn.dense_forward_packed_ternary(mats[i % nm], x, out=o),
                                steps, max(5, steps // 10), per_graph=min(nm, 64) if nm > 1 else 16)
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

    # ---------------- CPU baseline (oracle port of loom's bitnet_simd path) -------
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
        "value": round(b1 / cpu_s / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": f"config0 GEMV M=1 K=2560 N=6912 repeated {reps}x over {args.cpu_seconds:.0f}s "
                  f"({cpu_s * 1e3:.3f} ms/GEMV; AVX2 byte-code path, bitNetRunRows fan-out)",
        "simd": "avx2" if orc.simd_available() else "scalar",
    }
    log(f"cpu baseline {result['cpu_baseline']}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
