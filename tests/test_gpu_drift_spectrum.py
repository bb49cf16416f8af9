"""loom's drift-spectrum report for the AMD plugin path, on the GPU.

loom's bridge suites run each layer on loom's CPU path and through a vendor
plugin, then print, per layer, a parity class (max |loom - plugin|) and an
inference-determinism class (max |infer 1 - infer 2|) on the seven-bucket
spectrum EXACT / INDUS / LOWBIT / DRIFT / H-DRIFT / BROKE / FATAL
(lucy/examples/apple/dispatch.go:34-167, lucy/examples/apple/spectrum.go:8-70).
This test does the same for the plugin's BitNetLinear and BitNetSwiGLU layers
at the BASELINE shapes, through the v2 ABI (loom_amd.accel, the same
dlopen/dlsym sequence as loom's loader), with the oracle standing in for
loom's CPU path.  Besides loom's own row classes (GPU parity bar
max(10 tol, 0.05), determinism bar 10 tol) it classifies every output
element against the FP32 tolerance 1e-7 and prints the histogram.

Bars: every BitNetLinear output EXACT (the rescale is loom's fp64 multiply
in its order); BitNetSwiGLU in strict mode within LOWBIT of 1e-7 per element
(exp's last fp64 bit may move one fp32 ulp of h), in fast mode within DRIFT
(a 1-ulp move of h may move one int8 code), its loom row class EXACT or
INDUS; every layer's inference determinism EXACT.
"""
import numpy as np
import pytest

from tests import spectrum as sp

pytestmark = pytest.mark.gpu

FP32_TOL = sp.infer_tolerance("FP32")  # 1e-7

LINEAR_CASES = [  # (k, n, M, act)
    (2560, 6912, 1, -1),    # config 0
    (2560, 6912, 8, -1),    # config 1, up/gate
    (2560, 6912, 64, -1),
    (2560, 6912, 512, -1),
    (6912, 2560, 1, -1),    # config 1, down
    (6912, 2560, 8, -1),
    (6912, 2560, 64, -1),
    (6912, 2560, 512, -1),
    (2560, 2560, 1, -1),    # Q / O
    (2560, 640, 1, -1),     # K / V
    (2560, 6912, 4, 0),     # ReLU
    (2560, 6912, 4, 6),     # ReLU2
]
SWIGLU_CASES = [  # (hidden, inter, M, norm)
    (2560, 6912, 1, "strict"),
    (2560, 6912, 64, "strict"),
    (2560, 6912, 1, "fast"),
    (2560, 6912, 64, "fast"),
]

_rows = []


@pytest.fixture(scope="module")
def plugin():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from loom_amd import accel
    p = accel.open_amd(device="GPU")
    yield p
    p.close()
    if _rows:
        _print_report()


def _record(layer, size, ref, out1, out2, tol_row):
    parity = sp.max_abs_diff(ref, out1)
    det = sp.max_abs_diff(out1, out2)
    row = dict(layer=layer, size=size, parity=parity,
               parity_spec=sp.classify(parity, sp.gpu_parity_tolerance("FP32")),
               det=det, det_spec=sp.classify(det, sp.infer_tolerance("FP32") * 10),
               strict_spec=sp.classify(parity, tol_row),
               hist=sp.histogram(ref, out1, FP32_TOL))
    _rows.append(row)
    return row


def _print_report():
    print()
    print("drift spectrum, AMD plugin (GPU) vs loom CPU path (oracle); per-element classes at "
          f"FP32 tol {FP32_TOL:g}")
    head = f"{'layer':<13} {'size':<34} {'parity':>9} {'loom':<7} {'@1e-7':<7} {'det':<6} " + \
        " ".join(f"{lab:>8}" for lab in sp.LABELS)
    print(head)
    for r in _rows:
        print(f"{r['layer']:<13} {r['size']:<34} {r['parity']:9.2e} {sp.LABELS[r['parity_spec']]:<7} "
              f"{sp.LABELS[r['strict_spec']]:<7} {sp.LABELS[r['det_spec']]:<6} " +
              " ".join(f"{c:>8}" for c in r["hist"]))
    total = [sum(r["hist"][i] for r in _rows) for i in range(7)]
    print(f"{'all':<13} {'':<34} {'':>9} {'':<7} {'':<7} {'':<6} " + " ".join(f"{c:>8}" for c in total))


@pytest.mark.parametrize("k,n,M,act", LINEAR_CASES)
def test_spectrum_bitnet_linear(orc, plugin, k, n, M, act):
    from loom_amd import accel
    m = orc.random_matrix(n, k, seed=5000 + n + k)
    x = orc.normal_f32(M * k, seed=5100 + M).reshape(M, k)
    label = f"m={M},k={k},n={n},act={act}"
    res = plugin.compile_layer(accel.LayerDesc("BitNetLinear", "TERNARY", label), m.entity_blob())
    try:
        out1, out2 = bytearray(res.out_bytes), bytearray(res.out_bytes)
        res.layer.infer(x.tobytes(), out1)
        res.layer.infer(x.tobytes(), out2)
    finally:
        res.layer.release()
    ref = orc.dense_forward(m, x, activation=act, simd=True)
    want = ref.pre if act == -1 else ref.post
    got1 = np.frombuffer(bytes(out1), np.float32).reshape(M, n)
    got2 = np.frombuffer(bytes(out2), np.float32).reshape(M, n)
    row = _record("BitNetLinear", label, want, got1, got2, FP32_TOL)
    assert row["hist"][sp.EXACT] == got1.size, row
    assert row["parity_spec"] == sp.EXACT and row["det_spec"] == sp.EXACT, row


@pytest.mark.parametrize("hidden,inter,M,norm", SWIGLU_CASES)
def test_spectrum_bitnet_swiglu(orc, plugin, hidden, inter, M, norm):
    from loom_amd import accel
    g = orc.random_matrix(inter, hidden, seed=5200)
    u = orc.random_matrix(inter, hidden, seed=5201)
    d = orc.random_matrix(hidden, inter, seed=5202)
    wn = orc.uniform_f32(inter, 0.5, 1.5, seed=5203)
    x = orc.normal_f32(M * hidden, seed=5204 + M).reshape(M, hidden)
    label = f"m={M},k={hidden},n={inter},eps=1e-5,norm={norm}"
    blob = g.entity_blob() + u.entity_blob() + d.entity_blob() + wn.tobytes()
    res = plugin.compile_layer(accel.LayerDesc("BitNetSwiGLU", "TERNARY", label), blob)
    try:
        out1, out2 = bytearray(res.out_bytes), bytearray(res.out_bytes)
        res.layer.infer(x.tobytes(), out1)
        res.layer.infer(x.tobytes(), out2)
    finally:
        res.layer.release()
    ref = orc.swiglu_forward(g, u, d, x, inner_norm=wn, eps=1e-5, simd=True)
    got1 = np.frombuffer(bytes(out1), np.float32).reshape(M, hidden)
    got2 = np.frombuffer(bytes(out2), np.float32).reshape(M, hidden)
    row = _record("BitNetSwiGLU", label, ref.out, got1, got2, FP32_TOL)
    worst = max(i for i in range(7) if row["hist"][i])
    # strict: loom's sums in loom's order, only exp's last bit is free; fast:
    # the normalized h is within 1 fp32 ulp, and a 1-ulp move of h can move
    # one int8 code of the requantized row (an output step of os * 1)
    assert worst <= (sp.LOWBIT if norm == "strict" else sp.DRIFT), row
    assert row["parity_spec"] in (sp.EXACT, sp.INDUS) and row["det_spec"] == sp.EXACT, row
