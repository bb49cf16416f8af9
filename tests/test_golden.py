"""The committed golden fixtures (tests/golden/) against the CPU oracle and
loom's own known-answer vectors (CPU only).

The fixtures were written by tests/golden/make_golden.py from the oracle; this
test regenerates every case and requires identical bits, so a change to the
oracle that moves any output fails here.  Citations are relative to the loom
v0.83.0 tree.
"""
import json
import os

import numpy as np
import pytest

from tests.golden import make_golden as mg

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name))


@pytest.fixture(scope="module")
def manifest():
    with open(os.path.join(HERE, "manifest.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def kats():
    with open(os.path.join(HERE, "reference_kats.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", list(mg.DENSE_CASES))
def test_dense_fixtures(orc, manifest, name):
    w, x = mg.dense_inputs(name)
    m = manifest["dense"][name]
    assert mg.sha(w.words, np.float32(w.scale), x) == m["inputs_sha256"]
    r = orc.dense_forward(w, x, simd=True)
    assert mg.sha(r.pre) == m["pre_sha256"] and mg.sha(r.acc) == m["acc_sha256"]
    assert mg.sha(r.xq) == m["xq_sha256"]
    # the scalar kernel gives the same integers (poly/tests/bitnet_simd_test.go:13-45)
    s = orc.dense_forward(w, x, simd=False)
    assert np.array_equal(s.acc, r.acc) and np.array_equal(s.pre, r.pre)
    if os.path.exists(os.path.join(HERE, f"dense_{name}.npz")):
        f = load(f"dense_{name}.npz")
        assert np.array_equal(f["pre"], r.pre) and np.array_equal(f["acc"], r.acc)


def test_swiglu_fixture(orc, manifest):
    g, u, d, wn, x = mg.swiglu_inputs()
    assert mg.sha(g.words, u.words, d.words, wn, x) == manifest["swiglu_inputs_sha256"]
    f = load("swiglu_small.npz")
    for act in (mg.ACT_SILU, mg.ACT_RELU2):
        r = orc.swiglu_forward(g, u, d, x, inner_norm=wn, eps=1e-5, activation=act)
        assert np.array_equal(f[f"out_{act}"], r.out) and np.array_equal(f[f"h_{act}"], r.h)


def test_lm_head_fixture(orc, manifest):
    table, x = mg.lm_inputs()
    assert mg.sha(table, x) == manifest["lm_inputs_sha256"]
    f = load("lm_head_dottile.npz")
    for i, row in enumerate(x):
        assert np.array_equal(f["logits"][i], orc.lm_head(row, table, simd=True))
        assert f["ids"][i] == orc.argmax_first(f["logits"][i])


def test_block_fixture(orc, manifest):
    mats, vecs, xs = mg.block_inputs()
    assert mg.sha(*(m.words for m in mats.values()), *vecs.values(), *xs) == manifest["block_inputs_sha256"]
    blk = mg.oracle_block(mats, vecs)
    f = load("block_small.npz")
    for i, x in enumerate(xs):
        assert np.array_equal(f[f"out{i}"], blk.forward(x))


def test_reference_kats(orc, kats):
    k = kats["absmean_quantizer"]
    master = np.array(k["master"], np.float32)
    scale = orc.ternary_scale(master)
    assert abs(scale - k["scale"]) <= 1e-6
    assert [orc.quant_value(v, scale) for v in master] == k["values"]
    k = kats["microsoft_offline_decode"]
    m = orc.pack_ms_offline_bytes(np.array(k["packed"], np.uint8), k["rows"], k["cols"], scale=k["scale"])
    out, _ = orc.matvec_scalar(m, np.array(k["xq"], np.int8), orc.output_scale(m.scale, k["amax"]))
    assert np.allclose(out, k["out"], atol=1e-6, rtol=0)
    k = kats["entity_blob_round_trip"]
    words = np.full(2 * 4, k["word"], np.uint32)
    blob = orc.entity_encode(2, 64, 0, k["scale"], 4, words)
    back, off = orc.entity_decode(blob)
    assert np.array_equal(back.words, words) and back.scale == np.float32(k["scale"]) and off == 0
