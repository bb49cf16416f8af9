"""The screened greedy head's bound, checked on the CPU (no GPU).

The head (loom_amd/csrc/block.hip, lm_screen_kernel) keeps per vocab row an
int8 code row q and a scale s = fp32(max|w| / 127), sums A = s * sum_j x_j q_j
(an fp32 multiply-add chain per row, then one fp64 product) and claims

    |F - A| <= B = (k1 * s * X1 + 2^-24 * (|A| + s * X1) + 2^-150) * (1 + 2^-20),
    k1 = 1/2 + 2^-14 + 127 (g32 + g64) (1 + 2^-10),  X1 = sum_j |x_j|,

for loom's fp32 logit F (applyFP32LMHeadRows, poly/transformer.go:664-719;
the oracle's `lm_head`).  This restates the codes and the bound with numpy and
checks the inequality row by row on random tables and on rows built to
nearly reach it: every entry half a code step from its code, with x of the
error's sign, makes |F - A| about s * X1 / 2, so a coefficient below 1/2 fails
here.  The fp32 chain is emulated with an fp64 sum rounded to fp32 at each
step (within a relative 2^-24 (1 + 2^-29) of the fused step, which the bound's
g32 covers).
"""
import numpy as np
import pytest


def _codes(w):
    """Per-row scale (fp32 division) and codes, as lm_quant_rows_kernel forms them."""
    m = np.abs(w).max(axis=1).astype(np.float32)
    s = (m / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint((w / s[:, None]).astype(np.float32))
    r = np.where(s[:, None] == 0, 0, r)
    return s, np.clip(r, -127, 127).astype(np.int8)


def _screen(x, s, q):
    """A and B per row, in the kernel's arithmetic."""
    n = x.size
    g32 = (n + 64) * 2.0 ** -24 / (1 - (n + 64) * 2.0 ** -24)
    g64 = (n + 64) * 2.0 ** -53 / (1 - (n + 64) * 2.0 ** -53)
    k1 = 0.5 + 2.0 ** -14 + 127 * (g32 + g64) * (1 + 2.0 ** -10)
    a = np.zeros(q.shape[0], np.float32)
    xq = x.astype(np.float64)[None, :] * q.astype(np.float64)  # exact products
    for j in range(n):  # column order, one chain per row
        a = (a.astype(np.float64) + xq[:, j]).astype(np.float32)
    x1 = float(np.abs(x.astype(np.float64)).sum())
    sd = s.astype(np.float64)
    A = sd * a.astype(np.float64)
    sx = sd * x1
    B = (k1 * sx + 2.0 ** -24 * (np.abs(A) + sx) + 2.0 ** -150) * (1 + 2.0 ** -20)
    return A, B


@pytest.mark.parametrize("case", ["normal", "heavy", "mixed_scales", "adversarial"])
def test_screen_bound_holds(orc, case):
    rng = np.random.default_rng(17)
    vocab, hidden = 600, 256
    x = rng.standard_normal(hidden).astype(np.float32)
    if case == "normal":
        w = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float32)
    elif case == "heavy":  # a few large entries per row stretch the scale
        w = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float32)
        w[np.arange(vocab), rng.integers(0, hidden, vocab)] *= np.float32(40)
        x = (rng.standard_cauchy(hidden).clip(-50, 50)).astype(np.float32)
    elif case == "mixed_scales":  # rows from 1e-30 to 1e30
        w = (rng.standard_normal((vocab, hidden))
             * (10.0 ** rng.uniform(-30, 30, vocab))[:, None]).astype(np.float32)
        x = (rng.standard_normal(hidden) * 1e-3).astype(np.float32)
    else:  # every entry half a code step from its code, x of the error's sign
        s0 = np.float32(0.02)
        k = rng.integers(-126, 126, (vocab, hidden)).astype(np.float64)
        w = ((k + 0.4999) * np.float64(s0)).astype(np.float32)
        w[:, 0] = np.float32(127 * s0)  # pins the row maximum, hence the scale
        s, q = _codes(w)
        e = w.astype(np.float64) - s.astype(np.float64)[:, None] * q
        x = (np.sign(e[0]) * rng.uniform(0.5, 1.5, hidden)).astype(np.float32)
        w = np.tile(w[:1], (vocab, 1))  # every row the same: the worst row everywhere
    s, q = _codes(w)
    A, B = _screen(x, s, q)
    F = orc.lm_head(x, w, simd=True).astype(np.float64)
    ratio = np.abs(F - A) / B
    print(f"  {case}: max |F - A| / B = {ratio.max():.4f}", flush=True)
    assert np.isfinite(ratio).all()
    assert (np.abs(F - A) <= B).all()
    if case == "adversarial":
        assert ratio.max() > 0.9  # the bound's main term is nearly reached
