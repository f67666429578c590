"""GPU: the softmax + cross-entropy exact mode (ugk_set_softmax_exact(1)) against the CPU oracle, bit for
bit.

train_bnn.c:286-301 takes the row max, adds expf(x - max) one logit after another, divides each
exponential by that sum and takes -logf of the target's probability. The default kernels add the row
in a fixed tree (within float rounding of the CPU); in exact mode the library keeps the CPU's order
(one serial chain per row), so every probability and loss equals the oracle's, which is itself
bit-identical to train_bnn.c compiled here, and the reference build's golden fixture. Covered: row
counts on and off the 32-row workgroups, V on and off the 240-logit tiles (27 to 60,000, GPT-2's
50,257), special rows (uniform, shifted, -inf, NaN, +inf, all below the CPU's -1e30 start), 2,048 rows
of 50,257, the golden fixture, and the switch restoring the default kernels.
"""
import os

import numpy as np
import pytest
import torch

from test_head_gpu import bits_equal, dev, host
from test_oracle_head import head_inputs, special_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"


def assert_bits(got, want, what):
    g = np.ascontiguousarray(got, np.float32).ravel()
    c = np.ascontiguousarray(want, np.float32).ravel()
    bad = np.nonzero((g.view(np.uint32) != c.view(np.uint32)) & ~(np.isnan(g) & np.isnan(c)))[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {g.size} differ; first at {i}: gpu {g[i]!r} cpu {c[i]!r}")


class softmax_exact:
    def __init__(self, gpu):
        self.gpu = gpu

    def __enter__(self):
        self.gpu.set_softmax_exact(True)

    def __exit__(self, *a):
        self.gpu.set_softmax_exact(False)


def run(gpu, logits, targets, B, T, V):
    rows = B * T
    tp, tl = torch.empty(rows * V, device=DEV), torch.empty(rows, device=DEV)
    with softmax_exact(gpu):
        gpu.softmax_crossentropy(tl, tp, dev(logits), dev(targets), B, T, V)
    return host(tp).reshape(rows, V), host(tl)


def oracle_forward(oracle, logits, targets, B, T, V):
    cp, cl = np.zeros((B * T, V), np.float32), np.zeros(B * T, np.float32)
    oracle.softmax_crossentropy(cl, cp, np.ascontiguousarray(logits.reshape(B * T, V)), targets, B, T, V)
    return cp, cl


@pytest.mark.parametrize("B,T,V", [(4, 64, 27), (2, 3, 1000), (1, 5, 50257), (2, 3, 4097), (1, 3, 60000),
                                   (3, 2, 64), (1, 33, 240), (1, 32, 241), (2, 50, 239), (1, 1, 1), (1, 65, 480),
                                   (1, 3, 51393)])
def test_softmax_exact(gpu, oracle, B, T, V):
    print(f"softmax exact: B={B} T={T} V={V}", flush=True)
    logits, targets = head_inputs(B * 1000 + T * 10 + V, B, T, V)
    logits = logits.reshape(B * T, V)
    gp, gl = run(gpu, logits, targets, B, T, V)
    cp, cl = oracle_forward(oracle, logits, targets, B, T, V)
    assert_bits(gp, cp, f"probs B={B} T={T} V={V}")
    assert_bits(gl, cl, f"losses B={B} T={T} V={V}")


def nonfinite_rows(V):
    """A NaN among ordinary logits, a +inf among them, +inf and -inf together, and +-0 maxima."""
    g = np.random.default_rng(V)
    rows = []
    for pos, val in ((V // 3, np.nan), (V // 5, np.inf)):
        r = g.normal(0, 3, V).astype(np.float32)
        r[pos] = val
        rows.append(r)
    r = np.full(V, -np.inf, np.float32)
    r[0], r[-1] = np.inf, -1.0
    rows.append(r)
    r = np.full(V, -5.0, np.float32)
    r[1::2] = -0.0
    r[::3] = 0.0
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("V", [64, 50257])
def test_softmax_exact_special_rows(gpu, oracle, V):
    logits = np.concatenate([special_rows(V), nonfinite_rows(V)]).astype(np.float32)
    rows = logits.shape[0]
    targets = np.full(rows, V // 2, np.int32)
    gp, gl = run(gpu, logits, targets, 1, rows, V)
    cp, cl = oracle_forward(oracle, logits, targets, 1, rows, V)
    assert_bits(gp, cp, f"special rows probs, V={V}")
    assert_bits(gl, cl, f"special rows losses, V={V}")


def test_softmax_exact_gpt2_rows(gpu, oracle):
    B, T, V = 2, 1024, 50257
    print(f"softmax exact at {B * T} rows of {V}", flush=True)
    logits, targets = head_inputs(4242, B, T, V)
    logits = logits.reshape(B * T, V)
    gp, gl = run(gpu, logits, targets, B, T, V)
    cp, cl = oracle_forward(oracle, logits, targets, B, T, V)
    assert_bits(gp, cp, "probs, 2048 x 50257")
    assert_bits(gl, cl, "losses, 2048 x 50257")


def test_softmax_exact_golden_fixture(gpu):
    d = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "head.npz"))
    for p in ("s_", "l_"):
        B, T, V = (int(v) for v in d[p + "shape"])
        gp, gl = run(gpu, d[p + "logits"].reshape(B * T, V), d[p + "targets"], B, T, V)
        assert_bits(gp, d[p + "probs"], f"golden probs {p}")
        assert_bits(gl, d[p + "losses"], f"golden losses {p}")


def test_softmax_exact_switch_restores_default(gpu, oracle):
    B, T, V = 1, 4, 50257
    logits, targets = head_inputs(77, B, T, V)
    logits = logits.reshape(B * T, V)
    tl, tt = dev(logits), dev(targets)
    outs = []
    for exact in (False, True, False):
        gpu.set_softmax_exact(exact)
        try:
            tp, tlo = torch.empty(B * T * V, device=DEV), torch.empty(B * T, device=DEV)
            gpu.softmax_crossentropy(tlo, tp, tl, tt, B, T, V)
            outs.append(host(tp))
        finally:
            gpu.set_softmax_exact(False)
    assert not gpu.softmax_exact()
    assert bits_equal(outs[0], outs[2])
    cp, _ = oracle_forward(oracle, logits, targets, B, T, V)
    assert_bits(outs[1].reshape(B * T, V), cp, "exact probs")
    assert not bits_equal(outs[0], outs[1]), "the default tree sum should differ from the serial one somewhere"
