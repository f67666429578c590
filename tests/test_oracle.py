"""CPU tests that pin the oracle (oracle/cpu_ref.c) before anything is checked against it.

Three independent pins:
  1. the reference itself: train_bnn.c compiled from /root/reference
     (oracle/_ref, where it exists) must give bit-identical results;
  2. the committed golden fixtures, produced from that same reference build;
  3. mathematics that fixes each op without the loop code: closed forms,
     float64 recomputations with error bounds, invariants and special values.
"""
import json
import os
import subprocess

import numpy as np
import pytest

import gen

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    same = a.view(np.uint32) == b.view(np.uint32)
    same |= np.isnan(a) & np.isnan(b)
    return bool(same.all())


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---- 1. restatement == reference build, bit for bit ---------------------------

SHAPES = [(1, 1, 1), (2, 3, 4), (4, 64, 384), (3, 5, 13), (2, 7, 768)]


@pytest.mark.parametrize("B,T,C", SHAPES)
def test_matches_reference_encoder(oracle, ref_oracle, B, T, C):
    g = gen.rng(1000 + C)
    V = 11
    inp = gen.tokens_uniform(g, B * T, V)
    inp[: min(3, inp.size)] = 4  # repeats
    wte, wpe = gen.normal(g, (V, C), 0, 0.02), gen.normal(g, (T, C), 0, 0.01)
    dout = gen.normal(g, (B, T, C))
    outs = []
    for o in (oracle, ref_oracle):
        out = np.zeros((B, T, C), np.float32)
        o.encoder_forward(out, inp, wte, wpe, B, T, C)
        dwte, dwpe = gen.normal(gen.rng(5), (V, C)), gen.normal(gen.rng(6), (T, C))
        o.encoder_backward(dwte, dwpe, dout, inp, B, T, C)
        outs.append((out, dwte, dwpe))
    for a, b in zip(*outs):
        assert bits_equal(a, b)


@pytest.mark.parametrize("B,T,C", SHAPES)
def test_matches_reference_layernorm(oracle, ref_oracle, B, T, C):
    g = gen.rng(2000 + C)
    x = gen.normal(g, (B, T, C))
    w, b = gen.normal(g, (C,), 1, 0.1), gen.normal(g, (C,), 0, 0.1)
    dout = gen.normal(g, (B, T, C))
    outs = []
    for o in (oracle, ref_oracle):
        out = np.zeros_like(x)
        mean, rstd = np.zeros((B, T), np.float32), np.zeros((B, T), np.float32)
        o.layernorm_forward(out, mean, rstd, x, w, b, B, T, C)
        dinp, dw, db = gen.normal(gen.rng(7), (B, T, C)), gen.normal(gen.rng(8), (C,)), gen.normal(gen.rng(9), (C,))
        o.layernorm_backward(dinp, dw, db, dout, x, w, mean, rstd, B, T, C)
        outs.append((out, mean, rstd, dinp, dw, db))
    for a, b in zip(*outs):
        assert bits_equal(a, b)


@pytest.mark.parametrize("N", [1, 3, 1000, 65537])
def test_matches_reference_elementwise(oracle, ref_oracle, N):
    g = gen.rng(3000 + N)
    x = np.concatenate([gen.normal(g, (N,), 0, 3), gen.special_floats()]).astype(np.float32)
    y = gen.normal(g, x.shape)
    dout = gen.normal(g, x.shape)
    rho = np.concatenate([gen.normal(g, (N,), -5, 0.1), gen.special_floats()]).astype(np.float32)
    n = x.size
    res = []
    for o in (oracle, ref_oracle):
        go = np.zeros(n, np.float32)
        o.gelu_forward(go, x, n)
        gd = gen.normal(gen.rng(10), (n,))
        o.gelu_backward(gd, x, dout, n)
        ro = np.zeros(n, np.float32)
        o.residual_forward(ro, x, y, n)
        dx, dy = gen.normal(gen.rng(11), (n,)), gen.normal(gen.rng(12), (n,))
        o.residual_backward(dx, dy, dout, n)
        w = np.zeros(n, np.float32)
        o.bayes_materialize(w, y, rho, dout, n)
        res.append((go, gd, ro, dx, dy, w))
    for a, b in zip(*res):
        assert bits_equal(a, b)


# ---- 2. restatement == committed fixtures -------------------------------------

def test_golden_metadata():
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        meta = json.load(f)
    assert set(meta["sha256"]) == {"encoder", "layernorm", "gelu", "residual", "materialize", "posterior", "head"}


def test_golden_encoder(oracle):
    d = load("encoder")
    B, T, C = int(d["B"]), int(d["T"]), int(d["C"])
    out = np.zeros_like(d["out"])
    oracle.encoder_forward(out, d["inp"], d["wte"], d["wpe"], B, T, C)
    assert bits_equal(out, d["out"])
    dwte, dwpe = d["dwte0"].copy(), d["dwpe0"].copy()
    oracle.encoder_backward(dwte, dwpe, d["dout"], d["inp"], B, T, C)
    assert bits_equal(dwte, d["dwte"]) and bits_equal(dwpe, d["dwpe"])
    kw, kp = np.zeros_like(d["k_dwte"]), np.zeros_like(d["k_dwpe"])
    oracle.encoder_backward(kw, kp, d["k_dout"], d["k_inp"], 2, 3, 4)
    assert bits_equal(kw, d["k_dwte"]) and bits_equal(kp, d["k_dwpe"])


def test_golden_layernorm(oracle):
    d = load("layernorm")
    B, T, C = int(d["B"]), int(d["T"]), int(d["C"])
    out = np.zeros_like(d["out"])
    mean, rstd = np.zeros_like(d["mean"]), np.zeros_like(d["rstd"])
    oracle.layernorm_forward(out, mean, rstd, d["x"], d["w"], d["b"], B, T, C)
    for a, k in ((out, "out"), (mean, "mean"), (rstd, "rstd")):
        assert bits_equal(a, d[k]), k
    dinp, dw, db = d["dinp0"].copy(), d["dw0"].copy(), d["db0"].copy()
    oracle.layernorm_backward(dinp, dw, db, d["dout"], d["x"], d["w"], d["mean"], d["rstd"], B, T, C)
    for a, k in ((dinp, "dinp"), (dw, "dw"), (db, "db")):
        assert bits_equal(a, d[k]), k


def test_golden_elementwise(oracle):
    d = load("gelu")
    n = d["x"].size
    out = np.zeros(n, np.float32)
    oracle.gelu_forward(out, d["x"], n)
    assert bits_equal(out, d["out"])
    dinp = d["dinp0"].copy()
    oracle.gelu_backward(dinp, d["x"], d["dout"], n)
    assert bits_equal(dinp, d["dinp"])
    r = load("residual")
    n = r["x"].size
    out = np.zeros(n, np.float32)
    oracle.residual_forward(out, r["x"], r["y"], n)
    assert bits_equal(out, r["out"])
    dx, dy = r["dx0"].copy(), r["dy0"].copy()
    oracle.residual_backward(dx, dy, r["dout"], n)
    assert bits_equal(dx, r["dx"]) and bits_equal(dy, r["dy"])
    m = load("materialize")
    w = np.zeros_like(m["w"])
    oracle.bayes_materialize(w, m["mu"], m["rho"], m["eps"], w.size)
    assert bits_equal(w, m["w"])


# ---- 3. mathematics -----------------------------------------------------------

def test_math_encoder_forward_is_one_add(oracle):
    g = gen.rng(41)
    B, T, C, V = 3, 9, 20, 13
    inp = gen.tokens_uniform(g, B * T, V)
    wte, wpe = gen.normal(g, (V, C)), gen.normal(g, (T, C))
    out = np.zeros((B, T, C), np.float32)
    oracle.encoder_forward(out, inp, wte, wpe, B, T, C)
    want = wte[inp.reshape(B, T)] + wpe[None, :, :]  # numpy float32 add: one IEEE add
    assert bits_equal(out, want)


def test_math_encoder_backward_scatter(oracle):
    """Repeated-token case (train_bnn.c:1236-1238): row 5 gets 3 contributions, added in (b,t) order."""
    inp = np.array([5, 2, 5, 0, 5, 6], np.int32)
    dout = gen.normal(gen.rng(42), (2, 3, 4))
    dwte = gen.normal(gen.rng(43), (7, 4))
    dwpe = gen.normal(gen.rng(44), (3, 4))
    w0, p0 = dwte.copy(), dwpe.copy()
    oracle.encoder_backward(dwte, dwpe, dout, inp, 2, 3, 4)
    flat = dout.reshape(6, 4)
    row5 = ((w0[5] + flat[0]) + flat[2]) + flat[4]
    assert bits_equal(dwte[5], row5)
    assert bits_equal(dwte[1], w0[1]) and bits_equal(dwte[3], w0[3])  # untouched rows
    assert bits_equal(dwpe, (p0 + dout[0]) + dout[1])
    # float64 brute force on a larger random case, within the fp32 summation bound
    g = gen.rng(45)
    B, T, C, V = 4, 16, 8, 5
    inp = gen.tokens_uniform(g, B * T, V)
    dout = gen.normal(g, (B, T, C))
    dwte, dwpe = np.zeros((V, C), np.float32), np.zeros((T, C), np.float32)
    oracle.encoder_backward(dwte, dwpe, dout, inp, B, T, C)
    want = np.zeros((V, C))
    np.add.at(want, inp, dout.reshape(-1, C).astype(np.float64))
    bound = B * T * np.finfo(np.float32).eps * np.abs(dout).sum(axis=(0, 1)).max()
    assert np.abs(dwte - want).max() <= bound
    assert np.abs(dwpe - dout.astype(np.float64).sum(0)).max() <= bound


def test_math_layernorm(oracle):
    g = gen.rng(46)
    B, T, C = 2, 8, 384
    x = gen.normal(g, (B, T, C), 0.3, 2.0)
    w = np.ones(C, np.float32)
    b = np.zeros(C, np.float32)
    out = np.zeros_like(x)
    mean, rstd = np.zeros((B, T), np.float32), np.zeros((B, T), np.float32)
    oracle.layernorm_forward(out, mean, rstd, x, w, b, B, T, C)
    xd = x.astype(np.float64)
    m64 = xd.mean(-1)
    v64 = ((xd - m64[..., None]) ** 2).mean(-1)
    assert np.allclose(mean, m64, rtol=1e-5, atol=1e-6)
    assert np.allclose(rstd, 1 / np.sqrt(v64 + 1e-5), rtol=1e-5)
    # gamma=1, beta=0: rows have mean ~0 and mean square v/(v+eps)
    assert np.abs(out.astype(np.float64).mean(-1)).max() < 1e-6
    assert np.allclose((out.astype(np.float64) ** 2).mean(-1), v64 / (v64 + 1e-5), rtol=1e-5)
    # backward: dbias increment is the column sum; sum_c of the dinp increment is ~0
    dout = gen.normal(g, (B, T, C))
    wg = gen.normal(g, (C,), 1, 0.1)
    dinp, dw, db = np.zeros_like(x), np.zeros(C, np.float32), np.zeros(C, np.float32)
    oracle.layernorm_backward(dinp, dw, db, dout, x, wg, mean, rstd, B, T, C)
    assert np.allclose(db, dout.astype(np.float64).sum((0, 1)), rtol=1e-5, atol=1e-5)
    xhat = (xd - mean[..., None]) * rstd[..., None]
    assert np.allclose(dw, (dout * xhat).sum((0, 1)), rtol=1e-4, atol=1e-4)
    assert np.abs(dinp.astype(np.float64).sum(-1)).max() < 1e-4
    dn = dout * wg
    want = rstd[..., None] * (dn - dn.mean(-1, keepdims=True)
                              - xhat * (dn * xhat).mean(-1, keepdims=True))
    assert np.allclose(dinp, want, rtol=1e-4, atol=1e-5)


def test_math_gelu(oracle):
    x = np.concatenate([gen.normal(gen.rng(47), (20000,), 0, 3), np.linspace(-8, 8, 4001)]).astype(np.float32)
    n = x.size
    out = np.zeros(n, np.float32)
    oracle.gelu_forward(out, x, n)
    xd = x.astype(np.float64)
    k = np.float64(np.float32(0.7978845608))
    c = np.float64(np.float32(0.044715))
    want = 0.5 * xd * (1 + np.tanh(k * (xd + c * xd ** 3)))
    scale = 0.5 * np.abs(xd) * 2 + 1e-30
    assert (np.abs(out - want) / scale).max() < 1e-6
    z = np.zeros(3, np.float32)
    oracle.gelu_forward(z, np.zeros(3, np.float32), 3)
    assert (z == 0).all()
    d = np.zeros(1, np.float32)
    oracle.gelu_backward(d, np.zeros(1, np.float32), np.ones(1, np.float32), 1)
    assert d[0] == np.float32(0.5)
    dinp = np.zeros(n, np.float32)
    oracle.gelu_backward(dinp, x, np.ones(n, np.float32), n)
    th = np.tanh(k * (xd + c * xd ** 3))
    dwant = 0.5 * (1 + th) + 0.5 * xd * (1 - th * th) * k * (1 + 3 * c * xd * xd)
    assert np.abs(dinp - dwant).max() < 1e-5


def test_math_materialize(oracle):
    g = gen.rng(48)
    n = 4096
    mu = gen.normal(g, (n,), 0, 0.02)
    eps = gen.normal(g, (n,))
    w = np.zeros(n, np.float32)
    rho = gen.normal(g, (n,), -5, 0.1)
    oracle.bayes_materialize(w, mu, rho, np.zeros(n, np.float32), n)
    assert bits_equal(w, mu)  # eps = 0 -> w = mu exactly
    big = gen.normal(g, (n,), 40, 5).clip(20.5, None).astype(np.float32)
    oracle.bayes_materialize(w, mu, big, eps, n)
    assert bits_equal(w, mu + big * eps)  # rho > 20 -> softplus(rho) = rho
    tiny = np.full(n, -104.5, np.float32)
    oracle.bayes_materialize(w, mu, tiny, eps, n)
    assert bits_equal(w, mu)  # expf underflows to 0, log1pf(0) = 0
    sp = oracle.softplus(rho)
    want = np.log1p(np.exp(rho.astype(np.float64)))
    assert (np.abs(sp - want) / want).max() < 2.5 * np.finfo(np.float32).eps


# ---- the device math replica against the host libm ---------------------------

LIBM_BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "libm_exhaustive")


@pytest.mark.parametrize("fn", ["expf", "log1pf", "expm1f", "tanhf", "softplus", "logf_normal", "logf_normal0",
                                "cosf_small", "logf"])
def test_libm_replica_strided(fn):
    """ugk_libm.h equals glibc on every 1021st bit pattern (the full 2^32 sweep is
    `oracle/libm_exhaustive <fn> 1`; see oracle/Makefile). logf_normal and cosf_small are the
    Box-Muller transform's logf and cosf on their domains (normal x > 0, |x| < 120), with fused
    multiply-adds; logf_normal0 the unfused logf, which gives the same floats; logf the loss's logf
    on every input (zero, subnormal, negative, infinite and NaN included)."""
    if not os.path.exists(LIBM_BIN):
        subprocess.run(["make", "-C", os.path.dirname(LIBM_BIN), "libm_exhaustive"], check=True,
                       capture_output=True)
    r = subprocess.run([LIBM_BIN, fn, "1021", "4"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches=0" in r.stdout
