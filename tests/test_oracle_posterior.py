"""CPU tests that pin the oracle's posterior-update ops (oracle/cpu_ref.c) before the GPU is
checked against them: bayes_backward, kl_forward/backward, adamw_update (train_bnn.c), and the
Philox draw, k_bayes_sample, k_bayes_backward and k_bbb_step_fused of the GPU arms
(gpt2_kernels.cuh:148-192, train_bnn_gpu.cu:93-217).

Pins, as for the layer kernels:
  1. the reference build (oracle/_ref, where it exists) exports bayes_backward, kl_forward,
     kl_backward and adamw_update: bit-identical results;
  2. the committed fixture tests/golden/posterior.npz, produced from that build;
  3. mathematics: the published Random123 known-answer vectors of Philox4x32-10, a float64
     Box-Muller of the same counter words, the u01 end points, the KL gradient as a finite
     difference of the KL, closed forms of AdamW's first step, and the fused step against the
     composition of the unfused ops.
"""
import ctypes
import ctypes.util
import os

import numpy as np
import pytest

import gen

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
_libm.powf.restype = ctypes.c_float


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    same = a.view(np.uint32) == b.view(np.uint32)
    same |= np.isnan(a) & np.isnan(b)
    return bool(same.all())


def bias_corrections(beta1, beta2, t):
    """1 - beta^t with the host powf, as train_bnn.c:704-705 and train_bnn_gpu.cu:487-488."""
    return (np.float32(1.0) - np.float32(_libm.powf(beta1, float(t))),
            np.float32(1.0) - np.float32(_libm.powf(beta2, float(t))))


def posterior_inputs(seed, n):
    g = gen.rng(seed)
    mu = gen.normal(g, (n,), 0, 0.02)
    rho = (g.random(n) * 6.0 - 8.0).astype(np.float32)
    sign = np.where(g.random(n) < 0.5, -1.0, 1.0)
    dw = (sign * 10.0 ** (g.random(n) * 9.0 - 9.0)).astype(np.float32)
    eps = gen.normal(g, (n,))
    m = (dw * gen.normal(g, (n,), 1.0, 0.3)).astype(np.float32)
    v = (m.astype(np.float64) ** 2 * (1.0 + g.random(n))).astype(np.float32)
    return mu, rho, dw, eps, m, v


# ---- 1. restatement == reference build ---------------------------------------

@pytest.mark.parametrize("n", [1, 7, 5000])
def test_matches_reference_posterior(oracle, ref_oracle, n):
    mu, rho, dw, eps, m, v = posterior_inputs(700 + n, n)
    rho[: min(n, 3)] = np.array([25.0, -110.0, 0.0], np.float32)[: min(n, 3)]
    res = []
    for o in (oracle, ref_oracle):
        dmu, drho = gen.normal(gen.rng(1), (n,)), gen.normal(gen.rng(2), (n,))
        o.bayes_backward(dmu, drho, dw, eps, rho, n)
        kl = o.kl_forward(mu, rho, n, 0.1)
        kmu, krho = gen.normal(gen.rng(3), (n,)), gen.normal(gen.rng(4), (n,))
        o.kl_backward(kmu, krho, mu, rho, n, 0.1, 0.25)
        outs = [dmu, drho, kmu, krho]
        for t in (1, 2, 1000):
            p_, m_, v_ = mu.copy(), m.copy(), v.copy()
            o.adamw_update(p_, dw, m_, v_, n, t, 1e-3, 0.9, 0.999, 1e-8, 0.1)
            outs += [p_, m_, v_]
        res.append((kl, outs))
    assert res[0][0] == res[1][0]  # same loop, same double sum
    for a, b in zip(res[0][1], res[1][1]):
        assert bits_equal(a, b)


# ---- 2. restatement == committed fixture --------------------------------------

def test_golden_posterior(oracle):
    with np.load(os.path.join(GOLDEN, "posterior.npz"), allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    n = d["mu"].size
    dmu, drho = d["dmu0"].copy(), d["drho0"].copy()
    oracle.bayes_backward(dmu, drho, d["dw"], d["eps"], d["rho"], n)
    assert bits_equal(dmu, d["dmu"]) and bits_equal(drho, d["drho"])
    assert oracle.kl_forward(d["mu"], d["rho"], n, 0.1) == float(d["kl"])
    kmu, krho = d["dmu0"].copy(), d["drho0"].copy()
    oracle.kl_backward(kmu, krho, d["mu"], d["rho"], n, 0.1, 1.0 / 300000.0)
    assert bits_equal(kmu, d["kmu"]) and bits_equal(krho, d["krho"])
    for t in (1, 7):
        p_, m_, v_ = d["mu"].copy(), d["m0"].copy(), d["v0"].copy()
        oracle.adamw_update(p_, d["dw"], m_, v_, n, t, 3e-4, 0.9, 0.999, 1e-8, 0.01)
        assert bits_equal(p_, d[f"p{t}"]) and bits_equal(m_, d[f"m{t}"]) and bits_equal(v_, d[f"v{t}"])


# ---- 3. mathematics -----------------------------------------------------------

# Random123 kat_vectors, philox4x32 with 10 rounds: (counter, key, output).
PHILOX_KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff),
     (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(oracle, ctr, key, want):
    assert oracle.philox4x32_10(ctr, key).tolist() == list(want)


def test_u01_maps_words_into_the_unit_interval(oracle):
    two32 = np.float32(2.3283064365386963e-10)
    assert two32 == np.float32(2.0 ** -32)
    assert oracle.u01(0) == 0.5 * 2.0 ** -32
    # (float)0xffffffff rounds up to 2^32 and 2^32 + 0.5 rounds back to it: u01 = 1.0 exactly
    assert oracle.u01(0xFFFFFFFF) == 1.0
    for x in (1, 12345, 1 << 24, (1 << 24) + 1, 0x80000001, 0xDEADBEEF):
        want = (np.float32(x) + np.float32(0.5)) * two32
        assert oracle.u01(x) == float(want)


def u01_domain() -> np.ndarray:
    """Every value of u01(x) = ((float)x + 0.5f) * 2^-32 over x in [0, 2^32), ascending.

    (float)x is exact below 2^24 and rounds to the binade's step above. Adding 0.5 is exact
    below 2^23; in [2^23, 2^24) it ties and rounds to the even neighbour; above 2^24 it vanishes.
    The scaling by 2^-32 is exact.
    """
    lo = np.arange(1 << 23, dtype=np.float64) + 0.5
    mid = np.arange(1 << 23, 1 << 24, 2, dtype=np.float64)
    parts = [lo, mid]
    for e in range(24, 32):
        parts.append(np.arange(1 << 23, dtype=np.float64) * 2.0 ** (e - 23) + 2.0 ** e)
    parts.append(np.array([2.0 ** 32]))
    return (np.concatenate(parts) * 2.0 ** -32).astype(np.float32)


def test_u01_domain_is_the_image_of_u01(oracle):
    u = u01_domain()
    assert u.size == 79_691_777 and (np.diff(u) > 0).all()
    assert u[0] == oracle.u01(0) and u[-1] == oracle.u01(0xFFFFFFFF) == 1.0
    g = gen.rng(806)
    xs = np.concatenate([g.integers(0, 1 << 32, 20000, dtype=np.uint64),
                         np.arange((1 << 23) - 8, (1 << 23) + 8), np.arange((1 << 24) - 8, (1 << 24) + 8)])
    vals = np.array([oracle.u01(int(x)) for x in xs], np.float32)
    pos = np.searchsorted(u, vals)
    assert (u[np.minimum(pos, u.size - 1)] == vals).all()


def box_muller64(oracle, seed, step, index):
    """float64 Box-Muller of the same counter words (u1, u2 and theta rounded as in float)."""
    ctr = (index & 0xFFFFFFFF, index >> 32, step & 0xFFFFFFFF, 0)
    key = (seed & 0xFFFFFFFF, seed >> 32)
    w = oracle.philox4x32_10(ctr, key)
    u1, u2 = np.float32(oracle.u01(int(w[0]))), np.float32(oracle.u01(int(w[1])))
    theta = np.float32(np.float32(6.28318530717958647692) * u2)
    return np.sqrt(-2.0 * np.log(np.float64(u1))) * np.cos(np.float64(theta))


@pytest.mark.parametrize("seed,step", [(1234, 1), (0xDEADBEEFCAFEF00D, 7), (0, 0)])
def test_philox_normal_is_box_muller_of_the_stream(oracle, seed, step):
    idx = list(range(0, 512)) + [(1 << 32) + 5, (1 << 40) + 77, 123456789]
    eps = np.array([oracle.philox_normal(seed, step, i) for i in idx], np.float32)
    want = np.array([box_muller64(oracle, seed, step, i) for i in idx])
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert (np.abs(eps - want) <= 4 * ulp + 1e-12).all()
    # the bulk fill is the same function of the index
    assert bits_equal(oracle.philox_normal_n(512, seed, step), eps[:512])
    assert bits_equal(oracle.philox_normal_n(1, seed, step, (1 << 32) + 5), eps[512:513])


def test_philox_normal_moments(oracle):
    eps = oracle.philox_normal_n(1 << 20, 42, 3).astype(np.float64)
    n = eps.size
    assert abs(eps.mean()) < 5.0 / np.sqrt(n)
    assert abs(eps.var() - 1.0) < 5.0 * np.sqrt(2.0 / n)
    assert abs((np.abs(eps) < 1.0).mean() - 0.682689) < 0.003
    # different steps and seeds are different streams
    assert not np.array_equal(oracle.philox_normal_n(64, 42, 3), oracle.philox_normal_n(64, 42, 4))
    assert not np.array_equal(oracle.philox_normal_n(64, 42, 3), oracle.philox_normal_n(64, 43, 3))


def test_sample_and_backward_compose_from_the_stream(oracle):
    n = 3000
    mu, rho, dw, _, _, _ = posterior_inputs(801, n)
    eps = oracle.philox_normal_n(n, 99, 5)
    w, e = np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.bayes_sample_philox(w, e, mu, rho, n, 99, 5)
    want = np.zeros(n, np.float32)
    oracle.bayes_materialize(want, mu, rho, eps, n)
    assert bits_equal(e, eps) and bits_equal(w, want)
    w2 = np.zeros(n, np.float32)
    oracle.bayes_sample_philox(w2, None, mu, rho, n, 99, 5)
    assert bits_equal(w2, w)
    a_mu, a_rho = gen.normal(gen.rng(5), (n,)), gen.normal(gen.rng(6), (n,))
    b_mu, b_rho = a_mu.copy(), a_rho.copy()
    oracle.bayes_backward_philox(a_mu, a_rho, dw, rho, n, 99, 5)
    oracle.bayes_backward(b_mu, b_rho, dw, eps, rho, n)
    assert bits_equal(a_mu, b_mu) and bits_equal(a_rho, b_rho)


def test_bayes_backward_math(oracle):
    n = 2048
    g = gen.rng(802)
    dw, eps = gen.normal(g, (n,)), gen.normal(g, (n,))
    dmu, drho = np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.bayes_backward(dmu, drho, dw, eps, np.zeros(n, np.float32), n)
    assert bits_equal(dmu, dw)
    assert bits_equal(drho, (dw * eps) * np.float32(0.5))  # sigmoid(0) = 1/2 exactly
    rho = gen.normal(g, (n,), -5, 1)
    drho[:] = 0
    oracle.bayes_backward(dmu, drho, dw, eps, rho, n)
    want = dw.astype(np.float64) * eps * (1.0 / (1.0 + np.exp(-rho.astype(np.float64))))
    assert np.allclose(drho, want, rtol=4 * 2.0 ** -23, atol=0)


def test_kl_gradient_is_the_derivative_of_kl(oracle):
    n, sp = 6, 0.1
    g = gen.rng(803)
    mu = gen.normal(g, (n,), 0, 0.05)
    rho = np.array([-6.0, -4.0, -2.5, -2.25, 0.0, 1.5], np.float32)
    dmu, drho = np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.kl_backward(dmu, drho, mu, rho, n, sp, 1.0)
    for i in range(n):
        for arr, grad in ((mu, dmu), (rho, drho)):
            h = np.float32(1e-3) * max(np.float32(1.0), abs(arr[i]))
            a, b = arr.copy(), arr.copy()
            a[i] += h
            b[i] -= h
            args = (a, rho) if arr is mu else (mu, a)
            argsb = (b, rho) if arr is mu else (mu, b)
            fd = (oracle.kl_forward(*args, n, sp) - oracle.kl_forward(*argsb, n, sp)) / (float(a[i]) - float(b[i]))
            assert abs(fd - grad[i]) <= 2e-3 * abs(fd) + 1e-6, (i, fd, grad[i])
    # zero at sigma = sp: rho with softplus(rho) = sp gives dsigma = 0 up to rounding
    r = np.float32(np.log(np.expm1(sp)))
    d2mu, d2rho = np.zeros(1, np.float32), np.zeros(1, np.float32)
    oracle.kl_backward(d2mu, d2rho, np.zeros(1, np.float32), np.array([r], np.float32), 1, sp, 1.0)
    assert d2mu[0] == 0.0 and abs(d2rho[0]) < 1e-4
    # the KL of the prior against itself is 0
    assert abs(oracle.kl_forward(np.zeros(1, np.float32), np.array([r], np.float32), 1, sp)) < 1e-6


def test_adamw_first_step_closed_form(oracle):
    n = 4096
    g = gen.rng(804)
    p = gen.normal(g, (n,), 0, 0.02)
    grad = gen.normal(g, (n,), 0, 1e-2)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    lr, wd = 1e-3, 0.1
    p1 = p.copy()
    oracle.adamw_update(p1, grad, m, v, n, 1, lr, 0.9, 0.999, 1e-8, wd)
    # t = 1: m_hat = g and v_hat = g^2, so the step is lr * (g / (|g| + eps) + wd * p)
    g64, p64 = grad.astype(np.float64), p.astype(np.float64)
    want = p64 - lr * (g64 / (np.abs(g64) + 1e-8) + wd * p64)
    assert np.abs(p1 - want).max() <= 4e-6 * lr + np.spacing(np.float32(0.1))
    assert bits_equal(m, (np.float32(1.0) - np.float32(0.9)) * grad)  # (1 - beta1) rounded in float
    # a zero gradient with wd = 0 leaves the parameter alone
    p2, m2, v2 = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.adamw_update(p2, np.zeros(n, np.float32), m2, v2, n, 3, lr, 0.9, 0.999, 1e-8, 0.0)
    assert bits_equal(p2, p)


@pytest.mark.parametrize("klw", [0.0, 1.0 / 300000.0])
def test_fused_step_is_the_composition(oracle, klw):
    """k_bbb_step_fused == sample of step+1 after (bayes_backward, kl_backward, AdamW x 2)."""
    n, seed, step = 4000, 77, 12
    sp, lr, b1, b2, aeps, wd = 0.1, 3e-4, 0.9, 0.999, 1e-8, 0.0
    mu, rho, dw, _, m, v = posterior_inputs(805, n)
    m_mu, v_mu, m_rho, v_rho = m.copy(), v.copy(), (m * 0.5).astype(np.float32), (v * 0.25).astype(np.float32)
    bc1, bc2 = bias_corrections(b1, b2, step)
    # fused
    f = [a.copy() for a in (mu, rho, m_mu, v_mu, m_rho, v_rho)]
    fw, fdw = np.zeros(n, np.float32), dw.copy()
    oracle.bbb_step_fused(*f, fw, fdw, n, seed, step, sp, klw, bc1, bc2, lr, b1, b2, aeps, wd)
    # composed from the unfused ops
    dmu, drho = np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.bayes_backward_philox(dmu, drho, dw, rho, n, seed, step)
    if klw > 0:
        oracle.kl_backward(dmu, drho, mu, rho, n, sp, klw)
    c_mu, c_rho = mu.copy(), rho.copy()
    c = [m_mu.copy(), v_mu.copy(), m_rho.copy(), v_rho.copy()]
    oracle.adamw_update(c_mu, dmu, c[0], c[1], n, step, lr, b1, b2, aeps, wd)
    oracle.adamw_update(c_rho, drho, c[2], c[3], n, step, lr, b1, b2, aeps, wd)
    cw = np.zeros(n, np.float32)
    oracle.bayes_sample_philox(cw, None, c_mu, c_rho, n, seed, step + 1)
    for a, b in zip(f + [fw], [c_mu, c_rho] + c + [cw]):
        assert bits_equal(a, b)
    assert (fdw == 0).all()
