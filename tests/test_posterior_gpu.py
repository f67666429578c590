"""GPU parity of the posterior-update ops of libugk.so (called through the C-ABI) against the
CPU oracle: bayes_backward, kl_backward, adamw_update (bit-exact), kl_forward (double; within
summation-order rounding with ugk_set_kl_exact(1), within the bar its softplus implies by
default), and the Philox ops (bayes_sample, bayes_backward_philox,
bbb_step_fused).

The Philox ops split into an exact part and a float part:
  * the integer stream (Philox4x32-10 and u01) is bit-exact, checked on the device against the
    Random123 known-answer vectors and the oracle;
  * the Box-Muller transform takes glibc's logf and cosf (restated in ugk_libm.h; the glibc-exact
    form) or its radius from the hardware log2 and square root and the device library's cosf (the
    default form). Over every u01 value the stream can produce (all 79,691,777 of them) and every
    angle 2 pi u01 the restated logf and cosf equal the host glibc bit for bit, so in the
    glibc-exact form eps is the oracle's bit for bit; by default it is within 8 ulp of it;
  * with ugk_set_philox_exact(1), every output of every Philox op equals the oracle's bit for bit
    (the fused step included), and each Philox op equals its eps-taking twin fed the same eps;
  * by default the Philox ops take their softplus and sigmoid in the hardware-transcendental form,
    which is within the literal bar |a - b| <= 1e-6 + 1e-5 |b| of the glibc-exact form on every
    float input (exhaustive, below); downstream of eps they are held to the bar that follows from
    it (the form's bar times |eps| or |dw eps|, plus the rounding of the products and sums), and
    the fused step equals the composition of the unfused ops in the same form bit for bit.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest
import torch

import gen
from test_oracle_posterior import PHILOX_KAT, bias_corrections, posterior_inputs, u01_domain

pytestmark = pytest.mark.gpu

DEV = "cuda"
CFG5_N = 124_439_808  # GPT-2-124M with a tied head: param_offsets total at C=768 L=12 V=50257


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def assert_bits(g, c, what):
    g = np.ascontiguousarray(g, np.float32).ravel()
    c = np.ascontiguousarray(c, np.float32).ravel()
    bad = np.nonzero((g.view(np.uint32) != c.view(np.uint32)) & ~(np.isnan(g) & np.isnan(c)))[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {g.size} differ; first at {i}: gpu {g[i]!r} cpu {c[i]!r}")


def ordered(a):
    """float32 bit patterns as integers that increase with the value (ulp distances)."""
    i = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFFFFFF), i)


def ulp_dist(a, b):
    return np.abs(ordered(a) - ordered(b))


def assert_eps_close(g, c, what, max_ulp=8):
    g = np.asarray(g, np.float32)
    c = np.asarray(c, np.float32)
    d = ulp_dist(g, c)
    exact = float((d == 0).mean())
    print(f"{what}: {exact:.4%} bit-exact, max {int(d.max())} ulp over {d.size}")
    assert d.max() <= max_ulp, (what, int(d.max()), int(np.argmax(d)))
    if d.size >= 1000:  # a wrong mapping of the stream would match almost nowhere
        assert exact > 0.5, (what, exact)


# ---- the integer stream ---------------------------------------------------------------

def test_philox_device_known_answers_and_oracle(gpu, oracle):
    g = gen.rng(901)
    rand = g.integers(0, 1 << 32, size=(4096, 6), dtype=np.uint64).astype(np.uint32)
    kat = np.array([list(c) + list(k) for c, k, _ in PHILOX_KAT], np.uint32)
    tuples = np.concatenate([kat, rand])
    out = torch.empty(tuples.shape[0] * 4, dtype=torch.int32, device=DEV)
    gpu.diag_philox(out, dev(tuples.view(np.int32)))
    got = host(out).view(np.uint32).reshape(-1, 4)
    for i, (_, _, want) in enumerate(PHILOX_KAT):
        assert got[i].tolist() == list(want)
    want = np.array([oracle.philox4x32_10(t[:4], t[4:]) for t in tuples], np.uint32)
    assert (got == want).all()


# ---- the float transform over its whole input domain ------------------------------------

def test_device_logf_cosf_over_the_u01_domain(gpu, oracle):
    """The glibc-exact form's logf and cosf on the device (ugk_libm.h's restatements of glibc's) equal
    the host glibc on every u01 value the stream can produce and on every angle fl(2 pi u) of them:
    the Box-Muller transform's whole domain. The device library's own logf and cosf (variant 1) are
    printed for comparison (within 2 ulp)."""
    u = u01_domain()
    theta = np.float32(6.28318530717958647692) * u
    for fn, x, want in (("logf", u, oracle.logf(u)), ("cosf", theta, oracle.cosf(theta))):
        tx = dev(x)
        out = torch.empty_like(tx)
        gpu.diag_math_eval(fn, out, tx, 0)
        assert_bits(host(out), want, f"device {fn} (glibc restatement) vs host glibc over {x.size} inputs")
        gpu.diag_math_eval(fn, out, tx, 1)
        d = ulp_dist(host(out), want)
        print(f"device library {fn} vs glibc over {x.size} inputs: {(d == 0).mean():.4%} identical, "
              f"{int((d == 1).sum())} at 1 ulp, max {int(d.max())} ulp")
        assert d.max() <= 2, (fn, int(d.max()), float(x[np.argmax(d)]))
        del tx, out


@pytest.mark.parametrize("fn", ["logf", "cosf"])
def test_device_logf_cosf_strided_over_their_domains(gpu, oracle, fn):
    """The restated logf on every 61st bit pattern (zero, subnormal, negative, infinite and NaN
    inputs included: the softmax loss takes it on any probability) and cosf on every 61st float of
    |x| < 120 (the domains of the restatements, which the CPU checks against glibc on every input)
    equal the host glibc on the device too."""
    if fn == "logf":
        x = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
        x = np.concatenate([x, np.array([0, 0x80000000, 1, 0x007FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000],
                                        np.uint32)]).view(np.float32)
        want = oracle.logf(x)
    else:
        top = int(np.array([120.0], np.float32).view(np.uint32)[0])
        pos = np.arange(0, top, 61, dtype=np.uint64).astype(np.uint32)
        x = np.concatenate([pos, pos | np.uint32(0x80000000)]).view(np.float32)
        want = oracle.cosf(x)
    tx = dev(x)
    out = torch.empty_like(tx)
    gpu.diag_math_eval(fn, out, tx, 0)
    assert_bits(host(out), want, f"device {fn} (glibc restatement) vs host glibc, {x.size} inputs")


def test_device_sqrtf_is_correctly_rounded_everywhere(gpu, oracle):
    n, first = gpu.diag_math_mismatch("sqrtf")
    assert n == 0, hex(first)
    g = gen.rng(902)
    x = np.abs(np.concatenate([gen.normal(g, (1 << 20,), 0, 1e3), gen.special_floats()])).astype(np.float32)
    tx = dev(x)
    out = torch.empty_like(tx)
    gpu.diag_math_eval("sqrtf", out, tx)
    assert_bits(host(out), oracle.sqrtf(x), "sqrtf vs host")


@pytest.fixture
def philox_exact(gpu):
    """The glibc-exact softplus/sigmoid in the Philox ops for the duration of a test."""
    gpu.set_philox_exact(True)
    try:
        yield
    finally:
        gpu.set_philox_exact(False)


@pytest.mark.parametrize("fn", ["softplus_fast", "sigmoid_fast"])
def test_fast_transcendentals_exhaustive(gpu, fn):
    """The Philox ops' default softplus and sigmoid against the glibc-exact forms (train_bnn.c:814-816,
    :820-822) on all 2^32 float inputs: none outside the literal bar, and none more than 8 ulp away
    (the largest distance found is 5 ulp for both)."""
    assert not gpu.philox_exact()  # the default form
    n, first = gpu.diag_math_mismatch(fn)
    assert n == 0, (fn, n, hex(first))
    d, at = gpu.diag_math_ulp(fn)
    x = np.array([at], np.uint32).view(np.float32)[0]
    print(f"{fn}: 0 inputs outside the literal bar; at most {d} ulp from the glibc-exact form (at x = {x!r})")
    assert d <= 8, (fn, d, hex(at))  # 5 on MI355X


@pytest.mark.parametrize("fn", ["cosf_small"])
def test_box_muller_math_is_the_device_library(gpu, fn):
    """The default form's Box-Muller cosf (for 0 <= x < 2^17) is the device library's sequence without
    its cases for other arguments: the same bits as the library's cosf on every one of the 2^32 float
    inputs (the library's function outside that domain). The angle fl(2 pi u2) lies in (0, 2 pi]."""
    n, first = gpu.diag_math_mismatch(fn)
    assert n == 0, (fn, n, hex(first))


@pytest.mark.parametrize("fn", ["bm_radius_fast", "bm_radius"])
def test_box_muller_radius_ulp(gpu, fn):
    """The radius sqrt(-2 ln u1) of the Box-Muller transform on every float u1 in [2^-33, 1] (a superset
    of u01's image) against the double radius rounded to float: the default form (hardware log2 and
    square root) and the glibc-exact form (glibc's logf, the correctly rounded root). Both are within
    2 ulp on MI355X (the rounding of -2 ln u1 carries through the root)."""
    lo = int(np.array([2.0 ** -33], np.float32).view(np.uint32)[0])
    hi = int(np.array([1.0], np.float32).view(np.uint32)[0])
    d, at = gpu.diag_math_ulp(fn, lo, hi - lo + 1)
    x = np.array([at], np.uint32).view(np.float32)[0]
    print(f"{fn}: at most {d} ulp from the correctly rounded radius (at u1 = {x!r})")
    assert d <= 2, (fn, d, x)


# ---- the ops ----------------------------------------------------------------------------

SIZES = [1, 3, 5, 4096 + 3, (1 << 20) + 1]


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("offset", [0, 1])
def test_bayes_backward_kl_backward_adamw(gpu, oracle, n, offset):
    mu, rho, dw, eps, m, v = posterior_inputs(910 + n, n)
    rho[: min(n, 3)] = np.array([25.0, -110.0, 0.0], np.float32)[: min(n, 3)]
    big = lambda a: dev(np.concatenate([np.zeros(offset, np.float32), a]))[offset:]
    dmu0, drho0 = gen.normal(gen.rng(1), (n,), 0, 1e-3), gen.normal(gen.rng(2), (n,), 0, 1e-3)
    t_mu, t_rho, t_dw, t_eps = big(mu), big(rho), big(dw), big(eps)
    t_dmu, t_drho = big(dmu0), big(drho0)
    gpu.bayes_backward(t_dmu, t_drho, t_dw, t_eps, t_rho, n)
    dmu, drho = dmu0.copy(), drho0.copy()
    oracle.bayes_backward(dmu, drho, dw, eps, rho, n)
    assert_bits(host(t_dmu), dmu, "bayes_backward dmu")
    assert_bits(host(t_drho), drho, "bayes_backward drho")
    k_dmu, k_drho = big(dmu0), big(drho0)
    gpu.kl_backward(k_dmu, k_drho, t_mu, t_rho, n, 0.1, 1.0 / 300000.0)
    dmu, drho = dmu0.copy(), drho0.copy()
    oracle.kl_backward(dmu, drho, mu, rho, n, 0.1, 1.0 / 300000.0)
    assert_bits(host(k_dmu), dmu, "kl_backward dmu")
    assert_bits(host(k_drho), drho, "kl_backward drho")
    for t in (1, 7, 1000):
        tp, tm, tv = big(mu), big(m), big(v)
        gpu.adamw_update(tp, t_dw, tm, tv, n, t, 3e-4, 0.9, 0.999, 1e-8, 0.01)
        p_, m_, v_ = mu.copy(), m.copy(), v.copy()
        oracle.adamw_update(p_, dw, m_, v_, n, t, 3e-4, 0.9, 0.999, 1e-8, 0.01)
        assert_bits(host(tp), p_, f"adamw t={t} params")
        assert_bits(host(tm), m_, f"adamw t={t} m")
        assert_bits(host(tv), v_, f"adamw t={t} v")


def test_golden_posterior_on_gpu(gpu, oracle):
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "posterior.npz")
    with np.load(path, allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    n = d["mu"].size
    t_dmu, t_drho = dev(d["dmu0"]), dev(d["drho0"])
    gpu.bayes_backward(t_dmu, t_drho, dev(d["dw"]), dev(d["eps"]), dev(d["rho"]), n)
    assert_bits(host(t_dmu), d["dmu"], "golden bayes_backward dmu")
    assert_bits(host(t_drho), d["drho"], "golden bayes_backward drho")
    k_dmu, k_drho = dev(d["dmu0"]), dev(d["drho0"])
    gpu.kl_backward(k_dmu, k_drho, dev(d["mu"]), dev(d["rho"]), n, 0.1, 1.0 / 300000.0)
    assert_bits(host(k_dmu), d["kmu"], "golden kl_backward dmu")
    assert_bits(host(k_drho), d["krho"], "golden kl_backward drho")
    gpu.set_kl_exact(True)
    try:
        kl = gpu.kl_forward(dev(d["mu"]), dev(d["rho"]), n, 0.1)
    finally:
        gpu.set_kl_exact(False)
    assert abs(kl - float(d["kl"])) <= 1e-12 * abs(float(d["kl"]))
    kl = gpu.kl_forward(dev(d["mu"]), dev(d["rho"]), n, 0.1)
    assert abs(kl - float(d["kl"])) <= kl_fast_bar(oracle, d["rho"], 0.1) + 1e-12 * abs(float(d["kl"]))
    for t in (1, 7):
        tp, tm, tv = dev(d["mu"]), dev(d["m0"]), dev(d["v0"])
        gpu.adamw_update(tp, dev(d["dw"]), tm, tv, n, t, 3e-4, 0.9, 0.999, 1e-8, 0.01)
        assert_bits(host(tp), d[f"p{t}"], f"golden adamw t={t}")
        assert_bits(host(tm), d[f"m{t}"], f"golden adamw m t={t}")
        assert_bits(host(tv), d[f"v{t}"], f"golden adamw v t={t}")


@pytest.fixture
def kl_exact(gpu):
    """The glibc-exact softplus in kl_forward for the duration of a test."""
    gpu.set_kl_exact(True)
    try:
        yield
    finally:
        gpu.set_kl_exact(False)


KL_FAST_ULP = 8  # the fast softplus against the glibc-exact one, over every float input (fn 66)


def kl_fast_terms_bar(oracle, rho, sp):
    """Per term, how far the default form's KL term may lie from train_bnn.c's. The default form's
    sigma' = sigma (1 + d) with |d| <= 8 ulp / sigma <= 8 * 2^-23 while rho >= -80 (sigma a normal
    float); the term log(sp/sigma) + (sigma^2 + mu^2)/(2 sp^2) - 1/2 then moves by
    -log(1 + d) + sigma^2 (2 d + d^2)/(2 sp^2), at most |d| (1 + sigma^2/sp^2) to first order (the
    factor 1.001 covers the second). Below -80 the exact form is taken: no difference."""
    sigma, _ = oracle_softplus_sigmoid(oracle, np.ascontiguousarray(rho, np.float32))
    d = KL_FAST_ULP * 2.0 ** -23
    return np.where(np.asarray(rho) >= -80.0, 1.001 * d * (1.0 + sigma ** 2 / np.float64(sp) ** 2), 0.0)


def kl_fast_bar(oracle, rho, sp):
    return float(kl_fast_terms_bar(oracle, rho, sp).sum())


def shifted(a, offset):
    """a on the device, starting `offset` floats past a 16-byte boundary (offset 1: the scalar path)."""
    return dev(np.concatenate([np.zeros(offset, np.float32), a]))[offset:]


@pytest.mark.parametrize("n", [1, 1000, 5_000_003])
@pytest.mark.parametrize("offset", [0, 1])
def test_kl_forward(gpu, oracle, kl_exact, n, offset):
    mu, rho, _, _, _, _ = posterior_inputs(920 + n, n)
    want = oracle.kl_forward(mu, rho, n, 0.1)
    tm, tr = shifted(mu, offset), shifted(rho, offset)
    got = gpu.kl_forward(tm, tr, n, 0.1)
    assert abs(got - want) <= 1e-10 * abs(want), (got, want)
    assert gpu.kl_forward(tm, tr, n, 0.1) == got  # fixed summation order
    assert gpu.kl_forward(tm, tr, 0, 0.1) == 0.0


@pytest.mark.parametrize("n", [1, 1000, 5_000_003])
@pytest.mark.parametrize("offset", [0, 1])
def test_kl_forward_fast(gpu, oracle, n, offset):
    """The default form (hardware-transcendental softplus) against train_bnn.c's KL: within the sum
    of the per-term bars above plus the exact form's summation-order bar, deterministic, and within
    the literal bar |a - b| <= 1e-6 + 1e-5 |b|."""
    assert not gpu.kl_exact()
    mu, rho, _, _, _, _ = posterior_inputs(920 + n, n)
    want = oracle.kl_forward(mu, rho, n, 0.1)
    tm, tr = shifted(mu, offset), shifted(rho, offset)
    got = gpu.kl_forward(tm, tr, n, 0.1)
    bar = kl_fast_bar(oracle, rho, 0.1)
    print(f"kl_forward n={n} offset={offset}: default form {abs(got - want):.3g} from train_bnn.c "
          f"(bar {bar:.3g}, {abs(got - want) / abs(want):.3g} relative)")
    assert abs(got - want) <= bar + 1e-10 * abs(want), (got, want, bar)
    assert abs(got - want) <= 1e-6 + 1e-5 * abs(want), (got, want)
    assert gpu.kl_forward(tm, tr, n, 0.1) == got  # fixed summation order
    assert gpu.kl_forward(tm, tr, 0, 0.1) == 0.0


@pytest.mark.parametrize("exact", [False, True])
def test_kl_forward_nonfinite_terms(gpu, oracle, exact):
    """A term that is not finite decides the total in both forms, as in train_bnn.c's sum: sigma = 0
    (rho = -inf, or below about -104) gives +inf, sigma = +inf (rho = +inf) and NaN give NaN; a NaN
    term wins over an infinite one. Everything else in the vector is ordinary."""
    n = 4099
    mu, rho, _, _, _, _ = posterior_inputs(977, n)
    cases = {"rho=-inf": {17: -np.inf}, "rho=-200": {4000: -200.0}, "rho=+inf": {5: np.inf},
             "rho=nan": {2048: np.nan}, "mu=inf": {-1: None}, "-inf and nan": {3: -np.inf, 4097: np.nan}}
    gpu.set_kl_exact(exact)
    try:
        for name, edits in cases.items():
            m, r = mu.copy(), rho.copy()
            for k, v in edits.items():
                if v is None:
                    m[k] = np.inf
                else:
                    r[k] = v
            want = oracle.kl_forward(m, r, n, 0.1)
            got = gpu.kl_forward(dev(m), dev(r), n, 0.1)
            assert (np.isnan(got) and np.isnan(want)) or got == want, (name, got, want)
            assert not np.isfinite(want), (name, want)
    finally:
        gpu.set_kl_exact(False)


def kl_term_inputs():
    rho = [-200.0, -104.0, -100.0, -90.0, -88.0, -80.5, -79.5, -50.0, -5.0, -1.0, 0.0, 0.5, 5.0, 20.0,
           20.5, 100.0, 1e30]
    g = gen.rng(77)
    rho += list(np.log(np.expm1(np.float64(1.0) + (np.arange(128) + g.random(128)) / 128.0)).astype(np.float32))
    rho += list(gen.normal(g, (64,), -5.0, 3.0))
    mu = gen.normal(g, (len(rho),), 0, 0.05)
    return mu, np.array(rho, np.float32)


def test_kl_forward_terms(gpu, oracle, kl_exact):
    """Single KL terms across the range of sigma = softplus(rho): subnormal and zero sigma
    (rho below -87 and -103), the x > 20 shortcut, every cell of the logarithm's table
    (sigma with all 128 leading fraction patterns), against the oracle's double terms."""
    mu, rho = kl_term_inputs()
    for k in range(len(rho)):
        want = oracle.kl_forward(mu[k:k + 1], rho[k:k + 1], 1, 0.1)
        got = gpu.kl_forward(dev(mu[k:k + 1]), dev(rho[k:k + 1]), 1, 0.1)
        if np.isinf(want):
            assert got == want, (k, rho[k], got, want)
        else:
            assert abs(got - want) <= 1e-14 * max(1.0, abs(want)), (k, rho[k], got, want)


def test_kl_forward_terms_fast(gpu, oracle):
    """The same single terms in the default form: within the per-term bar where rho >= -80, and the
    exact form's term below (subnormal and zero sigma, where a few ulp would be a large share of
    sigma, take the glibc-exact softplus)."""
    mu, rho = kl_term_inputs()
    bars = kl_fast_terms_bar(oracle, rho, 0.1)
    worst = 0.0
    for k in range(len(rho)):
        want = oracle.kl_forward(mu[k:k + 1], rho[k:k + 1], 1, 0.1)
        got = gpu.kl_forward(dev(mu[k:k + 1]), dev(rho[k:k + 1]), 1, 0.1)
        if np.isinf(want):
            assert got == want, (k, rho[k], got, want)
            continue
        err = abs(got - want)
        if rho[k] >= -80.0:
            worst = max(worst, err / bars[k])
        assert err <= bars[k] + 1e-14 * max(1.0, abs(want)), (k, rho[k], got, want, bars[k])
    print(f"kl_forward single terms, default form: at most {worst:.3f} of the per-term bar")


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("offset", [0, 1])
def test_bayes_sample_and_backward_philox(gpu, oracle, philox_exact, n, offset):
    seed, step = 0x1234_5678_9ABC, 17
    mu, rho, dw, _, _, _ = posterior_inputs(930 + n, n)
    big = lambda a: dev(np.concatenate([np.zeros(offset, np.float32), a]))[offset:]
    t_mu, t_rho, t_dw = big(mu), big(rho), big(dw)
    t_w, t_eps, t_w2 = big(np.zeros(n, np.float32)), big(np.zeros(n, np.float32)), big(np.zeros(n, np.float32))
    gpu.bayes_sample(t_w, t_eps, t_mu, t_rho, n, seed, step)
    gpu.bayes_sample(t_w2, None, t_mu, t_rho, n, seed, step)
    eps_dev = host(t_eps)
    assert_bits(eps_dev, oracle.philox_normal_n(n, seed, step), f"eps n={n}")
    # downstream of eps: bit-exact
    w = np.zeros(n, np.float32)
    oracle.bayes_materialize(w, mu, rho, eps_dev, n)
    assert_bits(host(t_w), w, "bayes_sample w")
    assert_bits(host(t_w2), w, "bayes_sample w (no eps output)")
    dmu0, drho0 = gen.normal(gen.rng(3), (n,), 0, 1e-3), gen.normal(gen.rng(4), (n,), 0, 1e-3)
    t_dmu, t_drho = big(dmu0), big(drho0)
    gpu.bayes_backward_philox(t_dmu, t_drho, t_dw, t_rho, n, seed, step)
    dmu, drho = dmu0.copy(), drho0.copy()
    oracle.bayes_backward(dmu, drho, dw, eps_dev, rho, n)
    assert_bits(host(t_dmu), dmu, "bayes_backward_philox dmu")
    assert_bits(host(t_drho), drho, "bayes_backward_philox drho")


@pytest.mark.parametrize("klw", [0.0, 1.0 / 300000.0])
@pytest.mark.parametrize("n,offset", [(5, 0), (4096 + 3, 1), ((1 << 20) + 1, 0)])
def test_bbb_step_fused(gpu, oracle, philox_exact, klw, n, offset):
    seed, step = 77, 12
    sp, lr, b1, b2, aeps, wd = 0.1, 3e-4, 0.9, 0.999, 1e-8, 0.0
    mu, rho, dw, _, m, v = posterior_inputs(940 + n, n)
    state = [mu, rho, m, v, (m * 0.5).astype(np.float32), (v * 0.25).astype(np.float32)]
    bc1, bc2 = bias_corrections(b1, b2, step)
    big = lambda a: dev(np.concatenate([np.zeros(offset, np.float32), a]))[offset:]
    f = [big(a) for a in state]
    f_w, f_dw = big(np.zeros(n, np.float32)), big(dw)
    gpu.bbb_step_fused(*f, f_w, f_dw, n, seed, step, sp, klw, float(bc1), float(bc2), lr, b1, b2, aeps, wd)
    # the device's own unfused ops, fed the same Philox stream: bit-identical
    c_mu, c_rho, c_m1, c_v1, c_m2, c_v2 = (big(a) for a in state)
    g_mu, g_rho = big(np.zeros(n, np.float32)), big(np.zeros(n, np.float32))
    t_dw = big(dw)
    gpu.bayes_backward_philox(g_mu, g_rho, t_dw, c_rho, n, seed, step)
    if klw > 0:
        gpu.kl_backward(g_mu, g_rho, c_mu, c_rho, n, sp, klw)
    gpu.adamw_update(c_mu, g_mu, c_m1, c_v1, n, step, lr, b1, b2, aeps, wd)
    gpu.adamw_update(c_rho, g_rho, c_m2, c_v2, n, step, lr, b1, b2, aeps, wd)
    c_w, c_eps = big(np.zeros(n, np.float32)), big(np.zeros(n, np.float32))
    gpu.bayes_sample(c_w, c_eps, c_mu, c_rho, n, seed, step + 1)
    names = ("mu", "rho", "m_mu", "v_mu", "m_rho", "v_rho", "w")
    for name, a, b in zip(names, f + [f_w], [c_mu, c_rho, c_m1, c_v1, c_m2, c_v2, c_w]):
        assert_bits(host(a), host(b), f"fused vs unfused {name}")
    assert (host(f_dw) == 0).all()
    # and against the oracle's fused step (the same eps): bit-exact
    o = [a.copy() for a in state]
    o_w, o_dw = np.zeros(n, np.float32), dw.copy()
    oracle.bbb_step_fused(*o, o_w, o_dw, n, seed, step, sp, klw, bc1, bc2, lr, b1, b2, aeps, wd)
    for name, a, b in zip(names, f + [f_w], o + [o_w]):
        assert_bits(host(a), b, f"fused {name} vs oracle")
    assert (o_dw == 0).all()


def test_full_cfg5_bayes_sample(gpu, oracle, philox_exact):
    """The sample at GPT-2-124M size: indices up to 124M map to the oracle's stream."""
    n, seed, step = CFG5_N, 0xC0FFEE, 3
    g = gen.rng(950)
    mu = torch.empty(n, device=DEV).normal_(0, 0.02, generator=torch.Generator(DEV).manual_seed(1))
    rho = torch.empty(n, device=DEV).normal_(-5, 0.1, generator=torch.Generator(DEV).manual_seed(2))
    w = torch.empty(n, device=DEV)
    eps = torch.empty(n, device=DEV)
    gpu.bayes_sample(w, eps, mu, rho, n, seed, step)
    torch.cuda.synchronize()
    idx = np.unique(np.concatenate([g.integers(0, n, 200_000), np.arange(n - 1000, n), np.arange(1000)]))
    ti = torch.from_numpy(idx).to(DEV)
    e_dev = host(eps[ti])
    e_ref = np.array([oracle.philox_normal(seed, step, int(i)) for i in idx[:20000]], np.float32)
    assert_bits(e_dev[:20000], e_ref, "cfg5 eps (sampled)")
    w_ref = np.zeros(idx.size, np.float32)
    oracle.bayes_materialize(w_ref, host(mu[ti]), host(rho[ti]), e_dev, idx.size)
    assert_bits(host(w[ti]), w_ref, "cfg5 w (sampled)")
    mean, var = float(eps.double().mean()), float(eps.double().var())
    assert abs(mean) < 5.0 / np.sqrt(n) and abs(var - 1.0) < 5.0 * np.sqrt(2.0 / n), (mean, var)


# ---- the default (hardware-transcendental) form of the Philox ops ------------------------

EPS32 = float(np.finfo(np.float32).eps)


def oracle_softplus_sigmoid(oracle, rho):
    """softplus(rho) and sigmoid(rho) as train_bnn.c computes them (materialize with mu = 0, eps = 1;
    bayes_backward with dw = eps = 1 from zero)."""
    n = rho.size
    one, zero = np.ones(n, np.float32), np.zeros(n, np.float32)
    sp = np.zeros(n, np.float32)
    oracle.bayes_materialize(sp, zero, rho, one, n)
    dmu, sg = zero.copy(), zero.copy()
    oracle.bayes_backward(dmu, sg, one, one, rho, n)
    return sp.astype(np.float64), sg.astype(np.float64)


def assert_within(got, want, bar, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    bad = ~((np.abs(got - want) <= bar) | (np.isnan(got) & np.isnan(want)) | (got == want))
    if bad.any():
        i = int(np.argmax(bad))
        raise AssertionError(f"{what}: {int(bad.sum())} of {got.size} outside the bar; first at {i}: "
                             f"gpu {got[i]!r} want {want[i]!r} bar {bar.flat[i] if np.ndim(bar) else bar!r}")


@pytest.mark.parametrize("n", [5, 4096 + 3, (1 << 20) + 1])
def test_bayes_sample_and_backward_philox_fast(gpu, oracle, n):
    """w = mu + softplus(rho) eps and drho += dw eps sigmoid(rho) with the fast forms, against the
    oracle's eps-taking ops fed with the device's eps, within the bar the forms' own bar implies;
    rho spans the special values as well as the benchmark's -5 +- 0.1."""
    seed, step = 0x1234_5678_9ABC, 17
    mu, rho, dw, _, _, _ = posterior_inputs(960 + n, n)
    sp_ = gen.special_floats()
    rho[: min(n, sp_.size)] = sp_[: min(n, sp_.size)]
    t_mu, t_rho, t_dw = dev(mu), dev(rho), dev(dw)
    t_w, t_eps = torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)
    gpu.bayes_sample(t_w, t_eps, t_mu, t_rho, n, seed, step)
    eps = host(t_eps)
    assert_eps_close(eps, oracle.philox_normal_n(n, seed, step), f"eps n={n} (fast form)")
    w_ref = np.zeros(n, np.float32)
    oracle.bayes_materialize(w_ref, mu, rho, eps, n)
    sp, sg = oracle_softplus_sigmoid(oracle, rho)
    e64, m64, w64 = eps.astype(np.float64), mu.astype(np.float64), w_ref.astype(np.float64)
    # |sp_fast - sp| <= 1e-6 + 1e-5 sp, times |eps|, plus one rounding of the product and one of the sum
    bar = np.abs(e64) * (1e-6 + 1e-5 * sp) + EPS32 * (np.abs(sp * e64) + np.abs(w64)) + 1e-45
    assert_within(host(t_w), w_ref, bar, "bayes_sample w (fast form)")
    dmu0, drho0 = gen.normal(gen.rng(5), (n,), 0, 1e-3), gen.normal(gen.rng(6), (n,), 0, 1e-3)
    t_dmu, t_drho = dev(dmu0), dev(drho0)
    gpu.bayes_backward_philox(t_dmu, t_drho, t_dw, t_rho, n, seed, step)
    dmu, drho = dmu0.copy(), drho0.copy()
    oracle.bayes_backward(dmu, drho, dw, eps, rho, n)
    assert_bits(host(t_dmu), dmu, "bayes_backward_philox dmu (no transcendental)")
    g64 = np.abs(dw.astype(np.float64) * e64)
    bar = g64 * (1e-6 + 1e-5 * sg) + EPS32 * (2 * g64 * sg + np.abs(drho.astype(np.float64))) + 1e-45
    assert_within(host(t_drho), drho, bar, "bayes_backward_philox drho (fast form)")


@pytest.mark.parametrize("klw", [0.0, 1.0 / 300000.0])
def test_bbb_step_fused_fast(gpu, oracle, klw):
    """The fused step in the fast form equals the device's unfused sequence in the same form bit for
    bit when it has no KL term (bayes_backward_philox, two adamw_update, bayes_sample at step + 1);
    with the KL term, whose standalone op keeps the glibc-exact form, it is compared with the
    oracle's fused step as the exact form is (mu exactly; rho and the rho moments within 1e-5)."""
    n, seed, step = 4096 + 3, 77, 12
    sp, lr, b1, b2, aeps, wd = 0.1, 3e-4, 0.9, 0.999, 1e-8, 0.0
    mu, rho, dw, _, m, v = posterior_inputs(970, n)
    state = [mu, rho, m, v, (m * 0.5).astype(np.float32), (v * 0.25).astype(np.float32)]
    bc1, bc2 = bias_corrections(b1, b2, step)
    f = [dev(a) for a in state]
    f_w, f_dw = torch.zeros(n, device=DEV), dev(dw)
    gpu.bbb_step_fused(*f, f_w, f_dw, n, seed, step, sp, klw, float(bc1), float(bc2), lr, b1, b2, aeps, wd)
    assert (host(f_dw) == 0).all()
    if klw == 0.0:
        c_mu, c_rho, c_m1, c_v1, c_m2, c_v2 = (dev(a) for a in state)
        g_mu, g_rho = torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)
        gpu.bayes_backward_philox(g_mu, g_rho, dev(dw), c_rho, n, seed, step)
        gpu.adamw_update(c_mu, g_mu, c_m1, c_v1, n, step, lr, b1, b2, aeps, wd)
        gpu.adamw_update(c_rho, g_rho, c_m2, c_v2, n, step, lr, b1, b2, aeps, wd)
        c_w = torch.zeros(n, device=DEV)
        gpu.bayes_sample(c_w, None, c_mu, c_rho, n, seed, step + 1)
        names = ("mu", "rho", "m_mu", "v_mu", "m_rho", "v_rho", "w")
        for name, a, b in zip(names, f + [f_w], [c_mu, c_rho, c_m1, c_v1, c_m2, c_v2, c_w]):
            assert_bits(host(a), host(b), f"fused vs unfused {name} (fast form)")
    o = [a.copy() for a in state]
    o_w, o_dw = np.zeros(n, np.float32), dw.copy()
    oracle.bbb_step_fused(*o, o_w, o_dw, n, seed, step, sp, klw, bc1, bc2, lr, b1, b2, aeps, wd)
    assert_bits(host(f[0]), o[0], "fused mu vs oracle (fast form)")
    for name, a, b in zip(("rho", "m_rho", "v_rho"), (f[1], f[4], f[5]), (o[1], o[4], o[5])):
        assert np.allclose(host(a), b, rtol=1e-5, atol=1e-7 * float(np.abs(b).max())), name
