"""CPU tests that pin the oracle's softmax + cross-entropy forward and backward
(oracle/cpu_ref.c, restating train_bnn.c:279-304 and :358-378).

Pins: the reference build (bit-identical, several shapes and special rows), the committed fixture
tests/golden/head.npz from that build, and mathematics: probabilities are exp(x - max) / sum
against float64, rows sum to 1, the loss is -log of the target's probability, and the backward
row is (p - onehot) / (B*T), summing to zero.
"""
import os

import numpy as np
import pytest

import gen

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def head_inputs(seed, B, T, V, scale=3.0):
    g = gen.rng(seed)
    logits = gen.normal(g, (B, T, V), 0, scale)
    targets = g.integers(0, V, B * T).astype(np.int32)
    return logits, targets


def special_rows(V):
    """Rows that exercise the max rule and the exp range: ties, huge and tiny logits, -inf."""
    rows = [np.zeros(V, np.float32), np.full(V, 80.0, np.float32), np.linspace(-200, 100, V, dtype=np.float32)]
    r = np.full(V, -np.inf, np.float32)
    r[V // 2] = 1.0
    rows.append(r)
    r = np.full(V, -1e31, np.float32)  # below the -1e30 start of the CPU max
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("B,T,V", [(4, 64, 27), (2, 3, 1000), (1, 2, 50257), (1, 3, 60000)])
def test_matches_reference_head(oracle, ref_oracle, B, T, V):
    logits, targets = head_inputs(B * 100 + V, B, T, V)
    sp = special_rows(V)
    logits = np.concatenate([logits.reshape(-1, V), sp]).astype(np.float32)
    rows = logits.shape[0]
    targets = np.concatenate([targets, np.arange(sp.shape[0], dtype=np.int32) * (V // 7)]).astype(np.int32)
    res = []
    for o in (oracle, ref_oracle):
        losses, probs = np.zeros(rows, np.float32), np.zeros_like(logits)
        o.softmax_crossentropy(losses, probs, logits, targets, 1, rows, V)
        d = gen.normal(gen.rng(7), (rows, V))
        o.crossentropy_softmax_backward(d, probs, targets, 1, rows, V)
        res.append((losses, probs, d))
    for a, b in zip(*res):
        assert bits_equal(a, b)


def test_golden_head(oracle):
    with np.load(os.path.join(GOLDEN, "head.npz"), allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    for tag in ("s", "l"):
        B, T, V = (int(x) for x in d[f"{tag}_shape"])
        losses, probs = np.zeros(B * T, np.float32), np.zeros((B, T, V), np.float32)
        oracle.softmax_crossentropy(losses, probs, d[f"{tag}_logits"], d[f"{tag}_targets"], B, T, V)
        assert bits_equal(losses, d[f"{tag}_losses"]) and bits_equal(probs, d[f"{tag}_probs"])
        dl = d[f"{tag}_dlogits0"].copy()
        oracle.crossentropy_softmax_backward(dl, d[f"{tag}_probs"], d[f"{tag}_targets"], B, T, V)
        assert bits_equal(dl, d[f"{tag}_dlogits"])


@pytest.mark.parametrize("V", [27, 50257])
def test_math_softmax_crossentropy(oracle, V):
    """The CPU op is exp(x - max) / (sequential float sum), -logf(p[target]), and (p - onehot)/(B*T):
    rebuilt here from numpy's IEEE float32 arithmetic, the host expf/logf, and a sequential float32
    cumulative sum, it matches bit for bit; against float64 it is within the sequential sum's bound."""
    B, T = 2, 4
    logits, targets = head_inputs(900 + V, B, T, V, scale=5.0)
    losses, probs = np.zeros(B * T, np.float32), np.zeros_like(logits)
    oracle.softmax_crossentropy(losses, probs, logits, targets, B, T, V)
    x = logits.reshape(B * T, V)
    m = x.max(1, keepdims=True)
    e32 = oracle.expf(np.ascontiguousarray(x - m)).reshape(B * T, V)
    s32 = np.add.accumulate(e32, axis=1, dtype=np.float32)[:, -1:]  # sequential, in float32
    p32 = e32 / s32
    assert bits_equal(probs.reshape(B * T, V), p32)
    pt = np.ascontiguousarray(p32[np.arange(B * T), targets])
    assert bits_equal(losses, -oracle.logf(pt))
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    want = e / e.sum(1, keepdims=True)
    gamma = V * np.finfo(np.float32).eps  # bound of a sequential sum of V terms
    assert (np.abs(probs.reshape(B * T, V) - want) <= 2 * gamma * want + 1e-37).all()
    # backward: (p - onehot) * (1/(B*T)), rows sum to ~0
    d = np.zeros_like(logits)
    oracle.crossentropy_softmax_backward(d, probs, targets, B, T, V)
    onehot = np.zeros((B * T, V), np.float32)
    onehot[np.arange(B * T), targets] = 1.0
    assert bits_equal(d.reshape(B * T, V), (p32 - onehot) * (np.float32(1.0) / np.float32(B * T)))
    assert np.abs(d.reshape(B * T, V).astype(np.float64).sum(1)).max() < 2 * gamma / (B * T)


def test_math_softmax_special_rows(oracle):
    V = 64
    logits = special_rows(V)
    rows = logits.shape[0]
    targets = np.full(rows, V // 2, np.int32)
    losses, probs = np.zeros(rows, np.float32), np.zeros_like(logits)
    oracle.softmax_crossentropy(losses, probs, logits, targets, 1, rows, V)
    assert bits_equal(probs[0], np.full(V, np.float32(1.0) / np.float32(V)))  # all-equal row: 1/V each
    assert bits_equal(probs[1], probs[0])                                     # shift invariance at 80
    assert probs[3][V // 2] == 1.0 and (np.delete(probs[3], V // 2) == 0).all() and losses[3] == 0.0
    # every logit below the CPU's -1e30 start: max stays -1e30, exp underflows, 0/0 = nan
    assert np.isnan(probs[4]).all()


def test_shared_divisor_quotient_is_correctly_rounded(tmp_path):
    """The device softmax divides every e of a row by the row's sum s as q = e * y,
    r = fma(-s, q, e), fma(r, y, q) with y = 1 / s (Markstein's correction). On the CPU, with
    IEEE fmaf: equal to e / s for every e in [2^-86, 1] (the kernel's domain for this form; e
    below it takes the division), for divisors with all-ones and near-one significands and
    random ones in [1, 2^16)."""
    import shutil
    import subprocess
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "div_recip_check.c")
    exe = str(tmp_path / "div_recip_check")
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    for flags in (["-mfma", "-fopenmp"], ["-fopenmp"], []):
        if subprocess.run([gcc, "-O2", "-ffp-contract=off", *flags, src, "-o", exe, "-lm"],
                          capture_output=True).returncode == 0:
            break
    else:
        pytest.fail("div_recip_check.c does not build")
    f2u = lambda f: int(np.float32(f).view(np.uint32))
    bs = [1.0, 3.0, 50257.0, 21504.0, 12345.678]
    bs += [float(np.uint32((127 + e) << 23 | m).view(np.float32)) for e in (0, 1, 7, 15)
           for m in (0x7FFFFF, 0x7FFFFE, 0x000001, 0x400001)]
    g = np.random.default_rng(1)
    bs += [float(np.uint32((127 + int(e)) << 23 | int(m)).view(np.float32))
           for e, m in zip(g.integers(0, 16, 12), g.integers(0, 1 << 23, 12))]
    out = subprocess.run([exe] + [hex(f2u(b)) for b in bs], capture_output=True, text=True, check=True).stdout
    assert out.strip().splitlines()[-1] == "0", out
