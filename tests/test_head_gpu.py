"""GPU parity of softmax + cross-entropy forward and backward (train_bnn.c:279-304, :358-378)
against the CPU oracle.

Bars:
  * backward: bit-exact, given the same probabilities;
  * forward: the exponentials are glibc's bit for bit and only the row sum's order differs (a
    fixed tree on the GPU, sequential on the CPU), so per row every prob_gpu / prob_cpu is the same
    number up to 2 ulp (one division each), the GPU's probabilities and losses are at least as close
    to a float64 softmax as the CPU's, and both are within the sequential-sum bound 2 V eps of each
    other; the forward is deterministic. The literal 1e-5 bar is reported: at V = 50257 the CPU's own
    sequential fp32 sum is off by up to ~1e-4 relative, so it cannot hold against the CPU.
"""
import numpy as np
import pytest
import torch

import gen
import literal_bar
from test_oracle_head import head_inputs, special_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = float(np.finfo(np.float32).eps)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def check_forward(gpu_p, gpu_l, cpu_p, cpu_l, logits, targets):
    rows, V = cpu_p.shape
    finite = np.isfinite(cpu_p).all(1)
    gp, cp = gpu_p[finite].astype(np.float64), cpu_p[finite].astype(np.float64)
    # the ratio test runs over normal-range probabilities (subnormal quotients are quantised)
    nz = cp > 1e-30
    assert (gp[nz] > 0).all()
    ratio = np.where(nz, gp / np.where(nz, cp, 1.0), 1.0)
    rmax = np.where(nz, ratio, -np.inf).max(1)
    rmin = np.where(nz, ratio, np.inf).min(1)
    assert (rmax - rmin <= 4 * EPS * rmax).all(), float((rmax - rmin).max())
    x = logits[finite].astype(np.float64)
    e = np.exp(x - x.max(1, keepdims=True))
    want = e / e.sum(1, keepdims=True)
    gamma = V * EPS
    assert (np.abs(gp - cp) <= 2 * gamma * cp + 1e-37).all()
    err_g = (np.abs(gp - want) / np.maximum(want, 1e-30)).max()
    err_c = (np.abs(cp - want) / np.maximum(want, 1e-30)).max()
    assert err_g <= err_c + 4 * EPS, (err_g, err_c)
    l64 = -np.log(want[np.arange(want.shape[0]), targets[finite]])
    gl, cl = gpu_l[finite].astype(np.float64), cpu_l[finite].astype(np.float64)
    assert np.abs(gl - l64).max() <= np.abs(cl - l64).max() + 4 * EPS * np.abs(l64).max() + 1e-7
    literal = float((np.abs(gp - cp) <= 1e-6 + 1e-5 * cp).mean())
    literal_bar.record(f"softmax_crossentropy probs, V = {V}, {rows} rows", literal)
    print(f"V={V}: max rel error vs float64: GPU {err_g:.3g}, CPU {err_c:.3g}")


@pytest.mark.parametrize("B,T,V", [(4, 64, 27), (2, 3, 1000), (1, 5, 50257), (2, 3, 4097), (1, 3, 60000),
                                   (3, 2, 64), (1, 4, 16385), (1, 3, 51137), (1, 3, 51393), (1, 3, 51394), (1, 2, 32706), (2, 2, 961)])
def test_softmax_crossentropy(gpu, oracle, B, T, V):
    logits, targets = head_inputs(B * 1000 + T * 10 + V, B, T, V)
    logits = logits.reshape(B * T, V)
    rows = B * T
    tl, tt = dev(logits), dev(targets)
    outs = []
    for _ in range(2):
        tp, tlo = torch.empty(rows * V, device=DEV), torch.empty(rows, device=DEV)
        gpu.softmax_crossentropy(tlo, tp, tl, tt, B, T, V)
        outs.append((host(tp).reshape(rows, V), host(tlo)))
    assert bits_equal(outs[0][0], outs[1][0]) and bits_equal(outs[0][1], outs[1][1]), "not deterministic"
    cp, cl = np.zeros_like(logits), np.zeros(rows, np.float32)
    oracle.softmax_crossentropy(cl, cp, logits, targets, B, T, V)
    check_forward(outs[0][0], outs[0][1], cp, cl, logits, targets)
    # backward from the CPU's probabilities: bit-exact
    d0 = gen.normal(gen.rng(V), (rows, V), 0, 1e-3)
    td = dev(d0)
    gpu.crossentropy_softmax_backward(td, dev(cp), tt, B, T, V)
    d = d0.copy()
    oracle.crossentropy_softmax_backward(d, cp, targets, B, T, V)
    assert bits_equal(host(td).reshape(rows, V), d)


@pytest.mark.parametrize("V", [64, 50257])
def test_softmax_special_rows(gpu, oracle, V):
    logits = special_rows(V)
    rows = logits.shape[0]
    targets = np.full(rows, V // 2, np.int32)
    tp, tlo = torch.empty(rows * V, device=DEV), torch.empty(rows, device=DEV)
    gpu.softmax_crossentropy(tlo, tp, dev(logits), dev(targets), 1, rows, V)
    cp, cl = np.zeros_like(logits), np.zeros(rows, np.float32)
    oracle.softmax_crossentropy(cl, cp, logits, targets, 1, rows, V)
    gp = host(tp).reshape(rows, V)
    assert bits_equal(gp[0], cp[0]) and bits_equal(gp[1], cp[1])  # uniform rows: exact
    assert bits_equal(gp[3], cp[3]) and host(tlo)[3] == cl[3] == 0.0  # one finite logit
    assert np.isnan(gp[4]).all() and np.isnan(cp[4]).all()            # all below -1e30
    check_forward(gp, host(tlo), cp, cl, logits, targets)


@pytest.mark.parametrize("V", [961, 32706, 50257, 51393])
def test_softmax_loss_at_row_edges(gpu, oracle, V):
    """Targets at the first and last logit of rows with every start offset mod 64 (the kernels
    lay a row on the threads from a 256-byte boundary of probs, so the thread holding the
    target depends on the row's offset): the loss is -log of the stored probability."""
    rows = 66
    logits, _ = head_inputs(V + 7, 1, rows, V)
    logits = logits.reshape(rows, V)
    targets = np.where(np.arange(rows) % 2 == 0, 0, V - 1).astype(np.int32)
    tp, tlo = torch.empty(rows * V, device=DEV), torch.empty(rows, device=DEV)
    gpu.softmax_crossentropy(tlo, tp, dev(logits), dev(targets), 1, rows, V)
    gp, gl = host(tp).reshape(rows, V), host(tlo)
    pt = gp[np.arange(rows), targets].astype(np.float64)
    assert bits_equal(gl, (-np.log(pt)).astype(np.float32))
    cp, cl = np.zeros_like(logits), np.zeros(rows, np.float32)
    oracle.softmax_crossentropy(cl, cp, logits, targets, 1, rows, V)
    check_forward(gp, gl, cp, cl, logits, targets)


def test_softmax_ragged_and_empty(gpu):
    t = torch.zeros(8, device=DEV)
    gpu.softmax_crossentropy(t, t, t, torch.zeros(4, dtype=torch.int32, device=DEV), 0, 4, 2)  # B = 0
    # target 4 >= V: replaced on the device and reported by the next synchronize
    gpu.softmax_crossentropy(torch.empty(2, device=DEV), torch.empty(8, device=DEV), torch.zeros(8, device=DEV),
                             torch.tensor([0, 4], dtype=torch.int32, device=DEV), 1, 2, 4)
    with pytest.raises(gpu.UgkError):
        gpu.synchronize()


def test_full_cfg5_head(gpu, oracle):
    """GPT-2-124M head shape, B=8 T=1024 V=50257 (412M logits): sampled rows against the oracle,
    every row's probabilities summing to 1, and the backward's row sums to 0."""
    B, T, V = 8, 1024, 50257
    rows = B * T
    g = torch.Generator(DEV).manual_seed(5)
    logits = torch.randn(rows * V, device=DEV, generator=g) * 3.0
    targets = torch.randint(0, V, (rows,), device=DEV, dtype=torch.int32, generator=g)
    probs, losses = torch.empty_like(logits), torch.empty(rows, device=DEV)
    gpu.softmax_crossentropy(losses, probs, logits, targets, B, T, V)
    pv = probs.view(rows, V)
    assert torch.allclose(pv.double().sum(1), torch.ones(rows, dtype=torch.float64, device=DEV), atol=1e-5)
    pick = np.unique(np.concatenate([np.random.default_rng(3).integers(0, rows, 24), [0, rows - 1]]))
    ti = torch.from_numpy(pick).to(DEV)
    lg = host(logits.view(rows, V)[ti])
    tg = host(targets[ti])
    cp, cl = np.zeros_like(lg), np.zeros(pick.size, np.float32)
    oracle.softmax_crossentropy(cl, cp, lg, tg, 1, pick.size, V)
    check_forward(host(pv[ti]), host(losses[ti]), cp, cl, lg, tg)
    dl = torch.zeros_like(logits)
    gpu.crossentropy_softmax_backward(dl, probs, targets, B, T, V)
    rs = dl.view(rows, V).double().sum(1)
    assert rs.abs().max().item() < 1e-5 / rows
    # the CPU loop's arithmetic on these rows: 0 + (p - onehot) * (1.0f / (B*T)), in float32
    p_rows = host(pv[ti])
    onehot = np.zeros_like(p_rows)
    onehot[np.arange(pick.size), tg] = 1.0
    d = np.float32(0.0) + (p_rows - onehot) * (np.float32(1.0) / np.float32(rows))
    assert bits_equal(host(dl.view(rows, V)[ti]), d)


@pytest.mark.parametrize("B,T,V", [(8, 1024, 50257), (2, 3, 1000), (3, 5, 27), (1, 7, 50257), (2, 2, 3)])
def test_crossentropy_backward_zeroed(gpu, B, T, V):
    """crossentropy_softmax_backward_zeroed over garbage == crossentropy_softmax_backward over zeros,
    bit for bit (float4 stream and dword paths: V = 27 and 3 take the latter)."""
    rows = B * T
    g = torch.Generator(DEV).manual_seed(rows + V)
    probs = torch.rand(rows * V, device=DEV, generator=g)
    targets = torch.randint(0, V, (rows,), device=DEV, dtype=torch.int32, generator=g)
    want = torch.zeros(rows * V, device=DEV)
    gpu.crossentropy_softmax_backward(want, probs, targets, B, T, V)
    got = torch.randn(rows * V, device=DEV, generator=g) * 5.0
    gpu.crossentropy_softmax_backward_zeroed(got, probs, targets, B, T, V)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
