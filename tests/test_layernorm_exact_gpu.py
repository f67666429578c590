"""GPU: the LayerNorm exact mode (ugk_set_layernorm_exact(1)) against the CPU oracle, bit for bit.

train_bnn.c:81-115 and :439-477 sum each row one column at a time and dweight/dbias one row at a
time; in exact mode the library keeps those orders (serial chains, one per lane), so every output
(out, mean, rstd, dinp, dweight, dbias) equals the oracle's, which is itself bit-identical to
train_bnn.c compiled here. Covered: ragged shapes (rows a multiple of the 60-row workgroups and the
240-row column tiles or not, C a multiple of the 64-column tiles or not, C a multiple of 4, which
takes the float4 kernels, or not, a single element), misaligned buffers (the scalar kernels), the
benchmark shapes (8,192 and 16,384 rows of 768), backward accumulation into nonzero gradients,
the fused entry points (as the two reference ops in sequence), the allocation-free backward, the
golden fixture written by the reference build, and the mode switch restoring the default kernels.
"""
import os

import numpy as np
import pytest
import torch

import gen
from test_parity_gpu import assert_bits as _assert_bits, dev, host

pytestmark = pytest.mark.gpu
DEV = "cuda"


def assert_bits(got, want, what):
    _assert_bits(np.ravel(got), np.ravel(want), what)


class ln_exact:
    """Run a block with the LayerNorm exact mode on, then restore the default."""

    def __init__(self, gpu):
        self.gpu = gpu

    def __enter__(self):
        self.gpu.set_layernorm_exact(True)

    def __exit__(self, *a):
        self.gpu.set_layernorm_exact(False)


def put(a, offset=0):
    flat = np.concatenate([np.zeros(offset, np.float32), np.ascontiguousarray(a, np.float32).ravel()])
    return dev(flat)[offset:]


def inputs(B, T, C, seed):
    g = gen.rng(seed)
    x = gen.normal(g, (B, T, C), 0.3, 1.7)
    w, b = gen.normal(g, (C,), 1, 0.1), gen.normal(g, (C,), 0, 0.1)
    dout = gen.normal(g, (B, T, C))
    dinp0, dw0, db0 = gen.normal(g, (B, T, C)), gen.normal(g, (C,)), gen.normal(g, (C,))
    return x, w, b, dout, dinp0, dw0, db0


def exact_case(gpu, oracle, B, T, C, seed, offset=0):
    x, w, b, dout, dinp0, dw0, db0 = inputs(B, T, C, seed)
    rows, n = B * T, B * T * C
    with ln_exact(gpu):
        tx, tw, tb, tdo = put(x, offset), put(w, offset), put(b, offset), put(dout, offset)
        tout, tm, tr = put(np.zeros(n), offset), put(np.zeros(rows), offset), put(np.zeros(rows), offset)
        gpu.layernorm_forward(tout, tm, tr, tx, tw, tb, B, T, C)
        tdi, tdw, tdb = put(dinp0, offset), put(dw0, offset), put(db0, offset)
        gpu.layernorm_backward(tdi, tdw, tdb, tdo, tx, tw, tm, tr, B, T, C)
    out = np.zeros_like(x)
    mean, rstd = np.zeros((B, T), np.float32), np.zeros((B, T), np.float32)
    oracle.layernorm_forward(out, mean, rstd, x, w, b, B, T, C)
    assert_bits(host(tout), out, f"ln out {B}x{T}x{C}")
    assert_bits(host(tm), mean, f"ln mean {B}x{T}x{C}")
    assert_bits(host(tr), rstd, f"ln rstd {B}x{T}x{C}")
    dinp, dw, db = dinp0.copy(), dw0.copy(), db0.copy()
    oracle.layernorm_backward(dinp, dw, db, dout, x, w, mean, rstd, B, T, C)
    assert_bits(host(tdi), dinp, f"ln dinp {B}x{T}x{C}")
    assert_bits(host(tdw), dw, f"ln dweight {B}x{T}x{C}")
    assert_bits(host(tdb), db, f"ln dbias {B}x{T}x{C}")


@pytest.mark.parametrize("B,T,C", [(4, 64, 384), (1, 3, 768), (2, 5, 16), (1, 2, 2048), (1, 4, 13), (1, 2, 3000),
                                   (3, 7, 4), (2, 50, 600), (1, 9, 516), (1, 1, 1), (1, 65, 64), (1, 129, 130),
                                   (2, 300, 65), (1, 240, 64), (4, 120, 32)])
def test_layernorm_exact(gpu, oracle, B, T, C):
    exact_case(gpu, oracle, B, T, C, seed=B * 1000 + T * 10 + C)


def test_layernorm_exact_misaligned(gpu, oracle):
    exact_case(gpu, oracle, 2, 8, 384, seed=9, offset=1)
    exact_case(gpu, oracle, 3, 5, 13, seed=10, offset=3)


@pytest.mark.parametrize("B,T,C", [(8, 1024, 768), (16, 1024, 768)])
def test_layernorm_exact_benchmark_shapes(gpu, oracle, B, T, C):
    print(f"LayerNorm exact mode at {B * T} x {C}", flush=True)
    exact_case(gpu, oracle, B, T, C, seed=B + T + C)


def test_layernorm_exact_switch_restores_default(gpu, oracle):
    """With the mode off again, the default kernels run: their dweight sum differs from the CPU's
    serial one in some bits at this shape, while the exact mode's equals it."""
    B, T, C = 8, 1024, 768
    x, w, b, dout, dinp0, dw0, db0 = inputs(B, T, C, 3)
    tx, tw, tb, tdo = dev(x), dev(w), dev(b), dev(dout)
    tm, tr = torch.empty(B * T, device=DEV), torch.empty(B * T, device=DEV)
    mean, rstd = np.zeros((B, T), np.float32), np.zeros((B, T), np.float32)
    oracle.layernorm_forward(np.zeros_like(x), mean, rstd, x, w, b, B, T, C)
    dinp, dw, db = dinp0.copy(), dw0.copy(), db0.copy()
    oracle.layernorm_backward(dinp, dw, db, dout, x, w, mean, rstd, B, T, C)
    tm.copy_(torch.from_numpy(mean.ravel())), tr.copy_(torch.from_numpy(rstd.ravel()))
    results = {}
    for exact in (True, False):
        gpu.set_layernorm_exact(exact)
        try:
            assert gpu.layernorm_exact() == exact
            tdi, tdw, tdb = dev(dinp0), dev(dw0), dev(db0)
            gpu.layernorm_backward(tdi, tdw, tdb, tdo, tx, tw, tm, tr, B, T, C)
            results[exact] = host(tdw)
        finally:
            gpu.set_layernorm_exact(False)
    assert_bits(results[True], dw, "exact dweight")
    assert not np.array_equal(results[False].view(np.uint32), dw.view(np.uint32)), "the default kernels ran"


def test_layernorm_exact_fused_entry_points(gpu, oracle):
    """The fused pairs in exact mode are the reference's two ops in sequence, bit for bit."""
    B, T, C, V = 3, 40, 384, 97
    g = gen.rng(123)
    n, rows = B * T * C, B * T
    x, y, dout = gen.normal(g, (n,)), gen.normal(g, (n,)), gen.normal(g, (n,))
    w, b = gen.normal(g, (C,), 1, 0.1), gen.normal(g, (C,), 0, 0.1)
    with ln_exact(gpu):
        # residual -> LayerNorm forward
        tres, tout, tm, tr = (torch.empty(k, device=DEV) for k in (n, n, rows, rows))
        gpu.residual_layernorm_forward(tres, tout, tm, tr, dev(x), dev(y), dev(w), dev(b), B, T, C)
        res, out = np.zeros(n, np.float32), np.zeros(n, np.float32)
        mean, rstd = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
        oracle.residual_forward(res, x, y, n)
        oracle.layernorm_forward(out, mean, rstd, res, w, b, B, T, C)
        for got, want, what in ((tres, res, "res"), (tout, out, "out"), (tm, mean, "mean"), (tr, rstd, "rstd")):
            assert_bits(host(got), want, f"residual_layernorm_forward {what}")
        # encoder -> LayerNorm forward
        wte, wpe = gen.normal(g, (V, C), 0, 0.02), gen.normal(g, (T, C), 0, 0.01)
        ids = gen.tokens_uniform(g, rows, V)
        tenc = torch.empty(n, device=DEV)
        gpu.encoder_layernorm_forward(tenc, tout, tm, tr, torch.from_numpy(ids).to(DEV), dev(wte), dev(wpe),
                                      dev(w), dev(b), B, T, C)
        enc = np.zeros(n, np.float32)
        oracle.encoder_forward(enc, ids, wte, wpe, B, T, C)
        oracle.layernorm_forward(out, mean, rstd, enc, w, b, B, T, C)
        for got, want, what in ((tenc, enc, "enc"), (tout, out, "out"), (tm, mean, "mean"), (tr, rstd, "rstd")):
            assert_bits(host(got), want, f"encoder_layernorm_forward {what}")
        # LayerNorm -> residual backward
        dinp0, dx0, dy0 = gen.normal(g, (n,)), gen.normal(g, (n,)), gen.normal(g, (n,))
        dw0, db0 = gen.normal(g, (C,)), gen.normal(g, (C,))
        tdi, tdw, tdb, tdx, tdy = dev(dinp0), dev(dw0), dev(db0), dev(dx0), dev(dy0)
        gpu.layernorm_residual_backward(tdi, tdw, tdb, tdx, tdy, dev(dout), dev(enc), dev(w), dev(mean), dev(rstd),
                                        B, T, C)
    dinp, dw, db, dx, dy = dinp0.copy(), dw0.copy(), db0.copy(), dx0.copy(), dy0.copy()
    oracle.layernorm_backward(dinp, dw, db, dout, enc, w, mean, rstd, B, T, C)
    oracle.residual_backward(dx, dy, dinp, n)
    for got, want, what in ((tdi, dinp, "dinp"), (tdw, dw, "dweight"), (tdb, db, "dbias"), (tdx, dx, "dx"),
                            (tdy, dy, "dy")):
        assert_bits(host(got), want, f"layernorm_residual_backward {what}")


@pytest.mark.parametrize("B,T,C", [(8, 1024, 768), (2, 64, 1030)])
def test_layernorm_exact_noalloc(gpu, oracle, B, T, C):
    """The allocation-free backward follows the mode too (the exact kernels need no scratch)."""
    x, w, b, dout, dinp0, dw0, db0 = inputs(B, T, C, 31)
    mean, rstd = np.zeros((B, T), np.float32), np.zeros((B, T), np.float32)
    oracle.layernorm_forward(np.zeros_like(x), mean, rstd, x, w, b, B, T, C)
    tdi, tdw, tdb = dev(dinp0), dev(dw0), dev(db0)
    args = [dev(a) for a in (dout, x, w, mean, rstd)]
    with ln_exact(gpu):
        rc = gpu.lib.ugk_layernorm_backward_noalloc(tdi.data_ptr(), tdw.data_ptr(), tdb.data_ptr(),
                                                    *[a.data_ptr() for a in args], B, T, C)
        assert rc == 0, gpu.lib.ugk_last_error()
    dinp, dw, db = dinp0.copy(), dw0.copy(), db0.copy()
    oracle.layernorm_backward(dinp, dw, db, dout, x, w, mean, rstd, B, T, C)
    for got, want, what in ((tdi, dinp, "dinp"), (tdw, dw, "dweight"), (tdb, db, "dbias")):
        assert_bits(host(got), want, f"noalloc {what}")


def test_layernorm_exact_golden_fixture(gpu):
    """tests/golden/layernorm.npz, written by the reference's own train_bnn.c build: equal bit for bit."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layernorm.npz")
    with np.load(path, allow_pickle=False) as z:
        L = {k: z[k] for k in z.files}
    B, T, C = int(L["B"]), int(L["T"]), int(L["C"])
    n, rows = B * T * C, B * T
    with ln_exact(gpu):
        tout, tm, tr = torch.empty(n, device=DEV), torch.empty(rows, device=DEV), torch.empty(rows, device=DEV)
        gpu.layernorm_forward(tout, tm, tr, dev(L["x"]), dev(L["w"]), dev(L["b"]), B, T, C)
        tdi, tdw, tdb = dev(L["dinp0"]), dev(L["dw0"]), dev(L["db0"])
        gpu.layernorm_backward(tdi, tdw, tdb, dev(L["dout"]), dev(L["x"]), dev(L["w"]), dev(L["mean"]),
                               dev(L["rstd"]), B, T, C)
    for got, key in ((tout, "out"), (tm, "mean"), (tr, "rstd"), (tdi, "dinp"), (tdw, "dw"), (tdb, "db")):
        assert_bits(host(got), L[key].ravel(), f"golden layernorm {key}")
