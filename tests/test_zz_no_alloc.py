"""GPU: the allocation-free LayerNorm backward (ugk_layernorm_backward_noalloc, partial column sums in
the library's fixed device array) against ugk_layernorm_backward (partial sums in the workspace),
called through the C-ABI: two calls in a row, the second on a smaller input, each bit-identical
to the existing entry point on the same inputs (C <= 1,024: the same partial rows), with no
change in the workspace the library holds. A C beyond the array's capacity is refused."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(gpu, B, T, C, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    n, rows = B * T * C, B * T
    x, dout = torch.randn(n, generator=g, device=DEV), torch.randn(n, generator=g, device=DEV)
    w = torch.randn(C, generator=g, device=DEV) * 0.1 + 1.0
    b = torch.randn(C, generator=g, device=DEV) * 0.1
    out, mean, rstd = torch.empty(n, device=DEV), torch.empty(rows, device=DEV), torch.empty(rows, device=DEV)
    gpu.layernorm_forward(out, mean, rstd, x, w, b, B, T, C)
    grads = (torch.randn(n, generator=g, device=DEV), torch.randn(C, generator=g, device=DEV),
             torch.randn(C, generator=g, device=DEV))
    return x, dout, w, mean, rstd, grads


def run(lib, fn, grads, x, dout, w, mean, rstd, B, T, C):
    di, dw, db = (t.clone() for t in grads)
    rc = getattr(lib, fn)(di.data_ptr(), dw.data_ptr(), db.data_ptr(), dout.data_ptr(), x.data_ptr(), w.data_ptr(),
                          mean.data_ptr(), rstd.data_ptr(), B, T, C)
    assert rc == 0, f"{fn}: status {rc}: {lib.ugk_last_error().decode()}"
    return di, dw, db


def test_noalloc_layernorm_backward_equals_workspace_path(gpu):
    lib = gpu.lib
    for B, T, C in ((8, 1024, 768), (2, 100, 384)):  # the second call smaller
        print(f"no-alloc LayerNorm backward B={B} T={T} C={C}", flush=True)
        x, dout, w, mean, rstd, grads = case(gpu, B, T, C, seed=B * T + C)
        want = run(lib, "ugk_layernorm_backward", grads, x, dout, w, mean, rstd, B, T, C)
        torch.cuda.synchronize()
        held = gpu.scratch_bytes()
        got = run(lib, "ugk_layernorm_backward_noalloc", grads, x, dout, w, mean, rstd, B, T, C)
        torch.cuda.synchronize()
        assert gpu.scratch_bytes() == held, "the no-alloc call changed the workspace"
        for name, a, e in zip(("dinp", "dweight", "dbias"), got, want):
            assert torch.equal(a.view(torch.int32), e.view(torch.int32)), f"{name} differs at B={B} T={T} C={C}"


@pytest.mark.parametrize("B,T,C", [(8, 1024, 2048), (2, 64, 1030)])
def test_noalloc_layernorm_backward_fewer_partial_rows_and_scalar_path(gpu, oracle, B, T, C):
    """Shapes where the array holds fewer partial rows than the workspace path uses (C = 2,048 at
    8,192 rows: 512 instead of 1,024, so the column sums add in another order) and the scalar path
    (C not a multiple of 4): dinp bit-identical to ugk_layernorm_backward (each row's own sums do not
    depend on the partial rows), dweight/dbias within the scale-aware bar of the CPU oracle
    (train_bnn.c:439-477) and at least as close to a float64 sum as the CPU's."""
    import numpy as np
    lib = gpu.lib
    print(f"no-alloc LayerNorm backward B={B} T={T} C={C}", flush=True)
    x, dout, w, mean, rstd, grads = case(gpu, B, T, C, seed=B * T + C)
    want = run(lib, "ugk_layernorm_backward", grads, x, dout, w, mean, rstd, B, T, C)
    got = run(lib, "ugk_layernorm_backward_noalloc", grads, x, dout, w, mean, rstd, B, T, C)
    torch.cuda.synchronize()
    assert torch.equal(got[0].view(torch.int32), want[0].view(torch.int32)), "dinp differs"
    h = lambda t: t.detach().cpu().numpy()
    xs, ds, ws, ms, rs = h(x), h(dout), h(w), h(mean), h(rstd)
    di0, dw0, db0 = (h(t) for t in grads)
    cdi, cdw, cdb = di0.copy(), dw0.copy(), db0.copy()
    oracle.layernorm_backward(cdi, cdw, cdb, ds, xs, ws, ms, rs, B, T, C)
    xhat = (xs.astype(np.float64).reshape(-1, C) - ms[:, None]) * rs[:, None]
    d64 = ds.astype(np.float64).reshape(-1, C)
    for name, g_, cpu, init, terms in (("dweight", h(got[1]), cdw, dw0, d64 * xhat), ("dbias", h(got[2]), cdb, db0, d64)):
        f64 = init.astype(np.float64) + terms.sum(0)
        scale = np.abs(init) + np.abs(terms).sum(0)
        assert (np.abs(g_ - cpu) <= 1e-5 * scale).all(), f"{name}: beyond the scale-aware bar"
        assert np.abs(g_ - f64).max() <= np.abs(cpu - f64).max() + 1e-6 * scale.max(), f"{name}: less accurate"


def test_noalloc_layernorm_backward_refuses_too_wide_rows(gpu):
    C = (8 << 20) // 8 + 1  # one channel more than 8 MiB of partial rows of 2C floats hold
    t = torch.zeros(C, device=DEV)
    s = torch.ones(1, device=DEV)
    rc = gpu.lib.ugk_layernorm_backward_noalloc(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(),
                                                t.data_ptr(), s.data_ptr(), s.data_ptr(), 1, 1, C)
    assert rc == 1 and b"scratch" in gpu.lib.ugk_last_error()
