"""GPU: the per-op LayerNorm backward's two ways of finishing the dweight/dbias column sums
(train_bnn.c:439-477 sums each column over all rows; gpt2_kernels.cuh:290-316 adds per-block
atomics, in no fixed order). By default a second launch adds the partial rows; in the other mode
the main launch's workgroups add them themselves (the last workgroup of each group of rows, then
the last group). Both add in the same order, so they agree bit for bit, for
the plain op, the fused LayerNorm -> residual pair and the allocation-free entry point; repeated
calls find the in-launch counters reset (three accumulating calls give the same bits as three
two-launch calls). The accuracy of those sums against the oracle is tested in test_parity_gpu.py.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [(1, 3, 768), (2, 5, 16), (4, 64, 384), (1, 2, 2048), (1, 9, 516), (2, 50, 600), (3, 7, 4),
          (4, 256, 1024), (8, 1024, 768), (16, 1024, 768), (2, 1000, 2048), (1, 70000, 64)]


def inputs(B, T, C, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    n, rows = B * T * C, B * T
    r = lambda k, s=1.0: torch.randn(k, generator=g, device=DEV) * s
    x, dout, w, b = r(n), r(n), r(C, 0.1) + 1.0, r(C, 0.1)
    mean, rstd = torch.empty(rows, device=DEV), torch.empty(rows, device=DEV)
    return x, dout, w, b, mean, rstd, (r(n), r(C), r(C), r(n), r(n))


def run(gpu, B, T, C, data, fn, tail, reps=3):
    x, dout, w, b, mean, rstd, init = data
    di, dw, db, dx, dy = (t.clone() for t in init)
    prev = gpu.lib.ugk_diag_layernorm_tail(tail)
    try:
        for _ in range(reps):
            if fn == "plain":
                gpu.layernorm_backward(di, dw, db, dout, x, w, mean, rstd, B, T, C)
            elif fn == "fused":
                gpu.layernorm_residual_backward(di, dw, db, dx, dy, dout, x, w, mean, rstd, B, T, C)
            else:
                rc = gpu.lib.ugk_layernorm_backward_noalloc(di.data_ptr(), dw.data_ptr(), db.data_ptr(),
                                                            dout.data_ptr(), x.data_ptr(), w.data_ptr(),
                                                            mean.data_ptr(), rstd.data_ptr(), B, T, C)
                assert rc == 0, gpu.lib.ugk_last_error()
        torch.cuda.synchronize()
    finally:
        gpu.lib.ugk_diag_layernorm_tail(prev)
    return di, dw, db, dx, dy


@pytest.mark.parametrize("B,T,C", SHAPES)
def test_in_launch_column_sums_equal_the_second_launch(gpu, B, T, C):
    print(f"LayerNorm backward column sums B={B} T={T} C={C}", flush=True)
    data = inputs(B, T, C, seed=B * 7 + T * 3 + C)
    x, dout, w, b, mean, rstd, _ = data
    gpu.layernorm_forward(torch.empty_like(x), mean, rstd, x, w, b, B, T, C)
    assert gpu.lib.ugk_diag_layernorm_tail(-1) == 0  # the default: a second launch
    for fn in ("plain", "fused", "noalloc"):
        want = run(gpu, B, T, C, data, fn, tail=0)
        got = run(gpu, B, T, C, data, fn, tail=1)
        for name, a, e in zip(("dinp", "dweight", "dbias", "dx", "dy"), got, want):
            assert torch.equal(a.view(torch.int32), e.view(torch.int32)), f"{fn} {name} differs"
