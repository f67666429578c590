"""GPU: the device workspace and the ways a caller controls it.

* The encoder backward keeps no state on the host: one call captured in a HIP graph and replayed
  three times (an odd number, with eager calls on other buffers in between) accumulates exactly
  what three calls of train_bnn.c's encoder_backward (:647-662) accumulate.
* A caller-owned workspace (ugk_set_workspace, sized by ugk_workspace_bytes) gives results
  identical to the library-owned regions; a shape beyond the config it was sized for is refused
  with UGK_ENOMEM; NULL returns to library-owned regions.
* After ugk_reserve_config no entry point grows the workspace at shapes up to the config.
* The step driver's op timer records one event pair per library op, in the reference's order.
"""
import numpy as np
import pytest
import torch

import gen
from test_parity_gpu import assert_bits, dev, host

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def lib_stream(gpu):
    """A side stream for the library (restored afterwards)."""
    prev = gpu.lib.ugk_get_stream()
    s = torch.cuda.Stream()
    gpu.set_stream(s.cuda_stream)
    try:
        yield s
    finally:
        gpu.set_stream(prev)


def enc_case(g, B, T, C, V, hot):
    """Tokens with one token repeated `hot` times (a bucket beyond the 32 rows a slot keeps)."""
    inp = gen.tokens_uniform(g, B * T, V)
    inp[g.choice(B * T, size=hot, replace=False)] = 5
    return (inp, gen.normal(g, (B * T * C,)), gen.normal(g, (V * C,), 0, 0.02), gen.normal(g, (T * C,), 0, 0.01))


def test_encoder_backward_graph_replays(gpu, oracle, lib_stream):
    B, T, C, V = 4, 64, 384, 1000
    g = gen.rng(2718)
    inp, dout, dwte0, dwpe0 = enc_case(g, B, T, C, V, hot=100)
    inp2, dout2, dwte2, dwpe2 = enc_case(g, B, T, C, V, hot=40)
    s = lib_stream
    t_inp, t_dout, t_dwte, t_dwpe = dev(inp), dev(dout), dev(dwte0), dev(dwpe0)
    e_inp, e_dout, e_dwte, e_dwpe = dev(inp2), dev(dout2), dev(dwte2), dev(dwpe2)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        # an eager call first: the workspace is allocated and cleared outside the capture
        gpu.encoder_backward(e_dwte, e_dwpe, e_dout, e_inp, B, T, C)
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        gpu.encoder_backward(t_dwte, t_dwpe, t_dout, t_inp, B, T, C)
    for k in range(3):
        graph.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):  # eager work between replays, through the same table
            gpu.encoder_backward(e_dwte, e_dwpe, e_dout, e_inp, B, T, C)
        s.synchronize()
    want_wte, want_wpe = dwte0.copy(), dwpe0.copy()
    for _ in range(3):
        oracle.encoder_backward(want_wte, want_wpe, dout, inp, B, T, C)
    assert_bits(host(t_dwte), want_wte, "dwte after 3 replays")
    assert_bits(host(t_dwpe), want_wpe, "dwpe after 3 replays")
    want2_wte, want2_wpe = dwte2.copy(), dwpe2.copy()
    for _ in range(4):
        oracle.encoder_backward(want2_wte, want2_wpe, dout2, inp2, B, T, C)
    assert_bits(host(e_dwte), want2_wte, "dwte of the eager calls between replays")
    assert_bits(host(e_dwpe), want2_wpe, "dwpe of the eager calls between replays")


def run_ops(gpu, cfg, seed):
    """Every workspace user once at the config's shapes: LayerNorm backward (per op), encoder
    backward, KL total, the step driver. Returns the outputs (device tensors) and the KL."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    B, T, C, V = cfg.B, cfg.T, cfg.C, cfg.V
    rows, n = B * T, B * T * C
    r = lambda k, s=1.0: torch.randn(k, generator=g, device=DEV) * s
    x, dout, w = r(n), r(n), r(C, 0.1) + 1.0
    out, mean, rstd = torch.empty(n, device=DEV), torch.empty(rows, device=DEV), torch.empty(rows, device=DEV)
    gpu.layernorm_forward(out, mean, rstd, x, w, r(C, 0.1), B, T, C)
    dinp, dw, db = r(n), r(C), r(C)
    gpu.layernorm_backward(dinp, dw, db, dout, x, w, mean, rstd, B, T, C)
    inp = torch.randint(0, V, (rows,), generator=g, device=DEV, dtype=torch.int32)
    dwte, dwpe = r(V * C, 0.02), r(cfg.maxT * C, 0.01)
    gpu.encoder_backward(dwte, dwpe, dout, inp, B, T, C)
    mu, rho = r(4096, 0.02), r(4096, 0.1) - 5.0
    kl = gpu.kl_forward(mu, rho, 4096, 0.1)
    params = r(gpu.param_count(cfg), 0.02) + 0.5
    acts, grads, ga = r(gpu.act_count(cfg)), torch.zeros(gpu.param_count(cfg), device=DEV), r(gpu.act_count(cfg), 0.1)
    gpu.gpt2_layers_forward(acts, params, inp, cfg)
    gpu.gpt2_layers_backward(grads, ga, acts, params, inp, cfg)
    torch.cuda.synchronize()
    return [dinp, dw, db, dwte, dwpe, acts, grads, ga], kl


def test_caller_owned_workspace(gpu):
    cfg = gpu.Config(B=2, T=64, C=384, V=500, NH=6, maxT=64, L=2)
    gpu.set_workspace(None, cfg)
    want, kl_want = run_ops(gpu, cfg, seed=31)
    nbytes = gpu.workspace_bytes(cfg)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=DEV)
    off = (-ws.data_ptr()) % 256
    try:
        gpu.set_workspace(ws[off:off + nbytes], cfg)
        assert gpu.scratch_bytes() == nbytes
        got, kl_got = run_ops(gpu, cfg, seed=31)
        assert kl_got == kl_want
        for k, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"output {k} differs"
        # more LayerNorm partial rows than the config provides: refused, nothing launched
        rows = 128 * cfg.B * cfg.T
        t = torch.zeros(rows * cfg.C, device=DEV)
        c = torch.zeros(cfg.C, device=DEV)
        st = torch.ones(rows, device=DEV)
        with pytest.raises(gpu.UgkError) as err:
            gpu.layernorm_backward(t, c, c, t, t, c, st, st, 1, rows, cfg.C)
        assert err.value.status == 3 and "workspace" in str(err.value)
        assert gpu.scratch_bytes() == nbytes
        assert gpu.lib.ugk_set_workspace(ws.data_ptr() + off + 4, nbytes, cfg) == 1  # not 256-byte aligned
        assert gpu.lib.ugk_set_workspace(ws.data_ptr() + off, nbytes - 256, cfg) == 1  # too small for cfg
        assert gpu.scratch_bytes() == nbytes  # both refused without touching the workspace in use
    finally:
        gpu.set_workspace(None, cfg)
    got, kl_got = run_ops(gpu, cfg, seed=31)  # library-owned again
    assert kl_got == kl_want
    for k, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"output {k} differs after returning"


def test_reserve_config_then_no_growth(gpu):
    cfg = gpu.Config(B=4, T=128, C=768, V=1000, NH=12, maxT=128, L=3)
    gpu.reserve_config(cfg)
    held = gpu.scratch_bytes()
    assert held >= gpu.workspace_bytes(cfg) - 4 * 256
    run_ops(gpu, cfg, seed=5)
    assert gpu.scratch_bytes() == held
    small = gpu.Config(B=1, T=64, C=384, V=100, NH=6, maxT=128, L=1)
    run_ops(gpu, small, seed=6)
    assert gpu.scratch_bytes() == held


@pytest.mark.parametrize("C,NH,L", [(384, 6, 2), (384, 6, 16), (13, 1, 2)])
def test_op_timer_records_the_driver_sequence(gpu, C, NH, L):
    """One record per op, in issue order, also for ops of several kernels: at L = 16 the batched
    column sums take two launches, at C = 13 (scalar path) the fused LayerNorm backward pair does."""
    B, T, V = 2, 64, 100
    cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=T, L=L)
    g = torch.Generator(device=DEV)
    g.manual_seed(3)
    params = torch.randn(gpu.param_count(cfg), generator=g, device=DEV) * 0.02 + 0.5
    acts = torch.randn(gpu.act_count(cfg), generator=g, device=DEV)
    ga = torch.randn(gpu.act_count(cfg), generator=g, device=DEV) * 0.1
    grads = torch.zeros(gpu.param_count(cfg), device=DEV)
    inp = torch.randint(0, V, (B * T,), generator=g, device=DEV, dtype=torch.int32)
    gpu.op_timer_start(256)
    gpu.gpt2_layers_forward(acts, params, inp, cfg)
    gpu.gpt2_layers_backward(grads, ga, acts, params, inp, cfg)
    rec = gpu.op_timer_read(256)
    fwd = ["encoder_layernorm_forward"] + ["residual_layernorm_forward", "gelu_forward",
                                           "residual_layernorm_forward"] * L
    bwd = ["layernorm_residual_backward (main)"]
    for l in range(L - 1, -1, -1):
        bwd += ["gelu_backward", "layernorm_residual_backward (main)",
                "layernorm_residual_backward (main)" if l > 0 else "layernorm_backward (main)"]
    bwd += ["layernorm column sums (batched)", "encoder_backward"]
    assert [name for name, _ in rec] == fwd + bwd
    assert all(ms > 0 for _, ms in rec)
    # stopped: a further step records nothing
    gpu.gpt2_layers_forward(acts, params, inp, cfg)
    assert gpu.op_timer_read(256) == []
