"""GPU: the device workspace and the ways a caller controls it.

* The encoder backward keeps no state on the host: one call captured in a HIP graph and replayed
  three times (an odd number, with eager calls on other buffers in between) accumulates exactly
  what three calls of train_bnn.c's encoder_backward (:647-662) accumulate (exact mode), or three
  of its blocked order (the default).
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
from test_parity_gpu import assert_bits, blocked_encoder_backward, dev, encoder_mode, host

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


@pytest.mark.parametrize("exact", [True, False])
def test_encoder_backward_graph_replays(gpu, oracle, lib_stream, exact):
    with encoder_mode(gpu, exact):
        graph_replays(gpu, oracle, lib_stream, exact)


def graph_replays(gpu, oracle, lib_stream, exact):
    """Exact mode: the CPU's order (oracle); blocked mode: its numpy restatement (test_parity_gpu),
    whose per-(bucket, slice) counters must also return to zero within each replay."""
    backward = oracle.encoder_backward if exact else blocked_encoder_backward
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
        backward(want_wte, want_wpe, dout, inp, B, T, C)
    assert_bits(host(t_dwte), want_wte, "dwte after 3 replays")
    assert_bits(host(t_dwpe), want_wpe, "dwpe after 3 replays")
    want2_wte, want2_wpe = dwte2.copy(), dwpe2.copy()
    for _ in range(4):
        backward(want2_wte, want2_wpe, dout2, inp2, B, T, C)
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


def test_workspace_sized_for_more_rows_serves_fewer(gpu):
    """A caller-owned workspace sized for B=5, T=1024, C=768 serves every workspace user at B=4 and
    B=3 (the LayerNorm slots are sized by a bound that holds for every smaller call), with results
    identical to the library-owned regions."""
    cfg = gpu.Config(B=5, T=1024, C=768, V=1000, NH=12, maxT=1024, L=2)
    small = [gpu.Config(B=B, T=1024, C=768, V=1000, NH=12, maxT=1024, L=2) for B in (4, 3)]
    gpu.set_workspace(None, cfg)
    want = [run_ops(gpu, c, seed=40 + k) for k, c in enumerate(small)]
    nbytes = gpu.workspace_bytes(cfg)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=DEV)
    off = (-ws.data_ptr()) % 256
    try:
        gpu.set_workspace(ws[off:off + nbytes], cfg)
        del ws  # the binding keeps the workspace alive while the library uses it
        torch.cuda.empty_cache()
        for k, c in enumerate(small):
            got, kl = run_ops(gpu, c, seed=40 + k)
            assert kl == want[k][1]
            for j, (a, b) in enumerate(zip(got, want[k][0])):
                assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"B={c.B}: output {j} differs"
    finally:
        gpu.set_workspace(None, cfg)


def test_encoder_backward_capture_needs_prepared_state(gpu, oracle, lib_stream):
    """The encoder backward's state must be allocated and cleared outside a graph capture: with the
    library's regions just freed, a first call under capture is refused before it launches anything;
    after ugk_set_workspace (which clears the state at once) a first call may be captured, and its
    replays accumulate what the oracle's calls do."""
    B, T, C, V = 4, 64, 384, 1000
    cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=6, maxT=T, L=1)
    g = gen.rng(1618)
    inp, dout, dwte0, dwpe0 = enc_case(g, B, T, C, V, hot=70)
    s = lib_stream
    t_inp, t_dout, t_dwte, t_dwpe = dev(inp), dev(dout), dev(dwte0), dev(dwpe0)
    gpu.set_workspace(None, cfg)  # frees the library-owned regions
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        with pytest.raises(gpu.UgkError) as err:
            gpu.encoder_backward(t_dwte, t_dwpe, t_dout, t_inp, B, T, C)
    assert err.value.status == 3 and "capture" in str(err.value)
    del graph
    assert_bits(host(t_dwte), dwte0, "dwte untouched by the refused call")
    nbytes = gpu.workspace_bytes(cfg)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=DEV)
    off = (-ws.data_ptr()) % 256
    try:
        gpu.set_workspace(ws[off:off + nbytes], cfg)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):  # the first call on this workspace, captured
            gpu.encoder_backward(t_dwte, t_dwpe, t_dout, t_inp, B, T, C)
        for _ in range(2):
            graph.replay()
            torch.cuda.synchronize()
        want_wte, want_wpe = dwte0.copy(), dwpe0.copy()
        for _ in range(2):  # the default (blocked) order: a token of 70 rows
            blocked_encoder_backward(want_wte, want_wpe, dout, inp, B, T, C)
        assert_bits(host(t_dwte), want_wte, "dwte after 2 replays of a first call")
        assert_bits(host(t_dwpe), want_wpe, "dwpe after 2 replays of a first call")
        del graph
    finally:
        torch.cuda.synchronize()
        gpu.set_workspace(None, cfg)
