"""GPU: the fused pairs the step driver runs (residual -> LayerNorm forward, LayerNorm -> residual
backward) equal the unfused per-op calls bit for bit, and the driver equals a per-op replay of
the reference launch sequence (gpt2_kernels.cuh:775-894) bit for bit.

The per-op kernels are themselves checked against the CPU oracle in test_parity_gpu.py, so
bit-equality here carries their parity over to the fused forms.
"""
import numpy as np
import pytest
import torch

import gen
from test_parity_gpu import assert_bits, dev, host, ref_offsets

pytestmark = pytest.mark.gpu
DEV = "cuda"


def put(a, offset):
    return dev(np.concatenate([np.zeros(offset, np.float32), np.ascontiguousarray(a, np.float32).ravel()]))[offset:]


@pytest.mark.parametrize("B,T,C,offset", [(8, 1024, 768, 0), (4, 64, 384, 0), (1, 5, 2048, 0), (2, 3, 13, 0),
                                          (2, 8, 384, 1), (3, 7, 4, 0)])
def test_residual_layernorm_forward_fused(gpu, B, T, C, offset):
    g = gen.rng(B * 7919 + T * 31 + C)
    n, rows = B * T * C, B * T
    x, y = gen.normal(g, (n,)), gen.normal(g, (n,))
    w, b = gen.normal(g, (C,), 1, 0.1), gen.normal(g, (C,), 0, 0.1)
    tx, ty, tw, tb = put(x, offset), put(y, offset), put(w, offset), put(b, offset)
    z = lambda k: put(np.zeros(k, np.float32), offset)
    f_res, f_out, f_m, f_r = z(n), z(n), z(rows), z(rows)
    gpu.residual_layernorm_forward(f_res, f_out, f_m, f_r, tx, ty, tw, tb, B, T, C)
    u_res, u_out, u_m, u_r = z(n), z(n), z(rows), z(rows)
    gpu.residual_forward(u_res, tx, ty, n)
    gpu.layernorm_forward(u_out, u_m, u_r, u_res, tw, tb, B, T, C)
    for name, a, c in (("res", f_res, u_res), ("out", f_out, u_out), ("mean", f_m, u_m), ("rstd", f_r, u_r)):
        assert_bits(host(a), host(c), f"fused forward {name}")


@pytest.mark.parametrize("B,T,C,V,offset", [(8, 1024, 768, 50257, 0), (4, 64, 384, 27, 0), (1, 5, 2048, 7, 0),
                                            (2, 3, 13, 5, 0), (2, 8, 384, 11, 1), (64, 200, 768, 300, 0),
                                            (1, 3, 3000, 9, 0)])
def test_encoder_layernorm_forward_fused(gpu, B, T, C, V, offset):
    """The pass equals encoder_forward then layernorm_forward on its output, bit for bit: aligned
    and misaligned buffers, odd C and C past the vector path's 2,048 (two launches), and more rows
    than one round of wavefronts (12,800: one row per wavefront)."""
    g = gen.rng(B * 65537 + T * 13 + C)
    n, rows = B * T * C, B * T
    inp = gen.tokens_uniform(g, rows, V)
    wte, wpe = gen.normal(g, (V * C,), 0, 0.02), gen.normal(g, (T * C,), 0, 0.01)
    w, b = gen.normal(g, (C,), 1, 0.1), gen.normal(g, (C,), 0, 0.1)
    tinp = dev(inp)
    twte, twpe, tw, tb = put(wte, offset), put(wpe, offset), put(w, offset), put(b, offset)
    z = lambda k: put(np.zeros(k, np.float32), offset)
    f_enc, f_out, f_m, f_r = z(n), z(n), z(rows), z(rows)
    gpu.encoder_layernorm_forward(f_enc, f_out, f_m, f_r, tinp, twte, twpe, tw, tb, B, T, C)
    u_enc, u_out, u_m, u_r = z(n), z(n), z(rows), z(rows)
    gpu.encoder_forward(u_enc, tinp, twte, twpe, B, T, C)
    gpu.layernorm_forward(u_out, u_m, u_r, u_enc, tw, tb, B, T, C)
    for name, a, c in (("enc", f_enc, u_enc), ("out", f_out, u_out), ("mean", f_m, u_m), ("rstd", f_r, u_r)):
        assert_bits(host(a), host(c), f"fused encoder forward {name}")


@pytest.mark.parametrize("B,T,C,offset", [(8, 1024, 768, 0), (4, 64, 384, 0), (1, 5, 2048, 0), (2, 3, 13, 0),
                                          (2, 8, 384, 1), (1, 3, 3000, 0), (2, 50, 600, 0), (1, 9, 516, 0),
                                          (16, 1024, 768, 0), (1, 8192, 768, 0), (1, 8193, 768, 0)])
@pytest.mark.parametrize("same", [False, True])
def test_layernorm_residual_backward_fused(gpu, B, T, C, offset, same):
    """The pair equals layernorm_backward then residual_backward, bit for bit: at C = 516..768
    (three wavefronts per row, the third partly idle at 516 and 600) up to 32 rows per CU (8,192
    on MI355X), and with one wavefront per row beyond (8,193 and 16,384 rows) and at other C."""
    g = gen.rng(B * 104729 + T * 17 + C + same)
    n, rows = B * T * C, B * T
    x, dout = gen.normal(g, (n,)), gen.normal(g, (n,))
    w, b = gen.normal(g, (C,), 1, 0.1), gen.normal(g, (C,), 0, 0.1)
    dinp0, dw0, db0 = gen.normal(g, (n,)), gen.normal(g, (C,)), gen.normal(g, (C,))
    dx0, dy0 = gen.normal(g, (n,)), gen.normal(g, (n,))
    tx, tw, tb, tdo = put(x, offset), put(w, offset), put(b, offset), put(dout, offset)
    out, tm, tr = put(np.zeros(n, np.float32), offset), put(np.zeros(rows, np.float32), offset), \
        put(np.zeros(rows, np.float32), offset)
    gpu.layernorm_forward(out, tm, tr, tx, tw, tb, B, T, C)
    results = []
    for fused in (True, False):
        tdi, tdw, tdb = put(dinp0, offset), put(dw0, offset), put(db0, offset)
        tdx = put(dx0, offset)
        tdy = tdx if same else put(dy0, offset)
        if fused:
            gpu.layernorm_residual_backward(tdi, tdw, tdb, tdx, tdy, tdo, tx, tw, tm, tr, B, T, C)
        else:
            gpu.layernorm_backward(tdi, tdw, tdb, tdo, tx, tw, tm, tr, B, T, C)
            gpu.residual_backward(tdx, tdy, tdi, n)
        results.append([host(t) for t in (tdi, tdw, tdb, tdx, tdy)])
    for name, a, c in zip(("dinp", "dweight", "dbias", "dx", "dy"), *results):
        assert_bits(a, c, f"fused backward {name}")


def test_fused_backward_rejects_aliased_dinp(gpu):
    t = torch.zeros(64, device=DEV)
    with pytest.raises(gpu.UgkError):
        gpu.layernorm_residual_backward(t, t, t, t, torch.zeros(64, device=DEV), t, t, t, t, t, 1, 4, 16)


@pytest.mark.parametrize("B,T,L", [(2, 32, 3), (4, 128, 1)])
def test_step_driver_equals_per_op_replay_on_gpu(gpu, B, T, L):
    """ugk_gpt2_layers_forward/backward (fused pairs) == the reference launch sequence issued op by
    op through the same library, bit for bit, on every activation, every parameter gradient and
    every activation gradient but the fused backward pairs' dinp (resa and res1 of each block,
    which the reference reads only in the residual_backward that the pair fuses).
    The driver reduces all LayerNorms' partial rows in one batched launch, the per-op path each
    in its own: the same additions in the same order (8 and 64 partial rows, 1 and 4 per group)."""
    C, V, NH = 768, 50, 12
    maxT = max(T, 64)
    cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=maxT, L=L)
    p, prel, a, arel = ref_offsets(B, T, C, V, maxT, L)
    g = gen.rng(67)
    params = gen.normal(g, (p["total"],), 0, 0.02)
    for l in range(L):
        for k in ("lng", "ln2g"):
            s = p["blk0"] + l * p["bstride"] + prel[k]
            params[s:s + C] += 1.0
    params[p["flng"]:p["flng"] + C] += 1.0
    acts0 = gen.normal(g, (a["total"],))
    inputs = gen.tokens_uniform(g, B * T, V)
    tpar, tin = dev(params), dev(inputs)
    NB = B * T * C

    # driver
    d_acts = dev(acts0)
    gpu.gpt2_layers_forward(d_acts, tpar, tin, cfg)
    # per-op replay of gpt2_kernels.cuh:775-813
    r_acts = dev(acts0)
    A = lambda l, k, n: r_acts[a["blk0"] + l * a["bstride"] + arel[k]:][:n]
    P = lambda l, k, n: tpar[p["blk0"] + l * p["bstride"] + prel[k]:][:n]
    enc = r_acts[:NB]
    gpu.encoder_forward(enc, tin, tpar[:V * C], tpar[V * C:V * C + maxT * C], B, T, C)
    stream = enc
    for l in range(L):
        gpu.layernorm_forward(A(l, "lno", NB), A(l, "lnm", B * T), A(l, "lnr", B * T), stream, P(l, "lng", C),
                              P(l, "lnb", C), B, T, C)
        gpu.residual_forward(A(l, "resa", NB), stream, A(l, "apr", NB), NB)
        gpu.layernorm_forward(A(l, "ln2o", NB), A(l, "ln2m", B * T), A(l, "ln2r", B * T), A(l, "resa", NB),
                              P(l, "ln2g", C), P(l, "ln2b", C), B, T, C)
        gpu.gelu_forward(A(l, "gelu", 4 * NB), A(l, "fch", 4 * NB), 4 * NB)
        gpu.residual_forward(A(l, "res1", NB), A(l, "resa", NB), A(l, "mlpo", NB), NB)
        stream = A(l, "res1", NB)
    gpu.layernorm_forward(r_acts[a["flo"]:][:NB], r_acts[a["flm"]:][:B * T], r_acts[a["flr"]:][:B * T], stream,
                          tpar[p["flng"]:][:C], tpar[p["flnb"]:][:C], B, T, C)
    assert_bits(host(d_acts), host(r_acts), "driver forward activations")

    ga0 = np.zeros(a["total"], np.float32)
    ga0[a["flo"]:a["flo"] + NB] = gen.normal(g, (NB,))
    ga0[a["blk0"]:a["blk0"] + L * a["bstride"]] = gen.normal(g, (L * a["bstride"],), 0, 0.1)
    d_g, d_ga = dev(np.zeros(p["total"], np.float32)), dev(ga0)
    gpu.gpt2_layers_backward(d_g, d_ga, d_acts, tpar, tin, cfg)
    r_g, r_ga = dev(np.zeros(p["total"], np.float32)), dev(ga0)
    GA = lambda off, n: r_ga[off:][:n]
    AC = lambda off, n: d_acts[off:][:n]
    AO = lambda l, k: a["blk0"] + l * a["bstride"] + arel[k]
    PO = lambda l, k: p["blk0"] + l * p["bstride"] + prel[k]
    last = AO(L - 1, "res1")
    gpu.layernorm_backward(GA(last, NB), r_g[p["flng"]:][:C], r_g[p["flnb"]:][:C], GA(a["flo"], NB), AC(last, NB),
                           tpar[p["flng"]:][:C], AC(a["flm"], B * T), AC(a["flr"], B * T), B, T, C)
    for l in range(L - 1, -1, -1):
        st = a["enc"] if l == 0 else AO(l - 1, "res1")
        gpu.residual_backward(GA(AO(l, "resa"), NB), GA(AO(l, "mlpo"), NB), GA(AO(l, "res1"), NB), NB)
        gpu.gelu_backward(GA(AO(l, "fch"), 4 * NB), AC(AO(l, "fch"), 4 * NB), GA(AO(l, "gelu"), 4 * NB), 4 * NB)
        gpu.layernorm_backward(GA(AO(l, "resa"), NB), r_g[PO(l, "ln2g"):][:C], r_g[PO(l, "ln2b"):][:C],
                               GA(AO(l, "ln2o"), NB), AC(AO(l, "resa"), NB), tpar[PO(l, "ln2g"):][:C],
                               AC(AO(l, "ln2m"), B * T), AC(AO(l, "ln2r"), B * T), B, T, C)
        gpu.residual_backward(GA(st, NB), GA(AO(l, "apr"), NB), GA(AO(l, "resa"), NB), NB)
        gpu.layernorm_backward(GA(st, NB), r_g[PO(l, "lng"):][:C], r_g[PO(l, "lnb"):][:C], GA(AO(l, "lno"), NB),
                               AC(st, NB), tpar[PO(l, "lng"):][:C], AC(AO(l, "lnm"), B * T),
                               AC(AO(l, "lnr"), B * T), B, T, C)
    gpu.encoder_backward(r_g[:V * C], r_g[V * C:V * C + maxT * C], GA(a["enc"], NB), tin, B, T, C)
    # the pairs' dinp (resa and res1 of every block) is read but not written back by the driver
    dga, rga = host(d_ga), host(r_ga)
    for l in range(L):
        for k in ("resa", "res1"):
            dga[AO(l, k):AO(l, k) + NB] = 0
            rga[AO(l, k):AO(l, k) + NB] = 0
    assert_bits(dga, rga, "driver grads_acts")
    assert_bits(host(d_g), host(r_g), "driver grads")
