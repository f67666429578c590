"""GPU: the step driver (ugk_gpt2_layers_forward/backward) against a CPU replay of the reference
launch sequence (gpt2_kernels.cuh:775-813 forward, :846-894 backward) made of the oracle's ops
(train_bnn.c) on the reference's flat layout (gpt2_kernels.cuh:656-719, restated independently
in ref_offsets), at three shapes: a small one, benchmark config 1 exactly (GPT-2 L=6 H=6 C=384
V=27 B=4 T=64, maxT=1024 as the reference's CPU run allocates; the parameters materialised from
mu ~ N(0,0.02), rho = -5 + N(0,0.1), eps ~ N(0,1), then LayerNorm gamma = 1 and beta = 0), and
the rows and width of config 5 (B=8 T=1024 C=768 V=50257) at L=2 (a full L=12 replay would need
some 9 GB per activation buffer on the host).

The dense ops between the layer kernels (GEMMs, attention) are absent, so their output buffers
hold whatever the test puts there; only the regions of the activation buffers that the layer
kernels use are filled (the logits and probabilities, 823M floats at config 5, stay zero).

Bars: the encoder output and the residual stream are bit-exact (bit-exact ops on identical inputs);
each LayerNorm and GELU output is within the literal bar of one op (|gpu - cpu| <= 1e-6 + 1e-5
|cpu|); the backward's activation gradients accumulate the 2L+1 LayerNorm backwards' dinp through
the residual splits, and are held to 2e-5 of the sum of the magnitudes of what was added into
each (the literal bar of each LayerNorm and GELU term, plus the rounding of the sums), since the
terms (~50) can cancel to ~1e-3; each LayerNorm's dweight /
dbias (column sums over B*T rows, whose fp32 value depends on the order) to the scale-aware bar
1e-5 * sum of |terms| of the other LayerNorm tests; dwte / dwpe equal the oracle's encoder_backward
of the driver's own encoder gradient bit for bit (that gradient is held to the bar above), and no
other parameter gradient is written.
"""
import numpy as np
import pytest
import torch

import gen
from test_parity_gpu import assert_bits, assert_close, host, ref_offsets

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = {  # name: B, T, C, V, NH, maxT, L, materialise the parameters first
    "small": (2, 16, 64, 11, 2, 16, 2, False),
    "cfg1": (4, 64, 384, 27, 6, 1024, 6, True),
    "cfg5 rows L=2": (8, 1024, 768, 50257, 12, 1024, 2, False),
}


def literal(got, want, what):
    assert_close(got, want, what, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", list(SHAPES))
def test_step_driver_matches_oracle_replay(gpu, oracle, name):
    B, T, C, V, NH, maxT, L, materialise = SHAPES[name]
    print(f"step driver vs oracle replay: {name} B={B} T={T} C={C} V={V} L={L}", flush=True)
    cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=maxT, L=L)
    p, prel, a, arel = ref_offsets(B, T, C, V, maxT, L)
    assert gpu.param_count(cfg) == p["total"] and gpu.act_count(cfg) == a["total"]
    BT, NB = B * T, B * T * C
    g = gen.rng(66 + L)
    PO = lambda l, k: p["blk0"] + l * p["bstride"] + prel[k]
    AO = lambda l, k: a["blk0"] + l * a["bstride"] + arel[k]
    ln_params = [(PO(l, "lng"), PO(l, "lnb")) for l in range(L)] + [(PO(l, "ln2g"), PO(l, "ln2b")) for l in range(L)]
    ln_params.append((p["flng"], p["flnb"]))
    if materialise:
        n = p["total"]
        mu, rho, eps = gen.normal(g, (n,), 0, 0.02), gen.normal(g, (n,), -5, 0.1), gen.normal(g, (n,))
        tpar = torch.empty(n, device=DEV)
        gpu.bayes_materialize(tpar, torch.from_numpy(mu).to(DEV), torch.from_numpy(rho).to(DEV),
                              torch.from_numpy(eps).to(DEV), n)
        params = np.zeros(n, np.float32)
        oracle.bayes_materialize(params, mu, rho, eps, n)
        assert_bits(host(tpar), params, "materialised parameters")
        for gs, bs in ln_params:
            params[gs:gs + C] = 1.0
            params[bs:bs + C] = 0.0
        del mu, rho, eps
    else:
        params = gen.normal(g, (p["total"],), 0, 0.02)
        for gs, _ in ln_params:  # LN gains near 1
            params[gs:gs + C] += 1.0
    tpar = torch.from_numpy(params).to(DEV)
    # activations: the layer kernels' region (everything before the logits) on the host; the
    # dense ops' outputs (qkv, atty, apr, fch, mlpo) hold random data, the rest is overwritten
    used = a["flr"] + BT
    acts = gen.normal(g, (used,))
    inputs = gen.tokens_uniform(g, BT, V)
    tacts = torch.zeros(a["total"], device=DEV)
    tacts[:used] = torch.from_numpy(acts).to(DEV)
    tin = torch.from_numpy(inputs).to(DEV)
    gpu.gpt2_layers_forward(tacts, tpar, tin, cfg)
    gacts = host(tacts[:used])

    # CPU replay of gpt2_kernels.cuh:775-813 with the oracle's ops
    cacts = acts.copy()
    A = lambda l, k, n: cacts[AO(l, k):][:n]
    P = lambda l, k, n: params[PO(l, k):][:n]
    enc = cacts[:NB]
    oracle.encoder_forward(enc, inputs, params[:V * C], params[V * C:V * C + maxT * C], B, T, C)
    stream = enc
    for l in range(L):
        oracle.layernorm_forward(A(l, "lno", NB), A(l, "lnm", BT), A(l, "lnr", BT), stream,
                                 P(l, "lng", C), P(l, "lnb", C), B, T, C)
        oracle.residual_forward(A(l, "resa", NB), stream, A(l, "apr", NB), NB)
        oracle.layernorm_forward(A(l, "ln2o", NB), A(l, "ln2m", BT), A(l, "ln2r", BT), A(l, "resa", NB),
                                 P(l, "ln2g", C), P(l, "ln2b", C), B, T, C)
        oracle.gelu_forward(A(l, "gelu", 4 * NB), A(l, "fch", 4 * NB), 4 * NB)
        oracle.residual_forward(A(l, "res1", NB), A(l, "resa", NB), A(l, "mlpo", NB), NB)
        stream = A(l, "res1", NB)
    oracle.layernorm_forward(cacts[a["flo"]:][:NB], cacts[a["flm"]:][:BT], cacts[a["flr"]:][:BT], stream,
                             params[p["flng"]:][:C], params[p["flnb"]:][:C], B, T, C)
    G = lambda off, n: gacts[off:off + n]
    Cc = lambda off, n: cacts[off:off + n]
    assert_bits(G(0, NB), Cc(0, NB), "encoder output")
    for l in range(L):
        for k, n in (("resa", NB), ("res1", NB)):
            assert_bits(G(AO(l, k), n), Cc(AO(l, k), n), f"block {l} {k}")
        for k, n in (("lno", NB), ("lnm", BT), ("lnr", BT), ("ln2o", NB), ("ln2m", BT), ("ln2r", BT),
                     ("gelu", 4 * NB)):
            literal(G(AO(l, k), n), Cc(AO(l, k), n), f"block {l} {k}")
        for k, n in (("qkv", 3 * NB), ("atty", NB), ("apr", NB), ("fch", 4 * NB), ("mlpo", NB)):
            assert_bits(G(AO(l, k), n), Cc(AO(l, k), n), f"block {l} {k} (not a layer-kernel output)")
    for off, n, k in ((a["flo"], NB, "flo"), (a["flm"], BT, "flm"), (a["flr"], BT, "flr")):
        literal(G(off, n), Cc(off, n), f"final LayerNorm {k}")
    del cacts

    # backward from identical activations (the GPU forward's)
    ga0 = np.zeros(used, np.float32)
    ga0[a["flo"]:a["flo"] + NB] = gen.normal(g, (NB,))
    for l in range(L):  # the dense backward ops' outputs, which the layer kernels read
        for k, n in (("gelu", 4 * NB), ("ln2o", NB), ("lno", NB)):
            ga0[AO(l, k):AO(l, k) + n] = gen.normal(g, (n,))
    tg = torch.zeros(p["total"], device=DEV)
    tga = torch.zeros(a["total"], device=DEV)
    tga[:used] = torch.from_numpy(ga0).to(DEV)
    gpu.gpt2_layers_backward(tg, tga, tacts, tpar, tin, cfg)
    cg, cga, ca = np.zeros(p["total"], np.float32), ga0.copy(), gacts
    GA = lambda off, n: cga[off:][:n]
    lns = []  # (dout, x, mean, rstd, dweight offset, dbias offset) of each LayerNorm backward
    # The scale each activation gradient is held to: the sum of the magnitudes of what was added into
    # it. A LayerNorm or GELU backward adds a term computed afresh from given inputs (its error is
    # relative to itself); a residual split adds its dout, carrying dout's own scale. The fp32 sums
    # of terms of magnitude ~50 can cancel to ~1e-3, so a bar relative to the result alone is wrong.
    scale = np.zeros(used, np.float32)

    def fresh(off, n, before):
        scale[off:off + n] += np.abs(cga[off:off + n] - before)

    def ln_bwd(dinp, gs, bs, dout, x, mean, rstd):
        before = GA(dinp, NB).copy()
        oracle.layernorm_backward(GA(dinp, NB), cg[gs:][:C], cg[bs:][:C], GA(dout, NB), ca[x:][:NB],
                                  params[gs:][:C], ca[mean:][:BT], ca[rstd:][:BT], B, T, C)
        fresh(dinp, NB, before)
        lns.append((dout, x, mean, rstd, gs, bs))

    def res_bwd(dx, dy, dout):
        oracle.residual_backward(GA(dx, NB), GA(dy, NB), GA(dout, NB), NB)
        carried = scale[dout:dout + NB] + np.abs(GA(dout, NB))
        scale[dx:dx + NB] += carried
        scale[dy:dy + NB] += carried

    last = AO(L - 1, "res1")
    ln_bwd(last, p["flng"], p["flnb"], a["flo"], last, a["flm"], a["flr"])
    for l in range(L - 1, -1, -1):
        st = a["enc"] if l == 0 else AO(l - 1, "res1")
        res_bwd(AO(l, "resa"), AO(l, "mlpo"), AO(l, "res1"))
        before = GA(AO(l, "fch"), 4 * NB).copy()
        oracle.gelu_backward(GA(AO(l, "fch"), 4 * NB), ca[AO(l, "fch"):][:4 * NB], GA(AO(l, "gelu"), 4 * NB),
                             4 * NB)
        fresh(AO(l, "fch"), 4 * NB, before)
        ln_bwd(AO(l, "resa"), PO(l, "ln2g"), PO(l, "ln2b"), AO(l, "ln2o"), AO(l, "resa"), AO(l, "ln2m"),
               AO(l, "ln2r"))
        res_bwd(st, AO(l, "apr"), AO(l, "resa"))
        ln_bwd(st, PO(l, "lng"), PO(l, "lnb"), AO(l, "lno"), st, AO(l, "lnm"), AO(l, "lnr"))
    oracle.encoder_backward(cg[:V * C], cg[V * C:V * C + maxT * C], GA(a["enc"], NB), inputs, B, T, C)
    hga, hg = host(tga[:used]), host(tg)
    # the encoder backward on the driver's own encoder gradient: bit-exact (no token repeats more
    # than 32 times at these shapes, so the blocked and exact orders are the CPU's)
    want_wte, want_wpe = np.zeros(V * C, np.float32), np.zeros(maxT * C, np.float32)
    oracle.encoder_backward(want_wte, want_wpe, hga[a["enc"]:a["enc"] + NB], inputs, B, T, C)
    assert_bits(hg[:V * C], want_wte, "dwte from the driver's encoder gradient")
    assert_bits(hg[V * C:V * C + maxT * C], want_wpe, "dwpe from the driver's encoder gradient")
    hg[:V * C + maxT * C] = 0
    cg[:V * C + maxT * C] = 0
    # the fused LayerNorm -> residual pairs read resa and res1 of each block as dinp without writing
    # them back (the reference reads them only in the residual_backward the pair fuses)
    for l in range(L):
        for k in ("resa", "res1"):
            hga[AO(l, k):AO(l, k) + NB] = 0
            cga[AO(l, k):AO(l, k) + NB] = 0
    err = np.abs(hga.astype(np.float64) - cga)
    bar = 2e-5 * scale.astype(np.float64) + 1e-6
    bad = err > bar
    assert not bad.any(), (f"activation gradients: {int(bad.sum())} beyond 2e-5 of their scale; worst at "
                           f"{int(np.argmax(err - bar))}")
    print(f"{name}: activation gradients within {float((err / (scale + 1e-30)).max()):.2e} of their scale")
    # LayerNorm dweight / dbias: the scale-aware bar
    for dout, x, mean, rstd, gs, bs in lns:
        d64 = ga0[dout:dout + NB].astype(np.float64).reshape(BT, C)  # the dense ops' gradients, as given
        xhat = (ca[x:x + NB].astype(np.float64).reshape(BT, C) - ca[mean:mean + BT, None]) * ca[rstd:rstd + BT, None]
        for what, off, terms in (("dweight", gs, d64 * xhat), ("dbias", bs, d64)):
            scale = np.abs(terms).sum(0)
            got, want = hg[off:off + C].astype(np.float64), cg[off:off + C].astype(np.float64)
            assert (np.abs(got - want) <= 1e-5 * scale + 1e-30).all(), f"LayerNorm at {off}: {what}"
            hg[off:off + C] = 0
            cg[off:off + C] = 0
    assert not hg.any() and not cg.any(), "a parameter gradient outside the layer kernels' was written"
