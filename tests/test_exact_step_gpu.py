"""GPU: with every exact mode on (GELU, encoder backward, LayerNorm), the step driver
(ugk_gpt2_layers_forward/backward) equals a CPU replay of the reference launch sequence
(gpt2_kernels.cuh:775-813 forward, :846-894 backward) made of the oracle's ops (train_bnn.c) bit for
bit: every activation the layer kernels write, every activation gradient, and every parameter
gradient (LayerNorm dweight/dbias, dwte, dwpe). Shapes: a small one, benchmark config 1 exactly
(GPT-2 L=6 H=6 C=384 V=27 B=4 T=64, maxT=1024, the parameters materialised from mu, rho, eps with
LayerNorm gamma = 1 and beta = 0), and the rows and width of config 5 (B=8 T=1024 C=768 V=50257) at
L=2. The dense ops (GEMMs, attention) are absent; their output buffers hold random data, as in
test_driver_oracle_gpu.py, whose default-mode bars this test replaces by bit identity."""
import numpy as np
import pytest
import torch

import gen
from test_parity_gpu import assert_bits as _assert_bits, host, ref_offsets

pytestmark = pytest.mark.gpu
DEV = "cuda"


def assert_bits(got, want, what):
    _assert_bits(np.ravel(got), np.ravel(want), what)


SHAPES = {  # name: B, T, C, V, NH, maxT, L, materialise the parameters first
    "small": (2, 16, 64, 11, 2, 16, 2, False),
    "cfg1": (4, 64, 384, 27, 6, 1024, 6, True),
    "cfg5 rows L=2": (8, 1024, 768, 50257, 12, 1024, 2, False),
}


class all_exact:
    def __init__(self, gpu):
        self.gpu = gpu

    def __enter__(self):
        for f in (self.gpu.set_gelu_exact, self.gpu.set_encoder_exact, self.gpu.set_layernorm_exact):
            f(True)

    def __exit__(self, *a):
        for f in (self.gpu.set_gelu_exact, self.gpu.set_encoder_exact, self.gpu.set_layernorm_exact):
            f(False)


@pytest.mark.parametrize("zeroed", [False, True])
@pytest.mark.parametrize("name", list(SHAPES))
def test_exact_step_driver_equals_oracle_replay(gpu, oracle, name, zeroed):
    B, T, C, V, NH, maxT, L, materialise = SHAPES[name]
    print(f"exact step driver vs oracle replay: {name} B={B} T={T} C={C} V={V} L={L} zeroed={zeroed}", flush=True)
    cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=maxT, L=L)
    p, prel, a, arel = ref_offsets(B, T, C, V, maxT, L)
    BT, NB = B * T, B * T * C
    g = gen.rng(77 + L)
    PO = lambda l, k: p["blk0"] + l * p["bstride"] + prel[k]
    AO = lambda l, k: a["blk0"] + l * a["bstride"] + arel[k]
    ln_params = [(PO(l, "lng"), PO(l, "lnb")) for l in range(L)] + [(PO(l, "ln2g"), PO(l, "ln2b")) for l in range(L)]
    ln_params.append((p["flng"], p["flnb"]))
    if materialise:
        n = p["total"]
        mu, rho, eps = gen.normal(g, (n,), 0, 0.02), gen.normal(g, (n,), -5, 0.1), gen.normal(g, (n,))
        params = np.zeros(n, np.float32)
        oracle.bayes_materialize(params, mu, rho, eps, n)
        for gs, bs in ln_params:
            params[gs:gs + C] = 1.0
            params[bs:bs + C] = 0.0
        del mu, rho, eps
    else:
        params = gen.normal(g, (p["total"],), 0, 0.02)
        for gs, _ in ln_params:
            params[gs:gs + C] += 1.0
    tpar = torch.from_numpy(params).to(DEV)
    used = a["flr"] + BT
    acts = gen.normal(g, (used,))
    inputs = gen.tokens_uniform(g, BT, V)
    tacts = torch.zeros(a["total"], device=DEV)
    tacts[:used] = torch.from_numpy(acts).to(DEV)
    tin = torch.from_numpy(inputs).to(DEV)
    with all_exact(gpu):
        gpu.gpt2_layers_forward(tacts, tpar, tin, cfg)
    gacts = host(tacts[:used])

    # forward replay
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
    assert_bits(gacts, cacts, "forward activations (every layer-kernel output)")
    del cacts

    # backward: the dense ops' gradients as given; everything else zero on entry (what the
    # zeroed-gradient backward requires, and what the arms' memset provides)
    ga0 = np.zeros(used, np.float32)
    ga0[a["flo"]:a["flo"] + NB] = gen.normal(g, (NB,))
    for l in range(L):
        for k, n in (("gelu", 4 * NB), ("ln2o", NB), ("lno", NB)):
            ga0[AO(l, k):AO(l, k) + n] = gen.normal(g, (n,))
    tg = torch.zeros(p["total"], device=DEV)
    tga = torch.zeros(a["total"], device=DEV)
    tga[:used] = torch.from_numpy(ga0).to(DEV)
    with all_exact(gpu):
        (gpu.gpt2_layers_backward_zeroed if zeroed else gpu.gpt2_layers_backward)(tg, tga, tacts, tpar, tin, cfg)
    cg, cga, ca = np.zeros(p["total"], np.float32), ga0.copy(), gacts
    GA = lambda off, n: cga[off:][:n]

    def ln_bwd(dinp, gs, bs, dout, x, mean, rstd):
        oracle.layernorm_backward(GA(dinp, NB), cg[gs:][:C], cg[bs:][:C], GA(dout, NB), ca[x:][:NB],
                                  params[gs:][:C], ca[mean:][:BT], ca[rstd:][:BT], B, T, C)

    last = AO(L - 1, "res1")
    ln_bwd(last, p["flng"], p["flnb"], a["flo"], last, a["flm"], a["flr"])
    for l in range(L - 1, -1, -1):
        st = a["enc"] if l == 0 else AO(l - 1, "res1")
        oracle.residual_backward(GA(AO(l, "resa"), NB), GA(AO(l, "mlpo"), NB), GA(AO(l, "res1"), NB), NB)
        oracle.gelu_backward(GA(AO(l, "fch"), 4 * NB), ca[AO(l, "fch"):][:4 * NB], GA(AO(l, "gelu"), 4 * NB),
                             4 * NB)
        ln_bwd(AO(l, "resa"), PO(l, "ln2g"), PO(l, "ln2b"), AO(l, "ln2o"), AO(l, "resa"), AO(l, "ln2m"),
               AO(l, "ln2r"))
        oracle.residual_backward(GA(st, NB), GA(AO(l, "apr"), NB), GA(AO(l, "resa"), NB), NB)
        ln_bwd(st, PO(l, "lng"), PO(l, "lnb"), AO(l, "lno"), st, AO(l, "lnm"), AO(l, "lnr"))
    oracle.encoder_backward(cg[:V * C], cg[V * C:V * C + maxT * C], GA(a["enc"], NB), inputs, B, T, C)
    assert_bits(host(tga[:used]), cga, "activation gradients")
    assert_bits(host(tg), cg, "parameter gradients (LayerNorm dweight/dbias, dwte, dwpe)")
