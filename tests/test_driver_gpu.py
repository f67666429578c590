"""GPU: the step driver (ugk_gpt2_layers_forward/backward) against the reference launch sequence.

* At the benchmark's own shape (GPT-2-124M, B=8 T=1024 C=768 V=50257 L=12) and at L=16 (more
  than 32 LayerNorm backwards, so the batched column-sum launch runs twice), the driver's every
  activation, gradient and parameter gradient equals a per-op replay of gpt2_kernels.cuh:775-894
  issued through the same library, bit for bit. The per-op kernels are checked against the CPU
  oracle at these shapes in test_parity_gpu.py, so the driver inherits their parity.
* With dense-op callbacks, the driver calls them in the reference's order with the reference's
  buffer offsets and shapes (gpt2_kernels.cuh:787-808 forward, :852-891 backward), and the
  result equals the per-op replay with the same callbacks invoked where the reference calls
  matmul_forward/backward and the attention kernels.

Everything is generated and compared on the device (the buffers at the benchmark shape hold
about 9 GB each).
"""
import pytest
import torch

from test_parity_gpu import ref_offsets

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bits_equal_dev(a, b, what):
    ai, bi = a.view(torch.int32), b.view(torch.int32)
    if not torch.equal(ai, bi):
        bad = (ai != bi).nonzero()
        i = int(bad[0])
        raise AssertionError(f"{what}: {bad.numel()} of {a.numel()} differ; first at {i}: "
                             f"driver {float(a[i])!r} replay {float(b[i])!r}")


def pair_dinp_regions(a, arel, L, NB):
    """(offset, length) of the activation gradients the driver's fused LayerNorm -> residual
    backward pairs read but do not write back: resa and res1 of every block. In gpt2_backward
    (gpt2_kernels.cuh:846-894) each is read last by the residual_backward that follows its
    LayerNorm backward, so the replay's final values there are never used."""
    blk = lambda l, k: a["blk0"] + l * a["bstride"] + arel[k]
    return [(blk(l, k), NB) for l in range(L) for k in ("resa", "res1")]


def clear_regions(t, regions):
    for off, n in regions:
        t[off:off + n] = 0


class Layout:
    def __init__(self, B, T, C, V, maxT, L):
        self.B, self.T, self.C, self.V, self.maxT, self.L = B, T, C, V, maxT, L
        self.p, self.prel, self.a, self.arel = ref_offsets(B, T, C, V, maxT, L)
        self.NB = B * T * C
        self.M = B * T

    def pa(self, l, k):  # parameter offset of block l, tensor k
        return self.p["blk0"] + l * self.p["bstride"] + self.prel[k]

    def aa(self, l, k):  # activation offset of block l, tensor k
        return self.a["blk0"] + l * self.a["bstride"] + self.arel[k]


def make_inputs(gpu, lay, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    p, a, C, L = lay.p, lay.a, lay.C, lay.L
    params = torch.randn(p["total"], generator=g, device=DEV) * 0.02
    for l in range(L):
        for k in ("lng", "ln2g"):
            params[lay.pa(l, k):][:C] += 1.0
    params[p["flng"]:][:C] += 1.0
    acts0 = torch.randn(a["total"], generator=g, device=DEV)
    inputs = torch.randint(0, lay.V, (lay.M,), generator=g, device=DEV, dtype=torch.int32)
    ga0 = torch.zeros(a["total"], device=DEV)
    ga0[a["flo"]:][:lay.NB] = torch.randn(lay.NB, generator=g, device=DEV)
    nblk = L * a["bstride"]
    ga0[a["blk0"]:][:nblk] = torch.randn(nblk, generator=g, device=DEV) * 0.1
    return params, acts0, inputs, ga0


def replay_forward(gpu, lay, acts, params, inputs, dense=None):
    """gpt2_kernels.cuh:775-813 op by op, with the dense ops (if any) where the reference calls them."""
    B, T, C, V, L, NB, M = lay.B, lay.T, lay.C, lay.V, lay.L, lay.NB, lay.M
    A = lambda l, k, n: acts[lay.aa(l, k):][:n]
    P = lambda l, k, n: params[lay.pa(l, k):][:n]
    enc = acts[:NB]
    gpu.encoder_forward(enc, inputs, params[:V * C], params[V * C:][:lay.maxT * C], B, T, C)
    stream = enc
    for l in range(L):
        gpu.layernorm_forward(A(l, "lno", NB), A(l, "lnm", M), A(l, "lnr", M), stream, P(l, "lng", C),
                              P(l, "lnb", C), B, T, C)
        if dense:
            dense.mm_fwd(A(l, "qkv", 3 * NB), A(l, "lno", NB), P(l, "qw", 3 * C * C), P(l, "qb", 3 * C), M, C, 3 * C)
            dense.attn_fwd(A(l, "atty", NB), A(l, "qkv", 3 * NB), B, T, C)
            dense.mm_fwd(A(l, "apr", NB), A(l, "atty", NB), P(l, "pw", C * C), P(l, "pb", C), M, C, C)
        gpu.residual_forward(A(l, "resa", NB), stream, A(l, "apr", NB), NB)
        gpu.layernorm_forward(A(l, "ln2o", NB), A(l, "ln2m", M), A(l, "ln2r", M), A(l, "resa", NB),
                              P(l, "ln2g", C), P(l, "ln2b", C), B, T, C)
        if dense:
            dense.mm_fwd(A(l, "fch", 4 * NB), A(l, "ln2o", NB), P(l, "w1", 4 * C * C), P(l, "b1", 4 * C), M, C,
                         4 * C)
        gpu.gelu_forward(A(l, "gelu", 4 * NB), A(l, "fch", 4 * NB), 4 * NB)
        if dense:
            dense.mm_fwd(A(l, "mlpo", NB), A(l, "gelu", 4 * NB), P(l, "w2", 4 * C * C), P(l, "b2", C), M, 4 * C, C)
        gpu.residual_forward(A(l, "res1", NB), A(l, "resa", NB), A(l, "mlpo", NB), NB)
        stream = A(l, "res1", NB)
    a, p = lay.a, lay.p
    gpu.layernorm_forward(acts[a["flo"]:][:NB], acts[a["flm"]:][:M], acts[a["flr"]:][:M], stream,
                          params[p["flng"]:][:C], params[p["flnb"]:][:C], B, T, C)


def replay_backward(gpu, lay, grads, ga, acts, params, inputs, dense=None):
    """gpt2_kernels.cuh:846-894 op by op (the head's GEMM and cross-entropy excluded, as in the driver)."""
    B, T, C, V, L, NB, M = lay.B, lay.T, lay.C, lay.V, lay.L, lay.NB, lay.M
    a, p = lay.a, lay.p
    GA = lambda off, n: ga[off:][:n]
    AC = lambda off, n: acts[off:][:n]
    G = lambda off, n: grads[off:][:n]
    PR = lambda off, n: params[off:][:n]
    last = lay.aa(L - 1, "res1") if L > 0 else a["enc"]
    gpu.layernorm_backward(GA(last, NB), G(p["flng"], C), G(p["flnb"], C), GA(a["flo"], NB), AC(last, NB),
                           PR(p["flng"], C), AC(a["flm"], M), AC(a["flr"], M), B, T, C)
    for l in range(L - 1, -1, -1):
        st = a["enc"] if l == 0 else lay.aa(l - 1, "res1")
        gpu.residual_backward(GA(lay.aa(l, "resa"), NB), GA(lay.aa(l, "mlpo"), NB), GA(lay.aa(l, "res1"), NB), NB)
        if dense:
            dense.mm_bwd(GA(lay.aa(l, "gelu"), 4 * NB), G(lay.pa(l, "w2"), 4 * C * C), G(lay.pa(l, "b2"), C),
                         AC(lay.aa(l, "gelu"), 4 * NB), PR(lay.pa(l, "w2"), 4 * C * C), GA(lay.aa(l, "mlpo"), NB),
                         M, 4 * C, C)
        gpu.gelu_backward(GA(lay.aa(l, "fch"), 4 * NB), AC(lay.aa(l, "fch"), 4 * NB), GA(lay.aa(l, "gelu"), 4 * NB),
                          4 * NB)
        if dense:
            dense.mm_bwd(GA(lay.aa(l, "ln2o"), NB), G(lay.pa(l, "w1"), 4 * C * C), G(lay.pa(l, "b1"), 4 * C),
                         AC(lay.aa(l, "ln2o"), NB), PR(lay.pa(l, "w1"), 4 * C * C), GA(lay.aa(l, "fch"), 4 * NB),
                         M, C, 4 * C)
        gpu.layernorm_backward(GA(lay.aa(l, "resa"), NB), G(lay.pa(l, "ln2g"), C), G(lay.pa(l, "ln2b"), C),
                               GA(lay.aa(l, "ln2o"), NB), AC(lay.aa(l, "resa"), NB), PR(lay.pa(l, "ln2g"), C),
                               AC(lay.aa(l, "ln2m"), M), AC(lay.aa(l, "ln2r"), M), B, T, C)
        gpu.residual_backward(GA(st, NB), GA(lay.aa(l, "apr"), NB), GA(lay.aa(l, "resa"), NB), NB)
        if dense:
            dense.mm_bwd(GA(lay.aa(l, "atty"), NB), G(lay.pa(l, "pw"), C * C), G(lay.pa(l, "pb"), C),
                         AC(lay.aa(l, "atty"), NB), PR(lay.pa(l, "pw"), C * C), GA(lay.aa(l, "apr"), NB), M, C, C)
            dense.attn_bwd(GA(lay.aa(l, "qkv"), 3 * NB), GA(lay.aa(l, "atty"), NB), AC(lay.aa(l, "qkv"), 3 * NB),
                           B, T, C)
            dense.mm_bwd(GA(lay.aa(l, "lno"), NB), G(lay.pa(l, "qw"), 3 * C * C), G(lay.pa(l, "qb"), 3 * C),
                         AC(lay.aa(l, "lno"), NB), PR(lay.pa(l, "qw"), 3 * C * C), GA(lay.aa(l, "qkv"), 3 * NB),
                         M, C, 3 * C)
        gpu.layernorm_backward(GA(st, NB), G(lay.pa(l, "lng"), C), G(lay.pa(l, "lnb"), C), GA(lay.aa(l, "lno"), NB),
                               AC(st, NB), PR(lay.pa(l, "lng"), C), AC(lay.aa(l, "lnm"), M),
                               AC(lay.aa(l, "lnr"), M), B, T, C)
    gpu.encoder_backward(G(0, V * C), G(V * C, lay.maxT * C), GA(a["enc"], NB), inputs, B, T, C)


def run_driver_vs_replay(gpu, B, T, C, V, NH, maxT, L, seed, dense_factory=None):
    cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=maxT, L=L)
    lay = Layout(B, T, C, V, maxT, L)
    assert gpu.param_count(cfg) == lay.p["total"] and gpu.act_count(cfg) == lay.a["total"]
    params, acts0, inputs, ga0 = make_inputs(gpu, lay, seed)
    d_acts = acts0.clone()
    r_acts = acts0
    del acts0
    d_dense = dense_factory(params, d_acts) if dense_factory else None
    r_dense = dense_factory(params, r_acts) if dense_factory else None
    gpu.gpt2_layers_forward(d_acts, params, inputs, cfg, d_dense.ops if d_dense else None)
    replay_forward(gpu, lay, r_acts, params, inputs, r_dense)
    torch.cuda.synchronize()
    for d in (d_dense, r_dense):
        if d:
            d.raise_errors()
    bits_equal_dev(d_acts, r_acts, "driver forward activations")
    del r_acts
    d_g = torch.zeros(lay.p["total"], device=DEV)
    r_g = torch.zeros(lay.p["total"], device=DEV)
    d_ga = ga0.clone()
    r_ga = ga0
    del ga0
    if dense_factory:
        d_dense.bind_backward(d_g, d_ga)
        r_dense = dense_factory(params, d_acts)
        r_dense.bind_backward(r_g, r_ga)
    gpu.gpt2_layers_backward(d_g, d_ga, d_acts, params, inputs, cfg, d_dense.ops if d_dense else None)
    replay_backward(gpu, lay, r_g, r_ga, d_acts, params, inputs, r_dense)
    torch.cuda.synchronize()
    for d in (d_dense, r_dense):
        if d:
            d.raise_errors()
    skip = pair_dinp_regions(lay.a, lay.arel, L, lay.NB)
    clear_regions(d_ga, skip)
    clear_regions(r_ga, skip)
    bits_equal_dev(d_ga, r_ga, "driver grads_acts (all but the pairs' dinp)")
    bits_equal_dev(d_g, r_g, "driver grads")
    return d_dense


@pytest.mark.parametrize("B,T,C,V,L", [
    (8, 1024, 768, 50257, 12),  # the benchmark's step: GPT-2-124M, 25 LayerNorm backwards of 512 partial rows
    (2, 64, 768, 50, 16),       # 33 LayerNorm backwards: the batched column sums take two launches
    (2, 32, 384, 27, 6),        # config 1's width and depth
    (2, 32, 384, 27, 0),        # no block: the encoder -> LayerNorm pass writes the final LayerNorm
    (2, 16, 1024, 27, 2),       # four float4 per lane (GPT-2 medium's width)
    (1, 16, 2048, 11, 1),       # eight, the widest row held in registers
])
def test_step_driver_equals_per_op_replay_at_shape(gpu, B, T, C, V, L):
    print(f"driver vs replay B={B} T={T} C={C} V={V} L={L}", flush=True)
    prev = gpu.lib.ugk_get_stream()
    gpu.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        run_driver_vs_replay(gpu, B, T, C, V, 12 if C % 12 == 0 else 4, max(T, 64), L, seed=B * 1000 + L)
    finally:
        gpu.set_stream(prev)
        torch.cuda.empty_cache()


class TorchDense:
    """Dense-op callbacks for the driver: deterministic elementwise stand-ins for the GEMMs and the
    attention kernels, run with torch on views of the caller's buffers (found from the raw pointers
    the driver passes), on the library's stream. Each call is also recorded as (op, buffer, offset)
    per pointer plus its integer shape arguments."""

    def __init__(self, params, acts):
        self.bases = {"params": params, "acts": acts}
        self.calls, self.errors = [], []
        self.ops = gpu_dense_ops(self)

    def bind_backward(self, grads, grads_acts):
        self.bases.update({"grads": grads, "grads_acts": grads_acts})

    def where(self, ptr):
        for name, t in self.bases.items():
            lo = t.data_ptr()
            if lo <= ptr < lo + 4 * t.numel():
                assert (ptr - lo) % 4 == 0
                return name, (ptr - lo) // 4
        raise AssertionError(f"pointer {ptr:#x} is in none of the caller's buffers")

    def view(self, ptr, n):
        name, off = self.where(ptr)
        return self.bases[name][off:][:n]

    def record(self, op, ptrs, ints):
        self.calls.append((op, tuple(self.where(p) for p in ptrs), tuple(ints)))

    def raise_errors(self):
        if self.errors:
            raise AssertionError("dense callback failed: " + self.errors[0])

    # the stand-ins (same functions for the driver's callbacks and the replay's direct calls)
    @staticmethod
    def mm_fwd(out, inp, weight, bias, M, C, OC):
        idx = torch.arange(OC, device=DEV) % C
        out.view(M, OC).copy_(inp.view(M, C).index_select(1, idx) * 0.5 + bias.view(1, OC) +
                              weight[:OC].view(1, OC))

    @staticmethod
    def mm_bwd(dinp, dweight, dbias, inp, weight, dout, M, C, OC):
        idx = torch.arange(C, device=DEV) % OC
        dinp.view(M, C).add_(dout.view(M, OC).index_select(1, idx) * 0.25 + weight[:C].view(1, C))
        dweight[:OC].add_(dout.view(M, OC)[0] * inp[0])
        dbias.add_(dout.view(M, OC)[M - 1])

    @staticmethod
    def attn_fwd(out, qkv, B, T, C):
        q = qkv.view(B * T, 3 * C)
        out.view(B * T, C).copy_(q[:, :C] * 0.5 + q[:, 2 * C:] * 0.25)

    @staticmethod
    def attn_bwd(dqkv, dout, qkv, B, T, C):
        dq, d, q = dqkv.view(B * T, 3 * C), dout.view(B * T, C), qkv.view(B * T, 3 * C)
        dq[:, :C].add_(d * 0.5)
        dq[:, 2 * C:].add_(d * q[:, C:2 * C] * 0.125)


def gpu_dense_ops(td):
    import ugk

    def guard(fn):
        def wrapped(*a):
            try:
                fn(*a)
                return 0
            except Exception as e:  # a nonzero status makes the driver stop with an error
                td.errors.append(repr(e))
                return 1
        return wrapped

    def mm_fwd(ctx, out, inp, weight, bias, M, C, OC):
        td.record("matmul_forward", (out, inp, weight, bias), (M, C, OC))
        td.mm_fwd(td.view(out, M * OC), td.view(inp, M * C), td.view(weight, C * OC), td.view(bias, OC), M, C, OC)

    def mm_bwd(ctx, dinp, dweight, dbias, inp, weight, dout, M, C, OC):
        td.record("matmul_backward", (dinp, dweight, dbias, inp, weight, dout), (M, C, OC))
        td.mm_bwd(td.view(dinp, M * C), td.view(dweight, C * OC), td.view(dbias, OC), td.view(inp, M * C),
                  td.view(weight, C * OC), td.view(dout, M * OC), M, C, OC)

    def attn_fwd(ctx, out, qkv, B, T, C, NH):
        td.record("attention_forward", (out, qkv), (B, T, C, NH))
        td.attn_fwd(td.view(out, B * T * C), td.view(qkv, 3 * B * T * C), B, T, C)

    def attn_bwd(ctx, dqkv, dout, qkv, B, T, C, NH):
        td.record("attention_backward", (dqkv, dout, qkv), (B, T, C, NH))
        td.attn_bwd(td.view(dqkv, 3 * B * T * C), td.view(dout, B * T * C), td.view(qkv, 3 * B * T * C), B, T, C)

    td._keep = (ugk._MATMUL_FWD(guard(mm_fwd)), ugk._MATMUL_BWD(guard(mm_bwd)),
                ugk._ATTN_FWD(guard(attn_fwd)), ugk._ATTN_BWD(guard(attn_bwd)))
    return ugk.DenseOps(None, *td._keep)


def expected_dense_calls(lay, NH):
    """The dense calls of gpt2_forward/backward (gpt2_kernels.cuh:787-808, :852-891) between the
    encoder and the final LayerNorm, with (buffer, offset) per pointer, as TorchDense records them."""
    B, T, C, L, M = lay.B, lay.T, lay.C, lay.L, lay.M
    A = lambda l, k: ("acts", lay.aa(l, k))
    P = lambda l, k: ("params", lay.pa(l, k))
    G = lambda l, k: ("grads", lay.pa(l, k))
    GA = lambda l, k: ("grads_acts", lay.aa(l, k))
    fwd = []
    for l in range(L):
        fwd += [("matmul_forward", (A(l, "qkv"), A(l, "lno"), P(l, "qw"), P(l, "qb")), (M, C, 3 * C)),
                ("attention_forward", (A(l, "atty"), A(l, "qkv")), (B, T, C, NH)),
                ("matmul_forward", (A(l, "apr"), A(l, "atty"), P(l, "pw"), P(l, "pb")), (M, C, C)),
                ("matmul_forward", (A(l, "fch"), A(l, "ln2o"), P(l, "w1"), P(l, "b1")), (M, C, 4 * C)),
                ("matmul_forward", (A(l, "mlpo"), A(l, "gelu"), P(l, "w2"), P(l, "b2")), (M, 4 * C, C))]
    bwd = []
    for l in range(L - 1, -1, -1):
        bwd += [("matmul_backward", (GA(l, "gelu"), G(l, "w2"), G(l, "b2"), A(l, "gelu"), P(l, "w2"),
                                     GA(l, "mlpo")), (M, 4 * C, C)),
                ("matmul_backward", (GA(l, "ln2o"), G(l, "w1"), G(l, "b1"), A(l, "ln2o"), P(l, "w1"),
                                     GA(l, "fch")), (M, C, 4 * C)),
                ("matmul_backward", (GA(l, "atty"), G(l, "pw"), G(l, "pb"), A(l, "atty"), P(l, "pw"),
                                     GA(l, "apr")), (M, C, C)),
                ("attention_backward", (GA(l, "qkv"), GA(l, "atty"), A(l, "qkv")), (B, T, C, NH)),
                ("matmul_backward", (GA(l, "lno"), G(l, "qw"), G(l, "qb"), A(l, "lno"), P(l, "qw"),
                                     GA(l, "qkv")), (M, C, 3 * C))]
    return fwd, bwd


@pytest.mark.parametrize("B,T,C,NH,L", [(2, 16, 64, 2, 2), (2, 32, 384, 6, 3)])
def test_step_driver_dense_callbacks(gpu, B, T, C, NH, L):
    """The driver calls the dense ops in the reference's order, on the reference's buffers, and its
    result with them equals the reference sequence replayed op by op with the same dense ops."""
    V = 27
    prev = gpu.lib.ugk_get_stream()
    gpu.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        d = run_driver_vs_replay(gpu, B, T, C, V, NH, max(T, 32), L, seed=77 + L, dense_factory=TorchDense)
    finally:
        gpu.set_stream(prev)
    lay = Layout(B, T, C, V, max(T, 32), L)
    fwd, bwd = expected_dense_calls(lay, NH)
    assert d.calls[:len(fwd)] == fwd, "forward dense calls differ from gpt2_kernels.cuh:787-808"
    assert d.calls[len(fwd):] == bwd, "backward dense calls differ from gpt2_kernels.cuh:852-891"


def test_step_driver_reports_a_failing_callback(gpu):
    """A dense op that returns nonzero stops the driver with an error naming the op."""
    B, T, C, NH, L, V = 1, 8, 64, 2, 1, 11
    cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=8, L=L)
    acts = torch.zeros(gpu.act_count(cfg), device=DEV)
    params = torch.zeros(gpu.param_count(cfg), device=DEV)
    inputs = torch.zeros(B * T, device=DEV, dtype=torch.int32)
    import ugk
    fail = ugk._MATMUL_FWD(lambda *a: 7)
    ops = ugk.DenseOps(None, fail, ugk._MATMUL_BWD(), ugk._ATTN_FWD(), ugk._ATTN_BWD())
    with pytest.raises(gpu.UgkError, match="matmul_forward"):
        gpu.gpt2_layers_forward(acts, params, inputs, cfg, ops)


def first_write_regions(lay):
    """(offset, length) of the activation gradients that the layer kernels are the first to write in
    gpt2_backward (gpt2_kernels.cuh:846-894) when grads_acts starts at zero outside flo: enc and
    fch, mlpo, apr, resa and res1 of every block (GELU backward's dinp and the residual splits'
    dx and dy; res1 of the last block is the final LayerNorm's dinp)."""
    NB = lay.NB
    out = [(lay.a["enc"], NB)]
    for l in range(lay.L):
        out += [(lay.aa(l, "fch"), 4 * NB)] + [(lay.aa(l, k), NB) for k in ("mlpo", "apr", "resa", "res1")]
    return out


@pytest.mark.parametrize("B,T,C,V,L,garbage", [
    (8, 1024, 768, 50257, 12, True),  # the benchmark's step
    (2, 64, 768, 50, 3, True),        # row teams, few rows
    (2, 32, 384, 27, 6, True),        # the two-rows-per-wavefront kernels (C = 384)
    (2, 16, 1024, 27, 2, True),       # four float4 per lane
    (1, 16, 2048, 11, 1, True),       # eight float4 per lane
    (2, 32, 384, 27, 0, False),       # no block: the final LayerNorm reads enc
    (2, 16, 30, 11, 2, False),        # C = 30: the scalar LayerNorm path reads its residual targets
])
def test_zeroed_driver_equals_driver(gpu, B, T, C, V, L, garbage):
    """ugk_gpt2_layers_backward_zeroed on a grads_acts that is zero where the layer kernels write first
    equals ugk_gpt2_layers_backward on it, bit for bit (every parameter gradient, every activation
    gradient but the pairs' unwritten dinp). Where it reads none of those buffers (float4 path,
    L >= 1) it is also given garbage there instead of zeros, and must not notice."""
    print(f"zeroed driver B={B} T={T} C={C} V={V} L={L} garbage={garbage}", flush=True)
    prev = gpu.lib.ugk_get_stream()
    gpu.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        NH = 12 if C % 12 == 0 else (5 if C % 5 == 0 else 1)
        cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=max(T, 64), L=L)
        lay = Layout(B, T, C, V, max(T, 64), L)
        params, acts, inputs, ga0 = make_inputs(gpu, lay, seed=B * 100 + L)
        gpu.gpt2_layers_forward(acts, params, inputs, cfg)
        first = first_write_regions(lay)
        clear_regions(ga0, first)
        ga_acc, ga_zero = ga0.clone(), ga0.clone()
        if garbage:
            g = torch.Generator(device=DEV)
            g.manual_seed(7)
            for off, n in first:
                ga_zero[off:off + n] = torch.randn(n, generator=g, device=DEV) * 3.0
        g_acc = torch.zeros(lay.p["total"], device=DEV)
        g_zero = torch.zeros(lay.p["total"], device=DEV)
        gpu.gpt2_layers_backward(g_acc, ga_acc, acts, params, inputs, cfg)
        gpu.gpt2_layers_backward_zeroed(g_zero, ga_zero, acts, params, inputs, cfg)
        torch.cuda.synchronize()
        skip = pair_dinp_regions(lay.a, lay.arel, L, lay.NB)
        clear_regions(ga_acc, skip)
        clear_regions(ga_zero, skip)
        bits_equal_dev(ga_zero, ga_acc, "zeroed driver grads_acts (all but the pairs' dinp)")
        bits_equal_dev(g_zero, g_acc, "zeroed driver grads")
    finally:
        gpu.set_stream(prev)
        torch.cuda.empty_cache()


def test_zeroed_driver_with_dense_callbacks(gpu):
    """With dense-op callbacks (which accumulate, as the arms' GEMMs do) and grads_acts zero outside
    flo, the zeroed backward equals the accumulating one bit for bit."""
    B, T, C, V, NH, L = 2, 32, 384, 27, 6, 3
    prev = gpu.lib.ugk_get_stream()
    gpu.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        cfg = gpu.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=max(T, 32), L=L)
        lay = Layout(B, T, C, V, max(T, 32), L)
        params, acts, inputs, ga0 = make_inputs(gpu, lay, seed=91)
        ga0[lay.a["blk0"]:lay.a["blk0"] + L * lay.a["bstride"]] = 0  # the arms' memset (flo keeps its gradient)
        ga0[lay.a["enc"]:lay.a["enc"] + lay.NB] = 0
        dense = TorchDense(params, acts)
        gpu.gpt2_layers_forward(acts, params, inputs, cfg, dense.ops)
        torch.cuda.synchronize()
        dense.raise_errors()
        out = []
        for fn in (gpu.gpt2_layers_backward, gpu.gpt2_layers_backward_zeroed):
            g, ga = torch.zeros(lay.p["total"], device=DEV), ga0.clone()
            d = TorchDense(params, acts)
            d.bind_backward(g, ga)
            fn(g, ga, acts, params, inputs, cfg, d.ops)
            torch.cuda.synchronize()
            d.raise_errors()
            clear_regions(ga, pair_dinp_regions(lay.a, lay.arel, L, lay.NB))
            out.append((g, ga))
        bits_equal_dev(out[1][1], out[0][1], "zeroed driver grads_acts with callbacks")
        bits_equal_dev(out[1][0], out[0][0], "zeroed driver grads with callbacks")
    finally:
        gpu.set_stream(prev)
