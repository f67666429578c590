"""GPU: the Python binding's calls stay asynchronous.

The token and target ids that index tables (rows of wte, logits of a row) are checked on the device
(ugk_ids_guard, on the library's stream) instead of being read back to the host: no call of the
binding synchronises the device (checked with torch's sync debug mode), and an id out of range is
replaced in place, so that no kernel indexes outside its table, and reported by the next
synchronize(). The reference (train_bnn.c:41-65, :279-304, :358-378, :647-662) leaves
0 <= id < V to its callers; with valid ids every result is the oracle's.
"""
import numpy as np
import pytest
import torch

import gen
from test_parity_gpu import assert_bits, dev, host

pytestmark = pytest.mark.gpu
DEV = "cuda"


def head_case(g, rows, V):
    return gen.normal(g, (rows * V,), 0, 3.0), gen.tokens_uniform(g, rows, V)


# torch notes that its sync-debug mode is a prototype each time the mode is set; the notice is expected
@pytest.mark.filterwarnings("ignore:Synchronization debug mode is a prototype")
def test_token_ops_do_not_synchronize(gpu, oracle):
    B, T, C, V = 4, 64, 384, 27  # config 1
    g = gen.rng(777)
    inp = gen.tokens_uniform(g, B * T, V)
    wte, wpe, dout = gen.normal(g, (V * C,), 0, 0.02), gen.normal(g, (T * C,), 0, 0.01), gen.normal(g, (B * T * C,))
    w, b = gen.normal(g, (C,), 1, 0.1), gen.normal(g, (C,), 0, 0.1)
    logits, targets = head_case(g, B * T, V)
    t_inp, t_wte, t_wpe, t_dout, t_w, t_b = dev(inp), dev(wte), dev(wpe), dev(dout), dev(w), dev(b)
    t_log, t_tgt = dev(logits), dev(targets)
    out = torch.empty(B * T * C, device=DEV)
    enc, ln = torch.empty(B * T * C, device=DEV), torch.empty(B * T * C, device=DEV)
    mean, rstd = torch.empty(B * T, device=DEV), torch.empty(B * T, device=DEV)
    dwte, dwpe = torch.zeros(V * C, device=DEV), torch.zeros(T * C, device=DEV)
    probs, losses = torch.empty(B * T * V, device=DEV), torch.empty(B * T, device=DEV)
    dlog, dlog0 = torch.zeros(B * T * V, device=DEV), torch.full((B * T * V,), 7.0, device=DEV)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        gpu.encoder_forward(out, t_inp, t_wte, t_wpe, B, T, C)
        gpu.encoder_backward(dwte, dwpe, t_dout, t_inp, B, T, C)
        gpu.encoder_layernorm_forward(enc, ln, mean, rstd, t_inp, t_wte, t_wpe, t_w, t_b, B, T, C)
        gpu.softmax_crossentropy(losses, probs, t_log, t_tgt, B, T, V)
        gpu.crossentropy_softmax_backward(dlog, probs, t_tgt, B, T, V)
        gpu.crossentropy_softmax_backward_zeroed(dlog0, probs, t_tgt, B, T, V)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    gpu.synchronize()  # no id was out of range: nothing to report
    want = np.zeros(B * T * C, np.float32)
    oracle.encoder_forward(want, inp, wte, wpe, B, T, C)
    assert_bits(host(out), want, "encoder_forward")
    assert_bits(host(enc), want, "encoder_layernorm_forward enc")
    cw, cp = np.zeros(V * C, np.float32), np.zeros(T * C, np.float32)
    oracle.encoder_backward(cw, cp, dout, inp, B, T, C)
    assert_bits(host(dwte), cw, "encoder_backward dwte")
    assert_bits(host(dwpe), cp, "encoder_backward dwpe")
    cd = np.zeros(B * T * V, np.float32)
    oracle.crossentropy_softmax_backward(cd, host(probs), targets, B, T, V)
    assert_bits(host(dlog), cd, "crossentropy_softmax_backward")
    assert_bits(host(dlog0), cd, "crossentropy_softmax_backward_zeroed")
    assert np.array_equal(host(t_inp), inp) and np.array_equal(host(t_tgt), targets)  # ids in range: untouched


def test_ids_out_of_range_reported_at_synchronize(gpu, oracle):
    B, T, C, V = 2, 16, 64, 50
    g = gen.rng(778)
    inp = gen.tokens_uniform(g, B * T, V)
    bad_rows = [3, 17, 30]
    inp[bad_rows] = [V, -3, 1 << 30]
    wte, wpe, dout = gen.normal(g, (V * C,), 0, 0.02), gen.normal(g, (T * C,), 0, 0.01), gen.normal(g, (B * T * C,))
    good = np.setdiff1d(np.arange(B * T), bad_rows)
    # forward: the bad ids are replaced by 0 (in place), every row stays inside wte
    t_inp = dev(inp)
    out = torch.empty(B * T * C, device=DEV)
    gpu.encoder_forward(out, t_inp, dev(wte), dev(wpe), B, T, C)  # no exception at the call
    with pytest.raises(gpu.UgkError) as err:
        gpu.synchronize()
    assert err.value.status == 1 and "encoder_forward" in str(err.value)
    gpu.synchronize()  # reported once, then cleared
    fixed = inp.copy()
    fixed[bad_rows] = 0
    assert np.array_equal(host(t_inp), fixed)
    want = np.zeros(B * T * C, np.float32)
    oracle.encoder_forward(want, fixed, wte, wpe, B, T, C)
    assert_bits(host(out).reshape(B * T, C)[good], want.reshape(B * T, C)[good], "encoder_forward, valid rows")
    # backward: the bad ids become -1, whose rows are skipped (dwpe still takes every row)
    t_inp = dev(inp)
    dwte, dwpe = torch.zeros(V * C, device=DEV), torch.zeros(T * C, device=DEV)
    gpu.encoder_backward(dwte, dwpe, dev(dout), t_inp, B, T, C)
    with pytest.raises(gpu.UgkError) as err:
        gpu.synchronize()
    assert "encoder_backward" in str(err.value)
    keep = inp.copy()
    keep[bad_rows] = -1
    assert np.array_equal(host(t_inp), keep)
    cw, cp = np.zeros(V * C, np.float32), np.zeros(T * C, np.float32)
    oracle.encoder_backward(cw, cp, dout, np.where(keep < 0, 0, keep).astype(np.int32), B, T, C)
    cw2 = np.zeros(V * C, np.float32)  # the oracle without the skipped rows
    d2 = dout.reshape(B * T, C).copy()
    d2[bad_rows] = 0.0
    oracle.encoder_backward(cw2, np.zeros(T * C, np.float32), d2.ravel(), np.where(keep < 0, 0, keep).astype(np.int32),
                            B, T, C)
    assert_bits(host(dwpe), cp, "dwpe over every row")
    got = host(dwte).reshape(V, C)
    touched = np.unique(keep[keep >= 0])
    assert_bits(got[touched], cw2.reshape(V, C)[touched], "dwte of the valid rows")
    # softmax targets
    logits, targets = head_case(g, B * T, V)
    targets[5] = V
    t_tgt = dev(targets)
    probs, losses = torch.empty(B * T * V, device=DEV), torch.empty(B * T, device=DEV)
    gpu.softmax_crossentropy(losses, probs, dev(logits), t_tgt, B, T, V)
    with pytest.raises(gpu.UgkError) as err:
        gpu.synchronize()
    assert "softmax_crossentropy" in str(err.value)
    assert host(t_tgt)[5] == 0
    # the host-side mode: a ValueError at the call, the ids untouched
    gpu.set_sync_checks(True)
    try:
        t_inp = dev(inp)
        with pytest.raises(ValueError):
            gpu.encoder_forward(out, t_inp, dev(wte), dev(wpe), B, T, C)
        assert np.array_equal(host(t_inp), inp)
    finally:
        gpu.set_sync_checks(False)
    gpu.synchronize()
