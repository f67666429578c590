"""ugk - Python binding of libugk.so, the MI355X layer-kernel set of uncertain-gpt.

The functions mirror the CPU ops of the reference oracle ``train_bnn.c``
(names, argument order and ``+=`` semantics for every backward output) and run
the hand-written gfx950 HIP kernels of ``libugk.so`` through its C-ABI
(``include/ugk.h``). Arguments are torch tensors on the GPU (fp32, int32 for
token ids), or raw device addresses (``int``) for callers that manage memory
themselves. Every tensor argument is checked on the host for device, dtype,
contiguity and size before the call, so a kernel never sees a buffer smaller
than the shape it is told; a failing call raises :class:`UgkError` with the
library's message.

There is no CPU fallback: if ``libugk.so`` is missing this module raises on
import, and on a machine without a GPU the calls fail in the HIP runtime.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

__all__ = [
    "UgkError", "lib", "library_path",
    "encoder_forward", "encoder_backward", "layernorm_forward", "layernorm_backward",
    "gelu_forward", "gelu_backward", "residual_forward", "residual_backward",
    "bayes_materialize", "encoder_layernorm_forward", "residual_layernorm_forward", "layernorm_residual_backward",
    "softmax_crossentropy", "crossentropy_softmax_backward", "crossentropy_softmax_backward_zeroed",
    "bayes_sample", "bayes_backward",
    "bayes_backward_philox", "kl_forward", "kl_backward", "adamw_update", "bbb_step_fused",
    "Loader", "loader_count", "ckpt_path", "ckpt_save", "ckpt_load",
    "set_stream", "synchronize", "reserve", "scratch_bytes", "reserve_config", "workspace_bytes",
    "set_workspace", "set_sync_checks", "op_timer_start", "op_timer_read", "set_gelu_exact", "gelu_exact", "set_philox_exact", "philox_exact", "set_kl_exact", "kl_exact", "set_softmax_exact", "softmax_exact", "set_layernorm_exact", "layernorm_exact", "set_encoder_exact", "encoder_exact",
    "Config", "DenseOps", "param_count", "act_count", "gpt2_layers_forward",
    "gpt2_layers_backward", "gpt2_layers_backward_zeroed", "version",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
library_path = os.path.normpath(os.path.join(_HERE, "..", "libugk.so"))

if not os.path.exists(library_path):
    raise ImportError(
        f"libugk.so not found at {library_path}; build it with "
        "`make -C uncertain-gpt_amd/csrc` or `python -c 'import __graft_entry__ as g; g.build()'`")

lib = ctypes.CDLL(library_path)

_fp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_u64 = ctypes.c_ulonglong
_fl = ctypes.c_float


class Config(ctypes.Structure):
    """``Config`` of gpt2_kernels.cuh:634 (ugk_config)."""
    _fields_ = [("B", _i), ("T", _i), ("C", _i), ("V", _i), ("NH", _i), ("maxT", _i), ("L", _i)]


_MATMUL_FWD = ctypes.CFUNCTYPE(_i, _fp, _fp, _fp, _fp, _fp, _i, _i, _i)
_MATMUL_BWD = ctypes.CFUNCTYPE(_i, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _i, _i, _i)
_ATTN_FWD = ctypes.CFUNCTYPE(_i, _fp, _fp, _fp, _i, _i, _i, _i)
_ATTN_BWD = ctypes.CFUNCTYPE(_i, _fp, _fp, _fp, _fp, _i, _i, _i, _i)


class DenseOps(ctypes.Structure):
    """``ugk_dense_ops``: callbacks for the GEMM/attention steps between layer kernels."""
    _fields_ = [("ctx", _fp), ("matmul_forward", _MATMUL_FWD), ("matmul_backward", _MATMUL_BWD),
                ("attention_forward", _ATTN_FWD), ("attention_backward", _ATTN_BWD)]


_SIGS = {
    "ugk_encoder_forward": [_fp, _fp, _fp, _fp, _i, _i, _i],
    "ugk_encoder_backward": [_fp, _fp, _fp, _fp, _i, _i, _i],
    "ugk_layernorm_forward": [_fp, _fp, _fp, _fp, _fp, _fp, _i, _i, _i],
    "ugk_layernorm_backward": [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _i, _i, _i],
    "ugk_layernorm_backward_noalloc": [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _i, _i, _i],
    "ugk_encoder_layernorm_forward": [_fp] * 9 + [_i, _i, _i],
    "ugk_residual_layernorm_forward": [_fp] * 8 + [_i, _i, _i],
    "ugk_layernorm_residual_backward": [_fp] * 10 + [_i, _i, _i],
    "ugk_gelu_forward": [_fp, _fp, _i],
    "ugk_gelu_backward": [_fp, _fp, _fp, _i],
    "ugk_residual_forward": [_fp, _fp, _fp, _i],
    "ugk_residual_backward": [_fp, _fp, _fp, _i],
    "ugk_bayes_materialize": [_fp, _fp, _fp, _fp, _sz],
    "ugk_softmax_crossentropy": [_fp, _fp, _fp, _fp, _i, _i, _i],
    "ugk_crossentropy_softmax_backward": [_fp, _fp, _fp, _i, _i, _i],
    "ugk_crossentropy_softmax_backward_zeroed": [_fp, _fp, _fp, _i, _i, _i],
    "ugk_bayes_sample": [_fp, _fp, _fp, _fp, _sz, _u64, _i],
    "ugk_bayes_backward": [_fp, _fp, _fp, _fp, _fp, _sz],
    "ugk_bayes_backward_philox": [_fp, _fp, _fp, _fp, _sz, _u64, _i],
    "ugk_kl_forward": [ctypes.POINTER(ctypes.c_double), _fp, _fp, _sz, _fl],
    "ugk_kl_backward": [_fp, _fp, _fp, _fp, _sz, _fl, _fl],
    "ugk_adamw_update": [_fp, _fp, _fp, _fp, _sz, _i, _fl, _fl, _fl, _fl, _fl],
    "ugk_bbb_step_fused": [_fp] * 8 + [_sz, _u64, _i] + [_fl] * 9,
    "ugk_set_stream": [_fp],
    "ugk_get_stream": [],
    "ugk_reserve": [_i, _i],
    "ugk_reserve_config": [Config],
    "ugk_workspace_bytes": [Config],
    "ugk_set_workspace": [_fp, _sz, Config],
    "ugk_op_timer_start": [_i],
    "ugk_op_timer_read": [_fp, _fp, _i, ctypes.POINTER(_i)],
    "ugk_scratch_bytes": [],
    "ugk_synchronize": [],
    "ugk_version": [],
    "ugk_set_gelu_exact": [_i],
    "ugk_get_gelu_exact": [],
    "ugk_set_philox_exact": [_i],
    "ugk_set_encoder_exact": [_i],
    "ugk_get_encoder_exact": [],
    "ugk_get_philox_exact": [],
    "ugk_set_kl_exact": [_i],
    "ugk_get_kl_exact": [],
    "ugk_set_softmax_exact": [_i],
    "ugk_get_softmax_exact": [],
    "ugk_set_layernorm_exact": [_i],
    "ugk_get_layernorm_exact": [],
    "ugk_last_error": [],
    "ugk_param_count": [Config],
    "ugk_act_count": [Config],
    "ugk_gpt2_layers_forward": [_fp, _fp, _fp, Config, ctypes.POINTER(DenseOps)],
    "ugk_gpt2_layers_backward": [_fp, _fp, _fp, _fp, _fp, Config, ctypes.POINTER(DenseOps)],
    "ugk_gpt2_layers_backward_zeroed": [_fp, _fp, _fp, _fp, _fp, Config, ctypes.POINTER(DenseOps)],
    "ugk_diag_math_mismatch": [_i, ctypes.c_uint, ctypes.c_ulonglong, ctypes.POINTER(ctypes.c_ulonglong),
                               ctypes.POINTER(ctypes.c_uint)],
    "ugk_diag_math_eval": [_i, _i, _fp, _fp, _sz],
    "ugk_diag_philox": [_fp, _fp, _sz],
    "ugk_diag_math_ulp": [_i, ctypes.c_uint, ctypes.c_ulonglong, ctypes.POINTER(ctypes.c_uint),
                          ctypes.POINTER(ctypes.c_uint)],
    "ugk_diag_stream": [_fp, _sz, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int],
    "ugk_diag_layernorm_partial_rows": [_i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "ugk_ids_guard": [_fp, _i, _i, _i, _i],
    "ugk_diag_layernorm_tail": [_i],
    "ugk_loader_open": [ctypes.POINTER(_fp), ctypes.c_char_p],
    "ugk_loader_count": [ctypes.c_char_p, ctypes.POINTER(ctypes.c_long)],
    "ugk_loader_next": [_fp, _fp, _fp, _i],
    "ugk_loader_next_device": [_fp, _fp, _fp, _i],
    "ugk_loader_tokens": [_fp],
    "ugk_loader_position": [_fp],
    "ugk_loader_close": [_fp],
    "ugk_ckpt_path": [ctypes.c_char_p, _sz, ctypes.c_char_p, ctypes.c_char_p, Config, _i],
    "ugk_ckpt_save": [ctypes.c_char_p, _fp, _sz, Config, _i],
    "ugk_ckpt_load": [ctypes.c_char_p, _fp, _sz, Config, ctypes.POINTER(_i)],
}
_RET = {"ugk_last_error": ctypes.c_char_p, "ugk_get_stream": _fp, "ugk_scratch_bytes": _sz, "ugk_workspace_bytes": _sz,
        "ugk_loader_tokens": ctypes.c_long, "ugk_loader_position": ctypes.c_long,
        "ugk_param_count": _sz, "ugk_act_count": _sz}
for _name, _args in _SIGS.items():
    _f = getattr(lib, _name)
    _f.argtypes = _args
    _f.restype = _RET.get(_name, _i)


class UgkError(RuntimeError):
    """A libugk call returned a nonzero status (1 invalid argument, 2 HIP error, 3 out of memory)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[ugk status {status}] {message}")
        self.status = status


def _check(status: int) -> None:
    if status != 0:
        raise UgkError(status, lib.ugk_last_error().decode(errors="replace"))


def _ptr(x, what: str, need: int, dtype: str):
    """Device address of ``x`` after checking it can hold ``need`` elements of ``dtype``."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    import torch  # plumbing only: device memory
    want = {"f32": torch.float32, "i32": torch.int32}[dtype]
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{what}: expected a torch tensor or a device address, got {type(x)!r}")
    if x.device.type != "cuda":
        raise ValueError(f"{what}: tensor must be on the GPU, got {x.device}")
    if x.dtype != want:
        raise TypeError(f"{what}: dtype must be {want}, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    if x.numel() < need:
        raise ValueError(f"{what}: needs at least {need} elements, has {x.numel()}")
    return x.data_ptr()


# Token and target ids index tables (rows of wte, logits of a row): an id out of range would make a
# kernel read or write outside them. The reference leaves 0 <= id < V to its callers unchecked.
# Here each tensor of ids goes through ugk_ids_guard on the device first, on the library's stream:
# ids out of range are replaced in place (so no kernel indexes outside its table; ids in range are
# not written), and the library records the op, which the next synchronize() raises as UgkError.
# No host round trip, so the calls stay asynchronous and may be captured in a graph.
# set_sync_checks(True) checks on the host instead (reading the ids back, a device synchronisation
# per call) and raises ValueError at once, leaving the ids untouched.
_IDS_CODE = {"encoder_forward": 1, "encoder_backward": 2, "encoder_layernorm_forward": 3, "softmax_crossentropy": 4,
             "crossentropy_softmax_backward": 5, "crossentropy_softmax_backward_zeroed": 5}
_sync_checks = False


def set_sync_checks(on: bool) -> None:
    """Check token/target ids on the host before each call (a device sync per call; ValueError at
    once) instead of the default asynchronous device-side guard (UgkError at the next synchronize)."""
    global _sync_checks
    _sync_checks = bool(on)


def _guard_ids(ids, n: int, bound: int, fill: int, what: str) -> None:
    """Guard a device tensor of ids (see above); a device address, or a tensor that the argument
    checks reject, is left alone."""
    import torch
    if not (isinstance(ids, torch.Tensor) and ids.is_cuda and ids.dtype == torch.int32 and ids.is_contiguous()):
        return
    if n <= 0 or ids.numel() < n:
        return  # nothing to index, or the size check of the call rejects it
    if _sync_checks and not torch.cuda.is_current_stream_capturing():
        t = ids.reshape(-1)[:n]
        lo, hi = int(t.min()), int(t.max())
        if lo < 0 or hi >= bound:
            raise ValueError(f"{what}: ids must lie in [0, {bound}), got [{lo}, {hi}]")
        return
    _check(lib.ugk_ids_guard(ids.data_ptr(), n, bound, fill, _IDS_CODE[what]))


def _check_tokens(inp, table, C: int, n: int, what: str, fill: int = 0) -> None:
    """Token ids index rows of ``table`` (``table.numel() // C`` rows)."""
    import torch
    if isinstance(table, torch.Tensor) and table.is_cuda and C:
        _guard_ids(inp, n, table.numel() // C, fill, what)


def _check_targets(targets, V: int, rows: int, what: str) -> None:
    """Target ids index a row of V logits."""
    _guard_ids(targets, rows, V, 0, what)


def encoder_forward(out, inp, wte, wpe, B: int, T: int, C: int) -> None:
    """train_bnn.c:41-65. ``out[b,t,:] = wte[inp[b,t],:] + wpe[t,:]``."""
    _check_tokens(inp, wte, C, B * T, "encoder_forward")
    _check(lib.ugk_encoder_forward(_ptr(out, "out", B * T * C, "f32"), _ptr(inp, "inp", B * T, "i32"),
                                   _ptr(wte, "wte", C, "f32"), _ptr(wpe, "wpe", T * C, "f32"), B, T, C))


def encoder_backward(dwte, dwpe, dout, inp, B: int, T: int, C: int) -> None:
    """train_bnn.c:647-662. ``dwte[inp[b,t],:] += dout[b,t,:]``; ``dwpe[t,:] += dout[b,t,:]``."""
    _check_tokens(inp, dwte, C, B * T, "encoder_backward", fill=-1)  # a negative id: the row is skipped
    _check(lib.ugk_encoder_backward(_ptr(dwte, "dwte", C, "f32"), _ptr(dwpe, "dwpe", T * C, "f32"),
                                    _ptr(dout, "dout", B * T * C, "f32"), _ptr(inp, "inp", B * T, "i32"),
                                    B, T, C))


def layernorm_forward(out, mean, rstd, inp, weight, bias, B: int, T: int, C: int) -> None:
    """train_bnn.c:81-115."""
    n, r = B * T * C, B * T
    _check(lib.ugk_layernorm_forward(_ptr(out, "out", n, "f32"), _ptr(mean, "mean", r, "f32"),
                                     _ptr(rstd, "rstd", r, "f32"), _ptr(inp, "inp", n, "f32"),
                                     _ptr(weight, "weight", C, "f32"), _ptr(bias, "bias", C, "f32"),
                                     B, T, C))


def layernorm_backward(dinp, dweight, dbias, dout, inp, weight, mean, rstd, B: int, T: int, C: int) -> None:
    """train_bnn.c:439-477 (all three gradients accumulate)."""
    n, r = B * T * C, B * T
    _check(lib.ugk_layernorm_backward(_ptr(dinp, "dinp", n, "f32"), _ptr(dweight, "dweight", C, "f32"),
                                      _ptr(dbias, "dbias", C, "f32"), _ptr(dout, "dout", n, "f32"),
                                      _ptr(inp, "inp", n, "f32"), _ptr(weight, "weight", C, "f32"),
                                      _ptr(mean, "mean", r, "f32"), _ptr(rstd, "rstd", r, "f32"), B, T, C))


def encoder_layernorm_forward(enc, out, mean, rstd, inp, wte, wpe, weight, bias, B: int, T: int, C: int) -> None:
    """``encoder_forward(enc, inp, wte, wpe)`` then ``layernorm_forward(out, mean, rstd, enc, ...)``, one pass."""
    n, rows = B * T * C, B * T
    _check_tokens(inp, wte, C, rows, "encoder_layernorm_forward")
    _check(lib.ugk_encoder_layernorm_forward(
        _ptr(enc, "enc", n, "f32"), _ptr(out, "out", n, "f32"), _ptr(mean, "mean", rows, "f32"),
        _ptr(rstd, "rstd", rows, "f32"), _ptr(inp, "inp", rows, "i32"), _ptr(wte, "wte", C, "f32"),
        _ptr(wpe, "wpe", T * C, "f32"), _ptr(weight, "weight", C, "f32"), _ptr(bias, "bias", C, "f32"), B, T, C))


def residual_layernorm_forward(res, out, mean, rstd, x, y, weight, bias, B: int, T: int, C: int) -> None:
    """``res = x + y`` (residual_forward) then ``layernorm_forward(out, mean, rstd, res, ...)``, one pass."""
    n, rows = B * T * C, B * T
    _check(lib.ugk_residual_layernorm_forward(
        _ptr(res, "res", n, "f32"), _ptr(out, "out", n, "f32"), _ptr(mean, "mean", rows, "f32"),
        _ptr(rstd, "rstd", rows, "f32"), _ptr(x, "x", n, "f32"), _ptr(y, "y", n, "f32"),
        _ptr(weight, "weight", C, "f32"), _ptr(bias, "bias", C, "f32"), B, T, C))


def layernorm_residual_backward(dinp, dweight, dbias, dx, dy, dout, inp, weight, mean, rstd, B: int, T: int,
                                C: int) -> None:
    """``layernorm_backward`` then ``residual_backward(dx, dy, dinp)``, one pass."""
    n, rows = B * T * C, B * T
    _check(lib.ugk_layernorm_residual_backward(
        _ptr(dinp, "dinp", n, "f32"), _ptr(dweight, "dweight", C, "f32"), _ptr(dbias, "dbias", C, "f32"),
        _ptr(dx, "dx", n, "f32"), _ptr(dy, "dy", n, "f32"), _ptr(dout, "dout", n, "f32"),
        _ptr(inp, "inp", n, "f32"), _ptr(weight, "weight", C, "f32"), _ptr(mean, "mean", rows, "f32"),
        _ptr(rstd, "rstd", rows, "f32"), B, T, C))


def gelu_forward(out, inp, N: int) -> None:
    """train_bnn.c:163-170 (tanh approximation)."""
    _check(lib.ugk_gelu_forward(_ptr(out, "out", N, "f32"), _ptr(inp, "inp", N, "f32"), N))


def gelu_backward(dinp, inp, dout, N: int) -> None:
    """train_bnn.c:520-533. ``dinp += gelu'(inp) * dout``."""
    _check(lib.ugk_gelu_backward(_ptr(dinp, "dinp", N, "f32"), _ptr(inp, "inp", N, "f32"),
                                 _ptr(dout, "dout", N, "f32"), N))


def residual_forward(out, x, y, N: int) -> None:
    """train_bnn.c:182-186."""
    _check(lib.ugk_residual_forward(_ptr(out, "out", N, "f32"), _ptr(x, "x", N, "f32"),
                                    _ptr(y, "y", N, "f32"), N))


def residual_backward(dx, dy, dout, N: int) -> None:
    """train_bnn.c:491-496. ``dx += dout``; ``dy += dout``."""
    _check(lib.ugk_residual_backward(_ptr(dx, "dx", N, "f32"), _ptr(dy, "dy", N, "f32"),
                                     _ptr(dout, "dout", N, "f32"), N))


def bayes_materialize(w, mu, rho, eps, n: int) -> None:
    """train_bnn.c:831-835. ``w = mu + softplus(rho) * eps``."""
    _check(lib.ugk_bayes_materialize(_ptr(w, "w", n, "f32"), _ptr(mu, "mu", n, "f32"),
                                     _ptr(rho, "rho", n, "f32"), _ptr(eps, "eps", n, "f32"), n))


def softmax_crossentropy(losses, probs, logits, targets, B: int, T: int, V: int) -> None:
    """train_bnn.c:279-304. ``probs`` = row softmax of ``logits``; ``losses`` = -log probs[target]."""
    rows, n = B * T, B * T * V
    _check_targets(targets, V, rows, "softmax_crossentropy")
    _check(lib.ugk_softmax_crossentropy(_ptr(losses, "losses", rows, "f32"), _ptr(probs, "probs", n, "f32"),
                                        _ptr(logits, "logits", n, "f32"), _ptr(targets, "targets", rows, "i32"),
                                        B, T, V))


def crossentropy_softmax_backward(dlogits, probs, targets, B: int, T: int, V: int) -> None:
    """train_bnn.c:358-378. ``dlogits += (probs - onehot(target)) / (B*T)``."""
    rows, n = B * T, B * T * V
    _check_targets(targets, V, rows, "crossentropy_softmax_backward")
    _check(lib.ugk_crossentropy_softmax_backward(_ptr(dlogits, "dlogits", n, "f32"), _ptr(probs, "probs", n, "f32"),
                                                 _ptr(targets, "targets", rows, "i32"), B, T, V))


def crossentropy_softmax_backward_zeroed(dlogits, probs, targets, B: int, T: int, V: int) -> None:
    """crossentropy_softmax_backward for a dlogits that is zero before the call (the arms' memset of
    the activation gradients): it is written, not read."""
    rows, n = B * T, B * T * V
    _check_targets(targets, V, rows, "crossentropy_softmax_backward_zeroed")
    _check(lib.ugk_crossentropy_softmax_backward_zeroed(_ptr(dlogits, "dlogits", n, "f32"),
                                                        _ptr(probs, "probs", n, "f32"),
                                                        _ptr(targets, "targets", rows, "i32"), B, T, V))


def bayes_sample(w, eps, mu, rho, n: int, seed: int, step: int) -> None:
    """train_bnn.c:841-845 with the Philox draw of train_bnn_gpu.cu:93-97.

    ``w = mu + softplus(rho) * eps_i`` with ``eps_i = philox_normal(seed, step, i)``; ``eps`` may be
    None, otherwise the draws are stored there too.
    """
    _check(lib.ugk_bayes_sample(_ptr(w, "w", n, "f32"), _ptr(eps, "eps", n, "f32"), _ptr(mu, "mu", n, "f32"),
                                _ptr(rho, "rho", n, "f32"), n, seed, step))


def bayes_backward(dmu, drho, dw, eps, rho, n: int) -> None:
    """train_bnn.c:855-861. ``dmu += dw; drho += dw * eps * sigmoid(rho)``."""
    _check(lib.ugk_bayes_backward(_ptr(dmu, "dmu", n, "f32"), _ptr(drho, "drho", n, "f32"),
                                  _ptr(dw, "dw", n, "f32"), _ptr(eps, "eps", n, "f32"),
                                  _ptr(rho, "rho", n, "f32"), n))


def bayes_backward_philox(dmu, drho, dw, rho, n: int, seed: int, step: int) -> None:
    """train_bnn_gpu.cu:99-109 (k_bayes_backward): ``bayes_backward`` with eps regenerated."""
    _check(lib.ugk_bayes_backward_philox(_ptr(dmu, "dmu", n, "f32"), _ptr(drho, "drho", n, "f32"),
                                         _ptr(dw, "dw", n, "f32"), _ptr(rho, "rho", n, "f32"), n, seed, step))


def kl_forward(mu, rho, n: int, sigma_prior: float) -> float:
    """train_bnn.c:941-957. The KL of q(mu, softplus(rho)) against N(0, sigma_prior^2), in double."""
    out = ctypes.c_double(0.0)
    _check(lib.ugk_kl_forward(ctypes.byref(out), _ptr(mu, "mu", n, "f32"), _ptr(rho, "rho", n, "f32"), n,
                              sigma_prior))
    return float(out.value)


def kl_backward(dmu, drho, mu, rho, n: int, sigma_prior: float, weight: float) -> None:
    """train_bnn.c:966-979. Accumulates the weighted KL gradient onto dmu, drho."""
    _check(lib.ugk_kl_backward(_ptr(dmu, "dmu", n, "f32"), _ptr(drho, "drho", n, "f32"),
                               _ptr(mu, "mu", n, "f32"), _ptr(rho, "rho", n, "f32"), n, sigma_prior, weight))


def adamw_update(params, grads, m, v, n: int, t: int, lr: float, beta1: float, beta2: float, eps: float,
                 wd: float) -> None:
    """train_bnn.c:699-717. AdamW step ``t`` (>= 1) on params, m, v in place."""
    _check(lib.ugk_adamw_update(_ptr(params, "params", n, "f32"), _ptr(grads, "grads", n, "f32"),
                                _ptr(m, "m", n, "f32"), _ptr(v, "v", n, "f32"), n, t, lr, beta1, beta2, eps, wd))


def bbb_step_fused(mu, rho, m_mu, v_mu, m_rho, v_rho, w, dw, n: int, seed: int, step: int, sp: float,
                   klw: float, bc1: float, bc2: float, lr: float, beta1: float, beta2: float, aeps: float,
                   wd: float) -> None:
    """train_bnn_gpu.cu:173-217 (k_bbb_step_fused): one Bayes-by-Backprop update in one pass."""
    names = ("mu", "rho", "m_mu", "v_mu", "m_rho", "v_rho", "w", "dw")
    bufs = (mu, rho, m_mu, v_mu, m_rho, v_rho, w, dw)
    _check(lib.ugk_bbb_step_fused(*(_ptr(b, nm, n, "f32") for b, nm in zip(bufs, names)), n, seed, step, sp,
                                  klw, bc1, bc2, lr, beta1, beta2, aeps, wd))


def set_stream(stream: Optional[int]) -> None:
    """Queue later calls on ``stream`` (a hipStream_t address, e.g. ``torch.cuda.Stream().cuda_stream``)."""
    _check(lib.ugk_set_stream(stream or None))


def synchronize() -> None:
    """Wait for the library's stream; raises UgkError if the device-side id guard found an id out of
    range in a call since the last synchronize (the op is named)."""
    _check(lib.ugk_synchronize())


def reserve(rows: int, C: int) -> None:
    _check(lib.ugk_reserve(rows, C))


def scratch_bytes() -> int:
    return int(lib.ugk_scratch_bytes())


def reserve_config(cfg: Config) -> None:
    """Allocate the workspace every entry point needs at shapes up to ``cfg`` now."""
    _check(lib.ugk_reserve_config(cfg))


def workspace_bytes(cfg: Config) -> int:
    """Bytes of device workspace the entry points need at shapes up to ``cfg``."""
    return int(lib.ugk_workspace_bytes(cfg))


_workspace_refs = {}  # device index -> the caller's workspace tensor, kept alive while the library uses it


def set_workspace(buf, cfg: Config) -> None:
    """Hand the library a caller-owned workspace (a uint8/float device tensor of at least
    ``workspace_bytes(cfg)`` bytes, 256-byte aligned), or return to library-owned regions with None.
    The binding keeps a reference to the tensor until the next call of this function on its device,
    so that the caching allocator cannot hand its memory to other tensors meanwhile."""
    import torch
    if buf is None:
        _check(lib.ugk_set_workspace(None, 0, cfg))
        _workspace_refs.pop(torch.cuda.current_device(), None)
        return
    nbytes = buf.numel() * buf.element_size()
    if not buf.is_cuda or not buf.is_contiguous():
        raise ValueError("the workspace must be a contiguous device tensor")
    _check(lib.ugk_set_workspace(buf.data_ptr(), nbytes, cfg))
    _workspace_refs[buf.device.index] = buf


OP_NAMES = {1: "encoder_forward", 2: "layernorm_forward", 3: "residual_layernorm_forward", 4: "gelu_forward",
            5: "layernorm_backward (main)", 6: "layernorm_residual_backward (main)", 7: "gelu_backward",
            8: "layernorm column sums (batched)", 9: "encoder_backward", 10: "encoder_layernorm_forward"}


def op_timer_start(capacity: int = 1024) -> None:
    """Record a HIP event pair around each op the step driver issues (at most ``capacity``)."""
    _check(lib.ugk_op_timer_start(capacity))


def op_timer_read(capacity: int = 1024):
    """Stop the op timer; [(op name, milliseconds)] in issue order."""
    ms = (ctypes.c_float * capacity)()
    ops = (ctypes.c_int * capacity)()
    n = ctypes.c_int(0)
    _check(lib.ugk_op_timer_read(ms, ops, capacity, ctypes.byref(n)))
    return [(OP_NAMES.get(ops[i], str(ops[i])), float(ms[i])) for i in range(n.value)]


def version() -> int:
    return int(lib.ugk_version())


def set_gelu_exact(exact: bool) -> None:
    """GELU form: False (default) the logistic form, within 1e-5 rel / 1e-6 abs of train_bnn.c on every
    input; True the glibc-exact tanhf, bit-identical to it."""
    _check(lib.ugk_set_gelu_exact(1 if exact else 0))


def gelu_exact() -> bool:
    return bool(lib.ugk_get_gelu_exact())


def set_philox_exact(exact: bool) -> None:
    """Softplus/sigmoid and the eps draw's logf/cosf inside the ops that draw eps on the device:
    False (default) the hardware-transcendental forms, within 1e-5 rel / 1e-6 abs of train_bnn.c on
    every input (eps within a few ulp); True the glibc-exact forms, with which eps and every output
    of each Philox op equal the host's bit for bit."""
    _check(lib.ugk_set_philox_exact(1 if exact else 0))


def philox_exact() -> bool:
    return bool(lib.ugk_get_philox_exact())


def set_kl_exact(exact: bool) -> None:
    """Softplus inside kl_forward: False (default) the hardware-transcendental form where sigma is a
    normal float (each term within 8 * 2^-23 * (1 + sigma^2/sp^2) of train_bnn.c's); True the
    glibc-exact form throughout (the total within double rounding of train_bnn.c's)."""
    _check(lib.ugk_set_kl_exact(1 if exact else 0))


def kl_exact() -> bool:
    return bool(lib.ugk_get_kl_exact())


def set_softmax_exact(exact: bool) -> None:
    """Row sum inside softmax_crossentropy: False (default) a fixed tree (probabilities within float
    rounding of train_bnn.c's); True train_bnn.c's serial order, every probability and loss
    bit-identical to it."""
    _check(lib.ugk_set_softmax_exact(1 if exact else 0))


def softmax_exact() -> bool:
    return bool(lib.ugk_get_softmax_exact())


def set_layernorm_exact(exact: bool) -> None:
    """LayerNorm order of additions: False (default) tree row sums and per-workgroup partial column
    sums (within fp32 rounding and the scale-aware bar of train_bnn.c); True train_bnn.c's own serial
    order, every LayerNorm output bit-identical to it (fused pairs, the allocation-free backward and
    the step driver included)."""
    _check(lib.ugk_set_layernorm_exact(1 if exact else 0))


def layernorm_exact() -> bool:
    return bool(lib.ugk_get_layernorm_exact())


def set_encoder_exact(exact: bool) -> None:
    """Encoder backward, tokens with more than 32 rows in a chunk: False (default) blocked adds (64-row
    blocks in row order, block sums in block order; deterministic); True one add per row in row order,
    bit-identical to train_bnn.c."""
    _check(lib.ugk_set_encoder_exact(1 if exact else 0))


def encoder_exact() -> bool:
    return bool(lib.ugk_get_encoder_exact())


def param_count(cfg: Config) -> int:
    return int(lib.ugk_param_count(cfg))


def act_count(cfg: Config) -> int:
    return int(lib.ugk_act_count(cfg))


def _cfg_check(cfg: Config) -> None:
    if cfg.B < 0 or cfg.T < 0 or cfg.C <= 0 or cfg.V <= 0 or cfg.L < 0 or cfg.maxT < cfg.T:
        raise ValueError(f"bad config {[(f, getattr(cfg, f)) for f, _ in Config._fields_]}")


def gpt2_layers_forward(acts, params, inputs, cfg: Config, ops: Optional[DenseOps] = None) -> None:
    """Layer-kernel half of gpt2_forward (gpt2_kernels.cuh:756-813) on the reference's buffer layout."""
    _cfg_check(cfg)
    _check(lib.ugk_gpt2_layers_forward(_ptr(acts, "acts", act_count(cfg), "f32"),
                                       _ptr(params, "params", param_count(cfg), "f32"),
                                       _ptr(inputs, "inputs", cfg.B * cfg.T, "i32"), cfg,
                                       ctypes.byref(ops) if ops is not None else None))


def _layers_backward(fn, grads, grads_acts, acts, params, inputs, cfg, ops):
    _cfg_check(cfg)
    na, npar = act_count(cfg), param_count(cfg)
    _check(fn(_ptr(grads, "grads", npar, "f32"), _ptr(grads_acts, "grads_acts", na, "f32"),
              _ptr(acts, "acts", na, "f32"), _ptr(params, "params", npar, "f32"),
              _ptr(inputs, "inputs", cfg.B * cfg.T, "i32"), cfg, ctypes.byref(ops) if ops is not None else None))


def gpt2_layers_backward(grads, grads_acts, acts, params, inputs, cfg: Config,
                         ops: Optional[DenseOps] = None) -> None:
    """Layer-kernel half of gpt2_backward (gpt2_kernels.cuh:846-894)."""
    _layers_backward(lib.ugk_gpt2_layers_backward, grads, grads_acts, acts, params, inputs, cfg, ops)


def gpt2_layers_backward_zeroed(grads, grads_acts, acts, params, inputs, cfg: Config,
                                ops: Optional[DenseOps] = None) -> None:
    """gpt2_layers_backward for a grads_acts that is zero outside the incoming gradient (flo), as
    every reference arm leaves it before gpt2_backward (train_bnn_gpu.cu:475): the zeros are
    not read."""
    _layers_backward(lib.ugk_gpt2_layers_backward_zeroed, grads, grads_acts, acts, params, inputs, cfg, ops)


MATH_FUNCTIONS = {"expf": 0, "log1pf": 1, "expm1f": 2, "tanhf": 3, "softplus": 4, "logf": 5, "cosf": 6,
                  "sqrtf": 7, "gelu": 8, "gelu_grad": 9}
# the same functions with division sequence s (0 IEEE, 1-3 reciprocal + corrections)
MATH_FUNCTIONS.update({f"{name}/div{s}": base + s for name, base in (("tanhf", 10), ("log1pf", 20), ("expm1f", 30))
                       for s in range(4)})
# x / b for the eight divisors of the softmax quotient check
MATH_FUNCTIONS.update({f"div_recip{j}": 40 + j for j in range(8)})
# sqrtf for inputs >= 2^-96 (the Box-Muller transform's); 1 / x for x >= 1 (the sigmoid's)
MATH_FUNCTIONS.update({"sqrtf_large": 48})
MATH_FUNCTIONS.update({f"recip/div{s}": 49 + s for s in range(4)})
MATH_FUNCTIONS.update({"recip_ge1": 53})
# x / b for the launch-wide divisors of the posterior ops; sqrtf for any input
MATH_FUNCTIONS.update({f"div_shared{j}": 54 + j for j in range(8)})
MATH_FUNCTIONS.update({"sqrtf_any": 62})
# expf without branches for x <= 88.72 and NaN (the softmax's and softplus's)
MATH_FUNCTIONS.update({"expf_nooverflow": 63})
# the default (logistic-form) GELU and derivative; their "mismatches" are results outside the literal bar
MATH_FUNCTIONS.update({"gelu_fast": 64, "gelu_grad_fast": 65})
# the hardware-transcendental softplus and sigmoid of the Philox ops (the literal bar, likewise)
MATH_FUNCTIONS.update({"softplus_fast": 66, "sigmoid_fast": 67})
# the default form's Box-Muller cosf on its domain, against the device library's
MATH_FUNCTIONS.update({"cosf_small": 69})
# the Box-Muller radius sqrt(-2 ln u1) on [2^-33, 1]: the default form's and the glibc-exact form's
MATH_FUNCTIONS.update({"bm_radius_fast": 70, "bm_radius": 71})


def diag_math_mismatch(fn: str, lo: int = 0, count: int = 1 << 32):
    """(mismatches, first) of the kernels' float math against its IEEE restatement over bit patterns."""
    n, first = ctypes.c_ulonglong(0), ctypes.c_uint(0)
    _check(lib.ugk_diag_math_mismatch(MATH_FUNCTIONS[fn], lo, min(count, (1 << 32) - lo), ctypes.byref(n),
                                      ctypes.byref(first)))
    return int(n.value), int(first.value)


def diag_math_ulp(fn: str, lo: int = 0, count: int = 1 << 32):
    """(largest ulp distance, input pattern where it occurs) of a fast form against its reference."""
    d, at = ctypes.c_uint(0), ctypes.c_uint(0)
    _check(lib.ugk_diag_math_ulp(MATH_FUNCTIONS[fn], lo, min(count, (1 << 32) - lo), ctypes.byref(d),
                                 ctypes.byref(at)))
    return int(d.value), int(at.value)


def diag_math_eval(fn: str, out, inp, variant: int = 0) -> None:
    """``out = f(inp)`` on the device (variant 0 the kernels' math, 1 the restatement)."""
    n = inp.numel()
    _check(lib.ugk_diag_math_eval(MATH_FUNCTIONS[fn], variant, _ptr(out, "out", n, "f32"),
                                  _ptr(inp, "inp", n, "f32"), n))


def diag_philox(out, tuples) -> None:
    """Philox4x32-10 on the device: ``tuples`` is an int32 tensor of n x 6 words (counter, key),
    ``out`` an int32 tensor of n x 4 output words (bit patterns; read them as uint32)."""
    n = tuples.numel() // 6
    _check(lib.ugk_diag_philox(_ptr(out, "out", 4 * n, "i32"), _ptr(tuples, "tuples", 6 * n, "i32"), n))


def diag_stream(buf, n: int, nr: int, nw: int, per_thread: int = 2, block: int = 256) -> None:
    """A pure stream with nr input and nw output tensors of n floats each, laid out one after
    another in ``buf`` (a float32 tensor of at least (nr + nw) * n elements): out_w = sum of the
    inputs + w, ``per_thread`` float4 per thread in ``block``-thread workgroups. Times the HBM
    ceiling of a kernel's load/store mix."""
    _check(lib.ugk_diag_stream(_ptr(buf, "buf", (nr + nw) * n, "f32"), n, nr, nw, per_thread, block))


# ---- file formats ---------------------------------------------------------------

class Loader:
    """gpt2_kernels.cuh:898-930 (Loader): llm.c .bin token files. ``next`` fills host int32 arrays
    (numpy), ``next_device`` device int32 tensors from a copy of the tokens kept in device memory."""

    def __init__(self, path: str):
        h = _fp()
        _check(lib.ugk_loader_open(ctypes.byref(h), path.encode()))
        self._h = h

    @property
    def tokens(self) -> int:
        return int(lib.ugk_loader_tokens(self._h))

    @property
    def position(self) -> int:
        return int(lib.ugk_loader_position(self._h))

    def next(self, inp, tgt, BT: int) -> None:
        import numpy as np
        for a, nm in ((inp, "inp"), (tgt, "tgt")):
            if not (isinstance(a, np.ndarray) and a.dtype == np.int32 and a.flags.c_contiguous and a.size >= BT):
                raise ValueError(f"{nm}: expected a contiguous int32 numpy array of at least {BT} elements")
        _check(lib.ugk_loader_next(self._h, inp.ctypes.data, tgt.ctypes.data, BT))

    def next_device(self, inp, tgt, BT: int) -> None:
        _check(lib.ugk_loader_next_device(self._h, _ptr(inp, "inp", BT, "i32"), _ptr(tgt, "tgt", BT, "i32"), BT))

    def close(self) -> None:
        if self._h:
            h, self._h = self._h, None
            _check(lib.ugk_loader_close(h))

    def __del__(self):
        if getattr(self, "_h", None):
            lib.ugk_loader_close(self._h)


def loader_count(path: str) -> int:
    """gpt2_kernels.cuh:1318-1331: the token count from the header alone."""
    n = ctypes.c_long(0)
    _check(lib.ugk_loader_count(path.encode(), ctypes.byref(n)))
    return int(n.value)


def ckpt_path(arm: str, what: str, cfg: Config, steps: int) -> str:
    buf = ctypes.create_string_buffer(512)
    _check(lib.ugk_ckpt_path(buf, 512, arm.encode(), what.encode(), cfg, steps))
    return buf.value.decode()


def ckpt_save(path: str, buf, n: int, cfg: Config, steps: int) -> None:
    """gpt2_kernels.cuh:944-964: n floats of a device buffer behind the 8-int header."""
    _check(lib.ugk_ckpt_save(path.encode(), _ptr(buf, "buf", n, "f32"), n, cfg, steps))


def ckpt_load(path: str, buf, n: int, cfg: Config) -> int:
    """gpt2_kernels.cuh:1281-1316: fill a device buffer, checking the header; returns the step count."""
    steps = ctypes.c_int(0)
    _check(lib.ugk_ckpt_load(path.encode(), _ptr(buf, "buf", n, "f32"), n, cfg, ctypes.byref(steps)))
    return int(steps.value)
