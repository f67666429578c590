"""CPU oracle (numpy front end of liboracle.so). TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker and the timed CPU baseline; never by the product path (libugk.so and
the ugk package do not import it).

``Oracle()`` wraps this repo's restatement of the train_bnn.c ops
(oracle/cpu_ref.c). ``Oracle(reference=True)`` wraps the reference's own
train_bnn.c built by ``make -C oracle ref`` into oracle/_ref/libtrain_bnn.so
(present only where that build was made). Both expose the same methods, which
take numpy arrays, work in place with the C functions' semantics (backward
outputs accumulate), and return nothing.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtrain_bnn.so")

_f = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

_SIGS = {
    "encoder_forward": [_f, _f, _f, _f, _i, _i, _i],
    "encoder_backward": [_f, _f, _f, _f, _i, _i, _i],
    "layernorm_forward": [_f, _f, _f, _f, _f, _f, _i, _i, _i],
    "layernorm_backward": [_f, _f, _f, _f, _f, _f, _f, _f, _i, _i, _i],
    "gelu_forward": [_f, _f, _i],
    "gelu_backward": [_f, _f, _f, _i],
    "residual_forward": [_f, _f, _f, _i],
    "residual_backward": [_f, _f, _f, _i],
    "bayes_materialize": [_f, _f, _f, _f, _sz],
    "softmax_crossentropy": [_f, _f, _f, _f, _i, _i, _i],
    "crossentropy_softmax_backward": [_f, _f, _f, _i, _i, _i],
    "bayes_backward": [_f, _f, _f, _f, _f, _sz],
    "kl_backward": [_f, _f, _f, _f, _sz, ctypes.c_float, ctypes.c_float],
    "adamw_update": [_f, _f, _f, _f, _sz, _i, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                     ctypes.c_float, ctypes.c_float],
}
_u64 = ctypes.c_ulonglong
_fl = ctypes.c_float
# Restatement-only entry points (the reference keeps these in CUDA sources).
_SIGS_RESTATED = {
    "oracle_philox4x32_10": ([_f, _f, _f], None),
    "oracle_u01": ([ctypes.c_uint], _fl),
    "oracle_philox_normal": ([_u64, _i, _sz], _fl),
    "oracle_philox_normal_n": ([_f, _sz, _u64, _i, _sz], None),
    "oracle_bayes_sample_philox": ([_f, _f, _f, _f, _sz, _u64, _i], None),
    "oracle_bayes_backward_philox": ([_f, _f, _f, _f, _sz, _u64, _i], None),
    "oracle_bbb_step_fused": ([_f] * 8 + [_sz, _u64, _i] + [_fl] * 9, None),
}


def _p(a: np.ndarray, dtype) -> int:
    if a.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {a.dtype}")
    if not a.flags.c_contiguous:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data


class Oracle:
    def __init__(self, reference: bool = False):
        path = REF_SO if reference else ORACLE_SO
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.path = path
        self.lib = ctypes.CDLL(path)
        prefix = "" if reference else "oracle_"
        self._fn = {}
        for name, args in _SIGS.items():
            fn = getattr(self.lib, prefix + name)
            fn.argtypes = args
            fn.restype = None
            self._fn[name] = fn
        kl = getattr(self.lib, prefix + "kl_forward")
        kl.argtypes = [_f, _f, _sz, _fl]
        kl.restype = ctypes.c_double
        self._fn["kl_forward"] = kl
        if not reference:
            for name, (args, res) in _SIGS_RESTATED.items():
                fn = getattr(self.lib, name)
                fn.argtypes = args
                fn.restype = res
            for name in ("oracle_expf_n", "oracle_log1pf_n", "oracle_tanhf_n", "oracle_softplus_n",
                         "oracle_logf_n", "oracle_cosf_n", "oracle_sqrtf_n"):
                fn = getattr(self.lib, name)
                fn.argtypes = [_f, _f, _sz]
                fn.restype = None
            self.lib.oracle_float_range.argtypes = [_f, ctypes.c_uint, _sz]
            self.lib.oracle_float_range.restype = None
            self.lib.oracle_count_bit_mismatch.argtypes = [_f, _f, _sz, ctypes.POINTER(_sz)]
            self.lib.oracle_count_bit_mismatch.restype = _sz

    # ---- the ops, train_bnn.c argument order ----------------------------------
    def encoder_forward(self, out, inp, wte, wpe, B, T, C):
        self._fn["encoder_forward"](_p(out, np.float32), _p(inp, np.int32), _p(wte, np.float32),
                                    _p(wpe, np.float32), B, T, C)

    def encoder_backward(self, dwte, dwpe, dout, inp, B, T, C):
        self._fn["encoder_backward"](_p(dwte, np.float32), _p(dwpe, np.float32), _p(dout, np.float32),
                                     _p(inp, np.int32), B, T, C)

    def layernorm_forward(self, out, mean, rstd, inp, weight, bias, B, T, C):
        self._fn["layernorm_forward"](*(_p(a, np.float32) for a in (out, mean, rstd, inp, weight, bias)),
                                      B, T, C)

    def layernorm_backward(self, dinp, dweight, dbias, dout, inp, weight, mean, rstd, B, T, C):
        self._fn["layernorm_backward"](*(_p(a, np.float32) for a in
                                         (dinp, dweight, dbias, dout, inp, weight, mean, rstd)), B, T, C)

    def gelu_forward(self, out, inp, N):
        self._fn["gelu_forward"](_p(out, np.float32), _p(inp, np.float32), N)

    def gelu_backward(self, dinp, inp, dout, N):
        self._fn["gelu_backward"](_p(dinp, np.float32), _p(inp, np.float32), _p(dout, np.float32), N)

    def residual_forward(self, out, x, y, N):
        self._fn["residual_forward"](_p(out, np.float32), _p(x, np.float32), _p(y, np.float32), N)

    def residual_backward(self, dx, dy, dout, N):
        self._fn["residual_backward"](_p(dx, np.float32), _p(dy, np.float32), _p(dout, np.float32), N)

    def bayes_materialize(self, w, mu, rho, eps, n):
        self._fn["bayes_materialize"](*(_p(a, np.float32) for a in (w, mu, rho, eps)), n)

    def softmax_crossentropy(self, losses, probs, logits, targets, B, T, V):
        self._fn["softmax_crossentropy"](_p(losses, np.float32), _p(probs, np.float32), _p(logits, np.float32),
                                         _p(targets, np.int32), B, T, V)

    def crossentropy_softmax_backward(self, dlogits, probs, targets, B, T, V):
        self._fn["crossentropy_softmax_backward"](_p(dlogits, np.float32), _p(probs, np.float32),
                                                  _p(targets, np.int32), B, T, V)

    def bayes_backward(self, dmu, drho, dw, eps, rho, n):
        self._fn["bayes_backward"](*(_p(a, np.float32) for a in (dmu, drho, dw, eps, rho)), n)

    def kl_forward(self, mu, rho, n, sigma_prior) -> float:
        return float(self._fn["kl_forward"](_p(mu, np.float32), _p(rho, np.float32), n, sigma_prior))

    def kl_backward(self, dmu, drho, mu, rho, n, sigma_prior, weight):
        self._fn["kl_backward"](*(_p(a, np.float32) for a in (dmu, drho, mu, rho)), n, sigma_prior, weight)

    def adamw_update(self, params, grads, m, v, n, t, lr, beta1, beta2, eps, wd):
        self._fn["adamw_update"](*(_p(a, np.float32) for a in (params, grads, m, v)), n, t, lr, beta1,
                                 beta2, eps, wd)

    # ---- Philox and the GPU arms' ops (restatement only) ----------------------
    def philox4x32_10(self, ctr, key) -> np.ndarray:
        c = np.ascontiguousarray(ctr, dtype=np.uint32)
        k = np.ascontiguousarray(key, dtype=np.uint32)
        out = np.empty(4, np.uint32)
        self.lib.oracle_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
        return out

    def u01(self, x: int) -> float:
        return float(self.lib.oracle_u01(x))

    def philox_normal(self, seed: int, step: int, index: int) -> np.float32:
        return np.float32(self.lib.oracle_philox_normal(seed, step, index))

    def philox_normal_n(self, n: int, seed: int, step: int, first: int = 0) -> np.ndarray:
        eps = np.empty(n, np.float32)
        self.lib.oracle_philox_normal_n(eps.ctypes.data, n, seed, step, first)
        return eps

    def bayes_sample_philox(self, w, eps, mu, rho, n, seed, step):
        self.lib.oracle_bayes_sample_philox(_p(w, np.float32), None if eps is None else _p(eps, np.float32),
                                            _p(mu, np.float32), _p(rho, np.float32), n, seed, step)

    def bayes_backward_philox(self, dmu, drho, dw, rho, n, seed, step):
        self.lib.oracle_bayes_backward_philox(*(_p(a, np.float32) for a in (dmu, drho, dw, rho)), n, seed, step)

    def bbb_step_fused(self, mu, rho, m_mu, v_mu, m_rho, v_rho, w, dw, n, seed, step, sp, klw, bc1, bc2,
                       lr, beta1, beta2, aeps, wd):
        self.lib.oracle_bbb_step_fused(*(_p(a, np.float32) for a in (mu, rho, m_mu, v_mu, m_rho, v_rho, w, dw)),
                                       n, seed, step, sp, klw, bc1, bc2, lr, beta1, beta2, aeps, wd)

    # ---- file formats (restatement only) --------------------------------------
    def loader_windows(self, path: str, BT: int, steps: int):
        """(inputs, targets) of `steps` successive loader_next windows, or None if init fails."""
        class _L(ctypes.Structure):
            _fields_ = [("tokens", ctypes.c_void_p), ("n", ctypes.c_long), ("pos", ctypes.c_long)]
        ld = _L()
        self.lib.oracle_loader_init.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        self.lib.oracle_loader_init.restype = ctypes.c_int
        if self.lib.oracle_loader_init(ctypes.byref(ld), path.encode()) != 0:
            return None
        self.lib.oracle_loader_next.argtypes = [ctypes.c_void_p, _f, _f, _i]
        self.lib.oracle_loader_free.argtypes = [ctypes.c_void_p]
        inp = np.zeros((steps, BT), np.int32)
        tgt = np.zeros((steps, BT), np.int32)
        for k in range(steps):
            self.lib.oracle_loader_next(ctypes.byref(ld), inp[k].ctypes.data, tgt[k].ctypes.data, BT)
        self.lib.oracle_loader_free(ctypes.byref(ld))
        return inp, tgt

    def loader_count(self, path: str) -> int:
        self.lib.oracle_loader_count.argtypes = [ctypes.c_char_p]
        self.lib.oracle_loader_count.restype = ctypes.c_long
        return int(self.lib.oracle_loader_count(path.encode()))

    def ckpt_path(self, arm: str, what: str, C: int, L: int, steps: int) -> str:
        buf = ctypes.create_string_buffer(512)
        self.lib.oracle_ckpt_path.argtypes = [ctypes.c_char_p, _sz, ctypes.c_char_p, ctypes.c_char_p, _i, _i, _i]
        self.lib.oracle_ckpt_path(buf, 512, arm.encode(), what.encode(), C, L, steps)
        return buf.value.decode()

    def ckpt_header(self, n: int, C: int, L: int, V: int, NH: int, steps: int) -> np.ndarray:
        hdr = np.zeros(8, np.int32)
        self.lib.oracle_ckpt_header.argtypes = [_f, _sz, _i, _i, _i, _i, _i]
        self.lib.oracle_ckpt_header(hdr.ctypes.data, n, C, L, V, NH, steps)
        return hdr

    def ckpt_save(self, path: str, h: np.ndarray, C: int, L: int, V: int, NH: int, steps: int) -> int:
        self.lib.oracle_ckpt_save.argtypes = [ctypes.c_char_p, _f, _sz, _i, _i, _i, _i, _i]
        self.lib.oracle_ckpt_save.restype = ctypes.c_int
        return int(self.lib.oracle_ckpt_save(path.encode(), _p(h, np.float32), h.size, C, L, V, NH, steps))

    def ckpt_load(self, path: str, h: np.ndarray, C: int, L: int, V: int, NH: int) -> int:
        self.lib.oracle_ckpt_load.argtypes = [ctypes.c_char_p, _f, _sz, _i, _i, _i, _i]
        self.lib.oracle_ckpt_load.restype = ctypes.c_int
        return int(self.lib.oracle_ckpt_load(path.encode(), _p(h, np.float32), h.size, C, L, V, NH))

    # ---- host libm, elementwise (restatement only) ----------------------------
    def _map(self, name, x):
        y = np.empty_like(x)
        getattr(self.lib, name)(_p(y, np.float32), _p(x, np.float32), x.size)
        return y

    def expf(self, x):
        return self._map("oracle_expf_n", x)

    def log1pf(self, x):
        return self._map("oracle_log1pf_n", x)

    def tanhf(self, x):
        return self._map("oracle_tanhf_n", x)

    def softplus(self, x):
        return self._map("oracle_softplus_n", x)

    def logf(self, x):
        return self._map("oracle_logf_n", x)

    def cosf(self, x):
        return self._map("oracle_cosf_n", x)

    def sqrtf(self, x):
        return self._map("oracle_sqrtf_n", x)

    def float_range(self, lo: int, n: int) -> np.ndarray:
        x = np.empty(n, np.float32)
        self.lib.oracle_float_range(x.ctypes.data, lo, n)
        return x

    def bit_mismatches(self, a: np.ndarray, b: np.ndarray):
        """(count, first index) of positions whose bit patterns differ; NaN equals NaN."""
        first = _sz(0)
        n = self.lib.oracle_count_bit_mismatch(_p(a, np.float32), _p(b, np.float32), a.size,
                                               ctypes.byref(first))
        return int(n), (int(first.value) if n else -1)
