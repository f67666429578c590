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
        if not reference:
            for name in ("oracle_expf_n", "oracle_log1pf_n", "oracle_tanhf_n", "oracle_softplus_n"):
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
