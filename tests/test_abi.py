"""CPU tests of the C-ABI boundary: the library loads, exports exactly what
include/ugk.h declares, and rejects invalid calls on the host (no GPU needed:
argument checks run before any HIP call)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ugk.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ugk_\w+)\s*\(", text)) - {"ugk_status_"})


def test_library_exports_every_declared_symbol():
    import ugk
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(ugk.lib, n)]
    assert not missing, missing


def test_header_declares_reference_ops():
    names = set(declared_functions())
    for op in ("encoder_forward", "encoder_backward", "layernorm_forward", "layernorm_backward",
               "gelu_forward", "gelu_backward", "residual_forward", "residual_backward",
               "bayes_materialize", "bayes_sample", "bayes_backward", "kl_forward", "kl_backward",
               "adamw_update", "bbb_step_fused"):
        assert "ugk_" + op in names


def test_invalid_arguments_rejected_on_host():
    import ugk
    lib = ugk.lib
    assert lib.ugk_residual_forward(None, None, None, -1) == 1
    assert b"N must be >= 0" in lib.ugk_last_error()
    assert lib.ugk_gelu_forward(None, None, 5) == 1
    assert b"NULL" in lib.ugk_last_error()
    assert lib.ugk_layernorm_forward(None, None, None, None, None, None, -1, 2, 3) == 1
    assert lib.ugk_layernorm_forward(1, 1, 1, 1, 1, 1, 2, 2, 0) == 1  # C=0 with rows: empty mean
    assert lib.ugk_encoder_backward(None, None, None, None, 2, 2, 2) == 1
    assert lib.ugk_bayes_materialize(None, None, None, None, 3) == 1
    # zero-size work is a no-op that succeeds without touching the GPU
    assert lib.ugk_residual_forward(None, None, None, 0) == 0
    assert lib.ugk_layernorm_backward(None, None, None, None, None, None, None, None, 0, 5, 7) == 0
    assert lib.ugk_encoder_forward(None, None, None, None, 0, 0, 0) == 0
    assert lib.ugk_last_error() == b""


def test_posterior_ops_reject_invalid_arguments_on_host():
    import ugk
    lib = ugk.lib
    assert lib.ugk_bayes_sample(None, None, None, None, 4, 1, 1) == 1
    assert b"NULL" in lib.ugk_last_error()
    assert lib.ugk_bayes_sample(16, 16, 32, 48, 4, 1, 1) == 1  # w == eps
    assert b"distinct" in lib.ugk_last_error()
    assert lib.ugk_bayes_backward(16, 16, 32, 48, 64, 4) == 1  # dmu == drho
    assert lib.ugk_bayes_backward_philox(16, 16, 32, 48, 4, 1, 1) == 1
    assert lib.ugk_kl_backward(16, 16, 32, 48, 4, 0.1, 1.0) == 1
    assert lib.ugk_adamw_update(16, 32, 48, 64, 4, 0, 1e-3, 0.9, 0.999, 1e-8, 0.0) == 1  # t = 0
    assert b"t must be >= 1" in lib.ugk_last_error()
    assert lib.ugk_adamw_update(16, 32, 16, 64, 4, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0) == 1  # params == m
    assert lib.ugk_bbb_step_fused(*([16] * 8), 4, 1, 1, *([0.1] * 9)) == 1
    assert lib.ugk_kl_forward(None, 16, 32, 4, 0.1) == 1
    kl = ctypes.c_double(5.0)
    assert lib.ugk_kl_forward(ctypes.byref(kl), None, None, 0, 0.1) == 0 and kl.value == 0.0
    assert lib.ugk_bayes_sample(None, None, None, None, 0, 1, 1) == 0
    assert lib.ugk_bbb_step_fused(*([None] * 8), 0, 1, 1, *([0.1] * 9)) == 0
    assert lib.ugk_diag_philox(None, None, 3) == 1
    assert lib.ugk_last_error() != b""
    assert lib.ugk_diag_stream(16, 8, 0, 1, 2, 256) == 1 and b"nr" in lib.ugk_last_error()  # nr out of range
    assert lib.ugk_diag_stream(16, 8, 2, 4, 2, 256) == 1  # nw out of range
    assert lib.ugk_diag_stream(16, 6, 2, 1, 2, 256) == 1 and b"multiple of 4" in lib.ugk_last_error()
    assert lib.ugk_diag_stream(None, 0, 2, 1, 2, 256) == 0


def test_fused_pairs_reject_invalid_arguments_on_host():
    import ugk
    lib = ugk.lib
    assert lib.ugk_residual_layernorm_forward(*([None] * 8), 2, 3, 4) == 1
    assert lib.ugk_residual_layernorm_forward(*([16] * 8), 2, 3, 0) == 1  # C = 0 with rows
    assert lib.ugk_layernorm_residual_backward(*([16] * 10), 2, 3, 4) == 1  # dinp == dx
    assert b"distinct" in lib.ugk_last_error()
    assert lib.ugk_layernorm_residual_backward(*([None] * 10), -1, 3, 4) == 1
    assert lib.ugk_residual_layernorm_forward(*([None] * 8), 0, 3, 4) == 0
    assert lib.ugk_layernorm_residual_backward(*([None] * 10), 2, 3, 0) == 0
    assert lib.ugk_encoder_layernorm_forward(*([None] * 9), 2, 3, 4) == 1
    assert lib.ugk_encoder_layernorm_forward(*([16] * 9), 2, 3, 0) == 1  # C = 0 with rows
    assert lib.ugk_encoder_layernorm_forward(*([None] * 9), 0, 3, 4) == 0


def test_param_layout_counts():
    """Closed-form sizes of the reference layout (gpt2_kernels.cuh:656-719)."""
    import ugk
    # the reference's CPU-runnable configuration / the paper's P: C=384 L=6 V=27 maxT=1024 -> 11,061,531
    cfg = ugk.Config(B=4, T=64, C=384, V=27, NH=6, maxT=1024, L=6)
    assert ugk.param_count(cfg) == 11_061_531
    C, V, L, maxT = 768, 50257, 12, 1024
    cfg = ugk.Config(B=8, T=1024, C=C, V=V, NH=12, maxT=maxT, L=L)
    assert ugk.param_count(cfg) == V * C + maxT * C + L * (12 * C * C + 13 * C) + 2 * C + C * V + V
    BT = 8 * 1024
    # per block: lno qkv(3) atty apr resa ln2o fch(4) gelu(4) mlpo res1 = 18 C per row, + 4 row stats
    assert ugk.act_count(cfg) == BT * C + L * (BT * 18 * C + 4 * BT) + BT * C + 2 * BT + 2 * BT * V + BT


def test_config_checks():
    import ugk
    bad = ugk.Config(B=1, T=8, C=16, V=5, NH=1, maxT=4, L=1)  # maxT < T
    with pytest.raises(ValueError):
        ugk.gpt2_layers_forward(0, 0, 0, bad)
    lib = ugk.lib
    assert lib.ugk_gpt2_layers_forward(1, 1, 1, bad, None) == 1
    # both backwards check the config and their pointers on the host, before any HIP call
    for fn in (lib.ugk_gpt2_layers_backward, lib.ugk_gpt2_layers_backward_zeroed):
        assert fn(1, 1, 1, 1, 1, bad, None) == 1
        good = ugk.Config(B=1, T=8, C=16, V=5, NH=1, maxT=8, L=1)
        assert fn(None, 1, 1, 1, 1, good, None) == 1
        assert b"NULL pointer" in lib.ugk_last_error()
    with pytest.raises(ValueError):
        ugk.gpt2_layers_backward_zeroed(0, 0, 0, 0, 0, bad)


def test_binding_rejects_cpu_tensors():
    import torch
    import ugk
    x = torch.zeros(8)
    with pytest.raises(ValueError):
        ugk.residual_forward(x, x, x, 8)
    tok = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError):  # the token check leaves CPU tensors to the argument checks
        ugk.encoder_forward(x, tok, x, x, 1, 2, 4)
    with pytest.raises(ValueError):
        ugk.encoder_layernorm_forward(x, x, x[:2], x[:2], tok, x, x, x[:4], x[:4], 1, 2, 4)
    with pytest.raises(ValueError):
        ugk.softmax_crossentropy(x[:2], x, x, tok, 1, 2, 4)


def test_product_does_not_use_the_oracle():
    """The shipped code never imports, links or loads anything under oracle/."""
    pkg = os.path.join(ROOT, "uncertain-gpt_amd")
    uses = re.compile(r"import\s+oracle|from\s+oracle|liboracle|libtrain_bnn|_ref/|oracle_\w+\s*\(|"
                      r"#include\s+[\"<][^\">]*oracle")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp", "Makefile")):
                text = open(os.path.join(dirpath, f), errors="replace").read()
                assert not uses.search(text), os.path.join(dirpath, f)


def test_stream_roundtrip():
    import ugk
    assert ugk.lib.ugk_set_stream(None) == 0
    assert ugk.lib.ugk_get_stream() in (None, 0)
    assert ugk.version() >= 100


def test_layernorm_workspace_bound_covers_smaller_calls():
    """The LayerNorm slot of the workspace is sized by a bound on the partial rows that holds for
    every call with at most the config's rows (a path's own count drops once a call would exceed its
    cap, so sizing by the count at the config's rows alone left some smaller calls short)."""
    import ugk
    a, b = ctypes.c_int(0), ctypes.c_int(0)

    def rows_of(rows, C, fused):
        assert ugk.lib.ugk_diag_layernorm_partial_rows(rows, C, fused, ctypes.byref(a), ctypes.byref(b)) == 0
        return a.value, b.value

    for C in (4, 13, 384, 516, 766, 768, 772, 1024, 1030, 2048, 2052):
        for cfg_rows in (64, 1000, 2048, 3072, 4000, 4096, 5120, 8192, 12288, 16384, 40000):
            bound = rows_of(cfg_rows, C, 0)[1]
            for rows in sorted({1, 2, 15, 16, 17, 255, 256, 2047, 2048, 2049, 4095, 4096, 4097, 8191, 8192, 8193,
                                16383, 16384, 16385, cfg_rows // 3, cfg_rows // 2, cfg_rows - 1, cfg_rows}):
                if 0 < rows <= cfg_rows:
                    for fused in (0, 1):
                        actual, request = rows_of(rows, C, fused)
                        # what the call runs with, and what it asks the workspace for
                        assert actual <= request <= bound, (C, cfg_rows, rows, fused, actual, request, bound)
    # the case that failed: sized for B=5, T=1024 at C=768, called at B=4 (and B=3)
    bound = rows_of(5 * 1024, 768, 0)[1]
    assert rows_of(4 * 1024, 768, 0)[0] <= bound and rows_of(3 * 1024, 768, 1)[0] <= bound
    # and the workspace grows with the rows it is sized for
    sizes = [ugk.workspace_bytes(ugk.Config(B=B, T=1024, C=768, V=50257, NH=12, maxT=1024, L=12))
             for B in range(1, 17)]
    assert sizes == sorted(sizes)


def test_layernorm_partial_rows_within_bound_dense():
    """Every LayerNorm backward shape makes at most as many partial rows as the workspace bound at its
    own rows, for every row count up to 4,100, every 37th up to 70,000 and a few powers of two, at 14
    widths, plain and fused: the bound sizes the slot, and the launchers cap the workgroups at it."""
    import ugk
    a, b = ctypes.c_int(0), ctypes.c_int(0)
    rows_list = sorted(set(range(1, 4101)) | set(range(4100, 70000, 37)) | {8192, 16384, 32768, 65536, 131072})
    bad = []
    for C in (4, 64, 384, 512, 768, 772, 1024, 1028, 1030, 1600, 2048, 3072, 4096, 8192):
        for rows in rows_list:
            for fused in (0, 1):
                assert ugk.lib.ugk_diag_layernorm_partial_rows(rows, C, fused, ctypes.byref(a), ctypes.byref(b)) == 0
                if a.value > b.value:
                    bad.append((rows, C, fused, a.value, b.value))
    assert not bad, bad[:5]
