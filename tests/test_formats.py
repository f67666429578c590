"""CPU tests of the file formats (gpt2_kernels.cuh:898-964, :1281-1331): the llm.c .bin token
loader and the checkpoint header, against the oracle's restatement, which is pinned first against
the format as the reference's own writer defines it (data/data_common.py:40-60: 256 int32 header,
magic 20240520, version 1, the token count in header[2], then uint16 tokens) and against plain
numpy slicing of the token stream."""
import os

import numpy as np
import pytest

import gen


def write_tokens(path, toks, magic=20240520):
    """The reference writer's layout (data/data_common.py:40-60), restated."""
    header = np.zeros(256, np.int32)
    header[0], header[1], header[2] = magic, 1, len(toks)
    with open(path, "wb") as f:
        f.write(header.tobytes())
        f.write(np.asarray(toks, np.uint16).tobytes())


def expected_windows(toks, BT, steps):
    """gpt2_kernels.cuh:924-929 in numpy: restart at 0 when pos + BT + 1 > n."""
    toks = np.asarray(toks, np.int64)
    pos, inp, tgt = 0, [], []
    for _ in range(steps):
        if pos + BT + 1 > len(toks):
            pos = 0
        inp.append(toks[pos:pos + BT])
        tgt.append(toks[pos + 1:pos + BT + 1])
        pos += BT
    return np.array(inp, np.int32), np.array(tgt, np.int32)


@pytest.fixture
def token_file(tmp_path):
    g = gen.rng(31)
    toks = g.integers(0, 50257, 10_007).astype(np.uint16)
    toks[:3] = [0, 65535, 50256]
    path = str(tmp_path / "toks.bin")
    write_tokens(path, toks)
    return path, toks


def test_oracle_loader_is_the_reference_rule(oracle, token_file):
    path, toks = token_file
    assert oracle.loader_count(path) == len(toks)
    for BT in (1, 64, 1000, 5003):
        got = oracle.loader_windows(path, BT, 25)
        want = expected_windows(toks, BT, 25)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_loader_matches_oracle_on_host(oracle, token_file):
    import ugk
    path, toks = token_file
    assert ugk.loader_count(path) == len(toks)
    for BT in (1, 64, 1000, 5003, len(toks) - 1):
        ld = ugk.Loader(path)
        assert ld.tokens == len(toks)
        inp, tgt = oracle.loader_windows(path, BT, 12)
        for k in range(12):
            a, b = np.zeros(BT, np.int32), np.zeros(BT, np.int32)
            ld.next(a, b, BT)
            assert np.array_equal(a, inp[k]) and np.array_equal(b, tgt[k]), (BT, k)
        ld.close()


def test_loader_rejects_bad_files(oracle, tmp_path, token_file):
    import ugk
    path, toks = token_file
    bad = str(tmp_path / "bad.bin")
    write_tokens(bad, toks, magic=20240801)  # the llama-3 magic: not this format
    short = str(tmp_path / "short.bin")
    with open(path, "rb") as f, open(short, "wb") as g:
        g.write(f.read()[:1024 + 100])
    for p in (bad, short, str(tmp_path / "missing.bin")):
        with pytest.raises(ugk.UgkError):
            ugk.Loader(p)
        assert oracle.loader_windows(p, 4, 1) is None
    with pytest.raises(ugk.UgkError):
        ugk.loader_count(bad)
    ld = ugk.Loader(path)
    with pytest.raises(ugk.UgkError):  # a window needs BT + 1 tokens
        ld.next(np.zeros(len(toks), np.int32), np.zeros(len(toks), np.int32), len(toks))
    ld.close()


def test_ckpt_path_and_header(oracle):
    import ugk
    cfg = ugk.Config(B=8, T=1024, C=768, V=50257, NH=12, maxT=1024, L=12)
    assert ugk.ckpt_path("bbb", "mu", cfg, 20000) == oracle.ckpt_path("bbb", "mu", 768, 12, 20000) \
        == "runs/bbb_C768_L12_20k_mu.bin"
    # n above 2^32 splits into header[1] (low word) and header[7] (high word)
    n = (5 << 32) + 123
    h = oracle.ckpt_header(n, 768, 12, 50257, 12, 7)
    assert h.tolist() == [20240520, 123, 768, 12, 50257, 12, 7, 5]


def test_oracle_ckpt_round_trip(oracle, tmp_path):
    g = gen.rng(32)
    x = gen.normal(g, (1001,))
    p = str(tmp_path / "c.bin")
    assert oracle.ckpt_save(p, x, 384, 6, 27, 6, 5000) == 0
    raw = np.fromfile(p, np.int32, count=8)
    assert raw.tolist() == [20240520, 1001, 384, 6, 27, 6, 5000, 0]
    assert np.array_equal(np.fromfile(p, np.float32, offset=32), x)
    y = np.zeros_like(x)
    assert oracle.ckpt_load(p, y, 384, 6, 27, 6) == 5000 and np.array_equal(x, y)
    assert oracle.ckpt_load(p, y, 768, 6, 27, 6) == -1  # shape mismatch
