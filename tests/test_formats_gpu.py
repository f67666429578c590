"""GPU: checkpoints written from and read into device buffers are byte-identical to the oracle's
files (gpt2_kernels.cuh:944-964, :1281-1316), including buffers spanning several 64 MB staging
chunks; the device token windows equal the oracle loader's (gpt2_kernels.cuh:924-929)."""
import numpy as np
import pytest
import torch

import gen
from test_formats import write_tokens

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("n", [0, 1, 5_000_003, 40_000_001])
def test_ckpt_save_load_device(gpu, oracle, tmp_path, n):
    cfg = gpu.Config(B=8, T=1024, C=768, V=50257, NH=12, maxT=1024, L=12)
    g = torch.Generator(DEV).manual_seed(n % 1000)
    d = torch.randn(max(n, 1), device=DEV, generator=g)[:n] if n else torch.empty(0, device=DEV)
    path, ref = str(tmp_path / "dev.bin"), str(tmp_path / "ref.bin")
    gpu.ckpt_save(path, d, n, cfg, 20000)
    h = d.cpu().numpy()
    assert oracle.ckpt_save(ref, np.ascontiguousarray(h), 768, 12, 50257, 12, 20000) == 0
    assert open(path, "rb").read() == open(ref, "rb").read()
    back = torch.full((max(n, 1),), float("nan"), device=DEV)[:n] if n else torch.empty(0, device=DEV)
    assert gpu.ckpt_load(ref, back, n, cfg) == 20000
    torch.cuda.synchronize()
    assert torch.equal(back, d)


def test_ckpt_load_rejects_mismatch(gpu, oracle, tmp_path):
    x = gen.normal(gen.rng(5), (100,))
    p = str(tmp_path / "c.bin")
    oracle.ckpt_save(p, x, 384, 6, 27, 6, 1000)
    buf = torch.zeros(100, device=DEV)
    with pytest.raises(gpu.UgkError, match="shape mismatch"):
        gpu.ckpt_load(p, buf, 100, gpu.Config(B=4, T=64, C=768, V=27, NH=6, maxT=64, L=6))
    with pytest.raises(gpu.UgkError, match="shape mismatch"):
        gpu.ckpt_load(p, buf, 99, gpu.Config(B=4, T=64, C=384, V=27, NH=6, maxT=64, L=6))
    with open(p, "r+b") as f:
        f.write(np.int32(20240801).tobytes())
    with pytest.raises(gpu.UgkError, match="bad magic"):
        gpu.ckpt_load(p, buf, 100, gpu.Config(B=4, T=64, C=384, V=27, NH=6, maxT=64, L=6))
    assert torch.equal(buf, torch.zeros(100, device=DEV))  # nothing loaded on failure


@pytest.mark.parametrize("BT", [1, 4096, 8192])
def test_loader_device_windows(gpu, oracle, tmp_path, BT):
    toks = gen.rng(BT).integers(0, 50257, 3 * BT + 17).astype(np.uint16)
    path = str(tmp_path / "t.bin")
    write_tokens(path, toks)
    inp, tgt = oracle.loader_windows(path, BT, 9)
    ld = gpu.Loader(path)
    di, dt = torch.empty(BT, dtype=torch.int32, device=DEV), torch.empty(BT, dtype=torch.int32, device=DEV)
    for k in range(9):
        ld.next_device(di, dt, BT)
        torch.cuda.synchronize()
        assert np.array_equal(di.cpu().numpy(), inp[k]) and np.array_equal(dt.cpu().numpy(), tgt[k]), k
    ld.close()
