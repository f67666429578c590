"""Shared test setup: import paths, the `gpu` marker and common fixtures.

`-m "not gpu"` runs on any machine (CPU oracle, golden fixtures, host-side
argument checks, library exports). `-m gpu` needs a visible GPU and calls the
HIP kernels through the C-ABI of libugk.so.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "uncertain-gpt_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU; calls the HIP kernels through libugk.so")


def pytest_sessionfinish(session, exitstatus):
    import literal_bar
    literal_bar.write()


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref_oracle():
    from oracle import Oracle, REF_SO
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref/libtrain_bnn.so not built (needs /root/reference; make -C oracle ref)")
    return Oracle(reference=True)


@pytest.fixture(scope="session")
def gpu():
    """The ugk binding, on a machine whose GPU is visible."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import ugk
    return ugk
