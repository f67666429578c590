"""The drop-in boundary from C: include/ugk.h is a C99 header, and tests/c_host_check.c, a C
program built by gcc against it and linked with libugk.so, calls the layer ops with
train_bnn.c's argument lists and matches the CPU oracle (bit-exact for encoder, GELU, residual
and materialize; LayerNorm within 1e-5 relative / 1e-6 absolute) at config 1's shapes."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(ROOT, "uncertain-gpt_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")
SRC = os.path.join(ROOT, "tests", "c_host_check.c")


def gcc():
    g = shutil.which("gcc")
    if g is None:
        pytest.skip("gcc not available")
    return g


def test_header_compiles_as_c99(tmp_path):
    src = tmp_path / "h.c"
    src.write_text('#include "ugk.h"\nint main(void) { return ugk_version() > 0 ? 0 : 1; }\n')
    r = subprocess.run([gcc(), "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def build_c_host(tmp_path):
    for lib in (os.path.join(LIB_DIR, "libugk.so"), os.path.join(ORACLE_DIR, "liboracle.so")):
        if not os.path.exists(lib):
            pytest.skip(f"{os.path.basename(lib)} not built")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    exe = str(tmp_path / "c_host_check")
    r = subprocess.run([gcc(), "-std=c99", "-Wall", "-Wextra", "-Werror", "-O2", "-D__HIP_PLATFORM_AMD__",
                        "-I", os.path.join(rocm, "include"), "-I", os.path.join(ROOT, "include"), "-I", ORACLE_DIR,
                        SRC, "-o", exe, "-L", LIB_DIR, "-lugk", "-L", ORACLE_DIR, "-loracle",
                        "-L", os.path.join(rocm, "lib"), "-lamdhip64", "-lm",
                        "-Wl,-rpath," + LIB_DIR, "-Wl,-rpath," + ORACLE_DIR], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_c_host_program_builds(tmp_path):
    build_c_host(tmp_path)


@pytest.mark.gpu
def test_c_host_program_matches_oracle(tmp_path):
    exe = build_c_host(tmp_path)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("c host check: 0 failures"), r.stdout + r.stderr
