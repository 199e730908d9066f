"""The native C++ caller (triton-ext_amd/driver/tx_driver.cpp): it drives the
plugin through include/tx_plugin.h and libtxamd.so alone, with no Python or
torch in the process, and checks each hot-path entry point against closed-form
answers (every e4m3fn code round-trips, a scatter of ones fills each bin with
its known count, constant-operand GEMM / GEMV outputs are exact bf16/fp16
values)."""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER_DIR = os.path.join(REPO, "triton-ext_amd", "driver")
DRIVER = os.path.join(DRIVER_DIR, "tx_driver")


def _needed(path):
    out = subprocess.run(["readelf", "-d", path], check=True, capture_output=True, text=True).stdout
    return [line.split("[", 1)[1].split("]", 1)[0] for line in out.splitlines() if "(NEEDED)" in line]


def test_driver_links_only_the_c_abi(tx):
    """Builds from the public header and links against libtxamd.so and the HIP
    runtime only: nothing from torch or Python."""
    subprocess.run(["make", "-B", "-s", "-C", DRIVER_DIR, "CXX=g++"], check=True)
    needed = _needed(DRIVER)
    assert "libtxamd.so" in needed
    assert any(n.startswith("libamdhip64") for n in needed)
    assert not any("torch" in n or "python" in n or n.startswith("libc10") for n in needed), needed


@pytest.mark.gpu
def test_driver_checks_pass_on_the_gpu():
    if not os.path.exists(DRIVER):
        subprocess.run(["make", "-s", "-C", DRIVER_DIR], check=True)
    r = subprocess.run([DRIVER, "--check"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAILED" not in r.stdout
    assert "0 check(s) failed" in r.stdout
