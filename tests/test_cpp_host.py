"""The C++ mirror of GpuMoeDispatcher (silentotithrandousha_amd/host/gpu_moe_dispatcher.hpp),
compiled with g++ against the built library and driven by tests/cpp/dispatcher_test.cpp."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "silentotithrandousha_amd")
ORC = os.path.join(ROOT, "oracle")


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    for lib in (os.path.join(PKG, "libmxfp4moe.so"), os.path.join(ORC, "liborc.so")):
        if not os.path.exists(lib):
            pytest.fail(f"{lib} is not built (run __graft_entry__.build())")
    out = str(tmp_path_factory.mktemp("cpp") / "dispatcher_test")
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-o", out,
           os.path.join(ROOT, "tests", "cpp", "dispatcher_test.cpp"),
           f"-L{PKG}", "-lmxfp4moe", f"-L{ORC}", "-lorc", "-L/opt/rocm/lib",
           f"-Wl,-rpath,{PKG}:{ORC}"]
    subprocess.run(cmd, check=True)
    return out


def test_cpp_mirror_constructor_error_without_device(exe):
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is visible: the no-device error path cannot be exercised")
    r = subprocess.run([exe, "cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
def test_cpp_mirror_layer_vs_oracle(exe):
    r = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
