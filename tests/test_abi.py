"""CPU tests of the C ABI boundary: the library loads, exports every symbol the header
declares, and validates arguments on the host without a GPU."""
import ctypes
import os
import re

import pytest

from silentotithrandousha_amd import _ffi

HEADER = _ffi.HEADER_PATH


def declared_functions():
    names = []
    for h in _ffi.HEADER_PATHS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b((?:moe|beaver32)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_dispatcher_surface():
    names = declared_functions()
    for n in ["moe_create", "moe_destroy", "moe_preload_layer", "moe_dispatch_expert_preloaded",
              "moe_dispatch_expert", "moe_dispatch_experts_batched", "moe_init_lm_head",
              "moe_dispatch_lm_head", "moe_router_topk", "moe_layer_forward",
              "moe_mxfp4_dequant_device", "moe_last_error"]:
        assert n in names, n


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_ffi.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_functions()) == set(_ffi.SIGNATURES), \
        set(declared_functions()) ^ set(_ffi.SIGNATURES)


def test_host_side_validation_without_gpu():
    L = _ffi.lib()
    assert L.moe_mxfp4_packed_size(5760, 2880) == 5760 * 90 * 16 + 360 * 6 * 256
    assert L.moe_mxfp4_packed_size(10, 2880) == 0        # rows must be a multiple of 16
    assert L.moe_set_adaptive_topk(None, 1, 3, 0.9, 0.35, 0.98) == _ffi.MOE_ERR_INVALID
    assert b"null context" in L.moe_last_error()
    ctx = ctypes.c_void_p()
    assert L.moe_create(2880, 100, 7.0, ctypes.byref(ctx)) == _ffi.MOE_ERR_INVALID
    assert b"multiples of 32" in L.moe_last_error()
    assert L.moe_create(2880, 2880, float("nan"), ctypes.byref(ctx)) == _ffi.MOE_ERR_INVALID
    assert L.moe_dispatch_lm_head(None, None, 1, None) == _ffi.MOE_ERR_INVALID
    assert L.moe_version().startswith(b"mxfp4_moe")
    # GpuTripleGen32::new's parameter checks (gpu/mod.rs:525-536) come before any device query
    for n, t, msg in ((4, 2, b"n > 2t"), (9, 1, b"n <= 8"), (8, 1, b"HIM table")):
        assert L.beaver32_create(n, t, ctypes.byref(ctx)) == _ffi.MOE_ERR_INVALID
        assert msg in L.moe_last_error()
    assert L.beaver32_generate(None, 1, None, None, None, None, None) == _ffi.MOE_ERR_INVALID


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible")
def test_create_without_device_fails_cleanly():
    L = _ffi.lib()
    ctx = ctypes.c_void_p()
    rc = L.moe_create(2880, 2880, 7.0, ctypes.byref(ctx))
    assert rc in (_ffi.MOE_ERR_NO_DEVICE, _ffi.MOE_ERR_HIP)
    assert ctx.value is None
