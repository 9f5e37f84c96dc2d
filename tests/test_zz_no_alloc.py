"""The allocation-free forward (moe_layer_forward_device_noalloc) through the C ABI against
moe_layer_forward_device on the same device inputs: identical outputs on consecutive calls whose
sizes shrink (so a later call meets the scratch array as the earlier, larger call left it), on
the single-token one-launch path and the batch paths; within the tolerance of the oracle; sizes
beyond the scratch array refused."""
import ctypes

import numpy as np
import pytest

from silentotithrandousha_amd import DeviceBuffer, GpuMoeDispatcher
from silentotithrandousha_amd import synthetic as syn
from silentotithrandousha_amd._ffi import MoeError, check, lib
from tests.helpers import assert_bit_exact, assert_rel_l2

pytestmark = pytest.mark.gpu

H = I = 2880


def _run(d, fn, x, k):
    T = x.shape[0]
    xd = DeviceBuffer.from_array(x)
    yd = DeviceBuffer(T * H * 4)
    check(fn(d.ctx, 0, ctypes.c_void_p(xd.ptr), T, k, ctypes.c_void_p(yd.ptr), None))
    d.synchronize()
    return yd.download(np.float32, (T, H))


def test_noalloc_matches_device_forward(orc):
    L = syn.make_layer(H, I, 32, seed=480)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    na, ref = lib().moe_layer_forward_device_noalloc, lib().moe_layer_forward_device
    # two calls in a row, the second smaller, then the one-launch single token and a batch again
    for T, seed in ((96, 481), (64, 482), (5, 483), (1, 484), (2, 485), (64, 486)):
        x = syn.hidden(T, H, seed=seed)
        got = _run(d, na, x, 4)
        assert_bit_exact(got, _run(d, ref, x, 4), f"noalloc vs device forward T={T}")
        if T <= 8:
            assert_rel_l2(got, orc.moe_layer(x, L, 4)[0], f"noalloc vs oracle T={T}")
    with pytest.raises(MoeError, match="scratch"):
        _run(d, na, syn.hidden(512, H, seed=487), 4)
    d.close()


def test_noalloc_two_contexts_one_device():
    """Two contexts on one GPU use the same scratch array one after the other: each call's result
    equals its own context's allocating forward."""
    Ls = [syn.make_layer(256, 128, 8, seed=490 + i) for i in range(2)]
    ds = []
    for L in Ls:
        d = GpuMoeDispatcher(256, 128, 7.0)
        d.preload_layer(0, L)
        ds.append(d)
    na, ref = lib().moe_layer_forward_device_noalloc, lib().moe_layer_forward_device
    x = syn.hidden(40, 256, seed=495)
    xd = DeviceBuffer.from_array(x)
    for rep in range(2):
        for d in ds:
            outs = []
            for fn in (na, ref):
                yd = DeviceBuffer(40 * 256 * 4)
                check(fn(d.ctx, 0, ctypes.c_void_p(xd.ptr), 40, 4, ctypes.c_void_p(yd.ptr), None))
                d.synchronize()
                outs.append(yd.download(np.float32, (40, 256)))
            assert_bit_exact(outs[0], outs[1], f"context {ds.index(d)} rep {rep}")
    for d in ds:
        d.close()


def test_noalloc_under_graph_capture():
    """The property the entry point exists for: on a fresh context, whose workspace no call has
    sized, the allocation-free forward is captured into a HIP graph (the allocating forward
    refuses to size its workspace while capturing); every replay, with eager calls between them,
    gives the allocating forward's bits. Covers a batch (the grouped-GEMM path) and a single token
    (the one-launch path)."""
    L = syn.make_layer(H, I, 32, seed=500)
    for T, seed in ((48, 501), (1, 502)):
        d = GpuMoeDispatcher(H, I, 7.0)
        d.preload_layer(0, L)
        x = syn.hidden(T, H, seed=seed)
        xd, yd = DeviceBuffer.from_array(x), DeviceBuffer(T * H * 4)
        check(lib().moe_memset_device(ctypes.c_void_p(yd.ptr), 0, T * H * 4))
        ref_fn, na = lib().moe_layer_forward_device, lib().moe_layer_forward_device_noalloc
        with pytest.raises(MoeError):  # the allocating forward cannot size a workspace in a capture
            check(lib().moe_graph_begin(d.ctx))
            try:
                check(ref_fn(d.ctx, 0, ctypes.c_void_p(xd.ptr), T, 4, ctypes.c_void_p(yd.ptr), None))
            finally:
                g = ctypes.c_void_p()
                if lib().moe_graph_end(d.ctx, ctypes.byref(g)) == 0 and g.value:
                    lib().moe_graph_destroy(g)
        check(lib().moe_graph_begin(d.ctx))
        try:
            check(na(d.ctx, 0, ctypes.c_void_p(xd.ptr), T, 4, ctypes.c_void_p(yd.ptr), None))
        finally:
            g = ctypes.c_void_p()
            check(lib().moe_graph_end(d.ctx, ctypes.byref(g)))
        want = _run(d, ref_fn, x, 4)  # eager, after the capture (sizes the context's workspace)
        try:
            for rep in range(3):
                check(lib().moe_memset_device(ctypes.c_void_p(yd.ptr), 0xFF, T * H * 4))
                check(lib().moe_graph_launch(d.ctx, g))
                d.synchronize()
                assert_bit_exact(yd.download(np.float32, (T, H)), want, f"graph replay {rep} T={T}")
                _run(d, na, syn.hidden(T, H, seed=seed + 10 + rep), 4)  # eager work between replays
        finally:
            check(lib().moe_graph_destroy(g))
        d.close()
