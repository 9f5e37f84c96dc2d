"""Python host front end of the Beaver-triple generator (include/beaver32.h), mirroring the
reference's GpuTripleGen32 (src/gpu/mod.rs:511-1012). The reference draws the round seeds from
its rng inside the call (mod.rs:646); here the caller passes them (num_rounds = ceil(count /
spr) values), so runs are reproducible. OT correlations are accepted and not read: the kernel
uses them only for a_mixed, which no output depends on (shader32.metal:96-108)."""
import ctypes

import numpy as np

from ._ffi import check, lib


class GpuTripleGen32:
    """GpuTripleGen32::new(n, t) — gpu/mod.rs:523-634 (n > 2t, n <= 8, n - 2t <= 3)."""

    def __init__(self, n, t):
        ctx = ctypes.c_void_p()
        check(lib().beaver32_create(int(n), int(t), ctypes.byref(ctx)))
        self._ctx = ctx.value
        self.n, self.t = int(n), int(t)
        self.spr = int(lib().beaver32_spr(self._ctx))

    @property
    def ctx(self):
        return self._ctx

    def num_rounds(self, count):
        return -(-int(count) // self.spr)

    def generate(self, count, round_seeds, ot_correlations=None):
        """gpu/mod.rs:636-707: (a, b, c), each [n, count] uint32 (party-major)."""
        seeds = np.ascontiguousarray(round_seeds, np.uint32)
        assert seeds.size >= self.num_rounds(count)
        a, b, c = (np.empty((self.n, count), np.uint32) for _ in range(3))
        check(lib().beaver32_generate(self._ctx, count, None, seeds.ctypes.data, a.ctypes.data, b.ctypes.data,
                                      c.ctypes.data))
        return a, b, c

    def generate_single_party(self, party, count, round_seeds, ot_correlations=None):
        """gpu/mod.rs:709-765: party `party`'s (a, b, c), each [count] uint32."""
        seeds = np.ascontiguousarray(round_seeds, np.uint32)
        assert seeds.size >= self.num_rounds(count)
        a, b, c = (np.empty(count, np.uint32) for _ in range(3))
        check(lib().beaver32_generate_single_party(self._ctx, party, count, None, seeds.ctypes.data, a.ctypes.data,
                                                   b.ctypes.data, c.ctypes.data))
        return a, b, c

    def generate_device(self, party, count, seeds_dev, a_dev, b_dev, c_dev, stream=None):
        """Device buffers (DeviceBuffer or int addresses), asynchronous: the preallocated
        zero-copy path (mod.rs:840-938) for party >= 0, every party for party = -1."""
        dp = [ctypes.c_void_p(x.ptr if hasattr(x, "ptr") else int(x)) for x in (seeds_dev, a_dev, b_dev, c_dev)]
        check(lib().beaver32_generate_device(self._ctx, int(party), count, *dp, stream))

    def synchronize(self):
        check(lib().beaver32_synchronize(self._ctx))

    def close(self):
        if getattr(self, "_ctx", None):
            lib().beaver32_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
