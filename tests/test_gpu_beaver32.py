"""GPU parity of the Beaver-triple generator (include/beaver32.h; the reference's
GpuTripleGen32, src/gpu/mod.rs:511-1012, shader32.metal:75-167) through the C ABI: every output
word equal to the oracle's (orc_beaver32) for every party and single parties, at counts below one
threadgroup of rounds, with partial last groups, and at the reference's 2M-triple size; the
device-pointer form identical; the triple property (Shamir reconstruction gives c = a b)."""
import os
import sys

import numpy as np
import pytest

from silentotithrandousha_amd import DeviceBuffer, GpuTripleGen32
from silentotithrandousha_amd._ffi import MoeError

pytestmark = pytest.mark.gpu

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import beaver32_ref as ref  # noqa: E402


def _seeds(count, spr, seed):
    return np.random.default_rng(seed).integers(0, 1 << 32, -(-count // spr), dtype=np.uint64).astype(np.uint32)


@pytest.mark.parametrize("n,t,count", [(5, 1, 1), (5, 1, 100), (5, 1, 1000), (5, 1, 2_000_000), (3, 1, 777),
                                       (7, 2, 4099), (8, 3, 65)])
def test_triples_match_oracle(orc, n, t, count):
    g = GpuTripleGen32(n, t)
    seeds = _seeds(count, g.spr, 80 + n + count)
    want = orc.beaver32(n, t, count, seeds)
    got = g.generate(count, seeds)
    for w, x, name in zip(want, got, "abc"):
        assert np.array_equal(x, w), f"{name} n={n} t={t} count={count}"
    for p in sorted({0, n - 1}):
        sp = g.generate_single_party(p, count, seeds)
        for w, x, name in zip(want, sp, "abc"):
            assert np.array_equal(x, w[p]), f"{name} party {p}"
    g.close()


def test_device_form_and_property(orc):
    n, t, count = 5, 1, 30001
    g = GpuTripleGen32(n, t)
    seeds = _seeds(count, g.spr, 90)
    sd = DeviceBuffer.from_array(seeds)
    outs = [DeviceBuffer(n * count * 4) for _ in range(3)]
    g.generate_device(-1, count, sd, *outs)
    g.synchronize()
    got = [o.download(np.uint32, (n, count)) for o in outs]
    want = orc.beaver32(n, t, count, seeds)
    for w, x in zip(want, got):
        assert np.array_equal(x, w)
    g.generate_device(2, count, sd, *outs)
    g.synchronize()
    for w, o in zip(want, outs):
        assert np.array_equal(o.download(np.uint32, (count,)), w[2])
    a, b, c = got
    for k in range(0, count, 997):
        A = ref.lagrange_at_zero([int(a[p, k]) for p in range(n)], n)
        B = ref.lagrange_at_zero([int(b[p, k]) for p in range(n)], n)
        assert ref.lagrange_at_zero([int(c[p, k]) for p in range(n)], n) == A * B % ref.P
    with pytest.raises(MoeError, match="party"):
        g.generate_single_party(n, 10, seeds)
    g.close()
