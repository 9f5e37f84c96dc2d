"""CPU tests of the Beaver-triple oracle (oracle/moe_oracle.c, orc_beaver32: the reference's
shader32.metal:4-167 as dispatched by gpu/mod.rs:975-1000). The reference's tests check only
the triple property (c = a b after Shamir reconstruction, beaver.rs:3516-3568,
beaver32.rs:352-398); the oracle is pinned by that property, by field-arithmetic closed forms,
and by an independent Python-integer restatement (tests/golden/beaver32_ref.py)."""
import os
import sys

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import beaver32_ref as ref  # noqa: E402

P = ref.P


def test_field_ops_closed_forms(orc):
    L = orc.lib()
    rng = np.random.default_rng(70)
    vals = [0, 1, 2, P - 1, P - 2, 1 << 30, (1 << 30) + 1] + [int(v) for v in rng.integers(0, P, 200)]
    for a in vals:
        for b in vals[:12]:
            assert L.orc_m31_mul(a, b) == a * b % P
            assert L.orc_m31_add(a, b) == (a + b) % P
    assert L.orc_m31_mul(P - 1, P - 1) == 1          # (-1)^2
    assert L.orc_m31_mul(1 << 16, 1 << 15) == 1       # 2^31 = 1 (mod p)


def test_hash_matches_restatement(orc):
    rng = np.random.default_rng(71)
    for s, i in zip(rng.integers(0, 1 << 32, 300, dtype=np.uint64), rng.integers(0, 1 << 20, 300)):
        assert orc.lib().orc_chash32(int(s), int(i)) == ref.chash32(int(s), int(i))
    assert orc.lib().orc_chash32(0, 0) == 0
    assert all(orc.lib().orc_chash32(s, i) < P for s in (0, 1, 0xFFFFFFFF) for i in range(64))


@pytest.mark.parametrize("n,t,count", [(5, 1, 1), (5, 1, 7), (5, 1, 100), (5, 1, 1003), (3, 1, 50),
                                       (7, 2, 200), (8, 3, 97)])
def test_oracle_matches_restatement(orc, n, t, count):
    """Bit for bit against the Python restatement, every party and one party; counts below one
    threadgroup, across partial last groups and past whole ones."""
    spr = n - 2 * t
    seeds = np.random.default_rng(72 + count).integers(0, 1 << 32, -(-count // spr), dtype=np.uint64).astype(np.uint32)
    a, b, c = orc.beaver32(n, t, count, seeds)
    ra, rb, rc = ref.triples(n, t, count, [int(s) for s in seeds])
    assert np.array_equal(a, np.array(ra, np.uint32)) and np.array_equal(b, np.array(rb, np.uint32))
    assert np.array_equal(c, np.array(rc, np.uint32))
    for p in (0, n - 1):
        sa, sb, sc = orc.beaver32(n, t, count, seeds, party=p)
        assert np.array_equal(sa, a[p]) and np.array_equal(sb, b[p]) and np.array_equal(sc, c[p])


@pytest.mark.parametrize("n,t", [(5, 1), (3, 1), (7, 2), (8, 3)])
def test_triples_reconstruct_to_products(orc, n, t):
    """The reference's own check (beaver.rs:3541-3566): Shamir reconstruction at 0 of the n
    parties' shares gives c = a b for every triple."""
    count = 1000
    spr = n - 2 * t
    seeds = np.random.default_rng(73).integers(0, 1 << 32, -(-count // spr), dtype=np.uint64).astype(np.uint32)
    a, b, c = orc.beaver32(n, t, count, seeds)
    for k in range(count):
        A = ref.lagrange_at_zero([int(a[p, k]) for p in range(n)], n)
        B = ref.lagrange_at_zero([int(b[p, k]) for p in range(n)], n)
        C = ref.lagrange_at_zero([int(c[p, k]) for p in range(n)], n)
        assert C == A * B % P, k


def test_randomiser_only_in_first_eight_lanes(orc):
    """The kernel's SIMD reduction: rounds in lanes 8..31 of their 32-round threadgroup get
    bt_r = 0, so their c shares equal a0 b0 for every party; lanes 0..7 get the shared sum."""
    n, t, count = 5, 1, 3 * 64
    seeds = np.random.default_rng(74).integers(1, 1 << 32, 64, dtype=np.uint64).astype(np.uint32)
    a, b, c = orc.beaver32(n, t, count, seeds)
    for r in range(64):
        ks = range(3 * r, 3 * r + 3)
        const = all(len(set(int(c[p, k]) for p in range(n))) == 1 for k in ks)
        assert const == (r % 32 >= 8), r
