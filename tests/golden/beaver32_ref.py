"""Independent restatement of the reference's 32-bit Beaver-triple kernels
(src/gpu/shader32.metal:4-167, dispatched by src/gpu/mod.rs:975-1000) in Python integers, used
only to pin the C oracle. Written from the shader's arithmetic: field products and sums as
integers mod p = 2^31 - 1, the hash with explicit 32-bit wrap-around, and the SIMD reduction of
bt_r in closed form (the first 8 rounds of every threadgroup of min(32, rounds) rounds receive the
HIM-weighted sum of the hashes of the threadgroup's first n rounds; other rounds receive 0)."""

P = (1 << 31) - 1
M32 = 0xFFFFFFFF


def chash32(seed, idx):
    x = (seed ^ ((idx * 0x9E3779B9) & M32)) & M32
    x ^= x >> 16
    x = (x * 0x85EBCA6B) & M32
    x ^= x >> 13
    x = (x * 0xC2B2AE35) & M32
    x ^= x >> 16
    x &= 0x7FFFFFFF
    return x - P if x >= P else x


def triples(n, t, count, seeds, party=None):
    """Returns lists a, b, c: [count] for one party, or [n][count] for every party."""
    spr = n - 2 * t
    rounds = -(-count // spr)
    w = min(32, rounds)
    parties = [party] if party is not None else list(range(n))
    out = {p: ([0] * count, [0] * count, [0] * count) for p in parties}
    for k in range(count):
        r, j = divmod(k, spr)
        lane = r % w
        bt = 0
        if lane < 8:
            r0 = r - lane
            for i in range(n):
                if r0 + i < rounds:
                    bt += pow(i + 1, j, P) * chash32(seeds[r0 + i], 3 * i)
        bt %= P
        s = seeds[r]
        a0 = chash32(s, 3 * n + 2 * spr + 2 * j)
        b0 = chash32(s, 3 * n + 2 * spr + 2 * j + 1)
        ca = chash32(s, 3 * n + 2 * j)
        cb = chash32(s, 3 * n + 2 * j + 1)
        for p in parties:
            x = p + 1
            out[p][0][k] = (a0 + ca * x) % P
            out[p][1][k] = (b0 + cb * x) % P
            out[p][2][k] = (a0 * b0 + x * bt) % P
    if party is not None:
        return out[party]
    return tuple([out[p][q] for p in parties] for q in range(3))


def lagrange_at_zero(values, n):
    """Shamir reconstruction at 0 from the shares of parties 1..n (eval points 1..n)."""
    acc = 0
    for p in range(n):
        xp = p + 1
        num, den = 1, 1
        for q in range(n):
            if q != p:
                num = num * (-(q + 1)) % P
                den = den * (xp - (q + 1)) % P
        acc += values[p] * num * pow(den, P - 2, P)
    return acc % P
