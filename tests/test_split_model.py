"""Float64 model of the grouped GEMM's activation split (3 E2M3 terms per 32-value block, term t
at scale 2^(E - 2 - 5t) with the block maximum in [2^(E-1), 2^E)) and of the layer error it
causes; the evidence for the number of terms. The E2M3 rounding is pinned by its definition
(every representable value maps to itself, ties go to even codes, saturation at 7.5).

Run as a script for the GPT-OSS-20B shape (python -m tests.test_split_model [tokens]): it prints
the layer-output relative L2 of 3 and 2 terms on the benchmark's synthetic layer distribution."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import np_ref  # noqa: E402
from silentotithrandousha_amd import synthetic as syn  # noqa: E402


def q_e2m3(v):
    """Round to nearest even on the E2M3 grid (steps 1/8 below 2, 1/4 in [2, 4), 1/2 in [4, 8)),
    saturating at 7.5."""
    a = np.abs(v)
    e = np.floor(np.log2(np.maximum(a, 1e-300)))
    step = np.where(a < 1.0, 0.125, 2.0 ** (e - 3))
    q = np.minimum(np.round(a / step) * step, 7.5)  # numpy rounds half to even
    return np.sign(v) * q


def split(x, terms):
    """Sum of the first `terms` E2M3 terms of x, blocks of 32 along the last axis."""
    xb = np.asarray(x, np.float64).reshape(-1, 32)
    m = np.abs(xb).max(axis=1, keepdims=True)
    E = np.where(m > 0, np.floor(np.log2(np.maximum(m, 1e-300))) + 1, 0)
    r, out = xb.copy(), np.zeros_like(xb)
    for t in range(terms):
        sc = 2.0 ** (E - 2 - 5 * t)
        q = q_e2m3(r / sc) * sc
        out += q
        r = r - q
    return out.reshape(np.shape(x))


def layer(x, L, k, terms=None):
    """The MoE layer in float64 with x and h replaced by their `terms`-term splits (None: exact)."""
    x = np.asarray(x, np.float64)
    logits = np_ref.router_logits(L["router_w"], L["router_b"], x)
    idx, w = np_ref.topk(logits, k)
    xin = split(x, terms) if terms else x
    y = np.zeros_like(x)
    for e in range(L["E"]):
        sel = np.argwhere(idx == e)
        if not len(sel):
            continue
        t = sel[:, 0]
        gu = xin[t] @ np_ref.decode(L["gu_blocks"][e], L["gu_scales"][e]).T + L["gu_bias"][e]
        gate, up = np.minimum(gu[:, 0::2], 7.0), np.clip(gu[:, 1::2], -7, 7)
        with np.errstate(over="ignore"):
            h = (up + 1) * gate / (1 + np.exp(-1.702 * gate))
        if terms:
            h = split(h, terms)
        o = np.clip(h @ np_ref.decode(L["d_blocks"][e], L["d_scales"][e]).T + L["d_bias"][e], -65504, 65504)
        y[t] += w[sel[:, 0], sel[:, 1]][:, None] * o
    return y


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_e2m3_rounding_rules():
    grid = np.array([0, .125, .25, .375, .5, .625, .75, .875, 1, 1.125, 1.25, 1.375, 1.5, 1.625, 1.75,
                     1.875, 2, 2.25, 2.5, 2.75, 3, 3.25, 3.5, 3.75, 4, 4.5, 5, 5.5, 6, 6.5, 7, 7.5])
    assert np.array_equal(q_e2m3(grid), grid) and np.array_equal(q_e2m3(-grid), -grid)
    assert q_e2m3(np.array([0.0625]))[0] == 0.0       # tie -> even code (0)
    assert q_e2m3(np.array([0.1875]))[0] == 0.25      # tie between .125 (odd) and .25 (even)
    assert q_e2m3(np.array([2.125]))[0] == 2.0 and q_e2m3(np.array([2.375]))[0] == 2.5
    assert q_e2m3(np.array([7.74, 100.0]))[1] == 7.5 and q_e2m3(np.array([7.74]))[0] == 7.5


def test_split_error_bound():
    """The last term leaves at most half a step of its top binade: term t has scale 2^(E-2-5t)
    and its input residual stays below 4 of it (values in [2, 4) step 1/4), so |x - sum| <=
    2^(E-15) <= 2^-14 max|block|
    for 3 terms and 2^(E-10) <= 2^-9 max|block| for 2, with a block maximum in [2^(E-1), 2^E)."""
    x = np.random.default_rng(3).normal(0, 1, (256, 32)) * np.exp(np.random.default_rng(4).normal(0, 2, (256, 1)))
    m = np.abs(x).max(axis=1, keepdims=True)
    for terms, lim in ((3, 2.0 ** -14), (2, 2.0 ** -9)):
        assert np.all(np.abs(x - split(x, terms)) <= lim * m)
    assert np.max(np.abs(x - split(x, 2)) / m) > 2.0 ** -12   # 2 terms are 32x coarser


def test_layer_error_three_terms_within_tolerance_two_not():
    """At a test-sized layer of the benchmark's distribution (uniform nibbles, scales 2^-9..2^3,
    so gate/up pre-activations far beyond the SwiGLU clamp of 7) 3 terms stay well inside the
    1e-3 tolerance and 2 terms do not."""
    L = syn.make_layer(256, 128, 8, seed=30)
    x = syn.hidden(24, 256, seed=31).astype(np.float64)
    ref = layer(x, L, 4)
    e3, e2 = rel(layer(x, L, 4, 3), ref), rel(layer(x, L, 4, 2), ref)
    assert e3 < 3e-4, e3
    assert e2 > 1e-3, e2


if __name__ == "__main__":
    T = int(sys.argv[1]) if len(sys.argv) > 1 else 16
    L = syn.make_layer(2880, 2880, 32, seed=20)
    x = syn.hidden(T, 2880, seed=450).astype(np.float64)
    ref = layer(x, L, 4)
    for terms in (3, 2):
        print(f"{terms} E2M3 terms: layer-output relative L2 {rel(layer(x, L, 4, terms), ref):.3e}")
