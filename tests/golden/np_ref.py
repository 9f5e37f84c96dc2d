"""Independent float64 numpy restatement of the MoE path, used only to pin the C oracle.

Written from the mathematics rather than from the oracle's code: the E2M1 value is computed
from its sign/exponent/mantissa fields (OCP MX v1.0), the E8M0 scale as 2^(s-127) with the
reference's two departures from the spec (s = 0 decodes to +0.0 and s = 255 to +inf,
weights.rs:359 `f32::from_bits(s << 23)`), matrix products in float64, SwiGLU in float64.
"""
import numpy as np


def e2m1_value(n):
    """E2M1 nibble -> value: sign bit 3, exponent bits 2..1, mantissa bit 0."""
    n = np.asarray(n, np.int64)
    sign = np.where(n & 8, -1.0, 1.0)
    e = (n >> 1) & 3
    m = n & 1
    mag = np.where(e == 0, 0.5 * m, (2.0 ** (e - 1)) * (1.0 + 0.5 * m))
    return sign * mag


def e8m0_scale(s):
    """The reference's E8M0 decode: 2^(s-127), except 0 -> +0.0 and 255 -> +inf."""
    s = np.asarray(s, np.int64)
    v = np.ldexp(1.0, s - 127)
    v = np.where(s == 0, 0.0, v)
    return np.where(s == 255, np.inf, v)


def decode(blocks, scales):
    """blocks [R, NB, 16] u8, scales [R, NB] u8 -> float64 [R, 32 NB]; element 32b+2j is the
    low nibble of byte j of block b, element 32b+2j+1 its high nibble."""
    blocks = np.asarray(blocks, np.uint8)
    R, NB, _ = blocks.shape
    lo = e2m1_value(blocks & 0x0F)
    hi = e2m1_value(blocks >> 4)
    vals = np.stack([lo, hi], axis=-1).reshape(R, NB, 32)
    with np.errstate(invalid="ignore"):
        out = vals * e8m0_scale(scales)[:, :, None]
    return out.reshape(R, NB * 32)


def expert_ffn(x, gu_blocks, gu_scales, gu_bias, d_blocks, d_scales, d_bias, limit=7.0,
               alpha=1.702):
    """float64 expert: gate = row 2i, up = row 2i+1 of gate_up (interleaved checkpoint rows)."""
    x = np.asarray(x, np.float64).reshape(-1, np.asarray(gu_blocks).shape[1] * 32)
    Wgu = decode(gu_blocks, gu_scales)
    Wd = decode(d_blocks, d_scales)
    gu = x @ Wgu.T + np.asarray(gu_bias, np.float64)
    gate = np.minimum(gu[:, 0::2], limit)
    up = np.clip(gu[:, 1::2], -limit, limit)
    with np.errstate(over="ignore"):
        glu = gate / (1.0 + np.exp(-alpha * gate))
    h = (up + 1.0) * glu
    y = h @ Wd.T + np.asarray(d_bias, np.float64)
    return np.clip(y, -65504.0, 65504.0)


def bf16_to_f64(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)


def router_logits(w_bf16, bias, x):
    return np.asarray(x, np.float64) @ bf16_to_f64(w_bf16).T + np.asarray(bias, np.float64)


def topk(logits, k):
    """Order by logit descending, equal logits by lower index, NaN last; weights are the
    softmax over all experts renormalised over the kept ones (= softmax over kept logits)."""
    logits = np.asarray(logits, np.float64)
    T, E = logits.shape
    idx = np.empty((T, k), np.int64)
    w = np.empty((T, k), np.float64)
    for t in range(T):
        l = logits[t]
        nan = np.isnan(l)
        key = np.where(nan, -np.inf, l)
        order = np.lexsort((np.arange(E), nan, -key))  # primary: -key, then NaN flag, then idx
        idx[t] = order[:k]
        sel = l[order[:k]]
        m = np.nanmax(l) if not np.all(nan) else 0.0
        p = np.exp(sel - m)
        w[t] = p / p.sum()
    return idx, w


def moe_layer(x, layer, k, limit=7.0):
    x = np.asarray(x, np.float64).reshape(-1, layer["H"])
    logits = router_logits(layer["router_w"], layer["router_b"], x)
    idx, w = topk(logits, k)
    y = np.zeros_like(x)
    for t in range(x.shape[0]):
        for s in range(k):
            e = idx[t, s]
            out = expert_ffn(x[t], layer["gu_blocks"][e], layer["gu_scales"][e], layer["gu_bias"][e],
                             layer["d_blocks"][e], layer["d_scales"][e], layer["d_bias"][e], limit)
            y[t] += w[t, s] * out[0]
    return y, logits, idx, w


def e2m3_grid():
    """The 32 E2M3 magnitudes in code order (code = exponent bits << 3 | mantissa bits, bias 1):
    exponent 0 gives mantissa / 8, exponent e > 0 gives (1 + mantissa / 8) 2^(e - 1)."""
    c = np.arange(32)
    e, m = c >> 3, c & 7
    return np.where(e == 0, m / 8.0, (1.0 + m / 8.0) * 2.0 ** (e - 1))


def quant_mxfp6(x):
    """MXFP6 values of x (last axis in blocks of 32, a multiple of 32): per block the OCP MX scale
    2^(floor(log2 amax) - emax) with E2M3's emax = 2 (2^-3 for an all-zero block), then each
    scaled value replaced by the nearest grid magnitude, a tie going to the even code, values past
    the largest magnitude clamped to it; a block holding a non-finite value becomes NaN."""
    x = np.asarray(x, np.float64)
    xb = x.reshape(-1, 32)
    grid = e2m3_grid()
    out = np.empty_like(xb)
    for i, blk in enumerate(xb):
        if not np.all(np.isfinite(blk)):
            out[i] = np.nan
            continue
        amax = np.abs(blk).max()
        s = 2.0 ** (np.floor(np.log2(amax)) - 2) if amax > 0 else 2.0 ** -3
        s = max(s, 2.0 ** -126)
        a = np.minimum(np.abs(blk) / s, grid[-1])
        d = np.abs(a[:, None] - grid[None, :])
        best = d.min(axis=1, keepdims=True)
        cand = d == best                       # one code, or two at a tie
        code = np.where(cand[:, ::2].any(axis=1) & (cand.sum(axis=1) > 1),
                        np.argmax(cand & (np.arange(32) % 2 == 0), axis=1), np.argmax(cand, axis=1))
        out[i] = np.sign(blk) * grid[code] * s
    return out.reshape(x.shape)
