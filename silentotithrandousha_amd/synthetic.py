"""Seeded synthetic GPT-OSS-shaped MoE layers (host side, numpy) for tests and the CPU leg
of the benchmark. Distributions follow the benchmark configurations: block bytes uniform
0..255 (two nibbles uniform 0..15), E8M0 scales uniform in [scale_lo, scale_hi], router
weights bf16 ~ N(0, 0.02), router bias 0, expert biases bf16-rounded ~ N(0, 0.01).
Checkpoint layout as in weights.rs:17-27 / :283-316.
"""
import numpy as np

GPT_OSS_20B = dict(H=2880, I=2880, E=32, k=4, layers=24)
GPT_OSS_120B = dict(H=2880, I=2880, E=128, k=4, layers=36)


def bf16_bits(x):
    """f32 -> bf16 bits, round to nearest even (NaN quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def bf16_round(x):
    return bf16_to_f32(bf16_bits(x))


def make_layer(H, I, E, seed, scale_lo=118, scale_hi=130, router_sigma=0.02, bias_sigma=0.01,
               router=True):
    rng = np.random.default_rng(seed)
    nbh, nbi = H // 32, I // 32
    L = dict(H=H, I=I, E=E)
    L["gu_blocks"] = rng.integers(0, 256, size=(E, 2 * I, nbh, 16), dtype=np.uint8)
    L["gu_scales"] = rng.integers(scale_lo, scale_hi + 1, size=(E, 2 * I, nbh), dtype=np.uint8)
    L["gu_bias"] = bf16_round(rng.normal(0, bias_sigma, size=(E, 2 * I)).astype(np.float32))
    L["d_blocks"] = rng.integers(0, 256, size=(E, H, nbi, 16), dtype=np.uint8)
    L["d_scales"] = rng.integers(scale_lo, scale_hi + 1, size=(E, H, nbi), dtype=np.uint8)
    L["d_bias"] = bf16_round(rng.normal(0, bias_sigma, size=(E, H)).astype(np.float32))
    if router:
        L["router_w"] = bf16_bits(rng.normal(0, router_sigma, size=(E, H)).astype(np.float32))
        L["router_b"] = np.zeros(E, np.float32)
    return L


def expert_slice(layer, e):
    """The tensors of one expert (weights.rs:283-316 per-expert split)."""
    return (layer["gu_blocks"][e], layer["gu_scales"][e], layer["gu_bias"][e],
            layer["d_blocks"][e], layer["d_scales"][e], layer["d_bias"][e])


def hidden(T, H, seed, sigma=1.0):
    return np.random.default_rng(seed).normal(0, sigma, size=(T, H)).astype(np.float32)
