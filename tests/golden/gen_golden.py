"""Writes the committed fixtures of tests/golden/ from the independent float64 restatement
(np_ref.py). The reference repository holds no golden vectors for this path, so these
fixtures are generated here from the closed forms; run `python tests/golden/gen_golden.py`
to regenerate (the result is deterministic).

  mxfp4_decode_table.npz  every (nibble, E8M0 byte) pair: f32 bits of the reference decode
  tiny_layer.npz          one small MoE layer (H=64, I=32, E=8, k=4) and 3 tokens with the
                          float64 outputs, router logits and top-k of np_ref
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import np_ref  # noqa: E402

CANON_NAN = np.uint32(0x7FC00000)


def decode_table():
    nib = np.arange(16)
    sc = np.arange(256)
    with np.errstate(invalid="ignore", over="ignore"):  # 6 * 2^127 overflows to +inf as in f32
        v = (np_ref.e2m1_value(nib)[None, :] * np_ref.e8m0_scale(sc)[:, None]).astype(np.float32)
    bits = v.view(np.uint32).copy()
    bits[np.isnan(v)] = CANON_NAN
    return bits  # [256 scales, 16 nibbles]


def tiny_layer(seed=2024):
    rng = np.random.default_rng(seed)
    H, I, E, k = 64, 32, 8, 4
    L = dict(H=np.int64(H), I=np.int64(I), E=np.int64(E))
    L["gu_blocks"] = rng.integers(0, 256, size=(E, 2 * I, H // 32, 16), dtype=np.uint8)
    L["gu_scales"] = rng.integers(118, 124, size=(E, 2 * I, H // 32), dtype=np.uint8)
    L["gu_bias"] = rng.normal(0, 0.1, size=(E, 2 * I)).astype(np.float32)
    L["d_blocks"] = rng.integers(0, 256, size=(E, H, I // 32, 16), dtype=np.uint8)
    L["d_scales"] = rng.integers(118, 124, size=(E, H, I // 32), dtype=np.uint8)
    L["d_bias"] = rng.normal(0, 0.1, size=(E, H)).astype(np.float32)
    w = rng.normal(0, 0.2, size=(E, H)).astype(np.float32)
    L["router_w"] = ((w.view(np.uint32).astype(np.uint64) + 0x7FFF + ((w.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    L["router_b"] = rng.normal(0, 0.1, size=E).astype(np.float32)
    x = rng.normal(0, 1, size=(3, H)).astype(np.float32)
    lay = {kk: (int(v) if kk in ("H", "I", "E") else v) for kk, v in L.items()}
    y, logits, idx, wts = np_ref.moe_layer(x, lay, k)
    return dict(**L, k=np.int64(k), x=x, y=y, logits=logits, idx=idx, w=wts)


def main():
    np.savez_compressed(os.path.join(HERE, "mxfp4_decode_table.npz"), bits=decode_table())
    np.savez_compressed(os.path.join(HERE, "tiny_layer.npz"), **tiny_layer())
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
