"""Shared comparison helpers for the parity tests."""
import numpy as np

CANON_NAN = 0x7FC00000


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bit_exact(got, want, what):
    g, w = bits(got).ravel(), bits(want).ravel()
    bad = np.nonzero(g != w)[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[0]}: "
                           f"got {g[bad[0]]:#010x} want {w[bad[0]]:#010x}")


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


# Tolerance stated by the benchmark contract for matmul outputs: 1e-3 relative L2 against
# the fp32 reference path on the same inputs.
REL_L2_TOL = 1e-3


def assert_rel_l2(got, want, what, tol=REL_L2_TOL):
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN pattern differs"
    fin = ~np.isnan(want)
    e = rel_l2(np.asarray(got)[fin], np.asarray(want)[fin])
    assert e < tol, f"{what}: relative L2 {e:.3e} >= {tol}"
    return e


def write_safetensors(path, tensors, metadata=None, pad=0):
    """Minimal safetensors writer (u64 LE header length, JSON header, data): `tensors` maps a
    name to (dtype string, numpy array whose bytes are the tensor's, shape). Tensors are laid
    out in name order; `pad` spaces after the JSON exercise header padding."""
    import json
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name in sorted(tensors):
        dt, arr, shape = tensors[name]
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode() + b" " * pad
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def gpt_oss_layer_tensors(layer, li):
    """The checkpoint tensors of one synthetic layer under GPT-OSS names (weights.rs:262-283);
    biases and router bias as BF16 (rounded), as the checkpoint stores them."""
    from silentotithrandousha_amd import synthetic as syn
    E, H, I = layer["E"], layer["H"], layer["I"]
    p = f"model.layers.{li}.mlp."
    return {
        p + "experts.gate_up_proj_blocks": ("U8", layer["gu_blocks"], (E, 2 * I, H // 32, 16)),
        p + "experts.gate_up_proj_scales": ("U8", layer["gu_scales"], (E, 2 * I, H // 32)),
        p + "experts.gate_up_proj_bias": ("BF16", syn.bf16_bits(layer["gu_bias"]), (E, 2 * I)),
        p + "experts.down_proj_blocks": ("U8", layer["d_blocks"], (E, H, I // 32, 16)),
        p + "experts.down_proj_scales": ("U8", layer["d_scales"], (E, H, I // 32)),
        p + "experts.down_proj_bias": ("BF16", syn.bf16_bits(layer["d_bias"]), (E, H)),
        p + "router.weight": ("BF16", np.asarray(layer["router_w"], np.uint16), (E, H)),
        p + "router.bias": ("BF16", syn.bf16_bits(layer["router_b"]), (E,)),
    }
