"""Safetensors reader (weights.rs:103-139 ShardReader, tensor names :228-346): header parsing
against files written by this suite's writer and by the `safetensors` package (an independent
implementation of the format), and malformed files. No device needed."""
import os

import numpy as np
import pytest

from silentotithrandousha_amd import MoeError, safetensors_find
from silentotithrandousha_amd._ffi import MOE_ERR_INVALID, MOE_ERR_IO
from tests.helpers import write_safetensors


def test_find_own_writer(tmp_path):
    rng = np.random.default_rng(1)
    a = rng.integers(0, 256, size=(3, 5, 2, 16), dtype=np.uint8)
    b = rng.integers(0, 65536, size=(7, 3), dtype=np.uint16)
    c = rng.standard_normal(11).astype(np.float32)
    p = tmp_path / "x.safetensors"
    write_safetensors(p, {"blocks": ("U8", a, a.shape), "bias": ("BF16", b, b.shape), "f": ("F32", c, c.shape)},
                      metadata={"format": "pt"}, pad=5)
    raw = p.read_bytes()
    for name, arr, dt in (("blocks", a, "U8"), ("bias", b, "BF16"), ("f", c, "F32")):
        got_dt, shape, (beg, end) = safetensors_find(str(p), name)
        assert got_dt == dt and shape == arr.shape
        assert raw[beg:end] == arr.tobytes()


def test_find_package_writer(tmp_path):
    """Files written by the safetensors package (its own header layout and alignment)."""
    st = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(2)
    t = {"model.layers.0.mlp.experts.down_proj_blocks": rng.integers(0, 256, size=(2, 64, 2, 16), dtype=np.uint8),
         "model.layers.0.mlp.experts.down_proj_scales": rng.integers(118, 131, size=(2, 64, 2), dtype=np.uint8),
         "w": rng.standard_normal((4, 6)).astype(np.float32)}
    p = tmp_path / "pkg.safetensors"
    st.save_file(t, str(p), metadata={"note": "x"})
    raw = p.read_bytes()
    for name, arr in t.items():
        dt, shape, (beg, end) = safetensors_find(str(p), name)
        assert dt == {np.uint8: "U8", np.float32: "F32"}[arr.dtype.type] and shape == arr.shape
        assert raw[beg:end] == arr.tobytes()


@pytest.mark.parametrize("case", ["missing_file", "short", "header_past_end", "bad_json", "range_past_end",
                                  "float_shape", "missing_tensor", "wrapping_offsets"])
def test_malformed(tmp_path, case):
    p = tmp_path / "bad.safetensors"
    good = {"t": ("U8", np.zeros(16, np.uint8), (16,))}
    if case == "missing_file":
        p = tmp_path / "none.safetensors"
    elif case == "short":
        p.write_bytes(b"\x01\x00")
    elif case == "header_past_end":
        p.write_bytes((1000).to_bytes(8, "little") + b"{}")
    elif case == "bad_json":
        h = b'{"t": {"dtype": "U8", "shape": [16], "data_offsets": [0, 16]'  # unterminated
        p.write_bytes(len(h).to_bytes(8, "little") + h + bytes(16))
    elif case == "range_past_end":
        h = b'{"t": {"dtype": "U8", "shape": [64], "data_offsets": [0, 64]}}'
        p.write_bytes(len(h).to_bytes(8, "little") + h + bytes(16))
    elif case == "wrapping_offsets":
        # end = data0 + o1 wraps to 16 (inside the file) while begin = data0 + o0 stays near
        # 2^64: end - begin is the right byte count for a 32-byte tensor, so only an overflow
        # check on the offsets themselves refuses it
        tmpl = '{"t": {"dtype": "U8", "shape": [32], "data_offsets": [%d, %d]}}'
        n = len(tmpl % (2**64 - 1, 2**64 - 1))  # both offsets have 20 digits
        data0 = 8 + n
        o1 = 2**64 - data0 + 16
        h = (tmpl % (o1 - 32, o1)).encode()
        assert len(h) == n
        p.write_bytes(len(h).to_bytes(8, "little") + h + bytes(64))
    elif case == "float_shape":
        h = b'{"t": {"dtype": "U8", "shape": [1.5], "data_offsets": [0, 16]}}'
        p.write_bytes(len(h).to_bytes(8, "little") + h + bytes(16))
    else:
        write_safetensors(p, good)
    name = "absent" if case == "missing_tensor" else "t"
    with pytest.raises(MoeError) as e:
        safetensors_find(str(p), name)
    want = MOE_ERR_INVALID if case == "missing_tensor" else MOE_ERR_IO
    assert e.value.code == want, str(e.value)
