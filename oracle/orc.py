"""ctypes front end of the CPU oracle (oracle/liborc.so) — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
as the checker or as the timed CPU baseline. The product library never loads it.
The C sources cite the reference lines each function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liborc.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t


class Adaptive(ctypes.Structure):
    """orc_adaptive: the GPT_OSS_ADAPTIVE_* settings of session.rs:168-201."""
    _fields_ = [("enabled", ctypes.c_int), ("min_k", ctypes.c_size_t),
                ("top1_min_prob", ctypes.c_float), ("top1_min_margin", ctypes.c_float),
                ("top2_min_mass", ctypes.c_float)]


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    L.orc_dequant_mxfp4_row.argtypes = [_u8p, _u8p, _sz, _f32p]
    L.orc_dequant_mxfp4_matrix.argtypes = [_u8p, _u8p, _sz, _sz, _f32p]
    L.orc_dequant_gate_up_reordered.argtypes = [_u8p, _u8p, _sz, _sz, _f32p]
    L.orc_f16_mul_scalar.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
    L.orc_f16_mul_scalar.restype = ctypes.c_uint16
    L.orc_dequant_mxfp4_row_f16.argtypes = [_u8p, _u8p, _sz, _u16p]
    L.orc_dequant_gate_up_reordered_f16.argtypes = [_u8p, _u8p, _sz, _sz, _u16p]
    L.orc_dequant_down_f16.argtypes = [_u8p, _u8p, _sz, _sz, _u16p]
    L.orc_f32_to_f16_rne.argtypes = [ctypes.c_float]
    L.orc_f32_to_f16_rne.restype = ctypes.c_uint16
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_f32_to_bf16_rne.argtypes = [ctypes.c_float]
    L.orc_f32_to_bf16_rne.restype = ctypes.c_uint16
    L.orc_expert_ffn_f32.argtypes = [_f32p, _sz, _u8p, _u8p, _f32p, _u8p, _u8p, _f32p, _sz, _sz,
                                     ctypes.c_float, _f32p, ctypes.c_void_p]
    L.orc_mxfp4_matvec_f32.argtypes = [_u8p, _u8p, _sz, _sz, _f32p, _f32p]
    L.orc_router_logits.argtypes = [_u16p, _f32p, _f32p, _sz, _sz, _sz, _f32p]
    L.orc_router_logits_seq.argtypes = [_u16p, _f32p, _f32p, _sz, _sz, _sz, _f32p]
    L.orc_topk.argtypes = [_f32p, _sz, _sz, _sz, ctypes.c_void_p, _i32p, _f32p, ctypes.c_void_p,
                           ctypes.c_void_p]
    L.orc_moe_layer_f32.argtypes = [_f32p, _sz, _sz, _sz, _sz, _sz, ctypes.c_float, _u16p, _f32p,
                                    _u8p, _u8p, _f32p, _u8p, _u8p, _f32p, ctypes.c_void_p, _f32p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    L.orc_moe_layer_mxfp6.argtypes = L.orc_moe_layer_f32.argtypes
    L.orc_quant_mxfp6.argtypes = [_f32p, _sz, _sz, _f32p]
    L.orc_expert_ffn_mxfp6.argtypes = L.orc_expert_ffn_f32.argtypes
    L.orc_combine.argtypes = [_f32p, _f32p, _sz, _sz, ctypes.c_int, _f32p]
    L.orc_rms_inv.argtypes = [_f32p, _sz, ctypes.c_float]
    L.orc_rms_inv.restype = ctypes.c_float
    L.orc_rms_norm.argtypes = [_f32p, _sz, _sz, _f32p, ctypes.c_float, _f32p]
    L.orc_moe_block_f32.argtypes = [_f32p, _sz, _sz, _sz, _sz, _sz, ctypes.c_float, _f32p, ctypes.c_float,
                                    _u16p, _f32p, _u8p, _u8p, _f32p, _u8p, _u8p, _f32p, ctypes.c_void_p, _f32p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    L.orc_matvec_f16xf32.argtypes = [_u16p, _f32p, _f32p, _sz, _sz]
    L.orc_live_moe_token.argtypes = [_f32p, _sz, _sz, _sz, _i32p, _f32p, _u8p, _u8p, _f32p, _u8p,
                                     _u8p, _f32p, ctypes.c_int, _f32p]
    L.orc_live_moe_token.restype = ctypes.c_int
    L.orc_live_expert_f16.argtypes = [_u8p, _u8p, _f32p, _u8p, _u8p, _f32p, _sz, _sz, _u16p, _u16p,
                                      _u16p, _u16p]
    L.orc_live_moe_token_warm.argtypes = [_f32p, _sz, _sz, _sz, _f32p, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_int, _f32p]
    L.orc_live_moe_token_warm.restype = ctypes.c_int
    L.orc_omp_max_threads.restype = ctypes.c_int
    L.orc_lm_head_bf16.argtypes = [_u16p, _f32p, _sz, _sz, _f32p]
    _u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
    L.orc_m31_mul.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    L.orc_m31_mul.restype = ctypes.c_uint32
    L.orc_m31_add.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    L.orc_m31_add.restype = ctypes.c_uint32
    L.orc_chash32.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    L.orc_chash32.restype = ctypes.c_uint32
    L.orc_beaver32.argtypes = [_sz, _sz, ctypes.c_long, _sz, _u32p, _u32p, _u32p, _u32p]
    _lib = L
    return L


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def dequant_mxfp4(blocks, scales, rows, cols):
    """weights.rs:350-423: checkpoint-layout MXFP4 -> f32 [rows, cols]."""
    out = np.empty((rows, cols), np.float32)
    lib().orc_dequant_mxfp4_matrix(_c(blocks, np.uint8).reshape(-1), _c(scales, np.uint8).reshape(-1),
                                   rows, cols, out.reshape(-1))
    return out


def dequant_mxfp4_row(blocks, scales):
    nb = len(scales)
    out = np.empty(nb * 32, np.float32)
    lib().orc_dequant_mxfp4_row(_c(blocks, np.uint8).reshape(-1), _c(scales, np.uint8).reshape(-1),
                                nb, out)
    return out


def dequant_mxfp4_row_f16(blocks, scales):
    nb = len(scales)
    out = np.empty(nb * 32, np.uint16)
    lib().orc_dequant_mxfp4_row_f16(_c(blocks, np.uint8).reshape(-1),
                                    _c(scales, np.uint8).reshape(-1), nb, out)
    return out


def mxfp4_matvec(blocks, scales, rows, cols, x):
    y = np.empty(rows, np.float32)
    lib().orc_mxfp4_matvec_f32(_c(blocks, np.uint8).reshape(-1), _c(scales, np.uint8).reshape(-1),
                               rows, cols, _c(x, np.float32).reshape(-1), y)
    return y


def expert_ffn(x, gu_blocks, gu_scales, gu_bias, d_blocks, d_scales, d_bias, H, I, limit=7.0,
               want_h=False, mxfp6=False):
    """session.rs:87-124 on f32 weights; mxfp6: x and h as their MXFP6 values (quant_mxfp6)."""
    x = _c(x, np.float32).reshape(-1, H)
    T = x.shape[0]
    y = np.empty((T, H), np.float32)
    h = np.empty((T, I), np.float32) if want_h else None
    (lib().orc_expert_ffn_mxfp6 if mxfp6 else lib().orc_expert_ffn_f32)(x.reshape(-1), T, _c(gu_blocks, np.uint8).reshape(-1),
                             _c(gu_scales, np.uint8).reshape(-1), _c(gu_bias, np.float32).reshape(-1),
                             _c(d_blocks, np.uint8).reshape(-1), _c(d_scales, np.uint8).reshape(-1),
                             _c(d_bias, np.float32).reshape(-1), H, I, limit, y.reshape(-1),
                             _ptr(h))
    return (y, h) if want_h else y


def router_logits(w_bf16, bias, x, E, H, sequential=False):
    x = _c(x, np.float32).reshape(-1, H)
    T = x.shape[0]
    out = np.empty((T, E), np.float32)
    f = lib().orc_router_logits_seq if sequential else lib().orc_router_logits
    f(_c(w_bf16, np.uint16).reshape(-1), _c(bias, np.float32).reshape(-1), x.reshape(-1), T, E, H,
      out.reshape(-1))
    return out


def topk(logits, k, adaptive=None):
    logits = _c(logits, np.float32)
    T, E = logits.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    probs = np.empty((T, E), np.float32)
    kused = np.empty(T, np.int32)
    ad = ctypes.byref(adaptive) if adaptive is not None else None
    lib().orc_topk(logits.reshape(-1), T, E, k, ad, idx.reshape(-1), w.reshape(-1), _ptr(probs),
                   _ptr(kused))
    return idx, w, probs, kused


def quant_mxfp6(x):
    """MXFP6 values of x's rows in blocks of 32 (OCP MX scale 2^(floor(log2 amax) - 2), E2M3
    round to nearest even, saturation at 7.5; a block with a non-finite value -> NaN)."""
    x = _c(x, np.float32)
    cols = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_quant_mxfp6(x.reshape(-1), x.size // cols, cols, out.reshape(-1))
    return out


def moe_layer_mxfp6(x, layer, k, limit=7.0, adaptive=None):
    """moe_layer with each expert's x and SwiGLU output h as their MXFP6 values (the GPU's
    quantized-activation mode); routing on the unquantized x."""
    return moe_layer(x, layer, k, limit, adaptive, _fn="orc_moe_layer_mxfp6")


def moe_layer(x, layer, k, limit=7.0, adaptive=None, _fn="orc_moe_layer_f32"):
    """session.rs:818-980 MoE block on the fp32 path. `layer` is a dict of checkpoint tensors."""
    H = layer["H"]
    I = layer["I"]
    E = layer["E"]
    x = _c(x, np.float32).reshape(-1, H)
    T = x.shape[0]
    y = np.empty((T, H), np.float32)
    logits = np.empty((T, E), np.float32)
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    ad = ctypes.byref(adaptive) if adaptive is not None else None
    getattr(lib(), _fn)(x.reshape(-1), T, H, I, E, k, limit, _c(layer["router_w"], np.uint16).reshape(-1),
                            _c(layer["router_b"], np.float32).reshape(-1),
                            _c(layer["gu_blocks"], np.uint8).reshape(-1),
                            _c(layer["gu_scales"], np.uint8).reshape(-1),
                            _c(layer["gu_bias"], np.float32).reshape(-1),
                            _c(layer["d_blocks"], np.uint8).reshape(-1),
                            _c(layer["d_scales"], np.uint8).reshape(-1),
                            _c(layer["d_bias"], np.float32).reshape(-1), ad, y.reshape(-1),
                            _ptr(logits), _ptr(idx), _ptr(w))
    return y, logits, idx, w


def rms_inv(x, eps=1e-5):
    """1 / sqrt(mean(x^2) + eps) in the canonical lane-butterfly order (session.rs:483-487)."""
    x = _c(x, np.float32).reshape(-1)
    return lib().orc_rms_inv(x, x.size, eps)


def rms_norm(x, gamma, eps=1e-5):
    """session.rs:483-493: (x * inv_rms) * gamma per row."""
    gamma = _c(gamma, np.float32)
    H = gamma.size
    x = _c(x, np.float32).reshape(-1, H)
    n = np.empty_like(x)
    lib().orc_rms_norm(x.reshape(-1), x.shape[0], H, gamma, eps, n.reshape(-1))
    return n


def moe_block(x, layer, k, gamma, eps=1e-5, limit=7.0, adaptive=None):
    """x + MoE(RMSNorm(x) * gamma): the norm and residual around the path (executables.rs:260-317,
    session.rs:483-493, 982-994). Returns (out, logits, idx, w)."""
    H, I, E = layer["H"], layer["I"], layer["E"]
    x = _c(x, np.float32).reshape(-1, H)
    T = x.shape[0]
    out = np.empty((T, H), np.float32)
    logits = np.empty((T, E), np.float32)
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    ad = ctypes.byref(adaptive) if adaptive is not None else None
    lib().orc_moe_block_f32(x.reshape(-1), T, H, I, E, k, limit, _c(gamma, np.float32), eps,
                            _c(layer["router_w"], np.uint16).reshape(-1), _c(layer["router_b"], np.float32).reshape(-1),
                            _c(layer["gu_blocks"], np.uint8).reshape(-1), _c(layer["gu_scales"], np.uint8).reshape(-1),
                            _c(layer["gu_bias"], np.float32).reshape(-1), _c(layer["d_blocks"], np.uint8).reshape(-1),
                            _c(layer["d_scales"], np.uint8).reshape(-1), _c(layer["d_bias"], np.float32).reshape(-1),
                            ad, out.reshape(-1), _ptr(logits), _ptr(idx), _ptr(w))
    return out, logits, idx, w


def combine(outs, w, skip_nonfinite=False):
    outs = _c(outs, np.float32)
    n, H = outs.shape
    y = np.empty(H, np.float32)
    lib().orc_combine(outs.reshape(-1), _c(w, np.float32), n, H, int(skip_nonfinite), y)
    return y


def matvec_f16xf32(a_f16, x, rows, cols):
    y = np.empty(rows, np.float32)
    lib().orc_matvec_f16xf32(_c(a_f16, np.uint16).reshape(-1), _c(x, np.float32).reshape(-1), y,
                             rows, cols)
    return y


def live_moe_token(x, layer, idx, w, n_threads):
    """One token through the reference's live CPU MoE block (cold expert cache)."""
    H = layer["H"]
    I = layer["I"]
    y = np.empty(H, np.float32)
    rc = lib().orc_live_moe_token(_c(x, np.float32).reshape(-1), H, I, len(idx), _c(idx, np.int32),
                                  _c(w, np.float32), _c(layer["gu_blocks"], np.uint8).reshape(-1),
                                  _c(layer["gu_scales"], np.uint8).reshape(-1),
                                  _c(layer["gu_bias"], np.float32).reshape(-1),
                                  _c(layer["d_blocks"], np.uint8).reshape(-1),
                                  _c(layer["d_scales"], np.uint8).reshape(-1),
                                  _c(layer["d_bias"], np.float32).reshape(-1), n_threads, y)
    assert rc == 0
    return y


def live_expert_f16(layer, e):
    """The fp16 expert-cache entry of expert e (session.rs:875-899): (gu, gu_bias, down,
    down_bias) as uint16 arrays, gate/up de-interleaved."""
    H, I = layer["H"], layer["I"]
    gu = np.empty(2 * I * H, np.uint16)
    gub = np.empty(2 * I, np.uint16)
    d = np.empty(H * I, np.uint16)
    db = np.empty(H, np.uint16)
    lib().orc_live_expert_f16(_c(layer["gu_blocks"][e], np.uint8).reshape(-1),
                              _c(layer["gu_scales"][e], np.uint8).reshape(-1),
                              _c(layer["gu_bias"][e], np.float32).reshape(-1),
                              _c(layer["d_blocks"][e], np.uint8).reshape(-1),
                              _c(layer["d_scales"][e], np.uint8).reshape(-1),
                              _c(layer["d_bias"][e], np.float32).reshape(-1), H, I, gu, gub, d, db)
    return gu, gub, d, db


def live_moe_token_warm(x, H, I, entries, w, n_threads):
    """One token on the live path with the selected experts' fp16 entries (from
    live_expert_f16, in slot order) already cached."""
    n = len(entries)
    ptrs = [(ctypes.c_void_p * max(n, 1))(*[ent[i].ctypes.data for ent in entries]) for i in range(4)]
    y = np.empty(H, np.float32)
    rc = lib().orc_live_moe_token_warm(_c(x, np.float32).reshape(-1), H, I, n, _c(w, np.float32),
                                       ptrs[0], ptrs[1], ptrs[2], ptrs[3], n_threads, y)
    assert rc == 0
    return y


def omp_threads():
    return int(lib().orc_omp_max_threads())


def lm_head_bf16(w_bf16, x):
    """weights.rs:73-82 lm_head_dot over every row: bf16 [V, H] bits, x [H] -> f32 [V]."""
    w = _c(w_bf16, np.uint16)
    V, H = w.shape
    y = np.empty(V, np.float32)
    lib().orc_lm_head_bf16(w.reshape(-1), _c(x, np.float32).reshape(-1), V, H, y)
    return y


def beaver32(n, t, count, seeds, party=-1):
    """shader32.metal's triple kernels as dispatched by gpu/mod.rs: party >= 0 -> (a, b, c) of
    that party [count]; party = -1 -> every party's, each [n, count]."""
    spr = n - 2 * t
    seeds = _c(seeds, np.uint32)
    assert seeds.size >= (count + spr - 1) // spr
    shape = (count,) if party >= 0 else (n, count)
    a, b, c = (np.empty(shape, np.uint32) for _ in range(3))
    lib().orc_beaver32(n, spr, party, count, seeds, a.reshape(-1), b.reshape(-1), c.reshape(-1))
    return a, b, c
