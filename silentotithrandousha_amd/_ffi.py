"""ctypes binding of libmxfp4moe.so (the C ABI declared in include/mxfp4_moe.h).

The library is the product path; there is no fallback. If it is missing this module raises,
so nothing can silently run without the HIP kernels.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmxfp4moe.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "mxfp4_moe.h")
# every header of the library's C ABI: the MoE path and the Beaver-triple generator
HEADER_PATHS = [HEADER_PATH, os.path.join(os.path.dirname(_HERE), "include", "beaver32.h")]

MOE_OK = 0
MOE_ERR_INVALID = 1
MOE_ERR_STATE = 2
MOE_ERR_HIP = 3
MOE_ERR_NO_DEVICE = 4
MOE_ERR_OOM = 5
MOE_ERR_IO = 6

MOE_OPT_FUSED_DECODE = 1
MOE_OPT_SPIN_LIMIT = 2
MOE_OPT_BATCH_GEMM = 3
MOE_OPT_GEMM_SHAPE = 4
MOE_OPT_GEMM_BAND = 5
MOE_OPT_MATVEC = 6
MOE_OPT_GEMM_SHAPE_DOWN = 7
MOE_OPT_ACT_QUANT = 8
MOE_OPT_LOCAL_GROUP = 9

_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_int = ctypes.c_int
_f = ctypes.c_float


class MoeError(RuntimeError):
    """A non-zero status from the C ABI, with moe_last_error()'s message."""

    def __init__(self, code, msg):
        super().__init__(f"mxfp4_moe error {code}: {msg}")
        self.code = code


class ExpertRef(ctypes.Structure):
    """moe_expert_ref: one tuple of dispatch_experts_batched (moe_dispatch.rs:476)."""
    _fields_ = [("expert_idx", _sz), ("weight", _f),
                ("gate_up_blocks", _vp), ("gate_up_blocks_len", _sz),
                ("gate_up_scales", _vp), ("gate_up_scales_len", _sz),
                ("gate_up_bias", _vp), ("gate_up_bias_len", _sz),
                ("down_blocks", _vp), ("down_blocks_len", _sz),
                ("down_scales", _vp), ("down_scales_len", _sz),
                ("down_bias", _vp), ("down_bias_len", _sz)]


# name -> (restype, argtypes)
SIGNATURES = {
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_version": (ctypes.c_char_p, []),
    "moe_create": (_int, [_sz, _sz, _f, ctypes.POINTER(_vp)]),
    "moe_destroy": (None, [_vp]),
    "moe_set_adaptive_topk": (_int, [_vp, _int, _sz, _f, _f, _f]),
    "moe_set_option": (_int, [_vp, _int, ctypes.c_int64]),
    "moe_preload_layer": (_int, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
    "moe_preload_layer_device": (_int, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "moe_preload_expert": (_int, [_vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz,
                                  _vp, _sz, _vp, _sz]),
    "moe_preload_router": (_int, [_vp, _sz, _sz, _vp, _vp]),
    "moe_preload_router_f32": (_int, [_vp, _sz, _sz, _vp, _vp]),
    "moe_load_safetensors_layer": (_int, [_vp, ctypes.POINTER(ctypes.c_char_p), _sz, _sz, _sz, _f]),
    "moe_preload_norm": (_int, [_vp, _sz, _vp, _f]),
    "moe_block_forward": (_int, [_vp, _sz, _vp, _sz, _sz, _vp]),
    "moe_block_forward_device": (_int, [_vp, _sz, _vp, _sz, _sz, _vp, _vp]),
    "moe_safetensors_find": (_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _sz,
                                    ctypes.POINTER(ctypes.c_uint64), _sz, ctypes.POINTER(_sz),
                                    ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "moe_dispatch_expert_preloaded": (_int, [_vp, _vp, _sz, _sz, _vp]),
    "moe_dispatch_expert": (_int, [_vp, _vp, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz,
                                   _vp, _sz, _vp]),
    "moe_dispatch_experts_batched": (_int, [_vp, _vp, _sz, _vp, _vp]),
    "moe_init_lm_head": (_int, [_vp, _vp, _sz]),
    "moe_init_lm_head_bf16": (_int, [_vp, _vp, _sz]),
    "moe_init_lm_head_bf16_device": (_int, [_vp, _vp, _sz, _vp]),
    "moe_dispatch_lm_head": (_int, [_vp, _vp, _sz, _vp]),
    "moe_dispatch_lm_head_device": (_int, [_vp, _vp, _sz, _vp, _vp]),
    "moe_router_topk": (_int, [_vp, _sz, _vp, _sz, _sz, _vp, _vp, _vp]),
    "moe_layer_forward": (_int, [_vp, _sz, _vp, _sz, _sz, _vp]),
    "moe_layer_forward_device": (_int, [_vp, _sz, _vp, _sz, _sz, _vp, _vp]),
    "moe_layer_forward_device_noalloc": (_int, [_vp, _sz, _vp, _sz, _sz, _vp, _vp]),
    "moe_mxfp4_dequant_device": (_int, [_vp, _vp, _sz, _sz, _vp, _vp]),
    "moe_dequant_expert_device": (_int, [_vp, _sz, _sz, _int, _vp, _vp]),
    "moe_mxfp4_packed_size": (_sz, [_sz, _sz]),
    "moe_mxfp4_pack_device": (_int, [_vp, _vp, _sz, _sz, _vp, _vp]),
    "moe_mxfp4_matvec_device": (_int, [_vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    "moe_device_alloc": (_int, [_sz, ctypes.POINTER(_vp)]),
    "moe_device_free": (_int, [_vp]),
    "moe_memcpy_h2d": (_int, [_vp, _vp, _sz]),
    "moe_memcpy_d2h": (_int, [_vp, _vp, _sz]),
    "moe_memcpy_d2d": (_int, [_vp, _vp, _sz]),
    "moe_memset_device": (_int, [_vp, _int, _sz]),
    "moe_synchronize": (_int, [_vp]),
    "moe_stream": (_vp, [_vp]),
    "moe_synth_fill_device": (_int, [_vp, _sz, _int, ctypes.c_uint64, _f, _f, _vp]),
    "moe_graph_begin": (_int, [_vp]),
    "moe_graph_end": (_int, [_vp, ctypes.POINTER(_vp)]),
    "moe_graph_launch": (_int, [_vp, _vp]),
    "moe_graph_destroy": (_int, [_vp]),
    "moe_set_timing": (_int, [_vp, _int]),
    "moe_get_timing": (_int, [_vp, _int, ctypes.POINTER(ctypes.c_double),
                              ctypes.POINTER(ctypes.c_uint64)]),
    "moe_reset_timing": (_int, [_vp]),
    # include/beaver32.h
    "beaver32_create": (_int, [_sz, _sz, ctypes.POINTER(_vp)]),
    "beaver32_destroy": (None, [_vp]),
    "beaver32_spr": (_sz, [_vp]),
    "beaver32_generate": (_int, [_vp, _sz, _vp, _vp, _vp, _vp, _vp]),
    "beaver32_generate_single_party": (_int, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp]),
    "beaver32_generate_device": (_int, [_vp, ctypes.c_long, _sz, _vp, _vp, _vp, _vp, _vp]),
    "beaver32_synchronize": (_int, [_vp]),
}

_lib = None


def lib():
    """Load libmxfp4moe.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                          "(make -C silentotithrandousha_amd); there is no fallback path")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc):
    if rc != MOE_OK:
        raise MoeError(rc, lib().moe_last_error().decode())
    return rc
