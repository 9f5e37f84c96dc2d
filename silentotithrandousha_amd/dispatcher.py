"""Python host front end over the C ABI, mirroring the reference's GpuMoeDispatcher
(src/gpu/moe_dispatch.rs:36-684) plus the path-level calls of Session::decode_step_inner's
MoE block (src/gpt_oss/session.rs:818-980).

Method names follow the Rust API; errors raise MoeError where Rust returns Err or panics.
Arrays are numpy; device buffers are DeviceBuffer objects from the library's own allocator.
"""
import ctypes

import numpy as np

from ._ffi import ExpertRef, check, lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _dp(b):
    """Device pointer of a DeviceBuffer (or an int address)."""
    return ctypes.c_void_p(b.ptr if hasattr(b, "ptr") else int(b))


class DeviceBuffer:
    """A device allocation made through moe_device_alloc (freed on close / GC)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().moe_device_alloc(self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        if arr.nbytes:
            check(lib().moe_memcpy_h2d(b.ptr, arr.ctypes.data, arr.nbytes))
        return b

    def download(self, dtype, shape):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            check(lib().moe_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib().moe_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes))

    def close(self):
        if getattr(self, "ptr", None):
            lib().moe_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuMoeDispatcher:
    """GpuMoeDispatcher::new(hidden_size, inter_size, swiglu_clamp) — moe_dispatch.rs:60."""

    def __init__(self, hidden_size, inter_size, swiglu_clamp=7.0):
        self.hidden_size = int(hidden_size)
        self.inter_size = int(inter_size)
        self.swiglu_clamp = float(swiglu_clamp)
        ctx = ctypes.c_void_p()
        check(lib().moe_create(self.hidden_size, self.inter_size, self.swiglu_clamp,
                               ctypes.byref(ctx)))
        self._ctx = ctx.value
        self.lm_vocab = 0
        self.gemm_shape = 0  # MOE_OPT_GEMM_SHAPE as last set (set_gemm_shape)

    @property
    def ctx(self):
        return self._ctx

    def close(self):
        if getattr(self, "_ctx", None):
            lib().moe_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- weights
    def preload_layer(self, layer_idx, layer):
        """One layer of preload_experts (moe_dispatch.rs:149-229) plus its router."""
        E = layer["E"]
        check(lib().moe_preload_layer(
            self._ctx, layer_idx, E, _p(_c(layer["gu_blocks"], np.uint8)),
            _p(_c(layer["gu_scales"], np.uint8)), _p(_c(layer["gu_bias"], np.float32)),
            _p(_c(layer["d_blocks"], np.uint8)), _p(_c(layer["d_scales"], np.uint8)),
            _p(_c(layer["d_bias"], np.float32))))
        if "router_w" in layer:
            check(lib().moe_preload_router(self._ctx, layer_idx, E,
                                           _p(_c(layer["router_w"], np.uint16)),
                                           _p(_c(layer["router_b"], np.float32))))

    def load_safetensors_layer(self, shards, layer_idx, n_experts, rms_norm_eps=1e-5):
        """Layer `layer_idx`'s experts and router from local safetensors shards (the reference's
        ShardReader and tensor names, weights.rs:103-139, 228-346). `shards`: a directory (every
        *.safetensors in it, sorted, as the reference sorts the shard names) or a list of paths."""
        import os
        if isinstance(shards, (str, os.PathLike)) and os.path.isdir(shards):
            shards = sorted(os.path.join(shards, f) for f in os.listdir(shards) if f.endswith(".safetensors"))
        elif isinstance(shards, (str, os.PathLike)):
            shards = [shards]
        paths = (ctypes.c_char_p * len(shards))(*[os.fsencode(p) for p in shards])
        check(lib().moe_load_safetensors_layer(self._ctx, paths, len(shards), layer_idx, n_experts, rms_norm_eps))

    def preload_norm(self, layer_idx, gamma, eps=1e-5):
        """Post-attention RMSNorm weight (weights.rs:32, 267-268) and rms_norm_eps (config.rs:42-43)."""
        check(lib().moe_preload_norm(self._ctx, layer_idx, _p(_c(gamma, np.float32)), float(eps)))

    def block_forward(self, layer_idx, x, top_k):
        """x + MoE(RMSNorm(x) gamma): the post-attention norm and residual around the path
        (executables.rs:260-317, session.rs:483-493, 982-994)."""
        x = _c(x, np.float32).reshape(-1, self.hidden_size)
        out = np.empty_like(x)
        check(lib().moe_block_forward(self._ctx, layer_idx, _p(x), x.shape[0], top_k, _p(out)))
        return out

    def preload_experts(self, layers):
        """preload_experts(&layers, &config) — all layers, index = position."""
        for i, layer in enumerate(layers):
            self.preload_layer(i, layer)

    def preload_expert(self, layer_idx, n_experts, expert_idx, gu_blocks, gu_scales, gu_bias,
                       d_blocks, d_scales, d_bias):
        """One ExpertMxfp4 (weights.rs:17-27) of preload_experts' per-expert loop."""
        t = [_c(gu_blocks, np.uint8), _c(gu_scales, np.uint8), _c(gu_bias, np.float32),
             _c(d_blocks, np.uint8), _c(d_scales, np.uint8), _c(d_bias, np.float32)]
        args = []
        for a in t:
            args += [_p(a), a.size]
        check(lib().moe_preload_expert(self._ctx, layer_idx, n_experts, expert_idx, *args))

    def set_fused_decode(self, on):
        """True / 2: one launch (default); 1: two launches; False / 0: the batch path."""
        from ._ffi import MOE_OPT_FUSED_DECODE
        mode = 2 if on is True else (0 if on is False else int(on))
        check(lib().moe_set_option(self._ctx, MOE_OPT_FUSED_DECODE, mode))

    def set_batch_gemm(self, mode):
        """1 / True: grouped GEMM for large batches (default); 2: for every batch; 0: never."""
        from ._ffi import MOE_OPT_BATCH_GEMM
        check(lib().moe_set_option(self._ctx, MOE_OPT_BATCH_GEMM, int(mode)))

    def set_gemm_shape(self, shape, down=0):
        """Grouped GEMM block shape (0 by batch size, 1..19 forced alternatives; down: the same
        codes for the down GEMM alone, 0 = as shape; tuning only)."""
        from ._ffi import MOE_OPT_GEMM_SHAPE, MOE_OPT_GEMM_SHAPE_DOWN
        check(lib().moe_set_option(self._ctx, MOE_OPT_GEMM_SHAPE, int(shape)))
        check(lib().moe_set_option(self._ctx, MOE_OPT_GEMM_SHAPE_DOWN, int(down)))
        self.gemm_shape = int(shape)

    def set_gemm_band(self, band):
        """Row blocks per band of the grouped GEMM's per-XCD tile order (0 default; tuning only)."""
        from ._ffi import MOE_OPT_GEMM_BAND
        check(lib().moe_set_option(self._ctx, MOE_OPT_GEMM_BAND, int(band)))

    def set_matvec(self, one_launch):
        """mxfp4_matvec in one launch on the block-scaled MFMA (1, default) or as split + bf16
        GEMV (0); results agree to 1e-5."""
        from ._ffi import MOE_OPT_MATVEC
        check(lib().moe_set_option(self._ctx, MOE_OPT_MATVEC, int(one_launch)))

    def set_act_quant(self, on):
        """Grouped GEMM activations: 0 / False exact to ~2^-13 of each block maximum (default);
        1 / True quantized to MXFP6 (one E2M3 value per element, OCP MX block scale), whose results
        follow the f32 path applied to the quantized activations. Other values are refused."""
        from ._ffi import MOE_OPT_ACT_QUANT
        check(lib().moe_set_option(self._ctx, MOE_OPT_ACT_QUANT, int(on)))

    def set_local_group(self, on):
        """Small batches on the streamed gate_up GEMM: its workgroups group the entries by expert
        (1, default) or the router does (0); results identical."""
        from ._ffi import MOE_OPT_LOCAL_GROUP
        check(lib().moe_set_option(self._ctx, MOE_OPT_LOCAL_GROUP, int(on)))

    def set_spin_limit(self, polls):
        from ._ffi import MOE_OPT_SPIN_LIMIT
        check(lib().moe_set_option(self._ctx, MOE_OPT_SPIN_LIMIT, int(polls)))

    def set_adaptive_topk(self, enabled, min_k=3, top1_min_prob=0.90, top1_min_margin=0.35,
                          top2_min_mass=0.98):
        check(lib().moe_set_adaptive_topk(self._ctx, int(enabled), int(min_k), top1_min_prob,
                                          top1_min_margin, top2_min_mass))

    # ---- per-expert dispatch
    def dispatch_expert_preloaded(self, x, layer, expert_idx):
        y = np.empty(self.hidden_size, np.float32)
        check(lib().moe_dispatch_expert_preloaded(self._ctx, _p(_c(x, np.float32)), layer,
                                                  expert_idx, _p(y)))
        return y

    def dispatch_expert(self, x, gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks,
                        down_scales, down_bias):
        t = [_c(gate_up_blocks, np.uint8), _c(gate_up_scales, np.uint8),
             _c(gate_up_bias, np.float32), _c(down_blocks, np.uint8), _c(down_scales, np.uint8),
             _c(down_bias, np.float32)]
        y = np.empty(self.hidden_size, np.float32)
        check(lib().moe_dispatch_expert(self._ctx, _p(_c(x, np.float32)),
                                        _p(t[0]), t[0].size, _p(t[1]), t[1].size,
                                        _p(t[2]), t[2].size, _p(t[3]), t[3].size,
                                        _p(t[4]), t[4].size, _p(t[5]), t[5].size, _p(y)))
        return y

    def dispatch_experts_batched(self, x, experts):
        """experts: list of (expert_idx, weight, gu_blocks, gu_scales, gu_bias, d_blocks,
        d_scales, d_bias) as in moe_dispatch.rs:476."""
        keep = []
        refs = (ExpertRef * max(1, len(experts)))()
        for i, (eidx, w, gb, gs, gbias, db, ds, dbias) in enumerate(experts):
            arrs = [_c(gb, np.uint8), _c(gs, np.uint8), _c(gbias, np.float32), _c(db, np.uint8),
                    _c(ds, np.uint8), _c(dbias, np.float32)]
            keep.append(arrs)
            r = refs[i]
            r.expert_idx = eidx
            r.weight = w
            r.gate_up_blocks, r.gate_up_blocks_len = arrs[0].ctypes.data, arrs[0].size
            r.gate_up_scales, r.gate_up_scales_len = arrs[1].ctypes.data, arrs[1].size
            r.gate_up_bias, r.gate_up_bias_len = arrs[2].ctypes.data, arrs[2].size
            r.down_blocks, r.down_blocks_len = arrs[3].ctypes.data, arrs[3].size
            r.down_scales, r.down_scales_len = arrs[4].ctypes.data, arrs[4].size
            r.down_bias, r.down_bias_len = arrs[5].ctypes.data, arrs[5].size
        y = np.empty(self.hidden_size, np.float32)
        check(lib().moe_dispatch_experts_batched(self._ctx, _p(_c(x, np.float32)), len(experts),
                                                 ctypes.cast(refs, ctypes.c_void_p), _p(y)))
        return y

    # ---- LM head
    def init_lm_head(self, weights, vocab_size):
        w = _c(weights, np.float32)
        check(lib().moe_init_lm_head(self._ctx, _p(w), vocab_size))
        self.lm_vocab = vocab_size

    def init_lm_head_bf16(self, weights_bf16, vocab_size):
        """The checkpoint's BF16 lm_head.weight as bf16 bits [vocab, H] (weights.rs:56, 251;
        lm_head_dot weights.rs:73-82)."""
        w = _c(weights_bf16, np.uint16)
        check(lib().moe_init_lm_head_bf16(self._ctx, _p(w), vocab_size))
        self.lm_vocab = vocab_size

    def init_lm_head_bf16_device(self, weights_dev, vocab_size, stream=None):
        check(lib().moe_init_lm_head_bf16_device(self._ctx, _dp(weights_dev), vocab_size, stream))
        self.lm_vocab = vocab_size

    def dispatch_lm_head(self, x, vocab_size):
        y = np.empty(vocab_size, np.float32)
        check(lib().moe_dispatch_lm_head(self._ctx, _p(_c(x, np.float32)), vocab_size, _p(y)))
        return y

    def dispatch_lm_head_device(self, x_dev, vocab_size, logits_dev, stream=None):
        """Device pointers (DeviceBuffer or int), enqueued without synchronisation."""
        check(lib().moe_dispatch_lm_head_device(self._ctx, _dp(x_dev), vocab_size, _dp(logits_dev), stream))

    # ---- path level
    def router_topk(self, layer, x, top_k, want_logits=False, n_experts=None):
        x = _c(x, np.float32).reshape(-1, self.hidden_size)
        T = x.shape[0]
        idx = np.empty((T, top_k), np.int32)
        w = np.empty((T, top_k), np.float32)
        logits = np.empty((T, n_experts), np.float32) if want_logits else None
        check(lib().moe_router_topk(self._ctx, layer, _p(x), T, top_k, _p(idx), _p(w),
                                    _p(logits)))
        return (idx, w, logits) if want_logits else (idx, w)

    def layer_forward(self, layer, x, top_k):
        x = _c(x, np.float32).reshape(-1, self.hidden_size)
        y = np.empty_like(x)
        check(lib().moe_layer_forward(self._ctx, layer, _p(x), x.shape[0], top_k, _p(y)))
        return y

    def block_forward_device(self, layer, x_dev, n_tokens, top_k, out_dev, stream=None):
        check(lib().moe_block_forward_device(self._ctx, layer, x_dev.ptr, n_tokens, top_k, out_dev.ptr, stream))

    def layer_forward_device(self, layer, x_dev, n_tokens, top_k, y_dev, stream=None):
        check(lib().moe_layer_forward_device(self._ctx, layer, x_dev.ptr, n_tokens, top_k,
                                             y_dev.ptr, stream))

    def dequant_expert(self, layer, expert, which):
        rows, cols = ((2 * self.inter_size, self.hidden_size) if which == 0
                      else (self.hidden_size, self.inter_size))
        out = DeviceBuffer(rows * cols * 4)
        check(lib().moe_dequant_expert_device(self._ctx, layer, expert, which, out.ptr, None))
        self.synchronize()
        return out.download(np.float32, (rows, cols))

    def synchronize(self):
        check(lib().moe_synchronize(self._ctx))

    # ---- timing
    def set_timing(self, on):
        check(lib().moe_set_timing(self._ctx, int(on)))

    def get_timing(self, kernel):
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        check(lib().moe_get_timing(self._ctx, kernel, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def reset_timing(self):
        check(lib().moe_reset_timing(self._ctx))


def mxfp4_dequant(blocks, scales, rows, cols):
    """Bit-exact MXFP4 decode on the GPU (weights.rs:350-423). Host arrays in, f32 out."""
    b = DeviceBuffer.from_array(_c(blocks, np.uint8))
    s = DeviceBuffer.from_array(_c(scales, np.uint8))
    out = DeviceBuffer(rows * cols * 4)
    check(lib().moe_mxfp4_dequant_device(b.ptr, s.ptr, rows, cols, out.ptr, None))
    return out.download(np.float32, (rows, cols))


def mxfp4_pack(blocks_dev, scales_dev, rows, cols):
    n = lib().moe_mxfp4_packed_size(rows, cols)
    if n == 0:
        raise ValueError("rows must be a multiple of 16 and cols of 32")
    out = DeviceBuffer(n)
    check(lib().moe_mxfp4_pack_device(blocks_dev.ptr, scales_dev.ptr, rows, cols, out.ptr, None))
    return out


def mxfp4_matvec(disp, packed_dev, rows, cols, x_dev, y_dev, stream=None):
    check(lib().moe_mxfp4_matvec_device(disp.ctx, packed_dev.ptr, rows, cols, x_dev.ptr,
                                        y_dev.ptr, stream))


def safetensors_find(path, name):
    """Header entry of tensor `name` in a safetensors file: (dtype, shape, (begin, end)) with the
    byte range in the file. Needs no device."""
    import os
    dt = ctypes.create_string_buffer(16)
    shape = (ctypes.c_uint64 * 8)()
    rank = ctypes.c_size_t()
    b, e = ctypes.c_uint64(), ctypes.c_uint64()
    check(lib().moe_safetensors_find(os.fsencode(path), name.encode(), dt, 16, shape, 8, ctypes.byref(rank),
                                     ctypes.byref(b), ctypes.byref(e)))
    return dt.value.decode(), tuple(shape[i] for i in range(min(rank.value, 8))), (b.value, e.value)
