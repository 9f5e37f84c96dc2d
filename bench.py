"""Benchmark of the MXFP4 MoE path on one MI355X.

The headline line (`value`) is config 2 of the benchmark's configuration list: one
GPT-OSS-20B-shaped MoE layer at decode batch 1 — router 2880->32 (bf16), top-4, 4 experts of
gate_up 2880->5760 + down 2880->2880 in MXFP4, interleaved SwiGLU, weighted combine. A step is
one token through one layer. To keep the 256 MB MALL from serving the weights, 24 independent
layers (10.2 GB of experts) stay resident and consecutive steps walk through them with
distinct tokens, so every step streams its experts from HBM.

The default run (`--workload all`) also times the other configurations in the same process and
reports each under `configs` with its own dominant-kernel roofline: config 1 (one 2880x2880
MXFP4 matvec), config 3 (64 tokens through one layer), config 4 (4096 tokens through all 24
layers; once more with the grouped GEMM on MXFP6 activations, the opt-in MOE_OPT_ACT_QUANT
contract, as `config4_prefill_4096x24_mxfp6`), config 5 (a 120B-shaped layer, 128 experts, at 1
and 2048 tokens), and the next rows beside the path (the bf16 LM head, the Beaver-triple
generator). Those use their own step counts (in each entry); --steps / --warmup apply to the
headline.

Prints ONE JSON line. `--workload <name>` runs one configuration alone (for profiling).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from silentotithrandousha_amd import GpuMoeDispatcher, DeviceBuffer  # noqa: E402
from silentotithrandousha_amd import synthetic as syn  # noqa: E402
from silentotithrandousha_amd._ffi import check, lib  # noqa: E402

METRIC = "MoE layer tokens/s @GPT-OSS-20B shape (b=1,64,4096) + % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
MXFP4_PEAK_TFLOPS = 10100.0
H20 = I20 = 2880

ARITH_DECODE = ("MXFP4 weights as stored (E2M1 + E8M0) on the block-scaled MFMA; x as 4 fp8 e4m3 "
                "terms (exact to 2^-16), h as 4 fixed-exponent fp8 terms; f32 accumulate")
ARITH_GEMM = ("MXFP4 weights as stored (E2M1 + E8M0) on the block-scaled MFMA; activations as 3 "
              "fp6 E2M3 terms per 32-value block (exact to ~2^-13 of the block maximum); f32 "
              "accumulate")
ARITH_GEMM_Q = ("MXFP4 weights as stored on the block-scaled MFMA; activations (x and the SwiGLU "
                "output h) quantized to MXFP6 (one E2M3 value per element, OCP MX E8M0 scale per "
                "32-value block): the opt-in MOE_OPT_ACT_QUANT contract (the fp32 path on the "
                "quantized activations), not the default 1e-3 contract; f32 accumulate")
DTYPE_DECODE = "mxfp4 x f32(4 fp8 terms), f32 acc"
DTYPE_GEMM = "mxfp4 x f32(3 fp6 terms), f32 acc"
DTYPE_GEMM_Q = "mxfp4 x mxfp6, f32 acc"

# workload -> (config name, experts, tokens per layer, layers per step, default steps, warmup)
WORKLOADS = {
    "decode1": ("config2 gpt-oss-20b moe layer decode b=1", 32, 1, 1, 4800, 480),
    "decode64": ("config3 gpt-oss-20b moe layer decode b=64", 32, 64, 1, 960, 96),
    "prefill": ("config4 gpt-oss-20b moe prefill 4096 tokens x 24 layers", 32, 4096, 24, 8, 2),
    "decode1_120b": ("config5 gpt-oss-120b moe layer b=1", 128, 1, 1, 4800, 480),
    "prefill_120b": ("config5 gpt-oss-120b moe layer 2048 tokens", 128, 2048, 1, 48, 8),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ algorithmic bytes / flops
def expert_bytes(H, I):
    """Checkpoint-format bytes of one expert's gate_up and down (MXFP4 nibbles + E8M0 scales +
    bf16 biases)."""
    nbh, nbi = H // 32, I // 32
    gu = 2 * I * nbh * 16 + 2 * I * nbh + 2 * I * 2
    dn = H * nbi * 16 + H * nbi + H * 2
    return gu, dn


def layer_traffic(H, I, E, T, active):
    """Algorithmic HBM bytes of one layer step: `active` experts' weights once, the router
    (bf16 W + f32 bias) once, activations in and out in f32."""
    gu, dn = expert_bytes(H, I)
    return active * (gu + dn) + E * H * 2 + E * 4 + 2 * T * H * 4


def layer_flops(H, I, E, k, T):
    return 2.0 * T * E * H + 2.0 * T * k * (2 * I * H + H * I)


def expected_active(E, k, T):
    """Expected distinct experts of T tokens routed to k of E experts each (uniform routing)."""
    if T == 1:
        return min(E, k)
    return E * (1.0 - (1.0 - k / E) ** T)


# ------------------------------------------------------------------ resident synthetic model
class Model:
    """One dispatcher holding n_layers resident synthetic layers of one shape, generated on the
    device (nibbles uniform, E8M0 118..130, biases bf16 N(0, 0.01), router bf16 N(0, 0.02))."""

    def __init__(self, H, I, E, n_layers, opts, seed=1234):
        self.H, self.I, self.E, self.n_layers = H, I, E, n_layers
        self.disp = GpuMoeDispatcher(H, I, 7.0)
        self.disp.set_fused_decode(opts.fused)
        self.disp.set_batch_gemm(opts.batch_gemm)
        self.disp.set_gemm_shape(opts.gemm_shape, opts.gemm_shape_down)
        self.disp.set_gemm_band(opts.gemm_band)
        log(f"synthesising {n_layers} layers x {E} experts "
            f"({n_layers * E * sum(expert_bytes(H, I)) / 1e9:.2f} GB MXFP4)")
        nbh, nbi = H // 32, I // 32
        sizes = dict(gub=E * 2 * I * nbh * 16, gus=E * 2 * I * nbh, gubias=E * 2 * I * 4,
                     db=E * H * nbi * 16, ds=E * H * nbi, dbias=E * H * 4)
        stage = {n: DeviceBuffer(s) for n, s in sizes.items()}
        L = lib()
        rng = np.random.default_rng(seed)
        for l in range(n_layers):
            s0 = seed * 1000 + l * 16
            check(L.moe_synth_fill_device(stage["gub"].ptr, sizes["gub"], 0, s0 + 1, 0, 255, None))
            check(L.moe_synth_fill_device(stage["gus"].ptr, sizes["gus"], 0, s0 + 2, 118, 130, None))
            check(L.moe_synth_fill_device(stage["gubias"].ptr, sizes["gubias"] // 4, 3, s0 + 3, 0.01, 0, None))
            check(L.moe_synth_fill_device(stage["db"].ptr, sizes["db"], 0, s0 + 4, 0, 255, None))
            check(L.moe_synth_fill_device(stage["ds"].ptr, sizes["ds"], 0, s0 + 5, 118, 130, None))
            check(L.moe_synth_fill_device(stage["dbias"].ptr, sizes["dbias"] // 4, 3, s0 + 6, 0.01, 0, None))
            check(L.moe_preload_layer_device(self.disp.ctx, l, E, stage["gub"].ptr, stage["gus"].ptr,
                                             stage["gubias"].ptr, stage["db"].ptr, stage["ds"].ptr,
                                             stage["dbias"].ptr, None))
            rw = syn.bf16_bits(rng.normal(0, 0.02, size=(E, H)).astype(np.float32))
            rb = np.zeros(E, np.float32)
            check(L.moe_preload_router(self.disp.ctx, l, E, rw.ctypes.data, rb.ctypes.data))
            self.disp.synchronize()
        for b in stage.values():
            b.close()
        log(f"resident: {n_layers} layers")

    def close(self):
        self.disp.close()


class StreamEvents:
    """A pair of HIP events recorded on one stream (the context stream, where the kernels run;
    torch's events would see only torch's current stream). The HIP runtime is the one the
    library already loaded (same soname)."""

    def __init__(self, stream):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.stream = ctypes.c_void_p(stream)
        self.ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in self.ev:
            self._ok(self.hip.hipEventCreate(ctypes.byref(e)), "hipEventCreate")

    @staticmethod
    def _ok(rc, what):
        if rc:
            raise RuntimeError(f"{what} failed with HIP error {rc}")

    def start(self):
        self._ok(self.hip.hipEventRecord(self.ev[0], self.stream), "hipEventRecord")

    def stop(self):
        self._ok(self.hip.hipEventRecord(self.ev[1], self.stream), "hipEventRecord")

    def sync(self):
        """hipStreamSynchronize of the stream: the end of a timed window (the library's
        moe_synchronize also reads the kernels' error word back, a device-to-host copy that is
        no part of the timed work; callers run it after the window)."""
        self._ok(self.hip.hipStreamSynchronize(self.stream), "hipStreamSynchronize")

    def elapsed_ms(self):
        self._ok(self.hip.hipEventSynchronize(self.ev[1]), "hipEventSynchronize")
        ms = ctypes.c_float()
        self._ok(self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[0], self.ev[1]),
                 "hipEventElapsedTime")
        return ms.value

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


def capture(disp, fn, first, count):
    """A HIP graph of steps first .. first+count-1 on the context stream, launched once
    (upload and first replay, untimed)."""
    L = lib()
    check(L.moe_graph_begin(disp.ctx))
    for i in range(first, first + count):
        fn(i)
    g = ctypes.c_void_p()
    check(L.moe_graph_end(disp.ctx, ctypes.byref(g)))
    check(L.moe_graph_launch(disp.ctx, g.value))
    disp.synchronize()
    return g.value


KERNELS = ["route", "bucket", "gate_up", "down", "combine", "decode_gate_up", "decode_down",
           "decode_layer"]


# ------------------------------------------------------------------ layer workloads (configs 2-5)
def run_layer(model, workload, steps, warmup, graph=True, copy_mib=0, traffic_kib=0.0, act_quant=False):
    """act_quant: the grouped GEMM on MXFP6 activations (MOE_OPT_ACT_QUANT) for this run only."""
    disp = model.disp
    disp.set_act_quant(act_quant)
    try:
        return _run_layer(model, workload, steps, warmup, graph, copy_mib, traffic_kib, act_quant)
    finally:
        disp.set_act_quant(False)


def _run_layer(model, workload, steps, warmup, graph, copy_mib, traffic_kib, act_quant):
    config_name, E, T, lps, _, _ = WORKLOADS[workload]
    assert E == model.E
    H, I, k, n_layers = model.H, model.I, 4, model.n_layers
    disp, L = model.disp, lib()
    P = max(n_layers * 10, 8) if T == 1 else max(2 * n_layers, 2)  # distinct token slots
    x = DeviceBuffer(P * T * H * 4)
    y = DeviceBuffer(P * T * H * 4)
    check(L.moe_synth_fill_device(x.ptr, P * T * H, 2, 99, 1.0, 0, None))
    disp.synchronize()

    def step(i):
        for u in range(lps):
            c = i * lps + u
            j = c % P
            check(L.moe_layer_forward_device(disp.ctx, c % n_layers, x.ptr + j * T * H * 4, T, k,
                                             y.ptr + j * T * H * 4, None))

    for i in range(warmup):
        step(i)
    disp.synchronize()
    if copy_mib:
        copy_calibration(copy_mib)

    # every timed step replays from a HIP graph: G steps per launch of the main graph, and the
    # remainder of steps / G in a second graph
    graphs = []
    G = (min(steps, P) if lps == 1 else 1) if graph else 0
    n_full, rem = divmod(steps, G) if G else (0, steps)
    if G:
        graphs.append((capture(disp, step, 0, G), n_full))
        if rem:
            graphs.append((capture(disp, step, n_full * G, rem), 1))
    disp.synchronize()
    region = StreamEvents(L.moe_stream(disp.ctx))
    region.sync()
    t0 = time.perf_counter()
    region.start()
    if G:
        for g, n in graphs:
            for _ in range(n):
                check(L.moe_graph_launch(disp.ctx, g))
    else:
        for i in range(steps):
            step(i)
    region.stop()
    region.sync()
    elapsed = time.perf_counter() - t0
    disp.synchronize()  # the kernels' error word (a bounded wait that ran out) is reported here
    region_ms = region.elapsed_ms()
    region.close()
    for g, _ in graphs:
        check(L.moe_graph_destroy(g))

    # per-kernel durations: HIP events around every launch, eager, over the same steps
    disp.set_timing(True)
    disp.reset_timing()
    n_kt = min(steps, max(240 // lps, 1))
    for i in range(n_kt):
        step(i)
    disp.synchronize()
    kt = {name: disp.get_timing(kid) for kid, name in enumerate(KERNELS)}
    disp.set_timing(False)
    x.close()
    y.close()

    ms_per_step = elapsed * 1e3 / steps
    tokens_per_s = T * steps / elapsed  # a step takes T tokens through all lps layers
    active = expected_active(E, k, T)
    traffic = layer_traffic(H, I, E, T, active) * lps
    flops = layer_flops(H, I, E, k, T) * lps
    gu_b, _ = expert_bytes(H, I)
    dom = "decode_layer" if kt["decode_layer"][1] else "decode_gate_up" if kt["decode_gate_up"][1] else "gate_up"
    d_ms, d_n = kt[dom]
    d_avg_s = d_ms / max(d_n, 1) / 1e3
    timing_src = "HIP events around each launch (eager pass over the same steps)"
    if dom == "decode_layer" and lps == 1 and G:
        # every step is one launch of this kernel and nothing else: its average duration is the
        # timed region's span between two events on its stream over the launch count, free of
        # the per-launch event and dispatch overhead of the eager brackets
        d_avg_s = region_ms / steps / 1e3
        timing_src = "HIP events on the context stream around the graph-replayed timed region / launches"
    if dom == "decode_layer":  # the whole layer in one launch
        d_bytes, d_flops = layer_traffic(H, I, E, T, active), layer_flops(H, I, E, k, T)
        kname = "k_decode_layer"
    else:
        d_bytes = active * gu_b + T * H * 4 + T * k * I * 4
        d_flops = 2.0 * T * k * 2 * I * H
        kname = "k_gemm_fp8<gate_up>" if dom == "gate_up" else "k_decode_gate_up"
        # the library's choice of the grouped GEMM (gemm.hip launch_gemm_mode, by the mean entries
        # per expert): the wide streamed form at 14-44 and 60-72, the streamed form below 24,
        # unless a shape is forced
        shape = model.disp.gemm_shape
        mean = T * k // max(1, min(E, T * k))
        if dom == "gate_up":
            if shape == 14 or (shape == 0 and 14 <= mean and (mean < 44 or 60 <= mean < 72)):
                kname = "k_gemm_wide<gate_up>"
            elif shape in (12, 13) or (shape == 0 and mean < 24):
                kname = "k_gemm_stream<gate_up>"
    mfma_bound = T >= 4096  # config 4: arithmetic intensity above the MXFP4 ridge point
    res = {
        "value": round(tokens_per_s, 1), "unit": "tokens/s", "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_per_step, 6),
        "dtype": (DTYPE_DECODE if T == 1 and dom == "decode_layer" else DTYPE_GEMM_Q if act_quant and dom == "gate_up"
                  else DTYPE_GEMM),
        "config": {"workload": config_name, "name": workload, "hidden": H, "intermediate": I,
                   "experts": E, "top_k": k, "tokens_per_layer": T, "layers_per_step": lps,
                   "resident_layers": n_layers,
                   "weights": "MXFP4 E2M1 + E8M0 (checkpoint layout repacked on preload)",
                   "arithmetic": (ARITH_DECODE if dom == "decode_layer" else ARITH_GEMM_Q if act_quant and dom == "gate_up"
                                  else ARITH_GEMM),
                   "graph_replay": ("all steps: %d x graph of %d steps%s" % (n_full, G, f" + graph of {rem}" if rem else "")
                                    if G else "none (eager launches)")},
        "roofline": {"bound": "hbm", "kernel": kname,
                     "achieved": round(d_bytes / d_avg_s / 1e9, 1) if d_n else None,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(d_bytes / d_avg_s / 1e9 / HBM_PEAK_GBS, 4) if d_n else None,
                     "traffic": traffic_kib * 1024 if traffic_kib else None,
                     "algorithmic_bytes_per_launch": int(d_bytes), "flops_per_launch": d_flops,
                     "avg_launch_us": round(d_avg_s * 1e6, 3), "timing": timing_src,
                     "TFLOPs": round(d_flops / d_avg_s / 1e12, 2) if d_n else None},
        "layer_roofline": {"algorithmic_bytes_per_step": int(traffic), "flops_per_step": flops,
                           "achieved_GBps": round(traffic / (ms_per_step / 1e3) / 1e9, 1),
                           "frac_hbm": round(traffic / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                           "achieved_TFLOPs": round(flops / (ms_per_step / 1e3) / 1e12, 2),
                           "frac_mxfp4_peak": round(flops / (ms_per_step / 1e3) / 1e12 / MXFP4_PEAK_TFLOPS, 5)},
        "kernel_us": {n: round(v[0] * 1e3 / max(v[1], 1), 3) for n, v in kt.items() if v[1]},
    }
    if mfma_bound and d_n:
        # dense regime: the MFMA roofline against the MXFP4 peak, algorithmic flops (one
        # MXFP4 x MXFP4 product per multiply-add; the exact path issues 3 activation terms, the
        # quantized mode one, at the same fp4 x fp6 rate as fp4 x fp4)
        res["roofline"].update(bound="mfma", achieved=round(d_flops / d_avg_s / 1e12, 2),
                               peak=MXFP4_PEAK_TFLOPS, unit="TFLOP/s",
                               frac=round(d_flops / d_avg_s / 1e12 / MXFP4_PEAK_TFLOPS, 5),
                               hbm_GBps=round(d_bytes / d_avg_s / 1e9, 1))
    if not traffic_kib:
        attach_traffic(res["roofline"], kname, workload, act_quant)
    return res


def attach_traffic(roofline, kname, workload, act_quant=False):
    """The calibrated PMC measurement (rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE per launch) of the
    same kernel on the same workload, from profiles/traffic.json, into roofline["traffic"]."""
    tf = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(tf):
        return
    recs = json.load(open(tf))
    # (the quantized mode runs other kernels: its records are keyed apart)
    key = f"{kname}@{workload}" + ("+act_quant" if act_quant else "")
    rec = recs.get(key) or (None if act_quant else recs.get(kname))
    if rec and rec.get("workload") == workload:
        roofline["traffic"] = rec["bytes_per_launch"]
        roofline["traffic_source"] = rec["source"]


# ------------------------------------------------------------------ config 1: one MXFP4 matvec
def run_matvec(steps, warmup, graph=True):
    """y = W x, W 2880x2880 MXFP4; 96 distinct copies (283 MB, above the 256 MB MALL) back to
    back in a HIP graph."""
    L = lib()
    from silentotithrandousha_amd import mxfp4_matvec, mxfp4_pack
    R = C = 2880
    copies = 96
    disp = GpuMoeDispatcher(C, C, 7.0)
    nb = C // 32
    blocks = DeviceBuffer(R * nb * 16)
    scales = DeviceBuffer(R * nb)
    packed = []
    for c in range(copies):
        check(L.moe_synth_fill_device(blocks.ptr, R * nb * 16, 0, 7000 + 2 * c, 0, 255, None))
        check(L.moe_synth_fill_device(scales.ptr, R * nb, 0, 7001 + 2 * c, 118, 130, None))
        packed.append(mxfp4_pack(blocks, scales, R, C))
    x = DeviceBuffer(C * 4)
    y = DeviceBuffer(R * 4)
    check(L.moe_synth_fill_device(x.ptr, C, 2, 5, 1.0, 0, None))
    disp.synchronize()

    def one(i):
        mxfp4_matvec(disp, packed[i % copies], R, C, x, y)

    for i in range(warmup):
        one(i)
    disp.synchronize()
    g = capture(disp, one, 0, copies) if graph else None
    reps = max(1, steps // copies) if graph else 0
    steps = reps * copies if graph else steps
    region = StreamEvents(L.moe_stream(disp.ctx))
    t0 = time.perf_counter()
    region.start()
    if graph:
        for _ in range(reps):
            check(L.moe_graph_launch(disp.ctx, g))
    else:
        for i in range(steps):
            one(i)
    region.stop()
    region.sync()
    el = time.perf_counter() - t0
    disp.synchronize()
    region_s = region.elapsed_ms() / 1e3
    region.close()
    if g:
        check(L.moe_graph_destroy(g))
    for b in packed + [blocks, scales, x, y]:
        b.close()
    disp.close()
    byts = R * nb * 17 + C * 4 + R * 4
    kgbs = byts * steps / region_s / 1e9  # one k_matvec_fp4 launch per matvec
    return {"value": round(byts * steps / el / 1e9, 1), "unit": "GB/s",
            "matvecs_per_s": round(steps / el, 1), "steps": steps, "warmup": warmup,
            "ms_per_step": round(el * 1e3 / steps, 6), "dtype": DTYPE_DECODE,
            "config": {"workload": "config1 mxfp4 matvec 2880x2880", "copies": copies,
                       "graph_replay": f"{reps} x graph of {copies} matvecs" if graph else "none"},
            "roofline": {"bound": "hbm", "kernel": "k_matvec_fp4", "achieved": round(kgbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                         "traffic": None, "algorithmic_bytes_per_launch": byts,
                         "avg_launch_us": round(region_s / steps * 1e6, 3),
                         "timing": "HIP events on the context stream around the timed region / launches"}}


def run_lm_head(steps, warmup, H=2880, V=201088):
    """The next row after the MoE path: dispatch_lm_head (moe_dispatch.rs:624-683), logits[V] =
    W[V, H] x in f32 with the reference's f32 weights (201 088 x 2880 = 2.32 GB), device-resident
    input and logits."""
    rng = np.random.default_rng(9)
    log(f"lm head: {V} x {H} f32 ({V * H * 4 / 1e9:.2f} GB)")
    w = rng.standard_normal((V, H), dtype=np.float32)
    w *= np.float32(0.02)
    disp = GpuMoeDispatcher(H, H, 7.0)
    disp.init_lm_head(w, V)
    del w
    x = DeviceBuffer.from_array(rng.standard_normal(H, dtype=np.float32))
    y = DeviceBuffer(V * 4)
    for _ in range(warmup):
        disp.dispatch_lm_head_device(x, V, y)
    disp.synchronize()
    region = StreamEvents(lib().moe_stream(disp.ctx))
    t0 = time.perf_counter()
    region.start()
    for _ in range(steps):
        disp.dispatch_lm_head_device(x, V, y)
    region.stop()
    region.sync()
    el = time.perf_counter() - t0
    disp.synchronize()
    region_s = region.elapsed_ms() / 1e3
    region.close()
    byts = V * H * 4 + H * 4 + V * 4
    kgbs = byts * steps / region_s / 1e9  # one k_lm_head launch per step
    disp.close()
    return {"value": round(byts * steps / el / 1e9, 1), "unit": "GB/s", "steps": steps,
            "warmup": warmup, "ms_per_step": round(el * 1e3 / steps, 6), "dtype": "f32",
            "config": {"workload": "lm head (next row) 201088x2880 f32", "vocab": V, "hidden": H},
            "roofline": {"bound": "hbm", "kernel": "k_lm_head", "achieved": round(kgbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                         "traffic": None, "algorithmic_bytes_per_launch": byts,
                         "avg_launch_us": round(region_s / steps * 1e6, 3),
                         "timing": "HIP events on the context stream around the timed region / launches"}}


def run_lm_head_bf16(steps, warmup, H=2880, V=201088):
    """The LM head from the checkpoint's bf16 lm_head.weight (lm_head_dot, weights.rs:73-82):
    201 088 x 2880 bf16 = 1.16 GB streamed per call, device-resident input and logits; weights
    generated on the device (bf16 of N(0, 0.02))."""
    L = lib()
    log(f"lm head bf16: {V} x {H} ({V * H * 2 / 1e9:.2f} GB)")
    disp = GpuMoeDispatcher(H, H, 7.0)
    wd = DeviceBuffer(V * H * 2)
    check(L.moe_synth_fill_device(wd.ptr, V * H, 1, 77, 0.02, 0, None))
    disp.init_lm_head_bf16_device(wd, V)
    wd.close()
    x = DeviceBuffer(H * 4)
    check(L.moe_synth_fill_device(x.ptr, H, 2, 78, 1.0, 0, None))
    y = DeviceBuffer(V * 4)
    for _ in range(warmup):
        disp.dispatch_lm_head_device(x, V, y)
    disp.synchronize()
    region = StreamEvents(L.moe_stream(disp.ctx))
    t0 = time.perf_counter()
    region.start()
    for _ in range(steps):
        disp.dispatch_lm_head_device(x, V, y)
    region.stop()
    region.sync()
    el = time.perf_counter() - t0
    disp.synchronize()
    region_s = region.elapsed_ms() / 1e3
    region.close()
    for b in (x, y):
        b.close()
    disp.close()
    byts = V * H * 2 + H * 4 + V * 4
    kgbs = byts * steps / region_s / 1e9  # one k_lm_head_bf16 launch per step
    return {"value": round(byts * steps / el / 1e9, 1), "unit": "GB/s", "steps": steps,
            "warmup": warmup, "ms_per_step": round(el * 1e3 / steps, 6), "dtype": "bf16 x f32, f32 acc",
            "config": {"workload": "lm head (next row) 201088x2880 bf16 (checkpoint dtype)", "vocab": V, "hidden": H},
            "roofline": {"bound": "hbm", "kernel": "k_lm_head_bf16", "achieved": round(kgbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                         "traffic": None, "algorithmic_bytes_per_launch": byts,
                         "avg_launch_us": round(region_s / steps * 1e6, 3),
                         "timing": "HIP events on the context stream around the timed region / launches"}}


def run_beaver32(steps, warmup, n=5, t=1, count=50_000_000):
    """The Beaver-triple generator (§8's last row; the reference's GpuTripleGen32,
    gpu/mod.rs:511-1012): `count` triples of one party per call with device-resident seeds and
    outputs — the reference's kernel-only throughput path (dispatch_kernel_only, mod.rs:915-938,
    timed at 50M triples in beaver.rs:3576-3610, n = 5, t = 1)."""
    from silentotithrandousha_amd import GpuTripleGen32
    L = lib()
    g = GpuTripleGen32(n, t)
    rounds = g.num_rounds(count)
    seeds = DeviceBuffer(rounds * 4)
    check(L.moe_synth_fill_device(seeds.ptr, rounds * 4, 0, 91, 0, 255, None))
    outs = [DeviceBuffer(count * 4) for _ in range(3)]
    hip = ctypes.CDLL("libamdhip64.so.7")
    stream = ctypes.c_void_p()
    if hip.hipStreamCreate(ctypes.byref(stream)):
        raise RuntimeError("hipStreamCreate failed")
    for _ in range(warmup):
        g.generate_device(0, count, seeds, *outs, stream=stream)
    hip.hipStreamSynchronize(stream)
    region = StreamEvents(stream.value)  # events on the stream the kernels run on
    t0 = time.perf_counter()
    region.start()
    for _ in range(steps):
        g.generate_device(0, count, seeds, *outs, stream=stream)
    region.stop()
    hip.hipStreamSynchronize(stream)
    el = time.perf_counter() - t0
    region_s = region.elapsed_ms() / 1e3
    region.close()
    hip.hipStreamDestroy(stream)
    for b in outs + [seeds]:
        b.close()
    g.close()
    byts = count * 12 + rounds * 4  # a, b, c words written + the round seeds read
    return {"value": round(count * steps / el, 1), "unit": "triples/s", "steps": steps, "warmup": warmup,
            "ms_per_step": round(el * 1e3 / steps, 6), "dtype": "u32 (mod 2^31 - 1)",
            "config": {"workload": "beaver triples p = 2^31 - 1, one party, 50M per call", "n": n, "t": t,
                       "count": count},
            "roofline": {"bound": "hbm", "kernel": "k_beaver32", "achieved": round(byts * steps / region_s / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(byts * steps / region_s / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": None, "algorithmic_bytes_per_launch": byts,
                         "avg_launch_us": round(region_s / steps * 1e6, 3),
                         "timing": "HIP events on the launch stream around the timed region / launches"}}


def copy_calibration(mib):
    """One plain device-to-device copy of `mib` MiB (the runtime's blit kernel,
    __amd_rocclr_copyBuffer): under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE per dispatch
    calibrate the counters against a known byte count."""
    n = mib << 20
    a, b = DeviceBuffer(n), DeviceBuffer(n)
    check(lib().moe_memset_device(a.ptr, 1, n))
    check(lib().moe_memcpy_d2d(b.ptr, a.ptr, n))
    log(f"copy calibration: {mib} MiB device-to-device")
    a.close()
    b.close()


# ------------------------------------------------------------------ CPU baseline
def host_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "cpus_available": affinity}


def cpu_baseline(seconds, H, I, E, k):
    """The reference's live CPU MoE block restated in C (oracle/), on config 2's layer shape:
    router + top-4, then per selected expert cpu_expert_ffn with the NEON-order fp16 x f32
    matvec on k threads (rayon over the k slots, session.rs:953-972) and the slot-order combine.
    Three legs, each a bounded sample of `seconds`:
      cold  — fp16 expert cache missing every expert (random routing over 32 experts with the
              reference's 4 cache slots): MXFP4 -> fp16 decode of the 4 experts per token
              (session.rs:860-941) — the reference's live path on this workload, the headline;
      warm  — every selected expert already in the fp16 cache (matvecs only), its best case;
      fp32  — the reference's f32 helpers (weights.rs:350-423 decode + sequential f32 matvec,
              session.rs:75-85), the oracle's own path, on the oracle's OpenMP threads."""
    from oracle import orc
    layers = [syn.make_layer(H, I, E, seed=500 + i) for i in range(2)]
    xs = syn.hidden(64, H, seed=501)
    legs = {}

    def route(lay, x):
        logits = orc.router_logits(lay["router_w"], lay["router_b"], x, E, H)
        idx, w, _, _ = orc.topk(logits, k)
        return idx[0], w[0]

    # cold: decode on every token
    n, t0 = 0, time.perf_counter()
    while True:
        lay, x = layers[n % 2], xs[n % 64]
        idx, w = route(lay, x)
        orc.live_moe_token(x, lay, idx, w, k)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 3) or n >= 2000:
            break
    legs["cold"] = {"value": round(n / el, 3), "unit": "tokens/s", "threads": k,
                    "sample": f"{n} tokens, {el:.1f} s"}
    # warm: two tokens of one layer alternate, so at most 2k fp16 entries are built (outside
    # the timed calls) and every timed token finds its experts cached
    cache, n, el = {}, 0, 0.0
    while True:
        li = 0
        lay, x = layers[li], xs[n % 2]
        idx, w = route(lay, x)
        for e in idx:
            if (li, int(e)) not in cache:
                cache[(li, int(e))] = orc.live_expert_f16(lay, int(e))
        ents = [cache[(li, int(e))] for e in idx]
        t0 = time.perf_counter()
        route(lay, x)
        orc.live_moe_token_warm(x, H, I, ents, w, k)
        el += time.perf_counter() - t0
        n += 1
        if (el >= seconds / 2 and n >= 3) or n >= 2000:
            break
    legs["warm"] = {"value": round(n / el, 3), "unit": "tokens/s", "threads": k,
                    "sample": f"{n} tokens (2 alternating, {len(cache)} cached fp16 experts), {el:.1f} s timed"}
    del cache
    # fp32 path
    n, t0 = 0, time.perf_counter()
    while True:
        orc.moe_layer(xs[n % 64][None], layers[n % 2], k)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds / 2 and n >= 3) or n >= 2000:
            break
    legs["fp32"] = {"value": round(n / el, 3), "unit": "tokens/s", "threads": orc.omp_threads(),
                    "sample": f"{n} tokens, {el:.1f} s"}
    return {"value": legs["cold"]["value"], "unit": "tokens/s", "cores": k, "kind": "port",
            "sample": (f"config-2 layer shape, 2 synthetic layers x {E} experts, 64 tokens cycled; "
                       f"cold fp16 expert cache (the reference's live path under random routing): "
                       f"{legs['cold']['sample']} on {k} threads (rayon over the top-{k} slots)"),
            "legs": legs, "host": host_info()}


# ------------------------------------------------------------------ main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="headline steps (default: per workload)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="all",
                    choices=["all", "matvec", "lm_head", "lm_head_bf16", "beaver32"] + list(WORKLOADS))
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--layers-120b", type=int, default=6)
    ap.add_argument("--no-graph", dest="graph", action="store_false")
    ap.add_argument("--no-fused", dest="fused", action="store_false",
                    help="single-token steps through the multi-kernel path")
    ap.add_argument("--decode-mode", type=int, default=None, choices=(0, 1, 2),
                    help="single-token path: 2 one launch (default), 1 two launches (bf16 MFMA on decoded "
                         "weights), 0 the five-kernel batch path")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", dest="cpu", action="store_false")
    ap.add_argument("--gemm-shape", type=int, default=0, choices=range(20), help="grouped GEMM block shape (tuning)")
    ap.add_argument("--gemm-shape-down", type=int, default=0, choices=range(20),
                    help="block shape of the down GEMM alone (0: as --gemm-shape; tuning)")
    ap.add_argument("--gemm-band", type=int, default=0, help="grouped GEMM row blocks per band of the XCD tile order (tuning; 0 default)")
    ap.add_argument("--batch-gemm", type=int, default=1, choices=(0, 1, 2),
                    help="batches: 0 GEMV kernels, 1 grouped GEMM when experts average >= 4 entries, 2 always GEMM")
    ap.add_argument("--act-quant", action="store_true",
                    help="grouped GEMM on MXFP6 activations (MOE_OPT_ACT_QUANT; single --workload runs)")
    ap.add_argument("--traffic-kib", type=float, default=0.0,
                    help="HBM KiB per launch of the dominant kernel (overrides the calibrated "
                         "rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE figure in profiles/traffic.json)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (PMC calibration)")
    args = ap.parse_args()
    if args.decode_mode is not None:
        args.fused = args.decode_mode if args.decode_mode != 2 else True
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path (expert parallel / row split) is a design note, not built.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))
    head = "decode1" if args.workload == "all" else args.workload
    dsteps, dwarm = {"matvec": (4800, 480), "lm_head": (40, 4), "lm_head_bf16": (80, 8), "beaver32": (20, 3)}.get(
        head, WORKLOADS.get(head, (0,) * 6)[4:])
    steps = dsteps if args.steps is None else args.steps
    warmup = dwarm if args.warmup is None else args.warmup
    common = {"metric": METRIC, "n_gpus": 1, "higher_is_better": True, "scaling": "weak",
              "vs_baseline": None,
              "data": ("synthetic (seeded, device-generated; nibbles uniform 0..15, E8M0 118..130, "
                       "router N(0,0.02) bf16, biases N(0,0.01) bf16, x N(0,1))")}
    if head == "matvec":
        common["metric"] = "MXFP4 matvec 2880x2880 GB/s (config 1)"
    elif head in ("lm_head", "lm_head_bf16"):
        common["metric"] = "LM head GEMV 201088x2880 GB/s"
    elif head == "beaver32":
        common["metric"] = "Beaver triples/s, p = 2^31 - 1, n = 5, t = 1"
    t_start = time.perf_counter()
    def with_traffic(r, workload):  # the measured HBM traffic of the dominant kernel, when recorded
        attach_traffic(r["roofline"], r["roofline"]["kernel"], workload)
        return r

    if head in ("matvec", "lm_head", "lm_head_bf16", "beaver32") and args.copy_mib:
        copy_calibration(args.copy_mib)
    if head == "matvec":
        res = with_traffic(run_matvec(steps, warmup, args.graph), head)
    elif head == "lm_head":
        res = with_traffic(run_lm_head(steps, warmup), head)
    elif head == "lm_head_bf16":
        res = with_traffic(run_lm_head_bf16(steps, warmup), head)
    elif head == "beaver32":
        res = with_traffic(run_beaver32(steps, warmup), head)
    else:
        E = WORKLOADS[head][1]
        m = Model(H20, I20, E, args.layers if E == 32 else args.layers_120b, args)
        res = run_layer(m, head, steps, warmup, args.graph, args.copy_mib, args.traffic_kib, args.act_quant)
        log(f"{head}: {res['value']} tokens/s ({res['ms_per_step']} ms/step)")
        extras = {}
        if args.workload == "all":
            for w, key, q in (("decode64", "config3_decode64", False), ("prefill", "config4_prefill_4096x24", False),
                              ("prefill", "config4_prefill_4096x24_mxfp6", True)):
                extras[key] = run_layer(m, w, WORKLOADS[w][4], WORKLOADS[w][5], args.graph, act_quant=q)
                log(f"{key}: {extras[key]['value']} tokens/s")
            m.close()
            m = Model(H20, I20, 128, args.layers_120b, args)
            for w, key in (("decode1_120b", "config5_120b_decode1"), ("prefill_120b", "config5_120b_2048")):
                extras[key] = run_layer(m, w, WORKLOADS[w][4], WORKLOADS[w][5], args.graph)
                log(f"{w}: {extras[key]['value']} tokens/s")
            m.close()
            extras["config1_matvec"] = with_traffic(run_matvec(4800, 480, args.graph), "matvec")
            log(f"matvec: {extras['config1_matvec']['value']} GB/s")
            extras["next_lm_head_bf16"] = with_traffic(run_lm_head_bf16(80, 8), "lm_head_bf16")
            log(f"lm head bf16: {extras['next_lm_head_bf16']['value']} GB/s")
            extras["next_beaver32"] = with_traffic(run_beaver32(20, 3), "beaver32")
            log(f"beaver32: {extras['next_beaver32']['value']} triples/s")
            res["configs"] = extras
        else:
            m.close()
    out = dict(common)
    out.update(res)
    if args.cpu and rank == 0 and head == "decode1":
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds, H20, I20, 32, 4)
    log(f"done in {time.perf_counter() - t_start:.1f} s")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
