"""Benchmark of the MXFP4 MoE path on one MI355X.

Default workload (config 2 of the benchmark's configuration list): one GPT-OSS-20B-shaped MoE layer at decode batch 1 —
router 2880->32 (bf16), top-4, 4 experts of gate_up 2880->5760 + down 2880->2880 in MXFP4,
interleaved SwiGLU, weighted combine. A step is one token through one layer. To keep the
256 MB MALL from serving the weights, 24 independent layers (10.2 GB of experts) stay
resident and consecutive steps walk through them with distinct tokens, so every step
streams its experts from HBM.

Prints ONE JSON line (see the repository's benchmark contract). Other workloads
(--workload matvec|decode64|prefill|decode1_120b|prefill_120b) print the same kind of line
as well; the driver runs the default.
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
BF16_PEAK_TFLOPS = 2500.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ algorithmic bytes / flops
# Checkpoint-format bytes of one expert (MXFP4 nibbles + E8M0 scales + bf16 biases).
def expert_bytes(H, I):
    nbh, nbi = H // 32, I // 32
    gu = 2 * I * nbh * 16 + 2 * I * nbh + 2 * I * 2
    dn = H * nbi * 16 + H * nbi + H * 2
    return gu, dn


def layer_traffic(H, I, E, k, T, active):
    """Algorithmic HBM bytes of one layer step: `active` experts' weights once, the router
    (bf16 W + f32 bias) once, activations in and out in f32."""
    gu, dn = expert_bytes(H, I)
    return active * (gu + dn) + E * H * 2 + E * 4 + 2 * T * H * 4


def layer_flops(H, I, E, k, T):
    return 2.0 * T * E * H + 2.0 * T * k * (2 * I * H + H * I)


# ------------------------------------------------------------------ resident synthetic layers
class Layers:
    def __init__(self, disp, H, I, E, n_layers, seed=1234):
        self.disp, self.H, self.I, self.E = disp, H, I, E
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
            check(L.moe_preload_layer_device(disp.ctx, l, E, stage["gub"].ptr, stage["gus"].ptr,
                                             stage["gubias"].ptr, stage["db"].ptr, stage["ds"].ptr,
                                             stage["dbias"].ptr, None))
            rw = syn.bf16_bits(rng.normal(0, 0.02, size=(E, H)).astype(np.float32))
            rb = np.zeros(E, np.float32)
            check(L.moe_preload_router(disp.ctx, l, E, rw.ctypes.data, rb.ctypes.data))
            disp.synchronize()
            if l % 6 == 5 or l == n_layers - 1:
                log(f"resident layers {l + 1}/{n_layers}")
        for b in stage.values():
            b.close()


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

    def elapsed_ms(self):
        self._ok(self.hip.hipEventSynchronize(self.ev[1]), "hipEventSynchronize")
        ms = ctypes.c_float()
        self._ok(self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[0], self.ev[1]),
                 "hipEventElapsedTime")
        return ms.value

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


# ------------------------------------------------------------------ decode / prefill bench
def run_layer_bench(args, H, I, E, k, T, n_layers, workload, config_name, layers_per_step=1,
                    mfma_bound=False):
    """A step is `layers_per_step` consecutive resident layers, each on its own T tokens
    (layers_per_step = 24 for the 24-layer prefill of config 4)."""
    L = lib()
    disp = GpuMoeDispatcher(H, I, 7.0)
    disp.set_fused_decode(args.fused)
    disp.set_batch_gemm(args.batch_gemm)
    disp.set_gemm_shape(args.gemm_shape, args.gemm_shape_down)
    disp.set_gemm_band(args.gemm_band)
    log(f"synthesising {n_layers} layers x {E} experts ({n_layers * E * sum(expert_bytes(H, I)) / 1e9:.2f} GB MXFP4)")
    Layers(disp, H, I, E, n_layers)
    P = max(n_layers * 10, 8) if T == 1 else 2 * n_layers
    x = DeviceBuffer(P * T * H * 4)
    y = DeviceBuffer(P * T * H * 4)
    check(L.moe_synth_fill_device(x.ptr, P * T * H, 2, 99, 1.0, 0, None))
    disp.synchronize()

    def step(i, stream=None):
        for u in range(layers_per_step):
            c = i * layers_per_step + u
            j = c % P
            check(L.moe_layer_forward_device(disp.ctx, c % n_layers, x.ptr + j * T * H * 4, T, k,
                                             y.ptr + j * T * H * 4, stream))

    log("warmup")
    for i in range(args.warmup):
        step(i)
    disp.synchronize()

    if args.copy_mib:
        copy_calibration(args.copy_mib)
    graph = None
    G = (P if layers_per_step == 1 else 1) if args.graph else 0
    if args.graph:
        check(L.moe_graph_begin(disp.ctx))
        for i in range(G):
            step(i)
        g = ctypes.c_void_p()
        check(L.moe_graph_end(disp.ctx, ctypes.byref(g)))
        graph = g.value
        check(L.moe_graph_launch(disp.ctx, graph))  # upload / first replay untimed
        disp.synchronize()

    log(f"timed region: {args.steps} steps ({'graph x' + str(G) if graph else 'eager'})")
    disp.synchronize()
    region = StreamEvents(L.moe_stream(disp.ctx))
    t0 = time.perf_counter()
    region.start()
    if graph:
        n_full, rem = divmod(args.steps, G)
        for _ in range(n_full):
            check(L.moe_graph_launch(disp.ctx, graph))
        for i in range(rem):
            step(i)
    else:
        for i in range(args.steps):
            step(i)
    region.stop()
    disp.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    region_ms = region.elapsed_ms()
    region.close()

    # per-kernel durations: HIP events around every launch, same steps, eager
    log("kernel timing region")
    disp.set_timing(True)
    disp.reset_timing()
    n_kt = min(args.steps, max(240 // layers_per_step, G))
    for i in range(n_kt):
        step(i)
    disp.synchronize()
    kt = {name: disp.get_timing(kid) for kid, name in
          enumerate(["route", "bucket", "gate_up", "down", "combine", "decode_gate_up",
                     "decode_down", "decode_layer", "reserved"])}
    disp.set_timing(False)
    if graph:
        check(L.moe_graph_destroy(graph))

    tokens_per_s = T * args.steps / elapsed
    active = min(E, T * k) if T == 1 else E  # expected distinct experts per layer
    traffic = layer_traffic(H, I, E, k, T, active) * layers_per_step
    flops = layer_flops(H, I, E, k, T) * layers_per_step
    gu_b, dn_b = expert_bytes(H, I)
    dom = ("decode_layer" if kt["decode_layer"][1] else
           "decode_gate_up" if kt["decode_gate_up"][1] else "gate_up")
    gu_ms, gu_n = kt[dom]
    gu_avg_s = gu_ms / max(gu_n, 1) / 1e3
    timing_src = "HIP events around each launch (eager pass over the same steps)"
    if dom == "decode_layer" and layers_per_step == 1:
        # every step is one launch of this kernel and nothing else: its average duration is the
        # timed region's span between two events on its stream over the launch count, which
        # leaves out the per-launch event and dispatch overhead of the eager brackets
        gu_avg_s = region_ms / args.steps / 1e3
        timing_src = "HIP events on the context stream around the timed region / launches"
    if dom == "decode_layer":  # the whole layer in one launch
        gu_bytes = layer_traffic(H, I, E, k, T, active)
        gu_flops = layer_flops(H, I, E, k, T)
    else:
        gu_bytes = active * gu_b + T * H * 4 + T * k * I * 4
        gu_flops = 2.0 * T * k * 2 * I * H
    res = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded; nibbles uniform, E8M0 118..130, router N(0,0.02) bf16, biases N(0,0.01) bf16, x N(0,1); device-generated)",
        "config": {"workload": workload, "name": config_name, "hidden": H, "intermediate": I,
                   "experts": E, "top_k": k, "tokens_per_layer": T, "layers_per_step": layers_per_step,
                   "resident_layers": n_layers,
                   "weights": "MXFP4 E2M1 + E8M0 (checkpoint layout repacked on preload)",
                   "arithmetic": ("MXFP4 weights as stored on the block-scaled MFMA; x as 4 fp8 terms, h as "
                                  "fixed-exponent fp8 terms; f32 accumulate" if T == 1 and args.fused else
                                  "MXFP4 weights as stored on the block-scaled MFMA; activations as 3 E2M3 "
                                  "terms (grouped GEMM) or bf16 hi+lo (GEMV path); f32 accumulate"),
                   "graph_replay": bool(graph), "fused_decode": bool(args.fused and T == 1)},
        "roofline": {"bound": "hbm",
                     "kernel": {"decode_layer": "k_decode_layer", "decode_gate_up": "k_decode_gate_up",
                                "gate_up": "k_gemm_fp8<gate_up>"}[dom],
                     "achieved": round(gu_bytes / gu_avg_s / 1e9, 1) if gu_n else None,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_bytes / gu_avg_s / 1e9 / HBM_PEAK_GBS, 4) if gu_n else None,
                     "traffic": args.traffic_kib * 1024 if args.traffic_kib else None,
                     "algorithmic_bytes_per_launch": gu_bytes,
                     "avg_launch_us": round(gu_avg_s * 1e6, 3),
                     "timing": timing_src,
                     "mfma_TFLOPs": round(gu_flops / gu_avg_s / 1e12, 2) if gu_n else None},
        "layer_roofline": {"algorithmic_bytes_per_step": traffic, "flops_per_step": flops,
                           "achieved_GBps": round(traffic / (ms_per_step / 1e3) / 1e9, 1),
                           "frac_hbm": round(traffic / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                           "achieved_TFLOPs": round(flops / (ms_per_step / 1e3) / 1e12, 2),
                           "frac_mxfp4_peak": round(flops / (ms_per_step / 1e3) / 1e12 / MXFP4_PEAK_TFLOPS, 5)},
        "kernel_us": {n: round(v[0] * 1e3 / max(v[1], 1), 3) for n, v in kt.items() if v[1]},
    }
    if not args.traffic_kib:  # calibrated PMC measurement of the same kernel and workload
        tf = os.path.join(ROOT, "profiles", "traffic.json")
        kname = res["roofline"]["kernel"]
        if os.path.exists(tf):
            rec = json.load(open(tf)).get(kname)
            if rec and rec.get("workload") == config_name:
                res["roofline"]["traffic"] = rec["bytes_per_launch"]
                res["roofline"]["traffic_source"] = rec["source"]
    if mfma_bound and gu_n:
        # dense regime: the MFMA roofline against the MXFP4 peak (the arithmetic runs on the
        # bf16 MFMA with a hi+lo split of the activations, i.e. 2x these flops)
        res["roofline"].update(bound="mfma", achieved=round(gu_flops / gu_avg_s / 1e12, 2),
                               peak=MXFP4_PEAK_TFLOPS, unit="TFLOP/s",
                               frac=round(gu_flops / gu_avg_s / 1e12 / MXFP4_PEAK_TFLOPS, 5),
                               hbm_GBps=round(gu_bytes / gu_avg_s / 1e9, 1))
    disp.close()
    return res


def run_matvec_bench(args):
    """Config 1: y = W x, W 2880x2880 MXFP4; 64 distinct copies back to back."""
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
    for i in range(args.warmup):
        mxfp4_matvec(disp, packed[i % copies], R, C, x, y)
    disp.synchronize()
    # the copies back to back in one HIP graph (a matvec is ~0.6 us of HBM traffic, below the
    # cost of a host launch), replayed for the timed region
    graph = None
    if args.graph:
        check(L.moe_graph_begin(disp.ctx))
        for i in range(copies):
            mxfp4_matvec(disp, packed[i], R, C, x, y)
        g = ctypes.c_void_p()
        check(L.moe_graph_end(disp.ctx, ctypes.byref(g)))
        graph = g.value
        check(L.moe_graph_launch(disp.ctx, graph))
        disp.synchronize()
    reps = max(1, args.steps // copies) if graph else 0
    steps = reps * copies if graph else args.steps
    region = StreamEvents(L.moe_stream(disp.ctx))
    t0 = time.perf_counter()
    region.start()
    if graph:
        for _ in range(reps):
            check(L.moe_graph_launch(disp.ctx, graph))
    else:
        for i in range(steps):
            mxfp4_matvec(disp, packed[i % copies], R, C, x, y)
    region.stop()
    disp.synchronize()
    el = time.perf_counter() - t0
    region_s = region.elapsed_ms() / 1e3
    region.close()
    if graph:
        check(L.moe_graph_destroy(graph))
    byts = R * nb * 17 + C * 4 + R * 4
    gbs = byts * steps / el / 1e9
    kgbs = byts * steps / region_s / 1e9  # one k_matvec_fp4 launch per matvec
    return {"metric": "MXFP4 matvec 2880x2880 GB/s", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
            "ms_per_step": round(el * 1e3 / steps, 6), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "config1 matvec 2880x2880", "copies": copies,
                       "graph_replay": bool(graph)},
            "roofline": {"bound": "hbm", "kernel": "k_matvec_fp4",
                         "achieved": round(kgbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(kgbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes_per_launch": byts,
                         "avg_launch_us": round(region_s / steps * 1e6, 3),
                         "timing": "HIP events on the context stream around the timed region / launches"}}


def run_lm_head_bench(args, H, V):
    """The next row after the MoE path: dispatch_lm_head (moe_dispatch.rs:624-683), logits[V] =
    W[V, H] x in f32 with the reference's f32 weights (201 088 x 2880 = 2.32 GB), device-resident
    input and logits."""
    from silentotithrandousha_amd import DeviceBuffer
    rng = np.random.default_rng(9)
    log(f"lm head: {V} x {H} f32 ({V * H * 4 / 1e9:.2f} GB)")
    w = rng.standard_normal((V, H), dtype=np.float32)
    w *= np.float32(0.02)
    disp = GpuMoeDispatcher(H, H, 7.0)
    disp.init_lm_head(w, V)
    del w
    x = DeviceBuffer.from_array(rng.standard_normal(H, dtype=np.float32))
    y = DeviceBuffer(V * 4)
    for _ in range(args.warmup):
        disp.dispatch_lm_head_device(x, V, y)
    disp.synchronize()
    region = StreamEvents(lib().moe_stream(disp.ctx))
    t0 = time.perf_counter()
    region.start()
    for _ in range(args.steps):
        disp.dispatch_lm_head_device(x, V, y)
    region.stop()
    disp.synchronize()
    el = time.perf_counter() - t0
    region_s = region.elapsed_ms() / 1e3
    region.close()
    byts = V * H * 4 + H * 4 + V * 4
    gbs = byts * args.steps / el / 1e9
    kgbs = byts * args.steps / region_s / 1e9  # one k_lm_head launch per step
    disp.close()
    return {"metric": "LM head f32 GEMV 201088x2880 GB/s", "value": round(gbs, 1), "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(el * 1e3 / args.steps, 6), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic (weights N(0,0.02), x N(0,1))",
            "config": {"workload": "lm head (next row) 201088x2880 f32", "vocab": V, "hidden": H},
            "roofline": {"bound": "hbm", "kernel": "k_lm_head", "achieved": round(kgbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                         "traffic": None, "algorithmic_bytes_per_launch": byts,
                         "avg_launch_us": round(region_s / args.steps * 1e6, 3),
                         "timing": "HIP events on the context stream around the timed region / launches"}}


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
def cpu_baseline(seconds, H, I, E, k):
    """The reference's live CPU MoE block restated in C (oracle/): router + top-4, cold fp16
    expert cache (MXFP4 -> fp16 decode of the 4 selected experts, session.rs:860-941) and
    cpu_expert_ffn with the NEON matvec order, one thread per selected expert (rayon over
    k slots, session.rs:953-972), then the combine. Bounded sample, rank 0, N=1 only."""
    from oracle import orc
    layers = [syn.make_layer(H, I, E, seed=500 + i) for i in range(2)]
    xs = syn.hidden(64, H, seed=501)
    n = 0
    t0 = time.perf_counter()
    while True:
        lay = layers[n % 2]
        x = xs[n % 64]
        logits = orc.router_logits(lay["router_w"], lay["router_b"], x, E, H)
        idx, w, _, _ = orc.topk(logits, k)
        orc.live_moe_token(x, lay, idx[0], w[0], k)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 3) or n >= 1000:
            break
    return {"value": round(n / el, 3), "unit": "tokens/s", "cores": k, "kind": "port",
            "sample": f"{n} tokens of the config-2 layer (2 synthetic layers, cold fp16 expert "
                      f"cache: MXFP4->fp16 dequant + fp16xf32 matvec in the reference's NEON "
                      f"order, {k} threads as rayon over the top-{k} slots), {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="default: per workload")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode1",
                    choices=["decode1", "decode64", "prefill", "matvec", "decode1_120b", "prefill_120b", "lm_head"])
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--no-graph", dest="graph", action="store_false")
    ap.add_argument("--no-fused", dest="fused", action="store_false",
                    help="single-token steps through the multi-kernel path")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", dest="cpu", action="store_false")
    ap.add_argument("--gemm-shape", type=int, default=0, choices=range(8), help="grouped GEMM block shape (tuning)")
    ap.add_argument("--gemm-shape-down", type=int, default=0, choices=range(8),
                    help="block shape of the down GEMM alone (0: as --gemm-shape; tuning)")
    ap.add_argument("--gemm-band", type=int, default=0, help="grouped GEMM row blocks per band of the XCD tile order (tuning; 0 default)")
    ap.add_argument("--batch-gemm", type=int, default=1, choices=(0, 1, 2),
                    help="batches: 0 GEMV kernels, 1 grouped GEMM when experts average >= 4 entries, 2 always GEMM")
    ap.add_argument("--traffic-kib", type=float, default=0.0,
                    help="HBM KiB per launch of the dominant kernel (overrides the calibrated "
                         "rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE figure in profiles/traffic.json)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (PMC calibration)")
    args = ap.parse_args()
    dsteps, dwarm = {"decode1": (4800, 480), "decode1_120b": (4800, 480), "matvec": (4800, 480),
                     "decode64": (960, 96), "prefill": (8, 2), "prefill_120b": (48, 8),
                     "lm_head": (40, 4)}[args.workload]
    args.steps = dsteps if args.steps is None else args.steps
    args.warmup = dwarm if args.warmup is None else args.warmup
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path (expert parallel / row split) is a design note, not built.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))
    H = I = 2880
    if args.workload == "matvec":
        res = run_matvec_bench(args)
    elif args.workload == "lm_head":
        res = run_lm_head_bench(args, H, 201088)
    elif args.workload == "decode1":
        res = run_layer_bench(args, H, I, 32, 4, 1, args.layers, "config2 gpt-oss-20b moe layer decode b=1", "decode1")
    elif args.workload == "decode64":
        res = run_layer_bench(args, H, I, 32, 4, 64, args.layers, "config3 gpt-oss-20b moe layer decode b=64", "decode64")
    elif args.workload == "prefill":
        res = run_layer_bench(args, H, I, 32, 4, 4096, args.layers,
                              "config4 gpt-oss-20b moe prefill 4096 tokens x 24 layers", "prefill",
                              layers_per_step=args.layers, mfma_bound=True)
    elif args.workload == "decode1_120b":
        res = run_layer_bench(args, H, I, 128, 4, 1, args.layers, "config5 gpt-oss-120b moe layer decode b=1", "decode1_120b")
    else:
        res = run_layer_bench(args, H, I, 128, 4, 2048, args.layers, "config5 gpt-oss-120b moe layer 2048 tokens", "prefill_120b")
    if args.cpu and rank == 0 and args.workload == "decode1":
        log("cpu baseline")
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds, H, I, 32, 4)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
