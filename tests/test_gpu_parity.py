"""GPU parity tests: the HIP path through the C ABI against the CPU oracle.

Bar: bit-exact for the MXFP4 decode, the router logits and the top-k indices; 1e-3 relative
L2 (REL_L2_TOL) for matmul outputs against the fp32 reference path on the same inputs.
"""
import numpy as np
import pytest

from silentotithrandousha_amd import DeviceBuffer, GpuMoeDispatcher, mxfp4_dequant, mxfp4_matvec, mxfp4_pack
from silentotithrandousha_amd import synthetic as syn
from tests.helpers import REL_L2_TOL, assert_bit_exact, assert_rel_l2, rel_l2

pytestmark = pytest.mark.gpu

H20, I20, E20 = 2880, 2880, 32


def exhaustive_mxfp4():
    """256 rows (one per E8M0 byte) x 1 block whose 16 bytes hold every nibble twice."""
    blocks = np.zeros((256, 1, 16), np.uint8)
    for j in range(16):
        blocks[:, 0, j] = j | ((15 - j) << 4)
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    return blocks, scales


@pytest.fixture(scope="module")
def layer20():
    return syn.make_layer(H20, I20, E20, seed=20)


@pytest.fixture(scope="module")
def disp20(layer20):
    d = GpuMoeDispatcher(H20, I20, 7.0)
    d.preload_layer(0, layer20)
    yield d
    d.close()


# ---------------------------------------------------------------- decode

def test_dequant_exhaustive_bit_exact(orc):
    blocks, scales = exhaustive_mxfp4()
    got = mxfp4_dequant(blocks, scales, 256, 32)
    want = orc.dequant_mxfp4(blocks, scales, 256, 32)
    assert_bit_exact(got, want, "16x256 nibble/scale table")


def test_dequant_random_matrix_bit_exact(orc):
    rng = np.random.default_rng(1)
    rows, cols = 96, 2880
    blocks = rng.integers(0, 256, size=(rows, cols // 32, 16), dtype=np.uint8)
    scales = rng.integers(0, 256, size=(rows, cols // 32), dtype=np.uint8)
    assert_bit_exact(mxfp4_dequant(blocks, scales, rows, cols),
                     orc.dequant_mxfp4(blocks, scales, rows, cols), "random 96x2880")


def test_resident_copy_lossless(orc):
    """preload repacks; decoding the resident copy gives the checkpoint decode bit for bit."""
    H, I, E = 256, 128, 2
    L = syn.make_layer(H, I, E, seed=3, router=False)
    rng = np.random.default_rng(4)
    L["gu_scales"] = rng.integers(0, 256, size=L["gu_scales"].shape, dtype=np.uint8)
    L["d_scales"] = rng.integers(0, 256, size=L["d_scales"].shape, dtype=np.uint8)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    for e in range(E):
        gu = d.dequant_expert(0, e, 0)
        dn = d.dequant_expert(0, e, 1)
        assert_bit_exact(gu, orc.dequant_mxfp4(L["gu_blocks"][e], L["gu_scales"][e], 2 * I, H),
                         f"gate_up expert {e}")
        assert_bit_exact(dn, orc.dequant_mxfp4(L["d_blocks"][e], L["d_scales"][e], H, I),
                         f"down expert {e}")
    d.close()


# ---------------------------------------------------------------- MXFP4 matvec (config 1)

MATVEC_PATHS = [1, 0]  # one launch on the block-scaled MFMA; split + bf16 GEMV


def _matvec(disp, blocks, scales, rows, cols, x, path=1):
    disp.set_matvec(path)
    b = DeviceBuffer.from_array(blocks)
    s = DeviceBuffer.from_array(scales)
    packed = mxfp4_pack(b, s, rows, cols)
    xd = DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    yd = DeviceBuffer(rows * 4)
    mxfp4_matvec(disp, packed, rows, cols, xd, yd)
    disp.synchronize()
    return yd.download(np.float32, rows)


@pytest.mark.parametrize("path", MATVEC_PATHS)
def test_matvec_config1(orc, path):
    rows = cols = 2880
    rng = np.random.default_rng(11)
    blocks = rng.integers(0, 256, size=(rows, cols // 32, 16), dtype=np.uint8)
    scales = rng.integers(118, 131, size=(rows, cols // 32), dtype=np.uint8)
    x = rng.normal(0, 1, cols).astype(np.float32)
    d = GpuMoeDispatcher(cols, cols, 7.0)
    got = _matvec(d, blocks, scales, rows, cols, x, path)
    want = orc.mxfp4_matvec(blocks, scales, rows, cols, x)
    e = assert_rel_l2(got, want, "2880x2880 MXFP4 matvec")
    assert e < 1e-5, f"matvec error {e:.2e} larger than the activation split allows"
    d.close()


@pytest.mark.parametrize("path", MATVEC_PATHS)
def test_matvec_one_hot_columns_exact(orc, path):
    """x = e_k returns column k of W exactly: the in-kernel decode is bit-exact (up to the
    sign of zero, which a sum cannot carry)."""
    rows, cols = 64, 256
    rng = np.random.default_rng(12)
    blocks = rng.integers(0, 256, size=(rows, cols // 32, 16), dtype=np.uint8)
    scales = rng.integers(100, 160, size=(rows, cols // 32), dtype=np.uint8)
    W = orc.dequant_mxfp4(blocks, scales, rows, cols)
    d = GpuMoeDispatcher(cols, cols, 7.0)
    for k in [0, 1, 2, 7, 8, 31, 32, 33, 100, 255]:
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        got = _matvec(d, blocks, scales, rows, cols, x, path)
        assert np.array_equal(got, W[:, k]), f"column {k}"
    d.close()


@pytest.mark.parametrize("path", MATVEC_PATHS)
def test_matvec_ragged_shapes(orc, path):
    """Block counts that are not a multiple of 4 (partial last step) and of 16 (partial
    last scale word)."""
    rng = np.random.default_rng(13)
    d = GpuMoeDispatcher(32, 32, 7.0)
    for rows, nb in [(16, 1), (32, 2), (16, 3), (48, 5), (16, 17), (32, 90), (16, 95), (16, 96), (32, 97)]:
        cols = 32 * nb
        blocks = rng.integers(0, 256, size=(rows, nb, 16), dtype=np.uint8)
        scales = rng.integers(118, 131, size=(rows, nb), dtype=np.uint8)
        x = rng.normal(0, 1, cols).astype(np.float32)
        got = _matvec(d, blocks, scales, rows, cols, x, path)
        assert_rel_l2(got, orc.mxfp4_matvec(blocks, scales, rows, cols, x), f"{rows}x{cols}",
                      tol=1e-5)
    d.close()


@pytest.mark.parametrize("path", MATVEC_PATHS)
def test_matvec_edge_scales(orc, path):
    """E8M0 bytes 0 (scale +0.0) and 255 (scale +inf in the reference decode, NaN in the OCP
    MX spec). Rows touching a 255 block are non-finite exactly where the fp32 path is; the
    GEMV does not promise the reference's choice between +-inf and NaN there, because the
    activation enters as hi + lo and inf * lo can be inf * 0 (the bit-exact dequant kernel
    keeps the reference's +inf)."""
    rows, cols = 32, 64
    rng = np.random.default_rng(14)
    blocks = rng.integers(0, 256, size=(rows, 2, 16), dtype=np.uint8)
    scales = rng.integers(120, 128, size=(rows, 2), dtype=np.uint8)
    scales[3, 0] = 0
    scales[5, 1] = 0
    scales[9, 0] = 255
    blocks[9, 0, :] = 0x22  # no zero nibbles: +-inf products only
    scales[11, 1] = 255     # contains zero nibbles: 0 * inf = NaN
    blocks[11, 1, 0] = 0x10
    x = np.abs(rng.normal(0, 1, cols).astype(np.float32)) + 0.5
    d = GpuMoeDispatcher(cols, cols, 7.0)
    got = _matvec(d, blocks, scales, rows, cols, x, path)
    want = orc.mxfp4_matvec(blocks, scales, rows, cols, x)
    assert np.array_equal(np.isfinite(got), np.isfinite(want)), (got[[9, 11]], want[[9, 11]])
    assert not np.isfinite(want[9]) and not np.isfinite(want[11])
    fin = np.isfinite(want)
    assert rel_l2(got[fin], want[fin]) < 1e-5
    d.close()


# ---------------------------------------------------------------- LM head

def test_lm_head_host_and_device():
    """dispatch_lm_head (moe_dispatch.rs:624-683): logits = W x in f32, against a float64 dot
    (the kernel sums 64 lane-strided fused partial sums then a xor butterfly; tolerance 1e-5
    relative L2), and the device-pointer form gives the same bits; a vocab past the initialised
    one is refused."""
    from silentotithrandousha_amd import DeviceBuffer
    from silentotithrandousha_amd._ffi import MoeError
    H, V = 2880, 1000
    rng = np.random.default_rng(60)
    w = (rng.standard_normal((V, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    d = GpuMoeDispatcher(H, H, 7.0)
    d.init_lm_head(w, V)
    got = d.dispatch_lm_head(x, V)
    want = w.astype(np.float64) @ x.astype(np.float64)
    assert rel_l2(got, want) < 1e-5
    xd, yd = DeviceBuffer.from_array(x), DeviceBuffer(V * 4)
    d.dispatch_lm_head_device(xd, V - 7, yd)
    d.synchronize()
    assert np.array_equal(yd.download(np.float32, (V,))[:V - 7], got[:V - 7])
    with pytest.raises(MoeError):
        d.dispatch_lm_head(x, V + 1)
    d.close()


@pytest.mark.parametrize("H,V", [(2880, 50001), (64, 37)])
def test_lm_head_bf16(orc, H, V):
    """The checkpoint's bf16 LM head (lm_head_dot, weights.rs:73-82): every logit within the
    sum-of-products bound gamma_n sum |w x| of the float64 dot (n = H + 8: the kernel's fused
    lane chains and its 64-lane butterfly) and so of the oracle's sequential restatement; 50 001
    rows make every wavefront walk several row pairs and leave an odd last row. The host and
    device initialisations give the same bits; an f32 init after a bf16 one switches back."""
    from silentotithrandousha_amd import DeviceBuffer
    rng = np.random.default_rng(61)
    w = syn.bf16_bits((rng.standard_normal((V, H)) * 0.02).astype(np.float32))
    x = rng.standard_normal(H).astype(np.float32)
    d = GpuMoeDispatcher(H, H, 7.0)
    d.init_lm_head_bf16(w, V)
    got = d.dispatch_lm_head(x, V).astype(np.float64)
    W = syn.bf16_to_f32(w).astype(np.float64)
    y64 = W @ x.astype(np.float64)
    u = 2.0 ** -24
    n = H + 8
    bound = n * u / (1 - n * u) * (np.abs(W) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - y64) <= bound)
    want = orc.lm_head_bf16(w, x).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * bound)
    assert rel_l2(got, y64) < 1e-6
    wd, xd, yd = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), DeviceBuffer(V * 4)
    d.init_lm_head_bf16_device(wd, V)
    d.dispatch_lm_head_device(xd, V, yd)
    d.synchronize()
    assert np.array_equal(yd.download(np.float32, (V,)), got.astype(np.float32))
    # the bf16 head reads x with 16-byte loads: an input 4 bytes past an aligned address is refused
    from silentotithrandousha_amd._ffi import MoeError
    xo = DeviceBuffer((H + 4) * 4)
    with pytest.raises(MoeError, match="aligned"):
        d.dispatch_lm_head_device(xo.ptr + 4, V, yd)
    wf = syn.bf16_to_f32(w[:8])
    d.init_lm_head(wf, 8)
    assert rel_l2(d.dispatch_lm_head(x, 8), wf.astype(np.float64) @ x.astype(np.float64)) < 1e-5
    d.close()


# ---------------------------------------------------------------- router + top-k

def test_router_logits_and_topk_bit_exact(orc, disp20, layer20):
    x = syn.hidden(16, H20, seed=21)
    idx, w, logits = disp20.router_topk(0, x, 4, want_logits=True, n_experts=E20)
    want_logits = orc.router_logits(layer20["router_w"], layer20["router_b"], x, E20, H20)
    assert_bit_exact(logits, want_logits, "router logits (canonical order)")
    widx, ww, _, _ = orc.topk(want_logits, 4)
    assert np.array_equal(idx, widx)
    assert np.max(np.abs(w - ww) / ww) < 1e-6
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)


def test_topk_ties_and_nan(orc):
    """Equal logits rank by lower index; NaN logits rank last (session.rs:822-825 order,
    totalised)."""
    H, E = 64, 8
    w = np.zeros((E, H), np.float32)
    w[:, 0] = [0.5, 1.0, 1.0, 0.25, 1.0, -1.0, 0.0, 0.75]
    wb = syn.bf16_bits(w)
    wb[6, 1] = 0x7FC0  # NaN weight -> NaN logit for expert 6
    b = np.zeros(E, np.float32)
    L = syn.make_layer(H, 32, E, seed=5, router=False)
    L["router_w"], L["router_b"] = wb, b
    d = GpuMoeDispatcher(H, 32, 7.0)
    d.preload_layer(0, L)
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 2.0
    x[0, 1] = 1.0
    for k in (1, 3, 4, 8):
        idx, ww, logits = d.router_topk(0, x, k, want_logits=True, n_experts=E)
        widx, www, _, _ = orc.topk(orc.router_logits(wb, b, x, E, H), k)
        assert np.array_equal(idx, widx), (k, idx, widx)
        assert list(idx[0][:3]) == [1, 2, 4][:k]
    assert np.isnan(logits[0, 6]) and idx[0, -1] == 6
    d.close()


# ---------------------------------------------------------------- expert FFN

@pytest.mark.parametrize("scales", [(118, 130), (108, 114)], ids=["baseline", "mild"])
def test_expert_preloaded_matches_fp32(orc, scales):
    L = syn.make_layer(H20, I20, 2, seed=30 + scales[0], scale_lo=scales[0], scale_hi=scales[1],
                       router=False)
    d = GpuMoeDispatcher(H20, I20, 7.0)
    d.preload_layer(0, L)
    x = syn.hidden(1, H20, seed=31)[0]
    for e in range(2):
        got = d.dispatch_expert_preloaded(x, 0, e)
        want = orc.expert_ffn(x, *syn.expert_slice(L, e), H20, I20)
        assert_rel_l2(got, want[0], f"expert {e} scales {scales}")
    d.close()


def test_dispatch_expert_raw_and_batched(orc):
    H, I = 512, 256
    L = syn.make_layer(H, I, 3, seed=40, scale_lo=112, scale_hi=120, router=False)
    d = GpuMoeDispatcher(H, I, 7.0)
    x = syn.hidden(1, H, seed=41)[0]
    outs = []
    for e in range(3):
        got = d.dispatch_expert(x, *syn.expert_slice(L, e))
        want = orc.expert_ffn(x, *syn.expert_slice(L, e), H, I)[0]
        assert_rel_l2(got, want, f"dispatch_expert {e}")
        outs.append(want)
    # short bias slices are zero-padded (moe_dispatch.rs:352-359)
    gb, gs, gbias, db, ds, dbias = syn.expert_slice(L, 0)
    got = d.dispatch_expert(x, gb, gs, gbias[:100], db, ds, dbias[:7])
    gb2 = np.zeros_like(gbias); gb2[:100] = gbias[:100]
    db2 = np.zeros_like(dbias); db2[:7] = dbias[:7]
    assert_rel_l2(got, orc.expert_ffn(x, gb, gs, gb2, db, ds, db2, H, I)[0], "short biases")
    ws = [0.5, 0.3, 0.2]
    got = d.dispatch_experts_batched(x, [(e, ws[e], *syn.expert_slice(L, e)) for e in range(3)])
    assert_rel_l2(got, orc.combine(np.stack(outs), np.array(ws, np.float32), skip_nonfinite=True),
                  "batched")
    d.close()


# ---------------------------------------------------------------- layer forward

@pytest.mark.parametrize("T", [1, 2, 64])
def test_layer_forward_20b(orc, disp20, layer20, T):
    x = syn.hidden(T, H20, seed=100 + T)
    got = disp20.layer_forward(0, x, 4)
    want, logits, idx, w = orc.moe_layer(x, layer20, 4)
    gidx, gw = disp20.router_topk(0, x, 4)
    assert np.array_equal(gidx, idx)
    assert_rel_l2(got, want, f"20B layer T={T}")


# ---------------------------------------------------------------- fused single-token layer

# single-token modes: 2 = one launch, 1 = two launches, 0 = the batch path
MODES = [2, 1, 0]


def test_fused_decode_matches_oracle_and_unfused(orc, disp20, layer20):
    xs = syn.hidden(6, H20, seed=300)
    for i in range(6):
        x = xs[i:i + 1]
        want, _, idx, _ = orc.moe_layer(x, layer20, 4)
        outs = []
        for m in MODES:
            disp20.set_fused_decode(m)
            outs.append(disp20.layer_forward(0, x, 4))
            assert_rel_l2(outs[-1], want, f"mode {m} token {i}")
        disp20.set_fused_decode(True)
        # modes 1 and 0 run the same per-column arithmetic (bf16 hi+lo activations) and may
        # differ only in combine order; mode 2 sends activations as 4 fp8 terms (|error| <=
        # 2^-16 per value), which moves outputs by a few 1e-5 relative
        assert rel_l2(outs[1], outs[2]) < 1e-6
        assert rel_l2(outs[0], outs[1]) < 2e-4


@pytest.mark.parametrize("mode", [2, 1])
def test_fused_decode_repeated_calls_and_graph_replay(orc, disp20, layer20, mode):
    """The one-launch kernel clears its own counters and mailboxes: back-to-back launches and
    graph replays give the eager result every time."""
    import ctypes
    from silentotithrandousha_amd._ffi import check, lib
    disp20.set_fused_decode(mode)
    H = H20
    xs = syn.hidden(3, H, seed=301)
    want = [orc.moe_layer(xs[i:i + 1], layer20, 4)[0][0] for i in range(3)]
    xd = DeviceBuffer.from_array(xs)
    yd = DeviceBuffer(3 * H * 4)
    for rep in range(3):
        for i in range(3):
            check(lib().moe_layer_forward_device(disp20.ctx, 0, xd.ptr + i * H * 4, 1, 4,
                                                 yd.ptr + i * H * 4, None))
        disp20.synchronize()
        got = yd.download(np.float32, (3, H))
        for i in range(3):
            assert_rel_l2(got[i], want[i], f"eager rep {rep} token {i}")
    check(lib().moe_graph_begin(disp20.ctx))
    for i in range(3):
        check(lib().moe_layer_forward_device(disp20.ctx, 0, xd.ptr + i * H * 4, 1, 4,
                                             yd.ptr + i * H * 4, None))
    g = ctypes.c_void_p()
    check(lib().moe_graph_end(disp20.ctx, ctypes.byref(g)))
    try:
        for rep in range(4):
            check(lib().moe_memset_device(yd.ptr, 0, 3 * H * 4))
            check(lib().moe_graph_launch(disp20.ctx, g.value))
            disp20.synchronize()
            got = yd.download(np.float32, (3, H))
            for i in range(3):
                assert_rel_l2(got[i], want[i], f"graph replay {rep} token {i}")
            # eager work between replays
            disp20.layer_forward(0, xs[0:1], 4)
    finally:
        check(lib().moe_graph_destroy(g.value))
        disp20.set_fused_decode(True)


@pytest.mark.parametrize("mode", [2, 1])
@pytest.mark.parametrize("shape", [(64, 32, 32, 4), (64, 32, 8, 1), (320, 96, 64, 3), (1024, 512, 16, 2),
                                   (64, 32, 128, 4), (320, 96, 100, 3), (128, 64, 65, 2)])
def test_fused_decode_small_shapes(orc, mode, shape):
    """Small and ragged single-token shapes (one gate_up block per slot, few down blocks, k < 4,
    64 to 128 experts, router chains of 1..2 loads per lane) on both fused paths."""
    H, I, E, k = shape
    L = syn.make_layer(H, I, E, seed=310 + H + E, scale_lo=120, scale_hi=124)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    d.set_fused_decode(mode)
    for i, x in enumerate(syn.hidden(4, H, seed=311)):
        want, _, idx, _ = orc.moe_layer(x[None], L, k)
        gidx, _ = d.router_topk(0, x[None], k)
        assert np.array_equal(gidx, idx)
        assert_rel_l2(d.layer_forward(0, x[None], k), want, f"{shape} mode {mode} token {i}")
    d.close()


def test_one_launch_bounded_wait_reports_and_recovers(orc, disp20, layer20):
    """A spin limit of one poll makes the one-launch kernel's cross-block waits give up (the
    failure path, forced from the host): the call reports the error, outputs are not silently
    wrong, and the next call with the default limit is correct again."""
    from silentotithrandousha_amd._ffi import MoeError
    x = syn.hidden(1, H20, seed=340)
    want = orc.moe_layer(x, layer20, 4)[0]
    disp20.set_fused_decode(2)
    disp20.set_spin_limit(1)
    raised = 0
    try:
        for _ in range(3):
            try:
                got = disp20.layer_forward(0, x, 4)
                assert_rel_l2(got, want, "spin limit 1, no timeout")
            except MoeError as e:
                assert "wait ran out" in str(e)
                raised += 1
    finally:
        disp20.set_spin_limit(1 << 20)
    assert raised >= 1
    for _ in range(2):
        assert_rel_l2(disp20.layer_forward(0, x, 4), want, "after recovery")


def test_adaptive_topk_fused_and_unfused(orc):
    H, I, E = 256, 128, 8
    L = syn.make_layer(H, I, E, seed=320, scale_lo=116, scale_hi=122, router_sigma=0.2)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    # parameters chosen so that the kept count takes the values 1, 2 and 4 on these tokens
    ad = orc.Adaptive(1, 1, 0.7, 0.4, 0.85)
    d.set_adaptive_topk(True, 1, 0.7, 0.4, 0.85)
    xs = syn.hidden(16, H, seed=321, sigma=1.0)
    used = set()
    for fused in MODES:
        d.set_fused_decode(fused)
        for i in range(16):
            want, _, idx, w = orc.moe_layer(xs[i:i + 1], L, 4, adaptive=ad)
            used.add(int((idx[0] >= 0).sum()))
            gidx, gw = d.router_topk(0, xs[i:i + 1], 4)
            assert np.array_equal(gidx, idx)
            assert_rel_l2(d.layer_forward(0, xs[i:i + 1], 4), want, f"adaptive fused={fused} {i}")
    assert used == {1, 2, 4}, used
    d.close()


def test_120b_layer_decode(orc):
    """GPT-OSS-120B shape (128 experts, top-4) at batch 1 (every single-token path) and 8."""
    E = 128
    L = syn.make_layer(H20, I20, E, seed=330)
    d = GpuMoeDispatcher(H20, I20, 7.0)
    d.preload_layer(0, L)
    for T in (1, 8):
        x = syn.hidden(T, H20, seed=331 + T)
        want, _, idx, _ = orc.moe_layer(x, L, 4)
        gidx, _ = d.router_topk(0, x, 4)
        assert np.array_equal(gidx, idx)
        for mode in (MODES if T == 1 else [2]):
            d.set_fused_decode(mode)
            assert_rel_l2(d.layer_forward(0, x, 4), want, f"120B T={T} mode {mode}")
    d.close()


@pytest.mark.parametrize("mode", MODES)
def test_single_token_ties_and_nan_across_halves(orc, mode):
    """128 experts: tied logits on both sides of expert 64 keep the lower index first, a NaN
    logit in the upper half ranks last; k = 3 drops the last of the tied experts, so picking
    the wrong one changes the output."""
    H, I, E = 64, 32, 128
    L = syn.make_layer(H, I, E, seed=350, scale_lo=120, scale_hi=124, router=False)
    w = np.zeros((E, H), np.float32)
    w[:, 0] = -0.5
    w[[3, 67, 100], 0] = 1.0
    w[120, 0] = 1.5
    wb = syn.bf16_bits(w)
    wb[90, 1] = 0x7FC0  # NaN logit for expert 90
    L["router_w"], L["router_b"] = wb, np.zeros(E, np.float32)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    d.set_fused_decode(mode)
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 2.0
    x[0, 1] = 1.0
    for k in (3, 4):
        want, _, idx, _ = orc.moe_layer(x, L, k)
        assert list(idx[0]) == [120, 3, 67, 100][:k]
        assert_rel_l2(d.layer_forward(0, x, k), want, f"ties k={k} mode {mode}")
    d.close()


@pytest.mark.parametrize("mode", MODES)
def test_single_token_nonfinite_weights(orc, mode):
    """E8M0 255 blocks (+inf in the reference decode, NaN in the OCP MX spec and to the
    block-scaled MFMA). The contract on non-finite weights: every output the fp32 path makes
    non-finite is non-finite here; where the fp32 path clamps an infinite intermediate back to a
    finite value (SwiGLU's +-limit), the output is either that value (within tolerance) or NaN.
    Case 1: +-inf on an up row (clamped to +-7 in the fp32 path). Case 2: nibbles -1.0 against a
    positive x on a gate row of a chosen expert: gate = -inf, glu = -inf / inf = NaN, so that
    expert's whole down product is NaN."""
    H, I, E = 64, 64, 4
    L = syn.make_layer(H, I, E, seed=370, scale_lo=120, scale_hi=124)
    d = GpuMoeDispatcher(H, I, 7.0)
    x = (np.abs(syn.hidden(1, H, seed=371)) + 0.5).astype(np.float32)
    gs = L["gu_scales"].copy()
    gb = L["gu_blocks"].copy()
    gs[:, 11, 0] = 255          # up row of h[5]
    gb[:, 11, 0, :] = 0x22
    L["gu_scales"], L["gu_blocks"] = gs, gb
    d.preload_layer(0, L)
    d.set_fused_decode(mode)
    want, _, _, _ = orc.moe_layer(x, L, 2)
    got = d.layer_forward(0, x, 2)
    assert np.all(np.isfinite(want))
    if not np.all(np.isnan(got)):
        assert_rel_l2(got, want, f"clamped inf mode {mode}")
    gs[1, 10, 0] = 255          # gate row of h[5] of expert 1
    gb[1, 10, 0, :] = 0xAA
    L["gu_scales"], L["gu_blocks"] = gs, gb
    d.preload_layer(0, L)
    want, _, idx, _ = orc.moe_layer(x, L, E)
    got = d.layer_forward(0, x, E)
    assert 1 in idx[0] and not np.any(np.isfinite(want))
    assert not np.any(np.isfinite(got))
    d.close()


def test_one_launch_tiny_grids_in_sequence(orc):
    """A layer so small that the one-launch kernel has fewer blocks than logit copies (k gate_up
    blocks + 4 down blocks): consecutive tokens with different routings and k in one context
    must each match the oracle, so no copy or flag left by one launch is taken for the next's."""
    H, I, E = 64, 32, 40
    L = syn.make_layer(H, I, E, seed=360, scale_lo=120, scale_hi=124)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    d.set_fused_decode(2)
    for i, k in enumerate((1, 4, 2, 3, 4, 1, 4)):
        x = syn.hidden(1, H, seed=900 + i)
        want, _, idx, _ = orc.moe_layer(x, L, k)
        gidx, _ = d.router_topk(0, x, k)
        assert np.array_equal(gidx, idx)
        assert_rel_l2(d.layer_forward(0, x, k), want, f"call {i} k={k}")
    d.close()


# ---------------------------------------------------------------- committed fixture

@pytest.mark.parametrize("fused", [2, 1, 0])
def test_tiny_layer_fixture(fused):
    """The committed tiny layer (tests/golden/tiny_layer.npz, float64 numpy restatement):
    indices exact, outputs within the matmul tolerance, on both single-token paths."""
    import os
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_layer.npz"))
    lay = {k: f[k] for k in f.files}
    H, I, E, k = int(f["H"]), int(f["I"]), int(f["E"]), int(f["k"])
    lay.update(H=H, I=I, E=E)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, lay)
    d.set_fused_decode(fused)
    idx, w = d.router_topk(0, f["x"], k)
    assert np.array_equal(idx, f["idx"])
    assert np.allclose(w, f["w"], rtol=1e-5)
    for t in range(3):
        assert_rel_l2(d.layer_forward(0, f["x"][t:t + 1], k)[0], f["y"][t], f"token {t}")
    assert_rel_l2(d.layer_forward(0, f["x"], k), f["y"], "3 tokens")
    d.close()


# ---------------------------------------------------------------- grouped GEMM (batches)

@pytest.mark.parametrize("shape", [(512, 512, 16, 4, 300), (256, 128, 8, 2, 2), (1024, 512, 32, 4, 129),
                                   (256, 256, 8, 4, 64)])
def test_batch_gemm_matches_oracle_and_gemv(orc, shape):
    """Batches through the grouped GEMM (block-scaled fp4 x fp8 MFMA, 3 activation terms) vs the
    fp32 oracle (1e-3) and vs the per-tile GEMV path (bf16 hi+lo activations, 2e-4): uneven
    expert loads, partial column tiles, partial row blocks; 64-, 32- and 16-entry column tiles
    (mean entries per expert 75, 32, 16 and 1)."""
    H, I, E, k, T = shape
    L = syn.make_layer(H, I, E, seed=400 + T, scale_lo=120, scale_hi=126, router_sigma=0.1)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    x = syn.hidden(T, H, seed=401 + T)
    want, _, idx, _ = orc.moe_layer(x, L, k)
    gidx, _ = d.router_topk(0, x, k)
    assert np.array_equal(gidx, idx)
    d.set_batch_gemm(2)
    got = d.layer_forward(0, x, k)
    assert_rel_l2(got, want, f"gemm {shape}")
    d.set_batch_gemm(0)
    ref = d.layer_forward(0, x, k)
    assert rel_l2(got, ref) < 2e-4
    d.close()


def test_batch_gemm_block_shapes_identical(orc):
    """Every block shape (large-batch 8 wavefronts as 4 x 2 or 8 x 1; the 512 x 128 block of 4
    wavefronts of 256 rows x 64 entries; forced 256-row x 32- and
    16-entry blocks; 128-row blocks of 4 or 2 wavefronts, the 2-row-tile one for down only)
    accumulates every output in the same K and term order: identical results."""
    H, I, E, k, T = 512, 512, 16, 4, 300
    L = syn.make_layer(H, I, E, seed=410, scale_lo=120, scale_hi=126, router_sigma=0.1)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    x = syn.hidden(T, H, seed=411)
    d.set_batch_gemm(2)
    outs = []
    shapes = [(0, 0), (1, 0), (2, 0), (3, 0), (4, 0), (5, 0), (6, 0), (7, 0), (8, 0), (0, 4), (2, 5), (5, 4),
              (7, 6), (8, 8), (11, 11), (0, 11), (12, 12), (13, 13), (12, 0), (0, 13), (14, 14), (14, 0), (0, 14),
              (15, 15)]
    for shape, down in shapes:
        d.set_gemm_shape(shape, down)
        outs.append(d.layer_forward(0, x, k))
    d.set_gemm_shape(0)
    for (shape, down), o in zip(shapes[1:], outs[1:]):
        assert np.array_equal(outs[0], o), f"shape {shape} down {down}"
    want = orc.moe_layer(x, L, k)[0]
    assert_rel_l2(outs[1], want, "gemm shape 1")
    # the 32 x 32 x 64 form (code 10) sums 64 products per MFMA where the others sum 128: the same
    # products, another f32 summation order
    for shape, down in [(10, 10), (1, 10), (0, 10)]:
        d.set_gemm_shape(shape, down)
        o = d.layer_forward(0, x, k)
        e = rel_l2(o, outs[0])
        assert e < 2e-5, f"shape {shape} down {down}: {e:.2e} from the 16 x 16 x 128 shapes"
        assert_rel_l2(o, want, f"gemm shape {shape} down {down}")
    d.set_gemm_shape(0)
    d.close()


@pytest.mark.parametrize("shape", [(512, 512, 16, 4, 300), (256, 128, 8, 2, 2), (1024, 512, 32, 4, 129),
                                   (256, 256, 8, 4, 64), (512, 1024, 64, 4, 48), (1024, 2880, 8, 4, 2),
                                   (64, 64, 8, 4, 40), (256, 256, 4, 4, 600)])
def test_batch_gemm_streamed_identical(orc, shape):
    """The streamed grouped GEMM (codes 12 and 13, and the default below 24 entries per expert:
    one workgroup per CU taking four units at a time from a contiguous share of 16-entry chunks
    x row groups, rings running on across rounds) against the 128 x 16 block (code 5): the same
    MFMAs in the same order, identical results; ragged expert loads (1 to 75 entries), experts
    with entries past one 16-entry chunk, rounds and workgroup ranges that cross chunks, K = 512
    (4 of the 24 loop positions real) and K = 2880 (down: 23); H = I = 64, where gate_up has 2
    units per chunk, falls back to the block shapes. The wide streamed form (code 14: units of a
    group of up to 5 chunks of one expert) on the same cases, including 600 entries per expert (8
    groups each, rounds of 2 units, most workgroups without a round)."""
    H, I, E, k, T = shape
    L = syn.make_layer(H, I, E, seed=470 + T, scale_lo=120, scale_hi=126, router_sigma=0.1)
    d = GpuMoeDispatcher(H, I, 7.0)
    try:
        d.preload_layer(0, L)
        x = syn.hidden(T, H, seed=471 + T)
        d.set_batch_gemm(2)
        d.set_gemm_shape(5, 5)
        base = d.layer_forward(0, x, k)
        for shape_c, down in [(12, 12), (13, 13), (12, 5), (5, 13), (0, 0), (14, 14), (14, 12), (5, 14)]:
            d.set_gemm_shape(shape_c, down)
            o = d.layer_forward(0, x, k)
            assert np.array_equal(base, o), f"{shape}: shape {shape_c} down {down}"
            # the router's grouping in place of the streamed GEMM's own (small batches)
            d.set_local_group(0)
            o = d.layer_forward(0, x, k)
            d.set_local_group(1)
            assert np.array_equal(base, o), f"{shape}: shape {shape_c} down {down}, router grouping"
        d.set_gemm_shape(0)
        want = orc.moe_layer(x, L, k)[0]
        assert_rel_l2(base, want, f"gemm {shape}")
    finally:
        d.close()


def test_batch_gemm_block_shapes_identical_20b(orc, disp20, layer20):
    """The block shapes at the 20B dimensions, where K = 2880 takes 23 steps: with a ring of
    three slots the loop ends with the repeat of the last step still loading into the slot that
    the gate_up epilogue stages its SwiGLU values in (a missing wait there corrupted the h
    records of the small-block shapes)."""
    x = syn.hidden(64, H20, seed=430)
    want = orc.moe_layer(x, layer20, 4)[0]
    disp20.set_batch_gemm(2)
    outs = []
    shapes = [(0, 0), (3, 3), (5, 5), (6, 6), (7, 7), (2, 2), (5, 4), (12, 12), (13, 13), (12, 5), (14, 14),
              (14, 5), (15, 15), (15, 5), (5, 15), (16, 16), (17, 17), (18, 18), (19, 19)]
    for shape, down in shapes:
        disp20.set_gemm_shape(shape, down)
        outs.append(disp20.layer_forward(0, x, 4))
    disp20.set_gemm_shape(10, 10)  # the 32 x 32 x 64 form; experts average 8 entries, so most
    o32 = disp20.layer_forward(0, x, 4)  # tiles hold fewer than 32 (their second wavefront pair idles)
    disp20.set_gemm_shape(0)
    disp20.set_batch_gemm(1)
    assert_rel_l2(outs[0], want, "20B gemm T=64")
    for (shape, down), o in zip(shapes[1:], outs[1:]):
        assert np.array_equal(outs[0], o), f"shape {shape} down {down}"
    assert rel_l2(o32, outs[0]) < 1e-4
    assert_rel_l2(o32, want, "20B gemm T=64 shape 10")


def test_batch_gemm_pipelined_k3072(orc):
    """The pipelined 512 x 64 step at its other compile-time length, 24 K-steps (K = 3072 for
    both GEMMs: the default there, codes 15-17 forced), against the 128 x 16 block (code 5) and
    the 256 x 32 block of 4 wavefronts (code 2): the same MFMAs in the same order, identical
    results; sampled tokens within the tolerance of the oracle."""
    H = I = 3072
    E, k, T = 8, 4, 160  # 80 entries per expert: the 512 x 64 block
    L = syn.make_layer(H, I, E, seed=490, scale_lo=120, scale_hi=126, router_sigma=0.1)
    d = GpuMoeDispatcher(H, I, 7.0)
    try:
        d.preload_layer(0, L)
        x = syn.hidden(T, H, seed=491)
        d.set_batch_gemm(2)
        d.set_gemm_shape(5, 5)
        base = d.layer_forward(0, x, k)
        for shape_c, down in [(0, 0), (15, 15), (16, 16), (17, 17), (18, 18), (19, 19), (18, 0), (2, 2)]:
            d.set_gemm_shape(shape_c, down)
            o = d.layer_forward(0, x, k)
            assert np.array_equal(base, o), f"K=3072: shape {shape_c} down {down}"
        d.set_gemm_shape(0)
        sample = np.arange(0, T, 20)
        want = orc.moe_layer(x[sample], L, k)[0]
        assert_rel_l2(base[sample], want, "K=3072 sampled tokens vs oracle")
    finally:
        d.close()


def _prefill_parity(orc, d, layer, T, seed, n_sample):
    """A T-token layer through the default path (the 8-token router blocks, the grouped GEMM at
    the real K: the 512-row x 64-entry block at 512 entries per expert, the wide streamed form at
    64): top-k indices of every token exact against the
    oracle's router; n_sample tokens (per-token outputs do not depend on the other tokens)
    within the tolerance of the oracle; the whole output within 6e-4 of the GEMV path; the
    other large-batch block shape and the 4-wavefront shapes bit-identical.
    The GEMV path is exact to 2^-17 and the grouped GEMM's 3 E2M3 terms to ~2^-14 of each
    block maximum; on this synthetic layer the gate/up pre-activations reach hundreds against
    the SwiGLU clamp of 7, so the x split's error is amplified where gate or up sits in the
    SwiGLU's sloped range: a float64 model of the split on 16 of these tokens gives 3.1e-4
    relative L2 on the layer output (x split alone 3.1e-4, h split alone 7e-6)."""
    E, k = layer["E"], 4
    x = syn.hidden(T, H20, seed=seed)
    logits = orc.router_logits(layer["router_w"], layer["router_b"], x, E, H20)
    widx, _, _, _ = orc.topk(logits, k)
    gidx, _ = d.router_topk(0, x, k)
    assert np.array_equal(gidx, widx)
    counts = np.bincount(widx.ravel(), minlength=E)
    assert counts.mean() >= 48, "the default shape needs experts averaging 48+ entries"
    d.set_batch_gemm(1)
    d.set_gemm_shape(0)
    got = d.layer_forward(0, x, k)
    sample = np.random.default_rng(seed + 1).choice(T, n_sample, replace=False)
    sample.sort()
    want, _, idx_s, _ = orc.moe_layer(x[sample], layer, k)
    assert np.array_equal(idx_s, widx[sample])
    assert_rel_l2(got[sample], want, f"T={T} E={E} sampled tokens vs oracle")
    d.set_batch_gemm(0)
    ref = d.layer_forward(0, x, k)
    d.set_batch_gemm(1)
    e = rel_l2(got, ref)
    assert e < 6e-4, f"T={T} E={E} grouped GEMM vs GEMV path {e:.2e}"
    for shape, down in [(1, 0), (8, 8), (2, 2), (3, 3), (0, 4), (11, 11), (14, 14), (0, 14), (15, 15), (15, 0), (0, 15), (16, 16), (17, 17), (18, 18), (19, 19), (18, 0), (0, 18)]:
        d.set_gemm_shape(shape, down)
        o = d.layer_forward(0, x, k)
        assert np.array_equal(got, o), f"T={T} E={E} shape {shape} down {down}"
    # the 32 x 32 x 64 form: the same products in another f32 summation order (an h value whose
    # third E2M3 term rounds the other way moves its entry by ~2^-14 of the block maximum)
    d.set_gemm_shape(10, 10)
    o = d.layer_forward(0, x, k)
    d.set_gemm_shape(0)
    e = rel_l2(o, got)
    assert e < 1e-4, f"T={T} E={E} shape 10: {e:.2e} from the default shape"
    assert_rel_l2(o[sample], want, f"T={T} E={E} shape 10 sampled tokens vs oracle")


def test_prefill_4096_tokens_20b(orc, disp20, layer20):
    """Config 4's layer shape: 4096 tokens of a 20B layer (32 experts, 512 entries each on
    average)."""
    _prefill_parity(orc, disp20, layer20, 4096, seed=450, n_sample=64)


def test_prefill_2048_tokens_120b(orc):
    """Config 5b: 2048 tokens of a 120B layer (128 experts, 64 entries each on average)."""
    L = syn.make_layer(H20, I20, 128, seed=460)
    d = GpuMoeDispatcher(H20, I20, 7.0)
    try:
        d.preload_layer(0, L)
        _prefill_parity(orc, d, L, 2048, seed=461, n_sample=32)
    finally:
        d.close()


# ---------------------------------------------------------------- quantized activations (opt-in)

def test_prefill_partial_router_block_20b(orc, disp20, layer20):
    """2053 tokens, a multiple of 8 plus 5: the last 8-token router block holds 5 tokens (its
    idle top-k wavefronts and the wavefronts that write the GEMM records see a partial block).
    Top-k indices of every token exact against the oracle's router; tokens of the first, the
    last full and the partial block within the tolerance of the oracle, on the exact path and on
    the quantized one (against the MXFP6 oracle)."""
    T, k = 2053, 4
    x = syn.hidden(T, H20, seed=470)
    logits = orc.router_logits(layer20["router_w"], layer20["router_b"], x, E20, H20)
    widx, _, _, _ = orc.topk(logits, k)
    gidx, _ = disp20.router_topk(0, x, k)
    assert np.array_equal(gidx, widx)
    rows = np.array([0, 1, 7, 2040, 2047, 2048, 2049, 2050, 2051, 2052])
    disp20.set_batch_gemm(1)
    disp20.set_gemm_shape(0)
    got = disp20.layer_forward(0, x, k)
    want, _, idx, _ = orc.moe_layer(x[rows], layer20, k)
    assert np.array_equal(idx, widx[rows])
    assert_rel_l2(got[rows], want, "T=2053 exact split")
    disp20.set_act_quant(1)
    try:
        gq = disp20.layer_forward(0, x, k)
    finally:
        disp20.set_act_quant(0)
    wq, _, _, _ = orc.moe_layer_mxfp6(x[rows], layer20, k)
    assert_rel_l2(gq[rows], wq, "T=2053 quantized", tol=2e-4)


def _act_quant_check(orc, d, layer, x, k, what, n_sample=None, seed=0, shapes=(), shapes_close=()):
    """MOE_OPT_ACT_QUANT 1: top-k exact; the output (or n_sample sampled tokens) within the
    tolerance of the fp32 path on MXFP6 activations (orc.moe_layer_mxfp6: the GPU and the oracle
    quantize the same x to the same codes; h differs by summation order, so an h value at a
    rounding midpoint may take the neighbouring code); the forced shapes bit-identical; the
    exact mode afterwards bit-identical to before (the h records are re-laid out)."""
    d.set_batch_gemm(1)
    d.set_gemm_shape(0)
    exact = d.layer_forward(0, x, k)
    d.set_act_quant(1)
    try:
        got = d.layer_forward(0, x, k)
        for shape, down in shapes:
            d.set_gemm_shape(shape, down)
            assert np.array_equal(d.layer_forward(0, x, k), got), f"{what}: shape {shape} down {down}"
        for shape, down in shapes_close:  # the 32 x 32 x 64 form: another f32 summation order
            d.set_gemm_shape(shape, down)
            e = rel_l2(d.layer_forward(0, x, k), got)
            assert e < 2e-4, f"{what}: shape {shape} down {down}: {e:.2e}"
        d.set_gemm_shape(0)
    finally:
        d.set_act_quant(0)
    assert np.array_equal(d.layer_forward(0, x, k), exact), f"{what}: exact mode after the quantized one"
    rows = np.arange(x.shape[0])
    if n_sample:
        rows = np.sort(np.random.default_rng(seed).choice(x.shape[0], n_sample, replace=False))
    want, _, idx, _ = orc.moe_layer_mxfp6(x[rows], layer, k)
    gidx, _ = d.router_topk(0, x[rows], k)
    assert np.array_equal(gidx, idx)
    # measured ~1e-7 (no code differs); one h value on its neighbouring code moves its token's
    # output by ~1e-3 / sqrt(entries), so 2e-4 leaves room for a few
    e = assert_rel_l2(got[rows], want, f"{what} vs mxfp6 oracle", tol=2e-4)
    strict = rel_l2(got[rows], orc.moe_layer(x[rows], layer, k)[0])
    print(f"{what}: rel-L2 {e:.2e} vs the MXFP6 oracle, {strict:.2e} vs the fp32 path")
    return e


@pytest.mark.parametrize("shape", [(512, 512, 16, 4, 300), (256, 256, 8, 4, 64)])
def test_act_quant_small(orc, shape):
    H, I, E, k, T = shape
    L = syn.make_layer(H, I, E, seed=480 + T, scale_lo=120, scale_hi=126, router_sigma=0.1)
    d = GpuMoeDispatcher(H, I, 7.0)
    try:
        d.preload_layer(0, L)
        x = syn.hidden(T, H, seed=481 + T)
        _act_quant_check(orc, d, L, x, k, f"act_quant {shape}",
                         shapes=[(1, 0), (5, 0), (7, 0), (5, 7), (1, 5), (9, 9), (0, 9), (12, 12), (13, 0),
                                 (14, 14), (14, 0)],
                         shapes_close=[(10, 10)])
    finally:
        d.close()


def test_act_quant_20b_decode64_and_prefill(orc, disp20, layer20):
    """The 20B layer at 64 tokens (128- and 256-row shapes), at 512 tokens (experts averaging 64
    entries: the 512-row x 64-entry shape at K = 2880) and at 4096 tokens (512 entries: the
    512 x 128 block), quantized activations."""
    _act_quant_check(orc, disp20, layer20, syn.hidden(64, H20, seed=490), 4, "act_quant 20B T=64",
                     shapes=[(5, 5), (7, 7), (7, 5), (12, 12), (13, 13)])
    _act_quant_check(orc, disp20, layer20, syn.hidden(512, H20, seed=493), 4, "act_quant 20B T=512",
                     n_sample=32, seed=494, shapes=[(1, 0), (9, 9), (0, 9), (14, 14)], shapes_close=[(10, 10)])
    _act_quant_check(orc, disp20, layer20, syn.hidden(4096, H20, seed=491), 4, "act_quant 20B T=4096",
                     n_sample=48, seed=492, shapes=[(1, 0), (1, 7), (9, 9), (9, 0)])


def test_act_quant_option_checks(disp20):
    from silentotithrandousha_amd._ffi import MoeError
    with pytest.raises(MoeError, match="ACT_QUANT"):
        disp20.set_act_quant(2)


def test_empty_batches(orc, disp20, layer20):
    """Zero tokens: every forward entry point succeeds and writes nothing (the reference's loops
    over tokens and slots simply do not run); the batched dispatch over an empty expert list
    returns zeros (moe_dispatch.rs:473-607 sums an empty list); the next real call still matches
    the oracle."""
    x0 = np.zeros((0, H20), np.float32)
    assert disp20.layer_forward(0, x0, 4).shape == (0, H20)
    idx, w = disp20.router_topk(0, x0, 4)
    assert idx.shape == (0, 4) and w.shape == (0, 4)
    sentinel = np.full(64, 7.0, np.float32)
    yd = DeviceBuffer.from_array(sentinel)
    xd = DeviceBuffer.from_array(np.zeros(64, np.float32))
    disp20.layer_forward_device(0, xd, 0, 4, yd)
    disp20.synchronize()
    assert np.array_equal(yd.download(np.float32, 64), sentinel)
    x1 = syn.hidden(1, H20, seed=475)[0]
    assert np.array_equal(disp20.dispatch_experts_batched(x1, []), np.zeros(H20, np.float32))
    want, _, widx, _ = orc.moe_layer(x1[None], layer20, 4)
    gidx, _ = disp20.router_topk(0, x1[None], 4)
    assert np.array_equal(gidx, widx)
    assert_rel_l2(disp20.layer_forward(0, x1[None], 4), want, "after the empty calls")


def test_invalid_calls_leave_context_usable(orc, disp20, layer20):
    """Calls refused for their arguments (top-k 0 or above the expert count, a layer never
    loaded) change nothing: the next valid call of each size still matches the oracle."""
    from silentotithrandousha_amd._ffi import MoeError
    for T in (1, 64):
        x = syn.hidden(T, H20, seed=470 + T)
        for bad_k in (0, 33, 1 << 40):
            with pytest.raises(MoeError, match="top_k"):
                disp20.layer_forward(0, x, bad_k)
        for bad_k in (0, 33):
            with pytest.raises(MoeError, match="top_k"):
                disp20.router_topk(0, x, bad_k)
        with pytest.raises(MoeError):
            disp20.layer_forward(5, x, 4)
        want, _, idx, _ = orc.moe_layer(x, layer20, 4)
        gidx, _ = disp20.router_topk(0, x, 4)
        assert np.array_equal(gidx, idx)
        assert_rel_l2(disp20.layer_forward(0, x, 4), want, f"after refused calls T={T}")


@pytest.mark.parametrize("H,E", [(64, 8), (64, 32), (512, 128)])
def test_batch_grouping_in_router_and_separate(orc, H, E):
    """The router's last block groups the entries by expert when its x staging holds the
    grouping's LDS (18 E ints within one token's staging: H = 64 with 8 experts, 512 with 128),
    else the separate grouping kernel runs (H = 64 with 32 experts); both give the oracle's
    routing and outputs, on the GEMM and the GEMV paths, over repeated calls."""
    I, k = 32, 4
    L = syn.make_layer(H, I, E, seed=440 + E, scale_lo=120, scale_hi=126, router_sigma=0.2)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    for T in (2, 5, 70):
        x = syn.hidden(T, H, seed=441 + T)
        want, _, idx, _ = orc.moe_layer(x, L, k)
        for gemm in (2, 0):
            d.set_batch_gemm(gemm)
            for _ in range(2):
                got = d.layer_forward(0, x, k)
                assert_rel_l2(got, want, f"H={H} E={E} T={T} gemm {gemm}")
        gidx, _ = d.router_topk(0, x, k)
        assert np.array_equal(gidx, idx)
    d.close()


def test_batch_gemm_adaptive_dropped_slots(orc):
    """Adaptive top-k drops slots: their entries are absent from the expert groups."""
    H, I, E = 256, 128, 8
    L = syn.make_layer(H, I, E, seed=420, scale_lo=116, scale_hi=122, router_sigma=0.2)
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, L)
    ad = orc.Adaptive(1, 1, 0.7, 0.4, 0.85)
    d.set_adaptive_topk(True, 1, 0.7, 0.4, 0.85)
    d.set_batch_gemm(2)
    xs = syn.hidden(40, H, seed=421, sigma=1.0)
    want, _, idx, _ = orc.moe_layer(xs, L, 4, adaptive=ad)
    assert (idx < 0).any()
    got = d.layer_forward(0, xs, 4)
    assert_rel_l2(got, want, "adaptive batch gemm")
    # the streamed GEMM, whose workgroups group the entries themselves (dropped slots skipped),
    # and with the router's grouping: the same bits
    d.set_gemm_shape(12, 12)
    o_local = d.layer_forward(0, xs, 4)
    d.set_local_group(0)
    o_router = d.layer_forward(0, xs, 4)
    d.set_local_group(1)
    d.set_gemm_shape(0)
    assert np.array_equal(o_local, got) and np.array_equal(o_router, got)
    d.close()


# ---------------------------------------------------------------- safetensors loader

def test_load_safetensors_layer(orc, tmp_path):
    """A checkpoint layer in GPT-OSS tensor names (weights.rs:262-283), split over two shards
    (experts in one, router in the other, as the reference searches every shard): loaded through
    moe_load_safetensors_layer it gives the same bits as preload_layer on the decoded tensors
    (bf16 biases widened to f32), both within tolerance of the oracle; a wrong shape is refused
    naming the tensor."""
    from tests.helpers import gpt_oss_layer_tensors, write_safetensors
    from silentotithrandousha_amd._ffi import MoeError
    H, I, E, li = 64, 64, 8, 3
    L = syn.make_layer(H, I, E, seed=400)
    L["gu_bias"] = syn.bf16_round(L["gu_bias"])
    L["d_bias"] = syn.bf16_round(L["d_bias"])
    t = gpt_oss_layer_tensors(L, li)
    experts = {k: v for k, v in t.items() if ".experts." in k}
    router = {k: v for k, v in t.items() if ".router." in k}
    write_safetensors(tmp_path / "model-00001-of-00002.safetensors", experts, metadata={"format": "pt"})
    gamma = syn.bf16_round((1 + 0.1 * np.random.default_rng(402).standard_normal(H)).astype(np.float32))
    router[f"model.layers.{li}.post_attention_layernorm.weight"] = ("BF16", syn.bf16_bits(gamma), (H,))
    write_safetensors(tmp_path / "model-00002-of-00002.safetensors", router, pad=7)
    x = syn.hidden(3, H, seed=401)
    d1 = GpuMoeDispatcher(H, I, 7.0)
    d1.load_safetensors_layer(str(tmp_path), li, E)
    d2 = GpuMoeDispatcher(H, I, 7.0)
    d2.preload_layer(li, L)
    for mode in (2, 0):
        d1.set_fused_decode(mode)
        d2.set_fused_decode(mode)
        for T in (1, 3):
            got = d1.layer_forward(li, x[:T], 4)
            assert_bit_exact(got, d2.layer_forward(li, x[:T], 4), f"loader vs preload mode {mode} T={T}")
            want, _, _, _ = orc.moe_layer(x[:T], L, 4)
            assert_rel_l2(got, want, f"loader vs oracle mode {mode} T={T}")
    d2.preload_norm(li, gamma, 1e-5)
    for T in (1, 3):
        assert_bit_exact(d1.block_forward(li, x[:T], 4), d2.block_forward(li, x[:T], 4), f"loaded norm T={T}")
    bad = dict(experts)
    k = f"model.layers.{li}.mlp.experts.down_proj_scales"
    bad[k] = ("U8", L["d_scales"][:, :, :1], (E, H, 1))
    write_safetensors(tmp_path / "bad.safetensors", bad)
    with pytest.raises(MoeError, match="down_proj_scales"):
        d1.load_safetensors_layer([str(tmp_path / "bad.safetensors"), str(tmp_path / "model-00002-of-00002.safetensors")], li, E)
    d1.close()
    d2.close()


# ---------------------------------------------------------------- RMSNorm + router + residual

@pytest.mark.parametrize("T", [1, 2, 64])
def test_block_forward_norm_and_residual(orc, disp20, layer20, T):
    """out = x + MoE(RMSNorm(x) gamma) (executables.rs:260-317, session.rs:483-493, 982-994).
    The norm is bit-exact with the oracle's canonical order: for every path (one launch with the
    norm fused into its router and gate_up blocks, two launches, the batch path) the block gives
    the same bits as x + layer_forward(oracle RMSNorm(x)); and within tolerance of the oracle's
    whole block."""
    rng = np.random.default_rng(500 + T)
    gamma = (1 + 0.2 * rng.standard_normal(H20)).astype(np.float32)
    disp20.preload_norm(0, gamma, 1e-5)
    x = (syn.hidden(T, H20, seed=501 + T) * 3).astype(np.float32)
    n = orc.rms_norm(x, gamma, 1e-5)
    want, _, idx, _ = orc.moe_block(x, layer20, 4, gamma, 1e-5)
    for mode in (MODES if T == 1 else [2]):
        disp20.set_fused_decode(mode)
        got = disp20.block_forward(0, x, 4)
        ref = disp20.layer_forward(0, n, 4)
        assert_bit_exact(got, (x + ref).astype(np.float32), f"block vs x + layer(n) T={T} mode {mode}")
        assert_rel_l2(got - x, want - x, f"block vs oracle T={T} mode {mode}")
    disp20.set_fused_decode(2)


def test_block_forward_needs_norm():
    from silentotithrandousha_amd._ffi import MoeError
    H, I, E = 64, 32, 4
    d = GpuMoeDispatcher(H, I, 7.0)
    d.preload_layer(0, syn.make_layer(H, I, E, seed=510))
    with pytest.raises(MoeError, match="RMSNorm"):
        d.block_forward(0, syn.hidden(1, H, seed=511), 2)
    d.close()
