"""Host-side bounds replay of the batch router kernel k_route (silentotithrandousha_amd/csrc/
kernels.hip, `k_route<KI, TB>` and its launcher `launch_route_ki`): every global and LDS index
the kernel computes, enumerated over the whole grid of a launch, against the sizes the library
allocates (moe_api.cpp `carve_work`, `router_bytes`) and the LDS the launch reserves. Covers x
staging, the xsplit rows, the router-weight loads, the logit table, the grouped-GEMM activation
records (rec_split_block's byte offsets), the per-wavefront top-k stores, the grouping's
per-block counts and ranks, the last block's count table in the x staging area and its scatter
(a value-dependent index: ge = base[e] + prefix over blocks + rank, replayed on random routings,
so it must land on every entry exactly once), and the per-block timing stamps of the
realtime-counter trace copy (`rt_ts[blockIdx.x * 16 + i]`, i <= 9, over 4096 * 16 entries).

It is a model of the kernel's index arithmetic, not the kernel: it restates each index
expression with a citation of the code it follows, so a change to those expressions needs the
same change here."""
import numpy as np
import pytest

K_ROUTE_THREADS = 1024          # kernels.hip: kRouteThreads
K_ROUTE_TOKENS = 8              # kernels.hip: kRouteTokens
K_MAX_EXPERTS = 256             # kernels.hpp: kMaxExperts
K_MAX_TOPK = 16                 # kernels.hpp: kMaxTopK
K_GEMM_NS = 24                  # kernels.hpp: kGemmNs
LDS_BYTES = 160 * 1024          # gfx950 LDS per workgroup
RT_STAMPS = 4096 * 16           # the trace copy's rt_ts array


def rec_step(nt):               # kernels.hpp GemmRecT<NT>::kStep / kBytes
    return nt * 96 + 16


def rec_offsets(nt, blk):
    """Byte ranges [lo, hi) rec_split_block writes for block blk (device.hpp rec_split_block,
    GemmRecT::dword / ::scale)."""
    st, i = blk >> 2, blk & 3
    out = []
    for t in range(nt):
        base = st * rec_step(nt) + t * 96
        out.append((base + 16 * i, base + 16 * i + 16))            # dwords 0-3: uint4
        out.append((base + 64 + 8 * i, base + 64 + 8 * i + 8))     # dwords 4-5: uint2
        sc = st * rec_step(nt) + nt * 96 + 4 * t + i
        out.append((sc, sc + 1))                                   # the scale byte
    return out


def launch_shape(T, H):
    """launch_route_ki: TB and the dynamic LDS of the launch."""
    nq = ((H + 63) // 64 + 7) // 8
    hp = nq * 8 * 64                                   # route_hp(H), floats
    if T >= 2048 and K_ROUTE_TOKENS * hp * 4 <= 144 * 1024:
        return nq, hp, K_ROUTE_TOKENS, K_ROUTE_TOKENS * hp * 4
    return nq, hp, 1, hp * 4


def static_lds(TB):
    """k_route's __shared__ arrays in bytes: s_logit, s_p, s_order, s_w, s_sel, s_last, s_cnt."""
    return 4 * (TB * K_MAX_EXPERTS + K_MAX_EXPERTS + TB * K_MAX_TOPK * 2 + TB + 1 + K_MAX_EXPERTS)


def check(name, idx, size):
    idx = np.asarray(idx)
    if idx.size:
        lo, hi = int(idx.min()), int(idx.max())
        assert lo >= 0 and hi < size, f"{name}: index range [{lo}, {hi}] outside [0, {size})"


def replay(T, E, k, H, rec_terms=3, xsplit=True, seed=0, stamps=False):
    nq, Hp, TB, dyn = launch_shape(T, H)
    KI = nq if nq in (1, 2, 6) else 0
    grid = (T + TB - 1) // TB
    N = T * k
    nw = K_ROUTE_THREADS // 64
    assert dyn + static_lds(TB) <= LDS_BYTES, "LDS of the launch"
    per_wave = k <= 4 and E <= 128
    assert TB < nw                                       # the kernel's static_assert
    lane = np.arange(64)
    rec_bytes = K_GEMM_NS * rec_step(rec_terms)
    assert H <= 128 * K_GEMM_NS                           # launch_route: xrec needs H <= 128 kGemmNs
    # routing of the replay: k distinct experts per token
    rng = np.random.default_rng(seed)
    order = np.argsort(rng.random((T, E)), axis=1)[:, :k].astype(np.int64)
    blk_count = np.zeros((grid, E), np.int64)
    rank = np.full(N, -1, np.int64)
    for b in range(grid):
        t0 = b * TB
        nt = min(TB, T - t0)
        # x loads and staging (kernels.hip k_route: xv[tb][q], stage(tb, k, xv))
        tb = np.arange(nt)[:, None]
        kk = np.arange(Hp)[None, :]
        check("x", ((t0 + tb) * H + kk)[np.broadcast_to(kk < H, (nt, Hp))], T * H)
        check("s_x staging", (tb * Hp + kk).ravel(), dyn // 4)
        if xsplit:
            kh = np.arange(H)[None, :]
            check("xsplit", np.concatenate([((t0 + tb) * 2 * H + kh).ravel(),
                                            ((t0 + tb) * 2 * H + H + kh).ravel()]), T * 2 * H)
        # router weights (uint4 units): the first expert's (TB == 1) and the pair loads
        if KI:
            w_u4 = E * nq * 64
            if TB == 1:
                wv = np.arange(min(nw, E))[:, None, None]
                check("router w (first)", (wv * nq * 64 + lane[None, :, None] + 64 * np.arange(KI)[None, None, :]).ravel(), w_u4)
            e = np.arange(0, E, 1)[:, None]                  # every e some wavefront takes
            e1 = np.minimum(e + nw, E - 1)
            q = 64 * np.arange(KI)[None, :]
            check("router w (pair)", np.concatenate([(e * nq * 64 + q).ravel(), (e1 * nq * 64 + q + 63).ravel()]), w_u4)
            xs = lane[:, None] + 64 * (8 * np.arange(KI)[None, :, None] + np.arange(8)[None, None, :]).reshape(1, -1)
            check("router x reads", xs.ravel(), Hp)
        check("s_logit", [(nt - 1) * K_MAX_EXPERTS + E - 1], TB * K_MAX_EXPERTS)
        # activation records: a lane per 32-value block (write_records)
        u = np.arange(nt * 4 * K_GEMM_NS)
        rtb, blk = u // (4 * K_GEMM_NS), u % (4 * K_GEMM_NS)
        k0 = 32 * blk
        rd = (rtb * Hp)[:, None] + k0[:, None] + 4 * np.arange(8)[None, :]
        ok = (k0[:, None] + 4 * np.arange(8)[None, :] + 3) < Hp
        check("records: staging reads", (rd + 3)[ok], dyn // 4)
        spans = np.array([rec_offsets(rec_terms, int(x_)) for x_ in range(4 * K_GEMM_NS)])  # [blk][n][2]
        lo = (t0 + rtb)[:, None] * rec_bytes + spans[blk][:, :, 0]
        hi = (t0 + rtb)[:, None] * rec_bytes + spans[blk][:, :, 1] - 1
        check("xrec", np.concatenate([lo.ravel(), hi.ravel()]), T * rec_bytes)
        # top-k stores
        t = t0 + np.arange(nt)[:, None]
        if per_wave:
            le = np.concatenate([lane[lane < E], lane[lane + 64 < E] + 64])
            check("logits", (t * E + le[None, :]).ravel(), T * E)
            check("s_logit top-k reads", le, K_MAX_EXPERTS)
        else:
            check("logits", (t * E + np.arange(E)[None, :]).ravel(), T * E)
        check("idx / wts", (t * k + np.arange(k)[None, :]).ravel(), N)
        # per-block counts and ranks (the table path's wavefront 0)
        ent = order[t0:t0 + nt].ravel()
        l = np.arange(nt * k)
        for j_, e_ in enumerate(ent):
            rank[t0 * k + j_] = blk_count[b, e_]
            blk_count[b, e_] += 1
        check("rank", t0 * k + l, N)
        check("blk_count", b * E + np.arange(E), T * E)
        if stamps:
            check("rt_ts stamps", b * 16 + np.array([0, 1, 3, 4, 5, 6, 9]), RT_STAMPS)
    # the last block: the count table in the x staging area, expert-major rows ld_bc apart
    ld_bc = grid + 1
    table = ld_bc * E + 2 * E <= TB * Hp
    if table:
        i = np.arange(grid * E)
        bi = i // E
        check("s_bc fill", (i - bi * E) * ld_bc + bi, ld_bc * E)
        check("s_tot / s_base", ld_bc * E + np.arange(2 * E), dyn // 4)
        pref = np.zeros((E, grid), np.int64)               # exclusive prefix over blocks
        pref[:, 1:] = np.cumsum(blk_count.T, axis=1)[:, :-1]
        tot = blk_count.sum(axis=0)
        base = np.concatenate([[0], np.cumsum(tot)[:-1]])  # expert_list_wave: expert id order
        n = np.arange(N)
        e = order.ravel()
        ge = base[e] + pref[e, (n // k) // TB] + rank
        check("entry_src / pos scatter", ge, N)
        assert np.array_equal(np.sort(ge), n), "the scatter writes every entry exactly once"
        # entries of one expert ordered by t k + slot
        for ex in range(E):
            sel = np.nonzero(e == ex)[0]
            assert np.all(np.diff(ge[sel]) == 1)
    else:
        # bucket_block in the staging area: (2 + 16) E ints, checked by the host (route_bucket_fits)
        assert 18 * E <= Hp
    return dict(TB=TB, grid=grid, table=table, dyn=dyn)


@pytest.mark.parametrize("T,E,k", [(1, 32, 4), (2, 32, 4), (64, 32, 4), (2053, 32, 4), (4096, 32, 4),
                                   (2048, 128, 4), (64, 128, 4), (37, 32, 16), (2048, 32, 1)])
def test_route_indices_in_bounds(T, E, k):
    replay(T, E, k, 2880, rec_terms=3, xsplit=T < 64, seed=T + E)


def test_route_trace_copy_configuration():
    """The configuration of the realtime-stamp trace copy: T = 4096, E = 32, k = 4 on the 20B
    shape, TB = 8, grid 512, dynamic LDS 8 Hp floats, the count table in the staging area; every
    index of the kernel and of the stamps in bounds, for both record forms."""
    for terms in (3, 1):
        r = replay(4096, 32, 4, 2880, rec_terms=terms, xsplit=False, seed=4096 + terms, stamps=True)
        assert (r["TB"], r["grid"], r["table"], r["dyn"]) == (8, 512, True, 8 * 3072 * 4)


def test_route_replay_detects_a_planted_overflow():
    """The replay's checks fire: a staging row one float longer than the launch's dynamic LDS."""
    with pytest.raises(AssertionError, match="s_x staging"):
        check("s_x staging", np.arange(8 * 3072 + 1), 8 * 3072)
