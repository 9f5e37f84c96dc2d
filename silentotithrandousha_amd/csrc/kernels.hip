// HIP kernels of the MXFP4 MoE path, written for gfx950 (CDNA4, wave64).
//
//   k_route        router GEMV in the canonical order + top-k + softmax renorm + bf16 split
//                  (session.rs:495-520, :818-841)
//   k_bucket       deterministic token -> expert grouping (stable counting sort)
//   k_expert_gemv  MXFP4 x bf16(hi,lo) on v_mfma_f32_16x16x32_bf16, one wavefront per
//                  16-row tile, with the gate_up SwiGLU epilogue (session.rs:101-117), the
//                  down bias + clamp epilogue (session.rs:119-123) or a raw output
//   k_combine      weighted sum over slots in rank order (session.rs:974-980)
//   k_dequant_*    bit-exact decode of weights.rs:350-371 (checkpoint or resident layout)
//   k_pack_*       checkpoint layout -> resident tile16 layout (layout.hpp)
//
// Numerics of the GEMV: the weight decode (v_cvt_scalef32_pk_bf16_fp4) is exact because
// E2M1 * 2^k has at most two significant bits; activations enter as x = hi + lo with hi, lo
// bf16 (16 significant bits, |x - (hi+lo)| <= 2^-17 |x|); products are exact and accumulate
// in f32 inside the MFMA.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device.hpp"
#include "kernels.hpp"

namespace moe {

// ------------------------------------------------------------------ router + top-k

constexpr int kRouteThreads = 1024;
constexpr int kRouteTokens = 8;  // tokens per block for large batches: the router weights load once per block

// Groups the T*k (token, slot) entries by expert, in one block of 1024 threads. Active
// experts are listed in ascending id; entries of one expert are ordered by t*k + slot.
// pos[t*k + slot] = entry index (or -1). LDS: s_count[E], s_base[E], s_wave[16][E].
template <bool kAgentLoads>  // idx written by other blocks of the same launch: agent-scope loads
__device__ __forceinline__ void bucket_block(const int32_t *idx, int T, int k, int E, int32_t *n_active,
                             int32_t *active_ids, int32_t *active_off, int32_t *entry_src,
                             int32_t *pos, int *s_count, int *s_base, int *s_wave) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int N = T * k;
  for (int e = tid; e < E; e += 1024) s_count[e] = 0;
  for (int i = tid; i < 16 * E; i += 1024) s_wave[i] = 0;
  __syncthreads();
  auto ld_idx = [&](int n) {
    return kAgentLoads ? (int)ld_agent(reinterpret_cast<const uint32_t *>(idx) + n) : idx[n];
  };
  // counts, 8 loads in flight per thread at a time (one round trip per 8 K entries)
  for (int n0 = tid; n0 < N; n0 += 8 * 1024) {
    int ev[8];
#pragma unroll
    for (int i = 0; i < 8; i++) ev[i] = n0 + 1024 * i < N ? ld_idx(n0 + 1024 * i) : -1;
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (ev[i] >= 0) atomicAdd(&s_count[ev[i]], 1);
  }
  __syncthreads();
  if (wv == 0) expert_list_wave(s_count, E, lane, s_base, active_ids, active_off, n_active);
  __syncthreads();
  int e_next = tid < N ? ld_idx(tid) : -1;
  for (int c0 = 0; c0 < N; c0 += 1024) {
    const int n = c0 + tid;
    const int e = e_next;
    e_next = n + 1024 < N ? ld_idx(n + 1024) : -1;  // the next chunk's entry, in flight meanwhile
    // lanes of this wavefront holding the same value (9-bit match through ballots)
    const uint32_t v = (uint32_t)(e + 1);
    uint64_t same = ~0ull;
#pragma unroll
    for (int bit = 0; bit < 9; bit++) {
      uint64_t b = __ballot((v >> bit) & 1u);
      same &= ((v >> bit) & 1u) ? b : ~b;
    }
    const int rank_in_wave = __popcll(same & ((1ull << lane) - 1ull));
    const bool leader = (same & ((1ull << lane) - 1ull)) == 0;
    if (leader && e >= 0) s_wave[wv * E + e] = __popcll(same);
    __syncthreads();
    for (int ee = tid; ee < E; ee += 1024) {  // exclusive prefix over wavefronts
      int run = 0;
      for (int w = 0; w < 16; w++) {
        int c = s_wave[w * E + ee];
        s_wave[w * E + ee] = run;
        run += c;
      }
      s_count[ee] = run;  // this chunk's total for expert ee
    }
    __syncthreads();
    if (e >= 0) {
      int ge = s_base[e] + s_wave[wv * E + e] + rank_in_wave;
      entry_src[ge] = n / k;
      pos[n] = ge;
    } else if (n < N) {
      pos[n] = -1;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += 1024) s_base[ee] += s_count[ee];
    for (int i = tid; i < 16 * E; i += 1024) s_wave[i] = 0;
    __syncthreads();
  }
}

// Length of a token's x staging in k_route (floats): the router lane chains' length.
__host__ __device__ constexpr int route_hp(int H) { return ((H + 63) / 64 + 7) / 8 * 512; }

// Router + top-k for TB tokens per block (block b: tokens TB b .. TB b + TB - 1). x of the tokens
// is staged in LDS (zero padded to the router chains' length; with xsplit != NULL its bf16
// hi + lo split is written for the GEMV path); wavefront w computes experts w, w + 16, ... for
// every token of the block from one load of the expert's weights (router_dot's canonical order
// per token); then wavefront w runs the top-k of token w (wave_topk_order/weights, k <= 4,
// E <= 128: block_topk's arithmetic), or for larger k the block runs block_topk per token.
// With xrec the block also writes its tokens' grouped-GEMM records; with bucket_ticket the last
// block to finish groups every entry by expert (bucket_block) in its free x staging area.
template <int KI, int TB>
__global__ __launch_bounds__(kRouteThreads) void k_route(RouteArgs a) {
  __shared__ float s_logit[TB][kMaxExperts];
  __shared__ float s_p[kMaxExperts];
  __shared__ int s_order[TB][kMaxTopK];
  __shared__ float s_w[TB][kMaxTopK];
  __shared__ int s_sel[TB];
  __shared__ int s_last;
  __shared__ int s_cnt[kMaxExperts];  // the grouping's per-expert counts of the block's entries
  const int t0 = blockIdx.x * TB;
  const int nt = min(TB, a.T - t0);
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int nw = kRouteThreads / 64;
  const int H = a.H, E = a.E;
  const int nq = ((H + 63) / 64 + 7) / 8;  // uint4 per lane chain
  const int Hp = route_hp(H);
  extern __shared__ float s_x[];  // TB * Hp floats
  // one token per block: the weights of the wavefront's first expert, in flight while x is
  // staged (with 8 tokens they would stay live through the records' split and spill)
  uint4 v[KI > 0 ? KI : 1];
  if (KI > 0 && TB == 1 && wv < E) {
    const uint4 *wq = reinterpret_cast<const uint4 *>(a.w + (size_t)wv * nq * 512) + lane;
#pragma unroll
    for (int q = 0; q < KI; q++) v[q] = wq[q * 64];
  }
  auto stage = [&](int tb, int k, float xv) {
    s_x[tb * Hp + k] = xv;
    if (a.xsplit && k < H) {
      uint16_t *xs = a.xsplit + (size_t)(t0 + tb) * 2 * H;
      uint16_t hi, lo;
      split_bf16(xv, hi, lo);
      xs[k] = hi;
      xs[H + k] = lo;
    }
  };
  if constexpr (KI > 0) {
    // the chain length is KI * 512 values: every x load of the block's tokens in flight at once
    // (a loop with a runtime trip count waited for each load before the next)
    constexpr int kPer = (KI * 512 + kRouteThreads - 1) / kRouteThreads;
    float xv[TB][kPer];
#pragma unroll
    for (int tb = 0; tb < TB; tb++)
#pragma unroll
      for (int q = 0; q < kPer; q++) {
        const int k = (int)threadIdx.x + q * kRouteThreads;
        xv[tb][q] = tb < nt && k < H ? a.x[(size_t)(t0 + tb) * H + k] : 0.0f;
      }
#pragma unroll
    for (int tb = 0; tb < TB; tb++)
#pragma unroll
      for (int q = 0; q < kPer; q++) {
        const int k = (int)threadIdx.x + q * kRouteThreads;
        if (tb < nt && k < Hp) stage(tb, k, xv[tb][q]);
      }
  } else {
    for (int tb = 0; tb < nt; tb++)
      for (int k = threadIdx.x; k < Hp; k += kRouteThreads) stage(tb, k, k < H ? a.x[(size_t)(t0 + tb) * H + k] : 0.0f);
  }
  __syncthreads();
  // the grouped GEMM's activation records of the block's tokens, a lane per 32-value block, by
  // threads u0, u0 + stride, ... (after the router, beside the top-k: off the critical path)
  auto write_records = [&](int u0, int stride) {
    if (!a.xrec) return;
    constexpr int kRecBlocks = 4 * kGemmNs;
    for (int u = u0; u < nt * kRecBlocks; u += stride) {
      const int tb = u / kRecBlocks, blk = u - tb * kRecBlocks, k0 = 32 * blk;
      const float *xt = s_x + tb * Hp;
      float xv[32];
#pragma unroll
      for (int q = 0; q < 8; q++) {  // the staging row holds zeros from H to Hp; 16-byte reads there
        const float4 x4 = k0 + 4 * q + 3 < Hp ? *reinterpret_cast<const float4 *>(xt + k0 + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
        xv[4 * q] = k0 + 4 * q < H ? x4.x : 0.0f;
        xv[4 * q + 1] = k0 + 4 * q + 1 < H ? x4.y : 0.0f;
        xv[4 * q + 2] = k0 + 4 * q + 2 < H ? x4.z : 0.0f;
        xv[4 * q + 3] = k0 + 4 * q + 3 < H ? x4.w : 0.0f;
      }
      if (a.rec_terms == 1)
        rec_split_block<1>(xv, blk, a.xrec + (size_t)(t0 + tb) * GemmRecT<1>::kBytes);
      else
        rec_split_block<kGemmTerms>(xv, blk, a.xrec + (size_t)(t0 + tb) * GemmRec::kBytes);
    }
  };
  if constexpr (KI > 0) {
    // experts in pairs (e, e + nw): each x value is read from LDS once for both chains (the
    // reads, not the FMAs, bound this loop); each chain keeps router_dot's order
    for (int e = wv; e < E; e += 2 * nw) {
      const int e1 = e + nw;
      uint4 wa[KI], wb[KI];
      const uint4 *qa = reinterpret_cast<const uint4 *>(a.w + (size_t)e * nq * 512) + lane;
      const uint4 *qb = reinterpret_cast<const uint4 *>(a.w + (size_t)min(e1, E - 1) * nq * 512) + lane;
#pragma unroll
      for (int q = 0; q < KI; q++) {
        wa[q] = TB == 1 && e == wv ? v[q] : qa[q * 64];  // (the first expert's loaded at the start)
        wb[q] = qb[q * 64];
      }
#pragma unroll 1
      for (int tb = 0; tb < nt; tb++) {  // (one token at a time: the chains' registers fit)
        {
          const float *xt = s_x + tb * Hp;
          float pa = 0.0f, pb = 0.0f;
#pragma unroll
          for (int q = 0; q < KI; q++) {
            const uint32_t ua[4] = {wa[q].x, wa[q].y, wa[q].z, wa[q].w};
            const uint32_t ub[4] = {wb[q].x, wb[q].y, wb[q].z, wb[q].w};
#pragma unroll
            for (int h = 0; h < 8; h++) {
              const float xv = xt[lane + 64 * (8 * q + h)];
              pa = __builtin_fmaf(bf16_to_f32((uint16_t)(ua[h >> 1] >> (16 * (h & 1)))), xv, pa);
              pb = __builtin_fmaf(bf16_to_f32((uint16_t)(ub[h >> 1] >> (16 * (h & 1)))), xv, pb);
            }
          }
          pa = wave_sum_xor(pa);
          pb = wave_sum_xor(pb);
          if (lane == 0) {
            s_logit[tb][e] = canon_nan(pa + a.bias[e]);
            if (e1 < E) s_logit[tb][e1] = canon_nan(pb + a.bias[e1]);
          }
        }
      }
    }
  } else {
    for (int e = wv; e < E; e += nw) {
      const uint16_t *w_e = a.w + (size_t)e * nq * 512;
      for (int tb = 0; tb < nt; tb++) {
        const float p = router_dot<0>(w_e, s_x + tb * Hp, nq, lane);
        if (lane == 0) s_logit[tb][e] = canon_nan(p + a.bias[e]);
      }
    }
  }
  __syncthreads();

  const TopkCfg c{E, a.k, a.adaptive, a.min_k, a.top1_min, a.margin_min, a.top2_mass};
  const bool per_wave = a.k <= 4 && E <= 128;
  // per-wavefront top-k: wavefronts TB .. 15 write the records meanwhile; else all threads first
  static_assert(TB < kRouteThreads / 64, "a wavefront per token, and wavefronts for the records");
  if (!per_wave || wv >= TB)
    write_records(per_wave ? (int)threadIdx.x - 64 * TB : (int)threadIdx.x, per_wave ? kRouteThreads - 64 * TB : kRouteThreads);
  if (per_wave) {
    if (wv < nt) {
      const int tb = wv, t = t0 + tb;
      float l[2];
      l[0] = lane < E ? s_logit[tb][lane] : 0.0f;
      l[1] = lane + 64 < E ? s_logit[tb][lane + 64] : 0.0f;
      if (lane < E) a.logits[(size_t)t * E + lane] = l[0];
      if (lane + 64 < E) a.logits[(size_t)t * E + lane + 64] = l[1];
      int ord[4];
      if (E <= 64) {
        const float l1[1] = {l[0]};
        wave_topk_order<1>(c, l1, lane, ord);
        wave_topk_weights<1>(c, l1, lane, ord, true, s_order[tb], s_w[tb], &s_sel[tb]);
      } else {
        wave_topk_order<2>(c, l, lane, ord);
        wave_topk_weights<2>(c, l, lane, ord, true, s_order[tb], s_w[tb], &s_sel[tb]);
      }
      if (lane < a.k) {
        const size_t o = (size_t)t * a.k + lane;
        st_agent(reinterpret_cast<uint32_t *>(a.idx) + o, (uint32_t)s_order[tb][lane]);
        a.wts[o] = s_w[tb][lane];
      }
    }
  } else {
    for (int tb = 0; tb < nt; tb++) {
      const int t = t0 + tb;
      for (int e = threadIdx.x; e < E; e += kRouteThreads) a.logits[(size_t)t * E + e] = s_logit[tb][e];
      block_topk(c, s_logit[tb], s_p, s_order[tb], s_w[tb], &s_sel[tb]);
      if (threadIdx.x < a.k) {
        const size_t o = (size_t)t * a.k + threadIdx.x;
        st_agent(reinterpret_cast<uint32_t *>(a.idx) + o, (uint32_t)s_order[tb][threadIdx.x]);
        a.wts[o] = s_w[tb][threadIdx.x];
      }
    }
  }
  if (a.fuse_bucket && threadIdx.x == 0) {  // single token (TB = 1): the expert list is the slot list
    const int sel = s_sel[0];
    *a.n_active = sel;
    for (int s2 = 0; s2 < sel; s2++) {
      a.active_ids[s2] = s_order[0][s2];
      a.active_off[s2] = s2;
      a.entry_src[s2] = 0;
    }
    a.active_off[sel] = sel;
    for (int s2 = 0; s2 < a.k; s2++) a.pos[s2] = s2 < sel ? s2 : -1;
  }
  if (a.bucket_ticket) {
    // The grouping. When the per-block count table fits the block's LDS, in parallel: every
    // block counts its entries per expert (blk_count[block][e]) and ranks each entry among the
    // block's entries of its expert, in entry order t k + slot (rank[t k + slot]); the last
    // block loads the whole table (and every entry's expert and rank) in one round of loads,
    // turns it into per-block bases (an exclusive prefix over blocks, per expert) in LDS and
    // scatters every entry to base + rank. Otherwise the last block runs bucket_block. Either
    // way the entries of one expert end up ordered by t k + slot.
    const int nblk = (int)gridDim.x, N = a.T * a.k;
    const int ld_bc = nblk + 1;  // LDS row of one expert's counts (odd: rows on distinct banks)
    const bool table = (size_t)ld_bc * E + 2 * (size_t)E <= (size_t)TB * Hp;
    __syncthreads();  // s_order of every token of the block
    if (table && wv == 0) {
      const int ne = nt * a.k;
      for (int e = lane; e < E; e += 64) s_cnt[e] = 0;
      for (int p0 = 0; p0 < ne; p0 += 64) {
        const int l = p0 + lane, tb = l / a.k, slot = l - tb * a.k;
        const int e = l < ne ? s_order[tb][slot] : -1;
        const uint32_t v = (uint32_t)(e + 1);  // 0 .. kMaxExperts: 9 bits
        uint64_t same = ~0ull;
#pragma unroll
        for (int bit = 0; bit < 9; bit++) {
          const uint64_t bb = __ballot((v >> bit) & 1u);
          same &= ((v >> bit) & 1u) ? bb : ~bb;
        }
        const uint64_t below = same & ((1ull << lane) - 1ull);
        const int base = e >= 0 ? s_cnt[e] : 0;
        if (e >= 0) {
          st_agent(reinterpret_cast<uint32_t *>(a.rank) + (size_t)t0 * a.k + l, (uint32_t)(base + __popcll(below)));
          if (below == 0) s_cnt[e] = base + __popcll(same);  // the group's first lane
        }
      }
      for (int e = lane; e < E; e += 64)
        st_agent(reinterpret_cast<uint32_t *>(a.blk_count) + (size_t)blockIdx.x * E + e, (uint32_t)s_cnt[e]);
    }
    wait_mem();  // this thread's idx, rank and count stores (agent scope) have completed
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(a.bucket_ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (!s_last) return;
    if (threadIdx.x == 0) st_agent(a.bucket_ticket, 0u);  // zero again for the next launch
    if (!table) {
      int *ws = reinterpret_cast<int *>(s_x);  // (2 + 16) E ints; the host checked they fit
      bucket_block<true>(a.idx, a.T, a.k, E, a.n_active, a.active_ids, a.active_off, a.entry_src,
                         a.pos, ws, ws + E, ws + 2 * E);
      return;
    }
    // s_bc: the table expert-major in LDS, [e][block] with rows ld_bc apart
    int *s_bc = reinterpret_cast<int *>(s_x), *s_tot = s_bc + (size_t)ld_bc * E, *s_base = s_tot + E;
    const uint32_t *bc = reinterpret_cast<const uint32_t *>(a.blk_count);
    const uint32_t *ix = reinterpret_cast<const uint32_t *>(a.idx), *rk = reinterpret_cast<const uint32_t *>(a.rank);
    constexpr int kPerT = 16;  // entries per thread per round
    // the count table into LDS, and the first round's entries, in one round of loads
    int ev[kPerT], rv[kPerT];
#pragma unroll
    for (int i = 0; i < kPerT; i++) {
      const int n = (int)threadIdx.x + i * kRouteThreads;
      ev[i] = n < N ? (int)ld_agent(ix + n) : -1;
      rv[i] = n < N ? (int)ld_agent(rk + n) : 0;
    }
    for (int i0 = threadIdx.x; i0 < nblk * E; i0 += 8 * kRouteThreads) {
      uint32_t cv[8];
#pragma unroll
      for (int q = 0; q < 8; q++) cv[q] = i0 + q * kRouteThreads < nblk * E ? ld_agent(bc + i0 + q * kRouteThreads) : 0u;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const int i = i0 + q * kRouteThreads, bi = i / E;
        if (i < nblk * E) s_bc[(i - bi * E) * ld_bc + bi] = (int)cv[q];
      }
    }
    __syncthreads();
    // per expert, bases = exclusive prefix of the counts over blocks: a wavefront per expert,
    // lane l summing blocks [l S, l S + S) serially, then one wave scan of the 64 lane sums
    const int S = (nblk + 63) / 64;
    for (int e = wv; e < E; e += nw) {
      int *row = s_bc + (size_t)e * ld_bc;
      int sum = 0;
      for (int q = 0; q < S; q++) {
        const int bi = lane * S + q;
        if (bi < nblk) sum += row[bi];
      }
      int incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o);
        if (lane >= o) incl += u;
      }
      int run = incl - sum;
      for (int q = 0; q < S; q++) {
        const int bi = lane * S + q;
        if (bi < nblk) {
          const int c = row[bi];
          row[bi] = run;
          run += c;
        }
      }
      if (lane == 63) s_tot[e] = incl;
    }
    __syncthreads();
    if (wv == 0) expert_list_wave(s_tot, E, lane, s_base, a.active_ids, a.active_off, a.n_active);
    __syncthreads();
    for (int n0 = threadIdx.x;; n0 += kPerT * kRouteThreads) {
#pragma unroll
      for (int i = 0; i < kPerT; i++) {
        const int n = n0 + i * kRouteThreads;
        if (n >= N) break;
        if (ev[i] < 0) {
          a.pos[n] = -1;
        } else {
          const int ge = s_base[ev[i]] + s_bc[ev[i] * ld_bc + (n / a.k) / TB] + rv[i];
          a.entry_src[ge] = n / a.k;
          a.pos[n] = ge;
        }
      }
      if (n0 + kPerT * kRouteThreads >= N) break;
#pragma unroll
      for (int i = 0; i < kPerT; i++) {  // the next round's entries
        const int n = n0 + (kPerT + i) * kRouteThreads;
        ev[i] = n < N ? (int)ld_agent(ix + n) : -1;
        rv[i] = n < N ? (int)ld_agent(rk + n) : 0;
      }
    }
  }
}

template <int KI>
static hipError_t launch_route_ki(const RouteArgs &a, int nq, hipStream_t s) {
  const size_t hp = (size_t)nq * 8 * 64 * sizeof(float);
  if (a.T >= 2048 && kRouteTokens * hp <= 144 * 1024) {
    // TB tokens of x may exceed the default 64 KB of dynamic LDS
    static DynLdsOnce once;
    const hipError_t e = ensure_dyn_lds(once, reinterpret_cast<const void *>(&k_route<KI, kRouteTokens>),
                                        kRouteTokens * hp);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_route<KI, kRouteTokens>), dim3((unsigned)((a.T + kRouteTokens - 1) / kRouteTokens)),
                       dim3(kRouteThreads), kRouteTokens * hp, s, a);
  } else {
    hipLaunchKernelGGL((k_route<KI, 1>), dim3((unsigned)a.T), dim3(kRouteThreads), hp, s, a);
  }
  return hipGetLastError();
}

bool route_bucket_fits(int H, int E) { return 18 * E <= route_hp(H); }

hipError_t launch_route(const RouteArgs &a, hipStream_t s) {
  if (a.E < 1 || a.E > kMaxExperts || a.k < 1 || a.k > kMaxTopK || a.k > a.E || a.T < 1 ||
      a.H < 1 || (a.fuse_bucket && a.T != 1) || (a.xrec && a.H > 128 * kGemmNs) ||
      (a.bucket_ticket && (a.fuse_bucket || !route_bucket_fits(a.H, a.E) || !a.blk_count || !a.rank)))
    return hipErrorInvalidValue;
  const int nq = ((a.H + 63) / 64 + 7) / 8;
  const size_t lds = (size_t)nq * 8 * 64 * sizeof(float);
  if (lds > 65536) return hipErrorInvalidValue;
  switch (nq) {  // 2880 -> 45 chain terms -> 6 loads per lane
    case 1: return launch_route_ki<1>(a, nq, s);
    case 2: return launch_route_ki<2>(a, nq, s);
    case 6: return launch_route_ki<6>(a, nq, s);
    default: return launch_route_ki<0>(a, nq, s);
  }
}

// ------------------------------------------------------------------ bucketing

__global__ __launch_bounds__(1024) void k_bucket(const int32_t *idx, int T, int k, int E,
                                                 int32_t *n_active, int32_t *active_ids,
                                                 int32_t *active_off, int32_t *entry_src,
                                                 int32_t *pos) {
  __shared__ int s_count[kMaxExperts];
  __shared__ int s_base[kMaxExperts];
  __shared__ int s_wave[16 * kMaxExperts];
  bucket_block<false>(idx, T, k, E, n_active, active_ids, active_off, entry_src, pos, s_count, s_base, s_wave);
}

hipError_t launch_bucket(const int32_t *idx, int T, int k, int E, int32_t *n_active,
                         int32_t *active_ids, int32_t *active_off, int32_t *entry_src,
                         int32_t *pos, hipStream_t s) {
  if (E < 1 || E > kMaxExperts || k < 1 || T < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_bucket, dim3(1), dim3(1024), 0, s, idx, T, k, E, n_active, active_ids,
                     active_off, entry_src, pos);
  return hipGetLastError();
}

// ------------------------------------------------------------------ MXFP4 GEMV on MFMA

// Small-batch variant (at most NE entries per expert, at most NSMAX steps per tile): a
// workgroup is 4 wavefronts on 4 consecutive tiles of one expert. Each wavefront issues every
// weight and scale load of its tile before computing, so a tile's 23 KB are in flight at
// once; the workgroup stages its entries' B operands (hi/lo rows) in LDS first.
template <int MODE, int NE, int NSMAX>
__global__ __launch_bounds__(256) void k_expert_gemv_small(GemvArgs a) {
  extern __shared__ uint4 s_b[];
  constexpr int SBMAX = 3 * NE;  // staging loads per thread: NE * 2 rows of <= 384 uint4
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int tiles = (int)a.d.tiles;
  const int tgs = (tiles + 3) >> 2;
  const int act = blockIdx.x / tgs;
  const int t = (blockIdx.x - act * tgs) * 4 + wv;
  if (act >= a.max_active) return;
  // independent loads (one round trip); the arrays hold max_active (+1) entries
  const int n_act = *a.n_active;
  const int expert = a.active_ids[act];
  const int beg = a.active_off[act];
  int nent = a.active_off[act + 1] - beg;
  if (act >= n_act) return;
  if (nent > NE) nent = NE;
  const uint8_t *rec = a.base + (size_t)expert * a.stride;
  const uint8_t *mat = rec + a.mat_off;
  const bool tile_ok = t < tiles;
  const int j = lane & 15;
  const int row_u4 = (int)a.d.nb * 4;  // uint4 per (entry, term) row of K bf16

  // 1. B operand rows of this expert's entries (read first: the barrier waits only for them)
  int src[NE];
#pragma unroll
  for (int e = 0; e < NE; e++)
    src[e] = e < nent ? (a.entry_src ? a.entry_src[beg + e] : beg + e) : 0;
  const int nstg = nent * 2 * row_u4;
  uint4 stg[SBMAX];
#pragma unroll
  for (int i = 0; i < SBMAX; i++) {
    // always a valid address (row 0 of entry 0 when idx is past the staged range)
    const int idx = threadIdx.x + 256 * i;
    const int ci = idx < nstg ? idx : 0;
    const int e = ci / (2 * row_u4), r = ci - e * 2 * row_u4;
    int se = src[0];
#pragma unroll
    for (int q = 1; q < NE; q++) se = (e == q) ? src[q] : se;
    stg[i] = reinterpret_cast<const uint4 *>(a.bsrc)[(size_t)se * 2 * row_u4 + r];
  }
  // 2. every weight and scale load of the tile
  TileRegs<NSMAX> r;
  tile_load<NSMAX>(r, mat, a.d, t, tile_ok, lane);
#pragma unroll
  for (int i = 0; i < SBMAX; i++) {
    const int idx = threadIdx.x + 256 * i;
    if (idx < nstg) s_b[idx] = stg[i];
  }
  __syncthreads();
  if (!tile_ok) return;

  // 3. MFMA sweep over the tile
  const int ent = j >> 1, term = j & 1;
  const f32x4 acc = tile_mfma<NSMAX>(r, a.d, s_b + (size_t)(ent * 2 + term) * row_u4, ent < nent, lane);
  gemv_epilogue<MODE>(a, acc, rec, beg, 0, nent, t, lane);
}

constexpr int kSmallNsMax = 24;  // tiles of up to 96 blocks (K <= 3072)

template <int MODE, int NE>
static hipError_t launch_small(const GemvArgs &a, hipStream_t s) {
  const size_t lds = (size_t)NE * 2 * a.d.nb * 32 * 2;
  if (lds > 65536) {
    static DynLdsOnce once;
    const hipError_t e = ensure_dyn_lds(
        once, reinterpret_cast<const void *>(&k_expert_gemv_small<MODE, NE, kSmallNsMax>), 160 * 1024);
    if (e != hipSuccess) return e;
  }
  const size_t wgs = (size_t)a.max_active * ((a.d.tiles + 3) / 4);
  hipLaunchKernelGGL((k_expert_gemv_small<MODE, NE, kSmallNsMax>), dim3((unsigned)wgs), dim3(256),
                     lds, s, a);
  return hipGetLastError();
}

// One wavefront computes one 16-row tile of one active expert's matrix against the B
// operands of that expert's entries, CH chunks of 8 entries at a time. MFMA columns:
// column j of a chunk is entry j/2, term j%2 (hi, lo). The MFMA result for lane l holds
// rows 4*(l/16)+i (i = 0..3) of column l%16; hi and lo columns are summed across lane pairs.
template <int MODE, int CH>
__global__ __launch_bounds__(256) void k_expert_gemv(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int tiles = (int)a.d.tiles;
  const int act = wid / tiles;
  const int t = wid - act * tiles;
  if (act >= a.max_active) return;
  if (act >= *a.n_active) return;
  const int expert = a.active_ids[act];
  const int beg = a.active_off[act];
  const int nent = a.active_off[act + 1] - beg;
  const uint8_t *rec = a.base + (size_t)expert * a.stride;
  const uint8_t *mat = rec + a.mat_off;
  const int nb = (int)a.d.nb, ns = (int)a.d.ns, nq = (int)a.d.nq;
  const uint4 *wp = reinterpret_cast<const uint4 *>(mat) + (size_t)t * 16 * nb;
  const uint32_t *sp = reinterpret_cast<const uint32_t *>(mat + pack_weight_bytes(a.d)) +
                       (size_t)t * nq * 64;
  const int g = lane >> 4, j = lane & 15;
  const size_t K = (size_t)nb * 32;

  for (int c0 = 0; c0 < nent; c0 += 8 * CH) {
    f32x4 acc[CH];
    const uint16_t *bp[CH];
    bool bval[CH];
#pragma unroll
    for (int cc = 0; cc < CH; cc++) {
      acc[cc] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const int el = c0 + 8 * cc + (j >> 1);
      bval[cc] = el < nent;
      const int src = bval[cc] ? (a.entry_src ? a.entry_src[beg + el] : beg + el) : 0;
      bp[cc] = a.bsrc + ((size_t)src * 2 + (j & 1)) * K;
    }
    for (int q = 0; q < nq; q++) {
      const uint32_t sw = sp[q * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int s = q * 4 + i;
        if (s >= ns) break;
        const int b = 4 * s + g;
        const bool v = b < nb;
        uint4 raw = make_uint4(0u, 0u, 0u, 0u);
        if (v) raw = wp[s * 64 + lane];
        const float sc = __uint_as_float(((sw >> (8 * i)) & 0xFFu) << 23);
        const bf16x8 A0 = decode8(raw.x, sc), A1 = decode8(raw.y, sc);
        const bf16x8 A2 = decode8(raw.z, sc), A3 = decode8(raw.w, sc);
#pragma unroll
        for (int cc = 0; cc < CH; cc++) {
          uint4 b0 = make_uint4(0u, 0u, 0u, 0u), b1 = b0, b2 = b0, b3 = b0;
          if (v && bval[cc]) {
            const uint4 *src = reinterpret_cast<const uint4 *>(bp[cc] + 32 * (size_t)b);
            b0 = src[0];
            b1 = src[1];
            b2 = src[2];
            b3 = src[3];
          }
          acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, as_bf16x8(b0), acc[cc], 0, 0, 0);
          acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, as_bf16x8(b1), acc[cc], 0, 0, 0);
          acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A2, as_bf16x8(b2), acc[cc], 0, 0, 0);
          acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A3, as_bf16x8(b3), acc[cc], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int cc = 0; cc < CH; cc++) gemv_epilogue<MODE>(a, acc[cc], rec, beg, c0 + 8 * cc, nent, t, lane);
  }
}

template <int MODE>
static hipError_t launch_gemv_mode(const GemvArgs &a, hipStream_t s) {
  if (a.d.ns <= (uint32_t)kSmallNsMax && a.max_entries_per_expert <= 8) {
    if (a.max_entries_per_expert <= 1) return launch_small<MODE, 1>(a, s);
    if (a.max_entries_per_expert <= 2) return launch_small<MODE, 2>(a, s);
    if (a.max_entries_per_expert <= 4) return launch_small<MODE, 4>(a, s);
    return launch_small<MODE, 8>(a, s);
  }
  const size_t waves = (size_t)a.max_active * a.d.tiles;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  if (a.max_entries_per_expert <= 8)
    hipLaunchKernelGGL((k_expert_gemv<MODE, 1>), grid, block, 0, s, a);
  else if (a.max_entries_per_expert <= 16)
    hipLaunchKernelGGL((k_expert_gemv<MODE, 2>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((k_expert_gemv<MODE, 4>), grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gemv(GemvMode mode, const GemvArgs &a, hipStream_t s) {
  if (a.d.rows == 0 || a.d.rows % 16 || a.d.nb == 0 || a.max_active < 1 || !a.base || !a.bsrc ||
      !a.out || !a.n_active || !a.active_ids || !a.active_off)
    return hipErrorInvalidValue;
  if ((size_t)a.max_active * a.d.tiles > (size_t)0x7FFFFFFF * 4) return hipErrorInvalidValue;
  switch (mode) {
    case GEMV_GATE_UP: return launch_gemv_mode<GEMV_GATE_UP>(a, s);
    case GEMV_DOWN: return launch_gemv_mode<GEMV_DOWN>(a, s);
    default: return launch_gemv_mode<GEMV_RAW>(a, s);
  }
}

// ------------------------------------------------------------------ combine

// y[t, d] = sum over slots s (rank order) of w[t, s] * o[pos[t, s], d], accumulated from 0
// with separate rounding of each product and sum (session.rs:975-980). skip_nonfinite drops
// non-finite o elements (moe_dispatch.rs:598-601).
__global__ __launch_bounds__(256) void k_combine(const float *o, const int32_t *pos,
                                                 const float *w, int T, int k, int H,
                                                 int skip_nonfinite, float *y) {
  const int h4 = H / 4;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)T * h4) return;
  const int t = (int)(i / h4), d4 = (int)(i % h4);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < k; s++) {
    const int p = pos[(size_t)t * k + s];
    if (p < 0) continue;
    const float ws = w[(size_t)t * k + s];
    const float4 v = reinterpret_cast<const float4 *>(o + (size_t)p * H)[d4];
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      if (skip_nonfinite && !isfinite(vv[c])) continue;
      acc[c] = acc[c] + ws * vv[c];
    }
  }
  reinterpret_cast<float4 *>(y + (size_t)t * H)[d4] =
      make_float4(canon_nan(acc[0]), canon_nan(acc[1]), canon_nan(acc[2]), canon_nan(acc[3]));
}

// k_combine for a fixed k: every slot's row load is issued before the first product, instead of
// one round trip per slot (the same products and sums in the same order).
template <int K>
__global__ __launch_bounds__(256) void k_combine_k(const float *o, const int32_t *pos,
                                                   const float *w, int T, int H, int skip_nonfinite,
                                                   float *y) {
  const int h4 = H / 4;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)T * h4) return;
  const int t = (int)(i / h4), d4 = (int)(i % h4);
  int p[K];
  float ws[K];
  float4 v[K];
#pragma unroll
  for (int s = 0; s < K; s++) {
    p[s] = pos[(size_t)t * K + s];
    ws[s] = w[(size_t)t * K + s];
  }
#pragma unroll
  for (int s = 0; s < K; s++)  // a dropped slot (p < 0) reads row 0 and is not used
    v[s] = reinterpret_cast<const float4 *>(o + (size_t)(p[s] < 0 ? 0 : p[s]) * H)[d4];
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < K; s++) {
    if (p[s] < 0) continue;
    const float vv[4] = {v[s].x, v[s].y, v[s].z, v[s].w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      if (skip_nonfinite && !isfinite(vv[c])) continue;
      acc[c] = acc[c] + ws[s] * vv[c];
    }
  }
  reinterpret_cast<float4 *>(y + (size_t)t * H)[d4] =
      make_float4(canon_nan(acc[0]), canon_nan(acc[1]), canon_nan(acc[2]), canon_nan(acc[3]));
}

hipError_t launch_combine(const float *o, const int32_t *pos, const float *w, int T, int k, int H,
                          int skip_nonfinite, float *y, hipStream_t s) {
  if (H % 4 || T < 1 || k < 1) return hipErrorInvalidValue;
  const size_t n = (size_t)T * (H / 4);
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (k == 4)
    hipLaunchKernelGGL(k_combine_k<4>, grid, block, 0, s, o, pos, w, T, H, skip_nonfinite, y);
  else
    hipLaunchKernelGGL(k_combine, grid, block, 0, s, o, pos, w, T, k, H, skip_nonfinite, y);
  return hipGetLastError();
}

// ------------------------------------------------------------------ split

__global__ __launch_bounds__(256) void k_split(const float *x, size_t n_rows, size_t K,
                                               uint16_t *xs) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_rows * K) return;
  const size_t r = i / K, k = i % K;
  uint16_t hi, lo;
  split_bf16(x[i], hi, lo);
  xs[r * 2 * K + k] = hi;
  xs[r * 2 * K + K + k] = lo;
}

hipError_t launch_split(const float *x, size_t n_rows, size_t K, uint16_t *xsplit, hipStream_t s) {
  const size_t n = n_rows * K;
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_split, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n_rows, K,
                     xsplit);
  return hipGetLastError();
}

// ------------------------------------------------------------------ bit-exact dequant

__device__ __forceinline__ void decode_block_f32(uint4 raw, uint32_t sbyte, float *out) {
  const float sc = __uint_as_float(sbyte << 23);  // weights.rs:359
  const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
  float4 *o4 = reinterpret_cast<float4 *>(out);
#pragma unroll
  for (int d = 0; d < 4; d++) {
    float v[8];
#pragma unroll
    for (int bb = 0; bb < 4; bb++) {
      const uint32_t byte = (wv[d] >> (8 * bb)) & 0xFFu;
      v[2 * bb] = canon_nan(e2m1_to_f32(byte & 0xFu) * sc);
      v[2 * bb + 1] = canon_nan(e2m1_to_f32(byte >> 4) * sc);
    }
    o4[2 * d] = make_float4(v[0], v[1], v[2], v[3]);
    o4[2 * d + 1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

__global__ __launch_bounds__(256) void k_dequant_hf(const uint8_t *blocks, const uint8_t *scales,
                                                    size_t n_blocks, float *out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_blocks) return;
  const uint4 raw = reinterpret_cast<const uint4 *>(blocks)[i];
  decode_block_f32(raw, scales[i], out + i * 32);
}

hipError_t launch_dequant_hf(const uint8_t *blocks, const uint8_t *scales, size_t rows,
                             size_t cols, float *out, hipStream_t s) {
  if (cols % 32) return hipErrorInvalidValue;
  const size_t n = rows * (cols / 32);
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_dequant_hf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, blocks,
                     scales, n, out);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_dequant_packed(const uint8_t *packed, PackDims d,
                                                        float *out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)d.rows * d.nb) return;
  const size_t row = i / d.nb;
  const uint32_t b = (uint32_t)(i % d.nb);
  const size_t t = row / 16;
  const uint32_t rl = (uint32_t)(row % 16), s = b / 4, g = b % 4, l = 16 * g + rl;
  const uint4 raw = reinterpret_cast<const uint4 *>(packed)[t * 16 * d.nb + 64 * s + l];
  const uint32_t *sw = reinterpret_cast<const uint32_t *>(packed + pack_weight_bytes(d));
  const uint32_t word = sw[(t * d.nq + s / 4) * 64 + l];
  decode_block_f32(raw, (word >> (8 * (s % 4))) & 0xFFu, out + i * 32);
}

hipError_t launch_dequant_packed(const uint8_t *packed, size_t rows, size_t cols, float *out,
                                 hipStream_t s) {
  if (cols % 32 || rows % 16) return hipErrorInvalidValue;
  const PackDims d = pack_dims(rows, cols);
  const size_t n = rows * d.nb;
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_dequant_packed, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, packed,
                     d, out);
  return hipGetLastError();
}

// ------------------------------------------------------------------ repack

__global__ __launch_bounds__(256) void k_pack_weights(const uint8_t *blocks, PackDims d,
                                                      uint8_t *packed) {
  const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;  // destination chunk
  if (c >= (size_t)d.rows * d.nb) return;
  const size_t per_tile = (size_t)16 * d.nb;
  const size_t t = c / per_tile;
  const uint32_t p = (uint32_t)(c % per_tile), s = p / 64, l = p % 64;
  const size_t row = t * 16 + (l & 15);
  const uint32_t b = 4 * s + (l >> 4);
  reinterpret_cast<uint4 *>(packed)[c] =
      reinterpret_cast<const uint4 *>(blocks)[row * d.nb + b];
}

__global__ __launch_bounds__(256) void k_pack_scales(const uint8_t *scales, PackDims d,
                                                     uint8_t *packed) {
  const size_t wi = (size_t)blockIdx.x * 256 + threadIdx.x;  // destination word
  if (wi >= (size_t)d.tiles * d.nq * 64) return;
  const size_t t = wi / ((size_t)d.nq * 64);
  const uint32_t q = (uint32_t)((wi / 64) % d.nq), l = (uint32_t)(wi % 64);
  const size_t row = t * 16 + (l & 15);
  uint32_t word = 0;
#pragma unroll
  for (uint32_t i = 0; i < 4; i++) {
    const uint32_t s = 4 * q + i, b = 4 * s + (l >> 4);
    if (s < d.ns && b < d.nb) word |= (uint32_t)scales[row * d.nb + b] << (8 * i);
  }
  reinterpret_cast<uint32_t *>(packed + pack_weight_bytes(d))[wi] = word;
}

hipError_t launch_pack(const uint8_t *blocks, const uint8_t *scales, size_t rows, size_t cols,
                       uint8_t *packed, hipStream_t s) {
  if (cols % 32 || rows % 16 || !rows || !cols) return hipErrorInvalidValue;
  const PackDims d = pack_dims(rows, cols);
  const size_t nc = (size_t)d.rows * d.nb, nw = (size_t)d.tiles * d.nq * 64;
  hipLaunchKernelGGL(k_pack_weights, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, s, blocks,
                     d, packed);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_pack_scales, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, s, scales,
                     d, packed);
  return hipGetLastError();
}

// ------------------------------------------------------------------ synthetic data

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_synth(void *dst, size_t n, int kind, uint64_t seed,
                                               float a, float b) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint64_t r = splitmix64(seed * 0xD1342543DE82EF95ull + i);
  if (kind == 0) {
    const uint32_t lo = (uint32_t)a, hi = (uint32_t)b;
    reinterpret_cast<uint8_t *>(dst)[i] = (uint8_t)(lo + (uint32_t)(r % (uint64_t)(hi - lo + 1)));
    return;
  }
  const uint64_t r2 = splitmix64(r ^ 0x5851F42D4C957F2Dull);
  const float u1 = ((float)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
  const float u2 = (float)(r2 >> 40) * (1.0f / 16777216.0f);
  const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2) * a;
  if (kind == 1)
    reinterpret_cast<uint16_t *>(dst)[i] = f32_to_bf16_rne(z);
  else if (kind == 2)
    reinterpret_cast<float *>(dst)[i] = z;
  else
    reinterpret_cast<float *>(dst)[i] = bf16_to_f32(f32_to_bf16_rne(z));
}

hipError_t launch_synth(void *dst, size_t n, int kind, uint64_t seed, float a, float b,
                        hipStream_t s) {
  if (kind < 0 || kind > 3) return hipErrorInvalidValue;
  if (kind == 0 && !(a >= 0.0f && b <= 255.0f && a <= b)) return hipErrorInvalidValue;
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_synth, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, n, kind,
                     seed, a, b);
  return hipGetLastError();
}

// ------------------------------------------------------------------ LM head (f32 GEMV)

// logits[v] = W[v, :] . x ; one wavefront per row, float4 loads, xor-butterfly reduction.
__global__ __launch_bounds__(256) void k_lm_head(const float *w, const float *x, size_t vocab,
                                                 size_t H, float *y) {
  const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= vocab) return;
  const float4 *wr = reinterpret_cast<const float4 *>(w + row * H);
  const float4 *xv = reinterpret_cast<const float4 *>(x);
  float acc = 0.0f;
  for (size_t k = lane; k < H / 4; k += 64) {
    const float4 a = wr[k], b = xv[k];
    acc = __builtin_fmaf(a.x, b.x, acc);
    acc = __builtin_fmaf(a.y, b.y, acc);
    acc = __builtin_fmaf(a.z, b.z, acc);
    acc = __builtin_fmaf(a.w, b.w, acc);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o);
  if (lane == 0) y[row] = acc;
}

// logits[v] = sum_i bf16_to_f32(W[v, i]) x[i] with the checkpoint's bf16 rows (lm_head_dot,
// weights.rs:73-82: bf16 widened exactly, f32 accumulation). A wavefront walks rows v = wave,
// wave + n_waves, ... two at a time; lane l keeps x[8 (l + 64 q) .. + 7] (q < kLmQ) in registers
// for all its rows and accumulates its 16-byte pieces of a row with fused multiply-adds in q
// order, then a xor butterfly over the 64 lanes. Weights are streamed with non-temporal loads.
constexpr int kLmQ = 6;  // 16-byte pieces per lane per row: H <= 64 * 8 * kLmQ = 3072
__global__ __launch_bounds__(256) void k_lm_head_bf16(const uint16_t *w, const float *x, size_t vocab, int H,
                                                      float *y) {
  const int lane = threadIdx.x & 63;
  const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6), n_waves = (size_t)gridDim.x * 4;
  const int nq = H / 8;  // 16-byte pieces per row
  float xr[kLmQ][8];
#pragma unroll
  for (int q = 0; q < kLmQ; q++) {
    const int p = lane + 64 * q;
    if (p < nq) {
      const float4 a = reinterpret_cast<const float4 *>(x)[2 * p];
      const float4 b = reinterpret_cast<const float4 *>(x)[2 * p + 1];
      xr[q][0] = a.x; xr[q][1] = a.y; xr[q][2] = a.z; xr[q][3] = a.w;
      xr[q][4] = b.x; xr[q][5] = b.y; xr[q][6] = b.z; xr[q][7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) xr[q][i] = 0.0f;
    }
  }
  for (size_t v0 = wave * 2; v0 < vocab; v0 += 2 * n_waves) {
    const size_t v1 = v0 + 1 < vocab ? v0 + 1 : v0;  // an odd last row is computed twice, stored once
    u32x4 wv[2][kLmQ];
#pragma unroll
    for (int q = 0; q < kLmQ; q++) {
      const int p = lane + 64 * q;
      wv[0][q] = p < nq ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + v0 * H) + p) : u32x4{0, 0, 0, 0};
      wv[1][q] = p < nq ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + v1 * H) + p) : u32x4{0, 0, 0, 0};
    }
    float acc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 2; r++) {
#pragma unroll
      for (int q = 0; q < kLmQ; q++) {
#pragma unroll
        for (int h = 0; h < 4; h++) {
          const uint32_t u = wv[r][q][h];
          acc[r] = __builtin_fmaf(__uint_as_float(u << 16), xr[q][2 * h], acc[r]);
          acc[r] = __builtin_fmaf(__uint_as_float(u & 0xFFFF0000u), xr[q][2 * h + 1], acc[r]);
        }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      acc[0] = acc[0] + __shfl_xor(acc[0], o);
      acc[1] = acc[1] + __shfl_xor(acc[1], o);
    }
    if (lane == 0) {
      y[v0] = acc[0];
      if (v1 != v0) y[v1] = acc[1];
    }
  }
}

// ------------------------------------------------------------------ RMSNorm and residual

// n[t] = (x[t] * inv_rms) * gamma, one wavefront per row (session.rs:483-493, the sum of squares
// in rms_inv_wave's order).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *x, int T, int H, const float *gamma, float eps,
                                                 float *n) {
  const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float *xr = x + (size_t)t * H;
  // rms_inv_wave's arithmetic with kNB loads in flight per lane at a time (a loop with a runtime
  // trip count waits for each load in turn)
  constexpr int kNB = 16;
  float p = 0.0f;
  for (int i0 = lane; i0 < H; i0 += 64 * kNB) {
    float v[kNB];
#pragma unroll
    for (int u = 0; u < kNB; u++) v[u] = i0 + 64 * u < H ? xr[i0 + 64 * u] : 0.0f;
#pragma unroll
    for (int u = 0; u < kNB; u++) {
      if (i0 + 64 * u >= H) break;
      const float sq = v[u] * v[u];
      p = p + sq;
    }
  }
  const float r = 1.0f / sqrtf(wave_sum_xor(p) / (float)H + eps);
  for (int d0 = lane; d0 < H; d0 += 64 * kNB) {
    float v[kNB], g[kNB];
#pragma unroll
    for (int u = 0; u < kNB; u++) {
      const bool in = d0 + 64 * u < H;
      v[u] = in ? xr[d0 + 64 * u] : 0.0f;
      g[u] = in ? gamma[d0 + 64 * u] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kNB; u++) {
      if (d0 + 64 * u >= H) break;
      const float vr = v[u] * r;
      n[(size_t)t * H + d0 + 64 * u] = vr * g[u];
    }
  }
}

hipError_t launch_rmsnorm(const float *x, size_t T, size_t H, const float *gamma, float eps, float *n,
                          hipStream_t s) {
  if (!T) return hipSuccess;
  if (H > (size_t)INT32_MAX || T > (size_t)INT32_MAX / 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s, x, (int)T, (int)H, gamma, eps, n);
  return hipGetLastError();
}

// y = x + y (session.rs:982-994: hidden + moe_out), NaN canonical.
__global__ __launch_bounds__(256) void k_add_rows(float *y, const float *x, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = canon_nan(x[i] + y[i]);
}

hipError_t launch_add_rows(float *y, const float *x, size_t n, hipStream_t s) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_add_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, x, n);
  return hipGetLastError();
}

hipError_t launch_lm_head_bf16(const uint16_t *w, const float *x, size_t vocab, size_t H, float *y, int n_cu,
                               hipStream_t s) {
  if (H % 8 || H > 64 * 8 * kLmQ || !vocab || (reinterpret_cast<uintptr_t>(x) & 15) ||
      (reinterpret_cast<uintptr_t>(w) & 15))
    return hipErrorInvalidValue;
  // four blocks (16 wavefronts) per CU, each wavefront a grid-stride walk over row pairs
  const size_t pairs_blocks = (vocab + 7) / 8;
  const unsigned blocks = (unsigned)std::min<size_t>(pairs_blocks, (size_t)4 * (n_cu > 0 ? n_cu : 256));
  hipLaunchKernelGGL(k_lm_head_bf16, dim3(blocks), dim3(256), 0, s, w, x, vocab, (int)H, y);
  return hipGetLastError();
}

hipError_t launch_lm_head(const float *w, const float *x, size_t vocab, size_t H, float *y,
                          hipStream_t s) {
  if (H % 4 || !vocab) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_lm_head, dim3((unsigned)((vocab + 3) / 4)), dim3(256), 0, s, w, x, vocab,
                     H, y);
  return hipGetLastError();
}

}  // namespace moe
