// Single-token MoE layer for gfx950 in ONE launch — the MoE block of
// Session::decode_step_inner (session.rs:818-980) for one token, with the down projection's
// weight stream overlapping the gate_up phase.
//
// Blocks of 4 wavefronts (3 per CU, so all blocks of the GPT-OSS shape are resident at once),
// three roles by block index:
//   [0, n_rt)         router blocks (n_rt = ceil(E / 4)): wavefront w computes logit w;
//   then k*NGS        gate_up blocks: block (slot s, i) streams the 4 gate_up tiles (64 rows)
//                     of slot s's expert that produce h[32i, 32i+32), one tile per wavefront;
//   then H/16         down blocks: one 16-row output tile, wavefront = slot; bias, clamp and the
//                     slot-ordered combine into y.
// Router: each logit in the canonical order (same arithmetic as k_route), written, tagged, into
// nrep = min(kReplicas, readers) copies of the logit vector; reader block b (counted from the
// first gate_up block) reads copy b % nrep and runs the top-k itself (identical arithmetic everywhere,
// so every block selects the same experts and weights). Block 0 also writes the logits,
// indices and weights.
// Matmuls: v_mfma_scale_f32_16x16x128_f8f6f4 with the MXFP4 weights as stored (no decode
// instructions) and the activation as kTerms fp8 terms with E8M0 scales (split8_fp8):
// x is split by every gate_up block into LDS; each gate_up block splits its 32 h values and
// publishes them; down blocks copy the h terms of the kept slots into LDS.
//
// Cross-block signalling without fences over the L2: every value read by another block
// (logits, h terms, flags) is written with agent-scope relaxed atomic stores (write-through)
// and read with agent-scope loads that bypass the L2 (relaxed atomic loads, or LDS-direct
// loads with the same cache policy); a writer waits for its stores to complete (s_waitcnt)
// before it raises the flag that publishes them.
//   * logits: every block adds 1 to its copy's counter after reading the copy; the block that
//     brings it to the copy's reader count clears the copy and the counter and advances the
//     copy's launch number (epoch). Every copy advances exactly once per launch, so all copies
//     hold the same epoch when a launch starts, and a block reads its copy's epoch before its
//     own count can let the copy advance;
//   * h block i of slot s: once its h terms are complete, the gate_up block stores epoch + 1
//     into flag (s, i) of each of kFlagReplicas replicas; down wavefront s waits until the NGS
//     flags of slot s in its replica read epoch + 1. Flags are never cleared: a flag from an
//     earlier launch holds a smaller number.
// So no atomic and no second hop sits between the last h store and the down blocks. Copies and
// counters are zero again when the kernel ends. The blocks that wait on gate_up blocks have
// higher indices, and workgroups are dispatched in index order, so waiting blocks never hold
// back the blocks they wait for; the router wavefronts are in the lowest blocks. Every wait is
// bounded by `spin_limit` polls; a wait that runs out sets the sticky error word, the block
// writes NaN to its outputs, and later launches return NaN at once until the host clears the
// error (it reports it at its next synchronisation and zeroes the signalling area, epochs
// included).
#include <algorithm>

#include "device.hpp"
#include "kernels.hpp"

namespace moe {

// Timeline tracing for development builds (-DMOE_TRACE_TIMELINE): thread 0 of each block
// records the realtime counter (100 MHz) at numbered points into moe_trace_ts[block][8],
// read back with moe_trace_read(). Compiled out otherwise.
#ifdef MOE_TRACE_TIMELINE
__device__ long long moe_trace_ts[4096 * 8];
#define MOE_TRACE(i)                                                                        \
  do {                                                                                      \
    if (threadIdx.x == 0) moe_trace_ts[blockIdx.x * 8 + (i)] = (long long)__builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define MOE_TRACE(i) \
  do {               \
  } while (0)
#endif

constexpr int kLayerWaves = 4;
constexpr int kLayerThreads = 64 * kLayerWaves;
constexpr int kLayerNs = 24;  // steps per tile: K <= 3072
constexpr int kLayerNq = kLayerNs / 4;
using Act = ActRecord<kLayerNs>;  // x and h records: 4 fp8 terms of up to 3072 values

constexpr int kReplicas = 16;

constexpr int kLayerMaxE = 128;

struct LogitCopy {               // kCopyBytes apart
  uint64_t logit[kLayerMaxE];    // (1 << 32) | f32 bits of logit e, 0 when empty
  uint32_t readers_done;
  uint32_t epoch;                // launches completed
};
constexpr size_t kCopyBytes = 1088;
static_assert(sizeof(LogitCopy) <= kCopyBytes, "copy layout");

constexpr int kFlagReplicas = 4;
constexpr int kMaxHBlocks = 128;  // h blocks of 32 per slot (K <= 3072 -> 96)

struct LayerSyncHdr {
  uint32_t err;          // sticky: a bounded wait ran out
  uint32_t pad0[63];
  uint32_t hflag[kFlagReplicas][4][kMaxHBlocks];  // epoch + 1: h block i of slot s is published
};

size_t layer_sync_bytes() { return sizeof(LayerSyncHdr) + kReplicas * kCopyBytes; }

// h records of the slots, in HBM and in a down block's LDS: Act::kBytes apart (a multiple of 16,
// so a record is whole 16-byte lane pieces of LDS-direct loads).
static_assert(Act::kBytes % 16 == 0, "h record size");

__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent64(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent64(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this wavefront issued has completed.
__device__ __forceinline__ void wait_mem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ LogitCopy *logit_copy(void *sync, int r) {
  return reinterpret_cast<LogitCopy *>(reinterpret_cast<uint8_t *>(sync) + sizeof(LayerSyncHdr) +
                                       (size_t)r * kCopyBytes);
}

// Logit of expert e in the canonical order (router_compute's arithmetic for one expert);
// every lane returns it. xr[i] = x[lane + 64 i], zero past H.
template <int RNQ>
__device__ __forceinline__ float router_logit(const uint16_t *rw, const float *rb, const float *xr,
                                              int e, int lane) {
  const uint4 *wq = reinterpret_cast<const uint4 *>(rw + (size_t)e * RNQ * 512) + lane;
  uint4 v[RNQ];
#pragma unroll
  for (int q = 0; q < RNQ; q++) v[q] = wq[q * 64];
  float p = 0.0f;
#pragma unroll
  for (int q = 0; q < RNQ; q++) {
#pragma unroll
    for (int h = 0; h < 8; h++) {
      const uint32_t u = h < 2 ? v[q].x : (h < 4 ? v[q].y : (h < 6 ? v[q].z : v[q].w));
      p = __builtin_fmaf(bf16_to_f32((uint16_t)(u >> (16 * (h & 1)))), xr[8 * q + h], p);
    }
  }
  return canon_nan(wave_sum_xor(p) + rb[e]);
}

// Wavefront 0 of a block: wait for the E tagged logits in copy `cp`; logit 64 q + lane in l[q],
// the copy's epoch in *ep (read in the same polls, and complete before this returns, so before
// the block's count on the copy is issued). Returns false when the wait ran out.
__device__ __forceinline__ bool await_logits(LogitCopy *cp, int E, uint32_t spin_limit, int lane, float (&l)[2],
                                             uint32_t *ep) {
  uint64_t v0 = 0, v1 = 0;
  uint32_t e = 0;
  bool ok = true;
  for (uint32_t n = 0;; n++) {
    e = ld_agent(&cp->epoch);
    v0 = lane < E ? ld_agent64(&cp->logit[lane]) : (1ull << 32);
    v1 = lane + 64 < E ? ld_agent64(&cp->logit[lane + 64]) : (1ull << 32);
    if (__all((v0 >> 32) == 1ull && (v1 >> 32) == 1ull)) break;
    if (n >= spin_limit) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  *ep = (uint32_t)__builtin_amdgcn_readfirstlane((int)e);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  l[0] = __uint_as_float((uint32_t)v0);
  l[1] = __uint_as_float((uint32_t)v1);
  return ok;
}

// The routing on the critical path: the winners -> s_order, and the kept count -> *s_sel. With
// adaptive k the count depends on the probabilities, so the whole top-k runs here; otherwise
// the kept count is min(k, E) and the weights follow later (route_weights), overlapping the
// weight loads.
__device__ __forceinline__ void route_order(const TopkCfg &c, const float (&l)[2], int lane, int (&ord)[4],
                                            int *s_order, float *s_w, int *s_sel) {
  if (c.E <= 64) {
    const float l1[1] = {l[0]};
    wave_topk_order<1>(c, l1, lane, ord);
    if (c.adaptive) wave_topk_weights<1>(c, l1, lane, ord, true, s_order, s_w, s_sel);
  } else {
    wave_topk_order<2>(c, l, lane, ord);
    if (c.adaptive) wave_topk_weights<2>(c, l, lane, ord, true, s_order, s_w, s_sel);
  }
  if (!c.adaptive) {
#pragma unroll
    for (int s = 0; s < 4; s++)
      if (lane == s && s < c.k) s_order[s] = ord[s];
    if (lane == 0) *s_sel = c.k < c.E ? c.k : c.E;
  }
}

// The slot weights -> s_w, when route_order left them for later.
__device__ __forceinline__ void route_weights(const TopkCfg &c, const float (&l)[2], int lane, const int (&ord)[4],
                                              int *s_order, float *s_w, int *s_sel) {
  if (c.adaptive) return;
  if (c.E <= 64) {
    const float l1[1] = {l[0]};
    wave_topk_weights<1>(c, l1, lane, ord, false, s_order, s_w, s_sel);
  } else {
    wave_topk_weights<2>(c, l, lane, ord, false, s_order, s_w, s_sel);
  }
}

// Wavefront 0, after its routing read: count this block as a reader of copy `cp`; the last of
// its `readers` clears it and advances its epoch for the next launch. Two halves, so that the
// atomic's round trip overlaps the weight loads issued between them: release_begin returns the
// count before ours (lane 0), release_end acts on it.
__device__ __forceinline__ uint32_t release_begin(LogitCopy *cp, int lane) {
  uint32_t old = 0;
  if (lane == 0)
    old = __hip_atomic_fetch_add(&cp->readers_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return old;
}

// With fewer blocks than kReplicas only copies 0 .. nrep-1 are written and read; the last
// reader of copy r also advances the epochs of the unused copies r + nrep, r + 2 nrep, ...
__device__ __forceinline__ void release_end(void *sync, int r, int nrep, uint32_t old, int readers, int E,
                                            uint32_t ep, int lane) {
  old = (uint32_t)__builtin_amdgcn_readfirstlane((int)old);
  if (old == (uint32_t)readers - 1) {
    LogitCopy *cp = logit_copy(sync, r);
    if (lane < E) st_agent64(&cp->logit[lane], 0ull);
    if (lane + 64 < E) st_agent64(&cp->logit[lane + 64], 0ull);
    if (lane == 0) st_agent(&cp->readers_done, 0u);
    if (lane < kReplicas && lane % nrep == r) st_agent(&logit_copy(sync, lane)->epoch, ep + 1);
  }
}

template <int RNQ>
__global__ __launch_bounds__(kLayerThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_decode_layer(LayerArgs la) {
  extern __shared__ uint4 smem[];
  __shared__ int s_order[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  __shared__ int s_sel;
  __shared__ int s_flag;
  __shared__ uint32_t s_ep;
  __shared__ int s_wfail[4];
  __shared__ float s_h32[32];
  __shared__ float s_o[4][16];

  const DecodeArgs &a = la.d;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int H = a.H, E = a.E, K = a.k;
  const int NGS = la.n_gu_per_slot;
  const int n_gu = K * NGS, n_rd = n_gu + la.n_dn;         // blocks that read the routing
  const int nrep = n_rd < kReplicas ? n_rd : kReplicas;    // logit copies in use
  constexpr int XI = 8 * RNQ;  // x values per lane of the router chain

  // ---------------------------------------------------------------- router blocks
  // Wavefront w of the first n_rt = ceil(E / 4) blocks computes logit w and leaves; the blocks
  // that wait for the routing come after them.
  if ((int)blockIdx.x < la.n_rt) {
    const int e = (int)blockIdx.x * kLayerWaves + wv;
    if (e < E) {
      float xr[XI];
#pragma unroll
      for (int i = 0; i < XI; i++) xr[i] = a.x[min(lane + 64 * i, H - 1)];
#pragma unroll
      for (int i = 0; i < XI; i++)
        if (lane + 64 * i >= H) xr[i] = 0.0f;
      const float lg = router_logit<RNQ>(a.rw, a.rb, xr, e, lane);
      if (lane < nrep) st_agent64(&logit_copy(la.sync, lane)->logit[e], (1ull << 32) | __float_as_uint(lg));
    }
    return;
  }

  const int b = (int)blockIdx.x - la.n_rt;  // gate_up blocks [0, n_gu), then down blocks
  LayerSyncHdr *hdr = reinterpret_cast<LayerSyncHdr *>(la.sync);
  const int rc = b % nrep;
  LogitCopy *cp = logit_copy(la.sync, rc);
  const int readers = n_rd / nrep + (rc < n_rd % nrep ? 1 : 0);
  const uint32_t err0 = ld_agent(&hdr->err);  // tested late: the load overlaps the routing wait
  const TopkCfg tc{E, K, a.adaptive, a.min_k, a.top1_min, a.margin_min, a.top2_mass};
  const int j = lane & 15, g = lane >> 4;
  MOE_TRACE(0);

  if (b < n_gu) {
    // ================================================================ gate_up block
    // 1. x as kTerms fp8 terms in LDS, 8 values per thread (a quad of lanes = one 32-block);
    //    blocks past H up to nbpx are zeros.
    uint8_t *s_x = reinterpret_cast<uint8_t *>(smem);  // activation record of x
    for (int u = tid; u < 16 * kLayerNs; u += kLayerThreads) {  // uniform trip count per quad
      float xv[8];
      if (8 * u < H) {
        const float4 v0 = reinterpret_cast<const float4 *>(a.x)[2 * u];
        const float4 v1 = reinterpret_cast<const float4 *>(a.x)[2 * u + 1];
        xv[0] = v0.x; xv[1] = v0.y; xv[2] = v0.z; xv[3] = v0.w;
        xv[4] = v1.x; xv[5] = v1.y; xv[6] = v1.z; xv[7] = v1.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = 0.0f;
      }
      uint2 q[kTerms];
      uint32_t s4;
      split8_fp8(xv, q, s4);
      const int bb = u >> 2;
#pragma unroll
      for (int t = 0; t < kTerms; t++) *reinterpret_cast<uint2 *>(s_x + Act::term(t, bb) + 8 * (u & 3)) = q[t];
      if ((u & 3) == 0) {
#pragma unroll
        for (int t = 0; t < kTerms; t++) s_x[Act::scale(t, bb)] = (uint8_t)(s4 >> (8 * t));
      }
    }
    MOE_TRACE(1);
    // 2. routing
    uint32_t rel = 0, ep = 0;
    float l[2];
    int ord[4];
    if (wv == 0) {
      const bool ok = await_logits(cp, E, la.spin_limit, lane, l, &ep);
      if (ok) route_order(tc, l, lane, ord, s_order, s_w, &s_sel);
      rel = release_begin(cp, lane);
      if (lane == 0) s_flag = !ok;
    }
    __syncthreads();
    MOE_TRACE(2);
    const bool timeout = s_flag;
    const int sel = s_sel;
    const int slot = b / NGS;
    if (timeout || err0 || slot >= sel) {  // uniform over the block; no barrier follows
      if (timeout && tid == 0) st_agent(&hdr->err, 1u);
      if (wv == 0) release_end(la.sync, rc, nrep, rel, readers, E, ep, lane);
      return;
    }
    // 3. this wavefront's gate_up tile (rows 16t .. 16t+15 -> h[8t, 8t+8)); bias with it
    const int hb = b - slot * NGS;
    const int t = hb * 4 + wv;
    const uint8_t *rec = a.base + (size_t)s_order[slot] * a.stride;
    TileRegs<kLayerNs> r;
    tile_load<kLayerNs>(r, rec + a.gu_off, a.gu, t, true, lane);
    const float4 bias = reinterpret_cast<const float4 *>(rec + a.gub_off)[t * 4 + g];
    if (b == 0 && wv == 0) {  // block 0 reports the routing (the weights overlap its tile loads)
      route_weights(tc, l, lane, ord, s_order, s_w, &s_sel);
      if (lane < E) a.logits[lane] = l[0];
      if (lane + 64 < E) a.logits[lane + 64] = l[1];
      if (lane < K) {
        a.idx[lane] = s_order[lane];
        a.wts[lane] = s_w[lane];
      }
    }
    uint32_t bsw[kLayerNq];
    load_bsw<kLayerNs>(s_x, bsw, lane);
    const f32x4 acc = tile_mfma_f8<kLayerNs>(r, s_x, bsw, lane);
    float v[4];
    sum_terms(acc, v);
    if (wv == 0) release_end(la.sync, rc, nrep, rel, readers, E, ep, lane);
    MOE_TRACE(3);
    if (j == 0) {
      s_h32[wv * 8 + 2 * g] = swiglu(v[0] + bias.x, v[1] + bias.y, a.limit);
      s_h32[wv * 8 + 2 * g + 1] = swiglu(v[2] + bias.z, v[3] + bias.w, a.limit);
    }
    __syncthreads();
    MOE_TRACE(5);
    // 4. h[32 hb, 32 hb + 32) as kTerms fp8 terms -> this slot's h record (lanes 0..3 of
    //    wavefront 0 hold 8 values each); once the stores are complete, the flags
    if (wv == 0) {
      if (lane < 4) {
        float hv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) hv[i] = s_h32[8 * lane + i];
        uint2 q[kTerms];
        uint32_t s4;
        split8_fp8(hv, q, s4);
        uint8_t *rec_h = la.hterm + (size_t)slot * Act::kBytes;
#pragma unroll
        for (int tt = 0; tt < kTerms; tt++) {
          uint32_t *dst = reinterpret_cast<uint32_t *>(rec_h + Act::term(tt, hb) + 8 * lane);
          st_agent(dst, q[tt].x);
          st_agent(dst + 1, q[tt].y);
        }
        if (lane == 0) {
#pragma unroll
          for (int tt = 0; tt < kTerms; tt++)
            __hip_atomic_store(rec_h + Act::scale(tt, hb), (uint8_t)(s4 >> (8 * tt)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      wait_mem();
      MOE_TRACE(6);
      if (lane < kFlagReplicas) st_agent(&hdr->hflag[lane][slot][hb], ep + 1);
      MOE_TRACE(4);
    }
    return;
  }

  // ================================================================== down block
  const int t = b - n_gu, slot = wv;
  uint8_t *s_h = reinterpret_cast<uint8_t *>(smem);  // [slot] activation records of h
  // 1. routing
  uint32_t rel = 0, ep = 0;
  float l[2];
  int ord[4];
  if (wv == 0) {
    const bool ok = await_logits(cp, E, la.spin_limit, lane, l, &ep);
    if (ok) route_order(tc, l, lane, ord, s_order, s_w, &s_sel);
    rel = release_begin(cp, lane);
    if (lane == 0) {
      s_flag = !ok || err0;
      s_ep = ep;
    }
  }
  __syncthreads();
  MOE_TRACE(1);
  const bool timeout = s_flag;
  const int sel = timeout ? 0 : s_sel;
  const bool ok = slot < sel && slot < K;
  const uint8_t *rec = a.base + (size_t)(ok ? s_order[slot] : 0) * a.stride;
  // 2. the down tile and its bias, streamed while gate_up runs
  TileRegs<kLayerNs> r;
  tile_load<kLayerNs>(r, rec + a.dn_off, a.dn, ok ? t : 0, ok, lane);
  const float4 bias = reinterpret_cast<const float4 *>(rec + a.dnb_off)[(ok ? t : 0) * 4 + g];
  if (wv == 0) {
    release_end(la.sync, rc, nrep, rel, readers, E, ep, lane);
    if (!timeout) route_weights(tc, l, lane, ord, s_order, s_w, &s_sel);  // read after the combine's barrier
  }
  // 3. wavefront `slot`: wait for the NGS h blocks of its slot, then bring the slot's h record
  //    into LDS, 1 KB per instruction, straight into LDS (the last instruction only on the lanes
  //    inside the record, so no byte of a neighbour's record is written)
  bool wfail = false;
  if (ok) {
    const uint32_t want = s_ep + 1;
    const uint32_t *f = hdr->hflag[t % kFlagReplicas][slot];
    for (uint32_t n = 0;; n++) {
      const bool d0 = lane >= NGS || ld_agent(f + lane) == want;
      const bool d1 = lane + 64 >= NGS || ld_agent(f + lane + 64) == want;
      if (__all(d0 && d1)) break;
      if (n >= la.spin_limit) {
        wfail = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    MOE_TRACE(2);
    if (!wfail) {
      const uint8_t *src = la.hterm + (size_t)slot * Act::kBytes;
      uint8_t *dst = s_h + (size_t)slot * Act::kBytes;
#pragma unroll
      for (int cix = 0; cix < Act::kBytes / 1024; cix++)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(src + (size_t)cix * 1024) + lane,
                                         (__attribute__((address_space(3))) void *)(dst + (size_t)cix * 1024),
                                         16, 0, 16);
      constexpr int kTail = Act::kBytes % 1024;
      if (kTail && 16 * lane < kTail)
        __builtin_amdgcn_global_load_lds(
            reinterpret_cast<const uint4 *>(src + (size_t)(Act::kBytes - kTail)) + lane,
            (__attribute__((address_space(3))) void *)(dst + (size_t)(Act::kBytes - kTail)), 16, 0, 16);
      wait_mem();
    }
    MOE_TRACE(3);
  }
  if (lane == 0) s_wfail[wv] = wfail;
  if (ok && !wfail) {
    const uint8_t *hrec = s_h + (size_t)slot * Act::kBytes;
    uint32_t bsw[kLayerNq];
    load_bsw<kLayerNs>(hrec, bsw, lane);
    const f32x4 acc = tile_mfma_f8<kLayerNs>(r, hrec, bsw, lane);
    float v[4];
    sum_terms(acc, v);
    if (j == 0) {
      s_o[slot][g * 4 + 0] = canon_nan(rclamp(v[0] + bias.x, -65504.0f, 65504.0f));
      s_o[slot][g * 4 + 1] = canon_nan(rclamp(v[1] + bias.y, -65504.0f, 65504.0f));
      s_o[slot][g * 4 + 2] = canon_nan(rclamp(v[2] + bias.z, -65504.0f, 65504.0f));
      s_o[slot][g * 4 + 3] = canon_nan(rclamp(v[3] + bias.w, -65504.0f, 65504.0f));
    }
  }
  __syncthreads();
  MOE_TRACE(5);
  const bool failed = timeout || s_wfail[0] || s_wfail[1] || s_wfail[2] || s_wfail[3];
  if (tid < 16) {  // session.rs:974-980: y = 0; y += w_s * out_s in slot order
    float y = 0.0f;
    if (failed) {
      y = __uint_as_float(0x7FC00000u);
    } else {
      for (int s = 0; s < 4 && s < K; s++)
        if (s < sel) y = y + s_w[s] * s_o[s][tid];
    }
    a.y[t * 16 + tid] = canon_nan(y);
  }
  MOE_TRACE(4);
  if (tid == 0 && failed) st_agent(&hdr->err, 1u);
}

size_t decode_layer_lds(const LayerArgs &) { return (size_t)4 * Act::kBytes; }

// Derived geometry of the one-launch kernel for la.d (the host fills la.d, sync, hterm and
// spin_limit).
void layer_geometry(LayerArgs &la) {
  la.n_gu_per_slot = (int)(la.d.gu.tiles / 4);
  la.n_dn = (int)la.d.dn.tiles;
  la.n_rt = (la.d.E + kLayerWaves - 1) / kLayerWaves;
}

size_t layer_hterm_bytes() { return (size_t)4 * Act::kBytes; }

bool decode_layer_supported(const LayerArgs &la) {
  const DecodeArgs &a = la.d;
  return a.k >= 1 && a.k <= 4 && a.E >= 1 && a.E <= kLayerMaxE && a.k <= a.E && a.rnq >= 1 && a.rnq <= 6 &&
         (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
         a.gu.ns <= (uint32_t)kLayerNs && a.dn.ns <= (uint32_t)kLayerNs && a.H % 32 == 0 &&
         a.I % 32 == 0 && a.gu.tiles % 4 == 0 && a.gu.tiles / 4 <= (uint32_t)kMaxHBlocks &&
         la.n_rt == (a.E + kLayerWaves - 1) / kLayerWaves &&
         la.n_rt + a.k * la.n_gu_per_slot + la.n_dn <= kLayerMaxBlocks;
}

hipError_t launch_decode_layer(const LayerArgs &la, hipStream_t s) {
  const DecodeArgs &a = la.d;
  if (!decode_layer_supported(la) || !la.sync || !la.hterm) return hipErrorInvalidValue;
  const dim3 grid(la.n_rt + a.k * la.n_gu_per_slot + la.n_dn), block(kLayerThreads);
  const size_t lds = decode_layer_lds(la);
  switch (a.rnq) {  // router chain length per lane, in 16-byte loads (6 for H = 2880)
    case 1: hipLaunchKernelGGL(k_decode_layer<1>, grid, block, lds, s, la); break;
    case 2: hipLaunchKernelGGL(k_decode_layer<2>, grid, block, lds, s, la); break;
    case 3: hipLaunchKernelGGL(k_decode_layer<3>, grid, block, lds, s, la); break;
    case 4: hipLaunchKernelGGL(k_decode_layer<4>, grid, block, lds, s, la); break;
    case 5: hipLaunchKernelGGL(k_decode_layer<5>, grid, block, lds, s, la); break;
    default: hipLaunchKernelGGL(k_decode_layer<6>, grid, block, lds, s, la); break;
  }
  return hipGetLastError();
}

}  // namespace moe

#ifdef MOE_TRACE_TIMELINE
extern "C" int moe_trace_read(long long *out, int n_blocks) {
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(moe::moe_trace_ts), (size_t)n_blocks * 8 * 8, 0,
                                  hipMemcpyDeviceToHost);
}
#endif
