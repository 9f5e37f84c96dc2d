// Single-token MoE layer for gfx950 in ONE launch — the MoE block of
// Session::decode_step_inner (session.rs:818-980) for one token, with the down projection's
// weight stream overlapping the gate_up phase.
//
// Blocks of 4 wavefronts, sized so the grid is two blocks per CU and every CU streams about the
// same weight bytes (a CU's share of the HBM stream, not its block count, sets when it is done):
//   [0, n_rt)         router blocks (n_rt = ceil(E / 4)): wavefront w computes logit w;
//   then n_gu         gate_up blocks: block b streams gate_up tiles 4b .. 4b+3 (16 rows each, one
//                     per wavefront, one chunk of 32 h values of one slot), and X of them (spread
//                     evenly) one more tile, split by K over the 4 wavefronts; the tiles are
//                     numbered slot-major over the k * TPS tiles of the chosen experts;
//   then H/16         down blocks: one 16-row output tile, wavefront = slot; bias, clamp and the
//                     slot-ordered combine into y.
// Router: each logit in the canonical order (same arithmetic as k_route), written, tagged, into
// nrep = min(kReplicas, readers) copies of the logit vector; reader block b (counted from the
// first gate_up block) reads copy b % nrep and runs the top-k itself (identical arithmetic
// everywhere, so every block selects the same experts and weights). Gate_up block 0 also writes
// the logits, indices and weights.
// Matmuls: v_mfma_scale_f32_16x16x128_f8f6f4 with the MXFP4 weights as stored (no decode
// instructions). x enters as kTerms fp8 terms with per-block E8M0 scales (split8_fp8, split by
// every gate_up block into LDS). h is bounded (|h| <= max(limit, 1/4) * (limit + 1)), so each
// gate_up tile splits its 8 values into kTerms fp8 terms with fixed exponents (split2_fp8_fixed)
// without waiting for the rest of the 32-value block, and its block stores the 32-byte pieces of
// its tiles as whole lines of the slot's tile-major h record; down blocks copy the records of
// the kept slots into LDS.
//
// Cross-block signalling without fences over the L2: every value read by another block
// (logits, h records, flags) is written with agent-scope relaxed atomic stores (write-through)
// and read with agent-scope loads that bypass the L2 (relaxed atomic loads, or LDS-direct
// loads with the same cache policy); a writer waits for its stores to complete (s_waitcnt)
// before it raises the flag that publishes them.
//   * logits: every block adds 1 to its copy's counter after reading the copy; the block that
//     brings it to the copy's reader count clears the copy and the counter and advances the
//     copy's launch number (epoch) and those of the unused copies it stands for. Every copy
//     advances exactly once per launch, so all copies hold the same epoch when a launch starts,
//     and a block reads its copy's epoch before its own count can let the copy advance;
//   * h: once every h store of a gate_up block is complete, it stores epoch + 1 into its flag in
//     each of kFlagReplicas replicas; wavefront 0 of a down block waits until all n_gu flags of
//     its replica read epoch + 1. Flags are never cleared: a flag from an earlier launch holds a
//     smaller number.
// Copies and counters are zero again when the kernel ends. The blocks that wait on others have
// higher indices, and workgroups are dispatched in index order, so waiting blocks never hold
// back the blocks they wait for. Every wait is bounded by `spin_limit` polls; a wait that runs
// out sets the sticky error word, the block writes NaN to its outputs, and later launches return
// NaN at once until the host clears the error (it reports it at its next synchronisation and
// zeroes the signalling area, epochs included).
#include <algorithm>
#include <cmath>

#include "device.hpp"
#include "kernels.hpp"

namespace moe {

// Timeline tracing for development builds (-DMOE_TRACE_TIMELINE): thread 0 of each block
// records the realtime counter (100 MHz) at numbered points into moe_trace_ts[block][16],
// read back with moe_trace_read(). Compiled out otherwise.
#ifdef MOE_TRACE_TIMELINE
__device__ long long moe_trace_ts[4096 * 16];
#define MOE_TRACE(i)                                                                        \
  do {                                                                                      \
    if (threadIdx.x == 0) moe_trace_ts[blockIdx.x * 16 + (i)] = (long long)__builtin_amdgcn_s_memrealtime(); \
  } while (0)
// slot 7: where the block runs, XCC_ID << 16 | HW_ID bits 8..15 (CU, shader array, engine)
#define MOE_TRACE_WHERE()                                                                         \
  do {                                                                                            \
    if (threadIdx.x == 0)                                                                         \
      moe_trace_ts[blockIdx.x * 16 + 7] = ((long long)__builtin_amdgcn_s_getreg((15 << 11) | 20) << 16) | \
                                         ((__builtin_amdgcn_s_getreg((31 << 11) | 4) >> 8) & 0xFF); \
  } while (0)
#else
#define MOE_TRACE_WHERE() \
  do {                    \
  } while (0)
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

constexpr int kFlagReplicas = 16;
constexpr int kLayerMaxK = 32 * 4 * kLayerNs;      // 3072: longest K of a tile
constexpr int kLayerMaxTps = 2 * kLayerMaxK / 16;  // gate_up tiles per slot (I <= 3072 -> 384)
constexpr int kLayerMaxGu = kLayerMaxTps;          // gate_up blocks (4 slots x 384 tiles / 4)
static_assert(kLayerMaxGu % 64 == 0, "flag poll shape");

struct LayerSyncHdr {
  uint32_t err;          // sticky: a bounded wait ran out
  uint32_t pad0[63];
  uint32_t gflag[kFlagReplicas][kLayerMaxGu];  // epoch + 1: gate_up block i has published its h
};

size_t layer_sync_bytes() { return sizeof(LayerSyncHdr) + kReplicas * kCopyBytes; }

constexpr int kLayerMaxHexp = 5;

// h record of a slot (HBM, and a down block's LDS): tile-major, gate_up tile t's 8 values
// h[8t, 8t+8) at 32 t, term j of them at 32 t + 8 j (value i at byte i), kTerms = 4 fp8 terms
// with the fixed exponents hexp - 4j; values past I are zero. 12 KB for K <= 3072.
constexpr int kHRecBytes = kLayerMaxK / 8 * 32;
static_assert(kTerms == 4, "h record piece = 4 terms x 8 bytes");

// LDS-DMA of 16 bytes per lane (lane l's bytes land at lds + 16 l) with the agent-coherent cache
// policy (sc1: the h records are written by other blocks with agent-scope stores), written as
// inline assembly so that the compiler's wait tracking does not see it (with the builtin it makes
// every later LDS read wait for all DMAs in flight); the caller waits with counted vmcnt. Every
// LDS-DMA of this kernel goes through here, so the compiler keeps no value of its own in m0.
__device__ __forceinline__ void lds_dma16_sc1(const void *g, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(g), "s"(la) : "memory", "m0");
}

// The down sweep of a loaded down tile against its slot's h record: the record (tile-major, 512
// bytes per MFMA step) comes into LDS at hdst by 12 LDS-DMAs of 1 KB, two steps each, and the MFMAs
// start as soon as the first KB has landed: step q's bytes lie in DMA q / 2, complete once at most
// 11 - q / 2 of the wavefront's DMAs are outstanding (they complete in order). B operand of
// tile_mfma_f8 from the tile-major layout: lane (column j = term j % 4, group gb) takes, for step s,
// values 16(gb&1) .. +15 of block 4s + (gb>>1) (two 8-value pieces, 32 bytes apart) and the same
// values of block 4s + 2 + (gb>>1) (256 bytes further); sb = the lane's B scale byte in every byte
// (term j's fixed scale, 0 for columns >= kTerms). Step s accumulates into chain s % 4 (four short
// dependent chains), summed (c0 + c1) + (c2 + c3) at the end.
template <int NSMAX>
__device__ __forceinline__ f32x4 tile_mfma_h_stream(const TileRegs<NSMAX> &r, const uint8_t *hsrc, uint8_t *hdst,
                                                    uint32_t sb, int lane) {
  constexpr int kD = kHRecBytes / 1024;  // DMAs of the record
  static_assert(NSMAX == 2 * kD, "two MFMA steps per DMA");
#pragma unroll
  for (int c = 0; c < kD; c++) lds_dma16_sc1(hsrc + 1024 * c + 16 * lane, hdst + 1024 * c);
  const int j = lane & 15, gb = lane >> 4;
  const uint8_t *bt = hdst + 128 * (gb >> 1) + 64 * (gb & 1) + 8 * (j & (kTerms - 1));
  f32x4 acc[4];
#pragma unroll
  for (int c = 0; c < 4; c++) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int PD = 2;  // B of step s is read two steps ahead
  uint2 pb[PD][4];
  __builtin_amdgcn_s_waitcnt(vm_wait(kD - 1));  // steps 0 and 1
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
  for (int s = 0; s < PD; s++) {
    pb[s][0] = *reinterpret_cast<const uint2 *>(bt + 512 * s);
    pb[s][1] = *reinterpret_cast<const uint2 *>(bt + 512 * s + 32);
    pb[s][2] = *reinterpret_cast<const uint2 *>(bt + 512 * s + 256);
    pb[s][3] = *reinterpret_cast<const uint2 *>(bt + 512 * s + 288);
  }
#pragma unroll
  for (int s = 0; s < NSMAX; s++) {
    const uint2 b0 = pb[s % PD][0], b1 = pb[s % PD][1], b2 = pb[s % PD][2], b3 = pb[s % PD][3];
    if (s + PD < NSMAX) {
      if ((s + PD) % 2 == 0) {  // the first step of a DMA: wait for it
        wait_vmcnt_upto15(kD - 1 - (s + PD) / 2);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
      }
      pb[s % PD][0] = *reinterpret_cast<const uint2 *>(bt + 512 * (s + PD));
      pb[s % PD][1] = *reinterpret_cast<const uint2 *>(bt + 512 * (s + PD) + 32);
      pb[s % PD][2] = *reinterpret_cast<const uint2 *>(bt + 512 * (s + PD) + 256);
      pb[s % PD][3] = *reinterpret_cast<const uint2 *>(bt + 512 * (s + PD) + 288);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint4 a = r.raw[s];
    const i32x8 A = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    const i32x8 B = {(int)b0.x, (int)b0.y, (int)b1.x, (int)b1.y, (int)b2.x, (int)b2.y, (int)b3.x, (int)b3.y};
    acc[s % 4] = mfma_fp4_fp8(s & 3, A, B, acc[s % 4], r.sw[s / 4], sb);
  }
  return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// The extra gate_up tile of gate_up block b (index e in [0, X) of the X = k TPS - 4 n_gu tiles past
// the first 4 n_gu), or -1. Workgroups are dispatched in index order, breadth first over the CUs,
// so with a grid of G in (n_cu, 2 n_cu] blocks i and i + n_cu share a CU (measured: 97 % of the
// pairs), and a CU's share of the weight stream sets when it is done (measured: a CU streaming 10
// tiles finishes its gate_up tiles ~2.3 us after one streaming 8). The extra tiles therefore go
// first to the gate_up blocks whose partner is a router block or missing (class 0), then to those
// whose partner is a down block (class 1), then to the lower (class 2) and last to the upper
// (class 3) block of each gate_up pair: every CU streams at most one tile more than the lightest
// CU of two full blocks. The classes partition the gate_up blocks [R, R + n_gu) into the
// intervals below; a block's rank is the count of blocks before it in class order. Other grids
// spread the extra tiles evenly.
__host__ __device__ inline int layer_extra_tile(int b, int n_rt, int n_gu, int n_dn, int n_cu, int X) {
  const int G = n_rt + n_gu + n_dn, N = n_cu, R = n_rt, i = R + b;
  if (G <= N || G > 2 * N || R >= N) {
    const int lo = (int)((long long)b * X / n_gu), hi = (int)((long long)(b + 1) * X / n_gu);
    return hi > lo ? lo : -1;
  }
  const int iv[4][2] = {{G - N, N + R},                                   // partner router / none
                        {R + n_gu - N, G - N},                            // partner down
                        {R - N, R + n_gu - N < G - N ? R + n_gu - N : G - N},  // lower of a gate_up pair
                        {N + R, N + R + n_gu}};                           // upper of a gate_up pair
  int rank = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const int lo = iv[c][0] > R ? iv[c][0] : R, hi = iv[c][1] < R + n_gu ? iv[c][1] : R + n_gu;
    if (i >= lo && i < hi) return rank + (i - lo) < X ? rank + (i - lo) : -1;
    rank += hi > lo ? hi - lo : 0;
  }
  return -1;  // (unreachable: the classes cover every gate_up block)
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
__global__ __launch_bounds__(kLayerThreads) __attribute__((amdgpu_waves_per_eu(2, 3))) void k_decode_layer(LayerArgs la) {
  extern __shared__ uint4 smem[];
  __shared__ int s_order[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  __shared__ int s_sel;
  __shared__ int s_flag;
  __shared__ uint32_t s_ep;
  __shared__ int s_wfail[1];
  __shared__ float s_rinv;
  __shared__ float s_o[4][16];
  __shared__ __align__(16) uint8_t s_hp[32 * (kLayerWaves + 1)];  // h record pieces of a gate_up block's tiles
  __shared__ __align__(16) float s_xp[kLayerWaves][16];             // the extra tile's partial sums

  const DecodeArgs &a = la.d;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int H = a.H, E = a.E, K = a.k;
  const int TPS = la.n_tps;                                 // gate_up tiles per slot
  const int n_gu = la.n_gu, n_rd = n_gu + la.n_dn;          // blocks that read the routing
  const int nrep = n_rd < kReplicas ? n_rd : kReplicas;     // logit copies in use
  constexpr int XI = 8 * RNQ;  // x values per lane of the router chain

  // ---------------------------------------------------------------- router blocks
  // Wavefront w of the first n_rt = ceil(E / 4) blocks computes logit w and leaves; the blocks
  // that wait for the routing come after them.
  if ((int)blockIdx.x < la.n_rt) {
    const int e = (int)blockIdx.x * kLayerWaves + wv;
    MOE_TRACE(0);
    MOE_TRACE_WHERE();
    if (e < E) {
      float xr[XI];
#pragma unroll
      for (int i = 0; i < XI; i++) xr[i] = a.x[min(lane + 64 * i, H - 1)];
#pragma unroll
      for (int i = 0; i < XI; i++)
        if (lane + 64 * i >= H) xr[i] = 0.0f;
      if (la.gamma) {  // the block forward: the router reads RMSNorm(x) gamma (rms_inv_wave's order)
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < XI; i++) {
          const float sq = xr[i] * xr[i];
          p = p + sq;
        }
        const float r = 1.0f / sqrtf(wave_sum_xor(p) / (float)H + la.eps);
#pragma unroll
        for (int i = 0; i < XI; i++) {
          const float v = xr[i] * r;
          xr[i] = lane + 64 * i < H ? v * la.gamma[min(lane + 64 * i, H - 1)] : 0.0f;
        }
      }
      const float lg = router_logit<RNQ>(a.rw, a.rb, xr, e, lane);
      MOE_TRACE(1);
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
  MOE_TRACE_WHERE();

  if (b < n_gu) {
    // ================================================================ gate_up block
    // 1. x as kTerms fp8 terms in LDS, 8 values per thread (a quad of lanes = one 32-block);
    //    blocks past H up to nbpx are zeros.
    uint8_t *s_x = reinterpret_cast<uint8_t *>(smem);  // activation record of x
    if (la.gamma) {  // the block forward: x is RMSNorm(x) gamma; wavefront 0 finds 1 / rms
      if (wv == 0) {
        const float r = rms_inv_wave(a.x, H, la.eps, lane);
        if (lane == 0) s_rinv = r;
      }
      __syncthreads();
    }
    for (int u = tid; u < 16 * kLayerNs; u += kLayerThreads) {  // uniform trip count per quad
      float xv[8];
      if (8 * u < H) {
        const float4 v0 = reinterpret_cast<const float4 *>(a.x)[2 * u];
        const float4 v1 = reinterpret_cast<const float4 *>(a.x)[2 * u + 1];
        xv[0] = v0.x; xv[1] = v0.y; xv[2] = v0.z; xv[3] = v0.w;
        xv[4] = v1.x; xv[5] = v1.y; xv[6] = v1.z; xv[7] = v1.w;
        if (la.gamma) {
          const float r = s_rinv;
          const float4 g0 = reinterpret_cast<const float4 *>(la.gamma)[2 * u];
          const float4 g1 = reinterpret_cast<const float4 *>(la.gamma)[2 * u + 1];
          const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const float v = xv[i] * r;
            xv[i] = v * gv[i];
          }
        }
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
      if (lane == 0) {
        s_flag = !ok;
        s_ep = ep;
      }
    }
    __syncthreads();
    MOE_TRACE(2);
    const bool timeout = s_flag;
    const int sel = s_sel;
    if (timeout || err0) {  // uniform over the block; no barrier follows
      if (timeout && tid == 0) st_agent(&hdr->err, 1u);
      if (wv == 0) release_end(la.sync, rc, nrep, rel, readers, E, ep, lane);
      return;
    }
    ep = s_ep;
    // 3. this wavefront's gate_up tile: tile 4b + wv; and for X of the blocks (spread evenly)
    //    one of the X = k * TPS - 4 * n_gu tiles past the first 4 * n_gu (X <= n_gu; which blocks:
    //    layer_extra_tile), split by K over the 4 wavefronts (steps [6 wv, 6 wv + 6)), so its
    //    bytes stream with the others.
    //    Tile u is row tile u % TPS (rows 16 t .. 16 t + 15 -> h[8t, 8t+8)) of slot u / TPS;
    //    tiles of dropped slots are skipped (uniformly over the block: 4b .. 4b+3 share a slot).
    const int n_tiles = K * TPS, W = 4 * n_gu, X = n_tiles > W ? n_tiles - W : 0;
    const int ex = X > 0 ? layer_extra_tile(b, la.n_rt, n_gu, la.n_dn, la.n_cu, X) : -1;
    const int u0 = 4 * b + wv, ux = ex >= 0 ? W + ex : n_tiles;
    const int slot0 = u0 / TPS, tt0 = u0 - slot0 * TPS, slotx = ux / TPS, ttx = ux - slotx * TPS;
    const bool act0 = u0 < n_tiles && slot0 < sel, actx = ux < n_tiles && slotx < sel;
    const uint8_t *rec0 = a.base + (size_t)(act0 ? s_order[slot0] : s_order[0]) * a.stride;
    const uint8_t *recx = a.base + (size_t)(actx ? s_order[slotx] : s_order[0]) * a.stride;
    TileRegs<kLayerNs> r;
    tile_load<kLayerNs>(r, rec0 + a.gu_off, a.gu, tt0, act0, lane);
    const float4 bias0 = act0 ? reinterpret_cast<const float4 *>(rec0 + a.gub_off)[tt0 * 4 + g] : make_float4(0.f, 0.f, 0.f, 0.f);
    constexpr int kXs = (kLayerNs + kLayerWaves - 1) / kLayerWaves;  // extra-tile steps per wavefront
    uint4 xraw[kXs];
    uint32_t xsw[kLayerNq];
    {
      const int ns = (int)a.gu.ns, nb = (int)a.gu.nb;
      const uint4 *wp = reinterpret_cast<const uint4 *>(recx + a.gu_off) + (size_t)ttx * 16 * nb;
      const uint32_t *sp = reinterpret_cast<const uint32_t *>(recx + a.gu_off + pack_weight_bytes(a.gu)) + (size_t)ttx * a.gu.nq * 64;
#pragma unroll
      for (int k = 0; k < kXs; k++) {
        const int st = kXs * wv + k;
        xraw[k] = make_uint4(0u, 0u, 0u, 0u);
        if (actx && st < ns && 4 * st + g < nb) {
          const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wp) + st * 64 + lane);
          xraw[k] = make_uint4(v.x, v.y, v.z, v.w);
        }
      }
#pragma unroll
      for (int q = 0; q < kLayerNq; q++) xsw[q] = actx && q < (int)a.gu.nq ? sp[q * 64 + lane] : 0u;
    }
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
    // 4. the tile: MFMA sweep, bias, SwiGLU; lanes j == 0 hold h[8t + 2g], h[8t + 2g + 1], split
    //    them into the fixed-exponent fp8 terms: the tile's 32-byte piece of the h record, staged
    //    in LDS. The extra tile: each wavefront's partial sums to LDS.
    if (act0) {
      const f32x4 acc = tile_mfma_f8<kLayerNs>(r, s_x, bsw, lane);
      float v[4];
      sum_terms(acc, v);
      if (wv == 0) release_end(la.sync, rc, nrep, rel, readers, E, ep, lane);
      if (j == 0) {
        const float h0 = swiglu(v[0] + bias0.x, v[1] + bias0.y, a.limit);
        const float h1 = swiglu(v[2] + bias0.z, v[3] + bias0.w, a.limit);
        const uint64_t q = split2_fp8_fixed(h0, h1, la.hexp);
#pragma unroll
        for (int te = 0; te < kTerms; te++)
          *reinterpret_cast<uint16_t *>(s_hp + 32 * wv + 8 * te + 2 * g) = (uint16_t)(q >> (16 * te));
      }
    } else if (wv == 0) {
      release_end(la.sync, rc, nrep, rel, readers, E, ep, lane);
    }
    if (actx) {
      f32x4 acc;
      switch (wv) {  // the step range as a constant, so every scale word index is static
        case 0: acc = tile_mfma_f8_steps<kLayerNs, kXs, 0>(xraw, xsw, s_x, bsw, lane); break;
        case 1: acc = tile_mfma_f8_steps<kLayerNs, kXs, kXs>(xraw, xsw, s_x, bsw, lane); break;
        case 2: acc = tile_mfma_f8_steps<kLayerNs, kXs, 2 * kXs>(xraw, xsw, s_x, bsw, lane); break;
        default: acc = tile_mfma_f8_steps<kLayerNs, kXs, 3 * kXs>(xraw, xsw, s_x, bsw, lane); break;
      }
      float v[4];
      sum_terms(acc, v);
      if (j == 0) *reinterpret_cast<float4 *>(&s_xp[wv][4 * g]) = make_float4(v[0], v[1], v[2], v[3]);
    }
    MOE_TRACE(3);
    __syncthreads();
    MOE_TRACE(5);
    // 5. the block's 4 consecutive tiles are 128 contiguous bytes of one slot's record: whole
    //    lines, stored by 16 lanes of wavefront 0. Wavefront 3 sums the extra tile's partials (in
    //    wavefront order), finishes it like the others and stores its 32 bytes.
    if (wv == 0 && act0 && lane < 16)
      st_agent64(reinterpret_cast<uint64_t *>(la.hterm + (size_t)slot0 * kHRecBytes + 32 * tt0) + lane,
                 *reinterpret_cast<const uint64_t *>(s_hp + 8 * lane));
    if (wv == kLayerWaves - 1 && actx) {
      if (j == 0) {
        const float4 biasx = reinterpret_cast<const float4 *>(recx + a.gub_off)[ttx * 4 + g];
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = ((s_xp[0][4 * g + e] + s_xp[1][4 * g + e]) + s_xp[2][4 * g + e]) + s_xp[3][4 * g + e];
        const float h0 = swiglu(v[0] + biasx.x, v[1] + biasx.y, a.limit);
        const float h1 = swiglu(v[2] + biasx.z, v[3] + biasx.w, a.limit);
        const uint64_t q = split2_fp8_fixed(h0, h1, la.hexp);
#pragma unroll
        for (int te = 0; te < kTerms; te++)
          *reinterpret_cast<uint16_t *>(s_hp + 32 * kLayerWaves + 8 * te + 2 * g) = (uint16_t)(q >> (16 * te));
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (lane < 4)
        st_agent64(reinterpret_cast<uint64_t *>(la.hterm + (size_t)slotx * kHRecBytes + 32 * ttx) + lane,
                   *reinterpret_cast<const uint64_t *>(s_hp + 32 * kLayerWaves + 8 * lane));
    }
    wait_mem();
    MOE_TRACE(6);
    __syncthreads();
    if (wv == 0 && lane < kFlagReplicas) st_agent(&hdr->gflag[lane][b], ep + 1);
    MOE_TRACE(4);
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
  MOE_TRACE(9);
  if (wv == 0) {
    release_end(la.sync, rc, nrep, rel, readers, E, ep, lane);
    if (!timeout) route_weights(tc, l, lane, ord, s_order, s_w, &s_sel);  // read after the combine's barrier
  }
  // 3. wavefront 0 waits until every gate_up block has published (its replica of the block flags
  //    reads epoch + 1); then wavefront `slot` brings its slot's h record (the kTerms term rows)
  //    into LDS, 1 KB per instruction, straight into LDS, and sweeps it as it lands
  bool wfail = false;
  if (wv == 0 && sel > 0) {
    const uint32_t want = s_ep + 1;
    const uint32_t *f = hdr->gflag[t % kFlagReplicas];
    for (uint32_t n = 0;; n++) {
      // all of a poll's loads in flight at once (flags past n_gu are in bounds and ignored); a
      // short-circuit test would issue them one round trip after another
      uint32_t fv[kLayerMaxGu / 64];
#pragma unroll
      for (int i = 0; i < kLayerMaxGu / 64; i++) fv[i] = ld_agent(f + lane + 64 * i);
      bool d = true;
#pragma unroll
      for (int i = 0; i < kLayerMaxGu / 64; i++) d = d & ((lane + 64 * i >= n_gu) | (fv[i] == want));
      if (__all(d)) break;
      if (n >= la.spin_limit) {
        wfail = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  if (wv == 0 && lane == 0) s_wfail[0] = wfail;
  __syncthreads();
  MOE_TRACE(2);
  wfail = s_wfail[0];
  MOE_TRACE(3);
  if (ok && !wfail) {
    // the slot's h record into LDS, the MFMAs following the DMAs as they land
    const uint32_t sb = j < kTerms ? (uint32_t)(127 + la.hexp - 4 * j) * 0x01010101u : 0u;
    const f32x4 acc = tile_mfma_h_stream<kLayerNs>(r, la.hterm + (size_t)slot * kHRecBytes,
                                                   s_h + (size_t)slot * kHRecBytes, sb, lane);
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
  const bool failed = timeout || wfail;
  if (tid < 16) {  // session.rs:974-980: y = 0; y += w_s * out_s in slot order
    float y = 0.0f;
    if (failed) {
      y = __uint_as_float(0x7FC00000u);
    } else {
      for (int s = 0; s < 4 && s < K; s++)
        if (s < sel) y = y + s_w[s] * s_o[s][tid];
    }
    if (la.gamma) y = a.x[t * 16 + tid] + y;  // the block forward's residual (session.rs:982-994)
    a.y[t * 16 + tid] = canon_nan(y);
  }
  MOE_TRACE(4);
  if (tid == 0 && failed) st_agent(&hdr->err, 1u);
}

size_t decode_layer_lds(const LayerArgs &) { return (size_t)4 * Act::kBytes; }
static_assert(kHRecBytes <= Act::kBytes, "down blocks hold 4 h records");

// Derived geometry of the one-launch kernel for la.d on a device of n_cu compute units (the
// host fills la.d, sync, hterm and spin_limit): router blocks, down blocks, and as many gate_up
// blocks as make the grid two blocks per CU (each CU then streams about the same bytes: 4 or 5
// weight tiles per block), within [ceil(tiles / 5), ceil(tiles / 4)] so a block takes 4 or 5
// tiles.
void layer_geometry(LayerArgs &la, int n_cu) {
  const DecodeArgs &a = la.d;
  la.n_tps = (int)a.gu.tiles;
  la.n_dn = (int)a.dn.tiles;
  la.n_rt = (a.E + kLayerWaves - 1) / kLayerWaves;
  la.n_cu = n_cu;
  const int tiles = a.k * la.n_tps;
  const int lo = (tiles + 4) / 5, hi = (tiles + 3) / 4;
  la.n_gu = std::min(hi, std::max(lo, 2 * n_cu - la.n_rt - la.n_dn));
  la.hexp = layer_hexp(a.limit);
}

// The exponent of the first h term: |h| <= max(limit, 1/4) * (limit + 1) for every finite h
// (gate <= limit, |up| <= limit, gate * sigmoid(1.702 gate) >= -1/4), so h * 2^-hexp stays below
// 256, inside e4m3's range. Large limits leave small values below the last term's resolution
// (2^(hexp - 21)); kLayerMaxHexp bounds that at 2^-16.
int layer_hexp(float limit) {
  const float bound = std::max(limit, 0.25f) * (limit + 1.0f);
  int e;
  (void)std::frexp(bound, &e);  // bound in [2^(e-1), 2^e)
  return e - 1 - 7;
}

size_t layer_hterm_bytes() { return (size_t)4 * kHRecBytes; }

bool decode_layer_supported(const LayerArgs &la) {
  const DecodeArgs &a = la.d;
  const int tiles = a.k * la.n_tps;
  return a.k >= 1 && a.k <= 4 && a.E >= 1 && a.E <= kLayerMaxE && a.k <= a.E && a.rnq >= 1 && a.rnq <= 6 &&
         (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
         a.gu.ns <= (uint32_t)kLayerNs && a.dn.ns <= (uint32_t)kLayerNs && a.H % 32 == 0 &&
         a.I % 32 == 0 && a.I <= kLayerMaxK && la.n_tps == (int)a.gu.tiles && la.n_tps <= kLayerMaxTps &&
         la.n_rt == (a.E + kLayerWaves - 1) / kLayerWaves && la.n_gu >= 1 && la.n_gu <= kLayerMaxGu &&
         5 * la.n_gu >= tiles && la.hexp == layer_hexp(a.limit) && la.hexp <= kLayerMaxHexp &&
         la.n_rt + la.n_gu + la.n_dn <= kLayerMaxBlocks;
}

hipError_t launch_decode_layer(const LayerArgs &la, hipStream_t s) {
  const DecodeArgs &a = la.d;
  if (!decode_layer_supported(la) || !la.sync || !la.hterm) return hipErrorInvalidValue;
  const dim3 grid(la.n_rt + la.n_gu + la.n_dn), block(kLayerThreads);
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
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(moe::moe_trace_ts), (size_t)n_blocks * 16 * 8, 0,
                                  hipMemcpyDeviceToHost);
}
#endif
