// Single-token MoE layer for gfx950 in two launches — the MoE block of
// Session::decode_step_inner (session.rs:818-980) for one token:
//
//   k_decode_gate_up  every block computes the router logits itself (canonical order, the
//                     same arithmetic as k_route, so every block selects the same experts),
//                     runs the top-k, then streams 4 consecutive 16-row gate_up tiles of one
//                     slot's expert and writes SwiGLU(h) as bf16 hi/lo. Block 0 publishes
//                     logits, indices and weights.
//   k_decode_down     one 16-row tile of the output for every slot (wavefront = slot): bias,
//                     clamp to +-65504 and the slot-ordered combine in LDS, then y.
//
// The kernel boundary is the only synchronisation: no counters, no atomics, no spin waits.
// Recomputing the router per block costs reads of the 184 KB router from L2 (resident after
// the first block of each XCD touches it) and 92k FMAs per block. Exchanging logits and h
// between blocks inside one launch needs same-address device atomics and polling instead,
// which serialise at ~12 ns per operation on this part and cost far more at ~540 blocks.
#include <algorithm>

#include "device.hpp"
#include "kernels.hpp"

namespace moe {

constexpr int kDecodeNs = 24;  // tiles of up to 96 blocks per row (K <= 3072)

template <int RNQ>
__global__ __launch_bounds__(256, 2) void k_decode_gate_up(DecodeArgs a) {
  extern __shared__ uint4 smem[];
  __shared__ float s_logit[kMaxExperts];
  __shared__ float s_pn[kMaxTopK];
  __shared__ int s_order[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  __shared__ int s_sel;

  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int H = a.H, I = a.I, E = a.E;
  uint16_t *s_xb = reinterpret_cast<uint16_t *>(smem);  // x bf16: hi row, lo row

  // 1. x[lane + 64 i] straight into registers (clamped indices: every load valid, none waits
  //    on another), then the first batch of router weights
  constexpr int RQ = RNQ > 0 ? RNQ : 1;
  constexpr int XI = 8 * RQ;  // chain terms per lane (48 for 2880)
  constexpr int RB = 4;
  float xr[XI];
  if (RNQ > 0) {
#pragma unroll
    for (int i = 0; i < XI; i++) xr[i] = a.x[min(lane + 64 * i, H - 1)];
  }
  RouterRegs<RQ, RB> R;
  if (RNQ > 0) router_load<RQ, RB>(R, a.rw, E, wv, 4, lane);
  if (RNQ > 0) {
#pragma unroll
    for (int i = 0; i < XI; i++) {
      const int k = lane + 64 * i;
      if (k >= H) xr[i] = 0.0f;  // zero padding of the canonical chain
    }
    // 2. router: wavefront wv handles experts wv, wv+4, ...; RB per batch with hoisted loads
    router_compute<RQ, RB>(R, a.rb, xr, E, wv, 4, lane, s_logit);
    for (int e0 = wv + 4 * RB; e0 < E; e0 += 4 * RB) {
      router_load<RQ, RB>(R, a.rw, E, e0, 4, lane);
      router_compute<RQ, RB>(R, a.rb, xr, E, e0, 4, lane, s_logit);
    }
    // 3. x as bf16 hi/lo rows for the MFMA (each wavefront writes a quarter of the row)
#pragma unroll
    for (int i = 0; i < XI; i++) {
      const int k = lane + 64 * i;
      if ((i & 3) == wv && k < H) {
        uint16_t hi, lo;
        split_bf16(xr[i], hi, lo);
        s_xb[k] = hi;
        s_xb[H + k] = lo;
      }
    }
  } else {
    float *s_xr = reinterpret_cast<float *>(smem + (size_t)2 * H * 2 / 16);  // a.Hr floats
    for (int k = tid; k < a.Hr; k += 256) {
      const float v = k < H ? a.x[k] : 0.0f;
      s_xr[k] = v;
      if (k < H) {
        uint16_t hi, lo;
        split_bf16(v, hi, lo);
        s_xb[k] = hi;
        s_xb[H + k] = lo;
      }
    }
    __syncthreads();
    for (int e = wv; e < E; e += 4) {
      const float p = router_dot<0>(a.rw + (size_t)e * a.rnq * 512, s_xr, a.rnq, lane);
      if (lane == 0) s_logit[e] = canon_nan(p + a.rb[e]);
    }
  }
  __syncthreads();
  const TopkCfg c{E, a.k, a.adaptive, a.min_k, a.top1_min, a.margin_min, a.top2_mass};
  block_topk(c, s_logit, s_pn, s_order, s_w, &s_sel);
  if (b == 0) {
    for (int e = tid; e < E; e += 256) a.logits[e] = s_logit[e];
    if (tid < a.k) {
      a.idx[tid] = s_order[tid];
      a.wts[tid] = s_w[tid];
    }
  }
  const int slot = b / a.n_gu_wg_per_slot;
  const int t = (b - slot * a.n_gu_wg_per_slot) * 4 + wv;
  if (!(slot < s_sel && t < (int)a.gu.tiles)) return;  // no barrier follows
  const uint8_t *rec = a.base + (size_t)s_order[slot] * a.stride;
  TileRegs<kDecodeNs> r;
  tile_load<kDecodeNs>(r, rec + a.gu_off, a.gu, t, true, lane);
  const int j = lane & 15, g = lane >> 4;
  const f32x4 acc = tile_mfma<kDecodeNs>(
      r, a.gu, reinterpret_cast<const uint4 *>(s_xb) + (size_t)(j & 1) * (H / 8), j < 2, lane);
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; i++) v[i] = acc[i] + xor_lane<1>(acc[i]);
  if (j == 0) {
    const float *bias = reinterpret_cast<const float *>(rec + a.gub_off);
    const int r0 = t * 16 + g * 4;
    const float h0 = swiglu(v[0] + bias[r0], v[1] + bias[r0 + 1], a.limit);
    const float h1 = swiglu(v[2] + bias[r0 + 2], v[3] + bias[r0 + 3], a.limit);
    uint16_t hi0, lo0, hi1, lo1;
    split_bf16(h0, hi0, lo0);
    split_bf16(h1, hi1, lo1);
    uint16_t *hs = a.hsplit + (size_t)slot * 2 * I;
    const int ii = r0 / 2;
    *reinterpret_cast<uint32_t *>(hs + ii) = (uint32_t)hi0 | ((uint32_t)hi1 << 16);
    *reinterpret_cast<uint32_t *>(hs + I + ii) = (uint32_t)lo0 | ((uint32_t)lo1 << 16);
  }
}

__global__ __launch_bounds__(256) void k_decode_down(DecodeArgs a) {
  extern __shared__ uint4 smem[];  // [4 slots][hi row, lo row][I bf16]
  __shared__ float s_o[4][16];
  __shared__ float s_ws[4];
  __shared__ int s_ok[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, slot = tid >> 6;
  const int I = a.I;
  // 1. this slot's h rows (independent of the routing: issued first, clamped to valid slots)
  constexpr int HQ = 12;  // uint4 per lane: 2*I/8 <= 768 (I <= 3072)
  const int nh = 2 * I / 8;
  const uint4 *src = reinterpret_cast<const uint4 *>(a.hsplit + (size_t)min(slot, a.k - 1) * 2 * I);
  uint4 hv[HQ];
#pragma unroll
  for (int i = 0; i < HQ; i++) hv[i] = src[min(lane + 64 * i, nh - 1)];
  // 2. routing of this slot, then every weight load of the tile
  const int e = slot < a.k ? a.idx[slot] : -1;  // -1: beyond k or the adaptive count
  const bool ok = e >= 0;
  const uint8_t *rec = a.base + (size_t)(ok ? e : 0) * a.stride;
  TileRegs<kDecodeNs> r;
  tile_load<kDecodeNs>(r, rec + a.dn_off, a.dn, t, ok, lane);
  uint4 *s_h = smem + (size_t)slot * nh;
#pragma unroll
  for (int i = 0; i < HQ; i++)
    if (lane + 64 * i < nh) s_h[lane + 64 * i] = hv[i];
  if (lane == 0) {
    s_ws[slot] = ok ? a.wts[slot] : 0.0f;
    s_ok[slot] = ok;
  }
  __syncthreads();
  const int j = lane & 15, g = lane >> 4;
  if (ok) {
    const f32x4 acc = tile_mfma<kDecodeNs>(r, a.dn, s_h + (size_t)(j & 1) * (I / 8), j < 2, lane);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = acc[i] + xor_lane<1>(acc[i]);
    if (j == 0) {
      const float *bias = reinterpret_cast<const float *>(rec + a.dnb_off);
      const int r0 = t * 16 + g * 4;
#pragma unroll
      for (int i = 0; i < 4; i++)
        s_o[slot][g * 4 + i] = canon_nan(rclamp(v[i] + bias[r0 + i], -65504.0f, 65504.0f));
    }
  }
  __syncthreads();
  if (tid < 16) {  // session.rs:974-980: y = 0; y += w_s * out_s in slot order
    float y = 0.0f;
    for (int s = 0; s < 4 && s < a.k; s++)
      if (s_ok[s]) y = y + s_ws[s] * s_o[s][tid];
    a.y[t * 16 + tid] = canon_nan(y);
  }
}

size_t decode_lds_gate_up(const DecodeArgs &a) { return (size_t)2 * a.H * 2 + (size_t)a.Hr * 4; }
size_t decode_lds_down(const DecodeArgs &a) { return (size_t)4 * 2 * a.I * 2; }

bool decode_supported(const DecodeArgs &a) {
  return a.k >= 1 && a.k <= 4 && a.E >= 1 && a.E <= kMaxExperts && a.k <= a.E &&
         a.gu.ns <= (uint32_t)kDecodeNs && a.dn.ns <= (uint32_t)kDecodeNs && a.H % 32 == 0 &&
         a.I % 32 == 0 && a.Hr <= 4096 && a.I <= 3072 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
         decode_lds_gate_up(a) <= 64 * 1024 && decode_lds_down(a) <= 64 * 1024;
}

hipError_t launch_decode_gate_up(const DecodeArgs &a, hipStream_t s) {
  if (!decode_supported(a)) return hipErrorInvalidValue;
  const dim3 grid(a.k * a.n_gu_wg_per_slot), block(256);
  const size_t lds = decode_lds_gate_up(a);
  if (a.rnq == 6)
    hipLaunchKernelGGL(k_decode_gate_up<6>, grid, block, lds, s, a);
  else
    hipLaunchKernelGGL(k_decode_gate_up<0>, grid, block, lds, s, a);
  return hipGetLastError();
}

hipError_t launch_decode_down(const DecodeArgs &a, hipStream_t s) {
  if (!decode_supported(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_decode_down, dim3(a.dn.tiles), dim3(256), decode_lds_down(a), s, a);
  return hipGetLastError();
}

}  // namespace moe
