// Device helpers shared by the kernels of the MXFP4 MoE path (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ scalar helpers

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// x = hi + lo, both bf16; a non-finite hi carries the value alone.
__device__ __forceinline__ void split_bf16(float x, uint16_t &hi, uint16_t &lo) {
  hi = f32_to_bf16_rne(x);
  float h = bf16_to_f32(hi);
  lo = f32_to_bf16_rne(isfinite(h) ? x - h : 0.0f);
}

__device__ __forceinline__ float canon_nan(float v) {
  return isnan(v) ? __uint_as_float(0x7FC00000u) : v;
}

// Rust f32::clamp: a NaN stays NaN.
__device__ __forceinline__ float rclamp(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

// swiglu with the hardware exponential (v_exp_f32 on x log2(e), ~1 ulp) and reciprocal instead
// of the correctly rounded expf and division: for the grouped GEMM, whose h then enters as three
// fp6 terms (relative error ~1e-5), so the last bits of h do not reach the output.
__device__ __forceinline__ float swiglu_fast(float g, float u, float limit) {
  float gate = g != g ? g : fminf(g, limit);
  float up = rclamp(u, -limit, limit);
  float glu = gate * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gate * (-1.702f * 1.4426950408889634f)));
  return (up + 1.0f) * glu;
}

// E2M1 nibble -> f32 bits: sign | (e == 0 ? 0.5*m : 2^(e-1) * (1 + m/2)).
__device__ __forceinline__ float e2m1_to_f32(uint32_t n) {
  uint32_t mag = n & 7u;
  uint32_t bits = mag == 0 ? 0u : (mag == 1 ? 0x3F000000u : (((mag >> 1) + 126u) << 23) | ((mag & 1u) << 22));
  return __uint_as_float(bits | ((n & 8u) << 28));
}

// GPT-OSS SwiGLU of session.rs:109-117: gate = min(g, L), up = clamp(u, +-L),
// glu = gate / (1 + exp(-gate * 1.702)), h = (up + 1) * glu. Identical for every non-NaN g; a NaN
// g stays NaN here, where the reference's NaN-ignoring min gives L. A NaN gate only arises from
// non-finite weights or inputs, where these paths can hold NaN in place of the reference's
// infinity (an E8M0 255 block is NaN to the block-scaled MFMA); propagating it keeps every
// output that is non-finite in the fp32 path non-finite here.
__device__ __forceinline__ float swiglu(float g, float u, float limit) {
  float gate = g != g ? g : fminf(g, limit);
  float up = rclamp(u, -limit, limit);
  float glu = gate / (1.0f + expf(-gate * 1.702f));
  return (up + 1.0f) * glu;
}

// 8 nibbles (one dword of a block) -> 8 bf16, element order preserved (low nibble first).
__device__ __forceinline__ bf16x8 decode8(uint32_t w, float sc) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
  uint4 u;
  u.x = __builtin_bit_cast(uint32_t, p0);
  u.y = __builtin_bit_cast(uint32_t, p1);
  u.z = __builtin_bit_cast(uint32_t, p2);
  u.w = __builtin_bit_cast(uint32_t, p3);
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Ranking of session.rs:822-825 made total: greater logit first, equal logits (including
// +0 / -0) -> lower index first, NaN after every number.
__device__ __forceinline__ bool ranks_before(float a, int ia, float b, int ib) {
  bool an = isnan(a), bn = isnan(b);
  if (an || bn) return (an && bn) ? ia < ib : bn;
  if (a > b) return true;
  if (a < b) return false;
  return ia < ib;
}

// Value of lane (lane ^ O) for a compile-time O: DPP quad permutes for 1 and 2, ds_swizzle
// (bitmask mode) for 4..16, ds_bpermute for 32.
template <int O>
__device__ __forceinline__ float xor_lane(float v) {
  const int i = __float_as_int(v);
  if constexpr (O == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false));
  else if constexpr (O == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, i, 0x4E, 0xF, 0xF, false));
  else if constexpr (O < 32) return __int_as_float(__builtin_amdgcn_ds_swizzle(i, 0x1F | (O << 10)));
  else return __shfl_xor(v, 32);
}

// Xor butterfly p_l <- p_l + p_{l^o} for o = 32, 16, ..., 1; every lane ends with the same sum.
__device__ __forceinline__ float wave_sum_xor(float p) {
  p = p + xor_lane<32>(p);
  p = p + xor_lane<16>(p);
  p = p + xor_lane<8>(p);
  p = p + xor_lane<4>(p);
  p = p + xor_lane<2>(p);
  p = p + xor_lane<1>(p);
  return p;
}

// 1 / sqrt(sum(x^2) / H + eps) of a row, every lane of the wavefront taking part: lane l sums
// x[l + 64 i]^2 over i ascending (squares rounded, then added), the xor butterfly of
// wave_sum_xor combines the 64 partial sums (each step adds a commuted pair, so every lane holds
// the same bits), then the mean, sqrt and reciprocal, each correctly rounded (session.rs:483-487
// up to the order of the sum).
__device__ __forceinline__ float rms_inv_wave(const float *x, int H, float eps, int lane) {
  float p = 0.0f;
  for (int i = lane; i < H; i += 64) {
    const float sq = x[i] * x[i];
    p = p + sq;
  }
  const float mean = wave_sum_xor(p) / (float)H;
  return 1.0f / sqrtf(mean + eps);
}

__device__ __forceinline__ float wave_max(float m) {
  m = fmaxf(m, xor_lane<32>(m));
  m = fmaxf(m, xor_lane<16>(m));
  m = fmaxf(m, xor_lane<8>(m));
  m = fmaxf(m, xor_lane<4>(m));
  m = fmaxf(m, xor_lane<2>(m));
  m = fmaxf(m, xor_lane<1>(m));
  return m;
}

// Canonical order: lane l accumulates k = l, l+64, ... (k < H) with fused multiply-adds; the
// 64 partials are combined by a xor butterfly (32, 16, ..., 1); then the bias is added.
// Device layout of the router ("load-major"): lane l's chain k = l + 64 i, i = 0..KIp-1
// (KIp = ceil(H/64) rounded up to 8, zero padded) is read with KIp/8 16-byte loads; load q of
// expert e holds W[e][l + 64 (8q + h)], h = 0..7, at uint4 index (e * NQ + q) * 64 + l, so one
// load instruction of a wavefront reads 1 KB of consecutive bytes. x is staged with zeros past
// H; padded terms are fmaf(0, 0, p) = p exactly (p starts at +0 and can never become -0), so
// the chain equals the unpadded one. NQ = KIp/8 (0: runtime loop). w_e: expert e's weights.
template <int NQ>
__device__ __forceinline__ float router_dot(const uint16_t *w_e, const float *s_x, int nq,
                                            int lane) {
  float p = 0.0f;
  const uint4 *wq = reinterpret_cast<const uint4 *>(w_e) + lane;
  if (NQ > 0) {
    uint4 v[NQ > 0 ? NQ : 1];
#pragma unroll
    for (int q = 0; q < NQ; q++) v[q] = wq[q * 64];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
      const uint32_t u[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
      for (int h = 0; h < 8; h++) {
        const uint16_t b = (uint16_t)(u[h >> 1] >> (16 * (h & 1)));
        p = __builtin_fmaf(bf16_to_f32(b), s_x[lane + 64 * (8 * q + h)], p);
      }
    }
  } else {
    for (int q = 0; q < nq; q++) {
      const uint4 vq = wq[q * 64];
      const uint32_t u[4] = {vq.x, vq.y, vq.z, vq.w};
      for (int h = 0; h < 8; h++) {
        const uint16_t b = (uint16_t)(u[h >> 1] >> (16 * (h & 1)));
        p = __builtin_fmaf(bf16_to_f32(b), s_x[lane + 64 * (8 * q + h)], p);
      }
    }
  }
  return wave_sum_xor(p);
}

// Router logits of RB experts e0 + r*estride (r < RB) for the calling wavefront, RNQ 16-byte
// loads per lane chain, split in two so the loads can be issued early: router_load issues
// every weight load of the batch; router_compute runs the RB chains interleaved, each in the
// canonical order, and lane 0 writes s_logit[e] for e < E.
template <int RNQ, int RB>
struct RouterRegs {
  uint4 v[RB][RNQ];
};

template <int RNQ, int RB>
__device__ __forceinline__ void router_load(RouterRegs<RNQ, RB> &R, const uint16_t *rw, int E,
                                            int e0, int estride, int lane) {
#pragma unroll
  for (int r = 0; r < RB; r++) {
    const int e = min(e0 + r * estride, E - 1);
    const uint4 *wq = reinterpret_cast<const uint4 *>(rw + (size_t)e * RNQ * 512) + lane;
#pragma unroll
    for (int q = 0; q < RNQ; q++) R.v[r][q] = wq[q * 64];
  }
}

// xr[i] = x[lane + 64 i] (0 past H) for i < 8 * RNQ, in registers.
template <int RNQ, int RB>
__device__ __forceinline__ void router_compute(const RouterRegs<RNQ, RB> &R, const float *rb,
                                               const float *xr, int E, int e0, int estride,
                                               int lane, float *s_logit) {
  float p[RB];
#pragma unroll
  for (int r = 0; r < RB; r++) p[r] = 0.0f;
#pragma unroll
  for (int q = 0; q < RNQ; q++) {
#pragma unroll
    for (int h = 0; h < 8; h++) {
      const float xv = xr[8 * q + h];
#pragma unroll
      for (int r = 0; r < RB; r++) {
        const uint4 &w = R.v[r][q];
        const uint32_t u = h < 2 ? w.x : (h < 4 ? w.y : (h < 6 ? w.z : w.w));
        p[r] = __builtin_fmaf(bf16_to_f32((uint16_t)(u >> (16 * (h & 1)))), xv, p[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RB; r++) p[r] = wave_sum_xor(p[r]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RB; r++) {
      const int e = e0 + r * estride;
      if (e < E) s_logit[e] = canon_nan(p[r] + rb[e]);
    }
  }
}

// Epilogue of one 16-row tile x 8-entry chunk. acc holds rows 4*(lane/16)+i of column
// lane%16 (entry (lane%16)/2, term hi/lo); hi and lo columns are summed across lane pairs.
template <int MODE>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, const f32x4 &acc,
                                              const uint8_t *rec, int beg, int c0, int nent,
                                              int t, int lane) {
  const int g = lane >> 4, j = lane & 15;
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; i++) r[i] = acc[i] + xor_lane<1>(acc[i]);
  const int el = c0 + (j >> 1);
  if ((j & 1) || el >= nent) return;
  const int ge = beg + el;
  const int r0 = t * 16 + g * 4;
  if (MODE == GEMV_GATE_UP) {
    const float *bias = reinterpret_cast<const float *>(rec + a.bias_off);
    const int I = (int)a.d.rows / 2;
    const float h0 = swiglu(r[0] + bias[r0], r[1] + bias[r0 + 1], a.limit);
    const float h1 = swiglu(r[2] + bias[r0 + 2], r[3] + bias[r0 + 3], a.limit);
    uint16_t hi0, lo0, hi1, lo1;
    split_bf16(h0, hi0, lo0);
    split_bf16(h1, hi1, lo1);
    uint16_t *hs = reinterpret_cast<uint16_t *>(a.out) + (size_t)ge * 2 * I;
    const int ii = r0 / 2;
    *reinterpret_cast<uint32_t *>(hs + ii) = (uint32_t)hi0 | ((uint32_t)hi1 << 16);
    *reinterpret_cast<uint32_t *>(hs + I + ii) = (uint32_t)lo0 | ((uint32_t)lo1 << 16);
  } else if (MODE == GEMV_DOWN) {
    const float *bias = reinterpret_cast<const float *>(rec + a.bias_off);
    float *o = reinterpret_cast<float *>(a.out) + (size_t)ge * a.d.rows + r0;
    float4 v4;
    v4.x = canon_nan(rclamp(r[0] + bias[r0], -65504.0f, 65504.0f));
    v4.y = canon_nan(rclamp(r[1] + bias[r0 + 1], -65504.0f, 65504.0f));
    v4.z = canon_nan(rclamp(r[2] + bias[r0 + 2], -65504.0f, 65504.0f));
    v4.w = canon_nan(rclamp(r[3] + bias[r0 + 3], -65504.0f, 65504.0f));
    *reinterpret_cast<float4 *>(o) = v4;
  } else {
    float *o = reinterpret_cast<float *>(a.out) + (size_t)ge * a.d.rows + r0;
    *reinterpret_cast<float4 *>(o) =
        make_float4(canon_nan(r[0]), canon_nan(r[1]), canon_nan(r[2]), canon_nan(r[3]));
  }
}

// ------------------------------------------------------------------ top-k of one token

struct TopkCfg {
  int E, k;
  int adaptive, min_k;
  float top1_min, margin_min, top2_mass;
};

// Integer key with the order of ranks_before: NaN lowest, -0 equal to +0, otherwise the float
// order (sign-magnitude mapped to an unsigned order).
__device__ __forceinline__ uint32_t rank_key(float v) {
  if (isnan(v)) return 0u;
  if (v == 0.0f) v = 0.0f;
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Softmax over all experts (session.rs:511-520: max ignoring NaN, exp, sum, divide if the sum
// is positive; the sum is a tree here, so probabilities can differ from the sequential sum in
// the last bits), order by ranks_before (session.rs:822-825 totalised, through rank_key),
// optional adaptive count (session.rs:569-583), renormalisation over the kept slots
// (session.rs:826-839). Wavefront 0 does the work with logits in registers and other lanes'
// keys read with v_readlane; every thread of the block calls (two barriers). s_logit[E] is
// read. On return s_order[s] holds the expert of slot s (-1 past the kept count), s_w[s] its
// weight and *s_sel the kept count. s_pn: kMaxTopK floats of scratch.
// Q = ceil(E / 64) logits per lane (1 for E <= 64, the GPT-OSS-20B router).
template <int Q = kMaxExperts / 64>
__device__ __forceinline__ void block_topk(const TopkCfg &c, const float *s_logit, float *s_pn,
                                           int *s_order, float *s_w, int *s_sel) {
  const int E = c.E;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    float l[Q], p[Q];
    uint32_t key[Q];
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < Q; q++) {
      const int e = lane + 64 * q;
      l[q] = s_logit[min(e, E - 1)];
      key[q] = rank_key(l[q]);
      if (e < E) m = fmaxf(m, l[q]);
    }
    m = wave_max(m);
    float ls = 0.0f;
#pragma unroll
    for (int q = 0; q < Q; q++) {
      p[q] = lane + 64 * q < E ? expf(l[q] - m) : 0.0f;
      ls = ls + p[q];
    }
    const float sum = wave_sum_xor(ls);
    const bool norm = sum > 0.0f;
    int rank[Q] = {};
#pragma unroll
    for (int qf = 0; qf < Q; qf++) {
      const int nf = min(64, E - 64 * qf);
      for (int fl = 0; fl < nf; fl++) {
        const uint32_t kf = (uint32_t)__builtin_amdgcn_readlane((int)key[qf], fl);
        const int f = 64 * qf + fl;
#pragma unroll
        for (int q = 0; q < Q; q++)
          rank[q] += (kf > key[q] || (kf == key[q] && f < lane + 64 * q)) ? 1 : 0;
      }
    }
#pragma unroll
    for (int q = 0; q < Q; q++) {
      if (lane + 64 * q < E && rank[q] < c.k) {
        s_order[rank[q]] = lane + 64 * q;
        s_pn[rank[q]] = norm ? p[q] / sum : p[q];
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int kk = c.k < E ? c.k : E;
    int sel = kk;
    if (c.adaptive && kk > 1) {
      const float p1 = s_pn[0], p2 = s_pn[1];
      const float margin = fmaxf(p1 - p2, 0.0f);
      if (p1 >= c.top1_min && margin >= c.margin_min)
        sel = 1;
      else if (p1 + p2 >= c.top2_mass)
        sel = 2;
      const int mk = c.min_k < kk ? c.min_k : kk;
      if (sel < mk) sel = mk;
      if (sel > kk) sel = kk;
    }
    float top_sum = 0.0f;
    for (int s = 0; s < sel; s++) top_sum = top_sum + s_pn[s];
    const bool ok = isfinite(top_sum) && top_sum > 0.0f;
    for (int s = 0; s < c.k; s++) {
      if (s < sel) {
        s_w[s] = ok ? canon_nan(s_pn[s] / top_sum) : 1.0f / (float)sel;
      } else {
        s_order[s] = -1;
        s_w[s] = 0.0f;
      }
    }
    *s_sel = sel;
  }
  __syncthreads();
}

// Maximum over the wavefront: DPP within each row of 16 lanes (quad permutes, half-row and row
// mirrors: after the quad steps a quad is uniform, so the mirrors pair it with the other quad /
// half), then the four row results through v_readlane. Exact for any combining order.
__device__ __forceinline__ uint32_t row_max_dpp(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = row_max_dpp(v);
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(r0, r1), max(r2, r3));
}

__device__ __forceinline__ float wave_fmax_dpp(float m) {
  const int i = __float_as_int(m);
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false)));
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x140, 0xF, 0xF, false)));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// block_topk's result for k <= 4, computed by one wavefront with logit e = 64 q + lane in l[q]
// (entries past E ignored), in two parts so that a caller can act on the winners before the
// probabilities exist. wave_topk_order: the winners by k rounds of a wave arg-max over rank_key
// (ties: the lowest index, i.e. the lowest q with a candidate, then the lowest lane), which is
// ranks_before's order; ord[s] (uniform) for s < min(k, E), -1 after.
template <int Q>
__device__ __forceinline__ void wave_topk_order(const TopkCfg &c, const float (&l)[Q], int lane, int (&ord)[4]) {
  const int E = c.E;
  bool avail[Q];
  uint32_t key[Q];
#pragma unroll
  for (int q = 0; q < Q; q++) {
    avail[q] = 64 * q + lane < E;
    key[q] = rank_key(l[q]);
  }
  const int kk = c.k < E ? c.k : E;
#pragma unroll
  for (int s = 0; s < 4; s++) {  // the single-token kernels keep k <= 4
    ord[s] = -1;
    if (s < kk) {
      uint32_t best = 0;
#pragma unroll
      for (int q = 0; q < Q; q++)
        if (avail[q]) best = max(best, key[q]);
      best = wave_max_u32(best);
      int win = -1;
#pragma unroll
      for (int q = 0; q < Q; q++) {
        const uint64_t mask = __ballot(avail[q] && key[q] == best);
        if (win < 0 && mask) win = 64 * q + __builtin_ctzll(mask);
      }
#pragma unroll
      for (int q = 0; q < Q; q++)
        if (64 * q + lane == win) avail[q] = false;
      ord[s] = win;
    }
  }
}

// wave_topk_weights: the same softmax as block_topk (max, exp, the same xor-butterfly sum,
// divide), the probabilities of the winners ord, the adaptive count and the renormalisation.
// Writes s_w (lanes s < k), *s_sel (lane 0) and, if write_order, s_order.
template <int Q>
__device__ __forceinline__ void wave_topk_weights(const TopkCfg &c, const float (&l)[Q], int lane,
                                                  const int (&ord)[4], bool write_order, int *s_order,
                                                  float *s_w, int *s_sel) {
  const int E = c.E;
  float m = -INFINITY;
#pragma unroll
  for (int q = 0; q < Q; q++)
    if (64 * q + lane < E) m = fmaxf(m, l[q]);
  m = wave_fmax_dpp(m);
  float p[Q], ls = 0.0f;
#pragma unroll
  for (int q = 0; q < Q; q++) {
    p[q] = 64 * q + lane < E ? expf(l[q] - m) : 0.0f;
    ls = ls + p[q];
  }
  const float sum = wave_sum_xor(ls);
  float pn[Q];
#pragma unroll
  for (int q = 0; q < Q; q++) pn[q] = sum > 0.0f ? p[q] / sum : p[q];
  const int kk = c.k < E ? c.k : E;
  float ps[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    ps[s] = 0.0f;
    if (s < kk) {
#pragma unroll
      for (int q = 0; q < Q; q++)
        if ((ord[s] >> 6) == q) ps[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pn[q]), ord[s] & 63));
    }
  }
  int sel = kk;
  if (c.adaptive && kk > 1) {
    const float margin = fmaxf(ps[0] - ps[1], 0.0f);
    if (ps[0] >= c.top1_min && margin >= c.margin_min)
      sel = 1;
    else if (ps[0] + ps[1] >= c.top2_mass)
      sel = 2;
    const int mk = c.min_k < kk ? c.min_k : kk;
    if (sel < mk) sel = mk;
    if (sel > kk) sel = kk;
  }
  float top_sum = 0.0f;
#pragma unroll
  for (int s = 0; s < 4; s++)
    if (s < sel) top_sum = top_sum + ps[s];
  const bool ok = isfinite(top_sum) && top_sum > 0.0f;
#pragma unroll
  for (int s = 0; s < 4; s++) {
    if (lane == s && s < c.k) {
      if (write_order) s_order[s] = s < sel ? ord[s] : -1;
      s_w[s] = s < sel ? (ok ? canon_nan(ps[s] / top_sum) : 1.0f / (float)sel) : 0.0f;
    }
  }
  if (lane == 0) *s_sel = sel;
}

// ------------------------------------------------------------------ fp8 activation terms
//
// The block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4) takes the MXFP4 weights as they are
// (E2M1 nibbles with their E8M0 scales) and the activation as OCP fp8 e4m3 with one E8M0 scale
// per 32 values. An f32 activation block is sent as kTerms fp8 terms, x = sum_t q_t 2^(e_t),
// with e_0 chosen so the block's largest magnitude scales into [128, 256) and e_t = e_0 - 4t.
// Term t rounds the residual left by the terms before it to e4m3 (round to nearest even, 4
// significant bits), so each term divides a value's remaining error by at least 2^4 while it
// stays in e4m3's normal range, and the residual after the last term is below 2^-16 of the
// value (the bf16 hi+lo split keeps 2^-17). Every residual is exact in f32 (the rounded term is
// within a factor of two of the residual it rounds). Products of E2M1, e4m3 and power-of-two
// scales are exact in the MFMA, which accumulates in f32.
// Splits the 8 consecutive values x[0..7] of a lane; the 4 lanes of an aligned quad hold one
// 32-value block (lane % 4 = which 8). q[t] = the 8 term-t bytes (value i in byte i % 4 of
// word i / 4); s4 byte t = E8M0 scale of term t (uniform over the quad). A non-finite value in
// the block makes term 0 all fp8 NaN (0x7F), so every product with the block is NaN where the
// f32 path's result would be non-finite.
// The split once the block's largest magnitude m and its non-finite flag are known.
__device__ __forceinline__ void split8_fp8_with_max(const float x[8], float m, bool bad, uint2 q[kTerms],
                                                    uint32_t &s4) {
  if (bad) {
    q[0] = make_uint2(0x7F7F7F7Fu, 0x7F7F7F7Fu);
#pragma unroll
    for (int t = 1; t < kTerms; t++) q[t] = make_uint2(0u, 0u);
    s4 = 127u;
    return;
  }
  int e0 = -127;
  if (m > 0.0f) {
    int E;
    (void)frexpf(m, &E);  // m in [2^(E-1), 2^E)
    e0 = max(E - 8, -127);
  }
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; i++) r[i] = x[i];
  s4 = 0u;
#pragma unroll
  for (int t = 0; t < kTerms; t++) {
    const int e = max(e0 - 4 * t, -127);
    uint32_t w[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int p = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(r[4 * h], -e), ldexpf(r[4 * h + 1], -e), 0, false);
      p = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(r[4 * h + 2], -e), ldexpf(r[4 * h + 3], -e), p, true);
      w[h] = (uint32_t)p;
      r[4 * h + 0] = r[4 * h + 0] - ldexpf(__builtin_amdgcn_cvt_f32_fp8(p, 0), e);
      r[4 * h + 1] = r[4 * h + 1] - ldexpf(__builtin_amdgcn_cvt_f32_fp8(p, 1), e);
      r[4 * h + 2] = r[4 * h + 2] - ldexpf(__builtin_amdgcn_cvt_f32_fp8(p, 2), e);
      r[4 * h + 3] = r[4 * h + 3] - ldexpf(__builtin_amdgcn_cvt_f32_fp8(p, 3), e);
    }
    q[t] = make_uint2(w[0], w[1]);
    s4 |= (uint32_t)(e + 127) << (8 * t);
  }
}

// Two values of a range known in advance (|v| < 2^(e0 + 8)) as kTerms e4m3 terms with the fixed
// exponents e_t = e0 - 4t, no block maximum needed: the same term arithmetic as above, so each
// term divides a value's remaining error by at least 2^4 until the residual falls below the last
// term's resolution 2^(e0 - 4(kTerms-1) - 9). Bits 16t .. 16t+15 of the result: term t of v0
// (low byte) and of v1. A NaN value gives NaN bytes in every term.
__device__ __forceinline__ uint64_t split2_fp8_fixed(float v0, float v1, int e0) {
  uint64_t out = 0;
#pragma unroll
  for (int t = 0; t < kTerms; t++) {
    const int e = e0 - 4 * t;
    const int p = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(v0, -e), ldexpf(v1, -e), 0, false);
    v0 = v0 - ldexpf(__builtin_amdgcn_cvt_f32_fp8(p, 0), e);
    v1 = v1 - ldexpf(__builtin_amdgcn_cvt_f32_fp8(p, 1), e);
    out |= (uint64_t)(p & 0xFFFF) << (16 * t);
  }
  return out;
}

__device__ __forceinline__ void split8_fp8(const float x[8], uint2 q[kTerms], uint32_t &s4) {
  float m = 0.0f, bad = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    m = fmaxf(m, fabsf(x[i]));
    if (!isfinite(x[i])) bad = 1.0f;
  }
  m = fmaxf(m, xor_lane<1>(m));
  m = fmaxf(m, xor_lane<2>(m));
  bad = fmaxf(bad, xor_lane<1>(bad));
  bad = fmaxf(bad, xor_lane<2>(bad));
  split8_fp8_with_max(x, m, bad != 0.0f, q, s4);
}

// ------------------------------------------------------------------ one 16-row MXFP4 tile

// Registers of one tile: every 16-byte weight chunk and scale word a lane needs.
template <int NSMAX>
struct TileRegs {
  uint4 raw[NSMAX];
  uint32_t sw[(NSMAX + 3) / 4];
};

// Issues every weight and scale load of tile t of a resident matrix (layout.hpp). Lanes of
// missing blocks (the partial last step) and !ok tiles load nothing and hold zeros. The weights
// are read once per use, so they are loaded non-temporally (measured ~5% faster for the
// single-token layer than cached loads).
template <int NSMAX>
__device__ __forceinline__ void tile_load(TileRegs<NSMAX> &r, const uint8_t *mat, const PackDims &d,
                                          int t, bool ok, int lane) {
  const size_t tt = ok ? (size_t)t : 0;
  const uint4 *wp = reinterpret_cast<const uint4 *>(mat) + tt * 16 * d.nb;
  const uint32_t *sp = reinterpret_cast<const uint32_t *>(mat + pack_weight_bytes(d)) + tt * d.nq * 64;
  const int g = lane >> 4;
#pragma unroll
  for (int q = 0; q < (NSMAX + 3) / 4; q++) r.sw[q] = (ok && q < (int)d.nq) ? sp[q * 64 + lane] : 0u;
#pragma unroll
  for (int s = 0; s < NSMAX; s++) {
    r.raw[s] = make_uint4(0u, 0u, 0u, 0u);
    if (ok && s < (int)d.ns && 4 * s + g < (int)d.nb) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wp) + s * 64 + lane);
      r.raw[s] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
}

// MFMA sweep of a loaded tile against one B row pair in LDS (brow: the lane's hi or lo row of
// K bf16 as uint4, valid when bv). Returns the lane's 4 accumulators (rows 4*(lane/16)+i of
// column lane%16).
template <int NSMAX>
__device__ __forceinline__ f32x4 tile_mfma(const TileRegs<NSMAX> &r, const PackDims &d,
                                           const uint4 *brow, bool bv, int lane) {
  const int g = lane >> 4;
  // four independent accumulators (one per 8-element slice of a block) keep the dependent
  // MFMA chain a quarter as long; they are summed at the end
  f32x4 acc0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0, acc2 = acc0, acc3 = acc0;
#pragma unroll
  for (int s = 0; s < NSMAX; s++) {
    if (s < (int)d.ns) {
      const int b = 4 * s + g;
      const float sc = __uint_as_float(((r.sw[s / 4] >> (8 * (s % 4))) & 0xFFu) << 23);
      const bf16x8 A0 = decode8(r.raw[s].x, sc), A1 = decode8(r.raw[s].y, sc);
      const bf16x8 A2 = decode8(r.raw[s].z, sc), A3 = decode8(r.raw[s].w, sc);
      uint4 b0 = make_uint4(0u, 0u, 0u, 0u), b1 = b0, b2 = b0, b3 = b0;
      if (bv && b < (int)d.nb) {
        b0 = brow[4 * b];
        b1 = brow[4 * b + 1];
        b2 = brow[4 * b + 2];
        b3 = brow[4 * b + 3];
      }
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, as_bf16x8(b0), acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, as_bf16x8(b1), acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A2, as_bf16x8(b2), acc2, 0, 0, 0);
      acc3 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A3, as_bf16x8(b3), acc3, 0, 0, 0);
    }
  }
  return (acc0 + acc1) + (acc2 + acc3);
}

// One block-scaled MFMA, A = E2M1, B = e4m3, scales = byte `op` of the scale words (op is a
// constant after unrolling; the instruction needs it as an immediate).
template <int OP>
__device__ __forceinline__ f32x4 mfma_fp4_fp8_op(const i32x8 &A, const i32x8 &B, f32x4 c, uint32_t sa,
                                                 uint32_t sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, c, 4, 0, OP, (int)sa, OP, (int)sb);
}
__device__ __forceinline__ f32x4 mfma_fp4_fp8(int op, const i32x8 &A, const i32x8 &B, f32x4 c,
                                              uint32_t sa, uint32_t sb) {
  switch (op) {
    case 0: return mfma_fp4_fp8_op<0>(A, B, c, sa, sb);
    case 1: return mfma_fp4_fp8_op<1>(A, B, c, sa, sb);
    case 2: return mfma_fp4_fp8_op<2>(A, B, c, sa, sb);
    default: return mfma_fp4_fp8_op<3>(A, B, c, sa, sb);
  }
}

// Same with the B scale in byte 0 of its word (the lane has shifted its own byte there).
__device__ __forceinline__ f32x4 mfma_fp4_fp8_bs0(int op, const i32x8 &A, const i32x8 &B, f32x4 c,
                                                  uint32_t sa, uint32_t sb) {
  switch (op) {
    case 0: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, c, 4, 0, 0, (int)sa, 0, (int)sb);
    case 1: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, c, 4, 0, 1, (int)sa, 0, (int)sb);
    case 2: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, c, 4, 0, 2, (int)sa, 0, (int)sb);
    default: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, c, 4, 0, 3, (int)sa, 0, (int)sb);
  }
}

// Activation record in LDS or HBM for the block-scaled MFMA, for rows of up to 4 * NSMAX
// 32-value blocks (blocks past the row are zero): term t, block b, value i at byte
// t * kTermStride + 32 b + i; the E8M0 scale of (t, b) at byte
// kTerms * kTermStride + (4 t + b % 4) * NSMAX + b / 4, so a lane of group g finds the scales of
// its blocks 4s + g, s = 0..NSMAX-1, in consecutive bytes. The term stride is 64 bytes past a
// multiple of 256, so the 4 terms read by one MFMA step fall in different LDS banks.
template <int NSMAX>
struct ActRecord {
  static constexpr int kTermStride = 4 * NSMAX * 32 + 64;
  static constexpr int kScaleOff = kTerms * kTermStride;
  static constexpr int kBytes = kScaleOff + kTerms * 4 * NSMAX;
  __host__ __device__ static constexpr int term(int t, int b) { return t * kTermStride + 32 * b; }
  __host__ __device__ static constexpr int scale(int t, int b) { return kScaleOff + (4 * t + (b & 3)) * NSMAX + (b >> 2); }
};

// MFMA sweep of a loaded tile against an activation record (split8_fp8 terms) on
// v_mfma_scale_f32_16x16x128_f8f6f4: A = the tile's raw E2M1 chunks with their E8M0 scale words
// (lane group g holds block 4s+g, its scale in byte s%4 of word s/4; steps past the tile's are
// zero), B column j = term j % kTerms. B lane layout (measured on gfx950): lane (column j,
// group gb) supplies bytes 0..15 = values 16(gb&1)..16(gb&1)+15 of block 4s+(gb>>1), bytes
// 16..31 = the same values of block 4s+2+(gb>>1), and the scale of block 4s+gb. Lanes of
// columns >= kTerms read the same bytes as column j % kTerms (a broadcast) with scale byte 0;
// their columns are never read. bsw: the lane's B scale words (byte i of word q = scale of
// block 4(4q+i)+gb of its term; 0 for columns >= kTerms). Runs all NSMAX steps without
// branches. Returns rows 4*(lane/16)+i of column lane%16.
template <int NSMAX>
__device__ __forceinline__ f32x4 tile_mfma_f8(const TileRegs<NSMAX> &r, const uint8_t *rec,
                                              const uint32_t *bsw, int lane) {
  using R = ActRecord<NSMAX>;
  const int j = lane & 15, gb = lane >> 4;
  const uint8_t *bt = rec + R::term(j & (kTerms - 1), gb >> 1) + 16 * (gb & 1);
  f32x4 acc0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
  // B of step s is read two steps ahead so the LDS latency hides behind the MFMAs
  constexpr int PD = 2;
  uint4 pb0[PD], pb1[PD];
#pragma unroll
  for (int s = 0; s < PD; s++) {
    pb0[s] = *reinterpret_cast<const uint4 *>(bt + s * 128);
    pb1[s] = *reinterpret_cast<const uint4 *>(bt + s * 128 + 64);
  }
#pragma unroll
  for (int s = 0; s < NSMAX; s++) {
    const uint4 b0 = pb0[s % PD], b1 = pb1[s % PD];
    if (s + PD < NSMAX) {
      pb0[s % PD] = *reinterpret_cast<const uint4 *>(bt + (s + PD) * 128);
      pb1[s % PD] = *reinterpret_cast<const uint4 *>(bt + (s + PD) * 128 + 64);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the reads PD steps ahead of their MFMA
    const uint4 a = r.raw[s];
    const i32x8 A = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    const i32x8 B = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                     (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    if (s & 1)
      acc1 = mfma_fp4_fp8(s & 3, A, B, acc1, r.sw[s / 4], bsw[s / 4]);
    else
      acc0 = mfma_fp4_fp8(s & 3, A, B, acc0, r.sw[s / 4], bsw[s / 4]);
  }
  return acc0 + acc1;
}

// The lane's B scale words for tile_mfma_f8 from an activation record.
template <int NSMAX>
__device__ __forceinline__ void load_bsw(const uint8_t *rec, uint32_t *bsw, int lane) {
  using R = ActRecord<NSMAX>;
  const int j = lane & 15, gb = lane >> 4;
#pragma unroll
  for (int q = 0; q < NSMAX / 4; q++)
    bsw[q] = j < kTerms ? *reinterpret_cast<const uint32_t *>(rec + R::scale(j, gb) + 4 * q) : 0u;
}

// Cross-block communication without fences: agent-scope (device-coherent) relaxed loads and
// stores, which bypass the non-coherent cache levels, and a wait for the wavefront's own memory
// operations; a writer stores, waits, then signals; a reader sees the signal, then loads.
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
// Wavefront 0 of a block: from the per-expert entry counts cnt[0..E), the active experts in
// ascending id (active_ids, active_off, *n_active; the entries of active expert i are
// [active_off[i], active_off[i + 1])) and every expert's first entry base[e], by wave prefix
// sums over 64 experts at a time.
__device__ __forceinline__ void expert_list_wave(const int *cnt, int E, int lane, int *base, int32_t *active_ids,
                                                 int32_t *active_off, int32_t *n_active) {
  int off = 0, na = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const int c = e < E ? cnt[e] : 0;
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o);
      if (lane >= o) incl += u;
    }
    const uint64_t act = __ballot(c > 0);
    const int slot = na + __popcll(act & ((1ull << lane) - 1ull));
    if (e < E) base[e] = off + incl - c;
    if (c > 0) {
      active_ids[slot] = e;
      active_off[slot] = off + incl - c;
    }
    off += __shfl(incl, 63);
    na += __popcll(act);
  }
  if (lane == 0) {
    active_off[na] = off;
    *n_active = na;
  }
}

// s_waitcnt immediate that waits until at most n vector-memory operations of the wavefront are
// outstanding (vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left at their maxima). n must fit
// the 6-bit vmcnt field: a count outside [0, 63] reaches the non-constexpr function below, and
// since __builtin_amdgcn_s_waitcnt takes only a constant expression, such a wait does not compile.
__host__ __device__ inline int vmcnt_outside_6_bits() { return 0; }
constexpr int vm_wait(int n) {
  return n >= 0 && n <= 63 ? (0x0F70 | (n & 0xF) | ((n >> 4) << 14)) : vmcnt_outside_6_bits();
}
// The same with lgkmcnt 0: also this wavefront's LDS operations complete.
constexpr int vm_lgkm_wait(int n) { return vm_wait(n) & ~0x0F00; }

// s_waitcnt vmcnt(n) for n in [0, 15] held in a variable that loop unrolling makes a constant (the
// switch then folds to one instruction; the builtin itself takes only a constant expression).
__device__ __forceinline__ void wait_vmcnt_upto15(int n) {
#define MOE_VM_CASE(k) \
  case k: __builtin_amdgcn_s_waitcnt(vm_wait(k)); break;
  switch (n) {
    MOE_VM_CASE(0) MOE_VM_CASE(1) MOE_VM_CASE(2) MOE_VM_CASE(3) MOE_VM_CASE(4) MOE_VM_CASE(5)
    MOE_VM_CASE(6) MOE_VM_CASE(7) MOE_VM_CASE(8) MOE_VM_CASE(9) MOE_VM_CASE(10) MOE_VM_CASE(11)
    MOE_VM_CASE(12) MOE_VM_CASE(13) MOE_VM_CASE(14)
    default: __builtin_amdgcn_s_waitcnt(vm_wait(15)); break;
  }
#undef MOE_VM_CASE
}

// Wait until every memory operation this wavefront issued has completed.
__device__ __forceinline__ void wait_mem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ------------------------------------------------------------------ fp6 activation terms

// E2M3 (fp6: sign, 2 exponent bits with bias 1, 3 mantissa bits; no Inf/NaN, largest 7.5)
// conversion in hardware: v_cvt_scalef32_2xpk16_fp6_f32 divides 2 x 16 f32 by a power-of-two
// scale and rounds each to the nearest E2M3 code, ties to even, saturating at +-7.5; output
// field 2i is a[i], field 2i+1 is b[i] (value u of a 32-value group at bits 6u); the pk32 back
// conversion returns the codes' values times the scale in field order. Measured on gfx950 against
// a software RNE on every E2M3 grid point, every midpoint, values past 7.5, +-inf and random
// values: identical codes except -0 for -0.0. The destination must not share registers with the
// sources (register allocations that reuse the unused upper source registers for the result gave
// wrong codes, deterministically), so both are issued as inline assembly with early-clobber
// outputs.
typedef float f32x16v __attribute__((ext_vector_type(16)));
typedef float f32x32v __attribute__((ext_vector_type(32)));
typedef uint32_t u32x6v __attribute__((ext_vector_type(6)));

// Scale exponent of term t of an NT-term split of a block whose maximum is m = f 2^E, f in
// [1/2, 1). Several terms: 2^(E - 2 - 5t) (term 0 holds the block in [-4, 4), so its residual
// never saturates; each later term removes 5 more bits). One term (the quantized mode): the OCP
// MX rule, 2^(floor(log2 m) - 2) = 2^(E - 3), the block maximum in [4, 8) (values past 7.5
// saturate). Stops at 2^-126 (a normal f32) for blocks below about 2^-120.
template <int NT>
__device__ __forceinline__ int split_scale_exp(int E, int t) {
  return max(NT == 1 ? E - 3 : E - 2 - 5 * t, -126);
}

// Split of 16 values of a 32-value block (block max |x| = m, bad = some value of the block is
// not finite) into NT E2M3 terms at split_scale_exp's scales, each taking the exact residual of
// the terms before it (3 terms: the activation is exact to about 2^-13 of the block maximum).
// Codes of value u at bits 6u of d[t][0..2]; sb byte t = the E8M0 scale of term t (0xFF, NaN, for
// a bad block: the products come out NaN, as the f32 arithmetic would).
template <int NT>
__device__ __forceinline__ void split16_fp6(const float (&x)[16], float m, bool bad, uint32_t (&d)[NT][3],
                                            uint32_t &sb) {
  int E = 0;
  if (m > 0.0f && isfinite(m)) frexpf(m, &E);
  float r[16];
#pragma unroll
  for (int i = 0; i < 16; i++) r[i] = bad ? 0.0f : x[i];
  sb = 0;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int se = split_scale_exp<NT>(E, t);
    sb |= (bad ? 0xFFu : (uint32_t)(se + 127)) << (8 * t);
    const float sc = __builtin_amdgcn_ldexpf(1.0f, se);
    f32x16v a = {}, b = {};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      a[i] = r[2 * i];
      b[i] = r[2 * i + 1];
    }
    u32x6v c;
    f32x32v q;
    asm volatile("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, %3" : "=&v"(c) : "v"(a), "v"(b), "v"(sc));
    if (t + 1 < NT) {  // the residual feeds the next term
      asm volatile("v_cvt_scalef32_pk32_f32_fp6 %0, %1, %2" : "=&v"(q) : "v"(c), "v"(sc));
#pragma unroll
      for (int i = 0; i < 16; i++) r[i] = r[i] - q[i];
    }
    d[t][0] = c[0];
    d[t][1] = c[1];
    d[t][2] = c[2];
  }
}


// split16_fp6 for a whole 32-value block in one lane (x[u] = value u, m = its maximum |x|): the
// conversions take all 32 values at once, and term t's codes are the 6 dwords of the block's
// B operand (value u at bits 6u). Same codes and scales as two split16_fp6 halves.
template <int NT>
__device__ __forceinline__ void split32_fp6(const float (&x)[32], float m, bool bad, uint32_t (&d)[NT][6],
                                            uint32_t &sb) {
  int E = 0;
  if (m > 0.0f && isfinite(m)) frexpf(m, &E);
  float r[32];
#pragma unroll
  for (int i = 0; i < 32; i++) r[i] = bad ? 0.0f : x[i];
  sb = 0;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int se = split_scale_exp<NT>(E, t);
    sb |= (bad ? 0xFFu : (uint32_t)(se + 127)) << (8 * t);
    const float sc = __builtin_amdgcn_ldexpf(1.0f, se);
    f32x16v a, b;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      a[i] = r[2 * i];
      b[i] = r[2 * i + 1];
    }
    u32x6v c;
    asm volatile("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, %3" : "=&v"(c) : "v"(a), "v"(b), "v"(sc));
#pragma unroll
    for (int k = 0; k < 6; k++) d[t][k] = c[k];
    if (t + 1 < NT) {  // the residual feeds the next term (the last term needs none)
      f32x32v q;
      asm volatile("v_cvt_scalef32_pk32_f32_fp6 %0, %1, %2" : "=&v"(q) : "v"(c), "v"(sc));
#pragma unroll
      for (int i = 0; i < 32; i++) r[i] = r[i] - q[i];
    }
  }
}

// Block blk (values 32 blk .. 32 blk + 31, in v; 0 <= blk < 4 kGemmNs) of a row into the row's
// GemmRecT<NT> record r: one lane per block (split32_fp6): the NT terms' codes and scale bytes.
template <int NT>
__device__ __forceinline__ void rec_split_block(const float (&v)[32], int blk, uint8_t *r) {
  using R = GemmRecT<NT>;
  float m = 0.0f;
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    m = fmaxf(m, fabsf(v[i]));
    bad = bad || !isfinite(v[i]);
  }
  uint32_t d[NT][6], sb;
  split32_fp6<NT>(v, m, bad, d, sb);
  const int st = blk >> 2, i = blk & 3;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    *reinterpret_cast<uint4 *>(r + R::dword(st, t, i, 0)) = make_uint4(d[t][0], d[t][1], d[t][2], d[t][3]);
    *reinterpret_cast<uint2 *>(r + R::dword(st, t, i, 4)) = make_uint2(d[t][4], d[t][5]);
    r[R::scale(st, t) + i] = (uint8_t)(sb >> (8 * t));
  }
}

// tile_mfma_f8 over steps [s0, s0 + NS) of a tile whose chunks for those steps are in raw[] (zeros
// past the tile) and whose scale words are all in sw[]; rec, bsw as for tile_mfma_f8. One
// accumulator: a quarter of a tile's steps is a short chain.
template <int NSMAX, int NS, int s0>
__device__ __forceinline__ f32x4 tile_mfma_f8_steps(const uint4 (&raw)[NS], const uint32_t *sw,
                                                    const uint8_t *rec, const uint32_t *bsw, int lane) {
  using R = ActRecord<NSMAX>;
  const int j = lane & 15, gb = lane >> 4;
  const uint8_t *bt = rec + R::term(j & (kTerms - 1), gb >> 1) + 16 * (gb & 1);
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < NS; k++) {
    const int s = s0 + k;
    if (s < NSMAX) {
      const uint4 b0 = *reinterpret_cast<const uint4 *>(bt + s * 128);
      const uint4 b1 = *reinterpret_cast<const uint4 *>(bt + s * 128 + 64);
      const uint4 a = raw[k];
      const i32x8 A = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
      const i32x8 B = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                       (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
      acc = mfma_fp4_fp8(s & 3, A, B, acc, sw[s / 4], bsw[s / 4]);
    }
  }
  return acc;
}

// Sum of the kTerms term columns of an MFMA result: lanes with lane % 16 == 0 get
// (t0 + t1) + (t2 + t3) for each of their 4 rows.
__device__ __forceinline__ void sum_terms(const f32x4 &acc, float v[4]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float u = acc[i] + xor_lane<1>(acc[i]);
    v[i] = u + xor_lane<2>(u);
  }
}

}  // namespace moe
