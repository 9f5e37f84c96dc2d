/*
 * CPU ORACLE — test infrastructure only (see moe_oracle.h). Restates the reference's
 * MXFP4 MoE path in plain C. Never linked into, loaded by or called from the HIP library.
 *
 * Reference files restated (gabearro/SilentOTITHRanDouSha):
 *   src/gpt_oss/weights.rs:350-371, 373-460, 593-702   (MXFP4 decode, de-interleave, fp16 decode)
 *   src/gpt_oss/session.rs:16-124, 495-520, 569-583, 818-980  (matvec, expert FFN, router, top-k, combine)
 * Third-party arithmetic at the boundary: half 2.7.1 (bf16/f16 conversions) — restated as IEEE.
 */
#include "moe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__AVX2__) && defined(__F16C__) && defined(__FMA__)
#include <immintrin.h>
#define ORC_HAVE_AVX2 1
#endif

#define ORC_CANON_NAN 0x7FC00000u

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline float canon(float f) { return isnan(f) ? u2f(ORC_CANON_NAN) : f; }

/* ------------------------------------------------------------------ conversions */

float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t orc_f32_to_bf16_rne(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in f32 */
    float v = (float)man * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16_rne(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFF) return (uint16_t)(man ? (sign | 0x7E00u | (man >> 13)) : (sign | 0x7C00u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000u;
    int shift = 14 - e;
    uint32_t q = m >> shift;
    uint32_t half = 1u << (shift - 1);
    uint32_t rem = m & ((half << 1) - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = man >> 13;
  uint32_t rem = man & 0x1FFFu;
  uint32_t out = sign | ((uint32_t)e << 10) | q;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) out++;
  return (uint16_t)out;
}

/* ------------------------------------------------------------------ MXFP4 -> f32 */

/* E2M1 values of the 16 nibbles; weights.rs:352-354 (equal to the OCP MX v1.0 table). */
static const float FP4_LUT[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                  -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

void orc_dequant_mxfp4_row(const uint8_t *blocks, const uint8_t *scales, size_t nb, float *out) {
  for (size_t bi = 0; bi < nb; bi++) {
    /* E8M0 decoded as the f32 whose exponent field is the byte (weights.rs:359):
     * 0 -> +0.0, 255 -> +inf. */
    float scale = u2f((uint32_t)scales[bi] << 23);
    const uint8_t *blk = blocks + bi * 16;
    for (size_t j = 0; j < 16; j++) {
      uint8_t byte = blk[j];
      out[bi * 32 + 2 * j] = canon(FP4_LUT[byte & 0x0F] * scale);
      out[bi * 32 + 2 * j + 1] = canon(FP4_LUT[byte >> 4] * scale);
    }
  }
}

void orc_dequant_mxfp4_matrix(const uint8_t *blocks, const uint8_t *scales, size_t rows,
                              size_t cols, float *out) {
  size_t nb = cols / 32;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; r++)
    orc_dequant_mxfp4_row(blocks + (size_t)r * nb * 16, scales + (size_t)r * nb, nb,
                          out + (size_t)r * cols);
}

void orc_dequant_gate_up_reordered(const uint8_t *blocks, const uint8_t *scales, size_t inter,
                                   size_t cols, float *out) {
  size_t nb = cols / 32;
  for (size_t i = 0; i < inter; i++) {
    size_t src = 2 * i;
    orc_dequant_mxfp4_row(blocks + src * nb * 16, scales + src * nb, nb, out + i * cols);
    src = 2 * i + 1;
    orc_dequant_mxfp4_row(blocks + src * nb * 16, scales + src * nb, nb,
                          out + (inter + i) * cols);
  }
}

/* ------------------------------------------------------------------ MXFP4 -> fp16 */

/* weights.rs:465-485: the LUT as fp16 bits (exact). */
static const uint16_t FP4_LUT_F16[16] = {0x0000, 0x3800, 0x3C00, 0x3E00, 0x4000, 0x4200,
                                         0x4400, 0x4600, 0x8000, 0xB800, 0xBC00, 0xBE00,
                                         0xC000, 0xC200, 0xC400, 0xC600};

uint16_t orc_f16_mul_scalar(uint16_t val_bits, uint16_t scale_bits) {
  if (val_bits == 0 || val_bits == 0x8000) return val_bits;
  if (scale_bits == 0) return (uint16_t)(val_bits & 0x8000);
  uint16_t sign = val_bits & 0x8000;
  int val_exp = (val_bits >> 10) & 0x1F;
  uint16_t val_mant = val_bits & 0x03FF;
  int scale_exp = (scale_bits >> 10) & 0x1F;
  int new_exp = val_exp + scale_exp - 15;
  if (new_exp <= 0) return sign;
  if (new_exp >= 31) return (uint16_t)(sign | 0x7C00);
  return (uint16_t)(sign | ((uint16_t)new_exp << 10) | val_mant);
}

void orc_dequant_mxfp4_row_f16(const uint8_t *blocks, const uint8_t *scales, size_t nb,
                               uint16_t *out) {
  for (size_t bi = 0; bi < nb; bi++) {
    int scale_exp = (int)scales[bi] - 112;
    uint16_t scale_f16 =
        scale_exp <= 0 ? 0 : (scale_exp >= 31 ? 0x7C00 : (uint16_t)(scale_exp << 10));
    const uint8_t *blk = blocks + bi * 16;
    for (size_t j = 0; j < 16; j++) {
      uint8_t byte = blk[j];
      out[bi * 32 + 2 * j] = orc_f16_mul_scalar(FP4_LUT_F16[byte & 0x0F], scale_f16);
      out[bi * 32 + 2 * j + 1] = orc_f16_mul_scalar(FP4_LUT_F16[byte >> 4], scale_f16);
    }
  }
}

void orc_dequant_gate_up_reordered_f16(const uint8_t *blocks, const uint8_t *scales,
                                       size_t inter, size_t cols, uint16_t *out) {
  size_t nb = cols / 32;
  for (size_t i = 0; i < inter; i++) {
    size_t src = 2 * i;
    orc_dequant_mxfp4_row_f16(blocks + src * nb * 16, scales + src * nb, nb, out + i * cols);
    src = 2 * i + 1;
    orc_dequant_mxfp4_row_f16(blocks + src * nb * 16, scales + src * nb, nb,
                              out + (inter + i) * cols);
  }
}

void orc_dequant_down_f16(const uint8_t *blocks, const uint8_t *scales, size_t rows, size_t cols,
                          uint16_t *out) {
  size_t nb = cols / 32;
  for (size_t r = 0; r < rows; r++)
    orc_dequant_mxfp4_row_f16(blocks + r * nb * 16, scales + r * nb, nb, out + r * cols);
}

/* ------------------------------------------------------------------ fp32 expert path */

/* Rust f32::clamp: NaN stays NaN. */
static inline float rclamp(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

/* Sequential, non-fused dot product (session.rs:75-85 order): acc = 0; acc += x[k] * w[k].
 * Eight independent rows/tokens are interleaved only for instruction-level parallelism;
 * each chain keeps the reference order. */
static void dot_rows_seq(const float *W, size_t rows, size_t cols, const float *x, float *y) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; r++) {
    const float *w = W + (size_t)r * cols;
    float acc = 0.0f;
    for (size_t k = 0; k < cols; k++) acc = acc + x[k] * w[k];
    y[r] = acc;
  }
}

/* T tokens against one row-major f32 matrix; xs is [T, cols], ys is [T, rows]. */
static void matmul_seq(const float *W, size_t rows, size_t cols, const float *xs, size_t T,
                       float *ys) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; r++) {
    const float *w = W + (size_t)r * cols;
    size_t t = 0;
    for (; t + 8 <= T; t += 8) {
      float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (size_t k = 0; k < cols; k++) {
        float wk = w[k];
        for (int u = 0; u < 8; u++) a[u] = a[u] + xs[(t + u) * cols + k] * wk;
      }
      for (int u = 0; u < 8; u++) ys[(t + u) * rows + r] = a[u];
    }
    for (; t < T; t++) {
      float acc = 0.0f;
      const float *x = xs + t * cols;
      for (size_t k = 0; k < cols; k++) acc = acc + x[k] * w[k];
      ys[t * rows + r] = acc;
    }
  }
}

void orc_mxfp4_matvec_f32(const uint8_t *blocks, const uint8_t *scales, size_t rows, size_t cols,
                          const float *x, float *y) {
  float *W = (float *)malloc(rows * cols * sizeof(float));
  orc_dequant_mxfp4_matrix(blocks, scales, rows, cols, W);
  dot_rows_seq(W, rows, cols, x, y);
  for (size_t r = 0; r < rows; r++) y[r] = canon(y[r]);
  free(W);
}

/* ------------------------------------------------------------------ MXFP6 activations */

/* |v| (already divided by its block scale, so |v| < 8) on the E2M3 grid: steps of 1/8 below 2,
 * 1/4 in [2, 4), 1/2 in [4, 8); round to nearest, ties to the even code (rintf in the default
 * rounding mode: the step count is even exactly when the code's last mantissa bit is 0);
 * everything from 7.5 up saturates to 7.5 (the largest E2M3 magnitude). */
static float e2m3_rne(float v) {
  const float a = fabsf(v);
  float q;
  if (a >= 7.5f) q = 7.5f;
  else {
    const float step = a < 2.0f ? 0.125f : (a < 4.0f ? 0.25f : 0.5f);
    q = rintf(a / step) * step;
  }
  return v < 0.0f ? -q : q;
}

void orc_quant_mxfp6(const float *x, size_t rows, size_t cols, float *out) {
  for (size_t r = 0; r < rows; r++) {
    const float *xr = x + r * cols;
    float *o = out + r * cols;
    for (size_t b0 = 0; b0 < cols; b0 += 32) {
      const size_t n = cols - b0 < 32 ? cols - b0 : 32;
      float m = 0.0f;
      int bad = 0;
      for (size_t i = 0; i < n; i++) {
        if (!isfinite(xr[b0 + i])) bad = 1;
        else if (fabsf(xr[b0 + i]) > m) m = fabsf(xr[b0 + i]);
      }
      if (bad) {
        for (size_t i = 0; i < n; i++) o[b0 + i] = u2f(ORC_CANON_NAN);
        continue;
      }
      int E = 0;
      if (m > 0.0f) frexpf(m, &E); /* m = f 2^E, f in [1/2, 1) */
      int se = E - 3;              /* 2^(floor(log2 m) - 2): the block maximum in [4, 8) */
      if (se < -126) se = -126;
      for (size_t i = 0; i < n; i++) o[b0 + i] = ldexpf(e2m3_rne(ldexpf(xr[b0 + i], -se)), se);
    }
  }
}

static void expert_ffn(const float *x, size_t T, const uint8_t *gu_blocks, const uint8_t *gu_scales,
                       const float *gu_bias, const uint8_t *d_blocks, const uint8_t *d_scales,
                       const float *d_bias, size_t H, size_t I, float limit, int quant, float *y,
                       float *h_out) {
  const float alpha = 1.702f; /* session.rs:99 */
  float *Wgu = (float *)malloc(2 * I * H * sizeof(float));
  float *Wd = (float *)malloc(H * I * sizeof(float));
  float *gu = (float *)malloc(T * 2 * I * sizeof(float));
  float *h = (float *)malloc(T * I * sizeof(float));
  float *xq = quant ? (float *)malloc(T * H * sizeof(float)) : NULL;
  orc_dequant_mxfp4_matrix(gu_blocks, gu_scales, 2 * I, H, Wgu);
  orc_dequant_mxfp4_matrix(d_blocks, d_scales, H, I, Wd);
  if (quant) orc_quant_mxfp6(x, T, H, xq);
  matmul_seq(Wgu, 2 * I, H, quant ? xq : x, T, gu);
  for (size_t t = 0; t < T; t++) {
    float *g = gu + t * 2 * I;
    for (size_t r = 0; r < 2 * I; r++) g[r] = g[r] + gu_bias[r];
    /* interleaved rows: gate = row 2i, up = row 2i+1 (weights.rs:425-460 then session.rs:109-117) */
    for (size_t i = 0; i < I; i++) {
      float gate = fminf(g[2 * i], limit);
      float up = rclamp(g[2 * i + 1], -limit, limit);
      float glu = gate / (1.0f + expf(-gate * alpha));
      h[t * I + i] = (up + 1.0f) * glu;
    }
  }
  if (quant) orc_quant_mxfp6(h, T, I, h);
  matmul_seq(Wd, H, I, h, T, y);
  for (size_t t = 0; t < T; t++)
    for (size_t r = 0; r < H; r++)
      y[t * H + r] = canon(rclamp(y[t * H + r] + d_bias[r], -65504.0f, 65504.0f));
  if (h_out)
    for (size_t i = 0; i < T * I; i++) h_out[i] = canon(h[i]);
  free(Wgu);
  free(Wd);
  free(gu);
  free(h);
  free(xq);
}

void orc_expert_ffn_f32(const float *x, size_t T, const uint8_t *gu_blocks,
                        const uint8_t *gu_scales, const float *gu_bias, const uint8_t *d_blocks,
                        const uint8_t *d_scales, const float *d_bias, size_t H, size_t I,
                        float limit, float *y, float *h_out) {
  expert_ffn(x, T, gu_blocks, gu_scales, gu_bias, d_blocks, d_scales, d_bias, H, I, limit, 0, y, h_out);
}

void orc_expert_ffn_mxfp6(const float *x, size_t T, const uint8_t *gu_blocks,
                          const uint8_t *gu_scales, const float *gu_bias, const uint8_t *d_blocks,
                          const uint8_t *d_scales, const float *d_bias, size_t H, size_t I,
                          float limit, float *y, float *h_out) {
  expert_ffn(x, T, gu_blocks, gu_scales, gu_bias, d_blocks, d_scales, d_bias, H, I, limit, 1, y, h_out);
}

/* ------------------------------------------------------------------ router */

void orc_router_logits(const uint16_t *w_bf16, const float *bias, const float *x, size_t T,
                       size_t E, size_t H, float *logits) {
#pragma omp parallel for schedule(static)
  for (long te = 0; te < (long)(T * E); te++) {
    size_t t = (size_t)te / E, e = (size_t)te % E;
    const uint16_t *w = w_bf16 + e * H;
    const float *xt = x + t * H;
    float p[64];
    for (int l = 0; l < 64; l++) p[l] = 0.0f;
    for (size_t k = 0; k < H; k++) p[k & 63] = fmaf(orc_bf16_to_f32(w[k]), xt[k], p[k & 63]);
    for (int o = 32; o >= 1; o >>= 1) {
      float q[64];
      for (int l = 0; l < 64; l++) q[l] = p[l] + p[l ^ o];
      memcpy(p, q, sizeof(p));
    }
    logits[t * E + e] = canon(p[0] + bias[e]);
  }
}

void orc_router_logits_seq(const uint16_t *w_bf16, const float *bias, const float *x, size_t T,
                           size_t E, size_t H, float *logits) {
  for (size_t t = 0; t < T; t++)
    for (size_t e = 0; e < E; e++) {
      float acc = bias[e];
      for (size_t d = 0; d < H; d++) acc = acc + orc_bf16_to_f32(w_bf16[e * H + d]) * x[t * H + d];
      logits[t * E + e] = canon(acc);
    }
}

/* Ranking used to order experts: (a, ia) before (b, ib)?  Greater logit first; logits
 * that compare equal (including +0 and -0) fall back to the lower index; NaN after all. */
static int ranks_before(float a, int ia, float b, int ib) {
  int an = isnan(a), bn = isnan(b);
  if (an || bn) {
    if (an && bn) return ia < ib;
    return bn;
  }
  if (a > b) return 1;
  if (a < b) return 0;
  return ia < ib;
}

void orc_topk(const float *logits, size_t T, size_t E, size_t k, const orc_adaptive *ad,
              int32_t *idx, float *w, float *probs, int32_t *k_used) {
  float *p = (float *)malloc(E * sizeof(float));
  int32_t *order = (int32_t *)malloc(E * sizeof(int32_t));
  char *taken = (char *)malloc(E);
  for (size_t t = 0; t < T; t++) {
    const float *l = logits + t * E;
    /* softmax over all experts, session.rs:511-520 */
    float m = -INFINITY;
    for (size_t e = 0; e < E; e++) m = fmaxf(m, l[e]);
    float s = 0.0f;
    for (size_t e = 0; e < E; e++) {
      p[e] = expf(l[e] - m);
      s = s + p[e];
    }
    if (s > 0.0f)
      for (size_t e = 0; e < E; e++) p[e] = p[e] / s;
    if (probs)
      for (size_t e = 0; e < E; e++) probs[t * E + e] = canon(p[e]);
    /* ranking (session.rs:822-825, totalised) */
    memset(taken, 0, E);
    size_t kk = k < E ? k : E;
    for (size_t s2 = 0; s2 < kk; s2++) {
      int best = -1;
      for (size_t e = 0; e < E; e++) {
        if (taken[e]) continue;
        if (best < 0 || ranks_before(l[e], (int)e, l[best], best)) best = (int)e;
      }
      if (best < 0) break;
      taken[best] = 1;
      order[s2] = best;
    }
    /* adaptive count, session.rs:569-583 */
    size_t sel = kk;
    if (ad && ad->enabled && kk > 1) {
      float p1 = kk >= 1 ? p[order[0]] : 0.0f;
      float p2 = kk >= 2 ? p[order[1]] : 0.0f;
      float margin = fmaxf(p1 - p2, 0.0f);
      if (p1 >= ad->top1_min_prob && margin >= ad->top1_min_margin)
        sel = 1;
      else if (kk >= 2 && (p1 + p2) >= ad->top2_min_mass)
        sel = 2;
      size_t mk = ad->min_k < kk ? ad->min_k : kk;
      if (sel < mk) sel = mk;
      if (sel > kk) sel = kk;
    }
    /* renormalise, session.rs:829-839 */
    float top_sum = 0.0f;
    for (size_t s2 = 0; s2 < sel; s2++) top_sum = top_sum + p[order[s2]];
    for (size_t s2 = 0; s2 < k; s2++) {
      if (s2 < sel) {
        idx[t * k + s2] = order[s2];
        w[t * k + s2] = (isfinite(top_sum) && top_sum > 0.0f) ? canon(p[order[s2]] / top_sum)
                                                              : 1.0f / (float)sel;
      } else {
        idx[t * k + s2] = -1;
        w[t * k + s2] = 0.0f;
      }
    }
    if (k_used) k_used[t] = (int32_t)sel;
  }
  free(p);
  free(order);
  free(taken);
}

void orc_combine(const float *outs, const float *w, size_t n, size_t H, int skip_nonfinite,
                 float *y) {
  for (size_t d = 0; d < H; d++) {
    float acc = 0.0f;
    for (size_t s = 0; s < n; s++) {
      float v = outs[s * H + d];
      if (skip_nonfinite && !isfinite(v)) continue;
      acc = acc + w[s] * v;
    }
    y[d] = canon(acc);
  }
}

float orc_rms_inv(const float *x, size_t H, float eps) {
  float p[64];
  for (size_t l = 0; l < 64; l++) {
    float a = 0.0f;
    for (size_t i = l; i < H; i += 64) {
      const float sq = x[i] * x[i];
      a = a + sq;
    }
    p[l] = a;
  }
  for (size_t o = 32; o >= 1; o >>= 1) {
    float q[64];
    for (size_t l = 0; l < 64; l++) q[l] = p[l] + p[l ^ o];
    memcpy(p, q, sizeof(p));
  }
  const float mean = p[0] / (float)H;
  return 1.0f / sqrtf(mean + eps); /* session.rs:487: (mean_sq + eps).sqrt().recip() */
}

void orc_rms_norm(const float *x, size_t T, size_t H, const float *gamma, float eps, float *n) {
  for (size_t t = 0; t < T; t++) {
    const float r = orc_rms_inv(x + t * H, H, eps);
    for (size_t d = 0; d < H; d++) {
      const float v = x[t * H + d] * r; /* session.rs:491: hidden * inv_rms * gamma, left to right */
      n[t * H + d] = v * gamma[d];
    }
  }
}

void orc_moe_block_f32(const float *x, size_t T, size_t H, size_t I, size_t E, size_t k, float limit,
                       const float *gamma, float eps, const uint16_t *router_w_bf16, const float *router_b,
                       const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                       const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                       const orc_adaptive *ad, float *out, float *logits, int32_t *idx, float *w) {
  float *n = (float *)malloc(T * H * sizeof(float));
  float *y = (float *)malloc(T * H * sizeof(float));
  orc_rms_norm(x, T, H, gamma, eps, n);
  orc_moe_layer_f32(n, T, H, I, E, k, limit, router_w_bf16, router_b, gu_blocks, gu_scales, gu_bias, d_blocks,
                    d_scales, d_bias, ad, y, logits, idx, w);
  for (size_t i = 0; i < T * H; i++) out[i] = canon(x[i] + y[i]); /* session.rs:982-994 residual add */
  free(n);
  free(y);
}

static void moe_layer(const float *x, size_t T, size_t H, size_t I, size_t E, size_t k, float limit,
                      const uint16_t *router_w_bf16, const float *router_b, const uint8_t *gu_blocks,
                      const uint8_t *gu_scales, const float *gu_bias, const uint8_t *d_blocks,
                      const uint8_t *d_scales, const float *d_bias, const orc_adaptive *ad, int quant,
                      float *y, float *logits_out, int32_t *idx_out, float *w_out) {
  size_t nbh = H / 32, nbi = I / 32;
  float *logits = (float *)malloc(T * E * sizeof(float));
  int32_t *idx = (int32_t *)malloc(T * k * sizeof(int32_t));
  float *w = (float *)malloc(T * k * sizeof(float));
  float *outs = (float *)malloc(T * k * H * sizeof(float));
  orc_router_logits(router_w_bf16, router_b, x, T, E, H, logits);
  orc_topk(logits, T, E, k, ad, idx, w, NULL, NULL);
  /* group tokens by expert so each expert is decoded once */
  float *xs = (float *)malloc(T * H * sizeof(float));
  float *ys = (float *)malloc(T * H * sizeof(float));
  size_t *slot_of = (size_t *)malloc(T * k * sizeof(size_t));
  for (size_t e = 0; e < E; e++) {
    size_t n = 0;
    for (size_t t = 0; t < T; t++)
      for (size_t s = 0; s < k; s++)
        if (idx[t * k + s] == (int32_t)e) {
          memcpy(xs + n * H, x + t * H, H * sizeof(float));
          slot_of[n++] = t * k + s;
        }
    if (!n) continue;
    expert_ffn(xs, n, gu_blocks + e * 2 * I * nbh * 16, gu_scales + e * 2 * I * nbh, gu_bias + e * 2 * I,
               d_blocks + e * H * nbi * 16, d_scales + e * H * nbi, d_bias + e * H, H, I, limit, quant, ys, NULL);
    for (size_t j = 0; j < n; j++) memcpy(outs + slot_of[j] * H, ys + j * H, H * sizeof(float));
  }
  for (size_t t = 0; t < T; t++) {
    size_t n = 0;
    while (n < k && idx[t * k + n] >= 0) n++;
    orc_combine(outs + t * k * H, w + t * k, n, H, 0, y + t * H);
  }
  if (logits_out) memcpy(logits_out, logits, T * E * sizeof(float));
  if (idx_out) memcpy(idx_out, idx, T * k * sizeof(int32_t));
  if (w_out) memcpy(w_out, w, T * k * sizeof(float));
  free(logits); free(idx); free(w); free(outs); free(xs); free(ys); free(slot_of);
}

void orc_moe_layer_f32(const float *x, size_t T, size_t H, size_t I, size_t E, size_t k,
                       float limit, const uint16_t *router_w_bf16, const float *router_b,
                       const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                       const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                       const orc_adaptive *ad, float *y, float *logits, int32_t *idx, float *w) {
  moe_layer(x, T, H, I, E, k, limit, router_w_bf16, router_b, gu_blocks, gu_scales, gu_bias, d_blocks, d_scales,
            d_bias, ad, 0, y, logits, idx, w);
}

void orc_moe_layer_mxfp6(const float *x, size_t T, size_t H, size_t I, size_t E, size_t k,
                         float limit, const uint16_t *router_w_bf16, const float *router_b,
                         const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                         const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                         const orc_adaptive *ad, float *y, float *logits, int32_t *idx, float *w) {
  moe_layer(x, T, H, I, E, k, limit, router_w_bf16, router_b, gu_blocks, gu_scales, gu_bias, d_blocks, d_scales,
            d_bias, ad, 1, y, logits, idx, w);
}

/* ------------------------------------------------------------------ live CPU path */

void orc_matvec_f16xf32(const uint16_t *a_f16, const float *x, float *y, size_t rows,
                        size_t cols) {
  for (size_t r = 0; r < rows; r++) {
    const uint16_t *a = a_f16 + r * cols;
    float acc[16];
    size_t k = 0;
#ifdef ORC_HAVE_AVX2
    __m256 v0 = _mm256_setzero_ps(), v1 = _mm256_setzero_ps();
    for (; k + 16 <= cols; k += 16) {
      __m256 w0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(a + k)));
      __m256 w1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(a + k + 8)));
      v0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k), w0, v0);
      v1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k + 8), w1, v1);
    }
    for (; k + 8 <= cols; k += 8) {
      __m256 w0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(a + k)));
      v0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k), w0, v0);
    }
    _mm256_storeu_ps(acc, v0);
    _mm256_storeu_ps(acc + 8, v1);
#else
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    for (; k + 16 <= cols; k += 16)
      for (int i = 0; i < 16; i++) acc[i] = fmaf(x[k + i], orc_f16_to_f32(a[k + i]), acc[i]);
    for (; k + 8 <= cols; k += 8)
      for (int i = 0; i < 8; i++) acc[i] = fmaf(x[k + i], orc_f16_to_f32(a[k + i]), acc[i]);
#endif
    float v[4];
    for (int i = 0; i < 4; i++) v[i] = (acc[i] + acc[4 + i]) + (acc[8 + i] + acc[12 + i]);
    y[r] = (v[0] + v[1]) + (v[2] + v[3]);
  }
}

void orc_cpu_expert_ffn_f16(const float *x, const uint16_t *gu_w, const uint16_t *gu_bias,
                            const uint16_t *d_w, const uint16_t *d_bias, float *out,
                            float *gate_up_buf, float *gated_buf, size_t H, size_t I) {
  const float limit = 7.0f, alpha = 1.702f; /* session.rs:98-99 */
  orc_matvec_f16xf32(gu_w, x, gate_up_buf, 2 * I, H);
  for (size_t j = 0; j < 2 * I; j++) gate_up_buf[j] = gate_up_buf[j] + orc_f16_to_f32(gu_bias[j]);
  for (size_t j = 0; j < I; j++) {
    float gate = fminf(gate_up_buf[j], limit);
    float up = rclamp(gate_up_buf[I + j], -limit, limit);
    float glu = gate / (1.0f + expf(-gate * alpha));
    gated_buf[j] = (up + 1.0f) * glu;
  }
  orc_matvec_f16xf32(d_w, gated_buf, out, H, I);
  for (size_t j = 0; j < H; j++)
    out[j] = rclamp(out[j] + orc_f16_to_f32(d_bias[j]), -65504.0f, 65504.0f);
}

typedef struct live_job {
  const float *x;
  size_t H, I;
  const uint8_t *gub, *gus, *db, *ds;
  const float *gubias, *dbias;
  float *out;
} live_job;

void orc_live_expert_f16(const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                         const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                         size_t H, size_t I, uint16_t *gu, uint16_t *gub, uint16_t *d, uint16_t *db) {
  orc_dequant_gate_up_reordered_f16(gu_blocks, gu_scales, I, H, gu);
  for (size_t i = 0; i < I; i++) {
    gub[i] = orc_f32_to_f16_rne(gu_bias[2 * i]);
    gub[I + i] = orc_f32_to_f16_rne(gu_bias[2 * i + 1]);
  }
  orc_dequant_down_f16(d_blocks, d_scales, H, I, d);
  for (size_t i = 0; i < H; i++) db[i] = orc_f32_to_f16_rne(d_bias[i]);
}

/* One selected expert on the cache-miss path: MXFP4 -> fp16 (session.rs:875-899), then
 * cpu_expert_ffn (session.rs:959-970). */
static void *live_worker(void *arg) {
  live_job *j = (live_job *)arg;
  size_t H = j->H, I = j->I;
  uint16_t *gu = (uint16_t *)malloc(2 * I * H * 2);
  uint16_t *gub = (uint16_t *)malloc(2 * I * 2);
  uint16_t *d = (uint16_t *)malloc(H * I * 2);
  uint16_t *db = (uint16_t *)malloc(H * 2);
  float *gbuf = (float *)malloc(2 * I * 4);
  float *hbuf = (float *)malloc(I * 4);
  orc_live_expert_f16(j->gub, j->gus, j->gubias, j->db, j->ds, j->dbias, H, I, gu, gub, d, db);
  orc_cpu_expert_ffn_f16(j->x, gu, gub, d, db, j->out, gbuf, hbuf, H, I);
  free(gu); free(gub); free(d); free(db); free(gbuf); free(hbuf);
  return NULL;
}

typedef struct warm_job {
  const float *x;
  size_t H, I;
  const uint16_t *gu, *gub, *d, *db;
  float *out;
} warm_job;

/* One selected expert on the cache-hit path: cpu_expert_ffn on the cached fp16 entry
 * (session.rs:959-970). */
static void *warm_worker(void *arg) {
  warm_job *j = (warm_job *)arg;
  float *gbuf = (float *)malloc(2 * j->I * 4);
  float *hbuf = (float *)malloc(j->I * 4);
  orc_cpu_expert_ffn_f16(j->x, j->gu, j->gub, j->d, j->db, j->out, gbuf, hbuf, j->H, j->I);
  free(gbuf); free(hbuf);
  return NULL;
}

/* Runs n jobs of `size` bytes at `jobs` with `worker`, at most n_threads at a time (rayon's
 * par_iter_mut over the k slots, session.rs:953-972). */
static void run_slots(void *jobs, size_t size, size_t n, int n_threads, void *(*worker)(void *)) {
  pthread_t *th = (pthread_t *)malloc(n * sizeof(pthread_t));
  if (n_threads < 1) n_threads = 1;
  for (size_t s0 = 0; s0 < n; s0 += (size_t)n_threads) {
    size_t s1 = s0 + (size_t)n_threads < n ? s0 + (size_t)n_threads : n;
    for (size_t s = s0; s < s1; s++) {
      void *a = (char *)jobs + s * size;
      if (pthread_create(&th[s], NULL, worker, a) != 0) worker(a), th[s] = 0;
    }
    for (size_t s = s0; s < s1; s++)
      if (th[s]) pthread_join(th[s], NULL);
  }
  free(th);
}

/* session.rs:974-980: sequential weighted accumulation in slot order */
static void live_combine(const float *outs, const float *w, size_t n, size_t H, float *y) {
  for (size_t d = 0; d < H; d++) {
    float acc = 0.0f;
    for (size_t s = 0; s < n; s++) acc = acc + w[s] * outs[s * H + d];
    y[d] = acc;
  }
}

int orc_live_moe_token_warm(const float *x, size_t H, size_t I, size_t n, const float *w,
                            const uint16_t *const *gu, const uint16_t *const *gub,
                            const uint16_t *const *d, const uint16_t *const *db, int n_threads,
                            float *y) {
  float *outs = (float *)malloc((n ? n : 1) * H * sizeof(float));
  warm_job *jobs = (warm_job *)malloc((n ? n : 1) * sizeof(warm_job));
  for (size_t s = 0; s < n; s++) jobs[s] = (warm_job){x, H, I, gu[s], gub[s], d[s], db[s], outs + s * H};
  run_slots(jobs, sizeof(warm_job), n, n_threads, warm_worker);
  live_combine(outs, w, n, H, y);
  free(outs); free(jobs);
  return 0;
}

#ifdef _OPENMP
#include <omp.h>
int orc_omp_max_threads(void) { return omp_get_max_threads(); }
#else
int orc_omp_max_threads(void) { return 1; }
#endif

int orc_live_moe_token(const float *x, size_t H, size_t I, size_t k, const int32_t *idx,
                       const float *w, const uint8_t *gu_blocks, const uint8_t *gu_scales,
                       const float *gu_bias, const uint8_t *d_blocks, const uint8_t *d_scales,
                       const float *d_bias, int n_threads, float *y) {
  size_t nbh = H / 32, nbi = I / 32;
  size_t n = 0;
  while (n < k && idx[n] >= 0) n++;
  float *outs = (float *)malloc((n ? n : 1) * H * sizeof(float));
  live_job *jobs = (live_job *)malloc((n ? n : 1) * sizeof(live_job));
  for (size_t s = 0; s < n; s++) {
    size_t e = (size_t)idx[s];
    jobs[s] = (live_job){x, H, I, gu_blocks + e * 2 * I * nbh * 16, gu_scales + e * 2 * I * nbh,
                         d_blocks + e * H * nbi * 16, d_scales + e * H * nbi, gu_bias + e * 2 * I,
                         d_bias + e * H, outs + s * H};
  }
  run_slots(jobs, sizeof(live_job), n, n_threads, live_worker);
  live_combine(outs, w, n, H, y);
  free(outs); free(jobs);
  return 0;
}

/* ------------------------------------------------------------------ LM head (bf16 rows) */

/* ModelWeights::lm_head_dot (weights.rs:73-82) for every row: w = bf16 -> f32 (exact),
 * acc = 0; acc += w * x[i] (separate product and sum, sequential in i). */
void orc_lm_head_bf16(const uint16_t *w_bf16, const float *x, size_t vocab, size_t H, float *y) {
#pragma omp parallel for schedule(static)
  for (long v = 0; v < (long)vocab; v++) {
    const uint16_t *row = w_bf16 + (size_t)v * H;
    float acc = 0.0f;
    for (size_t i = 0; i < H; i++) acc = acc + orc_bf16_to_f32(row[i]) * x[i];
    y[v] = canon(acc);
  }
}

/* ------------------------------------------------------------------ Beaver triples, p = 2^31 - 1 */

/* Field ops and hash of shader32.metal:4-33 (fmul folds 2^31 = 1; every result in [0, p)). */
#define ORC_P32 0x7FFFFFFFu
uint32_t orc_m31_mul(uint32_t a, uint32_t b) {
  uint64_t x = (uint64_t)a * (uint64_t)b;
  uint32_t lo = (uint32_t)(x & ORC_P32), hi = (uint32_t)(x >> 31);
  uint32_t r = lo + hi;
  r = (r >> 31) + (r & ORC_P32);
  return r >= ORC_P32 ? r - ORC_P32 : r;
}
uint32_t orc_m31_add(uint32_t a, uint32_t b) {
  uint32_t r = a + b;
  return r >= ORC_P32 ? r - ORC_P32 : r;
}
uint32_t orc_chash32(uint32_t seed, uint32_t idx) {
  uint32_t x = seed ^ (idx * 0x9e3779b9u);
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  x &= 0x7FFFFFFFu;
  return x >= ORC_P32 ? x - ORC_P32 : x;
}

/* beaver_triple_gen_32 (party < 0) / beaver_triple_gen_single_party_32 (party >= 0),
 * shader32.metal:75-167, run as the Metal dispatch runs it (gpu/mod.rs:975-1000): one thread
 * per round, threadgroups of w = min(32, num_rounds) threads, one SIMD group of 32 lanes per
 * threadgroup, lane = index in the threadgroup. Lanes past the last round do not exist; a
 * shuffle from a lane that does not exist is taken as 0 (the Metal result there is undefined).
 * him[j][i] = (i + 1)^j for j < spr (mod.rs:606-612), eval_raw[p] = p + 1 (mod.rs:561). */
void orc_beaver32(size_t n, size_t spr, long party, size_t count, const uint32_t *seeds,
                  uint32_t *a_out, uint32_t *b_out, uint32_t *c_out) {
  size_t rounds = (count + spr - 1) / spr;
  size_t w = rounds < 32 ? rounds : 32;
  uint32_t him[3][8], ev[8];
  for (size_t i = 0; i < 8; i++) ev[i] = (uint32_t)(i + 1);
  for (size_t j = 0; j < 3; j++)
    for (size_t i = 0; i < 8; i++) {
      uint32_t v = 1;
      for (size_t e = 0; e < j; e++) v = orc_m31_mul(v, (uint32_t)(i + 1));
      him[j][i] = v;
    }
  for (size_t g0 = 0; g0 < rounds; g0 += w) {
    size_t lanes = rounds - g0 < w ? rounds - g0 : w;
    uint32_t rt[32] = {0};
    int exists[32] = {0};
    for (size_t l = 0; l < lanes; l++) {
      exists[l] = 1;
      uint32_t i = (uint32_t)(l % n);
      rt[l] = l < n ? orc_chash32(seeds[g0 + l], i * 3u) : 0u;
    }
    for (size_t l = 0; l < lanes; l++) {
      size_t round = g0 + l, base = round * spr;
      for (size_t j = 0; j < spr && base + j < count; j++) {
        /* simd_fadd_reduce over xor 1, 2, 4: the aligned group of 8 lanes holding l */
        uint32_t bt = 0;
        for (size_t q = l & ~(size_t)7; q < (l & ~(size_t)7) + 8; q++) {
          if (!exists[q]) continue;
          uint32_t m = q < n ? him[j][q % n] : 0u;
          bt = orc_m31_add(bt, orc_m31_mul(m, rt[q]));
        }
        uint32_t seed = seeds[round];
        uint32_t a0 = orc_chash32(seed, (uint32_t)(n * 3 + spr * 2 + j * 2));
        uint32_t b0 = orc_chash32(seed, (uint32_t)(n * 3 + spr * 2 + j * 2 + 1));
        uint32_t ca = orc_chash32(seed, (uint32_t)(n * 3 + j * 2));
        uint32_t cb = orc_chash32(seed, (uint32_t)(n * 3 + j * 2 + 1));
        size_t out = base + j;
        if (party >= 0) {
          uint32_t x = ev[party];
          a_out[out] = orc_m31_add(a0, orc_m31_mul(ca, x));
          b_out[out] = orc_m31_add(b0, orc_m31_mul(cb, x));
          c_out[out] = orc_m31_add(orc_m31_mul(a0, b0), orc_m31_mul(x, bt));
        } else {
          for (size_t p = 0; p < n; p++) {
            uint32_t x = ev[p];
            size_t d = p * count + out;
            a_out[d] = orc_m31_add(a0, orc_m31_mul(ca, x));
            b_out[d] = orc_m31_add(b0, orc_m31_mul(cb, x));
            c_out[d] = orc_m31_add(orc_m31_mul(a0, b0), orc_m31_mul(x, bt));
          }
        }
      }
    }
  }
}
