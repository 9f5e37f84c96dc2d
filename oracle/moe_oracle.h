/*
 * CPU ORACLE — test infrastructure only, never product code.
 *
 * A plain-C restatement of the reference's GPT-OSS MXFP4 mixture-of-experts path
 * (gabearro/SilentOTITHRanDouSha, src/gpt_oss/{weights,session}.rs). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker or as the timed CPU baseline; the HIP library never links it.
 *
 * Every function names the reference lines it restates. Pinning (what checks each function
 * against something other than itself) lives in tests/test_oracle.py: the committed
 * closed-form decode table and float64 restatement under tests/golden/, brute-force top-k,
 * order-sensitive vectors for the router and the NEON matvec, special cases of the SwiGLU.
 * Parity unpinned (no vector can exist offline): the ANE fp16 router numerics the fp32
 * router replaces (executables.rs:260-317), macOS libm expf last-ulp behaviour
 * (session.rs:114), and the `half` 2.7.1 crate calls themselves (pinned only by their closed
 * forms: bf16/f16 -> f32 exact, f32 -> f16 IEEE round-to-nearest-even).
 *
 * Floating-point rules: compiled with -ffp-contract=off so every `a * b + c` written as
 * separate operations rounds twice, as Rust does (Rust never contracts to FMA); fused
 * multiply-adds appear only where the reference uses them (NEON vfmaq in
 * matvec_f16xf32) or where the canonical router order defines them (fmaf).
 * NaNs produced by invalid operations are canonicalised to 0x7FC00000, the aarch64
 * default NaN, because the reference runs on aarch64 (x86 would give 0xFFC00000).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (half 2.7.1 semantics, Cargo.lock) ---- */
float orc_bf16_to_f32(uint16_t b);            /* bf16::from_bits(..).to_f32(): exact */
uint16_t orc_f32_to_bf16_rne(float f);        /* round-to-nearest-even, NaN kept quiet */
float orc_f16_to_f32(uint16_t h);             /* f16::from_bits(..).to_f32(): exact */
uint16_t orc_f32_to_f16_rne(float f);         /* f16::from_f32: IEEE RNE */

/* ---- MXFP4 decode ---- */
/* weights.rs:350-371 dequant_mxfp4_row: out[32b+2j] = LUT[lo]*2^(s-127), out[32b+2j+1] = LUT[hi]*... */
void orc_dequant_mxfp4_row(const uint8_t *blocks, const uint8_t *scales, size_t nb, float *out);
/* weights.rs:373-423 dequant_expert_{gate_up,down}_into: row loop of the above */
void orc_dequant_mxfp4_matrix(const uint8_t *blocks, const uint8_t *scales, size_t rows,
                              size_t cols, float *out);
/* weights.rs:425-452 de-interleave: source row 2i -> gate row i, 2i+1 -> up row inter+i */
void orc_dequant_gate_up_reordered(const uint8_t *blocks, const uint8_t *scales, size_t inter,
                                   size_t cols, float *out);

/* ---- MXFP4 -> fp16 decode of the live path (scalar fallback, weights.rs:593-639) ---- */
uint16_t orc_f16_mul_scalar(uint16_t val_bits, uint16_t scale_bits);   /* weights.rs:619-639 */
void orc_dequant_mxfp4_row_f16(const uint8_t *blocks, const uint8_t *scales, size_t nb,
                               uint16_t *out);                        /* weights.rs:593-616 */
void orc_dequant_gate_up_reordered_f16(const uint8_t *blocks, const uint8_t *scales,
                                       size_t inter, size_t cols, uint16_t *out); /* :641-664 */
void orc_dequant_down_f16(const uint8_t *blocks, const uint8_t *scales, size_t rows,
                          size_t cols, uint16_t *out);                /* weights.rs:666-682 */

/* ---- fp32 reference expert FFN (the parity oracle) ----
 * x: [T, H] f32. Weights in the checkpoint layout: gate_up blocks [2I, H/32, 16], scales
 * [2I, H/32], bias [2I] (interleaved gate/up rows); down blocks [H, I/32, 16], scales
 * [H, I/32], bias [H]. y: [T, H]. Decode = weights.rs:350-371; arithmetic = session.rs:89-124
 * with f32 weights and biases: sequential non-fused dot products (session.rs:75-85 order),
 * gate = min(g, limit) (NaN-ignoring f32::min), up = clamp(u, -limit, limit) (NaN-propagating),
 * glu = gate / (1 + exp(-gate * 1.702)), h = (up + 1) * glu, y = clamp(down + bias, +-65504).
 * h_out (optional, [T, I]) receives the SwiGLU output. */
void orc_expert_ffn_f32(const float *x, size_t T, const uint8_t *gu_blocks,
                        const uint8_t *gu_scales, const float *gu_bias, const uint8_t *d_blocks,
                        const uint8_t *d_scales, const float *d_bias, size_t H, size_t I,
                        float limit, float *y, float *h_out);
/* ---- quantized-activation mode (no counterpart in the reference: the GPU's opt-in
 * MOE_OPT_ACT_QUANT contract) ----
 * orc_quant_mxfp6: each row's values in blocks of 32 (a short last block as it is) replaced by
 * their MXFP6 value: scale 2^(floor(log2 amax) - 2) = 2^(E - 3) where amax = f 2^E, f in
 * [1/2, 1) (OCP MX v1.0 with E2M3's largest exponent 2; 2^-3 for an all-zero block, at least
 * 2^-126), each value divided by it, rounded to nearest (ties to even) on the E2M3 grid and
 * saturated at 7.5, then multiplied back. A block holding a non-finite value becomes NaN.
 * out may equal x.
 * orc_expert_ffn_mxfp6 (and orc_moe_layer_mxfp6 below): orc_expert_ffn_f32 with the
 * expert's input x and its SwiGLU output h replaced by their MXFP6 values before each product
 * (routing reads x unquantized). */
void orc_quant_mxfp6(const float *x, size_t rows, size_t cols, float *out);
void orc_expert_ffn_mxfp6(const float *x, size_t T, const uint8_t *gu_blocks,
                          const uint8_t *gu_scales, const float *gu_bias, const uint8_t *d_blocks,
                          const uint8_t *d_scales, const float *d_bias, size_t H, size_t I,
                          float limit, float *y, float *h_out);
/* y = W x with W decoded by weights.rs:350-371; sequential non-fused sum per row. */
void orc_mxfp4_matvec_f32(const uint8_t *blocks, const uint8_t *scales, size_t rows, size_t cols,
                          const float *x, float *y);

/* ---- router ----
 * Canonical order (declared; the GPU kernel computes exactly this): for expert e, 64
 * partial sums p_l = fmaf-chain over k = l, l+64, ... (k < H, increasing), then a
 * xor-butterfly p_l <- p_l + p_{l^o} for o = 32,16,8,4,2,1, then logit = p_0 + bias[e].
 * W is bf16 (weights.rs:280-281 loads it through bf16 -> f32, exact). */
void orc_router_logits(const uint16_t *w_bf16, const float *bias, const float *x, size_t T,
                       size_t E, size_t H, float *logits);
/* session.rs:503-510 order: acc = bias; acc += w*x sequentially (non-fused). Comparison only. */
void orc_router_logits_seq(const uint16_t *w_bf16, const float *bias, const float *x, size_t T,
                           size_t E, size_t H, float *logits);

typedef struct orc_adaptive {
  int enabled;          /* GPT_OSS_ADAPTIVE_MOE_TOPK */
  size_t min_k;         /* GPT_OSS_ADAPTIVE_MIN_K */
  float top1_min_prob;  /* GPT_OSS_ADAPTIVE_TOP1_MIN */
  float top1_min_margin;/* GPT_OSS_ADAPTIVE_TOP1_MARGIN_MIN */
  float top2_min_mass;  /* GPT_OSS_ADAPTIVE_TOP2_MASS_MIN */
} orc_adaptive;

/* Softmax over all E (session.rs:511-520), order by probability descending (session.rs:822-825)
 * refined to a total order: logit descending, equal logits -> lower index, NaN last;
 * keep k (or the adaptive count, session.rs:569-583); renormalise (session.rs:826-839).
 * idx/w: [T, k]; slots past the adaptive count get idx -1 and weight 0. probs (optional):
 * [T, E] softmax probabilities. Returns nothing; k_used (optional, [T]) gets the count. */
void orc_topk(const float *logits, size_t T, size_t E, size_t k, const orc_adaptive *ad,
              int32_t *idx, float *w, float *probs, int32_t *k_used);

/* Whole MoE block of session.rs:818-980 on the fp32 path. Experts are given as per-layer
 * packed tensors [E, ...] in the checkpoint layout (weights.rs:283-316 slicing).
 * logits/idx/w outputs optional. */
void orc_moe_layer_f32(const float *x, size_t T, size_t H, size_t I, size_t E, size_t k,
                       float limit, const uint16_t *router_w_bf16, const float *router_b,
                       const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                       const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                       const orc_adaptive *ad, float *y, float *logits, int32_t *idx, float *w);
/* The same with the experts' activations as MXFP6 (orc_expert_ffn_mxfp6). */
void orc_moe_layer_mxfp6(const float *x, size_t T, size_t H, size_t I, size_t E, size_t k,
                         float limit, const uint16_t *router_w_bf16, const float *router_b,
                         const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                         const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                         const orc_adaptive *ad, float *y, float *logits, int32_t *idx, float *w);

/* Post-attention RMSNorm of the reference's fp32 restatement (session.rs:483-493):
 * inv_rms = 1 / sqrt(mean(x^2) + eps) (mean = sum / H, sqrt and reciprocal correctly rounded),
 * n[d] = (x[d] * inv_rms) * gamma[d]. The sum of squares runs in the canonical order of the GPU
 * kernels, not the reference's sequential one (they differ by rounding only): 64 lane partials
 * p_l = sum over i ascending of x[l + 64 i]^2, then the xor butterfly p_l += p_(l^o) for
 * o = 32, 16, 8, 4, 2, 1 (every lane ends with the same bits: each step adds a commuted pair). */
float orc_rms_inv(const float *x, size_t H, float eps);
void orc_rms_norm(const float *x, size_t T, size_t H, const float *gamma, float eps, float *n);

/* The MoE block with the norm and residual around it (executables.rs:260-317 router fusion,
 * session.rs:483-493, 943-997): n = RMSNorm(x) * gamma, y = MoE(n) as orc_moe_layer_f32,
 * out = x + y. */
void orc_moe_block_f32(const float *x, size_t T, size_t H, size_t I, size_t E, size_t k, float limit,
                       const float *gamma, float eps, const uint16_t *router_w_bf16, const float *router_b,
                       const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                       const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                       const orc_adaptive *ad, float *out, float *logits, int32_t *idx, float *w);

/* session.rs:974-980 combine: y[d] = 0; y[d] += w_s * out_s[d] for slots in rank order.
 * skip_nonfinite = 1 gives the moe_dispatch.rs:594-603 variant (non-finite out_s[d] skipped). */
void orc_combine(const float *outs, const float *w, size_t n, size_t H, int skip_nonfinite,
                 float *y);

/* ---- live CPU path of the reference (the timed CPU baseline) ---- */
/* session.rs:20-73 NEON matvec order: 16 fused partial sums (4 x float32x4), 8-wide tail,
 * then (acc0+acc1)+(acc2+acc3) lane-wise and a pairwise horizontal add. */
void orc_matvec_f16xf32(const uint16_t *a_f16, const float *x, float *y, size_t rows,
                        size_t cols);
/* session.rs:89-124 cpu_expert_ffn on fp16 weights/biases (reordered gate/up). */
void orc_cpu_expert_ffn_f16(const float *x, const uint16_t *gu_w, const uint16_t *gu_bias,
                            const uint16_t *d_w, const uint16_t *d_bias, float *out,
                            float *gate_up_buf, float *gated_buf, size_t H, size_t I);
/* One token through the live MoE block (session.rs:851-980) with `cold` experts decoded from
 * MXFP4 to fp16 first (the cache-miss case) or taken from a caller-provided warm cache.
 * Experts run on one thread per slot, like rayon's par_iter over k slots (session.rs:953-972).
 * idx/w come from orc_topk. Returns 0 on success. */
int orc_live_moe_token(const float *x, size_t H, size_t I, size_t k, const int32_t *idx,
                       const float *w, const uint8_t *gu_blocks, const uint8_t *gu_scales,
                       const float *gu_bias, const uint8_t *d_blocks, const uint8_t *d_scales,
                       const float *d_bias, int n_threads, float *y);
/* The reference's fp16 expert-cache entry for one expert (session.rs:126-136, filled on a miss
 * at :875-899): gate/up de-interleaved to [gate I; up I] x H fp16 (weights.rs:641-660), biases
 * rounded f32 -> fp16 (weights.rs:686-702), down H x I fp16. */
void orc_live_expert_f16(const uint8_t *gu_blocks, const uint8_t *gu_scales, const float *gu_bias,
                         const uint8_t *d_blocks, const uint8_t *d_scales, const float *d_bias,
                         size_t H, size_t I, uint16_t *gu, uint16_t *gub, uint16_t *d, uint16_t *db);
/* One token on the live path with every selected expert already in the fp16 cache (the hit
 * path of session.rs:851-941): cpu_expert_ffn per slot on up to n_threads threads
 * (session.rs:953-972) and the slot-order combine (:974-980). gu[s] ... db[s]: slot s's entry. */
int orc_live_moe_token_warm(const float *x, size_t H, size_t I, size_t n, const float *w,
                            const uint16_t *const *gu, const uint16_t *const *gub,
                            const uint16_t *const *d, const uint16_t *const *db, int n_threads,
                            float *y);
/* ModelWeights::lm_head_dot (weights.rs:73-82) for all rows of a bf16 [vocab, H] LM head. */
void orc_lm_head_bf16(const uint16_t *w_bf16, const float *x, size_t vocab, size_t H, float *y);
/* Beaver triples over p = 2^31 - 1 (shader32.metal:4-167 as dispatched by gpu/mod.rs:975-1000):
 * field ops, the hash, and both kernels (party < 0: every party, outputs [n][count]). */
uint32_t orc_m31_mul(uint32_t a, uint32_t b);
uint32_t orc_m31_add(uint32_t a, uint32_t b);
uint32_t orc_chash32(uint32_t seed, uint32_t idx);
void orc_beaver32(size_t n, size_t spr, long party, size_t count, const uint32_t *seeds,
                  uint32_t *a_out, uint32_t *b_out, uint32_t *c_out);
/* OpenMP threads the oracle's parallel loops use (the fp32 path's matmuls). */
int orc_omp_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
