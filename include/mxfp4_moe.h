/*
 * mxfp4_moe.h — C ABI of the MI355X (gfx950) MXFP4 mixture-of-experts path.
 *
 * Drop-in replacement for the GPU backend of gabearro/SilentOTITHRanDouSha's GPT-OSS MoE
 * block. Each entry point names the reference item it replaces (file:line in that repo).
 * All entry points return 0 (MOE_OK) or a MOE_ERR_* code; the message of the last failure
 * on the calling thread is returned by moe_last_error() (this replaces the reference's
 * Result<_, String>). No C++ exception crosses this boundary.
 *
 * Layout conventions (the checkpoint's, weights.rs:17-27 and :283-316):
 *   gate_up blocks [E, 2*I, H/32, 16] u8   — interleaved rows: row 2i = gate i, 2i+1 = up i
 *   gate_up scales [E, 2*I, H/32]     u8   — E8M0
 *   gate_up bias   [E, 2*I]           f32
 *   down    blocks [E, H, I/32, 16]   u8
 *   down    scales [E, H, I/32]       u8
 *   down    bias   [E, H]             f32
 *   Block byte j of block b holds element 32b+2j in its low nibble and 32b+2j+1 in its high.
 *   router weight  [E, H] bf16 bits (as stored in the checkpoint), bias [E] f32.
 *
 * Pointers: host pointers unless the name ends in _device, whose arguments are device
 * pointers (HBM) and a stream (a hipStream_t passed as void*, NULL = the context's stream).
 * Host-pointer calls are synchronous (the reference's commit()+wait_until_completed()).
 * Device calls are asynchronous on the given stream.
 *
 * Threading: a context owns device scratch that every dispatch writes (as the reference's
 * GpuMoeDispatcher does through shared buffers, moe_dispatch.rs:245-251). Calls on one
 * context must be serialised by the caller; distinct contexts are independent.
 */
#ifndef MXFP4_MOE_H
#define MXFP4_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moe_ctx moe_ctx;

enum moe_status {
  MOE_OK = 0,
  MOE_ERR_INVALID = 1,   /* bad argument, shape or length */
  MOE_ERR_STATE = 2,     /* call out of order: layer / router / LM head not loaded */
  MOE_ERR_HIP = 3,       /* HIP runtime error (message names the call) */
  MOE_ERR_NO_DEVICE = 4, /* no gfx950 device visible */
  MOE_ERR_OOM = 5,       /* device allocation failed */
  MOE_ERR_IO = 6         /* a file cannot be opened, mapped or parsed */
};

/* Message of the last failing call on this thread ("" if none). */
const char *moe_last_error(void);
/* Library version string. */
const char *moe_version(void);

/* ------------------------------------------------------------------ context */

/* GpuMoeDispatcher::new(hidden_size, inter_size, swiglu_clamp) — moe_dispatch.rs:60-146.
 * hidden_size and inter_size must be positive multiples of 32 (MXFP4 block length).
 * swiglu_clamp is GptOssConfig::swiglu_limit (config.rs:50, default 7.0). */
int moe_create(size_t hidden_size, size_t inter_size, float swiglu_clamp, moe_ctx **out);
/* Drop (no reference counterpart beyond Rust's Drop of GpuMoeDispatcher). */
void moe_destroy(moe_ctx *ctx);

/* Adaptive top-k of session.rs:168-201 / :569-583 (GPT_OSS_ADAPTIVE_MOE_TOPK and friends).
 * Off by default, as in the reference. enabled=0 turns it off. */
int moe_set_adaptive_topk(moe_ctx *ctx, int enabled, size_t min_k, float top1_min_prob,
                          float top1_min_margin, float top2_min_mass);

/* Options (no reference counterpart).
 * MOE_OPT_FUSED_DECODE selects how single-token forwards run: 2 (default) one launch (router,
 * top-k, gate_up, SwiGLU, down and combine, with the down weights streaming during gate_up;
 * up to 128 experts), 1 two launches (router + gate_up; down + combine), 0 the five-kernel
 * path that batches take. Shapes a mode does not support take the next lower one. Results
 * agree to the matmul tolerance; routing is identical.
 * MOE_OPT_SPIN_LIMIT: polls before a cross-block wait of the one-launch kernel gives up
 * (default 2^20); a wait that gives up makes the outputs NaN and the next moe_synchronize or
 * moe_layer_forward return MOE_ERR_HIP (which clears the condition).
 * MOE_OPT_BATCH_GEMM: batches (n_tokens > 1) run through the grouped GEMM on the block-scaled
 * MFMA (activations as fp8 terms, exact to 2^-12) when 1 (default) and experts average at
 * least 4 entries, or always when 2; otherwise, and when 0, through the per-tile GEMV kernels
 * (bf16 hi+lo activations). Results agree to the matmul tolerance; routing is identical.
 * MOE_OPT_GEMM_SHAPE: block shape of the grouped GEMM: 0 (default) by the mean entries per
 * expert (14 to 44, 60 to 72, and for the down GEMM 14 to 72: the wide streamed form of code 14;
 * otherwise 48+: 512 rows x 64 entries in 8 wavefronts, at K of 2817-3072 with the pipelined step
 * of code 15 (the down GEMM: of code 17); 24+: 128 x 32 in 2; else the streamed form of code 12, or
 * 128 x 16 in 2 where neither fits);
 * for experts averaging 48+ entries 1 selects 8 wavefronts as 8 x 1 instead of 4 x 2; 2 and 3
 * force 256-row x 32- and 16-entry blocks of 4 wavefronts, 4 the 128-row x 16-entry block of 4
 * wavefronts (down only; gate_up takes 3), 5 the 128 x 16 block of 2 wavefronts, 6 a 64 x 16
 * block of 1, 7 the 128 x 32 block of 2, 8 the 512 x 128 block of 4 wavefronts (one per SIMD,
 * each 256 rows x 64 entries, B operands held for a whole K-step), 9 the 512 x 128 block of 8
 * wavefronts (each 128 rows x 64 entries; quantized activations only, the default there for
 * experts averaging 96+ entries; with the exact split it selects the default shape), 10 the
 * 512 x 64 block of 8 wavefronts on the 32 x 32 x 64 block-scaled MFMA (each 128 rows x 32
 * entries), 11 the 512 x 128 block of 8 wavefronts each holding 256 rows x 32 entries (B held
 * for a K-step), 12 the streamed form for a few entries per expert (one workgroup per CU taking a
 * contiguous share of the (16-entry chunk x 64 rows (gate_up) or 32 rows (down)) units, four at
 * a time: the weights through register rings, the shared activation records through an LDS ring
 * loaded by a fifth wavefront; launches it does not fit take the 128 x 16 block), 13 the same
 * with other ring depths, 14 the wide streamed form for tens of entries per expert (units of
 * 64 (gate_up) or 32 (down) rows x a group of up to 5 16-entry chunks of one expert, so every
 * weight tile streams once per group; launches it does not fit take the default), 15 the 512 x 64
 * block with the pipelined step (each wavefront reads the next K-step's operands while its MFMAs
 * run; one barrier per step; K of 2817 to 3072 values, other K the plain step), 16 and 17 the same
 * with separate rings for the weights and the activation records (16: records three steps deep,
 * 17: weights three deep; the default for the down GEMM where code 15's K applies), 18 and 19 the
 * pipelined step (each GEMM with its default rings) on one workgroup per CU taking its tiles from
 * a queue, the next tile's first DMAs issued inside the current tile's epilogue (18: the per-XCD
 * ranges of MOE_OPT_GEMM_BAND's order when that applies; 19: one queue in the plain order; exact
 * split, K of 2817 to 3072 values, otherwise as code 0) (tuning; codes 0-9 and 11-19 give
 * identical results, code 10 the same to f32 rounding: its MFMA sums 64 products where the others
 * sum 128). MOE_OPT_GEMM_SHAPE_DOWN: the same codes for the down GEMM alone
 * (0, default: as MOE_OPT_GEMM_SHAPE).
 * MOE_OPT_GEMM_BAND: row blocks per band of the grouped GEMM's per-XCD tile order for both
 * matrices, 1..64; 0 (default): gate_up in workgroup order, down in bands of 1 (tuning; results
 * identical).
 * MOE_OPT_MATVEC: moe_mxfp4_matvec_device runs in one launch on the block-scaled MFMA (x as 4
 * fp8 terms, exact to 2^-16) when 1 (default) and cols <= 3072 with x 16-byte aligned; otherwise,
 * and when 0, as two launches on the bf16 MFMA (x as bf16 hi + lo). Results agree to 1e-5.
 * MOE_OPT_ACT_QUANT: 0 (default) the grouped GEMM takes its activations (x, and the SwiGLU output
 * h) exact to about 2^-13 of each 32-value block's maximum (3 E2M3 terms), within the 1e-3
 * tolerance of the f32 path; 1 quantizes them to MXFP6 (one E2M3 value per element, one E8M0
 * scale per 32-value block, the OCP MX rule: scale 2^(floor(log2 amax) - 2), round to nearest
 * even, saturate at 7.5): a third of the MFMA work, and results that follow the f32 path applied
 * to those quantized activations (not the f32 path itself). Routing is unchanged (the router
 * reads x unquantized); single-token forwards and the GEMV batch path are unaffected. In this mode
 * MOE_OPT_GEMM_SHAPE(_DOWN) codes 2, 3, 4, 6 and 8 select the default shape. Changing it
 * re-lays out the context's h records: the call waits until the whole device is idle
 * (hipDeviceSynchronize), so forwards enqueued on any stream finish first, and it is refused
 * during graph capture.
 * MOE_OPT_LOCAL_GROUP: 1 (default) batches of at most 1024 (token, slot) entries whose gate_up
 * GEMM runs in the streamed form have the GEMM's workgroups group the entries by expert
 * themselves, from the top-k indices (the router then skips its grouping); 0 the router groups
 * them (tuning; results identical). */
enum moe_option {
  MOE_OPT_FUSED_DECODE = 1,
  MOE_OPT_SPIN_LIMIT = 2,
  MOE_OPT_BATCH_GEMM = 3,
  MOE_OPT_GEMM_SHAPE = 4,
  MOE_OPT_GEMM_BAND = 5,
  MOE_OPT_MATVEC = 6,
  MOE_OPT_GEMM_SHAPE_DOWN = 7,
  MOE_OPT_ACT_QUANT = 8,
  MOE_OPT_LOCAL_GROUP = 9
};
int moe_set_option(moe_ctx *ctx, int option, int64_t value);

/* ------------------------------------------------------------------ weights */

/* GpuMoeDispatcher::preload_experts — moe_dispatch.rs:149-229, one layer per call.
 * Copies one layer's experts (checkpoint layout above) into HBM, repacked for the kernels.
 * The repack is a lossless permutation; moe_dequant_expert reads it back. Re-preloading a
 * layer index replaces it. Short bias arrays are not accepted: pass full [E,2I] / [E,H]. */
int moe_preload_layer(moe_ctx *ctx, size_t layer, size_t n_experts,
                      const uint8_t *gate_up_blocks, const uint8_t *gate_up_scales,
                      const float *gate_up_bias, const uint8_t *down_blocks,
                      const uint8_t *down_scales, const float *down_bias);
/* Same, with the checkpoint tensors already in device memory (e.g. memory-mapped upload). */
int moe_preload_layer_device(moe_ctx *ctx, size_t layer, size_t n_experts,
                             const uint8_t *gate_up_blocks, const uint8_t *gate_up_scales,
                             const float *gate_up_bias, const uint8_t *down_blocks,
                             const uint8_t *down_scales, const float *down_bias, void *stream);
/* One expert of GpuMoeDispatcher::preload_experts — moe_dispatch.rs:149-229, whose loop
 * creates per-expert device buffers from each ExpertMxfp4 (weights.rs:17-27). Tensors are that
 * expert's alone (no [E] dimension); lengths as for moe_dispatch_expert (blocks and scales
 * exact, biases may be short and are zero-padded). A layer is usable by the path-level calls
 * once all n_experts of it are preloaded; a different n_experts for a layer discards it. */
int moe_preload_expert(moe_ctx *ctx, size_t layer, size_t n_experts, size_t expert_idx,
                       const uint8_t *gate_up_blocks, size_t gate_up_blocks_len,
                       const uint8_t *gate_up_scales, size_t gate_up_scales_len,
                       const float *gate_up_bias, size_t gate_up_bias_len,
                       const uint8_t *down_blocks, size_t down_blocks_len,
                       const uint8_t *down_scales, size_t down_scales_len,
                       const float *down_bias, size_t down_bias_len);
/* Router weights of one layer (LayerWeights::router_weight/bias, weights.rs:44-46, loaded at
 * weights.rs:280-281). In the reference the router runs on the ANE inside
 * build_decode_output_proj_router (executables.rs:301-313); here it runs on the GPU. */
int moe_preload_router(moe_ctx *ctx, size_t layer, size_t n_experts,
                       const uint16_t *weight_bf16, const float *bias);
/* Same with f32 weights; every value must be exactly representable in bf16 (true for
 * weights loaded through bf16_to_f32, weights.rs:141-147), else MOE_ERR_INVALID. */
int moe_preload_router_f32(moe_ctx *ctx, size_t layer, size_t n_experts, const float *weight,
                           const float *bias);

/* Post-attention RMSNorm weight of one layer (LayerWeights::post_attn_layernorm_weight,
 * weights.rs:32, loaded at weights.rs:267-268, bf16 widened to f32) and
 * GptOssConfig::rms_norm_eps (config.rs:42-43, default 1e-5 at :59-61). */
int moe_preload_norm(moe_ctx *ctx, size_t layer, const float *gamma, float eps);

/* Safetensors MXFP4 loader — the reference's ShardReader (weights.rs:103-139) and the per-layer
 * tensor names of load_weights (weights.rs:228-346), reading local shards instead of the hub
 * download (weights.rs:168-213). Loads layer `layer`'s experts
 *   model.layers.{layer}.mlp.experts.{gate_up,down}_proj_{blocks,scales} (U8) and _bias (BF16)
 * and router model.layers.{layer}.mlp.router.{weight,bias} (BF16), each from the first shard
 * that has it, checking dtype and shape against the context (E = n_experts, H, I); the experts
 * go through moe_preload_layer straight from the memory-mapped shard (biases widened from bf16
 * to f32, exactly), the router through moe_preload_router; and, when the shards hold it,
 * model.layers.{layer}.post_attention_layernorm.weight (BF16 [H]) through moe_preload_norm with
 * rms_norm_eps. MOE_ERR_IO: a shard cannot be opened or its header parsed; MOE_ERR_INVALID: a
 * tensor is missing or has another dtype or shape. */
int moe_load_safetensors_layer(moe_ctx *ctx, const char *const *shard_paths, size_t n_shards, size_t layer,
                               size_t n_experts, float rms_norm_eps);
/* Header lookup (no device needed): dtype (NUL-terminated, truncated to dtype_cap), rank, the
 * first shape_cap dimensions and the tensor's byte range [begin, end) in the file. */
int moe_safetensors_find(const char *path, const char *name, char *dtype, size_t dtype_cap, uint64_t *shape,
                         size_t shape_cap, size_t *rank, uint64_t *begin, uint64_t *end);

/* ------------------------------------------------------------------ per-expert dispatch */

/* GpuMoeDispatcher::dispatch_expert_preloaded — moe_dispatch.rs:232-324.
 * output[H] = clamp(down(SwiGLU(gate_up(input))), +-65504) for one preloaded expert, with the
 * GPT-OSS activation of session.rs:101-123: gate = min(g, clamp), up = clamp(u, +-clamp),
 * (up + 1) * gate * sigmoid(1.702 gate). The unused Metal shader (moe_shader.metal:4-101)
 * computes a different activation and decodes E8M0 255 as 0; its semantics are not followed. */
int moe_dispatch_expert_preloaded(moe_ctx *ctx, const float *input, size_t layer,
                                  size_t expert_idx, float *output);

/* GpuMoeDispatcher::dispatch_expert — moe_dispatch.rs:327-469. One expert from caller-owned
 * checkpoint tensors of that expert alone (no [E] dimension). Block and scale lengths must
 * equal the expert's sizes; bias lengths may be short and are zero-padded (:352-359). */
int moe_dispatch_expert(moe_ctx *ctx, const float *input, const uint8_t *gate_up_blocks,
                        size_t gate_up_blocks_len, const uint8_t *gate_up_scales,
                        size_t gate_up_scales_len, const float *gate_up_bias,
                        size_t gate_up_bias_len, const uint8_t *down_blocks,
                        size_t down_blocks_len, const uint8_t *down_scales,
                        size_t down_scales_len, const float *down_bias, size_t down_bias_len,
                        float *output);

/* One tuple of dispatch_experts_batched (moe_dispatch.rs:476). */
typedef struct moe_expert_ref {
  size_t expert_idx; /* carried for the caller, unused (as in the reference) */
  float weight;
  const uint8_t *gate_up_blocks;
  size_t gate_up_blocks_len;
  const uint8_t *gate_up_scales;
  size_t gate_up_scales_len;
  const float *gate_up_bias;
  size_t gate_up_bias_len;
  const uint8_t *down_blocks;
  size_t down_blocks_len;
  const uint8_t *down_scales;
  size_t down_scales_len;
  const float *down_bias;
  size_t down_bias_len;
} moe_expert_ref;

/* GpuMoeDispatcher::dispatch_experts_batched — moe_dispatch.rs:473-607.
 * output[H] = sum over experts in order of weight * expert_output, where non-finite expert
 * output elements are skipped (:594-603). n = 0 gives zeros. */
int moe_dispatch_experts_batched(moe_ctx *ctx, const float *input, size_t n,
                                 const moe_expert_ref *experts, float *output);

/* ------------------------------------------------------------------ LM head */

/* GpuMoeDispatcher::init_lm_head — moe_dispatch.rs:611-621. weights [vocab, H] f32. */
int moe_init_lm_head(moe_ctx *ctx, const float *weights, size_t vocab_size);
/* The LM head from the checkpoint's BF16 lm_head.weight [vocab, H] (weights.rs:56, loaded at
 * :251) — the live path's form: ModelWeights::lm_head_dot (weights.rs:73-82, bf16 widened exactly
 * to f32, f32 accumulation) and the bf16 chunks of session.rs:425-450; half the bytes of the f32
 * form. Replaces an earlier init (f32 or bf16); dispatch_lm_head(_device) then reads these rows.
 * Needs H % 8 == 0 and H <= 3072. The _device form copies from device memory on `stream`. */
int moe_init_lm_head_bf16(moe_ctx *ctx, const uint16_t *weights_bf16, size_t vocab_size);
int moe_init_lm_head_bf16_device(moe_ctx *ctx, const uint16_t *weights_bf16, size_t vocab_size,
                                 void *stream);
/* GpuMoeDispatcher::dispatch_lm_head — moe_dispatch.rs:624-683. logits[vocab] = W input.
 * Returns MOE_ERR_STATE where the reference panics ("call init_lm_head first"). */
int moe_dispatch_lm_head(moe_ctx *ctx, const float *input, size_t vocab_size, float *logits);
/* The same with device pointers, enqueued on `stream` (NULL = the context's stream); no
 * synchronisation (no reference counterpart: the device-resident form of dispatch_lm_head).
 * After moe_init_lm_head_bf16(_device) `input` must be 16-byte aligned (MOE_ERR_INVALID
 * otherwise); the f32 head takes any 4-byte aligned input. */
int moe_dispatch_lm_head_device(moe_ctx *ctx, const float *input, size_t vocab_size, float *logits,
                                void *stream);

/* ------------------------------------------------------------------ path-level entry points */

/* Router + top-k + renormalisation for n_tokens hidden states — session.rs:818-841 with the
 * fp32 router of session.rs:495-520 evaluated in the library's canonical summation order
 * (64 strided fused partial sums + xor butterfly, then + bias). idx/weights: [n_tokens, top_k];
 * slots beyond an adaptive count hold idx -1, weight 0. logits (optional, may be NULL):
 * [n_tokens, E]. */
int moe_router_topk(moe_ctx *ctx, size_t layer, const float *x, size_t n_tokens, size_t top_k,
                    int32_t *idx, float *weights, float *logits);

/* The MoE block of Session::decode_step_inner — session.rs:818-980: router, top-k,
 * per-expert SwiGLU FFN, weighted combine in slot order. x, y: [n_tokens, H]. */
int moe_layer_forward(moe_ctx *ctx, size_t layer, const float *x, size_t n_tokens,
                      size_t top_k, float *y);
/* Same on device buffers, asynchronous on `stream`. */
int moe_layer_forward_device(moe_ctx *ctx, size_t layer, const float *x, size_t n_tokens,
                             size_t top_k, float *y, void *stream);

/* The same forward without allocating: no reference counterpart. For callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses that forbid it): the
 * per-call workspace comes from a fixed 16 MiB device array that the library holds on every GPU
 * it runs on until the process ends, so neither this call nor its first call allocates (the
 * context's other device memory is allocated by moe_create and the preload calls). Calls whose
 * workspace would exceed 16 MiB (about 110 tokens at top-4 for hidden = intermediate = 2880)
 * return MOE_ERR_INVALID; timing must be off (MOE_ERR_STATE otherwise). Every context on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two contexts, two threads)
 * race and must be serialised by the caller. Results are identical to moe_layer_forward_device. */
int moe_layer_forward_device_noalloc(moe_ctx *ctx, size_t layer, const float *x, size_t n_tokens,
                                     size_t top_k, float *y, void *stream);

/* The MoE block with the post-attention RMSNorm before it and the residual add after it: the
 * router fusion of build_decode_output_proj_router (executables.rs:260-317: router(RMSNorm(h)))
 * in the fp32 form of session.rs:483-493, and the residual add of session.rs:982-994:
 * out = x + MoE(n), n = (x * inv_rms) * gamma, inv_rms = 1 / sqrt(sum(x^2) / H + eps).
 * The sum of squares is taken in a fixed order (64 lane-strided partial sums combined by a xor
 * butterfly) rather than the reference's sequential one, so inv_rms can differ from it in the
 * last bit; the single-token one-launch kernel fuses the norm into its router and gate_up blocks
 * and the residual into its combine. Needs moe_preload_norm. x, out: [n_tokens, H]. */
int moe_block_forward(moe_ctx *ctx, size_t layer, const float *x, size_t n_tokens, size_t top_k,
                      float *out);
int moe_block_forward_device(moe_ctx *ctx, size_t layer, const float *x, size_t n_tokens,
                             size_t top_k, float *out, void *stream);

/* ------------------------------------------------------------------ MXFP4 primitives */

/* dequant_mxfp4_row / dequant_expert_{gate_up,down}_into — weights.rs:350-423, bit-exact:
 * out[r, 32b+2j] = LUT[lo] * f32_from_bits(scale << 23) (scale 0 -> +0.0, 255 -> +inf).
 * blocks [rows, cols/32, 16], scales [rows, cols/32], out [rows, cols] f32; device buffers. */
int moe_mxfp4_dequant_device(const uint8_t *blocks, const uint8_t *scales, size_t rows,
                             size_t cols, float *out, void *stream);
/* Decode of one preloaded expert matrix from its resident (repacked) copy, in the
 * reference's logical layout: which = 0 -> gate_up [2I, H] (interleaved rows as in the
 * checkpoint), 1 -> down [H, I]. out is a device buffer. Proves the resident copy lossless. */
int moe_dequant_expert_device(moe_ctx *ctx, size_t layer, size_t expert_idx, int which,
                              float *out, void *stream);
/* Bytes of the resident (repacked) form of a [rows, cols] MXFP4 matrix. */
size_t moe_mxfp4_packed_size(size_t rows, size_t cols);
/* Repack checkpoint-layout MXFP4 (device) into the resident form (device, packed_size bytes). */
int moe_mxfp4_pack_device(const uint8_t *blocks, const uint8_t *scales, size_t rows, size_t cols,
                          uint8_t *packed, void *stream);
/* y[rows] = W x for a packed MXFP4 matrix (the reference's dequant + matvec, weights.rs:350-371
 * with session.rs:75-85). x, y: device f32. One launch (MOE_OPT_MATVEC); the two-launch form
 * uses ctx scratch for the split of x. */
int moe_mxfp4_matvec_device(moe_ctx *ctx, const uint8_t *packed, size_t rows, size_t cols,
                            const float *x, float *y, void *stream);

/* ------------------------------------------------------------------ device memory helpers */
/* Thin wrappers so hosts without a HIP runtime binding (ctypes, Rust FFI) can stage data. */
int moe_device_alloc(size_t bytes, void **ptr);
int moe_device_free(void *ptr);
int moe_memcpy_h2d(void *dst, const void *src, size_t bytes);
int moe_memcpy_d2h(void *dst, const void *src, size_t bytes);
/* Device-to-device copy (the runtime's blit kernel); also the known-size copy that calibrates
 * the FETCH_SIZE / WRITE_SIZE counters in profiles. */
int moe_memcpy_d2d(void *dst, const void *src, size_t bytes);
int moe_memset_device(void *dst, int value, size_t bytes);
int moe_synchronize(moe_ctx *ctx);
/* The context's stream (a hipStream_t) for callers that enqueue their own work. */
void *moe_stream(moe_ctx *ctx);

/* Seeded synthetic fill of device memory for benchmarks (no reference counterpart): kind 0 =
 * bytes uniform in [lo, hi]; kind 1 = bf16 bits of N(0, sigma) rounded to nearest even;
 * kind 2 = f32 N(0, sigma); kind 3 = f32 of bf16-rounded N(0, sigma). n = element count. */
int moe_synth_fill_device(void *dst, size_t n, int kind, uint64_t seed, float a, float b,
                          void *stream);

/* ------------------------------------------------------------------ HIP graphs */
/* Capture of device-pointer calls on the context stream into a HIP graph, for callers whose
 * per-call GPU work is shorter than the host launch path (batch-1 decode). No reference
 * counterpart (Metal command buffers were re-encoded per call, moe_dispatch.rs:404-458).
 * Between begin and end only *_device calls with stream NULL may be issued; the context
 * workspace must already be sized by one uncaptured call of the same shape, and timing must
 * be off. The graph reads the buffers it was captured with at replay time. */
int moe_graph_begin(moe_ctx *ctx);
int moe_graph_end(moe_ctx *ctx, void **graph_exec);
int moe_graph_launch(moe_ctx *ctx, void *graph_exec);
int moe_graph_destroy(void *graph_exec);

/* ------------------------------------------------------------------ timing */
/* Per-kernel GPU time of the last device forward calls, accumulated with HIP events on the
 * stream the kernels run on when enabled (no reference counterpart). */
int moe_set_timing(moe_ctx *ctx, int enabled);
/* kernel: 0 route (on the grouped GEMM path also the activation records and, mostly, the
 * grouping by expert), 1 bucket (the separate grouping), 2 gate_up, 3 down, 4 combine,
 * 5 single-token router+gate_up, 6 single-token down+combine, 7 single-token layer in one
 * launch, 8 reserved (no kernel records it), 9 RMSNorm and residual add of moe_block_forward
 * where they are not fused.
 * Returns accumulated milliseconds
 * and launch count since the last reset; synchronises the context stream. */
int moe_get_timing(moe_ctx *ctx, int kernel, double *ms, uint64_t *launches);
int moe_reset_timing(moe_ctx *ctx);

#ifdef __cplusplus
}
#endif
#endif /* MXFP4_MOE_H */
