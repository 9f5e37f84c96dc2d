/*
 * beaver32.h — C ABI of the MI355X (gfx950) Beaver-triple generator over the 31-bit Mersenne
 * field p = 2^31 - 1: the GPU backend GpuTripleGen32 of gabearro/SilentOTITHRanDouSha
 * (src/gpu/mod.rs:511-1012, kernels src/gpu/shader32.metal:1-167). Each entry point names the
 * reference item it replaces. Status codes and moe_last_error() are shared with mxfp4_moe.h.
 *
 * Semantics (shader32.metal:75-167), per round r (spr = n - 2t triples per round, round r makes
 * triples r * spr + j, j < spr, up to `count`), with seed = round_seeds[r] and eval_p = p + 1:
 *   a0 = H(seed, 3n + 2 spr + 2j), b0 = H(seed, 3n + 2 spr + 2j + 1),
 *   ca = H(seed, 3n + 2j),         cb = H(seed, 3n + 2j + 1),          (H = chash32)
 *   a_p = a0 + ca eval_p,  b_p = b0 + cb eval_p,  c_p = a0 b0 + eval_p bt_r(r, j)   (mod p)
 * bt_r reproduces the kernel's SIMD reduction on 32-wide SIMD groups with threadgroups of
 * w = min(32, num_rounds) threads (mod.rs:989-994): for the first 8 rounds of each group of w
 * (r mod w < 8), bt_r(r, j) = sum_{i < n} him[j][i] H(round_seeds[r - (r mod w) + i], 3i) with
 * him[j][i] = (i + 1)^j, counting only rounds that exist; 0 for the other rounds. The OT
 * correlations feed only the kernel's a_mixed term, which no output uses (shader32.metal:96-108),
 * so they are accepted for the interface and not read.
 * Output layout: all-party calls write a, b, c as [n][count] (party-major, as
 * BeaverTripleBatch32); single-party calls write [count].
 */
#ifndef BEAVER32_H
#define BEAVER32_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct beaver32_ctx beaver32_ctx;

/* GpuTripleGen32::new(n, t) — gpu/mod.rs:523-634. Needs n > 2t and n <= 8 (as the reference);
 * also n - 2t <= 3: the kernel's HIM table has 3 rows (shader32.metal:41, mod.rs:606-612), and the
 * reference reads past it for more. MOE_ERR_INVALID otherwise; MOE_ERR_NO_DEVICE without gfx950. */
int beaver32_create(size_t n, size_t t, beaver32_ctx **out);
void beaver32_destroy(beaver32_ctx *ctx);
/* Triples per round (n - 2t). */
size_t beaver32_spr(const beaver32_ctx *ctx);

/* GpuTripleGen32::generate — gpu/mod.rs:636-707: every party's shares of `count` triples.
 * ot_values: n pointers to each party's ExpandedCorrelations32::random_values (>= num_rounds
 * values; may be NULL, unread); round_seeds: num_rounds = ceil(count / spr) values (the
 * reference draws them with rng.gen::<u32>(), mod.rs:646). a, b, c: [n * count] host arrays. */
int beaver32_generate(beaver32_ctx *ctx, size_t count, const uint32_t *const *ot_values,
                      const uint32_t *round_seeds, uint32_t *a, uint32_t *b, uint32_t *c);
/* GpuTripleGen32::generate_single_party — gpu/mod.rs:709-765: party `party`'s shares [count]. */
int beaver32_generate_single_party(beaver32_ctx *ctx, size_t party, size_t count,
                                   const uint32_t *const *ot_values, const uint32_t *round_seeds,
                                   uint32_t *a, uint32_t *b, uint32_t *c);
/* Device-pointer form, asynchronous on `stream` (a hipStream_t, NULL = the context's stream):
 * the zero-copy preallocated path of generate_single_party_prealloc / dispatch_kernel_only
 * (gpu/mod.rs:840-938) for party >= 0, of generate / generate_streaming (mod.rs:636-707,
 * 767-838) for party = -1 (outputs [n * count]). round_seeds: device [num_rounds]. */
int beaver32_generate_device(beaver32_ctx *ctx, long party, size_t count, const uint32_t *round_seeds,
                             uint32_t *a, uint32_t *b, uint32_t *c, void *stream);
int beaver32_synchronize(beaver32_ctx *ctx);

#ifdef __cplusplus
}
#endif
#endif /* BEAVER32_H */
