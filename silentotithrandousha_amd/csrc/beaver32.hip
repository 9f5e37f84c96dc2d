// Beaver-triple generation over p = 2^31 - 1 for gfx950 (include/beaver32.h): the GPU backend
// GpuTripleGen32 of the reference (src/gpu/mod.rs:511-1012; kernels shader32.metal:75-167).
//
// A thread produces triple j of 16 rounds 64 apart, so each pass of a wavefront stores 64
// consecutive words of each output array; a block takes 1024 whole rounds. The field products
// are exact 32 x 32 -> 64-bit multiplies folded by 2^31 = 1 (mod p), those by the parties'
// evaluation points 1..8 sums of 31-bit rotations; every value is kept in [0, p).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/beaver32.h"
#include "../../include/mxfp4_moe.h"

namespace moe {
int api_fail(int code, const char *msg);
}

namespace {

constexpr uint32_t kP = 0x7FFFFFFFu;

__host__ __device__ __forceinline__ uint32_t fmul(uint32_t a, uint32_t b) {
  const uint64_t x = (uint64_t)a * b;
  uint32_t r = (uint32_t)(x & kP) + (uint32_t)(x >> 31);
  r = (r >> 31) + (r & kP);
  return r >= kP ? r - kP : r;
}

__host__ __device__ __forceinline__ uint32_t fadd(uint32_t a, uint32_t b) {
  const uint32_t r = a + b;
  return r >= kP ? r - kP : r;
}

// The kernel's integer hash of (seed, index) into [0, p) (shader32.metal:26-33).
__host__ __device__ __forceinline__ uint32_t chash32(uint32_t seed, uint32_t idx) {
  uint32_t x = seed ^ (idx * 0x9e3779b9u);
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  x &= 0x7FFFFFFFu;
  return x >= kP ? x - kP : x;
}

struct TripleArgs {
  const uint32_t *seeds;
  uint32_t *a, *b, *c;
  uint32_t n, count, num_rounds, group;  // group: the reference's threadgroup width (<= 32)
  int party;                             // >= 0: that party's shares; -1: every party
  uint32_t him[3][8];                    // (i + 1)^j
  uint32_t eval[8];                      // i + 1
  uint32_t hmul[3][4];                   // idx * 0x9e3779b9 of the hashes of triple j: a0 b0 ca cb
};

__device__ __forceinline__ uint32_t chash32_m(uint32_t seed, uint32_t idx_mul) {  // idx pre-multiplied
  uint32_t x = seed ^ idx_mul;
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  x &= 0x7FFFFFFFu;
  return x >= kP ? x - kP : x;
}

// c * 2^k mod p for c in [0, p), k in [0, 30]: 2^31 = 1 (mod p), so the product is c rotated
// left by k within 31 bits (a 31-bit pattern other than all ones stays below p).
__device__ __forceinline__ uint32_t frot(uint32_t c, uint32_t k) {
  return k ? ((c << k) | (c >> (31u - k))) & kP : c;
}

// c * x mod p for a small wavefront-uniform x (the parties' evaluation points 1..8): a sum of
// rotations by the set bits of x, each a field value, instead of a 32 x 32 -> 64-bit product
// (two quarter-rate multiplies). Equal to fmul(c, x) for every c in [0, p).
__device__ __forceinline__ uint32_t fmul_small(uint32_t c, uint32_t x) {
  uint32_t r = (x & 1u) ? c : 0u;
  if (x & 2u) r = fadd(r, frot(c, 1));
  if (x & 4u) r = fadd(r, frot(c, 2));
  if (x & 8u) r = fadd(r, frot(c, 3));
  return r;
}

// A block takes kRounds = 64 kIter consecutive rounds: thread (kl, j) of its 64 SPR threads
// produces triple j of rounds R0 + kl + 64 m, m = 0 .. kIter - 1, so each pass of a wavefront
// stores 64 consecutive words of each output array. bt_r is the SIMD-group reduction of the
// reference kernel: lanes i < n of a threadgroup of `group` rounds hold H(seed of round
// r0 + i, 3i), and the reduction over 8 lanes (xor 1, 2, 4) gives the first 8 rounds of the
// threadgroup sum_i him[j][i] H(...) and every other round 0 (its lanes are inactive, weight
// 0); rounds past num_rounds add nothing. The block's threadgroups (at most kRounds / group + 1
// of them) get their hashes and sums once, in LDS, before the passes.
constexpr uint32_t kIter = 16;
constexpr uint32_t kRounds = 64 * kIter;
constexpr uint32_t kMaxGroups = kRounds / 32 + 1;  // threadgroups of 32 rounds a block overlaps

template <int SPR>
__global__ __launch_bounds__(64 * SPR) void k_beaver32(TripleArgs a) {
  __shared__ uint32_t s_rt[kMaxGroups][8];
  __shared__ uint32_t s_bt[kMaxGroups][SPR];
  const uint32_t R0 = blockIdx.x * kRounds, tid = threadIdx.x;
  // group < 32 only when num_rounds < 32: a single block, whose rounds lie in group 0
  const uint32_t g0 = a.group == 32u ? R0 / 32u : 0u;  // first threadgroup overlapping the block
  const uint32_t ng = a.group == 32u ? kMaxGroups : 1u;
  for (uint32_t u = tid; u < ng * 8u; u += 64u * SPR) {  // hashes of each group's first n rounds
    const uint32_t gi = u / 8u, i = u % 8u, r = (g0 + gi) * a.group + i;
    s_rt[gi][i] = i < a.n && r < a.num_rounds && i < a.group ? chash32(a.seeds[r], 3u * i) : 0u;
  }
  __syncthreads();
  for (uint32_t u = tid; u < ng * SPR; u += 64u * SPR) {
    const uint32_t gi = u / SPR, j = u % SPR;
    uint32_t acc = 0u;
    for (uint32_t i = 0; i < a.n; i++) acc = fadd(acc, fmul(a.him[j][i], s_rt[gi][i]));
    s_bt[gi][j] = acc;
  }
  __syncthreads();
  const uint32_t kl = tid / SPR, j = tid - kl * SPR;  // round within a pass, triple within it
  const uint32_t h0 = a.hmul[j][0], h1 = a.hmul[j][1], h2 = a.hmul[j][2], h3 = a.hmul[j][3];
  // every round's seed in flight at once (loaded pass by pass, each pass waited for its load)
  uint32_t seedv[kIter];
#pragma unroll
  for (uint32_t m = 0; m < kIter; m++) {
    const uint32_t r = R0 + 64u * m + kl;
    seedv[m] = r < a.num_rounds ? a.seeds[r] : 0u;
  }
#pragma unroll
  for (uint32_t m = 0; m < kIter; m++) {
    const uint32_t r = R0 + 64u * m + kl, k = r * SPR + j;
    if (k >= a.count) return;  // rounds increase with m
    const uint32_t seed = seedv[m];
    const uint32_t a0 = chash32_m(seed, h0), b0 = chash32_m(seed, h1);
    const uint32_t ca = chash32_m(seed, h2), cb = chash32_m(seed, h3);
    // lane r % group of threadgroup r / group (group = 32, or the one group of a short call)
    const uint32_t lane = a.group == 32u ? (r & 31u) : r;
    const uint32_t bt = lane < 8u ? s_bt[a.group == 32u ? (r >> 5) - g0 : 0u][j] : 0u;
    const uint32_t ab = fmul(a0, b0);
    if (a.party >= 0) {
      const uint32_t x = a.eval[a.party];
      // streaming stores: the outputs are written once and not read back by this kernel
      __builtin_nontemporal_store(fadd(a0, fmul_small(ca, x)), a.a + k);
      __builtin_nontemporal_store(fadd(b0, fmul_small(cb, x)), a.b + k);
      __builtin_nontemporal_store(fadd(ab, fmul_small(bt, x)), a.c + k);
    } else {
      for (uint32_t p = 0; p < a.n; p++) {
        const uint32_t x = a.eval[p];
        const size_t o = (size_t)p * a.count + k;
        __builtin_nontemporal_store(fadd(a0, fmul_small(ca, x)), a.a + o);
        __builtin_nontemporal_store(fadd(b0, fmul_small(cb, x)), a.b + o);
        __builtin_nontemporal_store(fadd(ab, fmul_small(bt, x)), a.c + o);
      }
    }
  }
}

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return moe::api_fail(code, buf);
}

#define BV_HIP(call)                                                                          \
  do {                                                                                        \
    hipError_t e_ = (call);                                                                   \
    if (e_ != hipSuccess)                                                                     \
      return fail(e_ == hipErrorOutOfMemory ? MOE_ERR_OOM : MOE_ERR_HIP, "%s: %s", #call,     \
                  hipGetErrorString(e_));                                                     \
  } while (0)

}  // namespace

struct beaver32_ctx {
  int dev = 0;
  hipStream_t stream = nullptr;
  uint32_t n = 0, t = 0, spr = 0;
  uint32_t him[3][8] = {};
  uint32_t eval[8] = {};
  void *buf = nullptr;  // staging for the host-pointer calls: seeds + a, b, c
  size_t cap = 0;
};

namespace {

uint32_t fpow(uint32_t b, uint32_t e) {
  uint32_t r = 1u;
  for (uint32_t i = 0; i < e; i++) r = fmul(r, b);
  return r;
}

int check_count(const beaver32_ctx *c, size_t count) {
  if (count > 0xFFFFFFFFull / 8) return fail(MOE_ERR_INVALID, "count %zu too large", count);
  (void)c;
  return MOE_OK;
}

int launch(beaver32_ctx *c, long party, size_t count, const uint32_t *seeds, uint32_t *a, uint32_t *b,
           uint32_t *cc, hipStream_t s) {
  if (!count) return MOE_OK;
  if (party >= (long)c->n || party < -1) return fail(MOE_ERR_INVALID, "party %ld outside [-1, %u)", party, c->n);
  if (!seeds || !a || !b || !cc) return fail(MOE_ERR_INVALID, "null argument");
  if (int r = check_count(c, count)) return r;
  TripleArgs ta{};
  ta.seeds = seeds;
  ta.a = a;
  ta.b = b;
  ta.c = cc;
  ta.n = c->n;
  ta.count = (uint32_t)count;
  ta.num_rounds = (uint32_t)((count + c->spr - 1) / c->spr);
  ta.group = ta.num_rounds < 32u ? ta.num_rounds : 32u;  // min(thread_execution_width, rounds)
  ta.party = (int)party;
  std::memcpy(ta.him, c->him, sizeof(ta.him));
  std::memcpy(ta.eval, c->eval, sizeof(ta.eval));
  for (uint32_t j = 0; j < c->spr; j++) {  // hash indices of triple j (shader32.metal:104-107)
    const uint32_t base = 3u * c->n + 2u * j;
    ta.hmul[j][0] = (base + 2u * c->spr) * 0x9e3779b9u;
    ta.hmul[j][1] = (base + 2u * c->spr + 1u) * 0x9e3779b9u;
    ta.hmul[j][2] = base * 0x9e3779b9u;
    ta.hmul[j][3] = (base + 1u) * 0x9e3779b9u;
  }
  const dim3 grid((unsigned)((ta.num_rounds + kRounds - 1) / kRounds));
  switch (c->spr) {
    case 1: hipLaunchKernelGGL(k_beaver32<1>, grid, dim3(64), 0, s, ta); break;
    case 2: hipLaunchKernelGGL(k_beaver32<2>, grid, dim3(128), 0, s, ta); break;
    default: hipLaunchKernelGGL(k_beaver32<3>, grid, dim3(192), 0, s, ta); break;
  }
  BV_HIP(hipGetLastError());
  return MOE_OK;
}

int host_call(beaver32_ctx *c, long party, size_t count, const uint32_t *round_seeds, uint32_t *a,
              uint32_t *b, uint32_t *cc) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  if (!count) return MOE_OK;
  if (!round_seeds || !a || !b || !cc) return fail(MOE_ERR_INVALID, "null argument");
  if (int r = check_count(c, count)) return r;
  BV_HIP(hipSetDevice(c->dev));
  const size_t rounds = (count + c->spr - 1) / c->spr;
  const size_t outs = (party < 0 ? c->n : 1) * count;
  const size_t o_seed = 0, o_a = (rounds * 4 + 255) / 256 * 256, o_b = o_a + (outs * 4 + 255) / 256 * 256,
               o_c = o_b + (outs * 4 + 255) / 256 * 256, total = o_c + outs * 4;
  if (total > c->cap) {  // the new buffer first, so a failure leaves the old one in place
    void *q = nullptr;
    BV_HIP(hipMalloc(&q, total));
    if (c->buf) (void)hipFree(c->buf);
    c->buf = q;
    c->cap = total;
  }
  char *d = (char *)c->buf;
  BV_HIP(hipMemcpyAsync(d + o_seed, round_seeds, rounds * 4, hipMemcpyHostToDevice, c->stream));
  if (int r = launch(c, party, count, (const uint32_t *)(d + o_seed), (uint32_t *)(d + o_a),
                     (uint32_t *)(d + o_b), (uint32_t *)(d + o_c), c->stream))
    return r;
  BV_HIP(hipMemcpyAsync(a, d + o_a, outs * 4, hipMemcpyDeviceToHost, c->stream));
  BV_HIP(hipMemcpyAsync(b, d + o_b, outs * 4, hipMemcpyDeviceToHost, c->stream));
  BV_HIP(hipMemcpyAsync(cc, d + o_c, outs * 4, hipMemcpyDeviceToHost, c->stream));
  BV_HIP(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

}  // namespace

extern "C" {

int beaver32_create(size_t n, size_t t, beaver32_ctx **out) {
  if (!out) return fail(MOE_ERR_INVALID, "null out");
  *out = nullptr;
  if (n <= 2 * t) return fail(MOE_ERR_INVALID, "need n > 2t, got n=%zu, t=%zu", n, t);
  if (n > 8) return fail(MOE_ERR_INVALID, "GPU kernel supports n <= 8, got %zu", n);
  if (n - 2 * t > 3)
    return fail(MOE_ERR_INVALID, "n - 2t = %zu triples per round: the kernel's HIM table holds 3 rows", n - 2 * t);
  int nd = 0;
  if (hipGetDeviceCount(&nd) != hipSuccess || nd < 1) return fail(MOE_ERR_NO_DEVICE, "no HIP device");
  int dev = 0;
  BV_HIP(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  BV_HIP(hipGetDeviceProperties(&prop, dev));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MOE_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950", dev, prop.gcnArchName);
  beaver32_ctx *c = new beaver32_ctx();
  c->dev = dev;
  c->n = (uint32_t)n;
  c->t = (uint32_t)t;
  c->spr = (uint32_t)(n - 2 * t);
  for (uint32_t i = 0; i < c->n; i++) c->eval[i] = i + 1;  // Fp32::new(i + 1).raw()
  for (uint32_t j = 0; j < c->spr; j++)
    for (uint32_t i = 0; i < c->n; i++) c->him[j][i] = fpow(i + 1, j);  // alpha_{i+1}^j
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return fail(MOE_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  *out = c;
  return MOE_OK;
}

void beaver32_destroy(beaver32_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->dev);
  (void)hipStreamSynchronize(c->stream);
  if (c->buf) (void)hipFree(c->buf);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

size_t beaver32_spr(const beaver32_ctx *c) { return c ? c->spr : 0; }

int beaver32_generate(beaver32_ctx *c, size_t count, const uint32_t *const *ot_values,
                      const uint32_t *round_seeds, uint32_t *a, uint32_t *b, uint32_t *cc) {
  (void)ot_values;
  return host_call(c, -1, count, round_seeds, a, b, cc);
}

int beaver32_generate_single_party(beaver32_ctx *c, size_t party, size_t count,
                                   const uint32_t *const *ot_values, const uint32_t *round_seeds,
                                   uint32_t *a, uint32_t *b, uint32_t *cc) {
  (void)ot_values;
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  if (party >= c->n) return fail(MOE_ERR_INVALID, "party %zu >= n %u", party, c->n);
  return host_call(c, (long)party, count, round_seeds, a, b, cc);
}

int beaver32_generate_device(beaver32_ctx *c, long party, size_t count, const uint32_t *round_seeds,
                             uint32_t *a, uint32_t *b, uint32_t *cc, void *stream) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  BV_HIP(hipSetDevice(c->dev));
  return launch(c, party, count, round_seeds, a, b, cc, stream ? (hipStream_t)stream : c->stream);
}

int beaver32_synchronize(beaver32_ctx *c) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  BV_HIP(hipSetDevice(c->dev));
  BV_HIP(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

}  // extern "C"
