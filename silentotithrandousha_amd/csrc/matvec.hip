// One MXFP4 matvec y = W x in one launch (the matvec of session.rs:16-85, here on the resident
// tile16 layout): one block per 16-row tile, whose kMvWaves wavefronts split K (wavefront w
// takes steps [kMvSteps w, kMvSteps (w + 1)), 4 MXFP4 blocks per step). Each wavefront issues
// its weight loads first;
// while they are in flight the block splits x into the 4-term fp8 activation record in LDS
// (split8_fp8); then every wavefront runs the block-scaled MFMA over its steps and the partial
// sums are added in wavefront order.
#include "device.hpp"
#include "kernels.hpp"

namespace moe {
namespace {

constexpr int kMvWaves = 8;
constexpr int kMvNs = 24;                    // steps per tile: K <= 3072
constexpr int kMvSteps = kMvNs / kMvWaves;   // steps per wavefront
using MvAct = ActRecord<kMvNs>;
static_assert(kMvNs % kMvWaves == 0, "whole step ranges");

// The MFMA sweep of wavefront wv's step range, with the range as a template constant (so every
// scale word index is static).
template <int W>
__device__ __forceinline__ f32x4 mv_steps(int wv, const uint4 (&raw)[kMvSteps], const uint32_t *sw,
                                          const uint8_t *s_x, const uint32_t *bsw, int lane) {
  if constexpr (W + 1 == kMvWaves) {
    return tile_mfma_f8_steps<kMvNs, kMvSteps, W * kMvSteps>(raw, sw, s_x, bsw, lane);
  } else {
    if (wv == W) return tile_mfma_f8_steps<kMvNs, kMvSteps, W * kMvSteps>(raw, sw, s_x, bsw, lane);
    return mv_steps<W + 1>(wv, raw, sw, s_x, bsw, lane);
  }
}

__global__ __launch_bounds__(64 * kMvWaves) void k_matvec_fp4(const uint8_t *mat, PackDims d,
                                                              const float *x, float *y) {
  __shared__ __align__(16) uint8_t s_x[MvAct::kBytes];
  __shared__ float s_p[kMvWaves][16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, j = lane & 15;
  const int t = blockIdx.x;
  const int ns = (int)d.ns, nb = (int)d.nb, K = 32 * nb;
  // 1. the wavefront's weight chunks (zeros past the tile) and the tile's scale words
  const uint4 *wp = reinterpret_cast<const uint4 *>(mat) + (size_t)t * 16 * nb;
  const uint32_t *sp = reinterpret_cast<const uint32_t *>(mat + pack_weight_bytes(d)) + (size_t)t * d.nq * 64;
  uint4 raw[kMvSteps];
#pragma unroll
  for (int k = 0; k < kMvSteps; k++) {
    const int st = kMvSteps * wv + k;
    raw[k] = make_uint4(0u, 0u, 0u, 0u);
    if (st < ns && 4 * st + g < nb) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wp) + st * 64 + lane);
      raw[k] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
  uint32_t sw[kMvNs / 4];
#pragma unroll
  for (int q = 0; q < kMvNs / 4; q++) sw[q] = q < (int)d.nq ? sp[q * 64 + lane] : 0u;
  // 2. x as kTerms fp8 terms, 8 values per thread (a quad of lanes = one 32-value block; the
  //    trip count is uniform per quad); blocks past K are zeros
  for (int u = tid; u < 16 * kMvNs; u += 64 * kMvWaves) {
    float xv[8];
    if (8 * u < K) {
      const float4 v0 = reinterpret_cast<const float4 *>(x)[2 * u];
      const float4 v1 = reinterpret_cast<const float4 *>(x)[2 * u + 1];
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
    for (int te = 0; te < kTerms; te++) *reinterpret_cast<uint2 *>(s_x + MvAct::term(te, bb) + 8 * (u & 3)) = q[te];
    if ((u & 3) == 0) {
#pragma unroll
      for (int te = 0; te < kTerms; te++) s_x[MvAct::scale(te, bb)] = (uint8_t)(s4 >> (8 * te));
    }
  }
  __syncthreads();
  // 3. the wavefront's steps on the block-scaled MFMA, the 4 term columns summed
  uint32_t bsw[kMvNs / 4];
  load_bsw<kMvNs>(s_x, bsw, lane);
  const f32x4 acc = mv_steps<0>(wv, raw, sw, s_x, bsw, lane);
  float v[4];
  sum_terms(acc, v);
  if (j == 0) *reinterpret_cast<float4 *>(&s_p[wv][4 * g]) = make_float4(v[0], v[1], v[2], v[3]);
  __syncthreads();
  // 4. the partial sums in wavefront order
  if (tid < 16) {
    float sum = s_p[0][tid];
#pragma unroll
    for (int w = 1; w < kMvWaves; w++) sum = sum + s_p[w][tid];
    y[(size_t)t * 16 + tid] = canon_nan(sum);
  }
}

}  // namespace

bool matvec_fp4_supported(size_t rows, size_t cols, const float *x) {
  return rows % 16 == 0 && cols % 32 == 0 && cols <= (size_t)32 * 4 * kMvNs &&
         reinterpret_cast<uintptr_t>(x) % 16 == 0;
}

hipError_t launch_matvec_fp4(const uint8_t *packed, size_t rows, size_t cols, const float *x,
                             float *y, hipStream_t s) {
  if (!matvec_fp4_supported(rows, cols, x) || rows == 0) return hipErrorInvalidValue;
  const PackDims d = pack_dims(rows, cols);
  hipLaunchKernelGGL(k_matvec_fp4, dim3((unsigned)d.tiles), dim3(64 * kMvWaves), 0, s, packed, d, x, y);
  return hipGetLastError();
}

}  // namespace moe
