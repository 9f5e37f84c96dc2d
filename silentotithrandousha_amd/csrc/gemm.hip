// Grouped expert GEMM for batched decode and prefill (the per-expert FFN of session.rs:87-124
// applied to every (token, slot) entry routed to an expert, session.rs:943-972) on the
// block-scaled MFMA v_mfma_scale_f32_16x16x128_f8f6f4: A = the expert's MXFP4 weights as
// stored (E2M1 nibbles + E8M0 scales, resident tile16 layout), B = the activations of the
// expert's entries as kTerms fp8 terms (split8_fp8), f32 accumulation.
//
//   k_split_rows   f32 rows (x) -> step-major activation records
//   k_gemm_fp8     one block = 512 weight rows x 64 entries of one expert; each wavefront owns
//                  128 rows (8 tiles of 16) x the 64 entries (4 column groups) x kGemmTerms
//                  activation terms.
//                  Per K-step of 128: the B records of the 64 entries go through registers
//                  into a double-buffered LDS area; A tiles load straight into registers.
//                  GATE_UP epilogue: bias, SwiGLU (gate = row 2i, up = row 2i+1) and the split
//                  of the wavefront's 32 h values per entry into the h records; DOWN epilogue:
//                  bias and +-65504 clamp into f32 [entry][H].
#include <algorithm>

#include "device.hpp"
#include "kernels.hpp"

namespace moe {

using G = GemmRec;  // step-major activation record (kernels.hpp)

// Quad of lanes 16 apart (lane, lane+16, lane+32, lane+48) holding one 32-value block: the
// split of split8_fp8 with the block reductions across lane bits 4 and 5.
__device__ __forceinline__ void split8_fp8_cols(const float x[8], uint2 q[kTerms], uint32_t &s4) {
  float m = 0.0f, bad = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    m = fmaxf(m, fabsf(x[i]));
    if (!isfinite(x[i])) bad = 1.0f;
  }
  m = fmaxf(m, xor_lane<16>(m));
  m = fmaxf(m, xor_lane<32>(m));
  bad = fmaxf(bad, xor_lane<16>(bad));
  bad = fmaxf(bad, xor_lane<32>(bad));
  split8_fp8_with_max(x, m, bad != 0.0f, q, s4);
}

// ------------------------------------------------------------------ activation records

// grid (ceil(4 ns / 64), rows), 256 threads: thread quad q of block x handles 32-block
// b = 64 x + q of row `row` (values past K are zeros, blocks up to 4 * kGemmNs written).
__global__ __launch_bounds__(256) void k_split_rows(const float *src, int K, uint8_t *rec) {
  const int row = blockIdx.y, tid = threadIdx.x;
  const int b = blockIdx.x * 64 + (tid >> 2), part = tid & 3;
  if (blockIdx.x * 64 >= 4 * kGemmNs) return;
  float v[8];
  const int k0 = 32 * b + 8 * part;
  if (b < 4 * kGemmNs && k0 < K) {
    const float4 a0 = *reinterpret_cast<const float4 *>(src + (size_t)row * K + k0);
    const float4 a1 = *reinterpret_cast<const float4 *>(src + (size_t)row * K + k0 + 4);
    v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
    v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.0f;
  }
  uint2 q[kTerms];
  uint32_t s4;
  split8_fp8(v, q, s4);
  if (b >= 4 * kGemmNs) return;
  uint8_t *r = rec + (size_t)row * G::kBytes;
  const int s = b >> 2, i = b & 3;
#pragma unroll
  for (int t = 0; t < kTerms; t++) *reinterpret_cast<uint2 *>(r + G::data(s, t) + 32 * i + 8 * part) = q[t];
  if (part == 0) {
#pragma unroll
    for (int t = 0; t < kTerms; t++) r[G::scale(s, t) + i] = (uint8_t)(s4 >> (8 * t));
  }
}

hipError_t launch_split_rows(const float *src, size_t rows, size_t K, uint8_t *rec, hipStream_t s) {
  if (K % 8 || K > (size_t)kGemmNs * 128) return hipErrorInvalidValue;
  if (!rows) return hipSuccess;
  hipLaunchKernelGGL(k_split_rows, dim3((4 * kGemmNs + 63) / 64, (unsigned)rows), dim3(256), 0, s, src,
                     (int)K, rec);
  return hipGetLastError();
}

// ------------------------------------------------------------------ grouped GEMM

constexpr int kGemmThreads = 256;
constexpr int kGemmRT = 8;                       // 16-row tiles per wavefront
constexpr int kGemmRowsPerWave = 16 * kGemmRT;
constexpr int kGemmRows = 4 * kGemmRowsPerWave;  // weight rows per block
constexpr int kGemmCols = 64;                    // entries per block
// The batch path multiplies by the first kGemmTerms terms of the records (3 of 4: the
// activation is then exact to 2^-12 of each value, well inside the 1e-3 tolerance; the fourth
// term would add a third more MFMA work and LDS traffic for precision no caller needs).
constexpr int kGemmTerms = 3;
constexpr int kEntryStep = kGemmTerms * 128 + 16;   // LDS bytes of one entry's K-step
constexpr int kBufBytes = kGemmCols * kEntryStep;   // one K-step of B for 64 entries
static_assert(G::kStep == kTerms * 128 + 16, "a K-step of a record = term data + 16 scale bytes");
static_assert(kEntryStep % 64 == 16, "entry stride: 16-byte aligned, spreads over the LDS banks");
constexpr int kChunks = kEntryStep / 16;            // 16-byte chunks per entry K-step (25)
constexpr int kChunksPerThread = (kChunks + 3) / 4;  // 4 threads per entry

// MFMAs of one K-step for a wavefront: 4 row tiles x 4 column groups x kTerms terms; OP = the
// step's A-scale byte (s % 4).
template <int OP>
__device__ __forceinline__ void gemm_step(f32x4 (&acc)[kGemmRT][4], const uint4 (&ar)[kGemmRT],
                                          const uint32_t (&sw)[kGemmRT], const uint8_t *cur, int j, int g) {
#pragma unroll
  for (int c = 0; c < 4; c++) {
    __builtin_amdgcn_sched_barrier(0);  // one column group's B operands live at a time
    const uint8_t *eb = cur + (16 * c + j) * kEntryStep;
#pragma unroll
    for (int t = 0; t < kGemmTerms; t++) {
      const uint4 b0 = *reinterpret_cast<const uint4 *>(eb + t * 128 + 32 * (g >> 1) + 16 * (g & 1));
      const uint4 b1 = *reinterpret_cast<const uint4 *>(eb + t * 128 + 64 + 32 * (g >> 1) + 16 * (g & 1));
      const uint32_t bs = *reinterpret_cast<const uint32_t *>(eb + kGemmTerms * 128 + 4 * t) >> (8 * g);
      const i32x8 B = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
#pragma unroll
      for (int r = 0; r < kGemmRT; r++) {
        const i32x8 A = {(int)ar[r].x, (int)ar[r].y, (int)ar[r].z, (int)ar[r].w, 0, 0, 0, 0};
        acc[r][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[r][c], 4, 0, OP, (int)sw[r], 0, (int)bs);
      }
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_gemm_fp8(GemmArgs a) {
  extern __shared__ uint4 smem[];
  __shared__ int s_tile[4];  // expert record index, first entry, entry count, row block
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int j = lane & 15, g = lane >> 4;

  // ---- tile: global column tile cl (over the experts' 64-entry tiles) and row block, row
  //      blocks fastest, so neighbouring blocks share the entries' activation records
  if (tid == 0) {
    int cl = (int)blockIdx.x / a.n_row_blocks;
    const int rb = (int)blockIdx.x - cl * a.n_row_blocks;
    const int na = min(*a.n_active, a.max_active);
    int ex = -1, beg = 0, cnt = 0;
    for (int ai = 0; ai < na; ai++) {
      const int o0 = a.active_off[ai], o1 = a.active_off[ai + 1];
      const int nct = (o1 - o0 + kGemmCols - 1) / kGemmCols;
      if (cl < nct) {
        ex = a.active_ids[ai];
        beg = o0 + cl * kGemmCols;
        cnt = min(kGemmCols, o1 - beg);
        break;
      }
      cl -= nct;
    }
    s_tile[0] = ex;
    s_tile[1] = beg;
    s_tile[2] = cnt;
    s_tile[3] = rb;
  }
  __syncthreads();
  const int ex = s_tile[0], beg = s_tile[1], ncol = s_tile[2];
  if (ex < 0) return;
  const int rblk = s_tile[3];
  const int t0 = (rblk * kGemmRows + wv * kGemmRowsPerWave) / 16;  // first 16-row tile of wave
  const uint8_t *rec = a.base + (size_t)ex * a.stride;
  const uint8_t *mat = rec + a.mat_off;
  const PackDims d = a.d;

  // ---- B: thread (entry e = tid / 4, part p = tid % 4) moves 16-byte chunks p, p+4, ... of
  //      the entry's K-step as it sits in LDS: the first kGemmTerms terms' bytes, then the 16
  //      scale bytes; padding columns repeat a valid entry
  uint8_t *const buf0 = reinterpret_cast<uint8_t *>(smem);
  uint8_t *const buf1 = buf0 + kBufBytes;
  const int be = tid >> 2, bp = tid & 3;
  const uint8_t *bsrc;
  {
    const int ge = beg + min(be, ncol - 1);
    const int row = a.entry_src ? a.entry_src[ge] : ge;
    bsrc = a.brec + (size_t)row * G::kBytes;
  }
  uint4 bst[kChunksPerThread];
  auto load_b = [&](int s) {
    const uint8_t *p = bsrc + (size_t)s * G::kStep;
#pragma unroll
    for (int k = 0; k < kChunksPerThread; k++) {
      const int ch = bp + 4 * k;  // chunk of the LDS entry step; the last one is the scales
      const int off = ch < kChunks - 1 ? 16 * ch : kTerms * 128;
      if (ch < kChunks) bst[k] = *reinterpret_cast<const uint4 *>(p + off);
    }
  };
  auto store_b = [&](uint8_t *bf) {
    uint8_t *q = bf + be * kEntryStep;
#pragma unroll
    for (int k = 0; k < kChunksPerThread; k++) {
      const int ch = bp + 4 * k;
      if (ch < kChunks) *reinterpret_cast<uint4 *>(q + 16 * ch) = bst[k];
    }
  };

  // ---- A: kGemmRT tiles of 16 rows, one 16-byte chunk per lane per step (zeros past the matrix)
  const uint4 *wp = reinterpret_cast<const uint4 *>(mat);
  const uint32_t *sp = reinterpret_cast<const uint32_t *>(mat + pack_weight_bytes(d));
  bool tv[kGemmRT];
#pragma unroll
  for (int r = 0; r < kGemmRT; r++) tv[r] = t0 + r < (int)d.tiles;
  auto load_a = [&](int s, uint4 (&ar)[kGemmRT]) {
#pragma unroll
    for (int r = 0; r < kGemmRT; r++) {
      const bool v = tv[r] && s < (int)d.ns && 4 * s + g < (int)d.nb;
      const uint4 x = wp[v ? ((size_t)(t0 + r) * 16 * d.nb) + s * 64 + lane : 0];
      ar[r] = v ? x : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto load_as = [&](int q, uint32_t (&sw)[kGemmRT]) {
#pragma unroll
    for (int r = 0; r < kGemmRT; r++) {
      const bool v = tv[r] && q < (int)d.nq;
      const uint32_t x = sp[v ? ((size_t)(t0 + r) * d.nq + q) * 64 + lane : 0];
      sw[r] = v ? x : 0u;
    }
  };

  f32x4 acc[kGemmRT][4];
#pragma unroll
  for (int r = 0; r < kGemmRT; r++)
#pragma unroll
    for (int c = 0; c < 4; c++) acc[r][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- K loop: step s computes from LDS buffer s % 2 and registers while the loads of step
  //      s + 1 (B into staging registers, A into the next register set) are in flight
  const int ns = (int)d.ns;
  uint4 a_cur[kGemmRT], a_nxt[kGemmRT];
  uint32_t sw[kGemmRT];
  load_b(0);
  load_a(0, a_cur);
  load_as(0, sw);
  store_b(buf0);
  __syncthreads();
  for (int s = 0; s < ns; s++) {
    const bool more = s + 1 < ns;
    if (more) {
      load_b(s + 1);
      load_a(s + 1, a_nxt);
    }
    const uint8_t *cur = (s & 1) ? buf1 : buf0;
    switch (s & 3) {
      case 0: gemm_step<0>(acc, a_cur, sw, cur, j, g); break;
      case 1: gemm_step<1>(acc, a_cur, sw, cur, j, g); break;
      case 2: gemm_step<2>(acc, a_cur, sw, cur, j, g); break;
      default: gemm_step<3>(acc, a_cur, sw, cur, j, g); break;
    }
    if (more) {
      store_b((s & 1) ? buf0 : buf1);
#pragma unroll
      for (int r = 0; r < kGemmRT; r++) a_cur[r] = a_nxt[r];
      if ((s & 3) == 3) load_as((s + 1) / 4, sw);
    }
    __syncthreads();  // buffer (s+1)%2 is complete and buffer s%2 is free
  }

  // ---- epilogue
  const float *bias = reinterpret_cast<const float *>(rec + a.bias_off);
  if (MODE == GEMV_GATE_UP) {
    // every 4 row tiles (64 rows) of the wavefront = h block W (h values 32 W .. 32 W + 31)
    uint8_t *hout = reinterpret_cast<uint8_t *>(a.out);
#pragma unroll
    for (int hbk = 0; hbk < kGemmRT / 4; hbk++) {
      if (!tv[4 * hbk]) break;  // the matrix has whole h blocks (rows % 64 == 0)
      const int W = t0 / 4 + hbk;
      float4 bv[4];
#pragma unroll
      for (int r = 0; r < 4; r++) bv[r] = reinterpret_cast<const float4 *>(bias)[(t0 + 4 * hbk + r) * 4 + g];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        float hv[8];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const f32x4 &av = acc[4 * hbk + r][c];
          hv[2 * r] = swiglu(av[0] + bv[r].x, av[1] + bv[r].y, a.limit);
          hv[2 * r + 1] = swiglu(av[2] + bv[r].z, av[3] + bv[r].w, a.limit);
        }
        uint2 q[kTerms];
        uint32_t s4;
        split8_fp8_cols(hv, q, s4);
        const int e = 16 * c + j;
        if (e < ncol) {
          uint8_t *hr = hout + (size_t)(beg + e) * G::kBytes;
          const int s = W >> 2, i = W & 3;
#pragma unroll
          for (int t = 0; t < kTerms; t++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {  // h 8r + 2g, 8r + 2g + 1 of the block = bytes 2r, 2r+1
              const uint32_t w = r < 2 ? q[t].x : q[t].y;
              *reinterpret_cast<uint16_t *>(hr + G::data(s, t) + 32 * i + 8 * r + 2 * g) = (uint16_t)(w >> (16 * (r & 1)));
            }
            if (g == 0) hr[G::scale(s, t) + i] = (uint8_t)(s4 >> (8 * t));
          }
        }
      }
    }
  } else {
    float *out = reinterpret_cast<float *>(a.out);
    const int R = (int)d.rows;
#pragma unroll
    for (int r = 0; r < kGemmRT; r++) {
      if (!tv[r]) continue;
      const float4 b4 = reinterpret_cast<const float4 *>(bias)[(t0 + r) * 4 + g];
      const int row = (t0 + r) * 16 + 4 * g;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int e = 16 * c + j;
        if (e >= ncol) continue;
        float4 o;
        o.x = canon_nan(rclamp(acc[r][c][0] + b4.x, -65504.0f, 65504.0f));
        o.y = canon_nan(rclamp(acc[r][c][1] + b4.y, -65504.0f, 65504.0f));
        o.z = canon_nan(rclamp(acc[r][c][2] + b4.z, -65504.0f, 65504.0f));
        o.w = canon_nan(rclamp(acc[r][c][3] + b4.w, -65504.0f, 65504.0f));
        *reinterpret_cast<float4 *>(out + (size_t)(beg + e) * R + row) = o;
      }
    }
  }
}

size_t gemm_lds_bytes() { return (size_t)2 * kBufBytes; }

hipError_t launch_gemm_fp8(GemvMode mode, const GemmArgs &args, hipStream_t s) {
  GemmArgs a = args;
  a.n_row_blocks = (int)((a.d.rows + kGemmRows - 1) / kGemmRows);
  if (a.d.ns > (uint32_t)kGemmNs || (mode == GEMV_GATE_UP && a.d.rows % 64)) return hipErrorInvalidValue;
  const size_t blocks = (size_t)a.n_row_blocks * a.max_col_tiles;
  if (!blocks) return hipSuccess;
  const size_t lds = gemm_lds_bytes();
  if (mode == GEMV_GATE_UP)
    hipLaunchKernelGGL(k_gemm_fp8<GEMV_GATE_UP>, dim3((unsigned)blocks), dim3(kGemmThreads), lds, s, a);
  else
    hipLaunchKernelGGL(k_gemm_fp8<GEMV_DOWN>, dim3((unsigned)blocks), dim3(kGemmThreads), lds, s, a);
  return hipGetLastError();
}

}  // namespace moe
