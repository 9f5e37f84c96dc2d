// Grouped expert GEMM for batched decode and prefill (the per-expert FFN of session.rs:87-124
// applied to every (token, slot) entry routed to an expert, session.rs:943-972) on the
// block-scaled MFMA v_mfma_scale_f32_16x16x128_f8f6f4: A = the expert's MXFP4 weights as
// stored (E2M1 nibbles + E8M0 scales, resident tile16 layout), B = the activations of the
// expert's entries as kTerms fp8 terms (split8_fp8), f32 accumulation.
//
//   k_split_rows   f32 rows (x) -> step-major activation records
//   k_gemm_fp8     one block = 64 RT weight rows x 16 CG entries of one expert; each wavefront
//                  owns 16 RT rows (RT tiles of 16) x all the block's entries (CG column
//                  groups) x kGemmTerms activation terms.
//                  K-steps of 128 run through a ring of 3: the B records of the entries go
//                  straight into LDS by LDS-DMA (global_load_lds), A tiles into registers, two
//                  steps ahead of the MFMAs.
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

// The batch path multiplies by the first kGemmTerms terms of the records (3 of 4: the
// activation is then exact to 2^-12 of each value, well inside the 1e-3 tolerance; the fourth
// term would add a third more MFMA work and LDS traffic for precision no caller needs).
constexpr int kGemmTerms = 3;
constexpr int kEntryStep = kGemmTerms * 128 + 16;   // LDS bytes of one entry's K-step
static_assert(G::kStep == kTerms * 128 + 16, "a K-step of a record = term data + 16 scale bytes");
static_assert(kEntryStep % 64 == 16, "entry stride: 16-byte aligned, spreads over the LDS banks");
constexpr int kChunks = kEntryStep / 16;            // 16-byte chunks per entry K-step (25)

// s_waitcnt immediate that waits until at most n vector-memory operations of the wavefront are
// outstanding (vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left at their maxima).
constexpr int vm_wait(int n) { return 0x0F70 | (n & 0xF) | ((n >> 4) << 14); }
// The same with lgkmcnt 0: also this wavefront's LDS operations complete.
constexpr int vm_lgkm_wait(int n) { return vm_wait(n) & ~0x0F00; }

// LDS-DMA of 16 (dwordx4) or 4 (dword) bytes per lane: lane l's bytes land at LDS address
// lds + l * size (lds uniform over the wavefront). Written as inline assembly so that the compiler does not see these LDS writes:
// it would otherwise make later LDS reads wait for every DMA in flight (it cannot always tell
// the ring slots apart). The kernel orders them itself: vmcnt waits counted per step, then a
// barrier, with compiler fences around it.
__device__ __forceinline__ void lds_dma16(const void *g, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(la) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void *g, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(la) : "memory", "m0");
}

// Block shape: W wavefronts x RT tiles of 16 weight rows each, x CG column groups of 16
// entries shared by the W wavefronts. Every operand goes through LDS by LDS-DMA
// (global_load_lds) into a ring of D K-steps: per step, the B records of the entries (kDma
// 1 KB pieces per wavefront), and per wavefront its RT A chunks (1 KB each) and RT A-scale words
// (256 B each).
template <int RT, int CG, int W, int D>
struct GemmShape {
  static constexpr int kThreads = 64 * W;
  static constexpr int kRows = 16 * RT * W;                  // weight rows per block
  static constexpr int kCols = 16 * CG;                      // entries per block
  static constexpr int kStepChunks = kCols * kChunks;        // 16-byte chunks of one K-step of B
  static constexpr int kGroups = (kStepChunks + 63) / 64;    // 1 KB pieces holding them
  static constexpr int kDma = (kGroups + W - 1) / W;         // B pieces per wavefront per step
  static constexpr int kBufB = kDma * W * 1024;              // one step of B (+ the pieces past kGroups)
  static constexpr int kBufA = W * RT * 1024;                // A chunks of one step
  static constexpr int kBufS = W * RT * 256;                 // A-scale words of one step
  static constexpr int kSlot = kBufB + kBufA + kBufS;        // one ring slot
  static constexpr int kLds = D * kSlot;
  static constexpr int kIssue = kDma + 2 * RT;               // VMEM operations per wavefront per step
};

// B operands of one column group for the wavefront's lanes (entry j, lane group g): per term the
// 32 bytes of the MFMA B layout and the E8M0 scale of the lane's block.
struct GemmB {
  i32x8 v[kGemmTerms];
  uint32_t sc[kGemmTerms];
};

__device__ __forceinline__ void gemm_read_b(GemmB &b, const uint8_t *eb, int g) {
#pragma unroll
  for (int t = 0; t < kGemmTerms; t++) {
    const uint4 b0 = *reinterpret_cast<const uint4 *>(eb + t * 128 + 32 * (g >> 1) + 16 * (g & 1));
    const uint4 b1 = *reinterpret_cast<const uint4 *>(eb + t * 128 + 64 + 32 * (g >> 1) + 16 * (g & 1));
    b.v[t] = i32x8{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    b.sc[t] = *reinterpret_cast<const uint32_t *>(eb + kGemmTerms * 128 + 4 * t) >> (8 * g);
  }
}

// MFMAs of one K-step for a wavefront: RT row tiles x CG column groups x kGemmTerms terms, all
// operands from the step's ring slot; sh = 8 * (s % 4) selects the step's byte of the A-scale
// words. The B operands of column group c + 1 are read while the MFMAs of group c run. Column
// groups past the block's entries compute on repeated entries (not stored).
template <int RT, int CG, int W, int D>
__device__ __forceinline__ void gemm_step(f32x4 (&acc)[RT][CG], const uint8_t *slot, int wv, int lane, int sh) {
  using S = GemmShape<RT, CG, W, D>;
  const int j = lane & 15, g = lane >> 4;
  const uint8_t *bb = slot + j * kEntryStep, *ab = slot + S::kBufB + wv * RT * 1024,
                *sb = slot + S::kBufB + S::kBufA + wv * RT * 256;
  uint4 ar[RT];
  uint32_t sw[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) {
    ar[r] = *reinterpret_cast<const uint4 *>(ab + r * 1024 + 16 * lane);
    sw[r] = *reinterpret_cast<const uint32_t *>(sb + r * 256 + 4 * lane) >> sh;
  }
  GemmB bc, bn;
  gemm_read_b(bc, bb, g);
#pragma unroll
  for (int c = 0; c < CG; c++) {
    if (c + 1 < CG) gemm_read_b(bn, bb + 16 * (c + 1) * kEntryStep, g);
    __builtin_amdgcn_sched_barrier(0);  // the next group's reads issue before this group's MFMAs
#pragma unroll
    for (int t = 0; t < kGemmTerms; t++) {
#pragma unroll
      for (int r = 0; r < RT; r++) {
        const i32x8 A = {(int)ar[r].x, (int)ar[r].y, (int)ar[r].z, (int)ar[r].w, 0, 0, 0, 0};
        acc[r][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, bc.v[t], acc[r][c], 4, 0, 0, (int)sw[r], 0,
                                                                     (int)bc.sc[t]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < CG) bc = bn;
  }
}

template <int MODE, int RT, int CG, int W, int D>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4))) void k_gemm_fp8(GemmArgs a) {
  using S = GemmShape<RT, CG, W, D>;
  // the ring slots as separate LDS objects: the LDS-DMA into one slot is then known not to
  // alias the reads of another, so those reads do not wait for it
  __shared__ __attribute__((aligned(1024))) uint8_t s_r0[S::kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t s_r1[S::kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t s_r2[D == 3 ? S::kSlot : 16];
  __shared__ int s_tile[4];  // expert record index, first entry, entry count, row block
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int j = lane & 15, g = lane >> 4;

  // ---- tile: global column tile cl (over the experts' kCols-entry tiles) and row block, row
  //      blocks fastest, so neighbouring blocks share the entries' activation records.
  //      Wavefront 0 finds the expert of tile cl: lanes read 64 experts' entry ranges at once,
  //      a prefix sum of their tile counts places cl.
  if (wv == 0) {
    const int cl = (int)blockIdx.x / a.n_row_blocks;
    const int na = min(*a.n_active, a.max_active);
    int ex = -1, beg = 0, cnt = 0, base = 0;
    for (int q0 = 0; q0 < na; q0 += 64) {
      const int ai = q0 + lane;
      int o0 = 0, o1 = 0;
      if (ai < na) {
        o0 = a.active_off[ai];
        o1 = a.active_off[ai + 1];
      }
      const int nct = (o1 - o0 + S::kCols - 1) / S::kCols;
      int incl = nct;  // inclusive prefix sum over the lanes
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
      }
      const int start = base + incl - nct;
      const uint64_t hit = __ballot(ai < na && cl >= start && cl < start + nct);
      if (hit) {
        const int hl = __builtin_ctzll(hit);
        if (lane == hl) {
          ex = a.active_ids[ai];
          beg = o0 + (cl - start) * S::kCols;
          cnt = min(S::kCols, o1 - beg);
        }
        ex = __shfl(ex, hl);
        beg = __shfl(beg, hl);
        cnt = __shfl(cnt, hl);
        break;
      }
      base += __shfl(incl, 63);
    }
    if (lane == 0) {
      s_tile[0] = ex;
      s_tile[1] = beg;
      s_tile[2] = cnt;
      s_tile[3] = (int)blockIdx.x - cl * a.n_row_blocks;
    }
  }
  __syncthreads();
  const int ex = s_tile[0], beg = s_tile[1], ncol = s_tile[2];
  if (ex < 0) return;
  const int rblk = s_tile[3];
  const int t0 = (rblk * S::kRows + wv * 16 * RT) / 16;  // first 16-row tile of the wavefront
  const uint8_t *rec = a.base + (size_t)ex * a.stride;
  const uint8_t *mat = rec + a.mat_off;
  const PackDims d = a.d;

  // ---- sources. B: piece i of the wavefront = 1 KB piece 4 i + wv of the step, chunk c =
  //      64 (4 i + wv) + lane (entry c / kChunks, part c % kChunks: the first kGemmTerms terms'
  //      16-byte pieces, then the 16 scale bytes); padding entries repeat a valid entry; pieces
  //      past kGroups land in the unused tail of the slot's B area. A: chunk (step, lane) of each of the wavefront's RT
  //      tiles; tiles past the matrix read the last tile (results not stored); a lane's K-block
  //      past the matrix reads an in-range chunk, whose scale byte is 0 (the packer zero-fills
  //      them) while the B records hold zeros there, so it adds exact zeros. Every lane of every
  //      DMA runs, so each wavefront issues exactly kIssue VMEM operations per step, which the
  //      vmcnt waits count on.
  const uint8_t *bsrc[S::kDma];
#pragma unroll
  for (int i = 0; i < S::kDma; i++) {
    const int c = min(64 * (W * i + wv) + lane, S::kStepChunks - 1);
    const int e = c / kChunks, part = c % kChunks;
    const int ge = beg + min(e, ncol - 1);
    const int row = a.entry_src ? a.entry_src[ge] : ge;
    bsrc[i] = a.brec + (size_t)row * G::kBytes + (part < kChunks - 1 ? 16 * part : kTerms * 128);
  }
  const uint8_t *asrc[RT];
  const uint8_t *ssrc[RT];
  bool tv[RT];
  const size_t last_chunk = (size_t)d.rows * d.nb - 1;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    tv[r] = t0 + r < (int)d.tiles;
    const int tl = min(t0 + r, (int)d.tiles - 1);
    asrc[r] = mat + (size_t)tl * 16 * d.nb * 16;
    ssrc[r] = mat + pack_weight_bytes(d) + (size_t)tl * d.nq * 256 + 4 * lane;
  }
  const uint8_t *alast = mat + last_chunk * 16;
#define GEMM_LOAD(step, sl)                                                                         \
  do {                                                                                              \
    _Pragma("unroll") for (int i = 0; i < S::kDma; i++) {                                           \
      lds_dma16(bsrc[i] + (size_t)(step) * G::kStep, (sl) + 1024 * (W * i + wv));                  \
    }                                                                                               \
    _Pragma("unroll") for (int r = 0; r < RT; r++) {                                                \
      const uint8_t *src = asrc[r] + (size_t)(step) * 1024 + 16 * lane;                             \
      lds_dma16(src < alast ? src : alast, (sl) + S::kBufB + (wv * RT + r) * 1024);                 \
    }                                                                                               \
    _Pragma("unroll") for (int r = 0; r < RT; r++)                                                  \
      lds_dma4(ssrc[r] + (size_t)((step) >> 2) * 256, (sl) + S::kBufB + S::kBufA + (wv * RT + r) * 256); \
  } while (0)

  f32x4 acc[RT][CG];
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int c = 0; c < CG; c++) acc[r][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- bias of the epilogue, loaded now so that its latency hides under the K loop
  const float *bias = reinterpret_cast<const float *>(rec + a.bias_off);
  float4 bv[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) bv[r] = reinterpret_cast<const float4 *>(bias)[min(t0 + r, (int)d.tiles - 1) * 4 + g];

  // ---- K loop, unrolled by D so that each step names its ring slots: step s computes from
  //      slot s % D while steps s + 1 .. s + D - 1 load. Every step issues one step's loads
  //      (past the last step: a repeat of step ns - 1 into the free slot), so the VMEM count is
  //      the same at every step and the wait needs no branch: each step ends with this
  //      wavefront's loads of step s + 1 complete (issued after them: D - 2 steps' loads) and
  //      its LDS reads done, then a barrier: slot (s + 1) % D is whole, slot s % D is free.
  static_assert(D == 2 || D == 3, "ring depth");
  const int ns = (int)d.ns;
#define GEMM_STEP(st, cur, nxt)                                                                     \
  do {                                                                                              \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    GEMM_LOAD(min((st) + D - 1, ns - 1), nxt);                                                      \
    gemm_step<RT, CG, W, D>(acc, cur, wv, lane, 8 * ((st) & 3));                                    \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    __builtin_amdgcn_s_waitcnt(vm_lgkm_wait((D - 2) * S::kIssue));                                  \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                        \
    __builtin_amdgcn_s_barrier();                                                                   \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                        \
  } while (0)
  GEMM_LOAD(0, s_r0);
  if (D == 3) GEMM_LOAD(min(1, ns - 1), s_r1);
  __builtin_amdgcn_s_waitcnt(vm_lgkm_wait((D - 2) * S::kIssue));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (D == 2) {
    for (int s = 0; s < ns; s += 2) {
      GEMM_STEP(s, s_r0, s_r1);
      if (s + 1 < ns) GEMM_STEP(s + 1, s_r1, s_r0);
    }
  } else {
    for (int s = 0; s < ns; s += 3) {
      GEMM_STEP(s, s_r0, s_r2);
      if (s + 1 < ns) GEMM_STEP(s + 1, s_r1, s_r0);
      if (s + 2 < ns) GEMM_STEP(s + 2, s_r2, s_r1);
    }
  }
#undef GEMM_STEP
#undef GEMM_LOAD

  // ---- epilogue
  if (MODE == GEMV_GATE_UP) {
    // every 4 row tiles (64 rows) of the wavefront = h block hb (h values 32 hb .. 32 hb + 31)
    // of its entries. The h terms are staged per entry in the (now free) ring as [4 terms x 32
    // bytes | 4 scale bytes], then copied to the h records with 16-byte stores.
    static_assert(RT % 4 == 0, "whole h blocks per wavefront");
    constexpr int kStage = 144;  // bytes per entry, 16-byte aligned
    static_assert(W <= 8 && 4 * S::kCols * kStage <= S::kSlot, "staging fits in two ring slots");
    uint8_t *hout = reinterpret_cast<uint8_t *>(a.out);
    uint8_t *stage = (wv < 4 ? s_r0 : s_r1) + (wv & 3) * S::kCols * kStage;
#pragma unroll
    for (int hbk = 0; hbk < RT / 4; hbk++) {
      if (!tv[4 * hbk]) break;  // the matrix has whole h blocks (rows % 64 == 0)
      const int hb = t0 / 4 + hbk;
#pragma unroll
      for (int c = 0; c < CG; c++) {
        if (16 * c >= ncol) break;
        float hv[8];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const f32x4 &av = acc[4 * hbk + r][c];
          const float4 &b4 = bv[4 * hbk + r];
          hv[2 * r] = swiglu(av[0] + b4.x, av[1] + b4.y, a.limit);
          hv[2 * r + 1] = swiglu(av[2] + b4.z, av[3] + b4.w, a.limit);
        }
        uint2 q[kTerms];
        uint32_t s4;
        split8_fp8_cols(hv, q, s4);
        uint8_t *se = stage + (16 * c + j) * kStage;
#pragma unroll
        for (int t = 0; t < kTerms; t++) {
#pragma unroll
          for (int r = 0; r < 4; r++) {  // h 8r + 2g, 8r + 2g + 1 of the block = bytes 2r, 2r+1
            const uint32_t w = r < 2 ? q[t].x : q[t].y;
            *reinterpret_cast<uint16_t *>(se + t * 32 + 8 * r + 2 * g) = (uint16_t)(w >> (16 * (r & 1)));
          }
        }
        if (g == 0) *reinterpret_cast<uint32_t *>(se + 128) = s4;
      }
      const int st = hb >> 2, i = hb & 3;
      for (int p = lane; p < ncol * 8; p += 64) {
        const int e = p >> 3, t = (p >> 1) & 3, half = p & 1;
        *reinterpret_cast<uint4 *>(hout + (size_t)(beg + e) * G::kBytes + G::data(st, t) + 32 * i + 16 * half) =
            *reinterpret_cast<const uint4 *>(stage + e * kStage + t * 32 + 16 * half);
      }
      for (int p = lane; p < ncol * kTerms; p += 64) {
        const int e = p / kTerms, t = p % kTerms;
        hout[(size_t)(beg + e) * G::kBytes + G::scale(st, t) + i] = stage[e * kStage + 128 + t];
      }
      __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));  // staging reads done before the next h block
    }
  } else {
    float *out = reinterpret_cast<float *>(a.out);
    const int R = (int)d.rows;
#pragma unroll
    for (int r = 0; r < RT; r++) {
      if (!tv[r]) continue;
      const float4 b4 = bv[r];
      const int row = (t0 + r) * 16 + 4 * g;
#pragma unroll
      for (int c = 0; c < CG; c++) {
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

template <int MODE, int RT, int CG, int W, int D>
static hipError_t launch_gemm_shape(GemmArgs a, hipStream_t s) {
  using S = GemmShape<RT, CG, W, D>;
  static_assert(S::kLds <= 160 * 1024 - 64, "LDS");
  a.n_row_blocks = (int)((a.d.rows + S::kRows - 1) / S::kRows);
  const size_t col_tiles = (size_t)a.max_active + (a.n_entries + S::kCols - 1) / S::kCols;
  const size_t blocks = (size_t)a.n_row_blocks * col_tiles;
  if (!blocks) return hipSuccess;
  hipLaunchKernelGGL((k_gemm_fp8<MODE, RT, CG, W, D>), dim3((unsigned)blocks), dim3(S::kThreads), 0, s, a);
  return hipGetLastError();
}

// Column tile width from the mean entries per active expert (the per-expert counts live on the
// device): 64 entries once experts average 48 or more (8 wavefronts, two per SIMD, so that one
// wavefront's LDS reads overlap the other's MFMAs), down to 16 for a few per expert.
template <int MODE>
static hipError_t launch_gemm_mode(const GemmArgs &a, hipStream_t s) {
  const size_t active = std::max<size_t>(1, std::min<size_t>((size_t)a.max_active, a.n_entries));
  const size_t mean = a.n_entries / active;
  if (mean >= 48) return a.shape == 1 ? launch_gemm_shape<MODE, 8, 4, 4, 2>(a, s) : launch_gemm_shape<MODE, 4, 4, 8, 2>(a, s);
  if (mean >= 24) return launch_gemm_shape<MODE, 4, 2, 4, 3>(a, s);
  return launch_gemm_shape<MODE, 4, 1, 4, 3>(a, s);
}

hipError_t launch_gemm_fp8(GemvMode mode, const GemmArgs &a, hipStream_t s) {
  if (a.d.ns > (uint32_t)kGemmNs || (mode == GEMV_GATE_UP && a.d.rows % 64)) return hipErrorInvalidValue;
  return mode == GEMV_GATE_UP ? launch_gemm_mode<GEMV_GATE_UP>(a, s) : launch_gemm_mode<GEMV_DOWN>(a, s);
}

}  // namespace moe
