// Grouped expert GEMM for batched decode and prefill (the per-expert FFN of session.rs:87-124
// applied to every (token, slot) entry routed to an expert, session.rs:943-972) on the
// block-scaled MFMA v_mfma_scale_f32_16x16x128_f8f6f4: A = the expert's MXFP4 weights as
// stored (E2M1 nibbles + E8M0 scales, resident tile16 layout), B = the activations of the
// expert's entries as NT E2M3 terms per value (kGemmTerms: the exact split, the default; 1: the
// quantized-activation mode, one MXFP6 term), written as GemmRecT<NT> records (the batch router
// writes the tokens', rec_split_block; the gate_up epilogue the entries' h), f32 accumulation.
//
//   k_gemm_fp8     one block = WR x WC wavefronts; wavefront (wr, wc) owns RT tiles of 16 weight
//                  rows x CGW column groups of 16 entries of one expert, x NT terms.
//                  K-steps of 128 run through a ring of D = 2 or 3 LDS slots: the entries' B
//                  records, the A chunks and their scale words all go into LDS by LDS-DMA
//                  (global_load_lds), D - 1 steps ahead of the MFMAs.
//                  GATE_UP epilogue: bias, SwiGLU (gate = row 2i, up = row 2i+1) and the split
//                  of the wavefront's 32 h values per entry into the h records; DOWN epilogue:
//                  bias and +-65504 clamp into f32 [entry][H].
#include <algorithm>
#include <atomic>

#include "device.hpp"
#include "kernels.hpp"
#include "stream.hpp"

namespace moe {

// ------------------------------------------------------------------ grouped GEMM

// The batch path's activations are kGemmTerms E2M3 terms (exact to about 2^-13 of each block's
// maximum, well inside the 1e-3 tolerance): the fp4 x fp6 MFMA issues in 16 cycles where fp4 x
// fp8 takes 32, and a K-step of a record is 304 bytes instead of 400 for three fp8 terms (112
// bytes and a third of the MFMAs with one term, in the quantized mode).
// B in LDS, per K-step: the entries' record steps one after the other (GemmRecT<NT>::kStep bytes
// each, as the LDS-DMA copies them: each DMA reads whole record steps, a few rows per instruction).


// LDS-DMA of 16 (dwordx4) or 4 (dword) bytes per lane: lane l's bytes land at LDS address
// lds + l * size (lds uniform over the wavefront). Written as inline assembly so that the compiler does not see these LDS writes:
// it would otherwise make later LDS reads wait for every DMA in flight (it cannot always tell
// the ring slots apart). The kernel orders them itself: vmcnt waits counted per step, then a
// barrier, with compiler fences around it.
__device__ __forceinline__ void lds_dma16(const void *g, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(la) : "memory", "m0");
}
// The same with the non-temporal cache policy: for weight chunks read once per launch (the small
// blocks of batches of a few entries per expert; measured at 64 tokens: down 37.5 -> 36.0 us; where
// column tiles of one expert re-read the chunks, at prefill, it cost 4 %).
__device__ __forceinline__ void lds_dma16_nt(const void *g, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(la) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void *g, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(la) : "memory", "m0");
}

// The LDS byte address of p (a pointer into a __shared__ object).
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}
// LDS-DMA of 16 bytes per lane to the LDS byte address la (wavefront-uniform), from sbase + voff.
__device__ __forceinline__ void lds_dma16_sa(uint32_t voff, const void *sbase, uint32_t la) {
  la = __builtin_amdgcn_readfirstlane(la);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(la) : "memory", "m0");
}

// The same with a wavefront-uniform 64-bit base in SGPRs and a 32-bit per-lane offset
// (global address = sbase + voff): one VGPR per lane instead of a 64-bit pointer.
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void *sbase, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(la) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4_s(uint32_t voff, const void *sbase, const void *lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(la) : "memory", "m0");
}

// Block shape: WR x WC wavefronts; wavefront (wr, wc) owns RT tiles of 16 weight rows (row
// group wr) x CGW column groups of 16 entries (entry group wc). Every operand goes through LDS by
// LDS-DMA (global_load_lds) into a ring of D K-steps: per step, the B records of the block's
// entries (kDma 1 KB pieces per wavefront), the block's WR * RT A chunks (1 KB each) and A-scale
// words (256 B each), kDmaA of each per wavefront.
template <int RT, int CGW, int WR, int WC, int D, int NT>
struct GemmShape {
  static constexpr int kChunks = GemmRecT<NT>::kChunks;     // 16-byte chunks per entry K-step
  static constexpr int W = WR * WC;
  static constexpr int kThreads = 64 * W;
  static constexpr int kRows = 16 * RT * WR;                 // weight rows per block
  static constexpr int kCols = 16 * CGW * WC;                // entries per block
  static constexpr int kStepChunks = kCols * kChunks;        // 16-byte chunks of one K-step of B
  static constexpr int kGroups = (kStepChunks + 63) / 64;    // 1 KB pieces holding them
  static constexpr int kDma = (kGroups + W - 1) / W;         // B pieces per wavefront per step
  static constexpr int kTilesA = WR * RT;                    // A tiles of the block
  static constexpr int kDmaA = kTilesA / W;                  // A tiles (and scale words) per wavefront
  static_assert(kTilesA % W == 0, "A tiles shared evenly");
  // one wavefront per SIMD with 16+ row tiles (B-stationary steps): B holds exactly kGroups pieces
  // and the pieces past them land in a dummy area; otherwise the slot also holds those pieces
  static constexpr bool kBStat = RT >= 16;
  // D = 2, and D = 3 with 512 rows (whose 8 KB of scale words per step would leave no room for a
  // third slot): the A-scale words (one byte per step) go once per 4 steps into a pair of buffers
  // outside the ring, and B pieces past kGroups are not loaded (11 of the 64 KB a 512 x 64 step
  // moved were such repeats), so the number of a step's DMAs varies and the waits count it
  static constexpr bool kScale4 = !kBStat && (D == 2 || kRows >= 512);
  // (the 3-slot ring keeps only the kGroups pieces in a slot, so that three fit)
  static constexpr int kBufB = (kBStat || (kScale4 && D == 3) ? kGroups : kDma * W) * 1024;
  static constexpr int kBufA = kTilesA * 1024;               // A chunks of one step
  // two steps in flight (operands read into registers, then the slot refilled), for column
  // groups narrow enough to hold a step's operands
  static constexpr bool kTwoAhead = kScale4 && D == 2 && CGW <= 2;
  // DMA addresses as wavefront-uniform bases plus 32-bit lane offsets (fewer VGPRs)
  static constexpr bool kSAddr = kBStat || kTwoAhead || (kScale4 && D == 3);
  static constexpr int kBufS = kScale4 ? 0 : kTilesA * 256;  // A-scale words of one step
  static constexpr int kSlot = kBufB + kBufA + kBufS;        // one ring slot
  static constexpr int kLds = D * kSlot;
  static constexpr int kIssue = kDma + 2 * kDmaA;            // VMEM operations per wavefront per step
  // the counted waits hold at most two steps' loads of a wavefront outstanding (its B pieces, A
  // tiles and scale words), which must fit the 6-bit vmcnt field
  static_assert(2 * kIssue <= 63, "a step's loads fit the vmcnt field");
};

// B operands of one column group for the wavefront's lanes (entry j, lane group g): per term the
// 32 bytes of the MFMA B layout and the E8M0 scale of the lane's block.
template <int NT>
struct GemmB {
  i32x8 v[NT];
  uint32_t sc[NT];
};

// Term t of lane (j, g) from entry j's record step at eb: the first 16 bytes of block g (chunk
// 6t + g) and the last 8 (half g & 1 of chunk 6t + 4 + g / 2). Both are 16-byte reads (twice the
// bytes per cycle of 8-byte reads): the pair chunk is read whole by both lanes of a pair, so 16
// lanes share one address pair-wise and the reads of a 32-lane half have no bank conflicts; the
// first-16-byte reads (records 304 bytes apart) take two passes where 8-byte reads took two each.
// (Tails in the block order 0, 2, 1, 3, read by lane groups g and g ^ 2, cost 4 % at prefill.)
template <int NT>
__device__ __forceinline__ void gemm_read_b_t(GemmB<NT> &b, const uint8_t *eb, int g, int t) {
  const uint4 x = *reinterpret_cast<const uint4 *>(eb + (6 * t + g) * 16);
  const uint4 y = *reinterpret_cast<const uint4 *>(eb + (6 * t + 4 + (g >> 1)) * 16);
  const bool odd = (g & 1) != 0;
  b.v[t] = i32x8{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)(odd ? y.z : y.x), (int)(odd ? y.w : y.y), 0, 0};
}

// The scale words of the terms (the last chunk of the record step; byte g is the lane's block).
template <int NT>
__device__ __forceinline__ void gemm_read_sc(GemmB<NT> &b, const uint8_t *eb, int g) {
  const uint8_t *p = eb + (GemmRecT<NT>::kChunks - 1) * 16;
  if constexpr (NT == 1) {
    b.sc[0] = *reinterpret_cast<const uint32_t *>(p) >> (8 * g);
  } else {
    const uint4 sc = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[3] = {sc.x, sc.y, sc.z};
#pragma unroll
    for (int t = 0; t < NT; t++) b.sc[t] = w[t] >> (8 * g);
  }
}

template <int NT>
__device__ __forceinline__ void gemm_read_b(GemmB<NT> &b, const uint8_t *eb, int g) {
#pragma unroll
  for (int t = 0; t < NT; t++) gemm_read_b_t(b, eb, g, t);
  gemm_read_sc(b, eb, g);
}

// MFMAs of one K-step for a wavefront: RT row tiles x CG column groups x NT terms, all
// operands from the step's ring slot (sw4: the wavefront's A-scale words of the current 4 steps,
// read from LDS once per 4 steps); sh = 8 * (s % 4) selects the step's byte of them. The B operands of column group c + 1 are read while the MFMAs of group c
// run. Column groups past the block's entries compute on repeated entries (not stored).
template <int RT, int CGW, int WR, int WC, int D, int NT>
__device__ __forceinline__ void gemm_step(f32x4 (&acc)[RT][CGW], const uint8_t *slot, const uint32_t (&sw4)[RT], int wr,
                                          int wc, int lane, int sh) {
  using S = GemmShape<RT, CGW, WR, WC, D, NT>;
  constexpr int CG = CGW, kEntryStep = GemmRecT<NT>::kStep;
  const int j = lane & 15, g = lane >> 4;
  const uint8_t *bb = slot + (16 * CGW * wc + j) * kEntryStep, *ab = slot + S::kBufB + wr * RT * 1024;
  uint4 ar[RT];
  uint32_t sw[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) {
    ar[r] = *reinterpret_cast<const uint4 *>(ab + r * 1024 + 16 * lane);
    sw[r] = sw4[r] >> sh;
  }
  GemmB<NT> bc, bn;
  gemm_read_b(bc, bb, g);
#pragma unroll
  for (int c = 0; c < CG; c++) {
    if (c + 1 < CG) gemm_read_b(bn, bb + 16 * (c + 1) * kEntryStep, g);
    __builtin_amdgcn_sched_barrier(0);  // the next group's reads issue before this group's MFMAs
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
      for (int r = 0; r < RT; r++) {
        const i32x8 A = {(int)ar[r].x, (int)ar[r].y, (int)ar[r].z, (int)ar[r].w, 0, 0, 0, 0};
        // cbsz 4: A is fp4 (E2M1); blgp 2: B is fp6 (E2M3)
        acc[r][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, bc.v[t], acc[r][c], 4, 2, 0, (int)sw[r], 0,
                                                                     (int)bc.sc[t]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < CG) bc = bn;
  }
}

// All operands of one K-step for a wavefront (gemm_step's, read up front): the A chunks and scale
// words of its RT row tiles and the B operands of its CG column groups.
template <int RT, int CG, int NT>
struct GemmOps {
  uint4 ar[RT];
  uint32_t sw[RT];
  GemmB<NT> b[CG];
};

// One column group's B as read (both 16-byte chunks of each term, the scale chunk), before
// gemm_read_b_t's half selection: reads issued early, selected once they are needed.
template <int NT>
struct GemmBRaw {
  uint4 x[NT], y[NT];
  uint32_t sc[NT];
};
template <int NT>
__device__ __forceinline__ void gemm_read_b_raw(GemmBRaw<NT> &b, const uint8_t *eb, int g) {
#pragma unroll
  for (int t = 0; t < NT; t++) {
    b.x[t] = *reinterpret_cast<const uint4 *>(eb + (6 * t + g) * 16);
    b.y[t] = *reinterpret_cast<const uint4 *>(eb + (6 * t + 4 + (g >> 1)) * 16);
  }
  const uint8_t *p = eb + (GemmRecT<NT>::kChunks - 1) * 16;
  if constexpr (NT == 1) {
    b.sc[0] = *reinterpret_cast<const uint32_t *>(p);
  } else {
    const uint4 sc = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[3] = {sc.x, sc.y, sc.z};
#pragma unroll
    for (int t = 0; t < NT; t++) b.sc[t] = w[t];
  }
}
template <int NT>
__device__ __forceinline__ void gemm_select_b(GemmB<NT> &b, const GemmBRaw<NT> &r, int g) {
  const bool odd = (g & 1) != 0;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const uint4 &x = r.x[t], &y = r.y[t];
    b.v[t] = i32x8{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)(odd ? y.z : y.x), (int)(odd ? y.w : y.y), 0, 0};
    b.sc[t] = r.sc[t] >> (8 * g);
  }
}

// The A operands and the B operands of column groups [0, C1) (selected); C1 < CGW: the later
// groups are read with gemm_read_b_raw and selected by the caller. sw4: the wavefront's A-scale
// words of the current 4 steps (read from LDS once per 4 steps; sh selects the step's byte).
template <int RT, int CGW, int WR, int WC, int D, int NT, int C1 = CGW>
__device__ __forceinline__ void gemm_read_ops(GemmOps<RT, CGW, NT> &o, const uint8_t *slot, const uint32_t *sw4, int wr,
                                              int wc, int lane, int sh) {
  using S = GemmShape<RT, CGW, WR, WC, D, NT>;
  constexpr int kEntryStep = GemmRecT<NT>::kStep;
  const int j = lane & 15, g = lane >> 4;
  const uint8_t *bb = slot + (16 * CGW * wc + j) * kEntryStep, *ab = slot + S::kBufB + wr * RT * 1024;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    o.ar[r] = *reinterpret_cast<const uint4 *>(ab + r * 1024 + 16 * lane);
    o.sw[r] = sw4[r] >> sh;
  }
#pragma unroll
  for (int c = 0; c < C1; c++) gemm_read_b(o.b[c], bb + 16 * c * kEntryStep, g);
}

// The MFMAs of gemm_step for column groups [C0, C1) on operands already in registers (per output
// the terms t = 0, 1, 2 in turn, as gemm_step, so both give the same bits), with dma(0) before
// them (it may branch) and dma(1 .. NI - 1) spread over them (they must not branch, or the MFMAs
// move out of order): the CU's memory pipeline accepts about 64 bytes per cycle, so issuing a
// step's ~60 KB of LDS-DMA takes about as long as the MFMAs, which run meanwhile. The empty asm
// at the end takes the groups' accumulators as operands, so their MFMAs stay before the barrier
// that follows (the compiler otherwise moved them past it, where they ran after every other part
// of the step).
template <int RT, int CGW, int NT, int C0, int C1, int NI, typename F>
__device__ __forceinline__ void gemm_mfma_ops(f32x4 (&acc)[RT][CGW], const GemmOps<RT, CGW, NT> &o, F &&dma) {
  constexpr int NM = (C1 - C0) * NT * RT;
  if constexpr (NI > 0) dma(0);
  __builtin_amdgcn_sched_barrier(0);  // (a branch in dma(0) ends the block here)
#pragma unroll
  for (int c = C0; c < C1; c++) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
      for (int r = 0; r < RT; r++) {
        const i32x8 A = {(int)o.ar[r].x, (int)o.ar[r].y, (int)o.ar[r].z, (int)o.ar[r].w, 0, 0, 0, 0};
        // cbsz 4: A is fp4 (E2M1); blgp 2: B is fp6 (E2M3)
        acc[r][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, o.b[c].v[t], acc[r][c], 4, 2, 0, (int)o.sw[r], 0,
                                                                     (int)o.b[c].sc[t]);
        const int m = ((c - C0) * NT + t) * RT + r;
#pragma unroll
        for (int i = 1; i < NI; i++) {
          // DMA i after MFMA (i NM) / NI - 1; with more DMAs than MFMAs (one term) several
          // share an MFMA, the first ones MFMA 0
          if (m == max((i * NM) / (NI > 0 ? NI : 1) - 1, 0)) {
            __builtin_amdgcn_sched_barrier(0);
            dma(i);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int c = C0; c < C1; c++) asm volatile("" : "+v"(acc[r][c]));
}

// ---- the 32x32x64 form (v_mfma_scale_f32_32x32x64_f8f6f4) of the 512 x 64 two-ahead shape: a
//      wavefront holds 4 row tiles of 32 rows (its 8 tile16 chunks taken in pairs) x 32 entries,
//      and a K-step of 128 is two 64-value halves h. Lane layouts (measured on gfx950): A lane l =
//      row l % 32, K-block 2h + l / 32 of the step (16 bytes of E2M1, its E8M0 scale); B lane l =
//      entry l % 32, the same K-block (24 bytes of E2M3, its scale); accumulator v of lane l = row
//      8 (v / 4) + 4 (l / 32) + v % 4, entry l % 32. The A operand comes from the tile16 chunks as
//      stored: lane m = (l % 16) + 16 (2h + l / 32) of chunk (l % 32) / 16 of the pair, so the same
//      DMA layout serves both forms; a lane reads each term's 48 bytes of a step as two 16-byte and
//      two 8-byte reads (none discarded); a step is 24 MFMAs of 32 x 32 x 64 where the 16 x 16 x 128
//      form issues 48 (measured: 1.66x the issue cycles for 2x the work). Measured slower than the
//      16 x 16 x 128 form at prefill all the same (gate_up 581 against 548 us, down 315 against
//      306): the loop is bound by its LDS reads and waits, not the MFMA issue, and the 16-register
//      accumulators at the 256-register limit make the compiler move them between steps.
template <int NT>
struct Gemm32Ops {
  uint4 a[4][2];       // [row tile][half]
  uint32_t sa[4][2];   // A scale of the step (byte 0)
  i32x8 b[NT][2];      // [term][half]: the lane's 24 bytes of E2M3 (the MFMA operand; built as read,
                       // so no wider load spans two fields and the operands stay in registers)
  uint32_t sb[NT][2];  // B scale of the step (byte 0)
};

// The wavefront's A-scale words of the current 4 steps for (row tile R, half h), from the 4-step
// scale buffer: words of the tile16 chunk and lane the A operand of (R, h) comes from.
template <int RT>
__device__ __forceinline__ void gemm32_read_sw4(uint32_t (&sw4)[4][2], const uint8_t *sbuf, int wr, int lane) {
  const int m0 = lane & 15, u = lane >> 5, cpair = (lane & 31) >> 4;
#pragma unroll
  for (int R = 0; R < 4; R++)
#pragma unroll
    for (int h = 0; h < 2; h++)
      sw4[R][h] = *reinterpret_cast<const uint32_t *>(sbuf + (wr * RT + 2 * R + cpair) * 256 + 4 * (m0 + 16 * (2 * h + u)));
}

// Every operand of one K-step for the wavefront, half 0 first (its MFMAs can start while half 1's
// reads are in flight).
template <int RT, int NT, int kBufB>
__device__ __forceinline__ void gemm32_read_ops(Gemm32Ops<NT> &o, const uint8_t *slot, const uint32_t (&sw4)[4][2],
                                                int wr, int wc, int lane, int sh) {
  constexpr int kEntryStep = GemmRecT<NT>::kStep;
  const int j = lane & 31, u = lane >> 5, m0 = lane & 15, cpair = (lane & 31) >> 4;
  const uint8_t *ab = slot + kBufB + wr * RT * 1024, *eb = slot + (32 * wc + j) * kEntryStep;
  const uint8_t *scp = eb + (GemmRecT<NT>::kChunks - 1) * 16;
  uint32_t w[NT];
  if constexpr (NT == 1) {
    w[0] = *reinterpret_cast<const uint32_t *>(scp);
  } else {
    const uint4 sc = *reinterpret_cast<const uint4 *>(scp);
    const uint32_t ww[3] = {sc.x, sc.y, sc.z};
#pragma unroll
    for (int t = 0; t < NT; t++) w[t] = ww[t];
  }
#pragma unroll
  for (int h = 0; h < 2; h++) {
#pragma unroll
    for (int R = 0; R < 4; R++) {
      o.a[R][h] = *reinterpret_cast<const uint4 *>(ab + (2 * R + cpair) * 1024 + 16 * (m0 + 16 * (2 * h + u)));
      o.sa[R][h] = sw4[R][h] >> sh;
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      // the operand's 6 registers must be contiguous: the 16 head bytes and the 8 tail bytes of
      // block 2h + u are two reads straight into them
      const uint4 pv = *reinterpret_cast<const uint4 *>(eb + (6 * t + 2 * h + u) * 16);
      const uint2 qv = *reinterpret_cast<const uint2 *>(eb + (6 * t + 4) * 16 + 8 * (2 * h + u));
      o.b[t][h] = i32x8{(int)pv.x, (int)pv.y, (int)pv.z, (int)pv.w, (int)qv.x, (int)qv.y, 0, 0};
      o.sb[t][h] = w[t] >> (8 * (2 * h + u));
      // (the compiler would merge neighbouring 8-byte tail reads into one wider read and copy)
      asm volatile("" ::: "memory");
    }
  }
}

// The MFMAs of half H of a step (per row tile R: terms t = 0, 1, .. in turn, so every output
// accumulates half 0's terms then half 1's), with dma(0) before them and dma(1 .. NI - 1) spread
// over them, as gemm_mfma_ops. Every MFMA issues, as in the 16 x 16 x 128 shapes: rows past the
// matrix compute on clamped rows that are not stored, and the second half of the last step on
// zero-scale weights and zero activations (adds exact zeros); a branch around them made the
// compiler copy the accumulators and operands between the paths. The empty asm keeps the MFMAs
// before the barrier that follows.
template <int NT, int H, int NI, typename F>
__device__ __forceinline__ void gemm32_mfma_half(f32x16 (&acc)[4], const Gemm32Ops<NT> &o, F &&dma) {
  constexpr int NM = NT * 4;
  if constexpr (NI > 0) dma(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int R = 0; R < 4; R++) {
      {
        const uint4 &av = o.a[R][H];
        const i32x8 A = {(int)av.x, (int)av.y, (int)av.z, (int)av.w, 0, 0, 0, 0};
        const i32x8 &B = o.b[t][H];
        // cbsz 4: A is fp4 (E2M1); blgp 2: B is fp6 (E2M3)
        acc[R] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B, acc[R], 4, 2, 0, (int)o.sa[R][H], 0,
                                                                 (int)o.sb[t][H]);
      }
      const int m = t * 4 + R;
#pragma unroll
      for (int i = 1; i < NI; i++) {
        if (m == max((i * NM) / (NI > 0 ? NI : 1) - 1, 0)) {
          __builtin_amdgcn_sched_barrier(0);
          dma(i);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // (the accumulators as inputs only: an in-out operand redefines them, and the compiler then moves
  // all 64 registers between the steps' register assignments)
#pragma unroll
  for (int R = 0; R < 4; R++) asm volatile("" ::"v"(acc[R]));
}

// MFMAs of one K-step for a wavefront with many row tiles (one wavefront per SIMD): the B
// operands of all CG column groups are read once and held for the step; row tiles go in pairs,
// the A chunks of the next pair read while the MFMAs of this pair run (8 independent
// accumulators between two MFMAs into the same one). Per output the terms still accumulate in
// order t = 0, 1, 2 (the order of gemm_step, so every shape gives the same bits). FULL: every
// row tile of the wavefront is inside the matrix (no test in the loop); otherwise row pairs from
// nrt_valid on issue no MFMAs (a pair straddling the end computes its second tile on a clamped
// tile, not stored).
template <int RT, int CGW, int WR, int WC, int D, int NT, bool FULL>
__device__ __forceinline__ void gemm_step_bstat(f32x4 (&acc)[RT][CGW], const uint8_t *slot, int wr, int wc,
                                                int lane, int sh, int nrt_valid) {
  using S = GemmShape<RT, CGW, WR, WC, D, NT>;
  static_assert(RT % 2 == 0, "row tiles in pairs");
  constexpr int CG = CGW, kEntryStep = GemmRecT<NT>::kStep;
  const int j = lane & 15, g = lane >> 4;
  const uint8_t *bb = slot + (16 * CGW * wc + j) * kEntryStep, *ab = slot + S::kBufB + wr * RT * 1024,
                *sb = slot + S::kBufB + S::kBufA + wr * RT * 256;
  // the first pair's A, then B term by term: the first MFMAs (term 0 of every column group) can
  // start before the other terms have arrived
  uint4 a0 = *reinterpret_cast<const uint4 *>(ab + 16 * lane);
  uint4 a1 = *reinterpret_cast<const uint4 *>(ab + 1024 + 16 * lane);
  uint32_t s0 = *reinterpret_cast<const uint32_t *>(sb + 4 * lane) >> sh;
  uint32_t s1 = *reinterpret_cast<const uint32_t *>(sb + 256 + 4 * lane) >> sh;
  GemmB<NT> b[CG];
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int c = 0; c < CG; c++) gemm_read_b_t(b[c], bb + 16 * c * kEntryStep, g, t);
  }
#pragma unroll
  for (int c = 0; c < CG; c++) gemm_read_sc(b[c], bb + 16 * c * kEntryStep, g);
#pragma unroll
  for (int r = 0; r < RT; r += 2) {
    uint4 n0 = a0, n1 = a1;
    uint32_t t0s = s0, t1s = s1;
    if (r + 2 < RT) {
      n0 = *reinterpret_cast<const uint4 *>(ab + (r + 2) * 1024 + 16 * lane);
      n1 = *reinterpret_cast<const uint4 *>(ab + (r + 3) * 1024 + 16 * lane);
      t0s = *reinterpret_cast<const uint32_t *>(sb + (r + 2) * 256 + 4 * lane) >> sh;
      t1s = *reinterpret_cast<const uint32_t *>(sb + (r + 3) * 256 + 4 * lane) >> sh;
    }
    __builtin_amdgcn_sched_barrier(0);  // the next pair's A reads issue before this pair's MFMAs
    if (FULL || r < nrt_valid) {
      const i32x8 A0 = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, 0, 0, 0, 0};
      const i32x8 A1 = {(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w, 0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < NT; t++) {
#pragma unroll
        for (int c = 0; c < CG; c++) {
          // cbsz 4: A is fp4 (E2M1); blgp 2: B is fp6 (E2M3)
          acc[r][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A0, b[c].v[t], acc[r][c], 4, 2, 0, (int)s0, 0,
                                                                       (int)b[c].sc[t]);
          acc[r + 1][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A1, b[c].v[t], acc[r + 1][c], 4, 2, 0,
                                                                           (int)s1, 0, (int)b[c].sc[t]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    a0 = n0;
    a1 = n1;
    s0 = t0s;
    s1 = t1s;
  }
}

// The shapes that run a persistent grid: the plain two-ahead step for gate_up (the pipelined step
// measured faster on one workgroup per tile: its workgroups then turn over without a loop-top
// barrier, and the hardware dispatches the next tile's workgroup as soon as one ends).
template <int MODE, typename S, int NSP>
constexpr bool gemm_persistent() { return S::kTwoAhead && MODE == GEMV_GATE_UP && NSP == 0; }

// M32: the 32x32x64 form of the 512 x 64 two-ahead shape (gemm32_*): the same DMA layout, ring and
// waits; other MFMAs, operand reads and epilogue staging. NSP > 0: the pipelined two-ahead step
// for launches of exactly NSP K-steps.
template <int MODE, int RT, int CGW, int WR, int WC, int D, int NT, bool M32 = false, int NSP = 0, int RING = 0>
__global__ __launch_bounds__(64 * WR * WC) __attribute__((amdgpu_waves_per_eu(WR * WC / 4, WR * WC / 4))) void k_gemm_fp8(GemmArgs a) {
  using S = GemmShape<RT, CGW, WR, WC, D, NT>;
  static_assert(!M32 || (RT == 8 && CGW == 2 && S::kTwoAhead), "the 32x32 form: 128 rows x 32 entries per wavefront");
  static_assert(NSP == 0 || (!M32 && S::kTwoAhead && NSP <= kGemmNs), "the pipelined form of the two-ahead step");
  static_assert(RING == 0 || NSP > 0, "separate ring depths: the pipelined step");
  // the pipelined step's rings, in one LDS area (A slots first): RING 0 both 2 slots deep; RING 1
  // A 2 and B 3; RING 2 A 3 and B 2
  constexpr int kRingA = RING == 2 ? 3 : 2, kRingB = RING == 1 ? 3 : 2;
  constexpr int kRingBytes = NSP ? kRingA * S::kBufA + kRingB * S::kGroups * 1024 : 16;
  using G = GemmRecT<NT>;  // the activation records (x or h) of the launch
  constexpr int W = S::W, CG = CGW, kChunks = G::kChunks, kEntryStep = G::kStep;
  // the ring slots as separate LDS objects: the LDS-DMA into one slot is then known not to
  // alias the reads of another, so those reads do not wait for it
  __shared__ __attribute__((aligned(1024))) uint8_t s_r0[NSP ? 16 : S::kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t s_r1[NSP ? 16 : S::kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t s_ring[kRingBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t s_r2[D == 3 ? S::kSlot : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t s_sc[2][S::kScale4 ? S::kTilesA * 256 : 16];
  constexpr int kBiasTiles = RT < 4 ? 4 : RT;  // the bias DMA moves 64 rows (4 tiles) per wavefront load
  // per wavefront: its rows' bias (the B-stationary shape reads its bias from global memory in the
  // epilogue, and its B pieces past the step's kGroups land in s_dummy)
  __shared__ __attribute__((aligned(16))) float s_bias[S::kBStat ? 4 : W * kBiasTiles * 16];
  __shared__ __attribute__((aligned(1024))) uint8_t s_dummy[S::kBStat && S::kDma * W > S::kGroups ? 1024 : 16];
  __shared__ int s_tile[4];  // expert record index, first entry, entry count, row block
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wr = wv % WR, wc = wv / WR;
  const int j = lane & 15, g = lane >> 4;

  // ---- tile: global column tile cl (over the experts' kCols-entry tiles) and row block rblk.
  //      a.band == 0: workgroup p is tile p, row blocks fastest. a.band > 0: workgroups go to
  //      the 8 XCDs round-robin (workgroup p to XCD p % 8), so XCD x takes the logical tiles
  //      [x C, x C + C) in order, and logical tiles run in bands of a.band row blocks, column
  //      tile by column tile. The orders differ by a few percent, by matrix (measured).
  //      Wavefront 0 finds the expert of tile cl: lanes read 64 experts' entry ranges at once,
  //      a prefix sum of their tile counts places cl.
  // Workgroup p of the launch's a.n_blocks: the two-ahead gate_up shape runs a persistent grid
  // (one workgroup per CU, each taking p = blockIdx.x, + gridDim.x, ...: the same XCD for every
  // p, p % 8); the others one workgroup per p (for the down shape the loop cost 8 %, measured).
  constexpr bool kPersist = gemm_persistent<MODE, S, NSP>();
  for (int p = (int)blockIdx.x; p < a.n_blocks; p += (int)gridDim.x) {
  if (p != (int)blockIdx.x) __syncthreads();  // the previous tile's LDS reads are done
  int cl, rblk_l;
  {
    const int C = (a.n_tiles + 7) / 8;
    const int L = a.band ? (p % 8) * C + p / 8 : p;
    if (L >= a.n_tiles) {
      if constexpr (kPersist) continue;
      else return;
    }
    const int nrb = a.n_row_blocks, nct = a.n_tiles / nrb, RB = a.band ? min(a.band, nrb) : nrb, full = nrb / RB;
    if (L < full * RB * nct) {
      const int band = L / (RB * nct), r = L - band * RB * nct;
      cl = r / RB;
      rblk_l = band * RB + r % RB;
    } else {
      const int rem = nrb - full * RB, r = L - full * RB * nct;
      cl = r / rem;
      rblk_l = full * RB + r % rem;
    }
  }
  if (wv == 0) {
    // the expert count and every lane's entry range and expert id in one round of loads: lanes
    // below max_active (the lists' length) load before the count is known, lanes past the count
    // are ignored
    constexpr int kQ = (kMaxExperts + 63) / 64;
    const int ma = min(a.max_active, kMaxExperts);
    int lo[kQ], lh[kQ], lid[kQ];
#pragma unroll
    for (int q = 0; q < kQ; q++) {
      const int ai = 64 * q + lane;
      lo[q] = lh[q] = 0;
      lid[q] = -1;
      if (ai < ma) {
        lo[q] = a.active_off[ai];
        lh[q] = a.active_off[ai + 1];
        lid[q] = a.active_ids[ai];
      }
    }
    const int na = min(*a.n_active, ma);
    int ex = -1, beg = 0, cnt = 0, base = 0;
#pragma unroll
    for (int q = 0; q < kQ; q++) {
      const int q0 = 64 * q;
      if (q0 >= na) break;
      const int ai = q0 + lane;
      const int o0 = ai < na ? lo[q] : 0, o1 = ai < na ? lh[q] : 0;
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
          ex = lid[q];
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
      s_tile[3] = rblk_l;
    }
  }
  __syncthreads();
  // block-uniform (read from LDS, so made scalar explicitly: the bounds below then branch on SGPRs)
  const int ex = __builtin_amdgcn_readfirstlane(s_tile[0]), beg = __builtin_amdgcn_readfirstlane(s_tile[1]),
            ncol = __builtin_amdgcn_readfirstlane(s_tile[2]);
  if (ex < 0) {
    if constexpr (kPersist) continue;
    else return;
  }
  const int rblk = __builtin_amdgcn_readfirstlane(s_tile[3]);
  const int tb = rblk * S::kRows / 16;  // first 16-row tile of the block
  const int t0 = tb + wr * RT;           // first 16-row tile of the wavefront
  const uint8_t *rec = a.base + (size_t)ex * a.stride;
  const uint8_t *mat = rec + a.mat_off;
  const PackDims d = a.d;

  // ---- sources. B: piece i of the wavefront = 1 KB piece W i + wv of the step, chunk c =
  //      64 (W i + wv) + lane (entry c / kChunks, 16-byte part c % kChunks of the record
  //      step); padding entries repeat a valid entry; pieces past kGroups land in the unused
  //      tail of the slot's B area. A: the block's WR RT tiles, tile W i + wv by this
  //      wavefront, chunk (step, lane) of each; tiles past the matrix read the last tile
  //      (results not stored); a lane's K-block past the matrix reads an in-range chunk, whose
  //      scale byte is 0 (the packer zero-fills them) while the B records hold zeros there, so
  //      it adds exact zeros. Every lane of every DMA runs, so each wavefront issues exactly
  //      kIssue VMEM operations per step, which the vmcnt waits count on.
  const uint8_t *bsrc[S::kSAddr ? 1 : S::kDma];
  uint32_t boff[S::kSAddr ? S::kDma : 1];  // offsets from a.brec (records < 4 GB)
#pragma unroll
  for (int i = 0; i < S::kDma; i++) {
    const int c = min(64 * (W * i + wv) + lane, S::kStepChunks - 1);
    const int e = c / kChunks, part = c % kChunks;
    const int ge = beg + min(e, ncol - 1);
    const int row = a.entry_src ? a.entry_src[ge] : ge;
    if constexpr (S::kSAddr)
      boff[i] = (uint32_t)row * (uint32_t)G::kBytes + 16u * part;
    else
      bsrc[i] = a.brec + (size_t)row * G::kBytes + 16 * part;
  }
  const uint8_t *asrc[S::kDmaA];  // the wavefront's share of the block's A tiles: W i + wv
  const uint8_t *ssrc[S::kDmaA];
  const size_t last_chunk = (size_t)d.rows * d.nb - 1;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
#pragma unroll
  for (int i = 0; i < S::kDmaA; i++) {
    const int tl = min(tb + W * i + wvu, (int)d.tiles - 1);
    if constexpr (S::kSAddr) {  // tile bases (wavefront-uniform); the lane part is added per step
      asrc[i] = mat + (size_t)tl * 16 * d.nb * 16;
      ssrc[i] = mat + pack_weight_bytes(d) + (size_t)tl * d.nq * 256;
    } else {
      asrc[i] = mat + (size_t)tl * 16 * d.nb * 16;
      ssrc[i] = mat + pack_weight_bytes(d) + (size_t)tl * d.nq * 256 + 4 * lane;
    }
  }
  // the last 16-byte chunk of a tile (with kSAddr, a lane's chunk past it, in the last step, is
  // clamped into the tile: its scale byte is 0 and its B values are 0, so it adds 0)
  const uint32_t a_last = 16u * d.nb * 16u - 16u;
  bool tv[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) tv[r] = t0 + r < (int)d.tiles;
  // wavefront-uniform bound of the B-stationary step: its row tiles inside the matrix
  const int nrt_valid = __builtin_amdgcn_readfirstlane(min(RT, (int)d.tiles - t0));
  const uint8_t *alast = mat + last_chunk * 16;
#define GEMM_LOAD_S(step, sl)                                                                       \
  do {                                                                                              \
    const uint8_t *bb_ = a.brec + (size_t)(step) * G::kStep;                                        \
    _Pragma("unroll") for (int i = 0; i < S::kDma; i++) {                                           \
      /* (the two LDS objects as 32-bit LDS addresses before the select: a select of the generic \
         pointers hit a compiler error in one shape) */                                          \
      lds_dma16_sa(boff[i], bb_, W * i + wvu >= S::kGroups ? lds_addr(s_dummy) : lds_addr((sl) + 1024 * (W * i + wvu))); \
    }                                                                                               \
    const uint32_t ao_ = min((uint32_t)(step) * 1024u + 16u * lane, a_last);                        \
    _Pragma("unroll") for (int i = 0; i < S::kDmaA; i++)                                            \
      lds_dma16_s(ao_, asrc[i], (sl) + S::kBufB + (W * i + wvu) * 1024);                           \
    const uint32_t so_ = (uint32_t)((step) >> 2) * 256u + 4u * lane;                                 \
    _Pragma("unroll") for (int i = 0; i < S::kDmaA; i++)                                            \
      lds_dma4_s(so_, ssrc[i], (sl) + S::kBufB + S::kBufA + (W * i + wvu) * 256);                  \
  } while (0)
// fresh: step is the next step to load (not the repeat of the last one past the end)
#define GEMM_LOAD(step, sl, fresh)                                                                  \
  do {                                                                                              \
    if constexpr (S::kBStat) {                                                                      \
      GEMM_LOAD_S(step, sl);                                                                        \
    } else if constexpr (S::kSAddr && !S::kTwoAhead) { /* the 3-slot ring, scale words per 4 steps */ \
      const uint8_t *bb_ = a.brec + (size_t)(step) * G::kStep;                                      \
      _Pragma("unroll") for (int i = 0; i < S::kDma; i++) {                                         \
        if (W * i + wvu < S::kGroups) lds_dma16_s(boff[i], bb_, (sl) + 1024 * (W * i + wvu));        \
      }                                                                                             \
      const uint32_t ao_ = min((uint32_t)(step) * 1024u + 16u * lane, a_last);                      \
      _Pragma("unroll") for (int i = 0; i < S::kDmaA; i++)                                          \
        lds_dma16_s(ao_, asrc[i], (sl) + S::kBufB + (W * i + wvu) * 1024);                         \
      if ((fresh) && ((step) & 3) == 0) {                                                           \
        const uint32_t so_ = (uint32_t)((step) >> 2) * 256u + 4u * lane;                             \
        _Pragma("unroll") for (int i = 0; i < S::kDmaA; i++)                                        \
          lds_dma4_s(so_, ssrc[i], s_sc[((step) >> 2) & 1] + (W * i + wvu) * 256);                  \
      }                                                                                             \
    } else if constexpr (!S::kTwoAhead) {                                                           \
      _Pragma("unroll") for (int i = 0; i < S::kDma; i++) {                                         \
        if (!S::kScale4 || W * i + wvu < S::kGroups)                                                \
          lds_dma16(bsrc[S::kSAddr ? 0 : i] + (size_t)(step) * G::kStep, (sl) + 1024 * (W * i + wv)); \
      }                                                                                             \
      _Pragma("unroll") for (int i = 0; i < S::kDmaA; i++) {                                        \
        const uint8_t *src = asrc[i] + (size_t)(step) * 1024 + 16 * lane;                           \
        lds_dma16_nt(src < alast ? src : alast, (sl) + S::kBufB + (W * i + wv) * 1024);             \
      }                                                                                             \
      if constexpr (S::kScale4) {                                                                   \
        if ((fresh) && ((step) & 3) == 0) {                                                         \
          _Pragma("unroll") for (int i = 0; i < S::kDmaA; i++)                                      \
            lds_dma4(ssrc[i] + (size_t)((step) >> 2) * 256, s_sc[((step) >> 2) & 1] + (W * i + wv) * 256); \
        }                                                                                           \
      } else {                                                                                      \
        _Pragma("unroll") for (int i = 0; i < S::kDmaA; i++)                                        \
          lds_dma4(ssrc[i] + (size_t)((step) >> 2) * 256, (sl) + S::kBufB + S::kBufA + (W * i + wv) * 256); \
      }                                                                                             \
    }                                                                                               \
  } while (0)

  f32x4 acc[RT][CG];
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int c = 0; c < CG; c++) acc[r][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  f32x16 acc32[M32 ? 4 : 1];  // the 32x32 form's accumulators: row tile R of 32 rows
#pragma unroll
  for (int r = 0; r < (M32 ? 4 : 1); r++) acc32[r] = f32x16{};

  // ---- bias of the wavefront's rows into LDS by DMA before the K loop (complete at the first
  //      wait), read in the epilogue
  const float *bias = reinterpret_cast<const float *>(rec + a.bias_off);
  if constexpr (!S::kBStat) {
#pragma unroll
    for (int k = 0; k < kBiasTiles / 4; k++)
      lds_dma4(bias + min(t0 * 16 + 64 * k + lane, (int)d.rows - 1), s_bias + (wv * kBiasTiles + 4 * k) * 16);
  }

  // ---- K loop, unrolled by D so that each step names its ring slots: step s computes from
  //      slot s % D while steps s + 1 .. s + D - 1 load. Every step issues one step's loads
  //      (past the last step: a repeat of step ns - 1 into the free slot), so the VMEM count is
  //      the same at every step and the wait needs no branch: each step ends with this
  //      wavefront's loads of step s + 1 complete (issued after them: D - 2 steps' loads) and
  //      its LDS reads done, then a barrier: slot (s + 1) % D is whole, slot s % D is free.
  static_assert(D == 2 || D == 3, "ring depth");
  const int ns = (int)d.ns;
  // The wait that ends a step (ld: the step whose loads it issued, fresh: not a repeat): this
  // wavefront's loads of the next step complete, those of step ld (D - 2 steps' loads) in flight.
  // With kScale4 and D = 3 their number is this wavefront's B pieces (the last one only inside
  // kGroups), its A tiles and, for a fresh step that is a multiple of 4, its scale words.
  const bool fullb3 = W * (S::kDma - 1) + wvu < S::kGroups;
#define GEMM_WAIT_AHEAD(ld, fresh)                                                                  \
  do {                                                                                              \
    if constexpr (D == 2) {                                                                         \
      __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));                                                  \
    } else if constexpr (!S::kScale4) {                                                             \
      __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kIssue));                                          \
    } else {                                                                                        \
      const bool sc_ = (fresh) && ((ld) & 3) == 0;                                                  \
      if (fullb3) {                                                                                 \
        if (sc_) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma + 2 * S::kDmaA));                 \
        else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma + S::kDmaA));                         \
      } else {                                                                                      \
        if (sc_) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1 + 2 * S::kDmaA));             \
        else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1 + S::kDmaA));                     \
      }                                                                                             \
    }                                                                                               \
  } while (0)
#define GEMM_STEP(st, cur, nxt)                                                                     \
  do {                                                                                              \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    GEMM_LOAD(min((st) + D - 1, ns - 1), nxt, (st) + D - 1 < ns);                                   \
    if constexpr (S::kBStat) {                                                                      \
      gemm_step_bstat<RT, CGW, WR, WC, D, NT, false>(acc, cur, wr, wc, lane, 8 * ((st) & 3), nrt_valid); \
    } else {                                                                                        \
      if (((st) & 3) == 0) { /* the scale words of steps st .. st + 3 (whole since step st - 1) */  \
        const uint8_t *sb_ = (S::kScale4 ? s_sc[((st) >> 2) & 1] : (cur) + S::kBufB + S::kBufA) + wr * RT * 256; \
        _Pragma("unroll") for (int r_ = 0; r_ < RT; r_++)                                           \
          sw4_[r_] = *reinterpret_cast<const uint32_t *>(sb_ + r_ * 256 + 4 * lane);                \
      }                                                                                             \
      gemm_step<RT, CGW, WR, WC, D, NT>(acc, cur, sw4_, wr, wc, lane, 8 * ((st) & 3));              \
    }                                                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    GEMM_WAIT_AHEAD(min((st) + D - 1, ns - 1), (st) + D - 1 < ns);                                  \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                        \
    __builtin_amdgcn_s_barrier();                                                                   \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                        \
  } while (0)
  if constexpr (S::kTwoAhead) {
    // ---- two steps in flight in the 2-slot ring: step s reads all of its operands from slot
    //      s % 2 into registers, a barrier frees the slot, the slot receives the DMA of step
    //      s + 2 while the MFMAs of step s run, and the step ends when this wavefront's DMA of
    //      step s + 1 is complete (then a barrier: slot (s + 1) % 2 is whole). A step's loads miss
    //      the L2 often enough that one step of prefetch left every step waiting for a miss.
    //      The DMAs of a step, per wavefront: nb B pieces (kDma, or kDma - 1 for the wavefronts
    //      past the step's kGroups pieces), kDmaA A tiles, and kDmaA scale words every 4 steps.
    static_assert(W * (S::kDma - 1) < S::kGroups, "only the last B piece can fall past the step");
    constexpr int kCSplit = CGW / 2;  // column groups computed before the slot is released
    const bool fullb = W * (S::kDma - 1) + wvu < S::kGroups;
    // DMA k of step ld into ring slot sl: 0 = the last B piece (only wavefronts inside kGroups),
    // 1 .. kDma - 1 = the other B pieces, then the A tiles, then the A-scale words (issued only
    // for steps that are multiples of 4, into s_sc)
    auto dma2 = [&](int k, int ld, uint8_t *sl) {
      if (k == 0) {
        if (fullb) lds_dma16_s(boff[S::kDma - 1], a.brec + (size_t)ld * G::kStep, sl + 1024 * (W * (S::kDma - 1) + wvu));
      } else if (k < S::kDma) {
        lds_dma16_s(boff[(k - 1) % S::kDma], a.brec + (size_t)ld * G::kStep, sl + 1024 * (W * (k - 1) + wvu));
      } else if (k < S::kDma + S::kDmaA) {
        const int i = (k - S::kDma) % S::kDmaA;
        lds_dma16_s(min((uint32_t)ld * 1024u + 16u * lane, a_last), asrc[i], sl + S::kBufB + (W * i + wvu) * 1024);
      } else {
        const int i = (k - S::kDma - S::kDmaA) % S::kDmaA;
        lds_dma4_s((uint32_t)(ld >> 2) * 256u + 4u * lane, ssrc[i], s_sc[(ld >> 2) & 1] + (W * i + wvu) * 256);
      }
    };
#define GEMM_VM_WAIT(extra)                                                                         \
  do {                                                                                              \
    if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma + (extra)));                         \
    else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1 + (extra)));                           \
  } while (0)
#define GEMM_BARRIER()                                                                              \
  do {                                                                                              \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                        \
    __builtin_amdgcn_s_barrier();                                                                   \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                        \
  } while (0)
#define GEMM_STEP2(st, cur, jj)                                                                     \
  do {                                                                                              \
    GemmOps<RT, CGW, NT> ops_;                                                                      \
    if ((jj) == 0) {                                                                                \
      _Pragma("unroll") for (int r_ = 0; r_ < RT; r_++)                                             \
        sw4_[r_] = *reinterpret_cast<const uint32_t *>(s_sc[((st) >> 2) & 1] + (wr * RT + r_) * 256 + 4 * lane); \
    }                                                                                               \
    gemm_read_ops<RT, CGW, WR, WC, D, NT, kCSplit>(ops_, cur, sw4_, wr, wc, lane, 8 * (jj));        \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    /* the first column groups' MFMAs run while the other groups' operands arrive */               \
    GemmBRaw<NT> raw_[CGW - kCSplit];                                                               \
    _Pragma("unroll") for (int c_ = kCSplit; c_ < CGW; c_++)                                        \
      gemm_read_b_raw(raw_[c_ - kCSplit], cur + (16 * CGW * wc + (lane & 15) + 16 * c_) * kEntryStep, lane >> 4); \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    gemm_mfma_ops<RT, CGW, NT, 0, kCSplit, 0>(acc, ops_, [](int) {});                               \
    _Pragma("unroll") for (int c_ = kCSplit; c_ < CGW; c_++)                                        \
      gemm_select_b(ops_.b[c_], raw_[c_ - kCSplit], lane >> 4);                                     \
    __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));                                                   \
    GEMM_BARRIER();                                                                                 \
    const int ld_ = (st) + 2;                                                                       \
    auto dma_ = [&](int k_) { dma2(k_, ld_, cur); };                                                \
    if ((st) + 2 < ns)                                                                              \
      gemm_mfma_ops<RT, CGW, NT, kCSplit, CGW, S::kDma + S::kDmaA + ((jj) == 2 ? S::kDmaA : 0)>(acc, ops_, dma_); \
    else                                                                                            \
      gemm_mfma_ops<RT, CGW, NT, kCSplit, CGW, 0>(acc, ops_, dma_);                                 \
    const bool more_ = (st) + 2 < ns;                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    if (more_) GEMM_VM_WAIT(S::kDmaA + ((jj) == 2 ? S::kDmaA : 0));                                 \
    else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));                                               \
    GEMM_BARRIER();                                                                                 \
  } while (0)
    // the A-scale words of the current 4 steps, read from LDS once per 4 steps (their DMA is
    // complete from the step before the first of them until the DMA of the quad after next)
    uint32_t sw4_[RT];
    if constexpr (NSP > 0) {
      // ---- the pipelined step (ns == NSP, every step a constant): a wavefront holds two operand
      //      sets. Step s reads its last column groups' B while its first groups' MFMAs run, then
      //      waits for its reads and for its DMAs of step s + 1, and one barrier makes step s's
      //      ring slots free (every wavefront has read all of step s) and step s + 1's whole. The
      //      last groups' MFMAs then run while the freed slots receive DMAs and the wavefront reads
      //      step s + 1's A chunks and first groups' B into the other set: every LDS read overlaps
      //      MFMAs of the same wavefront, where the plain step reads all its operands between two
      //      barriers before its MFMAs. Same MFMAs in the same order per output, so the same bits.
      //      The A chunks and the B records have rings of their own: both two slots deep (RING 0;
      //      the slots of step s receive step s + 2), or one of them three deep, so that its DMA
      //      has two steps to land. DMAs issued after step s's barrier: RING 0: B(s + 2), A(s + 2);
      //      RING 1: A(s + 2), then B(s + 3); RING 2: B(s + 2), then A(s + 3); the A-scale words of
      //      quad q go with A(4q). The wait before step s's barrier completes A(s + 1) and B(s + 1)
      //      and leaves the deeper ring's step s + 2 in flight. B's last piece (only the wavefronts
      //      inside kGroups load one) is the one DMA issued under a branch: RINGs 0 and 2 issue it
      //      first (before the MFMAs), RING 1 after them.
      constexpr int DA = kRingA, DB = kRingB, kBufBr = S::kGroups * 1024;
      auto slA = [&](int st) { return s_ring + (st % DA) * S::kBufA; };
      auto slB = [&](int st) { return s_ring + DA * S::kBufA + (st % DB) * kBufBr; };
      auto dmaB_last = [&](int ld) {
        if (fullb) lds_dma16_s(boff[S::kDma - 1], a.brec + (size_t)ld * G::kStep, slB(ld) + 1024 * (W * (S::kDma - 1) + wvu));
      };
      auto dmaB = [&](int k, int ld) {  // k < kDma - 1: the unconditional pieces
        lds_dma16_s(boff[k], a.brec + (size_t)ld * G::kStep, slB(ld) + 1024 * (W * k + wvu));
      };
      auto dmaA = [&](int k, int ld) {  // k < kDmaA: A tiles; then the scale words (ld % 4 == 0)
        if (k < S::kDmaA) {
          lds_dma16_s(min((uint32_t)ld * 1024u + 16u * lane, a_last), asrc[k], slA(ld) + (W * k + wvu) * 1024);
        } else {
          const int i = k - S::kDmaA;
          lds_dma4_s((uint32_t)(ld >> 2) * 256u + 4u * lane, ssrc[i], s_sc[(ld >> 2) & 1] + (W * i + wvu) * 256);
        }
      };
      auto nA = [&](int ld) { return ld < NSP ? S::kDmaA + ((ld & 3) == 0 ? S::kDmaA : 0) : 0; };
      auto issueA = [&](int ld) {
        for (int k = 0; k < nA(ld); k++) dmaA(k, ld);
      };
      auto issueB = [&](int ld) {
        if (ld >= NSP) return;
        for (int k = 0; k < S::kDma - 1; k++) dmaB(k, ld);
        dmaB_last(ld);
      };
      // prologue: step 0 whole, steps 1 (and 2 of the deeper ring) in flight, in the order of
      // the loop's groups, so that the first wait counts the same way as every later one
      issueA(0);
      issueB(0);
      if constexpr (RING == 1) {
        issueA(1);
        issueB(1);
        issueB(2);
        if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(nA(1) + 2 * S::kDma));
        else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(nA(1) + 2 * (S::kDma - 1)));
      } else if constexpr (RING == 2) {
        issueB(1);
        issueA(1);
        issueA(2);
        if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma + nA(1) + nA(2)));
        else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1 + nA(1) + nA(2)));
      } else {
        issueB(1);
        issueA(1);
        if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma + nA(1)));
        else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1 + nA(1)));
      }
      GEMM_BARRIER();
      constexpr int kNextA = RT, kNextB = kCSplit * (NT + 1);
      GemmOps<RT, CGW, NT> opE_, opO_;
      GemmBRaw<NT> rbE_[kCSplit], rbO_[kCSplit];
#pragma unroll
      for (int r_ = 0; r_ < RT; r_++) {
        sw4_[r_] = *reinterpret_cast<const uint32_t *>(s_sc[0] + (wr * RT + r_) * 256 + 4 * lane);
        opE_.ar[r_] = *reinterpret_cast<const uint4 *>(slA(0) + (wr * RT + r_) * 1024 + 16 * lane);
        opE_.sw[r_] = sw4_[r_];
      }
#pragma unroll
      for (int c_ = 0; c_ < kCSplit; c_++) gemm_read_b_raw(rbE_[c_], slB(0) + (16 * CGW * wc + j + 16 * c_) * kEntryStep, g);
      str_static_for<0, NSP>([&](auto stc) {
        constexpr int st = decltype(stc)::value;
        GemmOps<RT, CGW, NT> &oc = (st & 1) ? opO_ : opE_;
        GemmOps<RT, CGW, NT> &on = (st & 1) ? opE_ : opO_;
        GemmBRaw<NT>(&rc)[kCSplit] = (st & 1) ? rbO_ : rbE_;
        GemmBRaw<NT>(&rn)[kCSplit] = (st & 1) ? rbE_ : rbO_;
        const uint8_t *bc = slB(st);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c_ = 0; c_ < kCSplit; c_++) gemm_select_b(oc.b[c_], rc[c_], g);
        GemmBRaw<NT> raw_[CGW - kCSplit];
#pragma unroll
        for (int c_ = kCSplit; c_ < CGW; c_++)
          gemm_read_b_raw(raw_[c_ - kCSplit], bc + (16 * CGW * wc + j + 16 * c_) * kEntryStep, g);
        __builtin_amdgcn_sched_barrier(0);
        gemm_mfma_ops<RT, CGW, NT, 0, kCSplit, 0>(acc, oc, [](int) {});
#pragma unroll
        for (int c_ = kCSplit; c_ < CGW; c_++) gemm_select_b(oc.b[c_], raw_[c_ - kCSplit], g);
        // A(st + 1) and B(st + 1) complete; the deeper ring's step st + 2 may stay in flight
        if constexpr (RING == 1) {
          if constexpr (st + 2 < NSP) {
            if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma));
            else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1));
          } else {
            __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));
          }
        } else if constexpr (RING == 2) {
          constexpr int kOut = st + 2 < NSP ? S::kDmaA + (((st + 2) & 3) == 0 ? S::kDmaA : 0) : 0;
          __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(kOut));
        } else {
          __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));
        }
        GEMM_BARRIER();
        // hooks: this step's DMA group (RING 1: A(st + 2), B(st + 3)'s unconditional pieces;
        // RINGs 0 and 2: B, then A, into the slots just freed), then the reads of step st + 1's set
        constexpr int ldA = st + DA, ldB = st + DB;
        constexpr int kNA = ldA < NSP ? S::kDmaA + ((ldA & 3) == 0 ? S::kDmaA : 0) : 0;
        constexpr int kNB = ldB < NSP ? (RING == 1 ? S::kDma - 1 : S::kDma) : 0;
        constexpr int kD = kNA + kNB;
        constexpr int kR = st + 1 < NSP ? kNextA + kNextB : 0;
        constexpr int sh = 8 * ((st + 1) & 3);
        const uint8_t *nb = slB(st + 1) + (16 * CGW * wc + j) * kEntryStep;
        const uint8_t *na = slA(st + 1) + wr * RT * 1024;
        auto hook = [&](int k_) {
          if (k_ < kD) {
            if constexpr (RING == 1) {
              if (k_ < kNA) dmaA(k_, ldA);
              else dmaB(k_ - kNA, ldB);
            } else {
              if (k_ == 0) dmaB_last(ldB);  // (the branch: before the MFMAs)
              else if (k_ < kNB) dmaB(k_ - 1, ldB);
              else dmaA(k_ - kNB, ldA);
            }
          } else if (k_ - kD < kNextA) {
            const int r_ = k_ - kD;
            if (((st + 1) & 3) == 0)
              sw4_[r_] = *reinterpret_cast<const uint32_t *>(s_sc[((st + 1) >> 2) & 1] + (wr * RT + r_) * 256 + 4 * lane);
            on.ar[r_] = *reinterpret_cast<const uint4 *>(na + r_ * 1024 + 16 * lane);
            on.sw[r_] = sw4_[r_] >> sh;
          } else {
            const int i_ = k_ - kD - kNextA, c_ = i_ / (NT + 1), t_ = i_ % (NT + 1);
            const uint8_t *eb = nb + 16 * c_ * kEntryStep;
            if (t_ < NT) {
              rn[c_].x[t_] = *reinterpret_cast<const uint4 *>(eb + (6 * t_ + g) * 16);
              rn[c_].y[t_] = *reinterpret_cast<const uint4 *>(eb + (6 * t_ + 4 + (g >> 1)) * 16);
            } else if constexpr (NT == 1) {
              rn[c_].sc[0] = *reinterpret_cast<const uint32_t *>(eb + (G::kChunks - 1) * 16);
            } else {
              const uint4 sc = *reinterpret_cast<const uint4 *>(eb + (G::kChunks - 1) * 16);
              const uint32_t w3[3] = {sc.x, sc.y, sc.z};
#pragma unroll
              for (int q_ = 0; q_ < NT; q_++) rn[c_].sc[q_] = w3[q_];
            }
          }
        };
        gemm_mfma_ops<RT, CGW, NT, kCSplit, CGW, kD + kR>(acc, oc, hook);
        if constexpr (RING == 1 && ldB < NSP) dmaB_last(ldB);
      });
    } else {
    constexpr int kAll = S::kDma + 2 * S::kDmaA;  // the DMAs of a step whose scale words load
#pragma unroll
    for (int k = 0; k < kAll; k++) dma2(k, 0, s_r0);
    if (ns > 1) {
#pragma unroll
      for (int k = 0; k < kAll - S::kDmaA; k++) dma2(k, 1, s_r1);
      GEMM_VM_WAIT(S::kDmaA);
    } else {
      __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));
    }
    GEMM_BARRIER();
    if constexpr (M32) {
      uint32_t sw32_[4][2];
#define GEMM_STEP32(st, cur, jj)                                                                    \
  do {                                                                                              \
    Gemm32Ops<NT> ops_;                                                                             \
    if ((jj) == 0) gemm32_read_sw4<RT>(sw32_, s_sc[((st) >> 2) & 1], wr, lane);                     \
    gemm32_read_ops<RT, NT, S::kBufB>(ops_, cur, sw32_, wr, wc, lane, 8 * (jj));                    \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    gemm32_mfma_half<NT, 0, 0>(acc32, ops_, [](int) {});                                            \
    __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));                                                   \
    GEMM_BARRIER();                                                                                 \
    const int ld_ = (st) + 2;                                                                       \
    auto dma_ = [&](int k_) { dma2(k_, ld_, cur); };                                                \
    if ((st) + 2 < ns)                                                                              \
      gemm32_mfma_half<NT, 1, S::kDma + S::kDmaA + ((jj) == 2 ? S::kDmaA : 0)>(acc32, ops_, dma_);  \
    else                                                                                            \
      gemm32_mfma_half<NT, 1, 0>(acc32, ops_, dma_);                                                \
    const bool more_ = (st) + 2 < ns;                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    if (more_) GEMM_VM_WAIT(S::kDmaA + ((jj) == 2 ? S::kDmaA : 0));                                 \
    else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));                                               \
    GEMM_BARRIER();                                                                                 \
  } while (0)
      for (int s = 0; s < ns; s += 4) {
        GEMM_STEP32(s, s_r0, 0);
        if (s + 1 < ns) GEMM_STEP32(s + 1, s_r1, 1);
        if (s + 2 < ns) GEMM_STEP32(s + 2, s_r0, 2);
        if (s + 3 < ns) GEMM_STEP32(s + 3, s_r1, 3);
      }
#undef GEMM_STEP32
    } else {
    for (int s = 0; s < ns; s += 4) {
      GEMM_STEP2(s, s_r0, 0);
      if (s + 1 < ns) GEMM_STEP2(s + 1, s_r1, 1);
      if (s + 2 < ns) GEMM_STEP2(s + 2, s_r0, 2);
      if (s + 3 < ns) GEMM_STEP2(s + 3, s_r1, 3);
    }
    }
    }  // NSP == 0
#undef GEMM_STEP2
#undef GEMM_BARRIER
#undef GEMM_VM_WAIT
  } else {
  uint32_t sw4_[RT];  // the A-scale words of the current 4 steps (gemm_step)
  GEMM_LOAD(0, s_r0, true);
  if (D == 3) GEMM_LOAD(min(1, ns - 1), s_r1, true);
  GEMM_WAIT_AHEAD(min(1, ns - 1), true);
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
  }
#undef GEMM_STEP
#undef GEMM_WAIT_AHEAD
#undef GEMM_LOAD
#undef GEMM_LOAD_S

  // ---- epilogue
  float4 bv[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) {
    if constexpr (S::kBStat)
      bv[r] = *reinterpret_cast<const float4 *>(bias + min(t0 + r, (int)d.tiles - 1) * 16 + 4 * g);
    else
      bv[r] = *reinterpret_cast<const float4 *>(s_bias + (wv * kBiasTiles + r) * 16 + 4 * g);
  }
  if constexpr (MODE == GEMV_GATE_UP) {
    // every 4 row tiles (64 rows) of the wavefront = h block hb (h values 32 hb .. 32 hb + 31)
    // of its entries. The SwiGLU values are staged in the (now free) ring as f32 [entry][32];
    // then lane 2 e + h takes half h of entry e's block: the NT E2M3 terms of its 16
    // values (block maximum shared with the neighbouring lane) go to the h record.
    static_assert(RT % 4 == 0, "whole h blocks per wavefront");
    constexpr int kWaveCols = 16 * CGW;  // entries of the wavefront
    static_assert(kWaveCols <= 32 || kWaveCols == 64, "one or two passes of 64 lanes");
    // staging rows of kRow floats (36, not 32: 16 consecutive rows' 16-byte reads then hit
    // distinct banks, and their 8-byte writes two ways at most)
    constexpr int kRow = 36;
    static_assert(W <= 8 && (W < 4 ? W : 4) * kWaveCols * kRow * 4 <= S::kSlot, "staging fits in two ring slots");
    // with D = 3 the loop ends with one step's loads (the repeat of the last step) still in
    // flight into a ring slot, which may be a staging slot: every wavefront's loads complete
    // before any wavefront stages
    if constexpr (D > 2) {
      __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    uint8_t *hout = reinterpret_cast<uint8_t *>(a.out);
    const int e0 = kWaveCols * wc;                                     // first entry of the wavefront
    const int nloc = max(0, min(kWaveCols, ncol - e0));                // its entries in the tile
    // All of the wavefront's h blocks staged at once when they fit (rows of 36 floats: the
    // 16-byte reads of 16 consecutive rows then hit distinct banks), then one lane per (h block,
    // entry) splits the whole 32-value block (split32_fp6: a third fewer instructions than two
    // 16-value halves) and stores each term's 24 bytes as one 16- and one 8-byte store.
    constexpr int NHB = RT / 4;                        // h blocks of the wavefront
    constexpr int kStageW = NHB * kWaveCols * kRow * 4;  // staging bytes per wavefront
    constexpr int kHalf = W > 1 ? W / 2 : 1;           // wavefronts per ring slot
    if constexpr (kHalf * kStageW <= S::kSlot && NHB * kWaveCols <= 64) {  // one lane pass
      float *st32 = NSP ? reinterpret_cast<float *>(s_ring + wv * kStageW)
                        : reinterpret_cast<float *>((wv < kHalf ? s_r0 : s_r1) + (wv % kHalf) * kStageW);
      static_assert(!NSP || W * kStageW <= kRingBytes, "staging fits the rings");
#pragma unroll
      for (int hbk = 0; hbk < NHB; hbk++) {
        if (!tv[4 * hbk]) break;  // the matrix has whole h blocks (rows % 64 == 0)
        if constexpr (M32) {
          // h block hbk = the wavefront's 32-row tiles 2 hbk, 2 hbk + 1; lane (entry l % 32, u =
          // l / 32) holds rows 8 v + 4 u .. +3 of each (v = 0..3): h values 16 Rr + 4 v + 2 u, + 1
          if (nloc <= 0) break;
          const int e32 = lane & 31, u = lane >> 5;
          float *se = st32 + (hbk * kWaveCols + e32) * kRow;
#pragma unroll
          for (int Rr = 0; Rr < 2; Rr++) {
            const f32x16 &av = acc32[2 * hbk + Rr];
#pragma unroll
            for (int v = 0; v < 4; v++) {  // rows 32 R + 8 v + 4 u: tile16 chunk 2 R + v / 2, row 8 (v % 2) + 4 u
              const float4 b4 = *reinterpret_cast<const float4 *>(
                  s_bias + (wv * kBiasTiles + 4 * hbk + 2 * Rr + v / 2) * 16 + 8 * (v % 2) + 4 * u);
              *reinterpret_cast<float2 *>(se + 16 * Rr + 4 * v + 2 * u) =
                  make_float2(swiglu_fast(av[4 * v] + b4.x, av[4 * v + 1] + b4.y, a.limit),
                              swiglu_fast(av[4 * v + 2] + b4.z, av[4 * v + 3] + b4.w, a.limit));
            }
          }
        } else {
#pragma unroll
        for (int c = 0; c < CG; c++) {
          if (16 * c >= nloc) break;
          float *se = st32 + (hbk * kWaveCols + 16 * c + j) * kRow;
#pragma unroll
          for (int r = 0; r < 4; r++) {  // h values 8r + 2g, 8r + 2g + 1 of the block
            const f32x4 &av = acc[4 * hbk + r][c];
            const float4 &b4 = bv[4 * hbk + r];
            *reinterpret_cast<float2 *>(se + 8 * r + 2 * g) =
                make_float2(swiglu_fast(av[0] + b4.x, av[1] + b4.y, a.limit), swiglu_fast(av[2] + b4.z, av[3] + b4.w, a.limit));
          }
        }
        }
      }
      constexpr int kPairs = NHB * kWaveCols;
#pragma unroll
      for (int pass = 0; pass < (kPairs + 63) / 64; pass++) {
        const int idx = 64 * pass + lane, hbk = min(idx / kWaveCols, NHB - 1), e = idx % kWaveCols;
        const bool valid = idx < kPairs && tv[4 * hbk] && e < nloc;
        const float *row = st32 + (valid ? hbk * kWaveCols + e : 0) * kRow;
        float v[32];
#pragma unroll
        for (int q = 0; q < 8; q++) {
          const float4 x = *reinterpret_cast<const float4 *>(row + 4 * q);
          v[4 * q] = x.x;
          v[4 * q + 1] = x.y;
          v[4 * q + 2] = x.z;
          v[4 * q + 3] = x.w;
        }
        float m = 0.0f;
        bool bad = false;
#pragma unroll
        for (int k = 0; k < 32; k++) {
          m = fmaxf(m, fabsf(v[k]));
          bad = bad || !isfinite(v[k]);
        }
        uint32_t dq[NT][6], sb;
        split32_fp6<NT>(v, m, bad, dq, sb);
        if (valid) {
          const int hb = t0 / 4 + hbk, st = hb >> 2, i = hb & 3;
          uint8_t *hr = hout + (size_t)(beg + e0 + e) * G::kBytes;
#pragma unroll
          for (int t = 0; t < NT; t++) {
            *reinterpret_cast<uint4 *>(hr + G::dword(st, t, i, 0)) = make_uint4(dq[t][0], dq[t][1], dq[t][2], dq[t][3]);
            *reinterpret_cast<uint2 *>(hr + G::dword(st, t, i, 4)) = make_uint2(dq[t][4], dq[t][5]);
            hr[G::scale(st, t) + i] = (uint8_t)(sb >> (8 * t));
          }
        }
      }
    } else {
    float *stage = reinterpret_cast<float *>((wv < 4 ? s_r0 : s_r1) + (wv & 3) * kWaveCols * kRow * 4);
#pragma unroll
    for (int hbk = 0; hbk < RT / 4; hbk++) {
      if (!tv[4 * hbk]) break;  // the matrix has whole h blocks (rows % 64 == 0)
      const int hb = t0 / 4 + hbk;
#pragma unroll
      for (int c = 0; c < CG; c++) {
        if (16 * c >= nloc) break;
        float *se = stage + (16 * c + j) * kRow;
#pragma unroll
        for (int r = 0; r < 4; r++) {  // h values 8r + 2g, 8r + 2g + 1 of the block
          const f32x4 &av = acc[4 * hbk + r][c];
          const float4 &b4 = bv[4 * hbk + r];
          *reinterpret_cast<float2 *>(se + 8 * r + 2 * g) =
              make_float2(swiglu_fast(av[0] + b4.x, av[1] + b4.y, a.limit), swiglu_fast(av[2] + b4.z, av[3] + b4.w, a.limit));
        }
      }
      const int st = hb >> 2, i = hb & 3;
#pragma unroll
      for (int pass = 0; pass < (kWaveCols + 31) / 32; pass++) {
        const int e = 32 * pass + (lane >> 1), h = lane & 1;
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float4 x = *reinterpret_cast<const float4 *>(stage + min(e, kWaveCols - 1) * kRow + 16 * h + 4 * q);
          v[4 * q] = x.x;
          v[4 * q + 1] = x.y;
          v[4 * q + 2] = x.z;
          v[4 * q + 3] = x.w;
        }
        float m = 0.0f, bad = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) {
          m = fmaxf(m, fabsf(v[k]));
          if (!isfinite(v[k])) bad = 1.0f;
        }
        m = fmaxf(m, xor_lane<1>(m));
        bad = fmaxf(bad, xor_lane<1>(bad));
        uint32_t dq[NT][3], sb;
        split16_fp6<NT>(v, m, bad != 0.0f, dq, sb);
        if (e < nloc) {
          uint8_t *hr = hout + (size_t)(beg + e0 + e) * G::kBytes;
#pragma unroll
          for (int t = 0; t < NT; t++) {
#pragma unroll
            for (int u = 0; u < 3; u++) *reinterpret_cast<uint32_t *>(hr + G::dword(st, t, i, 3 * h + u)) = dq[t][u];
          }
          if (h == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) hr[G::scale(st, t) + i] = (uint8_t)(sb >> (8 * t));
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));  // staging reads done before the next h block
    }
    }
  } else {
    float *out = reinterpret_cast<float *>(a.out);
    const int R = (int)d.rows;
    if constexpr (M32) {
      // lane (entry l % 32, u = l / 32): rows 32 Rt + 8 v + 4 u .. +3 of the wavefront (tile16 chunk
      // 2 Rt + v / 2, inside the matrix or not as a whole)
      const int e = 32 * wc + (lane & 31), u = lane >> 5;
      if (e < ncol) {
#pragma unroll
        for (int Rt = 0; Rt < 4; Rt++) {
#pragma unroll
          for (int v = 0; v < 4; v++) {
            const int ch = 2 * Rt + v / 2;
            if (!tv[ch]) continue;
            const float4 b4 = *reinterpret_cast<const float4 *>(s_bias + (wv * kBiasTiles + ch) * 16 + 8 * (v % 2) + 4 * u);
            const f32x16 &av = acc32[Rt];
            float4 o;
            o.x = canon_nan(rclamp(av[4 * v] + b4.x, -65504.0f, 65504.0f));
            o.y = canon_nan(rclamp(av[4 * v + 1] + b4.y, -65504.0f, 65504.0f));
            o.z = canon_nan(rclamp(av[4 * v + 2] + b4.z, -65504.0f, 65504.0f));
            o.w = canon_nan(rclamp(av[4 * v + 3] + b4.w, -65504.0f, 65504.0f));
            *reinterpret_cast<float4 *>(out + (size_t)(beg + e) * R + (t0 + ch) * 16 + 8 * (v % 2) + 4 * u) = o;
          }
        }
      }
    } else {
#pragma unroll
    for (int r = 0; r < RT; r++) {
      if (!tv[r]) continue;
      const float4 b4 = bv[r];
      const int row = (t0 + r) * 16 + 4 * g;
#pragma unroll
      for (int c = 0; c < CG; c++) {
        const int e = 16 * (CGW * wc + c) + j;
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
    if constexpr (!kPersist) break;  // (no loop at all in the other shapes' code)
  }  // workgroup p
}

// ------------------------------------------------------------------ the pipelined step on a
// persistent grid with a tile queue
//
// k_gemm_fp8's pipelined 512 x 64 step (NSP K-steps, rings RING) on one workgroup per CU that takes
// its tiles from a queue in device memory, a.queue: [0, 8) the counters of the XCDs' ranges of the
// banded tile order, [8] the counter of the plain order, [9] the workgroups done; all zero between
// launches (the last workgroup to finish clears them). One workgroup per tile pays, per tile, the
// tile search, the first DMAs' round trip and the workgroup turnover after the epilogue (measured at
// prefill: 1.1, 2.3 and 2.3 us for gate_up, 1.1, 4.2 and 0.8 us for down, against ~30 us of steps).
// Here they overlap: wavefront 0 takes and searches tile i + 1 while the DMAs of tile i's first
// steps are in flight, and tile i + 1's bias and first steps' DMAs are issued inside tile i's
// epilogue as soon as the ring is free (down: at its start; gate_up: once the SwiGLU values staged
// in the ring have been read back). Same steps and epilogue as k_gemm_fp8: bit-identical results.
// GLOBALQ: one queue in the plain order (row blocks fastest) whatever a.band asks.
__device__ __forceinline__ void pq_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int MODE, int NSP, int RING, bool GLOBALQ>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_pq(GemmArgs a) {
  constexpr int RT = 8, CGW = 2, WR = 4, WC = 2, D = 2, NT = kGemmTerms;
  using S = GemmShape<RT, CGW, WR, WC, D, NT>;
  static_assert(S::kTwoAhead && S::kSAddr && NSP >= 4 && NSP <= kGemmNs, "the pipelined 512 x 64 step");
  constexpr int kRingA = RING == 2 ? 3 : 2, kRingB = RING == 1 ? 3 : 2;
  constexpr int kRingBytes = kRingA * S::kBufA + kRingB * S::kGroups * 1024;
  using G = GemmRecT<NT>;
  constexpr int W = S::W, CG = CGW, kEntryStep = G::kStep;
  constexpr int kCSplit = CGW / 2;
  constexpr int kBiasTiles = RT;
  __shared__ __attribute__((aligned(1024))) uint8_t s_ring[kRingBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t s_sc[2][S::kTilesA * 256];
  __shared__ __attribute__((aligned(16))) float s_bias[W * kBiasTiles * 16];
  __shared__ int s_tile[2][4];  // tile i in s_tile[i & 1]: expert record index (-1: none), first entry, entries, row block
  __shared__ int s_off[kMaxExperts + 1], s_id[kMaxExperts];  // the launch's expert lists
  // lane and its parts are redefined (opaquely) at the top of every tile, so that the compiler
  // does not hoist the steps' lane-dependent LDS addresses out of the tile loop and keep them live
  const int tid = threadIdx.x, wv = tid >> 6;
  int lane = tid & 63;
  const int wr = wv % WR, wc = wv / WR;
  int j = lane & 15, g = lane >> 4;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  const PackDims d = a.d;
  const int band = GLOBALQ ? 0 : a.band;
  const int xcd = (int)blockIdx.x % 8;  // (workgroups go to the XCDs round-robin)
  int *const ctr = a.queue + (band ? xcd : 8);

  // ---- the expert lists into LDS once; the launch's tiles: n_real = row blocks x the column tiles
  //      the experts' entries fill (kCols entries each), in k_gemm_fp8's orders over those
  const int ma = min(a.max_active, kMaxExperts);
  for (int i = tid; i <= ma; i += 64 * W) s_off[i] = a.active_off[i];
  for (int i = tid; i < ma; i += 64 * W) s_id[i] = a.active_ids[i];
  const int na = min(*a.n_active, ma);
  __syncthreads();
  constexpr int kQ = (kMaxExperts + 63) / 64;
  int nct_real = 0;
#pragma unroll
  for (int qq = 0; qq < kQ; qq++) {
    const int ai = 64 * qq + lane;
    const int n = ai < na ? (s_off[ai + 1] - s_off[ai] + S::kCols - 1) / S::kCols : 0;
    int v = n;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
    nct_real += v;
  }
  nct_real = __builtin_amdgcn_readfirstlane(nct_real);
  const int nrb = a.n_row_blocks, n_real = nrb * nct_real;

  // ---- wavefront 0: take a queue position (its atomic is issued a tile before the position is
  //      used, so its round trip stays off the path); the tile at queue position q, its expert,
  //      entries and row block into dst (expert -1: the queue is exhausted)
  auto take = [&]() {
    int q = 0;
    if (lane == 0) q = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return q;
  };
  auto find_next = [&](int qv, int *dst) {
    const int q = __builtin_amdgcn_readfirstlane(__shfl(qv, 0));
    const int C = (n_real + 7) / 8;
    const int L = band ? (q < C ? xcd * C + q : n_real) : q;
    int ex = -1, beg = 0, cnt = 0, rblk_l = 0;
    if (L < n_real) {
      int cl;
      const int nct = nct_real, RB = band ? min(band, nrb) : nrb, full = nrb / RB;
      if (L < full * RB * nct) {
        const int bd = L / (RB * nct), r = L - bd * RB * nct;
        cl = r / RB;
        rblk_l = bd * RB + r % RB;
      } else {
        const int rem = nrb - full * RB, r = L - full * RB * nct;
        cl = r / rem;
        rblk_l = full * RB + r % rem;
      }
      int base = 0;
#pragma unroll
      for (int qq = 0; qq < kQ; qq++) {
        const int q0 = 64 * qq;
        if (q0 >= na) break;
        const int ai = q0 + lane;
        const int o0 = ai < na ? s_off[ai] : 0, o1 = ai < na ? s_off[ai + 1] : 0;
        const int nct_e = (o1 - o0 + S::kCols - 1) / S::kCols;
        int incl = nct_e;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int v = __shfl_up(incl, o);
          if (lane >= o) incl += v;
        }
        const int start = base + incl - nct_e;
        const uint64_t hit = __ballot(ai < na && cl >= start && cl < start + nct_e);
        if (hit) {
          const int hl = __builtin_ctzll(hit);
          if (lane == hl) {
            ex = s_id[ai];
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
    }
    if (lane == 0) {
      dst[0] = ex;
      dst[1] = beg;
      dst[2] = cnt;
      dst[3] = rblk_l;
    }
  };

  // ---- per tile: the DMA sources (as in k_gemm_fp8) and the epilogue's bounds
  int ex, beg, ncol, t0;
  const uint8_t *rec, *mat;
  uint32_t boff[S::kDma];
  const uint8_t *asrc[S::kDmaA];
  const uint8_t *ssrc[S::kDmaA];
  // set_tile in two parts: the tile's bounds and its entries' record rows (loads, issued early),
  // then the DMA sources once the rows are needed
  int rowv[S::kDma];
  int tb = 0;
  auto load_tile = [&](const int *src) {
    ex = __builtin_amdgcn_readfirstlane(src[0]);
    beg = __builtin_amdgcn_readfirstlane(src[1]);
    ncol = __builtin_amdgcn_readfirstlane(src[2]);
    const int rblk = __builtin_amdgcn_readfirstlane(src[3]);
    if (ex < 0) return;
    tb = rblk * S::kRows / 16;
    t0 = tb + wr * RT;
    rec = a.base + (size_t)ex * a.stride;
    mat = rec + a.mat_off;
#pragma unroll
    for (int i = 0; i < S::kDma; i++) {
      const int c = min(64 * (W * i + wv) + lane, S::kStepChunks - 1);
      const int ge = beg + min(c / G::kChunks, ncol - 1);
      rowv[i] = a.entry_src ? a.entry_src[ge] : ge;
    }
  };
  auto set_tile = [&]() {
    if (ex < 0) return;
#pragma unroll
    for (int i = 0; i < S::kDma; i++) {
      const int c = min(64 * (W * i + wv) + lane, S::kStepChunks - 1);
      boff[i] = (uint32_t)rowv[i] * (uint32_t)G::kBytes + 16u * (c % G::kChunks);
    }
#pragma unroll
    for (int i = 0; i < S::kDmaA; i++) {
      const int tl = min(tb + W * i + wvu, (int)d.tiles - 1);
      asrc[i] = mat + (size_t)tl * 16 * d.nb * 16;
      ssrc[i] = mat + pack_weight_bytes(d) + (size_t)tl * d.nq * 256;
    }
  };
  const uint32_t a_last = 16u * d.nb * 16u - 16u;
  const bool fullb = W * (S::kDma - 1) + wvu < S::kGroups;
  static_assert(W * (S::kDma - 1) < S::kGroups, "only the last B piece can fall past the step");

  constexpr int DA = kRingA, DB = kRingB, kBufBr = S::kGroups * 1024;
  auto slA = [&](int st) { return s_ring + (st % DA) * S::kBufA; };
  auto slB = [&](int st) { return s_ring + DA * S::kBufA + (st % DB) * kBufBr; };
  auto dmaB_last = [&](int ld) {
    if (fullb) lds_dma16_s(boff[S::kDma - 1], a.brec + (size_t)ld * G::kStep, slB(ld) + 1024 * (W * (S::kDma - 1) + wvu));
  };
  auto dmaB = [&](int k, int ld) {
    lds_dma16_s(boff[k], a.brec + (size_t)ld * G::kStep, slB(ld) + 1024 * (W * k + wvu));
  };
  auto dmaA = [&](int k, int ld) {
    if (k < S::kDmaA) {
      lds_dma16_s(min((uint32_t)ld * 1024u + 16u * lane, a_last), asrc[k], slA(ld) + (W * k + wvu) * 1024);
    } else {
      const int i = k - S::kDmaA;
      lds_dma4_s((uint32_t)(ld >> 2) * 256u + 4u * lane, ssrc[i], s_sc[(ld >> 2) & 1] + (W * i + wvu) * 256);
    }
  };
  auto nA = [&](int ld) { return ld < NSP ? S::kDmaA + ((ld & 3) == 0 ? S::kDmaA : 0) : 0; };
  auto issueA = [&](int ld) {
    for (int k = 0; k < nA(ld); k++) dmaA(k, ld);
  };
  auto issueB = [&](int ld) {
    if (ld >= NSP) return;
    for (int k = 0; k < S::kDma - 1; k++) dmaB(k, ld);
    dmaB_last(ld);
  };
  // the tile's bias (into the wavefront's part of s_bias) and the DMAs of its first steps, in the
  // order of k_gemm_fp8's prologue
  auto issue_first = [&]() {
    const float *bias = reinterpret_cast<const float *>(rec + a.bias_off);
#pragma unroll
    for (int k = 0; k < kBiasTiles / 4; k++)
      lds_dma4(bias + min(t0 * 16 + 64 * k + lane, (int)d.rows - 1), s_bias + (wv * kBiasTiles + 4 * k) * 16);
    issueA(0);
    issueB(0);
    if constexpr (RING == 1) {
      issueA(1);
      issueB(1);
      issueB(2);
    } else if constexpr (RING == 2) {
      issueB(1);
      issueA(1);
      issueA(2);
    } else {
      issueB(1);
      issueA(1);
    }
  };

  int qn = 0;  // wavefront 0: the queue position of the tile after the next
  if (wv == 0) {
    find_next(take(), s_tile[0]);
    qn = take();
  }
  __syncthreads();
  load_tile(s_tile[0]);
  set_tile();
  if (ex >= 0) issue_first();
  for (int it = 0; ex >= 0; it++) {
    asm volatile("" : "+v"(lane), "+v"(j), "+v"(g));
    if (wv == 0) find_next(qn, s_tile[(it + 1) & 1]);  // read by every wavefront after the barrier below
    // step 0 whole, the deeper ring's steps in flight (whatever the previous epilogue stored
    // after them is waited for too: loads and stores complete in order)
    if constexpr (RING == 1) {
      if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(nA(1) + 2 * S::kDma));
      else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(nA(1) + 2 * (S::kDma - 1)));
    } else if constexpr (RING == 2) {
      if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma + nA(1) + nA(2)));
      else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1 + nA(1) + nA(2)));
    } else {
      if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma + nA(1)));
      else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1 + nA(1)));
    }
    pq_barrier();
    f32x4 acc[RT][CG];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int c = 0; c < CG; c++) acc[r][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t sw4_[RT];
    {
      constexpr int kNextA = RT, kNextB = kCSplit * (NT + 1);
      GemmOps<RT, CGW, NT> opE_, opO_;
      GemmBRaw<NT> rbE_[kCSplit], rbO_[kCSplit];
#pragma unroll
      for (int r_ = 0; r_ < RT; r_++) {
        sw4_[r_] = *reinterpret_cast<const uint32_t *>(s_sc[0] + (wr * RT + r_) * 256 + 4 * lane);
        opE_.ar[r_] = *reinterpret_cast<const uint4 *>(slA(0) + (wr * RT + r_) * 1024 + 16 * lane);
        opE_.sw[r_] = sw4_[r_];
      }
#pragma unroll
      for (int c_ = 0; c_ < kCSplit; c_++) gemm_read_b_raw(rbE_[c_], slB(0) + (16 * CGW * wc + j + 16 * c_) * kEntryStep, g);
      str_static_for<0, NSP>([&](auto stc) {
        constexpr int st = decltype(stc)::value;
        GemmOps<RT, CGW, NT> &oc = (st & 1) ? opO_ : opE_;
        GemmOps<RT, CGW, NT> &on = (st & 1) ? opE_ : opO_;
        GemmBRaw<NT>(&rc)[kCSplit] = (st & 1) ? rbO_ : rbE_;
        GemmBRaw<NT>(&rn)[kCSplit] = (st & 1) ? rbE_ : rbO_;
        const uint8_t *bc = slB(st);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c_ = 0; c_ < kCSplit; c_++) gemm_select_b(oc.b[c_], rc[c_], g);
        GemmBRaw<NT> raw_[CGW - kCSplit];
#pragma unroll
        for (int c_ = kCSplit; c_ < CGW; c_++)
          gemm_read_b_raw(raw_[c_ - kCSplit], bc + (16 * CGW * wc + j + 16 * c_) * kEntryStep, g);
        __builtin_amdgcn_sched_barrier(0);
        gemm_mfma_ops<RT, CGW, NT, 0, kCSplit, 0>(acc, oc, [](int) {});
#pragma unroll
        for (int c_ = kCSplit; c_ < CGW; c_++) gemm_select_b(oc.b[c_], raw_[c_ - kCSplit], g);
        if constexpr (RING == 1) {
          if constexpr (st + 2 < NSP) {
            if (fullb) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma));
            else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(S::kDma - 1));
          } else {
            __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));
          }
        } else if constexpr (RING == 2) {
          constexpr int kOut = st + 2 < NSP ? S::kDmaA + (((st + 2) & 3) == 0 ? S::kDmaA : 0) : 0;
          __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(kOut));
        } else {
          __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));
        }
        pq_barrier();
        constexpr int ldA = st + DA, ldB = st + DB;
        constexpr int kNA = ldA < NSP ? S::kDmaA + ((ldA & 3) == 0 ? S::kDmaA : 0) : 0;
        constexpr int kNB = ldB < NSP ? (RING == 1 ? S::kDma - 1 : S::kDma) : 0;
        constexpr int kD = kNA + kNB;
        constexpr int kR = st + 1 < NSP ? kNextA + kNextB : 0;
        constexpr int sh = 8 * ((st + 1) & 3);
        const uint8_t *nb = slB(st + 1) + (16 * CGW * wc + j) * kEntryStep;
        const uint8_t *na = slA(st + 1) + wr * RT * 1024;
        auto hook = [&](int k_) {
          if (k_ < kD) {
            if constexpr (RING == 1) {
              if (k_ < kNA) dmaA(k_, ldA);
              else dmaB(k_ - kNA, ldB);
            } else {
              if (k_ == 0) dmaB_last(ldB);
              else if (k_ < kNB) dmaB(k_ - 1, ldB);
              else dmaA(k_ - kNB, ldA);
            }
          } else if (k_ - kD < kNextA) {
            const int r_ = k_ - kD;
            if (((st + 1) & 3) == 0)
              sw4_[r_] = *reinterpret_cast<const uint32_t *>(s_sc[((st + 1) >> 2) & 1] + (wr * RT + r_) * 256 + 4 * lane);
            on.ar[r_] = *reinterpret_cast<const uint4 *>(na + r_ * 1024 + 16 * lane);
            on.sw[r_] = sw4_[r_] >> sh;
          } else {
            const int i_ = k_ - kD - kNextA, c_ = i_ / (NT + 1), t_ = i_ % (NT + 1);
            const uint8_t *eb = nb + 16 * c_ * kEntryStep;
            if (t_ < NT) {
              rn[c_].x[t_] = *reinterpret_cast<const uint4 *>(eb + (6 * t_ + g) * 16);
              rn[c_].y[t_] = *reinterpret_cast<const uint4 *>(eb + (6 * t_ + 4 + (g >> 1)) * 16);
            } else {
              const uint4 sc = *reinterpret_cast<const uint4 *>(eb + (G::kChunks - 1) * 16);
              const uint32_t w3[3] = {sc.x, sc.y, sc.z};
#pragma unroll
              for (int q_ = 0; q_ < NT; q_++) rn[c_].sc[q_] = w3[q_];
            }
          }
        };
        gemm_mfma_ops<RT, CGW, NT, kCSplit, CGW, kD + kR>(acc, oc, hook);
        if constexpr (RING == 1 && ldB < NSP) dmaB_last(ldB);
      });
    }

    // ---- epilogue of this tile; the next tile's first DMAs as soon as the ring is free
    const int cex = ex, cbeg = beg, cncol = ncol, ct0 = t0;
    bool tv[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) tv[r] = ct0 + r < (int)d.tiles;
    float4 bv[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) bv[r] = *reinterpret_cast<const float4 *>(s_bias + (wv * kBiasTiles + r) * 16 + 4 * g);
    __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));  // (the bias reads done before its next DMA)
    (void)cex;
    // the next tile's record rows in flight from the start of the epilogue
    load_tile(s_tile[(it + 1) & 1]);
    auto next_first = [&]() {
      set_tile();
      if (ex >= 0) issue_first();
    };
    if constexpr (MODE == GEMV_GATE_UP) {
      // as k_gemm_fp8's one-pass split: the wavefront's 2 h blocks x 32 entries staged in the ring
      constexpr int kWaveCols = 16 * CGW, NHB = RT / 4, kRow = 36;
      constexpr int kStageW = NHB * kWaveCols * kRow * 4;
      static_assert(W * kStageW <= kRingBytes && NHB * kWaveCols == 64, "one lane pass, staged in the ring");
      uint8_t *hout = reinterpret_cast<uint8_t *>(a.out);
      const int e0 = kWaveCols * wc;
      const int nloc = max(0, min(kWaveCols, cncol - e0));
      float *st32 = reinterpret_cast<float *>(s_ring + wv * kStageW);
#pragma unroll
      for (int hbk = 0; hbk < NHB; hbk++) {
        if (!tv[4 * hbk]) break;
#pragma unroll
        for (int c = 0; c < CG; c++) {
          if (16 * c >= nloc) break;
          float *se = st32 + (hbk * kWaveCols + 16 * c + j) * kRow;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const f32x4 &av = acc[4 * hbk + r][c];
            const float4 &b4 = bv[4 * hbk + r];
            *reinterpret_cast<float2 *>(se + 8 * r + 2 * g) =
                make_float2(swiglu_fast(av[0] + b4.x, av[1] + b4.y, a.limit), swiglu_fast(av[2] + b4.z, av[3] + b4.w, a.limit));
          }
        }
      }
      const int hbk = min(lane / kWaveCols, NHB - 1), e = lane % kWaveCols;
      const bool valid = tv[4 * hbk] && e < nloc;
      const float *row = st32 + (valid ? hbk * kWaveCols + e : 0) * kRow;
      float v[32];
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float4 x = *reinterpret_cast<const float4 *>(row + 4 * q);
        v[4 * q] = x.x;
        v[4 * q + 1] = x.y;
        v[4 * q + 2] = x.z;
        v[4 * q + 3] = x.w;
      }
      __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));  // the staging reads done
      pq_barrier();                              // ... in every wavefront: the ring is free
      next_first();
      float m = 0.0f;
      bool bad = false;
#pragma unroll
      for (int k = 0; k < 32; k++) {
        m = fmaxf(m, fabsf(v[k]));
        bad = bad || !isfinite(v[k]);
      }
      uint32_t dq[NT][6], sb;
      split32_fp6<NT>(v, m, bad, dq, sb);
      if (valid) {
        const int hb = ct0 / 4 + hbk, st = hb >> 2, i = hb & 3;
        uint8_t *hr = hout + (size_t)(cbeg + e0 + e) * G::kBytes;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          *reinterpret_cast<uint4 *>(hr + G::dword(st, t, i, 0)) = make_uint4(dq[t][0], dq[t][1], dq[t][2], dq[t][3]);
          *reinterpret_cast<uint2 *>(hr + G::dword(st, t, i, 4)) = make_uint2(dq[t][4], dq[t][5]);
          hr[G::scale(st, t) + i] = (uint8_t)(sb >> (8 * t));
        }
      }
    } else {
      next_first();
      float *out = reinterpret_cast<float *>(a.out);
      const int R = (int)d.rows;
#pragma unroll
      for (int r = 0; r < RT; r++) {
        if (!tv[r]) continue;
        const float4 b4 = bv[r];
        const int row = (ct0 + r) * 16 + 4 * g;
#pragma unroll
        for (int c = 0; c < CG; c++) {
          const int e = 16 * (CGW * wc + c) + j;
          if (e >= cncol) continue;
          float4 o;
          o.x = canon_nan(rclamp(acc[r][c][0] + b4.x, -65504.0f, 65504.0f));
          o.y = canon_nan(rclamp(acc[r][c][1] + b4.y, -65504.0f, 65504.0f));
          o.z = canon_nan(rclamp(acc[r][c][2] + b4.z, -65504.0f, 65504.0f));
          o.w = canon_nan(rclamp(acc[r][c][3] + b4.w, -65504.0f, 65504.0f));
          *reinterpret_cast<float4 *>(out + (size_t)(cbeg + e) * R + row) = o;
        }
      }
    }
    // the queue position of the tile after the next, last of the epilogue's memory operations (a
    // wait for anything issued before it would otherwise wait for its round trip too)
    if (wv == 0 && ex >= 0) qn = take();
  }
  // the queue is exhausted for this workgroup: the last one out clears the counters
  if (tid == 0) {
    const int n = __hip_atomic_fetch_add(a.queue + 9, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n == (int)gridDim.x - 1) {
      for (int q = 0; q < 10; q++) st_agent(reinterpret_cast<uint32_t *>(a.queue + q), 0u);
    }
  }
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static std::atomic<int> cus[64] = {};  // (threads racing here store the same value)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (!c) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
    c = n / 8 * 8;
    cus[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

template <int MODE, int RT, int CGW, int WR, int WC, int D, int NT, bool M32 = false, int NSP = 0, int RING = 0>
static hipError_t launch_gemm_shape(GemmArgs a, hipStream_t s) {
  using S = GemmShape<RT, CGW, WR, WC, D, NT>;
  static_assert(S::kLds <= 160 * 1024 - 64, "LDS");
  a.n_row_blocks = (int)((a.d.rows + S::kRows - 1) / S::kRows);
  const size_t col_tiles = (size_t)a.max_active + (a.n_entries + S::kCols - 1) / S::kCols;
  const size_t tiles = (size_t)a.n_row_blocks * col_tiles;
  if (!tiles) return hipSuccess;
  if (tiles > (size_t)INT32_MAX - 8) return hipErrorInvalidValue;
  a.n_tiles = (int)tiles;
  const size_t blocks = a.band ? (tiles + 7) / 8 * 8 : tiles;
  a.n_blocks = (int)blocks;
  // persistent shapes: one workgroup per CU (a multiple of 8, so p % 8 stays the XCD of p)
  const size_t grid = gemm_persistent<MODE, S, NSP>() ? std::min<size_t>(blocks, (size_t)device_cus()) : blocks;
  if (NSP && a.d.ns != (uint32_t)NSP) return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_gemm_fp8<MODE, RT, CGW, WR, WC, D, NT, M32, NSP, RING>), dim3((unsigned)grid), dim3(S::kThreads), 0, s, a);
  return hipGetLastError();
}

// The pipelined 512 x 64 step on one workgroup per CU taking tiles from the queue (k_gemm_pq).
template <int MODE, int NSP, int RING, bool GLOBALQ>
static hipError_t launch_gemm_pq(GemmArgs a, hipStream_t s) {
  using S = GemmShape<8, 2, 4, 2, 2, kGemmTerms>;
  if (!a.queue || a.d.ns != (uint32_t)NSP) return hipErrorInvalidValue;
  a.n_row_blocks = (int)((a.d.rows + S::kRows - 1) / S::kRows);
  const size_t col_tiles = (size_t)a.max_active + (a.n_entries + S::kCols - 1) / S::kCols;
  const size_t tiles = (size_t)a.n_row_blocks * col_tiles;
  if (!tiles) return hipSuccess;
  if (tiles > (size_t)INT32_MAX - 8) return hipErrorInvalidValue;
  a.n_tiles = (int)tiles;
  a.n_blocks = (int)tiles;
  hipLaunchKernelGGL((k_gemm_pq<MODE, NSP, RING, GLOBALQ>), dim3((unsigned)device_cus()), dim3(S::kThreads), 0, s, a);
  return hipGetLastError();
}

// Column tile width from the mean entries per active expert (the per-expert counts live on the
// device): 64 entries once experts average 48 or more (8 wavefronts, two per SIMD, so that one
// wavefront's LDS reads overlap the other's MFMAs); below that 128-row blocks of 2 wavefronts
// with 32 or 16 entries, small enough (50-60 KB of LDS) for 2-3 blocks per CU, which keeps
// every CU streaming weights when the grid is only a few blocks per CU (measured at 64, 128 and
// 256 tokens against the 256-row blocks of 4 wavefronts: 4-10 % faster layers). Below 24 entries
// the streamed form (gemm_stream.hip) takes the launch when it fits; the 128 x 16 block then
// remains for launches it does not fit.
template <int MODE, int NT>
static hipError_t launch_gemm_mode(const GemmArgs &a, hipStream_t s) {
  const size_t active = std::max<size_t>(1, std::min<size_t>((size_t)a.max_active, a.n_entries));
  const size_t mean = a.n_entries / active;
  if constexpr (NT == kGemmTerms) {  // tuning shapes of the exact split only (the quantized mode
                                      // takes its default shape for these codes)
    if (a.shape == 2) return launch_gemm_shape<MODE, 4, 2, 4, 1, 3, NT>(a, s);
    if (a.shape == 3) return launch_gemm_shape<MODE, 4, 1, 4, 1, 3, NT>(a, s);
    if (a.shape == 4) {  // 128 rows in 4 wavefronts of 2 row tiles: down only (gate_up needs whole h blocks)
      if constexpr (MODE == GEMV_GATE_UP) return launch_gemm_shape<MODE, 4, 1, 4, 1, 3, NT>(a, s);
      else return launch_gemm_shape<MODE, 2, 1, 4, 1, 3, NT>(a, s);
    }
    if (a.shape == 6) return launch_gemm_shape<MODE, 4, 1, 1, 1, 3, NT>(a, s);
    if (a.shape == 8) return launch_gemm_shape<MODE, 16, 4, 2, 2, 2, NT>(a, s);
  }
  // one activation term: 512 rows x 128 entries, a wavefront holding 128 x 64 (twice the entries
  // per A read of the 512 x 64 block; with three terms its operands do not fit the registers of
  // two wavefronts per SIMD). Measured at prefill: gate_up 322 -> 297 us, down 203 -> 181 us.
  if constexpr (NT == 1) {
    if (a.shape == 9 || (a.shape == 0 && mean >= 96)) return launch_gemm_shape<MODE, 8, 4, 4, 2, 3, NT>(a, s);
  }
  if (a.shape == 5) return launch_gemm_shape<MODE, 4, 1, 2, 1, 3, NT>(a, s);
  if (a.shape == 7) return launch_gemm_shape<MODE, 4, 2, 2, 1, 3, NT>(a, s);
  // the wide streamed form (gemm_wide.hip): every weight tile once per group of up to 80 entries.
  // By default for experts averaging 14 to 44 entries, 60 to 72 (gate_up) and 14 to 72 (down):
  // measured on the 20B and 120B layers (K = 2880) against the shapes below (gate_up / down, us):
  // 120B at 1024 tokens (32 entries) 302 / 177 against 425 / 227, at 2048 (64) 394 / 223 against
  // 417 / 265; 20B at 320 tokens (40) 93 / 58 against 145 / 77. At 48-56 entries the 512 x 64
  // block's gate_up is faster (309 against 348 us at 120B x 1536: its 64-entry tiles then hold
  // nearly every expert whole), and from ~80 entries every expert needs two groups.
  const bool wide_default = mean >= 14 && (mean < 44 || (mean >= 60 && mean < 72) ||
                                           (MODE == GEMV_DOWN && mean < 72));
  if (a.shape == 14 || (a.shape == 0 && wide_default)) {
    const hipError_t e = launch_gemm_wide(MODE == GEMV_GATE_UP ? GEMV_GATE_UP : GEMV_DOWN, a, s);
    if (e != hipErrorNotSupported) return e;
  }
  // experts averaging fewer than 24 entries: the streamed form (gemm_stream.hip; measured on the
  // 20B layer at 32-128 tokens: gate_up 6-12 us and down 1-8 us faster than the 128 x 16 blocks)
  if (a.shape == 12 || a.shape == 13 || (a.shape == 0 && mean < 24)) {
    const hipError_t e = launch_gemm_stream(MODE == GEMV_GATE_UP ? GEMV_GATE_UP : GEMV_DOWN, a, s, a.shape == 13);
    if (e != hipErrorNotSupported) return e;
  }
  if (a.shape == 10) return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, true>(a, s);
  // the 512 x 64 block with the pipelined step (K-steps 23 or 24; otherwise the plain step)
  if (a.shape == 15) {
    if (a.d.ns == 23) return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 23>(a, s);
    if (a.d.ns == 24) return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 24>(a, s);
    return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT>(a, s);
  }
  if (a.shape == 16 || a.shape == 17) {  // the pipelined step with separate A and B rings
    if (a.d.ns == 23)
      return a.shape == 16 ? launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 23, 1>(a, s)
                           : launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 23, 2>(a, s);
    if (a.d.ns == 24)
      return a.shape == 16 ? launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 24, 1>(a, s)
                           : launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 24, 2>(a, s);
    return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT>(a, s);
  }
  if (a.shape == 11) return launch_gemm_shape<MODE, 16, 2, 2, 4, 2, NT>(a, s);
  if constexpr (NT == kGemmTerms) {
    // the pipelined step on a persistent grid with a tile queue (18: the XCD ranges of the banded
    // order when the launch asks for one; 19: one queue in the plain order), each GEMM with the
    // rings of its default
    if ((a.shape == 18 || a.shape == 19) && (a.d.ns == 23 || a.d.ns == 24)) {
      constexpr int kR = MODE == GEMV_DOWN ? 2 : 0;
      if (a.d.ns == 23)
        return a.shape == 18 ? launch_gemm_pq<MODE, 23, kR, false>(a, s) : launch_gemm_pq<MODE, 23, kR, true>(a, s);
      return a.shape == 18 ? launch_gemm_pq<MODE, 24, kR, false>(a, s) : launch_gemm_pq<MODE, 24, kR, true>(a, s);
    }
  }
  if (mean >= 48) {
    if (a.shape == 1) return launch_gemm_shape<MODE, 4, 4, 8, 1, 2, NT>(a, s);
    // the pipelined step (measured at prefill, 20B x 4096 tokens, paired runs: down 292 -> 278 us;
    // gate_up 517.5 -> 493 us on one workgroup per tile, where on the persistent grid it had
    // stayed at 526 us); the down GEMM with its weights in a ring of 3 (278 -> 264 us; gate_up
    // unchanged with either ring three deep, so it keeps the shared ring); other K: the plain
    // step (gate_up on the persistent grid)
    if constexpr (MODE == GEMV_DOWN) {
      if (a.d.ns == 23) return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 23, 2>(a, s);
      if (a.d.ns == 24) return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 24, 2>(a, s);
    }
    if (a.d.ns == 23) return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 23>(a, s);
    if (a.d.ns == 24) return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT, false, 24>(a, s);
    return launch_gemm_shape<MODE, 8, 2, 4, 2, 2, NT>(a, s);
  }
  if (mean >= 24) return launch_gemm_shape<MODE, 4, 2, 2, 1, 3, NT>(a, s);
  return launch_gemm_shape<MODE, 4, 1, 2, 1, 3, NT>(a, s);
}

bool gemm_stream_local_ok(const GemmArgs &a);  // gemm_stream.hip

// launch_gemm_mode's choice for gate_up with the exact split: the streamed form by default below 14
// entries per expert on average (and for codes 12, 13), when it fits and the batch is small enough
// for its workgroups to group the entries themselves.
bool gemm_gate_up_groups_locally(const GemmArgs &a) {
  if (a.terms != kGemmTerms || a.d.ns > (uint32_t)kGemmNs || a.d.rows % 64) return false;
  const size_t active = std::max<size_t>(1, std::min<size_t>((size_t)a.max_active, a.n_entries));
  const size_t mean = a.n_entries / active;
  const bool stream = a.shape == 12 || a.shape == 13 || (a.shape == 0 && mean < 14);
  return stream && a.n_entries > 0 && gemm_stream_local_ok(a);
}

hipError_t launch_gemm_fp8(GemvMode mode, const GemmArgs &a, hipStream_t s) {
  if (a.d.ns > (uint32_t)kGemmNs || (mode == GEMV_GATE_UP && a.d.rows % 64)) return hipErrorInvalidValue;
  if (a.terms == 1)
    return mode == GEMV_GATE_UP ? launch_gemm_mode<GEMV_GATE_UP, 1>(a, s) : launch_gemm_mode<GEMV_DOWN, 1>(a, s);
  if (a.terms != kGemmTerms) return hipErrorInvalidValue;
  return mode == GEMV_GATE_UP ? launch_gemm_mode<GEMV_GATE_UP, kGemmTerms>(a, s)
                              : launch_gemm_mode<GEMV_DOWN, kGemmTerms>(a, s);
}

}  // namespace moe
