// Wide streamed grouped GEMM: the per-expert FFN of session.rs:87-124 applied to every (token,
// slot) entry routed to an expert (session.rs:943-972), for batches of tens of entries per expert
// (the 120B layer at 2048 tokens: 64 on average), on v_mfma_scale_f32_16x16x128_f8f6f4.
//
// At these batches the block kernel (gemm.hip) re-reads an expert's weights once per column tile
// of 64 entries, and the streamed kernel (gemm_stream.hip) once per 16-entry chunk. Here every
// weight tile streams from HBM once per group of up to NCH chunks (NCH x 16 entries) and is
// multiplied against all of them:
//
//   group   an expert's entries split into ceil(chunks / NCH) groups of near-equal size (each at
//           most 16 NCH entries); a group's activation records (B) are shared by all its units;
//   unit    one group x RT consecutive 16-row weight tiles (gate_up: RT = 4, 64 rows = one
//           32-value h block; down: RT = 2);
//   round   4 consecutive units of one group (the last round of a group may hold fewer), one per
//           compute wavefront; rounds never span two groups, so one LDS area holds a round's B.
//
// All rounds of the launch, group-major, are split into eight contiguous ranges, one per XCD, and
// the persistent grid of one workgroup per CU takes an XCD's range strided: workgroup w of the
// XCD's n runs rounds w, w + n, w + 2n, ... So the XCD's workgroups work on one or two groups at a
// time and its L2 holds their records (a group's are read once per round: 584 KB at 80 entries;
// with contiguous ranges per workgroup, 32 groups' records per XCD missed the L2 at every round),
// and every CU streams about the same weight bytes.
//
// Six wavefronts per workgroup: four compute wavefronts, a B loader and an A loader. The compute
// wavefronts work in pairs: pair h owns units 2h and 2h + 1 of the round (2 RT tiles), its two
// wavefronts the first and the second half of the group's entries, so that every B operand read
// from LDS feeds 2 RT MFMAs (with a unit per wavefront and all the entries each, the four
// wavefronts' B reads took the LDS's whole read bandwidth: 1.1 us of a 1.3 us step at 120B x 2048
// tokens, against 0.6 us of MFMA issue). The A loader streams the round's weights — each unit's
// RT tiles' 1 KB chunks per K-step and,
// every 4 steps, their E8M0 scale words — by LDS-DMA into a ring of R steps (R - 1 steps ahead, on
// across round boundaries); the B loader brings the round's activation record steps into a ring
// of kWidePB steps. A barrier per loop position hands a step over; each loader counts its own
// DMAs (a fixed number per position) in waits of its own. With the weights in per-wavefront
// register rings instead (loads issued by the compute wavefronts once per step, after its MFMAs)
// a step took (latency + MFMA time) / ring depth: 1.3 us at 120B x 2048 tokens (the weight stream
// at ~3 TB/s); from the A loader, which issues at every barrier, the bound is max(MFMA time,
// latency / (R - 1)). Per output the MFMAs run step by step, terms 0, 1, 2 in turn, from zero —
// the order of every other grouped-GEMM shape, so the results are bit-identical to theirs.
#pragma once
#include <algorithm>
#include <type_traits>

#include "device.hpp"
#include "kernels.hpp"
#include "stream.hpp"

namespace moe {

constexpr int kWideCompute = 4;                // compute wavefronts: one unit each per round
constexpr int kWideWaves = kWideCompute + 2;   // and the B and A loaders
constexpr int kWideCols = 16;                  // entries per chunk: one MFMA column group
constexpr int kWideNch = 5;                    // chunks per group (80 entries)
constexpr int kWideMaxGroups = 512;            // groups of a launch (LDS table; the host checks)
constexpr int kWideRowsIssue = 0;              // position at which the B loader DMAs the next rows
constexpr int kWidePos = 24;                   // loop positions of a round (kGemmNs steps)
static_assert(kGemmNs == kWidePos, "one loop position per record step");
constexpr int kWideRow = 36;                   // staging row of the gate_up epilogue (floats)
constexpr int kWideBiasIssue = 4;              // position at which the loader DMAs the round's biases
constexpr int kWidePB = 3;                     // B ring slots: the loader runs 2 steps ahead
constexpr int kWideRowsPos = 12;               // position at which the loader stores the next rows

// The A loader's rings per unit height: R K-steps of weights (R divides the 24 positions, so a
// step's slot is fixed per position), NS quads of scale words (NS divides a round's 6 quads), the
// scale words of quad Q DMA'd in four parts (one wavefront's tiles each) at positions 4Q - D ..
// 4Q - D + 3: complete before barrier 4Q (D >= R + 2: the wait before barrier p completes the
// positions up to p - R + 1) and after the slot's previous quad Q - NS was read at step 4(Q - NS)
// (D <= 4 NS - 1).
template <int RT>
struct WideA;
template <>
struct WideA<4> {
  static constexpr int R = 4, NS = 2, D = 6;
};
template <>
struct WideA<2> {
  static constexpr int R = 6, NS = 3, D = 8;
};
template <int RT, int NSR>
struct WideALoader {
  using P = WideA<RT>;
  static constexpr int R = P::R, NS = P::NS, D = P::D;
  static_assert(kWidePos % R == 0 && (kWidePos / 4) % NS == 0 && D >= R + 2 && D <= 4 * NS - 1, "ring shape");
  static constexpr int kA = kWideCompute * RT;  // weight DMAs per step
  static constexpr int kS = RT;                 // scale-word DMAs per position (one wavefront's tiles)
  // DMAs issued at position x: the weights of step x + R - 1 (this round's or the next one's),
  // if that step exists, and one part of a quad's scale words
  static constexpr int issued(int x) { return ((x + R - 1) % kWidePos < NSR ? kA : 0) + kS; }
  // before barrier p: the DMAs issued at positions p - R + 2 .. p - 1 may stay outstanding
  static constexpr int wait(int p) {
    int c = 0;
    for (int x = p - R + 2; x <= p - 1; x++) c += issued((x % kWidePos + kWidePos) % kWidePos);
    return c;
  }
  static constexpr int max_outstanding() {
    int m = 0;
    for (int p = 0; p < kWidePos; p++) {
      int c = 0;
      for (int x = p - R + 2; x <= p; x++) c += issued((x % kWidePos + kWidePos) % kWidePos);
      m = c > m ? c : m;
    }
    return m;
  }
  static_assert(max_outstanding() <= 63, "the DMAs in flight fit the vmcnt field");
};

// B of one group in LDS, per step: entry m's record step (kStep bytes) at m * kStep, as kDma
// LDS-DMA pieces of 1 KB (lane l of piece i: 16-byte chunk 64 i + l of the group's step). Once a
// round, at position kWideBiasIssue after that position's pieces, one more DMA brings the four
// units' biases.
template <int NCH, int NT, int NSR, int RD>
struct WideLoader {
  using G = GemmRecT<NT>;
  static constexpr int kEntries = NCH * kWideCols;
  static constexpr int kDma = (kEntries * G::kChunks + 63) / 64;
  static constexpr int kSlot = kDma * 1024;
  // DMAs issued at position x: those of step x + kWidePB - 1 (this round's or the next one's),
  // the biases, and RD DMAs of the next round's record rows
  static constexpr int issued(int x) {
    return ((x + kWidePB - 1) % kWidePos < NSR ? kDma : 0) + (x == kWideBiasIssue ? 1 : 0) +
           (x == kWideRowsIssue ? RD : 0);
  }
  // before step p: the loader's DMAs issued after those of step p
  static constexpr int wait(int p) {
    int c = 0;
    for (int x = p - kWidePB + 2; x <= p - 1; x++) c += issued((x % kWidePos + kWidePos) % kWidePos);
    return c;
  }
  // most DMAs in flight: after the issue at position p, those of positions p - PB + 2 .. p (the
  // wait before barrier p completed everything issued earlier)
  static constexpr int max_outstanding() {
    int m = 0;
    for (int p = 0; p < kWidePos; p++) {
      int c = 0;
      for (int x = p - kWidePB + 2; x <= p; x++) c += issued((x % kWidePos + kWidePos) % kWidePos);
      m = c > m ? c : m;
    }
    return m;
  }
  static_assert(max_outstanding() <= 63, "the DMAs in flight fit the vmcnt field");
};

// One item's B operand as read: the first 16 bytes of the lane's block, the 16-byte chunk holding
// its last 8 (selected by g & 1 at use), and the term's scale word (byte g = the lane's block).
struct WideT3 {
  uint4 x, y;
  uint32_t sc;
};

// A round: its group's expert (matrix and bias), first entry and entry count, and the first row
// group of its four units.
struct WideRound {
  const uint8_t *mat;   // the expert's packed matrix
  const float *bias;    // the expert's bias (all rows)
  int beg, cnt, grp0;
  bool real;            // a round of the range (not a repeat of the last one)
};

template <int MODE, int RT, int NSR, int NT>
__global__ __launch_bounds__(64 * kWideWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_wide(GemmArgs a) {
  static_assert(MODE != GEMV_GATE_UP || RT == 4, "gate_up units are whole h blocks");
  static_assert(NSR == 23 || NSR == 24, "23 steps (K = 2880) or up to 24");
  constexpr int NCH = kWideNch;
  // the gate_up B records are the tokens' (rows from entry_src, DMA'd), the down ones the entries'
  constexpr int RD = MODE == GEMV_GATE_UP ? 2 : 0;
  using L = WideLoader<NCH, NT, NSR, RD>;
  static_assert(L::kEntries <= 128, "record rows per group");
  using LA = WideALoader<RT, NSR>;
  using G = GemmRecT<NT>;
  constexpr int RA = LA::R, NS = LA::NS, D = LA::D;
  __shared__ __attribute__((aligned(1024))) uint8_t sB[kWidePB][L::kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t sA[RA][kWideCompute][RT][1024];  // weight chunks per step
  __shared__ __attribute__((aligned(256))) uint32_t sS[NS][kWideCompute][RT][64];   // scale words per quad
  __shared__ int2 s_grp[kWideMaxGroups];                // per group: first entry, expert << 8 | entry count
  __shared__ int s_row[2][128];                         // B record row of each entry of a round's group
  __shared__ __attribute__((aligned(16))) float s_stage[kWideCompute][MODE == GEMV_GATE_UP ? kWideCols * kWideRow : 4];
  __shared__ __attribute__((aligned(16))) float s_bias[256];  // the round's units' biases, 16 RT floats each
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  const bool loader = wvu >= kWideCompute;  // the B loader (kWideCompute) or the A loader
  const int j = lane & 15, g = lane >> 4;
  const PackDims d = a.d;
  const int ns = (int)d.ns, nq = (int)d.nq;
  const int Gu = (int)d.tiles / RT;            // units per group
  const int RG = (Gu + kWideCompute - 1) / kWideCompute;  // rounds per group
  // ---- the experts' groups: lane l of round r holds active expert 64 r + l: its entry range,
  //      id, group count and first group (prefix sum)
  constexpr int kR = kMaxExperts / 64;
  const int ma = min(a.max_active, kMaxExperts);
  int lo[kR], hi[kR], id[kR], g0[kR], ng[kR];
#pragma unroll
  for (int r = 0; r < kR; r++) {
    const int i = 64 * r + lane;
    lo[r] = hi[r] = 0;
    id[r] = 0;
    if (i < ma) {
      lo[r] = a.active_off[i];
      hi[r] = a.active_off[i + 1];
      id[r] = a.active_ids[i];
    }
  }
  const int na = min(*a.n_active, ma);
  int NG = 0;
#pragma unroll
  for (int r = 0; r < kR; r++) {
    if (64 * r + lane >= na) lo[r] = hi[r] = 0;
    const int nc = (hi[r] - lo[r] + kWideCols - 1) / kWideCols;
    ng[r] = (nc + NCH - 1) / NCH;
    int incl = ng[r];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    g0[r] = NG + incl - ng[r];
    NG += __shfl(incl, 63);
  }
  NG = min(__builtin_amdgcn_readfirstlane(NG), kWideMaxGroups);  // (bounded by the host)
  // ---- the group table: group g0 + i of an expert with n entries in ng groups holds entries
  //      [lo + i (n / ng) + min(i, n % ng), + n / ng + (i < n % ng))
  if (wv == 0) {
#pragma unroll
    for (int r = 0; r < kR; r++) {
      if (64 * r + lane < na) {
        const int n = hi[r] - lo[r], n_ = ng[r];
        const int base = n_ ? n / n_ : 0, rem = n - base * n_;
        for (int i = 0; i < n_ && g0[r] + i < kWideMaxGroups; i++)
          s_grp[g0[r] + i] = make_int2(lo[r] + i * base + min(i, rem), (id[r] << 8) | (base + (i < rem ? 1 : 0)));
      }
    }
  }
  // ---- this workgroup's rounds: XCD x (workgroup b runs on XCD b % 8) takes rounds [X0, X1) of
  //      the R = NG RG, its workgroup w = b / 8 rounds X0 + w + k n for k = 0 .. n_rounds - 1
  const int NB = (int)gridDim.x, b = (int)blockIdx.x, NBX = NB / 8, xcd = b % 8, w = b / 8;
  const long long R = (long long)NG * RG;
  const int X0 = (int)(R * xcd / 8), X1 = (int)(R * (xcd + 1) / 8);
  const int n_rounds = __builtin_amdgcn_readfirstlane(X1 - X0 > w ? (X1 - X0 - w + NBX - 1) / NBX : 0);
  if (n_rounds <= 0) return;  // (uniform over the workgroup)
  __syncthreads();

  const uint32_t tbytes = d.nb * 256u;  // one 16-row tile of weights
  const uint32_t a_last = tbytes - 16u;  // its last 16-byte chunk
  const size_t wbytes = pack_weight_bytes(d);
  // round k (k past the last round: a repeat of the last one, loaded, not used)
  auto round = [&](int k) {
    WideRound t;
    const bool real = k < n_rounds;
    k = min(k, n_rounds - 1);
    const int r = X0 + w + k * NBX;
    const int grp_i = r / RG;
    t.grp0 = 4 * (r - grp_i * RG);
    t.real = real;
    const int2 gd = s_grp[grp_i];
    const int ex = __builtin_amdgcn_readfirstlane(gd.y >> 8);
    t.beg = __builtin_amdgcn_readfirstlane(gd.x);
    t.cnt = __builtin_amdgcn_readfirstlane(gd.y & 0xFF);
    const uint8_t *rec = a.base + (size_t)ex * a.stride;
    t.mat = rec + a.mat_off;
    t.bias = reinterpret_cast<const float *>(rec + a.bias_off);
    return t;
  };

  if (wvu == kWideCompute + 1) {
    // ================================================================ the A loader
    // step s of round t into slot sl: wavefront w's tile r (row group min(grp0 + w, Gu - 1)) at
    // sA[sl][w][r]; part w of quad q's scale words into sS[sl][w]
    auto a_dma = [&](const WideRound &t, int s, int sl) {
      const uint32_t ao = min(1024u * (uint32_t)s + 16u * lane, a_last);
#pragma unroll
      for (int w_ = 0; w_ < kWideCompute; w_++) {
        const int t0 = min(t.grp0 + w_, Gu - 1) * RT;
#pragma unroll
        for (int r = 0; r < RT; r++) str_dma16_nt((uint32_t)(t0 + r) * tbytes + ao, t.mat, str_lds(&sA[sl][w_][r][0]));
      }
    };
    auto s_dma = [&](const WideRound &t, int q, int w_, int sl) {
      const int t0 = min(t.grp0 + w_, Gu - 1) * RT, qc = min(q, nq - 1);
#pragma unroll
      for (int r = 0; r < RT; r++)
        str_dma4((uint32_t)wbytes + ((uint32_t)(t0 + r) * (uint32_t)nq + (uint32_t)qc) * 256u + 4u * lane, t.mat,
                 str_lds(&sS[sl][w_][r][0]));
    };
    const WideRound r0d = round(0);
    // what the previous round's positions 24 - D .. 23 would have issued for round 0
    str_static_for<kWidePos - D, kWidePos>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      constexpr int s = x + RA - 1 - kWidePos, qq = (x + D) / 4 - kWidePos / 4, part = (x + D) % 4;
      if constexpr (s >= 0 && s < NSR) a_dma(r0d, s, s % RA);
      if constexpr (qq >= 0) s_dma(r0d, qq, part, qq % NS);
    });
    WideRound acur = r0d;
    for (int k = 0; k < n_rounds; k++) {
      const WideRound anxt = round(k + 1);
      str_static_for<0, kWidePos>([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        if constexpr (p < NSR) __builtin_amdgcn_s_waitcnt(vm_wait(LA::wait(p)));  // this loader's DMAs of step p
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        constexpr int s = p + RA - 1;  // into slot (p - 1) % RA, read at the start of step p - 1
        if constexpr (s < kWidePos) {
          if constexpr (s < NSR) a_dma(acur, s, s % RA);
        } else if constexpr (s - kWidePos < NSR) {
          a_dma(anxt, s - kWidePos, (s - kWidePos) % RA);
        }
        constexpr int qq = (p + D) / 4, part = (p + D) % 4;
        if constexpr (qq < kWidePos / 4) s_dma(acur, qq, part, qq % NS);
        else s_dma(anxt, qq - kWidePos / 4, part, qq % NS);
      });
      acur = anxt;
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    return;
  }
  if (loader) {
    // ================================================================ the B loader
    // the record rows of a round's group (entries past its count: its first entry's), for round k
    // in s_row[k & 1]: gate_up (rows from entry_src) by two DMAs at position kWideRowsIssue of
    // round k - 1, complete before barrier kWideRowsPos; down (the entries themselves) written
    // there. Ordinary loads would make the compiler wait for every DMA in flight where the values
    // are stored (measured: a 2.6 us step once per round).
    auto rows_dma = [&](const WideRound &t, int buf) {
#pragma unroll
      for (int q = 0; q < RD; q++) {
        const int m = 64 * q + lane, e = t.beg + (m < t.cnt ? m : 0);
        str_dma4(4u * (uint32_t)e, a.entry_src, str_lds(&s_row[buf][64 * q]));
      }
    };
    auto rows_direct = [&](const WideRound &t, int buf) {
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int m = 64 * q + lane;
        s_row[buf][m] = t.beg + (m < t.cnt ? m : 0);
      }
    };
    uint32_t boff[L::kDma], nboff[L::kDma];
    auto pieces = [&](const WideRound &t, int buf, uint32_t (&off)[L::kDma]) {
      const uint32_t r_first = (uint32_t)s_row[buf][0] * (uint32_t)G::kBytes;
#pragma unroll
      for (int i = 0; i < L::kDma; i++) {
        const int c = 64 * i + lane, m = c / G::kChunks;
        off[i] = m < t.cnt ? (uint32_t)s_row[buf][m] * (uint32_t)G::kBytes + 16u * (uint32_t)(c - m * G::kChunks)
                           : r_first;  // past the group: one shared line
      }
    };
    auto load_b = [&](const uint32_t (&off)[L::kDma], int s, int sl) {
      const uint8_t *bs = a.brec + (size_t)min(s, kGemmNs - 1) * G::kStep;
#pragma unroll
      for (int i = 0; i < L::kDma; i++) str_dma16(off[i], bs, str_lds(&sB[sl][i * 1024]));
    };
    // the round's biases: lane l -> unit u = (l / (4 RT)) % 4 (16 bytes of its 16 RT floats at
    // byte 64 RT u of s_bias; lanes past the four units repeat them)
    auto load_bias = [&](const WideRound &t) {
      const int u = (lane / (4 * RT)) % kWideCompute, gw = min(t.grp0 + u, Gu - 1);
      const uint32_t voff = (uint32_t)(gw * RT * 16 + 4 * (lane % (4 * RT))) * 4u;
      str_dma16(voff, t.bias, str_lds(s_bias));  // (lane l's bytes land at byte 16 l)
    };
    WideRound rcur = round(0);
    if constexpr (RD > 0) {
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int m = 64 * q + lane, e = rcur.beg + (m < rcur.cnt ? m : 0);
        s_row[0][m] = a.entry_src[e];
      }
    } else {
      rows_direct(rcur, 0);
    }
    pieces(rcur, 0, boff);
    str_static_for<kWidePos - kWidePB + 1, kWidePos>([&](auto xc) {  // what a previous round's last positions would have issued
      constexpr int x = decltype(xc)::value;
      constexpr int s = (x + kWidePB - 1) % kWidePos;
      if constexpr (s < NSR) load_b(boff, s, s % kWidePB);
    });
    for (int k = 0; k < n_rounds; k++) {
      const WideRound rnxt = round(k + 1);
      str_static_for<0, kWidePos>([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        if constexpr (p < NSR) __builtin_amdgcn_s_waitcnt(vm_wait(L::wait(p)));  // this loader's DMAs of step p
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        constexpr int Ld = p + kWidePB - 1;  // into slot (p - 1) % PB, read at the previous position
        if constexpr (Ld < kWidePos) {
          if constexpr (Ld < NSR) load_b(boff, Ld, Ld % kWidePB);
        } else if constexpr (Ld - kWidePos < NSR) {
          load_b(nboff, Ld - kWidePos, (Ld - kWidePos) % kWidePB);
        }
        // the biases, read in the epilogue of this round (complete before barrier kWideBiasIssue +
        // 2; the previous round's epilogue read them before barrier 0)
        if constexpr (p == kWideBiasIssue) load_bias(rcur);
        // the next round's record rows and DMA offsets (used from position kWidePos - kWidePB + 1)
        if constexpr (p == kWideRowsIssue && RD > 0) rows_dma(rnxt, (k + 1) & 1);
        if constexpr (p == kWideRowsPos) {
          if constexpr (RD == 0) rows_direct(rnxt, (k + 1) & 1);
          pieces(rnxt, (k + 1) & 1, nboff);
        }
      });
#pragma unroll
      for (int i = 0; i < L::kDma; i++) boff[i] = nboff[i];
      rcur = rnxt;
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    return;
  }

  // ================================================================== compute wavefronts
  // wavefront w: units u0 = 2 (w >> 1) and u0 + 1 of the round (WT = 2 RT tiles: tile r is tile
  // r % RT of unit u0 + r / RT), entries of half w & 1 of the group ([0, h0) or [h0, cnt),
  // h0 = ceil(cnt / 2)), at most NCHH chunks of 16
  constexpr int WT = 2 * RT, NCHH = (L::kEntries / 2 + kWideCols - 1) / kWideCols;
  const int u0 = 2 * (wvu >> 1), eh = wvu & 1;
  WideRound cur = round(0);
  constexpr int NI = NCHH * NT, BA = 3, BQ = BA + 1;
  const bool odd = (g & 1) != 0;
  WideT3 bq[BQ];          // the item operands in flight
  uint4 av[2][WT];        // the weight chunks of a step, by step parity
  uint32_t swq[2][WT];    // the scale words of a quad, by quad parity
  f32x4 acc[NCHH][WT];
#pragma unroll
  for (int c = 0; c < NCHH; c++)
#pragma unroll
    for (int r = 0; r < WT; r++) acc[c][r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int k = 0; k < n_rounds; k++) {
    const WideRound nxt = round(k + 1);
    const int h0 = (cur.cnt + 1) >> 1;
    const int mbeg = __builtin_amdgcn_readfirstlane(eh ? h0 : 0);
    const int mcnt = __builtin_amdgcn_readfirstlane(eh ? cur.cnt - h0 : h0);
    const int nchk = __builtin_amdgcn_readfirstlane((mcnt + kWideCols - 1) / kWideCols);
    // lane (j, g)'s entry of chunk c in the slot (past the slot's entries: its last)
    uint32_t ebo[NCHH];
#pragma unroll
    for (int c = 0; c < NCHH; c++) ebo[c] = (uint32_t)min(mbeg + kWideCols * c + j, L::kEntries - 1) * G::kStep;
    // items i = (term i / NCHH, chunk i % NCHH) of a step: per output the terms 0, 1, 2 in turn
    // (the order of every other shape), and NCHH x WT MFMAs between two on one accumulator (chunk by
    // chunk, the next term's MFMA waited for the last one's result). Item (P, i) is read BA items
    // ahead of its MFMAs into bq[(NI P + i) % BQ]: its 24 operand bytes (two 16-byte reads) and its
    // term's scale word. Every item is read (past the group's entries stale values) and only the
    // MFMAs of chunks from nchk on are skipped: with reads on both sides of a branch the compiler
    // could not count the LDS reads in flight and waited for all of them before every item.
    auto rd_item = [&](auto pc2, auto ic) {
      constexpr int P2 = decltype(pc2)::value, i = decltype(ic)::value, tt = i / NCHH, c = i % NCHH;
      const uint8_t *eb = &sB[P2 % kWidePB][0] + ebo[c];
      WideT3 &b = bq[(NI * P2 + i) % BQ];
      b.x = *reinterpret_cast<const uint4 *>(eb + tt * G::kTermBytes + 16 * g);
      b.y = *reinterpret_cast<const uint4 *>(eb + tt * G::kTermBytes + 64 + 16 * (g >> 1));
      b.sc = *reinterpret_cast<const uint32_t *>(eb + NT * G::kTermBytes + 4 * tt);
    };
    // the weight chunks of step P2 (and, at a quad's first step, its scale words), double-buffered
    // by step parity
    auto rd_a = [&](auto pc2) {
      constexpr int P2 = decltype(pc2)::value;
      if constexpr (P2 % 4 == 0) {
#pragma unroll
        for (int r = 0; r < WT; r++) swq[(P2 / 4) & 1][r] = sS[(P2 / 4) % NS][u0 + r / RT][r % RT][lane];
      }
#pragma unroll
      for (int r = 0; r < WT; r++)
        av[P2 & 1][r] = *reinterpret_cast<const uint4 *>(&sA[P2 % RA][u0 + r / RT][r % RT][16 * lane]);
    };
    auto mfma_item = [&](auto pc2, auto ic, int sh) {
      constexpr int P2 = decltype(pc2)::value, i = decltype(ic)::value, c = i % NCHH;
      const WideT3 &b = bq[(NI * P2 + i) % BQ];
      const i32x8 B = {(int)b.x.x, (int)b.x.y, (int)b.x.z, (int)b.x.w, (int)(odd ? b.y.z : b.y.x),
                       (int)(odd ? b.y.w : b.y.y), 0, 0};
      const int sb = (int)(b.sc >> (8 * g));
#pragma unroll
      for (int r = 0; r < WT; r++) {
        const uint4 &a4 = av[P2 & 1][r];
        const i32x8 A = {(int)a4.x, (int)a4.y, (int)a4.z, (int)a4.w, 0, 0, 0, 0};
        // cbsz 4: A is fp4 (E2M1); blgp 2: B is fp6 (E2M3)
        acc[c][r] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[c][r], 4, 2, 0,
                                                                      (int)(swq[(P2 / 4) & 1][r] >> sh), 0, sb);
      }
    };
    str_static_for<0, kWidePos>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      // barrier p: the loaders' DMAs of step p complete; their slots of step p - 1 free
      auto bar = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
      };
      if constexpr (NSR == 23) {
        // ---- K = 2880, every one of the 23 steps computed: pipelined across steps. Barrier p + 1
        //      is taken inside step p, right after its last LDS reads complete, and the first BA
        //      items and the weight chunks of step p + 1 are read during the last BA items' MFMAs
        //      of step p (with the barrier at each step's start, every wavefront's first reads
        //      queued at the LDS together while the MFMAs waited, and the last MFMAs ran with the
        //      LDS idle: a step took about the sum of the two). Not across rounds: the epilogue
        //      follows step 22.
        if constexpr (p == 0 || p == kWidePos - 1) bar();
        if constexpr (p < NSR) {
          if constexpr (p == 0) {
            rd_a(std::integral_constant<int, 0>{});
            str_static_for<0, BA>([&](auto ic) { rd_item(std::integral_constant<int, 0>{}, ic); });
          }
          const int sh = 8 * (p % 4);
          str_static_for<0, NI>([&](auto ic) {
            constexpr int i = decltype(ic)::value, c = i % NCHH, ni = i + BA;
            if constexpr (ni < NI) {
              rd_item(pc, std::integral_constant<int, ni>{});
            } else if constexpr (p + 1 < NSR) {
              if constexpr (ni == NI) {
                // this wavefront's reads of step p's slots complete before the loaders may refill them
                __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));
                bar();
                rd_a(std::integral_constant<int, p + 1>{});
              }
              rd_item(std::integral_constant<int, p + 1>{}, std::integral_constant<int, ni - NI>{});
            }
            __builtin_amdgcn_sched_barrier(0);  // the reads BA items ahead issue before this item's MFMAs
            if (c < nchk) mfma_item(pc, ic, sh);
            __builtin_amdgcn_sched_barrier(0);
          });
#pragma unroll
          for (int c = 0; c < NCHH; c++)
#pragma unroll
            for (int r = 0; r < WT; r++) asm volatile("" ::"v"(acc[c][r]) : "memory");
        }
      } else {
        // ---- K below 3072 other than 2880: steps from ns on are repeats, skipped at run time;
        //      each step's reads follow its barrier
        bar();
        if constexpr (p < NSR) {
          if (p < ns) {
            rd_a(pc);
            str_static_for<0, BA>([&](auto ic) { rd_item(pc, ic); });
            const int sh = 8 * (p % 4);
            str_static_for<0, NI>([&](auto ic) {
              constexpr int i = decltype(ic)::value, c = i % NCHH;
              if constexpr (i + BA < NI) rd_item(pc, std::integral_constant<int, i + BA>{});
              __builtin_amdgcn_sched_barrier(0);
              if (c < nchk) mfma_item(pc, ic, sh);
              __builtin_amdgcn_sched_barrier(0);
            });
#pragma unroll
            for (int c = 0; c < NCHH; c++)
#pragma unroll
              for (int r = 0; r < WT; r++) asm volatile("" ::"v"(acc[c][r]) : "memory");
          }
        }
      }
      if constexpr (p == kWidePos - 1) {
        // ---- epilogue of this wavefront's units of round k, chunk by chunk (units past the
        //      group's row groups, and the repeat of the last round, are not stored)
        str_static_for<0, NCHH>([&](auto cc) {
          constexpr int c = decltype(cc)::value;
          if (c < nchk) {
            const int e0 = cur.beg + mbeg + kWideCols * c, ec = min(kWideCols, mcnt - kWideCols * c);
#pragma unroll
            for (int ut = 0; ut < 2; ut++) {
              const int gw = cur.grp0 + u0 + ut;
              if (!cur.real || gw >= Gu) continue;
              const float *bu = s_bias + (u0 + ut) * 16 * RT;
              if constexpr (MODE == GEMV_GATE_UP) {
                // lane (j, g) holds rows 16 r + 4 g .. + 3 of the unit (gate = row 2i, up = row
                // 2i + 1): h values 8 r + 2 g, 8 r + 2 g + 1 of entry j's 32-value block; staged
                // per wavefront, then lane e splits entry e's whole block into the NT terms of its
                // h record
                float *st = s_stage[wvu];
#pragma unroll
                for (int r = 0; r < RT; r++) {
                  const float4 b4 = *reinterpret_cast<const float4 *>(bu + r * 16 + 4 * g);
                  const f32x4 &av = acc[c][ut * RT + r];
                  *reinterpret_cast<float2 *>(st + j * kWideRow + 8 * r + 2 * g) =
                      make_float2(swiglu_fast(av[0] + b4.x, av[1] + b4.y, a.limit),
                                  swiglu_fast(av[2] + b4.z, av[3] + b4.w, a.limit));
                }
                if (lane < ec) {
                  float v[32];
#pragma unroll
                  for (int k4 = 0; k4 < 8; k4++) {
                    const float4 x = *reinterpret_cast<const float4 *>(st + lane * kWideRow + 4 * k4);
                    v[4 * k4] = x.x;
                    v[4 * k4 + 1] = x.y;
                    v[4 * k4 + 2] = x.z;
                    v[4 * k4 + 3] = x.w;
                  }
                  float m = 0.0f;
                  bool bad = false;
#pragma unroll
                  for (int q = 0; q < 32; q++) {
                    m = fmaxf(m, fabsf(v[q]));
                    bad = bad || !isfinite(v[q]);
                  }
                  uint32_t dq[NT][6], sbw;
                  split32_fp6<NT>(v, m, bad, dq, sbw);
                  const int st_ = gw >> 2, i = gw & 3;
                  uint8_t *hr = reinterpret_cast<uint8_t *>(a.out) + (size_t)(e0 + lane) * G::kBytes;
#pragma unroll
                  for (int tt = 0; tt < NT; tt++) {
                    str_st16(hr + G::dword(st_, tt, i, 0), make_uint4(dq[tt][0], dq[tt][1], dq[tt][2], dq[tt][3]));
                    str_st8(hr + G::dword(st_, tt, i, 4), make_uint2(dq[tt][4], dq[tt][5]));
                    str_st1(hr + G::scale(st_, tt) + i, (sbw >> (8 * tt)) & 0xFFu);
                  }
                }
              } else {
                if (j < ec) {
                  float *o = reinterpret_cast<float *>(a.out) + (size_t)(e0 + j) * d.rows + (size_t)gw * RT * 16 + 4 * g;
#pragma unroll
                  for (int r = 0; r < RT; r++) {
                    const float4 b4 = *reinterpret_cast<const float4 *>(bu + r * 16 + 4 * g);
                    const f32x4 &av = acc[c][ut * RT + r];
                    float4 v;
                    v.x = canon_nan(rclamp(av[0] + b4.x, -65504.0f, 65504.0f));
                    v.y = canon_nan(rclamp(av[1] + b4.y, -65504.0f, 65504.0f));
                    v.z = canon_nan(rclamp(av[2] + b4.z, -65504.0f, 65504.0f));
                    v.w = canon_nan(rclamp(av[3] + b4.w, -65504.0f, 65504.0f));
                    str_st16(o + r * 16, make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                                                    __float_as_uint(v.w)));
                  }
                }
              }
            }
          }
        });
#pragma unroll
        for (int c = 0; c < NCHH; c++)
#pragma unroll
          for (int r = 0; r < WT; r++) acc[c][r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    });
    cur = nxt;
  }
  __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));  // (the last round's repeats and the stores)
}

// Launch of one instantiation (grid: n_wg workgroups, one per CU).
template <int MODE, int RT, int NT>
inline hipError_t launch_wide_rt(const GemmArgs &a, hipStream_t s, int n_wg) {
  if (a.d.ns == 23)
    hipLaunchKernelGGL((k_gemm_wide<MODE, RT, 23, NT>), dim3((unsigned)n_wg), dim3(64 * kWideWaves), 0, s, a);
  else
    hipLaunchKernelGGL((k_gemm_wide<MODE, RT, 24, NT>), dim3((unsigned)n_wg), dim3(64 * kWideWaves), 0, s, a);
  return hipGetLastError();
}

// The launchers of each mode live in their own translation unit (gemm_wide_gu.hip,
// gemm_wide_dn.hip), so that the instantiations compile in parallel.
hipError_t launch_wide_gate_up(const GemmArgs &a, hipStream_t s, int n_wg);
hipError_t launch_wide_down(const GemmArgs &a, hipStream_t s, int n_wg);

}  // namespace moe
