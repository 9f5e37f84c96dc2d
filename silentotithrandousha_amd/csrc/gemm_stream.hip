// Streamed grouped GEMM for batches of a few entries per expert (the per-expert FFN of
// session.rs:87-124 applied to every (token, slot) entry routed to an expert, session.rs:943-972)
// on v_mfma_scale_f32_16x16x128_f8f6f4, for the batches where the weight stream, not the MFMA,
// bounds the layer (a few to about a dozen entries per expert).
//
// Work: every active expert's entries in chunks of up to 16 (one MFMA column group); a unit is
// one chunk x RT consecutive 16-row weight tiles (gate_up: RT = 4, 64 rows = one 32-value h block
// of SwiGLU outputs; down: RT = 2). All units of the launch, chunk-major, are split into
// contiguous ranges, one per workgroup of a persistent grid of one workgroup per CU (the ranges
// of an XCD's workgroups contiguous, so its L2 holds the records of its experts only): every CU
// streams the same share of the weight bytes. A workgroup takes its range in rounds of 4
// consecutive units, one per compute wavefront; the units of a round lie in at most two chunks,
// whose B operands (the entries' activation records) all four share.
//
// A round steps through K in steps of 128, 24 loop positions (steps from NSR on empty). Each
// compute wavefront streams the A chunks of its RT tiles (1 KB each, non-temporal) and, every 4
// steps, their E8M0 scale words straight into a ring of PA steps of registers, PA steps ahead of
// its MFMAs and on across round boundaries (the next round's first steps load during this round's
// last ones, so the HBM stream does not pause at a round's end); these are ordinary loads, so the
// compiler counts the outstanding ones before each use. A fifth wavefront loads the round's B
// record steps by LDS-DMA (global_load_lds) into a ring of PB steps in LDS, PB - 1 steps ahead,
// with waits of its own (a fixed number of DMAs per position). A barrier per position: the
// step's B complete, the slot read at the previous step free. Each wavefront's queue holds only
// its own kind of load, so every wait counts exactly what it needs (loads complete in order: a
// wave waiting for one load waits for all older ones). The same MFMAs as k_gemm_fp8 (per output:
// step by step, terms 0, 1, 2 in turn, from zero) give the same bits.
//
// The epilogue's global stores are inline assembly (str_st*, stream.hpp): with stores pending
// among the loads the compiler would wait for every load, and the ring would drain at each
// round's end.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "device.hpp"
#include "kernels.hpp"
#include "stream.hpp"

namespace moe {

constexpr int kStrCompute = 4;                // compute wavefronts: one unit each per round
constexpr int kStrWaves = kStrCompute + 1;    // and the B loader
constexpr int kStrCols = 16;    // entries per chunk: one MFMA column group
constexpr int kStrMaxSeg = 32;  // chunks one workgroup's range may touch (the host checks)
constexpr int kStrPos = 24;     // loop positions of a round (kGemmNs steps)
static_assert(kGemmNs == kStrPos, "one loop position per record step");
constexpr int kStrRow = 36;     // staging row of the gate_up epilogue (floats)
constexpr int kStrBiasPos = 12; // position of a round whose loads include the unit's bias

// The B loader's DMAs per position and its wait before each step (NSR real steps per round;
// NSR = 24 takes any ns <= 24, steps from ns on loaded as in-range repeats and not computed).
template <int NSR, int PB, int NT>
struct StrLoader {
  using G = GemmRecT<NT>;
  static constexpr int kPieces = (kStrCols * G::kStep + 1023) / 1024;  // 1 KB pieces of a chunk's B step
  static constexpr int kDma = 2 * kPieces;                             // two chunk areas per step
  static_assert(kStrPos % PB == 0 && PB >= 3, "ring slots fixed per position");
  // DMAs issued at position x: those of step x + PB - 1 (this round's or the next one's)
  static constexpr int issued(int x) { return (x + PB - 1) % kStrPos < NSR ? kDma : 0; }
  // before step p: the loader's DMAs issued after those of step p (positions p - PB + 2 .. p - 1)
  static constexpr int wait(int p) {
    int c = 0;
    for (int x = p - PB + 2; x <= p - 1; x++) c += issued((x % kStrPos + kStrPos) % kStrPos);
    return c;
  }
  static constexpr int max_outstanding() {
    int m = 0;
    for (int p = 0; p < kStrPos; p++) {
      int c = 0;
      for (int x = p - PB + 1; x <= p; x++) c += issued((x % kStrPos + kStrPos) % kStrPos);
      m = c > m ? c : m;
    }
    return m;
  }
  static_assert(max_outstanding() <= 63, "the DMAs in flight fit the vmcnt field");
};

// One K-step of a compute wavefront's ring: the lane's A chunks of its RT tiles.
template <int RT>
struct StrSlot {
  uint4 a[RT];
};

// A round as one wavefront sees it: its unit (or, for a wavefront past the range, the round's
// first unit, computed but not stored), and for the loader the B pieces of the round's chunks.
struct StrRound {
  const uint8_t *tile;  // the unit's first 16-row weight tile
  const uint8_t *sca;   // its scale words
  const float *bias;    // its rows' bias
  int beg, cnt, grp;    // the chunk's first entry and entry count; the unit's row group
  bool store;           // a unit of the range (not a stand-in)
  int area;             // B area of the unit's chunk: 0 (the round's first chunk) or 1
  bool two;             // the round has a second chunk
  int qf;               // the round's first chunk (segment index)
};

template <int MODE, int RT, int NSR, int PA, int PB, int NT>
__global__ __launch_bounds__(64 * kStrWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_stream(GemmArgs a) {
  static_assert(MODE != GEMV_GATE_UP || RT == 4, "gate_up units are whole h blocks");
  static_assert(NSR == 23 || NSR == 24, "23 steps (K = 2880) or up to 24");
  static_assert(kStrPos % PA == 0 && PA >= 2, "A ring slots fixed per position");
  using L = StrLoader<NSR, PB, NT>;
  using G = GemmRecT<NT>;
  constexpr int kPieces = L::kPieces, kBArea = kPieces * 1024;
  constexpr int QR = PA <= 4 ? 2 : 3;  // A-scale quads held at once
  static_assert((kStrPos / 4) % QR == 0, "a round's quads map to fixed scale slots");
  __shared__ __attribute__((aligned(1024))) uint8_t sB[PB][2][kBArea];
  __shared__ __attribute__((aligned(1024))) uint8_t sBd[1024];  // target of the absent second chunk's pieces
  __shared__ __attribute__((aligned(16))) float s_stage[kStrCompute][MODE == GEMV_GATE_UP ? kStrCols * kStrRow : 4];
  __shared__ int s_seg[kStrMaxSeg][3];         // expert, first entry, entry count
  __shared__ int s_row[kStrMaxSeg][kStrCols];  // B record row of each entry
  // local grouping: entry n's expert, then its grouped position; grouped entry -> token; the
  // experts' counts (then running ranks), first entries and the active list
  __shared__ int s_ge[MODE == GEMV_GATE_UP ? kLocalGroupMax : 1];
  __shared__ int s_esrc[MODE == GEMV_GATE_UP ? kLocalGroupMax : 1];
  __shared__ int s_gcnt[MODE == GEMV_GATE_UP ? kMaxExperts : 1], s_gbase[MODE == GEMV_GATE_UP ? kMaxExperts : 1];
  __shared__ int s_aid[MODE == GEMV_GATE_UP ? kMaxExperts : 1], s_aoff[MODE == GEMV_GATE_UP ? kMaxExperts + 1 : 1];
  __shared__ int s_na;
  __shared__ int s_ccnt[MODE == GEMV_GATE_UP ? kLocalGroupMax / 64 : 1][MODE == GEMV_GATE_UP ? kMaxExperts : 1];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  const bool loader = wvu == kStrCompute;
  const int j = lane & 15, g = lane >> 4;
  const PackDims d = a.d;
  const int ns = (int)d.ns, nq = (int)d.nq;
  const int Gu = (int)d.tiles / RT;  // units per chunk
  // ---- the experts' chunks: lane l of round r holds active expert 64 r + l: its entry range,
  //      id, chunk count and first chunk (prefix sum)
  constexpr int kR = kMaxExperts / 64;
  // (the lists hold max_active (+1) entries: lanes below it load before the count is known, in
  // the same round trip, and lanes past the count are cleared)
  const int ma = min(a.max_active, kMaxExperts);
  int lo[kR], hi[kR], id[kR], c0[kR], nc[kR];
  const bool local = MODE == GEMV_GATE_UP && a.group_idx != nullptr;
  int na;
  if (local) {
    // ---- the grouping of session.rs:943-972's entries by expert (k_route / bucket_block's: active
    //      experts ascending, an expert's entries in entry order t k + slot), from the top-k
    //      indices, in LDS. Entries in chunks of 64, chunk ch by wavefront ch % 5: per chunk the
    //      count of each expert and each entry's rank among the chunk's entries of its expert
    //      (9-bit match by ballots); per expert an exclusive prefix of its counts over the chunks
    //      (a thread per expert); the expert list (wavefront 0); then every entry's position.
    const int N = (int)a.n_entries, E = a.group_E, tid = threadIdx.x;
    constexpr int kCh = kLocalGroupMax / 64, kPerW = (kCh + kStrWaves - 1) / kStrWaves;
    const int nch = (N + 63) / 64;
    for (int i = tid; i < nch * E; i += kStrWaves * 64) s_ccnt[i / E][i % E] = 0;
    __syncthreads();
    int ge_e[kPerW], ge_r[kPerW];
#pragma unroll
    for (int q = 0; q < kPerW; q++) {
      const int ch = wv + kStrWaves * q, n = 64 * ch + lane;
      ge_e[q] = ch < nch && n < N ? a.group_idx[n] : -1;
    }
#pragma unroll
    for (int q = 0; q < kPerW; q++) {
      const int ch = wv + kStrWaves * q, e = ge_e[q];
      const uint32_t v = (uint32_t)(e + 1);  // 0 .. kMaxExperts: 9 bits
      uint64_t same = ~0ull;
#pragma unroll
      for (int bit = 0; bit < 9; bit++) {
        const uint64_t bb = __ballot((v >> bit) & 1u);
        same &= ((v >> bit) & 1u) ? bb : ~bb;
      }
      const uint64_t below = same & ((1ull << lane) - 1ull);
      ge_r[q] = __popcll(below);
      if (ch < nch && e >= 0 && below == 0) s_ccnt[ch][e] = __popcll(same);  // (the group's first lane)
    }
    __syncthreads();
    for (int e = tid; e < E; e += kStrWaves * 64) {
      int run = 0;
      for (int ch = 0; ch < nch; ch++) {
        const int c = s_ccnt[ch][e];
        s_ccnt[ch][e] = run;
        run += c;
      }
      s_gcnt[e] = run;
    }
    __syncthreads();
    if (wv == 0) expert_list_wave(s_gcnt, E, lane, s_gbase, s_aid, s_aoff, &s_na);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPerW; q++) {
      const int ch = wv + kStrWaves * q, n = 64 * ch + lane, e = ge_e[q];
      if (ch < nch && n < N) {
        if (e >= 0) {
          const int ge = s_gbase[e] + s_ccnt[ch][e] + ge_r[q];
          s_esrc[ge] = n / a.group_k;
          s_ge[n] = ge;
        } else {
          s_ge[n] = -1;
        }
      }
    }
    __syncthreads();
    if (blockIdx.x == 0) {  // the lists for the down GEMM and the combine
      const int nl = s_na;
      for (int n = tid; n < N; n += kStrWaves * 64) {
        a.w_pos[n] = s_ge[n];
        a.w_entry_src[n] = s_esrc[n];  // (entries past the grouped ones: unread)
      }
      for (int i = tid; i <= nl; i += kStrWaves * 64) {
        a.w_active_off[i] = s_aoff[i];
        if (i < nl) a.w_active_ids[i] = s_aid[i];
      }
      if (tid == 0) *a.w_n_active = nl;
    }
#pragma unroll
    for (int r = 0; r < kR; r++) {
      const int i = 64 * r + lane;
      lo[r] = hi[r] = 0;
      id[r] = 0;
      if (i < s_na) {
        lo[r] = s_aoff[i];
        hi[r] = s_aoff[i + 1];
        id[r] = s_aid[i];
      }
    }
    na = s_na;
  } else {
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
    na = min(*a.n_active, ma);
  }
  int NC = 0;
#pragma unroll
  for (int r = 0; r < kR; r++) {
    if (64 * r + lane >= na) lo[r] = hi[r] = 0;
    nc[r] = (hi[r] - lo[r] + kStrCols - 1) / kStrCols;
    int incl = nc[r];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    c0[r] = NC + incl - nc[r];
    NC += __shfl(incl, 63);
  }
  NC = __builtin_amdgcn_readfirstlane(NC);
  // ---- this workgroup's units [u0, u1): workgroups numbered XCD by XCD (workgroup b runs on
  //      XCD b % 8)
  const int NB = (int)gridDim.x, b = (int)blockIdx.x;
  const int gb = (b % 8) * (NB / 8) + b / 8;
  const long long U = (long long)NC * Gu;
  const int u0 = __builtin_amdgcn_readfirstlane((int)(U * gb / NB)),
            u1 = __builtin_amdgcn_readfirstlane((int)(U * (gb + 1) / NB));
  if (u0 >= u1) return;  // (uniform over the workgroup)
  const int ci0 = u0 / Gu, nseg = min((u1 - 1) / Gu - ci0 + 1, kStrMaxSeg);
  if (wv == 0) {
    for (int q = 0; q < nseg; q++) {
      const int ci = ci0 + q;
      int ex = 0, beg = 0, cnt = 0;
#pragma unroll
      for (int r = 0; r < kR; r++) {
        const uint64_t hit = __ballot(64 * r + lane < na && ci >= c0[r] && ci < c0[r] + nc[r]);
        if (hit) {
          const int hl = __builtin_ctzll(hit);
          const int e_ = __shfl(id[r], hl), l_ = __shfl(lo[r], hl), h_ = __shfl(hi[r], hl), s_ = __shfl(c0[r], hl);
          ex = e_;
          beg = l_ + (ci - s_) * kStrCols;
          cnt = min(kStrCols, h_ - beg);
        }
      }
      if (lane == 0) {
        s_seg[q][0] = ex;
        s_seg[q][1] = beg;
        s_seg[q][2] = cnt;
      }
    }
  }
  __syncthreads();
  if (loader) {
    // the entries' B record rows, read by the loader alone: the compute wavefronts meanwhile
    // issue their first weight loads, which need only the chunk table
    for (int q4 = 0; q4 < nseg; q4 += 4) {  // lane (q4 + lane / 16, entry j)
      const int q = q4 + g;
      if (q < nseg) {
        const int beg = s_seg[q][1], cnt = s_seg[q][2];
        const int e = beg + min(j, max(cnt, 1) - 1);
        s_row[q][j] = local ? s_esrc[e] : (a.entry_src ? a.entry_src[e] : e);
      }
    }
  }

  const uint32_t tbytes = d.nb * 256u;  // one 16-row tile of weights
  const uint32_t a_last = tbytes - 16u;  // its last 16-byte chunk
  const size_t wbytes = pack_weight_bytes(d);
  const int n_rounds = (u1 - u0 + kStrCompute - 1) / kStrCompute;
  auto seg_of = [&](int u) { return min(u / Gu - ci0, kStrMaxSeg - 1); };  // (bounded by the host)
  // round k (k past the last round: a repeat of the last one, loaded, not used)
  auto round = [&](int k) {
    StrRound t;
    k = min(k, n_rounds - 1);
    const int ub = u0 + kStrCompute * k;
    const int uw = ub + (loader ? 0 : wvu);
    t.store = !loader && uw < u1;
    const int u = t.store ? uw : ub;
    const int q = seg_of(u);
    t.qf = seg_of(ub);
    t.two = seg_of(min(ub + kStrCompute - 1, u1 - 1)) > t.qf;
    t.area = q - t.qf;  // 0 or 1: four consecutive units touch at most two chunks (units per chunk >= 3)
    t.grp = u - (u / Gu) * Gu;
    const int ex = __builtin_amdgcn_readfirstlane(s_seg[q][0]);
    t.beg = __builtin_amdgcn_readfirstlane(s_seg[q][1]);
    t.cnt = __builtin_amdgcn_readfirstlane(s_seg[q][2]);
    const uint8_t *rec = a.base + (size_t)ex * a.stride;
    const uint8_t *mat = rec + a.mat_off;
    const int t0 = t.grp * RT;
    t.tile = mat + (size_t)t0 * tbytes;
    t.sca = mat + wbytes + (size_t)t0 * nq * 256;
    t.bias = reinterpret_cast<const float *>(rec + a.bias_off) + t0 * 16;
    return t;
  };

  if (loader) {
    // ================================================================ the B loader
    // piece i (< kPieces: the round's first chunk, then its second, or for a round with one
    // chunk the first record step's first 16 bytes into the dummy piece): lane l holds 16-byte
    // chunk 64 (i % kPieces) + l of the chunk's 16 record steps (entry c / kChunks, part c %
    // kChunks; entries past the chunk's repeat its last)
    uint32_t boff[L::kDma], nboff[L::kDma];
    bool breal[L::kDma], nbreal[L::kDma];
    auto pieces = [&](const StrRound &t, uint32_t (&off)[L::kDma], bool (&real)[L::kDma]) {
#pragma unroll
      for (int i = 0; i < L::kDma; i++) {
        const int ar = i / kPieces, pc = i % kPieces;
        const int c = min(64 * pc + lane, kStrCols * G::kChunks - 1);
        real[i] = ar == 0 || t.two;
        const int qa = min(t.qf + ar, kStrMaxSeg - 1);
        off[i] = real[i] ? (uint32_t)s_row[qa][c / G::kChunks] * (uint32_t)G::kBytes + 16u * (c % G::kChunks) : 0u;
      }
    };
    auto load_b = [&](const uint32_t (&off)[L::kDma], const bool (&real)[L::kDma], int s, int sl) {
      const uint8_t *bs = a.brec + (size_t)min(s, kGemmNs - 1) * G::kStep;
#pragma unroll
      for (int i = 0; i < L::kDma; i++)
        str_dma16(off[i], bs, real[i] ? str_lds(&sB[sl][i / kPieces][(i % kPieces) * 1024]) : str_lds(sBd));
    };
    pieces(round(0), boff, breal);
    str_static_for<kStrPos - PB + 1, kStrPos>([&](auto xc) {  // what a previous round's last positions would have issued
      constexpr int x = decltype(xc)::value;
      constexpr int s = (x + PB - 1) % kStrPos;
      if constexpr (s < NSR) load_b(boff, breal, s, s % PB);
    });
    for (int k = 0; k < n_rounds; k++) {
      pieces(round(k + 1), nboff, nbreal);
      str_static_for<0, kStrPos>([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        if constexpr (p < NSR) __builtin_amdgcn_s_waitcnt(vm_wait(L::wait(p)));  // this loader's DMAs of step p
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        constexpr int Ld = p + PB - 1;  // into slot (p - 1) % PB, read at the previous position
        if constexpr (Ld < kStrPos) {
          if constexpr (Ld < NSR) load_b(boff, breal, Ld, Ld % PB);
        } else if constexpr (Ld - kStrPos < NSR) {
          load_b(nboff, nbreal, Ld - kStrPos, (Ld - kStrPos) % PB);
        }
      });
#pragma unroll
      for (int i = 0; i < L::kDma; i++) {
        boff[i] = nboff[i];
        breal[i] = nbreal[i];
      }
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    return;
  }

  // ================================================================== compute wavefronts
  StrRound cur = round(0);
  // Loads of step s (s >= ns: in-range repeats) of round t into ring slot sl, and every 4 steps
  // the scale words of the next 4 into scale slot (s / 4) % QR.
  StrSlot<RT> ring[PA];
  uint32_t sw[QR][RT];
  auto load_step = [&](const StrRound &t, int s, int sl) {
    if (s % 4 == 0) {
      const int qc = min(s / 4, nq - 1);
#pragma unroll
      for (int r = 0; r < RT; r++)
        sw[(s / 4) % QR][r] = *reinterpret_cast<const uint32_t *>(t.sca + ((size_t)r * nq + qc) * 256 + 4 * lane);
    }
    const uint32_t ao = min(1024u * (uint32_t)s + 16u * lane, a_last);
#pragma unroll
    for (int r = 0; r < RT; r++) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(t.tile + (size_t)r * tbytes + ao));
      ring[sl].a[r] = make_uint4(v.x, v.y, v.z, v.w);
    }
  };
  float4 bias[RT];
  f32x4 acc[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) acc[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // prologue: steps 0 .. PA - 1 of round 0 (in the loop's order, step by step: the compiler's
  // wait counts at the loop head merge this path with the loop's own)
  str_static_for<0, PA>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    __builtin_amdgcn_sched_barrier(0);
    load_step(cur, s, s % PA);
  });
  __builtin_amdgcn_sched_barrier(0);

  for (int k = 0; k < n_rounds; k++) {
    const StrRound nxt = round(k + 1);
    str_static_for<0, kStrPos>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      __builtin_amdgcn_sched_barrier(0);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_barrier();  // the loader's DMAs of step p complete; slot (p - 1) % PB free
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if constexpr (p == kStrBiasPos) {
#pragma unroll
        for (int r = 0; r < RT; r++) bias[r] = *reinterpret_cast<const float4 *>(cur.bias + r * 16 + 4 * g);
      }
      if constexpr (p < NSR) {
        if (NSR == 23 || p < ns) {  // (NSR = 24: steps from ns on are repeats)
          const uint8_t *eb = &sB[p % PB][0][0] + cur.area * kBArea + j * G::kStep;
          i32x8 bv[NT];
#pragma unroll
          for (int tt = 0; tt < NT; tt++) {
            const uint4 h = *reinterpret_cast<const uint4 *>(eb + tt * G::kTermBytes + 16 * g);
            const uint2 tl = *reinterpret_cast<const uint2 *>(eb + tt * G::kTermBytes + 64 + 8 * g);
            bv[tt] = i32x8{(int)h.x, (int)h.y, (int)h.z, (int)h.w, (int)tl.x, (int)tl.y, 0, 0};
          }
          const uint4 bsc = *reinterpret_cast<const uint4 *>(eb + NT * G::kTermBytes);
          const StrSlot<RT> &sl = ring[p % PA];
          const uint32_t(&sa)[RT] = sw[(p / 4) % QR];
          const int sh = 8 * (p % 4);
#pragma unroll
          for (int tt = 0; tt < NT; tt++) {
            const uint32_t wsc = tt == 0 ? bsc.x : (tt == 1 ? bsc.y : bsc.z);
            const int sb = (int)(wsc >> (8 * g));
#pragma unroll
            for (int r = 0; r < RT; r++) {
              const i32x8 A = {(int)sl.a[r].x, (int)sl.a[r].y, (int)sl.a[r].z, (int)sl.a[r].w, 0, 0, 0, 0};
              // cbsz 4: A is fp4 (E2M1); blgp 2: B is fp6 (E2M3)
              acc[r] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, bv[tt], acc[r], 4, 2, 0, (int)(sa[r] >> sh), 0, sb);
            }
          }
          // the step's MFMAs stay here (IR passes otherwise sink them towards the epilogue, keeping
          // every step's operands live at once)
#pragma unroll
          for (int r = 0; r < RT; r++) asm volatile("" ::"a"(acc[r]) : "memory");
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // the loads PA steps ahead: this round's, or the next round's first steps
      {
        constexpr int sp = p + PA;
        if constexpr (sp < kStrPos) {
          if constexpr (sp < NSR) load_step(cur, sp, sp % PA);
        } else if constexpr (sp - kStrPos < NSR) {
          load_step(nxt, sp - kStrPos, (sp - kStrPos) % PA);
        }
      }
      if constexpr (p == kStrPos - 1) {
        // ---- epilogue of this wavefront's unit of round k
        if (cur.store) {
          if constexpr (MODE == GEMV_GATE_UP) {
            // lane (j, g) holds rows 16 r + 4 g .. + 3 of the group (gate = row 2i, up = row 2i + 1):
            // h values 8 r + 2 g, 8 r + 2 g + 1 of entry j's 32-value block; staged per wavefront,
            // then lane e splits entry e's whole block into the NT terms of its h record
            float *st = s_stage[wvu];
#pragma unroll
            for (int r = 0; r < RT; r++) {
              const float4 b4 = bias[r];
              *reinterpret_cast<float2 *>(st + j * kStrRow + 8 * r + 2 * g) =
                  make_float2(swiglu_fast(acc[r][0] + b4.x, acc[r][1] + b4.y, a.limit),
                              swiglu_fast(acc[r][2] + b4.z, acc[r][3] + b4.w, a.limit));
            }
            if (lane < cur.cnt) {
              float v[32];
#pragma unroll
              for (int k4 = 0; k4 < 8; k4++) {
                const float4 x = *reinterpret_cast<const float4 *>(st + lane * kStrRow + 4 * k4);
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
              const int hb = cur.grp, st_ = hb >> 2, i = hb & 3;
              uint8_t *hr = reinterpret_cast<uint8_t *>(a.out) + (size_t)(cur.beg + lane) * G::kBytes;
#pragma unroll
              for (int tt = 0; tt < NT; tt++) {
                str_st16(hr + G::dword(st_, tt, i, 0), make_uint4(dq[tt][0], dq[tt][1], dq[tt][2], dq[tt][3]));
                str_st8(hr + G::dword(st_, tt, i, 4), make_uint2(dq[tt][4], dq[tt][5]));
                str_st1(hr + G::scale(st_, tt) + i, (sbw >> (8 * tt)) & 0xFFu);
              }
            }
          } else {
            if (j < cur.cnt) {
              float *o = reinterpret_cast<float *>(a.out) + (size_t)(cur.beg + j) * d.rows + (size_t)cur.grp * RT * 16 + 4 * g;
#pragma unroll
              for (int r = 0; r < RT; r++) {
                const float4 b4 = bias[r];
                float4 v;
                v.x = canon_nan(rclamp(acc[r][0] + b4.x, -65504.0f, 65504.0f));
                v.y = canon_nan(rclamp(acc[r][1] + b4.y, -65504.0f, 65504.0f));
                v.z = canon_nan(rclamp(acc[r][2] + b4.z, -65504.0f, 65504.0f));
                v.w = canon_nan(rclamp(acc[r][3] + b4.w, -65504.0f, 65504.0f));
                str_st16(o + r * 16, make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                                                __float_as_uint(v.w)));
              }
            }
          }
        }
#pragma unroll
        for (int r = 0; r < RT; r++) acc[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    });
    cur = nxt;
  }
  __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(0));  // (the last round's repeats and the stores)
}

// Whether a gate_up launch with these arguments would run the streamed kernel (its shape choice in
// launch_gemm_fp8 and the fit below) with a batch small enough to group locally.
bool gemm_stream_local_ok(const GemmArgs &a);

// Whether the launch fits the streamed kernel: whole units, K <= 3072, at least 3 units per chunk
// (4 consecutive units then touch at most two chunks) and, from the host's upper bound on the
// chunks (entries / 16 + active experts), at most kStrMaxSeg chunks per workgroup range.
static bool gemm_stream_fits(const GemmArgs &a, int rt, int n_wg) {
  if (a.d.tiles % rt || a.d.ns > (uint32_t)kGemmNs || a.max_active > kMaxExperts || n_wg % 8) return false;
  const long long gu = a.d.tiles / rt;
  if (gu < 3) return false;
  const long long nc = (long long)(a.n_entries / kStrCols) + std::min<long long>(a.max_active, (long long)a.n_entries);
  if (gu * nc > INT32_MAX / 2) return false;
  const long long per = (gu * nc + n_wg - 1) / n_wg;
  const long long segs = per > 0 ? (per + gu - 2) / gu + 1 : 1;
  return segs <= kStrMaxSeg;
}

static int stream_cus();
bool gemm_stream_local_ok(const GemmArgs &a) {
  return a.n_entries <= (size_t)kLocalGroupMax && a.terms == kGemmTerms && gemm_stream_fits(a, 4, stream_cus());
}

static int stream_cus() {
  static std::atomic<int> cus[64] = {};
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

template <int MODE, int RT, int PA, int PB, int NT>
static hipError_t launch_stream_rt(const GemmArgs &a, hipStream_t s, int n_wg) {
  if (a.d.ns == 23)
    hipLaunchKernelGGL((k_gemm_stream<MODE, RT, 23, PA, PB, NT>), dim3((unsigned)n_wg), dim3(64 * kStrWaves), 0, s, a);
  else
    hipLaunchKernelGGL((k_gemm_stream<MODE, RT, 24, PA, PB, NT>), dim3((unsigned)n_wg), dim3(64 * kStrWaves), 0, s, a);
  return hipGetLastError();
}

// The streamed kernel for this launch, or hipErrorNotSupported when it does not fit (the caller
// then runs k_gemm_fp8). Register rings of PA steps for A (gate_up 3, down 8), LDS rings of 4
// steps for B (measured at 64, 96 and 128 tokens: as fast or faster than deeper B rings); alt:
// 4 and 6 for A, 6 for B (tuning).
hipError_t launch_gemm_stream(GemvMode mode, const GemmArgs &a, hipStream_t s, bool alt) {
  const int n_wg = stream_cus();
  if (!a.n_entries) return hipSuccess;
  const bool one = a.terms == 1;
  if (mode == GEMV_GATE_UP) {
    if (!gemm_stream_fits(a, 4, n_wg)) return hipErrorNotSupported;
    if (alt)
      return one ? launch_stream_rt<GEMV_GATE_UP, 4, 4, 6, 1>(a, s, n_wg) : launch_stream_rt<GEMV_GATE_UP, 4, 4, 6, kGemmTerms>(a, s, n_wg);
    return one ? launch_stream_rt<GEMV_GATE_UP, 4, 3, 4, 1>(a, s, n_wg) : launch_stream_rt<GEMV_GATE_UP, 4, 3, 4, kGemmTerms>(a, s, n_wg);
  }
  if (!gemm_stream_fits(a, 2, n_wg)) return hipErrorNotSupported;
  if (alt)
    return one ? launch_stream_rt<GEMV_DOWN, 2, 6, 6, 1>(a, s, n_wg) : launch_stream_rt<GEMV_DOWN, 2, 6, 6, kGemmTerms>(a, s, n_wg);
  return one ? launch_stream_rt<GEMV_DOWN, 2, 8, 4, 1>(a, s, n_wg) : launch_stream_rt<GEMV_DOWN, 2, 8, 4, kGemmTerms>(a, s, n_wg);
}

}  // namespace moe
