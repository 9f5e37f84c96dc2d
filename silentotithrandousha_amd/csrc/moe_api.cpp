// C ABI of the MXFP4 MoE path (include/mxfp4_moe.h): context, HBM residency, dispatch.
// Host logic only; every kernel lives in kernels.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/mxfp4_moe.h"
#include "kernels.hpp"
#include "layout.hpp"

using namespace moe;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define HIP_TRY(call)                                                                      \
  do {                                                                                     \
    hipError_t e_ = (call);                                                                \
    if (e_ != hipSuccess)                                                                  \
      return fail(e_ == hipErrorOutOfMemory ? MOE_ERR_OOM : MOE_ERR_HIP, "%s: %s (%s:%d)", \
                  #call, hipGetErrorString(e_), __FILE__, __LINE__);                       \
  } while (0)

#define RETURN_IF(rc) \
  do {                \
    int r_ = (rc);    \
    if (r_) return r_; \
  } while (0)

struct DevBuf {
  void *p = nullptr;
  size_t cap = 0;
  // Grows the buffer. The new allocation is made before the old one is freed, so a failed
  // call leaves the buffer (and every pointer carved from it) as it was.
  int ensure(size_t bytes) {
    if (bytes <= cap) return MOE_OK;
    const size_t want = std::max(bytes, (size_t)4096);
    void *q = nullptr;
    hipError_t e = hipMalloc(&q, want);
    if (e != hipSuccess) return fail(MOE_ERR_OOM, "hipMalloc(%zu): %s", want, hipGetErrorString(e));
    if (p) (void)hipFree(p);
    p = q;
    cap = want;
    return MOE_OK;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
  }
};

struct Layer {
  DevBuf experts;  // n_experts * stride
  size_t n_experts = 0;
  std::vector<uint8_t> loaded;  // per expert: its record has been written
  size_t n_loaded = 0;
  DevBuf router;   // load-major bf16 [E][KIp/8][64][8] then [E] f32
  size_t router_experts = 0;
  DevBuf norm;     // post-attention RMSNorm weight, f32 [H]
  float eps = 0.0f;
  bool has_norm = false;
};

// Per-call device scratch, carved from one allocation.
struct Work {
  float *x, *y, *logits, *wts, *o, *xn;  // xn: normalised rows of the block forward
  uint16_t *xsplit, *hsplit;
  uint8_t *xrec, *hrec;  // grouped GEMM activation records: tokens, entries (padding zero)
  int32_t *idx, *n_active, *active_ids, *active_off, *entry_src, *pos;
  int32_t *blk_count, *rank;  // the router's grouping: per-block expert counts, per-entry ranks
  size_t hrec_bytes;     // bytes of hrec, which must hold zeros where no kernel writes
};

enum {
  K_ROUTE = 0, K_BUCKET, K_GATE_UP, K_DOWN, K_COMBINE, K_DECODE_GATE_UP, K_DECODE_DOWN,
  K_DECODE_LAYER, K_RESERVED, K_NORM, K_COUNT
};

struct TimingRec {
  int kernel;
  hipEvent_t a, b;
};

}  // namespace

struct moe_ctx {
  int dev = 0;
  hipStream_t stream = nullptr;
  size_t H = 0, I = 0;
  float clamp = 7.0f;
  ExpertLayout L;
  std::vector<Layer> layers;
  int ad_enabled = 0;
  size_t ad_min_k = 1;
  float ad_top1 = 0.9f, ad_margin = 0.35f, ad_top2 = 0.98f;
  DevBuf work;
  size_t work_T = 0, work_k = 0, work_E = 0;
  Work w{};
  DevBuf scratch_experts;  // dispatch_expert / batched: experts uploaded per call
  DevBuf stage;            // checkpoint-layout staging for uploads
  DevBuf mv_split;         // matvec: [one-entry expert list | x split]
  void *mv_list_at = nullptr;  // mv_split.p when its list was written
  DevBuf lm_w, lm_x, lm_y;
  size_t lm_vocab = 0;
  bool lm_bf16 = false;  // lm_w holds the checkpoint's bf16 rows (else f32)
  bool timing = false;
  bool capturing = false;
  // single-token forwards: 0 = the batch path, 1 = two decode kernels, 2 = one launch
  // (falls back to 1, then 0, where a shape is not supported)
  int decode_mode = 2;
  int batch_gemm = 1;  // batches: 1 grouped GEMM when experts average >= 4 entries, 2 always, 0 never
  int gemm_shape = 0;  // grouped GEMM block shape override (tuning)
  int matvec_one_launch = 1;  // moe_mxfp4_matvec_device: one launch (1) or split + GEMV (0)
  int gemm_band = 0;
  int gemm_shape_down = 0;  // block shape of the down GEMM (0: as gemm_shape)
  int act_quant = 0;  // grouped GEMM activations: 0 the exact kGemmTerms split, 1 one MXFP6 term
  int local_group = 1;  // small batches on the streamed GEMM: its workgroups group the entries
  DevBuf route_ticket;  // k_route's block counter for the fused bucketing, zero between launches
  DevBuf gemm_queue;    // the persistent grouped GEMM's tile queue (10 counters), zero between launches
  DevBuf layer_sync;  // cross-block signalling of the one-launch kernel, zero between launches
  DevBuf layer_h;     // h records of the one-launch kernel's slots (values past I stay zero)
  int n_cu = 256;     // compute units of the device (the one-launch grid is sized to it)
  uint32_t spin_limit = 1u << 20;
  void *scratch = nullptr;  // this device's scratch array (moe_layer_forward_device_noalloc)
  std::vector<TimingRec> recs;
  std::vector<hipEvent_t> pool;
  double acc_ms[K_COUNT] = {};
  uint64_t acc_n[K_COUNT] = {};
};

namespace {

int use_dev(moe_ctx *c) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  HIP_TRY(hipSetDevice(c->dev));
  return MOE_OK;
}

hipStream_t pick(moe_ctx *c, void *s) { return s ? (hipStream_t)s : c->stream; }

int take_event(moe_ctx *c, hipEvent_t *e) {
  if (!c->pool.empty()) {
    *e = c->pool.back();
    c->pool.pop_back();
    return MOE_OK;
  }
  HIP_TRY(hipEventCreate(e));
  return MOE_OK;
}

// Launch wrapper: records a HIP event pair around the launch when timing is on.
template <class F>
int timed(moe_ctx *c, int kernel, hipStream_t s, F &&launch) {
  TimingRec r{kernel, nullptr, nullptr};
  if (c->timing) {
    RETURN_IF(take_event(c, &r.a));
    RETURN_IF(take_event(c, &r.b));
    HIP_TRY(hipEventRecord(r.a, s));
  }
  hipError_t e = launch();
  if (e != hipSuccess) return fail(MOE_ERR_HIP, "kernel %d launch: %s", kernel, hipGetErrorString(e));
  if (c->timing) {
    HIP_TRY(hipEventRecord(r.b, s));
    c->recs.push_back(r);
  }
  return MOE_OK;
}

int collect_timing(moe_ctx *c) {
  for (auto &r : c->recs) {
    HIP_TRY(hipEventSynchronize(r.b));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, r.a, r.b));
    c->acc_ms[r.kernel] += ms;
    c->acc_n[r.kernel] += 1;
    c->pool.push_back(r.a);
    c->pool.push_back(r.b);
  }
  c->recs.clear();
  return MOE_OK;
}

size_t al(size_t v) { return align_up(v, 256); }

constexpr size_t kMaxTokens = (size_t)1 << 20;  // tokens per path-level call

// Router chain length per lane, rounded up to whole 16-byte loads (8 bf16).
size_t router_kip(size_t H) { return ((H + 63) / 64 + 7) / 8 * 8; }
size_t router_bytes(size_t H, size_t E) { return E * 64 * router_kip(H) * 2; }

// Lays out the per-call workspace of T tokens, top-k k and E experts at `b` (nullptr: sizes
// only) and returns its bytes. host_io adds the staging rows of host-pointer calls (x, y) and
// the normalised rows of the unfused block forward (xn).
size_t carve_work(Work &w, char *b, size_t T, size_t k, size_t E, size_t H, size_t I, bool host_io) {
  const size_t N = T * k;
  size_t off = 0;
  auto take = [&](size_t bytes) -> char * {
    const size_t o = off;
    off = al(off + bytes);
    return b && bytes ? b + o : nullptr;
  };
  w.x = (float *)take(host_io ? T * H * 4 : 0);
  w.y = (float *)take(host_io ? T * H * 4 : 0);
  w.xn = (float *)take(host_io ? T * H * 4 : 0);
  w.logits = (float *)take(T * E * 4);
  w.wts = (float *)take(N * 4);
  w.o = (float *)take(N * H * 4);
  w.xsplit = (uint16_t *)take(T * 2 * H * 2);
  w.hsplit = (uint16_t *)take(N * 2 * I * 2);
  w.idx = (int32_t *)take(N * 4);
  w.n_active = (int32_t *)take(4);
  w.active_ids = (int32_t *)take(E * 4);
  w.active_off = (int32_t *)take((E + 1) * 4);
  w.entry_src = (int32_t *)take(N * 4);
  w.pos = (int32_t *)take(N * 4);
  w.blk_count = (int32_t *)take(T * E * 4);  // router blocks <= T
  w.rank = (int32_t *)take(N * 4);
  w.xrec = (uint8_t *)take(T * GemmRec::kBytes);
  w.hrec_bytes = N * GemmRec::kBytes;
  w.hrec = (uint8_t *)take(w.hrec_bytes);
  return off;
}

int ensure_work(moe_ctx *c, size_t T, size_t k, size_t E) {
  if (T <= c->work_T && k <= c->work_k && E <= c->work_E) return MOE_OK;
  if (c->capturing)
    return fail(MOE_ERR_STATE, "workspace too small for this call during graph capture; run it once uncaptured first");
  T = std::max(T, c->work_T);
  k = std::max(k, c->work_k);
  E = std::max({E, c->work_E, (size_t)kMaxExperts});
  Work w{};
  // ensure() may release the old buffer: forget it first, so that a failure below leaves an empty
  // workspace (the next call sizes it again) and never pointers into freed memory
  c->w = Work{};
  c->work_T = c->work_k = c->work_E = 0;
  RETURN_IF(c->work.ensure(carve_work(w, nullptr, T, k, E, c->H, c->I, true)));
  carve_work(w, (char *)c->work.p, T, k, E, c->H, c->I, true);
  // h records are written block by block; their padding past I must read as zeros
  HIP_TRY(hipMemset(w.hrec, 0, w.hrec_bytes));
  c->w = w;
  c->work_T = T;
  c->work_k = k;
  c->work_E = E;
  return MOE_OK;
}

GemvArgs gemv_args(moe_ctx *c, const Work &w, const uint8_t *base, bool gate_up) {
  GemvArgs a{};
  a.base = base;
  a.stride = c->L.stride;
  a.mat_off = gate_up ? c->L.gu_off : c->L.dn_off;
  a.bias_off = gate_up ? c->L.gub_off : c->L.dnb_off;
  a.d = gate_up ? c->L.gu : c->L.dn;
  a.n_active = w.n_active;
  a.active_ids = w.active_ids;
  a.active_off = w.active_off;
  a.limit = c->clamp;
  return a;
}

// gate_up -> down for the expert list already in the workspace; outputs in w.o[entry].
int run_experts(moe_ctx *c, const Work &w, const uint8_t *base, int max_active, int max_entries,
                hipStream_t s) {
  GemvArgs gu = gemv_args(c, w, base, true);
  gu.entry_src = w.entry_src;
  gu.bsrc = w.xsplit;
  gu.out = w.hsplit;
  gu.max_active = max_active;
  gu.max_entries_per_expert = max_entries;
  RETURN_IF(timed(c, K_GATE_UP, s, [&] { return launch_gemv(GEMV_GATE_UP, gu, s); }));
  GemvArgs dn = gemv_args(c, w, base, false);
  dn.entry_src = nullptr;
  dn.bsrc = w.hsplit;
  dn.out = w.o;
  dn.max_active = max_active;
  dn.max_entries_per_expert = max_entries;
  RETURN_IF(timed(c, K_DOWN, s, [&] { return launch_gemv(GEMV_DOWN, dn, s); }));
  return MOE_OK;
}

// The one-launch kernel sets a sticky error word when one of its bounded waits ran out (its
// outputs are NaN from then on). Reports it once and clears the signalling area.
int check_layer_sync(moe_ctx *c) {
  uint32_t err = 0;
  HIP_TRY(hipMemcpy(&err, c->layer_sync.p, 4, hipMemcpyDeviceToHost));
  if (!err) return MOE_OK;
  HIP_TRY(hipMemset(c->layer_sync.p, 0, layer_sync_bytes()));
  return fail(MOE_ERR_HIP, "single-token layer kernel: a cross-block wait ran out (outputs since "
                           "the last synchronisation are NaN)");
}

// expert < 0: every expert of the layer must be preloaded; else that one expert.
int check_layer(moe_ctx *c, size_t layer, bool need_router, long expert = -1) {
  if (layer >= c->layers.size() || !c->layers[layer].experts.p)
    return fail(MOE_ERR_STATE, "layer %zu has no preloaded experts", layer);
  if (expert >= 0) {
    if ((size_t)expert >= c->layers[layer].n_experts)
      return fail(MOE_ERR_INVALID, "expert %ld >= %zu", expert, c->layers[layer].n_experts);
    if (!c->layers[layer].loaded[expert])
      return fail(MOE_ERR_STATE, "layer %zu expert %ld is not preloaded", layer, expert);
  } else if (c->layers[layer].n_loaded != c->layers[layer].n_experts)
    return fail(MOE_ERR_STATE, "layer %zu has %zu of its %zu experts preloaded", layer,
                c->layers[layer].n_loaded, c->layers[layer].n_experts);
  if (need_router && !c->layers[layer].router.p)
    return fail(MOE_ERR_STATE, "layer %zu has no router weights", layer);
  return MOE_OK;
}

// Token count and top-k of a path-level call on a loaded layer (checked before any workspace
// is sized for them).
// E: the experts top_k selects from (the layer's, or its router's for a router-only call).
int check_tokens(size_t E, size_t T, size_t k) {
  if (k < 1 || k > (size_t)kMaxTopK || k > E)
    return fail(MOE_ERR_INVALID, "top_k %zu outside [1, min(%d, %zu)]", k, kMaxTopK, E);
  if (T > kMaxTokens) return fail(MOE_ERR_INVALID, "n_tokens %zu above %zu", T, kMaxTokens);
  return MOE_OK;
}

// Expert sizes in the checkpoint layout.
struct ExpertBytes {
  size_t gub, gus, gubias, db, ds, dbias;
};
ExpertBytes expert_bytes(const moe_ctx *c) {
  const size_t H = c->H, I = c->I;
  return {2 * I * (H / 32) * 16, 2 * I * (H / 32), 2 * I, H * (I / 32) * 16, H * (I / 32), H};
}

// Packs one expert from device checkpoint tensors into its resident record.
int pack_expert(moe_ctx *c, uint8_t *rec, const uint8_t *gub, const uint8_t *gus,
                const float *gubias, const uint8_t *db, const uint8_t *ds, const float *dbias,
                hipStream_t s) {
  HIP_TRY(launch_pack(gub, gus, 2 * c->I, c->H, rec + c->L.gu_off, s));
  HIP_TRY(launch_pack(db, ds, c->H, c->I, rec + c->L.dn_off, s));
  HIP_TRY(hipMemcpyAsync(rec + c->L.gub_off, gubias, 2 * c->I * 4, hipMemcpyDeviceToDevice, s));
  HIP_TRY(hipMemcpyAsync(rec + c->L.dnb_off, dbias, c->H * 4, hipMemcpyDeviceToDevice, s));
  return MOE_OK;
}

// Uploads one expert given as host tensors (biases zero-padded) into `rec`, via staging.
int upload_expert(moe_ctx *c, uint8_t *rec, const uint8_t *gub, size_t gub_len,
                  const uint8_t *gus, size_t gus_len, const float *gubias, size_t gubias_len,
                  const uint8_t *db, size_t db_len, const uint8_t *ds, size_t ds_len,
                  const float *dbias, size_t dbias_len) {
  const ExpertBytes eb = expert_bytes(c);
  if (!gub || !gus || !db || !ds) return fail(MOE_ERR_INVALID, "null expert tensor");
  if (gub_len != eb.gub || gus_len != eb.gus || db_len != eb.db || ds_len != eb.ds)
    return fail(MOE_ERR_INVALID,
                "expert tensor lengths (%zu,%zu,%zu,%zu) differ from (%zu,%zu,%zu,%zu)", gub_len,
                gus_len, db_len, ds_len, eb.gub, eb.gus, eb.db, eb.ds);
  if (gubias_len > eb.gubias || dbias_len > eb.dbias || (gubias_len && !gubias) ||
      (dbias_len && !dbias))
    return fail(MOE_ERR_INVALID, "bias longer than the expert's rows or null");
  const size_t o_gub = 0, o_gus = al(o_gub + eb.gub), o_db = al(o_gus + eb.gus),
               o_ds = al(o_db + eb.db), o_gb = al(o_ds + eb.ds), o_dbias = al(o_gb + eb.gubias * 4),
               total = al(o_dbias + eb.dbias * 4);
  RETURN_IF(c->stage.ensure(total));
  uint8_t *st = (uint8_t *)c->stage.p;
  std::vector<float> gb(eb.gubias, 0.0f), dbv(eb.dbias, 0.0f);
  if (gubias_len) std::memcpy(gb.data(), gubias, gubias_len * 4);
  if (dbias_len) std::memcpy(dbv.data(), dbias, dbias_len * 4);
  HIP_TRY(hipMemcpyAsync(st + o_gub, gub, eb.gub, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(st + o_gus, gus, eb.gus, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(st + o_db, db, eb.db, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(st + o_ds, ds, eb.ds, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(st + o_gb, gb.data(), eb.gubias * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(st + o_dbias, dbv.data(), eb.dbias * 4, hipMemcpyHostToDevice, c->stream));
  RETURN_IF(pack_expert(c, rec, st + o_gub, st + o_gus, (const float *)(st + o_gb), st + o_db,
                        st + o_ds, (const float *)(st + o_dbias), c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));  // staging is reused by the next upload
  return MOE_OK;
}

// Writes the expert list of a single-token dispatch over `n` experts (record ids 0..n-1 or
// `ids`) with unit entries, all reading B row 0, and pos[s] = s.
int set_single_token_list(moe_ctx *c, size_t n, const int32_t *ids) {
  std::vector<int32_t> h(3 * n + 2);
  int32_t *act = h.data(), *off = act + n, *src = off + n + 1;
  for (size_t i = 0; i < n; i++) {
    act[i] = ids ? ids[i] : (int32_t)i;
    off[i] = (int32_t)i;
    src[i] = 0;
  }
  off[n] = (int32_t)n;
  int32_t na = (int32_t)n;
  HIP_TRY(hipMemcpyAsync(c->w.n_active, &na, 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(c->w.active_ids, act, n * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(c->w.active_off, off, (n + 1) * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(c->w.entry_src, src, n * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(c->w.pos, off, n * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

// norm: the block forward (RMSNorm of x before, x + result after); the one-launch decode fuses
// both, the other paths run k_rmsnorm into the workspace first and k_add_rows last.
// w: the workspace, sized for (T, k, E) by the caller (ensure_work, or the scratch array of the
// allocation-free entry point).
int forward_device(moe_ctx *c, const Work &w, size_t layer, const float *x, size_t T, size_t k,
                   float *y, hipStream_t s, bool norm = false) {
  RETURN_IF(check_layer(c, layer, true));
  Layer &Ly = c->layers[layer];
  const size_t E = Ly.n_experts;
  if (Ly.router_experts != E)
    return fail(MOE_ERR_STATE, "layer %zu router has %zu experts, layer has %zu", layer,
                Ly.router_experts, E);
  if (T == 0) return MOE_OK;
  if (!x || !y) return fail(MOE_ERR_INVALID, "null x or y");
  RETURN_IF(check_tokens(c->layers[layer].n_experts, T, k));
  if (norm && !Ly.has_norm) return fail(MOE_ERR_STATE, "layer %zu has no RMSNorm weight", layer);
  const float *resid = nullptr;  // x for the residual add of the unfused paths
  if (norm) {
    const bool fused = T == 1 && c->decode_mode == 2;
    if (!fused || (reinterpret_cast<uintptr_t>(x) & 15)) {
      RETURN_IF(timed(c, K_NORM, s, [&] {
        return launch_rmsnorm(x, T, c->H, (const float *)Ly.norm.p, Ly.eps, w.xn, s);
      }));
      resid = x;
      x = w.xn;
      norm = false;
    }
  }
  if (T == 1 && c->decode_mode > 0) {
    DecodeArgs da{};
    da.rw = (const uint16_t *)Ly.router.p;
    da.rb = (const float *)((const char *)Ly.router.p + al(router_bytes(c->H, E)));
    da.rnq = (int)(router_kip(c->H) / 8);
    da.Hr = da.rnq * 8 * 64;
    da.base = (const uint8_t *)Ly.experts.p;
    da.stride = c->L.stride;
    da.gu_off = c->L.gu_off;
    da.dn_off = c->L.dn_off;
    da.gub_off = c->L.gub_off;
    da.dnb_off = c->L.dnb_off;
    da.gu = c->L.gu;
    da.dn = c->L.dn;
    da.H = (int)c->H;
    da.I = (int)c->I;
    da.E = (int)E;
    da.k = (int)k;
    da.limit = c->clamp;
    da.adaptive = c->ad_enabled;
    da.min_k = (int)c->ad_min_k;
    da.top1_min = c->ad_top1;
    da.margin_min = c->ad_margin;
    da.top2_mass = c->ad_top2;
    da.x = x;
    da.y = y;
    da.logits = w.logits;
    da.idx = w.idx;
    da.wts = w.wts;
    da.hsplit = w.hsplit;
    da.n_gu_wg_per_slot = (int)((c->L.gu.tiles + 3) / 4);
    LayerArgs la{};
    la.d = da;
    la.sync = c->layer_sync.p;
    la.hterm = (uint8_t *)c->layer_h.p;
    la.spin_limit = c->spin_limit;
    if (norm) {
      la.gamma = (const float *)Ly.norm.p;
      la.eps = Ly.eps;
    }
    layer_geometry(la, c->n_cu);
    if (c->decode_mode == 2 && decode_layer_supported(la))
      return timed(c, K_DECODE_LAYER, s, [&] { return launch_decode_layer(la, s); });
    if (norm) {  // the fused kernel refused the shape: normalise first, add the residual last
      RETURN_IF(timed(c, K_NORM, s, [&] {
        return launch_rmsnorm(x, T, c->H, (const float *)Ly.norm.p, Ly.eps, w.xn, s);
      }));
      resid = x;
      x = w.xn;
      da.x = x;
    }
    if (decode_supported(da)) {
      RETURN_IF(timed(c, K_DECODE_GATE_UP, s, [&] { return launch_decode_gate_up(da, s); }));
      RETURN_IF(timed(c, K_DECODE_DOWN, s, [&] { return launch_decode_down(da, s); }));
      if (resid) RETURN_IF(timed(c, K_NORM, s, [&] { return launch_add_rows(y, resid, T * c->H, s); }));
      return MOE_OK;
    }
  }
  RouteArgs ra{};
  ra.w = (const uint16_t *)Ly.router.p;
  ra.bias = (const float *)((const char *)Ly.router.p + al(router_bytes(c->H, E)));
  ra.x = x;
  ra.T = (int)T;
  ra.E = (int)E;
  ra.H = (int)c->H;
  ra.k = (int)k;
  ra.adaptive = c->ad_enabled;
  ra.min_k = (int)c->ad_min_k;
  ra.top1_min = c->ad_top1;
  ra.margin_min = c->ad_margin;
  ra.top2_mass = c->ad_top2;
  ra.logits = w.logits;
  ra.idx = w.idx;
  ra.wts = w.wts;
  // the grouped GEMM (16- to 64-entry column tiles) pays off once experts average a few
  // entries; smaller batches stream each weight tile through the GEMV kernels, which read the
  // bf16 hi + lo split of x that the router writes
  const bool use_gemm = c->batch_gemm && T > 1 && (c->batch_gemm == 2 || T * k >= 4 * E) &&
                        c->L.gu.ns <= (uint32_t)kGemmNs && c->L.dn.ns <= (uint32_t)kGemmNs &&
                        (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  ra.xsplit = use_gemm ? nullptr : w.xsplit;
  ra.xrec = use_gemm ? w.xrec : nullptr;  // the router writes the GEMM's activation records
  ra.rec_terms = c->act_quant ? 1 : kGemmTerms;
  ra.fuse_bucket = T == 1;
  ra.n_active = w.n_active;
  ra.active_ids = w.active_ids;
  ra.active_off = w.active_off;
  ra.entry_src = w.entry_src;
  ra.pos = w.pos;
  const int max_active = (int)std::min(E, T * k);
  GemmArgs ga{}, gu{};
  if (use_gemm) {
    const size_t N = T * k;
    ga.base = (const uint8_t *)Ly.experts.p;
    ga.stride = c->L.stride;
    ga.n_active = w.n_active;
    ga.active_ids = w.active_ids;
    ga.active_off = w.active_off;
    ga.limit = c->clamp;
    ga.max_active = max_active;
    ga.n_entries = N;
    ga.shape = c->gemm_shape;
    ga.band = c->gemm_band;  // default: gate_up in workgroup order, down in XCD bands of 1 row block
    ga.terms = c->act_quant ? 1 : kGemmTerms;
    ga.queue = (int32_t *)c->gemm_queue.p;
    gu = ga;
    gu.mat_off = c->L.gu_off;
    gu.bias_off = c->L.gub_off;
    gu.d = c->L.gu;
    gu.entry_src = w.entry_src;
    gu.brec = w.xrec;
    gu.out = w.hrec;
  }
  // small batches on the streamed gate_up GEMM: its workgroups group the entries by expert
  // themselves (one round trip for the top-k indices, where the router's grouping took a
  // grid-wide ticket and a pass of its last block, and the GEMM two dependent round trips for
  // the lists and entry_src); its workgroup 0 writes the lists for the down GEMM and the combine
  const bool local_group = use_gemm && c->local_group && gemm_gate_up_groups_locally(gu);
  if (local_group) {
    gu.group_idx = w.idx;
    gu.group_k = (int)k;
    gu.group_E = (int)E;
    gu.w_n_active = w.n_active;
    gu.w_active_ids = w.active_ids;
    gu.w_active_off = w.active_off;
    gu.w_entry_src = w.entry_src;
    gu.w_pos = w.pos;
  }
  const bool fuse_bucket = T > 1 && !local_group && route_bucket_fits((int)c->H, (int)E);
  ra.bucket_ticket = fuse_bucket ? (uint32_t *)c->route_ticket.p : nullptr;
  ra.blk_count = w.blk_count;
  ra.rank = w.rank;
  RETURN_IF(timed(c, K_ROUTE, s, [&] { return launch_route(ra, s); }));
  if (T > 1 && !fuse_bucket && !local_group)
    RETURN_IF(timed(c, K_BUCKET, s, [&] {
      return launch_bucket(w.idx, (int)T, (int)k, (int)E, w.n_active, w.active_ids,
                           w.active_off, w.entry_src, w.pos, s);
    }));
  if (use_gemm) {
    RETURN_IF(timed(c, K_GATE_UP, s, [&] { return launch_gemm_fp8(GEMV_GATE_UP, gu, s); }));
    GemmArgs dn = ga;
    if (!c->gemm_band) dn.band = 1;
    if (c->gemm_shape_down) dn.shape = c->gemm_shape_down;
    dn.mat_off = c->L.dn_off;
    dn.bias_off = c->L.dnb_off;
    dn.d = c->L.dn;
    dn.entry_src = nullptr;
    dn.brec = w.hrec;
    dn.out = w.o;
    RETURN_IF(timed(c, K_DOWN, s, [&] { return launch_gemm_fp8(GEMV_DOWN, dn, s); }));
  } else {
    RETURN_IF(run_experts(c, w, (const uint8_t *)Ly.experts.p, max_active, (int)std::min(T, (size_t)1 << 30), s));
  }
  RETURN_IF(timed(c, K_COMBINE, s, [&] {
    return launch_combine(w.o, w.pos, w.wts, (int)T, (int)k, (int)c->H, 0, y, s);
  }));
  if (resid) RETURN_IF(timed(c, K_NORM, s, [&] { return launch_add_rows(y, resid, T * c->H, s); }));
  return MOE_OK;
}

}  // namespace

// ======================================================================== exported

extern "C" {

const char *moe_last_error(void) { return g_last_error.c_str(); }
const char *moe_version(void) { return "mxfp4_moe 0.1 (gfx950)"; }

int moe_create(size_t hidden_size, size_t inter_size, float swiglu_clamp, moe_ctx **out) {
  if (!out) return fail(MOE_ERR_INVALID, "null out");
  *out = nullptr;
  if (!hidden_size || !inter_size || hidden_size % 32 || inter_size % 32)
    return fail(MOE_ERR_INVALID, "hidden_size %zu and inter_size %zu must be positive multiples of 32",
                hidden_size, inter_size);
  if (!(swiglu_clamp > 0.0f) || !std::isfinite(swiglu_clamp))
    return fail(MOE_ERR_INVALID, "swiglu_clamp must be positive and finite");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return fail(MOE_ERR_NO_DEVICE, "no HIP device");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, dev));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MOE_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950", dev,
                prop.gcnArchName);
  moe_ctx *c = new moe_ctx();
  c->dev = dev;
  c->n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  c->H = hidden_size;
  c->I = inter_size;
  c->clamp = swiglu_clamp;
  c->L = expert_layout(hidden_size, inter_size);
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return fail(MOE_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  // this device's copy of the allocation-free forward's scratch array (resolved once per device)
  e = noalloc_scratch_ptr(dev, &c->scratch);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return fail(MOE_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  }
  const size_t sb = layer_sync_bytes(), hb = layer_hterm_bytes();
  if (c->layer_sync.ensure(sb) != MOE_OK || hipMemset(c->layer_sync.p, 0, sb) != hipSuccess ||
      c->route_ticket.ensure(256) != MOE_OK || hipMemset(c->route_ticket.p, 0, 256) != hipSuccess ||
      c->gemm_queue.ensure(256) != MOE_OK || hipMemset(c->gemm_queue.p, 0, 256) != hipSuccess ||
      c->layer_h.ensure(hb) != MOE_OK || hipMemset(c->layer_h.p, 0, hb) != hipSuccess) {
    moe_destroy(c);
    return fail(MOE_ERR_OOM, "signalling area of %zu bytes", sb);
  }
  *out = c;
  return MOE_OK;
}

void moe_destroy(moe_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->dev);
  (void)hipStreamSynchronize(c->stream);
  for (auto &r : c->recs) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (auto e : c->pool) (void)hipEventDestroy(e);
  for (auto &l : c->layers) {
    l.experts.release();
    l.router.release();
    l.norm.release();
  }
  c->work.release();
  c->layer_sync.release();
  c->route_ticket.release();
  c->gemm_queue.release();
  c->layer_h.release();
  c->scratch_experts.release();
  c->stage.release();
  c->mv_split.release();
  c->lm_w.release();
  c->lm_x.release();
  c->lm_y.release();
  (void)hipStreamDestroy(c->stream);
  delete c;
}

int moe_set_adaptive_topk(moe_ctx *c, int enabled, size_t min_k, float top1_min_prob,
                          float top1_min_margin, float top2_min_mass) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  if (enabled && min_k < 1) return fail(MOE_ERR_INVALID, "min_k must be >= 1");
  c->ad_enabled = enabled ? 1 : 0;
  c->ad_min_k = min_k;
  c->ad_top1 = top1_min_prob;
  c->ad_margin = top1_min_margin;
  c->ad_top2 = top2_min_mass;
  return MOE_OK;
}

static int preload_common(moe_ctx *c, size_t layer, size_t n_experts) {
  RETURN_IF(use_dev(c));
  if (!n_experts || n_experts > (size_t)kMaxExperts)
    return fail(MOE_ERR_INVALID, "n_experts %zu outside [1, %d]", n_experts, kMaxExperts);
  if (layer > 4096) return fail(MOE_ERR_INVALID, "layer index %zu too large", layer);
  if (c->layers.size() <= layer) c->layers.resize(layer + 1);
  Layer &Ly = c->layers[layer];
  if (Ly.n_experts != n_experts) {  // a new expert count discards the layer's experts
    // the layer is empty until the new records exist (a failed allocation leaves it empty)
    Ly.n_experts = 0;
    Ly.loaded.clear();
    Ly.n_loaded = 0;
    if (Ly.experts.cap < n_experts * c->L.stride) Ly.experts.release();
    RETURN_IF(Ly.experts.ensure(n_experts * c->L.stride));
    Ly.n_experts = n_experts;
    Ly.loaded.assign(n_experts, 0);
    Ly.n_loaded = 0;
  }
  return MOE_OK;
}

static void mark_loaded(Layer &Ly, size_t e) {
  if (!Ly.loaded[e]) {
    Ly.loaded[e] = 1;
    Ly.n_loaded++;
  }
}

int moe_preload_expert(moe_ctx *c, size_t layer, size_t n_experts, size_t expert_idx,
                       const uint8_t *gub, size_t gub_len, const uint8_t *gus, size_t gus_len,
                       const float *gubias, size_t gubias_len, const uint8_t *db, size_t db_len,
                       const uint8_t *ds, size_t ds_len, const float *dbias, size_t dbias_len) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  if (expert_idx >= n_experts)
    return fail(MOE_ERR_INVALID, "expert %zu >= n_experts %zu", expert_idx, n_experts);
  RETURN_IF(preload_common(c, layer, n_experts));
  Layer &Ly = c->layers[layer];
  RETURN_IF(upload_expert(c, (uint8_t *)Ly.experts.p + expert_idx * c->L.stride, gub, gub_len,
                          gus, gus_len, gubias, gubias_len, db, db_len, ds, ds_len, dbias,
                          dbias_len));
  mark_loaded(Ly, expert_idx);
  return MOE_OK;
}

int moe_preload_layer(moe_ctx *c, size_t layer, size_t n_experts, const uint8_t *gub,
                      const uint8_t *gus, const float *gubias, const uint8_t *db,
                      const uint8_t *ds, const float *dbias) {
  if (!gub || !gus || !gubias || !db || !ds || !dbias) return fail(MOE_ERR_INVALID, "null tensor");
  RETURN_IF(preload_common(c, layer, n_experts));
  const ExpertBytes eb = expert_bytes(c);
  uint8_t *base = (uint8_t *)c->layers[layer].experts.p;
  for (size_t e = 0; e < n_experts; e++)
    RETURN_IF(upload_expert(c, base + e * c->L.stride, gub + e * eb.gub, eb.gub, gus + e * eb.gus,
                            eb.gus, gubias + e * eb.gubias, eb.gubias, db + e * eb.db, eb.db,
                            ds + e * eb.ds, eb.ds, dbias + e * eb.dbias, eb.dbias));
  for (size_t e = 0; e < n_experts; e++) mark_loaded(c->layers[layer], e);
  return MOE_OK;
}

int moe_preload_layer_device(moe_ctx *c, size_t layer, size_t n_experts, const uint8_t *gub,
                             const uint8_t *gus, const float *gubias, const uint8_t *db,
                             const uint8_t *ds, const float *dbias, void *stream) {
  if (!gub || !gus || !gubias || !db || !ds || !dbias) return fail(MOE_ERR_INVALID, "null tensor");
  RETURN_IF(preload_common(c, layer, n_experts));
  hipStream_t s = pick(c, stream);
  const ExpertBytes eb = expert_bytes(c);
  uint8_t *base = (uint8_t *)c->layers[layer].experts.p;
  for (size_t e = 0; e < n_experts; e++)
    RETURN_IF(pack_expert(c, base + e * c->L.stride, gub + e * eb.gub, gus + e * eb.gus,
                          gubias + e * eb.gubias, db + e * eb.db, ds + e * eb.ds,
                          dbias + e * eb.dbias, s));
  for (size_t e = 0; e < n_experts; e++) mark_loaded(c->layers[layer], e);
  return MOE_OK;
}

int moe_preload_router(moe_ctx *c, size_t layer, size_t n_experts, const uint16_t *w,
                       const float *bias) {
  RETURN_IF(use_dev(c));
  if (!w || !bias) return fail(MOE_ERR_INVALID, "null router tensor");
  if (!n_experts || n_experts > (size_t)kMaxExperts)
    return fail(MOE_ERR_INVALID, "n_experts %zu outside [1, %d]", n_experts, kMaxExperts);
  if (c->layers.size() <= layer) c->layers.resize(layer + 1);
  Layer &Ly = c->layers[layer];
  // load-major layout of the router (device.hpp, router_dot): [E][KIp/8][64 lanes][8]
  const size_t kip = router_kip(c->H);
  const size_t wb = router_bytes(c->H, n_experts), tot = al(wb) + n_experts * 4;
  RETURN_IF(Ly.router.ensure(tot));
  std::vector<uint16_t> lm(n_experts * 64 * kip, 0);
  for (size_t e = 0; e < n_experts; e++)
    for (size_t k = 0; k < c->H; k++) {
      const size_t i = k / 64;  // position in lane k % 64's chain
      lm[((e * (kip / 8) + i / 8) * 64 + k % 64) * 8 + i % 8] = w[e * c->H + k];
    }
  HIP_TRY(hipMemcpy(Ly.router.p, lm.data(), wb, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy((char *)Ly.router.p + al(wb), bias, n_experts * 4, hipMemcpyHostToDevice));
  Ly.router_experts = n_experts;
  return MOE_OK;
}

int moe_preload_router_f32(moe_ctx *c, size_t layer, size_t n_experts, const float *w,
                           const float *bias) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  if (!w || !bias) return fail(MOE_ERR_INVALID, "null router tensor");
  std::vector<uint16_t> b(n_experts * c->H);
  for (size_t i = 0; i < b.size(); i++) {
    uint32_t u;
    std::memcpy(&u, &w[i], 4);
    if (u & 0xFFFFu)
      return fail(MOE_ERR_INVALID, "router weight %zu (%g) is not exactly representable in bf16",
                  i, (double)w[i]);
    b[i] = (uint16_t)(u >> 16);
  }
  return moe_preload_router(c, layer, n_experts, b.data(), bias);
}

int moe_dispatch_expert_preloaded(moe_ctx *c, const float *input, size_t layer, size_t expert,
                                  float *output) {
  RETURN_IF(use_dev(c));
  if (!input || !output) return fail(MOE_ERR_INVALID, "null input or output");
  RETURN_IF(check_layer(c, layer, false, (long)expert));
  RETURN_IF(ensure_work(c, 1, 1, 1));
  HIP_TRY(hipMemcpyAsync(c->w.x, input, c->H * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(launch_split(c->w.x, 1, c->H, c->w.xsplit, c->stream));
  const int32_t id = (int32_t)expert;
  RETURN_IF(set_single_token_list(c, 1, &id));
  RETURN_IF(run_experts(c, c->w, (const uint8_t *)c->layers[layer].experts.p, 1, 1, c->stream));
  HIP_TRY(hipMemcpyAsync(output, c->w.o, c->H * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

int moe_dispatch_expert(moe_ctx *c, const float *input, const uint8_t *gub, size_t gub_len,
                        const uint8_t *gus, size_t gus_len, const float *gubias,
                        size_t gubias_len, const uint8_t *db, size_t db_len, const uint8_t *ds,
                        size_t ds_len, const float *dbias, size_t dbias_len, float *output) {
  RETURN_IF(use_dev(c));
  if (!input || !output) return fail(MOE_ERR_INVALID, "null input or output");
  RETURN_IF(c->scratch_experts.ensure(c->L.stride));
  RETURN_IF(upload_expert(c, (uint8_t *)c->scratch_experts.p, gub, gub_len, gus, gus_len, gubias,
                          gubias_len, db, db_len, ds, ds_len, dbias, dbias_len));
  RETURN_IF(ensure_work(c, 1, 1, 1));
  HIP_TRY(hipMemcpyAsync(c->w.x, input, c->H * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(launch_split(c->w.x, 1, c->H, c->w.xsplit, c->stream));
  RETURN_IF(set_single_token_list(c, 1, nullptr));
  RETURN_IF(run_experts(c, c->w, (const uint8_t *)c->scratch_experts.p, 1, 1, c->stream));
  HIP_TRY(hipMemcpyAsync(output, c->w.o, c->H * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

int moe_dispatch_experts_batched(moe_ctx *c, const float *input, size_t n,
                                 const moe_expert_ref *ex, float *output) {
  RETURN_IF(use_dev(c));
  if (!input || !output || (n && !ex)) return fail(MOE_ERR_INVALID, "null argument");
  if (n == 0) {
    std::memset(output, 0, c->H * 4);
    return MOE_OK;
  }
  if (n > (size_t)kMaxExperts) return fail(MOE_ERR_INVALID, "n %zu > %d", n, kMaxExperts);
  if (c->scratch_experts.cap < n * c->L.stride) c->scratch_experts.release();
  RETURN_IF(c->scratch_experts.ensure(n * c->L.stride));
  uint8_t *base = (uint8_t *)c->scratch_experts.p;
  for (size_t i = 0; i < n; i++) {
    const moe_expert_ref &r = ex[i];
    RETURN_IF(upload_expert(c, base + i * c->L.stride, r.gate_up_blocks, r.gate_up_blocks_len,
                            r.gate_up_scales, r.gate_up_scales_len, r.gate_up_bias,
                            r.gate_up_bias_len, r.down_blocks, r.down_blocks_len, r.down_scales,
                            r.down_scales_len, r.down_bias, r.down_bias_len));
  }
  RETURN_IF(ensure_work(c, 1, n, n));
  HIP_TRY(hipMemcpyAsync(c->w.x, input, c->H * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(launch_split(c->w.x, 1, c->H, c->w.xsplit, c->stream));
  RETURN_IF(set_single_token_list(c, n, nullptr));
  std::vector<float> wts(n);
  for (size_t i = 0; i < n; i++) wts[i] = ex[i].weight;
  HIP_TRY(hipMemcpyAsync(c->w.wts, wts.data(), n * 4, hipMemcpyHostToDevice, c->stream));
  RETURN_IF(run_experts(c, c->w, base, (int)n, 1, c->stream));
  HIP_TRY(launch_combine(c->w.o, c->w.pos, c->w.wts, 1, (int)n, (int)c->H, 1, c->w.y, c->stream));
  HIP_TRY(hipMemcpyAsync(output, c->w.y, c->H * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

static int init_lm_head_common(moe_ctx *c, const void *weights, size_t vocab, size_t elem,
                               hipMemcpyKind kind, hipStream_t s);

int moe_init_lm_head(moe_ctx *c, const float *weights, size_t vocab) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  return init_lm_head_common(c, weights, vocab, 4, hipMemcpyHostToDevice, c->stream);
}

// LM head weights [vocab, H] into lm_w: f32 or the checkpoint's bf16 rows; kind of the source
// pointer given by `kind`.
static int init_lm_head_common(moe_ctx *c, const void *weights, size_t vocab, size_t elem,
                               hipMemcpyKind kind, hipStream_t s) {
  RETURN_IF(use_dev(c));
  if (!weights || !vocab) return fail(MOE_ERR_INVALID, "null weights or zero vocab");
  if (vocab > ((size_t)1 << 40) / c->H) return fail(MOE_ERR_INVALID, "vocab_size %zu too large", vocab);
  c->lm_vocab = 0;  // not initialised until the new weights are resident
  if (c->lm_w.cap < vocab * c->H * elem) c->lm_w.release();
  RETURN_IF(c->lm_w.ensure(vocab * c->H * elem));
  RETURN_IF(c->lm_x.ensure(c->H * 4));
  RETURN_IF(c->lm_y.ensure(vocab * 4));
  HIP_TRY(hipMemcpyAsync(c->lm_w.p, weights, vocab * c->H * elem, kind, s));
  HIP_TRY(hipStreamSynchronize(s));
  c->lm_bf16 = elem == 2;
  c->lm_vocab = vocab;
  return MOE_OK;
}

int moe_init_lm_head_bf16(moe_ctx *c, const uint16_t *weights_bf16, size_t vocab) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  if (c->H % 8 || c->H > 3072) return fail(MOE_ERR_INVALID, "bf16 LM head needs hidden %% 8 == 0 and <= 3072");
  return init_lm_head_common(c, weights_bf16, vocab, 2, hipMemcpyHostToDevice, c->stream);
}

int moe_init_lm_head_bf16_device(moe_ctx *c, const uint16_t *weights_bf16, size_t vocab, void *stream) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  if (c->H % 8 || c->H > 3072) return fail(MOE_ERR_INVALID, "bf16 LM head needs hidden %% 8 == 0 and <= 3072");
  return init_lm_head_common(c, weights_bf16, vocab, 2, hipMemcpyDeviceToDevice, pick(c, stream));
}

static hipError_t lm_head_launch(moe_ctx *c, const float *x, size_t vocab, float *y, hipStream_t s) {
  if (c->lm_bf16)
    return launch_lm_head_bf16((const uint16_t *)c->lm_w.p, x, vocab, c->H, y, c->n_cu, s);
  return launch_lm_head((const float *)c->lm_w.p, x, vocab, c->H, y, s);
}

int moe_dispatch_lm_head(moe_ctx *c, const float *input, size_t vocab, float *logits) {
  RETURN_IF(use_dev(c));
  if (!c->lm_vocab) return fail(MOE_ERR_STATE, "call init_lm_head first");
  if (!input || !logits) return fail(MOE_ERR_INVALID, "null input or logits");
  if (vocab > c->lm_vocab)
    return fail(MOE_ERR_INVALID, "vocab_size %zu exceeds the initialised %zu", vocab, c->lm_vocab);
  HIP_TRY(hipMemcpyAsync(c->lm_x.p, input, c->H * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(lm_head_launch(c, (const float *)c->lm_x.p, vocab, (float *)c->lm_y.p, c->stream));
  HIP_TRY(hipMemcpyAsync(logits, c->lm_y.p, vocab * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

int moe_dispatch_lm_head_device(moe_ctx *c, const float *input, size_t vocab, float *logits, void *stream) {
  RETURN_IF(use_dev(c));
  if (!c->lm_vocab) return fail(MOE_ERR_STATE, "call init_lm_head first");
  if (!input || !logits) return fail(MOE_ERR_INVALID, "null input or logits");
  if (c->lm_bf16 && (reinterpret_cast<uintptr_t>(input) & 15))
    return fail(MOE_ERR_INVALID, "the bf16 LM head reads input with 16-byte loads: input must be 16-byte aligned");
  if (vocab > c->lm_vocab)
    return fail(MOE_ERR_INVALID, "vocab_size %zu exceeds the initialised %zu", vocab, c->lm_vocab);
  HIP_TRY(lm_head_launch(c, input, vocab, logits, pick(c, stream)));
  return MOE_OK;
}

int moe_router_topk(moe_ctx *c, size_t layer, const float *x, size_t T, size_t k, int32_t *idx,
                    float *weights, float *logits) {
  RETURN_IF(use_dev(c));
  if (!x || !idx || !weights) return fail(MOE_ERR_INVALID, "null argument");
  RETURN_IF(check_layer(c, layer, true));
  const size_t E = c->layers[layer].router_experts;
  if (T == 0) return MOE_OK;
  RETURN_IF(check_tokens(E, T, k));
  RETURN_IF(ensure_work(c, T, k, E));
  HIP_TRY(hipMemcpyAsync(c->w.x, x, T * c->H * 4, hipMemcpyHostToDevice, c->stream));
  RouteArgs ra{};
  Layer &Ly = c->layers[layer];
  ra.w = (const uint16_t *)Ly.router.p;
  ra.bias = (const float *)((const char *)Ly.router.p + al(router_bytes(c->H, E)));
  ra.x = c->w.x;
  ra.T = (int)T;
  ra.E = (int)E;
  ra.H = (int)c->H;
  ra.k = (int)k;
  ra.adaptive = c->ad_enabled;
  ra.min_k = (int)c->ad_min_k;
  ra.top1_min = c->ad_top1;
  ra.margin_min = c->ad_margin;
  ra.top2_mass = c->ad_top2;
  ra.logits = c->w.logits;
  ra.idx = c->w.idx;
  ra.wts = c->w.wts;
  ra.xsplit = nullptr;
  ra.fuse_bucket = 0;
  HIP_TRY(launch_route(ra, c->stream));
  HIP_TRY(hipMemcpyAsync(idx, c->w.idx, T * k * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipMemcpyAsync(weights, c->w.wts, T * k * 4, hipMemcpyDeviceToHost, c->stream));
  if (logits)
    HIP_TRY(hipMemcpyAsync(logits, c->w.logits, T * E * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return MOE_OK;
}

int moe_layer_forward(moe_ctx *c, size_t layer, const float *x, size_t T, size_t k, float *y) {
  RETURN_IF(use_dev(c));
  if (!x || !y) return fail(MOE_ERR_INVALID, "null x or y");
  if (T == 0) return MOE_OK;
  RETURN_IF(check_layer(c, layer, true));
  RETURN_IF(check_tokens(c->layers[layer].n_experts, T, k));
  RETURN_IF(ensure_work(c, T, k, c->layers[layer].n_experts));
  HIP_TRY(hipMemcpyAsync(c->w.x, x, T * c->H * 4, hipMemcpyHostToDevice, c->stream));
  RETURN_IF(forward_device(c, c->w, layer, c->w.x, T, k, c->w.y, c->stream));
  HIP_TRY(hipMemcpyAsync(y, c->w.y, T * c->H * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return check_layer_sync(c);
}

int moe_layer_forward_device(moe_ctx *c, size_t layer, const float *x, size_t T, size_t k,
                             float *y, void *stream) {
  RETURN_IF(use_dev(c));
  RETURN_IF(check_layer(c, layer, true));
  if (T == 0) return MOE_OK;
  RETURN_IF(check_tokens(c->layers[layer].n_experts, T, k));
  RETURN_IF(ensure_work(c, T, k, c->layers[layer].n_experts));
  return forward_device(c, c->w, layer, x, T, k, y, pick(c, stream));
}

int moe_layer_forward_device_noalloc(moe_ctx *c, size_t layer, const float *x, size_t T, size_t k,
                                     float *y, void *stream) {
  RETURN_IF(use_dev(c));
  if (c->timing)
    return fail(MOE_ERR_STATE, "the allocation-free forward runs with timing off (timing creates events)");
  RETURN_IF(check_layer(c, layer, true));
  if (T == 0) return MOE_OK;
  if (!x || !y) return fail(MOE_ERR_INVALID, "null x or y");
  RETURN_IF(check_tokens(c->layers[layer].n_experts, T, k));
  if (!c->scratch) return fail(MOE_ERR_STATE, "no scratch array address for device %d", c->dev);
  const size_t E = c->layers[layer].n_experts;
  Work w{};
  const size_t need = carve_work(w, nullptr, T, k, E, c->H, c->I, false);
  if (need > noalloc_scratch_bytes())
    return fail(MOE_ERR_INVALID,
                "%zu tokens at top-%zu over %zu experts need %zu bytes of workspace; the allocation-free "
                "forward's scratch holds %zu (use moe_layer_forward_device)",
                T, k, E, need, noalloc_scratch_bytes());
  carve_work(w, (char *)c->scratch, T, k, E, c->H, c->I, false);
  const hipStream_t s = pick(c, stream);
  // the array keeps the previous call's contents: the h records' padding must read as zeros
  HIP_TRY(launch_zero(w.hrec, w.hrec_bytes, s));
  return forward_device(c, w, layer, x, T, k, y, s);
}

int moe_block_forward(moe_ctx *c, size_t layer, const float *x, size_t T, size_t k, float *out) {
  RETURN_IF(use_dev(c));
  if (!x || !out) return fail(MOE_ERR_INVALID, "null x or out");
  if (T == 0) return MOE_OK;
  RETURN_IF(check_layer(c, layer, true));
  RETURN_IF(check_tokens(c->layers[layer].n_experts, T, k));
  RETURN_IF(ensure_work(c, T, k, c->layers[layer].n_experts));
  HIP_TRY(hipMemcpyAsync(c->w.x, x, T * c->H * 4, hipMemcpyHostToDevice, c->stream));
  RETURN_IF(forward_device(c, c->w, layer, c->w.x, T, k, c->w.y, c->stream, true));
  HIP_TRY(hipMemcpyAsync(out, c->w.y, T * c->H * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return check_layer_sync(c);
}

int moe_block_forward_device(moe_ctx *c, size_t layer, const float *x, size_t T, size_t k,
                             float *out, void *stream) {
  RETURN_IF(use_dev(c));
  if (x == out) return fail(MOE_ERR_INVALID, "out must not alias x");
  RETURN_IF(check_layer(c, layer, true));
  if (T == 0) return MOE_OK;
  RETURN_IF(check_tokens(c->layers[layer].n_experts, T, k));
  RETURN_IF(ensure_work(c, T, k, c->layers[layer].n_experts));
  return forward_device(c, c->w, layer, x, T, k, out, pick(c, stream), true);
}

int moe_preload_norm(moe_ctx *c, size_t layer, const float *gamma, float eps) {
  RETURN_IF(use_dev(c));
  if (!gamma) return fail(MOE_ERR_INVALID, "null gamma");
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(MOE_ERR_INVALID, "eps must be finite and >= 0");
  if (c->layers.size() <= layer) c->layers.resize(layer + 1);
  Layer &Ly = c->layers[layer];
  RETURN_IF(Ly.norm.ensure(c->H * 4));
  HIP_TRY(hipMemcpy(Ly.norm.p, gamma, c->H * 4, hipMemcpyHostToDevice));
  Ly.eps = eps;
  Ly.has_norm = true;
  return MOE_OK;
}

int moe_mxfp4_dequant_device(const uint8_t *blocks, const uint8_t *scales, size_t rows,
                             size_t cols, float *out, void *stream) {
  if (!blocks || !scales || !out) return fail(MOE_ERR_INVALID, "null argument");
  if (cols % 32) return fail(MOE_ERR_INVALID, "cols %zu not a multiple of 32", cols);
  HIP_TRY(launch_dequant_hf(blocks, scales, rows, cols, out, (hipStream_t)stream));
  return MOE_OK;
}

int moe_dequant_expert_device(moe_ctx *c, size_t layer, size_t expert, int which, float *out,
                              void *stream) {
  RETURN_IF(use_dev(c));
  RETURN_IF(check_layer(c, layer, false, (long)expert));
  if ((which != 0 && which != 1) || !out) return fail(MOE_ERR_INVALID, "bad which / out");
  const uint8_t *rec = (const uint8_t *)c->layers[layer].experts.p + expert * c->L.stride;
  if (which == 0)
    HIP_TRY(launch_dequant_packed(rec + c->L.gu_off, 2 * c->I, c->H, out, pick(c, stream)));
  else
    HIP_TRY(launch_dequant_packed(rec + c->L.dn_off, c->H, c->I, out, pick(c, stream)));
  return MOE_OK;
}

size_t moe_mxfp4_packed_size(size_t rows, size_t cols) {
  if (rows % 16 || cols % 32) return 0;
  return pack_total_bytes(pack_dims(rows, cols));
}

int moe_mxfp4_pack_device(const uint8_t *blocks, const uint8_t *scales, size_t rows, size_t cols,
                          uint8_t *packed, void *stream) {
  if (!blocks || !scales || !packed) return fail(MOE_ERR_INVALID, "null argument");
  if (!rows || !cols || rows % 16 || cols % 32)
    return fail(MOE_ERR_INVALID, "rows %zu must be a multiple of 16 and cols %zu of 32", rows, cols);
  HIP_TRY(launch_pack(blocks, scales, rows, cols, packed, (hipStream_t)stream));
  return MOE_OK;
}

int moe_mxfp4_matvec_device(moe_ctx *c, const uint8_t *packed, size_t rows, size_t cols,
                            const float *x, float *y, void *stream) {
  RETURN_IF(use_dev(c));
  if (!packed || !x || !y) return fail(MOE_ERR_INVALID, "null argument");
  if (!rows || !cols || rows % 16 || cols % 32)
    return fail(MOE_ERR_INVALID, "rows %zu must be a multiple of 16 and cols %zu of 32", rows, cols);
  hipStream_t s = pick(c, stream);
  if (c->matvec_one_launch && matvec_fp4_supported(rows, cols, x)) {
    HIP_TRY(launch_matvec_fp4(packed, rows, cols, x, y, s));
    return MOE_OK;
  }
  RETURN_IF(ensure_work(c, 1, 1, 1));
  const size_t cap0 = c->mv_split.cap;
  RETURN_IF(c->mv_split.ensure(256 + al(cols * 2 * 2)));
  if (c->mv_split.cap != cap0) c->mv_list_at = nullptr;  // a new allocation holds no list
  int32_t *lists = (int32_t *)c->mv_split.p;
  uint16_t *xs = (uint16_t *)((char *)c->mv_split.p + 256);
  if (c->mv_list_at != c->mv_split.p) {  // once per buffer: the one-entry expert list
    // n_active, active_ids[0], active_off[0..1], entry_src[0]
    static const int32_t list[5] = {1, 0, 0, 1, 0};
    HIP_TRY(hipMemcpyAsync(lists, list, sizeof(list), hipMemcpyHostToDevice, s));
    c->mv_list_at = c->mv_split.p;
  }
  HIP_TRY(launch_split(x, 1, cols, xs, s));
  GemvArgs a{};
  a.base = packed;
  a.stride = 0;
  a.mat_off = 0;
  a.bias_off = 0;
  a.d = pack_dims(rows, cols);
  a.n_active = lists;
  a.active_ids = lists + 1;
  a.active_off = lists + 2;
  a.entry_src = lists + 4;
  a.bsrc = xs;
  a.out = y;
  a.limit = c->clamp;
  a.max_active = 1;
  a.max_entries_per_expert = 1;
  HIP_TRY(launch_gemv(GEMV_RAW, a, s));
  return MOE_OK;
}

int moe_device_alloc(size_t bytes, void **ptr) {
  if (!ptr) return fail(MOE_ERR_INVALID, "null ptr");
  HIP_TRY(hipMalloc(ptr, bytes ? bytes : 1));
  return MOE_OK;
}
int moe_device_free(void *ptr) {
  HIP_TRY(hipFree(ptr));
  return MOE_OK;
}
int moe_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return MOE_OK;
}
int moe_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return MOE_OK;
}
int moe_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
  return MOE_OK;
}
int moe_memset_device(void *dst, int value, size_t bytes) {
  HIP_TRY(hipMemset(dst, value, bytes));
  return MOE_OK;
}
int moe_synchronize(moe_ctx *c) {
  RETURN_IF(use_dev(c));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return check_layer_sync(c);
}

int moe_set_option(moe_ctx *c, int option, int64_t value) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  switch (option) {
    case MOE_OPT_FUSED_DECODE:
      if (value < 0 || value > 2) return fail(MOE_ERR_INVALID, "MOE_OPT_FUSED_DECODE is 0, 1 or 2");
      c->decode_mode = (int)value;
      return MOE_OK;
    case MOE_OPT_BATCH_GEMM:
      if (value < 0 || value > 2) return fail(MOE_ERR_INVALID, "MOE_OPT_BATCH_GEMM is 0, 1 or 2");
      c->batch_gemm = (int)value;
      return MOE_OK;
    case MOE_OPT_GEMM_SHAPE:
      if (value < 0 || value > 19) return fail(MOE_ERR_INVALID, "MOE_OPT_GEMM_SHAPE is 0..19");
      c->gemm_shape = (int)value;
      return MOE_OK;
    case MOE_OPT_GEMM_BAND:
      if (value < 0 || value > 64) return fail(MOE_ERR_INVALID, "MOE_OPT_GEMM_BAND is 0..64");
      c->gemm_band = (int)value;
      return MOE_OK;
    case MOE_OPT_GEMM_SHAPE_DOWN:
      if (value < 0 || value > 19) return fail(MOE_ERR_INVALID, "MOE_OPT_GEMM_SHAPE_DOWN is 0..19");
      c->gemm_shape_down = (int)value;
      return MOE_OK;
    case MOE_OPT_MATVEC:
      if (value < 0 || value > 1) return fail(MOE_ERR_INVALID, "MOE_OPT_MATVEC is 0 or 1");
      c->matvec_one_launch = (int)value;
      return MOE_OK;
    case MOE_OPT_ACT_QUANT:
      if (value < 0 || value > 1) return fail(MOE_ERR_INVALID, "MOE_OPT_ACT_QUANT is 0 or 1");
      if ((int)value != c->act_quant && c->w.hrec) {
        // the two record layouts place h blocks differently, and the padding blocks past I, which
        // no kernel writes, must read as zeros in the new one
        if (c->capturing) return fail(MOE_ERR_STATE, "MOE_OPT_ACT_QUANT cannot change during graph capture");
        RETURN_IF(use_dev(c));
        // forwards may be in flight on caller streams (the _device calls): the whole device
        // drains before the records are cleared, so no old-layout write lands after the clear
        HIP_TRY(hipDeviceSynchronize());
        HIP_TRY(hipMemset(c->w.hrec, 0, c->w.hrec_bytes));
        HIP_TRY(hipDeviceSynchronize());
      }
      c->act_quant = (int)value;
      return MOE_OK;
    case MOE_OPT_LOCAL_GROUP:
      if (value < 0 || value > 1) return fail(MOE_ERR_INVALID, "MOE_OPT_LOCAL_GROUP is 0 or 1");
      c->local_group = (int)value;
      return MOE_OK;
    case MOE_OPT_SPIN_LIMIT:
      if (value < 1 || value > 0xFFFFFFFFll) return fail(MOE_ERR_INVALID, "spin limit outside [1, 2^32)");
      c->spin_limit = (uint32_t)value;
      return MOE_OK;
    default: return fail(MOE_ERR_INVALID, "unknown option %d", option);
  }
}
void *moe_stream(moe_ctx *c) { return c ? (void *)c->stream : nullptr; }

int moe_synth_fill_device(void *dst, size_t n, int kind, uint64_t seed, float a, float b,
                          void *stream) {
  if (!dst && n) return fail(MOE_ERR_INVALID, "null dst");
  hipError_t e = launch_synth(dst, n, kind, seed, a, b, (hipStream_t)stream);
  if (e != hipSuccess) return fail(MOE_ERR_INVALID, "synth fill: %s", hipGetErrorString(e));
  return MOE_OK;
}

int moe_graph_begin(moe_ctx *c) {
  RETURN_IF(use_dev(c));
  if (c->timing) return fail(MOE_ERR_STATE, "turn timing off before capturing a graph");
  if (c->capturing) return fail(MOE_ERR_STATE, "capture already in progress");
  HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  c->capturing = true;
  return MOE_OK;
}

int moe_graph_end(moe_ctx *c, void **graph_exec) {
  RETURN_IF(use_dev(c));
  if (!c->capturing) return fail(MOE_ERR_STATE, "no capture in progress");
  if (!graph_exec) return fail(MOE_ERR_INVALID, "null graph_exec");
  c->capturing = false;
  hipGraph_t g = nullptr;
  HIP_TRY(hipStreamEndCapture(c->stream, &g));
  hipGraphExec_t ge = nullptr;
  hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return fail(MOE_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  *graph_exec = (void *)ge;
  return MOE_OK;
}

int moe_graph_launch(moe_ctx *c, void *graph_exec) {
  RETURN_IF(use_dev(c));
  if (!graph_exec) return fail(MOE_ERR_INVALID, "null graph_exec");
  HIP_TRY(hipGraphLaunch((hipGraphExec_t)graph_exec, c->stream));
  return MOE_OK;
}

int moe_graph_destroy(void *graph_exec) {
  if (graph_exec) HIP_TRY(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
  return MOE_OK;
}

int moe_set_timing(moe_ctx *c, int enabled) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  c->timing = enabled != 0;
  return MOE_OK;
}

int moe_get_timing(moe_ctx *c, int kernel, double *ms, uint64_t *launches) {
  RETURN_IF(use_dev(c));
  if (kernel < 0 || kernel >= K_COUNT) return fail(MOE_ERR_INVALID, "kernel %d", kernel);
  RETURN_IF(collect_timing(c));
  if (ms) *ms = c->acc_ms[kernel];
  if (launches) *launches = c->acc_n[kernel];
  return MOE_OK;
}

int moe_reset_timing(moe_ctx *c) {
  RETURN_IF(use_dev(c));
  RETURN_IF(collect_timing(c));
  for (int i = 0; i < K_COUNT; i++) {
    c->acc_ms[i] = 0.0;
    c->acc_n[i] = 0;
  }
  return MOE_OK;
}

}  // extern "C"

// For the library's other host sources (safetensors.cpp): record the failure message that
// moe_last_error returns, and read a context's dimensions.
namespace moe {
int api_fail(int code, const char *msg) { return fail(code, "%s", msg); }
int ctx_dims(const moe_ctx *c, size_t *H, size_t *I) {
  if (!c) return fail(MOE_ERR_INVALID, "null context");
  *H = c->H;
  *I = c->I;
  return MOE_OK;
}
}  // namespace moe
