// Kernel launch interface (host side). Every launcher checks its own shape assumptions
// before enqueuing and returns the HIP error of the launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>

#include "layout.hpp"

namespace moe {

// Raises a kernel's dynamic-LDS limit on the current device once per device. One DynLdsOnce per
// kernel (a function-local static at the launch site); thread-safe; a failed call is returned
// and retried by the next launch.
struct DynLdsOnce {
  static constexpr int kDevices = 64;
  std::mutex mu;
  bool done[kDevices] = {};
};
inline hipError_t ensure_dyn_lds(DynLdsOnce &once, const void *kernel, size_t bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= DynLdsOnce::kDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(once.mu);
  if (once.done[dev]) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) once.done[dev] = true;
  return e;
}

constexpr int kMaxExperts = 256;  // router / bucketing LDS tables
constexpr int kMaxTopK = 16;

enum GemvMode { GEMV_GATE_UP = 0, GEMV_DOWN = 1, GEMV_RAW = 2 };

struct RouteArgs {
  const uint16_t *w;     // load-major router: [E][KIp/8][64 lanes][8] bf16 bits (router_dot)
  const float *bias;     // [E]
  const float *x;        // [T, H]
  int T, E, H, k;
  int adaptive, min_k;
  float top1_min, margin_min, top2_mass;
  float *logits;         // [T, E]
  int32_t *idx;          // [T, k]
  float *wts;            // [T, k]
  uint16_t *xsplit;      // [T, 2, H] bf16 hi / lo
  uint8_t *xrec;         // [T] GemmRecT<rec_terms> records of x (grouped GEMM operands; H <= 128 kGemmNs)
  int rec_terms;         // kGemmTerms (exact split) or 1 (one MXFP6 term per value)
  int fuse_bucket;       // T == 1: also write the expert list
  int32_t *n_active, *active_ids, *active_off, *entry_src, *pos;
  uint32_t *bucket_ticket;  // T > 1: zeroed counter; the last block buckets (route_bucket_fits)
  int32_t *blk_count;       // with bucket_ticket: [route blocks][E] per-block expert counts
  int32_t *rank;            // with bucket_ticket: [T, k] rank of each entry in its block and expert
};

struct GemvArgs {
  const uint8_t *base;     // first expert record of the region
  size_t stride;           // bytes between expert records
  size_t mat_off;          // packed matrix offset inside a record
  size_t bias_off;         // f32 bias offset inside a record (ignored for GEMV_RAW)
  PackDims d;              // matrix dimensions
  const int32_t *n_active; // device scalar: active experts this call
  const int32_t *active_ids, *active_off;
  const int32_t *entry_src;  // B row of each entry (NULL: the entry itself)
  const uint16_t *bsrc;      // [rows_b, 2, K] bf16 hi/lo operands, K = d.nb * 32
  void *out;                 // GATE_UP: u16 [entry, 2, rows/2]; DOWN/RAW: f32 [entry, rows]
  float limit;
  int max_active;            // grid covers max_active * d.tiles wavefronts
  int max_entries_per_expert;
};

// fp8 terms per activation value for the block-scaled MFMA paths (device.hpp, split8_fp8).
constexpr int kTerms = 4;

// Step-major activation record of one row (token or entry) for the grouped GEMM (gemm.hip):
// NT fp6 (E2M3) terms per value, rows of up to 4 * kGemmNs 32-value blocks. The B operand of
// block 4s + b (b = 0..3, the MFMA lane group b: K = 32 b + u, value u at bits 6u) is 6 dwords;
// K-step s holds, per term t, 96 bytes: dwords 0-3 of blocks 0..3 (16 bytes each, block b at 16 b),
// then dwords 4-5 of blocks 0..3 (8 bytes each, at 64 + 8 b); then [term t][4 scale bytes, byte
// i = E8M0 of block 4s+i] (4 NT bytes) and pad bytes to 16. A step is kChunks 16-byte chunks:
// chunk 6t + b = the first 16 bytes of block b, chunk 6t + 4 + (b >> 1) = the last 8 bytes of
// blocks b and b ^ 1, chunk 6 NT = the scales (the grouped GEMM stages them chunk by chunk).
// Blocks past the row are zero. NT = kGemmTerms: the exact split (the default); NT = 1: the
// quantized-activation mode (one MXFP6 term per value).
constexpr int kGemmNs = 24;
constexpr int kGemmTerms = 3;
template <int NT>
struct GemmRecT {
  static constexpr int kNT = NT;
  static constexpr int kTermBytes = 96;
  static constexpr int kStep = NT * kTermBytes + 16;
  static constexpr int kChunks = kStep / 16;
  static constexpr int kBytes = kGemmNs * kStep;
  // byte offset of dword d (0..5) of the B operand of block b (0..3) of step s, term t
  MOE_HD static constexpr int dword(int s, int t, int b, int d) {
    return s * kStep + t * kTermBytes + (d < 4 ? 16 * b + 4 * d : 64 + 8 * b + 4 * (d - 4));
  }
  MOE_HD static constexpr int scale(int s, int t) { return s * kStep + NT * kTermBytes + 4 * t; }
  static_assert(NT >= 1 && NT <= 3 && kStep % 16 == 0 && kChunks == 6 * NT + 1, "record chunks");
};
using GemmRec = GemmRecT<kGemmTerms>;

struct GemmArgs {
  const uint8_t *base;       // expert records of the layer
  size_t stride, mat_off, bias_off;
  PackDims d;                // weight matrix (rows x K)
  const int32_t *n_active, *active_ids, *active_off;  // entries grouped by expert (k_bucket)
  const int32_t *entry_src;  // B record of each entry (NULL: the entry's own)
  const uint8_t *brec;       // B records (GemmRec)
  void *out;                 // GATE_UP: h records (GemmRec) per entry; DOWN: f32 [entry][rows]
  float limit;
  int max_active;            // upper bound of *n_active
  size_t n_entries;          // entries over all experts (sets the column tiles)
  int shape;                 // block shape override for tuning (0: by the mean entries per expert)
  int band;                  // row blocks per band of the XCD-local tile order (0: workgroup order)
  int n_row_blocks;          // set by launch_gemm_fp8: row blocks of the launch
  int n_tiles;               //                         row blocks x column tiles
  int n_blocks;              //                         workgroups of the tile order (>= n_tiles)
  int terms;                 // E2M3 terms per activation value: kGemmTerms, or 1 (quantized mode)
  int32_t *queue;            // tile queue of the persistent pipelined step: 10 counters, zero between launches
  // Local grouping (the streamed gate_up GEMM of a batch of at most kLocalGroupMax entries): with
  // group_idx set (the top-k indices [T][group_k] over group_E experts, -1 for a dropped slot)
  // every workgroup groups the entries by expert itself, in place of the router's grouping, and
  // workgroup 0 writes the expert lists, entry_src and pos (the w_ pointers) for the down GEMM
  // and the combine.
  const int32_t *group_idx;
  int group_k, group_E;
  int32_t *w_n_active, *w_active_ids, *w_active_off, *w_entry_src, *w_pos;
};
constexpr int kLocalGroupMax = 1024;
// Whether the gate_up launch of these arguments (group_idx unset) runs the streamed kernel with
// local grouping when asked to (gemm.hip: the same shape choice as launch_gemm_fp8).
bool gemm_gate_up_groups_locally(const GemmArgs &a);
hipError_t launch_gemm_fp8(GemvMode mode, const GemmArgs &a, hipStream_t s);
// The streamed form for batches of a few entries per expert (gemm_stream.hip); hipErrorNotSupported
// when the launch does not fit it.
hipError_t launch_gemm_stream(GemvMode mode, const GemmArgs &a, hipStream_t s, bool alt);
// The wide streamed form for batches of tens of entries per expert (gemm_wide.hip): every weight
// tile streams once per group of up to 5 16-entry chunks; hipErrorNotSupported when the launch
// does not fit it.
hipError_t launch_gemm_wide(GemvMode mode, const GemmArgs &a, hipStream_t s);

// Single-token MoE layer in two launches (decode.hip).
struct DecodeArgs {
  const uint16_t *rw;  // load-major router (see router_dot)
  const float *rb;     // [E]
  int rnq, Hr;         // 16-byte loads per router lane chain; router x length (64 * 8 * rnq)
  const uint8_t *base; // expert records of the layer
  size_t stride, gu_off, dn_off, gub_off, dnb_off;
  PackDims gu, dn;
  int H, I, E, k;
  float limit;
  int adaptive, min_k;
  float top1_min, margin_min, top2_mass;
  const float *x;      // [H]
  float *y;            // [H]
  float *logits;       // [E]   written by gate_up block 0
  int32_t *idx;        // [k]   written by gate_up block 0, read by down
  float *wts;          // [k]
  uint16_t *hsplit;    // [k, 2, I]
  int n_gu_wg_per_slot;
};

// One-launch single-token layer (decode_layer.hip): DecodeArgs plus the cross-block
// signalling area (zeroed once at context creation and after a reported error; its logit copies
// return to zero after every launch, its launch numbers and h flags only advance) and the
// h records of the four slots (zeroed once; the values past I stay zero).
constexpr int kLayerMaxBlocks = 1024;
struct LayerArgs {
  DecodeArgs d;
  void *sync;            // layer_sync_bytes() bytes
  uint8_t *hterm;        // layer_hterm_bytes() bytes: per slot the fp8 term rows of h
  uint32_t spin_limit;   // polls before a wait gives up
  int hexp;              // filled by layer_geometry: exponent of the first h term
  const float *gamma;    // non-null: the block forward (RMSNorm of d.x before, d.x + y after)
  float eps;
  int n_tps;             // filled by layer_geometry: gate_up tiles per slot
  int n_gu;              //                           gate_up blocks
  int n_dn;              //                           down blocks = down tiles
  int n_rt;              //                           router blocks, ceil(E / 4)
  int n_cu;              //                           compute units of the device
};
size_t layer_sync_bytes();
size_t layer_hterm_bytes();
int layer_hexp(float limit);
void layer_geometry(LayerArgs &la, int n_cu);
bool decode_layer_supported(const LayerArgs &la);
hipError_t launch_decode_layer(const LayerArgs &a, hipStream_t s);

bool decode_supported(const DecodeArgs &a);
hipError_t launch_decode_gate_up(const DecodeArgs &a, hipStream_t s);
hipError_t launch_decode_down(const DecodeArgs &a, hipStream_t s);

hipError_t launch_route(const RouteArgs &a, hipStream_t s);
// Whether k_route's x staging (one token) holds bucket_block's LDS for E experts.
bool route_bucket_fits(int H, int E);
hipError_t launch_bucket(const int32_t *idx, int T, int k, int E, int32_t *n_active,
                         int32_t *active_ids, int32_t *active_off, int32_t *entry_src,
                         int32_t *pos, hipStream_t s);
hipError_t launch_gemv(GemvMode mode, const GemvArgs &a, hipStream_t s);
hipError_t launch_combine(const float *o, const int32_t *pos, const float *w, int T, int k, int H,
                          int skip_nonfinite, float *y, hipStream_t s);
hipError_t launch_split(const float *x, size_t n_rows, size_t K, uint16_t *xsplit, hipStream_t s);
hipError_t launch_dequant_hf(const uint8_t *blocks, const uint8_t *scales, size_t rows,
                             size_t cols, float *out, hipStream_t s);
hipError_t launch_dequant_packed(const uint8_t *packed, size_t rows, size_t cols, float *out,
                                 hipStream_t s);
hipError_t launch_pack(const uint8_t *blocks, const uint8_t *scales, size_t rows, size_t cols,
                       uint8_t *packed, hipStream_t s);
hipError_t launch_synth(void *dst, size_t n, int kind, uint64_t seed, float a, float b,
                        hipStream_t s);
// One MXFP4 matvec in one launch on the block-scaled MFMA (matvec.hip): rows % 16 == 0,
// cols % 32 == 0, cols <= 3072, x 16-byte aligned.
bool matvec_fp4_supported(size_t rows, size_t cols, const float *x);
hipError_t launch_matvec_fp4(const uint8_t *packed, size_t rows, size_t cols, const float *x,
                             float *y, hipStream_t s);
hipError_t launch_lm_head(const float *w, const float *x, size_t vocab, size_t H, float *y,
                          hipStream_t s);
hipError_t launch_lm_head_bf16(const uint16_t *w, const float *x, size_t vocab, size_t H, float *y, int n_cu,
                               hipStream_t s);
// Post-attention RMSNorm of T rows (rms_inv_wave's order) and the residual add y += x.
hipError_t launch_rmsnorm(const float *x, size_t T, size_t H, const float *gamma, float eps, float *n,
                          hipStream_t s);
hipError_t launch_add_rows(float *y, const float *x, size_t n, hipStream_t s);

// Allocation-free forward (noalloc.hip): bytes of each device's scratch array, its device address
// (resolved once per device, with that device current), and a kernel that zeroes device memory.
size_t noalloc_scratch_bytes();
hipError_t noalloc_scratch_ptr(int dev, void **ptr);
hipError_t launch_zero(void *p, size_t bytes, hipStream_t s);

}  // namespace moe
