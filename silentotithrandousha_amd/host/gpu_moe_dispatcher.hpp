// C++ host mirror of the reference's GpuMoeDispatcher (src/gpu/moe_dispatch.rs:36-684) over
// the C ABI of libmxfp4moe.so (include/mxfp4_moe.h). Header-only; link -lmxfp4moe.
//
// Same method names, argument meaning and error behaviour as the Rust type:
//   * the constructor is the only fallible call and returns Result<GpuMoeDispatcher>
//     (Rust: Result<Self, String>, moe_dispatch.rs:60);
//   * dispatch calls are infallible in Rust and panic on misuse (dispatch_lm_head before
//     init_lm_head, moe_dispatch.rs:629-631); here they throw MoePanic with the library's
//     message;
//   * inputs are borrowed, outputs are returned by value (Rust: &[f32] in, Vec<f32> out);
//   * one dispatcher is not reentrant (the reference shares its Metal buffers between calls).
// The device buffers behind PreloadedExperts are owned by the dispatcher's context, so a
// PreloadedExperts value is only a handle (Rust owns them in the struct, moe_dispatch.rs:22-27).
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/mxfp4_moe.h"

namespace silentot {

// A panic of the Rust dispatcher (or a HIP failure it would have hit as one).
struct MoePanic : std::runtime_error {
  int status;
  MoePanic(int s, const std::string &m) : std::runtime_error(m), status(s) {}
};

inline void moe_check(int status) {
  if (status != MOE_OK) throw MoePanic(status, moe_last_error());
}

template <class T>
class Result {  // Rust's Result<T, String>
 public:
  static Result ok(T v) { return Result(std::move(v)); }
  static Result err(std::string e) { return Result(std::move(e), 0); }
  bool is_ok() const { return ok_; }
  const std::string &error() const { return err_; }
  T unwrap() && {
    if (!ok_) throw MoePanic(MOE_ERR_STATE, "called unwrap on an Err value: " + err_);
    return std::move(val_);
  }

 private:
  explicit Result(T v) : ok_(true), val_(std::move(v)) {}
  Result(std::string e, int) : ok_(false), err_(std::move(e)) {}
  bool ok_;
  T val_{};
  std::string err_;
};

// ExpertMxfp4 (weights.rs:17-27): one expert's checkpoint tensors.
struct ExpertMxfp4 {
  std::vector<uint8_t> gate_up_blocks;  // [2I, H/32, 16]
  std::vector<uint8_t> gate_up_scales;  // [2I, H/32]
  std::vector<float> gate_up_bias;      // [2I]
  std::vector<uint8_t> down_blocks;     // [H, I/32, 16]
  std::vector<uint8_t> down_scales;     // [H, I/32]
  std::vector<float> down_bias;         // [H]
};

// The MoE part of LayerWeights (weights.rs:29-47): router (bf16 values held as f32,
// weights.rs:280-281) and experts.
struct LayerWeights {
  std::vector<float> router_weight;  // [E, H]
  std::vector<float> router_bias;    // [E]
  std::vector<ExpertMxfp4> experts;
};

// The fields of GptOssConfig (config.rs:31-57) the MoE path reads.
struct GptOssConfig {
  size_t hidden_size = 2880;
  size_t intermediate_size = 2880;
  size_t num_local_experts = 32;
  size_t num_experts_per_tok = 4;
  float swiglu_limit = 7.0f;
};

struct PreloadedExperts {
  size_t n_layers = 0;
  size_t n_experts = 0;
};

// One tuple of dispatch_experts_batched (moe_dispatch.rs:476):
// (expert_idx, weight, gu_blocks, gu_scales, gu_bias, d_blocks, d_scales, d_bias).
struct ExpertSlice {
  size_t expert_idx;
  float weight;
  const ExpertMxfp4 *expert;
};

class GpuMoeDispatcher {
 public:
  // GpuMoeDispatcher::new — moe_dispatch.rs:60-146.
  static Result<GpuMoeDispatcher> create(size_t hidden_size, size_t inter_size,
                                         float swiglu_clamp) {
    moe_ctx *c = nullptr;
    if (moe_create(hidden_size, inter_size, swiglu_clamp, &c) != MOE_OK)
      return Result<GpuMoeDispatcher>::err(moe_last_error());
    return Result<GpuMoeDispatcher>::ok(GpuMoeDispatcher(c, hidden_size, inter_size));
  }

  GpuMoeDispatcher() = default;
  GpuMoeDispatcher(GpuMoeDispatcher &&o) noexcept { *this = std::move(o); }
  GpuMoeDispatcher &operator=(GpuMoeDispatcher &&o) noexcept {
    std::swap(ctx_, o.ctx_);
    hidden_size_ = o.hidden_size_;
    inter_size_ = o.inter_size_;
    return *this;
  }
  GpuMoeDispatcher(const GpuMoeDispatcher &) = delete;
  GpuMoeDispatcher &operator=(const GpuMoeDispatcher &) = delete;
  ~GpuMoeDispatcher() {
    if (ctx_) moe_destroy(ctx_);
  }

  size_t hidden_size() const { return hidden_size_; }
  size_t inter_size() const { return inter_size_; }
  moe_ctx *raw() const { return ctx_; }

  // preload_experts — moe_dispatch.rs:149-229: every expert of every layer into device
  // memory (here also the router, which the reference kept on the ANE).
  PreloadedExperts preload_experts(const std::vector<LayerWeights> &layers,
                                   const GptOssConfig &config) const {
    const size_t ne = config.num_local_experts;
    for (size_t l = 0; l < layers.size(); l++) {
      const LayerWeights &lw = layers[l];
      if (lw.experts.size() != ne)
        throw MoePanic(MOE_ERR_INVALID, "layer " + std::to_string(l) + " has " +
                                            std::to_string(lw.experts.size()) + " experts, config " +
                                            std::to_string(ne));
      for (size_t e = 0; e < ne; e++) {
        const ExpertMxfp4 &x = lw.experts[e];
        moe_check(moe_preload_expert(ctx_, l, ne, e, x.gate_up_blocks.data(),
                                     x.gate_up_blocks.size(), x.gate_up_scales.data(),
                                     x.gate_up_scales.size(), x.gate_up_bias.data(),
                                     x.gate_up_bias.size(), x.down_blocks.data(),
                                     x.down_blocks.size(), x.down_scales.data(),
                                     x.down_scales.size(), x.down_bias.data(),
                                     x.down_bias.size()));
      }
      if (!lw.router_weight.empty())
        moe_check(moe_preload_router_f32(ctx_, l, ne, lw.router_weight.data(),
                                         lw.router_bias.data()));
    }
    return PreloadedExperts{layers.size(), ne};
  }

  // dispatch_expert_preloaded — moe_dispatch.rs:232-324.
  std::vector<float> dispatch_expert_preloaded(const std::vector<float> &input,
                                               const PreloadedExperts &preloaded, size_t layer,
                                               size_t expert_idx) const {
    need(input.size() == hidden_size_, "input length");
    need(layer < preloaded.n_layers && expert_idx < preloaded.n_experts, "layer/expert index");
    std::vector<float> out(hidden_size_);
    moe_check(moe_dispatch_expert_preloaded(ctx_, input.data(), layer, expert_idx, out.data()));
    return out;
  }

  // dispatch_expert — moe_dispatch.rs:327-469.
  std::vector<float> dispatch_expert(const std::vector<float> &input,
                                     const std::vector<uint8_t> &gate_up_blocks,
                                     const std::vector<uint8_t> &gate_up_scales,
                                     const std::vector<float> &gate_up_bias,
                                     const std::vector<uint8_t> &down_blocks,
                                     const std::vector<uint8_t> &down_scales,
                                     const std::vector<float> &down_bias) const {
    need(input.size() == hidden_size_, "input length");
    std::vector<float> out(hidden_size_);
    moe_check(moe_dispatch_expert(ctx_, input.data(), gate_up_blocks.data(),
                                  gate_up_blocks.size(), gate_up_scales.data(),
                                  gate_up_scales.size(), gate_up_bias.data(), gate_up_bias.size(),
                                  down_blocks.data(), down_blocks.size(), down_scales.data(),
                                  down_scales.size(), down_bias.data(), down_bias.size(),
                                  out.data()));
    return out;
  }

  // dispatch_experts_batched — moe_dispatch.rs:473-607.
  std::vector<float> dispatch_experts_batched(const std::vector<float> &input,
                                              const std::vector<ExpertSlice> &experts) const {
    need(input.size() == hidden_size_, "input length");
    std::vector<moe_expert_ref> refs;
    refs.reserve(experts.size());
    for (const ExpertSlice &s : experts) {
      const ExpertMxfp4 &x = *s.expert;
      refs.push_back(moe_expert_ref{s.expert_idx, s.weight, x.gate_up_blocks.data(),
                                    x.gate_up_blocks.size(), x.gate_up_scales.data(),
                                    x.gate_up_scales.size(), x.gate_up_bias.data(),
                                    x.gate_up_bias.size(), x.down_blocks.data(),
                                    x.down_blocks.size(), x.down_scales.data(),
                                    x.down_scales.size(), x.down_bias.data(), x.down_bias.size()});
    }
    std::vector<float> out(hidden_size_);
    moe_check(moe_dispatch_experts_batched(ctx_, input.data(), refs.size(), refs.data(),
                                           out.data()));
    return out;
  }

  // init_lm_head — moe_dispatch.rs:611-621.
  void init_lm_head(const std::vector<float> &weights, size_t vocab_size) {
    need(weights.size() == vocab_size * hidden_size_, "LM head weight length");
    moe_check(moe_init_lm_head(ctx_, weights.data(), vocab_size));
  }

  // dispatch_lm_head — moe_dispatch.rs:624-683 (throws where Rust panics, :629-631).
  std::vector<float> dispatch_lm_head(const std::vector<float> &input, size_t vocab_size) const {
    need(input.size() == hidden_size_, "input length");
    std::vector<float> logits(vocab_size);
    moe_check(moe_dispatch_lm_head(ctx_, input.data(), vocab_size, logits.data()));
    return logits;
  }

  // The MoE block of Session::decode_step_inner (session.rs:818-980), batched over tokens.
  std::pair<std::vector<int32_t>, std::vector<float>> router_topk(size_t layer,
                                                                   const std::vector<float> &x,
                                                                   size_t top_k) const {
    need(x.size() % hidden_size_ == 0, "x length");
    const size_t T = x.size() / hidden_size_;
    std::vector<int32_t> idx(T * top_k);
    std::vector<float> w(T * top_k);
    moe_check(moe_router_topk(ctx_, layer, x.data(), T, top_k, idx.data(), w.data(), nullptr));
    return {std::move(idx), std::move(w)};
  }

  std::vector<float> layer_forward(size_t layer, const std::vector<float> &x, size_t top_k) const {
    need(x.size() % hidden_size_ == 0, "x length");
    std::vector<float> y(x.size());
    moe_check(moe_layer_forward(ctx_, layer, x.data(), x.size() / hidden_size_, top_k, y.data()));
    return y;
  }

 private:
  GpuMoeDispatcher(moe_ctx *c, size_t h, size_t i) : ctx_(c), hidden_size_(h), inter_size_(i) {}
  static void need(bool ok, const char *what) {
    if (!ok) throw MoePanic(MOE_ERR_INVALID, std::string("bad ") + what);
  }
  moe_ctx *ctx_ = nullptr;
  size_t hidden_size_ = 0, inter_size_ = 0;
};

}  // namespace silentot
