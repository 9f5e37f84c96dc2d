// Drives the C++ GpuMoeDispatcher mirror (silentotithrandousha_amd/host/gpu_moe_dispatcher.hpp)
// the way the reference's session would, and checks it against the CPU oracle (oracle/liborc.so,
// linked here as the checker only).
//   dispatcher_test cpu   host-only behaviour (no device calls): Result error of the constructor
//                         when no GPU is visible
//   dispatcher_test gpu   tiny GPT-OSS-shaped layer on the GPU vs the oracle
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>

#include "../../oracle/moe_oracle.h"
#include "../../silentotithrandousha_amd/host/gpu_moe_dispatcher.hpp"

using namespace silentot;

static int failures = 0;
#define EXPECT(c, ...)                                  \
  do {                                                  \
    if (!(c)) {                                         \
      std::printf("FAIL %s:%d: ", __FILE__, __LINE__);  \
      std::printf(__VA_ARGS__);                         \
      std::printf("\n");                                \
      failures++;                                       \
    }                                                   \
  } while (0)

static double rel_l2(const std::vector<float> &a, const std::vector<float> &b) {
  double num = 0, den = 0;
  for (size_t i = 0; i < a.size(); i++) {
    num += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
    den += (double)b[i] * b[i];
  }
  return std::sqrt(num / (den > 0 ? den : 1));
}

static float bf16_round(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  std::memcpy(&f, &u, 4);
  return f;
}

static int run_cpu() {
  auto r = GpuMoeDispatcher::create(2880, 2880, 7.0f);
  EXPECT(!r.is_ok(), "constructor succeeded without a device");
  EXPECT(!r.error().empty(), "empty error string");
  bool threw = false;
  try {
    (void)std::move(r).unwrap();
  } catch (const MoePanic &) {
    threw = true;
  }
  EXPECT(threw, "unwrap of Err did not panic");
  auto bad = GpuMoeDispatcher::create(2880, 2881, 7.0f);
  EXPECT(!bad.is_ok(), "hidden/inter not multiple of 32 accepted");
  std::printf("cpu: %s (constructor error: %s)\n", failures ? "FAILED" : "ok", r.error().c_str());
  return failures ? 1 : 0;
}

static int run_gpu() {
  const size_t H = 128, I = 64, E = 8, K = 4, T = 3, L = 2;
  GptOssConfig cfg;
  cfg.hidden_size = H;
  cfg.intermediate_size = I;
  cfg.num_local_experts = E;
  cfg.num_experts_per_tok = K;
  std::mt19937_64 rng(7);
  std::uniform_int_distribution<int> byte(0, 255), scale(118, 125);
  std::normal_distribution<float> nrm(0.0f, 1.0f);
  std::vector<LayerWeights> layers(L);
  for (auto &lw : layers) {
    lw.router_weight.resize(E * H);
    lw.router_bias.resize(E);
    for (auto &v : lw.router_weight) v = bf16_round(0.2f * nrm(rng));
    for (auto &v : lw.router_bias) v = 0.1f * nrm(rng);
    lw.experts.resize(E);
    for (auto &x : lw.experts) {
      x.gate_up_blocks.resize(2 * I * (H / 32) * 16);
      x.gate_up_scales.resize(2 * I * (H / 32));
      x.gate_up_bias.resize(2 * I);
      x.down_blocks.resize(H * (I / 32) * 16);
      x.down_scales.resize(H * (I / 32));
      x.down_bias.resize(H);
      for (auto &v : x.gate_up_blocks) v = (uint8_t)byte(rng);
      for (auto &v : x.gate_up_scales) v = (uint8_t)scale(rng);
      for (auto &v : x.gate_up_bias) v = 0.1f * nrm(rng);
      for (auto &v : x.down_blocks) v = (uint8_t)byte(rng);
      for (auto &v : x.down_scales) v = (uint8_t)scale(rng);
      for (auto &v : x.down_bias) v = 0.1f * nrm(rng);
    }
  }
  auto r = GpuMoeDispatcher::create(H, I, cfg.swiglu_limit);
  if (!r.is_ok()) {
    std::printf("FAIL: constructor: %s\n", r.error().c_str());
    return 1;
  }
  GpuMoeDispatcher d = std::move(r).unwrap();
  const PreloadedExperts pre = d.preload_experts(layers, cfg);
  EXPECT(pre.n_layers == L && pre.n_experts == E, "preloaded handle");

  std::vector<float> x(T * H);
  for (auto &v : x) v = nrm(rng);
  const std::vector<float> x0(x.begin(), x.begin() + H);

  for (size_t l = 0; l < L; l++) {
    const LayerWeights &lw = layers[l];
    // per-expert: dispatch_expert_preloaded and dispatch_expert vs the fp32 oracle expert
    for (size_t e = 0; e < E; e += 3) {
      const ExpertMxfp4 &xe = lw.experts[e];
      std::vector<float> ref(H);
      orc_expert_ffn_f32(x0.data(), 1, xe.gate_up_blocks.data(), xe.gate_up_scales.data(),
                         xe.gate_up_bias.data(), xe.down_blocks.data(), xe.down_scales.data(),
                         xe.down_bias.data(), H, I, cfg.swiglu_limit, ref.data(), nullptr);
      const auto a = d.dispatch_expert_preloaded(x0, pre, l, e);
      const auto b = d.dispatch_expert(x0, xe.gate_up_blocks, xe.gate_up_scales, xe.gate_up_bias,
                                       xe.down_blocks, xe.down_scales, xe.down_bias);
      EXPECT(rel_l2(a, ref) < 1e-3, "layer %zu expert %zu preloaded rel-L2 %g", l, e, rel_l2(a, ref));
      EXPECT(rel_l2(b, ref) < 1e-3, "layer %zu expert %zu raw rel-L2 %g", l, e, rel_l2(b, ref));
    }
    // the whole block vs the oracle layer (top-k exact, outputs within 1e-3)
    std::vector<uint16_t> rw(E * H);
    for (size_t i = 0; i < rw.size(); i++) {
      uint32_t u;
      std::memcpy(&u, &lw.router_weight[i], 4);
      rw[i] = (uint16_t)(u >> 16);
    }
    std::vector<uint8_t> gub, gus, db, ds;
    std::vector<float> gubias, dbias;
    for (const auto &xe : lw.experts) {
      gub.insert(gub.end(), xe.gate_up_blocks.begin(), xe.gate_up_blocks.end());
      gus.insert(gus.end(), xe.gate_up_scales.begin(), xe.gate_up_scales.end());
      gubias.insert(gubias.end(), xe.gate_up_bias.begin(), xe.gate_up_bias.end());
      db.insert(db.end(), xe.down_blocks.begin(), xe.down_blocks.end());
      ds.insert(ds.end(), xe.down_scales.begin(), xe.down_scales.end());
      dbias.insert(dbias.end(), xe.down_bias.begin(), xe.down_bias.end());
    }
    std::vector<float> yref(T * H), wref(T * K);
    std::vector<int32_t> iref(T * K);
    orc_moe_layer_f32(x.data(), T, H, I, E, K, cfg.swiglu_limit, rw.data(), lw.router_bias.data(),
                      gub.data(), gus.data(), gubias.data(), db.data(), ds.data(), dbias.data(),
                      nullptr, yref.data(), nullptr, iref.data(), wref.data());
    const auto tk = d.router_topk(l, x, K);
    EXPECT(tk.first == iref, "layer %zu top-k indices differ", l);
    for (size_t i = 0; i < T * K; i++)
      EXPECT(std::fabs(tk.second[i] - wref[i]) <= 1e-6f, "layer %zu weight %zu", l, i);
    const auto y = d.layer_forward(l, x, K);
    EXPECT(rel_l2(y, yref) < 1e-3, "layer %zu forward rel-L2 %g", l, rel_l2(y, yref));
    const auto y1g = d.layer_forward(l, x0, K);
    EXPECT(rel_l2(y1g, std::vector<float>(yref.begin(), yref.begin() + H)) < 1e-3,
           "layer %zu single-token forward", l);
    // dispatch_experts_batched with the routed experts of token 0 vs the oracle combine
    std::vector<ExpertSlice> sl;
    for (size_t s = 0; s < K; s++) sl.push_back(ExpertSlice{(size_t)iref[s], wref[s], &lw.experts[iref[s]]});
    const auto yb = d.dispatch_experts_batched(x0, sl);
    EXPECT(rel_l2(yb, std::vector<float>(yref.begin(), yref.begin() + H)) < 1e-3,
           "layer %zu batched rel-L2 %g", l, rel_l2(yb, std::vector<float>(yref.begin(), yref.begin() + H)));
  }
  // LM head: panics before init (moe_dispatch.rs:629-631), then a plain f32 GEMV
  bool threw = false;
  try {
    (void)d.dispatch_lm_head(x0, 16);
  } catch (const MoePanic &p) {
    threw = p.status == MOE_ERR_STATE;
  }
  EXPECT(threw, "dispatch_lm_head before init_lm_head did not panic");
  const size_t V = 40;
  std::vector<float> lm(V * H);
  for (auto &v : lm) v = nrm(rng);
  d.init_lm_head(lm, V);
  const auto logits = d.dispatch_lm_head(x0, V);
  std::vector<float> lref(V);
  for (size_t v = 0; v < V; v++) {
    double s = 0;
    for (size_t k = 0; k < H; k++) s += (double)lm[v * H + k] * x0[k];
    lref[v] = (float)s;
  }
  EXPECT(rel_l2(logits, lref) < 1e-5, "lm head rel-L2 %g", rel_l2(logits, lref));
  std::printf("gpu: %s\n", failures ? "FAILED" : "ok");
  return failures ? 1 : 0;
}

int main(int argc, char **argv) {
  if (argc > 1 && std::strcmp(argv[1], "gpu") == 0) return run_gpu();
  return run_cpu();
}
