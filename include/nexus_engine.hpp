// nexus_engine.hpp — C++ host API over libnexus_hip.so that mirrors the
// reference's MoE helper and backend interface (header-only).
//
// Mirrors (paths relative to the Nexus repository):
//   MoeRoute, MoeExpertWeights, MoeDispatchConfig   src/engine/mod.rs:133-153
//   InferenceEngine::route_moe_experts              src/engine/mod.rs:918-966
//   InferenceEngine::dispatch_moe_ffn               src/engine/mod.rs:969-1024
//   Backend trait (name, backend_type, is_available, memory_info,
//   capabilities, synchronize)                      src/backend/mod.rs:74-96
//   BackendCapabilities / MemoryInfo                src/backend/mod.rs:25-31, 98-113
// Same names, argument meaning and error strings; Result<T> stands in for
// Rust's Result<T, String>.  All arithmetic runs on the GPU through the C ABI.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "nexus_hip.h"

namespace nexus {

template <typename T>
class Result {
 public:
  static Result ok(T v) { return Result(std::move(v), std::string(), true); }
  static Result err(std::string e) { return Result(T(), std::move(e), false); }
  bool is_ok() const { return ok_; }
  bool is_err() const { return !ok_; }
  const T &unwrap() const {
    if (!ok_) throw std::runtime_error("called unwrap on an Err: " + err_);
    return val_;
  }
  const std::string &unwrap_err() const {
    if (ok_) throw std::runtime_error("called unwrap_err on an Ok value");
    return err_;
  }

 private:
  Result(T v, std::string e, bool ok) : val_(std::move(v)), err_(std::move(e)), ok_(ok) {}
  T val_;
  std::string err_;
  bool ok_;
};

namespace detail {
inline std::string last_error() { return std::string(nx_last_error()); }
}  // namespace detail

// ---------------------------------------------------------------- backend
namespace backend {

enum class BackendType { CpuSimd, Metal, Hip, Vulkan, WebGpu };

inline const char *backend_name(BackendType t) {
  switch (t) {
  case BackendType::CpuSimd: return "cpu-simd";
  case BackendType::Metal: return "metal";
  case BackendType::Hip: return "hip";
  case BackendType::Vulkan: return "vulkan";
  case BackendType::WebGpu: return "webgpu";
  }
  return "?";
}

struct MemoryInfo {
  size_t total_memory = 0, free_memory = 0, used_memory = 0;
  float utilization() const {
    return total_memory == 0 ? 0.0f : (float)used_memory / (float)total_memory;
  }
};

struct BackendCapabilities {
  BackendType backend;
  bool available;
  std::vector<const char *> features;
  std::vector<const char *> supported_ops;
};

// The HIP backend that takes the place of the reference's CUDA placeholder
// (src/backend/mod.rs:206-212, 221-230).  One context (stream) per backend.
class HipBackend {
 public:
  explicit HipBackend(int device = 0) {
    int n = 0;
    nx_device_count(&n);
    if (n > device && nx_ctx_create(device, &ctx_) == NX_OK) available_ = true;
  }
  ~HipBackend() {
    if (ctx_) nx_ctx_destroy(ctx_);
  }
  HipBackend(const HipBackend &) = delete;
  HipBackend &operator=(const HipBackend &) = delete;

  const char *name() const { return "hip"; }
  BackendType backend_type() const { return BackendType::Hip; }
  bool is_available() const { return available_; }
  MemoryInfo memory_info() const {
    MemoryInfo m;
    if (ctx_) {
      size_t f = 0, t = 0;
      if (nx_mem_info(ctx_, &f, &t) == NX_OK) {
        m.total_memory = t;
        m.free_memory = f;
        m.used_memory = t - f;
      }
    }
    return m;
  }
  BackendCapabilities capabilities() const {
    BackendCapabilities c{BackendType::Hip, available_, {}, {}};
    if (available_) {
      c.features = {"gfx950", "mfma-f16", "mfma-bf16", "q4_k", "q8_0", "q4_0"};
      c.supported_ops = {"moe_route_topk", "moe_permute", "moe_ffn", "dequantize", "quantize"};
    }
    return c;
  }
  void synchronize() const {
    if (ctx_) nx_sync(ctx_);
  }
  nx_ctx *ctx() const { return ctx_; }

 private:
  nx_ctx *ctx_ = nullptr;
  bool available_ = false;
};

}  // namespace backend

// ---------------------------------------------------------------- engine
namespace engine {

struct MoeRoute {
  size_t expert;
  float weight;
  bool operator==(const MoeRoute &o) const { return expert == o.expert && weight == o.weight; }
};

struct MoeExpertWeights {
  const std::vector<std::vector<float>> &gate;
  const std::vector<std::vector<float>> &up;
  const std::vector<std::vector<float>> &down;
};

struct MoeDispatchConfig {
  size_t top_k;
  size_t hidden_size;
  size_t ff_dim;
};

// Quantized, device-resident experts for the batched sibling of
// dispatch_moe_ffn (weights stay in HBM across calls).
class DeviceExperts {
 public:
  DeviceExperts(backend::HipBackend &be, int fmt, size_t num_experts, size_t hidden,
                size_t ff_dim)
      : be_(be), hidden_(hidden), experts_(num_experts) {
    if (nx_experts_create(be.ctx(), fmt, (int)num_experts, (int)hidden, (int)ff_dim, &ex_) != NX_OK)
      throw std::runtime_error(detail::last_error());
  }
  ~DeviceExperts() {
    if (ex_) nx_experts_destroy(ex_);
  }
  DeviceExperts(const DeviceExperts &) = delete;
  DeviceExperts &operator=(const DeviceExperts &) = delete;
  // role: NX_ROLE_GATE / NX_ROLE_UP / NX_ROLE_DOWN; payload in GGUF block format
  Result<bool> load(size_t expert, int role, const void *payload, size_t bytes) {
    if (nx_experts_load(be_.ctx(), ex_, (int)expert, role, payload, bytes, 0) != NX_OK)
      return Result<bool>::err(detail::last_error());
    return Result<bool>::ok(true);
  }
  nx_experts *handle() const { return ex_; }
  size_t hidden() const { return hidden_; }
  size_t num_experts() const { return experts_; }
  backend::HipBackend &backend() const { return be_; }

 private:
  backend::HipBackend &be_;
  nx_experts *ex_ = nullptr;
  size_t hidden_, experts_;
};

class InferenceEngine {
 public:
  // Process-wide default backend for the stateless associated functions.
  static backend::HipBackend &default_backend() {
    static backend::HipBackend be(0);
    return be;
  }

  /// Select top-k experts per token from router logits (src/engine/mod.rs:918-966).
  static std::vector<std::vector<MoeRoute>> route_moe_experts(const std::vector<float> &router_logits,
                                                              size_t num_tokens, size_t num_experts,
                                                              size_t top_k) {
    std::vector<std::vector<MoeRoute>> routes;
    if (num_tokens == 0 || num_experts == 0 || top_k == 0) return routes;
    backend::HipBackend &be = default_backend();
    if (!be.is_available()) throw std::runtime_error("HIP backend unavailable: " + detail::last_error());
    std::lock_guard<std::mutex> lock(mutex());
    std::vector<int32_t> ex(num_tokens * top_k), cnt(num_tokens);
    std::vector<float> w(num_tokens * top_k);
    int lists = 0;
    if (nx_route_topk(be.ctx(), router_logits.data(), router_logits.size(), (int)num_tokens,
                      (int)num_experts, (int)top_k, NX_SCORE_SOFTMAX, ex.data(), w.data(),
                      cnt.data(), &lists) != NX_OK)
      throw std::runtime_error(detail::last_error());
    routes.resize((size_t)lists);
    for (int t = 0; t < lists; ++t)
      for (int r = 0; r < cnt[t]; ++r)
        routes[t].push_back(MoeRoute{(size_t)ex[(size_t)t * top_k + r], w[(size_t)t * top_k + r]});
    return routes;
  }

  /// Dispatch one hidden state through top-k routed SwiGLU experts
  /// (src/engine/mod.rs:969-1024).  F32 weights are uploaded for the routed
  /// experts on each call; use dispatch_moe_ffn_batch with DeviceExperts to
  /// keep (quantized) weights resident.
  static Result<std::vector<float>> dispatch_moe_ffn(const std::vector<float> &hidden,
                                                     const std::vector<float> &router_logits,
                                                     MoeExpertWeights experts,
                                                     MoeDispatchConfig config) {
    using R = Result<std::vector<float>>;
    const size_t num_experts = experts.gate.size();
    if (num_experts == 0 || experts.up.size() != num_experts || experts.down.size() != num_experts)
      return R::err("MoE expert weight lists must be non-empty and aligned");
    if (hidden.size() != config.hidden_size)
      return R::err("MoE hidden shape mismatch: got " + std::to_string(hidden.size()) +
                    ", expected " + std::to_string(config.hidden_size));
    const auto routes = route_moe_experts(router_logits, 1, num_experts, config.top_k);
    if (routes.empty()) return R::err("MoE router produced no routes");
    const size_t H = config.hidden_size, F = config.ff_dim;
    // matvec's checks, in the order the reference reaches them
    for (const MoeRoute &r : routes[0]) {
      const size_t e = r.expert;
      if (experts.gate[e].size() < F * H) return R::err(too_small(experts.gate[e].size(), F * H));
      if (experts.up[e].size() < F * H) return R::err(too_small(experts.up[e].size(), F * H));
      if (experts.down[e].size() < H * F) return R::err(too_small(experts.down[e].size(), H * F));
    }
    std::vector<float> out(H, 0.0f);
    if (routes[0].empty()) return R::ok(out);  // no finite logits: zero output
    backend::HipBackend &be = default_backend();
    std::lock_guard<std::mutex> lock(mutex());
    nx_experts *ex = nullptr;
    if (nx_experts_create(be.ctx(), NX_FMT_F32, (int)num_experts, (int)H, (int)F, &ex) != NX_OK)
      return R::err(detail::last_error());
    std::unique_ptr<nx_experts, int (*)(nx_experts *)> guard(ex, nx_experts_destroy);
    for (const MoeRoute &r : routes[0]) {
      const size_t e = r.expert;
      const std::vector<float> *m[3] = {&experts.gate[e], &experts.up[e], &experts.down[e]};
      for (int role = 0; role < 3; ++role)
        if (nx_experts_load(be.ctx(), ex, (int)e, role, m[role]->data(), F * H * sizeof(float), 0) != NX_OK)
          return R::err(detail::last_error());
    }
    std::vector<float> logits(router_logits.begin(), router_logits.begin() + (long)num_experts);
    if (nx_moe_forward(be.ctx(), ex, hidden.data(), logits.data(), 1, (int)config.top_k,
                       NX_SCORE_SOFTMAX, NX_PATH_GEMV, out.data()) != NX_OK)
      return R::err(detail::last_error());
    return R::ok(out);
  }

  /// Batched sibling over resident (quantized) experts: row t of the result
  /// equals dispatch_moe_ffn on row t.  x is [num_tokens x hidden], logits
  /// [num_tokens x num_experts].
  static Result<std::vector<float>> dispatch_moe_ffn_batch(const DeviceExperts &experts,
                                                           const std::vector<float> &x,
                                                           const std::vector<float> &router_logits,
                                                           size_t num_tokens, size_t top_k,
                                                           int score_mode = NX_SCORE_SOFTMAX,
                                                           int path = NX_PATH_AUTO) {
    using R = Result<std::vector<float>>;
    const size_t H = experts.hidden(), E = experts.num_experts();
    if (x.size() != num_tokens * H)
      return R::err("MoE hidden shape mismatch: got " + std::to_string(x.size()) + ", expected " +
                    std::to_string(num_tokens * H));
    if (router_logits.size() < num_tokens * E || top_k == 0)
      return R::err("MoE router produced no routes");
    std::vector<float> out(num_tokens * H, 0.0f);
    std::lock_guard<std::mutex> lock(mutex());
    if (nx_moe_forward(experts.backend().ctx(), experts.handle(), x.data(), router_logits.data(),
                       (int)num_tokens, (int)top_k, score_mode, path, out.data()) != NX_OK)
      return R::err(detail::last_error());
    return R::ok(out);
  }

 private:
  static std::mutex &mutex() {
    static std::mutex m;
    return m;
  }
  static std::string too_small(size_t got, size_t want) {
    return "Matvec weight too small: got " + std::to_string(got) + ", expected at least " +
           std::to_string(want);
  }
};

}  // namespace engine
}  // namespace nexus
