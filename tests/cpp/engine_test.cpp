// engine_test.cpp — the reference's MoE helper and backend tests, restated
// against the C++ host API (include/nexus_engine.hpp) running on the GPU.
//   test_route_moe_experts_selects_top_k      src/engine/mod.rs:1622-1630
//   test_dispatch_moe_ffn_runs_top_k_experts  src/engine/mod.rs:1632-1656
//     (plus its closed-form value: expert 1 with weight 1 gives 0.2*silu(1.5)*0.75)
//   error strings                             src/engine/mod.rs:975-991, 777-788
//   test_backend_capabilities                 src/backend/mod.rs:274-285
//     (with HIP present where the reference asserts CUDA unavailable)
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "nexus_engine.hpp"

using namespace nexus;
using namespace nexus::engine;

static int failures = 0;
#define CHECK(cond)                                                       \
  do {                                                                    \
    if (!(cond)) {                                                        \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);         \
      ++failures;                                                         \
    }                                                                     \
  } while (0)

static std::vector<float> identity(size_t rows, size_t cols) {
  std::vector<float> w(rows * cols, 0.0f);
  for (size_t i = 0; i < rows && i < cols; ++i) w[i * cols + i] = 1.0f;
  return w;
}

static void test_route_moe_experts_selects_top_k() {
  auto routes = InferenceEngine::route_moe_experts({0.1f, 3.0f, 1.0f, 2.0f, 0.5f, 0.2f}, 2, 3, 2);
  CHECK(routes.size() == 2);
  CHECK(routes[0][0].expert == 1);
  CHECK(routes[0][1].expert == 2);
  float sum = 0.0f;
  for (auto &r : routes[0]) sum += r.weight;
  CHECK(std::fabs(sum - 1.0f) < 1e-6f);
}

static void test_dispatch_moe_ffn_runs_top_k_experts() {
  std::vector<float> hidden = {1.0f, 2.0f};
  std::vector<std::vector<float>> gate = {identity(2, 2), std::vector<float>(4, 0.5f)};
  std::vector<std::vector<float>> up = {identity(2, 2), std::vector<float>(4, 0.25f)};
  std::vector<std::vector<float>> down = {identity(2, 2), std::vector<float>(4, 0.1f)};
  auto out = InferenceEngine::dispatch_moe_ffn(hidden, {0.0f, 4.0f}, MoeExpertWeights{gate, up, down},
                                               MoeDispatchConfig{1, 2, 2});
  CHECK(out.is_ok());
  const auto &v = out.unwrap();
  CHECK(v.size() == 2);
  CHECK(std::isfinite(v[0]) && std::isfinite(v[1]));
  const double a = 1.5 / (1.0 + std::exp(-1.5)) * 0.75;
  CHECK(std::fabs(v[0] - 0.2 * a) < 1e-6 && std::fabs(v[1] - 0.2 * a) < 1e-6);
}

static void test_dispatch_errors() {
  auto I = identity(2, 2);
  std::vector<std::vector<float>> two = {I, I}, none;
  auto e1 = InferenceEngine::dispatch_moe_ffn({1, 2, 3}, {0, 1}, {two, two, two}, {1, 2, 2});
  CHECK(e1.is_err() && e1.unwrap_err() == "MoE hidden shape mismatch: got 3, expected 2");
  auto e2 = InferenceEngine::dispatch_moe_ffn({1, 2}, {0, 1}, {two, two, two}, {0, 2, 2});
  CHECK(e2.is_err() && e2.unwrap_err() == "MoE router produced no routes");
  auto e3 = InferenceEngine::dispatch_moe_ffn({1, 2}, {0}, {two, two, two}, {1, 2, 2});
  CHECK(e3.is_err() && e3.unwrap_err() == "MoE router produced no routes");
  std::vector<std::vector<float>> short_gate = {I, std::vector<float>(3, 1.0f)};
  auto e4 = InferenceEngine::dispatch_moe_ffn({1, 2}, {0, 1}, {short_gate, two, two}, {1, 2, 2});
  CHECK(e4.is_err() && e4.unwrap_err() == "Matvec weight too small: got 3, expected at least 4");
  auto e5 = InferenceEngine::dispatch_moe_ffn({1, 2}, {0, 1}, {none, none, none}, {1, 2, 2});
  CHECK(e5.is_err() && e5.unwrap_err() == "MoE expert weight lists must be non-empty and aligned");
  // all logits non-finite: one empty route list and a zero output
  auto z = InferenceEngine::dispatch_moe_ffn({1, 2}, {NAN, INFINITY}, {two, two, two}, {2, 2, 2});
  CHECK(z.is_ok() && z.unwrap()[0] == 0.0f && z.unwrap()[1] == 0.0f);
  // an un-routed expert may be empty; longer weights are accepted
  std::vector<std::vector<float>> g2 = {{}, {1, 0, 0, 1, 9}}, u2 = {{}, I}, d2 = {{}, I};
  auto ok = InferenceEngine::dispatch_moe_ffn({1, 2}, {0, 1}, {g2, u2, d2}, {1, 2, 2});
  CHECK(ok.is_ok());
}

static void test_backend_capabilities() {
  backend::HipBackend be(0);
  CHECK(std::string(be.name()) == "hip");
  CHECK(be.is_available());
  auto caps = be.capabilities();
  CHECK(caps.available);
  bool has_moe = false;
  for (auto op : caps.supported_ops) has_moe |= std::string(op) == "moe_ffn";
  CHECK(has_moe);
  auto mem = be.memory_info();
  CHECK(mem.total_memory > 0);
  CHECK(mem.utilization() >= 0.0f && mem.utilization() <= 1.0f);
  be.synchronize();
}

static void test_batched_sibling_matches_rows() {
  // Q8_0 experts built from exact codes: each block is 32 codes with scale 1/64
  const size_t E = 4, H = 64, F = 64, T = 5, k = 2;
  backend::HipBackend &be = InferenceEngine::default_backend();
  DeviceExperts dev(be, NX_FMT_Q8_0, E, H, F);
  std::vector<std::vector<float>> gate(E), up(E), down(E);
  const uint16_t scale_bits = 0x2400;  // f16 1/64
  unsigned seed = 12345;
  auto rnd = [&]() { seed = seed * 1103515245u + 12345u; return (int)((seed >> 16) % 31) - 15; };
  for (size_t e = 0; e < E; ++e) {
    for (int role = 0; role < 3; ++role) {
      std::vector<uint8_t> payload;
      std::vector<float> dense;
      for (size_t b = 0; b < H * F / 32; ++b) {
        payload.push_back(scale_bits & 0xFF);
        payload.push_back(scale_bits >> 8);
        for (int i = 0; i < 32; ++i) {
          const int q = rnd();
          payload.push_back((uint8_t)(int8_t)q);
          dense.push_back((float)q / 64.0f);
        }
      }
      CHECK(dev.load(e, role, payload.data(), payload.size()).is_ok());
      (role == 0 ? gate : role == 1 ? up : down)[e] = dense;
    }
  }
  std::vector<float> x(T * H), logits(T * E);
  for (auto &v : x) v = (float)rnd() / 8.0f;
  for (auto &v : logits) v = (float)rnd() / 4.0f;
  auto batch = InferenceEngine::dispatch_moe_ffn_batch(dev, x, logits, T, k, NX_SCORE_SOFTMAX, NX_PATH_GEMV);
  CHECK(batch.is_ok());
  for (size_t t = 0; t < T; ++t) {
    std::vector<float> xt(x.begin() + t * H, x.begin() + (t + 1) * H);
    std::vector<float> lt(logits.begin() + t * E, logits.begin() + (t + 1) * E);
    auto one = InferenceEngine::dispatch_moe_ffn(xt, lt, {gate, up, down}, {k, H, F});
    CHECK(one.is_ok());
    double num = 0, den = 0;
    for (size_t h = 0; h < H; ++h) {
      const double d = batch.unwrap()[t * H + h] - one.unwrap()[h];
      num += d * d;
      den += (double)one.unwrap()[h] * one.unwrap()[h];
    }
    CHECK(std::sqrt(num / (den > 0 ? den : 1)) < 1e-5);
  }
}

int main() {
  test_route_moe_experts_selects_top_k();
  test_dispatch_moe_ffn_runs_top_k_experts();
  test_dispatch_errors();
  test_backend_capabilities();
  test_batched_sibling_matches_rows();
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
