/*
 * nx_oracle.h — CPU restatement of the Nexus MoE routed-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the oracle that the HIP product is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it.
 *
 * Every function restates one reference function (file:line relative to the
 * reference repository root) with the same arithmetic order, compiled with
 * -O2 -ffp-contract=off and no fast-math so that f32 sums are unfused and
 * left-to-right, as Rust evaluates them.
 */
#ifndef NX_ORACLE_H
#define NX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* half 2.x: f16::to_f32 (exact) and f16::from_f32 (IEEE round-to-nearest-even). */
float nxo_f16_to_f32(uint16_t h);
uint16_t nxo_f32_to_f16(float f);
void nxo_f32_to_f16_array(const float *src, size_t n, uint16_t *dst);

/* Block byte sizes: src/gguf/mod.rs:262-272. */
size_t nxo_quant_bytes(int gguf_type, size_t n_elems);

/* QuantEngine::quantize_q8_0 / quantize_q4_0 / quantize_q4_k
 * (src/quant/mod.rs:669-687, 705-721, 756-818).  `nthreads` splits the work
 * on block boundaries; blocks are independent so the bytes do not depend on it. */
size_t nxo_quantize(int gguf_type, const float *src, size_t n, uint8_t *dst, int nthreads);

/* QuantEngine::dequantize_* (src/quant/mod.rs:689-703, 723-745, 820-849).
 * Returns the number of values written (stops at output_len or at the last
 * whole block, as the reference does). */
size_t nxo_dequantize(int gguf_type, const uint8_t *src, size_t src_bytes, size_t output_len,
                      float *dst, int nthreads);

/* unpack_q4_k_scales / pack_q4_k_scales (src/quant/mod.rs:1153-1170). */
void nxo_unpack_q4k_scales(const uint8_t *packed12, uint8_t *scales8, uint8_t *mins8);
void nxo_pack_q4k_scales(const uint8_t *scales8, const uint8_t *mins8, uint8_t *packed12);

/* InferenceEngine::route_moe_experts (src/engine/mod.rs:918-966).
 * Writes route lists row-major [tokens x top_k] (expert=-1, weight=0 padding)
 * and counts[tokens].  Returns the number of route lists produced (the
 * reference stops early when a token's logits run past the slice end).
 * score_mode 0 = reference softmax over the selected logits;
 * score_mode 1 = sigmoid scores renormalised over the selected set (an
 * extension with no reference counterpart; selection order is identical). */
size_t nxo_route(const float *logits, size_t logits_len, size_t num_tokens, size_t num_experts,
                 size_t top_k, int score_mode, int32_t *experts, float *weights, int32_t *counts);

/* Token -> expert permutation: stable counting sort of the (token, slot)
 * pairs by expert (no reference counterpart; the reference visits the same
 * pairs token by token in src/engine/mod.rs:994).  offsets has E+1 entries;
 * inv_pos[t*k + r] = position of pair (t, r) in the permuted order or -1. */
size_t nxo_permute(const int32_t *experts, const int32_t *counts_per_token, size_t num_tokens,
                   size_t top_k, size_t num_experts, int32_t *expert_counts, int32_t *offsets,
                   int32_t *perm_token, int32_t *perm_slot, int32_t *inv_pos);

/* kernel::rms_norm (src/kernel/mod.rs:199-209) of one row of dim values. */
void nxo_rms_norm(const float *x, const float *w, size_t dim, float eps, float *out);

/* InferenceEngine::matvec (src/engine/mod.rs:775-801).  0 = ok, else an
 * error code whose message is written to err. */
int nxo_matvec(const float *w, size_t w_len, size_t rows, size_t cols, const float *x,
               size_t x_len, float *y, char *err, size_t err_cap);

/* InferenceEngine::dispatch_moe_ffn (src/engine/mod.rs:969-1024) for one
 * token.  Expert matrices are passed as pointer + length per expert so a
 * missing (NULL, 0) expert behaves like an empty Vec. */
int nxo_dispatch_moe_ffn(const float *hidden, size_t hidden_len, const float *logits,
                         size_t logits_len, const float *const *gate, const size_t *gate_len,
                         const float *const *up, const size_t *up_len, const float *const *down,
                         const size_t *down_len, size_t num_experts, size_t top_k,
                         size_t hidden_size, size_t ff_dim, float *out, char *err, size_t err_cap);

/* Batched layer: token t's output equals nxo_dispatch_moe_ffn on row t, with
 * the sigmoid score extension and an optional always-on shared expert
 * (weight 1, added after the routed experts).  Shared pointers may be NULL. */
int nxo_moe_layer(const float *x, const float *logits, size_t num_tokens, size_t num_experts,
                  size_t top_k, int score_mode, const float *const *gate,
                  const float *const *up, const float *const *down, const float *shared_gate,
                  const float *shared_up, const float *shared_down, size_t hidden_size,
                  size_t ff_dim, size_t shared_ff_dim, float *out, int nthreads);

/* kernel::swiglu_ffn (src/kernel/mod.rs:104-157): (w1.x) * silu(w3.x), then w2. */
void nxo_swiglu_ffn(const float *input, size_t input_len, const float *w1, const float *w3,
                    const float *w2, size_t hidden_size, size_t ff_dim, float *out);

/* CpuBackend::matmul (src/backend/cpu.rs:23-38): C[m x n] = A[m x k] B[k x n],
 * rows split across threads. */
void nxo_cpu_matmul(const float *a, const float *b, size_t m, size_t n, size_t k, float *c,
                    int nthreads);

#ifdef __cplusplus
}
#endif
#endif
