/*
 * nexus_hip.h — C ABI of libnexus_hip.so, the MI355X (gfx950) MoE routed-FFN
 * path for Nexus.
 *
 * Plain C: pointers, sizes and int status codes only.  Every call returns
 * NX_OK (0) or an NX_ERR_* code and, on failure, sets a thread-local message
 * readable with nx_last_error().  Calls whose pointers are host pointers block
 * until the result is in host memory (the reference path is synchronous);
 * *_dev calls take device pointers and are asynchronous on the context's
 * stream.  A context is not thread-safe: use one context per host thread.
 *
 * Reference interfaces replaced (paths relative to the Nexus repository):
 *   nx_moe_forward / nx_moe_forward_dev
 *       InferenceEngine::dispatch_moe_ffn   src/engine/mod.rs:969-1024
 *       (row t of a batch == dispatch_moe_ffn on row t; the expert products
 *        InferenceEngine::matvec src/engine/mod.rs:775-801 run on device)
 *   nx_router_logits / nx_router_logits_dev
 *       InferenceEngine::matvec             src/engine/mod.rs:775-801
 *       applied to the router weight, one call per token
 *   nx_rms_norm / nx_rms_norm_dev
 *       kernel::rms_norm                    src/kernel/mod.rs:199-209
 *   nx_moe_block / nx_moe_block_dev
 *       the FFN half of a decode_with_cache layer (rms_norm, the FFN, the
 *       residual add_inplace)               src/engine/mod.rs:1129-1142, 803-807
 *       with the MoE layer (router matvec + dispatch_moe_ffn) as the FFN
 *   nx_route_topk
 *       InferenceEngine::route_moe_experts  src/engine/mod.rs:918-966
 *   nx_permute
 *       the per-token route loop             src/engine/mod.rs:994-1021
 *   nx_dequant / nx_dequant_dev
 *       GgufReader::tensor_bytes_to_f32 for Q4_0/Q8_0/Q4_K
 *                                            src/gguf/mod.rs:962-1056
 *       (== QuantEngine::dequantize          src/quant/mod.rs:643-849)
 *   nx_quantize / nx_quantize_dev
 *       QuantEngine::quantize_weights        src/quant/mod.rs:623-818
 *   nx_experts_*
 *       the load-time expert tensors of ModelWeights (src/engine/mod.rs:642),
 *       kept quantized and resident in HBM instead of dequantized to f32
 *   nx_gguf_*
 *       GgufReader::parse_file / parse_from_bytes, ModelMetadata::{get_tensor,
 *       get_usize, get_f32, get_str, absolute_tensor_offset}
 *                                            src/gguf/mod.rs:485-596, 869-900,
 *                                            1091-1310
 *   nx_experts_load_gguf
 *       the tensor loop of InferenceEngine::new (src/engine/mod.rs:600-650)
 *       for a block's expert tensors, without the f32 step or the 10M cap
 *   nx_device_count / nx_ctx_* / nx_sync / nx_mem_info
 *       Backend::{is_available, memory_info, synchronize}
 *                                            src/backend/mod.rs:74-96
 *       for the HIP backend that replaces the CUDA placeholder
 *                                            src/backend/mod.rs:206-212,221-230
 */
#ifndef NEXUS_HIP_H
#define NEXUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define NX_OK 0
#define NX_ERR_INVALID_ARG 1 /* null pointer, bad enum, negative size */
#define NX_ERR_SHAPE 2       /* sizes inconsistent with each other */
#define NX_ERR_UNSUPPORTED 3 /* valid request the library does not implement */
#define NX_ERR_DEVICE 4      /* HIP runtime failure or no gfx950 device */
#define NX_ERR_OOM 5         /* device allocation failed */
#define NX_ERR_TRUNCATED 6   /* quantized payload shorter than its element count */
#define NX_ERR_NO_ROUTES 7   /* router produced no route lists (k == 0, E == 0, ...) */
#define NX_ERR_NOT_FOUND 8   /* named tensor or metadata key absent */
#define NX_ERR_IO 9          /* file could not be opened or mapped */

/* weight formats: GGUF tensor type ids (src/gguf/mod.rs:106-118) */
#define NX_FMT_F32 0
#define NX_FMT_Q4_0 2
#define NX_FMT_Q8_0 8
#define NX_FMT_Q4_K 12
#define NX_FMT_Q2_K 10 /* GEMV path only (decode); dequant/quantize bit-exact */
#define NX_FMT_F16 1   /* IEEE half, GEMV path only; dequant exact (src/gguf/mod.rs:921-933) */
#define NX_FMT_BF16 28 /* bfloat16 (the reference's id, src/gguf/mod.rs:135), GEMV path only;
                          dequant exact (src/gguf/mod.rs:934-946) */

/* router score modes */
#define NX_SCORE_SOFTMAX 0 /* reference: softmax over the selected top-k logits */
#define NX_SCORE_SIGMOID 1 /* extension: sigmoid scores renormalised over the top-k */

/* expert-product paths */
#define NX_PATH_AUTO 0      /* by tokens per expert: GEMV, then (Q4_K and Q2_K with no shared
                               expert or one as wide as the routed experts; Q4_0 and Q8_0 in
                               whole 256-weight chunks with no shared expert) the
                               split-activation MFMA path, then (not Q2_K) the grouped GEMM
                               on bf16 operands */
#define NX_PATH_GEMV 1      /* dequant-in-register GEMV, fp32 accumulate */
#define NX_PATH_MFMA_F16 2  /* grouped GEMM on fp16 MFMA, fp32 accumulate; activations and
                               SwiGLU outputs must stay within fp16's range (|v| < 65504) */
#define NX_PATH_MFMA_BF16 3 /* same on bf16 MFMA */
#define NX_PATH_MFMA_SPLIT 4 /* few tokens per expert (decode batches), Q4_K, Q2_K, or Q4_0 and
                                Q8_0 whose hidden and ff dims are multiples of 256: fp16 MFMA
                                on the raw codes with activations split into two fp16 halves,
                                block and sub-block scales applied to the products; no
                                dequantization.  A shared expert must have the routed experts'
                                ff_dim */

/* expert matrix roles */
#define NX_ROLE_GATE 0 /* [ff_dim x hidden] */
#define NX_ROLE_UP 1   /* [ff_dim x hidden] */
#define NX_ROLE_DOWN 2 /* [hidden x ff_dim] */
#define NX_EXPERT_SHARED (-1)

typedef struct nx_ctx nx_ctx;
typedef struct nx_experts nx_experts;
typedef struct nx_matrix nx_matrix;

/* ---------------------------------------------------------------- runtime */
const char *nx_last_error(void);
int nx_version(void);
/* Number of visible gfx950 devices (Backend::is_available). */
int nx_device_count(int *count);
int nx_ctx_create(int device, nx_ctx **out);
int nx_ctx_destroy(nx_ctx *ctx);
/* Use a caller-owned hipStream_t (NULL restores the context's own stream). */
int nx_ctx_set_stream(nx_ctx *ctx, void *hip_stream);
int nx_ctx_get_stream(nx_ctx *ctx, void **hip_stream);
int nx_sync(nx_ctx *ctx);
int nx_mem_info(nx_ctx *ctx, size_t *free_bytes, size_t *total_bytes);
/* Per-kernel HIP-event timing of *_dev launches (0 = off).  Stats accumulate
 * until reset; index runs over the kernels launched so far. */
int nx_profile_enable(nx_ctx *ctx, int enable);
int nx_profile_reset(nx_ctx *ctx);
int nx_profile_count(nx_ctx *ctx, int *n_kernels);
int nx_profile_get(nx_ctx *ctx, int index, char *name, size_t name_cap, int *launches,
                   double *total_ms);

/* ---------------------------------------------------------------- quant */
/* Payload bytes of n elements (src/gguf/mod.rs:249-293). */
int nx_quant_bytes(int fmt, size_t n_elems, size_t *bytes);
/* Bit-exact dequantization of a GGUF payload; n_elems = output_len. */
int nx_dequant(nx_ctx *ctx, int fmt, const void *src, size_t src_bytes, size_t n_elems,
               float *dst);
int nx_dequant_dev(nx_ctx *ctx, int fmt, const void *d_src, size_t src_bytes, size_t n_elems,
                   float *d_dst);
/* Bit-exact restatement of the reference quantizer on device. */
int nx_quantize(nx_ctx *ctx, int fmt, const float *src, size_t n_elems, void *dst,
                size_t dst_bytes);
int nx_quantize_dev(nx_ctx *ctx, int fmt, const float *d_src, size_t n_elems, void *d_dst,
                    size_t dst_bytes);

/* ---------------------------------------------------------------- routing */
/* Router logits: logits[t * E + e] = sum_c w_router[e * H + c] * x[t * H + c]
 * for T = num_tokens, E = num_experts, H = hidden, all fp32.
 * exact != 0: each (t, e) is summed from 0.0f in column order with every
 * product and every sum rounded once, the order of InferenceEngine::matvec
 * (src/engine/mod.rs:775-801) on token row t, so the logits are bit-identical
 * to the reference's and top-k picks the same experts.  exact == 0: parallel
 * order with fma; |fast - exact| <= 2 (H+1) 2^-24 sum_c |w x|.
 * Errors as in matvec (NX_ERR_SHAPE): x_len != T*H gives "Matvec input shape
 * mismatch: got <x_len>, expected <T*H>"; w_len < E*H gives "Matvec weight
 * too small: got <w_len>, expected at least <E*H>". */
int nx_router_logits(nx_ctx *ctx, const float *w_router, size_t w_len, const float *x,
                     size_t x_len, int num_tokens, int num_experts, int hidden, int exact,
                     float *logits);
int nx_router_logits_dev(nx_ctx *ctx, const float *d_w_router, size_t w_len, const float *d_x,
                         size_t x_len, int num_tokens, int num_experts, int hidden, int exact,
                         float *d_logits);
/* RMSNorm of T = num_tokens rows of H = hidden floats: out[t] = x[t] * rstd_t *
 * w with rstd_t = 1 / sqrt(sum_i x[t][i]^2 / H + eps) (kernel::rms_norm,
 * src/kernel/mod.rs:199-209).  exact != 0: the sum in the reference's order,
 * output bit-identical; exact == 0: parallel sum.  NX_ERR_SHAPE "RMSNorm input
 * shape mismatch: got <x_len>, expected <T*H>" or "RMSNorm weight too small:
 * got <w_len>, expected at least <H>" (the reference panics on the latter). */
int nx_rms_norm(nx_ctx *ctx, const float *x, size_t x_len, const float *weight, size_t w_len,
                float eps, int num_tokens, int hidden, int exact, float *out);
int nx_rms_norm_dev(nx_ctx *ctx, const float *d_x, size_t x_len, const float *d_weight,
                    size_t w_len, float eps, int num_tokens, int hidden, int exact, float *d_out);
/* Top-k routing of [num_tokens x num_experts] logits.  Outputs are
 * [num_tokens x top_k] (expert -1 / weight 0 padding) and counts[num_tokens].
 * *lists is the number of route lists produced (tokens whose logits lie
 * wholly inside logits_len, as in the reference). */
int nx_route_topk(nx_ctx *ctx, const float *logits, size_t logits_len, int num_tokens,
                  int num_experts, int top_k, int score_mode, int32_t *experts, float *weights,
                  int32_t *counts, int *lists);
/* Stable counting sort of (token, slot) pairs by expert: expert_counts[E],
 * offsets[E+1], perm_token/perm_slot[sum(counts)], inv_pos[T x k] (-1 pad). */
int nx_permute(nx_ctx *ctx, const int32_t *experts, const int32_t *counts, int num_tokens,
               int top_k, int num_experts, int32_t *expert_counts, int32_t *offsets,
               int32_t *perm_token, int32_t *perm_slot, int32_t *inv_pos);

/* ---------------------------------------------------------------- experts */
/* A device-resident expert set: E routed experts of [ff_dim x hidden] gate and
 * up and [hidden x ff_dim] down in one format.  Quantized formats need the
 * row length (hidden for gate/up, ff_dim for down) to be a whole number of
 * blocks (256 for Q4_K, 32 for Q8_0/Q4_0). */
int nx_experts_create(nx_ctx *ctx, int fmt, int num_experts, int hidden, int ff_dim,
                      nx_experts **out);
/* Adds one always-on shared expert of shared_ff_dim (weight 1, added after
 * the routed experts). */
int nx_experts_add_shared(nx_ctx *ctx, nx_experts *ex, int shared_ff_dim);
/* Loads one matrix from a GGUF payload (host or device memory) into the
 * resident layout.  expert = 0..E-1 or NX_EXPERT_SHARED. */
int nx_experts_load(nx_ctx *ctx, nx_experts *ex, int expert, int role, const void *src,
                    size_t src_bytes, int src_on_device);
int nx_experts_info(const nx_experts *ex, int *fmt, int *num_experts, int *hidden, int *ff_dim,
                    int *shared_ff_dim, size_t *device_bytes);
// Frees the set's device planes (after the device's work in flight); the
// set may be destroyed before or after its context.
int nx_experts_destroy(nx_experts *ex);

/* ---------------------------------------------------------------- dense matrices */
/* A device-resident dense weight matrix, rows x cols, row-major (a GGUF 2-D
 * tensor of dims [cols, rows]), kept in its quantized format: the q/k/v/o
 * projections and the output head of the decode step
 * (src/engine/mod.rs:1108-1126, 1032-1043), which the reference dequantizes
 * to f32 at load.  Quantized formats need cols to be a whole number of
 * blocks. */
int nx_matrix_create(nx_ctx *ctx, int fmt, int rows, int cols, nx_matrix **out);
/* Loads the GGUF payload (host or device memory).  A payload holding fewer
 * than rows*cols weights gives NX_ERR_SHAPE "Matvec weight too small: got
 * <weights>, expected at least <rows*cols>" (InferenceEngine::matvec,
 * src/engine/mod.rs:775-801). */
int nx_matrix_load(nx_ctx *ctx, nx_matrix *m, const void *src, size_t src_bytes,
                   int src_on_device);
int nx_matrix_info(const nx_matrix *m, int *fmt, int *rows, int *cols, size_t *device_bytes);
int nx_matrix_destroy(nx_matrix *m);
/* y[t * rows + r] = sum_c W[r][c] x[t * cols + c] for T = num_tokens, fp32
 * in and out: InferenceEngine::matvec (src/engine/mod.rs:775-801) on each
 * token row, with the dot product in parallel order (fp32 accumulate) over
 * weights dequantized in registers.  x_len != T*cols gives NX_ERR_SHAPE
 * "Matvec input shape mismatch: got <x_len>, expected <T*cols>". */
int nx_matvec(nx_ctx *ctx, const nx_matrix *m, const float *x, size_t x_len, int num_tokens,
              float *y);
int nx_matvec_dev(nx_ctx *ctx, const nx_matrix *m, const float *d_x, size_t x_len,
                  int num_tokens, float *d_y);

/* ---------------------------------------------------------------- GGUF */
typedef struct nx_gguf nx_gguf;
/* Q4_K code order of a file's payloads */
#define NX_Q4K_REFERENCE 0 /* the reference's (element i<128: low nibble of byte i, else high
                              nibble of byte i-128; src/quant/mod.rs:833-841) */
#define NX_Q4K_GGML 1      /* upstream ggml's (per 64 elements: low nibbles, then high) */

/* Memory-maps and parses a GGUF v2/v3 file as GgufReader::parse_file does
 * (src/gguf/mod.rs:869-876, 1091-1310), with its error messages ("Invalid
 * GGUF magic", "Unsupported GGUF version: 1", "Unexpected EOF reading ...",
 * "Unknown value type: N", "Unknown data type: N", ...).  No GPU needed. */
int nx_gguf_open(const char *path, nx_gguf **out);
int nx_gguf_close(nx_gguf *g);
/* data_offset: start of the tensor data (table end rounded up to alignment). */
int nx_gguf_info(const nx_gguf *g, uint32_t *version, size_t *tensor_count, size_t *kv_count,
                 size_t *alignment, uint64_t *data_offset);
/* Tensor `index`: name, GGUF type id, dims (innermost first, up to dims_cap),
 * absolute file offset and payload bytes (TensorInfo::data_size). */
int nx_gguf_tensor(const nx_gguf *g, size_t index, char *name, size_t name_cap, uint32_t *type,
                   uint32_t *n_dims, uint64_t *dims, size_t dims_cap, uint64_t *offset,
                   uint64_t *bytes);
/* NX_ERR_NOT_FOUND "Missing tensor: <name>" if absent. */
int nx_gguf_find_tensor(const nx_gguf *g, const char *name, size_t *index);
/* Pointer into the mapping; NX_ERR_TRUNCATED if the payload passes the file end. */
int nx_gguf_tensor_data(const nx_gguf *g, size_t index, const void **data, uint64_t *bytes);
/* ModelMetadata::get_usize (U64, U32, non-negative I64/I32), get_f32, get_str. */
int nx_gguf_meta_usize(const nx_gguf *g, const char *key, uint64_t *value);
int nx_gguf_meta_f32(const nx_gguf *g, const char *key, float *value);
int nx_gguf_meta_str(const nx_gguf *g, const char *key, char *buf, size_t cap, size_t *len);
/* The MoE expert tensors of block `layer`: merged blk.L.ffn_{gate,up,down}_exps
 * ([H,F,E] / [F,H,E], innermost first) or one tensor per expert
 * (blk.L.ffn_gate.e.weight, Mixtral-HF ...experts.e.w1/w3/w2, ...mlp.experts.e.
 * {gate,up,down}_proj), plus a shared expert (blk.L.ffn_gate_shexp.weight, ...). */
int nx_gguf_moe_info(const nx_gguf *g, int layer, int *fmt, int *num_experts, int *hidden,
                     int *ff_dim, int *shared_ff_dim);
/* Loads block `layer`'s experts into a new resident set, payloads kept
 * quantized (no f32 copy); q4k_order says how the file orders Q4_K codes. */
int nx_experts_load_gguf(nx_ctx *ctx, const nx_gguf *g, int layer, int q4k_order,
                         nx_experts **out);
/* Loads the tensor called `name` into a new dense matrix (rows = product of
 * dims[1..], cols = dims[0]); NX_ERR_NOT_FOUND "Missing tensor: <name>" if
 * absent (InferenceEngine::tensor, src/engine/mod.rs:718-725). */
int nx_matrix_load_gguf(nx_ctx *ctx, const nx_gguf *g, const char *name, int q4k_order,
                        nx_matrix **out);
/* Q4_K blocks from upstream ggml's code order to the reference's (host). */
int nx_q4k_from_ggml(const void *src, void *dst, size_t blocks);

/* ---------------------------------------------------------------- forward */
/* The MoE layer for a batch: out[t] = sum_r w[t,r] * FFN_{e[t,r]}(x[t])
 * (+ shared FFN(x[t])).  x [T x hidden], logits [T x E], out [T x hidden],
 * fp32.  Row t equals dispatch_moe_ffn(x[t], logits[t]). */
int nx_moe_forward(nx_ctx *ctx, const nx_experts *ex, const float *x, const float *logits,
                   int num_tokens, int top_k, int score_mode, int path, float *out);
int nx_moe_forward_dev(nx_ctx *ctx, const nx_experts *ex, const float *d_x,
                       const float *d_logits, int num_tokens, int top_k, int score_mode,
                       int path, float *d_out);

/* The routes of the last nx_moe_forward[_dev|_noalloc] or nx_moe_block[_dev]
 * on this context, as route_moe_experts returns them (src/engine/mod.rs:
 * 918-966): experts / weights [num_tokens x top_k] (-1 / 0 padding) and
 * counts[num_tokens], copied to host memory.  num_tokens and top_k must be the
 * last call's; valid until the next call on the context (or, after the
 * no-allocation entry point, the next such call on the device).  For a
 * single token on the GEMV path these are the routes the gate/up kernel
 * computed itself.  A forward that failed records no routes: this call then
 * returns NX_ERR_INVALID_ARG until a forward completes. */
int nx_moe_last_routes(nx_ctx *ctx, int num_tokens, int top_k, int32_t *experts, float *weights,
                       int32_t *counts);

/* No counterpart in the reference.  nx_moe_forward_dev for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): same arguments, semantics and
 * kernels, but every intermediate buffer (routes, permutation, SwiGLU
 * activations, per-pair outputs, tile lists) is carved from one static
 * 64 MiB device array that each GPU holds until the process ends, and the
 * call makes no hipMalloc, hipFree, hipMemset or event call.  A call whose
 * intermediates do not fit returns NX_ERR_UNSUPPORTED before any kernel of the
 * layer writes d_out (the Mixtral shape fits up to 32 tokens on the decode
 * paths; prefill batches use nx_moe_forward_dev).  Profiling must
 * be off.  Every call on one GPU shares that GPU's array, whatever the
 * context or stream: calls that overlap in time on one GPU race. */
int nx_moe_forward_noalloc(nx_ctx *ctx, const nx_experts *ex, const float *d_x,
                           const float *d_logits, int num_tokens, int top_k, int score_mode,
                           int path, float *d_out);

/* One MoE block of a decoder layer, in place on hidden [T x H]:
 *   normed = rms_norm(hidden, norm_w, eps); logits = W_r . normed;
 *   hidden += MoE(normed, logits).
 * exact != 0: rms_norm and the logits are bit-identical to the reference's,
 * so routing is the reference's.  Errors as nx_rms_norm and nx_router_logits
 * (router_len < E*H: "Matvec weight too small"), then nx_moe_forward. */
int nx_moe_block(nx_ctx *ctx, const nx_experts *ex, float *hidden, const float *norm_w,
                 size_t norm_len, float eps, const float *router_w, size_t router_len,
                 int num_tokens, int top_k, int score_mode, int path, int exact);
int nx_moe_block_dev(nx_ctx *ctx, const nx_experts *ex, float *d_hidden, const float *d_norm_w,
                     size_t norm_len, float eps, const float *d_router_w, size_t router_len,
                     int num_tokens, int top_k, int score_mode, int path, int exact);

#ifdef __cplusplus
}
#endif
#endif
