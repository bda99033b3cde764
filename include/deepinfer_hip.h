/*
 * deepinfer_hip.h - C ABI of libdeepinfer_hip, the MI355X (gfx950) quantized-matmul
 * library for Qwen3.6-35B-A3B MLX-affine group-64 weights (5-bit and 8-bit).
 *
 * Conventions shared by every entry point:
 *   - Handles are opaque pointers. Functions returning a handle return NULL on failure.
 *   - Functions returning int return 0 on success and -1 on failure.
 *   - `error`/`capacity`: a caller buffer (the managed caller uses 2048 bytes) that
 *     receives a NUL-terminated UTF-8 message on failure (bridge.mm:9-15).
 *   - Every argument is validated before any GPU work is queued: an invalid call
 *     launches nothing and leaves outputs untouched (QuantizedTests.cs:118-135, 210-227).
 *   - Weight layout is the checkpoint's MLX affine layout, unchanged:
 *       packed  uint32 [experts, rows, columns*bits/32], codes LSB-first (bit c*bits)
 *       scales  bf16   [experts, rows, columns/64]
 *       biases  bf16   [experts, rows, columns/64]
 *     w = float(code)*scale + bias (quantized.mm:41-53).
 *   - Entry points whose name does not start with dih_quant_ take DEVICE pointers and a
 *     hipStream_t passed as void* (NULL = the context's own stream). They only enqueue
 *     work; the caller synchronizes the stream. bf16 buffers are raw uint16 bit patterns.
 *     The context's stream is a blocking stream: work on it is ordered against the HIP
 *     null stream in both directions (the legacy default-stream rule), so buffers a caller
 *     fills on the null stream are complete before a NULL-stream call reads them.
 *   - Entry points named dih_quant_* take HOST pointers and are synchronous, like the
 *     reference's di_quant_* functions.
 *   - A call's work is complete when its stream's work is (dih_moe_prefill's side-stream
 *     branch joins back into it). A context has no internal locking: callers serialize
 *     calls on one context (the reference serializes through Qwen36Model.cs:18, 47).
 */
#ifndef DEEPINFER_HIP_H
#define DEEPINFER_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One independent GEMV job. Same field order and sizes as QuantJob (quantized.mm:24-30)
 * and QuantNative.Job (QuantizedMetal.cs:250-258). */
typedef struct dih_job {
    void *matrix;
    const float *input;
    float *output;
    const uint32_t *experts;
    int32_t count, batched;
} dih_job;

/* ---- context ------------------------------------------------------------------- */

/* Replaces di_quant_create (quantized.mm:282-286). Uses device 0 of the process's
 * visible HIP devices and creates one blocking stream (ordered against the null stream),
 * plus a non-blocking side stream that dih_moe_prefill forks from and joins back into the
 * call's stream (default priority, both). */
void *dih_quant_create(char *error, int capacity);
/* Replaces di_quant_create_configured (quantized.mm:242-281). `resident` (0/1) and
 * `refresh` (0..60000 ms) are validated like the reference; HIP device memory needs no
 * residency set, so `resident` only switches dih_quant_residency_bytes reporting on. */
void *dih_quant_create_configured(int resident, int refresh, char *error, int capacity);
/* Replaces di_quant_destroy (quantized.mm:293). Frees every scratch buffer. */
void dih_quant_destroy(void *context);
/* Replaces di_quant_residency_bytes (quantized.mm:287-289): device bytes held by the
 * weights of live matrices when created with resident=1, else 0. */
uint64_t dih_quant_residency_bytes(void *context);
/* Replaces di_quant_residency_prepare (quantized.mm:290-292). No work on HIP. */
void dih_quant_residency_prepare(void *context);

/* ---- matrices -------------------------------------------------------------------- */

/* Replaces di_quant_matrix_create (quantized.mm:294-315). Checks 1<=experts<=256,
 * rows>=1, columns a multiple of 64, bits 5 or 8, group 64. Unlike the reference, columns
 * are limited to 8192 (the GEMV kernels hold a call's activations, up to 8192 of them, in
 * LDS or registers; the model's widest input is 4096): wider matrices are refused here,
 * with the usual error, rather than by the calls. A 5-bit matrix with columns a multiple of
 * 512 also holds a second device copy of its codes in 128-row tile-major order, rows padded
 * to whole 256-row tiles (the prefill GEMM reads that one), which every write path below
 * keeps current; its bytes count in dih_quant_residency_bytes. */
void *dih_quant_matrix_create(void *context, int experts, int rows, int columns, int bits,
                              int group, char *error, int capacity);
/* Replaces di_quant_matrix_buffer (quantized.mm:316-319). index 0 packed, 1 scales,
 * 2 biases. Metal returns unified memory; here the pointer is a pinned HOST staging
 * copy of that buffer. Asking for the pointer marks the buffer dirty and the next call
 * that reads the matrix uploads it, so `write through the pointer, then multiply`
 * (QuantizedMetal.cs:171-178) works unchanged. NULL on a bad index. */
void *dih_quant_matrix_buffer(void *matrix, int index);
/* Replaces di_quant_matrix_destroy (quantized.mm:320). */
void dih_quant_matrix_destroy(void *matrix);

/* New (HIP has no unified memory): copies `bytes` from `source` (host or device memory)
 * into buffer
 * `index` at byte `offset` of the device copy directly, without a staging copy. */
int dih_quant_matrix_write(void *matrix, int index, size_t offset, const void *source,
                           size_t bytes, char *error, int capacity);
/* New: uploads a dirty staging buffer now and releases the host staging copy; also
 * brings the tile-major copy of 5-bit codes up to date after writes through the
 * dih_quant_matrix_device pointer. */
int dih_quant_matrix_commit(void *matrix, char *error, int capacity);
/* New: device pointer of buffer `index` (0 packed, 1 scales, 2 biases) for callers
 * that fill weights on the device; uploads a dirty staging copy first. Codes of a 5-bit
 * matrix written through it are seen by every later call: once the codes' pointer has been
 * handed out, each call that uses the matrix first rewrites the prefill GEMM's tile-major
 * copy of the codes (host-synchronous, a pass over the codes), until
 * dih_quant_matrix_commit after the last write ends that. */
void *dih_quant_matrix_device(void *matrix, int index);
/* New: shape query; any out pointer may be NULL. */
int dih_quant_matrix_shape(void *matrix, int *experts, int *rows, int *columns, int *bits);

/* ---- synchronous host-pointer compute (reference ABI) ---------------------------- */

/* Replaces di_quant_batch (quantized.mm:321-345): 1..8 jobs with distinct matrices;
 * y[slot*rows+row] = sum_c w(experts[slot],row,c) * x[(batched?slot*columns:0)+c].
 * `ms` receives the GPU interval of the submission. */
int dih_quant_batch(void *context, const dih_job *jobs, int count, double *ms, char *error,
                    int capacity);
/* Replaces di_quant_matvec (quantized.mm:346-349). */
int dih_quant_matvec(void *context, void *matrix, const float *x, float *out,
                     const uint32_t *experts, int count, int batched, double *ms, char *error,
                     int capacity);
/* Replaces di_quant_experts (quantized.mm:350-383): per slot, act = silu(gate.x)*(up.x),
 * out[slot] = down[expert].act; sharedOut = shared.sharedInput. Three kernels, one
 * submission. */
int dih_quant_experts(void *context, void *gate, void *up, void *down, void *shared,
                      const float *input, const float *sharedInput, const uint32_t *experts,
                      int count, float *expertOutput, float *sharedOutput, double *ms,
                      char *error, int capacity);
/* Replaces di_quant_embedding (quantized.mm:384-397): dequantizes row `token` of a
 * single-expert matrix into out[columns]. Returns -1 on bad arguments. */
int dih_quant_embedding(void *matrix, int token, float *out);

/* ---- device-resident hot path ------------------------------------------------------ */

enum { DIH_F32 = 0, DIH_BF16 = 1 };

/* Decode qmv (M=1 GEMV, quant_rows semantics quantized.mm:119-144 and g_gemv
 * gpu_graph.mm:285-294). x is bf16 or f32 [count or 1][columns]; y is f32 or bf16
 * [count][rows]. `experts` is a DEVICE array of `count` ids or NULL (expert 0,
 * count must be 1); an id >= experts yields NaN outputs for its slot. */
int dih_qmv(void *context, void *matrix, const void *x, int x_dtype, void *y, int y_dtype,
            const uint32_t *experts, int count, int batched, void *stream, char *error,
            int capacity);

/* Fused gate/up + SwiGLU GEMV (expert_gate_up, quantized.mm:148-189):
 * act[slot*rows+row] = silu(gate.x) * (up.x), f32 output. x is shared by all slots. */
int dih_qmv_swiglu(void *context, void *gate, void *up, const void *x, int x_dtype,
                   float *act, const uint32_t *experts, int count, void *stream, char *error,
                   int capacity);

/* Split lm_head + argmax (classifier GEMV gpu_graph.mm:446-448; argmax
 * gpu_graph.mm:160-175). `slices` are single-expert 8- or 5-bit matrices with the same
 * columns whose rows concatenate to the vocabulary; x is bf16 [columns]; logits f32
 * [sum rows]; next (u32, device) = lowest index of the maximum, 0xffffffff when any
 * logit is not finite. */
int dih_lm_head(void *context, void *const *slices, int slice_count, const void *x,
                float *logits, uint32_t *next, void *stream, char *error, int capacity);

/* Argmax alone over n f32 device values (gpu_graph.mm:160-175). */
int dih_argmax(void *context, const float *values, int n, uint32_t *next, void *stream,
               char *error, int capacity);

/* Router selection: per token top-8 of `experts` logits (f32 or bf16 [tokens][experts]),
 * ties to the lowest id, probabilities = softmax over the eight chosen logits
 * (Qwen36Model.cs:246-262, graph_top8 gpu_graph.mm:134-146). ids u32 [tokens][8],
 * probs f32 [tokens][8]. `status` (device u32, may be NULL) is set to 1 when a logit
 * is not finite (the reference throws, Qwen36Model.cs:252). experts <= 256. */
int dih_top8(void *context, const void *logits, int logits_dtype, int tokens, int experts,
             uint32_t *ids, float *probs, uint32_t *status, void *stream, char *error,
             int capacity);

/* Route grouping (prefill_build_groups, prefill_moe.mm:8-17, made deterministic):
 * counts[e] = routes r = t*8+slot with ids[r]==e; routes[e*tokens + k] lists them in
 * ascending order. Devices arrays: ids u32 [tokens*8], counts u32 [experts],
 * routes u32 [experts*tokens]. */
int dih_build_groups(void *context, const uint32_t *ids, int tokens, int experts,
                     uint32_t *counts, uint32_t *routes, void *stream, char *error,
                     int capacity);

/* Dequantize one expert of a matrix to bf16 [rows][columns] with round-to-nearest-even
 * (expanded_weights, prefill_bf16_expanded.mm:8-16). */
int dih_dequant_bf16(void *context, void *matrix, int expert, uint16_t *out, void *stream,
                     char *error, int capacity);

/* Weights of one MoE layer (Qwen36Weights.cs:93-100). router and shared_route are
 * 8-bit; gate/up [E, I, H], down [E, H, I], shared_gate/shared_up [1, Is, H],
 * shared_down [1, H, Is], shared_route [1, 1, H]. router may be NULL when the caller
 * supplies logits. */
typedef struct dih_moe_layer {
    void *router;
    void *gate, *up, *down;
    void *shared_gate, *shared_up, *shared_down;
    void *shared_route;
} dih_moe_layer;

/* Optional device outputs for inspection; any field may be NULL. */
typedef struct dih_moe_trace {
    float *logits;    /* f32 [tokens][E] router logits (decode: computed; prefill: copied) */
    uint32_t *ids;    /* u32 [tokens][8] */
    float *probs;     /* f32 [tokens][8] */
    float *expert_out;/* f32 [tokens*8 + tokens][H] per-route down outputs before weighting
                         (decode: the 8 slots then the shared expert, like the outputs of
                         di_quant_experts); shared expert rows follow the routed ones */
    uint32_t *status; /* u32, set to 1 when a router logit is not finite (the reference
                         throws, Qwen36Model.cs:252); the caller zeroes it */
} dih_moe_trace;

/* Decode MoE step for one token (g_router, gpu_graph.mm:307-320, host form
 * Qwen36Model.cs:218-245): logits = router.x (or `logits` if non-NULL, f32 [E]),
 * top-8, act = silu(gate.x)*(up.x) for the 8 experts and the shared expert,
 * y = sigmoid(shared_route.x)*shared_down.sact + sum_slot p_slot*down[e_slot].act_slot
 * (slot order 0..7), residual = bf16(residual + y). x, residual: bf16 [H]. */
int dih_moe_decode(void *context, const dih_moe_layer *layer, const void *x,
                   const float *logits, void *residual, const dih_moe_trace *trace,
                   void *stream, char *error, int capacity);

/* Residual storage and next-layer norm for the MoE steps (graph_merge_norm,
 * gpu_graph.mm:48-61; prefill_merge, gpu_prefill.mm:140-150). residual_f32 = 1 keeps the
 * residual stream in f32 like the reference (0: bf16 bit patterns). With norm_weight
 * (f32 [H]) the step also writes normed[t] = r[t] * rsqrt(sum_h r[t][h]^2 / H + epsilon) *
 * norm_weight over the stored residual r (f32 when normed_f32 = 1, else bf16); epsilon must be
 * finite and > 0 (Qwen36Weights.cs:51) and normed must not be the residual buffer. */
typedef struct dih_moe_merge {
    int residual_f32;
    const float *norm_weight;
    float epsilon;
    void *normed;
    int normed_f32;
} dih_moe_merge;

/* dih_moe_decode with merge options (NULL: bf16 residual, no norm). The norm is one more
 * single-block launch after the merge (every output row must be final before the sum of
 * squares). */
int dih_moe_decode_norm(void *context, const dih_moe_layer *layer, const void *x,
                        const float *logits, void *residual, const dih_moe_merge *merge,
                        const dih_moe_trace *trace, void *stream, char *error, int capacity);

/* No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * dih_moe_decode_norm with the same arguments, kernels and results, whose intermediate
 * buffers come from a fixed 128 KiB device array that the library holds on every GPU it
 * runs on until the process ends, instead of the context's grow-only scratch. It calls no
 * hipMalloc or hipFree and records no profiling events. Limit: the step's buffers
 * (256-byte aligned: logits [E], SwiGLU rows [8*I + Is], shared down [H], ids, probs and
 * 128 router candidates) must fit in 128 KiB; every layer shape the MoE entry points accept
 * (E <= 256, I and Is <= 2048, H <= 8192) does, and a larger one is rejected with an error.
 * Calls on one GPU share that array (it keeps the last call's contents; nothing in it needs
 * clearing): calls that overlap on one GPU, from any context or stream, race. */
int dih_moe_decode_noalloc(void *context, const dih_moe_layer *layer, const void *x,
                           const float *logits, void *residual, const dih_moe_merge *merge,
                           const dih_moe_trace *trace, void *stream, char *error, int capacity);

/* Prefill MoE chunk (gpu_prefill.mm:700-706 with packed_expert_gate_fused /
 * packed_expert_down, prefill_expert_packed.mm, and prefill_merge gpu_prefill.mm:140-150):
 * top-8 of logits (bf16 or f32 [T][E]) -> grouped per-expert route lists -> bf16 MFMA
 * gate/up + SwiGLU over gathered tokens -> bf16 MFMA down -> weighted sum with the
 * sigmoid-gated shared expert -> residual = bf16(residual + y). x, residual bf16 [T][H].
 * Scratch lives in the context and grows on demand (hipMalloc only when a larger chunk
 * than any before is seen). With 5-bit experts averaging more than 48 routes, the shared
 * expert's gate/up and down run on the context's side stream, forked from `stream` and
 * joined back into it through events (both branches land in a graph captured on
 * `stream`): the call's work is complete when `stream`'s work is. */
int dih_moe_prefill(void *context, const dih_moe_layer *layer, int tokens, const void *x,
                    const void *logits, int logits_dtype, void *residual,
                    const dih_moe_trace *trace, void *stream, char *error, int capacity);

/* dih_moe_prefill with merge options (NULL: bf16 residual, no norm); the norm is fused into
 * the per-token merge (prefill_merge, gpu_prefill.mm:140-150). */
int dih_moe_prefill_norm(void *context, const dih_moe_layer *layer, int tokens, const void *x,
                         const void *logits, int logits_dtype, void *residual,
                         const dih_moe_merge *merge, const dih_moe_trace *trace, void *stream,
                         char *error, int capacity);

/* One grouped expert projection of prefill: the grouped gate/up (p_gate,
 * gpu_prefill.mm:621-633) or the grouped down (p_gemv with experts, gpu_prefill.mm:603-620)
 * on its own, over route lists from dih_build_groups. For every expert e and route
 * r = routes[e*tokens + k], k < counts[e]:
 *   up_matrix NULL:  y[r][row] = W[e][row] . x_in(r)
 *   up_matrix set:   y[r][row] = silu(g) * u, g = W[e][row] . x_in(r), u = U[e][row] . x_in(r)
 * with x_in(r) = x[r / 8] for input_mode 1 (the token's row: gate/up) and x[r] for
 * input_mode 0 (the route's own row: down). bf16 operands (weights dequantized and rounded
 * RNE), f32 accumulation; y f32 or bf16 [tokens*8][rows], rows of routes not listed are
 * left unchanged. x bf16 [tokens or tokens*8][columns]; counts u32 [experts], routes u32
 * [experts*tokens] (device). */
int dih_grouped_qmm(void *context, void *matrix, void *up_matrix, int tokens, const void *x,
                    int input_mode, const uint32_t *counts, const uint32_t *routes, void *y,
                    int y_dtype, void *stream, char *error, int capacity);

/* Dense batched projection (p_gemv dense path, gpu_prefill.mm:603-620, prefill_bf16.mm:7-53):
 * Y[t][r] = sum_c w(0,r,c)*X[t][c]. Up to 4 tokens: a batched f32 GEMV; up to 1023 tokens
 * (511 for matrices of up to 4096 rows): the fused MFMA qmm with bf16 operands; longer
 * chunks: the matrix dequantized once into bf16 context scratch (2*R*C bytes), then the
 * library's bf16 MFMA GEMM. bf16 operands, f32 accumulation in every MFMA form. x bf16
 * [T][C]; y f32 or bf16 [T][R]. */
int dih_dense(void *context, void *matrix, int tokens, const void *x, void *y, int y_dtype,
              void *stream, char *error, int capacity);

/* Causal GQA attention of `tokens` query tokens at cache positions position ..
 * position+tokens-1, with the output gate: the BF16 prefill attention and its partition
 * combine (prefill_attention_bf16.mm:13-55, graph_attention_combine gpu_graph.mm:177-213),
 * dispatched by p_fused_attention (gpu_prefill.mm:552-570) for a prefill chunk and by
 * g_try_fused_attention (gpu_prefill.mm:579-584) for one decode token. Geometry is the
 * model's: 16 query heads over 2 KV heads, head dim 256.
 *   q       [tokens][16][256] f32 or bf16 (q_dtype): normed, rotated queries
 *   keys, values  bf16 cache [cache_positions][2][256]; rows 0..position+tokens-1 hold keys
 *           and values of this chunk and everything before it
 *   gate    [tokens][16][512] f32 or bf16: the q projection output; head h's gate values
 *           sit at h*512+256 .. h*512+511
 *   out     [tokens][16][256] f32 or bf16:
 *           softmax(q.k/16 over keys 0..position+t) . v * sigmoid(gate)
 *   partition  the rounding partition: keys 0.., partition.., 2*partition.. whose
 *           probabilities are rounded against one running maximum; a multiple of 32, 0 for
 *           the reference's default of 1024 (attentionPartitionTokens, gpu_prefill.mm:393,
 *           486-489, 554). Keys are scanned in 32-key blocks; each block's probabilities are
 *           rounded to bf16 against the running maximum of its partition through that block,
 *           as the reference rounds them. 32 makes every block its own partition, the
 *           fastest decode form. How the keys are split over the GPU is the library's choice
 *           and does not change the rounding points.
 * Device pointers; runs on `stream` (NULL: the context's stream). Returns 0, or -1 with a
 * message when an argument is invalid (nothing is launched then). */
int dih_attention(void *context, const void *q, int q_dtype, const uint16_t *keys,
                  const uint16_t *values, int cache_positions, const void *gate, int gate_dtype,
                  void *out, int out_dtype, int position, int tokens, int partition,
                  void *stream, char *error, int capacity);

/* The rounding partition dih_attention uses for these arguments (`partition` itself when
 * it is positive, else 1024); -1 for invalid arguments. */
int dih_attention_partition(int position, int tokens, int partition);

/* Gated delta rule of a linear-attention (Gated DeltaNet) layer over a chunk of `tokens`
 * tokens: p_delta (gpu_prefill.mm:540-551), i.e. the sequential prefill_delta
 * (gpu_prefill.mm:177-191) or the chunkwise prefill_delta_prepare / prefill_delta_apply
 * (prefill_delta.mm:8-181); like the reference, the library switches to the chunkwise form
 * at 64 tokens, which is also where the two cost the same on MI355X. For every token t, value
 * head h (32) and value row r (128), with key head h/2:
 *   S[h][r] *= decay[t][h];  c = (v - S[h][r].k) * beta[t][h];  S[h][r] += c k;
 *   out[t][h*128+r] = S[h][r].q
 * where the convolved row conv[t] [8192] holds q (16 x 128) at 0, k at 2048 and v
 * (32 x 128) at 4096. Then the convolution history [3][8192] rolls forward over the raw
 * projection rows raw[t] [8192] (gpu_prefill.mm:189-190).
 *   state   f32 [32][128][128], read and updated in place
 *   history f32 [3][8192], updated in place
 *   conv, raw f32 [tokens][8192]; decay, beta f32 [tokens][32]; out f32 [tokens][4096]
 *   path    0: the library's choice; 1: sequential; 2: chunkwise (any token count)
 * Device pointers; runs on `stream` (NULL: the context's stream). Returns 0, or -1 with a
 * message when an argument is invalid (nothing is launched then). */
int dih_delta_rule(void *context, float *state, float *history, const float *conv,
                   const float *decay, const float *beta, const float *raw, float *out,
                   int tokens, int path, void *stream, char *error, int capacity);

/* ---- host-pointer gated delta step (DeltaMemory) ----------------------------------- */

/* Replaces di_delta_create (quantized.mm:398-406): a device-resident recurrent state
 * f32 [32][128][128], zeroed, owned by `context`; NULL on failure. */
void *dih_delta_create(void *context);
/* Replaces di_delta_destroy (quantized.mm:407). */
void dih_delta_destroy(void *state);
/* Replaces di_delta_step (quantized.mm:408-423): one token of the gated delta rule
 * (the dih_delta_rule recurrence without the history roll) on HOST pointers, synchronous:
 *   q, k f32 [16][128] (key heads), v f32 [32][128], decay, beta f32 [32], out f32 [4096].
 * For value head h and row r (key head h/2): S *= decay[h]; c = (v[h][r] - S.k) * beta[h];
 * S += c k; out[h*128+r] = S.q. `ms` receives the GPU time of the step. Returns 0, or -1
 * with "Null delta argument" when a pointer is NULL (nothing is launched then). */
int dih_delta_step(void *context, void *state, const float *q, const float *k, const float *v,
                   const float *decay, const float *beta, float *out, double *ms, char *error,
                   int capacity);

/* Per-stage GPU timing (the reference's DEEPINFER_METAL_GPU_PROFILE per-dispatch
 * timestamps, gpu_graph.mm:329-338, as a runtime switch instead of getenv). While enabled,
 * every device-resident call records HIP events on its own stream between its kernels.
 * dih_set_profiling clears the records (and synchronizes the device if any were taken);
 * dih_profile_read waits for the last event and writes, per distinct stage name, the summed
 * milliseconds and the number of recorded launches. Returns the number of stages. */
int dih_set_profiling(void *context, int enabled);
int dih_profile_read(void *context, double *total_ms, int *counts, const char **names,
                     int capacity);

/* ---- Checkpoint loading (host code; no GPU work except the uploads of dih_checkpoint_*) ----
 * Status codes of this group: 0 ok, -1 invalid data (the reference's InvalidDataException),
 * -2 unsupported (NotSupportedException); the message text is the reference's. */

/* Safetensors reader (SafeTensors.cs:13-44): validates the header (u64 LE length in
 * [2, 16 MiB] and inside the file; dtypes BF16/F32/U32 only, else -2; rank 1..8, dims >= 1;
 * data_offsets inside the data section with end-begin = elements*dtype size; no duplicate
 * names; no overlapping ranges). `status` (optional) receives the code. */
void *dih_safetensors_open(const char *path, int *status, char *error, int capacity);
void dih_safetensors_close(void *file);
/* Number of tensors, and tensor `index` in header order: dtype 1 BF16, 2 F32, 3 U32;
 * shape[rank] (rank <= 8); byte length. */
int dih_safetensors_count(void *file);
int dih_safetensors_info(void *file, int index, char *name, int name_capacity, int *dtype,
                         int *rank, int64_t *shape, uint64_t *bytes);
/* SafeTensors.Get (SafeTensors.cs:45-50): 0 when `name` exists with exactly this shape,
 * else -1 "Missing tensor or shape mismatch: NAME." */
int dih_safetensors_get(void *file, const char *name, const int64_t *shape, int rank,
                        char *error, int capacity);
/* SafeTensors.ReadInto (SafeTensors.cs:57-63) into host memory; `bytes` must equal the
 * tensor's byte length. dtype 1 (BF16) additionally requires a BF16 tensor
 * (ReadBFloat16, SafeTensors.cs:51-56); dtype 0 accepts any. */
int dih_safetensors_read(void *file, const char *name, int dtype, void *destination,
                         uint64_t bytes, char *error, int capacity);
/* SafeTensors.ReadFloat (SafeTensors.cs:64-80): F32 as stored or BF16 widened to f32;
 * `count` must equal the element count; any non-finite value fails. */
int dih_safetensors_read_float(void *file, const char *name, float *destination,
                               uint64_t count, char *error, int capacity);

/* MLX checkpoint directory (Qwen36Weights.cs:26-65): config.json must describe the
 * Qwen3.6-35B-A3B text geometry, unscaled RoPE, affine group-64 5- or 8-bit quantization;
 * model.safetensors.index.json maps tensors to shard files (plain file names only). Shards
 * open on first use. */
void *dih_checkpoint_open(const char *directory, int *status, char *error, int capacity);
void dih_checkpoint_close(void *checkpoint);
int dih_checkpoint_info(void *checkpoint, int *bits, float *epsilon, float *rope_theta);
/* Qwen36Weights.Matrix (Qwen36Weights.cs:66-81): tensors PREFIX.weight (U32
 * [experts,] rows, columns*bits/32), PREFIX.scales and PREFIX.biases (BF16 [experts,]
 * rows, columns/64); experts == 1 means no leading expert dimension; bits 0 = the
 * checkpoint's; a per-prefix quantization override must agree. Returns a matrix handle
 * (free with dih_quant_matrix_destroy) whose device buffers hold the tensor bytes, streamed
 * through pinned staging (the reference reads into unified memory, QuantizedMetal.cs:177). */
void *dih_checkpoint_matrix(void *checkpoint, void *context, const char *prefix, int rows,
                            int columns, int experts, int bits, int *status, char *error,
                            int capacity);
/* Qwen36Weights.Vector (Qwen36Weights.cs:82): ReadFloat of a tensor of exactly `shape`. */
int dih_checkpoint_vector(void *checkpoint, const char *name, const int64_t *shape, int rank,
                          float *destination, uint64_t count, char *error, int capacity);
/* The eight MoE matrices of decoder layer `layer` (Qwen36Weights.cs:90-99): router
 * mlp.gate [256, 2048] 8-bit, mlp.switch_mlp.{gate,up}_proj [256, 512, 2048],
 * mlp.switch_mlp.down_proj [256, 2048, 512], mlp.shared_expert.{gate,up}_proj [512, 2048],
 * mlp.shared_expert.down_proj [2048, 512], mlp.shared_expert_gate [1, 2048] 8-bit. On
 * failure no matrix is left allocated. */
int dih_checkpoint_moe_layer(void *checkpoint, void *context, int layer, dih_moe_layer *out,
                             char *error, int capacity);

/* Library build string (kernels' target and version). */
const char *dih_version(void);

#ifdef __cplusplus
}
#endif
#endif
