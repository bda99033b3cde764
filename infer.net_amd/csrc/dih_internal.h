// Host-side internals of libdeepinfer_hip: context and matrix objects, scratch
// management, kernel launchers shared between translation units.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/deepinfer_hip.h"

namespace dih {

struct Context;

// One MLX-affine matrix [experts, rows, columns] (QMatrix, quantized.mm:16-20).
struct Matrix {
    Context *ctx = nullptr;
    int experts = 0, rows = 0, columns = 0, bits = 0;
    void *dev[3] = {nullptr, nullptr, nullptr};   // packed, scales, biases (device)
    void *host[3] = {nullptr, nullptr, nullptr};  // pinned staging (lazy)
    bool dirty[3] = {false, false, false};
    size_t bytes[3] = {0, 0, 0};
    float *stage_in = nullptr, *stage_out = nullptr;  // f32 staging for host-pointer calls
    size_t stage_in_bytes = 0, stage_out_bytes = 0;
    // 5-bit matrices with K a multiple of 512: a second copy of the codes in 128-row
    // tile-major order, [expert][row tile][K step][row in tile][40 bytes], rows padded to
    // a multiple of 256 with zeros, read by the streaming grouped/dense GEMM (one K step of
    // a row tile is then 5,120 contiguous bytes instead of 128 40-byte pieces 1,280 bytes
    // apart). Kept equal to dev[0] by every write path (matrix_retile).
    void *tiled = nullptr;
    size_t tiled_bytes = 0;
    // the codes' device pointer has been handed out since the last dih_quant_matrix_commit:
    // every call that uses the matrix rewrites the tile-major copy first (sync_matrix)
    bool tiled_stale = false;
    uint32_t magic = 0x44494d58u;

    const uint32_t *packed() const { return static_cast<const uint32_t *>(dev[0]); }
    const uint16_t *scales() const { return static_cast<const uint16_t *>(dev[1]); }
    const uint16_t *biases() const { return static_cast<const uint16_t *>(dev[2]); }
    size_t words_per_row() const { return (size_t)columns * bits / 32; }
    size_t groups_per_row() const { return (size_t)columns / 64; }
    // per expert: whole 256-row tiles, so that the dense two-slab tiles (256 rows) read
    // padding, not past the copy
    size_t tiled_rows() const { return ((size_t)rows + 255) / 256 * 256; }
};

// Grow-only device scratch buffer.
struct Scratch {
    void *ptr = nullptr;
    size_t bytes = 0;
};

struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    // side stream of the prefill MoE step (the shared expert beside the routed experts)
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool resident = false;
    uint64_t weight_bytes = 0;
    // profiling: one start/stop event pair per kernel launch of device-resident calls,
    // aggregated per stage name when read
    bool profiling = false;
    std::vector<hipEvent_t> prof_pool;        // reused across resets
    struct ProfRec { int begin, end; const char *name; };
    std::vector<ProfRec> prof_recs;
    int prof_used = 0;                        // events taken from the pool since reset
    // named scratch
    Scratch ws[32];
    // this device's copy of the fixed scratch array of dih_moe_decode_noalloc (its device
    // address, looked up once per device), or null with the lookup's error
    void *noalloc = nullptr;
    std::string noalloc_error;
    uint32_t magic = 0x44494358u;
};

enum ScratchId {
    S_IDS, S_PROBS, S_STATUS, S_LOGITS, S_SROUTE, S_SACT, S_ACT, S_SOUT,
    S_COUNTS, S_ROUTES, S_CHUNKS, S_NCHUNKS, S_ACTBF, S_ROUTEOUT, S_ARGVAL, S_ARGIDX,
    S_STAGE_X, S_STAGE_Y, S_APART, S_ASTAT, S_DW, S_DU, S_DQ, S_DCU, S_DF, S_ASCORE, S_W16, S_COUNT_
};
static_assert(S_COUNT_ <= (int)(sizeof(Context::ws) / sizeof(Scratch)), "scratch table too small");

// Error helpers (bridge.mm:9-15 convention).
void set_error(char *error, int capacity, const std::string &message);
bool hip_ok(hipError_t e, char *error, int capacity, const char *what);
void *ctx_scratch(Context *c, ScratchId id, size_t bytes, char *error, int capacity);
bool sync_matrix(Matrix *m, char *error, int capacity);
// Rewrites the tile-major copy of flattened code rows [first, first + count) (row index
// expert * rows + row) from dev[0]; no work for matrices without one. Host-synchronous.
bool matrix_retile(Matrix *m, size_t first, size_t count, char *error, int capacity);

// Profiling. While a ProfScope for a profiling context is alive on this thread, every
// launch goes through hipExtLaunchKernelGGL with a start/stop event pair taken from the
// context's pool; the command processor stamps those events at the kernel's own start
// and end, so the recorded interval is the kernel alone (no host or queue gaps). The
// record carries the stage name set by prof_stage().
struct ProfScope {
    explicit ProfScope(Context *c);
    ~ProfScope();
};
void prof_stage(const char *name);
bool prof_events(hipEvent_t *start, hipEvent_t *stop);  // false when not profiling

// Launch with the thread's sticky HIP error cleared first, so that the hipGetLastError()
// check after the launch reports this launch only (another runtime user, e.g. the
// caller's own HIP calls, can leave an unread error behind).
template <typename... KArgs, typename... Args>
void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t s,
            Args... args) {
    (void)hipGetLastError();
    hipEvent_t a, b;
    if (prof_events(&a, &b))
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, a, b, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
}
#define DIH_LAUNCH(kernel, ...) ::dih::launch(kernel, __VA_ARGS__)

// ---- launchers (defined in the .hip translation units) ----

// Generic GEMV segment: rows of one matrix (or a gate/up pair for SwiGLU) for
// `count` slots whose expert ids come from a device array.
struct QmvSeg {
    const uint32_t *p0 = nullptr; const uint16_t *s0 = nullptr, *b0 = nullptr;
    const uint32_t *p1 = nullptr; const uint16_t *s1 = nullptr, *b1 = nullptr;  // SwiGLU up
    const uint32_t *ids = nullptr;  // device expert ids or null (expert 0)
    int rows = 0, columns = 0, count = 1;
    int experts = 1;                // ids >= experts produce NaN outputs (no fault)
    int top8 = 0;                   // 1: slot ids are the top-8 of Top8Source::logits
    const void *x = nullptr; int x_bf16 = 0; int x_slot_stride = 0;  // elements
    void *y = nullptr; int y_bf16 = 0;
};
// Launches up to 4 segments of equal bit width in one kernel. A segment flagged `top8`
// takes its 8 slot experts from the top-8 of `logits` (every wave selects them itself; the
// segment's first wave publishes ids/probs/status for later kernels).
struct Top8Source {
    const float *logits = nullptr; int experts = 0;
    uint32_t *ids = nullptr; float *probs = nullptr; uint32_t *status = nullptr;
};
bool launch_qmv(const QmvSeg *segs, int nseg, int bits, const Top8Source *top8,
                hipStream_t s, char *error, int capacity);

// Residual update and next-layer norm of the MoE steps (graph_merge_norm,
// gpu_graph.mm:48-61; prefill_merge, gpu_prefill.mm:140-150): residual += y in f32 or bf16
// storage; with norm_w, normed = r * rsqrt(mean(r^2) + eps) * norm_w of the stored r.
struct MergeOut {
    int residual_f32 = 0;
    const float *norm_w = nullptr;
    float eps = 0.f;
    void *normed = nullptr;
    int normed_f32 = 0;
};

bool launch_moe_down_merge(const Matrix *down, const float *act, const uint32_t *ids,
                           const float *probs, const float *shared_out, const float *sroute,
                           void *residual, int residual_f32, float *route_out, hipStream_t s,
                           char *error, int capacity);

// normed[t] = r[t] * rsqrt(mean(r[t]^2) + eps) * w, one block per token (the norm half of
// graph_merge_norm / prefill_add_norm, gpu_graph.mm:40-61). With `probs` (the tokens' top-8
// probabilities), a token whose probabilities are NaN (non-finite router logits, merge
// skipped) keeps its normed row.
bool launch_rmsnorm(const void *r, int r_f32, int tokens, int hidden, const float *w, float eps,
                    void *out, int out_f32, const float *probs, hipStream_t s, char *error, int capacity);

bool launch_top8(const void *logits, int logits_bf16, int tokens, int experts, uint32_t *ids,
                 float *probs, uint32_t *status, float *logits_copy, uint32_t *zero_word,
                 hipStream_t s, char *error, int capacity);

bool launch_build_groups(const uint32_t *ids, int tokens, int experts, int with_shared,
                         uint32_t *counts, uint32_t *routes, hipStream_t s, char *error, int capacity);

struct QmmArgs {
    // routed matrices (gate or down) and optional up for the gated kernel
    const Matrix *m0 = nullptr, *m1 = nullptr;
    // shared-expert matrices used for the group with index == experts
    const Matrix *sm0 = nullptr, *sm1 = nullptr;
    int tokens = 0;         // T
    int dense = 0;          // 1: identity routes over `tokens`, no groups
    const uint32_t *routes = nullptr;   // [ngroups * T] ascending route lists
    const uint32_t *counts = nullptr;   // [ngroups] device
    int ngroups = 0;                    // experts (+1 with a shared expert)
    const uint16_t *x = nullptr;        // bf16 input rows
    int in_mode = 0;                    // 0: row = route; 1: gate input row (route/8, shared)
    void *y = nullptr; int y_bf16 = 0;  // output rows indexed by route
};
bool launch_qmm(const QmmArgs &a, hipStream_t s, char *error, int capacity);
// The grouped gate/up launch of `tokens` tokens over `gate` takes the wide (96/128-route)
// 5-bit tiles: 5-bit, K a multiple of 512, more than 48 routes an expert on average.
bool qmm_wide_gated(const Matrix *gate, int tokens);

bool launch_moe_merge(const Matrix *shared_route, const uint16_t *x, int tokens, int hidden,
                      const float *route_out, const float *probs, void *residual,
                      const MergeOut &mo, hipStream_t s, char *error, int capacity);

// Decode MoE step in three launches (decode.hip). Device buffers: logits [E], sact [I],
// sroute [1], act [8*I], ids [8], probs [8], status [1] (may be null), route_out [9*H]
// (may be null).
struct DecodeLaunch {
    const Matrix *router = nullptr, *gate = nullptr, *up = nullptr, *down = nullptr;
    const Matrix *shared_gate = nullptr, *shared_up = nullptr, *shared_down = nullptr;
    const Matrix *shared_route = nullptr;
    const float *logits_in = nullptr;
    float *logits = nullptr;
    float *sact = nullptr, *sroute = nullptr, *act = nullptr;
    uint32_t *ids = nullptr;
    float *probs = nullptr;
    uint32_t *status = nullptr;
    const uint16_t *x = nullptr;
    void *residual = nullptr;
    int residual_f32 = 0;
    float *route_out = nullptr;
};
bool decode_fast_path_ok(const Matrix *router, const Matrix *gate, const Matrix *down, const Matrix *sg,
                         const Matrix *sd, const Matrix *sr);
bool launch_moe_decode(const DecodeLaunch &a, hipStream_t s, char *error, int capacity);

constexpr int kArgmaxPer = 1024;   // values per first-level argmax block (partials per call)

bool launch_argmax(const float *values, int n, float *part_val, uint32_t *part_idx,
                   uint32_t *next, hipStream_t s, char *error, int capacity);

bool launch_dequant_bf16(const Matrix *m, int expert, uint16_t *out, hipStream_t s, char *error,
                         int capacity);
bool launch_embedding(const Matrix *m, int token, float *out, hipStream_t s, char *error,
                      int capacity);

// Causal GQA attention over a bf16 KV cache (attention.hip). Geometry 16 query heads,
// 2 KV heads, head dim 256; `partition` keys per partition (a multiple of 32). With more
// than one partition, pacc [tokens*16*nparts*256] f32 and pstat [tokens*16*nparts] float2
// hold the partition results, nparts = ceil((position + tokens) / partition).
struct AttentionArgs {
    const void *q = nullptr; int q_bf16 = 0;
    const uint16_t *keys = nullptr, *values = nullptr;
    const void *gate = nullptr; int gate_bf16 = 0;
    void *out = nullptr; int out_bf16 = 0;
    float *pacc = nullptr; float *pstat = nullptr;
    float *scores = nullptr;   // decode with rounding partitions: attention_score_floats floats
    int position = 0, tokens = 0, partition = 0, round = 0;
};
// Rounding partition of a call (keys whose probabilities are rounded against one running
// maximum): `requested` when positive, else the reference's 1024.
int attention_partition(int position, int tokens, int requested);
// Work partition (keys one block scans) for that rounding partition: whole rounding
// partitions, enough of them that the blocks fill the GPU; 32 for one decode token on the
// decode kernels.
int attention_split(int position, int tokens, int round);
// Partial-result slots per (token, head) a call with that work partition writes (1: none).
int attention_partials(int position, int tokens, int partition);
// Floats of score scratch the decode scores pass needs (0: none).
size_t attention_score_floats(int position, int tokens, int round, int partition);

// Dense projection of a long chunk (gemm.hip): the matrix dequantized into bf16 scratch,
// then the library's bf16 MFMA GEMM with f32 accumulation, Y[T][R] = X[T][C] * W16[R][C]^T.
bool launch_dense_gemm(Context *c, const Matrix *m, int tokens, const uint16_t *x, void *y, bool y_bf16,
                       hipStream_t s, char *error, int capacity);
bool launch_gemm_bf16(const uint16_t *w16, int R, int C, int tokens, const uint16_t *x, void *y, bool y_bf16,
                      hipStream_t s, char *error, int capacity);
bool launch_dequant_bf16_rows(const uint32_t *packed, const uint16_t *scales, const uint16_t *biases, int bits,
                              int rows, int columns, uint16_t *out, hipStream_t s, char *error, int capacity);
bool launch_attention(const AttentionArgs &a, hipStream_t s, char *error, int capacity);

// Gated delta rule over a chunk (delta.hip): state [32][128][128] f32 and history
// [3][8192] f32 updated in place; conv/raw [tokens][8192], decay/beta [tokens][32], out
// [tokens][4096], all f32. The chunkwise path needs w, u, qp, cu
// [ceil(tokens/32)*32*32*128] and factors [ceil(tokens/32)*32*32*2] f32 scratch.
struct DeltaArgs {
    const float *conv = nullptr, *decay = nullptr, *beta = nullptr, *raw = nullptr;
    float *state = nullptr, *history = nullptr, *out = nullptr;
    float *w = nullptr, *u = nullptr, *qp = nullptr, *cu = nullptr, *factors = nullptr;
    int tokens = 0;
    int chunked = 0;
};
bool launch_delta_rule(const DeltaArgs &a, hipStream_t s, char *error, int capacity);

}  // namespace dih
