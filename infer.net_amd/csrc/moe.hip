// MoE routing, grouping, merge and argmax kernels (integer/bandwidth work, no MFMA).
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

// ------------------------------------------------------------------------------ top-8

// One wave per token (prefill_top8 gpu_prefill.mm:151-161 / SelectExperts
// Qwen36Model.cs:246-262): eight rounds of wave max with ties to the lowest expert id,
// then softmax over the eight chosen logits (largest subtracted, summed in slot order).
// A non-finite logit sets *status = 1, the token's ids to 0 and its probabilities to NaN: the
// merge then leaves that token's residual (and normed row) unchanged, where the reference's
// host path throws before writing (SelectExperts, Qwen36Model.cs:252).
__global__ __launch_bounds__(256) void top8_kernel(const void *logits, int logits_bf16, int tokens,
                                                   int experts, uint32_t *ids, float *probs,
                                                   uint32_t *status, float *logits_copy,
                                                   uint32_t *zero_word) {
    if (zero_word && blockIdx.x == 0 && threadIdx.x == 0) *zero_word = 0u;
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= tokens) return;
    float cand[4];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        float v = -INFINITY;
        if (e < experts) {
            const size_t at = (size_t)t * experts + e;
            v = logits_bf16 ? bf16_to_f32(static_cast<const uint16_t *>(logits)[at])
                            : static_cast<const float *>(logits)[at];
            if (!isfinite(v)) bad = true;
            if (logits_copy) logits_copy[at] = v;
        }
        cand[j] = v;
    }
    const bool any_bad = __any(bad);
    float chosen[8];
    uint32_t picked[8];
#pragma unroll
    for (int n = 0; n < 8; n++) {
        float best = cand[0];
        uint32_t id = (uint32_t)lane;
#pragma unroll
        for (int j = 1; j < 4; j++)
            if (cand[j] > best) { best = cand[j]; id = (uint32_t)(lane + 64 * j); }
        const float m = wave_max(best);
        const uint32_t sel = wave_min_u32(best == m ? id : 0xffffffffu);
        chosen[n] = m;
        picked[n] = sel;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if ((uint32_t)(lane + 64 * j) == sel) cand[j] = -INFINITY;
    }
    if (lane == 0) {
        float p[8], total = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) { p[i] = __expf(chosen[i] - chosen[0]); total += p[i]; }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            ids[(size_t)t * 8 + i] = any_bad ? 0u : picked[i];
            probs[(size_t)t * 8 + i] = any_bad ? __builtin_nanf("") : p[i] / total;
        }
        if (any_bad && status) *status = 1u;
    }
}

bool launch_top8(const void *logits, int logits_bf16, int tokens, int experts, uint32_t *ids,
                 float *probs, uint32_t *status, float *logits_copy, uint32_t *zero_word,
                 hipStream_t s, char *error, int capacity) {
    DIH_LAUNCH(top8_kernel, dim3((tokens + 3) / 4), dim3(256), 0, s, logits, logits_bf16,
                       tokens, experts, ids, probs, status, logits_copy, zero_word);
    return hip_ok(hipGetLastError(), error, capacity, "top8 launch");
}

// ------------------------------------------------------------------------- grouping

// Block e lists the routes r (= token*8 + slot) with ids[r] == e in ascending order
// (prefill_build_groups prefill_moe.mm:8-17 uses a SIMD prefix sum per 32 routes). Here a
// thread takes 64 consecutive routes a pass (16 K routes per pass of 256 threads, all its
// loads issued together), counts its matches and places them after an add-scan of the
// block's counts: one barrier per pass. Block `experts` (when with_shared) lists the
// shared expert's routes T*8 + t for every token. Blocks do not communicate: the GEMM
// derives its chunks from the counts (in expert order, so the order is deterministic where
// the reference's atomic tile append, prefill_moe.mm:15, is not).
__global__ __launch_bounds__(256) void group_kernel(const uint32_t *ids, int tokens, int experts,
                                                    int with_shared, uint32_t *counts,
                                                    uint32_t *routes) {
    constexpr int kPer = 64;   // routes per thread and pass
    __shared__ uint32_t wave_tot[2][4];
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int T8 = tokens * 8;
    uint32_t *out = routes + (size_t)e * tokens;
    if (e == experts) {
        for (int t = tid; t < tokens; t += 256) out[t] = (uint32_t)(T8 + t);
        if (tid == 0) counts[e] = (uint32_t)tokens;
        return;
    }
    uint32_t total = 0;
    int buf = 0;
    for (int base = 0; base < T8; base += 256 * kPer, buf ^= 1) {
        const int r0 = base + kPer * tid;
        // 16-byte loads at clamped offsets (T8 is a multiple of 8), masked past the routes
        uint4 v[kPer / 4];
#pragma unroll
        for (int k4 = 0; k4 < kPer / 4; k4++)
            v[k4] = *reinterpret_cast<const uint4 *>(ids + min(r0 + 4 * k4, T8 - 4));
        uint64_t hit = 0;
#pragma unroll
        for (int k4 = 0; k4 < kPer / 4; k4++) {
            if (r0 + 4 * k4 >= T8) continue;
            const uint64_t h = (uint64_t)(v[k4].x == (uint32_t)e) | (uint64_t)(v[k4].y == (uint32_t)e) << 1 |
                               (uint64_t)(v[k4].z == (uint32_t)e) << 2 | (uint64_t)(v[k4].w == (uint32_t)e) << 3;
            hit |= h << (4 * k4);
        }
        const uint32_t cnt = (uint32_t)__popcll(hit);
        uint32_t incl = cnt;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t y = __shfl_up(incl, d, 64);
            if (lane >= d) incl += y;
        }
        if (lane == 63) wave_tot[buf][wave] = incl;
        __syncthreads();
        uint32_t off = total + incl - cnt;
        for (int w = 0; w < wave; w++) off += wave_tot[buf][w];
        // A token lists an expert at most once, so count <= tokens; ids that repeat an
        // expert within a token are truncated here instead of overrunning the list.
        while (hit) {
            const int k = __builtin_ctzll(hit);
            hit &= hit - 1;
            if (off < (uint32_t)tokens) out[off] = (uint32_t)(r0 + k);
            off++;
        }
        total += wave_tot[buf][0] + wave_tot[buf][1] + wave_tot[buf][2] + wave_tot[buf][3];
    }
    if (tid == 0) counts[e] = min(total, (uint32_t)tokens);
}

bool launch_build_groups(const uint32_t *ids, int tokens, int experts, int with_shared,
                         uint32_t *counts, uint32_t *routes, hipStream_t s, char *error, int capacity) {
    DIH_LAUNCH(group_kernel, dim3(experts + with_shared), dim3(256), 0, s, ids, tokens, experts,
               with_shared, counts, routes);
    return hip_ok(hipGetLastError(), error, capacity, "grouping launch");
}

// ---------------------------------------------------------------------------- merge

// One block per token (prefill_merge gpu_prefill.mm:140-150): gate = sigmoid(shared_route .
// x[t]); y = gate*out[T*8+t] + sum_{slot 0..7} p*out[t*8+slot]; residual[t] += y (f32 or
// bf16 storage); with norm_w, normed[t] = r * rsqrt(mean(r^2) + eps) * norm_w over the
// stored r (each thread re-reads only the elements it wrote).
template <int BITS>
__global__ __launch_bounds__(256) void merge_kernel(const uint32_t *sr_packed,
                                                    const uint16_t *sr_scales,
                                                    const uint16_t *sr_biases,
                                                    const uint16_t *x, int tokens, int H,
                                                    const float *route_out, const float *probs,
                                                    void *residual, MergeOut mo) {
    __shared__ float part[4];
    __shared__ float sq[4];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nchunk = H >> 5;
    float d = 0.f;
    for (int ch = tid; ch < nchunk; ch += 256) {
        Chunk<BITS> c;
        load_chunk<BITS>(c, sr_packed, ch);
        float xr[32];
        load_x32(xr, x + (size_t)t * H, 1, ch * 32);
        float xs = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) xs += xr[i];
        d += bf16_to_f32(sr_scales[ch >> 1]) * chunk_dot<BITS>(c, xr) + bf16_to_f32(sr_biases[ch >> 1]) * xs;
    }
    d = wave_sum(d);
    if (lane == 0) part[wave] = d;
    __syncthreads();
    const float gate = sigmoidf_((part[0] + part[1]) + (part[2] + part[3]));
    float p[8];
#pragma unroll
    for (int s = 0; s < 8; s++) p[s] = probs[(size_t)t * 8 + s];
    // a token whose router logits were not finite (NaN probabilities) keeps its residual
    // and normed row unchanged (uniform over the block: one token)
    if (__builtin_isnan(p[0])) return;
    const float *sh = route_out + ((size_t)tokens * 8 + t) * H;
    const float *ro = route_out + (size_t)t * 8 * H;
    float ss = 0.f;
    for (int c = tid; c < H; c += 256) {
        float y = sh[c] * gate;
#pragma unroll
        for (int s = 0; s < 8; s++) y += ro[(size_t)s * H + c] * p[s];
        const size_t at = (size_t)t * H + c;
        const float r = residual_store(residual, mo.residual_f32, at, residual_load(residual, mo.residual_f32, at) + y);
        ss += r * r;
    }
    if (!mo.norm_w) return;  // uniform over the launch
    ss = wave_sum(ss);
    if (lane == 0) sq[wave] = ss;
    __syncthreads();
    const float scale = rsqrtf(((sq[0] + sq[1]) + (sq[2] + sq[3])) / (float)H + mo.eps);
    for (int c = tid; c < H; c += 256) {
        const size_t at = (size_t)t * H + c;
        const float v = residual_load(residual, mo.residual_f32, at) * scale * mo.norm_w[c];
        if (mo.normed_f32) static_cast<float *>(mo.normed)[at] = v;
        else static_cast<uint16_t *>(mo.normed)[at] = f32_to_bf16(v);
    }
}

bool launch_moe_merge(const Matrix *shared_route, const uint16_t *x, int tokens, int hidden,
                      const float *route_out, const float *probs, void *residual,
                      const MergeOut &mo, hipStream_t s, char *error, int capacity) {
    if (shared_route->bits == 8)
        DIH_LAUNCH((merge_kernel<8>), dim3(tokens), dim3(256), 0, s, shared_route->packed(),
                           shared_route->scales(), shared_route->biases(), x, tokens, hidden, route_out,
                           probs, residual, mo);
    else
        DIH_LAUNCH((merge_kernel<5>), dim3(tokens), dim3(256), 0, s, shared_route->packed(),
                           shared_route->scales(), shared_route->biases(), x, tokens, hidden, route_out,
                           probs, residual, mo);
    return hip_ok(hipGetLastError(), error, capacity, "merge launch");
}

// ---------------------------------------------------------------------------- norm

// One block per token: normed[t] = r[t] * rsqrt(sum(r[t]^2)/H + eps) * w (the norm of
// graph_merge_norm / prefill_add_norm, gpu_graph.mm:40-61).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void *r, int r_f32, int H, const float *w,
                                                      float eps, void *out, int out_f32, const float *probs) {
    __shared__ float sq[4];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the token's merge was skipped (non-finite router logits): its normed row stays as it was
    if (probs && __builtin_isnan(probs[(size_t)t * 8])) return;
    float ss = 0.f;
    for (int c = tid; c < H; c += 256) {
        const float v = residual_load(r, r_f32, (size_t)t * H + c);
        ss += v * v;
    }
    ss = wave_sum(ss);
    if (lane == 0) sq[wave] = ss;
    __syncthreads();
    const float scale = rsqrtf(((sq[0] + sq[1]) + (sq[2] + sq[3])) / (float)H + eps);
    for (int c = tid; c < H; c += 256) {
        const size_t at = (size_t)t * H + c;
        const float v = residual_load(r, r_f32, at) * scale * w[c];
        if (out_f32) static_cast<float *>(out)[at] = v;
        else static_cast<uint16_t *>(out)[at] = f32_to_bf16(v);
    }
}

bool launch_rmsnorm(const void *r, int r_f32, int tokens, int hidden, const float *w, float eps,
                    void *out, int out_f32, const float *probs, hipStream_t s, char *error, int capacity) {
    DIH_LAUNCH(rmsnorm_kernel, dim3(tokens), dim3(256), 0, s, r, r_f32, hidden, w, eps, out, out_f32, probs);
    return hip_ok(hipGetLastError(), error, capacity, "norm launch");
}

// --------------------------------------------------------------------------- argmax

// Two levels, two launches (graph_argmax_blocks/final gpu_graph.mm:160-175): each block of
// the first reduces 1024 values to (max, lowest index), flagging non-finite values (one
// 16-byte load a thread, so the pass is one memory round trip over 243 blocks for the
// 248,320 logits; 4096 values a block, 61 blocks, took 5.6 us); one block of the second
// reduces the partials. Result 0xffffffff when any value is not finite. (One
// launch with a last-block ticket measured 10.7-12 us: the ticket's release fence and
// device-scope atomic from every block cost more than the second launch.)

// (max, lowest index) of a block's candidates; pairs whose index is 0xfffffffe mark a
// non-finite value, and 0xffffffff marks "no candidate". Thread 0 gets the result.
DIH_DEV void argmax_block(float best, uint32_t id, bool bad, float *wv, uint32_t *wi,
                          float &bm, uint32_t &bi) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool any_bad_w = __any(bad);
    const float m = wave_max(best);
    const uint32_t sel = wave_min_u32(best == m ? id : 0xffffffffu);
    if (lane == 0) { wv[wave] = m; wi[wave] = any_bad_w ? 0xfffffffeu : sel; }
    __syncthreads();
    bm = -INFINITY;
    bi = 0xffffffffu;
    if (tid == 0) {
        bool invalid = false;
        for (int w = 0; w < 4; w++) {
            if (wi[w] == 0xfffffffeu) { invalid = true; continue; }
            if (wi[w] != 0xffffffffu && (wv[w] > bm || (wv[w] == bm && wi[w] < bi))) { bm = wv[w]; bi = wi[w]; }
        }
        if (invalid) bi = 0xfffffffeu;
    }
}

__global__ __launch_bounds__(256) void argmax_blocks_kernel(const float *v, int n, float *pval,
                                                            uint32_t *pidx) {
    __shared__ float wv[4];
    __shared__ uint32_t wi[4];
    const int tid = threadIdx.x;
    const int base = blockIdx.x * kArgmaxPer;
    float x[4];
    // a coalesced 16-byte load a thread when the block is whole and aligned, else scalar
    if (base + kArgmaxPer <= n && (reinterpret_cast<uintptr_t>(v) & 15) == 0) {
        const float4 q = *reinterpret_cast<const float4 *>(v + base + 4 * tid);
        x[0] = q.x; x[1] = q.y; x[2] = q.z; x[3] = q.w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int at = base + 4 * tid + k;
            x[k] = at < n ? v[at] : -INFINITY;
        }
    }
    float best = -INFINITY;
    uint32_t id = 0xffffffffu;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int at = base + 4 * tid + k;
        if (at < n) {
            if (!isfinite(x[k])) bad = true;
            else if (x[k] > best || (x[k] == best && (uint32_t)at < id)) { best = x[k]; id = (uint32_t)at; }
        }
    }
    float bm;
    uint32_t bi;
    argmax_block(best, id, bad, wv, wi, bm, bi);
    if (tid == 0) { pval[blockIdx.x] = bm; pidx[blockIdx.x] = bi; }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float *pval, const uint32_t *pidx,
                                                           int nparts, uint32_t *next) {
    __shared__ float wv[4];
    __shared__ uint32_t wi[4];
    float best = -INFINITY;
    uint32_t id = 0xffffffffu;
    bool bad = false;
    for (int k = threadIdx.x; k < nparts; k += 256) {
        const uint32_t pi = pidx[k];
        const float pv = pval[k];
        if (pi == 0xfffffffeu) bad = true;
        else if (pi != 0xffffffffu && (pv > best || (pv == best && pi < id))) { best = pv; id = pi; }
    }
    float bm;
    uint32_t bi;
    argmax_block(best, id, bad, wv, wi, bm, bi);
    if (threadIdx.x == 0) *next = bi == 0xfffffffeu ? 0xffffffffu : bi;
}

bool launch_argmax(const float *values, int n, float *part_val, uint32_t *part_idx,
                   uint32_t *next, hipStream_t s, char *error, int capacity) {
    static_assert(kArgmaxPer == 4 * 256, "4 values a thread");
    const int blocks = (n + kArgmaxPer - 1) / kArgmaxPer;
    DIH_LAUNCH(argmax_blocks_kernel, dim3(blocks), dim3(256), 0, s, values, n, part_val, part_idx);
    if (!hip_ok(hipGetLastError(), error, capacity, "argmax launch")) return false;
    DIH_LAUNCH(argmax_final_kernel, dim3(1), dim3(256), 0, s, part_val, part_idx, blocks, next);
    return hip_ok(hipGetLastError(), error, capacity, "argmax launch");
}

}  // namespace dih
