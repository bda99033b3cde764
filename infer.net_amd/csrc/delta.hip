// Gated delta rule of the linear-attention (Gated DeltaNet) layers over a prefill chunk:
// p_delta (gpu_prefill.mm:540-551) with the sequential kernel prefill_delta
// (gpu_prefill.mm:177-191) below 64 tokens and the chunkwise pair prefill_delta_prepare /
// prefill_delta_apply (prefill_delta.mm:8-123) from 64 tokens on, plus the convolution
// history roll both end with.
//
// Geometry (fixed by the model): the convolved row [8192] holds q (16 key heads x 128) at
// 0, k at 2048, v (32 value heads x 128) at 4096; value head h reads key head h/2; state
// [32][128 value rows][128 key dims] f32; decay a and beta b [token][32]; out [token][4096].
// For every token: S *= a; S += (v - S k) b k^T; out = S q.
//
// Chunkwise form over 32-token blocks (per head; g_t = a_1..a_t within the block, d(t,j) =
// a_{j+1}..a_t as a direct product, which stays exact through zero or underflowing decays):
//   L = strict_tril(diag(b) (d o K K^T)),  T = (I + L)^-1  (column-wise forward solve)
//   W = T diag(b g) K,  U = T diag(b) V,  C = tril(d o Q K^T)
//   D = U - W S^T                      (the block's corrections, one row per token)
//   out = diag(g) Q S^T + C D,  S <- g_last S + D^T diag(g_last / g) K
// prepare forms T, W, U, C per (head, block) in parallel; apply walks the blocks in order
// with S resident in MFMA accumulators. All arithmetic is f32 (v_mfma_f32_32x32x2_f32).
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {
namespace {

constexpr int kVHeads = 32, kDim = 128, kBlk = 32, kRowLen = 8192;
constexpr int kQ = 0, kK = 2048, kV = 4096;
constexpr int kPad = kDim + 2;   // f32 row stride of [32][128] LDS tiles: two lanes halves hit disjoint banks
constexpr int kSq = kBlk + 1;    // f32 row stride of [32][32] LDS tiles

struct DeltaParams {
    const float *conv, *decay, *beta, *raw;
    float *state, *history, *out;
    float *w, *u, *causal, *factors;   // chunkwise scratch, indexed by tile = block * 32 + head
    int tokens, nblocks;
};

DIH_DEV dih_f32x16 mfma_f32(float a, float b, dih_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// history[j] <- j + tokens < 3 ? history[j + tokens] : raw[j + tokens - 3], one dim per
// thread (each thread reads its three old values before writing).
DIH_DEV void roll_history(const DeltaParams &P, int d) {
    if (d >= kRowLen) return;
    float next[3];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int at = j + P.tokens;
        next[j] = at < 3 ? P.history[at * kRowLen + d] : P.raw[(size_t)(at - 3) * kRowLen + d];
    }
#pragma unroll
    for (int j = 0; j < 3; j++) P.history[j * kRowLen + d] = next[j];
}

// ---- sequential: one wave per value row, two key dims per lane (prefill_delta).
__global__ __launch_bounds__(256) void delta_seq_kernel(DeltaParams P) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave, head = row >> 7, kh = head >> 1;
    float *srow = P.state + (size_t)row * kDim;
    float s0 = srow[lane], s1 = srow[lane + 64];
    for (int t = 0; t < P.tokens; t++) {
        const float *c = P.conv + (size_t)t * kRowLen;
        const float a = P.decay[t * kVHeads + head], b = P.beta[t * kVHeads + head];
        const float k0 = c[kK + kh * kDim + lane], k1 = c[kK + kh * kDim + lane + 64];
        const float q0 = c[kQ + kh * kDim + lane], q1 = c[kQ + kh * kDim + lane + 64];
        const float v = c[kV + row];
        s0 *= a;
        s1 *= a;
        const float pred = wave_sum(s0 * k0 + s1 * k1);
        const float corr = (v - pred) * b;
        s0 += k0 * corr;
        s1 += k1 * corr;
        const float o = wave_sum(s0 * q0 + s1 * q1);
        if (lane == 0) P.out[(size_t)t * (kVHeads * kDim) + row] = o;
    }
    srow[lane] = s0;
    srow[lane + 64] = s1;
    if (blockIdx.x < kRowLen / 256) roll_history(P, blockIdx.x * 256 + threadIdx.x);
}

// ---- chunkwise prepare: one block per (head, 32-token block), 4 waves.
__global__ __launch_bounds__(256) void delta_prepare_kernel(DeltaParams P) {
    __shared__ float ks[kBlk * kPad], qs[kBlk * kPad], vs[kBlk * kPad];
    __shared__ float kk[kBlk * kSq], qk[kBlk * kSq], lt[kBlk * kSq], ti[kBlk * kSq];
    __shared__ float a[kBlk], b[kBlk], g[kBlk];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 31, h = lane >> 5;
    const int head = blockIdx.x, blk = blockIdx.y, base = blk * kBlk, kh = head >> 1;
    const int valid = min(kBlk, P.tokens - base);
    const size_t tile = (size_t)blk * kVHeads + head;

    for (int i = tid; i < kBlk * kDim; i += 256) {
        const int t = i >> 7, d = i & (kDim - 1);
        const float *c = P.conv + (size_t)(base + t) * kRowLen;
        const bool ok = t < valid;
        ks[t * kPad + d] = ok ? c[kK + kh * kDim + d] : 0.f;
        qs[t * kPad + d] = ok ? c[kQ + kh * kDim + d] : 0.f;
        vs[t * kPad + d] = ok ? c[kV + head * kDim + d] : 0.f;
    }
    if (tid < kBlk) {
        a[tid] = tid < valid ? P.decay[(base + tid) * kVHeads + head] : 1.f;
        b[tid] = tid < valid ? P.beta[(base + tid) * kVHeads + head] : 0.f;
    }
    __syncthreads();
    if (tid < kBlk) {
        // g_t = a_0..a_t and the tail a_{t+1}..a_{valid-1}, both as direct products
        float p = 1.f, tail = 1.f;
        for (int j = 0; j <= tid; j++) p *= a[j];
        for (int j = tid + 1; j < valid; j++) tail *= a[j];
        g[tid] = p;
        P.factors[(tile * kBlk + tid) * 2] = p;
        P.factors[(tile * kBlk + tid) * 2 + 1] = tid < valid ? tail : 0.f;
    }
    // K K^T (wave 0) and Q K^T (wave 1): C[t][j] over 128 dims, 64 MFMAs each
    if (wave < 2) {
        const float *x = wave == 0 ? ks : qs;
        dih_f32x16 acc;
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = 0.f;
#pragma unroll 8
        for (int s = 0; s < kDim / 2; s++)
            acc = mfma_f32(x[r * kPad + 2 * s + h], ks[r * kPad + 2 * s + h], acc);
        float *dst = wave == 0 ? kk : qk;
#pragma unroll
        for (int i = 0; i < 16; i++) dst[(8 * (i >> 2) + 4 * h + (i & 3)) * kSq + r] = acc[i];
    }
    __syncthreads();
    // C (to global) and L (to LDS) with d(t,j) = a_{j+1}..a_t
    for (int i = tid; i < kBlk * kBlk; i += 256) {
        const int t = i >> 5, j = i & 31;
        float d = 0.f;
        if (t < valid && j <= t) {
            d = 1.f;
            for (int z = j + 1; z <= t; z++) d *= a[z];
        }
        P.causal[tile * (kBlk * kBlk) + i] = qk[t * kSq + j] * d;
        lt[t * kSq + j] = t > j ? b[t] * d * kk[t * kSq + j] : 0.f;
    }
    __syncthreads();
    // T = (I + L)^-1, lane c solving column c: T[t][c] = -(L[t][c] + sum_{c<j<t} L[t][j] T[j][c])
    if (tid < kBlk) {
        const int c = tid;
        for (int t = 0; t < kBlk; t++) ti[t * kSq + c] = t == c ? 1.f : 0.f;
        for (int t = c + 1; t < kBlk; t++) {
            float sum = lt[t * kSq + c];
            for (int j = c + 1; j < t; j++) sum += lt[t * kSq + j] * ti[j * kSq + c];
            ti[t * kSq + c] = -sum;
        }
    }
    __syncthreads();
    // W = T diag(b g) K and U = T diag(b) V: wave w forms dims 32w..32w+31 of both
    {
        dih_f32x16 wa, ua;
#pragma unroll
        for (int i = 0; i < 16; i++) { wa[i] = 0.f; ua[i] = 0.f; }
        const int dcol = 32 * wave + r;
#pragma unroll 4
        for (int s = 0; s < kBlk / 2; s++) {
            const int j = 2 * s + h;
            const float tj = ti[r * kSq + j];
            wa = mfma_f32(tj, b[j] * g[j] * ks[j * kPad + dcol], wa);
            ua = mfma_f32(tj, b[j] * vs[j * kPad + dcol], ua);
        }
        float *wt = P.w + tile * (kBlk * kDim), *ut = P.u + tile * (kBlk * kDim);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = 8 * (i >> 2) + 4 * h + (i & 3);
            wt[t * kDim + dcol] = wa[i];
            ut[t * kDim + dcol] = ua[i];
        }
    }
}

// ---- chunkwise apply: one block per (head, 32 value rows), 4 waves; wave w holds the
// state's key dims 32w..32w+31 as S^T (C[m = dim][n = value row]), so every product
// below takes the state, or the corrections D^T (same layout), as its B operand straight
// from registers: the k-pair of each MFMA is (8j + c, 8j + 4 + c), which is register
// 4j + c of both lane halves.
__global__ __launch_bounds__(256) void delta_apply_kernel(DeltaParams P) {
    __shared__ float ws[kBlk * kPad], gq[kBlk * kPad], tk[kBlk * kPad];
    __shared__ float cs[kBlk * kSq];
    __shared__ __align__(16) float part[4][2][64 * 16];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 31, h = lane >> 5;
    const int head = blockIdx.x >> 2, row0 = (blockIdx.x & 3) * 32, kh = head >> 1;
    const int d0 = 32 * wave;

    float *sbase = P.state + ((size_t)head * kDim + row0 + r) * kDim + d0;
    dih_f32x16 st;
#pragma unroll
    for (int i = 0; i < 16; i++) st[i] = sbase[8 * (i >> 2) + 4 * h + (i & 3)];

    for (int blk = 0; blk < P.nblocks; blk++) {
        const int base = blk * kBlk, valid = min(kBlk, P.tokens - base);
        const size_t tile = (size_t)blk * kVHeads + head;
        const float *fac = P.factors + tile * kBlk * 2;
        __syncthreads();   // the previous block's LDS reads are done
        for (int i = tid; i < kBlk * kDim; i += 256) {
            const int t = i >> 7, d = i & (kDim - 1);
            const float *c = P.conv + (size_t)(base + t) * kRowLen;
            const bool ok = t < valid;
            ws[t * kPad + d] = P.w[tile * (kBlk * kDim) + i];
            gq[t * kPad + d] = ok ? fac[2 * t] * c[kQ + kh * kDim + d] : 0.f;
            tk[t * kPad + d] = ok ? fac[2 * t + 1] * c[kK + kh * kDim + d] : 0.f;
        }
        for (int i = tid; i < kBlk * kBlk; i += 256) cs[(i >> 5) * kSq + (i & 31)] = P.causal[tile * (kBlk * kBlk) + i];
        __syncthreads();

        // partial (over this wave's dims) W S^T and diag(g) Q S^T: C[m = token][n = row]
        dih_f32x16 p1, p2;
#pragma unroll
        for (int i = 0; i < 16; i++) { p1[i] = 0.f; p2[i] = 0.f; }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int d = d0 + 8 * (i >> 2) + 4 * h + (i & 3);
            p1 = mfma_f32(ws[r * kPad + d], st[i], p1);
            p2 = mfma_f32(gq[r * kPad + d], st[i], p2);
        }
        float4 *mine = reinterpret_cast<float4 *>(&part[wave][0][lane * 16]);
        float4 *mine2 = reinterpret_cast<float4 *>(&part[wave][1][lane * 16]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            mine[i] = make_float4(p1[4 * i], p1[4 * i + 1], p1[4 * i + 2], p1[4 * i + 3]);
            mine2[i] = make_float4(p2[4 * i], p2[4 * i + 1], p2[4 * i + 2], p2[4 * i + 3]);
        }
        __syncthreads();
        // D^T = U^T - sum_waves(W S^T), the output's first term likewise
        const float *ut = P.u + tile * (kBlk * kDim) + row0 + r;
        dih_f32x16 dd, o;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = 8 * (i >> 2) + 4 * h + (i & 3);
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                s1 += part[w][0][lane * 16 + i];
                s2 += part[w][1][lane * 16 + i];
            }
            dd[i] = ut[t * kDim] - s1;
            o[i] = s2;
        }
        // out = diag(g) Q S^T + C D, by one wave per block in turn
        if (wave == (blk & 3)) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int k = 8 * (i >> 2) + 4 * h + (i & 3);
                o = mfma_f32(cs[r * kSq + k], dd[i], o);
            }
            float *ob = P.out + (size_t)base * (kVHeads * kDim) + head * kDim + row0 + r;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int t = 8 * (i >> 2) + 4 * h + (i & 3);
                if (t < valid) ob[(size_t)t * (kVHeads * kDim)] = o[i];
            }
        }
        // S^T <- g_last S^T + (tail o K)^T D^T
        const float glast = fac[2 * (valid - 1)];
#pragma unroll
        for (int i = 0; i < 16; i++) st[i] *= glast;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = 8 * (i >> 2) + 4 * h + (i & 3);
            st = mfma_f32(tk[t * kPad + d0 + r], dd[i], st);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) sbase[8 * (i >> 2) + 4 * h + (i & 3)] = st[i];
    if (blockIdx.x < kRowLen / 256) roll_history(P, blockIdx.x * 256 + tid);
}

}  // namespace

bool launch_delta_rule(const DeltaArgs &a, hipStream_t s, char *error, int capacity) {
    DeltaParams P;
    P.conv = a.conv; P.decay = a.decay; P.beta = a.beta; P.raw = a.raw;
    P.state = a.state; P.history = a.history; P.out = a.out;
    P.w = a.w; P.u = a.u; P.causal = a.causal; P.factors = a.factors;
    P.tokens = a.tokens;
    P.nblocks = (a.tokens + kBlk - 1) / kBlk;
    if (!a.chunked) {
        DIH_LAUNCH(delta_seq_kernel, dim3(kVHeads * kDim / 4), dim3(256), 0, s, P);
        return hip_ok(hipGetLastError(), error, capacity, "delta launch");
    }
    if (!P.w || !P.u || !P.causal || !P.factors) {
        set_error(error, capacity, "Chunkwise delta rule needs its scratch buffers");
        return false;
    }
    prof_stage("delta_prepare");
    DIH_LAUNCH(delta_prepare_kernel, dim3(kVHeads, P.nblocks), dim3(256), 0, s, P);
    if (!hip_ok(hipGetLastError(), error, capacity, "delta prepare launch")) return false;
    prof_stage("delta_apply");
    DIH_LAUNCH(delta_apply_kernel, dim3(kVHeads * 4), dim3(256), 0, s, P);
    return hip_ok(hipGetLastError(), error, capacity, "delta apply launch");
}

}  // namespace dih
