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
// prepare forms, per (head, block) in parallel, everything that does not involve S:
//   W~ = diag(tail) W,  U~ = diag(tail) U   (tail = g_last / g, zero past the chunk)
//   Q' = diag(g) Q - C W,  CU = C U
// so that apply, walking the blocks in order with S resident in MFMA accumulators, only
// forms D~ = U~ - W~ S^T = diag(tail) D,  out = Q' S^T + CU,  S <- g_last S + D~^T K.
// All arithmetic is f32 (v_mfma_f32_32x32x2_f32 in prepare, 16x16x4 in apply).
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {
namespace {

constexpr int kVHeads = 32, kDim = 128, kBlk = 32, kRowLen = 8192;
constexpr int kQ = 0, kK = 2048, kV = 4096;

struct DeltaParams {
    const float *conv, *decay, *beta, *raw;
    float *state, *history, *out;
    float *w, *u, *qp, *cu, *factors;   // chunkwise scratch, indexed by tile = block * 32 + head
    int tokens, nblocks;
};

// (native vectors, not HIP's float4: copies of that struct go through memory, and such a
// copy live across the loop is promoted to LDS)
typedef dih_f32x4 f4;

DIH_DEV f4 ld4(const float *p) { return *reinterpret_cast<const f4 *>(p); }
DIH_DEV void st4(float *p, f4 v) { *reinterpret_cast<f4 *>(p) = v; }

DIH_DEV f4 mask4(f4 v, bool keep) {
    const f4 z = {0.f, 0.f, 0.f, 0.f};
    return keep ? v : z;
}

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

// ---- sequential (prefill_delta): 16 lanes per value row, eight key dims per lane, a block
// of four waves = 16 rows of one head. Token operands (keys and queries of the head's key
// head, the block's 16 values, decay, beta) are staged through LDS 32 tokens at a time,
// double-buffered: the next 32 tokens' global loads are in flight while the current ones
// run, and each token's operands are read from LDS one token ahead.
constexpr int kSeqChunk = 32;

struct SeqStage {
    float k[kSeqChunk * kDim], q[kSeqChunk * kDim], v[kSeqChunk * 16], a[kSeqChunk], b[kSeqChunk];
};

struct SeqRegs {
    float4 k0, k1, k2, k3, q0, q1, q2, q3;
    float v0, v1, ab;
};

// Thread t loads float4 j of keys / queries at flat index 4*(t + 256 j) of the chunk's
// [32][128], values (token, row) = (t + 256 j) / 16, % 16, and decay (t < 32) or beta
// (32 <= t < 64) of token t % 32. Tokens past the chunk end load token `last`.
DIH_DEV float4 seq_row4(const DeltaParams &P, int t0, int last, int j, int tid, int off) {
    const int i = 4 * (tid + 256 * j), t = min(t0 + (i >> 7), last), d = i & (kDim - 1);
    return *reinterpret_cast<const float4 *>(P.conv + (size_t)t * kRowLen + off + d);
}

DIH_DEV void seq_load(SeqRegs &g, const DeltaParams &P, int t0, int head, int kh, int row0, int tid) {
    const int last = P.tokens - 1;
    g.k0 = seq_row4(P, t0, last, 0, tid, kK + kh * kDim);
    g.k1 = seq_row4(P, t0, last, 1, tid, kK + kh * kDim);
    g.k2 = seq_row4(P, t0, last, 2, tid, kK + kh * kDim);
    g.k3 = seq_row4(P, t0, last, 3, tid, kK + kh * kDim);
    g.q0 = seq_row4(P, t0, last, 0, tid, kQ + kh * kDim);
    g.q1 = seq_row4(P, t0, last, 1, tid, kQ + kh * kDim);
    g.q2 = seq_row4(P, t0, last, 2, tid, kQ + kh * kDim);
    g.q3 = seq_row4(P, t0, last, 3, tid, kQ + kh * kDim);
    const float *vrow = P.conv + kV + head * kDim + row0 + (tid & 15);
    g.v0 = vrow[(size_t)min(t0 + (tid >> 4), last) * kRowLen];
    g.v1 = vrow[(size_t)min(t0 + ((tid + 256) >> 4), last) * kRowLen];
    const int t = min(t0 + (tid & 31), last);
    g.ab = (tid < 32 ? P.decay : P.beta)[t * kVHeads + head];   // used by threads 0..63 only
}

DIH_DEV void seq_store(const SeqRegs &g, SeqStage &st, int tid) {
    float4 *k = reinterpret_cast<float4 *>(st.k) + tid, *q = reinterpret_cast<float4 *>(st.q) + tid;
    k[0] = g.k0; k[256] = g.k1; k[512] = g.k2; k[768] = g.k3;
    q[0] = g.q0; q[256] = g.q1; q[512] = g.q2; q[768] = g.q3;
    st.v[tid] = g.v0;
    st.v[tid + 256] = g.v1;
    if (tid < 32) st.a[tid] = g.ab;
    else if (tid < 64) st.b[tid - 32] = g.ab;
}

struct TokenOps {
    float4 k0, k1, q0, q1;
    float a, b, v;
};

DIH_DEV void read_token(TokenOps &o, const SeqStage &st, int t, int sub, int rsub) {
    const float4 *kp = reinterpret_cast<const float4 *>(&st.k[t * kDim + 8 * sub]);
    const float4 *qp = reinterpret_cast<const float4 *>(&st.q[t * kDim + 8 * sub]);
    o.k0 = kp[0]; o.k1 = kp[1];
    o.q0 = qp[0]; o.q1 = qp[1];
    o.a = st.a[t];
    o.b = st.b[t];
    o.v = st.v[t * 16 + rsub];
}

DIH_DEV float dot8(const float (&s)[8], float4 x0, float4 x1) {
    return (s[0] * x0.x + s[1] * x0.y + s[2] * x0.z + s[3] * x0.w) +
           (s[4] * x1.x + s[5] * x1.y + s[6] * x1.z + s[7] * x1.w);
}

__global__ __launch_bounds__(256) void delta_seq_kernel(DeltaParams P) {
    __shared__ __align__(16) SeqStage stage[2];
    const int tid = threadIdx.x, lane = tid & 63, sub = lane & 15, rsub = tid >> 4;
    const int row0 = blockIdx.x * 16, row = row0 + rsub, head = row >> 7, kh = head >> 1;
    const int hrow0 = row0 & (kDim - 1);
    float4 *srow = reinterpret_cast<float4 *>(P.state + (size_t)row * kDim + 8 * sub);
    float s[8];
    {
        const float4 a0 = srow[0], a1 = srow[1];
        s[0] = a0.x; s[1] = a0.y; s[2] = a0.z; s[3] = a0.w; s[4] = a1.x; s[5] = a1.y; s[6] = a1.z; s[7] = a1.w;
    }
    SeqRegs g;
    seq_load(g, P, 0, head, kh, hrow0, tid);
    seq_store(g, stage[0], tid);
    __syncthreads();
    for (int t0 = 0, buf = 0; t0 < P.tokens; t0 += kSeqChunk, buf ^= 1) {
        const bool more = t0 + kSeqChunk < P.tokens;
        if (more) seq_load(g, P, t0 + kSeqChunk, head, kh, hrow0, tid);
        const SeqStage &st = stage[buf];
        const int n = min(kSeqChunk, P.tokens - t0);
        TokenOps cur, nxt;
        read_token(cur, st, 0, sub, rsub);
        for (int t = 0; t < n; t++) {
            if (t + 1 < n) read_token(nxt, st, t + 1, sub, rsub);
#pragma unroll
            for (int i = 0; i < 8; i++) s[i] *= cur.a;
            const float pred = group_sum(dot8(s, cur.k0, cur.k1), 16);
            const float corr = (cur.v - pred) * cur.b;
            const float kv[8] = {cur.k0.x, cur.k0.y, cur.k0.z, cur.k0.w, cur.k1.x, cur.k1.y, cur.k1.z, cur.k1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) s[i] += kv[i] * corr;
            const float o = group_sum(dot8(s, cur.q0, cur.q1), 16);
            if (sub == 0) P.out[(size_t)(t0 + t) * (kVHeads * kDim) + row] = o;
            cur = nxt;
        }
        if (more) seq_store(g, stage[buf ^ 1], tid);   // the other buffer's readers finished a chunk ago
        __syncthreads();
    }
    srow[0] = make_float4(s[0], s[1], s[2], s[3]);
    srow[1] = make_float4(s[4], s[5], s[6], s[7]);
    if (blockIdx.x < kRowLen / 256) roll_history(P, blockIdx.x * 256 + tid);
}

// ---- chunkwise prepare: one block per (head, 32-token block), 4 waves.
constexpr int kApplyRows = 16;   // value rows per apply block
constexpr int kPad4 = kDim + 4;   // f32 row stride of [32][128] tiles: 16-byte rows, conflict-free 128-bit reads
constexpr int kSq4 = kBlk + 4;    // f32 row stride of [32][32] and [128][32] tiles, same property

DIH_DEV void load_rows4(float *dst, const float *src_row0, int tid, int valid, int off) {
    // [32][128] rows from the convolved rows (stride kRowLen) at column `off`; zero past `valid`
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i4 = tid + 256 * j, t = i4 >> 5, d = 4 * (i4 & 31);
        // load the clamped row unconditionally and mask the value (a conditional load
        // becomes a load through a selected pointer)
        st4(dst + t * kPad4 + d, mask4(ld4(src_row0 + (size_t)min(t, valid - 1) * kRowLen + off + d), t < valid));
    }
}

__global__ __launch_bounds__(256) void delta_prepare_kernel(DeltaParams P) {
    __shared__ __align__(16) float ks[kBlk * kPad4], qs[kBlk * kPad4], vs[kBlk * kPad4];
    // K K^T and Q K^T, each as two partial sums over the halves of the key dims; then C over
    // the first Q K^T half, L over the first K K^T half, T over the second K K^T half
    __shared__ __align__(16) float kkp[2][kBlk * kSq4], qkp[2][kBlk * kSq4];
    __shared__ __align__(16) float a[kBlk], b[kBlk], bg[kBlk], gs[kBlk], tl[kBlk];
    float *const cs = qkp[0], *const lt = kkp[0], *const ti = kkp[1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 31, h = lane >> 5;
    const int head = blockIdx.x, blk = blockIdx.y, base = blk * kBlk, kh = head >> 1;
    const int valid = min(kBlk, P.tokens - base);
    const size_t tile = (size_t)blk * kVHeads + head;
    const float *rows = P.conv + (size_t)base * kRowLen;

    load_rows4(ks, rows, tid, valid, kK + kh * kDim);
    load_rows4(qs, rows, tid, valid, kQ + kh * kDim);
    load_rows4(vs, rows, tid, valid, kV + head * kDim);
    if (tid < kBlk) {
        a[tid] = tid < valid ? P.decay[(base + tid) * kVHeads + head] : 1.f;
        b[tid] = tid < valid ? P.beta[(base + tid) * kVHeads + head] : 0.f;
    }
    __syncthreads();
    // waves 0, 1: K K^T over dims [0, 64) and [64, 128); waves 2, 3: Q K^T likewise. MFMA
    // (m, e) pairs dims (64hh + 4m + e, 64hh + 32 + 4m + e), lane half h taking the second,
    // on two accumulator chains
    {
        const int hh = wave & 1;
        const float *x = wave < 2 ? ks : qs;
        dih_f32x16 acc0, acc1;
#pragma unroll
        for (int i = 0; i < 16; i++) { acc0[i] = 0.f; acc1[i] = 0.f; }
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const int d = 64 * hh + 32 * h + 4 * m;
            const f4 xa = ld4(x + r * kPad4 + d), ka = ld4(ks + r * kPad4 + d);
            acc0 = mfma_f32(xa[0], ka[0], acc0);
            acc1 = mfma_f32(xa[1], ka[1], acc1);
            acc0 = mfma_f32(xa[2], ka[2], acc0);
            acc1 = mfma_f32(xa[3], ka[3], acc1);
        }
        float *dst = (wave < 2 ? kkp : qkp)[hh];
#pragma unroll
        for (int i = 0; i < 16; i++) dst[(8 * (i >> 2) + 4 * h + (i & 3)) * kSq4 + r] = acc0[i] + acc1[i];
    }
    __syncthreads();
    // C and L, thread (j = column, rows 4q..4q+3); d(t,j) = a_{j+1}..a_t as a direct
    // product, the decays held in registers
    {
        float ar[kBlk];
#pragma unroll
        for (int k4 = 0; k4 < kBlk / 4; k4++) {
            const f4 v = ld4(a + 4 * k4);
            ar[4 * k4] = v[0]; ar[4 * k4 + 1] = v[1]; ar[4 * k4 + 2] = v[2]; ar[4 * k4 + 3] = v[3];
        }
        const int j = tid & 31, t0 = 4 * (tid >> 5);
        float d = 1.f;
#pragma unroll
        for (int k = 1; k < kBlk; k++) d *= k > j && k <= t0 ? ar[k] : 1.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + i;
            if (i > 0 && t > j) d *= a[t];
            const float dd = t < valid && j <= t ? d : 0.f;
            const int at = t * kSq4 + j;
            cs[at] = (qkp[0][at] + qkp[1][at]) * dd;
            lt[at] = t > j ? b[t] * dd * (kkp[0][at] + kkp[1][at]) : 0.f;
        }
        // g_t = a_0..a_t and the tail a_{t+1}..a_{valid-1}, both as direct products (no
        // quotients), by prefix and suffix product scans over lanes 0..31
        if (tid < kBlk) {
            const int t = tid;
            float p = a[t], sfx = t < valid ? a[t] : 1.f;
#pragma unroll
            for (int d = 1; d < kBlk; d <<= 1) {
                const float up = __shfl_up(p, d, kBlk), down = __shfl_down(sfx, d, kBlk);
                if (t >= d) p *= up;
                if (t + d < kBlk) sfx *= down;
            }
            float tail = __shfl_down(sfx, 1, kBlk);
            if (t == kBlk - 1) tail = 1.f;
            bg[t] = b[t] * p;
            gs[t] = p;
            tl[t] = t < valid ? tail : 0.f;
            P.factors[(tile * kBlk + t) * 2] = p;
            P.factors[(tile * kBlk + t) * 2 + 1] = t < valid ? tail : 0.f;
        }
    }
    __syncthreads();
    // T = (I + L)^-1 by 16x16 blocks, on wave 0: lanes 0..15 and 16..31 invert the diagonal
    // blocks column by column (x[t] = [t == c] for t <= c, x[t] = -sum_{j<t} L[t][j] x[j]
    // after; x[j] = 0 for j < c, so the full sums are exact), then T21 = -T22 (L21 T11) on
    // 16x16x4 MFMAs
    if (wave == 0) {
        if (lane < 32) {
            const int o = 16 * (lane >> 4), c = lane & 15;
            float x[16];
#pragma unroll
            for (int t = 0; t < 16; t++) {
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int j4 = 0; j4 < t; j4 += 4) {
                    const f4 l4 = ld4(lt + (o + t) * kSq4 + o + j4);
                    s0 += l4[0] * x[j4];
                    if (j4 + 1 < t) s1 += l4[1] * x[j4 + 1];
                    if (j4 + 2 < t) s0 += l4[2] * x[j4 + 2];
                    if (j4 + 3 < t) s1 += l4[3] * x[j4 + 3];
                }
                x[t] = t < c ? 0.f : t == c ? 1.f : -(s0 + s1);
            }
#pragma unroll
            for (int t = 0; t < 16; t++) {
                ti[(o + t) * kSq4 + o + c] = x[t];
                ti[(o == 0 ? t : t + 16) * kSq4 + (o == 0 ? 16 + c : c)] = 0.f;   // T12 = 0; T21 below
            }
        }
        wait_lgkm0();
        // step s covers k = 4g + s (lane group g = lane / 16), so the product M = L21 T11 in
        // its accumulator layout (register s: row 4g + s) is the B operand of the next
        const int n = lane & 15, g = lane >> 4;
        f4 m = {0.f, 0.f, 0.f, 0.f}, t21 = m;
#pragma unroll
        for (int s = 0; s < 4; s++)
            m = __builtin_amdgcn_mfma_f32_16x16x4f32(lt[(16 + n) * kSq4 + 4 * g + s], ti[(4 * g + s) * kSq4 + n], m,
                                                     0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; s++)
            t21 = __builtin_amdgcn_mfma_f32_16x16x4f32(ti[(16 + n) * kSq4 + 16 + 4 * g + s], m[s], t21, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) ti[(16 + 4 * g + i) * kSq4 + n] = -t21[i];
    }
    __syncthreads();
    // W = T diag(b g) K and U = T diag(b) V: wave w forms dims 32w..32w+31 of both; MFMA s
    // pairs tokens (s, 16 + s)
    {
        dih_f32x16 wa, ua;
#pragma unroll
        for (int i = 0; i < 16; i++) { wa[i] = 0.f; ua[i] = 0.f; }
        const int dcol = 32 * wave + r;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const f4 t4 = ld4(ti + r * kSq4 + 16 * h + 4 * m);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int j = 16 * h + 4 * m + e;
                wa = mfma_f32(t4[e], bg[j] * ks[j * kPad4 + dcol], wa);
                ua = mfma_f32(t4[e], b[j] * vs[j * kPad4 + dcol], ua);
            }
        }
        // C W and C U: MFMA (j, e) pairs tokens (8j + e, 8j + 4 + e), which is register
        // 4j + e of W and U in both lane halves
        dih_f32x16 cw, cu;
#pragma unroll
        for (int i = 0; i < 16; i++) { cw[i] = 0.f; cu[i] = 0.f; }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f4 ca = ld4(cs + r * kSq4 + 8 * j + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                cw = mfma_f32(ca[e], wa[4 * j + e], cw);
                cu = mfma_f32(ca[e], ua[4 * j + e], cu);
            }
        }
        float *wt = P.w + tile * (kBlk * kDim), *qt = P.qp + tile * (kBlk * kDim);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = 8 * (i >> 2) + 4 * h + (i & 3);
            wt[t * kDim + dcol] = tl[t] * wa[i];
            qt[t * kDim + dcol] = gs[t] * qs[t * kPad4 + dcol] - cw[i];
        }
        // U~ and C U in the apply blocks' layout (value row c = 16 rg + n, token
        // t = 16 tt + 4 g + i at [rg][tt][g][n][i]): registers 4q..4q+3 are four
        // consecutive tokens of one column, one 16-byte store
        const size_t cb = tile * (kBlk * kDim) + (dcol >> 4) * (kBlk * kApplyRows) + (dcol & 15) * 4;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int t0 = 8 * q + 4 * h, at = (t0 >> 4) * 256 + ((t0 >> 2) & 3) * 64;
            st4(P.u + cb + at, f4{tl[t0] * ua[4 * q], tl[t0 + 1] * ua[4 * q + 1], tl[t0 + 2] * ua[4 * q + 2],
                                  tl[t0 + 3] * ua[4 * q + 3]});
            st4(P.cu + cb + at, f4{cu[4 * q], cu[4 * q + 1], cu[4 * q + 2], cu[4 * q + 3]});
        }
    }
}

// ---- chunkwise apply: one block per (head, 16 value rows), 256 blocks of 5 waves. Waves
// 0..3 compute; wave w holds the state's key dims 32w..32w+31 as S^T in two 16x16 MFMA
// accumulators (register i of lane l: dim 32w + 16mt + 4(l/16) + i, value row l%16). With
// v_mfma_f32_16x16x4_f32 the k index of a product is the lane group l/16, so the k-steps
// are chosen to take the state, or D~ (same layout), as the B operand straight from
// registers: step (mt, i) covers dims 32w + 16mt + 4g + i (g = 0..3), and its A operands
// are four consecutive floats of an LDS row (one 128-bit read per four MFMAs).
//
// Wave 4 only copies: a block's operands (W~, Q', K rows, the block's U~ and CU, the
// factors: 53 KB) go global -> LDS directly (global_load_lds), double-buffered, the next
// block's while the current one computes. The copies pass the CU's address unit at about
// 64 bytes a clock, so a wave issuing them stalls for most of a block; a wave of their own
// keeps those stalls off the MFMA waves. Rows of 128 floats are stored with 16-byte piece
// p of row t at slot p ^ (t & 31), so both the 128-bit reads of a row segment and the
// 32-bit reads of a key column are conflict-free. Rows past the chunk's end read the
// chunk's last token: their W~, U~, Q' and CU rows are zero, so they add nothing to the
// state or to the stored rows.
struct ApplySet {
    float w[kBlk * kDim], q[kBlk * kDim], k[kBlk * kDim];
    float u[kBlk * kApplyRows], cu[kBlk * kApplyRows];   // [tt][g][n][i], as prepare writes them
    float f[2 * kBlk];                                    // (g, tail) per token
};

DIH_DEV int slot128(int t, int p) { return 4 * (p ^ (t & 31)); }

DIH_DEV f4 mfma16(float a, float b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// A quarter of a block's copies, by copy wave c: row pairs 4c..4c+3 of W~, Q' and K, one
// half of U~ (c = 0, 1) or CU (c = 2, 3); copy wave 0 also the 64 factors.
DIH_DEV void copy_block(ApplySet &S, const DeltaParams &P, int blk, int head, int kh, int rg, int c, int lane) {
    const int base = blk * kBlk, valid = min(kBlk, P.tokens - base);
    const size_t tile = (size_t)blk * kVHeads + head;
    const float *wt = P.w + tile * (kBlk * kDim), *qt = P.qp + tile * (kBlk * kDim);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int pair = 4 * c + i, t = 2 * pair + (lane >> 5), p = (lane & 31) ^ (t & 31);
        to_lds<16>(wt + t * kDim + 4 * p, S.w + 2 * pair * kDim);
        to_lds<16>(qt + t * kDim + 4 * p, S.q + 2 * pair * kDim);
        to_lds<16>(P.conv + (size_t)(base + min(t, valid - 1)) * kRowLen + kK + kh * kDim + 4 * p,
                   S.k + 2 * pair * kDim);
    }
    const int half = c & 1;
    const float *src = (c < 2 ? P.u : P.cu) + tile * (kBlk * kDim) + rg * (kBlk * kApplyRows) + 256 * half;
    to_lds<16>(src + 4 * lane, (c < 2 ? S.u : S.cu) + 256 * half);
    if (c == 0) to_lds<4>(P.factors + tile * (2 * kBlk) + lane, S.f);
}

// The block's partial products of the four waves: D~ needs all of W~ S^T (eight 128-bit
// reads: wave w2, token tile tt at byte offset 1024 (2 w2 + tt)), out one quarter of
// Q' S^T (four 64-bit reads 2 KB apart).
DIH_DEV void part_sums(const float *p1, const float *p2, f4 &d0, f4 &d1, dih_f32x2 &o) {
    d0 = (ld4(p1) + ld4(p1 + 512)) + (ld4(p1 + 1024) + ld4(p1 + 1536));
    d1 = (ld4(p1 + 256) + ld4(p1 + 768)) + (ld4(p1 + 1280) + ld4(p1 + 1792));
    const dih_f32x2 *q = reinterpret_cast<const dih_f32x2 *>(p2);
    o = (q[0] + q[256]) + (q[512] + q[768]);
}

// One block on a compute wave, from the set `S` the copy wave filled.
DIH_DEV void apply_block(const ApplySet &S, float (&part)[2][4][2][64 * 4], f4 (&st)[2], const DeltaParams &P,
                         int blk, int head, int rg, int wave, int lane) {
    const int n = lane & 15, g = lane >> 4;
    const int base = blk * kBlk, valid = min(kBlk, P.tokens - base);

    // partial (over this wave's dims) W~ S^T and Q' S^T, token tiles tt: C[m = token][n = row];
    // all eight operand reads first (the scheduler would otherwise wait on each pair just
    // before its MFMAs)
    f4 wa[2][2], qa[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const int t = 16 * tt + n, at = t * kDim + slot128(t, 8 * wave + 4 * mt + g);
            wa[tt][mt] = ld4(S.w + at);
            qa[tt][mt] = ld4(S.q + at);
        }
    __builtin_amdgcn_sched_barrier(0);
    f4 p1[2], p2[2];
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
        p1[tt] = f4{0.f, 0.f, 0.f, 0.f};
        p2[tt] = p1[tt];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p1[tt] = mfma16(wa[tt][mt][i], st[mt][i], p1[tt]);
                p2[tt] = mfma16(qa[tt][mt][i], st[mt][i], p2[tt]);
            }
    }
    // the state update's key operands, read ahead of the barrier: step (tt, i) covers tokens
    // 16tt + 4g + i, tile mt dims 32w + 16mt + n
    float ka[2][2][4];
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const int t = 16 * tt + 4 * g + i, dim = 32 * wave + 16 * mt + n;
                ka[tt][mt][i] = S.k[t * kDim + slot128(t, dim >> 2) + (dim & 3)];
            }
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
        st4(&part[0][wave][tt][lane * 4], p1[tt]);
        st4(&part[1][wave][tt][lane * 4], p2[tt]);
    }
    wait_lgkm0();
    barrier_no_fence();
    // D~ = U~ - sum_waves(W~ S^T) in full; out = CU + sum_waves(Q' S^T) for this wave's
    // quarter: token tile wave / 2, registers 2 (wave & 1) and 2 (wave & 1) + 1
    const int ot = wave >> 1, oi = 2 * (wave & 1);
    f4 s0, s1;
    dih_f32x2 o;
    part_sums(&part[0][0][0][lane * 4], &part[1][0][ot][lane * 4 + oi], s0, s1, o);
    const f4 d0 = ld4(S.u + lane * 4) - s0, d1 = ld4(S.u + 256 + lane * 4) - s1;
    o += *reinterpret_cast<const dih_f32x2 *>(S.cu + 256 * ot + lane * 4 + oi);
    float *ob = P.out + (size_t)(base + 16 * ot + 4 * g + oi) * (kVHeads * kDim) + head * kDim + rg * kApplyRows + n;
    if (16 * ot + 4 * g + oi < valid) ob[0] = o[0];
    if (16 * ot + 4 * g + oi + 1 < valid) ob[kVHeads * kDim] = o[1];

    // S^T <- g_last S^T + K^T D~: step (tt, i) covers tokens 16tt + 4g + i (the two state
    // tiles' chains in turn: two chains keep the MFMA pipe full)
    const float glast = S.f[2 * (valid - 1)];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) st[mt] *= glast;
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
        const f4 d = tt ? d1 : d0;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int mt = 0; mt < 2; mt++) st[mt] = mfma16(ka[tt][mt][i], d[i], st[mt]);
    }
}

// Blocks: XCD x (block b runs on XCD b % 8) takes value heads 2x, 2x + 1, 2x + 16, 2x + 17
// (two key heads), eight row groups each, so the blocks sharing a head's W~, Q' and K
// tiles share one L2. Two barriers a block: after the partial products (the sums need all
// four), and at its end (the copy wave's copies of the next block have landed, and the
// compute waves are done with this block's set and partial sums).
__global__ __launch_bounds__(512, 1) void delta_apply_kernel(DeltaParams P) {
    __shared__ __align__(16) ApplySet sets[2];
    __shared__ __align__(16) float part[2][4][2][64 * 4];
    lds_escape(sets, part);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, hl = slot >> 3, rg = slot & 7;
    const int head = 2 * xcd + (hl & 1) + 16 * (hl >> 1), kh = head >> 1;

    // (barriers without the memory fence: __syncthreads() would make the copy wave wait for
    // its copies at the mid-block barrier, and the compute waves for their row stores)
    if (wave >= 4) {
        copy_block(sets[0], P, 0, head, kh, rg, wave - 4, lane);
        wait_vm<0>();
        barrier_no_fence();
        for (int blk = 0; blk < P.nblocks; blk++) {
            if (blk + 1 < P.nblocks) copy_block(sets[(blk + 1) & 1], P, blk + 1, head, kh, rg, wave - 4, lane);
            barrier_no_fence();
            wait_vm<0>();
            barrier_no_fence();
        }
    } else {
        float *sbase =
            P.state + ((size_t)head * kDim + rg * kApplyRows + (lane & 15)) * kDim + 32 * wave + 4 * (lane >> 4);
        f4 st[2] = {ld4(sbase), ld4(sbase + 16)};
        barrier_no_fence();
        for (int blk = 0; blk < P.nblocks; blk++) {
            apply_block(sets[blk & 1], part, st, P, blk, head, rg, wave, lane);
            barrier_no_fence();
        }
        st4(sbase, st[0]);
        st4(sbase + 16, st[1]);
        if (blockIdx.x < kRowLen / 256) roll_history(P, blockIdx.x * 256 + tid);
    }
}

}  // namespace

bool launch_delta_rule(const DeltaArgs &a, hipStream_t s, char *error, int capacity) {
    DeltaParams P;
    P.conv = a.conv; P.decay = a.decay; P.beta = a.beta; P.raw = a.raw;
    P.state = a.state; P.history = a.history; P.out = a.out;
    P.w = a.w; P.u = a.u; P.qp = a.qp; P.cu = a.cu; P.factors = a.factors;
    P.tokens = a.tokens;
    P.nblocks = (a.tokens + kBlk - 1) / kBlk;
    if (!a.chunked) {
        DIH_LAUNCH(delta_seq_kernel, dim3(kVHeads * kDim / 16), dim3(256), 0, s, P);
        return hip_ok(hipGetLastError(), error, capacity, "delta launch");
    }
    if (!P.w || !P.u || !P.qp || !P.cu || !P.factors) {
        set_error(error, capacity, "Chunkwise delta rule needs its scratch buffers");
        return false;
    }
    prof_stage("delta_prepare");
    DIH_LAUNCH(delta_prepare_kernel, dim3(kVHeads, P.nblocks), dim3(256), 0, s, P);
    if (!hip_ok(hipGetLastError(), error, capacity, "delta prepare launch")) return false;
    prof_stage("delta_apply");
    DIH_LAUNCH(delta_apply_kernel, dim3(kVHeads * (kDim / kApplyRows)), dim3(512), 0, s, P);
    return hip_ok(hipGetLastError(), error, capacity, "delta apply launch");
}

}  // namespace dih
