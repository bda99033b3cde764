// Causal GQA attention of a prefill chunk (or one decode token) over a bf16 KV cache:
// prefill_attention_bf16 + graph_attention_combine (prefill_attention_bf16.mm:13-55,
// gpu_graph.mm:177-213; dispatch p_fused_attention, gpu_prefill.mm:552-570).
//
// Geometry (fixed by the model): 16 query heads, 2 KV heads (8 query heads per KV head),
// head dim 256. Cache rows [position][kv head][256] bf16; queries [token][16][256] f32 or
// bf16; gate source [token][16][512] (head h's gate at h*512+256); out [token][16][256].
//
// One block = 16 query tokens (four waves, decode and short chunks) or 32 query tokens
// (eight waves) x the 8 heads of one KV head x one partition of keys; each wave owns 32
// rows (4 tokens x 8 heads). Per 32-key tile:
//   S^T = K Q^T   16 v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = the wave's queries
//                 held in registers as bf16); the accumulator layout gives every lane one
//                 query row (lane & 31) and 16 of the tile's keys, so the row maximum and
//                 sum need one exchange with lane ^ 32 and the probabilities are already
//                 the B operand of the next product;
//   O^T += V^T P^T  16 MFMAs (A = the tile's values transposed into LDS, B = the bf16
//                 probabilities), again one row per lane: the rescale by exp(m_old - m_new)
//                 and the final 1/sum are lane-local.
// Probabilities are exp(s - m) against the running maximum including the current tile,
// summed unrounded and multiplied into the values as bf16 (RNE), the reference's rounding
// points (prefill_attention_bf16.mm:40-43). Scores are kept in log2 units
// (q.k * log2(e)/16) so each exponential is one v_exp_f32.
//
// Keys are split into partitions when the (tile, KV head) items alone cannot fill the
// GPU; each partition writes (max, sum) and its unnormalized 256 values and a combine
// kernel merges them (graph_attention_combine). With one partition the block finishes
// the output itself.
#include <algorithm>

#include "dih_device.h"
#include "dih_internal.h"

namespace dih {
namespace {

constexpr int kHeads = 16, kKvHeads = 2, kDim = 256, kGroup = kHeads / kKvHeads;
constexpr int kTok = 16;               // query tokens per block (128 rows)
constexpr int kKeys = 32;              // keys per tile
constexpr int kVtStride = kKeys + 4;   // bf16 per transposed value row: 72 B, conflict-free reads
constexpr float kLog2eOver16 = 1.4426950408889634f / 16.f;

struct AttnParams {
    const void *q; int q_bf16;
    const uint16_t *keys, *values;
    const void *gate; int gate_bf16;
    void *out; int out_bf16;
    float *pacc;       // [token][16][nparts][256] unnormalized partition outputs (split only)
    float2 *pstat;     // [token][16][nparts] (max in log2 units, sum)
    int position, tokens, partition, nparts, ntiles;
    int round;         // keys per rounding partition (a multiple of 32 dividing `partition`)
    float *scores;     // decode with rounding partitions: [2][tiles][32 lanes][8] raw scores
    float *tmax;       // and [2][tiles][8] tile maxima (log2 units)
};

DIH_DEV float sigmoid_f(float g) { return 1.f / (1.f + __expf(-g)); }

// Four consecutive output values of one row: out = acc * inv * sigmoid(gate).
DIH_DEV void store_out4(const AttnParams &P, int tok, int head, int d0, const float (&a)[4], float inv) {
    const size_t gi = (size_t)tok * (kHeads * 2 * kDim) + head * 2 * kDim + kDim + d0;
    const size_t oi = (size_t)tok * (kHeads * kDim) + head * kDim + d0;
    float g[4];
    if (P.gate_bf16) {
        const uint2 gb = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(P.gate) + gi);
        g[0] = __uint_as_float(gb.x << 16); g[1] = __uint_as_float(gb.x & 0xffff0000u);
        g[2] = __uint_as_float(gb.y << 16); g[3] = __uint_as_float(gb.y & 0xffff0000u);
    } else {
        const float4 gf = *reinterpret_cast<const float4 *>(static_cast<const float *>(P.gate) + gi);
        g[0] = gf.x; g[1] = gf.y; g[2] = gf.z; g[3] = gf.w;
    }
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = a[j] * inv * sigmoid_f(g[j]);
    if (P.out_bf16) {
        uint2 ob;
        ob.x = pack_bf16x2(v[0], v[1]);
        ob.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(P.out) + oi) = ob;
    } else {
        *reinterpret_cast<float4 *>(static_cast<float *>(P.out) + oi) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// Keys reach LDS by direct global->LDS copies (no registers): key row kl (512 B) holds its
// 16-byte piece c at slot c ^ (kl & 15), which makes the MFMA operand reads (16 lanes = 16
// keys, one piece each) conflict-free. Of a block of NW waves, wave w copies rows
// (32/NW)w .. (32/NW)(w+1)-1, two rows per instruction. Key indices past the partition end
// are clamped to its last key (finite data; those keys are masked).
template <int NW>
DIH_DEV void issue_keys(const uint16_t *kbase, uint16_t *ksbuf, int kb, int kend, int wave, int lane) {
    constexpr int RPW = kKeys / NW;   // rows per wave, two per copy instruction
#pragma unroll
    for (int i = 0; i < RPW / 2; i++) {
        const int kl = RPW * wave + 2 * i + (lane >> 5);
        const int c = (lane & 31) ^ (kl & 15);
        const uint32_t key = (uint32_t)min(kb + kl, kend - 1);
        // 32-bit element offset from the wave-uniform base (the cache is below 2^31 elements)
        const uint32_t off = key * (uint32_t)(kKvHeads * kDim) + 8u * (uint32_t)c;
        to_lds<16>(kbase + off, ksbuf + (RPW * wave + 2 * i) * kDim);
    }
}

// Values reach LDS the same way, untransposed (raw rows of 512 B, piece c at slot
// c ^ (kl & 15)), into one buffer that is consumed by the transpose below before the next
// tile's copies are issued.
template <int NW>
DIH_DEV void issue_values(const uint16_t *vbase, uint16_t *vraw, int kb, int kend, int wave, int lane) {
    issue_keys<NW>(vbase, vraw, kb, kend, wave, lane);
}

DIH_DEV void store_vt_pair(uint16_t *vt, int d, int vq, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    // each word holds dims d (low half) and d+1 (high half) of one key
    uint2 lo, hi;
    lo.x = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
    lo.y = __builtin_amdgcn_perm(w3, w2, 0x05040100u);
    hi.x = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
    hi.y = __builtin_amdgcn_perm(w3, w2, 0x07060302u);
    *reinterpret_cast<uint2 *>(vt + d * kVtStride + 4 * vq) = lo;
    *reinterpret_cast<uint2 *>(vt + (d + 1) * kVtStride + 4 * vq) = hi;
}

// Transpose: thread t reads the 8 dims of chunk t/8 of keys 4*(t%8) + i from the raw rows
// and writes dim d of those four keys as one 8-byte word of row d.
DIH_DEV void transpose_values(const uint16_t *vraw, uint16_t *vt, int vq, int vc) {
    uint4 v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int kl = 4 * vq + i;
        v[i] = *reinterpret_cast<const uint4 *>(vraw + kl * kDim + 8 * (vc ^ (kl & 15)));
    }
    const int d = 8 * vc;
    store_vt_pair(vt, d, vq, v[0].x, v[1].x, v[2].x, v[3].x);
    store_vt_pair(vt, d + 2, vq, v[0].y, v[1].y, v[2].y, v[3].y);
    store_vt_pair(vt, d + 4, vq, v[0].z, v[1].z, v[2].z, v[3].z);
    store_vt_pair(vt, d + 6, vq, v[0].w, v[1].w, v[2].w, v[3].w);
}

// The same for 512 threads: thread t reads 4 dims (4*(t/8)..+3) of keys 4*(t%8)..+3.
DIH_DEV void transpose_values8(const uint16_t *vraw, uint16_t *vt, int t) {
    const int vq = t & 7, vd = t >> 3;
    uint2 v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int kl = 4 * vq + i;
        v[i] = *reinterpret_cast<const uint2 *>(vraw + kl * kDim + 8 * ((vd >> 1) ^ (kl & 15)) + 4 * (vd & 1));
    }
    // word x of each key holds dims 4vd (low half), 4vd+1; word y dims 4vd+2, 4vd+3
    const uint32_t lo[4] = {v[0].x, v[1].x, v[2].x, v[3].x}, hi[4] = {v[0].y, v[1].y, v[2].y, v[3].y};
    uint16_t *row = vt + 4 * vd * kVtStride + 4 * vq;
    *reinterpret_cast<uint2 *>(row) = make_uint2(__builtin_amdgcn_perm(lo[1], lo[0], 0x05040100u),
                                                 __builtin_amdgcn_perm(lo[3], lo[2], 0x05040100u));
    *reinterpret_cast<uint2 *>(row + kVtStride) = make_uint2(__builtin_amdgcn_perm(lo[1], lo[0], 0x07060302u),
                                                             __builtin_amdgcn_perm(lo[3], lo[2], 0x07060302u));
    *reinterpret_cast<uint2 *>(row + 2 * kVtStride) = make_uint2(__builtin_amdgcn_perm(hi[1], hi[0], 0x05040100u),
                                                                 __builtin_amdgcn_perm(hi[3], hi[2], 0x05040100u));
    *reinterpret_cast<uint2 *>(row + 3 * kVtStride) = make_uint2(__builtin_amdgcn_perm(hi[1], hi[0], 0x07060302u),
                                                                 __builtin_amdgcn_perm(hi[3], hi[2], 0x07060302u));
}

// ---- the parts of a wave's work shared by both block shapes. A wave owns 32 rows: 4
// tokens x the 8 query heads of one KV head; lane (r, h) holds row r.

// The wave's queries as MFMA B operands: qreg[s] = q[row][16s + 8h .. +8] in bf16.
DIH_DEV void load_queries(dih_bf16x8 (&qreg)[16], const AttnParams &P, int my_tok, bool row_ok, int head, int h) {
    const size_t qi = (size_t)(row_ok ? my_tok : 0) * (kHeads * kDim) + head * kDim + 8 * h;
#pragma unroll
    for (int s = 0; s < 16; s++) {
        uint4 u;
        if (P.q_bf16) {
            u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(P.q) + qi + 16 * s);
        } else {
            const float4 *f = reinterpret_cast<const float4 *>(static_cast<const float *>(P.q) + qi + 16 * s);
            const float4 f0 = f[0], f1 = f[1];
            u.x = pack_bf16x2(f0.x, f0.y); u.y = pack_bf16x2(f0.z, f0.w);
            u.z = pack_bf16x2(f1.x, f1.y); u.w = pack_bf16x2(f1.z, f1.w);
        }
        if (!row_ok) u = make_uint4(0, 0, 0, 0);
        qreg[s] = __builtin_bit_cast(dih_bf16x8, u);
    }
}

// A row's softmax state over the keys a block scans. Probabilities are rounded against
// `m`, the running maximum of the current rounding partition (restarted at its first key),
// and the accumulators and `sum` are kept in the scale 2^-(m + ak). Normally ak = 0: the
// accumulators follow the rounding maximum, and after a restart (a partition whose maximum
// is below an earlier one) they are scaled up by 2^(old - new) rather than the new
// partition's probabilities being scaled down, which keeps the bf16 probabilities exactly as
// rounded. Only when that would put the scale more than 2^kMaxUp below `seen` (the maximum
// of every key scanned; accumulators near 2^(15 + kMaxUp) times the largest value) does ak
// rise, and the partition's probabilities enter scaled by the exact power of two 2^-ak. All
// maxima are in log2 units (score * log2(e) / 16).
constexpr float kMaxUp = 64.f;
struct RowState {
    float m = -INFINITY, seen = -INFINITY, ak = 0.f, sum = 0.f;
    DIH_DEV float scale_max() const { return m == -INFINITY ? -INFINITY : m + ak; }
};

// bf16 pair `w` times the power of two `f` (exact: only the exponents change, values below
// the normal range excepted, which are negligible next to the row's sum).
DIH_DEV uint32_t scale_bf16x2(uint32_t w, float f) {
    return pack_bf16x2(__uint_as_float(w << 16) * f, __uint_as_float(w & 0xffff0000u) * f);
}

// One 32-key tile (keys kb.., rows from ksb, values transposed in vtb) for the wave's rows.
// `full`: every row of the wave sees the whole tile (no mask needed). RESTARTS: the block's
// keys span more than one rounding partition; `restart`: this tile starts one (and is not
// the block's first tile).
template <bool RESTARTS>
DIH_DEV void attend_tile(const uint16_t *ksb, const uint16_t *vtb, const dih_bf16x8 (&qreg)[16],
                         dih_f32x16 (&acc)[8], RowState &st, int kb, int kend, bool full, bool restart,
                         int my_last, int r, int h) {    // ---- S^T = K Q^T: s[k] is key kb + 8(k/4) + 4h + k%4 of row r
    dih_f32x16 s;
#pragma unroll
    for (int k = 0; k < 16; k++) s[k] = 0.f;
#pragma unroll
    for (int st = 0; st < 16; st++) {
        const dih_bf16x8 a = *reinterpret_cast<const dih_bf16x8 *>(ksb + r * kDim + 8 * ((2 * st + h) ^ (r & 15)));
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[st], s, 0, 0, 0);
    }
    // ---- online softmax for row r. Scores stay raw here; the log2 scale enters the
    // exponent's FMA.
    float mx = -INFINITY;
    if (full) {
#pragma unroll
        for (int k = 0; k < 16; k++) mx = fmaxf(mx, s[k]);
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int key = kb + 8 * (k >> 2) + 4 * h + (k & 3);
            s[k] = key <= my_last && key < kend ? s[k] : -INFINITY;
            mx = fmaxf(mx, s[k]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float tmax = mx * kLog2eOver16;
    float r_new, alpha, f = 1.f;
    if constexpr (RESTARTS) {
        // a row with no visible key in this tile has none in any later one (causal and kend
        // masks only grow): it keeps its maximum, its p are 0 and alpha is 1
        r_new = restart && tmax != -INFINITY ? tmax : fmaxf(st.m, tmax);
        const float seen = fmaxf(st.seen, tmax);
        const float k_new = fmaxf(ceilf(seen - r_new) - kMaxUp, 0.f);   // (NaN: nothing seen -> 0)
        alpha = st.m == -INFINITY ? 0.f : exp2f((st.m - r_new) + (st.ak - k_new));
        f = __builtin_amdgcn_ldexpf(1.f, -(int)k_new);
        st.seen = seen;
        st.ak = k_new;
    } else {
        r_new = fmaxf(st.m, tmax);
        alpha = st.m == -INFINITY ? 0.f : exp2f(st.m - r_new);
    }
    st.m = r_new;
    const float m_use = r_new == -INFINITY ? 0.f : r_new;   // all keys masked: p = 0
    float psum = 0.f;
    uint32_t pw[8];
#pragma unroll
    for (int k = 0; k < 16; k += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(s[k], kLog2eOver16, -m_use));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(s[k + 1], kLog2eOver16, -m_use));
        psum += p0 + p1;
        pw[k >> 1] = pack_bf16x2(p0, p1);
    }
    psum += __shfl_xor(psum, 32, 64);
    st.sum = st.sum * alpha + psum * f;
    // probabilities of a partition far below the scale: rounded above, then scaled exactly
    if (RESTARTS && __ballot(f != 1.f)) {
#pragma unroll
        for (int i = 0; i < 8; i++) pw[i] = scale_bf16x2(pw[i], f);
    }
    // rescale only when some row's scale moved (alpha == 1 exactly otherwise)
    if (__ballot(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int k = 0; k < 16; k++) acc[dt][k] *= alpha;
    }
    const dih_bf16x8 pb0 = __builtin_bit_cast(dih_bf16x8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
    const dih_bf16x8 pb1 = __builtin_bit_cast(dih_bf16x8, make_uint4(pw[4], pw[5], pw[6], pw[7]));
    // ---- O^T = O^T * alpha + V^T P^T: acc[dt][k] is dim 32dt + 8(k/4) + 4h + k%4 of row r
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
        const uint16_t *vrow = vtb + (32 * dt + r) * kVtStride + 4 * h;
        const uint2 a0 = *reinterpret_cast<const uint2 *>(vrow);
        const uint2 a1 = *reinterpret_cast<const uint2 *>(vrow + 8);
        const uint2 a2 = *reinterpret_cast<const uint2 *>(vrow + 16);
        const uint2 a3 = *reinterpret_cast<const uint2 *>(vrow + 24);
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(dih_bf16x8, make_uint4(a0.x, a0.y, a1.x, a1.y)), pb0, acc[dt], 0, 0, 0);
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(dih_bf16x8, make_uint4(a2.x, a2.y, a3.x, a3.y)), pb1, acc[dt], 0, 0, 0);
    }
}

// The wave's rows after the partition: the output itself, or the partition's statistics
// and unnormalized values for the combine.
DIH_DEV void finish_rows(const AttnParams &P, const dih_f32x16 (&acc)[8], const RowState &st, int my_tok,
                         int head, int part, int h) {
    if (P.nparts == 1) {
        const float inv = 1.f / st.sum;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float a4[4] = {acc[dt][4 * i], acc[dt][4 * i + 1], acc[dt][4 * i + 2], acc[dt][4 * i + 3]};
                store_out4(P, my_tok, head, 32 * dt + 8 * i + 4 * h, a4, inv);
            }
    } else {
        const size_t pi = ((size_t)my_tok * kHeads + head) * P.nparts + part;
        if (h == 0) P.pstat[pi] = make_float2(st.scale_max(), st.sum);
        float *pa = P.pacc + pi * kDim;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                *reinterpret_cast<float4 *>(pa + 32 * dt + 8 * i + 4 * h) =
                    make_float4(acc[dt][4 * i], acc[dt][4 * i + 1], acc[dt][4 * i + 2], acc[dt][4 * i + 3]);
    }
}

template <bool RESTARTS>
__global__ __launch_bounds__(256, 2) void attn_kernel(AttnParams P) {
    __shared__ __align__(16) uint16_t ks[2][kKeys * kDim];
    __shared__ __align__(16) uint16_t vraw[kKeys * kDim];
    __shared__ __align__(16) uint16_t vt[kDim * kVtStride];

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, r = lane & 31, h = lane >> 5;
    // ---- work item. Blocks are dealt round-robin to the 8 XCDs (block b on XCD b % 8):
    // XCDs 0-3 take KV head 0 and 4-7 KV head 1, so one XCD's L2 holds one head's keys
    // and values; within a head the items run heaviest (latest query tile) first.
    const int b = blockIdx.x, x = b & 7, kh = x >> 2;
    const int idx = (x & 3) + 4 * (b >> 3);
    if (idx >= P.ntiles * P.nparts) return;
    const int tile = P.ntiles - 1 - idx / P.nparts, part = idx - (idx / P.nparts) * P.nparts;
    const int tok0 = tile * kTok;
    const int tok_hi = min(tok0 + kTok, P.tokens) - 1;
    const int kstart = part * P.partition;
    const int kend = min(kstart + P.partition, P.position + tok_hi + 1);
    if (kstart >= kend) return;

    const int wtok0 = tok0 + 4 * wave;                      // the wave's first token
    const bool wave_ok = wtok0 < P.tokens;
    const int wave_last = P.position + min(wtok0 + 3, P.tokens - 1);   // last key any row may see
    const int my_tok = wtok0 + (r >> 3), head = kh * kGroup + (r & 7);
    const bool row_ok = my_tok < P.tokens;
    const int my_last = row_ok ? P.position + my_tok : -1;

    dih_bf16x8 qreg[16];
    load_queries(qreg, P, my_tok, row_ok, head, h);

    // ---- tiles are copied one compute phase ahead
    const uint16_t *kbase = P.keys + kh * kDim, *vbase = P.values + kh * kDim;
    const int vq = t & 7, vc = t >> 3;
    RowState st;
    dih_f32x16 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int k = 0; k < 16; k++) acc[i][k] = 0.f;

    issue_keys<4>(kbase, ks[0], kstart, kend, wave, lane);
    issue_values<4>(vbase, vraw, kstart, kend, wave, lane);
    int buf = 0;
    for (int kb = kstart; kb < kend; kb += kKeys, buf ^= 1) {
        wait_vm<0>();             // this thread's copies have landed
        __syncthreads();          // every thread's copies are in LDS; the previous tile's reads are done
        transpose_values(vraw, vt, vq, vc);
        __syncthreads();          // vt complete, vraw consumed
        if (kb + kKeys < kend) {
            issue_keys<4>(kbase, ks[buf ^ 1], kb + kKeys, kend, wave, lane);
            issue_values<4>(vbase, vraw, kb + kKeys, kend, wave, lane);
        }
        if (!wave_ok || kb > wave_last) continue;
        const bool full = kb + kKeys - 1 <= P.position + wtok0 && kb + kKeys <= kend;
        attend_tile<RESTARTS>(ks[buf], vt, qreg, acc, st, kb, kend, full,
                              RESTARTS && kb != kstart && kb % P.round == 0, my_last, r, h);
    }
    if (!row_ok) return;
    finish_rows(P, acc, st, my_tok, head, part, h);
}

// ---- eight-wave form: 32 query tokens (256 rows) per block share each key/value tile.
// Keys are triple-buffered and values double-buffered (raw copies and transposed), so one
// barrier per tile suffices and every tile's copies are issued two tiles ahead:
//   top of tile j: tile j's keys and transposed values are in LDS, tile j+1's copies landed
//   issue tile j+2's copies (into the buffers tile j-1 used), compute tile j, transpose
//   tile j+1's values, wait for this thread's copies, barrier.
template <bool RESTARTS>
__global__ __launch_bounds__(512, 1) void attn8_kernel(AttnParams P) {
    __shared__ __align__(16) uint16_t ks[3][kKeys * kDim];
    __shared__ __align__(16) uint16_t vraw[2][kKeys * kDim];
    __shared__ __align__(16) uint16_t vt[2][kDim * kVtStride];
    lds_escape(ks, vraw, vt);

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, r = lane & 31, h = lane >> 5;
    // work item: as attn_kernel, with 32-token tiles
    const int b = blockIdx.x, x = b & 7, kh = x >> 2;
    const int idx = (x & 3) + 4 * (b >> 3);
    if (idx >= P.ntiles * P.nparts) return;
    const int tile = P.ntiles - 1 - idx / P.nparts, part = idx - (idx / P.nparts) * P.nparts;
    const int tok0 = tile * (2 * kTok);
    const int tok_hi = min(tok0 + 2 * kTok, P.tokens) - 1;
    const int kstart = part * P.partition;
    const int kend = min(kstart + P.partition, P.position + tok_hi + 1);
    if (kstart >= kend) return;

    const int wtok0 = tok0 + 4 * wave;
    const bool wave_ok = wtok0 < P.tokens;
    const int wave_last = P.position + min(wtok0 + 3, P.tokens - 1);
    const int my_tok = wtok0 + (r >> 3), head = kh * kGroup + (r & 7);
    const bool row_ok = my_tok < P.tokens;
    const int my_last = row_ok ? P.position + my_tok : -1;

    dih_bf16x8 qreg[16];
    load_queries(qreg, P, my_tok, row_ok, head, h);
    RowState st;
    dih_f32x16 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int k = 0; k < 16; k++) acc[i][k] = 0.f;

    const uint16_t *kbase = P.keys + kh * kDim, *vbase = P.values + kh * kDim;
    const int ntile = (kend - kstart + kKeys - 1) / kKeys;
    issue_keys<8>(kbase, ks[0], kstart, kend, wave, lane);
    issue_values<8>(vbase, vraw[0], kstart, kend, wave, lane);
    if (ntile > 1) {
        issue_keys<8>(kbase, ks[1], kstart + kKeys, kend, wave, lane);
        issue_values<8>(vbase, vraw[1], kstart + kKeys, kend, wave, lane);
        wait_vm<4>();         // tile 0's four copies of this thread (tile 1's may stay in flight)
    } else {
        wait_vm<0>();
    }
    barrier_no_fence();
    transpose_values8(vraw[0], vt[0], t);
    wait_vm<0>();
    wait_lgkm0();
    barrier_no_fence();

    int k3 = 0;   // j % 3
    for (int j = 0; j < ntile; j++) {
        const int kb = kstart + j * kKeys;
        if (j + 2 < ntile) {
            const int k3n = k3 == 0 ? 2 : k3 - 1;   // (j + 2) % 3
            issue_keys<8>(kbase, ks[k3n], kb + 2 * kKeys, kend, wave, lane);
            issue_values<8>(vbase, vraw[j & 1], kb + 2 * kKeys, kend, wave, lane);
        }
        if (wave_ok && kb <= wave_last) {
            const bool full = kb + kKeys - 1 <= P.position + wtok0 && kb + kKeys <= kend;
            attend_tile<RESTARTS>(ks[k3], vt[j & 1], qreg, acc, st, kb, kend, full,
                                  RESTARTS && kb != kstart && kb % P.round == 0, my_last, r, h);
        }
        if (j + 1 < ntile) transpose_values8(vraw[(j + 1) & 1], vt[(j + 1) & 1], t);
        wait_vm<0>();
        wait_lgkm0();
        barrier_no_fence();
        k3 = k3 == 2 ? 0 : k3 + 1;
    }
    if (!row_ok) return;
    finish_rows(P, acc, st, my_tok, head, part, h);
}

// One wave per (token, head), four dims per lane: merge the partitions that hold keys of
// this token (graph_attention_combine, gpu_graph.mm:199-213). Each lane computes the
// weight exp(m_p - M) of one partition of a 64-partition chunk; the chunk's partial rows
// are then read eight at a time (independent loads) with the weights broadcast by lane.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams P) {
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int th = blockIdx.x * 4 + wv;            // tok * 16 + head
    if (th >= P.tokens * kHeads) return;
    const int tok = th / kHeads, head = th - tok * kHeads;
    const int np = (P.position + tok) / P.partition + 1;
    const size_t pi = (size_t)th * P.nparts;
    const float2 *st = P.pstat + pi;
    float m = -INFINITY;
    for (int p = lane; p < np; p += 64) m = fmaxf(m, st[p].x);
    m = wave_max(m);
    float total = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 *pa = reinterpret_cast<const float4 *>(P.pacc + pi * kDim) + lane;
    for (int c0 = 0; c0 < np; c0 += 64) {
        const int n = min(64, np - c0);
        float w = 0.f;
        if (lane < n) {
            const float2 v = st[c0 + lane];
            w = exp2f(v.x - m);
            total += w * v.y;
        }
        int p = 0;
        for (; p + 8 <= n; p += 8) {
            float4 a[8];
#pragma unroll
            for (int j = 0; j < 8; j++) a[j] = pa[(size_t)(c0 + p + j) * (kDim / 4)];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float wj = __shfl(w, p + j, 64);
                acc.x += wj * a[j].x; acc.y += wj * a[j].y; acc.z += wj * a[j].z; acc.w += wj * a[j].w;
            }
        }
        for (; p < n; p++) {
            const float4 a = pa[(size_t)(c0 + p) * (kDim / 4)];
            const float wj = __shfl(w, p, 64);
            acc.x += wj * a.x; acc.y += wj * a.y; acc.z += wj * a.z; acc.w += wj * a.w;
        }
    }
    total = wave_sum(total);
    const float a4[4] = {acc.x, acc.y, acc.z, acc.w};
    store_out4(P, tok, head, 4 * lane, a4, 1.f / total);
}

// ---- decode (one query token): a block is four waves, each one 32-key tile of one KV
// head (128 keys a block). Every tile is its own partition of 32 keys (the partition-32
// rounding points: probabilities against the tile's maximum) and the block merges its four
// as the combine does. A wave has no barrier before the merge: its keys (MFMA A operand),
// values and queries are loaded straight into registers, 48 x 16 bytes a lane all in
// flight at once, and only the values pass through LDS, to be transposed for O^T = V^T P^T.
// Products are v_mfma_f32_16x16x32_bf16 (lane l: row l % 16, k = 8(l / 16)..+7; result
// rows 4(l / 16) + i).
constexpr int kDecKeys = 4 * kKeys;   // keys per decode block
// the reference's default rounding partition (attentionPartitionTokens, gpu_prefill.mm:393)
constexpr int kDefaultRound = 1024;
// longest rounding partition the decode scores pass serves (a lane reads a quarter of its
// tile maxima: 32 at most); longer ones run the general kernel
constexpr int kMaxPremaxRound = 4096;

DIH_DEV dih_f32x4 mfma16_bf16(dih_bf16x8 a, dih_bf16x8 b, dih_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Decode with rounding partitions longer than a tile (PREMAX): attn_decode_scores_kernel
// first writes every tile's raw scores and per-row maxima; the decode kernel then takes its
// tile's scores from there and rounds the probabilities against the running maximum of the
// rounding partition up to and including its tile (the maxima of that partition's earlier
// tiles, read back), which is the reference's rounding point, while the blocks still split
// the keys 128 at a time.
//
// Scores kernel: the same block and wave mapping as the decode kernel. Lane (n < 8, g) of a
// tile's wave stores s[mt][i] (key kb + 16mt + 4g + i, head 8kh + n) at
// scores[((kh * tiles + tile) * 32 + 8g + n) * 8 + 4mt + i] and lane (n, 0) the row maximum
// at tmax[(kh * tiles + tile) * 8 + n]; masked keys are -inf.
template <bool QBF16>
__global__ __launch_bounds__(256) void attn_decode_scores_kernel(AttnParams P) {
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, n = lane & 15, g = lane >> 4;
    const int b = blockIdx.x, x = b & 7, kh = x >> 2;
    const int idx = (x & 3) + 4 * (b >> 3);
    if (idx >= P.nparts) return;   // whole block
    const int kend = P.position + 1;
    const int kb = idx * kDecKeys + kKeys * wave;
    const uint16_t *kbase = P.keys + kh * kDim;
    dih_bf16x8 ka[2][8];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        const uint32_t key = (uint32_t)min(kb + 16 * mt + n, kend - 1);
#pragma unroll
        for (int s = 0; s < 8; s++)
            ka[mt][s] = *reinterpret_cast<const dih_bf16x8 *>(kbase + key * (uint32_t)(kKvHeads * kDim) + 32 * s + 8 * g);
    }
    const int qhead = kh * kGroup + (n & 7);
    dih_bf16x8 qb[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        uint4 u = make_uint4(0, 0, 0, 0);
        if (n < kGroup) {
            if constexpr (QBF16) {
                u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(P.q) + (size_t)qhead * kDim + 32 * s + 8 * g);
            } else {
                const float *qs = static_cast<const float *>(P.q) + (size_t)qhead * kDim + 32 * s + 8 * g;
                const float4 f0 = *reinterpret_cast<const float4 *>(qs), f1 = *reinterpret_cast<const float4 *>(qs + 4);
                u.x = pack_bf16x2(f0.x, f0.y); u.y = pack_bf16x2(f0.z, f0.w);
                u.z = pack_bf16x2(f1.x, f1.y); u.w = pack_bf16x2(f1.z, f1.w);
            }
        }
        qb[s] = __builtin_bit_cast(dih_bf16x8, u);
    }
    dih_f32x4 sc[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        sc[mt] = dih_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; s++) sc[mt] = mfma16_bf16(ka[mt][s], qb[s], sc[mt]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = kb + 16 * mt + 4 * g + i;
            sc[mt][i] = key < kend ? sc[mt][i] : -INFINITY;
            mx = fmaxf(mx, sc[mt][i]);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (n < kGroup) {
        const size_t ti = (size_t)kh * (4 * P.nparts) + 4 * idx + wave;
        float4 *dst = reinterpret_cast<float4 *>(P.scores + (ti * 32 + 8 * g + n) * 8);
        dst[0] = make_float4(sc[0][0], sc[0][1], sc[0][2], sc[0][3]);
        dst[1] = make_float4(sc[1][0], sc[1][1], sc[1][2], sc[1][3]);
        if (g == 0) P.tmax[ti * 8 + n] = mx * kLog2eOver16;
    }
}

// Largest of the tile maxima tm[8 * tt] for tt = first + g, first + g + 4, .. <= tile (L
// of them at most): independent loads (indices past `tile` repeat it), so that they are all
// in flight together rather than one round trip each.
template <int L>
DIH_DEV float tile_prefix_max(const float *tm, int first, int tile, int g) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < L; j++) m = fmaxf(m, tm[8 * min(first + g + 4 * j, tile)]);
    return m;
}

template <bool QBF16, bool PREMAX>
__global__ __launch_bounds__(256, 2) void attn_decode_kernel(AttnParams P) {
    __shared__ __align__(16) uint16_t vt[4][kDim * kVtStride];   // per wave; its partial sums after
    __shared__ __align__(16) uint16_t pb[4][16 * kKeys];         // per wave: bf16 probabilities [row][key]
    __shared__ float2 stat[4][kGroup];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, n = lane & 15, g = lane >> 4;
    // blocks dealt round-robin to the 8 XCDs: XCDs 0-3 take KV head 0, 4-7 KV head 1
    const int b = blockIdx.x, x = b & 7, kh = x >> 2;
    const int idx = (x & 3) + 4 * (b >> 3);
    if (idx >= P.nparts) return;   // whole block
    const int kend = P.position + 1;
    const int kb = idx * kDecKeys + kKeys * wave;
    const uint16_t *kbase = P.keys + kh * kDim, *vbase = P.values + kh * kDim;

    // keys, the A operand: m-tile mt, k-step s: key kb + 16mt + n, dims 32s + 8g..+7
    // (indices past the visible keys clamped to the last one; those scores are masked)
    dih_bf16x8 ka[2][8];
    if constexpr (!PREMAX) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const uint32_t key = (uint32_t)min(kb + 16 * mt + n, kend - 1);
#pragma unroll
            for (int s = 0; s < 8; s++)
                ka[mt][s] = *reinterpret_cast<const dih_bf16x8 *>(kbase + key * (uint32_t)(kKvHeads * kDim) + 32 * s + 8 * g);
        }
    }
    // values for the transpose: keys kb + 4vq + i, dims 8vc..8vc+7, vc = lane / 8 + 8j
    const int vq = lane & 7;
    uint4 vv[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t key = (uint32_t)min(kb + 4 * vq + i, kend - 1);
#pragma unroll
        for (int j = 0; j < 4; j++)
            vv[j][i] = *reinterpret_cast<const uint4 *>(vbase + key * (uint32_t)(kKvHeads * kDim) + 8 * ((lane >> 3) + 8 * j));
    }
    // queries, the B operand of S = K Q^T: lane (row n, g) holds dims 32s + 8g..+7 of head
    // 8kh + n (rows 8..15 zero); loaded raw behind the keys and values, converted after, so
    // that all of the wave's loads are in flight together
    const int qhead = kh * kGroup + (n & 7);
    // PREMAX: the tile's scores (rows 8..15: none, -inf) and the rounding maximum, the
    // largest of the tile maxima from the rounding partition's first tile through this one
    // (lane (n, g) reads every fourth of them, then the four lanes of row n combine)
    float4 sv[2] = {make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY),
                    make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY)};
    float rmax = -INFINITY;
    if constexpr (PREMAX) {
        if (n < kGroup) {
            const size_t ti0 = (size_t)kh * (4 * P.nparts);
            const int tile = 4 * idx + wave, first = tile - tile % (P.round / kKeys);
            const float4 *src = reinterpret_cast<const float4 *>(P.scores + ((ti0 + tile) * 32 + 8 * g + n) * 8);
            sv[0] = src[0];
            sv[1] = src[1];
            const float *tm = P.tmax + ti0 * 8 + n;
            const int span = tile - first;   // earlier tiles of the rounding partition
            rmax = span < 32 ? tile_prefix_max<8>(tm, first, tile, g)
                 : span < 64 ? tile_prefix_max<16>(tm, first, tile, g) : tile_prefix_max<32>(tm, first, tile, g);
        }
    }
    // (rows 8..15 load nothing: a branch, so that their lanes are off for the loads)
    float4 qf[8][2] = {};
    uint4 qu[8] = {};
    if (!PREMAX && n < kGroup) {
        if constexpr (QBF16) {
            const uint16_t *qs = static_cast<const uint16_t *>(P.q) + (size_t)qhead * kDim + 8 * g;
#pragma unroll
            for (int s = 0; s < 8; s++) qu[s] = *reinterpret_cast<const uint4 *>(qs + 32 * s);
        } else {
            const float *qs = static_cast<const float *>(P.q) + (size_t)qhead * kDim + 8 * g;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                qf[s][0] = *reinterpret_cast<const float4 *>(qs + 32 * s);
                qf[s][1] = *reinterpret_cast<const float4 *>(qs + 32 * s + 4);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    dih_bf16x8 qb[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        uint4 u = qu[s];
        if constexpr (!QBF16) {
            u.x = pack_bf16x2(qf[s][0].x, qf[s][0].y); u.y = pack_bf16x2(qf[s][0].z, qf[s][0].w);
            u.z = pack_bf16x2(qf[s][1].x, qf[s][1].y); u.w = pack_bf16x2(qf[s][1].z, qf[s][1].w);
        }
        if (n >= kGroup) u = make_uint4(0, 0, 0, 0);
        qb[s] = __builtin_bit_cast(dih_bf16x8, u);
    }

    // ---- S = K Q^T: s[mt][i] is key kb + 16mt + 4g + i of row n
    dih_f32x4 sc[2];
    if constexpr (PREMAX) {
        sc[0] = dih_f32x4{sv[0].x, sv[0].y, sv[0].z, sv[0].w};
        sc[1] = dih_f32x4{sv[1].x, sv[1].y, sv[1].z, sv[1].w};
    } else {
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            sc[mt] = dih_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; s++) sc[mt] = mfma16_bf16(ka[mt][s], qb[s], sc[mt]);
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = kb + 16 * mt + 4 * g + i;
            sc[mt][i] = key < kend ? sc[mt][i] : -INFINITY;
            mx = fmaxf(mx, sc[mt][i]);
        }
    if constexpr (PREMAX) mx = rmax;   // the rounding maximum is in log2 units already
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = PREMAX ? mx : mx * kLog2eOver16;
    const float m_use = m_new == -INFINITY ? 0.f : m_new;   // a tile past the keys: p = 0
    float psum = 0.f;
    uint16_t *pbw = pb[wave];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p[i] = __builtin_amdgcn_exp2f(fmaf(sc[mt][i], kLog2eOver16, -m_use));
            psum += p[i];
        }
        *reinterpret_cast<uint2 *>(pbw + n * kKeys + 16 * mt + 4 * g) =
            make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]));
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);

    // ---- values transposed into the wave's LDS rows (dim d: its 32 keys, 72-byte rows)
    uint16_t *vtw = vt[wave];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int d = 8 * ((lane >> 3) + 8 * j);
        store_vt_pair(vtw, d, vq, vv[j][0].x, vv[j][1].x, vv[j][2].x, vv[j][3].x);
        store_vt_pair(vtw, d + 2, vq, vv[j][0].y, vv[j][1].y, vv[j][2].y, vv[j][3].y);
        store_vt_pair(vtw, d + 4, vq, vv[j][0].z, vv[j][1].z, vv[j][2].z, vv[j][3].z);
        store_vt_pair(vtw, d + 6, vq, vv[j][0].w, vv[j][1].w, vv[j][2].w, vv[j][3].w);
    }
    // ---- O^T = V^T P^T: o[dt][i] is dim 16dt + 4g + i of row n
    const dih_bf16x8 pk = *reinterpret_cast<const dih_bf16x8 *>(pbw + n * kKeys + 8 * g);
    dih_f32x4 o[16];
#pragma unroll
    for (int dt = 0; dt < 16; dt++) {
        const uint16_t *vrow = vtw + (16 * dt + n) * kVtStride + 8 * g;
        const uint2 a0 = *reinterpret_cast<const uint2 *>(vrow), a1 = *reinterpret_cast<const uint2 *>(vrow + 4);
        o[dt] = mfma16_bf16(__builtin_bit_cast(dih_bf16x8, make_uint4(a0.x, a0.y, a1.x, a1.y)), pk,
                            dih_f32x4{0.f, 0.f, 0.f, 0.f});
    }
    // ---- merge the four tiles: the partial sums of rows 0..7 go over the wave's own LDS
    // rows (its reads of them are done: their values fed the MFMAs above)
    float *accw = reinterpret_cast<float *>(vtw);   // [8 rows][256]
    asm volatile("" ::: "memory");   // (the value rows above are read as uint16_t, written as float)
    if (n < kGroup) {
#pragma unroll
        for (int dt = 0; dt < 16; dt++) *reinterpret_cast<dih_f32x4 *>(accw + n * kDim + 16 * dt + 4 * g) = o[dt];
        if (g == 0) stat[wave][n] = make_float2(m_new, psum);
    }
    __syncthreads();
    // thread: row t / 32, dims 8(t % 32)..+7
    const int row = t >> 5, d0 = 8 * (t & 31);
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; w++) m = fmaxf(m, stat[w][row].x);
    float total = 0.f, a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float2 st = stat[w][row];
        const float wt = exp2f(st.x - m);   // 0 for a tile past the keys (max -inf)
        total += wt * st.y;
        const float *src = reinterpret_cast<const float *>(vt[w]) + row * kDim + d0;
        const float4 u0 = *reinterpret_cast<const float4 *>(src), u1 = *reinterpret_cast<const float4 *>(src + 4);
        a[0] += wt * u0.x; a[1] += wt * u0.y; a[2] += wt * u0.z; a[3] += wt * u0.w;
        a[4] += wt * u1.x; a[5] += wt * u1.y; a[6] += wt * u1.z; a[7] += wt * u1.w;
    }
    const int head = kh * kGroup + row;
    if (P.nparts == 1) {
        const float a0[4] = {a[0], a[1], a[2], a[3]}, a1[4] = {a[4], a[5], a[6], a[7]};
        store_out4(P, 0, head, d0, a0, 1.f / total);
        store_out4(P, 0, head, d0 + 4, a1, 1.f / total);
    } else {
        const size_t pi = (size_t)head * P.nparts + idx;
        if ((t & 31) == 0) P.pstat[pi] = make_float2(m, total);
        float4 *pa = reinterpret_cast<float4 *>(P.pacc + pi * kDim + d0);
        pa[0] = make_float4(a[0], a[1], a[2], a[3]);
        pa[1] = make_float4(a[4], a[5], a[6], a[7]);
    }
}

// Combine of many partitions (decode): block = (token, head, 32 dims); thread (partition
// group pg = t / 8 of 32, dims 4(t % 8)..+3) sums every 32nd partition, then the groups
// are summed through shuffles and LDS.
__global__ __launch_bounds__(256) void attn_combine_wide_kernel(AttnParams P) {
    __shared__ float red[4][8][5];
    __shared__ float wmax[4];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int th = blockIdx.x >> 3, tok = th / kHeads, head = th - tok * kHeads;
    const int d0 = 32 * (blockIdx.x & 7) + 4 * (t & 7), pg = t >> 3;
    const int np = (P.position + tok) / P.partition + 1;
    const size_t pi = (size_t)th * P.nparts;
    const float2 *st = P.pstat + pi;
    // eight of the group's partitions at a time, their loads issued together. Up to 256
    // partitions (32K keys) the partial rows are loaded with the statistics, before the
    // maximum is known: one global round trip instead of two.
    constexpr int U = 8;
    const bool one = np <= 32 * U;
    float m = -INFINITY;
    float2 sv[U];
    float4 av[U];
    for (int p0 = pg; p0 < np; p0 += 32 * U) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int p = min(p0 + 32 * u, np - 1);
            sv[u] = st[p];
            if (one) av[u] = *reinterpret_cast<const float4 *>(P.pacc + (pi + p) * kDim + d0);
        }
#pragma unroll
        for (int u = 0; u < U; u++) m = fmaxf(m, sv[u].x);
    }
    m = wave_max(m);
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    float total = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (one && pg < np) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float w = pg + 32 * u < np ? exp2f(sv[u].x - m) : 0.f;
            total += w * sv[u].y;
            acc.x += w * av[u].x; acc.y += w * av[u].y; acc.z += w * av[u].z; acc.w += w * av[u].w;
        }
    }
    for (int p0 = one ? np : pg; p0 < np; p0 += 32 * U) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int p = min(p0 + 32 * u, np - 1);
            sv[u] = st[p];
            av[u] = *reinterpret_cast<const float4 *>(P.pacc + (pi + p) * kDim + d0);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float w = p0 + 32 * u < np ? exp2f(sv[u].x - m) : 0.f;
            total += w * sv[u].y;
            acc.x += w * av[u].x; acc.y += w * av[u].y; acc.z += w * av[u].z; acc.w += w * av[u].w;
        }
    }
    // the eight groups of a wave: lanes 8 apart
#pragma unroll
    for (int s = 8; s < 64; s <<= 1) {
        total += __shfl_xor(total, s, 64);
        acc.x += __shfl_xor(acc.x, s, 64); acc.y += __shfl_xor(acc.y, s, 64);
        acc.z += __shfl_xor(acc.z, s, 64); acc.w += __shfl_xor(acc.w, s, 64);
    }
    if (lane < 8) {
        red[wave][lane][0] = acc.x; red[wave][lane][1] = acc.y; red[wave][lane][2] = acc.z;
        red[wave][lane][3] = acc.w; red[wave][lane][4] = total;
    }
    __syncthreads();
    if (t < 8) {
        float s5[5];
#pragma unroll
        for (int k = 0; k < 5; k++) s5[k] = red[0][t][k] + red[1][t][k] + red[2][t][k] + red[3][t][k];
        const float a4[4] = {s5[0], s5[1], s5[2], s5[3]};
        store_out4(P, tok, head, d0, a4, 1.f / s5[4]);
    }
}

}  // namespace

// Eight-wave blocks (32 tokens each) for chunks of more than one such tile; four-wave
// blocks (16 tokens) for decode and short chunks, whose rows would mostly sit idle.
static bool wide_blocks(int tokens) { return tokens > 2 * kTok; }

int attention_partition(int position, int tokens, int requested) {
    (void)position; (void)tokens;
    return requested > 0 ? requested : kDefaultRound;
}

int attention_split(int position, int tokens, int round) {
    // one decode token: the decode kernels (128-key blocks of 32-key tiles); their own
    // rounding when the partition is one tile, else the scores pass first
    if (tokens == 1 && (round == kKeys || (round % kDecKeys == 0 && round <= kMaxPremaxRound))) return kKeys;
    const bool wide = wide_blocks(tokens);
    const int tile_tokens = wide ? 2 * kTok : kTok;
    const int ntiles = (tokens + tile_tokens - 1) / tile_tokens;
    const int keys = position + tokens;
    int part;
    if (ntiles == 1) {
        // short chunks: the key stream is latency-bound; about 128 partitions per KV head
        // of at least 128 keys (measured best at 8K and 32K positions)
        part = std::max(128, (((keys + 127) / 128) + 127) / 128 * 128);
    } else {
        // (tile, KV head, partition) items: eight-wave blocks, one resident per CU, take one
        // round of the 256-CU part (measured at 16K and 32K positions: 8 partitions of 4096
        // keys 1.33 ms, 4 of 8192 1.19 ms, 2 of 16384 1.12 ms for the last 2048-token chunk
        // of a 32K prompt); four-wave blocks two per CU, more when the keys are long
        const int items = ntiles * kKvHeads;
        const int target = wide ? 256 : 512 * std::min(4, std::max(1, keys / 8192));
        if (items >= target) {
            part = ((keys + kKeys - 1) / kKeys) * kKeys;
        } else {
            const int parts = (target + items - 1) / items;
            part = std::max(256, ((keys + parts - 1) / parts + 255) / 256 * 256);
        }
    }
    // work partitions hold whole rounding partitions (one partition may cover every key)
    if (part >= keys) return ((keys + kKeys - 1) / kKeys) * kKeys;
    return (part + round - 1) / round * round;
}

int attention_partials(int position, int tokens, int partition) {
    if (tokens == 1 && partition == kKeys) return (position + kDecKeys) / kDecKeys;   // decode blocks
    return (position + tokens + partition - 1) / partition;
}

size_t attention_score_floats(int position, int tokens, int round, int partition) {
    if (tokens != 1 || partition != kKeys || round == kKeys) return 0;
    const size_t tiles = 4 * (size_t)attention_partials(position, tokens, partition);
    return kKvHeads * tiles * (32 * 8 + 8);
}

bool launch_attention(const AttentionArgs &a, hipStream_t s, char *error, int capacity) {
    AttnParams P;
    P.q = a.q; P.q_bf16 = a.q_bf16;
    P.keys = a.keys; P.values = a.values;
    P.gate = a.gate; P.gate_bf16 = a.gate_bf16;
    P.out = a.out; P.out_bf16 = a.out_bf16;
    P.pacc = a.pacc; P.pstat = reinterpret_cast<float2 *>(a.pstat);
    P.position = a.position; P.tokens = a.tokens; P.partition = a.partition; P.round = a.round;
    P.scores = a.scores; P.tmax = nullptr;
    P.nparts = attention_partials(a.position, a.tokens, a.partition);
    if (P.round < kKeys || P.round % kKeys != 0 || (a.partition != kKeys && a.partition % P.round != 0 &&
                                                    a.partition < a.position + a.tokens)) {
        set_error(error, capacity, "Attention work partitions must hold whole rounding partitions");
        return false;
    }
    const bool wide = wide_blocks(a.tokens);
    P.ntiles = (a.tokens + (wide ? 2 * kTok : kTok) - 1) / (wide ? 2 * kTok : kTok);
    if (P.nparts > 1 && (!P.pacc || !P.pstat)) {
        set_error(error, capacity, "Attention partitions need partial buffers");
        return false;
    }
    if (a.tokens == 1 && a.partition == kKeys) {
        // decode: four 32-key tiles a block, merged there; the blocks' partial results are
        // combined by (token, head, 32 dims)
        P.partition = kDecKeys;
        const dim3 grid(2 * ((P.nparts + 3) / 4 * 4));
        if (P.round != kKeys) {
            if (!P.scores) {
                set_error(error, capacity, "Decode attention with rounding partitions needs a score buffer");
                return false;
            }
            P.tmax = P.scores + (size_t)kKvHeads * 4 * P.nparts * 32 * 8;
            prof_stage("attention_scores");
            if (P.q_bf16)
                DIH_LAUNCH(attn_decode_scores_kernel<true>, grid, dim3(256), 0, s, P);
            else
                DIH_LAUNCH(attn_decode_scores_kernel<false>, grid, dim3(256), 0, s, P);
            if (!hip_ok(hipGetLastError(), error, capacity, "attention scores launch")) return false;
        }
        prof_stage("attention");
        if (P.round != kKeys) {
            if (P.q_bf16)
                DIH_LAUNCH((attn_decode_kernel<true, true>), grid, dim3(256), 0, s, P);
            else
                DIH_LAUNCH((attn_decode_kernel<false, true>), grid, dim3(256), 0, s, P);
        } else if (P.q_bf16) {
            DIH_LAUNCH((attn_decode_kernel<true, false>), grid, dim3(256), 0, s, P);
        } else {
            DIH_LAUNCH((attn_decode_kernel<false, false>), grid, dim3(256), 0, s, P);
        }
        if (!hip_ok(hipGetLastError(), error, capacity, "attention launch")) return false;
        if (P.nparts > 1) {
            prof_stage("attention_combine");
            DIH_LAUNCH(attn_combine_wide_kernel, dim3(kHeads * 8), dim3(256), 0, s, P);
            if (!hip_ok(hipGetLastError(), error, capacity, "attention combine launch")) return false;
        }
        return true;
    }
    const int per = ((P.ntiles * P.nparts + 3) / 4) * 4;
    // blocks whose keys span one rounding partition run the plain online softmax
    const bool restarts = P.partition > P.round;
    prof_stage("attention");
    if (wide && restarts)
        DIH_LAUNCH(attn8_kernel<true>, dim3(2 * per), dim3(512), 0, s, P);
    else if (wide)
        DIH_LAUNCH(attn8_kernel<false>, dim3(2 * per), dim3(512), 0, s, P);
    else if (restarts)
        DIH_LAUNCH(attn_kernel<true>, dim3(2 * per), dim3(256), 0, s, P);
    else
        DIH_LAUNCH(attn_kernel<false>, dim3(2 * per), dim3(256), 0, s, P);
    if (!hip_ok(hipGetLastError(), error, capacity, "attention launch")) return false;
    if (P.nparts > 1) {
        prof_stage("attention_combine");
        DIH_LAUNCH(attn_combine_kernel, dim3((a.tokens * kHeads + 3) / 4), dim3(256), 0, s, P);
        if (!hip_ok(hipGetLastError(), error, capacity, "attention combine launch")) return false;
    }
    return true;
}

}  // namespace dih
