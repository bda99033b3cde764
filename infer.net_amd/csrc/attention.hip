// Causal GQA attention of a prefill chunk (or one decode token) over a bf16 KV cache:
// prefill_attention_bf16 + graph_attention_combine (prefill_attention_bf16.mm:13-55,
// gpu_graph.mm:177-213; dispatch p_fused_attention, gpu_prefill.mm:552-570).
//
// Geometry (fixed by the model): 16 query heads, 2 KV heads (8 query heads per KV head),
// head dim 256. Cache rows [position][kv head][256] bf16; queries [token][16][256] f32 or
// bf16; gate source [token][16][512] (head h's gate at h*512+256); out [token][16][256].
//
// One block = 16 query tokens x the 8 heads of one KV head (128 rows) x one partition of
// keys; each of its 4 waves owns 32 rows (4 tokens x 8 heads). Per 32-key tile:
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
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {
namespace {

constexpr int kHeads = 16, kKvHeads = 2, kDim = 256, kGroup = kHeads / kKvHeads;
constexpr int kTok = 16;               // query tokens per block (128 rows)
constexpr int kKeys = 32;              // keys per tile
constexpr int kKsStride = kDim + 8;    // bf16 per key row in LDS: 528 B, 16 B aligned
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
};

DIH_DEV float load_any(const void *p, int bf16, size_t i) {
    return bf16 ? bf16_to_f32(static_cast<const uint16_t *>(p)[i]) : static_cast<const float *>(p)[i];
}

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

__global__ __launch_bounds__(256, 2) void attn_kernel(AttnParams P) {
    __shared__ __align__(16) uint16_t ks[kKeys * kKsStride];
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

    // ---- the wave's queries as MFMA B operands: qreg[s] = q[row][16s + 8h .. +8] in bf16
    dih_bf16x8 qreg[16];
    {
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

    // ---- tile loads. Keys: thread t copies 16 B (8 dims) of keys t/32 + 8i. Values: thread
    // t loads 8 dims (chunk t/8) of the 4 keys 4*(t%8) + i and writes them transposed.
    // Key indices past the partition end are clamped to its last key (finite data; those
    // keys are masked).
    const uint16_t *kbase = P.keys + kh * kDim, *vbase = P.values + kh * kDim;
    const int kc = t & 31, kr = t >> 5;
    const int vq = t & 7, vc = t >> 3;
    uint4 kreg[4], vreg[4];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = min(kb + kr + 8 * i, kend - 1);
            kreg[i] = *reinterpret_cast<const uint4 *>(kbase + (size_t)key * (kKvHeads * kDim) + 8 * kc);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = min(kb + 4 * vq + i, kend - 1);
            vreg[i] = *reinterpret_cast<const uint4 *>(vbase + (size_t)key * (kKvHeads * kDim) + 8 * vc);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<uint4 *>(ks + (kr + 8 * i) * kKsStride + 8 * kc) = kreg[i];
        const uint32_t w0[4] = {vreg[0].x, vreg[0].y, vreg[0].z, vreg[0].w};
        const uint32_t w1[4] = {vreg[1].x, vreg[1].y, vreg[1].z, vreg[1].w};
        const uint32_t w2[4] = {vreg[2].x, vreg[2].y, vreg[2].z, vreg[2].w};
        const uint32_t w3[4] = {vreg[3].x, vreg[3].y, vreg[3].z, vreg[3].w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // word w of each key holds dims 2w (low half) and 2w+1 (high half)
            uint2 lo, hi;
            lo.x = __builtin_amdgcn_perm(w1[w], w0[w], 0x05040100u);
            lo.y = __builtin_amdgcn_perm(w3[w], w2[w], 0x05040100u);
            hi.x = __builtin_amdgcn_perm(w1[w], w0[w], 0x07060302u);
            hi.y = __builtin_amdgcn_perm(w3[w], w2[w], 0x07060302u);
            *reinterpret_cast<uint2 *>(vt + (8 * vc + 2 * w) * kVtStride + 4 * vq) = lo;
            *reinterpret_cast<uint2 *>(vt + (8 * vc + 2 * w + 1) * kVtStride + 4 * vq) = hi;
        }
    };

    float m_run = -INFINITY, l_run = 0.f;
    dih_f32x16 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int k = 0; k < 16; k++) acc[i][k] = 0.f;

    load_tile(kstart);
    for (int kb = kstart; kb < kend; kb += kKeys) {
        __syncthreads();          // the previous tile's LDS reads are done
        store_tile();
        __syncthreads();
        if (kb + kKeys < kend) load_tile(kb + kKeys);
        if (!wave_ok || kb > wave_last) continue;

        // ---- S^T = K Q^T: s[k] is key kb + 8(k/4) + 4h + k%4 of row r
        dih_f32x16 s;
#pragma unroll
        for (int k = 0; k < 16; k++) s[k] = 0.f;
#pragma unroll
        for (int st = 0; st < 16; st++) {
            const dih_bf16x8 a = *reinterpret_cast<const dih_bf16x8 *>(ks + r * kKsStride + 16 * st + 8 * h);
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[st], s, 0, 0, 0);
        }
        // ---- online softmax for row r
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int key = kb + 8 * (k >> 2) + 4 * h + (k & 3);
            const bool ok = key <= my_last && key < kend;
            s[k] = ok ? s[k] * kLog2eOver16 : -INFINITY;
            mx = fmaxf(mx, s[k]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_run == -INFINITY ? 0.f : exp2f(m_run - m_new);
        float psum = 0.f;
        uint32_t pw[8];
#pragma unroll
        for (int k = 0; k < 16; k += 2) {
            const float p0 = s[k] == -INFINITY ? 0.f : exp2f(s[k] - m_new);
            const float p1 = s[k + 1] == -INFINITY ? 0.f : exp2f(s[k + 1] - m_new);
            psum += p0 + p1;
            pw[k >> 1] = pack_bf16x2(p0, p1);
        }
        psum += __shfl_xor(psum, 32, 64);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        const dih_bf16x8 pb0 = __builtin_bit_cast(dih_bf16x8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
        const dih_bf16x8 pb1 = __builtin_bit_cast(dih_bf16x8, make_uint4(pw[4], pw[5], pw[6], pw[7]));
        // ---- O^T = O^T * alpha + V^T P^T: acc[dt][k] is dim 32dt + 8(k/4) + 4h + k%4 of row r
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
#pragma unroll
            for (int k = 0; k < 16; k++) acc[dt][k] *= alpha;
            const uint16_t *vrow = vt + (32 * dt + r) * kVtStride + 4 * h;
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
    if (!row_ok) return;

    // ---- epilogue
    if (P.nparts == 1) {
        const float inv = 1.f / l_run;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float a4[4] = {acc[dt][4 * i], acc[dt][4 * i + 1], acc[dt][4 * i + 2], acc[dt][4 * i + 3]};
                store_out4(P, my_tok, head, 32 * dt + 8 * i + 4 * h, a4, inv);
            }
    } else {
        const size_t pi = ((size_t)my_tok * kHeads + head) * P.nparts + part;
        if (h == 0) P.pstat[pi] = make_float2(m_run, l_run);
        float *pa = P.pacc + pi * kDim;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                *reinterpret_cast<float4 *>(pa + 32 * dt + 8 * i + 4 * h) =
                    make_float4(acc[dt][4 * i], acc[dt][4 * i + 1], acc[dt][4 * i + 2], acc[dt][4 * i + 3]);
    }
}

// One block per (token, head), one thread per dim: merge the partitions that hold keys
// of this token (graph_attention_combine, gpu_graph.mm:199-213).
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams P) {
    const int th = blockIdx.x, tok = th / kHeads, head = th - tok * kHeads, d = threadIdx.x;
    const int np = (P.position + tok) / P.partition + 1;
    const size_t pi = ((size_t)tok * kHeads + head) * P.nparts;
    float m = -INFINITY;
    for (int p = 0; p < np; p++) m = fmaxf(m, P.pstat[pi + p].x);
    float total = 0.f, acc = 0.f;
    for (int p = 0; p < np; p++) {
        const float2 st = P.pstat[pi + p];
        const float w = exp2f(st.x - m);
        total += w * st.y;
        acc += w * P.pacc[(pi + p) * kDim + d];
    }
    const float v = acc / total * sigmoid_f(load_any(P.gate, P.gate_bf16,
                                                     (size_t)tok * (kHeads * 2 * kDim) + head * 2 * kDim + kDim + d));
    const size_t oi = (size_t)tok * (kHeads * kDim) + head * kDim + d;
    if (P.out_bf16)
        static_cast<uint16_t *>(P.out)[oi] = f32_to_bf16(v);
    else
        static_cast<float *>(P.out)[oi] = v;
}

}  // namespace

int attention_partition(int position, int tokens, int requested) {
    if (requested > 0) return requested;
    const int ntiles = (tokens + kTok - 1) / kTok;
    const int items = ntiles * kKvHeads;
    const int keys = position + tokens;
    // Enough (tile, head, partition) items for about two blocks per CU of a 256-CU part.
    constexpr int kTarget = 512;
    if (items >= kTarget) return ((keys + kKeys - 1) / kKeys) * kKeys;
    const int parts = (kTarget + items - 1) / items;
    int part = (keys + parts - 1) / parts;
    part = ((part + 255) / 256) * 256;
    return part < 256 ? 256 : part;
}

bool launch_attention(const AttentionArgs &a, hipStream_t s, char *error, int capacity) {
    AttnParams P;
    P.q = a.q; P.q_bf16 = a.q_bf16;
    P.keys = a.keys; P.values = a.values;
    P.gate = a.gate; P.gate_bf16 = a.gate_bf16;
    P.out = a.out; P.out_bf16 = a.out_bf16;
    P.pacc = a.pacc; P.pstat = reinterpret_cast<float2 *>(a.pstat);
    P.position = a.position; P.tokens = a.tokens; P.partition = a.partition;
    P.nparts = (a.position + a.tokens + a.partition - 1) / a.partition;
    P.ntiles = (a.tokens + kTok - 1) / kTok;
    if (P.nparts > 1 && (!P.pacc || !P.pstat)) {
        set_error(error, capacity, "Attention partitions need partial buffers");
        return false;
    }
    const int per = ((P.ntiles * P.nparts + 3) / 4) * 4;
    DIH_LAUNCH(attn_kernel, dim3(2 * per), dim3(256), 0, s, P);
    if (!hip_ok(hipGetLastError(), error, capacity, "attention launch")) return false;
    if (P.nparts > 1) {
        DIH_LAUNCH(attn_combine_kernel, dim3(a.tokens * kHeads), dim3(256), 0, s, P);
        if (!hip_ok(hipGetLastError(), error, capacity, "attention combine launch")) return false;
    }
    return true;
}

}  // namespace dih
