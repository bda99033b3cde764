// Decode GEMV kernels for MLX-affine 5/8-bit weights on gfx950 (wave64).
//
// Mapping: a row of C columns is split into C/32 lane chunks (32 codes = half of one
// affine group). `lpr` lanes (a power of two <= 64) share a row; a wave therefore works
// on 64/lpr rows ("a row group") at once and each lane owns CPL chunks of its row. Row sums
// use  sum_c (q_c*s_g + b_g)*x_c = s_g*sum_c q_c*x_c + b_g*sum_c x_c  per chunk, so the
// inner loop is one code extraction/convert and one FMA per code; sum_c x_c is computed
// once per lane per launch. This is the semantics of quant_rows / quant_dot
// (quantized.mm:83-144) and expert_gate_up (quantized.mm:148-189), re-tiled for wave64.
//
// Latency hiding: each wave keeps D row groups in flight in a register ring. The raw
// words of a row group (codes and the bf16 bit patterns of its scales and biases) stay
// untouched until the group is consumed, and every load is unconditional (row and chunk
// indices are clamped in bounds, out-of-range lanes are masked at the reduction), so the
// only wait before consuming ring slot d is for the loads issued before it: the D-1 later
// groups stay in flight. Waves walk their row groups strided by the number of waves of
// the slot, so the chip reads one contiguous region at a time.
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

constexpr int kMaxSeg = 4;
constexpr int kWavesTarget = 4096;   // 16 resident waves per CU on 256 CUs

struct QmvParams {
    QmvSeg seg[kMaxSeg];
    int start[kMaxSeg + 1];  // first block of each segment
    int lpr[kMaxSeg];
    int blocks_per_slot[kMaxSeg];
    int waves_per_slot[kMaxSeg];
    int iters[kMaxSeg];      // row groups per wave
    int nseg;
    Top8Source top8;
};

// Raw words of one row group for one lane.
template <int BITS, int CPL, bool GATED>
struct RawGroup {
    Chunk<BITS> w[CPL];
    Chunk<BITS> u[GATED ? CPL : 1];
    uint32_t s[CPL], b[CPL];
    uint32_t su[GATED ? CPL : 1], bu[GATED ? CPL : 1];
};

template <int BITS, int CPL, bool GATED, int D>
DIH_DEV void qmv_wave(const QmvSeg &S, int lpr, int slot, uint32_t e, bool bad_id, int wi, int W,
                      int K) {
    const int lane = threadIdx.x & 63;
    const int rpw = 64 / lpr;  // rows per row group
    const int g = lane / lpr, j = lane - g * lpr;
    const int nchunk = S.columns >> 5;
    const size_t wpr = (size_t)S.columns * BITS / 32, gpr = (size_t)(S.columns >> 6);
    const size_t ebase = (size_t)e * S.rows;
    int chc[CPL];
    bool valid[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const int ch = j + c * lpr;
        valid[c] = ch < nchunk;
        chc[c] = valid[c] ? ch : nchunk - 1;
    }

    auto load = [&](RawGroup<BITS, CPL, GATED> &st, int grp) {
        int r = grp * rpw + g;
        r = r < S.rows ? r : S.rows - 1;
        const size_t rowi = ebase + r;
        const uint32_t *wrow = S.p0 + rowi * wpr;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            load_chunk<BITS>(st.w[c], wrow, chc[c]);
            st.s[c] = S.s0[rowi * gpr + (chc[c] >> 1)];
            st.b[c] = S.b0[rowi * gpr + (chc[c] >> 1)];
            if constexpr (GATED) {
                load_chunk<BITS>(st.u[c], S.p1 + rowi * wpr, chc[c]);
                st.su[c] = S.s1[rowi * gpr + (chc[c] >> 1)];
                st.bu[c] = S.b1[rowi * gpr + (chc[c] >> 1)];
            }
        }
    };

    RawGroup<BITS, CPL, GATED> ring[D];
#pragma unroll
    for (int d = 0; d < D; d++) load(ring[d], wi + d * W);

    // This lane's activations and their chunk sums (zero for masked chunks).
    float xr[CPL][32];
    float xs[CPL];
    const void *xb = S.x_bf16
        ? (const void *)(static_cast<const uint16_t *>(S.x) + (size_t)slot * S.x_slot_stride)
        : (const void *)(static_cast<const float *>(S.x) + (size_t)slot * S.x_slot_stride);
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        load_x32(xr[c], xb, S.x_bf16, chc[c] * 32);
        xs[c] = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            xr[c][i] = valid[c] ? xr[c][i] : 0.f;
            xs[c] += xr[c][i];
        }
    }

    auto consume = [&](const RawGroup<BITS, CPL, GATED> &st, int grp) {
        const int r = grp * rpw + g;
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const float v = bf16_to_f32(st.s[c]) * chunk_dot<BITS>(st.w[c], xr[c]) + bf16_to_f32(st.b[c]) * xs[c];
            a += valid[c] ? v : 0.f;
            if constexpr (GATED) {
                const float vu = bf16_to_f32(st.su[c]) * chunk_dot<BITS>(st.u[c], xr[c]) + bf16_to_f32(st.bu[c]) * xs[c];
                b += valid[c] ? vu : 0.f;
            }
        }
        a = group_sum(a, lpr);
        if constexpr (GATED) b = group_sum(b, lpr);
        if (j == 0 && r < S.rows) {
            float v = a;
            if constexpr (GATED) v = siluf_(a) * b;
            if (bad_id) v = __builtin_nanf("");
            const size_t o = (size_t)slot * S.rows + r;
            if (S.y_bf16)
                static_cast<uint16_t *>(S.y)[o] = f32_to_bf16(v);
            else
                static_cast<float *>(S.y)[o] = v;
        }
    };

    for (int k0 = 0; k0 < K; k0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            consume(ring[d], wi + (k0 + d) * W);
            // refill with the group D iterations ahead (clamped in bounds past the end)
            if (D > 1 || k0 + D < K) load(ring[d], wi + (k0 + d + D) * W);
        }
    }
}

template <int BITS, int CPL, int D>
__global__ __launch_bounds__(256) void qmv_kernel(QmvParams P) {
    const int blk = blockIdx.x;
    int k = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; i++)
        if (i < P.nseg && blk >= P.start[i]) k = i;
    const QmvSeg &S = P.seg[k];
    const int local = blk - P.start[k];
    const int slot = local / P.blocks_per_slot[k];
    const int wi = (local - slot * P.blocks_per_slot[k]) * 4 + (threadIdx.x >> 6);
    const int W = P.waves_per_slot[k];
    if (wi >= W) return;
    const int lane = threadIdx.x & 63;

    // Expert of this slot: a device id, or top-8 of the router logits computed by this
    // wave (the first wave of the segment publishes ids/probs for the next kernel).
    uint32_t e = 0u;
    if (S.top8) {
        uint32_t ids[8];
        float probs[8];
        bool bad;
        wave_top8(P.top8.logits, P.top8.experts, ids, probs, bad);
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (q == slot) e = ids[q];
        if (local == 0 && threadIdx.x < 8) {
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (q == lane) { P.top8.ids[q] = ids[q]; P.top8.probs[q] = probs[q]; }
            if (lane == 0 && bad && P.top8.status) *P.top8.status = 1u;
        }
    } else if (S.ids) {
        e = S.ids[slot];
    }
    const bool bad_id = e >= (uint32_t)S.experts;
    if (bad_id) e = 0u;
    if (S.p1)
        qmv_wave<BITS, CPL, true, D>(S, P.lpr[k], slot, e, bad_id, wi, W, P.iters[k]);
    else
        qmv_wave<BITS, CPL, false, D>(S, P.lpr[k], slot, e, bad_id, wi, W, P.iters[k]);
}

static int pow2ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

bool launch_qmv(const QmvSeg *segs, int nseg, int bits, const Top8Source *top8, hipStream_t s,
                char *error, int capacity) {
    if (nseg < 1 || nseg > kMaxSeg) {
        set_error(error, capacity, "Invalid GEMV segment count");
        return false;
    }
    QmvParams P{};
    P.nseg = nseg;
    int cpl = 1;
    long groups[kMaxSeg];
    long total = 0;
    for (int i = 0; i < nseg; i++) {
        P.seg[i] = segs[i];
        if (segs[i].top8 && (!top8 || !top8->logits || segs[i].count != 8)) {
            set_error(error, capacity, "Router selection segment without logits");
            return false;
        }
        const int nchunk = segs[i].columns / 32;
        const int lpr = nchunk >= 64 ? 64 : pow2ceil(nchunk);
        const int c = (nchunk + 63) / 64;
        if (c > cpl) cpl = c;
        P.lpr[i] = lpr;
        groups[i] = (segs[i].rows + (64 / lpr) - 1) / (64 / lpr);
        total += groups[i] * segs[i].count;
    }
    // Row groups per wave: one while the launch has at most kWavesTarget row groups,
    // else enough that the waves number about kWavesTarget.
    const long per = std::max(1L, (total + kWavesTarget - 1) / kWavesTarget);
    int kmax = 1;
    int blocks = 0;
    for (int i = 0; i < nseg; i++) {
        const long w = (groups[i] + per - 1) / per;
        const long it = (groups[i] + w - 1) / w;
        P.waves_per_slot[i] = (int)w;
        P.iters[i] = (int)it;
        P.blocks_per_slot[i] = (int)((w + 3) / 4);
        if (it > kmax) kmax = (int)it;
        P.start[i] = blocks;
        blocks += P.blocks_per_slot[i] * segs[i].count;
    }
    P.start[nseg] = blocks;
    if (top8) P.top8 = *top8;
    // ring depth: up to four row groups in flight; wide rows (C > 2048) hold more
    // registers per group, so their depth is capped to stay clear of spills
    int depth = kmax >= 4 ? 4 : kmax >= 2 ? 2 : 1;
    if (cpl == 2 && depth > 2) depth = 2;
    if (cpl > 2) {
        cpl = 4;
        depth = 1;
    }
    dim3 grid(blocks), block(256);
#define DIH_QMV_CASE(B, C, D)                                                  \
    if (bits == B && cpl <= C && depth == D) {                                  \
        DIH_LAUNCH((qmv_kernel<B, C, D>), grid, block, 0, s, P);               \
        return hip_ok(hipGetLastError(), error, capacity, "qmv launch");       \
    }
    DIH_QMV_CASE(8, 1, 1) DIH_QMV_CASE(8, 1, 2) DIH_QMV_CASE(8, 1, 4)
    DIH_QMV_CASE(8, 2, 1) DIH_QMV_CASE(8, 2, 2) DIH_QMV_CASE(8, 4, 1)
    DIH_QMV_CASE(5, 1, 1) DIH_QMV_CASE(5, 1, 2) DIH_QMV_CASE(5, 1, 4)
    DIH_QMV_CASE(5, 2, 1) DIH_QMV_CASE(5, 2, 2) DIH_QMV_CASE(5, 4, 1)
#undef DIH_QMV_CASE
    set_error(error, capacity, "Unsupported GEMV shape");
    return false;
}

// Decode expert down projection for the eight selected slots fused with the MoE merge
// (quant_rows batched down + graph_merge_norm's weighted sum, gpu_graph.mm:48-61, and
// Qwen36Model.cs:242-244): y = sigmoid(sroute)*shared_out[h] + sum_{slot 0..7}
// p_slot * (down[e_slot][h] . act[slot]); residual[h] += y (f32 or bf16 storage).
// A block of eight waves owns ROWS output rows; wave w computes slot w for all of them
// (its activation chunk is loaded once), the slot results meet in LDS and the first ROWS
// threads merge them in slot order.
template <int BITS, int LPR>
__global__ __launch_bounds__(512) void moe_down_merge_kernel(
    const uint32_t *__restrict__ packed, const uint16_t *__restrict__ scales,
    const uint16_t *__restrict__ biases, int H, int I, const float *__restrict__ act,
    const uint32_t *__restrict__ ids, const float *__restrict__ probs,
    const float *__restrict__ shared_out, const float *__restrict__ sroute,
    void *__restrict__ residual, int residual_f32, float *__restrict__ route_out) {
    constexpr int GROUPS = 64 / LPR;                      // rows per pass of a wave
    constexpr int ROWS = GROUPS > 16 ? GROUPS : 16;       // output rows per block
    constexpr int PASSES = ROWS / GROUPS;
    __shared__ float part[8][ROWS];
    const int slot = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane / LPR, j = lane - g * LPR;
    const int nchunk = I >> 5;
    const size_t wpr = (size_t)I * BITS / 32, gpr = (size_t)(I >> 6);
    const int row0 = blockIdx.x * ROWS;
    const uint32_t e = ids[slot];
    // weights first: every pass of this wave in flight at once
    // raw words first (bf16 bit patterns converted only when consumed), every pass of this
    // wave in flight at once; lanes past the row's chunks load a clamped chunk and are masked
    const bool valid = j < nchunk;
    const int jc = valid ? j : nchunk - 1;
    Chunk<BITS> wc[PASSES];
    uint32_t sc[PASSES], bc[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        int h = row0 + p * GROUPS + g;
        h = h < H ? h : H - 1;
        const size_t rowi = (size_t)e * H + h;
        load_chunk<BITS>(wc[p], packed + rowi * wpr, jc);
        sc[p] = scales[rowi * gpr + (jc >> 1)];
        bc[p] = biases[rowi * gpr + (jc >> 1)];
    }
    float xr[32];
    float xs = 0.f;
    load_x32(xr, act + (size_t)slot * I, 0, jc * 32);
#pragma unroll
    for (int i = 0; i < 32; i++) xs += xr[i];
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        float v = bf16_to_f32(sc[p]) * chunk_dot<BITS>(wc[p], xr) + bf16_to_f32(bc[p]) * xs;
        v = valid ? v : 0.f;
        v = group_sum(v, LPR);
        if (j == 0) part[slot][p * GROUPS + g] = v;
    }
    __syncthreads();
    if (threadIdx.x < ROWS) {
        const int r = threadIdx.x, h = row0 + r;
        if (h < H) {
            const float sh = shared_out[h];
            float y = sh * sigmoidf_(sroute[0]);
#pragma unroll
            for (int q = 0; q < 8; q++) y += part[q][r] * probs[q];
            residual_store(residual, residual_f32, h, residual_load(residual, residual_f32, h) + y);
            if (route_out) {
#pragma unroll
                for (int q = 0; q < 8; q++) route_out[(size_t)q * H + h] = part[q][r];
                route_out[(size_t)8 * H + h] = sh;
            }
        }
    }
}

bool launch_moe_down_merge(const Matrix *down, const float *act, const uint32_t *ids,
                           const float *probs, const float *shared_out, const float *sroute,
                           void *residual, int residual_f32, float *route_out, hipStream_t s,
                           char *error, int capacity) {
    const int H = down->rows, I = down->columns;
    const int nchunk = I / 32;
    if (nchunk > 64) {
        set_error(error, capacity, "Down projection wider than 2048 columns is not supported");
        return false;
    }
    const int lpr = pow2ceil(nchunk);
    const int rows = std::max(16, 64 / lpr);
    const int blocks = (H + rows - 1) / rows;
#define DIH_DM_CASE(B, L)                                                                            \
    if (down->bits == B && lpr == L) {                                                               \
        DIH_LAUNCH((moe_down_merge_kernel<B, L>), dim3(blocks), dim3(512), 0, s, down->packed(),     \
                   down->scales(), down->biases(), H, I, act, ids, probs, shared_out, sroute,        \
                   residual, residual_f32, route_out);                                               \
        return hip_ok(hipGetLastError(), error, capacity, "down/merge launch");                      \
    }
    DIH_DM_CASE(8, 2) DIH_DM_CASE(8, 4) DIH_DM_CASE(8, 8) DIH_DM_CASE(8, 16) DIH_DM_CASE(8, 32) DIH_DM_CASE(8, 64)
    DIH_DM_CASE(5, 2) DIH_DM_CASE(5, 4) DIH_DM_CASE(5, 8) DIH_DM_CASE(5, 16) DIH_DM_CASE(5, 32) DIH_DM_CASE(5, 64)
#undef DIH_DM_CASE
    set_error(error, capacity, "Unsupported down projection width");
    return false;
}

// Full-matrix dequantization to bf16 (expanded_weights, prefill_bf16_expanded.mm:8-16):
// one thread per 32-code chunk.
template <int BITS>
__global__ void dequant_bf16_kernel(const uint32_t *packed, const uint16_t *scales,
                                    const uint16_t *biases, int rows, int columns, uint16_t *out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int nchunk = columns >> 5;
    if (i >= (size_t)rows * nchunk) return;
    const size_t r = i / nchunk;
    const int ch = (int)(i - r * nchunk);
    Chunk<BITS> c;
    load_chunk<BITS>(c, packed + r * ((size_t)columns * BITS / 32), ch);
    float s = bf16_to_f32(scales[r * (columns >> 6) + (ch >> 1)]);
    float b = bf16_to_f32(biases[r * (columns >> 6) + (ch >> 1)]);
    dih_bf16x8 op[4];
    chunk_to_bf16<BITS>(c, s, b, op);
    uint4 *o = reinterpret_cast<uint4 *>(out + r * columns + (size_t)ch * 32);
#pragma unroll
    for (int q = 0; q < 4; q++) o[q] = __builtin_bit_cast(uint4, op[q]);
}

bool launch_dequant_bf16(const Matrix *m, int expert, uint16_t *out, hipStream_t s, char *error,
                         int capacity) {
    const size_t off = (size_t)expert * m->rows;
    const size_t n = (size_t)m->rows * (m->columns / 32);
    dim3 grid((unsigned)((n + 255) / 256)), block(256);
    const uint32_t *p = m->packed() + off * m->words_per_row();
    const uint16_t *sc = m->scales() + off * m->groups_per_row();
    const uint16_t *bi = m->biases() + off * m->groups_per_row();
    if (m->bits == 8)
        DIH_LAUNCH((dequant_bf16_kernel<8>), grid, block, 0, s, p, sc, bi, m->rows, m->columns, out);
    else
        DIH_LAUNCH((dequant_bf16_kernel<5>), grid, block, 0, s, p, sc, bi, m->rows, m->columns, out);
    return hip_ok(hipGetLastError(), error, capacity, "dequant launch");
}

// One row to f32 (di_quant_embedding quantized.mm:384-397 / graph_embedding
// gpu_graph.mm:22-31): one thread per column.
__global__ void embedding_kernel(const uint32_t *packed, const uint16_t *scales,
                                 const uint16_t *biases, int bits, int columns, int token,
                                 float *out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= columns) return;
    const uint32_t *w = packed + (size_t)token * ((size_t)columns * bits / 32);
    uint32_t bit = (uint32_t)c * bits, at = bit >> 5, shift = bit & 31u;
    uint32_t q = w[at] >> shift;
    if (shift + bits > 32) q |= w[at + 1] << (32 - shift);
    q &= (1u << bits) - 1u;
    size_t p = (size_t)token * (columns >> 6) + (c >> 6);
    out[c] = (float)q * bf16_to_f32(scales[p]) + bf16_to_f32(biases[p]);
}

bool launch_embedding(const Matrix *m, int token, float *out, hipStream_t s, char *error,
                      int capacity) {
    DIH_LAUNCH(embedding_kernel, dim3((m->columns + 255) / 256), dim3(256), 0, s, m->packed(), m->scales(),
               m->biases(), m->bits, m->columns, token, out);
    return hip_ok(hipGetLastError(), error, capacity, "embedding launch");
}

}  // namespace dih
