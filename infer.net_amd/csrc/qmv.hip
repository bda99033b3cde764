// Decode GEMV kernels for MLX-affine 5/8-bit weights on gfx950 (wave64).
//
// Mapping: a row of C columns is split into C/32 lane chunks (32 codes = half of one
// affine group). `lpr` lanes (a power of two <= 64) share a row; a wave therefore works
// on 64/lpr rows at once and each lane owns CPL chunks of its row. Row sums use the
// identity  sum_c (q_c*s_g + b_g)*x_c = s_g*sum_c q_c*x_c + b_g*sum_c x_c  per chunk, so
// the inner loop is one code extraction/convert and one FMA per code; sum_c x_c is
// computed once per lane per launch. This is the semantics of quant_rows / quant_dot
// (quantized.mm:83-144) and expert_gate_up (quantized.mm:148-189), re-tiled for wave64
// and 16-byte loads rather than translated.
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

constexpr int kMaxSeg = 4;
constexpr int kRowsPerLaneGroup = 2;  // rows in flight per lane group

struct QmvParams {
    QmvSeg seg[kMaxSeg];
    int start[kMaxSeg + 1];  // first block of each segment
    int lpr[kMaxSeg];
    int blocks_per_slot[kMaxSeg];
    int nseg;
    Top8Epilogue top8;
};

// Top-8 of up to 256 logits by one wave (graph_top8 gpu_graph.mm:134-146 semantics:
// repeated wave max, ties to the lowest id; softmax over the chosen eight with the
// first (largest) subtracted, summed in slot order).
DIH_DEV void wave_top8(const float *logits, int experts, uint32_t *ids, float *probs,
                       uint32_t *status, int lane) {
    float cand[4];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int e = lane + 64 * j;
        float v = e < experts ? logits[e] : -INFINITY;
        if (e < experts && !isfinite(v)) bad = true;
        cand[j] = v;
    }
    bool any_bad = __any(bad);
    float chosen[8];
    uint32_t picked[8];
#pragma unroll
    for (int n = 0; n < 8; n++) {
        float best = cand[0];
        uint32_t id = (uint32_t)lane;
#pragma unroll
        for (int j = 1; j < 4; j++)
            if (cand[j] > best) { best = cand[j]; id = (uint32_t)(lane + 64 * j); }
        float m = wave_max(best);
        uint32_t sel = wave_min_u32(best == m ? id : 0xffffffffu);
        chosen[n] = m;
        picked[n] = sel;
        if ((int)(sel & 63u) == lane) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if ((uint32_t)(lane + 64 * j) == sel) cand[j] = -INFINITY;
        }
    }
    if (lane == 0) {
        float p[8], total = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) { p[i] = __expf(chosen[i] - chosen[0]); total += p[i]; }
#pragma unroll
        for (int i = 0; i < 8; i++) { ids[i] = any_bad ? 0u : picked[i]; probs[i] = p[i] / total; }
        if (status && any_bad) *status = 1u;
    }
}

template <int BITS, int CPL>
__global__ __launch_bounds__(256) void qmv_kernel(QmvParams P) {
    const int blk = blockIdx.x;
    int k = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; i++)
        if (i < P.nseg && blk >= P.start[i]) k = i;
    const QmvSeg &S = P.seg[k];
    const int lpr = P.lpr[k];
    const int local = blk - P.start[k];
    const int slot = local / P.blocks_per_slot[k];
    const int rb = local - slot * P.blocks_per_slot[k];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rpw = 64 / lpr;  // row groups per wave
    const int g = lane / lpr, j = lane - g * lpr;
    const int nchunk = S.columns >> 5;
    const int rows_per_block = 4 * rpw * kRowsPerLaneGroup;
    uint32_t e = S.ids ? S.ids[slot] : 0u;
    const bool bad_id = e >= (uint32_t)S.experts;
    if (bad_id) e = 0u;
    const size_t wpr = (size_t)S.columns * BITS / 32, gpr = (size_t)(S.columns >> 6);

    // This lane's activations and their chunk sums.
    float xr[CPL][32];
    float xs[CPL];
    const void *xb = S.x_bf16
        ? (const void *)(static_cast<const uint16_t *>(S.x) + (size_t)slot * S.x_slot_stride)
        : (const void *)(static_cast<const float *>(S.x) + (size_t)slot * S.x_slot_stride);
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const int ch = j + c * lpr;
        xs[c] = 0.f;
        if (ch < nchunk) {
            load_x32(xr[c], xb, S.x_bf16, ch * 32);
#pragma unroll
            for (int i = 0; i < 32; i++) xs[c] += xr[c][i];
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) xr[c][i] = 0.f;
        }
    }

    const bool gated = S.p1 != nullptr;
    int rows[kRowsPerLaneGroup];
    Chunk<BITS> wc[kRowsPerLaneGroup][CPL], uc[kRowsPerLaneGroup][CPL];
    float sc[kRowsPerLaneGroup][CPL], bc[kRowsPerLaneGroup][CPL];
    float su[kRowsPerLaneGroup][CPL], bu[kRowsPerLaneGroup][CPL];
#pragma unroll
    for (int u = 0; u < kRowsPerLaneGroup; u++) {
        int r = rb * rows_per_block + (wave * kRowsPerLaneGroup + u) * rpw + g;
        rows[u] = r;
        int rr = r < S.rows ? r : S.rows - 1;
        const size_t rowi = (size_t)e * S.rows + rr;
        const uint32_t *wrow = S.p0 + rowi * wpr;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int ch = j + c * lpr;
            if (ch < nchunk) {
                load_chunk<BITS>(wc[u][c], wrow, ch);
                sc[u][c] = bf16_to_f32(S.s0[rowi * gpr + (ch >> 1)]);
                bc[u][c] = bf16_to_f32(S.b0[rowi * gpr + (ch >> 1)]);
                if (gated) {
                    load_chunk<BITS>(uc[u][c], S.p1 + rowi * wpr, ch);
                    su[u][c] = bf16_to_f32(S.s1[rowi * gpr + (ch >> 1)]);
                    bu[u][c] = bf16_to_f32(S.b1[rowi * gpr + (ch >> 1)]);
                }
            }
        }
    }
#pragma unroll
    for (int u = 0; u < kRowsPerLaneGroup; u++) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int ch = j + c * lpr;
            if (ch < nchunk) {
                a += sc[u][c] * chunk_dot<BITS>(wc[u][c], xr[c]) + bc[u][c] * xs[c];
                if (gated) b += su[u][c] * chunk_dot<BITS>(uc[u][c], xr[c]) + bu[u][c] * xs[c];
            }
        }
        a = group_sum(a, lpr);
        if (gated) b = group_sum(b, lpr);
        if (j == 0 && rows[u] < S.rows) {
            float v = bad_id ? __builtin_nanf("") : (gated ? siluf_(a) * b : a);
            size_t o = (size_t)slot * S.rows + rows[u];
            if (S.y_bf16)
                static_cast<uint16_t *>(S.y)[o] = f32_to_bf16(v);
            else
                static_cast<float *>(S.y)[o] = v;
        }
    }

    if (P.top8.ticket) {
        __shared__ int last;
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned t = atomicAdd(P.top8.ticket, 1u);
            last = (t == gridDim.x - 1);
        }
        __syncthreads();
        if (last) {
            __threadfence();
            if (wave == 0) {
                wave_top8(P.top8.logits, P.top8.experts, P.top8.ids, P.top8.probs,
                          P.top8.status, lane);
                if (lane == 0) *P.top8.ticket = 0u;
            }
        }
    }
}

static int pow2ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

bool launch_qmv(const QmvSeg *segs, int nseg, int bits, const Top8Epilogue *top8,
                hipStream_t s, char *error, int capacity) {
    if (nseg < 1 || nseg > kMaxSeg) {
        set_error(error, capacity, "Invalid GEMV segment count");
        return false;
    }
    QmvParams P{};
    P.nseg = nseg;
    int cpl = 1, blocks = 0;
    for (int i = 0; i < nseg; i++) {
        P.seg[i] = segs[i];
        int nchunk = segs[i].columns / 32;
        int lpr = nchunk >= 64 ? 64 : pow2ceil(nchunk);
        int c = (nchunk + 63) / 64;
        if (c > cpl) cpl = c;
        P.lpr[i] = lpr;
        int rows_per_block = 4 * (64 / lpr) * kRowsPerLaneGroup;
        P.blocks_per_slot[i] = (segs[i].rows + rows_per_block - 1) / rows_per_block;
        P.start[i] = blocks;
        blocks += P.blocks_per_slot[i] * segs[i].count;
    }
    P.start[nseg] = blocks;
    if (top8) P.top8 = *top8;
    dim3 grid(blocks), block(256);
#define DIH_QMV_CASE(B, C)                                                   \
    if (bits == B && cpl <= C) {                                             \
        hipLaunchKernelGGL((qmv_kernel<B, C>), grid, block, 0, s, P);        \
        return hip_ok(hipGetLastError(), error, capacity, "qmv launch");     \
    }
    DIH_QMV_CASE(8, 1)
    DIH_QMV_CASE(8, 2)
    DIH_QMV_CASE(8, 4)
    DIH_QMV_CASE(5, 1)
    DIH_QMV_CASE(5, 2)
    DIH_QMV_CASE(5, 4)
#undef DIH_QMV_CASE
    set_error(error, capacity, "Unsupported GEMV shape");
    return false;
}

// Decode expert down projection for the eight selected slots fused with the MoE merge
// (quant_rows batched down + graph_merge_norm's weighted sum, gpu_graph.mm:48-61, and
// Qwen36Model.cs:242-244): y = sigmoid(sroute)*shared_out[h] + sum_{slot 0..7}
// p_slot * (down[e_slot][h] . act[slot]); residual[h] = bf16(residual[h] + y).
// lpr lanes per slot-row; a wave covers 64/lpr slots per pass.
template <int BITS>
__global__ __launch_bounds__(256) void moe_down_merge_kernel(
    const uint32_t *__restrict__ packed, const uint16_t *__restrict__ scales,
    const uint16_t *__restrict__ biases, int H, int I, const float *__restrict__ act,
    const uint32_t *__restrict__ ids, const float *__restrict__ probs,
    const float *__restrict__ shared_out, const float *__restrict__ sroute,
    uint16_t *__restrict__ residual, float *__restrict__ route_out, int lpr, int rows_per_wave) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int groups = 64 / lpr, g = lane / lpr, j = lane - g * lpr;
    const int nchunk = I >> 5;
    const int passes = (8 + groups - 1) / groups;
    const size_t wpr = (size_t)I * BITS / 32, gpr = (size_t)(I >> 6);
    const int row0 = (blockIdx.x * 4 + wave) * rows_per_wave;
    for (int rr = 0; rr < rows_per_wave; rr++) {
        const int h = row0 + rr;
        if (h >= H) break;
        float mine[8];
#pragma unroll
        for (int p = 0; p < 8; p++) mine[p] = 0.f;
        for (int p = 0; p < passes; p++) {
            const int slot = p * groups + g;
            float v = 0.f;
            if (slot < 8 && j < nchunk) {
                const uint32_t e = ids[slot];
                const size_t rowi = (size_t)e * H + h;
                Chunk<BITS> wc;
                load_chunk<BITS>(wc, packed + rowi * wpr, j);
                float xr[32];
                load_x32(xr, act + (size_t)slot * I, 0, j * 32);
                float xs = 0.f;
#pragma unroll
                for (int i = 0; i < 32; i++) xs += xr[i];
                v = bf16_to_f32(scales[rowi * gpr + (j >> 1)]) * chunk_dot<BITS>(wc, xr) +
                    bf16_to_f32(biases[rowi * gpr + (j >> 1)]) * xs;
            }
            v = group_sum(v, lpr);
            // gather slot results of this pass into every lane
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (q / groups == p) mine[q] = __shfl(v, (q % groups) * lpr, 64);
        }
        if (lane == 0) {
            float y = shared_out[h] * sigmoidf_(sroute[0]);
#pragma unroll
            for (int q = 0; q < 8; q++) y += mine[q] * probs[q];
            residual[h] = f32_to_bf16(bf16_to_f32(residual[h]) + y);
            if (route_out) {
#pragma unroll
                for (int q = 0; q < 8; q++) route_out[(size_t)q * H + h] = mine[q];
                route_out[(size_t)8 * H + h] = shared_out[h];
            }
        }
    }
}

bool launch_moe_down_merge(const Matrix *down, const float *act, const uint32_t *ids,
                           const float *probs, const float *shared_out, const float *sroute,
                           uint16_t *residual, float *route_out, hipStream_t s, char *error,
                           int capacity) {
    const int H = down->rows, I = down->columns;
    int nchunk = I / 32;
    if (nchunk > 64) {
        set_error(error, capacity, "Down projection wider than 2048 columns is not supported");
        return false;
    }
    int lpr = pow2ceil(nchunk);
    const int rows_per_wave = 2;
    int blocks = (H + 4 * rows_per_wave - 1) / (4 * rows_per_wave);
    if (down->bits == 8)
        hipLaunchKernelGGL((moe_down_merge_kernel<8>), dim3(blocks), dim3(256), 0, s, down->packed(),
                           down->scales(), down->biases(), H, I, act, ids, probs, shared_out, sroute,
                           residual, route_out, lpr, rows_per_wave);
    else
        hipLaunchKernelGGL((moe_down_merge_kernel<5>), dim3(blocks), dim3(256), 0, s, down->packed(),
                           down->scales(), down->biases(), H, I, act, ids, probs, shared_out, sroute,
                           residual, route_out, lpr, rows_per_wave);
    return hip_ok(hipGetLastError(), error, capacity, "down/merge launch");
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
        hipLaunchKernelGGL((dequant_bf16_kernel<8>), grid, block, 0, s, p, sc, bi, m->rows, m->columns, out);
    else
        hipLaunchKernelGGL((dequant_bf16_kernel<5>), grid, block, 0, s, p, sc, bi, m->rows, m->columns, out);
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
    hipLaunchKernelGGL(embedding_kernel, dim3((m->columns + 255) / 256), dim3(256), 0, s,
                       m->packed(), m->scales(), m->biases(), m->bits, m->columns, token, out);
    return hip_ok(hipGetLastError(), error, capacity, "embedding launch");
}

}  // namespace dih
