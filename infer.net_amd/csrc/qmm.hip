// Grouped (MoE) and dense quantized GEMM on gfx950 bf16 MFMA.
//
// Each block owns 128 weight rows (four waves x 32 rows) of one expert and one chunk
// of up to 32*NT routes of that expert. Every wave computes a 32-row x 32*NT-route tile
// with v_mfma_f32_32x32x16_bf16 and fp32 accumulators over K in 64-column affine
// groups.
//
// K permutation (no LDS needed for the weights): MFMA j (j = 0..3) of a 64-column group
// takes its 16 K-slots from columns {32h + 8j + i : h in {0,1}, i in 0..7}, where h is
// the lane's half of the wave. Then lane (row r, half h) needs exactly the 32
// consecutive codes [32h, 32h+32) of its row in that group (one Chunk: 32 bytes 8-bit,
// 20 bytes 5-bit) and lane (route n, half h) needs the 32 consecutive bf16 activations
// [32h, 32h+32) of its route. Both are dequantized/loaded straight into MFMA operand
// registers. Dequantized weights are bf16(fp32(q*scale+bias)) with round-to-nearest-even
// and activations are bf16, so operand values match the reference's BF16 path
// (prefill_expert_packed.mm:24-35, 64-65); accumulation order differs (fp32).
//
// Work order: the route chunks are listed expert by expert (ascending), chunks of one
// expert consecutive. Logical block L = rowtile * n_chunks + chunk, and physical block b
// runs logical (b % 8) * ceil(n_work / 8) + b / 8, so consecutive logical blocks land on
// the same XCD at nearly the same time: chunks of one popular expert then share that
// expert's weight rows in the XCD's L2. Blocks past n_work exit at once, which replaces
// the reference's indirect dispatch (prefill_group_dispatch, prefill_moe.mm:18-22).
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

struct QmmParams {
    const uint32_t *p0, *p1; const uint16_t *s0, *s1, *b0, *b1;     // routed
    const uint32_t *sp0, *sp1; const uint16_t *ss0, *ss1, *sb0, *sb1;  // shared expert
    int experts, rows, columns, tokens, dense, in_mode, y_bf16, row_tiles;
    const uint32_t *routes; const int4 *chunks; const uint32_t *nchunks;
    const uint16_t *x; void *y;
};

template <int BITS>
struct KStep {
    Chunk<BITS> a0, a1;
    float s0, bb0, s1, bb1;
};

template <int BITS, bool GATED, int NT>
__global__ __launch_bounds__(256, 2) void qmm_kernel(QmmParams P) {
    const int n_chunks = P.dense ? (P.tokens + 63) / 64 : (int)*P.nchunks;
    const int n_work = P.row_tiles * n_chunks;
    const int per = (n_work + 7) / 8;
    const int b = blockIdx.x;
    const int jj = b >> 3;
    if (jj >= per) return;
    const int L = (b & 7) * per + jj;
    if (L >= n_work) return;
    const int rt = L / n_chunks, ci = L - rt * n_chunks;

    int e, start, nvalid;
    if (P.dense) {
        e = 0; start = ci * 64; nvalid = min(64, P.tokens - start);
    } else {
        int4 c = P.chunks[ci];
        e = c.x; start = c.y; nvalid = c.z;
    }
    const bool shared = !P.dense && e == P.experts;
    const uint32_t *pw0 = shared ? P.sp0 : P.p0;
    const uint16_t *ps0 = shared ? P.ss0 : P.s0, *pb0 = shared ? P.sb0 : P.b0;
    const uint32_t *pw1 = shared ? P.sp1 : P.p1;
    const uint16_t *ps1 = shared ? P.ss1 : P.s1, *pb1 = shared ? P.sb1 : P.b1;
    const int eix = shared ? 0 : e;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
    const int R = P.rows, C = P.columns, G = C >> 6;
    const int row = rt * 128 + wave * 32 + r;
    const int rr = row < R ? row : R - 1;
    const size_t rowi = (size_t)eix * R + rr;
    const size_t wpr = (size_t)C * BITS / 32;
    const uint32_t *w0 = pw0 + rowi * wpr;
    const uint32_t *w1 = GATED ? pw1 + rowi * wpr : nullptr;
    const uint16_t *sc0 = ps0 + rowi * G, *bi0 = pb0 + rowi * G;
    const uint16_t *sc1 = GATED ? ps1 + rowi * G : nullptr, *bi1 = GATED ? pb1 + rowi * G : nullptr;

    // Route of each of this lane's columns (one per tile) and its input row.
    const int T8 = P.tokens * 8;
    const uint32_t *rlist = P.dense ? nullptr : P.routes + (size_t)e * P.tokens + start;
    const uint16_t *xrow[NT];
    int ntiles = (nvalid + 31) >> 5;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        int n = t * 32 + r;
        int nn = n < nvalid ? n : 0;
        int route = P.dense ? start + nn : (int)rlist[nn];
        int in_row = route;
        if (P.in_mode == 1) in_row = route < T8 ? (route >> 3) : route - T8;
        xrow[t] = P.x + (size_t)in_row * C + 32 * h;
    }

    dih_f32x16 acc0[NT], acc1[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
        for (int i = 0; i < 16; i++) { acc0[t][i] = 0.f; acc1[t][i] = 0.f; }
    }

    KStep<BITS> cur, nxt;
    auto load_step = [&](KStep<BITS> &k, int kg) {
        load_chunk<BITS>(k.a0, w0, 2 * kg + h);
        k.s0 = bf16_to_f32(sc0[kg]);
        k.bb0 = bf16_to_f32(bi0[kg]);
        if constexpr (GATED) {
            load_chunk<BITS>(k.a1, w1, 2 * kg + h);
            k.s1 = bf16_to_f32(sc1[kg]);
            k.bb1 = bf16_to_f32(bi1[kg]);
        }
    };
    uint4 xb[NT][4], xn[NT][4];
    auto load_x = [&](uint4 (&dst)[NT][4], int kg) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t < ntiles) {
                const uint4 *p = reinterpret_cast<const uint4 *>(xrow[t] + 64 * kg);
#pragma unroll
                for (int q = 0; q < 4; q++) dst[t][q] = p[q];
            }
        }
    };

    load_step(cur, 0);
    load_x(xb, 0);
    for (int kg = 0; kg < G; kg++) {
        if (kg + 1 < G) {
            load_step(nxt, kg + 1);
            load_x(xn, kg + 1);
        }
        dih_bf16x8 a0[4], a1[4];
        chunk_to_bf16<BITS>(cur.a0, cur.s0, cur.bb0, a0);
        if constexpr (GATED) chunk_to_bf16<BITS>(cur.a1, cur.s1, cur.bb1, a1);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t < ntiles) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    dih_bf16x8 bx = __builtin_bit_cast(dih_bf16x8, xb[t][j]);
                    acc0[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[j], bx, acc0[t], 0, 0, 0);
                    if constexpr (GATED)
                        acc1[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[j], bx, acc1[t], 0, 0, 0);
                }
            }
        }
        if (kg + 1 < G) {
            cur = nxt;
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) xb[t][q] = xn[t][q];
        }
    }

    // Epilogue: lane holds column n = t*32 + r, rows 8*(i/4) + 4h + (i%4) of the tile.
    const int row_base = rt * 128 + wave * 32;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int n = t * 32 + r;
        if (t >= ntiles || n >= nvalid) continue;
        const int route = P.dense ? start + n : (int)rlist[n];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int m0 = row_base + 8 * q + 4 * h;
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float g = acc0[t][4 * q + k];
                v[k] = GATED ? siluf_(g) * acc1[t][4 * q + k] : g;
            }
            const size_t o = (size_t)route * R + m0;
            // vector stores only where the row offset keeps them naturally aligned
            if ((R & 3) == 0 && m0 + 3 < R) {
                if (P.y_bf16) {
                    uint2 pk = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(P.y) + o) = pk;
                } else {
                    *reinterpret_cast<float4 *>(static_cast<float *>(P.y) + o) =
                        make_float4(v[0], v[1], v[2], v[3]);
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if (m0 + k < R) {
                        if (P.y_bf16)
                            static_cast<uint16_t *>(P.y)[o + k] = f32_to_bf16(v[k]);
                        else
                            static_cast<float *>(P.y)[o + k] = v[k];
                    }
                }
            }
        }
    }
}

bool launch_qmm(const QmmArgs &a, hipStream_t s, char *error, int capacity) {
    QmmParams P{};
    const Matrix *m0 = a.m0, *m1 = a.m1;
    P.p0 = m0->packed(); P.s0 = m0->scales(); P.b0 = m0->biases();
    if (m1) { P.p1 = m1->packed(); P.s1 = m1->scales(); P.b1 = m1->biases(); }
    if (a.sm0) { P.sp0 = a.sm0->packed(); P.ss0 = a.sm0->scales(); P.sb0 = a.sm0->biases(); }
    if (a.sm1) { P.sp1 = a.sm1->packed(); P.ss1 = a.sm1->scales(); P.sb1 = a.sm1->biases(); }
    P.experts = m0->experts; P.rows = m0->rows; P.columns = m0->columns;
    P.tokens = a.tokens; P.dense = a.dense; P.in_mode = a.in_mode; P.y_bf16 = a.y_bf16;
    P.row_tiles = (m0->rows + 127) / 128;
    P.routes = a.routes; P.chunks = a.chunks; P.nchunks = a.nchunks;
    P.x = a.x; P.y = a.y;
    const int max_chunks = a.dense ? (a.tokens + 63) / 64 : a.max_chunks;
    const long work = (long)P.row_tiles * max_chunks;
    const long blocks = 8 * ((work + 7) / 8);
    if (blocks <= 0 || blocks > 0x7fffffffL) {
        set_error(error, capacity, "Invalid qmm grid");
        return false;
    }
    dim3 grid((unsigned)blocks), block(256);
    const bool gated = m1 != nullptr;
    if (m0->bits == 8) {
        if (gated) DIH_LAUNCH((qmm_kernel<8, true, 2>), grid, block, 0, s, P);
        else DIH_LAUNCH((qmm_kernel<8, false, 2>), grid, block, 0, s, P);
    } else {
        if (gated) DIH_LAUNCH((qmm_kernel<5, true, 2>), grid, block, 0, s, P);
        else DIH_LAUNCH((qmm_kernel<5, false, 2>), grid, block, 0, s, P);
    }
    return hip_ok(hipGetLastError(), error, capacity, "qmm launch");
}

}  // namespace dih
