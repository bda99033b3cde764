/*
 * oracle.c - CPU restatement of the reference's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or as the timed CPU
 * baseline. The product library (infer.net_amd) never calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates. Two kinds
 * of arithmetic are provided:
 *   - fp64 oracles (orc_*_f64): dequantize exactly, accumulate in double. Optionally the
 *     operands are first rounded to bf16 with round-to-nearest-even, as the reference's
 *     BF16 prefill kernels do (prefill_expert_packed.mm:34, prefill_bf16_expanded.mm:24)
 *     and as its own checks model it (prefill_expert_checks.mm:24,56).
 *   - the reference-faithful fp32 CPU path (orc_cpu_*): scalar affine dequant of a row
 *     (quantized.mm:384-397) followed by CpuMatVecDevice's 8-lane partial sums,
 *     horizontal sum and scalar tail (MatVec.cs:40-55). This is the CPU baseline.
 * Integer work (unpack, top-8 ids, grouping, argmax) is exact by construction.
 *
 * The checks that pin each function against the reference's own closed forms, known
 * answers and independent mathematics live in tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* bf16 -> f32 is a 16-bit shift (quantized.mm:50-51: as_type<float>(uint(s)<<16)). */
static inline float bf(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
ORC_API float orc_bf16_to_f32(uint16_t h) { return bf(h); }

/* f32 -> bf16 round-to-nearest-even exactly as prefill_expert_checks.mm:24 and
 * bf16_checks.mm:4 (bits + 0x7fff + lsb, truncate). NaN inputs are not used. */
static inline uint16_t rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u = (u + 0x7fffu + ((u >> 16) & 1u));
    return (uint16_t)(u >> 16);
}
ORC_API uint16_t orc_f32_to_bf16(float f) { return rne(f); }
static inline float round_bf(float f) { return bf(rne(f)); }

/* Code c of a row, LSB-first at bit c*bits, straddling into the next word
 * (quant_gemv quantized.mm:44-48; quant_code quantized.mm:62-67). */
static inline uint32_t code_at(const uint32_t *row, int bits, int c) {
    uint32_t bit = (uint32_t)c * (uint32_t)bits, at = bit >> 5, shift = bit & 31u;
    uint32_t q = row[at] >> shift;
    if (shift + (uint32_t)bits > 32u) q |= row[at + 1] << (32u - shift);
    return q & ((1u << bits) - 1u);
}
ORC_API uint32_t orc_code(const uint32_t *row, int bits, int c) { return code_at(row, bits, c); }

typedef struct orc_matrix {
    const uint32_t *packed;
    const uint16_t *scales;
    const uint16_t *biases;
    int experts, rows, columns, bits;
} orc_matrix;

static inline const uint32_t *row_words(const orc_matrix *m, int e, int r) {
    return m->packed + ((size_t)e * m->rows + r) * (size_t)(m->columns * m->bits / 32);
}
static inline size_t row_params(const orc_matrix *m, int e, int r) {
    return ((size_t)e * m->rows + r) * (size_t)(m->columns / 64);
}

/* Scalar affine dequant of one row in fp32: float(q)*scale + bias
 * (di_quant_embedding quantized.mm:384-397). */
ORC_API void orc_dequant_row(const orc_matrix *m, int e, int r, float *out) {
    const uint32_t *w = row_words(m, e, r);
    size_t p = row_params(m, e, r);
    for (int c = 0; c < m->columns; c++) {
        float scale = bf(m->scales[p + c / 64]), bias = bf(m->biases[p + c / 64]);
        out[c] = (float)code_at(w, m->bits, c) * scale + bias;
    }
}

/* Dequantized weight in double: exact value of q*scale+bias (the fp32 form above differs
 * from it by at most one fp32 rounding). With round_weights, the fp32 value is rounded to
 * bf16 first (packed_expert_load prefill_expert_packed.mm:34). */
static inline double weight_at(const orc_matrix *m, int e, int r, int c, int round_weights) {
    const uint32_t *w = row_words(m, e, r);
    size_t p = row_params(m, e, r) + (size_t)(c / 64);
    float scale = bf(m->scales[p]), bias = bf(m->biases[p]);
    uint32_t q = code_at(w, m->bits, c);
    if (round_weights) return (double)round_bf((float)q * scale + bias);
    return (double)q * (double)scale + (double)bias;
}

/* fp64 GEMV with quant_rows semantics (quantized.mm:119-144):
 * y[slot*rows+row] = sum_c w(experts[slot], row, c) * x[(batched?slot*columns:0)+c].
 * x is f32. QuantizedTests.cs:64-69 is the reference's own form of this oracle. */
ORC_API void orc_qmv_f64(const orc_matrix *m, const float *x, const uint32_t *experts,
                         int count, int batched, double *y) {
    for (int s = 0; s < count; s++) {
        int e = experts ? (int)experts[s] : 0;
        const float *xs = x + (batched ? (size_t)s * m->columns : 0);
        for (int r = 0; r < m->rows; r++) {
            double acc = 0;
            for (int c = 0; c < m->columns; c++) acc += weight_at(m, e, r, c, 0) * (double)xs[c];
            y[(size_t)s * m->rows + r] = acc;
        }
    }
}

/* fp64 batched (dense) product Y[t][r] = sum_c w(e,r,c) X[t][c] with optional bf16
 * rounding of weights and of X (prefill_bf16_product prefill_bf16.mm:26-37; the
 * reference's oracle form prefill_expert_checks.mm:55-56 and bf16_checks.mm:30-31). */
ORC_API void orc_dense_f64(const orc_matrix *m, int expert, const float *x, int tokens,
                           int round_operands, double *y) {
    int C = m->columns, R = m->rows;
    double *wrow = (double *)malloc(sizeof(double) * (size_t)C);
    double *xr = (double *)malloc(sizeof(double) * (size_t)C * tokens);
    for (int t = 0; t < tokens; t++)
        for (int c = 0; c < C; c++) {
            float v = x[(size_t)t * C + c];
            xr[(size_t)t * C + c] = round_operands ? (double)round_bf(v) : (double)v;
        }
    for (int r = 0; r < R; r++) {
        for (int c = 0; c < C; c++) wrow[c] = weight_at(m, expert, r, c, round_operands);
        for (int t = 0; t < tokens; t++) {
            double acc = 0;
            const double *xt = xr + (size_t)t * C;
            for (int c = 0; c < C; c++) acc += wrow[c] * xt[c];
            y[(size_t)t * R + r] = acc;
        }
    }
    free(wrow);
    free(xr);
}

static inline double sigmoid_d(double v) { return 1.0 / (1.0 + exp(-v)); }

/* Router selection (SelectExperts Qwen36Model.cs:246-262): insertion top-8 with strict
 * '>' so ties keep the lowest id first; probabilities = softmax over the eight chosen
 * logits with the max subtracted (Softmax Qwen36Model.cs:293-298), computed in fp32 in
 * the same order as the reference. Returns -1 on a non-finite logit (the reference
 * throws, Qwen36Model.cs:252). `experts` logits, 8 <= experts <= 256. */
ORC_API int orc_top8(const float *logits, int experts, int32_t *ids, float *probs) {
    for (int j = 0; j < 8; j++) ids[j] = -1;
    for (int e = 0; e < experts; e++) {
        if (!isfinite(logits[e])) return -1;
        for (int j = 0; j < 8; j++)
            if (ids[j] < 0 || logits[e] > logits[ids[j]]) {
                for (int k = 7; k > j; k--) ids[k] = ids[k - 1];
                ids[j] = e;
                break;
            }
    }
    float max = -INFINITY;
    for (int i = 0; i < 8; i++) {
        probs[i] = logits[ids[i]];
        max = fmaxf(max, probs[i]);
    }
    float sum = 0;
    for (int i = 0; i < 8; i++) {
        probs[i] = expf(probs[i] - max);
        sum += probs[i];
    }
    for (int i = 0; i < 8; i++) probs[i] /= sum;
    return 0;
}

/* Top-8 for T tokens of bf16 logits [T][experts]; returns the first failing token or -1.
 * (prefill_top8 gpu_prefill.mm:151-161 applies graph_top8's rule per token.) */
ORC_API int orc_top8_bf16(const uint16_t *logits, int tokens, int experts, int32_t *ids,
                          float *probs) {
    float *row = (float *)malloc(sizeof(float) * (size_t)experts);
    for (int t = 0; t < tokens; t++) {
        for (int e = 0; e < experts; e++) row[e] = bf(logits[(size_t)t * experts + e]);
        if (orc_top8(row, experts, ids + 8 * t, probs + 8 * t)) {
            free(row);
            return t;
        }
    }
    free(row);
    return -1;
}

/* Route grouping (prefill_build_groups prefill_moe.mm:8-17): for each expert, the routes
 * r (= token*8 + slot) with ids[r] == expert in ascending order, and their count.
 * routes has room for experts*tokens entries: routes[e*tokens + k]. */
ORC_API void orc_build_groups(const uint32_t *ids, int tokens, int experts, uint32_t *counts,
                              uint32_t *routes) {
    for (int e = 0; e < experts; e++) counts[e] = 0;
    for (int r = 0; r < tokens * 8; r++) {
        uint32_t e = ids[r];
        if ((int)e < experts) {
            routes[(size_t)e * tokens + counts[e]] = (uint32_t)r;
            counts[e]++;
        }
    }
}

/* Argmax (graph_argmax_blocks/final gpu_graph.mm:160-175; ArgMax Qwen36Model.cs:153-162):
 * lowest index of the maximum; 0xffffffff if any value is not finite. */
ORC_API uint32_t orc_argmax(const float *v, int n) {
    uint32_t index = 0;
    for (int i = 0; i < n; i++) {
        if (!isfinite(v[i])) return 0xffffffffu;
        if (v[i] > v[index]) index = (uint32_t)i;
    }
    return index;
}

/* Decode fused expert MLP in fp64 (expert_gate_up quantized.mm:148-189 followed by the
 * batched down GEMV and the shared down GEMV, di_quant_experts quantized.mm:357-383;
 * the reference's oracle form is QuantizedTests.cs:89-114).
 * act[s][i] = silu(g)*u, out[s][h] = down[e_s][h] . act[s], shared_out = shared . sx. */
ORC_API void orc_expert_mlp_f64(const orc_matrix *gate, const orc_matrix *up,
                                const orc_matrix *down, const orc_matrix *shared,
                                const float *x, const float *sx, const uint32_t *experts,
                                int count, double *out, double *shared_out) {
    int I = gate->rows, C = gate->columns, H = down->rows;
    double *act = (double *)malloc(sizeof(double) * (size_t)I);
    for (int s = 0; s < count; s++) {
        int e = (int)experts[s];
        for (int i = 0; i < I; i++) {
            double g = 0, u = 0;
            for (int c = 0; c < C; c++) {
                g += weight_at(gate, e, i, c, 0) * (double)x[c];
                u += weight_at(up, e, i, c, 0) * (double)x[c];
            }
            act[i] = g * sigmoid_d(g) * u;
        }
        for (int h = 0; h < H; h++) {
            double acc = 0;
            for (int i = 0; i < I; i++) acc += weight_at(down, e, h, i, 0) * act[i];
            out[(size_t)s * H + h] = acc;
        }
    }
    if (shared)
        for (int h = 0; h < shared->rows; h++) {
            double acc = 0;
            for (int c = 0; c < shared->columns; c++) acc += weight_at(shared, 0, h, c, 0) * (double)sx[c];
            shared_out[h] = acc;
        }
    free(act);
}

typedef struct orc_moe_layer {
    const orc_matrix *router, *gate, *up, *down;
    const orc_matrix *shared_gate, *shared_up, *shared_down, *shared_route;
} orc_moe_layer;

/* MoE block in fp64 for T tokens given the selected ids/probs per token
 * (Moe Qwen36Model.cs:218-245; merge order of prefill_merge gpu_prefill.mm:140-150:
 * y = shared*sigmoid(route) then += expert_slot*p_slot for slot 0..7).
 * x is f32 [T][H] (callers pass bf16 values widened to f32). `bf16_operands` rounds the
 * weights, x and the activation fed to down to bf16 like the prefill MFMA path
 * (prefill_expert_packed.mm:34; expanded_pack prefill_bf16_expanded.mm:24).
 * y_out f64 [T][H] receives the MoE output before it is added to the residual;
 * route_out (optional) f64 [T*8 + T][H] receives per-route down outputs. */
/* Dequantized weights of expert e of m in double, row-major [rows][columns]. */
static void dequant_expert(const orc_matrix *m, int e, int round_w, double *out) {
    for (int r = 0; r < m->rows; r++)
        for (int c = 0; c < m->columns; c++) out[(size_t)r * m->columns + c] = weight_at(m, e, r, c, round_w);
}

ORC_API void orc_moe_f64(const orc_moe_layer *L, int tokens, const float *x,
                         const int32_t *ids, const float *probs, int bf16_operands,
                         double *y_out, double *route_out) {
    int H = L->gate->columns, I = L->gate->rows, Is = L->shared_gate->rows, E = L->gate->experts;
    int Imax = I > Is ? I : Is;
    size_t T = (size_t)tokens;
    /* Work is grouped by expert: each expert's weights are dequantized once and applied to
     * all of its routes; every dot product keeps its summation order (columns ascending
     * for gate/up, intermediate index ascending for down), so each route's output and the
     * merged sum below are the same numbers as a token-by-token evaluation. */
    double *ro = route_out ? route_out : (double *)malloc(sizeof(double) * T * 9 * (size_t)H);
    double *xd = (double *)malloc(sizeof(double) * T * (size_t)H);
    int *order = (int *)malloc(sizeof(int) * T * 8);
    int *start = (int *)calloc((size_t)E + 1, sizeof(int));
    for (size_t i = 0; i < T * (size_t)H; i++) xd[i] = bf16_operands ? (double)round_bf(x[i]) : (double)x[i];
    for (size_t r = 0; r < T * 8; r++) start[ids[r] + 1]++;
    for (int e = 0; e < E; e++) start[e + 1] += start[e];
    {
        int *fill = (int *)malloc(sizeof(int) * (size_t)E);
        memcpy(fill, start, sizeof(int) * (size_t)E);
        for (size_t r = 0; r < T * 8; r++) order[fill[ids[r]]++] = (int)r;   /* routes ascending */
        free(fill);
    }
#pragma omp parallel
    {
        double *wg = (double *)malloc(sizeof(double) * (size_t)Imax * H);
        double *wu = (double *)malloc(sizeof(double) * (size_t)Imax * H);
        double *wd = (double *)malloc(sizeof(double) * (size_t)H * Imax);
        double *act = (double *)malloc(sizeof(double) * (size_t)Imax);
        /* group -1 is the shared expert (every token), then the routed experts */
#pragma omp for schedule(dynamic)
        for (int g = -1; g < E; g++) {
            const int shared = g < 0, n = shared ? tokens : start[g + 1] - start[g];
            if (n == 0) continue;
            const orc_matrix *mg = shared ? L->shared_gate : L->gate, *mu = shared ? L->shared_up : L->up;
            const orc_matrix *md = shared ? L->shared_down : L->down;
            const int e = shared ? 0 : g, In = mg->rows;
            dequant_expert(mg, e, bf16_operands, wg);
            dequant_expert(mu, e, bf16_operands, wu);
            dequant_expert(md, e, bf16_operands, wd);
            for (int k = 0; k < n; k++) {
                const size_t route = shared ? T * 8 + (size_t)k : (size_t)order[start[g] + k];
                const double *xt = xd + (shared ? (size_t)k : route / 8) * H;
                for (int i = 0; i < In; i++) {
                    double a = 0, b = 0;
                    const double *gi = wg + (size_t)i * H, *ui = wu + (size_t)i * H;
                    for (int c = 0; c < H; c++) {
                        a += gi[c] * xt[c];
                        b += ui[c] * xt[c];
                    }
                    act[i] = a * sigmoid_d(a) * b;
                    if (bf16_operands) act[i] = (double)round_bf((float)act[i]);
                }
                for (int h = 0; h < H; h++) {
                    double acc = 0;
                    const double *dh = wd + (size_t)h * In;
                    for (int i = 0; i < In; i++) acc += dh[i] * act[i];
                    ro[route * H + h] = acc;
                }
            }
        }
        free(wg);
        free(wu);
        free(wd);
        free(act);
        /* merge in the reference's order: shared * sigmoid(route), then slots 0..7. The
         * shared expert's sigmoid gate is never rounded: the reference evaluates it with
         * the fp32 GEMV (gpu_prefill.mm:700). */
#pragma omp for schedule(static)
        for (int t = 0; t < tokens; t++) {
            double route = 0;
            for (int c = 0; c < H; c++) route += weight_at(L->shared_route, 0, 0, c, 0) * (double)x[(size_t)t * H + c];
            const double gate = sigmoid_d(route);
            double *y = y_out + (size_t)t * H;
            const double *so = ro + (T * 8 + (size_t)t) * H;
            for (int h = 0; h < H; h++) y[h] = so[h] * gate;
            for (int s = 0; s < 8; s++) {
                const double p = (double)probs[t * 8 + s];
                const double *o = ro + ((size_t)t * 8 + s) * H;
                for (int h = 0; h < H; h++) y[h] += o[h] * p;
            }
        }
    }
    if (!route_out) free(ro);
    free(xd);
    free(order);
    free(start);
}

/* ---------------- reference-faithful fp32 CPU path (the CPU baseline) -------------- */

/* CpuMatVecDevice.Multiply for one row (MatVec.cs:44-53): 8-lane Vector<float> partial
 * sums over the row, Vector.Sum, then the scalar tail. */
static inline float cpu_dot8(const float *w, const float *x, int n) {
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int c = 0;
    for (; c <= n - 8; c += 8)
        for (int j = 0; j < 8; j++) lane[j] += w[c + j] * x[c + j];
    float v = 0;
    for (int j = 0; j < 8; j++) v += lane[j];
    for (; c < n; c++) v += w[c] * x[c];
    return v;
}

/* Dequant-then-matmul for count slots: scalar row dequant (quantized.mm:384-397) then
 * the CPU GEMV row (MatVec.cs:40-55). `threads` > 1 splits rows across OpenMP threads. */
ORC_API void orc_cpu_qmv(const orc_matrix *m, const float *x, const uint32_t *experts,
                         int count, int batched, float *y, int threads) {
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)m->columns);
        for (int s = 0; s < count; s++) {
            int e = experts ? (int)experts[s] : 0;
            const float *xs = x + (batched ? (size_t)s * m->columns : 0);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int r = 0; r < m->rows; r++) {
                orc_dequant_row(m, e, r, row);
                y[(size_t)s * m->rows + r] = cpu_dot8(row, xs, m->columns);
            }
        }
        free(row);
    }
}

static inline float silu_f(float v) { return v * (1.0f / (1.0f + expf(-v))); }

/* The reference's host MoE for one token in fp32 (Moe Qwen36Model.cs:218-245 with the
 * unfused diagnostic ordering :237-240): router/shared GEMVs, SelectExperts, SiLU*up,
 * expert gate/up/down GEMVs, sigmoid-scaled shared output plus the probability-weighted
 * expert outputs (AddScaled, slot order). Returns -1 on non-finite router logits.
 * y receives the MoE output for the token. */
ORC_API int orc_cpu_moe_token(const orc_moe_layer *L, const float *x, float *y, int threads) {
    int H = L->gate->columns, I = L->gate->rows, Is = L->shared_gate->rows;
    int E = L->router->rows;
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    float *sg = (float *)malloc(sizeof(float) * (size_t)Is), *su = (float *)malloc(sizeof(float) * (size_t)Is);
    float route;
    float *g = (float *)malloc(sizeof(float) * (size_t)8 * I), *u = (float *)malloc(sizeof(float) * (size_t)8 * I);
    float *eo = (float *)malloc(sizeof(float) * (size_t)8 * H);
    int32_t ids[8];
    float probs[8];
    uint32_t uids[8];
    orc_cpu_qmv(L->router, x, NULL, 1, 0, logits, threads);
    orc_cpu_qmv(L->shared_gate, x, NULL, 1, 0, sg, threads);
    orc_cpu_qmv(L->shared_up, x, NULL, 1, 0, su, threads);
    orc_cpu_qmv(L->shared_route, x, NULL, 1, 0, &route, threads);
    int rc = orc_top8(logits, E, ids, probs);
    if (rc == 0) {
        for (int i = 0; i < Is; i++) sg[i] = silu_f(sg[i]) * su[i];
        for (int s = 0; s < 8; s++) uids[s] = (uint32_t)ids[s];
        orc_cpu_qmv(L->gate, x, uids, 8, 0, g, threads);
        orc_cpu_qmv(L->up, x, uids, 8, 0, u, threads);
        for (int i = 0; i < 8 * I; i++) g[i] = silu_f(g[i]) * u[i];
        orc_cpu_qmv(L->down, g, uids, 8, 1, eo, threads);
        orc_cpu_qmv(L->shared_down, sg, NULL, 1, 0, y, threads);
        float scale = 1.0f / (1.0f + expf(-route));
        for (int h = 0; h < H; h++) y[h] *= scale;
        for (int s = 0; s < 8; s++)
            for (int h = 0; h < H; h++) y[h] += probs[s] * eo[(size_t)s * H + h];
    }
    free(logits); free(sg); free(su); free(g); free(u); free(eo);
    return rc;
}

ORC_API int orc_openmp_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------- attention inputs
 * The reference's attention checks draw every input from one xorshift32 stream
 * (shifts 13, 17, 5) mapped to value = (int)(s % 10001) - 5000) / 12500 in f32
 * (prefill_attention_checks.mm:17-18; attention_batch_checks.mm:19). `interleave` > 1
 * deals consecutive draws round-robin into that many output arrays, as the checks fill
 * keys and values from one stream (prefill_attention_checks.mm:20-24). */
ORC_API uint32_t orc_xorshift_fill(uint32_t seed, float *const *out, int interleave, size_t n) {
    for (size_t i = 0; i < n; i++)
        for (int k = 0; k < interleave; k++) {
            seed ^= seed << 13;
            seed ^= seed >> 17;
            seed ^= seed << 5;
            out[k][i] = (float)((int)(seed % 10001u) - 5000) / 12500.0f;
        }
    return seed;
}
