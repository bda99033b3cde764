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
// Activations: each block stages its slot's x once in LDS (loads issued before the weight
// ring, so waiting for them does not wait for weights). With 8-bit codes and bf16 x the
// copy is f16: each 32-column chunk is scaled by a power of two that puts its largest
// magnitude in [2^14, 2^15), which is exact and keeps every bf16 value within 2^29 of the
// chunk's largest a normal (exact) f16. The dot takes two codes per instruction
// (chunk_dot_h8); otherwise it is f32. Each chunk also stores the sum of its staged values
// and its scale.
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

// LDS copy of one slot's activations: f16 pieces at xh_dw(c, p) (chunk c, 16-byte piece p
// rotated by c/2 against bank conflicts), or f32 at xf_at(c, i); then per chunk the sum of
// the stored values and (f16) its power-of-two scale. Sizes: f16 C*2 + C/8 bytes, f32
// C*4 + C/8 bytes.
DIH_DEV int xh_dw(int c, int p) { return c * 16 + 4 * ((p + (c >> 1)) & 3); }
DIH_DEV int xf_at(int c, int i) { return c * 32 + ((i + 4 * (c & 7)) & 31); }

// This thread's raw activations: columns 8*(t + 256k) .. +8 (bf16: v[k][0]; f32: both).
template <int CPL>
struct XStage {
    uint4 v[CPL][2];
};

template <int CPL>
DIH_DEV void xstage_load(XStage<CPL> &X, const QmvSeg &S, int slot) {
    const int t = threadIdx.x, n8 = S.columns >> 3;
#pragma unroll
    for (int k = 0; k < CPL; k++) {
        int i = t + 256 * k;
        i = i < n8 ? i : n8 - 1;
        if (S.x_bf16) {
            const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(S.x) + (size_t)slot * S.x_slot_stride);
            X.v[k][0] = p[i];
            X.v[k][1] = make_uint4(0, 0, 0, 0);
        } else {
            const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const float *>(S.x) + (size_t)slot * S.x_slot_stride);
            X.v[k][0] = p[2 * i];
            X.v[k][1] = p[2 * i + 1];
        }
    }
}

// Write the staged activations to LDS; four consecutive threads hold one 32-value chunk.
template <int CPL, bool XH>
DIH_DEV void xstage_store(const XStage<CPL> &X, const QmvSeg &S, uint32_t *lds) {
    const int t = threadIdx.x, n8 = S.columns >> 3, nch = S.columns >> 5;
    float *sums = reinterpret_cast<float *>(lds) + (XH ? (S.columns >> 1) : S.columns);
    float *mults = sums + nch;
#pragma unroll
    for (int k = 0; k < CPL; k++) {
        const int i = t + 256 * k, c = i >> 2;
        float f[8];
        if (S.x_bf16) {
            const uint32_t u[4] = {X.v[k][0].x, X.v[k][0].y, X.v[k][0].z, X.v[k][0].w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                f[2 * q] = __uint_as_float(u[q] << 16);
                f[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
            }
        } else {
            const uint4 a = X.v[k][0], b = X.v[k][1];
            f[0] = __uint_as_float(a.x); f[1] = __uint_as_float(a.y); f[2] = __uint_as_float(a.z); f[3] = __uint_as_float(a.w);
            f[4] = __uint_as_float(b.x); f[5] = __uint_as_float(b.y); f[6] = __uint_as_float(b.z); f[7] = __uint_as_float(b.w);
        }
        float sum;
        if constexpr (XH) {
            float m = 0.f;
#pragma unroll
            for (int q = 0; q < 8; q++) m = fmaxf(m, fabsf(f[q]));
            m = fmaxf(m, dppf<DIH_DPP_XOR1>(m));
            m = fmaxf(m, dppf<DIH_DPP_XOR2>(m));
            const int ex = (int)((__float_as_uint(m) >> 23) & 255u) - 126;
            const int sc = max(ex - 15, -100);   // (an all-zero chunk: any scale)
            uint32_t pk[4];
            sum = 0.f;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const _Float16 h0 = (_Float16)ldexpf(f[2 * q], -sc), h1 = (_Float16)ldexpf(f[2 * q + 1], -sc);
                sum += (float)h0 + (float)h1;
                pk[q] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            }
            if (i < n8) {
                *reinterpret_cast<uint4 *>(&lds[xh_dw(c, i & 3)]) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
                if ((i & 3) == 0) mults[c] = __uint_as_float((uint32_t)(127 + sc) << 23);
            }
        } else {
            sum = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
            if (i < n8) {
                float *xl = reinterpret_cast<float *>(lds);
                const int i0 = (i & 3) * 8;
                *reinterpret_cast<float4 *>(&xl[xf_at(c, i0)]) = make_float4(f[0], f[1], f[2], f[3]);
                *reinterpret_cast<float4 *>(&xl[xf_at(c, i0 + 4)]) = make_float4(f[4], f[5], f[6], f[7]);
            }
        }
        sum += dppf<DIH_DPP_XOR1>(sum);
        sum += dppf<DIH_DPP_XOR2>(sum);
        if (i < n8 && (i & 3) == 0) sums[c] = sum;
    }
}

template <int BITS, int CPL, bool GATED, int D, bool XH, bool PLAIN>
DIH_DEV void qmv_wave(const QmvSeg &S, int lpr, int slot, uint32_t e, bool bad_id, int wi, int W,
                      int K, bool active, const XStage<CPL> &X, uint32_t *lds) {
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
            load_chunk<BITS, !PLAIN>(st.w[c], wrow, chc[c]);
            st.s[c] = S.s0[rowi * gpr + (chc[c] >> 1)];
            st.b[c] = S.b0[rowi * gpr + (chc[c] >> 1)];
            if constexpr (GATED) {
                load_chunk<BITS, !PLAIN>(st.u[c], S.p1 + rowi * wpr, chc[c]);
                st.su[c] = S.s1[rowi * gpr + (chc[c] >> 1)];
                st.bu[c] = S.b1[rowi * gpr + (chc[c] >> 1)];
            }
        }
    };

    RawGroup<BITS, CPL, GATED> ring[D];
    if (active) {
#pragma unroll
        for (int d = 0; d < D; d++) load(ring[d], wi + d * W);
    }

    // the block's activations into LDS (every wave of the block takes part), then this
    // lane's chunks from there
    xstage_store<CPL, XH>(X, S, lds);
    __syncthreads();
    if (!active) return;
    const float *sums = reinterpret_cast<const float *>(lds) + (XH ? (S.columns >> 1) : S.columns);
    const float *mults = sums + nchunk;
    float xr[CPL][XH ? 1 : 32];
    uint32_t xq[CPL][XH ? 16 : 1];
    float xs[CPL], xm[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        xs[c] = sums[chc[c]];
        if constexpr (XH) {
            xm[c] = mults[chc[c]];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&lds[xh_dw(chc[c], p)]);
                xq[c][4 * p] = v.x; xq[c][4 * p + 1] = v.y; xq[c][4 * p + 2] = v.z; xq[c][4 * p + 3] = v.w;
            }
        } else {
            xm[c] = 1.f;
            const float *xl = reinterpret_cast<const float *>(lds);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 v = *reinterpret_cast<const float4 *>(&xl[xf_at(chc[c], 4 * q)]);
                xr[c][4 * q] = v.x; xr[c][4 * q + 1] = v.y; xr[c][4 * q + 2] = v.z; xr[c][4 * q + 3] = v.w;
            }
        }
    }

    // one chunk's affine dot: s*sum(q*x) + b*sum(x)
    auto dot = [&](const Chunk<BITS> &w, uint32_t sb, uint32_t bb, int c) -> float {
        if constexpr (XH) {
            const float d = chunk_dot_h8(reinterpret_cast<const Chunk<8> &>(w), xq[c]) - 1024.f * xs[c];
            return xm[c] * (bf16_to_f32(sb) * d + bf16_to_f32(bb) * xs[c]);
        } else {
            return bf16_to_f32(sb) * chunk_dot<BITS>(w, xr[c]) + bf16_to_f32(bb) * xs[c];
        }
    };

    auto consume = [&](const RawGroup<BITS, CPL, GATED> &st, int grp) {
        const int r = grp * rpw + g;
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const float v = dot(st.w[c], st.s[c], st.b[c], c);
            a += valid[c] ? v : 0.f;
            if constexpr (GATED) {
                const float vu = dot(st.u[c], st.su[c], st.bu[c], c);
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

// PLAIN: plain weight loads for the long streams (the lm_head), non-temporal otherwise
template <int BITS, int CPL, int D, bool PLAIN>
__global__ __launch_bounds__(256) void qmv_kernel(QmvParams P) {
    extern __shared__ __align__(16) uint32_t qx[];   // the block's staged activations
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
    // waves past the slot's rows still stage activations and meet the block barrier
    const bool active = wi < W;
    const int lane = threadIdx.x & 63;
    XStage<CPL> X;
    xstage_load<CPL>(X, S, slot);

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
    const bool xh = BITS == 8 && S.x_bf16;   // uniform over the block
    if (!PLAIN && S.p1) {   // (long streams are single-matrix segments)
        if (xh) qmv_wave<BITS, CPL, true, D, BITS == 8, PLAIN>(S, P.lpr[k], slot, e, bad_id, wi, W, P.iters[k], active, X, qx);
        else qmv_wave<BITS, CPL, true, D, false, PLAIN>(S, P.lpr[k], slot, e, bad_id, wi, W, P.iters[k], active, X, qx);
    } else {
        if (xh) qmv_wave<BITS, CPL, false, D, BITS == 8, PLAIN>(S, P.lpr[k], slot, e, bad_id, wi, W, P.iters[k], active, X, qx);
        else qmv_wave<BITS, CPL, false, D, false, PLAIN>(S, P.lpr[k], slot, e, bad_id, wi, W, P.iters[k], active, X, qx);
    }
}

// One-shot GEMV for single-matrix launches of 8-bit rows of 2048 columns with bf16
// activations and no expert ids (the lm_head, a single decode GEMV): wave w computes rows
// R*w .. R*w + R - 1 of its slot and exits. Lane l owns columns 32l .. 32l+31
// of every row and stages its own activations in registers (f16, scaled by a power of two
// as in xstage_store): no LDS and no barrier, so a block is only its waves' loads in
// flight, and the launch is many short blocks rather than a resident set walking rows.
// Rows a wave: three for long launches (the lm_head: 83 us against 97 us for the resident
// qmv_kernel; 1, 2, 4 and 8 rows took 131, 85, 88 and 87 us, two- and eight-wave blocks
// 85 us, non-temporal loads 99 us), two otherwise (a 4096-row GEMV: 4.47 us a call
// against 5.29 us resident; one row 4.87, three 5.4).
template <int R>
__global__ __launch_bounds__(256) void qmv_stream_kernel(QmvParams P) {
    const int blk = blockIdx.x;
    int k = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; i++)
        if (i < P.nseg && blk >= P.start[i]) k = i;
    const QmvSeg &S = P.seg[k];
    const int local = blk - P.start[k];
    const int slot = local / P.blocks_per_slot[k];
    const int r0 = ((local - slot * P.blocks_per_slot[k]) * 4 + (threadIdx.x >> 6)) * R;
    const int lane = threadIdx.x & 63;
    const uint4 *xp = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(S.x) + (size_t)slot * S.x_slot_stride) + lane * 4;
    uint4 xv[4];
#pragma unroll
    for (int q = 0; q < 4; q++) xv[q] = xp[q];
    Chunk<8> w[R];
    uint32_t sc[R], bi[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
        const int r = min(r0 + q, S.rows - 1);
        load_chunk<8, false>(w[q], S.p0 + (size_t)r * 512, lane);
        sc[q] = S.s0[(size_t)r * 32 + (lane >> 1)];
        bi[q] = S.b0[(size_t)r * 32 + (lane >> 1)];
    }
    float f[32];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t u[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
#pragma unroll
        for (int m = 0; m < 4; m++) {
            f[8 * q + 2 * m] = __uint_as_float(u[m] << 16);
            f[8 * q + 2 * m + 1] = __uint_as_float(u[m] & 0xffff0000u);
        }
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(f[i]));
    const int ex = (int)((__float_as_uint(mx) >> 23) & 255u) - 126;
    const int scl = max(ex - 15, -100);   // (an all-zero chunk: any scale)
    uint32_t xq[16];
    float xs = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const _Float16 h0 = (_Float16)ldexpf(f[2 * i], -scl), h1 = (_Float16)ldexpf(f[2 * i + 1], -scl);
        xs += (float)h0 + (float)h1;
        xq[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    }
    const float mult = __uint_as_float((uint32_t)(127 + scl) << 23);
#pragma unroll
    for (int q = 0; q < R; q++) {
        const float d = chunk_dot_h8(w[q], xq) - 1024.f * xs;
        const float v = wave_sum(mult * (bf16_to_f32(sc[q]) * d + bf16_to_f32(bi[q]) * xs));
        if (lane == 0 && r0 + q < S.rows) {
            const size_t o = (size_t)slot * S.rows + r0 + q;
            if (S.y_bf16)
                static_cast<uint16_t *>(S.y)[o] = f32_to_bf16(v);
            else
                static_cast<float *>(S.y)[o] = v;
        }
    }
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
    // else enough that the waves number about kWavesTarget. Long launches run the one-shot
    // qmv_stream_kernel when their rows allow it (8-bit, 2048 columns, bf16 x, no expert
    // ids: the lm_head), else the single-matrix kernel instance (102 VGPRs: four waves per
    // SIMD, so all kWavesTarget waves are resident at once, no trailing partial round).
    const bool longrun = total > 4L * kWavesTarget;
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
    // staged activations: f32 (4 B per column) plus per-chunk sum and scale
    int maxc = 0;
    for (int i = 0; i < nseg; i++) maxc = std::max(maxc, segs[i].columns);
    const uint32_t lds = (uint32_t)maxc * 4 + (uint32_t)(maxc / 32) * 8;
    // plain loads and the single-matrix instance for the other long four-deep launches
    // (measured 107 -> 98 us on the lm_head before the one-shot kernel; plain loads are 5 %
    // slower on a 4096-row GEMV and equal on the decode step)
    bool plain = longrun && depth == 4 && cpl == 1;
    for (int i = 0; i < nseg; i++) plain = plain && !segs[i].p1;
    bool stream = bits == 8 && cpl == 1;
    for (int i = 0; i < nseg; i++)
        stream = stream && !segs[i].p1 && segs[i].columns == 2048 && segs[i].x_bf16 && !segs[i].ids &&
                 !segs[i].top8;
    if (stream) {
        const int rows = longrun ? 3 : 2;
        int b = 0;
        for (int i = 0; i < nseg; i++) {
            P.blocks_per_slot[i] = (segs[i].rows + 4 * rows - 1) / (4 * rows);
            P.start[i] = b;
            b += P.blocks_per_slot[i] * segs[i].count;
        }
        P.start[nseg] = b;
        if (longrun) DIH_LAUNCH((qmv_stream_kernel<3>), dim3(b), dim3(256), 0, s, P);
        else DIH_LAUNCH((qmv_stream_kernel<2>), dim3(b), dim3(256), 0, s, P);
        return hip_ok(hipGetLastError(), error, capacity, "qmv launch");
    }
    if (plain) {
        if (bits == 8) DIH_LAUNCH((qmv_kernel<8, 1, 4, true>), grid, block, lds, s, P);
        else DIH_LAUNCH((qmv_kernel<5, 1, 4, true>), grid, block, lds, s, P);
        return hip_ok(hipGetLastError(), error, capacity, "qmv launch");
    }
#define DIH_QMV_CASE(B, C, D)                                                  \
    if (bits == B && cpl <= C && depth == D) {                                  \
        DIH_LAUNCH((qmv_kernel<B, C, D, false>), grid, block, lds, s, P);      \
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
            // NaN probabilities: non-finite router logits, the residual stays as it was
            if (!__builtin_isnan(probs[0]))
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
