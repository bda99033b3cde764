// Decode MoE step for one token in three launches (g_router, gpu_graph.mm:296-320, with
// graph_top8 gpu_graph.mm:134-146 and graph_merge_norm gpu_graph.mm:48-61; host form
// Qwen36Model.cs:218-245):
//
//   K1 router/shared  : four-wave blocks spread over many CUs. Router logits four experts
//                       a block at 2048 columns (one row a wave: a block's weights are
//                       8.7 KB, so the router's 557 KB spread over 64 CUs). The same launch
//                       computes the shared expert's gate/up SwiGLU and the shared-expert
//                       sigmoid gate row.
//   K2 experts gate/up: every block ranks the <= 256 logits (top-8 of each 32, then the 64
//                       kept; ties to the lowest id) and streams one gated row group per
//                       wave of its slot's expert.
//   K3 down + merge   : blocks of nine waves; waves 0..7 compute the selected experts'
//                       down rows for the block's output rows, wave 8 the shared expert's;
//                       the merge y = sigmoid(route)*shared + sum_slot p_slot*expert_slot
//                       (slot order 0..7) and residual += y (f32 or bf16 storage) happen in LDS.
//
// Kernel boundaries are the only cross-block synchronization: on MI355X a device-scope
// counter or flag shared by hundreds of blocks costs more than a launch. Every wave issues
// all of its weight loads before it waits on any of them; scale/bias words stay raw until
// they are consumed.
#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

#ifdef DIH_DECODE_TIMELINE
// Measurement build only (make timeline): lane 0 of every wave of the first kTlBlocks blocks
// of each kernel writes the constant 100 MHz clock at four points. Each call overwrites the
// previous call's stamps, so a read after a sequence holds its last call.
constexpr int kTlBlocks = 512, kTlWaves = 16, kTlPoints = 4;
__device__ unsigned long long g_decode_timeline[3 * kTlBlocks * kTlWaves * kTlPoints];
#define DIH_TL(kern, point)                                                                       \
    do {                                                                                          \
        if ((threadIdx.x & 63) == 0 && blockIdx.x < kTlBlocks)                                    \
            g_decode_timeline[(((kern) * kTlBlocks + blockIdx.x) * kTlWaves + (threadIdx.x >> 6)) * \
                                  kTlPoints + (point)] = wall_clock64();                          \
    } while (0)
#else
#define DIH_TL(kern, point) \
    do {                    \
    } while (0)
#endif

namespace {

constexpr int kK1Waves = 4;        // waves per K1 block: the launch spreads over many CUs
constexpr int kWaves = 16;         // waves per K2 block
constexpr int kRouterGroups = 1;   // K1 router: row groups per wave
constexpr int kMaxExperts = 256;   // routed experts: K2 ranks them with four lanes each
constexpr int kDownGroups = 2;     // K3: row groups per wave

// One lane's share of NG row groups of one matrix.
template <int BITS, int NG>
struct Rows {
    Chunk<BITS> w[NG];
    uint32_t s[NG], b[NG];
};

// Row of group q for this lane: row0 + q*rpw + g, clamped into [0, nrows).
template <int BITS, int NG>
DIH_DEV void rows_load(Rows<BITS, NG> &R, const uint32_t *p, const uint16_t *sc, const uint16_t *bi,
                       size_t rowbase, int nrows, int row0, int rpw, int g, int jc, int columns) {
    const size_t wpr = (size_t)columns * BITS / 32, gpr = (size_t)(columns >> 6);
#pragma unroll
    for (int q = 0; q < NG; q++) {
        int r = row0 + q * rpw + g;
        r = r < nrows ? r : nrows - 1;
        const size_t ri = rowbase + r;
        load_chunk<BITS>(R.w[q], p + ri * wpr, jc);
        R.s[q] = sc[ri * gpr + (jc >> 1)];
        R.b[q] = bi[ri * gpr + (jc >> 1)];
    }
}

// Per-lane partial dot of group q (masked lanes contribute 0), then the row sum over
// the lpr lanes of the row.
template <int BITS, int NG>
DIH_DEV void rows_dot(const Rows<BITS, NG> &R, const float (&x)[32], float xs, bool valid, int lpr,
                      float (&out)[NG]) {
#pragma unroll
    for (int q = 0; q < NG; q++) {
        float v = bf16_to_f32(R.s[q]) * chunk_dot<BITS>(R.w[q], x) + bf16_to_f32(R.b[q]) * xs;
        out[q] = group_sum(valid ? v : 0.f, lpr);
    }
}

// Lane geometry of a row of `columns` codes: lpr lanes per row, this lane's chunk.
struct LaneGeom {
    int lpr, rpw, g, j, jc;
    bool valid;
};
DIH_DEV LaneGeom lane_geom(int columns, int lpr) {
    LaneGeom L;
    const int lane = threadIdx.x & 63, nchunk = columns >> 5;
    L.lpr = lpr;
    L.rpw = 64 / lpr;
    L.g = lane / lpr;
    L.j = lane - L.g * lpr;
    L.valid = L.j < nchunk;
    L.jc = L.valid ? L.j : nchunk - 1;
    return L;
}

// Activations staged once per block in LDS as f32, plus their 32-column sums. Element i
// of chunk c sits at c*32 + ((i + 4*(c & 7)) & 31): a lane reading its chunk as eight
// 16-byte pieces then hits a different bank quad than its seven neighbours.
DIH_DEV int xl_at(int c, int i) { return c * 32 + ((i + 4 * (c & 7)) & 31); }

// Raw bf16 activations of this thread's eight columns (issued before the weights so that
// waiting for them does not wait for the weight stream).
DIH_DEV uint4 stage_x_load(const uint16_t *x, int H) {
    const int t = threadIdx.x;
    return t < (H >> 3) ? reinterpret_cast<const uint4 *>(x)[t] : make_uint4(0, 0, 0, 0);
}

DIH_DEV void stage_x_store(const uint4 v, int H, float *xl, float *xsl) {
    const int t = threadIdx.x;
    if (t < (H >> 3)) {
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
        float f[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            f[2 * k] = __uint_as_float(u[k] << 16);
            f[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
        }
        const int c = t >> 2, i0 = (t & 3) * 8;
        *reinterpret_cast<float4 *>(&xl[xl_at(c, i0)]) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4 *>(&xl[xl_at(c, i0 + 4)]) = make_float4(f[4], f[5], f[6], f[7]);
        float sum = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
        sum += dppf<DIH_DPP_XOR1>(sum);
        sum += dppf<DIH_DPP_XOR2>(sum);
        if ((t & 3) == 0) xsl[c] = sum;
    }
}

// This lane's 32 activations from the staged copy, and their sum.
DIH_DEV float lane_x_lds(float (&x)[32], const float *xl, const float *xsl, const LaneGeom &L) {
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const float4 v = *reinterpret_cast<const float4 *>(&xl[xl_at(L.jc, 4 * q)]);
        x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
    }
    return xsl[L.jc];
}

// Activations of this lane's chunk as f32 straight from global memory, and their sum.
DIH_DEV float lane_x(float (&x)[32], const void *base, int x_bf16, const LaneGeom &L) {
    load_x32(x, base, x_bf16, L.jc * 32);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) s += x[i];
    return s;
}

// Activations staged for the 8-bit f16 dot (chunk_dot_h8). Chunk c (32 columns) is stored
// as f16 values x * 2^-k_c, with k_c chosen so that the chunk's largest |x| lands in
// [2^14, 2^15) (a power-of-two scale is exact, and every bf16 value within 2^29 of the
// largest stays a normal, exact f16; small chunks are scaled up), as four 16-byte pieces
// rotated by c/2 so that eight lanes reading eight chunks hit distinct bank groups. Per
// chunk: the f32 sum of the stored f16 values (so that the 1024 offset cancels against
// exactly the values the dot used) and 2^k_c.
DIH_DEV int xh_at(int c, int p) { return c * 16 + 4 * ((p + (c >> 1)) & 3); }

DIH_DEV void stage_xh_store(const uint4 v, int H, uint32_t *xh, float *xhs, float *xhm) {
    const int t = threadIdx.x;
    if (t < (H >> 3)) {
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
        float f[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            f[2 * k] = __uint_as_float(u[k] << 16);
            f[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
        }
        // chunk maximum over its four staging threads; m < 2^e
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) m = fmaxf(m, fabsf(f[i]));
        m = fmaxf(m, dppf<DIH_DPP_XOR1>(m));
        m = fmaxf(m, dppf<DIH_DPP_XOR2>(m));
        const int e = (int)((__float_as_uint(m) >> 23) & 255u) - 126;
        const int k = max(e - 15, -100);   // (an all-zero chunk: any scale)
        uint32_t p[4];
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const _Float16 h0 = (_Float16)ldexpf(f[2 * i], -k), h1 = (_Float16)ldexpf(f[2 * i + 1], -k);
            sum += (float)h0 + (float)h1;
            p[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        }
        const int c = t >> 2;
        *reinterpret_cast<uint4 *>(&xh[xh_at(c, t & 3)]) = make_uint4(p[0], p[1], p[2], p[3]);
        sum += dppf<DIH_DPP_XOR1>(sum);
        sum += dppf<DIH_DPP_XOR2>(sum);
        if ((t & 3) == 0) {
            xhs[c] = sum;
            xhm[c] = __uint_as_float((uint32_t)(127 + k) << 23);
        }
    }
}

// This lane's chunk of f16 activations; returns their sum, `mult` = 2^k of the chunk.
DIH_DEV float lane_xh(uint32_t (&xr)[16], const uint32_t *xh, const float *xhs, const float *xhm,
                      const LaneGeom &L, float &mult) {
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint4 v = *reinterpret_cast<const uint4 *>(&xh[xh_at(L.jc, p)]);
        xr[4 * p] = v.x; xr[4 * p + 1] = v.y; xr[4 * p + 2] = v.z; xr[4 * p + 3] = v.w;
    }
    mult = xhm[L.jc];
    return xhs[L.jc];
}

// rows_dot for 8-bit rows against f16-staged activations:
// sum_i (q_i*s + b) * x_i = 2^k * (s * (sum_i (1024+q_i) x'_i - 1024 * xs') + b * xs').
template <int NG>
DIH_DEV void rows_dot_h8(const Rows<8, NG> &R, const uint32_t (&xr)[16], float xs, float mult, bool valid,
                         int lpr, float (&out)[NG]) {
#pragma unroll
    for (int q = 0; q < NG; q++) {
        const float d = chunk_dot_h8(R.w[q], xr) - 1024.f * xs;
        const float v = mult * (bf16_to_f32(R.s[q]) * d + bf16_to_f32(R.b[q]) * xs);
        out[q] = group_sum(valid ? v : 0.f, lpr);
    }
}

// Order-preserving key of a router logit: larger key = larger value, -0 equal to +0. Finite
// values map to keys >= 0x00800000, so key 0 can stand for "no expert".
DIH_DEV uint32_t logit_key(float v) {
    uint32_t u = __float_as_uint(v);
    u = u == 0x80000000u ? 0u : u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave-uniform value of VGPR `v` in lane `l`.
DIH_DEV uint32_t lane_value(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }

// 64-bit rank key of expert `id`'s logit: a larger key comes first in (value desc, id asc)
// order. Slots past the expert count get key (0, ~id): distinct, and behind every expert.
DIH_DEV unsigned long long rank_key(float v, uint32_t id, bool expert) {
    return ((unsigned long long)(expert ? logit_key(v) : 0u) << 32) | (uint32_t)~id;
}

// Sum of `r` over the four lanes of each quad (DPP quad permutes, no LDS).
DIH_DEV int quad_sum(int r) {
    r += __builtin_amdgcn_mov_dpp(r, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    r += __builtin_amdgcn_mov_dpp(r, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    return r;
}

}  // namespace

struct DecodeParams {
    const uint32_t *rp; const uint16_t *rs, *rb;           // router [E, H], 8-bit (or null)
    const float *logits_in;                                 // supplied logits [E] (router null)
    float *logits;                                          // router logits out [E]
    const uint32_t *sgp, *sup; const uint16_t *sgs, *sgb, *sus, *sub;  // shared gate/up [I, H]
    const uint32_t *srp; const uint16_t *srs, *srb;         // shared route [1, H], 8-bit
    float *sact;                                            // [I]
    float *sroute;                                          // [1]
    const uint32_t *gp, *upp; const uint16_t *gs, *gb, *us, *ub;  // experts gate/up [E, I, H]
    const uint32_t *dp; const uint16_t *ds, *db;            // experts down [E, H, I]
    const uint32_t *sdp; const uint16_t *sds, *sdb;         // shared down [1, H, I]
    float *act;                                             // [8, I]
    uint32_t *ids; float *probs; uint32_t *status;          // published by K2
    const uint16_t *x;                                      // bf16 [H]
    void *residual;                                         // bf16 or f32 [H]
    int residual_f32;
    float *route_out;                                       // optional [9, H]
    int E, H, I;
    int lpr_h, lpr_i;
    int nchunks;          // router blocks (ceil(E / (kK1Waves * rows per wave)))
    int shared_blocks;    // K1 blocks for the shared gate/up
    int gate_blocks;      // K2 blocks per slot
    int down_rows;        // K3 output rows per block
};

// ------------------------------------------------------------------------------- K1

template <int BITS>
__global__ __launch_bounds__(256) void decode_router_kernel(DecodeParams P) {
    __shared__ __align__(16) float xl[2048];
    __shared__ float xsl[64];
    __shared__ __align__(16) uint32_t xh[1024];
    __shared__ float xhs[64], xhm[64];
    const int b = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const LaneGeom L = lane_geom(P.H, P.lpr_h);
    DIH_TL(0, 0);
    if (b < P.nchunks) {
        // router rows b*chunk + wave*rpw + g (8-bit), one row group a wave
        const int chunk = kK1Waves * kRouterGroups * L.rpw;
        const int wrow = wave * kRouterGroups * L.rpw;
        const int base = b * chunk + wrow;
        const int n = min(chunk, P.E - b * chunk);
        if (P.rp) {
            const uint4 xv = stage_x_load(P.x, P.H);
            Rows<8, kRouterGroups> R;
            rows_load<8, kRouterGroups>(R, P.rp, P.rs, P.rb, 0, P.E, base, L.rpw, L.g, L.jc, P.H);
            stage_xh_store(xv, P.H, xh, xhs, xhm);
            __syncthreads();
            DIH_TL(0, 1);
            uint32_t xr[16];
            float mult;
            const float xs = lane_xh(xr, xh, xhs, xhm, L, mult);
            float v[kRouterGroups];
            rows_dot_h8<kRouterGroups>(R, xr, xs, mult, L.valid, L.lpr, v);
            DIH_TL(0, 2);
#pragma unroll
            for (int q = 0; q < kRouterGroups; q++) {
                const int o = wrow + q * L.rpw + L.g;  // row within the block's experts
                if (L.j == 0 && o < n) P.logits[b * chunk + o] = v[q];
            }
        } else if ((int)threadIdx.x < n) {
            P.logits[b * chunk + threadIdx.x] = P.logits_in[b * chunk + threadIdx.x];
        }
        DIH_TL(0, 3);
        return;
    }
    const int sb = b - P.nchunks;
    if (sb < P.shared_blocks) {
        // shared expert gate/up SwiGLU: one row group (rpw rows) per wave
        const int base = (sb * kK1Waves + wave) * L.rpw;
        const uint4 xv = stage_x_load(P.x, P.H);
        Rows<BITS, 1> G, U;
        rows_load<BITS, 1>(G, P.sgp, P.sgs, P.sgb, 0, P.I, base, L.rpw, L.g, L.jc, P.H);
        rows_load<BITS, 1>(U, P.sup, P.sus, P.sub, 0, P.I, base, L.rpw, L.g, L.jc, P.H);
        float a[1], c[1];
        if constexpr (BITS == 8) {
            stage_xh_store(xv, P.H, xh, xhs, xhm);
            __syncthreads();
            DIH_TL(0, 1);
            uint32_t xr[16];
            float mult;
            const float xs = lane_xh(xr, xh, xhs, xhm, L, mult);
            rows_dot_h8<1>(G, xr, xs, mult, L.valid, L.lpr, a);
            rows_dot_h8<1>(U, xr, xs, mult, L.valid, L.lpr, c);
            DIH_TL(0, 2);
        } else {
            stage_x_store(xv, P.H, xl, xsl);
            __syncthreads();
            float x[32];
            const float xs = lane_x_lds(x, xl, xsl, L);
            rows_dot<BITS, 1>(G, x, xs, L.valid, L.lpr, a);
            rows_dot<BITS, 1>(U, x, xs, L.valid, L.lpr, c);
        }
        if (L.j == 0 && base + L.g < P.I) P.sact[base + L.g] = siluf_(a[0]) * c[0];
        DIH_TL(0, 3);
        return;
    }
    // shared-expert gate row (sigmoid applied at the merge)
    if (wave == 0) {
        Rows<8, 1> R;
        rows_load<8, 1>(R, P.srp, P.srs, P.srb, 0, 1, 0, L.rpw, 0, L.jc, P.H);
        float x[32];
        const float xs = lane_x(x, P.x, 1, L);
        float v[1];
        rows_dot<8, 1>(R, x, xs, L.valid && L.g == 0, 64, v);
        if (lane == 0) P.sroute[0] = v[0];
    }
}

// ------------------------------------------------------------------------------- K2

template <int BITS>
__global__ __launch_bounds__(kWaves * 64) void decode_experts_kernel(DecodeParams P) {
    __shared__ __align__(16) float xl[BITS == 8 ? 1 : 2048];
    __shared__ float xsl[BITS == 8 ? 1 : 64];
    __shared__ __align__(16) uint32_t xh[BITS == 8 ? 1024 : 1];
    __shared__ float xhs[BITS == 8 ? 64 : 1], xhm[BITS == 8 ? 64 : 1];
    __shared__ __align__(16) unsigned long long ck[kMaxExperts];
    __shared__ float cv[kMaxExperts];
    __shared__ __align__(16) unsigned long long cm[64];
    __shared__ int rk[64];
    __shared__ int any_bad;
    static_assert(kWaves * 64 == 4 * kMaxExperts && kWaves * 4 == 64, "rank layout");
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int slot = blockIdx.x / P.gate_blocks;
    const LaneGeom L = lane_geom(P.H, P.lpr_h);
    const int base = ((blockIdx.x - slot * P.gate_blocks) * kWaves + wave) * L.rpw;
    DIH_TL(1, 0);
    // The token's experts, ranked once per block in two rounds on 64-bit keys (value desc,
    // id asc, as the reference's insertion with `>`, SelectExperts Qwen36Model.cs:246-261):
    // each group of 32 logits keeps its top-8 (four lanes a logit, eight comparisons each),
    // then the 64 kept are ranked by all 16 waves (four comparisons a lane).
    if (t < kMaxExperts) {
        const bool ex = t < P.E;
        const float v = ex ? P.logits[t] : 0.f;
        ck[t] = rank_key(v, (uint32_t)t, ex);
        cv[t] = v;
        if (t < 64) rk[t] = 0;
        if (t == 0) any_bad = 0;
    }
    if constexpr (BITS == 8) stage_xh_store(stage_x_load(P.x, P.H), P.H, xh, xhs, xhm);
    else stage_x_store(stage_x_load(P.x, P.H), P.H, xl, xsl);
    __syncthreads();
    {
        const int c = t >> 2, p = t & 3, grp = c >> 5;
        const unsigned long long me = ck[c];
        const unsigned long long *q = &ck[grp * 32 + p * 8];
        int r = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) r += q[k] > me ? 1 : 0;
        r = quad_sum(r);
        if (p == 0) {
            if (r < 8) cm[grp * 8 + r] = me;
            if (c < P.E && !isfinite(cv[c])) any_bad = 1;
        }
    }
    __syncthreads();
    {
        const unsigned long long me = cm[lane];
        int r = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) r += cm[wave * 4 + k] > me ? 1 : 0;
        if (r) atomicAdd(&rk[lane], r);
    }
    __syncthreads();
    // kept key `lane` has rank rk[lane]; the low word of a key is ~id
    const int myrank = rk[lane];
    const uint32_t myid = ~(uint32_t)cm[lane];
    const bool bad = any_bad != 0;
    const uint32_t e = bad ? 0u : lane_value(myid, __ffsll((long long)__ballot(myrank == slot)) - 1);
    DIH_TL(1, 1);
    // one gated row group of expert e per wave
    const size_t ebase = (size_t)e * P.I;
    Rows<BITS, 1> G, U;
    rows_load<BITS, 1>(G, P.gp, P.gs, P.gb, ebase, P.I, base, L.rpw, L.g, L.jc, P.H);
    rows_load<BITS, 1>(U, P.upp, P.us, P.ub, ebase, P.I, base, L.rpw, L.g, L.jc, P.H);
    if (blockIdx.x == 0 && wave == 0) {
        // lane s < 8 publishes slot s: softmax over the eight chosen logits, the first
        // (largest) subtracted, summed in slot order (Softmax Qwen36Model.cs:293-298)
        uint32_t sid = 0;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const uint32_t id = lane_value(myid, __ffsll((long long)__ballot(myrank == s)) - 1);
            sid = lane == s ? id : sid;
        }
        const float sv = cv[sid];
        const float v0 = __uint_as_float(lane_value(__float_as_uint(sv), 0));
        float total = 0.f;
#pragma unroll
        for (int s = 0; s < 8; s++) total += __expf(__uint_as_float(lane_value(__float_as_uint(sv), s)) - v0);
        if (lane < 8) {
            P.ids[lane] = bad ? 0u : sid;
            // NaN marks the step as failed: K3 leaves the residual unchanged
            P.probs[lane] = bad ? __builtin_nanf("") : __expf(sv - v0) / total;
        }
        if (lane == 0 && bad && P.status) *P.status = 1u;
    }
    float a[1], u[1];
    if constexpr (BITS == 8) {
        uint32_t xr[16];
        float mult;
        const float xs = lane_xh(xr, xh, xhs, xhm, L, mult);
        rows_dot_h8<1>(G, xr, xs, mult, L.valid, L.lpr, a);
        rows_dot_h8<1>(U, xr, xs, mult, L.valid, L.lpr, u);
    } else {
        float x[32];
        const float xs = lane_x_lds(x, xl, xsl, L);
        rows_dot<BITS, 1>(G, x, xs, L.valid, L.lpr, a);
        rows_dot<BITS, 1>(U, x, xs, L.valid, L.lpr, u);
    }
    DIH_TL(1, 2);
    if (L.j == 0 && base + L.g < P.I) P.act[(size_t)slot * P.I + base + L.g] = siluf_(a[0]) * u[0];
    DIH_TL(1, 3);
}

// ------------------------------------------------------------------------------- K3

template <int BITS, int NV>
__global__ __launch_bounds__(576) void decode_down_kernel(DecodeParams P) {
    __shared__ float part[9][64];
    // the nine activation rows (8 slots, then the shared expert) staged once per block as f32
    // in the xl_at layout, row r at r*I, plus per-row chunk sums at 9*I + r*I/32
    extern __shared__ __align__(16) float stage[];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int row0 = blockIdx.x * P.down_rows;
    const LaneGeom L = lane_geom(P.I, P.lpr_i);
    DIH_TL(2, 0);
    // merge operands first (wave 0 lanes < down_rows merge); the residual bits are loaded
    // unconditionally and converted at the merge, so that no wait follows the load
    const int h = row0 + lane;
    const float route = P.sroute[0];
    float pr[8];
#pragma unroll
    for (int s = 0; s < 8; s++) pr[s] = P.probs[s];
    const int hc = h < P.H ? h : P.H - 1;
    const uint32_t rbits = P.residual_f32 ? static_cast<const uint32_t *>(P.residual)[hc]
                                          : (uint32_t) static_cast<const uint16_t *>(P.residual)[hc];
    const bool shared = wave == 8;
    // activations first (NV coalesced float4 per thread), then the expert id (a
    // wave-uniform scalar load, so waiting for it does not wait for the activations), then
    // the weights that depend on it
    const int n4 = 9 * (P.I >> 2), q4 = P.I >> 2;
    float4 av[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        int i = t + 576 * k;
        i = i < n4 ? i : n4 - 1;
        const int slot = i / q4, f = i - slot * q4;
        const float *src = slot < 8 ? P.act + (size_t)slot * P.I : P.sact;
        av[k] = reinterpret_cast<const float4 *>(src)[f];
    }
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t e = wv == 8 ? 0u : P.ids[wv];
    const uint32_t *wp = shared ? P.sdp : P.dp;
    const uint16_t *ws = shared ? P.sds : P.ds, *wb = shared ? P.sdb : P.db;
    Rows<BITS, kDownGroups> R;
    rows_load<BITS, kDownGroups>(R, wp, ws, wb, (size_t)e * P.H, P.H, row0, L.rpw, L.g, L.jc, P.I);
    DIH_TL(2, 1);
    // staging: eight consecutive threads hold the eight float4 of one 32-value chunk
    float *xsums = stage + 9 * P.I;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int i = t + 576 * k;
        float sum = (av[k].x + av[k].y) + (av[k].z + av[k].w);
        sum += dppf<DIH_DPP_XOR1>(sum);
        sum += dppf<DIH_DPP_XOR2>(sum);
        sum += dppf<DIH_DPP_HALF_MIRROR>(sum);
        if (i < n4) {
            const int slot = i / q4, f = i - slot * q4, c = f >> 3;
            *reinterpret_cast<float4 *>(&stage[slot * P.I + xl_at(c, 4 * (f & 7))]) = av[k];
            if ((f & 7) == 0) xsums[slot * (P.I >> 5) + c] = sum;
        }
    }
    __syncthreads();
    float x[32];
    const float xs = lane_x_lds(x, stage + wave * P.I, xsums + wave * (P.I >> 5), L);
    float v[kDownGroups];
    rows_dot<BITS, kDownGroups>(R, x, xs, L.valid, L.lpr, v);
    DIH_TL(2, 2);
#pragma unroll
    for (int q = 0; q < kDownGroups; q++)
        if (L.j == 0) part[wave][q * L.rpw + L.g] = v[q];
    __syncthreads();
    if (wave == 0 && lane < P.down_rows && h < P.H) {
        const float sh = part[8][lane];
        float y = sh * sigmoidf_(route);
#pragma unroll
        for (int s = 0; s < 8; s++) y += part[s][lane] * pr[s];
        // NaN probabilities: non-finite router logits, the residual stays as it was
        if (!__builtin_isnan(pr[0]))
            residual_store(P.residual, P.residual_f32, h, (P.residual_f32 ? __uint_as_float(rbits) : bf16_to_f32(rbits)) + y);
        if (P.route_out) {
#pragma unroll
            for (int s = 0; s < 8; s++) P.route_out[(size_t)s * P.H + h] = part[s][lane];
            P.route_out[(size_t)8 * P.H + h] = sh;
        }
    }
    DIH_TL(2, 3);
}

// ----------------------------------------------------------------------------- host

static int pow2ceil_(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

bool decode_fast_path_ok(const Matrix *router, const Matrix *gate, const Matrix *down, const Matrix *sg,
                         const Matrix *sd, const Matrix *sr) {
    const int E = gate->experts, H = gate->columns, I = gate->rows;
    return (!router || router->bits == 8) && sr->bits == 8 && sg->bits == gate->bits &&
           sd->bits == gate->bits && down->bits == gate->bits && sg->rows == I && sd->columns == I &&
           H <= 2048 && I <= 1024 && E <= kMaxExperts && (gate->bits == 8 || gate->bits == 5);
}

bool launch_moe_decode(const DecodeLaunch &a, hipStream_t s, char *error, int capacity) {
    DecodeParams P{};
    const Matrix *gate = a.gate;
    P.E = gate->experts; P.H = gate->columns; P.I = gate->rows;
    P.lpr_h = std::min(64, pow2ceil_(P.H / 32));
    P.lpr_i = std::min(64, pow2ceil_(P.I / 32));
    if (a.router) { P.rp = a.router->packed(); P.rs = a.router->scales(); P.rb = a.router->biases(); }
    P.logits_in = a.logits_in;
    P.logits = a.logits;
    P.sgp = a.shared_gate->packed(); P.sgs = a.shared_gate->scales(); P.sgb = a.shared_gate->biases();
    P.sup = a.shared_up->packed(); P.sus = a.shared_up->scales(); P.sub = a.shared_up->biases();
    P.srp = a.shared_route->packed(); P.srs = a.shared_route->scales(); P.srb = a.shared_route->biases();
    P.sact = a.sact; P.sroute = a.sroute;
    P.gp = gate->packed(); P.gs = gate->scales(); P.gb = gate->biases();
    P.upp = a.up->packed(); P.us = a.up->scales(); P.ub = a.up->biases();
    P.dp = a.down->packed(); P.ds = a.down->scales(); P.db = a.down->biases();
    P.sdp = a.shared_down->packed(); P.sds = a.shared_down->scales(); P.sdb = a.shared_down->biases();
    P.act = a.act; P.ids = a.ids; P.probs = a.probs; P.status = a.status;
    P.x = a.x; P.residual = a.residual; P.residual_f32 = a.residual_f32; P.route_out = a.route_out;
    const int rpw = 64 / P.lpr_h;
    P.nchunks = (P.E + kK1Waves * kRouterGroups * rpw - 1) / (kK1Waves * kRouterGroups * rpw);
    P.shared_blocks = (P.I + kK1Waves * rpw - 1) / (kK1Waves * rpw);
    P.gate_blocks = (P.I + kWaves * rpw - 1) / (kWaves * rpw);
    P.down_rows = std::min(64, kDownGroups * (64 / P.lpr_i));
    const int k1 = P.nchunks + P.shared_blocks + 1;
    const int k2 = 8 * P.gate_blocks;
    const int k3 = (P.H + P.down_rows - 1) / P.down_rows;
    const size_t k3_lds = (size_t)9 * P.I * 4 + (size_t)9 * (P.I / 32) * 4;
    if (gate->bits == 8) {
        prof_stage("decode_router_shared");
        DIH_LAUNCH(decode_router_kernel<8>, dim3(k1), dim3(256), 0, s, P);
        prof_stage("decode_experts_gate_up");
        DIH_LAUNCH(decode_experts_kernel<8>, dim3(k2), dim3(kWaves * 64), 0, s, P);
        prof_stage("decode_down_merge");
        // float4 activation loads per K3 thread: 9 rows of I floats over 576 threads
        // (I <= 1024: at most four; the staged rows then take at most 37 KB of LDS)
        const int nv = (9 * (P.I / 4) + 575) / 576;
        if (nv <= 1) DIH_LAUNCH((decode_down_kernel<8, 1>), dim3(k3), dim3(576), k3_lds, s, P);
        else if (nv <= 2) DIH_LAUNCH((decode_down_kernel<8, 2>), dim3(k3), dim3(576), k3_lds, s, P);
        else DIH_LAUNCH((decode_down_kernel<8, 4>), dim3(k3), dim3(576), k3_lds, s, P);
    } else {
        prof_stage("decode_router_shared");
        DIH_LAUNCH(decode_router_kernel<5>, dim3(k1), dim3(256), 0, s, P);
        prof_stage("decode_experts_gate_up");
        DIH_LAUNCH(decode_experts_kernel<5>, dim3(k2), dim3(kWaves * 64), 0, s, P);
        prof_stage("decode_down_merge");
        const int nv = (9 * (P.I / 4) + 575) / 576;
        if (nv <= 1) DIH_LAUNCH((decode_down_kernel<5, 1>), dim3(k3), dim3(576), k3_lds, s, P);
        else if (nv <= 2) DIH_LAUNCH((decode_down_kernel<5, 2>), dim3(k3), dim3(576), k3_lds, s, P);
        else DIH_LAUNCH((decode_down_kernel<5, 4>), dim3(k3), dim3(576), k3_lds, s, P);
    }
    return hip_ok(hipGetLastError(), error, capacity, "decode MoE launch");
}

}  // namespace dih

#ifdef DIH_DECODE_TIMELINE
// Measurement build only: copy out / clear the stamps (layout [kernel][block][wave][point]).
extern "C" __attribute__((visibility("default"))) int dih_decode_timeline_read(unsigned long long *host, int n) {
    if (n < 0 || (size_t)n > sizeof(dih::g_decode_timeline) / 8) return -1;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(dih::g_decode_timeline), (size_t)n * 8) == hipSuccess ? 0 : -1;
}
extern "C" __attribute__((visibility("default"))) int dih_decode_timeline_clock_khz() {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    return hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess ? khz : -1;
}
extern "C" __attribute__((visibility("default"))) int dih_decode_timeline_clear() {
    static unsigned long long zero[sizeof(dih::g_decode_timeline) / 8];
    return hipMemcpyToSymbol(HIP_SYMBOL(dih::g_decode_timeline), zero, sizeof(zero)) == hipSuccess ? 0 : -1;
}
#endif
