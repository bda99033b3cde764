// Grouped (MoE) and dense quantized GEMM on gfx950 bf16 MFMA.
//
// Block: four waves sharing one tile of up to BN = 32*NT routes (tokens) of one expert; wave
// w owns 32 weight rows (and, for the gated kernel, the same 32 rows of the up matrix),
// so a block covers 128 weight rows. Each wave computes 32 rows x 32*ntiles routes with
// v_mfma_f32_32x32x16_bf16 and fp32 accumulators, K streamed in 64-column affine groups.
//
// K permutation: MFMA j (j = 0..3) of a 64-column group takes its 16 K-slots from columns
// {32h + 8j + i : h in {0,1}, i in 0..7}, h being the lane's half of the wave. Lane
// (row r, half h) then needs exactly the 32 consecutive codes [32h, 32h+32) of its row in
// that group (one Chunk: 32 bytes 8-bit, 20 bytes 5-bit), dequantized in registers
// straight into MFMA A operands as bf16(fp32(q*scale+bias)) with round-to-nearest-even
// (the rounding of prefill_expert_packed.mm:24-35), and lane (route n, half h) needs the
// 32 consecutive bf16 activations [32h, 32h+32) of its route.
//
// Activations (B): the block gathers each K step's tile (routes x 64 bf16) from global
// memory by route (gate/up: token row = route/8, shared expert rows after the routed ones;
// down: row = route) into an LDS double buffer whose rows are padded to 144 bytes, so the
// 16-byte MFMA operand reads of 32 consecutive routes hit distinct banks. The next step's
// tile is fetched into registers while the current step's MFMAs run.
//
// Pipeline: a K step's weight words (codes and the raw bf16 bits of scales and biases) and
// its activation tile are requested D steps before they are used, into register rings of
// depth D. Vector-memory counters retire in issue order, so the only waits are for loads
// issued D-1 steps earlier: the weight words of the current step, and the activation tile
// of the next step, which is written to the other LDS buffer after this step's MFMAs.
//
// Work: grouped launches list no chunks on the host. Every block reads the E(+1) route
// counts, forms ceil(count/BN) chunks per expert in expert order with a wave prefix sum and
// finds its own (row tile, chunk); blocks past the work exit. Logical work item
// L = rowtile * n_chunks + chunk runs on physical block b with L = (b % 8) * ceil(W/8) +
// b / 8, so consecutive items land on one XCD at nearly the same time and chunks of one
// popular expert share that expert's weight rows in the XCD's L2. This replaces the
// reference's atomic tile list and indirect dispatch (prefill_moe.mm:8-22) with a
// deterministic order.
#include <type_traits>

#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

namespace {

constexpr int kRowPad = 72;          // bf16 per LDS activation row (64 + 8 pad = 144 B)

struct QmmParams {
    const uint32_t *p0, *p1; const uint16_t *s0, *s1, *b0, *b1;     // routed
    const uint32_t *sp0, *sp1; const uint16_t *ss0, *ss1, *sb0, *sb1;  // shared expert
    int experts, rows, columns, tokens, dense, in_mode, y_bf16, row_tiles;
    int rtb, rt_groups;                // streaming kernel: row tiles per block, groups of them
    int ngroups;                       // experts (+1 with a shared expert)
    const uint32_t *routes;            // [ngroups * tokens]
    const uint32_t *counts;            // [ngroups]
    int max_work;                      // grid work items (upper bound)
    const uint16_t *x; void *y;
};

template <int BITS, bool GATED>
struct KStep {
    Chunk<BITS> a0;
    Chunk<BITS> a1[1];
    uint32_t s0, bb0, s1, bb1;
};

// Chunks of up to BN routes per group, in group order: returns the group of chunk `ci`
// and the chunk's first route within that group, plus the total number of chunks. One
// wave; every lane receives the result.
template <int BN>
DIH_DEV int chunk_of(const uint32_t *counts, int ngroups, int ci, int &group, int &first, int &count) {
    const int lane = threadIdx.x & 63;
    // lane l owns groups 5l .. 5l+4 (ngroups <= 320)
    int cnt[5], raw[5], run = 0;
#pragma unroll
    for (int i = 0; i < 5; i++) {
        const int g = lane * 5 + i;
        raw[i] = g < ngroups ? (int)counts[g] : 0;
        cnt[i] = (raw[i] + BN - 1) / BN;
        run += cnt[i];
    }
    // inclusive wave prefix sum of the lane totals
    int incl = run;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        if (lane >= d) incl += v;
    }
    const int total = __shfl(incl, 63, 64);
    const int excl = incl - run;
    // the lane whose range holds chunk ci
    const bool mine = ci >= excl && ci < incl;
    const unsigned long long m = __ballot(mine);
    const int owner = m ? (int)__builtin_ctzll(m) : 0;
    int g = 0, f = 0, n = 0;
    if (mine) {
        int c = ci - excl;
#pragma unroll
        for (int i = 0; i < 5; i++) {
            if (c >= 0 && c < cnt[i]) { g = lane * 5 + i; f = c * BN; n = raw[i]; }
            c -= cnt[i];
        }
    }
    group = __shfl(g, owner, 64);
    first = __shfl(f, owner, 64);
    count = __shfl(n, owner, 64);
    return total;
}

// Total chunks of up to BN routes over the groups, the count chunk_of returns. One wave;
// every lane receives it.
template <int BN>
DIH_DEV int chunk_total(const uint32_t *counts, int ngroups) {
    const int lane = threadIdx.x & 63;
    int run = 0;
#pragma unroll
    for (int i = 0; i < 5; i++) {
        const int g = lane * 5 + i;
        const int raw = g < ngroups ? (int)counts[g] : 0;
        run += (raw + BN - 1) / BN;
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) run += __shfl_xor(run, d, 64);
    return run;
}

// The MFMAs of one 64-column K step over the first NTU route tiles; each 16-column slice's
// B operands are read from LDS before its MFMAs so the reads overlap.
template <bool GATED, int NTU, int NT>
DIH_DEV void mfma_step(const uint16_t *bb, const dih_bf16x8 (&a0)[4], const dih_bf16x8 (&a1)[4],
                       dih_f32x16 (&acc0)[NT], dih_f32x16 (&acc1)[GATED ? NT : 1]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        dih_bf16x8 bx[NTU];
#pragma unroll
        for (int i = 0; i < NTU; i++)
            bx[i] = *reinterpret_cast<const dih_bf16x8 *>(bb + (32 * i) * kRowPad + 8 * j);
#pragma unroll
        for (int i = 0; i < NTU; i++) {
            acc0[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[j], bx[i], acc0[i], 0, 0, 0);
            if constexpr (GATED)
                acc1[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[j], bx[i], acc1[i], 0, 0, 0);
        }
    }
}

}  // namespace

template <int BITS, bool GATED, int NT, int D>
__global__ __launch_bounds__(256, 2) void qmm_kernel(QmmParams P) {
    constexpr int BN = 32 * NT;
    __shared__ __align__(16) uint16_t bs[2][BN * kRowPad];
    __shared__ int xoff[BN];           // element offset of each route's input row
    __shared__ int route_s[BN];
    __shared__ int work[4];            // expert, first route, valid routes, row tile

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    // ---- which work item is this block? Physical block b runs logical item
    // L = xcd_item(b, items) (consecutive items on one XCD at nearly the same time),
    // item L = chunk * row_tiles + row tile.
    if (wave == 0) {
        int e = 0, first = 0, nvalid = 0, rt = -1;
        const int chunks = P.dense ? (P.tokens + BN - 1) / BN : chunk_total<BN>(P.counts, P.ngroups);
        const int L = xcd_item((int)blockIdx.x, chunks * P.row_tiles);
        const int ci = L < 0 ? chunks : L / P.row_tiles;
        if (P.dense) {
            if (L >= 0 && ci * BN < P.tokens) {
                rt = L - ci * P.row_tiles;
                first = ci * BN;
                nvalid = min(BN, P.tokens - first);
            }
        } else {
            int count;
            const int total = chunk_of<BN>(P.counts, P.ngroups, ci, e, first, count);
            if (L >= 0 && ci < total) {
                rt = L - ci * P.row_tiles;
                nvalid = min(BN, count - first);
            }
        }
        if (lane == 0) { work[0] = e; work[1] = first; work[2] = nvalid; work[3] = rt; }
    }
    __syncthreads();
    const int rt = work[3];
    if (rt < 0) return;
    const int e = work[0], first = work[1], nvalid = work[2];
    const int ntiles = (nvalid + 31) >> 5;
    const int C = P.columns, R = P.rows, G = C >> 6;

    // ---- the chunk's route ids first (their wait must not include the weight stream)
    int my_route = 0;
    if (t < BN) {
        const int n = t < nvalid ? t : 0;
        my_route = P.dense ? first + n : (int)P.routes[(size_t)e * P.tokens + first + n];
    }

    // ---- weights of this wave's 32 rows
    const bool shared = !P.dense && e == P.experts;
    const uint32_t *pw0 = shared ? P.sp0 : P.p0;
    const uint16_t *ps0 = shared ? P.ss0 : P.s0, *pb0 = shared ? P.sb0 : P.b0;
    const uint32_t *pw1 = shared ? P.sp1 : P.p1;
    const uint16_t *ps1 = shared ? P.ss1 : P.s1, *pb1 = shared ? P.sb1 : P.b1;
    const int eix = shared ? 0 : e;
    const int r = lane & 31, h = lane >> 5;
    const int row = rt * 128 + wave * 32 + r;
    const int rr = row < R ? row : R - 1;
    const size_t rowi = (size_t)eix * R + rr;
    const size_t wpr = (size_t)C * BITS / 32;
    const uint32_t *w0 = pw0 + rowi * wpr;
    const uint32_t *w1 = GATED ? pw1 + rowi * wpr : nullptr;
    const uint16_t *sc0 = ps0 + rowi * G, *bi0 = pb0 + rowi * G;
    const uint16_t *sc1 = GATED ? ps1 + rowi * G : nullptr, *bi1 = GATED ? pb1 + rowi * G : nullptr;

    KStep<BITS, GATED> ring[D];
    auto load_a = [&](KStep<BITS, GATED> &k, int kg) {
        kg = kg < G ? kg : G - 1;
        load_chunk<BITS>(k.a0, w0, 2 * kg + h);
        k.s0 = sc0[kg];
        k.bb0 = bi0[kg];
        if constexpr (GATED) {
            load_chunk<BITS>(k.a1[0], w1, 2 * kg + h);
            k.s1 = sc1[kg];
            k.bb1 = bi1[kg];
        }
    };

#pragma unroll
    for (int d = 0; d < D; d++) load_a(ring[d], d);

    // ---- input rows of the chunk's routes (past nvalid: the first route's row)
    const int T8 = P.tokens * 8;
    if (t < BN) {
        int in_row = my_route;
        if (P.in_mode == 1) in_row = my_route < T8 ? (my_route >> 3) : my_route - T8;
        route_s[t] = my_route;
        xoff[t] = in_row * C;
    }

    __syncthreads();  // xoff ready
    // ---- activation tile loader: thread t moves 16-byte piece p of routes n0 + 32*i
    const int p = t & 7, n0 = t >> 3;
    int xo[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) xo[i] = xoff[i * 32 < nvalid ? n0 + 32 * i : n0] + 8 * p;
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    u32x4 bv[D][NT];
    // (unconditional: tiles past ntiles re-read the first route's row, a cache hit, and
    // keep the ring in registers)
    auto load_b = [&](u32x4 (&v)[NT], int kg) {
        kg = kg < G ? kg : G - 1;
#pragma unroll
        for (int i = 0; i < NT; i++) v[i] = *reinterpret_cast<const u32x4 *>(P.x + xo[i] + 64 * kg);
    };
    auto store_b = [&](const u32x4 (&v)[NT], int buf) {
#pragma unroll
        for (int i = 0; i < NT; i++) *reinterpret_cast<u32x4 *>(&bs[buf][(n0 + 32 * i) * kRowPad + 8 * p]) = v[i];
    };
#pragma unroll
    for (int d = 0; d < D; d++) load_b(bv[d], d);
    store_b(bv[0], 0);
    __syncthreads();

    dih_f32x16 acc0[NT], acc1[GATED ? NT : 1];
#pragma unroll
    for (int i = 0; i < NT; i++) {
#pragma unroll
        for (int k = 0; k < 16; k++) acc0[i][k] = 0.f;
    }
    if constexpr (GATED) {
#pragma unroll
        for (int i = 0; i < NT; i++) {
#pragma unroll
            for (int k = 0; k < 16; k++) acc1[i][k] = 0.f;
        }
    }

    for (int kg0 = 0; kg0 < G; kg0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int kg = kg0 + d;
            if (kg < G) {
                // keep each step's work inside its step: hoisting a later step's dequant
                // would make this step wait for that step's loads
                __builtin_amdgcn_sched_barrier(0);
                const int buf = kg & 1;
                dih_bf16x8 a0[4], a1[4];
                chunk_to_bf16<BITS>(ring[d].a0, bf16_to_f32(ring[d].s0), bf16_to_f32(ring[d].bb0), a0);
                if constexpr (GATED) chunk_to_bf16<BITS>(ring[d].a1[0], bf16_to_f32(ring[d].s1), bf16_to_f32(ring[d].bb1), a1);
                // step kg + D: weights and activations (clamped in bounds past the end)
                load_a(ring[d], kg + D);
                load_b(bv[d], kg + D);
                const uint16_t *bb = &bs[buf][r * kRowPad + 32 * h];
                // all NT tiles, branch-free (tiles past ntiles compute on a repeated route and
                // are not stored; for chunks of a few routes the weight stream, not the MFMA
                // pipe, bounds the step)
                mfma_step<GATED, NT, NT>(bb, a0, a1, acc0, acc1);
                // the next step's activations (requested D-1 steps ago) into the other buffer
                if (kg + 1 < G) store_b(bv[(d + 1) % D], buf ^ 1);
                __syncthreads();
            }
        }
    }

    // ---- epilogue: lane holds route n = 32i + r, rows 8*(k/4) + 4h + (k%4) of the tile
    const int row_base = rt * 128 + wave * 32;
#pragma unroll
    for (int i = 0; i < NT; i++) {
        const int n = 32 * i + r;
        if (i >= ntiles || n >= nvalid) continue;
        const int route = route_s[n];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int m0 = row_base + 8 * q + 4 * h;
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float g = acc0[i][4 * q + k];
                if constexpr (GATED) v[k] = siluf_(g) * acc1[i][4 * q + k];
                else v[k] = g;
            }
            const size_t o = (size_t)route * R + m0;
            // vector stores only where the row offset keeps them naturally aligned
            if ((R & 3) == 0 && m0 + 3 < R) {
                if (P.y_bf16) {
                    uint2 pk = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(P.y) + o) = pk;
                } else {
                    *reinterpret_cast<float4 *>(static_cast<float *>(P.y) + o) = make_float4(v[0], v[1], v[2], v[3]);
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

// ---------------------------------------------------------------------------------------
// Streaming variant for K a multiple of 512 (every model shape): weight codes and activation
// tiles reach LDS through direct global->LDS loads (global_load_lds), S stages deep, so the
// memory instructions are coalesced (a weight tile is read four lanes per 64-byte row
// segment; an activation tile eight lanes per 128-byte route segment) instead of one
// lane per row. Both tiles are stored with a 16-byte-piece swizzle that makes the MFMA
// operand reads conflict-free:
//   weights, 8-bit : row r, piece p (of 4) at r*64 + 16*(p ^ ((r >> 2) & 3))
//   weights, 5-bit : row r, dword d (of 10) at (r*10 + d)*4 (10 is coprime to 32 banks/2)
//   activations    : route n, piece p (of 8) at n*128 + 16*(p ^ ((n >> 1) & 7))
// Scales and biases come from registers: each lane loads its row's bf16 bits for eight
// groups at a time (one 16-byte load per array per eight K steps).
// One explicit vmcnt wait and one barrier per K step: step kg's copies were issued S-1
// steps earlier; the copies of the following S-2 steps stay in flight.
// A block streams up to rtb row tiles of one route chunk as one continuous step sequence
// (the ring runs across tile boundaries; each tile ends with its epilogue). Only the stages
// live in LDS: every wave derives the work item and its routes itself, so narrow tiles
// (64 routes, one matrix) fit two blocks per CU.

// (to_lds, wait_vm, wait_lgkm0 and barrier_no_fence are in dih_device.h)

// Blocks per CU the streaming kernel is built for: two for the narrow route tiles (two
// 32-route tiles per matrix, three for one 5-bit matrix) when four stages fit in half the
// LDS; the VGPR budget is then 256 per lane, accumulators included. The split gated form
// (eight waves) runs one block.
template <int BITS, bool GATED, int NT, bool SPLIT>
constexpr int qmm_lds_occupancy() {
    return !SPLIT && (GATED ? 2 : 1) * NT <= (BITS == 5 ? 3 : 2) &&
                   4 * ((GATED ? 2 : 1) * 128 * (64 * BITS / 8) + 32 * NT * 128) <= 80 * 1024
               ? 2 : 1;
}

// SPLIT (gated only): eight waves, waves 0-3 the gate matrix and 4-7 the up matrix of the
// same four 32-row slabs, so that two waves share each SIMD and one's dequant overlaps the
// other's MFMAs and waits; the SwiGLU epilogue meets the two halves in LDS.
// RS (dense only): 32-row slabs per wave, so a block's row tile is 128*RS rows. Two slabs
// double the MFMA work per activation tile read from LDS (each wave reads the whole tile
// every step), which otherwise costs as much LDS bandwidth as the MFMAs take time.
// TL: the codes come from the matrix's 128-row tile-major copy (5-bit): a K step of 128 rows
// is one contiguous 5,120-byte block, so each dword copy instruction of a wave reads 256
// contiguous bytes instead of pieces of six or seven rows 1,280 bytes apart.
// NTC: route tiles multiplied (chunks of 32 * NTC routes) out of the NT tiles' slots the
// copies fill (slots past NTC tiles repeat the chunk's first route and are not multiplied):
// 96-route chunks for the 5-bit gated launches of config-4-like routing, where no expert
// then needs a second chunk.
template <int BITS, bool GATED, int NT, int S, bool SPLIT, int RS = 1, bool TL = false, int NTC = NT>
__global__ __launch_bounds__(SPLIT ? 512 : 256, (RS > 1 ? 1 : qmm_lds_occupancy<BITS, GATED, NT, SPLIT>())) void qmm_lds_kernel(QmmParams P) {
    // 32-route tiles (NT = 1) serve the 8-bit grouped down projection of sparse routing only
    // (gate/up measured slower: config 3 181 -> 247 us). Their earlier wrong results, like
    // other schedule-dependent failures of this kernel, came from MFMAs reading bf16 operands
    // converted by inline asm one instruction earlier; the conversion is now visible to the
    // compiler.
    static_assert(!SPLIT || GATED, "only the gated kernel splits its matrices over waves");
    static_assert(RS == 1 || (!GATED && !SPLIT), "two slabs a wave: non-gated only");
    static_assert(!TL || BITS == 5, "tile-major codes: 5-bit only");
    constexpr int TR = 128 * RS;             // rows per row tile
    constexpr int NW = SPLIT ? 8 : 4;        // waves per block
    static_assert(NTC >= 1 && NTC <= NT, "compute tiles within the copied route slots");
    constexpr int BN = 32 * NTC;             // routes per chunk (multiplied)
    constexpr int BC = 32 * NT;              // route slots copied per step (>= BN)
    constexpr int AB = 64 * BITS / 8;        // bytes of one row's codes per K step
    constexpr int A_ST = TR * AB;            // one matrix, one stage
    constexpr int NMAT = GATED ? 2 : 1;
    constexpr int WMAT = SPLIT ? 1 : NMAT;   // matrices one wave dequantizes
    constexpr int B_ST = BC * 128;
    constexpr int ST = NMAT * A_ST + B_ST;   // bytes per stage
    constexpr int AQ = (BITS == 8 ? 2 : 5) * RS;   // direct copies per wave per matrix per step
    constexpr int NBW = 4 * NT / NW;         // activation copies (8 routes each) per wave
    static_assert(NBW >= 1 && NBW * NW == 4 * NT, "activation pieces split evenly over the waves");
    constexpr int LPS = WMAT * AQ + NBW;     // copies per thread per step
    static_assert(S == 4, "the stage of step s is s % 4, static within the eight-step unroll");
    // one array per stage: with the stage known at compile time the compiler can tell that an
    // operand read does not alias the copies in flight to the other stages. Nothing else
    // lives in LDS (the split form adds the SwiGLU exchange), so that two blocks fit on a
    // CU when the stages take half of it.
    __shared__ __align__(16) unsigned char st0[ST], st1[ST], st2[ST], st3[ST];
    // split: silu(gate) of XNT route tiles at a time (in halves when four tiles would not fit
    // beside the stages)
    constexpr int XNT = SPLIT && NTC > 3 ? NTC / 2 : NTC;
    __shared__ __align__(16) float xch[SPLIT ? 4 * XNT * 16 * 64 : 1];
    lds_escape(st0, st1, st2, st3, xch);
    auto stage_base = [&](int stage) -> unsigned char * {
        return stage == 0 ? st0 : stage == 1 ? st1 : stage == 2 ? st2 : st3;
    };

    // the wave index is uniform: in a scalar register, LDS copy destinations need no readfirstlane
    const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const int slab = wave & 3;                // 32-row slab of the 128-row tile
    const int mw = SPLIT ? wave >> 2 : 0;     // split: the matrix this wave computes
    // ---- work item (every wave derives it): physical block b runs logical item
    // L = xcd_item(b, items); L = chunk * rt_groups + row-tile group, a group being up to
    // rtb consecutive row tiles
    int e = 0, first = 0, nvalid = 0, rt0 = -1, nrt = 0;
    {
        const int chunks = P.dense ? (P.tokens + BN - 1) / BN : chunk_total<BN>(P.counts, P.ngroups);
        const int L = xcd_item((int)blockIdx.x, chunks * P.rt_groups);
        const int ci = L < 0 ? chunks : L / P.rt_groups;
        bool ok;
        if (P.dense) {
            ok = L >= 0 && ci * BN < P.tokens;
            if (ok) { first = ci * BN; nvalid = min(BN, P.tokens - first); }
        } else {
            int count;
            const int total = chunk_of<BN>(P.counts, P.ngroups, ci, e, first, count);
            ok = L >= 0 && ci < total;
            if (ok) nvalid = min(BN, count - first);
        }
        if (ok) {
            rt0 = (L - ci * P.rt_groups) * P.rtb;
            nrt = min(P.rtb, P.row_tiles - rt0);
        }
    }
    // the work item is the same in every lane (it came through cross-lane shuffles, which
    // the compiler cannot see are uniform): keep it in scalar registers so that the step
    // bookkeeping and the loops over tiles stay scalar
    e = __builtin_amdgcn_readfirstlane(e);
    first = __builtin_amdgcn_readfirstlane(first);
    nvalid = __builtin_amdgcn_readfirstlane(nvalid);
    rt0 = __builtin_amdgcn_readfirstlane(rt0);
    nrt = __builtin_amdgcn_readfirstlane(nrt);
    if (rt0 < 0) return;
    const int C = P.columns, R = P.rows, G = C >> 6;
    // route of the chunk's n-th slot (slots past the chunk repeat its first route)
    auto route_at = [&](int n) -> int {
        n = n < nvalid ? n : 0;
        return P.dense ? first + n : (int)P.routes[(size_t)e * P.tokens + first + n];
    };

    // ---- weights
    const bool shared = !P.dense && e == P.experts;
    const char *pw[2] = {reinterpret_cast<const char *>(shared ? P.sp0 : P.p0),
                         reinterpret_cast<const char *>(shared ? P.sp1 : P.p1)};
    const uint16_t *psc[2] = {shared ? P.ss0 : P.s0, shared ? P.ss1 : P.s1};
    const uint16_t *pbi[2] = {shared ? P.sb0 : P.b0, shared ? P.sb1 : P.b1};
    const size_t ebase = (size_t)(shared ? 0 : e) * R;
    const size_t row_bytes = (size_t)C * BITS / 8;
    auto row_index = [&](int rt, int rb) {  // (row tile, row in tile) -> matrix row (clamped)
        const int row = rt * TR + rb;
        return ebase + (row < R ? row : R - 1);
    };
    // this lane's copy rows within a tile and byte offsets within a row's K-step segment
    int crow[AQ], coff[AQ];
#pragma unroll
    for (int q = 0; q < AQ; q++) {
        if constexpr (BITS == 8) {
            const int rl = 16 * q + (lane >> 2), sl = lane & 3;
            crow[q] = slab * 32 * RS + rl;
            coff[q] = 16 * (sl ^ ((rl >> 2) & 3));
        } else {
            const int i = 64 * q + lane, rl = i / 10;
            crow[q] = slab * 32 * RS + rl;
            coff[q] = 4 * (i - rl * 10);
        }
    }
    // this lane's MFMA row; its scale/bias bf16 bits come eight groups per 16-byte load
    const int r = lane & 31, h = lane >> 5;
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    // The loads go through global-address-space pointers: with the matrix picked by the wave
    // (split form) the compiler cannot tell the generic pointer is global, emits FLAT loads,
    // and a FLAT load may read LDS, so it first waits for every LDS copy in flight (a full
    // drain of the copy pipeline once per eight steps).
    typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
    auto win_load = [&](u32x4 (&sw)[RS][2][2], int ti, int w) {
#pragma unroll
        for (int rs = 0; rs < RS; rs++) {
            const size_t mrow = row_index(rt0 + ti, slab * 32 * RS + 32 * rs + r);
#pragma unroll
            for (int m = 0; m < WMAT; m++) {
                sw[rs][m][0] = *(g_u32x4 *)(psc[m + mw] + mrow * G + 8 * w);
                sw[rs][m][1] = *(g_u32x4 *)(pbi[m + mw] + mrow * G + 8 * w);
            }
        }
    };

    // ---- routes -> input row offsets of this lane's activation copies
    const int T8 = P.tokens * 8;
    const uint16_t *bsrc[NBW];
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const int n = (NW * i + wave) * 8 + (lane >> 3), sl = lane & 7;
        const int route = route_at(n);
        const int in_row = P.in_mode == 1 ? (route < T8 ? (route >> 3) : route - T8) : route;
        bsrc[i] = P.x + (size_t)in_row * C + 8 * (sl ^ ((n >> 1) & 7));
    }
    // output routes of this lane's accumulator columns
    int out_route[NTC];
#pragma unroll
    for (int i = 0; i < NTC; i++) out_route[i] = route_at(32 * i + r);
    // route tiles holding a valid route (wave-uniform): the main loop is specialized on it, and
    // the MFMAs and operand reads of the other tiles are skipped (their accumulator columns
    // are never stored)
    const int ntu = __builtin_amdgcn_readfirstlane((nvalid + 31) >> 5);

    // Copy sources: the expert's first row in each matrix (wave-uniform) plus a 32-bit lane
    // offset of the row within the expert (an expert's rows span less than 2^31 bytes, checked
    // on the host); a K step adds the wave-uniform offset kg * KSTEP. Row-major codes: a row
    // starts row * row_bytes in, a K step is AB bytes further. Tile-major codes (experts padded
    // to whole 256-row tiles, so a 256-row dense tile stays inside the copy): a 128-row tile starts tile * 128 * row_bytes in, its row rr
    // rr * AB further, and a K step is 128 * AB bytes. The issue position (the next step to
    // copy, as tile and K step) is wave-uniform, so the step bookkeeping is scalar and no step
    // index is divided at run time.
    constexpr uint32_t KSTEP = TL ? 128 * AB : AB;
    const size_t wrows = TL ? (size_t)((R + 255) & ~255) : (size_t)R;  // code rows per expert
    const char *wbase[WMAT];
#pragma unroll
    for (int mm = 0; mm < WMAT; mm++) wbase[mm] = pw[mm + mw] + (size_t)(shared ? 0 : e) * wrows * row_bytes;
    // Tile-major: the lane's offset within a row tile's first K step is fixed, and a tile adds
    // the wave-uniform tile * TR * row_bytes. No clamp: an expert's last tile reads zero
    // padding rows (in bounds; their outputs are not stored). Held so, the 5-bit kernels spend
    // one add a copy instead of the clamp and index arithmetic (config 4 gate/up 227 -> 216
    // us, down 131 -> 125 us). (8-bit full tiles held the same way measured slower: gate/up
    // 164 -> 178 us on config 3.)
    uint32_t woff[AQ], tpart[AQ];
#pragma unroll
    for (int q = 0; q < AQ; q++)
        tpart[q] = (uint32_t)(crow[q] >> 7) * (uint32_t)(128 * row_bytes) + (uint32_t)(crow[q] & 127) * (uint32_t)AB +
                   (uint32_t)coff[q];
    auto set_tile = [&](int ti) {
        if constexpr (TL) {
            const uint32_t tb = (uint32_t)((rt0 + ti) * TR) * (uint32_t)row_bytes;
#pragma unroll
            for (int q = 0; q < AQ; q++) woff[q] = tb + tpart[q];
        } else {
#pragma unroll
            for (int q = 0; q < AQ; q++) {
                const int row0 = (rt0 + ti) * TR + crow[q];
                const uint32_t row = (uint32_t)(row0 < R ? row0 : R - 1);
                woff[q] = row * (uint32_t)row_bytes + (uint32_t)coff[q];
            }
        }
    };
    int iss_ti = 0, iss_kg = 0;
    set_tile(0);
    // copies step (iss_ti, iss_kg) into `stage`, then moves to the next step; past the last
    // step the last one is copied again
    auto issue = [&](int stage) {
        unsigned char *base = stage_base(stage);
        // The lane offsets are recomputed at every step (a few VALU operations a copy) rather
        // than held across steps: the schedule was tuned this way. (Builds that held them
        // failed parity on one route tile; that failure was most likely the operand hazard of
        // the former inline-asm bf16 conversion, whose placement moved with the schedule.)
        set_tile(iss_ti);
        const uint32_t koff = (uint32_t)iss_kg * KSTEP;
#pragma unroll
        for (int mm = 0; mm < WMAT; mm++) {
            const int m = mm + mw;
#pragma unroll
            for (int q = 0; q < AQ; q++) {
                const char *src = wbase[mm] + (woff[q] + koff);
                if constexpr (BITS == 8)
                    to_lds<16>(src, base + m * A_ST + (slab * 32 * RS + 16 * q) * 64);
                else
                    to_lds<4>(src, base + m * A_ST + slab * 32 * RS * 40 + q * 256);
            }
        }
#pragma unroll
        for (int i = 0; i < NBW; i++) to_lds<16>(bsrc[i] + 64 * iss_kg, base + NMAT * A_ST + (NW * i + wave) * 8 * 128);
        if (iss_kg + 1 < G) {
            iss_kg++;
        } else if (iss_ti + 1 < nrt) {
            iss_ti++;
            iss_kg = 0;
        }
    };

#pragma unroll
    for (int st = 0; st < S - 1; st++) issue(st);
    u32x4 win[RS][2][2], win_next[RS][2][2];
    win_load(win, 0, 0);

    dih_f32x16 acc0[RS][NTC], acc1[GATED && !SPLIT ? NTC : 1];
    auto zero_acc = [&]() {
#pragma unroll
        for (int rs = 0; rs < RS; rs++)
#pragma unroll
            for (int i = 0; i < NTC; i++) {
#pragma unroll
                for (int k = 0; k < 16; k++) acc0[rs][i][k] = 0.f;
            }
        if constexpr (GATED && !SPLIT) {
#pragma unroll
            for (int i = 0; i < NTC; i++) {
#pragma unroll
                for (int k = 0; k < 16; k++) acc1[i][k] = 0.f;
            }
        }
    };
    zero_acc();

    auto run = [&](auto ntu_c) {
    constexpr int NTU = decltype(ntu_c)::value;
    for (int ti = 0; ti < nrt; ti++) {
        for (int kw = 0; kw < G; kw += 8) {
            // the next window of scales: this tile's next one, or the next tile's first
            const bool more = kw + 8 < G || ti + 1 < nrt;
            if (more) win_load(win_next, kw + 8 < G ? ti : ti + 1, kw + 8 < G ? (kw >> 3) + 1 : 0);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                wait_vm<(S - 2) * LPS>();
                barrier_no_fence();
                issue((u + S - 1) % S);
                const unsigned char *base = stage_base(u % S);
                // this step's weights -> bf16 A operands (a[rs * WMAT + m]: slab rs, matrix m)
                dih_bf16x8 a[RS * 2][4];
#pragma unroll
                for (int rs = 0; rs < RS; rs++)
#pragma unroll
                for (int m = 0; m < WMAT; m++) {
                    Chunk<BITS> c;
                    const int wr = slab * 32 * RS + 32 * rs + r;   // row within the tile
                    if constexpr (BITS == 8) {
                        const int sw = (r >> 2) & 3;
                        const unsigned char *ra = base + (m + mw) * A_ST + wr * 64;
                        const u32x4 v0 = *reinterpret_cast<const u32x4 *>(ra + 16 * ((2 * h) ^ sw));
                        const u32x4 v1 = *reinterpret_cast<const u32x4 *>(ra + 16 * ((2 * h + 1) ^ sw));
                        c.w[0] = v0.x; c.w[1] = v0.y; c.w[2] = v0.z; c.w[3] = v0.w;
                        c.w[4] = v1.x; c.w[5] = v1.y; c.w[6] = v1.z; c.w[7] = v1.w;
                    } else {
                        const uint32_t *ra = reinterpret_cast<const uint32_t *>(base + (m + mw) * A_ST) + wr * 10 + 5 * h;
#pragma unroll
                        for (int k = 0; k < 5; k++) c.w[k] = ra[k];
                    }
                    const uint32_t sbits = (win[rs][m][0][u >> 1] >> (16 * (u & 1))) & 0xffffu;
                    const uint32_t bbits = (win[rs][m][1][u >> 1] >> (16 * (u & 1))) & 0xffffu;
                    chunk_to_bf16<BITS>(c, bf16_to_f32(sbits), bf16_to_f32(bbits), a[rs * WMAT + m]);
                }
                // MFMAs over all NT route tiles
                const unsigned char *bb = base + NMAT * A_ST;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    dih_bf16x8 bx[NTU];
#pragma unroll
                    for (int i = 0; i < NTU; i++) {
                        const int n = 32 * i + r, pc = 4 * h + j;
                        bx[i] = *reinterpret_cast<const dih_bf16x8 *>(bb + n * 128 + 16 * (pc ^ ((n >> 1) & 7)));
                    }
#pragma unroll
                    for (int i = 0; i < NTU; i++) {
#pragma unroll
                        for (int rs = 0; rs < RS; rs++)
                            acc0[rs][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[rs * WMAT][j], bx[i], acc0[rs][i], 0, 0, 0);
                        if constexpr (GATED && !SPLIT)
                            acc1[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][j], bx[i], acc1[i], 0, 0, 0);
                    }
                }
            }
            if (more) {
#pragma unroll
                for (int rs = 0; rs < RS; rs++)
#pragma unroll
                    for (int m = 0; m < WMAT; m++) { win[rs][m][0] = win_next[rs][m][0]; win[rs][m][1] = win_next[rs][m][1]; }
            }
        }

        // ---- epilogue of row tile rt0 + ti: lane holds route n = 32i + r, rows
        // 8*(k/4) + 4h + (k%4) of the slab's 32. Split: the gate waves hand silu(g) to the up
        // waves of the same slab through LDS (identical lane layouts), XNT route tiles at a
        // time; the up waves store.
#pragma unroll
        for (int half = 0; half < NTC / XNT; half++) {
        if constexpr (SPLIT) {
            if (half > 0) {   // the up waves have read the previous half
                wait_lgkm0();
                barrier_no_fence();
            }
            float *xw = xch + slab * XNT * 16 * 64 + lane;
            if (mw == 0) {
#pragma unroll
                for (int i = 0; i < XNT; i++) {
#pragma unroll
                    for (int k = 0; k < 16; k++) xw[(i * 16 + k) * 64] = siluf_(acc0[0][half * XNT + i][k]);
                }
            }
            wait_lgkm0();
            barrier_no_fence();
        }
#pragma unroll
        for (int rs = 0; rs < RS; rs++) {
        const int row_base = (rt0 + ti) * TR + slab * 32 * RS + 32 * rs;
#pragma unroll
        for (int ii = 0; ii < XNT; ii++) {
            const int i = half * XNT + ii;
            const int n = 32 * i + r;
            if (n >= nvalid || (SPLIT && mw == 0)) continue;
            const int route = out_route[i];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int m0 = row_base + 8 * q + 4 * h;
                float v[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float g = acc0[rs][i][4 * q + k];
                    if constexpr (SPLIT) v[k] = xch[(slab * XNT * 16 + ii * 16 + 4 * q + k) * 64 + lane] * g;
                    else if constexpr (GATED) v[k] = siluf_(g) * acc1[i][4 * q + k];
                    else v[k] = g;
                }
                const size_t o = (size_t)route * R + m0;
                if ((R & 3) == 0 && m0 + 3 < R) {
                    if (P.y_bf16) {
                        uint2 pk = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(P.y) + o) = pk;
                    } else {
                        *reinterpret_cast<float4 *>(static_cast<float *>(P.y) + o) = make_float4(v[0], v[1], v[2], v[3]);
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
        }
        zero_acc();
    }
    };
    if constexpr (NTC == 4) {
        if (ntu >= 4) run(std::integral_constant<int, 4>{});
        else if (ntu == 3) run(std::integral_constant<int, 3>{});
        else if (ntu == 2) run(std::integral_constant<int, 2>{});
        else run(std::integral_constant<int, 1>{});
    } else if constexpr (NTC == 3) {
        if (ntu >= 3) run(std::integral_constant<int, 3>{});
        else if (ntu == 2) run(std::integral_constant<int, 2>{});
        else run(std::integral_constant<int, 1>{});
    } else if constexpr (NTC == 2) {
        if (ntu >= 2) run(std::integral_constant<int, 2>{});
        else run(std::integral_constant<int, 1>{});
    } else {
        run(std::integral_constant<int, 1>{});
    }
    // no copy may still be writing this block's LDS when the block exits
    __builtin_amdgcn_s_waitcnt(0);
}

// One dword of the tile-major 5-bit copy per thread: flattened row f (= expert * rows + row)
// of [first, first + count), K step kg, dword d of the row's 40-byte piece. Reads walk dev[0]
// in row-major order.
__global__ __launch_bounds__(256) void retile5_kernel(const uint32_t *__restrict__ src, uint32_t *__restrict__ dst,
                                                      size_t first, size_t count, int rows, int G, size_t tile_rows) {
    const size_t total = count * (size_t)G * 10;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t f = first + i / ((size_t)G * 10);
        const int kg = (int)(i / 10 % (size_t)G), d = (int)(i % 10);
        const size_t e = f / (size_t)rows, row = f % (size_t)rows;
        const size_t tile = e * (tile_rows / 128) + row / 128;
        dst[((tile * G + kg) * 128 + row % 128) * 10 + d] = src[f * (size_t)G * 10 + (size_t)kg * 10 + d];
    }
}

bool matrix_retile(Matrix *m, size_t first, size_t count, char *error, int capacity) {
    if (!m->tiled || count == 0) return true;
    const size_t total = count * m->groups_per_row() * 10;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 8192);
    DIH_LAUNCH(retile5_kernel, dim3(blocks), dim3(256), 0, nullptr, m->packed(), static_cast<uint32_t *>(m->tiled),
               first, count, m->rows, (int)m->groups_per_row(), m->tiled_rows());
    return hip_ok(hipGetLastError(), error, capacity, "weight retile") &&
           hip_ok(hipStreamSynchronize(nullptr), error, capacity, "weight retile");
}

// Upper bound of (row tile, chunk) work items: sum_g ceil(count_g / BN) <= routes / BN +
// (groups holding any route); a shared-expert group adds `tokens` routes.
static size_t qmm_max_work(int rows, int tokens, int ngroups, int dense, int bn, int tile_rows = 128) {
    const size_t row_tiles = (size_t)(rows + tile_rows - 1) / tile_rows;
    if (dense) return row_tiles * ((size_t)(tokens + bn - 1) / bn);
    const size_t routes = (size_t)tokens * 9;
    return row_tiles * (routes / bn + std::min<size_t>((size_t)ngroups, routes));
}

bool qmm_wide_gated(const Matrix *gate, int tokens) {
    return gate->bits == 5 && gate->columns % 512 == 0 &&
           (size_t)tokens * 8 > (size_t)48 * (size_t)std::max(1, gate->experts);
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
    P.ngroups = a.ngroups;
    P.routes = a.routes; P.counts = a.counts;
    P.x = a.x; P.y = a.y;
    if (!a.dense && (a.ngroups < 1 || a.ngroups > 320 || !a.routes || !a.counts)) {
        set_error(error, capacity, "Invalid grouped qmm arguments");
        return false;
    }
    // the streaming kernel addresses an expert's weight rows (padded to whole 256-row tiles
    // in the tile-major copy) with 32-bit offsets
    if (m0->tiled_rows() * ((size_t)m0->columns * m0->bits / 8) > 0x7fffffffu) {
        set_error(error, capacity, "Matrix too large for one grouped/dense qmm launch");
        return false;
    }
    // input row offsets (row * columns) are 32-bit in the kernel
    if ((size_t)a.tokens * 9 * (size_t)m0->columns > 0x7fffffffu) {
        set_error(error, capacity, "Chunk too large for one grouped/dense qmm launch");
        return false;
    }
    // Route tile width: 64 routes for the gated kernels, 128 otherwise (the register-ring
    // kernel measured faster so than with narrower tiles and deeper rings). Grouped
    // non-gated streaming launches (K a multiple of 512) use 64: experts average a few
    // routes, and the narrower tile lets two blocks share a CU. Exceptions by the routes
    // per expert follow.
    const bool gated = m1 != nullptr;
    const bool streaming = m0->columns % 512 == 0;
    // 5-bit gated takes 128 route slots when experts average
    // more than 48 routes (uniform routing over E experts: 8T/E): 64-route tiles would give
    // an expert of 65-127 routes a second, mostly empty chunk and dequantize its weights
    // twice (config 4: 64 routes on average, at most ~90)
    const bool wide_gated = streaming && gated && !a.dense && qmm_wide_gated(m0, a.tokens);
    // The grouped 5-bit down projection takes 96-route tiles (still two blocks a CU) when
    // experts average more than 48 routes: config 4's experts (at most ~90 routes) then need
    // one chunk each (down 126 -> 119 us; 128-route tiles, one block a CU, measured 211 ->
    // 274 us). The 8-bit one takes 32-route tiles (three blocks a CU) when experts average
    // at most 16 routes (config 3 down 88.7 -> 86.2 us). Others keep 64-route tiles.
    const bool wide_down = streaming && !gated && !a.dense && m0->bits == 5 &&
                           (size_t)a.tokens * 8 > (size_t)48 * (size_t)std::max(1, m0->experts);
    const bool narrow_down = streaming && !gated && !a.dense && m0->bits == 8 &&
                             (size_t)a.tokens * 8 <= (size_t)16 * (size_t)std::max(1, m0->experts);
    const int nt = streaming && !a.dense && !gated ? (wide_down ? 3 : narrow_down ? 1 : 2)
                                                   : (gated ? (wide_gated ? 4 : 2) : 4);
    // wide 5-bit gated chunks of 96 routes when experts average at most 64 routes (the copies
    // still fill 128 route slots; the MFMAs cover 96)
    const int ntc = wide_gated && (size_t)a.tokens * 8 <= (size_t)64 * (size_t)std::max(1, m0->experts) ? 3 : nt;
    const int bn = 32 * ntc;
    // dense streaming GEMMs with enough (256-row tile, route chunk) items to fill the GPU:
    // two 32-row slabs per wave (256-row tiles)
    const bool two_slabs = streaming && a.dense && !gated &&
                           (size_t)((m0->rows + 255) / 256) * (size_t)((a.tokens + bn - 1) / bn) >= 256;
    const int tile_rows = two_slabs ? 256 : 128;
    P.row_tiles = (m0->rows + tile_rows - 1) / tile_rows;
    const size_t work = qmm_max_work(m0->rows, a.tokens, a.ngroups, a.dense, bn, tile_rows);
    const size_t blocks = 8 * ((work + 7) / 8);
    if (blocks == 0 || blocks > 0x7fffffffu) {
        set_error(error, capacity, "Invalid qmm grid");
        return false;
    }
    P.max_work = (int)work;
    dim3 grid((unsigned)blocks), block(256);
    if (streaming) {
        // row tiles per block: enough blocks to fill the GPU about twice, up to four tiles
        // streamed back to back per block
        const size_t chunks = work / (size_t)P.row_tiles;
        const size_t per_tile = (size_t)P.row_tiles * chunks;
        int rtb = (int)std::min<size_t>(4, std::max<size_t>(1, per_tile / 512));
        // Gated launches (one block per CU): single row tiles. 5-bit: its work items are
        // nearly equal, and with four tiles a block the last round of blocks ran almost empty
        // (config 4 gate/up 457 -> 380 us). 8-bit: since the MFMAs of empty route tiles are
        // skipped, single tiles measured faster too (config 3 gate/up 166 -> 154 us); the
        // non-gated down projection keeps up to four (single tiles: 89 -> 101 us)
        if (gated) rtb = 1;
        rtb = std::min(rtb, P.row_tiles);
        P.rtb = rtb;
        P.rt_groups = (P.row_tiles + rtb - 1) / rtb;
        const size_t lwork = chunks * (size_t)P.rt_groups;
        grid = dim3((unsigned)(8 * ((lwork + 7) / 8)));
        // 5-bit codes stream from the tile-major copies (every matrix of the launch has one:
        // same bits and K)
        if (m0->bits == 5) {
            const Matrix *ms[4] = {m0, m1, a.sm0, a.sm1};
            for (const Matrix *mm : ms)
                if (mm && !mm->tiled) {
                    set_error(error, capacity, "Missing tile-major 5-bit codes");
                    return false;
                }
            P.p0 = static_cast<const uint32_t *>(m0->tiled);
            if (m1) P.p1 = static_cast<const uint32_t *>(m1->tiled);
            if (a.sm0) P.sp0 = static_cast<const uint32_t *>(a.sm0->tiled);
            if (a.sm1) P.sp1 = static_cast<const uint32_t *>(a.sm1->tiled);
        }
        // Gated launches: the split eight-wave form (gate and up on different waves, so one
        // wave's dequant overlaps the other's MFMAs and waits): 6 % faster on config 4, and,
        // since empty route tiles are skipped, config 3 gate/up 154 -> 143 us
#define DIH_QMM_LDS_CASE(B, GT, N, R2, NC)                                          \
        if (m0->bits == B && gated == GT && nt == N && two_slabs == R2 && ntc == NC) { \
            constexpr bool SP = GT;                                                 \
            DIH_LAUNCH((qmm_lds_kernel<B, GT, N, 4, SP, R2 ? 2 : 1, B == 5, NC>), grid, dim3(SP ? 512 : 256), 0, s, P); \
            return hip_ok(hipGetLastError(), error, capacity, "qmm launch");        \
        }
        DIH_QMM_LDS_CASE(8, true, 2, false, 2) DIH_QMM_LDS_CASE(8, false, 2, false, 2) DIH_QMM_LDS_CASE(8, false, 1, false, 1) DIH_QMM_LDS_CASE(8, false, 4, false, 4)
        DIH_QMM_LDS_CASE(5, true, 2, false, 2) DIH_QMM_LDS_CASE(5, false, 2, false, 2) DIH_QMM_LDS_CASE(5, false, 3, false, 3) DIH_QMM_LDS_CASE(5, false, 4, false, 4)
        DIH_QMM_LDS_CASE(5, true, 4, false, 4) DIH_QMM_LDS_CASE(5, true, 4, false, 3)
        DIH_QMM_LDS_CASE(8, false, 4, true, 4) DIH_QMM_LDS_CASE(5, false, 4, true, 4)
#undef DIH_QMM_LDS_CASE
    }
#define DIH_QMM_CASE(B, GT, N, D)                                                   \
    if (m0->bits == B && gated == GT && nt == N) {                                  \
        DIH_LAUNCH((qmm_kernel<B, GT, N, D>), grid, block, 0, s, P);                \
        return hip_ok(hipGetLastError(), error, capacity, "qmm launch");            \
    }
    DIH_QMM_CASE(8, true, 2, 2) DIH_QMM_CASE(8, false, 4, 2)
    DIH_QMM_CASE(5, true, 2, 2) DIH_QMM_CASE(5, false, 4, 2)
#undef DIH_QMM_CASE
    set_error(error, capacity, "Unsupported qmm configuration");
    return false;
}

}  // namespace dih
