// Dense projections of long chunks (dih_dense at many tokens): the matrix is dequantized once
// into a bf16 copy, then Y[T][R] = X[T][C] * W16[R][C]^T runs as a bf16 GEMM with f32
// accumulation on gfx950 MFMA. This is the reference's BF16 dense path (prefill_bf16.mm:7-53,
// dispatched by gpu_prefill.mm:603-614): dequantize-then-matmul with bf16 operands, each
// weight rounded bf16(fp32(q * scale + bias)) to nearest even as prefill_bf16.mm rounds it.
// The fused qmm tile re-dequantizes every weight tile once per 128-token route chunk (32 times
// at 4096 tokens), so at long chunks its VALU work, not its MFMAs, sets the pace; one
// dequantization pass costs R*C*(bits/8 + 2) bytes of HBM traffic and leaves the GEMM
// MFMA-bound.
//
// dequant_bf16_kernel. 8-bit: one thread per sixteen codes (a 16-byte load and two 16-byte
// stores, contiguous across the wave); 5-bit: one thread per 32-code chunk (20 bytes), written
// as four 16-byte stores.
//
// gemm_bf16_kernel<WGM, WGN, WTM, WTN, S>. A block computes a tile of BM = 32*WTM*WGM weight
// rows by BN = 32*WTN*WGN tokens with WGM x WGN waves; wave (wm, wn) owns WTM x WTN 32x32
// accumulators (v_mfma_f32_32x32x16_bf16, weights as the A operand so that a lane's four
// consecutive accumulator rows are four consecutive output columns of Y). K advances 64
// columns a step; each step's weight rows and token rows (128 bytes each) reach LDS by
// direct global->LDS copies (global_load_lds, 16 bytes a lane, eight lanes per row), S
// stages deep, one wait and one barrier per step. A row's 16-byte piece p sits at
// row*128 + 16*(p ^ ((row >> 1) & 7)), so the operand reads (lane: row lane%32, piece
// 2j + lane/32 of slice j) of 16 consecutive lanes fall on distinct banks; the copy lanes
// read their row's pieces in that permuted order, still one 128-byte segment per row.
// Tiles are spread over the eight XCDs (physical block b runs item (b%8)*ceil(items/8) +
// b/8), and consecutive items of one XCD form groups of `group` row tiles x all token tiles,
// so the blocks resident on an XCD at once share a few weight and token panels in its L2.
#include <algorithm>
#include <type_traits>

#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

namespace {

template <int BITS>
__global__ __launch_bounds__(256) void dequant_bf16_kernel(const uint32_t *packed, const uint16_t *scales,
                                                           const uint16_t *biases, int rows, int columns,
                                                           uint16_t *out) {
    if constexpr (BITS == 8) {
        // flat index of sixteen codes; rows are whole groups of 64 codes, so a piece never
        // straddles a row and the group index is the piece index / 4
        const size_t n16 = (size_t)rows * (size_t)(columns >> 4);
        const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
        if (i >= n16) return;
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(packed) + i);
        const float sc = bf16_to_f32(scales[i >> 2]), bi = bf16_to_f32(biases[i >> 2]);
        uint32_t p[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = w[k >> 1];
            const int sh = 16 * (k & 1);
            p[k] = pack_bf16x2(fmaf((float)((v >> sh) & 255u), sc, bi), fmaf((float)((v >> (sh + 8)) & 255u), sc, bi));
        }
        uint4 *dst = reinterpret_cast<uint4 *>(out) + 2 * i;
        dst[0] = make_uint4(p[0], p[1], p[2], p[3]);
        dst[1] = make_uint4(p[4], p[5], p[6], p[7]);
        return;
    }
    const int cpr = columns >> 5;
    const size_t nch = (size_t)rows * cpr;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nch) return;
    const size_t row = i / (size_t)cpr;
    const int ch = (int)(i - row * (size_t)cpr);
    Chunk<BITS> c;
    load_chunk<BITS, true>(c, packed + row * ((size_t)columns * BITS / 32), ch);
    const size_t g = row * (size_t)(columns >> 6) + (size_t)(ch >> 1);
    dih_bf16x8 op[4];
    chunk_to_bf16<BITS>(c, bf16_to_f32(scales[g]), bf16_to_f32(biases[g]), op);
    uint4 *dst = reinterpret_cast<uint4 *>(out + row * (size_t)columns + (size_t)ch * 32);
#pragma unroll
    for (int j = 0; j < 4; j++) dst[j] = __builtin_bit_cast(uint4, op[j]);
}

constexpr int kLdsBytes = 160 * 1024;   // LDS per CU (gfx950)

// Output staging bytes per wave: the largest power of two up to 4 KB within `avail`.
constexpr int staging_bytes(int avail) {
    int b = 4096;
    while (b > avail) b >>= 1;
    return b;
}

// Stores a wave's finished WTM x WTN accumulator tiles (rows = output columns rbase ..
// rbase + 32*WTM, tokens tbase .. tbase + 32*WTN) through its EB-byte LDS buffer, so that each
// store instruction writes whole row segments (16 bytes a lane, CH lanes a token row)
// instead of 8- or 16-byte pieces of 32 rows. Per pass of TP tokens: the lanes holding those
// tokens write their values (chunk c of a token row at (c ^ swizzle(row)) * 16, so that the
// 16 lanes of one write or read touch distinct banks), then every lane reads one 16-byte
// chunk and stores it (element by element where the tile crosses column R or rows are
// not 16-byte aligned).
template <int ESZ, int WTM, int WTN, int EB>
DIH_DEV void staged_store(const dih_f32x16 (&acc)[WTM][WTN], unsigned char *buf, void *y, int R, int T, int rbase,
                          int tbase, int r, int h, int lane) {
    constexpr int ROWB = 32 * WTM * ESZ;                // bytes of one token row of the tile
    constexpr int CH = ROWB / 16;                       // 16-byte chunks per row
    constexpr int TP = EB / ROWB < 32 ? EB / ROWB : 32;  // tokens per pass
    constexpr int SH = ROWB >= 256 ? 0 : ROWB == 128 ? 1 : 2;
    constexpr int RPI = 64 / CH;                        // token rows per store instruction
    static_assert(TP >= 1 && 32 % TP == 0 && TP % RPI == 0, "passes of whole store instructions");
    auto swz = [&](int row) { return (((row >> SH) << (ESZ == 4 ? 1 : 0))) & (CH - 1); };
    char *yb = static_cast<char *>(y);
    // every column of the tile below R, and rows 16-byte aligned: whole-chunk stores
    const bool full = rbase + 32 * WTM <= R && (R * ESZ) % 16 == 0;
#pragma unroll
    for (int p = 0; p < 32 * WTN / TP; p++) {
        const int n = p * TP / 32, t_lo = p * TP % 32;
        if (r >= t_lo && r < t_lo + TP) {
            const int tl = r - t_lo, sw = swz(tl);
#pragma unroll
            for (int i = 0; i < WTM; i++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int col = 32 * i + 8 * q + 4 * h;
                    if constexpr (ESZ == 2) {
                        const int c = col >> 3;   // 16-byte chunk; h picks its half
                        const uint2 pk = {pack_bf16x2(acc[i][n][4 * q], acc[i][n][4 * q + 1]),
                                          pack_bf16x2(acc[i][n][4 * q + 2], acc[i][n][4 * q + 3])};
                        *reinterpret_cast<uint2 *>(buf + tl * ROWB + ((c ^ sw) << 4) + 8 * h) = pk;
                    } else {
                        const int c = col >> 2;
                        *reinterpret_cast<float4 *>(buf + tl * ROWB + ((c ^ sw) << 4)) =
                            make_float4(acc[i][n][4 * q], acc[i][n][4 * q + 1], acc[i][n][4 * q + 2], acc[i][n][4 * q + 3]);
                    }
                }
        }
#pragma unroll
        for (int rr = 0; rr < TP; rr += RPI) {
            const int tr = rr + lane / CH, c = lane % CH;
            const uint4 v = *reinterpret_cast<const uint4 *>(buf + tr * ROWB + ((c ^ swz(tr)) << 4));
            const int tok = tbase + 32 * n + t_lo + tr;
            constexpr int PER = 16 / ESZ;   // elements per chunk
            const int col = rbase + c * PER;
            if (tok < T) {
                char *dst = yb + ((size_t)tok * (size_t)R + (size_t)col) * ESZ;
                if (full) {
                    *reinterpret_cast<uint4 *>(dst) = v;
                } else {
                    // ragged or unaligned rows: element stores below R
                    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < PER; e++)
                        if (col + e < R) {
                            if constexpr (ESZ == 2) reinterpret_cast<uint16_t *>(dst)[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                            else reinterpret_cast<uint32_t *>(dst)[e] = w[e];
                        }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Direct copies global -> LDS of 16 (or 4) bytes a lane: lane i's bytes from base + off land
// at LDS byte lds + 16 i (or 4 i); M0 holds the wave's LDS destination. Issued as inline asm,
// so that the compiler does not track these LDS writes: it would otherwise make every LDS
// read wait for all copies in flight, since it cannot tell the stages apart. The kernels
// order the copies themselves (vmcnt waits on their own copies, then a barrier, before a
// stage is read).
DIH_DEV void copy16_to_lds(const void *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}

struct GemmParams {
    const uint16_t *w;          // [R][C] bf16 weights
    const uint16_t *x;          // [T][C] bf16
    void *y;                    // [T][R] f32 or bf16
    int R, T, C, y_bf16;
    int tiles_m, tiles_n;       // weight-row tiles, token tiles
    int group;                  // row tiles per group of consecutive items
};

template <int WGM, int WGN, int WTM, int WTN, int S, int BK>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_bf16_kernel(GemmParams P) {
    constexpr int NW = WGM * WGN;
    constexpr int BM = 32 * WTM * WGM, BN = 32 * WTN * WGN;
    static_assert(BK == 32 || BK == 64, "32 or 64 K columns a step");
    constexpr int RB = 2 * BK;                   // bytes of one row's step
    constexpr int PR = BK / 8;                   // 16-byte pieces per row
    constexpr int RPC = 1024 / RB;               // rows one wave copy fills
    constexpr int NSL = BK / 16;                 // 16-column MFMA slices per step
    constexpr int BOFF = BM * RB;                // token rows within a stage
    constexpr int ST = (BM + BN) * RB;           // bytes per stage: weight rows, then token rows
    constexpr int CPA = BM / (RPC * NW), CPB = BN / (RPC * NW);   // copies per wave per step
    constexpr int NV = CPA + CPB;
    static_assert(CPA * RPC * NW == BM && CPB * RPC * NW == BN, "copies split evenly over the waves");
    // piece p of row n sits at n * RB + 16 * (p ^ swz(n)): the 16 lanes of an operand read
    // (16 consecutive rows, one piece) then fall on distinct banks of the 256-byte bank row
    auto swz = [](int n) { return BK == 64 ? (n >> 1) & 7 : (n >> 2) & 3; };
    static_assert(S >= 2 && S <= 4, "two to four stages");
    // per-wave output staging in the LDS the stages leave free (up to 4 KB a wave)
    constexpr int EB = staging_bytes((kLdsBytes - S * ST - 64) / NW);
    static_assert(EB >= 512, "room for the output staging");
    __shared__ __align__(16) unsigned char lds[S * ST];
    __shared__ __align__(16) unsigned char epi[NW * EB];
    lds_escape(lds, epi);

    const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const int R = P.R, T = P.T, C = P.C, nk = C / BK;
    // Persistent blocks: XCD x (blocks b with b % 8 == x) owns items [x*per, x*per + per),
    // and its j-th block takes items lo + j, lo + j + nxb, ...; the blocks of an XCD thus run
    // a window of consecutive items at a time.
    const int items = P.tiles_m * P.tiles_n;
    const int nxb = (int)(gridDim.x >> 3), jb = (int)(blockIdx.x >> 3);
    const int per = (items + 7) >> 3;
    const int lo = (int)(blockIdx.x & 7) * per, hi = min(items, lo + per);
    const int my_items = lo + jb < hi ? (hi - lo - jb + nxb - 1) / nxb : 0;
    if (my_items == 0) return;
    // item -> (first weight row, first token): groups of `group` row tiles x all token tiles
    auto tile_of = [&](int idx, int &row0, int &tok0) {
        const int L = lo + jb + idx * nxb;
        const int width = P.group * P.tiles_n;
        const int g = L / width, within = L - g * width;
        const int gm = min(P.group, P.tiles_m - g * P.group);
        row0 = (g * P.group + within % gm) * BM;
        tok0 = (within / gm) * BN;
    };

    // Copy sources: copy q of this wave fills LDS rows RPC*(q*NW + wave) .. +RPC of its matrix;
    // lane: row n = RPC*(q*NW + wave) + lane/PR, slot lane%PR = piece (lane%PR) ^ swz(n).
    // Rows past the matrix read its last row (in bounds; those outputs are not stored).
    // The copies run S - 1 steps ahead of the MFMAs, across item boundaries: (iss_idx,
    // iss_k) is the next step to copy; past the block's last step that step is copied again
    // (never read), which keeps the outstanding copies per step constant.
    const char *wsrc = reinterpret_cast<const char *>(P.w), *xsrc = reinterpret_cast<const char *>(P.x);
    uint32_t aoff[CPA], boff[CPB];
    auto set_sources = [&](int idx) {
        int row0, tok0;
        tile_of(idx, row0, tok0);
#pragma unroll
        for (int q = 0; q < CPA; q++) {
            const int n = RPC * (q * NW + wave) + lane / PR;
            const int row = min(row0 + n, R - 1);
            aoff[q] = (uint32_t)row * (uint32_t)(2 * C) + 16u * (uint32_t)((lane % PR) ^ swz(n));
        }
#pragma unroll
        for (int q = 0; q < CPB; q++) {
            const int n = RPC * (q * NW + wave) + lane / PR;
            const int tok = min(tok0 + n, T - 1);
            boff[q] = (uint32_t)tok * (uint32_t)(2 * C) + 16u * (uint32_t)((lane % PR) ^ swz(n));
        }
    };
    int iss_idx = 0, iss_k = 0;
    set_sources(0);
    auto advance = [&]() {
        if (iss_k + 1 < nk) {
            iss_k++;
        } else if (iss_idx + 1 < my_items) {
            iss_idx++;
            iss_k = 0;
            set_sources(iss_idx);
        }
    };

    // operand reads: lane (r = lane%32, h = lane/32) reads row r of each 32-row tile, piece
    // 2j + h (K columns 16j + 8h .. +8) of slice j
    const int wm = wave / WGN, wn = wave - wm * WGN;
    const int r = lane & 31, h = lane >> 5;
    const uint32_t a_row = (uint32_t)(wm * 32 * WTM + r) * RB;
    const uint32_t b_row = (uint32_t)BOFF + (uint32_t)(wn * 32 * WTN + r) * RB;
    uint32_t pofs[NSL];
#pragma unroll
    for (int j = 0; j < NSL; j++) pofs[j] = 16u * (uint32_t)((2 * j + h) ^ swz(r));

    dih_f32x16 acc[WTM][WTN];
    dih_bf16x8 a[2][WTM], b[2][WTN];
    const uint32_t lds_base = (uint32_t)(uintptr_t)lds;
    // operand reads of slice j of a stage into buffer `buf`
    auto read = [&](int stage, int j, int buf) {
        const unsigned char *base = lds + stage * ST;
#pragma unroll
        for (int i = 0; i < WTM; i++)
            a[buf][i] = *reinterpret_cast<const dih_bf16x8 *>(base + a_row + 32u * RB * i + pofs[j]);
#pragma unroll
        for (int n = 0; n < WTN; n++)
            b[buf][n] = *reinterpret_cast<const dih_bf16x8 *>(base + b_row + 32u * RB * n + pofs[j]);
    };
    // copies of the step (iss_idx, iss_k) into a stage, then the next step to copy
    auto issue = [&](int cstage) {
        const uint32_t cbase = lds_base + (uint32_t)(cstage * ST);
        const uint32_t ko = (uint32_t)iss_k * (uint32_t)RB;
#pragma unroll
        for (int v = 0; v < CPA; v++) copy16_to_lds(wsrc, aoff[v] + ko, cbase + (uint32_t)((v * NW + wave) * 1024));
#pragma unroll
        for (int v = 0; v < CPB; v++)
            copy16_to_lds(xsrc, boff[v] + ko, cbase + (uint32_t)(BOFF + (v * NW + wave) * 1024));
        advance();
    };
    // the MFMAs of one 16-column slice (operands in buffer `buf`)
    auto mfma = [&](int buf) {
#pragma unroll
        for (int i = 0; i < WTM; i++)
#pragma unroll
            for (int n = 0; n < WTN; n++)
                acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[buf][i], b[buf][n], acc[i][n], 0, 0, 0);
    };
    // a region: one MFMA (its wait covers the reads of the region before), the region's
    // operand reads (they then have the remaining MFMAs to land), the other MFMAs
    auto pin = [&]() {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, WTM + WTN, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, WTM * WTN - 1, 0);
    };

    // Step schedule, stage = step % S over the block's items' K steps as one sequence.
    // Regions 0 .. NSL-2 run the MFMAs of slices 0 .. NSL-2 while the operands of the slice
    // after each are read. Then the wait for the next step's copies and the barrier (every
    // wave has read its last operands of this stage, and every wave's copies of the next step
    // are visible), the copies of step + S into this stage, and the last region: the MFMAs
    // of the last slice while the next step's slice-0 operands are read. No operand read
    // waits behind the barrier, and the copies have S - 1 steps to land.
    // prologue: copies of the first S steps, then the first step's slice-0 operands
#pragma unroll
    for (int s = 0; s < S; s++) issue(s);
    wait_vm<(S - 1) * NV>();
    barrier_no_fence();
    read(0, 0, 0);
    int stage = 0;
    for (int idx = 0; idx < my_items; idx++) {
#pragma unroll
        for (int i = 0; i < WTM; i++)
#pragma unroll
            for (int n = 0; n < WTN; n++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[i][n][v] = 0.f;
        for (int k = 0; k < nk; k++) {
            const int next = stage == S - 1 ? 0 : stage + 1;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NSL - 1; j++) {
                read(stage, j + 1, (j + 1) & 1);
                mfma(j & 1);
                pin();
                __builtin_amdgcn_sched_barrier(0);
            }
            // this wave's copies of the next step have landed once at most the copies of
            // the S - 2 steps after it are outstanding
            wait_vm<(S - 2) * NV>();
            barrier_no_fence();
            issue(stage);
            read(next, 0, 0);
            mfma((NSL - 1) & 1);
            pin();
            __builtin_amdgcn_sched_barrier(0);
            stage = next;
        }
        // epilogue: accumulator (i, n) element v is row 32i + 8(v/4) + 4h + v%4 of the
        // wave's rows, token 32n + r of its tokens; the next item's first copies are in flight
        int row0, tok0;
        tile_of(idx, row0, tok0);
        const int rbase = row0 + wm * 32 * WTM, tbase = tok0 + wn * 32 * WTN;
        if (P.y_bf16) staged_store<2, WTM, WTN, EB>(acc, epi + wave * EB, P.y, R, T, rbase, tbase, r, h, lane);
        else staged_store<4, WTM, WTN, EB>(acc, epi + wave * EB, P.y, R, T, rbase, tbase, r, h, lane);
    }
    // no copy may still be writing this block's LDS when the block exits
    wait_vm<0>();
}

// Block shapes, chosen per call by the tiles they make (a shape fills the GPU when its
// tiles reach about one per CU).
template <int WGM, int WGN, int WTM, int WTN, int S, int BK>
bool run_gemm(const GemmParams &p0, int group, hipStream_t s, char *error, int capacity) {
    constexpr int BM = 32 * WTM * WGM, BN = 32 * WTN * WGN;
    GemmParams p = p0;
    p.tiles_m = (p.R + BM - 1) / BM;
    p.tiles_n = (p.T + BN - 1) / BN;
    p.group = std::max(1, std::min(group, p.tiles_m));
    const size_t items = (size_t)p.tiles_m * (size_t)p.tiles_n;
    if (items > 0x7fffffffu) {
        set_error(error, capacity, "Invalid dense GEMM grid");
        return false;
    }
    // one block per CU (256 CUs, 32 per XCD), fewer when the items do not fill them
    const size_t blocks = std::min<size_t>(256, 8 * ((items + 7) / 8));
    DIH_LAUNCH((gemm_bf16_kernel<WGM, WGN, WTM, WTN, S, BK>), dim3((unsigned)blocks), dim3(64 * WGM * WGN), 0, s, p);
    return hip_ok(hipGetLastError(), error, capacity, "dense GEMM launch");
}

size_t tiles_of(int R, int T, int bm, int bn) { return (size_t)((R + bm - 1) / bm) * (size_t)((T + bn - 1) / bn); }

}  // namespace

bool launch_dequant_bf16_rows(const uint32_t *packed, const uint16_t *scales, const uint16_t *biases, int bits,
                              int rows, int columns, uint16_t *out, hipStream_t s, char *error, int capacity) {
    const size_t items = (size_t)rows * (bits == 8 ? columns / 16 : columns / 32);
    const dim3 grid((unsigned)((items + 255) / 256));
    if (bits == 8)
        DIH_LAUNCH(dequant_bf16_kernel<8>, grid, dim3(256), 0, s, packed, scales, biases, rows, columns, out);
    else
        DIH_LAUNCH(dequant_bf16_kernel<5>, grid, dim3(256), 0, s, packed, scales, biases, rows, columns, out);
    return hip_ok(hipGetLastError(), error, capacity, "dequant launch");
}

bool launch_dequant_bf16(const Matrix *m, int expert, uint16_t *out, hipStream_t s, char *error,
                         int capacity) {
    const size_t off = (size_t)expert * m->rows;
    return launch_dequant_bf16_rows(m->packed() + off * m->words_per_row(), m->scales() + off * m->groups_per_row(),
                                    m->biases() + off * m->groups_per_row(), m->bits, m->rows, m->columns, out, s,
                                    error, capacity);
}

bool launch_gemm_bf16(const uint16_t *w16, int R, int C, int tokens, const uint16_t *x, void *y, bool y_bf16,
                      hipStream_t s, char *error, int capacity) {
    if (R < 1 || tokens < 1 || C < 64 || C % 64 != 0 || (size_t)R * (size_t)C * 2 > 0xffffffffu ||
        (size_t)tokens * (size_t)C * 2 > 0xffffffffu) {
        set_error(error, capacity, "Unsupported dense GEMM shape");
        return false;
    }
    GemmParams p{};
    p.w = w16; p.x = x; p.y = y; p.R = R; p.T = tokens; p.C = C; p.y_bf16 = y_bf16 ? 1 : 0;
    // the largest block shape whose tiles still give about one per CU
    constexpr size_t kFill = 240;
    if (tiles_of(R, tokens, 256, 256) >= kFill) return run_gemm<4, 2, 2, 4, 2, 64>(p, 8, s, error, capacity);
    if (tiles_of(R, tokens, 256, 128) >= kFill) return run_gemm<4, 2, 2, 2, 2, 64>(p, 8, s, error, capacity);
    if (tiles_of(R, tokens, 128, 128) >= kFill) return run_gemm<2, 2, 2, 2, 4, 64>(p, 8, s, error, capacity);
    return run_gemm<2, 2, 2, 1, 4, 64>(p, 8, s, error, capacity);
}

bool launch_dense_gemm(Context *c, const Matrix *m, int tokens, const uint16_t *x, void *y, bool y_bf16,
                       hipStream_t s, char *error, int capacity) {
    const int R = m->rows, C = m->columns;
    if (C % 64 != 0 || (m->bits != 8 && m->bits != 5)) {
        set_error(error, capacity, "Unsupported dense projection shape");
        return false;
    }
    uint16_t *w16 = static_cast<uint16_t *>(ctx_scratch(c, S_W16, (size_t)R * C * 2, error, capacity));
    if (!w16) return false;
    prof_stage("dense_dequant");
    if (!launch_dequant_bf16_rows(m->packed(), m->scales(), m->biases(), m->bits, R, C, w16, s, error, capacity))
        return false;
    prof_stage("dense_gemm");
    return launch_gemm_bf16(w16, R, C, tokens, x, y, y_bf16, s, error, capacity);
}

}  // namespace dih
