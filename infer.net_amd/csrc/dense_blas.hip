// Dense projections of long chunks (dih_dense at many tokens): the matrix is dequantized
// once into bf16, then multiplied by one bf16 GEMM with f32 accumulation. This is the
// reference's BF16 dense path (prefill_bf16.mm:7-53, dispatched by gpu_prefill.mm:603-614):
// dequantize-then-matmul with bf16 operands. The fused qmm kernel re-dequantizes every
// weight tile once per 128-token route chunk, 32 times at 4096 tokens, so at long chunks
// its VALU work, not the MFMAs, sets its pace; a dequantized copy makes the product a plain
// library GEMM, which hipBLASLt runs at 1.3-1.9 PFLOP/s on gfx950 for these shapes.
//
// dequant_bf16_kernel: bf16(fp32(q * scale + bias)) rounded to nearest even exactly as the
// qmm kernel rounds its A operands. 8-bit: one thread per eight codes (an 8-byte load and a
// 16-byte store, both contiguous across the wave); 5-bit: one thread per 32-code chunk
// (20 bytes), written as four 16-byte stores.
//
// The GEMM: Y[T][R] = X[T][C] * W16[R][C]^T. In hipBLASLt's column-major terms that is
// D (R x T, ld R) = op(A) * B with A = W16 as a C x R matrix (ld C) transposed and B = X as
// a C x T matrix (ld C): the "TN" form. One hipBLASLt handle per context; the algorithm
// for each (R, C, T, output type) is chosen on first use from the heuristic's first 16
// candidates by timing three back-to-back runs of each after one untimed run (skipped,
// taking the heuristic's first, when the stream is being captured into a graph), and kept.
// (Sixteen candidates instead of four found a faster in_proj kernel: 171 -> 163 us.)
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

#include "dih_device.h"
#include "dih_internal.h"

namespace dih {

namespace {

template <int BITS>
__global__ __launch_bounds__(256) void dequant_bf16_kernel(const uint32_t *packed, const uint16_t *scales,
                                                           const uint16_t *biases, int rows, int columns,
                                                           uint16_t *out) {
    if constexpr (BITS == 8) {
        // flat index of eight codes; rows are whole groups of 64 codes, so a piece never
        // straddles a row and the group index is the piece index / 8
        const size_t n8 = (size_t)rows * (size_t)(columns >> 3);
        const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
        if (i >= n8) return;
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(packed) + i);
        const float sc = bf16_to_f32(scales[i >> 3]), bi = bf16_to_f32(biases[i >> 3]);
        uint32_t p[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t v = k < 2 ? w.x : w.y;
            const int sh = 16 * (k & 1);
            p[k] = pack_bf16x2(fmaf((float)((v >> sh) & 255u), sc, bi), fmaf((float)((v >> (sh + 8)) & 255u), sc, bi));
        }
        reinterpret_cast<uint4 *>(out)[i] = make_uint4(p[0], p[1], p[2], p[3]);
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

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t workspace = 0;
};

struct BlasState {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<int, int, int, int>, Plan> plans;
};

const char *blas_status(hipblasStatus_t s) {
    switch (s) {
        case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
        case HIPBLAS_STATUS_ALLOC_FAILED: return "allocation failed";
        case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
        case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
        case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
        case HIPBLAS_STATUS_INTERNAL_ERROR: return "internal error";
        default: return "error";
    }
}

bool blas_ok(hipblasStatus_t s, char *error, int capacity, const char *what) {
    if (s == HIPBLAS_STATUS_SUCCESS) return true;
    set_error(error, capacity, std::string("hipBLASLt ") + what + ": " + blas_status(s));
    return false;
}

void destroy_plan(Plan &p) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.ld) hipblasLtMatrixLayoutDestroy(p.ld);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    p = Plan{};
}

// Creates the descriptors of Y[T][R] = X[T][C] * W16[R][C]^T and picks its algorithm.
bool make_plan(Context *c, BlasState &b, int R, int C, int T, bool y_bf16, const void *w16, const void *x,
               void *y, hipStream_t s, Plan &p, char *error, int capacity) {
    if (!blas_ok(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), error, capacity, "descriptor"))
        return false;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (!blas_ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)), error,
                 capacity, "descriptor") ||
        !blas_ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)), error,
                 capacity, "descriptor") ||
        !blas_ok(hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, C, R, C), error, capacity, "layout") ||
        !blas_ok(hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, C, T, C), error, capacity, "layout") ||
        !blas_ok(hipblasLtMatrixLayoutCreate(&p.ld, y_bf16 ? HIP_R_16BF : HIP_R_32F, R, T, R), error, capacity,
                 "layout"))
        return false;
    constexpr size_t kMaxWorkspace = (size_t)64 << 20;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (!blas_ok(hipblasLtMatmulPreferenceCreate(&pref), error, capacity, "preference")) return false;
    const uint64_t wmax = kMaxWorkspace;
    hipblasLtMatmulHeuristicResult_t cand[16];
    int n = 0;
    hipblasStatus_t st =
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wmax, sizeof(wmax));
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulAlgoGetHeuristic(b.handle, p.desc, p.la, p.lb, p.ld, p.ld, pref, 16, cand, &n);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (!blas_ok(st, error, capacity, "heuristic")) return false;
    if (n < 1) {
        set_error(error, capacity, "hipBLASLt has no algorithm for this dense projection");
        return false;
    }
    size_t ws_need = 0;
    for (int i = 0; i < n; i++) ws_need = std::max(ws_need, cand[i].workspaceSize);
    void *ws = ws_need ? ctx_scratch(c, S_BLASWS, ws_need, error, capacity) : nullptr;
    if (ws_need && !ws) return false;
    int best = -1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (n > 1 && hipStreamIsCapturing(s, &cap) == hipSuccess && cap == hipStreamCaptureStatusNone) {
        // time each candidate once (after one untimed run) on the caller's stream
        const float alpha = 1.f, beta = 0.f;
        float best_ms = 0.f;
        for (int i = 0; i < n; i++) {
            if (hipblasLtMatmul(b.handle, p.desc, &alpha, w16, p.la, x, p.lb, &beta, y, p.ld, y, p.ld, &cand[i].algo,
                                ws, cand[i].workspaceSize, s) != HIPBLAS_STATUS_SUCCESS)
                continue;
            if (hipEventRecord(c->start, s) != hipSuccess) break;
            bool okr = true;
            for (int rep = 0; rep < 3 && okr; rep++)
                okr = hipblasLtMatmul(b.handle, p.desc, &alpha, w16, p.la, x, p.lb, &beta, y, p.ld, y, p.ld, &cand[i].algo,
                                      ws, cand[i].workspaceSize, s) == HIPBLAS_STATUS_SUCCESS;
            if (!okr) continue;
            float ms = 0.f;
            if (hipEventRecord(c->stop, s) != hipSuccess || hipEventSynchronize(c->stop) != hipSuccess ||
                hipEventElapsedTime(&ms, c->start, c->stop) != hipSuccess)
                break;
            if (best < 0 || ms < best_ms) { best = i; best_ms = ms; }
        }
    }
    if (best < 0) best = 0;
    p.algo = cand[best].algo;
    p.workspace = cand[best].workspaceSize;
    return true;
}

}  // namespace

void blas_release(Context *c) {
    auto *b = static_cast<BlasState *>(c->blas);
    if (!b) return;
    for (auto &kv : b->plans) destroy_plan(kv.second);
    if (b->handle) hipblasLtDestroy(b->handle);
    delete b;
    c->blas = nullptr;
}

bool launch_dense_blas(Context *c, const Matrix *m, int tokens, const uint16_t *x, void *y, bool y_bf16,
                       hipStream_t s, char *error, int capacity) {
    const int R = m->rows, C = m->columns;
    if (C % 64 != 0 || (m->bits != 8 && m->bits != 5)) {
        set_error(error, capacity, "Unsupported dense projection shape");
        return false;
    }
    auto *b = static_cast<BlasState *>(c->blas);
    if (!b) {
        b = new BlasState();
        if (!blas_ok(hipblasLtCreate(&b->handle), error, capacity, "handle")) {
            delete b;
            return false;
        }
        c->blas = b;
    }
    uint16_t *w16 = static_cast<uint16_t *>(ctx_scratch(c, S_W16, (size_t)R * C * 2, error, capacity));
    if (!w16) return false;
    const size_t items = (size_t)R * (m->bits == 8 ? C / 8 : C / 32);
    const dim3 grid((unsigned)((items + 255) / 256));
    prof_stage("dense_dequant");
    if (m->bits == 8)
        DIH_LAUNCH(dequant_bf16_kernel<8>, grid, dim3(256), 0, s, m->packed(), m->scales(), m->biases(), R, C, w16);
    else
        DIH_LAUNCH(dequant_bf16_kernel<5>, grid, dim3(256), 0, s, m->packed(), m->scales(), m->biases(), R, C, w16);
    if (!hip_ok(hipGetLastError(), error, capacity, "dequant launch")) return false;

    const auto key = std::make_tuple(R, C, tokens, y_bf16 ? 1 : 0);
    auto it = b->plans.find(key);
    if (it == b->plans.end()) {
        Plan p;
        if (!make_plan(c, *b, R, C, tokens, y_bf16, w16, x, y, s, p, error, capacity)) {
            destroy_plan(p);
            return false;
        }
        it = b->plans.emplace(key, p).first;
    }
    const Plan &p = it->second;
    void *ws = p.workspace ? ctx_scratch(c, S_BLASWS, p.workspace, error, capacity) : nullptr;
    if (p.workspace && !ws) return false;
    const float alpha = 1.f, beta = 0.f;
    prof_stage("dense_gemm");
    hipEvent_t e0, e1;
    const bool prof = prof_events(&e0, &e1);
    if (prof) (void)hipEventRecord(e0, s);
    const hipblasStatus_t st = hipblasLtMatmul(b->handle, p.desc, &alpha, w16, p.la, x, p.lb, &beta, y, p.ld, y,
                                               p.ld, &p.algo, ws, p.workspace, s);
    if (prof) (void)hipEventRecord(e1, s);
    return blas_ok(st, error, capacity, "matmul");
}

}  // namespace dih
