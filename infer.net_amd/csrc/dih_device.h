// Device helpers shared by the gfx950 kernels: bf16 conversion, MLX-affine code
// extraction for one lane's 32-code chunk, wave reductions.
//
// Lane chunk: the kernels give every lane 32 consecutive codes of one row, i.e. half of
// one 64-column affine group (one scale, one bias). For 8-bit that is 32 bytes (8 dwords,
// 32-byte aligned); for 5-bit it is 20 bytes (5 dwords, 4-byte aligned) because two
// groups occupy exactly 80 bytes. Bit c*bits of the row holds code c LSB-first, and a
// code may straddle two words (quantized.mm:62-82 restated as an unrolled extraction
// whose word index and shift are compile-time constants).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DIH_DEV __device__ __forceinline__


typedef __attribute__((__vector_size__(8 * sizeof(short)))) short dih_bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float dih_f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float dih_f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float dih_f32x2;

DIH_DEV float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even f32 -> bf16, two values per v_cvt_pk_bf16_f32 (gfx950), through
// the compiler's vector conversion rather than inline asm: an MFMA that reads a VGPR a VALU
// instruction has just written needs two wait states, which the compiler inserts only for
// instructions it can see. (With the conversion in inline asm, some builds placed an MFMA
// one SALU instruction after it, and that MFMA read the operand's previous contents.)
typedef __bf16 dih_bf16x2 __attribute__((ext_vector_type(2)));
typedef float dih_f32v2 __attribute__((ext_vector_type(2)));
DIH_DEV uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((dih_f32v2){lo, hi}, dih_bf16x2));
}
DIH_DEV uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Residual storage: f32 (the reference's) or bf16 bit patterns.
DIH_DEV float residual_load(const void *r, int f32, size_t i) {
    return f32 ? static_cast<const float *>(r)[i] : bf16_to_f32(static_cast<const uint16_t *>(r)[i]);
}
DIH_DEV float residual_store(void *r, int f32, size_t i, float v) {  // returns the stored value
    if (f32) {
        static_cast<float *>(r)[i] = v;
        return v;
    }
    const uint16_t b = f32_to_bf16(v);
    static_cast<uint16_t *>(r)[i] = b;
    return bf16_to_f32(b);
}

template <int BITS>
struct Chunk {
    uint32_t w[BITS];  // 32 codes * BITS bits = BITS dwords
};

// Loads the 32-code chunk `chunk` (0-based, 32 columns each) of a row starting at `row`,
// with the non-temporal hint (NT: the decode step's kernels, measured 0.5 % faster with
// it) or plain loads (the long GEMV streams, measured 4-6 % faster without it).
template <int BITS, bool NT = true>
DIH_DEV void load_chunk(Chunk<BITS> &c, const uint32_t *row, int chunk) {
    const uint32_t *p = row + chunk * BITS;
    if constexpr (BITS == 8) {
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 *q = reinterpret_cast<const u32x4 *>(p);
        u32x4 a, b;
        if constexpr (NT) {
            a = __builtin_nontemporal_load(q);
            b = __builtin_nontemporal_load(q + 1);
        } else {
            a = q[0];
            b = q[1];
        }
        c.w[0] = a.x; c.w[1] = a.y; c.w[2] = a.z; c.w[3] = a.w;
        c.w[4] = b.x; c.w[5] = b.y; c.w[6] = b.z; c.w[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < BITS; i++) c.w[i] = NT ? __builtin_nontemporal_load(p + i) : p[i];
    }
}

// Code i (0..31) of a chunk.
template <int BITS>
DIH_DEV uint32_t chunk_code(const Chunk<BITS> &c, int i) {
    const int bit = i * BITS, w = bit >> 5, s = bit & 31;
    uint32_t v;
    if (s + BITS <= 32)
        v = c.w[w] >> s;
    else
        v = __builtin_amdgcn_alignbit(c.w[w + 1], c.w[w], s);
    return v & ((1u << BITS) - 1u);
}

// sum_i code_i * x_i over the chunk, four independent partial sums.
template <int BITS>
DIH_DEV float chunk_dot(const Chunk<BITS> &c, const float *x) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        a0 = fmaf((float)chunk_code<BITS>(c, i + 0), x[i + 0], a0);
        a1 = fmaf((float)chunk_code<BITS>(c, i + 1), x[i + 1], a1);
        a2 = fmaf((float)chunk_code<BITS>(c, i + 2), x[i + 2], a2);
        a3 = fmaf((float)chunk_code<BITS>(c, i + 3), x[i + 3], a3);
    }
    return (a0 + a1) + (a2 + a3);
}

// 8-bit codes against f16 activations, two codes per instruction: v_perm_b32 turns bytes
// q0..q3 of a code word into the f16 pairs (1024+q0, 1024+q1) and (1024+q2, 1024+q3)
// (0x64 is the high byte of f16 1024.0, whose unit in the last place is 1, so 1024+q is
// exact), and v_dot2_f32_f16 accumulates pair . (x_i, x_i+1) in f32. Returns
// sum_i (1024 + q_i) * x_i; the caller subtracts 1024 * sum_i x_i. xh holds the chunk's 32
// activations as 16 f16 pairs.
typedef _Float16 dih_half2 __attribute__((ext_vector_type(2)));
DIH_DEV float chunk_dot_h8(const Chunk<8> &c, const uint32_t (&xh)[16]) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, c.w[w], 0x04010400u);
        const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, c.w[w], 0x04030402u);
        a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(dih_half2, lo), __builtin_bit_cast(dih_half2, xh[2 * w]), a0, false);
        a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(dih_half2, hi), __builtin_bit_cast(dih_half2, xh[2 * w + 1]), a1, false);
    }
    return a0 + a1;
}

// Dequantize a chunk to bf16 MFMA operands: operand j holds codes 8j..8j+7 as
// bf16(code*scale + bias) with the fp32 value rounded to nearest even (the reference's
// bfloat(float(q)*scale+bias), prefill_expert_packed.mm:34).
template <int BITS>
DIH_DEV void chunk_to_bf16(const Chunk<BITS> &c, float scale, float bias, dih_bf16x8 (&op)[4]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t p[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float lo = fmaf((float)chunk_code<BITS>(c, 8 * j + 2 * k), scale, bias);
            float hi = fmaf((float)chunk_code<BITS>(c, 8 * j + 2 * k + 1), scale, bias);
            p[k] = pack_bf16x2(lo, hi);
        }
        op[j] = __builtin_bit_cast(dih_bf16x8, (uint4){p[0], p[1], p[2], p[3]});
    }
}

// ---- cross-lane all-reduce without LDS (gfx950) ----
// Within 16-lane rows: DPP quad_perm [1,0,3,2] and [2,3,0,1] (xor 1, xor 2),
// row_half_mirror (lane i <-> 7-i in each 8-lane half: joins quads 0 and 1) and row_mirror
// (lane i <-> 15-i: joins the two 8-lane halves). Across rows: v_permlane16_swap pairs rows
// (0,1),(2,3) and v_permlane32_swap pairs the wave halves; with both operands equal, the sum
// (or max/min) of the two returned registers is the pair's combination in every lane.
#define DIH_DPP_XOR1 0xB1
#define DIH_DPP_XOR2 0x4E
#define DIH_DPP_HALF_MIRROR 0x141
#define DIH_DPP_MIRROR 0x140

template <int CTRL>
DIH_DEV uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
DIH_DEV float dppf(float v) {
    return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(uint32_t, v)));
}

struct OpAdd { DIH_DEV float operator()(float a, float b) const { return a + b; } };
struct OpMax { DIH_DEV float operator()(float a, float b) const { return fmaxf(a, b); } };

// All-reduce of a float over aligned groups of `width` lanes (power of two <= 64); every
// lane of a group receives the group's result.
template <typename Op>
DIH_DEV float group_reduce(float v, int width, Op op) {
    if (width >= 2) v = op(v, dppf<DIH_DPP_XOR1>(v));
    if (width >= 4) v = op(v, dppf<DIH_DPP_XOR2>(v));
    if (width >= 8) v = op(v, dppf<DIH_DPP_HALF_MIRROR>(v));
    if (width >= 16) v = op(v, dppf<DIH_DPP_MIRROR>(v));
    if (width >= 32) {
        uint32_t u = __builtin_bit_cast(uint32_t, v);
        auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        v = op(__builtin_bit_cast(float, (uint32_t)p[0]), __builtin_bit_cast(float, (uint32_t)p[1]));
    }
    if (width >= 64) {
        uint32_t u = __builtin_bit_cast(uint32_t, v);
        auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        v = op(__builtin_bit_cast(float, (uint32_t)p[0]), __builtin_bit_cast(float, (uint32_t)p[1]));
    }
    return v;
}
DIH_DEV float group_sum(float v, int width) { return group_reduce(v, width, OpAdd()); }
DIH_DEV float wave_sum(float v) { return group_reduce(v, 64, OpAdd()); }
DIH_DEV float wave_max(float v) { return group_reduce(v, 64, OpMax()); }

DIH_DEV uint32_t umin_(uint32_t a, uint32_t b) { return a < b ? a : b; }
DIH_DEV uint32_t wave_min_u32(uint32_t v) {
    v = umin_(v, dpp<DIH_DPP_XOR1>(v));
    v = umin_(v, dpp<DIH_DPP_XOR2>(v));
    v = umin_(v, dpp<DIH_DPP_HALF_MIRROR>(v));
    v = umin_(v, dpp<DIH_DPP_MIRROR>(v));
    auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = umin_((uint32_t)p[0], (uint32_t)p[1]);
    auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return umin_((uint32_t)q[0], (uint32_t)q[1]);
}

// Top-8 of up to 256 logits by one wave (graph_top8 gpu_graph.mm:134-146 semantics:
// repeated wave max, ties to the lowest id; softmax over the chosen eight with the first
// (largest) subtracted, summed in slot order). Every lane receives ids/probs. `bad` is
// set when a logit is not finite: the ids are then all 0 and the probabilities NaN, which
// the merge kernels take as "leave this token's residual unchanged".
DIH_DEV void wave_top8(const float *logits, int experts, uint32_t (&ids)[8], float (&probs)[8],
                       bool &bad) {
    const int lane = threadIdx.x & 63;
    float cand[4];
    bool nf = false;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        float v = e < experts ? logits[e] : -INFINITY;
        if (e < experts && !isfinite(v)) nf = true;
        cand[j] = v;
    }
    bad = __any(nf);
    float chosen[8];
#pragma unroll
    for (int n = 0; n < 8; n++) {
        float best = cand[0];
        uint32_t id = (uint32_t)lane;
#pragma unroll
        for (int j = 1; j < 4; j++)
            if (cand[j] > best) { best = cand[j]; id = (uint32_t)(lane + 64 * j); }
        const float m = wave_max(best);
        const uint32_t sel = wave_min_u32(best == m ? id : 0xffffffffu);
        chosen[n] = m;
        ids[n] = bad ? 0u : sel;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if ((uint32_t)(lane + 64 * j) == sel) cand[j] = -INFINITY;
    }
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) { probs[i] = __expf(chosen[i] - chosen[0]); total += probs[i]; }
#pragma unroll
    for (int i = 0; i < 8; i++) probs[i] = bad ? __builtin_nanf("") : probs[i] / total;
}

DIH_DEV float sigmoidf_(float v) { return 1.0f / (1.0f + __expf(-v)); }
DIH_DEV float siluf_(float v) { return v * sigmoidf_(v); }

// Loads 32 activations of one chunk as f32 (from f32 or bf16 storage).
DIH_DEV void load_x32(float *x, const void *base, int x_bf16, int offset) {
    if (x_bf16) {
        const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(base) + offset);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint4 v = p[q];
            uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                x[8 * q + 2 * k] = __uint_as_float(u[k] << 16);
                x[8 * q + 2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
            }
        }
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(base) + offset);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            float4 v = p[q];
            x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
        }
    }
}

// ---- direct global->LDS copies and the waits around them

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;

template <int SIZE>
DIH_DEV void to_lds(const void *src, void *lds_wave_base) {
    if constexpr (SIZE == 16)
        __builtin_amdgcn_global_load_lds((gbl_void_t *)src, (lds_void_t *)lds_wave_base, 16, 0, 0);
    else
        __builtin_amdgcn_global_load_lds((gbl_void_t *)src, (lds_void_t *)lds_wave_base, 4, 0, 0);
}

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding)
template <int N>
DIH_DEV void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}

// s_waitcnt lgkmcnt(0) leaving the other counters alone
DIH_DEV void wait_lgkm0() { __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14)); }

// Workgroup barrier without a memory fence: __syncthreads() would also wait for every
// outstanding copy (the fence counts LDS copies as pending stores). Callers first wait
// for their own copies of the step with wait_vm. The barrier itself first waits for this
// wave's LDS reads (lgkmcnt 0): a read still queued at the barrier would race with the
// copies other waves issue right after it into the buffer being read (write after read),
// and a copy that hits L2 can land before a read queued behind other waves' LDS traffic.
// The "memory" clobber keeps the compiler from moving LDS accesses across the barrier,
// for LDS arrays that have escaped (see lds_escape).
DIH_DEV void barrier_no_fence() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Makes LDS arrays escape, so that alias analysis treats them as memory that an asm with a
// "memory" clobber (barrier_no_fence) may touch; without it a __shared__ array that never
// escapes can have its accesses reordered across such an asm.
template <typename T>
DIH_DEV void lds_escape_one(T *p) { asm volatile("" ::"r"(p) : "memory"); }
template <typename... P>
DIH_DEV void lds_escape(P... p) { (lds_escape_one(p), ...); }

// Logical work item of physical block b when `items` items run on a grid sized for an
// upper bound of them: L = (b % 8) * per + b / 8 with per = ceil(items / 8), so that
// consecutive items share an XCD (and its L2) and the actual items, not the bound, are
// spread over all eight XCDs. -1 for a block with no item.
DIH_DEV int xcd_item(int b, int items) {
    const int per = (items + 7) >> 3;
    const int L = (b & 7) * per + (b >> 3);
    return (b >> 3) < per && L < items ? L : -1;
}

