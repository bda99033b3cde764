// On-box ceilings for the roofline: a streaming HBM read and a dense bf16 MFMA loop.
//
// These two kernels are measurement probes that sit beside the hot path, not part of it.
// They answer "what does this particular MI355X deliver" so that roofline fractions can
// be read against both the published peaks (8 TB/s HBM3E, 2.5 PFLOP/s dense bf16) and the
// measured ones. Both kernels compute a checkable result so that neither the loads nor the
// MFMAs can be removed by the compiler, and so that a test can confirm they did the work.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dih_peaks.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kReadThreads = 256;

// XOR of every 32-bit word in [p, p + n16 * 16 bytes). Each thread keeps four 16-byte
// loads in flight per iteration (grid-stride, fully coalesced dwordx4), the wave folds its
// lanes with xor-shuffles and one lane per block writes the block's word to sink[block].
__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const uint4 *__restrict__ p, size_t n16,
                                                                   uint32_t *__restrict__ sink) {
    const size_t stride = size_t(gridDim.x) * kReadThreads;
    size_t i = size_t(blockIdx.x) * kReadThreads + threadIdx.x;
    uint4 a = make_uint4(0, 0, 0, 0), b = a, c = a, d = a;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 u = p[i], v = p[i + stride], w = p[i + 2 * stride], x = p[i + 3 * stride];
        a.x ^= u.x; a.y ^= u.y; a.z ^= u.z; a.w ^= u.w;
        b.x ^= v.x; b.y ^= v.y; b.z ^= v.z; b.w ^= v.w;
        c.x ^= w.x; c.y ^= w.y; c.z ^= w.z; c.w ^= w.w;
        d.x ^= x.x; d.y ^= x.y; d.z ^= x.z; d.w ^= x.w;
    }
    for (; i < n16; i += stride) {
        const uint4 u = p[i];
        a.x ^= u.x; a.y ^= u.y; a.z ^= u.z; a.w ^= u.w;
    }
    uint32_t r = a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    for (int o = 32; o > 0; o >>= 1) r ^= __shfl_xor(r, o, 64);
    __shared__ uint32_t part[kReadThreads / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (int w = 0; w < kReadThreads / 64; ++w) s ^= part[w];
        sink[blockIdx.x] = s;
    }
}

// One-shot form: block b XORs the 32 KB at p + b * 32 KB (each thread eight 16-byte
// non-temporal loads, all in flight before the first is used), so the grid is
// bytes / 32 KB blocks that each read one contiguous piece and exit.
constexpr int kPieceLoads = 8;
constexpr size_t kPieceBytes = (size_t)kReadThreads * kPieceLoads * 16;

__global__ __launch_bounds__(kReadThreads) void stream_read_pieces_kernel(const uint4 *__restrict__ p, size_t n16,
                                                                          uint32_t *__restrict__ sink) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const size_t base = (size_t)blockIdx.x * (kPieceBytes / 16) + threadIdx.x;
    u32x4 v[kPieceLoads];
#pragma unroll
    for (int u = 0; u < kPieceLoads; u++) {
        const size_t k = base + (size_t)u * kReadThreads;
        v[u] = k < n16 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p + k)) : u32x4{0, 0, 0, 0};
    }
    uint32_t r = 0;
#pragma unroll
    for (int u = 0; u < kPieceLoads; u++) r ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    for (int o = 32; o > 0; o >>= 1) r ^= __shfl_xor(r, o, 64);
    __shared__ uint32_t part[kReadThreads / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (int w = 0; w < kReadThreads / 64; ++w) s ^= part[w];
        sink[blockIdx.x] = s;
    }
}

constexpr int kMfmaThreads = 256;
constexpr int kChains = 4;

// `iters` rounds of kChains independent v_mfma_f32_32x32x16_bf16 per wave, operands taken
// from `ab` (8 bf16 per lane, the same for A and B). Each lane writes the sum of its
// 4 x 16 accumulators: with all operands 1.0 that is 4 * 16 * 16 * iters = 1024 * iters, exact
// in fp32 while 1024 * iters stays below 2^24.
__global__ __launch_bounds__(kMfmaThreads) void mfma_loop_kernel(const short *__restrict__ ab, int iters,
                                                                 float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    bf16x8 a;
    for (int j = 0; j < 8; ++j) a[j] = ab[lane * 8 + j];
    f32x16 acc[kChains];
    for (int c = 0; c < kChains; ++c)
        for (int j = 0; j < 16; ++j) acc[c][j] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, acc[c], 0, 0, 0);
    }
    float s = 0.f;
    for (int c = 0; c < kChains; ++c)
        for (int j = 0; j < 16; ++j) s += acc[c][j];
    out[size_t(blockIdx.x) * kMfmaThreads + threadIdx.x] = s;
}

}  // namespace

extern "C" {

int dihp_stream_read(const void *buffer, size_t bytes, uint32_t *sink, int blocks, hipStream_t stream) {
    if (!buffer || !sink || blocks <= 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(buffer) % 16 != 0)
        return int(hipErrorInvalidValue);
    hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(kReadThreads), 0, stream,
                       static_cast<const uint4 *>(buffer), bytes / 16, sink);
    return int(hipGetLastError());
}

int dihp_stream_read_pieces(const void *buffer, size_t bytes, uint32_t *sink, hipStream_t stream) {
    if (!buffer || !sink || bytes == 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(buffer) % 16 != 0)
        return int(hipErrorInvalidValue);
    const size_t blocks = (bytes + kPieceBytes - 1) / kPieceBytes;
    if (blocks > 0x7fffffffu) return int(hipErrorInvalidValue);
    hipLaunchKernelGGL(stream_read_pieces_kernel, dim3((unsigned)blocks), dim3(kReadThreads), 0, stream,
                       static_cast<const uint4 *>(buffer), bytes / 16, sink);
    return int(hipGetLastError());
}

size_t dihp_stream_read_pieces_blocks(size_t bytes) { return (bytes + kPieceBytes - 1) / kPieceBytes; }

int dihp_mfma_loop(const short *operands, int iters, float *out, int blocks, hipStream_t stream) {
    if (!operands || !out || blocks <= 0 || iters <= 0) return int(hipErrorInvalidValue);
    hipLaunchKernelGGL(mfma_loop_kernel, dim3(blocks), dim3(kMfmaThreads), 0, stream, operands, iters, out);
    return int(hipGetLastError());
}

double dihp_mfma_loop_flops(int iters, int blocks) {
    return double(blocks) * (kMfmaThreads / 64) * kChains * double(iters) * (2.0 * 32 * 32 * 16);
}

int dihp_mfma_threads(void) { return kMfmaThreads; }

}  // extern "C"
