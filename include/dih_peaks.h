/* libdih_peaks: on-box ceilings for the roofline (MI355X, gfx950).
 *
 * Measurement probes only, with no counterpart in the reference: the reference publishes no
 * hardware bandwidth or MFMA figure for its path. bench.py times these kernels with HIP events
 * on the stream it passes and reports the measured HBM read and bf16 MFMA ceilings beside the
 * published peaks. The hot-path library (deepinfer_hip.h) does not depend on them.
 *
 * All calls are asynchronous on `stream` and return a hipError_t value (0 = launched).
 */
#ifndef DIH_PEAKS_H
#define DIH_PEAKS_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Streaming read of `bytes` (a multiple of 16, 16-byte aligned) at `buffer` with `blocks`
 * blocks of 256 threads. sink[b] receives the XOR of the 32-bit words block b read, so the
 * XOR over sink[0..blocks) equals the XOR of every word of the buffer. */
int dihp_stream_read(const void *buffer, size_t bytes, uint32_t *sink, int blocks, hipStream_t stream);

/* The same read as one-shot blocks: block b XORs the 32 KB piece at buffer + b * 32 KB
 * (non-temporal loads, eight 16-byte loads a thread in flight at once) into sink[b]; the
 * grid is dihp_stream_read_pieces_blocks(bytes) blocks. */
int dihp_stream_read_pieces(const void *buffer, size_t bytes, uint32_t *sink, hipStream_t stream);
size_t dihp_stream_read_pieces_blocks(size_t bytes);

/* `blocks` blocks of dihp_mfma_threads() threads; every wave issues `iters` rounds of four
 * independent v_mfma_f32_32x32x16_bf16 with A = B = operands[lane*8 .. lane*8+8) (bf16 bits,
 * 64 lanes x 8). out[block*threads + t] receives the sum of lane t's accumulators; with every
 * operand 1.0 that is 1024 * iters. */
int dihp_mfma_loop(const short *operands, int iters, float *out, int blocks, hipStream_t stream);

/* FLOPs one dihp_mfma_loop launch performs (2 * 32 * 32 * 16 per MFMA). */
double dihp_mfma_loop_flops(int iters, int blocks);

/* Threads per block of dihp_mfma_loop. */
int dihp_mfma_threads(void);

#ifdef __cplusplus
}
#endif

#endif
