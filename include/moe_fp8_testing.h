/*
 * Test and measurement instrumentation exported by the same library as
 * include/moe_fp8.h (lib15642_moe_fp8.so).  None of these functions has a
 * counterpart in the reference, and none is part of the forward path: they
 * synthesise inputs for tests and benchmarks, probe the FP8 MFMA
 * instruction's accumulation accuracy, and measure the sustained FP8 MFMA
 * rate.  Status codes and moe_last_error() are those of moe_fp8.h.
 */
#ifndef MOE_FP8_TESTING_H
#define MOE_FP8_TESTING_H

#include <stddef.h>
#include <stdint.h>

#include "moe_fp8.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Synthetic e4m3 data, ~N(0,1) (Irwin-Hall of four 16-bit hash fields),
 * bit-identical to the host generator for the same (seed, stream_id).
 * Test/benchmark input synthesis; no counterpart in the reference.
 */
int moe_fill_normal_e4m3(void* out, size_t n, uint64_t seed, uint64_t stream_id, void* stream);

/*
 * Host (CPU) twin of moe_fill_normal_e4m3 writing elements
 * [first_index, first_index + n) of the same sequence into host memory, on
 * `threads` CPU threads (<= 0: all).  Needs no GPU.
 */
int moe_host_fill_normal_e4m3(void* out, size_t n, uint64_t seed, uint64_t stream_id, uint64_t first_index,
                              int threads);

/*
 * n independent 16x16 products D[t] = A[t] (16x128 e4m3, row-major) x B[t]
 * (128x16 e4m3, given as 16 columns of 128 contiguous K bytes) through the
 * FP8 MFMA instruction the GEMMs use; D fp32 [n, 16, 16] row-major.  Test
 * instrumentation for the instruction's accumulation accuracy; no
 * counterpart in the reference.
 */
int moe_mfma_tiles(const void* a, const void* b, float* d, int n, void* stream);

/*
 * Measurement instrumentation, no counterpart in the reference: the FP8
 * MFMA rate the chip sustains with nothing but MFMAs in flight.  `grid`
 * workgroups of 512 threads each run `iters` rounds of 4 independent
 * 32x32x64 FP8 MFMAs per wave on register operands (2 waves per SIMD, as
 * in the prefill GEMMs); 2 * 32 * 32 * 64 * 4 * 8 * iters FLOPs per
 * workgroup.  out: [grid * 512] fp32 (the accumulator sums, finite);
 * clocks: [grid][2] uint64 per workgroup, elapsed ticks of the constant
 * 100 MHz counter and of the shader clock (their ratio x 100 MHz is the
 * mean shader clock while it ran).  iters in [1, 2^20], grid in [1, 65536].
 */
int moe_mfma_ceiling(float* out, uint64_t* clocks, int iters, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_FP8_TESTING_H */
