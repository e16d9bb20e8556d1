/*
 * nncpu_calib.h — calibration kernels of libnncpu_calib.so: the measured
 * denominators of the benchmark's rooflines on the box it runs on. Not part
 * of the matmul path and no counterpart in the reference, whose own
 * benchmark states host DRAM bandwidth with a single-thread load-only stream
 * (crates/nncpu/src/kernels/tests.rs:1306-1321); these are that calibration
 * for HBM and for the matrix unit.
 *
 * Every function is asynchronous on `stream` (a hipStream_t, NULL = the null
 * stream) and returns 0, 1 for a bad argument, 2 for a launch failure.
 */
#ifndef NNCPU_CALIB_H
#define NNCPU_CALIB_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Read `bytes` (a multiple of 16) of device memory at p once, 16-byte
 * non-temporal loads, `unroll` (4 or 16) per thread issued before any is
 * used. `out` is a device word the kernel never writes in practice. */
int nnc_read_stream(const void* p, size_t bytes, int unroll, void* out, void* stream);

/* Dense matrix-unit loop: `blocks` workgroups of 4 waves, each wave running
 * four independent accumulator chains of `iters` MFMAs, of
 * v_mfma_i32_32x32x32_i8 (NNC_MFMA_I8) or v_mfma_f32_32x32x16_bf16
 * (NNC_MFMA_BF16). `out` is device memory of 256 words the kernel never
 * writes in practice. nnc_mfma_ops gives the operations (2 per
 * multiply-add) one launch performs. */
enum { NNC_MFMA_I8 = 1, NNC_MFMA_BF16 = 2 };
int nnc_mfma_loop(int kind, int iters, int blocks, void* out, void* stream);
long long nnc_mfma_ops(int kind, int iters, int blocks);

/* The shader clock: `blocks` one-wave workgroups each time a dependent
 * chain of `iters` FMAs with the core-clock counter and the constant 100 MHz
 * counter; out (device, 2 * blocks u64) receives per workgroup {core cycles,
 * 100 MHz ticks}. The clock in MHz is 100 * cycles / ticks. */
int nnc_clock_probe(int blocks, int iters, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NNCPU_CALIB_H */
