/*
 * fence/wave_clock.h -- per-wave timing of the Q6_K GEMV kernels, exported
 * only by the instrumented library libfence_ops_waveclock.so (the same
 * sources built with FENCE_WAVE_CLOCK=1); libfence_ops.so has neither these
 * symbols nor the instrumentation.  No counterpart in the reference: it
 * exists to show where a launch's waves spend its time (dispatch ramp, row
 * groups, tail).
 *
 * Each wave of a staged Q6_K GEMV launch writes one record of four 64-bit
 * words into a device buffer (up to 65536 waves; the latest launch
 * overwrites):
 *   [0] entry time, [1] exit time -- s_memrealtime, the 100 MHz constant
 *       clock shared by the whole device (10 ns per tick);
 *   [2] HW_ID register (bits 0-31: wave, SIMD, CU, shader array, shader
 *       engine ...) | XCC_ID register << 32;
 *   [3] row groups the wave computed.
 * Record i belongs to wave i = workgroup * waves_per_workgroup + wave.
 */
#ifndef FENCE_WAVE_CLOCK_H
#define FENCE_WAVE_CLOCK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Zero the record buffer (synchronises the device). */
int fence_wave_clock_clear(void);

/* Copy the first min(max_waves, 65536) records (4 words each) to host memory
 * at dst (synchronises the device first). */
int fence_wave_clock_read(uint64_t* dst, int64_t max_waves);

#ifdef __cplusplus
}
#endif

#endif /* FENCE_WAVE_CLOCK_H */
