/* agk_bench.h -- measurement probes of libagk_bench.so, the benchmark's own
 * library.  Not part of the product ABI (include/): nothing in libagk_rmsnorm.so
 * or the graph layer uses these, and they have no counterpart in the
 * reference.  bench.py loads this library for --stream-probe and --mfma-probe
 * only.  Return values are agk_status codes (include/agk_rmsnorm.h). */
#ifndef AGK_BENCH_H
#define AGK_BENCH_H

#include <stdint.h>

#include "agk_rmsnorm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* HBM streaming probe, the practical ceiling the row kernels are measured
 * against.  grid > 0: a grid-stride kernel of `grid` 256-lane workgroups;
 * grid == 0: one 256-lane workgroup per contiguous 16 KiB chunk of each
 * buffer.  It moves `bytes` (a multiple of 16) per buffer in 16-byte slots:
 * reads == 1 reads a, reads == 2 reads a and b; writes == 1 writes c (a, or
 * a ^ b), writes == 2 writes c and d, writes == 0 writes nothing (c must still
 * point at 16 writable bytes).  nontemporal != 0 sets the non-temporal cache
 * policy on every access, as the row kernels do.                           */
int agk_probe_stream(const void* a, const void* b, void* c, void* d, int64_t bytes, int reads,
                     int writes, int nontemporal, int grid, agk_stream_t stream);

/* MFMA probe: the bf16 GEMM's inner loop without its global loads and
 * barriers, to measure what the matrix cores sustain on this device with a
 * given operand content.  `workgroups` workgroups of 4 waves; each wave keeps
 * the GEMM's 16 v_mfma_f32_32x32x16_bf16 accumulators (a 128 x 128 block) and
 * runs `steps` 64-deep k-steps of 64 MFMAs.  mode 0: each substep's 8 operand
 * fragments are read from a 64 KiB LDS tile filled once from `src` (the
 * GEMM's LDS traffic, no global loads); mode 1: the fragments stay in
 * registers (two sets, loaded once from `src`), only the MFMAs run; modes 2
 * and 3: modes 0 and 1 on v_mfma_f32_16x16x32_bf16 (the same 128 x 128 block
 * per wave as 8 x 8 accumulators, 128 MFMAs per k-step, the same FLOP).  src:
 * 64 KiB of bf16 operand data (random, zeros, ...).  out: 4 floats per
 * workgroup (a checksum of the accumulators, so the work is not removed).
 * clocks (may be NULL): per workgroup, the shader clock counter
 * (s_memtime) and the constant-rate counter (s_memrealtime, 100 MHz) read
 * by wave 0 before and after its loop, 4 uint64 per workgroup.
 * FLOP per launch: workgroups * 4 * steps * 64 * 32768.                    */
int agk_probe_mfma(const void* src, float* out, uint64_t* clocks, int workgroups, int steps,
                   int mode, agk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AGK_BENCH_H */
