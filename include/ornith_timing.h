/* Kernel launch timing for measurement.  No counterpart in the reference:
 * used by benchmarks to time one kernel of the path with HIP events on the
 * stream it is launched on, while the path runs unchanged.
 *
 * ornith_mi355x_timing_arm(kernel, capacity): from now on, each launch of the
 *   kernel named `kernel` ("*" = every kernel), up to `capacity` launches, is
 *   made with hipExtLaunchKernelGGL and a start/stop event pair attached to
 *   the kernel's own dispatch on its stream (the interval is the kernel's
 *   execution).  kernel == NULL or capacity <= 0
 *   disarms and frees the events.  Not safe against concurrent arm calls.
 * ornith_mi355x_timing_read(kernel, launches, total_ms): waits for the
 *   recorded launches of `kernel` ("*" = all) and returns their count and the
 *   sum of their event intervals in milliseconds.
 * ornith_mi355x_timing_names(out, capacity): comma-separated distinct names
 *   recorded so far; returns the length of the full list.
 *
 * Kernel names: route1, gateup1, down1 (single token); route, gateup, down
 * (2..32 tokens); router, topk, permute_count, permute_scan,
 * permute_scatter, act, gateup_mfma, quant_middle, down_mfma, reduce
 * (prefill); dense_gemv, head_encode, head_project, argmax, act_middle,
 * transform, dequantize, fill. */
#ifndef ORNITH_TIMING_H
#define ORNITH_TIMING_H
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif
#ifndef ORNITH_EXPORT
#define ORNITH_EXPORT __attribute__((visibility("default")))
#endif

ORNITH_EXPORT hipError_t ornith_mi355x_timing_arm(const char* kernel, int capacity);
ORNITH_EXPORT hipError_t ornith_mi355x_timing_read(const char* kernel, int* launches, double* total_ms);
ORNITH_EXPORT int ornith_mi355x_timing_names(char* out, int capacity);
/* Stage trace of the single-token layer kernel, for measurement.  Only a
 * library built with -DORNITH_STAGE_TRACE (ornith_g256._build.build_stage_trace)
 * records it; every other build returns hipErrorNotSupported.  Copies
 * 64 calls x 256 blocks x 16 stage words (entries >= 262144) to the device
 * buffer out_u64 on `stream`.  Call c of a run fills slot (its sequence
 * number % 64); word = steady-clock ticks (100 MHz) in bits 0..51 | low 12
 * bits of the sequence number << 52, 0 where the block did not reach the
 * stage.  Stages: 0 block start, 1 router row published, 2 all logits seen,
 * 3 experts selected, 4 routed gate-up dots done, 5 routed middle row
 * published, 6/7/8 middle rows of slots 0/7/shared seen by the down waves,
 * 9 down dots of slot 0 done, 10 output columns stored, 11 shared middle
 * row published, 12 speculative expert picks published, 13 shared gate
 * logit seen, 14 gate-up dots of the four gate-up waves done. */
ORNITH_EXPORT hipError_t ornith_mi355x_stage_trace_read(void* out_u64, size_t entries, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
