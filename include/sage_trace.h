/*
 * sage_trace.h — phase trace of the attention kernel (measurement build only).
 *
 * No counterpart in the reference (TriBench has no profiler hook).  Only
 * libsage_attn_trace.so, built by `python -m tribench_amd.build --trace`
 * from the same sources with SAGE_TRACE=1, exports this entry point; the
 * product library libsage_attn.so does not.  It is for the phase-split
 * measurement of tribench_amd/trace_phases.py.
 *
 * After sage_trace_attach(buf, words) every attention launch of the library
 * (sage_attn_fwd, sage_attn_fwd_q, sage_flash_fwd) writes 16 words per wave
 * into buf, at ((blockIdx.x * 8 + wave) * 16): s_memtime at the kernel's
 * entry, the end of its prologue, after iteration 0, after the mask-free
 * loops, after the generic iterations and after the epilogue [0..5]; the
 * cycles spent at the per-iteration barrier over all iterations [6] and in
 * the mask-free loops [7]; the barrier counts (all | mask-free << 32) [8];
 * s_memrealtime (100 MHz) at entry and exit [9, 10]; HW_ID | XCC_ID << 32
 * [11]; the work-group's remapped index [12]; s_memtime after the
 * prologue's Q quantization and after its tile wait [13, 14] (0 for the
 * kernels that take Q8 from the pre-pass or fp16/bf16 Q); [15] is 0.  A launch
 * whose grid needs more than `words` fails with "invalid argument".
 * buf = NULL detaches.  Returns 0 on success.
 */
#ifndef SAGE_TRACE_H
#define SAGE_TRACE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int sage_trace_attach(unsigned long long* buf, int64_t words);

#ifdef __cplusplus
}
#endif

#endif /* SAGE_TRACE_H */
