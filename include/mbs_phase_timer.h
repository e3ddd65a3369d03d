/*
 * mbs_phase_timer.h -- extra C ABI of the phase-timer build of the GEMM
 * library (mbs_amd/lib/libmbs_gemm_phase.so: the same kernels compiled with
 * MBS_PHASE_TIMER=1; `python -m mbs_amd._build --phase-timer`).  A
 * measurement tool, not part of the product library; no counterpart in the
 * reference's C ABI (the reference's MBS_TIMING build, kernel/gemm_a4w4.hip:
 * 56-76 of the reference, reads its buckets through mbs_timing_read).
 *
 * Every persistent-kernel launch after mbs_phase_timer_attach(sums) adds,
 * per wave, the shader-clock cycles (s_memtime) it spent in each phase of
 * its loop into the device array `sums`: mbs_phase_timer_slots() uint64
 * words per workgroup (workgroup g at sums + g * slots; size it for the
 * largest grid, 1024 workgroups, and zero it), in the order:
 *   0 prologue, 1 stage-top vmcnt waits, 2 barriers, 3 stage bodies,
 *   4 MFMA drain + epilogue, 5 next-unit set-up, 6 stages, 7 work units,
 *   8 / 9 s_memtime / s_memrealtime (100 MHz) ticks of the whole kernel,
 *   summed over wave 0 of every workgroup (8 / 9 * 100 MHz = shader clock).
 */
#ifndef MBS_PHASE_TIMER_H_
#define MBS_PHASE_TIMER_H_

#ifdef __cplusplus
extern "C" {
#endif

void mbs_phase_timer_attach(unsigned long long* sums);
int mbs_phase_timer_slots(void);

#ifdef __cplusplus
}
#endif

#endif /* MBS_PHASE_TIMER_H_ */
