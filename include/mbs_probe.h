/*
 * mbs_probe.h -- C ABI of libmbs_probe.so, a measurement tool beside the GEMM
 * library (no counterpart in the reference).
 *
 * mbs_probe_stream_read: one launch that reads `bytes` (a multiple of 16,
 * below 2^31, from a 16-byte aligned device buffer) with 16-byte
 * non-temporal loads, `grid` workgroups of 256 threads, 8 loads in flight per
 * thread; writes one word per wave into `sink` (grid * 4 uint32).  Its time
 * is the floor a memory-bound (decode) GEMM reading the same bytes is held
 * against.  Returns 0, 1 (bad argument) or 3 (launch failed).
 */
#ifndef MBS_PROBE_H_
#define MBS_PROBE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int mbs_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MBS_PROBE_H_ */
