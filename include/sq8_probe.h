/*
 * sq8_probe.h - measurement probe of the gfx950 backend (no counterpart in the reference).
 *
 * A read-only streaming kernel: the lower bound on the time of any kernel that reads `bytes`
 * once, with the same launch, ramp-up and tail costs as the decode GEMV. The benchmark times it
 * at each projection's size to state how close the GEMV is to what the GPU can stream.
 */
#ifndef SQ8_PROBE_H_
#define SQ8_PROBE_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads bytes (a multiple of 16, 16-byte aligned p) with nontemporal 16-byte loads, each lane
 * issuing chunks_per_lane (1, 2, 4 or 8) loads per iteration, workgroups_per_cu 256-thread
 * workgroups per compute unit (1..32) striding over the buffer. Workgroup b adds the wrapping
 * uint32 sum of the 32-bit words it read to sink[b % sink_len] (device counters; a few thousand
 * keep the final atomics from serialising), so the counters sum to the buffer's word sum.
 * Asynchronous on hip_stream. */
int sq8_probe_stream_read(const void* p, size_t bytes, unsigned* sink, int sink_len,
                          int workgroups_per_cu, int chunks_per_lane, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* SQ8_PROBE_H_ */
