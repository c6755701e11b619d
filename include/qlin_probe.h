/*
 * qlin_probe.h -- a measurement aid with no counterpart in the reference: a plain streaming read of a
 * device buffer, the floor that a bandwidth-bound launch of the same bytes can reach on this GPU.
 * bench.py's decode-stream-floor workload replays it at the decode step's launch sizes.  Conventions
 * as in qlin.h: a caller-owned device buffer, asynchronous on qlin_set_stream's stream, nothing
 * allocated, a qlin_status returned.
 *
 *   qlin_probe_stream_read  reads bytes (a multiple of 16, buf 16-byte aligned) with `workgroups`
 *                           workgroups of 256 threads, each thread loading 16-byte words grid-stride;
 *                           writes *sink only for one improbable checksum value, so the loads cannot
 *                           be dropped.  bytes = 0 launches the same kernel with nothing to read.
 */
#ifndef QLIN_PROBE_H
#define QLIN_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int qlin_probe_stream_read(const void *buf, size_t bytes, int workgroups, float *sink);

#ifdef __cplusplus
}
#endif

#endif /* QLIN_PROBE_H */
