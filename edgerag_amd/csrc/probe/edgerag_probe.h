/*
 * Measurement probes of libedgerag_probe.so, a bench-only library (not part of the decoder
 * step): HBM ceilings of the access patterns the kernels use, for the rooflines bench.py
 * reports. No counterpart in the reference. Both launch on `stream`, allocate nothing, and return 0 or EDGERAG_EINVAL.
 */
#ifndef EDGERAG_PROBE_H
#define EDGERAG_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Streaming read of `bytes` (a multiple of 16) from the 16-byte-aligned device buffer `src`:
 * `workgroups` workgroups of 256 threads, each reading one contiguous slice with 16-byte loads,
 * `unroll` (1, 2 or 4) loads in flight per thread. `sink` is a 4-byte device word that is never
 * written by real data. */
int edgerag_probe_read(const void* src, int64_t bytes, int32_t workgroups, int32_t unroll,
                       void* sink, void* stream);

/* Random gather: `waves` wavefronts, wave w reading the `per_wave` chunks
 * chunk_ids[w * per_wave ...] of `chunk_bytes` (1024, 2048 or 4096) at base + id * chunk_bytes,
 * with wave-wide 1 KiB loads, two chunks in flight; non-temporal loads when `nontemporal` != 0
 * (the decode rows' loads). */
int edgerag_probe_gather(const void* base, const int32_t* chunk_ids, int32_t waves,
                         int32_t per_wave, int32_t chunk_bytes, int32_t nontemporal, void* sink,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif  /* EDGERAG_PROBE_H */
