/* nq_bench.h — C ABI of libnq_bench.so, the benchmark's measurement helpers.
 * Not part of the quantized path and not in libnq_hip.so; bench.py loads it
 * for the read-floor context beside the decode GEMVs. No reference
 * counterpart. Return codes are nq_status values (0 OK, 2 misaligned, 3 launch
 * failed, 4 bad argument). */
#ifndef NQ_BENCH_H
#define NQ_BENCH_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One streaming read of `bytes` (16-byte aligned, a multiple of 16) with
 * 16-byte non-temporal loads: workgroups of `threads` lanes (256, 512 or 1024),
 * each lane `loads_per_lane` loads in flight (1, 2, 4 or 8; 1024 lanes: up to
 * 4); then the first out_bytes / 16 lanes of the grid store 16 bytes each to
 * `out` (out_bytes may be 0: nothing stored). sink: >= 64 ints, written only
 * in a case the data never produces. */
int nq_probe_read_cfg(const void* p, size_t bytes, int threads, int loads_per_lane, void* out,
                      size_t out_bytes, int* sink, void* stream);
/* nq_probe_read_cfg(p, bytes, 256, 4, NULL, 0, sink, stream). */
int nq_probe_read(const void* p, size_t bytes, int* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NQ_BENCH_H */
