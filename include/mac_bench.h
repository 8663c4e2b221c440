/*
 * mac_bench.h -- C ABI of libmac_bench.so, a measurement helper kept out of
 * the decode library: the rate a plain streaming read of HBM reaches on the
 * current GPU, as context for the decode kernels' fractions of the 8 TB/s
 * nameplate.  No reference counterpart.
 */
#ifndef MAC_BENCH_H_
#define MAC_BENCH_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define MAC_BENCH_API __attribute__((visibility("default")))
#else
#define MAC_BENCH_API
#endif

/* Reads the first floor(bytes / 16) 16-byte words of `src` (device memory,
 * 16-byte aligned) once with the non-temporal policy the decode kernels
 * stream K/V with, on a grid of min(sink_len, 8 x CUs) workgroups of 256
 * threads, and stores one XOR word per workgroup into sink[0 .. grid).
 * Returns 0, or 1 for invalid arguments / 2 for a HIP error, with a message
 * in mac_bench_last_error(). */
MAC_BENCH_API int mac_bench_stream_read(const void* src, int64_t bytes, uint32_t* sink, int32_t sink_len,
                                        void* stream);

/* Message of the last failed call on this thread ("" if none). */
MAC_BENCH_API const char* mac_bench_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MAC_BENCH_H_ */
