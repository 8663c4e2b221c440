/*
 * mac_bench.h -- C ABI of libmac_bench.so, measurement helpers kept out of
 * the decode library: the rate a plain streaming read of HBM reaches on the
 * current GPU, as context for the decode kernels' fractions of the 8 TB/s
 * nameplate, and the decode step with HIP events between its kernels (the
 * decode source compiled into this library once more, with nothing of it
 * exported but this entry).  No reference counterpart.
 */
#ifndef MAC_BENCH_H_
#define MAC_BENCH_H_

#include <stdint.h>

#include "mac_attention_amd.h"

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

/* The decode step of mac_persistent_decode_bf16 (same arguments and
 * effects) with HIP events recorded on `stream` around each of its kernels;
 * synchronises on the last event and stores the elapsed milliseconds of the
 * decision kernel (match_decide, with the range scan when the ring is split),
 * span_attention and merge_write in ms[0..2].  Not graph-capturable.  (The
 * reference stamps clock64() phases into phase_cycles instead,
 * DECODE:4751-4929; the product library does the same with debug_enabled >= 2.) */
MAC_BENCH_API int mac_bench_decode_timed(const MacDecodeArgs* args, void* stream, float* ms);

/* Message of the last failed call on this thread ("" if none). */
MAC_BENCH_API const char* mac_bench_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MAC_BENCH_H_ */
