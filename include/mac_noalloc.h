/*
 * mac_noalloc.h -- C ABI of libmac_noalloc.so: the decode step with its
 * workspaces in a static device array of that library.  Links against
 * libmac_hip.so (mac_attention_amd.h).
 */
#ifndef MAC_NOALLOC_H_
#define MAC_NOALLOC_H_

#include "mac_attention_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* No counterpart in the reference: for callers that cannot allocate device
 * memory or hand over workspaces (code under graph capture, tight serving
 * loops, harnesses that forbid allocation).  Same step and effects on the
 * caller's tensors as mac_persistent_decode_bf16 (out / out_lse, the ring row
 * at past_len % M, phase_cycles), with every workspace in one static device
 * array of libmac_noalloc.so (about 65 MiB per GPU, reserved on each GPU the
 * library is used on until the process ends; processes that only load
 * libmac_hip.so do not pay it): the workspace pointers and their sizes in
 * `args` (match_*, head_*, group_*, complete_task_*, task_counts, partial_*)
 * are ignored, may be NULL, and the decisions are not returned.  Limits:
 * N * Hq <= 4096 query heads, M <= 2048 ring slots; larger steps are
 * rejected with MAC_ERR_INVALID_ARGUMENT.  Calls allocate nothing.  All calls
 * on one GPU share its array: calls that overlap on one GPU (different
 * streams) race. */
MAC_API int mac_persistent_decode_bf16_noalloc(const MacDecodeArgs* args, void* stream);

/* Message of the last failed mac_persistent_decode_bf16_noalloc call on this
 * thread ("" if none), including failures of the decode step it runs. */
MAC_API const char* mac_noalloc_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MAC_NOALLOC_H_ */
