// mac_noalloc.hip -- libmac_noalloc.so: the decode step for callers that
// cannot allocate device memory or hand over workspaces (code under graph
// capture, tight serving loops, harnesses that forbid allocation).  No
// counterpart in the reference.
//
// mac_persistent_decode_bf16_noalloc runs libmac_hip.so's decode step with
// every workspace (decisions, task table, partial (o, lse) results, counters)
// in one file-scope device array of this library instead of caller memory.
// It is a library of its own so that the array (about 65 MiB, reserved on
// every GPU the library's code object is loaded on, until the process ends)
// is paid only by processes that load it.  Its limits size the array: at
// most kMaxHeads decode query heads (N * Hq), rings of at most
// 256 * kMatchTiles slots, and kPartialSlots partial slots per group (the
// task plan enlarges a long group's chunks to fit them).  Every call on a
// device shares that device's array: calls that overlap on one GPU
// (different streams) race.  Nothing in it needs clearing between calls:
// the decode step's first kernel zeroes the task counter and rewrites every
// per-group field a later kernel reads.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>

#include "mac_attention_amd.h"
#include "mac_noalloc.h"

namespace {

constexpr int kMaxHeads = 4096;
constexpr int kPartialSlots = 32;
constexpr int kMatchTiles = 8;
constexpr int kHeadDim = 128;
constexpr int kTaskExtra = 6;  // complete_task_* entries beyond 2 N Hkv

constexpr size_t up256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct Layout {  // byte offsets into the scratch array
  static constexpr size_t H = kMaxHeads;
  static constexpr size_t kMatch = up256(H * kMatchTiles * 4);  // one match array
  static constexpr size_t kHead = up256(H * 4);                 // one head_* / group_* array
  static constexpr size_t kTask = up256((2 * H + kTaskExtra) * 4);  // complete_task_go / _tile
  static constexpr size_t match_dist = 0;
  static constexpr size_t match_pos = match_dist + kMatch;
  static constexpr size_t match_slot = match_pos + kMatch;
  static constexpr size_t head0 = match_slot + kMatch;  // 6 head arrays
  static constexpr size_t group0 = head0 + 6 * kHead;   // 7 group arrays (groups <= heads)
  static constexpr size_t task_go = group0 + 7 * kHead;
  static constexpr size_t task_tile = task_go + kTask;
  static constexpr size_t task_counts = task_tile + kTask;
  static constexpr size_t partial_lse = task_counts + 256;
  static constexpr size_t partial_o = partial_lse + up256(H * kPartialSlots * 4);
  static constexpr size_t bytes = partial_o + up256(H * kPartialSlots * kHeadDim * 4);
};

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace

static __device__ __align__(256) unsigned char scratch[Layout::bytes];

namespace {

std::mutex g_scratch_mu;
std::map<int, unsigned char*> g_scratch;

// Device address of this device's scratch array, looked up once per device
// with that device current.  The array's name is not a device address in
// host code: every kernel argument and copy uses this pointer.
int scratch_base(int dev, unsigned char** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find(dev);
  if (it == g_scratch.end()) {
    unsigned char* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail(MAC_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    if (ptr == nullptr) return fail(MAC_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    it = g_scratch.emplace(dev, ptr).first;
  }
  *out = it->second;
  return MAC_OK;
}

}  // namespace

extern "C" int mac_persistent_decode_bf16_noalloc(const MacDecodeArgs* a, void* stream_ptr) {
  g_err[0] = '\0';
  if (a == nullptr) return fail(MAC_ERR_INVALID_ARGUMENT, "args must not be NULL");
  if (a->struct_size != sizeof(MacDecodeArgs) || a->abi_version != MAC_ABI_VERSION)
    return fail(MAC_ERR_INVALID_ARGUMENT, "MacDecodeArgs size/version mismatch (got %u/%u, library expects %zu/%d)",
                a->struct_size, a->abi_version, sizeof(MacDecodeArgs), MAC_ABI_VERSION);
  const int64_t heads = static_cast<int64_t>(a->N) * a->Hq;
  if (heads > kMaxHeads)
    return fail(MAC_ERR_INVALID_ARGUMENT,
                "no-allocation decode supports at most %d query heads per step (N * Hq = %lld)", kMaxHeads,
                static_cast<long long>(heads));
  if (a->M > 256 * kMatchTiles)
    return fail(MAC_ERR_INVALID_ARGUMENT, "no-allocation decode supports rings of at most %d slots (M = %d)",
                256 * kMatchTiles, a->M);
  if (a->max_context <= 0) return fail(MAC_ERR_INVALID_ARGUMENT, "max_context must be positive");
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MAC_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  unsigned char* base = nullptr;
  int rc = scratch_base(dev, &base);
  if (rc != MAC_OK) return rc;
  using L = Layout;
  MacDecodeArgs w = *a;
  auto i32 = [&](size_t off) { return reinterpret_cast<int32_t*>(base + off); };
  w.match_dist = reinterpret_cast<float*>(base + L::match_dist);
  w.match_pos = i32(L::match_pos);
  w.match_slot = i32(L::match_slot);
  int32_t** heads_ws[6] = {&w.head_hit, &w.head_match_slot, &w.head_match_pos,
                           &w.head_prefix_end, &w.head_rect_start, &w.head_new_end};
  for (int i = 0; i < 6; ++i) *heads_ws[i] = i32(L::head0 + i * L::kHead);
  int32_t** groups_ws[7] = {&w.group_rect_begin, &w.group_rect_end, &w.group_rect_tiles, &w.group_tail_begin,
                            &w.group_tail_end, &w.group_tail_tiles, &w.group_mode};
  for (int i = 0; i < 7; ++i) *groups_ws[i] = i32(L::group0 + i * L::kHead);
  w.complete_task_go = i32(L::task_go);
  w.complete_task_tile = i32(L::task_tile);
  w.task_counts = i32(L::task_counts);
  w.partial_lse = reinterpret_cast<float*>(base + L::partial_lse);
  w.partial_o = base + L::partial_o;
  w.partial_o_is_bf16 = 0;
  w.max_match_tiles = kMatchTiles;
  w.match_tile_slots = 256;
  w.max_tiles_context = kPartialSlots;
  w.tile_tokens = (a->max_context + kPartialSlots - 1) / kPartialSlots;
  w.complete_task_len = 2 * static_cast<int64_t>(a->N) * (a->Hkv > 0 ? a->Hkv : 1) + kTaskExtra;
  w.workspace_rows = a->N;
  rc = mac_persistent_decode_bf16(&w, stream_ptr);
  if (rc != MAC_OK) fail(rc, "%s", mac_last_error());
  return rc;
}

extern "C" const char* mac_noalloc_last_error(void) { return g_err; }
