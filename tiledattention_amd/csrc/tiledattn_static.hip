// ta_sdpa_fwd_split_static: the split-key-range forward with its workspace in a file-scope
// device array instead of caller memory, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The workspace of the split path (fp32 partial outputs and log-sum-exps, see
// ta_split_workspace_size) is the library's only device scratch.  Here it is `scratch`, a
// static __device__ array of kStaticScratchBytes: every GPU the library runs on holds its
// own copy at its own address until the process ends.  In host code the array's name is
// only a stand-in for the symbol, never a device address: its address on a device comes
// from hipGetSymbolAddress, called once per device with that device current (on the entry
// point's first call on the device), and only that pointer is handed to the kernels.
//
// Calls on one GPU share its array: two calls whose work overlaps on that GPU (different
// streams, or host threads racing) race on it.  The split kernels write every partial slot
// they later read, so nothing needs clearing between calls.  Nothing here allocates or
// frees device memory.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/tiledattn.h"

namespace {

constexpr int64_t kStaticScratchBytes = int64_t(64) << 20;  // TA_STATIC_SCRATCH_BYTES
static_assert(kStaticScratchBytes == TA_STATIC_SCRATCH_BYTES, "header and library agree");

static __device__ __align__(256) char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once resolved

// The array's address on `device`, resolved on first use with the device current.
ta_status scratch_on_device(int device, void** out, const char** why) {
  if (device < 0 || device >= kMaxDevices) {
    *why = "device ordinal out of range";
    return TA_EINVAL;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] != nullptr) {
    *out = g_scratch_ptr[device];
    return TA_OK;
  }
  int prev = -1;
  if (hipGetDevice(&prev) != hipSuccess) {
    *why = "hipGetDevice failed";
    (void)hipGetLastError();
    return TA_EHIP;
  }
  if (prev != device && hipSetDevice(device) != hipSuccess) {
    *why = "hipSetDevice failed";
    (void)hipGetLastError();
    return TA_EHIP;
  }
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (prev != device) (void)hipSetDevice(prev);
  if (e != hipSuccess || ptr == nullptr) {
    *why = "hipGetSymbolAddress(scratch) failed";
    (void)hipGetLastError();
    return TA_EHIP;
  }
  g_scratch_ptr[device] = ptr;
  *out = ptr;
  return TA_OK;
}

}  // namespace

// Reports a failure through the library's error channel (ta_last_error), defined in
// tiledattn.cpp.
extern "C" __attribute__((visibility("hidden"))) ta_status ta_internal_fail(ta_status st, const char* msg);

extern "C" ta_status ta_sdpa_fwd_split_static(const ta_fwd_args* args, int32_t chunk_steps,
                                              void* stream) {
  if (args == nullptr) return ta_internal_fail(TA_EINVAL, "args is NULL");
  int64_t need = 0;
  // Shape checks and the workspace size, without touching a device.
  ta_status st = ta_split_workspace_size(args, chunk_steps, &need);
  if (st != TA_OK) return st;
  if (need == 0) return ta_sdpa_fwd(args, stream);  // nothing is split: no scratch used
  if (need > kStaticScratchBytes) {
    char msg[160];
    snprintf(msg, sizeof(msg),
             "split workspace of %lld bytes exceeds the static scratch of %lld bytes "
             "(use ta_sdpa_fwd_split with a caller workspace, or a longer chunk)",
             (long long)need, (long long)kStaticScratchBytes);
    return ta_internal_fail(TA_EINVAL, msg);
  }
  void* ptr = nullptr;
  const char* why = "";
  st = scratch_on_device(args->device, &ptr, &why);
  if (st != TA_OK) return ta_internal_fail(st, why);
  return ta_sdpa_fwd_split(args, chunk_steps, ptr, kStaticScratchBytes, stream);
}
