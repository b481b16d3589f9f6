// mimir_prefixlm_fwd_noalloc: the forward without a caller-provided workspace,
// for callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).
//
// The forward's only scratch memory here is the heaviest-first query-tile work
// list (int4 per 128-row tile, ceil(T / 128) + numseqs entries) and the K scan's
// slots, which the prologue writes completely on every call (entries past the
// last tile are padding), so nothing in it has to start at zero.  The array is
// far below the size at which the forward cuts key ranges into parts
// (mimir_prefixlm_fwd_workspace_size), so those parts' slots are never used.  Here it lives in a file-scope device array
// of kNoAllocScratchBytes, one copy per GPU, held until the process ends.  Host
// code never passes the array's name to a kernel (in host code that name is a
// host-side stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, looked up on the first call per device with that device
// current, and kept for the life of the process (a hipDeviceReset or another
// re-creation of the device's primary context would make it stale: the entry
// point is not for use across one).  Every call on one GPU shares that GPU's
// array, so calls that overlap on one GPU (two streams, two host threads) race.
#include <mutex>
#include <string>

#include "prefixlm_common.h"

namespace {

constexpr size_t kNoAllocScratchBytes = 128 * 1024;  // 8064 list entries + the K-scan slots
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// The device address of `scratch` on the current device, looked up on the first
// call per device; nullptr (and the library's last error set) on failure.
void* scratch_on_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    mimir::fail_with(MIMIR_ERR_HIP, std::string("mimir_prefixlm_fwd_noalloc: no usable current HIP device: ") +
                                        hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      mimir::fail_with(MIMIR_ERR_HIP, std::string("mimir_prefixlm_fwd_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                                          hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int mimir_prefixlm_fwd_noalloc(const MimirPrefixLMFwdParams* p, void* stream) {
  if (p == nullptr) return mimir::fail_with(MIMIR_ERR_INVALID_ARGUMENT, "params is NULL");
  // The size check needs no device: a call that does not fit is refused before
  // anything touches the GPU.
  const size_t need = mimir_prefixlm_fwd_workspace_bytes(p->total_tokens, p->numseqs, p->max_seqlen_all);
  if (need > kNoAllocScratchBytes)
    return mimir::fail_with(MIMIR_ERR_UNSUPPORTED_SHAPE,
                            "mimir_prefixlm_fwd_noalloc: the tile work list needs " + std::to_string(need) +
                                " bytes (ceil(total_tokens / 128) + numseqs entries of 16 bytes and 2 KiB of K-scan slots), above its fixed " +
                                std::to_string(kNoAllocScratchBytes) +
                                "-byte device array; use mimir_prefixlm_fwd with a workspace");
  MimirPrefixLMFwdParams q = *p;
  q.workspace = nullptr;
  q.workspace_bytes = 0;
  if (need > 0) {
    void* ptr = scratch_on_current_device();
    if (ptr == nullptr) return MIMIR_ERR_HIP;
    q.workspace = ptr;
    q.workspace_bytes = kNoAllocScratchBytes;
  }
  return mimir_prefixlm_fwd(&q, stream);
}
