// oc_decode_layer_noalloc: the decode layer for callers that cannot allocate
// device memory, run in scratch memory the library owns (one static array
// per GPU) instead of a caller workspace.  Declaration and limits:
// include/orthocache_hip.h.
#include <atomic>
#include <mutex>

#include "oc_api_internal.h"

// The scratch array: one copy on every GPU the library runs on, loaded with
// the code object and held until the process ends.  In host code `scratch`
// names a host-side stand-in, not device memory, so nothing here passes it
// to a kernel or a copy: the device address comes from hipGetSymbolAddress,
// looked up once per device with that device current.
static __device__ __align__(256) unsigned char scratch[OC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array.
int scratch_address(void** out) {
  int dev = -1;
  int rc = oc::api_hip_check(hipGetDevice(&dev), "oc_decode_layer_noalloc: hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return oc::api_fail(OC_ERR_UNSUPPORTED, "oc_decode_layer_noalloc: device %d (at most %d devices)", dev,
                        kMaxDevices);
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      rc = oc::api_hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                             "oc_decode_layer_noalloc: hipGetSymbolAddress(scratch)");
      if (rc) return rc;
      if (!p) return oc::api_fail(OC_ERR_HIP, "oc_decode_layer_noalloc: no device address for the scratch array");
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return OC_OK;
}

}  // namespace

extern "C" int oc_decode_layer_noalloc(const oc_layer_args* a, void* stream) {
  static const char* name = "oc_decode_layer_noalloc";
  if (!a) return oc::api_fail(OC_ERR_INVALID_ARGUMENT, "%s: args is NULL", name);
  // Zero when the arguments are invalid (the layer's own validation then
  // reports why) or when the layer needs no workspace at all.
  const size_t need = oc_decode_layer_workspace_size(a);
  if (need == 0) return oc::decode_layer_run(a, nullptr, 0, stream, name);
  if (need > OC_NOALLOC_SCRATCH_BYTES)
    return oc::api_fail(OC_ERR_WORKSPACE,
                        "%s: this layer needs %zu bytes of scratch, more than the %zu the library holds per GPU; "
                        "call oc_decode_layer with a workspace of oc_decode_layer_workspace_size() bytes",
                        name, need, (size_t)OC_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return oc::decode_layer_run(a, ws, OC_NOALLOC_SCRATCH_BYTES, stream, name);
}
