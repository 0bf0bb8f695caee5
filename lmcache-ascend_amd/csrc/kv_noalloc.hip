// lmc_fused_multi_layer_kv_transfer_noalloc: the staged multi-layer transfer
// (fused_transfer, kv_transfer.hip) through a static per-GPU device area
// instead of a caller's staging_cache.  It has no counterpart in the
// reference; it serves callers that cannot allocate device memory (code
// under HIP graph capture, serving loops that forbid hipMalloc).
//
// The area is this file's own code object's, so a process reserves its
// LMC_NOALLOC_STAGING_BYTES on a GPU only once this entry point has run
// there; the other transfers never load it.
#include <mutex>

#include "kv_fused.h"

namespace lmc {
namespace {

// The staging area.  Host code never uses this name as an address: it is
// resolved once per device with hipGetSymbolAddress (area() below).
static __device__ __align__(256) uint8_t scratch[LMC_NOALLOC_STAGING_BYTES];

constexpr int kMaxDevices = 64;

// Per GPU: the area's device address and an event recorded after each eager
// call's work, which the next eager call's stream waits for before it
// touches the area, so eager calls on different streams (a store on an
// offload stream, a load on a load stream) run one after the other.  `mu`
// makes the wait, the enqueue and the record of one call a unit, so two
// threads cannot both wait for the same earlier call.
struct DeviceArea {
  std::mutex mu;
  uint8_t *ptr = nullptr;
  hipEvent_t last = nullptr;
};
std::mutex g_setup_mu;
DeviceArea g_area[kMaxDevices];

// Set-up on the first call per device, with that device current: the
// area's address and the ordering event.  Nothing is allocated afterwards.
DeviceArea &area(int device) {
  check(device >= 0 && device < kMaxDevices,
        "fused_multi_layer_kv_transfer_noalloc: device " +
            std::to_string(device) + " out of range");
  std::lock_guard<std::mutex> lock(g_setup_mu);
  DeviceArea &a = g_area[device];
  if (a.ptr == nullptr) {
    DeviceGuard guard(device);
    void *p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
              "hipGetSymbolAddress(staging area)");
    check(p != nullptr, "hipGetSymbolAddress returned a null staging area");
    hip_check(hipEventCreateWithFlags(&a.last, hipEventDisableTiming),
              "hipEventCreateWithFlags(staging area order)");
    a.ptr = static_cast<uint8_t *>(p);
  }
  return a;
}

} // namespace
} // namespace lmc

using namespace lmc;

extern "C" int lmc_fused_multi_layer_kv_transfer_noalloc(
    const lmc_tensor *key_value, const lmc_tensor *key_value_ptrs,
    const lmc_tensor *slot_mapping, int32_t paged_device,
    int64_t page_buffer_size, int32_t direction, int32_t use_mla,
    int32_t kvcache_format, int64_t k_hidden_dims, int64_t v_hidden_dims,
    int64_t dsa_hidden_dims, void *stream) {
  return guarded([&] {
    const lmc_tensor &kv = deref(key_value, "key_value");
    int device = paged_device;
    if (device < 0) hip_check(hipGetDevice(&device), "hipGetDevice");
    DeviceArea &a = area(device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Under capture the graph's own order applies (waiting for an event
    // recorded outside the capture is not part of a graph); replays that
    // overlap eager calls on another stream of the same GPU race.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hip_check(hipStreamIsCapturing(s, &cap), "hipStreamIsCapturing");
    const bool eager = cap == hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(a.mu);
    if (eager)
      hip_check(hipStreamWaitEvent(s, a.last, 0),
                "hipStreamWaitEvent(staging area order)");
    fused_transfer(kv, a.ptr, device, LMC_NOALLOC_STAGING_BYTES,
                   "fused_multi_layer_kv_transfer_noalloc: the transfer "
                   "exceeds the library's staging area",
                   true, key_value_ptrs, slot_mapping, device,
                   page_buffer_size, direction != 0, use_mla != 0,
                   kvcache_format, k_hidden_dims, v_hidden_dims,
                   dsa_hidden_dims, s);
    if (eager)
      hip_check(hipEventRecord(a.last, s),
                "hipEventRecord(staging area order)");
  });
}
