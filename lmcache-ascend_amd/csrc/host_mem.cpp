// Pinned host memory for the zero-copy store/retrieve mode, and the
// host -> device address registry the gather/scatter entry points consult
// for host-resident LMCache memory objects.
//
// Reference behaviour mirrored here (csrc/common/managed_mem.cpp:50-236,
// 374-422; csrc/common/mem_alloc.cpp:19-52): a map of registered ranges,
// looked up by range containment with a required size; alloc_pinned_ptr
// returns page-locked memory that kernels can address.
//
// On MI355X, hipHostMalloc returns memory that is mapped into every GPU's
// address space at the same virtual address (the device address equals the
// host address), so no per-device remap is needed; hipHostGetDevicePointer
// supplies the device address for any HIP-pinned range, including the
// buffers torch allocates with pin_memory=True, which are found even when
// they were never recorded here.
#include "common.h"
#include "mem_policy.h"

#include <cstring>
#include <map>
#include <mutex>
#include <shared_mutex>

namespace lmc {

namespace {

struct Record {
  uintptr_t host;
  uintptr_t dev;
  size_t size;
  bool owned;  // allocated by lmc_alloc_pinned_ptr
};

class Registry {
public:
  static Registry &get() {
    static Registry r;
    return r;
  }

  uintptr_t add(uintptr_t host, uintptr_t dev, size_t size, bool owned) {
    std::unique_lock<std::shared_mutex> g(mu_);
    auto it = map_.find(host);
    if (it != map_.end()) return it->second.dev;
    map_[host] = Record{host, dev, size, owned};
    return dev;
  }

  // Range lookup: the record with the greatest start <= host.  Records never
  // overlap (each is a distinct allocation), so one candidate suffices.
  // Returns false when no record contains `host`; otherwise true, with *dev
  // the translated address, or 0 when the record is too short for
  // `required` bytes.
  bool range(uintptr_t host, PinnedRange *out) const {
    std::shared_lock<std::shared_mutex> g(mu_);
    auto it = map_.upper_bound(host);
    if (it == map_.begin()) return false;
    --it;
    const Record &r = it->second;
    if (host - r.host >= r.size) return false;
    *out = PinnedRange{r.host, r.size, r.dev};
    return true;
  }

  bool find(uintptr_t host, size_t required, uintptr_t *dev) const {
    std::shared_lock<std::shared_mutex> g(mu_);
    auto it = map_.upper_bound(host);
    if (it == map_.begin()) return false;
    --it;
    const Record &r = it->second;
    const size_t off = host - r.host;
    if (off >= r.size) return false;
    *dev = required <= r.size - off ? r.dev + off : 0;
    return true;
  }

  // Removes the record starting at `host` when `pred(record)` holds.
  template <typename P> bool remove_if(uintptr_t host, P pred) {
    std::unique_lock<std::shared_mutex> g(mu_);
    auto it = map_.find(host);
    if (it == map_.end() || !pred(it->second)) return false;
    map_.erase(it);
    return true;
  }

private:
  mutable std::shared_mutex mu_;
  std::map<uintptr_t, Record> map_;
};

thread_local std::string g_last_error;

} // namespace

void set_last_error(const std::string &msg) { g_last_error = msg; }

bool pinned_range(uintptr_t host, PinnedRange *out) {
  if (host == 0) return false;
  if (Registry::get().range(host, out)) return true;
  // Not recorded: ask HIP whether this is pinned (hipHostMalloc) memory, and
  // for the extent of its allocation.  Failed queries leave a sticky error,
  // cleared here for the next call.
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof(attr));
  if (hipPointerGetAttributes(&attr, reinterpret_cast<void *>(host)) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  if (attr.type != hipMemoryTypeHost || attr.devicePointer == nullptr) return false;
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(host)) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const uintptr_t b = reinterpret_cast<uintptr_t>(base);
  if (b > host || host - b >= size) return false;
  // devicePointer is the mapped address of `host` itself
  *out = PinnedRange{b, size, reinterpret_cast<uintptr_t>(attr.devicePointer) - (host - b)};
  return true;
}

uintptr_t translate_host_ptr(uintptr_t host, size_t required) {
  if (host == 0 || required == 0) return 0;
  PinnedRange r;
  if (!pinned_range(host, &r)) return 0;
  const size_t off = host - r.host;
  return required <= r.size - off ? r.dev + off : 0;
}

} // namespace lmc

using namespace lmc;

extern "C" {

const char *lmc_last_error(void) { return lmc::g_last_error.c_str(); }

const char *lmc_version(void) { return "lmcache_amd 0.1 gfx950"; }

int lmc_get_device_ptr(uintptr_t host_ptr, size_t required_size,
                       uintptr_t *out_device_ptr) {
  return guarded([&] {
    check_value(out_device_ptr != nullptr, "out_device_ptr is null");
    *out_device_ptr = translate_host_ptr(host_ptr, required_size);
  });
}

int lmc_register_mapping(uintptr_t host_ptr, uintptr_t dev_ptr, size_t size,
                         uintptr_t *out_device_ptr) {
  return guarded([&] {
    check_value(host_ptr != 0 && dev_ptr != 0 && size > 0,
                "register_mapping needs non-null pointers and a size");
    uintptr_t d = Registry::get().add(host_ptr, dev_ptr, size, false);
    if (out_device_ptr) *out_device_ptr = d;
  });
}

int lmc_unregister_ptr(uintptr_t host_ptr, int32_t *out_status) {
  return guarded([&] {
    const bool removed =
        Registry::get().remove_if(host_ptr, [](const Record &) { return true; });
    if (out_status) *out_status = removed ? 0 : -1;
  });
}

int lmc_alloc_pinned_ptr(size_t size, uint32_t flags, uintptr_t *out_ptr) {
  return guarded([&] {
    check_value(out_ptr != nullptr, "out_ptr is null");
    check_value(size > 0, "alloc_pinned_ptr: size must be positive");
    // Portable + mapped: visible to every GPU at the host virtual address.
    // `flags` is accepted for interface parity and OR-ed into the defaults.
    void *p = nullptr;
    hip_check(hipHostMalloc(&p, size,
                            hipHostMallocPortable | hipHostMallocMapped | flags),
              "hipHostMalloc");
    void *d = nullptr;
    hipError_t e = hipHostGetDevicePointer(&d, p, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(p);
      hip_check(e, "hipHostGetDevicePointer");
    }
    Registry::get().add(reinterpret_cast<uintptr_t>(p),
                        reinterpret_cast<uintptr_t>(d), size, true);
    *out_ptr = reinterpret_cast<uintptr_t>(p);
  });
}

int lmc_free_pinned_ptr(uintptr_t ptr) {
  return guarded([&] {
    const bool owned =
        Registry::get().remove_if(ptr, [](const Record &r) { return r.owned; });
    check(owned, "free_pinned_ptr: pointer was not allocated by "
                 "alloc_pinned_ptr");
    hip_check(hipHostFree(reinterpret_cast<void *>(ptr)), "hipHostFree");
  });
}

int lmc_alloc_pinned_numa_ptr(size_t size, int32_t node, uintptr_t *out_ptr) {
  return guarded([&] {
    check_value(out_ptr != nullptr, "out_ptr is null");
    check(size > 0, "alloc_pinned_numa_ptr: size must be positive");
    check(node >= 0 && node < 1024, "NUMA node must be in [0, 1024)");
    // The reference binds a fresh mapping to `node` and registers it
    // (csrc/common/mem_alloc.cpp:56-92).  Here the pinned allocation itself
    // follows the calling thread's policy (hipHostMallocNumaUser), bound to
    // `node` for the duration of the call.
    void *p = nullptr;
    {
      numa::ThreadNodeBinding bind(node);
      hip_check(hipHostMalloc(&p, size,
                              hipHostMallocPortable | hipHostMallocMapped |
                                  hipHostMallocNumaUser),
                "hipHostMalloc (NUMA)");
      std::memset(p, 0, size);  // any page not placed yet lands on `node`
    }
    void *d = nullptr;
    hipError_t e = hipHostGetDevicePointer(&d, p, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(p);
      hip_check(e, "hipHostGetDevicePointer");
    }
    Registry::get().add(reinterpret_cast<uintptr_t>(p),
                        reinterpret_cast<uintptr_t>(d), size, true);
    *out_ptr = reinterpret_cast<uintptr_t>(p);
  });
}

int lmc_free_pinned_numa_ptr(uintptr_t ptr, size_t size) {
  (void)size;  // the allocation's own size is known to the runtime
  return lmc_free_pinned_ptr(ptr);
}

int lmc_get_gpu_pci_bus_id(int32_t device, char *buf, int32_t buf_len) {
  return guarded([&] {
    check_value(buf != nullptr && buf_len > 0, "buffer is null");
    hip_check(hipDeviceGetPCIBusId(buf, buf_len, device),
              "hipDeviceGetPCIBusId");
  });
}

} // extern "C"
