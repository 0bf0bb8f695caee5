// Named shared-memory CPU cache slabs (POSIX shm), shared between the
// serving processes of one host.
//
// Entry points replaced: alloc_shm_pinned_ptr, attach_shm_pinned_ptr,
// free_shm_pinned_ptr, detach_shm_pinned_ptr, unlink_shm
// (csrc/common/mem_alloc.cpp:252-410, bound at csrc/pybind.cpp:352-363).
//
// Creating a slab is a short pipeline over two owners that undo their step
// when a later one fails: a Segment (the name and its descriptor: closed and
// unlinked unless the creation completes) and a Mapping (unmapped unless
// handed out).  The steps:
//   1. create the name exclusively and give the object its size;
//   2. with NUMA nodes, map it and attach an interleave policy to the object
//      itself (mbind), before any page exists, so the pages land spread over
//      the nodes however they are allocated later, and the calling thread's
//      own policy is never touched;
//   3. reserve every page now (fallocate), so a slab larger than what
//      /dev/shm can hold fails here instead of faulting on a later write;
//   4. map with MAP_POPULATE, so the creator's page tables are filled in the
//      kernel's own pass over the reserved pages.
// Attaching maps an existing slab (also populated), after checking that the
// slab is as large as the caller's view of it.
//
// The reference additionally registers every mapping with the accelerator.
// HIP can only make memory that already exists device-visible through
// hipHostRegister, which this library does not use, so a slab is ordinary
// pageable memory to the GPU: transfers reach it through the staged copy
// paths (hipMemcpyAsync), and its address is not in the pinned registry.
#include "common.h"
#include "mem_policy.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <vector>

namespace lmc {
namespace {

std::string why(int err) { return std::strerror(err); }

// The shared-memory object being created.  Until keep() it owns the name:
// destruction closes the descriptor and, for an unkept object, removes the
// name, so a failed creation leaves nothing behind in /dev/shm.
class Segment {
public:
  explicit Segment(const std::string &name) : name_(name) {
    fd_ = shm_open(name.c_str(), O_CREAT | O_EXCL | O_RDWR, 0600);
    if (fd_ < 0) {
      const int err = errno;
      fail(LMC_ERR_RUNTIME,
           "cannot create shared slab " + name + ": " + why(err) +
               (err == EEXIST ? " (the name is taken: another live slab uses it, or a process "
                                "that exited without cleaning up left it; pick another name or "
                                "unlink_shm it)"
                              : ""));
    }
  }
  ~Segment() {
    if (fd_ >= 0) close(fd_);
    if (!kept_) shm_unlink(name_.c_str());
  }
  Segment(const Segment &) = delete;
  Segment &operator=(const Segment &) = delete;
  int fd() const { return fd_; }
  void keep() { kept_ = true; }

private:
  std::string name_;
  int fd_ = -1;
  bool kept_ = false;
};

// A shared mapping of a whole object; unmapped on destruction unless handed
// out with release().
class Mapping {
public:
  Mapping(int fd, size_t size, int prot, int extra_flags, void *at, const std::string &what)
      : size_(size) {
    void *p = mmap(at, size, prot, MAP_SHARED | extra_flags, fd, 0);
    if (p == MAP_FAILED) fail(LMC_ERR_RUNTIME, what + ": " + why(errno));
    addr_ = p;
  }
  ~Mapping() {
    if (addr_ != nullptr) munmap(addr_, size_);
  }
  Mapping(const Mapping &) = delete;
  Mapping &operator=(const Mapping &) = delete;
  void *addr() const { return addr_; }
  uintptr_t release() {
    void *p = addr_;
    addr_ = nullptr;
    return reinterpret_cast<uintptr_t>(p);
  }

private:
  void *addr_ = nullptr;
  size_t size_;
};

void check_size_and_name(const char *op, size_t size, const std::string &name) {
  check(size > 0, std::string(op) + ": size must be positive (slab '" + name + "')");
  check(!name.empty(), std::string(op) + ": a slab name is required");
  check(size <= static_cast<size_t>(std::numeric_limits<off_t>::max()),
        std::string(op) + ": " + std::to_string(size) + " bytes do not fit a file offset");
}

uintptr_t create(size_t size, const std::string &name, const std::vector<int> &nodes) {
  check_size_and_name("alloc_shm_pinned_ptr", size, name);
  if (!nodes.empty()) (void)numa::mask_of(nodes);  // validates the node ids first
  Segment seg(name);
  if (ftruncate(seg.fd(), static_cast<off_t>(size)) != 0)
    fail(LMC_ERR_RUNTIME, "cannot size shared slab " + name + " to " + std::to_string(size) +
                              " bytes: " + why(errno));
  const std::string map_err = "cannot map shared slab " + name;
  void *at = nullptr;
  Mapping *placed = nullptr;
  std::unique_ptr<Mapping> policy_map;
  if (!nodes.empty()) {
    policy_map.reset(new Mapping(seg.fd(), size, PROT_READ | PROT_WRITE, 0, nullptr, map_err));
    numa::interleave_range(policy_map->addr(), size, nodes);
    placed = policy_map.get();
    at = placed->addr();
  }
  const int err = fallocate(seg.fd(), 0, 0, static_cast<off_t>(size));
  if (err != 0)
    fail(LMC_ERR_RUNTIME, "cannot reserve " + std::to_string(size) + " bytes for shared slab " + name +
                              " in /dev/shm: " + why(errno) +
                              " (free space in /dev/shm or choose a smaller CPU cache)");
  // Replace the policy mapping in place (or map afresh) with a populated one.
  Mapping final_map(seg.fd(), size, PROT_READ | PROT_WRITE, MAP_POPULATE | (at ? MAP_FIXED : 0), at,
                    map_err);
  if (placed != nullptr) placed->release();  // the populated mapping now covers its range
  seg.keep();
  return final_map.release();
}

uintptr_t attach(size_t size, const std::string &name, bool writable) {
  check_size_and_name("attach_shm_pinned_ptr", size, name);
  const int fd = shm_open(name.c_str(), writable ? O_RDWR : O_RDONLY, 0600);
  if (fd < 0) fail(LMC_ERR_RUNTIME, "cannot open shared-memory segment " + name + ": " + why(errno));
  struct FdCloser {
    int fd;
    ~FdCloser() { close(fd); }
  } closer{fd};
  struct stat st;
  if (fstat(fd, &st) != 0) fail(LMC_ERR_RUNTIME, "cannot stat shared slab " + name + ": " + why(errno));
  if (static_cast<uint64_t>(st.st_size) < size)
    fail(LMC_ERR_RUNTIME, "shared slab " + name + " holds " + std::to_string(st.st_size) +
                              " bytes, fewer than the " + std::to_string(size) + " requested");
  Mapping m(fd, size, writable ? PROT_READ | PROT_WRITE : PROT_READ, MAP_POPULATE, nullptr,
            "cannot map shared slab " + name);
  return m.release();
}

void unmap(const char *op, uintptr_t ptr, size_t size) {
  check(ptr != 0, std::string(op) + ": the slab pointer is null");
  check(size > 0, std::string(op) + ": size must be positive");
  if (munmap(reinterpret_cast<void *>(ptr), size) != 0)
    fail(LMC_ERR_RUNTIME, std::string(op) + ": munmap failed: " + why(errno));
}

} // namespace
} // namespace lmc

using namespace lmc;

extern "C" {

int lmc_alloc_shm_pinned_ptr(size_t size, const char *shm_name, const int32_t *nodes,
                             int32_t n_nodes, uintptr_t *out_ptr) {
  return guarded([&] {
    check_value(out_ptr != nullptr, "out_ptr is null");
    check_value(n_nodes >= 0 && (n_nodes == 0 || nodes != nullptr), "bad NUMA node list");
    *out_ptr = create(size, shm_name ? shm_name : "", std::vector<int>(nodes, nodes + n_nodes));
  });
}

int lmc_attach_shm_pinned_ptr(size_t size, const char *shm_name, int32_t writable,
                              uintptr_t *out_ptr) {
  return guarded([&] {
    check_value(out_ptr != nullptr, "out_ptr is null");
    *out_ptr = attach(size, shm_name ? shm_name : "", writable != 0);
  });
}

// Unmaps the creator's view and removes the name; peers keep their views
// until they detach.  A name that is already gone is not an error.
int lmc_free_shm_pinned_ptr(uintptr_t ptr, size_t size, const char *shm_name) {
  return guarded([&] {
    const std::string name = shm_name ? shm_name : "";
    unmap("free_shm_pinned_ptr", ptr, size);
    if (shm_unlink(name.c_str()) != 0 && errno != ENOENT)
      fail(LMC_ERR_RUNTIME, "free_shm_pinned_ptr: cannot remove shared slab " + name + ": " + why(errno));
  });
}

int lmc_detach_shm_pinned_ptr(uintptr_t ptr, size_t size) {
  return guarded([&] { unmap("detach_shm_pinned_ptr", ptr, size); });
}

int lmc_unlink_shm(const char *shm_name) {
  return guarded([&] {
    const std::string name = shm_name ? shm_name : "";
    if (shm_unlink(name.c_str()) != 0 && errno != ENOENT)
      fail(LMC_ERR_RUNTIME, "cannot remove shared slab " + name + ": " + why(errno));
  });
}

} // extern "C"
