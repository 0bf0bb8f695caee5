// Named shared-memory CPU cache slabs (POSIX shm), shared between the
// serving processes of one host.
//
// Replaces alloc_shm_pinned_ptr / attach_shm_pinned_ptr /
// free_shm_pinned_ptr / detach_shm_pinned_ptr / unlink_shm
// (csrc/common/mem_alloc.cpp:108-410, bound at csrc/pybind.cpp:352-363).
// The creator reserves the whole slab in /dev/shm (posix_fallocate) and
// prefaults it while an optional MPOL_INTERLEAVE policy over the given NUMA
// nodes is active, so the pages are spread before any peer attaches.
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
#include <string>
#include <vector>

namespace lmc {
namespace {

std::string errstr(int e) { return std::strerror(e); }

void first_touch(void *p, size_t size) {
  // Page tables are populated by the kernel in one call where it can; a
  // resource failure aborts the creation, an unsupported advice falls back
  // to touching one byte per page.
  if (madvise(p, size, MADV_POPULATE_WRITE) == 0) return;
  const int err = errno;
  if (err != EINVAL && err != ENOSYS && err != EOPNOTSUPP)
    fail(LMC_ERR_RUNTIME, "shared slab prefault failed: " + errstr(err));
  const long ps = sysconf(_SC_PAGESIZE);
  check(ps > 0, "unable to determine shared slab page size");
  volatile char *c = static_cast<volatile char *>(p);
  for (size_t off = 0; off < size; off += static_cast<size_t>(ps)) c[off] = 0;
}

void reserve(int fd, size_t size, const std::string &name) {
  check(size <= static_cast<size_t>(std::numeric_limits<off_t>::max()),
        "shm size exceeds off_t max for " + name);
  const int err = posix_fallocate(fd, 0, static_cast<off_t>(size));
  if (err != 0)
    fail(LMC_ERR_RUNTIME,
         "posix_fallocate failed for " + name +
             " before first_touch (not enough /dev/shm space or quota for shared "
             "CPU cache slab; reduce max_local_cpu_size/shared_cpu_cache_size_gb "
             "or increase /dev/shm): " +
             errstr(err));
}

uintptr_t create(size_t size, const std::string &name, const std::vector<int> &nodes) {
  check(size > 0, "alloc_shm_pinned_ptr requires size > 0 for " + name);
  check(!name.empty(), "alloc_shm_pinned_ptr requires a shm_name");
  for (int n : nodes) check(n >= 0, "NUMA interleave nodes must be non-negative");
  ScopedMemPolicy policy(MPOL_INTERLEAVE, nodes, /*require_default=*/true);
  const int fd = shm_open(name.c_str(), O_CREAT | O_EXCL | O_RDWR, 0600);
  if (fd < 0)
    fail(LMC_ERR_RUNTIME,
         "shm_open create failed for " + name +
             " (shared CPU cache segment already exists or cannot be created; "
             "this usually means a live name collision or stale segment from an "
             "unclean shutdown, so choose a unique shared_cpu_cache_name or unlink "
             "the stale segment before restart): " +
             errstr(errno));
  void *p = MAP_FAILED;
  try {
    if (ftruncate(fd, static_cast<off_t>(size)) != 0)
      fail(LMC_ERR_RUNTIME, "ftruncate failed for " + name + ": " + errstr(errno));
    reserve(fd, size, name);
    p = mmap(nullptr, size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    if (p == MAP_FAILED) fail(LMC_ERR_RUNTIME, "mmap failed for " + name + ": " + errstr(errno));
    close(fd);
    first_touch(p, size);
    policy.restore();
  } catch (...) {
    if (p != MAP_FAILED)
      munmap(p, size);
    else
      close(fd);
    shm_unlink(name.c_str());
    throw;
  }
  return reinterpret_cast<uintptr_t>(p);
}

uintptr_t attach(size_t size, const std::string &name, bool writable) {
  check(size > 0, "attach_shm_pinned_ptr requires size > 0 for " + name);
  check(!name.empty(), "attach_shm_pinned_ptr requires a shm_name");
  const int fd = shm_open(name.c_str(), writable ? O_RDWR : O_RDONLY, 0600);
  if (fd < 0)
    fail(LMC_ERR_RUNTIME, "shm_open attach failed for " + name + ": " + errstr(errno));
  struct stat st;
  const bool sized = fstat(fd, &st) == 0 && static_cast<uint64_t>(st.st_size) >= size;
  if (!sized) {
    close(fd);
    fail(LMC_ERR_RUNTIME, "shm segment " + name + " is smaller than the requested " +
                              std::to_string(size) + " bytes");
  }
  void *p = mmap(nullptr, size, writable ? PROT_READ | PROT_WRITE : PROT_READ, MAP_SHARED, fd, 0);
  const int err = errno;
  close(fd);
  if (p == MAP_FAILED) fail(LMC_ERR_RUNTIME, "mmap attach failed for " + name + ": " + errstr(err));
  return reinterpret_cast<uintptr_t>(p);
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
    std::vector<int> list(nodes, nodes + n_nodes);
    *out_ptr = create(size, shm_name ? shm_name : "", list);
  });
}

int lmc_attach_shm_pinned_ptr(size_t size, const char *shm_name, int32_t writable,
                              uintptr_t *out_ptr) {
  return guarded([&] {
    check_value(out_ptr != nullptr, "out_ptr is null");
    *out_ptr = attach(size, shm_name ? shm_name : "", writable != 0);
  });
}

int lmc_free_shm_pinned_ptr(uintptr_t ptr, size_t size, const char *shm_name) {
  return guarded([&] {
    const std::string name = shm_name ? shm_name : "";
    check(ptr != 0, "free_shm_pinned_ptr requires non-null ptr");
    check(size > 0, "free_shm_pinned_ptr requires size > 0 for " + name);
    const int rc = munmap(reinterpret_cast<void *>(ptr), size);
    const int err = errno;
    shm_unlink(name.c_str());
    if (rc != 0) fail(LMC_ERR_RUNTIME, "munmap failed: " + std::to_string(err));
  });
}

int lmc_detach_shm_pinned_ptr(uintptr_t ptr, size_t size) {
  return guarded([&] {
    check(ptr != 0, "detach_shm_pinned_ptr requires non-null ptr");
    check(size > 0, "detach_shm_pinned_ptr requires size > 0");
    if (munmap(reinterpret_cast<void *>(ptr), size) != 0)
      fail(LMC_ERR_RUNTIME, "munmap detach failed: " + std::to_string(errno));
  });
}

int lmc_unlink_shm(const char *shm_name) {
  return guarded([&] {
    const std::string name = shm_name ? shm_name : "";
    if (shm_unlink(name.c_str()) != 0 && errno != ENOENT)
      fail(LMC_ERR_RUNTIME, "shm_unlink failed for " + name + ": " + errstr(errno));
  });
}

} // extern "C"
