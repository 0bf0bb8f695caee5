// NUMA placement for the host allocators.  The memory-policy syscalls are
// issued directly, so no NUMA library is linked.
#pragma once

#include "common.h"

#include <numaif.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <array>
#include <cerrno>
#include <cstring>
#include <string>
#include <vector>

namespace lmc {
namespace numa {

constexpr int kNodeLimit = 1024;  // node ids accepted: [0, kNodeLimit)
using NodeMask = std::array<unsigned long, kNodeLimit / (8 * sizeof(unsigned long))>;

inline NodeMask mask_of(const std::vector<int> &nodes) {
  NodeMask m{};
  constexpr int kBitsPerWord = 8 * sizeof(unsigned long);
  for (int n : nodes) {
    if (n < 0 || n >= kNodeLimit)
      fail(LMC_ERR_RUNTIME, "NUMA node " + std::to_string(n) + " is not a valid node id (expected a non-negative "
                            "id below " + std::to_string(kNodeLimit) + ")");
    m[n / kBitsPerWord] |= 1UL << (n % kBitsPerWord);
  }
  return m;
}

// Spreads the pages later allocated for [addr, addr + len) of a shared
// mapping round-robin over `nodes`.  For a shared-memory object the policy
// is kept by the object itself, so it decides where the object's pages land
// whichever process or call allocates them.
inline void interleave_range(void *addr, size_t len, const std::vector<int> &nodes) {
  const NodeMask m = mask_of(nodes);
  if (syscall(SYS_mbind, addr, len, MPOL_INTERLEAVE, m.data(), kNodeLimit + 1, 0) != 0)
    fail(LMC_ERR_RUNTIME, std::string("interleaving the shared slab over its NUMA nodes failed (mbind): ") +
                              std::strerror(errno));
}

// Restricts the calling thread's page allocations to one node for the
// lifetime of the object, then puts the thread's previous policy back.
class ThreadNodeBinding {
public:
  explicit ThreadNodeBinding(int node) {
    if (syscall(SYS_get_mempolicy, &saved_mode_, saved_.data(), kNodeLimit + 1, nullptr, 0) != 0)
      fail(LMC_ERR_RUNTIME, std::string("reading the thread's NUMA policy failed: ") + std::strerror(errno));
    const NodeMask m = mask_of({node});
    if (syscall(SYS_set_mempolicy, MPOL_BIND, m.data(), kNodeLimit + 1) != 0)
      fail(LMC_ERR_RUNTIME, "binding the thread to NUMA node " + std::to_string(node) +
                                " failed: " + std::strerror(errno));
  }
  ~ThreadNodeBinding() {
    if (saved_mode_ == MPOL_DEFAULT)
      (void)syscall(SYS_set_mempolicy, MPOL_DEFAULT, nullptr, 0);
    else
      (void)syscall(SYS_set_mempolicy, saved_mode_, saved_.data(), kNodeLimit + 1);
  }
  ThreadNodeBinding(const ThreadNodeBinding &) = delete;
  ThreadNodeBinding &operator=(const ThreadNodeBinding &) = delete;

private:
  int saved_mode_ = MPOL_DEFAULT;
  NodeMask saved_{};
};

} // namespace numa
} // namespace lmc
