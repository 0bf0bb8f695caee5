// Thread memory policy (NUMA) for the host allocators.
#pragma once

#include "common.h"

#include <numaif.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <string>
#include <vector>

namespace lmc {

// Sets the calling thread's memory policy to `mode` over `nodes` (an empty
// list leaves the policy alone) and restores the previous one when
// destroyed or on restore().  The syscalls are issued directly, so no NUMA
// library is linked.
class ScopedMemPolicy {
public:
  ScopedMemPolicy(int mode, const std::vector<int> &nodes, bool require_default = false) {
    if (nodes.empty()) return;
    if (syscall(SYS_get_mempolicy, &old_mode_, old_mask_, kBits + 1, nullptr, 0) != 0)
      fail(LMC_ERR_RUNTIME, std::string("get_mempolicy failed: ") + std::strerror(errno));
    if (require_default && old_mode_ != MPOL_DEFAULT)
      fail(LMC_ERR_RUNTIME,
           "shared CPU cache NUMA interleave requires the default thread memory "
           "policy; remove the external numactl policy");
    unsigned long mask[kWords] = {};
    for (int n : nodes) {
      if (n < 0 || n >= kBits)
        fail(LMC_ERR_RUNTIME, "NUMA nodes must be in [0, " + std::to_string(kBits) + ")");
      mask[n / 64] |= 1UL << (n % 64);
    }
    if (syscall(SYS_set_mempolicy, mode, mask, kBits + 1) != 0)
      fail(LMC_ERR_RUNTIME, std::string("set_mempolicy failed: ") + std::strerror(errno));
    active_ = true;
  }
  ~ScopedMemPolicy() {
    if (active_) (void)put_back();
  }
  void restore() {
    if (active_ && put_back() != 0)
      fail(LMC_ERR_RUNTIME, std::string("restore mempolicy failed: ") + std::strerror(errno));
  }

private:
  static constexpr int kBits = 1024;
  static constexpr int kWords = kBits / 64;
  long put_back() {
    active_ = false;
    if (old_mode_ == MPOL_DEFAULT) return syscall(SYS_set_mempolicy, MPOL_DEFAULT, nullptr, 0);
    return syscall(SYS_set_mempolicy, old_mode_, old_mask_, kBits + 1);
  }
  bool active_ = false;
  int old_mode_ = MPOL_DEFAULT;
  unsigned long old_mask_[kWords] = {};
};

} // namespace lmc
