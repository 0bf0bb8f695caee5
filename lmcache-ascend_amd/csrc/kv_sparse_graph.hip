// Sparse-attention KV copy for graph replay ("sfa_copy") on MI355X (gfx950).
//
// Replaces sparse_graph_kv_transfer (csrc/mem_kernels.cpp:754-831; device
// semantics csrc/graph/sparse_graph_kernel.cpp:6-72).  Requests are rows of
// a packed [requests, row_width] matrix of selected tokens and destination
// slots; row r is active for its first min(counts[r * stride], row_width)
// columns, and not at all when its count or limits[r] is <= 0.  Entry
// (r, j) copies token `selected[r, j]` (valid in [0, limits[r])) of
// request r: chunk = token / chunk_size, row token % chunk_size of the
// chunk's K and PE sources, found in the two plane tables
// ptrs[0, r * chunks_per_request + chunk] and ptrs[1, ...] (a null source
// skips the entry), into row slots[r, j] of the K and PE caches (flat rows
// of k_bytes and pe_bytes).  Everything the entries read is decided on the
// device from this replay's counts and limits, and every bound is checked
// before an address is formed.
//
// Work mapping: a group of G lanes (a power of two up to 64, enough for
// four 16-byte accesses per lane to cover the wider of the two rows) owns
// one entry and issues both rows' loads before their stores; rows whose
// source or destination is not 16-byte aligned are copied bytewise.
#include "common.h"
#include "gmem.h"

#include <algorithm>
#include <cstring>

namespace lmc {

namespace {

constexpr int kSfaThreads = 256;
constexpr int kSfaUnroll = 4;  // 16-byte accesses per lane and row in one pass
// Rows are stored with the streaming hint: the destinations are always the
// device caches, and the copy leaves nothing another kernel reads soon.
// Measured on MI355X (64 requests x 2048 selected MLA rows, three runs
// each): device sources 0.0684-0.0687 -> 0.0530-0.0532 ms, pinned host
// sources unchanged (2.764 ms); streaming loads as well gave 0.0675-0.0678
// ms from device sources, so loads stay plain.

struct SfaJob {
  uint64_t k;
  uint64_t pe;
  const void *slots;
  const void *selected;
  const int32_t *counts;
  const int32_t *limits;
  const uint64_t *table;
  int32_t slot_i64;
  int32_t sel_i64;
  int32_t chunk_size;
  int32_t chunks_per_request;
  int32_t requests;
  int32_t row_width;
  int32_t count_stride;
  int32_t k_bytes;
  int32_t pe_bytes;
  int32_t group_shift;
  int32_t one_pass;
  int64_t dest_slots;
};

using SfaVec = unsigned int __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void sfa_row(uint8_t *dst, const uint8_t *src,
                                        int bytes, int gl, int G) {
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
    for (int v = gl; v < bytes / 16; v += G)
      gstore_nt(reinterpret_cast<SfaVec *>(dst) + v, gload(reinterpret_cast<const SfaVec *>(src) + v));
  } else {
    for (int b = gl; b < bytes; b += G) dst[b] = src[b];
  }
}

__global__ void __launch_bounds__(kSfaThreads) sfa_copy(SfaJob job) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kSfaThreads + threadIdx.x;
  const int64_t e = gid >> job.group_shift;
  const int G = 1 << job.group_shift;
  const int gl = static_cast<int>(gid & (G - 1));
  if (e >= static_cast<int64_t>(job.requests) * job.row_width) return;
  const int r = static_cast<int>(e / job.row_width);
  const int col = static_cast<int>(e - static_cast<int64_t>(r) * job.row_width);
  // The row's count and limit and the entry's token and slot are
  // independent loads, issued together.
  const int32_t cnt = job.counts[static_cast<int64_t>(r) * job.count_stride];
  const int32_t lim = job.limits[r];
  const int64_t token = job.sel_i64 ? static_cast<const int64_t *>(job.selected)[e]
                                    : static_cast<const int32_t *>(job.selected)[e];
  const int64_t dest = job.slot_i64 ? static_cast<const int64_t *>(job.slots)[e]
                                    : static_cast<const int32_t *>(job.slots)[e];
  const int32_t active = (lim <= 0 || cnt <= 0) ? 0 : (cnt < job.row_width ? cnt : job.row_width);
  if (col >= active) return;
  if (token < 0 || token >= lim || dest < 0 || dest >= job.dest_slots) return;
  const int64_t chunk = token / job.chunk_size;
  if (chunk >= job.chunks_per_request) return;
  const int64_t off = token % job.chunk_size;
  const int64_t ti = static_cast<int64_t>(r) * job.chunks_per_request + chunk;
  const uint64_t ks = job.table[ti];
  const uint64_t ps = job.table[static_cast<int64_t>(job.requests) * job.chunks_per_request + ti];
  if (ks == 0 || ps == 0) return;
  const uint8_t *ksrc = reinterpret_cast<const uint8_t *>(ks) + off * job.k_bytes;
  const uint8_t *psrc = reinterpret_cast<const uint8_t *>(ps) + off * job.pe_bytes;
  uint8_t *kdst = reinterpret_cast<uint8_t *>(job.k) + dest * job.k_bytes;
  uint8_t *pdst = reinterpret_cast<uint8_t *>(job.pe) + dest * job.pe_bytes;
  const uintptr_t align = reinterpret_cast<uintptr_t>(ksrc) | reinterpret_cast<uintptr_t>(psrc) |
                          reinterpret_cast<uintptr_t>(kdst) | reinterpret_cast<uintptr_t>(pdst);
  if (job.one_pass && (align & 15) == 0) {
    // Both rows fit kSfaUnroll passes of the group: all loads, then all
    // stores.
    const int kv = job.k_bytes / 16, pv = job.pe_bytes / 16;
    SfaVec xk[kSfaUnroll], xp[kSfaUnroll];
#pragma unroll
    for (int u = 0; u < kSfaUnroll; ++u) {
      const int v = gl + u * G;
      if (v < kv) xk[u] = gload(reinterpret_cast<const SfaVec *>(ksrc) + v);
      if (v < pv) xp[u] = gload(reinterpret_cast<const SfaVec *>(psrc) + v);
    }
#pragma unroll
    for (int u = 0; u < kSfaUnroll; ++u) {
      const int v = gl + u * G;
      if (v < kv) gstore_nt(reinterpret_cast<SfaVec *>(kdst) + v, xk[u]);
      if (v < pv) gstore_nt(reinterpret_cast<SfaVec *>(pdst) + v, xp[u]);
    }
    return;
  }
  sfa_row(kdst, ksrc, job.k_bytes, gl, G);
  sfa_row(pdst, psrc, job.pe_bytes, gl, G);
}

bool contiguous(const lmc_tensor &t) {
  int64_t expect = 1;
  for (int i = t.ndim - 1; i >= 0; --i) {
    if (t.sizes[i] != 1 && t.strides[i] != expect) return false;
    expect *= t.sizes[i];
  }
  return true;
}

// The input conditions of csrc/mem_kernels.cpp:758-800 (messages in this
// library's words).
void sparse_graph(const lmc_tensor &k, const lmc_tensor &pe, int64_t kH, int64_t peH,
                  const lmc_tensor &slots, const lmc_tensor &sel, const lmc_tensor &counts,
                  const lmc_tensor &ptrs, const lmc_tensor &limits, int64_t chunk_size,
                  int64_t max_cores, hipStream_t stream) {
  check(sel.ndim == 2 && contiguous(sel), "sparse graph: selected tokens are not a contiguous [rows, columns] matrix");
  bool same = slots.ndim == 2 && contiguous(slots);
  for (int i = 0; same && i < 2; ++i) same = slots.sizes[i] == sel.sizes[i];
  check(same, "sparse graph: slots and selected tokens differ in shape or layout");
  check(sel.dtype == LMC_I32 || sel.dtype == LMC_I64, "sparse graph: selected tokens are neither int32 nor int64");
  check(slots.dtype == LMC_I32 || slots.dtype == LMC_I64, "sparse graph: slots are neither int32 nor int64");
  const int64_t requests = sel.sizes[0];
  check(requests > 0 && sel.sizes[1] > 0 && numel(sel) <= INT32_MAX,
        "sparse graph: no rows, or more selected entries than int32 indexes");
  const int64_t cstride = counts.ndim > 0 ? counts.strides[0] : 0;
  check((counts.ndim == 1 || (counts.ndim == 2 && counts.sizes[1] > 0)) &&
            counts.sizes[0] == requests && counts.dtype == LMC_I32 && cstride > 0 &&
            cstride <= INT32_MAX,
        "sparse graph: counts are not one int32 per row");
  check((requests - 1) * cstride + 1 <= extent_bytes(counts) / 4,
        "sparse graph: counts are not one int32 per row");
  check(numel(limits) == requests && contiguous(limits) && limits.dtype == LMC_I32,
        "sparse graph: limits are not one contiguous int32 per row");
  check(ptrs.ndim == 2 && ptrs.sizes[0] == 2 && ptrs.sizes[1] > 0 &&
            ptrs.sizes[1] % requests == 0 && contiguous(ptrs) && ptrs.dtype == LMC_I64,
        "sparse graph: chunk sources are not a contiguous int64 [2, chunks] table");
  check(chunk_size > 0 && chunk_size <= INT32_MAX && ptrs.sizes[1] <= INT32_MAX / chunk_size,
        "sparse graph: chunk tokens exceed int32 indexing");
  check(k.dtype == LMC_F16 || k.dtype == LMC_BF16, "sparse graph: caches are neither float16 nor bfloat16");
  if (kH <= 0) kH = size(k, -2) * size(k, -1);
  if (peH <= 0) peH = size(pe, -2) * size(pe, -1);
  const int64_t k_bytes = kH * 2, pe_bytes = peH * 2;
  check(k.data && pe.data && k_bytes > 0 && pe_bytes > 0 && k_bytes % 32 == 0 &&
            pe_bytes % 32 == 0 && k_bytes <= 16384 && pe_bytes <= 16384,
        "sparse graph: K and PE rows must be non-empty multiples of 32 bytes up to 16 KiB");
  check(sel.device >= 0 && slots.device == sel.device && counts.device == sel.device &&
            ptrs.device == sel.device && limits.device == sel.device &&
            k.device == sel.device && pe.device == sel.device,
        "the graph transfer's tensors are on different GPUs");
  check(max_cores >= 0 && max_cores <= UINT32_MAX,
        "max_aiv_cores is negative or above the uint32 range");
  DeviceGuard guard(sel.device);
  SfaJob job;
  std::memset(&job, 0, sizeof(job));
  job.k = reinterpret_cast<uint64_t>(k.data);
  job.pe = reinterpret_cast<uint64_t>(pe.data);
  job.slots = slots.data;
  job.selected = sel.data;
  job.counts = static_cast<const int32_t *>(counts.data);
  job.limits = static_cast<const int32_t *>(limits.data);
  job.table = static_cast<const uint64_t *>(ptrs.data);
  job.slot_i64 = slots.dtype == LMC_I64;
  job.sel_i64 = sel.dtype == LMC_I64;
  job.chunk_size = static_cast<int32_t>(chunk_size);
  job.chunks_per_request = static_cast<int32_t>(ptrs.sizes[1] / requests);
  job.requests = static_cast<int32_t>(requests);
  job.row_width = static_cast<int32_t>(sel.sizes[1]);
  job.count_stride = static_cast<int32_t>(cstride);
  job.k_bytes = static_cast<int32_t>(k_bytes);
  job.pe_bytes = static_cast<int32_t>(pe_bytes);
  job.dest_slots = std::min(nbytes(k) / k_bytes, nbytes(pe) / pe_bytes);
  // Lanes per entry: enough for kSfaUnroll accesses per lane to cover the
  // wider row (up to a wave), so a wave holds several entries and each lane
  // keeps several loads in flight.
  const int64_t vecs = std::max(k_bytes, pe_bytes) / 16;
  int shift = 0;
  while ((int64_t(kSfaUnroll) << shift) < vecs && shift < 6) ++shift;
  job.group_shift = shift;
  job.one_pass = vecs <= (int64_t(kSfaUnroll) << shift);
  const int64_t threads = numel(sel) << shift;
  const int64_t blocks = (threads + kSfaThreads - 1) / kSfaThreads;
  // max_aiv_cores caps the reference's AI-vector cores for prefetch callers;
  // the launch here is sized by the entries.
  hipLaunchKernelGGL(sfa_copy, dim3(static_cast<unsigned>(blocks)), dim3(kSfaThreads), 0,
                     stream, job);
  hip_check(hipGetLastError(), "sfa_copy launch");
}

} // namespace
} // namespace lmc

using namespace lmc;

extern "C" {

int lmc_sparse_graph_kv_transfer(const lmc_tensor *k_cache, const lmc_tensor *pe_cache,
                                 int64_t k_hidden_dims, int64_t pe_hidden_dims,
                                 const lmc_tensor *slots, const lmc_tensor *selected,
                                 const lmc_tensor *counts, const lmc_tensor *ptrs,
                                 const lmc_tensor *limits, int64_t chunk_size,
                                 int64_t max_aiv_cores, void *stream) {
  return guarded([&] {
    sparse_graph(deref(k_cache, "k_cache"), deref(pe_cache, "pe_cache"), k_hidden_dims,
                 pe_hidden_dims, deref(slots, "slots"), deref(selected, "selected"),
                 deref(counts, "counts"), deref(ptrs, "ptrs"), deref(limits, "limits"),
                 chunk_size, max_aiv_cores, static_cast<hipStream_t>(stream));
  });
}

} // extern "C"
