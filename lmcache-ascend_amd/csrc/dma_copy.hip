// Layerwise prefill DMA: host<->device byte rows.
//
// Replaces layerwise_prefill_dma_copy and its diagnostic twin
// (csrc/pybind.cpp:263-310).  The reference submits one async memcpy per
// (dst, src, bytes) row on the current stream.  The rows come from a
// planner that emits one row per (token range, plane), split where the
// block ids stop being consecutive
// (lmcache_ascend/v1/npu_connector/layerwise_dma.py:147-211, 558-594).
//
// On MI355X a copy-engine (SDMA) copy costs several microseconds beyond its
// bytes, so one copy per scattered 256 KiB row reaches a third of PCIe and
// one per 32 KiB row a tenth.  When no two destinations overlap the order
// of the rows does not change the result, and the submission is reshaped:
//   1. rows are ordered by their device-side address (each plane's cache is
//      one allocation, so its rows stay together);
//   2. rows adjacent in both address spaces are merged;
//   3. rows whose host side lies in pinned, device-mapped memory are copied
//      by one small kernel (at most 64 workgroups, so a prefill running
//      beside it keeps nearly every compute unit), 64 rows per launch with
//      the row table in the kernel arguments;
//   4. rows over pageable host memory, and rows of 4 MiB or more, go to the
//      copy engines: runs of four or more equal-length rows at constant
//      pitches as one rectangular copy, the rest one by one.
// Rectangular copies between device and pinned memory were measured at
// 53 GB/s on a fresh process but 20 GB/s after a long run of other work,
// while the kernel held 54 GB/s in both; pinned rows therefore always take
// the kernel.  With overlapping destinations the rows are submitted in the
// caller's order on the copy engines, merging only consecutive adjacent
// rows, which keeps the last-writer-wins result of the reference.
#include "common.h"
#include "gmem.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <vector>

namespace lmc {
namespace {

struct Seg {
  uint64_t dst, src, bytes;
};

constexpr int kRowsPerLaunch = 64;
constexpr int kSegThreads = 256;
constexpr int kSegUnroll = 8;                                   // 16-byte vectors per thread
constexpr uint32_t kPieceBytes = kSegThreads * kSegUnroll * 16;  // 32 KiB per block-step
constexpr int kSegMaxBlocks = 64;
constexpr uint64_t kEngineRowBytes = 4ull << 20;
constexpr size_t kMinRun = 4;

// Row table of one launch, passed by value.  Row r covers pieces
// [piece_end[r - 1], piece_end[r]) of kPieceBytes each.
struct SegTable {
  uint64_t dst[kRowsPerLaunch];
  uint64_t src[kRowsPerLaunch];
  uint32_t bytes[kRowsPerLaunch];
  uint32_t piece_end[kRowsPerLaunch];
  int32_t rows;
};

__global__ void __launch_bounds__(kSegThreads) seg_copy(SegTable t) {
  using V = unsigned int __attribute__((ext_vector_type(4)));
  const uint32_t total = t.piece_end[t.rows - 1];
  for (uint32_t piece = blockIdx.x; piece < total; piece += gridDim.x) {
    int lo = 0, hi = t.rows - 1;  // first row whose piece_end > piece
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (t.piece_end[mid] > piece) hi = mid;
      else lo = mid + 1;
    }
    const uint32_t first = lo ? t.piece_end[lo - 1] : 0;
    const uint64_t off = static_cast<uint64_t>(piece - first) * kPieceBytes;
    const uint32_t n = static_cast<uint32_t>(
        t.bytes[lo] - off < kPieceBytes ? t.bytes[lo] - off : kPieceBytes);
    uint8_t *dst = reinterpret_cast<uint8_t *>(t.dst[lo]) + off;
    const uint8_t *src = reinterpret_cast<const uint8_t *>(t.src[lo]) + off;
    if (((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0) {
      const uint32_t nv = n / 16;
      if (nv == kSegThreads * kSegUnroll) {
        V v[kSegUnroll];
#pragma unroll
        for (int k = 0; k < kSegUnroll; ++k)
          v[k] = gload(reinterpret_cast<const V *>(src) + k * kSegThreads + threadIdx.x);
#pragma unroll
        for (int k = 0; k < kSegUnroll; ++k)
          gstore(reinterpret_cast<V *>(dst) + k * kSegThreads + threadIdx.x, v[k]);
      } else {
        for (uint32_t k = threadIdx.x; k < nv; k += kSegThreads)
          gstore(reinterpret_cast<V *>(dst) + k, gload(reinterpret_cast<const V *>(src) + k));
      }
      for (uint32_t b = nv * 16 + threadIdx.x; b < n; b += kSegThreads) dst[b] = src[b];
    } else {
      for (uint32_t b = threadIdx.x; b < n; b += kSegThreads) dst[b] = src[b];
    }
  }
}

void submit_1d(const Seg &s, hipMemcpyKind kind, hipStream_t stream) {
  hipError_t e = hipMemcpyAsync(reinterpret_cast<void *>(s.dst), reinterpret_cast<const void *>(s.src),
                                s.bytes, kind, stream);
  if (e != hipSuccess)
    fail(LMC_ERR_RUNTIME, std::string("layerwise prefill copies were not enqueued: status ") +
                              std::to_string(static_cast<int>(e)) + " bytes=" + std::to_string(s.bytes) +
                              " (" + hipGetErrorString(e) + ")");
}

// One rectangular copy of rows [first, first + n), which share their length
// and repeat at pitches dp and sp.  The runtime refuses a rectangle whose
// span leaves one allocation (two planes' caches, two host buffers) before
// queueing anything; the refusal is cleared from the thread's last-error
// state and the rows are handed back to be copied one by one.
bool submit_run(const std::vector<Seg> &segs, size_t first, size_t n, uint64_t dp, uint64_t sp,
                hipMemcpyKind kind, hipStream_t stream) {
  const Seg &a = segs[first];
  hipError_t e = hipMemcpy2DAsync(reinterpret_cast<void *>(a.dst), dp, reinterpret_cast<const void *>(a.src), sp,
                                  a.bytes, n, kind, stream);
  if (e == hipSuccess) return true;
  (void)hipGetLastError();
  return false;
}

// Largest row pitch a rectangular copy accepts on the current device.
uint64_t device_max_pitch() {
  static std::atomic<int64_t> cache[64];
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev >= 0 && dev < 64) {
    const int64_t v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return static_cast<uint64_t>(v);
  }
  int pitch = 0;
  hip_check(hipDeviceGetAttribute(&pitch, hipDeviceAttributeMaxPitch, dev), "hipDeviceGetAttribute");
  if (pitch <= 0) return 0;
  if (dev >= 0 && dev < 64) cache[dev].store(pitch, std::memory_order_relaxed);
  return static_cast<uint64_t>(pitch);
}

// Appends `s` to `out`, merging it into the last row when the two are
// adjacent in both address spaces.
void push_merged(std::vector<Seg> &out, const Seg &s) {
  if (!out.empty()) {
    Seg &b = out.back();
    if (b.dst + b.bytes == s.dst && b.src + b.bytes == s.src) {
      b.bytes += s.bytes;
      return;
    }
  }
  out.push_back(s);
}

// Device-visible address of host range [h, h + n), or 0 when it is not
// inside one pinned, mapped allocation.  `seen` caches the allocations
// found during this call.
uint64_t mapped(uint64_t h, uint64_t n, std::vector<PinnedRange> &seen) {
  for (const PinnedRange &r : seen)
    if (h >= r.host && h - r.host < r.size) return n <= r.size - (h - r.host) ? r.dev + (h - r.host) : 0;
  PinnedRange r;
  if (!pinned_range(h, &r)) return 0;
  seen.push_back(r);
  return n <= r.size - (h - r.host) ? r.dev + (h - r.host) : 0;
}

void launch_rows(const std::vector<Seg> &rows, hipStream_t stream) {
  for (size_t base = 0; base < rows.size(); base += kRowsPerLaunch) {
    SegTable t;
    const int n = static_cast<int>(std::min<size_t>(kRowsPerLaunch, rows.size() - base));
    uint32_t pieces = 0;
    for (int r = 0; r < n; ++r) {
      const Seg &s = rows[base + r];
      t.dst[r] = s.dst;
      t.src[r] = s.src;
      t.bytes[r] = static_cast<uint32_t>(s.bytes);
      pieces += static_cast<uint32_t>((s.bytes + kPieceBytes - 1) / kPieceBytes);
      t.piece_end[r] = pieces;
    }
    t.rows = n;
    const unsigned grid = std::min<uint32_t>(pieces, kSegMaxBlocks);
    hipLaunchKernelGGL(seg_copy, dim3(grid), dim3(kSegThreads), 0, stream, t);
    hip_check(hipGetLastError(), "seg_copy launch");
  }
}

void dma_copy(const lmc_dma_segment *rows, int64_t n, bool d2h, hipStream_t stream) {
  check_value(n >= 0 && (n == 0 || rows != nullptr), "copies is null");
  const hipMemcpyKind kind = d2h ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice;
  std::vector<Seg> segs;
  segs.reserve(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) {
    if (rows[i].bytes == 0) continue;
    check(rows[i].dst != 0 && rows[i].src != 0, "Layerwise prefill DMA row " + std::to_string(i) +
                                                    " has a null address");
    check(rows[i].dst + rows[i].bytes > rows[i].dst && rows[i].src + rows[i].bytes > rows[i].src,
          "Layerwise prefill DMA row " + std::to_string(i) + " wraps the address space");
    segs.push_back({rows[i].dst, rows[i].src, rows[i].bytes});
  }
  if (segs.empty()) return;
  std::vector<Seg> sorted = segs;
  std::stable_sort(sorted.begin(), sorted.end(), [](const Seg &a, const Seg &b) { return a.dst < b.dst; });
  bool disjoint = true;
  for (size_t i = 1; i < sorted.size() && disjoint; ++i)
    disjoint = sorted[i - 1].dst + sorted[i - 1].bytes <= sorted[i].dst;
  std::vector<Seg> merged;
  merged.reserve(segs.size());
  if (!disjoint) {
    for (const Seg &s : segs) push_merged(merged, s);
    for (const Seg &s : merged) submit_1d(s, kind, stream);
    return;
  }
  if (d2h)
    std::stable_sort(sorted.begin(), sorted.end(), [](const Seg &a, const Seg &b) { return a.src < b.src; });
  for (const Seg &s : sorted) push_merged(merged, s);

  // Rows over pinned, device-mapped host memory go to the copy kernel;
  // rows over pageable memory, and rows of kEngineRowBytes or more, to the
  // copy engines.
  std::vector<PinnedRange> seen;
  std::vector<Seg> kernel_rows;  // device-visible addresses on both sides
  std::vector<Seg> kernel_orig;  // the same rows as given
  std::vector<Seg> engine_rows;
  for (const Seg &s : merged) {
    const uint64_t h = d2h ? s.dst : s.src;
    const uint64_t dev = s.bytes < kEngineRowBytes ? mapped(h, s.bytes, seen) : 0;
    if (dev == 0) {
      engine_rows.push_back(s);
      continue;
    }
    kernel_rows.push_back(d2h ? Seg{dev, s.src, s.bytes} : Seg{s.dst, dev, s.bytes});
    kernel_orig.push_back(s);
  }
  // one row alone gains nothing from a launch over a copy-engine copy
  if (kernel_rows.size() == 1)
    engine_rows.push_back(kernel_orig[0]);
  else if (!kernel_rows.empty())
    launch_rows(kernel_rows, stream);
  if (engine_rows.empty()) return;

  const uint64_t max_pitch = device_max_pitch();
  // A run needs both pitches positive and at least one row long, so that
  // neither its destination rows nor its source rows overlap.  Runs shorter
  // than kMinRun rows cost the copy engines as much as their rows one by
  // one.
  auto pitch_ok = [&](const Seg &p, const Seg &q, uint64_t *dp, uint64_t *sp) {
    if (q.bytes != p.bytes || q.dst <= p.dst || q.src <= p.src) return false;
    *dp = q.dst - p.dst;
    *sp = q.src - p.src;
    return *dp >= p.bytes && *sp >= p.bytes && *dp <= max_pitch && *sp <= max_pitch;
  };
  size_t i = 0;
  while (i < engine_rows.size()) {
    uint64_t dp = 0, sp = 0, dq = 0, sq = 0;
    size_t j = i + 1;
    if (j < engine_rows.size() && pitch_ok(engine_rows[i], engine_rows[j], &dp, &sp)) {
      ++j;
      while (j < engine_rows.size() && pitch_ok(engine_rows[j - 1], engine_rows[j], &dq, &sq) && dq == dp &&
             sq == sp)
        ++j;
    }
    if (j - i >= kMinRun) {
      if (!submit_run(engine_rows, i, j - i, dp, sp, kind, stream))
        for (size_t k = i; k < j; ++k) submit_1d(engine_rows[k], kind, stream);
      i = j;
    } else {
      submit_1d(engine_rows[i], kind, stream);
      ++i;
    }
  }
}

void dma_copy_diagnose(const lmc_dma_segment *rows, int64_t n, bool d2h, hipStream_t stream, double *copy_us) {
  check_value(n >= 0 && (n == 0 || (rows != nullptr && copy_us != nullptr)), "copies is null");
  const hipMemcpyKind kind = d2h ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice;
  using Clock = std::chrono::steady_clock;
  for (int64_t i = 0; i < n; ++i) {
    const auto t0 = Clock::now();
    hipError_t e = hipMemcpyAsync(reinterpret_cast<void *>(rows[i].dst),
                                  reinterpret_cast<const void *>(rows[i].src), rows[i].bytes, kind, stream);
    copy_us[i] = std::chrono::duration<double, std::micro>(Clock::now() - t0).count();
    if (e != hipSuccess)
      fail(LMC_ERR_RUNTIME, std::string("diagnostic copies were not enqueued: status ") +
                                std::to_string(static_cast<int>(e)) + " segment=" + std::to_string(i) +
                                " bytes=" + std::to_string(rows[i].bytes));
  }
}

} // namespace
} // namespace lmc

using namespace lmc;

extern "C" {

int lmc_layerwise_prefill_dma_copy(const lmc_dma_segment *copies, int64_t n, int32_t device_to_host,
                                   void *stream) {
  return guarded([&] { dma_copy(copies, n, device_to_host != 0, static_cast<hipStream_t>(stream)); });
}

int lmc_layerwise_prefill_dma_copy_diagnose(const lmc_dma_segment *copies, int64_t n, int32_t device_to_host,
                                            void *stream, double *copy_us) {
  return guarded(
      [&] { dma_copy_diagnose(copies, n, device_to_host != 0, static_cast<hipStream_t>(stream), copy_us); });
}

} // extern "C"
