// Sparse and direct gather/scatter for MI355X (gfx950).
//
// Replaces the reference's sparse / multi-chunk ("direct") transfer family
// and its staged batched paths (csrc/mem_kernels.cpp:336-1339; kernel
// declarations csrc/mem_kernels.h:59-154; host planning csrc/utils.cpp:
// 408-998):
//
//   sparse_single_layer_kv_transfer            paged[slot[i]] = LMC[sel[i]]
//   sparse_mla_dsa_batched_direct_kv_transfer  the same from host chunks
//     (+ _fast, _prepared)                      (token -> chunk token/size)
//   dense_mla_dsa_batched_direct_kv_transfer   token g <-> chunk holding g,
//     (+ _fast, _prepared, group)               either direction
//   batched_fused_single_layer_kv_transfer     single-layer copy through a
//   batched_fused_sparse_single_layer_...      device staging buffer plus
//                                              per-chunk DMA copies
//
// One kernel serves the first three.  An entry is one token: a paged slot
// and a set of LMC rows.  Entry e resolves on the device to
//
//   dense   token g = e, slot = slot_mapping[g], chunk c holding g (fixed
//           chunk size, or the ascending chunk_offsets / chunk_sizes tables)
//   sparse  token = selected[e], slot = slot_mapping_packed[e]; chunk
//           token / chunk_size of a host-chunk table, or a flat LMC buffer
//
// and plane p's LMC row lies at
//
//   chunk_base + lmc_off_fixed[p] + lmc_off_per_t[p] * n_c
//              + t * lmc_token_stride[p]
//
// with t the token's index in its chunk and n_c the chunk's token count
// (stacked host chunks [K: n_c*kH | V: n_c*vH | DSA] put plane p at
// prefix_p * n_c; interleaved chunks hold per-token [K | V | DSA] rows).
// The semantics follow the reference's CPU restatement of these paths
// (tools/cpu_vllm_runtime.py:288-419): entries whose slot lies outside the
// cache, whose token lies outside [0, total_tokens), past its row's count
// or in no chunk, are skipped.
//
// Work mapping: a group of G lanes (a power of two, 1..64, covering the
// widest plane row in VEC-byte accesses; 16 lanes walking the row when it
// is read from host memory) owns one entry at a time and copies its
// planes' rows one after the other.  Chunk addresses come from a device
// table, so alignment is checked per entry: a chunk base that is not
// VEC-aligned is copied bytewise.  Host chunks are read or written over
// PCIe, so those copies are PCIe-bound; flat device buffers are HBM-bound.
#include "kv_geom.h"

namespace lmc {

namespace {

constexpr int kEntThreads = 256;
constexpr int kEntUnroll = 4;  // accesses per lane and plane in one pass
constexpr int kEntHostReadBlocks = 512;  // grid cap for reads of host memory

enum EntryMode : int32_t {
  kDenseFixed = 0,
  kDenseVar = 1,
  kSparseChunked = 2,
  kSparseFlat = 3,
  kDenseInline = 4,
};

constexpr int kInlineChunks = 64;  // chunk table entries carried in kernargs

struct EntryJob {
  PlaneDesc plane[kMaxPlanes];
  uint64_t base[kMaxPlanes];
  int32_t n_planes;
  int32_t block_size;          // 0: flat paged rows
  int64_t num_slots;           // valid slots are [0, num_slots)
  int32_t page2lmc;            // 1: paged -> LMC, 0: LMC -> paged
  int32_t mode;                // EntryMode
  const void *slots;
  const void *tokens;          // sparse: LMC token per entry
  int32_t slot_i32;
  int32_t tok_i32;
  const int64_t *chunk_ptrs;   // kernel-visible chunk addresses
  const int32_t *chunk_offs;   // dense, variable chunks (ascending)
  const int32_t *chunk_sizes;
  const int32_t *counts;       // sparse: valid entries per row, or null
  int32_t n_chunks;
  int32_t chunk_size;          // fixed chunk size (dense fixed, sparse)
  int32_t total_tokens;
  int32_t row_width;           // entries per counted row
  int32_t count_stride;        // elements between two rows' counts
  int32_t n_rows;
  uint64_t lmc_flat;           // sparse flat: LMC buffer
  int64_t lmc_tokens;          // tokens the flat buffer holds
  int64_t n_entries;
  int32_t group_shift;         // log2 of lanes per entry
  int32_t one_pass;            // every plane row fits one pass of the group
  // kDenseInline: entry e is token tok_base + e of slot_mapping; chunk c
  // covers tokens [inl_off[c], inl_off[c] + inl_size[c]) (ascending).
  int64_t tok_base;
  uint64_t inl_ptr[kInlineChunks];
  int32_t inl_off[kInlineChunks];
  int32_t inl_size[kInlineChunks];
  // Optional second destination (dense modes): token g's row of plane p is
  // also written at mirror + mirror_off[p] + g * mirror_stride[p].
  uint64_t mirror;
  int64_t mirror_off[kMaxPlanes];
  int64_t mirror_stride[kMaxPlanes];
};

__device__ __forceinline__ int64_t load_index(const void *p, int is32,
                                              int64_t i) {
  return is32 ? static_cast<int64_t>(static_cast<const int32_t *>(p)[i])
              : static_cast<const int64_t *>(p)[i];
}

// Resolves entry e to its slot, its token g in slot_mapping (dense modes),
// the token index t inside its chunk, the chunk's token count and base;
// false when the entry's token lies in no chunk (the slot is checked by the
// caller).
__device__ __forceinline__ bool resolve(const EntryJob &job, int64_t e,
                                        int64_t &slot, int64_t &g, int64_t &t,
                                        int64_t &nc, uint64_t &lbase) {
  if (job.mode == kDenseFixed || job.mode == kDenseVar || job.mode == kDenseInline) {
    g = job.tok_base + e;
    slot = load_index(job.slots, job.slot_i32, g);
    int64_t c, start;
    if (job.mode == kDenseFixed) {
      c = g / job.chunk_size;
      start = c * job.chunk_size;
      nc = min(static_cast<int64_t>(job.chunk_size),
               static_cast<int64_t>(job.total_tokens) - start);
    } else {
      // Last chunk whose offset is <= g.
      const int32_t *offs = job.mode == kDenseInline ? job.inl_off : job.chunk_offs;
      if (offs[0] > g) return false;
      int lo = 0, hi = job.n_chunks - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (offs[mid] <= g) lo = mid;
        else hi = mid - 1;
      }
      c = lo;
      start = offs[c];
      nc = job.mode == kDenseInline ? job.inl_size[c] : job.chunk_sizes[c];
    }
    if (c >= job.n_chunks || g >= start + nc) return false;
    t = g - start;
    lbase = job.mode == kDenseInline ? job.inl_ptr[c] : static_cast<uint64_t>(job.chunk_ptrs[c]);
  } else {
    g = e;
    if (job.counts != nullptr) {
      const int64_t r = e / job.row_width;
      if (r >= job.n_rows ||
          e - r * job.row_width >= job.counts[r * job.count_stride])
        return false;
    }
    const int64_t tok = load_index(job.tokens, job.tok_i32, e);
    slot = load_index(job.slots, job.slot_i32, e);
    if (job.mode == kSparseChunked) {
      if (tok < 0 || tok >= job.total_tokens) return false;
      const int64_t c = tok / job.chunk_size;
      if (c >= job.n_chunks) return false;
      t = tok - c * job.chunk_size;
      nc = min(static_cast<int64_t>(job.chunk_size),
               static_cast<int64_t>(job.total_tokens) - c * job.chunk_size);
      lbase = static_cast<uint64_t>(job.chunk_ptrs[c]);
    } else {
      if (tok < 0 || tok >= job.lmc_tokens) return false;
      t = tok;
      nc = 0;
      lbase = job.lmc_flat;
    }
  }
  return true;
}

// Moves entry e's rows; lane gl of the entry's group of G lanes.
template <int VEC, bool NT>
__device__ __forceinline__ void copy_entry(const EntryJob &job, int64_t e, int gl, int G) {
  using V = typename VecOf<VEC>::T;
  int64_t slot, g, t, nc;
  uint64_t lbase;
  if (!resolve(job, e, slot, g, t, nc, lbase)) return;
  // A skipped slot moves nothing, except with a mirror (the staging buffer
  // of the batched paths): the memory object row and the staging row are
  // then exchanged as the staged copies would (staging -> object when
  // storing, object -> staging when loading).
  const bool slot_ok = slot >= 0 && slot < job.num_slots;
  if (!slot_ok && !job.mirror) return;
  const bool third = job.mirror && slot_ok;
  uint8_t *src[kMaxPlanes], *dst[kMaxPlanes], *mir[kMaxPlanes];
#pragma unroll
  for (int p = 0; p < kMaxPlanes; ++p) {
    src[p] = dst[p] = mir[p] = nullptr;
    if (p >= job.n_planes) continue;
    const PlaneDesc &pd = job.plane[p];
    uint8_t *lm = reinterpret_cast<uint8_t *>(lbase) + pd.lmc_off_fixed +
                  pd.lmc_off_per_t * nc + t * pd.lmc_token_stride;
    uint8_t *m = job.mirror ? reinterpret_cast<uint8_t *>(job.mirror) + job.mirror_off[p] +
                                  g * job.mirror_stride[p]
                            : nullptr;
    uint8_t *other;
    if (slot_ok) {
      int64_t poff = pd.paged_off;
      if (job.block_size > 0)
        poff += (slot / job.block_size) * pd.blk_stride +
                (slot % job.block_size) * pd.row_pitch;
      else
        poff += slot * pd.row_pitch;
      other = reinterpret_cast<uint8_t *>(job.base[p]) + poff;
      mir[p] = m;
    } else {
      other = m;
    }
    dst[p] = job.page2lmc ? lm : other;
    src[p] = job.page2lmc ? other : lm;
  }
  if ((lbase & (VEC - 1)) != 0) {  // unaligned chunk base: bytewise
#pragma unroll
    for (int p = 0; p < kMaxPlanes; ++p) {
      if (p >= job.n_planes) continue;
      for (int64_t b = gl; b < job.plane[p].row_bytes; b += G) {
        const uint8_t x = src[p][b];
        dst[p][b] = x;
        if (third) mir[p][b] = x;
      }
    }
    return;
  }
  if (job.one_pass) {
    // Every plane's row fits kEntUnroll passes of the group: all loads,
    // then all stores.
    V x[kMaxPlanes][kEntUnroll];
#pragma unroll
    for (int p = 0; p < kMaxPlanes; ++p)
#pragma unroll
      for (int k = 0; k < kEntUnroll; ++k) {
        const int v = gl + k * G;
        if (p < job.n_planes && static_cast<int64_t>(v) * VEC < job.plane[p].row_bytes)
          x[p][k] = gload(reinterpret_cast<const V *>(src[p]) + v);
      }
#pragma unroll
    for (int p = 0; p < kMaxPlanes; ++p)
#pragma unroll
      for (int k = 0; k < kEntUnroll; ++k) {
        const int v = gl + k * G;
        if (p < job.n_planes && static_cast<int64_t>(v) * VEC < job.plane[p].row_bytes) {
          st<V, NT>(reinterpret_cast<V *>(dst[p]) + v, x[p][k]);
          if (third) st<V, NT>(reinterpret_cast<V *>(mir[p]) + v, x[p][k]);
        }
      }
    return;
  }
#pragma unroll
  for (int p = 0; p < kMaxPlanes; ++p) {
    if (p >= job.n_planes) continue;
    const int64_t nv = job.plane[p].row_bytes / VEC;
    for (int64_t v = gl; v < nv; v += G) {
      const V x = gload(reinterpret_cast<const V *>(src[p]) + v);
      st<V, NT>(reinterpret_cast<V *>(dst[p]) + v, x);
      if (third) st<V, NT>(reinterpret_cast<V *>(mir[p]) + v, x);
    }
  }
}

// A group of 2^group_shift lanes per entry; the groups stride over the
// entries when the grid is smaller than the entry count.
template <int VEC, bool NT>
__global__ void __launch_bounds__(kEntThreads) kv_entry_copy(EntryJob job) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kEntThreads + threadIdx.x;
  const int G = 1 << job.group_shift;
  const int gl = static_cast<int>(gid & (G - 1));
  const int64_t step = (static_cast<int64_t>(gridDim.x) * kEntThreads) >> job.group_shift;
  for (int64_t e = gid >> job.group_shift; e < job.n_entries; e += step)
    copy_entry<VEC, NT>(job, e, gl, G);
}

// Two entries per group for the flat sparse mode (kSparseFlat, one_pass, no
// mirror, the flat buffer in device memory).  Every index load of both
// entries is issued before any is used (indices clamped into their arrays),
// then both entries' row loads, then the stores: the dependent chain index
// -> row is paid once for two entries.  The checks are those of resolve()
// and copy_entry().  Measured on MI355X, 65536 MLA tokens (1024 + 128-byte
// rows) scattered from a device buffer: 29.6 us against 30.7 us with one
// entry per group.
// Row loads of these kernels are plain (no streaming hint): their rows are
// gathered at random, and the same scatter took 31.6-32.1 us (events)
// with streaming loads against 27.8-28.0 us without; the host-memory
// paths measure the same either way.  Stores keep st().
template <int VEC, bool NT>
__global__ void __launch_bounds__(kEntThreads) kv_entry_pair_copy(EntryJob job) {
  using V = typename VecOf<VEC>::T;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kEntThreads + threadIdx.x;
  const int G = 1 << job.group_shift;
  const int gl = static_cast<int>(gid & (G - 1));
  const int64_t e0 = (gid >> job.group_shift) * 2;
  if (e0 >= job.n_entries || (job.counts != nullptr && job.n_rows <= 0)) return;
  int64_t tok[2], slot[2];
  bool ok[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int64_t e = e0 + k < job.n_entries ? e0 + k : job.n_entries - 1;
    tok[k] = load_index(job.tokens, job.tok_i32, e);
    slot[k] = load_index(job.slots, job.slot_i32, e);
    ok[k] = e0 + k < job.n_entries;
    if (job.counts != nullptr) {
      const int64_t r = e / job.row_width;
      const int64_t rr = r < job.n_rows ? r : job.n_rows - 1;
      const int32_t cnt = job.counts[rr * job.count_stride];
      ok[k] = ok[k] && r < job.n_rows && e - r * job.row_width < cnt;
    }
  }
  int64_t t[2], nc[2];
  uint64_t lbase[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    ok[k] = ok[k] && slot[k] >= 0 && slot[k] < job.num_slots;
    ok[k] = ok[k] && tok[k] >= 0 && tok[k] < job.lmc_tokens;
    t[k] = tok[k];
    nc[k] = 0;
    lbase[k] = job.lmc_flat;
  }
  uint8_t *src[2][kMaxPlanes], *dst[2][kMaxPlanes];
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int p = 0; p < kMaxPlanes; ++p) {
      src[k][p] = dst[k][p] = nullptr;
      if (p >= job.n_planes) continue;
      const PlaneDesc &pd = job.plane[p];
      uint8_t *lm = reinterpret_cast<uint8_t *>(lbase[k]) + pd.lmc_off_fixed +
                    pd.lmc_off_per_t * nc[k] + t[k] * pd.lmc_token_stride;
      int64_t poff = pd.paged_off;
      if (job.block_size > 0)
        poff += (slot[k] / job.block_size) * pd.blk_stride + (slot[k] % job.block_size) * pd.row_pitch;
      else
        poff += slot[k] * pd.row_pitch;
      uint8_t *other = reinterpret_cast<uint8_t *>(job.base[p]) + poff;
      dst[k][p] = job.page2lmc ? lm : other;
      src[k][p] = job.page2lmc ? other : lm;
    }
  // A chunk base that is not VEC-aligned (a device value) moves bytewise.
  bool vec[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) vec[k] = (lbase[k] & (VEC - 1)) == 0;
  V x[2][kMaxPlanes][kEntUnroll];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (!(ok[k] && vec[k])) continue;
#pragma unroll
    for (int p = 0; p < kMaxPlanes; ++p)
#pragma unroll
      for (int u = 0; u < kEntUnroll; ++u) {
        const int v = gl + u * G;
        if (p < job.n_planes && static_cast<int64_t>(v) * VEC < job.plane[p].row_bytes)
          x[k][p][u] = gload(reinterpret_cast<const V *>(src[k][p]) + v);
      }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (!ok[k]) continue;
    if (vec[k]) {
#pragma unroll
      for (int p = 0; p < kMaxPlanes; ++p)
#pragma unroll
        for (int u = 0; u < kEntUnroll; ++u) {
          const int v = gl + u * G;
          if (p < job.n_planes && static_cast<int64_t>(v) * VEC < job.plane[p].row_bytes)
            st<V, NT>(reinterpret_cast<V *>(dst[k][p]) + v, x[k][p][u]);
        }
    } else {
#pragma unroll
      for (int p = 0; p < kMaxPlanes; ++p) {
        if (p >= job.n_planes) continue;
        for (int64_t b = gl; b < job.plane[p].row_bytes; b += G) dst[k][p][b] = src[k][p][b];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

EntryJob entry_job(const LayerGeom &g, bool page2lmc) {
  EntryJob job;
  std::memset(&job, 0, sizeof(job));
  job.n_planes = g.n_planes;
  job.block_size = g.block_size;
  job.num_slots = g.num_slots;
  job.page2lmc = page2lmc ? 1 : 0;
  for (int p = 0; p < g.n_planes; ++p) {
    job.plane[p] = g.plane[p];
    job.base[p] = g.base[p];
  }
  return job;
}

// LMC side of memory objects laid out by plane: stacked planes
// [K: n_c*kH | V: n_c*vH | DSA: n_c*dsaH] or per-token [K | V | DSA] rows
// (csrc/utils.cpp:500-546; tools/cpu_vllm_runtime.py:299-338, 366-381).
// For MERGED/SEPARATE (planes K, V of width W) these are the [2, n, W] and
// [n, 2, W] objects of the batched paths.
void chunk_layout(const LayerGeom &g, bool interleaved, EntryJob &job) {
  for (int p = 0; p < g.n_planes; ++p) {
    PlaneDesc &d = job.plane[p];
    if (interleaved) {
      d.lmc_off_fixed = g.prefix[p] * g.es;
      d.lmc_off_per_t = 0;
      d.lmc_token_stride = g.plane_elems * g.es;
    } else {
      d.lmc_off_fixed = 0;
      d.lmc_off_per_t = g.prefix[p] * g.es;
      d.lmc_token_stride = g.width[p] * g.es;
    }
  }
}

void launch_entries(EntryJob job, bool host_lmc, hipStream_t stream) {
  if (job.n_entries <= 0) return;
  int64_t gv = 16;
  int64_t widest = 0;
  for (int p = 0; p < job.n_planes; ++p) {
    const PlaneDesc &d = job.plane[p];
    for (int64_t v : {d.row_bytes, d.lmc_off_fixed, d.lmc_off_per_t, d.lmc_token_stride,
                      d.paged_off, d.blk_stride, d.row_pitch,
                      static_cast<int64_t>(job.base[p] & 0xff)})
      gv = gcd64(gv, v);
    widest = std::max(widest, d.row_bytes);
  }
  if (job.mode == kSparseFlat) gv = gcd64(gv, static_cast<int64_t>(job.lmc_flat & 0xff));
  if (job.mirror) {
    gv = gcd64(gv, static_cast<int64_t>(job.mirror & 0xff));
    for (int p = 0; p < job.n_planes; ++p)
      gv = gcd64(gcd64(gv, job.mirror_off[p]), job.mirror_stride[p]);
  }
  const int vec = vec_for(gv);
  const int64_t vecs = std::max<int64_t>(1, widest / vec);
  // Lanes per entry: enough for kEntUnroll accesses per lane to cover the
  // widest row (up to a wave), so a wave holds several entries and each
  // lane keeps several loads in flight.  Reads of host memory instead keep
  // one access per lane in flight, 16 lanes per entry walking the row, on
  // at most kEntHostReadBlocks blocks that stride over the entries: the
  // PCIe read path moves fewer bytes per second with more reads in flight.
  // Measured on MI355X (pinned objects; Llama layer 2 x 2 KiB rows / MLA
  // 1 KiB + 128 B rows, dense / 2048 sparse tokens): 55.0 / 55.5 / 46.0
  // GB/s, against 50.0 / 52.5 / 37.4 with a wave per row and 45 / 48 / 38
  // with four accesses per lane in flight.  Writes to host memory show no
  // such dependence.
  const bool host_read = host_lmc && !job.page2lmc;
  const int unroll = host_read ? 1 : kEntUnroll;
  const int max_shift = host_read ? 4 : 6;
  int shift = 0;
  while ((int64_t(unroll) << shift) < vecs && shift < max_shift) ++shift;
  job.group_shift = shift;
  job.one_pass = vecs <= (int64_t(unroll) << shift);
  // Flat sparse entries between device buffers go two per group.
  const bool pair = !host_lmc && job.one_pass && !job.mirror && job.mode == kSparseFlat;
  const int64_t threads = (pair ? (job.n_entries + 1) / 2 : job.n_entries) << shift;
  int64_t blocks = (threads + kEntThreads - 1) / kEntThreads;
  if (host_read) blocks = std::min<int64_t>(blocks, kEntHostReadBlocks);
  check(blocks < (int64_t(1) << 31), "too many entries in one call");
  const dim3 grid(static_cast<unsigned>(blocks)), block(kEntThreads);
  const bool nt = nontemporal_enabled() && !host_lmc;
#define LMC_ENTRY_LAUNCH(V)                                                  \
  if (pair && nt) hipLaunchKernelGGL((kv_entry_pair_copy<V, true>), grid, block, 0, stream, job); \
  else if (pair) hipLaunchKernelGGL((kv_entry_pair_copy<V, false>), grid, block, 0, stream, job); \
  else if (nt) hipLaunchKernelGGL((kv_entry_copy<V, true>), grid, block, 0, stream, job); \
  else hipLaunchKernelGGL((kv_entry_copy<V, false>), grid, block, 0, stream, job);
  switch (vec) {
  case 16: LMC_ENTRY_LAUNCH(16) break;
  case 8: LMC_ENTRY_LAUNCH(8) break;
  case 4: LMC_ENTRY_LAUNCH(4) break;
  case 2: LMC_ENTRY_LAUNCH(2) break;
  default: LMC_ENTRY_LAUNCH(1) break;
  }
#undef LMC_ENTRY_LAUNCH
  hip_check(hipGetLastError(), "kv_entry_copy launch");
}

const lmc_tensor &index_tensor(const lmc_tensor *t, const char *name) {
  const lmc_tensor &x = deref(t, name);
  check(x.dtype == LMC_I32 || x.dtype == LMC_I64,
        std::string(name) + " must be int32 or int64");
  int64_t expect = 1;
  for (int i = x.ndim - 1; i >= 0; --i) {
    check(x.sizes[i] <= 1 || x.strides[i] == expect,
          std::string(name) + " must be contiguous");
    expect *= x.sizes[i];
  }
  return x;
}

// The input conditions of csrc/utils.cpp:968-998 (messages in this library's
// words).
void validate_sparse_inputs(const lmc_tensor &slots, const lmc_tensor &sel) {
  if ((slots.ndim != 1 && slots.ndim != 2) || slots.ndim != sel.ndim)
    fail(LMC_ERR_VALUE, "slot_mapping_packed and selected_token_idx: one is 1-D "
                        "and the other 2-D, or neither is 1-D or 2-D");
  for (int i = 0; i < slots.ndim; ++i)
    if (slots.sizes[i] != sel.sizes[i])
      fail(LMC_ERR_VALUE, "slot_mapping_packed and selected_token_idx differ "
                          "in shape");
  if (sel.dtype != LMC_I32)
    fail(LMC_ERR_VALUE, "selected_token_idx holds int32 token indices");
  if (sel.device < 0)
    fail(LMC_ERR_VALUE, "selected_token_idx is not a GPU tensor");
}

void set_sparse_indices(EntryJob &job, const lmc_tensor &slots,
                        const lmc_tensor &sel) {
  check(numel(slots) == numel(sel),
        "slot_mapping_packed and selected_token_idx differ in length");
  job.slots = kernel_ptr(slots);
  job.slot_i32 = slots.dtype == LMC_I32;
  job.tokens = kernel_ptr(sel);
  job.tok_i32 = sel.dtype == LMC_I32;
  job.n_entries = numel(sel);
}

void sparse_single_layer(const lmc_tensor *lmc_t, const lmc_tensor *caches,
                         int n, const lmc_tensor *slots_t,
                         const lmc_tensor *sel_t, int fmt, bool token_major,
                         bool two_major, int64_t kH, int64_t vH, int64_t dsaH,
                         hipStream_t stream) {
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &lmc = deref(lmc_t, "lmc_key_value_cache");
  const lmc_tensor &slots = index_tensor(slots_t, "slot_mapping_packed");
  const lmc_tensor &sel = index_tensor(sel_t, "selected_token_idx");
  validate_sparse_inputs(slots, sel);
  DeviceGuard guard(g.device);
  EntryJob job = entry_job(g, false);
  job.mode = kSparseFlat;
  job.lmc_tokens = single_layer_lmc(g, lmc, token_major, job.plane);
  job.lmc_flat = reinterpret_cast<uint64_t>(kernel_ptr(lmc));
  set_sparse_indices(job, slots, sel);
  launch_entries(job, lmc.device < 0, stream);
}

const lmc_tensor &chunk_table(const lmc_tensor *t) {
  const lmc_tensor &x = deref(t, "chunk_ptrs_npu");
  check(x.dtype == LMC_I64, "chunk_ptrs_npu holds int64 addresses");
  check(x.device >= 0, "chunk_ptrs_npu is not a GPU tensor");
  check(numel(x) > 0, "chunk_ptrs_npu lists no chunk");
  check(x.ndim == 1 && (x.sizes[0] <= 1 || x.strides[0] == 1),
        "chunk_ptrs_npu must be a contiguous 1-D table");
  check(numel(x) < (int64_t(1) << 31), "too many chunks");
  return x;
}

void sparse_direct(const lmc_tensor *ptrs_t, const lmc_tensor *sample_t,
                   const lmc_tensor *caches, int n, const lmc_tensor *slots_t,
                   const lmc_tensor *sel_t, const lmc_tensor *counts_t,
                   int64_t chunk_size, int64_t total_tokens, int fmt,
                   bool token_major, bool two_major, int64_t kH, int64_t vH,
                   int64_t dsaH, bool interleaved, bool validate,
                   hipStream_t stream) {
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &slots = index_tensor(slots_t, "slot_mapping_packed");
  const lmc_tensor &sel = index_tensor(sel_t, "selected_token_idx");
  if (validate) validate_sparse_inputs(slots, sel);
  // csrc/mem_kernels.cpp:601-602, 692-693.
  check(chunk_size > 0, "chunk_size is not positive");
  check(total_tokens > 0, "total_tokens is not positive");
  check(chunk_size < (int64_t(1) << 31) && total_tokens < (int64_t(1) << 31),
        "chunk_size and total_tokens must fit int32");
  const lmc_tensor &ptrs = chunk_table(ptrs_t);
  DeviceGuard guard(g.device);
  EntryJob job = entry_job(g, false);
  job.mode = kSparseChunked;
  if (g.mla_dsa) {
    chunk_layout(g, interleaved, job);
  } else {
    check(sample_t != nullptr,
          "MERGED/SEPARATE direct transfer needs an LMC layout sample");
    single_layer_lmc(g, *sample_t, token_major, job.plane);
  }
  job.chunk_ptrs = reinterpret_cast<const int64_t *>(kernel_ptr(ptrs));
  job.n_chunks = static_cast<int32_t>(numel(ptrs));
  job.chunk_size = static_cast<int32_t>(chunk_size);
  job.total_tokens = static_cast<int32_t>(total_tokens);
  set_sparse_indices(job, slots, sel);
  if (job.n_entries == 0) return;
  if (counts_t != nullptr) {
    // Count-aware rows (csrc/mem_kernels.cpp:636-650): selected tokens form
    // rows of num_sparse / requests entries; row r holds counts[r] valid
    // entries, the rest is padding.
    const lmc_tensor &counts = deref(counts_t, "selected_token_counts");
    check(counts.dtype == LMC_I32, "selected_token_counts must be torch.int32.");
    check(counts.device >= 0, "selected_token_counts must be on the GPU.");
    const int64_t rows = numel(counts);
    check(rows > 0 && rows <= job.n_entries,
          "selected_token_counts needs between 1 and num_sparse rows");
    const int64_t cstride = counts.ndim > 0 ? counts.strides[0] : 1;
    check(cstride > 0 && cstride < (int64_t(1) << 31), "bad selected_token_counts stride");
    check((rows - 1) * cstride + 1 <= extent_bytes(counts) / 4,
          "selected_token_counts rows (numel) times stride(0) exceed the tensor");
    job.counts = reinterpret_cast<const int32_t *>(kernel_ptr(counts));
    job.n_rows = static_cast<int32_t>(rows);
    job.row_width = static_cast<int32_t>(job.n_entries / rows);
    job.count_stride = static_cast<int32_t>(cstride);
  }
  launch_entries(job, true, stream);
}

// The input conditions of csrc/mem_kernels.cpp:978-1034 (messages in this
// library's words).
void validate_dense_inputs(const lmc_tensor &slots, const lmc_tensor &ptrs,
                           const lmc_tensor &offs, const lmc_tensor &sizes,
                           int64_t total_tokens, int64_t fixed) {
  check(slots.ndim == 1, "slot_mapping_full is not a vector");
  check(ptrs.ndim == 1, "chunk_ptrs_npu is not a vector");
  check(offs.ndim == 1, "chunk_offsets_npu is not a vector");
  check(sizes.ndim == 1, "chunk_sizes_npu is not a vector");
  check(offs.dtype == LMC_I32, "chunk_offsets_npu holds int32 token offsets");
  check(sizes.dtype == LMC_I32, "chunk_sizes_npu holds int32 token counts");
  if (fixed > 0)
    check(numel(offs) > 0 && numel(sizes) > 0,
          "fixed-size dense direct chunks need chunk offset and size tensors with entries");
  else
    check(numel(ptrs) == numel(offs) && numel(ptrs) == numel(sizes),
          "chunk_ptrs_npu, chunk_offsets_npu and chunk_sizes_npu differ in length");
  check(total_tokens > 0, "total_tokens is not positive");
  check(fixed >= 0, "fixed_chunk_size is negative");
  check(slots.sizes[0] <= total_tokens,
        "slot_mapping_full is longer than total_tokens");
  if (fixed > 0) {
    const int64_t nc = numel(ptrs);
    check((nc - 1) * fixed < total_tokens && nc * fixed >= total_tokens,
          "the chunks of fixed_chunk_size tokens do not span total_tokens");
  }
  check(slots.device >= 0, "slot_mapping_full is not a GPU tensor");
  check(offs.device >= 0, "chunk_offsets_npu is not a GPU tensor");
  check(sizes.device >= 0, "chunk_sizes_npu is not a GPU tensor");
}

void dense_direct(const lmc_tensor *ptrs_t, const lmc_tensor *caches, int n,
                  const lmc_tensor *slots_t, const lmc_tensor *offs_t,
                  const lmc_tensor *sizes_t, int64_t total_tokens,
                  int64_t fixed, int fmt, bool two_major, int64_t kH,
                  int64_t vH, int64_t dsaH, bool interleaved, bool page2lmc,
                  bool validate, hipStream_t stream) {
  check(is_mla_dsa(fmt), "dense direct transfers move MLA/DSA formats (3-6) only");
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &slots = index_tensor(slots_t, "slot_mapping_full");
  const lmc_tensor &ptrs = chunk_table(ptrs_t);
  const lmc_tensor &offs = index_tensor(offs_t, "chunk_offsets_npu");
  const lmc_tensor &sizes = index_tensor(sizes_t, "chunk_sizes_npu");
  if (validate) validate_dense_inputs(slots, ptrs, offs, sizes, total_tokens, fixed);
  // Checks every call keeps (the kernel's reads must stay in bounds).
  check(slots.ndim == 1, "slot_mapping_full is not a vector");
  check(total_tokens > 0 && total_tokens < (int64_t(1) << 31) && fixed >= 0 &&
            fixed < (int64_t(1) << 31),
        "total_tokens and fixed_chunk_size must fit int32");
  check(slots.sizes[0] <= total_tokens,
        "slot_mapping_full is longer than total_tokens");
  if (fixed == 0)
    check(offs.dtype == LMC_I32 && sizes.dtype == LMC_I32 &&
              numel(offs) >= numel(ptrs) && numel(sizes) >= numel(ptrs),
          "chunk offset and size tables must be int32 with one entry per chunk");
  DeviceGuard guard(g.device);
  EntryJob job = entry_job(g, page2lmc);
  job.mode = fixed > 0 ? kDenseFixed : kDenseVar;
  chunk_layout(g, interleaved, job);
  job.slots = kernel_ptr(slots);
  job.slot_i32 = slots.dtype == LMC_I32;
  job.chunk_ptrs = reinterpret_cast<const int64_t *>(kernel_ptr(ptrs));
  job.n_chunks = static_cast<int32_t>(numel(ptrs));
  if (fixed == 0) {
    job.chunk_offs = reinterpret_cast<const int32_t *>(kernel_ptr(offs));
    job.chunk_sizes = reinterpret_cast<const int32_t *>(kernel_ptr(sizes));
  }
  job.chunk_size = static_cast<int32_t>(fixed);
  job.total_tokens = static_cast<int32_t>(total_tokens);
  job.n_entries = slots.sizes[0];
  launch_entries(job, true, stream);
}

// --- staged batched paths (csrc/mem_kernels.cpp:336-416, 1308-1339;
//     host copies csrc/utils.cpp:500-733) -----------------------------------

void copy_async(void *dst, const void *src, int64_t bytes, hipStream_t s) {
  if (bytes <= 0) return;
  hip_check(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDefault, s),
            "hipMemcpyAsync");
}

void copy_2d_async(void *dst, int64_t dpitch, const void *src, int64_t spitch,
                   int64_t width, int64_t rows, hipStream_t s) {
  if (width <= 0 || rows <= 0) return;
  hip_check(hipMemcpy2DAsync(dst, static_cast<size_t>(dpitch), src,
                             static_cast<size_t>(spitch), static_cast<size_t>(width),
                             static_cast<size_t>(rows), hipMemcpyDefault, s),
            "hipMemcpy2DAsync");
}

// Moves chunk i's tokens between the staging buffer (tokens
// [off, off + n)) and its memory object.  Staging has the single-layer
// layout `sp` (planes of `g`); memory objects are
//   MLA/DSA:      stacked planes per chunk, or per-token [K|V|DSA] rows
//                 (token_major)
//   MERGED/SEP.:  [n, 2, W] (token_major: one contiguous range) or
//                 [2, n, W] (K range, then V range at the object's stride 0)
void stage_chunk(const LayerGeom &g, const PlaneDesc *sp, uint8_t *staging,
                 const lmc_tensor &obj, int64_t off, int64_t n,
                 bool token_major, bool to_host, hipStream_t s) {
  // DMA copies take the object's own address (pinned or pageable host
  // memory, or device memory).
  uint8_t *host = static_cast<uint8_t *>(obj.data);
  check(host != nullptr || obj.ndim == 0, "memory object has no storage");
  const int64_t es = g.es;
  check(elem_size(obj) == es, "memory object and cache dtypes differ");
  auto move = [&](uint8_t *stg, uint8_t *obj_p, int64_t bytes) {
    if (to_host) copy_async(obj_p, stg, bytes, s);
    else copy_async(stg, obj_p, bytes, s);
  };
  if (g.mla_dsa) {
    check(extent_bytes(obj) >= n * g.plane_elems * es,
          "memory object is smaller than its chunk");
    for (int p = 0; p < g.n_planes; ++p) {
      const int64_t rb = g.width[p] * es;
      uint8_t *stg = staging + sp[p].lmc_off_fixed + off * rb;
      if (token_major) {
        uint8_t *o = host + g.prefix[p] * es;
        const int64_t opitch = g.plane_elems * es;
        if (to_host) copy_2d_async(o, opitch, stg, rb, rb, n, s);
        else copy_2d_async(stg, rb, o, opitch, rb, n, s);
      } else {
        move(stg, host + g.prefix[p] * n * es, n * rb);
      }
    }
    return;
  }
  const int64_t tok = sp[0].lmc_token_stride;  // bytes per staging token
  if (token_major) {
    check(extent_bytes(obj) >= n * tok, "memory object is smaller than its chunk");
    move(staging + off * tok, host, n * tok);
    return;
  }
  check(obj.ndim >= 2, "memory object must be [2, tokens, W]");
  const int64_t voff = stride(obj, 0) * es;
  check(extent_bytes(obj) >= voff + n * tok, "memory object is smaller than its chunk");
  move(staging + off * tok, host, n * tok);
  move(staging + sp[1].lmc_off_fixed + off * tok, host + voff, n * tok);
}

void stage_chunks(const LayerGeom &g, const lmc_tensor &staging,
                  const lmc_tensor *objs, int n_objs, const int64_t *offs,
                  const int64_t *sizes, bool token_major, bool to_host,
                  hipStream_t s) {
  PlaneDesc sp[kMaxPlanes];
  std::memcpy(sp, g.plane, sizeof(sp));
  const int64_t cap = single_layer_lmc(g, staging, token_major, sp);
  check(staging.device >= 0, "staging_cache must be on the GPU");
  uint8_t *stg = kernel_ptr(staging);
  for (int i = 0; i < n_objs; ++i) {
    check(offs[i] >= 0 && sizes[i] >= 0 && offs[i] + sizes[i] <= cap,
          "chunk " + std::to_string(i) + " lies outside the staging buffer");
    stage_chunk(g, sp, stg, objs[i], offs[i], sizes[i], token_major, to_host, s);
  }
}

// The batched path in one pass: when the memory objects are kernel-visible,
// their chunks cover the staging tokens [0, T) in order and each object has
// the layout the staged copies assume, every token's rows move between the
// paged cache and its object by the entry kernel, which also writes them to
// the staging buffer (the staging content the two-step path leaves, so the
// results are the same bytes).  Returns false when the call does not
// qualify; the caller then runs the two steps.
bool batched_direct(const LayerGeom &g, const lmc_tensor &staging,
                    const lmc_tensor *objs, int n_objs, const int64_t *offs,
                    const int64_t *sizes, const lmc_tensor *slots_t,
                    bool direction, bool token_major, hipStream_t stream) {
  const lmc_tensor &slots = slots_of(slots_t);
  const int64_t T = slots.sizes[0];
  if (n_objs <= 0 || T <= 0 || T >= (int64_t(1) << 31) || staging.device < 0) return false;
  PlaneDesc sp[kMaxPlanes];
  std::memcpy(sp, g.plane, sizeof(sp));
  if (elem_size(staging) != g.es || single_layer_lmc(g, staging, token_major, sp) < T) return false;
  const int64_t W = g.width[0];
  std::vector<uint64_t> ptrs(n_objs);
  bool host = false;
  for (int i = 0; i < n_objs; ++i) {
    const int64_t n = sizes[i];
    if (n <= 0 || offs[i] != (i == 0 ? 0 : offs[i - 1] + sizes[i - 1])) return false;
    const lmc_tensor &o = objs[i];
    if (elem_size(o) != g.es) return false;
    int64_t need = n * g.plane_elems * g.es;
    if (!g.mla_dsa && !token_major)
      if (o.ndim < 2 || stride(o, 0) != n * W) return false;
    if (extent_bytes(o) < need) return false;
    if (o.device >= 0) {
      ptrs[i] = reinterpret_cast<uint64_t>(o.data);
    } else {
      ptrs[i] = translate_host_ptr(reinterpret_cast<uintptr_t>(o.data),
                                   static_cast<size_t>(need));
      if (ptrs[i] == 0) return false;
      host = true;
    }
  }
  if (offs[n_objs - 1] + sizes[n_objs - 1] != T) return false;
  EntryJob job = entry_job(g, direction);
  job.mode = kDenseInline;
  chunk_layout(g, token_major, job);
  job.slots = kernel_ptr(slots);
  job.slot_i32 = slots.dtype == LMC_I32;
  job.mirror = reinterpret_cast<uint64_t>(kernel_ptr(staging));
  for (int p = 0; p < g.n_planes; ++p) {
    job.mirror_off[p] = sp[p].lmc_off_fixed;
    job.mirror_stride[p] = sp[p].lmc_token_stride;
  }
  for (int c0 = 0; c0 < n_objs; c0 += kInlineChunks) {
    const int nc = std::min(kInlineChunks, n_objs - c0);
    EntryJob j = job;
    j.n_chunks = nc;
    for (int i = 0; i < nc; ++i) {
      j.inl_ptr[i] = ptrs[c0 + i];
      j.inl_off[i] = static_cast<int32_t>(offs[c0 + i]);
      j.inl_size[i] = static_cast<int32_t>(sizes[c0 + i]);
    }
    j.tok_base = offs[c0];
    j.n_entries = offs[c0 + nc - 1] + sizes[c0 + nc - 1] - offs[c0];
    launch_entries(j, host, stream);
  }
  return true;
}

void batched_fused(const lmc_tensor *objs, int n_objs, const lmc_tensor *staging_t,
                   const lmc_tensor *caches, int n, const lmc_tensor *slots_t,
                   const int64_t *offs, const int64_t *sizes, bool direction,
                   int fmt, bool token_major, bool two_major, int64_t kH,
                   int64_t vH, int64_t dsaH, hipStream_t stream) {
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &staging = deref(staging_t, "staging_cache");
  check(n_objs >= 0 && (n_objs == 0 || (objs && offs && sizes)), "bad chunk list");
  DeviceGuard guard(g.device);
  if (batched_direct(g, staging, objs, n_objs, offs, sizes, slots_t, direction,
                     token_major, stream))
    return;
  if (direction) {
    single_layer(staging_t, caches, n, slots_t, true, fmt, token_major, two_major,
                 kH, vH, dsaH, stream);
    stage_chunks(g, staging, objs, n_objs, offs, sizes, token_major, true, stream);
  } else {
    stage_chunks(g, staging, objs, n_objs, offs, sizes, token_major, false, stream);
    single_layer(staging_t, caches, n, slots_t, false, fmt, token_major, two_major,
                 kH, vH, dsaH, stream);
  }
}

void batched_fused_sparse(const lmc_tensor *objs, int n_objs,
                          const lmc_tensor *staging_t, const lmc_tensor *caches,
                          int n, const lmc_tensor *slots_t, const lmc_tensor *sel_t,
                          const int64_t *offs, const int64_t *sizes, int fmt,
                          bool token_major, bool two_major, int64_t kH,
                          int64_t vH, int64_t dsaH, hipStream_t stream) {
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &staging = deref(staging_t, "staging_cache");
  validate_sparse_inputs(index_tensor(slots_t, "slot_mapping_packed"),
                         index_tensor(sel_t, "selected_token_idx"));
  check(n_objs >= 0 && (n_objs == 0 || (objs && offs && sizes)), "bad chunk list");
  DeviceGuard guard(g.device);
  // Every chunk is staged whole (the reference stages only the selected
  // tokens when fewer than 3/4 are selected, csrc/utils.cpp:760-772); the
  // paged result is the same, as only selected tokens are read back.
  stage_chunks(g, staging, objs, n_objs, offs, sizes, token_major, false, stream);
  sparse_single_layer(staging_t, caches, n, slots_t, sel_t, fmt, token_major,
                      two_major, kH, vH, dsaH, stream);
}

} // namespace
} // namespace lmc

using namespace lmc;

extern "C" {

int lmc_sparse_single_layer_kv_transfer(
    const lmc_tensor *lmc_key_value_cache, const lmc_tensor *vllm_kv_caches,
    int32_t n_caches, const lmc_tensor *slot_mapping_packed,
    const lmc_tensor *selected_token_idx, int32_t kvcache_format,
    int32_t token_major, int32_t vllm_two_major, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream) {
  return guarded([&] {
    sparse_single_layer(lmc_key_value_cache, vllm_kv_caches, n_caches,
                        slot_mapping_packed, selected_token_idx, kvcache_format,
                        token_major != 0, vllm_two_major != 0, k_hidden_dims,
                        v_hidden_dims, dsa_hidden_dims, static_cast<hipStream_t>(stream));
  });
}

int lmc_sparse_direct_kv_transfer(
    const lmc_tensor *chunk_ptrs, const lmc_tensor *lmc_layout_sample,
    const lmc_tensor *vllm_kv_caches, int32_t n_caches,
    const lmc_tensor *slot_mapping_packed, const lmc_tensor *selected_token_idx,
    const lmc_tensor *selected_token_counts, int64_t chunk_size,
    int64_t total_tokens, int32_t kvcache_format, int32_t token_major,
    int32_t vllm_two_major, int64_t k_hidden_dims, int64_t v_hidden_dims,
    int64_t dsa_hidden_dims, int32_t lmc_host_interleaved,
    int32_t validate_inputs, void *stream) {
  return guarded([&] {
    sparse_direct(chunk_ptrs, lmc_layout_sample, vllm_kv_caches, n_caches,
                  slot_mapping_packed, selected_token_idx, selected_token_counts,
                  chunk_size, total_tokens, kvcache_format, token_major != 0,
                  vllm_two_major != 0, k_hidden_dims, v_hidden_dims,
                  dsa_hidden_dims, lmc_host_interleaved != 0, validate_inputs != 0,
                  static_cast<hipStream_t>(stream));
  });
}

int lmc_dense_direct_kv_transfer(
    const lmc_tensor *chunk_ptrs, const lmc_tensor *vllm_kv_caches,
    int32_t n_caches, const lmc_tensor *slot_mapping_full,
    const lmc_tensor *chunk_offsets, const lmc_tensor *chunk_sizes,
    int64_t total_tokens, int64_t fixed_chunk_size, int32_t kvcache_format,
    int32_t vllm_two_major, int64_t k_hidden_dims, int64_t v_hidden_dims,
    int64_t dsa_hidden_dims, int32_t lmc_host_interleaved, int32_t direction,
    int32_t validate_inputs, void *stream) {
  return guarded([&] {
    dense_direct(chunk_ptrs, vllm_kv_caches, n_caches, slot_mapping_full,
                 chunk_offsets, chunk_sizes, total_tokens, fixed_chunk_size,
                 kvcache_format, vllm_two_major != 0, k_hidden_dims, v_hidden_dims,
                 dsa_hidden_dims, lmc_host_interleaved != 0, direction != 0,
                 validate_inputs != 0, static_cast<hipStream_t>(stream));
  });
}

int lmc_batched_fused_single_layer_kv_transfer(
    const lmc_tensor *lmc_tensors, int32_t n_chunks, const lmc_tensor *staging_cache,
    const lmc_tensor *vllm_kv_caches, int32_t n_caches,
    const lmc_tensor *slot_mapping_full, const int64_t *chunk_offsets,
    const int64_t *chunk_sizes, int32_t direction, int32_t kvcache_format,
    int32_t token_major, int32_t vllm_two_major, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream) {
  return guarded([&] {
    batched_fused(lmc_tensors, n_chunks, staging_cache, vllm_kv_caches, n_caches,
                  slot_mapping_full, chunk_offsets, chunk_sizes, direction != 0,
                  kvcache_format, token_major != 0, vllm_two_major != 0,
                  k_hidden_dims, v_hidden_dims, dsa_hidden_dims,
                  static_cast<hipStream_t>(stream));
  });
}

int lmc_batched_fused_sparse_single_layer_kv_transfer(
    const lmc_tensor *lmc_tensors, int32_t n_chunks, const lmc_tensor *staging_cache,
    const lmc_tensor *vllm_kv_caches, int32_t n_caches,
    const lmc_tensor *slot_mapping_packed, const lmc_tensor *selected_token_idx,
    const int64_t *chunk_offsets, const int64_t *chunk_sizes,
    int32_t kvcache_format, int32_t token_major, int32_t vllm_two_major,
    int64_t k_hidden_dims, int64_t v_hidden_dims, int64_t dsa_hidden_dims,
    void *stream) {
  return guarded([&] {
    batched_fused_sparse(lmc_tensors, n_chunks, staging_cache, vllm_kv_caches,
                         n_caches, slot_mapping_packed, selected_token_idx,
                         chunk_offsets, chunk_sizes, kvcache_format, token_major != 0,
                         vllm_two_major != 0, k_hidden_dims, v_hidden_dims,
                         dsa_hidden_dims, static_cast<hipStream_t>(stream));
  });
}

int lmc_check_kv_caches(const lmc_tensor *vllm_kv_caches, int32_t n_caches,
                        int32_t kvcache_format, int32_t vllm_two_major,
                        int64_t k_hidden_dims, int64_t v_hidden_dims,
                        int64_t dsa_hidden_dims) {
  return guarded([&] {
    layer_geom(vllm_kv_caches, n_caches, kvcache_format, vllm_two_major != 0,
               k_hidden_dims, v_hidden_dims, dsa_hidden_dims);
  });
}

} // extern "C"
