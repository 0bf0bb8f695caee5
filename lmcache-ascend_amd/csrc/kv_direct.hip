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
// widest plane row in VEC-byte accesses) owns one entry and copies its
// planes' rows one after the other.  Chunk addresses come from a device
// table, so alignment is checked per entry: a chunk base that is not
// VEC-aligned is copied bytewise.  Host chunks are read or written over
// PCIe, so those copies are PCIe-bound; flat device buffers are HBM-bound.
#include "kv_geom.h"

namespace lmc {

namespace {

constexpr int kEntThreads = 256;

enum EntryMode : int32_t {
  kDenseFixed = 0,
  kDenseVar = 1,
  kSparseChunked = 2,
  kSparseFlat = 3,
};

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
};

__device__ __forceinline__ int64_t load_index(const void *p, int is32,
                                              int64_t i) {
  return is32 ? static_cast<int64_t>(static_cast<const int32_t *>(p)[i])
              : static_cast<const int64_t *>(p)[i];
}

// Resolves entry e to its slot, the token index t inside its chunk, the
// chunk's token count and base; false when the entry is skipped.
__device__ __forceinline__ bool resolve(const EntryJob &job, int64_t e,
                                        int64_t &slot, int64_t &t,
                                        int64_t &nc, uint64_t &lbase) {
  if (job.mode == kDenseFixed || job.mode == kDenseVar) {
    slot = load_index(job.slots, job.slot_i32, e);
    int64_t c, start;
    if (job.mode == kDenseFixed) {
      c = e / job.chunk_size;
      start = c * job.chunk_size;
      nc = min(static_cast<int64_t>(job.chunk_size),
               static_cast<int64_t>(job.total_tokens) - start);
    } else {
      // Last chunk whose offset is <= e.
      if (job.chunk_offs[0] > e) return false;
      int lo = 0, hi = job.n_chunks - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (job.chunk_offs[mid] <= e) lo = mid;
        else hi = mid - 1;
      }
      c = lo;
      start = job.chunk_offs[c];
      nc = job.chunk_sizes[c];
    }
    if (c >= job.n_chunks || e >= start + nc) return false;
    t = e - start;
    lbase = static_cast<uint64_t>(job.chunk_ptrs[c]);
  } else {
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
  return slot >= 0 && slot < job.num_slots;
}

template <int VEC, bool NT>
__global__ void __launch_bounds__(kEntThreads) kv_entry_copy(EntryJob job) {
  using V = typename VecOf<VEC>::T;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kEntThreads + threadIdx.x;
  const int64_t e = gid >> job.group_shift;
  if (e >= job.n_entries) return;
  const int G = 1 << job.group_shift;
  const int gl = static_cast<int>(gid & (G - 1));
  int64_t slot, t, nc;
  uint64_t lbase;
  if (!resolve(job, e, slot, t, nc, lbase)) return;
  const bool aligned = (lbase & (VEC - 1)) == 0;
#pragma unroll
  for (int p = 0; p < kMaxPlanes; ++p) {
    if (p >= job.n_planes) break;
    const PlaneDesc &pd = job.plane[p];
    int64_t poff = pd.paged_off;
    if (job.block_size > 0)
      poff += (slot / job.block_size) * pd.blk_stride +
              (slot % job.block_size) * pd.row_pitch;
    else
      poff += slot * pd.row_pitch;
    uint8_t *paged = reinterpret_cast<uint8_t *>(job.base[p]) + poff;
    uint8_t *lm = reinterpret_cast<uint8_t *>(lbase) + pd.lmc_off_fixed +
                  pd.lmc_off_per_t * nc + t * pd.lmc_token_stride;
    uint8_t *dst = job.page2lmc ? lm : paged;
    const uint8_t *src = job.page2lmc ? paged : lm;
    if (aligned) {
      const int64_t nv = pd.row_bytes / VEC;
      for (int64_t v = gl; v < nv; v += G)
        st<V, NT>(reinterpret_cast<V *>(dst) + v,
                  ld<V, NT>(reinterpret_cast<const V *>(src) + v));
    } else {
      for (int64_t b = gl; b < pd.row_bytes; b += G) dst[b] = src[b];
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

// LMC side of host chunks of MLA/DSA formats: stacked planes
// [K: n_c*kH | V: n_c*vH | DSA: n_c*dsaH] or per-token [K | V | DSA] rows
// (csrc/utils.cpp:500-546; tools/cpu_vllm_runtime.py:299-338, 366-381).
void chunk_layout_mla(const LayerGeom &g, bool interleaved, EntryJob &job) {
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
  const int vec = vec_for(gv);
  const int64_t vecs = std::max<int64_t>(1, widest / vec);
  int shift = 0;
  while ((int64_t(1) << shift) < vecs && shift < 6) ++shift;
  job.group_shift = shift;
  const int64_t threads = job.n_entries << shift;
  const int64_t blocks = (threads + kEntThreads - 1) / kEntThreads;
  check(blocks < (int64_t(1) << 31), "too many entries in one call");
  const dim3 grid(static_cast<unsigned>(blocks)), block(kEntThreads);
  const bool nt = nontemporal_enabled() && !host_lmc;
#define LMC_ENTRY_LAUNCH(V)                                                  \
  if (nt) hipLaunchKernelGGL((kv_entry_copy<V, true>), grid, block, 0, stream, job); \
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

// csrc/utils.cpp:968-998, with the reference's messages.
void validate_sparse_inputs(const lmc_tensor &slots, const lmc_tensor &sel) {
  if ((slots.ndim != 1 && slots.ndim != 2) || slots.ndim != sel.ndim)
    fail(LMC_ERR_VALUE, "slot_mapping_packed and selected_token_idx must both "
                        "be 1D or both be 2D.");
  for (int i = 0; i < slots.ndim; ++i)
    if (slots.sizes[i] != sel.sizes[i])
      fail(LMC_ERR_VALUE, "slot_mapping_packed and selected_token_idx must "
                          "have the same length.");
  if (sel.dtype != LMC_I32)
    fail(LMC_ERR_VALUE, "selected_token_idx must be torch.int32.");
  if (sel.device < 0)
    fail(LMC_ERR_VALUE, "selected_token_idx must be on the GPU.");
}

void set_sparse_indices(EntryJob &job, const lmc_tensor &slots,
                        const lmc_tensor &sel) {
  check(numel(slots) == numel(sel),
        "slot_mapping_packed and selected_token_idx must have the same length.");
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
  check(x.dtype == LMC_I64, "chunk_ptrs_npu must be torch.int64.");
  check(x.device >= 0, "chunk_ptrs_npu must be on the GPU.");
  check(numel(x) > 0, "chunk_ptrs_npu must not be empty.");
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
  // csrc/mem_kernels.cpp:604-606, 734-739.
  check(chunk_size > 0, "chunk_size must be positive.");
  check(total_tokens > 0, "total_tokens must be positive.");
  check(chunk_size < (int64_t(1) << 31) && total_tokens < (int64_t(1) << 31),
        "chunk_size and total_tokens must fit int32");
  const lmc_tensor &ptrs = chunk_table(ptrs_t);
  DeviceGuard guard(g.device);
  EntryJob job = entry_job(g, false);
  job.mode = kSparseChunked;
  if (g.mla_dsa) {
    chunk_layout_mla(g, interleaved, job);
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
    // Count-aware rows (csrc/mem_kernels.cpp:641-649): selected tokens form
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

// csrc/mem_kernels.cpp:1061-1129, with the reference's messages.
void validate_dense_inputs(const lmc_tensor &slots, const lmc_tensor &ptrs,
                           const lmc_tensor &offs, const lmc_tensor &sizes,
                           int64_t total_tokens, int64_t fixed) {
  check(slots.ndim == 1, "slot_mapping_full must be 1D.");
  check(ptrs.ndim == 1, "chunk_ptrs_npu must be 1D.");
  check(offs.ndim == 1, "chunk_offsets_npu must be 1D.");
  check(sizes.ndim == 1, "chunk_sizes_npu must be 1D.");
  check(offs.dtype == LMC_I32, "chunk_offsets_npu must be torch.int32.");
  check(sizes.dtype == LMC_I32, "chunk_sizes_npu must be torch.int32.");
  if (fixed > 0)
    check(numel(offs) > 0 && numel(sizes) > 0,
          "fixed dense direct metadata tensors must not be empty.");
  else
    check(numel(ptrs) == numel(offs) && numel(ptrs) == numel(sizes),
          "chunk pointer, offset and size tensors must have the same length.");
  check(total_tokens > 0, "total_tokens must be positive.");
  check(fixed >= 0, "fixed_chunk_size must be non-negative.");
  check(slots.sizes[0] <= total_tokens,
        "slot_mapping_full length cannot exceed total_tokens.");
  if (fixed > 0) {
    const int64_t nc = numel(ptrs);
    check((nc - 1) * fixed < total_tokens && nc * fixed >= total_tokens,
          "fixed_chunk_size does not cover total_tokens.");
  }
  check(slots.device >= 0, "slot_mapping_full must be on the GPU.");
  check(offs.device >= 0, "chunk_offsets_npu must be on the GPU.");
  check(sizes.device >= 0, "chunk_sizes_npu must be on the GPU.");
}

void dense_direct(const lmc_tensor *ptrs_t, const lmc_tensor *caches, int n,
                  const lmc_tensor *slots_t, const lmc_tensor *offs_t,
                  const lmc_tensor *sizes_t, int64_t total_tokens,
                  int64_t fixed, int fmt, bool two_major, int64_t kH,
                  int64_t vH, int64_t dsaH, bool interleaved, bool page2lmc,
                  bool validate, hipStream_t stream) {
  check(is_mla_dsa(fmt), "Dense direct transfer only supports MLA/DSA formats.");
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &slots = index_tensor(slots_t, "slot_mapping_full");
  const lmc_tensor &ptrs = chunk_table(ptrs_t);
  const lmc_tensor &offs = index_tensor(offs_t, "chunk_offsets_npu");
  const lmc_tensor &sizes = index_tensor(sizes_t, "chunk_sizes_npu");
  if (validate) validate_dense_inputs(slots, ptrs, offs, sizes, total_tokens, fixed);
  // Checks every call keeps (the kernel's reads must stay in bounds).
  check(slots.ndim == 1, "slot_mapping_full must be 1D.");
  check(total_tokens > 0 && total_tokens < (int64_t(1) << 31) && fixed >= 0 &&
            fixed < (int64_t(1) << 31),
        "total_tokens and fixed_chunk_size must fit int32");
  check(slots.sizes[0] <= total_tokens,
        "slot_mapping_full length cannot exceed total_tokens.");
  if (fixed == 0)
    check(offs.dtype == LMC_I32 && sizes.dtype == LMC_I32 &&
              numel(offs) >= numel(ptrs) && numel(sizes) >= numel(ptrs),
          "chunk offset and size tables must be int32 with one entry per chunk");
  DeviceGuard guard(g.device);
  EntryJob job = entry_job(g, page2lmc);
  job.mode = fixed > 0 ? kDenseFixed : kDenseVar;
  chunk_layout_mla(g, interleaved, job);
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

// --- staged batched paths (csrc/mem_kernels.cpp:336-413, 1291-1339;
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
  uint8_t *host = kernel_ptr(obj);
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

void batched_fused(const lmc_tensor *objs, int n_objs, const lmc_tensor *staging_t,
                   const lmc_tensor *caches, int n, const lmc_tensor *slots_t,
                   const int64_t *offs, const int64_t *sizes, bool direction,
                   int fmt, bool token_major, bool two_major, int64_t kH,
                   int64_t vH, int64_t dsaH, hipStream_t stream) {
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &staging = deref(staging_t, "staging_cache");
  check(n_objs >= 0 && (n_objs == 0 || (objs && offs && sizes)), "bad chunk list");
  DeviceGuard guard(g.device);
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
