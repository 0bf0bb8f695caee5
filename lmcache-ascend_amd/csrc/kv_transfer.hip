// Paged-KV gather / scatter for MI355X (gfx950).
//
// One kernel family serves every gather/scatter entry point of the
// reference's c_ops surface: multi_layer_kv_transfer (and its batched and
// staged "fused" forms), single_layer_kv_transfer, load_and_reshape_flash and
// reshape_and_cache_back_flash.  Each of them is a pure byte copy of rows:
// for every (plane p, layer l, token t) with s = slot_mapping[t],
//
//     LMC row (p, l, t)  <->  paged row (l, p, s)
//
// (reference docstring csrc/mem_kernels.cpp:54-74).  The host planner below
// turns a call's tensors into a CopyJob: per plane, the byte geometry of the
// LMCache side (plane / layer / token strides) and of the paged side (base
// pointer, block stride, row pitch).  The planner follows the reference's
// layout derivation (csrc/utils.cpp:29-86 for the multi-layer formats,
// csrc/utils.cpp:212-406 for the single-layer strides); the device side is
// written for CDNA4 rather than following the AscendC UB tiling:
//
//  * one wavefront owns a whole row, so the row index, the slot lookup and
//    all address arithmetic are wave-uniform scalar work;
//  * the 64 lanes move the row with 16-byte accesses (1 KiB per wave
//    instruction); each wave keeps ROWS_PER_WAVE rows x SEGS accesses in
//    flight per lane before the first store;
//  * grid.y enumerates LMCache chunks (memory objects), so a whole batch of
//    chunks is one launch; grid.x strides over rows.
//
// Slots outside [0, num_slots) are skipped: no read and no write.  The
// reference states that -1 never reaches its kernels
// (lmcache_ascend/v1/npu_connector/npu_connectors.py:1106-1112) while its
// in-tree kernels and CPU substitutes skip negative slots
// (csrc/graph/sparse_graph_kernel.cpp:45-48, tools/cpu_vllm_runtime.py:
// 379-380); skipping is the superset.
#include "kv_geom.h"
#include "kv_fused.h"

namespace lmc {

// Launch geometry (compile-time; the defaults are the measured best on
// MI355X for 2 KiB rows).
#ifndef LMC_KV_THREADS
#define LMC_KV_THREADS 256        // threads per block
#endif
#ifndef LMC_KV_ROWS_PER_WAVE
#define LMC_KV_ROWS_PER_WAVE 1    // work items a wave moves per pass
#endif
#ifndef LMC_KV_SEGS
#define LMC_KV_SEGS 2             // 64-lane accesses per work item
#endif
#ifndef LMC_KV_XCD_REMAP
#define LMC_KV_XCD_REMAP 0        // give each XCD a contiguous block range
#endif
#ifndef LMC_KV_LEAN
#define LMC_KV_LEAN 1             // lean row kernel for its geometry
#endif
#ifndef LMC_KV_LEAN_MAX_ROWS
#define LMC_KV_LEAN_MAX_ROWS 32768
#endif
#ifndef LMC_KV_LEAN_BATCH
#define LMC_KV_LEAN_BATCH 0       // lean kernel for multi-object launches too
#endif
#ifndef LMC_KV_GRID_CAP
#define LMC_KV_GRID_CAP 65535     // blocks per chunk (grid-stride beyond)
#endif

constexpr int kMaxChunks = 64;
constexpr int kThreads = LMC_KV_THREADS;
constexpr int kWaves = kThreads / 64;
constexpr int kRowsPerWave = LMC_KV_ROWS_PER_WAVE;
constexpr int kSegs = LMC_KV_SEGS;

struct CopyJob {
  PlaneDesc plane[kMaxPlanes];
  uint64_t base[kMaxPlanes];   // paged base per plane when table == nullptr
  const uint64_t *table;       // per-layer pointer table (multi-layer ops)
  int32_t table_ppl;           // pointers per layer in `table`
  int32_t table_idx[kMaxPlanes];
  const void *slots;           // slot_mapping (already offset to token 0)
  int32_t slot_i32;
  int32_t n_planes;
  int32_t n_layers;
  int32_t block_size;          // 0: flat rows
  int64_t num_slots;           // valid slots are [0, num_slots)
  int32_t page2lmc;            // 1: paged -> LMC (store), 0: LMC -> paged
  int32_t slices_per_row;      // work items per row (widest plane)
  int32_t bs_shift;            // log2(block_size) for the lean kernel
  int32_t spr_shift;           // log2(slices_per_row) for the lean kernel
  int32_t idx_step;            // lean kernel: table_idx[p] == p * idx_step
};

// The chunks of one launch.  A launch over one chunk (the per-object call the
// connector makes) takes the one-entry form, so its kernel arguments stay
// small.
template <int NC> struct ChunkListT {
  uint64_t lmc[NC];               // kernel-visible LMC chunk address
  int32_t tok_start[NC];          // chunk c: slot_mapping[start, start+count)
  int32_t tok_count[NC];
};
using ChunkList = ChunkListT<kMaxChunks>;


// Resolves row `row` of chunk `c` to (src, dst); returns the row's byte count,
// or 0 when the slot is skipped.  All inputs are wave-uniform.
template <bool SLOT32, bool TABLE>
__device__ __forceinline__ int64_t row_ptrs(const CopyJob &job, uint8_t *lmc,
                                            int tok0, int T, int per_plane,
                                            int row, const uint8_t *&src,
                                            uint8_t *&dst) {
  const int p = row / per_plane;
  const int rem = row - p * per_plane;
  const int l = rem / T;
  const int t = rem - l * T;
  // Independent loads, issued together: the slot and the plane's paged base
  // (the empty asm takes both as scalar operands, so one wait covers both
  // and the range check does not sit between them).
  const int64_t slot = SLOT32 ? static_cast<int64_t>(static_cast<const int32_t *>(job.slots)[tok0 + t])
                              : static_cast<const int64_t *>(job.slots)[tok0 + t];
  const uint64_t pbase =
      TABLE ? job.table[static_cast<int64_t>(l) * job.table_ppl + job.table_idx[p]] : job.base[p];
  asm volatile("" ::"s"(slot), "s"(pbase));
  if (slot < 0 || slot >= job.num_slots) return 0;
  const PlaneDesc &pd = job.plane[p];
  int64_t poff = pd.paged_off;
  if (job.block_size > 0) {
    const uint32_t s32 = static_cast<uint32_t>(slot);
    const uint32_t bs = static_cast<uint32_t>(job.block_size);
    const uint32_t blk = s32 / bs;
    poff += static_cast<int64_t>(blk) * pd.blk_stride +
            static_cast<int64_t>(s32 - blk * bs) * pd.row_pitch;
  } else {
    poff += slot * pd.row_pitch;
  }
  uint8_t *paged = reinterpret_cast<uint8_t *>(pbase) + poff;
  uint8_t *lm = lmc + pd.lmc_off_fixed + pd.lmc_off_per_t * T +
                static_cast<int64_t>(l) *
                    (pd.lmc_layer_fixed + pd.lmc_layer_per_t * T) +
                static_cast<int64_t>(t) * pd.lmc_token_stride;
  if (job.page2lmc) {
    src = paged;
    dst = lm;
  } else {
    src = lm;
    dst = paged;
  }
  return pd.row_bytes;
}

// One work item is a slice of one row: kSegs 64-lane accesses of VEC bytes
// (2 KiB with 16-byte accesses, a whole row at the Llama-3-8B shape).  A
// wave owns kRowsPerWave items per pass: it resolves their addresses with
// scalar work, issues every load, then every store.
template <int VEC, bool NT, int NC, bool SLOT32, bool TABLE>
__global__ void __launch_bounds__(kThreads)
    kv_rows_copy(const CopyJob job, const ChunkListT<NC> chunks) {
  using V = typename VecOf<VEC>::T;
  constexpr int kSlice = 64 * VEC * kSegs;
  const int c = blockIdx.y;
  const int tok0 = chunks.tok_start[c];
  const int T = chunks.tok_count[c];
  const int per_plane = job.n_layers * T;
  const int spr = job.slices_per_row;
  const int items = job.n_planes * per_plane * spr;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t *lmc = reinterpret_cast<uint8_t *>(chunks.lmc[c]);
  int bx = blockIdx.x;
#if LMC_KV_XCD_REMAP
  // Blocks are dispatched round-robin over the 8 XCDs; map each XCD's
  // blocks onto one contiguous range of work.
  if ((gridDim.x & 7) == 0) bx = (bx & 7) * (gridDim.x >> 3) + (bx >> 3);
#endif
  const int step = gridDim.x * kWaves * kRowsPerWave;

  for (int i0 = (bx * kWaves + wave) * kRowsPerWave; i0 < items; i0 += step) {
    const uint8_t *src[kRowsPerWave];
    uint8_t *dst[kRowsPerWave];
    int64_t nb[kRowsPerWave], off0[kRowsPerWave];
    bool slow = false;
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
      nb[r] = 0;
      off0[r] = 0;
      src[r] = nullptr;
      dst[r] = nullptr;
      const int item = i0 + r;
      if (item < items) {
        const int row = item / spr;
        off0[r] = static_cast<int64_t>(item - row * spr) * kSlice;
        nb[r] = row_ptrs<SLOT32, TABLE>(job, lmc, tok0, T, per_plane, row, src[r], dst[r]);
      }
      // The host checked every alignment it can see; a table entry (a device
      // value) that is not VEC-aligned sends the item to the byte path.
      if (nb[r] > off0[r] &&
          ((reinterpret_cast<uintptr_t>(src[r]) |
            reinterpret_cast<uintptr_t>(dst[r])) &
           (VEC - 1)) != 0) {
        slow = true;
      }
    }
    if (slow) {
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) {
        const int64_t end = nb[r] < off0[r] + kSlice ? nb[r] : off0[r] + kSlice;
        for (int64_t o = off0[r] + lane; o < end; o += 64) dst[r][o] = src[r][o];
      }
      continue;
    }
    V v[kRowsPerWave][kSegs];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int s = 0; s < kSegs; ++s) {
        const int64_t o = off0[r] + (s * 64 + lane) * VEC;
        if (o < nb[r]) v[r][s] = ld<V, NT>(reinterpret_cast<const V *>(src[r] + o));
      }
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int s = 0; s < kSegs; ++s) {
        const int64_t o = off0[r] + (s * 64 + lane) * VEC;
        if (o < nb[r]) st<V, NT, false>(reinterpret_cast<V *>(dst[r] + o), v[r][s]);
      }
  }
}

// Lean row kernel, for the common geometry: every plane's row is the same
// power-of-two number of 2 KiB slices, the block size (when rows are block
// strided) is a power of two, and plane p's pointer-table entry of layer l is
// l * ppl + p * idx_step.  A wave owns kR consecutive slices of one (plane,
// layer) (consecutive slices of a row, or the slices of consecutive tokens);
// the grid is (slice groups, plane x layer, chunk).  Everything the
// wave reads from its kernel arguments is at a fixed offset (all planes'
// descriptors are read and one is selected), so one wait covers them; the
// slot and the pointer-table entry are then loaded together, and the row
// loads follow.  The dependent chain of a wave is kernel arguments -> {slot,
// table entry} -> row loads -> row stores, which is what a launch over one
// 256-token chunk (the connector's per-object call) pays on its first and
// last waves.  Chunks of a launch hold at least one token (the host drops
// empty ones).
// Slices per wave: one for pointer-table launches (per-object calls), two
// for flat per-layer launches (flash calls), whose 8192-row grids lose less
// to dispatch with half the workgroups.  Measured on MI355X, 8B shape, three
// interleaved runs: 16 per-object calls 0.215 ms with one slice per wave,
// 0.224 with two, 0.232 with four; 32 flash calls (store / retrieve) 0.264 /
// 0.255 ms with one, 0.259 / 0.243 with two, 0.281 / 0.267 with four.
#ifndef LMC_KV_LEAN_R
#define LMC_KV_LEAN_R 1
#endif
#ifndef LMC_KV_LEAN_R_FLAT
#define LMC_KV_LEAN_R_FLAT 2
#endif
constexpr int kLeanR = LMC_KV_LEAN_R;
constexpr int kLeanRFlat = LMC_KV_LEAN_R_FLAT;

template <bool NT, int NC, bool TABLE, int NP, bool SLOT32>
__global__ void __launch_bounds__(kThreads)
    kv_rows_lean(const CopyJob job, const ChunkListT<NC> chunks) {
  constexpr int kR = TABLE ? kLeanR : kLeanRFlat;
  using V = u32x4;
  constexpr int kSlice = 64 * 16 * kSegs;
  const int c = NC == 1 ? 0 : static_cast<int>(blockIdx.z);
  const int y = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * kWaves + wave;
  // Kernel arguments (fixed offsets).
  const int L = job.n_layers;
  const int T = chunks.tok_count[c];
  const int64_t tok_start = chunks.tok_start[c];
  uint8_t *const lmc = reinterpret_cast<uint8_t *>(chunks.lmc[c]);
  const int spr_shift = job.spr_shift;
  const int bs_shift = job.bs_shift;
  const bool page2lmc = job.page2lmc != 0;
  const int p = NP == 1 ? 0 : (y >= L) + (NP == 3 ? (y >= 2 * L) : 0);
  // The plane's descriptor fields, each selected from the NP kernel-argument
  // values (no private array: the compiler turns a selection over one into
  // an indexed access of per-lane scratch memory).
  const PlaneDesc &d0 = job.plane[0];
  const PlaneDesc &d1 = job.plane[NP > 1 ? 1 : 0];
  const PlaneDesc &d2 = job.plane[NP > 2 ? 2 : 0];
  auto pick = [&](int64_t v0, int64_t v1, int64_t v2) -> int64_t {
    return NP == 1 ? v0 : NP == 2 ? (p == 1 ? v1 : v0) : (p == 2 ? v2 : p == 1 ? v1 : v0);
  };
  const int64_t paged_off = pick(d0.paged_off, d1.paged_off, d2.paged_off);
  const int64_t blk_stride = pick(d0.blk_stride, d1.blk_stride, d2.blk_stride);
  const int64_t row_pitch = pick(d0.row_pitch, d1.row_pitch, d2.row_pitch);
  const int64_t lmc_fixed = pick(d0.lmc_off_fixed, d1.lmc_off_fixed, d2.lmc_off_fixed);
  const int64_t lmc_per_t = pick(d0.lmc_off_per_t, d1.lmc_off_per_t, d2.lmc_off_per_t);
  const int64_t layer_fixed = pick(d0.lmc_layer_fixed, d1.lmc_layer_fixed, d2.lmc_layer_fixed);
  const int64_t layer_per_t = pick(d0.lmc_layer_per_t, d1.lmc_layer_per_t, d2.lmc_layer_per_t);
  const int64_t tok_stride = pick(d0.lmc_token_stride, d1.lmc_token_stride, d2.lmc_token_stride);
  const int l = y - p * L;
  // Independent loads: the slots and the plane's paged base.
  int t[kR];
  int64_t slot[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    t[r] = (item * kR + r) >> spr_shift;
    const int tc = t[r] < T ? t[r] : T - 1;  // in-range token for the slot load
    slot[r] = SLOT32 ? static_cast<int64_t>(static_cast<const int32_t *>(job.slots)[tok_start + tc])
                     : static_cast<const int64_t *>(job.slots)[tok_start + tc];
  }
  const uint64_t pbase =
      TABLE ? job.table[static_cast<int64_t>(l) * job.table_ppl + p * job.idx_step]
            : pick(static_cast<int64_t>(job.base[0]), static_cast<int64_t>(job.base[NP > 1 ? 1 : 0]),
                   static_cast<int64_t>(job.base[NP > 2 ? 2 : 0]));
  // One wait covers all of these loads: without this the compiler places the
  // range check between them and issues the table load only after the slot.
#pragma unroll
  for (int r = 0; r < kR; ++r) asm volatile("" ::"s"(slot[r]));
  asm volatile("" ::"s"(pbase));
  // Addresses.  Flat rows are block rows with a zero shift (the host sets
  // blk_stride = row_pitch for them), so no branch splits the chain.
  const uint8_t *src[kR];
  uint8_t *dst[kR];
  bool live[kR];
  uintptr_t align = 0;
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int64_t blk = slot[r] >> bs_shift;
    const int64_t in_blk = slot[r] & ((int64_t(1) << bs_shift) - 1);
    const int64_t off0 = static_cast<int64_t>((item * kR + r) & ((1 << spr_shift) - 1)) * kSlice;
    uint8_t *paged = reinterpret_cast<uint8_t *>(pbase) + paged_off + blk * blk_stride + in_blk * row_pitch + off0;
    uint8_t *lm = lmc + lmc_fixed + lmc_per_t * T + static_cast<int64_t>(l) * (layer_fixed + layer_per_t * T) +
                  static_cast<int64_t>(t[r]) * tok_stride + off0;
    src[r] = page2lmc ? paged : lm;
    dst[r] = page2lmc ? lm : paged;
    live[r] = t[r] < T && static_cast<uint64_t>(slot[r]) < static_cast<uint64_t>(job.num_slots);
    if (live[r]) align |= reinterpret_cast<uintptr_t>(src[r]) | reinterpret_cast<uintptr_t>(dst[r]);
  }
  // A table entry (a device value) that is not 16-byte aligned sends the
  // slices to the byte path.
  if ((align & 15) != 0) {
#pragma unroll
    for (int r = 0; r < kR; ++r)
      if (live[r])
        for (int o = lane; o < kSlice; o += 64) dst[r][o] = src[r][o];
    return;
  }
  V v[kR][kSegs];
#pragma unroll
  for (int r = 0; r < kR; ++r)
    if (live[r])
#pragma unroll
      for (int s = 0; s < kSegs; ++s)
        v[r][s] = ld<V, NT>(reinterpret_cast<const V *>(src[r] + (s * 64 + lane) * 16));
#pragma unroll
  for (int r = 0; r < kR; ++r)
    if (live[r])
#pragma unroll
      for (int s = 0; s < kSegs; ++s)
        st<V, NT, false>(reinterpret_cast<V *>(dst[r] + (s * 64 + lane) * 16), v[r][s]);
}

// Tile kernel.  A wave owns a tile of up to 64 consecutive tokens of one
// (plane, layer) of a chunk.  Lane i resolves row i once (slot load, range
// check, paged and LMC addresses); the tile's bytes are then streamed as one
// flattened range of VEC-byte vectors, kTileU accesses in flight per lane,
// each lane fetching its row's addresses from the owning lane with a
// cross-lane shuffle.  The scalar work per tile (pointer-table entry, plane
// geometry) and the slot loads are amortised over the whole tile, and every
// access is full whatever the row width.
#ifndef LMC_KV_TILE_U
#define LMC_KV_TILE_U 4           // accesses in flight per lane
#endif
constexpr int kTileU = LMC_KV_TILE_U;

__device__ __forceinline__ uint64_t shfl64(uint64_t x, int src_lane) {
  const int lo = __shfl(static_cast<int>(x), src_lane, 64);
  const int hi = __shfl(static_cast<int>(x >> 32), src_lane, 64);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
         static_cast<uint32_t>(lo);
}

template <int VEC, bool NT, int NC, bool WT>
__global__ void __launch_bounds__(kThreads)
    kv_tiles_copy(const CopyJob job, const ChunkListT<NC> chunks, int tile_rows) {
  using V = typename VecOf<VEC>::T;
  const int c = blockIdx.y;
  const int tok0 = chunks.tok_start[c];
  const int T = chunks.tok_count[c];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t *lmc = reinterpret_cast<uint8_t *>(chunks.lmc[c]);
  const int tiles_per_pl = (T + tile_rows - 1) / tile_rows;
  const int n_tiles = job.n_planes * job.n_layers * tiles_per_pl;
  for (int tile = blockIdx.x * kWaves + wave; tile < n_tiles;
       tile += gridDim.x * kWaves) {
    const int pl = tile / tiles_per_pl;
    const int t0 = (tile - pl * tiles_per_pl) * tile_rows;
    const int p = pl / job.n_layers;
    const int l = pl - p * job.n_layers;
    const int nrows = T - t0 < tile_rows ? T - t0 : tile_rows;
    const PlaneDesc &pd = job.plane[p];
    uint64_t pbase;
    if (job.table != nullptr) {
      pbase = job.table[static_cast<int64_t>(l) * job.table_ppl + job.table_idx[p]];
      pbase = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(pbase))) |
              (static_cast<uint64_t>(static_cast<uint32_t>(
                   __builtin_amdgcn_readfirstlane(static_cast<int>(pbase >> 32))))
               << 32);
    } else {
      pbase = job.base[p];
    }
    uint8_t *lm_base = lmc + pd.lmc_off_fixed + pd.lmc_off_per_t * T +
                       static_cast<int64_t>(l) * (pd.lmc_layer_fixed + pd.lmc_layer_per_t * T);
    // Row setup: lane i owns row t0 + i.  A skipped slot leaves src == 0.
    uint64_t my_src = 0, my_dst = 0;
    if (lane < nrows) {
      const int t = t0 + lane;
      const int64_t slot = job.slot_i32
                               ? static_cast<int64_t>(static_cast<const int32_t *>(job.slots)[tok0 + t])
                               : static_cast<const int64_t *>(job.slots)[tok0 + t];
      if (slot >= 0 && slot < job.num_slots) {
        int64_t poff = pd.paged_off;
        if (job.block_size > 0) {
          const uint32_t s32 = static_cast<uint32_t>(slot);
          const uint32_t bs = static_cast<uint32_t>(job.block_size);
          const uint32_t blk = s32 / bs;
          poff += static_cast<int64_t>(blk) * pd.blk_stride +
                  static_cast<int64_t>(s32 - blk * bs) * pd.row_pitch;
        } else {
          poff += slot * pd.row_pitch;
        }
        const uint64_t paged = pbase + static_cast<uint64_t>(poff);
        const uint64_t lm = reinterpret_cast<uint64_t>(lm_base) +
                            static_cast<uint64_t>(static_cast<int64_t>(t) * pd.lmc_token_stride);
        my_src = job.page2lmc ? paged : lm;
        my_dst = job.page2lmc ? lm : paged;
      }
    }
    const int vpr = static_cast<int>(pd.row_bytes / VEC);
    const int total = nrows * vpr;
    // Any misaligned row (a misaligned table entry) sends the tile to the
    // byte path.
    const bool slow = __any(((my_src | my_dst) & (VEC - 1)) != 0);
    if (slow) {
      for (int r = 0; r < nrows; ++r) {
        const uint8_t *src = reinterpret_cast<const uint8_t *>(shfl64(my_src, r));
        uint8_t *dst = reinterpret_cast<uint8_t *>(shfl64(my_dst, r));
        if (src != nullptr)
          for (int64_t o = lane; o < pd.row_bytes; o += 64) dst[o] = src[o];
      }
      continue;
    }
    for (int f0 = 0; f0 < total; f0 += 64 * kTileU) {
      V v[kTileU];
      uint64_t dst[kTileU];
      bool live[kTileU];
#pragma unroll
      for (int u = 0; u < kTileU; ++u) {
        const int f = f0 + u * 64 + lane;
        const int r = f / vpr;
        const int col = f - r * vpr;
        const int src_lane = r < 64 ? r : 63;
        const uint64_t src = shfl64(my_src, src_lane);
        dst[u] = shfl64(my_dst, src_lane);
        live[u] = f < total && src != 0;
        if (live[u])
          v[u] = ld<V, NT>(reinterpret_cast<const V *>(src + static_cast<uint64_t>(col) * VEC));
        dst[u] += static_cast<uint64_t>(col) * VEC;
      }
#pragma unroll
      for (int u = 0; u < kTileU; ++u)
        if (live[u]) st<V, NT, WT>(reinterpret_cast<V *>(dst[u]), v[u]);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

namespace {

// Largest access width (16/8/4/2/1 bytes) dividing every host-visible offset,
// stride and address of the job.
int pick_vec(const CopyJob &job, const ChunkList &chunks, int n_chunks) {
  int64_t g = 16;
  auto fold = [&](int64_t v) { g = gcd64(g, v); };
  for (int p = 0; p < job.n_planes; ++p) {
    const PlaneDesc &d = job.plane[p];
    fold(d.row_bytes);
    fold(d.lmc_off_fixed);
    fold(d.lmc_off_per_t);
    fold(d.lmc_layer_fixed);
    fold(d.lmc_layer_per_t);
    fold(d.lmc_token_stride);
    fold(d.paged_off);
    fold(d.blk_stride);
    fold(d.row_pitch);
    if (job.table == nullptr) fold(static_cast<int64_t>(job.base[p] & 0xff));
  }
  for (int c = 0; c < n_chunks; ++c)
    fold(static_cast<int64_t>(chunks.lmc[c] & 0xff));
  if (g == 0) g = 16;
  if (g % 16 == 0) return 16;
  if (g % 8 == 0) return 8;
  if (g % 4 == 0) return 4;
  if (g % 2 == 0) return 2;
  return 1;
}

ChunkListT<1> first_chunk(const ChunkList &cl) {
  ChunkListT<1> one;
  one.lmc[0] = cl.lmc[0];
  one.tok_start[0] = cl.tok_start[0];
  one.tok_count[0] = cl.tok_count[0];
  return one;
}

template <int VEC, int NC, bool SLOT32, bool TABLE>
void launch_rows_st(const CopyJob &job, const ChunkListT<NC> &chunks, dim3 grid, dim3 block, bool nt,
                    hipStream_t stream) {
  if (nt) hipLaunchKernelGGL((kv_rows_copy<VEC, true, NC, SLOT32, TABLE>), grid, block, 0, stream, job, chunks);
  else hipLaunchKernelGGL((kv_rows_copy<VEC, false, NC, SLOT32, TABLE>), grid, block, 0, stream, job, chunks);
}

template <int VEC, int NC>
void launch_rows(const CopyJob &job, const ChunkListT<NC> &chunks, dim3 grid, dim3 block, bool nt,
                 hipStream_t stream) {
  if (job.slot_i32) {
    if (job.table != nullptr) launch_rows_st<VEC, NC, true, true>(job, chunks, grid, block, nt, stream);
    else launch_rows_st<VEC, NC, true, false>(job, chunks, grid, block, nt, stream);
  } else {
    if (job.table != nullptr) launch_rows_st<VEC, NC, false, true>(job, chunks, grid, block, nt, stream);
    else launch_rows_st<VEC, NC, false, false>(job, chunks, grid, block, nt, stream);
  }
}

template <bool NT, int NC, bool TABLE, bool SLOT32>
void launch_lean_p(const CopyJob &job, const ChunkListT<NC> &chunks, dim3 grid,
                   hipStream_t stream) {
  const dim3 block(kThreads);
  switch (job.n_planes) {
  case 1: hipLaunchKernelGGL((kv_rows_lean<NT, NC, TABLE, 1, SLOT32>), grid, block, 0, stream, job, chunks); break;
  case 2: hipLaunchKernelGGL((kv_rows_lean<NT, NC, TABLE, 2, SLOT32>), grid, block, 0, stream, job, chunks); break;
  default: hipLaunchKernelGGL((kv_rows_lean<NT, NC, TABLE, 3, SLOT32>), grid, block, 0, stream, job, chunks); break;
  }
}

template <bool NT, int NC, bool TABLE>
void launch_lean_s(const CopyJob &job, const ChunkListT<NC> &chunks, dim3 grid,
                   hipStream_t stream) {
  if (job.slot_i32) launch_lean_p<NT, NC, TABLE, true>(job, chunks, grid, stream);
  else launch_lean_p<NT, NC, TABLE, false>(job, chunks, grid, stream);
}

template <int NC>
void launch_lean_t(const CopyJob &job, const ChunkListT<NC> &chunks, dim3 grid,
                   bool nt, hipStream_t stream) {
  if (job.table != nullptr) {
    if (nt) launch_lean_s<true, NC, true>(job, chunks, grid, stream);
    else launch_lean_s<false, NC, true>(job, chunks, grid, stream);
  } else {
    if (nt) launch_lean_s<true, NC, false>(job, chunks, grid, stream);
    else launch_lean_s<false, NC, false>(job, chunks, grid, stream);
  }
}

void launch_lean(const CopyJob &job, const ChunkList &chunks, int n_chunks,
                 dim3 grid, bool nt, hipStream_t stream) {
  if (n_chunks == 1) launch_lean_t<1>(job, first_chunk(chunks), grid, nt, stream);
  else launch_lean_t<kMaxChunks>(job, chunks, grid, nt, stream);
}

template <int VEC>
void launch_vec(const CopyJob &job_in, const ChunkList &chunks, int n_chunks,
                int max_rows, bool nt, bool host_lmc, hipStream_t stream) {
  CopyJob job = job_in;
  constexpr int64_t kSlice = 64 * VEC * kSegs;
  int64_t widest = 0;
  for (int p = 0; p < job.n_planes; ++p)
    widest = std::max(widest, job.plane[p].row_bytes);
  job.slices_per_row = static_cast<int32_t>(std::max<int64_t>(1, (widest + kSlice - 1) / kSlice));
  bool whole_slices = true;
  for (int p = 0; p < job.n_planes; ++p)
    whole_slices = whole_slices && job.plane[p].row_bytes % kSlice == 0;
  dim3 block(kThreads);
  // The lean kernel takes rows of one power-of-two number of 16-byte-aligned
  // 2 KiB slices in every plane and a power-of-two block size.
  const auto pow2 = [](int64_t v) { return v > 0 && (v & (v - 1)) == 0; };
  bool lean = LMC_KV_LEAN && VEC == 16 && whole_slices && pow2(job.slices_per_row) &&
              (job.block_size == 0 || pow2(job.block_size)) &&
              static_cast<int64_t>(job.n_layers) * job.n_planes <= 65535;
  for (int p = 0; p < job.n_planes; ++p) lean = lean && job.plane[p].row_bytes == widest;
  // Plane p's pointer-table entry must be l * ppl + p * idx_step.
  job.idx_step = job.n_planes > 1 ? job.table_idx[1] : 0;
  for (int p = 0; p < job.n_planes; ++p) lean = lean && job.table_idx[p] == p * job.idx_step;
  // The lean kernel serves launches over one memory object of up to
  // LMC_KV_LEAN_MAX_ROWS rows (the per-object and per-layer calls, whose
  // time is mostly each launch's first and last waves).  Batches and larger
  // launches keep the general row kernel, which moved them 3-6% faster on
  // MI355X (8B shape, 16 objects; one 32768-token Qwen3-32B-shape layer).
  lean = lean && ((n_chunks == 1 && max_rows <= LMC_KV_LEAN_MAX_ROWS) || LMC_KV_LEAN_BATCH);
  if (lean) {
    job.spr_shift = __builtin_ctzll(static_cast<uint64_t>(job.slices_per_row));
    if (job.block_size > 0) {
      job.bs_shift = __builtin_ctzll(static_cast<uint64_t>(job.block_size));
    } else {
      // Flat rows as blocks of one row.
      job.bs_shift = 0;
      for (int p = 0; p < job.n_planes; ++p) job.plane[p].blk_stride = job.plane[p].row_pitch;
    }
    const int64_t max_tokens = max_rows / (job.n_planes * job.n_layers);
    const int64_t items = max_tokens * job.slices_per_row;
    check(items < (int64_t(1) << 31), "too many work items in one chunk");
    const int64_t per_block = kWaves * (job.table != nullptr ? kLeanR : kLeanRFlat);
    dim3 grid(static_cast<unsigned>(std::max<int64_t>(1, (items + per_block - 1) / per_block)),
              job.n_layers * job.n_planes, n_chunks);
    launch_lean(job, chunks, n_chunks, grid, nt, stream);
  } else if (whole_slices) {
    // Every row is a whole number of slices: one slice per wave.
    const int64_t max_items = static_cast<int64_t>(max_rows) * job.slices_per_row;
    check(max_items < (int64_t(1) << 31), "too many work items in one chunk");
    const int items_per_block = kWaves * kRowsPerWave;
    int gx = static_cast<int>((max_items + items_per_block - 1) / items_per_block);
    dim3 grid(std::max(1, std::min(gx, LMC_KV_GRID_CAP)), n_chunks);
    if (n_chunks == 1) launch_rows<VEC>(job, first_chunk(chunks), grid, block, nt, stream);
    else launch_rows<VEC>(job, chunks, grid, block, nt, stream);
  } else {
    // Narrower or odd rows: tiles of about 32 KiB of the widest plane,
    // 16..64 rows; a store between device buffers (paged reads) instead
    // takes tiles of one pass of the wave (64 lanes x kTileU accesses).
    // Measured on MI355X, store / retrieve: MLA 1152-byte rows, 28-row
    // tiles 0.434 / 0.386 ms, 3-row tiles 0.397 / 0.400; 256-byte rows,
    // 64-row tiles 0.242 / 0.255 ms, 16-row tiles 0.235 / 0.256.
    const int64_t w = std::max<int64_t>(1, widest);
    const int tile_rows = static_cast<int>(
        job.page2lmc && !host_lmc
            ? std::max<int64_t>(1, std::min<int64_t>(64, 64 * kTileU * VEC / w))
            : std::max<int64_t>(16, std::min<int64_t>(64, 32768 / w)));
    const int64_t max_tokens = max_rows / (job.n_planes * job.n_layers);
    const int64_t tiles = static_cast<int64_t>(job.n_planes) * job.n_layers *
                          ((max_tokens + tile_rows - 1) / tile_rows);
    check(widest / VEC * tile_rows < (int64_t(1) << 31) && tiles < (int64_t(1) << 31),
          "too many tiles in one chunk");
    int gx = static_cast<int>((tiles + kWaves - 1) / kWaves);
    dim3 grid(std::max(1, std::min(gx, LMC_KV_GRID_CAP)), n_chunks);
    // Stores into memory objects are written through, stores into the paged
    // caches stream (see st()).
    const bool wt = job.page2lmc != 0;
    if (n_chunks == 1) {
      const ChunkListT<1> one = first_chunk(chunks);
      if (nt && wt)
        hipLaunchKernelGGL((kv_tiles_copy<VEC, true, 1, true>), grid, block, 0, stream, job, one, tile_rows);
      else if (nt)
        hipLaunchKernelGGL((kv_tiles_copy<VEC, true, 1, false>), grid, block, 0, stream, job, one, tile_rows);
      else
        hipLaunchKernelGGL((kv_tiles_copy<VEC, false, 1, false>), grid, block, 0, stream, job, one, tile_rows);
    } else if (nt && wt) {
      hipLaunchKernelGGL((kv_tiles_copy<VEC, true, kMaxChunks, true>), grid, block, 0, stream, job, chunks,
                         tile_rows);
    } else if (nt) {
      hipLaunchKernelGGL((kv_tiles_copy<VEC, true, kMaxChunks, false>), grid, block, 0, stream, job, chunks,
                         tile_rows);
    } else {
      hipLaunchKernelGGL((kv_tiles_copy<VEC, false, kMaxChunks, false>), grid, block, 0, stream, job, chunks,
                         tile_rows);
    }
  }
}



// Launches one copy over `n` chunks (split into launches of kMaxChunks).
// `host_lmc`: the LMCache side is page-locked host memory reached over PCIe;
// the streaming (non-temporal) cache hints are used for HBM-only copies.
void launch_copy(const CopyJob &job, const std::vector<uint64_t> &all_lmc,
                 const std::vector<int64_t> &all_starts,
                 const std::vector<int64_t> &all_counts, bool host_lmc,
                 hipStream_t stream) {
  // Chunks without tokens move nothing; the kernels assume every chunk of a
  // launch holds at least one token.
  std::vector<uint64_t> lmc_ptrs;
  std::vector<int64_t> tok_starts, tok_counts;
  for (size_t i = 0; i < all_lmc.size(); ++i) {
    if (all_counts[i] <= 0) continue;
    lmc_ptrs.push_back(all_lmc[i]);
    tok_starts.push_back(all_starts[i]);
    tok_counts.push_back(all_counts[i]);
  }
  const size_t n = lmc_ptrs.size();
  const int64_t slot_es = job.slot_i32 ? 4 : 8;
  for (size_t c0 = 0; c0 < n; c0 += kMaxChunks) {
    const int nc = static_cast<int>(std::min<size_t>(kMaxChunks, n - c0));
    // Rebase the slot pointer to the smallest start of this group so the
    // per-chunk token offsets fit 32-bit kernel arithmetic.
    int64_t base_tok = tok_starts[c0];
    for (int i = 1; i < nc; ++i) base_tok = std::min(base_tok, tok_starts[c0 + i]);
    CopyJob j = job;
    j.slots = static_cast<const uint8_t *>(job.slots) + base_tok * slot_es;
    ChunkList cl;
    std::memset(&cl, 0, sizeof(cl));
    int max_rows = 0;
    for (int i = 0; i < nc; ++i) {
      const int64_t rel = tok_starts[c0 + i] - base_tok;
      const int64_t cnt = tok_counts[c0 + i];
      const int64_t rows = cnt * job.n_layers * job.n_planes;
      check(rel + cnt < (int64_t(1) << 31) && rows < (int64_t(1) << 31),
            "chunk does not fit 32-bit row indexing");
      cl.lmc[i] = lmc_ptrs[c0 + i];
      cl.tok_start[i] = static_cast<int32_t>(rel);
      cl.tok_count[i] = static_cast<int32_t>(cnt);
      max_rows = std::max<int>(max_rows, static_cast<int>(rows));
    }
    if (max_rows == 0) continue;
    const int vec = pick_vec(j, cl, nc);
    const bool nt = nontemporal_enabled() && !host_lmc;
    switch (vec) {
    case 16: launch_vec<16>(j, cl, nc, max_rows, nt, host_lmc, stream); break;
    case 8: launch_vec<8>(j, cl, nc, max_rows, nt, host_lmc, stream); break;
    case 4: launch_vec<4>(j, cl, nc, max_rows, nt, host_lmc, stream); break;
    case 2: launch_vec<2>(j, cl, nc, max_rows, nt, host_lmc, stream); break;
    default: launch_vec<1>(j, cl, nc, max_rows, nt, host_lmc, stream); break;
    }
    hip_check(hipGetLastError(), "kv_rows_copy launch");
  }
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }


// --- multi-layer planning (csrc/utils.cpp:29-86) ---------------------------

struct MultiLayerGeom {
  CopyJob job;                 // LMC geometry is per-T (filled per chunk)
  int64_t lmc_bytes_per_token; // LMC bytes one token occupies (all planes,
                               // all layers)
  int n_planes;
};

MultiLayerGeom plan_multi_layer(int64_t n_layers, int64_t last_dim,
                                int64_t es, const lmc_tensor &ptrs,
                                int64_t page_buffer_size, bool direction,
                                bool use_mla, int fmt, int64_t kH, int64_t vH,
                                int64_t dsaH) {
  MultiLayerGeom g;
  std::memset(&g, 0, sizeof(g));
  CopyJob &job = g.job;
  int64_t width[kMaxPlanes] = {0, 0, 0};
  int64_t paged_off[kMaxPlanes] = {0, 0, 0};
  int idx[kMaxPlanes] = {0, 0, 0};
  int planes = 0, ppl = 0;
  bool concatenated = false;  // [1, L, T, sum(W)] rows vs [P, L, T, W]
  switch (fmt) {
  case LMC_FMT_MERGED_KV:
    if (use_mla) {
      // Single-plane MLA latent cache: one [NB, BS, W] tensor per layer
      // (the upstream-LMCache use_mla meaning, also the MindSpore host path,
      // csrc/mindspore/mem_kernels.cpp:85-88).
      planes = 1; ppl = 1; width[0] = last_dim;
    } else {
      // ptrs[l] -> [2, NB, BS, H, D]; V plane follows page_buffer_size rows
      // of K (csrc/mem_kernels.cpp:58-69).
      planes = 2; ppl = 1; width[0] = width[1] = last_dim;
      idx[1] = 0;
      paged_off[1] = page_buffer_size * last_dim * es;
    }
    break;
  case LMC_FMT_SEPARATE_KV:
    if (use_mla) {
      planes = 1; ppl = 1; width[0] = last_dim;
    } else {
      planes = 2; ppl = 2; width[0] = width[1] = last_dim;
      idx[1] = 1;
    }
    break;
  case LMC_FMT_MLA_KV:
  case LMC_FMT_MLA_LATENT:
    planes = 2; ppl = 2; width[0] = kH; width[1] = vH; idx[1] = 1;
    concatenated = true;
    break;
  case LMC_FMT_DSA_KV:
    planes = 3; ppl = 3; width[0] = kH; width[1] = vH; width[2] = dsaH;
    idx[1] = 1; idx[2] = 2;
    concatenated = true;
    break;
  case LMC_FMT_DSA_INDEX:
    planes = 1; ppl = 1; width[0] = dsaH;
    concatenated = true;
    break;
  default:
    fail(LMC_ERR_RUNTIME, "multi-layer transfer: no plane layout for KV format " + std::to_string(fmt));
  }
  for (int p = 0; p < planes; ++p)
    check(width[p] > 0, "hidden dims must be positive for KV format " +
                            std::to_string(fmt));
  check(page_buffer_size > 0, "page_buffer_size must be positive");
  check(ptrs.dtype == LMC_I64 && ptrs.ndim == 1,
        "key_value_ptrs must be a 1-D int64 tensor");
  check(ptrs.device >= 0, "key_value_ptrs must be a device tensor");
  check(ptrs.sizes[0] >= n_layers * ppl,
        "key_value_ptrs has " + std::to_string(ptrs.sizes[0]) +
            " entries, need " + std::to_string(n_layers * ppl));
  check(ptrs.sizes[0] <= 1 || ptrs.strides[0] == 1,
        "key_value_ptrs must be contiguous");

  int64_t wsum = 0;
  for (int p = 0; p < planes; ++p) wsum += width[p];
  int64_t col = 0;
  for (int p = 0; p < planes; ++p) {
    PlaneDesc &d = job.plane[p];
    d.row_bytes = width[p] * es;
    if (concatenated) {
      d.lmc_off_fixed = col * es;
      d.lmc_layer_per_t = wsum * es;
      d.lmc_token_stride = wsum * es;
    } else {
      d.lmc_off_per_t = static_cast<int64_t>(p) * n_layers * width[p] * es;
      d.lmc_layer_per_t = width[p] * es;
      d.lmc_token_stride = width[p] * es;
    }
    d.paged_off = paged_off[p];
    d.row_pitch = width[p] * es;
    d.blk_stride = 0;
    job.table_idx[p] = idx[p];
    col += width[p];
  }
  job.table = reinterpret_cast<const uint64_t *>(ptrs.data);
  job.table_ppl = ppl;
  job.n_planes = planes;
  job.n_layers = static_cast<int32_t>(n_layers);
  job.block_size = 0;
  job.num_slots = page_buffer_size;
  job.page2lmc = direction ? 1 : 0;
  g.n_planes = planes;
  g.lmc_bytes_per_token = n_layers * wsum * es;
  return g;
}

void run_multi_layer(const lmc_tensor *chunks, int n_chunks,
                     const int64_t *token_starts, const lmc_tensor *ptrs_t,
                     const lmc_tensor *slots_t, int paged_device,
                     int64_t page_buffer_size, bool direction, bool use_mla,
                     int fmt, int64_t kH, int64_t vH, int64_t dsaH,
                     hipStream_t stream, bool batched) {
  check(n_chunks >= 0, "n_chunks must be non-negative");
  if (n_chunks == 0) return;
  const lmc_tensor &ptrs = deref(ptrs_t, "key_value_ptrs");
  const lmc_tensor &slots = slots_of(slots_t);
  const lmc_tensor &first = deref(&chunks[0], "key_value");
  check(first.ndim >= 2, "key_value must have at least 2 dims");
  const int64_t n_layers = size(first, 1);
  const int64_t last_dim = size(first, -1);
  const int64_t es = elem_size(first);
  MultiLayerGeom g = plan_multi_layer(n_layers, last_dim, es, ptrs,
                                      page_buffer_size, direction, use_mla,
                                      fmt, kH, vH, dsaH);
  DeviceGuard guard(paged_device >= 0 ? paged_device : ptrs.device);
  g.job.slots = kernel_ptr(slots);
  g.job.slot_i32 = slots.dtype == LMC_I32;

  std::vector<uint64_t> lmc_ptrs(n_chunks);
  std::vector<int64_t> starts(n_chunks), counts(n_chunks);
  bool host_lmc = false;
  for (int c = 0; c < n_chunks; ++c) {
    const lmc_tensor &kv = deref(&chunks[c], "key_value");
    check(kv.ndim >= 2 && size(kv, 1) == n_layers && size(kv, -1) == last_dim &&
              elem_size(kv) == es,
          "all memory objects of a batch must share layers, width and dtype");
    // The reference takes the token count from slot_mapping for a single
    // call (csrc/utils.cpp:43) and ignores key_value's strides, treating the
    // object as a flat [kv, L, T, W] buffer (csrc/mem_kernels.cpp:83).
    const int64_t T = batched ? size(kv, -2) : slots.sizes[0];
    const int64_t start = batched ? token_starts[c] : 0;
    check(start >= 0 && start + T <= slots.sizes[0],
          "chunk token range exceeds slot_mapping");
    const int64_t need = T * g.lmc_bytes_per_token;
    check(nbytes(kv) >= need,
          "key_value holds " + std::to_string(nbytes(kv)) +
              " bytes, the transfer needs " + std::to_string(need));
    lmc_ptrs[c] = reinterpret_cast<uint64_t>(
        T > 0 ? kernel_ptr(kv) : static_cast<uint8_t *>(kv.data));
    starts[c] = start;
    counts[c] = T;
    host_lmc = host_lmc || kv.device < 0;
  }
  launch_copy(g.job, lmc_ptrs, starts, counts, host_lmc, stream);
}

} // namespace

bool nontemporal_enabled() {
  static const bool on = [] {
    const char *e = std::getenv("LMC_AMD_NONTEMPORAL");
    return e == nullptr || e[0] != '0';
  }();
  return on;
}

const lmc_tensor &slots_of(const lmc_tensor *s) {
  const lmc_tensor &t = deref(s, "slot_mapping");
  check(t.ndim == 1, "slot_mapping must be 1-D");
  check(t.dtype == LMC_I64 || t.dtype == LMC_I32,
        "slot_mapping must be int64 or int32");
  check(t.sizes[0] <= 1 || t.strides[0] == 1,
        "slot_mapping must be contiguous");
  return t;
}

// --- single-layer planning (csrc/utils.cpp:212-406, 903-966) ---------------

void validate_vllm_caches(const lmc_tensor *caches, int n, int fmt) {
  if (fmt != LMC_FMT_MERGED_KV && fmt != LMC_FMT_SEPARATE_KV &&
      fmt != LMC_FMT_MLA_KV && fmt != LMC_FMT_DSA_KV &&
      fmt != LMC_FMT_MLA_LATENT && fmt != LMC_FMT_DSA_INDEX)
    fail(LMC_ERR_VALUE,
         "kvcache_format_raw " + std::to_string(fmt) +
             " is not a KV cache format (1 MERGED_KV, 2 SEPARATE_KV, 3 "
             "MLA_KV, 4 DSA_KV, 5 MLA_LATENT, 6 DSA_INDEX)");
  if (n <= 0) fail(LMC_ERR_VALUE, "vllm_kv_caches holds no tensor");
  auto same_sizes = [](const lmc_tensor &a, const lmc_tensor &b) {
    if (a.ndim != b.ndim) return false;
    for (int i = 0; i < a.ndim; ++i)
      if (a.sizes[i] != b.sizes[i]) return false;
    return true;
  };
  if (fmt == LMC_FMT_DSA_KV) {
    if (n != 3) fail(LMC_ERR_VALUE, "a DSA_KV layer takes three caches: K, V and the DSA keys");
  } else if (fmt == LMC_FMT_MLA_KV || fmt == LMC_FMT_MLA_LATENT) {
    if (n < 2)
      fail(LMC_ERR_VALUE, "an MLA_KV or MLA_LATENT layer takes two caches, K and V");
    if (same_sizes(caches[0], caches[1]))
      fail(LMC_ERR_VALUE, "MLA_KV / MLA_LATENT K and V caches of equal shape: "
                          "the latent and rope planes differ in width");
  } else if (fmt == LMC_FMT_DSA_INDEX) {
    // at least one tensor: already checked
  } else if (fmt == LMC_FMT_SEPARATE_KV) {
    if (n != 2) fail(LMC_ERR_VALUE, "a SEPARATE_KV layer takes two caches, K and V");
    if (!same_sizes(caches[0], caches[1]))
      fail(LMC_ERR_VALUE, "SEPARATE_KV K and V caches differ in shape");
  } else {
    if (n != 1) fail(LMC_ERR_VALUE, "a MERGED_KV layer takes one cache holding K and V");
  }
}

LayerGeom layer_geom(const lmc_tensor *caches, int n, int fmt, bool two_major,
                     int64_t kH, int64_t vH, int64_t dsaH) {
  validate_vllm_caches(caches, n, fmt);
  const lmc_tensor &k = deref(&caches[0], "vllm_kv_caches[0]");
  LayerGeom g;
  std::memset(&g, 0, sizeof(g));
  g.device = k.device;
  g.es = elem_size(k);
  g.mla_dsa = is_mla_dsa(fmt);
  if (g.mla_dsa) {
    // Hidden-dim defaults (csrc/utils.cpp:319-339).
    const lmc_tensor *v = nullptr, *dsa = nullptr;
    if (fmt != LMC_FMT_DSA_INDEX) v = &caches[1];
    if (fmt == LMC_FMT_DSA_KV) dsa = &caches[2];
    check(k.ndim >= 2, "paged cache must have at least 2 dims");
    if (kH <= 0) kH = size(k, -2) * size(k, -1);
    if (vH <= 0 && v != nullptr) vH = size(*v, -2) * size(*v, -1);
    if (dsaH <= 0 && dsa != nullptr) dsaH = size(*dsa, -2) * size(*dsa, -1);
    if (fmt == LMC_FMT_DSA_INDEX) {
      kH = dsaH > 0 ? dsaH : size(k, -2) * size(k, -1);
      vH = 0;
    }
    const lmc_tensor *tens[kMaxPlanes] = {&k, v, dsa};
    const int64_t w[kMaxPlanes] = {kH, fmt == LMC_FMT_DSA_INDEX ? 0 : vH,
                                   fmt == LMC_FMT_DSA_KV ? dsaH : 0};
    g.plane_elems = w[0] + w[1] + w[2];
    check(g.plane_elems > 0, "MLA/DSA caches give no row width");
    int64_t pre = 0;
    g.num_slots = INT64_MAX;
    for (int p = 0; p < kMaxPlanes; ++p) {
      if (w[p] <= 0 || tens[p] == nullptr) {
        pre += w[p];
        continue;
      }
      const int q = g.n_planes++;
      PlaneDesc &d = g.plane[q];
      d.row_bytes = w[p] * g.es;
      d.row_pitch = w[p] * g.es;
      g.base[q] = reinterpret_cast<uint64_t>(kernel_ptr(*tens[p]));
      g.width[q] = w[p];
      g.prefix[q] = pre;
      check(elem_size(*tens[p]) == g.es, "paged cache dtypes differ");
      g.num_slots = std::min(g.num_slots, numel(*tens[p]) / w[p]);
      pre += w[p];
    }
    g.block_size = 0;
  } else {
    check(k.ndim >= 3, "paged cache must have at least 3 dims");
    const int64_t H = size(k, -2), D = size(k, -1), BS = size(k, -3);
    const int64_t W = H * D;
    g.n_planes = 2;
    g.plane_elems = 2 * W;
    g.block_size = static_cast<int>(BS);
    for (int p = 0; p < 2; ++p) {
      g.plane[p].row_bytes = W * g.es;
      g.plane[p].row_pitch = W * g.es;
      g.width[p] = W;
      g.prefix[p] = p * W;
    }
    if (fmt == LMC_FMT_MERGED_KV) {
      // [2, NB, BS, H, D] (two-major) or [NB, 2, BS, H, D]
      // (csrc/utils.cpp:249-263).
      check(k.ndim == 5, "MERGED_KV cache must be 5-D");
      const int64_t blk = two_major ? stride(k, 1) : stride(k, 0);
      const int64_t voff = two_major ? stride(k, 0) : stride(k, 1);
      const int64_t NB = two_major ? size(k, 1) : size(k, 0);
      g.base[0] = g.base[1] = reinterpret_cast<uint64_t>(kernel_ptr(k));
      g.plane[0].blk_stride = g.plane[1].blk_stride = blk * g.es;
      g.plane[1].paged_off = voff * g.es;
      g.num_slots = NB * BS;
    } else {
      // SEPARATE: (K, V) each [NB, BS, H, D] (csrc/utils.cpp:266-282).
      const lmc_tensor &v = deref(&caches[1], "vllm_kv_caches[1]");
      check(elem_size(v) == g.es, "paged cache dtypes differ");
      g.base[0] = reinterpret_cast<uint64_t>(kernel_ptr(k));
      g.base[1] = reinterpret_cast<uint64_t>(kernel_ptr(v));
      g.plane[0].blk_stride = stride(k, 0) * g.es;
      g.plane[1].blk_stride = stride(v, 0) * g.es;
      g.num_slots = std::min(size(k, 0), size(v, 0)) * BS;
    }
  }
  return g;
}

int64_t single_layer_lmc(const LayerGeom &g, const lmc_tensor &lmc,
                         bool token_major, PlaneDesc *pl) {
  check(elem_size(lmc) == g.es, "LMC buffer and paged cache dtypes differ");
  if (g.mla_dsa) {
    // Stacked planes [K: N*kH | V: N*vH | DSA: N*dsaH] (csrc/utils.cpp:
    // 222-244, 350-357).
    const int64_t N = numel(lmc) / g.plane_elems;
    for (int p = 0; p < g.n_planes; ++p) {
      pl[p].lmc_off_fixed = g.prefix[p] * N * g.es;
      pl[p].lmc_token_stride = g.width[p] * g.es;
    }
    return N;
  }
  // Token-major [T, 2, W] or [2, T, W] by strides (csrc/utils.cpp:226-237).
  check(lmc.ndim >= 2, "LMC buffer must have at least 2 dims");
  const int64_t tok_stride = token_major ? stride(lmc, 0) : stride(lmc, 1);
  const int64_t val_off = token_major ? stride(lmc, 1) : stride(lmc, 0);
  for (int p = 0; p < 2; ++p) {
    pl[p].lmc_off_fixed = p == 0 ? 0 : val_off * g.es;
    pl[p].lmc_token_stride = tok_stride * g.es;
  }
  const int64_t room = extent_bytes(lmc) / g.es - val_off - g.width[0];
  if (room < 0) return 0;
  return tok_stride > 0 ? room / tok_stride + 1 : 1;
}

void single_layer(const lmc_tensor *lmc_t, const lmc_tensor *caches, int n,
                  const lmc_tensor *slots_t, bool direction, int fmt,
                  bool token_major, bool two_major, int64_t kH, int64_t vH,
                  int64_t dsaH, hipStream_t stream) {
  const LayerGeom g = layer_geom(caches, n, fmt, two_major, kH, vH, dsaH);
  const lmc_tensor &lmc = deref(lmc_t, "lmc_key_value_cache");
  const lmc_tensor &slots = slots_of(slots_t);
  DeviceGuard guard(g.device);
  const int64_t T = slots.sizes[0];

  CopyJob job;
  std::memset(&job, 0, sizeof(job));
  job.table = nullptr;
  job.slots = kernel_ptr(slots);
  job.slot_i32 = slots.dtype == LMC_I32;
  job.n_layers = 1;
  job.page2lmc = direction ? 1 : 0;
  job.n_planes = g.n_planes;
  job.block_size = g.block_size;
  job.num_slots = g.num_slots;
  // The kernels split a block-strided slot into (block, offset) in 32 bits.
  check(g.block_size == 0 || g.num_slots <= static_cast<int64_t>(UINT32_MAX),
        "paged caches of more than 2^32 slots are not supported");
  for (int p = 0; p < g.n_planes; ++p) {
    job.plane[p] = g.plane[p];
    job.base[p] = g.base[p];
  }
  const int64_t cap = single_layer_lmc(g, lmc, token_major, job.plane);
  if (g.mla_dsa)
    check(T <= cap, "LMC buffer holds " + std::to_string(cap) +
                        " tokens, slot_mapping has " + std::to_string(T));
  else
    check(T <= cap, "LMC buffer is too small for " + std::to_string(T) + " tokens");
  if (T == 0) return;
  std::vector<uint64_t> lp{reinterpret_cast<uint64_t>(kernel_ptr(lmc))};
  std::vector<int64_t> st{0}, ct{T};
  launch_copy(job, lp, st, ct, lmc.device < 0, stream);
}

void flash(const lmc_tensor *kv_t, const lmc_tensor *kc_t,
           const lmc_tensor *vc_t, const lmc_tensor *slots_t, int layer_idx,
           bool page2lmc, hipStream_t stream) {
  const lmc_tensor &kv = deref(kv_t, "key_value");
  const lmc_tensor &kc = deref(kc_t, "key_cache");
  const lmc_tensor &vc = deref(vc_t, "value_cache");
  const lmc_tensor &slots = slots_of(slots_t);
  DeviceGuard guard(kc.device);
  check(kv.ndim >= 2, "key_value must be [2, L, T, W]");
  const int64_t L = size(kv, 1), W = size(kv, -1), es = elem_size(kv);
  const int64_t T = slots.sizes[0];
  check(layer_idx >= 0 && layer_idx < L, "layer_idx out of range");
  check(elem_size(kc) == es && elem_size(vc) == es, "dtype mismatch");
  check(nbytes(kv) >= 2 * L * T * W * es, "key_value is too small");
  CopyJob job;
  std::memset(&job, 0, sizeof(job));
  job.slots = kernel_ptr(slots);
  job.slot_i32 = slots.dtype == LMC_I32;
  job.n_layers = 1;
  job.n_planes = 2;
  job.block_size = 0;
  job.page2lmc = page2lmc ? 1 : 0;
  job.num_slots = std::min(numel(kc), numel(vc)) / W;
  const lmc_tensor *caches[2] = {&kc, &vc};
  for (int p = 0; p < 2; ++p) {
    PlaneDesc &d = job.plane[p];
    d.row_bytes = W * es;
    d.lmc_off_fixed = (static_cast<int64_t>(p) * L + layer_idx) * T * W * es;
    d.lmc_token_stride = W * es;
    d.row_pitch = W * es;
    job.base[p] = reinterpret_cast<uint64_t>(kernel_ptr(*caches[p]));
  }
  if (T == 0) return;
  std::vector<uint64_t> lp{reinterpret_cast<uint64_t>(kernel_ptr(kv))};
  std::vector<int64_t> st{0}, ct{T};
  launch_copy(job, lp, st, ct, kv.device < 0, stream);
}

int64_t fused_required_size(int fmt, bool use_mla, int64_t L, int64_t T,
                            int64_t W, int64_t kH, int64_t vH, int64_t dsaH,
                            int64_t es) {
  // csrc/mem_kernels.cpp:143-165.
  switch (fmt) {
  case LMC_FMT_MLA_KV:
  case LMC_FMT_MLA_LATENT:
    return L * T * (kH + vH) * es;
  case LMC_FMT_DSA_KV:
    return L * T * (kH + vH + dsaH) * es;
  case LMC_FMT_DSA_INDEX:
    return L * T * dsaH * es;
  default:
    return (use_mla ? 1 : 2) * L * T * W * es;
  }
}

// Zeroes `n16` 16-byte words from `p` (a fill kernel, not hipMemsetAsync, so
// the call can be recorded into a HIP graph).
__global__ void __launch_bounds__(256) zero_words(u32x4 *p, int64_t n16) {
  const u32x4 z = {0u, 0u, 0u, 0u};
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<int64_t>(gridDim.x) * 256)
    gstore(p + i, z);
}

// Declared, with its contract, in kv_fused.h.
void fused_transfer(const lmc_tensor &kv, uint8_t *stg_data, int stg_device,
                    int64_t capacity, const char *too_small,
                    bool clear_before_store, const lmc_tensor *key_value_ptrs,
                    const lmc_tensor *slot_mapping, int32_t paged_device,
                    int64_t page_buffer_size, bool direction, bool use_mla,
                    int32_t kvcache_format, int64_t k_hidden_dims,
                    int64_t v_hidden_dims, int64_t dsa_hidden_dims,
                    hipStream_t s) {
  const lmc_tensor &slots = slots_of(slot_mapping);
  check(kv.ndim >= 2, "key_value must have at least 2 dims");
  const int64_t L = size(kv, 1), W = size(kv, -1), es = elem_size(kv);
  const int64_t T = slots.sizes[0];
  const int64_t required = fused_required_size(
      kvcache_format, use_mla, L, T, W, k_hidden_dims, v_hidden_dims,
      dsa_hidden_dims, es);
  check(capacity >= required, std::string(too_small) + ": need " +
                                  std::to_string(required) + " bytes, got " +
                                  std::to_string(capacity));
  check(nbytes(kv) >= required, "key_value is smaller than the transfer");
  DeviceGuard guard(paged_device >= 0 ? paged_device : stg_device);
  if (!direction && required > 0)
    hip_check(hipMemcpyAsync(stg_data, kv.data, required,
                             hipMemcpyHostToDevice, s),
              "copy of the host object into the staging buffer");
  if (direction && clear_before_store && required > 0) {
    const int64_t n16 = (required + 15) / 16;  // capacity is a multiple of 16
    const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_words, dim3(static_cast<uint32_t>(blocks)),
                       dim3(256), 0, s, reinterpret_cast<u32x4 *>(stg_data),
                       n16);
    hip_check(hipGetLastError(), "zero_words launch");
  }
  // The staging buffer is used as a flat buffer with key_value's logical
  // layout from its data pointer, whatever its view strides
  // (csrc/mem_kernels.cpp:124-126, 183-207); its capacity was checked
  // against `required` above.
  lmc_tensor view = kv;
  view.data = stg_data;
  view.device = stg_device;
  run_multi_layer(&view, 1, nullptr, key_value_ptrs, slot_mapping,
                  paged_device, page_buffer_size, direction, use_mla,
                  kvcache_format, k_hidden_dims, v_hidden_dims,
                  dsa_hidden_dims, s, false);
  if (direction && required > 0)
    hip_check(hipMemcpyAsync(kv.data, stg_data, required,
                             hipMemcpyDeviceToHost, s),
              "copy of the staging buffer into the host object");
}

} // namespace lmc

using namespace lmc;

extern "C" {

int lmc_multi_layer_kv_transfer(const lmc_tensor *key_value,
                                const lmc_tensor *key_value_ptrs,
                                const lmc_tensor *slot_mapping,
                                int32_t paged_device, int64_t page_buffer_size,
                                int32_t direction, int32_t use_mla,
                                int32_t kvcache_format, int64_t k_hidden_dims,
                                int64_t v_hidden_dims, int64_t dsa_hidden_dims,
                                void *stream) {
  return guarded([&] {
    run_multi_layer(key_value, 1, nullptr, key_value_ptrs, slot_mapping,
                    paged_device, page_buffer_size, direction != 0,
                    use_mla != 0, kvcache_format, k_hidden_dims,
                    v_hidden_dims, dsa_hidden_dims, as_stream(stream), false);
  });
}

int lmc_multi_layer_kv_transfer_batched(
    const lmc_tensor *chunks, int32_t n_chunks, const int64_t *token_starts,
    const lmc_tensor *key_value_ptrs, const lmc_tensor *slot_mapping,
    int32_t paged_device, int64_t page_buffer_size, int32_t direction,
    int32_t use_mla, int32_t kvcache_format, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream) {
  return guarded([&] {
    check(n_chunks == 0 || (chunks != nullptr && token_starts != nullptr),
          "chunks and token_starts are required");
    run_multi_layer(chunks, n_chunks, token_starts, key_value_ptrs,
                    slot_mapping, paged_device, page_buffer_size,
                    direction != 0, use_mla != 0, kvcache_format,
                    k_hidden_dims, v_hidden_dims, dsa_hidden_dims,
                    as_stream(stream), true);
  });
}

int lmc_fused_multi_layer_kv_transfer(
    const lmc_tensor *key_value, const lmc_tensor *staging_cache,
    const lmc_tensor *key_value_ptrs, const lmc_tensor *slot_mapping,
    int32_t paged_device, int64_t page_buffer_size, int32_t direction,
    int32_t use_mla, int32_t kvcache_format, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream) {
  return guarded([&] {
    const lmc_tensor &kv = deref(key_value, "key_value");
    const lmc_tensor &stg = deref(staging_cache, "staging_cache");
    check(stg.device >= 0, "staging_cache must be a device tensor");
    fused_transfer(kv, static_cast<uint8_t *>(stg.data), stg.device,
                   nbytes(stg), "staging_cache is smaller than the transfer", false,
                   key_value_ptrs, slot_mapping, paged_device,
                   page_buffer_size, direction != 0, use_mla != 0,
                   kvcache_format, k_hidden_dims, v_hidden_dims,
                   dsa_hidden_dims, as_stream(stream));
  });
}

int lmc_single_layer_kv_transfer(const lmc_tensor *lmc_key_value_cache,
                                 const lmc_tensor *caches, int32_t n_caches,
                                 const lmc_tensor *slot_mapping,
                                 int32_t direction, int32_t kvcache_format,
                                 int32_t token_major, int32_t vllm_two_major,
                                 int64_t k_hidden_dims, int64_t v_hidden_dims,
                                 int64_t dsa_hidden_dims, void *stream) {
  return guarded([&] {
    single_layer(lmc_key_value_cache, caches, n_caches, slot_mapping,
                 direction != 0, kvcache_format, token_major != 0,
                 vllm_two_major != 0, k_hidden_dims, v_hidden_dims,
                 dsa_hidden_dims, as_stream(stream));
  });
}

int lmc_load_and_reshape_flash(const lmc_tensor *key_value,
                               const lmc_tensor *key_cache,
                               const lmc_tensor *value_cache,
                               const lmc_tensor *slot_mapping,
                               int32_t layer_idx, void *stream) {
  return guarded([&] {
    flash(key_value, key_cache, value_cache, slot_mapping, layer_idx, true,
          as_stream(stream));
  });
}

int lmc_reshape_and_cache_back_flash(const lmc_tensor *key_value,
                                     const lmc_tensor *key_cache,
                                     const lmc_tensor *value_cache,
                                     const lmc_tensor *slot_mapping,
                                     int32_t layer_idx, void *stream) {
  return guarded([&] {
    flash(key_value, key_cache, value_cache, slot_mapping, layer_idx, false,
          as_stream(stream));
  });
}

} // extern "C"
