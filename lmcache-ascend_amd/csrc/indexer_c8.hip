// Indexer key / C8 packet transport for MI355X (gfx950).
//
// Replaces indexer_c8_transfer_prepared / indexer_c8_group_transfer_prepared
// and their state checks (csrc/indexer_c8.cpp:12-185; device semantics
// csrc/indexer_c8/kernel.cpp:29-121).  A layer's destination is a paged
// indexer cache: keys [NB, 128, 1, 128] (float16 / bfloat16, 256 bytes per
// slot; or int8, 128 bytes per slot, with float16 scales [NB, 128, 1, 1]).
// A packet holds one chunk of tokens: `count` key rows, then, for int8
// keys, `count` 2-byte scales.  Token t of chunk c is slot_mapping[start_c +
// t]; its physical cache slot is
//
//   block_map[slot / 128] * 128 + slot % 128            (block permutation)
//   slot + (slot / 128) * (slot_factor - 1) * 128       (otherwise)
//
// and its key row and scale move between packet and cache (from_npu: cache
// -> packet).  Chunks with a null packet or an impossible range, slots
// outside [0, cache_slots) and physical slots outside the cache are
// skipped, as in the reference kernel.
//
// Work mapping: grid (token tiles of the chunk capacity, chunk, layer); a
// group of lanes owns one or more tokens (8 lanes x 4 tokens when packing,
// 16 lanes x 4 tokens when unpacking), and the groups of a wave take
// consecutive tokens: the lanes move the key rows in 16-byte accesses
// (bytewise when the packet is not 16-byte aligned) and one lane per token
// its scale.  Every access is bounded by the checks above.
#include "common.h"
#include "gmem.h"

#include <algorithm>
#include <cstring>
#include <string>

namespace lmc {

namespace {

constexpr int kC8Threads = 256;
constexpr int kC8Layers = 32;            // layers per launch (kernargs)
// Lanes per token and tokens per lane group.  Packing reads the cache and
// keeps four tokens' rows in flight per lane.  Unpacking reads the packet,
// usually pinned host memory, and the PCIe read path moves most with 512
// bytes per wave access (16 lanes per token, half of them idle for 128-byte
// int8 keys).  Measured on MI355X, 8 layers x 16 x 1024 int8 tokens:
// unpacking pinned packets 16 x 4 55.5 GB/s, 16 x 1 53.5, 8 x 4 46.7;
// device packets 12.8, 14.3 and 10.3 us.  Packing pinned packets 8 x 4
// 54.6 GB/s.
constexpr int kPackGroup = 8, kPackUnroll = 4;
constexpr int kUnpackGroup = 16, kUnpackUnroll = 4;

struct C8Layer {
  uint64_t keys;
  uint64_t scales;     // 0: floating keys without scales
  uint64_t block_map;  // 0: no block permutation
  int32_t key_bytes;
  int32_t slot_factor;
};

struct C8Job {
  C8Layer layer[kC8Layers];
  const int64_t *packets;   // [layers, chunks] (rows of this launch)
  const void *offsets;
  const void *counts;
  const void *slots;
  int32_t meta_i32;
  int32_t slot_i32;
  int32_t from_npu;
  int32_t fixed;
  int64_t chunks;
  int64_t capacity;
  int64_t slot_count;
  int64_t cache_slots;
};

__device__ __forceinline__ int64_t c8_index(const void *p, int is32, int64_t i) {
  return is32 ? static_cast<int64_t>(static_cast<const int32_t *>(p)[i])
              : static_cast<const int64_t *>(p)[i];
}

// Grid (tiles of kC8Tokens tokens, chunks, layers).  A group of kC8Group
// lanes owns kC8Unroll tokens of the tile, 64 / kC8Group apart; a wave owns
// 64 / kC8Group x kC8Unroll consecutive tokens.  Each lane issues every key load of the group's tokens (one or two 16-byte
// accesses per token for 128- or 256-byte keys), then the stores; lane u of
// the group moves token u's 2-byte scale.
// Key rows are stored with the streaming hint when the destination is the
// cache (unpacking), which is always device memory; packing writes packets
// that may be page-locked host memory (the packet table holds device
// values, so the host cannot tell), and stores there keep the plain form.
// Measured on MI355X (8 layers x 16384 tokens, three runs each): unpack
// from device packets 0.0124 -> 0.0110 ms, from pinned packets unchanged
// (0.307 ms); streaming stores into device packets 0.0106 -> 0.0094 ms but
// into pinned packets 0.312 -> 0.362 ms.
template <bool kNtStores, typename T> __device__ __forceinline__ void c8_st(T *p, T v) {
  if constexpr (kNtStores) gstore_nt(p, v); else gstore(p, v);
}

template <int kC8Group, int kC8Unroll, bool kNtStores>
__global__ void __launch_bounds__(kC8Threads) indexer_c8_copy(C8Job job) {
  using V = unsigned int __attribute__((ext_vector_type(4)));
  constexpr int kKeyVecs = 256 / 16 / kC8Group;  // per lane, widest key row
  constexpr int kC8Tokens = kC8Threads / kC8Group * kC8Unroll;
  const int64_t c = blockIdx.y;
  const int li = blockIdx.z;
  const C8Layer &L = job.layer[li];
  constexpr int kGroupsPerWave = 64 / kC8Group;
  const int gl = threadIdx.x % kC8Group;
  const int gw = (threadIdx.x & 63) / kC8Group;
  const int wave = threadIdx.x >> 6;
  const int64_t start = job.fixed ? c * job.capacity : c8_index(job.offsets, job.meta_i32, c);
  const int64_t remaining = job.slot_count - start;
  const int64_t count = job.fixed ? (remaining < job.capacity ? remaining : job.capacity)
                                  : c8_index(job.counts, job.meta_i32, c);
  const uint64_t packet = static_cast<uint64_t>(job.packets[li * job.chunks + c]);
  if (!packet || count <= 0 || count > job.capacity || start < 0 || start > job.slot_count ||
      count > job.slot_count - start)
    return;
  // Token u of this group: the wave's groups take consecutive tokens, so
  // one access instruction of the wave covers kGroupsPerWave consecutive
  // packet rows.
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kC8Tokens +
                     wave * (kGroupsPerWave * kC8Unroll) + gw;
  const auto tok = [&](int u) { return t0 + static_cast<int64_t>(u) * kGroupsPerWave; };
  if (t0 >= count) return;
  const int kb = L.key_bytes;
  const bool vec = ((packet | L.keys) & 15) == 0;
  const int nv = kb / 16;
  V x[kC8Unroll][kKeyVecs];
  // Unpacking reads the packet, whose rows do not depend on the slots:
  // those loads go out before the slot lookups.
  if (!job.from_npu && vec) {
#pragma unroll
    for (int u = 0; u < kC8Unroll; ++u) {
      if (tok(u) >= count) continue;
      const V *src = reinterpret_cast<const V *>(packet + tok(u) * kb);
#pragma unroll
      for (int k = 0; k < kKeyVecs; ++k)
        if (gl + k * kC8Group < nv) x[u][k] = gload(src + gl + k * kC8Group);
    }
  }
  int64_t phys[kC8Unroll];
#pragma unroll
  for (int u = 0; u < kC8Unroll; ++u) {
    const int64_t t = tok(u);
    phys[u] = -1;
    if (t >= count) continue;
    const int64_t slot = c8_index(job.slots, job.slot_i32, start + t);
    if (slot < 0 || slot >= job.cache_slots) continue;
    const int64_t p =
        L.block_map
            ? static_cast<int64_t>(reinterpret_cast<const int32_t *>(L.block_map)[slot / 128]) * 128 +
                  slot % 128
            : slot + (slot / 128) * (L.slot_factor - 1) * 128;
    if (p >= 0 && p < job.cache_slots * L.slot_factor) phys[u] = p;
  }
  if (vec) {
    if (job.from_npu) {
#pragma unroll
      for (int u = 0; u < kC8Unroll; ++u) {
        if (phys[u] < 0) continue;
        const V *src = reinterpret_cast<const V *>(L.keys + phys[u] * kb);
#pragma unroll
        for (int k = 0; k < kKeyVecs; ++k)
          if (gl + k * kC8Group < nv) x[u][k] = gload(src + gl + k * kC8Group);
      }
    }
#pragma unroll
    for (int u = 0; u < kC8Unroll; ++u) {
      if (phys[u] < 0) continue;
      V *dst = reinterpret_cast<V *>(job.from_npu ? packet + tok(u) * kb : L.keys + phys[u] * kb);
#pragma unroll
      for (int k = 0; k < kKeyVecs; ++k)
        if (gl + k * kC8Group < nv) c8_st<kNtStores>(dst + gl + k * kC8Group, x[u][k]);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kC8Unroll; ++u) {
      if (phys[u] < 0) continue;
      uint8_t *pk = reinterpret_cast<uint8_t *>(packet) + tok(u) * kb;
      uint8_t *ck = reinterpret_cast<uint8_t *>(L.keys) + phys[u] * kb;
      uint8_t *dst = job.from_npu ? pk : ck;
      const uint8_t *src = job.from_npu ? ck : pk;
      for (int b = gl; b < kb; b += kC8Group) dst[b] = src[b];
    }
  }
  if (L.scales && gl < kC8Unroll) {
    // lane gl moves the scale of token gl (unrolled selection keeps phys[]
    // in registers)
    int64_t ph = -1;
#pragma unroll
    for (int u = 0; u < kC8Unroll; ++u)
      if (gl == u) ph = phys[u];
    if (ph >= 0) {
      const int64_t t = tok(gl);
      uint8_t *ps = reinterpret_cast<uint8_t *>(packet) + count * kb + t * 2;
      uint8_t *cs = reinterpret_cast<uint8_t *>(L.scales) + ph * 2;
      uint8_t *d = job.from_npu ? ps : cs;
      const uint8_t *s = job.from_npu ? cs : ps;
      if ((packet & 1) == 0) {
        *reinterpret_cast<uint16_t *>(d) = *reinterpret_cast<const uint16_t *>(s);
      } else {
        d[0] = s[0];
        d[1] = s[1];
      }
    }
  }
}

// IndexerC8State's conditions (csrc/indexer_c8.cpp:13-50).  Two messages keep
// the phrases the reference's test matches ("float16 scales", "int32/int64
// vectors": tests/standalone/test_indexer_c8_native.py:100,104).
void check_state(const lmc_tensor &keys, const lmc_tensor *scales,
                 int64_t factor, const lmc_tensor *block_map) {
  check(keys.device >= 0 && (scales == nullptr || scales->device == keys.device),
        "the C8 caches are on different GPUs");
  const bool quantized = keys.dtype == LMC_I8;
  check(quantized ? scales != nullptr && scales->dtype == LMC_F16
                  : scales == nullptr && (keys.dtype == LMC_F16 || keys.dtype == LMC_BF16),
        "indexer caches: float16/bfloat16 keys without scales, or int8 keys with float16 scales");
  auto contiguous = [](const lmc_tensor &t) {
    int64_t expect = 1;
    for (int i = t.ndim - 1; i >= 0; --i) {
      if (t.sizes[i] != 1 && t.strides[i] != expect) return false;
      expect *= t.sizes[i];
    }
    return true;
  };
  check(keys.ndim == 4 && keys.sizes[0] > 0 && keys.sizes[1] == 128 && keys.sizes[2] == 1 &&
            keys.sizes[3] == 128 && contiguous(keys),
        "indexer keys are not a contiguous [blocks, 128, 1, 128] cache");
  check((factor == 1 || (factor == 2 && quantized)) && keys.sizes[0] % factor == 0,
        "indexer block factor is neither 1 nor 2 (int8 keys), or does not divide the blocks");
  check(!quantized || (scales->ndim == 4 && scales->sizes[0] == keys.sizes[0] &&
                       scales->sizes[1] == 128 && scales->sizes[2] == 1 &&
                       scales->sizes[3] == 1 && contiguous(*scales)),
        "C8 scales are not a contiguous [blocks, 128, 1, 1] cache beside the keys");
  check(block_map == nullptr ||
            (quantized && factor == 1 && block_map->device == keys.device &&
             block_map->dtype == LMC_I32 && block_map->ndim == 1 &&
             block_map->sizes[0] == keys.sizes[0] && contiguous(*block_map)),
        "C8 block map: one contiguous int32 entry per block, on the keys' GPU, "
        "for int8 keys at factor 1");
}

int64_t cache_slots_of(const lmc_tensor &keys, int64_t factor) {
  return numel(keys) / 128 / factor;
}

void check_vector(const lmc_tensor &t, int device) {
  check(t.device == device && (t.dtype == LMC_I64 || t.dtype == LMC_I32) && t.ndim == 1 &&
            (t.sizes[0] <= 1 || t.strides[0] == 1),
        "C8 slots, offsets and counts: int32/int64 vectors, contiguous, on the keys' GPU");
}

void c8_transfer(const lmc_tensor *const *keys, const lmc_tensor *const *scales,
                 const lmc_tensor *const *maps, const int64_t *factors, int n_layers,
                 const lmc_tensor &ptrs, const lmc_tensor &offs, const lmc_tensor &counts,
                 const lmc_tensor &slots, int64_t capacity, bool from_npu, bool fixed,
                 hipStream_t stream) {
  check(n_layers > 0 && keys && factors, "C8 group holds no layer");
  C8Job job;
  std::memset(&job, 0, sizeof(job));
  const lmc_tensor &k0 = deref(keys[0], "keys");
  const int dev = k0.device;
  int64_t cache_slots = -1;
  for (int l = 0; l < n_layers; ++l) {
    const lmc_tensor &k = deref(keys[l], "keys");
    const lmc_tensor *s = scales ? scales[l] : nullptr;
    const lmc_tensor *m = maps ? maps[l] : nullptr;
    check_state(k, s, factors[l], m);
    const int64_t cs = cache_slots_of(k, factors[l]);
    check(k.device == dev && (cache_slots < 0 || cs == cache_slots),
          "C8 group layers differ in GPU or in slot capacity");
    cache_slots = cs;
  }
  // csrc/indexer_c8.cpp:65-95 (a group's pointers are [layers, chunks]).
  if (n_layers > 1 || ptrs.ndim == 2) {
    check(ptrs.ndim == 2 && ptrs.sizes[0] == n_layers &&
              (ptrs.sizes[1] <= 1 || (ptrs.strides[1] == 1 && ptrs.strides[0] == ptrs.sizes[1])),
          "C8 group packet pointers are not a contiguous [layers, chunks] table");
    check(ptrs.device == dev && ptrs.dtype == LMC_I64,
          "C8 slots, offsets and counts: int32/int64 vectors, contiguous, on the keys' GPU");
  } else {
    check_vector(ptrs, dev);
  }
  check_vector(offs, dev);
  check_vector(counts, dev);
  check_vector(slots, dev);
  check(ptrs.dtype == LMC_I64 && offs.dtype == counts.dtype,
        "C8 packet pointers are not int64, or offsets and counts differ in dtype");
  const int64_t chunks = ptrs.ndim == 2 ? ptrs.sizes[1] : ptrs.sizes[0];
  check(fixed || (numel(offs) == chunks && numel(counts) == chunks),
        "C8 packet pointers, offsets and counts differ in length");
  check(capacity > 0 && capacity <= INT32_MAX, "C8 chunk capacity is not in [1, 2^31)");
  if (chunks == 0) return;
  const int64_t slot_count = numel(slots);
  check(!fixed || (slot_count + capacity - 1) / capacity == chunks,
        "C8 fixed-capacity chunks and the slot mapping differ in token count");
  check(chunks <= 65535, "C8 transfer has more chunks than one launch grid holds");
  DeviceGuard guard(dev);
  job.offsets = offs.data;
  job.counts = counts.data;
  job.slots = slots.data;
  job.meta_i32 = offs.dtype == LMC_I32;
  job.slot_i32 = slots.dtype == LMC_I32;
  job.from_npu = from_npu ? 1 : 0;
  job.fixed = fixed ? 1 : 0;
  job.chunks = chunks;
  job.capacity = capacity;
  job.slot_count = slot_count;
  job.cache_slots = cache_slots;
  const int64_t tile_tokens = from_npu ? kC8Threads / kPackGroup * kPackUnroll
                                      : kC8Threads / kUnpackGroup * kUnpackUnroll;
  const int64_t tiles = (capacity + tile_tokens - 1) / tile_tokens;
  check(tiles < (int64_t(1) << 31), "C8 chunk capacity needs more tiles than one launch holds");
  for (int l0 = 0; l0 < n_layers; l0 += kC8Layers) {
    const int nl = std::min(kC8Layers, n_layers - l0);
    C8Job j = job;
    j.packets = static_cast<const int64_t *>(ptrs.data) + static_cast<int64_t>(l0) * chunks;
    for (int i = 0; i < nl; ++i) {
      const lmc_tensor &k = *keys[l0 + i];
      C8Layer &L = j.layer[i];
      L.keys = reinterpret_cast<uint64_t>(k.data);
      L.scales = scales && scales[l0 + i] ? reinterpret_cast<uint64_t>(scales[l0 + i]->data) : 0;
      L.block_map = maps && maps[l0 + i] ? reinterpret_cast<uint64_t>(maps[l0 + i]->data) : 0;
      L.key_bytes = static_cast<int32_t>(128 * elem_size(k));
      L.slot_factor = static_cast<int32_t>(factors[l0 + i]);
    }
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(chunks), nl);
    if (from_npu)
      hipLaunchKernelGGL((indexer_c8_copy<kPackGroup, kPackUnroll, false>), grid, dim3(kC8Threads), 0, stream,
                         j);
    else
      hipLaunchKernelGGL((indexer_c8_copy<kUnpackGroup, kUnpackUnroll, true>), grid, dim3(kC8Threads), 0, stream,
                         j);
    hip_check(hipGetLastError(), "indexer_c8_copy launch");
  }
}

} // namespace
} // namespace lmc

using namespace lmc;

extern "C" {

int lmc_indexer_c8_check_state(const lmc_tensor *keys, const lmc_tensor *scales,
                               int64_t slot_factor, const lmc_tensor *block_map) {
  return guarded([&] { check_state(deref(keys, "keys"), scales, slot_factor, block_map); });
}

int lmc_indexer_c8_transfer(const lmc_tensor *const *keys, const lmc_tensor *const *scales,
                            const lmc_tensor *const *block_maps, const int64_t *slot_factors,
                            int32_t n_layers, const lmc_tensor *packet_ptrs,
                            const lmc_tensor *chunk_offsets, const lmc_tensor *chunk_counts,
                            const lmc_tensor *slot_mapping, int64_t chunk_capacity,
                            int32_t from_npu, int32_t fixed_chunks, void *stream) {
  return guarded([&] {
    c8_transfer(keys, scales, block_maps, slot_factors, n_layers,
                deref(packet_ptrs, "packet_ptrs"), deref(chunk_offsets, "chunk_offsets"),
                deref(chunk_counts, "chunk_counts"), deref(slot_mapping, "slot_mapping"),
                chunk_capacity, from_npu != 0, fixed_chunks != 0,
                static_cast<hipStream_t>(stream));
  });
}

} // extern "C"
