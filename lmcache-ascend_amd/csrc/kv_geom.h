// Geometry shared by the gather/scatter kernels: per-plane byte geometry of
// the LMCache and paged sides, vector access types, and the paged-cache
// planner for one layer of vLLM caches (csrc/utils.cpp:212-406, 903-966).
#pragma once

#include "common.h"
#include "gmem.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace lmc {

constexpr int kMaxPlanes = 3;

// Byte geometry of one plane (K, V or DSA) of a copy.
struct PlaneDesc {
  int64_t row_bytes;           // bytes per row
  // LMCache side.  Offsets depend on the chunk's token count T (multi-layer
  // memory objects are [kv, L, T, W]), so each is fixed + per_T * T.
  int64_t lmc_off_fixed;
  int64_t lmc_off_per_t;
  int64_t lmc_layer_fixed;
  int64_t lmc_layer_per_t;
  int64_t lmc_token_stride;
  // Paged side: row(s) = base + paged_off + (s / BS) * blk_stride
  //                                        + (s % BS) * row_pitch
  // or, with block_size == 0, base + paged_off + s * row_pitch.
  int64_t paged_off;
  int64_t blk_stride;
  int64_t row_pitch;
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int VEC> struct VecOf;
template <> struct VecOf<16> { using T = u32x4; };
template <> struct VecOf<8> { using T = u32x2; };
template <> struct VecOf<4> { using T = uint32_t; };
template <> struct VecOf<2> { using T = uint16_t; };
template <> struct VecOf<1> { using T = uint8_t; };

#ifndef LMC_KV_NT_LOADS
#define LMC_KV_NT_LOADS 1         // streaming hint on loads of HBM copies
#endif
#ifndef LMC_KV_NT_STORES
#define LMC_KV_NT_STORES 1        // streaming hint on stores of HBM copies
#endif

// Loads and stores through the global address space (gmem.h).
template <typename T, bool NT> __device__ __forceinline__ T ld(const T *p) {
  if constexpr (NT && LMC_KV_NT_LOADS)
    return __builtin_nontemporal_load(
        reinterpret_cast<const __attribute__((address_space(1))) T *>(reinterpret_cast<uintptr_t>(p)));
  else return gload(p);
}
typedef __attribute__((address_space(1))) u32x4 GlobalU32x4;

#ifndef LMC_KV_WT_STORES
#define LMC_KV_WT_STORES 1        // device-scope write-through 16-byte stores
#endif

// Stores of HBM-only copies.  With WT a 16-byte store is issued at device
// (agent) scope, which writes through the XCD's L2 instead of leaving the
// line dirty there, so the kernel's end-of-launch L2 write-back has nothing
// left to flush; without it (and for narrower vectors) the store carries the
// streaming hint.  Which is faster depends on the kernel (MI355X, three
// interleaved runs each): the row kernels are faster with streaming stores
// (8B shape, 16 objects in one launch 0.172 -> 0.170 ms per direction; 32
// per-layer flash stores 0.259 -> 0.244 ms; Qwen3-32B shape, 128 objects
// stored in one launch 2.82 -> 2.70 ms), the tile kernel's stores to
// memory objects are faster written through (MLA-576 store 0.388 -> 0.402
// ms with streaming stores), and the direct kernels measure the same.
template <typename T, bool NT, bool WT = true> __device__ __forceinline__ void st(T *p, T v) {
  if constexpr (NT && WT && LMC_KV_WT_STORES && sizeof(T) == 16)
    __builtin_amdgcn_global_store_b128((GlobalU32x4 *)(p),
                                       __builtin_bit_cast(u32x4, v), "agent");
  else if constexpr (NT && LMC_KV_NT_STORES)
    __builtin_nontemporal_store(v, reinterpret_cast<__attribute__((address_space(1))) T *>(reinterpret_cast<uintptr_t>(p)));
  else gstore(p, v);
}

inline int64_t gcd64(int64_t a, int64_t b) {
  a = a < 0 ? -a : a;
  b = b < 0 ? -b : b;
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Widest access (16/8/4/2/1 bytes) dividing g (0 counts as 16).
inline int vec_for(int64_t g) {
  if (g == 0 || g % 16 == 0) return 16;
  if (g % 8 == 0) return 8;
  if (g % 4 == 0) return 4;
  if (g % 2 == 0) return 2;
  return 1;
}

inline bool is_mla_dsa(int fmt) {
  return fmt == LMC_FMT_MLA_KV || fmt == LMC_FMT_DSA_KV ||
         fmt == LMC_FMT_MLA_LATENT || fmt == LMC_FMT_DSA_INDEX;
}

// Streaming cache hints for HBM-only copies (LMC_AMD_NONTEMPORAL=0 turns
// them off).
bool nontemporal_enabled();

// Checks a 1-D contiguous int32/int64 slot_mapping tensor and returns it.
const lmc_tensor &slots_of(const lmc_tensor *s);

// The reference's format / cache-tuple checks (csrc/utils.cpp:903-966),
// in this library's words; ValueError on failure.
void validate_vllm_caches(const lmc_tensor *caches, int n, int fmt);

// Paged side of one layer's vLLM caches.  Planes are those present in the
// format (K, V, DSA for MLA/DSA; K, V for MERGED/SEPARATE); `plane[p]`
// carries row_bytes and the paged fields, `prefix[p]` the plane's element
// column inside an LMC token's [K | V | DSA] (MLA/DSA) and `width[p]` its
// elements per row.
struct LayerGeom {
  PlaneDesc plane[kMaxPlanes];
  uint64_t base[kMaxPlanes];
  int64_t width[kMaxPlanes];
  int64_t prefix[kMaxPlanes];
  int n_planes;
  int block_size;          // 0: flat rows (MLA/DSA caches viewed as [-1, W])
  int64_t num_slots;       // valid slots are [0, num_slots)
  int64_t es;              // element size
  int64_t plane_elems;     // elements of one LMC token over all planes
  int device;
  bool mla_dsa;
};

// Validates `caches` for `fmt` and resolves the MLA/DSA hidden-dim defaults
// (csrc/utils.cpp:310-339).
LayerGeom layer_geom(const lmc_tensor *caches, int n, int fmt, bool two_major,
                     int64_t kH, int64_t vH, int64_t dsaH);

// LMC side of a single-layer buffer: sets pl[p].lmc_off_fixed and
// lmc_token_stride for the planes of `g` (MLA/DSA stacked planes; otherwise
// [T, 2, W] or [2, T, W] by strides) and returns the tokens it holds.
int64_t single_layer_lmc(const LayerGeom &g, const lmc_tensor &lmc,
                         bool token_major, PlaneDesc *pl);

// single_layer_kv_transfer (csrc/mem_kernels.cpp:265-334) on `stream`.
void single_layer(const lmc_tensor *lmc, const lmc_tensor *caches, int n,
                  const lmc_tensor *slots, bool direction, int fmt,
                  bool token_major, bool two_major, int64_t kH, int64_t vH,
                  int64_t dsaH, hipStream_t stream);

} // namespace lmc
