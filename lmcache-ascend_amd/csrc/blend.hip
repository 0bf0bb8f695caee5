// Fused CacheBlend layer load for MI355X (gfx950).
//
// The blend connector's per-layer retrieve (lmcache_ascend/v1/npu_connector/
// npu_connectors.py:556-689) copies a layer's KV_2TD memory objects into a
// [2, N, W] device buffer (one copy per object and plane), zeroes the rows
// of tokens no object covers, re-rotates the K half in place with
// rotary_embedding_k_fused (csrc/pos_kernels.cpp:158-196), and scatters the
// buffer into the paged caches with single_layer_kv_transfer
// (csrc/mem_kernels.cpp:265-334, direction LMC -> paged, [2, N, W] layout).
// This kernel does the same in one pass and no buffer: each (token, plane)
// row is read from its memory object (pinned host memory over PCIe, or
// device memory), K rows are re-rotated in registers with the arithmetic of
// the K-RoPE kernel (rope_math.h), and the row is written to the paged slot;
// uncovered tokens write zero rows.  The bytes written equal the
// connector's sequence.
//
// Work mapping: a segment is one memory object or one run of uncovered
// tokens; grid.y enumerates the segments of a launch, grid.x the segment's
// tokens.  Two kernels:
//  - blend_layer_groups, for rows without re-rotation and for heads of 256
//    bytes rotated whole (the common bf16/fp16 x 128 case): a 16-lane group
//    per token moves its K row (re-rotated: neox partners sit 8 lanes apart
//    and are exchanged with one DPP rotation, GPT-J pairs are adjacent dims
//    of one lane), then its V row, one 16-byte access per lane in flight.
//  - blend_layer_rows, for the other head shapes: one wave per (token,
//    plane) row with the K and V rows of a token in adjacent waves; on K
//    rows with in-range positions lane work is a group of eight rotation
//    pairs (two 16-byte halves for neox, one 32-byte run for GPT-J), and
//    head_size - rot pass-through dims per head move as 16-byte pieces.
// Slots outside [0, num_slots) are skipped, as in the single-layer
// transfer.
#include "kv_geom.h"
#include "rope_math.h"

#include <algorithm>
#include <vector>

namespace lmc {

namespace {

constexpr int kBlendSegs = 64;    // segments per launch (kernel arguments)
constexpr int kBlendThreads = 256;
constexpr int kBlendWaves = kBlendThreads / 64;
constexpr int kVP = 8;            // rotation pairs per lane group
#ifndef LMC_BLEND_HOST_BLOCKS
#define LMC_BLEND_HOST_BLOCKS 512
#endif
constexpr int kBlendHostBlocks = LMC_BLEND_HOST_BLOCKS;  // grid cap for reads of host memory

// Rows are stored into the paged caches (device memory) with the streaming
// hint.  Measured on MI355X, one Llama-3-8B-shape layer (kernel times, two
// runs each): device objects 10.4-10.6 -> 9.3 us with re-rotation and
// 6.4 -> 5.9 us without; pinned objects unchanged (0.300 ms).
template <typename T> __device__ __forceinline__ void bst(T *p, T v) { gstore_nt(p, v); }

struct BlendSeg {
  uint64_t src;          // memory object (kernel-visible), 0 for uncovered tokens
  int64_t tok0;          // first token (index into slots / positions)
  int64_t count;         // tokens
  int64_t plane_bytes;   // bytes of one plane of the object ([2, n, W])
};

struct BlendJob {
  BlendSeg seg[kBlendSegs];
  PlaneDesc plane[2];
  uint64_t base[2];
  const void *slots;
  const void *old_pos;
  const void *new_pos;
  const void *cache;
  int64_t num_slots;
  int64_t max_pos;
  int64_t row_bytes;
  int32_t block_size;
  int32_t slot_i32;
  int32_t pos_i32;
  int32_t head_size;
  int32_t n_heads;
  int32_t rot;
};

// Whole 16-byte words of a Pack, through the global address space.
template <int N> struct Words {
  u32x4 w[N];
};
template <typename P> __device__ __forceinline__ P load_pack(const void *p) {
  static_assert(sizeof(P) % 16 == 0, "packs of whole 16-byte words");
  Words<sizeof(P) / 16> r;
#pragma unroll
  for (int k = 0; k < static_cast<int>(sizeof(P) / 16); ++k) r.w[k] = gload(static_cast<const u32x4 *>(p) + k);
  return __builtin_bit_cast(P, r);
}
template <typename P> __device__ __forceinline__ void store_pack(void *p, const P &v) {
  const Words<sizeof(P) / 16> r = __builtin_bit_cast(Words<sizeof(P) / 16>, v);
#pragma unroll
  for (int k = 0; k < static_cast<int>(sizeof(P) / 16); ++k) bst(static_cast<u32x4 *>(p) + k, r.w[k]);
}

// Four cos/sin values (8 bytes of bf16 / fp16, 16 of fp32), through the
// global address space.
template <typename CS> __device__ __forceinline__ Pack<CS, 4> load_half_pack(const CS *p) {
  if constexpr (sizeof(CS) == 4) {
    return __builtin_bit_cast(Pack<CS, 4>, gload(reinterpret_cast<const u32x4 *>(p)));
  } else {
    return __builtin_bit_cast(Pack<CS, 4>, gload(reinterpret_cast<const u32x2 *>(p)));
  }
}

__device__ __forceinline__ int64_t idx_at(const void *p, int is32, int64_t i) {
  return is32 ? static_cast<int64_t>(static_cast<const int32_t *>(p)[i]) : static_cast<const int64_t *>(p)[i];
}

template <typename KD, typename CD, bool NEOX, bool ROPE>
__global__ void __launch_bounds__(kBlendThreads) blend_layer_rows(const BlendJob job) {
  using V = u32x4;
  using KS = typename KD::S;
  using CS = typename CD::S;
  const BlendSeg &sg = job.seg[blockIdx.y];
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kBlendWaves + wave;
  const int64_t i = item >> 1;
  const int p = static_cast<int>(item & 1);
  if (i >= sg.count) return;
  const int64_t j = sg.tok0 + i;
  const int64_t slot = idx_at(job.slots, job.slot_i32, j);
  if (slot < 0 || slot >= job.num_slots) return;
  const PlaneDesc &pd = job.plane[p];
  int64_t poff = pd.paged_off;
  if (job.block_size > 0) {
    const uint32_t s32 = static_cast<uint32_t>(slot);
    const uint32_t bs = static_cast<uint32_t>(job.block_size);
    const uint32_t blk = s32 / bs;
    poff += static_cast<int64_t>(blk) * pd.blk_stride + static_cast<int64_t>(s32 - blk * bs) * pd.row_pitch;
  } else {
    poff += slot * pd.row_pitch;
  }
  uint8_t *dst = reinterpret_cast<uint8_t *>(job.base[p]) + poff;
  const int64_t rb = job.row_bytes;
  if (sg.src == 0) {  // a token no object covers: a zero row
    const V z = {0u, 0u, 0u, 0u};
    for (int64_t o = static_cast<int64_t>(lane) * 16; o < rb; o += 64 * 16)
      bst(reinterpret_cast<V *>(dst + o), z);
    return;
  }
  const uint8_t *src = reinterpret_cast<const uint8_t *>(sg.src) + p * sg.plane_bytes + i * rb;
  if constexpr (ROPE) {
    if (p == 0) {
      const int64_t po = idx_at(job.old_pos, job.pos_i32, j);
      const int64_t pn = idx_at(job.new_pos, job.pos_i32, j);
      if (po >= 0 && po < job.max_pos && pn >= 0 && pn < job.max_pos) {
        const int half = job.rot / 2;
        const int gph = half / kVP;  // pair groups per head
        const int groups = job.n_heads * gph;
        const CS *crow_o = static_cast<const CS *>(job.cache) + po * job.rot;
        const CS *crow_n = static_cast<const CS *>(job.cache) + pn * job.rot;
        const KS *ks = reinterpret_cast<const KS *>(src);
        KS *kd = reinterpret_cast<KS *>(dst);
        for (int g = lane; g < groups; g += 64) {
          const int h = g / gph;
          const int i0 = (g - h * gph) * kVP;
          const int64_t hb = static_cast<int64_t>(h) * job.head_size;
          const Pack<CS, kVP> co = load_pack<Pack<CS, kVP>>(crow_o + i0);
          const Pack<CS, kVP> so = load_pack<Pack<CS, kVP>>(crow_o + half + i0);
          const Pack<CS, kVP> cn = load_pack<Pack<CS, kVP>>(crow_n + i0);
          const Pack<CS, kVP> sn = load_pack<Pack<CS, kVP>>(crow_n + half + i0);
          float x1[kVP], x2[kVP], z1[kVP], z2[kVP];
          if constexpr (NEOX) {
            const Pack<KS, kVP> a = load_pack<Pack<KS, kVP>>(ks + hb + i0);
            const Pack<KS, kVP> b = load_pack<Pack<KS, kVP>>(ks + hb + half + i0);
#pragma unroll
            for (int v = 0; v < kVP; ++v) {
              x1[v] = to_f32<KD>(a.v[v]);
              x2[v] = to_f32<KD>(b.v[v]);
            }
          } else {
            const Pack<KS, 2 * kVP> ab = load_pack<Pack<KS, 2 * kVP>>(ks + hb + 2 * i0);
#pragma unroll
            for (int v = 0; v < kVP; ++v) {
              x1[v] = to_f32<KD>(ab.v[2 * v]);
              x2[v] = to_f32<KD>(ab.v[2 * v + 1]);
            }
          }
          rerotate<CD, kVP>(x1, x2, co, so, cn, sn, z1, z2);
          if constexpr (NEOX) {
            Pack<KS, kVP> a, b;
#pragma unroll
            for (int v = 0; v < kVP; ++v) {
              a.v[v] = from_f32<KD>(z1[v]);
              b.v[v] = from_f32<KD>(z2[v]);
            }
            store_pack(kd + hb + i0, a);
            store_pack(kd + hb + half + i0, b);
          } else {
            Pack<KS, 2 * kVP> ab;
#pragma unroll
            for (int v = 0; v < kVP; ++v) {
              ab.v[2 * v] = from_f32<KD>(z1[v]);
              ab.v[2 * v + 1] = from_f32<KD>(z2[v]);
            }
            store_pack(kd + hb + 2 * i0, ab);
          }
        }
        // Dims past the rotary dims of each head pass through.
        const int pass = (job.head_size - job.rot) * static_cast<int>(sizeof(KS)) / 16;  // pieces per head
        for (int q = lane; q < job.n_heads * pass; q += 64) {
          const int h = q / pass;
          const int64_t o = (static_cast<int64_t>(h) * job.head_size + job.rot) * static_cast<int64_t>(sizeof(KS)) +
                            static_cast<int64_t>(q - h * pass) * 16;
          bst(reinterpret_cast<V *>(dst + o), gload(reinterpret_cast<const V *>(src + o)));
        }
        return;
      }
    }
  }
  // V rows, K rows without re-rotation and K rows whose positions lie
  // outside the cache (left unchanged, as the K-RoPE kernel leaves them).
  V v[2];
  const int64_t o0 = static_cast<int64_t>(lane) * 16, o1 = o0 + 64 * 16;
  if (o0 < rb) v[0] = gload(reinterpret_cast<const V *>(src + o0));
  if (o1 < rb) v[1] = gload(reinterpret_cast<const V *>(src + o1));
  if (o0 < rb) bst(reinterpret_cast<V *>(dst + o0), v[0]);
  if (o1 < rb) bst(reinterpret_cast<V *>(dst + o1), v[1]);
  for (int64_t o = o0 + 2 * 64 * 16; o < rb; o += 64 * 16)
    bst(reinterpret_cast<V *>(dst + o), gload(reinterpret_cast<const V *>(src + o)));
}

// Tokens by 16-lane groups, for rows without re-rotation and for K rows
// whose heads are 256 bytes with every dim rotated (128 bf16 / fp16 dims:
// the 16 lanes' 16-byte accesses cover one head).  A group walks the
// token's K row, then its V row, kU 16-byte accesses per lane in flight,
// and the groups stride over the segment's tokens.  Objects in page-locked
// host memory take kU = 1: reads over PCIe move the most bytes with few
// reads in flight (the copy kernels of kv_direct.hip measured the same);
// objects in device memory take kU = 8 (a 2 KiB row per group in one
// pass).  Neox pairs (i, i + 64) sit in lanes q and q ^ 8 of a head: one
// DPP rotation by 8 within the 16-lane row gives each lane its partner's
// values, and each lane writes its own half.  GPT-J pairs are adjacent
// dims, four whole pairs per lane.  The cos/sin values a lane needs are the
// same for every head of the token and are loaded once.
template <typename KD, typename CD, bool NEOX, bool ROPE, int kU>
__global__ void __launch_bounds__(kBlendThreads) blend_layer_groups(const BlendJob job) {
  using V = u32x4;
  using KS = typename KD::S;
  using CS = typename CD::S;
  constexpr int kGroups = kBlendThreads / 16;
  constexpr int kPairs = NEOX ? 8 : 4;  // rotation pairs per lane and head
  const BlendSeg &sg = job.seg[blockIdx.y];
  const int q = threadIdx.x & 15;
  const int64_t rb = job.row_bytes;
  // kU > 1 (device objects): a group owns one (token, plane) row; the four
  // groups of an even wave take the K rows of four tokens and those of the
  // next wave the same tokens' V rows, so the re-rotation runs on full
  // waves.  kU = 1: a group owns a token.
  constexpr int kRowsPerItem = kU > 1 ? 1 : 2;
  const int64_t items = kU > 1 ? (sg.count + 3) / 4 * 8 : sg.count;
  for (int64_t it = static_cast<int64_t>(blockIdx.x) * kGroups + (threadIdx.x >> 4); it < items;
       it += static_cast<int64_t>(gridDim.x) * kGroups) {
    const int64_t i = kU > 1 ? ((it >> 2) >> 1) * 4 + (it & 3) : it;
    const int p0 = kU > 1 ? static_cast<int>((it >> 2) & 1) : 0;
    if (i >= sg.count) continue;
    const int64_t j = sg.tok0 + i;
    const int64_t slot = idx_at(job.slots, job.slot_i32, j);
    // Reads that do not depend on the slot are issued before it is checked:
    // a K row's positions and, for device objects, the row's first kU
    // pieces, so the slot, position and row reads are in flight together
    // (with a 2 KiB row the row loop below then loads nothing).  Measured
    // on MI355X, 32 Llama-3-8B-shape layers with device objects and
    // re-rotation, one call per layer (event time): 0.392 -> 0.363 ms.
    int64_t po = -1, pn = -1;
    if (ROPE && p0 == 0) {
      po = idx_at(job.old_pos, job.pos_i32, j);
      pn = idx_at(job.new_pos, job.pos_i32, j);
    }
    V pre[kU];
    const uint8_t *src0 = reinterpret_cast<const uint8_t *>(sg.src) + p0 * sg.plane_bytes + i * rb;
    if (kU > 1 && sg.src != 0) {
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (q * 16 + u * 256 < rb) pre[u] = gload(reinterpret_cast<const V *>(src0 + q * 16 + u * 256));
    }
    if (slot < 0 || slot >= job.num_slots) continue;
    int64_t blk = 0, in_blk = slot;
    if (job.block_size > 0) {
      const uint32_t s32 = static_cast<uint32_t>(slot);
      const uint32_t bs = static_cast<uint32_t>(job.block_size);
      blk = s32 / bs;
      in_blk = s32 - static_cast<uint32_t>(blk) * bs;
    }
    bool rotate = false;
    Pack<CS, kPairs> co{}, so{}, cn{}, sn{};
    if (ROPE && p0 == 0) {
      rotate = sg.src != 0 && po >= 0 && po < job.max_pos && pn >= 0 && pn < job.max_pos;
      if (rotate) {
        const CS *crow_o = static_cast<const CS *>(job.cache) + po * job.rot;
        const CS *crow_n = static_cast<const CS *>(job.cache) + pn * job.rot;
        const int i0 = NEOX ? (q & 7) * 8 : q * 4;
        if constexpr (NEOX) {
          co = load_pack<Pack<CS, 8>>(crow_o + i0);
          so = load_pack<Pack<CS, 8>>(crow_o + job.rot / 2 + i0);
          cn = load_pack<Pack<CS, 8>>(crow_n + i0);
          sn = load_pack<Pack<CS, 8>>(crow_n + job.rot / 2 + i0);
        } else {
          co = load_half_pack<CS>(crow_o + i0);
          so = load_half_pack<CS>(crow_o + job.rot / 2 + i0);
          cn = load_half_pack<CS>(crow_n + i0);
          sn = load_half_pack<CS>(crow_n + job.rot / 2 + i0);
        }
      }
    }
    // The item's rows: the token's K row, then its V row (or the one row).
    for (int r = 0; r < kRowsPerItem; ++r) {
      const int p = p0 + r;
      const PlaneDesc &pd = job.plane[p];
      uint8_t *dst = reinterpret_cast<uint8_t *>(job.base[p]) + pd.paged_off + blk * pd.blk_stride +
                     in_blk * pd.row_pitch;
      if (sg.src == 0) {  // a token no object covers: zero rows
        const V z = {0u, 0u, 0u, 0u};
        for (int64_t o = static_cast<int64_t>(q) * 16; o < rb; o += 256) bst(reinterpret_cast<V *>(dst + o), z);
        continue;
      }
      const uint8_t *src = reinterpret_cast<const uint8_t *>(sg.src) + p * sg.plane_bytes + i * rb;
      const bool rot_row = ROPE && p == 0 && rotate;
#pragma unroll 1
      for (int64_t base = static_cast<int64_t>(q) * 16; base < rb; base += kU * 256) {
        V raw[kU];
        if (kU > 1 && base == static_cast<int64_t>(q) * 16) {
#pragma unroll
          for (int u = 0; u < kU; ++u) raw[u] = pre[u];  // read before the slot check
        } else {
#pragma unroll
          for (int u = 0; u < kU; ++u)
            if (base + u * 256 < rb) raw[u] = gload(reinterpret_cast<const V *>(src + base + u * 256));
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int64_t o = base + u * 256;
          if (o >= rb) continue;
          V w = raw[u];
          if constexpr (ROPE) {
            // Rows that rotate are whole heads, so `o < rb` holds for all
            // 16 lanes of the group together (the DPP partner is active).
            if (rot_row) {
              const Pack<KS, 8> mine = __builtin_bit_cast(Pack<KS, 8>, w);
              Pack<KS, 8> out;
              if constexpr (NEOX) {
                V other;
#pragma unroll
                for (int k = 0; k < 4; ++k)  // row_ror:8 within the 16-lane row
                  other[k] = static_cast<uint32_t>(
                      __builtin_amdgcn_update_dpp(0, static_cast<int>(w[k]), 0x128, 0xF, 0xF, false));
                const Pack<KS, 8> part = __builtin_bit_cast(Pack<KS, 8>, other);
                const bool lo = q < 8;
                float x1[8], x2[8], z1[8], z2[8];
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                  x1[v] = to_f32<KD>(lo ? mine.v[v] : part.v[v]);
                  x2[v] = to_f32<KD>(lo ? part.v[v] : mine.v[v]);
                }
                rerotate<CD, 8>(x1, x2, co, so, cn, sn, z1, z2);
#pragma unroll
                for (int v = 0; v < 8; ++v) out.v[v] = from_f32<KD>(lo ? z1[v] : z2[v]);
              } else {
                float x1[4], x2[4], z1[4], z2[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                  x1[v] = to_f32<KD>(mine.v[2 * v]);
                  x2[v] = to_f32<KD>(mine.v[2 * v + 1]);
                }
                rerotate<CD, 4>(x1, x2, co, so, cn, sn, z1, z2);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                  out.v[2 * v] = from_f32<KD>(z1[v]);
                  out.v[2 * v + 1] = from_f32<KD>(z2[v]);
                }
              }
              w = __builtin_bit_cast(V, out);
            }
          }
          bst(reinterpret_cast<V *>(dst + o), w);
        }
      }
    }
  }
}

template <typename KD, typename CD, bool NEOX, bool ROPE>
void launch_groups(const BlendJob &job, dim3 grid, bool host_objs, hipStream_t s) {
  if (host_objs)
    hipLaunchKernelGGL((blend_layer_groups<KD, CD, NEOX, ROPE, 1>), grid, dim3(kBlendThreads), 0, s, job);
  else
    hipLaunchKernelGGL((blend_layer_groups<KD, CD, NEOX, ROPE, 8>), grid, dim3(kBlendThreads), 0, s, job);
}

template <typename KD, typename CD, bool NEOX, bool ROPE>
void launch_blend(const BlendJob &job, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((blend_layer_rows<KD, CD, NEOX, ROPE>), grid, dim3(kBlendThreads), 0, s, job);
}

template <typename KD>
void launch_blend_k(const BlendJob &job, dim3 grid, bool rope, int cache_dt, bool neox, hipStream_t s) {
  if (!rope) return launch_blend<KD, KD, true, false>(job, grid, s);
  switch (cache_dt) {
  case LMC_BF16: return neox ? launch_blend<KD, BF16, true, true>(job, grid, s)
                             : launch_blend<KD, BF16, false, true>(job, grid, s);
  case LMC_F16: return neox ? launch_blend<KD, F16, true, true>(job, grid, s)
                            : launch_blend<KD, F16, false, true>(job, grid, s);
  default: return neox ? launch_blend<KD, F32, true, true>(job, grid, s)
                       : launch_blend<KD, F32, false, true>(job, grid, s);
  }
}

template <typename KD>
void launch_groups_k(const BlendJob &job, dim3 grid, bool rope, int cache_dt, bool neox, bool host_objs,
                     hipStream_t s) {
  if (!rope) return launch_groups<KD, KD, true, false>(job, grid, host_objs, s);
  switch (cache_dt) {
  case LMC_BF16: return neox ? launch_groups<KD, BF16, true, true>(job, grid, host_objs, s)
                             : launch_groups<KD, BF16, false, true>(job, grid, host_objs, s);
  case LMC_F16: return neox ? launch_groups<KD, F16, true, true>(job, grid, host_objs, s)
                            : launch_groups<KD, F16, false, true>(job, grid, host_objs, s);
  default: return neox ? launch_groups<KD, F32, true, true>(job, grid, host_objs, s)
                       : launch_groups<KD, F32, false, true>(job, grid, host_objs, s);
  }
}

bool aligned16(uint64_t v) { return (v & 15) == 0; }

} // namespace

} // namespace lmc

using namespace lmc;

extern "C" int lmc_blend_layer_to_paged(const lmc_tensor *objects, int32_t n_objects,
                                        const int64_t *token_starts, const lmc_tensor *caches,
                                        int32_t n_caches, const lmc_tensor *slot_mapping,
                                        const lmc_tensor *old_positions, const lmc_tensor *new_positions,
                                        const lmc_tensor *cos_sin_cache, int64_t head_size, int32_t is_neox,
                                        int32_t kvcache_format, int32_t vllm_two_major, void *stream) {
  return guarded([&] {
    check(n_objects >= 0, "n_objects must be non-negative");
    check(n_objects == 0 || (objects != nullptr && token_starts != nullptr),
          "objects and token_starts are required");
    check(kvcache_format == LMC_FMT_MERGED_KV || kvcache_format == LMC_FMT_SEPARATE_KV,
          "blend_layer_to_paged: only MERGED_KV and SEPARATE_KV caches");
    const LayerGeom g = layer_geom(caches, n_caches, kvcache_format, vllm_two_major != 0, 0, 0, 0);
    check(g.n_planes == 2, "blend_layer_to_paged: caches must have a K and a V plane");
    const lmc_tensor &slots = slots_of(slot_mapping);
    check(slots.device < 0 || slots.device == g.device, "slot_mapping must be on the caches' device");
    const int64_t N = slots.sizes[0];
    const int64_t W = g.width[0];
    const int64_t es = g.es;
    const int64_t rb = W * es;
    check(g.width[1] == W, "K and V rows must have the same width");
    const int kdt = caches[0].dtype;
    const bool rope = old_positions != nullptr || new_positions != nullptr;
    BlendJob job;
    std::memset(&job, 0, sizeof(job));
    for (int p = 0; p < 2; ++p) {
      job.plane[p] = g.plane[p];
      job.base[p] = g.base[p];
    }
    job.block_size = g.block_size;
    job.num_slots = g.num_slots;
    check(g.block_size == 0 || g.num_slots <= static_cast<int64_t>(UINT32_MAX),
          "paged caches of more than 2^32 slots are not supported");
    job.slots = kernel_ptr(slots);
    job.slot_i32 = slots.dtype == LMC_I32;
    job.row_bytes = rb;
    // Segments in token order: the objects, and the runs of tokens no object
    // covers.
    std::vector<BlendSeg> segs;
    bool objs_aligned = true;
    bool host_objs = false;
    std::vector<std::pair<int64_t, int>> order;
    for (int o = 0; o < n_objects; ++o) order.emplace_back(token_starts[o], o);
    std::sort(order.begin(), order.end());
    int64_t cursor = 0;
    for (const auto &so : order) {
      const lmc_tensor &t = deref(&objects[so.second], "memory object");
      check(t.ndim == 3 && t.sizes[0] == 2 && t.sizes[2] == W,
            "memory objects must be KV_2TD [2, tokens, W] with the caches' row width");
      check(t.dtype == kdt, "memory objects must have the caches' dtype");
      check((t.sizes[1] <= 1 || t.strides[1] == W) && (W <= 1 || t.strides[2] == 1) &&
                (t.sizes[1] == 0 || t.strides[0] == t.sizes[1] * W),
            "memory objects must be contiguous");
      check(t.device < 0 || t.device == g.device,
            "memory objects must be in pinned host memory or on the caches' device");
      const int64_t n = t.sizes[1];
      const int64_t s0 = so.first;
      check(s0 >= 0, "token_starts must be non-negative");
      check(s0 >= cursor, "memory objects must not overlap");
      check(s0 + n <= N, "memory object token range exceeds slot_mapping");
      if (s0 > cursor) segs.push_back({0, cursor, s0 - cursor, 0});
      if (n > 0) {
        const uint64_t src = reinterpret_cast<uint64_t>(kernel_ptr(t));
        objs_aligned = objs_aligned && aligned16(src);
        host_objs = host_objs || t.device < 0;
        segs.push_back({src, s0, n, n * rb});
      }
      cursor = s0 + n;
    }
    if (cursor < N) segs.push_back({0, cursor, N - cursor, 0});
    // Geometry the fused kernel does not take (the Python layer then runs the
    // connector's own sequence): LMC_ERR_NOT_IMPLEMENTED, before any work.
    auto unsupported = [](const std::string &why) {
      fail(LMC_ERR_NOT_IMPLEMENTED, "blend_layer_to_paged: " + why);
    };
    if (kdt != LMC_BF16 && kdt != LMC_F16) unsupported("keys must be bf16 or fp16");
    if (!objs_aligned) unsupported("memory objects must be 16-byte aligned");
    if (rb % 16) unsupported("rows must be a multiple of 16 bytes");
    for (int p = 0; p < 2; ++p)
      if (!aligned16(job.base[p] + static_cast<uint64_t>(g.plane[p].paged_off)) ||
          (g.plane[p].blk_stride % 16) || (g.plane[p].row_pitch % 16))
        unsupported("paged rows must be 16-byte aligned");
    int cache_dt = kdt;
    if (rope) {
      const lmc_tensor &op = deref(old_positions, "old_positions");
      const lmc_tensor &np_ = deref(new_positions, "new_positions");
      const lmc_tensor &c = deref(cos_sin_cache, "cos_sin_cache");
      check(op.ndim == 1 && np_.ndim == 1 && op.sizes[0] == N && np_.sizes[0] == N,
            "positions must be 1-D with one entry per token");
      check(op.dtype == np_.dtype && (op.dtype == LMC_I64 || op.dtype == LMC_I32),
            "positions must both be int64 or int32");
      check((N <= 1 || (op.strides[0] == 1 && np_.strides[0] == 1)), "positions must be contiguous");
      check(op.device == g.device && np_.device == g.device && c.device == g.device,
            "positions and cos_sin_cache must be on the caches' device");
      check(c.ndim >= 1, "cos_sin_cache must have a last dimension");
      const int64_t rot = size(c, -1);
      check(head_size > 0 && W % head_size == 0, "key width is not a multiple of head_size");
      check(rot > 0 && rot % 2 == 0 && rot <= head_size, "rotary dim must be even and at most head_size");
      check(c.ndim == 1 || stride(c, -1) == 1, "cos_sin_cache must be contiguous");
      if (c.ndim >= 2) check(stride(c, -2) == rot, "cos_sin_cache must be contiguous");
      cache_dt = c.dtype;
      if (cache_dt != LMC_BF16 && cache_dt != LMC_F16 && cache_dt != LMC_F32)
        fail(LMC_ERR_RUNTIME, "cos_sin_cache dtype must be bf16, fp16 or fp32");
      const int64_t ces = elem_size(c);
      if ((rot / 2) % kVP) unsupported("rotary half must be a multiple of 8 dims");
      if (((head_size - rot) * es) % 16) unsupported("pass-through dims must be a multiple of 16 bytes");
      if ((head_size * es) % 16) unsupported("heads must be a multiple of 16 bytes");
      if (!aligned16(reinterpret_cast<uint64_t>(c.data)) || (rot * ces) % 16)
        unsupported("cos_sin_cache rows must be 16-byte aligned");
      job.old_pos = kernel_ptr(op);
      job.new_pos = kernel_ptr(np_);
      job.pos_i32 = op.dtype == LMC_I32;
      job.cache = kernel_ptr(c);
      job.max_pos = numel(c) / rot;
      job.rot = static_cast<int32_t>(rot);
      job.head_size = static_cast<int32_t>(head_size);
      job.n_heads = static_cast<int32_t>(W / head_size);
    }
    if (segs.empty()) return;
    // 16-lane groups unless K rows need the general re-rotation (heads
    // other than 256 bytes, or pass-through dims).
    const bool groups = !rope || (job.rot == job.head_size && job.head_size * es == 256);
    DeviceGuard guard(g.device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (size_t b = 0; b < segs.size(); b += kBlendSegs) {
      const size_t n = std::min<size_t>(kBlendSegs, segs.size() - b);
      int64_t most = 0;
      for (size_t k = 0; k < n; ++k) {
        job.seg[k] = segs[b + k];
        most = std::max(most, segs[b + k].count);
      }
      if (groups) {
        // A group per token (host objects) or per (token, plane) row (device
        // objects); reads of host memory: at most kBlendHostBlocks blocks in
        // all.
        const int64_t items = host_objs ? most : (most + 3) / 4 * 8;
        int64_t gx = (items + kBlendThreads / 16 - 1) / (kBlendThreads / 16);
        if (host_objs) gx = std::min<int64_t>(gx, std::max<int64_t>(1, kBlendHostBlocks / static_cast<int64_t>(n)));
        check(gx < (int64_t(1) << 31), "blend_layer_to_paged: too many tokens");
        const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(n));
        if (kdt == LMC_BF16) launch_groups_k<BF16>(job, grid, rope, cache_dt, is_neox != 0, host_objs, s);
        else launch_groups_k<F16>(job, grid, rope, cache_dt, is_neox != 0, host_objs, s);
      } else {
        const int64_t gx = (2 * most + kBlendWaves - 1) / kBlendWaves;
        check(gx < (int64_t(1) << 31), "blend_layer_to_paged: too many tokens");
        const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(n));
        if (kdt == LMC_BF16) launch_blend_k<BF16>(job, grid, rope, cache_dt, is_neox != 0, s);
        else launch_blend_k<F16>(job, grid, rope, cache_dt, is_neox != 0, s);
      }
      hip_check(hipGetLastError(), "blend_layer_to_paged launch");
    }
  });
}
