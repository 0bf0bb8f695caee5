// Code lengths of calculate_cdf's optimal alphabetic codes on the GPU.
//
// Rule L4 takes, for a stream with m >= 2 present symbols, the leaf depths
// of the Garsia-Wachs combination tree over the present symbols' counts in
// symbol order (A. M. Garsia and M. L. Wachs, "A new algorithm for minimum
// cost binary trees", SIAM J. Comput. 6(4), 1977): while more than one item
// is left, the first pair (x, y) of a triple x, y, z of consecutive weights
// with x <= z, taken from the left (the last pair when no triple qualifies),
// is combined and the combination re-inserted right after the nearest item
// to its left whose weight is >= x + y (at the front when there is none).
//
// The list lives in registers.  An item packs its weight with the set of
// leaves (present-symbol indices) below it, so that combining two items is
// one addition (the leaf sets are disjoint); leaf depths are counted in
// bit-sliced counters indexed by leaf.  A stream owns Q lanes (1, or a DPP
// quad): list position q is slot q / Q of lane q % Q, so a combination step
// costs each lane about 1/Q of the list, and the neighbours at q - 1, q + 1
// and q + 2 arrive by quad permutations.  Positions past the list hold an
// infinite weight, so every step processes a fixed number of slots; the
// list shrinks by one per step and the slot count with it, in phases.
#pragma once

#include <stdint.h>

#include <type_traits>

namespace lmc {
namespace cggw {

// Up to 16 leaves and weights below 2^16: (weight << 16) | leaves.
// kInf is the padding items' weight, above every real one.
struct Item16 {
  using V = uint32_t;
  using L = uint32_t;
  static constexpr uint32_t kInf = 0xFFFFu;
  static __device__ __forceinline__ V leaf(uint32_t w, int j) { return (w << 16) | (1u << j); }
  static __device__ __forceinline__ V inf() { return 0xFFFFFFFFu; }
  static __device__ __forceinline__ uint32_t weight(V v) { return v >> 16; }
  static __device__ __forceinline__ L leaves(V v) { return v & 0xFFFFu; }
  static __device__ __forceinline__ V add(V a, V b) { return a + b; }
  static __device__ __forceinline__ V zero() { return 0u; }
  static __device__ __forceinline__ V bor(V a, V b) { return a | b; }
};

// Up to 32 leaves: (weight << 32) | leaves.
struct Item32 {
  using V = uint64_t;
  using L = uint32_t;
  static constexpr uint32_t kInf = 0xFFFFFFFFu;
  static __device__ __forceinline__ V leaf(uint32_t w, int j) {
    return (static_cast<uint64_t>(w) << 32) | (1u << j);
  }
  static __device__ __forceinline__ V inf() { return ~0ull; }
  static __device__ __forceinline__ uint32_t weight(V v) { return static_cast<uint32_t>(v >> 32); }
  static __device__ __forceinline__ L leaves(V v) { return static_cast<uint32_t>(v); }
  static __device__ __forceinline__ V add(V a, V b) { return a + b; }
  static __device__ __forceinline__ V zero() { return 0ull; }
  static __device__ __forceinline__ V bor(V a, V b) { return a | b; }
};

// Up to 64 leaves: the leaf set and the weight side by side.
struct Item64 {
  struct V {
    uint64_t m;
    uint32_t w;
  };
  using L = uint64_t;
  static constexpr uint32_t kInf = 0xFFFFFFFFu;
  static __device__ __forceinline__ V leaf(uint32_t w, int j) { return V{1ull << j, w}; }
  static __device__ __forceinline__ V inf() { return V{0ull, kInf}; }
  static __device__ __forceinline__ uint32_t weight(V v) { return v.w; }
  static __device__ __forceinline__ L leaves(V v) { return v.m; }
  static __device__ __forceinline__ V add(V a, V b) { return V{a.m | b.m, a.w + b.w}; }
  static __device__ __forceinline__ V zero() { return V{0ull, 0u}; }
  static __device__ __forceinline__ V bor(V a, V b) { return V{a.m | b.m, a.w | b.w}; }
};

// Quad permutations: lane g of each group of four reads lane PERM[g].
constexpr int kRot1 = 0x39;  // [1, 2, 3, 0]: the next lane
constexpr int kRot2 = 0x4E;  // [2, 3, 0, 1]
constexpr int kRot3 = 0x93;  // [3, 0, 1, 2]: the previous lane
constexpr int kSwap = 0xB1;  // [1, 0, 3, 2]

// Every lane of a quad is a valid source, so no value for invalid lanes is
// needed (bound_ctrl set: no old value tied to the destination).
template <int CTRL>
__device__ __forceinline__ uint32_t qp(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint64_t qp(uint64_t v) {
  return (static_cast<uint64_t>(qp<CTRL>(static_cast<uint32_t>(v >> 32))) << 32) | qp<CTRL>(static_cast<uint32_t>(v));
}
template <int CTRL>
__device__ __forceinline__ Item64::V qp(Item64::V v) {
  return Item64::V{qp<CTRL>(v.m), qp<CTRL>(v.w)};
}

// A quad permutation whose result is then selected per lane.  The empty
// asm makes every lane execute the permutation: the compiler would
// otherwise fold the select into the permutation under a reduced exec
// mask, and a permutation reads 0 from the lanes that mask turns off.
template <int CTRL>
__device__ __forceinline__ uint32_t qps(uint32_t v) {
  uint32_t r = qp<CTRL>(v);
  asm volatile("" : "+v"(r));
  return r;
}

__device__ __forceinline__ uint32_t quad_min(uint32_t v) {
  v = min(v, qp<kSwap>(v));
  return min(v, qp<kRot2>(v));
}
__device__ __forceinline__ uint32_t quad_max(uint32_t v) {
  v = max(v, qp<kSwap>(v));
  return max(v, qp<kRot2>(v));
}
template <class It>
__device__ __forceinline__ typename It::V quad_or(typename It::V v) {
  v = It::bor(v, qp<kSwap>(v));
  return It::bor(v, qp<kRot2>(v));
}

// Per-slot conditions as VGPR words.  A compare writes an SGPR lane mask
// that a select may read only two wait states later, and the list update
// is a run of compare-select pairs on one mask register, so each pair
// waited; a slot's condition is instead bit i of a per-lane word, spread
// to a lane mask by a bit-field extract and applied by v_bfi_b32.
// All ones where bit i of `bits` is set (i a constant after unrolling).
__device__ __forceinline__ uint32_t bit_mask(uint32_t bits, int i) {
  return static_cast<uint32_t>(static_cast<int32_t>(bits << (31 - i)) >> 31);
}
// The same as one v_bfe_i32 written as asm, for words that are shifts of
// all ones, whose extract the compiler otherwise rewrites into two shifts
// per slot.
__device__ __forceinline__ uint32_t bit_mask1(uint32_t bits, int i) {
  uint32_t r;
  asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(r) : "v"(bits), "i"(i));
  return r;
}
// Bitwise m ? x : y.  Written as asm: the compiler turns the C form of a
// select on a sign mask back into a compare and an SGPR select.
__device__ __forceinline__ uint32_t bsel(uint32_t m, uint32_t x, uint32_t y) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(x), "v"(y));
  return r;
}
// Bit length of x: 0 for 0, else 1 + the index of the highest set bit.
__device__ __forceinline__ int bit_length(uint32_t x) { return 32 - static_cast<int>(__builtin_clzg(x, 32)); }

// The re-insertion point and the new list of a step for 32-bit items
// whose weight is the top 16 bits (Item16, ItemId): `kg` = k - g, `sum`
// the combined item.  Slot i holds position Q * i + g.  The point is
// right after the last position before k whose weight is >= sum's (0
// when none is): the sign bits of weight - sw, one per slot, are gathered
// into a word by funnel shifts, and the last slot that qualifies is the
// word's bit length.  The new list keeps [0, p), puts sum at p, takes
// (p, k] from one position to the left and the rest from one position to
// the right; each slot's three choices are selects on bits of per-lane
// threshold words.
template <int Q, int S, int CAP>
__device__ __forceinline__ void reinsert32(uint32_t (&a)[CAP], const uint32_t (&dn1)[S], const uint32_t (&up1)[S],
                                           int g, int kg, uint32_t sum) {
  static_assert(Q == 1 || Q == 4, "lanes per stream");
  constexpr int kLog = Q == 4 ? 2 : 0;
  const uint32_t sw = sum >> 16;
  uint32_t light = 0;  // bit i: slot i's weight is below sw
#pragma unroll
  for (int i = S - 1; i >= 0; --i) light = __builtin_amdgcn_alignbit(light, (a[i] >> 16) - sw, 31);
  // Slots before k: Q * i < kg, i < ceil(kg / Q) (kg >= 1 - Q).
  const uint32_t before_k = (1u << ((kg + Q - 1) >> kLog)) - 1u;
  const int bl = bit_length(~light & before_k);  // the last such slot + 1
  int p;
  if constexpr (Q == 1) {
    p = bl;
  } else {
    // Position 4 (bl - 1) + g + 1 of the lane's last heavy slot, or 0.
    const int pq = max(4 * bl + g - 3, 0);
    p = static_cast<int>(quad_max(static_cast<uint32_t>(pq)));
  }
  const int pg = p - g;
  const uint32_t to_left = (1u << ((kg + Q) >> kLog)) - 1u;   // Q * i <= kg
  const uint32_t keep = (1u << ((pg + Q - 1) >> kLog)) - 1u;  // Q * i < pg
  const uint32_t at_p = ((1u << ((pg + Q) >> kLog)) - 1u) ^ keep;  // Q * i == pg
  uint32_t na[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    uint32_t v = bsel(bit_mask(to_left, i), dn1[i], up1[i]);
    v = bsel(bit_mask(at_p, i), sum, v);
    na[i] = bsel(bit_mask(keep, i), a[i], v);
  }
#pragma unroll
  for (int i = 0; i < S; ++i) a[i] = na[i];
}

// Bit-sliced depth counters: bit j of d0..d3 is leaf j's depth (mod 16),
// bit j of ovf is set once it reaches 16.
template <class L>
struct Depths {
  L d0 = 0, d1 = 0, d2 = 0, d3 = 0, ovf = 0;
  // One more level for every leaf in `mm`.
  __device__ __forceinline__ void add(L mm) {
    L c = d0 & mm;
    d0 ^= mm;
    L n = d1 & c;
    d1 ^= c;
    c = d2 & n;
    d2 ^= n;
    n = d3 & c;
    d3 ^= c;
    ovf |= n;
  }
  // Leaves deeper than 12 (wide) or 8 bits.
  __device__ __forceinline__ L over(bool wide) const {
    return (wide ? (d3 & d2 & (d1 | d0)) : (d3 & (d2 | d1 | d0))) | ovf;
  }
  __device__ __forceinline__ uint32_t depth(int j) const {
    return static_cast<uint32_t>(((d0 >> j) & 1u) | (((d1 >> j) & 1u) << 1) | (((d2 >> j) & 1u) << 2) |
                                 (((d3 >> j) & 1u) << 3));
  }
};

// One combination step over a list of at most Q * S items (slots 0..S-1
// of every lane; positions from Q * S on are padding).  g: the lane's place
// in its stream's group; `active`: the stream still has two items or more.
template <int Q, int S, int CAP, class It>
__device__ __forceinline__ void step(typename It::V (&a)[CAP], int g, bool active,
                                     Depths<typename It::L> &dep) {
  using V = typename It::V;
  static_assert(S <= CAP, "slots");
  V up1[S], dn1[S];
  uint32_t up2[S];
  if constexpr (Q == 1) {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      up1[i] = i + 1 < S ? a[i + 1 < S ? i + 1 : 0] : It::inf();
      dn1[i] = i > 0 ? a[i > 0 ? i - 1 : 0] : It::inf();
      up2[i] = i + 2 < S ? It::weight(a[i + 2 < S ? i + 2 : 0]) : It::kInf;
    }
  } else {
    static_assert(Q == 4, "lanes per stream");
    V r1[S], r3[S];
    uint32_t r2[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      r1[i] = qp<kRot1>(a[i]);
      r3[i] = qp<kRot3>(a[i]);
      r2[i] = qp<kRot2>(It::weight(a[i]));
    }
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const V next1 = i + 1 < S ? r1[i + 1 < S ? i + 1 : 0] : It::inf();
      const V prev3 = i > 0 ? r3[i > 0 ? i - 1 : 0] : It::inf();
      const uint32_t next2 = i + 1 < S ? r2[i + 1 < S ? i + 1 : 0] : It::kInf;
      up1[i] = g == 3 ? next1 : r1[i];
      dn1[i] = g == 0 ? prev3 : r3[i];
      up2[i] = g >= 2 ? next2 : r2[i];
    }
  }
  // The first position k whose triple qualifies, and the combined item.
  int kslot = -1;
  V sloc = It::zero();
#pragma unroll
  for (int i = S - 1; i >= 0; --i) {
    const bool c = It::weight(a[i]) <= up2[i];
    kslot = c ? i : kslot;
    sloc = c ? It::add(a[i], up1[i]) : sloc;
  }
  int k;
  V sum;
  if constexpr (Q == 1) {
    k = kslot;
    sum = sloc;
  } else {
    const uint32_t kq = kslot >= 0 ? static_cast<uint32_t>(Q * kslot + g) : 0x3FFu;
    k = static_cast<int>(quad_min(kq));
    sum = quad_or<It>(kq == static_cast<uint32_t>(k) ? sloc : It::zero());
  }
  const int kg = k - g;
  if constexpr (std::is_same<V, uint32_t>::value) {
    reinsert32<Q, S, CAP>(a, dn1, up1, g, kg, sum);
  } else {
    // Re-insertion point: right after the last position before k whose
    // weight is >= the combined weight (0 when none is).
    const uint32_t sw = It::weight(sum);
    int pslot = -1;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const bool c = Q * i < kg && It::weight(a[i]) >= sw;
      pslot = c ? i : pslot;
    }
    int p;
    if constexpr (Q == 1) {
      p = pslot + 1;
    } else {
      const uint32_t pq = pslot >= 0 ? static_cast<uint32_t>(Q * pslot + g + 1) : 0u;
      p = static_cast<int>(quad_max(pq));
    }
    // New list: [0, p) kept, the combined item at p, (p, k] from one
    // position to the left, the rest from one position to the right (k and
    // k + 1 are gone).
    const int pg = p - g;
    V na[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      V v = Q * i <= kg ? dn1[i] : up1[i];
      v = Q * i == pg ? sum : v;
      na[i] = Q * i < pg ? a[i] : v;
    }
#pragma unroll
    for (int i = 0; i < S; ++i) a[i] = na[i];
  }
  dep.add(active ? It::leaves(sum) : typename It::L(0));
}

// Up to 32 leaves in a quad, weights below 2^16, by node id:
// (weight << 16) | id, leaves 0..31 and the node made by step t 32 + t.
// Items no longer carry their leaf sets: the stream's LDS column (stride
// 64 words) holds the set of every id, leaf j's {j} at word j and node
// 32 + t's at word 32 + t, stored by step t, so that the list moves 32-bit
// values.
struct ItemId {
  using V = uint32_t;
  using L = uint32_t;
  static constexpr uint32_t kInf = 0xFFFFu;
  static __device__ __forceinline__ V leaf(uint32_t w, int j) { return (w << 16) | static_cast<uint32_t>(j); }
  static __device__ __forceinline__ V inf() { return 0xFFFFFFFFu; }
  static __device__ __forceinline__ uint32_t weight(V v) { return v >> 16; }
};

// One combination step by node id for a quad (Q = 4) over at most 4 * S
// items; `t`: the step's index (wave-uniform), `tmax`: the last step's,
// `sets`: the stream's LDS column of leaf sets by id (33 + tmax words).  The
// list update is that of step(); the pair's leaf sets are read while the
// new list is formed, and the new node's set is stored and counted at the
// end.
template <int S, int CAP>
__device__ __forceinline__ void step_ids(uint32_t (&a)[CAP], int g, bool active, int t, int tmax, uint32_t *sets,
                                         Depths<uint32_t> &dep) {
  constexpr int Q = 4;
  using It = ItemId;
  static_assert(S <= CAP, "slots");
  uint32_t up1[S], dn1[S], up2[S];
  {
    uint32_t r1[S], r2[S], r3[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      r1[i] = qps<kRot1>(a[i]);
      r3[i] = qps<kRot3>(a[i]);
      r2[i] = qps<kRot2>(a[i]);
    }
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const uint32_t next1 = i + 1 < S ? r1[i + 1 < S ? i + 1 : 0] : It::inf();
      const uint32_t prev3 = i > 0 ? r3[i > 0 ? i - 1 : 0] : It::inf();
      const uint32_t next2 = i + 1 < S ? r2[i + 1 < S ? i + 1 : 0] : It::inf();
      up1[i] = g == 3 ? next1 : r1[i];
      dn1[i] = g == 0 ? prev3 : r3[i];
      up2[i] = g >= 2 ? next2 : r2[i];
    }
  }
  // The first position k whose triple qualifies, and the pair there.
  int kslot = -1;
  uint32_t xs = 0, ys = 0;
#pragma unroll
  for (int i = S - 1; i >= 0; --i) {
    const bool c = It::weight(a[i]) <= It::weight(up2[i]);
    kslot = c ? i : kslot;
    xs = c ? a[i] : xs;
    ys = c ? up1[i] : ys;
  }
  const uint32_t kq = kslot >= 0 ? static_cast<uint32_t>(Q * kslot + g) : 0x3FFu;
  const int k = static_cast<int>(quad_min(kq));
  const bool own = kq == static_cast<uint32_t>(k);
  const uint32_t x = quad_or<Item16>(own ? xs : 0u);
  const uint32_t y = quad_or<Item16>(own ? ys : 0u);
  // The pair's leaf sets, by id (ids clamped for the padding items of a
  // finished stream).
  const uint32_t top = static_cast<uint32_t>(32 + tmax);
  const uint32_t ix = min(x & 0xFFFFu, top), iy = min(y & 0xFFFFu, top);
  const uint32_t sx = sets[ix * 64];
  const uint32_t sy = sets[iy * 64];
  const uint32_t sw = It::weight(x) + It::weight(y);
  const uint32_t sum = (sw << 16) | static_cast<uint32_t>(32 + t);
  reinsert32<Q, S, CAP>(a, dn1, up1, g, k - g, sum);
  const uint32_t set = sx | sy;
  sets[(32 + t) * 64] = set;
  dep.add(active ? set : 0u);
}

// Combination steps while the wave's longest list has more than Q * (S - 1)
// items, then the phase with one slot fewer.  M: the wave's longest list
// (wave-uniform); t: steps taken; m_lane: this stream's present symbols.
template <int Q, int S, int CAP, class It>
__device__ __forceinline__ void phases(typename It::V (&a)[CAP], int g, int m_lane, int &M, int &t, int tmax,
                                       Depths<typename It::L> &dep, uint32_t *sets) {
  if constexpr (S >= 1) {
    while (M >= 2 && M > Q * (S - 1)) {
      if constexpr (std::is_same<It, ItemId>::value)
        step_ids<S, CAP>(a, g, t < m_lane - 1, t, tmax, sets, dep);
      else
        step<Q, S, CAP, It>(a, g, t < m_lane - 1, dep);
      --M;
      ++t;
    }
    phases<Q, S - 1, CAP, It>(a, g, m_lane, M, t, tmax, dep, sets);
  }
}

// Lane-major quads for ItemId.  With S slots a lane, list position q is
// slot q % S of lane q / S, so the neighbours at q - 1, q + 1 and q + 2 are
// the lane's own registers except across a lane boundary, where three quad
// permutations a step bring them (against three permutations and three
// selects a slot in the interleaved layout).  When the list has shrunk by
// four positions, the items move to the layout with one slot fewer
// (repack_lm); with one slot both layouts are the same.

// The re-insertion point and the new list in the lane-major layout: `base`
// is this lane's first position (g S).
template <int S, int CAP>
__device__ __forceinline__ void reinsert_lm(uint32_t (&a)[CAP], const uint32_t (&dn1)[S], const uint32_t (&up1)[S],
                                            int base, int k, uint32_t sum) {
  // Positions are below 4 S <= 32 and k <= 4 S - 2, so every shift below
  // is at most 31; the words are suffixes (bit i set for slots at or after
  // a bound), and bits at or above S are never read as slots.
  static_assert(S >= 1 && 4 * S <= 32, "slots");
  const uint32_t sw = sum >> 16;
  uint32_t light = ~0u;  // bit i < S: slot i's weight is below sw; above S: set
#pragma unroll
  for (int i = S - 1; i >= 0; --i) light = __builtin_amdgcn_alignbit(light, (a[i] >> 16) - sw, 31);
  const int kk = k - base;  // k's slot in this lane (may lie outside [0, S))
  const uint32_t from_k = ~0u << max(kk, 0);
  const int bl = bit_length(~(light | from_k));  // the lane's last heavy slot before k, + 1
  // Its position + 1, or 0 when the lane has none (bl << 6 exceeds every position).
  const int pq = min(base + bl, bl << 6);
  const int pp = static_cast<int>(quad_max(static_cast<uint32_t>(pq))) - base;
  const uint32_t right = ~0u << max(kk + 1, 0);  // positions after k
  const uint32_t from_p = ~0u << max(pp, 0);     // positions at or after p
  // Position p; for pp < 0 the bit lands at 32 + pp >= 32 - 3 S >= S.
  const uint32_t at_p = 1u << (static_cast<uint32_t>(pp) & 31u);
  uint32_t na[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    uint32_t v = bsel(bit_mask1(right, i), up1[i], dn1[i]);
    v = bsel(bit_mask1(at_p, i), sum, v);
    na[i] = bsel(bit_mask1(from_p, i), v, a[i]);
  }
#pragma unroll
  for (int i = 0; i < S; ++i) a[i] = na[i];
}

// One combination step in the lane-major layout (S >= 2); the rest as in
// step_ids.
template <int S, int CAP>
__device__ __forceinline__ void step_lm(uint32_t (&a)[CAP], int g, bool active, int t, int tmax, uint32_t *sets,
                                        Depths<uint32_t> &dep) {
  using It = ItemId;
  static_assert(S >= 2 && S <= CAP, "slots");
  // Lane g + 1's first two items (positions past the list for lane 3) and
  // lane g - 1's last (never taken by lane 0: position -1 is never moved).
  const bool last = g == 3;
  // (Each permutation is its own statement: an arm of ?: runs only where
  // it is chosen.)
  const uint32_t r0 = qps<kRot1>(a[0]);
  const uint32_t r1 = qps<kRot1>(a[1]);
  const uint32_t pv = qps<kRot3>(a[S - 1]);
  const uint32_t nx0 = last ? It::inf() : r0;
  const uint32_t nx1 = last ? It::inf() : r1;
  uint32_t up1[S], dn1[S], up2[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    up1[i] = i + 1 < S ? a[i + 1 < S ? i + 1 : 0] : nx0;
    dn1[i] = i > 0 ? a[i > 0 ? i - 1 : 0] : pv;
    up2[i] = i + 2 < S ? a[i + 2 < S ? i + 2 : 0] : (i + 2 == S ? nx0 : nx1);
  }
  const int base = g * S;
  int kslot = 0x3FF - base;  // no qualifying slot: position 0x3FF
  uint32_t xs = 0, ys = 0;
#pragma unroll
  for (int i = S - 1; i >= 0; --i) {
    const bool c = It::weight(a[i]) <= It::weight(up2[i]);
    kslot = c ? i : kslot;
    xs = c ? a[i] : xs;
    ys = c ? up1[i] : ys;
  }
  const uint32_t kq = static_cast<uint32_t>(base + kslot);
  const int k = static_cast<int>(quad_min(kq));
  const bool own = kq == static_cast<uint32_t>(k);
  const uint32_t x = quad_or<Item16>(own ? xs : 0u);
  const uint32_t y = quad_or<Item16>(own ? ys : 0u);
  const uint32_t top = static_cast<uint32_t>(32 + tmax);
  const uint32_t ix = min(x & 0xFFFFu, top), iy = min(y & 0xFFFFu, top);
  const uint32_t sx = sets[ix * 64];
  const uint32_t sy = sets[iy * 64];
  const uint32_t sw = It::weight(x) + It::weight(y);
  const uint32_t sum = (sw << 16) | static_cast<uint32_t>(32 + t);
  reinsert_lm<S, CAP>(a, dn1, up1, base, k, sum);
  const uint32_t set = sx | sy;
  sets[(32 + t) * 64] = set;
  dep.add(active ? set : 0u);
}

// Moves the lane-major layout from S slots a lane to S - 1 (S >= 3): new
// slot i of lane g is position g (S - 1) + i, which is the lane's own slot
// i - g when i >= g and otherwise slot S - g + i of lane g - 1 (S >= 3
// keeps every such position within one lane to the left).
template <int S, int CAP>
__device__ __forceinline__ void repack_lm(uint32_t (&a)[CAP], int g) {
  static_assert(S >= 3 && S <= CAP, "slots");
  uint32_t na[S - 1];
#pragma unroll
  for (int i = 0; i < S - 1; ++i) {
    // Own slot i - g (an index below 0 is not taken).
    uint32_t v = a[i];
    v = g == 1 ? a[i >= 1 ? i - 1 : 0] : v;
    v = g == 2 ? a[i >= 2 ? i - 2 : 0] : v;
    v = g == 3 ? a[i >= 3 ? i - 3 : 0] : v;
    if (i < 3) {
      // Lane h sends its slot S - 1 - h + i to lane h + 1, which takes it
      // when i < h + 1 (lanes h < i send a slot nobody takes).
      uint32_t send = a[S - 1];
      send = g == 1 && i <= 1 ? a[S - 2 + i] : send;
      send = g == 2 && i <= 2 ? a[S - 3 + i] : send;
      const uint32_t recv = qps<kRot3>(send);
      v = i < g ? recv : v;
    }
    na[i] = v;
  }
#pragma unroll
  for (int i = 0; i < S - 1; ++i) a[i] = na[i];
}

// From two slots a lane to one: lane g takes slot g & 1 of lane g >> 1.
template <int CAP>
__device__ __forceinline__ void repack_lm_2to1(uint32_t (&a)[CAP], int g) {
  constexpr int kHalf = 0x50;  // quad permutation [0, 0, 1, 1]
  const uint32_t s0 = qps<kHalf>(a[0]);
  const uint32_t s1 = qps<kHalf>(a[1]);
  a[0] = (g & 1) ? s1 : s0;
}

// Lane-major phases: steps while the wave's longest list has more than
// 4 (S - 1) items, then the layout with one slot fewer; from one slot on,
// the interleaved steps (the same layout).
template <int S, int CAP>
__device__ __forceinline__ void phases_lm(uint32_t (&a)[CAP], int g, int m_lane, int &M, int &t, int tmax,
                                          Depths<uint32_t> &dep, uint32_t *sets) {
  if constexpr (S >= 2) {
    while (M > 4 * (S - 1)) {
      step_lm<S, CAP>(a, g, t < m_lane - 1, t, tmax, sets, dep);
      --M;
      ++t;
    }
    if constexpr (S >= 3)
      repack_lm<S, CAP>(a, g);
    else
      repack_lm_2to1<CAP>(a, g);
    phases_lm<S - 1, CAP>(a, g, m_lane, M, t, tmax, dep, sets);
  } else {
    phases<4, 1, CAP, ItemId>(a, g, m_lane, M, t, tmax, dep, sets);
  }
}

// Leaf depths of one stream's Garsia-Wachs tree, its first m_lane items in
// a[] (the rest padding); m_max: the longest list of the wave, uniform.
// `sets`: for ItemId, the stream's LDS column of leaf sets by id (the
// leaves' written by the caller; 31 + m_max words at stride 64), otherwise
// unused.
template <int Q, int CAP, class It>
__device__ __forceinline__ void run(typename It::V (&a)[CAP], int g, int m_lane, int m_max,
                                    Depths<typename It::L> &dep, uint32_t *sets = nullptr) {
  int M = __builtin_amdgcn_readfirstlane(m_max);
  int t = 0;
  if constexpr (std::is_same<It, ItemId>::value && Q == 4)
    phases_lm<CAP, CAP>(a, g, m_lane, M, t, M - 2, dep, sets);
  else
    phases<Q, CAP, CAP, It>(a, g, m_lane, M, t, M - 2, dep, sets);
}

}  // namespace cggw
}  // namespace lmc
