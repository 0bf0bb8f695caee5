// CacheGen codec kernels for MI355X (gfx950): calculate_cdf, encode and
// decode of per-(layer, channel) prefix-code bitstreams.
//
// Replaces calculate_cdf / encode_fast_new / decode_fast_prefsum
// (csrc/cachegen_kernels.cpp:17-155).  The code is the one the reference's
// tests pin (tests/v1/test_cachegen_kernels.py:31-239;
// docs/cachegen/Cachegen.md:30-39): each symbol owns a power-of-two aligned
// interval of the 16-bit CDF range and is always written as the same bit
// string (the top l bits of its interval base), MSB first, each stream
// zero-padded to a byte.  The open points of that format are fixed as
// follows (the CPU oracle states the same rules):
//   L1  low 4 bits of a CDF entry = code length (0 = absent); bases are the
//       entry with those bits cleared; calculate_cdf emits lengths 1..12;
//   L2  bases never decrease: an entry below its predecessor stands for
//       0x10000, and entry n_bins is the end of the range (0x10000);
//   L3  length = low bits, or 16 - floor(log2(width)) when they are 0;
//   L4  calculate_cdf: the lengths of an optimal alphabetic code, the leaf
//       depths of the Garsia-Wachs tree over the present symbols' counts
//       (one present symbol: length 1), when the longest fits 8 bits (at
//       most 256 counted symbols) or 12 (more); otherwise Shannon lengths
//       ceil(log2(n / count)) clamped to [1, 12], Kraft-repaired by
//       lengthening the rarest present symbol; intervals assigned in symbol
//       order with widths halved until aligned (only ever needed for the
//       Shannon lengths), absent symbols at the next present base;
//   L5  encode writes at most `chunk` bytes per stream and reports the full
//       byte length;
//   L6  decode takes the largest symbol whose base is <= the next 16 bits.
//
// Work mapping: nothing here is a dense contraction, so there is no MFMA
// work.  One lane owns one (layer, channel) stream; a 256-lane block covers
// 256 consecutive channels of one layer, so symbol loads/stores of a token
// are one coalesced 256-byte row.  Per-stream tables (histogram, code table,
// decode table) live in LDS as [symbol][lane] so every lane works in its own
// column without bank conflicts or barriers.
#include <type_traits>
#include "common.h"
#include "cachegen_decode.h"
#include "cachegen_gw.h"
#include "gmem.h"

// Output words (CDF rows, bitstream words, decoded symbols) are stored with
// the streaming hint: nothing in the kernel reads them back.  Measured on
// MI355X (32 layers x 256 tokens x 1024 channels, K and V, three runs each,
// event times): decode 27.3-27.5 -> 25.2-25.3 us, encode 19.9-20.0 ->
// 19.2-19.5 us.
template <typename T> __device__ __forceinline__ void cg_st(T *p, T v) { gstore_nt(p, v); }
// The split encoder stages its CDF rows and symbols with the streaming hint
// (19.4-19.5 -> 18.9-19.1 us by events); calculate_cdf's and decode's
// staging loads stay plain (13.1 -> 14.0 and 25.6 -> 26.5 us with it).

namespace lmc {

namespace {

constexpr int kLanes = 256;
constexpr int kMaxBins = 64;
constexpr int kPrec = 16;
constexpr int kMaxLen = 12;
constexpr int kBatch = 32;  // symbol loads in flight per lane

// Copies `count` (>= 1) consecutive int16 CDF entries into LDS with every
// lane of the block, 8 loads per lane in flight: each load address is
// clamped into [0, count) so the batch has no branches between its loads.
template <int LANES>
__device__ __forceinline__ void stage_rows(const int16_t *__restrict__ src,
                                           int count, int16_t *dst) {
  constexpr int kB = 8;
  for (int i0 = 0; i0 < count; i0 += LANES * kB) {
    int16_t v[kB];
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = i0 + k * LANES + static_cast<int>(threadIdx.x);
      v[k] = src[i < count ? i : count - 1];
    }
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = i0 + k * LANES + static_cast<int>(threadIdx.x);
      if (i < count) dst[i] = v[k];
    }
  }
}

// Unpacks one stream's CDF row (staged in LDS) into the LDS column `col`
// (stride LANES) as (base << 8) | length per symbol (rules L1-L3).  `cur`
// is the unwrapped base of symbol s, `next` that of s + 1; once a base has
// wrapped to 0x10000, every later one is 0x10000 as well.
template <int LANES>
__device__ __forceinline__ void unpack_row(const int16_t *row, int nb,
                                           uint32_t *col) {
  uint32_t cur_raw = static_cast<uint16_t>(row[0]);
  uint32_t cur = cur_raw & 0xFFF0u;
  for (int s = 0; s < nb; ++s) {
    uint32_t next = 0x10000u, next_raw = 0;
    if (s + 1 < nb) {
      next_raw = static_cast<uint16_t>(row[s + 1]);
      next = next_raw & 0xFFF0u;
      if (next < cur) next = 0x10000u;
    }
    int len = static_cast<int>(cur_raw & 0xFu);
    if (len == 0) {
      const uint32_t w = next - cur;
      if (w != 0) len = kPrec - (31 - __builtin_clz(w));
    }
    col[s * LANES] = (cur << 8) | static_cast<uint32_t>(len);
    cur = next;
    cur_raw = next_raw;
  }
}

// calculate_cdf: 64 streams per block, four waves.  The block's symbols are
// staged into LDS 256 tokens at a time ([tokens][64] u8, 16-byte loads); wave
// q counts the q-th quarter of each staged piece into per-stream LDS
// histogram columns (no-return adds, one column per lane).  Wave q then
// takes symbols [j0, j1) of every stream (lane = stream) for the count sums
// and present-symbol counts.  The Garsia-Wachs steps (cachegen_gw.h) run
// next: one lane per stream in one wave (rotating with the block index, so
// that the blocks of a CU use different SIMDs) when no stream of the block
// has more than 16 present symbols, a quad of lanes per stream in all four
// waves otherwise; a stream whose tree fits the length limit leaves its
// depth counters in LDS and a flag.  The waves again take a quarter of the
// symbols each for the lengths (the tree's depths, or the Shannon lengths,
// the smallest l with count << l >= n from two leading-zero counts) and the
// partial sums of the interval widths, from which every wave writes the
// intervals of its symbols of the Garsia-Wachs streams; the rotating wave
// makes the serial aligned assignment of the other streams (the width of
// each interval capped by the lowest set bit of the running base, after the
// Kraft repair).  The block's 64 rows, contiguous in the output, leave as
// coalesced dword stores.
constexpr int kCdfWaves = 4;
constexpr int kCdfThreads = 64 * kCdfWaves;
constexpr int kCdfPiece = 256;  // tokens staged at a time
// Histogram entries after the derivation: (length << kLenShift) | count.
constexpr int kLenShift = 27;
constexpr uint32_t kCountMask = (1u << kLenShift) - 1u;

// Orders a wave's LDS writes before its later reads of other lanes' words
// (a wave's LDS accesses are performed in order).
__device__ __forceinline__ void wave_sync_cdf() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// LDS of cdf_tile_kernel: [staged symbols, later the compacted count lists]
// [histogram [nb][64] u32] [partial interval sums [4][64]] [count sums]
// [Garsia-Wachs flags] [present symbols] [rows [64][nb + 1] int16].  The
// partial sums' first row doubles as histogram row nb while the symbols are
// counted: symbols >= nb are counted there, and the row is written before
// it is read as partial sums.
// The first area holds a staged piece (at most 256 x 64 bytes), the count
// lists (nb <= 64 rows of 64 words) and the node-id mode's leaf sets (63
// rows): 64 rows of 64 words whatever T and nb.
__host__ __device__ constexpr int cdf_stage_words(int, int) { return 64 * 64; }
__host__ __device__ constexpr int cdf_lds_bytes(int T, int nb) {
  return 4 * (cdf_stage_words(T, nb) + nb * 64 + 3 * 64 + kCdfWaves * 64) + 64 * (nb + 1) * 2;
}

// Garsia-Wachs lengths for the streams of this lane's group (Q = 1: lane =
// stream, one wave; Q = 4: four lanes per stream, 16 streams per wave).
// When the longest depth fits the limit (8 bits for at most 256 counted
// symbols, else 12), stores the leaf depths' bit-sliced counters and the
// presence mask in the stream's list column and sets its flag in `gwok`.
template <int Q, int CAP, class It, int kBins>
__device__ __forceinline__ void gw_lengths(uint32_t *hist, uint32_t *lists, uint32_t *gwok, const uint32_t *nsum,
                                           int nb, int stream, int g, int m_max) {
  uint32_t *col = hist + stream;
  uint32_t *lst = lists + stream;
  // Compaction: the counts of the present symbols in symbol order.  Every
  // symbol's count is written at the next free position (m <= s < nb), so
  // an absent one is overwritten by the next present one or lies past the
  // list; the lanes of a group write the same words.  No branches.
  // The histogram holds plain counts here (lengths are stored later).
  using PM = typename std::conditional<(kBins <= 32), uint32_t, uint64_t>::type;
  PM pres = 0;
  int m = 0;
  uint32_t cs[kBins];
#pragma unroll
  for (int s = 0; s < kBins; ++s) cs[s] = s < nb ? col[s * 64] : 0u;
#pragma unroll
  for (int s = 0; s < kBins; ++s) {
    if (s < nb) lst[m * 64] = cs[s];
    const uint32_t here = min(cs[s], 1u);  // present: no compare, no SGPR mask
    pres |= static_cast<PM>(here) << s;
    m += static_cast<int>(here);
  }
  wave_sync_cdf();
  typename It::V a[CAP];
  uint32_t lw[CAP];
  // List position of slot i: lane-major (g CAP + i) for the node-id quads,
  // interleaved (Q i + g) otherwise.
  constexpr bool kLaneMajor = std::is_same<It, cggw::ItemId>::value && Q == 4;
  auto position = [g](int i) { return kLaneMajor ? g * CAP + i : Q * i + g; };
#pragma unroll
  for (int i = 0; i < CAP; ++i) {
    const int pos = position(i);
    lw[i] = lst[(pos < nb ? pos : nb - 1) * 64];
  }
#pragma unroll
  for (int i = 0; i < CAP; ++i) {
    // The empty asm takes the loaded word as an operand, so the loads stay
    // unconditional and back to back: otherwise the compiler moves each
    // load into a branch on `pos < m` and waits for it there (16 serial
    // LDS round trips in the one-lane mode).
    asm volatile("" : "+v"(lw[i]));
    const int pos = position(i);
    a[i] = pos < m ? It::leaf(lw[i], pos) : It::inf();
  }
  if constexpr (std::is_same<It, cggw::ItemId>::value) {
    // Leaf sets by id over the dead list: leaf j's at word j.
#pragma unroll
    for (int i = 0; i < CAP; ++i) lst[position(i) * 64] = 1u << position(i);
  }
  cggw::Depths<typename It::L> dep;
  cggw::run<Q, CAP, It>(a, g, m, m_max, dep, lst);
  const bool ok = m >= 2 && dep.over(nsum[stream] > 256u) == 0;
  if (!ok) return;
  // The lengths phase reads the depths by leaf from the stream's (dead)
  // list column: rows 0-3 the counters' low words, 4-7 their high words,
  // 8-9 the presence mask (the lanes of a group hold the same values).
  using L = typename It::L;
  const L d[4] = {dep.d0, dep.d1, dep.d2, dep.d3};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    lst[k * 64] = static_cast<uint32_t>(d[k]);
    lst[(4 + k) * 64] = static_cast<uint32_t>(static_cast<uint64_t>(d[k]) >> 32);
  }
  lst[8 * 64] = static_cast<uint32_t>(pres);
  lst[9 * 64] = static_cast<uint32_t>(static_cast<uint64_t>(pres) >> 32);
  gwok[stream] = 1u;
}

// kBins: register capacity for per-symbol values (nb <= kBins); kExact: nb
// == kBins, so every per-symbol bound is a constant.
template <int kBins, bool kExact>
__global__ void __launch_bounds__(kCdfThreads)
    cdf_tile_kernel(const uint8_t *__restrict__ in, int T, int C, int nb,
                    int16_t *__restrict__ out, int tiles, int vec_tile) {
  // Wave priority: 1, and 0 for a wave making the one-lane Garsia-Wachs
  // steps.  A step wave issues VALU almost every cycle and the SIMD arbiter
  // prefers the oldest wave among equals: with every wave at one priority,
  // the steps of an earlier block kept the later blocks' waves on the same
  // SIMD from counting their symbols (that phase took up to 2x longer).  The
  // one-lane steps (at most 16 present symbols) are the shortest chain of
  // the kernel, so they yield; the quad steps of the blocks with up to 32
  // present symbols, the longest chain, keep priority 1.  Measured on a
  // 32 x 256 x 1024 K+V chunk in a standalone build of this kernel: one
  // priority for every wave 26.1 us; priority 0 for both kinds of steps
  // 23.6 (23.3 once the lengths phase lost its branches); this 22.6.
  __builtin_amdgcn_s_setprio(1);
  if (kExact) nb = kBins;
  extern __shared__ uint32_t lds[];
  const int tid = static_cast<int>(threadIdx.x);
  // The wave index, read as a scalar: every per-wave bound below (a wave's
  // symbol share, the wave that runs the one-lane steps) is then uniform.
  const int q = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  const int l = blockIdx.x / tiles;
  const int c0 = (blockIdx.x % tiles) * 64;
  const int cnt = C - c0 < 64 ? C - c0 : 64;
  uint8_t *tile = reinterpret_cast<uint8_t *>(lds);
  uint32_t *hist = lds + cdf_stage_words(T, nb);
  uint32_t *psum = hist + nb * 64;          // [wave][stream]: partial interval sums
  uint32_t *nsum = psum + kCdfWaves * 64;   // per stream: symbol count
  uint32_t *gwok = nsum + 64;               // per stream: Garsia-Wachs lengths taken
  uint32_t *msum = gwok + 64;               // per stream: present symbols
  int16_t *rows = reinterpret_cast<int16_t *>(msum + 64);
  for (int i = tid; i < nb * 64; i += kCdfThreads) hist[i] = 0;
  if (tid < 192) nsum[tid] = 0;
  for (int t0 = 0; t0 < T; t0 += kCdfPiece) {
    const int tc = T - t0 < kCdfPiece ? T - t0 : kCdfPiece;
    if (t0 > 0) __syncthreads();  // the previous piece has been counted
    const uint8_t *src = in + (static_cast<int64_t>(l) * T + t0) * C + c0;
    const int pieces = tc * 4;
    if (vec_tile && cnt == 64) {
      typedef unsigned int w4 __attribute__((ext_vector_type(4)));
      w4 v[4];
      int pi[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = k * kCdfThreads + tid;
        pi[k] = i < pieces ? i : pieces - 1;
        v[k] = gload(reinterpret_cast<const w4 *>(src + static_cast<int64_t>(pi[k] >> 2) * C + (pi[k] & 3) * 16));
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) reinterpret_cast<w4 *>(tile)[pi[k]] = v[k];
    } else {
      for (int i = tid; i < tc * 64; i += kCdfThreads) {
        const int c = i % 64;
        tile[i] = c < cnt ? src[static_cast<int64_t>(i / 64) * C + c] : 0xFFu;
      }
    }
    __syncthreads();
    const int Tq = (tc + kCdfWaves - 1) / kCdfWaves;
    const int tb = q * Tq < tc ? q * Tq : tc;
    const int te = tb + Tq < tc ? tb + Tq : tc;
    if (lane < cnt && tb < te) {
      // Symbols >= nb (and the padding of a partial batch) are counted in
      // row nb, the partial sums' first row, which no count read sees: two
      // VALU operations per symbol (the row, then the address) and no branch.
      const int tq = te - tb;
      const uint8_t *scol = tile + tb * 64 + lane;
      for (int u0 = 0; u0 < tq; u0 += kBatch) {
        uint32_t sym[kBatch];
        if (u0 + kBatch <= tq) {
#pragma unroll
          for (int i = 0; i < kBatch; ++i) sym[i] = scol[(u0 + i) * 64];
        } else {
#pragma unroll
          for (int i = 0; i < kBatch; ++i) sym[i] = u0 + i < tq ? scol[(u0 + i) * 64] : 0xFFu;
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i)
          atomicAdd(&hist[min(sym[i], static_cast<uint32_t>(nb)) * 64 + lane], 1u);
      }
    }
  }
  __syncthreads();
  // Count sums and present-symbol counts, spread over the waves: wave q
  // takes symbols [j0, j1) of every stream (lane = stream).
  constexpr int kS = kBins / kCdfWaves;
  const int share = (nb + kCdfWaves - 1) / kCdfWaves;
  const int j0 = q * share;
  const int j1 = j0 + share < nb ? j0 + share : nb;
  {
    uint32_t part = 0, present = 0;
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      const uint32_t c = (k < share && j0 + k < j1) ? hist[(j0 + k) * 64 + lane] : 0u;
      part += c;
      present += min(c, 1u);
    }
    if (lane < cnt && part) {
      atomicAdd(nsum + lane, part);
      atomicAdd(msum + lane, present);
    }
  }
  __syncthreads();
  // Garsia-Wachs lengths; the mode depends on the block's largest number of
  // present symbols, the same in every wave.
  {
    // The wave's maximum by DPP within each 16-lane row (quad, half-row
    // mirror, row mirror), then the four rows' lane 0 by readlane.
    uint32_t m_max = msum[lane];
    m_max = max(m_max, cggw::qp<cggw::kSwap>(m_max));
    m_max = max(m_max, cggw::qp<cggw::kRot2>(m_max));
    m_max = max(m_max, cggw::qp<0x141>(m_max));  // row_half_mirror
    m_max = max(m_max, cggw::qp<0x140>(m_max));  // row_mirror
    const uint32_t r0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m_max), 0));
    const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m_max), 16));
    const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m_max), 32));
    const uint32_t r3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m_max), 48));
    const int mm = static_cast<int>(max(max(r0, r1), max(r2, r3)));
    uint32_t *lists = lds;  // the staged symbols are dead
    if (mm >= 2) {
      if (mm <= 16 && T < 65536) {
        __builtin_amdgcn_s_setprio(0);
        if (q == static_cast<int>(blockIdx.x % kCdfWaves))
          gw_lengths<1, 16, cggw::Item16, kBins>(hist, lists, gwok, nsum, nb, lane, 0, mm);
      } else if (mm <= 32 && T < 65536) {
        gw_lengths<4, 8, cggw::ItemId, kBins>(hist, lists, gwok, nsum, nb, q * 16 + lane / 4, lane & 3, mm);
      } else if (mm <= 32) {
        gw_lengths<4, 8, cggw::Item32, kBins>(hist, lists, gwok, nsum, nb, q * 16 + lane / 4, lane & 3, mm);
      } else if constexpr (kBins > 32) {
        gw_lengths<4, 16, cggw::Item64, kBins>(hist, lists, gwok, nsum, nb, q * 16 + lane / 4, lane & 3, mm);
      }
    }
  }
  __syncthreads();
  __builtin_amdgcn_s_setprio(1);
  // Lengths and interval assignment, spread over the waves: wave q takes
  // symbols [j0, j1) of every stream (lane = stream).  A Garsia-Wachs stream
  // keeps its tree's depths; the others (one present symbol, no counted
  // symbol, or a tree deeper than the limit) take the Shannon lengths
  // ceil(log2(n / count)) clamped to [1, 12].  Each wave sums its symbols'
  // widths 2^(16 - length) into LDS: for a Garsia-Wachs stream the lengths
  // form a complete alphabetic code, so each symbol's interval starts at the
  // sum of the widths before it, already aligned to its own width, and every
  // wave writes its own symbols' entries; an absent symbol (length 0) takes
  // the base of the next present one (or the end).
  const bool gw = gwok[lane] != 0;
  {
    const uint32_t n = nsum[lane];
    const int ln31 = -__builtin_clz(n | 1u);  // floor(log2 n) - 31
    // A Garsia-Wachs stream's depths by leaf (the leaf of symbol s is the
    // number of present symbols below it).
    const uint32_t *dcol = lds + lane;
    uint64_t dsl[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      dsl[k] = static_cast<uint64_t>(dcol[k * 64]) | (static_cast<uint64_t>(dcol[(4 + k) * 64]) << 32);
    const uint64_t pres = static_cast<uint64_t>(dcol[8 * 64]) | (static_cast<uint64_t>(dcol[9 * 64]) << 32);
    // The wave's counts (plain counts: no length is stored yet), all read
    // before the first is used; the empty asm keeps each read unconditional
    // (the compiler would otherwise move it into a branch and wait there).
    uint32_t cv[kS];
#pragma unroll
    for (int k = 0; k < kS; ++k) cv[k] = hist[min(j0 + k, nb - 1) * 64 + lane];
#pragma unroll
    for (int k = 0; k < kS; ++k) asm volatile("" : "+v"(cv[k]));
    uint32_t len[kS];
    uint32_t own = 0;
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      const bool in_range = kExact || (k < share && j0 + k < j1);  // uniform
      const int s = in_range ? j0 + k : 0;
      const uint32_t cs = in_range ? cv[k] : 0u;
      // The Shannon length: the smallest x with cs << x >= n, which is
      // x0 = floor(log2 n) - floor(log2 cs) or x0 + 1.  For cs >= 1,
      // cs << x0 < 2^(floor(log2 n) + 1) <= 2^26, so the test is a 32-bit
      // subtraction's sign.
      int x = ln31 + static_cast<int>(__builtin_clz(cs | 1u));  // x0
      x += static_cast<int>(((cs << x) - n) >> 31);
      x = min(max(x, 1), kMaxLen);
      const int j = kBins <= 32 ? __builtin_popcount(static_cast<uint32_t>(pres) & ((1u << s) - 1u))
                                : __builtin_popcountll(pres & ((1ull << s) - 1ull));
      uint32_t depth;
      if constexpr (kBins <= 32) {
        const uint32_t jj = static_cast<uint32_t>(j) & 31u;
        depth = __builtin_amdgcn_ubfe(static_cast<uint32_t>(dsl[0]), jj, 1u) |
                (__builtin_amdgcn_ubfe(static_cast<uint32_t>(dsl[1]), jj, 1u) << 1) |
                (__builtin_amdgcn_ubfe(static_cast<uint32_t>(dsl[2]), jj, 1u) << 2) |
                (__builtin_amdgcn_ubfe(static_cast<uint32_t>(dsl[3]), jj, 1u) << 3);
      } else {
        const int jj = j & 63;
        depth = static_cast<uint32_t>(((dsl[0] >> jj) & 1u) | (((dsl[1] >> jj) & 1u) << 1) |
                                      (((dsl[2] >> jj) & 1u) << 2) | (((dsl[3] >> jj) & 1u) << 3));
      }
      // Both lengths are computed for every symbol (no branch on cs).
      uint32_t xs = static_cast<uint32_t>(x);
      asm volatile("" : "+v"(xs), "+v"(depth));
      const uint32_t xl = cs ? (gw ? depth : xs) : 0u;
      len[k] = xl;
      own += 0x8000u >> ((xl - 1u) & 31u);  // 2^(16 - xl), 0 for xl = 0
      // Every lane stores; only the Shannon streams' words are read again.
      if (in_range) hist[s * 64 + lane] = (xl << kLenShift) | cs;
    }
    psum[q * 64 + lane] = own;
    __syncthreads();
    int16_t *row = rows + lane * (nb + 1);
    if (gw) {
      uint32_t pos = 0;
#pragma unroll
      for (int w = 0; w < kCdfWaves - 1; ++w) pos += w < q ? psum[w * 64 + lane] : 0u;
#pragma unroll
      for (int k = 0; k < kS; ++k) {
        if (kExact || (k < share && j0 + k < j1)) {
          row[j0 + k] = static_cast<int16_t>(static_cast<uint16_t>((pos | len[k]) & 0xFFFFu));
          pos += 0x8000u >> ((len[k] - 1u) & 31u);  // 2^(16 - len), 0 for len 0
        }
      }
    }
    if (q == 0) row[nb] = 0;
  }
  // The Shannon streams, in one wave: the Kraft repair (lengthen the rarest
  // present symbol below the cap, the last one among equals, until the code
  // fits; only a length capped at 12 bits, more than 4096 counted symbols,
  // can need it, so it runs out of line on the LDS column), then the aligned
  // in-order assignment: a symbol's base is the running position `pos`, its
  // width 2^(16 - length) capped by the lowest set bit of `pos` (the code
  // lengthened to match).
  if (q == static_cast<int>(blockIdx.x % kCdfWaves) && lane < cnt && !gw) {
    uint32_t *wcol = hist + lane;  // (length << kLenShift) | count
    uint32_t kraft = 0;            // units of 2^-16
#pragma unroll
    for (int w = 0; w < kCdfWaves; ++w) kraft += psum[w * 64 + lane];
    while (kraft > (1u << kPrec)) {
      int pick = -1;
      uint32_t best = 0;
#pragma unroll 1
      for (int s = 0; s < nb; ++s) {
        const uint32_t v = wcol[s * 64], ls = v >> kLenShift, cs = v & kCountMask;
        if (ls != 0 && ls < kMaxLen && (pick < 0 || cs <= best)) {
          pick = s;
          best = cs;
        }
      }
      if (pick < 0) break;
      const uint32_t lp = wcol[pick * 64] >> kLenShift;
      kraft -= 1u << (kPrec - lp - 1);
      wcol[pick * 64] += 1u << kLenShift;
    }
    uint32_t len[kBins];
#pragma unroll
    for (int s = 0; s < kBins; ++s) {
      const uint32_t v = wcol[(s < nb ? s : 0) * 64];  // every read issued before the first use
      len[s] = s < nb ? v >> kLenShift : 0u;
    }
    int16_t *row = rows + lane * (nb + 1);
    // r is the running base with bit 16 set, so its lowest set bit is the
    // base's alignment (0x10000 for base 0, above every width); the width
    // taken is min(2^(16 - length), that bit), and the length follows from
    // it.  The chain from one symbol to the next is four operations.
    uint32_t r = 1u << kPrec;
#pragma unroll
    for (int s = 0; s < kBins; ++s) {
      if (s < nb) {
        const uint32_t x0 = len[s];
        const uint32_t w0 = x0 ? 1u << (kPrec - x0) : 0u;
        const uint32_t w = min(w0, r & (0u - r));
        const uint32_t x = x0 ? static_cast<uint32_t>(__builtin_clz(w)) - (31u - kPrec) : 0u;
        row[s] = static_cast<int16_t>(static_cast<uint16_t>((r | x) & 0xFFFFu));
        r += w;
      }
    }
  }
  __syncthreads();
  // The block's rows are contiguous in the output.
  int16_t *dst = out + (static_cast<int64_t>(l) * C + c0) * (nb + 1);
  const int total = cnt * (nb + 1);
  if ((reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
    for (int i = tid; i < total / 2; i += kCdfThreads)
      cg_st(reinterpret_cast<uint32_t *>(dst) + i, reinterpret_cast<const uint32_t *>(rows)[i]);
    if ((total & 1) && tid == 0) dst[total - 1] = rows[total - 1];
  } else {
    for (int i = tid; i < total; i += kCdfThreads) dst[i] = rows[i];
  }
}

__device__ __forceinline__ void put_bytes(uint8_t *row, int64_t chunk,
                                          int64_t at, uint32_t word, int n) {
  // `n` most significant bytes of `word` at byte offset `at`.
  for (int b = 0; b < n; ++b)
    if (at + b < chunk) row[at + b] = static_cast<uint8_t>(word >> (24 - 8 * b));
}

// Encode: 64 streams per block (one wave); the block's 64 CDF rows are
// contiguous in memory and staged through LDS with coalesced loads.
constexpr int kEncLanes = 64;

__global__ void __launch_bounds__(kEncLanes)
    encode_kernel(const int16_t *__restrict__ cdf,
                  const uint8_t *__restrict__ in, int T, int C, int nb,
                  uint8_t *__restrict__ out, int64_t chunk,
                  int32_t *__restrict__ lens, int tiles, int word_stores) {
  extern __shared__ uint32_t lds[];
  // [nb][kEncLanes] u32 code table, then [kEncLanes][nb + 1] int16 rows.
  uint32_t *col = lds + threadIdx.x;
  int16_t *stage = reinterpret_cast<int16_t *>(lds + nb * kEncLanes);
  const int l = blockIdx.x / tiles;
  const int c0 = (blockIdx.x % tiles) * kEncLanes;
  const int cnt = C - c0 < kEncLanes ? C - c0 : kEncLanes;
  const int64_t s0 = static_cast<int64_t>(l) * C + c0;
  stage_rows<kEncLanes>(cdf + s0 * (nb + 1), cnt * (nb + 1), stage);
  __syncthreads();
  if (static_cast<int>(threadIdx.x) >= cnt) return;
  const int c = c0 + static_cast<int>(threadIdx.x);
  const int64_t stream = s0 + threadIdx.x;
  unpack_row<kEncLanes>(stage + threadIdx.x * (nb + 1), nb, col);
  // Code table: (code << 5) | length.
  for (int s = 0; s < nb; ++s) {
    const uint32_t e = col[s * kEncLanes];
    const uint32_t len = e & 0xFFu;
    const uint32_t base = e >> 8;
    const uint32_t code =
        len ? (base >> (kPrec - len)) & ((1u << len) - 1u) : 0u;
    col[s * kEncLanes] = (code << 5) | len;
  }
  uint8_t *row = out + stream * chunk;
  const uint8_t *p = in + static_cast<int64_t>(l) * T * C + c;
  uint64_t acc = 0;
  int nbits = 0;
  int64_t wpos = 0;  // bytes already written
  for (int t0 = 0; t0 < T; t0 += kBatch) {
    // All symbol loads of the batch in flight, then all table lookups, then
    // the serial bit packing.
    uint32_t e[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      e[i] = t0 + i < T ? p[static_cast<int64_t>(t0 + i) * C] : 0xFFu;
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      e[i] = e[i] < static_cast<uint32_t>(nb) ? col[e[i] * kEncLanes] : 0u;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int len = static_cast<int>(e[i] & 31u);
      acc = (acc << len) | (e[i] >> 5);
      nbits += len;
      if (nbits >= 32) {
        const uint32_t word = static_cast<uint32_t>(acc >> (nbits - 32));
        if (word_stores && wpos + 4 <= chunk)
          cg_st(reinterpret_cast<uint32_t *>(row + wpos), __builtin_bswap32(word));
        else
          put_bytes(row, chunk, wpos, word, 4);
        wpos += 4;
        nbits -= 32;
      }
    }
  }
  if (nbits > 0) {
    const uint32_t tail = static_cast<uint32_t>(acc << (32 - nbits));
    put_bytes(row, chunk, wpos, tail, (nbits + 7) >> 3);
  }
  lens[stream] = static_cast<int32_t>(wpos + ((nbits + 7) >> 3));
}

// Wave encode (T <= 256): 64 streams per block, four waves; a wave encodes
// one whole stream at a time, so no lane walks a serial chain of symbols.
//   1. The block's CDF rows and symbols are staged into LDS with coalesced
//      loads, all issued before any LDS store; the symbols are transposed
//      to one row per stream (an odd number of words per row).
//   2. Per stream, lane s builds symbol s's (code, length) from the staged
//      row (the wrap of rule L2 found with a ballot), and lane j takes the
//      stream's tokens 4j .. 4j + 3 with one LDS read and looks their codes
//      up with cross-lane shuffles.
//   3. The lane's four codes become one run of at most 64 bits; an
//      exclusive prefix sum over the wave gives the run's bit offset, and
//      the run is ORed into the (at most three) words it touches of the
//      wave's LDS bit buffer.
//   4. Lane k stores word k of the row: one coalesced store per 256 bytes,
//      and only bytes below min(chunk, stream length), as the single-lane
//      encoder writes them.
constexpr int kEncWaves = 4;
#ifndef LMC_ENC_SPLIT
#define LMC_ENC_SPLIT 1     // split encoder for full 64-channel blocks
#endif
#ifndef LMC_ENC_PIECES
#define LMC_ENC_PIECES 8    // waves (token pieces) per block of the split encoder
#endif
constexpr int kEncPieces = LMC_ENC_PIECES;
constexpr int kEncTileThreads = kEncLanes * kEncWaves;
constexpr int kEncTileMaxT = 4 * kEncLanes;

__device__ __forceinline__ void put_word(uint8_t *row, int64_t chunk, uint32_t idx, uint32_t word,
                                         int n, int word_stores) {
  const int64_t at = static_cast<int64_t>(idx) * 4;
  if (n == 4 && word_stores && at + 4 <= chunk)
    cg_st(reinterpret_cast<uint32_t *>(row + at), __builtin_bswap32(word));
  else
    put_bytes(row, chunk, at, word, n);
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves: shifts
// by 1, 2, 4 and 8 within each row of 16 lanes, then the last lane of row
// 0 (row_bcast:15) and of row 1 (row_bcast:31) added to the rows after it.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  int x = static_cast<int>(v);
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false); // row_bcast:15 to rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false); // row_bcast:31 to rows 2, 3
  return static_cast<uint32_t>(x);
}

// Encode staging: the block's CDF rows (contiguous in memory) into `stage`
// and its symbols, transposed to one row of `sym_stride` words per stream,
// into `tile`; every global load of a thread is issued before its LDS
// stores.  With `vec_tile` (a full block of 64 channels, C % 16 == 0 and a
// 16-byte aligned input) each token's 64 symbols are four 16-byte loads.
template <int NT>
__device__ __forceinline__ void enc_stage(const int16_t *__restrict__ cdf,
                                          const uint8_t *__restrict__ in, int T, int C, int nb,
                                          int l, int c0, int cnt, int64_t s0, int vec_tile,
                                          int sym_stride, int16_t *stage, uint8_t *tile) {
  const int tid = static_cast<int>(threadIdx.x);
  const int16_t *rsrc = cdf + s0 * (nb + 1);
  const int rcount = cnt * (nb + 1);
  constexpr int kR = 4;
  int16_t rv[kR];
  int ri[kR];
#pragma unroll
  for (int k = 0; k < kR; ++k) {
    const int i = k * NT + tid;
    ri[k] = i < rcount ? i : rcount - 1;
    rv[k] = rsrc[ri[k]];
  }
  const uint8_t *src = in + static_cast<int64_t>(l) * T * C + c0;
  const int pieces = T * 4;
  const int row_bytes = sym_stride * 4;
  if (vec_tile && cnt == kEncLanes) {
    constexpr int kV = (4 * kEncTileMaxT + NT - 1) / NT;  // 16-byte pieces per thread (T <= 256)
    uint4 v[kV];
    int pi[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int i = k * NT + tid;
      pi[k] = i < pieces ? i : pieces - 1;
      v[k] = *reinterpret_cast<const uint4 *>(src + static_cast<int64_t>(pi[k] >> 2) * C + (pi[k] & 3) * 16);
    }
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      uint8_t *d = tile + (pi[k] & 3) * 16 * row_bytes + (pi[k] >> 2);
      const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
      for (int j = 0; j < 16; ++j) d[j * row_bytes] = static_cast<uint8_t>(w[j >> 2] >> (8 * (j & 3)));
    }
  } else {
    for (int i = tid; i < T * kEncLanes; i += NT) {
      const int c = i % kEncLanes, t = i / kEncLanes;
      tile[c * row_bytes + t] = c < cnt ? src[static_cast<int64_t>(t) * C + c] : 0;
    }
  }
#pragma unroll
  for (int k = 0; k < kR; ++k) stage[ri[k]] = rv[k];
  for (int i = kR * NT + tid; i < rcount; i += NT) stage[i] = rsrc[i];
}

__global__ void __launch_bounds__(kEncTileThreads)
    encode_wave_kernel(const int16_t *__restrict__ cdf,
                       const uint8_t *__restrict__ in, int T, int C, int nb,
                       uint8_t *__restrict__ out, int64_t chunk,
                       int32_t *__restrict__ lens, int tiles, int word_stores, int vec_tile,
                       int sym_stride, int cap_words) {
  // [64][nb + 1] int16 rows | [64][sym_stride] u32 symbols | [4][2][cap_words] u32 bits
  extern __shared__ uint32_t lds[];
  const int tid = static_cast<int>(threadIdx.x);
  const int wv = tid / kEncLanes;
  const int lane = tid % kEncLanes;
  const int l = blockIdx.x / tiles;
  const int c0 = (blockIdx.x % tiles) * kEncLanes;
  const int cnt = C - c0 < kEncLanes ? C - c0 : kEncLanes;
  const int64_t s0 = static_cast<int64_t>(l) * C + c0;
  int16_t *stage = reinterpret_cast<int16_t *>(lds);
  const int rows_words = ((nb + 1) * kEncLanes * 2 + 15) / 16 * 4;
  uint8_t *tile = reinterpret_cast<uint8_t *>(lds + rows_words);
  uint32_t *bitbuf = lds + rows_words + kEncLanes * sym_stride + 2 * wv * cap_words;

  // 1. Rows and symbols: every load of the thread, then the LDS stores.
  enc_stage<kEncTileThreads>(cdf, in, T, C, nb, l, c0, cnt, s0, vec_tile, sym_stride, stage, tile);
  __syncthreads();

  // Two streams per step (st and st + kEncWaves), so their LDS round trips
  // overlap.
  for (int st0 = wv; st0 < cnt; st0 += 2 * kEncWaves) {
    int stv[2];
    bool on[2];
    int entry[2];
    uint32_t word[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      stv[j] = st0 + j * kEncWaves;
      on[j] = stv[j] < cnt;
      // 2. Code table: lane s holds symbol s's (code << 5) | length.
      const int16_t *row = stage + (on[j] ? stv[j] : st0) * (nb + 1);
      const uint32_t raw = lane < nb ? static_cast<uint16_t>(row[lane]) : 0u;
      const uint32_t raw_n = lane + 1 < nb ? static_cast<uint16_t>(row[lane + 1]) : 0u;
      const bool dec = lane + 1 < nb && (raw_n & 0xFFF0u) < (raw & 0xFFF0u);
      const uint64_t decs = __ballot(dec);
      const int wrap = decs ? __builtin_ctzll(decs) + 1 : nb;  // bases from here on are 0x10000
      const uint32_t base = lane < wrap ? (raw & 0xFFF0u) : 0x10000u;
      const uint32_t next = lane + 1 < wrap ? (raw_n & 0xFFF0u) : 0x10000u;
      uint32_t len = raw & 0xFu;
      if (len == 0 && next != base) len = kPrec - (31 - __builtin_clz(next - base));
      const uint32_t code = len ? (base >> (kPrec - len)) & ((1u << len) - 1u) : 0u;
      entry[j] = lane < nb ? static_cast<int>((code << 5) | len) : 0;
      // Tokens 4 * lane .. + 3.
      word[j] = (on[j] && 4 * lane < T)
                    ? reinterpret_cast<const uint32_t *>(tile)[stv[j] * sym_stride + lane] : 0u;
    }
    uint64_t run[2];
    uint32_t run_bits[2], pos[2], total[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      run[j] = 0;
      run_bits[j] = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t v = (word[j] >> (8 * b)) & 0xFFu;
        const uint32_t e = static_cast<uint32_t>(__shfl(entry[j], static_cast<int>(v & 63u)));
        const bool ok = on[j] && 4 * lane + b < T && v < static_cast<uint32_t>(nb);
        const uint32_t n = ok ? (e & 31u) : 0u;
        run[j] = (run[j] << n) | (ok ? (e >> 5) : 0u);
        run_bits[j] += n;
      }
    }
    // 3. Exclusive prefix sums of the runs' lengths.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t incl = wave_incl_scan(run_bits[j]);
      pos[j] = incl - run_bits[j];
      total[j] = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), kEncLanes - 1));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      for (int k = lane; k < cap_words; k += kEncLanes) bitbuf[j * cap_words + k] = 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (!run_bits[j]) continue;
      uint32_t *bb = bitbuf + j * cap_words;
      const uint64_t a = run[j] << (64 - run_bits[j]);  // top-aligned
      const uint32_t hi = static_cast<uint32_t>(a >> 32), lo = static_cast<uint32_t>(a);
      const uint32_t w0 = pos[j] >> 5, sh = pos[j] & 31u;
      if (w0 < static_cast<uint32_t>(cap_words)) atomicOr(&bb[w0], hi >> sh);
      if (sh + run_bits[j] > 32 && w0 + 1 < static_cast<uint32_t>(cap_words))
        atomicOr(&bb[w0 + 1], sh ? (hi << (32 - sh)) | (lo >> sh) : lo);
      if (sh + run_bits[j] > 64 && w0 + 2 < static_cast<uint32_t>(cap_words))
        atomicOr(&bb[w0 + 2], lo << (32 - sh));
    }
    // 4. The rows.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (!on[j]) continue;
      const int64_t tbytes = (total[j] + 7) >> 3;
      int64_t nbytes = tbytes < chunk ? tbytes : chunk;
      nbytes = nbytes < 4 * static_cast<int64_t>(cap_words) ? nbytes : 4 * static_cast<int64_t>(cap_words);
      uint8_t *orow = out + (s0 + stv[j]) * chunk;
      for (int k = lane; static_cast<int64_t>(k) * 4 < nbytes; k += kEncLanes) {
        const int64_t left = nbytes - 4 * static_cast<int64_t>(k);
        put_word(orow, chunk, static_cast<uint32_t>(k), bitbuf[j * cap_words + k],
                 left >= 4 ? 4 : static_cast<int>(left), word_stores);
      }
      if (lane == 0) lens[s0 + stv[j]] = static_cast<int32_t>(tbytes);
    }
  }
}

// Split encode (T <= 256, a full block of 64 channels): 64 streams per
// block and PIECES waves, wave w taking tokens [w * Q, (w + 1) * Q) of every
// stream (Q = 256 / PIECES), lane s stream s.  Each lane walks a serial
// chain of only Q codes, and every wave instruction works for 64 streams.
//   1. The block's CDF rows (contiguous in memory) are staged with dword
//      loads; its symbols are staged untransposed, [token][64 channels]
//      bytes, with 16-byte stores (tokens T .. 255 read as 0xFF, not
//      coded).  Lane s then reads token t's symbol at t * 64 + s: the 64
//      lanes read 16 consecutive words.
//   2. Code table in LDS, [symbol][stream] words of (code << 11) | length
//      (rules L1-L3), built with lane = stream, so its stores and the
//      lookups of step 3 each hit 64 distinct banks; row nb is all zeros
//      and takes every symbol >= nb.  Wave w writes the w-th share of the
//      symbols, after finding from the row whether the wrap of rule L2
//      (an entry below its predecessor) lies before its share.  The block
//      notes whether any code is longer than 8 bits.
//   3. Each lane looks up its Q codes into registers and sums their
//      lengths (the sum of the entries' low 11 bits: at most 64 x 15 bits,
//      so no carry reaches the code field).  The piece lengths of a stream
//      give each piece its bit offset.
//   4. The staged data is dead; the same LDS holds one zeroed bit row per
//      stream (2T bytes + a word: codes are at most 15 bits), and each lane
//      ORs its codes in as runs of at most 32 bits: four codes per run when
//      no code of the block is longer than 8 bits, else two.
//   5. Rows leave as in the wave encoder: wave w stores the rows of streams
//      w, w + PIECES, ..., lane k word k, only bytes below
//      min(chunk, stream length).
template <int PIECES>
__device__ __forceinline__ void enc_append(uint32_t *brow, uint32_t &pos, uint32_t run, uint32_t n) {
  // `run` holds n <= 32 bits (0 when n is 0); its top-aligned form is ORed
  // into the one or two words it touches.
  const uint32_t top = run << ((32u - n) & 31u);
  const uint32_t wi = pos >> 5, sh = pos & 31u;
  atomicOr(brow + wi, top >> sh);  // a no-op when n is 0
  if (sh + n > 32u) atomicOr(brow + wi + 1, top << (32u - sh));
  pos += n;
}

template <int PIECES>
__global__ void __launch_bounds__(64 * PIECES)
    encode_split_kernel(const int16_t *__restrict__ cdf,
                        const uint8_t *__restrict__ in, int T, int C, int nb,
                        uint8_t *__restrict__ out, int64_t chunk,
                        int32_t *__restrict__ lens, int tiles, int word_stores, int row_words,
                        int stage_words) {
  constexpr int NT = 64 * PIECES;
  constexpr int Q = kEncTileMaxT / PIECES;  // tokens per piece
  // Phase 1: [64][nb + 1] int16 rows | [256][64] u8 symbols | [nb + 1][64] u32 codes
  // Phase 2: [64][row_words] u32 bit rows (over phase 1)
  // Always:  [PIECES][64] u32 piece lengths, the long-code flag and [64] u64
  //          decrease masks, after both
  extern __shared__ uint32_t lds[];
  typedef unsigned int w4 __attribute__((ext_vector_type(4)));
  const int tid = static_cast<int>(threadIdx.x);
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l = blockIdx.x / tiles;
  const int c0 = (blockIdx.x % tiles) * kEncLanes;
  const int64_t s0 = static_cast<int64_t>(l) * C + c0;
  const int rows_words = ((nb + 1) * kEncLanes * 2 + 15) / 16 * 4;
  int16_t *stage = reinterpret_cast<int16_t *>(lds);
  uint8_t *tile = reinterpret_cast<uint8_t *>(lds + rows_words);
  uint32_t *tab = lds + rows_words + kEncTileMaxT * kEncLanes / 4;
  uint32_t *bits = lds;
  uint32_t *plen = lds + stage_words;
  uint32_t *long_flag = plen + PIECES * kEncLanes;
  uint64_t *dmask = reinterpret_cast<uint64_t *>(lds + ((stage_words + PIECES * kEncLanes + 2) & ~1));

  // 1. Staging: every global load of the thread, then its LDS stores.  The
  //    block's rows start at an even entry (s0 is a multiple of 64) and hold
  //    an even number of entries, so they are whole dwords.
  {
    const uint32_t *rsrc = reinterpret_cast<const uint32_t *>(cdf + s0 * (nb + 1));
    const int rcount = kEncLanes * (nb + 1) / 2;
    constexpr int kR = (kEncLanes * 33 / 2 + NT - 1) / NT;  // row dwords per thread for nb <= 32
    uint32_t rv[kR];
    int ri[kR];
#pragma unroll
    for (int k = 0; k < kR; ++k) {
      const int i = k * NT + tid;
      ri[k] = i < rcount ? i : rcount - 1;
      rv[k] = gload_nt(rsrc + ri[k]);
    }
    const uint8_t *src = in + static_cast<int64_t>(l) * T * C + c0;
    constexpr int kV = (4 * kEncTileMaxT + NT - 1) / NT;  // 16-byte pieces per thread
    const int pieces = T * 4;
    w4 v[kV];
    int pi[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int i = k * NT + tid;
      pi[k] = i < pieces ? i : pieces - 1;
      v[k] = gload_nt(reinterpret_cast<const w4 *>(src + static_cast<int64_t>(pi[k] >> 2) * C + (pi[k] & 3) * 16));
    }
    const w4 none = {0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu};
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int i = k * NT + tid;  // every piece of the 256 x 64 tile, in or past T
      reinterpret_cast<w4 *>(tile)[i] = i < pieces ? v[k] : none;
    }
    uint32_t *rdst = reinterpret_cast<uint32_t *>(stage);
#pragma unroll
    for (int k = 0; k < kR; ++k) rdst[ri[k]] = rv[k];
    for (int i = kR * NT + tid; i < rcount; i += NT) rdst[i] = rsrc[i];
    if (tid == 0) *long_flag = 0u;
    if (tid < kEncLanes) dmask[tid] = 0u;
  }
  __syncthreads();

  // 2. Code table, lane = stream; wave w writes symbols [j0, j1).  First
  //    each wave marks the decreases of rule L2 in its range (entry j below
  //    entry j - 1) in the stream's 64-bit mask, so that afterwards symbol j
  //    is wrapped exactly when the mask has a bit at or below j.
  {
    constexpr int kShare = (kMaxBins + PIECES - 1) / PIECES;
    const int16_t *row = stage + lane * (nb + 1);
    const int share = (nb + PIECES - 1) / PIECES;
    const int j0 = wv * share;
    const int j1 = j0 + share < nb ? j0 + share : nb;
    uint32_t m[kShare + 1];  // masked entries j0 .. j0 + kShare (0 past nb - 1)
#pragma unroll
    for (int k = 0; k <= kShare; ++k)
      m[k] = (k <= share && j0 + k < nb) ? (static_cast<uint16_t>(row[j0 + k]) & 0xFFF0u) : 0u;
    const uint32_t m_before = j0 > 0 && j0 < nb ? (static_cast<uint16_t>(row[j0 - 1]) & 0xFFF0u) : 0u;
    uint64_t dec = 0;
#pragma unroll
    for (int k = 0; k < kShare; ++k) {
      const int jj = j0 + k;
      const uint32_t prev = k == 0 ? m_before : m[k - 1];
      if (k < share && jj < j1 && jj >= 1 && m[k] < prev) dec |= uint64_t(1) << jj;
    }
    if (dec) atomicOr(dmask + lane, static_cast<unsigned long long>(dec));
    __syncthreads();
    const uint64_t D = dmask[lane];
    uint32_t longest = 0;
#pragma unroll
    for (int k = 0; k < kShare; ++k) {
      const int jj = j0 + k;
      if (k < share && jj < j1) {
        const uint32_t raw = static_cast<uint16_t>(row[jj]);
        const bool wrapped = (D & (~uint64_t(0) >> (63 - jj))) != 0;
        const bool has_n = jj + 1 < nb;
        const bool wrapped_n = has_n && (D & (~uint64_t(0) >> (62 - jj))) != 0;
        const uint32_t base = wrapped ? 0x10000u : m[k];
        const uint32_t next = (has_n && !wrapped_n) ? m[k + 1] : 0x10000u;
        const uint32_t width = next - base;
        // Rule L3: the low bits, else 16 - floor(log2(width)) (0 for an empty interval).
        const uint32_t wlen = width ? static_cast<uint32_t>(__builtin_clz(width)) - 15u : 0u;
        const uint32_t len = (raw & 0xFu) ? (raw & 0xFu) : wlen;
        const uint32_t code = __builtin_amdgcn_ubfe(base, kPrec - len, len);  // 0 when len is 0
        tab[jj * kEncLanes + lane] = (code << 11) | len;
        longest = len > longest ? len : longest;
      }
    }
    if (wv == 0) tab[nb * kEncLanes + lane] = 0u;
    if (__ballot(longest > 8u) && lane == 0) *long_flag = 1u;
  }
  __syncthreads();
  const bool long_codes = *long_flag != 0u;

  // 3. Lookups into registers, and the piece's length.
  uint32_t e[Q];
  uint32_t sum = 0;
  {
    const uint8_t *scol = tile + wv * Q * kEncLanes + lane;
    const uint32_t *tcol = tab + lane;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t v = scol[i * kEncLanes];
      e[i] = tcol[(v < static_cast<uint32_t>(nb) ? v : static_cast<uint32_t>(nb)) * kEncLanes];
    }
#pragma unroll
    for (int i = 0; i < Q; i += 2) sum += e[i] + e[i + 1];
  }
  plen[wv * kEncLanes + lane] = sum & 0x7FFu;
  __syncthreads();

  // 4. Bit rows: zeroed, then each piece ORed in at its offset.
  {
    const int n4 = (kEncLanes * row_words) / 4;
    w4 *b4 = reinterpret_cast<w4 *>(bits);
    const w4 z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < n4; i += NT) b4[i] = z;
    for (int i = 4 * n4 + tid; i < kEncLanes * row_words; i += NT) bits[i] = 0u;
  }
  uint32_t pos = 0, total = 0;
#pragma unroll
  for (int w = 0; w < PIECES; ++w) {
    const uint32_t n = plen[w * kEncLanes + lane];
    pos += w < wv ? n : 0u;
    total += n;
  }
  __syncthreads();
  {
    uint32_t *brow = bits + lane * row_words;
    if (!long_codes) {
      // Codes of at most 8 bits: four to a run.
#pragma unroll
      for (int i = 0; i < Q; i += 4) {
        uint32_t run = e[i] >> 11;
        run = (run << (e[i + 1] & 31u)) | (e[i + 1] >> 11);
        run = (run << (e[i + 2] & 31u)) | (e[i + 2] >> 11);
        run = (run << (e[i + 3] & 31u)) | (e[i + 3] >> 11);
        const uint32_t n = (e[i] + e[i + 1] + e[i + 2] + e[i + 3]) & 0x7FFu;
        enc_append<PIECES>(brow, pos, run, n);
      }
    } else {
#pragma unroll
      for (int i = 0; i < Q; i += 2) {
        const uint32_t run = ((e[i] >> 11) << (e[i + 1] & 31u)) | (e[i + 1] >> 11);
        const uint32_t n = (e[i] + e[i + 1]) & 0x7FFu;  // <= 30
        enc_append<PIECES>(brow, pos, run, n);
      }
    }
  }
  if (wv == 0) lens[s0 + lane] = static_cast<int32_t>((total + 7) >> 3);
  __syncthreads();

  // 5. The rows: full words as dword stores, the bytes of a last partial
  //    word by one lane each (a stream is at most 2T + 1 <= 513 bytes).
  for (int st = wv; st < kEncLanes; st += PIECES) {
    const uint32_t tb = __builtin_amdgcn_readlane(static_cast<int>(total), st);  // wave-uniform
    const uint32_t tbytes = (tb + 7) >> 3;
    const uint32_t nbytes = chunk < static_cast<int64_t>(tbytes) ? static_cast<uint32_t>(chunk) : tbytes;
    uint8_t *orow = out + (s0 + st) * chunk;
    const uint32_t *brow = bits + st * row_words;
    const uint32_t nw = word_stores ? nbytes >> 2 : 0u;
    for (uint32_t k = lane; k < nw; k += kEncLanes)
      cg_st(reinterpret_cast<uint32_t *>(orow) + k, __builtin_bswap32(brow[k]));
    for (uint32_t b = 4 * nw + lane; b < nbytes; b += kEncLanes)
      orow[b] = static_cast<uint8_t>(brow[b >> 2] >> (24 - 8 * (b & 3u)));
  }
}

// Decode: 64 streams per block (one wave) and 40 KiB of LDS per block, so
// the four blocks of a CU's four SIMDs fit its 160 KiB.  The block's 64
// streams are adjacent in the byte buffer; their CDF rows and (up to the
// window size) their bytes are staged into LDS with coalesced 16-byte
// loads, so the per-symbol loop touches no global memory except for
// streams that do not fit the window.
//
// Symbol lookup (rule L6) is table driven, with per-stream tables built in
// LDS from the staged rows.  n_bins <= 32 takes cgdec::ByteTables: one byte
// per 8-bit window prefix, so every code of at most 8 bits (all of them for
// chunks of up to 256 tokens) is one LDS read, and the table is built
// without data-dependent loops.  Larger n_bins take DecTables below.  Bases
// are multiples of 16, so the top 12 bits of the 16-bit window decide the
// symbol.  DecTables' L1 has one entry per 7-bit prefix: symbol | length <<
// 8 when one symbol owns the prefix's whole range; 0x8000 | k << 8 |
// s_first when symbol boundaries fall inside it, k naming one of the
// stream's kSubTables L2 tables whose 32 one-byte entries (next 5 bits)
// hold (s - s_first) << 4 | length; and kOverflow when the stream ran out
// of L2 tables (or a prefix spans more than 16 symbols), which falls back
// to a binary search over the bases.
constexpr int kDecLanes = cgdec::kLanes;
#ifndef LMC_DEC_LANES
#define LMC_DEC_LANES 1  // per-lane stream regions for n_bins <= 32
#endif
constexpr int kDirectBits = 7;
constexpr int kSubBits = 5;
constexpr int kSubTables = 4;
constexpr uint32_t kOverflow = 0xFFFFu;
constexpr int kDecLds = 40 * 1024;
constexpr int kL1Bytes = (1 << kDirectBits) * kDecLanes * 2;
constexpr int kL2Bytes = kSubTables * (1 << kSubBits) * kDecLanes;
constexpr int kObufBytes = 4 * kDecLanes;
static_assert(kObufBytes >= 256, "the byte table build writes past the table into the 256 bytes after it");
constexpr int kRowChunks = 5;   // 16-byte row chunks per lane and load batch (33 x 64 x 2 B)
constexpr int kWinChunks = 12;  // 16-byte window chunks per lane and load batch (12 KiB)

// Loads up to kDecLanes * N 16-byte chunks [j0, j0 + 64 N) of a run of n
// chunks at the 16-byte aligned global address src into registers, one
// chunk per lane and slot; indexes past the run are clamped to its last
// chunk (n >= 1).
// Global (not flat) loads: they are counted by vmcnt alone and return in
// order, so a store of an early chunk waits only for the loads before it.
typedef uint32_t chunk16 __attribute__((ext_vector_type(4)));
using global_chunk16 = const __attribute__((address_space(1))) chunk16;

template <int N>
__device__ __forceinline__ void load_chunks(uintptr_t src, int n, int j0, int lane, chunk16 (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int j = j0 + k * kDecLanes + lane;
    v[k] = reinterpret_cast<global_chunk16 *>(src)[j < n ? j : n - 1];
  }
}

// Stores the chunks of load_chunks to LDS at dst (several lanes may store
// the same clamped last chunk, with the same bytes); kSwap byte-reverses
// each dword (the big-endian order of the stream bits).
template <bool kSwap, int N>
__device__ __forceinline__ void store_chunks(uint8_t *dst, int n, int j0, int lane, const chunk16 (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int j = j0 + k * kDecLanes + lane;
    chunk16 w = v[k];
    if (kSwap) {
      w.x = __builtin_bswap32(w.x);
      w.y = __builtin_bswap32(w.y);
      w.z = __builtin_bswap32(w.z);
      w.w = __builtin_bswap32(w.w);
    }
    reinterpret_cast<chunk16 *>(dst)[j < n ? j : n - 1] = w;
  }
}

using cgdec::StagedRow;

// Per-lane decode tables: L1 and L2 columns of stride kDecLanes.
struct DecTables {
  static constexpr int kBytes = kL1Bytes + kL2Bytes;
  uint16_t *l1;
  uint8_t *l2;
  StagedRow row;
  int nb;
  int top;  // largest power of two below nb (1 if nb <= 2)

  __device__ __forceinline__ void bind(uint8_t *lds, int lane) {
    l1 = reinterpret_cast<uint16_t *>(lds) + lane;
    l2 = lds + kL1Bytes + lane;
  }

  // Builds L1/L2 from the staged row in one pass over the symbols (a loop
  // every lane runs in step).  Symbol s owns the windows [lo, hi): lo is
  // its base (0 for s = 0, which also takes windows below the first base),
  // hi the next base.  Prefixes entirely inside [lo, hi) get a direct
  // entry; a prefix holding a boundary is opened by the symbol covering its
  // start and filled by that symbol and the following ones.  Also finds
  // row.wrap.
  __device__ __forceinline__ void clear() {}   // build() writes every entry
  __device__ __forceinline__ void finish() {}  // build() sets row.wrap and top

  __device__ __forceinline__ void build(uint8_t *) {
    constexpr uint32_t span = 1u << (kPrec - kDirectBits);
    constexpr uint32_t sub = 1u << (kPrec - kDirectBits - kSubBits);
    row.wrap = nb;
    uint32_t raw = static_cast<uint16_t>(row.r[0]);
    uint32_t base = raw & 0xFFF0u;
    uint32_t last = base;  // last base before any wrap
    int open_k = -1, open_first = 0, nsub = 0;
    for (int s = 0; s < nb; ++s) {
      uint32_t next = 0x10000u, next_raw = 0;
      if (s + 1 < nb) {
        next_raw = static_cast<uint16_t>(row.r[s + 1]);
        const uint32_t nbase = next_raw & 0xFFF0u;
        if (row.wrap == nb && nbase >= last) {
          next = nbase;
          last = nbase;
        } else if (row.wrap == nb) {
          row.wrap = s + 1;
        }
      }
      int len = static_cast<int>(raw & 0xFu);
      if (len == 0) {
        const uint32_t w = next - base;
        if (w != 0) len = kPrec - (31 - __builtin_clz(w));
      }
      const uint32_t lo = s == 0 ? 0u : base, hi = next;
      if (hi > lo) {
        const uint32_t ent = static_cast<uint32_t>(s) | (static_cast<uint32_t>(len) << 8);
        uint32_t e = lo / span;
        if (lo % span) {  // inside a prefix opened by an earlier symbol
          if (open_k >= 0) {
            const int ds = s - open_first;
            if (ds > 15) {
              l1[e * kDecLanes] = static_cast<uint16_t>(kOverflow);
              open_k = -1;
            } else {
              const uint32_t j1 = hi - e * span < span ? (hi - e * span) / sub : span / sub;
              for (uint32_t j = (lo % span) / sub; j < j1; ++j)
                l2[(open_k * (1 << kSubBits) + j) * kDecLanes] =
                    static_cast<uint8_t>((ds << 4) | len);
            }
          }
          ++e;
        }
        for (; e < hi / span; ++e) l1[e * kDecLanes] = static_cast<uint16_t>(ent);
        if ((hi % span) && lo <= hi - hi % span) {  // opens the prefix holding hi
          e = hi / span;
          if (nsub < kSubTables) {
            open_k = nsub++;
            open_first = s;
            l1[e * kDecLanes] = static_cast<uint16_t>(0x8000u | (open_k << 8) | s);
            for (uint32_t j = 0; j < (hi % span) / sub; ++j)
              l2[(open_k * (1 << kSubBits) + j) * kDecLanes] = static_cast<uint8_t>(len);
          } else {
            open_k = -1;
            l1[e * kDecLanes] = static_cast<uint16_t>(kOverflow);
          }
        }
      }
      raw = next_raw;
      base = next;
    }
    top = 1;
    while (top * 2 < nb) top *= 2;
  }

  // Symbol and code length for the 16-bit window v.
  __device__ __forceinline__ void lookup(uint32_t v, int &s, int &len) const {
    const uint32_t d = l1[(v >> (kPrec - kDirectBits)) * kDecLanes];
    if (d < 0x8000u) {
      s = static_cast<int>(d & 0xFFu);
      len = static_cast<int>(d >> 8);
    } else if (d != kOverflow) {
      const uint32_t j = (v >> (kPrec - kDirectBits - kSubBits)) & ((1u << kSubBits) - 1);
      const uint32_t x = l2[(((d >> 8) & 0x7Fu) * (1 << kSubBits) + j) * kDecLanes];
      s = static_cast<int>((d & 0xFFu) + (x >> 4));
      len = static_cast<int>(x & 0xFu);
    } else {
      s = 0;
      for (int step = top; step > 0; step >>= 1)
        if (s + step < nb && row.base(s + step) <= v) s += step;
      len = row.len(s);
    }
  }
};

// Bytes of the aligned dword at address `a` that lie in [lo, hi), as a mask
// over the dword's little-endian value.
__device__ __forceinline__ uint32_t live_mask(uintptr_t a, uintptr_t lo, uintptr_t hi) {
  const int64_t from = static_cast<int64_t>(lo) - static_cast<int64_t>(a);
  const int64_t to = static_cast<int64_t>(hi) - static_cast<int64_t>(a);
  const int f = from < 0 ? 0 : (from > 4 ? 4 : static_cast<int>(from));
  const int t = to < 0 ? 0 : (to > 4 ? 4 : static_cast<int>(to));
  const uint32_t below_t = t >= 4 ? ~0u : ((1u << (8 * t)) - 1u);
  const uint32_t below_f = f >= 4 ? ~0u : ((1u << (8 * f)) - 1u);
  return below_t & ~below_f;
}

// Big-endian dword of the staged window at byte offset q (a multiple of 4),
// with the bytes at or past `hi` (an offset too) zeroed.  The read is
// clamped to the window's last dword; whatever it returns past hi is
// masked off.
__device__ __forceinline__ uint32_t win_word(const uint32_t *win, uint32_t last, uint32_t q,
                                             uint32_t hi) {
  const uint32_t w = win[(q < last ? q : last) >> 2];
  const int t = static_cast<int>(hi) - static_cast<int>(q);
  const int k = t < 0 ? 0 : (t > 4 ? 4 : t);
  return k >= 4 ? w : (w & ~(~0u >> (8 * k)));
}

// Keeps the bytes of a big-endian dword at stream offset q that lie before
// the stream end `hi` (bytes at or past hi read as zero).
__device__ __forceinline__ uint32_t clip_word(uint32_t w, uint32_t q, uint32_t hi) {
  const int t = static_cast<int>(hi) - static_cast<int>(q);
  const int k = t < 0 ? 0 : (t > 4 ? 4 : t);
  return k >= 4 ? w : (w & ~(~0u >> (8 * k)));
}

// Orders a wave's LDS writes before its later reads of other lanes' words.
// Decode blocks are one wave, and a wave's LDS accesses are performed in
// order, so no block barrier is needed.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// All 64 streams of the block lie in the window: L1/L2 lookups and symbols
// transposed through LDS so each lane stores one dword (4 channels of one
// token) per 4 tokens.  The bit window is refilled without branches: every
// symbol reads the window dword at q (the next one to append) alongside its
// L1 read, and the following symbol appends it when 32 bits or fewer are
// left, so no LDS latency beyond the table lookup sits on the chain.
template <class Tab>
__device__ __forceinline__ void decode_block_fast(const Tab &tb, int T, int C,
                                                  const uint32_t *win, uint32_t win_last,
                                                  uint32_t lo, uint32_t hi, uint8_t *obuf,
                                                  uint8_t *__restrict__ out_blk) {
  const int lane = static_cast<int>(threadIdx.x);
  uint32_t q = lo & ~3u;
  uint64_t buf = static_cast<uint64_t>(clip_word(win[q >> 2], q, hi)) << 32;
  buf <<= 8 * (lo & 3u);
  int have = 32 - 8 * static_cast<int>(lo & 3u);
  q += 4;
  uint32_t nraw = win[(q < win_last ? q : win_last) >> 2];
  auto step = [&]() -> int {
    const bool refill = have <= 32;  // leaves more than 32 bits; codes are <= 15
    const uint32_t w = refill ? clip_word(nraw, q, hi) : 0u;
    buf |= static_cast<uint64_t>(w) << (refill ? 32 - have : 0);
    have += refill ? 32 : 0;
    q += refill ? 4u : 0u;
    int s, len;
    const uint32_t v = static_cast<uint32_t>(buf >> 48);
    nraw = win[(q < win_last ? q : win_last) >> 2];
    tb.lookup(v, s, len);
    buf <<= len;
    have -= len;
    return s;
  };
  // Lane j stores token (t0 + j / 16), channels 4 * (j % 16) .. + 3.
  uint32_t *odst = reinterpret_cast<uint32_t *>(out_blk + static_cast<int64_t>(lane >> 4) * C) + (lane & 15);
  const int64_t step4 = static_cast<int64_t>(C);  // in dwords: 4 tokens of C bytes
  int t = 0;
  for (; t + 4 <= T; t += 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) obuf[i * kDecLanes + lane] = static_cast<uint8_t>(step());
    wave_sync();
    cg_st(odst, reinterpret_cast<const uint32_t *>(obuf)[lane]);
    odst += step4;
    wave_sync();
  }
  if (t < T) {
    for (int i = 0; t + i < T; ++i) obuf[i * kDecLanes + lane] = static_cast<uint8_t>(step());
    wave_sync();
    if ((lane >> 4) < T - t) cg_st(odst, reinterpret_cast<const uint32_t *>(obuf)[lane]);
  }
}


// Fast path of the byte tables: every stream of the block lies in the window
// and no table entry is an escape, so each symbol is one LDS read and the
// loop has no branches (cgdec::BitCursor, cgdec::ByteTables::step).
// Symbols go through the 4-token LDS transpose as in decode_block_fast.
__device__ __forceinline__ void decode_block_bytes(const cgdec::ByteTables &tb, int T, int C,
                                                   const uint32_t *win, uint32_t win_last,
                                                   uint32_t lo, uint32_t hi, uint8_t *obuf,
                                                   uint8_t *__restrict__ out_blk) {
  const int lane = static_cast<int>(threadIdx.x);
  cgdec::BitCursor cur;
  cur.start(win, win_last, 8 * lo, hi);
  auto step = [&]() -> uint32_t { return tb.step(cur) >> 3; };
  // Lane j stores token (t0 + j / 16), channels 4 * (j % 16) .. + 3.
  uint32_t *odst = reinterpret_cast<uint32_t *>(out_blk + static_cast<int64_t>(lane >> 4) * C) + (lane & 15);
  const int64_t step4 = static_cast<int64_t>(C);  // in dwords: 4 tokens of C bytes
  int t = 0;
  for (; t + 4 <= T; t += 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) obuf[i * kDecLanes + lane] = static_cast<uint8_t>(step());
    wave_sync();
    cg_st(odst, reinterpret_cast<const uint32_t *>(obuf)[lane]);
    odst += step4;
    wave_sync();
  }
  if (t < T) {
    for (int i = 0; t + i < T; ++i) obuf[i * kDecLanes + lane] = static_cast<uint8_t>(step());
    wave_sync();
    if ((lane >> 4) < T - t) cg_st(odst, reinterpret_cast<const uint32_t *>(obuf)[lane]);
  }
}

// Blocks whose streams all fit the window: byte tables without an escape
// entry in any lane take the branch-free loop, every other block the loop
// with the escape branch.
__device__ __forceinline__ void decode_fast(const cgdec::ByteTables &tb, int T, int C,
                                            const uint32_t *win, uint32_t win_last, uint32_t lo,
                                            uint32_t hi, uint8_t *obuf, uint8_t *__restrict__ out_blk) {
  if (__any(tb.escapes)) {
    cgdec::ByteTables t = tb;
    t.finish();
    decode_block_fast(t, T, C, win, win_last, lo, hi, obuf, out_blk);
  } else {
    decode_block_bytes(tb, T, C, win, win_last, lo, hi, obuf, out_blk);
  }
}

__device__ __forceinline__ void decode_fast(const DecTables &tb, int T, int C, const uint32_t *win,
                                            uint32_t win_last, uint32_t lo, uint32_t hi, uint8_t *obuf,
                                            uint8_t *__restrict__ out_blk) {
  decode_block_fast(tb, T, C, win, win_last, lo, hi, obuf, out_blk);
}

// One stream occupying [lo, hi) (addresses), symbols to o[0], o[C], ...
// kWin: every dword the stream needs is in the LDS window holding the bytes
// from a_lo to a_hi, read with the index clamped into the window.
// Otherwise dwords come from global memory, and only those holding a byte
// of [lo, hi) are read.
template <bool kWin, class Tab>
__device__ __forceinline__ void decode_stream(const Tab &tb, int T, int C,
                                              const uint8_t *__restrict__ bytes, const uint32_t *win,
                                              uintptr_t a_lo, uintptr_t a_hi, uintptr_t lo,
                                              uintptr_t hi, uint8_t *__restrict__ o) {
  const uintptr_t base0 = reinterpret_cast<uintptr_t>(bytes);
  auto word_at = [&](uintptr_t q) -> uint32_t {
    if (kWin) {
      const uint32_t last = static_cast<uint32_t>(a_hi - a_lo) - 4;
      return win_word(win, last, static_cast<uint32_t>(q - a_lo), static_cast<uint32_t>(hi - a_lo));
    }
    uint32_t raw = 0;
    if (q < hi) raw = *reinterpret_cast<const uint32_t *>(bytes + (q - base0));
    return __builtin_bswap32(raw & live_mask(q, lo, hi));
  };
  uintptr_t q = lo & ~uintptr_t(3);
  uint64_t buf = static_cast<uint64_t>(word_at(q)) << 32;
  q += 4;
  buf <<= 8 * (lo & 3);
  int have = 32 - 8 * static_cast<int>(lo & 3);
  for (int t = 0; t < T; ++t) {
    if (have <= 32) {
      buf |= static_cast<uint64_t>(word_at(q)) << (32 - have);
      have += 32;
      q += 4;
    }
    int s, len;
    tb.lookup(static_cast<uint32_t>(buf >> 48), s, len);
    o[static_cast<int64_t>(t) * C] = static_cast<uint8_t>(s);
    buf <<= len;
    have -= len;
  }
}

// Stream geometry of one decode block: lane i of a wave owns stream
// s0 + i; bytes of the block's streams are [B0, B1) of the byte buffer.
struct DecBlock {
  int l, c0, cnt;
  int64_t s0, start, end, B0, B1;
  uintptr_t R0, R1, r_lo;

  __device__ __forceinline__ void init(const int16_t *cdf, int64_t nbytes, const int32_t *prefix,
                                       int C, int nb, int tiles, int lane) {
    l = blockIdx.x / tiles;
    c0 = (blockIdx.x % tiles) * kDecLanes;
    cnt = C - c0 < kDecLanes ? C - c0 : kDecLanes;
    s0 = static_cast<int64_t>(l) * C + c0;
    const int64_t stream = s0 + (lane < cnt ? lane : 0);
    auto clampb = [&](int64_t x) { return x < 0 ? 0 : (x > nbytes ? nbytes : x); };
    start = clampb(stream == 0 ? 0 : prefix[stream - 1]);
    end = clampb(prefix[stream]);
    end = end < start ? start : end;
    B0 = clampb(s0 == 0 ? 0 : prefix[s0 - 1]);
    B1 = clampb(prefix[s0 + cnt - 1]);
    // Rows: bytes [R0, R1) from the 16-byte aligned address at or below R0.
    R0 = reinterpret_cast<uintptr_t>(cdf + s0 * (nb + 1));
    R1 = R0 + static_cast<uintptr_t>(cnt) * (nb + 1) * 2;
    r_lo = R0 & ~uintptr_t(15);
  }

  // 16-byte chunks of the window staged from a_lo: the block's bytes from
  // the 16-byte aligned address at or below B0, at most cap bytes.  Every
  // chunk staged (rows or window) holds a byte of its range, so no load
  // leaves the buffers' pages.
  __device__ __forceinline__ int win_chunks(uintptr_t base0, uintptr_t a_lo, int cap) const {
    if (B1 <= B0) return 0;
    const uintptr_t want = base0 + B1 - a_lo;
    const uintptr_t c = static_cast<uintptr_t>(cap);
    return static_cast<int>(((want < c ? want : c) + 15) >> 4);
  }
};

// One wave decodes the block's 64 streams, one lane per stream.
// LDS: [tables][obuf: 4 tokens x 64 lanes][staged rows][byte window].
template <class Tab>
__device__ __forceinline__ void decode_one_wave(uint8_t *lds, const int16_t *__restrict__ cdf,
                                                const uint8_t *__restrict__ bytes, int64_t nbytes,
                                                const int32_t *__restrict__ prefix, int T, int C,
                                                int nb, uint8_t *__restrict__ out, int tiles,
                                                int lane) {
  constexpr int kRowsOff = Tab::kBytes + kObufBytes;
  const int rows_cap = ((nb + 1) * kDecLanes * 2 + 32 + 15) & ~15;
  const int win_off = kRowsOff + rows_cap;
  const int win_cap = (kDecLds - win_off) & ~15;
  DecBlock bk;
  bk.init(cdf, nbytes, prefix, C, nb, tiles, lane);
  const int live = lane < bk.cnt;
  const uintptr_t base0 = reinterpret_cast<uintptr_t>(bytes);
  const uintptr_t a_lo = (base0 + bk.B0) & ~uintptr_t(15);
  const int n16 = bk.win_chunks(base0, a_lo, win_cap);
  const int nrow = static_cast<int>((bk.R1 - bk.r_lo + 15) >> 4);
  // The rows' loads are issued first and the window's behind them; the
  // table is built from the stored rows while the window is in flight.
  chunk16 rv[kRowChunks], wv[kWinChunks];
  load_chunks(bk.r_lo, nrow, 0, lane, rv);
  // Without a window the rows' first chunk is loaded and dropped, so no
  // branch separates these loads from the row stores that wait for rv only.
  load_chunks(n16 > 0 ? a_lo : bk.r_lo, n16 > 0 ? n16 : 1, 0, lane, wv);
  Tab tb;
  tb.bind(lds, lane);
  tb.clear();
  store_chunks<false>(lds + kRowsOff, nrow, 0, lane, rv);
  for (int j0 = kDecLanes * kRowChunks; j0 < nrow; j0 += kDecLanes * kRowChunks) {
    load_chunks(bk.r_lo, nrow, j0, lane, rv);
    store_chunks<false>(lds + kRowsOff, nrow, j0, lane, rv);
  }
  wave_sync();
  tb.row.r = reinterpret_cast<const int16_t *>(lds + kRowsOff + (bk.R0 - bk.r_lo)) + lane * (nb + 1);
  tb.nb = nb;
  if (live) tb.build(lds + Tab::kBytes + lane);  // obuf byte: scratch for skipped writes
  if (n16 > 0) {
    store_chunks<true>(lds + win_off, n16, 0, lane, wv);
    for (int j0 = kDecLanes * kWinChunks; j0 < n16; j0 += kDecLanes * kWinChunks) {
      load_chunks(a_lo, n16, j0, lane, wv);
      store_chunks<true>(lds + win_off, n16, j0, lane, wv);
    }
  }
  wave_sync();
  const uintptr_t lo = base0 + static_cast<uintptr_t>(bk.start);
  const uintptr_t hi = base0 + static_cast<uintptr_t>(bk.end);
  const uintptr_t a_hi = a_lo + 16 * static_cast<uintptr_t>(n16);
  const bool in_win = hi > lo && (lo & ~uintptr_t(3)) >= a_lo && ((hi + 3) & ~uintptr_t(3)) <= a_hi;
  const bool fast = bk.cnt == kDecLanes && (reinterpret_cast<uintptr_t>(out) & 3) == 0 && (C & 3) == 0 &&
                    __all(in_win);
  if (!live) return;
  const uint32_t *win = reinterpret_cast<const uint32_t *>(lds + win_off);
  uint8_t *out_blk = out + static_cast<int64_t>(bk.l) * T * C + bk.c0;
  if (fast) {
    decode_fast(tb, T, C, win, static_cast<uint32_t>(a_hi - a_lo) - 4,
                static_cast<uint32_t>(lo - a_lo), static_cast<uint32_t>(hi - a_lo),
                lds + Tab::kBytes, out_blk);
  } else {
    tb.finish();
    if (in_win)
      decode_stream<true>(tb, T, C, bytes, win, a_lo, a_hi, lo, hi, out_blk + lane);
    else
      decode_stream<false>(tb, T, C, bytes, win, a_lo, a_hi, lo, hi, out_blk + lane);
  }
}

// Byte tables with per-lane stream regions (cgdec::LaneRegion): each lane
// stages the 16-byte aligned chunks holding its own stream into its own LDS
// region and zeroes what lies past the stream's end, so the cursors read
// the region without masking the stream's end: cgdec::GroupCursor for
// tables without escapes (four codes per group, windows re-read from the
// region on a fixed schedule), cgdec::LaneCursor for the others.  The 256
// bytes after the table (obuf) are scratch while the table is built.
// Serves full 64-stream blocks with dword-aligned output rows whose regions
// fit the LDS left after the tables and rows; returns false, having written
// nothing, for any other block, which then takes decode_one_wave.
__device__ __forceinline__ bool decode_one_wave_lanes(uint8_t *lds, const int16_t *__restrict__ cdf,
                                                      const uint8_t *__restrict__ bytes, int64_t nbytes,
                                                      const int32_t *__restrict__ prefix, int T, int C, int nb,
                                                      uint8_t *__restrict__ out, int tiles, int lane) {
  using Tab = cgdec::ByteTables;
  constexpr int kRowsOff = Tab::kBytes + kObufBytes;
  constexpr int kLaneBatch = 8;  // 16-byte chunks per lane and load batch
  const int rows_cap = ((nb + 1) * kDecLanes * 2 + 32 + 15) & ~15;
  const int reg_off = kRowsOff + rows_cap;
  const uint32_t reg_cap = static_cast<uint32_t>((kDecLds - reg_off) & ~15);
  // LDS address of the block's table (the start of the kernel's dynamic
  // LDS); the table step ORs a dword offset into it.
  const uint32_t lds_at =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t *)lds));
  DecBlock bk;
  bk.init(cdf, nbytes, prefix, C, nb, tiles, lane);
  if (bk.cnt != kDecLanes || (reinterpret_cast<uintptr_t>(out) & 3) != 0 || (C & 3) != 0 ||
      (lds_at & (Tab::kBytes - 1)) != 0)
    return false;
  // The rows' loads depend on the block alone: issued before the stream
  // lengths (prefix loads) are waited for.
  const int nrow = static_cast<int>((bk.R1 - bk.r_lo + 15) >> 4);
  chunk16 rv[kRowChunks], cv[kLaneBatch];
  load_chunks(bk.r_lo, nrow, 0, lane, rv);
  const uintptr_t base0 = reinterpret_cast<uintptr_t>(bytes);
  const uintptr_t s_lo = base0 + static_cast<uintptr_t>(bk.start);
  const uintptr_t s_hi = base0 + static_cast<uintptr_t>(bk.end);
  const uint32_t len = static_cast<uint32_t>(bk.end - bk.start);
  const uintptr_t a0 = s_lo & ~uintptr_t(15);
  // Chunks [a0, a0 + 16 n_ch) each hold a byte of the stream, so no load
  // leaves the buffer's pages.
  const uint32_t n_ch = len ? static_cast<uint32_t>(((s_hi - 1) >> 4) - (s_lo >> 4) + 1) : 0u;
  const uint32_t rbytes = 16u * n_ch + cgdec::LaneRegion::kRoom;  // chunks plus the sealed room
  uint32_t incl = rbytes, n_max = n_ch;
#pragma unroll
  for (int d = 1; d < kDecLanes; d <<= 1) {
    const uint32_t v = __shfl_up(incl, d, kDecLanes);
    incl += lane >= d ? v : 0u;
    const uint32_t m = __shfl_xor(n_max, d, kDecLanes);
    n_max = m > n_max ? m : n_max;
  }
  const uint32_t total = __shfl(incl, kDecLanes - 1, kDecLanes);
  if (total > reg_cap) return false;
  uint8_t *region = lds + reg_off + (incl - rbytes);
  Tab tb;
  tb.bind(lds, lane, lds_at);
  tb.clear();
  store_chunks<false>(lds + kRowsOff, nrow, 0, lane, rv);
  for (int j0 = kDecLanes * kRowChunks; j0 < nrow; j0 += kDecLanes * kRowChunks) {
    load_chunks(bk.r_lo, nrow, j0, lane, rv);
    store_chunks<false>(lds + kRowsOff, nrow, j0, lane, rv);
  }
  // The first batch of the lane's chunks, issued once the rows have landed
  // (every wave of the launch loads its rows and streams at its start, so
  // the rows, which the table build needs first, do not share the memory
  // system with the larger streams); the table is built while the chunks
  // are in flight.
#pragma unroll
  for (int u = 0; u < kLaneBatch; ++u)
    if (static_cast<uint32_t>(u) < n_ch) cv[u] = reinterpret_cast<global_chunk16 *>(a0)[u];
  wave_sync();
  tb.row.r = reinterpret_cast<const int16_t *>(lds + kRowsOff + (bk.R0 - bk.r_lo)) + lane * (nb + 1);
  tb.nb = nb;
  tb.build(lds + Tab::kBytes + lane);  // obuf byte: scratch for skipped writes
#pragma unroll
  for (int u = 0; u < kLaneBatch; ++u)
    if (static_cast<uint32_t>(u) < n_ch) reinterpret_cast<chunk16 *>(region)[u] = cv[u];
  for (uint32_t k0 = kLaneBatch; k0 < n_max; k0 += kLaneBatch) {
#pragma unroll
    for (int u = 0; u < kLaneBatch; ++u)
      if (k0 + u < n_ch) cv[u] = reinterpret_cast<global_chunk16 *>(a0)[k0 + u];
#pragma unroll
    for (int u = 0; u < kLaneBatch; ++u)
      if (k0 + u < n_ch) reinterpret_cast<chunk16 *>(region)[k0 + u] = cv[u];
  }
  uint32_t *reg32 = reinterpret_cast<uint32_t *>(region);
  cgdec::LaneRegion::seal(reg32, static_cast<uint32_t>(s_lo - a0), len);
  uint8_t *obuf = lds + Tab::kBytes;
  uint8_t *out_blk = out + static_cast<int64_t>(bk.l) * T * C + bk.c0;
  // Lane j stores token (t0 + j / 16), channels 4 * (j % 16) .. + 3.
  uint32_t *odst = reinterpret_cast<uint32_t *>(out_blk + static_cast<int64_t>(lane >> 4) * C) + (lane & 15);
  const int64_t step4 = static_cast<int64_t>(C);  // in dwords: 4 tokens of C bytes
  if (!__any(tb.escapes)) {
    // Four tokens per group (cgdec::GroupCursor): the four table entries go
    // through the LDS transpose and the symbols of the resulting word are
    // extracted at once, (word >> 3) & 0x1F1F1F1F; each word is stored one
    // group late, so no group waits for its own transpose read.  The
    // transpose writes, that store and the transposing read sit between the
    // group's codes, each under a table read (the cursor's scheduling
    // barriers keep them there).  Measured on MI355X (symbol loop, shader
    // cycles per symbol, s_memtime stamps): 128-133 with the refilled lane
    // cursor (its chain four VALU instructions and the table read, the
    // refill on it every fourth code) -> 112 with this cursor -> 102 with
    // the transpose spread between the codes -> 100 with the window's
    // permutations one code later.  The chain alone, timed in isolation,
    // takes 72 cycles; the rest is issue of the other instructions under
    // it and LDS traffic.
    cgdec::GroupCursor gc;
    gc.start(tb, reg32, lds_at + static_cast<uint32_t>(region - lds), static_cast<uint32_t>(s_lo - a0), len);
    int t = 0;
    uint32_t word = 0;
    for (; t + 4 <= T; t += 4) {
      const uint32_t e0 = gc.step0(tb);
      const uint32_t e1 = gc.step1(tb);
      obuf[lane] = static_cast<uint8_t>(e0);
      if (t > 0) {
        cg_st(odst, (word >> 3) & 0x1F1F1F1Fu);
        odst += step4;
      }
      const uint32_t e2 = gc.step2(tb);
      obuf[kDecLanes + lane] = static_cast<uint8_t>(e1);
      const uint32_t e3 = gc.step3(tb);
      obuf[2 * kDecLanes + lane] = static_cast<uint8_t>(e2);
      obuf[3 * kDecLanes + lane] = static_cast<uint8_t>(e3);
      wave_sync();
      word = reinterpret_cast<const uint32_t *>(obuf)[lane];
      wave_sync();
    }
    if (t > 0) {
      cg_st(odst, (word >> 3) & 0x1F1F1F1Fu);
      odst += step4;
    }
    if (t < T) {
      for (int i = 0; t + i < T; ++i) obuf[i * kDecLanes + lane] = static_cast<uint8_t>(gc.single(tb));
      wave_sync();
      if ((lane >> 4) < T - t) cg_st(odst, reinterpret_cast<const uint32_t *>(obuf)[lane]);
    }
  } else {
    tb.finish();
    cgdec::LaneCursor cur;
    cur.start(reg32, static_cast<uint32_t>(s_lo - a0), len);
    auto step = [&]() -> uint8_t {
      int s, l;
      tb.lookup(cur.top16(), s, l);
      cur.consume(l);
      cur.refill();
      return static_cast<uint8_t>(s);
    };
    int t = 0;
    for (; t + 4 <= T; t += 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) obuf[i * kDecLanes + lane] = step();
      wave_sync();
      cg_st(odst, reinterpret_cast<const uint32_t *>(obuf)[lane]);
      odst += step4;
      wave_sync();
    }
    if (t < T) {
      for (int i = 0; t + i < T; ++i) obuf[i * kDecLanes + lane] = step();
      wave_sync();
      if ((lane >> 4) < T - t) cg_st(odst, reinterpret_cast<const uint32_t *>(obuf)[lane]);
    }
  }
  return true;
}

template <class Tab>
__global__ void __launch_bounds__(kDecLanes)
    decode_kernel(const int16_t *__restrict__ cdf,
                  const uint8_t *__restrict__ bytes, int64_t nbytes,
                  const int32_t *__restrict__ prefix, int T, int C, int nb,
                  uint8_t *__restrict__ out, int tiles) {
  extern __shared__ uint32_t lds_words[];
  uint8_t *lds = reinterpret_cast<uint8_t *>(lds_words);
  const int lane = static_cast<int>(threadIdx.x);
  if constexpr (std::is_same<Tab, cgdec::ByteTables>::value) {
    if (LMC_DEC_LANES && decode_one_wave_lanes(lds, cdf, bytes, nbytes, prefix, T, C, nb, out, tiles, lane))
      return;
  }
  decode_one_wave<Tab>(lds, cdf, bytes, nbytes, prefix, T, C, nb, out, tiles, lane);
}

// Row-major contiguity; a tensor without elements has no layout to check.
bool contiguous(const lmc_tensor &t) {
  if (numel(t) == 0) return true;
  int64_t expect = 1;
  for (int i = t.ndim - 1; i >= 0; --i) {
    if (t.sizes[i] != 1 && t.strides[i] != expect) return false;
    expect *= t.sizes[i];
  }
  return true;
}

void need_device(const lmc_tensor &t, const char *what) {
  check(t.device >= 0, std::string(what) + " is not a GPU tensor");
  check(contiguous(t), std::string(what) + " must be contiguous");
}

} // namespace

} // namespace lmc

using namespace lmc;

extern "C" {

int lmc_calculate_cdf(const lmc_tensor *input, int32_t n_bins,
                      const lmc_tensor *output, void *stream) {
  return guarded([&] {
    const lmc_tensor &in = deref(input, "input");
    const lmc_tensor &o = deref(output, "output");
    need_device(in, "input");
    need_device(o, "output");
    check(in.ndim == 3, "input must be [layers, tokens, channels]");
    check(in.dtype == LMC_U8 || in.dtype == LMC_I8, "input must be uint8/int8");
    check(o.dtype == LMC_I16, "output must be int16");
    check(n_bins >= 1 && n_bins <= kMaxBins,
          "n_bins must be in [1, " + std::to_string(kMaxBins) + "]");
    const int64_t L = in.sizes[0], T = in.sizes[1], C = in.sizes[2];
    check(o.ndim == 3 && o.sizes[0] == L && o.sizes[1] == C &&
              o.sizes[2] == n_bins + 1,
          "output must be [layers, channels, n_bins + 1]");
    check(T < (int64_t(1) << 26) && C < (int64_t(1) << 30), "input too large");
    if (L == 0 || C == 0) return;
    DeviceGuard guard(in.device);
    const int tiles64 = static_cast<int>((C + 63) / 64);
    const size_t lds = static_cast<size_t>(cdf_lds_bytes(static_cast<int>(T), n_bins));
    const int vec_tile = (C % 16 == 0 && (reinterpret_cast<uintptr_t>(in.data) & 15) == 0) ? 1 : 0;
    const auto kern = n_bins == 32         ? cdf_tile_kernel<32, true>
                      : n_bins < 32          ? cdf_tile_kernel<32, false>
                      : n_bins == kMaxBins   ? cdf_tile_kernel<kMaxBins, true>
                                             : cdf_tile_kernel<kMaxBins, false>;
    hipLaunchKernelGGL(kern, dim3(L * tiles64), dim3(kCdfThreads), lds, static_cast<hipStream_t>(stream),
                       static_cast<const uint8_t *>(in.data), (int)T, (int)C, n_bins,
                       static_cast<int16_t *>(o.data), tiles64, vec_tile);
    hip_check(hipGetLastError(), "cdf_tile_kernel launch");
  });
}

int lmc_encode_fast_new(const lmc_tensor *cdf_t, const lmc_tensor *input_sym,
                        const lmc_tensor *output_buffer,
                        const lmc_tensor *output_lengths, void *stream) {
  return guarded([&] {
    const lmc_tensor &cdf = deref(cdf_t, "cdf");
    const lmc_tensor &in = deref(input_sym, "input_sym");
    const lmc_tensor &ob = deref(output_buffer, "output_buffer");
    const lmc_tensor &ol = deref(output_lengths, "output_lengths");
    need_device(cdf, "cdf");
    need_device(in, "input_sym");
    need_device(ob, "output_buffer");
    need_device(ol, "output_lengths");
    check(in.ndim == 3 && cdf.ndim == 3 && ob.ndim == 3,
          "cdf, input_sym and output_buffer must be 3-D");
    const int64_t L = in.sizes[0], T = in.sizes[1], C = in.sizes[2];
    const int64_t nb = cdf.sizes[2] - 1;
    const int64_t chunk = ob.sizes[2];
    // csrc/cachegen_kernels.cpp:33-35
    check(C <= (1 << 15),
          "encode takes at most 32768 channels per layer");
    check(in.dtype == LMC_U8 || in.dtype == LMC_I8, "input_sym must be int8/uint8");
    check(cdf.dtype == LMC_I16, "cdf must be int16");
    check(ob.dtype == LMC_U8 || ob.dtype == LMC_I8, "output_buffer must be uint8");
    check(ol.dtype == LMC_I32 && numel(ol) == L * C, "output_lengths must be int32 [L, C]");
    check(nb >= 1 && nb <= kMaxBins, "number of bins must be in [1, 64]");
    check(cdf.sizes[0] == L && cdf.sizes[1] == C, "cdf must be [L, C, nbins + 1]");
    check(ob.sizes[0] == L && ob.sizes[1] == C, "output_buffer must be [L, C, chunk]");
    if (L == 0 || C == 0) return;
    DeviceGuard guard(in.device);
    const int tiles = static_cast<int>((C + kEncLanes - 1) / kEncLanes);
    const int word_stores =
        (chunk % 4 == 0 && (reinterpret_cast<uintptr_t>(ob.data) & 3) == 0) ? 1 : 0;
    const int vec_in = (C % 16 == 0 && (reinterpret_cast<uintptr_t>(in.data) & 15) == 0) ? 1 : 0;
    const bool rows_dw = (reinterpret_cast<uintptr_t>(cdf.data) & 3) == 0;
    if (LMC_ENC_SPLIT && T > 0 && T <= kEncTileMaxT && nb <= kEncLanes && C % kEncLanes == 0 && vec_in &&
        rows_dw) {
      // Split encoder: bit rows of 2T bytes plus one word (codes are at
      // most 16 bits), an odd number of words so that the lanes' rows start
      // in different banks.
      const int row_words = (static_cast<int>(T + 1) / 2 + 1) | 1;
      const int rows_words = static_cast<int>(((nb + 1) * kEncLanes * 2 + 15) / 16 * 4);
      const int phase1 = rows_words + kEncTileMaxT * kEncLanes / 4 + static_cast<int>(nb + 1) * kEncLanes;
      const int stage_words = std::max(phase1, kEncLanes * row_words);
      const size_t lds = 4 * (static_cast<size_t>((stage_words + kEncPieces * kEncLanes + 2) & ~1) + 2 * kEncLanes);
      check(lds <= 65536, "encode: LDS budget exceeded");
      hipLaunchKernelGGL(encode_split_kernel<kEncPieces>, dim3(L * tiles), dim3(64 * kEncPieces), lds,
                         static_cast<hipStream_t>(stream),
                         static_cast<const int16_t *>(cdf.data),
                         static_cast<const uint8_t *>(in.data), (int)T, (int)C,
                         (int)nb, static_cast<uint8_t *>(ob.data), chunk,
                         static_cast<int32_t *>(ol.data), tiles, word_stores, row_words, stage_words);
      hip_check(hipGetLastError(), "encode_split_kernel launch");
      return;
    }
    if (T > 0 && T <= kEncTileMaxT && nb <= kEncLanes) {
      // Bits past min(chunk, 2 bytes per symbol) are never written (codes
      // are at most 16 bits), so a wave's bit buffer holds that many bytes.
      const int64_t cap_bytes = std::min<int64_t>(chunk, 2 * T);
      const int cap_words = static_cast<int>((cap_bytes + 3) / 4);
      const int sym_stride = (((T + 3) / 4) + 1) | 1;
      const size_t lds = 4 * ((static_cast<size_t>(nb + 1) * kEncLanes * 2 + 15) / 16 * 4 +
                              static_cast<size_t>(kEncLanes) * sym_stride +
                              static_cast<size_t>(2 * kEncWaves) * cap_words);
      const int vec_tile = vec_in;
      check(lds <= 65536, "encode: LDS budget exceeded");
      hipLaunchKernelGGL(encode_wave_kernel, dim3(L * tiles), dim3(kEncTileThreads), lds,
                         static_cast<hipStream_t>(stream),
                         static_cast<const int16_t *>(cdf.data),
                         static_cast<const uint8_t *>(in.data), (int)T, (int)C,
                         (int)nb, static_cast<uint8_t *>(ob.data), chunk,
                         static_cast<int32_t *>(ol.data), tiles, word_stores, vec_tile, sym_stride,
                         cap_words);
      hip_check(hipGetLastError(), "encode_wave_kernel launch");
      return;
    }
    const size_t lds = static_cast<size_t>(nb) * kEncLanes * 4 +
                       static_cast<size_t>(nb + 1) * kEncLanes * 2;
    hipLaunchKernelGGL(encode_kernel, dim3(L * tiles), dim3(kEncLanes), lds,
                       static_cast<hipStream_t>(stream),
                       static_cast<const int16_t *>(cdf.data),
                       static_cast<const uint8_t *>(in.data), (int)T, (int)C,
                       (int)nb, static_cast<uint8_t *>(ob.data), chunk,
                       static_cast<int32_t *>(ol.data), tiles, word_stores);
    hip_check(hipGetLastError(), "encode_kernel launch");
  });
}

int lmc_decode_fast_new(const lmc_tensor *, const lmc_tensor *,
                        const lmc_tensor *, const lmc_tensor *, void *) {
  // csrc/cachegen_kernels.cpp:60-65
  set_last_error("decode_fast_new is not implemented; use decode_fast_prefsum");
  return LMC_ERR_NOT_IMPLEMENTED;
}

int lmc_decode_fast_prefsum(const lmc_tensor *cdf_t,
                            const lmc_tensor *bytestreams,
                            const lmc_tensor *lengths,
                            const lmc_tensor *output, void *stream) {
  return guarded([&] {
    const lmc_tensor &cdf = deref(cdf_t, "cdf");
    const lmc_tensor &bs = deref(bytestreams, "bytestreams");
    const lmc_tensor &ln = deref(lengths, "lengths");
    const lmc_tensor &o = deref(output, "output");
    // csrc/cachegen_kernels.cpp:78-88
    check(cdf.device >= 0, "cdf is not a GPU tensor");
    check(bs.device >= 0, "bytestreams is not a GPU tensor");
    check(ln.device >= 0, "lengths is not a GPU tensor");
    check(o.device >= 0, "output is not a GPU tensor");
    need_device(cdf, "cdf");
    need_device(bs, "bytestreams");
    need_device(ln, "lengths");
    need_device(o, "output");
    check(cdf.ndim == 3, "cdf must be [L, C, nbins + 1]");
    const int64_t L = cdf.sizes[0], C = cdf.sizes[1], nb = cdf.sizes[2] - 1;
    check(C % 32 == 0, "decode takes a channel count that is a multiple of 32");
    check(nb < 64, "decode takes fewer than 64 bins per stream");
    check(nb >= 1, "cdf needs at least one bin");
    check(cdf.dtype == LMC_I16, "cdf must be int16");
    check(bs.dtype == LMC_U8 || bs.dtype == LMC_I8, "bytestreams must be uint8");
    check(ln.dtype == LMC_I32 && numel(ln) == L * C, "lengths must be int32 [L, C]");
    check(o.dtype == LMC_U8 || o.dtype == LMC_I8, "output must be uint8");
    check(o.ndim >= 2, "output must be [L, T, C]");
    const int64_t T = o.sizes[1];
    check(numel(o) == L * T * C, "output must hold L * T * C symbols");
    if (L == 0 || C == 0 || T == 0) return;
    DeviceGuard guard(bs.device);
    const int tiles = static_cast<int>((C + kDecLanes - 1) / kDecLanes);
    const size_t lds = kDecLds;
    hipLaunchKernelGGL(nb <= cgdec::ByteTables::kMaxBins ? decode_kernel<cgdec::ByteTables>
                                                       : decode_kernel<DecTables>,
                       dim3(L * tiles), dim3(kDecLanes), lds,
                       static_cast<hipStream_t>(stream),
                       static_cast<const int16_t *>(cdf.data),
                       static_cast<const uint8_t *>(bs.data), numel(bs),
                       static_cast<const int32_t *>(ln.data), (int)T, (int)C,
                       (int)nb, static_cast<uint8_t *>(o.data), tiles);
    hip_check(hipGetLastError(), "decode_kernel launch");
  });
}

} // extern "C"
