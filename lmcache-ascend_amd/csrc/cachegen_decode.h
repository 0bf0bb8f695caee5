// Per-stream decode tables of the CacheGen decoder (rules L1-L3 and L6 of
// the codec: bases are the CDF entries with their low 4 bits cleared, the
// low bits carry the code length, an entry below its predecessor stands for
// 0x10000, and decode takes the largest symbol whose base is <= the next 16
// stream bits).
//
// This header holds only integer logic on plain pointers, so the same code
// can be compiled for the host and checked there against the rule.
#pragma once

#include <stdint.h>

namespace lmc {
namespace cgdec {

constexpr int kPrec = 16;
constexpr int kLanes = 64;  // streams per decode block (one wave)

// Bases and lengths read straight from a staged raw CDF row.  `wrap` is the
// first symbol whose entry is below its predecessor's (nb if none): it and
// every later symbol have base 0x10000.
struct StagedRow {
  const int16_t *r;
  int wrap;
  __device__ __forceinline__ uint32_t base(int s) const {
    return s >= wrap ? 0x10000u : (static_cast<uint32_t>(static_cast<uint16_t>(r[s])) & 0xFFF0u);
  }
  __device__ __forceinline__ int len(int s) const {
    const int nib = static_cast<uint16_t>(r[s]) & 0xF;
    if (nib) return nib;
    const uint32_t w = base(s + 1) - base(s);
    return w ? kPrec - (31 - __builtin_clz(w)) : 0;
  }
};

// The 32 bits of {hi, lo} starting s bits below the top of hi, for s in
// [1, 32] (one v_alignbit_b32).
__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t s) {
  return static_cast<uint32_t>(((static_cast<uint64_t>(hi) << 32) | lo) >> (32 - s));
}

// Bit cursor over one stream in a window of big-endian dwords (the first
// stream byte is the top byte of its dword).  The stream occupies window
// bytes [lo, hi); bytes at or past hi read as zero, and reads past the
// window's last dword (byte offset `last`) are clamped to it and masked.
// The next bits sit in three dwords a, b, c with o in [1, 32] bits of a
// consumed, so the next 32 bits are funnel(a, b, o); q is the window offset
// of the dword after c, read ahead into `ahead` at every advance so the
// shift that needs it never waits for it.  An advance of at most 32 bits
// shifts the dwords at most once.
struct BitCursor {
  const uint32_t *win;
  uint32_t last, hi;
  uint32_t a, b, c, ahead, o, q;

  __device__ __forceinline__ uint32_t word(uint32_t at) const {
    const int d = static_cast<int>(hi) - static_cast<int>(at);
    const int k = d < 0 ? 0 : (d > 4 ? 4 : d);
    const uint32_t live = static_cast<uint32_t>(0xFFFFFFFF00000000ull >> (8 * k));
    return win[(at < last ? at : last) >> 2] & live;
  }

  __device__ __forceinline__ void start(const uint32_t *w, uint32_t w_last, uint32_t lo,
                                        uint32_t end) {
    win = w;
    last = w_last;
    hi = end;
    q = lo & ~3u;
    o = 8 * (lo & 3u);
    a = 0;
    if (o == 0) {  // start at the top of b: o = 32 of a dword a that is never read
      o = 32;
      b = word(q);
      c = word(q + 4);
      q += 8;
    } else {
      a = word(q);
      b = word(q + 4);
      c = word(q + 8);
      q += 12;
    }
    ahead = word(q);
  }

  __device__ __forceinline__ uint32_t peek32() const { return funnel(a, b, o); }

  __device__ __forceinline__ void advance(uint32_t n) {
    o += n;
    const bool sh = o > 32;
    a = sh ? b : a;
    b = sh ? c : b;
    c = sh ? ahead : c;
    o -= sh ? 32u : 0u;
    q += sh ? 4u : 0u;
    ahead = word(q);
  }
};

// Byte table for n_bins <= 32: one entry per 8-bit prefix of the 16-bit
// window (256 per stream).  An entry is (s << 3) | (len - 1) when every
// window with that prefix decodes to symbol s of length 1..8, and kEscape
// (0xFF) otherwise: a symbol base strictly inside the prefix's range, a
// code longer than 8 bits or of length 0, or symbol 31 of length 8, the
// one code that would read as kEscape.  Escaped windows take a binary
// search over the bases.  Codes of calculate_cdf's rule on chunks of up to
// 256 tokens are at most 8 bits long and their bases are multiples of 256,
// so their tables hold no escapes.
//
// Layout: entry e of the lane's stream is byte (e / 4) * 256 + lane * 4 +
// e % 4 of the block's 16 KiB table, so a lane's four consecutive entries are
// one dword and the 64 lanes' lookups hit 64 distinct dwords.
//
// Build (no data-dependent loops): every symbol s >= 1 with a base b below
// 0x10000 writes its entry at prefix ceil(b / 256), where it becomes the
// decoded symbol, and kEscape at prefix floor(b / 256) when b is not a
// multiple of 256; symbols are taken in increasing order, so a later write
// at the same prefix wins, which is the larger symbol, as rule L6 wants.
// A scan then carries each written entry forward over the unwritten (zero)
// prefixes after it, starting from symbol 0's entry.  An escape written for
// a boundary is always followed by a written entry (the same symbol's, at
// the next prefix), so it never spreads; an escape written as a symbol's
// entry spreads exactly over that symbol's prefixes.
struct ByteTables {
  static constexpr int kBytes = 256 * kLanes;
  static constexpr uint32_t kEscape = 0xFFu;
  static constexpr int kMaxBins = 32;

  uint8_t *tab;  // block table + lane * 4
  StagedRow row;
  int nb;
  int top;      // largest power of two below nb (1 if nb <= 2)
  bool escapes;  // some entry is kEscape (set by build)

  __device__ __forceinline__ void bind(uint8_t *lds, int lane) { tab = lds + lane * 4; }

  __device__ __forceinline__ uint8_t *entry(uint32_t e) const {
    return tab + (e >> 2) * (kLanes * 4) + (e & 3u);
  }

  __device__ __forceinline__ void build() {
    uint32_t *t32 = reinterpret_cast<uint32_t *>(tab);
    for (int d = 0; d < 64; ++d) t32[d * kLanes] = 0;
    row.wrap = nb;
    uint32_t raw = static_cast<uint16_t>(row.r[0]);
    uint32_t base = raw & 0xFFF0u;
    uint32_t last = base;  // last base before any wrap
    uint32_t code0 = kEscape;
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
      const uint32_t code = (len >= 1 && len <= 8)
                                ? ((static_cast<uint32_t>(s) << 3) | static_cast<uint32_t>(len - 1))
                                : kEscape;
      if (s == 0) {
        code0 = code;
      } else if (base < 0x10000u) {
        if (base & 0xFFu) *entry(base >> 8) = static_cast<uint8_t>(kEscape);
        const uint32_t pos = (base + 0xFFu) >> 8;
        if (pos < 256u) *entry(pos) = static_cast<uint8_t>(code);
      }
      raw = next_raw;
      base = next;
    }
    uint32_t carry = code0, most = 0;
    for (int d = 0; d < 64; ++d) {
      const uint32_t w = t32[d * kLanes];
      uint32_t o = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t b = (w >> (8 * k)) & 0xFFu;
        carry = b ? b : carry;
        most = most > carry ? most : carry;
        o |= carry << (8 * k);
      }
      t32[d * kLanes] = o;
    }
    escapes = most == kEscape;
    top = 1;
    while (top * 2 < nb) top *= 2;
  }

  // One symbol at the cursor for a table without escapes (one LDS read, no
  // branches).
  __device__ __forceinline__ uint32_t step(BitCursor &cur) const {
    const uint32_t w = cur.peek32();
    const uint32_t e = tab[((w >> 26) << 8) + ((w >> 24) & 3u)];
    cur.advance((e & 7u) + 1);
    return e >> 3;
  }

  // Symbol and code length for the 16-bit window v.
  __device__ __forceinline__ void lookup(uint32_t v, int &s, int &len) const {
    const uint32_t b = tab[((v >> 10) << 8) + ((v >> 8) & 3u)];
    if (b != kEscape) {
      s = static_cast<int>(b >> 3);
      len = static_cast<int>(b & 7u) + 1;
    } else {
      s = 0;
      for (int step = top; step > 0; step >>= 1)
        if (s + step < nb && row.base(s + step) <= v) s += step;
      len = row.len(s);
    }
  }
};

}  // namespace cgdec
}  // namespace lmc
