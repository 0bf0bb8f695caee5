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

#ifdef __HIP__
// A dword of LDS by LDS address.
__device__ __forceinline__ uint32_t lds_dword(uint32_t at) {
  return *reinterpret_cast<const __attribute__((address_space(3))) uint32_t *>(static_cast<uintptr_t>(at));
}
// Byte k of the result is byte sel.byte[k] (0..7) of the 64-bit hi:lo.
__device__ __forceinline__ uint32_t byte_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
// The low 32 bits of the 64-bit hi:lo shifted right by s % 32.
__device__ __forceinline__ uint32_t align_bits(uint32_t hi, uint32_t lo, uint32_t s) {
  return __builtin_amdgcn_alignbit(hi, lo, s);
}
// True in every lane when b holds in some lane of the wave.
__device__ __forceinline__ bool wave_any(bool b) { return __any(b); }
#else
inline bool wave_any(bool b) { return b; }
inline uint32_t align_bits(uint32_t hi, uint32_t lo, uint32_t s) {
  return static_cast<uint32_t>(((static_cast<uint64_t>(hi) << 32) | lo) >> (s & 31u));
}
inline uint32_t byte_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  const uint64_t v = (static_cast<uint64_t>(hi) << 32) | lo;
  uint32_t r = 0;
  for (int k = 0; k < 4; ++k) r |= static_cast<uint32_t>((v >> (8 * ((sel >> (8 * k)) & 7u))) & 0xFFu) << (8 * k);
  return r;
}
// Host build of this header (tests/decode_tables_check.cpp): the table lives
// in host memory registered by host_lds_base.
inline const uint8_t *&host_lds_base() {
  static const uint8_t *base = nullptr;
  return base;
}
inline uint32_t lds_dword(uint32_t at) {
  uint32_t v;
  __builtin_memcpy(&v, host_lds_base() + at, 4);
  return v;
}
#endif
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

// Bit cursor over one stream in a window of big-endian dwords (the first
// stream byte is the top byte of its dword).  The stream occupies window
// bytes [lo, hi); bytes at or past hi read as zero, and reads past the
// window's last dword (byte offset `last`) are clamped to it and masked.
// The next bits sit in three dwords a, b, c: the next 32 bits are the 64-bit
// {a, b} shifted right by sh in [0, 31] (one v_alignbit_b32), so 32 - sh
// bits of a are consumed.  q is the window offset of the dword after c,
// read ahead into `ahead` at every advance so the shift that needs it never
// waits for it.  An advance of at most 32 bits shifts the dwords at most
// once.
struct BitCursor {
  const uint32_t *win;
  uint32_t last, hi;
  uint32_t a, b, c, ahead, q;
  int sh;

  __device__ __forceinline__ uint32_t word(uint32_t at) const {
    const int d = static_cast<int>(hi) - static_cast<int>(at);
    const int k = d < 0 ? 0 : (d > 4 ? 4 : d);
    const uint32_t live = static_cast<uint32_t>(0xFFFFFFFF00000000ull >> (8 * k));
    return win[(at < last ? at : last) >> 2] & live;
  }

  // Starts at window bit `bit` (bit 0 is the top bit of the first byte).
  __device__ __forceinline__ void start(const uint32_t *w, uint32_t w_last, uint32_t bit,
                                        uint32_t end) {
    win = w;
    last = w_last;
    hi = end;
    q = (bit >> 5) << 2;
    const uint32_t o = bit & 31u;
    a = 0;
    if (o == 0) {  // the top of b is next: a (never read) fully consumed
      sh = 0;
      b = word(q);
      c = word(q + 4);
      q += 8;
    } else {
      sh = static_cast<int>(32 - o);
      a = word(q);
      b = word(q + 4);
      c = word(q + 8);
      q += 12;
    }
    ahead = word(q);
  }

  __device__ __forceinline__ uint32_t peek32() const {
    return static_cast<uint32_t>(((static_cast<uint64_t>(a) << 32) | b) >> sh);
  }

  // Window bit of the next symbol (a holds the dword at byte q - 12).
  __device__ __forceinline__ uint32_t bitpos() const { return 8 * (q - 12) + 32 - sh; }

  // Consumes n (<= 32) bits.
  __device__ __forceinline__ void advance(int n) {
    sh -= n;
    const bool s = sh < 0;
    a = s ? b : a;
    b = s ? c : b;
    c = s ? ahead : c;
    sh &= 31;
    q += s ? 4u : 0u;
    ahead = word(q);
  }
};

// Per-lane stream regions.  A lane's stream, bytes [start, end) of the
// concatenated stream buffer, is staged as the raw little-endian dwords of
// the 16-byte aligned chunks that hold it (the first chunk starts at
// start & ~15, so the stream begins `off` = start & 15 bytes in), with
// kRoom bytes of room after them.  LaneRegion::seal zeroes what a cursor
// reads past the stream's end (the rest of the dword holding the end and
// the four dwords after it), so bits past the end read as zero; a cursor
// forms the stream's big-endian dword q from raw dwords off / 4 + q and the
// one after it with one byte permutation (swap and alignment together).
// Stream dwords from n_dw = ceil(len / 4) on read as zero through raw
// dwords n_dw .. n_dw + 3 (past off / 4), all inside the sealed part.
// An empty stream takes offset 0 (its region is the room alone).
struct LaneRegion {
  static constexpr uint32_t kRoom = 32;
  static __device__ __forceinline__ void seal(uint32_t *region, uint32_t off, uint32_t len) {
    off = len ? off : 0u;
    const uint32_t e = off + len, i = e >> 2, keep = e & 3u;
    region[i] &= keep ? 0xFFFFFFFFu >> (32u - 8u * keep) : 0u;
    region[i + 1] = 0u;
    region[i + 2] = 0u;
    region[i + 3] = 0u;
    region[i + 4] = 0u;
  }
};

// 64-bit windows of a sealed lane region: at(q) is the 64 stream bits from
// stream bit q (big-endian: the top bit is bit q), zeros past the stream's
// end.  Stream dwords j, j + 1, j + 2 (j = q / 32, clamped to n_dw, where
// every dword reads as zero) come from raw dwords j .. j + 3 by three byte
// permutations, and the window is their top 64 bits after a shift by
// q % 32, two 64-bit shifts.
struct LaneWindows {
  const uint32_t *w;  // raw region + off / 4
  uint32_t sel;       // byte permutation for the stream's offset in its dword
  uint32_t zl;        // n_dw

  __device__ __forceinline__ void start(const uint32_t *region, uint32_t off, uint32_t len) {
    off = len ? off : 0u;
    w = region + (off >> 2);
    sel = 0x00010203u + (off & 3u) * 0x01010101u;
    zl = (len + 3u) >> 2;
  }
  __device__ __forceinline__ uint64_t at(uint32_t q) const {
    const uint32_t j = (q >> 5) < zl ? (q >> 5) : zl;
    const uint32_t r0 = w[j], r1 = w[j + 1u], r2 = w[j + 2u], r3 = w[j + 3u];
    const uint32_t a = byte_perm(r1, r0, sel), b = byte_perm(r2, r1, sel), c = byte_perm(r3, r2, sel);
    const uint32_t o = q & 31u;
    const uint64_t ab = (static_cast<uint64_t>(a) << 32) | b, bc = (static_cast<uint64_t>(b) << 32) | c;
    return ((ab << o) & 0xFFFFFFFF00000000ull) | ((bc << o) >> 32);
  }
};

// Bit cursor over a sealed lane region for tables with escapes (codes of
// up to 16 bits): a 64-bit window whose top `have` bits are the stream's
// next bits (zeros past the end are real zeros), and `next`, the stream
// dword to append, read ahead.  refill() appends it when 32 bits or fewer
// are left, so after a refill more than 32 bits are valid: two codes of at
// most 16 bits can be taken between refills.  Stream dword k reads raw
// dwords min(k, n_dw) + off / 4 and the one after; from n_dw = ceil(len / 4)
// on that is sealed zeros.
struct LaneCursor {
  const uint32_t *w;  // raw region + off / 4
  uint32_t sel;       // byte permutation for the stream's offset in its dword
  uint32_t zl;        // n_dw
  uint32_t q;         // index of the stream dword in next_lo / next_hi
  uint64_t win;
  int have;
  uint32_t next_lo, next_hi;  // the raw dwords of stream dword q, read ahead

  // Big-endian: the result's top byte is the stream's first.
  __device__ __forceinline__ uint32_t form(uint32_t hi, uint32_t lo) const { return byte_perm(hi, lo, sel); }
  __device__ __forceinline__ void fetch(uint32_t k) {
    const uint32_t c = k < zl ? k : zl;
    next_lo = w[c];
    next_hi = w[c + 1u];
  }
  __device__ __forceinline__ void start(const uint32_t *region, uint32_t off, uint32_t len) {
    off = len ? off : 0u;
    w = region + (off >> 2);
    sel = 0x00010203u + (off & 3u) * 0x01010101u;
    zl = (len + 3u) >> 2;
    const uint32_t c1 = 1u < zl ? 1u : zl;
    win = (static_cast<uint64_t>(form(w[1], w[0])) << 32) | form(w[c1 + 1u], w[c1]);
    have = 64;
    q = 2u;
    fetch(q);
  }
  __device__ __forceinline__ uint32_t top16() const { return static_cast<uint32_t>(win >> 48); }
  __device__ __forceinline__ void consume(int n) {
    win <<= n;
    have -= n;
  }
  // The raw dwords are permuted here, a refill after they were read, so
  // their read is not waited for where it is issued.
  __device__ __forceinline__ void refill() {
    const bool need = have <= 32;
    const uint64_t add = static_cast<uint64_t>(form(next_hi, next_lo)) << ((32 - have) & 63);
    win |= need ? add : 0ull;
    have += need ? 32 : 0;
    q += need ? 1u : 0u;
    fetch(q);
  }
};

// Byte table for n_bins <= 32: one entry per 8-bit prefix of the 16-bit
// window (256 per stream).  An entry is (s << 3) | (len - 1) when every
// window with that prefix decodes to symbol s of length 1..8, and kEscape
// (0xFF) otherwise: a symbol base strictly inside the prefix's range, a
// code longer than 8 bits or of length 0, or symbol 31 of length 8, the one
// code that would read as kEscape.  Escaped windows take a binary search
// over the bases.  Codes of calculate_cdf's rule on chunks of up to 256
// tokens are at most 8 bits long and their bases are multiples of 256, so
// their tables hold no escapes.
//
// Layout: entry e of the lane's stream is byte (e / 4) * 256 + lane * 4 +
// e % 4 of the block's 16 KiB table, so a lane's four consecutive entries are
// one dword (the build scans dwords) and the 64 lanes' lookups hit 64
// distinct dwords; the byte offset is ((e << 6) | e) & 0x3F03 plus lane * 4.
//
// Build (no data-dependent loops): clear() zeroes the table; mark(), for
// every symbol s >= 1 with a base b below 0x10000, writes its entry at prefix
// ceil(b / 256), where it becomes the decoded symbol, and kEscape at prefix
// floor(b / 256) when b is not a multiple of 256; symbols are taken in
// increasing order, so a later write at the same prefix wins, which is the
// larger symbol, as rule L6 wants; symbol 0, which also owns the windows
// below the first base, is written at prefix 0.  scan() then carries each
// written entry forward over the unwritten (zero) prefixes after it.
// Entries grow with s, and s grows with the prefix, so that is a running
// maximum.  Once an escape has been written, the running maximum turns every
// later entry into an escape as well; those take the binary search, so each
// entry is either exact or an escape.
struct ByteTables {
  static constexpr int kBytes = 256 * kLanes;
  static constexpr uint32_t kEscape = 0xFFu;
  static constexpr int kMaxBins = 32;

  uint8_t *tab;      // block table + lane * 4
  uint32_t lane_at;  // LDS address of the lane's column (table address + lane * 4)
  StagedRow row;
  int nb;
  int top;       // largest power of two below nb (1 if nb <= 2)
  bool escapes;  // some scanned entry is kEscape

  // `lds_at` is the LDS address of `lds` (a multiple of kBytes).
  __device__ __forceinline__ void bind(uint8_t *lds, int lane, uint32_t lds_at = 0) {
    tab = lds + lane * 4;
    lane_at = lds_at + static_cast<uint32_t>(lane) * 4u;
  }

  __device__ __forceinline__ uint8_t *entry(uint32_t e) const {
    return tab + (e >> 2) * (kLanes * 4) + (e & 3u);
  }

  __device__ __forceinline__ void clear() {
    uint32_t *t32 = reinterpret_cast<uint32_t *>(tab);
    for (int d = 0; d < 64; ++d) t32[d * kLanes] = 0;
  }

  // Writes the entries of the cleared table.  The row is read into
  // registers (kMaxBins entries whatever nb is: entries past the row are
  // garbage and lie past the wrap).  Bases are taken in symbol order with a
  // sticky flag: from the wrap on (the first symbol whose base is below the
  // one before it, or nb), every base is 0x10000, which writes nothing.
  // Writes that fall outside the table go to `dummy`, a byte of the
  // caller's, so the loops have no branches.  When no row of the wave has a
  // base off a multiple of 256 (calculate_cdf's rows; checked for nb ==
  // kMaxBins, where every loaded entry belongs to the row), no base writes
  // an escape, and the loop without those writes is taken; its writes past
  // the table (base 0x10000: entry 256) land in the 256 bytes after the
  // table, which the caller keeps as scratch while the table is built.
  __device__ __forceinline__ void mark(uint8_t *dummy) {
    uint32_t rw[kMaxBins], eff[kMaxBins];
#pragma unroll
    for (int s = 0; s < kMaxBins; ++s) rw[s] = static_cast<uint16_t>(row.r[s]);
    bool wrapped = false;
    uint32_t prev = rw[0] & 0xFFF0u;
    eff[0] = prev;
#pragma unroll
    for (int s = 1; s < kMaxBins; ++s) {
      const uint32_t v = rw[s] & 0xFFF0u;
      wrapped = wrapped || v < prev || s >= nb;
      eff[s] = wrapped ? 0x10000u : v;
      prev = v;
    }
    bool aligned = false;
    if (nb == kMaxBins) {
      uint32_t acc = 0;
#pragma unroll
      for (int s = 0; s < kMaxBins; ++s) acc |= rw[s];
      aligned = !wave_any((acc & 0xF0u) != 0);
    }
    if (aligned)
      mark_rows<true>(rw, eff, dummy);
    else
      mark_rows<false>(rw, eff, dummy);
  }

  template <bool kAligned>
  __device__ __forceinline__ void mark_rows(const uint32_t (&rw)[kMaxBins], const uint32_t (&eff)[kMaxBins],
                                            uint8_t *dummy) {
#pragma unroll
    for (int s = 0; s < kMaxBins; ++s) {
      const uint32_t base = eff[s];
      const uint32_t next = s + 1 < kMaxBins ? eff[s + 1 < kMaxBins ? s + 1 : 0] : 0x10000u;
      const uint32_t nib = rw[s] & 0xFu;
      // 16 - floor(log2 w); w = 0 gives 16, an escape.
      const uint32_t wl = static_cast<uint32_t>(__builtin_clz((next - base) | 1u)) - 15u;
      const uint32_t len = nib != 0 ? nib : wl;
      const uint32_t code = len - 1u < 8u ? ((static_cast<uint32_t>(s) << 3) | (len - 1u)) : kEscape;
      if (s == 0) {  // owns the windows below every later base: prefix 0
        *entry(0) = static_cast<uint8_t>(code);
      } else if (kAligned) {
        // base is a multiple of 256 (entry base / 256), or 0x10000 from
        // the wrap on (entry 256, past the table).
        *(tab + ((base >> 2) & 0x7F00u) + ((base >> 8) & 3u)) = static_cast<uint8_t>(code);
      } else {
        // base is 0x10000 from the wrap on: no escape (its low byte is 0)
        // and no entry (it is not below 0xFF01).
        *((base & 0xFFu) ? entry(base >> 8) : dummy) = static_cast<uint8_t>(kEscape);
        *(base < 0xFF01u ? entry((base + 0xFFu) >> 8) : dummy) = static_cast<uint8_t>(code);
      }
    }
  }

  // Running maximum over dwords [d0, d1) starting from `carry` (the entry
  // before dword d0, 0 for d0 = 0).  One dword takes four byte maxima, each
  // written into its byte of the dword in place (SDWA with the other bytes
  // preserved), byte 0 against the previous dword's byte 3.
  __device__ __forceinline__ static uint32_t scan_dword(uint32_t w, uint32_t prev) {
#ifdef __HIP_DEVICE_COMPILE__
    asm("v_max_u32_sdwa %0, %1, %0 dst_sel:BYTE_0 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3 src1_sel:BYTE_0"
        : "+v"(w) : "v"(prev));
    asm("v_max_u32_sdwa %0, %0, %0 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0 src1_sel:BYTE_1"
        : "+v"(w));
    asm("v_max_u32_sdwa %0, %0, %0 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1 src1_sel:BYTE_2"
        : "+v"(w));
    asm("v_max_u32_sdwa %0, %0, %0 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_2 src1_sel:BYTE_3"
        : "+v"(w));
    return w;
#else
    uint32_t carry = prev >> 24, o = 0;
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = (w >> (8 * i)) & 0xFFu;
      carry = carry > v ? carry : v;
      o |= carry << (8 * i);
    }
    return o;
#endif
  }
  __device__ __forceinline__ void scan(int d0, int d1, uint32_t carry) {
    uint32_t *t32 = reinterpret_cast<uint32_t *>(tab);
    uint32_t prev = carry << 24;
    for (int d = d0; d < d1; d += 8) {
      uint32_t w[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = t32[(d + k) * kLanes];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        prev = scan_dword(w[k], prev);
        t32[(d + k) * kLanes] = prev;
      }
    }
    escapes = (prev >> 24) == kEscape;
  }

  // top and row.wrap, which only the binary search reads.
  __device__ __forceinline__ void finish() {
    top = 1;
    while (top * 2 < nb) top *= 2;
    int wrap = nb;
    uint32_t top_base = static_cast<uint16_t>(row.r[0]) & 0xFFF0u;
    for (int s = 1; s < kMaxBins; ++s) {
      const uint32_t v = static_cast<uint16_t>(row.r[s]) & 0xFFF0u;
      wrap = min(wrap, v < top_base ? s : kMaxBins);
      top_base = max(top_base, v);
    }
    row.wrap = wrap;
  }

  // Builds the table after clear().
  __device__ __forceinline__ void build(uint8_t *dummy) {
    mark(dummy);
    scan(0, 64, 0);
  }

  // One symbol at the cursor for a table without escapes (one LDS read, no
  // branches); returns the entry: symbol e >> 3, length (e & 7) + 1.
  __device__ __forceinline__ uint32_t step(BitCursor &cur) const {
    const uint32_t e = cur.peek32() >> 24;
    const uint32_t x = tab[((e << 6) | e) & 0x3F03u];
    cur.advance(static_cast<int>(x & 7u) + 1);
    return x;
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

// Cursor for byte tables without escapes over a sealed lane region
// (LaneWindows), four codes per group.  The chain from one code to the next
// is the table read and three VALU instructions: the entry's length field
// and the next code's table dword, addressed from the current code's window
// bits (the next window is this one shifted by length bits, so its top six
// bits are bits 62 - l .. 57 - l of this one, l = length - 1, which
// y = h >> 17 holds at 13 - l .. 8 - l: ((y << l) & 0x3F00) | lane_at).
// The rest, each code's window bits h (from which y and the byte's shift sh
// in its table dword) and the windows, is kept off that chain: h is taken
// from a 64-bit window v at offset o, and a group reads the window at its
// second code's stream bit, vn, and switches to it at its fourth code, so
// no window is refilled by a data-dependent shift.  v serves the codes from
// the fourth of the previous group to the third of this one (offsets up to
// 40); the next code's address needs 6 + l bits past the current code, so
// every bit read lies within the window's 64.  Scheduling barriers keep
// each chain (the wait for the entry, three instructions, the next read)
// free of other instructions, which are placed while a read is in flight.
struct GroupCursor {
  LaneWindows lw;
  uint32_t wa;  // LDS address of lw.w (raw region + off / 4)
  uint64_t v;   // window at stream bit qm + 1
  uint32_t qm;
  uint32_t o;   // offset in v of the current code
  uint32_t y;   // the current code's window bits 31 .. 17 (h >> 17)
  uint32_t sh;  // 8 x the current code's byte in its table dword
  uint32_t d;   // the current code's table dword (its read in flight)
  // The next window (read during a group): its stream bit less one, the
  // offset in v it starts at, its raw dwords, then its stream dwords, then
  // the window.
  uint32_t qn1, o1, r0, r1, r2, r3, a, b, c;
  uint64_t vn;

  static __device__ __forceinline__ void fence() {
#ifdef __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_sched_barrier(0);
#endif
  }

  __device__ __forceinline__ void place(uint64_t nv) {
    const uint32_t h = static_cast<uint32_t>((nv << o) >> 32);
    y = h >> 17;
    sh = (h >> 21) & 0x18u;
  }

  // region_at: the LDS address of region.
  __device__ __forceinline__ void start(const ByteTables &tb, const uint32_t *region, uint32_t region_at,
                                        uint32_t off, uint32_t len) {
    lw.start(region, off, len);
    wa = region_at + 4u * static_cast<uint32_t>(lw.w - region);
    qm = 0xFFFFFFFFu;
    v = lw.at(0);
    o = 0;
    place(v);
    d = lds_dword(((static_cast<uint32_t>(v >> 32) >> 18) & 0x3F00u) | tb.lane_at);
  }

  // The chain: the current code's length from its entry and the next code's
  // table read.  Returns the length - 1; e is the entry in the low byte.
  __device__ __forceinline__ uint32_t advance(const ByteTables &tb, uint32_t &e) {
    fence();
    const uint32_t dc = d;
    const uint32_t l = (dc >> sh) & 7u;
    d = lds_dword(((y << l) & 0x3F00u) | tb.lane_at);
    fence();
    e = dc >> sh;
    return l;
  }

  // The four codes of a group, each returning its entry; a caller may place
  // its own work between them (it lands under a table read).
  __device__ __forceinline__ uint32_t step0(const ByteTables &tb) {
    uint32_t e;
    const uint32_t l = advance(tb, e);
    o += l + 1u;
    place(v);
    // The next window's raw dwords, from stream bit qn1 + 1 (LaneWindows::at
    // with the bit less one: dwords j = qn1 / 32 on, shifted by
    // 31 - qn1 % 32, one alignbit per word): loads issued here.
    o1 = o;
    qn1 = qm + o1;
    const uint32_t j = (qn1 >> 5) < lw.zl ? (qn1 >> 5) : lw.zl;
    const uint32_t at = wa + (j << 2);
    r0 = lds_dword(at);
    r1 = lds_dword(at + 4u);
    r2 = lds_dword(at + 8u);
    r3 = lds_dword(at + 12u);
    return e;
  }
  __device__ __forceinline__ uint32_t step1(const ByteTables &tb) {
    uint32_t e;
    const uint32_t l = advance(tb, e);
    o += l + 1u;
    place(v);
    return e;
  }
  __device__ __forceinline__ uint32_t step2(const ByteTables &tb) {
    uint32_t e;
    const uint32_t l = advance(tb, e);
    a = byte_perm(r1, r0, lw.sel);
    b = byte_perm(r2, r1, lw.sel);
    c = byte_perm(r3, r2, lw.sel);
    const uint32_t sr = ~qn1;
    vn = (static_cast<uint64_t>(align_bits(a, b, sr)) << 32) | align_bits(b, c, sr);
    o += l + 1u - o1;
    place(vn);
    return e;
  }
  __device__ __forceinline__ uint32_t step3(const ByteTables &tb) {
    uint32_t e;
    const uint32_t l = advance(tb, e);
    o += l + 1u;
    place(vn);
    v = vn;
    qm = qn1;
    return e;
  }
  __device__ __forceinline__ void group(const ByteTables &tb, uint32_t &e0, uint32_t &e1, uint32_t &e2,
                                        uint32_t &e3) {
    e0 = step0(tb);
    e1 = step1(tb);
    e2 = step2(tb);
    e3 = step3(tb);
  }

  // One code read from a fresh window (the tail after the groups); returns
  // its symbol.
  __device__ __forceinline__ uint32_t single(const ByteTables &tb) {
    const uint32_t hh = static_cast<uint32_t>(lw.at(qm + 1u + o) >> 32);
    const uint32_t s8 = (hh >> 21) & 0x18u;
    const uint32_t e = lds_dword(((hh >> 18) & 0x3F00u) | tb.lane_at) >> s8;
    o += (e & 7u) + 1u;
    return (e >> 3) & 31u;
  }
};

}  // namespace cgdec
}  // namespace lmc
