// Host build of the CacheGen decoder's table and bit-cursor logic
// (lmcache-ascend_amd/csrc/cachegen_decode.h), checked against the CPU
// oracle's decoder (oracle/cachegen.c, oc_decode) on random CDF rows and
// random byte streams.  Built and run by tests/test_decode_tables_cpu.py.
//
// For every row: the table is built as the decode kernel builds it (clear,
// mark, scan, plus finish for the binary search), and several streams are
// decoded with each cursor.  The shared-window cursor: through
// ByteTables::step when the table holds no escape entry (the kernel's
// branch-free loop) and through ByteTables::lookup otherwise; each stream
// sits in a window of big-endian dwords between other streams' bytes, at a
// random byte offset, so reads past its end meet foreign bytes that must
// read as zero.  The lane-region cursors: the lane cursor on every table,
// and the group cursor (GroupCursor) on tables without escapes, over the
// stream's own sealed region, sized exactly as in the kernel (built with
// AddressSanitizer, a read past it fails the run).
//
// Usage: decode_tables_check <rows> <seed>; prints "ok ..." or the first
// mismatch and exits 1.
#define __device__
#define __forceinline__ inline
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>
using std::max;
using std::min;
#include "../lmcache-ascend_amd/csrc/cachegen_decode.h"

extern "C" void oc_decode(const int16_t *cdf, const uint8_t *bytes, int64_t nbytes,
                          const int32_t *prefix, int L, int T, int C, int nb, uint8_t *out);

using lmc::cgdec::BitCursor;
using lmc::cgdec::ByteTables;

namespace {

// A CDF row of one of several kinds: calculate_cdf-like (aligned power-of-
// two intervals of lengths 1..8 with gaps and absent symbols; kind 3 starts
// with codes that end exactly at prefix 127, then a gap), sorted bases in
// steps of 16 with random length nibbles, fully random entries, and any of
// these with a decreasing entry (a wrap).
void make_row(std::mt19937_64 &rng, int nb, int kind, int16_t *row) {
  if (kind == 0 || kind == 3) {
    uint32_t pos = 0;
    int s0 = 0;
    if (kind == 3) {
      // Codes of lengths 2, 3, .., 8, 8 fill prefixes 0 .. 127 exactly, the
      // last one a single prefix at 127, and a gap follows: the prefixes
      // after it take prefix 127's entry across the middle of the table
      // (the table's running maximum carries it over a dword boundary).
      for (int l = 2; l <= 9 && s0 < nb; ++l, ++s0) {
        const int len = l < 9 ? l : 8;
        row[s0] = static_cast<int16_t>(static_cast<uint16_t>(pos | static_cast<uint32_t>(len)));
        pos += 1u << (16 - len);
      }
      pos += 256u << (rng() % 6);
    }
    for (int s = s0; s < nb; ++s) {
      if (rng() % 5 == 0) {  // absent: the next present base, length 0
        row[s] = static_cast<int16_t>(static_cast<uint16_t>(pos & 0xFFF0u));
        continue;
      }
      const int l = 1 + static_cast<int>(rng() % 8);
      const uint32_t w = 1u << (16 - l);
      pos = (pos + w - 1) & ~(w - 1);
      if (pos + w > 0x10000u) {
        row[s] = 0;  // base 0x10000 wraps to 0
        pos = 0x10000u;
        continue;
      }
      row[s] = static_cast<int16_t>(static_cast<uint16_t>(pos | static_cast<uint32_t>(l)));
      pos += w;
      if (rng() % 6 == 0) pos = std::min(0x10000u, pos + (256u << (rng() % 6)));
      // Sometimes a gap right after a code ending at 0x8000.
      if (pos == 0x8000u && rng() % 2) pos += 256u << (rng() % 5);
    }
  } else if (kind == 1) {
    std::vector<uint32_t> b(nb);
    for (auto &x : b) x = static_cast<uint32_t>(rng() % 4096) * 16;
    std::sort(b.begin(), b.end());
    for (int s = 0; s < nb; ++s) {
      const uint32_t nib = rng() % 2 ? 0u : static_cast<uint32_t>(rng() % 16);
      row[s] = static_cast<int16_t>(static_cast<uint16_t>(b[s] | nib));
    }
  } else {
    for (int s = 0; s < nb; ++s) row[s] = static_cast<int16_t>(rng() & 0xFFFF);
  }
  if (nb > 2 && rng() % 4 == 0) row[1 + rng() % (nb - 1)] = 0;
  row[nb] = static_cast<int16_t>(rng() & 0xFFFF);  // entry n_bins: ignored by the rules
}

}  // namespace

int main(int argc, char **argv) {
  const int rows = argc > 1 ? atoi(argv[1]) : 2000;
  std::mt19937_64 rng(argc > 2 ? strtoull(argv[2], nullptr, 10) : 1);
  static uint8_t lds[ByteTables::kBytes + 256];  // the table and the 256 scratch bytes after it
  uint8_t dummy = 0;
  long long symbols = 0, fast_rows = 0, escaped_rows = 0;
  for (int it = 0; it < rows; ++it) {
    // Every third row has kMaxBins symbols: with aligned bases (kind 0) it
    // takes mark's loop without escape writes.
    const int nb = it % 3 == 1 ? ByteTables::kMaxBins : 1 + static_cast<int>(rng() % ByteTables::kMaxBins);
    int kind = it % 4 == 3 ? static_cast<int>(rng() % 3) : it % 3;
    if (nb == ByteTables::kMaxBins && kind == 0 && it % 2 == 0) kind = 3;
    // The kernel reads kMaxBins row entries whatever nb is; the row lives in a
    // larger buffer of foreign entries, as in the kernel's staged rows.
    std::vector<int16_t> buf(ByteTables::kMaxBins + 8);
    for (auto &x : buf) x = static_cast<int16_t>(rng() & 0xFFFF);
    make_row(rng, nb, kind, buf.data());
    ByteTables tb;
    memset(lds, 0xA5, sizeof lds);
    lmc::cgdec::host_lds_base() = lds;
    tb.bind(lds, static_cast<int>(rng() % lmc::cgdec::kLanes), 0);
    tb.row.r = buf.data();
    tb.nb = nb;
    tb.clear();
    tb.build(&dummy);
    tb.finish();
    (tb.escapes ? escaped_rows : fast_rows) += 1;
    for (int k = 0; k < 6; ++k) {
      const int T = 1 + static_cast<int>(rng() % 300);
      const uint32_t len = static_cast<uint32_t>(rng() % 160);
      const uint32_t lo = static_cast<uint32_t>(rng() % 16), hi = lo + len;
      std::vector<uint8_t> win_bytes(512);
      for (auto &x : win_bytes) x = static_cast<uint8_t>(rng());
      std::vector<uint32_t> win(win_bytes.size() / 4);
      for (size_t i = 0; i < win.size(); ++i)
        win[i] = static_cast<uint32_t>(win_bytes[4 * i]) << 24 | static_cast<uint32_t>(win_bytes[4 * i + 1]) << 16 |
                 static_cast<uint32_t>(win_bytes[4 * i + 2]) << 8 | win_bytes[4 * i + 3];
      const uint32_t last = 4 * static_cast<uint32_t>(win.size() - 1);
      std::vector<uint8_t> want(T), got(T);
      const int32_t prefix = static_cast<int32_t>(len);
      oc_decode(buf.data(), win_bytes.data() + lo, len, &prefix, 1, T, 1, nb, want.data());
      BitCursor cur;
      cur.start(win.data(), last, 8 * lo, hi);
      for (int t = 0; t < T; ++t) {
        if (!tb.escapes) {
          got[t] = static_cast<uint8_t>(tb.step(cur) >> 3);
        } else {
          int s, l;
          tb.lookup(cur.peek32() >> 16, s, l);
          got[t] = static_cast<uint8_t>(s);
          cur.advance(l);
        }
      }
      for (int t = 0; t < T; ++t)
        if (got[t] != want[t]) {
          printf("MISMATCH row %d (nb %d, kind %d, escapes %d) stream %d token %d: got %d want %d\n", it, nb,
                 kind, tb.escapes ? 1 : 0, k, t, got[t], want[t]);
          return 1;
        }
      // The lane-region path: the stream's 16-byte aligned chunks of the
      // byte buffer (foreign bytes around it) as raw little-endian dwords,
      // plus LaneRegion::kRoom bytes of garbage, sealed past the stream's
      // end.  Every table is decoded with the lane cursor (one code per
      // refill, binary search on escapes), and tables without escapes also
      // with the group cursor, as the kernel does: four codes per group,
      // single codes for the tail.
      {
        const uint32_t a0 = lo & ~15u;
        const uint32_t n_ch = len ? ((hi - 1) / 16 - lo / 16 + 1) : 0;
        std::vector<uint32_t> region(4 * n_ch + lmc::cgdec::LaneRegion::kRoom / 4);
        for (auto &x : region) x = static_cast<uint32_t>(rng());
        for (uint32_t i = 0; i < 16 * n_ch; ++i)
          reinterpret_cast<uint8_t *>(region.data())[i] = win_bytes[a0 + i];
        lmc::cgdec::LaneRegion::seal(region.data(), lo - a0, len);
        lmc::cgdec::LaneCursor lc;
        lc.start(region.data(), lo - a0, len);
        ByteTables ts = tb;
        ts.finish();
        for (int t = 0; t < T; ++t) {
          int s, l;
          ts.lookup(lc.top16(), s, l);
          got[t] = static_cast<uint8_t>(s);
          lc.consume(l);
          lc.refill();
        }
        for (int u = 0; u < T; ++u)
          if (got[u] != want[u]) {
            printf("LANE MISMATCH row %d (nb %d, kind %d, escapes %d) stream %d token %d: got %d want %d\n", it,
                   nb, kind, tb.escapes ? 1 : 0, k, u, got[u], want[u]);
            return 1;
          }
        if (!tb.escapes) {
          // The table, its 256 scratch bytes and the region in one buffer
          // addressed from 0 (LDS addresses), the region at its end, so a
          // read past the region fails the run.
          const size_t rb = region.size() * 4;
          std::vector<uint8_t> mem(ByteTables::kBytes + 256 + rb);
          memcpy(mem.data(), lds, ByteTables::kBytes + 256);
          memcpy(mem.data() + ByteTables::kBytes + 256, region.data(), rb);
          lmc::cgdec::host_lds_base() = mem.data();
          ByteTables tg = tb;
          tg.bind(mem.data(), static_cast<int>(tb.lane_at / 4), 0);
          lmc::cgdec::GroupCursor gc;
          gc.start(tg, reinterpret_cast<const uint32_t *>(mem.data() + ByteTables::kBytes + 256),
                   ByteTables::kBytes + 256, lo - a0, len);
          int t = 0;
          for (; t + 4 <= T; t += 4) {
            uint32_t e[4];
            gc.group(tg, e[0], e[1], e[2], e[3]);
            for (int j = 0; j < 4; ++j) got[t + j] = static_cast<uint8_t>((e[j] >> 3) & 31u);
          }
          for (; t < T; ++t) got[t] = static_cast<uint8_t>(gc.single(tg));
          lmc::cgdec::host_lds_base() = lds;
          for (int u = 0; u < T; ++u)
            if (got[u] != want[u]) {
              printf("GROUP MISMATCH row %d (nb %d, kind %d) stream %d token %d: got %d want %d\n", it, nb, kind, k,
                     u, got[u], want[u]);
              return 1;
            }
        }
      }
      symbols += T;
    }
  }
  printf("ok rows=%d (without escapes %lld, with %lld) symbols=%lld\n", rows, fast_rows, escaped_rows, symbols);
  return 0;
}
