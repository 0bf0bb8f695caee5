/*
 * CPU oracle for the CacheGen codec ops.  TEST INFRASTRUCTURE ONLY: built by
 * oracle/build_oracle.py into oracle/_build/liboracle_cachegen.so and called
 * from oracle/cachegen.py by the tests, smoke() and bench.py's cpu_baseline;
 * the product (liblmcache_amd.so) never links or loads it.
 *
 * The reference's device kernels are absent (third_party/kvcache-ops is an
 * empty submodule), so the codec is pinned by what the reference's tests and
 * docs fix (tests/v1/test_cachegen_kernels.py; docs/cachegen/Cachegen.md:
 * 30-39):
 *   - symbol s owns the CDF interval [cdf[s], cdf[s+1]) of the 16-bit range;
 *     the intervals are power-of-two aligned, so s is always coded as the same
 *     bit string: the top l_s bits of cdf[s], emitted MSB first, the stream
 *     zero-padded to a byte (test_cachegen_kernels.py:31-161);
 *   - cdf entries are int16 bit patterns of 16-bit values, the final 0x10000
 *     wrapping to 0 (the tests build them with float -> int16 casts);
 *   - CDF entries may carry the code length in their low bits
 *     (cdf[b] = b * 2^(16-n) | n, test_cachegen_kernels.py:205-214);
 *   - decode reads a concatenation of the streams in (layer, channel) order
 *     with inclusive prefix-summed byte lengths (:194-221).
 *
 * Rules this library fixes where the reference leaves them open (the exact
 * calculate_cdf values are "parity unpinned": only the absent kernel defines
 * them):
 *   L1  low 4 bits of an entry = code length l_s; interval bases are the
 *       entry with those bits cleared (multiples of 16); calculate_cdf emits
 *       lengths 1..12 for present symbols and 0 for absent ones.
 *   L2  bases never decrease: an entry smaller than its predecessor stands
 *       for 0x10000 (as does every later entry); entry n_bins is the end of
 *       the range, 0x10000, whatever is stored there.
 *   L3  l_s = low bits of cdf[s] when non-zero, else 16 - floor(log2 w_s)
 *       with w_s = base(s+1) - base(s); a symbol with w_s == 0 is absent and
 *       codes to nothing (as does a single symbol owning all of 0x10000).
 *   L4  calculate_cdf: counts c_s over the T tokens (symbols >= n_bins are
 *       not counted), n = sum of counts, m present symbols (c_s > 0).
 *       Lengths: one present symbol takes length 1.  For m >= 2 they are
 *       the leaf depths of the Garsia-Wachs combination tree over the
 *       present symbols' counts in symbol order, which are the lengths of an
 *       optimal alphabetic (order-preserving) prefix code (oc_gw_lengths
 *       states the tie rules), unless the longest exceeds Lmax = 8 when
 *       n <= 256, else 12; those rows take the Shannon rule instead:
 *       l_s = clamp(ceil(log2(n / c_s)), 1, 12), and while the Kraft sum
 *       exceeds 1, lengthen the present symbol with l < 12 and the smallest
 *       count (ties: the highest symbol).  Then assign intervals in symbol
 *       order from 0, each at the running position, halving a symbol's width
 *       (lengthening its code) until the position is a multiple of it (never
 *       needed for the Garsia-Wachs lengths); absent symbols take the base
 *       of the next present symbol (or the end of the used range).
 *   L5  encode writes at most `chunk` bytes per stream, leaves the rest of
 *       the row untouched and reports the full length in bytes; symbols
 *       >= n_bins code to nothing.
 *   L6  decode: symbol = largest s < n_bins with base(s) <= the next 16
 *       stream bits (bits past the stream's end read as 0); l_s bits are
 *       consumed.
 */
#include <stdint.h>
#include <string.h>

#define OC_PREC 16
#define OC_MAX_LEN 12
#define OC_LEN_MASK 0xF
#define OC_MAX_BINS 256

/* L1-L3: unwrapped bases u[0..nb] (u[nb] = 0x10000) and code lengths. */
static void oc_unpack(const int16_t *row, int nb, uint32_t *u, int *len) {
  uint32_t prev = 0;
  int wrapped = 0;
  for (int s = 0; s < nb; ++s) {
    uint32_t v = (uint32_t)(uint16_t)row[s] & 0xFFF0u;
    if (wrapped || (s > 0 && v < prev)) {
      wrapped = 1;
      v = 0x10000u;
    }
    u[s] = v;
    prev = v;
  }
  u[nb] = 0x10000u;
  for (int s = 0; s < nb; ++s) {
    int l = (uint16_t)row[s] & OC_LEN_MASK;
    if (l == 0) {
      uint32_t w = u[s + 1] - u[s];
      if (w != 0) {
        int k = 31 - __builtin_clz(w); /* floor(log2 w) */
        l = OC_PREC - k;
      }
    }
    len[s] = l;
  }
}

/* L4, optimal lengths: the leaf depths of the Garsia-Wachs combination tree
 * over w[0..m-1] (m >= 2), written to depth[]; returns the largest.  The
 * algorithm is A. M. Garsia and M. L. Wachs, "A new algorithm for minimum
 * cost binary trees", SIAM J. Comput. 6(4), 1977 (also Knuth, TAOCP vol. 3,
 * 6.2.2): while more than one weight is left, combine the first pair
 * (x, y) of a triple x, y, z of consecutive weights with x <= z, taken from
 * the left (the last pair when no triple qualifies, as if an infinite
 * weight followed the list); remove both and re-insert x + y right after
 * the nearest weight to the left of x's position that is >= x + y (at the
 * front when there is none).  The tree's leaf depths are those of an
 * optimal alphabetic tree over the weights in their order. */
static int oc_gw_lengths(const uint64_t *w, int m, int *depth) {
  uint64_t wt[2 * OC_MAX_BINS];
  int parent[2 * OC_MAX_BINS];
  int list[OC_MAX_BINS];
  int len = m, next = m;
  for (int i = 0; i < m; ++i) {
    wt[i] = w[i];
    list[i] = i;
  }
  while (len > 1) {
    int k = len - 2;
    for (int i = 0; i + 2 < len; ++i) {
#ifdef OC_PLANT_GW_STRICT
      /* planted mistake (tests only): the first triple with x < z */
      if (wt[list[i]] < wt[list[i + 2]]) {
#else
      if (wt[list[i]] <= wt[list[i + 2]]) {
#endif
        k = i;
        break;
      }
    }
    const int a = list[k], b = list[k + 1];
    const uint64_t sum = wt[a] + wt[b];
    const int node = next++;
    wt[node] = sum;
    parent[a] = parent[b] = node;
    for (int i = k; i + 2 < len; ++i) list[i] = list[i + 2];
    len -= 2;
    int p = 0;
#ifdef OC_PLANT_GW_IN_PLACE
    /* planted mistake (tests only): the combined weight stays at x's place */
    p = k;
#else
    for (int j = k - 1; j >= 0; --j)
      if (wt[list[j]] >= sum) {
#ifdef OC_PLANT_GW_BEFORE
        /* planted mistake (tests only): re-inserted before that weight */
        p = j;
#else
        p = j + 1;
#endif
        break;
      }
#endif
    for (int i = len; i > p; --i) list[i] = list[i - 1];
    list[p] = node;
    ++len;
  }
  /* Parents are created after their children: depths from the root down. */
  int d[2 * OC_MAX_BINS];
  d[next - 1] = 0;
  for (int id = next - 2; id >= 0; --id) d[id] = d[parent[id]] + 1;
  int longest = 0;
  for (int i = 0; i < m; ++i) {
    depth[i] = d[i];
    if (d[i] > longest) longest = d[i];
  }
  return longest;
}

/* L4 for one stream: counts -> int16 row of nb + 1 entries. */
static void oc_cdf_row(const uint32_t *count, int nb, int16_t *row) {
  uint64_t n = 0;
  for (int s = 0; s < nb; ++s) n += count[s];
  int len[OC_MAX_BINS];
  uint32_t base[OC_MAX_BINS];
  uint64_t w[OC_MAX_BINS];
  int sym[OC_MAX_BINS], depth[OC_MAX_BINS];
  int m = 0;
  for (int s = 0; s < nb; ++s) {
    len[s] = 0;
    if (count[s]) {
      w[m] = count[s];
      sym[m++] = s;
    }
  }
#ifdef OC_PLANT_LMAX9
  /* planted mistake (tests only): a 9-bit limit for short chunks */
  const int lmax = n <= 256 ? 9 : OC_MAX_LEN;
#else
  const int lmax = n <= 256 ? 8 : OC_MAX_LEN;
#endif
  int optimal = 0;
  if (m == 1) {
    len[sym[0]] = 1;
    optimal = 1;
  } else if (m >= 2 && oc_gw_lengths(w, m, depth) <= lmax) {
    for (int i = 0; i < m; ++i) len[sym[i]] = depth[i];
    optimal = 1;
  }
  uint64_t kraft = 0; /* in units of 2^-16 */
  for (int s = 0; s < nb && !optimal; ++s) {
    if (count[s] == 0) {
      len[s] = 0;
      continue;
    }
    int l = 0;
    while (((uint64_t)count[s] << l) < n) ++l; /* ceil(log2(n / c)) */
#ifdef OC_PLANT_FLOOR_LEN
    /* planted mistake (tests only): floor(log2(n / c)) */
    if (((uint64_t)count[s] << l) > n) --l;
#endif
    if (l < 1) l = 1;
    if (l > OC_MAX_LEN) l = OC_MAX_LEN;
    len[s] = l;
    kraft += (uint64_t)1 << (OC_PREC - l);
  }
  while (!optimal && kraft > ((uint64_t)1 << OC_PREC)) {
    int pick = -1;
    for (int s = 0; s < nb; ++s) {
      if (len[s] == 0 || len[s] >= OC_MAX_LEN) continue;
#ifdef OC_PLANT_TIE_LOW
      /* planted mistake (tests only): ties pick the lowest symbol */
      if (pick < 0 || count[s] < count[pick]) pick = s;
#else
      if (pick < 0 || count[s] <= count[pick]) pick = s;
#endif
    }
    if (pick < 0) break; /* unreachable: nb * 2^-12 <= 1 for nb <= 4096 */
    kraft -= (uint64_t)1 << (OC_PREC - len[pick] - 1);
    ++len[pick];
  }
  uint32_t pos = 0;
  for (int s = 0; s < nb; ++s) {
    if (len[s] == 0) continue;
    uint32_t wd = 1u << (OC_PREC - len[s]);
#ifdef OC_PLANT_ROUND_UP
    /* planted mistake (tests only): the base is rounded up to the width and
     * the length kept, instead of the width halved */
    pos = (pos + wd - 1) & ~(wd - 1);
#else
    while (pos & (wd - 1)) {
      wd >>= 1;
      ++len[s];
    }
#endif
    base[s] = pos;
    pos += wd;
  }
  uint32_t next = pos;
  for (int s = nb - 1; s >= 0; --s) {
    if (len[s] == 0)
      base[s] = next;
    else
      next = base[s];
  }
  for (int s = 0; s < nb; ++s)
    row[s] = (int16_t)(uint16_t)((base[s] | (uint32_t)len[s]) & 0xFFFFu);
  row[nb] = 0; /* 0x10000 */
}

/* input [L, T, C] u8; output [L, C, nb + 1] int16. */
void oc_calculate_cdf(const uint8_t *in, int L, int T, int C, int nb,
                      int16_t *out) {
  uint32_t count[OC_MAX_BINS];
  for (int l = 0; l < L; ++l)
    for (int c = 0; c < C; ++c) {
      memset(count, 0, sizeof(count));
      for (int t = 0; t < T; ++t) {
        uint8_t s = in[((int64_t)l * T + t) * C + c];
        if (s < nb) ++count[s];
      }
      oc_cdf_row(count, nb, out + ((int64_t)l * C + c) * (nb + 1));
    }
}

/* Appends `nbits` bits of `code` (MSB first) to a stream of `cap` bytes. */
static void oc_put_bits(uint8_t *dst, int64_t cap, uint64_t *bitpos,
                        uint32_t code, int nbits) {
  for (int i = nbits - 1; i >= 0; --i) {
    int bit = (code >> i) & 1;
    int64_t byte = (int64_t)(*bitpos >> 3);
    if (byte < cap) {
      if ((*bitpos & 7) == 0) dst[byte] = 0;
#ifdef OC_PLANT_LSB_FIRST
      /* Deliberately wrong bit order, compiled only by the test that checks
       * the reference's encode KATs catch it. */
      if (bit) dst[byte] |= (uint8_t)(1u << (*bitpos & 7));
#else
      if (bit) dst[byte] |= (uint8_t)(0x80u >> (*bitpos & 7));
#endif
    }
    ++*bitpos;
  }
}

/* cdf [L, C, nb + 1]; in [L, T, C]; out [L, C, chunk]; lens [L, C]. */
void oc_encode(const int16_t *cdf, const uint8_t *in, int L, int T, int C,
               int nb, uint8_t *out, int chunk, int32_t *lens) {
  uint32_t u[OC_MAX_BINS + 1];
  int len[OC_MAX_BINS];
  for (int l = 0; l < L; ++l)
    for (int c = 0; c < C; ++c) {
      oc_unpack(cdf + ((int64_t)l * C + c) * (nb + 1), nb, u, len);
      uint8_t *dst = out + ((int64_t)l * C + c) * chunk;
      uint64_t bitpos = 0;
      for (int t = 0; t < T; ++t) {
        int s = in[((int64_t)l * T + t) * C + c];
        if (s >= nb || len[s] == 0) continue;
        uint32_t code = u[s] >> (OC_PREC - len[s]);
        oc_put_bits(dst, chunk, &bitpos, code, len[s]);
      }
      lens[(int64_t)l * C + c] = (int32_t)((bitpos + 7) >> 3);
    }
}

/* Bit `pos` (MSB-first) of a stream of `n` bytes; 0 past its end. */
static int oc_get_bit(const uint8_t *src, int64_t n, uint64_t pos) {
  int64_t byte = (int64_t)(pos >> 3);
  if (byte >= n) return 0;
  return (src[byte] >> (7 - (pos & 7))) & 1;
}

/* cdf [L, C, nb + 1]; bytes: concatenated streams; prefix [L, C] inclusive
 * prefix sums of stream lengths; out [L, T, C]. */
void oc_decode(const int16_t *cdf, const uint8_t *bytes, int64_t nbytes,
               const int32_t *prefix, int L, int T, int C, int nb,
               uint8_t *out) {
  uint32_t u[OC_MAX_BINS + 1];
  int len[OC_MAX_BINS];
  for (int l = 0; l < L; ++l)
    for (int c = 0; c < C; ++c) {
      const int64_t i = (int64_t)l * C + c;
      int64_t start = i == 0 ? 0 : prefix[i - 1];
      int64_t end = prefix[i];
      if (start > nbytes) start = nbytes;
      if (end > nbytes) end = nbytes;
      if (end < start) end = start;
      oc_unpack(cdf + i * (nb + 1), nb, u, len);
      const uint8_t *src = bytes + start;
      const int64_t n = end - start;
      uint64_t pos = 0;
      for (int t = 0; t < T; ++t) {
        uint32_t v = 0;
        for (int b = 0; b < OC_PREC; ++b) v = (v << 1) | oc_get_bit(src, n, pos + b);
        int s = nb - 1;
        while (s > 0 && u[s] > v) --s;
        out[((int64_t)l * T + t) * C + c] = (uint8_t)s;
        pos += (uint64_t)len[s];
      }
    }
}
