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
//   L4  calculate_cdf: Shannon lengths ceil(log2(n / count)) clamped to
//       [1, 12], Kraft-repaired by lengthening the rarest present symbol,
//       intervals assigned in symbol order with widths halved until aligned,
//       absent symbols at the next present base;
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
#include "common.h"

namespace lmc {

namespace {

constexpr int kLanes = 256;
constexpr int kMaxBins = 64;
constexpr int kPrec = 16;
constexpr int kMaxLen = 12;

// Unpacks one stream's CDF row into LDS column `col` as
// (base << 8) | length per symbol (rules L1-L3).  `cur` is the unwrapped
// base of symbol s, `next` that of s + 1; once a base has wrapped to
// 0x10000, every later one is 0x10000 as well.
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
    col[s * kLanes] = (cur << 8) | static_cast<uint32_t>(len);
    cur = next;
    cur_raw = next_raw;
  }
}

__global__ void __launch_bounds__(kLanes)
    cdf_kernel(const uint8_t *__restrict__ in, int T, int C, int nb,
               int16_t *__restrict__ out, int tiles) {
  extern __shared__ uint32_t lds[];
  const int l = blockIdx.x / tiles;
  const int c = (blockIdx.x % tiles) * kLanes + threadIdx.x;
  if (c >= C) return;
  uint32_t *col = lds + threadIdx.x;
  for (int s = 0; s < nb; ++s) col[s * kLanes] = 0;
  const uint8_t *p = in + static_cast<int64_t>(l) * T * C + c;
#pragma unroll 8
  for (int t = 0; t < T; ++t) {
    const uint32_t s = p[static_cast<int64_t>(t) * C];
    if (s < static_cast<uint32_t>(nb)) col[s * kLanes] += 1u;
  }
  // Code lengths (rule L4); entries become (count << 5) | length.
  uint32_t n = 0;
  for (int s = 0; s < nb; ++s) n += col[s * kLanes];
  uint32_t kraft = 0;  // units of 2^-16; at most 64 * 2^15
  for (int s = 0; s < nb; ++s) {
    const uint32_t cnt = col[s * kLanes];
    uint32_t len = 0;
    if (cnt) {
      while ((static_cast<uint64_t>(cnt) << len) < n) ++len;
      len = len < 1 ? 1 : (len > kMaxLen ? kMaxLen : len);
      kraft += 1u << (kPrec - len);
    }
    col[s * kLanes] = (cnt << 5) | len;
  }
  while (kraft > (1u << kPrec)) {
    int pick = -1;
    uint32_t best = 0;
    for (int s = 0; s < nb; ++s) {
      const uint32_t e = col[s * kLanes];
      const uint32_t len = e & 31u;
      if (len == 0 || len >= kMaxLen) continue;
      if (pick < 0 || (e >> 5) <= best) {
        pick = s;
        best = e >> 5;
      }
    }
    if (pick < 0) break;
    const uint32_t e = col[pick * kLanes];
    kraft -= 1u << (kPrec - (e & 31u) - 1);
    col[pick * kLanes] = e + 1u;
  }
  // Aligned in-order assignment; entries become (base << 5) | length.
  uint32_t pos = 0;
  for (int s = 0; s < nb; ++s) {
    uint32_t len = col[s * kLanes] & 31u;
    if (len == 0) continue;
    uint32_t w = 1u << (kPrec - len);
    while (pos & (w - 1)) {
      w >>= 1;
      ++len;
    }
    col[s * kLanes] = (pos << 5) | len;
    pos += w;
  }
  int16_t *o = out + (static_cast<int64_t>(l) * C + c) * (nb + 1);
  uint32_t next = pos;
  for (int s = nb - 1; s >= 0; --s) {
    const uint32_t e = col[s * kLanes];
    const uint32_t len = e & 31u;
    uint32_t base;
    if (len == 0) {
      base = next;
    } else {
      base = e >> 5;
      next = base;
    }
    o[s] = static_cast<int16_t>(static_cast<uint16_t>((base | len) & 0xFFFFu));
  }
  o[nb] = 0;
}

__device__ __forceinline__ void put_bytes(uint8_t *row, int64_t chunk,
                                          int64_t at, uint32_t word, int n) {
  // `n` most significant bytes of `word` at byte offset `at`.
  for (int b = 0; b < n; ++b)
    if (at + b < chunk) row[at + b] = static_cast<uint8_t>(word >> (24 - 8 * b));
}

__global__ void __launch_bounds__(kLanes)
    encode_kernel(const int16_t *__restrict__ cdf,
                  const uint8_t *__restrict__ in, int T, int C, int nb,
                  uint8_t *__restrict__ out, int64_t chunk,
                  int32_t *__restrict__ lens, int tiles, int word_stores) {
  extern __shared__ uint32_t lds[];
  const int l = blockIdx.x / tiles;
  const int c = (blockIdx.x % tiles) * kLanes + threadIdx.x;
  if (c >= C) return;
  const int64_t stream = static_cast<int64_t>(l) * C + c;
  uint32_t *col = lds + threadIdx.x;
  unpack_row(cdf + stream * (nb + 1), nb, col);
  // Code table: (code << 5) | length.
  for (int s = 0; s < nb; ++s) {
    const uint32_t e = col[s * kLanes];
    const uint32_t len = e & 0xFFu;
    const uint32_t base = e >> 8;
    const uint32_t code =
        len ? (base >> (kPrec - len)) & ((1u << len) - 1u) : 0u;
    col[s * kLanes] = (code << 5) | len;
  }
  uint8_t *row = out + stream * chunk;
  const uint8_t *p = in + static_cast<int64_t>(l) * T * C + c;
  uint64_t acc = 0;
  int nbits = 0;
  int64_t wpos = 0;  // bytes already written
#pragma unroll 4
  for (int t = 0; t < T; ++t) {
    const uint32_t s = p[static_cast<int64_t>(t) * C];
    if (s >= static_cast<uint32_t>(nb)) continue;
    const uint32_t e = col[s * kLanes];
    const int len = static_cast<int>(e & 31u);
    acc = (acc << len) | (e >> 5);
    nbits += len;
    if (nbits >= 32) {
      const uint32_t word = static_cast<uint32_t>(acc >> (nbits - 32));
      if (word_stores && wpos + 4 <= chunk)
        *reinterpret_cast<uint32_t *>(row + wpos) = __builtin_bswap32(word);
      else
        put_bytes(row, chunk, wpos, word, 4);
      wpos += 4;
      nbits -= 32;
    }
  }
  if (nbits > 0) {
    const uint32_t tail = static_cast<uint32_t>(acc << (32 - nbits));
    put_bytes(row, chunk, wpos, tail, (nbits + 7) >> 3);
  }
  lens[stream] = static_cast<int32_t>(wpos + ((nbits + 7) >> 3));
}

__global__ void __launch_bounds__(kLanes)
    decode_kernel(const int16_t *__restrict__ cdf,
                  const uint8_t *__restrict__ bytes, int64_t nbytes,
                  const int32_t *__restrict__ prefix, int T, int C, int nb,
                  uint8_t *__restrict__ out, int tiles) {
  extern __shared__ uint32_t lds[];
  const int l = blockIdx.x / tiles;
  const int c = (blockIdx.x % tiles) * kLanes + threadIdx.x;
  if (c >= C) return;
  const int64_t stream = static_cast<int64_t>(l) * C + c;
  uint32_t *col = lds + threadIdx.x;
  unpack_row(cdf + stream * (nb + 1), nb, col);
  int64_t start = stream == 0 ? 0 : prefix[stream - 1];
  int64_t end = prefix[stream];
  start = start < 0 ? 0 : (start > nbytes ? nbytes : start);
  end = end > nbytes ? nbytes : (end < start ? start : end);
  uint64_t buf = 0;  // valid bits left-aligned
  int have = 0;
  int64_t rd = start;
  uint8_t *o = out + static_cast<int64_t>(l) * T * C + c;
  int top = 1;
  while (top * 2 < nb) top *= 2;
  for (int t = 0; t < T; ++t) {
    while (have <= 56) {
      const uint64_t b = rd < end ? bytes[rd] : 0u;
      ++rd;
      buf |= b << (56 - have);
      have += 8;
    }
    const uint32_t v = static_cast<uint32_t>(buf >> 48);
    int s = 0;
    for (int step = top; step > 0; step >>= 1)
      if (s + step < nb && (col[(s + step) * kLanes] >> 8) <= v) s += step;
    const int len = static_cast<int>(col[s * kLanes] & 0xFFu);
    o[static_cast<int64_t>(t) * C] = static_cast<uint8_t>(s);
    buf <<= len;
    have -= len;
  }
}

bool contiguous(const lmc_tensor &t) {
  int64_t expect = 1;
  for (int i = t.ndim - 1; i >= 0; --i) {
    if (t.sizes[i] != 1 && t.strides[i] != expect) return false;
    expect *= t.sizes[i];
  }
  return true;
}

void need_device(const lmc_tensor &t, const char *what) {
  check(t.device >= 0, std::string(what) + " should be on the GPU");
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
    const int tiles = static_cast<int>((C + kLanes - 1) / kLanes);
    const size_t lds = static_cast<size_t>(n_bins) * kLanes * 4;
    hipLaunchKernelGGL(cdf_kernel, dim3(L * tiles), dim3(kLanes), lds,
                       static_cast<hipStream_t>(stream),
                       static_cast<const uint8_t *>(in.data), (int)T, (int)C,
                       n_bins, static_cast<int16_t *>(o.data), tiles);
    hip_check(hipGetLastError(), "cdf_kernel launch");
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
          "Number of channels exceeds that supported be encode, contact "
          "LMCache Ascend about changing this limitation");
    check(in.dtype == LMC_U8 || in.dtype == LMC_I8, "input_sym must be int8/uint8");
    check(cdf.dtype == LMC_I16, "cdf must be int16");
    check(ob.dtype == LMC_U8 || ob.dtype == LMC_I8, "output_buffer must be uint8");
    check(ol.dtype == LMC_I32 && numel(ol) == L * C, "output_lengths must be int32 [L, C]");
    check(nb >= 1 && nb <= kMaxBins, "number of bins must be in [1, 64]");
    check(cdf.sizes[0] == L && cdf.sizes[1] == C, "cdf must be [L, C, nbins + 1]");
    check(ob.sizes[0] == L && ob.sizes[1] == C, "output_buffer must be [L, C, chunk]");
    if (L == 0 || C == 0) return;
    DeviceGuard guard(in.device);
    const int tiles = static_cast<int>((C + kLanes - 1) / kLanes);
    const size_t lds = static_cast<size_t>(nb) * kLanes * 4;
    const int word_stores =
        (chunk % 4 == 0 && (reinterpret_cast<uintptr_t>(ob.data) & 3) == 0) ? 1 : 0;
    hipLaunchKernelGGL(encode_kernel, dim3(L * tiles), dim3(kLanes), lds,
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
    check(cdf.device >= 0, "CDFs tensor should be on the GPU");
    check(bs.device >= 0, "Bytestreams tensor should be on the GPU");
    check(ln.device >= 0, "Lengths tensor should be on the GPU");
    check(o.device >= 0, "Output tensor should be on the GPU");
    need_device(cdf, "cdf");
    need_device(bs, "bytestreams");
    need_device(ln, "lengths");
    need_device(o, "output");
    check(cdf.ndim == 3, "cdf must be [L, C, nbins + 1]");
    const int64_t L = cdf.sizes[0], C = cdf.sizes[1], nb = cdf.sizes[2] - 1;
    check(C % 32 == 0,
          "Decode implementation relies on the number of channels being a "
          "multiple of 32, contact LMCache Ascend about changing this "
          "limitation");
    check(nb < 64, "Max bins constraint violated");
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
    const int tiles = static_cast<int>((C + kLanes - 1) / kLanes);
    const size_t lds = static_cast<size_t>(nb) * kLanes * 4;
    hipLaunchKernelGGL(decode_kernel, dim3(L * tiles), dim3(kLanes), lds,
                       static_cast<hipStream_t>(stream),
                       static_cast<const int16_t *>(cdf.data),
                       static_cast<const uint8_t *>(bs.data), numel(bs),
                       static_cast<const int32_t *>(ln.data), (int)T, (int)C,
                       (int)nb, static_cast<uint8_t *>(o.data), tiles);
    hip_check(hipGetLastError(), "decode_kernel launch");
  });
}

} // extern "C"
