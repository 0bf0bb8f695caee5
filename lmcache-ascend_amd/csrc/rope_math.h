// Element conversions and the fused K re-rotation of a group of pairs,
// shared by the K-RoPE kernel and the fused CacheBlend layer load.
//
// Arithmetic: the key and the cos/sin values are widened to fp32; the
// inverse rotation by the old angle and the forward rotation by the new one
// are evaluated as separate IEEE products and sums (contraction into FMA is
// disabled), and the caller rounds the result once to the key dtype (round
// to nearest even).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lmc {
namespace {

template <typename T, int N> struct alignas(sizeof(T) * N) Pack {
  T v[N];
};

// Element storage types: bf16 and fp16 as raw 16-bit patterns.
struct BF16 { using S = uint16_t; };
struct F16 { using S = uint16_t; };
struct F32 { using S = float; };

template <typename D> __device__ __forceinline__ float to_f32(typename D::S x);
template <> __device__ __forceinline__ float to_f32<BF16>(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}
template <> __device__ __forceinline__ float to_f32<F16>(uint16_t x) {
  _Float16 h;
  __builtin_memcpy(&h, &x, 2);
  return static_cast<float>(h);
}
template <> __device__ __forceinline__ float to_f32<F32>(float x) { return x; }

template <typename D> __device__ __forceinline__ typename D::S from_f32(float x);
template <> __device__ __forceinline__ uint16_t from_f32<BF16>(float x) {
  // Round to nearest even on the upper 16 bits; quiet NaNs stay NaN.
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
template <> __device__ __forceinline__ uint16_t from_f32<F16>(float x) {
  _Float16 h = static_cast<_Float16>(x);
  uint16_t r;
  __builtin_memcpy(&r, &h, 2);
  return r;
}
template <> __device__ __forceinline__ float from_f32<F32>(float x) { return x; }

// k <- R(new) R(old)^-1 k on VP pairs (x1[v], x2[v]): co/so are the cos/sin
// values of the old position, cn/sn those of the new one.
template <typename CD, int VP>
__device__ __forceinline__ void rerotate(const float (&x1)[VP], const float (&x2)[VP],
                                         const Pack<typename CD::S, VP> &co, const Pack<typename CD::S, VP> &so,
                                         const Pack<typename CD::S, VP> &cn, const Pack<typename CD::S, VP> &sn,
                                         float (&z1)[VP], float (&z2)[VP]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int v = 0; v < VP; ++v) {
    const float c0 = to_f32<CD>(co.v[v]), s0 = to_f32<CD>(so.v[v]);
    const float c1 = to_f32<CD>(cn.v[v]), s1 = to_f32<CD>(sn.v[v]);
    // R(old)^-1: rotation by -angle.
    const float y1 = x1[v] * c0 + x2[v] * s0;
    const float y2 = x2[v] * c0 - x1[v] * s0;
    // R(new).
    z1[v] = y1 * c1 - y2 * s1;
    z2[v] = y2 * c1 + y1 * s1;
  }
}

} // namespace
} // namespace lmc
