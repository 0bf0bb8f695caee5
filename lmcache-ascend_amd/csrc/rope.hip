// Fused K re-rotation for CacheBlend on MI355X (gfx950):
//     k <- R(new_pos) * R(old_pos)^-1 * k      (in place, per head)
//
// Replaces rotary_embedding_k_fused (csrc/pos_kernels.cpp:158-196).  The op
// is HBM-bound elementwise work (each key element is read and written once;
// the cos/sin rows of the two positions are shared by all heads of a token
// and stay in L2), so there is no tiling: one thread owns VP consecutive
// rotation pairs of one (token, head) and moves them with vector loads of up
// to 16 bytes (VP = 8 for bf16/fp16 neox).
//
// Arithmetic: the key and the cos/sin values are widened to fp32; the
// inverse rotation by the old angle and the forward rotation by the new one
// are evaluated as separate IEEE products and sums (contraction into FMA is
// disabled), then the result is rounded once to the key dtype (round to
// nearest even).  This is the fp32 path the reference's unified-buffer
// sizing implies (csrc/pos_kernels.cpp:119-126) and makes the result
// reproducible operation for operation on the CPU.
//
// rot = cos_sin_cache.size(-1) dims of each head are rotated (neox: halves
// [0, rot/2) and [rot/2, rot); GPT-J: interleaved pairs); the remaining
// head_size - rot dims pass through.  Tokens whose old or new position lies
// outside the cache are left unchanged.
#include "common.h"
#include "rope_math.h"

#include <cstring>

namespace lmc {

namespace {

template <typename KD, typename CD, bool NEOX, int VP>
__global__ void __launch_bounds__(256)
    rope_k_fused(const void *old_pos, const void *new_pos, int pos_i32,
                 typename KD::S *key, int64_t key_stride, int head_size,
                 int n_heads, int n_tokens, const typename CD::S *cache,
                 int64_t cache_stride, int64_t max_pos, int rot) {
#pragma clang fp contract(off)
  using KS = typename KD::S;
  using CS = typename CD::S;
  const int half = rot / 2;
  const int groups = half / VP;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(n_tokens) * n_heads * groups;
  if (g >= total) return;
  const int j = static_cast<int>(g % groups);
  const int64_t th = g / groups;
  const int h = static_cast<int>(th % n_heads);
  const int t = static_cast<int>(th / n_heads);
  const int64_t po = pos_i32 ? static_cast<const int32_t *>(old_pos)[t]
                             : static_cast<const int64_t *>(old_pos)[t];
  const int64_t pn = pos_i32 ? static_cast<const int32_t *>(new_pos)[t]
                             : static_cast<const int64_t *>(new_pos)[t];
  if (po < 0 || po >= max_pos || pn < 0 || pn >= max_pos) return;
  const int i0 = j * VP;
  const CS *crow_o = cache + po * cache_stride;
  const CS *crow_n = cache + pn * cache_stride;
  const Pack<CS, VP> co = *reinterpret_cast<const Pack<CS, VP> *>(crow_o + i0);
  const Pack<CS, VP> so = *reinterpret_cast<const Pack<CS, VP> *>(crow_o + half + i0);
  const Pack<CS, VP> cn = *reinterpret_cast<const Pack<CS, VP> *>(crow_n + i0);
  const Pack<CS, VP> sn = *reinterpret_cast<const Pack<CS, VP> *>(crow_n + half + i0);
  KS *head = key + static_cast<int64_t>(t) * key_stride +
             static_cast<int64_t>(h) * head_size;

  float x1[VP], x2[VP];
  if constexpr (NEOX) {
    const Pack<KS, VP> a = *reinterpret_cast<const Pack<KS, VP> *>(head + i0);
    const Pack<KS, VP> b = *reinterpret_cast<const Pack<KS, VP> *>(head + half + i0);
#pragma unroll
    for (int v = 0; v < VP; ++v) {
      x1[v] = to_f32<KD>(a.v[v]);
      x2[v] = to_f32<KD>(b.v[v]);
    }
  } else {
    const Pack<KS, 2 * VP> ab =
        *reinterpret_cast<const Pack<KS, 2 * VP> *>(head + 2 * i0);
#pragma unroll
    for (int v = 0; v < VP; ++v) {
      x1[v] = to_f32<KD>(ab.v[2 * v]);
      x2[v] = to_f32<KD>(ab.v[2 * v + 1]);
    }
  }
  float z1[VP], z2[VP];
  rerotate<CD, VP>(x1, x2, co, so, cn, sn, z1, z2);
  if constexpr (NEOX) {
    Pack<KS, VP> a, b;
#pragma unroll
    for (int v = 0; v < VP; ++v) {
      a.v[v] = from_f32<KD>(z1[v]);
      b.v[v] = from_f32<KD>(z2[v]);
    }
    *reinterpret_cast<Pack<KS, VP> *>(head + i0) = a;
    *reinterpret_cast<Pack<KS, VP> *>(head + half + i0) = b;
  } else {
    Pack<KS, 2 * VP> ab;
#pragma unroll
    for (int v = 0; v < VP; ++v) {
      ab.v[2 * v] = from_f32<KD>(z1[v]);
      ab.v[2 * v + 1] = from_f32<KD>(z2[v]);
    }
    *reinterpret_cast<Pack<KS, 2 * VP> *>(head + 2 * i0) = ab;
  }
}

struct RopeArgs {
  const void *old_pos, *new_pos;
  int pos_i32;
  void *key;
  int64_t key_stride;
  int head_size, n_heads, n_tokens;
  const void *cache;
  int64_t cache_stride, max_pos;
  int rot;
};

template <typename KD, typename CD, bool NEOX, int VP>
void launch(const RopeArgs &a, hipStream_t s) {
  const int64_t total =
      static_cast<int64_t>(a.n_tokens) * a.n_heads * (a.rot / 2 / VP);
  if (total == 0) return;
  const int64_t blocks = (total + 255) / 256;
  check(blocks < (int64_t(1) << 31), "rotary: too many tokens");
  hipLaunchKernelGGL((rope_k_fused<KD, CD, NEOX, VP>), dim3(blocks), dim3(256),
                     0, s, a.old_pos, a.new_pos, a.pos_i32,
                     static_cast<typename KD::S *>(a.key), a.key_stride,
                     a.head_size, a.n_heads, a.n_tokens,
                     static_cast<const typename CD::S *>(a.cache),
                     a.cache_stride, a.max_pos, a.rot);
  hip_check(hipGetLastError(), "rope_k_fused launch");
}

template <typename KD, typename CD, bool NEOX>
void launch_vp(const RopeArgs &a, int vp, hipStream_t s) {
  switch (vp) {
  case 8: launch<KD, CD, NEOX, 8>(a, s); break;
  case 4: launch<KD, CD, NEOX, 4>(a, s); break;
  case 2: launch<KD, CD, NEOX, 2>(a, s); break;
  default: launch<KD, CD, NEOX, 1>(a, s); break;
  }
}

template <typename KD>
void launch_cache(const RopeArgs &a, int cache_dt, bool neox, int vp,
                  hipStream_t s) {
  switch (cache_dt) {
  case LMC_BF16:
    neox ? launch_vp<KD, BF16, true>(a, vp, s) : launch_vp<KD, BF16, false>(a, vp, s);
    break;
  case LMC_F16:
    neox ? launch_vp<KD, F16, true>(a, vp, s) : launch_vp<KD, F16, false>(a, vp, s);
    break;
  case LMC_F32:
    neox ? launch_vp<KD, F32, true>(a, vp, s) : launch_vp<KD, F32, false>(a, vp, s);
    break;
  default:
    fail(LMC_ERR_RUNTIME, "cos_sin_cache dtype must be bf16, fp16 or fp32");
  }
}

} // namespace

} // namespace lmc

using namespace lmc;

extern "C" int lmc_rotary_embedding_k_fused(const lmc_tensor *old_positions,
                                            const lmc_tensor *new_positions,
                                            const lmc_tensor *key,
                                            int64_t head_size,
                                            const lmc_tensor *cos_sin_cache,
                                            int32_t is_neox, void *stream) {
  return guarded([&] {
    const lmc_tensor &op = deref(old_positions, "oldPositions");
    const lmc_tensor &np_ = deref(new_positions, "newPositions");
    const lmc_tensor &k = deref(key, "key");
    const lmc_tensor &c = deref(cos_sin_cache, "cosSinCache");
    // csrc/pos_kernels.cpp:47-57: only bf16 / fp16 / fp32 keys.
    if (k.dtype != LMC_BF16 && k.dtype != LMC_F16 && k.dtype != LMC_F32)
      fail(LMC_ERR_VALUE, "rotary_embedding_k_fused rotates bfloat16, float16 or "
                          "float32 keys only");
    check(k.ndim == 2, "key must be [num_tokens, num_heads * head_size]");
    check(head_size > 0 && size(k, 1) % head_size == 0,
          "key width is not a multiple of head_size");
    check(k.strides[1] == 1 || k.sizes[1] <= 1, "key rows must be contiguous");
    check(c.ndim >= 1, "cos_sin_cache must have a last dimension");
    const int64_t rot = size(c, -1);
    check(rot > 0 && rot % 2 == 0 && rot <= head_size,
          "rotary dim must be even and at most head_size");
    const int64_t max_pos = numel(c) / rot;
    check(c.ndim == 1 || stride(c, -1) == 1, "cos_sin_cache must be contiguous");
    if (c.ndim >= 2)
      check(stride(c, -2) == rot, "cos_sin_cache must be contiguous");
    check(op.ndim == 1 && np_.ndim == 1 && op.sizes[0] == k.sizes[0] &&
              np_.sizes[0] == k.sizes[0],
          "positions must be 1-D with one entry per token");
    check(op.dtype == np_.dtype && (op.dtype == LMC_I64 || op.dtype == LMC_I32),
          "positions must both be int64 or int32");
    check((op.sizes[0] <= 1 || op.strides[0] == 1) &&
              (np_.sizes[0] <= 1 || np_.strides[0] == 1),
          "positions must be contiguous");
    if (k.sizes[0] == 0) return;
    DeviceGuard guard(k.device);
    RopeArgs a;
    a.old_pos = kernel_ptr(op);
    a.new_pos = kernel_ptr(np_);
    a.pos_i32 = op.dtype == LMC_I32;
    a.key = kernel_ptr(k);
    a.key_stride = k.strides[0];
    a.head_size = static_cast<int>(head_size);
    a.n_heads = static_cast<int>(size(k, 1) / head_size);
    a.n_tokens = static_cast<int>(k.sizes[0]);
    a.cache = kernel_ptr(c);
    a.cache_stride = rot;
    a.max_pos = max_pos;
    a.rot = static_cast<int>(rot);
    // Widest pair group whose vector accesses stay aligned.
    const int64_t kes = elem_size(k), ces = elem_size(c);
    const int64_t half = rot / 2;
    auto aligned = [&](int vp) {
      if (half % vp) return false;
      const bool neox = is_neox != 0;
      const int64_t kvec = (neox ? vp : 2 * vp) * kes;  // key access bytes
      const int64_t cvec = vp * ces;
      auto ok = [](int64_t v, int64_t a) { return a <= 16 && v % a == 0; };
      return ok(reinterpret_cast<uintptr_t>(a.key), kvec) &&
             ok(a.key_stride * kes, kvec) && ok(head_size * kes, kvec) &&
             (!neox || ok(half * kes, kvec)) &&
             ok(reinterpret_cast<uintptr_t>(a.cache), cvec) &&
             ok(rot * ces, cvec) && ok(half * ces, cvec);
    };
    const int vp = aligned(8) ? 8 : aligned(4) ? 4 : aligned(2) ? 2 : 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (k.dtype) {
    case LMC_BF16: launch_cache<BF16>(a, c.dtype, is_neox != 0, vp, s); break;
    case LMC_F16: launch_cache<F16>(a, c.dtype, is_neox != 0, vp, s); break;
    default: launch_cache<F32>(a, c.dtype, is_neox != 0, vp, s); break;
    }
  });
}
