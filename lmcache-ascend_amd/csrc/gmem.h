// Vector loads and stores through the global address space.  Pointers the
// kernels form from loaded values (pointer tables, chunk tables, packet
// addresses) carry no address space, so the compiler would issue flat
// accesses for them, which also count against the LDS counter: every wait
// for such a load then waits for LDS work as well.  Device memory and
// page-locked host memory are both in the global address space.
#pragma once

template <typename T> __device__ __forceinline__ T gload(const T *p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) T *>(reinterpret_cast<uintptr_t>(p));
}
template <typename T> __device__ __forceinline__ void gstore(T *p, T v) {
  *reinterpret_cast<__attribute__((address_space(1))) T *>(reinterpret_cast<uintptr_t>(p)) = v;
}

// The same with the streaming (non-temporal) hint.
template <typename T> __device__ __forceinline__ T gload_nt(const T *p) {
  return __builtin_nontemporal_load(
      reinterpret_cast<const __attribute__((address_space(1))) T *>(reinterpret_cast<uintptr_t>(p)));
}
template <typename T> __device__ __forceinline__ void gstore_nt(T *p, T v) {
  __builtin_nontemporal_store(v, reinterpret_cast<__attribute__((address_space(1))) T *>(reinterpret_cast<uintptr_t>(p)));
}
