// sage_device.h — small gfx950 device helpers shared by the pre-pass and the
// attention kernel: element types, 16-byte loads, conversions, wave
// reductions, error reporting of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SAGE_HD __host__ __device__
#include "sage_quant_math.h"
#include "../../include/sage_attn.h"

namespace sage {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// element types
// ---------------------------------------------------------------------------
template <typename T>
struct Elt;
template <>
struct Elt<float> {
  static constexpr int kBytes = 4;
  static constexpr int kCode = SAGE_DTYPE_F32;
};
template <>
struct Elt<_Float16> {
  static constexpr int kBytes = 2;
  static constexpr int kCode = SAGE_DTYPE_F16;
};
template <>
struct Elt<__bf16> {
  static constexpr int kBytes = 2;
  static constexpr int kCode = SAGE_DTYPE_BF16;
};

// 8 consecutive elements of T held raw: 16 B for 2-byte types, 32 B for fp32.
template <typename T>
struct Raw8 {
  static constexpr int kU4 = Elt<T>::kBytes * 8 / 16;
  uint4 u[kU4];
};

template <typename T>
__device__ __forceinline__ Raw8<T> load8(const T* p) {
  Raw8<T> r;
  const uint4* s = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < Raw8<T>::kU4; ++i) r.u[i] = s[i];
  return r;
}

template <typename T>
__device__ __forceinline__ Raw8<T> zero8() {
  Raw8<T> r;
#pragma unroll
  for (int i = 0; i < Raw8<T>::kU4; ++i) r.u[i] = make_uint4(0, 0, 0, 0);
  return r;
}

__device__ __forceinline__ uint32_t word(const uint4& u, int i) {
  return i == 0 ? u.x : (i == 1 ? u.y : (i == 2 ? u.z : u.w));
}

// element e (0..7) of a raw 8-pack as fp32 (exact for every input type)
template <typename T>
__device__ __forceinline__ float elem(const Raw8<T>& r, int e);
template <>
__device__ __forceinline__ float elem<float>(const Raw8<float>& r, int e) {
  return __uint_as_float(word(r.u[e >> 2], e & 3));
}
template <>
__device__ __forceinline__ float elem<__bf16>(const Raw8<__bf16>& r, int e) {
  uint32_t w = word(r.u[0], e >> 1);
  return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
}
template <>
__device__ __forceinline__ float elem<_Float16>(const Raw8<_Float16>& r, int e) {
  uint32_t w = word(r.u[0], e >> 1);
  uint16_t hb = (uint16_t)((e & 1) ? (w >> 16) : (w & 0xFFFFu));
  _Float16 h = __builtin_bit_cast(_Float16, hb);
  return (float)h;
}

// ---------------------------------------------------------------------------
// wave64 reductions (xor butterflies over all 64 lanes)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// ---------------------------------------------------------------------------
// max of a non-negative value over the wave: DPP steps inside each 16-lane row
// (quad xor 1, quad xor 2, half-row mirror, row mirror), then the four row
// results via readlane.  Result is wave-uniform.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}

// max of a non-negative value over each group of W consecutive lanes (W = 4
// or 8: quad xor 1, quad xor 2, then the half-row mirror for 8); every lane
// of a group gets the group's max
template <int W>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  static_assert(W == 4 || W == 8, "group of 4 or 8 lanes");
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  if constexpr (W == 8) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  return v;
}

}  // namespace sage

// ---------------------------------------------------------------------------
// C-ABI error plumbing (defined in sage_abi.hip)
// ---------------------------------------------------------------------------
namespace sage {
int fail(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace sage
