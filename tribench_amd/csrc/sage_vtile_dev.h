// sage_vtile_dev.h — one V tile in the attention kernel's layout (device side
// of sage_vtiles.hip, shared with the pre-pass, which can produce the tiles in
// its own launches).
//
// Tile layout (element size EB: 2 for fp16/bf16, 1 for e4m3):
//   byte of (b, h, key n, channel d) =
//     ((((b*Hkv + h)*T + n/64)*D + d)*64 + pos(n % 64)) * EB,   T = ceil(Nkv/64)
//   pos(32t + 8i + 4h + r) = 32h + 16t + 4i + r
// pos() is the order in which lane half h of a 32x32 MFMA C tile holds the
// keys of its column (registers 4i + r of key tiles t = 0, 1).  Keys past Nkv
// hold 0.  e4m3 codes are RNE_sat(v / v_scale[d]) (0 where v_scale[d] == 0),
// the same codes as the pre-pass's row-major FP8 V.  Build with
// -ffp-contract=off (the e4m3 division must be IEEE).
#pragma once

#include "sage_device.h"

namespace sage {

__device__ __forceinline__ int vtile_pos(int k) {
  return ((k >> 2) & 1) * 32 + (k >> 5) * 16 + ((k >> 3) & 3) * 4 + (k & 3);
}

template <int PVM>
__device__ __forceinline__ uint16_t to16(float x);
template <>
__device__ __forceinline__ uint16_t to16<SAGE_PV_F16>(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}
template <>
__device__ __forceinline__ uint16_t to16<SAGE_PV_BF16>(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// LDS bytes vtile_block needs for its transpose (row pitch 64*EB + 4 bytes,
// an odd number of dwords, so the column writes do not conflict)
template <int D, int PVM>
constexpr int vtile_lds_bytes() {
  return D * (64 * (PVM == SAGE_PV_FP8 ? 1 : 2) + 4);
}

// One 64-key tile t of one (batch, head), by a 256-thread block: 16-byte
// loads along the rows of V (src: the head's first row, sn: row stride in
// elements), conversion, transposition through LDS (tile_s, 16-byte
// aligned, vtile_lds_bytes() bytes), 16-byte stores to dst (the tile's
// D*64*EB bytes).  vs_s: per-channel v_scale in LDS (FP8 only), visible to
// every thread before the call.
template <typename T, int D, int PVM>
__device__ __forceinline__ void vtile_block(const T* __restrict__ src, int64_t sn, int64_t Nkv, int64_t t,
                                            const float* vs_s, uint8_t* __restrict__ dst, char* tile_s) {
  constexpr bool kF8 = PVM == SAGE_PV_FP8;
  constexpr int EB = kF8 ? 1 : 2;
  constexpr int RP = 64 * EB + 4;
  constexpr int CG = D / 8;  // 8-channel groups per key row
  constexpr int NIT = 64 * CG / 256;
  const int tid = threadIdx.x;
  const int64_t k0 = t * 64;
#pragma unroll
  for (int i = 0; i < NIT; ++i) {
    const int it = tid + 256 * i;
    const int cg = it % CG, key = it / CG;
    const int64_t n = k0 + key;
    const Raw8<T> x = n < Nkv ? load8<T>(src + n * sn + 8 * cg) : zero8<T>();
    const int pos = vtile_pos(key);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * cg + e;
      const float val = elem<T>(x, e);
      if constexpr (kF8) {
        const float s = vs_s[d];
        *reinterpret_cast<uint8_t*>(tile_s + d * RP + pos) = f32_to_e4m3(s > 0.0f ? val / s : 0.0f);
      } else {
        *reinterpret_cast<uint16_t*>(tile_s + d * RP + 2 * pos) = to16<PVM>(val);
      }
    }
  }
  __syncthreads();
  constexpr int CPR = 4 * EB;  // 16-byte chunks per tile row
  for (int it = tid; it < D * CPR; it += 256) {
    const int d = it / CPR, c = it % CPR;
    const uint32_t* s4 = reinterpret_cast<const uint32_t*>(tile_s + d * RP + 16 * c);
    *reinterpret_cast<uint4*>(dst + (int64_t)d * 64 * EB + 16 * c) = make_uint4(s4[0], s4[1], s4[2], s4[3]);
  }
}

}  // namespace sage
