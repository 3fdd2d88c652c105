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

// Per-channel statistics in LDS (K channel means, V scales): channel c at
// float stat_slot(c), 4 floats of padding after every 32 channels, so that
// the reads of the quantizing lanes (16 or 8 consecutive channels per lane,
// lanes of different channel groups side by side) and the writes of one
// channel per thread meet (almost) no bank conflicts on 64 or 32 banks.
__device__ __forceinline__ int stat_slot(int c) { return c + 4 * (c >> 5); }
template <int D>
constexpr int stat_lds_floats() {
  return D + 4 * (D / 32);
}

// LDS bytes vtile_block needs for its transpose: the tile itself, unpadded
template <int D, int PVM>
constexpr int vtile_lds_bytes() {
  return D * 64 * (PVM == SAGE_PV_FP8 ? 1 : 2);
}

// Placement of the transpose in LDS.  A unit is the 4*EB bytes of four
// consecutive tile positions of one channel (16 units per channel row); the
// row of channel d sits at physical row vt_row(d) and its unit u at unit
// u ^ vt_swz(d).  With the thread mapping of vtile_block (a wave's lanes:
// channel groups cg fastest, then key quads) both the per-channel unit
// writes and the 16-byte reads of the copy-out touch every bank at most once
// per cycle, on 64 banks and on 32.  Both depend on the channel group only,
// and vt_row changes the low two bits of d alone.
template <int D, int EB>
__device__ __forceinline__ int vt_row(int d) {
  const int cg = d >> 3;
  if constexpr (EB == 2) return d ^ ((D == 128 ? cg >> 3 : cg) & 1);
  else return d ^ (cg & 3);
}
template <int D, int EB>
__device__ __forceinline__ int vt_swz(int d) {
  const int cg = d >> 3;
  if constexpr (EB == 1 && D == 128) return (cg >> 1) & 15;
  else return cg & 15;
}

// 16-bit code of element e of a raw 8-pack in the tile's type: the input's
// own bits when the types agree, else the RNE conversion of its fp32 value
template <typename T, int PVM>
__device__ __forceinline__ uint32_t code16(const Raw8<T>& r, int e) {
  constexpr bool kSame = (__is_same(T, _Float16) && PVM == SAGE_PV_F16) || (__is_same(T, __bf16) && PVM == SAGE_PV_BF16);
  if constexpr (kSame) {
    const uint32_t w = word(r.u[0], e >> 1);
    return (e & 1) ? (w >> 16) : (w & 0xFFFFu);
  } else {
    return to16<PVM>(elem<T>(r, e));
  }
}

// e4m3 codes of four fp32 values, byte r = code of t[r]: gfx950's packed
// conversion (OCP e4m3fn, round to nearest even).  It equals f32_to_e4m3 for
// every |t| <= 448 * (1 + 2^-23), which bounds every quotient v / v_scale the
// pre-pass forms (tests/native/e4m3_hw_check.hip compares all 2^32 inputs).
__device__ __forceinline__ uint32_t e4m3x4(float t0, float t1, float t2, float t3) {
  uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(t0, t1, 0, false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(t2, t3, w, true);
}

// One 64-key tile t of one (batch, head), by a 256-thread block: thread
// (cg, kq) = (tid % (D/8), tid / (D/8)) loads channels 8cg..8cg+7 of keys
// 4kq..4kq+3 (16-byte loads along the rows of V; src: the head's first row,
// sn: row stride in elements), converts them and writes, per channel, the
// four keys' codes as one unit into the transpose (tile_s, 16-byte aligned,
// vtile_lds_bytes() bytes); after a barrier the block copies the tile out
// with 16-byte stores to dst (the tile's D*64*EB bytes).  With D = 64 the
// threads past 16 * 8 take part in the copy-out only.  vs_s: per-channel
// v_scale in LDS at stat_slot() (FP8 only), visible to every thread before
// the call.
// FP8 codes are RNE_sat(v / v_scale[d]) with the quotient correctly rounded:
// Markstein's division (div_rn_signed) and the packed conversion when every scale
// of the wave lies in the fast range, IEEE division and f32_to_e4m3
// otherwise; 0 where v_scale[d] == 0.
template <typename T, int D, int PVM>
__device__ __forceinline__ void vtile_block(const T* __restrict__ src, int64_t sn, int64_t Nkv, int64_t t,
                                            const float* vs_s, uint8_t* __restrict__ dst, char* tile_s) {
  constexpr bool kF8 = PVM == SAGE_PV_FP8;
  constexpr int EB = kF8 ? 1 : 2;
  constexpr int ROWB = 64 * EB;  // bytes of a channel row
  constexpr int UNIT = 4 * EB;   // bytes of a unit
  constexpr int CG = D / 8;      // 8-channel groups per key row
  const int tid = threadIdx.x;
  if (tid < 16 * CG) {
    const int cg = tid % CG, kq = tid / CG;
    const int64_t n0 = t * 64 + 4 * kq;
    Raw8<T> x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = n0 + r < Nkv ? load8<T>(src + (n0 + r) * sn + 8 * cg) : zero8<T>();
    const int u = vtile_pos(4 * kq) >> 2;
    if constexpr (kF8) {
      float sc[8], rc[8];
      bool ok = true;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sc[e] = vs_s[stat_slot(8 * cg + e)];
        rc[e] = sc[e] > 0.0f ? 1.0f / sc[e] : 0.0f;
        ok = ok && fast_div_ok(sc[e]);
      }
      auto emit = [&](auto fast_tag) __attribute__((always_inline)) {
        constexpr bool kFast = decltype(fast_tag)::value;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          uint32_t w = 0;
          if constexpr (kFast) {
            float q[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) q[r] = div_rn_signed(elem<T>(x[r], e), sc[e], rc[e]);
            w = e4m3x4(q[0], q[1], q[2], q[3]);
          } else {  // scales out of range: quotients may leave the instruction's exact range
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float v = elem<T>(x[r], e);
              w |= (uint32_t)f32_to_e4m3(sc[e] > 0.0f ? v / sc[e] : 0.0f) << (8 * r);
            }
          }
          const int d = 8 * cg + e;
          *reinterpret_cast<uint32_t*>(tile_s + vt_row<D, EB>(d) * ROWB + (u ^ vt_swz<D, EB>(d)) * UNIT) = w;
        }
      };
      if (__builtin_amdgcn_ballot_w64(!ok) == 0) emit(std::true_type{});
      else emit(std::false_type{});
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * cg + e;
        const uint2 w = make_uint2(code16<T, PVM>(x[0], e) | (code16<T, PVM>(x[1], e) << 16),
                                   code16<T, PVM>(x[2], e) | (code16<T, PVM>(x[3], e) << 16));
        *reinterpret_cast<uint2*>(tile_s + vt_row<D, EB>(d) * ROWB + (u ^ vt_swz<D, EB>(d)) * UNIT) = w;
      }
    }
  }
  __syncthreads();
  constexpr int CPR = ROWB / 16;  // 16-byte chunks per channel row
  constexpr int UPC = 16 / UNIT;  // units per chunk
  for (int it = tid; it < D * CPR; it += 256) {
    const int d = it / CPR, c = it % CPR;
    const int g = vt_swz<D, EB>(d);
    // logical dword j of chunk c sits in physical chunk c ^ (g / UPC), dword j ^ s
    const int s = EB == 2 ? 2 * (g & 1) : (g & 3);
    const uint4 p = *reinterpret_cast<const uint4*>(tile_s + vt_row<D, EB>(d) * ROWB + 16 * (c ^ (g / UPC)));
    const bool s1 = s & 1, s2 = s & 2;
    const uint32_t b0 = s1 ? p.y : p.x, b1 = s1 ? p.x : p.y, b2 = s1 ? p.w : p.z, b3 = s1 ? p.z : p.w;
    *reinterpret_cast<uint4*>(dst + (int64_t)d * ROWB + 16 * c) =
        make_uint4(s2 ? b2 : b0, s2 ? b3 : b1, s2 ? b0 : b2, s2 ? b1 : b3);
  }
}

}  // namespace sage
