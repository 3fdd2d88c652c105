// sage_quant_math.h — element arithmetic of the SageAttention pre-pass.
//
// Plain C++ with no device intrinsics, so the same text is compiled into the
// gfx950 kernels (SAGE_HD = __host__ __device__) and into host programs that
// check it exhaustively against IEEE arithmetic (SAGE_HD empty).  Translation
// units that include it must be compiled with floating-point contraction off
// (-ffp-contract=off): every rounding below is deliberate.
#pragma once
#include <stdint.h>
#include <string.h>

#ifndef SAGE_HD
#define SAGE_HD
#endif

namespace sage {

// Scale of a quantization block: max|x| / 127 with IEEE division
// (triton_impl.py:28).
SAGE_HD inline float block_scale(float amax) { return amax / 127.0f; }

// Range of scales for which div_rn() below is used.  Outside it (including
// the all-zero block, scale == 0) the kernels fall back to a true division.
SAGE_HD inline bool fast_div_ok(float scale) { return scale >= 0x1p-100f && scale <= 0x1p+100f; }

// RN(x / scale) from rcp = RN(1 / scale) with Markstein's correction
// (P. Markstein, IBM J. Res. Dev. 34(1), 1990; Muller et al., Handbook of
// Floating-Point Arithmetic, thm. "Markstein"): with q0 within one ulp of
// x/scale and rcp within half an ulp of 1/scale, the residual
// e = x - q0*scale is exact and RN(q0 + e*rcp) is the correctly rounded
// quotient.  Three FMA-unit operations instead of a full division.
SAGE_HD inline float div_rn(float x, float scale, float rcp) {
  float q0 = x * rcp;
  float e = __builtin_fmaf(-q0, scale, x);
  return __builtin_fmaf(e, rcp, q0);
}

// div_rn with the sign of a zero quotient kept: x = -0 gives -0, as IEEE
// division does (div_rn's residual is +0 there, which turns the sum into
// +0).  Needed where the quotient's sign survives the rounding (FP8 codes:
// -0 encodes as 0x80); for nonzero x the sign is already that of x.
SAGE_HD inline float div_rn_signed(float x, float scale, float rcp) {
  return __builtin_copysignf(div_rn(x, scale, rcp), x);
}

// The reference's rounding (triton_impl.py:29-31): t += 0.5*sign(t) in fp32,
// then truncate toward zero.  Note fp32(0.49999997 + 0.5) == 1.0.
SAGE_HD inline int round_half_away(float t) {
  // copysign(0.5, t) equals (t >= 0 ? 0.5 : -0.5) except at t = -0, where
  // -0 - 0.5 and -0 + 0.5 both truncate to 0
  float u = t + __builtin_copysignf(0.5f, t);
  return (int)u;
}

// One element: x already multiplied by the Q multiplier (or smoothed).
// The all-zero block (scale == 0) is defined to quantize to 0; the reference
// would divide 0 by 0 there.
SAGE_HD inline int8_t quant_elem(float x, float scale, float rcp, bool fast) {
  float t;
  if (fast) {
    t = div_rn(x, scale, rcp);
  } else {
    t = (scale > 0.0f) ? x / scale : 0.0f;
  }
  return (int8_t)round_half_away(t);
}

SAGE_HD inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

// fp32 -> OCP FP8 e4m3 ("e4m3fn": bias 7, no infinities, 0x7F = NaN,
// max finite 448) with round-to-nearest-even and saturation to +-448.
// Agrees with torch's float8_e4m3fn cast for every |f| <= 464 (above that
// torch produces NaN); the pre-pass only produces |f| <= 448*(1+2^-23).
SAGE_HD inline uint8_t f32_to_e4m3(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0x7Fu;  // NaN
  float af;
  memcpy(&af, &a, 4);
  if (af >= 448.0f) return (uint8_t)(sign | 0x7Eu);
  uint32_t code;
  if (af < 0x1p-6f) {
    // subnormal range: code = RNE(af * 2^9) in 0..8 (8 is the smallest normal)
    float s = af * 512.0f;  // exact
    float r = __builtin_rintf(s);
    code = (uint32_t)r;
  } else {
    uint32_t e = (a >> 23) - 127u + 7u;  // 1..15
    uint32_t m = a & 0x7FFFFFu;
    uint32_t m3 = m >> 20;
    uint32_t rem = m & 0xFFFFFu;
    uint32_t up = (rem > 0x80000u) || (rem == 0x80000u && (m3 & 1u));
    code = (e << 3) + m3 + up;  // a mantissa carry moves into the exponent
    if (code > 0x7Eu) code = 0x7Eu;
  }
  return (uint8_t)(sign | code);
}

// Rows of a K-statistics chunk handled per pass and the chunking of the
// sequence.  The K channel mean is defined by this fixed reduction order:
//   lane sums:  thread (tl, cg) adds tokens n0+tl, n0+tl+TL, ... in order
//   lane tree:  acc[tl] += acc[tl + s] for s = TL/2, TL/4, ..., 1
//   chunk sum:  S = P_0 + P_1 + ... + P_{nch-1} (left to right)
//   mean:       km = S / (float)N
SAGE_HD inline int kstat_token_lanes(int D) { return 256 / (D / 8); }
SAGE_HD inline int64_t kstat_chunk_tokens(int64_t N) { return 256 * ((N + 4095) / 4096); }
SAGE_HD inline int64_t kstat_num_chunks(int64_t N) {
  int64_t ch = kstat_chunk_tokens(N);
  return (N + ch - 1) / ch;
}

}  // namespace sage
