// Host check of the pre-pass element arithmetic (tribench_amd/csrc/sage_quant_math.h).
//
// The header is compiled here by g++ with floating-point contraction off,
// exactly as the gfx950 build compiles it (__builtin_fmaf is a correctly
// rounded fma on both).  Modes:
//   div <scale_bits_hex> [k]   every fp32 x with |x| <= 127.5*scale (both signs;
//                              with k, only |x| >= scale*2^k):
//                              quant_elem must equal the reference rounding
//                              (t = x/s; t += +-0.5; trunc), and div_rn(x, s,
//                              RN(1/s)) must equal IEEE x/s for |x| >= 2^-100
//   divrand <n_scales> <n_x>   random scales in [2^-100, 2^100], random x
//   fp8div <bf16|f16> <stride> FP8 V codes through Markstein's division against
//                              IEEE division (div_rn_signed), every 16-bit x
//                              per stride-th amax
//   fp8divrand <n_amax> <n_x>  the same for random fp32 amax and x
//   e4m3 <stride> <out_file>   f32_to_e4m3 of every stride-th bit pattern below
//                              0x7F800001, written as bytes for comparison with
//                              the numpy oracle
// Prints "OK <count>" or the first mismatch and exits non-zero.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../tribench_amd/csrc/sage_quant_math.h"

static float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static int8_t ref_quant(float x, float scale) {
  float t = (scale > 0.0f) ? x / scale : 0.0f;
  float u = t + (t >= 0.0f ? 0.5f : -0.5f);
  return (int8_t)(int)u;
}

static int check_scale(float s, float xmin, uint64_t* count) {
  const float r = 1.0f / s;
  const bool fast = sage::fast_div_ok(s);
  const float lim = 127.5f * s;
  const uint32_t top = sage::f32_bits(lim);
  for (uint32_t b = sage::f32_bits(xmin); b <= top; ++b) {
    for (int sg = 0; sg < 2; ++sg) {
      const float x = sg ? -from_bits(b) : from_bits(b);
      const int8_t q = sage::quant_elem(x, s, r, fast);
      const int8_t w = ref_quant(x, s);
      if (q != w) {
        printf("MISMATCH quant scale=%a x=%a got %d want %d\n", s, x, q, w);
        return 1;
      }
      if (fast) {
        const float t = sage::div_rn(x, s, r), tw = x / s;
        // the quotient is the correctly rounded one whenever the residual of
        // the correction cannot underflow (|x| >= 2^-100; any x whose int8
        // rounding is in question has |x| >= scale/4 >= 2^-102 anyway, and
        // the int8 result is compared for every x above)
        if (t != tw && (x >= 0x1p-100f || x <= -0x1p-100f)) {
          printf("MISMATCH div scale=%a x=%a got %a want %a\n", s, x, t, tw);
          return 1;
        }
      }
      ++*count;
    }
  }
  return 0;
}

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd() {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return (uint32_t)(rng_state >> 16);
}

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  uint64_t count = 0;
  if (!strcmp(argv[1], "div") && (argc == 3 || argc == 4)) {
    const float s = from_bits((uint32_t)strtoul(argv[2], 0, 16));
    // optional: start at |x| = scale * 2^k (k < 0) instead of 0
    const float xmin = argc == 4 ? s * __builtin_ldexpf(1.0f, atoi(argv[3])) : 0.0f;
    if (check_scale(s, xmin, &count)) return 1;
  } else if (!strcmp(argv[1], "divrand") && argc == 4) {
    const int ns = atoi(argv[2]), nx = atoi(argv[3]);
    for (int i = 0; i < ns; ++i) {
      // amax in [2^-93, 2^107) -> scale in about [2^-100, 2^100]
      const float amax = from_bits(((uint32_t)(rnd() % 200 + 34) << 23) | (rnd() & 0x7FFFFF));
      const float s = sage::block_scale(amax);
      const float r = 1.0f / s;
      const bool fast = sage::fast_div_ok(s);
      for (int j = 0; j < nx; ++j) {
        float x = amax * ((float)(rnd() & 0xFFFFFF) / 16777216.0f);
        if (rnd() & 1) x = -x;
        if (j == 0) x = amax;
        const int8_t q = sage::quant_elem(x, s, r, fast), w = ref_quant(x, s);
        if (q != w || (fast && (x >= 0x1p-100f || x <= -0x1p-100f) && sage::div_rn(x, s, r) != x / s)) {
          printf("MISMATCH scale=%a x=%a got %d want %d\n", s, x, q, w);
          return 1;
        }
        ++count;
      }
    }
  } else if (!strcmp(argv[1], "fp8div") && argc == 4) {
    // FP8 V codes of 16-bit inputs: for every positive finite amax of the
    // type (every stride-th pattern) with v_scale = amax / 448 in the fast
    // range and every x of the type with |x| <= amax, both signs, the
    // kernels' fast path e4m3(div_rn(x, s, RN(1/s))) must equal e4m3(x / s)
    const bool bf = !strcmp(argv[2], "bf16");
    const uint32_t stride = (uint32_t)strtoul(argv[3], 0, 10);
    const uint32_t top = bf ? 0x7F80u : 0x7C00u;  // first non-finite pattern
    auto value = [bf](uint32_t h) {
      if (bf) return from_bits(h << 16);
      const uint32_t e = (h >> 10) & 31u, m = h & 1023u;  // fp16 (finite patterns only)
      return e ? __builtin_ldexpf((float)(1024u + m), (int)e - 25) : __builtin_ldexpf((float)m, -24);
    };
    for (uint32_t ha = 1; ha < top; ha += stride) {
      const float amax = value(ha);
      const float s = amax / 448.0f;
      if (!sage::fast_div_ok(s)) continue;
      const float r = 1.0f / s;
      for (uint32_t hx = 0; hx <= ha; ++hx) {
        for (int sg = 0; sg < 2; ++sg) {
          const float x = sg ? -value(hx) : value(hx);
          const uint8_t got = sage::f32_to_e4m3(sage::div_rn_signed(x, s, r)), want = sage::f32_to_e4m3(x / s);
          if (got != want) {
            printf("MISMATCH fp8 scale=%a x=%a got %02x want %02x\n", s, x, got, want);
            return 1;
          }
          ++count;
        }
      }
    }
  } else if (!strcmp(argv[1], "fp8divrand") && argc == 4) {
    // the same for fp32 inputs: random amax over the fast range, random x
    const int ns = atoi(argv[2]), nx = atoi(argv[3]);
    for (int i = 0; i < ns; ++i) {
      const float amax = from_bits(((uint32_t)(rnd() % 200 + 27) << 23) | (rnd() & 0x7FFFFF));
      const float s = amax / 448.0f;
      if (!sage::fast_div_ok(s)) continue;
      const float r = 1.0f / s;
      for (int j = 0; j < nx; ++j) {
        // |x| spread over 2^-24 .. 1 of amax, uniform in the exponent
        float x = __builtin_ldexpf(amax * (0.5f + 0.5f * (float)(rnd() & 0xFFFFFF) / 16777216.0f), -(int)(rnd() % 25));
        if (rnd() & 1) x = -x;
        if (j == 0) x = amax;
        const uint8_t got = sage::f32_to_e4m3(sage::div_rn_signed(x, s, r)), want = sage::f32_to_e4m3(x / s);
        if (got != want) {
          printf("MISMATCH fp8 scale=%a x=%a got %02x want %02x\n", s, x, got, want);
          return 1;
        }
        ++count;
      }
    }
  } else if (!strcmp(argv[1], "e4m3") && argc == 4) {
    const uint32_t stride = (uint32_t)strtoul(argv[2], 0, 10);
    FILE* f = fopen(argv[3], "wb");
    if (!f) return 2;
    for (uint64_t b = 0; b < 0x7F800001ull; b += stride) {
      const uint8_t c0 = sage::f32_to_e4m3(from_bits((uint32_t)b));
      const uint8_t c1 = sage::f32_to_e4m3(-from_bits((uint32_t)b));
      fputc(c0, f);
      fputc(c1, f);
      ++count;
    }
    fclose(f);
  } else {
    return 2;
  }
  printf("OK %llu\n", (unsigned long long)count);
  return 0;
}
