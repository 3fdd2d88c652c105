// power_model.hip — board power of each instruction class the attention loop
// is made of, run alone on every CU: the energy per instruction behind the
// kernel's speed when the part runs at its power cap.
//
// Every test runs one work-group of 8 waves (2 per SIMD, as the attention
// kernel) per CU, 120 KB of LDS each, repeatedly for a few seconds; a host
// thread samples the board's power from hwmon (power1_input, microwatts)
// every 100 ms and the test reports the median of the samples after its
// first 30 % (the sensor updates about once a second).  Cycles per step come
// from s_memtime, the clock from s_memtime over s_memrealtime (100 MHz).
// Operands change from instruction to instruction (pseudo-random bits,
// fp16 halves kept finite), since switching activity sets the energy.
// Tests (per wave and step):
//   idle           s_sleep: the clocks run, nothing issues
//   mfma_*         8 MFMAs on 4 accumulators, operands from 8 register sets:
//                  i32_32x32x32_i8, f32_32x32x16_f16 (the attention's QK and
//                  P.V), their 16x16 forms, and the e4m3 32x32x64 of FP8 P.V
//   v_fma_f32      16 independent accumulating FMAs
//   v_exp_f32      16 exps (their inputs settle to a fixed point: a lower bound)
//   v_pk_add_f16   16 packed adds
//   ds_read_b128   24 reads of 16 bytes per lane, conflict-free
//   ds_read_b64    24 reads of 8 bytes per lane
//   pipeline       one iteration of the attention loop's data flow without
//                  global memory (as issue_model.hip's pipeline test)
//   pipeline64     the same data flow with 64 query rows per wave and one
//                  wave per SIMD (4-wave work-groups; issue_model.hip's
//                  pipeline64): half the LDS operand bytes per block
//   pipeline16     the pipeline's data flow on the 16x16 MFMA shapes
//                  (i32_16x16x64_i8, f32_16x16x32_f16): the wave's 32 rows
//                  as two groups of 16, each LDS operand read feeding both
//                  groups' MFMAs, so the same LDS bytes and twice the MFMAs
// Output: one JSON line per test (cycles per step, clock, board watts,
// instructions of the class per second on the device).
//
// usage: power_model [seconds per test] [name prefix]
//                                             run the tests (default 3 s; with
//                                             a prefix, only the tests whose
//                                             name starts with it, and idle)
//        power_model --sample SECONDS         print the board power every 100 ms
//                                             (no GPU use: for timing another program)
#include <hip/hip_runtime.h>
#include <glob.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

#define CHECK(x)                                                                            \
  do {                                                                                      \
    hipError_t e_ = (x);                                                                    \
    if (e_ != hipSuccess) {                                                                 \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                         \
    }                                                                                       \
  } while (0)

constexpr int kLds = 120 * 1024;
enum Test { kIdle, kMfmaI8, kMfmaF16, kMfmaI8s, kMfmaF16s, kMfmaF8, kFma, kExp, kPkAdd, kLds128, kLds64, kPipeline,
            kPipeline64, kPipeline16 };
static const char* kName[] = {"idle(s_sleep)",
                              "mfma_i32_32x32x32_i8",
                              "mfma_f32_32x32x16_f16",
                              "mfma_i32_16x16x64_i8",
                              "mfma_f32_16x16x32_f16",
                              "mfma_scale_f32_32x32x64_f8f6f4(e4m3)",
                              "v_fma_f32",
                              "v_exp_f32",
                              "v_pk_add_f16",
                              "ds_read_b128",
                              "ds_read_b64",
                              "pipeline(attention iteration)",
                              "pipeline64(64 rows per wave, 1 wave per SIMD)",
                              "pipeline16(16x16 MFMA shapes)"};
// instructions of the measured class per wave and step
static const int kPerStep[] = {0, 8, 8, 8, 8, 8, 16, 16, 16, 24, 24, 24, 48, 48};
// steps per launch: 5-15 ms each
static const int kStepsPerLaunch[] = {20000, 60000, 60000, 60000, 60000, 30000, 60000, 60000, 60000, 25000, 25000, 8000,
                                      4000, 8000};

template <int T>
__global__ __launch_bounds__(512) void probe(long long* out, float* sink, int steps, float seed) {
  __shared__ __attribute__((aligned(16))) char lds[kLds];
  const int tid = threadIdx.x, lane = tid & 63;
  // random bits whose fp16 halves are finite (|x| < 2^15)
  for (int i = tid; i < kLds / 4; i += blockDim.x)
    reinterpret_cast<uint32_t*>(lds)[i] = ((i * 2654435761u) ^ 0x5bd1e995u) & 0xBBFFBBFFu;
  __syncthreads();
  // 8 operand sets of pseudo-random bits per lane
  constexpr bool kHalves = T == kMfmaF16 || T == kMfmaF16s;
  v4i op[8];
  for (int k = 0; k < 8; ++k)
    for (int e = 0; e < 4; ++e) {
      uint32_t x = (uint32_t)(lane * 131 + k * 17 + e * 7 + 1) * 2654435761u;
      x ^= x >> 13;
      x *= 0x85ebca6bu;
      op[k][e] = (int)(kHalves ? x & 0xBBFFBBFFu : T == kMfmaF8 ? x & 0x77777777u : x);  // e4m3: no NaN codes
    }
  v16f c[4] = {};
  v16i ci[4] = {};
  v4f cs[4] = {};
  v4i cis[4] = {};
  float r[32];
  for (int i = 0; i < 32; ++i) r[i] = seed * 1e-3f * (i + 1) + 1e-3f * lane;
  uint32_t u[32];
  for (int i = 0; i < 32; ++i) u[i] = (uint32_t)(lane * 977 + i * 313) * 2654435761u & 0x3BFF3BFFu;
  v4i acc4 = {0, 0, 0, 0};
  // pipeline state
  const int magic = 0x4B400000;
  v16i Sa[2], Sb[2];
  uint32_t Pa[16], Pb[16];
  for (int t = 0; t < 2; ++t)
    for (int v = 0; v < 16; ++v) {
      Sa[t][v] = magic + v * 37 + lane;
      Sb[t][v] = magic - v * 41 - lane;
    }
  for (int w = 0; w < 16; ++w) {
    Pa[w] = 0x3C003C00u ^ (uint32_t)(lane * w);
    Pb[w] = 0x3C003C01u ^ (uint32_t)(lane + w);
  }
  float lsum = 0.0f;
  const float csc = 1e-4f * seed, bias = 12582912.0f * csc;
  const int koff = lane * 16, voff = 8192 + lane * 16;
  // one attention iteration: 16 P.V MFMAs (A from LDS, B = P of the previous
  // step), 8 QK MFMAs (A from LDS, B = Q registers) into the other S buffer,
  // the softmax of the current S (32 FMA, 32 exp, 16 cvt, 15 packed adds),
  // a barrier; the LDS base moves over four 24 KB slots
  auto iter = [&](const uint32_t (&Pp)[16], const v16i (&Sc)[2], uint32_t (&Pc)[16], v16i (&Sn)[2], int it)
                  __attribute__((always_inline)) {
    const int base = (it & 3) * 24576;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const v4i va = *reinterpret_cast<const v4i*>(lds + base + voff + 1024 * (4 * dt + kk));
        const v4i pb = {(int)Pp[4 * kk], (int)Pp[4 * kk + 1], (int)Pp[4 * kk + 2], (int)Pp[4 * kk + 3]};
        c[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, va), __builtin_bit_cast(v8h, pb),
                                                       c[dt], 0, 0, 0);
      }
    const v16i mg = {magic, magic, magic, magic, magic, magic, magic, magic,
                     magic, magic, magic, magic, magic, magic, magic, magic};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const v4i ka = *reinterpret_cast<const v4i*>(lds + base + koff + 1024 * (4 * t + k));
        Sn[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka, op[k], k == 0 ? mg : Sn[t], 0, 0, 0);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float p[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(Sc[t][v]), csc, -bias));
#pragma unroll
      for (int w = 0; w < 8; ++w)
        Pc[8 * t + w] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){p[2 * w], p[2 * w + 1]}, h2));
    }
    h2 hs[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) hs[w] = __builtin_bit_cast(h2, Pc[w]) + __builtin_bit_cast(h2, Pc[8 + w]);
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
      for (int i = 0; i < w; ++i) hs[i] = hs[i] + hs[i + w];
    lsum = __builtin_amdgcn_fdot2(hs[0], (h2){(_Float16)1.0f, (_Float16)1.0f}, lsum, false);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // 16x16 pipeline state: O as [D chunk of 16][row group], S as [key chunk
  // of 16][row group], P as [32-key chunk][row group][4 words]
  v4f o16[16] = {};
  v4i S16a[8], S16b[8];
  uint32_t P16a[16], P16b[16];
  float lsum16[2] = {0.0f, 0.0f};
  if constexpr (T == kPipeline16) {
    for (int j = 0; j < 8; ++j)
      for (int v = 0; v < 4; ++v) {
        S16a[j][v] = magic + (4 * j + v) * 37 + lane;
        S16b[j][v] = magic - (4 * j + v) * 41 - lane;
      }
    for (int w = 0; w < 16; ++w) {
      P16a[w] = Pa[w];
      P16b[w] = Pb[w];
    }
  }
  // one attention iteration on the 16x16 shapes: 32 P.V MFMAs (A = a 16 D x
  // 32 key V fragment from LDS, shared by both row groups; B = P), 16 QK MFMAs
  // (A = a 16 key x 64 D K fragment from LDS, shared by both row groups; B =
  // Q registers) into the other S buffer, the softmax of the current S (32
  // FMA, 32 exp, 16 cvt, 14 packed adds, 2 dot2), a barrier
  auto iter16 = [&](const uint32_t (&Pp)[16], const v4i (&Sc)[8], uint32_t (&Pc)[16], v4i (&Sn)[8], int it)
                    __attribute__((always_inline)) {
    const int base = (it & 3) * 24576;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const v4i va = *reinterpret_cast<const v4i*>(lds + base + voff + 1024 * (2 * dt + kk));
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const v4i pb = {(int)Pp[8 * kk + 4 * g], (int)Pp[8 * kk + 4 * g + 1], (int)Pp[8 * kk + 4 * g + 2],
                          (int)Pp[8 * kk + 4 * g + 3]};
          o16[2 * dt + g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, va),
                                                                   __builtin_bit_cast(v8h, pb), o16[2 * dt + g], 0, 0, 0);
        }
      }
    const v4i mg4 = {magic, magic, magic, magic};
#pragma unroll
    for (int dc = 0; dc < 2; ++dc)
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const v4i ka = *reinterpret_cast<const v4i*>(lds + base + koff + 1024 * (2 * kc + dc));
#pragma unroll
        for (int g = 0; g < 2; ++g)
          Sn[2 * kc + g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, op[2 * g + dc], dc == 0 ? mg4 : Sn[2 * kc + g], 0, 0, 0);
      }
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        float p[8];
#pragma unroll
        for (int v = 0; v < 8; ++v)
          p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(Sc[2 * (2 * kk + v / 4) + g][v & 3]), csc, -bias));
#pragma unroll
        for (int w = 0; w < 4; ++w)
          Pc[8 * kk + 4 * g + w] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){p[2 * w], p[2 * w + 1]}, h2));
      }
      h2 hs[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) hs[w] = __builtin_bit_cast(h2, Pc[4 * g + w]) + __builtin_bit_cast(h2, Pc[8 + 4 * g + w]);
      hs[0] = hs[0] + hs[2];
      hs[1] = hs[1] + hs[3];
      hs[0] = hs[0] + hs[1];
      lsum16[g] = __builtin_amdgcn_fdot2(hs[0], (h2){(_Float16)1.0f, (_Float16)1.0f}, lsum16[g], false);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  const long long t0 = __builtin_amdgcn_s_memtime();
  const long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < steps; ++it) {
    if constexpr (T == kIdle) {
      __builtin_amdgcn_s_sleep(8);
    } else if constexpr (T == kMfmaI8) {
#pragma unroll
      for (int m = 0; m < 8; ++m)
        ci[m & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(op[m], op[(m + 3) & 7], ci[m & 3], 0, 0, 0);
    } else if constexpr (T == kMfmaF16) {
#pragma unroll
      for (int m = 0; m < 8; ++m)
        c[m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, op[m]),
                                                          __builtin_bit_cast(v8h, op[(m + 3) & 7]), c[m & 3], 0, 0, 0);
    } else if constexpr (T == kMfmaI8s) {
#pragma unroll
      for (int m = 0; m < 8; ++m)
        cis[m & 3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(op[m], op[(m + 3) & 7], cis[m & 3], 0, 0, 0);
    } else if constexpr (T == kMfmaF16s) {
#pragma unroll
      for (int m = 0; m < 8; ++m)
        cs[m & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, op[m]),
                                                           __builtin_bit_cast(v8h, op[(m + 3) & 7]), cs[m & 3], 0, 0, 0);
    } else if constexpr (T == kMfmaF8) {  // unit scales (127: 2^0), as the FP8 P.V MFMA
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const v4i x = op[m], y = op[(m + 1) & 7], z = op[(m + 3) & 7], w = op[(m + 5) & 7];
        const v8i a8 = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
        const v8i b8 = {z[0], z[1], z[2], z[3], w[0], w[1], w[2], w[3]};
        c[m & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c[m & 3], 0, 0, 0, 127, 0, 127);
      }
    } else if constexpr (T == kFma) {
#pragma unroll
      for (int i = 0; i < 16; ++i) r[i] = __builtin_fmaf(r[i + 16], r[16 + ((i + 5) & 15)], r[i]);
    } else if constexpr (T == kExp) {
#pragma unroll
      for (int i = 0; i < 16; ++i) r[i] = __builtin_amdgcn_exp2f(r[i] - r[i + 16]);
    } else if constexpr (T == kPkAdd) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        u[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, u[i]) + __builtin_bit_cast(h2, u[i + 16]));
    } else if constexpr (T == kLds128) {
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        v4i x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          x[i] = *reinterpret_cast<const v4i*>(lds + (((tid >> 6) * 8 + g * 8 + i + it) & 63) * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc4 ^= x[i];
      }
    } else if constexpr (T == kLds64) {
      v2i a2 = {0, 0};
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        v2i x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          x[i] = *reinterpret_cast<const v2i*>(lds + (((tid >> 6) * 8 + g * 8 + i + it) & 63) * 1024 + lane * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) a2 ^= x[i];
      }
      acc4.x ^= a2.x;
      acc4.y ^= a2.y;
    } else if constexpr (T == kPipeline16) {  // as below, on the 16x16 shapes
      iter16(P16a, S16a, P16b, S16b, it);
      iter16(P16b, S16b, P16a, S16a, it + 1);
      ++it;
    } else {  // two iterations per trip swap the S and P buffers (steps iterations in all)
      iter(Pa, Sa, Pb, Sb, it);
      iter(Pb, Sb, Pa, Sa, it + 1);
      ++it;
    }
  }
  const long long t1 = __builtin_amdgcn_s_memtime();
  const long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = lsum + (float)(acc4.x ^ acc4.y ^ acc4.z ^ acc4.w);
  for (int i = 0; i < 32; ++i) s += r[i] + (float)(u[i] & 0xFF);
  for (int q = 0; q < 4; ++q) {
    for (int i = 0; i < 16; ++i) s += c[q][i] + (float)ci[q][i];
    for (int i = 0; i < 4; ++i) s += cs[q][i] + (float)cis[q][i];
  }
  for (int i = 0; i < 16; ++i) s += (float)(Sa[0][i] + Sb[1][i]) + (float)(Pa[i] ^ Pb[i]);
  if constexpr (T == kPipeline16) {
    s += lsum16[0] + lsum16[1];
    for (int j = 0; j < 16; ++j) s += o16[j][0] + o16[j][3] + (float)(P16a[j] ^ P16b[j]);
    for (int j = 0; j < 8; ++j) s += (float)(S16a[j][1] + S16b[j][2]);
  }
  sink[blockIdx.x * blockDim.x + tid] = s;
  if (lane == 0) {
    long long* o = out + (blockIdx.x * (blockDim.x >> 6) + (tid >> 6)) * 4;
    o[0] = t0;
    o[1] = t1;
    o[2] = r0;
    o[3] = r1;
  }
}

// 64 query rows per wave, one wave per SIMD (4 waves per work-group): the
// wave's halves h = 0, 1 of 32 rows, half 0 one block ahead.  Phase X: P.V of
// half 0 (block i) and QK of half 1 (block i+1) while the VALU forms half 1's
// P (block i); phase Y: P.V of half 1 and QK of half 0 (block i+2) while it
// forms half 0's P (block i+1).  Each LDS operand read feeds two MFMAs.
// A step is one block of 64 keys for the wave's 64 rows.
__global__ __launch_bounds__(256) void probe64(long long* out, float* sink, int steps, float seed) {
  __shared__ __attribute__((aligned(16))) char lds[kLds];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < kLds / 4; i += blockDim.x)
    reinterpret_cast<uint32_t*>(lds)[i] = ((i * 2654435761u) ^ 0x5bd1e995u) & 0xBBFFBBFFu;
  __syncthreads();
  v16f o0[4] = {}, o1[4] = {};
  v4i q0[4], q1[4];
  for (int k = 0; k < 4; ++k)
    for (int e = 0; e < 4; ++e) {
      q0[k][e] = (int)((uint32_t)(lane * 131 + k * 17 + e * 7 + 1) * 2654435761u);
      q1[k][e] = (int)((uint32_t)(lane * 137 + k * 19 + e * 5 + 3) * 2654435761u);
    }
  const int magic = 0x4B400000;
  v16i S0a[2], S0b[2], S1a[2], S1b[2];
  uint32_t P0[16], P1[16];
  for (int t = 0; t < 2; ++t)
    for (int v = 0; v < 16; ++v) {
      S0a[t][v] = magic + v * 37 + lane;
      S0b[t][v] = magic - v * 41 - lane;
      S1a[t][v] = magic + v * 43 + 2 * lane;
      S1b[t][v] = magic - v * 47 - 2 * lane;
    }
  for (int w = 0; w < 16; ++w) {
    P0[w] = 0x3C003C00u ^ (uint32_t)(lane * w);
    P1[w] = 0x3C003C01u ^ (uint32_t)(lane + w);
  }
  float l0 = 0.0f, l1 = 0.0f;
  const float csc = 1e-4f * seed, bias = 12582912.0f * csc;
  const int koff = lane * 16, voff = 8192 + lane * 16;
  const v16i mg = {magic, magic, magic, magic, magic, magic, magic, magic,
                   magic, magic, magic, magic, magic, magic, magic, magic};
  // 16 P.V MFMAs into o with P pv, 8 QK MFMAs of q into sq, the softmax of ss
  auto phase = [&](v16f (&o)[4], const uint32_t (&pv)[16], const v4i (&q)[4], v16i (&sq)[2], const v16i (&ss)[2],
                   uint32_t (&pout)[16], float& lsum, int kofs, int vofs) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const v4i va = *reinterpret_cast<const v4i*>(lds + vofs + voff + 1024 * (4 * dt + kk));
        const v4i pb = {(int)pv[4 * kk], (int)pv[4 * kk + 1], (int)pv[4 * kk + 2], (int)pv[4 * kk + 3]};
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, va), __builtin_bit_cast(v8h, pb),
                                                       o[dt], 0, 0, 0);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const v4i ka = *reinterpret_cast<const v4i*>(lds + kofs + koff + 1024 * (4 * t + k));
        sq[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka, q[k], k == 0 ? mg : sq[t], 0, 0, 0);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float p[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(ss[t][v]), csc, -bias));
#pragma unroll
      for (int w = 0; w < 8; ++w)
        pout[8 * t + w] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){p[2 * w], p[2 * w + 1]}, h2));
    }
    h2 hs[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) hs[w] = __builtin_bit_cast(h2, pout[w]) + __builtin_bit_cast(h2, pout[8 + w]);
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
      for (int i = 0; i < w; ++i) hs[i] = hs[i] + hs[i + w];
    lsum = __builtin_amdgcn_fdot2(hs[0], (h2){(_Float16)1.0f, (_Float16)1.0f}, lsum, false);
  };
  auto iter = [&](v16i (&S0c)[2], v16i (&S0n)[2], v16i (&S1c)[2], v16i (&S1n)[2], int it)
                  __attribute__((always_inline)) {
    const int s0 = (it % 3) * 24576, s1 = ((it + 1) % 3) * 24576, s2 = ((it + 2) % 3) * 24576;
    phase(o0, P0, q1, S1n, S1c, P1, l1, s1, s0);  // X: PV_0(i), QK_1(i+1), SM_1(i)
    phase(o1, P1, q0, S0n, S0c, P0, l0, s2, s0);  // Y: PV_1(i), QK_0(i+2), SM_0(i+1)
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  const long long t0 = __builtin_amdgcn_s_memtime();
  const long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < steps; it += 2) {
    iter(S0a, S0b, S1a, S1b, it);
    iter(S0b, S0a, S1b, S1a, it + 1);
  }
  const long long t1 = __builtin_amdgcn_s_memtime();
  const long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = l0 + l1;
  for (int q = 0; q < 4; ++q)
    for (int i = 0; i < 16; ++i) s += o0[q][i] + o1[q][i];
  for (int i = 0; i < 16; ++i) s += (float)(S0a[0][i] + S1b[1][i]) + (float)(P0[i] ^ P1[i]);
  sink[blockIdx.x * blockDim.x + tid] = s;
  if (lane == 0) {
    long long* o = out + (blockIdx.x * (blockDim.x >> 6) + (tid >> 6)) * 4;
    o[0] = t0;
    o[1] = t1;
    o[2] = r0;
    o[3] = r1;
  }
}

// the board's power sensor (hwmon of the GPU's DRM device), first one that reads
static std::string power_file() {
  for (const char* pat : {"/sys/class/drm/card*/device/hwmon/hwmon*/power1_input",
                          "/sys/class/drm/card*/device/hwmon/hwmon*/power1_average"}) {
    glob_t g;
    std::string found;
    if (glob(pat, 0, nullptr, &g) == 0)
      for (size_t i = 0; i < g.gl_pathc && found.empty(); ++i) {
        FILE* p = std::fopen(g.gl_pathv[i], "r");
        long long uw = -1;
        if (p) {
          if (std::fscanf(p, "%lld", &uw) != 1) uw = -1;
          std::fclose(p);
        }
        if (uw > 0) found = g.gl_pathv[i];
      }
    globfree(&g);
    if (!found.empty()) return found;
  }
  return "";
}

static double read_watts(const std::string& f) {
  FILE* p = std::fopen(f.c_str(), "r");
  if (!p) return -1.0;
  long long uw = -1;
  if (std::fscanf(p, "%lld", &uw) != 1) uw = -1;
  std::fclose(p);
  return uw < 0 ? -1.0 : uw * 1e-6;
}

static double now_s() {
  return std::chrono::duration<double>(std::chrono::system_clock::now().time_since_epoch()).count();
}

template <int T>
static void launch(int cus, long long* d, float* sink, int steps) {
  if constexpr (T == kPipeline64) hipLaunchKernelGGL(probe64, dim3(cus), dim3(256), 0, 0, d, sink, steps, 1.0f);
  else hipLaunchKernelGGL((probe<T>), dim3(cus), dim3(512), 0, 0, d, sink, steps, 1.0f);
}

template <int T>
static void run(int cus, double seconds, const std::string& pf, long long* d, float* sink, const char* only) {
  if (only && T != kIdle && std::strncmp(kName[T], only, std::strlen(only)) != 0) return;
  const int waves = T == kPipeline64 ? 4 : 8, nw = cus * waves;
  const int steps = kStepsPerLaunch[T];
  launch<T>(cus, d, sink, 64);
  CHECK(hipDeviceSynchronize());
  std::atomic<bool> stop{false};
  std::vector<double> samples;
  std::thread sampler([&] {
    while (!stop.load()) {
      std::this_thread::sleep_for(std::chrono::milliseconds(100));
      if (!pf.empty()) samples.push_back(read_watts(pf));
    }
  });
  const auto tstart = std::chrono::steady_clock::now();
  const double wall0 = now_s();
  int launches = 0;
  std::vector<double> cyc, clk;
  std::vector<long long> h(4 * nw);
  while (std::chrono::duration<double>(std::chrono::steady_clock::now() - tstart).count() < seconds) {
    for (int k = 0; k < 8; ++k) launch<T>(cus, d, sink, steps);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    launches += 8;
    CHECK(hipMemcpy(h.data(), d, sizeof(long long) * 4 * nw, hipMemcpyDeviceToHost));
    for (int w = 0; w < nw; w += 7) {
      const double c = (double)(h[4 * w + 1] - h[4 * w]), r = (double)(h[4 * w + 3] - h[4 * w + 2]);
      cyc.push_back(c / steps);
      clk.push_back(c / r * 0.1);
    }
  }
  const double wall1 = now_s();
  stop = true;
  sampler.join();
  std::sort(cyc.begin(), cyc.end());
  std::sort(clk.begin(), clk.end());
  double pw = -1.0;
  if (samples.size() > 4) {
    std::vector<double> s(samples.begin() + samples.size() * 3 / 10, samples.end());
    std::sort(s.begin(), s.end());
    pw = s[s.size() / 2];
  }
  const double cps = cyc[cyc.size() / 2], ghz = clk[clk.size() / 2];
  const double ips = kPerStep[T] > 0 ? (double)kPerStep[T] * nw / (cps / (ghz * 1e9)) : 0.0;
  std::printf("{\"test\": \"%s\", \"cycles_per_step\": %.1f, \"clock_ghz\": %.3f, \"board_w\": %.1f, "
              "\"insts_per_s\": %.4e, \"launches\": %d, \"t0\": %.3f, \"t1\": %.3f}\n",
              kName[T], cps, ghz, pw, ips, launches, wall0, wall1);
  std::fflush(stdout);
}

int main(int argc, char** argv) {
  const std::string pf = power_file();
  if (argc > 2 && std::strcmp(argv[1], "--sample") == 0) {
    const double secs = std::atof(argv[2]);
    const double t0 = now_s();
    std::printf("{\"power_file\": \"%s\"}\n", pf.c_str());
    while (now_s() - t0 < secs) {
      std::printf("%.3f %.1f\n", now_s(), pf.empty() ? -1.0 : read_watts(pf));
      std::fflush(stdout);
      std::this_thread::sleep_for(std::chrono::milliseconds(100));
    }
    return 0;
  }
  const double secs = argc > 1 ? std::atof(argv[1]) : 3.0;
  const char* only = argc > 2 ? argv[2] : nullptr;
  hipDeviceProp_t p;
  CHECK(hipGetDeviceProperties(&p, 0));
  std::printf("{\"device\": \"%s\", \"arch\": \"%s\", \"compute_units\": %d, \"power_file\": \"%s\", \"watts_now\": %.1f}\n",
              p.name, p.gcnArchName, p.multiProcessorCount, pf.c_str(), pf.empty() ? -1.0 : read_watts(pf));
  std::fflush(stdout);
  const int cus = p.multiProcessorCount;
  long long* d;
  float* sink;
  CHECK(hipMalloc(&d, sizeof(long long) * 4 * cus * 8));
  CHECK(hipMalloc(&sink, sizeof(float) * cus * 512));
  run<kIdle>(cus, secs, pf, d, sink, only);
  run<kMfmaI8>(cus, secs, pf, d, sink, only);
  run<kMfmaF16>(cus, secs, pf, d, sink, only);
  run<kMfmaI8s>(cus, secs, pf, d, sink, only);
  run<kMfmaF16s>(cus, secs, pf, d, sink, only);
  run<kMfmaF8>(cus, secs, pf, d, sink, only);
  run<kFma>(cus, secs, pf, d, sink, only);
  run<kExp>(cus, secs, pf, d, sink, only);
  run<kPkAdd>(cus, secs, pf, d, sink, only);
  run<kLds128>(cus, secs, pf, d, sink, only);
  run<kLds64>(cus, secs, pf, d, sink, only);
  run<kPipeline>(cus, secs, pf, d, sink, only);
  run<kPipeline64>(cus, secs, pf, d, sink, only);
  run<kPipeline16>(cus, secs, pf, d, sink, only);
  run<kIdle>(cus, secs, pf, d, sink, only);
  CHECK(hipFree(d));
  CHECK(hipFree(sink));
  return 0;
}
