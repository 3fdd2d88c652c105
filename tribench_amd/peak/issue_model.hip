// issue_model.hip — how a gfx950 SIMD overlaps the instruction mix of the
// attention kernel's inner loop: the measurements its design rests on.
//
// Every test runs one work-group per CU (96-120 KB of LDS keeps it to one)
// of 4 or 8 waves (1 or 2 per SIMD) and times each wave with s_memtime;
// the clock comes from s_memtime over s_memrealtime (100 MHz).  Each prints
// one JSON line: cycles per step (the median and the slowest wave) and the
// clock.  Tests:
//   mfma        8 MFMAs (32x32x16 f16) on 4 accumulators per step
//   fma, exp    16 independent v_fma_f32 / v_exp_f32 per step
//   mix         one 64-key block of the attention loop without memory:
//               24 MFMAs, NF FMAs and 32 exps, evenly interleaved
//   lds         24 ds_read_b128 per step (lane-contiguous, conflict-free)
//   pipeline    the loop's data flow per step: 16 P.V MFMAs (A operand from
//               LDS, B = P of the previous step), 8 QK MFMAs (A from LDS,
//               B = Q registers) into a second S buffer, the softmax of the
//               current S (32 FMA, 32 exp, 16 cvt, 15 packed adds), a
//               work-group barrier
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
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

constexpr int kSteps = 512;
constexpr int kLds = 120 * 1024;
enum Test { kMfma, kFma, kExp, kMix, kLdsRead, kPipeline };

__device__ __forceinline__ void stamp(long long* out, long long t0, long long t1, long long r0, long long r1) {
  if ((threadIdx.x & 63) == 0) {
    long long* o = out + (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4;
    o[0] = t0;
    o[1] = t1;
    o[2] = r0;
    o[3] = r1;
  }
}

template <int T, int NF>
__global__ __launch_bounds__(512) void probe(long long* out, float* sink, float seed) {
  __shared__ __attribute__((aligned(16))) char lds[kLds];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < kLds / 4; i += blockDim.x) reinterpret_cast<int*>(lds)[i] = (i * 2654435761u) & 0x3F3F3F3F;
  __syncthreads();
  const v8h a = {(_Float16)seed, (_Float16)1, (_Float16)2, (_Float16)3, (_Float16)4, (_Float16)5, (_Float16)6,
                 (_Float16)(lane & 7)};
  v16f c[4] = {};
  float r[32];
  for (int i = 0; i < 32; ++i) r[i] = seed * 1e-3f * (i + 1) + 1e-3f * lane;
  v4i acc4 = {0, 0, 0, 0};
  // pipeline state
  v4i qreg[4];
  for (int k = 0; k < 4; ++k) qreg[k] = (v4i){lane + k, 3, 5, 7} & 0x3F;
  const int magic = 0x4B400000;
  v16i Sa[2], Sb[2];
  uint32_t Pa[16], Pb[16];
  for (int t = 0; t < 2; ++t)
    for (int v = 0; v < 16; ++v) {
      Sa[t][v] = magic + v;
      Sb[t][v] = magic - v;
    }
  for (int w = 0; w < 16; ++w) {
    Pa[w] = 0x3C003C00u;
    Pb[w] = 0x3C003C01u;
  }
  float lsum = 0.0f;
  const float cs = 1e-3f * seed, bias = 12582912.0f * cs;
  const int koff = lane * 16, voff = 8192 + lane * 16;

  auto iter = [&](const uint32_t (&Pp)[16], const v16i (&Sc)[2], uint32_t (&Pc)[16], v16i (&Sn)[2])
                  __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const v4i va = *reinterpret_cast<const v4i*>(lds + voff + 1024 * (4 * dt + kk));
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
        const v4i ka = *reinterpret_cast<const v4i*>(lds + koff + 1024 * (4 * t + k));
        Sn[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka, qreg[k], k == 0 ? mg : Sn[t], 0, 0, 0);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float p[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(Sc[t][v]), cs, -bias));
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

  const long long t0 = __builtin_amdgcn_s_memtime();
  const long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < kSteps; ++it) {
    if constexpr (T == kMfma) {
#pragma unroll
      for (int m = 0; m < 8; ++m) c[m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c[m & 3], 0, 0, 0);
    } else if constexpr (T == kFma) {
#pragma unroll
      for (int i = 0; i < 16; ++i) r[i] = __builtin_fmaf(r[i], 0.999f, 1e-4f);
    } else if constexpr (T == kExp) {
#pragma unroll
      for (int i = 0; i < 16; ++i) r[i] = __builtin_amdgcn_exp2f(r[i]);
    } else if constexpr (T == kMix) {
      // 24 MFMAs in 8 groups of 3; after each MFMA NF/24 FMAs, and 2, 1, 1
      // exps after the group's three MFMAs (32 per step)
#pragma unroll
      for (int g = 0; g < 8; ++g) {
#define SAGE_MIX_STEP(m, NE)                                                                                  \
  c[(3 * g + m) & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c[(3 * g + m) & 3], 0, 0, 0);             \
  _Pragma("unroll") for (int x = 0; x < NF / 24; ++x) {                                                       \
    const int i = ((3 * g + m) * (NF / 24) + x) & 31;                                                         \
    r[i] = __builtin_fmaf(r[i], 0.999f, 1e-4f);                                                               \
  }                                                                                                           \
  _Pragma("unroll") for (int x = 0; x < NE; ++x) {                                                            \
    const int i = ((3 * g + m) * 2 + x + 7) & 31;                                                             \
    r[i] = __builtin_amdgcn_exp2f(r[i]);                                                                      \
  }                                                                                                           \
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                          \
  __builtin_amdgcn_sched_group_barrier(0x002, NF / 24 + NE, 0);
        SAGE_MIX_STEP(0, 2)
        SAGE_MIX_STEP(1, 1)
        SAGE_MIX_STEP(2, 1)
#undef SAGE_MIX_STEP
      }
    } else if constexpr (T == kLdsRead) {
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        v4i x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          x[i] = *reinterpret_cast<const v4i*>(lds + (((tid >> 6) * 8 + g * 8 + i + it) & 63) * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc4 ^= x[i];
      }
    } else {  // two iterations per trip swap the S and P buffers (kSteps iterations in all)
      iter(Pa, Sa, Pb, Sb);
      iter(Pb, Sb, Pa, Sa);
      ++it;
    }
  }
  const long long t1 = __builtin_amdgcn_s_memtime();
  const long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = lsum + (float)(acc4.x ^ acc4.y ^ acc4.z ^ acc4.w);
  for (int i = 0; i < 32; ++i) s += r[i];
  for (int q = 0; q < 4; ++q)
    for (int i = 0; i < 16; ++i) s += c[q][i];
  for (int i = 0; i < 16; ++i) s += (float)(Sa[0][i] + Sb[1][i]) + (float)(Pa[i] ^ Pb[i]);
  sink[blockIdx.x * blockDim.x + tid] = s;
  stamp(out, t0, t1, r0, r1);
}

template <int T, int NF = 0>
static void run(const char* name, int cus, int waves, long long* d, float* sink) {
  const int threads = 64 * waves, nw = cus * waves;
  hipLaunchKernelGGL((probe<T, NF>), dim3(cus), dim3(threads), 0, 0, d, sink, 1.0f);
  hipLaunchKernelGGL((probe<T, NF>), dim3(cus), dim3(threads), 0, 0, d, sink, 1.0f);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  std::vector<long long> h(4 * nw);
  CHECK(hipMemcpy(h.data(), d, sizeof(long long) * 4 * nw, hipMemcpyDeviceToHost));
  std::vector<double> cyc, clk;
  for (int w = 0; w < nw; ++w) {
    const double c = (double)(h[4 * w + 1] - h[4 * w]), r = (double)(h[4 * w + 3] - h[4 * w + 2]);
    cyc.push_back(c / kSteps);
    clk.push_back(c / r * 0.1);
  }
  std::sort(cyc.begin(), cyc.end());
  std::sort(clk.begin(), clk.end());
  std::printf("{\"test\": \"%s\", \"waves_per_simd\": %d, \"cycles_per_step_p50\": %.1f, "
              "\"cycles_per_step_max\": %.1f, \"clock_ghz\": %.3f}\n",
              name, waves / 4, cyc[cyc.size() / 2], cyc.back(), clk[clk.size() / 2]);
  std::fflush(stdout);
}

// The same data flow with 64 query rows per wave and one wave per SIMD (4
// waves per work-group): halves h = 0, 1 of 32 rows, half 0 one block ahead.
// Phase X: P.V of half 0 (block i) and QK of half 1 (block i+1) on the matrix
// pipe while the VALU forms half 1's P (block i); phase Y: P.V of half 1 and
// QK of half 0 (block i+2) while it forms half 0's P (block i+1).  Half the
// LDS operand reads per MFMA, and no second wave on the SIMD.
__global__ __launch_bounds__(256) void probe64(long long* out, float* sink, float seed) {
  __shared__ __attribute__((aligned(16))) char lds[kLds];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < kLds / 4; i += blockDim.x) reinterpret_cast<int*>(lds)[i] = (i * 2654435761u) & 0x3F3F3F3F;
  __syncthreads();
  v16f o0[4] = {}, o1[4] = {};
  v4i q0[4], q1[4];
  for (int k = 0; k < 4; ++k) {
    q0[k] = (v4i){lane + k, 3, 5, 7} & 0x3F;
    q1[k] = (v4i){lane + 2 * k, 1, 5, 9} & 0x3F;
  }
  const int magic = 0x4B400000;
  v16i S0a[2], S0b[2], S1a[2], S1b[2];
  uint32_t P0[16], P1[16];
  for (int t = 0; t < 2; ++t)
    for (int v = 0; v < 16; ++v) {
      S0a[t][v] = magic + v;
      S0b[t][v] = magic - v;
      S1a[t][v] = magic + 2 * v;
      S1b[t][v] = magic - 2 * v;
    }
  for (int w = 0; w < 16; ++w) {
    P0[w] = 0x3C003C00u;
    P1[w] = 0x3C003C01u;
  }
  float l0 = 0.0f, l1 = 0.0f;
  const float cs = 1e-3f * seed, bias = 12582912.0f * cs;
  const int koff = lane * 16, voff = 8192 + lane * 16;
  const v16i mg = {magic, magic, magic, magic, magic, magic, magic, magic,
                   magic, magic, magic, magic, magic, magic, magic, magic};
  // one phase: 16 PV MFMAs into o with P pv, 8 QK MFMAs of q into sq, and the
  // softmax of ss into pout (lsum)
  auto phase = [&](v16f (&o)[4], const uint32_t (&pv)[16], const v4i (&q)[4], v16i (&sq)[2],
                   const v16i (&ss)[2], uint32_t (&pout)[16], float& lsum, int kofs, int vofs)
                   __attribute__((always_inline)) {
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
      for (int v = 0; v < 16; ++v) p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(ss[t][v]), cs, -bias));
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
    const int s0 = (it % 3) * 16384, s1 = ((it + 1) % 3) * 16384, s2 = ((it + 2) % 3) * 16384;
    phase(o0, P0, q1, S1n, S1c, P1, l1, s1, s0);  // X: PV_0(i), QK_1(i+1), SM_1(i)
    phase(o1, P1, q0, S0n, S0c, P0, l0, s2, s0);  // Y: PV_1(i), QK_0(i+2), SM_0(i+1)
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  const long long t0 = __builtin_amdgcn_s_memtime();
  const long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < kSteps; it += 2) {
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
  stamp(out, t0, t1, r0, r1);
}

static void run64(const char* name, int cus, long long* d, float* sink) {
  const int waves = 4, threads = 256, nw = cus * waves;
  hipLaunchKernelGGL(probe64, dim3(cus), dim3(threads), 0, 0, d, sink, 1.0f);
  hipLaunchKernelGGL(probe64, dim3(cus), dim3(threads), 0, 0, d, sink, 1.0f);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  std::vector<long long> h(4 * nw);
  CHECK(hipMemcpy(h.data(), d, sizeof(long long) * 4 * nw, hipMemcpyDeviceToHost));
  std::vector<double> cyc, clk;
  for (int w = 0; w < nw; ++w) {
    const double c = (double)(h[4 * w + 1] - h[4 * w]), r = (double)(h[4 * w + 3] - h[4 * w + 2]);
    cyc.push_back(c / kSteps);
    clk.push_back(c / r * 0.1);
  }
  std::sort(cyc.begin(), cyc.end());
  std::sort(clk.begin(), clk.end());
  std::printf("{\"test\": \"%s\", \"waves_per_simd\": 1, \"cycles_per_step_p50\": %.1f, "
              "\"cycles_per_step_max\": %.1f, \"clock_ghz\": %.3f}\n",
              name, cyc[cyc.size() / 2], cyc.back(), clk[clk.size() / 2]);
  std::fflush(stdout);
}

int main() {
  hipDeviceProp_t p;
  CHECK(hipGetDeviceProperties(&p, 0));
  const int cus = p.multiProcessorCount;
  long long* d;
  float* sink;
  CHECK(hipMalloc(&d, sizeof(long long) * 4 * cus * 8));
  CHECK(hipMalloc(&sink, sizeof(float) * cus * 512));
  for (int waves : {4, 8}) {
    run<kMfma>("mfma: 8 x v_mfma_f32_32x32x16_f16", cus, waves, d, sink);
    run<kFma>("fma: 16 x v_fma_f32", cus, waves, d, sink);
    run<kExp>("exp: 16 x v_exp_f32", cus, waves, d, sink);
    run<kMix, 0>("mix: 24 MFMA + 32 exp", cus, waves, d, sink);
    run<kMix, 96>("mix: 24 MFMA + 96 FMA + 32 exp", cus, waves, d, sink);
    run<kLdsRead>("lds: 24 x ds_read_b128 (24 KB per wave)", cus, waves, d, sink);
  }
  run<kPipeline>("pipeline: one attention-loop iteration without global memory", cus, 8, d, sink);
  run64("pipeline64: the same with 64 rows per wave, one wave per SIMD", cus, d, sink);
  CHECK(hipFree(d));
  CHECK(hipFree(sink));
  return 0;
}
