// mfma_peak.hip — MFMA-only throughput of the GPU: the measured side of the
// dense peaks that the roofline figures divide by (tribench_amd/harness/metrics.py).
//
// For each MFMA form the attention kernels use, every CU runs one work-group
// (96 KB of LDS keeps it to one per CU) of 4 or 8 waves (1 or 2 per SIMD);
// each wave issues ITERS x 8 MFMAs on 4 independent accumulators and nothing
// else.  Reported per form, as one JSON line:
//   cycles_per_mfma   s_memtime cycles per MFMA per SIMD (median wave)
//   clock_ghz         shader clock during the run: s_memtime ticks over the
//                     100 MHz s_memrealtime ticks (median wave)
//   ops_per_clk_cu    ops per clock per CU implied by cycles_per_mfma
//   tops_measured     ops of the whole launch / its wall time (hipEvents)
//   tops_at_max_clock ops_per_clk_cu x CUs x the device's maximum clock
// A short warm-up launch precedes each timed one.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define CHECK(x)                                                                            \
  do {                                                                                      \
    hipError_t e_ = (x);                                                                    \
    if (e_ != hipSuccess) {                                                                 \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                         \
    }                                                                                       \
  } while (0)

enum Form { kI8 = 0, kF16 = 1, kBF16 = 2, kF8 = 3 };
static const char* kName[] = {"i8 v_mfma_i32_32x32x32_i8", "f16 v_mfma_f32_32x32x16_f16",
                              "bf16 v_mfma_f32_32x32x16_bf16", "fp8 v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3)"};
static const double kOps[] = {2.0 * 32 * 32 * 32, 2.0 * 32 * 32 * 16, 2.0 * 32 * 32 * 16, 2.0 * 32 * 32 * 64};

template <int F>
__global__ __launch_bounds__(512) void mfma_only(long long* stamps, float* sink, int iters, int seed) {
  __shared__ char pad[96 * 1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  pad[threadIdx.x] = (char)seed;
  __syncthreads();
  const int s = seed + lane;
  v16f c[4] = {};
  v16i ci[4] = {};
  const v4i a4 = {s, s + 1, s + 2, s + 3};
  const v8i a8 = {s, s + 1, s + 2, s + 3, s + 4, s + 5, s + 6, s + 7};
  const v8h ah = __builtin_bit_cast(v8h, a4);
  const v8bf ab = __builtin_bit_cast(v8bf, a4);
  const long long t0 = __builtin_amdgcn_s_memtime();
  const long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if constexpr (F == kI8) ci[m & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, a4, ci[m & 3], 0, 0, 0);
      if constexpr (F == kF16) c[m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ah, c[m & 3], 0, 0, 0);
      if constexpr (F == kBF16) c[m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ab, ab, c[m & 3], 0, 0, 0);
      if constexpr (F == kF8)
        c[m & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, a8, c[m & 3], 0, 0, 0, 127, 0, 127);
    }
  }
  const long long t1 = __builtin_amdgcn_s_memtime();
  const long long r1 = __builtin_amdgcn_s_memrealtime();
  float acc = 0.0f;
  for (int q = 0; q < 4; ++q)
    for (int i = 0; i < 16; ++i) acc += c[q][i] + (float)ci[q][i];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = acc + pad[threadIdx.x];
  if (lane == 0) {
    long long* o = stamps + (blockIdx.x * (blockDim.x >> 6) + wave) * 4;
    o[0] = t0;
    o[1] = t1;
    o[2] = r0;
    o[3] = r1;
  }
}

template <int F>
static void run(int cus, int waves, int iters, double max_clock_ghz) {
  const int threads = 64 * waves;
  const int nw = cus * waves;
  long long* stamps;
  float* sink;
  CHECK(hipMalloc(&stamps, sizeof(long long) * 4 * nw));
  CHECK(hipMalloc(&sink, sizeof(float) * cus * threads));
  hipLaunchKernelGGL(mfma_only<F>, dim3(cus), dim3(threads), 0, 0, stamps, sink, iters / 10, 1);
  CHECK(hipGetLastError());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0, 0));
  hipLaunchKernelGGL(mfma_only<F>, dim3(cus), dim3(threads), 0, 0, stamps, sink, iters, 1);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1, 0));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  std::vector<long long> h(4 * nw);
  CHECK(hipMemcpy(h.data(), stamps, sizeof(long long) * 4 * nw, hipMemcpyDeviceToHost));
  std::vector<double> cyc, clk;
  for (int w = 0; w < nw; ++w) {
    const double c = (double)(h[4 * w + 1] - h[4 * w]), r = (double)(h[4 * w + 3] - h[4 * w + 2]);
    cyc.push_back(c / (8.0 * iters) / (waves / 4));  // per MFMA per SIMD (waves/4 waves share a SIMD)
    clk.push_back(c / r * 0.1);
  }
  std::sort(cyc.begin(), cyc.end());
  std::sort(clk.begin(), clk.end());
  const double cpm = cyc[cyc.size() / 2], ghz = clk[clk.size() / 2];
  const double ops = kOps[F] * 8.0 * iters * nw;
  const double per_clk_cu = kOps[F] / cpm * 4.0;  // 4 SIMDs per CU
  std::printf("{\"mfma\": \"%s\", \"waves_per_simd\": %d, \"ops_per_mfma\": %.0f, \"cycles_per_mfma\": %.2f, "
              "\"clock_ghz\": %.3f, \"ops_per_clk_cu\": %.0f, \"tops_measured\": %.1f, "
              "\"tops_at_measured_clock\": %.1f, \"tops_at_max_clock\": %.1f, \"wall_ms\": %.3f}\n",
              kName[F], waves / 4, kOps[F], cpm, ghz, per_clk_cu, ops / (ms * 1e-3) / 1e12,
              per_clk_cu * cus * ghz * 1e9 / 1e12, per_clk_cu * cus * max_clock_ghz * 1e9 / 1e12, ms);
  std::fflush(stdout);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  CHECK(hipFree(stamps));
  CHECK(hipFree(sink));
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
  hipDeviceProp_t p;
  CHECK(hipGetDeviceProperties(&p, 0));
  const int cus = p.multiProcessorCount;
  const double max_clock_ghz = p.clockRate * 1e-6;  // clockRate is in kHz
  std::printf("{\"device\": \"%s\", \"arch\": \"%s\", \"compute_units\": %d, \"max_clock_ghz\": %.3f}\n", p.name,
              p.gcnArchName, cus, max_clock_ghz);
  for (int waves : {4, 8}) {
    run<kI8>(cus, waves, iters, max_clock_ghz);
    run<kF16>(cus, waves, iters, max_clock_ghz);
    run<kBF16>(cus, waves, iters, max_clock_ghz);
    run<kF8>(cus, waves, iters, max_clock_ghz);
  }
  return 0;
}
