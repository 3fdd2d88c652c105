// hbm_peak.hip — what a streaming kernel of this GPU moves through HBM per
// second: the practical ceiling that the pre-pass's bytes are compared with
// (the published 8 TB/s is the interface's rate, not what kernels reach).
//
// Four traffic mixes, each over buffers far larger than the L2 and the
// memory-side cache (2 GiB in, 2 GiB out), with 16-byte accesses:
//   read        every source byte read once (a reduction)
//   write       every destination byte written once (a fill)
//   copy        1 byte read per byte written
//   read2write1 2 bytes read per byte written (a 16-bit to 8-bit conversion,
//               the mix of quantizing K)
// each with ordinary and with nontemporal stores, and each at several grid
// sizes (work-groups of 256 threads per CU) and 4 or 8 16-byte accesses in
// flight per thread.  One JSON line per mix: the best rate over those shapes
// (median of 5 timed launches after a warm-up, hipEvents) and the shape that
// gave it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                            \
  do {                                                                                      \
    hipError_t e_ = (x);                                                                    \
    if (e_ != hipSuccess) {                                                                 \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                         \
    }                                                                                       \
  } while (0)

enum Mix { kRead = 0, kWrite = 1, kCopy = 2, kR2W1 = 3 };
static const char* kMixName[] = {"read", "write", "copy", "read2write1"};

template <int M, bool NT>
__device__ __forceinline__ void put(uint4* p, uint4 v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(v.x, &p->x);
    __builtin_nontemporal_store(v.y, &p->y);
    __builtin_nontemporal_store(v.z, &p->z);
    __builtin_nontemporal_store(v.w, &p->w);
  } else {
    *p = v;
  }
}

// n: 16-byte destination items (kRead: source items).  kR2W1 reads src[2i]
// and src[2i+1] for destination item i, so src holds 2n items there.
template <int M, bool NT, int kUnroll>
__global__ __launch_bounds__(256) void stream_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                     int64_t n, uint32_t* sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (int64_t i0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i0 < n; i0 += stride * kUnroll) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * stride;
      if (i < n) {
        if constexpr (M == kRead || M == kCopy) {
          v[u] = src[i];
        } else if constexpr (M == kR2W1) {
          const uint4 a = src[2 * i], b = src[2 * i + 1];
          v[u] = make_uint4(a.x ^ b.y, a.y ^ b.x, a.z ^ b.w, a.w ^ b.z);
        } else {
          v[u] = make_uint4((uint32_t)i, 1u, 2u, 3u);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * stride;
      if (i < n) {
        if constexpr (M == kRead) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        else put<M, NT>(dst + i, v[u]);
      }
    }
  }
  if (M == kRead && acc == 0x9E3779B9u) sink[0] = acc;  // keeps the loads; practically never taken
}

template <int M, bool NT>
static void run(const uint4* src, uint4* dst, uint32_t* sink, int64_t bytes, int cus) {
  // 16-byte items of the destination (of the source for kRead)
  const int64_t n = bytes / 16;
  const double moved = M == kRead ? (double)bytes : M == kWrite ? (double)bytes : M == kCopy ? 2.0 * bytes : 3.0 * bytes;
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  double best = 0.0;
  int best_wg = 0, best_u = 0;
  for (int u : {4, 8}) {
    for (int wg : {1, 2, 4, 8, 16, 32}) {
      const dim3 grid((unsigned)(cus * wg));
      auto launch = [&]() {
        if (u == 4) hipLaunchKernelGGL((stream_kernel<M, NT, 4>), grid, dim3(256), 0, 0, src, dst, n, sink);
        else hipLaunchKernelGGL((stream_kernel<M, NT, 8>), grid, dim3(256), 0, 0, src, dst, n, sink);
        CHECK(hipGetLastError());
      };
      launch();
      std::vector<float> ms(5);
      for (float& t : ms) {
        CHECK(hipEventRecord(e0, 0));
        launch();
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        CHECK(hipEventElapsedTime(&t, e0, e1));
      }
      std::sort(ms.begin(), ms.end());
      const double tbs = moved / (ms[2] * 1e-3) / 1e12;
      if (tbs > best) {
        best = tbs;
        best_wg = wg;
        best_u = u;
      }
    }
  }
  std::printf("{\"mix\": \"%s\", \"nontemporal_stores\": %s, \"bytes_moved\": %.0f, \"tb_per_s\": %.3f, "
              "\"frac_of_8tbs\": %.3f, \"workgroups_per_cu\": %d, \"accesses_in_flight_per_thread\": %d}\n",
              kMixName[M], NT ? "true" : "false", moved, best, best / 8.0, best_wg, best_u);
  std::fflush(stdout);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main(int argc, char** argv) {
  const int64_t gib = argc > 1 ? std::atoll(argv[1]) : 2;
  const int64_t bytes = gib << 30;  // destination bytes (kR2W1 reads 2x from a source of 2x)
  hipDeviceProp_t p;
  CHECK(hipGetDeviceProperties(&p, 0));
  std::printf("{\"device\": \"%s\", \"arch\": \"%s\", \"compute_units\": %d, \"dst_bytes\": %lld}\n", p.name,
              p.gcnArchName, p.multiProcessorCount, (long long)bytes);
  uint4 *src, *dst;
  uint32_t* sink;
  CHECK(hipMalloc(&src, 2 * bytes));
  CHECK(hipMalloc(&dst, bytes));
  CHECK(hipMalloc(&sink, 64));
  CHECK(hipMemset(src, 0x5A, 2 * bytes));
  CHECK(hipMemset(dst, 0, bytes));
  CHECK(hipDeviceSynchronize());
  const int cus = p.multiProcessorCount;
  run<kRead, false>(src, dst, sink, bytes, cus);
  run<kWrite, false>(src, dst, sink, bytes, cus);
  run<kWrite, true>(src, dst, sink, bytes, cus);
  run<kCopy, false>(src, dst, sink, bytes, cus);
  run<kCopy, true>(src, dst, sink, bytes, cus);
  run<kR2W1, false>(src, dst, sink, bytes, cus);
  run<kR2W1, true>(src, dst, sink, bytes, cus);
  CHECK(hipFree(src));
  CHECK(hipFree(dst));
  CHECK(hipFree(sink));
  return 0;
}
