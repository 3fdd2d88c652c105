// Device check of gfx950's fp32 -> FP8 e4m3 conversion instruction
// (v_cvt_pk_fp8_f32, __builtin_amdgcn_cvt_pk_fp8_f32) against the pre-pass's
// own conversion sage::f32_to_e4m3 (tribench_amd/csrc/sage_quant_math.h: OCP
// e4m3fn, round to nearest even, saturation to +-448; host-checked against
// torch.float8_e4m3fn by tests/native/quant_math_check.cpp).
//
// Every one of the 2^32 fp32 bit patterns f is converted as the packed
// instruction is used in the kernels: word = cvt(f, -f) into the low half,
// then cvt(f, -f) into the high half of the same word, so all four bytes
// and both halves are compared.  Patterns are counted per class:
//   0  finite |f| <= 448 * (1 + 2^-23)   (every quotient the pre-pass forms)
//   1  finite 448 * (1 + 2^-23) < |f| < 464
//   2  |f| >= 464, infinities
//   3  NaN
// Output: one JSON line with the patterns and the mismatches per class and
// the first mismatching pattern of each class (or -1).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define SAGE_HD __host__ __device__
#include "../../tribench_amd/csrc/sage_quant_math.h"

#define CHECK(x)                                                                            \
  do {                                                                                      \
    hipError_t e_ = (x);                                                                    \
    if (e_ != hipSuccess) {                                                                 \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                         \
    }                                                                                       \
  } while (0)

struct Result {
  unsigned long long patterns[4];
  unsigned long long mismatches[4];
  unsigned long long first[4];  // smallest mismatching pattern + 1 (0: none)
};

__device__ __forceinline__ int klass(uint32_t u) {
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 3;
  if (a >= 0x43E80000u) return 2;  // 464
  if (a > 0x43E00000u) return 1;   // 448
  return 0;
}

__global__ __launch_bounds__(256) void check_kernel(Result* res) {
  unsigned long long pat[4] = {0, 0, 0, 0}, mis[4] = {0, 0, 0, 0};
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t b = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; b < (1ull << 32); b += stride) {
    const uint32_t u = (uint32_t)b;
    const float f = __builtin_bit_cast(float, u);
    const float g = __builtin_bit_cast(float, u ^ 0x80000000u);
    uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(f, g, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(f, g, w, true);
    const uint32_t sf = sage::f32_to_e4m3(f), sg = sage::f32_to_e4m3(g);
    const uint32_t want = sf | (sg << 8) | (sf << 16) | (sg << 24);
    const int c = klass(u);
    pat[c] += 1;
    if (w != want) {
      mis[c] += 1;
      atomicMin(&res->first[c], (unsigned long long)u + 1ull);
    }
  }
  for (int c = 0; c < 4; ++c) {
    if (pat[c]) atomicAdd(&res->patterns[c], pat[c]);
    if (mis[c]) atomicAdd(&res->mismatches[c], mis[c]);
  }
}

int main() {
  Result* d;
  CHECK(hipMalloc(&d, sizeof(Result)));
  Result h{};
  for (int c = 0; c < 4; ++c) h.first[c] = ~0ull;
  CHECK(hipMemcpy(d, &h, sizeof(Result), hipMemcpyHostToDevice));
  hipLaunchKernelGGL(check_kernel, dim3(8192), dim3(256), 0, 0, d);
  CHECK(hipGetLastError());
  CHECK(hipMemcpy(&h, d, sizeof(Result), hipMemcpyDeviceToHost));
  CHECK(hipFree(d));
  std::printf("{\"patterns\": [%llu, %llu, %llu, %llu], \"mismatches\": [%llu, %llu, %llu, %llu], \"first\": [",
              h.patterns[0], h.patterns[1], h.patterns[2], h.patterns[3], h.mismatches[0], h.mismatches[1],
              h.mismatches[2], h.mismatches[3]);
  for (int c = 0; c < 4; ++c) {
    const long long v = h.first[c] == ~0ull ? -1 : (long long)(h.first[c] - 1ull);
    std::printf("%s%lld", c ? ", " : "", v);
  }
  std::printf("]}\n");
  return 0;
}
