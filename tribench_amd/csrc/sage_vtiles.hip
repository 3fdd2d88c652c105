// sage_vtiles.hip — V in the attention kernel's tile layout.
//
// The counterpart of the reference's host-side `v.to(torch.float16)` before
// the attention launch (kernels/sage_attn/triton_impl.py:189), fused with the
// layout change the attention kernel wants: V^T in tiles of 64 keys, so the
// kernel copies each tile into LDS with direct (global -> LDS) loads and
// reads every P.V operand as whole 16-byte chunks.
//
// The tile layout and the per-tile work are in sage_vtile_dev.h (shared with
// the pre-pass): one block per tile, 256 threads load the 64 x D tile with
// 16-byte loads along the rows, convert, transpose through LDS and store
// 16-byte chunks.  Build with -ffp-contract=off (the e4m3 division must be
// IEEE).
#include "sage_vtile_dev.h"

namespace sage {

struct VtileArgs {
  const void* v;
  int64_t sv[3];  // batch, head, sequence strides (elements)
  int64_t Hkv, Nkv, ntile;
  const float* v_scale;  // [B, Hkv, D] (FP8 only)
  uint8_t* out;
};

template <typename T, int D, int PVM>
__global__ __launch_bounds__(256) void vtile_kernel(VtileArgs a) {
  __shared__ __attribute__((aligned(16))) char tile_s[vtile_lds_bytes<D, PVM>()];
  __shared__ float vs_s[stat_lds_floats<D>()];
  const int64_t r = blockIdx.x;
  const int64_t t = r % a.ntile, h = (r / a.ntile) % a.Hkv, b = r / (a.ntile * a.Hkv);
  if constexpr (PVM == SAGE_PV_FP8) {
    if (threadIdx.x < D) vs_s[stat_slot(threadIdx.x)] = a.v_scale[(b * a.Hkv + h) * D + threadIdx.x];
    __syncthreads();
  }
  constexpr int EB = PVM == SAGE_PV_FP8 ? 1 : 2;
  const T* src = static_cast<const T*>(a.v) + b * a.sv[0] + h * a.sv[1];
  uint8_t* dst = a.out + ((b * a.Hkv + h) * a.ntile + t) * (int64_t)D * 64 * EB;
  vtile_block<T, D, PVM>(src, a.sv[2], a.Nkv, t, vs_s, dst, tile_s);
}

template <typename T, int PVM>
static int launch_vtiles(const VtileArgs& a, int64_t nblk, int D, hipStream_t st) {
  if (D == 64)
    hipLaunchKernelGGL((vtile_kernel<T, 64, PVM>), dim3((unsigned)nblk), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((vtile_kernel<T, 128, PVM>), dim3((unsigned)nblk), dim3(256), 0, st, a);
  return check_launch("sage_vtiles");
}

template <typename T>
static int launch_vtiles_pv(const VtileArgs& a, int64_t nblk, int D, int pv_mode, hipStream_t st) {
  switch (pv_mode) {
    case SAGE_PV_F16: return launch_vtiles<T, SAGE_PV_F16>(a, nblk, D, st);
    case SAGE_PV_BF16: return launch_vtiles<T, SAGE_PV_BF16>(a, nblk, D, st);
    default: return launch_vtiles<T, SAGE_PV_FP8>(a, nblk, D, st);
  }
}

}  // namespace sage

using namespace sage;

extern "C" size_t sage_vtile_bytes(int64_t B, int64_t Hkv, int64_t Nkv, int64_t D, int pv_mode) {
  if (B <= 0 || Hkv <= 0 || Nkv <= 0 || D <= 0) return 0;
  const int64_t eb = pv_mode == SAGE_PV_FP8 ? 1 : 2;
  return (size_t)(B * Hkv * ((Nkv + 63) / 64) * D * 64 * eb);
}

extern "C" int sage_vtiles(const void* v, int in_dtype, int64_t B, int64_t Hkv, int64_t Nkv, int64_t D,
                           const int64_t* v_strides, int pv_mode, const float* v_scale, void* out,
                           size_t out_bytes, void* stream) {
  if (B <= 0 || Hkv <= 0 || Nkv <= 0) return fail("sage_vtiles: invalid argument: empty shape");
  if (D != 64 && D != 128) return fail("sage_vtiles: invalid argument: head_dim %lld", (long long)D);
  if (in_dtype != SAGE_DTYPE_F32 && in_dtype != SAGE_DTYPE_F16 && in_dtype != SAGE_DTYPE_BF16)
    return fail("sage_vtiles: invalid argument: in_dtype %d", in_dtype);
  if (pv_mode != SAGE_PV_F16 && pv_mode != SAGE_PV_BF16 && pv_mode != SAGE_PV_FP8)
    return fail("sage_vtiles: invalid argument: pv_mode %d", pv_mode);
  if (!v || !out || !v_strides || (pv_mode == SAGE_PV_FP8 && !v_scale))
    return fail("sage_vtiles: invalid argument: null pointer");
  const int es = in_dtype == SAGE_DTYPE_F32 ? 4 : 2;
  for (int i = 0; i < 3; ++i)
    if (v_strides[i] < 0 || (v_strides[i] * es) % 16 != 0)
      return fail("sage_vtiles: invalid argument: strides must keep 16-byte aligned rows");
  if (((uintptr_t)v | (uintptr_t)out) % 16 != 0)
    return fail("sage_vtiles: invalid argument: pointers must be 16-byte aligned");
  const size_t need = sage_vtile_bytes(B, Hkv, Nkv, D, pv_mode);
  if (out_bytes < need) return fail("sage_vtiles: invalid argument: out %zu bytes < %zu", out_bytes, need);
  VtileArgs a{};
  a.v = v;
  for (int i = 0; i < 3; ++i) a.sv[i] = v_strides[i];
  a.Hkv = Hkv;
  a.Nkv = Nkv;
  a.ntile = (Nkv + 63) / 64;
  a.v_scale = v_scale;
  a.out = static_cast<uint8_t*>(out);
  const int64_t nblk = B * Hkv * a.ntile;
  if (nblk > 0x7FFFFFFF) return fail("sage_vtiles: invalid argument: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case SAGE_DTYPE_F32: return launch_vtiles_pv<float>(a, nblk, (int)D, pv_mode, st);
    case SAGE_DTYPE_F16: return launch_vtiles_pv<_Float16>(a, nblk, (int)D, pv_mode, st);
    default: return launch_vtiles_pv<__bf16>(a, nblk, (int)D, pv_mode, st);
  }
}
