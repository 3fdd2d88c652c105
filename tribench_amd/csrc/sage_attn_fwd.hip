// sage_attn_fwd.hip — fused SageAttention forward for gfx950 (MI355X).
//
// Replaces _attn_fwd / _attn_fwd_inner (kernels/sage_attn/triton_impl.py:86-160)
// and its launch (:186-199).  Per key block of 64:
//   S^T = K8 . Q8^T            v_mfma_i32_16x16x64_i8   (INT8, i32 accumulate)
//   s   = float(S) * (q_scale * k_scale)          (triton_impl.py:99)
//   online base-2 softmax: m, l, p = exp2(s - m)   (triton_impl.py:102-109)
//   O^T += V^T . P^T           v_mfma_f32_16x16x32_{f16,bf16}, fp32 accumulate
// and O / l at the end (triton_impl.py:159).  Causal (top-left, like the
// torch.tril mask of reference.py:19-22), ragged tails and GQA
// (kv head = h / (Hq/Hkv), triton_impl.py:137,145,147) are handled here; the
// reference kernel ignores `causal`.
//
// Layout choices (CDNA4):
//  * The score tile is computed transposed, S^T[key][q].  Its MFMA C layout
//    (lane = 16*g + n holds q = n and keys 4g..4g+3 of a 16-key tile) is, after
//    conversion to 16 bit, exactly the B-operand layout of the P.V MFMA, so P
//    never leaves registers.  Row max and row sum are per lane plus two xor
//    shuffles across the four lane groups.
//  * K8 tiles live in LDS row-major with 16-byte chunks XOR-swizzled by the
//    128-byte line index (conflict-free ds_read_b128 for the A operand).
//  * V tiles are converted to the P.V type while being staged and stored
//    transposed (V^T[d][key], 8-byte chunks swizzled) so each lane's A operand
//    is two ds_read_b64.
//  * K/V tiles are double-buffered: global loads for block j+1 are in flight
//    while block j is computed; one barrier per block.
//  * Work-group ids are remapped so that all q-blocks of one (batch, kv head)
//    run on the same XCD (shared L2) — the hardware deals work-groups to the 8
//    XCDs round-robin.
#include "sage_device.h"

namespace sage {

struct AttnArgs {
  const int8_t* q8;
  const float* q_scale;
  const int8_t* k8;
  const float* k_scale;
  const void* v;
  const float* v_scale;
  void* o;
  int64_t sq[3], sk[3], sv[3], so[3];
  int B, Hq, Hkv, Nq, Nkv;
  int causal;
  int q_sub, blkk;
  int nqs, nks;  // q / k scales per head
};

template <typename P>
struct PvOps;
template <>
struct PvOps<_Float16> {
  typedef v8h V8;
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    h2 r = __builtin_convertvector((f2){a, b}, h2);
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ static __forceinline__ v4f mfma(const v4i& a, const v4i& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0,
                                                  0, 0);
  }
};
template <>
struct PvOps<__bf16> {
  typedef v8bf V8;
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    bf2 r = __builtin_convertvector((f2){a, b}, bf2);
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ static __forceinline__ v4f mfma(const v4i& a, const v4i& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c,
                                                   0, 0, 0);
  }
};

template <typename TO>
__device__ __forceinline__ void store4(TO* p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void store4<float>(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
template <>
__device__ __forceinline__ void store4<_Float16>(_Float16* p, float a, float b, float c, float d) {
  v2i w = {(int)PvOps<_Float16>::pack2(a, b), (int)PvOps<_Float16>::pack2(c, d)};
  *reinterpret_cast<v2i*>(p) = w;
}
template <>
__device__ __forceinline__ void store4<__bf16>(__bf16* p, float a, float b, float c, float d) {
  v2i w = {(int)PvOps<__bf16>::pack2(a, b), (int)PvOps<__bf16>::pack2(c, d)};
  *reinterpret_cast<v2i*>(p) = w;
}

// byte offset of 16-byte chunk L (= row * chunks_per_row + col) of a K8 tile
__device__ __forceinline__ int k_lds_off(int L) {
  const int line = L >> 3, pos = L & 7;
  return (line << 7) + ((pos ^ (line & 7)) << 4);
}
// byte offset of 8-byte chunk c (4 keys) of row d of the V^T tile (64 keys)
__device__ __forceinline__ int v_lds_off(int d, int c) {
  return (d << 7) + ((c ^ ((d ^ (d >> 3)) & 15)) << 3);
}

__device__ __forceinline__ int remap_xcd(int w, int n) {
  const int per = n >> 3, rem = n & 7;
  const int xcd = w & 7, loc = w >> 3;
  return xcd * per + min(xcd, rem) + loc;
}

template <int D, int NW, int QW, typename TV, typename PV, typename TO>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(AttnArgs a) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * QW;  // q rows per work-group
  constexpr int BN = 64;       // keys per block
  constexpr int QT = QW / 16;  // q tiles per wave
  constexpr int DH = D / 64;   // 64-wide slices of the QK contraction
  constexpr int DT = D / 16;   // 16-row d tiles of O^T
  constexpr int KT = BN / 16;  // 16-key tiles per block
  constexpr int CPR = D / 16;  // 16-byte chunks per K8 row
  constexpr int K_BYTES = BN * D;
  constexpr int V_BYTES = D * BN * 2;
  constexpr int BUF = K_BYTES + V_BYTES;
  constexpr int KCH = BN * CPR;             // K8 chunks per tile
  constexpr int KCH_T = (KCH + NT - 1) / NT;
  constexpr int VMT = (BN / 4) * (D / 8);   // 4-key x 8-d micro-tiles per V tile
  constexpr int VMT_T = (VMT + NT - 1) / NT;
  using Ops = PvOps<PV>;

  __shared__ __attribute__((aligned(16))) char smem[2 * BUF];

  const int nqb = (a.Nq + BM - 1) / BM;
  const int wg = remap_xcd((int)blockIdx.x, (int)gridDim.x);
  int qb = wg % nqb;
  const int h = (wg / nqb) % a.Hq;
  const int b = wg / (nqb * a.Hq);
  if (a.causal) qb = nqb - 1 - qb;  // longest rows first
  const int hk = h / (a.Hq / a.Hkv);

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int q0 = qb * BM;
  const int qa = q0 + wave * QW;  // first q row of this wave

  const int8_t* qbase = a.q8 + b * a.sq[0] + h * a.sq[1];
  const int8_t* kbase = a.k8 + b * a.sk[0] + hk * a.sk[1];
  const TV* vbase = static_cast<const TV*>(a.v) + b * a.sv[0] + hk * a.sv[1];
  const float* ksc_base = a.k_scale + ((int64_t)b * a.Hkv + hk) * a.nks;

  // ---- Q (B operand of S^T = K Q^T): q = qa + 16s + n, d = 64hh + 16g .. +16
  v4i qreg[QT][DH];
  float qsc[QT];
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    const int row = qa + 16 * s + n;
#pragma unroll
    for (int hh = 0; hh < DH; ++hh) {
      qreg[s][hh] = (v4i){0, 0, 0, 0};
      if (row < a.Nq) qreg[s][hh] = *reinterpret_cast<const v4i*>(qbase + row * a.sq[2] + 64 * hh + 16 * g);
    }
    const int si = min((qa + 16 * s) / a.q_sub, a.nqs - 1);
    qsc[s] = a.q_scale[((int64_t)b * a.Hq + h) * a.nqs + si];
  }

  // ---- key range
  const int nkb_all = (a.Nkv + BN - 1) / BN;
  int nkb = nkb_all;
  if (a.causal) nkb = min(nkb_all, (min(q0 + BM, a.Nq) - 1) / BN + 1);
  const int q_last = min(qa + QW, a.Nq) - 1;  // last valid row of this wave (< qa if none)

  // ---- staging registers
  v4i kst[KCH_T];
  Raw8<TV> vst[VMT_T][4];

  auto stage_load = [&](int j) {
    const int k0 = j * BN;
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      const int L = tid + i * NT;
      kst[i] = (v4i){0, 0, 0, 0};
      if (L < KCH) {
        const int row = L / CPR, c = L % CPR;
        if (k0 + row < a.Nkv) kst[i] = *reinterpret_cast<const v4i*>(kbase + (k0 + row) * a.sk[2] + 16 * c);
      }
    }
#pragma unroll
    for (int i = 0; i < VMT_T; ++i) {
      const int m = tid + i * NT;
      if (m < VMT) {
        const int dg = m % (D / 8), kq = m / (D / 8);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 4 * kq + r;
          vst[i][r] = key < a.Nkv ? load8<TV>(vbase + key * a.sv[2] + 8 * dg) : zero8<TV>();
        }
      }
    }
  };
  auto stage_store = [&](int buf) {
    char* ks = smem + buf * BUF;
    char* vs = ks + K_BYTES;
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      const int L = tid + i * NT;
      if (L < KCH) *reinterpret_cast<v4i*>(ks + k_lds_off(L)) = kst[i];
    }
#pragma unroll
    for (int i = 0; i < VMT_T; ++i) {
      const int m = tid + i * NT;
      if (m < VMT) {
        const int dg = m % (D / 8), kq = m / (D / 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v2i w;
          w.x = (int)Ops::pack2(elem<TV>(vst[i][0], e), elem<TV>(vst[i][1], e));
          w.y = (int)Ops::pack2(elem<TV>(vst[i][2], e), elem<TV>(vst[i][3], e));
          *reinterpret_cast<v2i*>(vs + v_lds_off(8 * dg + e, kq)) = w;
        }
      }
    }
  };

  // ---- accumulators
  v4f oacc[DT][QT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < QT; ++s) oacc[dt][s] = (v4f){0.f, 0.f, 0.f, 0.f};
  float m_i[QT], l_i[QT];
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    m_i[s] = -INFINITY;
    l_i[s] = 0.0f;
  }

  stage_load(0);
  stage_store(0);
  __syncthreads();

  for (int j = 0; j < nkb; ++j) {
    const bool has_next = j + 1 < nkb;
    if (has_next) stage_load(j + 1);
    const int k0 = j * BN;
    const bool active = q_last >= qa && (!a.causal || k0 <= q_last);
    if (active) {
      const char* ks = smem + (j & 1) * BUF;
      const char* vs = ks + K_BYTES;
      // S^T = K Q^T
      v4i sacc[KT][QT];
#pragma unroll
      for (int t = 0; t < KT; ++t) {
#pragma unroll
        for (int s = 0; s < QT; ++s) sacc[t][s] = (v4i){0, 0, 0, 0};
#pragma unroll
        for (int hh = 0; hh < DH; ++hh) {
          const v4i ka = *reinterpret_cast<const v4i*>(ks + k_lds_off((16 * t + n) * CPR + 4 * hh + g));
#pragma unroll
          for (int s = 0; s < QT; ++s)
            sacc[t][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, qreg[s][hh], sacc[t][s], 0, 0, 0);
        }
      }
      const float ksc = ksc_base[k0 / a.blkk];
      const bool masked = (k0 + BN > a.Nkv) || (a.causal && k0 + BN - 1 > qa);
      // online softmax (base 2) and P in B-operand layout
      v4i pk[QT][2];
#pragma unroll
      for (int s = 0; s < QT; ++s) {
        const float c = qsc[s] * ksc;
        const int qrow = qa + 16 * s + n;
        int mx = INT_MIN;
#pragma unroll
        for (int t = 0; t < KT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = k0 + 16 * t + 4 * g + r;
            const bool ok = !masked || (key < a.Nkv && (!a.causal || key <= qrow));
            if (ok) mx = max(mx, sacc[t][s][r]);
          }
        mx = max(mx, __shfl_xor(mx, 16));
        mx = max(mx, __shfl_xor(mx, 32));
        const float mblk = mx == INT_MIN ? -INFINITY : (float)mx * c;
        const float mnew = fmaxf(m_i[s], mblk);
        const float alpha = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_i[s] - mnew);
        const float msub = mnew == -INFINITY ? 0.0f : mnew;
        m_i[s] = mnew;
        l_i[s] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt][s] *= alpha;
        float p[KT][4];
#pragma unroll
        for (int t = 0; t < KT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = k0 + 16 * t + 4 * g + r;
            const bool ok = !masked || (key < a.Nkv && (!a.causal || key <= qrow));
            const float x = __builtin_fmaf((float)sacc[t][s][r], c, -msub);
            p[t][r] = ok ? __builtin_amdgcn_exp2f(x) : 0.0f;
            l_i[s] += p[t][r];
          }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          pk[s][u].x = (int)Ops::pack2(p[2 * u][0], p[2 * u][1]);
          pk[s][u].y = (int)Ops::pack2(p[2 * u][2], p[2 * u][3]);
          pk[s][u].z = (int)Ops::pack2(p[2 * u + 1][0], p[2 * u + 1][1]);
          pk[s][u].w = (int)Ops::pack2(p[2 * u + 1][2], p[2 * u + 1][3]);
        }
      }
      // O^T += V^T P^T
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 16 * dt + n;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const v2i lo = *reinterpret_cast<const v2i*>(vs + v_lds_off(d, 8 * u + g));
          const v2i hi = *reinterpret_cast<const v2i*>(vs + v_lds_off(d, 8 * u + 4 + g));
          const v4i va = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
          for (int s = 0; s < QT; ++s) oacc[dt][s] = Ops::mfma(va, pk[s][u], oacc[dt][s]);
        }
      }
    }
    if (has_next) stage_store((j + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: O / l, store rows q = qa + 16s + n, d = 16dt + 4g .. +4
  TO* obase = static_cast<TO*>(a.o) + b * a.so[0] + h * a.so[1];
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    float l = l_i[s];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    const int row = qa + 16 * s + n;
    if (row < a.Nq) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const v4f o = oacc[dt][s] * inv;
        store4<TO>(obase + row * a.so[2] + 16 * dt + 4 * g, o.x, o.y, o.z, o.w);
      }
    }
  }
}

template <int D, typename TV, typename PV>
static int launch_attn(const AttnArgs& a, hipStream_t st) {
  constexpr int NW = 8, QW = 32, BM = NW * QW;
  const int64_t nqb = (a.Nq + BM - 1) / BM;
  const int64_t grid = nqb * a.Hq * a.B;
  if (grid > 0x7FFFFFFF) return fail("sage_attn_fwd: invalid argument: grid too large");
  hipLaunchKernelGGL((attn_fwd_kernel<D, NW, QW, TV, PV, TV>), dim3((unsigned)grid), dim3(NW * 64), 0, st, a);
  return check_launch("sage_attn_fwd");
}

template <typename TV, typename PV>
static int launch_attn_d(const AttnArgs& a, int D, hipStream_t st) {
  return D == 64 ? launch_attn<64, TV, PV>(a, st) : launch_attn<128, TV, PV>(a, st);
}

static bool strides_ok(const int64_t* s, int esize) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] * esize) % 16 != 0) return false;
  return true;
}

}  // namespace sage

using namespace sage;

extern "C" int sage_attn_fwd(const int8_t* q8, const int64_t* q8_strides, const float* q_scale,
                             const int8_t* k8, const int64_t* k8_strides, const float* k_scale,
                             const void* v, int v_dtype, const int64_t* v_strides, const float* v_scale,
                             void* o, int o_dtype, const int64_t* o_strides, int64_t B, int64_t Hq,
                             int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, int causal, int blkq,
                             int blkk, int q_sub, int pv_mode, void* stream) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Nq <= 0 || Nkv <= 0)
    return fail("sage_attn_fwd: invalid argument: empty shape");
  if (D != 64 && D != 128) return fail("sage_attn_fwd: invalid argument: head_dim %lld (supported: 64, 128)",
                                       (long long)D);
  if (Hq % Hkv != 0) return fail("sage_attn_fwd: invalid argument: Hq %% Hkv != 0");
  if (Nq > 0x7FFFFFFF || Nkv > 0x7FFFFFFF || Hq > 0xFFFF || B > 0xFFFF)
    return fail("sage_attn_fwd: invalid argument: shape too large");
  if (blkk < 64 || blkk % 64 != 0) return fail("sage_attn_fwd: invalid argument: blkk=%d (multiple of 64)", blkk);
  if (q_sub < 16 || q_sub % 16 != 0 || blkq % q_sub != 0)
    return fail("sage_attn_fwd: invalid argument: q_sub=%d blkq=%d", q_sub, blkq);
  if (!q8 || !q_scale || !k8 || !k_scale || !v || !o || !q8_strides || !k8_strides || !v_strides || !o_strides)
    return fail("sage_attn_fwd: invalid argument: null pointer");
  if (v_dtype != o_dtype || (v_dtype != SAGE_DTYPE_F32 && v_dtype != SAGE_DTYPE_F16 && v_dtype != SAGE_DTYPE_BF16))
    return fail("sage_attn_fwd: invalid argument: v_dtype %d / o_dtype %d", v_dtype, o_dtype);
  if (pv_mode != SAGE_PV_F16 && pv_mode != SAGE_PV_BF16)
    return fail("sage_attn_fwd: invalid argument: pv_mode %d not available", pv_mode);
  const int es = v_dtype == SAGE_DTYPE_F32 ? 4 : 2;
  if (!strides_ok(q8_strides, 1) || !strides_ok(k8_strides, 1) || !strides_ok(v_strides, es) ||
      !strides_ok(o_strides, es))
    return fail("sage_attn_fwd: invalid argument: strides must keep 16-byte aligned rows");
  if (((uintptr_t)q8 | (uintptr_t)k8 | (uintptr_t)v | (uintptr_t)o) % 16 != 0)
    return fail("sage_attn_fwd: invalid argument: base pointers must be 16-byte aligned");

  AttnArgs a{};
  a.q8 = q8;
  a.q_scale = q_scale;
  a.k8 = k8;
  a.k_scale = k_scale;
  a.v = v;
  a.v_scale = v_scale;
  a.o = o;
  for (int i = 0; i < 3; ++i) {
    a.sq[i] = q8_strides[i];
    a.sk[i] = k8_strides[i];
    a.sv[i] = v_strides[i];
    a.so[i] = o_strides[i];
  }
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.Nq = (int)Nq;
  a.Nkv = (int)Nkv;
  a.causal = causal ? 1 : 0;
  a.q_sub = q_sub;
  a.blkk = blkk;
  a.nqs = (int)(((Nq + blkq - 1) / blkq) * (blkq / q_sub));
  a.nks = (int)((Nkv + blkk - 1) / blkk);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf = pv_mode == SAGE_PV_BF16;
  switch (v_dtype) {
    case SAGE_DTYPE_F32:
      return bf ? launch_attn_d<float, __bf16>(a, (int)D, st) : launch_attn_d<float, _Float16>(a, (int)D, st);
    case SAGE_DTYPE_F16:
      return bf ? launch_attn_d<_Float16, __bf16>(a, (int)D, st)
                : launch_attn_d<_Float16, _Float16>(a, (int)D, st);
    default:
      return bf ? launch_attn_d<__bf16, __bf16>(a, (int)D, st) : launch_attn_d<__bf16, _Float16>(a, (int)D, st);
  }
}
