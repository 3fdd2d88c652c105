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
#include <stdlib.h>

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
  int64_t sq[2], sk[2], sv[2], so[2];  // batch and head strides (elements)
  int sqn, skn, svn, son;              // row strides (elements); row offsets fit 32 bits
  int B, Hq, Hkv, Nq, Nkv;
  int causal;
  int q_sub, blkk_shift;  // k scale of key block j: k_scale[j >> blkk_shift]
  int nqs, nks;           // q / k scales per head
};

template <typename P>
struct PvOps;
template <>
struct PvOps<_Float16> {
  typedef v8h V8;
  __device__ static __forceinline__ v4i ones() { return (v4i){0x3C003C00, 0x3C003C00, 0x3C003C00, 0x3C003C00}; }
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
  __device__ static __forceinline__ v4i ones() { return (v4i){0x3F803F80, 0x3F803F80, 0x3F803F80, 0x3F803F80}; }
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

// ---------------------------------------------------------------------------
// LDS layouts (rows padded instead of swizzled, so every operand read is one
// per-lane base plus a compile-time offset and both reads and staging writes
// are bank-conflict free).  A tile holds the BNI = 64*SUB keys of one
// iteration:
//  K8 tile  [BNI keys][D] int8, row pitch D + 16 bytes
//  V^T tile [D][BNI keys] 16-bit, row pitch 2*BNI + 8 bytes
// ---------------------------------------------------------------------------
__device__ __forceinline__ int remap_xcd(int w, int n) {
  const int per = n >> 3, rem = n & 7;
  const int xcd = w & 7, loc = w >> 3;
  return xcd * per + min(xcd, rem) + loc;
}

// max over the lanes {l, l^16, l^32, l^48} (the four lane groups holding one
// q column of the score tile) with the gfx950 permlane swaps
__device__ __forceinline__ int max_over_groups(int v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  v = max((int)a[0], (int)a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return max((int)b[0], (int)b[1]);
}

// The int32 MFMA accumulator starts at the bit pattern of 2^23 + 2^22, so
// it reads as the float 12582912 + S, exact for |S| < 2^22 (|S| <= 127^2*D).
constexpr int kMagicI = 0x4B400000;
constexpr float kMagicF = 12582912.0f;
// A row's running max is only moved when a block's max exceeds it by more
// than kTau (log2 units); P values are then bounded by 2^kTau.
constexpr float kTau = 8.0f;

// NW waves of QW query rows each; SUB 64-key sub-blocks per iteration (one
// barrier and one prefetch per iteration).  One work-group per CU: NW/4 waves
// per SIMD, so the compiler may use the whole register file.
template <int D, int NW, int QW, int SUB, typename TV, typename PV, typename TO>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4))) void attn_fwd_kernel(
    AttnArgs a) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * QW;   // q rows per work-group
  constexpr int BN = 64;        // keys per softmax block (one k scale)
  constexpr int BNI = BN * SUB; // keys per iteration
  constexpr int QT = QW / 16;   // q tiles per wave
  constexpr int DH = D / 64;    // 64-wide slices of the QK contraction
  constexpr int DT = D / 16;    // 16-row d tiles of O^T
  constexpr int KT = BN / 16;   // 16-key tiles per block
  constexpr int CPR = D / 16;   // 16-byte chunks per K8 row
  constexpr int KP = D + 16;    // K8 row pitch in LDS
  constexpr int VPI = 2 * BNI + 8;  // V^T row pitch in LDS
  constexpr int KB = BNI * KP;      // bytes of a K8 tile
  constexpr int VB = D * VPI;       // bytes of a V^T tile
  constexpr int KCH = BNI * CPR;            // 16-byte K8 chunks per tile
  constexpr int VMT = (BNI / 2) * (D / 8);  // 2-key x 8-d micro-tiles per V tile
  static_assert(KCH % 64 == 0 && VMT % 64 == 0, "staging work must be whole waves");
  constexpr int KCH_T = (KCH + NT - 1) / NT;
  constexpr int VMT_T = (VMT + NT - 1) / NT;
  using Ops = PvOps<PV>;

  __shared__ __attribute__((aligned(16))) char smem[2 * KB + 2 * VB];
  __shared__ float ksc_s[2][SUB];  // k scales of the tile in each buffer
  char* const kbuf0 = smem;
  char* const vbuf0 = smem + 2 * KB;

  const int nqb = (a.Nq + BM - 1) / BM;
  const int wg = remap_xcd((int)blockIdx.x, (int)gridDim.x);
  int qb = wg % nqb;
  const int h = (wg / nqb) % a.Hq;
  const int b = wg / (nqb * a.Hq);
  if (a.causal) qb = nqb - 1 - qb;  // longest rows first
  const int hk = h / (a.Hq / a.Hkv);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int q0 = qb * BM;
  const int qa = q0 + wave * QW;  // first q row of this wave

  const int8_t* qbase = a.q8 + b * a.sq[0] + h * a.sq[1];
  const int8_t* kbase = a.k8 + b * a.sk[0] + hk * a.sk[1];
  const TV* vbase = static_cast<const TV*>(a.v) + b * a.sv[0] + hk * a.sv[1];
  const float* ksc_base = a.k_scale + ((int64_t)b * a.Hkv + hk) * a.nks;

  // ---- Q (B operand of S^T = K Q^T): q = qa + 16s + n, d = 64hh + 16g .. +16.
  // Rows past Nq read the last row; their results are never stored.
  v4i qreg[QT][DH];
  float qsc[QT];
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    const int row = min(qa + 16 * s + n, a.Nq - 1);
#pragma unroll
    for (int hh = 0; hh < DH; ++hh)
      qreg[s][hh] = *reinterpret_cast<const v4i*>(qbase + (uint32_t)(row * a.sqn + 64 * hh + 16 * g));
    const int si = min((qa + 16 * s) / a.q_sub, a.nqs - 1);
    qsc[s] = a.q_scale[((int64_t)b * a.Hq + h) * a.nqs + si];
  }

  // ---- key range (in 64-key blocks) of the work-group and of this wave
  const int nkb_all = (a.Nkv + BN - 1) / BN;
  int nkb = nkb_all;
  if (a.causal) nkb = min(nkb_all, (min(q0 + BM, a.Nq) - 1) / BN + 1);
  const int nit = (nkb + SUB - 1) / SUB;      // iterations
  const int q_last = min(qa + QW, a.Nq) - 1;  // last valid row of this wave (< qa if none)
  int jmax = nkb - 1;                          // last 64-key block this wave needs
  if (q_last < qa) jmax = -1;
  else if (a.causal) jmax = min(jmax, q_last / BN);

  // ---- per-lane LDS read bases; tiles and halves are immediate offsets
  const int kread = n * KP + 16 * g;   // + (64*sb + 16*t)*KP + 64*hh
  const int vread = n * VPI + 8 * g;   // + dt*16*VPI + 2*(64*sb + 32*u + 16*hf)

  // ---- staging.  K8: chunk L = tid + i*NT -> row L/CPR, column L%CPR.
  // V: micro-tile m = tid + i*NT -> keys 2*(m%(BNI/2)) + {0,1}, d = 8*(m/(BNI/2)) .. +8.
  // Keys past Nkv read the last key: their P is 0 and the data is finite.
  v4i kst[KCH_T];
  Raw8<TV> vst[VMT_T][2];
  float kscst = 0.0f;  // lanes 0..SUB-1 of wave 0: the tile's k scales
  auto load_tile = [&](int it) {
    const int k0 = it * BNI;
    if (wave == 0 && lane < SUB) kscst = ksc_base[min((it * SUB + lane) >> a.blkk_shift, a.nks - 1)];
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      if (wave * 64 + i * NT < KCH) {
        const int L = tid + i * NT;
        const int row = min(k0 + L / CPR, a.Nkv - 1);
        kst[i] = *reinterpret_cast<const v4i*>(kbase + (uint32_t)(row * a.skn + 16 * (L % CPR)));
      }
    }
#pragma unroll
    for (int i = 0; i < VMT_T; ++i) {
      if (wave * 64 + i * NT < VMT) {
        const int m = tid + i * NT;
        const int key = k0 + 2 * (m % (BNI / 2));
        const int col = 8 * (m / (BNI / 2));
        vst[i][0] = load8<TV>(vbase + (uint32_t)(min(key, a.Nkv - 1) * a.svn + col));
        vst[i][1] = load8<TV>(vbase + (uint32_t)(min(key + 1, a.Nkv - 1) * a.svn + col));
      }
    }
  };
  auto store_tile = [&](int buf) {
    char* ks = kbuf0 + buf * KB;
    char* vs = vbuf0 + buf * VB;
    if (wave == 0 && lane < SUB) ksc_s[buf][lane] = kscst;
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      if (wave * 64 + i * NT < KCH) {
        const int L = tid + i * NT;
        *reinterpret_cast<v4i*>(ks + (L / CPR) * KP + 16 * (L % CPR)) = kst[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VMT_T; ++i) {
      if (wave * 64 + i * NT < VMT) {
        const int m = tid + i * NT;
        char* dst = vs + 8 * (m / (BNI / 2)) * VPI + 4 * (m % (BNI / 2));
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<uint32_t*>(dst + e * VPI) = Ops::pack2(elem<TV>(vst[i][0], e), elem<TV>(vst[i][1], e));
      }
    }
  };

  // ---- accumulators
  v4f oacc[DT][QT];
  v4f lacc[QT];  // row sums of P via MFMA with an all-ones A operand
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    lacc[s] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt][s] = (v4f){0.f, 0.f, 0.f, 0.f};
  }
  float m_use[QT];
#pragma unroll
  for (int s = 0; s < QT; ++s) m_use[s] = -INFINITY;
  const v4i ones = Ops::ones();

  // ---- building blocks.  Operand reads are separate from the MFMAs that
  // use them so a phase can issue its reads first; the generic path fences
  // reads from MFMAs with a scheduling barrier, the hot path interleaves them
  // explicitly (see below).
  // K8 operand (t, hh) of sub-block sb: rows 16t + n, bytes 64hh + 16g .. +16
  auto read_k = [&](int buf, int sb, v4i (&ka)[KT][DH]) {
    const char* ks = kbuf0 + buf * KB + kread + sb * 64 * KP;
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int hh = 0; hh < DH; ++hh) ka[t][hh] = *reinterpret_cast<const v4i*>(ks + t * 16 * KP + 64 * hh);
  };
  auto mma_qk = [&](const v4i (&ka)[KT][DH], v4i (&sacc)[KT][QT]) {
#pragma unroll
    for (int t = 0; t < KT; ++t) {
#pragma unroll
      for (int s = 0; s < QT; ++s) sacc[t][s] = (v4i){kMagicI, kMagicI, kMagicI, kMagicI};
#pragma unroll
      for (int hh = 0; hh < DH; ++hh)
#pragma unroll
        for (int s = 0; s < QT; ++s)
          sacc[t][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[t][hh], qreg[s][hh], sacc[t][s], 0, 0, 0);
    }
  };
  // V^T operand (dt) of half u of sub-block sb: rows 16dt + n, keys
  // 32u + 4g..+3 and 32u + 16 + 4g..+3 of the sub-block
  auto read_v = [&](int buf, int sb, int u, v4i (&va)[DT]) {
    const char* vs = vbuf0 + buf * VB + vread + sb * 128 + 64 * u;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const v2i lo = *reinterpret_cast<const v2i*>(vs + dt * 16 * VPI);
      const v2i hi = *reinterpret_cast<const v2i*>(vs + dt * 16 * VPI + 32);
      va[dt] = (v4i){lo.x, lo.y, hi.x, hi.y};
    }
  };
  auto mma_pv = [&](const v4i (&va)[DT], int u, const v4i (&pk)[QT][2]) {
#pragma unroll
    for (int s = 0; s < QT; ++s) lacc[s] = Ops::mfma(ones, pk[s][u], lacc[s]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int s = 0; s < QT; ++s) oacc[dt][s] = Ops::mfma(va[dt], pk[s][u], oacc[dt][s]);
  };
  auto qk = [&](int buf, int sb, v4i (&sacc)[KT][QT]) {
    v4i ka[KT][DH];
    read_k(buf, sb, ka);
    __builtin_amdgcn_sched_barrier(0);
    mma_qk(ka, sacc);
  };
  auto pv = [&](int buf, int sb, const v4i (&pk)[QT][2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      v4i va[DT];
      read_v(buf, sb, u, va);
      __builtin_amdgcn_sched_barrier(0);
      mma_pv(va, u, pk);
    }
  };
  auto key_ok = [&](int key, int qrow) { return key < a.Nkv && (!a.causal || key <= qrow); };
  // block max of each q column of 64-key block kb (log2 units; -inf if all masked)
  auto rowmax = [&](int kb, float ksc, const v4i (&sacc)[KT][QT], float (&mblk)[QT], bool masked) {
    const int k0 = kb * BN;
#pragma unroll
    for (int s = 0; s < QT; ++s) {
      const int qrow = qa + 16 * s + n;
      int mx = INT_MIN;
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int v = sacc[t][s][r];
          if (masked) v = key_ok(k0 + 16 * t + 4 * g + r, qrow) ? v : INT_MIN;
          mx = max(mx, v);
        }
      mx = max_over_groups(mx);
      mblk[s] = mx == INT_MIN ? -INFINITY : (float)(mx - kMagicI) * (qsc[s] * ksc);
    }
  };
  // lazy max update: returns whether O and the row sums must be rescaled by
  // alpha[] (wave-uniform; applied by the caller at the right point)
  auto decide = [&](const float (&mblk)[QT], float (&alpha)[QT]) -> bool {
    bool need = false;
#pragma unroll
    for (int s = 0; s < QT; ++s) need |= mblk[s] > m_use[s] + kTau;
    const bool rescale = __builtin_amdgcn_ballot_w64(need) != 0;
#pragma unroll
    for (int s = 0; s < QT; ++s) alpha[s] = 1.0f;
    if (rescale) {
#pragma unroll
      for (int s = 0; s < QT; ++s) {
        const float mn = fmaxf(m_use[s], mblk[s]);
        alpha[s] = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_use[s] - mn);
        m_use[s] = mn;
      }
    }
    return rescale;
  };
  // P = exp2(S*c - m) of q tile s in B-operand layout (16-bit pairs)
  auto exps_s = [&](int kb, float ksc, const v4i (&sacc)[KT][QT], v4i (&pk)[QT][2], int s, bool masked) {
    const int k0 = kb * BN;
    {
      const float c = qsc[s] * ksc;
      const float m = m_use[s] == -INFINITY ? 0.0f : m_use[s];
      const float bias = __builtin_fmaf(kMagicF, c, m);  // x = (2^23+2^22+S)*c - bias = S*c - m
      const int qrow = qa + 16 * s + n;
      float p[KT][4];
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = __builtin_fmaf(__int_as_float(sacc[t][s][r]), c, -bias);
          float e = __builtin_amdgcn_exp2f(x);
          if (masked) e = key_ok(k0 + 16 * t + 4 * g + r, qrow) ? e : 0.0f;
          p[t][r] = e;
        }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        pk[s][u].x = (int)Ops::pack2(p[2 * u][0], p[2 * u][1]);
        pk[s][u].y = (int)Ops::pack2(p[2 * u][2], p[2 * u][3]);
        pk[s][u].z = (int)Ops::pack2(p[2 * u + 1][0], p[2 * u + 1][1]);
        pk[s][u].w = (int)Ops::pack2(p[2 * u + 1][2], p[2 * u + 1][3]);
      }
    }
  };
  auto exps = [&](int kb, float ksc, const v4i (&sacc)[KT][QT], v4i (&pk)[QT][2], bool masked) {
#pragma unroll
    for (int s = 0; s < QT; ++s) exps_s(kb, ksc, sacc, pk, s, masked);
  };
  auto apply_rescale = [&](const float (&alpha)[QT]) {
#pragma unroll
    for (int s = 0; s < QT; ++s) {
      lacc[s] *= alpha[s];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt][s] *= alpha[s];
    }
  };
  auto is_masked = [&](int kb) {
    const int k0 = kb * BN;
    return (k0 + BN > a.Nkv) || (a.causal && k0 + BN - 1 > qa);
  };
  // generic order for one 64-key block (masked blocks, partially active tiles)
  auto block_generic = [&](int buf, int sb, int kb, const v4i (&sacc)[KT][QT], v4i (&pk)[QT][2]) {
    const float ksc = ksc_s[buf][sb];
    const bool masked = is_masked(kb);
    float mblk[QT], alpha[QT];
    if (masked) rowmax(kb, ksc, sacc, mblk, true);
    else rowmax(kb, ksc, sacc, mblk, false);
    if (decide(mblk, alpha)) apply_rescale(alpha);
    if (masked) exps(kb, ksc, sacc, pk, true);
    else exps(kb, ksc, sacc, pk, false);
    pv(buf, sb, pk);
  };

  // ---- main loop: iteration it stages tile it+1 (global loads in flight
  // during the compute) and computes the SUB 64-key blocks of tile it.  The
  // QK of every sub-block is issued before the first softmax.
  load_tile(0);
  store_tile(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int it = 0; it < nit; ++it) {
    const bool more = it + 1 < nit;
    if (more) load_tile(it + 1);
    const int buf = it & 1;
    const int kb0 = it * SUB;
    if (kb0 <= jmax) {
      v4i S[SUB][KT][QT];
      v4i P[QT][2];
#pragma unroll
      for (int sb = 0; sb < SUB; ++sb)
        if (kb0 + sb <= jmax) qk(buf, sb, S[sb]);
#pragma unroll
      for (int sb = 0; sb < SUB; ++sb)
        if (kb0 + sb <= jmax) block_generic(buf, sb, kb0 + sb, S[sb], P);
    }
    if (more) store_tile((it + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: O / l, store rows q = qa + 16s + n, d = 16dt + 4g .. +4
  TO* obase = static_cast<TO*>(a.o) + b * a.so[0] + h * a.so[1];
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    const float inv = 1.0f / lacc[s][0];
    const int row = qa + 16 * s + n;
    if (row < a.Nq) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const v4f o = oacc[dt][s] * inv;
        store4<TO>(obase + (uint32_t)(row * a.son + 16 * dt + 4 * g), o.x, o.y, o.z, o.w);
      }
    }
  }
}

template <int D, int NW, int QW, int SUB, typename TV, typename PV>
static int launch_cfg(const AttnArgs& a, hipStream_t st) {
  constexpr int BM = NW * QW;
  const int64_t nqb = (a.Nq + BM - 1) / BM;
  const int64_t grid = nqb * a.Hq * a.B;
  if (grid > 0x7FFFFFFF) return fail("sage_attn_fwd: invalid argument: grid too large");
  hipLaunchKernelGGL((attn_fwd_kernel<D, NW, QW, SUB, TV, PV, TV>), dim3((unsigned)grid), dim3(NW * 64), 0, st,
                     a);
  return check_launch("sage_attn_fwd");
}

// Tiling variant: 0 = 8 waves x 32 rows, 64 keys per iteration (default);
// 1 = 8 waves x 32 rows, 128 keys per iteration.  SAGE_ATTN_VARIANT selects.
static int attn_variant() {
  static int v = [] {
    const char* e = getenv("SAGE_ATTN_VARIANT");
    return e ? atoi(e) : 0;
  }();
  return v;
}

template <int D, typename TV, typename PV>
static int launch_attn(const AttnArgs& a, hipStream_t st) {
  if (attn_variant() == 1) return launch_cfg<D, 8, 32, 2, TV, PV>(a, st);
  return launch_cfg<D, 8, 32, 1, TV, PV>(a, st);
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
  if (blkk != 64 && blkk != 128 && blkk != 256)
    return fail("sage_attn_fwd: invalid argument: blkk=%d (64, 128 or 256)", blkk);
  if (q_sub < 16 || q_sub % 16 != 0 || blkq % q_sub != 0)
    return fail("sage_attn_fwd: invalid argument: q_sub=%d blkq=%d", q_sub, blkq);
  if (!q8 || !q_scale || !k8 || !k_scale || !v || !o || !q8_strides || !k8_strides || !v_strides || !o_strides)
    return fail("sage_attn_fwd: invalid argument: null pointer");
  if (v_dtype != o_dtype || (v_dtype != SAGE_DTYPE_F32 && v_dtype != SAGE_DTYPE_F16 && v_dtype != SAGE_DTYPE_BF16))
    return fail("sage_attn_fwd: invalid argument: v_dtype %d / o_dtype %d", v_dtype, o_dtype);
  if (pv_mode != SAGE_PV_F16 && pv_mode != SAGE_PV_BF16)
    return fail("sage_attn_fwd: invalid argument: pv_mode %d not available", pv_mode);
  const int es = v_dtype == SAGE_DTYPE_F32 ? 4 : 2;
  const bool rows32 = Nq * q8_strides[2] + D < 0x7FFFFFFF && Nkv * k8_strides[2] + D < 0x7FFFFFFF &&
                      Nkv * v_strides[2] + D < 0x7FFFFFFF && Nq * o_strides[2] + D < 0x7FFFFFFF;
  if (!rows32) return fail("sage_attn_fwd: invalid argument: a head's rows must span < 2^31 elements");
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
  for (int i = 0; i < 2; ++i) {
    a.sq[i] = q8_strides[i];
    a.sk[i] = k8_strides[i];
    a.sv[i] = v_strides[i];
    a.so[i] = o_strides[i];
  }
  a.sqn = (int)q8_strides[2];
  a.skn = (int)k8_strides[2];
  a.svn = (int)v_strides[2];
  a.son = (int)o_strides[2];
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.Nq = (int)Nq;
  a.Nkv = (int)Nkv;
  a.causal = causal ? 1 : 0;
  a.q_sub = q_sub;
  a.blkk_shift = blkk == 64 ? 0 : (blkk == 128 ? 1 : 2);
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
