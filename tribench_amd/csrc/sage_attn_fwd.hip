// sage_attn_fwd.hip — fused SageAttention forward for gfx950 (MI355X).
//
// Replaces _attn_fwd / _attn_fwd_inner (kernels/sage_attn/triton_impl.py:86-160)
// and its launch (:186-199).  Per block of 64 keys:
//   S^T = K8 . Q8^T          v_mfma_i32_32x32x32_i8 (INT8, i32 accumulate)
//   s   = float(S) * (q_scale * k_scale)          (triton_impl.py:99)
//   online base-2 softmax: m, l, p = exp2(s - m)   (triton_impl.py:102-109)
//   O^T += V^T . P^T         v_mfma_f32_32x32x16_{f16,bf16}, or FP8 e4m3
//                            v_mfma_f32_32x32x64_f8f6f4; fp32 accumulate
// and O / l at the end (triton_impl.py:159).  Causal (top-left, the torch.tril
// mask of reference.py:19-22), ragged tails and GQA (kv head = h / (Hq/Hkv),
// triton_impl.py:137,145,147) are handled here.
//
// Organisation (CDNA4):
//  * A work-group covers 256 query rows of one (batch, head).  The launched
//    shape is 8 waves (2 per SIMD) of 32 rows each (one 32-row MFMA tile,
//    QT = 1): Q8 rows, S, P and the O^T accumulators (fp32, 32 x D) all live
//    in arch VGPRs.  The kernel also builds as 4 waves of 64 rows (QT = 2, O
//    in the accumulation registers, Q8 read from LDS), which halves LDS
//    operand traffic but leaves the compiler copying accumulators between
//    register files.
//  * K8 and V^T tiles of 64 keys are staged through LDS for all the waves:
//    the loads of tile j+2 are issued at the top of iteration j and written to
//    LDS at its end (2 K buffers, 4 V^T buffers, one barrier per iteration).
//    V is transposed (and converted to the P.V type) while staged.
//  * Software pipeline inside each wave: iteration j runs the P.V MFMAs of
//    block j-1 together with the softmax of block j (VALU), then the QK MFMAs
//    of block j+1, so the matrix cores and the vector ALUs work at the same
//    time.  Blocks that need no mask take a path with no masking code.
//  * The i32 score accumulator starts at the bit pattern of 2^23 + 2^22, so
//    it reads as the float 12582912 + S (exact for |S| < 2^22 >= 127^2 * D):
//    dequantisation and max-subtraction are one FMA per score.
//  * Lazy rescale: the running max moves only when a block's max exceeds it
//    by more than tau (log2 units), so P stays bounded (SoftmaxCfg); the O
//    rescale that a move needs is applied at the start of the next
//    iteration, once the P.V MFMAs of the previous block have retired.
//  * The MFMA C layout (lane 32h + n holds column n, rows 8i + 4h + r) is used
//    as the B operand of the P.V product directly: P never leaves
//    registers.  V^T columns are stored in LDS in the order in which a lane
//    half holds the keys, so each A operand is one or two ds_read_b128.
//  * Work-group ids are remapped so that all q-blocks of one (batch, head)
//    run on one XCD (shared L2): the hardware deals work-groups to the 8 XCDs
//    round-robin.
#include <stdlib.h>

#include "sage_device.h"

namespace sage {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

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

constexpr int kBM = 256;  // query rows per work-group
constexpr int kBN = 64;   // keys per block
constexpr int kKBuf = 2, kVBuf = 4;

// The int32 MFMA accumulator starts at the bit pattern of 2^23 + 2^22.
constexpr int kMagicI = 0x4B400000;
constexpr float kMagicF = 12582912.0f;

// Lazy rescale threshold (log2 units) and the power of two P is scaled by
// before rounding to the P.V type.  fp16/bf16: P = 2^(s-m) <= 2^8.  FP8 e4m3
// (normal from 2^-6, max 448): P = 2^(s-m+6) <= 2^8 with tau = 2, so every
// score within 12 of the running max rounds to a normal number.  The row
// sums use the same scaled P, so the scale cancels in O / l.
template <int M>
struct SoftmaxCfg {
  static constexpr float kTau = 8.0f, kShift = 0.0f;
};
template <>
struct SoftmaxCfg<SAGE_PV_FP8> {
  static constexpr float kTau = 2.0f, kShift = 6.0f;
};

// ---------------------------------------------------------------------------
// P.V operand types
// ---------------------------------------------------------------------------
template <int M>
struct PvT;
template <>
struct PvT<SAGE_PV_F16> {
  static constexpr int kEB = 2;   // bytes per V^T element in LDS
  static constexpr int kPW = 16;  // P dwords per lane per (block, q tile)
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, h2));
  }
  __device__ static __forceinline__ v16f mma(const v4i& a, const v4i& b, const v16f& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0,
                                                  0);
  }
};
template <>
struct PvT<SAGE_PV_BF16> {
  static constexpr int kEB = 2;
  static constexpr int kPW = 16;
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, bf2));
  }
  __device__ static __forceinline__ v16f mma(const v4i& a, const v4i& b, const v16f& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0,
                                                   0, 0);
  }
};
template <>
struct PvT<SAGE_PV_FP8> {
  static constexpr int kEB = 1;
  static constexpr int kPW = 8;
  // two fp32 -> two OCP e4m3 bytes (round to nearest even) in the low or high half
  __device__ static __forceinline__ uint32_t pack4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
  }
  __device__ static __forceinline__ v16f mma(const v8i& a, const v8i& b, const v16f& c) {
    // format 0 (e4m3) for both operands, unit E8M0 scales (127 = 2^0)
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
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
  v2i w = {(int)PvT<SAGE_PV_F16>::pack2(a, b), (int)PvT<SAGE_PV_F16>::pack2(c, d)};
  *reinterpret_cast<v2i*>(p) = w;
}
template <>
__device__ __forceinline__ void store4<__bf16>(__bf16* p, float a, float b, float c, float d) {
  v2i w = {(int)PvT<SAGE_PV_BF16>::pack2(a, b), (int)PvT<SAGE_PV_BF16>::pack2(c, d)};
  *reinterpret_cast<v2i*>(p) = w;
}

__device__ __forceinline__ int remap_xcd(int w, int n) {
  const int per = n >> 3, rem = n & 7;
  const int xcd = w & 7, loc = w >> 3;
  return xcd * per + min(xcd, rem) + loc;
}

// value of the partner lane l ^ 32 (the other half of a 32x32 C column)
__device__ __forceinline__ int max_halves(int v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((int)a[0], (int)a[1]);
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float((int)a[0]) + __int_as_float((int)a[1]);
}

// 4x4 byte transpose: out[i] = byte i of a, b, c, d
__device__ __forceinline__ void transpose4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&o)[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const uint32_t t1 = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const uint32_t t2 = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
  const uint32_t t3 = __builtin_amdgcn_perm(d, c, 0x07030602u);  // c2 d2 c3 d3
  o[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// LDS column of the 4-key group kg (keys 4kg..4kg+3) of a V^T tile, in units
// of 4 keys.  Key 32t + 8i + 4h + r sits at S^T row i*8 + 4h + r of key tile t,
// i.e. in register 4i + r of lane half h; lane half h reads its 32 keys
// contiguously from column 32h + 16t + 4i + r.
__device__ __forceinline__ int vcol4(int kg) { return 8 * (kg & 1) + 4 * (kg >> 3) + ((kg >> 1) & 3); }

// V staging source per P.V mode: TV elements (converted) or e4m3 codes
template <typename TV, int PVM>
struct VStage {
  Raw8<TV> r[4];  // 4 keys x 8 channels
};
template <typename TV>
struct VStage<TV, SAGE_PV_FP8> {
  uint4 r[4];  // 4 keys x 16 channels of e4m3 codes
};

// QT 32-row q tiles per wave: QT = 1 -> 8 waves (2 per SIMD), everything in
// arch VGPRs; QT = 2 -> 4 waves (1 per SIMD), O in the accumulation registers.
template <int D, int QT, typename TV, int PVM, typename TO>
__global__ __launch_bounds__(512 / QT) __attribute__((amdgpu_waves_per_eu(2 / QT, 2 / QT))) void attn_fwd_kernel(
    AttnArgs a) {
  constexpr int NW = 8 / QT;      // waves per work-group
  constexpr int NT = 64 * NW;     // threads per work-group
  constexpr int QW = 32 * QT;     // query rows per wave
  constexpr bool kQReg = QT == 1; // Q8 operand kept in registers (else read from LDS)
  constexpr bool kF8 = PVM == SAGE_PV_FP8;
  using Pv = PvT<PVM>;
  constexpr int KC = D / 32;          // 32-byte slices of the QK contraction
  constexpr int DT = D / 32;          // 32-row d tiles of O^T
  constexpr int PW = Pv::kPW;         // P dwords per lane per q tile
  constexpr int KP = D + 16;          // K8 tile row pitch (bytes)
  constexpr int VP = 64 * Pv::kEB + 16;  // V^T tile row pitch (bytes)
  constexpr int KTB = kBN * KP;
  constexpr int VTB = D * VP;
  constexpr int KCPR = D / 16;        // 16-byte chunks per K8 row
  constexpr int KCH = kBN * KCPR;     // 16-byte chunks per K8 tile
  constexpr int KCH_T = (KCH + NT - 1) / NT;
  constexpr int VCW = kF8 ? 16 : 8;   // channels per V micro-tile (4 keys each)
  constexpr int VMT = (kBN / 4) * (D / VCW);  // V micro-tiles per tile
  static_assert(KCH % NT == 0 || KCH < NT, "K staging");
  static_assert(VMT <= NT, "V staging: one micro-tile per thread");

  constexpr int QTB = kQReg ? 0 : kBM * KP;  // bytes of the work-group's Q8 rows in LDS
  __shared__ __attribute__((aligned(16))) char smem[QTB + kKBuf * KTB + kVBuf * VTB];
  __shared__ float ksc_s[kKBuf];
  char* const qbuf = smem;
  char* const kbuf0 = smem + QTB;
  char* const vbuf0 = smem + QTB + kKBuf * KTB;

  const int nqb = (a.Nq + kBM - 1) / kBM;
  const int wg = remap_xcd((int)blockIdx.x, (int)gridDim.x);
  int qb = wg % nqb;
  const int h = (wg / nqb) % a.Hq;
  const int b = wg / (nqb * a.Hq);
  if (a.causal) qb = nqb - 1 - qb;  // longest rows first
  const int hk = h / (a.Hq / a.Hkv);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hh = lane >> 5, n = lane & 31;
  const int q0 = qb * kBM;
  const int qa = q0 + wave * QW;  // first q row of this wave

  const int8_t* qbase = a.q8 + b * a.sq[0] + h * a.sq[1];
  const int8_t* kbase = a.k8 + b * a.sk[0] + hk * a.sk[1];
  const float* ksc_base = a.k_scale + ((int64_t)b * a.Hkv + hk) * a.nks;

  // ---- Q8 (B operand of S^T = K Q^T): rows qa + 32s + n, bytes 32c + 16hh.
  // Held in registers (QT = 1) or staged in LDS for the work-group (row pitch
  // KP).  Rows past Nq read the last row; their results are never stored.
  v4i qreg[QT][KC];
  if constexpr (kQReg) {
#pragma unroll
    for (int s = 0; s < QT; ++s) {
      const int row = min(qa + 32 * s + n, a.Nq - 1);
#pragma unroll
      for (int c = 0; c < KC; ++c)
        qreg[s][c] = *reinterpret_cast<const v4i*>(qbase + (uint32_t)(row * a.sqn + 32 * c + 16 * hh));
    }
  } else {
#pragma unroll
    for (int i = 0; i < (kBM * KCPR) / NT; ++i) {
      const int L = tid + i * NT;
      const int row = min(q0 + L / KCPR, a.Nq - 1);
      *reinterpret_cast<v4i*>(qbuf + (L / KCPR) * KP + 16 * (L % KCPR)) =
          *reinterpret_cast<const v4i*>(qbase + (uint32_t)(row * a.sqn + 16 * (L % KCPR)));
    }
  }
  float qsc[QT];
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    const int si = min((qa + 32 * s) / a.q_sub, a.nqs - 1);
    qsc[s] = a.q_scale[((int64_t)b * a.Hq + h) * a.nqs + si];
  }

  // ---- key blocks of the work-group and of this wave
  const int nkb_all = (a.Nkv + kBN - 1) / kBN;
  int nkb = nkb_all;
  if (a.causal) nkb = min(nkb_all, (min(q0 + kBM, a.Nq) - 1) / kBN + 1);
  const int q_last = min(qa + QW, a.Nq) - 1;  // last valid row of this wave (< qa if none)
  int jmax = nkb - 1;                           // last block this wave computes
  if (q_last < qa) jmax = -1;
  else if (a.causal) jmax = min(jmax, q_last / kBN);
  // leading blocks that need no mask: whole 64 keys inside Nkv and, when
  // causal, every key <= the wave's first row
  int nfull = a.Nkv / kBN;
  if (a.causal) nfull = min(nfull, qa / kBN);
  nfull = min(nfull, jmax + 1);

  // ---- staging: K8 chunk L = tid + i*256 -> row L / KCPR, chunk L % KCPR;
  // V micro-tile m = tid -> keys 4*(m % 16) .. +4, channels VCW*(m / 16) .. +VCW.
  // Keys past Nkv read the last key: their P is 0 and the data is finite.
  v4i kst[KCH_T];
  VStage<TV, PVM> vst;
  float kscst = 0.0f;
  const int vkg = tid & 15, vcg = tid >> 4;
  auto load_tile = [&](int j) __attribute__((always_inline)) {
    const int k0 = j * kBN;
    if (tid == 0) kscst = ksc_base[min(j >> a.blkk_shift, a.nks - 1)];
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      const int L = tid + i * NT;
      if (KCH % NT == 0 || L < KCH) {
        const int row = min(k0 + L / KCPR, a.Nkv - 1);
        kst[i] = *reinterpret_cast<const v4i*>(kbase + (uint32_t)(row * a.skn + 16 * (L % KCPR)));
      }
    }
    if (VMT == NT || tid < VMT) {
      if constexpr (kF8) {
        const uint8_t* vb = static_cast<const uint8_t*>(a.v) + b * a.sv[0] + hk * a.sv[1];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          vst.r[r] = *reinterpret_cast<const uint4*>(vb + (uint32_t)(min(k0 + 4 * vkg + r, a.Nkv - 1) * a.svn +
                                                                      VCW * vcg));
      } else {
        const TV* vb = static_cast<const TV*>(a.v) + b * a.sv[0] + hk * a.sv[1];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          vst.r[r] = load8<TV>(vb + (uint32_t)(min(k0 + 4 * vkg + r, a.Nkv - 1) * a.svn + VCW * vcg));
      }
    }
  };
  auto store_tile = [&](int j) __attribute__((always_inline)) {
    char* ks = kbuf0 + (j & 1) * KTB;
    char* vs = vbuf0 + (j & 3) * VTB;
    if (tid == 0) ksc_s[j & 1] = kscst;
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      const int L = tid + i * NT;
      if (KCH % NT == 0 || L < KCH)
        *reinterpret_cast<v4i*>(ks + (L / KCPR) * KP + 16 * (L % KCPR)) = kst[i];
    }
    if (VMT == NT || tid < VMT) {
      char* dst = vs + VCW * vcg * VP + 4 * Pv::kEB * vcol4(vkg);
      if constexpr (kF8) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t t[4];
          transpose4x4(word(vst.r[0], w), word(vst.r[1], w), word(vst.r[2], w), word(vst.r[3], w), t);
#pragma unroll
          for (int e = 0; e < 4; ++e) *reinterpret_cast<uint32_t*>(dst + (4 * w + e) * VP) = t[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v2i w = {(int)Pv::pack2(elem<TV>(vst.r[0], e), elem<TV>(vst.r[1], e)),
                   (int)Pv::pack2(elem<TV>(vst.r[2], e), elem<TV>(vst.r[3], e))};
          *reinterpret_cast<v2i*>(dst + e * VP) = w;
        }
      }
    }
  };

  // ---- accumulators and softmax state
  v16f oacc[DT][QT];
  float m_use[QT], lsum[QT], alpha_o[QT];  // lsum: this lane's share of the row sums
#pragma unroll
  for (int s = 0; s < QT; ++s) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt][s] = (v16f){};
    m_use[s] = -INFINITY;
    lsum[s] = 0.0f;
    alpha_o[s] = 1.0f;
  }
  bool pend = false;  // O must be multiplied by alpha_o before the next P.V
  v16i S[2][QT];      // S^T of key tile t, q tile s
  float ksc_cur = 0.0f;           // k scale of the block held in S
  uint32_t Pprev[QT][PW], Pcur[QT][PW];  // P of blocks j-1 and j
  const v16i magic = {kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI,
                      kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI};

  // ---- building blocks
  // S^T of block j (its K8 tile in buffer j & 1)
  // Q operand (s, c): row 32s + n of the wave's rows, bytes 32c + 16hh .. +16
  const char* qrd = qbuf + (wave * QW + n) * KP + 16 * hh;
  auto qk = [&](int j) __attribute__((always_inline)) {
    const char* ks = kbuf0 + (j & 1) * KTB + n * KP + 16 * hh;
    ksc_cur = ksc_s[j & 1];
    v4i qb[QT][KC];
#pragma unroll
    for (int s = 0; s < QT; ++s)
#pragma unroll
      for (int c = 0; c < KC; ++c)
        qb[s][c] = kQReg ? qreg[s][c] : *reinterpret_cast<const v4i*>(qrd + 32 * s * KP + 32 * c);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      v4i ka[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c) ka[c] = *reinterpret_cast<const v4i*>(ks + 32 * t * KP + 32 * c);
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int s = 0; s < QT; ++s)
          S[t][s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka[c], qb[s][c], c == 0 ? magic : S[t][s], 0, 0, 0);
    }
  };
  // O^T += V^T P^T of block j (its V^T tile in buffer j & 3)
  auto pv = [&](int j, const uint32_t (&P)[QT][PW]) __attribute__((always_inline)) {
    const char* vs = vbuf0 + (j & 3) * VTB + n * VP;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const char* vr = vs + 32 * dt * VP;
      if constexpr (kF8) {
        const v4i lo = *reinterpret_cast<const v4i*>(vr + 32 * hh);
        const v4i hi = *reinterpret_cast<const v4i*>(vr + 32 * hh + 16);
        const v8i va = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int s = 0; s < QT; ++s) {
          const v8i pb = {(int)P[s][0], (int)P[s][1], (int)P[s][2], (int)P[s][3],
                          (int)P[s][4], (int)P[s][5], (int)P[s][6], (int)P[s][7]};
          oacc[dt][s] = Pv::mma(va, pb, oacc[dt][s]);
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {  // 16-key steps: key tile kk/2, register half kk%2
          const v4i va = *reinterpret_cast<const v4i*>(vr + 64 * hh + 16 * kk);
#pragma unroll
          for (int s = 0; s < QT; ++s) {
            const v4i pb = {(int)P[s][4 * kk], (int)P[s][4 * kk + 1], (int)P[s][4 * kk + 2], (int)P[s][4 * kk + 3]};
            oacc[dt][s] = Pv::mma(va, pb, oacc[dt][s]);
          }
        }
      }
    }
  };
  // key of register v of key tile t in this lane, relative to the block
  auto key_of = [&](int t, int v) __attribute__((always_inline)) {
    return 32 * t + 8 * (v >> 2) + 4 * hh + (v & 3);
  };
  auto key_ok = [&](int key, int qrow) __attribute__((always_inline)) {
    return key < a.Nkv && (!a.causal || key <= qrow);
  };
  // softmax of block j held in S -> P (and the running max / sums)
  auto softmax = [&](int j, uint32_t (&P)[QT][PW], bool masked) __attribute__((always_inline)) {
    const int k0 = j * kBN;
#pragma unroll
    for (int s = 0; s < QT; ++s) {
      const int qrow = qa + 32 * s + n;
      const float c = qsc[s] * ksc_cur;
      int mx = INT_MIN;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          int x = S[t][s][v];
          if (masked) x = key_ok(k0 + key_of(t, v), qrow) ? x : INT_MIN;
          mx = max(mx, x);
        }
      mx = max_halves(mx);
      const float mblk = mx == INT_MIN ? -INFINITY : (float)(mx - kMagicI) * c;
      // lazy max update (per q column; both lane halves agree)
      const bool need = mblk > m_use[s] + SoftmaxCfg<PVM>::kTau;
      const float mnew = need ? mblk : m_use[s];
      const float alpha = need ? __builtin_amdgcn_exp2f(m_use[s] - mnew) : 1.0f;
      m_use[s] = mnew;
      lsum[s] *= alpha;
      alpha_o[s] *= alpha;
      pend |= __builtin_amdgcn_ballot_w64(need) != 0;
      const float m = (mnew == -INFINITY ? 0.0f : mnew) - SoftmaxCfg<PVM>::kShift;
      const float bias = __builtin_fmaf(kMagicF, c, m);  // x = (2^23+2^22+S)*c - bias = S*c - m
      float ls = 0.0f;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float e = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(S[t][s][v]), c, -bias));
          if (masked) e = key_ok(k0 + key_of(t, v), qrow) ? e : 0.0f;
          p[v] = e;
          ls += e;
        }
        if constexpr (kF8) {
#pragma unroll
          for (int w = 0; w < 4; ++w) P[s][4 * t + w] = Pv::pack4(p[4 * w], p[4 * w + 1], p[4 * w + 2], p[4 * w + 3]);
        } else {
#pragma unroll
          for (int w = 0; w < 8; ++w) P[s][8 * t + w] = Pv::pack2(p[2 * w], p[2 * w + 1]);
        }
      }
      lsum[s] += ls;
    }
  };
  // scheduling pattern of the fast path: per d tile, its V^T reads, then
  // each P.V MFMA followed by a share of the softmax VALU work
  auto interleave = [&]() __attribute__((always_inline)) {
    constexpr int kMma = kF8 ? QT : 4 * QT;  // MFMAs per d tile
    constexpr int kRd = kF8 ? 2 : 4;         // ds_read_b128 per d tile
    constexpr int kValu = (150 * QT + DT * kMma - 1) / (DT * kMma);  // softmax VALU share per MFMA
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      __builtin_amdgcn_sched_group_barrier(0x100, kRd, 0);
#pragma unroll
      for (int m = 0; m < kMma; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
      }
    }
  };
  auto rescale_o = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < QT; ++s) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt][s] *= alpha_o[s];
      alpha_o[s] = 1.0f;
    }
  };

  // ---- one iteration: P.V of block j-1, softmax of block j, S of block j+1,
  // staging of tile j+2.  Iteration nkb only finishes the last P.V.
  // ---- iterations.  Iteration j: P.V of block j-1, softmax of block j, S of
  // block j+1, staging of tile j+2; iteration nkb only finishes the last P.V.
  // Every wave runs nkb + 1 iterations (one barrier each).  The mask-free
  // steady state has a loop of its own so that the O accumulators are
  // updated from one place in each loop.
  auto keep_p = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < QT; ++s)
#pragma unroll
      for (int w = 0; w < PW; ++w) Pprev[s][w] = Pcur[s][w];
  };
  auto finish = [&](int j, bool stage) __attribute__((always_inline)) {
    if (j + 1 <= jmax) qk(j + 1);
    if (stage) store_tile(j + 2);
    __syncthreads();
  };
  auto generic_iter = [&](int j) __attribute__((always_inline)) {
    const bool stage = j + 2 < nkb;
    if (stage) load_tile(j + 2);
    if (pend) {
      rescale_o();
      pend = false;
    }
    if (j >= 1 && j - 1 <= jmax) pv(j - 1, Pprev);
    __builtin_amdgcn_sched_barrier(0);
    if (j <= jmax) {
      if (j < nfull) softmax(j, Pcur, false);
      else softmax(j, Pcur, true);
      keep_p();
    }
    finish(j, stage);
  };
  // blocks 1 <= j < j_fast: P.V of block j-1 (MFMA) interleaved with the
  // softmax of block j (VALU); S of block j+1 and tile j+2 always exist.
  // The empty asm statements pin values where the pipeline needs them: P
  // computed before the QK MFMAs, S written to arch registers, O in the
  // accumulation registers across iterations.
  auto fast_iter = [&](int j) __attribute__((always_inline)) {
    load_tile(j + 2);
    if (pend) {
      rescale_o();
      pend = false;
    }
    pv(j - 1, Pprev);
    softmax(j, Pcur, false);
    interleave();
#pragma unroll
    for (int s = 0; s < QT; ++s)
#pragma unroll
      for (int w = 0; w < PW; ++w) asm volatile("" ::"v"(Pcur[s][w]));
    keep_p();
    qk(j + 1);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s = 0; s < QT; ++s) asm volatile("" : "+v"(S[t][s]));
    store_tile(j + 2);
    if constexpr (QT == 2) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int s = 0; s < QT; ++s) asm volatile("" : "+a"(oacc[dt][s]));
    }
    __syncthreads();
  };

  // ---- prologue: tiles 0 and 1 staged, S of block 0
  load_tile(0);
  store_tile(0);
  if (nkb > 1) {
    load_tile(1);
    store_tile(1);
  }
  __syncthreads();
  if (jmax >= 0) qk(0);
  __syncthreads();  // block 0's K8 buffer is restaged in iteration 0

  const int j_fast = min(min(nfull, jmax), nkb - 2);
  generic_iter(0);
  int j = 1;
  for (; j < j_fast; ++j) fast_iter(j);
  for (; j <= nkb; ++j) generic_iter(j);

  // ---- epilogue: O / l, store rows q = qa + 32s + n, d = 32dt + 8i + 4hh .. +4
  if (pend) rescale_o();
  TO* obase = static_cast<TO*>(a.o) + b * a.so[0] + h * a.so[1];
  const float* vsc = kF8 ? a.v_scale + ((int64_t)b * a.Hkv + hk) * D : nullptr;
#pragma unroll
  for (int s = 0; s < QT; ++s) {
    const float inv = 1.0f / sum_halves(lsum[s]);
    const int row = qa + 32 * s + n;
    if (row < a.Nq) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = 32 * dt + 8 * i + 4 * hh;
          float4 f = make_float4(inv, inv, inv, inv);
          if constexpr (kF8) {
            const float4 vs4 = *reinterpret_cast<const float4*>(vsc + d0);
            f = make_float4(inv * vs4.x, inv * vs4.y, inv * vs4.z, inv * vs4.w);
          }
          const v16f& o = oacc[dt][s];
          store4<TO>(obase + (uint32_t)(row * a.son + d0), o[4 * i] * f.x, o[4 * i + 1] * f.y, o[4 * i + 2] * f.z,
                     o[4 * i + 3] * f.w);
        }
    }
  }
}

template <int D, typename TV, int PVM, typename TO>
static int launch_cfg(const AttnArgs& a, hipStream_t st) {
  constexpr int QT = 1;
  const int64_t nqb = (a.Nq + kBM - 1) / kBM;
  const int64_t grid = nqb * a.Hq * a.B;
  if (grid > 0x7FFFFFFF) return fail("sage_attn_fwd: invalid argument: grid too large");
  hipLaunchKernelGGL((attn_fwd_kernel<D, QT, TV, PVM, TO>), dim3((unsigned)grid), dim3(512 / QT), 0, st, a);
  return check_launch("sage_attn_fwd");
}

template <typename TV, int PVM, typename TO>
static int launch_d(const AttnArgs& a, int D, hipStream_t st) {
  return D == 64 ? launch_cfg<64, TV, PVM, TO>(a, st) : launch_cfg<128, TV, PVM, TO>(a, st);
}

static bool strides_ok(const int64_t* s, int esize) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] * esize) % 16 != 0) return false;
  return true;
}

static bool is_float_code(int c) { return c == SAGE_DTYPE_F32 || c == SAGE_DTYPE_F16 || c == SAGE_DTYPE_BF16; }

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
  if (q_sub < 32 || q_sub % 32 != 0 || blkq % q_sub != 0)
    return fail("sage_attn_fwd: invalid argument: q_sub=%d blkq=%d (q_sub: a multiple of 32 dividing blkq)", q_sub,
                blkq);
  if (!q8 || !q_scale || !k8 || !k_scale || !v || !o || !q8_strides || !k8_strides || !v_strides || !o_strides)
    return fail("sage_attn_fwd: invalid argument: null pointer");
  if (pv_mode != SAGE_PV_F16 && pv_mode != SAGE_PV_BF16 && pv_mode != SAGE_PV_FP8)
    return fail("sage_attn_fwd: invalid argument: pv_mode %d", pv_mode);
  if (!is_float_code(o_dtype)) return fail("sage_attn_fwd: invalid argument: o_dtype %d", o_dtype);
  if (pv_mode == SAGE_PV_FP8) {
    if (v_dtype != SAGE_DTYPE_FP8E4M3 || !v_scale)
      return fail("sage_attn_fwd: invalid argument: FP8 P.V needs e4m3 V codes and v_scale");
  } else if (v_dtype != o_dtype) {
    return fail("sage_attn_fwd: invalid argument: v_dtype %d / o_dtype %d", v_dtype, o_dtype);
  }
  const int ves = v_dtype == SAGE_DTYPE_F32 ? 4 : (v_dtype == SAGE_DTYPE_FP8E4M3 ? 1 : 2);
  const int oes = o_dtype == SAGE_DTYPE_F32 ? 4 : 2;
  const bool rows32 = Nq * q8_strides[2] + D < 0x7FFFFFFF && Nkv * k8_strides[2] + D < 0x7FFFFFFF &&
                      Nkv * v_strides[2] + D < 0x7FFFFFFF && Nq * o_strides[2] + D < 0x7FFFFFFF;
  if (!rows32) return fail("sage_attn_fwd: invalid argument: a head's rows must span < 2^31 elements");
  if (!strides_ok(q8_strides, 1) || !strides_ok(k8_strides, 1) || !strides_ok(v_strides, ves) ||
      !strides_ok(o_strides, oes))
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
  const int d = (int)D;
  if (pv_mode == SAGE_PV_FP8) {
    switch (o_dtype) {
      case SAGE_DTYPE_F32: return launch_d<uint8_t, SAGE_PV_FP8, float>(a, d, st);
      case SAGE_DTYPE_F16: return launch_d<uint8_t, SAGE_PV_FP8, _Float16>(a, d, st);
      default: return launch_d<uint8_t, SAGE_PV_FP8, __bf16>(a, d, st);
    }
  }
  const bool bf = pv_mode == SAGE_PV_BF16;
  switch (v_dtype) {
    case SAGE_DTYPE_F32:
      return bf ? launch_d<float, SAGE_PV_BF16, float>(a, d, st) : launch_d<float, SAGE_PV_F16, float>(a, d, st);
    case SAGE_DTYPE_F16:
      return bf ? launch_d<_Float16, SAGE_PV_BF16, _Float16>(a, d, st)
                : launch_d<_Float16, SAGE_PV_F16, _Float16>(a, d, st);
    default:
      return bf ? launch_d<__bf16, SAGE_PV_BF16, __bf16>(a, d, st) : launch_d<__bf16, SAGE_PV_F16, __bf16>(a, d, st);
  }
}
