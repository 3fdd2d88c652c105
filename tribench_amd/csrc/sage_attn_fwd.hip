// sage_attn_fwd.hip — fused SageAttention forward for gfx950 (MI355X).
//
// Replaces _attn_fwd / _attn_fwd_inner (kernels/sage_attn/triton_impl.py:86-160)
// and its launch (:186-199); with fp16/bf16 Q and K instead of INT8 (no
// quantization, S in fp32 from v_mfma_f32_32x32x16_{f16,bf16}) the same
// kernel replaces _flash_attn_fwd_kernel (kernels/flash_attn/triton_impl.py:
// 12-101).  Per block of 64 keys:
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
//  * A work-group is 8 waves (2 per SIMD) of 32 query rows (one 32-row MFMA
//    tile each) of one (batch, head): Q8 rows, S, P and the O^T accumulators
//    (fp32, 32 x D) all live in arch VGPRs.
//  * K8 rows and V^T rows reach LDS in tiles of 64 keys by direct global ->
//    LDS loads (global_load_lds_dwordx4), three tiles ahead of their use, in a
//    ring of 5 slots: no staging registers and no VALU work.  V arrives
//    already converted and transposed (sage_vtiles), so a tile is a plain
//    copy.  The 16-byte chunks of each LDS row are XOR-swizzled so that the
//    operand reads of 16 consecutive lanes (rows) hit distinct banks.
//  * Each wave waits (vmcnt) for exactly its own loads of the tile the next
//    iteration reads, then meets the others at a barrier without a memory
//    fence (__syncthreads' fence would drain the whole prefetch).
//  * Software pipeline inside each wave: iteration j runs the P.V MFMAs of
//    block j-1 together with the softmax of block j (VALU), then the QK MFMAs
//    of block j+1.  Blocks that need no mask take a path with no masking code.
//  * The i32 score accumulator starts at the bit pattern of 2^23 + 2^22, so
//    it reads as the float 12582912 + S (exact for |S| < 2^22 >= 127^2 * D):
//    dequantisation and max-subtraction are one FMA per score, rounded once
//    (the scale trimmed to 21 bits and the running max kept on a grid make
//    its bias exact).
//  * Lazy rescale: the running max moves only when a block's max exceeds it
//    by more than tau (log2 units), so P stays bounded (SoftmaxCfg); the O
//    rescale that a move needs is applied at the start of the next
//    iteration, once the P.V MFMAs of the previous block have retired.
//  * The MFMA C layout (lane 32h + n holds column n, rows 8i + 4h + r) is used
//    as the B operand of the P.V product directly: P never leaves
//    registers.  The V tiles store keys in the order a lane half holds them,
//    so each A operand is one or two ds_read_b128.
//  * Work-group ids are remapped so that all q-blocks of one (batch, head)
//    run on one XCD (shared L2): the hardware deals work-groups to the 8 XCDs
//    round-robin.
#include <type_traits>

#include "sage_device.h"

// SAGE_TRACE (a measurement build only, libsage_attn_trace.so): every wave
// records s_memtime at its phase boundaries and the cycles it spends at the
// per-iteration barrier into a buffer attached with sage_trace_attach().
#ifndef SAGE_TRACE
#define SAGE_TRACE 0
#endif

namespace sage {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct AttnArgs {
  const void* q8;         // INT8 Q (or fp16/bf16 Q of the unquantized kernel)
  const float* q_scale;
  const void* k8;         // INT8 K (or fp16/bf16 K)
  const float* k_scale;
  const void* v;          // V tiles (sage_vtiles layout)
  const float* v_scale;
  void* o;
  int64_t sq[2], sk[2], so[2];  // batch and head strides (elements)
  int sqn, skn, son;            // row strides (elements); row offsets fit 32 bits
  int B, Hq, Hkv, Nq, Nkv;
  int causal;
  int q_sub, blkk_shift;  // k scale of key block j: k_scale[j >> blkk_shift]
  int nqs, nks;           // q / k scales per head
  float qk_mul;           // unquantized kernel: score multiplier, fp32(sm_scale * log2(e))
  float q_mul;            // Q quantized here: its multiplier, fp32(sm_scale * 1.44269504)
  int8_t* q8_out;         // Q quantized here: optional copies of Q8 (q's strides) and q_scale
  float* qs_out;
#if SAGE_TRACE
  unsigned long long* trace;  // kTraceWords per wave, indexed by (blockIdx.x, wave)
#endif
};

#if SAGE_TRACE
// Words per wave of the phase trace: s_memtime at entry, end of the prologue
// (before iteration 0), after iteration 0, after the mask-free loops, after
// the generic iterations and after the epilogue's stores [0..5]; barrier wait
// cycles over all iterations [6] and in the mask-free loops [7]; barrier
// counts, all and mask-free [8]; s_memrealtime (100 MHz) at entry and exit
// [9, 10]; HW_ID and XCC_ID [11]; the work-group's remapped index [12];
// s_memtime after the prologue's Q quantization (its Q rows awaited) and
// after its tile wait [13, 14].
constexpr int kTraceWords = 16;

// the stamps' LDS (a function-scope array: only the kernels that call this
// allocate it)
template <int NW>
__device__ __forceinline__ unsigned long long* trace_lds() {
  __shared__ unsigned long long s[NW * kTraceWords];
  return s;
}
#endif

// Operand type of the QK product: INT8 with per-block scales (SageAttention;
// Q quantized by the pre-pass, or here from Q in the output type), or
// fp16 / bf16 (plain attention, no scales).
constexpr int kQkI8 = 0, kQkF16 = 1, kQkBF16 = 2, kQkI8Q = 3;

constexpr int kBN = 64;  // keys per block

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

// The same for work-groups of unequal length (causal).  Each XCD's
// dispatcher places its work-groups in order and deals them to its four
// shader engines in turn (local index mod 4), waiting for a free CU in the
// engine whose turn it is.  With lengths falling along the order, the engine
// that receives the longest of every four holds the others back (measured:
// consecutive work-groups on one CU 7.4 us apart at config 3, 0.5 us with
// equal lengths).  Every second complete group of four is taken in reverse,
// so that the engines receive equal work.
__device__ __forceinline__ int remap_xcd_snake(int w, int n) {
  const int per = n >> 3, rem = n & 7;
  const int xcd = w & 7;
  int loc = w >> 3;
  const int g = loc >> 2;
  if ((g & 1) && 4 * g + 3 < per + (xcd < rem ? 1 : 0)) loc = 4 * g + 3 - (loc & 3);
  return xcd * per + min(xcd, rem) + loc;
}

// value of the partner lane l ^ 32 (the other half of a 32x32 C column)
__device__ __forceinline__ int max_halves(int v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((int)a[0], (int)a[1]);
}
__device__ __forceinline__ float max_halves_f(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float((int)a[0]), __int_as_float((int)a[1]));
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float((int)a[0]) + __int_as_float((int)a[1]);
}

// s_waitcnt vmcnt(n) alone (gfx9 encoding: expcnt and lgkmcnt at their maxima)
#define SAGE_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
#define SAGE_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)

// Work-group barrier without the memory fence of __syncthreads(): the fence
// would drain every direct-to-LDS load in flight, i.e. the whole prefetch.
// Callers wait for exactly the loads and LDS reads that must be complete.
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// XOR swizzle of the 16-byte chunks of an LDS row of RB bytes: chunk c of row
// r is stored at chunk c ^ swz<RB>(r).  For a column read by 16 consecutive
// lanes (16 consecutive rows), every lane then hits its own 4 banks.
template <int RB>
__device__ __forceinline__ int swz(int r) {
  return (r / (256 / RB)) & (RB / 16 - 1);
}

typedef __attribute__((address_space(1))) const void gmem_t;
typedef __attribute__((address_space(3))) void lmem_t;

// One work-group: 8 waves (2 per SIMD) of 32 query rows (one 32-row MFMA tile
// each) of one (batch, head); Q rows, S, P and the O^T accumulators live in
// arch VGPRs.  Tiles of 64 keys (K rows and V^T rows) reach LDS by direct
// global -> LDS loads, three tiles ahead of their use, in a ring of 5.
template <int QKM, int D, int PVM, typename TO>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_kernel(AttnArgs a) {
  constexpr int NW = 8;
  constexpr int BM = 256;  // query rows per work-group
  constexpr bool kFQ = QKM == kQkI8Q;  // Q quantized in the prologue
  constexpr bool kI8 = QKM == kQkI8 || kFQ;
  constexpr bool kF8 = PVM == SAGE_PV_FP8;
  using Pv = PvT<PVM>;
  using SAcc = std::conditional_t<kI8, v16i, v16f>;  // S^T accumulator of one 32-key tile
  constexpr int QEB = kI8 ? 1 : 2;  // bytes per Q8 / K element in the QK operands
  constexpr int EB = Pv::kEB;
  constexpr int KRB = D * QEB;      // K row bytes
  constexpr int KC = KRB / 32;      // 32-byte slices of a K row: one QK MFMA each
  constexpr int DT = D / 32;        // 32-row d tiles of O^T
  constexpr int PW = Pv::kPW;       // P dwords per lane
  constexpr int VRB = 64 * EB;      // V^T row bytes
  constexpr int KTB = kBN * KRB;    // K tile bytes
  constexpr int VTB = D * VRB;      // V^T tile bytes
  constexpr int SLOT = KTB + VTB;
  constexpr int NBUF = 5;           // tiles j-1 .. j+3 of iteration j
  constexpr int KLD = KTB / 1024;   // 1 KB wave loads per K8 tile
  constexpr int VLD = VTB / 1024;
  constexpr int LPW = (KLD + VLD + NW - 1) / NW;  // wave loads per wave per tile
  static_assert(LPW * NW >= KLD + VLD && LPW <= 15, "tile loads");
  constexpr int SINK = LPW * NW > KLD + VLD ? 1024 : 0;  // target of spare loads

  __shared__ __attribute__((aligned(1024))) char smem[NBUF * SLOT + SINK];
#if SAGE_TRACE
  // stamps go to LDS as they are taken (kept in registers they would change
  // the kernel being measured; a global store would enter the vmcnt
  // accounting of the tile loads) and to the trace buffer at the end.  A
  // kernel whose tile ring leaves no room for them is not traced.
  constexpr bool kTrace = NBUF * SLOT + SINK + NW * kTraceWords * 8 <= 160 * 1024;
  unsigned long long* tr_s = nullptr;
  if constexpr (kTrace) tr_s = trace_lds<NW>();
  // every lane stores the same wave-uniform value (no branch around the store)
  auto tr_put = [&](int i, unsigned long long v) __attribute__((always_inline)) {
    if constexpr (kTrace) tr_s[__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * kTraceWords + i] = v;
  };
  tr_put(0, __builtin_amdgcn_s_memtime());
  tr_put(9, __builtin_amdgcn_s_memrealtime());
  uint32_t tr_wait = 0, tr_wait_fast = 0, tr_n = 0;  // barrier cycles; counts (mask-free << 16)
#endif

  const int nqb = (a.Nq + BM - 1) / BM;
  int wg, qb, h, b;
  if (!a.causal) {  // all q-blocks of one (batch, head) on one XCD, in order
    wg = remap_xcd((int)blockIdx.x, (int)gridDim.x);
    qb = wg % nqb;
    h = (wg / nqb) % a.Hq;
    b = wg / (nqb * a.Hq);
  } else {
    // longest rows first, the q-blocks of two (batch, head)s in turn (the
    // length falls by one block every second work-group), engines balanced
    wg = remap_xcd_snake((int)blockIdx.x, (int)gridDim.x);
    const int nbh = a.B * a.Hq, pair = wg / (2 * nqb), r = wg - pair * 2 * nqb;
    const bool two = 2 * pair + 1 < nbh;
    const int bh = 2 * pair + (two ? (r & 1) : 0);
    qb = nqb - 1 - (two ? r >> 1 : r);
    h = bh % a.Hq;
    b = bh / a.Hq;
  }
  const int hk = h / (a.Hq / a.Hkv);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hh = lane >> 5, n = lane & 31;
  const int q0 = qb * BM;
  const int qa = q0 + wave * 32;  // first q row of this wave

  const char* qbase = static_cast<const char*>(a.q8) + (b * a.sq[0] + h * a.sq[1]) * (kFQ ? (int)sizeof(TO) : QEB);
  const char* kbase = static_cast<const char*>(a.k8) + (b * a.sk[0] + hk * a.sk[1]) * QEB;
  // k scales are read through the constant address space (scalar loads, which
  // the tile-load accounting on vmcnt does not see); the kernel never writes them
  typedef __attribute__((address_space(4))) const float cfloat_t;
  cfloat_t* ksc_base = (cfloat_t*)(a.k_scale + ((int64_t)b * a.Hkv + hk) * a.nks);
  const int ntile = (a.Nkv + kBN - 1) / kBN;
  const uint8_t* vtbase = static_cast<const uint8_t*>(a.v) + ((int64_t)b * a.Hkv + hk) * ntile * (int64_t)VTB;

  // ---- the largest k scale of the head (INT8), for the grid of the running
  // max below; loaded before every other load, so that waiting for it waits
  // for nothing else
  uint32_t ksc_max_bits = 0;  // positive floats order as their bit patterns
  if constexpr (kI8) {
    const float* ks = a.k_scale + ((int64_t)b * a.Hkv + hk) * a.nks;
    for (int i = lane; i < a.nks; i += 64) ksc_max_bits = max(ksc_max_bits, __float_as_uint(ks[i]));
  }

  // ---- Q, the B operand of S^T = K Q^T: row qa + n, bytes 32c + 16hh .. +16.
  // Rows past Nq read the last row; their results are never stored.
  v4i qreg[KC];
  float qsc = 1.0f;
  if constexpr (!kFQ) {
    const int row = min(qa + n, a.Nq - 1);
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qreg[c] = *reinterpret_cast<const v4i*>(qbase + (uint32_t)(row * a.sqn * QEB + 32 * c + 16 * hh));
    if constexpr (kI8) {  // q_sub == 1: one scale per row, i.e. per lane column
      const int qi = a.q_sub == 1 ? qa + n : qa / a.q_sub;
      qsc = a.q_scale[((int64_t)b * a.Hq + h) * a.nqs + min(qi, a.nqs - 1)];
    }
  }
  // Q quantized here (kFQ): its raw rows are requested now, the quantization
  // runs in the prologue once the first tiles are requested too, so the Q
  // load latency overlaps theirs.  Lane (n, hh) holds elements 32c + 16hh ..
  // +16 of row qa + n, exactly the bytes of its Q8 operand.
  Raw8<TO> qraw[kFQ ? KC : 1][2];
  if constexpr (kFQ) {
    const TO* qr = reinterpret_cast<const TO*>(qbase) + (int64_t)min(qa + n, a.Nq - 1) * a.sqn;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      qraw[c][0] = load8<TO>(qr + 32 * c + 16 * hh);
      qraw[c][1] = load8<TO>(qr + 32 * c + 16 * hh + 8);
    }
  }

  // ---- key blocks of the work-group and of this wave
  const int nkb_all = ntile;
  int nkb = nkb_all;
  if (a.causal) nkb = min(nkb_all, (min(q0 + BM, a.Nq) - 1) / kBN + 1);
  const int q_last = min(qa + 32, a.Nq) - 1;  // last valid row of this wave (< qa if none)
  int jmax = nkb - 1;                          // last block this wave computes
  if (q_last < qa) jmax = -1;
  else if (a.causal) jmax = min(jmax, q_last / kBN);
  // leading blocks that need no mask: whole 64 keys inside Nkv and, when
  // causal, every key <= the wave's first row
  int nfull = a.Nkv / kBN;
  if (a.causal) nfull = min(nfull, (qa + 1) / kBN);
  nfull = min(nfull, jmax + 1);

  // ---- tile loads.  Wave load g = wave + 8i (i < LPW) of a tile is the 1 KB
  // LDS range [1024g, 1024g + 1024) of its slot (K8 rows first, then V^T rows);
  // lane l brings the 16-byte chunk that lands at offset 16l, i.e. the logical
  // chunk (physical chunk ^ swizzle of its row).  K8 rows past Nkv read the
  // last row (their P is 0); V^T tiles are zero past Nkv.  Loads past the
  // tile go to the sink, so every wave issues LPW loads per tile.
  auto load_tile = [&](int j, int sl) __attribute__((always_inline)) {  // sl = j % NBUF
    char* slot = smem + sl * SLOT;
    const int k0 = j * kBN;
    const uint8_t* vt = vtbase + (int64_t)j * VTB;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int g = wave + NW * i;  // wave-uniform
      const void* src;
      char* dst;
      if (g < KLD) {
        const int p = 64 * g + lane;
        const int r = p / (KRB / 16), pc = p % (KRB / 16);
        const int row = min(k0 + r, a.Nkv - 1);
        src = kbase + (uint32_t)(row * a.skn * QEB + 16 * (pc ^ swz<KRB>(r)));
        dst = slot + 1024 * g;
      } else if (g < KLD + VLD) {
        const int p = 64 * (g - KLD) + lane;
        const int d = p / (VRB / 16), pc = p % (VRB / 16);
        src = vt + d * VRB + 16 * (pc ^ swz<VRB>(d));
        dst = slot + KTB + 1024 * (g - KLD);
      } else {  // only when SINK > 0
        src = kbase;
        dst = smem + NBUF * SLOT;
      }
      __builtin_amdgcn_global_load_lds((gmem_t*)src, (lmem_t*)dst, 16, 0, 0);
    }
  };
  // Tile loads of the mask-free loop: only whole K tiles (every row < Nkv),
  // so each of the wave's LPW loads is a uniform tile base plus a lane offset
  // that does not change from tile to tile.
  uint32_t foff[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int g = wave + NW * i;
    if (g < KLD) {
      const int p = 64 * g + lane;
      const int r = p / (KRB / 16), pc = p % (KRB / 16);
      foff[i] = (uint32_t)(r * a.skn * QEB + 16 * (pc ^ swz<KRB>(r)));
    } else if (g < KLD + VLD) {
      const int p = 64 * (g - KLD) + lane;
      const int d = p / (VRB / 16), pc = p % (VRB / 16);
      foff[i] = (uint32_t)(d * VRB + 16 * (pc ^ swz<VRB>(d)));
    } else {
      foff[i] = 0;
    }
  }
  const int64_t ktile_bytes = (int64_t)kBN * a.skn * QEB;
  auto load_tile_fast = [&](int j, int sl) __attribute__((always_inline)) {  // sl = j % NBUF
    char* slot = smem + sl * SLOT;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int g = wave + NW * i;  // wave-uniform
      const char* base;
      char* dst;
      if (g < KLD) {
        base = kbase + j * ktile_bytes;
        dst = slot + 1024 * g;
      } else if (g < KLD + VLD) {
        base = reinterpret_cast<const char*>(vtbase) + (int64_t)j * VTB;
        dst = slot + KTB + 1024 * (g - KLD);
      } else {
        base = kbase;
        dst = smem + NBUF * SLOT;
      }
      __builtin_amdgcn_global_load_lds((gmem_t*)(base + foff[i]), (lmem_t*)dst, 16, 0, 0);
    }
  };
  // end of an iteration: this wave's loads of the tile needed next are done
  // (at most `ahead` younger tiles in flight), its LDS reads are done, barrier
  // (fast: called from the mask-free loops, for the trace's split)
  auto sync_tiles = [&](bool ahead, bool fast = false) __attribute__((always_inline)) {
    if (ahead) SAGE_WAIT_VM(LPW);
    else SAGE_WAIT_VM(0);
#if SAGE_TRACE >= 2
    const unsigned long long tb = __builtin_amdgcn_s_memtime();
#endif
    SAGE_WAIT_LGKM0();
    wg_barrier();
#if SAGE_TRACE >= 2
    const uint32_t dt = (uint32_t)(__builtin_amdgcn_s_memtime() - tb);
    tr_wait += dt;
    tr_n += fast ? 0x10001u : 1u;
    if (fast) tr_wait_fast += dt;
#endif
  };

  // ---- INT8 scores in one FMA, rounded once.  With the accumulator read as
  // F = kMagicF + S, s * c - m = F * c - (kMagicF * c + m): the FMA gives the
  // correctly rounded s * c - m when the bias kMagicF * c + m is exact.  It is
  // when c has at most 21 significant bits (kMagicF = 3 * 2^22, so
  // kMagicF * c has at most 23 and is an even multiple of its ulp), m is a
  // multiple of mgrid = 4 ulp(kMagicF * c_max), c_max the lane's largest c, and
  // |m| < kMagicF * c; with a larger |m| the bias is within an ulp of m.  c21
  // truncates q_scale * k_scale to 21 bits (a relative change below 2^-21),
  // and the running max moves on the grid, rounded up (P only shrinks, by
  // less than 2^mgrid).  The grid is at most 1 (log2 units), which covers
  // c_max up to about 0.16; beyond, the bias is within an ulp of
  // kMagicF * c (scores that coarse make the softmax nearly one-hot).
  // Rounded once per block instead, the bias would shift each block's scores
  // by up to 0.75 c log2 units, differently from block to block.
  auto c21 = [](float c) __attribute__((always_inline)) { return __uint_as_float(__float_as_uint(c) & ~3u); };
  float mgrid = 1.0f, mgrid_inv = 1.0f;  // set once Q's scale is known

  // ---- accumulators and softmax state
  v16f oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = (v16f){};
  float m_use = -INFINITY;
  float lsum = 0.0f;     // this lane's share of the row sum
  // FP8 P: the row sums come from the matrix pipe, one more P.V MFMA per
  // block with an all-ones A operand (e4m3 1.0 = 0x38): every row of osum is
  // the sum of the block's e4m3 P, accumulated in fp32 and rescaled with O.
  // It replaces 32 fp32 additions per lane and block on the VALU, which sets
  // the FP8 loop's pace, and sums exactly the P the P.V product uses.
  constexpr bool kSumMfma = kF8;
  v16f osum = (v16f){};
  v8i ones8 = {0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838};
  if constexpr (kSumMfma) asm volatile("" : "+v"(ones8));
  float alpha_o = 1.0f;  // pending factor of O
  bool pend = false;     // O must be multiplied by alpha_o before the next P.V
  SAcc S[2];             // S^T of key tiles 0 and 1 of the block in flight
  float ksc_cur = 0.0f;  // k scale of the block held in S (INT8)
  uint32_t Pprev[PW], Pcur[PW];  // P of blocks j-1 and j
  v16i magic = {kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI,
                kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI};
  // held in VGPRs for the whole kernel, so that the first MFMA of each S tile
  // reads it as srcC (the compiler would rebuild it from SGPRs every block);
  // measured faster with FP8 P and at D = 64, slower at D = 128 with fp16 P
  if constexpr (kI8 && (PVM == SAGE_PV_FP8 || D == 64)) asm volatile("" : "+v"(magic));

  // per-lane byte offsets of the swizzled operand chunks
  int koff[KC];  // K row 32t + n (swizzle independent of t), logical chunk 2c + hh
#pragma unroll
  for (int c = 0; c < KC; ++c) koff[c] = n * KRB + 16 * ((2 * c + hh) ^ swz<KRB>(n));
  constexpr int VCH = kF8 ? 2 : 4;  // chunks of a V^T operand read per d tile
  int voff[VCH];  // V^T row 32dt + n (swizzle independent of dt)
#pragma unroll
  for (int c = 0; c < VCH; ++c) voff[c] = KTB + n * VRB + 16 * ((VCH * hh + c) ^ swz<VRB>(n));

  // ---- building blocks
  // S^T of block j (its K tile in slot j % NBUF): K row 32t + n, bytes 32c + 16hh
  // (into the S buffer Sd, its k scale into kd)
  auto qk_into = [&](int j, int sl, SAcc (&Sd)[2], float& kd) __attribute__((always_inline)) {  // sl = j % NBUF
    const char* ks = smem + sl * SLOT;
    if constexpr (kI8) kd = ksc_base[min(j >> a.blkk_shift, a.nks - 1)];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      v4i ka[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c) ka[c] = *reinterpret_cast<const v4i*>(ks + 32 * t * KRB + koff[c]);
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        if constexpr (kI8) {
          Sd[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka[c], qreg[c], c == 0 ? magic : Sd[t], 0, 0, 0);
        } else if constexpr (QKM == kQkF16) {
          Sd[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, ka[c]), __builtin_bit_cast(v8h, qreg[c]),
                                                         c == 0 ? (v16f){} : Sd[t], 0, 0, 0);
        } else {
          Sd[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ka[c]),
                                                          __builtin_bit_cast(v8bf, qreg[c]), c == 0 ? (v16f){} : Sd[t],
                                                          0, 0, 0);
        }
      }
    }
  };
  auto qk = [&](int j, int sl) __attribute__((always_inline)) { qk_into(j, sl, S, ksc_cur); };
  // O^T += V^T P^T of block j (its V^T tile in slot j % NBUF)
  auto pv = [&](int sl, const uint32_t (&P)[PW]) __attribute__((always_inline)) {  // sl = j % NBUF
    const char* vs = smem + sl * SLOT;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const char* vr = vs + 32 * dt * VRB;
      if constexpr (kF8) {
        const v4i lo = *reinterpret_cast<const v4i*>(vr + voff[0]);
        const v4i hi = *reinterpret_cast<const v4i*>(vr + voff[1]);
        const v8i va = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        const v8i pb = {(int)P[0], (int)P[1], (int)P[2], (int)P[3], (int)P[4], (int)P[5], (int)P[6], (int)P[7]};
        oacc[dt] = Pv::mma(va, pb, oacc[dt]);
        if constexpr (kSumMfma)
          if (dt == DT - 1) osum = Pv::mma(ones8, pb, osum);
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {  // 16-key steps: key tile kk/2, register half kk%2
          const v4i va = *reinterpret_cast<const v4i*>(vr + voff[kk]);
          const v4i pb = {(int)P[4 * kk], (int)P[4 * kk + 1], (int)P[4 * kk + 2], (int)P[4 * kk + 3]};
          oacc[dt] = Pv::mma(va, pb, oacc[dt]);
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
  // softmax of block j held in S -> P (and the running max / sums).  Max and
  // sum are pairwise trees, not serial chains, to keep dependency depth low.
  // c > 0 scales S to log2 units: q_scale * k_scale (INT8) or qk_mul.
  // (softmax_on: of the S buffer Sx with k scale kx)
  auto softmax_on = [&](int j, uint32_t (&P)[PW], bool masked, const SAcc (&Sx)[2], float kx)
                        __attribute__((always_inline)) {
    const int k0 = j * kBN;
    const int qrow = qa + n;
    const float c = kI8 ? c21(qsc * kx) : a.qk_mul;
    float mblk;
    if constexpr (kI8) {
      int x[32];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          x[16 * t + v] = Sx[t][v];
          if (masked && !key_ok(k0 + key_of(t, v), qrow)) x[16 * t + v] = INT_MIN;
        }
#pragma unroll
      for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) x[i] = max(x[i], x[i + w]);
      const int mx = max_halves(x[0]);
      mblk = mx == INT_MIN ? -INFINITY : (float)(mx - kMagicI) * c;
    } else {
      float x[32];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          x[16 * t + v] = Sx[t][v];
          if (masked && !key_ok(k0 + key_of(t, v), qrow)) x[16 * t + v] = -INFINITY;
        }
#pragma unroll
      for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) x[i] = fmaxf(x[i], x[i + w]);
      mblk = max_halves_f(x[0]) * c;
    }
    // lazy max update (per q column; both lane halves agree)
    const bool need = mblk > m_use + SoftmaxCfg<PVM>::kTau;
    // INT8: m = mnew - kShift on the grid, rounded up (P only shrinks)
    const float mup = kI8 ? __builtin_ceilf((mblk - SoftmaxCfg<PVM>::kShift) * mgrid_inv) * mgrid + SoftmaxCfg<PVM>::kShift
                          : mblk;
    const float mnew = need ? mup : m_use;
    const float alpha = need ? __builtin_amdgcn_exp2f(m_use - mnew) : 1.0f;
    m_use = mnew;
    lsum *= alpha;
    alpha_o *= alpha;
    pend |= __builtin_amdgcn_ballot_w64(need) != 0;
    const float m = (mnew == -INFINITY ? 0.0f : mnew) - SoftmaxCfg<PVM>::kShift;
    // INT8: S reads as the float 2^23 + 2^22 + S, so S*c - m = that*c - bias,
    // the bias exact (see c21)
    const float bias = kI8 ? __builtin_fmaf(kMagicF, c, m) : m;
    // fp16 P: the row sum adds the fp16 values the P.V MFMAs consume, in a
    // packed fp16 tree (15 v_pk_add_f16 instead of 32 fp32 adds; P <= 2^kTau,
    // so the block's 32-term sum stays below 2^13 and its relative error below
    // 5 * 2^-11), then one dot2 adds it into the fp32 lsum
    constexpr bool kSumF16 = PVM == SAGE_PV_F16;
    float ls[2] = {0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float p[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float sv = kI8 ? __int_as_float((int)Sx[t][v]) : (float)Sx[t][v];
        float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv, c, -bias));
        if (masked) e = key_ok(k0 + key_of(t, v), qrow) ? e : 0.0f;
        p[v] = e;
      }
      if constexpr (kF8) {
#pragma unroll
        for (int w = 0; w < 4; ++w) P[4 * t + w] = Pv::pack4(p[4 * w], p[4 * w + 1], p[4 * w + 2], p[4 * w + 3]);
      } else {
#pragma unroll
        for (int w = 0; w < 8; ++w) P[8 * t + w] = Pv::pack2(p[2 * w], p[2 * w + 1]);
      }
      if constexpr (!kSumF16 && !kSumMfma) {
#pragma unroll
        for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
          for (int i = 0; i < w; ++i) p[i] += p[i + w];
        ls[t] = p[0];
      }
    }
    if constexpr (kSumF16) {
      h2 hs[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) hs[w] = __builtin_bit_cast(h2, P[w]) + __builtin_bit_cast(h2, P[8 + w]);
#pragma unroll
      for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) hs[i] = hs[i] + hs[i + w];
      lsum = __builtin_amdgcn_fdot2(hs[0], (h2){(_Float16)1.0f, (_Float16)1.0f}, lsum, false);
    } else if constexpr (!kSumMfma) {
      lsum += ls[0] + ls[1];
    }
  };
  auto softmax = [&](int j, uint32_t (&P)[PW], bool masked) __attribute__((always_inline)) {
    softmax_on(j, P, masked, S, ksc_cur);
  };
  // Mask-free block, row max not recomputed: P is formed against the running
  // max m_use straight away.  softmax() keeps m_use too unless the block max
  // exceeds it by more than kTau, that is unless some P exceeds
  // 2^(kTau + kShift).  A lane's partial row sum bounds each of its P (sums
  // of non-negative values, fp16 ones included, never fall below their
  // largest term), so if every lane's sum is at most 2^(kTau + kShift - 1)
  // the block max is within kTau of m_use and P and the new lsum are the
  // ones softmax() computes, bit for bit; nothing else changes.  The margin
  // covers the rounding of the scores (the INT8 bias is exact, or within an
  // ulp of m: see c21); an m_use of -inf (sums of +inf) and NaN
  // scores fail the test.  Otherwise softmax() redoes the block from the
  // untouched S.  Not used for FP8 P: with kShift = 6 the sums of a typical
  // block exceed the bound.
  auto softmax_fast_on = [&](int j, uint32_t (&P)[PW], const SAcc (&Sx)[2], float kx) __attribute__((always_inline)) {
    const float c = kI8 ? c21(qsc * kx) : a.qk_mul;
    const float m = m_use - SoftmaxCfg<PVM>::kShift;
    const float bias = kI8 ? __builtin_fmaf(kMagicF, c, m) : m;
    constexpr bool kSumF16 = PVM == SAGE_PV_F16;
    constexpr float kBound = (float)(1 << (int)(SoftmaxCfg<PVM>::kTau + SoftmaxCfg<PVM>::kShift - 1.0f));
    float ls[2] = {0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float p[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float sv = kI8 ? __int_as_float((int)Sx[t][v]) : (float)Sx[t][v];
        p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv, c, -bias));
      }
      if constexpr (!kF8) {
#pragma unroll
        for (int w = 0; w < 8; ++w) P[8 * t + w] = Pv::pack2(p[2 * w], p[2 * w + 1]);
      }
      if constexpr (!kSumF16) {
#pragma unroll
        for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
          for (int i = 0; i < w; ++i) p[i] += p[i + w];
        ls[t] = p[0];
      }
    }
    float part, lnew;  // the lane's sum; lsum plus it, as softmax() adds it
    if constexpr (kSumF16) {
      h2 hs[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) hs[w] = __builtin_bit_cast(h2, P[w]) + __builtin_bit_cast(h2, P[8 + w]);
#pragma unroll
      for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) hs[i] = hs[i] + hs[i + w];
      const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
      part = __builtin_amdgcn_fdot2(hs[0], ones, 0.0f, false);
      lnew = __builtin_amdgcn_fdot2(hs[0], ones, lsum, false);
    } else {
      part = ls[0] + ls[1];
      lnew = lsum + (ls[0] + ls[1]);
    }
    if (__builtin_amdgcn_ballot_w64(!(part <= kBound)) == 0) lsum = lnew;
    else softmax_on(j, P, false, Sx, kx);
  };
  auto softmax_fast = [&](int j, uint32_t (&P)[PW]) __attribute__((always_inline)) {
    softmax_fast_on(j, P, S, ksc_cur);
  };
  auto rescale_o = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha_o;
    if constexpr (kSumMfma) osum *= alpha_o;
    alpha_o = 1.0f;
  };
  auto keep_p = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int w = 0; w < PW; ++w) Pprev[w] = Pcur[w];
  };

  // ---- iterations.  Iteration j: loads of tile j+3, P.V of block j-1,
  // softmax of block j, S of block j+1, then tile j+2 complete and a barrier.
  // Iteration nkb only finishes the last P.V.  Every wave runs nkb + 1
  // iterations.  The mask-free steady state has a loop of its own so that the
  // O accumulators are updated from one place in each loop.
  auto generic_iter = [&](int j) __attribute__((always_inline)) {
    if (j + 3 < nkb) load_tile(j + 3, (j + 3) % NBUF);
    if (pend) {
      rescale_o();
      pend = false;
    }
    if (j >= 1 && j - 1 <= jmax) pv((j - 1) % NBUF, Pprev);
    __builtin_amdgcn_sched_barrier(0);
    if (j <= jmax) {
      if (j < nfull) softmax(j, Pcur, false);
      else softmax(j, Pcur, true);
      keep_p();
    }
    if (j + 1 <= jmax) qk(j + 1, (j + 1) % NBUF);
    sync_tiles(j + 3 < nkb);
  };
  // blocks 1 <= j < j_fast: every stage exists and no mask is needed; the P.V
  // MFMAs of block j-1 and the softmax VALU work of block j share one basic
  // block for the scheduler to interleave
  // sl: j % NBUF as a constant (the unrolled loop: operand offsets fold into
  // the LDS instructions), or -1 to compute the slots from j
  auto fast_iter = [&](int j, int sl) __attribute__((always_inline)) {
    load_tile_fast(j + 3, sl < 0 ? (j + 3) % NBUF : (sl + 3) % NBUF);
    if (pend) {
      rescale_o();
      pend = false;
    }
    pv(sl < 0 ? (j - 1) % NBUF : (sl + NBUF - 1) % NBUF, Pprev);
    __builtin_amdgcn_iglp_opt(0);  // LLVM's IGroupLP strategy 0, as in fused_iter below
    if constexpr (PVM != SAGE_PV_FP8) softmax_fast(j, Pcur);
    else softmax(j, Pcur, false);
    keep_p();
    qk(j + 1, sl < 0 ? (j + 1) % NBUF : (sl + 1) % NBUF);
    sync_tiles(true, true);
  };

  // INT8 with fp16 P, and fp16/bf16 QK at D = 64: the S of block j+1 goes to
  // a second buffer, so that its QK MFMAs share one basic block with the P.V
  // MFMAs of block j-1 and the softmax of block j (the scheduler interleaves
  // all three; measured -1.9 % per launch at config 2, -1.2 % at config 4,
  // -3 to -4.5 % for fp16/bf16 QK at D = 64; with FP8 P it was slower, and
  // fp16/bf16 QK at D = 128 has no registers left for it).  Two iterations
  // per trip swap the buffers' roles (ten at D = 64, where the ring slots are
  // constants too).  sl as for fast_iter.
  constexpr bool kTwoS = (kI8 && PVM == SAGE_PV_F16) || (!kI8 && D == 64);
  static_assert(!(kTwoS && PVM == SAGE_PV_FP8), "fused_iter uses the fp16/bf16 P shortcut of softmax_fast_on");
  SAcc S2[2];
  float ksc2 = 0.0f;
  auto fused_iter = [&](int j, int sl, SAcc (&Sa)[2], float ka, SAcc (&Sb)[2], float& kb)
                        __attribute__((always_inline)) {
    load_tile_fast(j + 3, sl < 0 ? (j + 3) % NBUF : (sl + 3) % NBUF);
    if (pend) {
      rescale_o();
      pend = false;
    }
    pv(sl < 0 ? (j - 1) % NBUF : (sl + NBUF - 1) % NBUF, Pprev);
    // LLVM's IGroupLP strategy 0 (LDS instructions interleaved with MFMAs)
    // for this scheduling region: measured -1.5 to -2 % per attention launch at
    // configs 2 and 3, -3 % at config 4, +-0 at config 5
    __builtin_amdgcn_iglp_opt(0);
    qk_into(j + 1, sl < 0 ? (j + 1) % NBUF : (sl + 1) % NBUF, Sb, kb);
    softmax_fast_on(j, Pcur, Sa, ka);
    keep_p();
    sync_tiles(true, true);
  };

  // Q quantization (kFQ) with the pre-pass's arithmetic (per_block_int8,
  // triton_impl.py:25-33, 69): x = fp32(q) * q_mul, scale = max|x| / 127 over
  // the q_sub rows of the scale (rows past Nq left out), q8 =
  // round-half-away(x / scale).  Waves of one scale meet through LDS and a
  // barrier without a memory fence (the tile loads stay in flight).
  auto quantize_q = [&]() __attribute__((always_inline)) {
    if constexpr (kFQ) {
#pragma clang fp contract(off)
      __shared__ float qamax_s[NW];
      const int row = qa + n;
      const bool valid = row < a.Nq;
      float xq[KC][16];
      float am = 0.0f;
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          xq[c][e] = elem<TO>(qraw[c][e >> 3], e & 7) * a.q_mul;
          am = fmaxf(am, fabsf(xq[c][e]));
        }
      if (a.q_sub == 1) {  // one scale per row: its two lane halves
        am = max_halves_f(valid ? am : 0.0f);
      } else {
        am = __uint_as_float(wave_max_u32(__float_as_uint(valid ? am : 0.0f)));  // the wave's 32 rows
      }
      if (a.q_sub > 32) {  // a scale spans q_sub / 32 waves
        if (lane == 0) qamax_s[wave] = am;
        SAGE_WAIT_LGKM0();
        wg_barrier();
        const int per = a.q_sub / 32, w0 = wave / per * per;
        for (int w = w0; w < w0 + per; ++w) am = fmaxf(am, qamax_s[w]);
      }
      qsc = block_scale(am);
      const float rc = qsc > 0.0f ? 1.0f / qsc : 0.0f;
      // one wave-uniform choice of the division (a per-lane flag would put a
      // branch around every element)
      auto quantize_regs = [&](auto fast_tag) __attribute__((always_inline)) {
        constexpr bool kFast = decltype(fast_tag)::value;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          int w[4] = {0, 0, 0, 0};
#pragma unroll
          for (int e = 0; e < 16; ++e)
            w[e >> 2] |= (int)(uint32_t)(uint8_t)quant_elem(xq[c][e], qsc, rc, kFast) << (8 * (e & 3));
          qreg[c] = (v4i){w[0], w[1], w[2], w[3]};
        }
      };
      if (__builtin_amdgcn_ballot_w64(!fast_div_ok(qsc)) == 0) quantize_regs(std::true_type{});
      else quantize_regs(std::false_type{});
      if (a.q8_out && valid) {
#pragma unroll
        for (int c = 0; c < KC; ++c)
          *reinterpret_cast<v4i*>(a.q8_out + b * a.sq[0] + h * a.sq[1] + (int64_t)row * a.sqn + 32 * c + 16 * hh) =
              qreg[c];
      }
      // every sub-block (row) of the ceil(Nq/128) blocks, those with no rows too (scale 0)
      if (a.qs_out && qa < (a.Nq + 127) / 128 * 128) {
        float* qs = a.qs_out + ((int64_t)b * a.Hq + h) * a.nqs;
        if (a.q_sub == 1) {
          if (hh == 0) qs[row] = qsc;
        } else if (lane == 0 && qa % a.q_sub == 0) {
          qs[qa / a.q_sub] = qsc;
        }
      }
    }
  };

  // ---- prologue: tiles 0, 1, 2 requested, 0 and 1 awaited; S of block 0.
  // With fewer than 3 tiles the last one is requested again (same data into
  // its own slot), so the number of loads issued after Q's is fixed and Q can
  // be waited for without draining the tile loads.
  load_tile(0, 0);
  load_tile(min(1, nkb - 1), min(1, nkb - 1));
  load_tile(min(2, nkb - 1), min(2, nkb - 1));
  quantize_q();
#if SAGE_TRACE
  tr_put(13, __builtin_amdgcn_s_memtime());
#endif
  sync_tiles(nkb > 2);
#if SAGE_TRACE
  tr_put(14, __builtin_amdgcn_s_memtime());
#endif
  if (jmax >= 0) qk(0, 0);

  if constexpr (kI8) {  // mgrid = 4 ulp(kMagicF * c_max): exponent field of that product - 21,
    // at least 2^-23 (a coarser grid keeps the bias exact; with a zero scale
    // the grid's inverse times m - kShift must not overflow) and at most 1
    const float cmax = c21(qsc * __uint_as_float(wave_max_u32(ksc_max_bits)));
    const int e = (int)((__float_as_uint(kMagicF * cmax) >> 23) & 0xFF);
    const int eg = min(max(e - 21, 104), 127);
    mgrid = __uint_as_float((uint32_t)eg << 23);
    mgrid_inv = __uint_as_float((uint32_t)(254 - eg) << 23);
  }
  const int j_fast = min(min(nfull, jmax), min(nkb, a.Nkv / kBN) - 3);  // tile j+3 whole
#if SAGE_TRACE
  tr_put(1, __builtin_amdgcn_s_memtime());
#endif
  generic_iter(0);
#if SAGE_TRACE
  tr_put(2, __builtin_amdgcn_s_memtime());
#endif
  int j = 1;
  // D = 64 (INT8 with fp16 P, and fp16/bf16 QK): constant ring slots, j % NBUF
  // == 1 at every trip (at D = 128 the copies run out of registers); then
  // INT8 with fp16 P five at a time with one S buffer
  if constexpr (kTwoS && D == 64)
    for (; j + 2 * NBUF <= j_fast; j += 2 * NBUF) {
      fused_iter(j, 1, S, ksc_cur, S2, ksc2);
      fused_iter(j + 1, 2, S2, ksc2, S, ksc_cur);
      fused_iter(j + 2, 3, S, ksc_cur, S2, ksc2);
      fused_iter(j + 3, 4, S2, ksc2, S, ksc_cur);
      fused_iter(j + 4, 0, S, ksc_cur, S2, ksc2);
      fused_iter(j + 5, 1, S2, ksc2, S, ksc_cur);
      fused_iter(j + 6, 2, S, ksc_cur, S2, ksc2);
      fused_iter(j + 7, 3, S2, ksc2, S, ksc_cur);
      fused_iter(j + 8, 4, S, ksc_cur, S2, ksc2);
      fused_iter(j + 9, 0, S2, ksc2, S, ksc_cur);
    }
  if constexpr (kI8 && D == 64 && PVM == SAGE_PV_F16)
    for (; j + NBUF <= j_fast; j += NBUF) {
      fast_iter(j, 1);
      fast_iter(j + 1, 2);
      fast_iter(j + 2, 3);
      fast_iter(j + 3, 4);
      fast_iter(j + 4, 0);
    }
  if constexpr (kTwoS && D == 128)
    for (; j + 2 <= j_fast; j += 2) {
      fused_iter(j, -1, S, ksc_cur, S2, ksc2);
      fused_iter(j + 1, -1, S2, ksc2, S, ksc_cur);
    }
  for (; j < j_fast; ++j) fast_iter(j, -1);
#if SAGE_TRACE
  tr_put(3, __builtin_amdgcn_s_memtime());
#endif
  for (; j <= nkb; ++j) generic_iter(j);
#if SAGE_TRACE
  tr_put(4, __builtin_amdgcn_s_memtime());
#endif

  // ---- epilogue: O / l, store row q = qa + n, d = 32dt + 8i + 4hh .. +4
  if (pend) rescale_o();
  TO* obase = static_cast<TO*>(a.o) + b * a.so[0] + h * a.so[1];
  const float* vsc = kF8 ? a.v_scale + ((int64_t)b * a.Hkv + hk) * D : nullptr;
  const float inv = 1.0f / (kSumMfma ? osum[0] : sum_halves(lsum));
  const int row = qa + n;
  auto out4 = [&](int dt, int i, TO* p) __attribute__((always_inline)) {
    const int d0 = 32 * dt + 8 * i + 4 * hh;
    float4 f = make_float4(inv, inv, inv, inv);
    if constexpr (kF8) {
      const float4 vs4 = *reinterpret_cast<const float4*>(vsc + d0);
      f = make_float4(inv * vs4.x, inv * vs4.y, inv * vs4.z, inv * vs4.w);
    }
    const v16f& o = oacc[dt];
    store4<TO>(p + d0, o[4 * i] * f.x, o[4 * i + 1] * f.y, o[4 * i + 2] * f.z, o[4 * i + 3] * f.w);
  };
  // The C layout gives each lane 8- or 16-byte pieces of 32 rows; written to
  // HBM directly that is 32 partial lines per store.  Where the wave's 32 x D
  // tile fits in its share of the (by now idle: the last iteration ended
  // with LDS reads and tile loads drained and a barrier) tile ring, it goes
  // through LDS and leaves as whole rows, 16 bytes per lane.
  constexpr int ORP = D * (int)sizeof(TO) + 16;  // LDS row pitch: rows 4 banks apart
  if constexpr (NW * 32 * ORP <= NBUF * SLOT) {
    char* st = smem + wave * 32 * ORP;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) out4(dt, i, reinterpret_cast<TO*>(st + n * ORP));
    constexpr int CPO = D * (int)sizeof(TO) / 16;  // 16-byte chunks per row
    constexpr int RPI = 64 / CPO;                  // rows per instruction
    const int rr = lane / CPO, cc = lane % CPO;
#pragma unroll
    for (int r0 = 0; r0 < 32; r0 += RPI) {
      const v4i val = *reinterpret_cast<const v4i*>(st + (r0 + rr) * ORP + 16 * cc);
      const int orow = qa + r0 + rr;
      if (orow < a.Nq)
        *reinterpret_cast<v4i*>(reinterpret_cast<char*>(obase + (uint32_t)(orow * a.son)) + 16 * cc) = val;
    }
  } else if (row < a.Nq) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) out4(dt, i, obase + (uint32_t)(row * a.son));
  }
#if SAGE_TRACE
  tr_put(5, __builtin_amdgcn_s_memtime());
  tr_put(10, __builtin_amdgcn_s_memrealtime());
  tr_put(6, tr_wait);
  tr_put(7, tr_wait_fast);
  tr_put(8, (unsigned long long)(tr_n & 0xFFFF) | ((unsigned long long)(tr_n >> 16) << 32));
  tr_put(11, (unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4) |
                 ((unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32));
  tr_put(12, (unsigned long long)wg);
  if constexpr (kTrace) {
    SAGE_WAIT_LGKM0();
    if (a.trace && lane < kTraceWords)
      a.trace[((size_t)blockIdx.x * NW + wave) * kTraceWords + lane] = tr_s[wave * kTraceWords + lane];
  }
#endif
}

#if SAGE_TRACE
static unsigned long long* g_trace = nullptr;
static int64_t g_trace_words = 0;
#endif

template <int QKM, int D, int PVM, typename TO>
static int launch_cfg(const AttnArgs& a, hipStream_t st, const char* who) {
  const int64_t nqb = (a.Nq + 255) / 256;
  const int64_t grid = nqb * a.Hq * a.B;
  if (grid > 0x7FFFFFFF) return fail("%s: invalid argument: grid too large", who);
#if SAGE_TRACE
  AttnArgs at = a;
  at.trace = g_trace;
  if (g_trace && grid * 8 * kTraceWords > g_trace_words)
    return fail("%s: invalid argument: trace buffer of %lld words < %lld", who, (long long)g_trace_words,
                (long long)(grid * 8 * kTraceWords));
  hipLaunchKernelGGL((attn_fwd_kernel<QKM, D, PVM, TO>), dim3((unsigned)grid), dim3(512), 0, st, at);
#else
  hipLaunchKernelGGL((attn_fwd_kernel<QKM, D, PVM, TO>), dim3((unsigned)grid), dim3(512), 0, st, a);
#endif
  return check_launch(who);
}

template <int PVM, typename TO>
static int launch_d(const AttnArgs& a, int D, hipStream_t st) {
  return D == 64 ? launch_cfg<kQkI8, 64, PVM, TO>(a, st, "sage_attn_fwd")
                 : launch_cfg<kQkI8, 128, PVM, TO>(a, st, "sage_attn_fwd");
}

template <int QKM, int PVM, typename TO>
static int launch_d(const AttnArgs& a, int D, hipStream_t st, const char* who) {
  return D == 64 ? launch_cfg<QKM, 64, PVM, TO>(a, st, who) : launch_cfg<QKM, 128, PVM, TO>(a, st, who);
}

template <typename TO>
static int launch_pv(const AttnArgs& a, int D, int pv_mode, hipStream_t st) {
  switch (pv_mode) {
    case SAGE_PV_F16: return launch_d<SAGE_PV_F16, TO>(a, D, st);
    case SAGE_PV_BF16: return launch_d<SAGE_PV_BF16, TO>(a, D, st);
    default: return launch_d<SAGE_PV_FP8, TO>(a, D, st);
  }
}

// INT8 attention with Q quantized in the kernel (Q and O share their type)
template <typename TO>
static int launch_pv_q(const AttnArgs& a, int D, int pv_mode, hipStream_t st) {
  const char* who = "sage_attn_fwd_q";
  switch (pv_mode) {
    case SAGE_PV_F16: return launch_d<kQkI8Q, SAGE_PV_F16, TO>(a, D, st, who);
    case SAGE_PV_BF16: return launch_d<kQkI8Q, SAGE_PV_BF16, TO>(a, D, st, who);
    default: return launch_d<kQkI8Q, SAGE_PV_FP8, TO>(a, D, st, who);
  }
}

// unquantized kernel: QK in the input type, P.V in the input type (the
// reference casts P to V's dtype, kernels/flash_attn/triton_impl.py:87-88)
template <int QKM, typename TO>
static int launch_flash(const AttnArgs& a, int D, hipStream_t st) {
  constexpr int PVM = QKM == kQkF16 ? SAGE_PV_F16 : SAGE_PV_BF16;
  return D == 64 ? launch_cfg<QKM, 64, PVM, TO>(a, st, "sage_flash_fwd")
                 : launch_cfg<QKM, 128, PVM, TO>(a, st, "sage_flash_fwd");
}

static bool strides_ok(const int64_t* s, int esize) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] * esize) % 16 != 0) return false;
  return true;
}

static bool is_float_code(int c) { return c == SAGE_DTYPE_F32 || c == SAGE_DTYPE_F16 || c == SAGE_DTYPE_BF16; }

// Checks and fills everything of AttnArgs but the Q operand.
static int attn_setup(AttnArgs& a, const char* who, const int64_t* q_strides, int q_es, const int8_t* k8,
                      const int64_t* k8_strides, const float* k_scale, const void* v, int v_dtype,
                      const float* v_scale, void* o, int o_dtype, const int64_t* o_strides, int64_t B, int64_t Hq,
                      int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, int causal, int blkq, int blkk, int q_sub,
                      int pv_mode) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Nq <= 0 || Nkv <= 0) return fail("%s: invalid argument: empty shape", who);
  if (D != 64 && D != 128) return fail("%s: invalid argument: head_dim %lld (supported: 64, 128)", who, (long long)D);
  if (Hq % Hkv != 0) return fail("%s: invalid argument: Hq %% Hkv != 0", who);
  if (Nq > 0x7FFFFFFF || Nkv > 0x7FFFFFFF || Hq > 0xFFFF || B > 0xFFFF)
    return fail("%s: invalid argument: shape too large", who);
  if (blkk != 64 && blkk != 128 && blkk != 256)
    return fail("%s: invalid argument: blkk=%d (64, 128 or 256)", who, blkk);
  if (q_sub != 1 && (q_sub < 32 || q_sub % 32 != 0 || blkq % q_sub != 0))
    return fail("%s: invalid argument: q_sub=%d blkq=%d (q_sub: 1 or a multiple of 32 dividing blkq)", who, q_sub,
                blkq);
  if (!k_scale || !k8 || !v || !o || !q_strides || !k8_strides || !o_strides)
    return fail("%s: invalid argument: null pointer", who);
  if (pv_mode != SAGE_PV_F16 && pv_mode != SAGE_PV_BF16 && pv_mode != SAGE_PV_FP8)
    return fail("%s: invalid argument: pv_mode %d", who, pv_mode);
  if (!is_float_code(o_dtype)) return fail("%s: invalid argument: o_dtype %d", who, o_dtype);
  if (v_dtype != SAGE_DTYPE_VTILES)
    return fail("%s: invalid argument: v_dtype %d (V must be in the tile layout of sage_vtiles)", who, v_dtype);
  if (pv_mode == SAGE_PV_FP8 && !v_scale) return fail("%s: invalid argument: FP8 P.V needs v_scale", who);
  const int oes = o_dtype == SAGE_DTYPE_F32 ? 4 : 2;
  const bool rows32 = (Nq * q_strides[2] + D) * q_es < 0x7FFFFFFF && Nkv * k8_strides[2] + D < 0x7FFFFFFF &&
                      Nq * o_strides[2] + D < 0x7FFFFFFF;
  if (!rows32) return fail("%s: invalid argument: a head's rows must span < 2^31 elements", who);
  if (!strides_ok(q_strides, q_es) || !strides_ok(k8_strides, 1) || !strides_ok(o_strides, oes))
    return fail("%s: invalid argument: strides must keep 16-byte aligned rows", who);
  if (((uintptr_t)k8 | (uintptr_t)v | (uintptr_t)o) % 16 != 0)
    return fail("%s: invalid argument: base pointers must be 16-byte aligned", who);
  a.k8 = k8;
  a.k_scale = k_scale;
  a.v = v;
  a.v_scale = v_scale;
  a.o = o;
  for (int i = 0; i < 2; ++i) {
    a.sq[i] = q_strides[i];
    a.sk[i] = k8_strides[i];
    a.so[i] = o_strides[i];
  }
  a.sqn = (int)q_strides[2];
  a.skn = (int)k8_strides[2];
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
  return 0;
}

}  // namespace sage

using namespace sage;

extern "C" int sage_attn_fwd(const int8_t* q8, const int64_t* q8_strides, const float* q_scale,
                             const int8_t* k8, const int64_t* k8_strides, const float* k_scale,
                             const void* v, int v_dtype, const int64_t* v_strides, const float* v_scale,
                             void* o, int o_dtype, const int64_t* o_strides, int64_t B, int64_t Hq,
                             int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, int causal, int blkq,
                             int blkk, int q_sub, int pv_mode, void* stream) {
  (void)v_strides;
  const char* who = "sage_attn_fwd";
  if (!q8 || !q_scale || !q8_strides) return fail("%s: invalid argument: null pointer", who);
  AttnArgs a{};
  if (int rc = attn_setup(a, who, q8_strides, 1, k8, k8_strides, k_scale, v, v_dtype, v_scale, o, o_dtype,
                          o_strides, B, Hq, Hkv, Nq, Nkv, D, causal, blkq, blkk, q_sub, pv_mode))
    return rc;
  if ((uintptr_t)q8 % 16 != 0) return fail("%s: invalid argument: base pointers must be 16-byte aligned", who);
  a.q8 = q8;
  a.q_scale = q_scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int d = (int)D;
  switch (o_dtype) {
    case SAGE_DTYPE_F32: return launch_pv<float>(a, d, pv_mode, st);
    case SAGE_DTYPE_F16: return launch_pv<_Float16>(a, d, pv_mode, st);
    default: return launch_pv<__bf16>(a, d, pv_mode, st);
  }
}

extern "C" int sage_attn_fwd_q(const void* q, const int64_t* q_strides, int q_dtype, float q_mul, int8_t* q8_out,
                               float* q_scale_out, const int8_t* k8, const int64_t* k8_strides,
                               const float* k_scale, const void* v, int v_dtype, const int64_t* v_strides,
                               const float* v_scale, void* o, const int64_t* o_strides, int64_t B, int64_t Hq,
                               int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, int causal, int blkq, int blkk,
                               int q_sub, int pv_mode, void* stream) {
  (void)v_strides;
  const char* who = "sage_attn_fwd_q";
  if (!q || !q_strides) return fail("%s: invalid argument: null pointer", who);
  if (!is_float_code(q_dtype)) return fail("%s: invalid argument: q_dtype %d", who, q_dtype);
  if (blkq != 128) return fail("%s: invalid argument: blkq=%d (128: the rows of 4 waves)", who, blkq);
  if (!(q_mul > 0.0f) || q_mul == INFINITY) return fail("%s: invalid argument: q_mul %g", who, q_mul);
  const int qes = q_dtype == SAGE_DTYPE_F32 ? 4 : 2;
  AttnArgs a{};
  if (int rc = attn_setup(a, who, q_strides, qes, k8, k8_strides, k_scale, v, v_dtype, v_scale, o, q_dtype,
                          o_strides, B, Hq, Hkv, Nq, Nkv, D, causal, blkq, blkk, q_sub, pv_mode))
    return rc;
  if (((uintptr_t)q | (uintptr_t)q8_out) % 16 != 0)
    return fail("%s: invalid argument: base pointers must be 16-byte aligned", who);
  a.q8 = q;
  a.q_mul = q_mul;
  a.q8_out = q8_out;
  a.qs_out = q_scale_out;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int d = (int)D;
  switch (q_dtype) {
    case SAGE_DTYPE_F32: return launch_pv_q<float>(a, d, pv_mode, st);
    case SAGE_DTYPE_F16: return launch_pv_q<_Float16>(a, d, pv_mode, st);
    default: return launch_pv_q<__bf16>(a, d, pv_mode, st);
  }
}

#if SAGE_TRACE
// Measurement build only (include/sage_trace.h): the attention launches that
// follow write their phase trace into buf (at least grid * 8 * 16 words), or
// into nothing again after a call with buf = NULL.
extern "C" int sage_trace_attach(unsigned long long* buf, int64_t words) {
  if (buf && words <= 0) return fail("sage_trace_attach: invalid argument: words %lld", (long long)words);
  g_trace = buf;
  g_trace_words = buf ? words : 0;
  return 0;
}
#endif

extern "C" int sage_flash_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                              const void* v, int v_dtype, const int64_t* v_strides, void* o,
                              const int64_t* o_strides, int in_dtype, int64_t B, int64_t Hq, int64_t Hkv,
                              int64_t Nq, int64_t Nkv, int64_t D, float qk_mul, int causal, void* stream) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Nq <= 0 || Nkv <= 0)
    return fail("sage_flash_fwd: invalid argument: empty shape");
  if (D != 64 && D != 128)
    return fail("sage_flash_fwd: invalid argument: head_dim %lld (supported: 64, 128)", (long long)D);
  if (Hq % Hkv != 0) return fail("sage_flash_fwd: invalid argument: Hq %% Hkv != 0");
  if (Nq > 0x7FFFFFFF || Nkv > 0x7FFFFFFF || Hq > 0xFFFF || B > 0xFFFF)
    return fail("sage_flash_fwd: invalid argument: shape too large");
  if (in_dtype != SAGE_DTYPE_F16 && in_dtype != SAGE_DTYPE_BF16)
    return fail("sage_flash_fwd: invalid argument: in_dtype %d (fp16 or bf16)", in_dtype);
  if (!q || !k || !v || !o || !q_strides || !k_strides || !o_strides)
    return fail("sage_flash_fwd: invalid argument: null pointer");
  if (v_dtype != SAGE_DTYPE_VTILES)
    return fail("sage_flash_fwd: invalid argument: v_dtype %d (V must be in the tile layout of sage_vtiles)",
                v_dtype);
  if (!(qk_mul > 0.0f) || qk_mul == INFINITY) return fail("sage_flash_fwd: invalid argument: qk_mul %g", qk_mul);
  const bool rows32 = (Nq * q_strides[2] + D) * 2 < 0x7FFFFFFF && (Nkv * k_strides[2] + D) * 2 < 0x7FFFFFFF &&
                      Nq * o_strides[2] + D < 0x7FFFFFFF;
  if (!rows32) return fail("sage_flash_fwd: invalid argument: a head's rows must span < 2^31 bytes");
  if (!strides_ok(q_strides, 2) || !strides_ok(k_strides, 2) || !strides_ok(o_strides, 2))
    return fail("sage_flash_fwd: invalid argument: strides must keep 16-byte aligned rows");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) % 16 != 0)
    return fail("sage_flash_fwd: invalid argument: base pointers must be 16-byte aligned");

  AttnArgs a{};
  a.q8 = q;
  a.k8 = k;
  a.v = v;
  a.o = o;
  for (int i = 0; i < 2; ++i) {
    a.sq[i] = q_strides[i];
    a.sk[i] = k_strides[i];
    a.so[i] = o_strides[i];
  }
  a.sqn = (int)q_strides[2];
  a.skn = (int)k_strides[2];
  a.son = (int)o_strides[2];
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.Nq = (int)Nq;
  a.Nkv = (int)Nkv;
  a.causal = causal ? 1 : 0;
  a.q_sub = 32;
  a.nqs = a.nks = 1;
  a.qk_mul = qk_mul;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int d = (int)D;
  return in_dtype == SAGE_DTYPE_F16 ? launch_flash<kQkF16, _Float16>(a, d, st)
                                    : launch_flash<kQkBF16, __bf16>(a, d, st);
}
