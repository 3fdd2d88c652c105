// sage_prepass.hip — HBM-bound pre-pass of the SageAttention hot path.
//
// Replaces per_block_int8() / quant_per_block_int8_kernel()
// (kernels/sage_attn/triton_impl.py:7-82) and adds what the reference only
// hooks (K smoothing, triton_impl.py:39-40) or lacks (per-channel FP8 V).
//
// Roles (one 256-thread block each, chosen by block index):
//   K statistics:  per (chunk, kv-head, batch) fp32 channel sums of K (and
//                  channel max|v| for FP8 V) in a fixed order
//   Q quant:       per (128-row block, head, batch) INT8 + scale(s)
//   K quant:       with the channel mean subtracted (+ FP8 V rows)
//   V tiles:       through sage_prepass_vt, the tiles of sage_vtiles (FP8
//                  tiles need v_scale, fp16/bf16 ones nothing)
// With statistics (K smoothing, FP8 V) launch A runs them; launch B the K
// quant, which needs the head's channel means, the Q quant and the V tiles
// (the fp16/bf16 ones in launch A when launch B has Q blocks).  Without
// statistics launch A alone.
//
// Every block is 256 threads.  A block's data is read once from HBM with
// 16-byte loads, held in registers while the block's max|x| is reduced, then
// quantized and written with 16-byte stores.  Build with -ffp-contract=off:
// the element arithmetic must round exactly like the reference's.
#include <mutex>
#include <type_traits>

#include "sage_device.h"
#include "sage_vtile_dev.h"

namespace sage {

constexpr int kPrepassThreads = 256;

struct PrepassArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t B, Hq, Hkv, Nq, Nkv;
  int64_t sq[3], sk[3], sv[3];     // input strides (batch, head, seq)
  int64_t sq8[3], sk8[3], sv8[3];  // output strides
  float q_mul;
  int blkq, blkk, q_sub;
  int smooth_k, v_fp8;  // v_fp8: V statistics and v_scale
  int v_rows;            // also the row-major e4m3 codes v8
  int8_t* q8;
  float* q_scale;
  int8_t* k8;
  float* k_scale;
  float* km;
  uint8_t* v8;
  float* v_scale;
  float* psum;   // [B, Hkv, nch, D] K channel sums per chunk
  float* pamax;  // [B, Hkv, nch, D] V channel max|v| per chunk
  int64_t nch, chunk;
  int64_t nqb, nkb;  // blocks per head
  int64_t n_stat, n_qblk_a, n_kblk_a;  // role counts of launch A
  int64_t n_kblk_b, n_qblk_b;          // role counts of launch B (K blocks first)
  uint8_t* vt;                         // V tiles (sage_prepass_vt), else NULL
  int pv_mode;                         // their type
  int64_t ntile;                       // 64-key tiles per head
  int64_t n_vt_a, n_vt_b;              // V tile roles of launch A / B (last in each)
};

// The V tile role r (tile, head, batch) in a block of this pre-pass; vs_s
// holds v_scale for FP8 (visible to every thread), pool >= the role's LDS.
template <typename T, int D>
__device__ __forceinline__ void vtile_role(const PrepassArgs& a, int64_t r, const float* vs_s, char* pool) {
  const int64_t t = r % a.ntile, h = (r / a.ntile) % a.Hkv, b = r / (a.ntile * a.Hkv);
  const T* src = static_cast<const T*>(a.v) + b * a.sv[0] + h * a.sv[1];
  const int64_t tile = (b * a.Hkv + h) * a.ntile + t;
  switch (a.pv_mode) {
    case SAGE_PV_F16:
      vtile_block<T, D, SAGE_PV_F16>(src, a.sv[2], a.Nkv, t, vs_s, a.vt + tile * D * 64 * 2, pool);
      break;
    case SAGE_PV_BF16:
      vtile_block<T, D, SAGE_PV_BF16>(src, a.sv[2], a.Nkv, t, vs_s, a.vt + tile * D * 64 * 2, pool);
      break;
    default:
      vtile_block<T, D, SAGE_PV_FP8>(src, a.sv[2], a.Nkv, t, vs_s, a.vt + tile * D * 64, pool);
      break;
  }
}

template <int D>
constexpr int vtile_pool_bytes() {
  return vtile_lds_bytes<D, SAGE_PV_F16>();  // the largest of the three types
}


// ---------------------------------------------------------------------------
// One quantization block: rows [0, rows_valid) of blk rows x D, scale per
// q_sub rows (q_sub == blk: one scale per block, triton_impl.py:28,33;
// q_sub == 1: one scale per row).
// x = fp32(in) * mul (if use_mul) - km[c] (if km_s; km[c] at stat_slot(c));
// tail rows are left out of the block max and not stored.  NI = 16-element items per thread
// (blk * D / 4096, at least 1; with fewer items than threads whole waves idle).
// ---------------------------------------------------------------------------
struct NoHook {
  __device__ void operator()() const {}
};

// after_loads() runs once the block's loads are issued and before km_s is
// read: a caller that fills km_s there (with a barrier) overlaps that work
// with the loads in flight.
template <typename T, int D, int NI, typename AfterLoads = NoHook>
__device__ __forceinline__ void quant_block(const T* __restrict__ src, int64_t sn, int rows_valid, int blk,
                            int q_sub, bool use_mul, float mul, const float* km_s,
                            int8_t* __restrict__ dst, int64_t dn, float* __restrict__ scale_dst,
                            uint32_t* amax_s, float* scl_s, float* rcp_s, AfterLoads after_loads = {}) {
  constexpr int CPR = D / 16;  // 16-element items per row
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int nit = blk * CPR;  // a multiple of 64: whole waves are valid or not
  const int nsub = blk / q_sub;

  if (tid < 16) amax_s[tid] = 0u;
  Raw8<T> raw[NI][2];
  float amx[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int it = tid + kPrepassThreads * j;
    const int row = it / CPR, c = it % CPR;
    if (it < nit && row < rows_valid) {
      const T* p = src + (int64_t)row * sn + c * 16;
      raw[j][0] = load8<T>(p);
      raw[j][1] = load8<T>(p + 8);
    } else {
      raw[j][0] = zero8<T>();
      raw[j][1] = zero8<T>();
    }
  }
  after_loads();
  // the thread's 16 channels are the same in every item (256 % CPR == 0):
  // their means go to registers once, not through LDS for every element.
  // Without smoothing they are +0, and x - (+0) == x for every x (-0 too).
  static_assert(kPrepassThreads % CPR == 0, "items of a thread share their channels");
  float kmr[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) kmr[e] = km_s ? km_s[stat_slot((tid % CPR) * 16 + e)] : 0.0f;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int it = tid + kPrepassThreads * j;
    const int row = it / CPR;
    float am = 0.0f;
    if (it < nit && row < rows_valid) {  // tail rows stay out of the block max
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = elem<T>(raw[j][e >> 3], e & 7);
        if (use_mul) x = x * mul;
        x = x - kmr[e];
        am = fmaxf(am, fabsf(x));
      }
    }
    amx[j] = am;
  }
  if (q_sub == 1) {  // (block-uniform) a row's CPR items sit in consecutive lanes
    float sc[NI], rc[NI];
    bool ok = true;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int it = tid + kPrepassThreads * j;
      const int row = it / CPR;
      sc[j] = block_scale(__uint_as_float(group_max_u32<CPR>(__float_as_uint(amx[j]))));
      rc[j] = sc[j] > 0.0f ? 1.0f / sc[j] : 0.0f;
      if (it < nit && it % CPR == 0) scale_dst[row] = sc[j];  // every row of the block (0 past the tail)
      if (it < nit && row < rows_valid) ok = ok && fast_div_ok(sc[j]);
    }
    // one wave-uniform choice of the division, as below
    auto quantize_rows = [&](auto fast_tag) __attribute__((always_inline)) {
      constexpr bool kFast = decltype(fast_tag)::value;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int it = tid + kPrepassThreads * j;
        const int row = it / CPR, c = it % CPR;
        if (it >= nit || row >= rows_valid) continue;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float x = elem<T>(raw[j][e >> 3], e & 7);
          if (use_mul) x = x * mul;
          x = x - kmr[e];
          const int8_t qv = quant_elem(x, sc[j], rc[j], kFast);
          w[e >> 2] |= ((uint32_t)(uint8_t)qv) << (8 * (e & 3));
        }
        *reinterpret_cast<uint4*>(dst + (int64_t)row * dn + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    };
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) quantize_rows(std::true_type{});
    else quantize_rows(std::false_type{});
    return;
  }
  __syncthreads();  // amax_s cleared
  if (nsub == 1) {
    float am = amx[0];
#pragma unroll
    for (int j = 1; j < NI; ++j) am = fmaxf(am, amx[j]);
    const uint32_t w = wave_max_u32(__float_as_uint(am));
    if (lane == 0) atomicMax(&amax_s[0], w);
  } else {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int it0 = tid - lane + kPrepassThreads * j;  // first item of this wave
      if (it0 < nit) {                                    // wave-uniform
        // a wave's 64 items cover 64/CPR consecutive rows inside one sub-block
        const uint32_t w = wave_max_u32(__float_as_uint(amx[j]));
        if (lane == 0) atomicMax(&amax_s[(it0 / CPR) / q_sub], w);
      }
    }
  }
  __syncthreads();
  if (tid < nsub) {
    const float sc = block_scale(__uint_as_float(amax_s[tid]));
    scl_s[tid] = sc;
    rcp_s[tid] = sc > 0.0f ? 1.0f / sc : 0.0f;
    scale_dst[tid] = sc;
  }
  __syncthreads();
  // one wave-uniform choice per block: the fast division when every sub-block
  // scale allows it (always, short of all-zero or extreme blocks)
  bool fast_all = true;
  for (int sb = 0; sb < nsub; ++sb) fast_all = fast_all && fast_div_ok(scl_s[sb]);
  auto quantize = [&](auto fast_tag) __attribute__((always_inline)) {
    constexpr bool kFast = decltype(fast_tag)::value;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int it = tid + kPrepassThreads * j;
      const int row = it / CPR, c = it % CPR;
      if (it >= nit || row >= rows_valid) continue;
      const int sub = row / q_sub;
      const float sc = scl_s[sub], rc = rcp_s[sub];
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = elem<T>(raw[j][e >> 3], e & 7);
        if (use_mul) x = x * mul;
        x = x - kmr[e];
        const int8_t qv = quant_elem(x, sc, rc, kFast);
        w[e >> 2] |= ((uint32_t)(uint8_t)qv) << (8 * (e & 3));
      }
      *reinterpret_cast<uint4*>(dst + (int64_t)row * dn + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  };
  if (__builtin_amdgcn_readfirstlane((int)fast_all)) quantize(std::true_type{});
  else quantize(std::false_type{});
}

// ---------------------------------------------------------------------------
// K statistics of one chunk [n0, n1): fp32 channel sums in the fixed order of
// sage_quant_math.h (if psum: K smoothing), and (if vsrc) channel max|v|.
// At least one of psum and vsrc is non-null.
// ---------------------------------------------------------------------------
template <typename T, int D>
__device__ __forceinline__ void kstats_chunk(const T* __restrict__ ksrc, int64_t ksn, const T* __restrict__ vsrc,
                             int64_t vsn, int64_t n0, int64_t n1, float* __restrict__ psum,
                             float* __restrict__ pamax, float* red_s) {
  constexpr int CG = D / 8;
  constexpr int TL = kPrepassThreads / CG;
  const int tid = threadIdx.x;
  const int cg = tid % CG, tl = tid / CG;
  float acc[8], vm[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] = 0.0f;
    vm[e] = 0.0f;
  }
  constexpr int U = 4;  // rows in flight per thread
  for (int64_t nb = n0 + tl; nb < n1; nb += (int64_t)TL * U) {
    Raw8<T> r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t n = nb + (int64_t)u * TL;
      r[u] = (n < n1) ? load8<T>(ksrc + n * ksn + cg * 8) : zero8<T>();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (nb + (int64_t)u * TL < n1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = acc[e] + elem<T>(r[u], e);
      }
    }
    if (vsrc) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t n = nb + (int64_t)u * TL;
        r[u] = (n < n1) ? load8<T>(vsrc + n * vsn + cg * 8) : zero8<T>();
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vm[e] = fmaxf(vm[e], fabsf(elem<T>(r[u], e)));
      }
    }
  }
  // tree over the TL token lanes: acc[tl] += acc[tl + s], s = TL/2 .. 1.
  // Row r of red_s holds channel group cg's values 0-3 and 4-7 as 16-byte
  // units cg and CG + cg, swapped in odd rows, so that the units a wave
  // writes or reads together never share a bank.
  auto at = [&](int r, int e) { return red_s + r * D + 4 * (cg + CG * ((e >> 2) ^ (r & 1))) + (e & 3); };
#pragma unroll
  for (int e = 0; e < 8; ++e) *at(tl, e) = acc[e];
  __syncthreads();
  for (int s = TL / 2; s >= 1; s >>= 1) {
    if (tl < s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) *at(tl, e) = *at(tl, e) + *at(tl + s, e);
    }
    __syncthreads();
  }
  if (psum && tl == 0) {  // (no K smoothing: FP8 V statistics only, no sums)
#pragma unroll
    for (int e = 0; e < 8; ++e) psum[cg * 8 + e] = *at(0, e);
  }
  if (vsrc) {
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 8; ++e) *at(tl, e) = vm[e];
    __syncthreads();
    for (int s = TL / 2; s >= 1; s >>= 1) {
      if (tl < s) {
#pragma unroll
        for (int e = 0; e < 8; ++e) *at(tl, e) = fmaxf(*at(tl, e), *at(tl + s, e));
      }
      __syncthreads();
    }
    if (tl == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pamax[cg * 8 + e] = *at(0, e);
    }
  }
}

// ---------------------------------------------------------------------------
// FP8 e4m3 V rows [0, rows_valid) of one block: v8 = RNE_sat(v / v_scale[c])
// (v_scale[c] == 0 -> 0).  A thread's items keep its 16 channels (256 % CPR
// == 0), so their scales and reciprocals sit in registers; the quotient is
// Markstein's (div_rn_signed) and the codes the packed conversion when every
// scale of the wave lies in the fast range, IEEE division and f32_to_e4m3
// otherwise.
// ---------------------------------------------------------------------------
template <typename T, int D>
__device__ __forceinline__ void vquant_rows(const T* __restrict__ src, int64_t sn, int rows_valid, int blk,
                                            const float* vs_s, uint8_t* __restrict__ dst, int64_t dn) {
  constexpr int CPR = D / 16;
  const int t = (int)threadIdx.x;
  const int c = t % CPR;
  float sc[16], rc[16];
  bool ok = true;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    sc[e] = vs_s[stat_slot(c * 16 + e)];
    rc[e] = sc[e] > 0.0f ? 1.0f / sc[e] : 0.0f;
    ok = ok && fast_div_ok(sc[e]);
  }
  auto rows = [&](auto fast_tag) __attribute__((always_inline)) {
    constexpr bool kFast = decltype(fast_tag)::value;
    for (int it = t; it < blk * CPR; it += kPrepassThreads) {
      const int row = it / CPR;
      if (row >= rows_valid) continue;
      const T* p = src + (int64_t)row * sn + c * 16;
      const Raw8<T> r0 = load8<T>(p), r1 = load8<T>(p + 8);
      uint32_t w[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = elem<T>(g < 2 ? r0 : r1, (4 * g + i) & 7);
        if constexpr (kFast) {
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = div_rn_signed(x[i], sc[4 * g + i], rc[4 * g + i]);
          w[g] = e4m3x4(x[0], x[1], x[2], x[3]);
        } else {
          w[g] = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float s = sc[4 * g + i];
            w[g] |= (uint32_t)f32_to_e4m3(s > 0.0f ? x[i] / s : 0.0f) << (8 * i);
          }
        }
      }
      *reinterpret_cast<uint4*>(dst + (int64_t)row * dn + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  };
  if (__builtin_amdgcn_ballot_w64(!ok) == 0) rows(std::true_type{});
  else rows(std::false_type{});
}

template <typename T, int D, int NI>
__device__ __forceinline__ void quant_q_role(const PrepassArgs& a, int64_t r, uint32_t* amax_s, float* scl_s,
                             float* rcp_s) {
  const int64_t qb = r % a.nqb, h = (r / a.nqb) % a.Hq, b = r / (a.nqb * a.Hq);
  const int64_t row0 = qb * a.blkq;
  const int rows_valid = (int)min<int64_t>(a.blkq, a.Nq - row0);
  const T* src = static_cast<const T*>(a.q) + b * a.sq[0] + h * a.sq[1] + row0 * a.sq[2];
  int8_t* dst = a.q8 + b * a.sq8[0] + h * a.sq8[1] + row0 * a.sq8[2];
  const int nsub = a.blkq / a.q_sub;
  float* sdst = a.q_scale + ((b * a.Hq + h) * a.nqb + qb) * nsub;
  quant_block<T, D, NI>(src, a.sq[2], rows_valid, a.blkq, a.q_sub, true, a.q_mul, nullptr, dst, a.sq8[2],
                        sdst, amax_s, scl_s, rcp_s);
}

template <typename T, int D, int NI, typename AfterLoads = NoHook>
__device__ __forceinline__ void quant_k_role(const PrepassArgs& a, int64_t r, const float* km_s, uint32_t* amax_s,
                             float* scl_s, float* rcp_s, AfterLoads after_loads = {}) {
  const int64_t kb = r % a.nkb, h = (r / a.nkb) % a.Hkv, b = r / (a.nkb * a.Hkv);
  const int64_t row0 = kb * a.blkk;
  const int rows_valid = (int)min<int64_t>(a.blkk, a.Nkv - row0);
  const T* src = static_cast<const T*>(a.k) + b * a.sk[0] + h * a.sk[1] + row0 * a.sk[2];
  int8_t* dst = a.k8 + b * a.sk8[0] + h * a.sk8[1] + row0 * a.sk8[2];
  float* sdst = a.k_scale + (b * a.Hkv + h) * a.nkb + kb;
  quant_block<T, D, NI>(src, a.sk[2], rows_valid, a.blkk, a.blkk, false, 1.0f, km_s, dst, a.sk8[2], sdst,
                        amax_s, scl_s, rcp_s, after_loads);
}

// NIQ / NIK: 16-element items per thread of a Q / K block (blk * D / 4096).
template <typename T, int D, int NIQ, int NIK>
__global__ __launch_bounds__(kPrepassThreads) void prepass_a_kernel(PrepassArgs a) {
  __shared__ uint32_t amax_s[16];
  __shared__ float scl_s[16], rcp_s[16];
  // one pool for the statistics' reduction rows or a V tile's transpose
  constexpr int kRed = kPrepassThreads / (D / 8) * D * (int)sizeof(float);
  __shared__ __attribute__((aligned(16))) char pool[kRed > vtile_pool_bytes<D>() ? kRed : vtile_pool_bytes<D>()];
  float* red_s = reinterpret_cast<float*>(pool);
  int64_t r = blockIdx.x;
  if (r < a.n_stat) {
    const int64_t c = r % a.nch, h = (r / a.nch) % a.Hkv, b = r / (a.nch * a.Hkv);
    const int64_t n0 = c * a.chunk, n1 = min<int64_t>(n0 + a.chunk, a.Nkv);
    const T* ks = static_cast<const T*>(a.k) + b * a.sk[0] + h * a.sk[1];
    const T* vs = a.v_fp8 ? static_cast<const T*>(a.v) + b * a.sv[0] + h * a.sv[1] : nullptr;
    const int64_t slot = ((b * a.Hkv + h) * a.nch + c) * D;
    // psum is NULL without K smoothing (the workspace then holds the V maxima only)
    kstats_chunk<T, D>(ks, a.sk[2], vs, a.sv[2], n0, n1, a.smooth_k ? a.psum + slot : nullptr,
                       a.v_fp8 ? a.pamax + slot : nullptr, red_s);
    return;
  }
  r -= a.n_stat;
  if (r < a.n_qblk_a) {
    quant_q_role<T, D, NIQ>(a, r, amax_s, scl_s, rcp_s);
    return;
  }
  r -= a.n_qblk_a;
  if (r < a.n_kblk_a) {
    quant_k_role<T, D, NIK>(a, r, nullptr, amax_s, scl_s, rcp_s);
    return;
  }
  r -= a.n_kblk_a;
  if (r < a.n_vt_a) vtile_role<T, D>(a, r, nullptr, pool);  // fp16 / bf16 tiles
}

// Channel mean of K (km_s) and FP8 V scale (vs_s, unless null) of one
// (batch, head) from launch A's per-chunk partials, into LDS (threads < D);
// the K block 0 role also writes them out.
template <int D>
__device__ __forceinline__ void head_stats(const PrepassArgs& a, int64_t b, int64_t h, bool write_out,
                                           float* km_s, float* vs_s) {
  const int tid = threadIdx.x;
  const int64_t base = (b * a.Hkv + h) * a.nch * D;
  if (tid >= D) return;
  if (a.smooth_k && km_s) {
    // issue every partial load first (nch <= 16), then add left to right
    float part[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) part[c] = c < a.nch ? a.psum[base + c * D + tid] : 0.0f;
    float s = part[0];
#pragma unroll
    for (int c = 1; c < 16; ++c)
      if (c < a.nch) s = s + part[c];
    const float m = s / (float)a.Nkv;
    km_s[stat_slot(tid)] = m;
    if (write_out) a.km[(b * a.Hkv + h) * D + tid] = m;
  }
  if (a.v_fp8 && vs_s) {
    float m = a.pamax[base + tid];
#pragma unroll
    for (int c = 1; c < 16; ++c)
      if (c < a.nch) m = fmaxf(m, a.pamax[base + c * D + tid]);
    const float sc = m / 448.0f;
    vs_s[stat_slot(tid)] = sc;
    if (write_out) a.v_scale[(b * a.Hkv + h) * D + tid] = sc;
  }
}

// Roles: K blocks, then Q blocks, then (FP8 P.V) V tiles.
template <typename T, int D, int NIQ, int NIK>
__global__ __launch_bounds__(kPrepassThreads) void prepass_b_kernel(PrepassArgs a) {
  __shared__ uint32_t amax_s[16];
  __shared__ float scl_s[16], rcp_s[16];
  __shared__ float km_s[stat_lds_floats<D>()], vs_s[stat_lds_floats<D>()];
  __shared__ __attribute__((aligned(16))) char pool[vtile_pool_bytes<D>()];
  int64_t r = blockIdx.x;
  if (r >= a.n_kblk_b + a.n_qblk_b) {
    r -= a.n_kblk_b + a.n_qblk_b;
    const int64_t h = (r / a.ntile) % a.Hkv, b = r / (a.ntile * a.Hkv);
    head_stats<D>(a, b, h, false, nullptr, vs_s);
    __syncthreads();
    vtile_role<T, D>(a, r, vs_s, pool);
    return;
  }
  if (r >= a.n_kblk_b) {
    quant_q_role<T, D, NIQ>(a, r - a.n_kblk_b, amax_s, scl_s, rcp_s);
    return;
  }
  const int64_t kb = r % a.nkb, h = (r / a.nkb) % a.Hkv, b = r / (a.nkb * a.Hkv);
  // the head's channel means (and the V scales that this block's FP8 V rows
  // or output need) are formed while the K block's loads are in flight
  quant_k_role<T, D, NIK>(a, r, a.smooth_k ? km_s : nullptr, amax_s, scl_s, rcp_s, [&]() {
    head_stats<D>(a, b, h, kb == 0, km_s, a.v_rows || kb == 0 ? vs_s : nullptr);
    __syncthreads();
  });
  if (a.v_rows) {
    const int64_t row0 = kb * a.blkk;
    const int rows_valid = (int)min<int64_t>(a.blkk, a.Nkv - row0);
    const T* src = static_cast<const T*>(a.v) + b * a.sv[0] + h * a.sv[1] + row0 * a.sv[2];
    uint8_t* dst = a.v8 + b * a.sv8[0] + h * a.sv8[1] + row0 * a.sv8[2];
    vquant_rows<T, D>(src, a.sv[2], rows_valid, a.blkk, vs_s, dst, a.sv8[2]);
  }
}

template <typename T, int D, int NIQ, int NIK>
static int launch_prepass_ni(const PrepassArgs& a, hipStream_t st) {
  const int64_t na = a.n_stat + a.n_qblk_a + a.n_kblk_a + a.n_vt_a;
  if (na > 0) {
    hipLaunchKernelGGL((prepass_a_kernel<T, D, NIQ, NIK>), dim3((unsigned)na), dim3(kPrepassThreads), 0, st, a);
    if (int rc = check_launch("sage_prepass (launch A)")) return rc;
  }
  if (a.n_kblk_b > 0) {
    const int64_t nb = a.n_kblk_b + a.n_qblk_b + a.n_vt_b;
    hipLaunchKernelGGL((prepass_b_kernel<T, D, NIQ, NIK>), dim3((unsigned)nb), dim3(kPrepassThreads), 0, st, a);
    if (int rc = check_launch("sage_prepass (launch B)")) return rc;
  }
  return 0;
}

// Exact-fit kernels for the reference's block sizes (BLKQ 128, BLKK 64);
// every other block size runs the 8-items-per-thread kernel.
template <typename T, int D>
static int launch_prepass(const PrepassArgs& a, hipStream_t st) {
  constexpr int NQ = 128 * D / 4096, NK = 64 * D / 4096 > 0 ? 64 * D / 4096 : 1;
  if (a.blkq == 128 && a.blkk == 64) return launch_prepass_ni<T, D, NQ, NK>(a, st);
  return launch_prepass_ni<T, D, 8, 8>(a, st);
}

static bool strides_ok(const int64_t* s, int esize) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] * esize) % 16 != 0) return false;
  return true;
}

}  // namespace sage

using namespace sage;

extern "C" size_t sage_prepass_workspace_bytes(int64_t B, int64_t Hkv, int64_t Nkv, int64_t D,
                                               int smooth_k, int v_mode) {
  if (B <= 0 || Hkv <= 0 || Nkv <= 0 || D <= 0) return 0;
  const int64_t per = B * Hkv * kstat_num_chunks(Nkv) * D * (int64_t)sizeof(float);
  size_t bytes = 0;
  if (smooth_k) bytes += (size_t)per;
  if (v_mode == SAGE_V_FP8 || v_mode == SAGE_V_FP8_SCALE) bytes += (size_t)per;
  return bytes;
}

static int prepass_impl(const char* who, const void* q, const void* k, const void* v, int in_dtype, int64_t B,
                        int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides, float q_mul, int blkq, int blkk,
                        int q_sub, int smooth_k, int v_mode, int8_t* q8, const int64_t* q8_strides, float* q_scale,
                        int8_t* k8, const int64_t* k8_strides, float* k_scale, float* km, uint8_t* v8,
                        const int64_t* v8_strides, float* v_scale, void* workspace, size_t workspace_bytes,
                        int pv_mode, void* vt, size_t vt_bytes, void* stream) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Nq <= 0 || Nkv <= 0)
    return fail("%s: invalid argument: empty shape B=%lld Hq=%lld Hkv=%lld Nq=%lld Nkv=%lld", who, (long long)B, (long long)Hq, (long long)Hkv, (long long)Nq, (long long)Nkv);
  if (D != 64 && D != 128)
    return fail("%s: invalid argument: head_dim %lld (supported: 64, 128)", who, (long long)D);
  if (Hq % Hkv != 0)
    return fail("%s: invalid argument: Hq=%lld not a multiple of Hkv=%lld", who, (long long)Hq,
                (long long)Hkv);
  if (in_dtype != SAGE_DTYPE_F32 && in_dtype != SAGE_DTYPE_F16 && in_dtype != SAGE_DTYPE_BF16)
    return fail("%s: invalid argument: in_dtype %d", who, in_dtype);
  auto blk_ok = [](int b) { return b >= 16 && b <= 256 && b % 16 == 0; };
  if (!blk_ok(blkq) || !blk_ok(blkk))
    return fail("%s: invalid argument: blkq=%d blkk=%d (16..256, multiples of 16)", who, blkq, blkk);
  if (q_sub != 1 && (q_sub < 16 || q_sub % 16 != 0 || blkq % q_sub != 0 || blkq / q_sub > 16))
    return fail("%s: invalid argument: q_sub=%d for blkq=%d", who, q_sub, blkq);
  if (v_mode != SAGE_V_NONE && v_mode != SAGE_V_FP8 && v_mode != SAGE_V_FP8_SCALE)
    return fail("%s: invalid argument: v_mode %d", who, v_mode);
  const bool vfp8 = v_mode != SAGE_V_NONE;  // V statistics and v_scale
  const bool vrows = v_mode == SAGE_V_FP8;  // row-major codes as well
  // q, q8 and q_scale all NULL: K (and V) only -- Q is quantized by sage_attn_fwd_q
  const bool do_q = q || q8 || q_scale;
  if ((do_q && (!q || !q8 || !q_scale || !q_strides || !q8_strides)) || !k || !k8 || !k_scale || !k_strides ||
      !k8_strides)
    return fail("%s: invalid argument: null pointer", who);
  if (smooth_k && !km) return fail("%s: invalid argument: km is null with smooth_k", who);
  if (vfp8 && (!v || !v_scale || !v_strides || (vrows && (!v8 || !v8_strides))))
    return fail("%s: invalid argument: null V pointer with v_mode %d", who, v_mode);
  const int es = in_dtype == SAGE_DTYPE_F32 ? 4 : 2;
  if ((do_q && (!strides_ok(q_strides, es) || !strides_ok(q8_strides, 1))) || !strides_ok(k_strides, es) ||
      !strides_ok(k8_strides, 1) || (vfp8 && !strides_ok(v_strides, es)) || (vrows && !strides_ok(v8_strides, 1)))
    return fail("%s: invalid argument: strides must keep 16-byte aligned rows", who);
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)q8 | (uintptr_t)k8 | (uintptr_t)(vfp8 ? v : nullptr) |
       (uintptr_t)(vrows ? v8 : nullptr)) % 16 != 0)
    return fail("%s: invalid argument: base pointers must be 16-byte aligned", who);
  if (vt) {  // V tiles (sage_prepass_vt)
    if (pv_mode != SAGE_PV_F16 && pv_mode != SAGE_PV_BF16 && pv_mode != SAGE_PV_FP8)
      return fail("%s: invalid argument: pv_mode %d", who, pv_mode);
    if (pv_mode == SAGE_PV_FP8 && !vfp8)
      return fail("%s: invalid argument: FP8 V tiles need v_mode FP8 or FP8_SCALE (v_scale)", who);
    if (!v || !v_strides) return fail("%s: invalid argument: null V pointer for the V tiles", who);
    if (!strides_ok(v_strides, es) || (uintptr_t)v % 16 != 0 || (uintptr_t)vt % 16 != 0)
      return fail("%s: invalid argument: V rows and the V tiles must be 16-byte aligned", who);
    const size_t vneed = sage_vtile_bytes(B, Hkv, Nkv, D, pv_mode);
    if (vt_bytes < vneed) return fail("%s: invalid argument: vtiles %zu bytes < %zu", who, vt_bytes, vneed);
  }
  const size_t need = sage_prepass_workspace_bytes(B, Hkv, Nkv, D, smooth_k, v_mode);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail("%s: invalid argument: workspace %zu bytes < %zu", who, workspace_bytes, need);

  PrepassArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Nq = Nq;
  a.Nkv = Nkv;
  for (int i = 0; i < 3; ++i) {
    a.sq[i] = do_q ? q_strides[i] : 0;
    a.sk[i] = k_strides[i];
    a.sq8[i] = do_q ? q8_strides[i] : 0;
    a.sk8[i] = k8_strides[i];
    a.sv[i] = vfp8 || vt ? v_strides[i] : 0;
    a.sv8[i] = vrows ? v8_strides[i] : 0;
  }
  a.q_mul = q_mul;
  a.blkq = blkq;
  a.blkk = blkk;
  a.q_sub = q_sub;
  a.smooth_k = smooth_k ? 1 : 0;
  a.v_fp8 = vfp8 ? 1 : 0;
  a.v_rows = vrows ? 1 : 0;
  a.q8 = q8;
  a.q_scale = q_scale;
  a.k8 = k8;
  a.k_scale = k_scale;
  a.km = km;
  a.v8 = v8;
  a.v_scale = v_scale;
  a.nch = kstat_num_chunks(Nkv);
  a.chunk = kstat_chunk_tokens(Nkv);
  const int64_t per = B * Hkv * a.nch * D;
  float* ws = static_cast<float*>(workspace);
  a.psum = smooth_k ? ws : nullptr;
  a.pamax = vfp8 ? ws + (smooth_k ? per : 0) : nullptr;
  a.nqb = (Nq + blkq - 1) / blkq;
  a.nkb = (Nkv + blkk - 1) / blkk;
  const bool need_b = a.smooth_k || a.v_fp8;
  // Launch A computes the K statistics; launch B then quantizes K (read
  // again: the statistics of a head must be complete first) and Q.  Without
  // statistics everything runs in launch A.
  a.n_stat = need_b ? a.nch * Hkv * B : 0;
  a.n_qblk_a = need_b || !do_q ? 0 : a.nqb * Hq * B;
  a.n_kblk_a = need_b ? 0 : a.nkb * Hkv * B;
  a.n_kblk_b = need_b ? a.nkb * Hkv * B : 0;
  a.n_qblk_b = need_b && do_q ? a.nqb * Hq * B : 0;
  // V tiles last in their launch: B for FP8 (they need v_scale), and B for
  // fp16/bf16 too when B quantizes only K (its VALU-bound K blocks then share
  // the launch with copy-like work, and launch A only reads K); A otherwise
  a.vt = static_cast<uint8_t*>(vt);
  a.pv_mode = pv_mode;
  a.ntile = (Nkv + 63) / 64;
  const bool vt_in_b = vt && (pv_mode == SAGE_PV_FP8 || (need_b && !do_q));
  a.n_vt_a = vt && !vt_in_b ? a.ntile * Hkv * B : 0;
  a.n_vt_b = vt_in_b ? a.ntile * Hkv * B : 0;
  if (a.n_stat + a.n_qblk_a + a.n_kblk_a + a.n_vt_a > 0x7FFFFFFF || a.n_kblk_b + a.n_qblk_b + a.n_vt_b > 0x7FFFFFFF)
    return fail("%s: invalid argument: grid too large", who);

  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case SAGE_DTYPE_F32:
      return D == 64 ? launch_prepass<float, 64>(a, st) : launch_prepass<float, 128>(a, st);
    case SAGE_DTYPE_F16:
      return D == 64 ? launch_prepass<_Float16, 64>(a, st) : launch_prepass<_Float16, 128>(a, st);
    default:
      return D == 64 ? launch_prepass<__bf16, 64>(a, st) : launch_prepass<__bf16, 128>(a, st);
  }
}

extern "C" int sage_prepass(const void* q, const void* k, const void* v, int in_dtype, int64_t B,
                            int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, float q_mul, int blkq, int blkk, int q_sub,
                            int smooth_k, int v_mode, int8_t* q8, const int64_t* q8_strides,
                            float* q_scale, int8_t* k8, const int64_t* k8_strides, float* k_scale,
                            float* km, uint8_t* v8, const int64_t* v8_strides, float* v_scale,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return prepass_impl("sage_prepass", q, k, v, in_dtype, B, Hq, Hkv, Nq, Nkv, D, q_strides, k_strides, v_strides,
                      q_mul, blkq, blkk, q_sub, smooth_k, v_mode, q8, q8_strides, q_scale, k8, k8_strides, k_scale,
                      km, v8, v8_strides, v_scale, workspace, workspace_bytes, -1, nullptr, 0, stream);
}

extern "C" int sage_prepass_vt(const void* q, const void* k, const void* v, int in_dtype, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D,
                               const int64_t* q_strides, const int64_t* k_strides,
                               const int64_t* v_strides, float q_mul, int blkq, int blkk, int q_sub,
                               int smooth_k, int v_mode, int8_t* q8, const int64_t* q8_strides,
                               float* q_scale, int8_t* k8, const int64_t* k8_strides, float* k_scale,
                               float* km, uint8_t* v8, const int64_t* v8_strides, float* v_scale,
                               void* workspace, size_t workspace_bytes, int pv_mode, void* vtiles,
                               size_t vtile_bytes, void* stream) {
  if (!vtiles) return fail("sage_prepass_vt: invalid argument: null pointer (vtiles)");
  return prepass_impl("sage_prepass_vt", q, k, v, in_dtype, B, Hq, Hkv, Nq, Nkv, D, q_strides, k_strides,
                      v_strides, q_mul, blkq, blkk, q_sub, smooth_k, v_mode, q8, q8_strides, q_scale, k8,
                      k8_strides, k_scale, km, v8, v8_strides, v_scale, workspace, workspace_bytes, pv_mode, vtiles,
                      vtile_bytes, stream);
}

// ---------------------------------------------------------------------------
// sage_prepass_vt_noalloc: sage_prepass_vt with the launch-A partials (K
// channel sums, V channel maxima) in a fixed scratch array of this library
// instead of a caller workspace, for callers that cannot allocate device
// memory.  Each GPU holds its own copy of the array until the process ends.
// Launch A writes every partial that launch B of the same call reads, so
// nothing needs clearing between calls; calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
namespace sage {

static __device__ __align__(256) char scratch[SAGE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* scratch_dev[kMaxDevices];  // device address of `scratch`, per GPU
static std::mutex scratch_mu;

// The current device's address of `scratch`, looked up once per device with
// that device current.  In host code the array's name is a host-side stand-in,
// never a device address: only this pointer may be handed to kernels.
static int scratch_address(const char* who, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail("%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail("%s: device %d beyond the %d supported", who, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail("%s: hipGetSymbolAddress(scratch): %s", who, hipGetErrorString(e));
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return 0;
}

}  // namespace sage

extern "C" int sage_prepass_vt_noalloc(const void* q, const void* k, const void* v, int in_dtype, int64_t B,
                                       int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D,
                                       const int64_t* q_strides, const int64_t* k_strides,
                                       const int64_t* v_strides, float q_mul, int blkq, int blkk, int q_sub,
                                       int smooth_k, int v_mode, int8_t* q8, const int64_t* q8_strides,
                                       float* q_scale, int8_t* k8, const int64_t* k8_strides, float* k_scale,
                                       float* km, uint8_t* v8, const int64_t* v8_strides, float* v_scale,
                                       int pv_mode, void* vtiles, size_t vtile_bytes, void* stream) {
  const char* who = "sage_prepass_vt_noalloc";
  if (!vtiles) return fail("%s: invalid argument: null pointer (vtiles)", who);
  const size_t need = sage_prepass_workspace_bytes(B, Hkv, Nkv, D, smooth_k, v_mode);
  if (need > SAGE_SCRATCH_BYTES)
    return fail("%s: invalid argument: the problem needs %zu bytes of scratch, the library's fixed scratch "
                "holds %zu (use sage_prepass_vt with a workspace)",
                who, need, (size_t)SAGE_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_address(who, &ws)) return rc;
  return prepass_impl(who, q, k, v, in_dtype, B, Hq, Hkv, Nq, Nkv, D, q_strides, k_strides, v_strides, q_mul,
                      blkq, blkk, q_sub, smooth_k, v_mode, q8, q8_strides, q_scale, k8, k8_strides, k_scale, km, v8,
                      v8_strides, v_scale, ws, SAGE_SCRATCH_BYTES, pv_mode, vtiles, vtile_bytes, stream);
}
