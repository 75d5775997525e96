// Device-side building blocks shared by the gfx950 MoE kernels: wave64
// reductions over DPP, the ballot-based top-K gate, 128-bit weight loads and
// the SwiGLU activation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "warp_route.h"

namespace wr {

constexpr int kWave = 64;

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Storage tags of weight types without arithmetic here: bfloat16 and OCP fp8
// E4M3 (sign, 4 exponent bits with bias 7, 3 mantissa bits).  Pointer
// arithmetic on them steps by their size; wdec decodes them.
struct bf16w {
  uint16_t bits;
};
struct fp8w {
  uint8_t bits;
};
// MXFP4: two E2M1 codes per byte (element 2i in bits 0-3), one E8M0 scale
// per 32 elements of a row, stored apart from the codes.
struct fp4x2 {
  uint8_t bits;
};
static_assert(sizeof(bf16w) == 2 && sizeof(fp8w) == 1 && sizeof(fp4x2) == 1,
              "weight tags must be packed");

// Matrix elements per storage unit of WT (two for MXFP4, else one); element
// offsets within a matrix become unit offsets with eoff.
template <typename WT>
constexpr int epu() {
  return std::is_same<WT, fp4x2>::value ? 2 : 1;
}
template <typename WT>
__host__ __device__ constexpr int64_t eoff(int64_t elems) {
  return elems / epu<WT>();
}

// A loaded MXFP4 vector: its codes and the raw E8M0 byte of its block scale.
// Vectors never straddle a 32-element block (32 elements per 16 bytes, or
// 2 per byte on the unaligned path).  The byte is turned into an fp32 scale
// where the codes are decoded, not where it is loaded: a conversion next to
// the load (which sits in a branch when the load is conditional) would make
// the wave wait for the byte before it issues its next loads.
struct fp4v32 {
  u32x4 q;
  uint32_t e;
};
struct fp4v2 {
  uint8_t q;
  uint32_t e;
};

// E8M0 scale byte -> 2^(e - 127) as fp32 (e = 0 is the subnormal 2^-127;
// 255, NaN in the format, is never written by the packer).
__device__ __forceinline__ float e8m0_value(uint32_t e) {
  return e == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(e << 23);
}

// Shape and layout of one MoE problem, passed to kernels by value.  Offsets
// and the expert stride are in elements of the weight type: the stride is a
// multiple of 128 bytes (src/expert_layout.cuh:43-45), so it divides evenly.
struct Geom {
  int E, h, I, k, renorm, B;
  int64_t stride, off_up, off_down;
  int64_t off_scale;  // fp8 only: byte offset of the scales in an expert block
};

// ---------------------------------------------------------------------------
// Wave64 reductions.  All 64 lanes must be active.  The in-row steps use
// quad_perm / row_half_mirror / row_mirror DPP moves; the cross-row steps use
// row_bcast:15 and row_bcast:31, after which lane 63 holds the total.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_mov(float old, float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                         CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float lane_bcast(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the wave; the result is returned uniformly to every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xb1>(0.0f, v);        // quad_perm [1,0,3,2]
  v += dpp_mov<0x4e>(0.0f, v);        // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(0.0f, v);       // row_half_mirror
  v += dpp_mov<0x140>(0.0f, v);       // row_mirror: every lane holds its row sum
  v += dpp_mov<0x142, 0xa>(0.0f, v);  // row_bcast:15 into rows 1 and 3
  v += dpp_mov<0x143, 0xc>(0.0f, v);  // row_bcast:31 into rows 2 and 3
  return lane_bcast(v, 63);
}

// The same four in-row steps alone: every lane gets the sum (max) of its
// 16-lane row.
__device__ __forceinline__ float row_sum(float v) {
  v += dpp_mov<0xb1>(0.0f, v);
  v += dpp_mov<0x4e>(0.0f, v);
  v += dpp_mov<0x141>(0.0f, v);
  v += dpp_mov<0x140>(0.0f, v);
  return v;
}
__device__ __forceinline__ float row_max(float v) {
  const float ninf = -__builtin_inff();
  v = fmaxf(v, dpp_mov<0xb1>(ninf, v));
  v = fmaxf(v, dpp_mov<0x4e>(ninf, v));
  v = fmaxf(v, dpp_mov<0x141>(ninf, v));
  v = fmaxf(v, dpp_mov<0x140>(ninf, v));
  return v;
}

// Max over the wave (IEEE maxNum: a NaN lane never wins), uniform result.
__device__ __forceinline__ float wave_max(float v) {
  const float ninf = -__builtin_inff();
  v = fmaxf(v, dpp_mov<0xb1>(ninf, v));
  v = fmaxf(v, dpp_mov<0x4e>(ninf, v));
  v = fmaxf(v, dpp_mov<0x141>(ninf, v));
  v = fmaxf(v, dpp_mov<0x140>(ninf, v));
  v = fmaxf(v, dpp_mov<0x142, 0xa>(ninf, v));
  v = fmaxf(v, dpp_mov<0x143, 0xc>(ninf, v));
  return lane_bcast(v, 63);
}

// Power-of-two exponent e that brings amax = max|v| into [2^14, 2^15) before
// the values v are split into two fp16 terms, hi = fp16(v 2^e) and
// lo = fp16(v 2^e - hi).  Then hi is finite (|v 2^e| < 2^15 < 65504), and
// |v 2^e - (hi + lo)| <= 2^-22 |v 2^e| + 2^-25: lo is an fp16 normal unless
// |v| < 2^-17 amax, and below that its absolute error (half the fp16
// subnormal spacing) is 2^-39 of the scaled maximum.  Returns 0 for amax 0,
// inf or NaN (nothing to scale, or no finite result anyway).  With
// no_down, e >= 0: fp16 inputs are never scaled down, so v 2^e stays exact
// in fp16 and lo = 0.
__device__ __forceinline__ int split_exp(float amax, bool no_down) {
  if (!(amax > 0.0f) || !(amax <= 3.402823466e38f)) return 0;
  int ex;
  (void)frexpf(amax, &ex);  // amax = m 2^ex, m in [0.5, 1)
  const int e = 15 - ex;
  return (no_down && e < 0) ? 0 : e;
}

// SiLU(g) = g / (1 + exp(-g)) (src/fused_moe.cu:30-32), with the accurate
// OCML expf and IEEE division.
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// Gate: softmax over E <= 64 logits and top-K, one wave.  Lane e owns expert
// e.  Each round takes the wave max of the still-available probabilities and
// the lowest lane holding it (first set bit of a 64-bit ballot), which is the
// reference's iterative argmax with a strict '>' (src/naive_moe.cu:164-174):
// ties go to the lower index and a NaN probability is never picked.  If no
// expert is pickable the round yields expert 0 with weight -FLT_MAX, as the
// reference loop does.
// ---------------------------------------------------------------------------
struct TopK {
  int id[WR_MAX_TOPK];
  float w[WR_MAX_TOPK];
  // The same selection spread over lanes (lane kk holds slot kk, lanes past
  // the last slot hold id 0 and weight 0), for reads with a runtime slot
  // index: a v_readlane into a scalar register.  A select chain over the
  // arrays can be folded back into a runtime-indexed array, which then
  // lives in scratch memory, and a scratch load's wait also waits for every
  // weight load issued before it.
  int lid;
  float lw;
};

// `l` is this lane's logit (lane e holds expert e; lanes >= E are ignored).
__device__ __forceinline__ void wave_select_topk_reg(float l_in, int E, int k, int renorm,
                                                     TopK& t) {
  const int lane = threadIdx.x & (kWave - 1);
  const bool valid = lane < E;
  const float l = valid ? l_in : -__builtin_inff();
  const float m = wave_max(l);
  const float ex = valid ? expf(l - m) : 0.0f;
  const float s = wave_sum(ex);
  const float p = ex / s;
  bool avail = valid;
  float tot = 0.0f;
  t.lid = 0;
  t.lw = 0.0f;
#pragma unroll
  for (int kk = 0; kk < WR_MAX_TOPK; ++kk) {
    t.id[kk] = 0;
    t.w[kk] = 0.0f;
    if (kk < k) {
      const bool cand = avail && (p > -3.402823466e38f);
      const float best = wave_max(cand ? p : -__builtin_inff());
      const uint64_t mask = __ballot(cand && p == best);
      const int id = mask ? (__ffsll((unsigned long long)mask) - 1) : 0;
      const float wv = mask ? best : -3.402823466e38f;
      t.id[kk] = __builtin_amdgcn_readfirstlane(id);
      t.w[kk] = wv;
      if (lane == kk) {
        t.lid = t.id[kk];
        t.lw = wv;
      }
      tot += wv;
      if (lane == id) avail = false;
    }
  }
  if (renorm) {
#pragma unroll
    for (int kk = 0; kk < WR_MAX_TOPK; ++kk)
      if (kk < k) t.w[kk] = t.w[kk] / tot;
    if (lane < k) t.lw = t.lw / tot;
  }
}

// Four selections at once, one per 16-lane row, for E <= 16: lane 16 r + e
// holds token r's logit e.  With E <= 16, every full-wave reduction of
// wave_select_topk_reg gives exactly its in-row result (the other rows hold
// zeros or -inf, and x + 0 = x, max(x, -inf) = x), so ids and weights are
// bit-identical to it.  Lane 16 r + kk (kk < k) gets slot kk of row r's
// selection in sid / sw (renormalised if asked); other lanes get 0.
__device__ __forceinline__ void row_select_topk(float l_in, int E, int k, int renorm, int& sid,
                                                float& sw) {
  const int lane = threadIdx.x & (kWave - 1);
  const int li = lane & 15, row = lane >> 4;
  const bool valid = li < E;
  const float l = valid ? l_in : -__builtin_inff();
  const float m = row_max(l);
  const float ex = valid ? expf(l - m) : 0.0f;
  const float s = row_sum(ex);
  const float p = ex / s;
  bool avail = valid;
  float tot = 0.0f;
  sid = 0;
  sw = 0.0f;
#pragma unroll
  for (int kk = 0; kk < WR_MAX_TOPK; ++kk) {
    if (kk < k) {
      const bool cand = avail && (p > -3.402823466e38f);
      const float best = row_max(cand ? p : -__builtin_inff());
      const unsigned rmask =
          (unsigned)(__ballot(cand && p == best) >> (16 * row)) & 0xffffu;  // this row's lanes
      const int id = rmask ? (__ffs(rmask) - 1) : 0;
      const float wv = rmask ? best : -3.402823466e38f;
      if (li == kk) {
        sid = id;
        sw = wv;
      }
      tot += wv;
      if (li == id) avail = false;
    }
  }
  if (renorm && li < k) sw = sw / tot;
}

// Lane e (< 16 NB) gets logit e from NB scalar loads of 16 floats, all issued
// before the first is used.
template <int NB>
__device__ __forceinline__ float lane_logit(const float* __restrict__ logits) {
  typedef float f16v __attribute__((ext_vector_type(16)));
  const int lane = threadIdx.x & (kWave - 1);
  f16v v[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) v[b] = reinterpret_cast<const f16v*>(logits)[b];
  float l = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) l = (lane == 16 * b + i) ? v[b][i] : l;
  return l;
}

// Same, reading the E logits of one token from memory (16-byte aligned, with
// WR_MAX_EXPERTS readable floats; entries >= E are ignored).  The reads are
// wave-uniform scalar loads: every wave of a grid reads the same line at
// kernel start, and through the scalar cache that costs one L2 request per
// cache instead of one per wave (per-wave vector loads serialise on one L2
// channel).  Only the 16-float batches that hold the E logits are loaded, all
// in flight together: under a saturated memory system each extra round trip
// before the first weight load costs microseconds per block.
__device__ __forceinline__ void wave_select_topk(const float* __restrict__ logits, int E, int k,
                                                 int renorm, TopK& t) {
  float l;
  if (E <= 16)
    l = lane_logit<1>(logits);
  else if (E <= 32)
    l = lane_logit<2>(logits);
  else
    l = lane_logit<4>(logits);
  wave_select_topk_reg(l, E, k, renorm, t);
}

// Block-wide variant (every thread of the block must call it): for E <= 16
// the wave-level scalar read above; for more experts wave 0 reads the logits
// with one 256-byte vector load into LDS and every wave selects from there,
// so the block waits for one memory round trip and sends one L2 request.
__device__ __forceinline__ void block_select_topk(const float* __restrict__ logits, int E, int k,
                                                  int renorm, TopK& t) {
  if (E <= 16) {
    wave_select_topk(logits, E, k, renorm, t);
    return;
  }
  __shared__ float s_logits[WR_MAX_EXPERTS];
  const int lane = threadIdx.x & (kWave - 1);
  if (threadIdx.x < kWave) s_logits[lane] = logits[lane];
  __syncthreads();
  wave_select_topk_reg(s_logits[lane], E, k, renorm, t);
}

// Contiguous share [begin, end) of `total` items for worker w of n; shares
// differ in size by at most one item.
__device__ __forceinline__ void share(int total, int w, int n, int& begin, int& end) {
  begin = (int)((int64_t)total * w / n);
  end = (int)((int64_t)total * (w + 1) / n);
}

// Hardware id of the XCD (accelerator complex die) this wave runs on
// (HW_REG_XCC_ID bits [3:0]).  Each XCD has its own L2.
__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 15u;
}

// The dispatch id of the running kernel: the index of its dispatch packet in
// its hardware queue (64-bit, one per launch, increasing along the queue; a
// replayed graph's kernels get new ones), the same for every workgroup.
extern "C" __device__ uint64_t wr_llvm_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

// A 64-bit tag of this kernel launch, the same in every workgroup of it: a
// hash of the launch's (hardware queue address, dispatch id), bijective in
// the dispatch id for a fixed queue, so no two launches on one queue share a
// tag, and launches on different queues share one with probability 2^-64.
__device__ __forceinline__ void launch_tag(uint32_t& lo, uint32_t& hi) {
  const uint64_t d = wr_llvm_dispatch_id();
  const uint64_t q = (uint64_t)(uintptr_t)__builtin_amdgcn_queue_ptr();
  uint64_t t = (d + 1u) * 0x9E3779B97F4A7C15ull;
  t ^= (q >> 4) * 0xC2B2AE3D27D4EB4Full;
  lo = __builtin_amdgcn_readfirstlane((uint32_t)t);
  hi = __builtin_amdgcn_readfirstlane((uint32_t)(t >> 32));
}

// Invalidate this CU's vector L1 and wait for it.  The CU's later loads then
// fetch from L2.
__device__ __forceinline__ void invalidate_l1() {
  asm volatile("buffer_inv sc0\n\ts_waitcnt vmcnt(0)" ::: "memory");
}

// Runtime-index read of a TopK slot (kk wave-uniform, 0 <= kk < WR_MAX_TOPK).
__device__ __forceinline__ int topk_id(const TopK& t, int kk) {
  return __builtin_amdgcn_readlane(t.lid, kk);
}
__device__ __forceinline__ float topk_w(const TopK& t, int kk) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t.lw), kk));
}
// Same for a slot index that may differ across the lanes of a wave.
__device__ __forceinline__ int topk_id_lanes(const TopK& t, int kk) {
  int r = __builtin_amdgcn_readlane(t.lid, 0);
#pragma unroll
  for (int i = 1; i < WR_MAX_TOPK; ++i) r = (kk == i) ? __builtin_amdgcn_readlane(t.lid, i) : r;
  return r;
}

// ---------------------------------------------------------------------------
// Vector loads.  VEC elements per lane: 16 x fp8, 8 x fp16 / bf16 or 4 x fp32
// is one 128-bit access; VEC = 1 is the scalar path for unaligned shapes.
// ---------------------------------------------------------------------------
template <typename T, int VEC>
struct WVec;
template <>
struct WVec<f16, 8> { typedef f16x8 type; };
template <>
struct WVec<f16, 1> { typedef f16 type; };
template <>
struct WVec<float, 4> { typedef f32x4 type; };
template <>
struct WVec<float, 1> { typedef float type; };
template <>
struct WVec<bf16w, 8> { typedef u32x4 type; };
template <>
struct WVec<bf16w, 1> { typedef uint16_t type; };
template <>
struct WVec<fp8w, 16> { typedef u32x4 type; };
template <>
struct WVec<fp8w, 1> { typedef uint8_t type; };
template <>
struct WVec<fp4x2, 32> { typedef fp4v32 type; };
template <>
struct WVec<fp4x2, 2> { typedef fp4v2 type; };

// Natural vector width of a weight type: elements per 128-bit access.
template <typename WT>
constexpr int wvec_width() {
  return 16 / (int)sizeof(WT) * epu<WT>();
}
// Elements per access on the unaligned path.
template <typename WT>
constexpr int wvec_scalar() {
  return epu<WT>();
}

// Streaming weight load: read once per call, so mark it non-temporal.
template <typename T, int VEC>
__device__ __forceinline__ typename WVec<T, VEC>::type load_w(const T* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename WVec<T, VEC>::type*>(p));
}

// Weight load with its block scale: for MXFP4, `sc` is the E8M0 byte of the
// block holding the first element; other types ignore it.
template <typename T, int VEC>
__device__ __forceinline__ typename WVec<T, VEC>::type load_wq(const T* p, const uint8_t* sc) {
  if constexpr (std::is_same<T, fp4x2>::value) {
    typename WVec<T, VEC>::type v;
    if constexpr (VEC == 32)
      v.q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else
      v.q = __builtin_nontemporal_load(reinterpret_cast<const uint8_t*>(p));
    v.e = *sc;
    return v;
  } else {
    (void)sc;
    return load_w<T, VEC>(p);
  }
}

template <typename V>
__device__ __forceinline__ float velem(const V& v, int i) {
  if constexpr (std::is_same<V, f16>::value || std::is_same<V, float>::value) {
    return (float)v;
  } else {
    return (float)v[i];
  }
}

// Element i of a loaded weight vector as fp32 (exact for every type).  bf16
// is the top half of an fp32; fp8 E4M3 goes through v_cvt_pk_f32_fp8, which
// on gfx950 decodes the OCP E4M3 format (checked against all 256 codes) and
// converts two bytes per instruction (the pair is shared by i and i ^ 1).
template <typename WT, typename V>
__device__ __forceinline__ float wdec(const V& v, int i) {
  if constexpr (std::is_same<WT, fp4x2>::value) {
    // v_cvt_scalef32_pk_f32_fp4: the two codes of one byte, times the scale
    // (checked against the E2M1 table for every byte on gfx950).
    const float sc = e8m0_value(v.e);
    if constexpr (std::is_same<V, fp4v2>::value) {
      return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((uint32_t)v.q, sc, 0)[i & 1];
    } else {
      const uint32_t w = v.q[i >> 3];
      f32x2 pr;
      switch ((i >> 1) & 3) {
        case 0: pr = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 0); break;
        case 1: pr = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 1); break;
        case 2: pr = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 2); break;
        default: pr = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 3); break;
      }
      return pr[i & 1];
    }
  } else if constexpr (std::is_same<WT, bf16w>::value) {
    if constexpr (std::is_same<V, uint16_t>::value) {
      return __uint_as_float((uint32_t)v << 16);
    } else {
      const uint32_t w = v[i >> 1];
      return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
    }
  } else if constexpr (std::is_same<WT, fp8w>::value) {
    if constexpr (std::is_same<V, uint8_t>::value) {
      return __builtin_amdgcn_cvt_pk_f32_fp8((int)v, false)[0];
    } else {
      const int w = (int)v[i >> 2];
      const f32x2 pr = (i & 2) ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true)
                               : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
      return pr[i & 1];
    }
  } else {
    return velem(v, i);
  }
}

// Per-row fp8 scales of expert block `blk` (three fp32 arrays of I values at
// byte offset off_scale: gate rows, up rows, down columns).
template <typename WT>
__device__ __forceinline__ const float* wscales(const WT* blk, int64_t off_scale) {
  return reinterpret_cast<const float*>(reinterpret_cast<const char*>(blk) + off_scale);
}

template <typename V>
__device__ __forceinline__ V vzero() {
  if constexpr (std::is_same<V, fp4v32>::value) {
    return fp4v32{u32x4{0u, 0u, 0u, 0u}, 127u};  // scale 1
  } else if constexpr (std::is_same<V, fp4v2>::value) {
    return fp4v2{0, 127u};
  } else if constexpr (std::is_same<V, f16>::value || std::is_same<V, float>::value ||
                       std::is_integral<V>::value) {
    return V(0);
  } else {
    V z;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(V) / sizeof(z[0])); ++i) z[i] = 0;
    return z;
  }
}

// VEC activation values as fp32 (cached load: reused across rows).
template <typename XT, int VEC>
__device__ __forceinline__ void load_x(const XT* __restrict__ p, float (&v)[VEC]) {
  if constexpr (std::is_same<XT, float>::value && VEC % 4 == 0) {
#pragma unroll
    for (int q = 0; q < VEC / 4; ++q) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(p + 4 * q);
      v[4 * q + 0] = t[0];
      v[4 * q + 1] = t[1];
      v[4 * q + 2] = t[2];
      v[4 * q + 3] = t[3];
    }
  } else if constexpr (std::is_same<XT, f16>::value && VEC % 8 == 0) {
#pragma unroll
    for (int q = 0; q < VEC / 8; ++q) {
      const f16x8 t = *reinterpret_cast<const f16x8*>(p + 8 * q);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[8 * q + i] = (float)t[i];
    }
  } else if constexpr (std::is_same<XT, f16>::value && VEC == 4) {
    const f16x4 t = *reinterpret_cast<const f16x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)t[i];
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = (float)p[i];
  }
}

template <typename OT>
__device__ __forceinline__ OT to_out(float v) {
  return (OT)v;
}

}  // namespace wr
