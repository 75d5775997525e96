// Fused decode-time MoE kernels for gfx950 (wave64).
//
// Every layer starts with k_router_logits: one 4-wave workgroup per (expert,
// token) computes the router dot product (src/fused_moe.cu:100-112); each
// wave covers a quarter of the row, so one memory round trip covers it.
// Every consumer then derives the top-K selection from the logits itself
// (wave_select_topk: DPP max/sum and a 64-bit ballot).  For layers of many
// gate/up blocks the single-token kernel computes the router rows itself
// instead (route_and_select), one launch per layer as in the reference.
//
// Single token (the decode hot path): k_fused_ffn, ONE launch whose first
// blocks stream the selected experts' gate/up rows and write
// act = w_kk * silu(gate . x) * (up . x) in fp32 (src/fused_moe.cu:192-201,
// silu at :30-32), and whose later blocks stream the selected down rows
// against act and write every output row once (src/fused_moe.cu:203-224,
// without the reference's repeated global read-modify-write of the output).
// The hand-off between the two is described at k_fused_ffn.
//
// Several tokens: k_gateup and k_down, persistent grids with one grid row per
// token; work shares are contiguous row ranges that differ by at most one
// item.
//
// The selected expert weights are the only large traffic: 128-bit
// non-temporal loads, 4 row streams per wave.  x, logits and act are small
// and served from cache.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "wr_device.h"
#include "wr_internal.h"
#include "wr_timeline.h"

// Single-token gate/up chunk slots beyond one round of resident blocks, up to
// this percentage of the round, are claimed by the launched blocks instead of
// being launched as blocks of their own.
#ifndef WR_GU_CLAIM_PCT
#define WR_GU_CLAIM_PCT 25
#endif
// Gate/up blocks per CU that make up that round: 0 = as many as are resident.
#ifndef WR_GU_BLOCKS_PER_CU
#define WR_GU_BLOCKS_PER_CU 0
#endif

#ifndef WR_GU_RPW
#define WR_GU_RPW 2  // gate/up rows per matrix in flight per wave
#endif
#ifndef WR_GU_U
#define WR_GU_U 4    // 64*VEC-element chunks per row per iteration
#endif
#ifndef WR_DN_RPD
#define WR_DN_RPD 2  // down rows per wave item
#endif
#ifndef WR_DN_U
#define WR_DN_U 4
#endif
#ifndef WR_FU_RPD
#define WR_FU_RPD 4  // single-token fused kernel: output rows per down block
#endif
#ifndef WR_FU_U
#define WR_FU_U 4    // single-token fused kernel: column chunks per down tile
#endif
#ifndef WR_WAVES_PER_CU
#define WR_WAVES_PER_CU 8  // persistent waves per CU (upper bound)
#endif
// fp8 weights in the single-token fused kernel (16 weights per 128-bit load)
#ifndef WR_F8_RPW
#define WR_F8_RPW 4  // gate/up rows per wave (2 or 4)
#endif
#ifndef WR_F8_U1
#define WR_F8_U1 2   // gate/up column chunks per row per iteration
#endif
#ifndef WR_F8_RPD
#define WR_F8_RPD 8  // output rows per down block
#endif
#ifndef WR_F8_U2
#define WR_F8_U2 2   // column chunks per down tile
#endif
// x staged in LDS by the gate/up blocks of the single-token fused kernel, for
// h up to these bounds (0: never); fp8 also needs at most WR_XL_FP8_BPC gate/up
// blocks per CU, fp16 and bf16 at most WR_XL_F16_BPC.  Measured: it gains for
// MXFP4 up to h = 6144, and for the other types when the gate/up blocks are
// few; it costs with many rounds of residency (Mixtral, 3584 blocks) or at
// h = 6144.  fp16 and bf16 take the lower bound because the register path
// has the down blocks' LDS-staged prefetch, which the x copy leaves no room
// for (Mixtral tp4 shard, 3.5 blocks per CU: 45.2 us against 48.3 with x in
// LDS; tp8 shard, 1.75 per CU: 30.7 against 29.6).
#ifndef WR_XL_FP8_MAXH
#define WR_XL_FP8_MAXH 4096
#endif
#ifndef WR_XL_F16_MAXH
#define WR_XL_F16_MAXH 4096
#endif
#ifndef WR_XL_FP8_BPC
#define WR_XL_FP8_BPC 4
#endif
#ifndef WR_XL_F16_BPC
#define WR_XL_F16_BPC 2
#endif
#ifndef WR_XL_FP4_MAXH
#define WR_XL_FP4_MAXH 6144
#endif
// Down blocks of the single-token fused kernel (register-path variant, 16-byte
// weight vectors) also stage this many 1 KB row-chunks per wave of their
// next down chunks in LDS before the hand-off wait, with direct global-to-LDS
// loads (no registers): 8 = 32 KB per block, 2 chunks of 4 rows (fp16, bf16)
// or 1 chunk of 8 rows (fp8).
#ifndef WR_DN_LDS_ROWCHUNKS
#define WR_DN_LDS_ROWCHUNKS 8
#endif
// MXFP4 weights in the single-token fused kernel (32 weights per 128-bit load)
#ifndef WR_F4_U1
#define WR_F4_U1 1   // gate/up column chunks per row per iteration (4 rows per wave)
#endif
#ifndef WR_F4_RPD
#define WR_F4_RPD 8  // output rows per down block
#endif
#ifndef WR_F4_U2
#define WR_F4_U2 1   // column chunks per down tile
#endif
// MXFP4 block scales staged in LDS (x-in-LDS variant) from this intermediate
// size up; smaller layers keep the per-load scale bytes.
#ifndef WR_F4_STG_MIN_I
#define WR_F4_STG_MIN_I 4096
#endif
// LDS buffer of the MXFP4 staged-scale kernel, in bytes: the gate/up role's x
// copy and scale bytes, or the down role's scale copy followed by one 8-row
// chunk per wave staged before the hand-off wait.  39 KB keeps 4 blocks per
// CU (160 KB) with the kernel's other shared words.
#ifndef WR_F4_STG_RAW
#define WR_F4_STG_RAW 39936
#endif
// 1: down blocks poll the last gate/up slot's arrival word alone until it is
// complete, then all 64 words; 0: all 64 words from the start.
#ifndef WR_POLL_ONE
#define WR_POLL_ONE 1
#endif
// MXFP4 x-in-LDS kernels without staged scales: their down blocks also stage
// one more weight chunk per wave in the x copy's bytes before the hand-off.
#ifndef WR_F4_XL_DN_STAGE
#define WR_F4_XL_DN_STAGE 1
#endif

namespace wr {

constexpr int kBlock = 256;  // 4 waves
constexpr int kWavesPerBlock = kBlock / kWave;

// ---------------------------------------------------------------------------
// Router
// ---------------------------------------------------------------------------
// Wave q (0..3) of a 4-wave group: fp32 partial dot over quarter q of the row
// (quarters are whole 64*VEC-element chunks).  Every producer of logits uses
// this and the same combine order, so all of them produce identical bits.
// With want_max it also sets xmax = max |x| over the quarter (every lane),
// from the same loads; the sums are unaffected.
template <typename XT, int VEC>
__device__ __forceinline__ float router_partial(const float* __restrict__ row,
                                                const XT* __restrict__ x, int h, int q,
                                                bool want_max, float& xmax) {
  const int lane = threadIdx.x & (kWave - 1);
  constexpr int CH = kWave * VEC;
  const int span = (h + 4 * CH - 1) / (4 * CH) * CH;
  const int beg = q * span;
  const int end = min(h, beg + span);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float m = 0.0f;
  for (int c0 = beg + lane * VEC; c0 < end; c0 += 8 * CH) {
    float w[8][VEC], xv[8][VEC];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = c0 + u * CH;
      if (c < end) {
        load_x<float, VEC>(row + c, w[u]);
        load_x<XT, VEC>(x + c, xv[u]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) w[u][i] = xv[u][i] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[u & 3] = fmaf(w[u][i], xv[u][i], acc[u & 3]);
    if (want_max) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) m = fmaxf(m, fabsf(xv[u][i]));
    }
  }
  xmax = want_max ? wave_max(m) : 0.0f;
  return wave_sum((acc[0] + acc[1]) + (acc[2] + acc[3]));
}

__device__ __forceinline__ float router_combine(const float* p) {
  return (p[0] + p[1]) + (p[2] + p[3]);
}

// x split into two 16-bit terms for the grouped batched path.  hi == NULL:
// no split.  bf16: bf16 terms x = hi + lo (bf16 keeps fp32's exponent range,
// so no scaling).  Otherwise fp16 terms of x 2^e, e = split_exp(max|x|), and
// exp[b] = e; amax (when not NULL) gets its k words of token b zeroed, every
// kAmaxStride words.
struct XSplit {
  f16* hi;
  f16* lo;
  int32_t* exp;
  unsigned* amax;
  int k;
  int bf16;
};

// grid (E, B), block 256.  Token b's logits go to logits[b * 64 + e] (padded
// so that consumers can read all 64 with scalar loads).  Block (0, 0) also
// zeroes the 8-byte words at zero + i * zstride, i < nzero <= kBlock (the
// single-token kernel's arrival words, timeout flag and claim counters),
// which the next kernel on the stream reads.  With xs.hi != NULL,
// block (e, b) also writes its 1/E
// share of token b's split x (XSplit); every block of the token derives the
// same exponent from the whole row.
template <typename XT, int VEC>
__global__ __launch_bounds__(kBlock) void k_router_logits(const float* __restrict__ gate_w,
                                                          const XT* __restrict__ x,
                                                          float* __restrict__ logits, int E,
                                                          int h, unsigned* __restrict__ zero,
                                                          int nzero, int zstride, XSplit xs) {
  __shared__ float part[4];
  __shared__ float pmax[4];
  const int q = threadIdx.x / kWave;
  const int e = blockIdx.x, b = blockIdx.y;
  const bool scaled = xs.hi != nullptr && !xs.bf16;
  float m = 0.0f;
  const float p = router_partial<XT, VEC>(gate_w + (int64_t)e * h, x + (int64_t)b * h, h, q,
                                          scaled, m);
  if ((threadIdx.x & (kWave - 1)) == 0) {
    part[q] = p;
    pmax[q] = m;
  }
  if (zero != nullptr && e == 0 && b == 0 && (int)threadIdx.x < nzero)
    *reinterpret_cast<uint64_t*>(zero + (int64_t)threadIdx.x * zstride) = 0ull;
  __syncthreads();
  if (threadIdx.x == 0) logits[(int64_t)b * WR_MAX_EXPERTS + e] = router_combine(part);
  if (xs.hi != nullptr) {
    const XT* xb = x + (int64_t)b * h;
    const int ex = scaled ? split_exp(fmaxf(fmaxf(pmax[0], pmax[1]), fmaxf(pmax[2], pmax[3])),
                                      std::is_same<XT, f16>::value)
                          : 0;
    const int cs = (h + E - 1) / E;
    const int end = min(h, (e + 1) * cs);
    for (int i = e * cs + (int)threadIdx.x; i < end; i += kBlock) {
      const float v = (float)xb[i];
      if (xs.bf16) {
        const __bf16 bh = (__bf16)v;
        const __bf16 bl = (__bf16)(v - (float)bh);
        xs.hi[(int64_t)b * h + i] = __builtin_bit_cast(f16, bh);
        xs.lo[(int64_t)b * h + i] = __builtin_bit_cast(f16, bl);
      } else {
        const float vs = ldexpf(v, ex);
        const f16 vh = (f16)vs;
        xs.hi[(int64_t)b * h + i] = vh;
        xs.lo[(int64_t)b * h + i] = (f16)(vs - (float)vh);
      }
    }
    if (e == 0) {
      if (threadIdx.x == 0 && xs.exp != nullptr) xs.exp[b] = ex;
      if (xs.amax != nullptr && (int)threadIdx.x < xs.k)
        xs.amax[((int64_t)b * xs.k + threadIdx.x) * BatchWs::kAmaxStride] = 0u;
    }
  }
}

// Standalone gate: grid B, block 1024 (four 4-wave groups).  Group g handles
// experts g, g+4, ...; wave 0 then selects and writes ids and weights.
template <typename XT, int VEC>
__global__ __launch_bounds__(1024) void k_gate_topk(const float* __restrict__ gate_w,
                                                    const XT* __restrict__ x, int E, int h,
                                                    int k, int renorm,
                                                    int32_t* __restrict__ ids_out,
                                                    float* __restrict__ w_out) {
  __shared__ float part[WR_MAX_EXPERTS][4];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int g = wave / 4, q = wave % 4;
  const int b = blockIdx.x;
  for (int e = g; e < E; e += 4) {
    float unused;
    const float p =
        router_partial<XT, VEC>(gate_w + (int64_t)e * h, x + (int64_t)b * h, h, q, false, unused);
    if (lane == 0) part[e][q] = p;
  }
  __syncthreads();
  if (wave == 0) {
    const float l = lane < E ? router_combine(part[lane]) : 0.0f;
    TopK t;
    wave_select_topk_reg(l, E, k, renorm, t);
#pragma unroll
    for (int kk = 0; kk < WR_MAX_TOPK; ++kk) {
      if (kk < k && lane == kk) {
        ids_out[(int64_t)b * k + kk] = t.id[kk];
        w_out[(int64_t)b * k + kk] = t.w[kk];
      }
    }
  }
}

// MXFP4: the block-scale bytes of row r of matrix m (0 gate, 1 up, 2 down)
// of the expert block at blk ([I][h/32], [I][h/32], [h][I/32] after the
// codes); the scale of element c of the row is at [c / 32].  nullptr for the
// other types.
template <typename WT>
__device__ __forceinline__ const uint8_t* mx_row(const WT* blk, const Geom& g, int m, int64_t r) {
  if constexpr (std::is_same<WT, fp4x2>::value) {
    const int64_t per = (int64_t)g.I * g.h / 32;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(blk) + g.off_scale + m * per;
    return base + r * ((m == 2 ? g.I : g.h) / 32);
  } else {
    (void)blk; (void)g; (void)m; (void)r;
    return nullptr;
  }
}

template <typename WT>
__device__ __forceinline__ const uint8_t* mx_at(const uint8_t* row, int64_t c) {
  if constexpr (std::is_same<WT, fp4x2>::value) return row + c / 32;
  else return nullptr;
}

// act for intermediate index r of the expert block at blk, from the gate and
// up dot products gs and us and the gate weight wk:
//   wk * silu(gs) * us                                  (unscaled types)
//   wk * silu(gs * s_gate[r]) * (us * s_up[r])          (fp8 row scales)
// The fp8 scales of rows [r0, r0 + RPW) are loaded by every lane, with the
// item's weights and outside any branch, so that the epilogue waits for
// them once (rows past nrows repeat a valid row; their values are unused).
template <typename WT, int RPW>
struct RowScales {
  float gate[RPW], up[RPW];
};
template <typename WT, int RPW>
__device__ __forceinline__ void load_row_scales(RowScales<WT, RPW>& rs, const WT* blk,
                                                const Geom& g, int r0, int nrows) {
#pragma unroll
  for (int j = 0; j < RPW; ++j) rs.gate[j] = rs.up[j] = 1.0f;
  if constexpr (std::is_same<WT, fp8w>::value) {
    const float* sc = wscales(blk, g.off_scale);
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int r = r0 + max(min(j, nrows - 1), 0);
      rs.gate[j] = sc[r];
      rs.up[j] = sc[g.I + r];
    }
  }
}
template <typename WT, int RPW>
__device__ __forceinline__ float act_value(const RowScales<WT, RPW>& rs, int j, float wk,
                                           float gs, float us) {
  if constexpr (std::is_same<WT, fp8w>::value) {
    return wk * (silu(gs * rs.gate[j]) * (us * rs.up[j]));
  } else {
    return wk * (silu(gs) * us);
  }
}

// fp8: scale of down row `row` of selected expert kk (s_down follows the I
// gate and I up scales).
template <typename WT>
__device__ __forceinline__ float down_scale(const WT* wbuf, const Geom& g, const TopK& t, int kk,
                                            int row) {
  return wscales(wbuf + (int64_t)topk_id(t, kk) * g.stride, g.off_scale)[2 * g.I + row];
}

// ---------------------------------------------------------------------------
// Gate/up: grid (ceil(nw / 4), B).  Wave w of token b owns items
// share(k * ceil(I / RPW), w, nw); item it covers rows [r0, r0 + RPW) of
// selected expert kk = it / ceil(I / RPW).
// ---------------------------------------------------------------------------
template <typename WT, typename XT, int VEC, int RPW, int U>
__global__ __launch_bounds__(kBlock) void k_gateup(const WT* __restrict__ wbuf,
                                                   const XT* __restrict__ x,
                                                   const float* __restrict__ logits,
                                                   float* __restrict__ act,
                                                   int32_t* __restrict__ ids_out,
                                                   float* __restrict__ w_out, Geom g, int nw) {
  typedef typename WVec<WT, VEC>::type V;
  constexpr int CH = kWave * VEC;
  const int lane = threadIdx.x & (kWave - 1);
  const int b = blockIdx.y;
  const int w = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (w >= nw) return;  // wave-uniform
  const int items = (g.I + RPW - 1) / RPW;
  int ib, ie;
  share(g.k * items, w, nw, ib, ie);

  TopK t;
  wave_select_topk(logits + (int64_t)b * WR_MAX_EXPERTS, g.E, g.k, g.renorm, t);
  if (w == 0) {
#pragma unroll
    for (int kk = 0; kk < WR_MAX_TOPK; ++kk) {
      if (kk < g.k && lane == kk) {
        if (ids_out != nullptr) ids_out[(int64_t)b * g.k + kk] = t.id[kk];
        if (w_out != nullptr) w_out[(int64_t)b * g.k + kk] = t.w[kk];
      }
    }
  }
  const XT* xb = x + (int64_t)b * g.h;

  for (int it = ib; it < ie; ++it) {
    const int kk = it / items;
    const int r0 = (it - kk * items) * RPW;
    const int e = topk_id(t, kk);
    const WT* blk = wbuf + (int64_t)e * g.stride;
    const WT* G = blk + eoff<WT>((int64_t)r0 * g.h);
    const WT* Up = G + g.off_up;
    const int nrows = min(RPW, g.I - r0);
    RowScales<WT, RPW> rs;
    load_row_scales<WT, RPW>(rs, blk, g, r0, nrows);

    float ag[RPW], au[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) ag[j] = au[j] = 0.0f;

    for (int c0 = lane * VEC; c0 < g.h; c0 += U * CH) {
      V wg[U][RPW], wu[U][RPW];
      float xv[U][VEC];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * CH;
        const bool ok = c < g.h;
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
          const bool okj = ok && j < nrows;
          wg[u][j] = okj ? load_wq<WT, VEC>(G + eoff<WT>((int64_t)j * g.h + c),
                                            mx_at<WT>(mx_row(blk, g, 0, r0 + j), c))
                         : vzero<V>();
          wu[u][j] = okj ? load_wq<WT, VEC>(Up + eoff<WT>((int64_t)j * g.h + c),
                                            mx_at<WT>(mx_row(blk, g, 1, r0 + j), c))
                         : vzero<V>();
        }
        if (ok) {
          load_x<XT, VEC>(xb + c, xv[u]);
        } else {
#pragma unroll
          for (int i = 0; i < VEC; ++i) xv[u][i] = 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            ag[j] = fmaf(wdec<WT>(wg[u][j], i), xv[u][i], ag[j]);
            au[j] = fmaf(wdec<WT>(wu[u][j], i), xv[u][i], au[j]);
          }
    }

    const float wk = topk_w(t, kk);
    float* a = act + ((int64_t)b * g.k + kk) * g.I + r0;
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const float gs = wave_sum(ag[j]);
      const float us = wave_sum(au[j]);
      if (lane == 0 && j < nrows) a[j] = act_value<WT, RPW>(rs, j, wk, gs, us);
    }
  }
}

// ---------------------------------------------------------------------------
// Down: grid (ceil(nw / 4), B).  Wave w of token b owns output-row items
// share(ceil(h / RPD), w, nw); for each it streams rows [r0, r0 + RPD) of
// every selected down matrix against that expert's act vector.
// ---------------------------------------------------------------------------
template <typename WT, typename OT, int VEC, int RPD, int U>
__global__ __launch_bounds__(kBlock) void k_down(const WT* __restrict__ wbuf,
                                                 const float* __restrict__ logits,
                                                 const float* __restrict__ act,
                                                 OT* __restrict__ out, Geom g, int nw) {
  typedef typename WVec<WT, VEC>::type V;
  constexpr int CH = kWave * VEC;
  const int lane = threadIdx.x & (kWave - 1);
  const int b = blockIdx.y;
  const int w = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (w >= nw) return;  // wave-uniform
  int ib, ie;
  share((g.h + RPD - 1) / RPD, w, nw, ib, ie);

  TopK t;
  wave_select_topk(logits + (int64_t)b * WR_MAX_EXPERTS, g.E, g.k, g.renorm, t);
  const float* ab = act + (int64_t)b * g.k * g.I;

  for (int it = ib; it < ie; ++it) {
    const int r0 = it * RPD;
    const int nrows = min(RPD, g.h - r0);
    float acc[RPD];
#pragma unroll
    for (int j = 0; j < RPD; ++j) acc[j] = 0.0f;

    constexpr bool kFp8 = std::is_same<WT, fp8w>::value;
    for (int kk = 0; kk < g.k; ++kk) {
      const WT* blk = wbuf + (int64_t)topk_id(t, kk) * g.stride;
      const WT* D = blk + g.off_down + eoff<WT>((int64_t)r0 * g.I);
      const float* a = ab + (int64_t)kk * g.I;
      // fp8: this expert's rows accumulate apart and are scaled per row below.
      float ek[RPD];
#pragma unroll
      for (int j = 0; j < RPD; ++j) ek[j] = 0.0f;
      float* const dst = kFp8 ? ek : acc;
      for (int c0 = lane * VEC; c0 < g.I; c0 += U * CH) {
        V wv[U][RPD];
        float av[U][VEC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = c0 + u * CH;
          const bool ok = c < g.I;
#pragma unroll
          for (int j = 0; j < RPD; ++j)
            wv[u][j] = (ok && j < nrows)
                           ? load_wq<WT, VEC>(D + eoff<WT>((int64_t)j * g.I + c),
                                              mx_at<WT>(mx_row(blk, g, 2, r0 + j), c))
                           : vzero<V>();
          if (ok) {
            load_x<float, VEC>(a + c, av[u]);
          } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) av[u][i] = 0.0f;
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < RPD; ++j)
#pragma unroll
            for (int i = 0; i < VEC; ++i) dst[j] = fmaf(wdec<WT>(wv[u][j], i), av[u][i], dst[j]);
      }
      if constexpr (kFp8) {
#pragma unroll
        for (int j = 0; j < RPD; ++j)
          if (j < nrows) acc[j] = fmaf(down_scale(wbuf, g, t, kk, r0 + j), ek[j], acc[j]);
      }
    }

#pragma unroll
    for (int j = 0; j < RPD; ++j) {
      const float s = wave_sum(acc[j]);
      if (lane == 0 && j < nrows) out[(int64_t)b * g.h + r0 + j] = to_out<OT>(s);
    }
  }
}

// ---------------------------------------------------------------------------
// Single-token fused FFN: ONE launch, grid = [n1 gate/up blocks][n2 down
// blocks], 4 waves per block.
//
// act is [k][act_row] fp32, in chunks of COLS = 4 RPW columns (RPW = rows
// per wave, 2 or 4); chunk G = kk * bpk + j holds columns [COLS j, COLS j +
// COLS) of selected expert kk (bpk = chunks per expert, act_row = bpk COLS).
// Gate/up block b computes chunk G = chunk_of_block<LB>(b): its wave w
// computes rows COLS j + RPW w .. + RPW of expert kk's gate and up matrices and
// stores w_kk * silu(gate . x) * (up . x) with agent-scope stores, which are
// written through to memory.  When all of them have completed, the block
// adds its arrival to arrival word b mod 64 (the words sit 256 bytes apart so
// that their atomics do not serialise on one address).
//
// Down block: owns RPD output rows.  It issues the loads of its first tile of
// down weights (they do not depend on act), then wave 0 polls the last
// slot's arrival word (lane 0 alone) and then the 64 words until all n1
// gate/up blocks have arrived, then the 4 waves stream strided
// column chunks of every selected down matrix and combine in LDS.  Every
// output row is written once.
//
// Why this cannot deadlock: workgroups of a grid are dispatched in index
// order (on each XCD), so every gate/up block is dispatched before any down
// block that could occupy its slot, and gate/up blocks never wait.  Every wait
// is nevertheless bounded (about 0.2 s), so the kernel cannot hang.  On
// expiry the block sets the timeout word and writes NaN to its output rows
// (its act reads may have been incomplete), so a broken hand-off can never
// pass for a plausible result; wr_fused_moe_status reports the word.
//
// Why down blocks read fresh act without invalidating L2 (each XCD has its
// own L2, not coherent with the others): blocks are dispatched to the XCDs
// round-robin, block b to XCD (b + r) mod 8 for some rotation r (0 for a
// plain launch; a launch from a captured graph was measured at r = 7).  So
// blocks whose indices agree mod 8 share an XCD.  A 128-byte L2 line holds
// LB = 32 / COLS chunks (4 or 2).  chunk_of_block<LB> maps the LB blocks
// 8 LB m + 8 s + x (s < LB), which share an XCD, to the LB chunks
// 8 LB m + LB x + s, i.e. one line.  So every act line is written by one XCD
// only.  At kernel start no L2 holds act lines (the kernel-boundary
// acquire invalidates them), and no wave reads act before every gate/up block
// has arrived.  Hence an XCD's L2 holds an act line only if its own writers
// put it there (all of the line's writers go through that L2) or if a reader
// fetched it from memory after it was complete.  Each gate/up block adds
// the rotation it actually ran with, r = (HW_REG_XCC_ID - b) mod 8, and r^2
// to its arrival word (arrival_word); a down block sums the 64 words it
// waited on and, unless (sum r)^2 = n sum r^2 (one rotation for the whole
// grid), falls back to a full agent-scope acquire (L2 and L1 invalidate).
// Otherwise it only invalidates its CU's L1,
// in case a writer on the same CU left a partial line there.  This saves the L2
// invalidate per down block (about 6 us per layer at the Mixtral shape) and
// keeps act dense, so the readers' loads stay fully coalesced.
// ---------------------------------------------------------------------------
struct Handoff {
  unsigned* ctrl;       // the control block: FusedWs::kCtrlWords 8-byte words zeroed at the
                        // start of each call, FusedWs::kCounterStride words apart
  uint64_t* slot;       // router slots (ROUTE), 2 words per expert (FusedWs::kSlotWord)
  const float* gate_w;  // router matrix [E][h]; nullptr: the logits are read from `logits`
  int nb;               // blocks in the grid
  int rvec;             // router rows and x in 128-bit loads (else scalar)
  unsigned* cnt;        // FusedWs::kCounters 64-bit arrival words, FusedWs::kCounterStride
                        // words apart (arrival_word)
  unsigned* timeout;    // set to 1 if a wait expired (that block's rows are then NaN)
  unsigned* host_flag;  // host-visible word also set to 1 then, or nullptr
  unsigned* claim;      // FusedWs::kClasses claim counters, FusedWs::kCounterStride words apart
  int n1;               // gate/up chunk slots, a multiple of 8 LB: one arrival each
  int n1b;              // gate/up blocks launched (the first n1b block ids), a multiple of
                        // 8 LB, at most n1; slots n1b .. n1 - 1 are claimed by them
  int chunks;           // k * bpk
  unsigned spin_limit;  // polls before a wait gives up
  unsigned wait_extra;  // added to every arrival target: 0, or (tests) a wait that cannot complete
#if WR_TIMELINE
  uint64_t* tl;         // per-block records (include/wr_timeline.h)
#endif
};

// Arrival word of counter (slot mod 64): 64 bits, {arrivals in bits 0-15, the
// sum of their XCD rotations r = (HW_REG_XCC_ID - block) mod 8 in bits 16-31,
// the sum of r^2 in bits 32-63}, so that one atomic add per gate/up slot
// counts it and records its rotation, and one load per lane gives a down
// block both.  The fields hold ceil(n1 / 64) <= kMaxArrivals arrivals per
// counter without carrying into the next one.
constexpr int kMaxArrivals = 9362;  // 7 kMaxArrivals < 2^16
__device__ __forceinline__ uint64_t* arrival_word(const Handoff& hs, int slot) {
  return reinterpret_cast<uint64_t*>(hs.cnt + (slot % FusedWs::kCounters) *
                                                  FusedWs::kCounterStride);
}
__device__ __forceinline__ uint64_t arrival_bits() {
  const uint64_t r = (xcc_id() - blockIdx.x) & 7u;
  return 1ull | (r << 16) | ((r * r) << 32);
}
__device__ __forceinline__ unsigned arrivals(uint64_t w) { return (unsigned)(w & 0xffffu); }

// A hand-off wait expired: the workspace's timeout word (read by
// wr_fused_moe_status) and the host-visible word (read by
// wr_fused_moe_expired without a synchronisation), both plain stores of 1.
__device__ __forceinline__ void set_expired(const Handoff& hs) {
  __hip_atomic_store(hs.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (hs.host_flag != nullptr)
    __hip_atomic_store(hs.host_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// WR_TIMELINE builds: thread 0 stores the wall clock as record `ev` of its
// workgroup (include/wr_timeline.h), a plain store that nothing waits for.
#if WR_TIMELINE
#define WR_TL_MARK(hs, ev)                                                              \
  do {                                                                                  \
    if (threadIdx.x == 0 && blockIdx.x < WR_TIMELINE_MAX_BLOCKS)                        \
      (hs).tl[(size_t)blockIdx.x * WR_TIMELINE_EVENTS + (ev)] = (uint64_t)wall_clock64(); \
  } while (0)
#define WR_TL_SET(hs, ev, v)                                                     \
  do {                                                                           \
    if (threadIdx.x == 0 && blockIdx.x < WR_TIMELINE_MAX_BLOCKS)                 \
      (hs).tl[(size_t)blockIdx.x * WR_TIMELINE_EVENTS + (ev)] = (uint64_t)(v);   \
  } while (0)
#else
#define WR_TL_MARK(hs, ev) \
  do {                     \
  } while (0)
#define WR_TL_SET(hs, ev, v) \
  do {                       \
  } while (0)
#endif

// The router inside k_fused_ffn, so that a layer is one launch as in the
// reference (src/fused_moe.cu:100-150 computes the logits inside its kernel).
//
// Block b computes router rows e = b, b + nb, ... < E with the router
// kernel's arithmetic (router_partial, router_combine: the same bits), or
// with gate_w == nullptr reads them from `logits` (written by an earlier
// router launch), and publishes row e as slot e: the 64-bit words
// {logit, tag lo} and {logit, tag hi}, where the tag is this launch's
// (launch_tag), in each of FusedWs::kSlotReplicas copies.  Block 0 first
// zeroes the control words of the hand-off (arrival words, timeout word,
// claim counters) and waits for those stores to complete.
// Wave 0 of every block then polls the E slots of its copy until each
// carries this launch's tag in both words, and every wave selects from the
// logits read (wave_select_topk_reg).
//
// Why nothing needs resetting between calls: a slot written by an earlier
// launch carries that launch's tag, never this one's, and any other bytes
// match both 32-bit halves with probability 2^-64.  Why the control words are
// zero when used: every block reads or updates them only after it has seen
// slot 0, which block 0 publishes after its zero stores completed.  Why this
// cannot deadlock: the blocks that compute rows are the lowest ids of the
// grid (at most 64 of them), dispatched before any other, and they wait for
// nothing before they publish.  The poll is bounded like the hand-off wait;
// on expiry the block sets the timeout word and returns false (no
// selection).  Every thread of the block must call it.
template <typename XT>
__device__ __forceinline__ bool route_and_select(const XT* __restrict__ x,
                                                 const float* __restrict__ logits, const Geom& g,
                                                 const Handoff& hs, TopK& t) {
  __shared__ float s_part[kWavesPerBlock];
  __shared__ float s_logit[kWave];
  __shared__ int s_routed;
  static_assert(FusedWs::kCtrlWords <= kBlock, "one thread zeroes each control word");
  constexpr int kRepWords = FusedWs::kReplicaBytes / 8;
  const int lane = threadIdx.x & (kWave - 1);
  const int q = (int)threadIdx.x / kWave;
  uint32_t tlo, thi;
  launch_tag(tlo, thi);
  // Block 0's zero stores go out before its router loads, so that the wait
  // for the loads covers them too.
  if (blockIdx.x == 0 && (int)threadIdx.x < FusedWs::kCtrlWords)
    __hip_atomic_store(
        reinterpret_cast<uint64_t*>(hs.ctrl + threadIdx.x * FusedWs::kCounterStride), 0ull,
        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int e = blockIdx.x; e < g.E; e += hs.nb) {  // block-uniform
    if (hs.gate_w != nullptr) {
      float unused;
      const float* row = hs.gate_w + (int64_t)e * g.h;
      const float p = hs.rvec ? router_partial<XT, 4>(row, x, g.h, q, false, unused)
                              : router_partial<XT, 1>(row, x, g.h, q, false, unused);
      if (lane == 0) s_part[q] = p;
    }
    if (e == 0) __builtin_amdgcn_s_waitcnt(0);  // this thread's zero store has completed
    __syncthreads();
    if (q == 0 && lane < FusedWs::kSlotReplicas) {  // lane r writes copy r
      const float l = hs.gate_w != nullptr ? router_combine(s_part) : logits[e];
      const uint64_t bits = __float_as_uint(l);
      uint64_t* sp = hs.slot + lane * kRepWords + 2 * e;
      __hip_atomic_store(sp, bits | ((uint64_t)tlo << 32), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(sp + 1, bits | ((uint64_t)thi << 32), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();  // s_part is reused by the next row
  }
  if (q == 0) {
    const uint64_t* rep = hs.slot + (blockIdx.x % FusedWs::kSlotReplicas) * kRepWords;
    float l = 0.0f;
    unsigned spins = 0;
    int ok_all = 1;
    for (;;) {
      bool ok = true;
      if (lane < g.E) {
        const uint64_t a = __hip_atomic_load(rep + 2 * lane, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t b = __hip_atomic_load(rep + 2 * lane + 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        ok = (uint32_t)(a >> 32) == tlo && (uint32_t)(b >> 32) == thi && (uint32_t)a == (uint32_t)b;
        l = __uint_as_float((uint32_t)a);
      }
      if (__ballot(!ok) == 0) break;
      if (++spins > hs.spin_limit) {
        ok_all = 0;
        if (lane == 0) set_expired(hs);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    s_logit[lane] = l;
    if (lane == 0) s_routed = ok_all;
  }
  __syncthreads();
  wave_select_topk_reg(s_logit[lane], g.E, g.k, g.renorm, t);
  return s_routed != 0;
}

// The chunk gate/up block b computes: a permutation of each aligned group of
// 8 LB blocks (LB = chunks per 128-byte act line).
template <int LB>
__host__ __device__ __forceinline__ int chunk_of_block(int b) {
  return (b & ~(8 * LB - 1)) + (b & 7) * LB + ((b >> 3) & (LB - 1));
}

// Rows [r0, r0 + RPW) of selected expert kk's gate/up matrices; the results go
// to a[0 .. RPW) with agent-scope stores.
template <typename WT, typename XT, int VEC, int RPW, int U>
__device__ __forceinline__ void gateup_item(const WT* __restrict__ wbuf, const XT* __restrict__ xb,
                                            float* a, const Geom& g, const TopK& t, int kk,
                                            int r0, int lane, const Handoff* hsp = nullptr) {
  (void)hsp;  // WR_TIMELINE builds of k_fused_ffn record a mark
  typedef typename WVec<WT, VEC>::type V;
  constexpr int CH = kWave * VEC;
  const WT* blk = wbuf + (int64_t)topk_id(t, kk) * g.stride;
  const WT* G = blk + eoff<WT>((int64_t)r0 * g.h);
  const WT* Up = G + g.off_up;
  const int nrows = min(RPW, g.I - r0);
  RowScales<WT, RPW> rs;
  load_row_scales<WT, RPW>(rs, blk, g, r0, nrows);
  float ag[RPW], au[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) ag[j] = au[j] = 0.0f;
  for (int c0 = lane * VEC; c0 < g.h; c0 += U * CH) {
    V wg[U][RPW], wu[U][RPW];
    float xv[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * CH;
      const bool ok = c < g.h;
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const bool okj = ok && j < nrows;
        wg[u][j] = okj ? load_wq<WT, VEC>(G + eoff<WT>((int64_t)j * g.h + c),
                                          mx_at<WT>(mx_row(blk, g, 0, r0 + j), c))
                       : vzero<V>();
        wu[u][j] = okj ? load_wq<WT, VEC>(Up + eoff<WT>((int64_t)j * g.h + c),
                                          mx_at<WT>(mx_row(blk, g, 1, r0 + j), c))
                       : vzero<V>();
      }
      if (ok) {
        load_x<XT, VEC>(xb + c, xv[u]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) xv[u][i] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < RPW; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          ag[j] = fmaf(wdec<WT>(wg[u][j], i), xv[u][i], ag[j]);
          au[j] = fmaf(wdec<WT>(wu[u][j], i), xv[u][i], au[j]);
        }
  }
#if WR_TIMELINE
  if (hsp != nullptr) WR_TL_MARK(*hsp, 7);
#endif
  const float wk = topk_w(t, kk);
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const float gs = wave_sum(ag[j]);
    const float us = wave_sum(au[j]);
    if (lane == 0 && j < nrows)
      __hip_atomic_store(a + j, act_value<WT, RPW>(rs, j, wk, gs, us), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// x staged in LDS (fp8 and MXFP4 gate/up blocks), in x's own dtype.  The
// copy is made of 16-byte slots; each VEC-element group of x (DS = VEC / E16
// slots, E16 elements per slot) is followed by one pad slot, so that the VEC
// values of lane l start at l (DS + 1) slots and the ds_read_b128s of 16
// consecutive lanes hit 16 distinct 4-bank groups.  h <= xl_max_h<WT>(): the
// copy is a static array of that size (at most 28 KB, so 4 blocks still fit a
// CU's LDS), because dynamic LDS keeps the compiler from holding the kernel's
// small arrays in registers.
template <typename WT>
constexpr int xl_max_h() {
  if constexpr (std::is_same<WT, fp8w>::value) return WR_XL_FP8_MAXH;
  if constexpr (std::is_same<WT, fp4x2>::value) return WR_XL_FP4_MAXH;
  if constexpr (std::is_same<WT, f16>::value || std::is_same<WT, bf16w>::value)
    return WR_XL_F16_MAXH;
  return 0;
}
template <typename XT, int VEC>
struct XlLayout {
  static constexpr int kE16 = 16 / (int)sizeof(XT);  // x elements per slot
  static constexpr int kDS = VEC / kE16;            // data slots per group
  static constexpr int kGS = kDS + 1;               // slots per group
  static_assert(VEC % kE16 == 0, "a group is whole slots");
  __host__ __device__ static constexpr int slots(int h) { return h / VEC * kGS; }
  __host__ __device__ static constexpr size_t bytes(int h) { return (size_t)slots(h) * 16; }
};

// MXFP4 with its block-scale bytes staged in LDS (STG): the weight loads
// fetch only the codes, and the scale byte is filled in from the LDS copy
// before the codes are decoded.
template <typename WT, int VEC, bool STG>
__device__ __forceinline__ typename WVec<WT, VEC>::type load_wq_or_codes(const WT* p,
                                                                        const uint8_t* sc) {
  if constexpr (STG) {
    static_assert(std::is_same<WT, fp4x2>::value && VEC == 32, "codes-only loads are MXFP4");
    (void)sc;
    typename WVec<WT, VEC>::type v;
    v.q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    v.e = 127u;
    return v;
  } else {
    return load_wq<WT, VEC>(p, sc);
  }
}

// Loads of round c0 of rows [r0, r0 + nrows) of one gate/up item.
template <typename WT, int VEC, int RPW, int U, bool STG = false>
__device__ __forceinline__ void gateup_issue(typename WVec<WT, VEC>::type (&wg)[U][RPW],
                                             typename WVec<WT, VEC>::type (&wu)[U][RPW],
                                             const WT* blk, const WT* G, const WT* Up,
                                             const Geom& g, int r0, int nrows, int c0) {
  typedef typename WVec<WT, VEC>::type V;
  constexpr int CH = kWave * VEC;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = c0 + u * CH;
    const bool ok = c < g.h;
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const bool okj = ok && j < nrows;
      wg[u][j] = okj ? load_wq_or_codes<WT, VEC, STG>(G + eoff<WT>((int64_t)j * g.h + c),
                                                      STG ? nullptr
                                                          : mx_at<WT>(mx_row(blk, g, 0, r0 + j), c))
                     : vzero<V>();
      wu[u][j] = okj ? load_wq_or_codes<WT, VEC, STG>(Up + eoff<WT>((int64_t)j * g.h + c),
                                                      STG ? nullptr
                                                          : mx_at<WT>(mx_row(blk, g, 1, r0 + j), c))
                     : vzero<V>();
    }
  }
}

// MXFP4 scale staging: n bytes (a multiple of 4, 4-byte aligned at both ends)
// from global src to LDS dst with direct global-to-LDS dword loads, issued by
// one wave (its 64-dword runs; the LDS base of each load is wave-uniform).
__device__ __forceinline__ void stage_bytes_lds(const uint8_t* src, unsigned char* dst, int n,
                                                int lane) {
  const int ndw = n / 4;
  for (int s0 = 0; s0 < ndw; s0 += kWave) {
    if (s0 + lane < ndw)
      __builtin_amdgcn_global_load_lds(
          static_cast<const void*>(src + 4 * (s0 + lane)),
          (__attribute__((address_space(3))) void*)(dst + 4 * s0), 4, 0, 0);
  }
}

// The block's x copy in LDS (XlLayout).  Slot s of the copy holds x[(s / GS)
// VEC + min(s % GS, DS - 1) E16 ..] (a pad slot repeats the group's last data
// slot).  Wave w fills the 64-slot runs w, w + 4, ... (one wave-uniform LDS
// base per load) with direct global-to-LDS loads; the caller waits for them.
template <typename XT, int VEC>
__device__ __forceinline__ void xl_copy(const XT* __restrict__ xb, unsigned char* xs_raw, int h,
                                        int wave, int lane) {
  typedef XlLayout<XT, VEC> L;
  const int nslots = L::slots(h);
  for (int s0 = wave * kWave; s0 < nslots; s0 += kBlock) {
    const int sl = s0 + lane;
    if (sl < nslots) {
      const int grp = sl / L::kGS;
      const int r = min(sl - grp * L::kGS, L::kDS - 1);
      __builtin_amdgcn_global_load_lds(
          static_cast<const void*>(xb + grp * VEC + r * L::kE16),
          (__attribute__((address_space(3))) void*)(xs_raw + (size_t)s0 * 16), 16,
          0, 0);
    }
  }
}

// x[c .. c + VEC) as fp32 from the copy; zeros for c >= h.
template <typename XT, int VEC>
__device__ __forceinline__ void xl_read(const unsigned char* xs_raw, int c, int h,
                                        float (&xv)[VEC]) {
  typedef XlLayout<XT, VEC> L;
  if (c < h) {
    const unsigned char* xp = xs_raw + (size_t)(c / VEC) * L::kGS * 16;
#pragma unroll
    for (int q = 0; q < L::kDS; ++q) {
      if constexpr (std::is_same<XT, float>::value) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(xp + 16 * q);
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[4 * q + i] = v[i];
      } else {
        const f16x8 v = *reinterpret_cast<const f16x8*>(xp + 16 * q);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[8 * q + i] = (float)v[i];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) xv[i] = 0.0f;
  }
}

// gateup_item with x read from the block's LDS copy (XlLayout).  Every wave
// of the block calls it, because the copy ends in a block barrier; a wave
// without an item passes nrows = 0.  The copy is made with direct
// global-to-LDS loads (no registers), issued before the first round of
// weight loads; one wait covers both, so the weights are the only
// long-lived registers and the copy costs no extra round trip.
template <typename WT, typename XT, int VEC, int RPW, int U, bool STG>
__device__ __forceinline__ void gateup_item_xl(const WT* __restrict__ wbuf,
                                               const XT* __restrict__ xb, float* a,
                                               const Geom& g, int eid, float wk, int r0,
                                               int nrows, int lane, unsigned char* xs_raw,
                                               const Handoff& hs) {
  (void)hs;  // WR_TIMELINE builds record two marks
  typedef typename WVec<WT, VEC>::type V;
  typedef XlLayout<XT, VEC> L;
  constexpr int CH = kWave * VEC;
  const WT* blk = wbuf + (int64_t)eid * g.stride;
  const WT* G = blk + eoff<WT>((int64_t)r0 * g.h);
  const WT* Up = G + g.off_up;

  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  xl_copy<XT, VEC>(xb, xs_raw, g.h, wave, lane);
  // STG (MXFP4 with h a multiple of 128): this wave's rows' block-scale
  // bytes, gate then up, [m][j][h / 32], copied to its own LDS area beside x
  // with the same kind of loads, so that each code load needs no scale load.
  const int hb = g.h / 32;
  unsigned char* scl =
      STG ? xs_raw + L::bytes(xl_max_h<WT>()) + wave * 2 * RPW * (xl_max_h<WT>() / 32) : xs_raw;
  if constexpr (STG) {
    if (nrows > 0) {
      stage_bytes_lds(mx_row(blk, g, 0, r0), scl, nrows * hb, lane);
      stage_bytes_lds(mx_row(blk, g, 1, r0), scl + RPW * hb, nrows * hb, lane);
    }
  } else {
    (void)hb;
    (void)scl;
  }
  V wg[U][RPW], wu[U][RPW];
  gateup_issue<WT, VEC, RPW, U, STG>(wg, wu, blk, G, Up, g, r0, nrows, lane * VEC);
  RowScales<WT, RPW> rs;
  load_row_scales<WT, RPW>(rs, blk, g, r0, nrows);
  __builtin_amdgcn_s_waitcnt(0);  // the copy's loads (and the weights) have landed
  __syncthreads();
  WR_TL_MARK(hs, 2);

  float ag[RPW], au[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) ag[j] = au[j] = 0.0f;
  for (int c0 = lane * VEC; c0 < g.h; c0 += U * CH) {
    if (c0 != lane * VEC)
      gateup_issue<WT, VEC, RPW, U, STG>(wg, wu, blk, G, Up, g, r0, nrows, c0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * CH;
      float xv[VEC];
      if constexpr (STG) {
        // Only rows that were loaded: the other rows' vectors are zero codes
        // with scale 1, and their LDS bytes were never written.
        if (c < g.h) {
#pragma unroll
          for (int j = 0; j < RPW; ++j) {
            if (j < nrows) {
              wg[u][j].e = scl[j * hb + c / 32];
              wu[u][j].e = scl[(RPW + j) * hb + c / 32];
            }
          }
        }
      }
      xl_read<XT, VEC>(xs_raw, c, g.h, xv);
#pragma unroll
      for (int j = 0; j < RPW; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          ag[j] = fmaf(wdec<WT>(wg[u][j], i), xv[i], ag[j]);
          au[j] = fmaf(wdec<WT>(wu[u][j], i), xv[i], au[j]);
        }
    }
  }
  WR_TL_MARK(hs, 7);
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const float gs = wave_sum(ag[j]);
    const float us = wave_sum(au[j]);
    if (lane == 0 && j < nrows)
      __hip_atomic_store(a + j, act_value<WT, RPW>(rs, j, wk, gs, us), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Down tile of a fused down block: U column chunks q = q0 + 4 u (chunk q is
// columns [(q mod nch) * 64 VEC, +64 VEC) of selected expert q / nch), RPD rows
// from r0.
template <typename WT, int VEC, int RPD, int U, bool STG = false>
__device__ __forceinline__ void down_tile_load(typename WVec<WT, VEC>::type (&wv)[U][RPD],
                                               const WT* __restrict__ wbuf, const Geom& g,
                                               const TopK& t, int r0, int nrows, int q0,
                                               int nch, int lane) {
  typedef typename WVec<WT, VEC>::type V;
  const int C = g.k * nch;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int q = q0 + u * kWavesPerBlock;
    const bool okq = q < C;                  // wave-uniform
    const int kk = okq ? q / nch : 0;        // a valid selection slot either way
    const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
    const bool ok = okq && c < g.I;
    const WT* blk = wbuf + (int64_t)topk_id(t, kk) * g.stride;
    const WT* D = blk + g.off_down + eoff<WT>((int64_t)r0 * g.I + c);
#pragma unroll
    for (int j = 0; j < RPD; ++j)
      wv[u][j] = (ok && j < nrows)
                     ? load_wq_or_codes<WT, VEC, STG>(
                           D + eoff<WT>((int64_t)j * g.I),
                           STG ? nullptr : mx_at<WT>(mx_row(blk, g, 2, r0 + j), c))
                     : vzero<V>();
  }
}

// MXFP4 down tile with staged scales: the scale byte of each loaded vector
// from the block's LDS copy, [kk][j][I / 32] (rows that were not loaded keep
// the zero vector's scale 1).
template <typename WT, int VEC, int RPD, int U>
__device__ __forceinline__ void down_tile_scales(typename WVec<WT, VEC>::type (&wv)[U][RPD],
                                                 const unsigned char* scl, const Geom& g,
                                                 int nrows, int q0, int nch, int lane) {
  const int C = g.k * nch, ib = g.I / 32;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int q = q0 + u * kWavesPerBlock;
    const int kk = q < C ? q / nch : 0;
    const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
    if (q < C && c < g.I) {
#pragma unroll
      for (int j = 0; j < RPD; ++j)
        if (j < nrows) wv[u][j].e = scl[(kk * RPD + j) * ib + c / 32];
    }
  }
}

// acc[j] += tile row j . act over the tile's chunks (act of expert kk at
// act + kk * act_row).  fp8: each chunk's products are summed apart and
// added times the row scale of the chunk's expert, sdn[kk * RPD + j].
template <typename WT, typename V, int VEC, int RPD, int U>
__device__ __forceinline__ void down_tile_fma(float (&acc)[RPD], const V (&wv)[U][RPD],
                                              const float* act, const Geom& g,
                                              int64_t act_row, int q0, int nch, int lane,
                                              const float* sdn) {
  const int C = g.k * nch;
  float av[U][VEC];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int q = q0 + u * kWavesPerBlock;
    const int kk = q / nch;
    const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
    if (q < C && c < g.I) {
      load_x<float, VEC>(act + kk * act_row + c, av[u]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) av[u][i] = 0.0f;
    }
  }
  if constexpr (std::is_same<WT, fp8w>::value) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = q0 + u * kWavesPerBlock;
      const int kk = q < C ? q / nch : 0;  // past the end: zero products, any valid scale
#pragma unroll
      for (int j = 0; j < RPD; ++j) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) d = fmaf(wdec<WT>(wv[u][j], i), av[u][i], d);
        acc[j] = fmaf(sdn[kk * RPD + j], d, acc[j]);
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < RPD; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[j] = fmaf(wdec<WT>(wv[u][j], i), av[u][i], acc[j]);
  }
}

// MXFP4 block-scale staging in LDS (STG): bytes of the kernel-wide LDS
// buffer beyond the x copy, per gate/up wave (2 RPW rows of the largest h).
template <typename WT, int RPW, bool STG>
constexpr size_t stg_gu_bytes() {
  return STG ? (size_t)kWavesPerBlock * 2 * RPW * (xl_max_h<WT>() / 32) : 0;
}
// Bytes of the kernel-wide LDS buffer of k_fused_ffn.
template <typename WT, typename XT, int VEC, int RPW, bool XL, bool STG>
constexpr size_t fused_raw_bytes() {
  if constexpr (XL) {
    constexpr size_t gu = XlLayout<XT, VEC>::bytes(xl_max_h<WT>()) + stg_gu_bytes<WT, RPW, STG>();
    static_assert(!STG || gu <= WR_F4_STG_RAW, "the staged-scale buffer holds the gate/up copy");
    return STG ? (size_t)WR_F4_STG_RAW : gu;
  } else {
    return 16;
  }
}

// WR_TIMELINE builds hold the claiming variant to 4 blocks per CU, the
// occupancy its default build has, so that the timeline shows the launch
// configuration the default build runs.
#if WR_TIMELINE
#define WR_FUSED_BOUNDS __launch_bounds__(kBlock, CLAIM ? 4 : 1)
#else
#define WR_FUSED_BOUNDS __launch_bounds__(kBlock)
#endif
template <typename WT, typename XT, int VEC, int RPW, int U1, int RPD, int U2, bool XL,
          bool STG, bool CLAIM = false, bool ROUTE = false>
__global__ WR_FUSED_BOUNDS void k_fused_ffn(
    const WT* __restrict__ wbuf, const XT* __restrict__ x, const float* __restrict__ logits,
    float* act, XT* __restrict__ out, int32_t* __restrict__ ids_out, float* __restrict__ w_out,
    Geom g, Handoff hs) {
  typedef typename WVec<WT, VEC>::type V;
  constexpr int COLS = kWavesPerBlock * RPW;  // act columns per gate/up block
  constexpr int LB = 32 / COLS;               // chunks per 128-byte act line
  static_assert(COLS * LB == 32 && COLS <= FusedWs::kMaxActCols, "unsupported rows per wave");
  const int lane = threadIdx.x & (kWave - 1);
  // With XL, readfirstlane keeps the (wave-uniform) wave index, and the item
  // indices derived from it, in SGPRs.
  const int wave = XL ? __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave)
                      : (int)threadIdx.x / kWave;
  const int64_t act_row = FusedWs::act_row(g.I, COLS);

  WR_TL_MARK(hs, 0);
  TopK t;
  bool routed = true;  // false: the router slots' wait expired (ROUTE)
  if constexpr (ROUTE)
    routed = route_and_select<XT>(x, logits, g, hs, t);
  else
    block_select_topk(logits, g.E, g.k, g.renorm, t);
  WR_TL_MARK(hs, 1);
#if WR_TIMELINE
  {
    unsigned hwid;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
    WR_TL_SET(hs, 5, (uint64_t)xcc_id() | ((uint64_t)hwid << 32));
    WR_TL_SET(hs, 6, (int)blockIdx.x < hs.n1b ? 0u : 1u);
  }
#endif
  // The x-in-LDS variant's buffer: the gate/up role's x copy (and, with
  // STG, its waves' scale bytes); the down role's scale copy with STG.
  static_assert(!STG || XL, "scale staging lives in the x-in-LDS variant's buffer");
  __shared__ __align__(16) unsigned char lds_raw[fused_raw_bytes<WT, XT, VEC, RPW, XL, STG>()];

  if ((int)blockIdx.x < hs.n1b) {
    // ---- gate/up block ----
    if (!routed) return;  // the slot wait expired (timeout word set); no arrival
    if (blockIdx.x == 0 && wave == 0) {
#pragma unroll
      for (int kk = 0; kk < WR_MAX_TOPK; ++kk) {
        if (kk < g.k && lane == kk) {
          if (ids_out != nullptr) ids_out[kk] = t.id[kk];
          if (w_out != nullptr) w_out[kk] = t.w[kk];
        }
      }
    }
    const int items = (g.I + RPW - 1) / RPW;
    const int bpk = (items + kWavesPerBlock - 1) / kWavesPerBlock;  // chunks per expert
    // Slot v = this block's id; with CLAIM (fewer blocks launched than slots)
    // then slots n1b + c + 8 i of this block's class c = id mod 8, claimed one
    // at a time until none is left.  A claimed slot's act line is then written
    // only by blocks of one class, as a launched slot's is.  The claiming loop
    // is a separate instantiation: it changes the register allocation of the
    // gate/up role.
    __shared__ int s_claim;
    const int cls = (int)blockIdx.x % FusedWs::kClasses;
    for (int v = blockIdx.x;;) {
      const int G = chunk_of_block<LB>(v);
      if constexpr (XL) {
        // Wave-uniform by construction; readfirstlane keeps them in SGPRs (the
        // TopK reads below take a scalar slot index).
        const int kk = __builtin_amdgcn_readfirstlane(G < hs.chunks ? G / bpk : 0);
        const int it = (G - kk * bpk) * kWavesPerBlock + wave;
        const int nrows = (G < hs.chunks && it < items) ? min(RPW, g.I - it * RPW) : 0;
        gateup_item_xl<WT, XT, VEC, RPW, U1, STG>(wbuf, x, act + kk * act_row + it * RPW, g,
                                                  topk_id(t, kk), topk_w(t, kk),
                                                  nrows > 0 ? it * RPW : 0, nrows, lane, lds_raw,
                                                  hs);
      } else if (G < hs.chunks) {
        const int kk = G / bpk;
        const int it = (G - kk * bpk) * kWavesPerBlock + wave;
        if (it < items)
          gateup_item<WT, XT, VEC, RPW, U1>(wbuf, x, act + kk * act_row + it * RPW, g, t, kk,
                                            it * RPW, lane, &hs);
      }
      __builtin_amdgcn_s_waitcnt(0);  // this wave's act stores have completed
      __syncthreads();
      if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(arrival_word(hs, v), arrival_bits(), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if constexpr (CLAIM)
          s_claim = hs.n1b + cls +
                    FusedWs::kClasses *
                        (int)__hip_atomic_fetch_add(hs.claim + cls * FusedWs::kCounterStride, 1u,
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if constexpr (!CLAIM) {
        break;
      } else {
        __syncthreads();
        v = s_claim;  // rewritten only after the next pass's barrier above
        if (v >= hs.n1) break;
      }
    }
    WR_TL_MARK(hs, 3);
    return;
  }

  // ---- down block ----
  constexpr bool kFp8 = std::is_same<WT, fp8w>::value;
  __shared__ float part[kWavesPerBlock][RPD];
  __shared__ float sdn[kFp8 ? WR_MAX_TOPK * RPD : 1];  // fp8 row scales [kk][j]
  __shared__ int expired;  // this block's wait gave up
  const int r0 = ((int)blockIdx.x - hs.n1b) * RPD;
  const int nrows = min(RPD, g.h - r0);
  const int nch = (g.I + kWave * VEC - 1) / (kWave * VEC);
  const int C = g.k * nch;
  if (!routed) {  // the slot wait expired (timeout word set): NaN rows, no loads
    if (wave == 0 && lane < nrows) out[r0 + lane] = to_out<XT>(__builtin_nanf(""));
    return;
  }

  // STG: every selected expert's block-scale bytes of rows r0 .. r0 + nrows,
  // [kk][j][I / 32], into lds_raw before the wait (they do not depend on act);
  // wave w copies experts w, w + 4, ...
  if constexpr (STG) {
    const int ib = g.I / 32;
    const int wu0 = __builtin_amdgcn_readfirstlane(wave);
    for (int kk = wu0; kk < g.k; kk += kWavesPerBlock)
      stage_bytes_lds(mx_row(wbuf + (int64_t)topk_id(t, kk) * g.stride, g, 2, r0),
                      lds_raw + (size_t)kk * RPD * ib, nrows * ib, lane);
  }
  V pre[U2][RPD];
  down_tile_load<WT, VEC, RPD, U2, STG>(pre, wbuf, g, t, r0, nrows, wave, nch, lane);
  // The next PRE chunks of this wave (after the U2 in registers) go to LDS:
  // the tail after the hand-off then has one dependent load round fewer, and
  // those bytes stream during the end of the gate/up phase.  Slot (v, j)
  // holds row j of chunk wave + 4 (U2 + v), lane l's 16 bytes at 16 l.
  // Register-path kernels only: the x-in-LDS variant's copy takes the LDS.
  constexpr int PRE = (!XL && sizeof(V) == 16) ? WR_DN_LDS_ROWCHUNKS / RPD : 0;
  constexpr int kPreBytes = kWavesPerBlock * PRE * RPD * kWave * 16;
  __shared__ __align__(16) unsigned char dpre[kPreBytes > 0 ? kPreBytes : 16];
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  if constexpr (PRE > 0) {
#pragma unroll
    for (int v = 0; v < PRE; ++v) {
      const int q = wu + kWavesPerBlock * (U2 + v);
      if (q < C) {  // wave-uniform
        const int kk = q / nch;
        const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
        const WT* D = wbuf + (int64_t)topk_id(t, kk) * g.stride + g.off_down +
                      eoff<WT>((int64_t)r0 * g.I + c);
#pragma unroll
        for (int j = 0; j < RPD; ++j) {
          if (j < nrows && c < g.I)
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(D + eoff<WT>((int64_t)j * g.I)),
                (__attribute__((address_space(3))) void*)(dpre + (size_t)((wu * PRE + v) * RPD + j) *
                                                                     kWave * 16),
                16, 0, 0);
        }
      }
    }
  }
  // MXFP4 x-in-LDS variants: the down role does not use the x copy's bytes
  // of lds_raw, so (after the STG scale copy) they hold one more 8-row chunk
  // for each wave there is room for (spre = 1): chunk wave + 4 U2, codes
  // only, staged the same way.  Without STG the chunk's block-scale bytes go
  // to registers (sscale), loaded with it.
  constexpr bool kStage =
      STG || (XL && std::is_same<WT, fp4x2>::value && VEC == 32 && WR_F4_XL_DN_STAGE);
  int spre = 0;
  const unsigned char* sp = lds_raw;
  uint32_t sscale[RPD];
#pragma unroll
  for (int j = 0; j < RPD; ++j) sscale[j] = 127u;
  if constexpr (kStage) {
    constexpr int kChunk = RPD * kWave * 16;
    const int sbytes = STG ? (g.k * RPD * (g.I / 32) + 255) & ~255 : 0;
    const int npre = ((int)sizeof(lds_raw) - sbytes) / kChunk;
    const int q = wu + kWavesPerBlock * U2;
    if (wu < npre && q < C) {  // wave-uniform
      spre = 1;
      sp = lds_raw + sbytes + wu * kChunk;
      const int kk = q / nch;
      const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
      const WT* blk = wbuf + (int64_t)topk_id(t, kk) * g.stride;
      const WT* D = blk + g.off_down + eoff<WT>((int64_t)r0 * g.I + c);
#pragma unroll
      for (int j = 0; j < RPD; ++j) {
        if (j < nrows && c < g.I) {
          __builtin_amdgcn_global_load_lds(
              static_cast<const void*>(D + eoff<WT>((int64_t)j * g.I)),
              (__attribute__((address_space(3))) void*)(lds_raw + sbytes + wu * kChunk +
                                                        j * kWave * 16),
              16, 0, 0);
          if constexpr (!STG) sscale[j] = *mx_at<WT>(mx_row(blk, g, 2, r0 + j), c);
        }
      }
    }
  }
  WR_TL_MARK(hs, 2);
  if constexpr (kFp8) {
    // Published to the block by the __syncthreads after the wait below.
    const int i = threadIdx.x, kk = i / RPD, j = i % RPD;
    if (kk < g.k)
      sdn[i] = j < nrows ? wscales(wbuf + (int64_t)topk_id_lanes(t, kk) * g.stride,
                                   g.off_scale)[2 * g.I + r0 + j]
                         : 0.0f;
  }

  if (wave == 0) {
    // Lane c waits for the blocks counted by counter c: ids b < n1, b % 64 == c.
    const int c = lane;
    const unsigned target =
        (c < hs.n1 ? (unsigned)((hs.n1 - c + FusedWs::kCounters - 1) / FusedWs::kCounters)
                   : 0u) + hs.wait_extra;
    const uint64_t* ctr = arrival_word(hs, c);
    unsigned spins = 0;
    int gave_up = 0;
    uint64_t w;
#if WR_POLL_ONE
    {
      // Until the word of the last gate/up slot (dispatched last, or claimed
      // last) is complete, poll that word alone: one request per poll
      // instead of 64 from every waiting down block, which the memory side
      // otherwise serves beside the weight stream.  Any order of completion
      // stays correct: the loop below then checks all 64.
      const int cl = (hs.n1 - 1) % FusedWs::kCounters;
      const unsigned tl =
          (unsigned)((hs.n1 - cl + FusedWs::kCounters - 1) / FusedWs::kCounters) + hs.wait_extra;
      const uint64_t* last = arrival_word(hs, cl);
      for (;;) {
        unsigned a = 0;
        if (lane == 0)
          a = arrivals(__hip_atomic_load(last, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (__builtin_amdgcn_readfirstlane(a) >= tl) break;
        if (++spins > hs.spin_limit) break;  // the loop below then expires at once
        __builtin_amdgcn_s_sleep(8);
      }
    }
#endif
    for (;;) {
      w = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__ballot(arrivals(w) < target) == 0) break;
      if (++spins > hs.spin_limit) {
        gave_up = 1;
        if (lane == 0) set_expired(hs);
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
    if (lane == 0) expired = gave_up;
    // One rotation r for every arrival <=> (sum r)^2 = n sum r^2 over all n
    // of them (Cauchy-Schwarz); the sums are small integers, exact in fp32.
    const float n = wave_sum((float)arrivals(w));
    const float sr = wave_sum((float)(unsigned)((w >> 16) & 0xffffu));
    const float sq = wave_sum((float)(unsigned)(w >> 32));
    if ((double)sr * sr != (double)n * sq)
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    else
      invalidate_l1();
  }
  if constexpr (kStage) __builtin_amdgcn_s_waitcnt(0);  // this wave's staged bytes have landed
  __syncthreads();
  WR_TL_MARK(hs, 3);

  float acc[RPD];
#pragma unroll
  for (int j = 0; j < RPD; ++j) acc[j] = 0.0f;
  if constexpr (STG) down_tile_scales<WT, VEC, RPD, U2>(pre, lds_raw, g, nrows, wave, nch, lane);
  down_tile_fma<WT, V, VEC, RPD, U2>(acc, pre, act, g, act_row, wave, nch, lane, sdn);
  if constexpr (PRE > 0) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's global-to-LDS loads have landed
    asm volatile("" ::: "memory");
#pragma unroll
    for (int v = 0; v < PRE; ++v) {
      const int q = wu + kWavesPerBlock * (U2 + v);
      if (q < C) {
        const int kk = q / nch;
        const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
        V lw[1][RPD];
#pragma unroll
        for (int j = 0; j < RPD; ++j)
          lw[0][j] = (j < nrows && c < g.I)
                         ? *reinterpret_cast<const V*>(
                               dpre + (size_t)((wu * PRE + v) * RPD + j) * kWave * 16 + lane * 16)
                         : vzero<V>();
        down_tile_fma<WT, V, VEC, RPD, 1>(acc, lw, act, g, act_row, q, nch, lane, sdn);
      }
    }
  }
  if constexpr (kStage) {
    // The staged chunk landed before the barrier after the wait (the wave
    // waited for all of its loads there).
    if (spre) {
      const int q = wu + kWavesPerBlock * U2;
      const int kk = q / nch;
      const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
      V lw[1][RPD];
#pragma unroll
      for (int j = 0; j < RPD; ++j)
        lw[0][j] = (j < nrows && c < g.I)
                       ? V{*reinterpret_cast<const u32x4*>(sp + j * kWave * 16 + lane * 16),
                           sscale[j]}
                       : vzero<V>();
      if constexpr (STG) down_tile_scales<WT, VEC, RPD, 1>(lw, lds_raw, g, nrows, q, nch, lane);
      down_tile_fma<WT, V, VEC, RPD, 1>(acc, lw, act, g, act_row, q, nch, lane, sdn);
    }
  }
  for (int q0 = wave + kWavesPerBlock * (U2 + PRE + spre); q0 < C; q0 += kWavesPerBlock * U2) {
    V wv[U2][RPD];
    down_tile_load<WT, VEC, RPD, U2, STG>(wv, wbuf, g, t, r0, nrows, q0, nch, lane);
    if constexpr (STG) down_tile_scales<WT, VEC, RPD, U2>(wv, lds_raw, g, nrows, q0, nch, lane);
    down_tile_fma<WT, V, VEC, RPD, U2>(acc, wv, act, g, act_row, q0, nch, lane, sdn);
  }
#pragma unroll
  for (int j = 0; j < RPD; ++j) {
    const float s = wave_sum(acc[j]);
    if (lane == 0) part[wave][j] = s;
  }
  __syncthreads();
  if (wave == 0 && lane < nrows)
    out[r0 + lane] = to_out<XT>(expired ? __builtin_nanf("")
                                        : (part[0][lane] + part[1][lane]) +
                                              (part[2][lane] + part[3][lane]));
  WR_TL_MARK(hs, 4);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace {

// Bytes per storage unit of a weight type (an MXFP4 unit is a byte of two codes).
int64_t weight_es(int wdt) {
  return wdt == WR_F32 ? 4 : ((wdt == WR_FP8_E4M3 || wdt == WR_MXFP4) ? 1 : 2);
}

Geom make_geom(const Problem& p) {
  const int64_t es = weight_es(p.wdt);
  Geom g;
  g.E = p.E;
  g.h = p.h;
  g.I = p.I;
  g.k = p.k;
  g.renorm = p.renorm;
  g.B = p.B;
  g.stride = p.stride_b / es;
  g.off_up = p.off_up_b / es;
  g.off_down = p.off_down_b / es;
  g.off_scale = p.off_scale_b;
  return g;
}

// Compute units of the current device, cached per device.
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Persistent waves per token: the fewest waves that keep the largest share
// minimal (ceil(items / cap)) with at most `cap` waves in total.
int waves_for(int items, int B) {
  const int cap = cu_count() * WR_WAVES_PER_CU;
  const int per_tok = cap / B > 0 ? cap / B : 1;
  const int ipw = (items + per_tok - 1) / per_tok;
  return (items + ipw - 1) / ipw;
}

// 128-bit router loads need h % 4 == 0 and 16-byte aligned rows and x.
bool router_vec4(const Problem& p) {
  const int xes = p.adt == WR_F16 ? 2 : 4;
  return p.h % 4 == 0 && ((uintptr_t)p.gate_w % 16) == 0 && ((uintptr_t)p.x % (4 * xes)) == 0;
}

template <typename XT>
hipError_t logits_t(const Problem& p, float* logits, unsigned* zero, int nzero, int zstride,
                    hipStream_t s, XSplit xs = XSplit{nullptr, nullptr, nullptr, nullptr, 0, 0}) {
  const dim3 grid(p.E, p.B);
  const XT* x = static_cast<const XT*>(p.x);
  if (router_vec4(p))
    hipLaunchKernelGGL((k_router_logits<XT, 4>), grid, dim3(kBlock), 0, s, p.gate_w, x, logits,
                       p.E, p.h, zero, nzero, zstride, xs);
  else
    hipLaunchKernelGGL((k_router_logits<XT, 1>), grid, dim3(kBlock), 0, s, p.gate_w, x, logits,
                       p.E, p.h, zero, nzero, zstride, xs);
  return hipGetLastError();
}

// Rows per gate/up wave of the single-token kernel: 4 (two column chunks in
// flight) when those two chunks cover a whole weight row (at most 2 KB), else
// 2 (four chunks in flight).  Either way a wave reads about 16-32 KB per
// iteration, and a row of at most 4 chunks takes one load round per wave
// instead of two dependent ones (DeepSeek's 4 KB rows: 31.3 -> 28.0 us).
// fp8 rows always take 4: four chunks of 16 fp32 x values per lane would
// cost 64 VGPRs and a wave per SIMD.
int fused_rpw(const Problem& p) {
  const int64_t row_bytes = (int64_t)p.h * weight_es(p.wdt);
  if (p.wdt == WR_FP8_E4M3) return p.vec > 1 ? WR_F8_RPW : 2;
  if (p.wdt == WR_MXFP4) return p.vec == 32 ? 4 : 2;
  return (p.vec > 1 && row_bytes <= 2048) ? 4 : 2;
}

// act chunks of the single-token fused kernel, and its gate/up blocks (the
// chunk count rounded up to whole groups of 8 LB blocks).
int fused_chunks(int I, int k, int rpw) {
  const int items = (I + rpw - 1) / rpw;
  return k * ((items + kWavesPerBlock - 1) / kWavesPerBlock);
}
int fused_n1(int I, int k, int rpw) {
  const int group = 8 * (32 / (kWavesPerBlock * rpw));
  return (fused_chunks(I, k, rpw) + group - 1) / group * group;
}

// MXFP4 block scales staged in LDS (x-in-LDS variant): rows hold whole
// dwords of them (h and I multiples of 128), the down role's copy fits the
// buffer (k RPD I / 32 bytes) and the down rows are long enough for the copy
// to pay (I >= WR_F4_STG_MIN_I).
bool f4_stg(const Problem& p) {
  return p.h % 128 == 0 && p.I % 128 == 0 && p.I >= WR_F4_STG_MIN_I &&
         (size_t)p.k * WR_F4_RPD * (p.I / 32) <= (size_t)WR_F4_STG_RAW;
}

// Blocks of `kernel` resident per CU (occupancy query, cached per kernel).
int blocks_per_cu(const void* kernel) {
  static std::mutex mu;
  static std::unordered_map<const void*, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(kernel);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kBlock, 0) != hipSuccess || n < 0)
    n = 0;
  cache.emplace(kernel, n);
  return n;
}

// Gate/up blocks to launch for n1 chunk slots (a multiple of 32): all of
// them, unless they overflow one round of resident blocks by at most
// WR_GU_CLAIM_PCT percent of it.  Then one round (rounded down to a multiple
// of 32) is launched and its blocks claim the remaining slots as they finish:
// the overflow runs on the first blocks to end, instead of as a second round
// of blocks that starts after them (DeepSeek: 1,056 slots for 1,024 resident
// blocks, the last 32 ending about 7 us after the others).
int gu_launch_blocks(const Problem& p, int n1, const void* kernel) {
  if (p.gu_blocks > 0) return std::min(n1, p.gu_blocks);
  const int bpc = WR_GU_BLOCKS_PER_CU > 0 ? WR_GU_BLOCKS_PER_CU : blocks_per_cu(kernel);
  const int slots = bpc * cu_count() / 32 * 32;
  if (slots >= 32 && n1 > slots && (int64_t)(n1 - slots) * 100 <= (int64_t)slots * WR_GU_CLAIM_PCT)
    return slots;
  return n1;
}

#if WR_TIMELINE
#define WR_TL_GRID(n) g_tl_blocks.store((n), std::memory_order_relaxed)
#else
#define WR_TL_GRID(n) \
  do {                \
  } while (0)
#endif

#if WR_TIMELINE
// The timeline records of the last single-token launch on each device, and
// that launch's workgroup count.
static __device__ uint64_t tl_buf[(size_t)WR_TIMELINE_MAX_BLOCKS * WR_TIMELINE_EVENTS];
std::atomic<int64_t> g_tl_blocks{0};

uint64_t* tl_ptr() {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(tl_buf)) != hipSuccess) return nullptr;
  return static_cast<uint64_t*>(p);
}
#endif

// Gate/up slots per CU from which the register-path kernel takes the router
// inside (one launch per layer).
constexpr int kFoldSlotsPerCu = 2;

// fold == nullptr: the kernel reads the logits an earlier router launch left
// in the workspace.  Otherwise a request to compute the router rows inside
// the kernel (one launch per layer): *fold tells whether this shape's variant
// did, and if not nothing was launched.
template <typename WT, typename XT, int VEC, int RPW, int U1>
hipError_t fused_rpw_t(const Problem& p, const FusedWs& w, bool* fold, hipStream_t s) {
  const Geom g = make_geom(p);
  Handoff hs;
#if WR_TIMELINE
  hs.tl = tl_ptr();
  if (hs.tl == nullptr) return hipErrorInvalidSymbol;
#endif
  hs.ctrl = w.ctrl;
  hs.slot = reinterpret_cast<uint64_t*>(w.ctrl + FusedWs::kSlotWord);
  hs.gate_w = fold != nullptr ? p.gate_w : nullptr;
  hs.rvec = router_vec4(p) ? 1 : 0;
  hs.cnt = w.ctrl;
  hs.timeout = w.ctrl + FusedWs::kTimeoutWord;
  hs.host_flag = p.expired_host;
  hs.claim = w.ctrl + FusedWs::kClaimWord;
  hs.n1 = fused_n1(p.I, p.k, RPW);
  if (hs.n1 > FusedWs::kCounters * kMaxArrivals) return hipErrorInvalidValue;
  hs.n1b = hs.n1;
  hs.chunks = fused_chunks(p.I, p.k, RPW);
  hs.spin_limit = p.spin_limit;
  hs.wait_extra = p.wait_extra;
  // fp8 down blocks take twice the rows and half the chunks in flight: the
  // same weight bytes per tile as fp16, and half the act reads per weight byte.
  // MXFP4 (32 act values per lane and chunk): 8 rows, one chunk in flight.
  constexpr bool kFp8 = std::is_same<WT, fp8w>::value;
  constexpr bool kFp4 = std::is_same<WT, fp4x2>::value;
  constexpr int RPD = kFp4 ? WR_F4_RPD : (kFp8 ? WR_F8_RPD : WR_FU_RPD);
  constexpr int U2 = kFp4 ? WR_F4_U2 : (kFp8 ? WR_F8_U2 : WR_FU_U);
  const int n2 = (p.h + RPD - 1) / RPD;
  // Gate/up blocks read x from an LDS copy for small enough h (and, except
  // for MXFP4, few enough gate/up blocks).
  constexpr int kXlMax = xl_max_h<WT>();
  constexpr bool kXl = kXlMax > 0 && VEC >= 8;
  if constexpr (kXl) {
    constexpr int kBpc = kFp8 ? WR_XL_FP8_BPC : WR_XL_F16_BPC;  // MXFP4: no bound
    if (p.h <= kXlMax && (kFp4 || hs.n1 <= kBpc * cu_count())) {
      if (fold != nullptr) {  // the x-in-LDS variants keep the router launch
        *fold = false;
        return hipSuccess;
      }
      // MXFP4: block-scale bytes staged in LDS under f4_stg's conditions.
      // Measured: Mixtral 57.5 -> 55.7 us, DBRX 105.0 -> 102.0 us; DeepSeek
      // (I = 1408) 18.7 -> 19.0 us.
      if constexpr (kFp4 && RPW == 4) {
        static_assert(fused_raw_bytes<WT, XT, VEC, RPW, true, true>() == WR_F4_STG_RAW &&
                          RPD == WR_F4_RPD,
                      "f4_stg sizes the down role's scale copy with these");
        if (f4_stg(p)) {
          hs.nb = hs.n1 + n2;
          WR_TL_GRID(hs.nb);
          hipLaunchKernelGGL((k_fused_ffn<WT, XT, VEC, RPW, U1, RPD, U2, true, true>),
                             dim3(hs.n1 + n2), dim3(kBlock), 0, s,
                             static_cast<const WT*>(p.wbuf), static_cast<const XT*>(p.x),
                             w.logits, w.act, static_cast<XT*>(p.out), p.topk_ids, p.topk_w, g,
                             hs);
          return hipGetLastError();
        }
      }
      // 16-bit weights: a layer whose gate/up and down blocks can all be
      // resident at once with half the column chunks in flight (fewer VGPRs,
      // more blocks per CU) takes that variant.  Measured (layer us): Mixtral
      // tp8 shard 27.03 -> 25.30; layers that would still wait for resident
      // slots lose with it (DeepSeek 25.51 -> 28.04, tp4 shard 42.96 ->
      // 45.33, Mixtral 114.50 -> 120.62).
      if constexpr (sizeof(WT) == 2 && U1 >= 2 && U2 >= 2) {
        auto ksm = k_fused_ffn<WT, XT, VEC, RPW, U1 / 2, RPD, U2 / 2, true, false>;
        if (hs.n1 + n2 <= blocks_per_cu(reinterpret_cast<const void*>(ksm)) * cu_count()) {
          hs.nb = hs.n1 + n2;
          WR_TL_GRID(hs.nb);
          hipLaunchKernelGGL(ksm, dim3(hs.n1 + n2), dim3(kBlock), 0, s,
                             static_cast<const WT*>(p.wbuf), static_cast<const XT*>(p.x),
                             w.logits, w.act, static_cast<XT*>(p.out), p.topk_ids, p.topk_w, g,
                             hs);
          return hipGetLastError();
        }
      }
      hs.nb = hs.n1 + n2;
      WR_TL_GRID(hs.nb);
      hipLaunchKernelGGL((k_fused_ffn<WT, XT, VEC, RPW, U1, RPD, U2, true, false>),
                         dim3(hs.n1 + n2), dim3(kBlock), 0, s,
                         static_cast<const WT*>(p.wbuf), static_cast<const XT*>(p.x), w.logits,
                         w.act, static_cast<XT*>(p.out), p.topk_ids, p.topk_w, g, hs);
      return hipGetLastError();
    }
  }
  // Register path: gate/up chunk slots that overflow one round of resident
  // blocks by a little are claimed by the launched blocks (CLAIM variant;
  // 16-bit and fp32 weights, whose small layers such as DeepSeek's take this
  // path; fp8 and MXFP4 layers of that size stage x in LDS).
  if constexpr (VEC > 1 && (sizeof(WT) == 2 || std::is_same<WT, float>::value)) {
    auto kc = k_fused_ffn<WT, XT, VEC, RPW, U1, RPD, U2, false, false, true>;
    const int n1b = gu_launch_blocks(p, hs.n1, reinterpret_cast<const void*>(kc));
    if (n1b < hs.n1) {
      if (fold != nullptr) {  // so does the claiming variant
        *fold = false;
        return hipSuccess;
      }
      hs.n1b = n1b;
      hs.nb = hs.n1b + n2;
      WR_TL_GRID(hs.nb);
      hipLaunchKernelGGL(kc, dim3(hs.n1b + n2), dim3(kBlock), 0, s,
                         static_cast<const WT*>(p.wbuf), static_cast<const XT*>(p.x), w.logits,
                         w.act, static_cast<XT*>(p.out), p.topk_ids, p.topk_w, g, hs);
      return hipGetLastError();
    }
  }
  if constexpr (kFp4 && U1 == 2) {
    // Whole MXFP4 rows in flight are chosen (f4_whole_rows) only for shapes
    // whose x the LDS copy holds, which returned above.
    return hipErrorInvalidValue;
  } else {
    hs.nb = hs.n1 + n2;
    WR_TL_GRID(hs.nb);
    if (fold != nullptr) {
      // The router inside the kernel (route_and_select) pays for layers of
      // at least kFoldSlotsPerCu gate/up slots per CU, whose gate/up phase
      // spans rounds of resident blocks; smaller layers keep the router
      // launch.  Measured (layer us): Mixtral 114.50 -> 113.54, DBRX 240.5 ->
      // 239.4, Mixtral tp4 shard 42.96 -> 42.53 folded; tp8 shard 27.03 ->
      // 27.74 and DeepSeek (claiming variant) 25.51 -> 26.37 would lose.
      *fold = hs.n1 >= kFoldSlotsPerCu * cu_count();
      if (!*fold) return hipSuccess;
      hipLaunchKernelGGL((k_fused_ffn<WT, XT, VEC, RPW, U1, RPD, U2, false, false, false, true>),
                         dim3(hs.n1 + n2), dim3(kBlock), 0, s, static_cast<const WT*>(p.wbuf),
                         static_cast<const XT*>(p.x), w.logits, w.act, static_cast<XT*>(p.out),
                         p.topk_ids, p.topk_w, g, hs);
      return hipGetLastError();
    }
    hipLaunchKernelGGL((k_fused_ffn<WT, XT, VEC, RPW, U1, RPD, U2, false, false>),
                       dim3(hs.n1 + n2), dim3(kBlock), 0, s, static_cast<const WT*>(p.wbuf),
                       static_cast<const XT*>(p.x), w.logits, w.act, static_cast<XT*>(p.out),
                       p.topk_ids, p.topk_w, g, hs);
    return hipGetLastError();
  }
}

// Column chunks in flight per gate/up row: fp8 WR_F8_U1, MXFP4 one (32 x
// values per lane and chunk), else WR_GU_U (halved for 4 rows per wave).
template <typename WT, int RPW>
constexpr int fused_u1() {
  if constexpr (std::is_same<WT, fp4x2>::value) return WR_F4_U1;
  if constexpr (std::is_same<WT, fp8w>::value) return WR_F8_U1;
  return RPW == 4 ? WR_GU_U / 2 : WR_GU_U;
}

// MXFP4 rows of two column chunks (2048 < h <= 4096) take both chunks of a
// row in one load round (U1 = 2) when every gate/up block of the layer is
// resident at once at that variant's occupancy (168-208 VGPRs: 2 or 3 blocks
// per CU): each block then ends after one round trip instead of two.  With a
// second round of blocks the lower occupancy costs more than it saves.
// Measured (fp32 x): Mixtral tp4 / tp8 shards 22.4 / 17.6 -> 21.1 / 17.4 us;
// full Mixtral 54.6 -> 57.4, tp2 shard 33.5 -> 33.7, DBRX 102.6 -> 122.0,
// DeepSeek 19.2 -> 23.7 us with U1 = 2 throughout.
template <typename WT, typename XT, int VEC>
bool f4_whole_rows(const Problem& p) {
  if constexpr (std::is_same<WT, fp4x2>::value && VEC == 32) {
    if (p.h <= kWave * VEC || p.h > 2 * kWave * VEC || p.h > WR_XL_FP4_MAXH) return false;
    constexpr int RPD = WR_F4_RPD, U2 = WR_F4_U2;
    const void* k = f4_stg(p)
                        ? reinterpret_cast<const void*>(
                              k_fused_ffn<WT, XT, VEC, 4, 2, RPD, U2, true, true>)
                        : reinterpret_cast<const void*>(
                              k_fused_ffn<WT, XT, VEC, 4, 2, RPD, U2, true, false>);
    return fused_n1(p.I, p.k, 4) <= blocks_per_cu(k) * cu_count();
  } else {
    (void)p;
    return false;
  }
}

template <typename WT, typename XT, int VEC>
hipError_t fused_t(const Problem& p, const FusedWs& w, bool* fold, hipStream_t s) {
  if (fused_rpw(p) == 4) {
    if constexpr (std::is_same<WT, fp4x2>::value && VEC == 32) {
      if (f4_whole_rows<WT, XT, VEC>(p)) return fused_rpw_t<WT, XT, VEC, 4, 2>(p, w, fold, s);
    }
    return fused_rpw_t<WT, XT, VEC, 4, fused_u1<WT, 4>()>(p, w, fold, s);
  }
  return fused_rpw_t<WT, XT, VEC, 2, fused_u1<WT, 2>()>(p, w, fold, s);
}

template <typename WT, typename XT, int VEC>
hipError_t ffn_t(const Problem& p, const FusedWs& w, bool* fold, hipStream_t s) {
  constexpr int RPW = WR_GU_RPW, RPD = WR_DN_RPD;
  // fp8: half the chunks in flight (16 fp32 x values per chunk and lane);
  // MXFP4: one chunk (32 values), and one chunk per down tile.
  constexpr bool kFp4 = std::is_same<WT, fp4x2>::value;
  constexpr int U1 = kFp4 ? 1 : (std::is_same<WT, fp8w>::value ? WR_GU_U / 2 : WR_GU_U);
  constexpr int UD = kFp4 ? 1 : WR_DN_U;
  if (p.B == 1) return fused_t<WT, XT, VEC>(p, w, fold, s);
  if (fold != nullptr) {  // several tokens: the router runs in its own launch
    *fold = false;
    return hipSuccess;
  }
  const Geom g = make_geom(p);
  const WT* wb = static_cast<const WT*>(p.wbuf);
  const int nw1 = waves_for(p.k * ((p.I + RPW - 1) / RPW), p.B);
  const dim3 g1((nw1 + kWavesPerBlock - 1) / kWavesPerBlock, p.B);
  hipLaunchKernelGGL((k_gateup<WT, XT, VEC, RPW, U1>), g1, dim3(kBlock), 0, s, wb,
                     static_cast<const XT*>(p.x), w.logits, w.act, p.topk_ids, p.topk_w, g, nw1);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int nw2 = waves_for((p.h + RPD - 1) / RPD, p.B);
  const dim3 g2((nw2 + kWavesPerBlock - 1) / kWavesPerBlock, p.B);
  hipLaunchKernelGGL((k_down<WT, XT, VEC, RPD, UD>), g2, dim3(kBlock), 0, s, wb, w.logits,
                     w.act, static_cast<XT*>(p.out), g, nw2);
  return hipGetLastError();
}

template <typename WT, typename XT>
hipError_t ffn_w(const Problem& p, const FusedWs& w, bool* fold, hipStream_t s) {
  constexpr int V = wvec_width<WT>(), V1 = wvec_scalar<WT>();
  return p.vec == V ? ffn_t<WT, XT, V>(p, w, fold, s) : ffn_t<WT, XT, V1>(p, w, fold, s);
}

template <typename XT>
hipError_t ffn_x(const Problem& p, const FusedWs& w, bool* fold, hipStream_t s) {
  switch (p.wdt) {
    case WR_F16: return ffn_w<f16, XT>(p, w, fold, s);
    case WR_BF16: return ffn_w<bf16w, XT>(p, w, fold, s);
    case WR_FP8_E4M3: return ffn_w<fp8w, XT>(p, w, fold, s);
    case WR_MXFP4: return ffn_w<fp4x2, XT>(p, w, fold, s);
    default: return ffn_w<float, XT>(p, w, fold, s);
  }
}

// Router logits into the workspace; for one token also the reset of the
// single-token kernel's control words, which start each call at zero.
hipError_t run_route(const Problem& p, hipStream_t s) {
  const FusedWs w = FusedWs::carve(p.ws, p.E, p.I, p.k, p.B);
  static_assert(FusedWs::kCtrlWords <= kBlock, "one router thread zeroes each control word");
  unsigned* zero = p.B == 1 ? w.ctrl : nullptr;
  const int nz = FusedWs::kCtrlWords, zs = FusedWs::kCounterStride;
  return p.adt == WR_F16 ? logits_t<f16>(p, w.logits, zero, nz, zs, s)
                         : logits_t<float>(p, w.logits, zero, nz, zs, s);
}

// The expert FFN from the logits run_route left in the workspace (fold =
// nullptr).  With fold != nullptr, one token's FFN kernel with the router
// inside when its variant takes it (*fold = true), else nothing (*fold =
// false).
hipError_t run_ffn_only(const Problem& p, bool* fold, hipStream_t s) {
  const FusedWs w = FusedWs::carve(p.ws, p.E, p.I, p.k, p.B);
  return p.adt == WR_F16 ? ffn_x<f16>(p, w, fold, s) : ffn_x<float>(p, w, fold, s);
}

// One token whose single-token kernel takes the router inside: one launch.
// Otherwise the router launch, then the FFN kernel(s).
hipError_t run_ffn(const Problem& p, hipStream_t s) {
  if (p.B == 1) {
    bool folded = false;
    const hipError_t err = run_ffn_only(p, &folded, s);
    if (err != hipSuccess || folded) return err;
  }
  const hipError_t err = run_route(p, s);
  if (err != hipSuccess) return err;
  return run_ffn_only(p, nullptr, s);
}

template <typename XT>
hipError_t gate_t(const Problem& p, hipStream_t s) {
  const XT* x = static_cast<const XT*>(p.x);
  if (router_vec4(p))
    hipLaunchKernelGGL((k_gate_topk<XT, 4>), dim3(p.B), dim3(1024), 0, s, p.gate_w, x, p.E, p.h,
                       p.k, p.renorm, p.topk_ids, p.topk_w);
  else
    hipLaunchKernelGGL((k_gate_topk<XT, 1>), dim3(p.B), dim3(1024), 0, s, p.gate_w, x, p.E, p.h,
                       p.k, p.renorm, p.topk_ids, p.topk_w);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_logits(const Problem& p, float* logits, hipStream_t s) {
  return p.adt == WR_F16 ? logits_t<f16>(p, logits, nullptr, 0, 0, s)
                         : logits_t<float>(p, logits, nullptr, 0, 0, s);
}

hipError_t launch_gate_topk(const Problem& p, hipStream_t s) {
  return p.adt == WR_F16 ? gate_t<f16>(p, s) : gate_t<float>(p, s);
}

hipError_t launch_fused(const Problem& p, hipStream_t s) { return run_ffn(p, s); }

hipError_t launch_fused_route(const Problem& p, hipStream_t s) { return run_route(p, s); }

hipError_t launch_fused_ffn(const Problem& p, hipStream_t s) { return run_ffn_only(p, nullptr, s); }

hipError_t launch_logits_split(const Problem& p, float* logits, f16* x_hi, f16* x_lo,
                               int32_t* x_exp, unsigned* amax, int split_bf16, hipStream_t s) {
  const XSplit xs{x_hi, x_lo, x_exp, amax, p.k, split_bf16};
  return p.adt == WR_F16 ? logits_t<f16>(p, logits, nullptr, 0, 0, s, xs)
                         : logits_t<float>(p, logits, nullptr, 0, 0, s, xs);
}

hipError_t launch_batched(const Problem& p, hipStream_t s) {
  if (grouped_ok(p)) return launch_grouped(p, s);
  return run_ffn(p, s);
}

}  // namespace wr

extern "C" WR_TL_API int64_t wr_timeline_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return -2;
  return khz;
}

extern "C" WR_TL_API int64_t wr_timeline_read(uint64_t* rec, int64_t max_blocks, void* stream) {
#if WR_TIMELINE
  if (rec == nullptr || max_blocks < 0) return -2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = std::min<int64_t>(
      std::min<int64_t>(wr::g_tl_blocks.load(std::memory_order_relaxed), WR_TIMELINE_MAX_BLOCKS),
      max_blocks);
  uint64_t* src = wr::tl_ptr();
  if (src == nullptr || hipStreamSynchronize(s) != hipSuccess) return -2;
  if (n > 0 && hipMemcpy(rec, src, (size_t)n * WR_TIMELINE_EVENTS * sizeof(uint64_t),
                         hipMemcpyDeviceToHost) != hipSuccess)
    return -2;
  return n;
#else
  (void)rec;
  (void)max_blocks;
  (void)stream;
  return -1;
#endif
}
