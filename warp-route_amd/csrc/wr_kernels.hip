// Fused decode-time MoE kernels for gfx950 (wave64).
//
// The layer is three streaming passes over HBM-resident data:
//   1. k_router_logits: one wave per (expert, token) computes the router dot
//      product (src/fused_moe.cu:100-112) into the workspace.
//   2. k_gateup: every wave re-derives the top-K selection from the logits
//      (wave_select_topk; a few dozen instructions), then streams RPW rows of
//      the selected expert's gate and up matrices with 128-bit non-temporal
//      loads, reduces each row across the wave and writes
//      act = w_kk * silu(gate . x) * (up . x) in fp32
//      (src/fused_moe.cu:192-201, silu at :30-32).
//   3. k_down: a workgroup owns RPD output rows; its four waves split the
//      concatenated k*I columns of the selected down matrices, accumulate in
//      fp32 registers, combine through LDS and write each output row once
//      (src/fused_moe.cu:203-224, without the reference's repeated global
//      read-modify-write of the output).
// Bytes that matter are the selected expert weights; x, logits and act are
// small and served from L2.  The batched entry point runs the same kernels
// with one grid row (blockIdx.y) per token.
#include <hip/hip_runtime.h>

#include "wr_device.h"
#include "wr_internal.h"

namespace wr {

constexpr int kBlock = 256;  // 4 waves
constexpr int kWavesPerBlock = kBlock / kWave;

// One wave's fp32 dot product of a router row with x.  Shared by every
// kernel that produces logits so that all of them produce identical bits.
template <typename XT, int VEC>
__device__ __forceinline__ float wave_router_dot(const float* __restrict__ row,
                                                 const XT* __restrict__ x, int h) {
  const int lane = threadIdx.x & (kWave - 1);
  float acc0 = 0.0f, acc1 = 0.0f;
  int c = lane * VEC;
  for (; c + kWave * VEC < h; c += 2 * kWave * VEC) {
    float w0[VEC], x0[VEC], w1[VEC], x1[VEC];
    load_x<float, VEC>(row + c, w0);
    load_x<XT, VEC>(x + c, x0);
    load_x<float, VEC>(row + c + kWave * VEC, w1);
    load_x<XT, VEC>(x + c + kWave * VEC, x1);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      acc0 = fmaf(w0[i], x0[i], acc0);
      acc1 = fmaf(w1[i], x1[i], acc1);
    }
  }
  if (c < h) {
    float w0[VEC], x0[VEC];
    load_x<float, VEC>(row + c, w0);
    load_x<XT, VEC>(x + c, x0);
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc0 = fmaf(w0[i], x0[i], acc0);
  }
  return wave_sum(acc0 + acc1);
}

// grid (ceil(E / 4), B), block 256: wave w of block bx computes expert
// 4*bx + w for token blockIdx.y.
template <typename XT, int VEC>
__global__ __launch_bounds__(kBlock) void k_router_logits(const float* __restrict__ gate_w,
                                                          const XT* __restrict__ x,
                                                          float* __restrict__ logits, int E,
                                                          int h) {
  const int wave = threadIdx.x / kWave;
  const int e = blockIdx.x * kWavesPerBlock + wave;
  const int b = blockIdx.y;
  if (e >= E) return;  // wave-uniform
  const float v = wave_router_dot<XT, VEC>(gate_w + (int64_t)e * h, x + (int64_t)b * h, h);
  if ((threadIdx.x & (kWave - 1)) == 0) logits[(int64_t)b * E + e] = v;
}

// Standalone gate: grid B, block 1024.  Logits go through LDS; wave 0 selects
// and writes ids/weights.  Same per-expert dot as k_router_logits.
template <typename XT, int VEC>
__global__ __launch_bounds__(1024) void k_gate_topk(const float* __restrict__ gate_w,
                                                    const XT* __restrict__ x, int E, int h,
                                                    int k, int renorm,
                                                    int32_t* __restrict__ ids_out,
                                                    float* __restrict__ w_out) {
  __shared__ float lg[WR_MAX_EXPERTS];
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int b = blockIdx.x;
  for (int e = wave; e < E; e += nw) {
    const float v = wave_router_dot<XT, VEC>(gate_w + (int64_t)e * h, x + (int64_t)b * h, h);
    if ((threadIdx.x & (kWave - 1)) == 0) lg[e] = v;
  }
  __syncthreads();
  if (wave == 0) {
    TopK t;
    wave_select_topk(lg, E, k, renorm, t);
    const int lane = threadIdx.x;
#pragma unroll
    for (int kk = 0; kk < WR_MAX_TOPK; ++kk) {
      if (kk < k && lane == kk) {
        ids_out[(int64_t)b * k + kk] = t.id[kk];
        w_out[(int64_t)b * k + kk] = t.w[kk];
      }
    }
  }
}

// grid (ceil(k * ceil(I / RPW) / 4), B), block 256.  Global wave gw handles
// rows [r0, r0 + RPW) of selected expert kk.
template <typename WT, typename XT, int VEC, int RPW, int U>
__global__ __launch_bounds__(kBlock) void k_gateup(const WT* __restrict__ wbuf,
                                                   const XT* __restrict__ x,
                                                   const float* __restrict__ logits,
                                                   float* __restrict__ act,
                                                   int32_t* __restrict__ ids_out,
                                                   float* __restrict__ w_out, Geom g) {
  typedef typename WVec<WT, VEC>::type V;
  const int lane = threadIdx.x & (kWave - 1);
  const int b = blockIdx.y;
  const int gw = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const int items = (g.I + RPW - 1) / RPW;
  if (gw >= g.k * items) return;  // wave-uniform

  TopK t;
  wave_select_topk(logits + (int64_t)b * g.E, g.E, g.k, g.renorm, t);
  if (gw == 0) {
#pragma unroll
    for (int kk = 0; kk < WR_MAX_TOPK; ++kk) {
      if (kk < g.k && lane == kk) {
        if (ids_out != nullptr) ids_out[(int64_t)b * g.k + kk] = t.id[kk];
        if (w_out != nullptr) w_out[(int64_t)b * g.k + kk] = t.w[kk];
      }
    }
  }

  const int kk = gw / items;
  const int r0 = (gw - kk * items) * RPW;
  const int e = topk_id(t, kk);
  const float wk = topk_w(t, kk);
  const WT* G = wbuf + (int64_t)e * g.stride + (int64_t)r0 * g.h;
  const WT* Up = G + g.off_up;
  const XT* xb = x + (int64_t)b * g.h;
  const int nrows = min(RPW, g.I - r0);

  float ag[RPW], au[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) ag[j] = au[j] = 0.0f;

  for (int c0 = lane * VEC; c0 < g.h; c0 += U * kWave * VEC) {
    V wg[U][RPW], wu[U][RPW];
    float xv[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * kWave * VEC;
      const bool ok = c < g.h;
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const bool okj = ok && j < nrows;
        wg[u][j] = okj ? load_w<WT, VEC>(G + (int64_t)j * g.h + c) : vzero<V>();
        wu[u][j] = okj ? load_w<WT, VEC>(Up + (int64_t)j * g.h + c) : vzero<V>();
      }
      if (ok) {
        load_x<XT, VEC>(xb + c, xv[u]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) xv[u][i] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          ag[j] = fmaf(velem(wg[u][j], i), xv[u][i], ag[j]);
          au[j] = fmaf(velem(wu[u][j], i), xv[u][i], au[j]);
        }
      }
    }
  }

  float* a = act + ((int64_t)b * g.k + kk) * g.I + r0;
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const float gs = wave_sum(ag[j]);
    const float us = wave_sum(au[j]);
    if (lane == 0 && j < nrows) a[j] = wk * (silu(gs) * us);
  }
}

// grid (ceil(h / RPD), B), block 256.  Block owns output rows [r0, r0+RPD)
// of token blockIdx.y; wave w takes column chunks w, w+4, ... of the
// concatenated k * I columns (chunk = 64 * VEC columns inside one expert).
template <typename WT, typename OT, int VEC, int RPD, int U>
__global__ __launch_bounds__(kBlock) void k_down(const WT* __restrict__ wbuf,
                                                 const float* __restrict__ logits,
                                                 const float* __restrict__ act,
                                                 OT* __restrict__ out, Geom g) {
  typedef typename WVec<WT, VEC>::type V;
  __shared__ float part[kWavesPerBlock][RPD];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int b = blockIdx.y;
  const int r0 = blockIdx.x * RPD;
  const int nrows = min(RPD, g.h - r0);

  TopK t;
  wave_select_topk(logits + (int64_t)b * g.E, g.E, g.k, g.renorm, t);

  const int nch = (g.I + kWave * VEC - 1) / (kWave * VEC);
  const int C = g.k * nch;
  const float* ab = act + (int64_t)b * g.k * g.I;

  float acc[RPD];
#pragma unroll
  for (int j = 0; j < RPD; ++j) acc[j] = 0.0f;

  for (int q0 = wave; q0 < C; q0 += U * kWavesPerBlock) {
    V wv[U][RPD];
    float av[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = q0 + u * kWavesPerBlock;
      const int kk = q / nch;
      const int c = (q - kk * nch) * kWave * VEC + lane * VEC;
      const bool ok = q < C && c < g.I;
      const int e = topk_id(t, kk < g.k ? kk : 0);
      const WT* D = wbuf + (int64_t)e * g.stride + g.off_down + (int64_t)r0 * g.I + c;
#pragma unroll
      for (int j = 0; j < RPD; ++j) {
        const bool okj = ok && j < nrows;
        wv[u][j] = okj ? load_w<WT, VEC>(D + (int64_t)j * g.I) : vzero<V>();
      }
      if (ok) {
        load_x<float, VEC>(ab + (int64_t)kk * g.I + c, av[u]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) av[u][i] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < RPD; ++j) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[j] = fmaf(velem(wv[u][j], i), av[u][i], acc[j]);
      }
    }
  }

#pragma unroll
  for (int j = 0; j < RPD; ++j) {
    const float s = wave_sum(acc[j]);
    if (lane == 0) part[wave][j] = s;
  }
  __syncthreads();
  if (wave == 0 && lane < nrows) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) s += part[w][lane];
    out[(int64_t)b * g.h + r0 + lane] = to_out<OT>(s);
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace {

constexpr int kRPW = 2, kUG = 4;  // gate/up: rows per wave, chunk unroll
constexpr int kRPD = 4, kUD = 4;  // down: rows per block, chunk unroll

Geom make_geom(const Problem& p) {
  const int64_t es = p.wdt == WR_F16 ? 2 : 4;
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
  return g;
}

// 128-bit router loads need h % 4 == 0 and 16-byte aligned rows and x.
bool router_vec4(const Problem& p) {
  const int xes = p.adt == WR_F16 ? 2 : 4;
  return p.h % 4 == 0 && ((uintptr_t)p.gate_w % 16) == 0 && ((uintptr_t)p.x % (4 * xes)) == 0;
}

template <typename XT>
hipError_t logits_t(const Problem& p, float* logits, hipStream_t s) {
  dim3 grid((p.E + kWavesPerBlock - 1) / kWavesPerBlock, p.B);
  const XT* x = static_cast<const XT*>(p.x);
  if (router_vec4(p))
    hipLaunchKernelGGL((k_router_logits<XT, 4>), grid, dim3(kBlock), 0, s, p.gate_w, x, logits,
                       p.E, p.h);
  else
    hipLaunchKernelGGL((k_router_logits<XT, 1>), grid, dim3(kBlock), 0, s, p.gate_w, x, logits,
                       p.E, p.h);
  return hipGetLastError();
}

template <typename WT, typename XT, int VEC>
hipError_t ffn_t(const Problem& p, const FusedWs& w, hipStream_t s) {
  const Geom g = make_geom(p);
  const WT* wb = static_cast<const WT*>(p.wbuf);
  const int items = (p.I + kRPW - 1) / kRPW;
  const int waves = p.k * items;
  dim3 g1((waves + kWavesPerBlock - 1) / kWavesPerBlock, p.B);
  hipLaunchKernelGGL((k_gateup<WT, XT, VEC, kRPW, kUG>), g1, dim3(kBlock), 0, s, wb,
                     static_cast<const XT*>(p.x), w.logits, w.act, p.topk_ids, p.topk_w, g);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  dim3 g2((p.h + kRPD - 1) / kRPD, p.B);
  hipLaunchKernelGGL((k_down<WT, XT, VEC, kRPD, kUD>), g2, dim3(kBlock), 0, s, wb, w.logits,
                     w.act, static_cast<XT*>(p.out), g);
  return hipGetLastError();
}

template <typename XT>
hipError_t ffn_x(const Problem& p, const FusedWs& w, hipStream_t s) {
  if (p.wdt == WR_F16)
    return p.vec == 8 ? ffn_t<f16, XT, 8>(p, w, s) : ffn_t<f16, XT, 1>(p, w, s);
  return p.vec == 4 ? ffn_t<float, XT, 4>(p, w, s) : ffn_t<float, XT, 1>(p, w, s);
}

hipError_t run_ffn(const Problem& p, hipStream_t s) {
  const FusedWs w = FusedWs::carve(p.ws, p.E, p.I, p.k, p.B);
  hipError_t err = launch_logits(p, w.logits, s);
  if (err != hipSuccess) return err;
  return p.adt == WR_F16 ? ffn_x<f16>(p, w, s) : ffn_x<float>(p, w, s);
}

}  // namespace

hipError_t launch_logits(const Problem& p, float* logits, hipStream_t s) {
  return p.adt == WR_F16 ? logits_t<f16>(p, logits, s) : logits_t<float>(p, logits, s);
}

hipError_t launch_gate_topk(const Problem& p, hipStream_t s) {
  const int threads = 1024;
  if (p.adt == WR_F16) {
    const f16* x = static_cast<const f16*>(p.x);
    if (router_vec4(p))
      hipLaunchKernelGGL((k_gate_topk<f16, 4>), dim3(p.B), dim3(threads), 0, s, p.gate_w, x, p.E,
                         p.h, p.k, p.renorm, p.topk_ids, p.topk_w);
    else
      hipLaunchKernelGGL((k_gate_topk<f16, 1>), dim3(p.B), dim3(threads), 0, s, p.gate_w, x, p.E,
                         p.h, p.k, p.renorm, p.topk_ids, p.topk_w);
  } else {
    const float* x = static_cast<const float*>(p.x);
    if (router_vec4(p))
      hipLaunchKernelGGL((k_gate_topk<float, 4>), dim3(p.B), dim3(threads), 0, s, p.gate_w, x,
                         p.E, p.h, p.k, p.renorm, p.topk_ids, p.topk_w);
    else
      hipLaunchKernelGGL((k_gate_topk<float, 1>), dim3(p.B), dim3(threads), 0, s, p.gate_w, x,
                         p.E, p.h, p.k, p.renorm, p.topk_ids, p.topk_w);
  }
  return hipGetLastError();
}

hipError_t launch_fused(const Problem& p, hipStream_t s) { return run_ffn(p, s); }

hipError_t launch_batched(const Problem& p, hipStream_t s) { return run_ffn(p, s); }

}  // namespace wr
