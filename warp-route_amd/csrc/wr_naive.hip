// Naive multi-kernel MoE baseline (the structure of src/naive_moe.cu:181-241):
//   router logits -> device-to-host copy + stream sync -> host softmax/top-K
//   -> per selected expert: gate matvec, up matvec, swiglu, down matvec,
//      weighted accumulate.
// It keeps the reference's launch count (3 + 5k kernels and one host round
// trip) so that it measures what fusion saves, but each matvec uses a
// multi-workgroup grid (one wave per output row) instead of the reference's
// single block, so that the comparison is fusion against fusion-free
// streaming rather than against a one-CU launch.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <vector>

#include "wr_device.h"
#include "wr_internal.h"

namespace wr {

namespace {

constexpr int kBlock = 256;
constexpr int kWpb = kBlock / kWave;

// y[r] = W[r, :] . v (times scale[r] when scale != nullptr: fp8 row scales)
// for r < rows; one wave per row (src/naive_moe.cu:79-111 computes the same
// product on one 256-thread block).  MXFP4: mx holds the matrix's block
// scales, [rows][cols / 32] bytes.
template <typename WT, typename VT, int VEC>
__global__ __launch_bounds__(kBlock) void k_matvec(const WT* __restrict__ W,
                                                   const VT* __restrict__ v,
                                                   float* __restrict__ y, int rows, int cols,
                                                   const float* __restrict__ scale,
                                                   const uint8_t* __restrict__ mx) {
  typedef typename WVec<WT, VEC>::type V;
  const int lane = threadIdx.x & (kWave - 1);
  const int r = blockIdx.x * kWpb + threadIdx.x / kWave;
  if (r >= rows) return;
  const WT* w = W + eoff<WT>((int64_t)r * cols);
  const uint8_t* mxr = mx != nullptr ? mx + (int64_t)r * (cols / 32) : nullptr;
  float acc = 0.0f;
  for (int c = lane * VEC; c < cols; c += kWave * VEC) {
    const V wv = load_wq<WT, VEC>(w + eoff<WT>(c), mxr != nullptr ? mxr + c / 32 : nullptr);
    float xv[VEC];
    load_x<VT, VEC>(v + c, xv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc = fmaf(wdec<WT>(wv, i), xv[i], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[r] = scale != nullptr ? acc * scale[r] : acc;
}

// act = silu(gate) * up (src/naive_moe.cu:117-128).
__global__ void k_swiglu(const float* __restrict__ gate, const float* __restrict__ up,
                         float* __restrict__ act, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) act[i] = silu(gate[i]) * up[i];
}

// accum = (first ? 0 : accum) + w * expert_out; the last expert also writes
// the output in its dtype (src/naive_moe.cu:134-145).
template <typename OT>
__global__ void k_weighted_accum(float* __restrict__ accum, const float* __restrict__ eo,
                                 float w, int n, int first, OT* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float v = (first ? 0.0f : accum[i]) + w * eo[i];
    accum[i] = v;
    if (out != nullptr) out[i] = to_out<OT>(v);
  }
}

struct HostTopK {
  int32_t id[WR_MAX_TOPK];
  float w[WR_MAX_TOPK];
};

// Copies the host-side selection into the caller's optional outputs (kernel
// arguments are captured at launch, so no host buffer must outlive the call).
__global__ void k_write_topk(HostTopK t, int k, int32_t* __restrict__ ids,
                             float* __restrict__ ws) {
  const int i = threadIdx.x;
  if (i < k) {
    if (ids != nullptr) ids[i] = t.id[i];
    if (ws != nullptr) ws[i] = t.w[i];
  }
}

// Host softmax + top-K (src/naive_moe.cu:152-175): max, exp, sequential fp32
// sum, divide; then k rounds of argmax over unused experts with a strict '>'
// starting from -FLT_MAX, so ties go to the lower index.
void host_softmax_topk(const float* logits, int E, int k, int renorm, HostTopK& t) {
  std::vector<float> probs(E);
  float vmax = -FLT_MAX;
  for (int e = 0; e < E; ++e) vmax = std::max(vmax, logits[e]);
  float sum = 0.0f;
  for (int e = 0; e < E; ++e) {
    probs[e] = std::exp(logits[e] - vmax);
    sum += probs[e];
  }
  for (int e = 0; e < E; ++e) probs[e] /= sum;
  std::vector<bool> used(E, false);
  float tot = 0.0f;
  for (int kk = 0; kk < k; ++kk) {
    int best = 0;
    float bval = -FLT_MAX;
    for (int e = 0; e < E; ++e) {
      if (!used[e] && probs[e] > bval) {
        bval = probs[e];
        best = e;
      }
    }
    t.id[kk] = best;
    t.w[kk] = bval;
    tot += bval;
    used[best] = true;
  }
  if (renorm)
    for (int kk = 0; kk < k; ++kk) t.w[kk] = t.w[kk] / tot;
}

template <typename WT, typename XT, int VEC>
hipError_t naive_t(const Problem& p, const NaiveWs& w, const HostTopK& t, hipStream_t s) {
  const char* base = static_cast<const char*>(p.wbuf);
  const XT* x = static_cast<const XT*>(p.x);
  XT* out = static_cast<XT*>(p.out);
  const dim3 gI((p.I + kWpb - 1) / kWpb), gH((p.h + kWpb - 1) / kWpb);
  for (int kk = 0; kk < p.k; ++kk) {
    const char* eb = base + (int64_t)t.id[kk] * p.stride_b;
    const WT* G = reinterpret_cast<const WT*>(eb);
    const WT* U = reinterpret_cast<const WT*>(eb + p.off_up_b);
    const WT* D = reinterpret_cast<const WT*>(eb + p.off_down_b);
    // fp8 row scales: s_gate[I], s_up[I], s_down[h]
    const float* sc = p.wdt == WR_FP8_E4M3
                          ? reinterpret_cast<const float*>(eb + p.off_scale_b)
                          : nullptr;
    // MXFP4 block scales: gate [I][h/32], up [I][h/32], down [h][I/32]
    const uint8_t* mx = p.wdt == WR_MXFP4
                            ? reinterpret_cast<const uint8_t*>(eb + p.off_scale_b)
                            : nullptr;
    const int64_t mxm = (int64_t)p.I * p.h / 32;
    hipLaunchKernelGGL((k_matvec<WT, XT, VEC>), gI, dim3(kBlock), 0, s, G, x, w.gate_vec, p.I,
                       p.h, sc, mx);
    hipLaunchKernelGGL((k_matvec<WT, XT, VEC>), gI, dim3(kBlock), 0, s, U, x, w.up_vec, p.I,
                       p.h, sc != nullptr ? sc + p.I : nullptr, mx != nullptr ? mx + mxm : nullptr);
    hipLaunchKernelGGL(k_swiglu, dim3((p.I + 255) / 256), dim3(256), 0, s, w.gate_vec, w.up_vec,
                       w.act_vec, p.I);
    hipLaunchKernelGGL((k_matvec<WT, float, VEC>), gH, dim3(kBlock), 0, s, D, w.act_vec,
                       w.expert_out, p.h, p.I, sc != nullptr ? sc + 2 * p.I : nullptr,
                       mx != nullptr ? mx + 2 * mxm : nullptr);
    hipLaunchKernelGGL((k_weighted_accum<XT>), dim3((p.h + 255) / 256), dim3(256), 0, s, w.accum,
                       w.expert_out, t.w[kk], p.h, kk == 0 ? 1 : 0,
                       kk == p.k - 1 ? out : static_cast<XT*>(nullptr));
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

template <typename WT, typename XT>
hipError_t naive_w(const Problem& p, const NaiveWs& w, const HostTopK& t, hipStream_t s) {
  constexpr int V = wvec_width<WT>(), V1 = wvec_scalar<WT>();
  return p.vec == V ? naive_t<WT, XT, V>(p, w, t, s) : naive_t<WT, XT, V1>(p, w, t, s);
}

template <typename XT>
hipError_t naive_x(const Problem& p, const NaiveWs& w, const HostTopK& t, hipStream_t s) {
  switch (p.wdt) {
    case WR_F16: return naive_w<f16, XT>(p, w, t, s);
    case WR_BF16: return naive_w<bf16w, XT>(p, w, t, s);
    case WR_FP8_E4M3: return naive_w<fp8w, XT>(p, w, t, s);
    case WR_MXFP4: return naive_w<fp4x2, XT>(p, w, t, s);
    default: return naive_w<float, XT>(p, w, t, s);
  }
}

}  // namespace

hipError_t run_naive(const Problem& p, hipStream_t s) {
  const NaiveWs w = NaiveWs::carve(p.ws, p.E, p.h, p.I);
  hipError_t err = launch_logits(p, w.logits, s);
  if (err != hipSuccess) return err;
  std::vector<float> hl(p.E);
  err = hipMemcpyAsync(hl.data(), w.logits, (size_t)p.E * sizeof(float), hipMemcpyDeviceToHost, s);
  if (err != hipSuccess) return err;
  err = hipStreamSynchronize(s);
  if (err != hipSuccess) return err;
  HostTopK t;
  for (int i = 0; i < WR_MAX_TOPK; ++i) {
    t.id[i] = 0;
    t.w[i] = 0.0f;
  }
  host_softmax_topk(hl.data(), p.E, p.k, p.renorm, t);
  if (p.topk_ids != nullptr || p.topk_w != nullptr) {
    hipLaunchKernelGGL(k_write_topk, dim3(1), dim3(kWave), 0, s, t, p.k, p.topk_ids, p.topk_w);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return p.adt == WR_F16 ? naive_x<f16>(p, w, t, s) : naive_x<float>(p, w, t, s);
}

}  // namespace wr
