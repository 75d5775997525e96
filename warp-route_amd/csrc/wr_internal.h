// Host-side interface between the C-ABI layer (wr_api.hip) and the kernel
// launchers.  A `Problem` is built only from arguments that passed
// validation.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "warp_route.h"

namespace wr {

struct Problem {
  const float* gate_w;
  const void* wbuf;
  int wdt;  // wr_dtype of the weights
  int adt;  // wr_dtype of x and out
  int E, h, I, k, renorm, B;
  const void* x;
  void* out;
  int32_t* topk_ids;
  float* topk_w;
  char* ws;
  size_t ws_bytes;
  int64_t stride_b, off_up_b, off_down_b;  // layout, bytes
  int vec;  // elements per lane per weight access: 8 (fp16), 4 (fp32) or 1
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
constexpr size_t kWsAlign = 256;

// Workspace carving.  Every region starts on a 256-byte boundary.
struct FusedWs {
  // Single-token hand-off, one 256-byte line per word: kCounters arrival
  // counters, the wait-timeout flag, and the flag "a gate/up block ran on an
  // unexpected XCD".  The router kernel of each single-token call zeroes them.
  static constexpr int kCounters = 64;
  static constexpr int kCounterStride = 64;  // words (256 bytes)
  static constexpr int kTimeoutWord = kCounters * kCounterStride;
  static constexpr int kXccFlagWord = kTimeoutWord + kCounterStride;
  static constexpr int kCtrlWords = kCounters + 2;  // zeroed words, kCounterStride apart
  static constexpr size_t kCtrlBytes = (size_t)kCtrlWords * kCounterStride * 4;
  // act rows are I rounded up to whole 8-column chunks.
  static constexpr int kActCols = 8;

  unsigned* ctrl;  // kCtrlBytes
  float* logits;   // [B][WR_MAX_EXPERTS]: token b's E logits, padded to 64
  float* act;      // B == 1: [k][act_row(I)]; B > 1: [B][k][I].
                   // Values are already scaled by the gate weight.

  __host__ __device__ static int64_t act_row(int I) {
    return (int64_t)((I + kActCols - 1) / kActCols) * kActCols;
  }
  static size_t act_floats(int I, int k, int B) {
    return B == 1 ? (size_t)k * act_row(I) : (size_t)B * k * I;
  }
  static size_t bytes(int E, int I, int k, int B) {
    (void)E;
    return kCtrlBytes + (size_t)B * WR_MAX_EXPERTS * 4 +
           align_up(act_floats(I, k, B) * 4, kWsAlign);
  }
  static FusedWs carve(char* ws, int E, int I, int k, int B) {
    FusedWs w;
    w.ctrl = reinterpret_cast<unsigned*>(ws);
    w.logits = reinterpret_cast<float*>(ws + kCtrlBytes);
    w.act = reinterpret_cast<float*>(ws + kCtrlBytes + (size_t)B * WR_MAX_EXPERTS * 4);
    (void)E;
    (void)I;
    (void)k;
    return w;
  }
};

struct NaiveWs {
  float *logits, *gate_vec, *up_vec, *act_vec, *expert_out, *accum;
  static size_t bytes(int E, int h, int I) {
    return align_up((size_t)E * 4, kWsAlign) + 3 * align_up((size_t)I * 4, kWsAlign) +
           2 * align_up((size_t)h * 4, kWsAlign);
  }
  static NaiveWs carve(char* ws, int E, int h, int I) {
    NaiveWs w;
    char* p = ws;
    w.logits = reinterpret_cast<float*>(p);
    p += align_up((size_t)E * 4, kWsAlign);
    w.gate_vec = reinterpret_cast<float*>(p);
    p += align_up((size_t)I * 4, kWsAlign);
    w.up_vec = reinterpret_cast<float*>(p);
    p += align_up((size_t)I * 4, kWsAlign);
    w.act_vec = reinterpret_cast<float*>(p);
    p += align_up((size_t)I * 4, kWsAlign);
    w.expert_out = reinterpret_cast<float*>(p);
    p += align_up((size_t)h * 4, kWsAlign);
    w.accum = reinterpret_cast<float*>(p);
    return w;
  }
};

// Launchers (wr_kernels.hip, wr_naive.hip).  Each returns the first HIP
// error it meets.
hipError_t launch_logits(const Problem& p, float* logits, hipStream_t s);
hipError_t launch_gate_topk(const Problem& p, hipStream_t s);
hipError_t launch_fused(const Problem& p, hipStream_t s);
hipError_t launch_batched(const Problem& p, hipStream_t s);
hipError_t run_naive(const Problem& p, hipStream_t s);

}  // namespace wr
