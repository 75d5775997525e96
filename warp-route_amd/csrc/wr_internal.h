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
  int64_t off_scale_b;  // fp8 scales [3][I] fp32 within an expert block, bytes; -1 if none
  int vec;  // elements per lane per weight access: 16 / element bytes, or 1
  // Single-token hand-off wait: polls before a down block gives up, and a
  // count added to every arrival target (nonzero only to force the expiry
  // path from the host in tests: the wait then cannot complete).
  unsigned spin_limit, wait_extra;
  // Single-token gate/up blocks launched: 0 = as many as are resident at once
  // (the rest of the gate/up chunks are claimed by the blocks that finish
  // first), else this many (tests).
  int gu_blocks;
  // Host-visible word (pinned host memory) that a single-token call's kernel
  // also sets when a hand-off wait expires, so that an expiry can be seen
  // without synchronising; nullptr: not written.
  unsigned* expired_host;
};

// Polls of the single-token hand-off wait before it expires (about 0.2 s).
constexpr unsigned kDefaultSpinLimit = 1u << 20;

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
constexpr size_t kWsAlign = 256;

// Workspace carving.  Every region starts on a 256-byte boundary.
struct FusedWs {
  // Single-token hand-off, one 256-byte line per word: kCounters 64-bit
  // arrival words (each gate/up slot adds its arrival and its XCD rotation,
  // (its XCD - block) mod 8, to word slot mod kCounters), the wait-timeout
  // flag, an unused word, then kClasses claim counters of the gate/up chunks
  // beyond the launched blocks (class b mod 8).  The router launch of each
  // single-token call zeroes the first 8 bytes of each line (when the router
  // runs inside the single-token kernel, that kernel's block 0 does, before
  // it publishes its router slot).
  static constexpr int kCounters = 64;
  static constexpr int kClasses = 8;
  static constexpr int kCounterStride = 64;  // words (256 bytes)
  static constexpr int kTimeoutWord = kCounters * kCounterStride;
  static constexpr int kClaimWord = kTimeoutWord + 2 * kCounterStride;
  static constexpr int kCtrlWords = kCounters + 2 + kClasses;  // zeroed lines, kCounterStride apart
  // Router slots (a kernel with the router inside) after the zeroed words, 16 bytes per
  // expert: two 64-bit words {logit bits, tag half} carrying the tag of the
  // call that wrote them (never zeroed: a slot counts only when it carries
  // the reader's own call tag).  kSlotReplicas copies, kReplicaBytes apart (9
  // cache lines, so that the copies start on different L2 channels); block b
  // polls copy b mod kSlotReplicas, which spreads the polls of a whole grid.
  static constexpr int kSlotWord = kCtrlWords * kCounterStride;
  static constexpr int kSlotBytes = 16;
  static constexpr int kSlotReplicas = 16;
  static constexpr int kReplicaBytes = 1152;
  static_assert(WR_MAX_EXPERTS * kSlotBytes <= kReplicaBytes, "a copy holds every slot");
  static constexpr size_t kCtrlBytes = (size_t)kSlotWord * 4 + (size_t)kSlotReplicas * kReplicaBytes;
  // Single-token act rows: I rounded up to whole chunks of `cols` columns, the
  // columns one gate/up block computes (4 waves x rows per wave: 8 or 16).
  static constexpr int kMaxActCols = 16;

  unsigned* ctrl;  // kCtrlBytes
  float* logits;   // [B][WR_MAX_EXPERTS]: token b's E logits, padded to 64
  float* act;      // B == 1: [k][act_row(I, cols)]; B > 1: [B][k][I].
                   // Values are already scaled by the gate weight.

  __host__ __device__ static int64_t act_row(int I, int cols) {
    return (int64_t)((I + cols - 1) / cols) * cols;
  }
  static size_t act_floats(int I, int k, int B) {
    return B == 1 ? (size_t)k * act_row(I, kMaxActCols) : (size_t)B * k * I;
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

// Grouped batched path (wr_batched.hip): (token, expert) pairs grouped by
// expert.  Pair q = t * k + kk is token t's kk-th selection; grouped index p
// orders the pairs by expert, tokens ascending.
struct BatchRoute {
  int32_t* sel_id;    // [P] by q
  float* sel_w;       // [P] by q
  int32_t* pair_tok;  // [P] by p: token
  float* pair_w;      // [P] by p: gate weight
  int32_t* tok_pair;  // [P] by q: p
  int32_t* off;       // [E + 1]: expert e's pairs are [off[e], off[e + 1])
  int32_t* active;    // [E]: experts with pairs, ascending
  int32_t* n_active;  // [2]: experts with pairs; how many have more than 32 (k_route)
};

struct BatchWs {
  static constexpr int kKSplit = 4;  // K slices of the down GEMM
  // Per-pair act maxima sit one per 256-byte line, so that the gate/up
  // blocks' atomic max updates of different pairs do not serialise.
  static constexpr int kAmaxStride = 64;  // words
  float* logits;  // [B][WR_MAX_EXPERTS]
  // x 2^x_exp[b] = hi + lo: fp16 terms (x_exp chosen so that max|x 2^x_exp|
  // lies in [2^14, 2^15)), or bf16 bit patterns for bf16-operand weights
  // (bf16 and MXFP4; x_exp = 0).
  _Float16* x_hi;  // [B][h]
  _Float16* x_lo;  // [B][h]
  int32_t* x_exp;  // [B]
  // amax[p * kAmaxStride]: max |act[p][:]| as fp32 bits (fp16-operand
  // weights only), built with atomic max by the gate/up kernel; the down
  // kernel scales pair p's act by a power of two from it before splitting.
  unsigned* amax;
  BatchRoute route;
  float* act;    // [P][I], grouped pair order, scaled by the gate weight
  float* ypart;  // [kKSplit][P][h]: down partial sums
  static size_t bytes(int E, int h, int I, int k, int B) {
    size_t n = 0;
    carve_into(nullptr, &n, E, h, I, k, B);
    return n;
  }
  static BatchWs carve(char* ws, int E, int h, int I, int k, int B) {
    return carve_into(ws, nullptr, E, h, I, k, B);
  }

 private:
  static BatchWs carve_into(char* ws, size_t* total, int E, int h, int I, int k, int B) {
    BatchWs w;
    size_t off = 0;
    auto take = [&](size_t bytes) {
      char* p = ws == nullptr ? nullptr : ws + off;
      off += align_up(bytes, kWsAlign);
      return p;
    };
    const size_t P = (size_t)B * k;
    w.logits = reinterpret_cast<float*>(take((size_t)B * WR_MAX_EXPERTS * 4));
    w.x_hi = reinterpret_cast<_Float16*>(take((size_t)B * h * 2));
    w.x_lo = reinterpret_cast<_Float16*>(take((size_t)B * h * 2));
    w.x_exp = reinterpret_cast<int32_t*>(take((size_t)B * 4));
    w.amax = reinterpret_cast<unsigned*>(take(P * kAmaxStride * 4));
    w.route.sel_id = reinterpret_cast<int32_t*>(take(P * 4));
    w.route.sel_w = reinterpret_cast<float*>(take(P * 4));
    w.route.pair_tok = reinterpret_cast<int32_t*>(take(P * 4));
    w.route.pair_w = reinterpret_cast<float*>(take(P * 4));
    w.route.tok_pair = reinterpret_cast<int32_t*>(take(P * 4));
    w.route.off = reinterpret_cast<int32_t*>(take((size_t)(E + 1) * 4));
    w.route.active = reinterpret_cast<int32_t*>(take((size_t)E * 4));
    w.route.n_active = reinterpret_cast<int32_t*>(take(8));
    w.act = reinterpret_cast<float*>(take(P * I * 4));
    w.ypart = reinterpret_cast<float*>(take((size_t)kKSplit * P * h * 4));
    if (total != nullptr) *total = off;
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
// Logits, plus x split into two 16-bit terms for the grouped batched path:
// bf16 terms x = hi + lo when split_bf16, else fp16 terms
// x 2^x_exp[b] = hi + lo (lo = 0 for fp16 x); also zeroes amax (k words per
// token, BatchWs::kAmaxStride apart) when it is not NULL.
hipError_t launch_logits_split(const Problem& p, float* logits, _Float16* x_hi, _Float16* x_lo,
                               int32_t* x_exp, unsigned* amax, int split_bf16, hipStream_t s);
// Grouped batched path: usable when grouped_ok(p).
bool grouped_ok(const Problem& p);
hipError_t launch_grouped(const Problem& p, hipStream_t s);
hipError_t launch_gate_topk(const Problem& p, hipStream_t s);
hipError_t launch_fused(const Problem& p, hipStream_t s);
// The two launches of launch_fused, for callers that issue them separately.
hipError_t launch_fused_route(const Problem& p, hipStream_t s);
hipError_t launch_fused_ffn(const Problem& p, hipStream_t s);
hipError_t launch_batched(const Problem& p, hipStream_t s);
hipError_t run_naive(const Problem& p, hipStream_t s);

}  // namespace wr
