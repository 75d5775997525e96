// Batched decode MoE for gfx950: tokens grouped by expert, each selected
// expert's weights streamed ONCE for all of its tokens, as small-M GEMMs on
// the matrix cores.
//
// The reference's batched kernel runs one warp per token and re-reads every
// selected expert's weights for every token (src/fused_moe_batched.cu:66-184).
// Here a call with B tokens is five launches:
//   1. k_router_logits (wr_kernels.hip): logits[B][64]; it also splits x into
//      two 16-bit terms.  fp16 terms are of x 2^e_b, with a power of two e_b
//      per token that puts max|x 2^e_b| in [2^14, 2^15): hi stays finite and
//      |x 2^e_b - (hi + lo)| <= 2^-22 |x 2^e_b| + 2^-25 (split_exp).
//   2. k_route: one block selects every token's top-K (the same
//      wave_select_topk as every other path, so ids and weights are
//      bit-identical to the single-token op) and groups the (token, expert)
//      pairs by expert, tokens ascending, with ballot prefix sums
//      (deterministic, no atomics).  For B <= WR_SMALL_TILE_MAX_B there is
//      no k_route launch: every gate/up block of step 3 does the same
//      routing in LDS (route_small), and block (0, 0) publishes it.
//   3. k_gu_mfma: block (row tile, expert slot): 4 waves x 16 gate rows and
//      the same 16 up rows each, all of the expert's tokens (up to 64 per
//      pass); the token tile is staged in LDS and shared by the 4 waves.
//      Tiles of 16 tokens for B <= 16 and 32 for B <= 32; beyond that both
//      the 32- and the 64-token kernels are launched and one of them runs,
//      as k_route's count of experts with more than 32 pairs says
//      (tile_slot).
//      v_mfma_f32_16x16x32_f16 with A = weight rows (fp16, or fp8 E4M3 codes
//      staged as they are and converted exactly to fp16 per fragment) and
//      B = the hi and lo terms of x; products are exact and accumulate in
//      fp32, and the epilogue
//      multiplies by 2^-e_b.  bf16 and MXFP4 weights (E2M1 codes times their
//      E8M0 block scale are exact in bf16 at every scale) use
//      v_mfma_f32_16x16x32_bf16 with x in two bf16 terms instead
//      (|x - (hi + lo)| <= 2^-18 |x|, with fp32's exponent range, so no
//      scaling).  Epilogue: act[pair][row] = w * silu(g) * u
//      (src/fused_moe.cu:192-201), with fp8 row scales applied to g and u (and
//      to the down sums in step 4).  With fp16 operands it also folds
//      max |act[pair][:]| into one word per pair (atomic max).
//   4. k_dn_mfma: block (row tile, K slice, expert slot): the same scheme on
//      the down rows against act, split into two terms while staging (fp16
//      terms of act 2^e_p, e_p from the pair's maximum, undone in the
//      epilogue), four K slices so that the grid has enough blocks; partial
//      sums per slice.  With 64-token tiles (and 32-token tiles of 8- and
//      4-bit weights) k_act_split makes the two terms once, in place, between
//      steps 3 and 4, instead of every row tile's blocks making them again.
//   5. k_combine: out[t] = sum over t's experts (selection order) and K
//      slices (ascending) of the partials, in that fixed order.
// Every sum has a fixed order, so results are deterministic.  The MFMA work
// is padded to 16 tokens per tile; at 2 MFMAs per product term it stays far
// below the time the weight stream takes (the path is HBM-bound).
//
// Requirements (else the per-token kernels in wr_kernels.hip run): fp16,
// bf16, fp8 or MXFP4 weights with 16-byte aligned rows, and h and I
// multiples of 128.  The power-of-two scaling leaves no range condition on x
// or act beyond fp32's own.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "wr_device.h"
#include "wr_internal.h"

namespace wr {

namespace {

#ifndef WR_SMALL_TILE_MAX_B
#define WR_SMALL_TILE_MAX_B 16  // batches up to this size use 16-token tiles
#endif
#ifndef WR_MID_TILE_MAX_B
#define WR_MID_TILE_MAX_B 32    // and up to this size 32-token tiles
#endif
// Larger batches launch both the 32- and the 64-token tile kernels, and one
// of them runs (tile_slot): the 32-token one when no expert has more than
// this many pairs, else the 64-token one, for every expert.  Mixtral, B = 64,
// per call, in 32-token tiles against 64-token tiles: random routing (26
// pairs per expert at most) fp16 486 against 527 us, fp8 316 against 346,
// MXFP4 241 against 290; clustered routing (64 pairs on the pair's experts)
// fp16 346 against 264.  Splitting one call's experts between the two
// launches by their own counts ran the launches one after the other, each on
// part of the chip: clustered fp8 212 against 197 us.
#ifndef WR_TILE_SPLIT_M
#define WR_TILE_SPLIT_M 32
#endif
#ifndef WR_MID_WIDE
#define WR_MID_WIDE 1  // MXFP4 32-token tiles in the wide K step (kc_wide)
#endif
#ifndef WR_W2
// MXFP4 64-token gate/up: weights in 256-column steps (8 rows x 128 bytes
// per load instruction), two 128-column token steps each.  B = 48 / 64:
// 167.0 / 198.8 -> 157.0 / 190.0 us per call (248 VGPRs, 2 blocks per CU).
#define WR_W2 1
#endif
#ifndef WR_W2DN
// The same for the MXFP4 64-token down kernel: B = 48 / 64 155.7 / 187.6 ->
// 147.8 / 180.0 us per call (152 VGPRs, 3 blocks per CU instead of 4).
#define WR_W2DN 1
#endif

constexpr int kBlk = 256;       // 4 waves
constexpr int kBK = 128;        // the base K step (columns); every step width is a multiple
constexpr int kBM = 64;         // rows per block: 4 waves x 16
constexpr int kMaxTok = 64;     // tokens per pass, at most: 4 MFMA N tiles

// The expert slot that z (the grid's slot index) runs in a TOK-token tile
// launch, or -1.  n_active[1] (k_route) counts the experts with more than
// WR_TILE_SPLIT_M pairs: with none, the 32-token launch takes every slot,
// else the 64-token launch does.  The other launch's blocks leave after one
// load.  16-token tiles run alone and take every slot.
template <int TOK>
__device__ __forceinline__ int tile_slot(const BatchRoute& r, int z) {
  static_assert(TOK == 16 || TOK == 32 || TOK == kMaxTok, "tile sizes");
  static_assert(WR_MID_TILE_MAX_B <= WR_TILE_SPLIT_M, "32-token batches lead with no 64-token class");
  if constexpr (TOK == 16) {
    return z < r.n_active[0] ? z : -1;
  } else {
    const int n = r.n_active[0], nb = r.n_active[1];
    const bool mine = TOK == kMaxTok ? nb > 0 : nb == 0;
    return mine && z < n ? z : -1;
  }
}

typedef f16x8 H8;  // eight 16-bit operands: fp16, or bf16 bit patterns
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// MFMA operand type of a weight type: bf16 for bf16 and MXFP4 weights, fp16
// otherwise (fp8 codes are decoded to fp16).
template <typename WT>
constexpr bool bf16_ops() {
  return std::is_same<WT, bf16w>::value || std::is_same<WT, fp4x2>::value;
}

template <bool BF>
__device__ __forceinline__ f32x4 mfma(const H8& a, const H8& b, const f32x4& c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ H8 h8zero() {
  H8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (f16)0.0f;
  return z;
}

// ---------------------------------------------------------------------------
// Routing: one block of 16 waves.  The per-pair selection lives in LDS when it
// fits (kRouteLds pairs), else in the workspace.
// ---------------------------------------------------------------------------
constexpr int kRouteLds = 4096;

// Groups the P = B k selections (sel_id / sel_w, index q = t k + kk) by
// expert: off[E + 1], active (experts with pairs, ascending), *na, and for
// pair p (expert-major, tokens ascending within an expert) pair_tok[p] and
// pair_w[p], with tok_pair[q] = p.  Ballot prefix sums, no atomics, so the
// order is deterministic.  cnt and off_s are LDS scratch of E and E + 1
// ints; the outputs may be LDS or global memory (off may be off_s).  Every
// thread of the block calls it.
__device__ __forceinline__ void group_pairs(int P, int E, int k, const int* sel_id,
                                            const float* sel_w, int* cnt, int* off_s, int* off,
                                            int* active, int* na, int32_t* pair_tok,
                                            float* pair_w, int32_t* tok_pair,
                                            int* nbig = nullptr) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  for (int e = wave; e < E; e += nw) {
    int c = 0;
    for (int q0 = 0; q0 < P; q0 += kWave) {
      const int q = q0 + lane;
      c += __popcll(__ballot(q < P && sel_id[q] == e));
    }
    if (lane == 0) cnt[e] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int o = 0, n = 0;
    for (int e = 0; e < E; ++e) {
      off_s[e] = o;
      off[e] = o;
      o += cnt[e];
    }
    off_s[E] = o;
    off[E] = o;
    int nb = 0;
    for (int e = 0; e < E; ++e) {
      if (cnt[e] > 0) active[n++] = e;
      nb += cnt[e] > WR_TILE_SPLIT_M;
    }
    *na = n;
    if (nbig != nullptr) *nbig = nb;  // experts for 64-token tiles (tile_slot)
  }
  __syncthreads();
  // Stable placement: expert e's pairs in token order.
  for (int e = wave; e < E; e += nw) {
    int j = off_s[e];
    for (int q0 = 0; q0 < P; q0 += kWave) {
      const int q = q0 + lane;
      const bool m = q < P && sel_id[q] == e;
      const unsigned long long mask = __ballot(m);
      if (m) {
        const int pos = j + __popcll(mask & ((1ull << lane) - 1ull));
        pair_tok[pos] = q / k;
        pair_w[pos] = sel_w[q];
        tok_pair[q] = pos;
      }
      j += __popcll(mask);
    }
  }
}

__global__ __launch_bounds__(1024) void k_route(const float* __restrict__ logits, int B, int E,
                                                int k, int renorm, int32_t* __restrict__ ids_out,
                                                float* __restrict__ w_out, BatchRoute r) {
  __shared__ int s_cnt[WR_MAX_EXPERTS];
  __shared__ int s_off[WR_MAX_EXPERTS + 1];
  __shared__ int s_id[kRouteLds];
  __shared__ float s_w[kRouteLds];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int P = B * k;
  int* sel_id = P <= kRouteLds ? s_id : r.sel_id;
  float* sel_w = P <= kRouteLds ? s_w : r.sel_w;

  // Selection.  E <= 16: four tokens per wave at once, one per 16-lane row
  // (row_select_topk).  Else lane e holds logit e, and a wave's next 4 tokens
  // are loaded at once.
  if (E <= 16) {
    const int row = lane >> 4, li = lane & 15;
    for (int t0 = 4 * wave; t0 < B; t0 += 4 * nw) {  // wave-uniform bound
      const int t = t0 + row;
      const float l = t < B ? logits[(int64_t)t * WR_MAX_EXPERTS + li] : 0.0f;
      int sid;
      float sw;
      row_select_topk(l, E, k, renorm, sid, sw);
      if (t < B && li < k) {
        const int q = t * k + li;
        sel_id[q] = sid;
        sel_w[q] = sw;
        if (ids_out != nullptr) ids_out[q] = sid;
        if (w_out != nullptr) w_out[q] = sw;
      }
    }
  } else {
    for (int t0 = wave; t0 < B; t0 += 4 * nw) {
      float l[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + i * nw;
        l[i] = t < B ? logits[(int64_t)t * WR_MAX_EXPERTS + lane] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + i * nw;
        if (t < B) {  // wave-uniform
          TopK tk;
          wave_select_topk_reg(l[i], E, k, renorm, tk);
          if (lane < k) {
            const int q = t * k + lane;
            sel_id[q] = tk.lid;
            sel_w[q] = tk.lw;
            if (ids_out != nullptr) ids_out[q] = tk.lid;
            if (w_out != nullptr) w_out[q] = tk.lw;
          }
        }
      }
    }
  }
  __syncthreads();
  group_pairs(P, E, k, sel_id, sel_w, s_cnt, s_off, r.off, r.active, r.n_active, r.pair_tok,
              r.pair_w, r.tok_pair, r.n_active + 1);
}

// In-block routing for small batches (B <= WR_SMALL_TILE_MAX_B): every
// gate/up block selects the B tokens' experts and groups the pairs itself,
// in LDS, instead of waiting for a separate k_route launch.  The selection
// is the same wave_select_topk_reg, so ids and weights are bit-identical.
constexpr int kSmallPairs = WR_SMALL_TILE_MAX_B * WR_MAX_TOPK;
struct SmallRoute {
  int cnt[WR_MAX_EXPERTS];
  int off[WR_MAX_EXPERTS + 1];
  int active[WR_MAX_EXPERTS];
  int na;
  int sel_id[kSmallPairs];
  float sel_w[kSmallPairs];
  int32_t pair_tok[kSmallPairs];
  float pair_w[kSmallPairs];
  int32_t tok_pair[kSmallPairs];
};

__device__ __forceinline__ void route_small(SmallRoute& sr, const float* __restrict__ logits,
                                            int B, int E, int k, int renorm) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  constexpr int nw = kBlk / kWave;
  if (E <= 16) {  // four tokens per wave at once, one per 16-lane row
    static_assert(WR_SMALL_TILE_MAX_B <= 4 * nw, "one pass");
    const int row = lane >> 4, li = lane & 15;
    const int t = 4 * wave + row;
    const float l = t < B ? logits[(int64_t)t * WR_MAX_EXPERTS + li] : 0.0f;
    int sid;
    float sw;
    row_select_topk(l, E, k, renorm, sid, sw);
    if (t < B && li < k) {
      sr.sel_id[t * k + li] = sid;
      sr.sel_w[t * k + li] = sw;
    }
  } else {
    constexpr int kPer = (WR_SMALL_TILE_MAX_B + nw - 1) / nw;  // tokens per wave, at most
    float l[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {  // all loads in flight before the first selection
      const int t = wave + i * nw;
      l[i] = t < B ? logits[(int64_t)t * WR_MAX_EXPERTS + lane] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int t = wave + i * nw;
      if (t < B) {  // wave-uniform
        TopK tk;
        wave_select_topk_reg(l[i], E, k, renorm, tk);
        if (lane < k) {
          sr.sel_id[t * k + lane] = tk.lid;
          sr.sel_w[t * k + lane] = tk.lw;
        }
      }
    }
  }
  __syncthreads();
  group_pairs(B * k, E, k, sr.sel_id, sr.sel_w, sr.cnt, sr.off, sr.off, sr.active, &sr.na,
              sr.pair_tok, sr.pair_w, sr.tok_pair);
  __syncthreads();
}

// Block (0, 0)'s copy of the routing, for the down and combine kernels (and
// the caller's ids and weights).
__device__ __forceinline__ void route_small_publish(const SmallRoute& sr, int B, int E, int k,
                                                    const BatchRoute& r,
                                                    int32_t* __restrict__ ids_out,
                                                    float* __restrict__ w_out) {
  const int P = B * k;
  for (int i = threadIdx.x; i < P; i += kBlk) {
    r.pair_tok[i] = sr.pair_tok[i];
    r.pair_w[i] = sr.pair_w[i];
    r.tok_pair[i] = sr.tok_pair[i];
    if (ids_out != nullptr) ids_out[i] = sr.sel_id[i];
    if (w_out != nullptr) w_out[i] = sr.sel_w[i];
  }
  for (int e = threadIdx.x; e <= E; e += kBlk) {
    r.off[e] = sr.off[e];
    if (e < E) r.active[e] = sr.active[e];
  }
  if (threadIdx.x == 0) *r.n_active = sr.na;
}

// ---------------------------------------------------------------------------
// K steps.  A step covers KC columns of the K dimension.  Weight rows are
// staged in LDS as the bytes they are and decoded per MFMA fragment, so a
// step's tile costs KC times the weight's bits, not 16 bits per weight.  With
// 16-token tiles the 16-bit and fp8 weights take a step of 256 bytes of row
// (KC = 128 fp16 / bf16, 256 fp8): each wave then has 8 KB of weights in
// flight per step and every load instruction reads 4 rows x 256 bytes (with
// 128-column steps fp8 had half of that in flight, in 8 x 128-byte pieces).
// MXFP4 takes KC = 256, 8 rows x 128 bytes per instruction (KC = 128 was 16
// x 64 bytes; KC = 512, 4 x 256 bytes, left room for fewer blocks per CU),
// with 32-token tiles too.  64-token tiles, the other types' 32-token tiles,
// and K dimensions that the wide step does not divide take KC = 128.
// ---------------------------------------------------------------------------
template <typename WT>
constexpr int wbits() {  // bits per stored weight
  return std::is_same<WT, fp4x2>::value ? 4 : (std::is_same<WT, fp8w>::value ? 8 : 16);
}
// The wide K step of 16-token tiles, in columns: 256 bytes of row for 16-bit
// and fp8 weights; 256 columns (128 bytes) for MXFP4, whose 512-column step
// took 73 KB of LDS and 224 VGPRs in gate/up (2 blocks per CU; 256 columns:
// 40 KB, 144 VGPRs, 3 blocks) and 3 down blocks per CU instead of 5 (B = 16
// 74.7 -> 72.2 us per call, B = 4 68.4 -> 67.8 us).
template <typename WT>
constexpr int kc_wide() {
  return std::is_same<WT, fp4x2>::value ? 256 : 256 * 8 / wbits<WT>();
}

// Token tiles in LDS: hi holds the hi terms, lo the lo terms; row n is token
// n of the pass, piece c covers columns [8 c, 8 c + 8) of the K step.  TOK
// tokens per pass (16, 32 or 64): a launch whose experts have at most 16 (32)
// tokens each takes the smaller tile, whose LDS and registers leave room for
// more blocks per CU.
template <int TOK, int KC>
struct TokTile {
  static constexpr int kP = KC / 8;  // 16-byte pieces per token row
  // The MFMA B-fragment reads (ds_read_b128, lane l at row l % 16, piece
  // 4 j + l / 16) are free of bank conflicts with rows padded by two pieces,
  // or unpadded with piece c of row n at slot c ^ (n mod 16); a one-piece pad
  // measured 4 conflict cycles per read on gfx950 (an LDS probe: 1.7x the
  // conflict-free time).  64-token tiles take the swizzle (4 KB less LDS per
  // block: B = 64 2-5 us faster per call), the others the pad (the swizzle
  // measured up to 1 us slower at B = 4 and 16 with fp8 and MXFP4 weights).
  static constexpr bool kSwz = TOK == 64;
  static_assert(!kSwz || kP % 16 == 0, "the swizzle permutes pieces within a row");
  H8 hi[TOK][kP + (kSwz ? 0 : 2)];
  H8 lo[TOK][kP + (kSwz ? 0 : 2)];
};

// Slot of piece c of token row n of a TokTile.
template <int TOK, int KC>
__device__ __forceinline__ int tslot(int n, int c) {
  return TokTile<TOK, KC>::kSwz ? (c ^ (n & 15)) : c;
}

// One thread's share of a token tile, held in registers between the global
// loads and the LDS stores: pieces i = threadIdx.x + kBlk * q, token row
// n = i / (KC / 8), 8 columns at 8 (i % (KC / 8)) of the K step.
template <int TOK, int KC>
constexpr int tile_pieces() {
  static_assert(TOK * (KC / 8) % kBlk == 0, "whole pieces per thread");
  return TOK * (KC / 8) / kBlk;  // 1, 2 or 4
}

// Element offset of each piece's row start (plus its column), or -1 for a
// padding token; fixed for a whole pass.
template <int KC, int TP>
__device__ __forceinline__ void tile_rows(int64_t (&off)[TP], const int32_t* rows, int direct0,
                                          int mt, int ld) {
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    const int i = threadIdx.x + kBlk * q;
    const int n = i / (KC / 8), c = i % (KC / 8);
    const int row = rows != nullptr ? (n < mt ? rows[n] : 0) : direct0 + n;
    off[q] = n < mt ? (int64_t)row * ld + c * 8 : -1;
  }
}

// Gate/up: x as two precomputed fp16 terms.
template <int TP>
__device__ __forceinline__ void gu_tile_load(H8 (&hi)[TP], H8 (&lo)[TP],
                                             const f16* __restrict__ x_hi,
                                             const f16* __restrict__ x_lo,
                                             const int64_t (&off)[TP], int kb, bool with_lo) {
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    hi[q] = lo[q] = h8zero();
    if (off[q] >= 0) {
      hi[q] = *reinterpret_cast<const H8*>(x_hi + off[q] + kb);
      if (with_lo) lo[q] = *reinterpret_cast<const H8*>(x_lo + off[q] + kb);
    }
  }
}

// Down: act rows, fp32, loaded raw (8 values per piece, zero for padding
// tokens) and split only when stored (dn_tile_split): a split right after the
// loads would wait for them, and, the load counter being in order, for the
// same K step's weight loads issued before them, so no step's loads would be
// in flight during the previous step's MFMAs.
template <int TP>
struct ActRaw {
  f32x4 v[TP][2];
};

template <int TP>
__device__ __forceinline__ void dn_tile_load(ActRaw<TP>& t, const float* __restrict__ act,
                                             const int64_t (&off)[TP], int kb) {
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    t.v[q][0] = t.v[q][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (off[q] >= 0) {
      const float* a = act + off[q] + kb;
      t.v[q][0] = *reinterpret_cast<const f32x4*>(a);
      t.v[q][1] = *reinterpret_cast<const f32x4*>(a + 4);
    }
  }
}

// The two terms of a raw act piece: bf16 terms (BF), or fp16 terms of
// act 2^sx[q] (sx: the piece's pair exponent, split_exp).
template <bool BF, int TP>
__device__ __forceinline__ void dn_tile_split(H8 (&hi)[TP], H8 (&lo)[TP], const ActRaw<TP>& t,
                                              const int (&sx)[TP]) {
#pragma unroll
  for (int q = 0; q < TP; ++q) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float r = t.v[q][i / 4][i % 4];
      const float v = BF ? r : ldexpf(r, sx[q]);
      if constexpr (BF) {
        const __bf16 vh = (__bf16)v;
        hi[q][i] = __builtin_bit_cast(f16, vh);
        lo[q][i] = __builtin_bit_cast(f16, (__bf16)(v - (float)vh));
      } else {
        const f16 vh = (f16)v;
        hi[q][i] = vh;
        lo[q][i] = (f16)(v - (float)vh);
      }
    }
  }
}

// Down with act split ahead of the kernel (k_act_split): each piece of 8
// values holds, in place of their 32 fp32 bytes, their 8 hi terms then their
// 8 lo terms.
template <int TP>
__device__ __forceinline__ void dn_tile_load_split(H8 (&hi)[TP], H8 (&lo)[TP],
                                                   const float* __restrict__ act,
                                                   const int64_t (&off)[TP], int kb) {
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    hi[q] = lo[q] = h8zero();
    if (off[q] >= 0) {
      const H8* a = reinterpret_cast<const H8*>(act + off[q] + kb);
      hi[q] = a[0];
      lo[q] = a[1];
    }
  }
}

template <int TOK, int KC, int TP>
__device__ __forceinline__ void tile_store(TokTile<TOK, KC>& xs, const H8 (&hi)[TP],
                                           const H8 (&lo)[TP], bool with_lo) {
  static_assert(TP == tile_pieces<TOK, KC>(), "tile shares");
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    const int i = threadIdx.x + kBlk * q;
    const int n = i / (KC / 8), c = i % (KC / 8);
    xs.hi[n][tslot<TOK, KC>(n, c)] = hi[q];
    if (with_lo) xs.lo[n][tslot<TOK, KC>(n, c)] = lo[q];
  }
}

// Weight tiles.  A wave's rows are loaded 16 bytes per lane, KC columns of a
// row per group of LR = KC / E lanes (E weights per 16 bytes: 8 fp16 / bf16,
// 16 fp8, 32 MXFP4), RP = 64 / LR rows per instruction: lane l takes row
// RP i + l / LR of group i, the 16 bytes at piece l % LR of the step.  A
// streaming probe measured 4 rows x 256 bytes per instruction at 6.2 TB/s
// against 5.5 TB/s for MFMA fragments loaded straight from memory (16 rows x
// 64 bytes).  The wave stores the bytes as they are into its own LDS tile
// (WTile: rows swizzled or padded for the fragment reads below), MXFP4's
// E8M0 scale bytes (one per piece: a piece is one 32-code block) beside them.  MFMA j of the step reads, in lane l, the 8
// weights of row l % 16 at columns 32 j + 8 (l / 16) and decodes them:
// fp16 and bf16 as they are, fp8 E4M3 codes to fp16 with
// v_cvt_scalef32_pk_f16_fp8 (scale 1: every E4M3 value is an fp16 value),
// MXFP4 codes times their block scale to bf16.
template <typename WT, int KC>
struct WGeo {
  static constexpr int kElems = 128 / wbits<WT>();   // weights per 16 bytes: 8, 16, 32
  static constexpr int kLaneRow = KC / kElems;       // lanes (16-byte pieces) per row
  static constexpr int kRowsPer = kWave / kLaneRow;  // rows per instruction
  static_assert(KC % kElems == 0 && kWave % kLaneRow == 0, "whole pieces, whole rows");
};

// 16-bit weights are read as whole pieces (ds_read_b128): their rows are not
// padded but XOR-swizzled, piece c of row r at slot c ^ (r mod 16), which an
// LDS probe measured free of bank conflicts (a one-piece pad: 4 conflict
// cycles per read).  fp8 fragments are 8-byte reads, conflict-free both with
// the one-piece pad and, in rows of 16 pieces (the 256-byte step), with the
// swizzle, which those tiles take (2 KB less LDS per block).  MXFP4's 4-byte
// reads keep the pad (about 2 conflict cycles per read in every layout tried).
template <typename WT, int ROWS, int KC>
struct WTile {
  static constexpr int kP = WGeo<WT, KC>::kLaneRow;
  static constexpr bool kSwz = wbits<WT>() == 16 || (wbits<WT>() == 8 && kP == 16);
  static_assert(!kSwz || kP == 16, "the swizzle permutes 16 pieces");
  H8 w[ROWS][kP + (kSwz ? 0 : 1)];
  uint8_t s[std::is_same<WT, fp4x2>::value ? ROWS : 1][KC / 32];  // MXFP4 scale bytes
};

template <typename WT, int ROWS, int KC>
__device__ __forceinline__ int wslot(int row, int c) {
  return WTile<WT, ROWS, KC>::kSwz ? (c ^ (row & 15)) : c;
}

// This lane's address of row group 0 at column 0 of the K loop, for the tile
// whose first row is `row` of a matrix with row length ld (elements).
template <typename WT, int KC>
__device__ __forceinline__ const WT* w_lane_base(const WT* mat, int row, int64_t ld, int lane) {
  typedef WGeo<WT, KC> G;
  return mat + eoff<WT>((int64_t)(row + lane / G::kLaneRow) * ld + (lane % G::kLaneRow) * G::kElems);
}

// MXFP4: this lane's E8M0 byte of the same block at column 0 of the K loop,
// for a matrix whose block scales start at sc ([rows][ld / 32] bytes).
template <typename WT, int KC>
__device__ __forceinline__ const uint8_t* w_lane_scale(const uint8_t* sc, int row, int64_t ld,
                                                       int lane) {
  typedef WGeo<WT, KC> G;
  return sc + (int64_t)(row + lane / G::kLaneRow) * (ld / 32) +
         (lane % G::kLaneRow) * G::kElems / 32;
}

template <typename WT, int ROWS, int KC>
struct WRegs {
  static constexpr int N = ROWS / WGeo<WT, KC>::kRowsPer;  // load instructions per K step
  u32x4 v[N];
  uint8_t e[std::is_same<WT, fp4x2>::value ? N : 1];  // MXFP4 E8M0 scale bytes
};

// Loads of one K step: base[i] is this lane's address for row group i at
// column 0 of the K loop (sc[i] its MXFP4 scale byte); kb is the step's
// first column.
template <typename WT, int ROWS, int KC>
__device__ __forceinline__ void w_load(WRegs<WT, ROWS, KC>& r,
                                       const WT* const (&base)[WRegs<WT, ROWS, KC>::N],
                                       const uint8_t* const (&sc)[WRegs<WT, ROWS, KC>::N],
                                       int kb) {
#pragma unroll
  for (int i = 0; i < WRegs<WT, ROWS, KC>::N; ++i) {
    r.v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base[i] + eoff<WT>(kb)));
    if constexpr (std::is_same<WT, fp4x2>::value) r.e[i] = sc[i][kb / 32];
  }
}

__device__ __forceinline__ H8 fp8x8_to_h8(uint32_t a, uint32_t b) {
  typedef f16 h2 __attribute__((ext_vector_type(2)));
  const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(a, 1.0f, false);
  const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(a, 1.0f, true);
  const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(b, 1.0f, false);
  const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(b, 1.0f, true);
  return H8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// MXFP4: eight codes (one 32-bit word, element 2i in the low nibble of byte
// i) -> eight bf16 values times the block scale
// (v_cvt_scalef32_pk_bf16_fp4).  An E2M1 value has at most two significant
// bits and the scale is a power of two, so the product is exact in bf16 at
// every scale bf16's exponent range holds (fp16 would overflow above 2^13 or
// round below 2^-24).
__device__ __forceinline__ H8 fp4x8_to_bf8(uint32_t w, float s) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0);
  const b2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1);
  const b2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2);
  const b2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3);
  return __builtin_bit_cast(H8, bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]});
}

template <typename WT, int ROWS, int KC>
__device__ __forceinline__ void w_store(WTile<WT, ROWS, KC>& t, const WRegs<WT, ROWS, KC>& r,
                                        int lane) {
  constexpr int LR = WGeo<WT, KC>::kLaneRow, RP = WGeo<WT, KC>::kRowsPer;
#pragma unroll
  for (int i = 0; i < WRegs<WT, ROWS, KC>::N; ++i) {
    const int row = RP * i + lane / LR;
    t.w[row][wslot<WT, ROWS, KC>(row, lane % LR)] = __builtin_bit_cast(H8, r.v[i]);
    if constexpr (std::is_same<WT, fp4x2>::value) t.s[row][lane % LR] = r.e[i];
  }
}

// The A operand of MFMA j of a step, in a lane of quadrant q (l / 16): the 8
// weights of tile row `row` at columns 32 j + 8 q, decoded.
template <typename WT, int ROWS, int KC>
__device__ __forceinline__ H8 a_frag(const WTile<WT, ROWS, KC>& t, int row, int j, int q) {
  if constexpr (wbits<WT>() == 16) {
    return t.w[row][wslot<WT, ROWS, KC>(row, 4 * j + q)];
  } else if constexpr (wbits<WT>() == 8) {
    // 16 codes per piece: piece 2 j + q / 2, bytes 8 (q % 2) ..
    const uint2 v = reinterpret_cast<const uint2*>(
        &t.w[row][wslot<WT, ROWS, KC>(row, 2 * j + (q >> 1))])[q & 1];
    return fp8x8_to_h8(v.x, v.y);
  } else {
    // 32 codes (one block) per piece: piece j, dword q
    const uint32_t v = reinterpret_cast<const uint32_t*>(&t.w[row][j])[q];
    return fp4x8_to_bf8(v, e8m0_value(t.s[row][j]));
  }
}

// ---------------------------------------------------------------------------
// Gate/up.  grid (I / 64, expert slots).  One pass covers up to 64 of the
// expert's tokens as NT MFMA tiles of 16; NT is a template parameter so that
// the K loop has no per-tile branches.  A wave's weight tile holds its 16 gate
// rows (tile rows 0-15) and the same 16 up rows (tile rows 16-31).
// ---------------------------------------------------------------------------
// Range scaling of the fp16-operand passes (unused with bf16 operands): x_exp
// = the tokens' x exponents, amax = the per-pair act maxima in global memory
// (kAmaxStride words apart), s_amax = this block's TOK-word LDS copy for the
// current pass, zero between passes.
struct GuScale {
  const int32_t* x_exp;
  unsigned* amax;
  unsigned* s_amax;
};

// WK: the weight K step, KC (the token step) or a multiple of it: each weight
// tile then serves WK / KC token steps (MXFP4 64-token tiles: 8 rows x 128
// bytes per weight load instruction, with the 128-column token tile).
template <typename WT, bool LO, int NT, int TOK, int KC, int WK = KC>
__device__ __forceinline__ void gu_pass(TokTile<TOK, KC>& xs, WTile<WT, 32, WK>& wt,
                                        const WT* const (&wbase)[WRegs<WT, 32, WK>::N],
                                        const uint8_t* const (&wsc)[WRegs<WT, 32, WK>::N],
                                        const f16* __restrict__ x_hi,
                                        const f16* __restrict__ x_lo, const BatchRoute& r,
                                        int p0, int mt, float* __restrict__ act, int row0,
                                        const float* __restrict__ sc, const GuScale& xsc,
                                        const Geom& g, int lane) {
  static_assert(WK % KC == 0 && (WK == KC || std::is_same<WT, fp4x2>::value),
                "a weight step of whole token steps (MXFP4 only)");
  constexpr int R = WK / KC;  // token steps per weight step; h % WK == 0
  f32x4 ag[NT], au[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) ag[n] = au[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int TP = tile_pieces<TOK, KC>();
  int64_t off[TP];
  tile_rows<KC>(off, r.pair_tok + p0, 0, mt, g.h);
  const int ns = g.h / KC;
  // fp16 operands: the epilogue tokens' x exponents, loaded here so that the
  // loads are in flight with the first K step's.
  constexpr bool SC = !bf16_ops<WT>();
  int xe[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int tn = n * 16 + (lane & 15);
    xe[n] = (SC && tn < mt) ? xsc.x_exp[r.pair_tok[p0 + tn]] : 0;
  }

  // Software pipeline, one K step deep: step s+1's token loads, and with the
  // first token step of a weight step the next weight step's loads, are
  // issued before step s's MFMAs.
  WRegs<WT, 32, WK> wr;
  H8 th[TP], tl[TP];
  w_load<WT, 32, WK>(wr, wbase, wsc, 0);
  gu_tile_load(th, tl, x_hi, x_lo, off, 0, LO);
  for (int s0 = 0; s0 < ns; s0 += R) {
#pragma unroll
    for (int hs = 0; hs < R; ++hs) {
      const int s = s0 + hs;
      __syncthreads();  // every wave is done reading the previous tiles
      tile_store(xs, th, tl, LO);
      if (hs == 0) w_store<WT, 32, WK>(wt, wr, lane);
      __syncthreads();
      if constexpr (R == 1) {
        if (s + 1 < ns) {
          w_load<WT, 32, WK>(wr, wbase, wsc, (s + 1) * KC);
          gu_tile_load(th, tl, x_hi, x_lo, off, (s + 1) * KC, LO);
        }
      } else {
        // The next token step's loads first: the load counter is in order,
        // so the store of that tile does not wait for the weights behind it.
        if (s + 1 < ns) gu_tile_load(th, tl, x_hi, x_lo, off, (s + 1) * KC, LO);
        if (hs == 0 && s0 + R < ns) w_load<WT, 32, WK>(wr, wbase, wsc, (s0 + R) * KC);
      }
      // MXFP4: the next step's loads stay ahead of this step's MFMAs (the
      // scheduler sank them below the MFMAs at 32 and 64 tokens, so each
      // step's loads were awaited with no MFMA work in flight).
      if constexpr (std::is_same<WT, fp4x2>::value) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < KC / 32; ++j) {
        const int c = 4 * j + (lane >> 4);
        const int jw = hs * (KC / 32) + j;  // MFMA j of the token step within the weight step
        const H8 ga = a_frag(wt, lane & 15, jw, lane >> 4);
        const H8 ua = a_frag(wt, 16 + (lane & 15), jw, lane >> 4);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const int tn = n * 16 + (lane & 15);
          constexpr bool BF = bf16_ops<WT>();
          const H8 bh = xs.hi[tn][tslot<TOK, KC>(tn, c)];
          ag[n] = mfma<BF>(ga, bh, ag[n]);
          au[n] = mfma<BF>(ua, bh, au[n]);
          if (LO) {
            const H8 bl = xs.lo[tn][tslot<TOK, KC>(tn, c)];
            ag[n] = mfma<BF>(ga, bl, ag[n]);
            au[n] = mfma<BF>(ua, bl, au[n]);
          }
        }
      }
    }
  }

  // D layout: lane holds token n*16 + (lane % 16), rows 4 (lane / 16) .. +4.
  // fp8: sc = the expert's row scales, gate rows at sc, up rows at sc + I.
  // fp16 operands: the sums are of x 2^e_t; ldexpf by -e_t undoes that
  // exactly (a power of two).
  const int rq = row0 + (lane >> 4) * 4;
  f32x4 sg, su;
  if constexpr (std::is_same<WT, fp8w>::value) {
    sg = *reinterpret_cast<const f32x4*>(sc + rq);
    su = *reinterpret_cast<const f32x4*>(sc + g.I + rq);
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int tn = n * 16 + (lane & 15);
    float m = 0.0f;
    if (tn < mt) {
      const int p = p0 + tn;
      const float w = r.pair_w[p];
      f32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gs = SC ? ldexpf(ag[n][i], -xe[n]) : ag[n][i];
        const float us = SC ? ldexpf(au[n][i], -xe[n]) : au[n][i];
        if constexpr (std::is_same<WT, fp8w>::value)
          v[i] = w * (silu(gs * sg[i]) * (us * su[i]));
        else
          v[i] = w * (silu(gs) * us);
        m = fmaxf(m, fabsf(v[i]));
      }
      *reinterpret_cast<f32x4*>(act + (int64_t)p * g.I + rq) = v;
    }
    if constexpr (SC) {
      // max over the 16 rows of this wave's tile (lanes l, l^16, l^32, l^48
      // hold the same token), then over the block's waves in LDS.
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      if (lane < 16 && tn < mt) atomicMax(xsc.s_amax + tn, __float_as_uint(m));
    }
  }
  if constexpr (SC) {
    // One global atomic per token of the pass.  Non-negative floats order
    // like their bit patterns.  The thread that reads an LDS word clears it
    // for the next pass, whose first write comes after the next pass's K-loop
    // barriers.
    __syncthreads();
    if ((int)threadIdx.x < mt) {
      const unsigned v = xsc.s_amax[threadIdx.x];
      xsc.s_amax[threadIdx.x] = 0u;
      __hip_atomic_fetch_max(xsc.amax + (int64_t)(p0 + threadIdx.x) * BatchWs::kAmaxStride, v,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// SmallRoute in LDS, for the ROUTE variant only.
template <bool ROUTE>
struct GuRouteLds {
  SmallRoute sr;
};
template <>
struct GuRouteLds<false> {};

// Blocks per CU the compiler is asked to fit (a VGPR bound; 1 = none), where
// LDS already allows that many and the kernels needed 8 VGPRs more: 64-token
// tiles of fp8 (176 -> 168) and MXFP4 (176 -> 160) weights, 3 blocks instead
// of 2 (B = 64: fp8 201 -> 195 us, MXFP4 202.5 -> 198 us per call); 32-token
// tiles of fp8 weights with fp32 x (136 -> 128), 4 blocks instead of 3 (B = 32
// unchanged); 16-token tiles of fp8 weights in 256-byte steps, with the
// swizzled weight tiles (53 KB of LDS), 3 blocks instead of 2 (176 -> 168;
// B = 4 fp8 94.5 -> 91.2 us, B = 16 95.5 -> 94.3 us).  None spills.
template <typename WT, bool LO, int TOK, int KC, int WK = KC>
constexpr int gu_min_blocks() {
  if (TOK == 64 && wbits<WT>() < 16 && WK == KC) return 3;
  if (TOK == 32 && wbits<WT>() == 8 && LO) return 4;
  if (TOK == 16 && wbits<WT>() == 8 && KC == kc_wide<WT>()) return 3;
  return 1;
}

// ROUTE: the block routes the batch itself (route_small) instead of reading
// k_route's output; block (0, 0) publishes the routing for the later kernels.
template <typename WT, bool LO, int TOK, bool ROUTE, int KC, int WK = KC>
__global__ __launch_bounds__(kBlk, (gu_min_blocks<WT, LO, TOK, KC, WK>())) void k_gu_mfma(const WT* __restrict__ wbuf,
                                                  const f16* __restrict__ x_hi,
                                                  const f16* __restrict__ x_lo,
                                                  const int32_t* __restrict__ x_exp,
                                                  unsigned* __restrict__ amax, BatchRoute r,
                                                  float* __restrict__ act, Geom g,
                                                  const float* __restrict__ logits,
                                                  int32_t* __restrict__ ids_out,
                                                  float* __restrict__ w_out) {
  __shared__ TokTile<TOK, KC> xs;
  __shared__ WTile<WT, 32, WK> wts[kBlk / kWave];
  __shared__ GuRouteLds<ROUTE> rl;
  __shared__ unsigned s_amax[bf16_ops<WT>() ? 1 : TOK];
  if (!bf16_ops<WT>() && (int)threadIdx.x < TOK) s_amax[threadIdx.x] = 0u;
  const GuScale xsc{x_exp, amax, s_amax};
  const int slot = blockIdx.y;
  int e, pbeg, M;
  if constexpr (ROUTE) {
    route_small(rl.sr, logits, g.B, g.E, g.k, g.renorm);
    if (blockIdx.x == 0 && blockIdx.y == 0)
      route_small_publish(rl.sr, g.B, g.E, g.k, r, ids_out, w_out);
    if (slot >= rl.sr.na) return;  // block-uniform
    e = rl.sr.active[slot];
    pbeg = rl.sr.off[e];
    M = rl.sr.off[e + 1] - pbeg;
    r.pair_tok = rl.sr.pair_tok;  // the passes read the LDS copy
    r.pair_w = rl.sr.pair_w;
  } else {
    (void)logits;
    (void)ids_out;
    (void)w_out;
    const int sl = tile_slot<TOK>(r, slot);
    if (sl < 0) return;  // block-uniform
    e = r.active[sl];
    pbeg = r.off[e];
    M = r.off[e + 1] - pbeg;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * kBM + wave * 16;
  const WT* blk = wbuf + (int64_t)e * g.stride;
  const WT* G = w_lane_base<WT, WK>(blk, row0, g.h, lane);
  // Tile rows 0-15: gate rows row0 ..; rows 16-31: the same up rows.
  constexpr int N = WRegs<WT, 32, WK>::N, RP = WGeo<WT, WK>::kRowsPer;
  const WT* wbase[N];
  const uint8_t* wsc[N];
  // MXFP4 block scales: gate [I][h/32], then up [I][h/32]
  const uint8_t* mxs = reinterpret_cast<const uint8_t*>(blk) + g.off_scale;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    wbase[i] = G + (i < N / 2 ? 0 : g.off_up) + eoff<WT>((int64_t)(RP * (i % (N / 2))) * g.h);
    wsc[i] = w_lane_scale<WT, WK>(mxs + (i < N / 2 ? 0 : (int64_t)g.I * g.h / 32), row0, g.h,
                                  lane) +
             (int64_t)(RP * (i % (N / 2))) * (g.h / 32);
  }
  const float* sc = nullptr;
  if constexpr (std::is_same<WT, fp8w>::value) sc = wscales(blk, g.off_scale);
  WTile<WT, 32, WK>& wt = wts[wave];
  for (int m0 = 0; m0 < M; m0 += TOK) {
    const int mt = min(TOK, M - m0);
    const int p0 = pbeg + m0;
    if constexpr (TOK == 16) {
      gu_pass<WT, LO, 1, TOK, KC, WK>(xs, wt, wbase, wsc, x_hi, x_lo, r, p0, mt, act, row0, sc, xsc, g, lane);
    } else if constexpr (TOK == 32) {
      if (mt <= 16)
        gu_pass<WT, LO, 1, TOK, KC, WK>(xs, wt, wbase, wsc, x_hi, x_lo, r, p0, mt, act, row0, sc, xsc, g, lane);
      else
        gu_pass<WT, LO, 2, TOK, KC, WK>(xs, wt, wbase, wsc, x_hi, x_lo, r, p0, mt, act, row0, sc, xsc, g, lane);
    } else {
      switch ((mt + 15) / 16) {
        case 1: gu_pass<WT, LO, 1, TOK, KC, WK>(xs, wt, wbase, wsc, x_hi, x_lo, r, p0, mt, act, row0, sc, xsc, g, lane); break;
        case 2: gu_pass<WT, LO, 2, TOK, KC, WK>(xs, wt, wbase, wsc, x_hi, x_lo, r, p0, mt, act, row0, sc, xsc, g, lane); break;
        case 3: gu_pass<WT, LO, 3, TOK, KC, WK>(xs, wt, wbase, wsc, x_hi, x_lo, r, p0, mt, act, row0, sc, xsc, g, lane); break;
        default: gu_pass<WT, LO, 4, TOK, KC, WK>(xs, wt, wbase, wsc, x_hi, x_lo, r, p0, mt, act, row0, sc, xsc, g, lane); break;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Down.  grid (h / 64, kKSplit, expert slots).  K slice ks covers steps
// [nsteps * ks / kKSplit, nsteps * (ks + 1) / kKSplit).
// ---------------------------------------------------------------------------
// The exponent e_p of pair p's act split (split_exp of its maximum); 0 with
// bf16 operands.
template <typename WT>
__device__ __forceinline__ int pair_exp(const unsigned* __restrict__ amax, int p) {
  if constexpr (bf16_ops<WT>()) {
    (void)amax;
    (void)p;
    return 0;
  } else {
    return split_exp(__uint_as_float(amax[(int64_t)p * BatchWs::kAmaxStride]), false);
  }
}

// WK as in gu_pass: a weight step of WK / KC token steps (MXFP4 64-token
// tiles, act split ahead); sb and se are then multiples of WK / KC.
template <typename WT, int NT, int TOK, int KC, bool PRE, int WK = KC>
__device__ __forceinline__ void dn_pass(TokTile<TOK, KC>& xs, WTile<WT, 16, WK>& wt,
                                        const WT* const (&wbase)[WRegs<WT, 16, WK>::N],
                                        const uint8_t* const (&wsc)[WRegs<WT, 16, WK>::N],
                                        const float* __restrict__ act,
                                        const unsigned* __restrict__ amax, int p0, int mt,
                                        int sb, int se, float* __restrict__ y, int row0,
                                        const float* __restrict__ sdown, const Geom& g,
                                        int lane) {
  static_assert(WK % KC == 0 && (WK == KC || (std::is_same<WT, fp4x2>::value && PRE)),
                "a weight step of whole token steps (MXFP4, act split ahead)");
  constexpr int R = WK / KC;
  f32x4 acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // The epilogue tokens' act exponents, loaded before the K loop.
  int ae[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int tn = n * 16 + (lane & 15);
    ae[n] = tn < mt ? pair_exp<WT>(amax, p0 + tn) : 0;
  }
  if (sb < se) {
    constexpr int TP = tile_pieces<TOK, KC>();
    int64_t off[TP];
    tile_rows<KC>(off, nullptr, p0, mt, g.I);
    int sx[TP];  // each staged piece's pair exponent (act split here)
#pragma unroll
    for (int q = 0; q < TP; ++q) {
      const int n = ((int)threadIdx.x + kBlk * q) / (KC / 8);
      sx[q] = (!PRE && n < mt) ? pair_exp<WT>(amax, p0 + n) : 0;
    }
    WRegs<WT, 16, WK> wr;
    ActRaw<PRE ? 1 : TP> ar;  // act split here: raw pieces
    H8 ph[TP], pl[TP];        // act split ahead: the two terms
    w_load<WT, 16, WK>(wr, wbase, wsc, sb * KC);
    if constexpr (PRE)
      dn_tile_load_split(ph, pl, act, off, sb * KC);
    else
      dn_tile_load(ar, act, off, sb * KC);
    for (int s0 = sb; s0 < se; s0 += R) {
#pragma unroll
      for (int hs = 0; hs < R; ++hs) {
        const int s = s0 + hs;
        __syncthreads();
        if constexpr (PRE) {
          tile_store(xs, ph, pl, true);
        } else {
          H8 th[TP], tl[TP];
          dn_tile_split<bf16_ops<WT>()>(th, tl, ar, sx);
          tile_store(xs, th, tl, true);
        }
        if (hs == 0) w_store<WT, 16, WK>(wt, wr, lane);
        __syncthreads();
        if constexpr (R == 1) {
          if (s + 1 < se) {
            w_load<WT, 16, WK>(wr, wbase, wsc, (s + 1) * KC);
            if constexpr (PRE)
              dn_tile_load_split(ph, pl, act, off, (s + 1) * KC);
            else
              dn_tile_load(ar, act, off, (s + 1) * KC);
          }
        } else {
          // The next act tile's loads first (in-order load counter), as in
          // gu_pass.
          if (s + 1 < se) dn_tile_load_split(ph, pl, act, off, (s + 1) * KC);
          if (hs == 0 && s0 + R < se) w_load<WT, 16, WK>(wr, wbase, wsc, (s0 + R) * KC);
        }
        if constexpr (std::is_same<WT, fp4x2>::value)
          __builtin_amdgcn_sched_barrier(0);  // loads ahead of the MFMAs, as in gu_pass
#pragma unroll
        for (int j = 0; j < KC / 32; ++j) {
          const int c = 4 * j + (lane >> 4);
          const H8 da = a_frag(wt, lane & 15, hs * (KC / 32) + j, lane >> 4);
#pragma unroll
          for (int n = 0; n < NT; ++n) {
            const int tn = n * 16 + (lane & 15);
            acc[n] = mfma<bf16_ops<WT>()>(da, xs.hi[tn][tslot<TOK, KC>(tn, c)], acc[n]);
            acc[n] = mfma<bf16_ops<WT>()>(da, xs.lo[tn][tslot<TOK, KC>(tn, c)], acc[n]);
          }
        }
      }
    }
  }
  // The sums are of act 2^e_p (fp16 operands): ldexpf by -e_p undoes that
  // exactly.  fp8: rows row0 + 4 (lane / 16) .. + 4 times their scales.
  const int rq = row0 + (lane >> 4) * 4;
  f32x4 sd;
  if constexpr (std::is_same<WT, fp8w>::value) sd = *reinterpret_cast<const f32x4*>(sdown + rq);
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int tn = n * 16 + (lane & 15);
    if (tn < mt) {
      f32x4 v = acc[n];
      if constexpr (!bf16_ops<WT>()) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = ldexpf(v[i], -ae[n]);
      }
      if constexpr (std::is_same<WT, fp8w>::value) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] *= sd[i];
      }
      *reinterpret_cast<f32x4*>(y + (int64_t)(p0 + tn) * g.h + rq) = v;
    }
  }
}

// PRE: act was split into its two terms by k_act_split.  WK: the weight K
// step (dn_pass); the K slices are then whole weight steps.
template <typename WT, int TOK, int KC, bool PRE = false, int WK = KC>
__global__ __launch_bounds__(kBlk) void k_dn_mfma(const WT* __restrict__ wbuf, BatchRoute r,
                                                  const float* __restrict__ act,
                                                  const unsigned* __restrict__ amax,
                                                  float* __restrict__ ypart, Geom g, int P) {
  __shared__ TokTile<TOK, KC> xs;
  __shared__ WTile<WT, 16, WK> wts[kBlk / kWave];
  const int slot = tile_slot<TOK>(r, blockIdx.z);
  if (slot < 0) return;
  const int e = r.active[slot];
  const int pbeg = r.off[e], M = r.off[e + 1] - pbeg;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  // Workgroups go to the 8 XCDs round-robin by linear id, so with the grid's
  // own (row tile, K slice) order every XCD ran all K slices and its L2
  // fetched the whole act tensor.  Relabel: XCD pair q serves K slice q, and
  // an XCD's L2 holds a quarter of act.  A bijection on (x, y) whenever
  // gridDim.x is even; the z plane keeps its XCD offset (x*y blocks, a
  // multiple of 8).
  constexpr int kXcd = 8, kPer = kXcd / BatchWs::kKSplit;
  static_assert(kXcd % BatchWs::kKSplit == 0, "K slices per XCD pair");
  int bx = blockIdx.x, ks = blockIdx.y;
  if (gridDim.x % kPer == 0) {
    const int l = blockIdx.x + gridDim.x * blockIdx.y;
    ks = (l % kXcd) / kPer;
    bx = l % kPer + kPer * (l / kXcd);
  }
  const int row0 = bx * kBM + wave * 16;
  constexpr int R = WK / KC;  // token steps per weight step (I % WK == 0)
  const int nsteps = g.I / WK;
  const int sb = nsteps * ks / BatchWs::kKSplit * R;
  const int se = nsteps * (ks + 1) / BatchWs::kKSplit * R;
  const WT* blk = wbuf + (int64_t)e * g.stride;
  const WT* D = w_lane_base<WT, WK>(blk + g.off_down, row0, g.I, lane);
  const float* sdown = nullptr;  // fp8: s_down[h] follows the I gate and I up scales
  if constexpr (std::is_same<WT, fp8w>::value) sdown = wscales(blk, g.off_scale) + 2 * g.I;
  constexpr int N = WRegs<WT, 16, WK>::N;
  const WT* wbase[N];
  const uint8_t* wsc[N];
  // MXFP4 down block scales [h][I/32], after the gate and up scales
  const uint8_t* mxs =
      reinterpret_cast<const uint8_t*>(blk) + g.off_scale + 2 * ((int64_t)g.I * g.h / 32);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    wbase[i] = D + eoff<WT>((int64_t)(WGeo<WT, WK>::kRowsPer * i) * g.I);
    wsc[i] = w_lane_scale<WT, WK>(mxs, row0, g.I, lane) +
             (int64_t)(WGeo<WT, WK>::kRowsPer * i) * (g.I / 32);
  }
  float* y = ypart + (int64_t)ks * P * g.h;
  WTile<WT, 16, WK>& wt = wts[wave];
  for (int m0 = 0; m0 < M; m0 += TOK) {
    const int mt = min(TOK, M - m0);
    if constexpr (TOK == 16) {
      dn_pass<WT, 1, TOK, KC, PRE, WK>(xs, wt, wbase, wsc, act, amax, pbeg + m0, mt, sb, se, y, row0, sdown, g, lane);
    } else if constexpr (TOK == 32) {
      if (mt <= 16)
        dn_pass<WT, 1, TOK, KC, PRE, WK>(xs, wt, wbase, wsc, act, amax, pbeg + m0, mt, sb, se, y, row0, sdown, g, lane);
      else
        dn_pass<WT, 2, TOK, KC, PRE, WK>(xs, wt, wbase, wsc, act, amax, pbeg + m0, mt, sb, se, y, row0, sdown, g, lane);
    } else {
      switch ((mt + 15) / 16) {
        case 1: dn_pass<WT, 1, TOK, KC, PRE, WK>(xs, wt, wbase, wsc, act, amax, pbeg + m0, mt, sb, se, y, row0, sdown, g, lane); break;
        case 2: dn_pass<WT, 2, TOK, KC, PRE, WK>(xs, wt, wbase, wsc, act, amax, pbeg + m0, mt, sb, se, y, row0, sdown, g, lane); break;
        case 3: dn_pass<WT, 3, TOK, KC, PRE, WK>(xs, wt, wbase, wsc, act, amax, pbeg + m0, mt, sb, se, y, row0, sdown, g, lane); break;
        default: dn_pass<WT, 4, TOK, KC, PRE, WK>(xs, wt, wbase, wsc, act, amax, pbeg + m0, mt, sb, se, y, row0, sdown, g, lane); break;
      }
    }
  }
}

// act [P][I] (fp32, I a multiple of 8) split into its two 16-bit terms once,
// in place: each piece of 8 values becomes their 8 hi terms followed by their
// 8 lo terms (bf16 terms with BF, else fp16 terms of act 2^e_p with the
// pair's exponent), the same terms k_dn_mfma's staging makes.  For 32- and
// 64-token tiles, where every 64-row tile's blocks would otherwise split the
// same values again (the down kernel's VALU work was about 2.3 times its
// gate/up kernel's at B = 64).
template <bool BF>
//
// only_big: when not null, the split runs only if *only_big > 0, i.e. when
// the 64-token launch runs (tile_slot); 16-bit weights' 32-token down kernel
// splits act while staging instead.
__global__ __launch_bounds__(kBlk) void k_act_split(float* __restrict__ act,
                                                    const unsigned* __restrict__ amax, int P,
                                                    int I, const int32_t* __restrict__ only_big) {
  if (only_big != nullptr && *only_big == 0) return;  // grid-uniform
  const int pp = I / 8;  // pieces per pair
  const int64_t n = (int64_t)P * pp;
  for (int64_t i = (int64_t)blockIdx.x * kBlk + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlk) {
    const int p = (int)(i / pp);
    float* a = act + i * 8;
    ActRaw<1> t;
    t.v[0][0] = *reinterpret_cast<const f32x4*>(a);
    t.v[0][1] = *reinterpret_cast<const f32x4*>(a + 4);
    const int sx[1] = {
        BF ? 0 : split_exp(__uint_as_float(amax[(int64_t)p * BatchWs::kAmaxStride]), false)};
    H8 hi[1], lo[1];
    dn_tile_split<BF>(hi, lo, t, sx);
    reinterpret_cast<H8*>(a)[0] = hi[0];
    reinterpret_cast<H8*>(a)[1] = lo[0];
  }
}

// ---------------------------------------------------------------------------
// fp32 weights (the reference's only format): v_mfma_f32_16x16x4f32, exact
// fp32 products accumulated in fp32, so x and act need no splitting and no
// scaling.  A K step is 64 columns (256 bytes of a row, as the 16-bit types'
// 128), so the weight loads, tile shapes and LDS footprint match the fp16
// kernels: a wave loads its rows 4 x 256 bytes per instruction into a padded
// tile of 16-byte pieces.  MFMA t = 4 s + m of a K step takes, in lane l
// (quadrant q = l / 16), column 4 (4 s + q) + m for A (weight row l % 16) and
// B (token l % 16) alike: a permutation of the step's 64 columns, the same
// for both operands, so every product is still summed exactly once, and each
// lane's operands for four MFMAs are one 16-byte LDS read.
// ---------------------------------------------------------------------------
constexpr int kBKF = 64;           // K step, fp32 columns
constexpr int kPF = kBKF / 4;      // 16-byte pieces per row of a step

// Rows of 16 pieces, XOR-swizzled: piece c of row r at slot c ^ (r mod 16),
// which keeps the 16-byte operand reads (lane l at row l % 16, piece 4 j + l / 16)
// free of LDS bank conflicts, as for the 16-bit weight tiles.
template <int ROWS>
struct TileF {
  f32x4 v[ROWS][kPF];
};
__device__ __forceinline__ int fslot(int row, int c) { return c ^ (row & 15); }

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One thread's pieces of a TOK-token tile (TOK * kPF / kBlk of them): token
// n = i / kPF, piece c = i % kPF; off = the token row's element offset plus
// 4 c, or -1 for a padding token.
template <int TOK>
constexpr int f32_tile_pieces() {
  static_assert(TOK * kPF % kBlk == 0, "whole pieces per thread");
  return TOK * kPF / kBlk;
}
template <int TP>
__device__ __forceinline__ void f32_tile_rows(int64_t (&off)[TP], const int32_t* rows,
                                              int direct0, int mt, int ld) {
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    const int i = threadIdx.x + kBlk * q;
    const int n = i / kPF, c = i % kPF;
    const int row = rows != nullptr ? (n < mt ? rows[n] : 0) : direct0 + n;
    off[q] = n < mt ? (int64_t)row * ld + c * 4 : -1;
  }
}
// A piece as loaded: four values of the source's own type (zero for a
// padding token).  fp16 x is widened only when stored (f32_tile_store): a
// conversion right after the loads would wait for them and, the load counter
// being in order, for the same K step's weight loads issued before them.
template <typename XT>
struct RawX4 {
  typedef f32x4 type;
};
template <>
struct RawX4<f16> {
  typedef f16x4 type;
};
template <typename XT, int TP>
__device__ __forceinline__ void f32_tile_load(typename RawX4<XT>::type (&t)[TP],
                                              const XT* __restrict__ src,
                                              const int64_t (&off)[TP], int kb) {
  typedef typename RawX4<XT>::type R;
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    t[q] = R{0, 0, 0, 0};
    if (off[q] >= 0) t[q] = *reinterpret_cast<const R*>(src + off[q] + kb);
  }
}
template <int TOK, typename R, int TP>
__device__ __forceinline__ void f32_tile_store(TileF<TOK>& xs, const R (&t)[TP]) {
#pragma unroll
  for (int q = 0; q < TP; ++q) {
    const int i = threadIdx.x + kBlk * q;
    xs.v[i / kPF][fslot(i / kPF, i % kPF)] =
        f32x4{(float)t[q][0], (float)t[q][1], (float)t[q][2], (float)t[q][3]};
  }
}

// A wave's weight rows: ROWS / 4 loads per K step, lane l: row 4 i + l / 16,
// columns 4 (l % 16) .. + 4 of the step.
template <int ROWS>
struct WRegsF {
  static constexpr int N = ROWS / 4;
  f32x4 v[N];
};
template <int ROWS>
__device__ __forceinline__ void f32_w_load(WRegsF<ROWS>& r, const float* const (&base)[ROWS / 4],
                                           int kb) {
#pragma unroll
  for (int i = 0; i < ROWS / 4; ++i)
    r.v[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(base[i] + kb));
}
template <int ROWS>
__device__ __forceinline__ void f32_w_store(TileF<ROWS>& t, const WRegsF<ROWS>& r, int lane) {
#pragma unroll
  for (int i = 0; i < ROWS / 4; ++i)
    t.v[4 * i + lane / 16][fslot(4 * i + lane / 16, lane % 16)] = r.v[i];
}

// Gate/up pass over up to TOK tokens (NT tiles of 16) of one expert, rows
// row0 .. + 16 of its gate and up matrices (tile rows 0-15 and 16-31).
template <typename XT, int NT, int TOK>
__device__ __forceinline__ void gu_pass_f32(TileF<TOK>& xs, TileF<32>& wt,
                                            const float* const (&wbase)[8],
                                            const XT* __restrict__ x, const BatchRoute& r,
                                            int p0, int mt, float* __restrict__ act, int row0,
                                            const Geom& g, int lane) {
  f32x4 ag[NT], au[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) ag[n] = au[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int TP = f32_tile_pieces<TOK>();
  int64_t off[TP];
  f32_tile_rows(off, r.pair_tok + p0, 0, mt, g.h);
  const int ns = g.h / kBKF;
  const int q = lane >> 4, rl = lane & 15;
  WRegsF<32> wr;
  typename RawX4<XT>::type tv[TP];
  f32_w_load<32>(wr, wbase, 0);
  f32_tile_load(tv, x, off, 0);
  for (int s = 0; s < ns; ++s) {
    __syncthreads();  // every wave is done reading the previous tiles
    f32_tile_store(xs, tv);
    f32_w_store<32>(wt, wr, lane);
    __syncthreads();
    if (s + 1 < ns) {
      f32_w_load<32>(wr, wbase, (s + 1) * kBKF);
      f32_tile_load(tv, x, off, (s + 1) * kBKF);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 ga = wt.v[rl][fslot(rl, 4 * j + q)];
      const f32x4 ua = wt.v[16 + rl][fslot(rl, 4 * j + q)];
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const f32x4 b = xs.v[n * 16 + rl][fslot(rl, 4 * j + q)];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          ag[n] = mfma_f32(ga[m], b[m], ag[n]);
          au[n] = mfma_f32(ua[m], b[m], au[n]);
        }
      }
    }
  }
  // D layout: lane holds token n*16 + (lane % 16), rows 4 (lane / 16) .. +4.
  const int rq = row0 + q * 4;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int tn = n * 16 + rl;
    if (tn < mt) {
      const int p = p0 + tn;
      const float w = r.pair_w[p];
      f32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = w * (silu(ag[n][i]) * au[n][i]);
      *reinterpret_cast<f32x4*>(act + (int64_t)p * g.I + rq) = v;
    }
  }
}

// grid (I / 64, expert slots); as k_gu_mfma, with x read as it is (fp32 or
// fp16) and no scaling.
template <typename XT, int TOK, bool ROUTE>
__global__ __launch_bounds__(kBlk) void k_gu_f32(const float* __restrict__ wbuf,
                                                 const XT* __restrict__ x, BatchRoute r,
                                                 float* __restrict__ act, Geom g,
                                                 const float* __restrict__ logits,
                                                 int32_t* __restrict__ ids_out,
                                                 float* __restrict__ w_out) {
  __shared__ TileF<TOK> xs;
  __shared__ TileF<32> wts[kBlk / kWave];
  __shared__ GuRouteLds<ROUTE> rl;
  const int slot = blockIdx.y;
  int e, pbeg, M;
  if constexpr (ROUTE) {
    route_small(rl.sr, logits, g.B, g.E, g.k, g.renorm);
    if (blockIdx.x == 0 && blockIdx.y == 0)
      route_small_publish(rl.sr, g.B, g.E, g.k, r, ids_out, w_out);
    if (slot >= rl.sr.na) return;  // block-uniform
    e = rl.sr.active[slot];
    pbeg = rl.sr.off[e];
    M = rl.sr.off[e + 1] - pbeg;
    r.pair_tok = rl.sr.pair_tok;
    r.pair_w = rl.sr.pair_w;
  } else {
    (void)logits;
    (void)ids_out;
    (void)w_out;
    if (slot >= *r.n_active) return;  // block-uniform
    e = r.active[slot];
    pbeg = r.off[e];
    M = r.off[e + 1] - pbeg;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * kBM + wave * 16;
  const float* blk = wbuf + (int64_t)e * g.stride;
  const float* G = blk + (int64_t)(row0 + lane / 16) * g.h + 4 * (lane % 16);
  const float* wbase[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) wbase[i] = G + (i < 4 ? 0 : g.off_up) + (int64_t)(4 * (i % 4)) * g.h;
  TileF<32>& wt = wts[wave];
  for (int m0 = 0; m0 < M; m0 += TOK) {
    const int mt = min(TOK, M - m0);
    const int p0 = pbeg + m0;
    if constexpr (TOK == 16) {
      gu_pass_f32<XT, 1, TOK>(xs, wt, wbase, x, r, p0, mt, act, row0, g, lane);
    } else if constexpr (TOK == 32) {
      if (mt <= 16)
        gu_pass_f32<XT, 1, TOK>(xs, wt, wbase, x, r, p0, mt, act, row0, g, lane);
      else
        gu_pass_f32<XT, 2, TOK>(xs, wt, wbase, x, r, p0, mt, act, row0, g, lane);
    } else {
      switch ((mt + 15) / 16) {
        case 1: gu_pass_f32<XT, 1, TOK>(xs, wt, wbase, x, r, p0, mt, act, row0, g, lane); break;
        case 2: gu_pass_f32<XT, 2, TOK>(xs, wt, wbase, x, r, p0, mt, act, row0, g, lane); break;
        case 3: gu_pass_f32<XT, 3, TOK>(xs, wt, wbase, x, r, p0, mt, act, row0, g, lane); break;
        default: gu_pass_f32<XT, 4, TOK>(xs, wt, wbase, x, r, p0, mt, act, row0, g, lane); break;
      }
    }
  }
}

// Down pass: K steps [sb, se) of 64 columns, rows row0 .. + 16 of the down
// matrix against the pass's act rows (fp32, as written by the gate/up pass).
template <int NT, int TOK>
__device__ __forceinline__ void dn_pass_f32(TileF<TOK>& xs, TileF<16>& wt,
                                            const float* const (&wbase)[4],
                                            const float* __restrict__ act, int p0, int mt,
                                            int sb, int se, float* __restrict__ y, int row0,
                                            const Geom& g, int lane) {
  f32x4 acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int q = lane >> 4, rl = lane & 15;
  if (sb < se) {
    constexpr int TP = f32_tile_pieces<TOK>();
    int64_t off[TP];
    f32_tile_rows(off, nullptr, p0, mt, g.I);
    WRegsF<16> wr;
    f32x4 tv[TP];
    f32_w_load<16>(wr, wbase, sb * kBKF);
    f32_tile_load(tv, act, off, sb * kBKF);
    for (int s = sb; s < se; ++s) {
      __syncthreads();
      f32_tile_store(xs, tv);
      f32_w_store<16>(wt, wr, lane);
      __syncthreads();
      if (s + 1 < se) {
        f32_w_load<16>(wr, wbase, (s + 1) * kBKF);
        f32_tile_load(tv, act, off, (s + 1) * kBKF);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 da = wt.v[rl][fslot(rl, 4 * j + q)];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const f32x4 b = xs.v[n * 16 + rl][fslot(rl, 4 * j + q)];
#pragma unroll
          for (int m = 0; m < 4; ++m) acc[n] = mfma_f32(da[m], b[m], acc[n]);
        }
      }
    }
  }
  const int rq = row0 + q * 4;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int tn = n * 16 + rl;
    if (tn < mt) *reinterpret_cast<f32x4*>(y + (int64_t)(p0 + tn) * g.h + rq) = acc[n];
  }
}

// grid (h / 64, kKSplit, expert slots); K slice ks covers steps
// [nsteps ks / kKSplit, nsteps (ks + 1) / kKSplit) of I / 64.
template <int TOK>
__global__ __launch_bounds__(kBlk) void k_dn_f32(const float* __restrict__ wbuf, BatchRoute r,
                                                 const float* __restrict__ act,
                                                 float* __restrict__ ypart, Geom g, int P) {
  __shared__ TileF<TOK> xs;
  __shared__ TileF<16> wts[kBlk / kWave];
  const int slot = blockIdx.z;
  if (slot >= *r.n_active) return;
  const int e = r.active[slot];
  const int pbeg = r.off[e], M = r.off[e + 1] - pbeg;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * kBM + wave * 16;
  const int ks = blockIdx.y;
  const int nsteps = g.I / kBKF;
  const int sb = nsteps * ks / BatchWs::kKSplit;
  const int se = nsteps * (ks + 1) / BatchWs::kKSplit;
  const float* D = wbuf + (int64_t)e * g.stride + g.off_down +
                   (int64_t)(row0 + lane / 16) * g.I + 4 * (lane % 16);
  const float* wbase[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wbase[i] = D + (int64_t)(4 * i) * g.I;
  float* y = ypart + (int64_t)ks * P * g.h;
  TileF<16>& wt = wts[wave];
  for (int m0 = 0; m0 < M; m0 += TOK) {
    const int mt = min(TOK, M - m0);
    if constexpr (TOK == 16) {
      dn_pass_f32<1, TOK>(xs, wt, wbase, act, pbeg + m0, mt, sb, se, y, row0, g, lane);
    } else if constexpr (TOK == 32) {
      if (mt <= 16)
        dn_pass_f32<1, TOK>(xs, wt, wbase, act, pbeg + m0, mt, sb, se, y, row0, g, lane);
      else
        dn_pass_f32<2, TOK>(xs, wt, wbase, act, pbeg + m0, mt, sb, se, y, row0, g, lane);
    } else {
      switch ((mt + 15) / 16) {
        case 1: dn_pass_f32<1, TOK>(xs, wt, wbase, act, pbeg + m0, mt, sb, se, y, row0, g, lane); break;
        case 2: dn_pass_f32<2, TOK>(xs, wt, wbase, act, pbeg + m0, mt, sb, se, y, row0, g, lane); break;
        case 3: dn_pass_f32<3, TOK>(xs, wt, wbase, act, pbeg + m0, mt, sb, se, y, row0, g, lane); break;
        default: dn_pass_f32<4, TOK>(xs, wt, wbase, act, pbeg + m0, mt, sb, se, y, row0, g, lane); break;
      }
    }
  }
}

// out[t][row]: grid (ceil(h / 256), B); K = k, so that every loop is exact.
// Every pair index, then every partial, is loaded before the first add (two
// round trips instead of 2 K); the adds keep their order (experts in
// selection order, K slices ascending).
template <typename OT, int K>
__global__ __launch_bounds__(kBlk) void k_combine(const float* __restrict__ ypart, BatchRoute r,
                                                  OT* __restrict__ out, int h, int P) {
  const int t = blockIdx.y;
  const int row = blockIdx.x * kBlk + threadIdx.x;
  if (row >= h) return;
  int p[K];
#pragma unroll
  for (int kk = 0; kk < K; ++kk) p[kk] = r.tok_pair[t * K + kk];
  float v[K][BatchWs::kKSplit];
#pragma unroll
  for (int kk = 0; kk < K; ++kk)
#pragma unroll
    for (int ks = 0; ks < BatchWs::kKSplit; ++ks)
      v[kk][ks] = ypart[((int64_t)ks * P + p[kk]) * h + row];
  float s = 0.0f;
#pragma unroll
  for (int kk = 0; kk < K; ++kk)
#pragma unroll
    for (int ks = 0; ks < BatchWs::kKSplit; ++ks) s += v[kk][ks];
  out[(int64_t)t * h + row] = to_out<OT>(s);
}

template <typename OT, int K>
hipError_t launch_combine(const BatchWs& w, const Problem& p, hipStream_t s) {
  hipLaunchKernelGGL((k_combine<OT, K>), dim3((p.h + kBlk - 1) / kBlk, p.B), dim3(kBlk), 0, s,
                     w.ypart, w.route, static_cast<OT*>(p.out), p.h, p.B * K);
  return hipGetLastError();
}

template <typename WT, typename XT>
hipError_t grouped_t(const Problem& p, const BatchWs& w, hipStream_t s) {
  constexpr int64_t es = sizeof(WT);  // bytes per storage unit (two MXFP4 codes per byte)
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
  const int P = p.B * p.k;
  const int slots = std::min(p.E, P);
  const WT* wb = static_cast<const WT*>(p.wbuf);

  hipError_t err = hipSuccess;
  // Small batches route inside the gate/up kernel (one launch fewer).
  if (p.B > WR_SMALL_TILE_MAX_B) {
    hipLaunchKernelGGL(k_route, dim3(1), dim3(1024), 0, s, w.logits, p.B, p.E, p.k, p.renorm,
                       p.topk_ids, p.topk_w, w.route);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // The lo term of x: fp32 x, or any x against bf16 (8-bit mantissa) terms.
  constexpr bool LO = std::is_same<XT, float>::value || bf16_ops<WT>();
  // An expert has at most B tokens (a token selects it at most once), so
  // small batches take token tiles of 16 or 32.
  if (p.B <= WR_SMALL_TILE_MAX_B) {
    // 16-token tiles: the wide K steps (kc_wide) where the K dimension (h for
    // gate/up, I for down) is a multiple of them.
    constexpr int KW = kc_wide<WT>();
    if (p.h % KW == 0)
      hipLaunchKernelGGL((k_gu_mfma<WT, LO, 16, true, KW>), dim3(p.I / kBM, slots), dim3(kBlk), 0,
                         s, wb, w.x_hi, w.x_lo, w.x_exp, w.amax, w.route, w.act, g, w.logits,
                         p.topk_ids, p.topk_w);
    else
      hipLaunchKernelGGL((k_gu_mfma<WT, LO, 16, true, kBK>), dim3(p.I / kBM, slots), dim3(kBlk), 0,
                         s, wb, w.x_hi, w.x_lo, w.x_exp, w.amax, w.route, w.act, g, w.logits,
                         p.topk_ids, p.topk_w);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (p.I % KW == 0)
      hipLaunchKernelGGL((k_dn_mfma<WT, 16, KW>), dim3(p.h / kBM, BatchWs::kKSplit, slots),
                         dim3(kBlk), 0, s, wb, w.route, w.act, w.amax, w.ypart, g, P);
    else
      hipLaunchKernelGGL((k_dn_mfma<WT, 16, kBK>), dim3(p.h / kBM, BatchWs::kKSplit, slots),
                         dim3(kBlk), 0, s, wb, w.route, w.act, w.amax, w.ypart, g, P);
  } else {
    // 64-token tiles, and 32-token tiles of 8- and 4-bit weights: act split
    // once between the two GEMMs (k_act_split).  Measured, per call: B = 64
    // fp16 281 -> 275 us, fp8 226 -> 213 us, MXFP4 218 -> 215 us, bf16
    // unchanged; B = 32 fp8 125 -> 123 us, MXFP4 124 -> 122 us, but fp16 164 ->
    // 168 us and bf16 161 -> 165 us (the launch costs more than the repeated
    // splits of 32-token tiles).
    constexpr bool kPre32 = wbits<WT>() < 16;
    const bool mid = p.B <= WR_MID_TILE_MAX_B;
    // MXFP4 32-token tiles: the wide step where it divides h (gate/up) or I
    // (down); its 128-column step loads 16 rows x 64 bytes per instruction.
    // B = 24 / 32: 115.1 / 119.6 -> 102.8 / 103.5 us per call (gate/up 176
    // VGPRs, 2 blocks per CU; a 3-block bound, 144 VGPRs, measured slower).
    constexpr int KM = (WR_MID_WIDE && std::is_same<WT, fp4x2>::value) ? kc_wide<WT>() : kBK;
    // Beyond WR_MID_TILE_MAX_B both tile launches are made and one of them
    // runs (tile_slot).
    if (KM != kBK && p.h % KM == 0)
      hipLaunchKernelGGL((k_gu_mfma<WT, LO, 32, false, KM>), dim3(p.I / kBM, slots), dim3(kBlk),
                         0, s, wb, w.x_hi, w.x_lo, w.x_exp, w.amax, w.route, w.act, g, nullptr,
                         nullptr, nullptr);
    else
      hipLaunchKernelGGL((k_gu_mfma<WT, LO, 32, false, kBK>), dim3(p.I / kBM, slots), dim3(kBlk),
                         0, s, wb, w.x_hi, w.x_lo, w.x_exp, w.amax, w.route, w.act, g, nullptr,
                         nullptr, nullptr);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (!mid) {
      bool wide = false;
      if constexpr (WR_W2 && std::is_same<WT, fp4x2>::value) {
        wide = p.h % kc_wide<WT>() == 0;
        if (wide)
          hipLaunchKernelGGL((k_gu_mfma<WT, LO, kMaxTok, false, kBK, kc_wide<WT>()>),
                             dim3(p.I / kBM, slots), dim3(kBlk), 0, s, wb, w.x_hi, w.x_lo,
                             w.x_exp, w.amax, w.route, w.act, g, nullptr, nullptr, nullptr);
      }
      if (!wide)
        hipLaunchKernelGGL((k_gu_mfma<WT, LO, kMaxTok, false, kBK>), dim3(p.I / kBM, slots),
                           dim3(kBlk), 0, s, wb, w.x_hi, w.x_lo, w.x_exp, w.amax, w.route, w.act,
                           g, nullptr, nullptr, nullptr);
    }
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (!mid || kPre32) {
      const int64_t pieces = (int64_t)P * (p.I / 8);
      const int split_blocks = (int)std::min<int64_t>((pieces + kBlk - 1) / kBlk, 4096);
      hipLaunchKernelGGL((k_act_split<bf16_ops<WT>()>), dim3(split_blocks), dim3(kBlk), 0, s,
                         w.act, w.amax, P, p.I,
                         kPre32 ? nullptr : static_cast<const int32_t*>(w.route.n_active + 1));
      if ((err = hipGetLastError()) != hipSuccess) return err;
    }
    if (mid && KM != kBK && p.I % KM == 0)
      hipLaunchKernelGGL((k_dn_mfma<WT, 32, KM, kPre32>), dim3(p.h / kBM, BatchWs::kKSplit, slots),
                         dim3(kBlk), 0, s, wb, w.route, w.act, w.amax, w.ypart, g, P);
    else if (mid)
      hipLaunchKernelGGL((k_dn_mfma<WT, 32, kBK, kPre32>), dim3(p.h / kBM, BatchWs::kKSplit, slots),
                         dim3(kBlk), 0, s, wb, w.route, w.act, w.amax, w.ypart, g, P);
    else {
      // act is split when the 64-token launch runs, and for 8- and 4-bit
      // weights always
      if (KM != kBK && p.I % KM == 0)
        hipLaunchKernelGGL((k_dn_mfma<WT, 32, KM, kPre32>),
                           dim3(p.h / kBM, BatchWs::kKSplit, slots), dim3(kBlk), 0, s, wb,
                           w.route, w.act, w.amax, w.ypart, g, P);
      else
        hipLaunchKernelGGL((k_dn_mfma<WT, 32, kBK, kPre32>),
                           dim3(p.h / kBM, BatchWs::kKSplit, slots), dim3(kBlk), 0, s, wb,
                           w.route, w.act, w.amax, w.ypart, g, P);
      if ((err = hipGetLastError()) != hipSuccess) return err;
      bool wide = false;
      if constexpr (WR_W2DN && std::is_same<WT, fp4x2>::value) {
        wide = p.I % kc_wide<WT>() == 0;
        if (wide)
          hipLaunchKernelGGL((k_dn_mfma<WT, kMaxTok, kBK, true, kc_wide<WT>()>),
                             dim3(p.h / kBM, BatchWs::kKSplit, slots), dim3(kBlk), 0, s, wb,
                             w.route, w.act, w.amax, w.ypart, g, P);
      }
      if (!wide)
        hipLaunchKernelGGL((k_dn_mfma<WT, kMaxTok, kBK, true>),
                           dim3(p.h / kBM, BatchWs::kKSplit, slots), dim3(kBlk), 0, s, wb,
                           w.route, w.act, w.amax, w.ypart, g, P);
    }
  }
  if ((err = hipGetLastError()) != hipSuccess) return err;
  static_assert(WR_MAX_TOPK == 6, "one combine instantiation per k");
  switch (p.k) {
    case 1: return launch_combine<XT, 1>(w, p, s);
    case 2: return launch_combine<XT, 2>(w, p, s);
    case 3: return launch_combine<XT, 3>(w, p, s);
    case 4: return launch_combine<XT, 4>(w, p, s);
    case 5: return launch_combine<XT, 5>(w, p, s);
    default: return launch_combine<XT, 6>(w, p, s);
  }
}

template <typename XT>
hipError_t grouped_f32(const Problem& p, const BatchWs& w, hipStream_t s) {
  Geom g;
  g.E = p.E;
  g.h = p.h;
  g.I = p.I;
  g.k = p.k;
  g.renorm = p.renorm;
  g.B = p.B;
  g.stride = p.stride_b / 4;
  g.off_up = p.off_up_b / 4;
  g.off_down = p.off_down_b / 4;
  g.off_scale = -1;
  const int P = p.B * p.k;
  const int slots = std::min(p.E, P);
  const float* wb = static_cast<const float*>(p.wbuf);
  const XT* x = static_cast<const XT*>(p.x);
  hipError_t err = hipSuccess;
  if (p.B > WR_SMALL_TILE_MAX_B) {
    hipLaunchKernelGGL(k_route, dim3(1), dim3(1024), 0, s, w.logits, p.B, p.E, p.k, p.renorm,
                       p.topk_ids, p.topk_w, w.route);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if (p.B <= WR_SMALL_TILE_MAX_B) {
    hipLaunchKernelGGL((k_gu_f32<XT, 16, true>), dim3(p.I / kBM, slots), dim3(kBlk), 0, s, wb, x,
                       w.route, w.act, g, w.logits, p.topk_ids, p.topk_w);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    hipLaunchKernelGGL((k_dn_f32<16>), dim3(p.h / kBM, BatchWs::kKSplit, slots), dim3(kBlk), 0, s,
                       wb, w.route, w.act, w.ypart, g, P);
  } else if (p.B <= WR_MID_TILE_MAX_B) {
    hipLaunchKernelGGL((k_gu_f32<XT, 32, false>), dim3(p.I / kBM, slots), dim3(kBlk), 0, s, wb, x,
                       w.route, w.act, g, nullptr, nullptr, nullptr);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    hipLaunchKernelGGL((k_dn_f32<32>), dim3(p.h / kBM, BatchWs::kKSplit, slots), dim3(kBlk), 0, s,
                       wb, w.route, w.act, w.ypart, g, P);
  } else {
    hipLaunchKernelGGL((k_gu_f32<XT, kMaxTok, false>), dim3(p.I / kBM, slots), dim3(kBlk), 0, s,
                       wb, x, w.route, w.act, g, nullptr, nullptr, nullptr);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    hipLaunchKernelGGL((k_dn_f32<kMaxTok>), dim3(p.h / kBM, BatchWs::kKSplit, slots), dim3(kBlk),
                       0, s, wb, w.route, w.act, w.ypart, g, P);
  }
  if ((err = hipGetLastError()) != hipSuccess) return err;
  switch (p.k) {
    case 1: return launch_combine<XT, 1>(w, p, s);
    case 2: return launch_combine<XT, 2>(w, p, s);
    case 3: return launch_combine<XT, 3>(w, p, s);
    case 4: return launch_combine<XT, 4>(w, p, s);
    case 5: return launch_combine<XT, 5>(w, p, s);
    default: return launch_combine<XT, 6>(w, p, s);
  }
}

}  // namespace

bool grouped_ok(const Problem& p) {
  if (p.B <= 1) return false;
  if (p.wdt == WR_F32)  // 64-column K steps, 16-byte rows
    return p.vec == 4 && p.h % kBKF == 0 && p.I % kBKF == 0;
  const bool wt = ((p.wdt == WR_F16 || p.wdt == WR_BF16) && p.vec == 8) ||
                  (p.wdt == WR_FP8_E4M3 && p.vec == 16) || (p.wdt == WR_MXFP4 && p.vec == 32);
  return wt && p.h % kBK == 0 && p.I % kBK == 0;
}

hipError_t launch_grouped(const Problem& p, hipStream_t s) {
  const BatchWs w = BatchWs::carve(p.ws, p.E, p.h, p.I, p.k, p.B);
  if (p.wdt == WR_F32) {  // exact fp32 products: x as it is, logits only
    hipError_t err = launch_logits(p, w.logits, s);
    if (err != hipSuccess) return err;
    return p.adt == WR_F16 ? grouped_f32<f16>(p, w, s) : grouped_f32<float>(p, w, s);
  }
  // bf16 operands (bf16 and MXFP4 weights): bf16 terms, no scaling.
  const bool bf = p.wdt == WR_BF16 || p.wdt == WR_MXFP4;
  hipError_t err = launch_logits_split(p, w.logits, w.x_hi, w.x_lo, w.x_exp,
                                       bf ? nullptr : w.amax, bf ? 1 : 0, s);
  if (err != hipSuccess) return err;
  if (p.wdt == WR_FP8_E4M3)
    return p.adt == WR_F16 ? grouped_t<fp8w, f16>(p, w, s) : grouped_t<fp8w, float>(p, w, s);
  if (p.wdt == WR_BF16)
    return p.adt == WR_F16 ? grouped_t<bf16w, f16>(p, w, s) : grouped_t<bf16w, float>(p, w, s);
  if (p.wdt == WR_MXFP4)
    return p.adt == WR_F16 ? grouped_t<fp4x2, f16>(p, w, s) : grouped_t<fp4x2, float>(p, w, s);
  return p.adt == WR_F16 ? grouped_t<f16, f16>(p, w, s) : grouped_t<f16, float>(p, w, s);
}

}  // namespace wr
