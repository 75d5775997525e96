/*
 * warp_route.h -- C-ABI of the MI355X (gfx950) decode-time MoE library
 * (libwarp_route_hip.so).
 *
 * This is the drop-in boundary beneath the PyTorch extension `warp_route._C`.
 * Every entry point takes plain pointers and sizes; there are no C++ or torch
 * types in the signatures, no exceptions, and no process exit.  Every
 * argument is validated before any HIP call, so argument errors are
 * reported as status codes even on a machine without a GPU.
 *
 * Semantics shared by all MoE entry points (reference citations are into
 * anishesg/warp-route):
 *   logits[e] = sum_i gate_w[e, i] * x[i]                (src/fused_moe.cu:100-112)
 *   p         = softmax(logits) over all E experts       (src/naive_moe.cu:156-162)
 *   ids       = k rounds of argmax over unused experts, strict '>', so ties go
 *               to the lower expert index                (src/naive_moe.cu:164-174)
 *   w[kk]     = p[ids[kk]], divided by sum_kk p[ids[kk]] when renormalize != 0
 *               (the reference never renormalises; renormalize = 0 is its
 *               behaviour)
 *   out       = sum_kk w[kk] * Wd_e (silu(Wg_e x) * (Wu_e x)),  e = ids[kk]
 *                                                        (src/fused_moe.cu:167-224)
 * Gating and accumulation are fp32.  Expert weights are fp32, fp16, bf16, fp8
 * (e4m3) or MXFP4 (e2m1 codes, two per byte, with an e8m0 scale per 32
 * elements of a row) in the packed expert layout (src/expert_layout.cuh:5-18):
 * per expert [gate I x h][up I x h][down h x I], row-major, expert stride
 * rounded up to 128 bytes.  fp8 blocks also hold fp32 row scales, MXFP4
 * blocks their scale bytes after the codes (wr_layout_dtype).
 *
 * Streams: work is enqueued asynchronously on `stream` (a hipStream_t passed
 * as void*, NULL = the null stream).  The reference launched on the legacy
 * default stream and called cudaDeviceSynchronize (src/bindings.cpp:54-55,
 * 93-94, 137-140); this library never synchronises the device.  The naive
 * entry point synchronises `stream` once, for its host-side top-K, as the
 * reference does (src/naive_moe.cu:197-199).
 */
#ifndef WARP_ROUTE_H
#define WARP_ROUTE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define WR_API __attribute__((visibility("default")))
#else
#define WR_API
#endif

/* Router limits: src/gate.cuh:5 (GATE_MAX_EXPERTS) and src/gate.cuh:7
 * (GATE_MAX_TOPK).  The reference's fused and batched launchers accept only
 * top_k in {1, 2} (src/fused_moe.cu:239-242, src/fused_moe_batched.cu:192-195);
 * here every entry point accepts 1 <= top_k <= min(WR_MAX_TOPK, num_experts). */
#define WR_MAX_EXPERTS 64
#define WR_MAX_TOPK 6
/* Expert stride alignment in bytes: src/expert_layout.cuh:43-45. */
#define WR_EXPERT_ALIGN 128
/* Bytes of device scratch wr_fused_moe_noalloc holds per GPU (1 MiB): enough
 * for wr_workspace_bytes(WR_KIND_FUSED, ...) up to k * roundup(I, 16) =
 * 253,248 (Mixtral needs 28,672, DBRX 43,008, DeepSeek 8,448). */
#define WR_NOALLOC_SCRATCH_BYTES (1u << 20)

typedef enum wr_status {
  WR_OK = 0,
  WR_EINVAL_NULL = 1,         /* a required pointer is NULL                    */
  WR_EINVAL_SHAPE = 2,        /* num_experts, hidden_dim or intermediate_dim < 1 */
  WR_EINVAL_TOPK = 3,         /* top_k outside [1, min(WR_MAX_TOPK, E)]        */
  WR_EINVAL_EXPERTS = 4,      /* num_experts > WR_MAX_EXPERTS                  */
  WR_EINVAL_DTYPE = 5,        /* unknown weight or activation dtype tag        */
  WR_EINVAL_WEIGHT_SIZE = 6,  /* weight_bytes < total packed layout bytes      */
  WR_EINVAL_WORKSPACE = 7,    /* workspace NULL or smaller than required       */
  WR_EINVAL_BATCH = 8,        /* batch_size < 0, or != 1 for a single-token op */
  WR_EINVAL_KIND = 9,         /* unknown wr_kind                               */
  WR_EINVAL_BLOCK = 10,       /* MXFP4 weights need h and I multiples of 32    */
  WR_ETIMEOUT = 11,           /* a single-token hand-off wait expired: the rows
                                 of the blocks that gave up are NaN            */
  WR_EINVAL_SCRATCH = 12,     /* the problem needs more workspace than the
                                 allocation-free entry point's fixed scratch
                                 (WR_NOALLOC_SCRATCH_BYTES)                   */
  WR_EHIP = 100               /* a HIP runtime call failed                     */
} wr_status;

/* Element type tags.  Expert weights may use any of them; x and out are
 * WR_F32 or WR_F16.  WR_BF16 is bfloat16 (the top 16 bits of an fp32).
 * WR_FP8_E4M3 is the OCP 8-bit float E4M3: sign, 4 exponent bits (bias 7),
 * 3 mantissa bits, subnormals, no infinities, NaN = S.1111.111, largest
 * finite value 448.  WR_MXFP4 is OCP Microscaling FP4: E2M1 elements (sign,
 * 2 exponent bits with bias 1, 1 mantissa bit: 0, 0.5, 1, 1.5, 2, 3, 4, 6),
 * two per byte (element 2i in bits 0-3), with one E8M0 scale 2^(s - 127) per
 * 32 consecutive elements of a row.  The reference stores fp32 only. */
typedef enum wr_dtype {
  WR_F32 = 0,
  WR_F16 = 1,
  WR_BF16 = 2,
  WR_FP8_E4M3 = 3,
  WR_MXFP4 = 4
} wr_dtype;

/* Which entry point a workspace is sized for. */
typedef enum wr_kind { WR_KIND_FUSED = 0, WR_KIND_BATCHED = 1, WR_KIND_NAIVE = 2 } wr_kind;

/* Byte offsets within one expert block.  Replaces `ExpertOffsets`
 * (src/expert_layout.cuh:27-32). */
typedef struct wr_offsets {
  int64_t gate_proj_offset;
  int64_t up_proj_offset;
  int64_t down_proj_offset;
  int64_t expert_stride;
} wr_offsets;

/* Arguments of one MoE call.  Replaces `FusedMoEParams`
 * (src/fused_moe.cuh:17-22), `BatchedFusedMoEParams`
 * (src/fused_moe_batched.cuh:18-24) and `NaiveMoEParams`
 * (src/naive_moe.cuh:17-22) plus their d_hidden/d_output arguments.  All
 * pointers are device pointers. */
typedef struct wr_moe_args {
  const float *gate_w;     /* [E, h] fp32 router, row-major                      */
  const void *weight_buf;  /* packed experts, element type weight_dtype          */
  int64_t weight_bytes;    /* bytes readable at weight_buf, >= wr_weight_bytes() */
  int32_t weight_dtype;    /* wr_dtype                                           */
  int32_t num_experts;     /* E                                                  */
  int32_t hidden_dim;      /* h                                                  */
  int32_t intermediate_dim;/* I                                                  */
  int32_t top_k;           /* k                                                  */
  int32_t renormalize;     /* 0: weights are the softmax probabilities (reference) */
  int32_t batch_size;      /* B tokens in x and out (1 for fused and naive)      */
  int32_t act_dtype;       /* wr_dtype of x and out                              */
  const void *x;           /* [B, h]                                             */
  void *out;               /* [B, h], fully overwritten                          */
  int32_t *topk_ids;       /* optional [B, k]: selected experts, descending weight */
  float *topk_weights;     /* optional [B, k]: their gate weights                */
  void *workspace;         /* device scratch, >= wr_workspace_bytes(...) bytes   */
  size_t workspace_bytes;
} wr_moe_args;

/* Expert block layout for a weight dtype.  For WR_F32, WR_F16 and WR_BF16
 * the offsets are those of wr_layout with elem_bytes 4, 2, 2 and
 * scale_offset is -1.  For WR_MXFP4 (h and I multiples of 32) the codes take
 * half a byte per element: gate [I][h/2] bytes at 0, up at I h / 2, down
 * [h][I/2] at I h; then at scale_offset = 3 I h / 2 rounded up to 16 bytes
 * the E8M0 block scales, one byte per 32 elements of a row: gate [I][h/32],
 * up [I][h/32], down [h][I/32]; expert_stride = scale_offset + 3 I h / 32
 * rounded up to 128 bytes; elem_bytes is 0 (half a byte).  For WR_FP8_E4M3 the three matrices hold 1-byte codes
 * q at the same element offsets (gate 0, up I h, down 2 I h), followed at
 * scale_offset = 3 I h rounded up to 16 bytes by one fp32 scale per output
 * row: s_gate[I], s_up[I], then s_down[h], with
 *   gate[r][c] = fp8(q_gate[r][c]) * s_gate[r]
 *   up[r][c]   = fp8(q_up[r][c])   * s_up[r]
 *   down[r][c] = fp8(q_down[r][c]) * s_down[r]
 * and expert_stride = scale_offset + 4 (2 I + h) rounded up to 128 bytes.
 * Kernels apply a row's scale to its dot product.  Has no counterpart in the
 * reference, whose layout is fp32 only. */
typedef struct wr_layout_info {
  int64_t gate_proj_offset;
  int64_t up_proj_offset;
  int64_t down_proj_offset;
  int64_t scale_offset;   /* -1: no scales                                  */
  int64_t expert_stride;
  int32_t elem_bytes;     /* bytes per matrix element: 4, 2 or 1; 0 for MXFP4 */
  int32_t weight_dtype;   /* wr_dtype                                       */
} wr_layout_info;

/* Options of the single-token fused kernel's hand-off between its gate/up
 * and down blocks (see wr_fused_moe_opts).  Zero-initialise for the
 * defaults. */
typedef struct wr_fused_opts {
  uint32_t spin_limit;  /* polls before a down block's wait expires; 0 = the
                           default (2^20 polls, about 0.2 s)                  */
  uint32_t wait_extra;  /* added to every arrival target.  0 in normal use; a
                           nonzero value makes every wait expire after
                           spin_limit polls, so that tests can exercise the
                           expiry path while every kernel still exits normally */
  uint32_t gu_blocks;   /* gate/up blocks to launch, rounded down to a multiple
                           of 32; 0 = the default (as many as the GPU holds at
                           once, the remaining gate/up chunks taken by the
                           blocks that finish first).  Fewer blocks than the
                           layer's chunks exercise that path at small shapes
                           (tests)                                            */
} wr_fused_opts;

/* Human-readable name of a status code (never NULL). */
WR_API const char *wr_status_str(int status);

/* Expert block offsets for element size elem_bytes (4 = fp32, 2 = fp16).
 * Replaces compute_offsets (src/expert_layout.cuh:34-47), which fixed the
 * element size at sizeof(float). */
WR_API int wr_layout(int num_experts, int hidden_dim, int intermediate_dim,
                     int elem_bytes, wr_offsets *out);

/* Total packed bytes of all experts, or -1 for invalid arguments.
 * Replaces total_weight_bytes (src/expert_layout.cuh:74-77). */
WR_API int64_t wr_total_weight_bytes(int num_experts, int hidden_dim,
                                     int intermediate_dim, int elem_bytes);

/* Layout of one expert block of weight_dtype (see wr_layout_info).  Extends
 * compute_offsets (src/expert_layout.cuh:34-47) to the reduced-precision
 * weight types. */
WR_API int wr_layout_dtype(int num_experts, int hidden_dim, int intermediate_dim,
                           int weight_dtype, wr_layout_info *out);

/* Total packed bytes of all experts for weight_dtype, or -1 for invalid
 * arguments.  Extends total_weight_bytes (src/expert_layout.cuh:74-77). */
WR_API int64_t wr_weight_bytes(int num_experts, int hidden_dim, int intermediate_dim,
                               int weight_dtype);

/* Device workspace an entry point of `kind` needs, or 0 for invalid
 * arguments.  The reference allocated naive scratch with cudaMalloc on every
 * call (src/bindings.cpp:53-56, src/naive_moe.cu:24-42); here the caller
 * provides it (the torch extension takes it from the caching allocator). */
WR_API size_t wr_workspace_bytes(int kind, int num_experts, int hidden_dim,
                                 int intermediate_dim, int top_k, int batch_size);

/* Router logits, softmax and top-K for B tokens; writes args->topk_ids and
 * args->topk_weights (both required here) and nothing else.  The device gate
 * shared by the fused and batched entry points.  Replaces warp_gate_topk
 * (src/gate.cu:103-116, declared at src/gate.cuh:21-27). */
WR_API int wr_gate_topk(const wr_moe_args *args, void *stream);

/* Single-token fused MoE (batch_size must be 1): one kernel for the
 * selection and the whole expert FFN, which also computes the router rows
 * for layers of at least 2 gate/up block slots per CU on its register path
 * (one launch per layer), else a router launch ahead of it.  The workspace needs no
 * initialisation (each call resets the control words it uses) and may be
 * reused by later calls on the same stream.  Replaces fused_moe_forward
 * (src/fused_moe.cu:233-263, declared at src/fused_moe.cuh:29-32). */
WR_API int wr_fused_moe(const wr_moe_args *args, void *stream);

/* wr_fused_moe with explicit hand-off options (opts may be NULL: defaults).
 * On expiry of a down block's bounded wait, that block writes NaN to its
 * output rows and sets the workspace's timeout word, which
 * wr_fused_moe_status reports.  The reference has no such wait: its fused
 * kernel is one warp (src/fused_moe.cu:76-227) and its error paths call
 * exit(1) (src/fused_moe.cu:9-15). */
WR_API int wr_fused_moe_opts(const wr_moe_args *args, const wr_fused_opts *opts, void *stream);

/* Status of the last single-token fused call that used `workspace` (size
 * workspace_bytes, at least wr_workspace_bytes(WR_KIND_FUSED, ...)): WR_OK, or
 * WR_ETIMEOUT if a hand-off wait expired (the output then holds NaN rows).
 * Reads the timeout word with a copy on `stream` and synchronises `stream`;
 * call it after the op and before the next single-token call on the same
 * workspace, which clears the word.  Has no counterpart in the
 * reference, whose fused kernel exits the process on error
 * (src/fused_moe.cu:9-15). */
WR_API int wr_fused_moe_status(const void *workspace, size_t workspace_bytes, void *stream);

/* Whether a single-token call's hand-off wait has expired since the last
 * call with clear != 0: 1 or 0.  A down block whose wait expires also stores
 * 1 to a host-visible word of the library (4 bytes of pinned host memory,
 * allocated by the first wr_fused_moe, wr_fused_moe_opts or wr_fused_moe_ffn
 * call, or wr_batched_fused_moe call with one token (which runs the same
 * kernel), made outside stream capture, held until the process ends;
 * wr_fused_moe_noalloc writes it once it exists).  This reads that word with
 * a host load: no HIP call, no synchronisation, so it may be called after
 * every op, also under graph capture.  An expiry is seen once its kernel has
 * run, so a check right after a call reports the expiries of calls that have
 * finished by then (an asynchronous report, like a device error).  With
 * clear != 0 a set word is cleared.  No counterpart in the reference, whose
 * fused kernel exits the process on error (src/fused_moe.cu:9-15). */
WR_API int wr_fused_moe_expired(int clear);

/* The two launches of wr_fused_moe, for callers that issue them separately
 * (to overlap the router with other work on the stream's timeline, or to time
 * the expert FFN alone).  wr_fused_moe_route computes the router logits into
 * the workspace and resets its control words; wr_fused_moe_ffn selects the
 * experts from those logits and runs the FFN.  Both take the arguments of
 * wr_fused_moe and validate them the same way.  Call them in this order, on
 * one stream, with one workspace and nothing else using that workspace in
 * between; together they do exactly what wr_fused_moe does.  The reference
 * has no split (fused_moe_forward, src/fused_moe.cu:233-263, computes the
 * router inside its one kernel). */
WR_API int wr_fused_moe_route(const wr_moe_args *args, void *stream);
WR_API int wr_fused_moe_ffn(const wr_moe_args *args, void *stream);

/* wr_fused_moe without a caller workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * args->workspace and args->workspace_bytes are ignored: the call uses a
 * fixed WR_NOALLOC_SCRATCH_BYTES device array of the library, one per GPU,
 * held until the process ends.  It allocates nothing (no hipMalloc, no
 * hipFree, no allocating library call); the first call on a GPU looks up
 * that GPU's array address once.  Returns WR_EINVAL_SCRATCH (before any HIP
 * call) when wr_workspace_bytes(WR_KIND_FUSED, E, h, I, k, 1) exceeds
 * WR_NOALLOC_SCRATCH_BYTES.  Every call on one GPU shares its array, and the
 * array keeps the last call's contents (each call clears the control words
 * it needs), so calls that overlap on one GPU -- on different streams, or
 * from different threads -- race and must be serialised by the caller.  The
 * call may be recorded into a HIP graph once a first call on the GPU has
 * looked up the array.  A hand-off expiry shows as NaN
 * output rows, and through wr_fused_moe_expired once another single-token
 * call has allocated its word: the timeout word lives in the library's
 * array, which wr_fused_moe_status cannot be given.  Otherwise identical to wr_fused_moe,
 * with the same kernels and results. */
WR_API int wr_fused_moe_noalloc(const wr_moe_args *args, void *stream);

/* B-token fused MoE (batch_size >= 0; 0 is a no-op as in
 * src/fused_moe_batched.cu:201).  Tokens that share an expert share its weight
 * reads.  Replaces batched_fused_moe_forward (src/fused_moe_batched.cu:186-214,
 * declared at src/fused_moe_batched.cuh:30-33). */
WR_API int wr_batched_fused_moe(const wr_moe_args *args, void *stream);

/* Single-token multi-kernel baseline with host softmax/top-K (batch_size must
 * be 1).  Synchronises `stream` once.  Replaces naive_moe_forward
 * (src/naive_moe.cu:181-241, declared at src/naive_moe.cuh:40-44). */
WR_API int wr_naive_moe(const wr_moe_args *args, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* WARP_ROUTE_H */
