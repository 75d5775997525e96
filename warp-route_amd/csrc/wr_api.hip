// extern "C" boundary of libwarp_route_hip.so (declared in include/warp_route.h).
//
// Every entry point validates all arguments before the first HIP call and
// reports problems as wr_status codes; nothing here exits the process (the
// reference printed and called exit(1), src/fused_moe.cu:9-15, 239-247).
// The argument checks mirror the reference's TORCH_CHECKs
// (src/bindings.cpp:9-23, 35-43, 71-83, 110-125).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>

#include "warp_route.h"
#include "wr_internal.h"

namespace {

using wr::Problem;

int64_t stride_bytes(int64_t E, int64_t h, int64_t I, int64_t es, int64_t* up, int64_t* down) {
  (void)E;
  const int64_t gateup = I * h, dn = h * I;
  const int64_t up_off = gateup * es;
  const int64_t down_off = up_off + gateup * es;
  const int64_t raw = down_off + dn * es;
  if (up) *up = up_off;
  if (down) *down = down_off;
  return (raw + WR_EXPERT_ALIGN - 1) / WR_EXPERT_ALIGN * WR_EXPERT_ALIGN;
}

int check_dims(int E, int h, int I, int k) {
  if (E < 1 || h < 1 || I < 1) return WR_EINVAL_SHAPE;
  if (E > WR_MAX_EXPERTS) return WR_EINVAL_EXPERTS;
  if (k < 1 || k > WR_MAX_TOPK || k > E) return WR_EINVAL_TOPK;
  return WR_OK;
}

bool act_dtype_ok(int d) { return d == WR_F32 || d == WR_F16; }

bool weight_dtype_ok(int d) { return d >= WR_F32 && d <= WR_MXFP4; }

// Bytes per matrix element of a weight dtype (0 for MXFP4: half a byte).
int weight_es(int d) {
  switch (d) {
    case WR_F32: return 4;
    case WR_F16: return 2;
    case WR_BF16: return 2;
    case WR_FP8_E4M3: return 1;
    default: return 0;
  }
}

// Expert block layout of a weight dtype (arguments already checked).
wr_layout_info layout_of(int64_t E, int64_t h, int64_t I, int wdt) {
  wr_layout_info o;
  o.weight_dtype = wdt;
  o.elem_bytes = weight_es(wdt);
  o.gate_proj_offset = 0;
  o.scale_offset = -1;
  if (wdt == WR_MXFP4) {
    o.up_proj_offset = I * h / 2;
    o.down_proj_offset = I * h;
    o.scale_offset = (3 * I * h / 2 + 15) / 16 * 16;
    const int64_t raw = o.scale_offset + 3 * I * h / 32;
    o.expert_stride = (raw + WR_EXPERT_ALIGN - 1) / WR_EXPERT_ALIGN * WR_EXPERT_ALIGN;
    return o;
  }
  if (wdt != WR_FP8_E4M3) {
    o.expert_stride = stride_bytes(E, h, I, o.elem_bytes, &o.up_proj_offset, &o.down_proj_offset);
    return o;
  }
  o.up_proj_offset = I * h;
  o.down_proj_offset = 2 * I * h;
  o.scale_offset = (3 * I * h + 15) / 16 * 16;
  const int64_t raw = o.scale_offset + (2 * I + h) * 4;
  o.expert_stride = (raw + WR_EXPERT_ALIGN - 1) / WR_EXPERT_ALIGN * WR_EXPERT_ALIGN;
  return o;
}

size_t ws_bytes(int kind, int E, int h, int I, int k, int B) {
  switch (kind) {
    case WR_KIND_FUSED:
      return wr::FusedWs::bytes(E, I, k, 1);
    case WR_KIND_BATCHED:
      // B > 1 runs either the grouped MFMA path or the per-token kernels,
      // depending on dtype and alignment: size for both.
      return B > 1 ? std::max(wr::FusedWs::bytes(E, I, k, B), wr::BatchWs::bytes(E, h, I, k, B))
                   : wr::FusedWs::bytes(E, I, k, 1);
    case WR_KIND_NAIVE:
      return wr::NaiveWs::bytes(E, h, I);
    default:
      return 0;
  }
}

// Elements per lane per weight access.  The 128-bit path needs every row and
// every expert block 16-byte aligned (h and I multiples of the vector width,
// 16-byte aligned weight and activation pointers); anything else takes the
// scalar path.
int choose_vec(const wr_moe_args* a) {
  if (a->weight_dtype == WR_MXFP4) {  // h, I multiples of 32: 32 elements per 16 bytes, else 2
    const bool al = reinterpret_cast<uintptr_t>(a->weight_buf) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(a->x) % 16 == 0;
    return al ? 32 : 2;
  }
  const int v = 16 / weight_es(a->weight_dtype);
  if (a->hidden_dim % v != 0 || a->intermediate_dim % v != 0) return 1;
  if (reinterpret_cast<uintptr_t>(a->weight_buf) % 16 != 0) return 1;
  if (reinterpret_cast<uintptr_t>(a->x) % 16 != 0) return 1;
  return v;
}

// kind: WR_KIND_* or -1 for the gate-only entry point.
int validate(const wr_moe_args* a, int kind, Problem* p) {
  if (a == nullptr) return WR_EINVAL_NULL;
  int st = check_dims(a->num_experts, a->hidden_dim, a->intermediate_dim, a->top_k);
  if (st != WR_OK) return st;
  if (!weight_dtype_ok(a->weight_dtype) || !act_dtype_ok(a->act_dtype)) return WR_EINVAL_DTYPE;
  if (a->weight_dtype == WR_MXFP4 && kind >= 0 &&
      (a->hidden_dim % 32 != 0 || a->intermediate_dim % 32 != 0))
    return WR_EINVAL_BLOCK;
  const bool single = kind == WR_KIND_FUSED || kind == WR_KIND_NAIVE;
  if (single ? a->batch_size != 1 : a->batch_size < 0) return WR_EINVAL_BATCH;
  if (a->batch_size == 0) {
    p->B = 0;
    return WR_OK;
  }
  if (a->gate_w == nullptr || a->x == nullptr) return WR_EINVAL_NULL;
  if (kind < 0) {
    if (a->topk_ids == nullptr || a->topk_weights == nullptr) return WR_EINVAL_NULL;
  } else {
    if (a->weight_buf == nullptr || a->out == nullptr) return WR_EINVAL_NULL;
    const wr_layout_info lo =
        layout_of(a->num_experts, a->hidden_dim, a->intermediate_dim, a->weight_dtype);
    if (a->weight_bytes < lo.expert_stride * a->num_experts) return WR_EINVAL_WEIGHT_SIZE;
    const size_t need = ws_bytes(kind, a->num_experts, a->hidden_dim, a->intermediate_dim,
                                 a->top_k, a->batch_size);
    if (a->workspace == nullptr || a->workspace_bytes < need) return WR_EINVAL_WORKSPACE;
    p->stride_b = lo.expert_stride;
    p->off_up_b = lo.up_proj_offset;
    p->off_down_b = lo.down_proj_offset;
    p->off_scale_b = lo.scale_offset;
  }
  p->gate_w = a->gate_w;
  p->wbuf = a->weight_buf;
  p->wdt = a->weight_dtype;
  p->adt = a->act_dtype;
  p->E = a->num_experts;
  p->h = a->hidden_dim;
  p->I = a->intermediate_dim;
  p->k = a->top_k;
  p->renorm = a->renormalize ? 1 : 0;
  p->B = a->batch_size;
  p->x = a->x;
  p->out = a->out;
  p->topk_ids = a->topk_ids;
  p->topk_w = a->topk_weights;
  p->ws = static_cast<char*>(a->workspace);
  p->ws_bytes = a->workspace_bytes;
  p->vec = kind < 0 ? 1 : choose_vec(a);
  p->spin_limit = wr::kDefaultSpinLimit;
  p->wait_extra = 0;
  p->gu_blocks = 0;
  return WR_OK;
}

int hip_status(hipError_t e) { return e == hipSuccess ? WR_OK : WR_EHIP; }

// The allocation-free entry point's workspace: one array per GPU (a
// __device__ variable exists once on every device the code object is loaded
// on), held until the process ends.  In host code `scratch` names a host-side
// stand-in, not device memory: its device address on the current GPU comes
// from hipGetSymbolAddress, looked up once per device and kept in
// g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[WR_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Device address of the current GPU's scratch array, or nullptr on a HIP
// error.  The first call on a device, with that device current, looks it up.
void* scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

// The host-visible expiry word of every single-token call: 4 bytes of
// pinned, coherent host memory mapped for every GPU, allocated once by the
// first call that takes a caller workspace outside stream capture, and held
// until the process ends.  A kernel whose hand-off wait expires stores 1 to
// it; wr_fused_moe_expired reads it with a host load.
std::once_flag g_expired_once;
std::atomic<unsigned*> g_expired{nullptr};

// The word's device address; allocates it when `alloc` (and the stream is
// not being captured).  nullptr: not available (the call then does not
// write it; its timeout word still records an expiry).
unsigned* expired_word(bool alloc, hipStream_t s) {
  unsigned* w = g_expired.load(std::memory_order_acquire);
  if (w != nullptr || !alloc) return w;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
    return nullptr;
  std::call_once(g_expired_once, [] {
    void* h = nullptr;
    if (hipHostMalloc(&h, sizeof(unsigned),
                      hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) !=
            hipSuccess ||
        h == nullptr) {
      (void)hipGetLastError();
      return;
    }
    *static_cast<volatile unsigned*>(h) = 0u;
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || d != h) {
      // Only a word whose host and device addresses agree is used, so that
      // the host reads what the kernels write.
      (void)hipGetLastError();
      return;
    }
    g_expired.store(static_cast<unsigned*>(h), std::memory_order_release);
  });
  return g_expired.load(std::memory_order_acquire);
}

}  // namespace

extern "C" {

WR_API const char* wr_status_str(int status) {
  switch (status) {
    case WR_OK: return "ok";
    case WR_EINVAL_NULL: return "a required pointer is NULL";
    case WR_EINVAL_SHAPE: return "num_experts, hidden_dim and intermediate_dim must be >= 1";
    case WR_EINVAL_TOPK: return "top_k must be in [1, min(6, num_experts)]";
    case WR_EINVAL_EXPERTS: return "num_experts exceeds WR_MAX_EXPERTS (64)";
    case WR_EINVAL_DTYPE:
      return "unsupported dtype (weights: fp32, fp16, bf16, fp8 e4m3 or mxfp4; activations: fp32 or "
             "fp16)";
    case WR_EINVAL_WEIGHT_SIZE: return "weight_buf is smaller than the packed expert layout";
    case WR_EINVAL_WORKSPACE: return "workspace is NULL or smaller than wr_workspace_bytes()";
    case WR_EINVAL_BATCH: return "invalid batch_size";
    case WR_EINVAL_KIND: return "unknown workspace kind";
    case WR_EINVAL_BLOCK:
      return "MXFP4 weights need hidden_dim and intermediate_dim to be multiples of 32";
    case WR_ETIMEOUT:
      return "a fused-kernel hand-off wait expired (the affected output rows are NaN)";
    case WR_EINVAL_SCRATCH:
      return "problem needs more workspace than the allocation-free entry point's 1 MiB scratch";
    case WR_EHIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

WR_API int wr_layout(int num_experts, int hidden_dim, int intermediate_dim, int elem_bytes,
                     wr_offsets* out) {
  if (out == nullptr) return WR_EINVAL_NULL;
  if (num_experts < 1 || hidden_dim < 1 || intermediate_dim < 1) return WR_EINVAL_SHAPE;
  if (elem_bytes != 2 && elem_bytes != 4) return WR_EINVAL_DTYPE;
  int64_t up = 0, down = 0;
  out->expert_stride = stride_bytes(num_experts, hidden_dim, intermediate_dim, elem_bytes, &up, &down);
  out->gate_proj_offset = 0;
  out->up_proj_offset = up;
  out->down_proj_offset = down;
  return WR_OK;
}

WR_API int64_t wr_total_weight_bytes(int num_experts, int hidden_dim, int intermediate_dim,
                                     int elem_bytes) {
  wr_offsets o;
  if (wr_layout(num_experts, hidden_dim, intermediate_dim, elem_bytes, &o) != WR_OK) return -1;
  return (int64_t)num_experts * o.expert_stride;
}

WR_API int wr_layout_dtype(int num_experts, int hidden_dim, int intermediate_dim,
                           int weight_dtype, wr_layout_info* out) {
  if (out == nullptr) return WR_EINVAL_NULL;
  if (num_experts < 1 || hidden_dim < 1 || intermediate_dim < 1) return WR_EINVAL_SHAPE;
  if (!weight_dtype_ok(weight_dtype)) return WR_EINVAL_DTYPE;
  if (weight_dtype == WR_MXFP4 && (hidden_dim % 32 != 0 || intermediate_dim % 32 != 0))
    return WR_EINVAL_BLOCK;
  *out = layout_of(num_experts, hidden_dim, intermediate_dim, weight_dtype);
  return WR_OK;
}

WR_API int64_t wr_weight_bytes(int num_experts, int hidden_dim, int intermediate_dim,
                               int weight_dtype) {
  wr_layout_info o;
  if (wr_layout_dtype(num_experts, hidden_dim, intermediate_dim, weight_dtype, &o) != WR_OK)
    return -1;
  return (int64_t)num_experts * o.expert_stride;
}

WR_API size_t wr_workspace_bytes(int kind, int num_experts, int hidden_dim, int intermediate_dim,
                                 int top_k, int batch_size) {
  if (check_dims(num_experts, hidden_dim, intermediate_dim, top_k) != WR_OK) return 0;
  if (batch_size < 0) return 0;
  return ws_bytes(kind, num_experts, hidden_dim, intermediate_dim, top_k, batch_size);
}

WR_API int wr_gate_topk(const wr_moe_args* args, void* stream) {
  Problem p{};
  const int st = validate(args, -1, &p);
  if (st != WR_OK || p.B == 0) return st;
  return hip_status(wr::launch_gate_topk(p, static_cast<hipStream_t>(stream)));
}

WR_API int wr_fused_moe(const wr_moe_args* args, void* stream) {
  Problem p{};
  const int st = validate(args, WR_KIND_FUSED, &p);
  if (st != WR_OK) return st;
  p.expired_host = expired_word(true, static_cast<hipStream_t>(stream));
  return hip_status(wr::launch_fused(p, static_cast<hipStream_t>(stream)));
}

WR_API int wr_fused_moe_opts(const wr_moe_args* args, const wr_fused_opts* opts, void* stream) {
  Problem p{};
  const int st = validate(args, WR_KIND_FUSED, &p);
  if (st != WR_OK) return st;
  if (opts != nullptr) {
    if (opts->spin_limit != 0) p.spin_limit = opts->spin_limit;
    p.wait_extra = opts->wait_extra;
    p.gu_blocks = (int)(opts->gu_blocks & 0x7fffffe0u);  // a multiple of 32, or 0
  }
  p.expired_host = expired_word(true, static_cast<hipStream_t>(stream));
  return hip_status(wr::launch_fused(p, static_cast<hipStream_t>(stream)));
}

WR_API int wr_fused_moe_noalloc(const wr_moe_args* args, void* stream) {
  if (args == nullptr) return WR_EINVAL_NULL;
  // Validate against the fixed scratch size first (no HIP call yet): any
  // workspace complaint is then the problem being too large for it.
  wr_moe_args a = *args;
  a.workspace = reinterpret_cast<void*>(uintptr_t{256});  // placeholder, never used
  a.workspace_bytes = WR_NOALLOC_SCRATCH_BYTES;
  Problem p{};
  const int st = validate(&a, WR_KIND_FUSED, &p);
  if (st == WR_EINVAL_WORKSPACE) return WR_EINVAL_SCRATCH;
  if (st != WR_OK) return st;
  void* ws = scratch_ptr();
  if (ws == nullptr) return WR_EHIP;
  p.ws = static_cast<char*>(ws);
  p.ws_bytes = WR_NOALLOC_SCRATCH_BYTES;
  p.expired_host = expired_word(false, nullptr);  // written once an earlier call made it
  return hip_status(wr::launch_fused(p, static_cast<hipStream_t>(stream)));
}

WR_API int wr_fused_moe_status(const void* workspace, size_t workspace_bytes, void* stream) {
  if (workspace == nullptr) return WR_EINVAL_NULL;
  if (workspace_bytes < wr::FusedWs::kCtrlBytes) return WR_EINVAL_WORKSPACE;
  const unsigned* word = static_cast<const unsigned*>(workspace) + wr::FusedWs::kTimeoutWord;
  unsigned v = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(&v, word, sizeof(v), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return WR_EHIP;
  return v != 0 ? WR_ETIMEOUT : WR_OK;
}

WR_API int wr_fused_moe_expired(int clear) {
  unsigned* w = g_expired.load(std::memory_order_acquire);
  if (w == nullptr) return 0;
  // Clearing swaps in 0, so that an expiry stored between a read and a
  // separate clear could not be lost.
  const unsigned v = clear != 0 ? __atomic_exchange_n(w, 0u, __ATOMIC_ACQ_REL)
                                : __atomic_load_n(w, __ATOMIC_ACQUIRE);
  return v != 0 ? 1 : 0;
}

WR_API int wr_fused_moe_route(const wr_moe_args* args, void* stream) {
  Problem p{};
  const int st = validate(args, WR_KIND_FUSED, &p);
  if (st != WR_OK) return st;
  return hip_status(wr::launch_fused_route(p, static_cast<hipStream_t>(stream)));
}

WR_API int wr_fused_moe_ffn(const wr_moe_args* args, void* stream) {
  Problem p{};
  const int st = validate(args, WR_KIND_FUSED, &p);
  if (st != WR_OK) return st;
  p.expired_host = expired_word(true, static_cast<hipStream_t>(stream));
  return hip_status(wr::launch_fused_ffn(p, static_cast<hipStream_t>(stream)));
}

WR_API int wr_batched_fused_moe(const wr_moe_args* args, void* stream) {
  Problem p{};
  const int st = validate(args, WR_KIND_BATCHED, &p);
  if (st != WR_OK || p.B == 0) return st;
  // One token runs the single-token kernel, whose hand-off expiry is reported
  // through the host-visible word.
  if (p.B == 1) p.expired_host = expired_word(true, static_cast<hipStream_t>(stream));
  return hip_status(wr::launch_batched(p, static_cast<hipStream_t>(stream)));
}

WR_API int wr_naive_moe(const wr_moe_args* args, void* stream) {
  Problem p{};
  const int st = validate(args, WR_KIND_NAIVE, &p);
  if (st != WR_OK) return st;
  return hip_status(wr::run_naive(p, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
