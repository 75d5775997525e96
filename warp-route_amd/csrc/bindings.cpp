// warp_route._C: the torch-op boundary (src/bindings.cpp:145-152 in the
// reference), implemented over the C-ABI of libwarp_route_hip.so.
//
// The three ops keep the reference's names and seven positional arguments
// (hidden, gate_w, weight_buf, num_experts, hidden_dim, intermediate_dim,
// top_k) and add trailing defaulted ones:
//   renormalize=False  divide the selected weights by their sum
//   topk_ids=None      optional int32 [k] / [B,k] output of selected experts
//   topk_weights=None  optional fp32 [k] / [B,k] output of their weights
// Differences from the reference, all compatible with its call forms:
//   * weight_buf may be float32 (the reference layout), float16, bfloat16,
//     float8_e4m3fn (codes plus fp32 row scales) or float4_e2m1fn_x2 (MXFP4
//     codes plus E8M0 block scales), laid out as wr_layout_dtype says; hidden
//     may be float32 or float16 and the output takes its dtype; gate_w is
//     float32.
//   * top_k may be 1..min(6, num_experts) on every op (the reference's fused
//     and batched ops accepted only 1 or 2, src/bindings.cpp:75,117).
//   * work is enqueued on the current HIP stream of hidden's device and the
//     device is not synchronised (the reference used stream 0 and
//     cudaDeviceSynchronize, src/bindings.cpp:54-55,93-94,137-140).
//   * scratch comes from the caching allocator; nothing calls hipMalloc per
//     call (the reference's naive op did, src/bindings.cpp:53-56).
// ROCm builds of torch report HIP tensors as device type "cuda"; the
// *MasqueradingAsCUDA guard and stream accessors accept that device type.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/extension.h>

#include <atomic>
#include <cstdlib>
#include <optional>

#include "warp_route.h"

namespace {

// When set, fused_moe_forward reads the hand-off status of its call
// (wr_fused_moe_status, which synchronises the stream) and raises if a wait
// expired.  Off by default: the check costs a stream synchronisation and
// cannot run under graph capture.  WARP_ROUTE_CHECK_HANDOFF=1 in the
// environment turns it on at import.
std::atomic<bool> g_check_handoff{[] {
  const char* v = std::getenv("WARP_ROUTE_CHECK_HANDOFF");
  return v != nullptr && v[0] != '\0' && v[0] != '0';
}()};

#define WR_CHECK_DEVICE(t) TORCH_CHECK((t).is_cuda(), #t " must be a CUDA (HIP) tensor")
#define WR_CHECK_CONTIGUOUS(t) TORCH_CHECK((t).is_contiguous(), #t " must be contiguous")

int dtype_tag(const torch::Tensor& t, const char* name) {
  if (t.scalar_type() == torch::kFloat32) return WR_F32;
  if (t.scalar_type() == torch::kFloat16) return WR_F16;
  TORCH_CHECK(false, name, " must be float32 or float16, got ", t.scalar_type());
  return -1;
}

int weight_dtype_tag(const torch::Tensor& t) {
  switch (t.scalar_type()) {
    case torch::kFloat32: return WR_F32;
    case torch::kFloat16: return WR_F16;
    case torch::kBFloat16: return WR_BF16;
    case torch::kFloat8_e4m3fn: return WR_FP8_E4M3;
    case torch::kFloat4_e2m1fn_x2: return WR_MXFP4;
    default:
      TORCH_CHECK(false,
                  "weight_buf must be float32, float16, bfloat16, float8_e4m3fn or "
                  "float4_e2m1fn_x2, got ",
                  t.scalar_type());
  }
  return -1;
}

void check_common(const torch::Tensor& gate_w, const torch::Tensor& weight_buf, int num_experts,
                  int hidden_dim, int intermediate_dim, int top_k,
                  const torch::Device& dev) {
  WR_CHECK_DEVICE(gate_w);
  WR_CHECK_CONTIGUOUS(gate_w);
  TORCH_CHECK(gate_w.scalar_type() == torch::kFloat32, "gate_w must be float32");
  TORCH_CHECK(gate_w.dim() == 2 && gate_w.size(0) == num_experts && gate_w.size(1) == hidden_dim,
              "gate_w must have shape [", num_experts, ", ", hidden_dim, "], got shape ",
              gate_w.sizes());
  WR_CHECK_DEVICE(weight_buf);
  WR_CHECK_CONTIGUOUS(weight_buf);
  const int wdt = weight_dtype_tag(weight_buf);
  TORCH_CHECK(gate_w.device() == dev && weight_buf.device() == dev,
              "hidden, gate_w and weight_buf must be on the same device");
  TORCH_CHECK(num_experts >= 1 && hidden_dim >= 1 && intermediate_dim >= 1,
              "num_experts, hidden_dim and intermediate_dim must be positive");
  TORCH_CHECK(num_experts <= WR_MAX_EXPERTS, "num_experts ", num_experts,
              " exceeds GATE_MAX_EXPERTS ", WR_MAX_EXPERTS);
  TORCH_CHECK(top_k >= 1 && top_k <= WR_MAX_TOPK && top_k <= num_experts,
              "top_k must be in [1, min(", WR_MAX_TOPK, ", num_experts)], got ", top_k);
  const int64_t es = weight_buf.element_size();
  TORCH_CHECK(wdt != WR_MXFP4 || (hidden_dim % 32 == 0 && intermediate_dim % 32 == 0),
              "MXFP4 weights need hidden_dim and intermediate_dim to be multiples of 32, got ",
              hidden_dim, " and ", intermediate_dim);
  const int64_t need = wr_weight_bytes(num_experts, hidden_dim, intermediate_dim, wdt);
  TORCH_CHECK(weight_buf.numel() * es >= need, "weight_buf too small: need ", need,
              " bytes, got ", weight_buf.numel() * es);
}

void check_topk_out(const std::optional<torch::Tensor>& t, c10::ScalarType st, int64_t n,
                    const torch::Device& dev, const char* name) {
  if (!t.has_value()) return;
  const torch::Tensor& v = *t;
  WR_CHECK_DEVICE(v);
  WR_CHECK_CONTIGUOUS(v);
  TORCH_CHECK(v.scalar_type() == st, name, " must be ", st);
  TORCH_CHECK(v.device() == dev, name, " must be on hidden's device");
  TORCH_CHECK(v.numel() == n, name, " must hold ", n, " elements, got ", v.numel());
}

wr_moe_args make_args(const torch::Tensor& hidden, const torch::Tensor& gate_w,
                      const torch::Tensor& weight_buf, int E, int h, int I, int k, bool renorm,
                      int B, torch::Tensor& out, const std::optional<torch::Tensor>& ids,
                      const std::optional<torch::Tensor>& ws_out) {
  wr_moe_args a{};
  a.gate_w = gate_w.data_ptr<float>();
  a.weight_buf = weight_buf.data_ptr();
  a.weight_bytes = weight_buf.numel() * (int64_t)weight_buf.element_size();
  a.weight_dtype = weight_dtype_tag(weight_buf);
  a.num_experts = E;
  a.hidden_dim = h;
  a.intermediate_dim = I;
  a.top_k = k;
  a.renormalize = renorm ? 1 : 0;
  a.batch_size = B;
  a.act_dtype = dtype_tag(hidden, "hidden");
  a.x = hidden.data_ptr();
  a.out = out.data_ptr();
  a.topk_ids = ids.has_value() ? ids->data_ptr<int32_t>() : nullptr;
  a.topk_weights = ws_out.has_value() ? ws_out->data_ptr<float>() : nullptr;
  return a;
}

torch::Tensor alloc_workspace(int kind, int E, int h, int I, int k, int B,
                              const torch::Device& dev) {
  const size_t n = wr_workspace_bytes(kind, E, h, I, k, B);
  TORCH_CHECK(n > 0, "invalid MoE shape for workspace sizing");
  return torch::empty({(int64_t)n}, torch::TensorOptions().dtype(torch::kUInt8).device(dev));
}

void check_status(int st, const char* op) {
  TORCH_CHECK(st == WR_OK, op, " failed: ", wr_status_str(st), " (status ", st, ")");
}

// Expiries of single-token hand-off waits, read from the library's
// host-visible word without a synchronisation: this reports the expiries of
// every single-token call whose kernel has run by now (this one or an
// earlier one), once each.
void check_expired(const char* op) {
  TORCH_CHECK(wr_fused_moe_expired(1) == 0, op,
              " failed: a single-token fused call's hand-off wait expired (that call's output "
              "rows are NaN); seen after its kernel ran, so it may have been an earlier call");
}

torch::Tensor single_token_op(int kind, torch::Tensor hidden, torch::Tensor gate_w,
                              torch::Tensor weight_buf, int num_experts, int hidden_dim,
                              int intermediate_dim, int top_k, bool renormalize,
                              std::optional<torch::Tensor> topk_ids,
                              std::optional<torch::Tensor> topk_weights) {
  WR_CHECK_DEVICE(hidden);
  WR_CHECK_CONTIGUOUS(hidden);
  dtype_tag(hidden, "hidden");
  TORCH_CHECK(hidden.dim() == 1 && hidden.size(0) == hidden_dim, "hidden must have shape [",
              hidden_dim, "], got shape ", hidden.sizes());
  const torch::Device dev = hidden.device();
  check_common(gate_w, weight_buf, num_experts, hidden_dim, intermediate_dim, top_k, dev);
  check_topk_out(topk_ids, torch::kInt32, top_k, dev, "topk_ids");
  check_topk_out(topk_weights, torch::kFloat32, top_k, dev, "topk_weights");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  torch::Tensor out = torch::empty_like(hidden);
  torch::Tensor ws = alloc_workspace(kind, num_experts, hidden_dim, intermediate_dim, top_k, 1, dev);
  wr_moe_args a = make_args(hidden, gate_w, weight_buf, num_experts, hidden_dim,
                            intermediate_dim, top_k, renormalize, 1, out, topk_ids, topk_weights);
  a.workspace = ws.data_ptr();
  a.workspace_bytes = (size_t)ws.numel();
  void* stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream();
  if (kind == WR_KIND_FUSED) {
    check_status(wr_fused_moe(&a, stream), "fused_moe_forward");
    if (g_check_handoff.load(std::memory_order_relaxed)) {
      const int st = wr_fused_moe_status(a.workspace, a.workspace_bytes, stream);
      if (st == WR_ETIMEOUT) (void)wr_fused_moe_expired(1);  // reported here, not again
      check_status(st, "fused_moe_forward");
    }
    check_expired("fused_moe_forward");
  } else
    check_status(wr_naive_moe(&a, stream), "naive_moe_forward");
  return out;
}

// fused_moe_forward(hidden, gate_w, weight_buf, num_experts, hidden_dim,
// intermediate_dim, top_k) -- src/bindings.cpp:62-97.
torch::Tensor fused_moe_forward(torch::Tensor hidden, torch::Tensor gate_w,
                                torch::Tensor weight_buf, int num_experts, int hidden_dim,
                                int intermediate_dim, int top_k, bool renormalize,
                                std::optional<torch::Tensor> topk_ids,
                                std::optional<torch::Tensor> topk_weights) {
  return single_token_op(WR_KIND_FUSED, hidden, gate_w, weight_buf, num_experts, hidden_dim,
                         intermediate_dim, top_k, renormalize, topk_ids, topk_weights);
}

// naive_moe_forward(...) -- src/bindings.cpp:26-59.
torch::Tensor naive_moe_forward(torch::Tensor hidden, torch::Tensor gate_w,
                                torch::Tensor weight_buf, int num_experts, int hidden_dim,
                                int intermediate_dim, int top_k, bool renormalize,
                                std::optional<torch::Tensor> topk_ids,
                                std::optional<torch::Tensor> topk_weights) {
  return single_token_op(WR_KIND_NAIVE, hidden, gate_w, weight_buf, num_experts, hidden_dim,
                         intermediate_dim, top_k, renormalize, topk_ids, topk_weights);
}

// batched_fused_moe_forward(hidden_batch [B,h], ...) -> [B,h] --
// src/bindings.cpp:101-143.
torch::Tensor batched_fused_moe_forward(torch::Tensor hidden_batch, torch::Tensor gate_w,
                                        torch::Tensor weight_buf, int num_experts, int hidden_dim,
                                        int intermediate_dim, int top_k, bool renormalize,
                                        std::optional<torch::Tensor> topk_ids,
                                        std::optional<torch::Tensor> topk_weights) {
  WR_CHECK_DEVICE(hidden_batch);
  WR_CHECK_CONTIGUOUS(hidden_batch);
  dtype_tag(hidden_batch, "hidden_batch");
  TORCH_CHECK(hidden_batch.dim() == 2 && hidden_batch.size(1) == hidden_dim,
              "hidden_batch must have shape [batch_size, ", hidden_dim, "], got shape ",
              hidden_batch.sizes());
  const torch::Device dev = hidden_batch.device();
  check_common(gate_w, weight_buf, num_experts, hidden_dim, intermediate_dim, top_k, dev);
  const int B = (int)hidden_batch.size(0);
  check_topk_out(topk_ids, torch::kInt32, (int64_t)B * top_k, dev, "topk_ids");
  check_topk_out(topk_weights, torch::kFloat32, (int64_t)B * top_k, dev, "topk_weights");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  torch::Tensor out = torch::empty_like(hidden_batch);
  if (B == 0) return out;
  torch::Tensor ws =
      alloc_workspace(WR_KIND_BATCHED, num_experts, hidden_dim, intermediate_dim, top_k, B, dev);
  wr_moe_args a = make_args(hidden_batch, gate_w, weight_buf, num_experts, hidden_dim,
                            intermediate_dim, top_k, renormalize, B, out, topk_ids, topk_weights);
  a.workspace = ws.data_ptr();
  a.workspace_bytes = (size_t)ws.numel();
  void* stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream();
  check_status(wr_batched_fused_moe(&a, stream), "batched_fused_moe_forward");
  check_expired("batched_fused_moe_forward");
  return out;
}

// gate_topk(hidden [h] or [B,h], gate_w, num_experts, hidden_dim, top_k,
// renormalize=False) -> (ids int32, weights fp32), shaped like hidden's batch
// dims + [k].  Router logits, softmax and top-K only (src/gate.cu:103-116).
std::tuple<torch::Tensor, torch::Tensor> gate_topk(torch::Tensor hidden, torch::Tensor gate_w,
                                                   int num_experts, int hidden_dim, int top_k,
                                                   bool renormalize) {
  WR_CHECK_DEVICE(hidden);
  WR_CHECK_CONTIGUOUS(hidden);
  dtype_tag(hidden, "hidden");
  TORCH_CHECK((hidden.dim() == 1 || hidden.dim() == 2) && hidden.size(-1) == hidden_dim,
              "hidden must have shape [", hidden_dim, "] or [batch_size, ", hidden_dim,
              "], got shape ", hidden.sizes());
  WR_CHECK_DEVICE(gate_w);
  WR_CHECK_CONTIGUOUS(gate_w);
  TORCH_CHECK(gate_w.scalar_type() == torch::kFloat32, "gate_w must be float32");
  TORCH_CHECK(gate_w.dim() == 2 && gate_w.size(0) == num_experts && gate_w.size(1) == hidden_dim,
              "gate_w must have shape [", num_experts, ", ", hidden_dim, "], got shape ",
              gate_w.sizes());
  TORCH_CHECK(gate_w.device() == hidden.device(), "hidden and gate_w must be on the same device");
  TORCH_CHECK(num_experts <= WR_MAX_EXPERTS, "num_experts ", num_experts,
              " exceeds GATE_MAX_EXPERTS ", WR_MAX_EXPERTS);
  TORCH_CHECK(top_k >= 1 && top_k <= WR_MAX_TOPK && top_k <= num_experts,
              "top_k must be in [1, min(", WR_MAX_TOPK, ", num_experts)], got ", top_k);
  const torch::Device dev = hidden.device();
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  const int B = hidden.dim() == 2 ? (int)hidden.size(0) : 1;
  std::vector<int64_t> shape;
  if (hidden.dim() == 2) shape.push_back(B);
  shape.push_back(top_k);
  torch::Tensor ids = torch::empty(shape, torch::TensorOptions().dtype(torch::kInt32).device(dev));
  torch::Tensor ws = torch::empty(shape, torch::TensorOptions().dtype(torch::kFloat32).device(dev));
  if (B == 0) return {ids, ws};
  wr_moe_args a{};
  a.gate_w = gate_w.data_ptr<float>();
  a.weight_dtype = WR_F32;
  a.num_experts = num_experts;
  a.hidden_dim = hidden_dim;
  a.intermediate_dim = 1;
  a.top_k = top_k;
  a.renormalize = renormalize ? 1 : 0;
  a.batch_size = B;
  a.act_dtype = dtype_tag(hidden, "hidden");
  a.x = hidden.data_ptr();
  a.topk_ids = ids.data_ptr<int32_t>();
  a.topk_weights = ws.data_ptr<float>();
  void* stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream();
  check_status(wr_gate_topk(&a, stream), "gate_topk");
  return {ids, ws};
}

void set_handoff_check(bool enabled) { g_check_handoff.store(enabled); }
bool handoff_check() { return g_check_handoff.load(); }

py::dict layout(int num_experts, int hidden_dim, int intermediate_dim, int elem_bytes) {
  wr_offsets o;
  check_status(wr_layout(num_experts, hidden_dim, intermediate_dim, elem_bytes, &o), "layout");
  py::dict d;
  d["gate_proj_offset"] = o.gate_proj_offset;
  d["up_proj_offset"] = o.up_proj_offset;
  d["down_proj_offset"] = o.down_proj_offset;
  d["expert_stride"] = o.expert_stride;
  return d;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  const auto opt = py::arg("topk_ids") = py::none();
  const auto optw = py::arg("topk_weights") = py::none();
  m.def("naive_moe_forward", &naive_moe_forward,
        "Naive multi-kernel MoE forward (host top-K; fp32, fp16, bf16, fp8 e4m3 or mxfp4 "
        "weights)",
        py::arg("hidden"),
        py::arg("gate_w"), py::arg("weight_buf"), py::arg("num_experts"), py::arg("hidden_dim"),
        py::arg("intermediate_dim"), py::arg("top_k"), py::arg("renormalize") = false, opt, optw);
  m.def("fused_moe_forward", &fused_moe_forward,
        "Fused decode MoE forward for one token (fp32, fp16, bf16, fp8 e4m3 or mxfp4 weights)",
        py::arg("hidden"),
        py::arg("gate_w"), py::arg("weight_buf"), py::arg("num_experts"), py::arg("hidden_dim"),
        py::arg("intermediate_dim"), py::arg("top_k"), py::arg("renormalize") = false, opt, optw);
  m.def("batched_fused_moe_forward", &batched_fused_moe_forward,
        "Batched fused MoE forward for B tokens (fp32, fp16, bf16, fp8 e4m3 or mxfp4 weights)",
        py::arg("hidden_batch"),
        py::arg("gate_w"), py::arg("weight_buf"), py::arg("num_experts"), py::arg("hidden_dim"),
        py::arg("intermediate_dim"), py::arg("top_k"), py::arg("renormalize") = false, opt, optw);
  m.def("gate_topk", &gate_topk, "Router logits, softmax and top-K", py::arg("hidden"),
        py::arg("gate_w"), py::arg("num_experts"), py::arg("hidden_dim"), py::arg("top_k"),
        py::arg("renormalize") = false);
  m.def("set_handoff_check", &set_handoff_check,
        "Make fused_moe_forward synchronise and raise if its hand-off wait expired",
        py::arg("enabled"));
  m.def("handoff_check", &handoff_check, "Whether fused_moe_forward checks its hand-off");
  m.def("layout", &layout, "Packed expert layout offsets in bytes", py::arg("num_experts"),
        py::arg("hidden_dim"), py::arg("intermediate_dim"), py::arg("elem_bytes"));
  m.def("total_weight_bytes", &wr_total_weight_bytes, "Packed layout size in bytes (-1 if invalid)",
        py::arg("num_experts"), py::arg("hidden_dim"), py::arg("intermediate_dim"),
        py::arg("elem_bytes"));
  m.def("weight_bytes", &wr_weight_bytes,
        "Packed layout size in bytes for a wr_dtype tag (-1 if invalid)", py::arg("num_experts"),
        py::arg("hidden_dim"), py::arg("intermediate_dim"), py::arg("weight_dtype"));
}
