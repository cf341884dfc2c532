// MoELayer.cpp -- the engine's MoE layer on the MI355X C ABI.
//
// Reference behaviour kept (src/main/neuralnetwork/layers/MoELayer.cpp):
//  * constructor :4-12 (router Linear C->E, E SwiGLU experts C->H->C);
//  * get_parameters order :225-236 ([W_r, b_r] then per expert
//    [W_g, b_g, W_u, b_u, W_d, b_d]), which the library's
//    mgpt_moe_load_parameters takes verbatim;
//  * forward_into :28-128: input [B,T,C], output allocated on the input's
//    device when empty, every element written;
//  * get_expert_counts (MoELayer.h:39): float counts of the last forward.
// The engine's tensors are fp32, so the handle is configured fp32/fp32 (the
// path that matches the reference within 1e-5 with bit-exact routing).
#include "MoELayer.h"

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

#include "Scratchpad.h"

namespace {

void check(int status, const char* what) {
  if (status != MGPT_OK)
    throw std::runtime_error(std::string("MoELayer: ") + what + ": " + mgpt_moe_last_error());
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw std::runtime_error(std::string("MoELayer: ") + what + ": " + hipGetErrorString(e));
}

}  // namespace

void MoELayer::HandleDeleter::operator()(mgpt_moe* h) const { mgpt_moe_destroy(h); }
void MoELayer::DeviceDeleter::operator()(void* p) const { (void)hipFree(p); }

MoELayer::MoELayer(int embed_dim, int hidden_dim, int num_experts, int top_k)
    : embed_dim(embed_dim),
      hidden_dim(hidden_dim == -1 ? 4 * embed_dim : hidden_dim),
      num_experts(num_experts),
      top_k(top_k),
      router(embed_dim, num_experts) {
  for (int i = 0; i < num_experts; i++) experts.emplace_back(embed_dim, hidden_dim);
}

mgpt_moe* MoELayer::get_handle() {
  if (!handle) {
    mgpt_moe_config cfg{embed_dim, hidden_dim, num_experts, top_k, MGPT_DTYPE_F32,
                        MGPT_DTYPE_F32};
    mgpt_moe* h = nullptr;
    check(mgpt_moe_create(&cfg, &h), "create");
    handle.reset(h);
  }
  return handle.get();
}

void MoELayer::ensure_packed() {
  mgpt_moe* h = get_handle();
  if (packed) return;
  std::vector<Tensor*> params = get_parameters();
  std::vector<const float*> ptrs;
  ptrs.reserve(params.size());
  const Device dev = params.front()->device;
  for (Tensor* p : params) {
    if (p->device != dev)
      throw std::runtime_error("MoELayer: parameters are split across devices");
    ptrs.push_back(p->get_data_ptr());
  }
  check(mgpt_moe_load_parameters(h, ptrs.data(), (int)ptrs.size(), dev == Device::CUDA ? 1 : 0,
                                 nullptr),
        "load_parameters");
  packed = true;
}

void* MoELayer::device_buffer(std::unique_ptr<void, DeviceDeleter>& buf, size_t& have,
                              size_t need) {
  if (need > have || !buf) {
    buf.reset();
    have = 0;
    void* p = nullptr;
    check_hip(hipMalloc(&p, need ? need : 256), "workspace allocation");
    buf.reset(p);
    have = need;
  }
  return buf.get();
}

const std::vector<float>& MoELayer::get_expert_counts() const {
  if (!counts_valid && handle) {
    std::vector<int32_t> c(num_experts);
    check(mgpt_moe_expert_counts(handle.get(), c.data(), num_experts), "expert_counts");
    cached_cpu_counts.assign(c.begin(), c.end());
    counts_valid = true;
  }
  return cached_cpu_counts;
}

void MoELayer::set_scratchpad(Scratchpad* pad) {
  Layer::set_scratchpad(pad);
  router.set_scratchpad(pad);
  for (auto& expert : experts) expert.set_scratchpad(pad);
}

Tensor MoELayer::forward(const Tensor& input) {
  forward_into(input, cached_out);
  return cached_out;
}

void MoELayer::forward_into(const Tensor& input, Tensor& output) {
  if (input.shape.size() != 3 || input.shape[2] != embed_dim)
    throw std::invalid_argument("MoELayer: input must be [B, T, embed_dim]");
  const int B = input.shape[0], T = input.shape[1], C = embed_dim;
  const int N = B * T;
  const bool on_dev = input.device == Device::CUDA;
  mgpt_moe* h = get_handle();
  ensure_packed();

  size_t ws_bytes = 0;
  check(mgpt_moe_workspace_bytes(h, N, &ws_bytes), "workspace_bytes");
  void* ws;
  if (scratchpad && on_dev)
    ws = scratchpad->get_address((ws_bytes + sizeof(float) - 1) / sizeof(float));
  else
    ws = device_buffer(owned_workspace, owned_workspace_bytes, ws_bytes);

  if (output.shape.empty()) output = Tensor({B, T, C}, 0.0f, input.device);
  if (output.size() != (size_t)N * C || output.device != input.device)
    throw std::invalid_argument("MoELayer: output must be [B, T, embed_dim] on the input's device");

  const size_t io_bytes = (size_t)N * C * sizeof(float);
  if (on_dev) {
    check(mgpt_moe_forward(h, input.get_data_ptr(), output.get_data_ptr(), N, ws, ws_bytes,
                           nullptr),
          "forward");
  } else {
    // Host tensors: stage x and y through device memory (default stream,
    // synchronous copies, as the engine's own host<->device copies).
    char* st = (char*)device_buffer(staging, staging_bytes, 2 * io_bytes + 512);
    void* dx = st;
    void* dy = st + ((io_bytes + 255) / 256) * 256;
    if (N > 0) check_hip(hipMemcpy(dx, input.get_data_ptr(), io_bytes, hipMemcpyHostToDevice), "copy x");
    check(mgpt_moe_forward(h, dx, dy, N, ws, ws_bytes, nullptr), "forward");
    if (N > 0) check_hip(hipMemcpy(output.get_data_ptr(), dy, io_bytes, hipMemcpyDeviceToHost), "copy y");
  }
  counts_valid = false;
}

Tensor MoELayer::backward(const Tensor& dout) {
  Tensor din;
  backward_into(dout, din);
  return din;
}

void MoELayer::backward_into(const Tensor&, Tensor&) {
  throw std::runtime_error("MoELayer: backward is not provided by the MI355X forward path");
}

std::vector<Tensor*> MoELayer::get_parameters() {
  std::vector<Tensor*> params = router.get_parameters();
  for (auto& expert : experts) {
    auto p = expert.get_parameters();
    params.insert(params.end(), p.begin(), p.end());
  }
  return params;
}

ScratchpadFootprint MoELayer::get_footprint(int B, int T) {
  size_t bytes = 0;
  check(mgpt_moe_workspace_bytes(get_handle(), B * T, &bytes), "workspace_bytes");
  // The workspace stays standing after forward (routing state), as the
  // engine's routing buffers do; no per-expert temporaries.
  return {(bytes + sizeof(float) - 1) / sizeof(float), 0, 0};
}

void MoELayer::to(Device target_device) {
  Layer::to(target_device);
  packed = false;
}
