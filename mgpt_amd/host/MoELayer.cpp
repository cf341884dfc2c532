// MoELayer.cpp -- the engine's MoE layer on the MI355X C ABI.
//
// Reference behaviour kept (src/main/neuralnetwork/layers/MoELayer.cpp):
//  * constructor :4-12 (router Linear C->E, E SwiGLU experts C->H->C);
//  * get_parameters order :225-236 ([W_r, b_r] then per expert
//    [W_g, b_g, W_u, b_u, W_d, b_d]), which the library's
//    mgpt_moe_load_parameters takes verbatim;
//  * forward_into :28-128: input [B,T,C], output allocated on the input's
//    device when empty, every element written, the backward's caches kept,
//    and the parameters' current values used (they are re-packed whenever
//    they may have changed);
//  * backward_into :130-223: din [B,T,C] for dout of the last forward, and
//    every parameter's gradient added to its Tensor::grad;
//  * get_expert_counts (MoELayer.h:39): float counts of the last forward.
// The engine's tensors are fp32.  By default the handle is fp32 throughout
// (the path that matches the reference within 1e-5 with bit-exact routing);
// set_expert_dtype() keeps the fp32 tensors and runs the expert products in
// bf16 or from fp8 weights.  Everything runs on the default stream, which is
// the stream the engine's own device tensors use.
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
    mgpt_moe_config cfg{embed_dim, hidden_dim, num_experts, top_k, MGPT_DTYPE_F32, expert_dtype};
    mgpt_moe* h = nullptr;
    check(mgpt_moe_create(&cfg, &h), "create");
    handle.reset(h);
  }
  return handle.get();
}

void MoELayer::set_expert_dtype(int dtype) {
  if (dtype != MGPT_DTYPE_F32 && dtype != MGPT_DTYPE_BF16 && dtype != MGPT_DTYPE_FP8_E4M3)
    throw std::invalid_argument("MoELayer: expert dtype must be MGPT_DTYPE_F32, _BF16 or _FP8_E4M3");
  if (dtype == expert_dtype) return;
  expert_dtype = dtype;
  handle.reset();   // a new handle packs the same parameters in the new format
  packed = false;
  last_ws = nullptr;
  counts_valid = false;
}

// Packs the parameters unless the handle already holds a pack of their
// current values: a pack is dropped by to(), set_expert_dtype(),
// refresh_weights() and every backward_into (after which the engine's
// optimizer writes new values into the same buffers), and a pack made from
// other buffers (a parameter reallocated, e.g. by a device round trip) is
// never reused.
void MoELayer::ensure_packed() {
  mgpt_moe* h = get_handle();
  std::vector<Tensor*> params = get_parameters();
  std::vector<const float*> ptrs;
  ptrs.reserve(params.size());
  const Device dev = params.front()->device;
  for (Tensor* p : params) {
    if (p->device != dev)
      throw std::runtime_error("MoELayer: parameters are split across devices");
    ptrs.push_back(p->get_data_ptr());
  }
  if (packed && ptrs == packed_from) return;
  check(mgpt_moe_load_parameters(h, ptrs.data(), (int)ptrs.size(), dev == Device::CUDA ? 1 : 0,
                                 nullptr),
        "load_parameters");
  packed_from = std::move(ptrs);
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
  const bool train = trains();
  mgpt_moe* h = get_handle();
  ensure_packed();

  // The training forward keeps what a following backward needs, as the
  // engine's layer always does; the inference forward keeps nothing.
  size_t ws_bytes = 0;
  if (train)
    check(mgpt_moe_train_workspace_bytes(h, N, &ws_bytes), "train_workspace_bytes");
  else
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
  auto run = [&](const void* x, void* y) {
    if (train)
      check(mgpt_moe_forward_train(h, x, y, N, ws, ws_bytes, nullptr), "forward");
    else
      check(mgpt_moe_forward(h, x, y, N, ws, ws_bytes, nullptr), "forward");
  };
  if (on_dev) {
    if (train) {
      // the backward reads x again: keep a copy (the engine's router Linear
      // keeps one too, layers/LinearLayer.cpp:24), stream-ordered, no wait
      void* xs = device_buffer(saved_x, saved_x_bytes, io_bytes);
      if (N > 0)
        check_hip(hipMemcpyAsync(xs, input.get_data_ptr(), io_bytes, hipMemcpyDeviceToDevice,
                                 nullptr),
                  "copy x");
      run(xs, output.get_data_ptr());
    } else {
      run(input.get_data_ptr(), output.get_data_ptr());
    }
  } else {
    // Host tensors: stage x and y through device memory (default stream,
    // synchronous copies, as the engine's own host<->device copies).
    void* xs = device_buffer(saved_x, saved_x_bytes, io_bytes);
    void* ys = device_buffer(staging, staging_bytes, io_bytes);
    if (N > 0) check_hip(hipMemcpy(xs, input.get_data_ptr(), io_bytes, hipMemcpyHostToDevice), "copy x");
    run(xs, ys);
    if (N > 0) check_hip(hipMemcpy(output.get_data_ptr(), ys, io_bytes, hipMemcpyDeviceToHost), "copy y");
  }
  last_ws = ws;
  last_ws_bytes = ws_bytes;
  last_B = B;
  last_T = T;
  last_trained = train;
  counts_valid = false;
}

Tensor MoELayer::backward(const Tensor& dout) {
  Tensor din;
  backward_into(dout, din);
  return din;
}

void MoELayer::backward_into(const Tensor& dout, Tensor& din) {
  if (!last_ws) throw std::runtime_error("MoELayer: backward before forward");
  if (!last_trained)
    throw std::runtime_error(
        "MoELayer: backward after an inference forward (set_inference(true) or bf16 / fp8 "
        "expert products keep no caches for a backward)");
  if (dout.shape != std::vector<int>({last_B, last_T, embed_dim}))
    throw std::invalid_argument("MoELayer: dout must have the last forward's [B, T, embed_dim]");
  const int N = last_B * last_T, C = embed_dim;
  const bool on_dev = dout.device == Device::CUDA;
  mgpt_moe* h = get_handle();
  if (din.shape.empty() || din.size() != (size_t)N * C || din.device != dout.device)
    din = Tensor({last_B, last_T, C}, 0.0f, dout.device);
  din.shape = {last_B, last_T, C};

  // The handle's gradient buffers hold this call's gradients only; they are
  // then added to the parameters' grads.
  check(mgpt_moe_zero_grad(h, nullptr), "zero_grad");
  const size_t io_bytes = (size_t)N * C * sizeof(float);
  if (on_dev) {
    check(mgpt_moe_backward(h, saved_x.get(), dout.get_data_ptr(), din.get_data_ptr(), N, last_ws,
                            last_ws_bytes, nullptr),
          "backward");
  } else {
    char* st = (char*)device_buffer(bwd_staging, bwd_staging_bytes, 2 * io_bytes + 512);
    void* ddy = st;
    void* ddx = st + ((io_bytes + 255) / 256) * 256;
    if (N > 0) check_hip(hipMemcpy(ddy, dout.get_data_ptr(), io_bytes, hipMemcpyHostToDevice), "copy dy");
    check(mgpt_moe_backward(h, saved_x.get(), ddy, ddx, N, last_ws, last_ws_bytes, nullptr),
          "backward");
    if (N > 0) check_hip(hipMemcpy(din.get_data_ptr(), ddx, io_bytes, hipMemcpyDeviceToHost), "copy dx");
  }

  // Tensor::add_grad of every parameter, done by the library into the grad
  // buffers themselves (no temporary per parameter).
  std::vector<Tensor*> params = get_parameters();
  std::vector<float*> ptrs;
  ptrs.reserve(params.size());
  for (Tensor* p : params) ptrs.push_back(p->get_grad_ptr());
  check(mgpt_moe_accumulate_gradients(h, ptrs.data(), (int)ptrs.size(),
                                      params.front()->device == Device::CUDA ? 1 : 0, nullptr),
        "accumulate_gradients");
  // The engine's optimizer updates the parameters in place after the
  // backward (Tensor::adamw_step / sgd_step, pipeline/Trainer.cpp:386):
  // the next forward re-packs them.
  packed = false;
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
  if (trains())
    check(mgpt_moe_train_workspace_bytes(get_handle(), B * T, &bytes), "train_workspace_bytes");
  else
    check(mgpt_moe_workspace_bytes(get_handle(), B * T, &bytes), "workspace_bytes");
  // The workspace stays standing after forward (routing state and, for
  // training, the backward's caches), as the engine's cached tensors do;
  // the backward works inside it.
  return {(bytes + sizeof(float) - 1) / sizeof(float), 0, 0};
}

void MoELayer::to(Device target_device) {
  Layer::to(target_device);
  packed = false;
}
