// MoELayer.h -- MI355X drop-in for the engine's Mixture-of-Experts layer.
//
// Same class name, constructor, virtual interface and parameter order as
// mgpt's src/main/neuralnetwork/layers/MoELayer.h:9-51, so TransformerBlock
// (layers/TransformerBlock.h:17) and the Trainer compile unchanged when the
// engine builds this file pair instead of its own MoELayer.{h,cpp}.  The
// forward runs on the GPU through the C ABI of include/mgpt_moe.h; the
// parameters stay the engine's fp32 Tensors (router LinearLayer + SwiGLU
// experts, initialised and ordered exactly as before) and are packed into
// the library's layouts on first use, after to(), or after refresh_weights().
//
// backward_into runs the library's backward on the caches the forward kept
// and adds every parameter's gradient with the engine's own
// Tensor::add_grad, as the engine's layer does through its Linear layers.
//
// Differences from the engine's layer, all deliberate:
//  * errors throw std::runtime_error with the library's message instead of
//    exiting the process;
//  * get_footprint() reports the library's training workspace (routing,
//    gathered rows, activations, the backward's caches) as standing memory,
//    taken from the Scratchpad when one is set and the input is on the
//    device.
#ifndef MGPT_AMD_MOELAYER_H
#define MGPT_AMD_MOELAYER_H

#include <memory>
#include <vector>

#include "Layer.h"
#include "LinearLayer.h"
#include "SwiGLU.h"
#include "mgpt_moe.h"

class MoELayer : public Layer {
 private:
  int embed_dim;
  int hidden_dim;
  int num_experts;
  int top_k;

  LinearLayer router;
  std::vector<SwiGLU> experts;

  struct HandleDeleter { void operator()(mgpt_moe* h) const; };
  struct DeviceDeleter { void operator()(void* p) const; };
  std::unique_ptr<mgpt_moe, HandleDeleter> handle;
  std::unique_ptr<void, DeviceDeleter> owned_workspace;   // when no Scratchpad is used
  size_t owned_workspace_bytes = 0;
  std::unique_ptr<void, DeviceDeleter> staging;           // x and y of host tensors
  size_t staging_bytes = 0;
  std::unique_ptr<void, DeviceDeleter> saved_x;           // the forward's input (device)
  size_t saved_x_bytes = 0;
  std::unique_ptr<void, DeviceDeleter> bwd_staging;       // dy and dx of host tensors
  size_t bwd_staging_bytes = 0;
  void* last_ws = nullptr;                                // workspace of the last forward
  size_t last_ws_bytes = 0;
  int last_B = 0, last_T = 0;
  bool packed = false;

  Tensor cached_out;
  mutable std::vector<float> cached_cpu_counts;
  mutable bool counts_valid = false;

  mgpt_moe* get_handle();
  void ensure_packed();
  void* device_buffer(std::unique_ptr<void, DeviceDeleter>& buf, size_t& have, size_t need);

 public:
  MoELayer(int embed_dim, int hidden_dim, int num_experts, int top_k);

  // Per-expert token counts of the last forward (floats, as the engine's).
  const std::vector<float>& get_expert_counts() const;

  void set_scratchpad(Scratchpad* pad) override;

  Tensor forward(const Tensor& input) override;
  void forward_into(const Tensor& input, Tensor& output) override;

  Tensor backward(const Tensor& dout) override;
  void backward_into(const Tensor& dout, Tensor& din) override;

  std::vector<Tensor*> get_parameters() override;
  ScratchpadFootprint get_footprint(int B, int T) override;

  void to(Device target_device) override;

  // Re-pack the parameters before the next forward (after an optimizer step
  // or any other write to the Tensors get_parameters() returns).
  void refresh_weights() { packed = false; }
};

#endif  // MGPT_AMD_MOELAYER_H
