// MoELayer.h -- MI355X drop-in for the engine's Mixture-of-Experts layer.
//
// Same class name, constructor, virtual interface and parameter order as
// mgpt's src/main/neuralnetwork/layers/MoELayer.h:9-51, so TransformerBlock
// (layers/TransformerBlock.h:17), the Trainer and the optimizers compile
// unchanged when the engine builds this file pair instead of its own
// MoELayer.{h,cpp}.  The forward runs on the GPU through the C ABI of
// include/mgpt_moe.h; the parameters stay the engine's fp32 Tensors (router
// LinearLayer + SwiGLU experts, initialised and ordered exactly as before)
// and are packed into the library's layouts before a forward whenever they
// may have changed since the last pack: on first use, after to(), after every
// backward (the engine's optimizer updates them in place between a backward
// and the next forward, pipeline/Trainer.cpp:386), when a parameter's buffer
// moved, and after refresh_weights().
//
// backward_into runs the library's backward on the caches the forward kept
// and adds every parameter's gradient into its Tensor::grad, as the engine's
// layer does through its Linear layers (Tensor::add_grad).
//
// Differences from the engine's layer, all deliberate:
//  * errors throw std::runtime_error with the library's message instead of
//    exiting the process;
//  * get_footprint() reports the library's workspace (routing, gathered
//    rows, activations, and for training the backward's caches) as standing
//    memory, taken from the Scratchpad when one is set and the input is on
//    the device;
//  * two options the engine's layer does not have (their defaults keep its
//    behaviour): set_expert_dtype() runs the expert products in bf16 or with
//    fp8 e4m3 weights behind the same fp32 Tensors (inference only), and
//    set_inference() skips the backward's caches and, for device inputs, the
//    copy of x that a following backward would read.
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
  std::unique_ptr<void, DeviceDeleter> saved_x;           // the training forward's input
  size_t saved_x_bytes = 0;
  std::unique_ptr<void, DeviceDeleter> bwd_staging;       // dy and dx of host tensors
  size_t bwd_staging_bytes = 0;
  void* last_ws = nullptr;                                // workspace of the last forward
  size_t last_ws_bytes = 0;
  int last_B = 0, last_T = 0;
  bool last_trained = false;                              // the last forward kept caches

  int expert_dtype = MGPT_DTYPE_F32;
  bool inference = false;
  bool packed = false;
  std::vector<const float*> packed_from;   // parameter buffers of the last pack

  Tensor cached_out;
  mutable std::vector<float> cached_cpu_counts;
  mutable bool counts_valid = false;

  mgpt_moe* get_handle();
  void ensure_packed();
  bool trains() const { return !inference && expert_dtype == MGPT_DTYPE_F32; }
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

  // Re-pack the parameters before the next forward.  Needed only after a
  // write to them that is neither an optimizer step after backward_into nor
  // a reallocation (e.g. values copied into the existing buffers after a
  // forward without a backward in between).
  void refresh_weights() { packed = false; }

  // Precision of the expert products: MGPT_DTYPE_F32 (default; trainable),
  // MGPT_DTYPE_BF16 or MGPT_DTYPE_FP8_E4M3 (per-output-channel scales).  The
  // Tensors stay fp32 and routing runs on their fp32 values either way; the
  // bf16 / fp8 products are an inference format (backward_into throws).
  void set_expert_dtype(int dtype);

  // Inference forwards (e.g. the Generator's sampling loop): no caches for a
  // backward, and a device input is read where it is, with no copy; a
  // backward_into after such a forward throws.
  void set_inference(bool on) { inference = on; }
};

#endif  // MGPT_AMD_MOELAYER_H
