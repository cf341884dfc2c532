/*
 * mgpt_moe.h -- C ABI of the MI355X (gfx950) Mixture-of-Experts block
 * forward and backward.
 *
 * Drop-in device path for mgpt's MoELayer (mrtcemberci/mgpt,
 * src/main/neuralnetwork/layers/MoELayer.{h,cpp}).  The engine's C++ layer
 * keeps its public API and calls these functions instead of the cuda_ops::
 * free functions it uses today (src/main/utils/cuda_ops.h:7-110).  Plain C:
 * no HIP, torch or C++ types cross the boundary.  Streams are passed as
 * `void*` holding a hipStream_t (NULL = the default stream); every device
 * pointer is a HIP device address.
 *
 * Semantics follow the reference CPU path exactly for routing (router
 * logits, clamped softmax, top-k with the lower-expert-id tie rule, expert
 * counts, and the stable expert-major permutation of flat assignment ids
 * i = t*k + j); expert outputs are within the precision of the configured
 * dtypes (fp32: 1e-5 relative; bf16: 2e-2; fp8 e4m3 weights: 6e-2).
 *
 * All functions return an mgpt_status; none exits the process.  After a
 * nonzero status, mgpt_moe_last_error() describes it (per host thread).
 * A handle is not safe for concurrent use from several host threads; use one
 * handle per concurrent stream.
 */
#ifndef MGPT_MOE_H
#define MGPT_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mgpt_status {
  MGPT_OK = 0,
  MGPT_ERR_INVALID_ARGUMENT = 1,   /* null pointer, bad size, bad shape */
  MGPT_ERR_UNSUPPORTED = 2,        /* valid but not built for (e.g. E > 512) */
  MGPT_ERR_WORKSPACE_TOO_SMALL = 3,
  MGPT_ERR_NOT_READY = 4,          /* forward before parameters were loaded */
  MGPT_ERR_HIP = 5,                /* a HIP runtime call failed */
  MGPT_ERR_OUT_OF_MEMORY = 6
} mgpt_status;

typedef enum mgpt_dtype {
  MGPT_DTYPE_F32 = 0,
  MGPT_DTYPE_BF16 = 1,
  MGPT_DTYPE_FP8_E4M3 = 2          /* OCP E4M3FN, per-output-channel fp32 scale */
} mgpt_dtype;

/* Shape and precision of one MoE block.  Replaces the constructor arguments
 * MoELayer(int embed_dim, int hidden_dim, int num_experts, int top_k)
 * (layers/MoELayer.cpp:4-12; hidden_dim -1 means 4*embed_dim as in
 * layers/SwiGLU.cpp:4-9). */
typedef struct mgpt_moe_config {
  int embed_dim;     /* C: any width >= 1 (widths that are not a multiple of 64
                        run on zero-padded rows inside the library) */
  int hidden_dim;    /* H: > 0, or -1 for 4*C */
  int num_experts;   /* E: 1..512 (E > 64 runs generic paths: split router,
                        grouped GEMMs, the backward's wide token and router
                        gradients) */
  int top_k;         /* k: 1..min(E, 8) */
  int act_dtype;     /* x and y: MGPT_DTYPE_F32 or MGPT_DTYPE_BF16 */
  int weight_dtype;  /* F32 (act F32 only), BF16 or FP8_E4M3.  With act F32
                        and BF16 / FP8 weights the caller's tensors stay fp32:
                        routing on the fp32 rows, expert products in bf16,
                        fp32 outputs (inference only) */
} mgpt_moe_config;

typedef struct mgpt_moe mgpt_moe;   /* opaque handle; owns packed weights */

/* Creates a handle on the current HIP device.  Replaces the MoELayer
 * constructor (layers/MoELayer.cpp:4-12). */
int mgpt_moe_create(const mgpt_moe_config* cfg, mgpt_moe** out);

/* Frees the handle and its device memory. */
int mgpt_moe_destroy(mgpt_moe* h);

/* Loads the 2 + 6E fp32 parameters in MoELayer::get_parameters() order
 * (layers/MoELayer.cpp:225-236, layers/SwiGLU.cpp:98-103,
 * layers/LinearLayer.cpp:87-89), each in reference layout:
 *   W_r [C,E], b_r [1,E], then for each expert e:
 *   W_gate [C,H], b_gate [1,H], W_up [C,H], b_up [1,H], W_down [H,C], b_down [1,C].
 * `params_on_device` = 1 if the pointers are device addresses, 0 for host.
 * The library copies and packs them (transposed tiles; bf16 rounding or
 * per-output-channel e4m3 quantisation for the expert weights; the router
 * stays fp32).  Replaces Layer::to(Device::CUDA) (layers/Layer.h:46-51) for
 * this layer.  The first load allocates the packed buffers and returns once
 * the packs are done; later loads re-pack into the same buffers.  Host
 * parameters are always waited for (they are staged through one device
 * buffer); a re-pack of device parameters is stream-ordered on `stream`,
 * with no allocation and no host wait (a training loop re-packs after every
 * optimizer step). */
int mgpt_moe_load_parameters(mgpt_moe* h, const float* const* params,
                             int num_params, int params_on_device, void* stream);

/* Device workspace needed by mgpt_moe_forward for num_tokens tokens.
 * Replaces MoELayer::get_footprint (layers/MoELayer.cpp:238-251) for the
 * forward pass; the caller may carve it from its Scratchpad arena. */
int mgpt_moe_workspace_bytes(const mgpt_moe* h, int num_tokens, size_t* bytes);

/* y[N,C] = MoE(x[N,C]) on `stream`, no host synchronisation.  x and y are
 * act_dtype, row-major, device memory; y must not alias x.  The workspace
 * (>= mgpt_moe_workspace_bytes) holds the routing of this call until the
 * next call that uses it.  num_tokens = 0 is a no-op.  Replaces
 * MoELayer::forward_into (layers/MoELayer.cpp:28-128) on the device.
 * No allocation, copy, memset or host synchronisation happens inside, so
 * the call may be captured into a HIP graph (stream capture) and replayed,
 * e.g. the fixed-length decode step of a sampling loop; under capture it
 * records no events (no stage timing; mgpt_moe_expert_counts then reports
 * MGPT_ERR_NOT_READY until the next eager forward). */
int mgpt_moe_forward(mgpt_moe* h, const void* x, void* y, int num_tokens,
                     void* workspace, size_t workspace_bytes, void* stream);

/* mgpt_moe_forward without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.  The
 * workspace is a scratch array built into the library, one per device, of
 * MGPT_MOE_NOALLOC_SCRATCH_BYTES (held from the library's load until the
 * process ends); a num_tokens whose workspace (mgpt_moe_workspace_bytes)
 * exceeds it returns MGPT_ERR_WORKSPACE_TOO_SMALL.  Nothing is allocated,
 * copied or waited for.  Every call on a device shares that device's array:
 * calls that overlap on one device (two streams, or two handles, in flight at
 * once) race and must be serialised by the caller; the array keeps the last
 * call's contents (its routing, until the next call). */
#define MGPT_MOE_NOALLOC_SCRATCH_BYTES (64u << 20)
int mgpt_moe_forward_noalloc(mgpt_moe* h, const void* x, void* y, int num_tokens, void* stream);

/* The MoE half of a transformer block, fused: out = x + MoE(RMSNorm(x) * gamma)
 * with RMSNorm(x) = x / sqrt(mean(x^2) + eps) per token, computed as the
 * engine's ln2 RMSNormLayer does (utils/Tensor.cpp:785-800: sequential sum of
 * squares, r = 1/sqrt(ms/C + eps), (x*r)*gamma).  Replaces the sequence
 * ln2.forward_into, mlp.forward_into, Tensor::add_into of
 * TransformerBlock::forward_into (layers/TransformerBlock.cpp:42-46) without
 * writing or re-reading the normalised rows and the MoE output: the router
 * normalises while it reads x (routing stays bit-exact with the reference on
 * the normalised rows), the permute gathers normalised rows and the combine
 * adds x.  gamma: device [C] fp32; x and out: act_dtype [N,C] (out must not
 * alias x); workspace as for mgpt_moe_forward.  Routing views and counts
 * refer to the normalised rows, as the reference's MoE sees them. */
int mgpt_moe_forward_block(mgpt_moe* h, const void* x, const float* gamma, float eps, void* out,
                           int num_tokens, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Device view of the per-token 1/rms (r above) that the last
 * mgpt_moe_forward_block wrote into `workspace` [N] fp32 (the reference's
 * RMSNormLayer cached_rsqrt). */
int mgpt_moe_get_rstd(const mgpt_moe* h, int num_tokens, void* workspace, float** rstd);

/* Device views of the routing produced by the last mgpt_moe_forward into
 * `workspace` (valid once that call has completed on its stream):
 *   topk_idx [N,k] int32, topk_p [N,k] fp32 (descending p; raw clamped
 *   softmax probabilities, not renormalised), counts [E] int32,
 *   perm [N*k] int32 (slot -> flat assignment id t*k+j, expert-major,
 *   ascending flat id within an expert), slot_of [N*k] int32 (its inverse).
 * Replaces the reference's cached_top_indices, cached_top_probs,
 * cached_expert_counts and cached_sorted_token_ids (layers/MoELayer.h:18-28),
 * which it stores as float; these are int32. */
typedef struct mgpt_moe_routing {
  int32_t* topk_idx;
  float* topk_p;
  int32_t* counts;
  int32_t* perm;
  int32_t* slot_of;
} mgpt_moe_routing;
int mgpt_moe_get_routing(const mgpt_moe* h, int num_tokens, void* workspace,
                         mgpt_moe_routing* out);

/* ---------------------------------------------------------------- training
 * The reference layer is trainable: forward_into caches what backward_into
 * needs, backward_into returns dL/dx and adds every parameter's gradient to
 * its Tensor::grad (add_grad, utils/Tensor.cpp:638-650).  Here the training
 * forward keeps those caches in the workspace, the backward reads them, and
 * the handle owns fp32 gradient buffers in the parameters' reference
 * layouts.  Training needs weight_dtype == act_dtype (fp32 or bf16);
 * fp8 handles return MGPT_ERR_UNSUPPORTED.  bf16 handles compute the
 * gradient products in bf16 with fp32 accumulation (within 2e-2 of the
 * fp32 reference). */

/* Workspace for mgpt_moe_forward_train + mgpt_moe_backward on num_tokens
 * tokens (the forward workspace plus the router probabilities, the gate/up
 * pre-activations and the backward's scratch).  Replaces the training part
 * of MoELayer::get_footprint (layers/MoELayer.cpp:238-251). */
int mgpt_moe_train_workspace_bytes(const mgpt_moe* h, int num_tokens, size_t* bytes);

/* mgpt_moe_forward that also keeps, in `workspace` (>= train workspace
 * bytes), the router probabilities and the gate/up pre-activations next to
 * the routing, gathered rows, SwiGLU outputs and expert outputs: the caches
 * of MoELayer::forward_into (layers/MoELayer.cpp:28-128) and
 * SwiGLU::forward_into (layers/SwiGLU.cpp:23-50). */
int mgpt_moe_forward_train(mgpt_moe* h, const void* x, void* y, int num_tokens,
                           void* workspace, size_t workspace_bytes, void* stream);

/* dx[N,C] = dL/dx for the upstream gradient dy[N,C], given the workspace of
 * the preceding mgpt_moe_forward_train on the same x (which must be passed
 * again, unchanged) and the same num_tokens; adds dL/dW for all 2 + 6E
 * parameters to the handle's gradient buffers, including the load-balance
 * term 0.01 * E * f_e / N on the router probabilities (f_e = count_e / N).
 * Experts no token chose get no gradient, as in the reference.  x, dy, dx
 * are act_dtype, device memory; dx must not overlap x or dy.  The workspace
 * is consumed (a second backward needs a new training forward).  Replaces
 * MoELayer::backward_into (layers/MoELayer.cpp:130-223) on the device.
 * Under HIP graph capture the backward always adds into the gradients (a
 * graph replays the mode it was captured in): zeros still pending from an
 * eager mgpt_moe_zero_grad are written into the graph first, so each replay
 * of a graph captured right after zero_grad starts from zero.  Part of the
 * work (the weight gradients, bf16 large-M shapes) runs on a second
 * stream the handle owns, forked from and joined back into `stream` with
 * events; every result is ordered on `stream` when the call's work there is
 * done, as if it had all run there. */
int mgpt_moe_backward(mgpt_moe* h, const void* x, const void* dy, void* dx, int num_tokens,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Training forward of the fused block: mgpt_moe_forward_block (out = x +
 * MoE(RMSNorm(x) * gamma)) that also keeps the training caches of
 * mgpt_moe_forward_train in `workspace` (>= train workspace bytes), next to
 * the per-token 1/rms.  Replaces, for training, the ln2.forward_into,
 * mlp.forward_into, Tensor::add_into sequence of
 * TransformerBlock::forward_into (layers/TransformerBlock.cpp:42-46). */
int mgpt_moe_forward_block_train(mgpt_moe* h, const void* x, const float* gamma, float eps,
                                 void* out, int num_tokens, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Backward of the fused block after mgpt_moe_forward_block_train on the same
 * x and gamma (passed again, unchanged) and the same num_tokens: for the
 * upstream gradient dout of out, writes dx = dL/dx = dout + ln2's backward
 * of the MoE input gradient, adds the ln2 scale's gradient into dgamma
 * [C] fp32 (device; dgamma[c] += sum over tokens, as the reference adds
 * into scale.grad) and the 2 + 6E MoE gradients into the handle's buffers
 * as mgpt_moe_backward does (the router's weight gradient from the
 * normalised rows).  Replaces mlp.backward_into, ln2.backward_into and
 * Tensor::add_into(dout, d_ln2, d_x1) of TransformerBlock::backward_into
 * (layers/TransformerBlock.cpp:81-85; RMSNormLayer::backward_into,
 * utils/Tensor.cpp:1665-1689).  x, dout, dx are act_dtype [N,C]; dx must not
 * overlap x or dout.  The sums over columns and tokens run in a fixed order
 * of their own (deterministic), not the reference's sequential one. */
int mgpt_moe_backward_block(mgpt_moe* h, const void* x, const float* gamma, const void* dout,
                            void* dx, float* dgamma, int num_tokens, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Sets every gradient to zero on `stream`.  Replaces Tensor::zero_grad
 * (utils/Tensor.cpp:181-187) over this layer's parameters.  Eagerly, before
 * any backward has been captured, no memory is written: the gradients are
 * marked zero on the host, the next mgpt_moe_backward stores them instead of
 * adding, and a read before that (get / accumulate) clears the buffer first.
 * On a capturing stream, or once a backward has been captured into a graph
 * (whose replays add), it enqueues a fill kernel on `stream` that clears the
 * gradients, so zero_grad between graph replays takes effect. */
int mgpt_moe_zero_grad(mgpt_moe* h, void* stream);

/* Copies the 2 + 6E fp32 gradients to grads[i] in get_parameters() order
 * and each parameter's reference layout (as in mgpt_moe_load_parameters);
 * grads_on_device = 1 for device destinations, 0 for host.  Returns once
 * the copies are complete.  Replaces reading Tensor::grad of the layer's
 * parameters (utils/Tensor.h:21). */
int mgpt_moe_get_gradients(mgpt_moe* h, float* const* grads, int num_params,
                           int grads_on_device, void* stream);

/* Adds the handle's 2 + 6E gradients to grads[i] (grads[i] += gradient,
 * one rounded add per element) in get_parameters() order and reference
 * layouts; grads_on_device = 1 for device destinations (stream-ordered, no
 * host synchronisation), 0 for host ones (returns once added).  Replaces the
 * Tensor::add_grad of each parameter that the reference's Linear layers do
 * in their backward (utils/Tensor.cpp:638-650, layers/LinearLayer.cpp:33-80),
 * so a caller accumulates without a temporary per parameter. */
int mgpt_moe_accumulate_gradients(mgpt_moe* h, float* const* grads, int num_params,
                                  int grads_on_device, void* stream);

/* Copies the per-expert token counts of the last forward to host memory,
 * waiting for that forward to finish.  Replaces MoELayer::get_expert_counts
 * (layers/MoELayer.h:39), which returns them as float. */
int mgpt_moe_expert_counts(mgpt_moe* h, int32_t* host_counts, int num_experts);

/* Measurement (no counterpart in the reference): while enabled, each
 * forward records HIP events on its stream at the stage boundaries (into a
 * ring of the last 64 forwards; enabling resets it).  mgpt_moe_stage_times
 * waits for the last profiled forward and returns the mean stage durations
 * in ms over the recorded forwards: [0] router+top-k+histogram, [1] dispatch
 * (count scan + permutation), [2] gate/up GEMM + SwiGLU, [3] down GEMM,
 * [4] combine; if n > 5, ms[5] receives the number of forwards averaged.
 * (Inference steps with fp8 weights, no gamma, bf16 or fp32 rows, an
 * embed_dim padded to a multiple of 128 (its tiled weight copy exists only
 * then) and at most 512 flat ids N*k, below 64*E, route inside the gate/up
 * GEMM: [1] is then only the gap between two events and [2] includes the
 * routing.  Other decode steps run the permute and split their stages as
 * usual.)
 * enable: 0 off, 1 every stage boundary, 2 only the two boundaries of the
 * gate/up GEMM (the other launches keep their spacing; stage_times then
 * returns -1 for the other stages).  The backward records its stages
 * with enable = 1 only. */
#define MGPT_MOE_NUM_STAGES 5
int mgpt_moe_set_profiling(mgpt_moe* h, int enable);
int mgpt_moe_stage_times(mgpt_moe* h, float* ms, int n);

/* The same for the backward (measurement, no counterpart in the reference):
 * while profiling is enabled each mgpt_moe_backward records its stage
 * boundaries too, and this returns the mean durations in ms of
 * [0] scatter backward, [1] d(act) product + SwiGLU backward, [2] dX
 * product, [3] down weight + bias gradients, [4] gate/up weight + bias
 * gradients, [5] per-token gather + softmax + router input gradient,
 * [6] router weight gradient; if n > 7, ms[7] = backwards averaged. */
#define MGPT_MOE_NUM_BWD_STAGES 7
int mgpt_moe_backward_stage_times(mgpt_moe* h, float* ms, int n);

/* fp8 handles only: copies expert `expert`'s quantised weight `which`
 * (0 = W_gate, 1 = W_up, 2 = W_down) to host in reference layout [in,out]
 * as e4m3 bytes, with its per-output-channel scales [out].  For tests of
 * the quantiser; no counterpart in the reference. */
int mgpt_moe_export_fp8(const mgpt_moe* h, int expert, int which,
                        uint8_t* q_host, float* scale_host);

/* Diagnostic (no counterpart in the reference): evaluates the router's
 * device expf -- the GPU restatement of the host C library's expf that the
 * reference's softmax calls (utils/Tensor.cpp:873) -- on n device floats,
 * so tests can compare it bit for bit with the host expf. */
int mgpt_moe_device_expf(const float* d_in, float* d_out, int n, void* stream);

/* ---- GPT checkpoint (.bin) weight path --------------------------------
 * The engine's checkpoint is GPT::save_weights_bin's file (nn/GPT.cpp:128-155):
 * int32 vocab_size, max_seq_len, embed_dim, num_layers, completed_steps,
 * then every parameter as float32 in GPT::get_parameters() order
 * (nn/GPT.cpp:115-126): tok_emb [V,C]; per block (TransformerBlock.cpp:105-112)
 * ln1 scale [C], attention W_QKV [C,3C], b_QKV [3C], W_O [C,C], b_O [C]
 * (MultiHeadAttentionLayer.cpp:178-189), ln2 scale [C], then the block's
 * 2 + 6E MoE parameters (as in mgpt_moe_load_parameters); ln_f scale and
 * shift [C]; lm_head W [C,V], b [V].  Older files have no completed_steps:
 * as GPT::load_weights_bin (nn/GPT.cpp:157-206) decides, the fifth integer
 * is read only when the file holds at least 5 ints plus every parameter. */
typedef struct mgpt_gpt_bin_info {
  int32_t vocab_size, max_seq_len, embed_dim, num_layers;
  int32_t completed_steps;    /* 0 for a 4-int header */
  int32_t header_ints;        /* 4 or 5 */
  int64_t file_bytes;
  int64_t param_floats;       /* every parameter of the model, in floats */
  int64_t block_floats;       /* one transformer block's parameters */
  int64_t moe_floats;         /* one block's 2 + 6E MoE parameters */
} mgpt_gpt_bin_info;

/* Reads a checkpoint's header and checks that its size fits a GPT with
 * num_experts experts of hidden size hidden_dim (> 0, or -1 for 4*C as
 * GPTConfig::default_hidden_scale gives, nn/GPT.cpp:9-10); these two are not
 * in the file.  The file must hold exactly 4 or 5 ints plus every
 * parameter, else MGPT_ERR_INVALID_ARGUMENT (the reference reads a short file
 * short and ignores trailing bytes without a word; exact sizes also catch a
 * wrong E or H).  Host only: no device call. */
int mgpt_gpt_bin_inspect(const char* path, int num_experts, int hidden_dim,
                         mgpt_gpt_bin_info* info);

/* Copies block `layer`'s ln2 scale (ln2_gamma: C floats, may be NULL) and
 * its 2 + 6E MoE parameters (moe_params: info.moe_floats floats, in
 * get_parameters() order and reference layouts, back to back as
 * mgpt_moe_load_parameters' pointers would address them) from the
 * checkpoint into host memory, reading only that block's bytes.  Replaces,
 * for this block, the parameter reads of GPT::load_weights_bin
 * (nn/GPT.cpp:194-203).  Host only. */
int mgpt_gpt_bin_read_block(const char* path, int num_experts, int hidden_dim, int layer,
                            float* ln2_gamma, float* moe_params, size_t moe_floats);

/* Loads block `layer`'s MoE parameters from the checkpoint into the handle
 * (its C, H, E; the file's embed_dim must equal C) and packs / quantises
 * them once, as mgpt_moe_load_parameters does; ln2_gamma (host, C floats,
 * may be NULL) receives the block's ln2 scale for mgpt_moe_forward_block.
 * Synchronous with respect to `stream`'s prior work. */
int mgpt_moe_load_gpt_bin(mgpt_moe* h, const char* path, int layer, float* ln2_gamma,
                          void* stream);

/* Description of the last error on this host thread ("" if none). */
const char* mgpt_moe_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* MGPT_MOE_H */
