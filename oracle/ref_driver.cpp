// ref_driver.cpp -- drives the reference's own MoELayer CPU forward.
//
// TEST INFRASTRUCTURE ONLY.  Linked with the reference's unmodified sources
// (compiled from /root/reference by oracle/Makefile into oracle/_ref/), it is
// used to (1) write the golden fixtures that pin oracle/moe_oracle.c and the
// HIP path (tests/golden/make_golden.py) and (2) time the reference CPU path
// for bench.py's cpu_baseline leg.  Nothing in the product links it.
//
//   ref_driver run  <in.bin> <out.bin>
//   ref_driver backward <in.bin> <dy.bin> <grad.bin>
//   ref_driver block <in.bin> <gamma.bin> <out.bin>
//   ref_driver block_backward <in.bin> <gamma.bin> <dy.bin> <grad.bin>
//   ref_driver bench <N> <C> <H> <E> <k> <reps>
//   ref_driver bench_train <N> <C> <H> <E> <k> <reps>   (zero_grad + forward + backward)
//   ref_driver bench_block <N> <C> <H> <E> <k> <reps>   (ln2 + MoE + residual)
//   ref_driver bench_block_train <N> <C> <H> <E> <k> <reps>
//            (zero_grad, ln2 + MoE + residual forward, then their backward)
//   ref_driver gptbin <out.bin> <side.bin> V S C L heads E k H steps seed
//   ref_driver gptlogits <model.bin> <heads> <E> <k> <H> <ids.bin> <out.bin>
//   ref_driver train <in.bin> <dy.bin> <out.bin> <steps> <lr>
//
// in.bin : "MGPTMOE1", int32 N C H E k, then float32 x[N*C] and the 2+6E
//          parameters in MoELayer::get_parameters() order
//          (layers/MoELayer.cpp:225-236): W_r[C*E], b_r[E], then per expert
//          W_g[C*H], b_g[H], W_u[C*H], b_u[H], W_d[H*C], b_d[C].
// out.bin: "MGPTOUT1", int32 N C E k, float32 y[N*C], int32 idx[N*k],
//          float32 topp[N*k], int32 counts[E], int32 offsets[E],
//          int32 perm[N*k], float32 logits[N*E], float32 probs[N*E].
// dy.bin : float32 dy[N*C] (the upstream gradient).
// block  : x of in.bin is the residual stream x1, gamma.bin float32 [C] the
//          ln2 scale; out.bin: "MGPTBLK1", int32 N C E k, float32 out[N*C]
//          (x1 + MoE(ln2(x1)), layers/TransformerBlock.cpp:42-46), float32
//          xn[N*C] (ln2's output), float32 rstd[N] (its cached_rsqrt),
//          int32 idx[N*k], float32 topp[N*k], int32 counts[E], int32 perm[N*k].
// block_backward: x of in.bin is x1 and dy.bin the upstream gradient of
//          out; grad.bin: "MGPTBBK1", int32 N C H E k, float32 dx1[N*C],
//          the ln2 scale's .grad [C], then the MoE parameters' .grad as in
//          grad.bin below.
// grad.bin: "MGPTGRD1", int32 N C H E k, float32 dx[N*C], then the .grad of
//          every parameter in get_parameters() order (sizes as in in.bin),
//          after one forward_into and one backward_into
//          (layers/MoELayer.cpp:130-223) on a fresh layer.
// gptbin : a GPT checkpoint written by the reference's own
//          GPT::save_weights_bin (nn/GPT.cpp:128-155) for GPTConfig{V, S, C,
//          L, heads, hidden_dim H, E, k}, every parameter a seeded normal
//          (std 0.3; RMSNorm scales 1 + 0.2 N(0,1)) rounded to a multiple of
//          1/64; side.bin: "MGPTGBS1",
//          int32 V S C L E k H steps, then per block its ln2 scale [C] and
//          its MoE parameters in get_parameters() order, read from the live
//          layers (not from file offsets).
// train  : `steps` training steps as the Trainer runs them
//          (pipeline/Trainer.cpp:303-386: zero every parameter's grad,
//          forward_into, backward_into with dout = dy, then
//          AdamWOptimizer(lr)::step over get_parameters(), other
//          hyper-parameters at their defaults), then one more forward_into;
//          out.bin: "MGPTTRN1", int32 N C H E k steps, float32 y[N*C] of each
//          of the steps + 1 forwards, then the parameters after each step
//          (all 2 + 6E in get_parameters() order, sizes as in in.bin).
// gptlogits: GPT::load_weights_bin of model.bin into the GPT its header and
//          the given heads / E / k / H describe, then GPT::forward on the
//          int32 token ids of ids.bin; writes the logits [T*V] float32.
#include <algorithm>
#include <fstream>
#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <iostream>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

// The routing arrays the reference caches for its backward pass are private
// members of MoELayer (layers/MoELayer.h:11-35); this driver reads them after
// forward_into.  Standard headers are included first so only the reference
// headers see the redefinition.
#define private public
#include "MoELayer.h"
#include "RMSNormLayer.h"
#undef private
#include "GPT.h"
#include "AdamWOptimiser.h"

namespace {

bool read_exact(FILE* f, void* dst, size_t bytes) {
  return std::fread(dst, 1, bytes, f) == bytes;
}

// Reads in.bin into x and a fresh layer's parameters; returns 0 on success.
int load(const char* in_path, int32_t dims[5], Tensor& x, std::unique_ptr<MoELayer>& layer) {
  FILE* f = std::fopen(in_path, "rb");
  if (!f) { std::perror(in_path); return 2; }
  char magic[8];
  if (!read_exact(f, magic, 8) || std::memcmp(magic, "MGPTMOE1", 8) != 0 ||
      !read_exact(f, dims, sizeof(int32_t) * 5)) {
    std::fprintf(stderr, "bad input header\n");
    return 2;
  }
  const int N = dims[0], C = dims[1], H = dims[2], E = dims[3], k = dims[4];
  x = Tensor({1, N, C}, 0.0f, Device::CPU);
  if (!read_exact(f, x.data.data(), sizeof(float) * (size_t)N * C)) return 3;
  layer.reset(new MoELayer(C, H, E, k));
  std::vector<Tensor*> params = layer->get_parameters();
  if ((int)params.size() != 2 + 6 * E) {
    std::fprintf(stderr, "unexpected parameter count %zu\n", params.size());
    return 4;
  }
  for (Tensor* p : params)
    if (!read_exact(f, p->data.data(), sizeof(float) * p->size())) return 3;
  std::fclose(f);
  return 0;
}

int run(const char* in_path, const char* out_path) {
  int32_t dims[5];
  Tensor x;
  std::unique_ptr<MoELayer> owner;
  if (int rc = load(in_path, dims, x, owner)) return rc;
  MoELayer& layer = *owner;
  const int N = dims[0], C = dims[1], E = dims[3], k = dims[4];

  Tensor y;
  layer.forward_into(x, y);

  const size_t A = (size_t)N * k;
  std::vector<int32_t> idx(A), perm(A), counts(E), offsets(E);
  for (size_t i = 0; i < A; ++i) idx[i] = (int32_t)layer.cached_top_indices.data[i];
  for (size_t i = 0; i < A; ++i) perm[i] = (int32_t)layer.cached_sorted_token_ids.data[i];
  for (int e = 0; e < E; ++e) counts[e] = (int32_t)layer.cached_cpu_counts[e];
  for (int e = 0; e < E; ++e) offsets[e] = (int32_t)layer.cached_cpu_offsets[e];

  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  int32_t odims[4] = {N, C, E, k};
  std::fwrite("MGPTOUT1", 1, 8, o);
  std::fwrite(odims, sizeof(int32_t), 4, o);
  std::fwrite(y.data.data(), sizeof(float), (size_t)N * C, o);
  std::fwrite(idx.data(), sizeof(int32_t), A, o);
  std::fwrite(layer.cached_top_probs.data.data(), sizeof(float), A, o);
  std::fwrite(counts.data(), sizeof(int32_t), E, o);
  std::fwrite(offsets.data(), sizeof(int32_t), E, o);
  std::fwrite(perm.data(), sizeof(int32_t), A, o);
  std::fwrite(layer.cached_router_logits.data.data(), sizeof(float), (size_t)N * E, o);
  std::fwrite(layer.cached_router_probs.data.data(), sizeof(float), (size_t)N * E, o);
  std::fclose(o);
  return 0;
}

int backward(const char* in_path, const char* dy_path, const char* out_path) {
  int32_t dims[5];
  Tensor x;
  std::unique_ptr<MoELayer> owner;
  if (int rc = load(in_path, dims, x, owner)) return rc;
  MoELayer& layer = *owner;
  const int N = dims[0], C = dims[1];
  Tensor dy({1, N, C}, 0.0f, Device::CPU);
  FILE* f = std::fopen(dy_path, "rb");
  if (!f) { std::perror(dy_path); return 2; }
  if (!read_exact(f, dy.data.data(), sizeof(float) * (size_t)N * C)) return 3;
  std::fclose(f);

  Tensor y, dx;
  layer.forward_into(x, y);
  layer.backward_into(dy, dx);

  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  std::fwrite("MGPTGRD1", 1, 8, o);
  std::fwrite(dims, sizeof(int32_t), 5, o);
  std::fwrite(dx.data.data(), sizeof(float), (size_t)N * C, o);
  for (Tensor* p : layer.get_parameters()) {
    if (p->grad.size() != p->size()) {
      std::fprintf(stderr, "parameter without a gradient buffer\n");
      return 4;
    }
    std::fwrite(p->grad.data(), sizeof(float), p->size(), o);
  }
  std::fclose(o);
  return 0;
}

int train(const char* in_path, const char* dy_path, const char* out_path, int steps, float lr) {
  int32_t dims[5];
  Tensor x;
  std::unique_ptr<MoELayer> owner;
  if (int rc = load(in_path, dims, x, owner)) return rc;
  MoELayer& layer = *owner;
  const int N = dims[0], C = dims[1];
  Tensor dy({1, N, C}, 0.0f, Device::CPU);
  FILE* f = std::fopen(dy_path, "rb");
  if (!f) { std::perror(dy_path); return 2; }
  if (!read_exact(f, dy.data.data(), sizeof(float) * (size_t)N * C)) return 3;
  std::fclose(f);

  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  const int32_t hdr[6] = {dims[0], dims[1], dims[2], dims[3], dims[4], steps};
  std::fwrite("MGPTTRN1", 1, 8, o);
  std::fwrite(hdr, sizeof(int32_t), 6, o);
  AdamWOptimizer opt(lr);
  std::vector<Tensor*> params = layer.get_parameters();
  std::vector<std::vector<float>> after;
  Tensor y, dx;
  for (int s = 0; s <= steps; ++s) {
    for (Tensor* p : params) p->zero_grad();
    layer.forward_into(x, y);
    std::fwrite(y.data.data(), sizeof(float), (size_t)N * C, o);
    if (s == steps) break;
    layer.backward_into(dy, dx);
    opt.step(params);
    for (Tensor* p : params) after.push_back(p->data);
  }
  for (const auto& v : after) std::fwrite(v.data(), sizeof(float), v.size(), o);
  std::fclose(o);
  return 0;
}

int block(const char* in_path, const char* g_path, const char* out_path) {
  int32_t dims[5];
  Tensor x1;
  std::unique_ptr<MoELayer> owner;
  if (int rc = load(in_path, dims, x1, owner)) return rc;
  MoELayer& layer = *owner;
  const int N = dims[0], C = dims[1], E = dims[3], k = dims[4];
  RMSNormLayer ln2(C);   // eps = 1e-5, layers/RMSNormLayer.h:23
  FILE* f = std::fopen(g_path, "rb");
  if (!f) { std::perror(g_path); return 2; }
  if (!read_exact(f, ln2.get_parameters()[0]->data.data(), sizeof(float) * C)) return 3;
  std::fclose(f);

  Tensor xn, y, out;
  ln2.forward_into(x1, xn);
  layer.forward_into(xn, y);
  Tensor::add_into(x1, y, out);

  const size_t A = (size_t)N * k;
  std::vector<int32_t> idx(A), perm(A), counts(E);
  for (size_t i = 0; i < A; ++i) idx[i] = (int32_t)layer.cached_top_indices.data[i];
  for (size_t i = 0; i < A; ++i) perm[i] = (int32_t)layer.cached_sorted_token_ids.data[i];
  for (int e = 0; e < E; ++e) counts[e] = (int32_t)layer.cached_cpu_counts[e];
  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  const int32_t odims[4] = {N, C, E, k};
  std::fwrite("MGPTBLK1", 1, 8, o);
  std::fwrite(odims, sizeof(int32_t), 4, o);
  std::fwrite(out.data.data(), sizeof(float), (size_t)N * C, o);
  std::fwrite(xn.data.data(), sizeof(float), (size_t)N * C, o);
  std::fwrite(ln2.cached_rsqrt.data.data(), sizeof(float), (size_t)N, o);
  std::fwrite(idx.data(), sizeof(int32_t), A, o);
  std::fwrite(layer.cached_top_probs.data.data(), sizeof(float), A, o);
  std::fwrite(counts.data(), sizeof(int32_t), E, o);
  std::fwrite(perm.data(), sizeof(int32_t), A, o);
  std::fclose(o);
  return 0;
}

// The MoE half of TransformerBlock::backward_into (layers/TransformerBlock.
// cpp:81-85) after its forward (:42-46) on a fresh ln2 RMSNormLayer and
// MoELayer: mlp.backward_into(dout, d_ln2), ln2.backward_into(d_ln2, d_ln2)
// (the same buffer, as there), Tensor::add_into(dout, d_ln2, d_x1).
int block_backward(const char* in_path, const char* g_path, const char* dy_path,
                   const char* out_path) {
  int32_t dims[5];
  Tensor x1;
  std::unique_ptr<MoELayer> owner;
  if (int rc = load(in_path, dims, x1, owner)) return rc;
  MoELayer& layer = *owner;
  const int N = dims[0], C = dims[1];
  RMSNormLayer ln2(C);
  Tensor& scale = *ln2.get_parameters()[0];
  FILE* f = std::fopen(g_path, "rb");
  if (!f) { std::perror(g_path); return 2; }
  if (!read_exact(f, scale.data.data(), sizeof(float) * C)) return 3;
  std::fclose(f);
  Tensor dout({1, N, C}, 0.0f, Device::CPU);
  f = std::fopen(dy_path, "rb");
  if (!f) { std::perror(dy_path); return 2; }
  if (!read_exact(f, dout.data.data(), sizeof(float) * (size_t)N * C)) return 3;
  std::fclose(f);

  Tensor xn, y, out, d_ln2, d_x1;
  ln2.forward_into(x1, xn);
  layer.forward_into(xn, y);
  Tensor::add_into(x1, y, out);
  layer.backward_into(dout, d_ln2);
  ln2.backward_into(d_ln2, d_ln2);
  Tensor::add_into(dout, d_ln2, d_x1);

  if (scale.grad.size() != scale.size()) {
    std::fprintf(stderr, "ln2 scale without a gradient buffer\n");
    return 4;
  }
  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  std::fwrite("MGPTBBK1", 1, 8, o);
  std::fwrite(dims, sizeof(int32_t), 5, o);
  std::fwrite(d_x1.data.data(), sizeof(float), (size_t)N * C, o);
  std::fwrite(scale.grad.data(), sizeof(float), C, o);
  for (Tensor* p : layer.get_parameters()) {
    if (p->grad.size() != p->size()) {
      std::fprintf(stderr, "parameter without a gradient buffer\n");
      return 4;
    }
    std::fwrite(p->grad.data(), sizeof(float), p->size(), o);
  }
  std::fclose(o);
  return 0;
}

// Times MoELayer::forward_into (train: forward_into then backward_into with
// dout ~ N(0,1); block: ln2 RMSNormLayer, MoELayer and the residual
// Tensor::add_into of layers/TransformerBlock.cpp:42-46) on one fresh layer
// (its CPU caches are sized on first use and never resized,
// layers/MoELayer.cpp:42-50): 1 warmup, then `reps` timed runs; prints one
// JSON line with every run and the median.
enum BenchPass { kBenchForward, kBenchTrain, kBenchBlock, kBenchBlockTrain };

int bench(int N, int C, int H, int E, int k, int reps, BenchPass pass) {
  const bool train = pass == kBenchTrain;
  std::mt19937 gen(20261201u);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  Tensor x({1, N, C}, 0.0f, Device::CPU);
  for (auto& v : x.data) v = nd(gen);
  for (int i = 0; i < N; ++i) {  // RMSNorm-like scaling to unit RMS
    double ss = 0;
    for (int c = 0; c < C; ++c) ss += (double)x.data[(size_t)i * C + c] * x.data[(size_t)i * C + c];
    float r = (float)(1.0 / std::sqrt(ss / C + 1e-5));
    for (int c = 0; c < C; ++c) x.data[(size_t)i * C + c] *= r;
  }
  MoELayer layer(C, H, E, k);
  for (Tensor* p : layer.get_parameters())
    for (auto& v : p->data) v = 0.02f * nd(gen);
  Tensor y, dx, xn, out, d_ln2;
  Tensor dy({1, N, C}, 0.0f, Device::CPU);
  for (auto& v : dy.data) v = nd(gen);
  RMSNormLayer ln2(C);
  for (auto& v : ln2.get_parameters()[0]->data) v = 1.0f + 0.2f * nd(gen);
  auto step = [&]() {
    if (pass == kBenchBlock || pass == kBenchBlockTrain) {
      if (pass == kBenchBlockTrain) {
        for (Tensor* p : layer.get_parameters()) p->zero_grad();
        ln2.get_parameters()[0]->zero_grad();
      }
      ln2.forward_into(x, xn);
      layer.forward_into(xn, y);
      Tensor::add_into(x, y, out);
      if (pass == kBenchBlockTrain) {   // layers/TransformerBlock.cpp:81-85
        layer.backward_into(dy, d_ln2);
        ln2.backward_into(d_ln2, d_ln2);
        Tensor::add_into(dy, d_ln2, dx);
      }
      return;
    }
    if (train)   // the Trainer's per-step order (pipeline/Trainer.cpp:303-305)
      for (Tensor* p : layer.get_parameters()) p->zero_grad();
    layer.forward_into(x, y);
    if (train) layer.backward_into(dy, dx);
  };
  step();  // warmup
  std::vector<double> t;
  for (int r = 0; r < reps; ++r) {
    auto t0 = std::chrono::steady_clock::now();
    step();
    auto t1 = std::chrono::steady_clock::now();
    t.push_back(std::chrono::duration<double>(t1 - t0).count());
  }
  std::vector<double> s = t;
  std::sort(s.begin(), s.end());
  double med = s[s.size() / 2];
  std::printf("{\"pass\": \"%s\", \"N\": %d, \"C\": %d, \"H\": %d, \"E\": %d, \"k\": %d, "
              "\"reps\": %d, \"median_s\": %.6f, \"runs_s\": [",
              train                        ? "zero_grad+forward+backward"
              : pass == kBenchBlock        ? "block"
              : pass == kBenchBlockTrain   ? "block zero_grad+forward+backward"
                                           : "forward",
              N, C, H, E, k, reps, med);
  for (size_t i = 0; i < t.size(); ++i) std::printf("%s%.6f", i ? ", " : "", t[i]);
  std::printf("], \"tokens_per_s\": %.3f, \"threads\": 1}\n", N / med);
  return 0;
}

int gptbin(const char* bin_path, const char* side_path, int V, int S, int C, int L, int heads,
           int E, int k, int H, int steps, unsigned seed) {
  GPTConfig cfg;
  cfg.vocab_size = V;
  cfg.max_seq_len = S;
  cfg.embed_dim = C;
  cfg.num_layers = L;
  cfg.num_heads = heads;
  cfg.hidden_dim = H;
  cfg.num_experts = E;
  cfg.top_k = k;
  GPT gpt(cfg);
  std::mt19937 gen(seed);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  // values on a 1/64 grid, so the committed checkpoint compresses well
  auto grid = [](float v) { return std::round(v * 64.0f) / 64.0f; };
  for (Tensor* p : gpt.get_parameters())
    for (auto& v : p->data) v = grid(0.3f * nd(gen));
  for (auto& b : gpt.blocks) {
    for (auto& v : b->ln1.get_parameters()[0]->data) v = 1.0f + grid(0.2f * nd(gen));
    for (auto& v : b->ln2.get_parameters()[0]->data) v = 1.0f + grid(0.2f * nd(gen));
  }
  gpt.save_weights_bin(bin_path, steps);
  FILE* o = std::fopen(side_path, "wb");
  if (!o) { std::perror(side_path); return 2; }
  const int32_t dims[8] = {V, S, C, L, E, k, H, steps};
  std::fwrite("MGPTGBS1", 1, 8, o);
  std::fwrite(dims, sizeof(int32_t), 8, o);
  for (auto& b : gpt.blocks) {
    const Tensor* g = b->ln2.get_parameters()[0];
    std::fwrite(g->data.data(), sizeof(float), g->data.size(), o);
    for (Tensor* p : b->mlp.get_parameters())
      std::fwrite(p->data.data(), sizeof(float), p->data.size(), o);
  }
  std::fclose(o);
  return 0;
}

int gptlogits(const char* bin, int heads, int E, int k, int H, const char* ids_path,
              const char* out_path) {
  int32_t hdr[4];
  FILE* f = std::fopen(bin, "rb");
  if (!f || std::fread(hdr, sizeof(int32_t), 4, f) != 4) { std::perror(bin); return 2; }
  std::fclose(f);
  GPTConfig cfg;
  cfg.vocab_size = hdr[0];
  cfg.max_seq_len = hdr[1];
  cfg.embed_dim = hdr[2];
  cfg.num_layers = hdr[3];
  cfg.num_heads = heads;
  cfg.num_experts = E;
  cfg.top_k = k;
  cfg.hidden_dim = H;
  cfg.use_flash_attention = false;
  GPT gpt(cfg);
  gpt.load_weights_bin(bin);
  FILE* fi = std::fopen(ids_path, "rb");
  if (!fi) { std::perror(ids_path); return 2; }
  std::vector<int32_t> ids;
  int32_t v;
  while (std::fread(&v, sizeof(int32_t), 1, fi) == 1) ids.push_back(v);
  std::fclose(fi);
  const int T = (int)ids.size();
  Tensor in({1, T}, 0.0f, Device::CPU);
  for (int t = 0; t < T; ++t) in.data[t] = (float)ids[t];
  Tensor out = gpt.forward(in);
  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  std::fwrite(out.data.data(), sizeof(float), out.data.size(), o);
  std::fclose(o);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc == 4 && std::string(argv[1]) == "run") return run(argv[2], argv[3]);
  if (argc == 5 && std::string(argv[1]) == "backward") return backward(argv[2], argv[3], argv[4]);
  if (argc == 5 && std::string(argv[1]) == "block") return block(argv[2], argv[3], argv[4]);
  if (argc == 6 && std::string(argv[1]) == "block_backward")
    return block_backward(argv[2], argv[3], argv[4], argv[5]);
  if (argc == 7 && std::string(argv[1]) == "train")
    return train(argv[2], argv[3], argv[4], std::atoi(argv[5]), (float)std::atof(argv[6]));
  if (argc == 9 && std::string(argv[1]) == "gptlogits")
    return gptlogits(argv[2], std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5]),
                     std::atoi(argv[6]), argv[7], argv[8]);
  if (argc == 14 && std::string(argv[1]) == "gptbin")
    return gptbin(argv[2], argv[3], std::atoi(argv[4]), std::atoi(argv[5]), std::atoi(argv[6]),
                  std::atoi(argv[7]), std::atoi(argv[8]), std::atoi(argv[9]), std::atoi(argv[10]),
                  std::atoi(argv[11]), std::atoi(argv[12]), (unsigned)std::atol(argv[13]));
  if (argc == 8 && (std::string(argv[1]) == "bench" || std::string(argv[1]) == "bench_train" ||
                    std::string(argv[1]) == "bench_block" ||
                    std::string(argv[1]) == "bench_block_train"))
    return bench(std::atoi(argv[2]), std::atoi(argv[3]), std::atoi(argv[4]),
                 std::atoi(argv[5]), std::atoi(argv[6]), std::atoi(argv[7]),
                 std::string(argv[1]) == "bench_train"         ? kBenchTrain
                 : std::string(argv[1]) == "bench_block"       ? kBenchBlock
                 : std::string(argv[1]) == "bench_block_train" ? kBenchBlockTrain
                                                               : kBenchForward);
  std::fprintf(stderr, "usage: ref_driver run <in> <out> | backward <in> <dy> <grad> | "
                       "block <in> <gamma> <out> | block_backward <in> <gamma> <dy> <grad> | "
                       "bench[_train|_block|_block_train] N C H E k reps | "
                       "gptbin <out> <side> V S C L heads E k H steps seed | "
                       "gptlogits <bin> heads E k H <ids> <out>\n");
  return 1;
}
