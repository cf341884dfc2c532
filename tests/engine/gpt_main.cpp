// gpt_main.cpp -- the engine's whole GPT with the MI355X MoELayer swapped in.
//
// TEST INFRASTRUCTURE.  Built by tests/engine/Makefile from the engine's own
// unmodified sources (GPT, TransformerBlock, attention, norms, embedding,
// Linear, SwiGLU, Tensor; through a tree of symbolic links) with
// mgpt_amd/host/MoELayer.{h,cpp} in place of the engine's MoE layer, linked
// against mgpt_amd/lib/libmgpt_moe.so.  The engine is built without USE_CUDA:
// its tensors live on the host and the drop-in stages them through the GPU.
//
//   gpt_main logits <model.bin> <heads> <E> <k> <H> <ids.bin> <out.bin>
//       builds the GPT that the checkpoint's header (vocab, max_seq_len,
//       embed_dim, layers) and the given heads / experts / top-k / hidden
//       describe, loads the file with the engine's own GPT::load_weights_bin
//       (nn/GPT.cpp:157-206), runs GPT::forward on ids.bin (int32 token ids,
//       one sequence) and writes the logits [T*V] float32 to out.bin.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "GPT.h"

namespace {

int logits(const char* bin, int heads, int E, int k, int H, const char* ids_path,
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
  try {
    if (argc == 9 && std::strcmp(argv[1], "logits") == 0)
      return logits(argv[2], std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5]),
                    std::atoi(argv[6]), argv[7], argv[8]);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 3;
  }
  std::fprintf(stderr, "usage: gpt_main logits <model.bin> <heads> <E> <k> <H> <ids> <out>\n");
  return 1;
}
