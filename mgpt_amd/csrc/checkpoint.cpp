// checkpoint.cpp -- the GPT checkpoint (.bin) weight path, host only.
//
// The engine saves a model as GPT::save_weights_bin does (nn/GPT.cpp:128-155):
// a 5-int header (vocab_size, max_seq_len, embed_dim, num_layers,
// completed_steps; older files lack the last) and then every parameter as
// float32 in GPT::get_parameters() order.  Only one transformer block's MoE
// parameters (and its ln2 scale) are wanted here, so instead of reading the
// whole model the file position of that block is computed from the header
// and the two dimensions the file does not store (E, H), and only those
// bytes are read.
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/mgpt_moe.h"
#include "capi_internal.hpp"

using mgpt::fail;

namespace {

// Floats of each part of the model, in GPT::get_parameters() order.
struct GptLayout {
  int64_t tok_emb, ln1, attn, ln2, moe, block, ln_f, lm_head, total;
  int64_t C;
};

GptLayout layout(int64_t V, int64_t C, int64_t L, int64_t E, int64_t H) {
  GptLayout g{};
  g.C = C;
  g.tok_emb = V * C;                              // EmbeddingLayer lookup_table [V,C]
  g.ln1 = C;                                      // RMSNormLayer scale [C]
  g.attn = (C * 3 * C + 3 * C) + (C * C + C);     // W_QKV, b_QKV, W_O, b_O
  g.ln2 = C;
  g.moe = (C * E + E) + E * (2 * (C * H + H) + (H * C + C));   // router, experts
  g.block = g.ln1 + g.attn + g.ln2 + g.moe;
  g.ln_f = 2 * C;                                 // LayerNormLayer scale, shift
  g.lm_head = C * V + V;                          // LinearLayer [C,V], [1,V]
  g.total = g.tok_emb + L * g.block + g.ln_f + g.lm_head;
  return g;
}

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

int open_and_inspect(const char* path, int E, int H_in, File& file, mgpt_gpt_bin_info* info,
                     GptLayout* lay) {
  if (!path || !info) return fail(MGPT_ERR_INVALID_ARGUMENT, "path or info is null");
  if (E < 1) return fail(MGPT_ERR_INVALID_ARGUMENT, "num_experts %d < 1", E);
  if (H_in == 0 || H_in < -1) return fail(MGPT_ERR_INVALID_ARGUMENT, "hidden_dim %d", H_in);
  file.f = std::fopen(path, "rb");
  if (!file.f) return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: %s", path, std::strerror(errno));
  if (std::fseek(file.f, 0, SEEK_END) != 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: cannot seek", path);
  const long long bytes = std::ftell(file.f);
  std::rewind(file.f);
  int32_t hdr[4];
  if (bytes < 16 || std::fread(hdr, sizeof(int32_t), 4, file.f) != 4)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: shorter than the 4-int header", path);
  const int32_t V = hdr[0], S = hdr[1], C = hdr[2], L = hdr[3];
  if (V < 1 || S < 1 || C < 1 || L < 1)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: bad header (%d, %d, %d, %d)", path, V, S, C, L);
  const int64_t H = H_in > 0 ? H_in : 4 * (int64_t)C;
  *lay = layout(V, C, L, E, H);
  const int64_t need = 4 * lay->total;
  info->vocab_size = V;
  info->max_seq_len = S;
  info->embed_dim = C;
  info->num_layers = L;
  info->file_bytes = bytes;
  info->param_floats = lay->total;
  info->block_floats = lay->block;
  info->moe_floats = lay->moe;
  info->completed_steps = 0;
  // nn/GPT.cpp:187-190: the fifth int is there iff the file can hold it
  // next to every parameter.  Sizes are matched exactly: GPT::save_weights_bin
  // writes nothing else, and E and H (not in the header) are then checked
  // in both directions.
  if (bytes == 20 + need) {
    int32_t steps = 0;
    if (std::fread(&steps, sizeof(int32_t), 1, file.f) != 1)
      return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: read failed", path);
    info->completed_steps = steps;
    info->header_ints = 5;
  } else if (bytes == 16 + need) {
    info->header_ints = 4;
  } else {
    return fail(MGPT_ERR_INVALID_ARGUMENT,
                "%s: %lld bytes is not a GPT with V=%d C=%d L=%d E=%d H=%lld "
                "(%lld bytes of parameters after a 4- or 5-int header)",
                path, bytes, V, C, L, E, (long long)H, (long long)need);
  }
  return MGPT_OK;
}

bool read_at(FILE* f, int64_t offset_bytes, float* dst, int64_t n) {
  if (std::fseek(f, (long)offset_bytes, SEEK_SET) != 0) return false;
  return std::fread(dst, sizeof(float), (size_t)n, f) == (size_t)n;
}

}  // namespace

extern "C" {

int mgpt_gpt_bin_inspect(const char* path, int num_experts, int hidden_dim,
                         mgpt_gpt_bin_info* info) {
  File file;
  GptLayout lay;
  return open_and_inspect(path, num_experts, hidden_dim, file, info, &lay);
}

int mgpt_gpt_bin_read_block(const char* path, int num_experts, int hidden_dim, int layer,
                            float* ln2_gamma, float* moe_params, size_t moe_floats) {
  File file;
  GptLayout lay;
  mgpt_gpt_bin_info info;
  if (int rc = open_and_inspect(path, num_experts, hidden_dim, file, &info, &lay)) return rc;
  if (layer < 0 || layer >= info.num_layers)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "layer %d outside 0..%d", layer, info.num_layers - 1);
  if (!moe_params) return fail(MGPT_ERR_INVALID_ARGUMENT, "moe_params is null");
  if ((int64_t)moe_floats != lay.moe)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "moe_floats %zu, the block holds %lld", moe_floats,
                (long long)lay.moe);
  const int64_t block0 = 4LL * info.header_ints + 4 * (lay.tok_emb + (int64_t)layer * lay.block);
  const int64_t ln2_at = block0 + 4 * (lay.ln1 + lay.attn);
  if (ln2_gamma && !read_at(file.f, ln2_at, ln2_gamma, lay.ln2))
    return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: reading ln2 of block %d failed", path, layer);
  if (!read_at(file.f, ln2_at + 4 * lay.ln2, moe_params, lay.moe))
    return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: reading the MoE of block %d failed", path, layer);
  return MGPT_OK;
}

}  // extern "C"
