// dropin_main.cpp -- runs the engine with the MI355X MoELayer swapped in.
//
// TEST INFRASTRUCTURE.  Built by tests/engine/Makefile from the engine's own
// unmodified Tensor / Scratchpad / LinearLayer / SwiGLU sources (under
// /root/reference) plus mgpt_amd/host/MoELayer.cpp in place of the engine's
// MoELayer.cpp, linked against mgpt_amd/lib/libmgpt_moe.so.  The engine is
// built without USE_CUDA, so its tensors live on the host and the drop-in
// stages them through device memory.
//
//   dropin_main run <in.bin> <out.bin>   (in.bin: the MGPTMOE1 format of
//       oracle/ref_driver.cpp; out.bin: "MGPTDRP1", int32 N C E, float32
//       y[N*C], float32 counts[E] from get_expert_counts())
//   dropin_main shapes                   (the engine's MoE shape test,
//       tests/networkTest/moeTests.cpp:6-19, at C = 64)
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "MoELayer.h"

namespace {

bool read_exact(FILE* f, void* dst, size_t bytes) { return std::fread(dst, 1, bytes, f) == bytes; }

int run(const char* in_path, const char* out_path) {
  FILE* f = std::fopen(in_path, "rb");
  if (!f) { std::perror(in_path); return 2; }
  char magic[8];
  int32_t dims[5];
  if (!read_exact(f, magic, 8) || std::memcmp(magic, "MGPTMOE1", 8) != 0 ||
      !read_exact(f, dims, sizeof(dims))) {
    std::fprintf(stderr, "bad input header\n");
    return 2;
  }
  const int N = dims[0], C = dims[1], H = dims[2], E = dims[3], k = dims[4];
  MoELayer layer(C, H, E, k);
  Tensor x({1, N, C});
  if (!read_exact(f, x.get_data_ptr(), sizeof(float) * x.size())) return 2;
  for (Tensor* p : layer.get_parameters())
    if (!read_exact(f, p->get_data_ptr(), sizeof(float) * p->size())) return 2;
  std::fclose(f);

  Tensor y = layer.forward(x);
  const std::vector<float>& counts = layer.get_expert_counts();

  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  const int32_t hdr[3] = {N, C, E};
  std::fwrite("MGPTDRP1", 1, 8, o);
  std::fwrite(hdr, sizeof(hdr), 1, o);
  std::fwrite(y.get_data_ptr(), sizeof(float), y.size(), o);
  std::fwrite(counts.data(), sizeof(float), counts.size(), o);
  std::fclose(o);
  return 0;
}

int fail(const char* what) {
  std::fprintf(stderr, "FAIL: %s\n", what);
  return 1;
}

// Shapes and bookkeeping of the engine's MoE test, plus what the drop-in adds:
// counts sum to N*k, outputs finite, errors raised as exceptions.
int shapes() {
  const int B = 2, T = 4, C = 64, E = 4, k = 2;
  MoELayer moe(C, -1, E, k);
  if (moe.get_parameters().size() != (size_t)(2 + 6 * E)) return fail("parameter count");
  if (moe.get_parameters()[2]->shape != std::vector<int>({C, 4 * C})) return fail("hidden -1 -> 4C");
  Tensor x({B, T, C}, 1.0f);
  Tensor y = moe.forward(x);
  if (y.shape != std::vector<int>({B, T, C})) return fail("output shape");
  float total = 0;
  for (float c : moe.get_expert_counts()) total += c;
  if (total != (float)(B * T * k)) return fail("counts sum");
  for (size_t i = 0; i < y.size(); ++i)
    if (!std::isfinite(y.get_data_ptr()[i])) return fail("finite output");
  Tensor out2;
  moe.forward_into(x, out2);
  if (std::memcmp(out2.get_data_ptr(), y.get_data_ptr(), sizeof(float) * y.size()) != 0)
    return fail("forward_into repeatable");
  if (moe.get_footprint(B, T).fwd_standing == 0) return fail("footprint");
  bool threw = false;
  try {
    moe.backward(y);
  } catch (const std::runtime_error&) {
    threw = true;
  }
  if (!threw) return fail("backward must throw");
  threw = false;
  try {
    Tensor bad({B, T, C + 64});
    moe.forward(bad);
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  if (!threw) return fail("shape mismatch must throw");
  std::printf("shapes ok\n");
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc == 4 && std::strcmp(argv[1], "run") == 0) return run(argv[2], argv[3]);
    if (argc == 2 && std::strcmp(argv[1], "shapes") == 0) return shapes();
  } catch (const std::exception& e) {
    std::fprintf(stderr, "exception: %s\n", e.what());
    return 3;
  }
  std::fprintf(stderr, "usage: dropin_main run <in> <out> | shapes\n");
  return 2;
}
