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
//   dropin_main backward <in.bin> <dy.bin> <grad.bin>   (forward, then
//       backward with dout = dy; grad.bin: the MGPTGRD1 format of
//       oracle/ref_driver.cpp, dx then every parameter's Tensor::grad)
//   dropin_main shapes                   (the engine's MoE shape and
//       backward test, tests/networkTest/moeTests.cpp:6-39, at C = 64)
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <vector>

#include "MoELayer.h"

namespace {

bool read_exact(FILE* f, void* dst, size_t bytes) { return std::fread(dst, 1, bytes, f) == bytes; }

// Reads in.bin into x and the layer's parameters; returns 0 on success.
int load(const char* in_path, int32_t (&dims)[5], Tensor& x, std::unique_ptr<MoELayer>& layer) {
  FILE* f = std::fopen(in_path, "rb");
  if (!f) { std::perror(in_path); return 2; }
  char magic[8];
  if (!read_exact(f, magic, 8) || std::memcmp(magic, "MGPTMOE1", 8) != 0 ||
      !read_exact(f, dims, sizeof(dims))) {
    std::fprintf(stderr, "bad input header\n");
    return 2;
  }
  const int N = dims[0], C = dims[1], H = dims[2], E = dims[3], k = dims[4];
  layer.reset(new MoELayer(C, H, E, k));
  x = Tensor({1, N, C});
  if (!read_exact(f, x.get_data_ptr(), sizeof(float) * x.size())) return 2;
  for (Tensor* p : layer->get_parameters())
    if (!read_exact(f, p->get_data_ptr(), sizeof(float) * p->size())) return 2;
  std::fclose(f);
  return 0;
}

int run(const char* in_path, const char* out_path) {
  int32_t dims[5];
  Tensor x;
  std::unique_ptr<MoELayer> owner;
  if (int rc = load(in_path, dims, x, owner)) return rc;
  MoELayer& layer = *owner;
  const int N = dims[0], C = dims[1], E = dims[3];

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

int backward(const char* in_path, const char* dy_path, const char* out_path) {
  int32_t dims[5];
  Tensor x;
  std::unique_ptr<MoELayer> owner;
  if (int rc = load(in_path, dims, x, owner)) return rc;
  MoELayer& layer = *owner;
  const int N = dims[0], C = dims[1];
  Tensor dy({1, N, C});
  FILE* f = std::fopen(dy_path, "rb");
  if (!f) { std::perror(dy_path); return 2; }
  if (!read_exact(f, dy.get_data_ptr(), sizeof(float) * dy.size())) return 2;
  std::fclose(f);

  Tensor y, dx;
  layer.forward_into(x, y);
  layer.backward_into(dy, dx);

  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  std::fwrite("MGPTGRD1", 1, 8, o);
  std::fwrite(dims, sizeof(int32_t), 5, o);
  std::fwrite(dx.get_data_ptr(), sizeof(float), dx.size(), o);
  for (Tensor* p : layer.get_parameters()) std::fwrite(p->get_grad_ptr(), sizeof(float), p->size(), o);
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
  // the engine's backward test (moeTests.cpp:22-39): dout = 1, din keeps
  // the input's shape; here also finite values and gradients added to the
  // parameters' grads
  Tensor dout({B, T, C}, 1.0f);
  moe.forward(x);
  Tensor din = moe.backward(dout);
  if (din.shape != std::vector<int>({B, T, C})) return fail("din shape");
  for (size_t i = 0; i < din.size(); ++i)
    if (!std::isfinite(din.get_data_ptr()[i])) return fail("finite din");
  double gsum = 0;
  for (Tensor* p : moe.get_parameters())
    for (size_t i = 0; i < p->size(); ++i) gsum += std::fabs(p->get_grad_ptr()[i]);
  if (!(gsum > 0) || !std::isfinite(gsum)) return fail("parameter gradients");
  bool threw = false;
  try {
    Tensor bad({B, T + 1, C}, 1.0f);
    moe.backward(bad);
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  if (!threw) return fail("dout shape mismatch must throw");
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
    if (argc == 5 && std::strcmp(argv[1], "backward") == 0) return backward(argv[2], argv[3], argv[4]);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "exception: %s\n", e.what());
    return 3;
  }
  std::fprintf(stderr, "usage: dropin_main run <in> <out> | backward <in> <dy> <grad> | shapes\n");
  return 2;
}
