// dropin_main.cpp -- runs the engine with the MI355X MoELayer swapped in.
//
// TEST INFRASTRUCTURE.  Built by tests/engine/Makefile from the engine's own
// unmodified Tensor / Scratchpad / LinearLayer / SwiGLU sources (under
// /root/reference) plus mgpt_amd/host/MoELayer.cpp in place of the engine's
// MoELayer.cpp, linked against mgpt_amd/lib/libmgpt_moe.so, twice:
//  * _build/dropin_main: the engine's CPU build (its cuda_ops are no-ops),
//    so every tensor lives on the host and the drop-in stages them through
//    device memory;
//  * _build/dropin_dev (-DDROPIN_DEVICE): the engine's device-memory
//    primitives over HIP (engine_hip_ops.hip), so the layer's parameters,
//    the inputs, the optimizer state and a Scratchpad live on the device, as
//    in the engine's GPU build: the drop-in's Device::CUDA and Scratchpad
//    branches run.
//
//   run <in.bin> <out.bin>   (in.bin: the MGPTMOE1 format of
//       oracle/ref_driver.cpp; out.bin: "MGPTDRP1", int32 N C E, float32
//       y[N*C], float32 counts[E] from get_expert_counts())
//   backward <in.bin> <dy.bin> <grad.bin>   (forward, then backward with
//       dout = dy; grad.bin: the MGPTGRD1 format of oracle/ref_driver.cpp,
//       dx then every parameter's Tensor::grad)
//   train <in.bin> <dy.bin> <out.bin> <steps> <lr>   (the Trainer's step,
//       pipeline/Trainer.cpp:303-386, `steps` times with the engine's own
//       AdamWOptimizer, then a forward; out.bin: the MGPTTRN1 format of
//       oracle/ref_driver.cpp)
//   shapes   (the engine's MoE test, tests/networkTest/moeTests.cpp:6-76, at
//       its own shape C = 16, plus the drop-in's bookkeeping)
//   decode <x.bin> <router.bin> <seed> <C> <H> <E> <k> <steps> <spin_ms> <out.bin>
//       (dropin_dev only) the Generator's loop, pipeline/Generator.cpp:24-36:
//       `steps` forwards of the same [1, N, C] device input through the
//       layer with fp8 expert weights and inference forwards, enqueued behind
//       a device spin of spin_ms; router.bin: float32 W_r [C*E] then b_r [E];
//       expert weights are the seeded N(0, 0.02^2) streams of
//       mgpt_amd/workload.py (zero biases); out.bin: "MGPTDEC1", int32 N C,
//       float32 enqueue_ms, float32 y[N*C] of the last step
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <vector>

#include "AdamWOptimiser.h"
#include "MoELayer.h"
#include "Scratchpad.h"

#ifdef DROPIN_DEVICE
extern "C" void engine_test_spin(double ms);
extern "C" void mgpt_wl_normal_f32(uint64_t seed, uint64_t stream, int64_t start, int64_t count,
                                   double std, float* out);
constexpr bool kDevice = true;
#else
constexpr bool kDevice = false;
#endif

namespace {

bool read_exact(FILE* f, void* dst, size_t bytes) { return std::fread(dst, 1, bytes, f) == bytes; }

// The engine's device, or the host for the CPU build.
Device dev() { return kDevice ? Device::CUDA : Device::CPU; }

// Host copy of a tensor's values.
std::vector<float> host_values(const Tensor& t) {
  std::vector<float> v(t.size());
  t.copy_to_host(v.data());
  return v;
}
std::vector<float> host_grad(Tensor& t) {
  std::vector<float> v(t.size());
  if (t.device == Device::CUDA) {
    Tensor g = Tensor::view(t.shape, t.get_grad_ptr(), Device::CUDA);
    g.copy_to_host(v.data());
  } else {
    std::memcpy(v.data(), t.get_grad_ptr(), sizeof(float) * v.size());
  }
  return v;
}

// A tensor on the engine's device holding host values.
Tensor on_device(const std::vector<int>& shape, const float* values) {
  Tensor t(shape, 0.0f, Device::CPU);
  std::memcpy(t.get_data_ptr(), values, sizeof(float) * t.size());
  t.to(dev());
  return t;
}

// The layer of in.bin (parameters moved to the engine's device) and its input.
struct Loaded {
  int32_t dims[5];
  std::unique_ptr<MoELayer> layer;
  Tensor x;
  std::unique_ptr<Scratchpad> pad;   // device build: the arena the engine would pass
};

int load(const char* in_path, Loaded& L) {
  FILE* f = std::fopen(in_path, "rb");
  if (!f) { std::perror(in_path); return 2; }
  char magic[8];
  if (!read_exact(f, magic, 8) || std::memcmp(magic, "MGPTMOE1", 8) != 0 ||
      !read_exact(f, L.dims, sizeof(L.dims))) {
    std::fprintf(stderr, "bad input header\n");
    return 2;
  }
  const int N = L.dims[0], C = L.dims[1], H = L.dims[2], E = L.dims[3], k = L.dims[4];
  L.layer.reset(new MoELayer(C, H, E, k));
  std::vector<float> x((size_t)N * C);
  if (!read_exact(f, x.data(), sizeof(float) * x.size())) return 2;
  for (Tensor* p : L.layer->get_parameters())
    if (!read_exact(f, p->get_data_ptr(), sizeof(float) * p->size())) return 2;
  std::fclose(f);
  L.x = on_device({1, N, C}, x.data());
  if (kDevice) {
    L.layer->to(Device::CUDA);
    // an arena of the layer's declared footprint, as GPT sizes its own
    // Scratchpad from get_footprint (nn/GPT.cpp:224-234)
    L.pad.reset(new Scratchpad(L.layer->get_footprint(1, N).fwd_peak() + 64,
                               ScratchpadDevice::CUDA));
    L.layer->set_scratchpad(L.pad.get());
  }
  return 0;
}

int read_dy(const char* path, int N, int C, Tensor& dy) {
  std::vector<float> v((size_t)N * C);
  FILE* f = std::fopen(path, "rb");
  if (!f) { std::perror(path); return 2; }
  if (!read_exact(f, v.data(), sizeof(float) * v.size())) return 2;
  std::fclose(f);
  dy = on_device({1, N, C}, v.data());
  return 0;
}

int run(const char* in_path, const char* out_path) {
  Loaded L;
  if (int rc = load(in_path, L)) return rc;
  const int N = L.dims[0], C = L.dims[1], E = L.dims[3];
  Tensor y = L.layer->forward(L.x);
  const std::vector<float>& counts = L.layer->get_expert_counts();
  const std::vector<float> yh = host_values(y);

  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  const int32_t hdr[3] = {N, C, E};
  std::fwrite("MGPTDRP1", 1, 8, o);
  std::fwrite(hdr, sizeof(hdr), 1, o);
  std::fwrite(yh.data(), sizeof(float), yh.size(), o);
  std::fwrite(counts.data(), sizeof(float), counts.size(), o);
  std::fclose(o);
  return 0;
}

int backward(const char* in_path, const char* dy_path, const char* out_path) {
  Loaded L;
  if (int rc = load(in_path, L)) return rc;
  const int N = L.dims[0], C = L.dims[1];
  Tensor dy;
  if (int rc = read_dy(dy_path, N, C, dy)) return rc;
  Tensor y, dx;
  L.layer->forward_into(L.x, y);
  L.layer->backward_into(dy, dx);

  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  std::fwrite("MGPTGRD1", 1, 8, o);
  std::fwrite(L.dims, sizeof(int32_t), 5, o);
  const std::vector<float> dxh = host_values(dx);
  std::fwrite(dxh.data(), sizeof(float), dxh.size(), o);
  for (Tensor* p : L.layer->get_parameters()) {
    const std::vector<float> g = host_grad(*p);
    std::fwrite(g.data(), sizeof(float), g.size(), o);
  }
  std::fclose(o);
  return 0;
}

int train(const char* in_path, const char* dy_path, const char* out_path, int steps, float lr) {
  Loaded L;
  if (int rc = load(in_path, L)) return rc;
  const int N = L.dims[0], C = L.dims[1];
  Tensor dy;
  if (int rc = read_dy(dy_path, N, C, dy)) return rc;
  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  const int32_t hdr[6] = {L.dims[0], L.dims[1], L.dims[2], L.dims[3], L.dims[4], steps};
  std::fwrite("MGPTTRN1", 1, 8, o);
  std::fwrite(hdr, sizeof(int32_t), 6, o);
  AdamWOptimizer opt(lr);
  std::vector<Tensor*> params = L.layer->get_parameters();
  std::vector<std::vector<float>> after;
  Tensor y, dx;
  for (int s = 0; s <= steps; ++s) {
    if (L.pad) L.pad->reset();   // the engine resets its arena every step
    for (Tensor* p : params) p->zero_grad();
    L.layer->forward_into(L.x, y);
    const std::vector<float> yh = host_values(y);
    std::fwrite(yh.data(), sizeof(float), yh.size(), o);
    if (s == steps) break;
    L.layer->backward_into(dy, dx);
    opt.step(params);
    for (Tensor* p : params) after.push_back(host_values(*p));
  }
  for (const auto& v : after) std::fwrite(v.data(), sizeof(float), v.size(), o);
  std::fclose(o);
  return 0;
}

int fail(const char* what) {
  std::fprintf(stderr, "FAIL: %s\n", what);
  return 1;
}

// The engine's MoE test (tests/networkTest/moeTests.cpp:6-76) at its own
// shape -- B = 2, T = 4, C = 16, E = 4, k = 2, hidden -1, all-ones input and
// dout -- on the engine's device, plus what the drop-in adds: counts sum to
// N*k, outputs finite, parameter gradients present, errors as exceptions.
int shapes() {
  const int B = 2, T = 4, C = 16, E = 4, k = 2;
  MoELayer moe(C, -1, E, k);
  if (moe.get_parameters().size() != (size_t)(2 + 6 * E)) return fail("parameter count");
  if (moe.get_parameters()[2]->shape != std::vector<int>({C, 4 * C})) return fail("hidden -1 -> 4C");
  moe.to(dev());
  Tensor x({B, T, C}, 1.0f, dev());
  Tensor y = moe.forward(x);
  if (y.shape != std::vector<int>({B, T, C})) return fail("output shape");
  float total = 0;
  for (float c : moe.get_expert_counts()) total += c;
  if (total != (float)(B * T * k)) return fail("counts sum");
  const std::vector<float> yh = host_values(y);
  for (float v : yh)
    if (!std::isfinite(v)) return fail("finite output");
  Tensor out2;
  moe.forward_into(x, out2);
  if (host_values(out2) != yh) return fail("forward_into repeatable");
  if (moe.get_footprint(B, T).fwd_standing == 0) return fail("footprint");
  // moeTests.cpp:22-39: dout = 1, din keeps the input's shape
  Tensor dout({B, T, C}, 1.0f, dev());
  moe.forward(x);
  Tensor din = moe.backward(dout);
  if (din.shape != std::vector<int>({B, T, C})) return fail("din shape");
  for (float v : host_values(din))
    if (!std::isfinite(v)) return fail("finite din");
  double gsum = 0;
  for (Tensor* p : moe.get_parameters())
    for (float v : host_grad(*p)) gsum += std::fabs(v);
  if (!(gsum > 0) || !std::isfinite(gsum)) return fail("parameter gradients");
  bool threw = false;
  try {
    Tensor bad({B, T + 1, C}, 1.0f, dev());
    moe.backward(bad);
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  if (!threw) return fail("dout shape mismatch must throw");
  threw = false;
  try {
    Tensor bad({B, T, C + 64}, 0.0f, dev());
    moe.forward(bad);
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  if (!threw) return fail("shape mismatch must throw");
  // an inference forward keeps no caches: a backward after it must throw
  moe.set_inference(true);
  moe.forward(x);
  threw = false;
  try {
    moe.backward(dout);
  } catch (const std::runtime_error&) {
    threw = true;
  }
  if (!threw) return fail("backward after an inference forward must throw");
  std::printf("shapes ok (%s)\n", kDevice ? "device tensors" : "host tensors");
  return 0;
}

#ifdef DROPIN_DEVICE
int decode(const char* x_path, const char* r_path, uint64_t seed, int C, int H, int E, int k,
           int steps, double spin_ms, const char* out_path) {
  FILE* f = std::fopen(x_path, "rb");
  if (!f) { std::perror(x_path); return 2; }
  std::vector<float> xv;
  float v;
  while (std::fread(&v, sizeof(float), 1, f) == 1) xv.push_back(v);
  std::fclose(f);
  const int N = (int)(xv.size() / C);
  MoELayer moe(C, H, E, k);
  std::vector<Tensor*> params = moe.get_parameters();
  f = std::fopen(r_path, "rb");
  if (!f) { std::perror(r_path); return 2; }
  if (!read_exact(f, params[0]->get_data_ptr(), sizeof(float) * params[0]->size()) ||
      !read_exact(f, params[1]->get_data_ptr(), sizeof(float) * params[1]->size()))
    return 2;
  std::fclose(f);
  // mgpt_amd/workload.py make_expert: stream 100 + 8e + {0: W_g, 1: W_u, 2: W_d}
  for (int e = 0; e < E; ++e) {
    Tensor** p = &params[2 + 6 * e];
    mgpt_wl_normal_f32(seed, 100 + 8 * e + 0, 0, (int64_t)C * H, 0.02, p[0]->get_data_ptr());
    mgpt_wl_normal_f32(seed, 100 + 8 * e + 1, 0, (int64_t)C * H, 0.02, p[2]->get_data_ptr());
    mgpt_wl_normal_f32(seed, 100 + 8 * e + 2, 0, (int64_t)H * C, 0.02, p[4]->get_data_ptr());
    p[1]->fill(0.0f);
    p[3]->fill(0.0f);
    p[5]->fill(0.0f);
  }
  moe.set_expert_dtype(MGPT_DTYPE_FP8_E4M3);
  moe.set_inference(true);
  moe.to(Device::CUDA);
  Scratchpad pad(moe.get_footprint(1, N).fwd_peak() + 64, ScratchpadDevice::CUDA);
  moe.set_scratchpad(&pad);
  Tensor x = on_device({1, N, C}, xv.data());
  Tensor y({1, N, C}, 0.0f, Device::CUDA);
  moe.forward_into(x, y);   // first call: packs and quantises the weights
  cuda_ops::synchronize();
  // the sampling loop's steps, enqueued behind a device spin: a host wait or
  // a synchronous copy inside a step would hold the host until the spin ends
  engine_test_spin(spin_ms);
  const auto t0 = std::chrono::steady_clock::now();
  for (int s = 0; s < steps; ++s) {
    pad.reset();
    moe.forward_into(x, y);
  }
  const auto t1 = std::chrono::steady_clock::now();
  cuda_ops::synchronize();
  const float enqueue_ms = std::chrono::duration<float, std::milli>(t1 - t0).count();
  const std::vector<float> yh = host_values(y);
  FILE* o = std::fopen(out_path, "wb");
  if (!o) { std::perror(out_path); return 2; }
  const int32_t hdr[2] = {N, C};
  std::fwrite("MGPTDEC1", 1, 8, o);
  std::fwrite(hdr, sizeof(int32_t), 2, o);
  std::fwrite(&enqueue_ms, sizeof(float), 1, o);
  std::fwrite(yh.data(), sizeof(float), yh.size(), o);
  std::fclose(o);
  std::printf("decode: %d steps enqueued in %.3f ms behind a %.0f ms spin\n", steps, enqueue_ms,
              spin_ms);
  return 0;
}
#endif

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc == 4 && std::strcmp(argv[1], "run") == 0) return run(argv[2], argv[3]);
    if (argc == 2 && std::strcmp(argv[1], "shapes") == 0) return shapes();
    if (argc == 5 && std::strcmp(argv[1], "backward") == 0) return backward(argv[2], argv[3], argv[4]);
    if (argc == 7 && std::strcmp(argv[1], "train") == 0)
      return train(argv[2], argv[3], argv[4], std::atoi(argv[5]), (float)std::atof(argv[6]));
#ifdef DROPIN_DEVICE
    if (argc == 12 && std::strcmp(argv[1], "decode") == 0)
      return decode(argv[2], argv[3], std::strtoull(argv[4], nullptr, 10), std::atoi(argv[5]),
                    std::atoi(argv[6]), std::atoi(argv[7]), std::atoi(argv[8]),
                    std::atoi(argv[9]), std::atof(argv[10]), argv[11]);
#endif
  } catch (const std::exception& e) {
    std::fprintf(stderr, "exception: %s\n", e.what());
    return 3;
  }
  std::fprintf(stderr,
               "usage: dropin_main run <in> <out> | backward <in> <dy> <grad> | "
               "train <in> <dy> <out> <steps> <lr> | shapes | decode ...\n");
  return 2;
}
