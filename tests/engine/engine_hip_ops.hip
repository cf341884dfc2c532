// engine_hip_ops.hip -- the engine's device-memory primitives over HIP.
//
// TEST INFRASTRUCTURE.  The engine's Tensor, Scratchpad and AdamW reach
// device memory only through these cuda_ops functions
// (src/main/utils/cuda_ops.h:7-110): allocation, copies, fill, the add of
// Tensor::add_grad and the AdamW update.  The engine's CPU build defines
// them as no-ops (utils/cuda_ops.cu:2009-2079), so its Device::CUDA tensors
// hold no memory.  Linked in place of that file, these definitions give
// tests/engine/_build/dropin_dev real device tensors, so the drop-in
// MoELayer runs its Device::CUDA and Scratchpad branches and the engine's
// AdamWOptimizer::step updates device parameters between forwards.  No other
// cuda_ops function is defined: the engine paths these tests take call none.
//
// adamw_step restates the update of the engine's CPU branch,
// Tensor::adamw_step (utils/Tensor.cpp:683-701), element for element.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <stdexcept>
#include <string>

namespace {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

__global__ void fill_kernel(float* p, float v, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void add_kernel(const float* a, const float* b, float* c, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    c[i] = a[i] + b[i];
}

__global__ void adamw_kernel(float* p, const float* g, float* m, float* v, float lr, float b1,
                             float b2, float eps, float wd, float m_scale, float v_scale,
                             size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float gi = g[i];
    const float mi = b1 * m[i] + (1.0f - b1) * gi;
    const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const float m_hat = mi * m_scale;
    const float v_hat = vi * v_scale;
    float x = p[i];
    x -= lr * wd * x;
    x -= lr * m_hat / (__fsqrt_rn(v_hat) + eps);
    p[i] = x;
  }
}

// Keeps the device busy for `cycles` ticks of the constant-rate wall clock
// and then exits (a bounded wait: the loop ends after the given time).
__global__ void spin_kernel(unsigned long long cycles) {
  const unsigned long long t0 = wall_clock64();
  while (wall_clock64() - t0 < cycles) __builtin_amdgcn_s_sleep(8);
}

dim3 grid_for(size_t n) {
  size_t b = (n + 255) / 256;
  return dim3((unsigned)(b < 4096 ? (b ? b : 1) : 4096));
}

}  // namespace

namespace cuda_ops {

void synchronize() { hip_check(hipDeviceSynchronize(), "synchronize"); }

void allocate_memory(float** ptr, size_t size) {
  if (size == 0) {
    *ptr = nullptr;
    return;
  }
  hip_check(hipMalloc((void**)ptr, size * sizeof(float)), "hipMalloc");
}

void free_memory(float* ptr) {
  if (ptr) hip_check(hipFree(ptr), "hipFree");
}

void copy_host_to_device(float* dst, const float* src, size_t size) {
  if (size == 0 || !dst || !src) return;
  hip_check(hipMemcpy(dst, src, size * sizeof(float), hipMemcpyHostToDevice), "copy H2D");
}

void copy_device_to_host(float* dst, const float* src, size_t size) {
  if (size == 0 || !dst || !src) return;
  hip_check(hipMemcpy(dst, src, size * sizeof(float), hipMemcpyDeviceToHost), "copy D2H");
}

void copy_device_to_device(float* dst, const float* src, size_t size) {
  if (size == 0 || !dst || !src) return;
  hip_check(hipMemcpy(dst, src, size * sizeof(float), hipMemcpyDeviceToDevice), "copy D2D");
}

void fill(float* ptr, float val, size_t size) {
  if (size == 0 || !ptr) return;
  hipLaunchKernelGGL(fill_kernel, grid_for(size), dim3(256), 0, nullptr, ptr, val, size);
  hip_check(hipGetLastError(), "fill");
}

void add(const float* A, const float* B, float* C, size_t size) {
  if (size == 0) return;
  hipLaunchKernelGGL(add_kernel, grid_for(size), dim3(256), 0, nullptr, A, B, C, size);
  hip_check(hipGetLastError(), "add");
}

void adamw_step(float* param, const float* grad, float* m, float* v, float lr, float beta1,
                float beta2, float eps, float weight_decay, int t, size_t size) {
  if (size == 0) return;
  // the bias corrections as the CPU branch forms them (in float, std::pow)
  const float m_scale = 1.0f / (1.0f - std::pow(beta1, (float)t));
  const float v_scale = 1.0f / (1.0f - std::pow(beta2, (float)t));
  hipLaunchKernelGGL(adamw_kernel, grid_for(size), dim3(256), 0, nullptr, param, grad, m, v, lr,
                     beta1, beta2, eps, weight_decay, m_scale, v_scale, size);
  hip_check(hipGetLastError(), "adamw_step");
}

}  // namespace cuda_ops

// Test hook: occupies the default stream for about `ms` milliseconds.
extern "C" void engine_test_spin(double ms) {
  int khz = 0;
  hip_check(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0), "wall clock rate");
  const unsigned long long cycles = (unsigned long long)(ms * (double)khz);
  hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(1), 0, nullptr, cycles);
  hip_check(hipGetLastError(), "spin");
}
