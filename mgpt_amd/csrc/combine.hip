// combine.hip -- gate-weighted sum of the expert outputs back to token order.
//
// Reference: zero-filled output (layers/MoELayer.cpp:121-122) and the CPU
// scatter utils/Tensor.cpp:1385-1408, which walks slots in ascending order
// and does y[i/k] += out[slot] * p[i].  Slots are expert-major, so each
// token's k contributions are added in ascending expert id, each as a
// rounded product followed by a rounded add onto a sum that starts at 0.
// This kernel gathers instead of scattering (no atomics, deterministic):
// one wave per token sorts its k choices by expert id and accumulates the
// k rows in that order with the same two roundings per term (the file is
// built with -ffp-contract=off), reading 16 bytes per lane per row.
#include "common.hpp"

namespace mgpt {
namespace {

template <typename ActT>
struct Vec16;
template <>
struct Vec16<bf16_t> {
  static constexpr int n = 8;
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[8]) {
    uint4 u;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
    u.x = w[0]; u.y = w[1]; u.z = w[2]; u.w = w[3];
    *reinterpret_cast<uint4*>(p) = u;
  }
};
template <>
struct Vec16<float> {
  static constexpr int n = 4;
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

constexpr int kTokPerBlock = 4;   // one wave per token

template <typename ActT>
__global__ __launch_bounds__(256) void combine_kernel(const ActT* __restrict__ out_rows,
                                                      const int32_t* __restrict__ topk_idx,
                                                      const float* __restrict__ topk_p,
                                                      const int32_t* __restrict__ slot_of, int N,
                                                      int C, int k, ActT* __restrict__ y) {
  __shared__ int s_slot[kTokPerBlock][kMaxTopK];
  __shared__ float s_p[kTokPerBlock][kMaxTopK];
  const int w = threadIdx.x / kWave;
  const int l = lane_id();
  const int t = blockIdx.x * kTokPerBlock + w;
  if (t >= N) return;   // whole wave exits together; no block barrier below
  if (l < k) {
    const int e = topk_idx[(size_t)t * k + l];
    // rank of this choice among the token's k choices by expert id
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      const int ej = topk_idx[(size_t)t * k + j];
      rank += (ej < e) || (ej == e && j < l);
    }
    s_slot[w][rank] = slot_of[(size_t)t * k + l];
    s_p[w][rank] = topk_p[(size_t)t * k + l];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int VN = Vec16<ActT>::n;
  for (int c = l * VN; c < C; c += kWave * VN) {
    float acc[VN];
#pragma unroll
    for (int i = 0; i < VN; ++i) acc[i] = 0.0f;
    for (int a = 0; a < k; ++a) {
      float v[VN];
      Vec16<ActT>::load(out_rows + (size_t)s_slot[w][a] * C + c, v);
      const float p = s_p[w][a];
#pragma unroll
      for (int i = 0; i < VN; ++i) acc[i] = acc[i] + v[i] * p;
    }
    Vec16<ActT>::store(y + (size_t)t * C + c, acc);
  }
}

}  // namespace

template <typename ActT>
hipError_t launch_combine(const ActT* out_rows, const int32_t* topk_idx, const float* topk_p,
                          const int32_t* slot_of, int N, int C, int k, ActT* y,
                          hipStream_t stream) {
  if (N == 0) return hipSuccess;
  const int nb = (N + kTokPerBlock - 1) / kTokPerBlock;
  hipLaunchKernelGGL(combine_kernel<ActT>, dim3(nb), dim3(256), 0, stream, out_rows, topk_idx,
                     topk_p, slot_of, N, C, k, y);
  return hipGetLastError();
}

template hipError_t launch_combine<float>(const float*, const int32_t*, const float*,
                                          const int32_t*, int, int, int, float*, hipStream_t);
template hipError_t launch_combine<bf16_t>(const bf16_t*, const int32_t*, const float*,
                                           const int32_t*, int, int, int, bf16_t*, hipStream_t);

}  // namespace mgpt
