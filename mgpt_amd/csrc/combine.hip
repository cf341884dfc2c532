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
// built with -ffp-contract=off), reading 16 bytes per lane per row chunk.
#include "common.hpp"

namespace mgpt {
namespace {

template <typename ActT>
struct Vec16;
template <>
struct Vec16<bf16_t> {
  static constexpr int n = 8;
  static __device__ __forceinline__ void unpack(const uint4 u, float (&v)[8]) {
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
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    u.x = w[0]; u.y = w[1]; u.z = w[2]; u.w = w[3];
    *reinterpret_cast<uint4*>(p) = u;
  }
};
template <>
struct Vec16<float> {
  static constexpr int n = 4;
  static __device__ __forceinline__ void unpack(const uint4 u, float (&v)[4]) {
    v[0] = __uint_as_float(u.x);
    v[1] = __uint_as_float(u.y);
    v[2] = __uint_as_float(u.z);
    v[3] = __uint_as_float(u.w);
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

// VN consecutive values of the output or residual type (VN = the values of
// one 16-byte chunk of expert rows: 8 for bf16 rows, 4 for fp32 rows).
template <typename T, int VN>
struct OutVec;
template <int VN>
struct OutVec<bf16_t, VN> {
  static_assert(VN == 8, "bf16 outputs come from bf16 rows");
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[VN]) {
    Vec16<bf16_t>::unpack(*reinterpret_cast<const uint4*>(p), v);
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[VN]) {
    Vec16<bf16_t>::store(p, v);
  }
};
template <int VN>
struct OutVec<float, VN> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[VN]) {
#pragma unroll
    for (int i = 0; i < VN; i += 4) {
      const float4 f = *reinterpret_cast<const float4*>(p + i);
      v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
    }
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[VN]) {
#pragma unroll
    for (int i = 0; i < VN; i += 4)
      *reinterpret_cast<float4*>(p + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
  }
};

// Fused block: y = x1 + the MoE sum (Tensor::add_into, utils/Tensor.cpp:
// 1579-1597, after the scatter), one rounded add per element.
template <typename T, int VN>
__device__ __forceinline__ void add_resid(const T* p, float (&v)[VN]) {
  float x[VN];
  OutVec<T, VN>::load(p, x);
#pragma unroll
  for (int i = 0; i < VN; ++i) v[i] = x[i] + v[i];
}

constexpr int kWavesPerBlock = 4;
// Tokens per wave of the k = 2 kernel.  Measured on MI355X at cfg3 shapes:
// 1 token (20.3 us) beats 2 (20.8 us); the extra loads in flight do not pay
// for the halved wave count.
constexpr int kTokensPerWave2 = 1;

// Each wave combines TPW consecutive tokens.  KT choices per token (0: the
// runtime k, one row at a time) and CH 16-byte chunks per lane and row.
// With KT fixed, all TPW * KT * CH chunk loads of a wave are issued before
// any is used, so each wave keeps them all in flight.
template <typename ActT, typename OutT, int TPW, int KT, int CH>
__global__ __launch_bounds__(256) void combine_kernel(const ActT* __restrict__ out_rows,
                                                      const int32_t* __restrict__ topk_idx,
                                                      const float* __restrict__ topk_p,
                                                      const int32_t* __restrict__ slot_of, int N,
                                                      int C, int k, const OutT* __restrict__ resid,
                                                      OutT* __restrict__ y) {
  static_assert(TPW * kMaxTopK <= kWave, "one lane per (token, choice)");
  __shared__ int s_slot[kWavesPerBlock][TPW][kMaxTopK];
  __shared__ float s_p[kWavesPerBlock][TPW][kMaxTopK];
  if constexpr (KT > 0) k = KT;
  const int w = threadIdx.x / kWave;
  const int l = lane_id();
  const int t0 = (blockIdx.x * kWavesPerBlock + w) * TPW;
  if (t0 >= N) return;   // whole wave exits together; no block barrier below
  {
    // lane u * kMaxTopK + j: choice j of token t0 + u
    const int u = l / kMaxTopK, j = l % kMaxTopK, t = t0 + u;
    if (u < TPW && j < k && t < N) {
      const int e = topk_idx[(size_t)t * k + j];
      // rank of this choice among the token's k choices by expert id
      int rank = 0;
      for (int i = 0; i < k; ++i) {
        const int ei = topk_idx[(size_t)t * k + i];
        rank += (ei < e) || (ei == e && i < j);
      }
      s_slot[w][u][rank] = slot_of[(size_t)t * k + j];
      s_p[w][u][rank] = topk_p[(size_t)t * k + j];
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int VN = Vec16<ActT>::n;
  for (int c0 = 0; c0 < C; c0 += kWave * VN * CH) {
    float acc[TPW][CH][VN];
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
      for (int ch = 0; ch < CH; ++ch)
#pragma unroll
        for (int i = 0; i < VN; ++i) acc[u][ch][i] = 0.0f;
    auto add_row = [&](int u, const uint4 (&raw)[CH], float p) __attribute__((always_inline)) {
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) {
        float v[VN];
        Vec16<ActT>::unpack(raw[ch], v);
#pragma unroll
        for (int i = 0; i < VN; ++i) acc[u][ch][i] = acc[u][ch][i] + v[i] * p;
      }
    };
    auto load_row = [&](int u, int a, uint4 (&raw)[CH]) __attribute__((always_inline)) {
      const ActT* src = out_rows + (size_t)s_slot[w][u][a] * C;
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) {
        const int c = c0 + (ch * kWave + l) * VN;
        raw[ch] = c < C ? *reinterpret_cast<const uint4*>(src + c) : make_uint4(0, 0, 0, 0);
      }
    };
    const int nt = min(TPW, N - t0);
    if constexpr (KT > 0) {
      uint4 raw[TPW][KT][CH];
#pragma unroll
      for (int u = 0; u < TPW; ++u)
        if (u < nt)
#pragma unroll
          for (int a = 0; a < KT; ++a) load_row(u, a, raw[u][a]);
#pragma unroll
      for (int u = 0; u < TPW; ++u)
        if (u < nt)
#pragma unroll
          for (int a = 0; a < KT; ++a) add_row(u, raw[u][a], s_p[w][u][a]);
    } else {
      for (int u = 0; u < nt; ++u)
        for (int a = 0; a < k; ++a) {
          uint4 raw[CH];
          load_row(u, a, raw);
          add_row(u, raw, s_p[w][u][a]);
        }
    }
#pragma unroll
    for (int u = 0; u < TPW; ++u)
      if (u < nt)
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
          const int c = c0 + (ch * kWave + l) * VN;
          if (c < C) {
            if (resid) add_resid<OutT, VN>(resid + (size_t)(t0 + u) * C + c, acc[u][ch]);
            OutVec<OutT, VN>::store(y + (size_t)(t0 + u) * C + c, acc[u][ch]);
          }
        }
  }
}

// k = 2: each wave combines TPW tokens whose two choices come from
// wave-uniform (scalar) loads of slot_of / topk_p; no LDS, no rank loop.  The
// rows are added in ascending slot order, which is ascending expert id:
// slots are expert-major and a token's choices are distinct experts.  All
// TPW * 2 * CH chunk loads are issued before any is used.
template <typename ActT, typename OutT, int TPW, int CH>
__global__ __launch_bounds__(256) void combine2_kernel(const ActT* __restrict__ out_rows,
                                                       const float* __restrict__ topk_p,
                                                       const int32_t* __restrict__ slot_of, int N,
                                                       int C, const OutT* __restrict__ resid,
                                                       OutT* __restrict__ y) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int l = lane_id();
  const int t0 = (blockIdx.x * kWavesPerBlock + w) * TPW;
  if (t0 >= N) return;
  const int nt = min(TPW, N - t0);
  int sl[TPW][2];
  float pr[TPW][2];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int t = min(t0 + u, N - 1);
    int s0 = __builtin_amdgcn_readfirstlane(slot_of[2 * t]);
    int s1 = __builtin_amdgcn_readfirstlane(slot_of[2 * t + 1]);
    float p0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(topk_p[2 * t])));
    float p1 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(topk_p[2 * t + 1])));
    if (s1 < s0) {
      const int ts = s0; s0 = s1; s1 = ts;
      const float tp = p0; p0 = p1; p1 = tp;
    }
    sl[u][0] = s0; sl[u][1] = s1;
    pr[u][0] = p0; pr[u][1] = p1;
  }
  constexpr int VN = Vec16<ActT>::n;
  for (int c0 = 0; c0 < C; c0 += kWave * VN * CH) {
    uint4 raw[TPW][2][CH];
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const ActT* src = out_rows + (size_t)sl[u][a] * C;
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
          const int c = c0 + (ch * kWave + l) * VN;
          raw[u][a][ch] = (c < C && u < nt) ? *reinterpret_cast<const uint4*>(src + c)
                                            : make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) {
        float acc[VN], v[VN];
#pragma unroll
        for (int i = 0; i < VN; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          Vec16<ActT>::unpack(raw[u][a][ch], v);
#pragma unroll
          for (int i = 0; i < VN; ++i) acc[i] = acc[i] + v[i] * pr[u][a];
        }
        const int c = c0 + (ch * kWave + l) * VN;
        if (c < C && u < nt) {
          if (resid) add_resid<OutT, VN>(resid + (size_t)(t0 + u) * C + c, acc);
          OutVec<OutT, VN>::store(y + (size_t)(t0 + u) * C + c, acc);
        }
      }
  }
}

template <typename ActT, typename OutT, int TPW, int KT>
void launch_combine_k(int chunks, hipStream_t stream, const ActT* out_rows,
                      const int32_t* topk_idx, const float* topk_p, const int32_t* slot_of, int N,
                      int C, int k, const OutT* resid, OutT* y) {
  const dim3 grid((N + kWavesPerBlock * TPW - 1) / (kWavesPerBlock * TPW));
  if (chunks >= 2)
    hipLaunchKernelGGL((combine_kernel<ActT, OutT, TPW, KT, 2>), grid, dim3(256), 0, stream,
                       out_rows, topk_idx, topk_p, slot_of, N, C, k, resid, y);
  else
    hipLaunchKernelGGL((combine_kernel<ActT, OutT, TPW, KT, 1>), grid, dim3(256), 0, stream,
                       out_rows, topk_idx, topk_p, slot_of, N, C, k, resid, y);
}

}  // namespace

// resid (nullable): the fused block's residual, y = resid + sum.  ActT: the
// expert rows; OutT: y and resid (fp32 outputs of bf16 rows keep the fp32
// sum unrounded).
template <typename ActT, typename OutT>
hipError_t launch_combine(const ActT* out_rows, const int32_t* topk_idx, const float* topk_p,
                          const int32_t* slot_of, int N, int C, int k, const OutT* resid, OutT* y,
                          hipStream_t stream) {
  if (N == 0) return hipSuccess;
  if (k < 1 || k > kMaxTopK) return hipErrorInvalidValue;
  const int per_chunk = kWave * Vec16<ActT>::n;   // elements one chunk covers
  const int chunks = (C + per_chunk - 1) / per_chunk;
  switch (k) {
    case 2: {
      const dim3 grid((N + kWavesPerBlock * kTokensPerWave2 - 1) /
                      (kWavesPerBlock * kTokensPerWave2));
      if (chunks >= 2)
        hipLaunchKernelGGL((combine2_kernel<ActT, OutT, kTokensPerWave2, 2>), grid, dim3(256), 0,
                           stream, out_rows, topk_p, slot_of, N, C, resid, y);
      else
        hipLaunchKernelGGL((combine2_kernel<ActT, OutT, kTokensPerWave2, 1>), grid, dim3(256), 0,
                           stream, out_rows, topk_p, slot_of, N, C, resid, y);
      break;
    }
    // fixed k: every row chunk of a token in flight at once
    case 6:
      launch_combine_k<ActT, OutT, 1, 6>(chunks, stream, out_rows, topk_idx, topk_p, slot_of, N,
                                         C, k, resid, y);
      break;
    case 8:
      launch_combine_k<ActT, OutT, 1, 8>(chunks, stream, out_rows, topk_idx, topk_p, slot_of, N,
                                         C, k, resid, y);
      break;
    default:
      launch_combine_k<ActT, OutT, 1, 0>(chunks, stream, out_rows, topk_idx, topk_p, slot_of, N,
                                         C, k, resid, y);
  }
  return hipGetLastError();
}

template hipError_t launch_combine<float, float>(const float*, const int32_t*, const float*,
                                                 const int32_t*, int, int, int, const float*,
                                                 float*, hipStream_t);
template hipError_t launch_combine<bf16_t, bf16_t>(const bf16_t*, const int32_t*, const float*,
                                                   const int32_t*, int, int, int, const bf16_t*,
                                                   bf16_t*, hipStream_t);
template hipError_t launch_combine<bf16_t, float>(const bf16_t*, const int32_t*, const float*,
                                                  const int32_t*, int, int, int, const float*,
                                                  float*, hipStream_t);

}  // namespace mgpt
