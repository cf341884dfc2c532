// backward.hip -- the non-GEMM stages of the MoE block backward.
//
// Reference: MoELayer::backward_into (layers/MoELayer.cpp:130-223), CPU
// branches of the tensor ops it calls (utils/Tensor.cpp):
//   scatter_bwd   moe_scatter_backward :1410-1438: per slot,
//                 dgo[slot] = dy[t] * p and dp[t*k+j] = <y_e[slot], dy[t]>
//   token_bwd     scatter_indices_into :1462-1484 + the load-balance term
//                 (layers/MoELayer.cpp:193-200) + softmax_backward :885-905
//                 on the clamped probabilities, then per token
//                 dx = sum over its slots (ascending) of dX_e (the gather
//                 backward :1440-1460) + dL . W_r^T (router
//                 LinearLayer::backward_into, layers/LinearLayer.cpp:33-80)
//   router_wgrad  dW_r += x^T . dL, db_r += sum_t dL (same Linear backward):
//                 per-chunk partial sums, then an in-order reduction, so the
//                 result does not depend on scheduling
//   transpose_pad the forward's packed weights, transposed per expert into
//                 the layouts the data-gradient products read.
#include "common.hpp"

namespace mgpt {
namespace {

// 16 bytes of activations: 8 bf16 or 4 fp32, widened / narrowed.
template <typename ActT> struct Vec;
template <> struct Vec<bf16_t> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(const uint4& q, float (&v)[8]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
  static __device__ __forceinline__ uint4 pack(const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct Vec<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void unpack(const uint4& q, float (&v)[4]) {
    v[0] = __uint_as_float(q.x);
    v[1] = __uint_as_float(q.y);
    v[2] = __uint_as_float(q.z);
    v[3] = __uint_as_float(q.w);
  }
  static __device__ __forceinline__ uint4 pack(const float (&v)[4]) {
    return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                      __float_as_uint(v[3]));
  }
};

// One wave per slot: dgo row = dy row * p, and the dot of the expert output
// row with the dy row (fp32, reduced across the wave).
template <typename ActT>
__global__ __launch_bounds__(256) void scatter_bwd_kernel(
    const ActT* __restrict__ dy, const ActT* __restrict__ ye, const int32_t* __restrict__ perm,
    const float* __restrict__ topk_p, int A, int C, int k, ActT* __restrict__ dgo,
    float* __restrict__ dtp) {
  using V = Vec<ActT>;
  const int slot = blockIdx.x * 4 + (int)(threadIdx.x / kWave);
  if (slot >= A) return;
  const int lane = lane_id();
  const int flat = perm[slot];
  const int t = flat / k;
  const float p = topk_p[flat];
  const uint4* d4 = reinterpret_cast<const uint4*>(dy + (size_t)t * C);
  const uint4* y4 = reinterpret_cast<const uint4*>(ye + (size_t)slot * C);
  uint4* o4 = reinterpret_cast<uint4*>(dgo + (size_t)slot * C);
  float dot = 0.0f;
  for (int i = lane; i < C / V::N; i += kWave) {
    float d[V::N], y[V::N], o[V::N];
    V::unpack(d4[i], d);
    V::unpack(y4[i], y);
#pragma unroll
    for (int q = 0; q < V::N; ++q) {
      o[q] = d[q] * p;
      dot += y[q] * d[q];
    }
    o4[i] = V::pack(o);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) dot += __shfl_xor(dot, m, kWave);
  if (lane == 0) dtp[flat] = dot;
}

constexpr int kTokBlock = 16;   // tokens per token_bwd block

// dL and dx of kTokBlock tokens.  Phase 1 (one thread per token): dP from
// the top-k entries and the load-balance term, s = sum_e dP*P in expert
// order, dL = P*(dP - s), the token's slots sorted ascending.  Phase 2 (a
// thread per 4 columns): the slot rows of dX_e summed in slot order, plus
// dL . W_r^T with W_r read from the router's packed [G][C][RE] layout.
template <typename ActT>
__global__ __launch_bounds__(256) void token_bwd_kernel(
    const ActT* __restrict__ dxe, const int32_t* __restrict__ slot_of,
    const int32_t* __restrict__ topk_idx, const float* __restrict__ dtp,
    const float* __restrict__ probs, const int32_t* __restrict__ counts,
    const float* __restrict__ wr_g, int RE, int N, int C, int E, int k,
    ActT* __restrict__ dx, float* __restrict__ dL) {
  __shared__ float s_dl[kTokBlock][kMaxExperts];
  __shared__ float s_lb[kMaxExperts];
  __shared__ int s_slot[kTokBlock][kMaxTopK];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * kTokBlock;
  if (tid < E) {
    // (alpha * E * f_e) / N with f_e = counts_e / N, alpha = 0.01
    const float fe = (float)counts[tid] / (float)N;
    s_lb[tid] = (0.01f * (float)E * fe) / (float)N;
  }
  __syncthreads();
  if (tid < kTokBlock && t0 + tid < N) {
    const int t = t0 + tid;
    float* d = s_dl[tid];
    for (int e = 0; e < E; ++e) d[e] = 0.0f;
    int* sl = s_slot[tid];
    for (int j = 0; j < k; ++j) {
      d[topk_idx[(size_t)t * k + j]] = dtp[(size_t)t * k + j];
      sl[j] = slot_of[(size_t)t * k + j];
    }
    const float* P = probs + (size_t)t * E;
    float s = 0.0f;
    for (int e = 0; e < E; ++e) {
      d[e] = d[e] + s_lb[e];
      s += d[e] * P[e];
    }
    for (int e = 0; e < E; ++e) {
      const float v = P[e] * (d[e] - s);
      d[e] = v;
      dL[(size_t)t * E + e] = v;
    }
    for (int a = 1; a < k; ++a) {   // insertion sort of the slots (in LDS)
      const int v = sl[a];
      int b = a;
      while (b > 0 && sl[b - 1] > v) {
        sl[b] = sl[b - 1];
        --b;
      }
      sl[b] = v;
    }
  }
  __syncthreads();
  const int nt = min(kTokBlock, N - t0);
  for (int cq = tid; cq < C / 4; cq += blockDim.x) {
    const int c = 4 * cq;
    float acc[kTokBlock][4];
#pragma unroll
    for (int r = 0; r < kTokBlock; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[r][q] = 0.0f;
    // router term, experts in ascending order
    for (int e = 0; e < E; ++e) {
      const float* wp = wr_g + ((size_t)(e / RE) * C + c) * RE + (e % RE);
      const float w0 = wp[0], w1 = wp[RE], w2 = wp[2 * RE], w3 = wp[3 * RE];
#pragma unroll
      for (int r = 0; r < kTokBlock; ++r) {
        const float g = s_dl[r][e];
        acc[r][0] += g * w0;
        acc[r][1] += g * w1;
        acc[r][2] += g * w2;
        acc[r][3] += g * w3;
      }
    }
#pragma unroll
    for (int r = 0; r < kTokBlock; ++r) {
      if (r < nt) {
        float gsum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j = 0; j < k; ++j) {
          const ActT* src = dxe + (size_t)s_slot[r][j] * C + c;
#pragma unroll
          for (int q = 0; q < 4; ++q) gsum[q] += to_f32(src[q]);
        }
        ActT* o = dx + (size_t)(t0 + r) * C + c;
#pragma unroll
        for (int q = 0; q < 4; ++q) store_act(o + q, gsum[q] + acc[r][q]);
      }
    }
  }
}

constexpr int kRwChunk = 256;   // tokens per router_wgrad partial

// partial[chunk][c][e] = sum over the chunk's tokens of x[t][c] * dL[t][e]
// (a thread per column, EP >= E experts in registers, dL rows read from LDS
// as float4 broadcasts), and in the blocks of the first column range
// partial_b[chunk][e] = sum_t dL[t][e].
template <typename ActT, int EP>
__global__ __launch_bounds__(256) void router_wgrad_kernel(const ActT* __restrict__ x,
                                                           const float* __restrict__ dL, int N,
                                                           int C, int E,
                                                           float* __restrict__ partial,
                                                           float* __restrict__ partial_b) {
  __shared__ float4 s_dl[64][EP / 4];
  const int tid = threadIdx.x;
  const int chunk = blockIdx.y;
  const int c = blockIdx.x * 256 + tid;
  const int t_begin = chunk * kRwChunk, t_end = min(N, t_begin + kRwChunk);
  float acc[EP];
#pragma unroll
  for (int e = 0; e < EP; ++e) acc[e] = 0.0f;
  float bsum = 0.0f;
  for (int tb = t_begin; tb < t_end; tb += 64) {
    const int nt = min(64, t_end - tb);
    __syncthreads();
    float* sl = reinterpret_cast<float*>(s_dl);
    for (int p = tid; p < 64 * EP; p += 256) {
      const int r = p / EP, e = p % EP;
      sl[p] = (r < nt && e < E) ? dL[(size_t)(tb + r) * E + e] : 0.0f;
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid < E)
      for (int r = 0; r < nt; ++r) bsum += sl[r * EP + tid];
    if (c < C) {
      for (int r = 0; r < nt; ++r) {
        const float xv = to_f32(x[(size_t)(tb + r) * C + c]);
#pragma unroll
        for (int e4 = 0; e4 < EP / 4; ++e4) {
          const float4 d = s_dl[r][e4];
          acc[4 * e4 + 0] += xv * d.x;
          acc[4 * e4 + 1] += xv * d.y;
          acc[4 * e4 + 2] += xv * d.z;
          acc[4 * e4 + 3] += xv * d.w;
        }
      }
    }
  }
  if (c < C) {
    float* o = partial + ((size_t)chunk * C + c) * E;
#pragma unroll
    for (int e = 0; e < EP; ++e)
      if (e < E) o[e] = acc[e];
  }
  if (blockIdx.x == 0 && tid < E) partial_b[(size_t)chunk * E + tid] = bsum;
}

// grad[i] += sum over chunks (in order) of partial[chunk][i], for the C*E
// weight entries followed by the E bias entries.
__global__ __launch_bounds__(256) void router_wgrad_reduce_kernel(
    const float* __restrict__ partial, const float* __restrict__ partial_b, int chunks, int CE,
    int E, float* __restrict__ gW, float* __restrict__ gb) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < CE) {
    float s = 0.0f;
    for (int ch = 0; ch < chunks; ++ch) s += partial[(size_t)ch * CE + i];
    gW[i] = gW[i] + s;
  } else if (i < CE + E) {
    const int e = i - CE;
    float s = 0.0f;
    for (int ch = 0; ch < chunks; ++ch) s += partial_b[(size_t)ch * E + e];
    gb[e] = gb[e] + s;
  }
}

// dst[e][r][c] = src[e][c][r] for r < src_cols and c < src_rows, else 0,
// for r < dst_rows and c < dst_cols, through a 64 x 64 LDS tile.
template <typename T>
__global__ __launch_bounds__(256) void transpose_pad_kernel(const T* __restrict__ src,
                                                            int src_rows, int src_cols,
                                                            size_t src_estride,
                                                            T* __restrict__ dst, int dst_rows,
                                                            int dst_cols, size_t dst_estride) {
  __shared__ T tile[64][65];
  const int e = blockIdx.z;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;   // dst tile origin
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  const T* s = src + (size_t)e * src_estride;
  T* d = dst + (size_t)e * dst_estride;
  for (int i = ty; i < 64; i += 4) {
    const int sr = c0 + i, sc = r0 + tx;   // src[sr][sc] -> dst[sc][sr]
    tile[i][tx] = (sr < src_rows && sc < src_cols) ? s[(size_t)sr * src_cols + sc] : T(0);
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int dr = r0 + i, dc = c0 + tx;
    if (dr < dst_rows && dc < dst_cols) d[(size_t)dr * dst_cols + dc] = tile[tx][i];
  }
}

}  // namespace

template <typename ActT>
hipError_t launch_scatter_bwd(const ActT* dy, const ActT* ye, const int32_t* perm,
                              const float* topk_p, int A, int C, int k, ActT* dgo, float* dtp,
                              hipStream_t stream) {
  if (A <= 0) return hipSuccess;
  if (C % Vec<ActT>::N) return hipErrorInvalidValue;
  hipLaunchKernelGGL(scatter_bwd_kernel<ActT>, dim3((A + 3) / 4), dim3(256), 0, stream, dy, ye,
                     perm, topk_p, A, C, k, dgo, dtp);
  return hipGetLastError();
}

template <typename ActT>
hipError_t launch_token_bwd(const ActT* dxe, const int32_t* slot_of, const int32_t* topk_idx,
                            const float* dtp, const float* probs, const int32_t* counts,
                            const float* wr_g, int RE, int N, int C, int E, int k, ActT* dx,
                            float* dL, hipStream_t stream) {
  if (N <= 0) return hipSuccess;
  if (C % 4 || E > kMaxExperts || k > kMaxTopK) return hipErrorInvalidValue;
  hipLaunchKernelGGL(token_bwd_kernel<ActT>, dim3((N + kTokBlock - 1) / kTokBlock), dim3(256), 0,
                     stream, dxe, slot_of, topk_idx, dtp, probs, counts, wr_g, RE, N, C, E, k, dx,
                     dL);
  return hipGetLastError();
}

int router_wgrad_chunks(int N) { return (N + kRwChunk - 1) / kRwChunk; }

template <typename ActT>
hipError_t launch_router_wgrad(const ActT* x, const float* dL, int N, int C, int E,
                               float* partial, float* partial_b, float* gW, float* gb,
                               hipStream_t stream) {
  if (N <= 0) return hipSuccess;
  const int chunks = router_wgrad_chunks(N);
  const dim3 grid((C + 255) / 256, chunks);
  if (E <= 16)
    hipLaunchKernelGGL((router_wgrad_kernel<ActT, 16>), grid, dim3(256), 0, stream, x, dL, N, C,
                       E, partial, partial_b);
  else if (E <= 32)
    hipLaunchKernelGGL((router_wgrad_kernel<ActT, 32>), grid, dim3(256), 0, stream, x, dL, N, C,
                       E, partial, partial_b);
  else
    hipLaunchKernelGGL((router_wgrad_kernel<ActT, 64>), grid, dim3(256), 0, stream, x, dL, N, C,
                       E, partial, partial_b);
  const int CE = C * E;
  hipLaunchKernelGGL(router_wgrad_reduce_kernel, dim3((CE + E + 255) / 256), dim3(256), 0, stream,
                     partial, partial_b, chunks, CE, E, gW, gb);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_transpose_pad(const T* src, int src_rows, int src_cols, size_t src_estride,
                                T* dst, int dst_rows, int dst_cols, size_t dst_estride, int E,
                                hipStream_t stream) {
  const dim3 grid((dst_cols + 63) / 64, (dst_rows + 63) / 64, E);
  hipLaunchKernelGGL(transpose_pad_kernel<T>, grid, dim3(256), 0, stream, src, src_rows, src_cols,
                     src_estride, dst, dst_rows, dst_cols, dst_estride);
  return hipGetLastError();
}

#define MGPT_INST_BWD(T)                                                                       \
  template hipError_t launch_scatter_bwd<T>(const T*, const T*, const int32_t*, const float*,  \
                                            int, int, int, T*, float*, hipStream_t);           \
  template hipError_t launch_token_bwd<T>(const T*, const int32_t*, const int32_t*,            \
                                          const float*, const float*, const int32_t*,          \
                                          const float*, int, int, int, int, int, T*, float*,   \
                                          hipStream_t);                                        \
  template hipError_t launch_router_wgrad<T>(const T*, const float*, int, int, int, float*,    \
                                             float*, float*, float*, hipStream_t);             \
  template hipError_t launch_transpose_pad<T>(const T*, int, int, size_t, T*, int, int, size_t, \
                                              int, hipStream_t);
MGPT_INST_BWD(bf16_t)
MGPT_INST_BWD(float)

}  // namespace mgpt
