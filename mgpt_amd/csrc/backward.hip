// backward.hip -- the non-GEMM stages of the MoE block backward.
//
// Reference: MoELayer::backward_into (layers/MoELayer.cpp:130-223), CPU
// branches of the tensor ops it calls (utils/Tensor.cpp):
//   scatter_bwd   moe_scatter_backward :1410-1438: per slot,
//                 dgo[slot] = dy[t] * p and dp[t*k+j] = <y_e[slot], dy[t]>
//   token_dl      scatter_indices_into :1462-1484 + the load-balance term
//                 (layers/MoELayer.cpp:193-200) + softmax_backward :885-905
//                 on the clamped probabilities
//   token_dx      per token dx = sum over its slots (ascending) of dX_e (the
//                 gather backward :1440-1460) + dL . W_r^T (router
//                 LinearLayer::backward_into, layers/LinearLayer.cpp:33-80)
//   router_wgrad  dW_r += x^T . dL, db_r += sum_t dL (same Linear backward):
//                 per-chunk partial sums, then an in-order reduction, so the
//                 result does not depend on scheduling
//   transpose_pad the forward's packed weights, transposed per expert into
//                 the layouts the data-gradient products read.
#include "common.hpp"

#include <type_traits>

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
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
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

// dL of every token: a group of EP lanes per token (EP a power of two >= E,
// <= 64, so a group never straddles a wave), lane e holding expert e:
// dP = the top-k entry (dp of that choice, else 0) + the load-balance term
// (alpha * E * f_e) / N with f_e = counts_e / N, alpha = 0.01;
// s = sum_e dP*P (a fixed-order shuffle tree); dL = P*(dP - s).
template <int EP>
__global__ __launch_bounds__(256) void token_dl_kernel(const int32_t* __restrict__ topk_idx,
                                                       const float* __restrict__ dtp,
                                                       const float* __restrict__ probs,
                                                       const int32_t* __restrict__ counts, int N,
                                                       int E, int k, float* __restrict__ dL) {
  const int gid = blockIdx.x * (256 / EP) + (int)threadIdx.x / EP;
  const int e = threadIdx.x % EP;
  const bool tok = gid < N;
  const bool live = tok && e < E;
  float dp = 0.0f, p = 0.0f;
  if (live) {
    const float fe = (float)counts[e] / (float)N;
    const float lb = (0.01f * (float)E * fe) / (float)N;
    float sel = 0.0f;
    for (int j = 0; j < k; ++j)
      if (topk_idx[(size_t)gid * k + j] == e) sel = dtp[(size_t)gid * k + j];
    dp = sel + lb;
    p = probs[(size_t)gid * E + e];
  }
  float sum = dp * p;
#pragma unroll
  for (int m = 1; m < EP; m <<= 1) sum += __shfl_xor(sum, m, kWave);
  if (live) dL[(size_t)gid * E + e] = p * (dp - sum);
}

// token_dl_kernel for more experts than a wave has lanes: one wave per
// token, lane l holding experts l, l + 64, ... (their terms added in that
// order, then the same shuffle tree over the lanes).
template <int kPerLane>   // experts per lane: ceil(E / 64)
__global__ __launch_bounds__(256) void token_dl_wide_kernel(const int32_t* __restrict__ topk_idx,
                                                            const float* __restrict__ dtp,
                                                            const float* __restrict__ probs,
                                                            const int32_t* __restrict__ counts,
                                                            int N, int E, int k,
                                                            float* __restrict__ dL) {
  const int gid = blockIdx.x * 4 + (int)threadIdx.x / kWave;
  if (gid >= N) return;   // wave-uniform
  const int l = lane_id();
  float dp[kPerLane], p[kPerLane];
  float sum = 0.0f;
#pragma unroll
  for (int u = 0; u < kPerLane; ++u) {
    const int e = l + u * kWave;
    dp[u] = 0.0f;
    p[u] = 0.0f;
    if (e < E) {
      const float fe = (float)counts[e] / (float)N;
      const float lb = (0.01f * (float)E * fe) / (float)N;
      float sel = 0.0f;
      for (int j = 0; j < k; ++j)
        if (topk_idx[(size_t)gid * k + j] == e) sel = dtp[(size_t)gid * k + j];
      dp[u] = sel + lb;
      p[u] = probs[(size_t)gid * E + e];
    }
    sum += dp[u] * p[u];
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) sum += __shfl_xor(sum, m, kWave);
#pragma unroll
  for (int u = 0; u < kPerLane; ++u) {
    const int e = l + u * kWave;
    if (e < E) dL[(size_t)gid * E + e] = p[u] * (dp[u] - sum);
  }
}

constexpr int kDxTokens = 8;   // tokens per token_dx wave

// dx of kDxTokens tokens x 512 columns per wave (8 columns per lane):
// the sum of the tokens' slot rows of dX_e in ascending slot order (the
// gather backward) plus dL . W_r^T (wrt = W_r as [E][C]; experts in
// ascending order, 4 experts' weights loaded at a time, fused multiply-adds).
template <typename ActT, int EMAX>
__global__ __launch_bounds__(64) void token_dx_kernel(const ActT* __restrict__ dxe,
                                                      const int32_t* __restrict__ slot_of,
                                                      const float* __restrict__ dL,
                                                      const float* __restrict__ wrt, int N, int C,
                                                      int E, int k, ActT* __restrict__ dx) {
  using V = Vec<ActT>;
  __shared__ float s_dl[kDxTokens][EMAX];
  __shared__ int s_slot[kDxTokens][kMaxTopK];
  const int lane = lane_id();
  const int t0 = blockIdx.x * kDxTokens;
  const int nt = min(kDxTokens, N - t0);
  for (int p = lane; p < kDxTokens * EMAX; p += kWave) {
    const int r = p / EMAX, e = p % EMAX;
    s_dl[r][e] = (r < nt && e < E) ? dL[(size_t)(t0 + r) * E + e] : 0.0f;
  }
  if (lane < nt) {
    int* sl = s_slot[lane];
    for (int j = 0; j < k; ++j) sl[j] = slot_of[(size_t)(t0 + lane) * k + j];
    for (int a = 1; a < k; ++a) {   // insertion sort: ascending slots
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
  const int c0 = blockIdx.y * 512 + lane * 8;
  if (c0 >= C) return;
  float acc[kDxTokens][8];
#pragma unroll
  for (int r = 0; r < kDxTokens; ++r)
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[r][q] = 0.0f;
  for (int e0 = 0; e0 < E; e0 += 4) {
    float w[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (e0 + u < E) {
        const float4 a = *reinterpret_cast<const float4*>(wrt + (size_t)(e0 + u) * C + c0);
        const float4 b = *reinterpret_cast<const float4*>(wrt + (size_t)(e0 + u) * C + c0 + 4);
        w[u][0] = a.x; w[u][1] = a.y; w[u][2] = a.z; w[u][3] = a.w;
        w[u][4] = b.x; w[u][5] = b.y; w[u][6] = b.z; w[u][7] = b.w;
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) w[u][q] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < kDxTokens; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float g = s_dl[r][e0 + u];
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[r][q] = __builtin_fmaf(g, w[u][q], acc[r][q]);
      }
  }
#pragma unroll
  for (int r = 0; r < kDxTokens; ++r) {
    if (r >= nt) break;
    float gs[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) gs[q] = 0.0f;
    for (int j = 0; j < k; ++j) {
      const ActT* src = dxe + (size_t)s_slot[r][j] * C + c0;
#pragma unroll
      for (int h = 0; h < 8 / V::N; ++h) {
        float v[V::N];
        V::unpack(*reinterpret_cast<const uint4*>(src + h * V::N), v);
#pragma unroll
        for (int q = 0; q < V::N; ++q) gs[h * V::N + q] += v[q];
      }
    }
    ActT* o = dx + (size_t)(t0 + r) * C + c0;
#pragma unroll
    for (int h = 0; h < 8 / V::N; ++h) {
      float v[V::N];
#pragma unroll
      for (int q = 0; q < V::N; ++q) v[q] = gs[h * V::N + q] + acc[r][h * V::N + q];
      *reinterpret_cast<uint4*>(o + h * V::N) = V::pack(v);
    }
  }
}

constexpr int kRwChunk = 64;    // tokens per router_wgrad partial

// CPT consecutive columns of row p of x as floats (one vector load).
template <int CPT>
__device__ __forceinline__ void rw_load_cols(const bf16_t* p, float (&v)[CPT]) {
  if constexpr (CPT == 4) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(w.x << 16);
    v[1] = __uint_as_float(w.x & 0xFFFF0000u);
    v[2] = __uint_as_float(w.y << 16);
    v[3] = __uint_as_float(w.y & 0xFFFF0000u);
  } else if constexpr (CPT == 2) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    v[0] = __uint_as_float(w << 16);
    v[1] = __uint_as_float(w & 0xFFFF0000u);
  } else {
    v[0] = bf16_to_f32(*p);
  }
}
template <int CPT>
__device__ __forceinline__ void rw_load_cols(const float* p, float (&v)[CPT]) {
  if constexpr (CPT == 4) {
    const float4 w = *reinterpret_cast<const float4*>(p);
    v[0] = w.x;
    v[1] = w.y;
    v[2] = w.z;
    v[3] = w.w;
  } else if constexpr (CPT == 2) {
    const float2 w = *reinterpret_cast<const float2*>(p);
    v[0] = w.x;
    v[1] = w.y;
  } else {
    v[0] = *p;
  }
}

// partial[chunk][e][c] = sum over the chunk's tokens of x[t][c] * dL[t][e]
// (tokens in order, fused multiply-adds).  A thread holds CPT consecutive
// columns x EP >= E experts (CPT * EP accumulators), reads each
// token's CPT values of x as one vector load and the token's dL row from
// LDS as float4 broadcasts: CPT * EP FMAs per 1 + EP / 4 loads.  The x
// loads run a group of 8 tokens ahead of the FMAs (two register groups;
// every load is issued, past the chunk's end at a clamped row whose
// values are then zeroed, so the wait counts stay exact), and each
// expert's CPT sums go out as one vector store, lanes on consecutive
// columns.  The blocks of the first column range also write
// partial_b[chunk][e] = sum_t dL[t][e].  NRM (fused block): the router's
// input is the normalised row, so x[t][c] is taken as (x[t][c] * rstd[t]) *
// gamma[c], the fp32 values the router formed its logits from.
template <typename ActT, int EP, int CPT, bool NRM>
__global__ __launch_bounds__(256) void router_wgrad_kernel(const ActT* __restrict__ x,
                                                           const float* __restrict__ dL, int N,
                                                           int C, int E,
                                                           float* __restrict__ partial,
                                                           float* __restrict__ partial_b,
                                                           const float* __restrict__ rstd,
                                                           const float* __restrict__ gamma) {
  constexpr int kG = 8;   // tokens per load group
  static_assert(kRwChunk % (2 * kG) == 0, "whole group pairs per chunk");
  __shared__ float4 s_dl[kRwChunk][EP / 4];
  const int tid = threadIdx.x;
  const int chunk = blockIdx.y;
  const int c0 = (blockIdx.x * 256 + tid) * CPT;
  const int t0 = chunk * kRwChunk, nt = min(kRwChunk, N - t0);
  // experts [e_base, e_base + Eg) of this block (one group of EP unless
  // E > 64: then blockIdx.z walks the groups)
  const int e_base = blockIdx.z * EP;
  const int Eg = min(EP, E - e_base);
  float* sl = reinterpret_cast<float*>(s_dl);
  for (int p = tid; p < kRwChunk * EP; p += 256) {
    const int r = p / EP, e = p % EP;
    sl[p] = (r < nt && e < Eg) ? dL[(size_t)(t0 + r) * E + e_base + e] : 0.0f;
  }
  __syncthreads();
  if (blockIdx.x == 0 && tid < Eg) {
    float bsum = 0.0f;
    for (int r = 0; r < nt; ++r) bsum += sl[r * EP + tid];
    partial_b[(size_t)chunk * E + e_base + tid] = bsum;
  }
  if (c0 >= C) return;   // C is a multiple of CPT
  float acc[CPT][EP];
#pragma unroll
  for (int cc = 0; cc < CPT; ++cc)
#pragma unroll
    for (int e = 0; e < EP; ++e) acc[cc][e] = 0.0f;
  const ActT* xp = x + (size_t)t0 * C + c0;
  float gm[CPT];
#pragma unroll
  for (int cc = 0; cc < CPT; ++cc) gm[cc] = NRM ? gamma[c0 + cc] : 1.0f;
  auto load = [&](int r0, float (&xv)[kG][CPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kG; ++u) {
      const int r = min(r0 + u, nt - 1);
      rw_load_cols<CPT>(xp + (size_t)r * C, xv[u]);
      if constexpr (NRM) {
        const float rs = rstd[t0 + r];
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) xv[u][cc] = (xv[u][cc] * rs) * gm[cc];
      }
    }
  };
  auto fmas = [&](int r0, float (&xv)[kG][CPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kG; ++u) {
      if (r0 + u >= nt) {   // a clamped row (its dL row is zero as well)
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) xv[u][cc] = 0.0f;
      }
#pragma unroll
      for (int e4 = 0; e4 < EP / 4; ++e4) {
        const float4 d = s_dl[r0 + u][e4];
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) {
          acc[cc][4 * e4 + 0] = __builtin_fmaf(xv[u][cc], d.x, acc[cc][4 * e4 + 0]);
          acc[cc][4 * e4 + 1] = __builtin_fmaf(xv[u][cc], d.y, acc[cc][4 * e4 + 1]);
          acc[cc][4 * e4 + 2] = __builtin_fmaf(xv[u][cc], d.z, acc[cc][4 * e4 + 2]);
          acc[cc][4 * e4 + 3] = __builtin_fmaf(xv[u][cc], d.w, acc[cc][4 * e4 + 3]);
        }
      }
    }
  };
  float xa[kG][CPT], xb[kG][CPT];
  load(0, xa);
  for (int r0 = 0; r0 < nt; r0 += 2 * kG) {
    load(r0 + kG, xb);
    fmas(r0, xa);
    if (r0 + 2 * kG < nt) load(r0 + 2 * kG, xa);
    fmas(r0 + kG, xb);
  }
  float* o = partial + (size_t)chunk * C * E + (size_t)e_base * C + c0;
#pragma unroll
  for (int e = 0; e < EP; ++e) {
    if (e >= Eg) break;
    if constexpr (CPT == 4) {
      *reinterpret_cast<float4*>(o + (size_t)e * C) =
          make_float4(acc[0][e], acc[1][e], acc[2][e], acc[3][e]);
    } else if constexpr (CPT == 2) {
      *reinterpret_cast<float2*>(o + (size_t)e * C) = make_float2(acc[0][e], acc[1][e]);
    } else {
      o[(size_t)e * C] = acc[0][e];
    }
  }
}

// grad += sum over chunks of partial[chunk][i], for the C*E weight
// entries (i = e * C + c, gradient entry gW[c][e]) followed by the E bias
// entries, as a fixed two-level tree (so the result does not depend on
// scheduling): a block takes 16 entries; thread (entry, g) adds the g-th of
// 16 consecutive chunk ranges in order, then one thread per entry adds the
// 16 range sums in order.  With `store` the gradient is taken to be zero
// and the sum is written without reading it.
__global__ __launch_bounds__(256) void router_wgrad_reduce_kernel(
    const float* __restrict__ partial, const float* __restrict__ partial_b, int chunks, int C,
    int E, float* __restrict__ gW, float* __restrict__ gb, int store) {
  const int CE = C * E;
  __shared__ float s_part[16][16];
  const int el = threadIdx.x % 16, g = threadIdx.x / 16;
  const int i = blockIdx.x * 16 + el;
  const bool live = i < CE + E;
  const bool w = i < CE;
  const float* src = w ? partial + i : partial_b + (i - CE);
  const size_t stride = w ? (size_t)CE : (size_t)E;
  const int per = (chunks + 15) / 16;
  const int ch0 = g * per, ch1 = min(chunks, ch0 + per);
  float s = 0.0f;
  for (int c0 = ch0; c0 < ch1; c0 += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      v[u] = (live && c0 + u < ch1) ? src[(size_t)(c0 + u) * stride] : 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (c0 + u < ch1) s += v[u];
  }
  s_part[g][el] = s;
  __syncthreads();
  if (g == 0 && live) {
    float t = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) t += s_part[q][el];
    float* o = w ? gW + (size_t)(i % C) * E + i / C : gb + (i - CE);
    *o = store ? t : *o + t;
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
                            const float* wrt, int N, int C, int E, int k, ActT* dx, float* dL,
                            hipStream_t stream) {
  if (N <= 0) return hipSuccess;
  if (E > kMaxExpertsWide || k > kMaxTopK || C % 8) return hipErrorInvalidValue;
  if (E > 256)
    hipLaunchKernelGGL((token_dl_wide_kernel<kMaxExpertsWide / kWave>), dim3((N + 3) / 4),
                       dim3(256), 0, stream, topk_idx, dtp, probs, counts, N, E, k, dL);
  else if (E > kMaxExperts)
    hipLaunchKernelGGL((token_dl_wide_kernel<4>), dim3((N + 3) / 4), dim3(256), 0, stream,
                       topk_idx, dtp, probs, counts, N, E, k, dL);
  else if (E <= 16)
    hipLaunchKernelGGL(token_dl_kernel<16>, dim3((N + 15) / 16), dim3(256), 0, stream, topk_idx,
                       dtp, probs, counts, N, E, k, dL);
  else if (E <= 32)
    hipLaunchKernelGGL(token_dl_kernel<32>, dim3((N + 7) / 8), dim3(256), 0, stream, topk_idx,
                       dtp, probs, counts, N, E, k, dL);
  else
    hipLaunchKernelGGL(token_dl_kernel<64>, dim3((N + 3) / 4), dim3(256), 0, stream, topk_idx,
                       dtp, probs, counts, N, E, k, dL);
  const dim3 gdx((N + kDxTokens - 1) / kDxTokens, (C + 511) / 512);
  if (E > 256)
    hipLaunchKernelGGL((token_dx_kernel<ActT, kMaxExpertsWide>), gdx, dim3(64), 0, stream, dxe,
                       slot_of, dL, wrt, N, C, E, k, dx);
  else if (E > kMaxExperts)
    hipLaunchKernelGGL((token_dx_kernel<ActT, 256>), gdx, dim3(64), 0, stream, dxe,
                       slot_of, dL, wrt, N, C, E, k, dx);
  else
    hipLaunchKernelGGL((token_dx_kernel<ActT, kMaxExperts>), gdx, dim3(64), 0, stream, dxe,
                       slot_of, dL, wrt, N, C, E, k, dx);
  return hipGetLastError();
}

int router_wgrad_chunks(int N) { return (N + kRwChunk - 1) / kRwChunk; }

template <typename ActT, bool NRM>
void launch_router_wgrad_products(const ActT* x, const float* dL, int N, int C, int E,
                                  float* partial, float* partial_b, const float* rstd,
                                  const float* gamma, int chunks, hipStream_t stream) {
  // a block covers 256 threads x CPT columns; E <= 32 takes two columns per
  // thread (at cfg3, E = 16, four columns per thread gave one wave per SIMD
  // and 42 us)
  if (E <= 16)
    hipLaunchKernelGGL((router_wgrad_kernel<ActT, 16, 2, NRM>), dim3((C + 511) / 512, chunks),
                       dim3(256), 0, stream, x, dL, N, C, E, partial, partial_b, rstd, gamma);
  else if (E <= 32)
    hipLaunchKernelGGL((router_wgrad_kernel<ActT, 32, 2, NRM>), dim3((C + 511) / 512, chunks),
                       dim3(256), 0, stream, x, dL, N, C, E, partial, partial_b, rstd, gamma);
  else   // groups of 64 experts along z (one group unless E > 64)
    hipLaunchKernelGGL((router_wgrad_kernel<ActT, 64, 1, NRM>),
                       dim3((C + 255) / 256, chunks, (E + 63) / 64), dim3(256), 0, stream, x, dL,
                       N, C, E, partial, partial_b, rstd, gamma);
}

// rstd / gamma (both null, or both set): the fused block's router input,
// (x * rstd[t]) * gamma[c].
template <typename ActT>
hipError_t launch_router_wgrad(const ActT* x, const float* dL, int N, int C, int E,
                               float* partial, float* partial_b, float* gW, float* gb,
                               bool store, const float* rstd, const float* gamma,
                               hipStream_t stream) {
  if (E <= 0 || E > kMaxExpertsWide || C % 4 || (!rstd) != (!gamma)) return hipErrorInvalidValue;
  if (N <= 0) return hipSuccess;
  const int chunks = router_wgrad_chunks(N);
  if (rstd)
    launch_router_wgrad_products<ActT, true>(x, dL, N, C, E, partial, partial_b, rstd, gamma,
                                             chunks, stream);
  else
    launch_router_wgrad_products<ActT, false>(x, dL, N, C, E, partial, partial_b, nullptr,
                                              nullptr, chunks, stream);
  const int CE = C * E;
  hipLaunchKernelGGL(router_wgrad_reduce_kernel, dim3((CE + E + 15) / 16), dim3(256), 0, stream,
                     partial, partial_b, chunks, C, E, gW, gb, (int)store);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Backward of the fused block's ln2 RMSNorm and residual (the MoE half of
// TransformerBlock::backward_into, layers/TransformerBlock.cpp:81-85, with
// RMSNormLayer::backward_into, utils/Tensor.cpp:1665-1689):
//   x_hat = x * r, dh = d * gamma, s = sum_c dh * x_hat,
//   dx1 = dout + r * (dh - x_hat * (s / C)),   dgamma[c] += sum_t d * x_hat,
// with d the gradient of the normalised rows (the MoE backward's dx).  A
// block of 256 threads takes kNbRows token rows, each thread the same
// column pieces (V consecutive columns) of every row: a first pass forms
// each row's s (per-thread partial sums, a wave sum, the four waves' sums
// added in wave order), a second writes dx1 in place of d and adds the
// rows' d * x_hat per column in registers, stored as partial[block][c];
// rmsnorm_dgamma_reduce_kernel adds the blocks' partials in a fixed order
// (deterministic).  Each thread reads its own elements of d before it
// overwrites them, so d and dx1 share the buffer.
constexpr int kNbRows = 16;

template <typename ActT, int V> struct NbVec;
template <> struct NbVec<bf16_t, 4> {
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[4]) {
    const uint2 q = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xFFFF0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xFFFF0000u);
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[4]) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  }
};
template <> struct NbVec<float, 4> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};
template <typename ActT> struct NbVec<ActT, 1> {
  static __device__ __forceinline__ void load(const ActT* p, float (&v)[1]) { v[0] = to_f32(*p); }
  static __device__ __forceinline__ void store(ActT* p, const float (&v)[1]) { store_act(p, v[0]); }
};

template <typename ActT, int V>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const ActT* __restrict__ x, ActT* d,
                                                          const ActT* __restrict__ dout,
                                                          const float* __restrict__ rstd,
                                                          const float* __restrict__ gamma, int N,
                                                          int C, float* __restrict__ partial) {
  using Vec = NbVec<ActT, V>;
  __shared__ float s_part[4][kNbRows];
  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
  const int t0 = blockIdx.x * kNbRows;
  const int nt = min(kNbRows, N - t0);
  float r[kNbRows], acc[kNbRows];
#pragma unroll
  for (int i = 0; i < kNbRows; ++i) {
    r[i] = rstd[t0 + min(i, nt - 1)];
    acc[i] = 0.0f;
  }
  for (int c = tid * V; c < C; c += 256 * V) {
    float g[V];
#pragma unroll
    for (int v = 0; v < V; ++v) g[v] = gamma[c + v];
    // rows past the block's last token re-read that token (in bounds) and
    // their sums are never used, so every load is issued unconditionally
#pragma unroll
    for (int i = 0; i < kNbRows; ++i) {
      const size_t row = (size_t)(t0 + min(i, nt - 1)) * C;
      float xv[V], dv[V];
      Vec::load(x + row + c, xv);
      Vec::load(d + row + c, dv);
#pragma unroll
      for (int v = 0; v < V; ++v) acc[i] = acc[i] + (dv[v] * g[v]) * (xv[v] * r[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < kNbRows; ++i) {
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) acc[i] = acc[i] + __shfl_xor(acc[i], m, kWave);
    if (lane == 0) s_part[w][i] = acc[i];
  }
  __syncthreads();
  const float cf = (float)C;
  float q[kNbRows];
#pragma unroll
  for (int i = 0; i < kNbRows; ++i)
    q[i] = (((s_part[0][i] + s_part[1][i]) + s_part[2][i]) + s_part[3][i]) / cf;
  for (int c = tid * V; c < C; c += 256 * V) {
    float g[V], dg[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      g[v] = gamma[c + v];
      dg[v] = 0.0f;
    }
    float xv[kNbRows][V], dv[kNbRows][V], ov[kNbRows][V];
#pragma unroll
    for (int i = 0; i < kNbRows; ++i) {
      const size_t row = (size_t)(t0 + min(i, nt - 1)) * C;
      Vec::load(x + row + c, xv[i]);
      Vec::load(d + row + c, dv[i]);
      Vec::load(dout + row + c, ov[i]);
    }
#pragma unroll
    for (int i = 0; i < kNbRows; ++i) {
      const bool live = i < nt;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float xh = xv[i][v] * r[i];
        dg[v] = dg[v] + (live ? dv[i][v] * xh : 0.0f);
        ov[i][v] = ov[i][v] + r[i] * (dv[i][v] * g[v] - xh * q[i]);
      }
      if (live) Vec::store(d + (size_t)(t0 + i) * C + c, ov[i]);
    }
    float* po = partial + (size_t)blockIdx.x * C + c;
#pragma unroll
    for (int v = 0; v < V; ++v) po[v] = dg[v];
  }
}

// The same for bf16 rows of at most 1024 columns (one 4-column piece per
// thread): every load of the block's rows is issued first and the values
// stay in registers for both passes, so the block makes one trip to
// memory instead of reading x and d twice.
__global__ __launch_bounds__(256) void rmsnorm_bwd_bf16_kernel(
    const bf16_t* __restrict__ x, bf16_t* d, const bf16_t* __restrict__ dout,
    const float* __restrict__ rstd, const float* __restrict__ gamma, int N, int C,
    float* __restrict__ partial) {
  using Vec = NbVec<bf16_t, 4>;
  __shared__ float s_part[4][kNbRows];
  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
  const int t0 = blockIdx.x * kNbRows;
  const int nt = min(kNbRows, N - t0);
  const int c = tid * 4;
  const bool has = c < C;   // this thread's piece exists
  uint2 xr[kNbRows], dr[kNbRows], orr[kNbRows];
  float r[kNbRows];
#pragma unroll
  for (int i = 0; i < kNbRows; ++i) {
    // rows past the block's last token re-read that token (in bounds)
    const size_t row = (size_t)(t0 + min(i, nt - 1)) * C + c;
    r[i] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(rstd[t0 + min(i, nt - 1)])));
    if (has) {
      xr[i] = *reinterpret_cast<const uint2*>(x + row);
      dr[i] = *reinterpret_cast<const uint2*>(d + row);
      orr[i] = *reinterpret_cast<const uint2*>(dout + row);
    } else {
      xr[i] = dr[i] = orr[i] = make_uint2(0u, 0u);
    }
  }
  float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (has) {
    const float4 gv = *reinterpret_cast<const float4*>(gamma + c);
    g[0] = gv.x; g[1] = gv.y; g[2] = gv.z; g[3] = gv.w;
  }
  auto unpack = [](const uint2& q, float (&v)[4]) __attribute__((always_inline)) {
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xFFFF0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xFFFF0000u);
  };
  float acc[kNbRows];
#pragma unroll
  for (int i = 0; i < kNbRows; ++i) {
    float xv[4], dv[4];
    unpack(xr[i], xv);
    unpack(dr[i], dv);
    acc[i] = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[i] = acc[i] + (dv[v] * g[v]) * (xv[v] * r[i]);
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) acc[i] = acc[i] + __shfl_xor(acc[i], m, kWave);
    if (lane == 0) s_part[w][i] = acc[i];
  }
  __syncthreads();
  if (!has) return;
  // the packed rows again (not the unpacked values of the first pass, which
  // would double the live registers)
#pragma unroll
  for (int i = 0; i < kNbRows; ++i) asm volatile("" : "+v"(xr[i]), "+v"(dr[i]), "+v"(orr[i]));
  const float cf = (float)C;
  float dg[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < kNbRows; ++i) {
    const float q = (((s_part[0][i] + s_part[1][i]) + s_part[2][i]) + s_part[3][i]) / cf;
    const bool live = i < nt;
    float xv[4], dv[4], ov[4];
    unpack(xr[i], xv);
    unpack(dr[i], dv);
    unpack(orr[i], ov);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float xh = xv[v] * r[i];
      dg[v] = dg[v] + (live ? dv[v] * xh : 0.0f);
      ov[v] = ov[v] + r[i] * (dv[v] * g[v] - xh * q);
    }
    if (live) Vec::store(d + (size_t)(t0 + i) * C + c, ov);
  }
  *reinterpret_cast<float4*>(partial + (size_t)blockIdx.x * C + c) =
      make_float4(dg[0], dg[1], dg[2], dg[3]);
}

// dgamma[c] += sum over the row blocks b of partial[b][c] in a fixed order:
// wave w of the block of 64 columns takes b = w + 16m, 32 loads in flight
// at a time, into eight running sums (m mod 8) joined pairwise; wave 0 adds
// the sixteen waves' sums in wave order.
__global__ __launch_bounds__(1024) void rmsnorm_dgamma_reduce_kernel(
    const float* __restrict__ partial, int nb, int C, float* __restrict__ dgamma) {
  __shared__ float s_w[16][kWave];
  const int lane = lane_id(), w = threadIdx.x / kWave;
  const int c = blockIdx.x * kWave + lane;
  float a[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) a[u] = 0.0f;
  if (c < C)
    for (int b0 = w; b0 < nb; b0 += 16 * 32) {
      float v[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) {
        const int b = b0 + 16 * u;
        v[u] = b < nb ? partial[(size_t)b * C + c] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 32; ++u) a[u % 8] = a[u % 8] + v[u];
    }
  s_w[w][lane] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  __syncthreads();
  if (w == 0 && c < C) {
    float t = 0.0f;
    for (int i = 0; i < 16; ++i) t = t + s_w[i][lane];
    dgamma[c] = dgamma[c] + t;
  }
}

int rmsnorm_bwd_blocks(int N) { return (N + kNbRows - 1) / kNbRows; }

// d [N][C] (the gradient of the normalised rows) becomes dx1 in place;
// partial: rmsnorm_bwd_blocks(N) x C floats.
template <typename ActT>
hipError_t launch_rmsnorm_bwd(const ActT* x, ActT* d, const ActT* dout, const float* rstd,
                              const float* gamma, int N, int C, float* partial, float* dgamma,
                              hipStream_t stream) {
  if (N < 0 || C <= 0) return hipErrorInvalidValue;
  if (N == 0) return hipSuccess;
  const int nb = rmsnorm_bwd_blocks(N);
  // pieces of 4 columns when every row starts on a piece-aligned boundary
  const size_t piece = 4 * sizeof(ActT);
  const bool vec = C % 4 == 0 && ((uintptr_t)x | (uintptr_t)d | (uintptr_t)dout) % piece == 0;
  bool single_pass = false;
  if constexpr (std::is_same<ActT, bf16_t>::value)
    single_pass = vec && C <= 1024 && (uintptr_t)gamma % 16 == 0;
  if (single_pass)
    hipLaunchKernelGGL(rmsnorm_bwd_bf16_kernel, dim3(nb), dim3(256), 0, stream,
                       reinterpret_cast<const bf16_t*>(x), reinterpret_cast<bf16_t*>(d),
                       reinterpret_cast<const bf16_t*>(dout), rstd, gamma, N, C, partial);
  else if (vec)
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<ActT, 4>), dim3(nb), dim3(256), 0, stream, x, d,
                       dout, rstd, gamma, N, C, partial);
  else
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<ActT, 1>), dim3(nb), dim3(256), 0, stream, x, d,
                       dout, rstd, gamma, N, C, partial);
  hipLaunchKernelGGL(rmsnorm_dgamma_reduce_kernel, dim3((C + kWave - 1) / kWave), dim3(1024), 0,
                     stream, partial, nb, C, dgamma);
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
                                          const float*, int, int, int, int, T*, float*,        \
                                          hipStream_t);                                        \
  template hipError_t launch_router_wgrad<T>(const T*, const float*, int, int, int, float*,    \
                                             float*, float*, float*, bool, const float*,       \
                                             const float*, hipStream_t);                       \
  template hipError_t launch_rmsnorm_bwd<T>(const T*, T*, const T*, const float*, const float*, \
                                            int, int, float*, float*, hipStream_t);            \
  template hipError_t launch_transpose_pad<T>(const T*, int, int, size_t, T*, int, int, size_t, \
                                              int, hipStream_t);
MGPT_INST_BWD(bf16_t)
MGPT_INST_BWD(float)

}  // namespace mgpt
