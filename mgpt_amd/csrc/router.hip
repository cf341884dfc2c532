// router.hip -- fused router GEMM + clamped softmax + top-k + block histogram.
//
// Reference path (all bit-exact): router Linear layers/LinearLayer.cpp:23-28
// -> Tensor::matmul_into utils/Tensor.cpp:1231-1249 -> matmul2d_raw :567-577
// (each logit is a sequential fp32 sum over c of rounded products, then the
// bias is added, :1499-1507 / :331-342); softmax utils/Tensor.cpp:850-883;
// top-k utils/Tensor.cpp:1296-1334; histogram utils/Tensor.cpp:1336-1352.
//
// One block owns 64 tokens (one per lane) and E/RE waves.  Phase 1: wave g
// computes the logits of experts [g*RE, g*RE+RE) for the 64 tokens, walking
// c = 0..C-1 in order with one rounded product and one rounded add per term
// (the file is built with -ffp-contract=off), so every logit has exactly the
// reference's rounding sequence; MFMA cannot be used here, its internal
// accumulation order differs.  The weights of a wave are wave-uniform and
// come through the scalar cache.  Phase 2: per-token max (strict '>' from
// element 0, as the reference, so NaN handling matches), the exponentials
// in parallel with glibc's expf algorithm, then per token the sequential
// sum, the clamp and the insertion top-k in registers.  Phase 3: block-local
// expert histogram (LDS atomics on ints; counts are order-free), written
// expert-major as hist[e][block] for the per-expert scan of dispatch.hip.
#include "common.hpp"
#include "glibc_expf.hpp"

namespace mgpt {

__constant__ uint64_t c_exp2_tab[32] = MGPT_EXP2_TABLE_INIT;

namespace {

constexpr int kRT = kRouterTokens;   // tokens per block (one per lane)

// Branch-free insertion of (v, e) into a descending top-K list, identical to
// the reference's shifting loop: the element at j-1 moves to j exactly when
// v > list[j-1]; a value not greater than list[K-1] changes nothing.
template <int K>
__device__ __forceinline__ void topk_insert(float (&ov)[K], int (&oi)[K], float v, int e) {
#pragma unroll
  for (int j = K - 1; j >= 0; --j) {
    const bool from_prev = (j > 0) && (v > ov[j > 0 ? j - 1 : 0]);
    const bool take_v = !from_prev && (v > ov[j]);
    const float nv = from_prev ? ov[j > 0 ? j - 1 : 0] : (take_v ? v : ov[j]);
    const int ni = from_prev ? oi[j > 0 ? j - 1 : 0] : (take_v ? e : oi[j]);
    ov[j] = nv;
    oi[j] = ni;
  }
}

template <int K>
__device__ __forceinline__ void softmax_topk_token(const float* __restrict__ ex, float inv, int E,
                                                   int32_t* __restrict__ idx_out,
                                                   float* __restrict__ p_out, int* s_hist) {
  float ov[K];
  int oi[K];
#pragma unroll
  for (int j = 0; j < K; ++j) { ov[j] = -1e9f; oi[j] = -1; }
  for (int v = 0; v < E; ++v) {
    const float p = fminf(fmaxf(ex[v] * inv, 1e-7f), 1.0f);
    topk_insert<K>(ov, oi, p, v);
  }
#pragma unroll
  for (int j = 0; j < K; ++j) {
    idx_out[j] = oi[j];
    p_out[j] = ov[j];
    if (oi[j] >= 0) atomicAdd(&s_hist[oi[j]], 1);
  }
}

template <typename ActT> struct Load8;
template <> struct Load8<bf16_t> {
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};
template <> struct Load8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
};

// Wave-uniform router weights.  A block owns 64 tokens (one per lane) and
// E/RE waves; wave g computes experts [g*RE, g*RE + RE) for all 64 tokens.
// Its slice of W_r is the same for every lane, so it is read with scalar
// loads into SGPRs (packed as [G][C][RE], 8*RE consecutive floats per 8 c),
// and each lane streams only its own token's row of x with 16-byte loads:
// no per-lane copies of the weights, no LDS and no barrier in the loop.
// Each logit accumulates c = 0, 1, ... in order, one rounded product and one
// rounded add per term (built with -ffp-contract=off), then the bias.
template <typename ActT, int RE>
__global__ __launch_bounds__(1024) void router_topk_uniform_kernel(
    const ActT* __restrict__ x, const float* __restrict__ wr_g, const float* __restrict__ br,
    int N, int C, int E, int k, int32_t* __restrict__ topk_idx, float* __restrict__ topk_p,
    int32_t* __restrict__ hist, int num_blocks) {
  __shared__ float s_l[kRT][kMaxExperts + 1];
  __shared__ float s_m[kRT];
  __shared__ int s_hist[kMaxExperts];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int g = __builtin_amdgcn_readfirstlane(tid / kWave);   // expert group of this wave
  const int tok0 = blockIdx.x * kRT;
  if (tid < kMaxExperts) s_hist[tid] = 0;

  const ActT* xrow = x + (size_t)min(tok0 + lane, N - 1) * C;   // rows past N: never stored
  const float* wg = wr_g + (size_t)g * C * RE;

  float acc[RE];
#pragma unroll
  for (int j = 0; j < RE; ++j) acc[j] = 0.0f;
#pragma unroll 2
  for (int c = 0; c < C; c += 8) {
    float xv[8];
    Load8<ActT>::load(xrow + c, xv);
    const float* wc = wg + (size_t)c * RE;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc)
#pragma unroll
      for (int j = 0; j < RE; ++j) acc[j] = acc[j] + xv[cc] * wc[cc * RE + j];
  }
#pragma unroll
  for (int j = 0; j < RE; ++j) {
    const int e = g * RE + j;
    if (e < E) s_l[lane][e] = acc[j] + br[e];
  }
  __syncthreads();
  if (tid < kRT) {
    float m = s_l[tid][0];
    for (int v = 1; v < E; ++v)
      if (s_l[tid][v] > m) m = s_l[tid][v];
    s_m[tid] = m;
  }
  __syncthreads();
  for (int p = tid; p < kRT * E; p += blockDim.x) {
    const int r = p / E, e = p % E;
    s_l[r][e] = mgpt_expf::expf_glibc(s_l[r][e] - s_m[r], c_exp2_tab);
  }
  __syncthreads();
  if (tid < kRT && tok0 + tid < N) {
    const float* ex = s_l[tid];
    float sum = 0.0f;
    for (int v = 0; v < E; ++v) sum = sum + ex[v];
    const float inv = 1.0f / fmaxf(sum, 1e-15f);
    int32_t* io = topk_idx + (size_t)(tok0 + tid) * k;
    float* po = topk_p + (size_t)(tok0 + tid) * k;
    switch (k) {
      case 1: softmax_topk_token<1>(ex, inv, E, io, po, s_hist); break;
      case 2: softmax_topk_token<2>(ex, inv, E, io, po, s_hist); break;
      case 3: softmax_topk_token<3>(ex, inv, E, io, po, s_hist); break;
      case 4: softmax_topk_token<4>(ex, inv, E, io, po, s_hist); break;
      case 5: softmax_topk_token<5>(ex, inv, E, io, po, s_hist); break;
      case 6: softmax_topk_token<6>(ex, inv, E, io, po, s_hist); break;
      case 7: softmax_topk_token<7>(ex, inv, E, io, po, s_hist); break;
      default: softmax_topk_token<8>(ex, inv, E, io, po, s_hist); break;
    }
  }
  __syncthreads();
  if (tid < E) hist[(size_t)tid * num_blocks + blockIdx.x] = s_hist[tid];
}

}  // namespace

template <typename ActT>
hipError_t launch_router(const ActT* x, const float* wr_g, const float* br, int N, int C, int E,
                         int k, int32_t* topk_idx, float* topk_p, int32_t* hist,
                         hipStream_t stream) {
  const int nb = (N + kRT - 1) / kRT;
  if (nb == 0) return hipSuccess;
  const int RE = router_experts_per_wave(E);
  const int waves = (E + RE - 1) / RE;
  const dim3 g(nb), b(waves * kWave);
  switch (RE) {
    case 1:
      hipLaunchKernelGGL((router_topk_uniform_kernel<ActT, 1>), g, b, 0, stream, x, wr_g, br, N,
                         C, E, k, topk_idx, topk_p, hist, nb);
      break;
    case 2:
      hipLaunchKernelGGL((router_topk_uniform_kernel<ActT, 2>), g, b, 0, stream, x, wr_g, br, N,
                         C, E, k, topk_idx, topk_p, hist, nb);
      break;
    default:
      hipLaunchKernelGGL((router_topk_uniform_kernel<ActT, 4>), g, b, 0, stream, x, wr_g, br, N,
                         C, E, k, topk_idx, topk_p, hist, nb);
  }
  return hipGetLastError();
}

template hipError_t launch_router<float>(const float*, const float*, const float*, int, int, int,
                                         int, int32_t*, float*, int32_t*, hipStream_t);
template hipError_t launch_router<bf16_t>(const bf16_t*, const float*, const float*, int, int,
                                          int, int, int32_t*, float*, int32_t*, hipStream_t);

// Device expf over a buffer (tests compare it with the host's glibc expf).
__global__ void expf_probe_kernel(const float* __restrict__ in, float* __restrict__ out, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = mgpt_expf::expf_glibc(in[i], c_exp2_tab);
}

hipError_t launch_expf_probe(const float* in, float* out, int n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(expf_probe_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in, out, n);
  return hipGetLastError();
}

}  // namespace mgpt
