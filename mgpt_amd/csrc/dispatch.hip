// dispatch.hip -- expert counts, per-block bases and the stable permutation.
//
// Reference: histogram utils/Tensor.cpp:1336-1352, host exclusive scan
// layers/MoELayer.cpp:61-80, gather utils/Tensor.cpp:1354-1383.  The
// reference CPU path assigns slots by walking the flat assignment ids
// i = t*k + j in ascending order and taking slot = offsets[e]++, so each
// expert's segment holds its assignments in ascending i.  Here that order is
// rebuilt as a counting sort that needs no host round-trip:
//   counts[e]      = sum over router blocks b of hist[e][b]
//   base[e][b]     = offset[e] + sum_{b' < b} hist[e][b']
//   slot(i)        = base[e][block(i)] + #{i' < i in block(i) : e(i') = e}
// For small dispatches each permute block sums the histogram columns it
// needs itself (E x nb ints, L2-resident), so the scan costs no launch of
// its own; large ones scan first (expert_scan_kernel).
// The within-block rank comes from wave ballots over 64 consecutive ids at
// a time (one ballot per bit of the expert ids: 6 for E <= 64, 8 for
// E <= 256, 9 for E <= 512).
// The permute kernel then copies each token's row once from HBM into all k
// of its slots with 16-byte loads and stores.
#include "common.hpp"

namespace mgpt {
namespace {

// Large dispatches (E x nb beyond kFoldScan): one block per expert scans
// hist[e][0..nb) into base[e][.] (the assignments of the router blocks
// before b) and counts[e]; the permute blocks then read their bases.
__global__ __launch_bounds__(256) void expert_scan_kernel(const int32_t* __restrict__ hist, int nb,
                                                          int32_t* __restrict__ base,
                                                          int32_t* __restrict__ counts) {
  __shared__ int s_wave[4];
  __shared__ int s_carry;
  const int e = blockIdx.x;
  const int tid = threadIdx.x;
  const int w = tid / kWave;
  if (tid == 0) s_carry = 0;
  __syncthreads();
  for (int b0 = 0; b0 < nb; b0 += 256) {
    const int b = b0 + tid;
    const int v = (b < nb) ? hist[(size_t)e * nb + b] : 0;
    const int incl = wave_incl_scan(v);
    if (lane_id() == kWave - 1) s_wave[w] = incl;
    __syncthreads();
    int pre = s_carry;
    for (int i = 0; i < w; ++i) pre += s_wave[i];
    if (b < nb) base[(size_t)e * nb + b] = pre + incl - v;
    __syncthreads();
    if (tid == 255) s_carry = pre + incl;
    __syncthreads();
  }
  if (tid == 0) counts[e] = s_carry;
}

// Histogram entries (E x nb) up to which each permute block sums the
// columns it needs itself instead of a scan launch: quadratic in nb, so
// cheap only for small dispatches (cfg1-cfg3, decode); measured on MI355X
// the fold saves ~5 us at cfg1/cfg2 and costs ~28 us at cfg4 (E x nb =
// 32768).
constexpr int kFoldScan = 8192;

// 16-byte vector of activations.
struct alignas(16) V16 {
  uint32_t w[4];
};

// The row normalisation of a fused block applied to one 16-byte chunk
// (columns c .. c + 16/sizeof(ActT) - 1): x -> (x * r) * gamma[c], two
// rounded products as the reference's RMSNorm forms them, then rounded to
// the activation type.
__device__ __forceinline__ V16 normalize16(const V16& v, float r, const float* g, float) {
  V16 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o.w[i] = __float_as_uint((__uint_as_float(v.w[i]) * r) * g[i]);
  return o;
}
__device__ __forceinline__ V16 normalize16(const V16& v, float r, const float* g, bf16_t) {
  float gv[8];
  if (((uintptr_t)g & 15) == 0) {   // the chunk's 8 scales as two 16-byte loads
    const float4 g0 = reinterpret_cast<const float4*>(g)[0], g1 = reinterpret_cast<const float4*>(g)[1];
    gv[0] = g0.x; gv[1] = g0.y; gv[2] = g0.z; gv[3] = g0.w;
    gv[4] = g1.x; gv[5] = g1.y; gv[6] = g1.z; gv[7] = g1.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) gv[i] = g[i];
  }
  V16 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = (__uint_as_float(v.w[i] << 16) * r) * gv[2 * i];
    const float b = (__uint_as_float(v.w[i] & 0xFFFF0000u) * r) * gv[2 * i + 1];
    o.w[i] = pack_bf16x2(a, b);
  }
  return o;
}

// One 16-byte chunk of a gathered row (OutT) and the input bytes it comes
// from: the same 16 bytes when the caller's rows have the gather's type, or
// 32 bytes of fp32 rounded to 8 bf16 (RNE) when a fp32 caller feeds bf16
// expert products.  With gamma set (fused block) the fp32 values are
// normalised, (x * r) * gamma[c], before that rounding.
template <typename InT, typename OutT>
struct RowChunk {
  static_assert(sizeof(InT) >= sizeof(OutT), "the gather only narrows");
  static constexpr int kIn = (int)(sizeof(InT) / sizeof(OutT));   // input V16 per output V16
  static constexpr int kPer = 16 / (int)sizeof(OutT);              // columns per chunk
  V16 raw[kIn];
  __device__ __forceinline__ void load(const InT* row, int q) {
#pragma unroll
    for (int i = 0; i < kIn; ++i) raw[i] = reinterpret_cast<const V16*>(row)[q * kIn + i];
  }
  __device__ __forceinline__ V16 out(float r, const float* g) const {
    if constexpr (kIn == 1) {
      return g ? normalize16(raw[0], r, g, OutT()) : raw[0];
    } else {
      V16 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = __uint_as_float(raw[i / 2].w[(2 * i) % 4]);
        float b = __uint_as_float(raw[i / 2].w[(2 * i) % 4 + 1]);
        if (g) {
          a = (a * r) * g[2 * i];
          b = (b * r) * g[2 * i + 1];
        }
        o.w[i] = pack_bf16x2(a, b);
      }
      return o;
    }
  }
};

// One block per (router block of TB tokens = TB*k flat ids, column slice):
// every slice ranks the block's ids (cheap), slice 0 writes perm/slot_of,
// and each slice copies its share of the row bytes.  Slices only matter for
// few tokens (decode shapes), where one block per 64 tokens would leave the
// GPU idle.
template <typename InT, typename ActT>
__global__ __launch_bounds__(256) void permute_kernel(
    const InT* __restrict__ x, const int32_t* __restrict__ topk_idx,
    const int32_t* __restrict__ hist, const int32_t* __restrict__ base, int nb, int N, int C,
    int E, int k, int32_t* __restrict__ counts, int32_t* __restrict__ perm,
    int32_t* __restrict__ slot_of, ActT* __restrict__ xg, const float* __restrict__ rstd,
    const float* __restrict__ gamma) {
  __shared__ int s_base[kMaxExpertsWide];
  __shared__ int s_pre[kMaxExpertsWide];
  __shared__ int s_tot[kMaxExpertsWide];
  __shared__ int s_run[kMaxExpertsWide];
  __shared__ int s_slot[kRouterTokens * kMaxTopK];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const bool writer = blockIdx.y == 0;
  const int TB = router_tokens_per_block(E);
  const int tok0 = b * TB;
  const int ntok = min(TB, N - tok0);
  const int nflat = ntok * k;
  const size_t flat0 = (size_t)tok0 * k;

  // Row copy geometry (used below): this slice's 16-byte chunks [q0, q1);
  // thread t takes chunk q0 + t % W of tokens t / W, t / W + R, ...
  // (W = min(slice width, 256) consecutive threads per row, R = 256 / W
  // rows per step), four tokens in flight before their k stores each.
  using Chunk = RowChunk<InT, ActT>;
  constexpr int U = 4;
  const int chunks = C * (int)sizeof(ActT) / 16;
  const int q0 = (int)((long)blockIdx.y * chunks / gridDim.y);
  const int q1 = (int)((long)(blockIdx.y + 1) * chunks / gridDim.y);
  const int W = min(q1 - q0, 256);
  const int R = 256 / W;
  const int rr = tid / W;
  const int qf = q0 + tid % W;
  // The rows do not depend on the slots: the first batch is loaded before
  // the ranking, so its latency overlaps the histogram and id loads.
  const bool have_pre = rr < R && qf < q1 && rr < ntok;
  Chunk pre[U];
  if (have_pre) {
#pragma unroll
    for (int u = 0; u < U; ++u) pre[u].load(x + (size_t)(tok0 + min(rr + R * u, ntok - 1)) * C, qf);
  }
  // every id of the block, for the ranking wave, loaded up front as well
  constexpr int kIdPerLane = kRouterTokens * kMaxTopK / kWave;
  int ids[kIdPerLane];
  if (tid < kWave) {
#pragma unroll
    for (int u = 0; u < kIdPerLane; ++u) {
      const int f = u * kWave + tid;
      ids[u] = f < nflat ? topk_idx[flat0 + f] : -1;
    }
  }
  for (int f = tid; f < kRouterTokens * kMaxTopK; f += 256) s_slot[f] = -1;
  if (base) {
    // scanned by expert_scan_kernel
    for (int e = tid; e < E; e += 256) {
      s_pre[e] = base[(size_t)e * nb + b];
      s_tot[e] = counts[e];
    }
  } else if (!hist) {
    // a single router block routed without a histogram (nb == 1): count its
    // ids (LDS integer atomics; counts do not depend on their order)
    for (int e = tid; e < E; e += 256) {
      s_pre[e] = 0;
      s_tot[e] = 0;
    }
    __syncthreads();
    for (int f = tid; f < nflat; f += 256) {
      const int e = topk_idx[flat0 + f];
      if (e >= 0 && e < E) atomicAdd(&s_tot[e], 1);
    }
  } else {
    // Per expert: the assignments of the router blocks before this one and
    // of all blocks.  G consecutive lanes of one wave share an expert (G =
    // 256 / E rounded to a power of two, at most 64; 1 past 256 experts),
    // each summing every G-th block, then reduce across the group; 256 / G
    // experts per pass (one pass unless E > 256).
    int ep = 1;
    while (ep < E) ep <<= 1;
    const int G = max(1, min(kWave, 256 / ep));
    const int part = tid % G;
    for (int e0 = 0; e0 < E; e0 += 256 / G) {
      const int e = e0 + tid / G;
      // 16 loads per lane in flight before the first add (one L2 round trip
      // per 16 entries instead of one per entry)
      constexpr int kHU = 16;
      int pre = 0, tot = 0;
      if (e < E) {
        const int32_t* hrow = hist + (size_t)e * nb;
        for (int bb0 = part; bb0 < nb; bb0 += kHU * G) {
          int v[kHU];
#pragma unroll
          for (int u = 0; u < kHU; ++u) {
            const int bb = bb0 + u * G;
            v[u] = bb < nb ? hrow[bb] : 0;
          }
#pragma unroll
          for (int u = 0; u < kHU; ++u) {
            tot += v[u];
            if (bb0 + u * G < b) pre += v[u];
          }
        }
      }
      for (int d = G / 2; d >= 1; d >>= 1) {
        pre += __shfl_xor(pre, d, kWave);
        tot += __shfl_xor(tot, d, kWave);
      }
      if (e < E && part == 0) {
        s_pre[e] = pre;
        s_tot[e] = tot;
      }
    }
  }
  __syncthreads();
  if (tid < kWave) {
    // Exclusive offsets of the experts, then this block's bases; block
    // (0, 0) publishes the counts for the GEMMs and the caller.  A wave
    // scans 64 experts at a time, carrying the total forward.
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += kWave) {
      const int l = e0 + tid;
      const int cnt = (l < E) ? s_tot[l] : 0;
      const int incl = wave_incl_scan(cnt);
      if (l < E) {
        s_base[l] = carry + incl - cnt + s_pre[l];
        s_run[l] = 0;
        if (!base && writer && b == 0) counts[l] = cnt;
      }
      carry += __shfl(incl, kWave - 1, kWave);
    }
  }
  __syncthreads();
  if (tid < kWave) {
    const int l = tid;
    const unsigned long long lt = (l == 0) ? 0ull : (~0ull >> (kWave - l));
    const int id_bits = E > 256 ? 9 : (E > kMaxExperts ? 8 : 6);
#pragma unroll
    for (int u = 0; u < kIdPerLane; ++u) {
      const int f0 = u * kWave;
      if (f0 >= nflat) break;
      const int f = f0 + l;
      int e = ids[u];
      // Ids outside [0, E) are skipped, as the reference's histogram and
      // gather skip them (utils/Tensor.cpp:1348, :1368).
      const bool valid = e >= 0 && e < E;
      if (!valid) e = 0;
      unsigned long long match = __ballot(valid);
#pragma unroll
      for (int bit = 0; bit < 9; ++bit) {
        if (bit >= id_bits) break;   // ids < 2^id_bits
        const unsigned long long on = __ballot(valid && ((e >> bit) & 1));
        match &= ((e >> bit) & 1) ? on : ~on;
      }
      if (valid) {
        const int run = s_run[e];
        const int rank = run + __popcll(match & lt);
        const int slot = s_base[e] + rank;
        s_slot[f] = slot;
        if (writer) {
          perm[slot] = (int32_t)(flat0 + f);
          slot_of[flat0 + f] = slot;
        }
        // The highest lane of each expert group advances the running count.
        if ((match >> l) == 1ull) s_run[e] = run + __popcll(match);
      }
    }
  }
  __syncthreads();
  // Row copy (a narrow slice still keeps nearly every lane busy).
  if (rr < R) {
    for (int q = qf; q < q1; q += W) {
      for (int r0 = rr; r0 < ntok; r0 += R * U) {
        Chunk in[U];
        if (q == qf && r0 == rr) {
#pragma unroll
          for (int u = 0; u < U; ++u) in[u] = pre[u];
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int r = min(r0 + R * u, ntok - 1);
            in[u].load(x + (size_t)(tok0 + r) * C, q);
          }
        }
        V16 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          // fused block: gather the normalised rows
          const int r = min(r0 + R * u, ntok - 1);
          v[u] = gamma ? in[u].out(rstd[tok0 + r], gamma + q * Chunk::kPer)
                       : in[u].out(1.0f, nullptr);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int r = r0 + R * u;
          if (r >= ntok) break;
          for (int j = 0; j < k; ++j) {
            const int slot = s_slot[r * k + j];
            if (slot < 0) continue;
            reinterpret_cast<V16*>(xg + (size_t)slot * C)[q] = v[u];
          }
        }
      }
    }
  }
}

}  // namespace

// rstd / gamma (both null, or both set): the fused block gathers
// (x * rstd[t]) * gamma instead of x.  InT: the caller's rows (fp32 rows may
// feed a bf16 gather); ActT: the gathered rows.
template <typename InT, typename ActT>
hipError_t launch_permute(const InT* x, const int32_t* topk_idx, const int32_t* hist,
                          int32_t* base, int N, int C, int E, int k, int32_t* counts,
                          int32_t* perm, int32_t* slot_of, ActT* xg, const float* rstd,
                          const float* gamma, hipStream_t stream) {
  const int TB = router_tokens_per_block(E);
  const int nb = (N + TB - 1) / TB;
  if (nb == 0) return hipSuccess;
  const bool fold = E * nb <= kFoldScan;
  if (!hist && nb != 1) return hipErrorInvalidValue;   // counting the ids needs one block
  if (E > kMaxExpertsWide) return hipErrorInvalidValue;
  if (!fold)
    hipLaunchKernelGGL(expert_scan_kernel, dim3(E), dim3(256), 0, stream, hist, nb, base, counts);
  // Column slices: enough blocks for ~512 in all, each slice >= 8 chunks
  // (128 bytes of a row).
  const int chunks = C * (int)sizeof(ActT) / 16;
  const int slices = max(1, min(chunks / 8, (512 + nb - 1) / nb));
  hipLaunchKernelGGL((permute_kernel<InT, ActT>), dim3(nb, slices), dim3(256), 0, stream, x, topk_idx,
                     hist, fold ? nullptr : base, nb, N, C, E, k, counts, perm, slot_of, xg, rstd,
                     gamma);
  return hipGetLastError();
}

template hipError_t launch_permute<float, float>(const float*, const int32_t*, const int32_t*,
                                                 int32_t*, int, int, int, int, int32_t*,
                                                 int32_t*, int32_t*, float*, const float*,
                                                 const float*, hipStream_t);
template hipError_t launch_permute<bf16_t, bf16_t>(const bf16_t*, const int32_t*, const int32_t*,
                                                   int32_t*, int, int, int, int, int32_t*,
                                                   int32_t*, int32_t*, bf16_t*, const float*,
                                                   const float*, hipStream_t);
template hipError_t launch_permute<float, bf16_t>(const float*, const int32_t*, const int32_t*,
                                                  int32_t*, int, int, int, int, int32_t*,
                                                  int32_t*, int32_t*, bf16_t*, const float*,
                                                  const float*, hipStream_t);

}  // namespace mgpt
