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
// accumulation order differs.  The weights of a wave are wave-uniform
// (broadcast loads).  Phase 2: per-token max (strict '>' from
// element 0, as the reference, so NaN handling matches), the exponentials
// in parallel with glibc's expf algorithm, then per token the sequential
// sum, the clamp and the insertion top-k in registers.  Phase 3: block-local
// expert histogram (LDS atomics on ints; counts are order-free), written
// expert-major as hist[e][block] for the per-expert scan of dispatch.hip.
// Decode shapes (few tokens, E > 16) split phase 1 over more blocks, one
// expert per wave, through a logits buffer.
#include <type_traits>

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

// Top-k of one token shared by L lanes of a wave (L a power of two, lanes
// L*r .. L*r+L-1): lane q runs the reference's insertion top-k over its
// experts v = q, q+L, ... in ascending order, then log2(L) merge rounds
// with the partner lanes (q^1, q^2, ...) combine the lists.  The insertion top-k with a
// strict '>' over ascending ids keeps exactly the k largest under the total
// order (p descending, id ascending), so merging lists under that order
// gives the reference's result.  A merge takes the elementwise better of
// one list and the other reversed (the top KP of both, as a bitonic
// sequence) and sorts it with a bitonic network.
__device__ __forceinline__ bool topk_before(float pa, int ea, float pb, int eb) {
  return pa > pb || (pa == pb && ea < eb);
}

template <int KP>
__device__ __forceinline__ void topk_merge_lanes(float (&ov)[KP], int (&oi)[KP], int mask) {
  float pv[KP];
  int pi[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    pv[j] = __shfl_xor(ov[j], mask);
    pi[j] = __shfl_xor(oi[j], mask);
  }
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    if (!topk_before(ov[j], oi[j], pv[KP - 1 - j], pi[KP - 1 - j])) {
      ov[j] = pv[KP - 1 - j];
      oi[j] = pi[KP - 1 - j];
    }
  }
#pragma unroll
  for (int d = KP / 2; d >= 1; d /= 2)
#pragma unroll
    for (int i = 0; i < KP; ++i)
      if ((i & d) == 0 && !topk_before(ov[i], oi[i], ov[i + d], oi[i + d])) {
        const float tp = ov[i];
        ov[i] = ov[i + d];
        ov[i + d] = tp;
        const int ti = oi[i];
        oi[i] = oi[i + d];
        oi[i + d] = ti;
      }
}

// The chosen experts are counted into hist[e * hist_stride] (LDS or global
// memory, integer atomics: the counts do not depend on the order).
template <int K>
__device__ __forceinline__ void softmax_topk_lanes(const float* __restrict__ ex, float inv, int E,
                                                  int q, int L, bool write,
                                                  int32_t* __restrict__ idx_out,
                                                  float* __restrict__ p_out, int* hist,
                                                  int hist_stride = 1) {
  constexpr int KP = K <= 1 ? 1 : (K <= 2 ? 2 : (K <= 4 ? 4 : 8));
  float lv[K];
  int li[K];
#pragma unroll
  for (int j = 0; j < K; ++j) { lv[j] = -1e9f; li[j] = -1; }
  for (int v = q; v < E; v += L) {
    const float p = fminf(fmaxf(ex[v] * inv, 1e-7f), 1.0f);
    topk_insert<K>(lv, li, p, v);
  }
  // unfilled entries (a lane with fewer than k experts) sort last
  float ov[KP];
  int oi[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const bool real = j < K && li[j < K ? j : 0] >= 0;
    ov[j] = real ? lv[j < K ? j : 0] : -1e9f;
    oi[j] = real ? li[j < K ? j : 0] : 0x7fffffff;
  }
  for (int mask = 1; mask < L; mask <<= 1) topk_merge_lanes<KP>(ov, oi, mask);
  if (write && q == 0) {
#pragma unroll
    for (int j = 0; j < K; ++j) {
      idx_out[j] = oi[j];
      p_out[j] = ov[j];
      atomicAdd(&hist[oi[j] * hist_stride], 1);
    }
  }
}

// Element i of a 16-byte row unit, widened to fp32 (bf16: a shift or a
// mask; fp32: as is).
template <typename ActT>
__device__ __forceinline__ float widen(const uint4& q, int i);
template <>
__device__ __forceinline__ float widen<bf16_t>(const uint4& q, int i) {
  const uint32_t w = (i < 2) ? q.x : (i < 4) ? q.y : (i < 6) ? q.z : q.w;
  return __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
}
template <>
__device__ __forceinline__ float widen<float>(const uint4& q, int i) {
  return __uint_as_float((i == 0) ? q.x : (i == 1) ? q.y : (i == 2) ? q.z : q.w);
}

typedef __attribute__((address_space(3))) char lds_char;

// One 1 KB direct-to-LDS load (lane l's 16 bytes at g land at lds + 16*l),
// as inline asm the compiler does not track; the caller waits for it.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}

// All of this wave's loads landed and its LDS accesses completed, then the
// workgroup barrier.
__device__ __forceinline__ void drain_barrier() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// This wave's LDS accesses completed, then the workgroup barrier (the
// direct-to-LDS loads in flight are not waited for).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// LDS budget of the logit stage: two buffers of (x chunk + weight chunk).
constexpr int kRouterLds = 96 * 1024;
#ifndef MGPT_SOFTMAX_THREADS
#define MGPT_SOFTMAX_THREADS 1024   // threads of the split path's softmax block
#endif
// The split path (few tokens, E > 16) has no softmax stage in its kernel and
// spends the whole budget on the logit stage's buffers.
#ifndef MGPT_ROUTER_SPLIT_LDS_KB
#define MGPT_ROUTER_SPLIT_LDS_KB 96
#endif
constexpr int kRouterSplitLds = MGPT_ROUTER_SPLIT_LDS_KB * 1024;

// LDS bytes of one group's weight chunk: whole 1 KB DMA blocks.
__device__ __forceinline__ int wgroup_bytes(int CB, int RE) { return max(CB * RE * 4, 1024); }

// Extra LDS a kernel that runs normalised rows provides beyond the stage
// budget, for the chunk's kRT fp32 normalised rows.
constexpr int kRouterNormLds = 32 * 1024;

// Columns per chunk: the largest power of two >= 64 whose two stages fit
// lds_bytes, or, with normalised rows, whose two stages and kRT x CB fp32
// rows fit lds_bytes + kRouterNormLds.  (Every case the launchers make gives
// bf16 rows of >= 256 bytes, 16 swizzle slots: two stages at 16 waves x 4
// experts and CB = 128 take 96 KB.)
template <typename ActT>
__device__ __forceinline__ int chunk_cols(int nw, int RE, int lds_bytes, bool norm) {
  auto stage = [&](int cb) { return kRT * cb * (int)sizeof(ActT) + nw * wgroup_bytes(cb, RE); };
  auto need = [&](int cb) { return 2 * stage(cb) + (norm ? kRT * cb * 4 : 0); };
  const int budget = lds_bytes + (norm ? kRouterNormLds : 0);
  int CB = 64;
  while (need(2 * CB) <= budget) CB *= 2;
  return CB;
}

// The logits of experts [g*RE, g*RE + RE) for the block's 64 tokens (one
// per lane), computed by the nw waves of a block (all threads call this;
// the weights of groups past g_valid are not loaded and those waves'
// results are garbage).  xblk is the block's first token row (rows past
// the last token, n_rows, re-read the last one); wsrc is packed [G][C][RE]
// from the block's first group on.
//
// Both operands are staged through LDS in column chunks, double-buffered
// and requested one chunk ahead with direct-to-LDS loads: every lane reads
// its own token row, so reading x straight from memory would touch 64
// cache lines per load instruction in every wave of the block (the load
// pipeline, not the VALU, bound that design); staged, each row is fetched
// once per block with whole-line loads.  Row units are swizzled (unit u of
// row r at slot u ^ (r & 15)) so the 16 rows read together hit 16 bank
// groups; the weights are the same for every lane of a wave (broadcast
// reads).  Each logit accumulates c = 0, 1, ... in order, one rounded
// product and one rounded add per term (built with -ffp-contract=off); the
// caller adds the bias.
// Row normalisation fused into the router (the engine's ln2 RMSNormLayer,
// utils/Tensor.cpp:785-800): with gamma set, a first pass over the staged
// chunks sums x^2 of the lane's row in column order, r = 1/sqrt(ms/C + eps)
// with IEEE division and square root, and the logits then use
// (x * r) * gamma[c], two rounded products as the reference forms them.
struct RowNorm {
  const float* gamma;   // null: no normalisation
  float eps;
  int cn;               // the row's true width (the mean's divisor; the
                        // columns past it are zero padding and add +0)
};

// Correctly rounded square root of a positive normal y.  The hardware
// v_sqrt_f32 is within an ulp but not always the nearest float, so the
// estimate s is corrected by the sign of the exact residuals y - s_-*s and
// y - s_+*s of its neighbours (one fused multiply-add each; the classic
// residual test for a one-ulp-accurate square root, Muller et al.,
// Handbook of Floating-Point Arithmetic, ch. 5): residuals are multiples
// of ulp(s)^2, so their signs decide the rounding exactly.
__device__ __forceinline__ float sqrt_rn(float y) {
  const float s = __builtin_amdgcn_sqrtf(y);
  if (!(y >= 0x1p-100f && y <= 0x1p100f)) return s;   // outside the normalisation's range
  const float sd = __uint_as_float(__float_as_uint(s) - 1u);
  const float su = __uint_as_float(__float_as_uint(s) + 1u);
  if (__builtin_fmaf(-sd, s, y) <= 0.0f) return sd;
  if (__builtin_fmaf(-su, s, y) > 0.0f) return su;
  return s;
}

template <typename ActT, int RE, bool NORM>
__device__ __forceinline__ void logit_chains(const ActT* __restrict__ xblk, int n_rows,
                                             const float* __restrict__ wsrc, int g_valid, int nw,
                                             int g, int C, char* smem, float (&acc)[RE],
                                             RowNorm nrm, float* r_out,
                                             int lds_bytes = kRouterLds) {
  constexpr int kPer = 16 / (int)sizeof(ActT);   // columns per 16-byte unit
  const int CB = chunk_cols<ActT>(nw, RE, lds_bytes, NORM);
  const int xrow_bytes = CB * (int)sizeof(ActT);   // LDS bytes per token row
  const int x_bytes = kRT * xrow_bytes;
  const int wgb = wgroup_bytes(CB, RE);
  const int w_bytes = nw * wgb;
  const int stage_bytes = x_bytes + w_bytes;
  const int lane = lane_id();
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)smem;
  const size_t xrow_g = (size_t)C * sizeof(ActT);

  // One chunk [c0, c0 + cnum) into stage b.  x: 1 KB blocks of whole rows
  // segments (xrow_bytes is a multiple of 128), lane l -> row
  // (blk*1024 + 16l) / xrow_bytes, slot s -> logical unit s ^ (row & 15).
  // Weights: group gg's cnum*RE floats in 1 KB blocks at a 1 KB-aligned
  // group stride; lanes past a partial block re-read the group's first
  // bytes (in bounds, never used).
  // the x part, rows of xrow bytes at dst
  auto x_dma = [&](int c0, int cnum, uint32_t dst, int xrow) __attribute__((always_inline)) {
    const int units_row = cnum * (int)sizeof(ActT) / 16;   // valid units per row
    const int x_blocks = kRT * xrow / 1024;
    for (int q = g; q < x_blocks; q += nw) {
      const int byte = q * 1024 + lane * 16;
      const int row = byte / xrow, slot = (byte % xrow) / 16;
      int unit = slot ^ (row & 15);
      if (unit >= units_row) unit = 0;
      const char* src = reinterpret_cast<const char*>(xblk) +
                        (size_t)min(row, n_rows - 1) * xrow_g + (size_t)c0 * sizeof(ActT) +
                        unit * 16;
      dma16(src, dst + (uint32_t)(q * 1024));
    }
  };
  auto chunk_dma = [&](int c0, int cnum, int b) __attribute__((always_inline)) {
    const uint32_t st = lds0 + (uint32_t)(b * stage_bytes);
    x_dma(c0, cnum, st, xrow_bytes);
    const int gbytes = cnum * RE * 4;
    const int gblocks = (gbytes + 1023) / 1024;
    for (int q = g; q < g_valid * gblocks; q += nw) {
      const int gg = q / gblocks, bk = q - gg * gblocks;
      const char* src = reinterpret_cast<const char*>(wsrc + ((size_t)gg * C + c0) * RE);
      const int off = bk * 1024 + lane * 16;
      dma16(src + (off < gbytes ? off : 0), st + (uint32_t)(x_bytes + gg * wgb + bk * 1024));
    }
  };

#pragma unroll
  for (int j = 0; j < RE; ++j) acc[j] = 0.0f;
  constexpr int kWU = kPer * RE / 4;   // float4 of weights per unit
  int b = 0;
  float r = 1.0f;
  // fused block: kRT fp32 normalised rows of the current chunk, 16-byte
  // units of row t at slot unit ^ (t & xn_sw), after the two stages
  float* xn_lds = reinterpret_cast<float*>(smem + 2 * stage_bytes);
  __shared__ float s_rr[kRT];
  if constexpr (NORM) {
    // pass 1: the row's sum of squares, columns in order (one chain per
    // token, so one wave forms them while the others only keep the chunks
    // moving; the result goes to every wave through LDS)
    // x alone in chunks of CB1 >= CB columns, the whole budget for two
    // stages (fewer, longer DMA rounds: this pass does little arithmetic)
    const int budget = lds_bytes + kRouterNormLds;
    int CB1 = CB;
    while (CB1 < C && 2 * kRT * (2 * CB1) * (int)sizeof(ActT) <= budget) CB1 *= 2;
    const int xrow1 = CB1 * (int)sizeof(ActT);
    const int st1 = kRT * xrow1;
    float ms = 0.0f;
    x_dma(0, min(CB1, C), lds0, xrow1);
    for (int c0 = 0; c0 < C; c0 += CB1) {
      const int cnum = min(CB1, C - c0);
      drain_barrier();
      if (c0 + CB1 < C)
        x_dma(c0 + CB1, min(CB1, C - c0 - CB1), lds0 + (uint32_t)((b ^ 1) * st1), xrow1);
      if (g == 0) {
        const char* xr = smem + b * st1 + lane * xrow1;
        for (int u = 0; u < cnum / kPer; ++u) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xr + ((u ^ (lane & 15)) << 4));
#pragma unroll
          for (int i = 0; i < kPer; ++i) {
            const float v = widen<ActT>(xv, i);
            ms = ms + v * v;
          }
        }
      }
      b ^= 1;
    }
    if (g == 0) s_rr[lane] = __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(ms, (float)nrm.cn) + nrm.eps));
    drain_barrier();   // r published; every wave done with the stages before they are refilled
    r = s_rr[lane];
    if (r_out) *r_out = r;
    b = 0;
  }
  chunk_dma(0, min(CB, C), 0);
  for (int c0 = 0; c0 < C; c0 += CB) {
    const int cnum = min(CB, C - c0);
    drain_barrier();   // chunk c0 landed; every wave done with the other stage
    if (c0 + CB < C) chunk_dma(c0 + CB, min(CB, C - c0 - CB), b ^ 1);
    const char* st = smem + b * stage_bytes;
    const char* xr = st + lane * xrow_bytes;
    const float* wq = reinterpret_cast<const float*>(st + x_bytes + g * wgb);
    const int units = cnum / kPer;
    if constexpr (!NORM) {
      // operands of unit u+1 are read while unit u is multiplied
      uint4 x0, x1;
      float4 w0[kWU], w1[kWU];
      auto rd = [&](int u, uint4& xv, float4 (&wv)[kWU]) __attribute__((always_inline)) {
        xv = *reinterpret_cast<const uint4*>(xr + ((u ^ (lane & 15)) << 4));
#pragma unroll
        for (int v = 0; v < kWU; ++v)
          wv[v] = reinterpret_cast<const float4*>(wq + u * kPer * RE)[v];
      };
      auto mul_add = [&](const uint4& xv, const float4 (&wv)[kWU]) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < kWU; ++v) {
          const float w4[4] = {wv[v].x, wv[v].y, wv[v].z, wv[v].w};
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const int idx = 4 * v + e4;   // = column * RE + expert
            acc[idx % RE] = acc[idx % RE] + widen<ActT>(xv, idx / RE) * w4[e4];
          }
        }
      };
      rd(0, x0, w0);
      for (int u = 0; u < units; u += 2) {   // units is even (cnum % 64 == 0)
        rd(u + 1, x1, w1);
        mul_add(x0, w0);
        if (u + 2 < units) rd(u + 2, x0, w0);
        mul_add(x1, w1);
      }
    } else {
      // normalised: every thread of the block turns some of the chunk's
      // 16-byte units into (x * r[t]) * gamma[c] in fp32 (the values each
      // product takes), then every wave reads them; the row-to-lane and
      // unit-to-slot maps match the x chunk's (slot = unit ^ (t & 15) for
      // ActT, 2*unit + h ^ (t & 31) or unit ^ (t & 31) for the fp32 rows)
      constexpr int kXnU = kPer / 4;   // fp32 units per ActT unit
      const int xn_row = CB * 4;        // bytes
      const int xn_sw = min(31, CB / 4 - 1);   // slot mask: 16-byte units per fp32 row - 1
      const int nthr = nw * kWave;
      for (int p = g * kWave + lane; p < kRT * units; p += nthr) {
        const int t = p / units, u = p - t * units;
        const uint4 xv = *reinterpret_cast<const uint4*>(st + t * xrow_bytes + ((u ^ (t & 15)) << 4));
        const float rt = s_rr[t];
        float o[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) o[i] = (widen<ActT>(xv, i) * rt) * nrm.gamma[c0 + u * kPer + i];
#pragma unroll
        for (int h = 0; h < kXnU; ++h)
          *reinterpret_cast<float4*>(reinterpret_cast<char*>(xn_lds) + t * xn_row +
                                     (((u * kXnU + h) ^ (t & xn_sw)) << 4)) =
              make_float4(o[4 * h], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
      }
      lds_barrier();
      const char* xnr = reinterpret_cast<const char*>(xn_lds) + lane * xn_row;
      for (int u = 0; u < units; ++u) {
        float4 wv[kWU];
#pragma unroll
        for (int v = 0; v < kWU; ++v)
          wv[v] = reinterpret_cast<const float4*>(wq + u * kPer * RE)[v];
        float xn[kPer];
#pragma unroll
        for (int h = 0; h < kXnU; ++h) {
          const float4 q =
              *reinterpret_cast<const float4*>(xnr + (((u * kXnU + h) ^ (lane & xn_sw)) << 4));
          xn[4 * h] = q.x;
          xn[4 * h + 1] = q.y;
          xn[4 * h + 2] = q.z;
          xn[4 * h + 3] = q.w;
        }
#pragma unroll
        for (int v = 0; v < kWU; ++v) {
          const float w4[4] = {wv[v].x, wv[v].y, wv[v].z, wv[v].w};
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const int idx = 4 * v + e4;
            acc[idx % RE] = acc[idx % RE] + xn[idx / RE] * w4[e4];
          }
        }
      }
      lds_barrier();   // every wave done with this chunk's fp32 rows
    }
    b ^= 1;
  }
  drain_barrier();   // the block may reuse the LDS after this
}

// Softmax, top-k and histogram of the block's kRT tokens for E <= 32, with
// no cross-lane traffic: each wave takes 64 / EP tokens at a time (EP = E
// rounded up to a power of two), lane e of a token's group of EP lanes
// holding expert e, and every lane runs the token's reductions itself over
// the row in LDS, in the reference's order: the running max from element 0
// with a strict '>' (NaN handling as the reference's), the glibc expf, the
// sequential sum and clamp, and its rank under (p descending, id
// ascending), which is the insertion top-k's order.  The entries past E
// are made neutral (-inf for the max, +0 for the sum, which is never -0, 0
// for the ranks, below every clamped probability), so every pass runs over
// EP entries without branches.  The choices are counted into s_hist with
// LDS atomics.  (The layout used for E > 32, L lanes per token merging
// partial maxima and top-k lists with shuffles, took 8.2 k cycles per block
// at cfg3 against 6.2 k here, barriers included.)
template <int EP, int LD = kMaxExperts + 1>
__device__ __forceinline__ void softmax_topk_group(float (*s_l)[LD], int* s_hist,
                                                   const uint64_t* tab, int tok0, int N, int E,
                                                   int k, int32_t* __restrict__ topk_idx,
                                                   float* __restrict__ topk_p,
                                                   float* __restrict__ probs) {
  constexpr int G = kWave / EP;   // tokens per wave and pass
  const int lane = lane_id();
  const int w = (int)threadIdx.x / kWave, nw = (int)blockDim.x / kWave;
  const int e = lane % EP;
  const bool mine = e < E;
  for (int r0 = w * G; r0 < kRT; r0 += nw * G) {
    const int r = r0 + lane / EP;
    float* row = s_l[r];
    float v[EP];
    auto load_row = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < EP; ++i) v[i] = row[i];
    };
    auto publish = [&](float value) __attribute__((always_inline)) {
      __builtin_amdgcn_wave_barrier();   // every lane has read the row
      row[e] = value;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    const float l = row[e];
    publish(mine ? l : -INFINITY);
    load_row();
    float m = v[0];
#pragma unroll
    for (int i = 1; i < EP; ++i)
      if (v[i] > m) m = v[i];
    const float ex = mgpt_expf::expf_glibc(l - m, tab);
    publish(mine ? ex : 0.0f);
    load_row();
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < EP; ++i) sum = sum + v[i];
    const float inv = 1.0f / fmaxf(sum, 1e-15f);
    const float p = fminf(fmaxf(ex * inv, 1e-7f), 1.0f);
    publish(mine ? p : 0.0f);
    load_row();
    int rank = 0;
#pragma unroll
    for (int i = 0; i < EP; ++i) rank += (v[i] > p) || (v[i] == p && i < e);
    const int t = tok0 + r;
    if (mine && t < N) {
      if (probs) probs[(size_t)t * E + e] = p;   // kept for the backward pass
      if (rank < k) {
        topk_idx[(size_t)t * k + rank] = e;
        topk_p[(size_t)t * k + rank] = p;
        atomicAdd(&s_hist[e], 1);
      }
    }
  }
}

// Softmax, top-k and the block histogram of kRT tokens whose logits are in
// s_l (all threads of the block call it).  Per token (L lanes): the
// max as the reference's strict '>' scan from element 0 computes it (so NaN
// handling matches), the exponentials in parallel with glibc's expf
// algorithm, then the sequential sum, the clamp and the top-k
// (softmax_topk_lanes).  The histogram counts are written expert-major as
// hist[e][block].
template <int LD = kMaxExperts + 1>
__device__ __forceinline__ void softmax_topk_block(float (*s_l)[LD], float* s_m,
                                                   int* s_hist, int tok0, int N, int E, int k,
                                                   int32_t* __restrict__ topk_idx,
                                                   float* __restrict__ topk_p,
                                                   int32_t* __restrict__ hist, int num_blocks,
                                                   float* __restrict__ probs) {
  const int tid = threadIdx.x;
  if (E <= 32) {
    __shared__ uint64_t s_tab32[32];
    if (tid < 32) s_tab32[tid] = c_exp2_tab[tid];
    __syncthreads();   // the table, and the logits the caller wrote
    if (E <= 2)
      softmax_topk_group<2, LD>(s_l, s_hist, s_tab32, tok0, N, E, k, topk_idx, topk_p, probs);
    else if (E <= 4)
      softmax_topk_group<4, LD>(s_l, s_hist, s_tab32, tok0, N, E, k, topk_idx, topk_p, probs);
    else if (E <= 8)
      softmax_topk_group<8, LD>(s_l, s_hist, s_tab32, tok0, N, E, k, topk_idx, topk_p, probs);
    else if (E <= 16)
      softmax_topk_group<16, LD>(s_l, s_hist, s_tab32, tok0, N, E, k, topk_idx, topk_p, probs);
    else
      softmax_topk_group<32, LD>(s_l, s_hist, s_tab32, tok0, N, E, k, topk_idx, topk_p, probs);
    __syncthreads();
    if (tid < E) hist[(size_t)tid * num_blocks + blockIdx.x] = s_hist[tid];
    return;
  }
  // L lanes per token: the largest power of two <= min(16, blockDim / 64),
  // so that the kRT tokens use (most of) the block
  int L = 1;
  while (2 * L <= 16 && 2 * L * kRT <= (int)blockDim.x) L *= 2;
  const int q = tid & (L - 1);
  const int groups = blockDim.x / L;
  // expf's 2^(i/32) table in LDS: read per lane at a data-dependent index,
  // from global memory each lookup would put a load round trip on the
  // critical path of every exponential
  __shared__ uint64_t s_tab[32];
  if (tid < 32) s_tab[tid] = c_exp2_tab[tid];
  // max per token (its L lanes): the maximum over the non-NaN logits,
  // unless logit 0 is NaN (the reference's running max starts at element 0
  // and '>' never replaces a NaN, nor picks one later)
  for (int r = tid / L; r < kRT; r += groups) {
    float m = -INFINITY;
    for (int v = q; v < E; v += L) {
      const float l = s_l[r][v];
      if (l > m) m = l;
    }
    for (int mask = 1; mask < L; mask <<= 1) {
      const float o = __shfl_xor(m, mask);
      if (o > m) m = o;
    }
    const float l0 = s_l[r][0];
    if (l0 != l0) m = l0;
    if (q == 0) s_m[r] = m;
  }
  __syncthreads();
  for (int p = tid; p < kRT * E; p += blockDim.x) {
    const int r = p / E, e = p % E;
    s_l[r][e] = mgpt_expf::expf_glibc(s_l[r][e] - s_m[r], s_tab);
  }
  __syncthreads();
  for (int r = tid / L; r < kRT; r += groups) {
    const float* ex = s_l[r];
    float sum = 0.0f;   // sequential, in expert order (every lane of the token)
    for (int v = 0; v < E; ++v) sum = sum + ex[v];
    const float inv = 1.0f / fmaxf(sum, 1e-15f);
    const bool write = tok0 + r < N;
    if (probs && write)   // the clamped probabilities, kept for the backward pass
      for (int v = q; v < E; v += L)
        probs[(size_t)(tok0 + r) * E + v] = fminf(fmaxf(ex[v] * inv, 1e-7f), 1.0f);
    int32_t* io = topk_idx + (size_t)(tok0 + r) * k;
    float* po = topk_p + (size_t)(tok0 + r) * k;
    switch (k) {
      case 1: softmax_topk_lanes<1>(ex, inv, E, q, L, write, io, po, s_hist); break;
      case 2: softmax_topk_lanes<2>(ex, inv, E, q, L, write, io, po, s_hist); break;
      case 3: softmax_topk_lanes<3>(ex, inv, E, q, L, write, io, po, s_hist); break;
      case 4: softmax_topk_lanes<4>(ex, inv, E, q, L, write, io, po, s_hist); break;
      case 5: softmax_topk_lanes<5>(ex, inv, E, q, L, write, io, po, s_hist); break;
      case 6: softmax_topk_lanes<6>(ex, inv, E, q, L, write, io, po, s_hist); break;
      case 7: softmax_topk_lanes<7>(ex, inv, E, q, L, write, io, po, s_hist); break;
      default: softmax_topk_lanes<8>(ex, inv, E, q, L, write, io, po, s_hist); break;
    }
  }
  __syncthreads();
  if (tid < E) hist[(size_t)tid * num_blocks + blockIdx.x] = s_hist[tid];
}

// Fused router: a block owns kRT tokens (one per lane) and ceil(E/RE) waves;
// wave g computes experts [g*RE, g*RE + RE) into LDS, then the block runs
// softmax, top-k and its histogram.
template <typename ActT, int RE, bool NORM>
__global__ __launch_bounds__(1024) void router_topk_uniform_kernel(
    const ActT* __restrict__ x, const float* __restrict__ wr_g, const float* __restrict__ br,
    int N, int C, int E, int k, int32_t* __restrict__ topk_idx, float* __restrict__ topk_p,
    int32_t* __restrict__ hist, int num_blocks, float* __restrict__ probs, RowNorm nrm,
    float* __restrict__ rstd) {
  __shared__ float s_l[kRT][kMaxExperts + 1];
  __shared__ float s_m[kRT];
  __shared__ int s_hist[kMaxExperts];
  // (NORM: nrm.gamma is set, and the normalised rows need kRouterNormLds more)
  __shared__ __attribute__((aligned(1024))) char smem[kRouterLds + (NORM ? kRouterNormLds : 0)];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int g = __builtin_amdgcn_readfirstlane(tid / kWave);   // expert group of this wave
  const int nw = blockDim.x / kWave;
  const int tok0 = blockIdx.x * kRT;
  if (tid < kMaxExperts) s_hist[tid] = 0;
  float acc[RE];
  float r = 1.0f;
  logit_chains<ActT, RE, NORM>(x + (size_t)tok0 * C, N - tok0, wr_g, nw, nw, g, C, smem, acc, nrm,
                               &r);
  if (NORM && g == 0 && tok0 + lane < N) rstd[tok0 + lane] = r;
#pragma unroll
  for (int j = 0; j < RE; ++j) {
    const int e = g * RE + j;
    if (e < E) s_l[lane][e] = acc[j] + br[e];
  }
  __syncthreads();
  softmax_topk_block(s_l, s_m, s_hist, tok0, N, E, k, topk_idx, topk_p, hist, num_blocks, probs);
}

// Few tokens, many experts (decode shapes): the fused kernel would run a
// handful of blocks whose waves each walk RE experts.  Here a block of
// kSplitExperts waves computes that many experts' logits (one each; wr1 =
// W_r transposed, [E][C]) for 64 tokens, written to global memory, and
// router_softmax_kernel finishes: the chains are as long as before, but
// spread over more CUs.
constexpr int kSplitExperts = 4;
template <typename ActT, bool NORM>
__global__ __launch_bounds__(kSplitExperts * 64) void router_logits_kernel(
    const ActT* __restrict__ x, const float* __restrict__ wr1, const float* __restrict__ br,
    int N, int C, int E, float* __restrict__ logits, RowNorm nrm, float* __restrict__ rstd) {
  __shared__ __attribute__((aligned(1024)))
  char smem[kRouterSplitLds + (NORM ? kRouterNormLds : 0)];
  const int lane = lane_id();
  const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int e0 = blockIdx.y * kSplitExperts;
  const int tok0 = blockIdx.x * kRT;
  float acc[1];
  float r = 1.0f;
  logit_chains<ActT, 1, NORM>(x + (size_t)tok0 * C, N - tok0, wr1 + (size_t)e0 * C,
                        min(kSplitExperts, E - e0), kSplitExperts, g, C, smem, acc, nrm, &r,
                        kRouterSplitLds);
  if (NORM && blockIdx.y == 0 && g == 0 && tok0 + lane < N) rstd[tok0 + lane] = r;
  const int e = e0 + g;
  if (e < E && tok0 + lane < N) logits[(size_t)(tok0 + lane) * E + e] = acc[0] + br[e];
}

// Logits of 64 experts per block for more experts than one router block
// takes: 16 waves x 4 experts, the fused router's chains over the same
// packed weights ([G][C][4]), blockIdx.y the group of 64 experts.  The
// activation rows are read once per group instead of once per 4 experts
// (router_logits_kernel) or per expert (router_logits_pc_kernel); the
// chains and their rounding are the fused router's, so the logits are the
// same bits.  router_softmax_wide_kernel follows.
template <typename ActT, bool NORM>
__global__ __launch_bounds__(1024) void router_logits_wide_kernel(
    const ActT* __restrict__ x, const float* __restrict__ wr_g, const float* __restrict__ br,
    int N, int C, int E, float* __restrict__ logits, RowNorm nrm, float* __restrict__ rstd) {
  constexpr int RE = 4;
  __shared__ __attribute__((aligned(1024))) char smem[kRouterLds + (NORM ? kRouterNormLds : 0)];
  const int lane = lane_id();
  const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int nw = blockDim.x / kWave;
  const int gb = blockIdx.y * nw;   // first weight group of this block
  const int tok0 = blockIdx.x * kRT;
  float acc[RE];
  float r = 1.0f;
  logit_chains<ActT, RE, NORM>(x + (size_t)tok0 * C, N - tok0, wr_g + (size_t)gb * C * RE,
                               min(nw, (E + RE - 1) / RE - gb), nw, g, C, smem, acc, nrm, &r);
  if (NORM && blockIdx.y == 0 && g == 0 && tok0 + lane < N) rstd[tok0 + lane] = r;
  if (tok0 + lane < N) {
#pragma unroll
    for (int j = 0; j < RE; ++j) {
      const int e = (gb + g) * RE + j;
      if (e < E) logits[(size_t)(tok0 + lane) * E + e] = acc[j] + br[e];
    }
  }
}

__global__ __launch_bounds__(1024) void router_softmax_kernel(const float* __restrict__ logits,
                                                             int N, int E, int k,
                                                             int32_t* __restrict__ topk_idx,
                                                             float* __restrict__ topk_p,
                                                             int32_t* __restrict__ hist,
                                                             int num_blocks,
                                                             float* __restrict__ probs) {
  __shared__ float s_l[kRT][kMaxExperts + 1];
  __shared__ float s_m[kRT];
  __shared__ int s_hist[kMaxExperts];
  const int tid = threadIdx.x;
  const int tok0 = blockIdx.x * kRT;
  if (tid < kMaxExperts) s_hist[tid] = 0;
  for (int p = tid; p < kRT * E; p += blockDim.x) {
    const int r = p / E, e = p % E;
    s_l[r][e] = tok0 + r < N ? logits[(size_t)(tok0 + r) * E + e] : 0.0f;
  }
  __syncthreads();
  softmax_topk_block(s_l, s_m, s_hist, tok0, N, E, k, topk_idx, topk_p, hist, num_blocks, probs);
}

// router_softmax_kernel for more experts than a wave has lanes (up to EW <=
// kMaxExpertsWide): the same per-token passes over a wider row in LDS (EW =
// 256 keeps the block's LDS at 66 KB, two blocks per CU; 512 takes 134 KB).
template <int EW>
__global__ __launch_bounds__(1024) void router_softmax_wide_kernel(
    const float* __restrict__ logits, int N, int E, int k, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_p, int32_t* __restrict__ hist, int num_blocks,
    float* __restrict__ probs) {
  __shared__ float s_l[kRT][EW + 1];
  __shared__ float s_m[kRT];
  __shared__ int s_hist[EW];
  const int tid = threadIdx.x;
  const int tok0 = blockIdx.x * kRT;
  if (tid < EW) s_hist[tid] = 0;
  for (int p = tid; p < kRT * E; p += blockDim.x) {
    const int r = p / E, e = p % E;
    s_l[r][e] = tok0 + r < N ? logits[(size_t)(tok0 + r) * E + e] : 0.0f;
  }
  __syncthreads();
  softmax_topk_block<EW + 1>(s_l, s_m, s_hist, tok0, N, E, k, topk_idx, topk_p, hist, num_blocks,
                             probs);
}

// Logits for decode shapes with the products and the chains on different
// waves.  A block owns kRT tokens and one expert e: wave 0 runs the 64
// chains acc = acc + p[c] (lane t = token t, columns ascending, bias last),
// reading four products per 16-byte LDS read, while waves 1-3 (the other
// SIMDs) load x and W_r[e] and write the products p[t][c] = x[t][c] *
// W_r[e][c] of the next 128-column chunk into the other half of a double
// buffer.  The chain wave then issues one add and a quarter of an LDS read
// per column instead of a product, an add and two half reads; the rounding
// sequence (one rounded product, one rounded add per term) is unchanged.
// Loads run two chunks ahead in registers.  hist[e][block] is cleared for
// router_softmax_wave_kernel.  Measured at cfg5 (64 tokens, C = 2048, E =
// 64): 15 us, against 23 us for four experts' chains per block with each
// wave forming its own products; the chains alone (products skipped) take
// 10.8 us, 2048 dependent fp32 adds of about 11 cycles each, which no
// block shape shortens.
template <int V>
struct IntC {
  static constexpr int value = V;
};
constexpr int kPcCB = 128;            // columns per chunk
constexpr int kPcLD = kPcCB + 4;      // floats per LDS product row
constexpr int kPcTokStep = 6;         // tokens between one lane's pieces (192 lanes / 32 quads)
constexpr int kPcPieces = (kRT + kPcTokStep - 1) / kPcTokStep;   // pieces per lane and chunk
// register stages: loads run two chunks ahead (three measured no faster)
constexpr int kPcStages = 3;
template <typename ActT> struct PcPiece;
template <> struct PcPiece<bf16_t> {
  using type = uint2;   // 4 bf16
  __device__ static float4 widen(const uint2& q) {
    return make_float4(__uint_as_float(q.x << 16), __uint_as_float(q.x & 0xFFFF0000u),
                       __uint_as_float(q.y << 16), __uint_as_float(q.y & 0xFFFF0000u));
  }
};
template <> struct PcPiece<float> {
  using type = uint4;   // 4 fp32
  __device__ static float4 widen(const uint4& q) {
    return make_float4(__uint_as_float(q.x), __uint_as_float(q.y), __uint_as_float(q.z),
                       __uint_as_float(q.w));
  }
};
template <typename ActT>
__global__ __launch_bounds__(256) void router_logits_pc_kernel(
    const ActT* __restrict__ x, const float* __restrict__ wr1, const float* __restrict__ br,
    int N, int C, int E, float* __restrict__ logits, int32_t* __restrict__ hist, int nb) {
  __shared__ float4 s_p[2][kRT * kPcLD / 4];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int tok0 = blockIdx.x * kRT;
  const int e = blockIdx.y;
  const int last_row = min(kRT, N - tok0) - 1;
  if (e == 0 && tid < E) hist[(size_t)tid * nb + blockIdx.x] = 0;
  const int nch = (C + kPcCB - 1) / kPcCB;
  auto cols = [&](int ch) { return min(kPcCB, C - ch * kPcCB); };   // a multiple of 64
  if (w == 0) {
    float acc = 0.0f;
    const float4* prow0 = &s_p[0][lane * kPcLD / 4];
    const float4* prow1 = &s_p[1][lane * kPcLD / 4];
    auto consume = [&](int ch) __attribute__((always_inline)) {
      const float4* pr = (ch & 1) ? prow1 : prow0;
      // all of the chunk's reads first (the scheduler otherwise keeps one
      // or two ahead and the chain waits an LDS latency every 8 columns)
      auto run = [&](auto n4_c) __attribute__((always_inline)) {
        constexpr int n4 = decltype(n4_c)::value;
        float4 p[n4];
#pragma unroll
        for (int u = 0; u < n4; ++u) p[u] = pr[u];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < n4; ++u) {
          acc = acc + p[u].x;
          acc = acc + p[u].y;
          acc = acc + p[u].z;
          acc = acc + p[u].w;
        }
      };
      if (cols(ch) == kPcCB)
        run(IntC<kPcCB / 4>{});
      else
        run(IntC<16>{});   // a last chunk of 64 columns
    };
    for (int i = 0; i <= nch; ++i) {
      if (i >= 1) consume(i - 1);
      __syncthreads();
    }
    if (lane <= last_row) logits[(size_t)(tok0 + lane) * E + e] = acc + br[e];
  } else {
    using PT = PcPiece<ActT>;
    using Piece = typename PT::type;
    const int pl = (w - 1) * kWave + lane;   // 0 .. 191
    const int c4 = pl % 32;                  // this lane's column quad in every chunk
    const int tq = pl / 32;                  // its first token; then every kPcTokStep-th
    const float* wrow = wr1 + (size_t)e * C;
    Piece xs[kPcStages][kPcPieces];
    float4 ws[kPcStages];
    // Every lane issues the same loads in every chunk (lanes past a 64-column
    // last chunk read a column quad that is in bounds and skip its
    // products): with a lane-dependent load count the compiler can only
    // wait for all loads (vmcnt(0)), which would also wait for the chunk
    // requested two ahead.
    auto load = [&](int ch, Piece (&xv)[kPcPieces], float4& wv) __attribute__((always_inline)) {
      const int c0 = ch * kPcCB + min(4 * c4, cols(ch) - 4);
#pragma unroll
      for (int j = 0; j < kPcPieces; ++j) {
        const int t = min(tq + kPcTokStep * j, last_row);
        xv[j] = *reinterpret_cast<const Piece*>(x + (size_t)(tok0 + t) * C + c0);
      }
      wv = *reinterpret_cast<const float4*>(wrow + c0);
    };
    auto compute = [&](int ch, const Piece (&xv)[kPcPieces], const float4& wv)
        __attribute__((always_inline)) {
      if (4 * c4 >= cols(ch)) return;
      float4* dst = s_p[ch & 1];
      // every product first, then the LDS writes: the chain wave's reads of
      // the previous chunk (issued at the same barrier) meet fewer writes
      float4 pv[kPcPieces];
#pragma unroll
      for (int j = 0; j < kPcPieces; ++j) {
        const float4 xf = PT::widen(xv[j]);
        pv[j] = make_float4(xf.x * wv.x, xf.y * wv.y, xf.z * wv.z, xf.w * wv.w);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < kPcPieces; ++j) {
        const int t = tq + kPcTokStep * j;
        if (t < kRT) dst[(t * kPcLD) / 4 + c4] = pv[j];
      }
    };
    // iteration i: request chunk i + kPcStages - 1, write chunk i's
    // products, meet the chain wave (which consumes chunk i - 1 meanwhile)
    auto step = [&](int i, auto s_c) __attribute__((always_inline)) {
      constexpr int st = decltype(s_c)::value;                    // chunk i's stage
      constexpr int ahead = (st + kPcStages - 1) % kPcStages;     // i + kPcStages - 1's
      if (i > nch) return;
      // past the last chunk the request repeats it (in bounds, never used),
      // so that every step issues the same loads
      load(min(i + kPcStages - 1, nch - 1), xs[ahead], ws[ahead]);
      if (i < nch) compute(i, xs[st], ws[st]);
      __syncthreads();
    };
#pragma unroll
    for (int j = 0; j < kPcStages - 1; ++j) load(min(j, nch - 1), xs[j], ws[j]);
    for (int i = 0; i <= nch; i += kPcStages) {
      step(i, IntC<0>{});
      step(i + 1, IntC<1>{});
      step(i + 2, IntC<2>{});
      if constexpr (kPcStages > 3) step(i + 3, IntC<3>{});
      static_assert(kPcStages == 3 || kPcStages == 4, "stages");
    }
  }
}

// Softmax, top-k and histogram for decode shapes: one wave per token, lane e
// holding expert e (E <= 64), the row in LDS.  Every lane computes the
// row's reductions itself, in the reference's order: the running max from
// element 0 with a strict '>' (NaN-aware as the reference is), then after the
// exponentials the sequential sum in expert order.  Lane e's rank among the
// clamped probabilities under (p descending, id ascending) -- the order the
// reference's insertion top-k with a strict '>' produces -- is the number of
// experts before it; ranks below k are the choices, written at their rank,
// and counted into hist[e][token / 64] with integer atomics
// (router_logits_pc_kernel cleared those entries).  No shuffles or merge
// rounds: four passes over the row in LDS, latency hidden across lanes.
// The softmax / top-k of one token on one wave (lane e = expert e, l its
// logit), with the row in LDS (row[e] = l for every lane already stored and
// visible to the wave).  hist == nullptr: no histogram (the caller's
// permute counts the ids itself).
// The softmax / top-k of one token on one wave (lane e = expert e, l its
// logit), with the row in LDS: row[e] = l for e < E and -inf for the lanes
// past E, stored by every lane and visible to the wave.  hist == nullptr: no
// histogram (the caller's permute counts the ids itself).
//
// Every pass reads the whole row (kMaxExperts floats, 16-byte aligned) as
// quads, all reads before the arithmetic, and runs over all kMaxExperts
// entries without branches: the lanes past E store neutral entries (-inf
// for the running max, which '>' never takes; +0 for the sum, which is
// never -0 and so is unchanged by adding +0; 0 for the ranks, below every
// clamped probability), and the reductions keep the reference's order.
__device__ __forceinline__ void softmax_topk_wave(float l, bool valid, int t, int e, int E,
                                                  int k, float* row, const uint64_t* tab,
                                                  int32_t* __restrict__ topk_idx,
                                                  float* __restrict__ topk_p,
                                                  int32_t* __restrict__ hist, int nb,
                                                  float* __restrict__ probs) {
  constexpr int kQ = kMaxExperts / 4;
  const float4* row4 = reinterpret_cast<const float4*>(row);
  auto load_row = [&](float (&r)[kMaxExperts]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const float4 v = row4[q];
      r[4 * q] = v.x;
      r[4 * q + 1] = v.y;
      r[4 * q + 2] = v.z;
      r[4 * q + 3] = v.w;
    }
  };
  const bool mine = e < E;
  float r[kMaxExperts];
  load_row(r);
  float m = r[0];
#pragma unroll
  for (int v = 1; v < kMaxExperts; ++v)
    if (r[v] > m) m = r[v];
  const float ex = mgpt_expf::expf_glibc(l - m, tab);
  __builtin_amdgcn_wave_barrier();   // every lane has read the logits
  row[e] = mine ? ex : 0.0f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  load_row(r);
  float sum = 0.0f;
#pragma unroll
  for (int v = 0; v < kMaxExperts; ++v) sum = sum + r[v];
  const float inv = 1.0f / fmaxf(sum, 1e-15f);
  const float p = fminf(fmaxf(ex * inv, 1e-7f), 1.0f);
  __builtin_amdgcn_wave_barrier();
  row[e] = mine ? p : 0.0f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (!valid || !mine) return;
  if (probs) probs[(size_t)t * E + e] = p;   // kept for the backward pass
  load_row(r);
  int rank = 0;
#pragma unroll
  for (int v = 0; v < kMaxExperts; ++v) rank += (r[v] > p) || (r[v] == p && v < e);
  if (rank < k) {
    topk_idx[(size_t)t * k + rank] = e;
    topk_p[(size_t)t * k + rank] = p;
    if (hist) atomicAdd(&hist[(size_t)e * nb + t / kRT], 1);
  }
}

constexpr int kSoftmaxWaves = 4;   // tokens per block
__global__ __launch_bounds__(kSoftmaxWaves * 64) void router_softmax_wave_kernel(
    const float* __restrict__ logits, int N, int E, int k, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_p, int32_t* __restrict__ hist, int nb, float* __restrict__ probs) {
  __shared__ __align__(16) float s_row[kSoftmaxWaves][kMaxExperts];
  __shared__ uint64_t s_tab[32];
  const int w = threadIdx.x / kWave, e = lane_id();
  const int t = blockIdx.x * kSoftmaxWaves + w;
  if (threadIdx.x < 32) s_tab[threadIdx.x] = c_exp2_tab[threadIdx.x];
  float* row = s_row[w];
  const bool valid = t < N;   // wave-uniform
  const float l = (valid && e < E) ? logits[(size_t)t * E + e] : 0.0f;
  row[e] = e < E ? l : -INFINITY;
  __syncthreads();
  softmax_topk_wave(l, valid, t, e, E, k, row, s_tab, topk_idx, topk_p, hist, nb, probs);
}

// Decode router for a single block of tokens (N <= 64, E > 16, no
// normalisation), logits and softmax in one launch.  A block owns one token
// t: wave 0 runs the 64 chains acc = acc + p[c] (lane e = expert e, columns
// ascending, then the bias: the reference's rounding sequence, as in the
// other router kernels) and then the softmax / top-k of the token with
// softmax_topk_wave; waves 1-3 (the other SIMDs) form the products p[e][c] =
// x[t][c] * W_r[c][e] of 15 of each step's 16 column quads (5 each) for step
// s + 2 into a triple-buffered LDS array while the chain wave adds step s's
// (the chain wave forms the 16th quad's products itself: with 6 + 5 + 5 the
// 6-quad wave set the pace).  No histogram: with one router block the
// permute counts the ids itself.
//
// A wave issues about one vector instruction per four cycles, so a chain
// wave that also formed its products took two issue slots per column (9-10
// cycles per column at cfg5, against 3.7 for the adds alone); here it
// issues one add and a quarter of an LDS read per column.  W_r comes from
// its column-quad copy wr4 = [C/4][E][4] (lane e's 16 bytes of quad q at
// (q*E + e)*16, so one load instruction reads 1 KB contiguous), requested
// kDrPS - 1 steps ahead into the producers' registers with buffer loads
// (scalar step offset, loop-invariant lane offsets); x[t] is widened into
// LDS once and read as 16-byte broadcasts.
constexpr int kDrCols = 64;               // columns per step
constexpr int kDrQ = kDrCols / 4;         // column quads per step
constexpr int kDrPLD = kDrCols + 4;       // floats per LDS product row
constexpr int kDrPS = 4;                  // producer register stages
constexpr int kDrPQ = 5;                  // column quads per producer wave and step
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// Word 3 of a raw buffer descriptor: DATA_FORMAT (bits 15-18) = 4, 32-bit
// elements, no swizzle; offsets are bytes, and reads past num_records
// return zeros (none are issued here).
constexpr int kBufWord3 = 0x00020000;

template <typename ActT>
__global__ __launch_bounds__(256) void router_decode_kernel(
    const ActT* __restrict__ x, const float4* __restrict__ wr4, const float* __restrict__ br,
    int N, int C, int E, int k, int32_t* __restrict__ topk_idx, float* __restrict__ topk_p,
    float* __restrict__ probs) {
  __shared__ float4 s_x[kDecodeRouterMaxC / 4];          // x[t] widened to fp32
  __shared__ float4 s_p[3][kMaxExperts * kDrPLD / 4];    // products [e][column]
  __shared__ __align__(16) float s_row[kMaxExperts];
  __shared__ uint64_t s_tab[32];
  const int tid = threadIdx.x;
  const int e = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int t = blockIdx.x;
  const int ee = min(e, E - 1);   // lanes past E repeat the last expert
  const int nst = C / kDrCols;    // steps (C is a multiple of 64)
  // the step barrier: this wave's LDS writes and reads are complete
  auto barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  if (w == 0 && e < 32) s_tab[e] = c_exp2_tab[e];
  // W_r for the producers: wave w owns quads [q0, q0 + kDrPQ) of every step
  // (5 + 5 + 5; the chain wave forms the last quad's products itself, which
  // balances the three), in kDrPS register stages requested kDrPS - 1 steps
  // ahead
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float4*>(wr4), (short)0, C * E * (int)sizeof(float), kBufWord3);
  float4 wv[kDrPS][kDrPQ];
  uint32_t off[kDrPQ];
  const int q0 = w > 0 ? (w - 1) * kDrPQ : 0;
#pragma unroll
  for (int q = 0; q < kDrPQ; ++q) off[q] = (uint32_t)((q0 + q) * E + ee) * 16u;
  auto load = [&](int j, float4 (&v)[kDrPQ]) __attribute__((always_inline)) {
    const int so = min(j, nst - 1) * kDrQ * E * 16;
#pragma unroll
    for (int q = 0; q < kDrPQ; ++q) {
      const u32x4 r = __builtin_amdgcn_raw_buffer_load_b128(wrs, off[q], so, 0);
      v[q] = make_float4(__uint_as_float(r.x), __uint_as_float(r.y), __uint_as_float(r.z),
                         __uint_as_float(r.w));
    }
  };
  {
    // x[t] into LDS as fp32 by all 256 threads, 8 columns per thread and
    // pass: every pass's load first, then the producers' first kDrPS - 1
    // W_r requests (so that both latencies overlap and the wait for x does
    // not wait for W_r), then the widened stores
    constexpr int kXP = kDecodeRouterMaxC / (8 * 256);   // passes at the widest row
    const ActT* xr = x + (size_t)t * C;
    using XPiece = typename std::conditional<sizeof(ActT) == 2, uint4, float4>::type;
    XPiece xv[kXP], xv2[kXP];
#pragma unroll
    for (int pp = 0; pp < kXP; ++pp) {
      const int c = min(8 * tid + 8 * 256 * pp, C - 8);   // in bounds; stored only if < C
      xv[pp] = *reinterpret_cast<const XPiece*>(xr + c);
      if constexpr (sizeof(ActT) == 4) xv2[pp] = *reinterpret_cast<const XPiece*>(xr + c + 4);
    }
    if (w > 0) {
#pragma unroll
      for (int j = 0; j < kDrPS - 1; ++j) load(j, wv[j]);
    }
#pragma unroll
    for (int pp = 0; pp < kXP; ++pp) {
      const int c = 8 * tid + 8 * 256 * pp;
      if (c < C) {
        float4 lo, hi;
        if constexpr (sizeof(ActT) == 2) {
          const uint4 v = xv[pp];
          lo = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                           __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
          hi = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xFFFF0000u),
                           __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xFFFF0000u));
        } else {
          lo = xv[pp];
          hi = xv2[pp];
        }
        s_x[c / 4] = lo;
        s_x[c / 4 + 1] = hi;
      }
    }
  }
  barrier();   // x[t] and the table are in LDS

  if (w > 0) {
    // step j: request W_r of step j + kDrPS - 1 into its stage, then form
    // step j's products from stage j % kDrPS into buffer j % 3 (row e,
    // columns 4 * (q0 + q) ..)
    auto produce = [&](int j, auto st_c) __attribute__((always_inline)) {
      constexpr int st = decltype(st_c)::value;
      constexpr int ahead = (st + kDrPS - 1) % kDrPS;
      load(j + kDrPS - 1, wv[ahead]);
      if (j >= nst) return;
      float4* prow = s_p[j % 3] + (e * kDrPLD) / 4;
      const float4* xs = s_x + (size_t)j * kDrQ;
#pragma unroll
      for (int q = 0; q < kDrPQ; ++q) {
        const float4 xv = xs[q0 + q];
        const float4 wq = wv[st][q];
        prow[q0 + q] = make_float4(xv.x * wq.x, xv.y * wq.y, xv.z * wq.z, xv.w * wq.w);
      }
    };
    produce(0, IntC<0>{});
    produce(1, IntC<1>{});
    barrier();   // steps 0 and 1 are in LDS
    for (int s = 0; s < nst; s += kDrPS) {
      // iteration s: form step s + 2 (buffer (s + 2) % 3, last read during
      // step s - 2's iteration, before the barrier just passed), then meet
      // the chain wave, which adds step s meanwhile
      produce(s + 2, IntC<2>{});
      barrier();
      if (s + 1 >= nst) break;
      produce(s + 3, IntC<3>{});
      barrier();
      if (s + 2 >= nst) break;
      produce(s + 4, IntC<0>{});
      barrier();
      if (s + 3 >= nst) break;
      produce(s + 5, IntC<1>{});
      barrier();
    }
    static_assert(kDrPS == 4, "the unrolled producer loop assumes 4 stages");
    // drain the requests of steps past the end before the wave ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }

  // the chain wave
  // The compiler does not read the waits in inline asm: it would still count
  // the products read a step earlier as pending where they are used and wait
  // there for all reads, the ones just issued included.  Passing the
  // registers through an empty asm after the barrier makes them that asm's
  // results, with nothing left to wait for.
  constexpr int kPQ = kDrQ - 1;   // product quads in LDS; the last is the chain wave's
  auto settle = [&](float4 (&v)[kPQ]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < kPQ; ++q)
      asm volatile("" : "+v"(v[q].x), "+v"(v[q].y), "+v"(v[q].z), "+v"(v[q].w));
  };
  auto read = [&](int j, float4 (&v)[kPQ]) __attribute__((always_inline)) {
    const float4* prow = s_p[min(j, nst - 1) % 3] + (e * kDrPLD) / 4;
#pragma unroll
    for (int q = 0; q < kPQ; ++q) v[q] = prow[q];
  };
  // W_r's last quad of each step, for the chain wave's own products,
  // requested two steps ahead
  const uint32_t off_c = (uint32_t)(kPQ * E + ee) * 16u;
  auto load_c = [&](int j) __attribute__((always_inline)) -> float4 {
    const u32x4 r = __builtin_amdgcn_raw_buffer_load_b128(wrs, off_c, min(j, nst - 1) * kDrQ * E * 16, 0);
    return make_float4(__uint_as_float(r.x), __uint_as_float(r.y), __uint_as_float(r.z),
                       __uint_as_float(r.w));
  };
  float4 wca = load_c(0), wcb = load_c(1);
  float acc = 0.0f;
  float4 pa[kPQ], pb[kPQ];
  barrier();   // steps 0 and 1 are in LDS
  read(0, pa);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  settle(pa);
  // step s: read x's last quad of step s and step s + 1's products (formed
  // before the last barrier), add step s's 15 quads from LDS and then its
  // last quad from products formed here, request W_r's last quad of step
  // s + 2, meet the producers
  auto step = [&](int s, float4 (&pc)[kPQ], float4 (&pn)[kPQ], float4& wc)
      __attribute__((always_inline)) {
    const float4 xq = s_x[(size_t)s * kDrQ + kPQ];
    read(s + 1, pn);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kPQ; ++q) {
      acc = acc + pc[q].x;
      acc = acc + pc[q].y;
      acc = acc + pc[q].z;
      acc = acc + pc[q].w;
    }
    acc = acc + xq.x * wc.x;
    acc = acc + xq.y * wc.y;
    acc = acc + xq.z * wc.z;
    acc = acc + xq.w * wc.w;
    wc = load_c(s + 2);
    __builtin_amdgcn_sched_barrier(0);
    barrier();
    settle(pn);
  };
  for (int s = 0; s < nst; s += 2) {
    step(s, pa, pb, wca);
    if (s + 1 >= nst) break;
    step(s + 1, pb, pa, wcb);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the requests past the last step
  const bool mine = e < E;
  const float l = mine ? acc + br[ee] : 0.0f;
  s_row[e] = mine ? l : -INFINITY;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  softmax_topk_wave(l, t < N, t, e, E, k, s_row, s_tab, topk_idx, topk_p, nullptr, 1, probs);
}


}  // namespace

// logits == nullptr: the fused kernel.  Otherwise (E > 16, few tokens) the
// split path through logits [N][E] (wr1 = W_r as [E][C]).  probs (nullable)
// receives the clamped softmax [N][E] (the reference's cached_router_probs).
// gamma (nullable): route on RMSNorm(x) * gamma instead of x, writing each
// token's 1/rms to rstd [N]; cn: the mean's divisor (C, or the caller's width
// when x's rows are zero-padded to C).
//
// wr4 (W_r as column quads [C/4][E][4]) set: the one-launch decode router,
// for N <= 64, E > 16, no normalisation and C a multiple of 64 up to
// kDecodeRouterMaxC; it writes no histogram (hist is unused).
template <typename ActT>
hipError_t launch_router(const ActT* x, const float* wr_g, const float* wr1, const float* wr4,
                         const float* br, int N, int C, int E, int k, int32_t* topk_idx,
                         float* topk_p, int32_t* hist, float* logits, float* probs,
                         const float* gamma, float eps, int cn, float* rstd, hipStream_t stream) {
  const RowNorm nrm{gamma, eps, cn};
  const int nb = (N + kRT - 1) / kRT;
  if (nb == 0) return hipSuccess;
  if (E > kMaxExperts) {
    // wide: per-expert logits (the split kernels, any E), then the block
    // softmax / top-k over rows of up to kMaxExpertsWide
    if (E > kMaxExpertsWide || !logits || wr4) return hipErrorInvalidValue;
    const int eg = (E + kMaxExperts - 1) / kMaxExperts;
    if (nb * eg >= 256 && router_experts_per_wave(E) == 4) {
      // enough (token block, 64 experts) blocks to fill the chip
      if (gamma)
        hipLaunchKernelGGL((router_logits_wide_kernel<ActT, true>), dim3(nb, eg), dim3(1024), 0,
                           stream, x, wr_g, br, N, C, E, logits, nrm, rstd);
      else
        hipLaunchKernelGGL((router_logits_wide_kernel<ActT, false>), dim3(nb, eg), dim3(1024), 0,
                           stream, x, wr_g, br, N, C, E, logits, nrm, rstd);
    } else if (gamma)
      hipLaunchKernelGGL((router_logits_kernel<ActT, true>),
                         dim3(nb, (E + kSplitExperts - 1) / kSplitExperts),
                         dim3(kSplitExperts * kWave), 0, stream, x, wr1, br, N, C, E, logits, nrm,
                         rstd);
    else
      hipLaunchKernelGGL((router_logits_pc_kernel<ActT>), dim3(nb, E), dim3(256), 0, stream, x,
                         wr1, br, N, C, E, logits, hist, nb);
    if (E <= 256)
      hipLaunchKernelGGL(router_softmax_wide_kernel<256>, dim3(nb), dim3(1024), 0, stream, logits,
                         N, E, k, topk_idx, topk_p, hist, nb, probs);
    else
      hipLaunchKernelGGL(router_softmax_wide_kernel<kMaxExpertsWide>, dim3(nb), dim3(1024), 0,
                         stream, logits, N, E, k, topk_idx, topk_p, hist, nb, probs);
    return hipGetLastError();
  }
  if (wr4) {
    if (N > kRT || E <= 16 || E > kMaxExperts || gamma || C % 64 || C > kDecodeRouterMaxC)
      return hipErrorInvalidValue;
    hipLaunchKernelGGL((router_decode_kernel<ActT>), dim3(N), dim3(256), 0, stream, x,
                       reinterpret_cast<const float4*>(wr4), br, N, C, E, k, topk_idx, topk_p,
                       probs);
    return hipGetLastError();
  }
  if (logits && !gamma) {
    // decode shapes without normalisation: products and chains on separate
    // waves, then the softmax / top-k with one wave per token
    hipLaunchKernelGGL((router_logits_pc_kernel<ActT>), dim3(nb, E), dim3(256), 0, stream, x, wr1,
                       br, N, C, E, logits, hist, nb);
    hipLaunchKernelGGL(router_softmax_wave_kernel, dim3((N + kSoftmaxWaves - 1) / kSoftmaxWaves),
                       dim3(kSoftmaxWaves * kWave), 0, stream, logits, N, E, k, topk_idx, topk_p,
                       hist, nb, probs);
    return hipGetLastError();
  }
  if (logits) {
    const dim3 lg(nb, (E + kSplitExperts - 1) / kSplitExperts), lb(kSplitExperts * kWave);
    if (nrm.gamma)
      hipLaunchKernelGGL((router_logits_kernel<ActT, true>), lg, lb, 0, stream, x, wr1, br, N, C,
                         E, logits, nrm, rstd);
    else
      hipLaunchKernelGGL((router_logits_kernel<ActT, false>), lg, lb, 0, stream, x, wr1, br, N, C,
                         E, logits, nrm, rstd);
    hipLaunchKernelGGL(router_softmax_kernel, dim3(nb), dim3(MGPT_SOFTMAX_THREADS), 0, stream,
                       logits, N, E, k,
                       topk_idx, topk_p, hist, nb, probs);
    return hipGetLastError();
  }
  const int RE = router_experts_per_wave(E);
  const int waves = (E + RE - 1) / RE;
  const dim3 g(nb), b(waves * kWave);
  auto fused = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, g, b, 0, stream, x, wr_g, br, N, C, E, k, topk_idx, topk_p, hist,
                       nb, probs, nrm, rstd);
  };
  const bool norm = nrm.gamma != nullptr;
  switch (RE) {
    case 1:
      norm ? fused(router_topk_uniform_kernel<ActT, 1, true>)
           : fused(router_topk_uniform_kernel<ActT, 1, false>);
      break;
    case 2:
      norm ? fused(router_topk_uniform_kernel<ActT, 2, true>)
           : fused(router_topk_uniform_kernel<ActT, 2, false>);
      break;
    default:
      norm ? fused(router_topk_uniform_kernel<ActT, 4, true>)
           : fused(router_topk_uniform_kernel<ActT, 4, false>);
  }
  return hipGetLastError();
}

template hipError_t launch_router<float>(const float*, const float*, const float*, const float*,
                                         const float*, int, int, int, int, int32_t*, float*,
                                         int32_t*, float*, float*, const float*, float, int,
                                         float*, hipStream_t);
template hipError_t launch_router<bf16_t>(const bf16_t*, const float*, const float*,
                                          const float*, const float*, int, int, int, int,
                                          int32_t*, float*, int32_t*, float*, float*,
                                          const float*, float, int, float*, hipStream_t);

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
