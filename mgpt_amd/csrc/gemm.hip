// gemm.hip -- grouped expert GEMMs on CDNA4 matrix cores.
//
// Reference: per expert e with count_e > 0, SwiGLU::forward_into
// (layers/SwiGLU.cpp:23-50): g = X_e W_g + b_g, u = X_e W_u + b_u,
// h = silu(g) * u (utils/Tensor.cpp:1986-2004), y_e = h W_d + b_d, run by a
// host loop over experts (layers/MoELayer.cpp:94-118).  Here each product is
// one launch over all experts: the rows of X are expert-contiguous segments
// (dispatch.hip), the grid covers an upper bound of m-tiles, and each block
// finds its expert from the device-side counts (common.hpp find_tile).
//
// Operands: A = activations [rows][K] (bf16 or fp32, K contiguous);
// B = packed weights [E][Npad][K] (K contiguous, so both MFMA operands are
// read as 16-byte K-runs); C = A . B^T.  Tiles: block BM x BN x BK with 4
// waves in a WM x WN grid; each wave owns (BM/WM) x (BN/WN) made of 32x32
// MFMA tiles: v_mfma_f32_32x32x16_bf16 for bf16 (and fp8 weights, which are
// widened to bf16 exactly while being staged into LDS), v_mfma_f32_32x32x2_f32
// for fp32.  Global -> register -> LDS double buffering: the next K-slab is
// fetched while the current one feeds the MFMAs; one barrier per slab.
//
// Epilogues: GATEUP (B rows interleaved in 64-row groups [32 gate | 32 up]
// for the same 32 hidden units, so a wave's two adjacent 32x32 tiles hold
// g and u of the same (row, h) in the same lane) computes
// h = silu(g*s_g + b_g) * (u*s_u + b_u) and stores bf16/fp32 h, and, when
// `aux` is given, also the pre-activations g, u in the interleaved layout
// (aux[row][packed column], the caches of layers/SwiGLU.cpp:30-31 that the
// backward pass reads);
// DOWN stores o = acc*s + b_d in the activation dtype (no bias if bias0 is
// null);
// SWIGLU_BWD treats the product as d(act)[row][h] and applies the CPU
// swiglu_backward of utils/Tensor.cpp:2006-2030 with the saved g, u read
// from aux: sig = 1/(1+exp(-g)), d_up = d*(g*sig),
// d_gate = (d*u)*(sig*(1+g*(1-sig))), written to out in the interleaved
// layout (out may equal aux: each element is read before it is written by
// the same thread).
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace mgpt {

namespace {

template <typename AT> struct KSlab;
template <> struct KSlab<bf16_t> { static constexpr int BK = 64; };
template <> struct KSlab<float> { static constexpr int BK = 32; };

struct alignas(16) U4 {
  uint32_t x, y, z, w;
};
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// e4m3 byte pair -> two bf16 in one dword (exact: every e4m3 value is a bf16 value).
template <bool HI>
__device__ __forceinline__ uint32_t e4m3x2_to_bf16x2(uint32_t packed_bytes) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)packed_bytes, 1.0f, HI);
  uint32_t r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}

template <int BM, int BN, int WM, int WN, typename AT, typename WT, int EPI, typename OutT>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(
    const AT* __restrict__ A, const WT* __restrict__ B, const float* __restrict__ wscale,
    const float* __restrict__ bias0, const float* __restrict__ bias1,
    const int32_t* __restrict__ counts, int E, int K, int Npad, int n_store, int bias_ld,
    OutT* out, int ldo, OutT* aux, int aux_ld, float* __restrict__ partials) {
  constexpr int BK = KSlab<AT>::BK;
  constexpr int PAD = 16 / (int)sizeof(AT);
  constexpr int LDK = BK + PAD;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(WM * WN == 4, "4 waves");
  static_assert(TM >= 1 && TN >= 1, "wave tile >= 32x32");
  static_assert(EPI != kEpiGateUp || (TN % 2 == 0), "gate/up pairs");
  constexpr bool kF32 = sizeof(AT) == 4;
  constexpr bool kFp8 = sizeof(WT) == 1;
  // 16-byte chunks per K-slab row, and per-thread chunk counts.
  constexpr int A_CPR = BK * (int)sizeof(AT) / 16;             // 8
  constexpr int B_CPR = BK * (int)sizeof(WT) / 16;             // 8 (bf16/f32) or 4 (fp8)
  constexpr int A_CH = BM * A_CPR / 256;
  constexpr int B_CH = BN * B_CPR / 256;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");

  __shared__ __attribute__((aligned(16))) AT sA[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) AT sB[2][BN][LDK];

  // XCD-aware order: the hardware deals consecutive workgroups round-robin
  // to the 8 XCDs (each with its own L2); remap so each XCD receives a
  // contiguous run of tiles, n fastest, so concurrently resident blocks on
  // one XCD share their A (activation) tile and neighbouring B tiles.
  const int nbx = gridDim.x;
  const int total = nbx * gridDim.y;
  int bid = blockIdx.y * nbx + blockIdx.x;
  const int per = total / kNumXcd;
  if (bid < per * kNumXcd) bid = (bid % kNumXcd) * per + bid / kNumXcd;
  const int mtile = bid / nbx;
  TileInfo ti;
  if (!find_tile<BM>(counts, E, mtile, &ti)) return;
  const int e = ti.expert;
  const int n0 = (bid % nbx) * BN;
  const int tid = threadIdx.x;
  const int w = tid / kWave, lane = lane_id();
  const int wm = w / WN, wn = w % WN;

  const AT* Ablk = A + (size_t)ti.row0 * K;
  const WT* Bblk = B + ((size_t)e * Npad + n0) * K;

  U4 ra[A_CH], rb[B_CH];
  auto gload = [&](int kt) __attribute__((always_inline)) {
    const char* abase = reinterpret_cast<const char*>(Ablk + (size_t)kt * BK);
    const char* bbase = reinterpret_cast<const char*>(Bblk + (size_t)kt * BK);
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int q = tid + 256 * i;
      const int r = q / A_CPR, c = q % A_CPR;
      const u32x4 v = *reinterpret_cast<const u32x4*>(abase + (size_t)r * K * sizeof(AT) + c * 16);
      ra[i].x = v.x; ra[i].y = v.y; ra[i].z = v.z; ra[i].w = v.w;
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int q = tid + 256 * i;
      const int r = q / B_CPR, c = q % B_CPR;
      const u32x4 v = *reinterpret_cast<const u32x4*>(bbase + (size_t)r * K * sizeof(WT) + c * 16);
      rb[i].x = v.x; rb[i].y = v.y; rb[i].z = v.z; rb[i].w = v.w;
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int q = tid + 256 * i;
      const int r = q / A_CPR, c = q % A_CPR;
      *reinterpret_cast<U4*>(reinterpret_cast<char*>(&sA[buf][r][0]) + c * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int q = tid + 256 * i;
      const int r = q / B_CPR, c = q % B_CPR;
      if constexpr (kFp8) {
        // 16 e4m3 bytes -> 16 bf16 (32 bytes) at element offset c*16.
        U4 lo, hi;
        lo.x = e4m3x2_to_bf16x2<false>(rb[i].x); lo.y = e4m3x2_to_bf16x2<true>(rb[i].x);
        lo.z = e4m3x2_to_bf16x2<false>(rb[i].y); lo.w = e4m3x2_to_bf16x2<true>(rb[i].y);
        hi.x = e4m3x2_to_bf16x2<false>(rb[i].z); hi.y = e4m3x2_to_bf16x2<true>(rb[i].z);
        hi.z = e4m3x2_to_bf16x2<false>(rb[i].w); hi.w = e4m3x2_to_bf16x2<true>(rb[i].w);
        U4* dst = reinterpret_cast<U4*>(&sB[buf][r][c * 16]);
        dst[0] = lo;
        dst[1] = hi;
      } else {
        *reinterpret_cast<U4*>(reinterpret_cast<char*>(&sB[buf][r][0]) + c * 16) = rb[i];
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // Split K (DOWN only, gridDim.z parts): part z takes slabs
  // [z*KT/S, (z+1)*KT/S) and stores its fp32 partial tile for
  // split_reduce_kernel instead of running the epilogue.
  const int S = gridDim.z, z = blockIdx.z;
  const int KT = K / BK / S;
  Ablk += (size_t)z * KT * BK;
  Bblk += (size_t)z * KT * BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    if constexpr (!kF32) {
      // Fragments of k-step ks+1 are read from LDS while the MFMAs of
      // k-step ks run.
      constexpr int KS = BK / 16;
      bf16x8 af[2][TM], bfr[2][TN];
      auto lds_frags = [&](int ks, bf16x8 (&a)[TM], bf16x8 (&b)[TN]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          a[i] = *reinterpret_cast<const bf16x8*>(
              &sA[cur][wm * WTM + i * 32 + lrow][ks * 16 + lhalf * 8]);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          b[j] = *reinterpret_cast<const bf16x8*>(
              &sB[cur][wn * WTN + j * 32 + lrow][ks * 16 + lhalf * 8]);
      };
      lds_frags(0, af[0], bfr[0]);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) lds_frags(ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][i], bfr[ks & 1][j],
                                                                acc[i][j], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < BK / 2; ++ks) {
        float af[TM], bfr[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = sA[cur][wm * WTM + i * 32 + lrow][ks * 2 + lhalf];
#pragma unroll
        for (int j = 0; j < TN; ++j) bfr[j] = sB[cur][wn * WTN + j * 32 + lrow][ks * 2 + lhalf];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue.  Accumulator register v of a 32x32 tile holds row
  // 8*(v/4) + 4*(lane/32) + v%4 and column lane%32.
  const int row_base = ti.row0 + wm * WTM;
  if constexpr (EPI == kEpiDown) {
    if (S > 1) {
      // the partial tile [BM][BN] in slot (z, m-tile, n-tile)
      float* P = partials + ((size_t)(z * gridDim.y + mtile) * gridDim.x + bid % nbx) * (BM * BN);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            P[(wm * WTM + i * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4)) * BN + wn * WTN + j * 32 +
              lrow] = acc[i][j][v];
      return;
    }
  }
  if constexpr (EPI == kEpiGateUp) {
#pragma unroll
    for (int q = 0; q < TN / 2; ++q) {
      const int prow = n0 + wn * WTN + q * 64 + lrow;   // packed row of the gate column
      const int hcol = (n0 + wn * WTN) / 2 + q * 32 + lrow;
      const float sg = kFp8 ? wscale[(size_t)e * Npad + prow] : 1.0f;
      const float su = kFp8 ? wscale[(size_t)e * Npad + prow + 32] : 1.0f;
      const float bg = bias0[(size_t)e * bias_ld + hcol];
      const float bu = bias1[(size_t)e * bias_ld + hcol];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = row_base + i * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4);
          if (row < ti.row_end) {
            float g = acc[i][2 * q][v];
            float u = acc[i][2 * q + 1][v];
            if (kFp8) { g = g * sg; u = u * su; }
            g = g + bg;
            u = u + bu;
            const float ex = kF32 ? expf(-g) : __expf(-g);
            const float hv = (g / (1.0f + ex)) * u;
            store_act(out + (size_t)row * ldo + hcol, hv);
            if (aux) {
              store_act(aux + (size_t)row * aux_ld + prow, g);
              store_act(aux + (size_t)row * aux_ld + prow + 32, u);
            }
          }
        }
      }
    }
  } else if constexpr (EPI == kEpiSwigluBwd) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int h = n0 + wn * WTN + j * 32 + lrow;
      if (h >= n_store) continue;
      const int pc = packed_gate_col(h);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = row_base + i * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4);
          if (row < ti.row_end) {
            const float d = acc[i][j][v];
            const float g = to_f32(aux[(size_t)row * aux_ld + pc]);
            const float u = to_f32(aux[(size_t)row * aux_ld + pc + 32]);
            const float ex = kF32 ? expf(-g) : __expf(-g);
            const float sig = 1.0f / (1.0f + ex);
            const float d_up = d * (g * sig);
            const float d_gate = (d * u) * (sig * (1.0f + g * (1.0f - sig)));
            store_act(out + (size_t)row * ldo + pc, d_gate);
            store_act(out + (size_t)row * ldo + pc + 32, d_up);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WTN + j * 32 + lrow;
      if (col >= n_store) continue;
      const float s = kFp8 ? wscale[(size_t)e * Npad + col] : 1.0f;
      const float b = bias0 ? bias0[(size_t)e * bias_ld + col] : 0.0f;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = row_base + i * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4);
          if (row < ti.row_end) {
            float o = acc[i][j][v];
            if (kFp8) o = o * s;
            store_act(out + (size_t)row * ldo + col, o + b);
          }
        }
      }
    }
  }
}

// The epilogue of a split DOWN product: block (n-tile x, m-tile y, slice z)
// takes every 4 consecutive outputs of its tile's slice z of kSlices, loads
// the S partial float4s at once, sums them in part order (deterministic),
// adds the bias and stores.
constexpr int kReduceSlices = 8;
#ifndef MGPT_MAX_KSPLIT
#define MGPT_MAX_KSPLIT 8   // at most 8 parts (the reduce keeps 8 float4s in flight)
#endif
template <int BM, int BN, typename OutT>
__global__ __launch_bounds__(256) void split_reduce_kernel(
    const float* __restrict__ partials, int S, const float* __restrict__ bias0,
    const int32_t* __restrict__ counts, int E, int n_store, int bias_ld, OutT* out, int ldo) {
  static_assert(BM * BN % (4 * 256 * kReduceSlices) == 0, "slices of whole float4 rows");
  TileInfo ti;
  if (!find_tile<BM>(counts, E, blockIdx.y, &ti)) return;
  const int n0 = blockIdx.x * BN;
  const size_t tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
  const size_t part_stride = (size_t)gridDim.y * gridDim.x * (BM * BN);
  constexpr int kPer = BM * BN / 4 / kReduceSlices;   // float4s per slice
  for (int q4 = blockIdx.z * kPer + threadIdx.x; q4 < (blockIdx.z + 1) * kPer; q4 += 256) {
    const int q = 4 * q4, r = q / BN, c = q % BN;
    const int row = ti.row0 + r, col = n0 + c;
    if (row >= ti.row_end || col >= n_store) continue;   // n_store is a multiple of 4
    const float4* P = reinterpret_cast<const float4*>(partials + tile * (BM * BN) + q);
    float4 v[8];
#pragma unroll
    for (int zz = 0; zz < 8; ++zz)
      if (zz < S) v[zz] = P[zz * (part_stride / 4)];
    float4 a = v[0];
#pragma unroll
    for (int zz = 1; zz < 8; ++zz)
      if (zz < S) {
        a.x += v[zz].x;
        a.y += v[zz].y;
        a.z += v[zz].z;
        a.w += v[zz].w;
      }
    const float* bp = bias0 ? bias0 + (size_t)ti.expert * bias_ld + col : nullptr;
    OutT* o = out + (size_t)row * ldo + col;
    store_act(o, a.x + (bp ? bp[0] : 0.0f));
    store_act(o + 1, a.y + (bp ? bp[1] : 0.0f));
    store_act(o + 2, a.z + (bp ? bp[2] : 0.0f));
    store_act(o + 3, a.w + (bp ? bp[3] : 0.0f));
  }
}

}  // namespace

// Host launcher.  max_mtiles must bound sum_e ceil(count_e / BM) (the
// caller uses ceil(A / BM) + E); surplus blocks exit after find_tile.
// aux / aux_ld: the pre-activation save of GATEUP (null: none) or the saved
// pre-activations SWIGLU_BWD reads (required).
// DOWN and SWIGLU_BWD cover only the n-tiles that hold stored columns
// (n_store; Npad is the weights' row stride).  partials (DOWN only, or
// null): with split_slots > 0 fp32 partial tiles for up to split_slots
// (part, m-tile, n-tile) items, the K dimension of a product with fewer
// tiles than that is split into S = 2, 4 or 8 parts (S * tiles <=
// split_slots), and split_reduce_kernel runs the epilogue.
template <int BM, int BN, int WM, int WN, typename AT, typename WT, int EPI, typename OutT>
hipError_t launch_grouped_gemm(const AT* A, const WT* B, const float* wscale, const float* bias0,
                               const float* bias1, const int32_t* counts, int E, int K, int Npad,
                               int n_store, int bias_ld, OutT* out, int ldo, int max_mtiles,
                               OutT* aux, int aux_ld, hipStream_t stream, float* partials,
                               int split_slots) {
  if (max_mtiles <= 0) return hipSuccess;
  if (EPI == kEpiSwigluBwd && aux == nullptr) return hipErrorInvalidValue;
  constexpr int BK = KSlab<AT>::BK;
  const int ntiles = EPI == kEpiGateUp ? Npad / BN : std::min(Npad / BN, (n_store + BN - 1) / BN);
  int S = 1;
  if (EPI == kEpiDown && partials && split_slots > 0 && n_store % 4 == 0 &&
      !std::is_same<WT, fp8_t>::value) {
    const int KT = K / BK;
    const long tiles = (long)ntiles * max_mtiles;
    while (S < MGPT_MAX_KSPLIT && (long)(2 * S) * tiles <= split_slots && KT % (2 * S) == 0)
      S *= 2;
  }
  dim3 grid(ntiles, max_mtiles, S);
  hipLaunchKernelGGL((grouped_gemm_kernel<BM, BN, WM, WN, AT, WT, EPI, OutT>), grid, dim3(256), 0,
                     stream, A, B, wscale, bias0, bias1, counts, E, K, Npad, n_store, bias_ld, out,
                     ldo, aux, aux_ld, partials);
  if constexpr (EPI == kEpiDown) {
    if (S > 1)
      hipLaunchKernelGGL((split_reduce_kernel<BM, BN, OutT>), dim3(ntiles, max_mtiles, kReduceSlices),
                         dim3(256), 0, stream, partials, S, bias0, counts, E, n_store, bias_ld, out,
                         ldo);
  }
  return hipGetLastError();
}

#define MGPT_INST_GEMM(BM, BN, WM, WN, AT, WT, EPI, OT)                                     \
  template hipError_t launch_grouped_gemm<BM, BN, WM, WN, AT, WT, EPI, OT>(                 \
      const AT*, const WT*, const float*, const float*, const float*, const int32_t*, int, int, \
      int, int, int, OT*, int, int, OT*, int, hipStream_t, float*, int);

// Large-M tiles (prefill-shaped segments).
MGPT_INST_GEMM(128, 128, 2, 2, bf16_t, bf16_t, kEpiGateUp, bf16_t)
MGPT_INST_GEMM(128, 128, 2, 2, bf16_t, bf16_t, kEpiDown, bf16_t)
MGPT_INST_GEMM(128, 128, 2, 2, bf16_t, fp8_t, kEpiGateUp, bf16_t)
MGPT_INST_GEMM(128, 128, 2, 2, bf16_t, fp8_t, kEpiDown, bf16_t)
// Small-M tiles (decode-shaped segments of a few rows per expert).
MGPT_INST_GEMM(32, 256, 1, 4, bf16_t, bf16_t, kEpiGateUp, bf16_t)
MGPT_INST_GEMM(32, 256, 1, 4, bf16_t, bf16_t, kEpiDown, bf16_t)
MGPT_INST_GEMM(32, 256, 1, 4, bf16_t, fp8_t, kEpiGateUp, bf16_t)
MGPT_INST_GEMM(32, 256, 1, 4, bf16_t, fp8_t, kEpiDown, bf16_t)
// fp32 path.
MGPT_INST_GEMM(64, 128, 2, 2, float, float, kEpiGateUp, float)
MGPT_INST_GEMM(64, 128, 2, 2, float, float, kEpiDown, float)
// Backward data-gradient products (d(act) with the SwiGLU backward; dX).
MGPT_INST_GEMM(128, 128, 2, 2, bf16_t, bf16_t, kEpiSwigluBwd, bf16_t)
MGPT_INST_GEMM(32, 256, 1, 4, bf16_t, bf16_t, kEpiSwigluBwd, bf16_t)
MGPT_INST_GEMM(64, 128, 2, 2, float, float, kEpiSwigluBwd, float)

}  // namespace mgpt
