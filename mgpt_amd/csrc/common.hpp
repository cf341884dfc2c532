// common.hpp -- shared device helpers for the gfx950 MoE kernels.
//
// All sources are compiled with -ffp-contract=off, so a * b + c is two
// correctly rounded operations unless fma() is written explicitly; the
// router's bit-exactness relies on that.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mgpt {

typedef uint16_t bf16_t;   // bfloat16 bit pattern
typedef uint8_t fp8_t;     // OCP E4M3FN bit pattern

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kNumXcd = 8;        // MI355X: 8 accelerator complex dies, one L2 each
// Experts the kernels that map one expert to one lane of a wave take (the
// fused prefill and decode routers, the weight-streaming GEMM, the weight
// gradients' row chunks); up to kMaxExpertsWide the layer runs the router's
// logits in groups of 64 experts and a wide softmax, the 256 x 256 GEMMs
// once per group of 64, the generic grouped GEMMs, a permute that scans the
// experts in wave-sized chunks, and the backward's wide token and router
// gradients.
constexpr int kMaxExperts = 64;
constexpr int kMaxExpertsWide = 512;
constexpr int kMaxTopK = 8;
// Tokens per router / permute block: block b owns tokens [b*64, (b+1)*64)
// and so the flat assignment ids [b*64*k, (b+1)*64*k).
constexpr int kRouterTokens = 64;
__host__ __device__ inline int router_tokens_per_block(int /*E*/) { return kRouterTokens; }

// Widest row the one-launch decode router takes (x[t] is widened into LDS as
// fp32, 32 KB at this width).
constexpr int kDecodeRouterMaxC = 8192;

// Router experts per wave (the router block has ceil(E / RE) <= 16 waves);
// router weights are packed [ceil(E/RE)][C][RE], zero-padded.  Two experts
// per wave share the activation loads and conversions of their chains:
// measured on MI355X at cfg3 (E = 16), 8 waves x 2 experts take 33.7 us,
// 16 x 1 take 37 us and 4 x 4 take 46 us.
__host__ __device__ inline int router_experts_per_wave(int E) {
  return E <= 8 ? 1 : (E <= 32 ? 2 : 4);
}

// Grouped-GEMM epilogues (gemm.hip, gemm_dma.hip).  kEpiGateUp: SwiGLU of
// the interleaved gate/up columns (optionally also saving the pre-activations
// for the backward pass); kEpiDown: + bias (none when the bias pointer is
// null); kEpiSwigluBwd: the backward of SwiGLU applied to the product
// d(act) = dY . W_down^T, reading the saved pre-activations and writing
// d(gate), d(up) in the same interleaved layout.
enum Epilogue { kEpiGateUp = 0, kEpiDown = 1, kEpiSwigluBwd = 2 };

// Column of hidden unit h (and, +32, of its up partner) in the gate/up
// interleaved layout [32 gate | 32 up] per 32 hidden units.
__host__ __device__ __forceinline__ int packed_gate_col(int h) { return (h >> 5) * 64 + (h & 31); }

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

// Round-to-nearest-even float -> bfloat16 (NaN stays NaN).
__host__ __device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  uint32_t u;
#ifdef __HIP_DEVICE_COMPILE__
  u = __float_as_uint(f);
#else
  __builtin_memcpy(&u, &f, 4);
#endif
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (bf16_t)((u | 0x00400000u) >> 16);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

// Two floats -> two bf16 in one word, the first in the low half
// (v_cvt_pk_bf16_f32: nearest even, fp32 denormals kept; f32_to_bf16's
// rounding in one instruction).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

template <typename T> struct ActTraits;
template <> struct ActTraits<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
};
template <> struct ActTraits<bf16_t> {
  static __device__ __forceinline__ float load(const bf16_t* p) { return bf16_to_f32(*p); }
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ void store_act(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_act(bf16_t* p, float v) { *p = f32_to_bf16(v); }

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int l = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    int t = __shfl_up(v, d, kWave);
    if (l >= d) v += t;
  }
  return v;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

// Which expert segment an m-tile belongs to.  Grouped GEMMs launch a grid
// over an upper bound of m-tiles; each block derives its expert, the
// segment's first row and its end row from the per-expert counts (wave 0
// scans them 64 experts at a time, any E), so no host round-trip is needed.  Returns false for blocks past the last
// tile.  Must be called by every thread of the block (uses shared memory);
// it may be called repeatedly (persistent kernels).
struct TileInfo {
  int expert;
  int row0;     // first row of this m-tile (global slot index)
  int row_end;  // one past the last row of the expert's segment
};

template <int BM>
__device__ __forceinline__ bool find_tile(const int32_t* __restrict__ counts, int E,
                                          int mtile, TileInfo* out) {
  __shared__ int s_info[4];
  __syncthreads();   // every wave has read the previous call's result
  if (threadIdx.x < kWave) {
    const int l = lane_id();
    int rows_carry = 0, tiles_carry = 0, found = -1, row0 = 0, rend = 0;
    for (int e0 = 0; e0 < E && found < 0; e0 += kWave) {
      const int e = e0 + l;
      const int cnt = (e < E) ? counts[e] : 0;
      const int tiles = (cnt + BM - 1) / BM;
      const int rows_incl = wave_incl_scan(cnt) + rows_carry;
      const int tiles_incl = wave_incl_scan(tiles) + tiles_carry;
      const int tiles_excl = tiles_incl - tiles;
      const bool mine = (e < E) && (mtile >= tiles_excl) && (mtile < tiles_incl);
      const unsigned long long m = __ballot(mine);
      const int owner = m ? (__ffsll((long long)m) - 1) : 0;
      const int r0 = __shfl((rows_incl - cnt) + (mtile - tiles_excl) * BM, owner, kWave);
      const int re = __shfl(rows_incl, owner, kWave);
      if (m) {
        found = e0 + owner;
        row0 = r0;
        rend = re;
      }
      rows_carry = __shfl(rows_incl, kWave - 1, kWave);
      tiles_carry = __shfl(tiles_incl, kWave - 1, kWave);
    }
    if (l == 0) {
      s_info[0] = found;
      s_info[1] = row0;
      s_info[2] = rend;
    }
  }
  __syncthreads();
  out->expert = s_info[0];
  out->row0 = s_info[1];
  out->row_end = s_info[2];
  return out->expert >= 0;
}

// A batch of gradient additions dst_j[r][c] += src[off_j + r * lds_j + c]
// (launch_add_jobs; passed by value as a kernel argument).
struct AddJobs {
  static constexpr int kMax = 24;
  float* dst[kMax];
  size_t off[kMax];
  int rows[kMax], cols[kMax], lds[kMax];
  int n;
};

// Per-expert gradient slices (expert e's slice of piece p: base[p] +
// e * len[p], len[p] floats) that launch_zero_idle_experts clears for the
// experts without rows; passed by value as a kernel argument.
struct IdleSlices {
  static constexpr int kMax = 6;
  float* base[kMax];
  size_t len[kMax];
  int n;
};

}  // namespace mgpt
