// gemm_dma.hip -- bf16 grouped expert GEMMs, direct-to-LDS pipeline.
//
// Same contract as gemm.hip's grouped_gemm_kernel for the bf16 x bf16 case
// (A = expert-contiguous activations [rows][K], B = packed weights
// [E][Npad][K], K contiguous; gate/up epilogue with SwiGLU or down epilogue
// with bias), built for the large prefill-shaped segments that dominate the
// MoE layer's time.
//
// CDNA4 design (choices measured on MI355X):
//  * 256 x 256 x 64 block tile, 8 waves (2 per SIMD) each owning 128 x 64:
//    4 x 2 tiles of v_mfma_f32_32x32x16_bf16, 128 accumulators in AGPRs.
//    Issue is in order within a wave, so with one wave per SIMD every LDS or
//    barrier wait idles the matrix core; with two, one wave's MFMAs cover
//    the other's waits.
//  * Operands move HBM -> LDS with global_load_lds_dwordx4 (one 1 KB row
//    block per wave instruction; no staging registers, no ds_write) into a
//    2-stage ring: the DMA of slab kt+1 is issued right after the barrier
//    that opens slab kt.  The barrier is a bare s_barrier after an explicit
//    vmcnt wait for the wave's own DMA; __syncthreads() would also drain the
//    prefetch in flight.
//  * LDS rows are 128 B (64 bf16); K-chunk c of row r sits at slot
//    c ^ ((r >> 1) & 7): gfx950's LDS has 64 banks, so the 16 lanes served
//    together (16 rows of one logical chunk) hit 16 distinct bank groups.
//  * Epilogue straight from the accumulators: SwiGLU with the hardware
//    exp/reciprocal (well inside the bf16 tolerance), bf16 stores.
#include "common.hpp"

namespace mgpt {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;                  // 8
constexpr int kBM = 256, kBN = 256, kBK = 64, kStages = 2;
constexpr int kWTM = 128, kWTN = 64;                      // wave tile
constexpr int kTM = kWTM / 32, kTN = kWTN / 32;           // 4 x 2 MFMA tiles
constexpr int kRowBytes = kBK * 2;                        // 128 B per LDS row
constexpr int kStageBytes = (kBM + kBN) * kRowBytes;      // 64 KB
constexpr int kDmaPerWave = kStageBytes / 1024 / kWaves;  // 8
constexpr int kRowsPerDma = 1024 / kRowBytes;             // 8

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void slab_barrier() {
  // This wave's DMA has landed (vmcnt(0)) and its LDS reads of the previous
  // slab are complete (lgkmcnt(0)); then meet the other waves.  The empty
  // asm statements keep the compiler from moving LDS reads across it.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float silu_mul_fast(float g, float u) {
  return g * u * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

__device__ __forceinline__ bf16_t bf16_rne(float f) {
  __bf16 b = (__bf16)f;   // round to nearest even
  bf16_t r;
  __builtin_memcpy(&r, &b, 2);
  return r;
}

template <int EPI>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(
    const bf16_t* __restrict__ A, const bf16_t* __restrict__ B, const float* __restrict__ bias0,
    const float* __restrict__ bias1, const int32_t* __restrict__ counts, int E, int K, int Npad,
    int n_store, int bias_ld, bf16_t* __restrict__ out, int ldo) {
  __shared__ __attribute__((aligned(1024))) char smem[kStages * kStageBytes];

  // XCD-aware tile order (see gemm.hip).
  const int nbx = gridDim.x;
  const int total = nbx * gridDim.y;
  int bid = blockIdx.y * nbx + blockIdx.x;
  const int per = total / kNumXcd;
  if (bid < per * kNumXcd) bid = (bid % kNumXcd) * per + bid / kNumXcd;
  TileInfo ti;
  if (!find_tile<kBM>(counts, E, bid / nbx, &ti)) return;
  const int e = ti.expert;
  const int n0 = (bid % nbx) * kBN;

  const int tid = threadIdx.x;
  const int w = tid / kWave, lane = lane_id();
  const int wm = w >> 2, wn = w & 3;                      // 2 x 4 waves
  const int lrow = lane & 31, lhalf = lane >> 5;
  const size_t row_bytes_g = (size_t)K * 2;

  // DMA: row block q = w*8 + i covers LDS rows 8q .. 8q+7 (rows 0..255 = A
  // tile, 256..511 = B tile): waves 0-3 fill A, waves 4-7 fill B.  Lane l
  // fills slot l%8 of row r = 8q + l/8 with logical chunk
  // (l%8) ^ ((r >> 1) & 7) = (l%8) ^ ((4*(q&1) + l/16) & 7).
  const char* gbase;
  {
    const char* Ag = reinterpret_cast<const char*>(A + (size_t)ti.row0 * K);
    const char* Bg = reinterpret_cast<const char*>(B + ((size_t)e * Npad + n0) * K);
    gbase = (w < 4 ? Ag : Bg) + (size_t)((w & 3) * kDmaPerWave * kRowsPerDma) * row_bytes_g;
  }
  const uint32_t lane_row = (uint32_t)(lane >> 3) * (uint32_t)row_bytes_g;
  const uint32_t lane_off0 = lane_row + ((uint32_t)((lane & 7) ^ (lane >> 4)) << 4);
  const uint32_t lane_off1 = lane_row + ((uint32_t)((lane & 7) ^ (4 | (lane >> 4))) << 4);
  auto dma = [&](int kt) __attribute__((always_inline)) {
    char* dst = smem + (kt & 1) * kStageBytes + w * kDmaPerWave * 1024;
    const char* g = gbase + (size_t)kt * kRowBytes;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i)
      __builtin_amdgcn_global_load_lds(
          g + (size_t)i * kRowsPerDma * row_bytes_g + ((i & 1) ? lane_off1 : lane_off0),
          (lds_void*)(dst + i * 1024), 16, 0, 0);
  };

  f32x16 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // Fragment rows start at multiples of 32: (row >> 1) & 7 = (lrow >> 1) & 7.
  int a_off[kTM], b_off[kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i) a_off[i] = (wm * kWTM + i * 32 + lrow) * kRowBytes;
#pragma unroll
  for (int j = 0; j < kTN; ++j) b_off[j] = (kBM + wn * kWTN + j * 32 + lrow) * kRowBytes;
  const int swz = (lrow >> 1) & 7;

  const int KT = K / kBK;
  dma(0);
  for (int kt = 0; kt < KT; ++kt) {
    slab_barrier();
    if (kt + 1 < KT) dma(kt + 1);
    const char* st = smem + (kt & 1) * kStageBytes;
    bf16x8 af[2][kTM], bfr[2][kTN];
    auto frags = [&](int ks, bf16x8 (&a)[kTM], bf16x8 (&b)[kTN]) __attribute__((always_inline)) {
      const int cofs = (((ks * 2 + lhalf) ^ swz) << 4);
#pragma unroll
      for (int i = 0; i < kTM; ++i) a[i] = *reinterpret_cast<const bf16x8*>(st + a_off[i] + cofs);
#pragma unroll
      for (int j = 0; j < kTN; ++j) b[j] = *reinterpret_cast<const bf16x8*>(st + b_off[j] + cofs);
    };
    frags(0, af[0], bfr[0]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks + 1 < 4) frags(ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][i], bfr[ks & 1][j],
                                                              acc[i][j], 0, 0, 0);
    }
  }

  // ---- epilogue straight from the accumulators.  Register v of a 32x32
  // tile holds row 8*(v/4) + 4*(lane/32) + v%4 and column lane%32.
  const int row_base = ti.row0 + wm * kWTM;
  if constexpr (EPI == kEpiGateUp) {
    // the wave's 64 packed columns are one [32 gate | 32 up] group
    const int hcol = (n0 + wn * kWTN) / 2 + lrow;
    const float bg = bias0[(size_t)e * bias_ld + hcol];
    const float bu = bias1[(size_t)e * bias_ld + hcol];
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = row_base + i * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4);
        if (row < ti.row_end)
          out[(size_t)row * ldo + hcol] =
              bf16_rne(silu_mul_fast(acc[i][0][v] + bg, acc[i][1][v] + bu));
      }
  } else {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int col = n0 + wn * kWTN + j * 32 + lrow;
      if (col >= n_store) continue;
      const float b = bias0[(size_t)e * bias_ld + col];
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = row_base + i * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4);
          if (row < ti.row_end) out[(size_t)row * ldo + col] = bf16_rne(acc[i][j][v] + b);
        }
    }
  }
}

}  // namespace

template <int EPI>
hipError_t launch_gemm_dma(const bf16_t* A, const bf16_t* B, const float* bias0,
                           const float* bias1, const int32_t* counts, int E, int K, int Npad,
                           int n_store, int bias_ld, bf16_t* out, int ldo, int max_mtiles,
                           hipStream_t stream) {
  if (max_mtiles <= 0) return hipSuccess;
  if (K % kBK != 0 || Npad % kBN != 0) return hipErrorInvalidValue;
  dim3 grid(Npad / kBN, max_mtiles);
  hipLaunchKernelGGL((gemm_dma_kernel<EPI>), grid, dim3(kThreads), 0, stream, A, B, bias0, bias1,
                     counts, E, K, Npad, n_store, bias_ld, out, ldo);
  return hipGetLastError();
}

template hipError_t launch_gemm_dma<kEpiGateUp>(const bf16_t*, const bf16_t*, const float*,
                                                const float*, const int32_t*, int, int, int, int,
                                                int, bf16_t*, int, int, hipStream_t);
template hipError_t launch_gemm_dma<kEpiDown>(const bf16_t*, const bf16_t*, const float*,
                                              const float*, const int32_t*, int, int, int, int,
                                              int, bf16_t*, int, int, hipStream_t);

}  // namespace mgpt
