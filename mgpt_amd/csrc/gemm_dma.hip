// gemm_dma.hip -- bf16 grouped expert GEMMs, direct-to-LDS pipeline.
//
// Same contract as gemm.hip's grouped_gemm_kernel for the bf16 x bf16 case
// (A = expert-contiguous activations [rows][K], B = packed weights
// [E][Npad][K], K contiguous; gate/up epilogue with SwiGLU or down epilogue
// with bias), built for the large prefill-shaped segments that dominate the
// MoE layer's time.
//
// CDNA4 design (choices measured on MI355X):
//  * Persistent: one 512-thread block per CU walks the 256 x 256 output
//    tiles t = blockIdx.x, +gridDim.x, ...; the first K-slab of the next
//    tile is requested while the last slab of the current one is multiplied,
//    so the DMA stream never drains between tiles.
//  * 8 waves (2 per SIMD) each own 64 output features x 128 tokens: 2 x 4
//    tiles of v_mfma_f32_32x32x16_bf16.  Issue is in order within a wave, so
//    one wave's MFMAs cover the other's LDS and barrier waits.
//  * The MFMA computes D = W . X^T (weights as the row operand), so each
//    lane holds 4 consecutive output features of one token: the epilogue
//    writes 8-byte vectors.
//  * Operands move HBM -> LDS with global_load_lds_dwordx4 (one 1 KB row
//    block per wave instruction; no staging registers, no ds_write) into a
//    2-stage ring.  The slab barrier is a bare s_barrier after an explicit
//    vmcnt wait for the wave's own DMA; __syncthreads() would also drain the
//    prefetch in flight.
//  * LDS rows are 128 B (64 bf16); K-chunk c of row r sits at slot
//    c ^ ((r >> 1) & 7): gfx950's LDS has 64 banks, so the 16 lanes served
//    together (16 rows of one logical chunk) hit 16 distinct bank groups.
//  * SwiGLU in the epilogue uses the hardware exp/reciprocal (well inside
//    the bf16 tolerance).
#include "common.hpp"

namespace mgpt {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;                  // 8
constexpr int kBM = 256, kBN = 256, kBK = 64;             // tokens x features x K
constexpr int kWTN = 64, kWTM = 128;                      // wave tile: features x tokens
constexpr int kTN = kWTN / 32, kTM = kWTM / 32;           // 2 x 4 MFMA tiles
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

// Four floats -> four bf16 (round to nearest even) in 8 bytes.
__device__ __forceinline__ uint2 pack4_bf16(float a, float b, float c, float d) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t lo = {(__bf16)a, (__bf16)b}, hi = {(__bf16)c, (__bf16)d};
  uint2 r;
  __builtin_memcpy(&r.x, &lo, 4);
  __builtin_memcpy(&r.y, &hi, 4);
  return r;
}

struct Tile {
  int expert, row0, row_end, n0;
};

// Tile t of the (m-tile, n-tile) grid; false past the last m-tile.
__device__ __forceinline__ bool load_tile(const int32_t* counts, int E, int nbx, int t, Tile* out) {
  TileInfo ti;
  const bool ok = find_tile<kBM>(counts, E, t / nbx, &ti);
  out->expert = ti.expert;
  out->row0 = ti.row0;
  out->row_end = ti.row_end;
  out->n0 = (t % nbx) * kBN;
  return ok;
}

template <int EPI>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(
    const bf16_t* __restrict__ A, const bf16_t* __restrict__ B, const float* __restrict__ bias0,
    const float* __restrict__ bias1, const int32_t* __restrict__ counts, int E, int K, int Npad,
    int n_store, int bias_ld, bf16_t* __restrict__ out, int ldo) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStageBytes];

  const int nbx = Npad / kBN;
  const int G = gridDim.x;
  int t = blockIdx.x;
  Tile cur;
  if (!load_tile(counts, E, nbx, t, &cur)) return;

  const int tid = threadIdx.x;
  const int w = tid / kWave, lane = lane_id();
  const int wn = w & 3, wm = w >> 2;                      // 4 (features) x 2 (tokens)
  const int lrow = lane & 31, lhalf = lane >> 5;
  const size_t row_bytes_g = (size_t)K * 2;

  // DMA: row block q = w*8 + i covers LDS rows 8q .. 8q+7 (rows 0..255 =
  // activation tile, 256..511 = weight tile): waves 0-3 fill activations,
  // waves 4-7 weights.  Lane l fills slot l%8 of row r = 8q + l/8 with
  // logical chunk (l%8) ^ ((r >> 1) & 7) = (l%8) ^ ((4*(q&1) + l/16) & 7).
  const uint32_t lane_row = (uint32_t)(lane >> 3) * (uint32_t)row_bytes_g;
  const uint32_t lane_off0 = lane_row + ((uint32_t)((lane & 7) ^ (lane >> 4)) << 4);
  const uint32_t lane_off1 = lane_row + ((uint32_t)((lane & 7) ^ (4 | (lane >> 4))) << 4);
  auto dma_base = [&](const Tile& tl) -> const char* {
    const char* p = (w < 4) ? reinterpret_cast<const char*>(A + (size_t)tl.row0 * K)
                            : reinterpret_cast<const char*>(B + ((size_t)tl.expert * Npad + tl.n0) * K);
    return p + (size_t)((w & 3) * kDmaPerWave * kRowsPerDma) * row_bytes_g;
  };
  auto dma = [&](const char* gbase, int kt, int stage) __attribute__((always_inline)) {
    char* dst = smem + stage * kStageBytes + w * kDmaPerWave * 1024;
    const char* g = gbase + (size_t)kt * kRowBytes;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i)
      __builtin_amdgcn_global_load_lds(
          g + (size_t)i * kRowsPerDma * row_bytes_g + ((i & 1) ? lane_off1 : lane_off0),
          (lds_void*)(dst + i * 1024), 16, 0, 0);
  };

  // Fragment rows start at multiples of 32: (row >> 1) & 7 = (lrow >> 1) & 7.
  int x_off[kTM], w_off[kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i) x_off[i] = (wm * kWTM + i * 32 + lrow) * kRowBytes;
#pragma unroll
  for (int j = 0; j < kTN; ++j) w_off[j] = (kBM + wn * kWTN + j * 32 + lrow) * kRowBytes;
  const int swz = (lrow >> 1) & 7;

  const int KT = K / kBK;
  const char* gcur = dma_base(cur);
  int stage = 0;
  dma(gcur, 0, 0);
  for (;;) {
    Tile nxt;
    const bool have_next = load_tile(counts, E, nbx, t + G, &nxt);
    const char* gnxt = have_next ? dma_base(nxt) : gcur;

    f32x16 acc[kTN][kTM];
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][i][v] = 0.0f;

    for (int kt = 0; kt < KT; ++kt) {
      slab_barrier();
      if (kt + 1 < KT) dma(gcur, kt + 1, stage ^ 1);
      else if (have_next) dma(gnxt, 0, stage ^ 1);
      const char* st = smem + stage * kStageBytes;
      bf16x8 xf[2][kTM], wf[2][kTN];
      auto frags = [&](int ks, bf16x8 (&xs)[kTM], bf16x8 (&ws)[kTN]) __attribute__((always_inline)) {
        const int cofs = (((ks * 2 + lhalf) ^ swz) << 4);
#pragma unroll
        for (int i = 0; i < kTM; ++i) xs[i] = *reinterpret_cast<const bf16x8*>(st + x_off[i] + cofs);
#pragma unroll
        for (int j = 0; j < kTN; ++j) ws[j] = *reinterpret_cast<const bf16x8*>(st + w_off[j] + cofs);
      };
      frags(0, xf[0], wf[0]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4) frags(ks + 1, xf[(ks + 1) & 1], wf[(ks + 1) & 1]);
#pragma unroll
        for (int j = 0; j < kTN; ++j)
#pragma unroll
          for (int i = 0; i < kTM; ++i)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks & 1][j], xf[ks & 1][i],
                                                                acc[j][i], 0, 0, 0);
      }
      stage ^= 1;
    }

    // ---- epilogue straight from the accumulators.  Register v of a 32x32
    // tile holds feature row 8*(v/4) + 4*(lane/32) + v%4 (four consecutive
    // features per group v/4) and token column lane%32.
    const int tok_base = cur.row0 + wm * kWTM + lrow;
    if constexpr (EPI == kEpiGateUp) {
      // the wave's 64 packed rows are one [32 gate | 32 up] group
      const int hbase = (cur.n0 + wn * kWTN) / 2 + 4 * lhalf;
      const float* bgp = bias0 + (size_t)cur.expert * bias_ld + hbase;
      const float* bup = bias1 + (size_t)cur.expert * bias_ld + hbase;
      float4 bg4[4], bu4[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bg4[g] = *reinterpret_cast<const float4*>(bgp + 8 * g);
        bu4[g] = *reinterpret_cast<const float4*>(bup + 8 * g);
      }
#pragma unroll
      for (int i = 0; i < kTM; ++i) {
        const int row = tok_base + i * 32;
        if (row < cur.row_end) {
          bf16_t* orow = out + (size_t)row * ldo + hbase;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x16& ga = acc[0][i];
            const f32x16& ua = acc[1][i];
            *reinterpret_cast<uint2*>(orow + 8 * g) =
                pack4_bf16(silu_mul_fast(ga[4 * g + 0] + bg4[g].x, ua[4 * g + 0] + bu4[g].x),
                           silu_mul_fast(ga[4 * g + 1] + bg4[g].y, ua[4 * g + 1] + bu4[g].y),
                           silu_mul_fast(ga[4 * g + 2] + bg4[g].z, ua[4 * g + 2] + bu4[g].z),
                           silu_mul_fast(ga[4 * g + 3] + bg4[g].w, ua[4 * g + 3] + bu4[g].w));
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        const int cbase = cur.n0 + wn * kWTN + j * 32 + 4 * lhalf;
        if (cbase >= n_store) continue;   // n_store is a multiple of 64
        const float* bdp = bias0 + (size_t)cur.expert * bias_ld + cbase;
        float4 b4[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) b4[g] = *reinterpret_cast<const float4*>(bdp + 8 * g);
#pragma unroll
        for (int i = 0; i < kTM; ++i) {
          const int row = tok_base + i * 32;
          if (row < cur.row_end) {
            bf16_t* orow = out + (size_t)row * ldo + cbase;
            const f32x16& a = acc[j][i];
#pragma unroll
            for (int g = 0; g < 4; ++g)
              *reinterpret_cast<uint2*>(orow + 8 * g) =
                  pack4_bf16(a[4 * g + 0] + b4[g].x, a[4 * g + 1] + b4[g].y,
                             a[4 * g + 2] + b4[g].z, a[4 * g + 3] + b4[g].w);
          }
        }
      }
    }
    if (!have_next) break;
    cur = nxt;
    gcur = gnxt;
    t += G;
  }
}

}  // namespace

// Persistent launch: one block per CU (the kernel walks the tiles itself).
// max_mtiles bounds sum_e ceil(count_e / 256); it only caps the grid.
template <int EPI>
hipError_t launch_gemm_dma(const bf16_t* A, const bf16_t* B, const float* bias0,
                           const float* bias1, const int32_t* counts, int E, int K, int Npad,
                           int n_store, int bias_ld, bf16_t* out, int ldo, int max_mtiles,
                           hipStream_t stream) {
  if (max_mtiles <= 0) return hipSuccess;
  if (K % kBK != 0 || Npad % kBN != 0 || n_store % 64 != 0) return hipErrorInvalidValue;
  static int num_cus = 0;
  if (num_cus == 0) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || num_cus <= 0) num_cus = 256;
  }
  const int tiles = max_mtiles * (Npad / kBN);
  const int grid = tiles < num_cus ? tiles : num_cus;
  hipLaunchKernelGGL((gemm_dma_kernel<EPI>), dim3(grid), dim3(kThreads), 0, stream, A, B, bias0,
                     bias1, counts, E, K, Npad, n_store, bias_ld, out, ldo);
  return hipGetLastError();
}

template hipError_t launch_gemm_dma<kEpiGateUp>(const bf16_t*, const bf16_t*, const float*,
                                                const float*, const int32_t*, int, int, int, int,
                                                int, bf16_t*, int, int, hipStream_t);
template hipError_t launch_gemm_dma<kEpiDown>(const bf16_t*, const bf16_t*, const float*,
                                              const float*, const int32_t*, int, int, int, int,
                                              int, bf16_t*, int, int, hipStream_t);

}  // namespace mgpt
