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
constexpr int kBM = 256, kBN = 256;                       // tokens x features per tile
constexpr int kWTN = 64, kWTM = 128;                      // wave tile: features x tokens
constexpr int kTN = kWTN / 32, kTM = kWTM / 32;           // 2 x 4 MFMA tiles
constexpr int kLdsBytes = 128 * 1024;                     // the operand ring

// K-slab geometry.  A slab is BK columns of the 256 activation rows and the
// 256 weight rows; the ring holds STAGES slabs (BK * STAGES = 128).
template <int BK>
struct Slab {
  static constexpr int kRowBytes = BK * 2;                   // LDS row
  static constexpr int kChunks = kRowBytes / 16;             // 16-byte chunks per row
  static constexpr int kRowsPerDma = 1024 / kRowBytes;       // rows per 1 KB DMA
  static constexpr int kStageBytes = (kBM + kBN) * kRowBytes;
  static constexpr int kDmaPerWave = kStageBytes / 1024 / kWaves;
  static constexpr int kSteps = BK / 16;                     // MFMA k-steps per slab
  // LDS bank swizzle: chunk c of row r sits in slot c ^ swz(r).  gfx950 LDS
  // serves 16 lanes of a 16-byte read per pass over 64 banks (256 bytes):
  // the 16 rows of one fragment column must land on 16 distinct 16-byte bank
  // groups, i.e. rows that share (r * kChunks) mod 16 need distinct slots.
  static constexpr int kSwzDiv = 16 / kChunks;
  static __device__ __forceinline__ int swz(int r) { return (r / kSwzDiv) & (kChunks - 1); }
};

typedef __attribute__((address_space(3))) char lds_char;

// One 1 KB direct-to-LDS load: lane l's 16 bytes at g land at LDS address
// lds + 16*l.  Written as inline asm so that the compiler does not track it:
// for the builtin it places a vmcnt(0) wait before every LDS read that it
// cannot prove disjoint from the DMA, which serialises the ring.  The
// kernel waits for the DMA itself (slab_barrier); M0 is an input operand.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}

// Start of a slab: this wave's DMA of the slab has landed (at most N of its
// later DMA loads still in flight) and its own LDS reads are complete; then
// meet the other waves.  Inline asm, because the compiler treats the
// builtin s_waitcnt as a hint it may relax (it dropped the lgkmcnt(0) that
// protects the stage the next DMA overwrites), and the memory clobber keeps
// LDS accesses from moving across it.
template <int N>
__device__ __forceinline__ void slab_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// A float read at a wave-uniform address, forced into an SGPR (so the
// compiler emits a scalar load).
__device__ __forceinline__ float uniform_load(const float* p) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(*p)));
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

constexpr int kGroupM = 4;   // m-tiles per group of the tile order

// Per-expert segment bookkeeping, computed once per wave from counts[] (lane
// e holds expert e; E <= 64), so that locating a tile needs no memory access
// and no barrier.
struct SegScan {
  int cnt, rows_incl, tiles_incl, tiles_excl, tm;
  __device__ __forceinline__ void init(const int32_t* __restrict__ counts, int E) {
    const int l = lane_id();
    cnt = (l < E) ? counts[l] : 0;
    const int tiles = (cnt + kBM - 1) / kBM;
    rows_incl = wave_incl_scan(cnt);
    tiles_incl = wave_incl_scan(tiles);
    tiles_excl = tiles_incl - tiles;
    tm = __builtin_amdgcn_readfirstlane(__shfl(tiles_incl, kWave - 1, kWave));   // all m-tiles
  }
};

// Tile of linear index v, or false past the last one.  Tiles are ordered in
// groups of kGroupM m-tiles (token blocks, over all experts' segments) x all
// n-tiles, m fastest, so that any 32 consecutive indices cover about 4 token
// blocks x 8 feature blocks: the 32 blocks of one XCD (see the remap in the
// kernel) then share 12 operand panels in that XCD's L2 instead of ~23.
__device__ __forceinline__ bool locate_tile(const SegScan& sc, int E, int nbx, int v, Tile* out) {
  if (v >= sc.tm * nbx) return false;
  const int g = v / (kGroupM * nbx);
  const int gsize = min(kGroupM, sc.tm - g * kGroupM);
  const int idx = v - g * kGroupM * nbx;
  const int mt = g * kGroupM + idx % gsize;
  const int l = lane_id();
  const bool mine = (l < E) && (mt >= sc.tiles_excl) && (mt < sc.tiles_incl);
  const unsigned long long m = __ballot(mine);
  const int owner = __ffsll((long long)m) - 1;   // exists: mt < tm
  out->expert = __builtin_amdgcn_readfirstlane(owner);
  out->row0 = __builtin_amdgcn_readfirstlane(
      __shfl((sc.rows_incl - sc.cnt) + (mt - sc.tiles_excl) * kBM, owner, kWave));
  out->row_end = __builtin_amdgcn_readfirstlane(__shfl(sc.rows_incl, owner, kWave));
  out->n0 = (idx / gsize) * kBN;
  return true;
}

// Epilogue straight from the accumulators of a wave's 64-feature x
// 128-token tile.  Register v of a 32x32 tile holds feature row
// 8*(v/4) + 4*(lane/32) + v%4 (four consecutive features per group v/4) and
// token column lane%32.  Biases are read at wave-uniform addresses (scalar
// loads): a vector load here would make the compiler wait for the DMA loads
// it does not track as well.
template <int EPI>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[kTN][kTM], const Tile& cur, int wn,
                                           int wm, int lrow, int lhalf,
                                           const float* __restrict__ bias0,
                                           const float* __restrict__ bias1, int n_store,
                                           int bias_ld, bf16_t* __restrict__ out, int ldo) {
    const int tok_base = cur.row0 + wm * kWTM + lrow;
    if constexpr (EPI == kEpiGateUp) {
      // the wave's 64 packed rows are one [32 gate | 32 up] group
      const int hb = (cur.n0 + wn * kWTN) / 2;
      const float* bgp = bias0 + (size_t)cur.expert * bias_ld + hb;
      const float* bup = bias1 + (size_t)cur.expert * bias_ld + hb;
      float bg[16], bu[16];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float g0 = uniform_load(bgp + 8 * g + q), g1 = uniform_load(bgp + 8 * g + 4 + q);
          const float u0 = uniform_load(bup + 8 * g + q), u1 = uniform_load(bup + 8 * g + 4 + q);
          bg[4 * g + q] = lhalf ? g1 : g0;
          bu[4 * g + q] = lhalf ? u1 : u0;
        }
#pragma unroll
      for (int i = 0; i < kTM; ++i) {
        const int row = tok_base + i * 32;
        if (row < cur.row_end) {
          bf16_t* orow = out + (size_t)row * ldo + hb + 4 * lhalf;
          const f32x16& ga = acc[0][i];
          const f32x16& ua = acc[1][i];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int v = 4 * g;
            *reinterpret_cast<uint2*>(orow + 8 * g) =
                pack4_bf16(silu_mul_fast(ga[v + 0] + bg[v + 0], ua[v + 0] + bu[v + 0]),
                           silu_mul_fast(ga[v + 1] + bg[v + 1], ua[v + 1] + bu[v + 1]),
                           silu_mul_fast(ga[v + 2] + bg[v + 2], ua[v + 2] + bu[v + 2]),
                           silu_mul_fast(ga[v + 3] + bg[v + 3], ua[v + 3] + bu[v + 3]));
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        const int cb = cur.n0 + wn * kWTN + j * 32;
        if (cb >= n_store) continue;   // n_store is a multiple of 64
        const float* bdp = bias0 + (size_t)cur.expert * bias_ld + cb;
        float b[16];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float b0 = uniform_load(bdp + 8 * g + q), b1 = uniform_load(bdp + 8 * g + 4 + q);
            b[4 * g + q] = lhalf ? b1 : b0;
          }
#pragma unroll
        for (int i = 0; i < kTM; ++i) {
          const int row = tok_base + i * 32;
          if (row < cur.row_end) {
            bf16_t* orow = out + (size_t)row * ldo + cb + 4 * lhalf;
            const f32x16& a = acc[j][i];
#pragma unroll
            for (int g = 0; g < 4; ++g)
              *reinterpret_cast<uint2*>(orow + 8 * g) =
                  pack4_bf16(a[4 * g + 0] + b[4 * g + 0], a[4 * g + 1] + b[4 * g + 1],
                             a[4 * g + 2] + b[4 * g + 2], a[4 * g + 3] + b[4 * g + 3]);
          }
        }
      }
    }
}

// The operand stream is a sequence of slabs (tile, kt) over the tiles this
// block owns.  A DMA cursor runs STAGES-1 slabs ahead of the MFMA consumer,
// crossing tile boundaries, so the ring never drains between tiles.  Needs
// K / BK >= STAGES - 1 (the cursor is then at most one tile ahead) and an
// even number of 16-wide k-steps per slab.
template <int EPI, int BK, int STAGES>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(
    const bf16_t* __restrict__ A, const bf16_t* __restrict__ B, const float* __restrict__ bias0,
    const float* __restrict__ bias1, const int32_t* __restrict__ counts, int E, int K, int Npad,
    int n_store, int bias_ld, bf16_t* __restrict__ out, int ldo) {
  using S = Slab<BK>;
  static_assert(STAGES * S::kStageBytes == kLdsBytes, "ring size");
  static_assert(S::kDmaPerWave * S::kRowsPerDma * 4 == kBM, "four waves per operand");
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];

  const int nbx = Npad / kBN;
  const int G = gridDim.x;
  // Blocks are dispatched round-robin over the 8 XCDs; give the blocks of
  // one XCD consecutive tile indices in every round.
  int t = (G % kNumXcd == 0) ? (blockIdx.x % kNumXcd) * (G / kNumXcd) + blockIdx.x / kNumXcd
                             : blockIdx.x;
  SegScan sc;
  sc.init(counts, E);
  Tile cur;
  if (!locate_tile(sc, E, nbx, t, &cur)) return;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave), lane = lane_id();
  const int wn = w & 3, wm = w >> 2;                      // 4 (features) x 2 (tokens)
  const int lrow = lane & 31, lhalf = lane >> 5;
  const size_t row_bytes_g = (size_t)K * 2;
  const int KT = K / BK;

  // DMA: waves 0-3 fill the activation rows 0..255 of a stage, waves 4-7 the
  // weight rows 256..511, 64 rows per wave in kDmaPerWave 1 KB blocks.  Lane
  // l of block i covers row r = 64*(w&3) + i*kRowsPerDma + l/kChunks, slot
  // l%kChunks, and so loads logical chunk slot ^ swz(r) of that row.
  uint32_t lane_off[S::kDmaPerWave];
#pragma unroll
  for (int i = 0; i < S::kDmaPerWave; ++i) {
    const int r = i * S::kRowsPerDma + lane / S::kChunks;   // within the wave's 64 rows
    const int c = (lane % S::kChunks) ^ S::swz(r);          // 64*(w&3) keeps swz(r)
    lane_off[i] = (uint32_t)r * (uint32_t)row_bytes_g + (uint32_t)(c * 16);
  }
  auto dma_base = [&](const Tile& tl) -> const char* {
    const char* p = (w < 4) ? reinterpret_cast<const char*>(A + (size_t)tl.row0 * K)
                            : reinterpret_cast<const char*>(B + ((size_t)tl.expert * Npad + tl.n0) * K);
    return p + (size_t)((w & 3) * 64) * row_bytes_g;
  };
  const uint32_t lds_base =
      (uint32_t)(uintptr_t)(lds_char*)smem + (uint32_t)(w * S::kDmaPerWave * 1024);
  auto dma = [&](const char* gbase, int kt, int stage) __attribute__((always_inline)) {
    const uint32_t dst = lds_base + (uint32_t)(stage * S::kStageBytes);
    const char* g = gbase + (size_t)kt * S::kRowBytes;
#pragma unroll
    for (int i = 0; i < S::kDmaPerWave; ++i) dma16(g + lane_off[i], dst + i * 1024);
  };

  // Fragment rows start at multiples of 32, so swz(row) = swz(lrow).
  int x_off[kTM], w_off[kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i) x_off[i] = (wm * kWTM + i * 32 + lrow) * S::kRowBytes;
#pragma unroll
  for (int j = 0; j < kTN; ++j) w_off[j] = (kBM + wn * kWTN + j * 32 + lrow) * S::kRowBytes;
  const int swz = S::swz(lrow);

  // DMA cursor: the next slab to load (tile dtile, column block dkt) and
  // its ring stage.
  Tile dtile = cur;
  int dt = t, dkt = 0, dstage = 0;
  bool dvalid = true;
  const char* dg = dma_base(cur);
  int ahead = 0;   // slabs issued after the newest slab known to have landed
  auto advance = [&]() __attribute__((always_inline)) {
    if (dvalid) {
      dma(dg, dkt, dstage);
      ++ahead;
    }
    dstage = dstage + 1 == STAGES ? 0 : dstage + 1;
    if (++dkt == KT) {
      dkt = 0;
      dt += G;
      if (dvalid) dvalid = locate_tile(sc, E, nbx, dt, &dtile);
      if (dvalid) dg = dma_base(dtile);
    }
  };
  // Barrier B_c before the first fragment read of slab c: slab c has landed
  // (the slabs issued after it may still be in flight: `ahead` of them), and
  // every wave has finished reading slab c-1, whose stage the DMA issued
  // right after the barrier refills.
  auto next_slab_barrier = [&]() __attribute__((always_inline)) {
    --ahead;
    if (ahead == STAGES - 2) slab_barrier<(STAGES - 2) * S::kDmaPerWave>();
    else slab_barrier<0>();
    advance();
  };

  bf16x8 xf[2][kTM], wf[2][kTN];
  auto frags = [&](int stage, int ks, bf16x8 (&xs)[kTM], bf16x8 (&ws)[kTN])
      __attribute__((always_inline)) {
    const char* st = smem + stage * S::kStageBytes;
    const int cofs = (((ks * 2 + lhalf) ^ swz) << 4);
#pragma unroll
    for (int i = 0; i < kTM; ++i) xs[i] = *reinterpret_cast<const bf16x8*>(st + x_off[i] + cofs);
#pragma unroll
    for (int j = 0; j < kTN; ++j) ws[j] = *reinterpret_cast<const bf16x8*>(st + w_off[j] + cofs);
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) advance();
  ++ahead;   // B_0 consumes slab 0
  next_slab_barrier();
  frags(0, 0, xf[0], wf[0]);
  int cstage = 0;

  for (;;) {
    Tile nxt;
    const bool have_next = locate_tile(sc, E, nbx, t + G, &nxt);
    f32x16 acc[kTN][kTM];
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][i][v] = 0.0f;

    // Fragments run one k-step ahead of the MFMAs, across slab (and tile)
    // boundaries: the reads of slab c+1's first k-step overlap the MFMAs of
    // slab c's last one.  S::kSteps is even, so k-step s uses buffer s & 1.
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int ks = 0; ks < S::kSteps; ++ks) {
        if (ks + 1 < S::kSteps) {
          frags(cstage, ks + 1, xf[(ks + 1) & 1], wf[(ks + 1) & 1]);
        } else {
          // Next slab (after the block's last one this reads a stale stage
          // whose values are never used: one code path keeps the compiler's
          // LDS wait counting exact).
          cstage = cstage + 1 == STAGES ? 0 : cstage + 1;
          next_slab_barrier();
          frags(cstage, 0, xf[0], wf[0]);
        }
#pragma unroll
        for (int j = 0; j < kTN; ++j)
#pragma unroll
          for (int i = 0; i < kTM; ++i)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks & 1][j], xf[ks & 1][i],
                                                                acc[j][i], 0, 0, 0);
        // Issue order: the next k-step's six fragment reads one per MFMA
        // from the start, so their latency hides under this k-step's MFMAs
        // (left alone, the scheduler sinks them to the end to reuse
        // registers).
#pragma unroll
        for (int q = 0; q < kTM + kTN; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kTM * kTN - (kTM + kTN), 0);
      }
    }

    store_tile<EPI>(acc, cur, wn, wm, lrow, lhalf, bias0, bias1, n_store, bias_ld, out, ldo);
    if (!have_next) break;
    t += G;
    cur = nxt;
  }
}


}  // namespace

// Persistent launch: one block per CU (the kernel walks the tiles itself).
// max_mtiles bounds sum_e ceil(count_e / 256); it only caps the grid.  The
// ring is 2 slabs of 64 columns: measured on MI355X, halving the barriers
// beats a deeper ring of 32-column slabs (4 x 32: 898 TFLOP/s, 2 x 64: 1036
// TFLOP/s on the cfg3 gate/up shape).
template <int EPI>
hipError_t launch_gemm_dma(const bf16_t* A, const bf16_t* B, const float* bias0,
                           const float* bias1, const int32_t* counts, int E, int K, int Npad,
                           int n_store, int bias_ld, bf16_t* out, int ldo, int max_mtiles,
                           hipStream_t stream) {
  if (max_mtiles <= 0) return hipSuccess;
  if (K % 64 != 0 || Npad % kBN != 0 || n_store % 64 != 0) return hipErrorInvalidValue;
  static int num_cus = 0;
  if (num_cus == 0) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || num_cus <= 0) num_cus = 256;
  }
  const int tiles = max_mtiles * (Npad / kBN);
  const int grid = tiles < num_cus ? tiles : num_cus;
  hipLaunchKernelGGL((gemm_dma_kernel<EPI, 64, 2>), dim3(grid), dim3(kThreads), 0, stream, A, B,
                     bias0, bias1, counts, E, K, Npad, n_store, bias_ld, out, ldo);
  return hipGetLastError();
}

template hipError_t launch_gemm_dma<kEpiGateUp>(const bf16_t*, const bf16_t*, const float*,
                                                const float*, const int32_t*, int, int, int, int,
                                                int, bf16_t*, int, int, hipStream_t);
template hipError_t launch_gemm_dma<kEpiDown>(const bf16_t*, const bf16_t*, const float*,
                                              const float*, const int32_t*, int, int, int, int,
                                              int, bf16_t*, int, int, hipStream_t);

}  // namespace mgpt
