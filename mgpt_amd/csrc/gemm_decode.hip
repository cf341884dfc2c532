// gemm_decode.hip -- fp8-weight grouped expert GEMMs for decode shapes.
//
// Few tokens per expert (a decode step: N = 64 tokens, k = 8, E = 64 gives
// about 8 rows per expert) make the expert GEMMs a weight stream: every
// weight byte is used by at most 32 rows, so the bound is HBM bandwidth,
// not MFMA.  This kernel is built for that bound:
//  * Work items are (expert m-tile of <= 32 rows, 256 output features); a
//    persistent block per CU walks them, and a direct-to-LDS ring of three
//    stages (256 weight rows x 128 fp8 columns + 32 activation rows x 128
//    bf16 columns, 40 KB) keeps two stages of loads in flight per CU across
//    item boundaries.  The loads are inline asm the compiler does not track,
//    with explicit waits (as in gemm_dma.hip).
//  * 4 waves each own 64 features (a [32 gate | 32 up] pair for gate/up) x
//    the 32 token rows: two v_mfma_f32_32x32x16_bf16 per 16 columns, the
//    fp8 weights converted to bf16 in registers (exact: every e4m3 value is
//    a bf16 value); the per-output-channel scale is applied in the epilogue.
//  * K order within a stage: lane half h holds k = 64h + 8*ks + e for k-step
//    ks (element e) in both operands, so a lane's weights for the stage are
//    64 contiguous bytes of its row (four 16-byte LDS reads).
// Same contract as gemm.hip's grouped_gemm_kernel (A = expert-contiguous
// activations [rows][K], B = fp8 weights in stage tiles
// [E][Npad/256][K/128][256][128] (pack.hip: tile_fp8_kernel) with scales
// [E][Npad], SwiGLU or bias epilogue).
#include "common.hpp"

namespace mgpt {
namespace {

constexpr int kDThreads = 256;
constexpr int kDBM = 32;                     // token rows per item
constexpr int kDBN = 256;                    // features per item
constexpr int kDBK = 128;                    // columns per stage
#ifndef MGPT_DECODE_STAGES
#define MGPT_DECODE_STAGES 3
#endif
constexpr int kDStages = MGPT_DECODE_STAGES;   // ring depth (LDS: 40 KB a stage, 48 KB for fp32 rows)
constexpr int kWBytes = kDBN * kDBK;         // 32 KB of fp8 weights
constexpr int kDmaW = kWBytes / 1024 / 4;    // 8 weight blocks per wave

typedef __attribute__((address_space(3))) char lds_char;

__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
// The same for the weight stream, with the non-temporal hint: every weight
// byte is read once per step, and a decode step's weights (hundreds of MB)
// would otherwise push the activations, the router's operands and the
// combine's rows out of the caches.  Measured at cfg5 (graph-replayed
// steps): gate/up 74.1 -> 64.7 us, down 39.7 -> 35.6 us.
__device__ __forceinline__ void dma16_stream(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

__device__ __forceinline__ float uniform_load(const float* p) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(*p)));
}

// e4m3 byte pair (low or high half of a dword) -> two bf16 in one dword.
template <bool HI>
__device__ __forceinline__ uint32_t e4m3x2_to_bf16x2(uint32_t packed) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)packed, 1.0f, HI);
  uint32_t r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}

// 8 fp8 weights (two dwords) -> a bf16x8 MFMA operand.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  const uint32_t w[4] = {e4m3x2_to_bf16x2<false>(lo), e4m3x2_to_bf16x2<true>(lo),
                         e4m3x2_to_bf16x2<false>(hi), e4m3x2_to_bf16x2<true>(hi)};
  bf16x8 r;
  __builtin_memcpy(&r, w, 16);
  return r;
}

__device__ __forceinline__ float silu_mul_fast(float g, float u) {
  return g * u * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

__device__ __forceinline__ uint2 pack4_bf16(float a, float b, float c, float d) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t lo = {(__bf16)a, (__bf16)b}, hi = {(__bf16)c, (__bf16)d};
  uint2 r;
  __builtin_memcpy(&r.x, &lo, 4);
  __builtin_memcpy(&r.y, &hi, 4);
  return r;
}

struct DItem {
  int expert, row0, row_end, n0;
};

// Per-wave register scan of the expert counts in 32-row m-tiles (lane e =
// expert e, E <= 64): items are m-tiles x feature blocks, feature-major
// within an m-tile.
struct DScan {
  int cnt, rows_incl, tiles_incl, tiles_excl, tm;
  __device__ __forceinline__ void init(const int32_t* counts, int E) {   // global or LDS
    const int l = lane_id();
    cnt = (l < E) ? counts[l] : 0;
    const int tiles = (cnt + kDBM - 1) / kDBM;
    rows_incl = wave_incl_scan(cnt);
    tiles_incl = wave_incl_scan(tiles);
    tiles_excl = tiles_incl - tiles;
    tm = __builtin_amdgcn_readfirstlane(__shfl(tiles_incl, kWave - 1, kWave));
  }
  __device__ __forceinline__ bool locate(int E, int nbx, int v, DItem* out) const {
    if (v >= tm * nbx) return false;
    const int mt = v / nbx;
    const int l = lane_id();
    const bool mine = (l < E) && (mt >= tiles_excl) && (mt < tiles_incl);
    const unsigned long long m = __ballot(mine);
    const int owner = __ffsll((long long)m) - 1;
    out->expert = __builtin_amdgcn_readfirstlane(owner);
    out->row0 = __builtin_amdgcn_readfirstlane(
        __shfl((rows_incl - cnt) + (mt - tiles_excl) * kDBM, owner, kWave));
    out->row_end = __builtin_amdgcn_readfirstlane(__shfl(rows_incl, owner, kWave));
    out->n0 = (v - mt * nbx) * kDBN;
    return true;
  }
};

// The routing of at most 512 flat ids (nflat = N * k), computed by each
// block of the gathering gate/up kernel instead of a separate permute
// launch: per-expert counts, expert-major slots in
// flat order within each expert (the permute's assignment, dispatch.hip),
// and the slot -> token map s_tok.  Ids outside [0, E) get no slot, as in
// the permute.  With publish set the block also writes counts, perm and
// slot_of for the down GEMM, the combine and the caller.  All threads call
// it; wave 0 does the work.
constexpr int kGatherFlat = kRouterTokens * kMaxTopK;
__device__ __forceinline__ void decode_rank(const int32_t* __restrict__ topk_idx, int nflat,
                                            int k, int E, int* s_cnt, int* s_base, int* s_run,
                                            int* s_tok, bool publish,
                                            int32_t* __restrict__ counts,
                                            int32_t* __restrict__ perm,
                                            int32_t* __restrict__ slot_of) {
  const int tid = threadIdx.x;
  if (tid < kWave) {
    const int l = tid;
    constexpr int kIdPerLane = kGatherFlat / kWave;
    int ids[kIdPerLane];
#pragma unroll
    for (int u = 0; u < kIdPerLane; ++u) {
      const int f = u * kWave + l;
      ids[u] = f < nflat ? topk_idx[f] : -1;
    }
    s_cnt[l] = 0;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int u = 0; u < kIdPerLane; ++u)
      if (ids[u] >= 0 && ids[u] < E) atomicAdd(&s_cnt[ids[u]], 1);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const int cnt = l < E ? s_cnt[l] : 0;
    s_base[l] = wave_incl_scan(cnt) - cnt;
    s_run[l] = 0;
    if (publish && l < E) counts[l] = cnt;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const unsigned long long lt = (l == 0) ? 0ull : (~0ull >> (kWave - l));
#pragma unroll
    for (int u = 0; u < kIdPerLane; ++u) {
      const int f0 = u * kWave;
      if (f0 >= nflat) break;
      const int f = f0 + l;
      int e = ids[u];
      const bool valid = e >= 0 && e < E;
      if (!valid) e = 0;
      unsigned long long match = __ballot(valid);
#pragma unroll
      for (int bit = 0; bit < 6; ++bit) {
        const unsigned long long on = __ballot(valid && ((e >> bit) & 1));
        match &= ((e >> bit) & 1) ? on : ~on;
      }
      if (valid) {
        const int run = s_run[e];
        const int slot = s_base[e] + run + __popcll(match & lt);
        s_tok[slot] = f / k;
        if (publish) {
          perm[slot] = f;
          slot_of[f] = slot;
        }
        // the highest lane of each expert group advances the running count
        if ((match >> l) == 1ull) s_run[e] = run + __popcll(match);
      }
    }
  }
  __syncthreads();
}

// GATHER (gate/up of at most 512 flat ids, bf16 rows): the activation rows
// come straight from the caller's x through s_tok instead of from the
// gathered copy A, and the routing is computed in the block (decode_rank).
template <int EPI, bool GATHER, typename XT>
__global__ __launch_bounds__(kDThreads) void gemm_decode_kernel(
    const XT* __restrict__ A, const fp8_t* __restrict__ B, const float* __restrict__ wscale,
    const float* __restrict__ bias0, const float* __restrict__ bias1,
    const int32_t* __restrict__ counts, int E, int K, int Npad, int n_store, int bias_ld,
    bf16_t* __restrict__ out, int ldo, const int32_t* __restrict__ topk_idx, int nflat, int k,
    int32_t* __restrict__ counts_out, int32_t* __restrict__ perm,
    int32_t* __restrict__ slot_of) {
  // Activation rows of XT (bf16, or the caller's fp32 rows when gathering):
  // kRowB bytes per stage row, staged as they are and converted to bf16 when
  // the fragments are read.
  constexpr int kXS = (int)sizeof(XT);
  constexpr int kAB = kDBM * kDBK * kXS;       // activation bytes per stage
  constexpr int kStage = kWBytes + kAB;
  constexpr int kDA = kAB / 1024 / 4;          // activation blocks per wave
  constexpr int kDm = kDmaW + kDA;             // loads per wave and stage
  constexpr int kRowB = kDBK * kXS;            // LDS bytes per activation row
  constexpr int kRowsPerBlk = 1024 / kRowB;
  constexpr int kChunks = kRowB / 16;          // 16-byte chunks per row
  static_assert(kXS == 2 || kXS == 4, "bf16 or fp32 rows");
  static_assert(kDStages * kStage + kGatherFlat * 4 <= 160 * 1024,
                "the ring does not fit in LDS at this MGPT_DECODE_STAGES");
  __shared__ __attribute__((aligned(1024))) char smem[kDStages * kStage];
  __shared__ int s_tok[GATHER ? kGatherFlat : 1];
  __shared__ int s_cnt[GATHER ? kMaxExperts : 1], s_base[GATHER ? kMaxExperts : 1],
      s_run[GATHER ? kMaxExperts : 1];
  const int nbx = Npad / kDBN;
  const int G = gridDim.x;
  const int32_t* cnts = counts;
  if constexpr (GATHER) {
    decode_rank(topk_idx, nflat, k, E, s_cnt, s_base, s_run, s_tok, blockIdx.x == 0, counts_out,
                perm, slot_of);
    cnts = s_cnt;
  }
  DScan sc;
  sc.init(cnts, E);
  int v = blockIdx.x;
  DItem cur;
  if (!sc.locate(E, nbx, v, &cur)) return;

  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int lane = lane_id();
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int KT = K / kDBK;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)smem;

  // DMA lane mapping.  Weights: 128-byte rows, wave w fills rows 64w ..
  // 64w+63 in 8 blocks of 8 rows; lane l covers row 8i + l/8, slot l%8 =
  // chunk ^ ((row >> 1) & 7).  Activations: kRowB-byte rows (256 for bf16,
  // 512 for fp32), wave w fills rows 8w .. 8w+7 in kDA blocks of
  // kRowsPerBlk rows; lane l covers row kRowsPerBlk*i + l/kChunks, slot
  // l%kChunks = chunk ^ (row & (kChunks - 1)).  Activation rows past the
  // item's last token re-read that token (in bounds, never stored).
  // Weights are in the tiled layout [E][Npad/256][K/128][256][128]: a
  // stage is one contiguous 32 KB block, rows 128 bytes apart.
  const size_t wrow_g = (size_t)kDBK;       // fp8 bytes between weight rows of a stage
  const size_t arow_g = (size_t)K * kXS;    // bytes per activation row
  uint32_t woff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = i * 8 + lane / 8;
    woff[i] = (uint32_t)(lane / 8) * (uint32_t)wrow_g + (uint32_t)(((lane % 8) ^ ((r >> 1) & 7)) * 16);
  }
  auto dma_stage = [&](const DItem& it, int kt, int stage) __attribute__((always_inline)) {
    const uint32_t st = lds0 + (uint32_t)(stage * kStage);
    const char* wg = reinterpret_cast<const char*>(B) +
                     (((size_t)it.expert * nbx + it.n0 / kDBN) * KT + kt) * (size_t)kWBytes +
                     (size_t)(64 * w) * wrow_g;
#pragma unroll
    for (int i = 0; i < kDmaW; ++i)
      dma16_stream(wg + (size_t)(8 * i) * wrow_g + woff[i & 1], st + (uint32_t)((w * kDmaW + i) * 1024));
#pragma unroll
    for (int i = 0; i < kDA; ++i) {
      const int r = 8 * w + kRowsPerBlk * i + lane / kChunks;   // activation row in the tile
      const int tok = min(it.row0 + r, it.row_end - 1);         // a slot
      const int chunk = (lane % kChunks) ^ (r & (kChunks - 1));
      const int src_row = GATHER ? s_tok[tok] : tok;
      const char* ag = reinterpret_cast<const char*>(A) + (size_t)src_row * arow_g +
                       (size_t)kt * kRowB + chunk * 16;
      dma16(ag, st + (uint32_t)(kWBytes + (w * kDA + i) * 1024));
    }
  };

  // DMA cursor (item dv, stage column block dkt), STAGES-1 stages ahead.
  DItem dit = cur;
  int dv = v, dkt = 0, dstage = 0;
  bool dvalid = true;
  int ahead = 0;   // stages issued and not yet waited for
  auto advance = [&]() __attribute__((always_inline)) {
    if (dvalid) {
      dma_stage(dit, dkt, dstage);
      ++ahead;
    }
    dstage = dstage + 1 == kDStages ? 0 : dstage + 1;
    if (++dkt == KT) {
      dkt = 0;
      dv += G;
      if (dvalid) dvalid = sc.locate(E, nbx, dv, &dit);
    }
  };
  // Barrier before consuming stage c: it landed, with the stages issued
  // after it (`ahead` once c is counted) possibly in flight; every wave is
  // done with stage c-1, which the DMA issued right after refills.
  auto next_stage_barrier = [&]() __attribute__((always_inline)) {
    --ahead;
    if (ahead >= kDStages - 2) stage_barrier<(kDStages - 2) * kDm>();
    else stage_barrier<0>();
    advance();
  };

  // Fragment reads.  Weights (A operand): this wave's rows 64w + 32j + lrow,
  // bytes 64*lhalf .. +63 of the stage row = chunks 4*lhalf .. +3.
  // Activations (B operand): token row lrow, k-step ks = chunk 8*lhalf + ks.
  const int wswz = (lrow >> 1) & 7;
  auto wfrag = [&](const char* st, int j, int q) -> uint4 {   // q = chunk pair index 0..3
    const int row = 64 * w + 32 * j + lrow;
    const int chunk = 4 * lhalf + q;
    return *reinterpret_cast<const uint4*>(st + row * kDBK + ((chunk ^ wswz) << 4));
  };
  auto afrag = [&](const char* st, int ks) -> bf16x8 {
    const int c = 8 * lhalf + ks;   // columns 8c .. 8c+7 of the stage
    const char* row = st + kWBytes + lrow * kRowB;
    if constexpr (kXS == 2) {
      return *reinterpret_cast<const bf16x8*>(row + ((c ^ (lrow & 15)) << 4));
    } else {
      // two 16-byte chunks of fp32 rounded to bf16 by v_cvt_pk_bf16_f32
      // (nearest even, fp32 denormals kept: the rounding f32_to_bf16 does in
      // software for the permute's gather, at 4 instructions a fragment)
      typedef float f32x8 __attribute__((ext_vector_type(8)));
      const float4 a = *reinterpret_cast<const float4*>(row + (((2 * c) ^ (lrow & 31)) << 4));
      const float4 b = *reinterpret_cast<const float4*>(row + (((2 * c + 1) ^ (lrow & 31)) << 4));
      const f32x8 v = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      return __builtin_convertvector(v, bf16x8);
    }
  };

#pragma unroll
  for (int s = 0; s < kDStages - 1; ++s) advance();
  next_stage_barrier();
  int cstage = 0;

  for (;;) {
    DItem nxt;
    const bool have_next = sc.locate(E, nbx, v + G, &nxt);
    f32x16 acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
    for (int kt = 0; kt < KT; ++kt) {
      const char* st = smem + cstage * kStage;
      // 8 k-steps: weights as 4 chunks of 16 fp8 per row (2 k-steps each)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 w0 = wfrag(st, 0, q), w1 = wfrag(st, 1, q);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int ks = 2 * q + h;
          const bf16x8 b = afrag(st, ks);
          const bf16x8 a0 = h ? fp8x8_to_bf16x8(w0.z, w0.w) : fp8x8_to_bf16x8(w0.x, w0.y);
          const bf16x8 a1 = h ? fp8x8_to_bf16x8(w1.z, w1.w) : fp8x8_to_bf16x8(w1.x, w1.y);
          acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b, acc[0], 0, 0, 0);
          acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b, acc[1], 0, 0, 0);
        }
      }
      cstage = cstage + 1 == kDStages ? 0 : cstage + 1;
      // next stage (after the block's last one this waits for nothing new)
      next_stage_barrier();
    }

    // Epilogue.  Register e of a 32x32 tile holds feature row
    // 8*(e/4) + 4*(lane/32) + e%4 and token column lane%32.
    const int row = cur.row0 + lrow;
    const float* sc_e = wscale + (size_t)cur.expert * Npad;
    if constexpr (EPI == kEpiGateUp) {
      // rows 64w .. 64w+31 gate, 64w+32 .. +63 up of hidden units hb .. hb+31
      const int p0 = cur.n0 + 64 * w;            // packed row of gate unit 0
      const int hb = p0 / 2;
      const float* bgp = bias0 + (size_t)cur.expert * bias_ld + hb;
      const float* bup = bias1 + (size_t)cur.expert * bias_ld + hb;
      if (row < cur.row_end) {
        bf16_t* orow = out + (size_t)row * ldo + hb + 4 * lhalf;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int f = 8 * g + q;   // feature within the 32 (lane half 0)
            const float sg0 = uniform_load(sc_e + p0 + f), sg1 = uniform_load(sc_e + p0 + f + 4);
            const float su0 = uniform_load(sc_e + p0 + 32 + f), su1 = uniform_load(sc_e + p0 + 32 + f + 4);
            const float bg0 = uniform_load(bgp + f), bg1 = uniform_load(bgp + f + 4);
            const float bu0 = uniform_load(bup + f), bu1 = uniform_load(bup + f + 4);
            const float gv = acc[0][4 * g + q] * (lhalf ? sg1 : sg0) + (lhalf ? bg1 : bg0);
            const float uv = acc[1][4 * g + q] * (lhalf ? su1 : su0) + (lhalf ? bu1 : bu0);
            o[q] = silu_mul_fast(gv, uv);
          }
          *reinterpret_cast<uint2*>(orow + 8 * g) = pack4_bf16(o[0], o[1], o[2], o[3]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cb = cur.n0 + 64 * w + 32 * j;
        if (cb >= n_store || row >= cur.row_end) continue;
        const float* bdp = bias0 + (size_t)cur.expert * bias_ld + cb;
        bf16_t* orow = out + (size_t)row * ldo + cb + 4 * lhalf;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int f = 8 * g + q;
            const float s0 = uniform_load(sc_e + cb + f), s1 = uniform_load(sc_e + cb + f + 4);
            const float b0 = uniform_load(bdp + f), b1 = uniform_load(bdp + f + 4);
            o[q] = acc[j][4 * g + q] * (lhalf ? s1 : s0) + (lhalf ? b1 : b0);
          }
          *reinterpret_cast<uint2*>(orow + 8 * g) = pack4_bf16(o[0], o[1], o[2], o[3]);
        }
      }
    }
    if (!have_next) break;
    v += G;
    cur = nxt;
  }
}

// Persistent launch, one block per CU.  Requires K % 128 == 0, Npad % 256 ==
// 0 and n_store % 64 == 0; max_mtiles bounds sum_e ceil(count_e / 32).
template <int EPI, bool GATHER, typename XT>
hipError_t launch_decode(const XT* A, const fp8_t* B, const float* wscale, const float* bias0,
                         const float* bias1, const int32_t* counts, int E, int K, int Npad,
                         int n_store, int bias_ld, bf16_t* out, int ldo, int max_mtiles,
                         const int32_t* topk_idx, int nflat, int k, int32_t* counts_out,
                         int32_t* perm, int32_t* slot_of, hipStream_t stream) {
  if (max_mtiles <= 0) return hipSuccess;
  if (K % kDBK != 0 || Npad % kDBN != 0 || n_store % 64 != 0) return hipErrorInvalidValue;
  static int num_cus = 0;
  if (num_cus == 0) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || num_cus <= 0) num_cus = 256;
  }
#ifndef MGPT_DECODE_BLOCKS_PER_CU
#define MGPT_DECODE_BLOCKS_PER_CU 1
#endif
  const int items = max_mtiles * (Npad / kDBN);
  const int slots = MGPT_DECODE_BLOCKS_PER_CU * num_cus;
  const int grid = items < slots ? items : slots;
  hipLaunchKernelGGL((gemm_decode_kernel<EPI, GATHER, XT>), dim3(grid), dim3(kDThreads), 0, stream, A,
                     B, wscale, bias0, bias1, counts, E, K, Npad, n_store, bias_ld, out, ldo,
                     topk_idx, nflat, k, counts_out, perm, slot_of);
  return hipGetLastError();
}

}  // namespace

template <int EPI>
hipError_t launch_gemm_decode(const bf16_t* A, const fp8_t* B, const float* wscale,
                              const float* bias0, const float* bias1, const int32_t* counts, int E,
                              int K, int Npad, int n_store, int bias_ld, bf16_t* out, int ldo,
                              int max_mtiles, hipStream_t stream) {
  return launch_decode<EPI, false, bf16_t>(A, B, wscale, bias0, bias1, counts, E, K, Npad, n_store,
                                   bias_ld, out, ldo, max_mtiles, nullptr, 0, 0, nullptr, nullptr,
                                   nullptr, stream);
}

template hipError_t launch_gemm_decode<kEpiGateUp>(const bf16_t*, const fp8_t*, const float*,
                                                   const float*, const float*, const int32_t*, int,
                                                   int, int, int, int, bf16_t*, int, int,
                                                   hipStream_t);
template hipError_t launch_gemm_decode<kEpiDown>(const bf16_t*, const fp8_t*, const float*,
                                                 const float*, const float*, const int32_t*, int,
                                                 int, int, int, int, bf16_t*, int, int,
                                                 hipStream_t);

// The gate/up GEMM of at most 512 flat ids (nflat = N * k) with the
// caller's rows x [N][K] (bf16, or fp32 rounded to bf16 as the permute
// would): routes the ids itself (the permute's
// counts, perm and slot_of, written by block 0) and reads the activation
// rows from x, so no permute kernel runs and no gathered copy is written.
template <typename XT>
hipError_t launch_gemm_decode_gather(const XT* x, const fp8_t* B, const float* wscale,
                                     const float* bias0, const float* bias1, const int32_t* topk_idx,
                                     int nflat, int k, int E, int K, int Npad, int n_store,
                                     int bias_ld, bf16_t* out, int ldo, int max_mtiles,
                                     int32_t* counts, int32_t* perm, int32_t* slot_of,
                                     hipStream_t stream) {
  if (nflat > kGatherFlat || E > kMaxExperts || k < 1) return hipErrorInvalidValue;
  return launch_decode<kEpiGateUp, true, XT>(x, B, wscale, bias0, bias1, nullptr, E, K, Npad, n_store,
                                         bias_ld, out, ldo, max_mtiles, topk_idx, nflat, k, counts,
                                         perm, slot_of, stream);
}
template hipError_t launch_gemm_decode_gather<bf16_t>(const bf16_t*, const fp8_t*, const float*,
                                                       const float*, const float*, const int32_t*,
                                                       int, int, int, int, int, int, int, bf16_t*,
                                                       int, int, int32_t*, int32_t*, int32_t*,
                                                       hipStream_t);
template hipError_t launch_gemm_decode_gather<float>(const float*, const fp8_t*, const float*,
                                                      const float*, const float*, const int32_t*,
                                                      int, int, int, int, int, int, int, bf16_t*,
                                                      int, int, int32_t*, int32_t*, int32_t*,
                                                      hipStream_t);

}  // namespace mgpt
