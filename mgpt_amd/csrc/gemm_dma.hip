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
//    tiles; the blocks of one XCD take consecutive tiles of an order that
//    groups 4 token blocks x all feature blocks, so they share operand
//    panels in their XCD's L2.  Tile lookup is a per-wave register scan of
//    the expert counts (no LDS, no barrier).
//  * 8 waves (2 per SIMD) each own 64 output features x 128 tokens: 2 x 4
//    tiles of v_mfma_f32_32x32x16_bf16.  Issue is in order within a wave, so
//    one wave's MFMAs cover the other's LDS and barrier waits.
//  * The MFMA computes D = W . X^T (weights as the row operand), so each
//    lane holds 4 consecutive output features of one token: the epilogue
//    writes 8-byte vectors.
//  * Operands move HBM -> LDS with global_load_lds_dwordx4 (1 KB per wave
//    instruction; no staging registers, no ds_write) into a ring of five
//    32 KB units (activations or weights of a 64-column slab) that runs
//    across tile boundaries.  The loads are inline asm the compiler does not
//    track, with explicit vmcnt waits: for the builtin it inserts vmcnt(0)
//    before LDS reads, which serialises the ring.
//  * Fragments are read one k-step ahead of the MFMAs, interleaved with
//    them (sched_group_barrier), across slab boundaries.
//  * LDS rows are 128 B (64 bf16); K-chunk c of row r sits at slot
//    c ^ ((r >> 1) & 7): gfx950's LDS has 64 banks, so the 16 lanes served
//    together (16 rows of one logical chunk) hit 16 distinct bank groups.
//  * SwiGLU in the epilogue uses the hardware exp/reciprocal (well inside
//    the bf16 tolerance).
#include <type_traits>

#include "common.hpp"

namespace mgpt {
namespace {

constexpr int kBM = 256, kBN = 256;                       // tokens x features per tile

// Wave layout of a block: NW waves as WN (features) x WM (tokens); each wave
// owns a WTN x WTM tile of TN x TM 32x32 MFMA tiles.
template <int NW>
struct Waves {
  static constexpr int kWaves = NW;
  static constexpr int kThreads = NW * kWave;
  static constexpr int WN = NW == 8 ? 4 : 2, WM = 2;
  static constexpr int WTN = kBN / WN, WTM = kBM / WM;
  static constexpr int TN = WTN / 32, TM = WTM / 32;
  static_assert(WN * WM == NW, "wave layout");
};

typedef __attribute__((address_space(3))) char lds_char;

template <int V>
struct IntC {
  static constexpr int value = V;
};

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
// e holds expert e_base + e of the launch's group of E <= 64 experts; more
// experts run one launch per group, whose rows start after the earlier
// groups' rows), so that locating a tile needs no memory access and no
// barrier.
struct SegScan {
  // (the exclusive counts are recomputed where needed: the kernel runs at
  // the register limit, and these live in every lane throughout)
  int cnt, rows_incl, tiles_incl, tm;
  __device__ __forceinline__ int tiles_excl() const { return tiles_incl - (cnt + kBM - 1) / kBM; }
  __device__ __forceinline__ void init(const int32_t* __restrict__ counts, int E, int e_base) {
    const int l = lane_id();
    cnt = (l < E) ? counts[e_base + l] : 0;
    const int tiles = (cnt + kBM - 1) / kBM;
    int before = 0;   // rows of the experts before the group
    if (e_base > 0) {
      for (int e = l; e < e_base; e += kWave) before += counts[e];
      before = __builtin_amdgcn_readfirstlane(__shfl(wave_incl_scan(before), kWave - 1, kWave));
    }
    rows_incl = wave_incl_scan(cnt) + before;
    tiles_incl = wave_incl_scan(tiles);
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
  const int texcl = sc.tiles_excl();
  const bool mine = (l < E) && (mt >= texcl) && (mt < sc.tiles_incl);
  const unsigned long long m = __ballot(mine);
  const int owner = __ffsll((long long)m) - 1;   // exists: mt < tm
  out->expert = __builtin_amdgcn_readfirstlane(owner);
  out->row0 = __builtin_amdgcn_readfirstlane(
      __shfl((sc.rows_incl - sc.cnt) + (mt - texcl) * kBM, owner, kWave));
  out->row_end = __builtin_amdgcn_readfirstlane(__shfl(sc.rows_incl, owner, kWave));
  out->n0 = (idx / gsize) * kBN;
  return true;
}

// The accumulators of one 32 x 32 tile as VGPR values.  With 4 waves per
// block (256 accumulators per lane) the accumulators live in AGPRs; reading
// them through v_accvgpr_read one tile at a time stops the compiler from
// copying all 256 into VGPRs at the loop exit (which spills).  The caller
// has waited out the MFMA result latency (mfma_drain).
template <int NW>
__device__ __forceinline__ f32x16 acc_fetch(const f32x16& a) {
  if constexpr (NW == 8) {
    return a;
  } else {
    f32x16 r;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      float x;
      asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(a[v]));
      r[v] = x;
    }
    return r;
  }
}

template <int NW>
__device__ __forceinline__ void mfma_drain() {
  if constexpr (NW != 8) asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");
}

// Stores the 32 outputs (features base .. base+31) of one token that a lane
// pair (l, l+32) holds as quads: q[g] of lane l are features 8g..8g+3, of lane
// l+32 features 8g+4..8g+7 (bf16 pairs).  Swapping two quads across the pair
// leaves lane l with the whole 8-feature groups 0 and 2 and lane l+32 with 1
// and 3, so each lane writes 16-byte vectors and a store covers 32 bytes of
// each of the 32 token rows (instead of 16).  The swap is gfx950's
// v_permlane32_swap (a VALU op, no LDS round trip): swap(a, b) gives lane
// l < 32 the pair (a[l], a[l+32]) and lane l >= 32 (b[l-32], b[l]), which
// with (a, b) = (q[0], q[1]) is each lane's 8-feature group as it is stored.
// Every lane of the pair must run this (it exchanges registers); `store`
// gates the memory writes.
__device__ __forceinline__ void store_group32(bf16_t* base, const uint2 (&q)[4], int lhalf,
                                              bool store) {
  const auto ax = __builtin_amdgcn_permlane32_swap(q[0].x, q[1].x, false, false);
  const auto ay = __builtin_amdgcn_permlane32_swap(q[0].y, q[1].y, false, false);
  const auto bx = __builtin_amdgcn_permlane32_swap(q[2].x, q[3].x, false, false);
  const auto by = __builtin_amdgcn_permlane32_swap(q[2].y, q[3].y, false, false);
  const uint4 w0 = make_uint4(ax[0], ay[0], ax[1], ay[1]);
  const uint4 w1 = make_uint4(bx[0], by[0], bx[1], by[1]);
  if (store) {
    *reinterpret_cast<uint4*>(base + 8 * lhalf) = w0;
    *reinterpret_cast<uint4*>(base + 16 + 8 * lhalf) = w1;
  }
}

// The inverse of store_group32: loads the 32 bf16 values (features base ..
// base+31) of one token as two 16-byte vectors per lane (lane half h takes
// features 8h..8h+7 and 16+8h..16+8h+7) and swaps quads with the partner
// lane, so that q[g] of lane half h holds features 8g+4h .. 8g+4h+3, the
// accumulator layout.  Rows past the segment read zeros (no access); every
// lane of the pair runs the swaps.
__device__ __forceinline__ void load_group32(const bf16_t* base, uint2 (&q)[4], int lhalf,
                                             bool load) {
  uint4 w0 = make_uint4(0u, 0u, 0u, 0u), w1 = w0;
  if (load) {
    w0 = *reinterpret_cast<const uint4*>(base + 8 * lhalf);
    w1 = *reinterpret_cast<const uint4*>(base + 16 + 8 * lhalf);
  }
  const auto s0 = __builtin_amdgcn_permlane32_swap(w0.x, w0.z, false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(w0.y, w0.w, false, false);
  const auto s2 = __builtin_amdgcn_permlane32_swap(w1.x, w1.z, false, false);
  const auto s3 = __builtin_amdgcn_permlane32_swap(w1.y, w1.w, false, false);
  q[0] = make_uint2(s0[0], s1[0]);
  q[1] = make_uint2(s0[1], s1[1]);
  q[2] = make_uint2(s2[0], s3[0]);
  q[3] = make_uint2(s2[1], s3[1]);
}

// Epilogue straight from the accumulators of a wave's WTN-feature x
// WTM-token tile.  Register v of a 32x32 tile holds feature row
// 8*(v/4) + 4*(lane/32) + v%4 (four consecutive features per group v/4) and
// token column lane%32.  Biases are read at wave-uniform addresses (scalar
// loads): a vector load here would make the compiler wait for the DMA loads
// it does not track as well.
template <int EPI, int NW, bool kSave>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[Waves<NW>::TN][Waves<NW>::TM],
                                           const Tile& cur, int wn, int wm, int lrow, int lhalf,
                                           int n_store, bf16_t* out, int ldo, bf16_t* save,
                                           int save_ld) {
  using W = Waves<NW>;
  const int tok_base = cur.row0 + wm * W::WTM + lrow;
  if constexpr (EPI == kEpiGateUp) {
    // each 64 packed rows of the wave are one [32 gate | 32 up] group
#pragma unroll
    for (int gi = 0; gi < W::TN / 2; ++gi) {
      const int hb = (cur.n0 + wn * W::WTN) / 2 + 32 * gi;
#pragma unroll
      for (int i = 0; i < W::TM; ++i) {
        const int row = tok_base + i * 32;
        const f32x16 ga = acc_fetch<NW>(acc[2 * gi][i]);
        const f32x16 ua = acc_fetch<NW>(acc[2 * gi + 1][i]);
        uint2 q[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int v = 4 * g;
          q[g] = pack4_bf16(silu_mul_fast(ga[v + 0], ua[v + 0]), silu_mul_fast(ga[v + 1], ua[v + 1]),
                            silu_mul_fast(ga[v + 2], ua[v + 2]), silu_mul_fast(ga[v + 3], ua[v + 3]));
        }
        store_group32(out + (size_t)row * ldo + hb, q, lhalf, row < cur.row_end);
        if constexpr (kSave) {
          // pre-activations for the backward pass, in the packed column order
          const int pc = cur.n0 + wn * W::WTN + 64 * gi;
          uint2 sg[4], su[4];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int v = 4 * g;
            sg[g] = pack4_bf16(ga[v], ga[v + 1], ga[v + 2], ga[v + 3]);
            su[g] = pack4_bf16(ua[v], ua[v + 1], ua[v + 2], ua[v + 3]);
          }
          store_group32(save + (size_t)row * save_ld + pc, sg, lhalf, row < cur.row_end);
          store_group32(save + (size_t)row * save_ld + pc + 32, su, lhalf, row < cur.row_end);
        }
      }
      // one column group at a time: keeps the scheduler from hoisting every
      // accumulator read (TN * TM * 16 values) ahead of the stores
      __builtin_amdgcn_sched_barrier(0);
    }
  } else if constexpr (EPI == kEpiSwigluBwd) {
    // The features are hidden units h and the accumulators d(act)[row][h];
    // save holds the pre-activations g, u of h at its packed columns (32 gate
    // then 32 up per 32 units), and d(gate), d(up) overwrite them there.
#pragma unroll
    for (int j = 0; j < W::TN; ++j) {
      const int hb = cur.n0 + wn * W::WTN + j * 32;
      if (hb >= n_store) continue;
      const int pc = packed_gate_col(hb);
      // the g and u loads of two 32-token sub-tiles at a time, as 16-byte
      // vectors: half the memory round trips of one at a time, within the
      // register budget (four at a time spill)
      constexpr int kPair = 2;
#pragma unroll
      for (int i2 = 0; i2 < W::TM; i2 += kPair) {
        uint2 gq[kPair][4], uq[kPair][4];
#pragma unroll
        for (int ii = 0; ii < kPair; ++ii) {
          const int row = tok_base + (i2 + ii) * 32;
          const bool ok = row < cur.row_end;
          const bf16_t* src = save + (size_t)row * save_ld + pc;
          load_group32(src, gq[ii], lhalf, ok);
          load_group32(src + 32, uq[ii], lhalf, ok);
        }
#pragma unroll
        for (int ii = 0; ii < kPair; ++ii) {
          const int i = i2 + ii;
          const int row = tok_base + i * 32;
          const bool ok = row < cur.row_end;
          const f32x16 a = acc_fetch<NW>(acc[j][i]);
          uint2 dq[4], uqo[4];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float dg[4], du[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t gw = q < 2 ? gq[ii][g].x : gq[ii][g].y;
              const uint32_t uw = q < 2 ? uq[ii][g].x : uq[ii][g].y;
              const float gv = __uint_as_float((q & 1) ? (gw & 0xFFFF0000u) : (gw << 16));
              const float uv = __uint_as_float((q & 1) ? (uw & 0xFFFF0000u) : (uw << 16));
              const float d = a[4 * g + q];
              const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-gv));
              du[q] = d * (gv * sig);
              dg[q] = (d * uv) * (sig * (1.0f + gv * (1.0f - sig)));
            }
            dq[g] = pack4_bf16(dg[0], dg[1], dg[2], dg[3]);
            uqo[g] = pack4_bf16(du[0], du[1], du[2], du[3]);
          }
          store_group32(out + (size_t)row * ldo + pc, dq, lhalf, ok);
          store_group32(out + (size_t)row * ldo + pc + 32, uqo, lhalf, ok);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int j = 0; j < W::TN; ++j) {
      const int cb = cur.n0 + wn * W::WTN + j * 32;
      if (cb >= n_store) continue;   // n_store is a multiple of 64
#pragma unroll
      for (int i = 0; i < W::TM; ++i) {
        const int row = tok_base + i * 32;
        const f32x16 a = acc_fetch<NW>(acc[j][i]);
        uint2 q[4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
          q[g] = pack4_bf16(a[4 * g + 0], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]);
        store_group32(out + (size_t)row * ldo + cb, q, lhalf, row < cur.row_end);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Work items of a persistent launch over T tiles with G blocks: the
// ceil(T/G)-th round would leave most blocks idle when T % G is small, so
// the tiles of that last round are split along K into s parts (s <= 8,
// G/(T % G) of them), each a work item of its own whose fp32 partial sums
// go to a workspace; gemm_split_reduce_kernel adds the parts in order and
// runs the epilogue.  All tiles of the full rounds are whole items.  A
// split item writes a 256 KB fp32 partial tile and the reduce kernel reads
// them back, a cost that only a long K amortises: tiles of fewer than
// kMinSplitSlabs 64-column slabs stay whole.  Measured on MI355X at the
// cfg3 shapes (skewed counts): gate/up (K = 1024, 16 slabs) 0.426 ms whole
// vs 0.439 split; down (K = 2816, 44 slabs) 0.214 split vs 0.246 whole.
constexpr int kMinSplitSlabs = 24;
struct SplitPlan {
  int full, rem, s, items;
  __device__ __forceinline__ void init(int T, int G, int KT, bool enable) {
    full = (T / G) * G;
    rem = T - full;
    s = 1;
    if (enable && rem > 0 && KT >= kMinSplitSlabs) {
      s = min(min(G / rem, 8), KT);
      if (s < 2) s = 1;
    }
    items = s > 1 ? full + rem * s : T;
  }
};

struct Work {
  Tile tile;
  int k0, k1;   // slab range
  int sidx;     // partial-sum slot, or -1 for a whole tile
};

__device__ __forceinline__ bool locate_work(const SegScan& sc, const SplitPlan& pl, int E,
                                            int nbx, int KT, int v, Work* wk) {
  if (v >= pl.items) return false;
  int tv;
  if (pl.s == 1 || v < pl.full) {
    tv = v;
    wk->k0 = 0;
    wk->k1 = KT;
    wk->sidx = -1;
  } else {
    const int u = v - pl.full;
    const int part = u % pl.s;
    tv = pl.full + u / pl.s;
    wk->k0 = part * KT / pl.s;
    wk->k1 = (part + 1) * KT / pl.s;
    wk->sidx = u;
  }
  return locate_tile(sc, E, nbx, tv, &wk->tile);
}

// The accumulators of a work item start from the biases of its features
// (the same for every token), or from zero for split-K parts (the reduce
// kernel adds the bias), the SwiGLU backward and a down product without
// bias.  Register v of a 32x32 tile holds feature 8*(v/4) + 4*(lane/32) +
// v%4.  The biases are read at wave-uniform addresses (scalar loads): a
// vector load would make the compiler wait for the ring's DMA loads, which
// it does not track, as well.
template <int EPI, int NW>
__device__ __forceinline__ void init_acc(f32x16 (&acc)[Waves<NW>::TN][Waves<NW>::TM],
                                         const Work& wk, int wn, int lhalf,
                                         const float* __restrict__ bias0,
                                         const float* __restrict__ bias1, int bias_ld) {
  using W = Waves<NW>;
  const bool has_bias = EPI != kEpiSwigluBwd && wk.sidx < 0 && bias0 != nullptr;
#pragma unroll
  for (int j = 0; j < W::TN; ++j) {
    f32x16 b;
    if (has_bias) {
      const float* src;
      if constexpr (EPI == kEpiGateUp) {
        // packed rows: each 64 of them are [32 gate | 32 up] of hidden units hb..hb+31
        const int hb = (wk.tile.n0 + wn * W::WTN) / 2 + 32 * (j / 2);
        src = ((j & 1) ? bias1 : bias0) + (size_t)wk.tile.expert * bias_ld + hb;
      } else {
        src = bias0 + (size_t)wk.tile.expert * bias_ld + wk.tile.n0 + wn * W::WTN + 32 * j;
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 v = *reinterpret_cast<const float4*>(src + 8 * g + 4 * lhalf);
        b[4 * g] = v.x;
        b[4 * g + 1] = v.y;
        b[4 * g + 2] = v.z;
        b[4 * g + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) b[v] = 0.0f;
    }
    // The wait for these loads happens here, at the item's start: past this
    // point the values count as computed, so sub-tiles that no MFMA
    // touches (MT < 4) do not make the epilogue wait for the loads and,
    // with them, for the ring's DMA.
    if constexpr (EPI != kEpiSwigluBwd) asm volatile("" : "+v"(b));
#pragma unroll
    for (int i = 0; i < W::TM; ++i) acc[j][i] = b;
    // one feature group at a time: keeps the scheduler from hoisting all
    // TN * 32 scalar loads together (SGPR pressure)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Partial sums of one work item, a whole 256 x 256 fp32 tile, stored as
// [TN*TM*4 float4 slots q][threads] so that every store and load is a
// coalesced row.  q = (j * kTM + i) * 4 + v4 holds acc[j][i][4v4 ..].
constexpr int kPartialFloats = 256 * 256;

// ---------------------------------------------------------------------------
// Split ring.  LDS holds 5 units of 32 KB, a unit being the 256 activation
// rows or the 256 weight rows of one 64-column slab (128-byte rows, as in
// the whole design).  Units are loaded in the order A0 B0 A1 B1 ...; slab s
// reads units 2s and 2s+1, and barrier B_s frees the two units of slab s-1
// and refills them with units 2s+3 (weights of slab s+1) and 2s+4
// (activations of slab s+2): the activations are requested two slabs ahead
// and the weights one (a 2-stage ring of 64 KB slabs manages one for both).
template <int EPI, int NW, bool kSave>
__global__ __launch_bounds__(NW * 64) void gemm_ring5_kernel(
    const bf16_t* __restrict__ A, const bf16_t* __restrict__ B, const float* __restrict__ bias0,
    const float* __restrict__ bias1, const int32_t* __restrict__ counts, int E, int e_base, int K,
    int Npad, int n_store, int bias_ld, bf16_t* out, int ldo, float* __restrict__ partials,
    bf16_t* save, int save_ld) {
  using W = Waves<NW>;
  constexpr int kTN = W::TN, kTM = W::TM;
  constexpr int kUnits = 5;
  constexpr int kRowBytes = 128;
  constexpr int kUnit = 256 * kRowBytes;           // 32 KB
  constexpr int kDmaPerWave = kUnit / 1024 / NW;   // 1 KB loads per wave and unit
  constexpr int kWaveRows = 256 / NW;              // unit rows each wave loads
  __shared__ __attribute__((aligned(1024))) char smem[kUnits * kUnit];

  const int nbx = Npad / kBN;
  const int G = gridDim.x;
  int t = (G % kNumXcd == 0) ? (blockIdx.x % kNumXcd) * (G / kNumXcd) + blockIdx.x / kNumXcd
                             : blockIdx.x;
  const int KT = K / 64;
  SegScan sc;
  sc.init(counts, E, e_base);
  SplitPlan plan;
  plan.init(sc.tm * nbx, G, KT, partials != nullptr);
  Work cur;
  if (!locate_work(sc, plan, E, nbx, KT, t, &cur)) return;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave), lane = lane_id();
  const int wn = w % W::WN, wm = w / W::WN;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const size_t row_bytes_g = (size_t)K * 2;

  // DMA of a unit: wave w fills its kWaveRows rows in blocks of 8 rows;
  // lane l covers row r = 8i + l/8, slot l%8 = chunk ^ ((r >> 1) & 7)
  // (kWaveRows is a multiple of 16, so the slot depends on i & 1 only).
  uint32_t lane_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = i * 8 + lane / 8;
    lane_off[i] = (uint32_t)(lane / 8) * (uint32_t)row_bytes_g +
                  (uint32_t)((((lane % 8) ^ ((r >> 1) & 7))) * 16);
  }
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char*)smem + (uint32_t)(w * kDmaPerWave * 1024);
  auto abase = [&](const Tile& tl) -> const char* {
    return reinterpret_cast<const char*>(A + ((size_t)tl.row0 + kWaveRows * w) * K);
  };
  auto bbase = [&](const Tile& tl) -> const char* {
    return reinterpret_cast<const char*>(B + ((size_t)tl.expert * Npad + tl.n0 + kWaveRows * w) * K);
  };

  // Cursor over units: (work item dwk, slab dkt, operand dop), ring slot
  // dslot.
  Work dwk = cur;
  int dt = t, dkt = cur.k0, dop = 0, dslot = 0;
  bool dvalid = true;
  const char* dga = abase(cur.tile);
  const char* dgb = bbase(cur.tile);
  const char* dlast = dga;
  // Source and ring slot of the next unit.  Past the end of the block's
  // work it repeats the last real unit (in bounds, into a freed slot), so
  // every slab issues the same loads and waits the same way.
  auto next_unit = [&](const char*& g, uint32_t& dst) __attribute__((always_inline)) {
    if (dvalid) dlast = (dop ? dgb : dga) + (size_t)dkt * kRowBytes;
    g = dlast;
    dst = lds_base + (uint32_t)(dslot * kUnit);
    dslot = dslot + 1 == kUnits ? 0 : dslot + 1;
    if (dop == 0) {
      dop = 1;
    } else {
      dop = 0;
      if (dvalid && ++dkt == dwk.k1) {
        dt += G;
        dvalid = locate_work(sc, plan, E, nbx, KT, dt, &dwk);
        if (dvalid) {
          dkt = dwk.k0;
          dga = abase(dwk.tile);
          dgb = bbase(dwk.tile);
        }
      }
    }
  };
  auto dma_loads = [&](const char* g, uint32_t dst, int i0, int n) __attribute__((always_inline)) {
#pragma unroll
    for (int i = i0; i < i0 + n; ++i)
      dma16(g + (size_t)(i * 8) * row_bytes_g + lane_off[i & 1], dst + i * 1024);
  };
  // The two units refilled after barrier B_s (weights of slab s+1, then
  // activations of slab s+2, into the slots of slab s-1) are issued a
  // quarter at a time in the four MFMA segments that follow, so that the
  // loads queue behind MFMAs instead of 64 of them reaching the load unit
  // together at the barrier.  B_s waits for units 2s and 2s+1 with the four
  // loads of unit 2s+2 still allowed in flight.
  const char* ug[2];
  uint32_t ud[2];
  auto quarter = [&](int q) __attribute__((always_inline)) {
    dma_loads(ug[q >> 1], ud[q >> 1], (q & 1) * (kDmaPerWave / 2), kDmaPerWave / 2);
  };
  auto slab_wait = [&]() __attribute__((always_inline)) {
    slab_barrier<kDmaPerWave>();
    next_unit(ug[0], ud[0]);
    next_unit(ug[1], ud[1]);
  };

  const int x_row = (wm * W::WTM + lrow) * kRowBytes;
  const int w_row = (wn * W::WTN + lrow) * kRowBytes;
  const int swz = (lrow >> 1) & 7;
  bf16x8 xf[2][kTM], wf[2][kTN];
  // k-step ks of the slab whose activation unit is in ring slot `aslot`
  // (its weight unit follows in the next slot)
  auto frags = [&](int aslot, int ks, bf16x8 (&xs)[kTM], bf16x8 (&ws)[kTN])
      __attribute__((always_inline)) {
    const int bslot = aslot + 1 == kUnits ? 0 : aslot + 1;
    const char* sa = smem + aslot * kUnit + x_row;
    const char* sb = smem + bslot * kUnit + w_row;
    const int cofs = (((ks * 2 + lhalf) ^ swz) << 4);
#pragma unroll
    for (int i = 0; i < kTM; ++i)
      xs[i] = *reinterpret_cast<const bf16x8*>(sa + i * 32 * kRowBytes + cofs);
#pragma unroll
    for (int j = 0; j < kTN; ++j)
      ws[j] = *reinterpret_cast<const bf16x8*>(sb + j * 32 * kRowBytes + cofs);
  };

  // Prologue: units 0, 1, 2 (A0 B0 A1), then B_0 and the first quarter.
  for (int u = 0; u < 3; ++u) {
    const char* g;
    uint32_t dst;
    next_unit(g, dst);
    dma_loads(g, dst, 0, kDmaPerWave);
  }
  slab_wait();
  quarter(0);
  frags(0, 0, xf[0], wf[0]);
  int aslot = 0;

  for (;;) {
    Work nxt;
    const bool have_next = locate_work(sc, plan, E, nbx, KT, t + G, &nxt);
    f32x16 acc[kTN][kTM];
    init_acc<EPI, NW>(acc, cur, wn, lhalf, bias0, bias1, bias_ld);

    // The k loop for MT live 32-token sub-tiles of this wave (the rest of
    // its 128 tokens lie past the segment: their MFMAs would only multiply
    // padding rows, which costs time and, the chip being power-limited,
    // clock).  Loads, fragment reads and barriers are the same for all MT.
    auto kloop = [&](auto mt_c) __attribute__((always_inline)) {
      constexpr int MT = decltype(mt_c)::value;
      constexpr int kReads = kTM + kTN, kMfma = kTN * MT;
      constexpr int kPairs = kReads < kMfma ? kReads : kMfma;
      for (int kt = cur.k0; kt < cur.k1; ++kt) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          if (ks + 1 < 4) {
            quarter(ks + 1);
            frags(aslot, ks + 1, xf[(ks + 1) & 1], wf[(ks + 1) & 1]);
          } else {
            // next slab; after the block's last slab this reads stale units
            // whose values are never used (one code path keeps the
            // compiler's LDS wait counting exact)
            aslot += 2;
            if (aslot >= kUnits) aslot -= kUnits;
            slab_wait();
            quarter(0);
            frags(aslot, 0, xf[0], wf[0]);
          }
#pragma unroll
          for (int j = 0; j < kTN; ++j)
#pragma unroll
            for (int i = 0; i < MT; ++i)
              acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks & 1][j], xf[ks & 1][i],
                                                                  acc[j][i], 0, 0, 0);
#pragma unroll
          for (int q = 0; q < kPairs; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
          }
          if constexpr (kMfma > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kPairs, 0);
          if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPairs, 0);
        }
      }
    };
    const int wrows = cur.tile.row_end - (cur.tile.row0 + wm * W::WTM);
    const int mt_live = wrows <= 0 ? 0 : min(kTM, (wrows + 31) / 32);
    static_assert(kTM == 4, "sub-tile dispatch below");
    switch (mt_live) {
      case 0: kloop(IntC<0>{}); break;
      case 1: kloop(IntC<1>{}); break;
      case 2: kloop(IntC<2>{}); break;
      case 3: kloop(IntC<3>{}); break;
      default: kloop(IntC<4>{}); break;
    }
    mfma_drain<NW>();
    if (cur.sidx < 0) {
      // The lane's row and half recomputed here rather than kept live from
      // the start: the kernel runs at the register limit, and a value held
      // across the k loop gets spilled (its reload then waits for the
      // ring's DMA loads as well).
      int lane_now;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0"
                   : "=v"(lane_now));
      store_tile<EPI, NW, kSave>(acc, cur.tile, wn, wm, lane_now & 31, lane_now >> 5, n_store,
                                 out, ldo, save, save_ld);
    } else {
      float4* P = reinterpret_cast<float4*>(partials + (size_t)cur.sidx * kPartialFloats) + tid;
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
#pragma unroll
        for (int i = 0; i < kTM; ++i) {
          const f32x16 a = acc_fetch<NW>(acc[j][i]);
#pragma unroll
          for (int v4 = 0; v4 < 4; ++v4)
            P[((j * kTM + i) * 4 + v4) * W::kThreads] =
                make_float4(a[4 * v4], a[4 * v4 + 1], a[4 * v4 + 2], a[4 * v4 + 3]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (!have_next) break;
    t += G;
    cur = nxt;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the repeated tail loads
}


// Sums the s partial tiles of each split tile in order and applies the
// epilogue, one output quad (4 features of one token) per thread and
// iteration: the s float4 loads of a quad are independent, so each thread
// keeps them all in flight, and the quads of all split tiles are spread over
// the whole grid.  The (GEMM thread, slot) -> (token, feature) mapping is
// the one store_tile applies to the GEMM's accumulators.
template <int EPI, int NW>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(
    const float* __restrict__ partials, const float* __restrict__ bias0,
    const float* __restrict__ bias1, const int32_t* __restrict__ counts, int E, int e_base, int K,
    int Npad, int n_store, int bias_ld, bf16_t* __restrict__ out, int ldo, int G) {
  using W = Waves<NW>;
  constexpr int kTM = W::TM, kT = W::kThreads;
  constexpr bool kGU = EPI == kEpiGateUp;
  // quads per tile: gate/up pairs two slots (gate j, up j+1) into one quad
  constexpr int kQuads = kT * W::TN * kTM * 4 / (kGU ? 2 : 1);
  const int nbx = Npad / kBN;
  const int KT = K / 64;
  SegScan sc;
  sc.init(counts, E, e_base);
  SplitPlan plan;
  plan.init(sc.tm * nbx, G, KT, true);
  if (plan.s == 1) return;
  const int total = plan.rem * kQuads;
  // kQuads is a multiple of 256, so r (and the tile) is uniform per block
  for (int u = blockIdx.x * 256 + threadIdx.x; u < total; u += gridDim.x * 256) {
    const int r = u / kQuads, uq = u % kQuads;
    Tile tile;
    if (!locate_tile(sc, E, nbx, plan.full + r, &tile)) return;
    const int tid = uq % kT, qq = uq / kT;
    const int w = tid / kWave, lane = tid % kWave;
    const int wn = w % W::WN, wm = w / W::WN, lrow = lane & 31, lhalf = lane >> 5;
    const int g = qq % 4, i = (qq / 4) % kTM, j = qq / (4 * kTM);   // j: column group (pair)
    const int row = tile.row0 + wm * W::WTM + lrow + i * 32;
    if (row >= tile.row_end) continue;
    const float4* P = reinterpret_cast<const float4*>(partials + (size_t)r * plan.s * kPartialFloats) + tid;
    if constexpr (kGU) {
      const int qg = ((2 * j) * kTM + i) * 4 + g, qu = ((2 * j + 1) * kTM + i) * 4 + g;
      float4 ga = make_float4(0.f, 0.f, 0.f, 0.f), ua = ga;
      for (int p = 0; p < plan.s; ++p) {
        const float4 x = P[(size_t)p * (kPartialFloats / 4) + qg * kT];
        const float4 y = P[(size_t)p * (kPartialFloats / 4) + qu * kT];
        ga.x += x.x; ga.y += x.y; ga.z += x.z; ga.w += x.w;
        ua.x += y.x; ua.y += y.y; ua.z += y.z; ua.w += y.w;
      }
      const int hb = (tile.n0 + wn * W::WTN) / 2 + 32 * j;
      const int f = hb + 8 * g + 4 * lhalf;
      const float* bg = bias0 + (size_t)tile.expert * bias_ld + f;
      const float* bu = bias1 + (size_t)tile.expert * bias_ld + f;
      *reinterpret_cast<uint2*>(out + (size_t)row * ldo + f) =
          pack4_bf16(silu_mul_fast(ga.x + bg[0], ua.x + bu[0]),
                     silu_mul_fast(ga.y + bg[1], ua.y + bu[1]),
                     silu_mul_fast(ga.z + bg[2], ua.z + bu[2]),
                     silu_mul_fast(ga.w + bg[3], ua.w + bu[3]));
    } else {
      const int cb = tile.n0 + wn * W::WTN + j * 32;
      if (cb >= n_store) continue;
      const int q = (j * kTM + i) * 4 + g;
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int p = 0; p < plan.s; ++p) {
        const float4 x = P[(size_t)p * (kPartialFloats / 4) + q * kT];
        a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
      }
      const int f = cb + 8 * g + 4 * lhalf;
      float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (bias0) {
        const float* bp = bias0 + (size_t)tile.expert * bias_ld + f;
        b[0] = bp[0]; b[1] = bp[1]; b[2] = bp[2]; b[3] = bp[3];
      }
      *reinterpret_cast<uint2*>(out + (size_t)row * ldo + f) =
          pack4_bf16(a.x + b[0], a.y + b[1], a.z + b[2], a.w + b[3]);
    }
  }
}

#ifndef MGPT_RING_WAVES
#define MGPT_RING_WAVES 8
#endif
constexpr int kRingWaves = MGPT_RING_WAVES;

}  // namespace

// Persistent launch: one block per CU (the kernel walks the tiles itself).
// max_mtiles bounds sum_e ceil(count_e / 256); it only caps the grid.
// partials (num_cus * kPartialFloats floats, or null to disable) holds the
// split last round; the reduce kernel that follows exits at once when the
// counts leave nothing to split.  save (gate/up only, and only without
// partials) also stores the pre-activations g + b_g, u + b_u as bf16 in the
// packed column order, save[row][n] with leading dimension save_ld.
// SWIGLU_BWD (no partials) reads those pre-activations from save and writes
// d(gate), d(up) to out in the same layout (out may equal save).  DOWN
// adds no bias when bias0 is null.  Measured on MI355X (cfg3 shapes, skewed
// counts): the split 5-unit ring (gate/up 1035, down 871 TFLOP/s) beats a
// 2-slab ring of 64 KB slabs (1034, 827) and 32-column slabs (4 x 32: 938,
// 724; 5 x 32 with 2 per barrier: 970, 786), whose 64-byte row segments
// double the DMA cost; a ping-pong schedule of the two waves of a SIMD
// (934) and weights loaded straight into registers in fragment order (990)
// did not help either.
template <int EPI>
hipError_t launch_gemm_dma(const bf16_t* A, const bf16_t* B, const float* bias0,
                           const float* bias1, const int32_t* counts, int E, int K, int Npad,
                           int n_store, int bias_ld, bf16_t* out, int ldo, int max_mtiles,
                           float* partials, int num_cus, bf16_t* save, int save_ld,
                           hipStream_t stream) {
  if (max_mtiles <= 0) return hipSuccess;
  if (E <= 0 || E > kMaxExpertsWide) return hipErrorInvalidValue;
  // 16-byte output vectors: ldo and the output base must keep 8-element alignment
  if (K % 64 != 0 || Npad % kBN != 0 || n_store % 64 != 0 || num_cus <= 0 || ldo % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(out) & 15) != 0)
    return hipErrorInvalidValue;
  if (save && (EPI == kEpiDown || partials || save_ld % 8 != 0 ||
               (reinterpret_cast<uintptr_t>(save) & 15) != 0))
    return hipErrorInvalidValue;
  if (EPI == kEpiSwigluBwd && !save) return hipErrorInvalidValue;
  // the accumulators start from the biases, read as 16-byte vectors
  if (((reinterpret_cast<uintptr_t>(bias0) | reinterpret_cast<uintptr_t>(bias1)) & 15) != 0 ||
      bias_ld % 4 != 0)
    return hipErrorInvalidValue;
  if (K / 64 < kMinSplitSlabs) partials = nullptr;   // no split, no reduce launch
  const int tiles = max_mtiles * (Npad / kBN);
  const int grid = tiles < num_cus ? tiles : num_cus;
  // More than 64 experts: one launch (and split reduce) per group of 64, the
  // weights and biases from the group's first expert on; the rows come in
  // expert order, so each group's follow the earlier groups'.
  for (int e0 = 0; e0 < E; e0 += kMaxExperts) {
    const int Eg = std::min(kMaxExperts, E - e0);
    const bf16_t* Bg = B + (size_t)e0 * Npad * K;
    const float* b0 = bias0 ? bias0 + (size_t)e0 * bias_ld : nullptr;
    const float* b1 = bias1 ? bias1 + (size_t)e0 * bias_ld : nullptr;
    // the gate/up epilogue's pre-activation stores are compiled only into
    // the training instance (fewer live registers in the inference one)
    auto launch = [&](auto save_c) {
      hipLaunchKernelGGL((gemm_ring5_kernel<EPI, kRingWaves, decltype(save_c)::value>),
                         dim3(grid), dim3(kRingWaves * kWave), 0, stream, A, Bg, b0, b1, counts,
                         Eg, e0, K, Npad, n_store, bias_ld, out, ldo, partials, save, save_ld);
    };
    if constexpr (EPI == kEpiGateUp) {
      if (save)
        launch(std::true_type{});
      else
        launch(std::false_type{});
    } else {
      launch(std::false_type{});
    }
    if constexpr (EPI != kEpiSwigluBwd) {
      if (partials)
        hipLaunchKernelGGL((gemm_split_reduce_kernel<EPI, kRingWaves>), dim3(8 * grid), dim3(256),
                           0, stream, partials, b0, b1, counts, Eg, e0, K, Npad, n_store, bias_ld,
                           out, ldo, grid);
    }
  }
  return hipGetLastError();
}

template hipError_t launch_gemm_dma<kEpiGateUp>(const bf16_t*, const bf16_t*, const float*,
                                                const float*, const int32_t*, int, int, int, int,
                                                int, bf16_t*, int, int, float*, int, bf16_t*, int,
                                                hipStream_t);
template hipError_t launch_gemm_dma<kEpiDown>(const bf16_t*, const bf16_t*, const float*,
                                              const float*, const int32_t*, int, int, int, int,
                                              int, bf16_t*, int, int, float*, int, bf16_t*, int,
                                              hipStream_t);
template hipError_t launch_gemm_dma<kEpiSwigluBwd>(const bf16_t*, const bf16_t*, const float*,
                                                   const float*, const int32_t*, int, int, int,
                                                   int, int, bf16_t*, int, int, float*, int,
                                                   bf16_t*, int, hipStream_t);

}  // namespace mgpt
