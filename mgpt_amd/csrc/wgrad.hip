// wgrad.hip -- weight and bias gradients of the expert Linear layers.
//
// Reference: LinearLayer::backward_into (layers/LinearLayer.cpp:33-80) run
// per expert by SwiGLU::backward_into (layers/SwiGLU.cpp:57-96) from the
// host loop of MoELayer::backward_into (layers/MoELayer.cpp:158-180):
//   dW += X_e^T . dY_e   (transpose + matmul2d_raw, utils/Tensor.cpp:567-577)
//   db += sum_rows(dY_e) (utils/Tensor.cpp:1599-1617), add_grad :638-650,
// where X_e / dY_e are the expert's rows.  Here one launch covers every
// expert: D_e[i][j] = sum over the expert's rows s of P[s][i] * Q[s][j],
// with P and Q the row-major activation / gradient buffers of the grouped
// forward (rows expert-contiguous), accumulated into fp32 gradients.
//
// The contraction runs over rows, which are the strided dimension of both
// operands, while the MFMA wants each lane's 8 (bf16) k-values contiguous.
// Each thread therefore loads an 8 x 8 (bf16; 4 x 4 for fp32) block of
// 16-byte row pieces, transposes it in registers, and writes 8 feature rows
// of 16 bytes into LDS tiles laid out [feature][64 rows] (128-byte rows),
// the same fragment layout the forward GEMMs read.  Global -> register ->
// LDS double buffering, one barrier per 64-row slab.
//
// Bias gradients are the column sums of Q: the threads that transpose Q
// blocks add up their rows while doing so, and the blocks of the first
// i-tile reduce and accumulate them.
//
// Block -> tile map.  An expert's tile grid (Iy x Jx tiles of 256 x 256) is
// cut into groups of up to 16 tiles (gy x gx rectangles), the groups of all
// experts are listed heaviest expert first (count descending, then id), and
// group j goes to XCD j % 8 (the hardware deals workgroup ids round-robin
// to the 8 XCDs).  The 32 CUs of an XCD thus run two 16-tile rectangles at
// a time and share their operand panels (gy P panels, gx Q panels) in the
// XCD's L2, instead of every tile reading both panels from HBM; the
// longest contractions start first.
#include "common.hpp"

#include <algorithm>
#include <climits>

namespace mgpt {
namespace {

constexpr int kTI = 256, kTJ = 256;   // output tile
constexpr int kThreads = 512;         // 8 waves: 2 (i) x 4 (j), 128 x 64 each
constexpr int kRowBytes = 128;        // LDS row: one feature's slab of rows
constexpr int kOpBytes = 256 * kRowBytes;   // one operand tile (32 KB)

template <typename T> struct WgT;
template <> struct WgT<bf16_t> { static constexpr int EPV = 8; };   // (wgrad_tr_kernel)
template <> struct WgT<float> { static constexpr int BK = 32, EPV = 4; };

// 16-byte chunk c of LDS row r sits at slot c ^ swz(r).  (r >> 1) spreads
// the 16 consecutive rows a fragment read serves together over all eight
// slots of both bank halves; (r >> 4) spreads the rows 8 apart that one
// transposed-block write covers.
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 4)) & 7; }

typedef __attribute__((address_space(3))) char lds_char;

// The tile and row segment of this block (see the block -> tile map
// above); false past the last tile.  Called by every thread of the block
// (shared memory and a barrier).  An expert's rows are cut into chunks of
// chunk_rows rows (the last one shorter), each a "virtual expert" with the
// expert's whole tile grid; lane v of wave 0 describes virtual expert v
// (at most 64 of them).  Chunk 0 of an expert accumulates into the
// gradient; chunk c >= 1 writes partial slot `pslot` (its expert's earlier
// chunks and the other experts' extra chunks before it, in expert order),
// which wgrad_reduce_kernel adds in chunk order afterwards.
struct WgTile {
  int seg0, cnt, e, ty, tx, pslot;
};

__device__ __forceinline__ bool wg_locate(const int32_t* __restrict__ counts, int E,
                                          int chunk_rows, int Iy, int Jx, int gy, int gx,
                                          WgTile* out) {
  __shared__ int s_seg[6];
  if (threadIdx.x < kWave && E > kWave) {
    // More experts than lanes (no row chunks then: chunk_rows is INT_MAX):
    // one virtual expert per expert with rows, in expert order, found by a
    // scan of the counts 64 experts at a time.
    const int l = lane_id();
    const int ngx = (Jx + gx - 1) / gx;
    const int ng = ((Iy + gy - 1) / gy) * ngx;
    const int b = blockIdx.x, sidx = b / kNumXcd;
    const int j = (sidx / 16) * kNumXcd + b % kNumXcd, r = sidx % 16;
    const int pos = j / ng, gi = j % ng;
    int rows_carry = 0, v_carry = 0, found = -1, seg = 0, vc = 0;
    for (int e0 = 0; e0 < E && found < 0; e0 += kWave) {
      const int e = e0 + l;
      const int cnt = e < E ? counts[e] : 0;
      const int has = cnt > 0 ? 1 : 0;
      const int rows_incl = wave_incl_scan(cnt) + rows_carry;
      const int v_incl = wave_incl_scan(has) + v_carry;
      const unsigned long long m = __ballot(has && v_incl - 1 == pos);
      const int owner = m ? (__ffsll((long long)m) - 1) : 0;
      const int sg = __shfl(rows_incl - cnt, owner, kWave);
      const int ct = __shfl(cnt, owner, kWave);
      if (m) {
        found = e0 + owner;
        seg = sg;
        vc = ct;
      }
      rows_carry = __shfl(rows_incl, kWave - 1, kWave);
      v_carry = __shfl(v_incl, kWave - 1, kWave);
    }
    if (l == 0) {
      const int ty = (gi / ngx) * gy + r / gx, tx = (gi % ngx) * gx + r % gx;
      const bool ok = found >= 0 && r < gy * gx && ty < Iy && tx < Jx;
      s_seg[0] = seg;
      s_seg[1] = vc;
      s_seg[2] = ok ? ty : -1;
      s_seg[3] = tx;
      s_seg[4] = found;
      s_seg[5] = -1;
    }
  } else if (threadIdx.x < kWave) {
    const int l = lane_id();
    const int cnt = l < E ? counts[l] : 0;
    const int incl = wave_incl_scan(cnt);
    const int nch = cnt > 0 ? (cnt - 1) / chunk_rows + 1 : 0;   // chunks of expert l
    const int ch_incl = wave_incl_scan(nch);
    const int xtra = nch > 0 ? nch - 1 : 0;                     // partial slots of expert l
    const int x_incl = wave_incl_scan(xtra);
    // (reads of one lane's value at a wave-uniform lane index are v_readlane,
    // not an LDS permute round trip per step)
    const int V = __builtin_amdgcn_readlane(ch_incl, kWave - 1);
    // virtual expert l: chunk c of expert ve (ve = experts whose chunks all
    // precede l); lanes l >= V describe nothing
    int ve = 0;
    for (int e2 = 0; e2 < E; ++e2) ve += __builtin_amdgcn_readlane(ch_incl, e2) <= l;
    const int src = ve < E ? ve : 0;
    const int c = l - (__shfl(ch_incl, src, kWave) - __shfl(nch, src, kWave));
    const int cnt_e = __shfl(cnt, src, kWave);
    const bool valid = l < V;
    const int off = valid ? c * chunk_rows : 0;   // c * chunk_rows < cnt_e on valid lanes
    const int vcnt = valid ? min(chunk_rows, cnt_e - off) : 0;
    const int vseg = __shfl(incl - cnt, src, kWave) + off;
    // (the cross-lane read outside the condition: lane src must be active)
    const int xex = __shfl(x_incl - xtra, src, kWave);
    const int pslot = c >= 1 ? xex + c - 1 : -1;
    // rank of virtual expert l in (rows descending, index ascending)
    int rank = 0;
    for (int v2 = 0; v2 < V; ++v2) {
      const int c2 = __builtin_amdgcn_readlane(vcnt, v2);
      rank += (c2 > vcnt) || (c2 == vcnt && v2 < l);
    }
    const int ngx = (Jx + gx - 1) / gx;
    const int ng = ((Iy + gy - 1) / gy) * ngx;   // groups per virtual expert
    const int b = blockIdx.x, sidx = b / kNumXcd;
    const int j = (sidx / 16) * kNumXcd + b % kNumXcd, r = sidx % 16;
    const int pos = j / ng, gi = j % ng;
    const bool mine = valid && rank == pos;
    const unsigned long long m = __ballot(mine);
    if (l == 0) {
      const int ty = (gi / ngx) * gy + r / gx, tx = (gi % ngx) * gx + r % gx;
      const bool ok = m != 0 && r < gy * gx && ty < Iy && tx < Jx;
      s_seg[2] = ok ? ty : -1;
      s_seg[3] = tx;
    }
    if (mine) {
      s_seg[0] = vseg;
      s_seg[1] = vcnt;
      s_seg[4] = src;
      s_seg[5] = pslot;
    }
  }
  __syncthreads();
  out->ty = s_seg[2];
  if (out->ty < 0) return false;
  out->seg0 = s_seg[0];
  out->cnt = s_seg[1];
  out->tx = s_seg[3];
  out->e = s_seg[4];
  out->pslot = s_seg[5];
  return out->cnt > 0;
}

// Accumulates a wave's 128 (i) x 32*TJ (j) block of D into the gradient
// (+=, like add_grad), or stores it when `store` (the gradient is known to
// be zero, so the read is skipped).  Register v of tile (ti, tj) is
// D[i][j] with i = 8*(v/4) + 4*lhalf + v%4 and j = lrow inside the tile.
// All loads of a 16-value group are issued before any add, so the
// read-modify-write costs one memory round trip per group instead of one
// per value; rows past i_store (only in the last row tile) take a guarded
// path.  MODE 1: the j columns are gate/up interleaved (32 gate, then 32
// up, per 32 units) and go to out0 / out1 at column h.
template <int MODE, int TJ>
__device__ __forceinline__ void wg_accumulate(const f32x16 (&acc)[4][TJ], int i_base, int j_base,
                                              int lrow, int lhalf, int e, float* out0,
                                              float* out1, int ldo, size_t out_estride,
                                              int i_store, int j_store, bool store) {
  constexpr int TI = 4;
  const bool rows_full = i_base + TI * 32 <= i_store;   // wave-uniform
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    const int j = j_base + tj * 32 + lrow;
    float* ob;
    int col;
    bool jok;
    if constexpr (MODE == 0) {
      ob = out0;
      col = j;
      jok = j < j_store;
    } else {
      ob = ((j >> 5) & 1) ? out1 : out0;
      col = (j >> 6) * 32 + (j & 31);
      jok = col < j_store;
    }
    if (!jok) continue;
    ob += (size_t)e * out_estride + col;
    float* orow = ob + (size_t)(i_base + 4 * lhalf) * ldo;
    if (rows_full && store) {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          orow[(size_t)(ti * 32 + 8 * (v / 4) + (v % 4)) * ldo] = acc[ti][tj][v];
    } else if (rows_full) {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti) {
        float old[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) old[v] = orow[(size_t)(ti * 32 + 8 * (v / 4) + (v % 4)) * ldo];
#pragma unroll
        for (int v = 0; v < 16; ++v)
          orow[(size_t)(ti * 32 + 8 * (v / 4) + (v % 4)) * ldo] = old[v] + acc[ti][tj][v];
      }
    } else {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int di = ti * 32 + 8 * (v / 4) + (v % 4);
          if (i_base + 4 * lhalf + di < i_store) {
            float* o = orow + (size_t)di * ldo;
            *o = store ? acc[ti][tj][v] : *o + acc[ti][tj][v];
          }
        }
    }
  }
}

// Adds column sum `sum` of tile column j to the bias gradient (stores it
// when `store`).
template <int MODE>
__device__ __forceinline__ void wg_bias_add(float sum, int j, int e, float* bias0, float* bias1,
                                            size_t bias_estride, int j_store,
                                            bool store = false) {
  float* bb;
  int col;
  bool ok;
  if constexpr (MODE == 0) {
    bb = bias0;
    col = j;
    ok = j < j_store;
  } else {
    bb = ((j >> 5) & 1) ? bias1 : bias0;
    col = (j >> 6) * 32 + (j & 31);
    ok = col < j_store;
  }
  if (ok) {
    float* o = bb + (size_t)e * bias_estride + col;
    *o = store ? sum : *o + sum;
  }
}

template <typename T, int MODE>
__global__ __launch_bounds__(kThreads) void wgrad_kernel(
    const T* __restrict__ P, int ldp, int p_valid, const T* __restrict__ Q, int ldq, int q_valid,
    const int32_t* __restrict__ counts, int E, int Iy, int Jx, int gy, int gx,
    float* __restrict__ out0, float* __restrict__ out1, int ldo, size_t out_estride, int i_store,
    int j_store, float* __restrict__ bias0, float* __restrict__ bias1, size_t bias_estride,
    int store) {
  constexpr int BK = WgT<T>::BK, EPV = WgT<T>::EPV;
  constexpr int NB = (BK / EPV) * (256 / EPV) / 256;   // transposed blocks per thread
  constexpr int FB = 256 / EPV;                        // feature blocks per tile
  constexpr bool kBf = sizeof(T) == 2;
  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * kOpBytes];
  const int tid = threadIdx.x;
  WgTile tl;
  if (!wg_locate(counts, E, INT_MAX, Iy, Jx, gy, gx, &tl)) return;
  const int seg0 = tl.seg0, cnt = tl.cnt, e = tl.e, ty = tl.ty, tx = tl.tx;
  const int seg_end = seg0 + cnt;
  const int i0 = ty * kTI, j0 = tx * kTJ;
  const bool do_bias = ty == 0 && bias0 != nullptr;

  // Loader role: waves 0-3 transpose P blocks, waves 4-7 Q blocks.
  const int op = tid / 256, tt = tid % 256;
  const T* src = op ? Q : P;
  const int ld = op ? ldq : ldp;
  const int valid = op ? q_valid : p_valid;
  const int f0 = op ? j0 : i0;
  const bool bias_role = op == 1 && do_bias;
  uint4 R[NB][EPV];
  float bacc[NB][EPV];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int c = 0; c < EPV; ++c) bacc[nb][c] = 0.0f;

  auto gload = [&](int kt) __attribute__((always_inline)) {
    const int s0 = seg0 + kt * BK;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int b = tt + 256 * nb;
      const int fb = b % FB, sb = b / FB;
      const int f = f0 + fb * EPV;
#pragma unroll
      for (int q = 0; q < EPV; ++q) {
        const int row = s0 + sb * EPV + q;
        if (row < seg_end && f < valid)
          R[nb][q] = *reinterpret_cast<const uint4*>(src + (size_t)row * ld + f);
        else
          R[nb][q] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
    char* base = smem + (buf * 2 + op) * kOpBytes;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int b = tt + 256 * nb;
      const int fb = b % FB, sb = b / FB;
#pragma unroll
      for (int c = 0; c < EPV; ++c) {
        uint4 t;
        if constexpr (kBf) {
          // t holds element c of rows q = 0..7 (two per dword, low half first)
          const int d = c >> 1;
          auto el = [&](int q) -> uint32_t {
            const uint4& r = R[nb][q];
            const uint32_t w = d == 0 ? r.x : (d == 1 ? r.y : (d == 2 ? r.z : r.w));
            return (c & 1) ? (w >> 16) : (w & 0xFFFFu);
          };
          t.x = el(0) | (el(1) << 16);
          t.y = el(2) | (el(3) << 16);
          t.z = el(4) | (el(5) << 16);
          t.w = el(6) | (el(7) << 16);
          if (bias_role) {
            const float v0 = bf16_to_f32(el(0)), v1 = bf16_to_f32(el(1));
            const float v2 = bf16_to_f32(el(2)), v3 = bf16_to_f32(el(3));
            const float v4 = bf16_to_f32(el(4)), v5 = bf16_to_f32(el(5));
            const float v6 = bf16_to_f32(el(6)), v7 = bf16_to_f32(el(7));
            bacc[nb][c] += ((((((v0 + v1) + v2) + v3) + v4) + v5) + v6) + v7;
          }
        } else {
          auto el = [&](int q) -> uint32_t {
            const uint4& r = R[nb][q];
            return c == 0 ? r.x : (c == 1 ? r.y : (c == 2 ? r.z : r.w));
          };
          t.x = el(0);
          t.y = el(1);
          t.z = el(2);
          t.w = el(3);
          if (bias_role)
            bacc[nb][c] += ((__uint_as_float(t.x) + __uint_as_float(t.y)) +
                            __uint_as_float(t.z)) + __uint_as_float(t.w);
        }
        const int row = fb * EPV + c;
        *reinterpret_cast<uint4*>(base + row * kRowBytes + ((sb ^ swz(row)) << 4)) = t;
      }
    }
  };

  const int w = tid / kWave, lane = lane_id();
  const int wi = w / 4, wj = w % 4;
  const int lrow = lane & 31, lhalf = lane >> 5;
  constexpr int TI = 4, TJ = 2;   // 32x32 tiles per wave: 128 (i) x 64 (j)
  f32x16 acc[TI][TJ];
#pragma unroll
  for (int a = 0; a < TI; ++a)
#pragma unroll
    for (int b = 0; b < TJ; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

  const int KT = (cnt + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    const char* pa = smem + (cur * 2 + 0) * kOpBytes;
    const char* qa = smem + (cur * 2 + 1) * kOpBytes;
    if constexpr (kBf) {
      bf16x8 af[2][TI], bfr[2][TJ];
      auto frags = [&](int ks, bf16x8 (&a)[TI], bf16x8 (&b)[TJ]) __attribute__((always_inline)) {
        const int ch = 2 * ks + lhalf;
#pragma unroll
        for (int ti = 0; ti < TI; ++ti) {
          const int r = wi * 128 + ti * 32 + lrow;
          a[ti] = *reinterpret_cast<const bf16x8*>(pa + r * kRowBytes + ((ch ^ swz(r)) << 4));
        }
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) {
          const int r = wj * 64 + tj * 32 + lrow;
          b[tj] = *reinterpret_cast<const bf16x8*>(qa + r * kRowBytes + ((ch ^ swz(r)) << 4));
        }
      };
      frags(0, af[0], bfr[0]);
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        if (ks + 1 < BK / 16) frags(ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
#pragma unroll
        for (int ti = 0; ti < TI; ++ti)
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj)
            acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][ti], bfr[ks & 1][tj],
                                                                  acc[ti][tj], 0, 0, 0);
      }
    } else {
#pragma unroll 4
      for (int ks = 0; ks < BK / 2; ++ks) {
        const int s = 2 * ks + lhalf;
        float af[TI], bfr[TJ];
#pragma unroll
        for (int ti = 0; ti < TI; ++ti) {
          const int r = wi * 128 + ti * 32 + lrow;
          af[ti] = *reinterpret_cast<const float*>(pa + r * kRowBytes +
                                                   (((s >> 2) ^ swz(r)) << 4) + (s & 3) * 4);
        }
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) {
          const int r = wj * 64 + tj * 32 + lrow;
          bfr[tj] = *reinterpret_cast<const float*>(qa + r * kRowBytes +
                                                    (((s >> 2) ^ swz(r)) << 4) + (s & 3) * 4);
        }
#pragma unroll
        for (int ti = 0; ti < TI; ++ti)
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj)
            acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[ti], bfr[tj], acc[ti][tj], 0, 0, 0);
      }
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  wg_accumulate<MODE>(acc, i0 + wi * 128, j0 + wj * 64, lrow, lhalf, e, out0, out1, ldo,
                      out_estride, i_store, j_store, store != 0);

  if (!do_bias) return;
  // Column sums: the partial of feature block fb from row block sb goes to
  // s_b[sb][feature]; then one thread per feature adds the 8 row blocks in
  // order.  The main loop ended with a barrier, so the LDS is free.
  float* s_b = reinterpret_cast<float*>(smem);
  if (op == 1) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int b = tt + 256 * nb;
      const int fb = b % FB, sb = b / FB;
#pragma unroll
      for (int c = 0; c < EPV; ++c) s_b[sb * 256 + fb * EPV + c] = bacc[nb][c];
    }
  }
  __syncthreads();
  if (tid < 256) {
    const int j = j0 + tid;
    float sum = 0.0f;
#pragma unroll
    for (int sb = 0; sb < BK / EPV; ++sb) sum += s_b[sb * 256 + tid];
    wg_bias_add<MODE>(sum, j, e, bias0, bias1, bias_estride, j_store, store != 0);
  }
}


// ---------------------------------------------------------------------------
// bf16: the operands go from HBM straight into LDS (global_load_lds, no
// registers) in their row-major layout, and the MFMA fragments are read
// with gfx950's transposing LDS read ds_read_b64_tr_b16.  Measured lane
// layout of that read: within each 16-lane group, output element q of lane
// i is element i%4 of the 8 bytes addressed by lane 4q + i/4.  So when lane
// 4q + r addresses row k0 + q, features m0 + 4r .. m0 + 4r + 3 of a
// [row][feature] tile, lane i receives feature m0 + i at rows k0 .. k0 + 3:
// two such reads give the 8 consecutive k of an MFMA operand.
//
// LDS: a ring of 4 stages of 32 rows (P rows, then Q rows; 512-byte rows of
// 256 features), filled 3 slabs ahead.  64-byte chunk c of row k sits at
// chunk c ^ (k & 3), so the 4 rows one read touches fall in distinct bank
// groups.  Rows past the expert's segment in the last slab are zeroed
// before use.
constexpr int kTrBK = 32;                         // rows per slab
constexpr int kTrStages = 4;
constexpr int kTrRowBytes = 512;                  // 256 bf16 features
constexpr int kTrOpBytes = kTrBK * kTrRowBytes;   // 16 KB
constexpr int kTrStageBytes = 2 * kTrOpBytes;

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

// One 1 KB direct-to-LDS load (lane l's 16 bytes land at lds + 16*l); the
// compiler does not track it, the kernel waits with tr_wait_barrier.
__device__ __forceinline__ void tr_dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}

// This wave's loads except the newest N have landed and its LDS accesses
// are complete; then meet the other waves.
template <int N>
__device__ __forceinline__ void tr_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

__device__ __forceinline__ bf16x8 tr_frag(const char* base, int kb, int c, int moff) {
  // rows kb .. kb+3 (first read) and kb+4 .. kb+7 (second); kb % 4 == 0
  const int k0 = kb, k1 = kb + 4;
  const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4s*)(base + k0 * kTrRowBytes + ((c ^ (k0 & 3)) << 6) + moff));
  const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4s*)(base + k1 * kTrRowBytes + ((c ^ (k1 & 3)) << 6) + moff));
  typedef short v8s __attribute__((ext_vector_type(8)));
  const v8s r = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, r);
}

template <int MODE>
__global__ __launch_bounds__(kThreads) void wgrad_tr_kernel(
    const bf16_t* __restrict__ P, int ldp, const bf16_t* __restrict__ Q, int ldq,
    const int32_t* __restrict__ counts, int E, int Iy, int Jx, int gy, int gx,
    float* __restrict__ out0, float* __restrict__ out1, int ldo, size_t out_estride, int i_store,
    int j_store, float* __restrict__ bias0, float* __restrict__ bias1, size_t bias_estride,
    int chunk_rows, float* __restrict__ part, float* __restrict__ bpart, int store) {
  __shared__ __attribute__((aligned(1024))) char smem[kTrStages * kTrStageBytes];
  const int tid = threadIdx.x;
  WgTile tl;
  if (!wg_locate(counts, E, chunk_rows, Iy, Jx, gy, gx, &tl)) return;
  const int seg0 = tl.seg0, cnt = tl.cnt, e = tl.e;
  const int i0 = tl.ty * kTI, j0 = tl.tx * kTJ;
  const bool do_bias = tl.ty == 0 && bias0 != nullptr;
  const int KT = (cnt + kTrBK - 1) / kTrBK;

  const int w = __builtin_amdgcn_readfirstlane(tid / kWave), lane = lane_id();
  // DMA role: waves 0-3 load P rows, waves 4-7 Q rows, 8 rows (4 x 1 KB) each
  const int op = w / 4, wl = w % 4;
  const bf16_t* src = op ? Q : P;
  const int ld = op ? ldq : ldp;
  const int f0 = op ? j0 : i0;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;
  const int slot = lane & 31;
  auto dma_slab = [&](int kt) __attribute__((always_inline)) {
    // past the last slab: repeat it (in bounds; the stage is never read)
    const int kk = kt < KT ? kt : KT - 1;
    const int s0 = seg0 + kk * kTrBK;
    const uint32_t base =
        lds0 + (uint32_t)((kt % kTrStages) * kTrStageBytes + op * kTrOpBytes + wl * 4096);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = wl * 8 + 2 * u + (lane >> 5);
      const int c = (slot >> 2) ^ (r & 3);
      const bf16_t* g = src + (size_t)(s0 + r) * ld + f0 + c * 32 + (slot & 3) * 8;
      tr_dma16(g, base + u * 1024);
    }
  };

  const int wi = w / 4, wj = w % 4;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int grp = lane >> 4, gl = lane & 15;
  // this lane's part of a transposing read: row offset and byte offset
  const int krow = 8 * (grp >> 1) + (gl >> 2);
  const int moff = (16 * (grp & 1) + 4 * (gl & 3)) * 2;
  constexpr int TI = 4, TJ = 2;
  f32x16 acc[TI][TJ];
#pragma unroll
  for (int a = 0; a < TI; ++a)
#pragma unroll
    for (int b = 0; b < TJ; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
  float bsum[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) bsum[q] = 0.0f;

  // Slab s becomes readable at its barrier: its DMA has landed, and every
  // wave has finished its reads of slab s - 1, whose stage then takes the
  // DMA of slab s + 3.  A slab's two 16-row k-steps are software-pipelined
  // across the barrier: the barrier of slab s + 1 sits between the MFMAs
  // of slab s's k-steps, so the fragment reads of slab s + 1 (issued just
  // after it) have the MFMAs of slab s's second k-step to hide their
  // latency instead of stalling behind the barrier.
  static_assert(kTrBK == 32, "two k-steps per slab");
  auto enter_slab = [&](int kt) __attribute__((always_inline)) {
    tr_wait_barrier<8>();
    const int valid = cnt - kt * kTrBK;
    if (valid < kTrBK) {
      // last slab: rows past the segment (other experts' rows or padding)
      // become zeros in both operands
      char* zs = smem + (kt % kTrStages) * kTrStageBytes;
      const int nz = (kTrBK - valid) * (kTrRowBytes / 16);   // 16-byte units per operand
      for (int u = tid; u < 2 * nz; u += kThreads) {
        const int o = u / nz, x = u % nz;
        *reinterpret_cast<uint4*>(zs + o * kTrOpBytes + valid * kTrRowBytes + x * 16) =
            make_uint4(0u, 0u, 0u, 0u);
      }
      __syncthreads();
    }
    dma_slab(kt + 3);   // into the stage of slab kt-1, which every wave has finished
    if (do_bias) {
      const char* qs = smem + (kt % kTrStages) * kTrStageBytes + kTrOpBytes;
      const int fb = tid & 31, c = fb >> 2, sub = fb & 3;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = (tid >> 5) + 16 * h;
        const uint4 v = *reinterpret_cast<const uint4*>(qs + r * kTrRowBytes +
                                                        ((c ^ (r & 3)) << 6) + sub * 16);
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bsum[2 * q] += __uint_as_float(wv[q] << 16);
          bsum[2 * q + 1] += __uint_as_float(wv[q] & 0xFFFF0000u);
        }
      }
    }
  };
  bf16x8 af[2][TI], bfr[2][TJ];
  auto frags = [&](int kt, int ks, bf16x8 (&a)[TI], bf16x8 (&b)[TJ]) __attribute__((always_inline)) {
    const char* ps = smem + (kt % kTrStages) * kTrStageBytes;
    const char* qs = ps + kTrOpBytes;
    const int kb = ks * 16 + krow;
#pragma unroll
    for (int ti = 0; ti < TI; ++ti) a[ti] = tr_frag(ps, kb, wi * 4 + ti, moff);
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj) b[tj] = tr_frag(qs, kb, wj * 2 + tj, moff);
  };
  auto mfmas = [&](const bf16x8 (&a)[TI], const bf16x8 (&b)[TJ]) __attribute__((always_inline)) {
#pragma unroll
    for (int ti = 0; ti < TI; ++ti)
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
        acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ti], b[tj], acc[ti][tj], 0, 0, 0);
  };
  dma_slab(0);
  dma_slab(1);
  dma_slab(2);
  enter_slab(0);
  frags(0, 0, af[0], bfr[0]);
  for (int kt = 0; kt < KT; ++kt) {
    frags(kt, 1, af[1], bfr[1]);
    mfmas(af[0], bfr[0]);
    if (kt + 1 < KT) {
      enter_slab(kt + 1);
      frags(kt + 1, 0, af[0], bfr[0]);
    }
    mfmas(af[1], bfr[1]);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the repeated tail loads

  if (tl.pslot < 0) {
    wg_accumulate<MODE>(acc, i0 + wi * 128, j0 + wj * 64, lrow, lhalf, e, out0, out1, ldo,
                        out_estride, i_store, j_store, store != 0);
  } else {
    // a later chunk: the whole 256 x 256 tile to its partial slot, [i][j]
    float* tp = part + ((size_t)tl.pslot * Iy * Jx + (size_t)tl.ty * Jx + tl.tx) * (kTI * kTJ);
#pragma unroll
    for (int ti = 0; ti < TI; ++ti)
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int li = wi * 128 + ti * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4);
          const int lj = wj * 64 + tj * 32 + lrow;
          tp[li * kTJ + lj] = acc[ti][tj][v];
        }
  }
  if (!do_bias) return;
  // Column sums: thread t holds features 8*(t%32) .. +7 of row group t/32;
  // one thread per feature then adds the 16 row groups in order.
  __syncthreads();   // every wave is done with the ring
  float* s_b = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int q = 0; q < 8; ++q) s_b[(tid >> 5) * 256 + (tid & 31) * 8 + q] = bsum[q];
  __syncthreads();
  if (tid < 256) {
    float sum = 0.0f;
    for (int g = 0; g < 16; ++g) sum += s_b[g * 256 + tid];
    if (tl.pslot < 0)
      wg_bias_add<MODE>(sum, j0 + tid, e, bias0, bias1, bias_estride, j_store, store != 0);
    else
      bpart[((size_t)tl.pslot * Jx + tl.tx) * kTJ + tid] = sum;
  }
}

// Adds the partial slots of every expert that was cut into chunks to its
// gradients, grad += (p_1 + p_2 + ...) in chunk order (chunk 0 accumulated
// or stored directly, before), so the result does not depend on which
// chunk finished first.
// Blocks b < 64 * Iy * Jx take 4 rows x 256 columns of tile b / 64, one
// float4 of 4 columns per thread; the Jx blocks after them take the bias
// columns of tile column b - 64 * Iy * Jx.  The chunking is recomputed from
// the counts exactly as wg_locate does it.
template <int MODE>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(
    const float* __restrict__ part, const float* __restrict__ bpart,
    const int32_t* __restrict__ counts, int E, int chunk_rows, int Iy, int Jx,
    float* __restrict__ out0, float* __restrict__ out1, int ldo, size_t out_estride, int i_store,
    int j_store, float* __restrict__ bias0, float* __restrict__ bias1, size_t bias_estride) {
  __shared__ int s_e[kWave], s_x0[kWave], s_n[kWave], s_ns;
  if (threadIdx.x < kWave) {
    const int l = lane_id();
    const int cnt = l < E ? counts[l] : 0;
    const int nch = cnt > 0 ? (cnt - 1) / chunk_rows + 1 : 0;
    const int xtra = nch > 0 ? nch - 1 : 0;
    const int x_incl = wave_incl_scan(xtra);
    const unsigned long long m = __ballot(xtra > 0);
    if (xtra > 0) {
      const int pos = __popcll(m & ((1ull << l) - 1ull));
      s_e[pos] = l;
      s_x0[pos] = x_incl - xtra;
      s_n[pos] = xtra;
    }
    if (l == 0) s_ns = __popcll(m);
  }
  __syncthreads();
  const int ns = s_ns;
  if (ns == 0) return;
  const int tiles = Iy * Jx;
  const int b = blockIdx.x;
  if (b < 64 * tiles) {
    const int tile = b / 64, ty = tile / Jx, tx = tile % Jx;
    const int li = (b % 64) * 4 + (int)threadIdx.x / 64;
    const int lj = ((int)threadIdx.x % 64) * 4;
    const int gi = ty * kTI + li;
    if (gi >= i_store) return;
    for (int q = 0; q < ns; ++q) {
      const int e = s_e[q], x0 = s_x0[q], n = s_n[q];
      float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      for (int c = 0; c < n; ++c) {
        const float4 v = *reinterpret_cast<const float4*>(
            part + ((size_t)(x0 + c) * tiles + tile) * (kTI * kTJ) + li * kTJ + lj);
        a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w;
      }
      // the 4 columns stay in one 32-column gate or up group, so they are
      // consecutive gradient entries: one float4 read-modify-write where the
      // row layout keeps them 16-byte aligned
      const int j = tx * kTJ + lj;
      float* ob;
      int col;
      if constexpr (MODE == 0) {
        ob = out0;
        col = j;
      } else {
        ob = ((j >> 5) & 1) ? out1 : out0;
        col = (j >> 6) * 32 + (j & 31);
      }
      float* o = ob + (size_t)e * out_estride + (size_t)gi * ldo + col;
      if (col + 3 < j_store && (reinterpret_cast<uintptr_t>(o) & 15) == 0) {
        float4 v = *reinterpret_cast<float4*>(o);
        v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
        *reinterpret_cast<float4*>(o) = v;
      } else {
        const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (col + t < j_store) o[t] = o[t] + av[t];
      }
    }
  } else {
    const int tx = b - 64 * tiles;
    if (!bias0 || tx >= Jx) return;
    for (int q = 0; q < ns; ++q) {
      const int e = s_e[q], x0 = s_x0[q], n = s_n[q];
      float sum = 0.0f;
      for (int c = 0; c < n; ++c) sum += bpart[((size_t)(x0 + c) * Jx + tx) * kTJ + threadIdx.x];
      wg_bias_add<MODE>(sum, tx * kTJ + (int)threadIdx.x, e, bias0, bias1, bias_estride, j_store);
    }
  }
}

// Zeroes the gradient slices of the experts that have no rows: expert e's
// slice of piece p is base[p] + e * len[p] .. + len[p].  Blocks (x, e); the
// experts with rows return at once.
__global__ __launch_bounds__(256) void zero_idle_experts_kernel(const int32_t* __restrict__ counts,
                                                                IdleSlices z) {
  const int e = blockIdx.y;
  if (counts[e] != 0) return;
  const size_t step = (size_t)gridDim.x * blockDim.x;
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int p = 0; p < z.n; ++p) {
    float* b = z.base[p] + (size_t)e * z.len[p];
    const size_t n = z.len[p];
    // scalar head up to 16-byte alignment, float4 body, scalar tail
    const size_t head = std::min(n, (size_t)((16 - (reinterpret_cast<uintptr_t>(b) & 15)) & 15) / 4);
    if (t0 < head) b[t0] = 0.0f;
    float4* b4 = reinterpret_cast<float4*>(b + head);
    const size_t n4 = (n - head) / 4;
    for (size_t i = t0; i < n4; i += step) b4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const size_t tail = head + 4 * n4;
    if (tail + t0 < n) b[tail + t0] = 0.0f;
  }
}

// n floats of p (16-byte aligned) set to zero: a kernel, so that a HIP graph
// captures a kernel node and not a memset node.
__global__ __launch_bounds__(256) void fill_zero_kernel(float4* __restrict__ p, size_t n4,
                                                        float* __restrict__ tail, int ntail) {
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (size_t i = t0; i < n4; i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (t0 < (size_t)ntail) tail[t0] = 0.0f;
}

}  // namespace

hipError_t launch_fill_zero(float* p, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  if ((reinterpret_cast<uintptr_t>(p) & 15) != 0) return hipErrorInvalidValue;
  const size_t n4 = n / 4;
  const size_t want = (n4 + 255) / 256;
  const int blocks = (int)std::max<size_t>(1, std::min<size_t>(want, 2048));
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream,
                     reinterpret_cast<float4*>(p), n4, p + 4 * n4, (int)(n - 4 * n4));
  return hipGetLastError();
}

// The store-mode companion of launch_wgrad: clears the slices of every
// expert with counts[e] == 0, which the weight-gradient launches leave as
// they were.
hipError_t launch_zero_idle_experts(const int32_t* counts, int E, const IdleSlices& z,
                                    hipStream_t stream) {
  if (E <= 0 || E > kMaxExpertsWide || z.n < 0 || z.n > IdleSlices::kMax)
    return hipErrorInvalidValue;
  if (z.n == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_idle_experts_kernel, dim3(256, E), dim3(256), 0, stream, counts, z);
  return hipGetLastError();
}

// D_e = P_e^T . Q_e accumulated into out (fp32) for every expert with rows:
// P [rows][ldp] with p_valid valid columns (the i dimension), Q [rows][ldq]
// with q_valid valid columns (j); rows of expert e are the counts-defined
// segment.  MODE 0: out0[e][i][j] (i < i_store, j < j_store); MODE 1: the
// j columns are gate/up interleaved and go to out0 (gate) / out1 (up) at
// column h (h < j_store).  bias0/bias1 (nullable) receive the column sums
// of Q the same way.  With `store` the gradients are taken to be zero
// and are written instead of read and added (experts without rows are not
// touched: launch_zero_idle_experts clears them).  p_valid and q_valid must
// be multiples of 8 (bf16) or 4 (fp32); ldp, ldq likewise, and P, Q 16-byte
// aligned.
template <typename T, int MODE>
hipError_t launch_wgrad(const T* P, int ldp, int p_valid, const T* Q, int ldq, int q_valid, const int32_t* counts, int E, float* out0, float* out1,
                        int ldo, size_t out_estride, int i_store, int j_store, float* bias0,
                        float* bias1, size_t bias_estride, int rows_total, float* part,
                        size_t part_bytes, float* bpart, size_t bpart_bytes, int num_cus,
                        bool store, hipStream_t stream) {
  constexpr int EPV = WgT<T>::EPV;
  if (E <= 0 || E > kMaxExpertsWide || p_valid % EPV || q_valid % EPV || ldp % EPV || ldq % EPV ||
      (reinterpret_cast<uintptr_t>(P) & 15) || (reinterpret_cast<uintptr_t>(Q) & 15) ||
      rows_total < 0 || (reinterpret_cast<uintptr_t>(part) & 15))
    return hipErrorInvalidValue;
  if (i_store <= 0 || q_valid <= 0) return hipSuccess;
  const int Iy = (i_store + kTI - 1) / kTI, Jx = (q_valid + kTJ - 1) / kTJ;
  const int gx = Jx < 4 ? Jx : 4, gy = 16 / gx;
  const int ng = ((Iy + gy - 1) / gy) * ((Jx + gx - 1) / gx);
  // Rows per chunk: about one CU's share of the whole contraction
  // (tiles x rows / CUs, at least kMinChunkRows, a multiple of the 32-row
  // slab), so that no tile's contraction is much longer than the average
  // CU's work while the partial tiles stay few: at most rows/chunk_rows <=
  // num_cus / tiles slots of 256 KB, num_cus x 256 KB in all.  bf16 only,
  // and only with a partial workspace that holds them; at most 64 chunks in
  // all (one lane each).
  constexpr long kMinChunkRows = 1024;
  int chunk_rows = INT_MAX, slots = 0;
  const long tiles = (long)Iy * Jx;
  if (sizeof(T) == 2 && part && bpart && E < 64 && num_cus > 0 && rows_total > 0) {
    long r = (tiles * rows_total + num_cus - 1) / num_cus;
    r = std::max(r, kMinChunkRows);
    r = std::max(r, ((long)rows_total + (63 - E)) / (64 - E));   // E + rows/r <= 64
    r = (r + 31) / 32 * 32;
    const long sl = rows_total / r;   // bound on the extra chunks over all experts
    if (r < INT_MAX && sl > 0 && (size_t)sl * tiles * kTI * kTJ * 4 <= part_bytes &&
        (size_t)sl * Jx * kTJ * 4 <= bpart_bytes) {
      chunk_rows = (int)r;
      slots = (int)sl;
    }
  }
  const int groups = (E + slots) * ng;
  const int blocks = 16 * kNumXcd * ((groups + kNumXcd - 1) / kNumXcd);
  if constexpr (sizeof(T) == 2) {
    hipLaunchKernelGGL((wgrad_tr_kernel<MODE>), dim3(blocks), dim3(kThreads), 0, stream, P, ldp,
                       Q, ldq, counts, E, Iy, Jx, gy, gx, out0, out1, ldo, out_estride, i_store,
                       j_store, bias0, bias1, bias_estride, chunk_rows, part, bpart, (int)store);
    if (slots > 0)
      hipLaunchKernelGGL((wgrad_reduce_kernel<MODE>), dim3((unsigned)(64 * tiles + Jx)), dim3(256),
                         0, stream, part, bpart, counts, E, chunk_rows, Iy, Jx, out0, out1, ldo,
                         out_estride, i_store, j_store, bias0, bias1, bias_estride);
  } else {
    hipLaunchKernelGGL((wgrad_kernel<T, MODE>), dim3(blocks), dim3(kThreads), 0, stream, P, ldp,
                       p_valid, Q, ldq, q_valid, counts, E, Iy, Jx, gy, gx, out0, out1, ldo,
                       out_estride, i_store, j_store, bias0, bias1, bias_estride, (int)store);
  }
  return hipGetLastError();
}

#define MGPT_INST_WGRAD(T, MODE)                                                             \
  template hipError_t launch_wgrad<T, MODE>(const T*, int, int, const T*, int, int,           \
                                            const int32_t*, int, float*, float*, int, size_t, \
                                            int, int, float*, float*, size_t, int, float*,     \
                                            size_t, float*, size_t, int, bool, hipStream_t);
MGPT_INST_WGRAD(bf16_t, 0)
MGPT_INST_WGRAD(bf16_t, 1)
MGPT_INST_WGRAD(float, 0)
MGPT_INST_WGRAD(float, 1)

}  // namespace mgpt
