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
#include "common.hpp"

namespace mgpt {
namespace {

constexpr int kTI = 256, kTJ = 256;   // output tile
constexpr int kThreads = 512;         // 8 waves: 2 (i) x 4 (j), 128 x 64 each
constexpr int kRowBytes = 128;        // LDS row: one feature's slab of rows
constexpr int kOpBytes = 256 * kRowBytes;   // one operand tile (32 KB)

template <typename T> struct WgT;
template <> struct WgT<bf16_t> { static constexpr int BK = 64, EPV = 8; };
template <> struct WgT<float> { static constexpr int BK = 32, EPV = 4; };

// 16-byte chunk c of LDS row r sits at slot c ^ swz(r).  (r >> 1) spreads
// the 16 consecutive rows a fragment read serves together over all eight
// slots of both bank halves; (r >> 4) spreads the rows 8 apart that one
// transposed-block write covers.
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 4)) & 7; }

typedef __attribute__((address_space(3))) char lds_char;

template <typename T, int MODE>
__global__ __launch_bounds__(kThreads) void wgrad_kernel(
    const T* __restrict__ P, int ldp, int p_valid, const T* __restrict__ Q, int ldq, int q_valid,
    const int32_t* __restrict__ counts, int E, float* __restrict__ out0,
    float* __restrict__ out1, int ldo, size_t out_estride, int i_store, int j_store,
    float* __restrict__ bias0, float* __restrict__ bias1, size_t bias_estride) {
  constexpr int BK = WgT<T>::BK, EPV = WgT<T>::EPV;
  constexpr int NB = (BK / EPV) * (256 / EPV) / 256;   // transposed blocks per thread
  constexpr int FB = 256 / EPV;                        // feature blocks per tile
  constexpr bool kBf = sizeof(T) == 2;
  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * kOpBytes];
  __shared__ int s_seg[2];

  const int e = blockIdx.z;
  const int tid = threadIdx.x;
  if (tid < kWave) {
    const int l = lane_id();
    const int cnt = l < E ? counts[l] : 0;
    const int incl = wave_incl_scan(cnt);
    if (l == e) {
      s_seg[0] = incl - cnt;
      s_seg[1] = cnt;
    }
  }
  __syncthreads();
  const int seg0 = s_seg[0], cnt = s_seg[1];
  if (cnt == 0) return;   // block-uniform: an unchosen expert gets no gradient
  const int seg_end = seg0 + cnt;
  const int i0 = blockIdx.y * kTI, j0 = blockIdx.x * kTJ;
  const bool do_bias = blockIdx.y == 0 && bias0 != nullptr;

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

  // Accumulate: register v of tile (ti, tj) is D[i][j] with
  // i = 8*(v/4) + 4*lhalf + v%4 and j = lrow inside the tile.
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    const int j = j0 + wj * 64 + tj * 32 + lrow;
    float* ob;
    int col;
    bool jok;
    if constexpr (MODE == 0) {
      ob = out0;
      col = j;
      jok = j < j_store;
    } else {
      // gate/up interleaved columns: 32 gate, then 32 up, per 32 units
      ob = ((j >> 5) & 1) ? out1 : out0;
      col = (j >> 6) * 32 + (j & 31);
      jok = col < j_store;
    }
    if (!jok) continue;
    ob += (size_t)e * out_estride + col;
#pragma unroll
    for (int ti = 0; ti < TI; ++ti)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = i0 + wi * 128 + ti * 32 + 8 * (v / 4) + 4 * lhalf + (v % 4);
        if (i < i_store) {
          float* o = ob + (size_t)i * ldo;
          *o = *o + acc[ti][tj][v];
        }
      }
  }

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
      *o = *o + sum;
    }
  }
}

}  // namespace

// D_e = P_e^T . Q_e accumulated into out (fp32) for every expert with rows:
// P [rows][ldp] with p_valid valid columns (the i dimension), Q [rows][ldq]
// with q_valid valid columns (j); rows of expert e are the counts-defined
// segment.  MODE 0: out0[e][i][j] (i < i_store, j < j_store); MODE 1: the
// j columns are gate/up interleaved and go to out0 (gate) / out1 (up) at
// column h (h < j_store).  bias0/bias1 (nullable) receive the column sums
// of Q the same way.  p_valid and q_valid must be multiples of 8 (bf16) or
// 4 (fp32); ldp, ldq likewise, and P, Q 16-byte aligned.
template <typename T, int MODE>
hipError_t launch_wgrad(const T* P, int ldp, int p_valid, const T* Q, int ldq, int q_valid, const int32_t* counts, int E, float* out0, float* out1,
                        int ldo, size_t out_estride, int i_store, int j_store, float* bias0,
                        float* bias1, size_t bias_estride, hipStream_t stream) {
  constexpr int EPV = WgT<T>::EPV;
  if (E <= 0 || E > kMaxExperts || p_valid % EPV || q_valid % EPV || ldp % EPV || ldq % EPV ||
      (reinterpret_cast<uintptr_t>(P) & 15) || (reinterpret_cast<uintptr_t>(Q) & 15))
    return hipErrorInvalidValue;
  if (i_store <= 0 || q_valid <= 0) return hipSuccess;
  const dim3 grid((q_valid + kTJ - 1) / kTJ, (i_store + kTI - 1) / kTI, E);
  hipLaunchKernelGGL((wgrad_kernel<T, MODE>), grid, dim3(kThreads), 0, stream, P, ldp, p_valid, Q,
                     ldq, q_valid, counts, E, out0, out1, ldo, out_estride, i_store, j_store,
                     bias0, bias1, bias_estride);
  return hipGetLastError();
}

#define MGPT_INST_WGRAD(T, MODE)                                                             \
  template hipError_t launch_wgrad<T, MODE>(const T*, int, int, const T*, int, int,           \
                                            const int32_t*, int, float*, float*, int, size_t, \
                                            int, int, float*, float*, size_t, hipStream_t);
MGPT_INST_WGRAD(bf16_t, 0)
MGPT_INST_WGRAD(bf16_t, 1)
MGPT_INST_WGRAD(float, 0)
MGPT_INST_WGRAD(float, 1)

}  // namespace mgpt
