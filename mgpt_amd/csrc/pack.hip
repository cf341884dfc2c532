// pack.hip -- weight packing: reference layout fp32 -> GEMM layouts.
//
// The reference stores a Linear weight as W[in][out] row-major
// (layers/LinearLayer.cpp:15-21).  The grouped GEMMs want each output
// channel's K-run contiguous (B[n][k]), so the weights are transposed once
// at load time through 64x64 LDS tiles (coalesced on both sides), converted
// to the compute type, and, for gate/up, interleaved in 64-row groups
// [32 gate rows | 32 up rows] of the same 32 hidden units.  fp8 weights are
// first packed as fp32 and then quantised row by row: per output channel,
// scale = amax / 448 (1 for an all-zero channel) and q = e4m3(w / scale),
// round-to-nearest-even, saturating at +-448, zero encoded as +0.
#include <algorithm>

#include "common.hpp"

namespace mgpt {
namespace {

__device__ __forceinline__ void put(float* p, float v) { *p = v; }
__device__ __forceinline__ void put(bf16_t* p, float v) { *p = f32_to_bf16(v); }

// dst row of source column n: gate/up interleave (mode 1) or identity (0).
__device__ __forceinline__ int dst_row(int n, int mode, int off) {
  return mode ? (n / 32) * 64 + (n % 32) + off : n;
}

// src [Kin][Nout] fp32 (leading dim Nout) -> dst[dst_row(n)][k] (leading dim ldd).
template <typename DT>
__global__ __launch_bounds__(256) void pack_transpose_kernel(const float* __restrict__ src, int Kin,
                                                             int Nout, DT* __restrict__ dst,
                                                             int ldd, int mode, int off) {
  __shared__ float tile[64][65];
  const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  for (int r = ty; r < 64; r += 4) {
    const int k = k0 + r, n = n0 + tx;
    tile[r][tx] = (k < Kin && n < Nout) ? src[(size_t)k * Nout + n] : 0.0f;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int n = n0 + r, k = k0 + tx;
    if (n < Nout && k < Kin) put(dst + (size_t)dst_row(n, mode, off) * ldd + k, tile[tx][r]);
  }
}

// OCP E4M3FN encode, nearest-even, saturating to 448.
__device__ __forceinline__ uint8_t f32_to_e4m3(float v) {
  const uint32_t sign = (__float_as_uint(v) >> 31) & 1u;
  const float a = fabsf(v);
  uint32_t code;
  if (!(a < 448.0f)) {
    code = 0x7E;
  } else if (a < 0x1p-6f) {
    code = (uint32_t)rintf(a * 512.0f);          // subnormal grid m * 2^-9 (m = 8 is 2^-6)
  } else {
    uint32_t b = __float_as_uint(a);
    uint32_t q = b >> 20;                          // exponent + top 3 mantissa bits
    const uint32_t rem = b & 0xFFFFFu;
    q += (rem > 0x80000u) || (rem == 0x80000u && (q & 1u));
    const int ex = (int)(q >> 3) - 127 + 7;
    code = ((uint32_t)ex << 3) | (q & 7u);
    if (code > 0x7E) code = 0x7E;
  }
  return (uint8_t)(code | ((sign && code) ? 0x80u : 0u));
}

// Row-wise quantisation of src [rows][K] fp32 -> q [rows][K] e4m3, scale[rows].
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ src, int K,
                                                            uint8_t* __restrict__ q,
                                                            float* __restrict__ scale) {
  __shared__ float s_red[4];
  const size_t r = blockIdx.x;
  const float* row = src + r * K;
  float m = 0.0f;
  for (int k = threadIdx.x; k < K; k += 256) m = fmaxf(m, fabsf(row[k]));
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, kWave));
  if (lane_id() == 0) s_red[threadIdx.x / kWave] = m;
  __syncthreads();
  const float amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
  for (int k = threadIdx.x; k < K; k += 256) q[r * K + k] = f32_to_e4m3(row[k] / s);
  if (threadIdx.x == 0) scale[r] = s;
}

// dst[i][0..n) = src[i][0..n), zero elsewhere up to ldd (bias padding).
__global__ void pad_rows_kernel(const float* __restrict__ src, int n, float* __restrict__ dst,
                                int ldd) {
  const int i = threadIdx.x + blockIdx.x * blockDim.x;
  if (i < ldd) dst[i] = i < n ? src[i] : 0.0f;
}

// Router weights W_r [Cx][E] -> [G][C][RE] (G = ceil(E/RE)), zero-padded
// over the experts past E and the columns c >= Cx of a padded width C.
__global__ void pack_router_kernel(const float* __restrict__ wr, int Cx, int C, int E, int RE,
                                   float* __restrict__ out, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int j = i % RE, c = (i / RE) % C, g = i / (RE * C);
  const int e = g * RE + j;
  out[i] = (e < E && c < Cx) ? wr[(size_t)c * E + e] : 0.0f;
}

// dst[r][0..ncopy) = src[r][0..ncopy), dst[r][ncopy..nfill) = 0: a row block
// moved between a caller's width and the library's zero-padded width.
template <typename T>
__global__ __launch_bounds__(256) void copy_cols_kernel(const T* __restrict__ src, int lds,
                                                        T* __restrict__ dst, int ldd, int ncopy,
                                                        int nfill, int rows) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= nfill) return;
  for (size_t r = blockIdx.y; r < (size_t)rows; r += gridDim.y)
    dst[r * ldd + c] = c < ncopy ? src[r * lds + c] : T(0);
}

// fp8 weights [E][Npad][K] -> the decode stream's tiles
// [E][Npad/256][K/128][256][128]: every 256-row x 128-column stage the decode
// GEMM loads is one contiguous 32 KB block.  One thread per 16-byte chunk.
__global__ __launch_bounds__(256) void tile_fp8_kernel(const uint4* __restrict__ src, int Npad,
                                                       int K, size_t chunks,
                                                       uint4* __restrict__ dst) {
  const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= chunks) return;
  const size_t row_chunks = (size_t)K / 16;
  const size_t row = q / row_chunks;               // e * Npad + n
  const int c16 = (int)(q % row_chunks);
  const size_t e = row / Npad;
  const int n = (int)(row % Npad);
  const int KT = K / 128;
  const size_t tile = (e * (size_t)(Npad / 256) + n / 256) * KT + c16 / 8;
  dst[(tile * 256 + n % 256) * 8 + c16 % 8] = src[q];
}

// dst_j[r][c] += src[off_j + r * lds_j + c]: the handle's gradients added
// into the caller's (Tensor::add_grad, one rounded add per element), a batch
// of tensors per launch (blockIdx.y = tensor).
__global__ __launch_bounds__(256) void add_jobs_kernel(const float* __restrict__ src,
                                                       AddJobs jobs) {
  const int j = blockIdx.y;
  const int cols = jobs.cols[j];
  const size_t total = (size_t)jobs.rows[j] * cols;
  float* __restrict__ dst = jobs.dst[j];
  const float* __restrict__ s = src + jobs.off[j];
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const size_t r = i / cols, c = i % cols;
    dst[i] = dst[i] + s[r * jobs.lds[j] + c];
  }
}

}  // namespace

hipError_t launch_add_jobs(const float* src, const AddJobs& jobs, size_t max_elems,
                           hipStream_t stream) {
  if (jobs.n <= 0) return hipSuccess;
  const unsigned gx = (unsigned)std::min<size_t>((max_elems + 255) / 256, 1024);
  hipLaunchKernelGGL(add_jobs_kernel, dim3(std::max(gx, 1u), jobs.n), dim3(256), 0, stream, src,
                     jobs);
  return hipGetLastError();
}

hipError_t launch_tile_fp8(const uint8_t* src, int E, int Npad, int K, uint8_t* dst,
                           hipStream_t stream) {
  if (Npad % 256 != 0 || K % 128 != 0) return hipErrorInvalidValue;
  const size_t chunks = (size_t)E * Npad * (K / 16);
  hipLaunchKernelGGL(tile_fp8_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream,
                     reinterpret_cast<const uint4*>(src), Npad, K, chunks,
                     reinterpret_cast<uint4*>(dst));
  return hipGetLastError();
}

// RE experts per wave group; the fused router uses router_experts_per_wave(E),
// the split decode path RE = 1 (W_r transposed).
// Cx <= C: the caller's width; columns past it are zero.
hipError_t launch_pack_router(const float* wr, int Cx, int C, int E, int RE, float* out,
                              hipStream_t stream) {
  const int total = ((E + RE - 1) / RE) * C * RE;
  hipLaunchKernelGGL(pack_router_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, wr, Cx,
                     C, E, RE, out, total);
  return hipGetLastError();
}

// W_r [Cx][E] -> column quads [C/4][E][4] (zero past Cx): expert e's
// columns 4q .. 4q+3 are one 16-byte entry, and the E entries of a quad are
// contiguous.
__global__ void pack_router_quads_kernel(const float* __restrict__ wr, int Cx, int C, int E,
                                         float* __restrict__ out, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int r = i % 4, e = (i / 4) % E, c = (i / (4 * E)) * 4 + r;
  out[i] = c < Cx ? wr[(size_t)c * E + e] : 0.0f;
}

hipError_t launch_pack_router_quads(const float* wr, int Cx, int C, int E, float* out,
                                    hipStream_t stream) {
  if (C % 4) return hipErrorInvalidValue;
  const int total = C * E;
  hipLaunchKernelGGL(pack_router_quads_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, wr,
                     Cx, C, E, out, total);
  return hipGetLastError();
}

// rows x nfill block: copy ncopy columns, zero the rest (pad), or copy
// ncopy = nfill columns of a wider source (unpad).
template <typename T>
hipError_t launch_copy_cols(const T* src, int lds, T* dst, int ldd, int rows, int ncopy, int nfill,
                            hipStream_t stream) {
  if (rows <= 0 || nfill <= 0) return hipSuccess;
  hipLaunchKernelGGL(copy_cols_kernel<T>, dim3((nfill + 255) / 256, std::min(rows, 16384)),
                     dim3(256), 0, stream, src, lds, dst, ldd, ncopy, nfill, rows);
  return hipGetLastError();
}
template hipError_t launch_copy_cols<float>(const float*, int, float*, int, int, int, int,
                                            hipStream_t);
template hipError_t launch_copy_cols<bf16_t>(const bf16_t*, int, bf16_t*, int, int, int, int,
                                             hipStream_t);

template <typename DT>
hipError_t launch_pack_transpose(const float* src, int Kin, int Nout, DT* dst, int ldd, int mode,
                                 int off, hipStream_t stream) {
  dim3 grid((Nout + 63) / 64, (Kin + 63) / 64);
  hipLaunchKernelGGL(pack_transpose_kernel<DT>, grid, dim3(256), 0, stream, src, Kin, Nout, dst,
                     ldd, mode, off);
  return hipGetLastError();
}
template hipError_t launch_pack_transpose<float>(const float*, int, int, float*, int, int, int,
                                                 hipStream_t);
template hipError_t launch_pack_transpose<bf16_t>(const float*, int, int, bf16_t*, int, int, int,
                                                  hipStream_t);

hipError_t launch_quantize_rows(const float* src, int rows, int K, uint8_t* q, float* scale,
                                hipStream_t stream) {
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(rows), dim3(256), 0, stream, src, K, q, scale);
  return hipGetLastError();
}

hipError_t launch_pad_row(const float* src, int n, float* dst, int ldd, hipStream_t stream) {
  hipLaunchKernelGGL(pad_rows_kernel, dim3((ldd + 255) / 256), dim3(256), 0, stream, src, n, dst,
                     ldd);
  return hipGetLastError();
}

}  // namespace mgpt
