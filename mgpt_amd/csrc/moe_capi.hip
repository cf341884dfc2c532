// moe_capi.hip -- the C ABI (include/mgpt_moe.h): handle, parameter packing,
// workspace layout, the forward pipeline and the backward pipeline.
//
// Forward = 6 stream-ordered launches and no host synchronisation:
//   router+top-k -> per-expert scan -> permute -> gate/up GEMM (+SwiGLU)
//   -> down GEMM -> combine.
// The reference's blocking device-to-host copy of the expert counts and the
// host prefix sum (layers/MoELayer.cpp:61-80) are replaced by device-side
// scans; the per-expert host loop of GEMM launches (:94-118) by one grouped
// launch per projection.
//
// Backward (layers/MoELayer.cpp:130-223) = 8 launches, again without host
// synchronisation: scatter backward -> d(act) product with the SwiGLU
// backward in its epilogue -> dX product -> down and gate/up weight
// gradients (with their bias sums) -> per-token gather + softmax + router
// backward -> router weight gradient (partials + in-order reduction).  It
// reads what the training forward kept in the workspace: the routing, the
// gathered rows, h, the expert outputs, the router probabilities and the
// gate/up pre-activations.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <mutex>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/mgpt_moe.h"
#include "capi_internal.hpp"
#include "common.hpp"

namespace mgpt {
// kernels (router.hip, dispatch.hip, gemm.hip, combine.hip, pack.hip)
template <typename ActT>
hipError_t launch_router(const ActT*, const float*, const float*, const float*, const float*, int,
                         int, int, int, int32_t*, float*, int32_t*, float*, float*, const float*,
                         float, int, float*, hipStream_t);
hipError_t launch_expf_probe(const float*, float*, int, hipStream_t);
template <typename InT, typename ActT>
hipError_t launch_permute(const InT*, const int32_t*, const int32_t*, int32_t*, int, int, int,
                          int, int32_t*, int32_t*, int32_t*, ActT*, const float*, const float*,
                          hipStream_t);
template <typename ActT, typename OutT>
hipError_t launch_combine(const ActT*, const int32_t*, const float*, const int32_t*, int, int, int,
                          const OutT*, OutT*, hipStream_t);
template <typename T>
hipError_t launch_copy_cols(const T*, int, T*, int, int, int, int, hipStream_t);
hipError_t launch_add_jobs(const float*, const AddJobs&, size_t, hipStream_t);
template <int BM, int BN, int WM, int WN, typename AT, typename WT, int EPI, typename OutT>
hipError_t launch_grouped_gemm(const AT*, const WT*, const float*, const float*, const float*,
                               const int32_t*, int, int, int, int, int, OutT*, int, int, OutT*,
                               int, hipStream_t, float* partials = nullptr, int split_slots = 0);
template <typename DT>
hipError_t launch_pack_transpose(const float*, int, int, DT*, int, int, int, hipStream_t);
hipError_t launch_quantize_rows(const float*, int, int, uint8_t*, float*, hipStream_t);
hipError_t launch_pad_row(const float*, int, float*, int, hipStream_t);
template <typename XT>
hipError_t launch_gemm_decode_gather(const XT*, const fp8_t*, const float*, const float*,
                                     const float*, const int32_t*, int, int, int, int, int, int,
                                     int, bf16_t*, int, int, int32_t*, int32_t*, int32_t*,
                                     hipStream_t);
hipError_t launch_pack_router(const float*, int, int, int, int, float*, hipStream_t);
hipError_t launch_pack_router_quads(const float*, int, int, int, float*, hipStream_t);
template <int EPI>
hipError_t launch_gemm_dma(const bf16_t*, const bf16_t*, const float*, const float*,
                           const int32_t*, int, int, int, int, int, bf16_t*, int, int, float*, int,
                           bf16_t*, int, hipStream_t);
// backward (backward.hip, wgrad.hip)
template <typename ActT>
hipError_t launch_scatter_bwd(const ActT*, const ActT*, const int32_t*, const float*, int, int,
                              int, ActT*, float*, hipStream_t);
template <typename ActT>
hipError_t launch_token_bwd(const ActT*, const int32_t*, const int32_t*, const float*,
                            const float*, const int32_t*, const float*, int, int, int, int, ActT*,
                            float*, hipStream_t);
int router_wgrad_chunks(int N);
template <typename ActT>
hipError_t launch_router_wgrad(const ActT*, const float*, int, int, int, float*, float*, float*,
                               float*, bool, const float*, const float*, hipStream_t);
int rmsnorm_bwd_blocks(int N);
template <typename ActT>
hipError_t launch_rmsnorm_bwd(const ActT*, ActT*, const ActT*, const float*, const float*, int,
                              int, float*, float*, hipStream_t);
template <typename T>
hipError_t launch_transpose_pad(const T*, int, int, size_t, T*, int, int, size_t, int,
                                hipStream_t);
template <typename T, int MODE>
hipError_t launch_wgrad(const T*, int, int, const T*, int, int, const int32_t*, int, float*,
                        float*, int, size_t, int, int, float*, float*, size_t, int, float*,
                        size_t, float*, size_t, int, bool, hipStream_t);
hipError_t launch_zero_idle_experts(const int32_t*, int, const IdleSlices&, hipStream_t);
hipError_t launch_fill_zero(float* p, size_t n, hipStream_t stream);
hipError_t launch_tile_fp8(const uint8_t*, int, int, int, uint8_t*, hipStream_t);
template <int EPI>
hipError_t launch_gemm_decode(const bf16_t*, const fp8_t*, const float*, const float*,
                              const float*, const int32_t*, int, int, int, int, int, bf16_t*, int,
                              int, hipStream_t);
}  // namespace mgpt

namespace mgpt {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

}  // namespace mgpt

using namespace mgpt;

namespace {

#define HIP_TRY(expr)                                                                  \
  do {                                                                                 \
    hipError_t _e = (expr);                                                            \
    if (_e != hipSuccess)                                                              \
      return fail(MGPT_ERR_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), \
                  __FILE__, __LINE__);                                                 \
  } while (0)

constexpr size_t kAlign = 256;
constexpr size_t kGemmPartialBytes = 512 * 128 * 4;   // one 256x256 fp32 tile
// fp32 handles: one 64x128 fp32 partial tile per CU for the split-K down
// product of small token counts (a fixed size, so the workspace stays
// monotonic in N)
constexpr size_t kF32PartialBytes = 64 * 128 * 4;
constexpr int kRowPad = 256;   // rows of slack after activation buffers (GEMM tile overrun)

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
int round_up(int v, int m) { return (v + m - 1) / m * m; }

struct Layout {
  size_t topk_idx, topk_p, slot_of, perm, hist, base, counts, logits, xg, hbuf, obuf, partials;
  size_t rstd;   // fused block: 1/rms of each token [N] f32
  // a caller width Cx that is not a multiple of 64: x and y at the padded
  // width C (boundary dtype), and the fused block's gamma [C] f32
  size_t xpad, ypad, gpad;
  // training only (after the forward regions, so those keep their offsets):
  // router probabilities [N][E] f32, gate/up pre-activations (then their
  // gradients) [A+pad][2Hp], dgo [A+pad][C], d(top-k p) [A] f32,
  // d(logits) [N][E] f32, router weight-gradient partials, and the bias
  // partials of the expert weight gradients' row chunks (their tile
  // partials reuse the split-K partial region)
  size_t probs, gu, dgo, dtp, dlog, rw_part, rw_part_b, wg_bpart;
  // the gate/up weight gradient's row-chunk partials while it runs beside
  // the dX product (which holds the split-K region)
  size_t wg_part2;
  size_t dypad, dxpad;   // padded width: dy and dx at width C
  size_t nrm_part;       // fused block backward: ln2 scale-gradient partials
  size_t total;
};

// The workspace of mgpt_moe_forward_noalloc: one array per device, part of
// the library's code object (no allocation call ever makes it), held until
// the process ends.  Host code never passes its name to a kernel or a copy:
// it uses the device address hipGetSymbolAddress returns for the current
// device (scratch_address below).
static __device__ __align__(256) char scratch[MGPT_MOE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device`, looked up once per device with
// that device current (mgpt_moe_create does it for the handle's device, so
// the noalloc forward only reads the cached address).
int scratch_address(int device, void** out) {
  if (device < 0 || device >= kMaxDevices)
    return fail(MGPT_ERR_UNSUPPORTED, "device %d beyond the %d the library tracks", device,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    int cur = -1;
    HIP_TRY(hipGetDevice(&cur));
    if (cur != device) HIP_TRY(hipSetDevice(device));
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != device) (void)hipSetDevice(cur);
    if (e != hipSuccess || !ptr)
      return fail(MGPT_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return MGPT_OK;
}

}  // namespace

struct mgpt_moe {
  // C: the width every kernel works at, the caller's embed_dim Cx rounded up
  // to a multiple of 64 (zero columns: weights, padded rows and gradients
  // carry zeros there, so routing and outputs are those of width Cx).
  int C, H, E, k, Hp, Cp;
  int Cx;
  // io: dtype of the caller's x, y, dx, dy; act: dtype of the gathered rows,
  // h and the expert outputs (bf16 whenever the weights are bf16 or fp8);
  // wdt: the packed expert weights.
  int io, act, wdt;
  int device;
  int num_cus = 0;         // compute units of the device (persistent grids)
  int gemm_tile = 256;     // block tile of the large-M bf16 GEMMs (256 or 128)
  float* wr_g = nullptr;   // router weights [G][C][RE] (router_experts_per_wave)
  float* wr1 = nullptr;    // router weights [E][C] (split decode router, E > 16)
  float* wr4 = nullptr;    // router weights [C/4][E][4] (one-launch decode router, E > 16)
  float* br = nullptr;     // [E]
  void* wgu = nullptr;     // [E][2Hp][C] of bf16 / fp8 / f32
  void* wd = nullptr;      // [E][Cp][Hp]
  // fp8 only: wgu and wd again in the decode stream's tiles
  // [E][Npad/256][K/128][256][128] (null when the shape does not tile)
  void* wgu_t = nullptr;
  void* wd_t = nullptr;
  float* sgu = nullptr;    // fp8 scales [E][2Hp] (packed-row order)
  float* sd = nullptr;     // fp8 scales [E][Cp]
  float* bg = nullptr;     // [E][Hp]
  float* bu = nullptr;     // [E][Hp]
  float* bd = nullptr;     // [E][Cp]
  // staging of host parameters (one of the largest size) and, for fp8, the
  // packed fp32 rows before quantisation; kept for later loads
  float* stage = nullptr;
  float* stage_tmp = nullptr;
  bool loaded = false;
  // Backward: the weights in the layouts the data-gradient products read,
  // derived from the forward packs on the first backward after a load
  // (wdb [E][Hq][C]: W_down rows h; wgub [E][Cp][2Hp]: W_gate/W_up rows c,
  // columns in the packed gate/up order), and the fp32 gradients.
  int Hq = 0;
  void* wdb = nullptr;
  void* wgub = nullptr;
  float* wrt = nullptr;    // W_r as [E][C] (fp32)
  bool bwd_ready = false;
  float* grad = nullptr;   // gWr [C][E], gbr [E], gWg [E][C][H], gbg [E][H],
                           // gWu [E][C][H], gbu [E][H], gWd [E][H][C], gbd [E][C]
  size_t g_off[8] = {};
  size_t g_total = 0;
  // The gradients are zero without the buffer holding zeros (set by
  // zero_grad and at allocation): the next backward writes every gradient
  // instead of adding to it, and a read clears the buffer first.
  bool grad_zero = false;
  // Set once a backward has been captured into a HIP graph: a graph keeps
  // the add mode it was captured in, so zero_grad then clears the buffer
  // (stream-ordered) instead of only marking it.
  bool bwd_captured = false;
  // Profiling ring: forward i records its stage boundaries into slot
  // i % kProfSlots; stage_times averages over the recorded slots.
  static constexpr int kProfSlots = 64;
  bool profiling = false;
  bool prof_gemm_only = false;   // forward: only the gate/up GEMM's two boundaries
  hipEvent_t ev[kProfSlots][MGPT_MOE_NUM_STAGES + 1] = {};
  int prof_count = 0;
  hipEvent_t evb[kProfSlots][MGPT_MOE_NUM_BWD_STAGES + 1] = {};
  int prof_b_count = 0;
  hipEvent_t done = nullptr;
  bool done_valid = false;
  // The backward's second stream (default priority) and its fork / join
  // events, created with the gradient buffer: the weight gradients run
  // beside the d(act) and dX products.
  hipStream_t side = nullptr;
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  int dact_cus = 0;   // persistent blocks of the d(act) product when forked
  int dx_cus = 0;     // persistent blocks of the dX product beside the gate/up weight gradient (0: serial)
  const int32_t* last_counts = nullptr;

  size_t act_bytes() const { return act == MGPT_DTYPE_BF16 ? 2 : 4; }
  size_t io_bytes() const { return io == MGPT_DTYPE_BF16 ? 2 : 4; }
  bool padded() const { return Cx != C; }
  // Few tokens and many experts: the router's logits are spread over more
  // blocks (one expert per wave) instead of one block per 64 tokens.
  bool router_split(int N) const { return E > 16 && (N < 4096 || wide()); }
  // more experts than a wave has lanes: the forward's generic paths only
  bool wide() const { return E > kMaxExperts; }
  // one router block of tokens: logits and softmax in one launch, and the
  // permute counts the ids itself (no histogram)
  bool router_one_launch(int N, bool norm) const {
    return wr4 && !wide() && N <= kRouterTokens && !norm && C % 64 == 0 &&
           C <= kDecodeRouterMaxC;
  }
  // The bf16 large-M path (gemm_dma.hip), which may split its last round.
  // bias partials of the weight gradients' row chunks: at most 64 chunks of
  // the wider tile row (2Hp gate/up columns or C down columns) of
  // 256-column tiles
  size_t wg_bpart_bytes() const {
    return (size_t)64 * ((std::max(2 * Hp, C) + 255) / 256) * 256 * 4;
  }
  bool uses_gemm_dma(int N) const {
    return act == MGPT_DTYPE_BF16 && wdt == MGPT_DTYPE_BF16 && gemm_tile == 256 &&
           (size_t)N * k >= (size_t)64 * E;
  }
  size_t w_bytes() const { return wdt == MGPT_DTYPE_FP8_E4M3 ? 1 : (wdt == MGPT_DTYPE_BF16 ? 2 : 4); }
  // h (SwiGLU output) is kept in the activation dtype.
  Layout layout(int N, bool train = false) const {
    Layout L{};
    const size_t A = (size_t)N * k;
    const size_t TB = router_tokens_per_block(E);
    const size_t nb = ((size_t)N + TB - 1) / TB;
    size_t off = 0;
    auto take = [&](size_t bytes) {
      size_t o = off;
      off = align_up(off + bytes, kAlign);
      return o;
    };
    L.topk_idx = take(A * 4);
    L.topk_p = take(A * 4);
    L.slot_of = take(A * 4);
    L.perm = take(A * 4);
    L.hist = take(nb * E * 4);
    L.base = take(nb * E * 4);
    L.counts = take((size_t)E * 4);
    // Sized for min(N, 4095) tokens whenever E > 16, so that the workspace
    // never shrinks as N grows past the split router's range.
    // (every N when E > 64: the wide forward always routes through the
    // split logits)
    L.logits = take(E > 16 ? (size_t)(wide() ? N : std::min(N, 4095)) * E * 4 : 0);
    L.xg = take((A + kRowPad) * C * act_bytes());
    L.hbuf = take((A + kRowPad) * Hp * act_bytes());
    L.obuf = take((A + kRowPad) * C * act_bytes());
    // fp32 partial tiles of the large-M GEMMs' split last round (one per CU)
    L.partials = take(uses_gemm_dma(N)             ? (size_t)num_cus * kGemmPartialBytes
                      : act == MGPT_DTYPE_F32 ? (size_t)num_cus * kF32PartialBytes
                                              : 0);
    L.rstd = take((size_t)N * 4);
    const size_t pad_rows = padded() ? (size_t)N * C * io_bytes() : 0;
    L.xpad = take(pad_rows);
    L.ypad = take(pad_rows);
    L.gpad = take(padded() ? (size_t)C * 4 : 0);
    if (train) {
      L.probs = take((size_t)N * E * 4);
      L.gu = take((A + kRowPad) * 2 * Hp * act_bytes());
      L.dgo = take((A + kRowPad) * C * act_bytes());
      L.dtp = take(A * 4);
      L.dlog = take((size_t)N * E * 4);
      const size_t chunks = (size_t)router_wgrad_chunks(N);
      L.rw_part = take(chunks * C * E * 4);
      L.rw_part_b = take(chunks * E * 4);
      L.wg_bpart = take(uses_gemm_dma(N) ? wg_bpart_bytes() : 0);
      L.wg_part2 = take(uses_gemm_dma(N) && dx_cus > 0 ? (size_t)num_cus * kGemmPartialBytes : 0);
      L.dypad = take(pad_rows);
      L.dxpad = take(pad_rows);
      L.nrm_part = take((size_t)rmsnorm_bwd_blocks(N) * C * 4);
    }
    L.total = off;
    return L;
  }
};

namespace {

int check_config(const mgpt_moe_config* c) {
  if (!c) return fail(MGPT_ERR_INVALID_ARGUMENT, "config is null");
  const int H = c->hidden_dim == -1 ? 4 * c->embed_dim : c->hidden_dim;
  if (c->embed_dim <= 0 || H <= 0 || c->num_experts <= 0 || c->top_k <= 0 ||
      c->top_k > c->num_experts)
    return fail(MGPT_ERR_INVALID_ARGUMENT,
                "invalid shape: embed_dim=%d hidden_dim=%d num_experts=%d top_k=%d",
                c->embed_dim, c->hidden_dim, c->num_experts, c->top_k);
  if (c->num_experts > kMaxExpertsWide)
    return fail(MGPT_ERR_UNSUPPORTED, "num_experts %d > %d", c->num_experts, kMaxExpertsWide);
  if (c->top_k > kMaxTopK)
    return fail(MGPT_ERR_UNSUPPORTED, "top_k %d > %d", c->top_k, kMaxTopK);
  // fp32 activations with bf16 / fp8 weights: the caller's tensors stay
  // fp32 (routing on the fp32 rows), the expert products run in bf16.
  const bool f32 = c->act_dtype == MGPT_DTYPE_F32 && c->weight_dtype == MGPT_DTYPE_F32;
  const bool lowp_w = c->weight_dtype == MGPT_DTYPE_BF16 || c->weight_dtype == MGPT_DTYPE_FP8_E4M3;
  const bool bf = (c->act_dtype == MGPT_DTYPE_BF16 || c->act_dtype == MGPT_DTYPE_F32) && lowp_w;
  if (!f32 && !bf)
    return fail(MGPT_ERR_UNSUPPORTED, "unsupported dtype pair act=%d weight=%d", c->act_dtype,
                c->weight_dtype);
  return MGPT_OK;
}

void free_weights(mgpt_moe* h) {
  void* ptrs[] = {h->wr_g, h->wr1, h->wr4,  h->br,  h->wgu,  h->wd,    h->sgu,  h->sd,    h->bg,
                  h->bu,   h->bd,  h->wdb,  h->wgub, h->wrt, h->wgu_t, h->wd_t, h->stage, h->stage_tmp};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  h->wr_g = h->wr1 = h->wr4 = h->br = h->sgu = h->sd = h->bg = h->bu = h->bd = h->wrt = nullptr;
  h->stage = h->stage_tmp = nullptr;
  h->wgu = h->wd = h->wdb = h->wgub = h->wgu_t = h->wd_t = nullptr;
  h->loaded = false;
  h->bwd_ready = false;
}

// Training is built for bf16 x bf16 and fp32 x fp32 handles (fp8 weights
// are an inference format here, and fp32 tensors over bf16 products an
// inference option).
bool trainable(const mgpt_moe* h) { return h->wdt == h->act && h->io == h->act; }

// Allocates the gradient buffer on first use, its contents logically zero.
int ensure_grad(mgpt_moe* h) {
  if (h->grad) return MGPT_OK;
  const size_t C = h->C, H = h->H, E = h->E;
  const size_t sizes[8] = {C * E, E, E * C * H, E * H, E * C * H, E * H, E * H * C, E * C};
  size_t off = 0;
  for (int i = 0; i < 8; ++i) {
    h->g_off[i] = off;
    off += sizes[i];
  }
  h->g_total = off;
  HIP_TRY(hipMalloc(&h->grad, sizeof(float) * off));
  h->grad_zero = true;
  if (!h->side) {
    HIP_TRY(hipStreamCreateWithFlags(&h->side, hipStreamNonBlocking));
    // device-scope ordering between the two streams only: no system-scope
    // fence (cache write-back and invalidate) at each record
    HIP_TRY(hipEventCreateWithFlags(&h->fork_ev, hipEventDisableTiming | hipEventDisableSystemFence));
    HIP_TRY(hipEventCreateWithFlags(&h->join_ev, hipEventDisableTiming | hipEventDisableSystemFence));
  }
  return MGPT_OK;
}

// The gradient buffer with its contents, zeroing it (stream-ordered) if
// it is only logically zero.
int materialize_grad(mgpt_moe* h, hipStream_t st) {
  if (int rc = ensure_grad(h)) return rc;
  if (h->grad_zero) {
    HIP_TRY(launch_fill_zero(h->grad, h->g_total, st));
    h->grad_zero = false;
  }
  return MGPT_OK;
}

// The backward weight layouts, transposed from the forward packs.
int ensure_bwd_weights(mgpt_moe* h, hipStream_t st) {
  if (h->bwd_ready) return MGPT_OK;
  const int C = h->C, E = h->E, Hp = h->Hp, Cp = h->Cp;
  h->Hq = round_up(Hp, 256);
  const size_t eb = h->act_bytes();
  if (!h->wdb) HIP_TRY(hipMalloc(&h->wdb, eb * E * h->Hq * C));
  if (!h->wgub) HIP_TRY(hipMalloc(&h->wgub, eb * E * Cp * 2 * Hp));
  // W_r [E][C] from the router pack [G][C][RE]: per group a [C][RE] -> [RE][C]
  // transpose (E is padded to G*RE there; the padding experts are never read)
  const int RE = router_experts_per_wave(E), G = (E + RE - 1) / RE;
  if (!h->wrt) HIP_TRY(hipMalloc(&h->wrt, sizeof(float) * (size_t)G * RE * C));
  HIP_TRY(launch_transpose_pad<float>(h->wr_g, C, RE, (size_t)C * RE, h->wrt, RE, C,
                                      (size_t)RE * C, G, st));
  if (h->act == MGPT_DTYPE_BF16) {
    HIP_TRY(launch_transpose_pad<bf16_t>((const bf16_t*)h->wd, Cp, Hp, (size_t)Cp * Hp,
                                         (bf16_t*)h->wdb, h->Hq, C, (size_t)h->Hq * C, E, st));
    HIP_TRY(launch_transpose_pad<bf16_t>((const bf16_t*)h->wgu, 2 * Hp, C, (size_t)2 * Hp * C,
                                         (bf16_t*)h->wgub, Cp, 2 * Hp, (size_t)Cp * 2 * Hp, E,
                                         st));
  } else {
    HIP_TRY(launch_transpose_pad<float>((const float*)h->wd, Cp, Hp, (size_t)Cp * Hp,
                                        (float*)h->wdb, h->Hq, C, (size_t)h->Hq * C, E, st));
    HIP_TRY(launch_transpose_pad<float>((const float*)h->wgu, 2 * Hp, C, (size_t)2 * Hp * C,
                                        (float*)h->wgub, Cp, 2 * Hp, (size_t)Cp * 2 * Hp, E, st));
  }
  h->bwd_ready = true;
  return MGPT_OK;
}

// Tile choice for the bf16 grouped GEMMs: decode-shaped (few rows per
// expert) segments use 32-row tiles so the MFMAs are not mostly padding.
bool small_m(const mgpt_moe* h, int N) { return (size_t)N * h->k < (size_t)64 * h->E; }

}  // namespace

extern "C" {

const char* mgpt_moe_last_error(void) { return g_last_error.c_str(); }

int mgpt_moe_create(const mgpt_moe_config* cfg, mgpt_moe** out) {
  if (!out) return fail(MGPT_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  int rc = check_config(cfg);
  if (rc) return rc;
  mgpt_moe* h = new (std::nothrow) mgpt_moe();
  if (!h) return fail(MGPT_ERR_OUT_OF_MEMORY, "host allocation failed");
  h->Cx = cfg->embed_dim;
  h->C = round_up(h->Cx, 64);
  h->H = cfg->hidden_dim == -1 ? 4 * cfg->embed_dim : cfg->hidden_dim;
  h->E = cfg->num_experts;
  h->k = cfg->top_k;
  h->io = cfg->act_dtype;
  h->wdt = cfg->weight_dtype;
  h->act = h->wdt == MGPT_DTYPE_F32 ? MGPT_DTYPE_F32 : MGPT_DTYPE_BF16;
  h->Hp = round_up(h->H, 128);
  h->Cp = round_up(h->C, 256);
  // Tuning override for the large-M tile (default 256x256).
  if (const char* t = std::getenv("MGPT_MOE_GEMM_TILE")) h->gemm_tile = std::atoi(t) == 128 ? 128 : 256;
  hipError_t e = hipGetDevice(&h->device);
  if (e == hipSuccess)
    e = hipDeviceGetAttribute(&h->num_cus, hipDeviceAttributeMultiprocessorCount, h->device);
  if (e == hipSuccess && h->num_cus <= 0) e = hipErrorInvalidDevice;
  // the backward's d(act) product beside the down weight gradient: 5/8 of
  // the CUs, a multiple of the XCD count (tuning override MGPT_MOE_DACT_CUS;
  // cfg3 step on MI355X: 2.29 ms at 160 of 256 CUs, 2.33 at 128, 2.34 at 176,
  // 2.31 at 200 and serial)
  h->dact_cus = std::max(kNumXcd, h->num_cus * 5 / 8 / kNumXcd * kNumXcd);
  if (const char* t = std::getenv("MGPT_MOE_DACT_CUS"))
    h->dact_cus = std::min(h->num_cus, std::max(kNumXcd, std::atoi(t) / kNumXcd * kNumXcd));
  // ... and the dX product beside the gate/up weight gradient: half the CUs
  // (MGPT_MOE_DX_CUS; 0 keeps the two serial)
  h->dx_cus = std::max(kNumXcd, h->num_cus / 2 / kNumXcd * kNumXcd);
  if (const char* t = std::getenv("MGPT_MOE_DX_CUS"))
    h->dx_cus = std::min(h->num_cus, std::max(0, std::atoi(t) / kNumXcd * kNumXcd));
  if (e == hipSuccess) {
    // Stage events only time: without the system-scope fence their record
    // does not write back and invalidate the caches, which otherwise leaves
    // a gap of several microseconds before the next launch.
    for (auto& slot : h->ev)
      for (auto& ev : slot)
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableSystemFence);
    for (auto& slot : h->evb)
      for (auto& ev : slot)
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableSystemFence);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&h->done, hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    mgpt_moe_destroy(h);
    return fail(MGPT_ERR_HIP, "device setup failed: %s", hipGetErrorString(e));
  }
  // The noalloc forward's scratch address on this device, looked up here
  // (once per device) so that a later mgpt_moe_forward_noalloc, possibly
  // under graph capture, makes no runtime call to find it.
  void* scratch_ptr = nullptr;
  if (int rc2 = scratch_address(h->device, &scratch_ptr)) {
    mgpt_moe_destroy(h);
    return rc2;
  }
  *out = h;
  return MGPT_OK;
}

int mgpt_moe_destroy(mgpt_moe* h) {
  if (!h) return MGPT_OK;
  free_weights(h);
  if (h->grad) (void)hipFree(h->grad);
  for (auto& slot : h->ev)
    for (auto& ev : slot)
      if (ev) (void)hipEventDestroy(ev);
  for (auto& slot : h->evb)
    for (auto& ev : slot)
      if (ev) (void)hipEventDestroy(ev);
  if (h->done) (void)hipEventDestroy(h->done);
  if (h->fork_ev) (void)hipEventDestroy(h->fork_ev);
  if (h->join_ev) (void)hipEventDestroy(h->join_ev);
  if (h->side) (void)hipStreamDestroy(h->side);
  delete h;
  return MGPT_OK;
}

int mgpt_moe_load_parameters(mgpt_moe* h, const float* const* params, int num_params,
                             int params_on_device, void* stream_ptr) {
  if (!h || !params) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle or params");
  if (num_params != 2 + 6 * h->E)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "expected %d parameters (2 + 6*E), got %d",
                2 + 6 * h->E, num_params);
  for (int i = 0; i < num_params; ++i)
    if (!params[i]) return fail(MGPT_ERR_INVALID_ARGUMENT, "parameter %d is null", i);
  hipStream_t st = (hipStream_t)stream_ptr;
  HIP_TRY(hipSetDevice(h->device));
  const int C = h->C, Cx = h->Cx, H = h->H, E = h->E, Hp = h->Hp, Cp = h->Cp;
  const size_t wb = h->w_bytes();
  const bool fp8 = h->wdt == MGPT_DTYPE_FP8_E4M3;
  const bool bf = h->wdt == MGPT_DTYPE_BF16;
  const int RE = router_experts_per_wave(E);
  // The packed buffers depend only on the handle's shape: the first load
  // allocates them (and zeroes the padding the packs never write), later
  // loads re-pack into them, stream-ordered, with no allocation.  The
  // backward's transposed copies are rebuilt from the new packs.
  h->loaded = false;
  h->bwd_ready = false;
  const bool first = h->wgu == nullptr;
  if (first) {
    HIP_TRY(hipMalloc(&h->wr_g, sizeof(float) * ((E + RE - 1) / RE) * RE * C));
    if (E > 16) HIP_TRY(hipMalloc(&h->wr1, sizeof(float) * E * C));
    if (E > 16 && C % 64 == 0 && C <= kDecodeRouterMaxC)
      HIP_TRY(hipMalloc(&h->wr4, sizeof(float) * E * C));
    HIP_TRY(hipMalloc(&h->br, sizeof(float) * E));
    HIP_TRY(hipMalloc(&h->bg, sizeof(float) * E * Hp));
    HIP_TRY(hipMalloc(&h->bu, sizeof(float) * E * Hp));
    HIP_TRY(hipMalloc(&h->bd, sizeof(float) * E * Cp));
    if (fp8) {
      HIP_TRY(hipMalloc(&h->sgu, sizeof(float) * E * 2 * Hp));
      HIP_TRY(hipMalloc(&h->sd, sizeof(float) * E * Cp));
    }
    HIP_TRY(hipMalloc(&h->wd, wb * E * Cp * Hp));
    HIP_TRY(hipMemsetAsync(h->wd, 0, wb * E * Cp * Hp, st));
    HIP_TRY(hipMalloc(&h->wgu, wb * E * 2 * Hp * C));
    HIP_TRY(hipMemsetAsync(h->wgu, 0, wb * E * 2 * Hp * C, st));
  }

  // Host parameters are staged through one device buffer of the largest size.
  const size_t max_elems = std::max<size_t>((size_t)Cx * std::max(H, E), (size_t)H * Cx);
  if (!params_on_device && !h->stage) HIP_TRY(hipMalloc(&h->stage, sizeof(float) * max_elems));
  if (fp8 && !h->stage_tmp)
    HIP_TRY(hipMalloc(&h->stage_tmp,
                      sizeof(float) * std::max<size_t>((size_t)2 * Hp * C, (size_t)Cp * Hp)));
  float* stage = h->stage;
  float* fp32tmp = h->stage_tmp;   // fp8: packed fp32 before quantisation
  int rc = MGPT_OK;
  auto src = [&](int i, size_t n) -> const float* {
    if (params_on_device) return params[i];
    hipError_t e = hipMemcpyAsync(stage, params[i], sizeof(float) * n, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) {
      rc = fail(MGPT_ERR_HIP, "parameter %d upload failed: %s", i, hipGetErrorString(e));
      return nullptr;
    }
    return stage;
  };
  auto pack = [&](const float* s, int Kin, int Nout, void* dst, int ldd, int mode, int off) {
    hipError_t e;
    if (bf)
      e = launch_pack_transpose<bf16_t>(s, Kin, Nout, (bf16_t*)dst, ldd, mode, off, st);
    else
      e = launch_pack_transpose<float>(s, Kin, Nout, (float*)dst, ldd, mode, off, st);
    if (e != hipSuccess) rc = fail(MGPT_ERR_HIP, "pack failed: %s", hipGetErrorString(e));
  };
  do {
    const float* s = src(0, (size_t)Cx * E);
    if (!s) break;
    if (launch_pack_router(s, Cx, C, E, RE, h->wr_g, st) != hipSuccess ||
        (h->wr1 && launch_pack_router(s, Cx, C, E, 1, h->wr1, st) != hipSuccess) ||
        (h->wr4 && launch_pack_router_quads(s, Cx, C, E, h->wr4, st) != hipSuccess)) {
      rc = fail(MGPT_ERR_HIP, "router pack failed");
      break;
    }
    s = src(1, E);
    if (!s) break;
    HIP_TRY(hipMemcpyAsync(h->br, s, sizeof(float) * E, hipMemcpyDeviceToDevice, st));
    for (int e = 0; e < E && rc == MGPT_OK; ++e) {
      const int p = 2 + 6 * e;
      const size_t gu_off = (size_t)e * 2 * Hp * C;
      const size_t d_off = (size_t)e * Cp * Hp;
      if (fp8) HIP_TRY(hipMemsetAsync(fp32tmp, 0, sizeof(float) * 2 * Hp * C, st));
      for (int which = 0; which < 2 && rc == MGPT_OK; ++which) {   // gate, up
        // [Cx][H] -> rows of the packed [2Hp][C]: columns past Cx stay zero
        if (!(s = src(p + 2 * which, (size_t)Cx * H))) break;
        if (fp8) {
          if (launch_pack_transpose<float>(s, Cx, H, fp32tmp, C, 1, 32 * which, st) != hipSuccess)
            rc = fail(MGPT_ERR_HIP, "pack failed");
        } else {
          pack(s, Cx, H, (char*)h->wgu + gu_off * h->w_bytes(), C, 1, 32 * which);
        }
        if (!(s = src(p + 2 * which + 1, H))) break;
        HIP_TRY(launch_pad_row(s, H, (which ? h->bu : h->bg) + (size_t)e * Hp, Hp, st));
      }
      if (rc) break;
      if (fp8)
        HIP_TRY(launch_quantize_rows(fp32tmp, 2 * Hp, C, (uint8_t*)h->wgu + gu_off,
                                     h->sgu + (size_t)e * 2 * Hp, st));
      // [H][Cx] -> rows 0..Cx of the packed [Cp][Hp]; the rest stay zero
      if (!(s = src(p + 4, (size_t)H * Cx))) break;
      if (fp8) {
        HIP_TRY(hipMemsetAsync(fp32tmp, 0, sizeof(float) * Cp * Hp, st));
        if (launch_pack_transpose<float>(s, H, Cx, fp32tmp, Hp, 0, 0, st) != hipSuccess)
          rc = fail(MGPT_ERR_HIP, "pack failed");
        HIP_TRY(launch_quantize_rows(fp32tmp, Cp, Hp, (uint8_t*)h->wd + d_off,
                                     h->sd + (size_t)e * Cp, st));
      } else {
        pack(s, H, Cx, (char*)h->wd + d_off * h->w_bytes(), Hp, 0, 0);
      }
      if (!(s = src(p + 5, Cx))) break;
      HIP_TRY(launch_pad_row(s, Cx, h->bd + (size_t)e * Cp, Cp, st));
      // Host sources are staged through one buffer: finish before reuse.
      if (!params_on_device) HIP_TRY(hipStreamSynchronize(st));
    }
    if (rc == MGPT_OK && fp8 && C % 128 == 0 && Hp % 128 == 0 && Cp % 256 == 0) {
      // the decode stream's contiguous 32 KB stage tiles (a second copy)
      if (!h->wgu_t) HIP_TRY(hipMalloc(&h->wgu_t, (size_t)E * 2 * Hp * C));
      if (!h->wd_t) HIP_TRY(hipMalloc(&h->wd_t, (size_t)E * Cp * Hp));
      HIP_TRY(launch_tile_fp8((const uint8_t*)h->wgu, E, 2 * Hp, C, (uint8_t*)h->wgu_t, st));
      HIP_TRY(launch_tile_fp8((const uint8_t*)h->wd, E, Cp, Hp, (uint8_t*)h->wd_t, st));
    }
  } while (0);
  if (rc) {
    (void)hipStreamSynchronize(st);
    free_weights(h);
    return rc;
  }
  // A first load (new allocations) and host sources finish before the call
  // returns; a re-pack of device parameters stays stream-ordered.
  if (first || !params_on_device) {
    const hipError_t se = hipStreamSynchronize(st);
    if (se != hipSuccess) {
      free_weights(h);
      return fail(MGPT_ERR_HIP, "parameter packing failed: %s", hipGetErrorString(se));
    }
  }
  h->loaded = true;
  return MGPT_OK;
}

int mgpt_moe_load_gpt_bin(mgpt_moe* h, const char* path, int layer, float* ln2_gamma,
                          void* stream) {
  if (!h) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle");
  mgpt_gpt_bin_info info;
  if (int rc = mgpt_gpt_bin_inspect(path, h->E, h->H, &info)) return rc;
  if (info.embed_dim != h->Cx)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "%s: embed_dim %d, the handle has C = %d", path,
                info.embed_dim, h->Cx);
  std::vector<float> buf;
  try {
    buf.resize((size_t)info.moe_floats);
  } catch (const std::bad_alloc&) {
    return fail(MGPT_ERR_OUT_OF_MEMORY, "host buffer of %lld floats", (long long)info.moe_floats);
  }
  if (int rc = mgpt_gpt_bin_read_block(path, h->E, h->H, layer, ln2_gamma, buf.data(),
                                       buf.size()))
    return rc;
  // pointers into the block's parameters, get_parameters() order
  const size_t C = h->Cx, H = h->H, E = h->E;
  std::vector<const float*> ptr;
  const float* p = buf.data();
  auto take = [&](size_t n) {
    ptr.push_back(p);
    p += n;
  };
  take(C * E);
  take(E);
  for (size_t e = 0; e < E; ++e) {
    take(C * H);
    take(H);
    take(C * H);
    take(H);
    take(H * C);
    take(C);
  }
  return mgpt_moe_load_parameters(h, ptr.data(), (int)ptr.size(), 0, stream);
}

int mgpt_moe_workspace_bytes(const mgpt_moe* h, int num_tokens, size_t* bytes) {
  if (!h || !bytes || num_tokens < 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle/bytes or negative num_tokens");
  *bytes = h->layout(num_tokens).total;
  return MGPT_OK;
}

}  // extern "C"

namespace {

// Block mode (gamma set): route and gather RMSNorm(x) * gamma and add x
// to the output (the MoE half of TransformerBlock::forward_into).
struct BlockArgs {
  const float* gamma = nullptr;
  float eps = 0.0f;
};

// IoT: the caller's x and y; ActT: the gathered rows, h and expert outputs.
template <typename IoT, typename ActT>
int forward_impl(mgpt_moe* h, const IoT* x, IoT* y, int N, char* ws, bool train,
                 hipStream_t st, BlockArgs blk = BlockArgs()) {
  const Layout L = h->layout(N, train);
  const int C = h->C, Cx = h->Cx, E = h->E, k = h->k, Hp = h->Hp, Cp = h->Cp;
  const size_t A = (size_t)N * k;
  int32_t* idx = (int32_t*)(ws + L.topk_idx);
  float* topp = (float*)(ws + L.topk_p);
  int32_t* slot_of = (int32_t*)(ws + L.slot_of);
  int32_t* perm = (int32_t*)(ws + L.perm);
  int32_t* hist = (int32_t*)(ws + L.hist);
  int32_t* base = (int32_t*)(ws + L.base);
  int32_t* counts = (int32_t*)(ws + L.counts);
  ActT* xg = (ActT*)(ws + L.xg);
  ActT* hb = (ActT*)(ws + L.hbuf);
  ActT* ob = (ActT*)(ws + L.obuf);
  // Under stream capture (a HIP graph of the forward, e.g. a fixed-length
  // decode step) the forward records no events: stage timing is off and
  // mgpt_moe_expert_counts reports NOT_READY until an eager forward.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(st, &cap));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  const bool prof = h->profiling && !capturing;
  const bool gemm_only = h->prof_gemm_only;
  hipEvent_t* evs = h->ev[h->prof_count % mgpt_moe::kProfSlots];
  auto mark = [&](int i) -> hipError_t {
    return prof && (!gemm_only || i == 2 || i == 3) ? hipEventRecord(evs[i], st) : hipSuccess;
  };

  HIP_TRY(mark(0));
  // A caller width that is not a multiple of 64: the rows (and gamma) are
  // copied into zero-padded ones of width C; the output comes back the same
  // way.  Padding adds +0 terms only, so routing and outputs are unchanged.
  const IoT* xi = x;
  IoT* yi = y;
  const float* gamma = blk.gamma;
  if (h->padded()) {
    IoT* xp = (IoT*)(ws + L.xpad);
    HIP_TRY(launch_copy_cols<IoT>(x, Cx, xp, C, N, Cx, C, st));
    xi = xp;
    yi = (IoT*)(ws + L.ypad);
    if (gamma) {
      float* gp = (float*)(ws + L.gpad);
      HIP_TRY(launch_copy_cols<float>(gamma, Cx, gp, C, 1, Cx, C, st));
      gamma = gp;
    }
  }
  float* logits = h->router_split(N) ? (float*)(ws + L.logits) : nullptr;
  // training: keep the router probabilities and the gate/up pre-activations
  float* probs = train ? (float*)(ws + L.probs) : nullptr;
  ActT* gu = train ? (ActT*)(ws + L.gu) : nullptr;
  float* rstd = gamma ? (float*)(ws + L.rstd) : nullptr;
  const bool one_launch = h->router_one_launch(N, gamma != nullptr);
  HIP_TRY(launch_router<IoT>(xi, h->wr_g, h->wr1, one_launch ? h->wr4 : nullptr, h->br, N, C, E,
                             k, idx, topp, hist, logits,
                             probs, gamma, blk.eps, Cx, rstd, st));
  HIP_TRY(mark(1));
  // A decode step of at most 512 flat ids (N * k) with fp8 weights (no
  // training caches): the gate/up weight-streaming GEMM routes the ids
  // itself and reads the caller's rows of x (bf16, or fp32 rounded as the
  // permute would), so no permute runs.
  const bool gather_decode = !train && !gamma && !h->wide() && h->wdt == MGPT_DTYPE_FP8_E4M3 &&
                             h->wgu_t &&
                             small_m(h, N) && A <= (size_t)kRouterTokens * kMaxTopK;
  if (!gather_decode)
    HIP_TRY((launch_permute<IoT, ActT>(xi, idx, one_launch ? nullptr : hist, base, N, C, E, k,
                                       counts, perm, slot_of, xg, rstd, gamma, st)));
  HIP_TRY(mark(2));
  if constexpr (sizeof(ActT) == 4) {
    const int mt = (int)((A + 63) / 64) + E;
    HIP_TRY((launch_grouped_gemm<64, 128, 2, 2, float, float, kEpiGateUp, float>(
        xg, (const float*)h->wgu, nullptr, h->bg, h->bu, counts, E, C, 2 * Hp, 2 * Hp, Hp, hb, Hp,
        mt, gu, 2 * Hp, st)));
    HIP_TRY(mark(3));
    // few tiles (small N): split along K over the CUs (fp32 partials, in-order reduce)
    HIP_TRY((launch_grouped_gemm<64, 128, 2, 2, float, float, kEpiDown, float>(
        hb, (const float*)h->wd, nullptr, h->bd, nullptr, counts, E, Hp, Cp, C, Cp, ob, C, mt,
        nullptr, 0, st, (float*)(ws + L.partials), h->num_cus)));
  } else {
    const bool fp8 = h->wdt == MGPT_DTYPE_FP8_E4M3;
    if (small_m(h, N)) {
      const int mt = (int)((A + 31) / 32) + E;
      if (fp8 && h->wgu_t && !h->wide()) {
        // weight streaming: the persistent direct-to-LDS decode kernel on the
        // tiled copies
        if (gather_decode)
          HIP_TRY(launch_gemm_decode_gather<IoT>(xi, (const fp8_t*)h->wgu_t, h->sgu, h->bg, h->bu, idx,
                                            (int)A, k, E, C, 2 * Hp, 2 * Hp, Hp, hb, Hp, mt, counts,
                                            perm, slot_of, st));
        else
          HIP_TRY(launch_gemm_decode<kEpiGateUp>(xg, (const fp8_t*)h->wgu_t, h->sgu, h->bg, h->bu,
                                                 counts, E, C, 2 * Hp, 2 * Hp, Hp, hb, Hp, mt,
                                                 st));
        HIP_TRY(mark(3));
        HIP_TRY(launch_gemm_decode<kEpiDown>(hb, (const fp8_t*)h->wd_t, h->sd, h->bd, nullptr,
                                             counts, E, Hp, Cp, C, Cp, ob, C, mt, st));
      } else if (fp8) {
        HIP_TRY((launch_grouped_gemm<32, 256, 1, 4, bf16_t, fp8_t, kEpiGateUp, bf16_t>(
            xg, (const fp8_t*)h->wgu, h->sgu, h->bg, h->bu, counts, E, C, 2 * Hp, 2 * Hp, Hp, hb,
            Hp, mt, nullptr, 0, st)));
        HIP_TRY(mark(3));
        HIP_TRY((launch_grouped_gemm<32, 256, 1, 4, bf16_t, fp8_t, kEpiDown, bf16_t>(
            hb, (const fp8_t*)h->wd, h->sd, h->bd, nullptr, counts, E, Hp, Cp, C, Cp, ob, C, mt,
            nullptr, 0, st)));
      } else {
        HIP_TRY((launch_grouped_gemm<32, 256, 1, 4, bf16_t, bf16_t, kEpiGateUp, bf16_t>(
            xg, (const bf16_t*)h->wgu, nullptr, h->bg, h->bu, counts, E, C, 2 * Hp, 2 * Hp, Hp,
            hb, Hp, mt, gu, 2 * Hp, st)));
        HIP_TRY(mark(3));
        HIP_TRY((launch_grouped_gemm<32, 256, 1, 4, bf16_t, bf16_t, kEpiDown, bf16_t>(
            hb, (const bf16_t*)h->wd, nullptr, h->bd, nullptr, counts, E, Hp, Cp, C, Cp, ob, C,
            mt, nullptr, 0, st)));
      }
    } else if (h->gemm_tile == 256 && !fp8) {
      // bf16 weights, prefill-shaped segments: 256x256 direct-to-LDS kernel.
      const int mt = (int)((A + 255) / 256) + E;
      float* part = (float*)(ws + L.partials);
      // The gate/up GEMM has ~12x more tiles than CUs at prefill shapes, so a
      // partial last round costs little; only the down GEMM splits it
      // (splitting gate/up's last round too measured within noise at cfg2-cfg4).
      HIP_TRY(launch_gemm_dma<kEpiGateUp>(xg, (const bf16_t*)h->wgu, h->bg, h->bu, counts, E, C,
                                          2 * Hp, 2 * Hp, Hp, hb, Hp, mt, nullptr, h->num_cus,
                                          (bf16_t*)gu, 2 * Hp, st));
      HIP_TRY(mark(3));
      HIP_TRY(launch_gemm_dma<kEpiDown>(hb, (const bf16_t*)h->wd, h->bd, nullptr, counts, E, Hp,
                                        Cp, C, Cp, ob, C, mt, part, h->num_cus, nullptr, 0, st));
    } else {
      const int mt = (int)((A + 127) / 128) + E;
      if (fp8) {
        HIP_TRY((launch_grouped_gemm<128, 128, 2, 2, bf16_t, fp8_t, kEpiGateUp, bf16_t>(
            xg, (const fp8_t*)h->wgu, h->sgu, h->bg, h->bu, counts, E, C, 2 * Hp, 2 * Hp, Hp, hb,
            Hp, mt, nullptr, 0, st)));
        HIP_TRY(mark(3));
        HIP_TRY((launch_grouped_gemm<128, 128, 2, 2, bf16_t, fp8_t, kEpiDown, bf16_t>(
            hb, (const fp8_t*)h->wd, h->sd, h->bd, nullptr, counts, E, Hp, Cp, C, Cp, ob, C, mt,
            nullptr, 0, st)));
      } else {
        HIP_TRY((launch_grouped_gemm<128, 128, 2, 2, bf16_t, bf16_t, kEpiGateUp, bf16_t>(
            xg, (const bf16_t*)h->wgu, nullptr, h->bg, h->bu, counts, E, C, 2 * Hp, 2 * Hp, Hp,
            hb, Hp, mt, gu, 2 * Hp, st)));
        HIP_TRY(mark(3));
        HIP_TRY((launch_grouped_gemm<128, 128, 2, 2, bf16_t, bf16_t, kEpiDown, bf16_t>(
            hb, (const bf16_t*)h->wd, nullptr, h->bd, nullptr, counts, E, Hp, Cp, C, Cp, ob, C,
            mt, nullptr, 0, st)));
      }
    }
  }
  HIP_TRY(mark(4));
  HIP_TRY((launch_combine<ActT, IoT>(ob, idx, topp, slot_of, N, C, k, gamma ? xi : nullptr, yi,
                                     st)));
  if (h->padded()) HIP_TRY(launch_copy_cols<IoT>(yi, C, y, Cx, N, Cx, Cx, st));
  HIP_TRY(mark(5));
  if (prof) ++h->prof_count;
  if (capturing) {
    h->done_valid = false;
  } else {
    HIP_TRY(hipEventRecord(h->done, st));
    h->done_valid = true;
  }
  h->last_counts = counts;
  return MGPT_OK;
}

template <typename ActT>
int backward_impl(mgpt_moe* h, const ActT* x, const ActT* dy, ActT* dx, int N, char* ws,
                  hipStream_t st, const float* gamma = nullptr) {
  const Layout L = h->layout(N, true);
  const int C = h->C, Cx = h->Cx, H = h->H, E = h->E, k = h->k, Hp = h->Hp, Cp = h->Cp;
  const int A = N * k;
  if (int rc = ensure_grad(h)) return rc;
  if (int rc = ensure_bwd_weights(h, st)) return rc;
  // padded width: dy in and dx out through zero-padded rows; x is the padded
  // copy the training forward left in the workspace
  ActT* dx_out = dx;
  if (h->padded()) {
    ActT* dyp = (ActT*)(ws + L.dypad);
    HIP_TRY(launch_copy_cols<ActT>(dy, Cx, dyp, C, N, Cx, C, st));
    dy = dyp;
    x = (const ActT*)(ws + L.xpad);
    dx = (ActT*)(ws + L.dxpad);
    if (gamma) gamma = (const float*)(ws + L.gpad);
  }
  // fused block (gamma set): the router's input was (x * rstd) * gamma
  const float* rstd = gamma ? (const float*)(ws + L.rstd) : nullptr;
  const int32_t* idx = (const int32_t*)(ws + L.topk_idx);
  const float* topp = (const float*)(ws + L.topk_p);
  const int32_t* slot_of = (const int32_t*)(ws + L.slot_of);
  const int32_t* perm = (const int32_t*)(ws + L.perm);
  const int32_t* counts = (const int32_t*)(ws + L.counts);
  const ActT* xg = (const ActT*)(ws + L.xg);
  const ActT* hb = (const ActT*)(ws + L.hbuf);
  ActT* ob = (ActT*)(ws + L.obuf);   // expert outputs, then dX of the experts
  const float* probs = (const float*)(ws + L.probs);
  ActT* gu = (ActT*)(ws + L.gu);     // pre-activations, then d(gate) / d(up)
  ActT* dgo = (ActT*)(ws + L.dgo);
  float* dtp = (float*)(ws + L.dtp);
  float* dlog = (float*)(ws + L.dlog);
  float* g = h->grad;
  const ActT* wdb = (const ActT*)h->wdb;
  const ActT* wgub = (const ActT*)h->wgub;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(st, &cap));
  // no stage events inside a captured graph (as in the forward)
  const bool prof = h->profiling && !h->prof_gemm_only && cap == hipStreamCaptureStatusNone;
  hipEvent_t* evs = h->evb[h->prof_b_count % mgpt_moe::kProfSlots];
  auto mark = [&](int i) -> hipError_t { return prof ? hipEventRecord(evs[i], st) : hipSuccess; };

  // dW_down [H][C] and db_down from (h, dgo); dW_gate/up [C][H] and their
  // biases from (gathered x, d(gate)/d(up))
  // (an expert's long contraction is cut into row chunks whose partial
  // tiles go to the split-K region when the dX product is not using it: the
  // down weight gradient runs before dX, the gate/up one after it or, beside
  // it, with a region of its own)
  float* wpart = h->uses_gemm_dma(N) ? (float*)(ws + L.partials) : nullptr;
  const size_t wpart_bytes = wpart ? (size_t)h->num_cus * kGemmPartialBytes : 0;
  float* wbpart = h->uses_gemm_dma(N) ? (float*)(ws + L.wg_bpart) : nullptr;
  const size_t wbpart_bytes = wbpart ? h->wg_bpart_bytes() : 0;
  // After zero_grad the gradients are written, not added to; the experts
  // without rows are cleared instead (before either weight gradient).
  const bool store = h->grad_zero;
  bool down_done = false, gateup_done = false;
  auto down_wgrad = [&](hipStream_t s) -> int {
    if (store) {
      IdleSlices z{};
      const size_t lens[6] = {(size_t)C * H, (size_t)H, (size_t)C * H, (size_t)H, (size_t)H * C,
                              (size_t)C};
      for (int p = 0; p < 6; ++p) {
        z.base[p] = g + h->g_off[2 + p];
        z.len[p] = lens[p];
      }
      z.n = 6;
      HIP_TRY(launch_zero_idle_experts(counts, E, z, s));
    }
    HIP_TRY((launch_wgrad<ActT, 0>(hb, Hp, Hp, dgo, C, C, counts, E, g + h->g_off[6], nullptr, C,
                                   (size_t)H * C, H, C, g + h->g_off[7], nullptr, (size_t)C, A,
                                   wpart, wpart_bytes, wbpart, wbpart_bytes, h->num_cus, store,
                                   s)));
    return MGPT_OK;
  };

  HIP_TRY(mark(0));
  HIP_TRY(launch_scatter_bwd<ActT>(dy, ob, perm, topp, A, C, k, dgo, dtp, st));
  HIP_TRY(mark(1));
  if constexpr (sizeof(ActT) == 4) {
    const int mt = (A + 63) / 64 + E;
    HIP_TRY((launch_grouped_gemm<64, 128, 2, 2, float, float, kEpiSwigluBwd, float>(
        dgo, wdb, nullptr, nullptr, nullptr, counts, E, C, h->Hq, Hp, 0, gu, 2 * Hp, mt, gu,
        2 * Hp, st)));
    HIP_TRY(mark(2));
    HIP_TRY((launch_grouped_gemm<64, 128, 2, 2, float, float, kEpiDown, float>(
        gu, wgub, nullptr, nullptr, nullptr, counts, E, 2 * Hp, Cp, C, 0, ob, C, mt, nullptr, 0,
        st)));
  } else if (h->uses_gemm_dma(N)) {
    // prefill-shaped segments: the 256x256 direct-to-LDS kernel; the dX
    // product splits its last round like the forward's down GEMM
    const int mt = (A + 255) / 256 + E;
    // The d(act) product's epilogue (read g, u; write d(gate), d(up)) keeps
    // HBM busy while its k loops leave it idle, and on half the CUs it takes
    // 579 instead of 352 us (cfg3): its epilogues are bound by the chip's
    // bandwidth more than by the CUs'.  So it runs persistent on part of
    // them, and the down weight gradient (which does not depend on it) runs
    // from the second stream on the rest; the dX product waits for both.
    // Stage timing keeps the launches serial.
    const bool fork = !prof && h->side && h->fork_ev && h->join_ev;
    if (fork) HIP_TRY(hipEventRecord(h->fork_ev, st));
    HIP_TRY(launch_gemm_dma<kEpiSwigluBwd>((const bf16_t*)dgo, (const bf16_t*)wdb, nullptr,
                                           nullptr, counts, E, C, h->Hq, Hp, 0, (bf16_t*)gu,
                                           2 * Hp, mt, nullptr, fork ? h->dact_cus : h->num_cus,
                                           (bf16_t*)gu, 2 * Hp, st));
    if (fork) {
      HIP_TRY(hipStreamWaitEvent(h->side, h->fork_ev, 0));
      if (int rc = down_wgrad(h->side)) return rc;
      HIP_TRY(hipEventRecord(h->join_ev, h->side));
      HIP_TRY(hipStreamWaitEvent(st, h->join_ev, 0));
      down_done = true;
    }
    HIP_TRY(mark(2));
    const bool fork2 = fork && h->dx_cus > 0;
    if (fork2) {
      // The gate/up weight gradient (it needs d(gate), d(up)) beside the dX
      // product, with its row-chunk partials in a region of its own: the two
      // fill each other's last rounds and reduce kernels (cfg3 step 2.24-2.25
      // -> 2.22-2.23 ms with dX on 128 of 256 CUs; 96: 2.26, 160: 2.23).
      HIP_TRY(hipEventRecord(h->fork_ev, st));
      HIP_TRY(hipStreamWaitEvent(h->side, h->fork_ev, 0));
      HIP_TRY((launch_wgrad<ActT, 1>(xg, C, C, gu, 2 * Hp, 2 * Hp, counts, E, g + h->g_off[2],
                                     g + h->g_off[4], H, (size_t)C * H, C, H, g + h->g_off[3],
                                     g + h->g_off[5], (size_t)H, A, (float*)(ws + L.wg_part2),
                                     wpart_bytes, wbpart, wbpart_bytes, h->num_cus, store,
                                     h->side)));
      HIP_TRY(hipEventRecord(h->join_ev, h->side));
      gateup_done = true;
    }
    HIP_TRY(launch_gemm_dma<kEpiDown>((const bf16_t*)gu, (const bf16_t*)wgub, nullptr, nullptr,
                                      counts, E, 2 * Hp, Cp, C, 0, (bf16_t*)ob, C, mt,
                                      (float*)(ws + L.partials), fork2 ? h->dx_cus : h->num_cus,
                                      nullptr, 0, st));
  } else if (small_m(h, N)) {
    const int mt = (A + 31) / 32 + E;
    HIP_TRY((launch_grouped_gemm<32, 256, 1, 4, bf16_t, bf16_t, kEpiSwigluBwd, bf16_t>(
        dgo, wdb, nullptr, nullptr, nullptr, counts, E, C, h->Hq, Hp, 0, gu, 2 * Hp, mt, gu,
        2 * Hp, st)));
    HIP_TRY(mark(2));
    HIP_TRY((launch_grouped_gemm<32, 256, 1, 4, bf16_t, bf16_t, kEpiDown, bf16_t>(
        gu, wgub, nullptr, nullptr, nullptr, counts, E, 2 * Hp, Cp, C, 0, ob, C, mt, nullptr, 0,
        st)));
  } else {
    const int mt = (A + 127) / 128 + E;
    HIP_TRY((launch_grouped_gemm<128, 128, 2, 2, bf16_t, bf16_t, kEpiSwigluBwd, bf16_t>(
        dgo, wdb, nullptr, nullptr, nullptr, counts, E, C, h->Hq, Hp, 0, gu, 2 * Hp, mt, gu,
        2 * Hp, st)));
    HIP_TRY(mark(2));
    HIP_TRY((launch_grouped_gemm<128, 128, 2, 2, bf16_t, bf16_t, kEpiDown, bf16_t>(
        gu, wgub, nullptr, nullptr, nullptr, counts, E, 2 * Hp, Cp, C, 0, ob, C, mt, nullptr, 0,
        st)));
  }
  HIP_TRY(mark(3));
  if (!down_done)
    if (int rc = down_wgrad(st)) return rc;
  HIP_TRY(mark(4));
  if (!gateup_done)
    HIP_TRY((launch_wgrad<ActT, 1>(xg, C, C, gu, 2 * Hp, 2 * Hp, counts, E, g + h->g_off[2],
                                   g + h->g_off[4], H, (size_t)C * H, C, H, g + h->g_off[3],
                                   g + h->g_off[5], (size_t)H, A, wpart, wpart_bytes, wbpart,
                                   wbpart_bytes, h->num_cus, store, st)));
  HIP_TRY(mark(5));
  HIP_TRY(launch_token_bwd<ActT>(ob, slot_of, idx, dtp, probs, counts, h->wrt, N, C, E, k, dx,
                                 dlog, st));
  HIP_TRY(mark(6));
  HIP_TRY(launch_router_wgrad<ActT>(x, dlog, N, C, E, (float*)(ws + L.rw_part),
                                    (float*)(ws + L.rw_part_b), g + h->g_off[0], g + h->g_off[1],
                                    store, rstd, gamma, st));
  if (gateup_done) HIP_TRY(hipStreamWaitEvent(st, h->join_ev, 0));
  h->grad_zero = false;
  if (h->padded()) HIP_TRY(launch_copy_cols<ActT>(dx, C, dx_out, Cx, N, Cx, Cx, st));
  HIP_TRY(mark(7));
  if (prof) ++h->prof_b_count;
  return MGPT_OK;
}

// The forward for the handle's (boundary, compute) dtype pair.
int dispatch_forward(mgpt_moe* h, const void* x, void* y, int N, char* ws, bool train,
                     hipStream_t st, BlockArgs blk) {
  if (h->act == MGPT_DTYPE_F32)
    return forward_impl<float, float>(h, (const float*)x, (float*)y, N, ws, train, st, blk);
  if (h->io == MGPT_DTYPE_F32)
    return forward_impl<float, bf16_t>(h, (const float*)x, (float*)y, N, ws, train, st, blk);
  return forward_impl<bf16_t, bf16_t>(h, (const bf16_t*)x, (bf16_t*)y, N, ws, train, st, blk);
}

// Shared argument checks of the forward entry points.
int check_forward_args(const mgpt_moe* h, const void* x, const void* y, int num_tokens,
                       const void* workspace, size_t workspace_bytes, bool train) {
  if (!h) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle");
  if (!h->loaded) return fail(MGPT_ERR_NOT_READY, "parameters not loaded");
  if (num_tokens < 0) return fail(MGPT_ERR_INVALID_ARGUMENT, "negative num_tokens");
  if (num_tokens == 0) return MGPT_OK;
  if (!x || !y || !workspace) return fail(MGPT_ERR_INVALID_ARGUMENT, "null x, y or workspace");
  if (((uintptr_t)x | (uintptr_t)y) % 16 != 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "x and y must be 16-byte aligned");
  if ((uintptr_t)workspace % kAlign != 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "workspace must be %zu-byte aligned", kAlign);
  const size_t need = h->layout(num_tokens, train).total;
  if (workspace_bytes < need)
    return fail(MGPT_ERR_WORKSPACE_TOO_SMALL, "workspace %zu bytes < required %zu",
                workspace_bytes, need);
  const size_t xbytes = (size_t)num_tokens * h->Cx * h->io_bytes();
  if ((const char*)x < (const char*)y + xbytes && (const char*)y < (const char*)x + xbytes)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "y must not overlap x");
  return MGPT_OK;
}

// Where parameter i's gradient lives in the handle's buffer: rows x cols
// floats at offset off with leading dimension ld (the buffers are at the
// padded width C; the caller's tensors at Cx, so [C][*] gradients give their
// first Cx rows and W_down's [H][C] the first Cx columns of each row).
struct GradPiece {
  size_t off;
  int rows, cols, ld;
};

GradPiece grad_piece(const mgpt_moe* h, int i) {
  const size_t C = h->C, H = h->H, E = h->E;
  const int Cx = h->Cx;
  if (i == 0) return {h->g_off[0], Cx, (int)E, (int)E};
  if (i == 1) return {h->g_off[1], 1, (int)E, (int)E};
  const size_t e = (size_t)(i - 2) / 6;
  switch ((i - 2) % 6) {
    case 0: return {h->g_off[2] + e * C * H, Cx, (int)H, (int)H};
    case 1: return {h->g_off[3] + e * H, 1, (int)H, (int)H};
    case 2: return {h->g_off[4] + e * C * H, Cx, (int)H, (int)H};
    case 3: return {h->g_off[5] + e * H, 1, (int)H, (int)H};
    case 4: return {h->g_off[6] + e * H * C, (int)H, Cx, (int)C};
    default: return {h->g_off[7] + e * C, 1, Cx, Cx};
  }
}

int check_grad_args(const mgpt_moe* h, float* const* grads, int num_params) {
  if (!h || !grads) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle or grads");
  if (num_params != 2 + 6 * h->E)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "expected %d gradients (2 + 6*E), got %d",
                2 + 6 * h->E, num_params);
  for (int i = 0; i < num_params; ++i)
    if (!grads[i]) return fail(MGPT_ERR_INVALID_ARGUMENT, "gradient %d is null", i);
  if (!trainable(h))
    return fail(MGPT_ERR_UNSUPPORTED, "training needs weight dtype == activation dtype");
  return MGPT_OK;
}

}  // namespace

extern "C" {

int mgpt_moe_forward(mgpt_moe* h, const void* x, void* y, int num_tokens, void* workspace,
                     size_t workspace_bytes, void* stream) {
  if (int rc = check_forward_args(h, x, y, num_tokens, workspace, workspace_bytes, false))
    return rc;
  if (num_tokens == 0) return MGPT_OK;
  HIP_TRY(hipSetDevice(h->device));
  hipStream_t st = (hipStream_t)stream;
  return dispatch_forward(h, x, y, num_tokens, (char*)workspace, false, st, BlockArgs());
}

int mgpt_moe_forward_noalloc(mgpt_moe* h, const void* x, void* y, int num_tokens, void* stream) {
  if (!h) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle");
  if (num_tokens < 0) return fail(MGPT_ERR_INVALID_ARGUMENT, "negative num_tokens");
  const size_t need = h->layout(num_tokens).total;
  if (need > (size_t)MGPT_MOE_NOALLOC_SCRATCH_BYTES)
    return fail(MGPT_ERR_WORKSPACE_TOO_SMALL,
                "%d tokens need %zu workspace bytes; the built-in scratch holds %zu "
                "(use mgpt_moe_forward with a caller workspace)",
                num_tokens, need, (size_t)MGPT_MOE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_address(h->device, &ws)) return rc;
  if (int rc = check_forward_args(h, x, y, num_tokens, ws, MGPT_MOE_NOALLOC_SCRATCH_BYTES, false))
    return rc;
  if (num_tokens == 0) return MGPT_OK;
  HIP_TRY(hipSetDevice(h->device));
  return dispatch_forward(h, x, y, num_tokens, (char*)ws, false, (hipStream_t)stream,
                          BlockArgs());
}

int mgpt_moe_forward_block(mgpt_moe* h, const void* x, const float* gamma, float eps, void* out,
                           int num_tokens, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (int rc = check_forward_args(h, x, out, num_tokens, workspace, workspace_bytes, false))
    return rc;
  if (num_tokens == 0) return MGPT_OK;
  if (!gamma) return fail(MGPT_ERR_INVALID_ARGUMENT, "null gamma");
  if (!(eps >= 0.0f)) return fail(MGPT_ERR_INVALID_ARGUMENT, "eps must be >= 0");
  HIP_TRY(hipSetDevice(h->device));
  hipStream_t st = (hipStream_t)stream;
  BlockArgs blk;
  blk.gamma = gamma;
  blk.eps = eps;
  return dispatch_forward(h, x, out, num_tokens, (char*)workspace, false, st, blk);
}

int mgpt_moe_get_rstd(const mgpt_moe* h, int num_tokens, void* workspace, float** rstd) {
  if (!h || !workspace || !rstd || num_tokens < 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "null argument or negative num_tokens");
  *rstd = (float*)((char*)workspace + h->layout(num_tokens).rstd);
  return MGPT_OK;
}

int mgpt_moe_train_workspace_bytes(const mgpt_moe* h, int num_tokens, size_t* bytes) {
  if (!h || !bytes || num_tokens < 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle/bytes or negative num_tokens");
  *bytes = h->layout(num_tokens, true).total;
  return MGPT_OK;
}

int mgpt_moe_forward_train(mgpt_moe* h, const void* x, void* y, int num_tokens, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (int rc = check_forward_args(h, x, y, num_tokens, workspace, workspace_bytes, true))
    return rc;
  if (!trainable(h))
    return fail(MGPT_ERR_UNSUPPORTED, "training needs weight dtype == activation dtype");
  if (num_tokens == 0) return MGPT_OK;
  HIP_TRY(hipSetDevice(h->device));
  hipStream_t st = (hipStream_t)stream;
  return dispatch_forward(h, x, y, num_tokens, (char*)workspace, true, st, BlockArgs());
}

namespace {

// mgpt_moe_backward and, with gamma / dgamma set, mgpt_moe_backward_block.
int backward_entry(mgpt_moe* h, const void* x, const void* dy, void* dx, int num_tokens,
                   void* workspace, size_t workspace_bytes, void* stream,
                   const float* gamma = nullptr, float* dgamma = nullptr) {
  if (!h) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle");
  if (!h->loaded) return fail(MGPT_ERR_NOT_READY, "parameters not loaded");
  if (!trainable(h))
    return fail(MGPT_ERR_UNSUPPORTED, "training needs weight dtype == activation dtype");
  if (num_tokens < 0) return fail(MGPT_ERR_INVALID_ARGUMENT, "negative num_tokens");
  if (num_tokens == 0) return MGPT_OK;
  if (!x || !dy || !dx || !workspace)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "null x, dy, dx or workspace");
  if (((uintptr_t)x | (uintptr_t)dy | (uintptr_t)dx) % 16 != 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "x, dy and dx must be 16-byte aligned");
  if ((uintptr_t)workspace % kAlign != 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "workspace must be %zu-byte aligned", kAlign);
  const size_t need = h->layout(num_tokens, true).total;
  if (workspace_bytes < need)
    return fail(MGPT_ERR_WORKSPACE_TOO_SMALL, "workspace %zu bytes < required %zu",
                workspace_bytes, need);
  const size_t nbytes = (size_t)num_tokens * h->Cx * h->io_bytes();
  auto overlap = [&](const void* a, const void* b) {
    return (const char*)a < (const char*)b + nbytes && (const char*)b < (const char*)a + nbytes;
  };
  if (overlap(dx, dy) || overlap(dx, x))
    return fail(MGPT_ERR_INVALID_ARGUMENT, "dx must not overlap x or dy");
  HIP_TRY(hipSetDevice(h->device));
  hipStream_t st = (hipStream_t)stream;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(st, &cap));
  if (cap != hipStreamCaptureStatusNone) {
    // A graph replays the mode it was captured in, so a captured backward
    // always adds: zeros still pending from zero_grad are written first
    // (into the graph), and later zero_grads clear the buffer on the stream.
    if (int rc = materialize_grad(h, st)) return rc;
    h->bwd_captured = true;
  }
  char* ws = (char*)workspace;
  float* nrm_part = (float*)(ws + h->layout(num_tokens, true).nrm_part);
  if (h->act == MGPT_DTYPE_BF16) {
    if (int rc = backward_impl<bf16_t>(h, (const bf16_t*)x, (const bf16_t*)dy, (bf16_t*)dx,
                                       num_tokens, ws, st, gamma))
      return rc;
    // dx holds the gradient of the normalised rows: ln2 backward + residual
    if (gamma)
      HIP_TRY(launch_rmsnorm_bwd<bf16_t>((const bf16_t*)x, (bf16_t*)dx, (const bf16_t*)dy,
                                         (const float*)(ws + h->layout(num_tokens).rstd), gamma,
                                         num_tokens, h->Cx, nrm_part, dgamma, st));
    return MGPT_OK;
  }
  if (int rc = backward_impl<float>(h, (const float*)x, (const float*)dy, (float*)dx, num_tokens,
                                    ws, st, gamma))
    return rc;
  if (gamma)
    HIP_TRY(launch_rmsnorm_bwd<float>((const float*)x, (float*)dx, (const float*)dy,
                                      (const float*)(ws + h->layout(num_tokens).rstd), gamma,
                                      num_tokens, h->Cx, nrm_part, dgamma, st));
  return MGPT_OK;
}

}  // namespace

int mgpt_moe_backward(mgpt_moe* h, const void* x, const void* dy, void* dx, int num_tokens,
                      void* workspace, size_t workspace_bytes, void* stream) {
  return backward_entry(h, x, dy, dx, num_tokens, workspace, workspace_bytes, stream);
}

int mgpt_moe_forward_block_train(mgpt_moe* h, const void* x, const float* gamma, float eps,
                                 void* out, int num_tokens, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (int rc = check_forward_args(h, x, out, num_tokens, workspace, workspace_bytes, true))
    return rc;
  if (!trainable(h))
    return fail(MGPT_ERR_UNSUPPORTED, "training needs weight dtype == activation dtype");
  if (num_tokens == 0) return MGPT_OK;
  if (!gamma) return fail(MGPT_ERR_INVALID_ARGUMENT, "null gamma");
  if (!(eps >= 0.0f)) return fail(MGPT_ERR_INVALID_ARGUMENT, "eps must be >= 0");
  HIP_TRY(hipSetDevice(h->device));
  BlockArgs blk;
  blk.gamma = gamma;
  blk.eps = eps;
  return dispatch_forward(h, x, out, num_tokens, (char*)workspace, true, (hipStream_t)stream,
                          blk);
}

int mgpt_moe_backward_block(mgpt_moe* h, const void* x, const float* gamma, const void* dout,
                            void* dx, float* dgamma, int num_tokens, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!gamma || !dgamma) return fail(MGPT_ERR_INVALID_ARGUMENT, "null gamma or dgamma");
  return backward_entry(h, x, dout, dx, num_tokens, workspace, workspace_bytes, stream, gamma,
                        dgamma);
}

int mgpt_moe_zero_grad(mgpt_moe* h, void* stream) {
  if (!h) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle");
  if (!trainable(h))
    return fail(MGPT_ERR_UNSUPPORTED, "training needs weight dtype == activation dtype");
  HIP_TRY(hipSetDevice(h->device));
  if (int rc = ensure_grad(h)) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(st, &cap));
  if (cap != hipStreamCaptureStatusNone || h->bwd_captured) {
    // under capture, or once a captured (adding) backward exists: clear the
    // buffer on the stream, a fill kernel (graph-safe)
    HIP_TRY(launch_fill_zero(h->grad, h->g_total, st));
    h->grad_zero = false;
    return MGPT_OK;
  }
  // eager: nothing is enqueued, the next backward stores instead of adding
  h->grad_zero = true;
  return MGPT_OK;
}

int mgpt_moe_get_gradients(mgpt_moe* h, float* const* grads, int num_params, int grads_on_device,
                           void* stream) {
  if (int rc = check_grad_args(h, grads, num_params)) return rc;
  HIP_TRY(hipSetDevice(h->device));
  hipStream_t st = (hipStream_t)stream;
  if (int rc = materialize_grad(h, st)) return rc;
  const hipMemcpyKind kind = grads_on_device ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost;
  for (int i = 0; i < num_params; ++i) {
    const GradPiece g = grad_piece(h, i);
    HIP_TRY(hipMemcpy2DAsync(grads[i], sizeof(float) * g.cols, h->grad + g.off,
                             sizeof(float) * g.ld, sizeof(float) * g.cols, g.rows, kind, st));
  }
  HIP_TRY(hipStreamSynchronize(st));
  return MGPT_OK;
}

int mgpt_moe_accumulate_gradients(mgpt_moe* h, float* const* grads, int num_params,
                                  int grads_on_device, void* stream) {
  if (int rc = check_grad_args(h, grads, num_params)) return rc;
  HIP_TRY(hipSetDevice(h->device));
  hipStream_t st = (hipStream_t)stream;
  if (int rc = materialize_grad(h, st)) return rc;
  if (grads_on_device) {
    AddJobs jobs{};
    size_t max_elems = 0;
    for (int i = 0; i < num_params; ++i) {
      const GradPiece g = grad_piece(h, i);
      const int j = jobs.n++;
      jobs.dst[j] = grads[i];
      jobs.off[j] = g.off;
      jobs.rows[j] = g.rows;
      jobs.cols[j] = g.cols;
      jobs.lds[j] = g.ld;
      max_elems = std::max(max_elems, (size_t)g.rows * g.cols);
      if (jobs.n == AddJobs::kMax || i == num_params - 1) {
        HIP_TRY(launch_add_jobs(h->grad, jobs, max_elems, st));
        jobs.n = 0;
        max_elems = 0;
      }
    }
    return MGPT_OK;
  }
  // Host destinations: the pieces in buffer order, gathered into windows of
  // consecutive pieces of at most kWindow floats (a larger piece is a window
  // of its own); one copy and one wait per window, then each piece of the
  // window is added in place.  A few waits in all (one at the shapes of the
  // tests) instead of one per parameter, and a bounded host buffer.
  constexpr size_t kWindow = (size_t)64 << 20;   // floats (256 MB)
  std::vector<int> order(num_params);
  for (int i = 0; i < num_params; ++i) order[i] = i;
  std::sort(order.begin(), order.end(),
            [&](int a, int b) { return grad_piece(h, a).off < grad_piece(h, b).off; });
  auto span = [&](int i) {
    const GradPiece g = grad_piece(h, i);
    return (size_t)(g.rows - 1) * g.ld + g.cols;   // floats from g.off to the piece's end
  };
  std::vector<float> tmp;
  for (int a = 0; a < num_params;) {
    const size_t w0 = grad_piece(h, order[a]).off;
    int b = a + 1;
    size_t w1 = w0 + span(order[a]);
    while (b < num_params) {
      const GradPiece g = grad_piece(h, order[b]);
      const size_t end = g.off + span(order[b]);
      if (end - w0 > kWindow) break;
      w1 = std::max(w1, end);
      ++b;
    }
    try {
      tmp.resize(w1 - w0);
    } catch (const std::bad_alloc&) {
      return fail(MGPT_ERR_OUT_OF_MEMORY, "host buffer of %zu floats", w1 - w0);
    }
    HIP_TRY(hipMemcpyAsync(tmp.data(), h->grad + w0, sizeof(float) * (w1 - w0),
                           hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    for (int q = a; q < b; ++q) {
      const GradPiece g = grad_piece(h, order[q]);
      float* d = grads[order[q]];
      for (int r = 0; r < g.rows; ++r) {
        const float* srow = tmp.data() + (g.off - w0) + (size_t)r * g.ld;
        float* drow = d + (size_t)r * g.cols;
        for (int c = 0; c < g.cols; ++c) drow[c] = drow[c] + srow[c];
      }
    }
    a = b;
  }
  return MGPT_OK;
}

int mgpt_moe_get_routing(const mgpt_moe* h, int num_tokens, void* workspace,
                         mgpt_moe_routing* out) {
  if (!h || !workspace || !out || num_tokens < 0)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "null argument or negative num_tokens");
  const Layout L = h->layout(num_tokens);
  char* ws = (char*)workspace;
  out->topk_idx = (int32_t*)(ws + L.topk_idx);
  out->topk_p = (float*)(ws + L.topk_p);
  out->counts = (int32_t*)(ws + L.counts);
  out->perm = (int32_t*)(ws + L.perm);
  out->slot_of = (int32_t*)(ws + L.slot_of);
  return MGPT_OK;
}

int mgpt_moe_expert_counts(mgpt_moe* h, int32_t* host_counts, int num_experts) {
  if (!h || !host_counts || num_experts != h->E)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "null argument or num_experts != E");
  if (!h->done_valid || !h->last_counts)
    return fail(MGPT_ERR_NOT_READY, "no forward has been run");
  HIP_TRY(hipEventSynchronize(h->done));
  HIP_TRY(hipMemcpy(host_counts, h->last_counts, sizeof(int32_t) * h->E, hipMemcpyDeviceToHost));
  return MGPT_OK;
}

int mgpt_moe_set_profiling(mgpt_moe* h, int enable) {
  if (!h) return fail(MGPT_ERR_INVALID_ARGUMENT, "null handle");
  if (enable < 0 || enable > 2) return fail(MGPT_ERR_INVALID_ARGUMENT, "enable must be 0, 1 or 2");
  h->profiling = enable != 0;
  h->prof_gemm_only = enable == 2;
  h->prof_count = 0;
  h->prof_b_count = 0;
  return MGPT_OK;
}

int mgpt_moe_backward_stage_times(mgpt_moe* h, float* ms, int n) {
  constexpr int S = MGPT_MOE_NUM_BWD_STAGES;
  if (!h || !ms || n < S) return fail(MGPT_ERR_INVALID_ARGUMENT, "need room for %d stage times", S);
  if (h->prof_b_count == 0) return fail(MGPT_ERR_NOT_READY, "no profiled backward has been run");
  const int slots = std::min(h->prof_b_count, mgpt_moe::kProfSlots);
  const int last = (h->prof_b_count - 1) % mgpt_moe::kProfSlots;
  HIP_TRY(hipEventSynchronize(h->evb[last][S]));
  for (int i = 0; i < S; ++i) {
    double sum = 0.0;
    for (int sl = 0; sl < slots; ++sl) {
      float t = 0.0f;
      HIP_TRY(hipEventElapsedTime(&t, h->evb[sl][i], h->evb[sl][i + 1]));
      sum += t;
    }
    ms[i] = (float)(sum / slots);
  }
  if (n > S) ms[S] = (float)slots;
  return MGPT_OK;
}

int mgpt_moe_stage_times(mgpt_moe* h, float* ms, int n) {
  if (!h || !ms || n < MGPT_MOE_NUM_STAGES)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "need room for %d stage times", MGPT_MOE_NUM_STAGES);
  if (h->prof_count == 0) return fail(MGPT_ERR_NOT_READY, "no profiled forward has been run");
  const int slots = std::min(h->prof_count, mgpt_moe::kProfSlots);
  const int last = (h->prof_count - 1) % mgpt_moe::kProfSlots;
  HIP_TRY(hipEventSynchronize(h->ev[last][h->prof_gemm_only ? 3 : MGPT_MOE_NUM_STAGES]));
  for (int i = 0; i < MGPT_MOE_NUM_STAGES; ++i) {
    if (h->prof_gemm_only && i != 2) {
      ms[i] = -1.0f;   // not recorded in this mode
      continue;
    }
    double sum = 0.0;
    for (int s = 0; s < slots; ++s) {
      float t = 0.0f;
      HIP_TRY(hipEventElapsedTime(&t, h->ev[s][i], h->ev[s][i + 1]));
      sum += t;
    }
    ms[i] = (float)(sum / slots);
  }
  if (n > MGPT_MOE_NUM_STAGES) ms[MGPT_MOE_NUM_STAGES] = (float)slots;
  return MGPT_OK;
}

int mgpt_moe_export_fp8(const mgpt_moe* h, int expert, int which, uint8_t* q_host,
                        float* scale_host) {
  if (!h || !q_host || !scale_host || expert < 0 || expert >= h->E || which < 0 || which > 2)
    return fail(MGPT_ERR_INVALID_ARGUMENT, "bad arguments");
  if (h->wdt != MGPT_DTYPE_FP8_E4M3) return fail(MGPT_ERR_INVALID_ARGUMENT, "not an fp8 handle");
  if (!h->loaded) return fail(MGPT_ERR_NOT_READY, "parameters not loaded");
  const int C = h->C, Cx = h->Cx, H = h->H, Hp = h->Hp, Cp = h->Cp;
  if (which < 2) {
    std::vector<uint8_t> q((size_t)2 * Hp * C);
    std::vector<float> s((size_t)2 * Hp);
    HIP_TRY(hipMemcpy(q.data(), (const uint8_t*)h->wgu + (size_t)expert * 2 * Hp * C, q.size(),
                      hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(s.data(), h->sgu + (size_t)expert * 2 * Hp, sizeof(float) * s.size(),
                      hipMemcpyDeviceToHost));
    for (int n = 0; n < H; ++n) {
      const int prow = (n / 32) * 64 + (n % 32) + 32 * which;
      scale_host[n] = s[prow];
      for (int c = 0; c < Cx; ++c) q_host[(size_t)c * H + n] = q[(size_t)prow * C + c];
    }
  } else {
    std::vector<uint8_t> q((size_t)Cp * Hp);
    std::vector<float> s((size_t)Cp);
    HIP_TRY(hipMemcpy(q.data(), (const uint8_t*)h->wd + (size_t)expert * Cp * Hp, q.size(),
                      hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(s.data(), h->sd + (size_t)expert * Cp, sizeof(float) * Cp,
                      hipMemcpyDeviceToHost));
    for (int c = 0; c < Cx; ++c) {
      scale_host[c] = s[c];
      for (int n = 0; n < H; ++n) q_host[(size_t)n * Cx + c] = q[(size_t)c * Hp + n];
    }
  }
  return MGPT_OK;
}

int mgpt_moe_device_expf(const float* d_in, float* d_out, int n, void* stream) {
  if (n < 0 || (n > 0 && (!d_in || !d_out)))
    return fail(MGPT_ERR_INVALID_ARGUMENT, "bad arguments");
  HIP_TRY(launch_expf_probe(d_in, d_out, n, (hipStream_t)stream));
  return MGPT_OK;
}

}  // extern "C"
