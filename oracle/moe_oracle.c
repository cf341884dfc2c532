/*
 * moe_oracle.c -- CPU restatement of mgpt's MoE block forward.
 *
 * TEST INFRASTRUCTURE ONLY (see moe_oracle.h): the checker for the HIP path,
 * never part of it.  Build with -O2/-O3 and -ffp-contract=off; FMA
 * contraction changes the bits (the reference is pinned with the same flag).
 *
 * Pinning (each function has at least one check that a plausible mistake
 * fails; tests/test_oracle.py):
 *   - all functions: bit-for-bit against the compiled reference on committed
 *     golden fixtures (tests/golden/, made by tests/golden/make_golden.py
 *     from oracle/_ref/ref_driver);
 *   - router/softmax/topk/dispatch/scatter: closed forms and brute force
 *     (one-hot W_r, softmax([1,2,3]), clamp and NaN cases, stable sort);
 *   - experts: fp64 textbook SwiGLU within an error bound, and the
 *     "all experts identical" invariant y = (sum_j p_j) * FFN(x).
 */
#include "moe_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Reference: std::exp(float) in utils/Tensor.cpp:873 (softmax) and :2000
 * (SwiGLU) resolves to glibc expf. */
float oracle_expf(float x) { return expf(x); }

void oracle_expf_array(const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = expf(in[i]);
}

/* utils/Tensor.cpp:567-577 (matmul2d_raw, i-k-j order) reached from
 * layers/LinearLayer.cpp:23-28 via Tensor::matmul_into :1231-1249, then the
 * bias add of add_broadcast_in_place :1499-1507 -> operator+ :331-342.  Per
 * output element: acc = 0; acc += a_k * w_kj for k ascending; acc + b_j. */
static void linear_row(int K, int Nout, const float* a, const float* W,
                       const float* b, float* out) {
  for (int j = 0; j < Nout; ++j) out[j] = 0.0f;
  for (int kk = 0; kk < K; ++kk) {
    const float av = a[kk];
    const float* wr = W + (size_t)kk * Nout;
    for (int j = 0; j < Nout; ++j) out[j] += av * wr[j];
  }
  for (int j = 0; j < Nout; ++j) out[j] = out[j] + b[j];
}

void oracle_router_logits(int N, int C, int E, const float* x, const float* Wr,
                          const float* br, float* logits) {
  for (int i = 0; i < N; ++i)
    linear_row(C, E, x + (size_t)i * C, Wr, br, logits + (size_t)i * E);
}

/* utils/Tensor.cpp:850-883 (Tensor::softmax, CPU branch), reached via
 * softmax_into :1486-1497 from layers/MoELayer.cpp:55.  max by strict '>'
 * starting from element 0; sequential sum; inv = 1/fmax(sum,1e-15);
 * p = fmin(fmax(e*inv, 1e-7), 1). */
void oracle_softmax(int N, int E, const float* logits, float* probs) {
  for (int i = 0; i < N; ++i) {
    const float* l = logits + (size_t)i * E;
    float* p = probs + (size_t)i * E;
    float m = l[0];
    for (int v = 1; v < E; ++v)
      if (l[v] > m) m = l[v];
    float s = 0.0f;
    for (int v = 0; v < E; ++v) {
      float e = expf(l[v] - m);
      p[v] = e;
      s += e;
    }
    float inv = 1.0f / fmaxf(s, 1e-15f);
    for (int v = 0; v < E; ++v) p[v] = fminf(fmaxf(p[v] * inv, 1e-7f), 1.0f);
  }
}

/* utils/Tensor.cpp:1296-1334 (Tensor::top_k_into, CPU branch).  Sentinels
 * -1e9 / -1; insert when p > last slot; shift while p > previous slot.  Ties
 * keep the lower expert id first. */
void oracle_topk(int N, int E, int k, const float* probs, int32_t* idx, float* topp) {
  for (int i = 0; i < N; ++i) {
    const float* p = probs + (size_t)i * E;
    float* ov = topp + (size_t)i * k;
    int32_t* oi = idx + (size_t)i * k;
    for (int j = 0; j < k; ++j) { ov[j] = -1e9f; oi[j] = -1; }
    for (int e = 0; e < E; ++e) {
      float v = p[e];
      if (v > ov[k - 1]) {
        int pos = k - 1;
        while (pos > 0 && v > ov[pos - 1]) {
          ov[pos] = ov[pos - 1];
          oi[pos] = oi[pos - 1];
          --pos;
        }
        ov[pos] = v;
        oi[pos] = e;
      }
    }
  }
}

/* utils/Tensor.cpp:1336-1352 (histogram, skipping ids outside [0,E)),
 * layers/MoELayer.cpp:67-80 (host exclusive scan into offsets) and
 * utils/Tensor.cpp:1354-1383 (gather: slot = offsets[e]++ for flat ids in
 * ascending order, map[slot] = flat id). */
void oracle_dispatch(int N, int E, int k, const int32_t* idx, int32_t* counts,
                     int32_t* offsets, int32_t* perm) {
  const int A = N * k;
  int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E > 0 ? E : 1));
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int i = 0; i < A; ++i)
    if (idx[i] >= 0 && idx[i] < E) counts[idx[i]] += 1;
  int run = 0;
  for (int e = 0; e < E; ++e) { offsets[e] = run; cur[e] = run; run += counts[e]; }
  for (int i = 0; i < A; ++i) {
    int e = idx[i];
    if (e >= 0) perm[cur[e]++] = i;
  }
  free(cur);
}

/* One SwiGLU expert on one row: layers/SwiGLU.cpp:23-50 with the Linear
 * layers of layers/LinearLayer.cpp:23-28 and the CPU swiglu_forward of
 * utils/Tensor.cpp:1986-2004: h = (g / (1 + exp(-g))) * u. */
static void expert_row(int C, int H, const float* xrow, const float* Wg,
                       const float* bg, const float* Wu, const float* bu,
                       const float* Wd, const float* bd, float* g, float* u,
                       float* out) {
  linear_row(C, H, xrow, Wg, bg, g);
  linear_row(C, H, xrow, Wu, bu, u);
  for (int h = 0; h < H; ++h) {
    float gv = g[h];
    float gs = gv / (1.0f + expf(-gv));
    g[h] = gs * u[h];
  }
  linear_row(H, C, g, Wd, bd, out);
}

#define EXPERT_PTRS(e)                                                     \
  Wg + (size_t)(e) * C * H, bg + (size_t)(e) * H, Wu + (size_t)(e) * C * H, \
      bu + (size_t)(e) * H, Wd + (size_t)(e) * H * C, bd + (size_t)(e) * C

/* layers/MoELayer.cpp:28-128 (forward_into), CPU path. */
int oracle_moe_forward(int N, int C, int H, int E, int k, const float* x,
                       const float* Wr, const float* br, const float* Wg,
                       const float* bg, const float* Wu, const float* bu,
                       const float* Wd, const float* bd, float* y,
                       float* logits, float* probs, int32_t* idx, float* topp,
                       int32_t* counts, int32_t* offsets, int32_t* perm) {
  if (N < 0 || C <= 0 || H <= 0 || E <= 0 || k <= 0 || k > E) return 1;
  const size_t A = (size_t)N * k;
  float* L = logits ? logits : (float*)malloc(sizeof(float) * ((size_t)N * E + 1));
  float* P = probs ? probs : (float*)malloc(sizeof(float) * ((size_t)N * E + 1));
  int32_t* I = idx ? idx : (int32_t*)malloc(sizeof(int32_t) * (A + 1));
  float* TP = topp ? topp : (float*)malloc(sizeof(float) * (A + 1));
  int32_t* CN = counts ? counts : (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int32_t* OF = offsets ? offsets : (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int32_t* PM = perm ? perm : (int32_t*)malloc(sizeof(int32_t) * (A + 1));
  float* g = (float*)malloc(sizeof(float) * (size_t)H);
  float* u = (float*)malloc(sizeof(float) * (size_t)H);
  float* o = (float*)malloc(sizeof(float) * (size_t)C);

  oracle_router_logits(N, C, E, x, Wr, br, L);
  oracle_softmax(N, E, L, P);
  oracle_topk(N, E, k, P, I, TP);
  oracle_dispatch(N, E, k, I, CN, OF, PM);

  /* Experts in id order over expert-contiguous slots (layers/MoELayer.cpp:
   * 94-118), then the slot-ordered gate-weighted scatter of utils/Tensor.cpp:
   * 1385-1408 into a zero-filled output (layers/MoELayer.cpp:121-123). */
  if (y) {
    memset(y, 0, sizeof(float) * (size_t)N * C);
    for (size_t slot = 0; slot < A; ++slot) {
      int flat = PM[slot];
      int t = flat / k;
      int e = I[flat];
      expert_row(C, H, x + (size_t)t * C, EXPERT_PTRS(e), g, u, o);
      float pr = TP[flat];
      float* yr = y + (size_t)t * C;
      for (int c = 0; c < C; ++c) yr[c] += o[c] * pr;
    }
  }
  if (!logits) free(L);
  if (!probs) free(P);
  if (!idx) free(I);
  if (!topp) free(TP);
  if (!counts) free(CN);
  if (!offsets) free(OF);
  if (!perm) free(PM);
  free(g); free(u); free(o);
  return 0;
}

/* Per-token form of the scatter (utils/Tensor.cpp:1385-1408): slots are
 * expert-major, so a token's k contributions arrive in ascending expert id
 * order; each is o*p rounded, added to a running sum that starts at 0. */
int oracle_moe_tokens(int C, int H, int E, int k, int n_sel, const int32_t* tok,
                      const float* x, const int32_t* idx, const float* topp,
                      const float* Wg, const float* bg, const float* Wu,
                      const float* bu, const float* Wd, const float* bd,
                      float* y_sel) {
  float* g = (float*)malloc(sizeof(float) * (size_t)H);
  float* u = (float*)malloc(sizeof(float) * (size_t)H);
  float* o = (float*)malloc(sizeof(float) * (size_t)C);
  int order[64];
  if (k > 64) return 1;
  for (int s = 0; s < n_sel; ++s) {
    int t = tok[s];
    const int32_t* it = idx + (size_t)t * k;
    for (int j = 0; j < k; ++j) order[j] = j;
    for (int a = 1; a < k; ++a) { /* insertion sort of choices by expert id */
      int v = order[a], b = a;
      while (b > 0 && it[order[b - 1]] > it[v]) { order[b] = order[b - 1]; --b; }
      order[b] = v;
    }
    float* yr = y_sel + (size_t)s * C;
    for (int c = 0; c < C; ++c) yr[c] = 0.0f;
    for (int a = 0; a < k; ++a) {
      int j = order[a];
      int e = it[j];
      if (e < 0 || e >= E) continue;
      expert_row(C, H, x + (size_t)t * C, EXPERT_PTRS(e), g, u, o);
      float pr = topp[(size_t)t * k + j];
      for (int c = 0; c < C; ++c) yr[c] += o[c] * pr;
    }
  }
  free(g); free(u); free(o);
  return 0;
}

/* utils/Tensor.cpp:769-802 (rms_norm_into, CPU branch) with scale = 1:
 * ms = sum x^2 sequential; r = 1/sqrt(ms/C + eps); out = (x*r)*1. */
void oracle_rmsnorm(int N, int C, float eps, const float* x, float* out) {
  for (int i = 0; i < N; ++i) {
    const float* xr = x + (size_t)i * C;
    float ms = 0.0f;
    for (int c = 0; c < C; ++c) ms += xr[c] * xr[c];
    float r = 1.0f / sqrtf(ms / C + eps);
    for (int c = 0; c < C; ++c) out[(size_t)i * C + c] = (xr[c] * r) * 1.0f;
  }
}
