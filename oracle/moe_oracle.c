/*
 * moe_oracle.c -- CPU restatement of mgpt's MoE block forward and backward.
 *
 * TEST INFRASTRUCTURE ONLY (see moe_oracle.h): the checker for the HIP path,
 * never part of it.  Build with -O2/-O3 and -ffp-contract=off; FMA
 * contraction changes the bits (the reference is pinned with the same flag).
 *
 * Pinning (each function has at least one check that a plausible mistake
 * fails; tests/test_oracle.py, tests/test_oracle_backward.py):
 *   - all functions: bit-for-bit against the compiled reference on committed
 *     golden fixtures (tests/golden/, made by tests/golden/make_golden.py
 *     from oracle/_ref/ref_driver);
 *   - router/softmax/topk/dispatch/scatter: closed forms and brute force
 *     (one-hot W_r, softmax([1,2,3]), clamp and NaN cases, stable sort);
 *   - experts: fp64 textbook SwiGLU within an error bound, and the
 *     "all experts identical" invariant y = (sum_j p_j) * FFN(x);
 *   - backward: every gradient against float64 central finite differences
 *     of the differentiated loss, plus softmax-Jacobian and routing
 *     invariants.  The ORACLE_PLANT_* macros each build a copy with one
 *     plausible mistake (dropped load-balance term, wrong sign in the SiLU
 *     derivative, ungated expert gradient, dgamma without x_hat, the RMSNorm
 *     backward without its projection term); the tests build those copies
 *     and show that both the golden and the finite-difference checks
 *     reject them.  The shipped build defines none of them;
 *   - block backward (tests/test_oracle_block.py): bit-for-bit against the
 *     reference's TransformerBlock MoE half (ln2 + MoE + residual backward),
 *     and dx1 / dgamma against float64 finite differences.
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

/* Backward of one Linear layer over `rows` rows, utils/Tensor.cpp CPU
 * branches as reached from layers/LinearLayer.cpp:33-80:
 *   db[j] += sum_r dout[r][j]            sum_rows_into :1599-1617, add_grad
 *                                        :638-650 (r ascending from 0)
 *   dW[i][j] += sum_r in[r][i]*dout[r][j] transpose + matmul2d_raw :567-577
 *                                        (i-k-j: the sum runs over r
 *                                        ascending, from 0, then add_grad)
 *   din[r][i] = sum_j dout[r][j]*W[i][j] matmul2d_raw against W^T (j asc.)
 * Input rows are addressed through in_rows[r], so gathered rows need no copy. */
static void linear_backward(int rows, int Kin, int Nout, const float* const* in_rows,
                            const float* dout, const float* W, float* dW,
                            float* db, float* din, float* tmp) {
  for (int j = 0; j < Nout; ++j) tmp[j] = 0.0f;
  for (int r = 0; r < rows; ++r)
    for (int j = 0; j < Nout; ++j) tmp[j] += dout[(size_t)r * Nout + j];
  for (int j = 0; j < Nout; ++j) db[j] += tmp[j];
  for (int i = 0; i < Kin; ++i) {
    for (int j = 0; j < Nout; ++j) tmp[j] = 0.0f;
    for (int r = 0; r < rows; ++r) {
      const float a = in_rows[r][i];
      const float* dr = dout + (size_t)r * Nout;
      for (int j = 0; j < Nout; ++j) tmp[j] += a * dr[j];
    }
    float* wr = dW + (size_t)i * Nout;
    for (int j = 0; j < Nout; ++j) wr[j] += tmp[j];
  }
  for (int r = 0; r < rows; ++r) {
    const float* dr = dout + (size_t)r * Nout;
    float* o = din + (size_t)r * Kin;
    for (int i = 0; i < Kin; ++i) {
      const float* wi = W + (size_t)i * Nout;
      float acc = 0.0f;
      for (int j = 0; j < Nout; ++j) acc += dr[j] * wi[j];
      o[i] = acc;
    }
  }
}

/* layers/MoELayer.cpp:130-223 (backward_into), CPU path, after the forward
 * of :28-128 on the same inputs:
 *   B1 scatter backward, utils/Tensor.cpp:1410-1438: per slot (ascending),
 *      dgo[slot] = dy[t]*p and dp[flat] = sum_c o[slot][c]*dy[t][c];
 *   B2 per expert in id order over its slots (layers/MoELayer.cpp:158-180),
 *      SwiGLU backward layers/SwiGLU.cpp:57-96: down Linear, then the fused
 *      swiglu_backward utils/Tensor.cpp:2006-2030 (sig = 1/(1+exp(-g));
 *      d_up = dd*(g*sig); d_gate = (dd*u)*(sig*(1+g*(1-sig)))), then the gate
 *      and up Linears, and din = d_gate_proj + d_up_proj;
 *   B3 gather backward utils/Tensor.cpp:1440-1460 into a zeroed dx, slots
 *      ascending;
 *   B4 scatter_indices_into :1462-1484: dP[t][idx] = dp (other entries 0);
 *   B5 load-balance term layers/MoELayer.cpp:193-200: dP[t][e] +=
 *      (0.01*E*f_e)/N with f_e = counts[e]/N (operator+ broadcast :331-342);
 *   B6 softmax backward on the clamped probs :885-905: s = sum_e dP*P
 *      (ascending); dL = P*(dP - s);
 *   B7 router Linear backward (as linear_backward);
 *   B8 dx = dx + router_din (Tensor::add_into :1579-1597). */
int oracle_moe_backward(int N, int C, int H, int E, int k, const float* x,
                        const float* Wr, const float* br, const float* Wg,
                        const float* bg, const float* Wu, const float* bu,
                        const float* Wd, const float* bd, const float* dy,
                        float* dx, float* dWr, float* dbr, float* dWg,
                        float* dbg, float* dWu, float* dbu, float* dWd,
                        float* dbd) {
  if (N < 0 || C <= 0 || H <= 0 || E <= 0 || k <= 0 || k > E) return 1;
  const size_t A = (size_t)N * k;
  const size_t NE = (size_t)N * E;
  float* L = (float*)malloc(sizeof(float) * (NE + 1));
  float* P = (float*)malloc(sizeof(float) * (NE + 1));
  int32_t* I = (int32_t*)malloc(sizeof(int32_t) * (A + 1));
  float* TP = (float*)malloc(sizeof(float) * (A + 1));
  int32_t* CN = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int32_t* OF = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int32_t* PM = (int32_t*)malloc(sizeof(int32_t) * (A + 1));
  float* G = (float*)malloc(sizeof(float) * (A * H + 1));   /* gate pre-act */
  float* U = (float*)malloc(sizeof(float) * (A * H + 1));   /* up */
  float* Act = (float*)malloc(sizeof(float) * (A * H + 1)); /* silu(g)*u */
  float* O = (float*)malloc(sizeof(float) * (A * C + 1));   /* expert outputs */
  float* dgo = (float*)malloc(sizeof(float) * (A * C + 1));
  float* dgi = (float*)malloc(sizeof(float) * (A * C + 1));
  float* dTP = (float*)malloc(sizeof(float) * (A + 1));
  float* dD = (float*)malloc(sizeof(float) * (A * H + 1)); /* d(act) */
  float* dGt = (float*)malloc(sizeof(float) * (A * H + 1));
  float* dUp = (float*)malloc(sizeof(float) * (A * H + 1));
  float* dinU = (float*)malloc(sizeof(float) * (A * C + 1));
  float* dP = (float*)malloc(sizeof(float) * (NE + 1));
  float* dL = (float*)malloc(sizeof(float) * (NE + 1));
  float* rdin = (float*)malloc(sizeof(float) * ((size_t)N * C + 1));
  const float** rows = (const float**)malloc(sizeof(float*) * (A + 1));
  const int tmpn = (C > H ? C : H) > E ? (C > H ? C : H) : E;
  float* tmp = (float*)malloc(sizeof(float) * (size_t)tmpn);

  oracle_router_logits(N, C, E, x, Wr, br, L);
  oracle_softmax(N, E, L, P);
  oracle_topk(N, E, k, P, I, TP);
  oracle_dispatch(N, E, k, I, CN, OF, PM);

  /* Forward activations per slot (the caches the reference keeps). */
  for (size_t slot = 0; slot < A; ++slot) {
    const int t = PM[slot] / k, e = I[PM[slot]];
    float* g = G + slot * H;
    float* u = U + slot * H;
    float* a = Act + slot * H;
    linear_row(C, H, x + (size_t)t * C, Wg + (size_t)e * C * H, bg + (size_t)e * H, g);
    linear_row(C, H, x + (size_t)t * C, Wu + (size_t)e * C * H, bu + (size_t)e * H, u);
    for (int h = 0; h < H; ++h) {
      float gs = g[h] / (1.0f + expf(-g[h]));
      a[h] = gs * u[h];
    }
    linear_row(H, C, a, Wd + (size_t)e * H * C, bd + (size_t)e * C, O + slot * C);
  }

  /* B1 */
  for (size_t slot = 0; slot < A; ++slot) {
    const int flat = PM[slot], t = flat / k;
    const float pr = TP[flat];
    const float* d = dy + (size_t)t * C;
    const float* o = O + slot * C;
    float* dg = dgo + slot * C;
    float dot = 0.0f;
    for (int c = 0; c < C; ++c) {
#ifndef ORACLE_PLANT_UNGATED
      dg[c] = d[c] * pr;
#else
      dg[c] = d[c];
#endif
      dot += o[c] * d[c];
    }
    dTP[flat] = dot;
  }

  /* B2 */
  for (int e = 0; e < E; ++e) {
    const int cnt = CN[e];
    if (cnt == 0) continue;
    const size_t s0 = (size_t)OF[e];
    for (int r = 0; r < cnt; ++r) rows[r] = Act + (s0 + r) * H;
    linear_backward(cnt, H, C, rows, dgo + s0 * C, Wd + (size_t)e * H * C,
                    dWd + (size_t)e * H * C, dbd + (size_t)e * C, dD + s0 * H, tmp);
    for (size_t i = s0 * H; i < (s0 + cnt) * H; ++i) {
      const float dd = dD[i], u = U[i], g = G[i];
      const float sig = 1.0f / (1.0f + expf(-g));
      dUp[i] = dd * (g * sig);
#ifndef ORACLE_PLANT_SILU_SIGN
      dGt[i] = (dd * u) * (sig * (1.0f + g * (1.0f - sig)));
#else
      dGt[i] = (dd * u) * (sig * (1.0f - g * (1.0f - sig)));
#endif
    }
    for (int r = 0; r < cnt; ++r) rows[r] = x + (size_t)(PM[s0 + r] / k) * C;
    linear_backward(cnt, C, H, rows, dGt + s0 * H, Wg + (size_t)e * C * H,
                    dWg + (size_t)e * C * H, dbg + (size_t)e * H, dgi + s0 * C, tmp);
    linear_backward(cnt, C, H, rows, dUp + s0 * H, Wu + (size_t)e * C * H,
                    dWu + (size_t)e * C * H, dbu + (size_t)e * H, dinU + s0 * C, tmp);
    for (size_t i = s0 * C; i < (s0 + cnt) * C; ++i) dgi[i] = dgi[i] + dinU[i];
  }

  /* B3 */
  memset(dx, 0, sizeof(float) * (size_t)N * C);
  for (size_t slot = 0; slot < A; ++slot) {
    float* o = dx + (size_t)(PM[slot] / k) * C;
    const float* g = dgi + slot * C;
    for (int c = 0; c < C; ++c) o[c] += g[c];
  }

  /* B4, B5 */
  memset(dP, 0, sizeof(float) * NE);
  for (size_t f = 0; f < A; ++f) dP[(f / k) * E + I[f]] = dTP[f];
  for (int e = 0; e < E; ++e) {
    const float fe = (float)CN[e] / (float)N;
    tmp[e] = (0.01f * (float)E * fe) / (float)N;
  }
#ifndef ORACLE_PLANT_NO_LOAD_BALANCE
  for (size_t i = 0; i < NE; ++i) dP[i] = dP[i] + tmp[i % E];
#endif

  /* B6 */
  for (int t = 0; t < N; ++t) {
    const float* p = P + (size_t)t * E;
    const float* d = dP + (size_t)t * E;
    float* o = dL + (size_t)t * E;
    float s = 0.0f;
    for (int e = 0; e < E; ++e) s += d[e] * p[e];
    for (int e = 0; e < E; ++e) o[e] = p[e] * (d[e] - s);
  }

  /* B7, B8 */
  for (int t = 0; t < N; ++t) rows[t] = x + (size_t)t * C;
  linear_backward(N, C, E, rows, dL, Wr, dWr, dbr, rdin, tmp);
  for (size_t i = 0; i < (size_t)N * C; ++i) dx[i] = dx[i] + rdin[i];

  free(L); free(P); free(I); free(TP); free(CN); free(OF); free(PM);
  free(G); free(U); free(Act); free(O); free(dgo); free(dgi); free(dTP);
  free(dD); free(dGt); free(dUp); free(dinU); free(dP); free(dL); free(rdin);
  free(rows); free(tmp);
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

/* utils/Tensor.cpp:785-800 (rms_norm_into, CPU branch), as called by
 * RMSNormLayer::forward_into (layers/RMSNormLayer.cpp:14-22):
 * ms = sum x^2 sequential; r = 1/sqrt(ms/C + eps); out = (x*r)*scale. */
void oracle_rmsnorm_scaled(int N, int C, float eps, const float* x, const float* scale,
                           float* out, float* rstd) {
  for (int i = 0; i < N; ++i) {
    const float* xr = x + (size_t)i * C;
    float ms = 0.0f;
    for (int c = 0; c < C; ++c) ms += xr[c] * xr[c];
    const float r = 1.0f / sqrtf(ms / C + eps);
    if (rstd) rstd[i] = r;
    for (int c = 0; c < C; ++c) {
      const float norm = xr[c] * r;
      out[(size_t)i * C + c] = norm * scale[c];
    }
  }
}

/* utils/Tensor.cpp:1665-1689 (rms_norm_backward_into, CPU branch), as
 * called by RMSNormLayer::backward_into (layers/RMSNormLayer.cpp:30-33):
 * per token, in column order, dh = dout*scale; dscale += dout*x_hat (added
 * token by token); s = sum dh*x_hat; then dx = r*(dh - x_hat*s/C).  dx may
 * alias dout (the engine passes the same buffer): every column of a row is
 * read before any is written. */
void oracle_rmsnorm_backward(int N, int C, const float* dout, const float* x_hat,
                             const float* scale, const float* rstd, float* dx, float* dscale) {
  for (int i = 0; i < N; ++i) {
    const float* d = dout + (size_t)i * C;
    const float* xh = x_hat + (size_t)i * C;
    float* o = dx + (size_t)i * C;
    const float r = rstd[i];
    float s = 0.0f;
    for (int c = 0; c < C; ++c) {
      const float dh = d[c] * scale[c];
#ifndef ORACLE_PLANT_DSCALE_UNHATTED
      dscale[c] += d[c] * xh[c];
#else
      dscale[c] += d[c];
#endif
      s += dh * xh[c];
    }
    for (int c = 0; c < C; ++c) {
      const float dh = d[c] * scale[c];
#ifndef ORACLE_PLANT_NORM_NO_PROJECTION
      o[c] = r * (dh - xh[c] * s / C);
#else
      o[c] = r * dh;
#endif
    }
  }
}

/* layers/TransformerBlock.cpp:42-46: ln2.forward_into(x1, xn),
 * mlp.forward_into(xn, y), Tensor::add_into(x1, y, out) (utils/Tensor.cpp:
 * 1579-1597: out = x1 + y elementwise). */
int oracle_moe_block(int N, int C, int H, int E, int k, float eps, const float* x1,
                     const float* gamma, const float* Wr, const float* br, const float* Wg,
                     const float* bg, const float* Wu, const float* bu, const float* Wd,
                     const float* bd, float* out, float* xn, float* rstd, int32_t* idx,
                     float* topp, int32_t* counts, int32_t* perm) {
  if (N < 0 || C <= 0) return 1;
  float* XN = xn ? xn : (float*)malloc(sizeof(float) * ((size_t)N * C + 1));
  float* Y = (float*)malloc(sizeof(float) * ((size_t)N * C + 1));
  oracle_rmsnorm_scaled(N, C, eps, x1, gamma, XN, rstd);
  int rc = oracle_moe_forward(N, C, H, E, k, XN, Wr, br, Wg, bg, Wu, bu, Wd, bd, Y, NULL, NULL,
                              idx, topp, counts, NULL, perm);
  if (rc == 0)
    for (size_t i = 0; i < (size_t)N * C; ++i) out[i] = x1[i] + Y[i];
  if (!xn) free(XN);
  free(Y);
  return rc;
}

/* layers/TransformerBlock.cpp:81-85 (backward_into, the MoE half): with
 * xn = ln2(x1) from the forward, mlp.backward_into(dout, d_ln2),
 * ln2.backward_into(d_ln2, d_ln2) and Tensor::add_into(dout, d_ln2, d_x1)
 * (utils/Tensor.cpp:1579-1597: a + b elementwise).  x_hat = x1 * r as
 * rms_norm_into caches it (utils/Tensor.cpp:796-797).  The MoE parameter
 * gradients and dgamma are ACCUMULATED (add_grad / scale.grad +=), as in
 * oracle_moe_backward; dx1 is written. */
int oracle_moe_block_backward(int N, int C, int H, int E, int k, float eps, const float* x1,
                              const float* gamma, const float* Wr, const float* br,
                              const float* Wg, const float* bg, const float* Wu,
                              const float* bu, const float* Wd, const float* bd,
                              const float* dout, float* dx1, float* dgamma, float* dWr,
                              float* dbr, float* dWg, float* dbg, float* dWu, float* dbu,
                              float* dWd, float* dbd) {
  if (N < 0 || C <= 0) return 1;
  const size_t NC = (size_t)N * C;
  float* XN = (float*)malloc(sizeof(float) * (NC + 1));
  float* XH = (float*)malloc(sizeof(float) * (NC + 1));
  float* R = (float*)malloc(sizeof(float) * ((size_t)N + 1));
  float* D = (float*)malloc(sizeof(float) * (NC + 1));
  oracle_rmsnorm_scaled(N, C, eps, x1, gamma, XN, R);
  for (int i = 0; i < N; ++i)
    for (int c = 0; c < C; ++c) XH[(size_t)i * C + c] = x1[(size_t)i * C + c] * R[i];
  int rc = oracle_moe_backward(N, C, H, E, k, XN, Wr, br, Wg, bg, Wu, bu, Wd, bd, dout, D, dWr,
                               dbr, dWg, dbg, dWu, dbu, dWd, dbd);
  if (rc == 0) {
    oracle_rmsnorm_backward(N, C, D, XH, gamma, R, D, dgamma);
    for (size_t i = 0; i < NC; ++i) dx1[i] = dout[i] + D[i];
  }
  free(XN); free(XH); free(R); free(D);
  return rc;
}
