/*
 * moe_oracle.h -- CPU restatement of mgpt's MoE block forward and backward.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the parity
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the
 * HIP path against.  It is never linked into, loaded by, or called from the
 * product library (mgpt_amd/), which fails loudly when its HIP build is
 * missing instead of falling back to anything here.
 *
 * Every function restates the reference CPU path (/root/reference, the
 * `#else` build of src/main/utils/cuda_ops.cu plus the CPU branches of
 * src/main/utils/Tensor.cpp) with the same arithmetic order, so that on the
 * same inputs it reproduces the reference's bits when compiled with
 * -ffp-contract=off.  Citations are per function in moe_oracle.c.
 *
 * Layouts (reference layout, F1): x [N,C] row-major; W_r [C,E]; b_r [E];
 * per expert e: W_g[e] [C,H], b_g[e] [H], W_u[e] [C,H], b_u[e] [H],
 * W_d[e] [H,C], b_d[e] [C].  The expert arrays below are stacked over e.
 */
#ifndef MGPT_MOE_ORACLE_H
#define MGPT_MOE_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* glibc expf, exactly as the reference calls it (std::exp(float)). */
float oracle_expf(float x);
void oracle_expf_array(const float* in, float* out, int64_t n);

/* logits[N,E] = x[N,C] . W_r[C,E] + b_r (sequential-k fp32, no FMA). */
void oracle_router_logits(int N, int C, int E, const float* x, const float* Wr,
                          const float* br, float* logits);

/* probs[N,E] = clamped softmax of logits (F2). */
void oracle_softmax(int N, int E, const float* logits, float* probs);

/* top-k insertion with strict '>' (F3): idx[N,k], topp[N,k]. */
void oracle_topk(int N, int E, int k, const float* probs, int32_t* idx, float* topp);

/* counts[E] histogram, offsets[E] exclusive scan, perm[N*k] stable
 * expert-major permutation of flat assignment ids (F5-F7). */
void oracle_dispatch(int N, int E, int k, const int32_t* idx, int32_t* counts,
                     int32_t* offsets, int32_t* perm);

/* Full forward (F1-F11).  Any of the optional outputs may be NULL. */
int oracle_moe_forward(int N, int C, int H, int E, int k, const float* x,
                       const float* Wr, const float* br, const float* Wg,
                       const float* bg, const float* Wu, const float* bu,
                       const float* Wd, const float* bd, float* y,
                       float* logits, float* probs, int32_t* idx, float* topp,
                       int32_t* counts, int32_t* offsets, int32_t* perm);

/* Output rows y[n_sel,C] for the tokens tok[0..n_sel) given their routing
 * (idx/topp rows of the full problem).  Because every reference output
 * element is an independent sequential sum, these rows equal the rows of a
 * full forward bit for bit. */
int oracle_moe_tokens(int C, int H, int E, int k, int n_sel, const int32_t* tok,
                      const float* x, const int32_t* idx, const float* topp,
                      const float* Wg, const float* bg, const float* Wu,
                      const float* bu, const float* Wd, const float* bd,
                      float* y_sel);

/* Backward of the block after a forward on the same inputs (B1-B9).
 * dx[N,C] is written; the parameter gradients are ACCUMULATED into
 * dWr[C,E], dbr[E], dWg[E,C,H], dbg[E,H], dWu[E,C,H], dbu[E,H], dWd[E,H,C],
 * dbd[E,C] like the reference's add_grad, so a caller that wants the
 * gradient of one call passes zeroed buffers.  Experts no token chose keep
 * their gradients untouched.  Returns 0, or 1 for a bad shape. */
int oracle_moe_backward(int N, int C, int H, int E, int k, const float* x,
                        const float* Wr, const float* br, const float* Wg,
                        const float* bg, const float* Wu, const float* bu,
                        const float* Wd, const float* bd, const float* dy,
                        float* dx, float* dWr, float* dbr, float* dWg,
                        float* dbg, float* dWu, float* dbu, float* dWd,
                        float* dbd);

/* out[N,C] = RMSNorm(x) * scale and rstd[N] = 1/rms, the engine's
 * RMSNormLayer (eps) forward; rstd may be NULL. */
void oracle_rmsnorm_scaled(int N, int C, float eps, const float* x, const float* scale,
                           float* out, float* rstd);

/* The MoE half of a transformer block: xn = RMSNorm(x1) * gamma, y = MoE(xn),
 * out = x1 + y.  xn (may be NULL) receives the normalised rows, rstd (may
 * be NULL) the per-token 1/rms; the routing outputs follow
 * oracle_moe_forward (any may be NULL). */
int oracle_moe_block(int N, int C, int H, int E, int k, float eps, const float* x1,
                     const float* gamma, const float* Wr, const float* br, const float* Wg,
                     const float* bg, const float* Wu, const float* bu, const float* Wd,
                     const float* bd, float* out, float* xn, float* rstd, int32_t* idx,
                     float* topp, int32_t* counts, int32_t* perm);

/* RMSNormLayer backward (eps-independent): dx[N,C] from dout, the cached
 * x_hat = x * rstd and scale; dscale[C] is ACCUMULATED.  dx may alias
 * dout. */
void oracle_rmsnorm_backward(int N, int C, const float* dout, const float* x_hat,
                             const float* scale, const float* rstd, float* dx, float* dscale);

/* Backward of oracle_moe_block for the upstream gradient dout of out:
 * dx1[N,C] is written (dout + the ln2 branch); dgamma[C] and the MoE
 * parameter gradients are ACCUMULATED as in oracle_moe_backward. */
int oracle_moe_block_backward(int N, int C, int H, int E, int k, float eps, const float* x1,
                              const float* gamma, const float* Wr, const float* br,
                              const float* Wg, const float* bg, const float* Wu,
                              const float* bu, const float* Wd, const float* bd,
                              const float* dout, float* dx1, float* dgamma, float* dWr,
                              float* dbr, float* dWg, float* dbg, float* dWu, float* dbu,
                              float* dWd, float* dbd);

/* x_hat[N,C] = RMSNorm(x) with gamma = 1 (input preparation, a1). */
void oracle_rmsnorm(int N, int C, float eps, const float* x, float* out);

#ifdef __cplusplus
}
#endif
#endif
