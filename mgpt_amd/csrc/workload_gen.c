/*
 * workload_gen.c -- host-side generator of the seeded synthetic inputs.
 *
 * C twin of mgpt_amd/workload.py (normal(), normal_f32()): the same
 * counter-based SplitMix64 streams and the same Box-Muller arithmetic with
 * polynomial log/cos, operation for operation, so both produce identical
 * float32 arrays (tests/test_workload.py checks this).  Only IEEE-754
 * correctly-rounded double +, -, *, / and sqrt are used; build with
 * -ffp-contract=off so no operation is fused.  Not part of the MoE C-ABI:
 * it feeds tests and benchmarks.
 */
#include <math.h>
#include <stdint.h>

#define GAMMA 0x9E3779B97F4A7C15ULL

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t mgpt_wl_stream_seed(uint64_t seed, uint64_t stream) {
  return mix64(seed * 0x100000001B3ULL + stream * 0x2545F4914F6CDD1DULL + GAMMA);
}

/* Coefficients exactly as workload.py computes them (1/(2j+1), +-1/(2n)!,
 * +-1/(2n+1)! rounded to double). */
static const double LOG_COEF[12] = {0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3, 0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4, 0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5};
static const double COS_COEF[12] = {0x1.0000000000000p+0, -0x1.0000000000000p-1, 0x1.5555555555555p-5, -0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37, 0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62, -0x1.0ce396db7f853p-70};
static const double SIN_COEF[12] = {0x1.0000000000000p+0, -0x1.5555555555555p-3, 0x1.1111111111111p-7, -0x1.a01a01a01a01ap-13, 0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33, -0x1.ae7f3e733b81fp-41, 0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57, 0x1.71b8ef6dcf572p-66, -0x1.761b413163819p-75};
static const double LN2 = 0x1.62e42fefa39efp-1;
static const double SQRT_HALF = 0x1.6a09e667f3bcdp-1;
static const double HALF_PI = 0x1.921fb54442d18p+0;

static inline double poly_log(double u) {
  int e;
  double m = frexp(u, &e);
  if (m < SQRT_HALF) { m = m * 2.0; e -= 1; }
  double s = (m - 1.0) / (m + 1.0);
  double s2 = s * s;
  double p = LOG_COEF[11];
  for (int j = 10; j >= 0; --j) p = p * s2 + LOG_COEF[j];
  return (double)e * LN2 + 2.0 * s * p;
}

static inline double poly_cos_2pi(double v) {
  double w = v * 4.0;
  double q = floor(w);
  double f = w - q;
  double x = f * HALF_PI;
  double x2 = x * x;
  double c = COS_COEF[11];
  for (int j = 10; j >= 0; --j) c = c * x2 + COS_COEF[j];
  double s = SIN_COEF[11];
  for (int j = 10; j >= 0; --j) s = s * x2 + SIN_COEF[j];
  s = s * x;
  int qi = (int)q;
  return qi == 0 ? c : qi == 1 ? -s : qi == 2 ? -c : s;
}

/* out[i] = (float)(std * z_{start+i}) of stream (seed, stream). */
void mgpt_wl_normal_f32(uint64_t seed, uint64_t stream, int64_t start,
                        int64_t count, double std, float* out) {
  const uint64_t s = mgpt_wl_stream_seed(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    uint64_t j = (uint64_t)(start + i);
    uint64_t b1 = mix64(s + (2 * j + 1) * GAMMA);
    uint64_t b2 = mix64(s + (2 * j + 2) * GAMMA);
    double u1 = ((double)(b1 >> 11) + 1.0) * 0x1p-53;
    double u2 = (double)(b2 >> 11) * 0x1p-53;
    double z = sqrt(-2.0 * poly_log(u1)) * poly_cos_2pi(u2);
    out[i] = (float)(z * std);
  }
}

/* OCP FP8 E4M3FN encode, round-to-nearest-even, saturating to +-448, zero
 * encoded as +0 (the rule of the library's load-time quantiser and of
 * workload.py's e4m3_encode). */
static inline uint8_t e4m3_encode1(float v) {
  union { float f; uint32_t u; } in = {v};
  const uint32_t sign = in.u >> 31;
  const float a = fabsf(v);
  uint32_t code;
  if (!(a < 448.0f)) {
    code = 0x7E;
  } else if (a < 0x1p-6f) {
    code = (uint32_t)rintf(a * 512.0f);
  } else {
    union { float f; uint32_t u; } b = {a};
    uint32_t q = b.u >> 20;
    const uint32_t rem = b.u & 0xFFFFFu;
    q += (rem > 0x80000u) || (rem == 0x80000u && (q & 1u));
    const int ex = (int)(q >> 3) - 127 + 7;
    code = ((uint32_t)ex << 3) | (q & 7u);
    if (code > 0x7E) code = 0x7E;
  }
  return (uint8_t)(code | ((sign && code) ? 0x80u : 0u));
}

static inline float e4m3_decode1(uint8_t b) {
  const int e = (b >> 3) & 0xF, m = b & 7;
  float v = e == 0 ? (float)m * 0x1p-9f : ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return (b & 0x80) ? -v : v;
}

/* Per-output-channel quantisation of a reference-layout weight W[in][out]:
 * scale[o] = amax_o / 448 (1 for an all-zero column), q = e4m3(w / scale),
 * deq = value(q) * scale. */
void mgpt_wl_quantize_e4m3(const float* w, int64_t rows_in, int64_t cols_out, uint8_t* q,
                           float* scale, float* deq) {
  for (int64_t o = 0; o < cols_out; ++o) scale[o] = 0.0f;
  for (int64_t i = 0; i < rows_in; ++i)
    for (int64_t o = 0; o < cols_out; ++o) {
      const float a = fabsf(w[i * cols_out + o]);
      if (a > scale[o]) scale[o] = a;
    }
  for (int64_t o = 0; o < cols_out; ++o) scale[o] = scale[o] > 0.0f ? scale[o] / 448.0f : 1.0f;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows_in; ++i)
    for (int64_t o = 0; o < cols_out; ++o) {
      const int64_t j = i * cols_out + o;
      const uint8_t c = e4m3_encode1(w[j] / scale[o]);
      q[j] = c;
      deq[j] = e4m3_decode1(c) * scale[o];
    }
}
