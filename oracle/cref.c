/* cref.c -- CPU oracle for the fused decode hot path (TEST INFRASTRUCTURE).
 *
 * Plain C restatement of the reference's arithmetic, used only by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
 * Nothing in the product links or calls this file.
 *
 * Two families of functions:
 *  - orc_*_f32: the float-in/float-out contracts of the reference's plain C++
 *    CPU reference (validation/src/reference/cpu_reference.{h,cpp}:7-111),
 *    computed with double accumulation.  Tests compare them against the
 *    reference's own code compiled into oracle/_ref and against the known
 *    answers of validation/src/tests/test_reference.cpp:32-158.
 *  - orc_*_f16 / *_f64: the reference's PyTorch stage definitions
 *    (src/decodebench/demos/llama_decode.py:36-43, 77-87, 120-134) on fp16
 *    data: fp16 rounding exactly where the torch stages round, sums in double
 *    (so the only difference to torch is summation order), plus exact (f64)
 *    variants for relative-error checks.
 *
 * fp16 conversions are implemented here (round to nearest even) so the oracle
 * does not depend on compiler support for _Float16; tests pin them against
 * numpy.float16 over every fp16 value and the midpoints between them.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

float orc_h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float f = (float)man * 5.9604644775390625e-8f;
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

/* float -> fp16, round to nearest, ties to even. */
uint16_t orc_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) { /* inf or nan */
    return sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u);
  }
  if (absx >= 0x477ff000u) /* >= 65520: rounds to inf */
    return sign | 0x7c00u;
  if (absx < 0x38800000u) { /* below the smallest normal 2^-14 */
    /* value = m * 2^-24 with m = round(|f| * 2^24); exact in double. */
    float a;
    memcpy(&a, &absx, 4);
    const double scaled = (double)a * 16777216.0;
    double r = floor(scaled);
    const double frac = scaled - r;
    if (frac > 0.5 || (frac == 0.5 && fmod(r, 2.0) != 0.0)) r += 1.0;
    return sign | (uint16_t)r; /* r <= 1024 gives the smallest normal */
  }
  /* normal: keep 10 mantissa bits, round on the 13 dropped bits */
  const uint32_t e = (absx >> 23) - 112u;
  const uint32_t m = absx & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rest = m & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
  return sign | (uint16_t)h;
}

void orc_h2f_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_h2f(in[i]);
}

void orc_f2h_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f2h(in[i]);
}

static inline float rn16(float v) { return orc_h2f(orc_f2h(v)); }

/* ----------------------------------------- cpu_reference.cpp contracts */

/* cpu_reference.cpp:7-18: out = x / sqrt(mean(x^2) + eps) * gamma */
void orc_rmsnorm_f32(const float* x, const float* gamma, float* out, int d,
                     float eps) {
  double ss = 0.0;
  for (int i = 0; i < d; ++i) ss += (double)x[i] * x[i];
  const double rms = sqrt(ss / d + (double)eps);
  for (int i = 0; i < d; ++i) out[i] = (float)((double)x[i] / rms * gamma[i]);
}

/* cpu_reference.cpp:21-29: row-major W[d_out][d_in] times x */
void orc_gemv_f32(const float* W, const float* x, float* out, int d_out,
                  int d_in) {
  for (int i = 0; i < d_out; ++i) {
    double acc = 0.0;
    const float* row = W + (size_t)i * d_in;
    for (int j = 0; j < d_in; ++j) acc += (double)row[j] * x[j];
    out[i] = (float)acc;
  }
}

/* cpu_reference.cpp:31-33 */
float orc_silu_f32(float x) { return (float)((double)x / (1.0 + exp(-(double)x))); }

/* cpu_reference.cpp:35-39 */
void orc_swiglu_f32(const float* g, const float* u, float* out, int n) {
  for (int i = 0; i < n; ++i) out[i] = (float)((double)orc_silu_f32(g[i]) * u[i]);
}

static void softmax_row_f64(const double* s, double* p, int n) {
  double mx = s[0];
  for (int i = 1; i < n; ++i) mx = s[i] > mx ? s[i] : mx;
  double sum = 0.0;
  for (int i = 0; i < n; ++i) {
    p[i] = exp(s[i] - mx);
    sum += p[i];
  }
  for (int i = 0; i < n; ++i) p[i] /= sum;
}

/* cpu_reference.cpp:42-62: softmax of each of n_heads rows */
void orc_softmax_f32(const float* scores, float* probs, int n_heads,
                     int seq_len) {
  double* s = (double*)malloc(sizeof(double) * (size_t)seq_len * 2);
  double* p = s + seq_len;
  for (int h = 0; h < n_heads; ++h) {
    for (int i = 0; i < seq_len; ++i) s[i] = scores[(size_t)h * seq_len + i];
    softmax_row_f64(s, p, seq_len);
    for (int i = 0; i < seq_len; ++i) probs[(size_t)h * seq_len + i] = (float)p[i];
  }
  free(s);
}

/* cpu_reference.cpp:64-111: unscaled single-query attention per head */
void orc_attention_f32(const float* q, const float* K, const float* V,
                       float* out, int n_heads, int seq_len, int head_dim) {
  double* s = (double*)malloc(sizeof(double) * (size_t)seq_len * 2);
  double* p = s + seq_len;
  for (int h = 0; h < n_heads; ++h) {
    const float* qh = q + (size_t)h * head_dim;
    const float* Kh = K + (size_t)h * seq_len * head_dim;
    const float* Vh = V + (size_t)h * seq_len * head_dim;
    for (int t = 0; t < seq_len; ++t) {
      double dot = 0.0;
      for (int d = 0; d < head_dim; ++d) dot += (double)qh[d] * Kh[(size_t)t * head_dim + d];
      s[t] = dot;
    }
    softmax_row_f64(s, p, seq_len);
    for (int d = 0; d < head_dim; ++d) {
      double acc = 0.0;
      for (int t = 0; t < seq_len; ++t) acc += p[t] * Vh[(size_t)t * head_dim + d];
      out[(size_t)h * head_dim + d] = (float)acc;
    }
  }
  free(s);
}

/* --------------------------------------- torch-stage semantics on fp16 */

/* llama_decode.py:36-39:
 *   var = mean(x.float()^2);  xh = (x.float() * rsqrt(var + eps)).half() * g
 * fp32 statistic (sum in double, rounded once), fp16 rounding of x*inv_rms,
 * then of the fp16 x fp16 product with g (exact in fp32, one rounding). */
void orc_rmsnorm_f16(const uint16_t* x, const uint16_t* g, uint16_t* out,
                     int B, int K, float eps) {
  for (int b = 0; b < B; ++b) {
    const uint16_t* xr = x + (size_t)b * K;
    double ss = 0.0;
    for (int k = 0; k < K; ++k) {
      const double v = orc_h2f(xr[k]);
      ss += v * v;
    }
    const float var = (float)ss / (float)K;
    const float inv = 1.0f / sqrtf(var + eps);
    for (int k = 0; k < K; ++k) {
      const float n = rn16(orc_h2f(xr[k]) * inv);
      out[(size_t)b * K + k] = orc_f2h(n * orc_h2f(g[k]));
    }
  }
}

/* y[b][n] = sum_k x[b][k] * W[n][k] in double (exact products). */
void orc_gemv_f64(const uint16_t* x, const uint16_t* W, double* y, int B,
                  int K, int N) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)B * K);
  orc_h2f_array(x, xf, (size_t)B * K);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint16_t* wr = W + (size_t)n * K;
    for (int b = 0; b < B; ++b) {
      const float* xb = xf + (size_t)b * K;
      double acc = 0.0;
      for (int k = 0; k < K; ++k) acc += (double)orc_h2f(wr[k]) * xb[k];
      y[(size_t)b * N + n] = acc;
    }
  }
  free(xf);
}

/* llama_decode.py:41-43 F.linear(xh, W): fp16 output of an fp32-accumulated
 * dot product; here the accumulation is exact-ish (double). */
void orc_gemv_f16(const uint16_t* x, const uint16_t* W, uint16_t* y, int B,
                  int K, int N) {
  double* acc = (double*)malloc(sizeof(double) * (size_t)B * N);
  orc_gemv_f64(x, W, acc, B, K, N);
  for (size_t i = 0; i < (size_t)B * N; ++i) y[i] = orc_f2h((float)acc[i]);
  free(acc);
}

/* llama_decode.py:85-87: silu(gate) * up on fp16 tensors: silu evaluated in
 * fp32 and rounded to fp16, then the fp16 product rounded to fp16. */
void orc_swiglu_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out,
                    size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float gv = orc_h2f(gate[i]);
    const float s = rn16((float)((double)gv / (1.0 + exp(-(double)gv))));
    out[i] = orc_f2h(s * orc_h2f(up[i]));
  }
}

/* Exact grouped-query attention for one token per sequence:
 *   o[b][h][:] = softmax_l(scale * q[b][h] . K[b][h/G][l]) V[b][h/G][l]
 * q [B,Hq,D], K/V [B,Hkv,L,D] fp16, o [B,Hq,D] double. */
void orc_attention_f64(const uint16_t* q, const uint16_t* K, const uint16_t* V,
                       double* o, int B, int Hq, int Hkv, int L, int D,
                       double scale) {
  const int G = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hq; ++h) {
      const int kvh = h / G;
      const uint16_t* qh = q + ((size_t)b * Hq + h) * D;
      const uint16_t* Kh = K + ((size_t)b * Hkv + kvh) * (size_t)L * D;
      const uint16_t* Vh = V + ((size_t)b * Hkv + kvh) * (size_t)L * D;
      double* s = (double*)malloc(sizeof(double) * (size_t)L * 2);
      double* p = s + L;
      double qf[1024];
      for (int d = 0; d < D; ++d) qf[d] = orc_h2f(qh[d]);
      for (int l = 0; l < L; ++l) {
        double dot = 0.0;
        for (int d = 0; d < D; ++d) dot += qf[d] * orc_h2f(Kh[(size_t)l * D + d]);
        s[l] = dot * scale;
      }
      softmax_row_f64(s, p, L);
      double* oh = o + ((size_t)b * Hq + h) * D;
      for (int d = 0; d < D; ++d) oh[d] = 0.0;
      for (int l = 0; l < L; ++l) {
        const uint16_t* vr = Vh + (size_t)l * D;
        for (int d = 0; d < D; ++d) oh[d] += p[l] * orc_h2f(vr[d]);
      }
      free(s);
    }
  }
}

/* The split-KV form of the same attention, restating the reference's
 * two-phase algorithm (validation/src/kernels/fused/f4.cu:160-319) in
 * double: the L rows are cut into S contiguous splits of ceil(L/S) rows;
 * split s keeps m_s = max score, l_s = sum e^{s-m_s}, o_s = sum e^{s-m_s} V
 * (empty splits: m=-inf, l=0, o=0); the merge is
 *   o = sum_s e^{m_s-M} o_s / sum_s e^{m_s-M} l_s,  M = max_s m_s.
 * Mathematically identical to orc_attention_f64 for every S >= 1. */
void orc_attention_splitkv_f64(const uint16_t* q, const uint16_t* K,
                               const uint16_t* V, double* o, int B, int Hq,
                               int Hkv, int L, int D, double scale, int S) {
  const int G = Hq / Hkv;
  const int per = (L + S - 1) / S;
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hq; ++h) {
      const int kvh = h / G;
      const uint16_t* qh = q + ((size_t)b * Hq + h) * D;
      const uint16_t* Kh = K + ((size_t)b * Hkv + kvh) * (size_t)L * D;
      const uint16_t* Vh = V + ((size_t)b * Hkv + kvh) * (size_t)L * D;
      double* pm = (double*)malloc(sizeof(double) * (size_t)S * (D + 2));
      double* pl = pm + S;
      double* po = pl + S;
      for (int s = 0; s < S; ++s) {
        const int l0 = s * per, l1 = (l0 + per < L) ? l0 + per : L;
        double m = -INFINITY, lsum = 0.0;
        double* os = po + (size_t)s * D;
        for (int d = 0; d < D; ++d) os[d] = 0.0;
        for (int l = l0; l < l1; ++l) {
          double dot = 0.0;
          for (int d = 0; d < D; ++d)
            dot += (double)orc_h2f(qh[d]) * orc_h2f(Kh[(size_t)l * D + d]);
          const double sc = dot * scale;
          const double m_new = sc > m ? sc : m;
          const double a = (m == -INFINITY) ? 0.0 : exp(m - m_new);
          const double p = exp(sc - m_new);
          lsum = lsum * a + p;
          for (int d = 0; d < D; ++d)
            os[d] = os[d] * a + p * orc_h2f(Vh[(size_t)l * D + d]);
          m = m_new;
        }
        pm[s] = m;
        pl[s] = lsum;
      }
      double M = -INFINITY;
      for (int s = 0; s < S; ++s) M = pm[s] > M ? pm[s] : M;
      double lt = 0.0;
      double* oh = o + ((size_t)b * Hq + h) * D;
      for (int d = 0; d < D; ++d) oh[d] = 0.0;
      for (int s = 0; s < S; ++s) {
        if (pm[s] == -INFINITY) continue;
        const double w = exp(pm[s] - M);
        lt += w * pl[s];
        for (int d = 0; d < D; ++d) oh[d] += w * po[(size_t)s * D + d];
      }
      for (int d = 0; d < D; ++d) oh[d] /= lt;
      free(pm);
    }
  }
}

/* ------------------------------------------------------------ fp8 e4m3 */

/* OCP FP8 E4M3 ("e4m3fn"): 1 sign, 4 exponent (bias 7), 3 mantissa bits, no
 * infinities, S.1111.111 is NaN, max finite 448, subnormals m * 2^-9. */
float orc_e4m3_to_f32(uint8_t v) {
  const int sign = v >> 7, e = (v >> 3) & 0xf, m = v & 7;
  float mag;
  if (e == 15 && m == 7) return NAN;
  if (e == 0)
    mag = (float)m * 0.001953125f; /* 2^-9 */
  else
    mag = ldexpf(1.0f + m / 8.0f, e - 7);
  return sign ? -mag : mag;
}

/* y[b][n] = scale[n] * sum_k e4m3(Wq[n][k]) * x[b][k]  (double). */
void orc_gemv_fp8_f64(const uint16_t* x, const uint8_t* Wq, const float* scale,
                      double* y, int B, int K, int N) {
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = orc_e4m3_to_f32((uint8_t)i);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint8_t* wr = Wq + (size_t)n * K;
    for (int b = 0; b < B; ++b) {
      const uint16_t* xb = x + (size_t)b * K;
      double acc = 0.0;
      for (int k = 0; k < K; ++k) acc += (double)lut[wr[k]] * orc_h2f(xb[k]);
      y[(size_t)b * N + n] = acc * scale[n];
    }
  }
}
