/*
 * cpu_simd.c -- TEST INFRASTRUCTURE ONLY: the CPU baseline of bench.py.
 *
 * An AVX-512 + OpenMP restatement of the fused per-token operations, the
 * stand-in for the reference's own AVX-512 CPU kernels (vestra-kernels, not
 * in the reference tree; the reference engine runs them with 16 threads,
 * docs/DA3_CPU_F32_STATUS.md:92-95).  Same algorithms and per-element
 * operation order as the scalar oracle (vestra_oracle.c) -- no FMA
 * contraction (-ffp-contract=off, explicit multiply then add) -- with the
 * row reductions done 16 lanes wide, as a SIMD kernel does:
 *   layernorm        two-pass biased variance, inv = 1/sqrtf(var + eps)
 *                    (crates/da-engine/src/dpt_head.rs:272-296);
 *   gelu             0.5 x (1 + erf(x/sqrt 2)), erf by Abramowitz & Stegun
 *                    7.1.26 (docs/plans/2026-07-18-rust-engine-v1.md:870-876),
 *                    its exp(-a^2) by Cody-Waite reduction x = n ln2 + r and a
 *                    degree-7 Taylor polynomial of e^r on |r| <= ln2/2
 *                    (relative error below 2e-8 before rounding);
 *   layerscale+res   t = y*g; x = x + t (vit_block.rs:755-758, 669-679);
 *   qk_norm_rope     LayerNorm over each 64-wide (head, token) row, then the
 *                    2D rotation (y half by the row coordinate, x half by the
 *                    column; rotate-half pairs (j, j+16)), cos/sin from a
 *                    table of the f32 angles evaluated in double, as the
 *                    oracle (vit_block.rs:911-924).
 * Results agree with the oracle within rtol 1e-5 / atol 1e-6
 * (tests/test_cpu_simd_baseline.py).  Built for x86-64-v4 (AVX-512 F, BW,
 * CD, DQ, VL), not -march=native: the library is built in one place and run
 * on the GPU box's host, whose CPU may differ; cs_available() reports
 * whether the host has those extensions.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int cs_available(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512dq") &&
         __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl");
}

void cs_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n < 1 ? 1 : n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------ helpers */

static inline float hsum(__m512 v) { return _mm512_reduce_add_ps(v); }

/* e^x for x <= 0 (the A&S erf takes exp(-a*a)): x = n*ln2 + r with ln2
 * split in a high part exact in f32 times small n and a low part
 * (Cody & Waite, "Software Manual for the Elementary Functions", 1980),
 * e^r by its Taylor series to degree 7 in Horner form, 2^n by exponent bits;
 * below -87 the result flushes to 0. */
static inline __m512 exp_neg(__m512 x) {
  const __m512 lo_lim = _mm512_set1_ps(-87.0f);
  const __mmask16 tiny = _mm512_cmp_ps_mask(x, lo_lim, _CMP_LT_OQ);
  x = _mm512_max_ps(x, lo_lim);
  const __m512 n = _mm512_roundscale_ps(_mm512_mul_ps(x, _mm512_set1_ps(1.44269504f)),
                                        _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m512 r = _mm512_sub_ps(x, _mm512_mul_ps(n, _mm512_set1_ps(0.693145752f)));
  r = _mm512_sub_ps(r, _mm512_mul_ps(n, _mm512_set1_ps(1.42860677e-06f)));
  __m512 p = _mm512_set1_ps(1.0f / 5040.0f);
  p = _mm512_add_ps(_mm512_mul_ps(p, r), _mm512_set1_ps(1.0f / 720.0f));
  p = _mm512_add_ps(_mm512_mul_ps(p, r), _mm512_set1_ps(1.0f / 120.0f));
  p = _mm512_add_ps(_mm512_mul_ps(p, r), _mm512_set1_ps(1.0f / 24.0f));
  p = _mm512_add_ps(_mm512_mul_ps(p, r), _mm512_set1_ps(1.0f / 6.0f));
  p = _mm512_add_ps(_mm512_mul_ps(p, r), _mm512_set1_ps(0.5f));
  p = _mm512_add_ps(_mm512_mul_ps(p, r), _mm512_set1_ps(1.0f));
  p = _mm512_add_ps(_mm512_mul_ps(p, r), _mm512_set1_ps(1.0f));
  const __m512i e = _mm512_slli_epi32(_mm512_add_epi32(_mm512_cvtps_epi32(n),
                                                       _mm512_set1_epi32(127)), 23);
  const __m512 out = _mm512_mul_ps(p, _mm512_castsi512_ps(e));
  return _mm512_maskz_mov_ps(~tiny, out);
}

/* ------------------------------------------------------------ LayerNorm */

static inline void ln_row(const float* x, float* y, size_t cols, const float* g,
                          const float* b, float eps) {
  const size_t nv = cols / 16;
  __m512 s = _mm512_setzero_ps();
  for (size_t i = 0; i < nv; ++i) s = _mm512_add_ps(s, _mm512_loadu_ps(x + 16 * i));
  float sum = hsum(s);
  for (size_t c = 16 * nv; c < cols; ++c) sum += x[c];
  const float mean = sum / (float)cols;
  const __m512 mv = _mm512_set1_ps(mean);
  __m512 q = _mm512_setzero_ps();
  for (size_t i = 0; i < nv; ++i) {
    const __m512 d = _mm512_sub_ps(_mm512_loadu_ps(x + 16 * i), mv);
    q = _mm512_add_ps(q, _mm512_mul_ps(d, d));
  }
  float sq = hsum(q);
  for (size_t c = 16 * nv; c < cols; ++c) {
    const float d = x[c] - mean;
    sq += d * d;
  }
  const float inv = 1.0f / sqrtf(sq / (float)cols + eps);
  const __m512 iv = _mm512_set1_ps(inv);
  for (size_t i = 0; i < nv; ++i) {
    const __m512 d = _mm512_sub_ps(_mm512_loadu_ps(x + 16 * i), mv);
    const __m512 t = _mm512_mul_ps(_mm512_mul_ps(d, iv), _mm512_loadu_ps(g + 16 * i));
    _mm512_storeu_ps(y + 16 * i, _mm512_add_ps(t, _mm512_loadu_ps(b + 16 * i)));
  }
  for (size_t c = 16 * nv; c < cols; ++c) y[c] = (x[c] - mean) * inv * g[c] + b[c];
}

void cs_layernorm_f32(const float* x, float* y, size_t rows, size_t cols, const float* gamma,
                      const float* beta, float eps) {
  long r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < (long)rows; ++r)
    ln_row(x + (size_t)r * cols, y + (size_t)r * cols, cols, gamma, beta, eps);
}

/* ------------------------------------------------------------ GELU */

void cs_gelu_f32(float* x, size_t n) {
  const size_t nv = n / 16;
  long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long)nv; ++i) {
    const __m512 v = _mm512_loadu_ps(x + 16 * (size_t)i);
    const __m512 z = _mm512_mul_ps(v, _mm512_set1_ps(0.70710678f));
    const __m512 a = _mm512_abs_ps(z);
    const __m512 t = _mm512_div_ps(_mm512_set1_ps(1.0f),
                                   _mm512_add_ps(_mm512_set1_ps(1.0f),
                                                 _mm512_mul_ps(_mm512_set1_ps(0.3275911f), a)));
    __m512 p = _mm512_sub_ps(_mm512_mul_ps(_mm512_set1_ps(1.0614054f), t),
                             _mm512_set1_ps(1.4531520f));
    p = _mm512_mul_ps(p, t);
    p = _mm512_add_ps(p, _mm512_set1_ps(1.4214137f));
    p = _mm512_sub_ps(_mm512_mul_ps(p, t), _mm512_set1_ps(0.28449674f));
    p = _mm512_add_ps(_mm512_mul_ps(p, t), _mm512_set1_ps(0.25482959f));
    const __m512 e = exp_neg(_mm512_sub_ps(_mm512_setzero_ps(), _mm512_mul_ps(a, a)));
    const __m512 yv = _mm512_sub_ps(_mm512_set1_ps(1.0f), _mm512_mul_ps(_mm512_mul_ps(p, t), e));
    /* erf = sign(z) * y */
    const __m512 sign = _mm512_castsi512_ps(
        _mm512_and_si512(_mm512_castps_si512(z), _mm512_set1_epi32((int)0x80000000u)));
    const __m512 erf = _mm512_castsi512_ps(
        _mm512_or_si512(_mm512_castps_si512(yv), _mm512_castps_si512(sign)));
    const __m512 h = _mm512_mul_ps(_mm512_set1_ps(0.5f), v);
    _mm512_storeu_ps(x + 16 * (size_t)i,
                     _mm512_mul_ps(h, _mm512_add_ps(_mm512_set1_ps(1.0f), erf)));
  }
  for (size_t j = 16 * nv; j < n; ++j) {
    const float z = x[j] * 0.70710678f;
    const float a = fabsf(z);
    const float t = 1.0f / (1.0f + 0.3275911f * a);
    float p = 1.0614054f * t - 1.4531520f;
    p = p * t;
    p = p + 1.4214137f;
    p = p * t - 0.28449674f;
    p = p * t + 0.25482959f;
    const float yv = 1.0f - p * t * expf(-a * a);
    x[j] = 0.5f * x[j] * (1.0f + (z < 0.0f ? -yv : yv));
  }
}

/* ------------------------------------------------------------ LayerScale + residual */

void cs_layerscale_residual_f32(float* x, const float* y, const float* gamma, size_t rows,
                                size_t cols) {
  const size_t nv = cols / 16;
  long r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < (long)rows; ++r) {
    float* xr = x + (size_t)r * cols;
    const float* yr = y + (size_t)r * cols;
    for (size_t i = 0; i < nv; ++i) {
      const __m512 t = _mm512_mul_ps(_mm512_loadu_ps(yr + 16 * i), _mm512_loadu_ps(gamma + 16 * i));
      _mm512_storeu_ps(xr + 16 * i, _mm512_add_ps(_mm512_loadu_ps(xr + 16 * i), t));
    }
    for (size_t c = 16 * nv; c < cols; ++c) xr[c] = xr[c] + yr[c] * gamma[c];
  }
}

/* ------------------------------------------------------------ Q/K-norm + RoPE */

/* table[p] = 16 cos then 16 sin of p * inv_freq_j, inv_freq_j = 1/base^(2j/32),
 * angle rounded in f32, trig in double, as the oracle */
static float* rope_table(int max_pos, float base) {
  float inv[16];
  for (int j = 0; j < 16; ++j) inv[j] = 1.0f / powf(base, (float)(2 * j) / 32.0f);
  float* t = (float*)aligned_alloc(64, (size_t)(max_pos + 1) * 32 * sizeof(float));
  for (int p = 0; p <= max_pos; ++p)
    for (int j = 0; j < 16; ++j) {
      const float angle = (float)p * inv[j];
      t[p * 32 + j] = (float)cos((double)angle);
      t[p * 32 + 16 + j] = (float)sin((double)angle);
    }
  return t;
}

/* one 64-wide row in four zmm: LayerNorm, then rotate (v0, v1) by py and
 * (v2, v3) by px */
static inline void qk_row(float* row, const float* g, const float* b, float eps,
                          const float* cy, const float* cx) {
  __m512 v0 = _mm512_loadu_ps(row), v1 = _mm512_loadu_ps(row + 16);
  __m512 v2 = _mm512_loadu_ps(row + 32), v3 = _mm512_loadu_ps(row + 48);
  const float mean = hsum(_mm512_add_ps(_mm512_add_ps(v0, v1), _mm512_add_ps(v2, v3))) / 64.0f;
  const __m512 mv = _mm512_set1_ps(mean);
  const __m512 d0 = _mm512_sub_ps(v0, mv), d1 = _mm512_sub_ps(v1, mv);
  const __m512 d2 = _mm512_sub_ps(v2, mv), d3 = _mm512_sub_ps(v3, mv);
  const __m512 q = _mm512_add_ps(_mm512_add_ps(_mm512_mul_ps(d0, d0), _mm512_mul_ps(d1, d1)),
                                 _mm512_add_ps(_mm512_mul_ps(d2, d2), _mm512_mul_ps(d3, d3)));
  const float inv = 1.0f / sqrtf(hsum(q) / 64.0f + eps);
  const __m512 iv = _mm512_set1_ps(inv);
#define LNV(d, o) _mm512_add_ps(_mm512_mul_ps(_mm512_mul_ps(d, iv), _mm512_loadu_ps(g + o)), \
                                _mm512_loadu_ps(b + o))
  v0 = LNV(d0, 0);
  v1 = LNV(d1, 16);
  v2 = LNV(d2, 32);
  v3 = LNV(d3, 48);
#undef LNV
  const __m512 c0 = _mm512_loadu_ps(cy), s0 = _mm512_loadu_ps(cy + 16);
  const __m512 c1 = _mm512_loadu_ps(cx), s1 = _mm512_loadu_ps(cx + 16);
  const __m512 neg = _mm512_set1_ps(-0.0f);
  _mm512_storeu_ps(row, _mm512_add_ps(_mm512_mul_ps(v0, c0),
                                      _mm512_mul_ps(_mm512_xor_ps(v1, neg), s0)));
  _mm512_storeu_ps(row + 16, _mm512_add_ps(_mm512_mul_ps(v1, c0), _mm512_mul_ps(v0, s0)));
  _mm512_storeu_ps(row + 32, _mm512_add_ps(_mm512_mul_ps(v2, c1),
                                           _mm512_mul_ps(_mm512_xor_ps(v3, neg), s1)));
  _mm512_storeu_ps(row + 48, _mm512_add_ps(_mm512_mul_ps(v3, c1), _mm512_mul_ps(v2, s1)));
}

/* q, k [heads, n, 64] in place; pos_yx [n*2] f32 (truncated like the oracle) */
void cs_qk_norm_rope_f32(float* q, float* k, const float* qg, const float* qb, const float* kg,
                         const float* kb, const float* pos_yx, size_t heads, size_t n, float base,
                         float eps) {
  int max_pos = 0;
  for (size_t t = 0; t < 2 * n; ++t) {
    const int p = (int)pos_yx[t];
    if (p > max_pos) max_pos = p;
  }
  float* tab = rope_table(max_pos, base);
  long hr;
#pragma omp parallel for schedule(static)
  for (hr = 0; hr < (long)(heads * n); ++hr) {
    const size_t t = (size_t)hr % n;
    int py = (int)pos_yx[2 * t], px = (int)pos_yx[2 * t + 1];
    if (py < 0) py = 0;
    if (px < 0) px = 0;
    qk_row(q + (size_t)hr * 64, qg, qb, eps, tab + (size_t)py * 32, tab + (size_t)px * 32);
    qk_row(k + (size_t)hr * 64, kg, kb, eps, tab + (size_t)py * 32, tab + (size_t)px * 32);
  }
  free(tab);
}
