/*
 * vestra_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Scalar CPU restatement of the reference's fused ViT-block per-token
 * operations.  It is the checker the HIP library is compared against; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Arithmetic rules (matching the reference's Rust scalar kernels):
 *   - IEEE f32 everywhere, each operation rounded (compiled with
 *     -ffp-contract=off, no -ffast-math: Rust never contracts a*b+c into FMA);
 *   - reductions are sequential, left to right over the row;
 *   - parameter vectors stored as binary16 are widened exactly.
 *
 * Pinning status per function (what checks it besides the GPU comparison):
 *   layernorm        pinned: in-tree restatement dpt_head.rs:272-296, tests
 *                    against float64 brute force and torch.nn.functional.
 *                    layer_norm fixtures, eps discriminator.
 *   gelu (A&S)       erf algorithm of vestra-kernels @783bd66 is not in the
 *                    reference tree; the documented scalar twin
 *                    (docs/plans/2026-07-18-rust-engine-v1.md:865-876) is
 *                    restated.  Pinned against exact-erf GELU fixtures within
 *                    the A&S error bound and the plan's known answers.
 *   layerscale/add   pinned by closed form and graph-op test values.
 *   rope positions   pinned: vit_block.rs:841-881 restated, tests reproduce
 *                    the reference's per-view special-token layout.
 *   rope2d rotation  PARITY UNPINNED against the reference: the pairing and
 *                    frequency exponent live only in the absent
 *                    vestra-kernels crate and absent dumps.  Both are
 *                    selectable (mode flags as the device ABI's VK_ROPE_*):
 *                    pairing rotate-half (i, i+d/4) inside each half (the
 *                    upstream DA3 RotaryPositionEmbedding2D, the default) or
 *                    interleaved (2i, 2i+1); exponent inv_freq_j =
 *                    base^(-2j/(d/2)) (default) or base^(-2j/d).  Tests pin
 *                    each form to the mathematics: complex-multiplication
 *                    twins, closed-form angles (j = 0 turns by p radians,
 *                    base 100 at j = 8 by p/10 or p/sqrt(10)), norm
 *                    preservation, identity at (0,0), relative positions.
 *   patch embed      pinned: patch_embed.rs:280-339 known answers (10, 18,
 *                    42, 50; bias broadcast), preprocess.rs:549-583
 *                    normalisation, float64 GEMM brute force.
 *   pos-embed        pos_embed.rs:73-83,122-169 restated; pinned by
 *                    pos_embed.rs:357-442 known answers, identity resize,
 *                    partition of unity and torch bicubic fixtures.
 */
#include "vestra_oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void ora_set_threads(int n) {
  g_threads = n < 1 ? 1 : n;
#ifdef _OPENMP
  omp_set_num_threads(g_threads);
#endif
}

int ora_get_threads(void) { return g_threads; }

/* IEEE binary16 -> binary32, exact (half 2.7.1 `f16::to_f32`, used by
 * crates/da-gguf/src/reader.rs:316). */
float ora_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      /* subnormal: renormalise */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

void ora_f16_to_f32_array(const uint16_t* h, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = ora_f16_to_f32(h[i]);
}

static float* widen(const uint16_t* h, size_t n) {
  float* f = (float*)malloc(n * sizeof(float));
  ora_f16_to_f32_array(h, f, n);
  return f;
}

/* One LayerNorm row.  vestra_kernels::scalar::layernorm as restated in-tree
 * by crates/da-engine/src/dpt_head.rs:272-296 and
 * docs/plans/2026-07-18-rust-engine-v1.md:854-863:
 *   mean = (sum x) / cols            sequential sum
 *   var  = (sum (x-mean)^2) / cols   sequential sum, biased, two-pass
 *   inv  = 1 / sqrt(var + eps)
 *   y    = (x - mean) * inv * gamma + beta   (left to right)            */
static void ln_row(const float* x, float* y, size_t cols, const float* gamma,
                   const float* beta, float eps) {
  float sum = 0.0f;
  for (size_t c = 0; c < cols; ++c) sum += x[c];
  const float mean = sum / (float)cols;
  float sq = 0.0f;
  for (size_t c = 0; c < cols; ++c) {
    const float d = x[c] - mean;
    sq += d * d;
  }
  const float var = sq / (float)cols;
  const float inv = 1.0f / sqrtf(var + eps);
  for (size_t c = 0; c < cols; ++c) y[c] = (x[c] - mean) * inv * gamma[c] + beta[c];
}

/* crates/da-engine/src/vit_block.rs:696-714 (run_layernorm: copy, then
 * scalar::layernorm in place); CUDA twin layernorm_f32_cpu_order at
 * vit_block.rs:528-537.  Out-of-place here; x == y is allowed. */
void ora_layernorm_f32(const float* x, float* y, size_t rows, size_t cols,
                       const float* gamma, const float* beta, float eps) {
  long r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < (long)rows; ++r)
    ln_row(x + (size_t)r * cols, y + (size_t)r * cols, cols, gamma, beta, eps);
}

void ora_layernorm_w16(const float* x, float* y, size_t rows, size_t cols,
                       const uint16_t* gamma, const uint16_t* beta, float eps) {
  float* g = widen(gamma, cols);
  float* b = widen(beta, cols);
  ora_layernorm_f32(x, y, rows, cols, g, b, eps);
  free(g);
  free(b);
}

/* Abramowitz & Stegun 7.1.26 (|error| < 1.5e-7), the erf of the reference's
 * documented scalar GELU twin, docs/plans/2026-07-18-rust-engine-v1.md:870-876.
 * Rust's f32::signum returns +1 for +0.0 and -1 for -0.0. */
float ora_erf_as7126(float x) {
  const float s = signbit(x) ? -1.0f : 1.0f;
  const float a = fabsf(x);
  const float t = 1.0f / (1.0f + 0.3275911f * a);
  float p = 1.0614054f * t - 1.4531520f;
  p = p * t;
  p = p + 1.4214137f;
  p = p * t - 0.28449674f;
  p = p * t + 0.25482959f;
  const float y = 1.0f - p * t * expf(-a * a);
  return s * y;
}

/* Exact-erf GELU, y = 0.5*x*(1+erf(x/sqrt2)), left to right
 * (docs/plans/2026-07-18-rust-engine-v1.md:865-868; Kernels::gelu call site
 * crates/da-engine/src/vit_block.rs:752-754; CUDA gelu_f32_in_place
 * vit_block.rs:578,642). */
void ora_gelu_f32(float* x, size_t n) {
  const float inv_sqrt2 = 0.70710678f;
  long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long)n; ++i) {
    const float v = x[i];
    x[i] = 0.5f * v * (1.0f + ora_erf_as7126(v * inv_sqrt2));
  }
}

void ora_gelu_erff_f32(float* x, size_t n) {
  const float inv_sqrt2 = 0.70710678f;
  long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long)n; ++i) {
    const float v = x[i];
    x[i] = 0.5f * v * (1.0f + erff(v * inv_sqrt2));
  }
}

/* scalar::layerscale, x[r,c] *= gamma[c]: op contract
 * crates/da-graph/src/graph.rs:58-66, call site vit_block.rs:755-759. */
void ora_layerscale_f32(float* x, size_t rows, size_t cols, const float* gamma) {
  long r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < (long)rows; ++r)
    for (size_t c = 0; c < cols; ++c) x[(size_t)r * cols + c] *= gamma[c];
}

/* Kernels::add / CUDA add_f32_in_place, dst += src
 * (crates/da-engine/src/vit_block.rs:669-679). */
void ora_add_f32(float* dst, const float* src, size_t n) {
  long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long)n; ++i) dst[i] += src[i];
}

/* LayerScale then residual add as the reference sequences them
 * (vit_block.rs:755-758 then add_residual 1090/1130): t = y*gamma (rounded),
 * x = x + t (rounded).  Two roundings, never an FMA. */
void ora_layerscale_residual_f32(float* x, const float* y, const float* gamma,
                                 size_t rows, size_t cols) {
  long r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < (long)rows; ++r) {
    for (size_t c = 0; c < cols; ++c) {
      const size_t i = (size_t)r * cols + c;
      const float t = y[i] * gamma[c];
      x[i] = x[i] + t;
    }
  }
}

void ora_layerscale_residual_w16(float* x, const float* y, const uint16_t* gamma,
                                 size_t rows, size_t cols) {
  float* g = widen(gamma, cols);
  ora_layerscale_residual_f32(x, y, g, rows, cols);
  free(g);
}

/* RoPE positions, crates/da-engine/src/vit_block.rs:841-881 (device twin
 * 512-526): per view the first n_special tokens keep (0,0); patch idx gets
 * (idx/gw + 1, idx%gw + 1) in local layers and (1,1) in global layers. */
void ora_rope_positions(float* pos_yx, size_t n_special, size_t gh, size_t gw,
                        size_t view_count, int global) {
  const size_t per_view = n_special + gh * gw;
  memset(pos_yx, 0, per_view * view_count * 2 * sizeof(float));
  for (size_t v = 0; v < view_count; ++v) {
    for (size_t lt = n_special; lt < per_view; ++lt) {
      const size_t t = v * per_view + lt;
      if (global) {
        pos_yx[2 * t] = 1.0f;
        pos_yx[2 * t + 1] = 1.0f;
      } else {
        const size_t idx = lt - n_special;
        pos_yx[2 * t] = (float)(idx / gw + 1);
        pos_yx[2 * t + 1] = (float)(idx % gw + 1);
      }
    }
  }
}

/* Inverse frequencies of one rotary half of width half = head_dim/2:
 * inv_freq_j = 1 / base^((2j)/denom) for j < half/2, each step in f32, with
 * denom = half (mode without ORA_ROPE_EXP_HEAD: RotaryPositionEmbedding2D
 * of upstream Depth-Anything-3, referenced by the reference's plan
 * docs/plans/2026-07-18-rust-engine-v1.md:1290: "head_dim in two halves y/x,
 * each rotary over its coordinate", frequency 100) or denom = head_dim
 * (ORA_ROPE_EXP_HEAD). */
void ora_rope_inv_freq_mode(float* inv_freq, size_t head_dim, float base, unsigned mode) {
  const size_t half = head_dim / 2;
  const float denom = (float)((mode & ORA_ROPE_EXP_HEAD) ? head_dim : half);
  for (size_t j = 0; j < half / 2; ++j) {
    const float e = (float)(2 * j) / denom;
    inv_freq[j] = 1.0f / powf(base, e);
  }
}

void ora_rope_inv_freq(float* inv_freq, size_t head_dim, float base) {
  ora_rope_inv_freq_mode(inv_freq, head_dim, base, 0);
}

/* cos/sin of angle = (float)pos * inv_freq (f32 product), evaluated in
 * double and rounded once to f32. */
static void rope_cs(float pos, float inv_freq, float* c, float* s) {
  const float angle = pos * inv_freq;
  *c = (float)cos((double)angle);
  *s = (float)sin((double)angle);
}

/* Rotate one half (width hd2) by coordinate p.  Pair i (i < hd2/2) is
 * (x[i], x[i+hd2/2]) with rotate-half pairing, (x[2i], x[2i+1]) with
 * ORA_ROPE_INTERLEAVED; a pair (a, b) becomes (a*cos_i - b*sin_i,
 * b*cos_i + a*sin_i), each product rounded then added (no FMA). */
static void rope_half(float* x, size_t hd2, float p, const float* inv_freq, unsigned mode) {
  const size_t q = hd2 / 2;
  const int inter = (mode & ORA_ROPE_INTERLEAVED) != 0;
  for (size_t i = 0; i < q; ++i) {
    float c, s;
    rope_cs(p, inv_freq[i], &c, &s);
    const size_t ia = inter ? 2 * i : i;
    const size_t ib = inter ? 2 * i + 1 : i + q;
    const float a = x[ia];
    const float b = x[ib];
    const float ac = a * c;
    const float nbs = (-b) * s;
    const float bc = b * c;
    const float as = a * s;
    x[ia] = ac + nbs;
    x[ib] = bc + as;
  }
}

/* vestra_kernels::rope2d(x[heads, n, head_dim], pos_yx[n*2] i64, base)
 * (interface docs/plans/2026-07-18-rust-engine-v1.md:1259; call site
 * crates/da-engine/src/vit_block.rs:944-948).  First half rotated by y,
 * second half by x. */
void ora_rope2d_mode_f32(float* x, size_t heads, size_t n, size_t head_dim,
                         const int64_t* pos_yx, float base, unsigned mode) {
  float inv_freq[512];
  ora_rope_inv_freq_mode(inv_freq, head_dim, base, mode);
  const size_t half = head_dim / 2;
  long hr;
#pragma omp parallel for schedule(static)
  for (hr = 0; hr < (long)(heads * n); ++hr) {
    const size_t t = (size_t)hr % n;
    float* row = x + (size_t)hr * head_dim;
    rope_half(row, half, (float)pos_yx[2 * t], inv_freq, mode);
    rope_half(row + half, half, (float)pos_yx[2 * t + 1], inv_freq, mode);
  }
}

void ora_rope2d_f32(float* x, size_t heads, size_t n, size_t head_dim,
                    const int64_t* pos_yx, float base) {
  ora_rope2d_mode_f32(x, heads, n, head_dim, pos_yx, base, 0);
}

/* qk_norm_rope_f32_da3_base: per (head, token) row LayerNorm over head_dim
 * with eps = QK_NORM_EPS (vit_block.rs:681-686), gamma/beta shared by all
 * heads, THEN 2D RoPE (order crates/da-graph/src/cpu_backend.rs:258-295;
 * fused call vit_block.rs:911-924; CUDA vit_block.rs:543-557).  Positions are
 * the reference's f32 device encoding, truncated to integers like the CPU
 * caller's `value as i64` (vit_block.rs:912). */
void ora_qk_norm_rope_mode_f32(float* q, float* k, const float* q_gamma,
                               const float* q_beta, const float* k_gamma,
                               const float* k_beta, const float* pos_yx,
                               size_t heads, size_t n, size_t head_dim,
                               float base, float eps, unsigned mode) {
  float inv_freq[512];
  ora_rope_inv_freq_mode(inv_freq, head_dim, base, mode);
  const size_t half = head_dim / 2;
  long hr;
#pragma omp parallel for schedule(static)
  for (hr = 0; hr < (long)(heads * n); ++hr) {
    const size_t t = (size_t)hr % n;
    const float py = (float)(int64_t)pos_yx[2 * t];
    const float px = (float)(int64_t)pos_yx[2 * t + 1];
    float* qr = q + (size_t)hr * head_dim;
    float* kr = k + (size_t)hr * head_dim;
    ln_row(qr, qr, head_dim, q_gamma, q_beta, eps);
    ln_row(kr, kr, head_dim, k_gamma, k_beta, eps);
    rope_half(qr, half, py, inv_freq, mode);
    rope_half(qr + half, half, px, inv_freq, mode);
    rope_half(kr, half, py, inv_freq, mode);
    rope_half(kr + half, half, px, inv_freq, mode);
  }
}

void ora_qk_norm_rope_f32(float* q, float* k, const float* q_gamma,
                          const float* q_beta, const float* k_gamma,
                          const float* k_beta, const float* pos_yx,
                          size_t heads, size_t n, size_t head_dim, float base,
                          float eps) {
  ora_qk_norm_rope_mode_f32(q, k, q_gamma, q_beta, k_gamma, k_beta, pos_yx, heads,
                            n, head_dim, base, eps, 0);
}

void ora_qk_norm_rope_w16(float* q, float* k, const uint16_t* q_gamma,
                          const uint16_t* q_beta, const uint16_t* k_gamma,
                          const uint16_t* k_beta, const float* pos_yx,
                          size_t heads, size_t n, size_t head_dim, float base,
                          float eps, unsigned mode) {
  float* qg = widen(q_gamma, head_dim);
  float* qb = widen(q_beta, head_dim);
  float* kg = widen(k_gamma, head_dim);
  float* kb = widen(k_beta, head_dim);
  ora_qk_norm_rope_mode_f32(q, k, qg, qb, kg, kb, pos_yx, heads, n, head_dim, base,
                            eps, mode);
  free(qg);
  free(qb);
  free(kg);
  free(kb);
}

/* preprocess normalisation, crates/da-engine/src/preprocess.rs:484-500:
 * HWC u8 -> CHW f32, v = u8/255 then (v - mean[c]) / std[c] (true division). */
void ora_normalize_u8_hwc(const uint8_t* img, float* chw, size_t h, size_t w,
                          const float mean[3], const float std_[3]) {
  for (size_t c = 0; c < 3; ++c)
    for (size_t y = 0; y < h; ++y)
      for (size_t x = 0; x < w; ++x) {
        const float v = (float)img[(y * w + x) * 3 + c] / 255.0f;
        chw[c * h * w + y * w + x] = (v - mean[c]) / std_[c];
      }
}

/* patchify_nchw_f32 (crates/da-engine/src/patch_embed.rs:221-223): NCHW ->
 * patch rows [gh*gw, C*p*p] with column index c*p*p + ky*p + kx (OIHW
 * flattening, patch_embed.rs:176-181), patch index r*gw + col. */
void ora_patchify_nchw(const float* img, float* rows_out, size_t h, size_t w,
                       size_t patch, size_t channels) {
  const size_t gh = h / patch, gw = w / patch, kdim = channels * patch * patch;
  for (size_t pr = 0; pr < gh; ++pr)
    for (size_t pc = 0; pc < gw; ++pc) {
      float* dst = rows_out + (pr * gw + pc) * kdim;
      for (size_t c = 0; c < channels; ++c)
        for (size_t ky = 0; ky < patch; ++ky)
          for (size_t kx = 0; kx < patch; ++kx)
            dst[c * patch * patch + ky * patch + kx] =
                img[c * h * w + (pr * patch + ky) * w + pc * patch + kx];
    }
}

/* run_linear without LayerScale (crates/da-engine/src/vit_block.rs:750-751):
 * out = x @ wt (scalar gemm_f32, sequential k, plans:817-826), then
 * add_bias_rows.  wt is [k, n] (the engine's transposed orientation,
 * engine.rs:110-126). */
void ora_linear_f32(const float* x, const float* wt, const float* bias,
                    float* out, size_t m, size_t k, size_t n) {
  long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long)m; ++i) {
    float* o = out + (size_t)i * n;
    for (size_t j = 0; j < n; ++j) o[j] = 0.0f;
    for (size_t p = 0; p < k; ++p) {
      const float a = x[(size_t)i * k + p];
      const float* b = wt + p * n;
      for (size_t j = 0; j < n; ++j) o[j] += a * b[j];
    }
    if (bias)
      for (size_t j = 0; j < n; ++j) o[j] += bias[j];
  }
}

/* patch_embed (crates/da-engine/src/patch_embed.rs:53-130): non-overlapping
 * conv with OIHW weight [embed, 3, p, p], bias, written token-major
 * [gh*gw, embed].  out[t, e] = (sum_k W[e,k] * patch_t[k]) + b[e], sequential
 * in k = c*p*p + ky*p + kx. */
void ora_patch_project_oihw(const float* img_chw, size_t h, size_t w,
                            size_t patch, const float* w_oihw,
                            const float* bias, size_t embed, float* out) {
  const size_t gh = h / patch, gw = w / patch, kdim = 3 * patch * patch;
  const size_t np = gh * gw;
  float* rows = (float*)malloc(np * kdim * sizeof(float));
  ora_patchify_nchw(img_chw, rows, h, w, patch, 3);
  long t;
#pragma omp parallel for schedule(static)
  for (t = 0; t < (long)np; ++t) {
    const float* a = rows + (size_t)t * kdim;
    for (size_t e = 0; e < embed; ++e) {
      const float* we = w_oihw + e * kdim;
      float acc = 0.0f;
      for (size_t kk = 0; kk < kdim; ++kk) acc += we[kk] * a[kk];
      out[(size_t)t * embed + e] = acc + bias[e];
    }
  }
  free(rows);
}

/* Keys cubic kernel, a = -0.75 (crates/da-engine/src/pos_embed.rs:73-83). */
static float cubic(float x) {
  const float A = -0.75f;
  x = fabsf(x);
  if (x < 1.0f) return ((A + 2.0f) * x - (A + 3.0f)) * x * x + 1.0f;
  if (x < 2.0f) return (((x - 5.0f) * x + 8.0f) * x - 4.0f) * A;
  return 0.0f;
}

static long clampl(long v, long lo, long hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* interpolate_pos_embed (crates/da-engine/src/pos_embed.rs:122-169): bicubic
 * resize of the learned [grid*grid+1, embed] table to [1+gh*gw, embed],
 * half-pixel centres, scale (g + offset)/grid, clamp-to-edge 4x4 taps,
 * acc += wy*wx*src in dy-major order, CLS row passed through. */
void ora_pos_embed_bicubic(const float* pos_embed, size_t grid, size_t embed,
                           size_t gh, size_t gw, float interp_offset,
                           float* out) {
  memcpy(out, pos_embed, embed * sizeof(float));
  const float m = (float)grid;
  const float sx = ((float)gw + interp_offset) / m;
  const float sy = ((float)gh + interp_offset) / m;
  long oy;
#pragma omp parallel for schedule(static)
  for (oy = 0; oy < (long)gh; ++oy) {
    const float iy = ((float)oy + 0.5f) / sy - 0.5f;
    const long y0 = (long)floorf(iy);
    const float fy = iy - (float)y0;
    for (size_t ox = 0; ox < gw; ++ox) {
      const float ix = ((float)ox + 0.5f) / sx - 0.5f;
      const long x0 = (long)floorf(ix);
      const float fx = ix - (float)x0;
      float* orow = out + (1 + (size_t)oy * gw + ox) * embed;
      for (size_t ch = 0; ch < embed; ++ch) {
        float acc = 0.0f;
        for (long dy = -1; dy <= 2; ++dy) {
          const float wy = cubic(fy - (float)dy);
          const long yy = clampl(y0 + dy, 0, (long)grid - 1);
          for (long dx = -1; dx <= 2; ++dx) {
            const float wx = cubic(fx - (float)dx);
            const long xx = clampl(x0 + dx, 0, (long)grid - 1);
            const float src = pos_embed[(1 + (size_t)yy * grid + (size_t)xx) * embed + ch];
            acc += wy * wx * src;
          }
        }
        orow[ch] = acc;
      }
    }
  }
}

/* assemble_tokens_from_patch_tokens (crates/da-engine/src/pos_embed.rs:254-306)
 * / CUDA prepend_cls_add_pos_f32 (patch_embed.rs:234-240): row 0 = cls +
 * pos[0]; rows 1..n_special-1 = register tokens, no position add; row
 * n_special + p = patch_p + pos[1 + p]. */
void ora_assemble_tokens(const float* patch_tokens, size_t gh, size_t gw,
                         size_t embed, const float* cls,
                         const float* registers, size_t n_register,
                         const float* pos_table, float* out) {
  const size_t np = gh * gw, ns = 1 + n_register;
  for (size_t c = 0; c < embed; ++c) out[c] = cls[c] + pos_table[c];
  for (size_t r = 0; r < n_register; ++r)
    for (size_t c = 0; c < embed; ++c) out[(1 + r) * embed + c] = registers[r * embed + c];
  for (size_t i = 0; i < np * embed; ++i)
    out[ns * embed + i] = patch_tokens[i] + pos_table[embed + i];
}

/* The whole per-image path: normalise (preprocess.rs:484-500) -> patch
 * projection (patch_embed.rs:53-130) -> token assembly (pos_embed.rs:254-306). */
void ora_patch_embed_u8(const uint8_t* img_hwc, size_t h, size_t w,
                        size_t patch, const float mean[3], const float std_[3],
                        const float* w_oihw, const float* bias, size_t embed,
                        const float* cls, const float* registers,
                        size_t n_register, const float* pos_table, float* out) {
  const size_t np = (h / patch) * (w / patch);
  float* chw = (float*)malloc(3 * h * w * sizeof(float));
  float* proj = (float*)malloc(np * embed * sizeof(float));
  ora_normalize_u8_hwc(img_hwc, chw, h, w, mean, std_);
  ora_patch_project_oihw(chw, h, w, patch, w_oihw, bias, embed, proj);
  ora_assemble_tokens(proj, h / patch, w / patch, embed, cls, registers,
                      n_register, pos_table, out);
  free(chw);
  free(proj);
}

/* overwrite_prefix_f32: camera-token slot write
 * (crates/da-engine/src/vit_block.rs:452-478; backbone.rs:446-457). */
void ora_overwrite_prefix_f32(float* tokens, const float* prefix, size_t len) {
  memcpy(tokens, prefix, len * sizeof(float));
}

/* split_qkv_hnd_f32: token-major QKV [n, 3*heads*head_dim] with column order
 * Q | K | V, each block [heads, head_dim] head-major, to three head-major
 * [heads, n, head_dim] tensors: the pack loop of
 * crates/da-engine/src/vit_block.rs:818-833 (dst = (h*n + t)*head_dim,
 * src = h*head_dim, + embed for K, + 2*embed for V). */
void ora_split_qkv_hnd(const float* qkv, size_t n, size_t heads, size_t head_dim,
                       float* q, float* k, float* v) {
  const size_t embed = heads * head_dim;
  for (size_t t = 0; t < n; ++t) {
    const float* row = qkv + t * 3 * embed;
    for (size_t h = 0; h < heads; ++h) {
      const size_t dst = (h * n + t) * head_dim, src = h * head_dim;
      memcpy(q + dst, row + src, head_dim * sizeof(float));
      memcpy(k + dst, row + embed + src, head_dim * sizeof(float));
      memcpy(v + dst, row + 2 * embed + src, head_dim * sizeof(float));
    }
  }
}

/* hnd_to_token_f32: attention output head-major [heads, n, head_dim] back to
 * token-major [n, heads*head_dim] (the inverse layout of the pack loop above;
 * crates/da-engine/src/vit_block.rs:560 calls it before the projection). */
void ora_hnd_to_token(const float* hnd, size_t n, size_t heads, size_t head_dim,
                      float* out) {
  for (size_t t = 0; t < n; ++t)
    for (size_t h = 0; h < heads; ++h)
      memcpy(out + (t * heads + h) * head_dim, hnd + (h * n + t) * head_dim,
             head_dim * sizeof(float));
}

/* Scaled dot-product attention softmax(Q K^T / sqrt(head_dim)) V over each of
 * `batches` independent head-major sequences [n, head_dim] (a head of one
 * view, or a head of the whole flattened sequence): the core of Op::Attention
 * (crates/da-graph/src/graph.rs:370-400, cpu_backend.rs:198-260) and of the
 * reference's `attention_online_f32` / `vestra_kernels::attention`
 * (crates/da-engine/src/vit_block.rs:363, 559, 952).  The reference's own
 * kernel is outside the tree; this restatement is the textbook max-shifted
 * softmax: s_j = (sum_d q_d k_jd) * (1/sqrt(head_dim)), p_j = expf(s_j - max),
 * out = (sum_j p_j v_j) / (sum_j p_j), every sum sequential in f32. */
void ora_attention_f32(const float* q, const float* k, const float* v, size_t batches,
                       size_t n, size_t head_dim, float* out) {
  const float scale = 1.0f / sqrtf((float)head_dim);
  #pragma omp parallel for schedule(static)
  for (long long bi = 0; bi < (long long)(batches * n); ++bi) {
    const size_t b = (size_t)bi / n, i = (size_t)bi % n;
    const float* qi = q + (b * n + i) * head_dim;
    const float* kb = k + b * n * head_dim;
    const float* vb = v + b * n * head_dim;
    float* o = out + (b * n + i) * head_dim;
    float* s = (float*)malloc(n * sizeof(float));
    float mx = -INFINITY;
    for (size_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (size_t d = 0; d < head_dim; ++d) acc += qi[d] * kb[j * head_dim + d];
      s[j] = acc * scale;
      if (s[j] > mx) mx = s[j];
    }
    float l = 0.0f;
    for (size_t j = 0; j < n; ++j) {
      s[j] = expf(s[j] - mx);
      l += s[j];
    }
    for (size_t d = 0; d < head_dim; ++d) {
      float acc = 0.0f;
      for (size_t j = 0; j < n; ++j) acc += s[j] * vb[j * head_dim + d];
      o[d] = acc / l;
    }
    free(s);
  }
}

/* ---------------------------------------------------------------------------
 * Image preprocessing resize (crates/da-engine/src/preprocess.rs:236-482).
 * u8 HWC RGB in and out; f32 arithmetic where the reference uses f32, f64
 * where it uses f64, every operation rounded; results rounded half-to-even
 * and clamped to [0, 255] (saturating_round_u8, preprocess.rs:234-236).
 * ------------------------------------------------------------------------- */
static uint8_t sat_round_u8(float v) {
  float r = rintf(v); /* default rounding mode: ties to even */
  if (r < 0.0f) r = 0.0f;
  if (r > 255.0f) r = 255.0f;
  return (uint8_t)r;
}

/* cubic_weight, Keys a = -0.75 (preprocess.rs:240-251), f32. */
static float cubic_w(float x) {
  const float A = -0.75f;
  x = fabsf(x);
  if (x < 1.0f) return ((A + 2.0f) * x - (A + 3.0f)) * x * x + 1.0f;
  if (x < 2.0f) return (((x - 5.0f) * x + 8.0f) * x - 4.0f) * A;
  return 0.0f;
}

/* resize_bilinear_u8 (preprocess.rs:253-280). */
void ora_resize_bilinear_u8(const uint8_t* src, size_t sw, size_t sh, uint8_t* dst, size_t dw,
                            size_t dh) {
  const float sx = (float)sw / (float)dw, sy = (float)sh / (float)dh;
  for (size_t y = 0; y < dh; ++y) {
    const float fy = ((float)y + 0.5f) * sy - 0.5f;
    const long y0 = (long)floorf(fy);
    const float wy = fy - (float)y0;
    const size_t y0c = (size_t)clampl(y0, 0, (long)sh - 1), y1c = (size_t)clampl(y0 + 1, 0, (long)sh - 1);
    for (size_t x = 0; x < dw; ++x) {
      const float fx = ((float)x + 0.5f) * sx - 0.5f;
      const long x0 = (long)floorf(fx);
      const float wx = fx - (float)x0;
      const size_t x0c = (size_t)clampl(x0, 0, (long)sw - 1), x1c = (size_t)clampl(x0 + 1, 0, (long)sw - 1);
      for (size_t c = 0; c < 3; ++c) {
        const float top = (float)src[(y0c * sw + x0c) * 3 + c] * (1.0f - wx) +
                          (float)src[(y0c * sw + x1c) * 3 + c] * wx;
        const float bottom = (float)src[(y1c * sw + x0c) * 3 + c] * (1.0f - wx) +
                             (float)src[(y1c * sw + x1c) * 3 + c] * wx;
        dst[(y * dw + x) * 3 + c] = sat_round_u8(top * (1.0f - wy) + bottom * wy);
      }
    }
  }
}

/* Taps of one output coordinate of the cubic resize: fx in f64, the
 * fractional part rounded to f32, weights in f32 (preprocess.rs:286-300). */
static void cubic_taps(size_t d, double s, size_t n_src, long idx[4], float w[4]) {
  const double f = ((double)d + 0.5) * s - 0.5;
  const long i = (long)floor(f);
  const float t = (float)(f - (double)i);
  w[0] = cubic_w(t + 1.0f);
  w[1] = cubic_w(t);
  w[2] = cubic_w(t - 1.0f);
  w[3] = cubic_w(t - 2.0f);
  for (int k = 0; k < 4; ++k) idx[k] = clampl(i - 1 + k, 0, (long)n_src - 1);
}

/* resize_cubic_u8 (preprocess.rs:282-338): horizontal pass over every source
 * row into f32, then the vertical pass, each a 4-tap sum from 0 in tap
 * order. */
void ora_resize_cubic_u8(const uint8_t* src, size_t sw, size_t sh, uint8_t* dst, size_t dw,
                         size_t dh) {
  const double sx = (double)sw / (double)dw, sy = (double)sh / (double)dh;
  float* tmp = (float*)malloc(sh * dw * 3 * sizeof(float));
  for (size_t x = 0; x < dw; ++x) {
    long ix[4];
    float wx[4];
    cubic_taps(x, sx, sw, ix, wx);
    for (size_t y = 0; y < sh; ++y)
      for (size_t c = 0; c < 3; ++c) {
        float sum = 0.0f;
        for (int k = 0; k < 4; ++k) sum += wx[k] * (float)src[(y * sw + (size_t)ix[k]) * 3 + c];
        tmp[(y * dw + x) * 3 + c] = sum;
      }
  }
  for (size_t y = 0; y < dh; ++y) {
    long iy[4];
    float wy[4];
    cubic_taps(y, sy, sh, iy, wy);
    for (size_t x = 0; x < dw; ++x)
      for (size_t c = 0; c < 3; ++c) {
        float sum = 0.0f;
        for (int k = 0; k < 4; ++k) sum += wy[k] * tmp[((size_t)iy[k] * dw + x) * 3 + c];
        dst[(y * dw + x) * 3 + c] = sat_round_u8(sum);
      }
  }
  free(tmp);
}

/* area_table taps of one destination (preprocess.rs:347-382), in the
 * reference's order; returns the count (at most cap). */
static int area_taps(size_t d, size_t n_src, size_t n_dst, long* src, float* w, int cap) {
  const double scale = (double)n_src / (double)n_dst;
  const double start_f = (double)d * scale;
  const double end_f = start_f + scale;
  const double cell = fmin(scale, (double)n_src - start_f);
  size_t start = (size_t)ceil(start_f);
  size_t end = (size_t)floor(end_f);
  if (end > n_src - 1) end = n_src - 1;
  if (start > end) start = end;
  int n = 0;
  if ((double)start - start_f > 1e-3 && n < cap) {
    src[n] = (long)start - 1;
    w[n++] = (float)(((double)start - start_f) / cell);
  }
  for (size_t s = start; s < end && n < cap; ++s) {
    src[n] = (long)s;
    w[n++] = (float)(1.0 / cell);
  }
  if (end_f - (double)end > 1e-3 && n < cap) {
    src[n] = (long)end;
    w[n++] = (float)(fmin(fmin(end_f - (double)end, 1.0), cell) / cell);
  }
  return n;
}

/* resize_area_u8 (preprocess.rs:384-409): bilinear when neither axis shrinks,
 * else the separable box filter, sums from 0 in tap order. */
void ora_resize_area_u8(const uint8_t* src, size_t sw, size_t sh, uint8_t* dst, size_t dw,
                        size_t dh) {
  if (dw >= sw && dh >= sh) {
    ora_resize_bilinear_u8(src, sw, sh, dst, dw, dh);
    return;
  }
  enum { CAP = 4096 };
  long* ts = (long*)malloc(CAP * sizeof(long));
  float* tw = (float*)malloc(CAP * sizeof(float));
  float* tmp = (float*)calloc(sh * dw * 3, sizeof(float));
  for (size_t x = 0; x < dw; ++x) {
    const int n = area_taps(x, sw, dw, ts, tw, CAP);
    for (size_t y = 0; y < sh; ++y)
      for (size_t c = 0; c < 3; ++c) {
        float acc = 0.0f;
        for (int k = 0; k < n; ++k) acc += tw[k] * (float)src[(y * sw + (size_t)ts[k]) * 3 + c];
        tmp[(y * dw + x) * 3 + c] = acc;
      }
  }
  for (size_t y = 0; y < dh; ++y) {
    const int n = area_taps(y, sh, dh, ts, tw, CAP);
    for (size_t x = 0; x < dw; ++x)
      for (size_t c = 0; c < 3; ++c) {
        float acc = 0.0f;
        for (int k = 0; k < n; ++k) acc += tw[k] * tmp[((size_t)ts[k] * dw + x) * 3 + c];
        dst[(y * dw + x) * 3 + c] = sat_round_u8(acc);
      }
  }
  free(ts);
  free(tw);
  free(tmp);
}

static size_t nearest_multiple(size_t v, size_t m) {
  const size_t down = v / m * m, up = down + m;
  const size_t du = up - v, dd = v - down;
  return du <= dd ? up : down;
}

/* preprocess's resize policy (preprocess.rs:432-469): the bound side (max
 * for upper-bound modes, min for "lower*") to image_size, sizes rounded half
 * to even, cubic when enlarging, area otherwise; then both sides snapped to
 * the nearest patch multiple with a second resize.  dims_out = boundary h,
 * w, output h, w.  Returns 0 when the scale is exactly 1 (plain copy). */
int ora_preprocess_shape(size_t h, size_t w, size_t image_size, size_t patch, int upper_bound,
                         size_t dims_out[4]) {
  const size_t target = image_size ? image_size : 1, p = patch ? patch : 1;
  const size_t bound = upper_bound ? (w > h ? w : h) : (w < h ? w : h);
  const double scale = (double)target / (double)bound;
  size_t bw = (size_t)nearbyint((double)w * scale), bh = (size_t)nearbyint((double)h * scale);
  if (bw < 1) bw = 1;
  if (bh < 1) bh = 1;
  size_t ow = nearest_multiple(bw, p), oh = nearest_multiple(bh, p);
  if (ow < 1) ow = 1;
  if (oh < 1) oh = 1;
  dims_out[0] = bh;
  dims_out[1] = bw;
  dims_out[2] = oh;
  dims_out[3] = ow;
  return fabs(scale - 1.0) < 2.220446049250313e-16 ? 0 : 1;
}

void ora_preprocess_resize_u8(const uint8_t* src, size_t h, size_t w, size_t image_size,
                              size_t patch, int upper_bound, uint8_t* dst) {
  size_t d[4];
  const int scaled = ora_preprocess_shape(h, w, image_size, patch, upper_bound, d);
  const size_t target = image_size ? image_size : 1;
  const size_t bound = upper_bound ? (w > h ? w : h) : (w < h ? w : h);
  const double scale = (double)target / (double)bound;
  uint8_t* mid = (uint8_t*)malloc(d[0] * d[1] * 3);
  if (!scaled)
    memcpy(mid, src, h * w * 3);
  else if (scale > 1.0)
    ora_resize_cubic_u8(src, w, h, mid, d[1], d[0]);
  else
    ora_resize_area_u8(src, w, h, mid, d[1], d[0]);
  if (d[2] != d[0] || d[3] != d[1]) {
    if (d[3] > d[1] || d[2] > d[0])
      ora_resize_cubic_u8(mid, d[1], d[0], dst, d[3], d[2]);
    else
      ora_resize_area_u8(mid, d[1], d[0], dst, d[3], d[2]);
  } else {
    memcpy(dst, mid, d[0] * d[1] * 3);
  }
  free(mid);
}
