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
 *                    vestra-kernels crate and absent dumps.  The convention of
 *                    the upstream DA3 RotaryPositionEmbedding2D is restated
 *                    (rotate-half pairs (i, i+d/4) inside each half,
 *                    inv_freq_j = base^(-2j/(d/2))); tests pin it by
 *                    invariants (norm preservation, identity at (0,0),
 *                    relative-position property, recovered angles).
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
 * inv_freq_j = 1 / base^((2j)/half) for j < half/2, each step in f32
 * (RotaryPositionEmbedding2D of upstream Depth-Anything-3, referenced by the
 * reference's plan docs/plans/2026-07-18-rust-engine-v1.md:1290: "head_dim in
 * two halves y/x, each rotary over its coordinate", frequency 100). */
void ora_rope_inv_freq(float* inv_freq, size_t head_dim, float base) {
  const size_t half = head_dim / 2;
  for (size_t j = 0; j < half / 2; ++j) {
    const float e = (float)(2 * j) / (float)half;
    inv_freq[j] = 1.0f / powf(base, e);
  }
}

/* cos/sin of angle = (float)pos * inv_freq (f32 product), evaluated in
 * double and rounded once to f32. */
static void rope_cs(float pos, float inv_freq, float* c, float* s) {
  const float angle = pos * inv_freq;
  *c = (float)cos((double)angle);
  *s = (float)sin((double)angle);
}

/* Rotate one half (width hd2) by coordinate p: rotate-half pairing
 * out[i] = x[i]*cos_i - x[i+q]*sin_i, out[i+q] = x[i+q]*cos_i + x[i]*sin_i,
 * q = hd2/2, each product rounded then added (no FMA). */
static void rope_half(float* x, size_t hd2, float p, const float* inv_freq) {
  const size_t q = hd2 / 2;
  for (size_t i = 0; i < q; ++i) {
    float c, s;
    rope_cs(p, inv_freq[i], &c, &s);
    const float a = x[i];
    const float b = x[i + q];
    const float ac = a * c;
    const float nbs = (-b) * s;
    const float bc = b * c;
    const float as = a * s;
    x[i] = ac + nbs;
    x[i + q] = bc + as;
  }
}

/* vestra_kernels::rope2d(x[heads, n, head_dim], pos_yx[n*2] i64, base)
 * (interface docs/plans/2026-07-18-rust-engine-v1.md:1259; call site
 * crates/da-engine/src/vit_block.rs:944-948).  First half rotated by y,
 * second half by x. */
void ora_rope2d_f32(float* x, size_t heads, size_t n, size_t head_dim,
                    const int64_t* pos_yx, float base) {
  float inv_freq[512];
  ora_rope_inv_freq(inv_freq, head_dim, base);
  const size_t half = head_dim / 2;
  long hr;
#pragma omp parallel for schedule(static)
  for (hr = 0; hr < (long)(heads * n); ++hr) {
    const size_t t = (size_t)hr % n;
    float* row = x + (size_t)hr * head_dim;
    rope_half(row, half, (float)pos_yx[2 * t], inv_freq);
    rope_half(row + half, half, (float)pos_yx[2 * t + 1], inv_freq);
  }
}

/* qk_norm_rope_f32_da3_base: per (head, token) row LayerNorm over head_dim
 * with eps = QK_NORM_EPS (vit_block.rs:681-686), gamma/beta shared by all
 * heads, THEN 2D RoPE (order crates/da-graph/src/cpu_backend.rs:258-295;
 * fused call vit_block.rs:911-924; CUDA vit_block.rs:543-557).  Positions are
 * the reference's f32 device encoding, truncated to integers like the CPU
 * caller's `value as i64` (vit_block.rs:912). */
void ora_qk_norm_rope_f32(float* q, float* k, const float* q_gamma,
                          const float* q_beta, const float* k_gamma,
                          const float* k_beta, const float* pos_yx,
                          size_t heads, size_t n, size_t head_dim, float base,
                          float eps) {
  float inv_freq[512];
  ora_rope_inv_freq(inv_freq, head_dim, base);
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
    rope_half(qr, half, py, inv_freq);
    rope_half(qr + half, half, px, inv_freq);
    rope_half(kr, half, py, inv_freq);
    rope_half(kr + half, half, px, inv_freq);
  }
}

void ora_qk_norm_rope_w16(float* q, float* k, const uint16_t* q_gamma,
                          const uint16_t* q_beta, const uint16_t* k_gamma,
                          const uint16_t* k_beta, const float* pos_yx,
                          size_t heads, size_t n, size_t head_dim, float base,
                          float eps) {
  float* qg = widen(q_gamma, head_dim);
  float* qb = widen(q_beta, head_dim);
  float* kg = widen(k_gamma, head_dim);
  float* kb = widen(k_beta, head_dim);
  ora_qk_norm_rope_f32(q, k, qg, qb, kg, kb, pos_yx, heads, n, head_dim, base, eps);
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
