/*
 * vestra_oracle.h -- CPU restatement of the Depth-Anything-3 ViT-block fused
 * per-token operations, used ONLY as the checker (tests, smoke, and the CPU
 * baseline leg of bench.py).  Nothing in the product library links or calls
 * this code.
 *
 * Every function restates the reference algorithm in plain scalar C with
 * IEEE single precision, left-to-right (sequential) reductions and no FMA
 * contraction (built with -ffp-contract=off), i.e. the arithmetic order of the
 * reference's Rust scalar kernels.  Each definition in vestra_oracle.c cites
 * the reference file:line it follows.
 *
 * Parameter vectors may be IEEE binary16 ("w16" variants): they are widened
 * to f32 exactly, as the reference's GGUF loader does at load time
 * (crates/da-gguf/src/reader.rs:303-318).
 *
 * Row-parallel loops use OpenMP when built with -fopenmp; every row is
 * computed by exactly one thread with the same scalar order, so results do
 * not depend on the thread count.
 */
#ifndef VESTRA_ORACLE_H
#define VESTRA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- thread control for the CPU baseline ---- */
void ora_set_threads(int n);
int ora_get_threads(void);

/* ---- conversions ---- */
float ora_f16_to_f32(uint16_t h);
void ora_f16_to_f32_array(const uint16_t* h, float* out, size_t n);

/* ---- LayerNorm (block LN and per-head Q/K LN) ---- */
void ora_layernorm_f32(const float* x, float* y, size_t rows, size_t cols,
                       const float* gamma, const float* beta, float eps);
void ora_layernorm_w16(const float* x, float* y, size_t rows, size_t cols,
                       const uint16_t* gamma, const uint16_t* beta, float eps);

/* ---- GELU (exact-erf form) ---- */
float ora_erf_as7126(float x);
void ora_gelu_f32(float* x, size_t n);      /* erf = Abramowitz-Stegun 7.1.26 */
void ora_gelu_erff_f32(float* x, size_t n); /* erf = C library erff          */

/* ---- LayerScale, residual add ---- */
void ora_layerscale_f32(float* x, size_t rows, size_t cols, const float* gamma);
void ora_add_f32(float* dst, const float* src, size_t n);
void ora_layerscale_residual_f32(float* x, const float* y, const float* gamma,
                                 size_t rows, size_t cols);
void ora_layerscale_residual_w16(float* x, const float* y, const uint16_t* gamma,
                                 size_t rows, size_t cols);

/* ---- RoPE 2D ---- */
/* positions [rows*2] (y, x) as f32, special tokens (0,0) per view */
void ora_rope_positions(float* pos_yx, size_t n_special, size_t gh, size_t gw,
                        size_t view_count, int global);
/* RoPE convention flags (the same bits as the device ABI's VK_ROPE_*):
 * pairing (i, i+d/4) inside each half unless ORA_ROPE_INTERLEAVED (2i, 2i+1);
 * exponent 2j/(d/2) unless ORA_ROPE_EXP_HEAD (2j/d).  0 is the default. */
#define ORA_ROPE_INTERLEAVED 1u
#define ORA_ROPE_EXP_HEAD 2u
/* inverse frequency and angle tables of the 2D rotary embedding */
void ora_rope_inv_freq(float* inv_freq, size_t head_dim, float base);
void ora_rope_inv_freq_mode(float* inv_freq, size_t head_dim, float base, unsigned mode);
void ora_rope2d_f32(float* x, size_t heads, size_t n, size_t head_dim,
                    const int64_t* pos_yx, float base);
void ora_rope2d_mode_f32(float* x, size_t heads, size_t n, size_t head_dim,
                         const int64_t* pos_yx, float base, unsigned mode);
void ora_qk_norm_rope_f32(float* q, float* k, const float* q_gamma,
                          const float* q_beta, const float* k_gamma,
                          const float* k_beta, const float* pos_yx,
                          size_t heads, size_t n, size_t head_dim, float base,
                          float eps);
void ora_qk_norm_rope_mode_f32(float* q, float* k, const float* q_gamma,
                               const float* q_beta, const float* k_gamma,
                               const float* k_beta, const float* pos_yx,
                               size_t heads, size_t n, size_t head_dim,
                               float base, float eps, unsigned mode);
void ora_qk_norm_rope_w16(float* q, float* k, const uint16_t* q_gamma,
                          const uint16_t* q_beta, const uint16_t* k_gamma,
                          const uint16_t* k_beta, const float* pos_yx,
                          size_t heads, size_t n, size_t head_dim, float base,
                          float eps, unsigned mode);

/* ---- patch embedding ---- */
void ora_normalize_u8_hwc(const uint8_t* img, float* chw, size_t h, size_t w,
                          const float mean[3], const float std_[3]);
void ora_patchify_nchw(const float* img, float* rows_out, size_t h, size_t w,
                       size_t patch, size_t channels);
/* out[m, n] = x[m, k] @ wt[k, n] + bias[n], sequential k */
void ora_linear_f32(const float* x, const float* wt, const float* bias,
                    float* out, size_t m, size_t k, size_t n);
/* conv weight OIHW [embed, 3, p, p] -> token-major patch projection */
void ora_patch_project_oihw(const float* img_chw, size_t h, size_t w,
                            size_t patch, const float* w_oihw,
                            const float* bias, size_t embed, float* out);
void ora_pos_embed_bicubic(const float* pos_embed, size_t grid, size_t embed,
                           size_t gh, size_t gw, float interp_offset,
                           float* out);
void ora_assemble_tokens(const float* patch_tokens, size_t gh, size_t gw,
                         size_t embed, const float* cls,
                         const float* registers, size_t n_register,
                         const float* pos_table, float* out);
void ora_patch_embed_u8(const uint8_t* img_hwc, size_t h, size_t w,
                        size_t patch, const float mean[3], const float std_[3],
                        const float* w_oihw, const float* bias, size_t embed,
                        const float* cls, const float* registers,
                        size_t n_register, const float* pos_table, float* out);
void ora_overwrite_prefix_f32(float* tokens, const float* prefix, size_t len);
void ora_split_qkv_hnd(const float* qkv, size_t n, size_t heads, size_t head_dim,
                       float* q, float* k, float* v);
void ora_hnd_to_token(const float* hnd, size_t n, size_t heads, size_t head_dim,
                      float* out);
void ora_attention_f32(const float* q, const float* k, const float* v, size_t batches,
                       size_t n, size_t head_dim, float* out);

void ora_resize_bilinear_u8(const uint8_t* src, size_t sw, size_t sh, uint8_t* dst, size_t dw,
                            size_t dh);
void ora_resize_cubic_u8(const uint8_t* src, size_t sw, size_t sh, uint8_t* dst, size_t dw,
                         size_t dh);
void ora_resize_area_u8(const uint8_t* src, size_t sw, size_t sh, uint8_t* dst, size_t dw,
                        size_t dh);
int ora_preprocess_shape(size_t h, size_t w, size_t image_size, size_t patch, int upper_bound,
                         size_t dims_out[4]);
void ora_preprocess_resize_u8(const uint8_t* src, size_t h, size_t w, size_t image_size,
                              size_t patch, int upper_bound, uint8_t* dst);

#ifdef __cplusplus
}
#endif
#endif
