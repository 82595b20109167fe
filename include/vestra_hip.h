/*
 * vestra_hip.h -- C ABI of the MI355X (gfx950) fused ViT-block operations.
 *
 * This is the drop-in boundary for the Depth-Anything-3 ViT block's fused
 * per-token path.  It mirrors the device runtime the reference engine calls
 * (`vestra_kernels::cuda::CudaRuntime`, used by
 * crates/da-engine/src/vit_block.rs:136-667 and
 * crates/da-engine/src/patch_embed.rs:139-245), so a Rust `extern "C"` binding
 * can stand where the CUDA runtime stood.  Every entry point names the
 * reference method it replaces.
 *
 * Conventions
 *  - Plain C types only: opaque handles, pointers and sizes.  No C++ or torch
 *    types cross this boundary.
 *  - Every function returns an `int` status (VK_OK == 0, negative on error)
 *    and never aborts.  The message of the last failure on the calling host
 *    thread is returned by vk_last_error().  VK_ERR_UNSUPPORTED marks a shape
 *    or option outside the kernels' qualified subset: a caller maps it to the
 *    reference's `None` (fall back to the CPU path), see vit_block.rs:331-333.
 *  - One HIP stream per runtime.  Device work is stream-ordered and
 *    asynchronous; vk_download_*, vk_runtime_synchronize and
 *    vk_event_elapsed_ms block.  A runtime must not be used from two host
 *    threads at once without external locking; separate runtimes are
 *    independent.
 *  - Tensors are flat, contiguous, typed device buffers (f32, f16, u8, or
 *    i32 / i64 for RoPE positions).
 *    Creators allocate; every creator has a matching destroy.  In-place
 *    operations take the tensor handle they modify; the reference's
 *    "consume and return the token tensor" (vit_block.rs:489-499,563) is
 *    "in place on the same handle" here.
 *  - Activations are f32.  Parameter vectors (LayerNorm/QK-norm gamma and
 *    beta, LayerScale gamma) may be f32 or f16 (GGUF F16 element layout,
 *    crates/da-gguf/src/reader.rs:303-318); f16 is widened exactly in
 *    registers, so results equal the f32 path on the widened values.
 */
#ifndef VESTRA_HIP_H
#define VESTRA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VK_ABI_VERSION 2

typedef enum vk_status {
  VK_OK = 0,
  VK_ERR_INVALID = -1,     /* bad handle, null pointer, size mismatch      */
  VK_ERR_UNSUPPORTED = -2, /* outside the qualified shape/option subset   */
  VK_ERR_HIP = -3,         /* HIP runtime error                            */
  VK_ERR_OOM = -4          /* device allocation failed                      */
} vk_status;

/* VK_I32 / VK_I64: integer RoPE positions (the reference's CPU kernels take
 * `&[i64]` positions, vit_block.rs:911-924, 944-948). */
typedef enum vk_dtype {
  VK_F32 = 0,
  VK_F16 = 1,
  VK_U8 = 2,
  VK_I32 = 3,
  VK_I64 = 4
} vk_dtype;

typedef struct vk_runtime vk_runtime;
typedef struct vk_tensor vk_tensor;
typedef struct vk_linear vk_linear;
typedef struct vk_event vk_event;
typedef struct vk_graph vk_graph;

/* ------------------------------------------------------------------ */
/* errors, version                                                      */
/* ------------------------------------------------------------------ */

/* Message of the last failed call on this host thread ("" if none).
 * Replaces the payload of `CudaError::Kernel(String)`
 * (crates/da-engine/src/patch_embed.rs:207-217). */
const char* vk_last_error(void);
int vk_abi_version(void);

/* ------------------------------------------------------------------ */
/* runtime                                                              */
/* ------------------------------------------------------------------ */

/* CudaRuntime::new(device) (engine.rs:284-385 enable_cuda_*). */
int vk_runtime_create(int device, vk_runtime** out);
/* Waits for the runtime's queued work and retires the handle: it takes no
 * new work (calls on it fail).  Tensors, linears and events created on it
 * may still be destroyed afterwards; the stream and the runtime's own
 * buffers are released with the last of them.  Launching a graph captured
 * on it fails afterwards (VK_ERR_INVALID). */
int vk_runtime_destroy(vk_runtime* rt);
/* Blocks until all work queued on the runtime's stream has finished. */
int vk_runtime_synchronize(vk_runtime* rt);
/* The runtime's hipStream_t, for callers that enqueue their own work. */
void* vk_runtime_stream(vk_runtime* rt);
/* Number of compute units of the runtime's device (0 on error). */
int vk_runtime_cu_count(vk_runtime* rt);

/* Summation order of the LayerNorm mean and variance, for every LayerNorm
 * the runtime enqueues after the call: vk_layernorm_f32 / _into, the fused
 * LayerScale + residual + LayerNorm (and the block's camera-slot form), the
 * capture and the token -> CHW hand-off, the LayerNorm the residual
 * projections write for the next block, and the per-(head, token) Q/K
 * LayerNorm (standalone, in the block sequences and in the QKV projection's
 * epilogue).
 *   VK_LN_ORDER_TREE (default): a wave-level tree; results match the CPU
 *     within rtol 1e-5 (every fused form gives the bits of the separate
 *     calls).
 *   VK_LN_ORDER_SEQUENTIAL: the CPU kernel's order, what the reference's
 *     layernorm_f32_cpu_order names (vit_block.rs:528-537; the sums of
 *     dpt_head.rs:272-296): mean = (x0 + x1 + ... ) / cols and the biased
 *     two-pass variance summed left to right, inv = 1/sqrtf(var + eps)
 *     correctly rounded, y = (x - mean) * inv * gamma + beta -- every
 *     LayerNorm then gives the CPU's bits.  Slower: a sum in that order is
 *     one chain of dependent adds per row.
 * The order of captured graphs is the order at capture.  Returns
 * VK_ERR_INVALID for other values. */
#define VK_LN_ORDER_TREE 0
#define VK_LN_ORDER_SEQUENTIAL 1
int vk_runtime_set_layernorm_order(vk_runtime* rt, int order);
/* The runtime's current LayerNorm order (negative status on error). */
int vk_runtime_layernorm_order(vk_runtime* rt);

/* ------------------------------------------------------------------ */
/* tensors and transfers                                                */
/* ------------------------------------------------------------------ */

/* Uninitialised device tensor of `len` elements. */
int vk_tensor_alloc(vk_runtime* rt, vk_dtype dtype, size_t len, vk_tensor** out);
/* Non-owning view of caller-owned device memory (destroy frees the handle
 * only). */
int vk_tensor_wrap(vk_runtime* rt, vk_dtype dtype, void* device_ptr, size_t len,
                   vk_tensor** out);
int vk_tensor_destroy(vk_tensor* t);
size_t vk_tensor_len(const vk_tensor* t);
int vk_tensor_dtype(const vk_tensor* t);
void* vk_tensor_device_ptr(const vk_tensor* t);

/* CudaRuntime::upload_f32 (vit_block.rs:161-184, 335). Synchronous. */
int vk_upload_f32(vk_runtime* rt, const float* host, size_t len, vk_tensor** out);
int vk_upload_f16(vk_runtime* rt, const uint16_t* host, size_t len, vk_tensor** out);
int vk_upload_u8(vk_runtime* rt, const uint8_t* host, size_t len, vk_tensor** out);
/* Integer RoPE positions [rows*2] (y, x) for vk_qk_norm_rope_mode_f32 and
 * vk_rope2d_f32.  Synchronous. */
int vk_upload_i32(vk_runtime* rt, const int32_t* host, size_t len, vk_tensor** out);
int vk_upload_i64(vk_runtime* rt, const int64_t* host, size_t len, vk_tensor** out);
/* Host -> existing tensor (len must equal the tensor length). Synchronous. */
int vk_write_f32(vk_runtime* rt, vk_tensor* t, const float* host, size_t len);
int vk_write_u8(vk_runtime* rt, vk_tensor* t, const uint8_t* host, size_t len);
/* CudaRuntime::download_f32 (vit_block.rs:370, 659-662). Blocks. */
int vk_download_f32(vk_runtime* rt, const vk_tensor* t, float* host, size_t len);
/* The same for u8 tensors (images). Blocks. */
int vk_download_u8(vk_runtime* rt, const vk_tensor* t, uint8_t* host, size_t len);
/* CudaRuntime::copy_f32 (backbone.rs:991-1027). New tensor. */
int vk_copy_f32(vk_runtime* rt, const vk_tensor* src, vk_tensor** out);
/* CudaRuntime::copy_segment_f32: new tensor = src[offset .. offset+len]. */
int vk_copy_segment_f32(vk_runtime* rt, const vk_tensor* src, size_t offset,
                        size_t len, vk_tensor** out);
/* CudaRuntime::copy_segment_into_f32: dst[dst_off..+len] = src[src_off..+len]. */
int vk_copy_segment_into_f32(vk_runtime* rt, vk_tensor* dst, size_t dst_offset,
                             const vk_tensor* src, size_t src_offset, size_t len);
/* CudaRuntime::overwrite_prefix_f32 (vit_block.rs:452-478): tokens[0..len] =
 * prefix[0..len] -- the camera-token slot write. */
int vk_overwrite_prefix_f32(vk_runtime* rt, vk_tensor* tokens,
                            const vk_tensor* prefix, size_t len);

/* ------------------------------------------------------------------ */
/* fused per-token operations                                            */
/* ------------------------------------------------------------------ */

/* CudaRuntime::layernorm_f32_cpu_order(x, gamma, beta, rows, cols, eps)
 * (vit_block.rs:528-537, 567-576, 627-636): row LayerNorm, biased two-pass
 * variance, y = (x-mean)*inv*gamma + beta.  Returns a new tensor.  The
 * mean and variance sum in the runtime's LayerNorm order
 * (vk_runtime_set_layernorm_order): a wave-level tree by default, matching
 * the CPU within rtol 1e-5; with VK_LN_ORDER_SEQUENTIAL the CPU's own
 * left-to-right order and its bits.  cols % 4 == 0, cols <= 8192. */
int vk_layernorm_f32(vk_runtime* rt, const vk_tensor* x, const vk_tensor* gamma,
                     const vk_tensor* beta, size_t rows, size_t cols, float eps,
                     vk_tensor** out);
/* Same into an existing tensor (out may equal x: in place, as
 * scalar::layernorm in vit_block.rs:712). */
int vk_layernorm_into_f32(vk_runtime* rt, const vk_tensor* x,
                          const vk_tensor* gamma, const vk_tensor* beta,
                          size_t rows, size_t cols, float eps, vk_tensor* out);

/* CudaRuntime::gelu_f32_in_place (vit_block.rs:578, 642): exact-erf GELU
 * 0.5*x*(1+erf(x/sqrt2)) with the erf of the reference's scalar kernel
 * (Abramowitz-Stegun 7.1.26, docs/plans/2026-07-18-rust-engine-v1.md:870-876). */
int vk_gelu_f32_inplace(vk_runtime* rt, vk_tensor* x);
/* Same with the device library's erff in place of A&S 7.1.26. */
int vk_gelu_erf_f32_inplace(vk_runtime* rt, vk_tensor* x);

/* CudaRuntime::add_f32_in_place (vit_block.rs:564, 580, 660): dst += src. */
int vk_add_f32_inplace(vk_runtime* rt, vk_tensor* dst, const vk_tensor* src);
/* scalar::layerscale (vit_block.rs:755-759; graph.rs:58-66): x[r,c] *= g[c]. */
int vk_layerscale_f32_inplace(vk_runtime* rt, vk_tensor* x, const vk_tensor* gamma,
                              size_t rows, size_t cols);
/* LayerScale + residual, fused: x += gamma (.) y, as t = y*gamma; x = x + t
 * (two roundings; the reference's LS-folded projection epilogue
 * vit_block.rs:214-222,303-313 followed by add_f32_in_place).  gamma NULL
 * means an unscaled residual add (presence gating, vit_block.rs:740-748). */
int vk_layerscale_residual_f32(vk_runtime* rt, vk_tensor* x, const vk_tensor* y,
                               const vk_tensor* gamma, size_t rows, size_t cols);
/* LayerScale + residual followed by the next LayerNorm in one pass:
 * x += gamma (.) y; ln_out = LayerNorm(x).  Equal to
 * vk_layerscale_residual_f32 then vk_layernorm_into_f32 (the block's
 * add_residual -> LN2 step, vit_block.rs:1090-1106; and the LS2 residual ->
 * next block's LN1).  No reference counterpart as one call. */
int vk_layerscale_residual_layernorm_f32(vk_runtime* rt, vk_tensor* x,
                                         const vk_tensor* y,
                                         const vk_tensor* ls_gamma,
                                         const vk_tensor* ln_gamma,
                                         const vk_tensor* ln_beta, size_t rows,
                                         size_t cols, float eps,
                                         vk_tensor* ln_out);

/* 2D RoPE convention, `rope_mode` = one pairing | one exponent flag.
 * Every row of head_dim 64 splits into a y half (elements 0..31, rotated by
 * the row's y coordinate) and an x half (32..63, rotated by x), with the
 * frequency base `freq` (100 for DA3, config.rs:375).  The pairing inside a
 * half and the frequency exponent are fixed only inside the reference's
 * kernel crate (vestra-kernels, absent from its tree; its value test needs
 * absent dumps, crates/da-engine/tests/kernel_rope_parity.rs:4-19), so both
 * are selectable.  The default (0) is the rotation of Depth-Anything-3's
 * RotaryPositionEmbedding2D. */
#define VK_ROPE_ROTATE_HALF 0u /* pairs (j, j+16) of each half, j < 16        */
#define VK_ROPE_INTERLEAVED 1u /* pairs (2i, 2i+1) of each half, i < 16        */
#define VK_ROPE_EXP_HALF 0u    /* pair j turns by p * freq^(-2j/32)            */
#define VK_ROPE_EXP_HEAD 2u    /* pair j turns by p * freq^(-2j/64)            */
#define VK_ROPE_DEFAULT 0u

/* CudaRuntime::qk_norm_rope_f32_da3_base(q, k, q_gamma, q_beta, k_gamma,
 * k_beta, positions, heads, rows, freq, eps) (vit_block.rs:343-357, 543-557):
 * in place on head-major q and k [heads, rows, 64]: LayerNorm over each
 * (head, token) row of 64 with eps (QK_NORM_EPS = 1e-5, vit_block.rs:686),
 * then 2D RoPE with positions [rows*2] (y, x) f32 on the device.  head_dim is
 * 64 (the reference's da3_base qualification). */
int vk_qk_norm_rope_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k,
                        const vk_tensor* q_gamma, const vk_tensor* q_beta,
                        const vk_tensor* k_gamma, const vk_tensor* k_beta,
                        const vk_tensor* positions, size_t heads, size_t rows,
                        float freq, float eps);
/* The same with an explicit RoPE convention (VK_ROPE_* flags; 0 gives
 * vk_qk_norm_rope_f32) and positions of dtype f32 (the CUDA runtime's
 * device encoding, truncated toward zero as `value as i64` reads it: NaN
 * gives 0, +-inf saturates), i32 or i64 (the CPU kernel's `&[i64]`,
 * qk_norm_rope_f32_da3_base at vit_block.rs:911-924).  Every position p of
 * any dtype and range turns by the angle (float)p * inv_freq_j, the CPU
 * kernel's conversion (an i64 of 2^32 + 5 rotates by (float)(2^32 + 5)).
 * Positions outside the runtime's cos/sin table (negative or above 1023
 * and every grid coordinate seen so far) take that f32 angle and the
 * device's single-precision sincosf (within 2 ulp of the table's
 * double-rounded values). */
int vk_qk_norm_rope_mode_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k,
                             const vk_tensor* q_gamma, const vk_tensor* q_beta,
                             const vk_tensor* k_gamma, const vk_tensor* k_beta,
                             const vk_tensor* positions, size_t heads,
                             size_t rows, float freq, float eps,
                             unsigned rope_mode);
/* vestra_kernels::rope2d(x, heads, n, head_dim, pos_yx, freq)
 * (vit_block.rs:944-948; cpu_backend.rs:286-295): the 2D rotation alone, in
 * place on one head-major tensor x [heads, rows, 64], positions [rows*2]
 * (y, x) of dtype f32, i32 or i64, convention `rope_mode`. */
int vk_rope2d_f32(vk_runtime* rt, vk_tensor* x, const vk_tensor* positions,
                  size_t heads, size_t rows, size_t head_dim, float freq,
                  unsigned rope_mode);

/* Layouts of q/k for the grid form below. */
typedef enum vk_qk_layout {
  /* [heads, view_count * tokens_per_view, head_dim]: one head-major sequence,
   * the flattened multi-view layout of global layers (backbone.rs:770-796). */
  VK_QK_HEADS_OUTER = 0,
  /* [view_count, heads, tokens_per_view, head_dim]: one head-major block per
   * view, i.e. view_count independent local-layer calls in one launch. */
  VK_QK_VIEWS_OUTER = 1
} vk_qk_layout;

/* Q/K-norm + RoPE with positions computed on the device from the patch grid
 * (vit_block.rs:841-881 / 512-526): per view, tokens < n_special get (0,0);
 * patch p gets (p/gw+1, p%gw+1), or (1,1) for every patch when `global` is
 * non-zero.  rows = view_count * (n_special + gh*gw).  Replaces the host
 * position build + upload of run_tail_device (vit_block.rs:512-526, 542).
 * q_gamma/q_beta/k_gamma/k_beta NULL skips the LayerNorm (qk-norm gating,
 * vit_block.rs:835-838); head_dim == 64. */
int vk_qk_norm_rope_grid_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k,
                             const vk_tensor* q_gamma, const vk_tensor* q_beta,
                             const vk_tensor* k_gamma, const vk_tensor* k_beta,
                             size_t heads, size_t head_dim, size_t n_special,
                             size_t gh, size_t gw, size_t view_count,
                             int global, vk_qk_layout layout, float freq,
                             float eps);
/* The grid form with an explicit RoPE convention (0 gives the call above). */
int vk_qk_norm_rope_grid_mode_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k,
                                  const vk_tensor* q_gamma,
                                  const vk_tensor* q_beta,
                                  const vk_tensor* k_gamma,
                                  const vk_tensor* k_beta, size_t heads,
                                  size_t head_dim, size_t n_special,
                                  size_t gh, size_t gw, size_t view_count,
                                  int global, vk_qk_layout layout,
                                  float freq, float eps, unsigned rope_mode);

/* Device positions tensor [rows*2] f32, as built on the host at
 * vit_block.rs:512-526 (for callers of vk_qk_norm_rope_f32). */
int vk_rope_positions_f32(vk_runtime* rt, size_t n_special, size_t gh,
                          size_t gw, size_t view_count, int global,
                          vk_tensor** out);

/* ------------------------------------------------------------------ */
/* patch embedding                                                      */
/* ------------------------------------------------------------------ */

/* CudaRuntime::patchify_nchw_f32(img, h, w, patch, channels)
 * (patch_embed.rs:221-223): NCHW f32 -> patch rows [gh*gw, channels*p*p],
 * column c*p*p + ky*p + kx. */
int vk_patchify_nchw_f32(vk_runtime* rt, const vk_tensor* img, size_t h,
                         size_t w, size_t patch, size_t channels,
                         vk_tensor** out);

/* CudaRuntime::prepare_linear_f32(in, out, W[in x out], bias, ls_gamma)
 * (vit_block.rs:214-222, 303-313; patch_embed.rs:176-189): caches the
 * weights on the device.  ls_gamma may be NULL.  Host pointers, synchronous. */
int vk_linear_prepare_f32(vk_runtime* rt, size_t in_features,
                          size_t out_features, const float* weight_in_out,
                          const float* bias, const float* ls_gamma,
                          vk_linear** out);
/* The same from an OIHW conv filter [out, in] (patch_embed.rs:176-181 does
 * this transpose on the host; here the kernel reads OIHW directly). */
int vk_linear_prepare_oihw_f32(vk_runtime* rt, size_t in_features,
                               size_t out_features, const float* weight_out_in,
                               const float* bias, vk_linear** out);
/* The same from the weight as a GGUF file stores it: IEEE binary16
 * (GGML_F16) or Q8_0 blocks (GGML_Q8_0: 34 bytes per 32 values, an f16
 * scale d then 32 int8 q, value d*q; crates/da-gguf/src/q8_0.rs:10-33).
 * The reference widens / dequantises at load (Gguf::tensor_f32,
 * crates/da-gguf/src/reader.rs:279-349) and prepares the f32 values; here
 * the stored bytes are uploaded and expanded on the device into the same
 * resident f32 layout.  Both conversions are exact, so runs give the bits
 * of vk_linear_prepare_f32 / _oihw_f32 on the widened weights.  Q8_0 needs
 * in*out % 32 == 0 and nbytes == in*out/32*34.  bias / ls_gamma are f32. */
int vk_linear_prepare_w16(vk_runtime* rt, size_t in_features,
                          size_t out_features, const uint16_t* weight_in_out,
                          const float* bias, const float* ls_gamma,
                          vk_linear** out);
int vk_linear_prepare_q8_0(vk_runtime* rt, size_t in_features,
                           size_t out_features, const uint8_t* blocks,
                           size_t nbytes, const float* bias,
                           const float* ls_gamma, vk_linear** out);
int vk_linear_prepare_oihw_w16(vk_runtime* rt, size_t in_features,
                               size_t out_features,
                               const uint16_t* weight_out_in,
                               const float* bias, vk_linear** out);
/* Gguf::tensor_f32 for F16 and Q8_0 tensors (reader.rs:302-337) on the
 * device: dst f32 [len] from an f16 tensor, or from u8 Q8_0 blocks holding
 * n values (n % 32 == 0). */
int vk_widen_f16_f32(vk_runtime* rt, const vk_tensor* src, vk_tensor* dst);
int vk_dequantize_q8_0_f32(vk_runtime* rt, const vk_tensor* blocks, size_t n,
                           vk_tensor* dst);
int vk_linear_destroy(vk_linear* lin);
size_t vk_linear_input_features(const vk_linear* lin);
/* CudaLinearF32::run(x, rows): y = (x @ W + b) [* gamma], F32 MFMA with f32
 * accumulation.  New tensor [rows, out]. */
int vk_linear_run_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x,
                      size_t rows, vk_tensor** out);
/* The same into a caller tensor out [rows, out] (no allocation; capturable
 * in a HIP graph).  out must not overlap x. */
int vk_linear_run_into_f32(vk_runtime* rt, const vk_linear* lin,
                           const vk_tensor* x, size_t rows, vk_tensor* out);
/* FC1 + GELU in one pass: out = GELU(x @ W + b), the erf of
 * vk_gelu_f32_inplace (A&S 7.1.26), bit-identical to vk_linear_run_into_f32
 * followed by vk_gelu_f32_inplace.  Replaces CudaLinearF32::run then
 * CudaRuntime::gelu_f32_in_place (vit_block.rs:578, 642), the reference's own
 * FC1-epilogue fusion on the CPU (docs/optimization-log.md:292).  The linear
 * must carry no LayerScale. */
int vk_linear_run_gelu_f32(vk_runtime* rt, const vk_linear* lin,
                           const vk_tensor* x, size_t rows, vk_tensor* out);
/* The same with the device erff (vk_gelu_erf_f32_inplace's GELU). */
int vk_linear_run_gelu_erf_f32(vk_runtime* rt, const vk_linear* lin,
                               const vk_tensor* x, size_t rows, vk_tensor* out);
/* proj / FC2 + LayerScale + residual in one pass:
 * residual += (x @ W + b) [* gamma], each step rounded as in the unfused
 * sequence (bit-identical to vk_linear_run_into_f32 then vk_add_f32_inplace).
 * Replaces CudaLinearF32::run with Some(ls) followed by
 * CudaRuntime::add_f32_in_place (vit_block.rs:214-222, 303-313, 563-564, 580).
 * residual [rows, out] must not overlap x. */
int vk_linear_run_residual_f32(vk_runtime* rt, const vk_linear* lin,
                               const vk_tensor* x, size_t rows,
                               vk_tensor* residual);

/* ------------------------------------------------------------------ */
/* attention-block layout glue (head_dim contiguous, head-major)        */
/* ------------------------------------------------------------------ */

/* CudaRuntime::split_qkv_hnd_f32(qkv, rows, heads, head_dim)
 * (vit_block.rs:539-541): token-major QKV [rows, 3*heads*head_dim], columns
 * Q | K | V each [heads, head_dim] (vit_block.rs:38-43), to head-major Q, K,
 * V [heads, rows, head_dim] (the pack loop of vit_block.rs:818-833).
 * head_dim % 4 == 0.  New tensors / caller tensors (no overlap). */
int vk_split_qkv_hnd_f32(vk_runtime* rt, const vk_tensor* qkv, size_t rows,
                         size_t heads, size_t head_dim, vk_tensor** q,
                         vk_tensor** k, vk_tensor** v);
int vk_split_qkv_hnd_into_f32(vk_runtime* rt, const vk_tensor* qkv,
                              size_t rows, size_t heads, size_t head_dim,
                              vk_tensor* q, vk_tensor* k, vk_tensor* v);
/* CudaRuntime::hnd_to_token_f32(hnd, rows, heads, head_dim)
 * (vit_block.rs:560): head-major [heads, rows, head_dim] to token-major
 * [rows, heads*head_dim]. */
int vk_hnd_to_token_f32(vk_runtime* rt, const vk_tensor* hnd, size_t rows,
                        size_t heads, size_t head_dim, vk_tensor** out);
int vk_hnd_to_token_into_f32(vk_runtime* rt, const vk_tensor* hnd,
                             size_t rows, size_t heads, size_t head_dim,
                             vk_tensor* out);
/* The QKV projection storing head-major Q, K, V directly: bit-identical to
 * vk_linear_run_into_f32 followed by vk_split_qkv_hnd_into_f32.  The device
 * form of vestra_kernels::qkv_f32_da3_base (vit_block.rs:813-814), replacing
 * CudaLinearF32::run + split_qkv_hnd_f32 (vit_block.rs:538-541).
 * head_dim 64, out_features = 3*heads*64, no LayerScale. */
int vk_linear_run_qkv_hnd_f32(vk_runtime* rt, const vk_linear* lin,
                              const vk_tensor* x, size_t rows, size_t heads,
                              size_t head_dim, vk_tensor* q, vk_tensor* k,
                              vk_tensor* v);
/* The QKV projection with Q/K-norm + 2D RoPE in its epilogue: bit-identical
 * to vk_linear_run_qkv_hnd_f32 followed by vk_qk_norm_rope_grid_f32 with
 * VK_QK_HEADS_OUTER (same arguments; q_gamma..k_beta NULL: RoPE only), and
 * one pass less over Q and K.  The device path of the QKV run + split +
 * qk_norm_rope_f32_da3_base of run_tail_device (vit_block.rs:537-557).
 * rows = view_count * (n_special + gh*gw); head_dim 64. */
int vk_linear_run_qkv_hnd_norm_rope_f32(
    vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
    size_t heads, size_t head_dim, vk_tensor* q, vk_tensor* k, vk_tensor* v,
    const vk_tensor* q_gamma, const vk_tensor* q_beta, const vk_tensor* k_gamma,
    const vk_tensor* k_beta, size_t n_special, size_t gh, size_t gw,
    size_t view_count, int global, float freq, float eps);
/* The same with an explicit RoPE convention (0 gives the call above). */
int vk_linear_run_qkv_hnd_norm_rope_mode_f32(
    vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
    size_t heads, size_t head_dim, vk_tensor* q, vk_tensor* k, vk_tensor* v,
    const vk_tensor* q_gamma, const vk_tensor* q_beta, const vk_tensor* k_gamma,
    const vk_tensor* k_beta, size_t n_special, size_t gh, size_t gw,
    size_t view_count, int global, float freq, float eps, unsigned rope_mode);
/* vk_linear_run_into_f32 that allocates nothing.  No counterpart in the
 * reference: for callers that cannot call hipMalloc (a sequence captured
 * into a HIP graph without an eager run first, serving loops, harnesses that
 * forbid allocation).  The same plan and bits as vk_linear_run_into_f32;
 * split-K partial sums (few rows: an 866-token image's FC2 needs 4 Mi
 * floats) go to a static device array of 8 Mi floats (32 MiB, held by each
 * device from the library's load until the process ends) instead of the
 * runtime's work buffer.  A plan needing more than that fails with
 * VK_ERR_UNSUPPORTED and enqueues nothing (e.g. 3,458 rows x 4096 -> 1024).
 * Every call on one device shares the array: calls on one device that
 * overlap in time (two runtimes' streams) race. */
int vk_linear_run_into_noalloc_f32(vk_runtime* rt, const vk_linear* lin,
                                   const vk_tensor* x, size_t rows,
                                   vk_tensor* out);
/* The output projection reading the head-major attention output
 * [heads, rows, 64] directly (in_features = heads*64): bit-identical to
 * vk_hnd_to_token_into_f32 followed by vk_linear_run_into_f32 /
 * vk_linear_run_residual_f32.  Replaces hnd_to_token_f32 + projection run
 * (+ add_f32_in_place) (vit_block.rs:560-563). */
int vk_linear_run_hnd_into_f32(vk_runtime* rt, const vk_linear* lin,
                               const vk_tensor* hnd, size_t rows, size_t heads,
                               size_t head_dim, vk_tensor* out);
int vk_linear_run_hnd_residual_f32(vk_runtime* rt, const vk_linear* lin,
                                   const vk_tensor* hnd, size_t rows,
                                   size_t heads, size_t head_dim,
                                   vk_tensor* residual);

/* CudaRuntime::attention_online_f32(q, k, v, heads, rows, head_dim)
 * (vit_block.rs:363, 559) and the CPU vestra_kernels::attention
 * (vit_block.rs:952): out = softmax(Q K^T / sqrt(head_dim)) V over each of
 * `heads` independent head-major sequences [rows, head_dim] of q, k, v
 * ([heads, rows, head_dim]).  A view-major local-layer batch
 * [views, heads, tokens, 64] is the same call with heads = views*heads and
 * rows = tokens.  head_dim 64.  New tensor / caller tensor (no overlap with
 * q, k or v). */
int vk_attention_online_f32(vk_runtime* rt, const vk_tensor* q,
                            const vk_tensor* k, const vk_tensor* v,
                            size_t heads, size_t rows, size_t head_dim,
                            vk_tensor** out);
int vk_attention_into_f32(vk_runtime* rt, const vk_tensor* q,
                          const vk_tensor* k, const vk_tensor* v,
                          size_t heads, size_t rows, size_t head_dim,
                          vk_tensor* out);

/* CudaRuntime::prepend_cls_add_pos_f32(patches, cls, pos, n_patches, embed)
 * (patch_embed.rs:234-240): row 0 = cls + pos[0]; row 1+p = patch_p + pos[1+p]. */
int vk_prepend_cls_add_pos_f32(vk_runtime* rt, const vk_tensor* patches,
                               const vk_tensor* cls, const vk_tensor* pos,
                               size_t n_patches, size_t embed, vk_tensor** out);

/* PosEmbedCache::get_or_build / interpolate_pos_embed (pos_embed.rs:122-218):
 * bicubic (Keys a=-0.75) resize of the learned [grid*grid+1, embed] table to
 * [1+gh*gw, embed], CLS row passed through.  Bit-identical to the scalar
 * restatement.  New tensor; callers cache it per (gh, gw). */
int vk_pos_embed_bicubic_f32(vk_runtime* rt, const vk_tensor* pos_embed,
                             size_t grid, size_t embed, size_t gh, size_t gw,
                             float interp_offset, vk_tensor** out);

/* ------------------------------------------------------------------ */
/* image preprocessing                                                  */
/* ------------------------------------------------------------------ */

/* Resamplers of crates/da-engine/src/preprocess.rs on u8 HWC RGB images:
 * resize_bilinear_u8 (253-280), resize_cubic_u8 (Keys a = -0.75, 282-338)
 * and resize_area_u8 (box taps of area_table, 347-409; bilinear when no
 * axis shrinks).  Bit-identical to the scalar path (same f32/f64 operation
 * order, round half to even, saturate). */
typedef enum vk_resize_mode {
  VK_RESIZE_BILINEAR = 0,
  VK_RESIZE_CUBIC = 1,
  VK_RESIZE_AREA = 2
} vk_resize_mode;

/* Bytes of device workspace vk_resize_u8 needs (0: none). */
size_t vk_resize_workspace_bytes(size_t sh, size_t sw, size_t dh, size_t dw,
                                 int mode);
/* dst [dh, dw, 3] u8 from src [sh, sw, 3] u8.  workspace: any tensor of at
 * least vk_resize_workspace_bytes bytes (may be NULL when that is 0). */
int vk_resize_u8(vk_runtime* rt, const vk_tensor* src, size_t sh, size_t sw,
                 vk_tensor* dst, size_t dh, size_t dw, int mode,
                 vk_tensor* workspace);

/* The resize half of preprocess (preprocess.rs:432-469): the bound side
 * (the longer one when upper_bound != 0, else the shorter: "lower*" modes)
 * scaled to image_size with sizes rounded half to even, cubic when enlarging
 * and area otherwise, then both sides snapped to the nearest multiple of
 * patch (a second resize).  vk_preprocess_shape gives the output size (host
 * only); out is u8 [out_h, out_w, 3], the input of vk_patch_embed_u8. */
int vk_preprocess_shape(size_t h, size_t w, size_t image_size, size_t patch,
                        int upper_bound, size_t* out_h, size_t* out_w);
size_t vk_preprocess_workspace_bytes(size_t h, size_t w, size_t image_size,
                                     size_t patch, int upper_bound);
int vk_preprocess_resize_u8(vk_runtime* rt, const vk_tensor* src, size_t h,
                            size_t w, size_t image_size, size_t patch,
                            int upper_bound, vk_tensor* workspace,
                            vk_tensor* out);
/* The normalisation half (preprocess.rs:471-482): u8 HWC -> f32 NCHW,
 * (v/255 - mean[c]) / std[c] -- the input of vk_patchify_nchw_f32. */
int vk_normalize_u8_hwc_nchw_f32(vk_runtime* rt, const vk_tensor* src,
                                 size_t h, size_t w, const float mean[3],
                                 const float std_[3], vk_tensor* out);

/* The whole per-image token preparation in one kernel: u8 HWC image ->
 * ImageNet-style normalisation (preprocess.rs:484-500) -> 14x14 unfold ->
 * F32 MFMA projection with the OIHW filter held by `proj` (prepared with
 * vk_linear_prepare_oihw_f32) + bias -> + position table -> token assembly
 * [CLS+pos0, registers (no position), patches+pos] (pos_embed.rs:254-306).
 * registers may be NULL when n_register == 0.  out has
 * (1 + n_register + gh*gw) * embed elements. */
int vk_patch_embed_u8(vk_runtime* rt, const vk_tensor* img_hwc, size_t h,
                      size_t w, size_t patch, const float mean[3],
                      const float std_[3], const vk_linear* proj,
                      const vk_tensor* cls, const vk_tensor* registers,
                      size_t n_register, const vk_tensor* pos_table,
                      vk_tensor* out);

/* vk_patch_embed_u8 for every view of a multi-view batch in one launch:
 * the per-view preprocess + prepare_tokens loop of prepare_multi_view
 * (engine.rs:573-626), whose views share one processed shape
 * (engine.rs:594-605).  images: u8 [views, h, w, 3], every view 8-byte
 * aligned (h*w*3 % 8 == 0 when views > 1, else VK_ERR_UNSUPPORTED); out:
 * the view-major tokens [views * (1 + n_register + gh*gw), embed], each
 * view's rows the bits vk_patch_embed_u8 writes for that image. */
int vk_patch_embed_views_u8(vk_runtime* rt, const vk_tensor* images,
                            size_t views, size_t h, size_t w, size_t patch,
                            const float mean[3], const float std_[3],
                            const vk_linear* proj, const vk_tensor* cls,
                            const vk_tensor* registers, size_t n_register,
                            const vk_tensor* pos_table, vk_tensor* out);

/* ------------------------------------------------------------------ */
/* backbone capture and head hand-off                                   */
/* ------------------------------------------------------------------ */

/* Backbone::post_process_capture (backbone.rs:1139-1179) for view_count
 * view-major views of n = n_special + n_patch tokens, embed columns:
 *   cat_token != 0: feat [views, n_patch, 2*embed] with row t =
 *     [local_x row n_special+t | LN(x row n_special+t)], cam [views, 2*embed]
 *     = [local_x row 0 | x row 0];
 *   cat_token == 0: feat [views, n_patch, embed] = LN(x patch rows), cam
 *     [views, embed] = x row 0; local_x may be NULL.
 * LN is the final vit.norm (norm_gamma/beta f32 or f16, eps = cfg.ln_eps):
 * bit-identical to vk_layernorm_into_f32 on the same rows.  local_x is the
 * pre-alternation snapshot the reference keeps (backbone.rs:488, 635). */
int vk_capture_f32(vk_runtime* rt, const vk_tensor* local_x,
                   const vk_tensor* x, size_t n, size_t n_special,
                   size_t embed, size_t view_count,
                   const vk_tensor* norm_gamma, const vk_tensor* norm_beta,
                   float eps, int cat_token, vk_tensor* feat, vk_tensor* cam);

/* token_major_to_chw_with_optional_layernorm (dpt_head.rs:260-301): token
 * rows tok [n_tok, c] to channel-major out [c, n_tok] (out[ch*n_tok + t]),
 * each row LayerNorm'd first when gamma/beta are given (the head uses
 * HEAD_NORM_EPS = 1e-5, dpt_head.rs:101).  Bit-identical to
 * vk_layernorm_into_f32 followed by the transpose (the reference's
 * materialised path, dpt_head.rs:513-518).  gamma/beta both NULL: transpose
 * only.  out must not alias tok. */
int vk_token_to_chw_f32(vk_runtime* rt, const vk_tensor* tok, size_t n_tok,
                        size_t c, const vk_tensor* gamma,
                        const vk_tensor* beta, float eps, vk_tensor* out);

/* ------------------------------------------------------------------ */
/* one ViT block's fused-op sequence                                    */
/* ------------------------------------------------------------------ */

/* Model shape and options (the ModelConfig fields the path reads,
 * crates/da-engine/src/config.rs:145-185). */
typedef struct vk_vit_config {
  size_t embed_dim;     /* D: 768 ViT-B, 1024 ViT-L                 */
  size_t num_heads;     /* H                                        */
  size_t head_dim;      /* 64                                       */
  size_t mlp_hidden;    /* M: 3072 / 4096                           */
  size_t num_register;  /* n_special = 1 + num_register             */
  float ln_eps;         /* block LayerNorm eps (1e-6 for DA3)       */
  float qk_norm_eps;    /* QK_NORM_EPS = 1e-5                       */
  float rope_freq;      /* 100                                      */
  int rope_start;       /* first layer with RoPE, -1 never          */
  int qknorm_start;     /* first layer with Q/K-norm, -1 never      */
  int alt_start;        /* first local/global alternation layer     */
  unsigned rope_mode;   /* VK_ROPE_* convention, 0 = default        */
} vk_vit_config;

/* Per-layer parameters (the vit.blk.{i}.* tensors of vit_block.rs:30-50).
 * qnorm/knorm NULL: Q/K-norm skipped; ls1/ls2 NULL: unscaled residual. */
typedef struct vk_vit_layer {
  const vk_tensor* norm1_gamma;
  const vk_tensor* norm1_beta;
  const vk_tensor* qnorm_gamma;
  const vk_tensor* qnorm_beta;
  const vk_tensor* knorm_gamma;
  const vk_tensor* knorm_beta;
  const vk_tensor* ls1;
  const vk_tensor* norm2_gamma;
  const vk_tensor* norm2_beta;
  const vk_tensor* ls2;
} vk_vit_layer;

/* Device activations of one block.  The GEMM/attention products between the
 * fused operations (q, k, attn_proj, hidden, mlp_out) are produced by the
 * caller's projections; this sequence owns the per-token work around them. */
typedef struct vk_vit_activations {
  vk_tensor* tokens;          /* [rows, D] residual stream, in/out        */
  vk_tensor* ln1;             /* [rows, D] LN1 output                      */
  vk_tensor* q;               /* [H, rows, 64] or per-view blocks          */
  vk_tensor* k;
  const vk_tensor* attn_proj; /* [rows, D] attention output projection     */
  vk_tensor* ln2;             /* [rows, D] LN2 output                      */
  vk_tensor* hidden;          /* [rows, M] FC1 output, GELU in place       */
  const vk_tensor* mlp_out;   /* [rows, D] FC2 output                      */
} vk_vit_activations;

#define VK_BLOCK_FUSE_LS_LN 1u      /* fuse LS1+res with LN2              */
#define VK_BLOCK_SKIP_LN1 2u        /* LN1 already produced (by the previous
                                       block's fused LS2+res+LN1)          */
#define VK_BLOCK_FUSE_NEXT_LN1 4u   /* finish with LS2+res fused with the next
                                       block's LN1 (next_layer required);
                                       when the next block is alt_start and
                                       `camera` is given, the camera-slot
                                       overwrite is fused too              */
#define VK_BLOCK_CAMERA_WRITTEN 8u  /* at alt_start: the previous block's
                                       fused LS2+res+LN1 already wrote the
                                       camera slot (and LN1).  Valid only
                                       with VK_BLOCK_SKIP_LN1, only at layer
                                       alt_start, and only after a
                                       VK_BLOCK_FUSE_NEXT_LN1 call at
                                       alt_start-1 that was given the camera
                                       token; other uses: VK_ERR_INVALID   */

/* One DA3 ViT block's fused per-token operations, in the reference order of
 * run_tail_device (vit_block.rs:489-582) and vit_block_with_views
 * (vit_block.rs:1019-1139):
 *   [camera overwrite at alt_start] -> LN1 -> Q/K-norm + RoPE (gated by
 *   qknorm_start / rope_start; positions per view, global layers (1,1)) ->
 *   tokens += ls1 (.) attn_proj -> LN2 -> GELU(hidden) ->
 *   tokens += ls2 (.) mlp_out [-> camera overwrite -> next block's LN1].
 * Every view of a multi-view batch is processed in one launch per operation
 * (rows = view_count * tokens_per_view, view-major); q/k use
 * VK_QK_HEADS_OUTER for global layers and VK_QK_VIEWS_OUTER for local ones.
 * camera: [2*D] (reference view slot 0, source views slot 1,
 * backbone.rs:746-768) or NULL when alt_start < 0; also read by the block
 * before alt_start when it fuses the next LN1 (VK_BLOCK_FUSE_NEXT_LN1), so
 * that the block at alt_start can take VK_BLOCK_SKIP_LN1 |
 * VK_BLOCK_CAMERA_WRITTEN. */
int vk_vit_block_fused_ops(vk_runtime* rt, const vk_vit_config* cfg,
                           size_t layer_idx, const vk_vit_layer* layer,
                           const vk_vit_layer* next_layer,
                           const vk_vit_activations* act, size_t gh, size_t gw,
                           size_t view_count, const vk_tensor* camera,
                           unsigned flags);

/* Cached device parameters of one whole block (the CudaAttentionLayer and
 * CudaMlpLayer of vit_block.rs:161-184): the vk_vit_layer vectors plus the
 * four prepared projections.  qkv: D -> 3D with bias, no LayerScale; proj:
 * D -> D with bias and ls1 as its LayerScale (or none); fc1: D -> M with
 * bias; fc2: M -> D with bias and ls2 (or none).  qnorm/knorm NULL: no
 * Q/K-norm. */
typedef struct vk_vit_block_weights {
  const vk_tensor* norm1_gamma;
  const vk_tensor* norm1_beta;
  const vk_linear* qkv;
  const vk_tensor* qnorm_gamma;
  const vk_tensor* qnorm_beta;
  const vk_tensor* knorm_gamma;
  const vk_tensor* knorm_beta;
  const vk_linear* proj;
  const vk_tensor* norm2_gamma;
  const vk_tensor* norm2_beta;
  const vk_linear* fc1;
  const vk_linear* fc2;
} vk_vit_block_weights;

/* Device scratch of one block, all f32: ln [rows*D]; q, k, v, attn
 * [H, rows, 64] each; hidden [rows*M].  Reused by every block of a pass. */
typedef struct vk_vit_block_workspace {
  vk_tensor* ln;
  vk_tensor* q;
  vk_tensor* k;
  vk_tensor* v;
  vk_tensor* attn;
  vk_tensor* hidden;
} vk_vit_block_workspace;

/* One whole DA3 ViT block on the device, in place on `tokens`
 * [rows = view_count*(1+num_register+gh*gw), D]: the device-resident
 * transformer tail CudaTransformerTailExecutor::run_tail_device
 * (vit_block.rs:489-582) for all views of a batch at once.
 *   [camera overwrite at alt_start] -> LN1 -> QKV projection storing
 *   head-major Q, K, V -> Q/K-norm + 2D RoPE (gated as in
 *   vk_vit_block_fused_ops) -> attention (global layers: each head over all
 *   rows; local layers: each head of each view over its own tokens) ->
 *   output projection (+b, *ls1) read head-major, added to tokens -> LN2 ->
 *   FC1 (+b) + GELU -> FC2 (+b, *ls2) added to tokens.
 * Global layers follow backbone.rs:459-460 (alt_start >= 0, layer >=
 * alt_start, odd layer).  Results equal the unfused reference sequence
 * within the dot-product bounds of the projections and attention. */
int vk_vit_block_forward_f32(vk_runtime* rt, const vk_vit_config* cfg,
                             size_t layer_idx, const vk_vit_block_weights* w,
                             vk_tensor* tokens, size_t gh, size_t gw,
                             size_t view_count, const vk_tensor* camera,
                             const vk_vit_block_workspace* ws);

/* The backbone's block loop on the device: Backbone::forward /
 * forward_multi_view_ordered (backbone.rs:390-532, 688-877) over `depth`
 * blocks (blocks[layer], the bits of vk_vit_block_forward_f32 each; the
 * FC2 of every block but the last and the one before alt_start also writes
 * the next block's LN1, in its split-K sum pass when it has one) on the
 * view-major tokens [view_count * (1+num_register+gh*gw), D], in place.  At each
 * out_layers[i] (in the caller's order) the capture of vk_capture_f32 with
 * the final vit.norm (norm_gamma/beta, cfg->ln_eps) fills feats[i]
 * [views, gh*gw, W] and cams[i] [views, W] (W = 2D with cat_token, else D);
 * captures at global layers pair the stream with local_x, the snapshot of
 * the last local layer (backbone.rs:816-830, 832-834).  local_x [rows*D] is
 * needed only when cat_token and some out layer is global (else NULL). */
int vk_backbone_forward_f32(vk_runtime* rt, const vk_vit_config* cfg,
                            size_t depth, const vk_vit_block_weights* blocks,
                            vk_tensor* tokens, size_t gh, size_t gw,
                            size_t view_count, const vk_tensor* camera,
                            const vk_tensor* norm_gamma,
                            const vk_tensor* norm_beta, int cat_token,
                            const int* out_layers, size_t n_out,
                            vk_tensor* const* feats, vk_tensor* const* cams,
                            const vk_vit_block_workspace* ws,
                            vk_tensor* local_x);

/* ------------------------------------------------------------------ */
/* timing and graphs                                                    */
/* ------------------------------------------------------------------ */

int vk_event_create(vk_runtime* rt, vk_event** out);
int vk_event_destroy(vk_event* ev);
/* Records on the runtime's stream. */
int vk_event_record(vk_runtime* rt, vk_event* ev);
/* Blocks until `stop` completes; milliseconds between the two events. */
int vk_event_elapsed_ms(vk_event* start, vk_event* stop, float* ms);

/* Stream capture of everything the runtime enqueues between begin and end
 * into a HIP graph, replayed with vk_graph_launch.  Nothing is allocated
 * while the stream captures: the runtime's work buffer (split-K partial sums
 * of linears over few rows, the key-split partials of attention over few
 * or unevenly spread query tiles, the row statistics of
 * vk_token_to_chw_f32) and its RoPE
 * tables grow only outside capture, so a sequence is run once eagerly
 * before it is captured; a call that would grow them during capture fails
 * with an error and enqueues nothing.  Buffers they replace stay valid for
 * graphs captured earlier until the runtime is released.  Device copies
 * (segment copies, the camera-slot write) are kernels, so a captured
 * sequence holds kernel nodes only.
 * Lifetime: a graph keeps its runtime alive and launches only on the
 * runtime it was captured on (another runtime, or one already passed to
 * vk_runtime_destroy, gives VK_ERR_INVALID).  vk_graph_destroy waits for
 * the runtime's stream before releasing the graph.  The tensors and linears
 * that the captured calls named must outlive every launch of the graph. */
int vk_graph_begin_capture(vk_runtime* rt);
int vk_graph_end_capture(vk_runtime* rt, vk_graph** out);
int vk_graph_launch(vk_runtime* rt, vk_graph* g);
int vk_graph_destroy(vk_graph* g);

#ifdef __cplusplus
}
#endif
#endif /* VESTRA_HIP_H */
