// Internal definitions shared by the runtime and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "vestra_hip.h"

// ---------------------------------------------------------------------------
// host-side objects behind the opaque handles
// ---------------------------------------------------------------------------

struct vk_runtime {
  // Handles that keep the runtime alive: the runtime handle itself plus
  // every tensor, linear and event created on it.  vk_runtime_destroy drops
  // the first; the stream and the runtime's buffers are released when the
  // last one goes, so objects destroyed after their runtime stay valid to
  // destroy.
  std::atomic<int> refs{1};
  // vk_runtime_destroy was called: the handle takes no new work.
  bool destroyed = false;
  int device = 0;
  hipStream_t stream = nullptr;
  int cu_count = 0;
  // cos/sin tables of the 2D rotary embedding, keyed by (frequency bits,
  // head_dim, exponent over the whole head): device pointer (owned by the
  // runtime) and the largest position the table covers.
  std::map<std::tuple<uint32_t, int, int>, std::pair<float*, int>> rope_tables;
  // Work buffer (f32) of launches that hand intermediate values from one
  // kernel to the next on the runtime's stream: split-K partial sums, the
  // row statistics of the token -> CHW hand-off.  Every user is ordered on
  // `stream`, so one buffer serves all of them.  Grown only outside stream
  // capture.
  float* work = nullptr;
  size_t work_len = 0;
  // Replaced device buffers (work buffers, smaller RoPE tables): graphs
  // captured earlier may still name them, so they live until the runtime
  // is destroyed.
  std::vector<void*> retired;
  // Summation order of every LayerNorm the runtime enqueues
  // (VK_LN_ORDER_TREE or VK_LN_ORDER_SEQUENTIAL), read at enqueue time.
  int ln_order = VK_LN_ORDER_TREE;
};

struct vk_tensor {
  vk_runtime* rt = nullptr;
  void* ptr = nullptr;
  size_t len = 0;
  vk_dtype dtype = VK_F32;
  bool owned = true;
};

struct vk_linear {
  vk_runtime* rt = nullptr;
  size_t in_features = 0;
  size_t out_features = 0;
  size_t k_pitch = 0;          // in_features rounded up to 16
  float* weight_nk = nullptr;  // [out, k_pitch], input dimension contiguous
  // For a 3x14x14 patch filter (in_features 588) only: the same rows with
  // the input dimension reordered (c, ky, kx) -> (ky, kx, c), the order in
  // which an HWC image holds a patch.
  float* weight_patch = nullptr;
  float* bias = nullptr;       // [out]
  float* ls_gamma = nullptr;   // [out] or null
};

struct vk_event {
  vk_runtime* rt = nullptr;
  hipEvent_t ev = nullptr;
};

struct vk_graph {
  // The runtime whose stream was captured: the graph keeps it alive (its
  // nodes name the runtime's work buffer and RoPE tables) and launches only
  // on its stream.
  vk_runtime* rt = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

// ---------------------------------------------------------------------------
// error plumbing
// ---------------------------------------------------------------------------

namespace vkd {

// Unsigned 32-bit division by a runtime-invariant divisor as a multiply-high
// and two shifts (Granlund & Montgomery, "Division by invariant integers
// using multiplication", PLDI 1994, fig. 4.1), exact for every n < 2^32.
// The divisor data is built on the host and passed to kernels by value.
struct FastDivU32 {
  uint32_t d;
  uint32_t m;
  uint32_t s1;
  uint32_t s2;
};

__host__ __device__ inline FastDivU32 make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;  // l = ceil(log2 d)
  const unsigned long long m =
      ((1ull << 32) * ((1ull << l) - d)) / d + 1;  // 2^l - d < 2^31: no overflow
  FastDivU32 f;
  f.d = d;
  f.m = static_cast<uint32_t>(m);
  f.s1 = l ? 1u : 0u;
  f.s2 = l ? l - 1 : 0u;
  return f;
}

}  // namespace vkd

namespace vk {

int set_error(int code, const char* fmt, ...);
void clear_error();
int hip_fail(hipError_t e, const char* what);
size_t dtype_size(vk_dtype d);
// Ensures the calling thread's current device is the runtime's device;
// fails for a destroyed runtime.
int bind(vk_runtime* rt);
// The same without the destroyed check: releasing objects of a destroyed
// runtime.
int bind_device(vk_runtime* rt);
// Reference counting of the runtime by the objects created on it.
void retain(vk_runtime* rt);
void release(vk_runtime* rt);
// Launch check: turns a failed launch into a status.
int check_launch(const char* what);
// Single-wave workgroups of a persistent stream over `units` equal units
// (rows, 3 KiB chunks): two units per wave when that puts every wave on the
// chip at once (cap < units <= 2 cap, cap = kStreamWavesPerCU waves per
// CU), so that a wave, which loads its next unit before it stores the
// current one, has issued all its reads before its first write; one unit
// per wave otherwise.  Measured for LayerNorm at 10,392 x 768 (256 CUs):
// two rows per wave 11.2 us, one 13.0, three 13.4; at 20,784 rows two rows
// per wave (10,392 waves) 23.9 us, four 24.6, one 23.4.  At least one wave.
constexpr int kStreamWavesPerCU = 24;
inline unsigned stream_waves(const vk_runtime* rt, long long units) {
  if (units <= 0) return 1;
  const long long cap =
      static_cast<long long>(rt->cu_count > 0 ? rt->cu_count : 256) * kStreamWavesPerCU;
  const long long per = units > cap && units <= 2 * cap ? 2 : 1;
  return static_cast<unsigned>((units + per - 1) / per);
}
// Device cos/sin table for the 2D RoPE (layout below) covering at least
// positions 0..max(min_max_pos, kRopeTableMax); *table_max receives the
// largest covered position.  Grows (re-allocates) when a larger grid needs
// it, so call it before any stream capture that uses the table.
int rope_table(vk_runtime* rt, float freq, int head_dim, unsigned rope_mode, int min_max_pos,
               const float** out, int* table_max);
// VK_ERR_INVALID for RoPE convention flags other than VK_ROPE_*.
int check_rope_mode(unsigned rope_mode);
// Looks up, once per device and with that device current, the device
// address of the allocation-free entry point's static scratch array.
void noalloc_setup(int device);
// For a linear of in_features 588 (a 3x14x14 patch filter): allocates and
// fills lin->weight_patch, the rows of lin->weight_nk with the input order
// (c, ky, kx) -> (ky, kx, c) of an HWC image's patch, zero-padded to 592, on
// the runtime's stream.  Any other linear: nothing.
int prepare_patch_filter(vk_runtime* rt, vk_linear* lin);
// Makes rt->work hold at least `floats` floats (at least 8 Mi once
// allocated, doubling on growth).  Growth is refused during stream capture:
// run the sequence once eagerly first.  The buffer it replaces is retired,
// not freed.
int ensure_work(vk_runtime* rt, size_t floats, const char* who);
// Stream-ordered device-to-device copy of `bytes` bytes as a kernel (a
// captured sequence then holds kernel nodes only).
int device_copy(vk_runtime* rt, void* dst, const void* src, size_t bytes);
// Camera-token slot write (backbone.rs:446-457, 746-768) as one launch:
// row v * tokens_per_view of the view-major `tokens` [views * tpv, D] takes
// camera slot 0 (v == 0, the reference view) or slot 1 (source views).
int write_camera_rows(vk_runtime* rt, float* tokens, const float* camera, size_t view_count,
                      size_t tokens_per_view, size_t D);
// tokens += ls (.) y, the camera-token slot (row 0 of each view of
// tokens_per_view rows) overwritten by `camera` when it is non-null, then
// ln_out = LN(tokens): the fused LayerScale+residual+LayerNorm with the
// overwrite that comes between them before block alt_start.
int ls_residual_layernorm_camera(vk_runtime* rt, vk_tensor* x, const vk_tensor* y,
                                 const vk_tensor* ls_gamma, const vk_tensor* ln_gamma,
                                 const vk_tensor* ln_beta, size_t rows, size_t cols, float eps,
                                 vk_tensor* ln_out, const vk_tensor* camera,
                                 size_t tokens_per_view);

// Q/K-norm + RoPE parameters of the QKV projection's fused epilogue: the
// row's token index m gives its position (rows are view-major tokens).
struct QkEpilogue {
  const void* qg;  // Q/K LayerNorm gamma / beta (f32 or f16), null for RoPE only
  const void* qb;
  const void* kg;
  const void* kb;
  const float* table;  // cos/sin table (layout below), covers every grid coordinate
  int table_max;
  uint32_t n_special;
  uint32_t global;
  vkd::FastDivU32 tpv;  // tokens per view
  vkd::FastDivU32 gw;   // patch grid width
  float eps;
  uint32_t interleaved;  // RoPE pairing: 0 (j, j+16), 1 (2i, 2i+1)
};

// F32 linear out[m, n] = epilogue(sum_k x[m, k] W[n, k] + b[n]).
struct LinearArgs {
  const float* x;     // [M, K]
  const float* wnk;   // [N, Kp], K contiguous, zero beyond K
  const float* bias;  // [N]
  const float* ls;    // [N] or null
  float* out;         // [M, N]
  int M, N, K, Kp;
  // head-major layouts of the attention block (head_dim 64), linear.hip only:
  float* q_out;  // non-null: out is split Q | K | V into q_out/k_out/v_out [N/192, M, 64]
  float* k_out;
  float* v_out;
  int a_hnd;     // 1: x is head-major [K/64, M, 64] (the attention output)
  // split-K (linear.hip only): `splits` workgroups share each output tile,
  // each over a contiguous run of 64-wide k chunks, writing raw sums to
  // partial [splits, M, N]; a second pass adds them in split order and
  // applies the epilogue.
  int splits;
  float* partial;
  // Q/K LayerNorm + 2D RoPE in the QKV epilogue (q_out set, qkn_mode != 0):
  // 1 LayerNorm with f32 parameters, 2 with f16 parameters, 3 RoPE only.
  int qkn_mode;
  QkEpilogue qkn;
  // LayerNorm of the finished rows after the residual epilogue (ln_out set):
  // ln_out = LN(out) with ln_gamma/ln_beta (f32, or f16 when ln_f16), the
  // bits of the separate LayerNorm.  With split-K and N of 768 or 1024 the
  // sum pass does it row by row; otherwise the LayerNorm kernel runs after.
  const void* ln_gamma;
  const void* ln_beta;
  int ln_f16;
  float ln_eps;
  float* ln_out;
};

// Epilogues of the linear: v = acc + b (then * ls when the linear has one),
// each rounding as in the unfused sequence, so a fused call gives the same
// bits as the linear followed by the separate stream kernel.
namespace linear_epilogue {
enum LinearEpilogue {
  kLinStore = 0,     // out = v
  kLinGelu = 1,      // out = GELU(v), A&S erf (the GELU stream's function)
  kLinGeluErf = 2,   // out = GELU(v), device erff
  kLinResidual = 3,  // out += v (out is the residual stream)
};
}  // namespace linear_epilogue

// The wide-tile linear (128 x 128, 64 x 128 or 64 x 64 tiles, split-K for
// few rows) for K % 4 == 0 and a 16-byte aligned x (linear.hip);
// the head-major layouts of LinearArgs need it.
// `partial` / `partial_floats`: the caller's buffer for split-K partial
// sums (nothing is allocated; a plan that needs more is refused); null: the
// runtime's work buffer, grown as needed.
int launch_linear_wide(vk_runtime* rt, const LinearArgs& g, int epi, float* partial = nullptr,
                       size_t partial_floats = 0);

// LayerNorm of `rows` x `cols` f32 rows on raw pointers, in the runtime's
// LayerNorm order; gamma/beta f16 when `f16`.
int layernorm_raw(vk_runtime* rt, const float* x, float* y, const void* gamma, const void* beta,
                  bool f16, int rows, int cols, float eps);
// The statistics of the sequential-order LayerNorm alone: stats[2r] = mean,
// stats[2r + 1] = 1/std of logical row r, read from stored row
// (r / np) * n + ns + r % np of x (np 0: row r); cols % 4 == 0, <= 8192.
int layernorm_stats_sequential(vk_runtime* rt, const float* x, float* stats, int rows, int cols,
                               float eps, int np, int n, int ns);

// Output projection of the head-major attention output with LayerScale +
// residual into `residual`, then ln_out = LayerNorm(residual): the calls
// vk_linear_run_hnd_residual_f32 + vk_layernorm_into_f32 with the same
// bits, one launch fewer when the projection runs split-K.
int linear_hnd_residual_layernorm(vk_runtime* rt, const vk_linear* lin, const vk_tensor* hnd,
                                  size_t rows, size_t heads, size_t head_dim,
                                  vk_tensor* residual, const vk_tensor* gamma,
                                  const vk_tensor* beta, float eps, vk_tensor* ln_out);

// The same for a token-major input: vk_linear_run_residual_f32 +
// vk_layernorm_into_f32 with the same bits (the block loop's FC2 followed by
// the next block's LN1).
int linear_residual_layernorm(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x,
                              size_t rows, vk_tensor* residual, const vk_tensor* gamma,
                              const vk_tensor* beta, float eps, vk_tensor* ln_out);

}  // namespace vk

#define VK_REQUIRE(cond, ...)                              \
  do {                                                     \
    if (!(cond)) return vk::set_error(VK_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define VK_UNSUPPORTED_IF(cond, ...)                       \
  do {                                                     \
    if (cond) return vk::set_error(VK_ERR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)

#define VK_HIP(call)                                       \
  do {                                                     \
    hipError_t e_ = (call);                                \
    if (e_ != hipSuccess) return vk::hip_fail(e_, #call);  \
  } while (0)

#define VK_TRY(call)                                       \
  do {                                                     \
    int s_ = (call);                                       \
    if (s_ != VK_OK) return s_;                            \
  } while (0)

// ---------------------------------------------------------------------------
// RoPE table layout (device, f32):
//   [0, table_max]              positions covered by the table
//                               (table_max >= kRopeTableMax)
//   entry p: 32 floats: cos(p*inv_freq_j) j<16, then sin(p*inv_freq_j) j<16
//   after the last entry: inv_freq_j, j<16 (for positions outside the table)
// ---------------------------------------------------------------------------
namespace vk {
constexpr int kRopeTableMax = 1023;
constexpr int kRopeQuarter = 16;  // head_dim 64: two halves of 32, 16 pairs each
}  // namespace vk

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

namespace vkd {

// Sum over the 16 lanes of a DPP row; every lane of the row receives the
// same (bitwise identical) value.
__device__ __forceinline__ float row16_sum(float v) {
  int iv;
  iv = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true);  // quad_perm 1,0,3,2
  v = v + __builtin_bit_cast(float, iv);
  iv = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true);  // quad_perm 2,3,0,1
  v = v + __builtin_bit_cast(float, iv);
  iv = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true); // row_half_mirror
  v = v + __builtin_bit_cast(float, iv);
  iv = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true); // row_mirror
  v = v + __builtin_bit_cast(float, iv);
  return v;
}

// Sum over a whole wave64; every lane receives the same value.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v = v + __shfl_xor(v, 16, 64);
  v = v + __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDivU32& f) {
  const uint32_t t = __umulhi(f.m, n);
  return (t + ((n - t) >> f.s1)) >> f.s2;
}

__device__ __forceinline__ uint32_t fmod_(uint32_t n, const FastDivU32& f) {
  return n - fdiv(n, f) * f.d;
}

// Mean and 1/sqrt(var + eps) of one row held by a wave as NV float4 per lane
// (lane l holds float4 l + 64 i of the row): sum in i order, wave tree,
// then the two-pass biased variance over the same registers.  Every
// LayerNorm of a full row (block LayerNorm, the fused LayerScale+residual
// form, the backbone's capture and the head's token->CHW hand-off) goes
// through here, so they all give the same bits for the same row.  !EXACT:
// float4 slots at or beyond cols/4 hold zeros and are left out.
template <int NV, bool EXACT>
__device__ __forceinline__ void row_mean_inv(const float4 (&v)[NV], int lane, int cols, float eps,
                                             float* mean_out, float* inv_out) {
  const int nvec = cols >> 2;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (EXACT || lane + i * 64 < nvec) {
      s += v[i].x;
      s += v[i].y;
      s += v[i].z;
      s += v[i].w;
    }
  }
  s = wave_sum(s);
  const float mean = s / static_cast<float>(cols);
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (EXACT || lane + i * 64 < nvec) {
      float d;
      d = v[i].x - mean; q += d * d;
      d = v[i].y - mean; q += d * d;
      d = v[i].z - mean; q += d * d;
      d = v[i].w - mean; q += d * d;
    }
  }
  q = wave_sum(q);
  const float var = q / static_cast<float>(cols);
  *mean_out = mean;
  *inv_out = 1.0f / sqrtf(var + eps);
}

// (v - mean) * inv * gamma + beta, each step rounded: the per-element
// LayerNorm output of the scalar reference order.
__device__ __forceinline__ float4 ln_apply4(float4 v, float mean, float inv, float4 g, float4 b) {
  float4 o;
  o.x = (v.x - mean) * inv * g.x + b.x;
  o.y = (v.y - mean) * inv * g.y + b.y;
  o.z = (v.z - mean) * inv * g.z + b.z;
  o.w = (v.w - mean) * inv * g.w + b.w;
  return o;
}

// Streaming (nontemporal) 128-bit loads and stores for activations that are
// touched once per kernel: they keep the stream from displacing reusable
// lines in L2 and the Infinity Cache.  Parameter vectors use ordinary loads.
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_stream(const float4* p) {
  const f32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
  return make_float4(t.x, t.y, t.z, t.w);
}

__device__ __forceinline__ void st_stream(float4* p, float4 v) {
  const f32x4_t t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<f32x4_t*>(p));
}

// Waits for every earlier vector memory operation of the wave, its
// previous stores included.  Issued before each store of a stream kernel it
// keeps one store of the wave in flight: out-of-place row streams and the
// LayerScale + residual stream measured faster so on MI355X (HBM reads are
// then not held up behind a backlog of the wave's writes).
__device__ __forceinline__ void wait_memory() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Raw buffer loads: a buffer resource (base address and byte size, held in
// scalar registers) plus a 32-bit per-lane byte offset and a uniform byte
// offset, with no 64-bit address arithmetic per load.  Reads at or past
// `bytes` return zeros.  Third descriptor word: the gfx9-family raw-buffer
// format (32-bit data, no swizzle).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ float4 buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t lane_off,
                                               uint32_t uniform_off) {
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
      r, static_cast<int>(lane_off), static_cast<int>(uniform_off), 0);
  return __builtin_bit_cast(float4, v);
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup i runs on
// XCD i % 8), and each XCD has its own L2.  Renumber so that an XCD's
// workgroups are consecutive tiles t of an N-major order (t -> m = t % gm,
// n = t / gm): they then share the same few weight columns in that L2.
// Bijective for any tile count n: XCD x holds n/8 tiles, one more if
// x < n % 8.
__device__ __forceinline__ int xcd_tile(int lin, int n) {
  const int q = n / 8, r = n % 8;
  const int xcd = lin % 8, slot = lin / 8;
  return slot + (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q);
}

// Abramowitz & Stegun 7.1.26 erf (|error| < 1.5e-7): the erf of the
// reference's scalar GELU (docs/plans/2026-07-18-rust-engine-v1.md:870-876),
// with the same evaluation order: t = 1/(1 + p*a);
// y = 1 - ((((a5*t + a4)*t + a3)*t + a2)*t + a1)*t * exp(-a*a); erf = sign*y.
// t takes the hardware reciprocal (v_rcp_f32, 1 ulp) and exp(-a*a) the
// hardware base-2 exponential of -a*a*log2(e) (v_exp_f32): a few ulp from
// the correctly rounded quotient and expf, for 2 instructions where those
// take about 23.  The Horner steps, 1 + p*a and 1 - (p*t)*e are single-
// rounding FMAs and the sign a copysign (a third fewer VALU instructions:
// the linear's GELU epilogue, which runs after its MFMAs with six waves per
// SIMD, measured 1-2.5% faster; max error against the exact GELU 3.7e-7).
// Shared by the GELU stream and the linear's GELU epilogue, so both give the
// same bits.
__device__ __forceinline__ float erf_as7126(float x) {
  const float a = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, a, 1.0f));
  float p = __builtin_fmaf(1.0614054f, t, -1.4531520f);
  p = __builtin_fmaf(p, t, 1.4214137f);
  p = __builtin_fmaf(p, t, -0.28449674f);
  p = __builtin_fmaf(p, t, 0.25482959f);
  const float e = __builtin_amdgcn_exp2f(-(a * a) * 1.44269504f);
  const float y = __builtin_fmaf(-(p * t), e, 1.0f);
  return __builtin_copysignf(y, x);
}

// GELU(v) = 0.5 v (1 + erf(v / sqrt 2)); MODE 0: A&S erf, 1: device erff.
template <int MODE>
__device__ __forceinline__ float gelu1(float v) {
  const float inv_sqrt2 = 0.70710678f;
  const float e = (MODE == 0) ? erf_as7126(v * inv_sqrt2) : erff(v * inv_sqrt2);
  const float h = 0.5f * v;
  return __builtin_fmaf(h, e, h);
}

// Parameter vector element loads (f32 or binary16 storage).
template <typename PT>
struct Param;

template <>
struct Param<float> {
  __device__ __forceinline__ static float4 load4(const float* p, size_t i4) {
    return reinterpret_cast<const float4*>(p)[i4];
  }
};

template <>
struct Param<uint16_t> {
  __device__ __forceinline__ static float4 load4(const uint16_t* p, size_t i4) {
    const ushort4 h = reinterpret_cast<const ushort4*>(p)[i4];
    return make_float4(f16_to_f32(h.x), f16_to_f32(h.y), f16_to_f32(h.z),
                       f16_to_f32(h.w));
  }
};

}  // namespace vkd
