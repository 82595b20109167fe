// Image preprocessing on the device (crates/da-engine/src/preprocess.rs:236-482):
// the aspect-preserving resize of a u8 HWC RGB frame to the model's patch
// grid, and the ImageNet normalisation to NCHW f32.
//
// The three resamplers are separable and bit-exact with the scalar path:
//  * bilinear: one thread per output pixel, f32 half-pixel coordinates;
//  * cubic (Keys a = -0.75) and area (OpenCV INTER_AREA-style box taps):
//    a horizontal pass over every source row into an f32 row buffer, then a
//    vertical pass that rounds half to even and saturates to u8.  Each thread
//    owns one output pixel (3 channels) and generates its taps on the fly in
//    the reference's order: coordinates in f64 where the reference uses f64,
//    weights and sums in f32, every operation rounded (no contraction), each
//    sum started from 0 and accumulated tap by tap.
// Scale factors are computed once on the host with the reference's
// expressions and passed by value.  Frames are small (a 640x427 frame is
// 0.8 MB), so the passes are launch-bound; they exist so that a frame goes
// to the device once, as bytes, and everything after stays resident.
#include <cmath>

#include "common.h"

namespace {

__device__ __forceinline__ uint8_t sat_round_u8(float v) {
  float r = rintf(v);  // ties to even
  r = fminf(fmaxf(r, 0.0f), 255.0f);
  return static_cast<uint8_t>(r);
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// cubic_weight (preprocess.rs:240-251), f32, the reference's operation order
__device__ __forceinline__ float cubic_w(float x) {
  const float A = -0.75f;
  x = fabsf(x);
  if (x < 1.0f) return ((A + 2.0f) * x - (A + 3.0f)) * x * x + 1.0f;
  if (x < 2.0f) return (((x - 5.0f) * x + 8.0f) * x - 4.0f) * A;
  return 0.0f;
}

__global__ __launch_bounds__(256) void resize_bilinear_kernel(const uint8_t* __restrict__ src,
                                                              int sw, int sh,
                                                              uint8_t* __restrict__ dst, int dw,
                                                              int dh, float sx, float sy) {
  const long long p = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= static_cast<long long>(dw) * dh) return;
  const int y = static_cast<int>(p / dw), x = static_cast<int>(p % dw);
  const float fy = (static_cast<float>(y) + 0.5f) * sy - 0.5f;
  const int y0 = static_cast<int>(floorf(fy));
  const float wy = fy - static_cast<float>(y0);
  const int y0c = clampi(y0, 0, sh - 1), y1c = clampi(y0 + 1, 0, sh - 1);
  const float fx = (static_cast<float>(x) + 0.5f) * sx - 0.5f;
  const int x0 = static_cast<int>(floorf(fx));
  const float wx = fx - static_cast<float>(x0);
  const int x0c = clampi(x0, 0, sw - 1), x1c = clampi(x0 + 1, 0, sw - 1);
  const uint8_t* r0 = src + static_cast<size_t>(y0c) * sw * 3;
  const uint8_t* r1 = src + static_cast<size_t>(y1c) * sw * 3;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float top = static_cast<float>(r0[x0c * 3 + c]) * (1.0f - wx) +
                      static_cast<float>(r0[x1c * 3 + c]) * wx;
    const float bottom = static_cast<float>(r1[x0c * 3 + c]) * (1.0f - wx) +
                         static_cast<float>(r1[x1c * 3 + c]) * wx;
    dst[static_cast<size_t>(p) * 3 + c] = sat_round_u8(top * (1.0f - wy) + bottom * wy);
  }
}

// The four cubic taps of output coordinate d (preprocess.rs:286-300).
__device__ __forceinline__ void cubic_taps(int d, double s, int n_src, int idx[4], float w[4]) {
  const double f = (static_cast<double>(d) + 0.5) * s - 0.5;
  const double fl = floor(f);
  const int i = static_cast<int>(fl);
  const float t = static_cast<float>(f - fl);
  w[0] = cubic_w(t + 1.0f);
  w[1] = cubic_w(t);
  w[2] = cubic_w(t - 1.0f);
  w[3] = cubic_w(t - 2.0f);
#pragma unroll
  for (int k = 0; k < 4; ++k) idx[k] = clampi(i - 1 + k, 0, n_src - 1);
}

// Area taps of destination d (area_table, preprocess.rs:347-382), visited in
// the reference's order: the partial left cell, the whole cells, the partial
// right cell.  fn(source, weight) is called once per tap.
template <typename F>
__device__ __forceinline__ void area_taps(int d, double scale, int n_src, F fn) {
  const double start_f = static_cast<double>(d) * scale;
  const double end_f = start_f + scale;
  const double cell = fmin(scale, static_cast<double>(n_src) - start_f);
  long long start = static_cast<long long>(ceil(start_f));
  long long end = static_cast<long long>(floor(end_f));
  if (end > n_src - 1) end = n_src - 1;
  if (start > end) start = end;
  if (static_cast<double>(start) - start_f > 1e-3)
    fn(static_cast<int>(start - 1), static_cast<float>((static_cast<double>(start) - start_f) / cell));
  const float whole = static_cast<float>(1.0 / cell);
  for (long long s = start; s < end; ++s) fn(static_cast<int>(s), whole);
  if (end_f - static_cast<double>(end) > 1e-3)
    fn(static_cast<int>(end),
       static_cast<float>(fmin(fmin(end_f - static_cast<double>(end), 1.0), cell) / cell));
}

enum { kCubic = 0, kArea = 1 };

// Horizontal pass: tmp[y][x][c] for every source row y, output column x.
template <int MODE>
__global__ __launch_bounds__(256) void resize_h_kernel(const uint8_t* __restrict__ src, int sw,
                                                       int sh, float* __restrict__ tmp, int dw,
                                                       double s) {
  const long long p = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= static_cast<long long>(dw) * sh) return;
  const int y = static_cast<int>(p / dw), x = static_cast<int>(p % dw);
  const uint8_t* row = src + static_cast<size_t>(y) * sw * 3;
  float acc[3] = {0.0f, 0.0f, 0.0f};
  if (MODE == kCubic) {
    int idx[4];
    float w[4];
    cubic_taps(x, s, sw, idx, w);
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int c = 0; c < 3; ++c) acc[c] += w[k] * static_cast<float>(row[idx[k] * 3 + c]);
  } else {
    area_taps(x, s, sw, [&](int i, float w) {
#pragma unroll
      for (int c = 0; c < 3; ++c) acc[c] += w * static_cast<float>(row[i * 3 + c]);
    });
  }
  float* o = tmp + static_cast<size_t>(p) * 3;
  o[0] = acc[0];
  o[1] = acc[1];
  o[2] = acc[2];
}

// Vertical pass: dst[y][x][c] from the f32 rows, rounded and saturated.
template <int MODE>
__global__ __launch_bounds__(256) void resize_v_kernel(const float* __restrict__ tmp, int sh,
                                                       int dw, uint8_t* __restrict__ dst, int dh,
                                                       double s) {
  const long long p = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= static_cast<long long>(dw) * dh) return;
  const int y = static_cast<int>(p / dw), x = static_cast<int>(p % dw);
  float acc[3] = {0.0f, 0.0f, 0.0f};
  if (MODE == kCubic) {
    int idx[4];
    float w[4];
    cubic_taps(y, s, sh, idx, w);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float* t = tmp + (static_cast<size_t>(idx[k]) * dw + x) * 3;
#pragma unroll
      for (int c = 0; c < 3; ++c) acc[c] += w[k] * t[c];
    }
  } else {
    area_taps(y, s, sh, [&](int i, float w) {
      const float* t = tmp + (static_cast<size_t>(i) * dw + x) * 3;
#pragma unroll
      for (int c = 0; c < 3; ++c) acc[c] += w * t[c];
    });
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) dst[static_cast<size_t>(p) * 3 + c] = sat_round_u8(acc[c]);
}

// u8 HWC -> f32 NCHW, (v/255 - mean[c]) / std[c] (preprocess.rs:471-482):
// one thread per pixel, three planes.
struct Norm3 {
  float mean[3];
  float sd[3];
};

__global__ __launch_bounds__(256) void normalize_nchw_kernel(const uint8_t* __restrict__ src,
                                                             float* __restrict__ dst,
                                                             long long plane, Norm3 nm) {
  const long long p = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= plane) return;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float v = static_cast<float>(src[p * 3 + c]) / 255.0f;
    dst[c * plane + p] = (v - nm.mean[c]) / nm.sd[c];
  }
}

unsigned blocks_for(long long n) { return static_cast<unsigned>((n + 255) / 256); }

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

size_t tmp_bytes(size_t sh, size_t sw, size_t dh, size_t dw, int mode) {
  if (mode == VK_RESIZE_BILINEAR) return 0;
  if (mode == VK_RESIZE_AREA && dw >= sw && dh >= sh) return 0;  // bilinear
  return align256(sh * dw * 3 * sizeof(float));
}

// Enqueues one resize; `tmp` holds at least tmp_bytes(...) bytes.
int enqueue_resize(vk_runtime* rt, const uint8_t* src, size_t sh, size_t sw, uint8_t* dst,
                   size_t dh, size_t dw, int mode, float* tmp) {
  if (mode == VK_RESIZE_AREA && dw >= sw && dh >= sh) mode = VK_RESIZE_BILINEAR;
  const int isw = static_cast<int>(sw), ish = static_cast<int>(sh), idw = static_cast<int>(dw),
            idh = static_cast<int>(dh);
  const long long out_px = static_cast<long long>(dw) * static_cast<long long>(dh);
  const long long mid_px = static_cast<long long>(dw) * static_cast<long long>(sh);
  if (mode == VK_RESIZE_BILINEAR) {
    const float sx = static_cast<float>(sw) / static_cast<float>(dw);
    const float sy = static_cast<float>(sh) / static_cast<float>(dh);
    hipLaunchKernelGGL(resize_bilinear_kernel, blocks_for(out_px), 256, 0, rt->stream, src, isw,
                       ish, dst, idw, idh, sx, sy);
    return vk::check_launch("resize_bilinear_kernel");
  }
  const double sx = static_cast<double>(sw) / static_cast<double>(dw);
  const double sy = static_cast<double>(sh) / static_cast<double>(dh);
  if (mode == VK_RESIZE_CUBIC) {
    hipLaunchKernelGGL(resize_h_kernel<kCubic>, blocks_for(mid_px), 256, 0, rt->stream, src, isw,
                       ish, tmp, idw, sx);
    hipLaunchKernelGGL(resize_v_kernel<kCubic>, blocks_for(out_px), 256, 0, rt->stream, tmp, ish,
                       idw, dst, idh, sy);
  } else {
    hipLaunchKernelGGL(resize_h_kernel<kArea>, blocks_for(mid_px), 256, 0, rt->stream, src, isw,
                       ish, tmp, idw, sx);
    hipLaunchKernelGGL(resize_v_kernel<kArea>, blocks_for(out_px), 256, 0, rt->stream, tmp, ish,
                       idw, dst, idh, sy);
  }
  return vk::check_launch("resize_h/v_kernel");
}

size_t nearest_multiple(size_t v, size_t m) {
  const size_t down = v / m * m, up = down + m;
  return (up - v) <= (v - down) ? up : down;
}

// preprocess's size policy (preprocess.rs:432-469)
struct PrepShape {
  size_t bh, bw, oh, ow;
  bool scaled;   // scale != 1
  bool enlarge;  // scale > 1
};

PrepShape prep_shape(size_t h, size_t w, size_t image_size, size_t patch, int upper_bound) {
  const size_t target = image_size ? image_size : 1, p = patch ? patch : 1;
  const size_t bound = upper_bound ? (w > h ? w : h) : (w < h ? w : h);
  const double scale = static_cast<double>(target) / static_cast<double>(bound);
  PrepShape s;
  s.bw = static_cast<size_t>(std::nearbyint(static_cast<double>(w) * scale));
  s.bh = static_cast<size_t>(std::nearbyint(static_cast<double>(h) * scale));
  if (s.bw < 1) s.bw = 1;
  if (s.bh < 1) s.bh = 1;
  s.ow = nearest_multiple(s.bw, p);
  s.oh = nearest_multiple(s.bh, p);
  if (s.ow < 1) s.ow = 1;
  if (s.oh < 1) s.oh = 1;
  s.scaled = std::fabs(scale - 1.0) >= 2.220446049250313e-16;
  s.enlarge = scale > 1.0;
  return s;
}

// Workspace of the preprocess resize: [first-pass rows][boundary image]
// [second-pass rows].
struct PrepLayout {
  size_t tmp1, mid, tmp2, total;
  int mode1, mode2;  // -1: no resize
};

PrepLayout prep_layout(size_t h, size_t w, const PrepShape& s) {
  PrepLayout l;
  l.mode1 = !s.scaled ? -1 : (s.enlarge ? VK_RESIZE_CUBIC : VK_RESIZE_AREA);
  const bool second = s.ow != s.bw || s.oh != s.bh;
  l.mode2 = !second ? -1 : ((s.ow > s.bw || s.oh > s.bh) ? VK_RESIZE_CUBIC : VK_RESIZE_AREA);
  l.tmp1 = l.mode1 < 0 ? 0 : tmp_bytes(h, w, s.bh, s.bw, l.mode1);
  l.mid = second ? align256(s.bh * s.bw * 3) : 0;
  l.tmp2 = l.mode2 < 0 ? 0 : tmp_bytes(s.bh, s.bw, s.oh, s.ow, l.mode2);
  l.total = l.tmp1 + l.mid + l.tmp2;
  return l;
}

bool dims_ok(size_t h, size_t w) {
  return h > 0 && w > 0 && h < (1u << 20) && w < (1u << 20) && h * w < (1ull << 31) / 3;
}

int check_u8(const vk_tensor* t, size_t len, const char* what) {
  VK_REQUIRE(t && t->dtype == VK_U8 && t->len == len, "resize: %s must be u8 [%zu]", what, len);
  return VK_OK;
}

}  // namespace

extern "C" {

size_t vk_resize_workspace_bytes(size_t sh, size_t sw, size_t dh, size_t dw, int mode) {
  return tmp_bytes(sh, sw, dh, dw, mode);
}

int vk_resize_u8(vk_runtime* rt, const vk_tensor* src, size_t sh, size_t sw, vk_tensor* dst,
                 size_t dh, size_t dw, int mode, vk_tensor* workspace) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(mode == VK_RESIZE_BILINEAR || mode == VK_RESIZE_CUBIC || mode == VK_RESIZE_AREA,
             "resize: unknown mode %d", mode);
  VK_UNSUPPORTED_IF(!dims_ok(sh, sw) || !dims_ok(dh, dw), "resize: %zux%zu -> %zux%zu", sh, sw,
                    dh, dw);
  VK_TRY(check_u8(src, sh * sw * 3, "src"));
  VK_TRY(check_u8(dst, dh * dw * 3, "dst"));
  const size_t need = tmp_bytes(sh, sw, dh, dw, mode);
  VK_REQUIRE(need == 0 || (workspace && workspace->len * vk::dtype_size(workspace->dtype) >= need),
             "resize: workspace of %zu bytes required", need);
  return enqueue_resize(rt, static_cast<const uint8_t*>(src->ptr), sh, sw,
                        static_cast<uint8_t*>(dst->ptr), dh, dw, mode,
                        need ? static_cast<float*>(workspace->ptr) : nullptr);
}

int vk_preprocess_shape(size_t h, size_t w, size_t image_size, size_t patch, int upper_bound,
                        size_t* out_h, size_t* out_w) {
  VK_REQUIRE(out_h && out_w, "null argument");
  VK_UNSUPPORTED_IF(!dims_ok(h, w), "preprocess: %zux%zu", h, w);
  const PrepShape s = prep_shape(h, w, image_size, patch, upper_bound);
  *out_h = s.oh;
  *out_w = s.ow;
  return VK_OK;
}

size_t vk_preprocess_workspace_bytes(size_t h, size_t w, size_t image_size, size_t patch,
                                     int upper_bound) {
  if (!dims_ok(h, w)) return 0;
  return prep_layout(h, w, prep_shape(h, w, image_size, patch, upper_bound)).total;
}

int vk_preprocess_resize_u8(vk_runtime* rt, const vk_tensor* src, size_t h, size_t w,
                            size_t image_size, size_t patch, int upper_bound,
                            vk_tensor* workspace, vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_UNSUPPORTED_IF(!dims_ok(h, w), "preprocess: %zux%zu", h, w);
  const PrepShape s = prep_shape(h, w, image_size, patch, upper_bound);
  VK_UNSUPPORTED_IF(!dims_ok(s.oh, s.ow) || !dims_ok(s.bh, s.bw), "preprocess: output too large");
  const PrepLayout l = prep_layout(h, w, s);
  VK_TRY(check_u8(src, h * w * 3, "src"));
  VK_TRY(check_u8(out, s.oh * s.ow * 3, "out"));
  VK_REQUIRE(l.total == 0 ||
                 (workspace && workspace->len * vk::dtype_size(workspace->dtype) >= l.total),
             "preprocess: workspace of %zu bytes required", l.total);
  VK_REQUIRE(reinterpret_cast<uintptr_t>(src->ptr) != reinterpret_cast<uintptr_t>(out->ptr),
             "preprocess: out must not be src");
  char* ws = workspace ? static_cast<char*>(workspace->ptr) : nullptr;
  float* tmp1 = l.tmp1 ? reinterpret_cast<float*>(ws) : nullptr;
  uint8_t* mid = l.mid ? reinterpret_cast<uint8_t*>(ws + l.tmp1) : nullptr;
  float* tmp2 = l.tmp2 ? reinterpret_cast<float*>(ws + l.tmp1 + l.mid) : nullptr;
  const auto* in = static_cast<const uint8_t*>(src->ptr);
  auto* dst = static_cast<uint8_t*>(out->ptr);
  // first resize (or copy) into the boundary image: straight into `out`
  // when no snap follows
  uint8_t* first = l.mode2 < 0 ? dst : mid;
  if (l.mode1 < 0) {
    VK_TRY(vk::device_copy(rt, first, in, h * w * 3));
  } else {
    VK_TRY(enqueue_resize(rt, in, h, w, first, s.bh, s.bw, l.mode1, tmp1));
  }
  if (l.mode2 >= 0) VK_TRY(enqueue_resize(rt, mid, s.bh, s.bw, dst, s.oh, s.ow, l.mode2, tmp2));
  return VK_OK;
}

int vk_normalize_u8_hwc_nchw_f32(vk_runtime* rt, const vk_tensor* src, size_t h, size_t w,
                                 const float mean[3], const float std_[3], vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(mean && std_, "null argument");
  VK_TRY(check_u8(src, h * w * 3, "src"));
  VK_REQUIRE(out && out->dtype == VK_F32 && out->len == h * w * 3,
             "normalize: out must be f32 [%zu]", h * w * 3);
  if (h * w == 0) return VK_OK;
  Norm3 nm;
  for (int c = 0; c < 3; ++c) {
    nm.mean[c] = mean[c];
    nm.sd[c] = std_[c];
  }
  const long long plane = static_cast<long long>(h * w);
  hipLaunchKernelGGL(normalize_nchw_kernel, blocks_for(plane), 256, 0, rt->stream,
                     static_cast<const uint8_t*>(src->ptr), static_cast<float*>(out->ptr), plane,
                     nm);
  return vk::check_launch("normalize_nchw_kernel");
}

}  // extern "C"
