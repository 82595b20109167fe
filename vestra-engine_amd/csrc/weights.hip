// Linear preparation for gfx950: the resident f32 weight layout of every
// projection, made from the reference's [in, out] f32 layout
// (prepare_linear_f32, vit_block.rs:214-222, 303-313), an OIHW filter
// (patch_embed.rs:176-181), or GGUF F16 / Q8_0 storage expanded on the
// device; and the flat F16 / Q8_0 conversions.
//
// Resident layout: [out, kp] rows, the input dimension contiguous and
// zero-padded to kp = in rounded up to 16, so 128-bit loads never straddle
// rows and a last partial 16-block multiplies zeros.  A 3x14x14 patch filter
// also gets the patch kernel's image-order copy (prepare_patch_filter).
#include <cstring>
#include <vector>

#include "common.h"
#include "mfma_f32.h"

namespace {

using vkm::kKAlign;

int alloc_copy(const float* host, size_t n, float** dev) {
  VK_HIP(hipMalloc(dev, n * sizeof(float)));
  hipError_t e = hipMemcpy(*dev, host, n * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(*dev);
    *dev = nullptr;
    return vk::hip_fail(e, "hipMemcpy(linear weights)");
  }
  return VK_OK;
}

// Weight rows [out][kp] with the input dimension contiguous and zero-padded
// to kp = in rounded up to a 16-block, so 128-bit loads never straddle rows
// and a last partial block multiplies zeros.
int make_linear(vk_runtime* rt, size_t in, size_t out, const std::vector<float>& wnk,
                const float* bias, const float* ls, vk_linear** res) {
  auto* lin = new vk_linear;
  lin->rt = rt;
  vk::retain(rt);
  lin->in_features = in;
  lin->out_features = out;
  lin->k_pitch = (in + kKAlign - 1) / kKAlign * kKAlign;
  int s = alloc_copy(wnk.data(), lin->k_pitch * out, &lin->weight_nk);
  if (s == VK_OK) s = vk::prepare_patch_filter(rt, lin);
  if (s == VK_OK) s = alloc_copy(bias, out, &lin->bias);
  if (s == VK_OK && ls) s = alloc_copy(ls, out, &lin->ls_gamma);
  if (s != VK_OK) {
    vk_linear_destroy(lin);
    return s;
  }
  *res = lin;
  return VK_OK;
}

// ---------------------------------------------------------------------------
// Weights in GGUF storage formats, expanded on the device.
//
// The reference widens F16 and dequantises Q8_0 tensors to f32 once, when
// it reads the model (Gguf::tensor_f32, crates/da-gguf/src/reader.rs:279-349;
// q8_0.rs:24-33), and its projections run on those f32 values.  Here the
// stored bytes are uploaded as they are (half or about a quarter of the f32
// bytes) and expanded by the kernels below straight into the linear's
// resident [out, kp] f32 layout.  Both conversions are exact (an f16 widens
// exactly; d*q of an f16 scale and an int8 needs at most 19 significant
// bits), so the projections give the bits of the f32 preparation of the
// same widened weights.  The matrix cores stay on the F32 path: keeping
// F16 / Q8_0 resident and widening inside the GEMM would add conversion
// work to every tile for no gain in time (the projections are MFMA-bound)
// nor in fit (288 GB of HBM).
// ---------------------------------------------------------------------------
enum WeightSrc { kSrcF16 = 0, kSrcQ8 = 1 };
constexpr int kQ8Block = 32;       // values per Q8_0 block (q8_0.rs:10)
constexpr int kQ8BlockBytes = 34;  // f16 scale + 32 int8

// Element f of a GGUF tensor in storage format SRC, as f32.
template <int SRC>
__device__ __forceinline__ float stored_value(const uint8_t* __restrict__ src, size_t f) {
  if (SRC == kSrcF16) return vkd::f16_to_f32(reinterpret_cast<const uint16_t*>(src)[f]);
  const uint8_t* b = src + (f / kQ8Block) * kQ8BlockBytes;
  const uint16_t d = static_cast<uint16_t>(b[0] | (b[1] << 8));
  const int8_t q = static_cast<int8_t>(b[2 + f % kQ8Block]);
  return vkd::f16_to_f32(d) * static_cast<float>(q);
}

// Flat tensor conversion: dst[f] = stored_value(src, f).
template <int SRC>
__global__ __launch_bounds__(256) void expand_flat_kernel(const uint8_t* __restrict__ src,
                                                          float* __restrict__ dst, long long n) {
  const long long f = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (f < n) dst[f] = stored_value<SRC>(src, static_cast<size_t>(f));
}

// Linear weight rows: wnk[o*kp + i] = W(i, o) for i < in, 0 for the padding;
// the stored tensor is [in, out] (IN_OUT, the projection layout of
// prepare_linear_f32) or [out, in] (an OIHW filter).
template <int SRC, bool IN_OUT>
__global__ __launch_bounds__(256) void expand_weight_kernel(const uint8_t* __restrict__ src,
                                                            float* __restrict__ wnk, int in,
                                                            int out, int kp) {
  const long long idx = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<long long>(out) * kp) return;
  const int o = static_cast<int>(idx / kp), i = static_cast<int>(idx % kp);
  float v = 0.0f;
  if (i < in)
    v = stored_value<SRC>(src, IN_OUT ? static_cast<size_t>(i) * out + o
                                      : static_cast<size_t>(o) * in + i);
  wnk[idx] = v;
}

unsigned grid_for(long long n) { return static_cast<unsigned>((n + 255) / 256); }

// Uploads `nbytes` of stored weights and expands them into a new linear.
int make_linear_stored(vk_runtime* rt, size_t in, size_t out, int src_kind, bool in_out,
                       const void* stored, size_t nbytes, const float* bias, const float* ls,
                       vk_linear** res) {
  auto* lin = new vk_linear;
  lin->rt = rt;
  vk::retain(rt);
  lin->in_features = in;
  lin->out_features = out;
  lin->k_pitch = (in + kKAlign - 1) / kKAlign * kKAlign;
  uint8_t* raw = nullptr;
  int s = VK_OK;
  const long long nw = static_cast<long long>(lin->k_pitch) * static_cast<long long>(out);
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&lin->weight_nk), nw * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&raw), nbytes);
  if (e == hipSuccess) e = hipMemcpy(raw, stored, nbytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) s = vk::hip_fail(e, "upload of stored linear weights");
  if (s == VK_OK) {
    const int ii = static_cast<int>(in), oo = static_cast<int>(out),
              kp = static_cast<int>(lin->k_pitch);
    if (src_kind == kSrcF16 && in_out)
      hipLaunchKernelGGL((expand_weight_kernel<kSrcF16, true>), grid_for(nw), 256, 0, rt->stream,
                         raw, lin->weight_nk, ii, oo, kp);
    else if (src_kind == kSrcF16)
      hipLaunchKernelGGL((expand_weight_kernel<kSrcF16, false>), grid_for(nw), 256, 0, rt->stream,
                         raw, lin->weight_nk, ii, oo, kp);
    else if (in_out)
      hipLaunchKernelGGL((expand_weight_kernel<kSrcQ8, true>), grid_for(nw), 256, 0, rt->stream,
                         raw, lin->weight_nk, ii, oo, kp);
    else
      hipLaunchKernelGGL((expand_weight_kernel<kSrcQ8, false>), grid_for(nw), 256, 0, rt->stream,
                         raw, lin->weight_nk, ii, oo, kp);
    s = vk::check_launch("expand_weight_kernel");
  }
  if (s == VK_OK) s = vk::prepare_patch_filter(rt, lin);
  if (raw) {
    // the expansion must finish before its source is released
    const hipError_t se = hipStreamSynchronize(rt->stream);
    if (s == VK_OK && se != hipSuccess) s = vk::hip_fail(se, "hipStreamSynchronize");
    (void)hipFree(raw);
  }
  if (s == VK_OK) s = alloc_copy(bias, out, &lin->bias);
  if (s == VK_OK && ls) s = alloc_copy(ls, out, &lin->ls_gamma);
  if (s != VK_OK) {
    vk_linear_destroy(lin);
    return s;
  }
  *res = lin;
  return VK_OK;
}

int check_prepare(size_t in_features, size_t out_features) {
  VK_REQUIRE(in_features > 0 && out_features > 0, "empty linear");
  VK_UNSUPPORTED_IF(out_features % 4 != 0, "linear: out_features=%zu must be a multiple of 4",
                    out_features);
  VK_UNSUPPORTED_IF(in_features > 0x7ffffff0 || out_features > 0x7fffffff ||
                        in_features * out_features > (1ULL << 36),
                    "linear too large");
  return VK_OK;
}

int expand_flat(vk_runtime* rt, int src_kind, const vk_tensor* src, size_t n, vk_tensor* dst) {
  if (n == 0) return VK_OK;
  const auto* s = static_cast<const uint8_t*>(src->ptr);
  auto* d = static_cast<float*>(dst->ptr);
  const long long nn = static_cast<long long>(n);
  if (src_kind == kSrcF16)
    hipLaunchKernelGGL((expand_flat_kernel<kSrcF16>), grid_for(nn), 256, 0, rt->stream, s, d, nn);
  else
    hipLaunchKernelGGL((expand_flat_kernel<kSrcQ8>), grid_for(nn), 256, 0, rt->stream, s, d, nn);
  return vk::check_launch("expand_flat_kernel");
}

}  // namespace

extern "C" {

int vk_linear_prepare_w16(vk_runtime* rt, size_t in_features, size_t out_features,
                          const uint16_t* weight_in_out, const float* bias, const float* ls_gamma,
                          vk_linear** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out && weight_in_out && bias, "null argument");
  VK_TRY(check_prepare(in_features, out_features));
  return make_linear_stored(rt, in_features, out_features, kSrcF16, true, weight_in_out,
                            in_features * out_features * 2, bias, ls_gamma, out);
}

int vk_linear_prepare_q8_0(vk_runtime* rt, size_t in_features, size_t out_features,
                           const uint8_t* blocks, size_t nbytes, const float* bias,
                           const float* ls_gamma, vk_linear** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out && blocks && bias, "null argument");
  VK_TRY(check_prepare(in_features, out_features));
  const size_t n = in_features * out_features;
  VK_REQUIRE(n % kQ8Block == 0, "q8_0: %zu elements, not a multiple of the block size %d", n,
             kQ8Block);
  VK_REQUIRE(nbytes == n / kQ8Block * kQ8BlockBytes, "q8_0: %zu bytes, expected %zu", nbytes,
             n / kQ8Block * kQ8BlockBytes);
  return make_linear_stored(rt, in_features, out_features, kSrcQ8, true, blocks, nbytes, bias,
                            ls_gamma, out);
}

int vk_linear_prepare_oihw_w16(vk_runtime* rt, size_t in_features, size_t out_features,
                               const uint16_t* weight_out_in, const float* bias, vk_linear** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out && weight_out_in && bias, "null argument");
  VK_TRY(check_prepare(in_features, out_features));
  return make_linear_stored(rt, in_features, out_features, kSrcF16, false, weight_out_in,
                            in_features * out_features * 2, bias, nullptr, out);
}

int vk_widen_f16_f32(vk_runtime* rt, const vk_tensor* src, vk_tensor* dst) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(src && dst, "null argument");
  VK_REQUIRE(src->dtype == VK_F16 && dst->dtype == VK_F32 && dst->len == src->len,
             "widen: src must be f16 and dst f32 of the same length");
  return expand_flat(rt, kSrcF16, src, src->len, dst);
}

int vk_dequantize_q8_0_f32(vk_runtime* rt, const vk_tensor* blocks, size_t n, vk_tensor* dst) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(blocks && dst, "null argument");
  VK_REQUIRE(n % kQ8Block == 0, "q8_0: %zu elements, not a multiple of the block size %d", n,
             kQ8Block);
  VK_REQUIRE(blocks->dtype == VK_U8 && blocks->len == n / kQ8Block * kQ8BlockBytes,
             "q8_0: blocks must be u8 [%zu]", n / kQ8Block * kQ8BlockBytes);
  VK_REQUIRE(dst->dtype == VK_F32 && dst->len == n, "q8_0: dst must be f32 [%zu]", n);
  return expand_flat(rt, kSrcQ8, blocks, n, dst);
}

int vk_linear_prepare_f32(vk_runtime* rt, size_t in_features, size_t out_features,
                          const float* weight_in_out, const float* bias, const float* ls_gamma,
                          vk_linear** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out && weight_in_out && bias, "null argument");
  VK_REQUIRE(in_features > 0 && out_features > 0, "empty linear");
  VK_UNSUPPORTED_IF(out_features % 4 != 0, "linear: out_features=%zu must be a multiple of 4",
                    out_features);
  VK_UNSUPPORTED_IF(in_features > 0x7ffffff0 || out_features > 0x7fffffff, "linear too large");
  const size_t kp = (in_features + kKAlign - 1) / kKAlign * kKAlign;
  std::vector<float> w(kp * out_features, 0.0f);
  for (size_t i = 0; i < in_features; ++i)
    for (size_t o = 0; o < out_features; ++o) w[o * kp + i] = weight_in_out[i * out_features + o];
  return make_linear(rt, in_features, out_features, w, bias, ls_gamma, out);
}

int vk_linear_prepare_oihw_f32(vk_runtime* rt, size_t in_features, size_t out_features,
                               const float* weight_out_in, const float* bias, vk_linear** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out && weight_out_in && bias, "null argument");
  VK_REQUIRE(in_features > 0 && out_features > 0, "empty linear");
  VK_UNSUPPORTED_IF(out_features % 4 != 0, "linear: out_features=%zu must be a multiple of 4",
                    out_features);
  VK_UNSUPPORTED_IF(in_features > 0x7ffffff0 || out_features > 0x7fffffff, "linear too large");
  const size_t kp = (in_features + kKAlign - 1) / kKAlign * kKAlign;
  std::vector<float> w(kp * out_features, 0.0f);
  for (size_t o = 0; o < out_features; ++o)
    std::memcpy(&w[o * kp], weight_out_in + o * in_features, in_features * sizeof(float));
  return make_linear(rt, in_features, out_features, w, bias, nullptr, out);
}

int vk_linear_destroy(vk_linear* lin) {
  if (!lin) return VK_OK;
  vk_runtime* rt = lin->rt;
  if (rt) (void)vk::bind_device(rt);
  if (rt) (void)hipStreamSynchronize(rt->stream);
  if (lin->weight_nk) (void)hipFree(lin->weight_nk);
  if (lin->weight_patch) (void)hipFree(lin->weight_patch);
  if (lin->bias) (void)hipFree(lin->bias);
  if (lin->ls_gamma) (void)hipFree(lin->ls_gamma);
  delete lin;
  vk::release(rt);
  return VK_OK;
}

size_t vk_linear_input_features(const vk_linear* lin) { return lin ? lin->in_features : 0; }

}  // extern "C"
