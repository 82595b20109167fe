// Layout glue of the attention block for gfx950: the fused QKV projection's
// output split into head-major Q, K, V, and the attention output back to
// token-major rows.  Both are pure permutations streamed through HBM: one
// thread per float4, coalesced on the token-major side, 256-byte contiguous
// runs (one head row of 64 floats) on the head-major side.
#include "common.h"

namespace {

using vkd::FastDivU32;
using vkd::fdiv;

// qkv [rows, 3*heads*hd] (Q | K | V, each [heads, hd]) -> q, k, v [heads, rows, hd].
// Thread f: row = f / (3*heads*hd4), which = rem / (heads*hd4), h, d4.
__global__ __launch_bounds__(256) void split_qkv_hnd_kernel(const float4* __restrict__ qkv,
                                                            float4* __restrict__ q,
                                                            float4* __restrict__ k,
                                                            float4* __restrict__ v,
                                                            uint32_t rows, uint32_t total,
                                                            FastDivU32 per_row,
                                                            FastDivU32 per_block,
                                                            FastDivU32 hd4) {
  const uint32_t f = blockIdx.x * 256u + threadIdx.x;
  if (f >= total) return;
  const uint32_t row = fdiv(f, per_row);
  const uint32_t rem = f - row * per_row.d;
  const uint32_t which = fdiv(rem, per_block);
  const uint32_t in_block = rem - which * per_block.d;
  const uint32_t h = fdiv(in_block, hd4);
  const uint32_t d4 = in_block - h * hd4.d;
  float4* dst = which == 0 ? q : (which == 1 ? k : v);
  dst[(static_cast<size_t>(h) * rows + row) * hd4.d + d4] = vkd::ld_stream(qkv + f);
}

// hnd [heads, rows, hd] -> out [rows, heads*hd].  Thread f indexes out.
__global__ __launch_bounds__(256) void hnd_to_token_kernel(const float4* __restrict__ hnd,
                                                           float4* __restrict__ out,
                                                           uint32_t rows, uint32_t total,
                                                           FastDivU32 per_row, FastDivU32 hd4) {
  const uint32_t f = blockIdx.x * 256u + threadIdx.x;
  if (f >= total) return;
  const uint32_t row = fdiv(f, per_row);
  const uint32_t rem = f - row * per_row.d;
  const uint32_t h = fdiv(rem, hd4);
  const uint32_t d4 = rem - h * hd4.d;
  vkd::st_stream(out + f, hnd[(static_cast<size_t>(h) * rows + row) * hd4.d + d4]);
}

int check_glue(size_t rows, size_t heads, size_t head_dim, size_t blocks) {
  VK_REQUIRE(heads > 0 && head_dim > 0, "heads=%zu, head_dim=%zu must be positive", heads,
             head_dim);
  VK_UNSUPPORTED_IF(head_dim % 4 != 0, "head_dim=%zu must be a multiple of 4", head_dim);
  VK_UNSUPPORTED_IF(rows * blocks * heads * head_dim / 4 >= 0x80000000ULL,
                    "layout: %zu rows too many", rows);
  return VK_OK;
}

int check_f32(const vk_tensor* t, size_t len, const char* what) {
  VK_REQUIRE(t && t->dtype == VK_F32 && t->len == len, "%s must be f32 [%zu] (holds %zu)", what,
             len, t ? t->len : 0);
  return VK_OK;
}

bool disjoint(const vk_tensor* a, const vk_tensor* b) {
  const char* pa = static_cast<const char*>(a->ptr);
  const char* pb = static_cast<const char*>(b->ptr);
  return a->len == 0 || b->len == 0 || pa + a->len * 4 <= pb || pb + b->len * 4 <= pa;
}

}  // namespace

extern "C" {

int vk_split_qkv_hnd_into_f32(vk_runtime* rt, const vk_tensor* qkv, size_t rows, size_t heads,
                              size_t head_dim, vk_tensor* q, vk_tensor* k, vk_tensor* v) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(qkv && q && k && v, "null argument");
  VK_TRY(check_glue(rows, heads, head_dim, 3));
  const size_t part = rows * heads * head_dim;
  VK_TRY(check_f32(qkv, 3 * part, "qkv"));
  VK_TRY(check_f32(q, part, "q"));
  VK_TRY(check_f32(k, part, "k"));
  VK_TRY(check_f32(v, part, "v"));
  VK_REQUIRE(disjoint(qkv, q) && disjoint(qkv, k) && disjoint(qkv, v) && disjoint(q, k) &&
                 disjoint(q, v) && disjoint(k, v),
             "split_qkv_hnd: tensors overlap");
  if (rows == 0) return VK_OK;
  const uint32_t hd4 = static_cast<uint32_t>(head_dim / 4);
  const uint32_t per_block = static_cast<uint32_t>(heads) * hd4;
  const uint32_t total = static_cast<uint32_t>(3 * part / 4);
  hipLaunchKernelGGL(split_qkv_hnd_kernel, dim3((total + 255) / 256), dim3(256), 0, rt->stream,
                     static_cast<const float4*>(qkv->ptr), static_cast<float4*>(q->ptr),
                     static_cast<float4*>(k->ptr), static_cast<float4*>(v->ptr),
                     static_cast<uint32_t>(rows), total, vkd::make_fastdiv(3 * per_block),
                     vkd::make_fastdiv(per_block), vkd::make_fastdiv(hd4));
  return vk::check_launch("split_qkv_hnd_kernel");
}

int vk_split_qkv_hnd_f32(vk_runtime* rt, const vk_tensor* qkv, size_t rows, size_t heads,
                         size_t head_dim, vk_tensor** q, vk_tensor** k, vk_tensor** v) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(qkv && q && k && v, "null argument");
  VK_TRY(check_glue(rows, heads, head_dim, 3));
  const size_t part = rows * heads * head_dim;
  VK_TRY(check_f32(qkv, 3 * part, "qkv"));
  vk_tensor *tq = nullptr, *tk = nullptr, *tv = nullptr;
  int s = vk_tensor_alloc(rt, VK_F32, part, &tq);
  if (s == VK_OK) s = vk_tensor_alloc(rt, VK_F32, part, &tk);
  if (s == VK_OK) s = vk_tensor_alloc(rt, VK_F32, part, &tv);
  if (s == VK_OK) s = vk_split_qkv_hnd_into_f32(rt, qkv, rows, heads, head_dim, tq, tk, tv);
  if (s != VK_OK) {
    vk_tensor_destroy(tq);
    vk_tensor_destroy(tk);
    vk_tensor_destroy(tv);
    return s;
  }
  *q = tq;
  *k = tk;
  *v = tv;
  return VK_OK;
}

int vk_hnd_to_token_into_f32(vk_runtime* rt, const vk_tensor* hnd, size_t rows, size_t heads,
                             size_t head_dim, vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(hnd && out, "null argument");
  VK_TRY(check_glue(rows, heads, head_dim, 1));
  const size_t len = rows * heads * head_dim;
  VK_TRY(check_f32(hnd, len, "hnd"));
  VK_TRY(check_f32(out, len, "out"));
  VK_REQUIRE(disjoint(hnd, out), "hnd_to_token: tensors overlap");
  if (rows == 0) return VK_OK;
  const uint32_t hd4 = static_cast<uint32_t>(head_dim / 4);
  const uint32_t total = static_cast<uint32_t>(len / 4);
  hipLaunchKernelGGL(hnd_to_token_kernel, dim3((total + 255) / 256), dim3(256), 0, rt->stream,
                     static_cast<const float4*>(hnd->ptr), static_cast<float4*>(out->ptr),
                     static_cast<uint32_t>(rows), total,
                     vkd::make_fastdiv(static_cast<uint32_t>(heads) * hd4),
                     vkd::make_fastdiv(hd4));
  return vk::check_launch("hnd_to_token_kernel");
}

int vk_hnd_to_token_f32(vk_runtime* rt, const vk_tensor* hnd, size_t rows, size_t heads,
                        size_t head_dim, vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(hnd && out, "null argument");
  VK_TRY(check_glue(rows, heads, head_dim, 1));
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, rows * heads * head_dim, &t));
  const int s = vk_hnd_to_token_into_f32(rt, hnd, rows, heads, head_dim, t);
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

}  // extern "C"
