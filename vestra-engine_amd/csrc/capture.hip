// The backbone's output capture and the DPT head's token -> CHW hand-off,
// both LayerNorm-then-relayout passes over token rows:
//
//  * capture_rows: Backbone::post_process_capture (backbone.rs:1139-1179).
//    For every view of a view-major batch, each patch row x[n_special + t]
//    is LayerNorm'd with vit.norm and written next to the same row of the
//    pre-alternation snapshot local_x: feat[t] = [local_x | LN(x)] (cat_token)
//    or LN(x); the camera/CLS row 0 goes to cam.  One wave per patch row
//    (plus one per view for the camera row), the row held in registers as
//    in the block LayerNorm; one launch covers all views.
//  * chw_row_stats + chw_tiles: token_major_to_chw_with_optional_layernorm
//    (dpt_head.rs:260-301).  One image's hand-off is a few hundred tokens,
//    too few rows to fill the chip if a workgroup owned whole rows, so the
//    LayerNorm statistics come first (one wave per row, mean and 1/std into
//    the runtime's work buffer) and the transpose is then tiled over
//    (64 tokens x 64 channels): each tile is read as 64 contiguous 256-byte
//    row pieces, normalised, turned through a [64][65] LDS tile and written
//    as 64 contiguous 256-byte channel pieces.  A 864-token, 1536-channel
//    hand-off is 14 x 24 = 336 workgroups.
//
// Row statistics and the per-element formula are vkd::row_mean_inv and
// vkd::ln_apply4, shared with the block LayerNorm: a captured or handed-off
// row has the bits vk_layernorm_into_f32 gives the same row.  In the
// runtime's sequential LayerNorm order the statistics come from the
// sequential-order kernel of the block LayerNorm instead (into the work
// buffer, then read by the same passes), with the same consequence.
#include "common.h"

namespace {

using vkd::Param;

// STATS: the row's mean and 1/std come from stats[r] (the sequential-order
// statistics of patch row r), not from the wave's own reduction.
template <int NV, typename PT, bool EXACT, bool CAT, bool STATS>
__global__ __launch_bounds__(64) void capture_rows(const float* __restrict__ local_x,
                                                   const float* __restrict__ x,
                                                   const PT* __restrict__ gamma,
                                                   const PT* __restrict__ beta,
                                                   float* __restrict__ feat,
                                                   float* __restrict__ cam, int n_patch, int n,
                                                   int n_special, int views, int D, float eps,
                                                   const float2* __restrict__ stats) {
  const int lane = threadIdx.x;
  const int r = blockIdx.x;
  const int nvec = D >> 2;
  const int feat_rows = views * n_patch;
  if (r >= feat_rows) {
    // camera/CLS row 0 of view v: [local_x row | x row] or x row
    const int v = r - feat_rows;
    const size_t src = static_cast<size_t>(v) * n * D;
    float* dst = cam + static_cast<size_t>(v) * (CAT ? 2 : 1) * D;
    for (int c = lane; c < nvec; c += 64) {
      if (CAT) {
        reinterpret_cast<float4*>(dst)[c] = reinterpret_cast<const float4*>(local_x + src)[c];
        reinterpret_cast<float4*>(dst + D)[c] = reinterpret_cast<const float4*>(x + src)[c];
      } else {
        reinterpret_cast<float4*>(dst)[c] = reinterpret_cast<const float4*>(x + src)[c];
      }
    }
    return;
  }
  const int v = r / n_patch;
  const int t = r - v * n_patch;
  const size_t src = (static_cast<size_t>(v) * n + n_special + t) * D;
  float* dst = feat + static_cast<size_t>(r) * (CAT ? 2 : 1) * D;
  const float4* xr = reinterpret_cast<const float4*>(x + src);
  float4 vv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * 64;
    vv[i] = (EXACT || c < nvec) ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float mean, inv;
  if (STATS) {
    const float2 ms = stats[r];
    mean = ms.x;
    inv = ms.y;
  } else {
    vkd::row_mean_inv<NV, EXACT>(vv, lane, D, eps, &mean, &inv);
  }
  float4* ln_dst = reinterpret_cast<float4*>(dst + (CAT ? D : 0));
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * 64;
    if (EXACT || c < nvec)
      ln_dst[c] = vkd::ln_apply4(vv[i], mean, inv, Param<PT>::load4(gamma, c),
                                 Param<PT>::load4(beta, c));
  }
  if (CAT) {
    const float4* lr = reinterpret_cast<const float4*>(local_x + src);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + i * 64;
      if (EXACT || c < nvec) reinterpret_cast<float4*>(dst)[c] = lr[c];
    }
  }
}

constexpr int kChwTok = 64;  // tokens per tile
constexpr int kChwCh = 64;   // channels per tile

// stats[2 t] = mean, stats[2 t + 1] = 1/std of token row t; wave per row.
template <int NV, bool EXACT>
__global__ __launch_bounds__(256) void chw_row_stats(const float* __restrict__ tok,
                                                     float* __restrict__ stats, int n_tok, int C,
                                                     float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tok) return;
  const int nvec = C >> 2;
  const float4* xr = reinterpret_cast<const float4*>(tok + static_cast<size_t>(t) * C);
  float4 vv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * 64;
    vv[i] = (EXACT || c < nvec) ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float mean, inv;
  vkd::row_mean_inv<NV, EXACT>(vv, lane, C, eps, &mean, &inv);
  if (lane == 0) *reinterpret_cast<float2*>(stats + 2 * static_cast<size_t>(t)) =
      make_float2(mean, inv);
}

// One (64-token x 64-channel) tile per workgroup; blockIdx.x = token tile,
// blockIdx.y = channel tile.
template <typename PT, bool NORM>
__global__ __launch_bounds__(256) void chw_tiles(const float* __restrict__ tok,
                                                 const float* __restrict__ stats,
                                                 const PT* __restrict__ gamma,
                                                 const PT* __restrict__ beta,
                                                 float* __restrict__ out, int n_tok, int C) {
  __shared__ float tile[kChwCh][kChwTok + 1];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int t0 = blockIdx.x * kChwTok;
  const int c0 = blockIdx.y * kChwCh;
  // 64 tokens x 16 float4: slot s = tid + 256 j -> token s/16, float4 s%16.
  // LDS bank of tile[4 c4 + k][rr] is (4 c4 + rr) mod 64: one wave's 64
  // lanes (16 c4 x 4 rr) hit 64 distinct banks.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int s = tid + 256 * j;
    const int rr = s >> 4, c4 = s & 15;
    const int t = t0 + rr, c = c0 + 4 * c4;
    if (t < n_tok && c < C) {
      float4 xv = *reinterpret_cast<const float4*>(tok + static_cast<size_t>(t) * C + c);
      if (NORM) {
        const float2 st = *reinterpret_cast<const float2*>(stats + 2 * static_cast<size_t>(t));
        xv = vkd::ln_apply4(xv, st.x, st.y, Param<PT>::load4(gamma, c >> 2),
                            Param<PT>::load4(beta, c >> 2));
      }
      tile[4 * c4 + 0][rr] = xv.x;
      tile[4 * c4 + 1][rr] = xv.y;
      tile[4 * c4 + 2][rr] = xv.z;
      tile[4 * c4 + 3][rr] = xv.w;
    }
  }
  __syncthreads();
  // wave w writes channel rows 16w..16w+15 of the tile, 64 tokens each
#pragma unroll 4
  for (int j = 0; j < 16; ++j) {
    const int cc = wave * 16 + j;
    const int c = c0 + cc, t = t0 + lane;
    if (c < C && t < n_tok) out[static_cast<size_t>(c) * n_tok + t] = tile[cc][lane];
  }
}

int nv_for(size_t cols) {
  const size_t nv = (cols + 255) / 256;
  if (nv <= 4) return static_cast<int>(nv);
  if (nv <= 6) return 6;
  if (nv <= 8) return 8;
  if (nv <= 12) return 12;
  return -1;
}

bool aligned16(const vk_tensor* t) {
  return t == nullptr || reinterpret_cast<uintptr_t>(t->ptr) % 16 == 0;
}

int check_norm_params(const vk_tensor* g, const vk_tensor* b, size_t cols, const char* who) {
  VK_REQUIRE(g && b, "%s: gamma and beta must both be given", who);
  VK_REQUIRE((g->dtype == VK_F32 || g->dtype == VK_F16) && g->dtype == b->dtype,
             "%s: gamma/beta must share dtype f32 or f16", who);
  VK_REQUIRE(g->len == cols && b->len == cols, "%s: gamma/beta must hold %zu values", who, cols);
  VK_REQUIRE(aligned16(g) && aligned16(b), "%s: gamma/beta must be 16-byte aligned", who);
  return VK_OK;
}

template <typename PT, bool CAT>
int launch_capture(vk_runtime* rt, int nv, bool exact, const float* lx, const float* x,
                   const void* g, const void* b, float* feat, float* cam, int n_patch, int n,
                   int ns, int views, int D, float eps) {
  const dim3 grid(static_cast<unsigned>(views * n_patch + views)), block(64);
  auto G = static_cast<const PT*>(g);
  auto B = static_cast<const PT*>(b);
  if (rt->ln_order == VK_LN_ORDER_SEQUENTIAL) {
    // the patch rows' statistics in the CPU's order first, into the work buffer
    VK_TRY(vk::ensure_work(rt, 2 * static_cast<size_t>(views) * n_patch, "capture"));
    VK_TRY(vk::layernorm_stats_sequential(rt, x, rt->work, views * n_patch, D, eps, n_patch, n,
                                          ns));
    const float2* st = reinterpret_cast<const float2*>(rt->work);
    hipLaunchKernelGGL((capture_rows<12, PT, false, CAT, true>), grid, block, 0, rt->stream, lx,
                       x, G, B, feat, cam, n_patch, n, ns, views, D, eps, st);
    return vk::check_launch("capture_rows");
  }
#define VK_CAP_CASE(N)                                                                         \
  case N:                                                                                      \
    if (exact)                                                                                 \
      hipLaunchKernelGGL((capture_rows<N, PT, true, CAT, false>), grid, block, 0, rt->stream, lx, x, G, B, feat, cam, n_patch, n, ns, views, D, eps, nullptr); \
    else                                                                                       \
      hipLaunchKernelGGL((capture_rows<N, PT, false, CAT, false>), grid, block, 0, rt->stream, lx, x, G, B, feat, cam, n_patch, n, ns, views, D, eps, nullptr); \
    break;
  switch (nv) {
    VK_CAP_CASE(1) VK_CAP_CASE(2) VK_CAP_CASE(3) VK_CAP_CASE(4) VK_CAP_CASE(6) VK_CAP_CASE(8)
    VK_CAP_CASE(12)
    default:
      return vk::set_error(VK_ERR_UNSUPPORTED, "capture: no instance for embed=%d", D);
  }
#undef VK_CAP_CASE
  return vk::check_launch("capture_rows");
}

template <typename PT, bool NORM>
int launch_chw(vk_runtime* rt, int nv, bool exact, const float* tok, const void* g,
               const void* b, float* out, int n_tok, int C, float eps) {
  const float* stats = nullptr;
  if (NORM) {
    VK_TRY(vk::ensure_work(rt, 2 * static_cast<size_t>(n_tok), "token_to_chw"));
    float* st = rt->work;
    if (rt->ln_order == VK_LN_ORDER_SEQUENTIAL) {
      VK_TRY(vk::layernorm_stats_sequential(rt, tok, st, n_tok, C, eps, 0, 0, 0));
      stats = st;
    }
    const dim3 sgrid(static_cast<unsigned>((n_tok + 3) / 4)), sblock(256);
#define VK_STAT_CASE(N)                                                                        \
  case N:                                                                                      \
    if (exact)                                                                                 \
      hipLaunchKernelGGL((chw_row_stats<N, true>), sgrid, sblock, 0, rt->stream, tok, st, n_tok, C, eps); \
    else                                                                                       \
      hipLaunchKernelGGL((chw_row_stats<N, false>), sgrid, sblock, 0, rt->stream, tok, st, n_tok, C, eps); \
    break;
    if (!stats) {
      switch (nv) {
        VK_STAT_CASE(1) VK_STAT_CASE(2) VK_STAT_CASE(3) VK_STAT_CASE(4) VK_STAT_CASE(6)
        VK_STAT_CASE(8) VK_STAT_CASE(12)
        default:
          return vk::set_error(VK_ERR_UNSUPPORTED, "token_to_chw: no instance for c=%d", C);
      }
      VK_TRY(vk::check_launch("chw_row_stats"));
      stats = st;
    }
  }
  const dim3 grid(static_cast<unsigned>((n_tok + kChwTok - 1) / kChwTok),
                  static_cast<unsigned>((C + kChwCh - 1) / kChwCh));
  hipLaunchKernelGGL((chw_tiles<PT, NORM>), grid, dim3(256), 0, rt->stream, tok, stats,
                     static_cast<const PT*>(g), static_cast<const PT*>(b), out, n_tok, C);
  return vk::check_launch("chw_tiles");
}

}  // namespace

extern "C" {

int vk_capture_f32(vk_runtime* rt, const vk_tensor* local_x, const vk_tensor* x, size_t n,
                   size_t n_special, size_t embed, size_t view_count,
                   const vk_tensor* norm_gamma, const vk_tensor* norm_beta, float eps,
                   int cat_token, vk_tensor* feat, vk_tensor* cam) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(x && feat && cam, "null argument");
  VK_REQUIRE(!cat_token || local_x, "capture: cat_token needs local_x");
  VK_REQUIRE(n_special <= n, "capture: n_special=%zu exceeds n=%zu", n_special, n);
  VK_UNSUPPORTED_IF(embed == 0 || embed % 4 != 0 || nv_for(embed) < 0,
                    "capture: embed=%zu (need a multiple of 4 up to 3072)", embed);
  VK_UNSUPPORTED_IF(view_count * n > 0x7fffffffULL, "capture: too many rows");
  const size_t n_patch = n - n_special;
  const size_t width = cat_token ? 2 * embed : embed;
  const size_t rows = view_count * n;
  VK_REQUIRE(x->dtype == VK_F32 && x->len == rows * embed, "capture: x must be f32 [%zu]",
             rows * embed);
  VK_REQUIRE(!cat_token || (local_x->dtype == VK_F32 && local_x->len == rows * embed),
             "capture: local_x must be f32 [%zu]", rows * embed);
  VK_REQUIRE(feat->dtype == VK_F32 && feat->len == view_count * n_patch * width,
             "capture: feat must be f32 [%zu]", view_count * n_patch * width);
  VK_REQUIRE(cam->dtype == VK_F32 && cam->len == view_count * width,
             "capture: cam must be f32 [%zu]", view_count * width);
  VK_TRY(check_norm_params(norm_gamma, norm_beta, embed, "capture"));
  VK_REQUIRE(aligned16(x) && aligned16(feat) && aligned16(cam) &&
                 (!cat_token || aligned16(local_x)),
             "capture: tensors must be 16-byte aligned");
  if (view_count == 0 || n == 0) return VK_OK;
  VK_REQUIRE(n_special >= 1, "capture: the camera/CLS row needs n_special >= 1");
  const int nv = nv_for(embed);
  const bool exact = embed == static_cast<size_t>(nv) * 256;
  const float* lx = cat_token ? static_cast<const float*>(local_x->ptr) : nullptr;
  const float* X = static_cast<const float*>(x->ptr);
  float* F = static_cast<float*>(feat->ptr);
  float* Cm = static_cast<float*>(cam->ptr);
  const int np = static_cast<int>(n_patch), nn = static_cast<int>(n),
            ns = static_cast<int>(n_special), vc = static_cast<int>(view_count),
            D = static_cast<int>(embed);
  const bool f16 = norm_gamma->dtype == VK_F16;
  if (cat_token)
    return f16 ? launch_capture<uint16_t, true>(rt, nv, exact, lx, X, norm_gamma->ptr,
                                                norm_beta->ptr, F, Cm, np, nn, ns, vc, D, eps)
               : launch_capture<float, true>(rt, nv, exact, lx, X, norm_gamma->ptr,
                                             norm_beta->ptr, F, Cm, np, nn, ns, vc, D, eps);
  return f16 ? launch_capture<uint16_t, false>(rt, nv, exact, lx, X, norm_gamma->ptr,
                                               norm_beta->ptr, F, Cm, np, nn, ns, vc, D, eps)
             : launch_capture<float, false>(rt, nv, exact, lx, X, norm_gamma->ptr,
                                            norm_beta->ptr, F, Cm, np, nn, ns, vc, D, eps);
}

int vk_token_to_chw_f32(vk_runtime* rt, const vk_tensor* tok, size_t n_tok, size_t c,
                        const vk_tensor* gamma, const vk_tensor* beta, float eps,
                        vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(tok && out, "null argument");
  VK_UNSUPPORTED_IF(c == 0 || c % 4 != 0 || nv_for(c) < 0,
                    "token_to_chw: c=%zu (need a multiple of 4 up to 3072)", c);
  VK_UNSUPPORTED_IF(n_tok > 0x7fffffffULL || n_tok * c > (1ULL << 40), "token_to_chw: too large");
  VK_REQUIRE(tok->dtype == VK_F32 && tok->len == n_tok * c, "token_to_chw: tok must be f32 [%zu]",
             n_tok * c);
  VK_REQUIRE(out->dtype == VK_F32 && out->len == n_tok * c, "token_to_chw: out must be f32 [%zu]",
             n_tok * c);
  {
    const char* a = static_cast<const char*>(tok->ptr);
    const char* o = static_cast<const char*>(out->ptr);
    const size_t bytes = n_tok * c * sizeof(float);
    VK_REQUIRE(bytes == 0 || a + bytes <= o || o + bytes <= a,
               "token_to_chw: out must not overlap tok");
  }
  VK_REQUIRE(aligned16(tok), "token_to_chw: tok must be 16-byte aligned");
  const bool norm = gamma || beta;
  if (norm) VK_TRY(check_norm_params(gamma, beta, c, "token_to_chw"));
  if (n_tok == 0) return VK_OK;
  const int nv = nv_for(c);
  const bool exact = c == static_cast<size_t>(nv) * 256;
  const float* T = static_cast<const float*>(tok->ptr);
  float* O = static_cast<float*>(out->ptr);
  const int nt = static_cast<int>(n_tok), C = static_cast<int>(c);
  if (!norm) return launch_chw<float, false>(rt, nv, exact, T, nullptr, nullptr, O, nt, C, eps);
  if (gamma->dtype == VK_F16)
    return launch_chw<uint16_t, true>(rt, nv, exact, T, gamma->ptr, beta->ptr, O, nt, C, eps);
  return launch_chw<float, true>(rt, nv, exact, T, gamma->ptr, beta->ptr, O, nt, C, eps);
}

}  // extern "C"
