// The F32 linear's C ABI for gfx950: the run entry points and their
// dispatch, the residual projection + LayerNorm plumbing of the block loop,
// and the allocation-free entry point.
//
// Every projection runs on the wide-tile kernel of linear.hip when its input
// rows can be read as float4 (K % 4 == 0 and a 16-byte aligned x); the
// narrow 48 x 64 kernel below (scalar loads of x, the tile of mfma_f32.h)
// takes any other K.  Both give out[m, n] = epilogue(sum_k x[m, k] W[n, k]
// + b[n]) with the epilogue's roundings in the order of the unfused
// sequence (bias, LayerScale, then GELU or the residual add).
#include "common.h"
#include "mfma_f32.h"

namespace {

using vk::LinearArgs;
using vkd::xcd_tile;
using namespace vk::linear_epilogue;
using namespace vkm;

// ---------------------------------------------------------------------------
// F32 linear: out[m, n] = (sum_k x[m, k] W[n, k] + b[n]) (* ls[n])
// K is staged through LDS in chunks of 192 (12 blocks); waves 0-3 take blocks
// 0-5 of a chunk, waves 4-7 blocks 6-11.  While the MFMAs consume one chunk,
// the next chunk's global loads are in flight into registers.
// ---------------------------------------------------------------------------
constexpr int KC = 192;
constexpr int kLinPitch = 196;  // 4 x 49
constexpr int kLinBlocks = KC / 16 / 2;  // per half
constexpr int kA_PER_THREAD = (KC * BM + kThreads - 1) / kThreads;        // 18
constexpr int kB_VEC_PER_THREAD = (KC * BN / 4 + kThreads - 1) / kThreads;  // 6
static_assert(kLinPitch % 4 == 0 && (kLinPitch / 4) % 2 == 1, "pitch must be 4 x odd");
static_assert(KC * BM % kThreads == 0 && KC * BN / 4 % kThreads == 0, "slots divide evenly");

// The loaders never branch around a global load: a load inside a guard
// makes the compiler wait for it before the next one, serialising the memory
// latency.  Slots outside the matrix read a clamped (valid) address and are
// zeroed when stored to LDS.  A slot e = tid + 512 i covers (m, kk) =
// (e / KC, e % KC): k fastest, so a wave's loads walk along matrix rows and
// its LDS stores hit consecutive banks.
struct LinearStage {
  float a[kA_PER_THREAD];
  float4 b[kB_VEC_PER_THREAD];
  uint32_t live_a, live_b;

  __device__ __forceinline__ void fetch(const LinearArgs& g, int m0, int n0, int k0, int tid) {
    live_a = 0;
#pragma unroll
    for (int i = 0; i < kA_PER_THREAD; ++i) {
      const int e = tid + kThreads * i;
      const int m = e / KC, kk = e % KC;
      const int gm = m0 + m, gk = k0 + kk;
      live_a |= static_cast<uint32_t>(gm < g.M && gk < g.K) << i;
      const int cm = gm < g.M ? gm : g.M - 1;
      const int ck = gk < g.K ? gk : g.K - 1;
      a[i] = g.x[static_cast<size_t>(cm) * g.K + ck];
    }
    live_b = 0;
#pragma unroll
    for (int i = 0; i < kB_VEC_PER_THREAD; ++i) {
      const int f = tid + kThreads * i;
      const int n = f / (KC / 4), j = f % (KC / 4);
      const int gn = n0 + n, gk = k0 + 4 * j;
      // Kp % 4 == 0 and gk % 4 == 0: a vector never straddles the row end
      live_b |= static_cast<uint32_t>(gn < g.N && gk < g.Kp) << i;
      const int cn = gn < g.N ? gn : g.N - 1;
      const int ck = gk < g.Kp ? gk : g.Kp - 4;
      b[i] = *reinterpret_cast<const float4*>(g.wnk + static_cast<size_t>(cn) * g.Kp + ck);
    }
  }
  __device__ __forceinline__ void store(float* As, float* Bs, int tid) const {
#pragma unroll
    for (int i = 0; i < kA_PER_THREAD; ++i) {
      const int e = tid + kThreads * i;
      As[(e / KC) * kLinPitch + e % KC] = ((live_a >> i) & 1) ? a[i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kB_VEC_PER_THREAD; ++i) {
      const int f = tid + kThreads * i;
      const bool on = (live_b >> i) & 1;
      const float4 v = make_float4(on ? b[i].x : 0.f, on ? b[i].y : 0.f, on ? b[i].z : 0.f,
                                   on ? b[i].w : 0.f);
      *reinterpret_cast<float4*>(Bs + (f / (KC / 4)) * kLinPitch + 4 * (f % (KC / 4))) = v;
    }
  }
};

template <int EPI>
__global__ __launch_bounds__(kThreads) void linear_kernel(LinearArgs g) {
  __shared__ __align__(16) float As[BM * kLinPitch];
  __shared__ __align__(16) float Bs[BN * kLinPitch];
  __shared__ float red[4 * 12 * 64];

  const int tid = threadIdx.x;
  __builtin_assume(tid < kThreads);
  const int wave = tid >> 6, lane = tid & 63;
  const int strip = wave & 3, half = wave >> 2;
  const int gm = (g.M + BM - 1) / BM;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int m0 = (tile % gm) * BM, n0 = (tile / gm) * BN;

  LinearStage st;
  st.fetch(g, m0, n0, 0, tid);

  f32x4 acc[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int kofs = 4 * (lane >> 4) + 16 * kLinBlocks * half;
  const float* arow = As + (lane & 15) * kLinPitch + kofs;
  const float* brow = Bs + (strip * 16 + (lane & 15)) * kLinPitch + kofs;

  for (int k0 = 0; k0 < g.K; k0 += KC) {
    st.store(As, Bs, tid);
    __syncthreads();
    if (k0 + KC < g.K) st.fetch(g, m0, n0, k0 + KC, tid);
#pragma unroll
    for (int j = 0; j < kLinBlocks; ++j) {
      const f32x4 b = *reinterpret_cast<const f32x4*>(brow + 16 * j);
      mfma_block(arow + 16 * j, 16 * kLinPitch, b, acc);
    }
    __syncthreads();
  }
  if (!reduce_halves(red, strip, half, lane, acc)) return;

  // epilogue: lane holds D[4*(lane/16) + r][lane%16] of each 16x16 tile
  const int col = n0 + strip * 16 + (lane & 15);
  if (col >= g.N) return;
  const float bias = g.bias[col];
  const float ls = g.ls ? g.ls[col] : 1.0f;
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + t * 16 + 4 * (lane >> 4) + r;
      if (row < g.M) {
        float v = acc[t][r] + bias;
        if (g.ls) v = v * ls;
        float* o = g.out + static_cast<size_t>(row) * g.N + col;
        if (EPI == kLinStore) *o = v;
        if (EPI == kLinGelu) *o = vkd::gelu1<0>(v);
        if (EPI == kLinGeluErf) *o = vkd::gelu1<1>(v);
        if (EPI == kLinResidual) *o = *o + v;
      }
    }
}

int check_linear(const vk_linear* lin, const vk_tensor* x, size_t rows) {
  VK_REQUIRE(x->dtype == VK_F32, "linear input must be f32");
  VK_REQUIRE(x->len == rows * lin->in_features, "linear: x holds %zu, rows*in=%zu", x->len,
             rows * lin->in_features);
  VK_UNSUPPORTED_IF(rows > 0x7fffffffULL, "linear: rows=%zu too large", rows);
  const long long tiles = static_cast<long long>((rows + BM - 1) / BM) *
                          static_cast<long long>((lin->out_features + BN - 1) / BN);
  VK_UNSUPPORTED_IF(tiles > 0x7fffffffLL, "linear: %lld tiles", tiles);
  return VK_OK;
}

// Output (or residual) checks; it must not overlap the input, which other
// workgroups may still be reading while one writes.
int check_linear_out(const vk_linear* lin, const vk_tensor* x, const vk_tensor* out, size_t rows,
                     const char* what) {
  VK_REQUIRE(out->dtype == VK_F32 && out->len == rows * lin->out_features,
             "linear: %s must be f32 [rows*out=%zu] (holds %zu)", what, rows * lin->out_features,
             out->len);
  const char* xb = static_cast<const char*>(x->ptr);
  const char* ob = static_cast<const char*>(out->ptr);
  VK_REQUIRE(ob + out->len * 4 <= xb || xb + x->len * 4 <= ob || rows == 0,
             "linear: %s overlaps the input", what);
  return VK_OK;
}

LinearArgs linear_args(const vk_linear* lin, const vk_tensor* x, size_t rows, vk_tensor* out) {
  LinearArgs g{};
  g.x = static_cast<const float*>(x->ptr);
  g.wnk = lin->weight_nk;
  g.bias = lin->bias;
  g.ls = lin->ls_gamma;
  g.out = out ? static_cast<float*>(out->ptr) : nullptr;
  g.M = static_cast<int>(rows);
  g.N = static_cast<int>(lin->out_features);
  g.K = static_cast<int>(lin->in_features);
  g.Kp = static_cast<int>(lin->k_pitch);
  return g;
}

bool tensors_disjoint(const vk_tensor* a, const vk_tensor* b) {
  const char* pa = static_cast<const char*>(a->ptr);
  const char* pb = static_cast<const char*>(b->ptr);
  return a->len == 0 || b->len == 0 || pa + a->len * 4 <= pb || pb + b->len * 4 <= pa;
}

// The head-major forms need the wide kernel: K % 4 == 0 and an aligned x.
int check_head_layout(const vk_linear* lin, const vk_tensor* x, size_t heads, size_t head_dim) {
  VK_UNSUPPORTED_IF(head_dim != 64, "linear: head_dim=%zu (qualified: 64)", head_dim);
  VK_REQUIRE(heads > 0, "linear: heads must be positive");
  VK_UNSUPPORTED_IF(lin->in_features % 4 != 0 || reinterpret_cast<uintptr_t>(x->ptr) % 16 != 0,
                    "linear: head-major forms need in_features %% 4 == 0 and an aligned input");
  return VK_OK;
}

int launch_linear(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
                  vk_tensor* out, int epi, float* partial = nullptr,
                  size_t partial_floats = 0) {
  if (rows == 0) return VK_OK;
  LinearArgs g{};
  g.x = static_cast<const float*>(x->ptr);
  g.wnk = lin->weight_nk;
  g.bias = lin->bias;
  g.ls = lin->ls_gamma;
  g.out = static_cast<float*>(out->ptr);
  g.M = static_cast<int>(rows);
  g.N = static_cast<int>(lin->out_features);
  g.K = static_cast<int>(lin->in_features);
  g.Kp = static_cast<int>(lin->k_pitch);
  // 128x128 tiles wherever rows of x can be read as float4; the 48x64 kernel
  // (scalar loads of x) for the rest
  if (g.K % 4 == 0 && reinterpret_cast<uintptr_t>(g.x) % 16 == 0)
    return vk::launch_linear_wide(rt, g, epi, partial, partial_floats);
  const unsigned tiles = static_cast<unsigned>(((g.M + BM - 1) / BM) * static_cast<long long>((g.N + BN - 1) / BN));
  const dim3 grid(tiles), block(kThreads);
  switch (epi) {
    case kLinStore: hipLaunchKernelGGL(linear_kernel<kLinStore>, grid, block, 0, rt->stream, g); break;
    case kLinGelu: hipLaunchKernelGGL(linear_kernel<kLinGelu>, grid, block, 0, rt->stream, g); break;
    case kLinGeluErf: hipLaunchKernelGGL(linear_kernel<kLinGeluErf>, grid, block, 0, rt->stream, g); break;
    default: hipLaunchKernelGGL(linear_kernel<kLinResidual>, grid, block, 0, rt->stream, g); break;
  }
  return vk::check_launch("linear_kernel");
}

}  // namespace

namespace vk {

namespace {

// The residual projection followed by ln_out = LayerNorm(residual), for a
// token-major input (heads == 0) or a head-major one.  The wide kernel takes
// the LayerNorm into its split-K sum pass; an input it cannot read (K % 4 or
// alignment) runs the two calls.
int residual_layernorm(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
                       size_t heads, size_t head_dim, vk_tensor* residual,
                       const vk_tensor* gamma, const vk_tensor* beta, float eps,
                       vk_tensor* ln_out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && residual && gamma && beta && ln_out, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  if (heads > 0) {
    VK_TRY(check_head_layout(lin, x, heads, head_dim));
    VK_REQUIRE(lin->in_features == heads * head_dim,
               "linear_residual_layernorm: in_features=%zu, expected heads*64=%zu",
               lin->in_features, heads * head_dim);
  }
  VK_TRY(check_linear_out(lin, x, residual, rows, "residual"));
  const size_t n = lin->out_features;
  VK_REQUIRE((gamma->dtype == VK_F32 || gamma->dtype == VK_F16) && gamma->dtype == beta->dtype &&
                 gamma->len == n && beta->len == n,
             "linear_residual_layernorm: gamma/beta must be f32 or f16 [%zu]", n);
  VK_UNSUPPORTED_IF(n > 8192, "linear_residual_layernorm: out_features=%zu (LayerNorm rows of "
                    "at most 8192)", n);
  VK_REQUIRE(ln_out->dtype == VK_F32 && ln_out->len == rows * n,
             "linear_residual_layernorm: ln_out must be f32 [%zu]", rows * n);
  VK_REQUIRE(tensors_disjoint(ln_out, residual) && tensors_disjoint(ln_out, x),
             "linear_residual_layernorm: ln_out must not overlap the other tensors");
  for (const vk_tensor* t : {static_cast<const vk_tensor*>(residual), gamma, beta,
                             static_cast<const vk_tensor*>(ln_out)})
    VK_REQUIRE(reinterpret_cast<uintptr_t>(t->ptr) % 16 == 0,
               "linear_residual_layernorm: tensors must be 16-byte aligned");
  if (rows == 0) return VK_OK;
  const bool wide = lin->in_features % 4 == 0 && reinterpret_cast<uintptr_t>(x->ptr) % 16 == 0;
  LinearArgs g = linear_args(lin, x, rows, residual);
  g.a_hnd = heads > 0 ? 1 : 0;
  // The sum pass's LayerNorm reduces in the tree order; the sequential order
  // (and an input the wide kernel cannot read) takes the two calls.
  if (!wide || rt->ln_order == VK_LN_ORDER_SEQUENTIAL) {
    VK_TRY(wide ? vk::launch_linear_wide(rt, g, kLinResidual)
                : launch_linear(rt, lin, x, rows, residual, kLinResidual));
    return vk::layernorm_raw(rt, static_cast<const float*>(residual->ptr),
                             static_cast<float*>(ln_out->ptr), gamma->ptr, beta->ptr,
                             gamma->dtype == VK_F16, static_cast<int>(rows),
                             static_cast<int>(n), eps);
  }
  g.ln_gamma = gamma->ptr;
  g.ln_beta = beta->ptr;
  g.ln_f16 = gamma->dtype == VK_F16 ? 1 : 0;
  g.ln_eps = eps;
  g.ln_out = static_cast<float*>(ln_out->ptr);
  return vk::launch_linear_wide(rt, g, kLinResidual);
}

}  // namespace

int linear_hnd_residual_layernorm(vk_runtime* rt, const vk_linear* lin, const vk_tensor* hnd,
                                  size_t rows, size_t heads, size_t head_dim,
                                  vk_tensor* residual, const vk_tensor* gamma,
                                  const vk_tensor* beta, float eps, vk_tensor* ln_out) {
  VK_REQUIRE(heads > 0, "linear: heads must be positive");
  return residual_layernorm(rt, lin, hnd, rows, heads, head_dim, residual, gamma, beta, eps,
                            ln_out);
}

int linear_residual_layernorm(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x,
                              size_t rows, vk_tensor* residual, const vk_tensor* gamma,
                              const vk_tensor* beta, float eps, vk_tensor* ln_out) {
  return residual_layernorm(rt, lin, x, rows, 0, 0, residual, gamma, beta, eps, ln_out);
}

}  // namespace vk

extern "C" {

int vk_linear_run_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
                      vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && out, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, rows * lin->out_features, &t));
  const int s = launch_linear(rt, lin, x, rows, t, kLinStore);
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

int vk_linear_run_into_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
                           vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && out, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  VK_TRY(check_linear_out(lin, x, out, rows, "out"));
  return launch_linear(rt, lin, x, rows, out, kLinStore);
}

int vk_linear_run_gelu_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
                           vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && out, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  VK_TRY(check_linear_out(lin, x, out, rows, "out"));
  VK_REQUIRE(lin->ls_gamma == nullptr, "linear_run_gelu: the linear carries a LayerScale");
  return launch_linear(rt, lin, x, rows, out, kLinGelu);
}

int vk_linear_run_gelu_erf_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x,
                               size_t rows, vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && out, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  VK_TRY(check_linear_out(lin, x, out, rows, "out"));
  VK_REQUIRE(lin->ls_gamma == nullptr, "linear_run_gelu_erf: the linear carries a LayerScale");
  return launch_linear(rt, lin, x, rows, out, kLinGeluErf);
}

int vk_linear_run_residual_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x,
                               size_t rows, vk_tensor* residual) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && residual, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  VK_TRY(check_linear_out(lin, x, residual, rows, "residual"));
  return launch_linear(rt, lin, x, rows, residual, kLinResidual);
}

int vk_linear_run_qkv_hnd_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x,
                              size_t rows, size_t heads, size_t head_dim, vk_tensor* q,
                              vk_tensor* k, vk_tensor* v) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && q && k && v, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  VK_TRY(check_head_layout(lin, x, heads, head_dim));
  VK_REQUIRE(lin->out_features == 3 * heads * head_dim,
             "linear_run_qkv_hnd: out_features=%zu, expected 3*heads*head_dim=%zu",
             lin->out_features, 3 * heads * head_dim);
  VK_REQUIRE(lin->ls_gamma == nullptr, "linear_run_qkv_hnd: the linear carries a LayerScale");
  const size_t part = rows * heads * head_dim;
  for (const vk_tensor* t : {q, k, v})
    VK_REQUIRE(t->dtype == VK_F32 && t->len == part, "q, k, v must be f32 [rows*heads*64=%zu]",
               part);
  VK_REQUIRE(tensors_disjoint(x, q) && tensors_disjoint(x, k) && tensors_disjoint(x, v) &&
                 tensors_disjoint(q, k) && tensors_disjoint(q, v) && tensors_disjoint(k, v),
             "linear_run_qkv_hnd: tensors overlap");
  if (rows == 0) return VK_OK;
  LinearArgs g = linear_args(lin, x, rows, nullptr);
  g.q_out = static_cast<float*>(q->ptr);
  g.k_out = static_cast<float*>(k->ptr);
  g.v_out = static_cast<float*>(v->ptr);
  return vk::launch_linear_wide(rt, g, kLinStore);
}

int vk_linear_run_qkv_hnd_norm_rope_f32(vk_runtime* rt, const vk_linear* lin,
                                        const vk_tensor* x, size_t rows, size_t heads,
                                        size_t head_dim, vk_tensor* q, vk_tensor* k,
                                        vk_tensor* v, const vk_tensor* q_gamma,
                                        const vk_tensor* q_beta, const vk_tensor* k_gamma,
                                        const vk_tensor* k_beta, size_t n_special, size_t gh,
                                        size_t gw, size_t view_count, int global, float freq,
                                        float eps) {
  return vk_linear_run_qkv_hnd_norm_rope_mode_f32(rt, lin, x, rows, heads, head_dim, q, k, v,
                                                  q_gamma, q_beta, k_gamma, k_beta, n_special,
                                                  gh, gw, view_count, global, freq, eps,
                                                  VK_ROPE_DEFAULT);
}

int vk_linear_run_qkv_hnd_norm_rope_mode_f32(vk_runtime* rt, const vk_linear* lin,
                                             const vk_tensor* x, size_t rows, size_t heads,
                                             size_t head_dim, vk_tensor* q, vk_tensor* k,
                                             vk_tensor* v, const vk_tensor* q_gamma,
                                             const vk_tensor* q_beta, const vk_tensor* k_gamma,
                                             const vk_tensor* k_beta, size_t n_special,
                                             size_t gh, size_t gw, size_t view_count,
                                             int global, float freq, float eps,
                                             unsigned rope_mode) {
  VK_TRY(vk::bind(rt));
  VK_TRY(vk::check_rope_mode(rope_mode));
  VK_REQUIRE(lin && x && q && k && v, "null argument");
  VK_UNSUPPORTED_IF(head_dim != 64, "qkv norm_rope: head_dim=%zu (qualified: 64)", head_dim);
  VK_REQUIRE(view_count > 0 && gw > 0, "view_count and gw must be > 0");
  VK_REQUIRE(rows == view_count * (n_special + gh * gw),
             "qkv norm_rope: rows=%zu, expected view_count*(n_special+gh*gw)=%zu", rows,
             view_count * (n_special + gh * gw));
  const bool any = q_gamma || q_beta || k_gamma || k_beta;
  const bool all = q_gamma && q_beta && k_gamma && k_beta;
  VK_REQUIRE(!any || all, "q/k norm parameters must be all present or all null");
  if (all) {
    for (const vk_tensor* t : {q_gamma, q_beta, k_gamma, k_beta})
      VK_REQUIRE((t->dtype == VK_F32 || t->dtype == VK_F16) && t->dtype == q_gamma->dtype &&
                     t->len == head_dim,
                 "q/k norm parameters must be f32 or f16 vectors of 64 sharing one dtype");
  }
  VK_UNSUPPORTED_IF(rows > 0x7fffffffULL, "qkv norm_rope: rows=%zu too large", rows);
  // Q|K|V projection checks (and nothing to do for zero rows)
  if (rows == 0) return vk_linear_run_qkv_hnd_f32(rt, lin, x, rows, heads, head_dim, q, k, v);
  VK_TRY(check_linear(lin, x, rows));
  VK_TRY(check_head_layout(lin, x, heads, head_dim));
  VK_REQUIRE(lin->out_features == 3 * heads * head_dim,
             "linear_run_qkv_hnd: out_features=%zu, expected 3*heads*head_dim=%zu",
             lin->out_features, 3 * heads * head_dim);
  VK_REQUIRE(lin->ls_gamma == nullptr, "linear_run_qkv_hnd: the linear carries a LayerScale");
  const size_t part = rows * heads * head_dim;
  for (const vk_tensor* t : {q, k, v})
    VK_REQUIRE(t->dtype == VK_F32 && t->len == part, "q, k, v must be f32 [rows*heads*64=%zu]",
               part);
  VK_REQUIRE(tensors_disjoint(x, q) && tensors_disjoint(x, k) && tensors_disjoint(x, v) &&
                 tensors_disjoint(q, k) && tensors_disjoint(q, v) && tensors_disjoint(k, v),
             "linear_run_qkv_hnd: tensors overlap");
  // the grid's largest coordinate is max(gh, gw) + 1: the table covers it
  const size_t max_coord = (gh > gw ? gh : gw) + 1;
  VK_UNSUPPORTED_IF(max_coord > (1u << 22), "patch grid %zux%zu too large", gh, gw);
  const float* table = nullptr;
  int table_max = 0;
  VK_TRY(vk::rope_table(rt, freq, 64, rope_mode, static_cast<int>(max_coord), &table,
                        &table_max));
  LinearArgs g = linear_args(lin, x, rows, nullptr);
  g.q_out = static_cast<float*>(q->ptr);
  g.k_out = static_cast<float*>(k->ptr);
  g.v_out = static_cast<float*>(v->ptr);
  if (all && rt->ln_order == VK_LN_ORDER_SEQUENTIAL) {
    // the epilogue's Q/K LayerNorm reduces in the tree order: the
    // sequential order stores Q, K, V and runs the Q/K pass over them (rows
    // in the same head-major order, the same grid positions)
    VK_TRY(vk::launch_linear_wide(rt, g, kLinStore));
    return vk_qk_norm_rope_grid_mode_f32(rt, q, k, q_gamma, q_beta, k_gamma, k_beta, heads,
                                         head_dim, n_special, gh, gw, view_count, global,
                                         VK_QK_HEADS_OUTER, freq, eps, rope_mode);
  }
  g.qkn_mode = !all ? 3 : (q_gamma->dtype == VK_F16 ? 2 : 1);
  g.qkn.qg = all ? q_gamma->ptr : nullptr;
  g.qkn.qb = all ? q_beta->ptr : nullptr;
  g.qkn.kg = all ? k_gamma->ptr : nullptr;
  g.qkn.kb = all ? k_beta->ptr : nullptr;
  g.qkn.table = table;
  g.qkn.table_max = table_max;
  g.qkn.n_special = static_cast<uint32_t>(n_special);
  g.qkn.global = global ? 1u : 0u;
  g.qkn.tpv = vkd::make_fastdiv(static_cast<uint32_t>(n_special + gh * gw));
  g.qkn.gw = vkd::make_fastdiv(static_cast<uint32_t>(gw));
  g.qkn.eps = eps;
  g.qkn.interleaved = (rope_mode & VK_ROPE_INTERLEAVED) ? 1u : 0u;
  return vk::launch_linear_wide(rt, g, kLinStore);
}

static int run_hnd(vk_runtime* rt, const vk_linear* lin, const vk_tensor* hnd, size_t rows,
                   size_t heads, size_t head_dim, vk_tensor* out, int epi, const char* what) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && hnd && out, "null argument");
  VK_TRY(check_linear(lin, hnd, rows));
  VK_TRY(check_head_layout(lin, hnd, heads, head_dim));
  VK_REQUIRE(lin->in_features == heads * head_dim, "%s: in_features=%zu, expected heads*64=%zu",
             what, lin->in_features, heads * head_dim);
  VK_TRY(check_linear_out(lin, hnd, out, rows, epi == kLinResidual ? "residual" : "out"));
  if (rows == 0) return VK_OK;
  LinearArgs g = linear_args(lin, hnd, rows, out);
  g.a_hnd = 1;
  return vk::launch_linear_wide(rt, g, epi);
}

int vk_linear_run_hnd_into_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* hnd,
                               size_t rows, size_t heads, size_t head_dim, vk_tensor* out) {
  return run_hnd(rt, lin, hnd, rows, heads, head_dim, out, kLinStore, "linear_run_hnd_into");
}

int vk_linear_run_hnd_residual_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* hnd,
                                   size_t rows, size_t heads, size_t head_dim,
                                   vk_tensor* residual) {
  return run_hnd(rt, lin, hnd, rows, heads, head_dim, residual, kLinResidual,
                 "linear_run_hnd_residual");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free linear: vk_linear_run_into_f32 with the split-K partial
// sums in a static device array instead of the runtime's work buffer.
//
// `scratch` is a file-scope device array: each device holds its own copy
// from the library's load until the process ends.  Host code never uses its
// name as an address (on the host it is a stand-in symbol): the device
// address is looked up once per device, with that device current, when a
// runtime is created on it (vk_runtime_create -> vk::noalloc_setup), and
// only that address is handed to kernels.  Every call on one device shares
// that device's array; each split writes its whole slice before the sum
// pass reads it, so nothing needs clearing, but calls that overlap on one
// device (two runtimes' streams at once) race on it.
// ---------------------------------------------------------------------------
constexpr size_t kScratchFloats = size_t{8} << 20;  // 32 MiB per device

static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};
bool g_scratch_done[kMaxDevices] = {};

}  // namespace

namespace vk {

void noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_done[device]) return;
  void* p = nullptr;
  // the caller (vk_runtime_create) made `device` current
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  g_scratch_err[device] = e;
  g_scratch_ptr[device] = e == hipSuccess ? static_cast<float*>(p) : nullptr;
  g_scratch_done[device] = true;
  // A failure is kept above and reported by the allocation-free entry point
  // alone; clear it from HIP's last-error state so that the next launch
  // check on this thread does not take it for its own.
  if (e != hipSuccess) (void)hipGetLastError();
}

}  // namespace vk

extern "C" {

int vk_linear_run_into_noalloc_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x,
                                   size_t rows, vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && out, "null argument");
  VK_TRY(check_linear(lin, x, rows));
  VK_TRY(check_linear_out(lin, x, out, rows, "out"));
  float* sp = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    VK_REQUIRE(rt->device < kMaxDevices && g_scratch_done[rt->device],
               "linear_run_into_noalloc: no scratch address for device %d", rt->device);
    if (g_scratch_err[rt->device] != hipSuccess)
      return vk::hip_fail(g_scratch_err[rt->device], "hipGetSymbolAddress(scratch)");
    sp = g_scratch_ptr[rt->device];
  }
  return launch_linear(rt, lin, x, rows, out, kLinStore, sp, kScratchFloats);
}

}  // extern "C"
