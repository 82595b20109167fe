// Scaled dot-product attention for gfx950, F32 in / F32 accumulate:
// out = softmax(Q K^T / sqrt(64)) V over independent head-major sequences
// [n, 64] (a head of one view for local layers, a head of the whole flattened
// multi-view sequence for global layers), with an online (one-pass) softmax.
//
// A 256-thread workgroup (4 waves) owns 64 queries of one sequence; wave w
// owns queries 16w..16w+15.  Keys and values stream through LDS in blocks of
// 64: K as [key][d] rows, V transposed as [d][key] rows, both with a pitch of
// 68 floats (4 x odd: 16-row fragment reads are bank-conflict free).
//
// Per key block a wave runs 128 v_mfma_f32_16x16x4_f32:
//  * S^T = K Q^T (A = K, B = Q^T).  The transposed product leaves, in lane l,
//    the scores of query l%16 for keys 16t + 4(l/16) + r (r = 0..3) of key
//    tile t; the row max and sum of a query are then in-register over r and
//    t plus two cross-group shuffles.
//  * O += P V (A = P, B = V).  In the k-permuted fragment order used
//    throughout this library (lane group g holds k = 16b + 4g + j in
//    component j, MFMA step j takes component j) the A operand of key tile t
//    is exactly the lane's four probabilities of that tile: P never leaves
//    registers.  O's rows are queries 4(l/16) + r, so the per-query rescale
//    factors reach them with four shuffles.
// Scores are kept in the base-2 domain: Q is read once per workgroup and
// pre-scaled by log2(e)/sqrt(64), so every softmax weight is one v_exp_f32
// (2^x) of a difference of scores: p = 2^(s' - m') = e^(s - m).
// Keys past n are masked to -inf (last block only); queries past n are
// computed on a clamped row and not stored.
//
// Staging: K goes to LDS row-major with 128-bit stores (16 lanes fill one
// 256-byte key row).  V is transposed on the way in; its loads are mapped so
// that the 64 lanes of a wave hold 16 keys x 4 float4 columns, which makes
// every transposed 32-bit store of the wave hit 64 distinct banks.
#include <cmath>

#include "common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int HD = 64;
constexpr int QB = 64;  // queries per workgroup
constexpr int KB = 64;  // keys per block
constexpr int PITCH = 68;
constexpr int kThreads = 256;
constexpr float kQScale = 0.125f * 1.44269504088896341f;  // log2(e) / sqrt(64)
static_assert(PITCH % 4 == 0 && (PITCH / 4) % 2 == 1, "pitch 4 x odd");
static_assert(PITCH % 16 == 4, "transposed V stores: 16 (l >> 4) + (l & 15) covers 64 banks");

__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

__device__ __forceinline__ float group_sum(float v) {
  v = v + __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}

__global__ __launch_bounds__(kThreads) void attention_kernel(const float* __restrict__ q,
                                                             const float* __restrict__ k,
                                                             const float* __restrict__ v,
                                                             float* __restrict__ out,
                                                             int sequences, int n) {
  __shared__ __align__(16) float Ks[KB * PITCH];
  __shared__ __align__(16) float Vt[HD * PITCH];

  const int tid = threadIdx.x;
  __builtin_assume(tid < kThreads);
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int nqb = (n + QB - 1) / QB;
  // XCD-major numbering: the query blocks of one sequence share an XCD's L2
  const int tile = vkd::xcd_tile(blockIdx.x, gridDim.x);
  const int seq = tile / nqb, q0 = (tile % nqb) * QB + wave * 16;
  const size_t base = static_cast<size_t>(seq) * n * HD;

  // Q^T fragments (B operand): query q0 + c16, d = 16 bd + 4 g + j
  f32x4 qf[4];
  {
    const int qi = q0 + c16 < n ? q0 + c16 : n - 1;
    const float* qrow = q + base + static_cast<size_t>(qi) * HD + 4 * g;
#pragma unroll
    for (int bd = 0; bd < 4; ++bd) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(qrow + 16 * bd);
      qf[bd] = t * kQScale;
    }
  }

  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;  // statistics of query q0 + c16

  const int skey = tid >> 4, sd = 4 * (tid & 15);  // K staging slot: key, d
  // V staging slot: key 16 w + (l & 15), float4 columns (l >> 4) + 4 i
  const int vkey = 16 * wave + (lane & 15), vcol = lane >> 4;
  const float* karow = Ks + c16 * PITCH + 4 * g;
  const float* vtrow = Vt + c16 * PITCH + 4 * g;

  for (int k0 = 0; k0 < n; k0 += KB) {
    // stage: slot f = tid + 256 i is key f/16, float4 f%16 of the block
    f32x4 kr[4], vr[4];
    {
      const int vk = k0 + vkey < n ? k0 + vkey : n - 1;
      const float* vrow = v + base + static_cast<size_t>(vk) * HD;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = k0 + skey + 16 * i;
        const int ck = key < n ? key : n - 1;
        kr[i] = *reinterpret_cast<const f32x4*>(k + base + static_cast<size_t>(ck) * HD + sd);
        vr[i] = *reinterpret_cast<const f32x4*>(vrow + 4 * (vcol + 4 * i));
      }
    }
    __syncthreads();  // the previous block is consumed
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<f32x4*>(Ks + (skey + 16 * i) * PITCH + sd) = kr[i];
      const int d = 4 * (vcol + 4 * i);
#pragma unroll
      for (int c = 0; c < 4; ++c) Vt[(d + c) * PITCH + vkey] = vr[i][c];
    }
    __syncthreads();

    // S^T tiles: s[t][r] = score of query q0 + c16 with key k0 + 16t + 4g + r
    f32x4 s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int bd = 0; bd < 4; ++bd) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(karow + t * 16 * PITCH + 16 * bd);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], qf[bd][j], s[t], 0, 0, 0);
      }
    }
    if (k0 + KB > n) {  // the last, partial block
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (k0 + 16 * t + 4 * g + r >= n) s[t][r] = -INFINITY;
    }
    float mb = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) mb = fmaxf(mb, s[t][r]);
    const float m_new = fmaxf(m_run, group_max(mb));
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first block
    float ps = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[t][r] = __builtin_amdgcn_exp2f(s[t][r] - m_new);
        ps += s[t][r];
      }
    l_run = l_run * alpha + group_sum(ps);
    m_run = m_new;

    // rescale O: row 4g + r belongs to query q0 + 4g + r, whose factor sits
    // in lane 4g + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt][r] *= ar;
    }
    // O += P V: A = the lane's probabilities of key tile t, B = V^T rows
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(vtrow + dt * 16 * PITCH + 16 * t);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(s[t][j], b[j], o[dt], 0, 0, 0);
      }
  }

  // out[query][d] = O / l, O row 4g + r, column 16 dt + c16
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float lr = __shfl(l_run, 4 * g + r, 64);
    const int qi = q0 + 4 * g + r;
    if (qi < n) {
      float* orow = out + base + static_cast<size_t>(qi) * HD + c16;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) orow[16 * dt] = o[dt][r] / lr;
    }
  }
}

int check_qkv(const vk_tensor* t, size_t len, const char* what) {
  VK_REQUIRE(t && t->dtype == VK_F32 && t->len == len, "attention: %s must be f32 [%zu] (holds %zu)",
             what, len, t ? t->len : 0);
  VK_REQUIRE(reinterpret_cast<uintptr_t>(t->ptr) % 16 == 0, "attention: %s must be 16-byte aligned",
             what);
  return VK_OK;
}

}  // namespace

extern "C" {

int vk_attention_into_f32(vk_runtime* rt, const vk_tensor* q, const vk_tensor* k,
                          const vk_tensor* v, size_t sequences, size_t n, size_t head_dim,
                          vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(q && k && v && out, "null argument");
  VK_UNSUPPORTED_IF(head_dim != HD, "attention: head_dim=%zu (qualified: 64)", head_dim);
  VK_UNSUPPORTED_IF(n > 0x7fffffffULL || sequences > 0x7fffffffULL, "attention: too large");
  const size_t len = sequences * n * HD;
  VK_TRY(check_qkv(q, len, "q"));
  VK_TRY(check_qkv(k, len, "k"));
  VK_TRY(check_qkv(v, len, "v"));
  VK_TRY(check_qkv(out, len, "out"));
  for (const vk_tensor* t : {q, k, v}) {
    const char* a = static_cast<const char*>(t->ptr);
    const char* b = static_cast<const char*>(out->ptr);
    VK_REQUIRE(len == 0 || a + len * 4 <= b || b + len * 4 <= a,
               "attention: out overlaps an input");
  }
  if (len == 0) return VK_OK;
  const long long blocks = static_cast<long long>(sequences) * ((n + QB - 1) / QB);
  VK_UNSUPPORTED_IF(blocks > 0x7fffffffLL, "attention: %lld workgroups", blocks);
  hipLaunchKernelGGL(attention_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     rt->stream, static_cast<const float*>(q->ptr),
                     static_cast<const float*>(k->ptr), static_cast<const float*>(v->ptr),
                     static_cast<float*>(out->ptr), static_cast<int>(sequences),
                     static_cast<int>(n));
  return vk::check_launch("attention_kernel");
}

int vk_attention_online_f32(vk_runtime* rt, const vk_tensor* q, const vk_tensor* k,
                            const vk_tensor* v, size_t heads, size_t rows, size_t head_dim,
                            vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out, "null argument");
  VK_UNSUPPORTED_IF(head_dim != HD, "attention: head_dim=%zu (qualified: 64)", head_dim);
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, heads * rows * head_dim, &t));
  const int s = vk_attention_into_f32(rt, q, k, v, heads, rows, head_dim, t);
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

}  // extern "C"
