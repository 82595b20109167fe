// Scaled dot-product attention for gfx950, F32 in / F32 accumulate:
// out = softmax(Q K^T / sqrt(64)) V over independent head-major sequences
// [n, 64] (a head of one view for local layers, a head of the whole flattened
// multi-view sequence for global layers), with an online (one-pass) softmax.
//
// A 256-thread workgroup (4 waves) owns 64 queries of one sequence; wave w
// owns queries 16w..16w+15.  Grids of fewer than two such workgroups per CU
// (a single image's local layer: 12 heads x 14 tiles) use workgroups of 32
// queries whose two halves split the key blocks (attention_kernel<2, 2>).  Keys and values stream through LDS in blocks of
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
constexpr int KB = 64;  // keys per block
constexpr int PITCH = 68;
constexpr int kSlots = KB * HD / 4;  // float4 of one K (or V) block: 1024
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

// QG query groups of 16 (one wave each) x KS key splits per workgroup.
// <4, 1>: 64 queries, every key block, the normal form.  <2, 2>: 32 queries,
// two halves of 2 waves that take alternate key blocks (each with its own
// staging buffers) and merge their partial results through LDS at the end
// -- the form for grids that would leave CUs idle (a single image's local
// layer: 12 heads x 14 tiles), keeping 4 waves and all four SIMDs per
// workgroup.
template <int QG, int KS>
__global__ __launch_bounds__(64 * QG * KS) void attention_kernel(const float* __restrict__ q,
                                                                 const float* __restrict__ k,
                                                                 const float* __restrict__ v,
                                                                 float* __restrict__ out,
                                                                 int sequences, int n) {
  constexpr int kThreads = 64 * QG * KS;
  constexpr int kHalf = 64 * QG;          // threads of one key split
  constexpr int QB = 16 * QG;             // queries per workgroup
  constexpr int kPer = kSlots / kHalf;    // staged float4 of K (and of V) per thread
  static_assert(KS == 1 || KS == 2, "one or two key splits");
  __shared__ __align__(16) float smem[KS * 2 * KB * PITCH];

  const int tid = threadIdx.x;
  __builtin_assume(tid < kThreads);
  const int wave = tid >> 6, lane = tid & 63;
  const int half = wave / QG, wq = wave % QG;  // key split, query group
  const int htid = tid - half * kHalf;         // thread index inside the split
  const int g = lane >> 4, c16 = lane & 15;
  float* Ks = smem + half * 2 * KB * PITCH;
  float* Vt = Ks + KB * PITCH;
  const int nqb = (n + QB - 1) / QB;
  // XCD-major numbering: the query blocks of one sequence share an XCD's L2
  const int tile = vkd::xcd_tile(blockIdx.x, gridDim.x);
  const int seq = tile / nqb, q0 = (tile % nqb) * QB + wq * 16;
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

  // K staging: slot f = htid + kHalf i is key f/16, float4 f%16 (16 lanes
  // fill one key row).  V staging: slot f -> w' = f/64, key 16 (w' % 4) +
  // (l & 15), float4 column (l >> 4) + 4 (w' / 4); one wave instruction covers
  // 16 keys x 4 columns.
  const int skey = htid >> 4, sd = 4 * (htid & 15);
  const float* karow = Ks + c16 * PITCH + 4 * g;
  const float* vtrow = Vt + c16 * PITCH + 4 * g;
  // Whole key blocks load through buffer resources: the lane's byte offset
  // inside a block is fixed, the block's offset is uniform, so the loads
  // carry no per-block vector address arithmetic.  (The kernel's tensors
  // are under 4 GiB, checked at launch.)
  const uint32_t bytes = 4u * static_cast<uint32_t>(sequences) * static_cast<uint32_t>(n) * HD;
  const __amdgpu_buffer_rsrc_t k_rsrc = vkd::buffer_rsrc(k, bytes);
  const __amdgpu_buffer_rsrc_t v_rsrc = vkd::buffer_rsrc(v, bytes);
  uint32_t k_off[kPer], v_off[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    k_off[i] = 4u * static_cast<uint32_t>((skey + (kHalf / 16) * i) * HD + sd);
    const int w2 = wq + QG * i;
    v_off[i] = 4u * static_cast<uint32_t>((16 * (w2 & 3) + (lane & 15)) * HD +
                                          4 * ((lane >> 4) + 4 * (w2 >> 2)));
  }

  const int nkb = (n + KB - 1) / KB;
  const int iters = (nkb + KS - 1) / KS;
  for (int it = 0; it < iters; ++it) {
    const int k0 = (it * KS + half) * KB;
    // uniform per split: with two splits the odd half may run out of blocks
    const bool active = KS == 1 || k0 < n;
    f32x4 kr[kPer], vr[kPer];
    if (active && k0 + KB <= n) {
      const uint32_t blk = 4u * (static_cast<uint32_t>(seq) * static_cast<uint32_t>(n) +
                                 static_cast<uint32_t>(k0)) * HD;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const float4 a = vkd::buffer_load4(k_rsrc, k_off[i], blk);
        const float4 b = vkd::buffer_load4(v_rsrc, v_off[i], blk);
        kr[i] = f32x4{a.x, a.y, a.z, a.w};
        vr[i] = f32x4{b.x, b.y, b.z, b.w};
      }
    } else if (active) {  // the last, partial block: keys past n read key n - 1
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int key = k0 + skey + (kHalf / 16) * i;
        const int ck = key < n ? key : n - 1;
        kr[i] = *reinterpret_cast<const f32x4*>(k + base + static_cast<size_t>(ck) * HD + sd);
        const int w2 = wq + QG * i;
        const int vkey = k0 + 16 * (w2 & 3) + (lane & 15);
        const int cv = vkey < n ? vkey : n - 1;
        vr[i] = *reinterpret_cast<const f32x4*>(v + base + static_cast<size_t>(cv) * HD +
                                                4 * ((lane >> 4) + 4 * (w2 >> 2)));
      }
    }
    __syncthreads();  // the previous block is consumed
    if (active) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        *reinterpret_cast<f32x4*>(Ks + (skey + (kHalf / 16) * i) * PITCH + sd) = kr[i];
        const int w2 = wq + QG * i;
        const int key = 16 * (w2 & 3) + (lane & 15);
        const int d = 4 * ((lane >> 4) + 4 * (w2 >> 2));
#pragma unroll
        for (int c = 0; c < 4; ++c) Vt[(d + c) * PITCH + key] = vr[i][c];
      }
    }
    __syncthreads();
    if (!active) continue;

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
    // in lane 4g + r.  Skipped when every factor of the wave is exactly 1 (no
    // row maximum grew): multiplying by 1 changes no bits.
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt][r] *= ar;
      }
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

  if constexpr (KS == 2) {
    // merge the odd-block half into the even-block half: the waves of one
    // query group hold the same queries in the same lane layout
    constexpr int kX = 18;  // o (16), m, l per lane
    __syncthreads();        // the staging buffers are free
    float* xr = smem + (wq * 64 + lane) * kX;
    if (half == 1) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) xr[dt * 4 + r] = o[dt][r];
      xr[16] = m_run;
      xr[17] = l_run;
    }
    __syncthreads();
    if (half == 1) return;
    const float m1 = xr[16], l1 = xr[17];
    const float m = fmaxf(m_run, m1);
    const float a0 = __builtin_amdgcn_exp2f(m_run - m);  // of query q0 + c16
    const float a1 = __builtin_amdgcn_exp2f(m1 - m);
    l_run = l_run * a0 + l1 * a1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float b0 = __shfl(a0, 4 * g + r, 64), b1 = __shfl(a1, 4 * g + r, 64);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt][r] = o[dt][r] * b0 + xr[dt * 4 + r] * b1;
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
  VK_UNSUPPORTED_IF(len >= (size_t{1} << 30), "attention: tensors of 4 GiB or more");
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
  // 64-query tiles unless they give fewer than two workgroups per CU; then
  // 32-query tiles with the keys split over two halves of the workgroup
  const long long tiles64 = static_cast<long long>(sequences) * ((n + 63) / 64);
  const bool narrow = tiles64 < 2LL * (rt->cu_count > 0 ? rt->cu_count : 256);
  const int qb = narrow ? 32 : 64;
  const long long blocks = static_cast<long long>(sequences) * ((n + qb - 1) / qb);
  VK_UNSUPPORTED_IF(blocks > 0x7fffffffLL, "attention: %lld workgroups", blocks);
  const auto* Q = static_cast<const float*>(q->ptr);
  const auto* K = static_cast<const float*>(k->ptr);
  const auto* V = static_cast<const float*>(v->ptr);
  auto* O = static_cast<float*>(out->ptr);
  const int S = static_cast<int>(sequences), N = static_cast<int>(n);
  if (narrow)
    hipLaunchKernelGGL((attention_kernel<2, 2>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                       0, rt->stream, Q, K, V, O, S, N);
  else
    hipLaunchKernelGGL((attention_kernel<4, 1>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                       0, rt->stream, Q, K, V, O, S, N);
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
