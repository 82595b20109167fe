// Scaled dot-product attention for gfx950, F32 in / F32 accumulate:
// out = softmax(Q K^T / sqrt(64)) V over independent head-major sequences
// [n, 64] (a head of one view for local layers, a head of the whole flattened
// multi-view sequence for global layers), with an online (one-pass) softmax.
//
// A 256-thread workgroup (4 waves) owns 64 queries of one sequence; wave w
// owns queries 16w..16w+15 (unsplit launches over short sequences: 512
// threads, 8 waves, 128 queries).  Grids of fewer than two 64-query
// workgroups per CU (a single image's layer: 12 heads x 14 tiles) split
// each tile's key blocks over several workgroups and merge the partial
// results in a second pass (attention_kernel<true, 4>,
// attention_merge_kernel).  Keys and values stream through LDS in blocks
// of 64: K as [key][d] rows, V transposed as
// [d][key] rows, both with a pitch of 68 floats (4 x odd: 16-row fragment
// reads are bank-conflict free).
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
// Unsplit launches over sequences of at most this many rows run 128-query
// workgroups of eight waves (two to a CU: four waves per SIMD, as four-wave
// workgroups four to a CU give, with half the K/V staging per query): a
// 12-view local layer (144 x 866) 259.6-265.4 -> 252.8-258.1 us, bits
// unchanged.  The global layer (10,392 rows) measured 1% slower in
// that form when it ran unsplit.
constexpr int kWideTileMaxN = 1024;
static_assert(PITCH % 4 == 0 && (PITCH / 4) % 2 == 1, "pitch 4 x odd");
static_assert(PITCH % 16 == 4, "transposed V stores: 16 (l >> 4) + (l & 15) covers 64 banks");

// Max and sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lane groups
// of one query column).  v_permlane16_swap / v_permlane32_swap with both
// operands v leave each lane its own value and that of lane l ^ 16 (l ^ 32)
// in the two results: a VALU exchange, with no LDS round trip.  Both
// operations are commutative, so the result has the bits of the butterfly
// v op shfl_xor(v, 16), then op shfl_xor(., 32).
__device__ __forceinline__ float xor16_pair(float v, float* other) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  *other = __uint_as_float(r[1]);
  return __uint_as_float(r[0]);
}

__device__ __forceinline__ float xor32_pair(float v, float* other) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  *other = __uint_as_float(r[1]);
  return __uint_as_float(r[0]);
}

__device__ __forceinline__ float group_max(float v) {
  float o;
  v = xor16_pair(v, &o);
  v = fmaxf(v, o);
  v = xor32_pair(v, &o);
  return fmaxf(v, o);
}

__device__ __forceinline__ float group_sum(float v) {
  float o;
  v = xor16_pair(v, &o);
  v = v + o;
  v = xor32_pair(v, &o);
  return v + o;
}

// QG query groups of 16 (one wave each) per workgroup: 16 QG queries over
// every key block.  PART: grids of fewer than two workgroups per CU (a
// single image's layer: 12 heads x 14 query tiles) split the key blocks of
// each query tile into `splits` contiguous runs, one workgroup each; a run
// writes its O (scaled to its own running max), the max and the sum to
// `part` ([splits][rows][64], then [splits][rows][2]) and
// attention_merge_kernel combines them in split order.
template <bool PART, int QG>
__global__ __launch_bounds__(64 * QG) void attention_kernel(const float* __restrict__ q,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        float* __restrict__ out, int sequences,
                                                        int n, int splits,
                                                        float* __restrict__ part) {
  constexpr int kThreads = 64 * QG;       // QG query groups (waves)
  constexpr int QB = 16 * QG;             // queries per workgroup
  constexpr int kPer = kSlots / kThreads; // staged float4 of K (and of V) per thread
  __shared__ __align__(16) float smem[2 * KB * PITCH];

  const int tid = threadIdx.x;
  __builtin_assume(tid < kThreads);
  const int wave = tid >> 6, lane = tid & 63;
  const int wq = wave;  // query group
  const int g = lane >> 4, c16 = lane & 15;
  float* Ks = smem;
  float* Vt = Ks + KB * PITCH;
  const int nqb = (n + QB - 1) / QB;
  // XCD-major numbering: the query blocks of one sequence share an XCD's L2
  const int tile_all = vkd::xcd_tile(blockIdx.x, gridDim.x);
  const int split = PART ? tile_all % splits : 0;
  const int tile = PART ? tile_all / splits : tile_all;
  const int seq = tile / nqb, q0 = (tile % nqb) * QB + wq * 16;
  const bool live = q0 < n;  // uniform over the wave
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

  // K staging: slot f = tid + 256 i is key f/16, float4 f%16 (16 lanes fill
  // one key row).  V staging: slot f -> w' = f/64, key 16 (w' % 4) + (l & 15),
  // float4 column (l >> 4) + 4 (w' / 4); one wave instruction covers 16 keys
  // x 4 columns.
  const int skey = tid >> 4, sd = 4 * (tid & 15);
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
    k_off[i] = 4u * static_cast<uint32_t>((skey + (kThreads / 16) * i) * HD + sd);
    const int w2 = wq + QG * i;
    v_off[i] = 4u * static_cast<uint32_t>((16 * (w2 & 3) + (lane & 15)) * HD +
                                          4 * ((lane >> 4) + 4 * (w2 >> 2)));
  }

  const int nkb = (n + KB - 1) / KB;
  const int kb_begin = PART ? split * nkb / splits : 0;
  const int kb_end = PART ? (split + 1) * nkb / splits : nkb;
  for (int kb = kb_begin; kb < kb_end; ++kb) {
    const int k0 = kb * KB;
    f32x4 kr[kPer], vr[kPer];
    if (k0 + KB <= n) {
      const uint32_t blk = 4u * (static_cast<uint32_t>(seq) * static_cast<uint32_t>(n) +
                                 static_cast<uint32_t>(k0)) * HD;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const float4 a = vkd::buffer_load4(k_rsrc, k_off[i], blk);
        const float4 b = vkd::buffer_load4(v_rsrc, v_off[i], blk);
        kr[i] = f32x4{a.x, a.y, a.z, a.w};
        vr[i] = f32x4{b.x, b.y, b.z, b.w};
      }
    } else {  // the last, partial block: keys past n read key n - 1
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int key = k0 + skey + (kThreads / 16) * i;
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
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      *reinterpret_cast<f32x4*>(Ks + (skey + (kThreads / 16) * i) * PITCH + sd) = kr[i];
      const int w2 = wq + QG * i;
      const int key = 16 * (w2 & 3) + (lane & 15);
      const int d = 4 * ((lane >> 4) + 4 * (w2 >> 2));
#pragma unroll
      for (int c = 0; c < 4; ++c) Vt[(d + c) * PITCH + key] = vr[i][c];
    }
    __syncthreads();
    // a wave whose 16 queries all lie past n only stages (the last query tile
    // of a sequence whose length is not a multiple of 64)
    if (!live) continue;

    // S^T tiles: s[t][r] = score of query q0 + c16 with key k0 + 16t + 4g + r
    // (K fragments of tile t + 1 are read while tile t's 16 MFMAs run)
    f32x4 s[4], ka[2][4];
#pragma unroll
    for (int bd = 0; bd < 4; ++bd)
      ka[0][bd] = *reinterpret_cast<const f32x4*>(karow + 16 * bd);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < 3) {
#pragma unroll
        for (int bd = 0; bd < 4; ++bd)
          ka[(t + 1) & 1][bd] =
              *reinterpret_cast<const f32x4*>(karow + (t + 1) * 16 * PITCH + 16 * bd);
      }
      __builtin_amdgcn_sched_barrier(0);
      s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int bd = 0; bd < 4; ++bd)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[t & 1][bd][j], qf[bd][j], s[t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
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
    // (V^T fragments of column tile dt + 1 are read while dt's MFMAs run)
    f32x4 vb[2][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) vb[0][t] = *reinterpret_cast<const f32x4*>(vtrow + 16 * t);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      if (dt < 3) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          vb[(dt + 1) & 1][t] =
              *reinterpret_cast<const f32x4*>(vtrow + (dt + 1) * 16 * PITCH + 16 * t);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(s[t][j], vb[dt & 1][t][j], o[dt], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if constexpr (PART) {
    // this split's O (rescaled to its own running max), max and sum
    const size_t rows = static_cast<size_t>(sequences) * n;
    float* po = part + (static_cast<size_t>(split) * rows + static_cast<size_t>(seq) * n) * HD;
    float* pml = part + static_cast<size_t>(splits) * rows * HD +
                 (static_cast<size_t>(split) * rows + static_cast<size_t>(seq) * n) * 2;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qi = q0 + 4 * g + r;
      if (qi < n) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) po[static_cast<size_t>(qi) * HD + 16 * dt + c16] = o[dt][r];
      }
    }
    if (g == 0 && q0 + c16 < n)
      *reinterpret_cast<float2*>(pml + 2 * static_cast<size_t>(q0 + c16)) =
          make_float2(m_run, l_run);
    return;
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

// Combines the key splits of the PART form: 16 threads per query row, one
// float4 of O each; the splits' weights 2^(m_s - m) and sums are taken in
// split order.  SP (the split count) is a template parameter so that every
// load of a row is issued before the first is used: with a run-time count
// each loop iteration waited for its own loads.
template <int SP>
__global__ __launch_bounds__(256) void attention_merge_kernel(const float* __restrict__ part,
                                                              float* __restrict__ out,
                                                              long long rows) {
  const long long idx = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  const long long row = idx >> 4;
  const int c4 = static_cast<int>(idx & 15);
  if (row >= rows) return;
  const float* ml = part + static_cast<size_t>(SP) * rows * HD;
  float2 st[SP];
  f32x4 po[SP];
#pragma unroll
  for (int sp = 0; sp < SP; ++sp) {
    st[sp] = *reinterpret_cast<const float2*>(ml + 2 * (sp * rows + row));
    po[sp] = *reinterpret_cast<const f32x4*>(part + (sp * rows + row) * HD + 4 * c4);
  }
  float m = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < SP; ++sp) m = fmaxf(m, st[sp].x);
  float l = 0.0f;
  f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < SP; ++sp) {
    const float w = __builtin_amdgcn_exp2f(st[sp].x - m);
    l = l + st[sp].y * w;
    o = o + po[sp] * w;
  }
  *reinterpret_cast<f32x4*>(out + row * HD + 4 * c4) =
      f32x4{o[0] / l, o[1] / l, o[2] / l, o[3] / l};
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
  // 64-query tiles.  When they give fewer than two workgroups per CU (one
  // ViT-B image: 168 tiles), each tile's key blocks are split over about two
  // workgroups per CU (at least two key blocks per split) and a second pass
  // merges the partial results.  Fuller grids split only where the last
  // round of workgroups leaves CUs unevenly loaded and a cost model puts the
  // split at least 1% below the unsplit launch: the busiest CU runs
  // ceil(tiles * s / CUs) workgroups of up to ceil(key blocks / s) blocks
  // (about 2.2 us per block of one of the four workgroups a CU holds), and a
  // split adds its partial results' traffic (s slices of rows x 66 floats
  // written and read back) and the merge pass (about 3 us).  ViT-L at 3,458
  // rows (880 tiles of 55 blocks, 3.4 per CU): 2 splits (425 us; unsplit
  // 464); the 12-view global layer (1,956 tiles of 163 blocks, model 1.6%
  // below unsplit): 3 splits (2,486 us; unsplit 2,582, 4 splits 2,528); the
  // 12-view local layers (14 blocks per tile) stay unsplit (260 us; 3
  // splits 288).
  const int cus = rt->cu_count > 0 ? rt->cu_count : 256;
  const long long tiles64 = static_cast<long long>(sequences) * ((n + 63) / 64);
  const int nkb = static_cast<int>((n + KB - 1) / KB);
  int splits = 1;
  if (tiles64 < 2LL * cus) {
    splits = static_cast<int>((2.0 * cus) / static_cast<double>(tiles64) + 0.5);
    if (splits > nkb / 2) splits = nkb / 2;
    if (splits > 8) splits = 8;
    if (splits < 1) splits = 1;
  } else {
    constexpr double kBlockUs = 2.2, kBytesPerUs = 5.5e6, kMergeUs = 3.0;
    const double row_bytes = 4.0 * (HD + 2) * static_cast<double>(sequences * n);
    const double unsplit = kBlockUs * static_cast<double>((tiles64 + cus - 1) / cus * nkb);
    double best = unsplit;
    for (int sp = 2; sp <= 8 && 2 * sp <= nkb; ++sp) {
      const long long load = (tiles64 * sp + cus - 1) / cus * ((nkb + sp - 1) / sp);
      const double us = kBlockUs * static_cast<double>(load) +
                        2.0 * sp * row_bytes / kBytesPerUs + kMergeUs;
      if (us < best && us < 0.99 * unsplit) {
        best = us;
        splits = sp;
      }
    }
  }
  const long long blocks = tiles64 * splits;
  VK_UNSUPPORTED_IF(blocks > 0x7fffffffLL, "attention: %lld workgroups", blocks);
  const auto* Q = static_cast<const float*>(q->ptr);
  const auto* K = static_cast<const float*>(k->ptr);
  const auto* V = static_cast<const float*>(v->ptr);
  auto* O = static_cast<float*>(out->ptr);
  const int S = static_cast<int>(sequences), N = static_cast<int>(n);
  if (splits > 1) {
    const size_t rows = sequences * n;
    VK_TRY(vk::ensure_work(rt, static_cast<size_t>(splits) * rows * (HD + 2), "attention"));
    float* part = rt->work;
    hipLaunchKernelGGL((attention_kernel<true, 4>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, rt->stream, Q, K, V, O, S, N, splits, part);
    VK_TRY(vk::check_launch("attention_kernel"));
    const long long threads = static_cast<long long>(rows) * 16;
    const dim3 mgrid(static_cast<unsigned>((threads + 255) / 256));
    const long long R = static_cast<long long>(rows);
    switch (splits) {
#define VK_MERGE_CASE(SPN)                                                                     \
  case SPN:                                                                                    \
    hipLaunchKernelGGL(attention_merge_kernel<SPN>, mgrid, dim3(256), 0, rt->stream, part, O, R); \
    break;
      VK_MERGE_CASE(2) VK_MERGE_CASE(3) VK_MERGE_CASE(4) VK_MERGE_CASE(5)
      VK_MERGE_CASE(6) VK_MERGE_CASE(7) VK_MERGE_CASE(8)
#undef VK_MERGE_CASE
      default:
        return vk::set_error(VK_ERR_INVALID, "attention: %d key splits", splits);
    }
    return vk::check_launch("attention_merge_kernel");
  }
  if (n <= kWideTileMaxN) {
    // unsplit short sequences: 128-query workgroups (eight waves), half the
    // K/V staging per query
    const long long t128 = static_cast<long long>(sequences) * ((n + 127) / 128);
    hipLaunchKernelGGL((attention_kernel<false, 8>), dim3(static_cast<unsigned>(t128)), dim3(512),
                       0, rt->stream, Q, K, V, O, S, N, 1, nullptr);
    return vk::check_launch("attention_kernel");
  }
  hipLaunchKernelGGL((attention_kernel<false, 4>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     rt->stream, Q, K, V, O, S, N, 1, nullptr);
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
