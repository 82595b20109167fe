// The F32 linear on wide tiles for gfx950: the block projections (QKV, proj,
// FC1, FC2) with their per-token epilogues (bias, LayerScale, GELU,
// residual add) fused into the store.
//
// A workgroup owns a TM x TN output tile (128 x 128 with 512 threads, or
// 64 x 128 / 64 x 64 with 256 for grids of few rows); wave w computes rows
// 32 (w/2) .. +32 and columns TN/2 (w%2) .. +TN/2 as 2 x TN/32 tiles of
// v_mfma_f32_16x16x4_f32 (F32 in, F32 accumulate): for 128-wide tiles 32
// MFMAs per 16-wide k-block from six 128-bit LDS reads.  K is staged through
// LDS in chunks of 64 by raw buffer loads (a lane's fixed offset plus the
// chunk's uniform offset), A as [m][k] and B as [n][k] rows with a pitch of
// 68 floats (4 x odd: the 16 rows of a fragment read start on 16 distinct
// 4-bank groups, and the staging stores of 16 lanes fill one row without
// conflicts).  The 70 KB of LDS of a 128 x 128 tile leaves room for a
// second workgroup on the CU, which computes while the first stages a chunk
// or runs its epilogue.  Grids of few tiles split K over several workgroups
// per tile (split-K: partial sums in the runtime's work buffer, added in
// split order by splitk_reduce_kernel).
//
// Fragment order as in the patch embedding: in block b, lane group g holds
// k = 16b + 4g + j in component j of a 128-bit read and MFMA step j uses
// component j, so four steps cover the block's 16 k once.
//
// Head-major layouts (head_dim 64): the QKV projection can store Q | K | V
// straight into three [heads, rows, 64] tensors (the split the attention
// kernels need), and the output projection can read its input from the
// head-major attention output; tiles start on 64-column head boundaries,
// and a float4 of A never crosses a head.  Both are pure address changes:
// the results are the bits of the linear plus the separate permutation.
//
// Q/K-norm + RoPE in the QKV epilogue (QKN != 0): after the last chunk the
// waves holding Q or K heads write their values (acc + b) to LDS and read
// them back as the Q/K kernel holds a row -- 16 lanes per 64-wide row, one
// float4 each -- and apply the same row transform (vkq::qk_row_transform)
// before storing the row head-major.  The values and the code path are
// those of the separate pass, so the bits are too.
//
// Traffic: a 128 x 128 tile moves (128 + 128) x 4 bytes of operands per k for
// 2 x 128 x 128 FLOP, 0.031 byte per FLOP from L2 (the 48 x 64 tiles of the
// narrow kernel need 0.073).  Tiles are numbered XCD-major (xcd_tile), so
// the workgroups of one XCD share weight columns in that XCD's L2.
#include "common.h"
#include "qk_rows.h"

namespace {

using vk::LinearArgs;
using namespace vk::linear_epilogue;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Tiles are TM x TN (TM 128 or 64, TN 128 or 64, template parameters); a
// wave owns a 32-row x TN/2-column strip.
constexpr int KC = 64;
constexpr int PITCH = 68;
static_assert(PITCH % 4 == 0 && (PITCH / 4) % 2 == 1 && PITCH >= KC, "pitch 4 x odd");

// Threads of a TM x 128 tile: one wave per 32 x 64 strip.
constexpr int threads_for(int tm) { return 4 * tm; }

enum Layout { kPlain = 0, kQkvHnd = 1, kAHnd = 2 };

// One output value: v = acc + b (then * ls), each step rounded, through the
// epilogue.
template <int EPI>
__device__ __forceinline__ float epi_value(const LinearArgs& g, float acc, float bias, float ls,
                                           float old) {
  float v = acc + bias;
  if (g.ls) v = v * ls;
  if (EPI == kLinGelu) return vkd::gelu1<0>(v);
  if (EPI == kLinGeluErf) return vkd::gelu1<1>(v);
  if (EPI == kLinResidual) return old + v;
  return v;
}

// Address of output element (row, col) in the output layout.
template <int LAY>
__device__ __forceinline__ float* out_addr(const LinearArgs& g, int row, int col) {
  if constexpr (LAY == kQkvHnd) {
    const int embed = g.N / 3;
    const int which = col >= embed ? (col >= 2 * embed ? 2 : 1) : 0;
    const int c = col - which * embed;
    float* base = which == 0 ? g.q_out : (which == 1 ? g.k_out : g.v_out);
    return base + (static_cast<size_t>(c >> 6) * g.M + row) * 64 + (c & 63);
  } else {
    return g.out + static_cast<size_t>(row) * g.N + col;
  }
}

template <int EPI, int LAY>
__device__ __forceinline__ void store_out(const LinearArgs& g, int row, int col, float acc,
                                          float bias, float ls, float old) {
  *out_addr<LAY>(g, row, col) = epi_value<EPI>(g, acc, bias, ls, old);
}

// QKN: 0 none; 1 / 2 Q/K LayerNorm (f32 / f16 parameters) + RoPE; 3 RoPE.
template <int QKN>
struct QknTraits;
template <>
struct QknTraits<1> {
  typedef float PT;
  static constexpr bool kNorm = true;
};
template <>
struct QknTraits<2> {
  typedef uint16_t PT;
  static constexpr bool kNorm = true;
};
template <>
struct QknTraits<3> {
  typedef float PT;
  static constexpr bool kNorm = false;
};

// Q/K-norm + RoPE of one 64-wide head row held as one float4 per lane of a
// 16-lane group (lane l: columns 4l..4l+3), for token `row` (clamped to a
// valid token; rows past M are computed and not stored).
template <int QKN>
__device__ __forceinline__ float4 qk_head_row(const LinearArgs& g, float4 v, int l, bool is_k,
                                              int row) {
  typedef typename QknTraits<QKN>::PT PT;
  const int rowc = row < g.M ? row : g.M - 1;
  float py, px;
  vkq::grid_position(vkd::fmod_(static_cast<uint32_t>(rowc), g.qkn.tpv), g.qkn.n_special,
                     g.qkn.global, g.qkn.gw, &py, &px);
  const PT* gm = static_cast<const PT*>(is_k ? g.qkn.kg : g.qkn.qg);
  const PT* bt = static_cast<const PT*>(is_k ? g.qkn.kb : g.qkn.qb);
  // the pairing is uniform over the launch: a scalar branch
  if (g.qkn.interleaved)
    return vkq::qk_row_transform<PT, QknTraits<QKN>::kNorm, vkq::kPosGrid, vkq::kInterleaved>(
        v, l, gm, bt, py, px, g.qkn.table, g.qkn.table_max, g.qkn.eps);
  return vkq::qk_row_transform<PT, QknTraits<QKN>::kNorm, vkq::kPosGrid, vkq::kRotateHalf>(
      v, l, gm, bt, py, px, g.qkn.table, g.qkn.table_max, g.qkn.eps);
}

// Most split-K slices a sum pass reads (the plan's limit, checked where it
// is defined).  The sum passes are instantiated for split-count buckets SPB
// of 2, 4 and 8 (split_bucket).
constexpr int kMaxSplits = 8;
constexpr int split_bucket(int splits) { return splits <= 2 ? 2 : (splits <= 4 ? 4 : 8); }

// The NV float4 at offsets e[i] of every split's slice (splits <= SPB),
// summed in split order.  All SPB x NV loads are issued before the first
// addition (a run-time loop over the splits waited for each iteration's
// load); slots past `splits` re-read the last slice and are not added.
template <int NV, int SPB>
__device__ __forceinline__ void split_sums(const float* __restrict__ partial, size_t mn,
                                           const size_t (&e)[NV], int splits, f32x4 (&acc)[NV]) {
  f32x4 p[NV][SPB];
#pragma unroll
  for (int sp = 0; sp < SPB; ++sp) {
    const size_t slice = static_cast<size_t>(sp < splits ? sp : splits - 1) * mn;
#pragma unroll
    for (int i = 0; i < NV; ++i) p[i][sp] = *reinterpret_cast<const f32x4*>(partial + slice + e[i]);
  }
  // all loads issued before the first addition (the scheduler would
  // otherwise roll them behind the additions, one round trip each)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    acc[i] = p[i][0];
#pragma unroll
    for (int sp = 1; sp < SPB; ++sp)
      if (sp < splits) acc[i] = acc[i] + p[i][sp];
  }
}

// KG: k groups.  With KG = 2 (64 x 64 tiles only) the workgroup has twice the
// waves: group 1 runs the second half of every chunk's 16-blocks on the same
// strips as group 0, and adds its sums to group 0's through LDS after the
// last chunk (group 0's + group 1's, in that order).  A grid of few tiles
// (one image: two workgroups per CU) then keeps four waves per SIMD instead
// of two.
//
// PF: the next chunk's loads are issued before this chunk's MFMAs and land in
// registers meanwhile.  It costs 2 (64 x 64) or 8 (128 x 128) more float4 per
// thread, so the 128 x 128 tile takes it only where a launch has at most one
// workgroup per CU (nothing else on the CU covers the load latency there,
// and the lower occupancy costs nothing).
template <int EPI, int LAY, int QKN, int TM, int TN, int KG = 1, bool PF = (KG == 2)>
__global__ __launch_bounds__(threads_for(TM) * KG,
                             TM == 128 ? (PF ? 1 : 2) : (TN == 128 ? 3 : (KG == 2 ? 3 : 4)))
    void linear_wide_kernel(LinearArgs g) {
  constexpr int WN = TN / 2;  // columns of a wave's strip
  constexpr int NU = WN / 16; // 16-column MFMA tiles per strip
  static_assert(TN == 128 || TN == 64, "tile widths 128 and 64");
  static_assert(KG == 1 || (KG == 2 && TM == 64 && TN == 64), "k groups: 64 x 64 tiles");
  constexpr int kThreads = threads_for(TM) * KG;
  constexpr int kGroupWaves = threads_for(TM) / 64;  // waves of one k group
  constexpr int kVA = TM * KC / 4 / kThreads;  // float4 of A per thread a chunk: 4
  constexpr int kVB = TN * KC / 4 / kThreads;  // float4 of B: TN / TM x 4
  static_assert(TM == 128 || TM == 64, "tile heights 128 and 64");
  static_assert(kVA * kThreads * 4 == TM * KC && kVB * kThreads * 4 == TN * KC, "slots");
  __shared__ __align__(16) float As[TM * PITCH];
  __shared__ __align__(16) float Bs[TN * PITCH];

  const int tid = threadIdx.x;
  __builtin_assume(tid < kThreads);
  const int wave = tid >> 6, lane = tid & 63;
  const int kh = KG == 1 ? 0 : wave / kGroupWaves;  // k group
  const bool lead = kh == 0;                          // holds the tile's sums at the end
  const int wl = wave % kGroupWaves;                  // wave within the k group
  const int wm = wl >> 1, wn = wl & 1;
  const int gmt = (g.M + TM - 1) / TM;
  const int gnt = (g.N + TN - 1) / TN;
  const int tile = vkd::xcd_tile(blockIdx.x, gridDim.x);
  const int m0 = (tile % gmt) * TM;
  const int rest = tile / gmt;
  const int n0 = (rest % gnt) * TN;
  const int split = rest / gnt;
  const int nch = (g.K + KC - 1) / KC;
  const int c_begin = split * nch / g.splits, c_end = (split + 1) * nch / g.splits;

  f32x4 acc[2][NU];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < NU; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kq = 4 * (lane >> 4) + kh * (KC / KG);
  const float* arow = As + (wm * 32 + (lane & 15)) * PITCH + kq;
  const float* brow = Bs + (wn * WN + (lane & 15)) * PITCH + kq;

  // Staging slot i of a thread: row r_i = tid/16 + (threads/16) i of the A
  // (or B) tile, float4 column c = 4 (tid % 16) of the chunk (a wave reads
  // four 256-byte row segments).  Rows past M or N read a clamped, valid
  // row: row i of A only reaches output row i and row j of B output column
  // j, so their values never reach a stored output.
  const int c_ld = 4 * (tid & 15);
  uint32_t a_off[kVA], b_off[kVB];  // byte offsets, the same for every chunk
  auto slot_row = [&](int i) { return (tid >> 4) + (kThreads / 16) * i; };
#pragma unroll
  for (int i = 0; i < kVA; ++i) {
    const int gm = m0 + slot_row(i);
    const uint32_t cm = static_cast<uint32_t>(gm < g.M ? gm : g.M - 1);
    a_off[i] = 4u * (LAY == kAHnd ? cm * 64u + c_ld : cm * static_cast<uint32_t>(g.K) + c_ld);
  }
#pragma unroll
  for (int i = 0; i < kVB; ++i) {
    const int gn = n0 + slot_row(i);
    const uint32_t cn = static_cast<uint32_t>(gn < g.N ? gn : g.N - 1);
    b_off[i] = 4u * (cn * static_cast<uint32_t>(g.Kp) + c_ld);
  }

  auto mma_chunk = [&]() {
#pragma unroll
    for (int b = 0; b < KC / 16 / KG; ++b) {
      f32x4 a[2], w[NU];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        a[t] = *reinterpret_cast<const f32x4*>(arow + t * 16 * PITCH + 16 * b);
#pragma unroll
      for (int u = 0; u < NU; ++u)
        w[u] = *reinterpret_cast<const f32x4*>(brow + u * 16 * PITCH + 16 * b);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < NU; ++u)
            acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][j], w[u][j], acc[t][u], 0, 0, 0);
    }
  };

  // Whole chunks (k0 + 64 <= K): buffer loads of the lane's fixed offset
  // plus the chunk's uniform offset, with no per-chunk address arithmetic or
  // selects.
  const int full = g.K / KC;
  const int c_full = c_end < full ? c_end : full;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      vkd::buffer_rsrc(g.x, 4u * static_cast<uint32_t>(g.M) * static_cast<uint32_t>(g.K));
  const __amdgpu_buffer_rsrc_t b_rsrc =
      vkd::buffer_rsrc(g.wnk, 4u * static_cast<uint32_t>(g.N) * static_cast<uint32_t>(g.Kp));
  auto load_chunk = [&](int ch, float4 (&ra)[kVA], float4 (&rb)[kVB]) {
    const uint32_t k0 = static_cast<uint32_t>(ch) * KC;
    const uint32_t a_chunk =
        4u * (LAY == kAHnd ? static_cast<uint32_t>(ch) * static_cast<uint32_t>(g.M) * 64u : k0);
#pragma unroll
    for (int i = 0; i < kVA; ++i) ra[i] = vkd::buffer_load4(a_rsrc, a_off[i], a_chunk);
#pragma unroll
    for (int i = 0; i < kVB; ++i) rb[i] = vkd::buffer_load4(b_rsrc, b_off[i], 4u * k0);
  };
  auto store_chunk = [&](const float4 (&ra)[kVA], const float4 (&rb)[kVB]) {
#pragma unroll
    for (int i = 0; i < kVA; ++i)
      *reinterpret_cast<float4*>(As + slot_row(i) * PITCH + c_ld) = ra[i];
#pragma unroll
    for (int i = 0; i < kVB; ++i)
      *reinterpret_cast<float4*>(Bs + slot_row(i) * PITCH + c_ld) = rb[i];
  };
  if constexpr (PF) {
    float4 ra[kVA], rb[kVB];
    if (c_begin < c_full) load_chunk(c_begin, ra, rb);
    for (int ch = c_begin; ch < c_full; ++ch) {
      __syncthreads();  // every wave is done reading the previous chunk
      store_chunk(ra, rb);
      __syncthreads();
      if (ch + 1 < c_full) load_chunk(ch + 1, ra, rb);
      mma_chunk();
    }
  } else {
    for (int ch = c_begin; ch < c_full; ++ch) {
      float4 ra[kVA], rb[kVB];
      load_chunk(ch, ra, rb);
      __syncthreads();  // every wave is done reading the previous chunk
      store_chunk(ra, rb);
      __syncthreads();
      mma_chunk();
    }
  }

  // The last, partial chunk (K % 64 != 0): k past K reads a clamped address
  // and stores zeros (A past K, B past its zero padding Kp).
  if (c_end > full && c_begin <= full) {
    const int k0 = full * KC;
    const int gk = k0 + c_ld;
    const bool ka = gk < g.K, kb = gk < g.Kp;
    const int ck = ka ? gk : g.K - 4;
    const int ckb = kb ? gk : g.Kp - 4;
    float4 ra[kVA], rb[kVB];
#pragma unroll
    for (int i = 0; i < kVA; ++i) {
      const int gm = m0 + slot_row(i);
      const int cm = gm < g.M ? gm : g.M - 1;
      const size_t ia = LAY == kAHnd
                            ? (static_cast<size_t>(ck >> 6) * g.M + cm) * 64 + (ck & 63)
                            : static_cast<size_t>(cm) * g.K + ck;
      ra[i] = *reinterpret_cast<const float4*>(g.x + ia);
    }
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      const int gn = n0 + slot_row(i);
      const int cn = gn < g.N ? gn : g.N - 1;
      rb[i] = *reinterpret_cast<const float4*>(g.wnk + static_cast<size_t>(cn) * g.Kp + ckb);
    }
    __syncthreads();
    // component selects: a select of whole float4 values becomes a select
    // of their addresses, which puts the staging arrays in scratch memory
#pragma unroll
    for (int i = 0; i < kVA; ++i)
      *reinterpret_cast<float4*>(As + slot_row(i) * PITCH + c_ld) =
          make_float4(ka ? ra[i].x : 0.f, ka ? ra[i].y : 0.f, ka ? ra[i].z : 0.f,
                      ka ? ra[i].w : 0.f);
#pragma unroll
    for (int i = 0; i < kVB; ++i)
      *reinterpret_cast<float4*>(Bs + slot_row(i) * PITCH + c_ld) =
          make_float4(kb ? rb[i].x : 0.f, kb ? rb[i].y : 0.f, kb ? rb[i].z : 0.f,
                      kb ? rb[i].w : 0.f);
    __syncthreads();
    mma_chunk();
  }

  // k groups: the two groups' sums meet through LDS (As, free after the
  // last chunk), one f32x4 per lane and MFMA tile, lane-contiguous.  For the
  // plain epilogue each group finishes one of the strip's two 16-row halves
  // (half kh: it hands the other half's sums over and takes this half's),
  // so all eight waves run the epilogue; the Q/K epilogue and split-K take
  // the whole sums in group 0.  Either way a sum is group 0's + group 1's.
  const bool half_epi = KG == 2 && QKN == 0 && g.splits == 1;
  if constexpr (KG == 2) {
    static_assert(kGroupWaves * 2 * NU * 256 <= TM * PITCH, "k-group sums fit in As");
    float* red = As + wl * (2 * NU * 256) + 4 * lane;
    __syncthreads();  // every wave is done reading the last chunk's operands
    if (half_epi) {
      // constant indices in both branches (kh is uniform over the wave): a
      // register array indexed by a run-time value would live in scratch
      if (lead) {
#pragma unroll
        for (int u = 0; u < NU; ++u)
          *reinterpret_cast<f32x4*>(red + (NU + u) * 256) = acc[1][u];
      } else {
#pragma unroll
        for (int u = 0; u < NU; ++u) *reinterpret_cast<f32x4*>(red + u * 256) = acc[0][u];
      }
      __syncthreads();
      if (lead) {
#pragma unroll
        for (int u = 0; u < NU; ++u)
          acc[0][u] = acc[0][u] + *reinterpret_cast<const f32x4*>(red + u * 256);
      } else {
#pragma unroll
        for (int u = 0; u < NU; ++u)
          acc[1][u] = *reinterpret_cast<const f32x4*>(red + (NU + u) * 256) + acc[1][u];
      }
    } else {
      if (!lead) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < NU; ++u)
            *reinterpret_cast<f32x4*>(red + (t * NU + u) * 256) = acc[t][u];
      }
      __syncthreads();
      if (lead) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < NU; ++u)
            acc[t][u] = acc[t][u] + *reinterpret_cast<const f32x4*>(red + (t * NU + u) * 256);
      }
    }
  }

  // split-K: raw sums to this split's slice of the partial buffer
  if (g.splits > 1) {
    if (lead) {
      float* part = g.partial + static_cast<size_t>(split) * g.M * g.N;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm * 32 + t * 16 + 4 * (lane >> 4) + r;
            const int col = n0 + wn * WN + u * 16 + (lane & 15);
            if (row < g.M && col < g.N) part[static_cast<size_t>(row) * g.N + col] = acc[t][u][r];
          }
    }
    return;
  }

  // epilogue: lane holds D[4*(lane/16) + r][lane%16] of each 16x16 tile.
  // Parameters and (for the residual) the old values are all loaded, on
  // clamped indices, before the first store.
  float bias[NU], ls[NU];
  if constexpr (QKN != 0) {
    static_assert(LAY == kQkvHnd && EPI == kLinStore, "Q/K epilogue of the QKV projection");
    // One head of Q, K or V: a 128-wide tile gives each wave a head of its
    // own (its 32 x 64 strip); a 64-wide tile is one head, whose 32-row
    // halves waves wn 0 and 1 hold 32 columns each of and then transform 16
    // rows each.
    // With k groups, the eight waves transform 8 rows each.
    const int col0 = TN == 128 ? n0 + wn * 64 : n0;
    const int cw0 = TN == 128 ? 0 : wn * 32;  // the wave's first column in the head
    constexpr int kRowsPerGroup = TN == 128 ? 8 : 4 / KG;
    const int rr0 = TN == 128 ? 0 : (wn * KG + kh) * (16 / KG);
    const int embed = g.N / 3;
    const int which = col0 < g.N ? col0 / embed : 2;
    const int g4 = lane >> 4, c16 = lane & 15;
    // 32-row staging regions: TN 128, one per wave (the A tile holds TM / 32
    // of them, the B tile the rest); TN 64, one per row half wm, in the A tile
    float* xs = TN == 64 ? As + wm * 32 * PITCH
                         : (wave < TM / 32 ? As + wave * 32 * PITCH
                                           : Bs + (wave - TM / 32) * 32 * PITCH);
    __syncthreads();  // every wave is done with the last chunk's operands
    if (which < 2 && lead) {
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const float b = g.bias[col0 + cw0 + u * 16 + c16];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            xs[(t * 16 + 4 * g4 + r) * PITCH + cw0 + u * 16 + c16] = acc[t][u][r] + b;
      }
    }
    __syncthreads();
    if (which < 2) {
      float* dst = (which == 0 ? g.q_out : g.k_out) +
                   static_cast<size_t>((col0 - which * embed) >> 6) * g.M * 64;
#pragma unroll 2
      for (int i = 0; i < kRowsPerGroup; ++i) {
        const int rr = rr0 + g4 * kRowsPerGroup + i;
        const int row = m0 + wm * 32 + rr;
        const float4 v = *reinterpret_cast<const float4*>(xs + rr * PITCH + 4 * c16);
        const float4 o = qk_head_row<QKN>(g, v, c16, which == 1, row);
        if (row < g.M) *reinterpret_cast<float4*>(dst + static_cast<size_t>(row) * 64 + 4 * c16) = o;
      }
      return;
    }
  }
  if (!lead && !half_epi) return;
  // Per 16-column strip u: bias, LayerScale and the address of the column
  // at row 0 (row r adds r x the row stride), computed once; a tile inside
  // the matrix stores without bounds checks.
  const bool interior = m0 + TM <= g.M && n0 + TN <= g.N;
  const size_t rs = LAY == kQkvHnd ? 64 : static_cast<size_t>(g.N);
  float* cptr[NU];
  bool cok[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int col = n0 + wn * WN + u * 16 + (lane & 15);
    cok[u] = col < g.N;
    const int cc = cok[u] ? col : g.N - 1;
    bias[u] = g.bias[cc];
    ls[u] = g.ls ? g.ls[cc] : 1.0f;
    cptr[u] = out_addr<LAY>(g, 0, cc);
  }
  float old[2][NU][4];
  if constexpr (EPI == kLinResidual) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (half_epi && t != kh) continue;
        const int row = m0 + wm * 32 + t * 16 + 4 * (lane >> 4) + r;
        const size_t cr = static_cast<size_t>(row < g.M ? row : g.M - 1);
#pragma unroll
        for (int u = 0; u < NU; ++u) old[t][u][r] = cptr[u][cr * rs];
      }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (half_epi && t != kh) continue;
      const int row = m0 + wm * 32 + t * 16 + 4 * (lane >> 4) + r;
      const bool rok = row < g.M;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const float val = epi_value<EPI>(g, acc[t][u][r], bias[u], ls[u],
                                         EPI == kLinResidual ? old[t][u][r] : 0.0f);
        if (interior || (rok && cok[u])) cptr[u][static_cast<size_t>(row) * rs] = val;
      }
    }
}

// Second pass of a split-K linear: one thread per 4 consecutive outputs of a
// row; the splits' partial sums are added in split order, then the epilogue
// of the single-pass kernel is applied.
template <int EPI, int LAY, int QKN, int SPB>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(LinearArgs g) {
  const long long i4 = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  const long long mn = static_cast<long long>(g.M) * g.N;
  if (i4 * 4 >= mn) return;  // whole 16-lane groups (M*N/4 is a multiple of 16 here)
  const size_t e = static_cast<size_t>(i4) * 4;
  const int row = static_cast<int>(e / g.N), col = static_cast<int>(e % g.N);
  const size_t es[1] = {e};
  // the epilogue's loads before the partial sums' and every store: a load
  // after a store to `out` would wait for it (the compiler cannot tell them
  // apart)
  const float4 bias = *reinterpret_cast<const float4*>(g.bias + col);
  const float4 ls = g.ls ? *reinterpret_cast<const float4*>(g.ls + col)
                         : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
  f32x4 old = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (EPI == kLinResidual) old = *reinterpret_cast<const f32x4*>(g.out + e);
  f32x4 accs[1];
  split_sums<1, SPB>(g.partial, static_cast<size_t>(mn), es, g.splits, accs);
  const f32x4 acc = accs[0];
  if constexpr (QKN != 0) {
    // 16 consecutive threads hold one 64-wide head row of one token
    const int embed = g.N / 3;
    const int which = col / embed;
    if (which < 2) {
      const int c = col - which * embed;
      float4 v;
      v.x = acc[0] + bias.x;
      v.y = acc[1] + bias.y;
      v.z = acc[2] + bias.z;
      v.w = acc[3] + bias.w;
      const float4 o = qk_head_row<QKN>(g, v, threadIdx.x & 15, which == 1, row);
      float* dst = (which == 0 ? g.q_out : g.k_out) +
                   (static_cast<size_t>(c >> 6) * g.M + row) * 64 + (c & 63);
      *reinterpret_cast<float4*>(dst) = o;
      return;
    }
  }
  const float bj[4] = {bias.x, bias.y, bias.z, bias.w};
  const float lj[4] = {ls.x, ls.y, ls.z, ls.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) store_out<EPI, LAY>(g, row, col + j, acc[j], bj[j], lj[j], old[j]);
}

// Sum pass of a split-K linear with the residual epilogue, followed by the
// LayerNorm of the finished rows: one wave per row, NV float4 per lane
// (column float4 lane + 64 i).  The partial sums are added in split order
// and the epilogue applied as in splitk_reduce_kernel, the row statistics
// and the normalisation are vkd::row_mean_inv / vkd::ln_apply4 over the same
// lane layout as layernorm_rows: the bits of the two separate passes.
template <int NV, typename PT, int SPB>
__global__ __launch_bounds__(64) void splitk_residual_ln_kernel(LinearArgs g) {
  const int lane = threadIdx.x;
  const size_t row = blockIdx.x;
  const size_t mn = static_cast<size_t>(g.M) * g.N;
  const size_t rb = row * g.N;
  size_t es[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) es[i] = rb + 4 * static_cast<size_t>(lane + 64 * i);
  // Every load of the row -- the residual, bias, LayerScale and LayerNorm
  // parameters, then the partial sums -- is issued before the first store:
  // the compiler cannot tell the stores to `out` from the parameter
  // pointers, so a load placed after a store would wait for it (one memory
  // round trip per float4 column of the lane).
  const PT* gm = static_cast<const PT*>(g.ln_gamma);
  const PT* bt = static_cast<const PT*>(g.ln_beta);
  f32x4 old[NV];
  float4 bias[NV], lsv[NV], lg[NV], lb[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c4 = lane + 64 * i;
    old[i] = *reinterpret_cast<const f32x4*>(g.out + es[i]);
    bias[i] = *reinterpret_cast<const float4*>(g.bias + 4 * c4);
    lsv[i] = g.ls ? *reinterpret_cast<const float4*>(g.ls + 4 * c4)
                  : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    lg[i] = vkd::Param<PT>::load4(gm, c4);
    lb[i] = vkd::Param<PT>::load4(bt, c4);
  }
  f32x4 accs[NV];
  split_sums<NV, SPB>(g.partial, mn, es, g.splits, accs);
  float4 vv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const f32x4 acc = accs[i];
    float4 v;
    v.x = epi_value<kLinResidual>(g, acc[0], bias[i].x, lsv[i].x, old[i][0]);
    v.y = epi_value<kLinResidual>(g, acc[1], bias[i].y, lsv[i].y, old[i][1]);
    v.z = epi_value<kLinResidual>(g, acc[2], bias[i].z, lsv[i].z, old[i][2]);
    v.w = epi_value<kLinResidual>(g, acc[3], bias[i].w, lsv[i].w, old[i][3]);
    *reinterpret_cast<float4*>(g.out + es[i]) = v;
    vv[i] = v;
  }
  float mean, inv;
  vkd::row_mean_inv<NV, true>(vv, lane, g.N, g.ln_eps, &mean, &inv);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c4 = lane + 64 * i;
    *reinterpret_cast<float4*>(g.ln_out + rb + 4 * static_cast<size_t>(c4)) =
        vkd::ln_apply4(vv[i], mean, inv, lg[i], lb[i]);
  }
}

}  // namespace

namespace vk {

namespace {

// Tile shape and split count, from a cost model fitted to plan sweeps of
// the ViT-B and ViT-L projections at 866 and 3,458 rows.  Workgroups are
// dealt round-robin to the CUs, so the busiest CU runs ceil(tiles * s / CUs)
// workgroups of up to ceil(chunks / s) K chunks each: about 5.5 us per
// chunk of a 128 x 128 tile, 0.6 of that for 64 x 128 and 0.28 for 64 x 64
// (a quarter of the MFMAs, more operand staging per MFMA, and more
// workgroups per CU to hide it: 1.0-1.5 us measured).  A split adds its
// partial sums (s x M x N floats written, then read by the sum pass, at
// about 5.5 TB/s) and the sum pass's launch (about 2 us).  The cheapest plan
// wins; on ties the larger tile, then the smaller count.  At least two
// chunks per split, at most VK_SPLITK_MAX slices and VK_SPLITK_MAX_FLOATS
// floats of partial sums.  One 866-token ViT-B image: QKV and FC1 64 x 64
// unsplit, projection 64 x 64 x 3, FC2 128 x 128 x 6; ViT-L at 3,458 rows:
// FC1 64 x 64, the others 128 x 128 (FC2 x 8); 10,392 rows: 128 x 128
// unsplit.
#ifndef VK_SPLITK_MAX
#define VK_SPLITK_MAX 8  // most partial slices
#endif
static_assert(VK_SPLITK_MAX >= 1 && VK_SPLITK_MAX <= kMaxSplits,
              "the sum passes read at most kMaxSplits slices");
#ifndef VK_SPLITK_MAX_FLOATS
#define VK_SPLITK_MAX_FLOATS (1LL << 26)  // 256 MB of partial sums
#endif
#ifndef VK_LINEAR_TILES
#define VK_LINEAR_TILES 7  // allowed tiles: bit 0 128x128, bit 1 64x128, bit 2 64x64
#endif

struct Plan {
  int tm, tn;
  int splits;
  long long tiles;
};

long long tile_count(int tm, int tn, int M, int N) {
  return static_cast<long long>((M + tm - 1) / tm) * static_cast<long long>((N + tn - 1) / tn);
}

Plan choose_plan(const vk_runtime* rt, int M, int N, int K) {
  constexpr double kChunkUs = 5.5, kBytesPerUs = 5.5e6, kSumLaunchUs = 2.0;
  // tile shape, cost of one of its K chunks relative to a 128 x 128 chunk
  struct Shape {
    int tm, tn, bit;
    double cost;
  };
  constexpr Shape kShapes[] = {{128, 128, 1, 1.0}, {64, 128, 2, 0.6}, {64, 64, 4, 0.28}};
  const long long cus = rt->cu_count > 0 ? rt->cu_count : 256;
  const int nch = (K + KC - 1) / KC;
  const long long mn = static_cast<long long>(M) * N;
  Plan best{0, 0, 1, 0};
  double best_us = 0.0;
  for (const Shape& sh : kShapes) {
    if (!(VK_LINEAR_TILES & sh.bit)) continue;
    const long long tiles = tile_count(sh.tm, sh.tn, M, N);
    for (int sp = 1; sp == 1 || (sp <= VK_SPLITK_MAX && 2 * sp <= nch &&
                                 sp * mn <= VK_SPLITK_MAX_FLOATS);
         ++sp) {
      const long long load = (tiles * sp + cus - 1) / cus * ((nch + sp - 1) / sp);
      double us = kChunkUs * sh.cost * static_cast<double>(load);
      if (sp > 1) us += 8.0 * static_cast<double>(sp * mn) / kBytesPerUs + kSumLaunchUs;
      if (best.tm == 0 || us < best_us) {
        best = Plan{sh.tm, sh.tn, sp, tiles};
        best_us = us;
      }
    }
  }
  return best;
}

template <int EPI, int LAY, int QKN = 0>
void launch_pair(vk_runtime* rt, const LinearArgs& g, const Plan& plan, dim3 grid,
                 bool sum_pass = true) {
  const long long cus = rt->cu_count > 0 ? rt->cu_count : 256;
  if (plan.tm == 128 && static_cast<long long>(grid.x) <= cus)
    hipLaunchKernelGGL((linear_wide_kernel<EPI, LAY, QKN, 128, 128, 1, true>), grid,
                       dim3(threads_for(128)), 0, rt->stream, g);
  else if (plan.tm == 128)
    hipLaunchKernelGGL((linear_wide_kernel<EPI, LAY, QKN, 128, 128>), grid,
                       dim3(threads_for(128)), 0, rt->stream, g);
  else if (plan.tn == 128)
    hipLaunchKernelGGL((linear_wide_kernel<EPI, LAY, QKN, 64, 128>), grid, dim3(threads_for(64)),
                       0, rt->stream, g);
  else
    hipLaunchKernelGGL((linear_wide_kernel<EPI, LAY, QKN, 64, 64, 2>), grid,
                       dim3(2 * threads_for(64)), 0, rt->stream, g);
  if (g.splits > 1 && sum_pass) {
    const long long n4 = static_cast<long long>(g.M) * g.N / 4;
    const dim3 sgrid(static_cast<unsigned>((n4 + 255) / 256));
    switch (split_bucket(g.splits)) {
      case 2:
        hipLaunchKernelGGL((splitk_reduce_kernel<EPI, LAY, QKN, 2>), sgrid, dim3(256), 0,
                           rt->stream, g);
        break;
      case 4:
        hipLaunchKernelGGL((splitk_reduce_kernel<EPI, LAY, QKN, 4>), sgrid, dim3(256), 0,
                           rt->stream, g);
        break;
      default:
        hipLaunchKernelGGL((splitk_reduce_kernel<EPI, LAY, QKN, 8>), sgrid, dim3(256), 0,
                           rt->stream, g);
        break;
    }
  }
}

}  // namespace

int launch_linear_wide(vk_runtime* rt, const LinearArgs& g0, int epi, float* partial,
                       size_t partial_floats) {
  LinearArgs g = g0;
  // An output element's bits depend on the plan (its split count, and the
  // two k groups of a 64 x 64 tile, added at the end) and the plan on
  // (M, N, K) alone, so every layout and epilogue of one shape gives the
  // same bits.
  const Plan plan = choose_plan(rt, g.M, g.N, g.K);
  g.splits = plan.splits;
  g.partial = nullptr;
  VK_UNSUPPORTED_IF(plan.tiles * g.splits > 0x7fffffffLL, "linear: %lld tiles", plan.tiles);
  // the staging loads address A and B rows with 32-bit byte offsets
  VK_UNSUPPORTED_IF(4LL * g.M * g.K >= (1LL << 32) || 4LL * g.N * g.Kp >= (1LL << 32),
                    "linear: operands of 4 GiB or more (M=%d, N=%d, K=%d)", g.M, g.N, g.K);
  if (g.splits > 1) {
    VK_REQUIRE(g.N % 4 == 0, "linear: split-K needs out_features % 4 == 0");
    const size_t need = static_cast<size_t>(g.splits) * g.M * g.N;
    if (partial) {
      VK_UNSUPPORTED_IF(need > partial_floats,
                        "linear (M=%d, N=%d, K=%d): %d split-K slices need %zu floats of "
                        "scratch, more than the %zu available",
                        g.M, g.N, g.K, g.splits, need, partial_floats);
      g.partial = partial;
    } else {
      VK_TRY(vk::ensure_work(rt, need, "linear (split-K)"));
      g.partial = rt->work;
    }
  }
  const dim3 grid(static_cast<unsigned>(plan.tiles * g.splits));
  // LayerNorm after the residual epilogue: in the sum pass when there is
  // one and a row is 768 or 1024 floats, else as a separate pass
  const bool post_ln = g.ln_out != nullptr;
  VK_REQUIRE(!post_ln || (epi == kLinResidual && !g.q_out),
             "linear: the LayerNorm follows the residual epilogue only");
  const bool fused_ln = post_ln && g.splits > 1 && (g.N == 768 || g.N == 1024);
  if (g.q_out) {
    VK_REQUIRE(epi == kLinStore, "linear: the Q|K|V split takes the store epilogue");
    switch (g.qkn_mode) {
      case 0: launch_pair<kLinStore, kQkvHnd>(rt, g, plan, grid); break;
      case 1: launch_pair<kLinStore, kQkvHnd, 1>(rt, g, plan, grid); break;
      case 2: launch_pair<kLinStore, kQkvHnd, 2>(rt, g, plan, grid); break;
      case 3: launch_pair<kLinStore, kQkvHnd, 3>(rt, g, plan, grid); break;
      default: return set_error(VK_ERR_INVALID, "linear: unknown Q/K epilogue %d", g.qkn_mode);
    }
  } else if (g.a_hnd) {
    if (epi == kLinResidual)
      launch_pair<kLinResidual, kAHnd>(rt, g, plan, grid, !fused_ln);
    else if (epi == kLinStore)
      launch_pair<kLinStore, kAHnd>(rt, g, plan, grid);
    else
      return set_error(VK_ERR_INVALID, "linear: head-major input takes store or residual");
  } else {
    switch (epi) {
      case kLinStore: launch_pair<kLinStore, kPlain>(rt, g, plan, grid); break;
      case kLinGelu: launch_pair<kLinGelu, kPlain>(rt, g, plan, grid); break;
      case kLinGeluErf: launch_pair<kLinGeluErf, kPlain>(rt, g, plan, grid); break;
      default: launch_pair<kLinResidual, kPlain>(rt, g, plan, grid, !fused_ln); break;
    }
  }
  VK_TRY(check_launch("linear_wide_kernel"));
  if (fused_ln) {
    const dim3 rows(static_cast<unsigned>(g.M));
    const bool f16 = g.ln_f16 != 0;
    const int nv = g.N == 768 ? 3 : 4;
    const int spb = split_bucket(g.splits);
#define VK_SKLN(NVV, PTT, SPBB)                                                                \
  if (nv == NVV && f16 == (sizeof(PTT) == 2) && spb == SPBB)                                    \
    hipLaunchKernelGGL((splitk_residual_ln_kernel<NVV, PTT, SPBB>), rows, dim3(64), 0,          \
                       rt->stream, g);
    VK_SKLN(3, float, 2) VK_SKLN(3, float, 4) VK_SKLN(3, float, 8)
    VK_SKLN(3, uint16_t, 2) VK_SKLN(3, uint16_t, 4) VK_SKLN(3, uint16_t, 8)
    VK_SKLN(4, float, 2) VK_SKLN(4, float, 4) VK_SKLN(4, float, 8)
    VK_SKLN(4, uint16_t, 2) VK_SKLN(4, uint16_t, 4) VK_SKLN(4, uint16_t, 8)
#undef VK_SKLN
    return check_launch("splitk_residual_ln_kernel");
  }
  if (post_ln)
    return layernorm_raw(rt, g.out, g.ln_out, g.ln_gamma, g.ln_beta, g.ln_f16 != 0, g.M, g.N,
                         g.ln_eps);
  return VK_OK;
}

}  // namespace vk
