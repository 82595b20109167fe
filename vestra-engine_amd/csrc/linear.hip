// The F32 linear on wide tiles for gfx950: the block projections (QKV, proj,
// FC1, FC2) with their per-token epilogues (bias, LayerScale, GELU,
// residual add) fused into the store.
//
// A workgroup of 512 threads (8 waves) owns a 128 x 128 output tile; wave w
// computes rows 32 (w/2) .. +32 and columns 64 (w%2) .. +64 as 2 x 4 tiles of
// v_mfma_f32_16x16x4_f32 (F32 in, F32 accumulate): 32 MFMAs per 16-wide
// k-block from six 128-bit LDS reads.  K is staged through LDS in chunks of
// 64, A as [m][k] and B as [n][k] rows with a pitch of 68 floats (4 x odd:
// the 16 rows of a fragment read start on 16 distinct 4-bank groups, and the
// staging stores of 16 lanes fill one row without conflicts).  The 70 KB of
// LDS leaves room for a second workgroup on the CU, which computes while the
// first stages a chunk or runs its epilogue.
//
// Fragment order as in the patch embedding: in block b, lane group g holds
// k = 16b + 4g + j in component j of a 128-bit read and MFMA step j uses
// component j, so four steps cover the block's 16 k once.
//
// Head-major layouts (head_dim 64): the QKV projection can store Q | K | V
// straight into three [heads, rows, 64] tensors (the split the attention
// kernels need), and the output projection can read its input from the
// head-major attention output; a 64-column strip of a wave is one head, and
// a float4 of A never crosses a head.  Both are pure address changes: the
// results are the bits of the linear plus the separate permutation.
//
// Traffic: a 128 x 128 tile moves (128 + 128) x 4 bytes of operands per k for
// 2 x 128 x 128 FLOP, 0.031 byte per FLOP from L2 (the 48 x 64 tiles of the
// narrow kernel need 0.073).  Tiles are numbered XCD-major (xcd_tile), so
// the workgroups of one XCD share weight columns in that XCD's L2.
#include "common.h"

namespace {

using vk::LinearArgs;
using namespace vk::linear_epilogue;

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TM = 128;
constexpr int TN = 128;
constexpr int KC = 64;
constexpr int PITCH = 68;
constexpr int kThreads = 512;
constexpr int kVec = TM * KC / 4 / kThreads;  // float4 of A (and of B) per thread a chunk: 4
static_assert(TM == TN && TM * KC / 4 % kThreads == 0, "staging slots divide evenly");
static_assert(PITCH % 4 == 0 && (PITCH / 4) % 2 == 1 && PITCH >= KC, "pitch 4 x odd");

enum Layout { kPlain = 0, kQkvHnd = 1, kAHnd = 2 };

template <int EPI, int LAY>
__global__ __launch_bounds__(kThreads, 2) void linear_wide_kernel(LinearArgs g) {
  __shared__ __align__(16) float As[TM * PITCH];
  __shared__ __align__(16) float Bs[TN * PITCH];

  const int tid = threadIdx.x;
  __builtin_assume(tid < kThreads);
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int gmt = (g.M + TM - 1) / TM;
  const int tile = vkd::xcd_tile(blockIdx.x, gridDim.x);
  const int m0 = (tile % gmt) * TM, n0 = (tile / gmt) * TN;

  f32x4 acc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kq = 4 * (lane >> 4);
  const float* arow = As + (wm * 32 + (lane & 15)) * PITCH + kq;
  const float* brow = Bs + (wn * 64 + (lane & 15)) * PITCH + kq;

  for (int k0 = 0; k0 < g.K; k0 += KC) {
    // stage the chunk: slot f = tid + 512 i is row f/16, float4 f%16 of the
    // chunk (a wave reads four 256-byte row segments).  Loads are never
    // guarded: out-of-range slots read a clamped address and store zeros.
    float4 ra[kVec], rb[kVec];
    bool oka[kVec], okb[kVec];
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const int f = tid + kThreads * i;
      const int r = f >> 4, c = 4 * (f & 15);
      const int gm = m0 + r, gn = n0 + r, gk = k0 + c;
      oka[i] = gm < g.M && gk < g.K;
      okb[i] = gn < g.N && gk < g.Kp;
      const int cm = gm < g.M ? gm : g.M - 1;
      const int cn = gn < g.N ? gn : g.N - 1;
      const int ck = gk < g.K ? gk : g.K - 4;
      const size_t ia = LAY == kAHnd
                            ? (static_cast<size_t>(ck >> 6) * g.M + cm) * 64 + (ck & 63)
                            : static_cast<size_t>(cm) * g.K + ck;
      ra[i] = *reinterpret_cast<const float4*>(g.x + ia);
      rb[i] = *reinterpret_cast<const float4*>(g.wnk + static_cast<size_t>(cn) * g.Kp +
                                                (gk < g.Kp ? gk : g.Kp - 4));
    }
    __syncthreads();  // every wave is done reading the previous chunk
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const int f = tid + kThreads * i;
      const int r = f >> 4, c = 4 * (f & 15);
      // component selects: a select of whole float4 values becomes a select
      // of their addresses, which puts the staging arrays in scratch memory
      const bool a_on = oka[i], b_on = okb[i];
      *reinterpret_cast<float4*>(As + r * PITCH + c) =
          make_float4(a_on ? ra[i].x : 0.f, a_on ? ra[i].y : 0.f, a_on ? ra[i].z : 0.f,
                      a_on ? ra[i].w : 0.f);
      *reinterpret_cast<float4*>(Bs + r * PITCH + c) =
          make_float4(b_on ? rb[i].x : 0.f, b_on ? rb[i].y : 0.f, b_on ? rb[i].z : 0.f,
                      b_on ? rb[i].w : 0.f);
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < KC / 16; ++b) {
      f32x4 a[2], w[4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        a[t] = *reinterpret_cast<const f32x4*>(arow + t * 16 * PITCH + 16 * b);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        w[u] = *reinterpret_cast<const f32x4*>(brow + u * 16 * PITCH + 16 * b);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < 4; ++u)
            acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][j], w[u][j], acc[t][u], 0, 0, 0);
    }
  }

  // epilogue: lane holds D[4*(lane/16) + r][lane%16] of each 16x16 tile.
  // Parameters and (for the residual) the old values are all loaded, on
  // clamped indices, before the first store.
  float bias[4], ls[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int col = n0 + wn * 64 + u * 16 + (lane & 15);
    const int cc = col < g.N ? col : g.N - 1;
    bias[u] = g.bias[cc];
    ls[u] = g.ls ? g.ls[cc] : 1.0f;
  }
  float old[2][4][4];
  if constexpr (EPI == kLinResidual) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + wm * 32 + t * 16 + 4 * (lane >> 4) + r;
          const int col = n0 + wn * 64 + u * 16 + (lane & 15);
          const int cr = row < g.M ? row : g.M - 1;
          const int cc = col < g.N ? col : g.N - 1;
          old[t][u][r] = g.out[static_cast<size_t>(cr) * g.N + cc];
        }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 32 + t * 16 + 4 * (lane >> 4) + r;
        const int col = n0 + wn * 64 + u * 16 + (lane & 15);
        if (row < g.M && col < g.N) {
          float v = acc[t][u][r] + bias[u];
          if (g.ls) v = v * ls[u];
          float* o;
          if constexpr (LAY == kQkvHnd) {
            const int embed = g.N / 3;
            const int which = col >= embed ? (col >= 2 * embed ? 2 : 1) : 0;
            const int c = col - which * embed;
            float* base = which == 0 ? g.q_out : (which == 1 ? g.k_out : g.v_out);
            o = base + (static_cast<size_t>(c >> 6) * g.M + row) * 64 + (c & 63);
          } else {
            o = g.out + static_cast<size_t>(row) * g.N + col;
          }
          if (EPI == kLinStore) *o = v;
          if (EPI == kLinGelu) *o = vkd::gelu1<0>(v);
          if (EPI == kLinGeluErf) *o = vkd::gelu1<1>(v);
          if (EPI == kLinResidual) *o = old[t][u][r] + v;
        }
      }
}

}  // namespace

namespace vk {

int launch_linear_wide(vk_runtime* rt, const LinearArgs& g, int epi) {
  const long long tiles =
      static_cast<long long>((g.M + TM - 1) / TM) * static_cast<long long>((g.N + TN - 1) / TN);
  VK_UNSUPPORTED_IF(tiles > 0x7fffffffLL, "linear: %lld tiles", tiles);
  const dim3 grid(static_cast<unsigned>(tiles)), block(kThreads);
  if (g.q_out) {
    VK_REQUIRE(epi == kLinStore, "linear: the Q|K|V split takes the store epilogue");
    hipLaunchKernelGGL((linear_wide_kernel<kLinStore, kQkvHnd>), grid, block, 0, rt->stream, g);
  } else if (g.a_hnd) {
    if (epi == kLinResidual)
      hipLaunchKernelGGL((linear_wide_kernel<kLinResidual, kAHnd>), grid, block, 0, rt->stream, g);
    else if (epi == kLinStore)
      hipLaunchKernelGGL((linear_wide_kernel<kLinStore, kAHnd>), grid, block, 0, rt->stream, g);
    else
      return set_error(VK_ERR_INVALID, "linear: head-major input takes store or residual");
  } else {
    switch (epi) {
      case kLinStore:
        hipLaunchKernelGGL((linear_wide_kernel<kLinStore, kPlain>), grid, block, 0, rt->stream, g);
        break;
      case kLinGelu:
        hipLaunchKernelGGL((linear_wide_kernel<kLinGelu, kPlain>), grid, block, 0, rt->stream, g);
        break;
      case kLinGeluErf:
        hipLaunchKernelGGL((linear_wide_kernel<kLinGeluErf, kPlain>), grid, block, 0, rt->stream,
                           g);
        break;
      default:
        hipLaunchKernelGGL((linear_wide_kernel<kLinResidual, kPlain>), grid, block, 0, rt->stream,
                           g);
        break;
    }
  }
  return check_launch("linear_wide_kernel");
}

}  // namespace vk
