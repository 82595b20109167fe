// Row-normalisation kernels for gfx950: block LayerNorm, the fused
// LayerScale+residual+LayerNorm, and the fused per-head Q/K LayerNorm + 2D
// RoPE.
//
// Mapping to CDNA4:
//  * LayerNorm rows (D = 768 / 1024): single-wave workgroups, each lane
//    holding D/256 float4 of a row in registers (128-bit coalesced loads: a
//    wave reads one contiguous KiB per instruction), mean and variance
//    reduced with DPP row reductions plus two cross-row swizzles; every row
//    read from HBM once and written once, both with nontemporal (streaming)
//    hints.  The waves are persistent: wave w takes rows w, w + W, ... (W =
//    vk::stream_waves), loading its next row before it reduces the current
//    one, so at the 12-view shape (10,392 rows, two per wave) each wave
//    reads both its rows before it writes either; once the rows are a
//    bandwidth-bound stream each store is also issued after the wave's
//    earlier memory operations (vkd::wait_memory: one store of a wave in
//    flight).  At 10,392 x 768: LayerNorm 11.2 us against 13.0-13.3 for one
//    row per wave, the fused LayerScale + residual + LayerNorm 22.4 against
//    23.7.  In-place element-wise streams (GELU, the Q/K rows) measured
//    slower in this form and keep theirs.
//  * Q/K rows (head_dim 64): 16 lanes per (head, token) row, one float4 per
//    lane, so a row's LayerNorm reduces inside one DPP row (4 DPP steps) and
//    the RoPE partner element (i <-> i+16 inside each 32-wide half) sits
//    exactly 4 lanes away: one swizzle, no LDS round trip.  Q and K rows are
//    covered by one launch; each 16-lane group streams two rows (both loads
//    in flight before the first reduction).
//  * Arithmetic per element follows the scalar reference order with every
//    product and sum rounded (built with -ffp-contract=off); by default only
//    the order of the mean/variance reductions differs (wave tree vs
//    sequential).  The runtime's sequential LayerNorm order replaces the
//    trees by the scalar order's chains (seq_layernorm_rows; the Q/K rows
//    through qk_apply_rows) and gives the CPU's bits.
#include <algorithm>

#include "common.h"
#include "qk_rows.h"

namespace {

using vkd::Param;

// ---------------------------------------------------------------------------
// Row streams shared by the LayerNorm kernels: a wave's NV float4 of row
// `row` (lane l: float4 l + 64 i), unguarded when EXACT (cols == 256 NV, so
// no lane is out of the row and no load waits behind a guard), zeros past
// the row otherwise.
// ---------------------------------------------------------------------------
template <int NV, bool EXACT>
__device__ __forceinline__ void load_row(float4 (&v)[NV], const float* base, int row, int cols,
                                         int lane) {
  const int nvec = cols >> 2;
  const float4* r = reinterpret_cast<const float4*>(base + static_cast<size_t>(row) * cols);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * 64;
    v[i] = (EXACT || c < nvec) ? vkd::ld_stream(r + c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// The next row is prefetched while the current one is reduced up to 8
// float4 per lane; wider rows walk their rows one at a time (register use).
template <int NV>
constexpr bool kRowPrefetch = NV <= 8;

// A copy of a parameter pointer that the compiler cannot see through: loads
// through it are not loop-invariant, so each row's parameter loads stay in
// the row loop, between the wave's stores, where the store waits
// (vkd::wait_memory) also wait for them.  At 10,392 x 768 the persistent
// LayerNorm measured 11.0 us so, 12.3 with the parameters held in registers
// across rows, and 12.6 without the waits (the compiler then issues a
// row's parameter loads ahead of its stores).  The pointer is offset by an
// opaque zero, not passed through the asm itself, so it keeps its global
// address space (global, not flat, loads).
template <typename T>
__device__ __forceinline__ const T* per_row(const T* p) {
  int zero = 0;
  asm volatile("" : "+s"(zero));
  return p + zero;
}

// ---------------------------------------------------------------------------
// LayerNorm over rows of `cols` floats.  NV = float4 per lane (cols <= 256
// NV).  Persistent single-wave workgroups: wave w normalises rows w, w + W,
// ... (W = gridDim.x, from vk::stream_waves), the next row's loads issued
// before the current row's reductions, the parameters re-read for each row
// (per_row) and, with SER, each store issued after the wave's earlier
// memory operations.  The per-row arithmetic is row_mean_inv + ln_apply4,
// the same as every other LayerNorm of a full row.  x and y may alias (each
// row is read and written only by its own wave).
// ---------------------------------------------------------------------------
template <int NV, typename PT, bool EXACT, bool SER>
__global__ __launch_bounds__(64) void layernorm_rows(const float* x, float* y,
                                                     const PT* __restrict__ gamma,
                                                     const PT* __restrict__ beta, int rows,
                                                     int cols, float eps) {
  const int lane = threadIdx.x;
  const int stride = static_cast<int>(gridDim.x);
  int row = blockIdx.x;
  if (row >= rows) return;
  const int nvec = cols >> 2;
  float4 cur[NV], nxt[NV];
  load_row<NV, EXACT>(cur, x, row, cols, lane);
  for (;;) {
    const int nrow = row + stride;
    const bool more = nrow < rows;
    if (kRowPrefetch<NV> && more) load_row<NV, EXACT>(nxt, x, nrow, cols, lane);
    float mean, inv;
    vkd::row_mean_inv<NV, EXACT>(cur, lane, cols, eps, &mean, &inv);
    float4* yr = reinterpret_cast<float4*>(y + static_cast<size_t>(row) * cols);
    const PT* g = per_row(gamma);
    const PT* b = per_row(beta);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + i * 64;
      if (EXACT || c < nvec) {
        const float4 o = vkd::ln_apply4(cur[i], mean, inv, Param<PT>::load4(g, c),
                                        Param<PT>::load4(b, c));
        if (SER) vkd::wait_memory();
        vkd::st_stream(yr + c, o);
      }
    }
    if (!more) break;
    if constexpr (kRowPrefetch<NV>) {
      for (int i = 0; i < NV; ++i) cur[i] = nxt[i];
    } else {
      load_row<NV, EXACT>(cur, x, nrow, cols, lane);
    }
    row = nrow;
  }
}

// ---------------------------------------------------------------------------
// x += ls (.) yb (t = yb*ls rounded, x = x + t rounded); ln_out = LN(x).
// HAS_LS false: unscaled residual add.  One wave per row, both streams'
// loads first: the latency-bound sizes (below kSerRowsPerCU rows per CU),
// where it measured 3.4 us cold at 866 x 768 against 4.0 for the persistent
// form below.
// CAM: the camera-token slot, row 0 of every view of tpv rows, then takes
// the camera token (cam[0..cols) for view 0, cam[cols..2 cols) for the
// others) in x and in the LayerNorm, as an overwrite between the residual
// update and the LayerNorm would.
// ---------------------------------------------------------------------------
template <int NV, typename PT, bool HAS_LS, bool EXACT, bool CAM>
__global__ __launch_bounds__(64) void ls_residual_layernorm_row(
    float* __restrict__ x, const float* __restrict__ yb, const PT* __restrict__ ls,
    const PT* __restrict__ gamma, const PT* __restrict__ beta,
    float* __restrict__ ln_out, int rows, int cols, float eps,
    const float* __restrict__ cam, int tpv) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x;
  if (row >= rows) return;
  const int nvec = cols >> 2;
  const size_t base = static_cast<size_t>(row) * cols;
  float4* xr = reinterpret_cast<float4*>(x + base);
  const float4* yr = reinterpret_cast<const float4*>(yb + base);
  // uniform over the wave
  const float4* camr = CAM && row % tpv == 0
                           ? reinterpret_cast<const float4*>(cam + (row >= tpv ? cols : 0))
                           : nullptr;
  float4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * 64;
    if (EXACT || c < nvec) {
      float4 a = vkd::ld_stream(xr + c);
      const float4 b = vkd::ld_stream(yr + c);
      if (HAS_LS) {
        const float4 g = Param<PT>::load4(ls, c);
        float t;
        t = b.x * g.x; a.x = a.x + t;
        t = b.y * g.y; a.y = a.y + t;
        t = b.z * g.z; a.z = a.z + t;
        t = b.w * g.w; a.w = a.w + t;
      } else {
        a.x = a.x + b.x;
        a.y = a.y + b.y;
        a.z = a.z + b.z;
        a.w = a.w + b.w;
      }
      if (CAM && camr) a = camr[c];
      vkd::st_stream(xr + c, a);
      v[i] = a;
    } else {
      v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float mean, inv;
  vkd::row_mean_inv<NV, EXACT>(v, lane, cols, eps, &mean, &inv);
  float4* outr = reinterpret_cast<float4*>(ln_out + base);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * 64;
    if (EXACT || c < nvec) {
      vkd::st_stream(outr + c, vkd::ln_apply4(v[i], mean, inv, Param<PT>::load4(gamma, c),
                                              Param<PT>::load4(beta, c)));
    }
  }
}

// ---------------------------------------------------------------------------
// x += ls (.) yb (t = yb*ls rounded, x = x + t rounded); ln_out = LN(x).
// HAS_LS false: unscaled residual add.  Persistent single-wave workgroups
// over rows w, w + W, ... as layernorm_rows, the next row's x and yb loaded
// (interleaved float4 by float4) before the current row's arithmetic; SER:
// every store issued after the wave's earlier memory operations.  The
// pointers carry no __restrict__: with it the compiler batched the
// parameter loads ahead of the stores and the stream measured 24.4 us
// instead of 22.4 at 10,392 x 768 (one row per wave: 23.7).
// CAM: the camera-token slot, row 0 of every view of tpv rows, then takes
// the camera token (cam[0..cols) for view 0, cam[cols..2 cols) for the
// others) in x and in the LayerNorm, as an overwrite between the residual
// update and the LayerNorm would.
// ---------------------------------------------------------------------------
template <int NV, typename PT, bool HAS_LS, bool EXACT, bool SER, bool CAM>
__global__ __launch_bounds__(64) void ls_residual_layernorm_rows(
    float* x, const float* yb, const PT* ls, const PT* gamma, const PT* beta, float* ln_out,
    int rows, int cols, float eps, const float* cam, int tpv) {
  const int lane = threadIdx.x;
  const int stride = static_cast<int>(gridDim.x);
  int row = blockIdx.x;
  const int nvec = cols >> 2;
  float4 ca[NV], cb[NV], na[NV], nb[NV];
  if (row < rows) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      const bool in = EXACT || c < nvec;
      ca[i] = in ? vkd::ld_stream(reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * cols) + c)
                 : make_float4(0.f, 0.f, 0.f, 0.f);
      cb[i] = in ? vkd::ld_stream(reinterpret_cast<const float4*>(yb + static_cast<size_t>(row) * cols) + c)
                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  while (row < rows) {
    const int nrow = row + stride;
    if (kRowPrefetch<NV> && nrow < rows) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = lane + 64 * i;
        const bool in = EXACT || c < nvec;
        na[i] = in ? vkd::ld_stream(reinterpret_cast<const float4*>(x + static_cast<size_t>(nrow) * cols) + c)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
        nb[i] = in ? vkd::ld_stream(reinterpret_cast<const float4*>(yb + static_cast<size_t>(nrow) * cols) + c)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    // uniform over the wave
    const float4* camr = CAM && row % tpv == 0
                             ? reinterpret_cast<const float4*>(cam + (row >= tpv ? cols : 0))
                             : nullptr;
    float4* xr = reinterpret_cast<float4*>(x + static_cast<size_t>(row) * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (EXACT || c < nvec) {
        float4 a = ca[i];
        const float4 b = cb[i];
        if (HAS_LS) {
          const float4 g = Param<PT>::load4(ls, c);
          float t;
          t = b.x * g.x; a.x = a.x + t;
          t = b.y * g.y; a.y = a.y + t;
          t = b.z * g.z; a.z = a.z + t;
          t = b.w * g.w; a.w = a.w + t;
        } else {
          a.x = a.x + b.x;
          a.y = a.y + b.y;
          a.z = a.z + b.z;
          a.w = a.w + b.w;
        }
        if (CAM && camr) a = camr[c];
        if (SER) vkd::wait_memory();
        vkd::st_stream(xr + c, a);
        ca[i] = a;
      }
    }
    float mean, inv;
    vkd::row_mean_inv<NV, EXACT>(ca, lane, cols, eps, &mean, &inv);
    float4* outr = reinterpret_cast<float4*>(ln_out + static_cast<size_t>(row) * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (EXACT || c < nvec) {
        const float4 o = vkd::ln_apply4(ca[i], mean, inv, Param<PT>::load4(gamma, c),
                                        Param<PT>::load4(beta, c));
        if (SER) vkd::wait_memory();
        vkd::st_stream(outr + c, o);
      }
    }
    if constexpr (kRowPrefetch<NV>) {
      for (int i = 0; i < NV; ++i) {
        ca[i] = na[i];
        cb[i] = nb[i];
      }
    } else if (nrow < rows) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = lane + 64 * i;
        const bool in = EXACT || c < nvec;
        ca[i] = in ? vkd::ld_stream(reinterpret_cast<const float4*>(x + static_cast<size_t>(nrow) * cols) + c)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
        cb[i] = in ? vkd::ld_stream(reinterpret_cast<const float4*>(yb + static_cast<size_t>(nrow) * cols) + c)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    row = nrow;
  }
}

// ---------------------------------------------------------------------------
// LayerNorm in the scalar reference's summation order (the runtime's
// VK_LN_ORDER_SEQUENTIAL): mean = ((x0 + x1) + x2 + ...) / cols and the
// biased two-pass variance summed the same way, left to right, then
// 1/sqrtf(var + eps) correctly rounded -- the bits of the CPU kernel
// (dpt_head.rs:272-296).  A sum in that order is one chain of `cols`
// dependent adds, which no wave reduction reproduces, so a 256-thread
// workgroup owns `rpw` whole rows: it loads them (coalesced float4, kept in
// registers) into LDS, lane r of wave 0 walks row r of the LDS copy for the
// mean, every thread replaces its elements in LDS by their rounded squared
// deviations, lane r walks those for the variance, and every thread applies
// the LayerNorm to its registers.  The rows of a workgroup walk in parallel
// (one lane each); the chains (2 x cols adds per row) are the latency, which
// the CU's other workgroups overlap with their loads and stores.
//
// LSRES: x += ls (.) yb (or + yb) first, written back to x, with the camera
// slot (row 0 of every view of tpv rows) overwritten when CAM -- the fused
// LayerScale + residual + LayerNorm's arithmetic, then its LayerNorm in
// this order.  out null: only the statistics (mean, 1/std) go to `stats`,
// for logical row r read from stored row (r / np) * n + ns + r % np (np 0:
// row r) -- the capture's patch rows.
// ---------------------------------------------------------------------------
constexpr int kSeqThreads = 256;
constexpr int kSeqMaxRows = 64;  // one chain lane per row, all in wave 0

struct SeqLnArgs {
  float* x;
  const float* yb;
  const void* ls;
  const void* gamma;
  const void* beta;
  float* out;
  float2* stats;
  const float* cam;
  int tpv;
  int rows, cols, rpw;
  float eps;
  vkd::FastDivU32 c4;  // cols / 4
  int np, n, ns;
  vkd::FastDivU32 fnp;
};

// ((0 + e0) + e1) + ... over the n4 float4 of one LDS row: one chain of
// dependent adds in element order (eight LDS reads in flight per step).
__device__ __forceinline__ float seq_row_sum(const float4* rp, int n4) {
  float s = 0.0f;
#pragma unroll 8
  for (int c = 0; c < n4; ++c) {
    const float4 w = rp[c];
    s += w.x;
    s += w.y;
    s += w.z;
    s += w.w;
  }
  return s;
}

template <int NV, typename PT, bool LSRES, bool HAS_LS, bool CAM>
__global__ __launch_bounds__(kSeqThreads) void seq_layernorm_rows(SeqLnArgs a) {
  // rpw rows of c4 + 1 float4 (the pad puts the 16 chain lanes' reads on
  // distinct 4-bank groups), then the rows' (mean, 1/std)
  __shared__ float4 rows_lds[NV * kSeqThreads + kSeqMaxRows];
  __shared__ float2 st[kSeqMaxRows];
  const int tid = threadIdx.x;
  const int c4 = static_cast<int>(a.c4.d);
  const int pitch4 = c4 + 1;
  const int r0 = blockIdx.x * a.rpw;
  const int nr = min(a.rpw, a.rows - r0);
  const int slots = nr * c4;
  float4 v[NV];
  // every load first (clamped to a valid slot: no load waits behind a
  // guard or a store), then the arithmetic, the stores and the LDS copy
  float4 b[LSRES ? NV : 1];
  int lrow[NV], col[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + kSeqThreads * i;
    const int ec = e < slots ? e : slots - 1;
    lrow[i] = static_cast<int>(vkd::fdiv(static_cast<uint32_t>(ec), a.c4));
    col[i] = ec - lrow[i] * c4;
    const int r = r0 + lrow[i];
    size_t row = static_cast<size_t>(r);
    if (!LSRES && a.np) {
      const int vw = static_cast<int>(vkd::fdiv(static_cast<uint32_t>(r), a.fnp));
      row = static_cast<size_t>(vw) * a.n + a.ns + (r - vw * a.np);
    }
    const size_t off = row * a.cols + 4 * static_cast<size_t>(col[i]);
    v[i] = vkd::ld_stream(reinterpret_cast<const float4*>(a.x + off));
    if (LSRES) b[i] = vkd::ld_stream(reinterpret_cast<const float4*>(a.yb + off));
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + kSeqThreads * i;
    if (LSRES) {
      const int c = col[i], r = r0 + lrow[i];
      if (HAS_LS) {
        const float4 g = Param<PT>::load4(static_cast<const PT*>(a.ls), c);
        float t;
        t = b[i].x * g.x; v[i].x = v[i].x + t;
        t = b[i].y * g.y; v[i].y = v[i].y + t;
        t = b[i].z * g.z; v[i].z = v[i].z + t;
        t = b[i].w * g.w; v[i].w = v[i].w + t;
      } else {
        v[i].x = v[i].x + b[i].x;
        v[i].y = v[i].y + b[i].y;
        v[i].z = v[i].z + b[i].z;
        v[i].w = v[i].w + b[i].w;
      }
      if (CAM && r % a.tpv == 0)
        v[i] = reinterpret_cast<const float4*>(a.cam + (r >= a.tpv ? a.cols : 0))[c];
      if (e < slots)
        vkd::st_stream(reinterpret_cast<float4*>(a.x + static_cast<size_t>(r) * a.cols + 4 * c),
                       v[i]);
    }
    if (e < slots) rows_lds[lrow[i] * pitch4 + col[i]] = v[i];
  }
  __syncthreads();
  if (tid < nr) st[tid].x = seq_row_sum(rows_lds + tid * pitch4, c4) / static_cast<float>(a.cols);
  __syncthreads();
  // squared deviations, each rounded, in place of the values
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + kSeqThreads * i;
    if (e < slots) {
      const float m = st[lrow[i]].x;
      float4 d;
      d.x = v[i].x - m; d.x = d.x * d.x;
      d.y = v[i].y - m; d.y = d.y * d.y;
      d.z = v[i].z - m; d.z = d.z * d.z;
      d.w = v[i].w - m; d.w = d.w * d.w;
      rows_lds[lrow[i] * pitch4 + col[i]] = d;
    }
  }
  __syncthreads();
  if (tid < nr) {
    const float var = seq_row_sum(rows_lds + tid * pitch4, c4) / static_cast<float>(a.cols);
    const float inv = 1.0f / sqrtf(var + a.eps);
    st[tid].y = inv;
    if (a.stats) a.stats[r0 + tid] = make_float2(st[tid].x, inv);
  }
  if (!a.out) return;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + kSeqThreads * i;
    if (e < slots) {
      const float2 ms = st[lrow[i]];
      // the output forms keep the stored row order (no row map)
      const size_t off = static_cast<size_t>(r0 + lrow[i]) * a.cols + 4 * col[i];
      vkd::st_stream(reinterpret_cast<float4*>(a.out + off),
                     vkd::ln_apply4(v[i], ms.x, ms.y,
                                    Param<PT>::load4(static_cast<const PT*>(a.gamma), col[i]),
                                    Param<PT>::load4(static_cast<const PT*>(a.beta), col[i])));
    }
  }
}

// ---------------------------------------------------------------------------
// Q/K LayerNorm (head_dim 64) + 2D RoPE, in place.
// ---------------------------------------------------------------------------
using namespace vkq;

// With Q and K, each 16-lane group owns kQkRowsPerGroup / 2 (head, token)
// pairs of a Q row and a K row: one position and one cos/sin lookup serve
// both rows of a pair, and every row's loads are issued before any row's
// reductions, doubling the bytes in flight per wave.  A single tensor (the
// rotation alone), or an odd kQkRowsPerGroup, gives each group
// kQkRowsPerGroup consecutive rows.
#ifndef VK_QK_ROWS_PER_GROUP
#define VK_QK_ROWS_PER_GROUP 2
#endif
constexpr int kQkRowsPerGroup = VK_QK_ROWS_PER_GROUP;
constexpr int kQkThreads = 256;  // threads per workgroup: kQkThreads / 16 row groups

// The rows of every 16-lane group in the sequential LayerNorm order
// (SEQ): the group's rows go to LDS (row pitch 17 float4, so the chain lanes
// of a wave read distinct 4-bank groups), lane j of the group walks row j's
// 64 values left to right for the sum, every lane writes its rounded
// squared deviations back, lane j walks those for the variance, and every
// lane then normalises with 1/sqrtf(var + eps) and rotates: the bits of the
// CPU's LayerNorm and rotation of each row.  One chain lane per row issues
// a fraction of the VALU work of a chain every lane runs redundantly.
template <int R, bool HAS_NORM, int PAIR, bool SEQ>
__device__ __forceinline__ void qk_apply_rows(float4 (&v)[R], int l, const QkRowOperands (&op)[R],
                                              float eps) {
  if constexpr (HAS_NORM && SEQ) {
    __shared__ float4 rows[kQkThreads / 16 * R * 17];
    __shared__ float stat[kQkThreads / 16 * R];
    const int grp = threadIdx.x >> 4;
    float4* gr = rows + grp * R * 17;
#pragma unroll
    for (int j = 0; j < R; ++j) gr[j * 17 + l] = v[j];
    __syncthreads();
    if (l < R) {
      const float4* rp = gr + l * 17;
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float4 w = rp[c];
        s += w.x;
        s += w.y;
        s += w.z;
        s += w.w;
      }
      stat[grp * R + l] = s / 64.0f;
    }
    __syncthreads();
    float mean[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      mean[j] = stat[grp * R + j];
      float4 d;
      d.x = v[j].x - mean[j]; d.x = d.x * d.x;
      d.y = v[j].y - mean[j]; d.y = d.y * d.y;
      d.z = v[j].z - mean[j]; d.z = d.z * d.z;
      d.w = v[j].w - mean[j]; d.w = d.w * d.w;
      gr[j * 17 + l] = d;
    }
    __syncthreads();
    if (l < R) {
      const float4* rp = gr + l * 17;
      float q = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float4 w = rp[c];
        q += w.x;
        q += w.y;
        q += w.z;
        q += w.w;
      }
      stat[grp * R + l] = 1.0f / sqrtf(q / 64.0f + eps);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < R; ++j)
      v[j] = qk_row_rope<PAIR>(qk_norm_apply(v[j], mean[j], stat[grp * R + j], op[j]), l, op[j]);
  } else {
#pragma unroll
    for (int j = 0; j < R; ++j) v[j] = qk_row_apply<HAS_NORM, PAIR>(v[j], l, op[j], eps);
  }
}

template <typename PT, bool HAS_NORM, int POS, int PAIR, bool SEQ = false>
__global__ __launch_bounds__(kQkThreads) void qk_norm_rope_rows(
    float* __restrict__ q, float* __restrict__ k, const PT* __restrict__ qg,
    const PT* __restrict__ qb, const PT* __restrict__ kg, const PT* __restrict__ kb,
    const void* __restrict__ pos_yx, const float* __restrict__ table, QkShape sh,
    float eps) {
  const int l = threadIdx.x & 15;
  const uint32_t grp = blockIdx.x * (kQkThreads / 16u) + (threadIdx.x >> 4);
  const uint32_t total = sh.tensors * sh.rows_per_tensor;
  // every row's loads (data, parameters, cos/sin) before any row's
  // arithmetic: one memory round trip per wave
  float4 v[kQkRowsPerGroup];
  QkRowOperands op[kQkRowsPerGroup];
  if (kQkRowsPerGroup % 2 == 0 && sh.tensors == 2) {
    // Q row and K row pairs of one (head, token) each: one position and one
    // cos/sin lookup per pair
    constexpr int NP = kQkRowsPerGroup / 2;
    uint32_t rr[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const uint32_t r = grp * NP + p;
      rr[p] = r < sh.rows_per_tensor ? r : sh.rows_per_tensor - 1;
      float py, px;
      qk_row_position<POS>(rr[p], sh, pos_yx, &py, &px);
      v[2 * p] = vkd::ld_stream(reinterpret_cast<const float4*>(q + static_cast<size_t>(rr[p]) * 64) + l);
      v[2 * p + 1] =
          vkd::ld_stream(reinterpret_cast<const float4*>(k + static_cast<size_t>(rr[p]) * 64) + l);
      op[2 * p] = qk_row_operands<PT, HAS_NORM, POS, PAIR>(l, qg, qb, py, px, table, sh.table_max);
      op[2 * p + 1] = op[2 * p];
      if (HAS_NORM) {
        op[2 * p + 1].g = qk_param4(kg, l);
        op[2 * p + 1].b = qk_param4(kb, l);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    qk_apply_rows<kQkRowsPerGroup, HAS_NORM, PAIR, SEQ>(v, l, op, eps);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (grp * NP + p < sh.rows_per_tensor) {
        vkd::st_stream(reinterpret_cast<float4*>(q + static_cast<size_t>(rr[p]) * 64) + l, v[2 * p]);
        vkd::st_stream(reinterpret_cast<float4*>(k + static_cast<size_t>(rr[p]) * 64) + l,
                       v[2 * p + 1]);
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < kQkRowsPerGroup; ++j) {
    const uint32_t gr = grp * kQkRowsPerGroup + j;
    // rows past the end read the last row (always valid) and are not stored
    const uint32_t gc = gr < total ? gr : total - 1;
    const bool is_k = gc >= sh.rows_per_tensor;
    const uint32_t r = is_k ? gc - sh.rows_per_tensor : gc;
    float py, px;
    qk_row_position<POS>(r, sh, pos_yx, &py, &px);
    v[j] = vkd::ld_stream(reinterpret_cast<const float4*>((is_k ? k : q) + static_cast<size_t>(r) * 64) + l);
    op[j] = qk_row_operands<PT, HAS_NORM, POS, PAIR>(l, is_k ? kg : qg, is_k ? kb : qb, py, px,
                                                     table, sh.table_max);
  }
  __builtin_amdgcn_sched_barrier(0);
  qk_apply_rows<kQkRowsPerGroup, HAS_NORM, PAIR, SEQ>(v, l, op, eps);
#pragma unroll
  for (int j = 0; j < kQkRowsPerGroup; ++j) {
    const uint32_t gr = grp * kQkRowsPerGroup + j;
    if (gr < total) {
      const bool is_k = gr >= sh.rows_per_tensor;
      const uint32_t r = is_k ? gr - sh.rows_per_tensor : gr;
      vkd::st_stream(reinterpret_cast<float4*>((is_k ? k : q) + static_cast<size_t>(r) * 64) + l, v[j]);
    }
  }
}

// positions tensor [rows*2] as the reference's host builder produces it
__global__ void rope_positions_kernel(float* __restrict__ pos, long long rows,
                                      int tokens_per_view, int n_special, int gw,
                                      int global) {
  const long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= rows) return;
  const int lt = static_cast<int>(t % tokens_per_view);
  float y = 0.0f, x = 0.0f;
  if (lt >= n_special) {
    if (global) {
      y = 1.0f;
      x = 1.0f;
    } else {
      const int p = lt - n_special;
      y = static_cast<float>(p / gw + 1);
      x = static_cast<float>(p % gw + 1);
    }
  }
  pos[2 * t] = y;
  pos[2 * t + 1] = x;
}

// ---------------------------------------------------------------------------
// host dispatch helpers
// ---------------------------------------------------------------------------

bool param_ok(const vk_tensor* t, size_t len) {
  return t && (t->dtype == VK_F32 || t->dtype == VK_F16) && t->len == len;
}

int ln_instance_cols(int cols) {
  int nv = (cols + 255) / 256;
  if (nv <= 8) return nv;
  if (nv <= 12) return 12;
  if (nv <= 16) return 16;
  if (nv <= 32) return 32;
  return -1;
}

// Rows per workgroup of the sequential-order kernel for rows of `cols`
// floats (at most 12 float4 per thread, one chain lane per row) and the
// instance (float4 per thread) that holds them.
SeqLnArgs seq_args(float* x, int rows, int cols, float eps, int* nv) {
  SeqLnArgs a{};
  a.x = x;
  a.rows = rows;
  a.cols = cols;
  a.eps = eps;
  a.rpw = std::max(1, std::min(kSeqMaxRows, 12 * kSeqThreads * 4 / cols));
  a.c4 = vkd::make_fastdiv(static_cast<uint32_t>(cols / 4));
  a.tpv = 1;
  const int need = (a.rpw * (cols / 4) + kSeqThreads - 1) / kSeqThreads;
  *nv = need <= 4 ? 4 : (need <= 8 ? 8 : 12);
  return a;
}

template <typename PT, bool LSRES, bool HAS_LS, bool CAM>
int launch_seq(vk_runtime* rt, const SeqLnArgs& a, int nv) {
  const dim3 grid(static_cast<unsigned>((a.rows + a.rpw - 1) / a.rpw)), block(kSeqThreads);
  switch (nv) {
    case 4:
      hipLaunchKernelGGL((seq_layernorm_rows<4, PT, LSRES, HAS_LS, CAM>), grid, block, 0,
                         rt->stream, a);
      break;
    case 8:
      hipLaunchKernelGGL((seq_layernorm_rows<8, PT, LSRES, HAS_LS, CAM>), grid, block, 0,
                         rt->stream, a);
      break;
    default:
      hipLaunchKernelGGL((seq_layernorm_rows<12, PT, LSRES, HAS_LS, CAM>), grid, block, 0,
                         rt->stream, a);
      break;
  }
  return vk::check_launch("seq_layernorm_rows");
}

// Stores serialised per wave (SER) once the rows are a bandwidth-bound
// stream: at least kSerRowsPerCU rows per CU (2,048 on 256 CUs).  At one
// image (866 rows) the launch is latency-bound and the waits cost time
// (LayerNorm 2.9 -> 3.2 us, the fused form 3.4 -> 4.0 us in cold HBM).
constexpr int kSerRowsPerCU = 8;

bool serialise_stores(const vk_runtime* rt, int rows) {
  return rows >= (rt->cu_count > 0 ? rt->cu_count : 256) * kSerRowsPerCU;
}

template <typename PT>
int launch_layernorm(vk_runtime* rt, const float* x, float* y, const void* g,
                     const void* b, int rows, int cols, float eps) {
  if (rt->ln_order == VK_LN_ORDER_SEQUENTIAL) {
    int snv = 0;
    SeqLnArgs a = seq_args(const_cast<float*>(x), rows, cols, eps, &snv);
    a.gamma = g;
    a.beta = b;
    a.out = y;
    return launch_seq<PT, false, false, false>(rt, a, snv);
  }
  const int nv = ln_instance_cols(cols);
  const dim3 grid(vk::stream_waves(rt, rows)), block(64);
  const bool ser = serialise_stores(rt, rows);
  auto G = static_cast<const PT*>(g);
  auto B = static_cast<const PT*>(b);
#define VK_LN_CASE(N)                                                                          \
  case N:                                                                                      \
    if (cols == N * 256 && ser)                                                                \
      hipLaunchKernelGGL((layernorm_rows<N, PT, true, true>), grid, block, 0, rt->stream, x, y, G, B, rows, cols, eps); \
    else if (cols == N * 256)                                                                  \
      hipLaunchKernelGGL((layernorm_rows<N, PT, true, false>), grid, block, 0, rt->stream, x, y, G, B, rows, cols, eps); \
    else                                                                                       \
      hipLaunchKernelGGL((layernorm_rows<N, PT, false, false>), grid, block, 0, rt->stream, x, y, G, B, rows, cols, eps); \
    break;
  switch (nv) {
    VK_LN_CASE(1) VK_LN_CASE(2) VK_LN_CASE(3) VK_LN_CASE(4)
    VK_LN_CASE(5) VK_LN_CASE(6) VK_LN_CASE(7) VK_LN_CASE(8)
    VK_LN_CASE(12) VK_LN_CASE(16) VK_LN_CASE(32)
    default:
      return vk::set_error(VK_ERR_UNSUPPORTED, "layernorm: no instance for cols=%d", cols);
  }
#undef VK_LN_CASE
  return vk::check_launch("layernorm_rows");
}

template <typename PT, bool HAS_LS>
int launch_ls_res_ln(vk_runtime* rt, float* x, const float* yb, const void* ls,
                     const void* g, const void* b, float* out, int rows, int cols,
                     float eps, const float* cam = nullptr, int tpv = 1) {
  if (rt->ln_order == VK_LN_ORDER_SEQUENTIAL) {
    int snv = 0;
    SeqLnArgs a = seq_args(x, rows, cols, eps, &snv);
    a.yb = yb;
    a.ls = ls;
    a.gamma = g;
    a.beta = b;
    a.out = out;
    a.cam = cam;
    a.tpv = tpv;
    return cam ? launch_seq<PT, true, HAS_LS, true>(rt, a, snv)
               : launch_seq<PT, true, HAS_LS, false>(rt, a, snv);
  }
  const int nv = ln_instance_cols(cols);
  const dim3 grid(vk::stream_waves(rt, rows)), block(64);
  const bool ser = serialise_stores(rt, rows);
  auto LS = static_cast<const PT*>(ls);
  auto G = static_cast<const PT*>(g);
  auto B = static_cast<const PT*>(b);
#define VK_LSLN_LAUNCH(N, EX, SR, CM)                                                          \
  hipLaunchKernelGGL((ls_residual_layernorm_rows<N, PT, HAS_LS, EX, SR, CM>), grid, block, 0, \
                     rt->stream, x, yb, LS, G, B, out, rows, cols, eps, cam, tpv)
#define VK_LSLN_ROW(N, EX, CM)                                                                 \
  hipLaunchKernelGGL((ls_residual_layernorm_row<N, PT, HAS_LS, EX, CM>), dim3(rows), block, 0,  \
                     rt->stream, x, yb, LS, G, B, out, rows, cols, eps, cam, tpv)
#define VK_LSLN_CASE(N)                                                                        \
  case N:                                                                                      \
    if (cols == N * 256 && ser) {                                                              \
      if (cam) VK_LSLN_LAUNCH(N, true, true, true); else VK_LSLN_LAUNCH(N, true, true, false); \
    } else if (cols == N * 256) {                                                              \
      if (cam) VK_LSLN_ROW(N, true, true); else VK_LSLN_ROW(N, true, false);                   \
    } else if (cam) {                                                                          \
      VK_LSLN_ROW(N, false, true);                                                             \
    } else {                                                                                   \
      VK_LSLN_ROW(N, false, false);                                                            \
    }                                                                                          \
    break;
  switch (nv) {
    VK_LSLN_CASE(1) VK_LSLN_CASE(2) VK_LSLN_CASE(3) VK_LSLN_CASE(4)
    VK_LSLN_CASE(5) VK_LSLN_CASE(6) VK_LSLN_CASE(7) VK_LSLN_CASE(8)
    VK_LSLN_CASE(12) VK_LSLN_CASE(16) VK_LSLN_CASE(32)
    default:
      return vk::set_error(VK_ERR_UNSUPPORTED, "ls_residual_layernorm: no instance for cols=%d", cols);
  }
#undef VK_LSLN_CASE
#undef VK_LSLN_LAUNCH
#undef VK_LSLN_ROW
  return vk::check_launch("ls_residual_layernorm_rows");
}

template <typename PT, bool HAS_NORM, int POS, int PAIR>
int launch_qk(vk_runtime* rt, float* q, float* k, const void* qg, const void* qb,
              const void* kg, const void* kb, const void* pos, const float* table,
              const QkShape& sh, float eps) {
  const long long total = static_cast<long long>(sh.tensors) * sh.rows_per_tensor;
  const long long groups = (total + kQkRowsPerGroup - 1) / kQkRowsPerGroup;
  const long long blocks = (groups + kQkThreads / 16 - 1) / (kQkThreads / 16);
  if constexpr (HAS_NORM) {
    if (rt->ln_order == VK_LN_ORDER_SEQUENTIAL) {
      hipLaunchKernelGGL((qk_norm_rope_rows<PT, HAS_NORM, POS, PAIR, true>),
                         dim3(static_cast<unsigned>(blocks)), dim3(kQkThreads), 0, rt->stream, q,
                         k, static_cast<const PT*>(qg), static_cast<const PT*>(qb),
                         static_cast<const PT*>(kg), static_cast<const PT*>(kb), pos, table, sh,
                         eps);
      return vk::check_launch("qk_norm_rope_rows");
    }
  }
  hipLaunchKernelGGL((qk_norm_rope_rows<PT, HAS_NORM, POS, PAIR>),
                     dim3(static_cast<unsigned>(blocks)), dim3(kQkThreads), 0, rt->stream, q, k,
                     static_cast<const PT*>(qg), static_cast<const PT*>(qb),
                     static_cast<const PT*>(kg), static_cast<const PT*>(kb), pos, table, sh, eps);
  return vk::check_launch("qk_norm_rope_rows");
}

template <int POS, int PAIR>
int dispatch_qk_pair(vk_runtime* rt, float* Q, float* K, const vk_tensor* qg,
                     const vk_tensor* qb, const vk_tensor* kg, const vk_tensor* kb,
                     const void* pos, const float* table, const QkShape& sh, float eps) {
  if (!qg)
    return launch_qk<float, false, POS, PAIR>(rt, Q, K, nullptr, nullptr, nullptr, nullptr, pos,
                                              table, sh, eps);
  if (qg->dtype == VK_F16)
    return launch_qk<uint16_t, true, POS, PAIR>(rt, Q, K, qg->ptr, qb->ptr, kg->ptr, kb->ptr,
                                                pos, table, sh, eps);
  return launch_qk<float, true, POS, PAIR>(rt, Q, K, qg->ptr, qb->ptr, kg->ptr, kb->ptr, pos,
                                           table, sh, eps);
}

// q, k: the tensors (k == q with sh.tensors == 1); qg..kb null: RoPE only.
template <int POS>
int dispatch_qk(vk_runtime* rt, float* Q, float* K, const vk_tensor* qg, const vk_tensor* qb,
                const vk_tensor* kg, const vk_tensor* kb, const void* pos, const float* table,
                const QkShape& sh, float eps, unsigned rope_mode) {
  if (rope_mode & VK_ROPE_INTERLEAVED)
    return dispatch_qk_pair<POS, kInterleaved>(rt, Q, K, qg, qb, kg, kb, pos, table, sh, eps);
  return dispatch_qk_pair<POS, kRotateHalf>(rt, Q, K, qg, qb, kg, kb, pos, table, sh, eps);
}

// Explicit positions: the f32, i32 or i64 instance for the tensor's dtype.
int dispatch_qk_explicit(vk_runtime* rt, float* Q, float* K, const vk_tensor* qg,
                         const vk_tensor* qb, const vk_tensor* kg, const vk_tensor* kb,
                         const vk_tensor* positions, const float* table, const QkShape& sh,
                         float eps, unsigned rope_mode) {
  switch (positions->dtype) {
    case VK_I32:
      return dispatch_qk<kPosExplicitI32>(rt, Q, K, qg, qb, kg, kb, positions->ptr, table, sh,
                                          eps, rope_mode);
    case VK_I64:
      return dispatch_qk<kPosExplicitI64>(rt, Q, K, qg, qb, kg, kb, positions->ptr, table, sh,
                                          eps, rope_mode);
    default:
      return dispatch_qk<kPosExplicit>(rt, Q, K, qg, qb, kg, kb, positions->ptr, table, sh, eps,
                                       rope_mode);
  }
}

bool positions_ok(const vk_tensor* p) {
  return p && (p->dtype == VK_F32 || p->dtype == VK_I32 || p->dtype == VK_I64);
}

// The positions-tensor shape of the reference-signature forms: rows_per_tensor
// = heads * rows, one sequence of `rows` tokens.
QkShape explicit_shape(size_t heads, size_t rows, int table_max, uint32_t tensors) {
  QkShape sh;
  sh.rows_per_tensor = static_cast<uint32_t>(heads * rows);
  sh.tensors = tensors;
  sh.table_max = table_max;
  sh.n_special = 0;
  sh.global = 0;
  sh.layout = VK_QK_HEADS_OUTER;
  sh.ntok = vkd::make_fastdiv(static_cast<uint32_t>(rows));
  sh.tpv = sh.ntok;
  sh.per_view = vkd::make_fastdiv(static_cast<uint32_t>(heads * rows));
  sh.gw = vkd::make_fastdiv(1);
  return sh;
}

int check_qk_params(const vk_tensor* qg, const vk_tensor* qb, const vk_tensor* kg,
                    const vk_tensor* kb, size_t head_dim) {
  const bool any = qg || qb || kg || kb;
  const bool all = qg && qb && kg && kb;
  VK_REQUIRE(!any || all, "q/k norm parameters must be all present or all null");
  if (all) {
    VK_REQUIRE(param_ok(qg, head_dim) && param_ok(qb, head_dim) && param_ok(kg, head_dim) &&
                   param_ok(kb, head_dim),
               "q/k norm parameters must be f32 or f16 vectors of head_dim=%zu", head_dim);
    VK_REQUIRE(qg->dtype == qb->dtype && qg->dtype == kg->dtype && qg->dtype == kb->dtype,
               "q/k norm parameters must share one dtype");
  }
  return VK_OK;
}

}  // namespace

namespace vk {

int layernorm_raw(vk_runtime* rt, const float* x, float* y, const void* gamma, const void* beta,
                  bool f16, int rows, int cols, float eps) {
  if (rows == 0) return VK_OK;
  return f16 ? launch_layernorm<uint16_t>(rt, x, y, gamma, beta, rows, cols, eps)
             : launch_layernorm<float>(rt, x, y, gamma, beta, rows, cols, eps);
}

int layernorm_stats_sequential(vk_runtime* rt, const float* x, float* stats, int rows, int cols,
                               float eps, int np, int n, int ns) {
  if (rows == 0) return VK_OK;
  int nv = 0;
  SeqLnArgs a = seq_args(const_cast<float*>(x), rows, cols, eps, &nv);
  a.stats = reinterpret_cast<float2*>(stats);
  a.np = np;
  a.n = n;
  a.ns = ns;
  a.fnp = vkd::make_fastdiv(static_cast<uint32_t>(np > 0 ? np : 1));
  return launch_seq<float, false, false, false>(rt, a, nv);
}

}  // namespace vk

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int vk_layernorm_into_f32(vk_runtime* rt, const vk_tensor* x, const vk_tensor* gamma,
                          const vk_tensor* beta, size_t rows, size_t cols, float eps,
                          vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(x && out, "null tensor");
  VK_REQUIRE(x->dtype == VK_F32 && out->dtype == VK_F32, "layernorm activations must be f32");
  VK_REQUIRE(x->len == rows * cols && out->len == rows * cols,
             "layernorm: x (%zu) / out (%zu) must hold rows*cols=%zu", x->len, out->len,
             rows * cols);
  VK_REQUIRE(param_ok(gamma, cols) && param_ok(beta, cols) && gamma->dtype == beta->dtype,
             "layernorm: gamma/beta must be f32 or f16 vectors of cols=%zu", cols);
  VK_UNSUPPORTED_IF(cols == 0 || cols % 4 != 0 || cols > 8192,
                    "layernorm: cols=%zu (need a multiple of 4 up to 8192)", cols);
  VK_UNSUPPORTED_IF(rows > 0x7fffffffULL, "layernorm: rows=%zu too large", rows);
  if (rows == 0) return VK_OK;
  const float* X = static_cast<const float*>(x->ptr);
  float* Y = static_cast<float*>(out->ptr);
  const int r = static_cast<int>(rows), c = static_cast<int>(cols);
  VK_UNSUPPORTED_IF(ln_instance_cols(c) < 0, "layernorm: cols=%zu", cols);
  if (gamma->dtype == VK_F16)
    return launch_layernorm<uint16_t>(rt, X, Y, gamma->ptr, beta->ptr, r, c, eps);
  return launch_layernorm<float>(rt, X, Y, gamma->ptr, beta->ptr, r, c, eps);
}

int vk_layernorm_f32(vk_runtime* rt, const vk_tensor* x, const vk_tensor* gamma,
                     const vk_tensor* beta, size_t rows, size_t cols, float eps,
                     vk_tensor** out) {
  VK_REQUIRE(out != nullptr, "null output handle");
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, rows * cols, &t));
  int s = vk_layernorm_into_f32(rt, x, gamma, beta, rows, cols, eps, t);
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

int vk_layerscale_residual_layernorm_f32(vk_runtime* rt, vk_tensor* x, const vk_tensor* y,
                                         const vk_tensor* ls_gamma,
                                         const vk_tensor* ln_gamma,
                                         const vk_tensor* ln_beta, size_t rows,
                                         size_t cols, float eps, vk_tensor* ln_out) {
  return vk::ls_residual_layernorm_camera(rt, x, y, ls_gamma, ln_gamma, ln_beta, rows, cols, eps,
                                          ln_out, nullptr, 0);
}

}  // extern "C"

namespace vk {

int ls_residual_layernorm_camera(vk_runtime* rt, vk_tensor* x, const vk_tensor* y,
                                 const vk_tensor* ls_gamma, const vk_tensor* ln_gamma,
                                 const vk_tensor* ln_beta, size_t rows, size_t cols, float eps,
                                 vk_tensor* ln_out, const vk_tensor* camera,
                                 size_t tokens_per_view) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(x && y && ln_out, "null tensor");
  VK_REQUIRE(x->dtype == VK_F32 && y->dtype == VK_F32 && ln_out->dtype == VK_F32,
             "activations must be f32");
  VK_REQUIRE(x->len == rows * cols && y->len == rows * cols && ln_out->len == rows * cols,
             "x, y and ln_out must hold rows*cols=%zu", rows * cols);
  VK_REQUIRE(x->ptr != y->ptr && x->ptr != ln_out->ptr && y->ptr != ln_out->ptr,
             "x, y and ln_out must be distinct buffers");
  VK_REQUIRE(param_ok(ln_gamma, cols) && param_ok(ln_beta, cols) &&
                 ln_gamma->dtype == ln_beta->dtype,
             "LayerNorm gamma/beta must be f32 or f16 vectors of cols=%zu", cols);
  VK_REQUIRE(!ls_gamma || (param_ok(ls_gamma, cols) && ls_gamma->dtype == ln_gamma->dtype),
             "LayerScale gamma must be a vector of cols=%zu with the LayerNorm dtype", cols);
  VK_UNSUPPORTED_IF(cols == 0 || cols % 4 != 0 || cols > 8192 || ln_instance_cols(static_cast<int>(cols)) < 0,
                    "ls_residual_layernorm: cols=%zu", cols);
  VK_UNSUPPORTED_IF(rows > 0x7fffffffULL, "rows=%zu too large", rows);
  if (camera) {
    VK_REQUIRE(camera->dtype == VK_F32, "camera token must be f32");
    VK_REQUIRE(tokens_per_view > 0 && rows % tokens_per_view == 0 &&
                   tokens_per_view <= 0x7fffffffULL,
               "rows=%zu is not a whole number of views of %zu tokens", rows, tokens_per_view);
    VK_REQUIRE(camera->len >= (rows > tokens_per_view ? 2 : 1) * cols,
               "camera token must hold %s (%zu f32)",
               rows > tokens_per_view ? "reference and source slots" : "one slot",
               (rows > tokens_per_view ? 2 : 1) * cols);
  }
  if (rows == 0) return VK_OK;
  float* X = static_cast<float*>(x->ptr);
  const float* Yb = static_cast<const float*>(y->ptr);
  float* O = static_cast<float*>(ln_out->ptr);
  const int r = static_cast<int>(rows), c = static_cast<int>(cols);
  const void* ls = ls_gamma ? ls_gamma->ptr : nullptr;
  const float* cam = camera ? static_cast<const float*>(camera->ptr) : nullptr;
  const int tpv = camera ? static_cast<int>(tokens_per_view) : 1;
  if (ln_gamma->dtype == VK_F16) {
    return ls ? launch_ls_res_ln<uint16_t, true>(rt, X, Yb, ls, ln_gamma->ptr, ln_beta->ptr, O, r, c, eps, cam, tpv)
              : launch_ls_res_ln<uint16_t, false>(rt, X, Yb, ls, ln_gamma->ptr, ln_beta->ptr, O, r, c, eps, cam, tpv);
  }
  return ls ? launch_ls_res_ln<float, true>(rt, X, Yb, ls, ln_gamma->ptr, ln_beta->ptr, O, r, c, eps, cam, tpv)
            : launch_ls_res_ln<float, false>(rt, X, Yb, ls, ln_gamma->ptr, ln_beta->ptr, O, r, c, eps, cam, tpv);
}

}  // namespace vk

extern "C" {

int vk_qk_norm_rope_mode_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k,
                             const vk_tensor* q_gamma, const vk_tensor* q_beta,
                             const vk_tensor* k_gamma, const vk_tensor* k_beta,
                             const vk_tensor* positions, size_t heads, size_t rows, float freq,
                             float eps, unsigned rope_mode) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(q && k && positions, "null tensor");
  VK_REQUIRE(q->dtype == VK_F32 && k->dtype == VK_F32, "q and k must be f32");
  VK_REQUIRE(positions_ok(positions), "positions must be f32, i32 or i64");
  const size_t head_dim = 64;
  VK_REQUIRE(heads > 0 && q->len == heads * rows * head_dim && k->len == q->len,
             "q/k must hold heads*rows*64 = %zu elements (q %zu, k %zu)",
             heads * rows * head_dim, q->len, k->len);
  VK_REQUIRE(positions->len == rows * 2, "positions must hold rows*2 = %zu (got %zu)",
             rows * 2, positions->len);
  VK_REQUIRE(q->ptr != k->ptr, "q and k must be distinct buffers");
  VK_TRY(check_qk_params(q_gamma, q_beta, k_gamma, k_beta, head_dim));
  VK_UNSUPPORTED_IF(2 * heads * rows > 0x7fffffffULL, "heads*rows=%zu too large", heads * rows);
  VK_TRY(vk::check_rope_mode(rope_mode));
  if (rows == 0) return VK_OK;
  const float* table = nullptr;
  int table_max = 0;
  VK_TRY(vk::rope_table(rt, freq, 64, rope_mode, 0, &table, &table_max));
  const QkShape sh = explicit_shape(heads, rows, table_max, 2);
  return dispatch_qk_explicit(rt, static_cast<float*>(q->ptr), static_cast<float*>(k->ptr),
                              q_gamma, q_beta, k_gamma, k_beta, positions, table, sh, eps,
                              rope_mode);
}

int vk_qk_norm_rope_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k, const vk_tensor* q_gamma,
                        const vk_tensor* q_beta, const vk_tensor* k_gamma,
                        const vk_tensor* k_beta, const vk_tensor* positions, size_t heads,
                        size_t rows, float freq, float eps) {
  VK_REQUIRE(positions == nullptr || positions->dtype == VK_F32, "positions must be f32");
  return vk_qk_norm_rope_mode_f32(rt, q, k, q_gamma, q_beta, k_gamma, k_beta, positions, heads,
                                  rows, freq, eps, VK_ROPE_DEFAULT);
}

int vk_rope2d_f32(vk_runtime* rt, vk_tensor* x, const vk_tensor* positions, size_t heads,
                  size_t rows, size_t head_dim, float freq, unsigned rope_mode) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(x && positions, "null tensor");
  VK_REQUIRE(x->dtype == VK_F32, "x must be f32");
  VK_REQUIRE(positions_ok(positions), "positions must be f32, i32 or i64");
  VK_UNSUPPORTED_IF(head_dim != 64, "rope2d: head_dim=%zu (qualified: 64)", head_dim);
  VK_REQUIRE(heads > 0 && x->len == heads * rows * head_dim,
             "x must hold heads*rows*64 = %zu elements (got %zu)", heads * rows * head_dim,
             x->len);
  VK_REQUIRE(positions->len == rows * 2, "positions must hold rows*2 = %zu (got %zu)",
             rows * 2, positions->len);
  VK_UNSUPPORTED_IF(heads * rows > 0x7fffffffULL, "heads*rows=%zu too large", heads * rows);
  VK_TRY(vk::check_rope_mode(rope_mode));
  if (rows == 0) return VK_OK;
  const float* table = nullptr;
  int table_max = 0;
  VK_TRY(vk::rope_table(rt, freq, 64, rope_mode, 0, &table, &table_max));
  const QkShape sh = explicit_shape(heads, rows, table_max, 1);
  float* X = static_cast<float*>(x->ptr);
  return dispatch_qk_explicit(rt, X, X, nullptr, nullptr, nullptr, nullptr, positions, table, sh,
                              0.0f, rope_mode);
}

int vk_qk_norm_rope_grid_mode_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k,
                                  const vk_tensor* q_gamma, const vk_tensor* q_beta,
                                  const vk_tensor* k_gamma, const vk_tensor* k_beta,
                                  size_t heads, size_t head_dim, size_t n_special, size_t gh,
                                  size_t gw, size_t view_count, int global,
                                  vk_qk_layout layout, float freq, float eps,
                                  unsigned rope_mode) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(q && k, "null tensor");
  VK_REQUIRE(q->dtype == VK_F32 && k->dtype == VK_F32, "q and k must be f32");
  VK_UNSUPPORTED_IF(head_dim != 64, "qk_norm_rope: head_dim=%zu (qualified: 64)", head_dim);
  VK_REQUIRE(layout == VK_QK_HEADS_OUTER || layout == VK_QK_VIEWS_OUTER, "unknown layout %d",
             static_cast<int>(layout));
  VK_REQUIRE(view_count > 0 && heads > 0 && gw > 0, "view_count, heads and gw must be > 0");
  const size_t tpv = n_special + gh * gw;
  const size_t rows = tpv * view_count;
  VK_REQUIRE(q->len == heads * rows * head_dim && k->len == q->len,
             "q/k must hold heads*view_count*(n_special+gh*gw)*64 = %zu (q %zu, k %zu)",
             heads * rows * head_dim, q->len, k->len);
  VK_REQUIRE(q->ptr != k->ptr, "q and k must be distinct buffers");
  VK_TRY(check_qk_params(q_gamma, q_beta, k_gamma, k_beta, head_dim));
  VK_UNSUPPORTED_IF(2 * heads * rows > 0x7fffffffULL, "heads*rows=%zu too large", heads * rows);
  VK_TRY(vk::check_rope_mode(rope_mode));
  if (rows == 0) return VK_OK;
  // the grid's largest coordinate is max(gh, gw) + 1: size the table to it
  const float* table = nullptr;
  int table_max = 0;
  const size_t max_coord = (gh > gw ? gh : gw) + 1;
  VK_UNSUPPORTED_IF(max_coord > (1u << 22), "patch grid %zux%zu too large", gh, gw);
  VK_TRY(vk::rope_table(rt, freq, 64, rope_mode, static_cast<int>(max_coord), &table,
                        &table_max));
  QkShape sh;
  sh.rows_per_tensor = static_cast<uint32_t>(heads * rows);
  sh.tensors = 2;
  sh.table_max = table_max;
  sh.n_special = static_cast<uint32_t>(n_special);
  sh.global = global ? 1u : 0u;
  sh.layout = static_cast<uint32_t>(layout);
  sh.ntok = vkd::make_fastdiv(static_cast<uint32_t>(rows));
  sh.tpv = vkd::make_fastdiv(static_cast<uint32_t>(tpv));
  sh.per_view = vkd::make_fastdiv(static_cast<uint32_t>(heads * tpv));
  sh.gw = vkd::make_fastdiv(static_cast<uint32_t>(gw));
  return dispatch_qk<kPosGrid>(rt, static_cast<float*>(q->ptr), static_cast<float*>(k->ptr),
                               q_gamma, q_beta, k_gamma, k_beta, nullptr, table, sh, eps,
                               rope_mode);
}

int vk_qk_norm_rope_grid_f32(vk_runtime* rt, vk_tensor* q, vk_tensor* k,
                             const vk_tensor* q_gamma, const vk_tensor* q_beta,
                             const vk_tensor* k_gamma, const vk_tensor* k_beta, size_t heads,
                             size_t head_dim, size_t n_special, size_t gh, size_t gw,
                             size_t view_count, int global, vk_qk_layout layout, float freq,
                             float eps) {
  return vk_qk_norm_rope_grid_mode_f32(rt, q, k, q_gamma, q_beta, k_gamma, k_beta, heads,
                                       head_dim, n_special, gh, gw, view_count, global, layout,
                                       freq, eps, VK_ROPE_DEFAULT);
}

int vk_rope_positions_f32(vk_runtime* rt, size_t n_special, size_t gh, size_t gw,
                          size_t view_count, int global, vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out != nullptr, "null output handle");
  VK_REQUIRE(gw > 0 && view_count > 0, "gw and view_count must be > 0");
  const size_t tpv = n_special + gh * gw;
  const size_t rows = tpv * view_count;
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, rows * 2, &t));
  if (rows > 0) {
    const unsigned blocks = static_cast<unsigned>((rows + 255) / 256);
    hipLaunchKernelGGL(rope_positions_kernel, dim3(blocks), dim3(256), 0, rt->stream,
                       static_cast<float*>(t->ptr), static_cast<long long>(rows),
                       static_cast<int>(tpv), static_cast<int>(n_special),
                       static_cast<int>(gw), global ? 1 : 0);
    int s = vk::check_launch("rope_positions_kernel");
    if (s != VK_OK) {
      vk_tensor_destroy(t);
      return s;
    }
  }
  *out = t;
  return VK_OK;
}

}  // extern "C"
