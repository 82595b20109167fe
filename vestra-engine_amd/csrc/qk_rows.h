// Per-row Q/K LayerNorm (head_dim 64) + 2D RoPE on a 16-lane DPP row that
// holds the 64 values as one float4 per lane (lane l: elements 4l..4l+3).
// Shared by the Q/K kernel and the QKV projection's fused epilogue, so the
// two give the same bits for the same row.
#pragma once

#include "common.h"

namespace vkq {

// Where a row's position comes from: a positions tensor [tokens*2] (y, x)
// of f32 (the CUDA runtime's device encoding), i32 or i64 (the CPU kernels'
// integer positions), or the patch grid.
enum PosMode { kPosExplicit = 0, kPosGrid = 1, kPosExplicitI32 = 2, kPosExplicitI64 = 3 };

// RoPE pairing inside each 32-wide half: element j with j + 16 (rotate-half)
// or element 2i with 2i + 1 (interleaved).
enum Pairing { kRotateHalf = 0, kInterleaved = 1 };

struct QkShape {
  uint32_t rows_per_tensor;  // heads * total tokens; 2 * rows_per_tensor < 2^31
  uint32_t tensors;          // 2: Q then K; 1: Q only (the rotation of one tensor)
  int table_max;             // largest position the cos/sin table covers
  uint32_t n_special;
  uint32_t global;
  uint32_t layout;           // vk_qk_layout
  vkd::FastDivU32 ntok;      // total tokens (view_count * tokens_per_view)
  vkd::FastDivU32 tpv;       // tokens per view
  vkd::FastDivU32 per_view;  // heads * tokens per view
  vkd::FastDivU32 gw;        // patch grid width
};

// cos/sin of the frequencies j0..j0+NF-1 for a coordinate outside the
// table (positions past 1023, or negative): the same f32 angle as the table,
// its cosine and sine from the device's single-precision sincosf (within 2
// ulp of the table's double-rounded values).  Only the explicit-position
// forms can meet such a coordinate (grid forms size the table on the host).
// Double-precision trig here, out of line or inline, took the streaming
// kernel's register footprint from ~45 to ~100 VGPRs and every launch with
// explicit positions 12% longer, whether or not a coordinate left the table.
struct RopeCs {
  float4 c, s;  // components 0..NF-1
};
template <int NF>
__device__ __forceinline__ RopeCs rope_cs_slow(const float* __restrict__ table, int table_max,
                                               float p, int j0) {
  float cv[4] = {0.f, 0.f, 0.f, 0.f}, sv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < NF; ++u) {
    const float inv_freq = table[static_cast<size_t>(table_max + 1) * 32 + j0 + u];
    const float angle = p * inv_freq;
    sincosf(angle, &sv[u], &cv[u]);
  }
  return RopeCs{make_float4(cv[0], cv[1], cv[2], cv[3]), make_float4(sv[0], sv[1], sv[2], sv[3])};
}

__device__ __forceinline__ float4 swizzle_xor4(float4 v) {
  // ds_swizzle bit-mask mode: and_mask 0x1f, or_mask 0, xor_mask 4.
  constexpr int pat = (4 << 10) | 0x1f;
  float4 r;
  r.x = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v.x), pat));
  r.y = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v.y), pat));
  r.z = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v.z), pat));
  r.w = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v.w), pat));
  return r;
}

// Position (y, x) of token lt of a view (vit_block.rs:841-881): specials
// (0, 0); patch p at (p / gw + 1, p % gw + 1), or (1, 1) in global layers.
__device__ __forceinline__ void grid_position(uint32_t lt, uint32_t n_special, uint32_t global,
                                              const vkd::FastDivU32& gw, float* py, float* px) {
  int y = 0, x = 0;
  if (lt >= n_special) {
    if (global) {
      y = 1;
      x = 1;
    } else {
      const uint32_t p = lt - n_special;
      const uint32_t row = vkd::fdiv(p, gw);
      y = static_cast<int>(row) + 1;
      x = static_cast<int>(p - row * gw.d) + 1;
    }
  }
  *py = static_cast<float>(y);
  *px = static_cast<float>(x);
}

// An f32 device position as the reference's `value as i64` reads it, then
// as the f32 the angle is computed from: truncated toward zero, NaN to 0,
// saturated at +-2^63 (the f32 nearest i64::MAX / i64::MIN).
__device__ __forceinline__ float f32_position(float v) {
  if (v != v) return 0.0f;
  return fminf(fmaxf(truncf(v), -9223372036854775808.0f), 9223372036854775808.0f);
}

// Position (y, x) of Q/K row r (head-major index inside one tensor), as the
// f32 value the rotation angle is computed from: an integer position p
// gives (float)p exactly as the CPU kernel converts its i64 positions, so a
// coordinate of any i64 value (2^32 + 5 included) takes the rotation of
// that f32 value -- through the table when it is an entry of it, through
// sincosf otherwise.  All index math is 32-bit with multiply-shift division
// by the shape constants.
template <int POS>
__device__ __forceinline__ void qk_row_position(uint32_t r, const QkShape& sh,
                                                const void* __restrict__ pos_yx, float* py,
                                                float* px) {
  uint32_t t;   // index in the position sequence
  uint32_t lt;  // index inside its view
  if (sh.layout == VK_QK_HEADS_OUTER) {
    t = vkd::fmod_(r, sh.ntok);
    lt = vkd::fmod_(t, sh.tpv);
  } else {
    const uint32_t v = vkd::fdiv(r, sh.per_view);
    lt = vkd::fmod_(r, sh.tpv);
    t = v * sh.tpv.d + lt;
  }
  if (POS == kPosExplicit) {
    // the reference's f32 device encoding, truncated like `value as i64`
    const float* p = static_cast<const float*>(pos_yx);
    *py = f32_position(p[2 * static_cast<size_t>(t)]);
    *px = f32_position(p[2 * static_cast<size_t>(t) + 1]);
  } else if (POS == kPosExplicitI32) {
    const int2 p = static_cast<const int2*>(pos_yx)[t];
    *py = static_cast<float>(p.x);
    *px = static_cast<float>(p.y);
  } else if (POS == kPosExplicitI64) {
    const long long* p = static_cast<const long long*>(pos_yx);
    *py = static_cast<float>(p[2 * static_cast<size_t>(t)]);
    *px = static_cast<float>(p[2 * static_cast<size_t>(t) + 1]);
  } else {
    grid_position(lt, sh.n_special, sh.global, sh.gw, py, px);
  }
}

// The per-row operands of the transform below: the lane's LayerNorm gamma
// and beta (four elements each) and the cos/sin of its rotated pairs (four
// frequencies with rotate-half pairing, two with interleaved pairing).
// Loading them is a stage of its own, so a caller holding several rows can
// issue every row's loads before any row's arithmetic.
// A lane's four LayerNorm parameters (64 per row, F32 or F16) by a raw
// buffer load: a buffer load holds up the wave's other instructions less
// than a 64-bit address load (measured on this kernel: 23.6 against 24.1 us
// at 12 views of 10,392 rows).
template <typename PT>
__device__ __forceinline__ float4 qk_param4(const PT* p, int l) {
  const __amdgpu_buffer_rsrc_t r = vkd::buffer_rsrc(p, 64 * sizeof(PT));
  if constexpr (sizeof(PT) == 4) {
    return vkd::buffer_load4(r, 16u * l, 0);
  } else {
    typedef int i32x2_t __attribute__((ext_vector_type(2)));
    const i32x2_t h = __builtin_amdgcn_raw_buffer_load_b64(r, 8 * l, 0, 0);
    const uint32_t a = static_cast<uint32_t>(h.x), b = static_cast<uint32_t>(h.y);
    return make_float4(vkd::f16_to_f32(static_cast<uint16_t>(a & 0xffffu)),
                       vkd::f16_to_f32(static_cast<uint16_t>(a >> 16)),
                       vkd::f16_to_f32(static_cast<uint16_t>(b & 0xffffu)),
                       vkd::f16_to_f32(static_cast<uint16_t>(b >> 16)));
  }
}

struct QkRowOperands {
  float4 g, b;  // LayerNorm parameters (unused without the norm)
  float4 c, s;  // cos/sin: components 0..3 (rotate-half) or 0..1 (interleaved)
};

template <typename PT, bool HAS_NORM, int POS, int PAIR>
__device__ __forceinline__ QkRowOperands qk_row_operands(int l, const PT* __restrict__ g,
                                                         const PT* __restrict__ b, float py,
                                                         float px,
                                                         const float* __restrict__ table,
                                                         int table_max) {
  QkRowOperands o;
  if (HAS_NORM) {
    o.g = qk_param4(g, l);
    o.b = qk_param4(b, l);
  }
  // lanes 0-7 rotate by the row coordinate, lanes 8-15 by the column
  // the coordinate is an integral f32: an entry of the table when it lies
  // in 0..table_max (exactly representable, so the comparison is exact)
  const float coord = (l < 8) ? py : px;
  const bool in_table =
      POS == kPosGrid || (coord >= 0.0f && coord <= static_cast<float>(table_max));
  const uint32_t eo = static_cast<uint32_t>(in_table ? static_cast<int>(coord) : 0) * 128u;
  if (PAIR == kRotateHalf) {
    const int j0 = (l & 3) * 4;  // frequencies j0..j0+3
    if (in_table) {
      // the table row by raw buffer loads, like the parameters
      const __amdgpu_buffer_rsrc_t tr =
          vkd::buffer_rsrc(table, static_cast<uint32_t>(table_max + 1) * 32u * 4u);
      o.c = vkd::buffer_load4(tr, eo + 4u * j0, 0);
      o.s = vkd::buffer_load4(tr, eo + 4u * j0, 64);
    } else {
      const RopeCs cs = rope_cs_slow<4>(table, table_max, coord, j0);
      o.c = cs.c;
      o.s = cs.s;
    }
  } else {
    const int j0 = (l & 7) * 2;  // frequencies j0, j0+1
    float2 c, sn;
    if (in_table) {
      typedef int i32x2_t __attribute__((ext_vector_type(2)));
      const __amdgpu_buffer_rsrc_t tr =
          vkd::buffer_rsrc(table, static_cast<uint32_t>(table_max + 1) * 32u * 4u);
      c = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(tr, eo + 4u * j0, 0, 0));
      sn = __builtin_bit_cast(float2,
                              __builtin_amdgcn_raw_buffer_load_b64(tr, eo + 4u * j0, 64, 0));
    } else {
      const RopeCs cs = rope_cs_slow<2>(table, table_max, coord, j0);
      c = make_float2(cs.c.x, cs.c.y);
      sn = make_float2(cs.s.x, cs.s.y);
    }
    o.c = make_float4(c.x, c.y, 0.0f, 0.0f);
    o.s = make_float4(sn.x, sn.y, 0.0f, 0.0f);
  }
  return o;
}

// (v - mean) * inv * gamma + beta for the lane's four elements, each step
// rounded.
__device__ __forceinline__ float4 qk_norm_apply(float4 v, float mean, float inv,
                                                const QkRowOperands& op) {
  v.x = (v.x - mean) * inv * op.g.x + op.b.x;
  v.y = (v.y - mean) * inv * op.g.y + op.b.y;
  v.z = (v.z - mean) * inv * op.g.z + op.b.z;
  v.w = (v.w - mean) * inv * op.g.w + op.b.w;
  return v;
}

// The 2D rotation of one 64-wide row held as one float4 per lane of a
// 16-lane DPP row, with the cos/sin of qk_row_operands.  Lanes 0-7 hold the
// y half (elements 0..31), lanes 8-15 the x half.  Every rotated pair
// (a, b) with angle frequency j becomes (a*cos - b*sin, b*cos + a*sin),
// each product rounded, then the sum.
template <int PAIR>
__device__ __forceinline__ float4 qk_row_rope(float4 v, int l, const QkRowOperands& op) {
  const float4 c = op.c, s = op.s;
  float4 o;
  if (PAIR == kRotateHalf) {
    // Inside a half, lanes with bit 2 clear hold elements j (j < 16) and
    // rotate against the lane 4 above, which holds element j + 16.
    const float4 p = swizzle_xor4(v);
    if ((l & 4) == 0) {
      // out[j] = x[j]*cos - x[j+16]*sin
      o.x = v.x * c.x + (-p.x) * s.x;
      o.y = v.y * c.y + (-p.y) * s.y;
      o.z = v.z * c.z + (-p.z) * s.z;
      o.w = v.w * c.w + (-p.w) * s.w;
    } else {
      // out[j+16] = x[j+16]*cos + x[j]*sin
      o.x = v.x * c.x + p.x * s.x;
      o.y = v.y * c.y + p.y * s.y;
      o.z = v.z * c.z + p.z * s.z;
      o.w = v.w * c.w + p.w * s.w;
    }
  } else {
    // The lane's four elements 4m..4m+3 of its half are the pairs 2m and
    // 2m + 1: no lane exchange.
    o.x = v.x * c.x + (-v.y) * s.x;
    o.y = v.y * c.x + v.x * s.x;
    o.z = v.z * c.y + (-v.w) * s.y;
    o.w = v.w * c.y + v.z * s.y;
  }
  return o;
}

// LayerNorm of one 64-wide row (the tree order: each lane's four values,
// then the 16-lane DPP sum) and then its rotation, with the operands of
// qk_row_operands.
template <bool HAS_NORM, int PAIR>
__device__ __forceinline__ float4 qk_row_apply(float4 v, int l, const QkRowOperands& op,
                                               float eps) {
  if (HAS_NORM) {
    float s = v.x;
    s += v.y;
    s += v.z;
    s += v.w;
    s = vkd::row16_sum(s);
    const float mean = s / 64.0f;
    float d, sq;
    d = v.x - mean; sq = d * d;
    d = v.y - mean; sq += d * d;
    d = v.z - mean; sq += d * d;
    d = v.w - mean; sq += d * d;
    sq = vkd::row16_sum(sq);
    const float var = sq / 64.0f;
    // hardware reciprocal square root (v_rsq_f32, 1 ulp): the correctly
    // rounded 1/sqrtf costs ~18 VALU instructions per row
    const float inv = __builtin_amdgcn_rsqf(var + eps);
    v = qk_norm_apply(v, mean, inv, op);
  }
  return qk_row_rope<PAIR>(v, l, op);
}

// Both stages for one row (the QKV projection's epilogue).
template <typename PT, bool HAS_NORM, int POS, int PAIR>
__device__ __forceinline__ float4 qk_row_transform(float4 v, int l, const PT* __restrict__ g,
                                                   const PT* __restrict__ b, float py, float px,
                                                   const float* __restrict__ table,
                                                   int table_max, float eps) {
  const QkRowOperands op =
      qk_row_operands<PT, HAS_NORM, POS, PAIR>(l, g, b, py, px, table, table_max);
  return qk_row_apply<HAS_NORM, PAIR>(v, l, op, eps);
}

}  // namespace vkq
