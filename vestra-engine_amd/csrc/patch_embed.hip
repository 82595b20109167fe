// Fused patch embedding for gfx950: the 14x14 / stride-14 patch convolution
// of the u8 image, and the reference-shaped split entries around it
// (patchify, CLS + position add, the bicubic position table).
//
// The convolution is a GEMM
//   tokens[p, e] = sum_k A[p, k] * W[e, k] + b[e]
// with A the normalised, unfolded image.  Both kernels below do it all in
// one pass: A is taken straight from the u8 HWC image and normalised
// through a 3x256 lookup table in LDS (the table holds exactly
// (u8/255 - mean)/std, so the normalisation is bit-identical to the scalar
// path), the filter is read from a copy of its rows reordered at prepare
// time to the image's byte order (prepare_patch_filter below), the products
// run on v_mfma_f32_16x16x4_f32 (F32 in, F32 accumulate), and the epilogue
// adds the bias and the position table and writes the assembled token rows
// (CLS + pos[0], register rows, patch rows) so nothing round-trips through
// HBM.  patch_embed_gather_kernel takes one image (or a few views),
// patch_embed_pipelined_kernel the many tiles of a multi-view batch; both
// give every output element the same operation order, so a view's tokens
// have the same bits whichever kernel computes them.
#include "common.h"
#include "mfma_f32.h"

#include <type_traits>

namespace {

using vkd::xcd_tile;
using namespace vkm;

#ifndef VK_PE_PIPELINED
#define VK_PE_PIPELINED 1  // multi-view launches: the pipelined kernel
#endif

constexpr int kPatch = 14;

// ---------------------------------------------------------------------------
// K is taken in the image's own order, k = ky*42 + kx*3 + c (the filter is
// reordered to match at prepare time), so one patch row is 42 contiguous
// bytes of the HWC image and 42 consecutive k.  K is padded to 592 = 37
// blocks of 16.  In block b, lane group g = lane / 16 holds k = 16 b + 4 g + j
// in component j of one fragment read, and MFMA step j multiplies component
// j.  The operation order every output element follows: two k halves, each
// a chain of blocks in one accumulator -- half 0 blocks 0-9, 21-28 and then
// 10, half 1 blocks 11-20 and 29-36 -- then (half 0 + half 1), + bias,
// + position.
// ---------------------------------------------------------------------------
constexpr int kPeRowBytes = 3 * kPatch;    // 42 bytes per patch row
constexpr int kPeK = kPatch * kPeRowBytes; // 588
constexpr int kPeKp = 592;                 // 37 blocks of 16
constexpr int kPeBlocks = kPeKp / 16;
constexpr int kPeBlocksA = 8 * kPeRowBytes / 16;         // 21: blocks of pixel rows 0-7
constexpr int kPePhase1 = kPeBlocksA / 2;                // 10: half 0 blocks 0-9, half 1 11-20
constexpr int kPePhase2 = (kPeBlocks - kPeBlocksA) / 2;  // 8: half 0 21-28, half 1 29-36
constexpr int kPeSeq = kPePhase1 + kPePhase2 + 1;        // + half 0's last block, 10
constexpr int kPePitch = 596;              // normalised A row pitch in LDS: 4 x 149
constexpr int kPeStagers = 256;            // staging waves of the pipelined kernel
constexpr int kPeThreads = kThreads + kPeStagers;
static_assert(kPeKp % 16 == 0 && kPeKp >= kPeK && kPeKp == (kPeK + kKAlign - 1) / kKAlign * kKAlign,
              "weight rows padded to a 16-block");
static_assert(kPeBlocksA == 2 * kPePhase1 + 1 && kPeBlocks - kPeBlocksA == 2 * kPePhase2,
              "block split");
static_assert(3 * 256 == kPeThreads, "one table entry per thread of the pipelined kernel");
static_assert(kPePitch % 4 == 0 && (kPePitch / 4) % 2 == 1 && kPePitch >= kPeKp, "pitch 4 x odd");

struct PatchArgs {
  const uint8_t* img;  // [views, H, W, 3], 8-byte aligned views
  const float* wpk;    // [N, 592], k = ky*42 + kx*3 + c, zero beyond 588
  const float* bias;   // [N]
  const float* pos;    // [(1 + M), N]
  const float* cls;    // [N]
  const float* regs;   // [n_register, N] or null
  float* out;          // [views, (1 + n_register + M), N]
  uint32_t img_bytes;  // H*W*3 of one view, a multiple of 4
  int tiles;           // output tiles of one view
  int views;
  int W, gw, M, N, n_register;
  vkd::FastDivU32 fgw;  // division by gw
  float mean[3], sd[3];
};

// One patch row: its 42 bytes, starting at byte `st` of the image, read as
// five aligned 8-byte words and two 4-byte words (48 bytes from st rounded
// down to 8; st is even, so that covers st..st+41), then funnel-shifted so
// that dword i holds row bytes 4i..4i+3, normalised through the table and
// written to A[m][ky*42 ..] two floats at a time.  Every read stays inside
// the image: the last word is clamped and is only consumed when it lies
// inside.
struct PatchRow {
  uint32_t w[12];
  uint32_t s8;
  __device__ __forceinline__ void load(const uint8_t* img, uint32_t st, uint32_t img_bytes) {
    const uint32_t a8 = st & ~7u;
    s8 = st & 7u;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      const uint2 v = *reinterpret_cast<const uint2*>(img + a8 + 8 * j);
      w[2 * j] = v.x;
      w[2 * j + 1] = v.y;
    }
    w[10] = *reinterpret_cast<const uint32_t*>(img + a8 + 40);
    const uint32_t a44 = a8 + 44 <= img_bytes - 4 ? a8 + 44 : img_bytes - 4;
    w[11] = *reinterpret_cast<const uint32_t*>(img + a44);
  }
  // w[i] (i < 11) := row bytes 4i..4i+3 (bytes 42, 43 are padding)
  __device__ __forceinline__ void align() {
    const bool dw = s8 >= 4;
    const uint32_t sh = s8 & 3u;
    uint32_t t[12];
#pragma unroll
    for (int i = 0; i < 11; ++i) t[i] = dw ? w[i + 1] : w[i];
    t[11] = dw ? 0u : w[11];
#pragma unroll
    for (int i = 0; i < 11; ++i) w[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh);
  }
  // pairs q0 <= q < q1 of the aligned row (pair q = bytes 2q, 2q+1)
  __device__ __forceinline__ void store(float2* dst, const float* lut, int q0, int q1) const {
#pragma unroll
    for (int q = q0; q < q1; ++q) {
      const int b = 2 * q;
      const uint32_t v0 = (w[b >> 2] >> (8 * (b & 3))) & 0xffu;
      const uint32_t v1 = (w[(b + 1) >> 2] >> (8 * ((b + 1) & 3))) & 0xffu;
      dst[q] = make_float2(lut[(b % 3) * 256 + v0], lut[((b + 1) % 3) * 256 + v1]);
    }
  }
};

// ---------------------------------------------------------------------------
// Gathered patch embedding, for one image (and launches of few views).
// Tiles are 32 patches x 96 outputs (a 336 x 504 image: 27 x 8 = 216
// workgroups, numbered XCD-major, so each XCD's L2 holds one 96-column slice
// of the filter).  The A tile stays in LDS as the table address of every
// element (the byte offset 4 v + 1024 c), written straight from the image
// bytes; the MFMA waves read their fragments' addresses and gather the
// normalised values from the table themselves.  So the MFMAs start as soon
// as the address tile and the table are in LDS: there is no normalised tile
// to build first, and no wave stages while the MFMAs run.  Eight waves, two
// per SIMD: wave w takes patches 16 (w % 2) .. +16, the three 16-column
// strips 3 ((w / 2) % 2) .. +3 and k half w / 4 (each SIMD runs one wave of
// either half: 19 + 18 blocks), and one gathered fragment feeds three
// strips.  Every output element takes the block sequence, k-half split and
// epilogue order above.
//
// Addresses are held as u32 (91 KB of LDS, one workgroup per CU: a launch
// of one round of tiles, and four addresses per 128-bit read) or as u16
// (54 KB, two workgroups per CU for launches of several rounds; four
// addresses per 64-bit read, split one block after the read).
// ---------------------------------------------------------------------------
constexpr int kGm = 32;           // patches per tile
constexpr int kGn = 96;           // outputs per tile
constexpr int kGThreads = 512;
constexpr int kGZero = 3 * 256;   // table entry 768 holds 0: the K padding's address
constexpr int kGAhead = 3;        // B fragments this many blocks ahead
constexpr int kGLook = 2;         // gathered values this many blocks ahead, addresses one more
static_assert(kGm * kPatch <= kGThreads && kGThreads - kGm * kPatch >= 2 * kGm,
              "one patch row per staging thread; the padding by the others");
static_assert(kGn == 6 * 16 && kGm == 2 * 16, "waves: 2 patch strips x 2 k halves x 2 column groups");

template <bool U16>
struct GatherTile {
  typedef typename std::conditional<U16, uint16_t, uint32_t>::type Addr;
  static constexpr int kPitch = U16 ? 600 : 596;  // addresses per patch in LDS
};
static_assert(GatherTile<false>::kPitch >= kPeKp && GatherTile<false>::kPitch % 4 == 0 &&
                  (GatherTile<false>::kPitch / 4) % 2 == 1,
              "u32: 128-bit reads of 16 patches start on 16 distinct 4-bank groups");
static_assert(GatherTile<true>::kPitch >= kPeKp && GatherTile<true>::kPitch % 4 == 0,
              "u16: 64-bit reads aligned");
typedef uint32_t __attribute__((may_alias)) u32_alias;

// Block s of a k half's sequence (the order above): positions
// 0-9 are blocks first1 + s, positions 10-17 blocks first2 + s - 10, and
// half 0's position 18 is block 10.  Both halves run the same code (one
// instruction stream through the instruction cache: two streams measured
// slower) with two base pointers per operand, so every block offset is an
// immediate.
constexpr int kGSeg = kPePhase1;               // positions in the first segment
constexpr int kGSeg2 = kPePhase1 + kPePhase2;  // end of the second

template <bool U16>
__global__ __launch_bounds__(kGThreads) void patch_embed_gather_kernel(PatchArgs p) {
  using Addr = typename GatherTile<U16>::Addr;
  constexpr int kPitch = GatherTile<U16>::kPitch;
  // one LDS block with the table first, at offset 0: the gathers' addresses
  // then fit the LDS instructions' 16-bit offset field (no address adds)
  __shared__ struct __align__(16) {
    float lut[3 * 256 + 4];
    Addr At[kGm * kPitch];
    float red[4 * 12 * 64];
  } sm;
  float* const lut = sm.lut;
  Addr* const At = sm.At;
  float* const red = sm.red;
  // every argument the first addresses and the epilogue need, fetched in
  // one batch (each fetch otherwise waits for the one before it)
  asm volatile("" ::"s"(p.img), "s"(p.wpk), "s"(p.bias), "s"(p.pos), "s"(p.out),
               "s"(p.img_bytes), "s"(p.tiles), "s"(p.W), "s"(p.gw), "s"(p.M), "s"(p.N),
               "s"(p.n_register), "s"(p.fgw.m), "s"(p.fgw.s1), "s"(p.fgw.s2), "s"(gridDim.x));
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rs = wave & 1, cg = (wave >> 1) & 1, half = wave >> 2;
  const int first1 = half ? kPePhase1 + 1 : 0;
  const int first2 = kPeBlocksA + half * kPePhase2;
  const int len = half ? kPeSeq - 1 : kPeSeq;
  const int g = lane >> 4;
  const int gmt = (p.M + kGm - 1) / kGm;
  const int tile_all = xcd_tile(blockIdx.x, gridDim.x);
  const int view = tile_all / p.tiles;
  const int tile = tile_all - view * p.tiles;
  const uint8_t* const img = p.img + static_cast<size_t>(view) * p.img_bytes;
  float* out = p.out + static_cast<size_t>(view) * (1 + p.n_register + p.M) * p.N;
  int mt = tile % gmt;
  int m0 = mt * kGm, n0 = (tile / gmt) * kGn;
  // computed once: the epilogue would otherwise redo the divisions
  asm volatile("" : "+s"(out), "+s"(mt), "+s"(m0), "+s"(n0));

  // 1. patch row (m, ky) = (tid % 32, tid / 32) for tid < 448 (patches past
  // the image clamp to the last one: their rows are never stored)
  const bool stg = tid < kGm * kPatch;
  PatchRow row;
  if (stg) {
    const int gm = m0 + (tid & 31);
    const int cm = gm < p.M ? gm : p.M - 1;
    const uint32_t py = vkd::fdiv(static_cast<uint32_t>(cm), p.fgw);
    const uint32_t px = static_cast<uint32_t>(cm) - py * static_cast<uint32_t>(p.gw);
    row.load(img, ((py * kPatch + (tid >> 5)) * static_cast<uint32_t>(p.W) + px * kPatch) * 3u,
             p.img_bytes);
  }

  // 2. the table, exactly (v/255 - mean[c]) / std[c] (mean and std taken
  // from the scalar arguments: an indexed load of them would wait behind the
  // image rows), and its zero entry
  float mean[3], sd[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    mean[c] = p.mean[c];
    sd[c] = p.sd[c];
    asm volatile("" : "+s"(mean[c]), "+s"(sd[c]));  // kept in SGPRs, not reloaded
  }
  for (int e = tid; e < 3 * 256; e += kGThreads) {
    const int c = e / 256, v = e % 256;
    const float mc = c == 0 ? mean[0] : (c == 1 ? mean[1] : mean[2]);
    const float sc = c == 0 ? sd[0] : (c == 1 ? sd[1] : sd[2]);
    const float u = static_cast<float>(v) / 255.0f;
    lut[e] = (u - mc) / sc;
  }
  if (tid == 0) lut[kGZero] = 0.0f;

  // 3. B fragments of this wave's three column strips, first blocks: raw
  // buffer loads (a lane byte offset per strip and segment, the block's
  // offset an immediate), which hold up the MFMA issue less than 64-bit
  // address loads (a microbenchmark of this loop: 34.2 against 36.8 cycles
  // per MFMA with three fragment loads per 12 MFMAs)
  const __amdgpu_buffer_rsrc_t wsrc =
      vkd::buffer_rsrc(p.wpk, static_cast<uint32_t>(p.N) * kPeKp * 4u);
  uint32_t wrow[3][2];
#pragma unroll
  for (int cs = 0; cs < 3; ++cs) {
    const int col = n0 + 48 * cg + 16 * cs + (lane & 15);
    const uint32_t ccol = static_cast<uint32_t>(col < p.N ? col : p.N - 1);
    const uint32_t w = (ccol * kPeKp + 4 * g) * 4u;
    wrow[cs][0] = w + 64u * first1;
    wrow[cs][1] = w + 64u * first2;
  }
  // position s's operand: segment base + immediate offset (position 18 is
  // block 10 from the first segment's base, which is block 0 in half 0)
  auto seg = [](int s) { return s < kGSeg ? 0 : (s < kGSeg2 ? 1 : 0); };
  auto off = [](int s) { return s < kGSeg ? s : (s < kGSeg2 ? s - kGSeg : kPePhase1); };
  auto valid = [&](int s) { return s < kGSeg2 || (s < kPeSeq && len == kPeSeq); };
  f32x4 bf[kPeSeq][3];
  auto load_b = [&](int s) {
    if (valid(s)) {
#pragma unroll
      for (int cs = 0; cs < 3; ++cs)
        bf[s][cs] = __builtin_bit_cast(f32x4, vkd::buffer_load4(wsrc, wrow[cs][seg(s)], 64u * off(s)));
    }
  };
#pragma unroll
  for (int s = 0; s < kGAhead; ++s) load_b(s);

  // 4. the address tile: row (m, ky)'s 42 bytes -> byte offsets 4 v + 1024 c
  // at element m * pitch + 42 ky (c = byte % 3: k = ky*42 + kx*3 + c); the
  // other threads point the K padding 588..591 at the zero entry
  if (stg) {
    row.align();
    if constexpr (U16) {
      u32_alias* dst =
          reinterpret_cast<u32_alias*>(At + (tid & 31) * kPitch + (tid >> 5) * kPeRowBytes);
#pragma unroll
      for (int q = 0; q < kPeRowBytes / 2; ++q) {
        // bytes 2q, 2q+1 into the two u16 halves (one byte permute), then
        // times 4 plus both channels' table offsets
        const int b = 2 * q;
        const uint32_t v01 =
            __builtin_amdgcn_perm(0u, row.w[b >> 2], (b & 3) == 0 ? 0x0c010c00u : 0x0c030c02u);
        dst[q] = (v01 << 2) | ((1024u * (b % 3)) | ((1024u * ((b + 1) % 3)) << 16));
      }
    } else {
      Addr* dst = At + (tid & 31) * kPitch + (tid >> 5) * kPeRowBytes;
#pragma unroll
      for (int b = 0; b < kPeRowBytes; ++b)
        dst[b] = 4u * ((row.w[b >> 2] >> (8 * (b & 3))) & 0xffu) + 1024u * (b % 3);
    }
  } else {
    const int t = tid - kGm * kPatch;
    if (t < 2 * kGm) {
      Addr* pad = At + (t & 31) * kPitch + kPeK + 2 * (t >> 5);
      pad[0] = 4u * kGZero;
      pad[1] = 4u * kGZero;
    }
  }
  __syncthreads();

  // 5. MFMAs: element k = 16 b + 4 g + j of patch m = lane % 16 has its
  // address at arow[16 b + j]
  const Addr* const arow0 = At + (16 * rs + (lane & 15)) * kPitch + 4 * g;
  const Addr* const arow[2] = {arow0 + 16 * first1, arow0 + 16 * first2};
  const char* lutb = reinterpret_cast<const char*>(lut);
  f32x4 acc[3];
#pragma unroll
  for (int cs = 0; cs < 3; ++cs) acc[cs] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint32_t ad[kPeSeq][4];
  float av[kPeSeq][4];
  uint2 raw[kPeSeq];
  // u16: four addresses in one 64-bit read, split one block later (so the
  // split does not wait for the read); u32: one 128-bit read
  auto load_raw = [&](int s) {
    if constexpr (U16) {
      if (valid(s)) raw[s] = *reinterpret_cast<const uint2*>(arow[seg(s)] + 16 * off(s));
    }
  };
  auto load_ad = [&](int s) {
    if (valid(s)) {
      if constexpr (U16) {
        ad[s][0] = raw[s].x & 0xffffu;
        ad[s][1] = raw[s].x >> 16;
        ad[s][2] = raw[s].y & 0xffffu;
        ad[s][3] = raw[s].y >> 16;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) ad[s][j] = arow[seg(s)][16 * off(s) + j];
      }
    }
  };
  auto gather = [&](int s) {
    if (valid(s)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) av[s][j] = *reinterpret_cast<const float*>(lutb + ad[s][j]);
    }
  };
  float bias[3] = {0.f, 0.f, 0.f};
  float addend[3][4];
  auto load_epilogue = [&]() {
#pragma unroll
    for (int cs = 0; cs < 3; ++cs) {
      const int col = n0 + 48 * cg + 16 * cs + (lane & 15);
      const int ccol = col < p.N ? col : p.N - 1;
      bias[cs] = p.bias[ccol];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rw = m0 + 16 * rs + 4 * g + r;
        const int crow = rw < p.M ? rw : p.M - 1;
        addend[cs][r] = p.pos[static_cast<size_t>(1 + crow) * p.N + ccol];
      }
    }
  };
  auto mma = [&](int s) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int cs = 0; cs < 3; ++cs)
        acc[cs] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s][j], bf[s][cs][j], acc[cs], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Each block's MFMAs come first and the LDS reads of later blocks after
  // them: LDS reads complete in issue order, so a read issued just before
  // the MFMAs would hold them up.
#pragma unroll
  for (int s = 0; s <= kGLook + 1; ++s) load_raw(s);
#pragma unroll
  for (int s = 0; s <= kGLook; ++s) load_ad(s);
#pragma unroll
  for (int s = 0; s < kGLook; ++s) gather(s);
#pragma unroll
  for (int s = 0; s < kGSeg2; ++s) {
    mma(s);
    load_raw(s + kGLook + 2);
    load_ad(s + kGLook + 1);
    gather(s + kGLook);
    load_b(s + kGAhead);
    if (s == kPeSeq - kGAhead - 1 && half == 0) load_epilogue();
  }
  if (len == kPeSeq) mma(kGSeg2);  // half 0's position 18: block 10

  // 6. the k halves meet: half 1 hands its sums to half 0
  const int pair = rs + 2 * cg;
  if (half == 1) {
#pragma unroll
    for (int cs = 0; cs < 3; ++cs)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(pair * 12 + cs * 4 + r) * 64 + lane] = acc[cs][r];
  }
  __syncthreads();
  if (half == 1) return;
#pragma unroll
  for (int cs = 0; cs < 3; ++cs)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[cs][r] += red[(pair * 12 + cs * 4 + r) * 64 + lane];

  // 7. epilogue: lane holds D[4 g + r][lane % 16] of each 16x16 tile
#pragma unroll
  for (int cs = 0; cs < 3; ++cs) {
    const int col = n0 + 48 * cg + 16 * cs + (lane & 15);
    if (col < p.N) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rw = m0 + 16 * rs + 4 * g + r;
        if (rw < p.M)
          out[static_cast<size_t>(1 + p.n_register + rw) * p.N + col] =
              (acc[cs][r] + bias[cs]) + addend[cs][r];
      }
    }
  }
  if (mt == 0 && rs == 0) {
    // special rows of this wave's 48 columns, four rows per pass (one per
    // lane group): row 0 = CLS + pos[0], rows 1.. = registers
    for (int r0 = 0; r0 <= p.n_register; r0 += 4) {
      const int r = r0 + g;
#pragma unroll
      for (int cs = 0; cs < 3; ++cs) {
        const int col = n0 + 48 * cg + 16 * cs + (lane & 15);
        if (r <= p.n_register && col < p.N)
          out[static_cast<size_t>(r) * p.N + col] =
              r == 0 ? p.cls[col] + p.pos[col] : p.regs[static_cast<size_t>(r - 1) * p.N + col];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined patch embedding, for launches of many tiles (the views of a
// multi-view batch).  Tiles are 32 patches x 64 outputs, numbered with the
// output columns fastest, t = (view * gmt + mt) * gnt + nt, and each
// persistent workgroup runs one contiguous range of them, so consecutive
// tiles share their A tile (the 32 normalised patches): it is staged once
// per M tile of the range instead of once per tile.  Two A buffers (32 x
// 596 floats each): M tile j of the range lives in buffer j % 2.  The
// prologue stages the first two M tiles with every thread; while M tile j
// (j >= 1) runs, the staging waves stage M tile j + 1 into the other buffer,
// a slice of its rows per tile (that buffer's last reader, M tile j - 1,
// finished before M tile j began).  The two k halves' sums meet in a small
// LDS buffer; the half that adds and stores alternates from tile to tile,
// so one barrier per tile suffices (a wave that writes the buffer in one
// tile read it in the previous one).  Every output element takes
// block sequence, k-half split and epilogue order above: the same bits as
// the gathered kernel.
// ---------------------------------------------------------------------------
constexpr int kPp = 32;                  // patches per tile
constexpr int kPpRows = kPp * kPatch;    // 448 patch rows
constexpr int kPpBuf = kPp * kPePitch;   // floats per A buffer
constexpr int kPpAhead = 4;              // B prefetch distance in blocks (8 spills here)
static_assert(kPpRows <= kPeThreads && 2 * kPpRows <= 2 * kPeThreads &&
                  kPpRows <= 2 * kPeStagers && 2 * kPp * 4 <= kPeThreads,
              "prologue: at most two rows per thread; stagers: at most two rows each; the "
              "padding zeroed by one pass");

__global__ __launch_bounds__(kPeThreads) void patch_embed_pipelined_kernel(PatchArgs p) {
  __shared__ float lut[3 * 256];
  __shared__ __align__(16) float As[2 * kPpBuf];
  __shared__ __align__(16) float red[4 * 8 * 64];  // one k half's sums (160 KiB in all)

  const int tid = threadIdx.x;
  __builtin_assume(tid < kPeThreads);
  const int wave = tid >> 6, lane = tid & 63;
  const bool stager = tid >= kThreads;
  const int strip = wave & 3, half = (wave >> 2) & 1;
  const int gmt = (p.M + kPp - 1) / kPp;
  const int gnt = (p.N + BN - 1) / BN;
  const long long total = static_cast<long long>(p.tiles) * p.views;
  const int t0 = static_cast<int>(total * blockIdx.x / gridDim.x);
  const int t1 = static_cast<int>(total * (blockIdx.x + 1) / gridDim.x);  // > t0: grid <= total
  const int vm0 = t0 / gnt;                   // the range's first M tile (view * gmt + mt)
  const int nvm = (t1 - 1) / gnt - vm0 + 1;   // M tiles in the range

  // Patch row R of an M tile (0..447): groups of 32 rows are 16 patches x 2
  // pixel rows (so a half-wave's 8-byte LDS writes hit all 64 banks once):
  // m = 16 ((R / 32) % 2) + R % 16, ky = 2 (R / 64) + (R / 16) % 2.
  auto row_m = [](int r) { return 16 * ((r >> 5) & 1) + (r & 15); };
  auto row_ky = [](int r) { return 2 * (r >> 6) + ((r >> 4) & 1); };
  struct MTile {
    const uint8_t* img;
    float* out;
    int m0, mt;
  };
  auto mtile = [&](int vm) {
    const int view = vm / gmt;
    MTile a;
    a.mt = vm - view * gmt;
    a.m0 = a.mt * kPp;
    a.img = p.img + static_cast<size_t>(view) * p.img_bytes;
    a.out = p.out + static_cast<size_t>(view) * (1 + p.n_register + p.M) * p.N;
    return a;
  };
  auto row_start = [&](const MTile& a, int r) {
    const int gm = a.m0 + row_m(r);
    const int cm = gm < p.M ? gm : p.M - 1;
    const uint32_t py = vkd::fdiv(static_cast<uint32_t>(cm), p.fgw);
    const uint32_t px = static_cast<uint32_t>(cm) - py * static_cast<uint32_t>(p.gw);
    return ((py * kPatch + row_ky(r)) * static_cast<uint32_t>(p.W) + px * kPatch) * 3u;
  };
  auto row_dst = [&](int buf, int r) {
    return reinterpret_cast<float2*>(As + buf * kPpBuf + row_m(r) * kPePitch +
                                     row_ky(r) * kPeRowBytes);
  };

  // prologue: rows R = tid and tid + 768 of the first two M tiles' 896
  // (R / 448 = the M tile), the table, the K padding of both buffers
  {
    const MTile a0 = mtile(vm0), a1 = mtile(nvm > 1 ? vm0 + 1 : vm0);
    const int R0 = tid, R1 = tid + kPeThreads;
    const bool s0 = R0 < kPpRows || nvm > 1;
    const bool s1 = R1 < 2 * kPpRows && nvm > 1;
    const bool lo0 = R0 < kPpRows;
    PatchRow r0, r1;
    if (s0) r0.load(lo0 ? a0.img : a1.img, row_start(lo0 ? a0 : a1, lo0 ? R0 : R0 - kPpRows),
                    p.img_bytes);
    if (s1) r1.load(a1.img, row_start(a1, R1 - kPpRows), p.img_bytes);
    const int c = tid / 256, v = tid % 256;
    const float u = static_cast<float>(v) / 255.0f;
    lut[tid] = (u - p.mean[c]) / p.sd[c];
    if (tid < 2 * kPp * 4)
      As[(tid >> 7) * kPpBuf + ((tid >> 2) & 31) * kPePitch + kPeK + (tid & 3)] = 0.0f;
    __syncthreads();  // table visible
    if (s0) {
      r0.align();
      r0.store(row_dst(lo0 ? 0 : 1, lo0 ? R0 : R0 - kPpRows), lut, 0, kPeRowBytes / 2);
    }
    if (s1) {
      r1.align();
      r1.store(row_dst(1, R1 - kPpRows), lut, 0, kPeRowBytes / 2);
    }
  }

  // the compute waves' B fragments: column strip of the tile, block
  // sequence above (waves 0-3: blocks 0-9, 21-28, 10; waves
  // 4-7: 11-20, 29-36), kPpAhead blocks ahead of the MFMAs
  const int first1 = half ? kPePhase1 + 1 : 0;
  const int first2 = kPeBlocksA + half * kPePhase2;
  auto seq_block = [&](int s) {
    return s < kPePhase1 ? first1 + s
                         : (s < kPePhase1 + kPePhase2 ? first2 + s - kPePhase1 : kPePhase1);
  };
  f32x4 bf[kPeSeq];
  const float* wrow = nullptr;
  auto set_col = [&](int n0) {
    const int col = n0 + strip * 16 + (lane & 15);
    const int ccol = col < p.N ? col : p.N - 1;
    wrow = p.wpk + static_cast<size_t>(ccol) * kPeKp + 4 * (lane >> 4);
  };
  auto load_b = [&](int s) {
    if (s < kPeSeq) bf[s] = *reinterpret_cast<const f32x4*>(wrow + 16 * seq_block(s));
  };
  if (!stager) {
    set_col((t0 % gnt) * BN);
#pragma unroll
    for (int s = 0; s < kPpAhead; ++s) load_b(s);
  }
  __syncthreads();  // the first two M tiles are staged

  struct AFrag {
    f32x4 a[2];
  };
  for (int t = t0; t < t1; ++t) {
    const int vm = t / gnt;
    const int n0 = (t - vm * gnt) * BN;
    const int j = vm - vm0;
    const int b = j & 1;
    const MTile cur = mtile(vm);
    // the half that adds the two sums and stores alternates per tile
    const bool fin = half == ((t - t0) & 1);
    f32x4 acc[2];
    float bias = 0.0f, addend[2][4];
    if (stager) {
      // during M tile j >= 1 (whole: it started inside the range and is not
      // its last), M tile j + 1 into the other buffer, rows [lo, hi) now
      if (j >= 1 && j + 1 < nvm) {
        const int i = t - vm * gnt;
        const int lo = i * kPpRows / gnt, hi = (i + 1) * kPpRows / gnt;
        const int ra = lo + (tid - kThreads), rb = ra + kPeStagers;
        const MTile nm = mtile(vm + 1);
        PatchRow x0, x1;
        if (ra < hi) x0.load(nm.img, row_start(nm, ra), p.img_bytes);
        if (rb < hi) x1.load(nm.img, row_start(nm, rb), p.img_bytes);
        if (ra < hi) {
          x0.align();
          x0.store(row_dst(b ^ 1, ra), lut, 0, kPeRowBytes / 2);
        }
        if (rb < hi) {
          x1.align();
          x1.store(row_dst(b ^ 1, rb), lut, 0, kPeRowBytes / 2);
        }
      }
    } else {
      // epilogue operands first: their latency hides behind the MFMAs
      const int col = n0 + strip * 16 + (lane & 15);
      const int ccol = col < p.N ? col : p.N - 1;
      if (fin) {
        bias = p.bias[ccol];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = cur.m0 + tt * 16 + 4 * (lane >> 4) + r;
            const int crow = row < p.M ? row : p.M - 1;
            addend[tt][r] = p.pos[static_cast<size_t>(1 + crow) * p.N + ccol];
          }
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const float* arow = As + b * kPpBuf + (lane & 15) * kPePitch + 4 * (lane >> 4);
      auto load_a = [&](int s, AFrag& f) {
        const float* q = arow + 16 * seq_block(s);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          f.a[tt] = *reinterpret_cast<const f32x4*>(q + tt * 16 * kPePitch);
      };
      auto mma = [&](const AFrag& f, const f32x4& bb) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[tt][jj], bb[jj], acc[tt], 0, 0, 0);
      };
      constexpr int kRun = kPePhase1 + kPePhase2;  // positions of both halves
      AFrag f0, f1, f2;
      load_a(0, f0);
      load_a(1, f1);
#pragma unroll
      for (int s = 0; s < kRun; ++s) {
        if (s + 2 < kRun) load_a(s + 2, f2);
        load_b(s + kPpAhead);
        __builtin_amdgcn_sched_barrier(0);
        mma(f0, bf[s]);
        f0 = f1;
        f1 = f2;
      }
      if (half == 0) {  // waves 0-3's last block, 10
        AFrag f;
        load_a(kPeSeq - 1, f);
        mma(f, bf[kPeSeq - 1]);
      }
      // the next tile's first B fragments load during the hand-over below
      if (t + 1 < t1) {
        set_col(((t + 1) % gnt) * BN);
#pragma unroll
        for (int s = 0; s < kPpAhead; ++s) load_b(s);
      }
      if (!fin) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int r = 0; r < 4; ++r) red[(strip * 8 + tt * 4 + r) * 64 + lane] = acc[tt][r];
      }
    }
    // the other half's sums in `red`; this tile's rows of the next M tile
    // staged; every read of the buffer a later tile's staging overwrites done
    __syncthreads();
    if (!stager && fin) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[tt][r] += red[(strip * 8 + tt * 4 + r) * 64 + lane];
      // lane holds D[4*(lane/16) + r][lane%16] of each 16x16 tile
      const int col = n0 + strip * 16 + (lane & 15);
      if (col < p.N) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = cur.m0 + tt * 16 + 4 * (lane >> 4) + r;
            if (row < p.M)
              cur.out[static_cast<size_t>(1 + p.n_register + row) * p.N + col] =
                  (acc[tt][r] + bias) + addend[tt][r];
          }
      }
      if (cur.mt == 0) {
        for (int r0 = 0; r0 <= p.n_register; r0 += 4) {
          const int r = r0 + (lane >> 4);
          if (r <= p.n_register && col < p.N)
            cur.out[static_cast<size_t>(r) * p.N + col] =
                r == 0 ? p.cls[col] + p.pos[col]
                       : p.regs[static_cast<size_t>(r - 1) * p.N + col];
        }
      }
    }
  }
}

// NCHW f32 -> patch rows [gh*gw, C*p*p], column c*p*p + ky*p + kx.
__global__ void patchify_kernel(const float* __restrict__ img, float* __restrict__ out, int h,
                                int w, int p, int channels, long long total) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int kdim = channels * p * p;
  const int gw = w / p;
  const long long patch = i / kdim;
  const int k = static_cast<int>(i % kdim);
  const int c = k / (p * p);
  const int ky = (k % (p * p)) / p;
  const int kx = k % p;
  const int pr = static_cast<int>(patch / gw), pc = static_cast<int>(patch % gw);
  out[i] = img[(static_cast<size_t>(c) * h + pr * p + ky) * w + pc * p + kx];
}

// row 0 = cls + pos[0]; row 1+p = patch_p + pos[1+p]
__global__ void prepend_cls_add_pos_kernel(const float* __restrict__ patches,
                                           const float* __restrict__ cls,
                                           const float* __restrict__ pos,
                                           float* __restrict__ out, long long n_patches,
                                           int embed) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  const long long total = (n_patches + 1) * embed;
  if (i >= total) return;
  if (i < embed)
    out[i] = cls[i] + pos[i];
  else
    out[i] = patches[i - embed] + pos[i];
}

__device__ __forceinline__ float cubic_keys(float x) {
  const float A = -0.75f;
  x = fabsf(x);
  if (x < 1.0f) return ((A + 2.0f) * x - (A + 3.0f)) * x * x + 1.0f;
  if (x < 2.0f) return (((x - 5.0f) * x + 8.0f) * x - 4.0f) * A;
  return 0.0f;
}

// Bicubic position-table resize, one thread per (output row, channel); same
// f32 operation order as the scalar interpolate_pos_embed.
__global__ void pos_embed_bicubic_kernel(const float* __restrict__ src, float* __restrict__ out,
                                         int grid, int embed, int gh, int gw,
                                         float interp_offset) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  const long long total = static_cast<long long>(1 + gh * gw) * embed;
  if (i >= total) return;
  const int ch = static_cast<int>(i % embed);
  const long long orow = i / embed;
  if (orow == 0) {
    out[i] = src[ch];
    return;
  }
  const int oy = static_cast<int>((orow - 1) / gw);
  const int ox = static_cast<int>((orow - 1) % gw);
  const float m = static_cast<float>(grid);
  const float sx = (static_cast<float>(gw) + interp_offset) / m;
  const float sy = (static_cast<float>(gh) + interp_offset) / m;
  const float iy = (static_cast<float>(oy) + 0.5f) / sy - 0.5f;
  const int y0 = static_cast<int>(floorf(iy));
  const float fy = iy - static_cast<float>(y0);
  const float ix = (static_cast<float>(ox) + 0.5f) / sx - 0.5f;
  const int x0 = static_cast<int>(floorf(ix));
  const float fx = ix - static_cast<float>(x0);
  float acc = 0.0f;
  for (int dy = -1; dy <= 2; ++dy) {
    const float wy = cubic_keys(fy - static_cast<float>(dy));
    const int yy = min(max(y0 + dy, 0), grid - 1);
    for (int dx = -1; dx <= 2; ++dx) {
      const float wx = cubic_keys(fx - static_cast<float>(dx));
      const int xx = min(max(x0 + dx, 0), grid - 1);
      const float v = src[(1 + static_cast<size_t>(yy) * grid + xx) * embed + ch];
      acc += wy * wx * v;
    }
  }
  out[i] = acc;
}

// The patch kernel's copy of a 3x14x14 filter: input order (c, ky, kx) ->
// (ky, kx, c), zero beyond 588 (made at prepare time by prepare_patch_filter).
__global__ __launch_bounds__(256) void patch_order_kernel(const float* __restrict__ wnk,
                                                          float* __restrict__ wp, int out, int kp) {
  const long long idx = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<long long>(out) * kPeKp) return;
  const int o = static_cast<int>(idx / kPeKp), k = static_cast<int>(idx % kPeKp);
  float v = 0.0f;
  if (k < kPeK) {
    const int ky = k / kPeRowBytes, rem = k % kPeRowBytes;
    const int kx = rem / 3, c = rem % 3;
    v = wnk[static_cast<size_t>(o) * kp + (c * kPatch + ky) * kPatch + kx];
  }
  wp[idx] = v;
}

}  // namespace

namespace vk {

int prepare_patch_filter(vk_runtime* rt, vk_linear* lin) {
  if (lin->in_features != static_cast<size_t>(kPeK)) return VK_OK;
  const long long np = static_cast<long long>(kPeKp) * static_cast<long long>(lin->out_features);
  VK_HIP(hipMalloc(reinterpret_cast<void**>(&lin->weight_patch), np * sizeof(float)));
  hipLaunchKernelGGL(patch_order_kernel, dim3(static_cast<unsigned>((np + 255) / 256)), dim3(256),
                     0, rt->stream, lin->weight_nk, lin->weight_patch,
                     static_cast<int>(lin->out_features), static_cast<int>(lin->k_pitch));
  return vk::check_launch("patch_order_kernel");
}

}  // namespace vk

extern "C" {

int vk_patchify_nchw_f32(vk_runtime* rt, const vk_tensor* img, size_t h, size_t w,
                         size_t patch, size_t channels, vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(img && out, "null argument");
  VK_REQUIRE(img->dtype == VK_F32, "image must be f32 NCHW");
  VK_REQUIRE(patch > 0 && channels > 0 && h > 0 && w > 0, "empty patchify shape");
  VK_REQUIRE(h % patch == 0 && w % patch == 0, "h=%zu and w=%zu must be multiples of patch=%zu",
             h, w, patch);
  VK_REQUIRE(img->len == channels * h * w, "image holds %zu, channels*h*w=%zu", img->len,
             channels * h * w);
  const long long total = static_cast<long long>((h / patch) * (w / patch) * channels * patch * patch);
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, static_cast<size_t>(total), &t));
  hipLaunchKernelGGL(patchify_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256),
                     0, rt->stream, static_cast<const float*>(img->ptr),
                     static_cast<float*>(t->ptr), static_cast<int>(h), static_cast<int>(w),
                     static_cast<int>(patch), static_cast<int>(channels), total);
  int s = vk::check_launch("patchify_kernel");
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

int vk_prepend_cls_add_pos_f32(vk_runtime* rt, const vk_tensor* patches, const vk_tensor* cls,
                               const vk_tensor* pos, size_t n_patches, size_t embed,
                               vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(patches && cls && pos && out, "null argument");
  VK_REQUIRE(patches->dtype == VK_F32 && cls->dtype == VK_F32 && pos->dtype == VK_F32,
             "operands must be f32");
  VK_REQUIRE(patches->len == n_patches * embed, "patches hold %zu, n_patches*embed=%zu",
             patches->len, n_patches * embed);
  VK_REQUIRE(cls->len == embed, "cls holds %zu, embed=%zu", cls->len, embed);
  VK_REQUIRE(pos->len == (n_patches + 1) * embed, "pos holds %zu, (n_patches+1)*embed=%zu",
             pos->len, (n_patches + 1) * embed);
  const long long total = static_cast<long long>((n_patches + 1) * embed);
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, static_cast<size_t>(total), &t));
  hipLaunchKernelGGL(prepend_cls_add_pos_kernel, dim3(static_cast<unsigned>((total + 255) / 256)),
                     dim3(256), 0, rt->stream, static_cast<const float*>(patches->ptr),
                     static_cast<const float*>(cls->ptr), static_cast<const float*>(pos->ptr),
                     static_cast<float*>(t->ptr), static_cast<long long>(n_patches),
                     static_cast<int>(embed));
  int s = vk::check_launch("prepend_cls_add_pos_kernel");
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

int vk_pos_embed_bicubic_f32(vk_runtime* rt, const vk_tensor* pos_embed, size_t grid,
                             size_t embed, size_t gh, size_t gw, float interp_offset,
                             vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(pos_embed && out, "null argument");
  VK_REQUIRE(pos_embed->dtype == VK_F32, "pos_embed must be f32");
  VK_REQUIRE(grid > 0 && embed > 0, "empty pos_embed");
  VK_REQUIRE(pos_embed->len == (grid * grid + 1) * embed,
             "pos_embed holds %zu, (grid*grid+1)*embed=%zu", pos_embed->len,
             (grid * grid + 1) * embed);
  const long long total = static_cast<long long>((1 + gh * gw) * embed);
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, static_cast<size_t>(total), &t));
  hipLaunchKernelGGL(pos_embed_bicubic_kernel, dim3(static_cast<unsigned>((total + 255) / 256)),
                     dim3(256), 0, rt->stream, static_cast<const float*>(pos_embed->ptr),
                     static_cast<float*>(t->ptr), static_cast<int>(grid),
                     static_cast<int>(embed), static_cast<int>(gh), static_cast<int>(gw),
                     interp_offset);
  int s = vk::check_launch("pos_embed_bicubic_kernel");
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

int vk_patch_embed_views_u8(vk_runtime* rt, const vk_tensor* images, size_t views, size_t h,
                            size_t w, size_t patch, const float mean[3], const float std_[3],
                            const vk_linear* proj, const vk_tensor* cls,
                            const vk_tensor* registers, size_t n_register,
                            const vk_tensor* pos_table, vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(images && mean && std_ && proj && cls && pos_table && out, "null argument");
  VK_REQUIRE(views > 0, "patch_embed: no views");
  VK_UNSUPPORTED_IF(patch != static_cast<size_t>(kPatch),
                    "patch_embed_u8: patch=%zu (qualified: 14)", patch);
  VK_REQUIRE(h > 0 && w > 0 && h % patch == 0 && w % patch == 0,
             "h=%zu and w=%zu must be positive multiples of patch=%zu", h, w, patch);
  VK_REQUIRE(images->dtype == VK_U8 && images->len == views * h * w * 3,
             "images must be u8 [views, h, w, 3] with %zu bytes (got %zu)", views * h * w * 3,
             images->len);
  const size_t gh = h / patch, gw = w / patch, np = gh * gw;
  const size_t embed = proj->out_features;
  VK_REQUIRE(proj->in_features == 3 * patch * patch, "projection in_features=%zu, expected %zu",
             proj->in_features, 3 * patch * patch);
  VK_REQUIRE(proj->ls_gamma == nullptr, "patch projection must not carry a LayerScale");
  VK_REQUIRE(cls->dtype == VK_F32 && cls->len == embed, "cls must be f32 [embed=%zu]", embed);
  VK_REQUIRE(n_register == 0 || (registers && registers->dtype == VK_F32 &&
                                 registers->len == n_register * embed),
             "registers must be f32 [n_register*embed=%zu]", n_register * embed);
  VK_REQUIRE(pos_table->dtype == VK_F32 && pos_table->len == (1 + np) * embed,
             "pos_table must be f32 [(1+gh*gw)*embed=%zu] (got %zu)", (1 + np) * embed,
             pos_table->len);
  VK_REQUIRE(out->dtype == VK_F32 && out->len == views * (1 + n_register + np) * embed,
             "out must be f32 [views*(1+n_register+gh*gw)*embed=%zu] (got %zu)",
             views * (1 + n_register + np) * embed, out->len);
  VK_UNSUPPORTED_IF(h * w * 3 > 0x7fffffffULL || np > 0x7fffffffULL, "image too large");
  // the filter is read through a buffer descriptor of 32-bit byte size
  VK_UNSUPPORTED_IF(embed * kPeKp * 4 > 0x7fffffffULL, "patch_embed_u8: embed=%zu", embed);
  for (int c = 0; c < 3; ++c) VK_REQUIRE(std_[c] != 0.0f, "std[%d] is zero", c);
  VK_REQUIRE(proj->weight_patch != nullptr, "projection has no patch-order filter");
  // every view's rows are read as aligned 8-byte words
  VK_UNSUPPORTED_IF(reinterpret_cast<uintptr_t>(images->ptr) % 8 != 0 ||
                        (views > 1 && (h * w * 3) % 8 != 0),
                    "patch_embed_u8: every image must start 8-byte aligned");
  PatchArgs a{};
  a.img = static_cast<const uint8_t*>(images->ptr);
  a.img_bytes = static_cast<uint32_t>(h * w * 3);
  a.wpk = proj->weight_patch;
  a.bias = proj->bias;
  a.pos = static_cast<const float*>(pos_table->ptr);
  a.cls = static_cast<const float*>(cls->ptr);
  a.regs = n_register ? static_cast<const float*>(registers->ptr) : nullptr;
  a.out = static_cast<float*>(out->ptr);
  a.W = static_cast<int>(w);
  a.gw = static_cast<int>(gw);
  a.fgw = vkd::make_fastdiv(static_cast<uint32_t>(gw));
  a.M = static_cast<int>(np);
  a.N = static_cast<int>(embed);
  a.n_register = static_cast<int>(n_register);
  for (int c = 0; c < 3; ++c) {
    a.mean[c] = mean[c];
    a.sd[c] = std_[c];
  }
  a.views = static_cast<int>(views);
  const long long cus = rt->cu_count > 0 ? rt->cu_count : 256;
#if VK_PE_PIPELINED
  const long long tiles32 =
      static_cast<long long>((a.M + kPp - 1) / kPp) * ((a.N + BN - 1) / BN);
  if (views > 1 && tiles32 * static_cast<long long>(views) > cus) {
    VK_UNSUPPORTED_IF(tiles32 * static_cast<long long>(views) > 0x7fffffffLL,
                      "patch_embed_u8: %lld tiles", tiles32 * static_cast<long long>(views));
    a.tiles = static_cast<int>(tiles32);
    hipLaunchKernelGGL(patch_embed_pipelined_kernel, dim3(static_cast<unsigned>(cus)),
                       dim3(kPeThreads), 0, rt->stream, a);
    return vk::check_launch("patch_embed_pipelined_kernel");
  }
#endif
  // one round of tiles: u32 addresses; several rounds: u16 (two workgroups
  // per CU)
  const long long gtiles = static_cast<long long>((a.M + kGm - 1) / kGm) * ((a.N + kGn - 1) / kGn);
  VK_UNSUPPORTED_IF(gtiles * static_cast<long long>(views) > 0x7fffffffLL,
                    "patch_embed_u8: %lld tiles", gtiles * static_cast<long long>(views));
  a.tiles = static_cast<int>(gtiles);
  const dim3 grid(static_cast<unsigned>(gtiles * views));
  if (gtiles * static_cast<long long>(views) <= cus)
    hipLaunchKernelGGL(patch_embed_gather_kernel<false>, grid, dim3(kGThreads), 0, rt->stream, a);
  else
    hipLaunchKernelGGL(patch_embed_gather_kernel<true>, grid, dim3(kGThreads), 0, rt->stream, a);
  return vk::check_launch("patch_embed_gather_kernel");
}

int vk_patch_embed_u8(vk_runtime* rt, const vk_tensor* img_hwc, size_t h, size_t w,
                      size_t patch, const float mean[3], const float std_[3],
                      const vk_linear* proj, const vk_tensor* cls, const vk_tensor* registers,
                      size_t n_register, const vk_tensor* pos_table, vk_tensor* out) {
  return vk_patch_embed_views_u8(rt, img_hwc, 1, h, w, patch, mean, std_, proj, cls, registers,
                                 n_register, pos_table, out);
}

}  // extern "C"
