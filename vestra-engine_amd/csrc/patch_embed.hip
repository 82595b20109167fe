// Patch embedding for gfx950: the only MFMA contraction of the fused path.
//
// The 14x14 / stride-14 patch convolution is a GEMM
//   tokens[p, e] = sum_k A[p, k] * W[e, k] + b[e],   k = c*196 + ky*14 + kx,
// with A the normalised, unfolded image.  One kernel does it all: the A
// operand is gathered straight from the u8 HWC image and normalised through a
// 3x256 lookup table in LDS (the table holds exactly (u8/255 - mean)/std, so
// the normalisation is bit-identical to the scalar path), the filter is
// streamed from a [K, N] copy made at prepare time, the products run on
// v_mfma_f32_16x16x4_f32 (F32 in, F32 accumulate), and the epilogue adds the
// bias and the position table and writes the assembled token rows (CLS +
// pos[0], register rows, patch rows) so nothing round-trips through HBM.
//
// Tiling: a 256-thread workgroup (4 waves) owns a 48 (patches) x 64 (embed)
// output tile; wave w owns 16 embed columns across all 48 rows (three 16x16
// accumulators).  K is consumed in chunks of 196 = one input channel of a
// 14x14 patch (3 chunks per image), staged in LDS as A^T[k][m] and B[k][n]
// with a row pitch of 80 floats, which makes both fragment reads bank-conflict
// free.  While the MFMAs consume one chunk from LDS, the next chunk's global
// loads are already in flight into registers, so each chunk's load latency is
// hidden behind the previous chunk's 147 MFMAs.  The 125 KB of LDS allows one
// workgroup per CU: ViT-B at 504x336 is 864 x 768 outputs -> 18 x 12 = 216
// workgroups, one round on 256 CUs.
#include <cstring>
#include <vector>

#include "common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 48;
constexpr int BN = 64;
constexpr int KC = 196;
constexpr int PA = 80;  // LDS pitch of A^T rows (BM + 32)
constexpr int PB = 80;  // LDS pitch of B rows (BN + 16)
constexpr int kPatch = 14;
constexpr int kThreads = 256;
constexpr int kA_PER_THREAD = (KC * BM + kThreads - 1) / kThreads;        // 37
constexpr int kB_VEC_PER_THREAD = (KC * BN / 4 + kThreads - 1) / kThreads;  // 13

enum Epilogue { kEpiLinear = 0, kEpiTokens = 1 };

struct GemmArgs {
  const float* wkn;    // [K, N]
  const float* bias;   // [N]
  const float* ls;     // [N] or null (linear epilogue)
  float* out;
  int M, N, K;
  // token epilogue
  const float* pos;    // [(1 + M), N]
  const float* cls;    // [N]
  const float* regs;   // [n_register, N] or null
  int n_register;
};

// The loaders below never branch around a global load: a load inside a
// guard makes the compiler wait for it before the next one, serialising the
// memory latency.  Slots outside the matrix read a clamped (valid) address
// and are zeroed when stored to LDS.

// A operand from a row-major f32 matrix x[M, K]; element slot i of a thread
// covers (m, kk) = (e / KC, e % KC), e = tid + 256 i (k fastest: coalesced).
struct RowsA {
  const float* x;
  float reg[kA_PER_THREAD];
  uint64_t live;  // bit i: slot i inside the matrix for the current chunk
  __device__ __forceinline__ void init(const float*, int, int, int) {}
  __device__ __forceinline__ void fetch(int m0, int k0, int M, int K, int tid) {
    live = 0;
#pragma unroll
    for (int i = 0; i < kA_PER_THREAD; ++i) {
      const int e = tid + kThreads * i;
      const int kk = e % KC;
      const int m = e / KC;
      const int gm = m0 + m, gk = k0 + kk;
      const bool ok = e < KC * BM && gm < M && gk < K;
      live |= static_cast<uint64_t>(ok) << i;
      const int cm = gm < M ? gm : M - 1;
      const int ck = gk < K ? gk : K - 1;
      reg[i] = x[static_cast<size_t>(cm) * K + ck];
    }
  }
  __device__ __forceinline__ void store(float (*As)[PA], int tid) const {
#pragma unroll
    for (int i = 0; i < kA_PER_THREAD; ++i) {
      const int e = tid + kThreads * i;
      if (e < KC * BM) As[e % KC][e / KC] = ((live >> i) & 1) ? reg[i] : 0.0f;
    }
  }
};

// A operand gathered from the u8 HWC image: one chunk is one input channel c
// of the 48 patches' 14x14 windows.  Slot i covers (m, kk) = (e % 48, e / 48)
// (patch fastest), kk = ky*14 + kx; its byte offset for channel 0 is computed
// once, a chunk adds the channel.  Bytes are normalised at LDS store time.
struct ImageA {
  const uint8_t* img;
  int W;   // image width in pixels
  int gw;  // patches per image row
  const float* lut;  // LDS, [3][256]
  int off[kA_PER_THREAD];
  uint32_t reg[kA_PER_THREAD];
  uint64_t live;
  int chan;

  __device__ __forceinline__ void init(const float* l, int m0, int M, int tid) {
    lut = l;
    live = 0;
#pragma unroll
    for (int i = 0; i < kA_PER_THREAD; ++i) {
      const int e = tid + kThreads * i;
      const int m = e % BM;
      const int kk = e / BM;
      const int gm = m0 + m;
      const bool ok = e < KC * BM && gm < M;
      live |= static_cast<uint64_t>(ok) << i;
      const int cm = gm < M ? gm : M - 1;
      const int ckk = kk < KC ? kk : KC - 1;
      const int py = cm / gw, px = cm - py * gw;
      const int ky = ckk / kPatch, kx = ckk - ky * kPatch;
      off[i] = ((py * kPatch + ky) * W + px * kPatch + kx) * 3;
    }
  }
  __device__ __forceinline__ void fetch(int, int k0, int, int, int) {
    chan = k0 / (kPatch * kPatch);
#pragma unroll
    for (int i = 0; i < kA_PER_THREAD; ++i) reg[i] = img[off[i] + chan];
  }
  __device__ __forceinline__ void store(float (*As)[PA], int tid) const {
    const float* t = lut + chan * 256;
#pragma unroll
    for (int i = 0; i < kA_PER_THREAD; ++i) {
      const int e = tid + kThreads * i;
      if (e < KC * BM) As[e / BM][e % BM] = ((live >> i) & 1) ? t[reg[i]] : 0.0f;
    }
  }
};

struct BRegs {
  float4 reg[kB_VEC_PER_THREAD];
  uint32_t live;
  __device__ __forceinline__ void fetch(const GemmArgs& g, int n0, int k0, int tid) {
    live = 0;
#pragma unroll
    for (int i = 0; i < kB_VEC_PER_THREAD; ++i) {
      const int f = tid + kThreads * i;
      const int kk = f / (BN / 4);
      const int c4 = f % (BN / 4);
      const int gk = k0 + kk, gn = n0 + c4 * 4;
      // N % 4 == 0: a vector never straddles the edge
      const bool ok = f < KC * BN / 4 && gk < g.K && gn < g.N;
      live |= static_cast<uint32_t>(ok) << i;
      const int ck = gk < g.K ? gk : g.K - 1;
      const int cn = gn < g.N ? gn : g.N - 4;
      reg[i] = *reinterpret_cast<const float4*>(g.wkn + static_cast<size_t>(ck) * g.N + cn);
    }
  }
  __device__ __forceinline__ void store(float (*Bs)[PB], int tid) const {
#pragma unroll
    for (int i = 0; i < kB_VEC_PER_THREAD; ++i) {
      const int f = tid + kThreads * i;
      if (f < KC * BN / 4)
        *reinterpret_cast<float4*>(&Bs[f / (BN / 4)][(f % (BN / 4)) * 4]) =
            ((live >> i) & 1) ? reg[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
};

template <class ALoader, int EPI>
__global__ __launch_bounds__(256) void mfma_gemm_kernel(ALoader a_src, GemmArgs g,
                                                        float m0n, float m1n, float m2n,
                                                        float s0, float s1, float s2) {
  __shared__ float As[KC][PA];
  __shared__ float Bs[KC][PB];
  __shared__ float lut[EPI == kEpiTokens ? 3 * 256 : 1];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int m0 = blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;

  if constexpr (EPI == kEpiTokens) {
    // (v/255 - mean[c]) / std[c], exactly as the scalar normalisation
    for (int e = tid; e < 3 * 256; e += kThreads) {
      const int c = e / 256, v = e % 256;
      const float mean = c == 0 ? m0n : (c == 1 ? m1n : m2n);
      const float sd = c == 0 ? s0 : (c == 1 ? s1 : s2);
      const float u = static_cast<float>(v) / 255.0f;
      lut[e] = (u - mean) / sd;
    }
  }
  a_src.init(lut, m0, g.M, tid);

  f32x4 acc[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  BRegs b_src;
  a_src.fetch(m0, 0, g.M, g.K, tid);
  b_src.fetch(g, n0, 0, tid);
  __syncthreads();  // LUT visible before the first normalised store
  for (int k0 = 0; k0 < g.K; k0 += KC) {
    a_src.store(As, tid);
    b_src.store(Bs, tid);
    __syncthreads();
    if (k0 + KC < g.K) {
      // next chunk's global loads overlap this chunk's MFMAs
      a_src.fetch(m0, k0 + KC, g.M, g.K, tid);
      b_src.fetch(g, n0, k0 + KC, tid);
    }
#pragma unroll 7
    for (int ks = 0; ks < KC; ks += 4) {
      const float b = Bs[ks + (lane >> 4)][wave * 16 + (lane & 15)];
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const float a = As[ks + (lane >> 4)][t * 16 + (lane & 15)];
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[t], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // epilogue: lane holds D[4*(lane/16) + r][lane%16] of each 16x16 tile
  const int col = n0 + wave * 16 + (lane & 15);
  if (col < g.N) {
    const float bias = g.bias[col];
    float ls = 1.0f;
    if (EPI == kEpiLinear && g.ls) ls = g.ls[col];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + t * 16 + 4 * (lane >> 4) + r;
        if (row < g.M) {
          float v = acc[t][r] + bias;
          if (EPI == kEpiLinear) {
            if (g.ls) v = v * ls;
            g.out[static_cast<size_t>(row) * g.N + col] = v;
          } else {
            v = v + g.pos[static_cast<size_t>(1 + row) * g.N + col];
            g.out[static_cast<size_t>(1 + g.n_register + row) * g.N + col] = v;
          }
        }
      }
    }
    if (EPI == kEpiTokens && blockIdx.x == 0 && lane < 16) {
      // special rows of this column strip: CLS + pos[0], then registers
      g.out[col] = g.cls[col] + g.pos[col];
      for (int r = 0; r < g.n_register; ++r)
        g.out[static_cast<size_t>(1 + r) * g.N + col] = g.regs[static_cast<size_t>(r) * g.N + col];
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

int alloc_copy(const float* host, size_t n, float** dev) {
  VK_HIP(hipMalloc(dev, n * sizeof(float)));
  hipError_t e = hipMemcpy(*dev, host, n * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(*dev);
    *dev = nullptr;
    return vk::hip_fail(e, "hipMemcpy(linear weights)");
  }
  return VK_OK;
}

int make_linear(vk_runtime* rt, size_t in, size_t out, const std::vector<float>& wkn,
                const float* bias, const float* ls, vk_linear** res) {
  auto* lin = new vk_linear;
  lin->rt = rt;
  lin->in_features = in;
  lin->out_features = out;
  int s = alloc_copy(wkn.data(), in * out, &lin->weight_kn);
  if (s == VK_OK) s = alloc_copy(bias, out, &lin->bias);
  if (s == VK_OK && ls) s = alloc_copy(ls, out, &lin->ls_gamma);
  if (s != VK_OK) {
    vk_linear_destroy(lin);
    return s;
  }
  *res = lin;
  return VK_OK;
}

}  // namespace

extern "C" {

int vk_linear_prepare_f32(vk_runtime* rt, size_t in_features, size_t out_features,
                          const float* weight_in_out, const float* bias, const float* ls_gamma,
                          vk_linear** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out && weight_in_out && bias, "null argument");
  VK_REQUIRE(in_features > 0 && out_features > 0, "empty linear");
  VK_UNSUPPORTED_IF(out_features % 4 != 0, "linear: out_features=%zu must be a multiple of 4",
                    out_features);
  VK_UNSUPPORTED_IF(in_features > 0x7fffffff || out_features > 0x7fffffff, "linear too large");
  std::vector<float> w(weight_in_out, weight_in_out + in_features * out_features);
  return make_linear(rt, in_features, out_features, w, bias, ls_gamma, out);
}

int vk_linear_prepare_oihw_f32(vk_runtime* rt, size_t in_features, size_t out_features,
                               const float* weight_out_in, const float* bias, vk_linear** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(out && weight_out_in && bias, "null argument");
  VK_REQUIRE(in_features > 0 && out_features > 0, "empty linear");
  VK_UNSUPPORTED_IF(out_features % 4 != 0, "linear: out_features=%zu must be a multiple of 4",
                    out_features);
  VK_UNSUPPORTED_IF(in_features > 0x7fffffff || out_features > 0x7fffffff, "linear too large");
  std::vector<float> w(in_features * out_features);
  for (size_t o = 0; o < out_features; ++o)
    for (size_t i = 0; i < in_features; ++i) w[i * out_features + o] = weight_out_in[o * in_features + i];
  return make_linear(rt, in_features, out_features, w, bias, nullptr, out);
}

int vk_linear_destroy(vk_linear* lin) {
  if (!lin) return VK_OK;
  if (lin->rt) (void)vk::bind(lin->rt);
  if (lin->rt) (void)hipStreamSynchronize(lin->rt->stream);
  if (lin->weight_kn) (void)hipFree(lin->weight_kn);
  if (lin->bias) (void)hipFree(lin->bias);
  if (lin->ls_gamma) (void)hipFree(lin->ls_gamma);
  delete lin;
  return VK_OK;
}

size_t vk_linear_input_features(const vk_linear* lin) { return lin ? lin->in_features : 0; }

int vk_linear_run_f32(vk_runtime* rt, const vk_linear* lin, const vk_tensor* x, size_t rows,
                      vk_tensor** out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(lin && x && out, "null argument");
  VK_REQUIRE(x->dtype == VK_F32, "linear input must be f32");
  VK_REQUIRE(x->len == rows * lin->in_features, "linear: x holds %zu, rows*in=%zu", x->len,
             rows * lin->in_features);
  VK_UNSUPPORTED_IF(rows > 0x7fffffffULL, "linear: rows=%zu too large", rows);
  vk_tensor* t = nullptr;
  VK_TRY(vk_tensor_alloc(rt, VK_F32, rows * lin->out_features, &t));
  if (rows > 0) {
    GemmArgs g{};
    g.wkn = lin->weight_kn;
    g.bias = lin->bias;
    g.ls = lin->ls_gamma;
    g.out = static_cast<float*>(t->ptr);
    g.M = static_cast<int>(rows);
    g.N = static_cast<int>(lin->out_features);
    g.K = static_cast<int>(lin->in_features);
    RowsA a{static_cast<const float*>(x->ptr)};
    dim3 grid((g.M + BM - 1) / BM, (g.N + BN - 1) / BN);
    hipLaunchKernelGGL((mfma_gemm_kernel<RowsA, kEpiLinear>), grid, dim3(256), 0, rt->stream, a,
                       g, 0.f, 0.f, 0.f, 1.f, 1.f, 1.f);
    int s = vk::check_launch("mfma_gemm_kernel<rows>");
    if (s != VK_OK) {
      vk_tensor_destroy(t);
      return s;
    }
  }
  *out = t;
  return VK_OK;
}

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

int vk_patch_embed_u8(vk_runtime* rt, const vk_tensor* img_hwc, size_t h, size_t w,
                      size_t patch, const float mean[3], const float std_[3],
                      const vk_linear* proj, const vk_tensor* cls, const vk_tensor* registers,
                      size_t n_register, const vk_tensor* pos_table, vk_tensor* out) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(img_hwc && mean && std_ && proj && cls && pos_table && out, "null argument");
  VK_UNSUPPORTED_IF(patch != static_cast<size_t>(kPatch),
                    "patch_embed_u8: patch=%zu (qualified: 14)", patch);
  VK_REQUIRE(h > 0 && w > 0 && h % patch == 0 && w % patch == 0,
             "h=%zu and w=%zu must be positive multiples of patch=%zu", h, w, patch);
  VK_REQUIRE(img_hwc->dtype == VK_U8 && img_hwc->len == h * w * 3,
             "image must be u8 HWC with h*w*3=%zu bytes (got %zu)", h * w * 3, img_hwc->len);
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
  VK_REQUIRE(out->dtype == VK_F32 && out->len == (1 + n_register + np) * embed,
             "out must be f32 [(1+n_register+gh*gw)*embed=%zu] (got %zu)",
             (1 + n_register + np) * embed, out->len);
  VK_UNSUPPORTED_IF(h * w * 3 > 0x7fffffffULL || np > 0x7fffffffULL, "image too large");
  for (int c = 0; c < 3; ++c) VK_REQUIRE(std_[c] != 0.0f, "std[%d] is zero", c);
  GemmArgs g{};
  g.wkn = proj->weight_kn;
  g.bias = proj->bias;
  g.ls = nullptr;
  g.out = static_cast<float*>(out->ptr);
  g.M = static_cast<int>(np);
  g.N = static_cast<int>(embed);
  g.K = static_cast<int>(proj->in_features);
  g.pos = static_cast<const float*>(pos_table->ptr);
  g.cls = static_cast<const float*>(cls->ptr);
  g.regs = n_register ? static_cast<const float*>(registers->ptr) : nullptr;
  g.n_register = static_cast<int>(n_register);
  ImageA a{};
  a.img = static_cast<const uint8_t*>(img_hwc->ptr);
  a.W = static_cast<int>(w);
  a.gw = static_cast<int>(gw);
  dim3 grid((g.M + BM - 1) / BM, (g.N + BN - 1) / BN);
  hipLaunchKernelGGL((mfma_gemm_kernel<ImageA, kEpiTokens>), grid, dim3(256), 0, rt->stream, a, g,
                     mean[0], mean[1], mean[2], std_[0], std_[1], std_[2]);
  return vk::check_launch("mfma_gemm_kernel<image>");
}

}  // extern "C"
