// Runtime, tensors, transfers, events and graphs of the C ABI.
//
// Mirrors the host-facing half of the reference's device runtime
// (`vestra_kernels::cuda::CudaRuntime`: new/upload/download/copy/segment
// copies/prefix overwrite, called from crates/da-engine/src/vit_block.rs:
// 161-184, 335, 370, 402-478 and backbone.rs:991-1027).
#include <cmath>
#include <cstring>
#include <tuple>
#include <vector>

#include "common.h"

namespace vk {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int hip_fail(hipError_t e, const char* what) {
  const int code = (e == hipErrorOutOfMemory) ? VK_ERR_OOM : VK_ERR_HIP;
  return set_error(code, "%s failed: %s (%d)", what, hipGetErrorString(e),
                   static_cast<int>(e));
}

size_t dtype_size(vk_dtype d) {
  switch (d) {
    case VK_F32: return 4;
    case VK_F16: return 2;
    case VK_U8: return 1;
    case VK_I32: return 4;
    case VK_I64: return 8;
  }
  return 0;
}

int bind(vk_runtime* rt) {
  VK_REQUIRE(rt != nullptr, "null runtime");
  VK_REQUIRE(!rt->destroyed, "runtime was destroyed");
  return bind_device(rt);
}

int bind_device(vk_runtime* rt) {
  VK_REQUIRE(rt != nullptr, "null runtime");
  int cur = -1;
  VK_HIP(hipGetDevice(&cur));
  if (cur != rt->device) VK_HIP(hipSetDevice(rt->device));
  return VK_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, what);
  return VK_OK;
}

int check_rope_mode(unsigned rope_mode) {
  VK_REQUIRE((rope_mode & ~(VK_ROPE_INTERLEAVED | VK_ROPE_EXP_HEAD)) == 0,
             "unknown RoPE convention flags 0x%x", rope_mode);
  return VK_OK;
}

// Host build of the RoPE cos/sin table for head_dim 64 (two rotary halves of
// 32, 16 frequency pairs each).  inv_freq_j = 1 / base^((2j)/32) (exponent
// over the half, the default), or 1 / base^((2j)/64) with VK_ROPE_EXP_HEAD,
// each step in f32; angle = (f32)p * inv_freq_j as one f32 product; cos/sin
// evaluated in double and rounded once (the published
// RotaryPositionEmbedding2D of Depth-Anything-3 computes the same f32
// angle).  The pairing does not change the table: frequency j belongs to
// pair (j, j+16) or (2j, 2j+1).
int rope_table(vk_runtime* rt, float freq, int head_dim, unsigned rope_mode, int min_max_pos,
               const float** out, int* table_max) {
  VK_UNSUPPORTED_IF(head_dim != 64, "RoPE table supports head_dim 64 (got %d)", head_dim);
  VK_UNSUPPORTED_IF(min_max_pos > (1 << 22), "RoPE positions up to %d exceed the table limit",
                    min_max_pos);
  VK_TRY(check_rope_mode(rope_mode));
  const bool exp_head = (rope_mode & VK_ROPE_EXP_HEAD) != 0;
  uint32_t fbits;
  std::memcpy(&fbits, &freq, sizeof fbits);
  auto key = std::make_tuple(fbits, head_dim, exp_head ? 1 : 0);
  auto it = rt->rope_tables.find(key);
  if (it != rt->rope_tables.end() && it->second.second >= min_max_pos) {
    *out = it->second.first;
    *table_max = it->second.second;
    return VK_OK;
  }
  const int max_pos = min_max_pos > kRopeTableMax ? min_max_pos : kRopeTableMax;
  const int half = head_dim / 2;
  const int quarter = half / 2;
  std::vector<float> inv_freq(quarter);
  // exponent denominator: the rotary half's width, or the whole head
  const float denom = static_cast<float>(exp_head ? head_dim : half);
  for (int j = 0; j < quarter; ++j) {
    const float e = static_cast<float>(2 * j) / denom;
    inv_freq[j] = 1.0f / std::pow(freq, e);
  }
  const size_t entries = static_cast<size_t>(max_pos) + 1;
  std::vector<float> host(entries * 32 + 16, 0.0f);
  for (size_t p = 0; p < entries; ++p) {
    for (int j = 0; j < quarter; ++j) {
      const float angle = static_cast<float>(p) * inv_freq[j];
      host[p * 32 + j] = static_cast<float>(std::cos(static_cast<double>(angle)));
      host[p * 32 + 16 + j] = static_cast<float>(std::sin(static_cast<double>(angle)));
    }
  }
  for (int j = 0; j < quarter; ++j) host[entries * 32 + j] = inv_freq[j];
  VK_TRY(bind(rt));
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  VK_HIP(hipStreamIsCapturing(rt->stream, &st));
  VK_REQUIRE(st == hipStreamCaptureStatusNone,
             "RoPE table for positions up to %d must be built before stream capture "
             "(run the sequence once eagerly first)", min_max_pos);
  float* dev = nullptr;
  VK_HIP(hipMalloc(&dev, host.size() * sizeof(float)));
  hipError_t e = hipMemcpy(dev, host.data(), host.size() * sizeof(float),
                           hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    return hip_fail(e, "hipMemcpy(rope table)");
  }
  if (it != rt->rope_tables.end()) {
    // the smaller table may still be read by queued kernels or named by a
    // graph captured earlier: keep it until the runtime is destroyed
    rt->retired.push_back(it->second.first);
  }
  rt->rope_tables[key] = std::make_pair(dev, max_pos);
  *out = dev;
  *table_max = max_pos;
  return VK_OK;
}

void retain(vk_runtime* rt) {
  if (rt) rt->refs.fetch_add(1, std::memory_order_relaxed);
}

void release(vk_runtime* rt) {
  if (!rt || rt->refs.fetch_sub(1, std::memory_order_acq_rel) != 1) return;
  (void)bind_device(rt);
  (void)hipStreamSynchronize(rt->stream);
  for (auto& kv : rt->rope_tables) (void)hipFree(kv.second.first);
  if (rt->work) (void)hipFree(rt->work);
  for (void* p : rt->retired) (void)hipFree(p);
  (void)hipStreamDestroy(rt->stream);
  delete rt;
}

int ensure_work(vk_runtime* rt, size_t floats, const char* who) {
  if (rt->work_len >= floats) return VK_OK;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  VK_HIP(hipStreamIsCapturing(rt->stream, &st));
  VK_REQUIRE(st == hipStreamCaptureStatusNone,
             "%s: the work buffer must grow to %zu floats before stream capture "
             "(run the sequence once eagerly first)", who, floats);
  size_t len = floats > 2 * rt->work_len ? floats : 2 * rt->work_len;
  if (len < (size_t{8} << 20)) len = size_t{8} << 20;
  float* p = nullptr;
  VK_HIP(hipMalloc(reinterpret_cast<void**>(&p), len * sizeof(float)));
  // queued kernels or graphs captured earlier may still name the old one
  if (rt->work) rt->retired.push_back(rt->work);
  rt->work = p;
  rt->work_len = len;
  return VK_OK;
}

// Device-to-device copies as kernels.  16-byte aligned copies: persistent
// single-wave workgroups over 3 KiB chunks (three float4 per lane), wave w
// taking chunks w, w + W, ... (W = vk::stream_waves), the next chunk loaded
// before the current one is stored and each store issued after the wave's
// earlier memory operations (vkd::wait_memory), streaming (nontemporal)
// loads and stores -- the form of the path's out-of-place row streams
// (64 MB: 10.9 us against 12.3 for a whole-tensor grid of two float4 per
// thread); the last workgroup also copies the remainder (< 192 float4).
// Other alignments: 4-byte or 1-byte elements in a grid-stride loop over at
// most 4096 workgroups of 256 threads.
constexpr int kCopyChunk = 192;  // float4 per chunk: 3 per lane

__global__ __launch_bounds__(64) void copy16_kernel(float4* __restrict__ dst,
                                                    const float4* __restrict__ src,
                                                    size_t chunks, size_t n16) {
  const int lane = threadIdx.x;
  const size_t stride = gridDim.x;
  size_t ch = blockIdx.x;
  if (ch < chunks) {
    float4 cur[3], nxt[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) cur[i] = vkd::ld_stream(src + ch * kCopyChunk + lane + 64 * i);
    for (;;) {
      const size_t nch = ch + stride;
      const bool more = nch < chunks;
      if (more) {
#pragma unroll
        for (int i = 0; i < 3; ++i) nxt[i] = vkd::ld_stream(src + nch * kCopyChunk + lane + 64 * i);
      }
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        vkd::wait_memory();
        vkd::st_stream(dst + ch * kCopyChunk + lane + 64 * i, cur[i]);
      }
      if (!more) break;
      for (int i = 0; i < 3; ++i) cur[i] = nxt[i];
      ch = nch;
    }
  }
  if (blockIdx.x == gridDim.x - 1) {
    for (size_t i = chunks * kCopyChunk + lane; i < n16; i += 64)
      vkd::st_stream(dst + i, vkd::ld_stream(src + i));
  }
}

template <typename T>
__global__ void copy_elems_kernel(T* __restrict__ dst, const T* __restrict__ src, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride)
    dst[i] = src[i];
}

// One workgroup per view: row v * tpv of tokens <- camera slot (v > 0).
__global__ void camera_rows_kernel(float* __restrict__ tokens, const float* __restrict__ camera,
                                   size_t tpv, size_t D) {
  const size_t v = blockIdx.x;
  const float* src = camera + (v > 0 ? D : 0);
  float* dst = tokens + v * tpv * D;
  for (size_t c = threadIdx.x; c < D; c += blockDim.x) dst[c] = src[c];
}

int device_copy(vk_runtime* rt, void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return VK_OK;
  const uintptr_t a = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes;
  const size_t unit = (a & 15) == 0 ? 16 : (a & 3) == 0 ? 4 : 1;
  const size_t n = bytes / unit;
  if (unit == 16) {
    const size_t chunks = n / kCopyChunk;
    hipLaunchKernelGGL(copy16_kernel, dim3(stream_waves(rt, static_cast<long long>(chunks))),
                       dim3(64), 0, rt->stream, static_cast<float4*>(dst),
                       static_cast<const float4*>(src), chunks, n);
    return check_launch("device copy");
  }
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  if (unit == 4)
    hipLaunchKernelGGL(copy_elems_kernel<uint32_t>, grid, block, 0, rt->stream,
                       static_cast<uint32_t*>(dst), static_cast<const uint32_t*>(src), n);
  else
    hipLaunchKernelGGL(copy_elems_kernel<uint8_t>, grid, block, 0, rt->stream,
                       static_cast<uint8_t*>(dst), static_cast<const uint8_t*>(src), n);
  return check_launch("device copy");
}

int write_camera_rows(vk_runtime* rt, float* tokens, const float* camera, size_t view_count,
                      size_t tokens_per_view, size_t D) {
  if (view_count == 0 || D == 0) return VK_OK;
  VK_UNSUPPORTED_IF(view_count > 0x7fffffffULL, "camera write: %zu views", view_count);
  hipLaunchKernelGGL(camera_rows_kernel, dim3(static_cast<unsigned>(view_count)), dim3(256), 0,
                     rt->stream, tokens, camera, tokens_per_view, D);
  return check_launch("camera_rows_kernel");
}

static int new_tensor(vk_runtime* rt, vk_dtype dtype, size_t len, vk_tensor** out) {
  VK_REQUIRE(out != nullptr, "null output handle");
  VK_REQUIRE(dtype_size(dtype) != 0, "unknown dtype %d", static_cast<int>(dtype));
  VK_TRY(bind(rt));
  void* p = nullptr;
  if (len > 0) VK_HIP(hipMalloc(&p, len * dtype_size(dtype)));
  auto* t = new vk_tensor;
  t->rt = rt;
  retain(rt);
  t->ptr = p;
  t->len = len;
  t->dtype = dtype;
  t->owned = true;
  *out = t;
  return VK_OK;
}

static int upload(vk_runtime* rt, vk_dtype dtype, const void* host, size_t len,
                  vk_tensor** out) {
  VK_REQUIRE(host != nullptr || len == 0, "null host pointer");
  vk_tensor* t = nullptr;
  VK_TRY(new_tensor(rt, dtype, len, &t));
  if (len > 0) {
    hipError_t e = hipMemcpyAsync(t->ptr, host, len * dtype_size(dtype),
                                  hipMemcpyHostToDevice, rt->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) {
      vk_tensor_destroy(t);
      return hip_fail(e, "upload");
    }
  }
  *out = t;
  return VK_OK;
}

}  // namespace vk

using namespace vk;

extern "C" {

const char* vk_last_error(void) { return g_last_error.c_str(); }

int vk_abi_version(void) { return VK_ABI_VERSION; }

int vk_runtime_create(int device, vk_runtime** out) {
  clear_error();
  VK_REQUIRE(out != nullptr, "null output handle");
  int count = 0;
  VK_HIP(hipGetDeviceCount(&count));
  VK_REQUIRE(device >= 0 && device < count, "device %d out of range (%d devices)",
             device, count);
  VK_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  VK_HIP(hipGetDeviceProperties(&prop, device));
  // with `device` current: the allocation-free entry point's scratch address
  vk::noalloc_setup(device);
  auto* rt = new vk_runtime;
  rt->device = device;
  rt->cu_count = prop.multiProcessorCount;
  // Default priority, non-blocking with respect to the null stream.
  hipError_t e = hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete rt;
    return hip_fail(e, "hipStreamCreateWithFlags");
  }
  *out = rt;
  return VK_OK;
}

int vk_runtime_destroy(vk_runtime* rt) {
  if (!rt) return VK_OK;
  VK_TRY(bind(rt));  // also refuses a second destroy of a runtime still alive
  (void)hipStreamSynchronize(rt->stream);
  rt->destroyed = true;
  release(rt);
  return VK_OK;
}

int vk_runtime_synchronize(vk_runtime* rt) {
  VK_TRY(bind(rt));
  VK_HIP(hipStreamSynchronize(rt->stream));
  return VK_OK;
}

void* vk_runtime_stream(vk_runtime* rt) { return rt ? static_cast<void*>(rt->stream) : nullptr; }

int vk_runtime_cu_count(vk_runtime* rt) { return rt ? rt->cu_count : 0; }

int vk_runtime_set_layernorm_order(vk_runtime* rt, int order) {
  VK_REQUIRE(rt != nullptr, "null runtime");
  VK_REQUIRE(!rt->destroyed, "runtime was destroyed");
  VK_REQUIRE(order == VK_LN_ORDER_TREE || order == VK_LN_ORDER_SEQUENTIAL,
             "unknown LayerNorm order %d", order);
  rt->ln_order = order;
  return VK_OK;
}

int vk_runtime_layernorm_order(vk_runtime* rt) {
  VK_REQUIRE(rt != nullptr, "null runtime");
  return rt->ln_order;
}

int vk_tensor_alloc(vk_runtime* rt, vk_dtype dtype, size_t len, vk_tensor** out) {
  return new_tensor(rt, dtype, len, out);
}

int vk_tensor_wrap(vk_runtime* rt, vk_dtype dtype, void* device_ptr, size_t len,
                   vk_tensor** out) {
  VK_REQUIRE(rt != nullptr && out != nullptr, "null runtime or output handle");
  VK_REQUIRE(device_ptr != nullptr || len == 0, "null device pointer");
  VK_REQUIRE(dtype_size(dtype) != 0, "unknown dtype %d", static_cast<int>(dtype));
  VK_REQUIRE(!rt->destroyed, "runtime was destroyed");
  auto* t = new vk_tensor;
  t->rt = rt;
  retain(rt);
  t->ptr = device_ptr;
  t->len = len;
  t->dtype = dtype;
  t->owned = false;
  *out = t;
  return VK_OK;
}

int vk_tensor_destroy(vk_tensor* t) {
  if (!t) return VK_OK;
  vk_runtime* rt = t->rt;
  hipError_t e = hipSuccess;
  if (t->owned && t->ptr) {
    VK_TRY(bind_device(rt));
    // Stream-ordered: pending kernels that read the buffer finish first.
    (void)hipStreamSynchronize(rt->stream);
    e = hipFree(t->ptr);
  }
  delete t;
  release(rt);
  if (e != hipSuccess) return hip_fail(e, "hipFree");
  return VK_OK;
}

size_t vk_tensor_len(const vk_tensor* t) { return t ? t->len : 0; }

int vk_tensor_dtype(const vk_tensor* t) { return t ? static_cast<int>(t->dtype) : -1; }

void* vk_tensor_device_ptr(const vk_tensor* t) { return t ? t->ptr : nullptr; }

int vk_upload_f32(vk_runtime* rt, const float* host, size_t len, vk_tensor** out) {
  return upload(rt, VK_F32, host, len, out);
}

int vk_upload_f16(vk_runtime* rt, const uint16_t* host, size_t len, vk_tensor** out) {
  return upload(rt, VK_F16, host, len, out);
}

int vk_upload_u8(vk_runtime* rt, const uint8_t* host, size_t len, vk_tensor** out) {
  return upload(rt, VK_U8, host, len, out);
}

int vk_upload_i32(vk_runtime* rt, const int32_t* host, size_t len, vk_tensor** out) {
  return upload(rt, VK_I32, host, len, out);
}

int vk_upload_i64(vk_runtime* rt, const int64_t* host, size_t len, vk_tensor** out) {
  return upload(rt, VK_I64, host, len, out);
}

static int write_host(vk_runtime* rt, vk_tensor* t, vk_dtype dtype,
                      const void* host, size_t len) {
  VK_REQUIRE(t != nullptr && (host != nullptr || len == 0), "null tensor or host pointer");
  VK_REQUIRE(t->dtype == dtype, "tensor dtype %d, expected %d",
             static_cast<int>(t->dtype), static_cast<int>(dtype));
  VK_REQUIRE(t->len == len, "length mismatch: tensor %zu, host %zu", t->len, len);
  VK_TRY(bind(rt));
  if (len == 0) return VK_OK;
  VK_HIP(hipMemcpyAsync(t->ptr, host, len * dtype_size(dtype), hipMemcpyHostToDevice,
                        rt->stream));
  VK_HIP(hipStreamSynchronize(rt->stream));
  return VK_OK;
}

int vk_write_f32(vk_runtime* rt, vk_tensor* t, const float* host, size_t len) {
  return write_host(rt, t, VK_F32, host, len);
}

int vk_write_u8(vk_runtime* rt, vk_tensor* t, const uint8_t* host, size_t len) {
  return write_host(rt, t, VK_U8, host, len);
}

int vk_download_f32(vk_runtime* rt, const vk_tensor* t, float* host, size_t len) {
  VK_REQUIRE(t != nullptr && (host != nullptr || len == 0), "null tensor or host pointer");
  VK_REQUIRE(t->dtype == VK_F32, "download_f32 of a non-f32 tensor");
  VK_REQUIRE(t->len == len, "length mismatch: tensor %zu, host %zu", t->len, len);
  VK_TRY(bind(rt));
  if (len > 0)
    VK_HIP(hipMemcpyAsync(host, t->ptr, len * 4, hipMemcpyDeviceToHost, rt->stream));
  VK_HIP(hipStreamSynchronize(rt->stream));
  return VK_OK;
}

int vk_download_u8(vk_runtime* rt, const vk_tensor* t, uint8_t* host, size_t len) {
  VK_REQUIRE(t != nullptr && (host != nullptr || len == 0), "null tensor or host pointer");
  VK_REQUIRE(t->dtype == VK_U8, "download_u8 of a non-u8 tensor");
  VK_REQUIRE(t->len == len, "length mismatch: tensor %zu, host %zu", t->len, len);
  VK_TRY(bind(rt));
  if (len > 0) VK_HIP(hipMemcpyAsync(host, t->ptr, len, hipMemcpyDeviceToHost, rt->stream));
  VK_HIP(hipStreamSynchronize(rt->stream));
  return VK_OK;
}

int vk_copy_f32(vk_runtime* rt, const vk_tensor* src, vk_tensor** out) {
  VK_REQUIRE(src != nullptr, "null source");
  return vk_copy_segment_f32(rt, src, 0, src->len, out);
}

int vk_copy_segment_f32(vk_runtime* rt, const vk_tensor* src, size_t offset,
                        size_t len, vk_tensor** out) {
  VK_REQUIRE(src != nullptr && out != nullptr, "null source or output handle");
  VK_REQUIRE(src->dtype == VK_F32, "copy_segment_f32 of a non-f32 tensor");
  VK_REQUIRE(offset <= src->len && len <= src->len - offset,
             "segment [%zu, +%zu) outside tensor of %zu", offset, len, src->len);
  vk_tensor* t = nullptr;
  VK_TRY(new_tensor(rt, VK_F32, len, &t));
  const int s = device_copy(rt, t->ptr, static_cast<const float*>(src->ptr) + offset, len * 4);
  if (s != VK_OK) {
    vk_tensor_destroy(t);
    return s;
  }
  *out = t;
  return VK_OK;
}

int vk_copy_segment_into_f32(vk_runtime* rt, vk_tensor* dst, size_t dst_offset,
                             const vk_tensor* src, size_t src_offset, size_t len) {
  VK_REQUIRE(dst != nullptr && src != nullptr, "null tensor");
  VK_REQUIRE(dst->dtype == VK_F32 && src->dtype == VK_F32, "non-f32 tensor");
  VK_REQUIRE(src_offset <= src->len && len <= src->len - src_offset,
             "source segment [%zu, +%zu) outside tensor of %zu", src_offset, len, src->len);
  VK_REQUIRE(dst_offset <= dst->len && len <= dst->len - dst_offset,
             "destination segment [%zu, +%zu) outside tensor of %zu", dst_offset, len,
             dst->len);
  VK_TRY(bind(rt));
  return device_copy(rt, static_cast<float*>(dst->ptr) + dst_offset,
                     static_cast<const float*>(src->ptr) + src_offset, len * 4);
}

int vk_overwrite_prefix_f32(vk_runtime* rt, vk_tensor* tokens, const vk_tensor* prefix,
                            size_t len) {
  return vk_copy_segment_into_f32(rt, tokens, 0, prefix, 0, len);
}

int vk_event_create(vk_runtime* rt, vk_event** out) {
  VK_REQUIRE(out != nullptr, "null output handle");
  VK_TRY(bind(rt));
  auto* e = new vk_event;
  e->rt = rt;
  hipError_t err = hipEventCreate(&e->ev);
  if (err != hipSuccess) {
    delete e;
    return hip_fail(err, "hipEventCreate");
  }
  retain(rt);
  *out = e;
  return VK_OK;
}

int vk_event_destroy(vk_event* ev) {
  if (!ev) return VK_OK;
  vk_runtime* rt = ev->rt;
  if (bind_device(rt) == VK_OK) (void)hipEventDestroy(ev->ev);
  delete ev;
  release(rt);
  return VK_OK;
}

int vk_event_record(vk_runtime* rt, vk_event* ev) {
  VK_REQUIRE(ev != nullptr, "null event");
  VK_TRY(bind(rt));
  VK_HIP(hipEventRecord(ev->ev, rt->stream));
  return VK_OK;
}

int vk_event_elapsed_ms(vk_event* start, vk_event* stop, float* ms) {
  VK_REQUIRE(start && stop && ms, "null argument");
  VK_HIP(hipEventSynchronize(stop->ev));
  VK_HIP(hipEventElapsedTime(ms, start->ev, stop->ev));
  return VK_OK;
}

int vk_graph_begin_capture(vk_runtime* rt) {
  VK_TRY(bind(rt));
  VK_HIP(hipStreamBeginCapture(rt->stream, hipStreamCaptureModeThreadLocal));
  return VK_OK;
}

int vk_graph_end_capture(vk_runtime* rt, vk_graph** out) {
  VK_REQUIRE(out != nullptr, "null output handle");
  VK_TRY(bind(rt));
  hipGraph_t g = nullptr;
  VK_HIP(hipStreamEndCapture(rt->stream, &g));
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(e, "hipGraphInstantiate");
  }
  auto* vg = new vk_graph;
  vg->rt = rt;
  retain(rt);
  vg->graph = g;
  vg->exec = exec;
  *out = vg;
  return VK_OK;
}

int vk_graph_launch(vk_runtime* rt, vk_graph* g) {
  VK_REQUIRE(g != nullptr && g->exec != nullptr, "null graph");
  // a graph's nodes use its runtime's work buffer and tables: it runs on
  // that runtime's stream only, and not after the runtime was destroyed
  VK_REQUIRE(rt == g->rt, "graph was captured on another runtime");
  VK_TRY(bind(rt));
  VK_HIP(hipGraphLaunch(g->exec, rt->stream));
  return VK_OK;
}

int vk_graph_destroy(vk_graph* g) {
  if (!g) return VK_OK;
  vk_runtime* rt = g->rt;
  if (bind_device(rt) == VK_OK) {
    // launches still queued on the stream finish before their exec goes
    (void)hipStreamSynchronize(rt->stream);
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
  }
  delete g;
  release(rt);
  return VK_OK;
}

}  // extern "C"
