"""Python binding of libvestra_hip.so (the C ABI declared in include/vestra_hip.h).

The classes mirror the reference engine's device runtime,
``vestra_kernels::cuda::CudaRuntime`` (called from
crates/da-engine/src/vit_block.rs:136-667 and patch_embed.rs:139-245): the
same method names, argument meaning and error behaviour.  A failed call raises
``VestraError`` carrying the C status and message (the reference's
``CudaError::Kernel(String)``); ``UnsupportedShape`` marks a shape outside the
qualified subset, which the reference maps to ``None`` / CPU fallback
(vit_block.rs:331-333).

The library must be built in-tree (``make -C vestra-engine_amd``); importing
this module without it raises immediately -- there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvestra_hip.so")

VK_OK = 0
VK_ERR_INVALID = -1
VK_ERR_UNSUPPORTED = -2
VK_ERR_HIP = -3
VK_ERR_OOM = -4

VK_F32, VK_F16, VK_U8, VK_I32, VK_I64 = 0, 1, 2, 3, 4
# 2D RoPE convention flags (pairing | exponent); 0 is the default
VK_ROPE_ROTATE_HALF, VK_ROPE_INTERLEAVED = 0, 1
VK_ROPE_EXP_HALF, VK_ROPE_EXP_HEAD = 0, 2
VK_ROPE_DEFAULT = 0
VK_QK_HEADS_OUTER, VK_QK_VIEWS_OUTER = 0, 1
# LayerNorm summation order of a runtime (vk_runtime_set_layernorm_order)
VK_LN_ORDER_TREE, VK_LN_ORDER_SEQUENTIAL = 0, 1
VK_RESIZE_BILINEAR, VK_RESIZE_CUBIC, VK_RESIZE_AREA = 0, 1, 2

VK_BLOCK_FUSE_LS_LN = 1
VK_BLOCK_SKIP_LN1 = 2
VK_BLOCK_FUSE_NEXT_LN1 = 4
VK_BLOCK_CAMERA_WRITTEN = 8

QK_NORM_EPS = 1e-5  # vit_block.rs:686


class VestraError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class UnsupportedShape(VestraError):
    pass


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C {_HERE}` "
            "(there is no non-HIP fallback)")
    return C.CDLL(LIB_PATH)


lib = _load()

_vp = C.c_void_p
_sz = C.c_size_t
_i = C.c_int
_f = C.c_float
_pp = C.POINTER(C.c_void_p)


class VitConfig(C.Structure):
    _fields_ = [("embed_dim", _sz), ("num_heads", _sz), ("head_dim", _sz),
                ("mlp_hidden", _sz), ("num_register", _sz), ("ln_eps", _f),
                ("qk_norm_eps", _f), ("rope_freq", _f), ("rope_start", _i),
                ("qknorm_start", _i), ("alt_start", _i), ("rope_mode", C.c_uint)]


class VitLayer(C.Structure):
    _fields_ = [(n, _vp) for n in (
        "norm1_gamma", "norm1_beta", "qnorm_gamma", "qnorm_beta", "knorm_gamma",
        "knorm_beta", "ls1", "norm2_gamma", "norm2_beta", "ls2")]


class VitActivations(C.Structure):
    _fields_ = [(n, _vp) for n in (
        "tokens", "ln1", "q", "k", "attn_proj", "ln2", "hidden", "mlp_out")]


class VitBlockWeights(C.Structure):
    _fields_ = [(n, _vp) for n in (
        "norm1_gamma", "norm1_beta", "qkv", "qnorm_gamma", "qnorm_beta", "knorm_gamma",
        "knorm_beta", "proj", "norm2_gamma", "norm2_beta", "fc1", "fc2")]


class VitBlockWorkspace(C.Structure):
    _fields_ = [(n, _vp) for n in ("ln", "q", "k", "v", "attn", "hidden")]


_SIGS = {
    "vk_last_error": ([], C.c_char_p),
    "vk_abi_version": ([], _i),
    "vk_runtime_create": ([_i, _pp], _i),
    "vk_runtime_destroy": ([_vp], _i),
    "vk_runtime_synchronize": ([_vp], _i),
    "vk_runtime_stream": ([_vp], _vp),
    "vk_runtime_cu_count": ([_vp], _i),
    "vk_runtime_set_layernorm_order": ([_vp, _i], _i),
    "vk_runtime_layernorm_order": ([_vp], _i),
    "vk_tensor_alloc": ([_vp, _i, _sz, _pp], _i),
    "vk_tensor_wrap": ([_vp, _i, _vp, _sz, _pp], _i),
    "vk_tensor_destroy": ([_vp], _i),
    "vk_tensor_len": ([_vp], _sz),
    "vk_tensor_dtype": ([_vp], _i),
    "vk_tensor_device_ptr": ([_vp], _vp),
    "vk_upload_f32": ([_vp, _vp, _sz, _pp], _i),
    "vk_upload_f16": ([_vp, _vp, _sz, _pp], _i),
    "vk_upload_u8": ([_vp, _vp, _sz, _pp], _i),
    "vk_upload_i32": ([_vp, _vp, _sz, _pp], _i),
    "vk_upload_i64": ([_vp, _vp, _sz, _pp], _i),
    "vk_write_f32": ([_vp, _vp, _vp, _sz], _i),
    "vk_write_u8": ([_vp, _vp, _vp, _sz], _i),
    "vk_download_f32": ([_vp, _vp, _vp, _sz], _i),
    "vk_download_u8": ([_vp, _vp, _vp, _sz], _i),
    "vk_copy_f32": ([_vp, _vp, _pp], _i),
    "vk_copy_segment_f32": ([_vp, _vp, _sz, _sz, _pp], _i),
    "vk_copy_segment_into_f32": ([_vp, _vp, _sz, _vp, _sz, _sz], _i),
    "vk_overwrite_prefix_f32": ([_vp, _vp, _vp, _sz], _i),
    "vk_layernorm_f32": ([_vp, _vp, _vp, _vp, _sz, _sz, _f, _pp], _i),
    "vk_layernorm_into_f32": ([_vp, _vp, _vp, _vp, _sz, _sz, _f, _vp], _i),
    "vk_gelu_f32_inplace": ([_vp, _vp], _i),
    "vk_gelu_erf_f32_inplace": ([_vp, _vp], _i),
    "vk_add_f32_inplace": ([_vp, _vp, _vp], _i),
    "vk_layerscale_f32_inplace": ([_vp, _vp, _vp, _sz, _sz], _i),
    "vk_layerscale_residual_f32": ([_vp, _vp, _vp, _vp, _sz, _sz], _i),
    "vk_layerscale_residual_layernorm_f32": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _f, _vp], _i),
    "vk_qk_norm_rope_f32": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _f, _f], _i),
    "vk_qk_norm_rope_mode_f32": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _f, _f, C.c_uint], _i),
    "vk_rope2d_f32": ([_vp, _vp, _vp, _sz, _sz, _sz, _f, C.c_uint], _i),
    "vk_qk_norm_rope_grid_f32": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _i, _i, _f, _f], _i),
    "vk_qk_norm_rope_grid_mode_f32": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _i, _i, _f, _f,
         C.c_uint], _i),
    "vk_rope_positions_f32": ([_vp, _sz, _sz, _sz, _sz, _i, _pp], _i),
    "vk_patchify_nchw_f32": ([_vp, _vp, _sz, _sz, _sz, _sz, _pp], _i),
    "vk_linear_prepare_f32": ([_vp, _sz, _sz, _vp, _vp, _vp, _pp], _i),
    "vk_linear_prepare_oihw_f32": ([_vp, _sz, _sz, _vp, _vp, _pp], _i),
    "vk_linear_prepare_w16": ([_vp, _sz, _sz, _vp, _vp, _vp, _pp], _i),
    "vk_linear_prepare_q8_0": ([_vp, _sz, _sz, _vp, _sz, _vp, _vp, _pp], _i),
    "vk_linear_prepare_oihw_w16": ([_vp, _sz, _sz, _vp, _vp, _pp], _i),
    "vk_widen_f16_f32": ([_vp, _vp, _vp], _i),
    "vk_dequantize_q8_0_f32": ([_vp, _vp, _sz, _vp], _i),
    "vk_linear_destroy": ([_vp], _i),
    "vk_linear_input_features": ([_vp], _sz),
    "vk_linear_run_f32": ([_vp, _vp, _vp, _sz, _pp], _i),
    "vk_linear_run_into_f32": ([_vp, _vp, _vp, _sz, _vp], _i),
    "vk_linear_run_into_noalloc_f32": ([_vp, _vp, _vp, _sz, _vp], _i),
    "vk_linear_run_gelu_f32": ([_vp, _vp, _vp, _sz, _vp], _i),
    "vk_linear_run_gelu_erf_f32": ([_vp, _vp, _vp, _sz, _vp], _i),
    "vk_linear_run_residual_f32": ([_vp, _vp, _vp, _sz, _vp], _i),
    "vk_linear_run_qkv_hnd_f32": ([_vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp], _i),
    "vk_linear_run_qkv_hnd_norm_rope_f32": (
        [_vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _i,
         _f, _f], _i),
    "vk_linear_run_qkv_hnd_norm_rope_mode_f32": (
        [_vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _i,
         _f, _f, C.c_uint], _i),
    "vk_linear_run_hnd_into_f32": ([_vp, _vp, _vp, _sz, _sz, _sz, _vp], _i),
    "vk_linear_run_hnd_residual_f32": ([_vp, _vp, _vp, _sz, _sz, _sz, _vp], _i),
    "vk_split_qkv_hnd_f32": ([_vp, _vp, _sz, _sz, _sz, _pp, _pp, _pp], _i),
    "vk_split_qkv_hnd_into_f32": ([_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp], _i),
    "vk_hnd_to_token_f32": ([_vp, _vp, _sz, _sz, _sz, _pp], _i),
    "vk_hnd_to_token_into_f32": ([_vp, _vp, _sz, _sz, _sz, _vp], _i),
    "vk_capture_f32": ([_vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _vp, _f, _i, _vp, _vp], _i),
    "vk_token_to_chw_f32": ([_vp, _vp, _sz, _sz, _vp, _vp, _f, _vp], _i),
    "vk_resize_workspace_bytes": ([_sz, _sz, _sz, _sz, _i], _sz),
    "vk_resize_u8": ([_vp, _vp, _sz, _sz, _vp, _sz, _sz, _i, _vp], _i),
    "vk_preprocess_shape": ([_sz, _sz, _sz, _sz, _i, C.POINTER(_sz), C.POINTER(_sz)], _i),
    "vk_preprocess_workspace_bytes": ([_sz, _sz, _sz, _sz, _i], _sz),
    "vk_preprocess_resize_u8": ([_vp, _vp, _sz, _sz, _sz, _sz, _i, _vp, _vp], _i),
    "vk_normalize_u8_hwc_nchw_f32": ([_vp, _vp, _sz, _sz, _vp, _vp, _vp], _i),
    "vk_attention_online_f32": ([_vp, _vp, _vp, _vp, _sz, _sz, _sz, _pp], _i),
    "vk_attention_into_f32": ([_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp], _i),
    "vk_prepend_cls_add_pos_f32": ([_vp, _vp, _vp, _vp, _sz, _sz, _pp], _i),
    "vk_pos_embed_bicubic_f32": ([_vp, _vp, _sz, _sz, _sz, _sz, _f, _pp], _i),
    "vk_patch_embed_u8": ([_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp], _i),
    "vk_patch_embed_views_u8": (
        [_vp, _vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp], _i),
    "vk_vit_block_fused_ops": (
        [_vp, C.POINTER(VitConfig), _sz, C.POINTER(VitLayer), C.POINTER(VitLayer),
         C.POINTER(VitActivations), _sz, _sz, _sz, _vp, C.c_uint], _i),
    "vk_vit_block_forward_f32": (
        [_vp, C.POINTER(VitConfig), _sz, C.POINTER(VitBlockWeights), _vp, _sz, _sz, _sz, _vp,
         C.POINTER(VitBlockWorkspace)], _i),
    "vk_backbone_forward_f32": (
        [_vp, C.POINTER(VitConfig), _sz, C.POINTER(VitBlockWeights), _vp, _sz, _sz, _sz, _vp,
         _vp, _vp, _i, C.POINTER(C.c_int), _sz, C.POINTER(_vp), C.POINTER(_vp),
         C.POINTER(VitBlockWorkspace), _vp], _i),
    "vk_event_create": ([_vp, _pp], _i),
    "vk_event_destroy": ([_vp], _i),
    "vk_event_record": ([_vp, _vp], _i),
    "vk_event_elapsed_ms": ([_vp, _vp, C.POINTER(C.c_float)], _i),
    "vk_graph_begin_capture": ([_vp], _i),
    "vk_graph_end_capture": ([_vp, _pp], _i),
    "vk_graph_launch": ([_vp, _vp], _i),
    "vk_graph_destroy": ([_vp], _i),
}

for _name, (_args, _res) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res


def _check(status: int) -> None:
    if status != VK_OK:
        msg = lib.vk_last_error().decode(errors="replace")
        cls = UnsupportedShape if status == VK_ERR_UNSUPPORTED else VestraError
        raise cls(status, msg)


def _ptr(a: np.ndarray) -> C.c_void_p:
    # data_as keeps a reference to the array alive as long as the pointer
    return a.ctypes.data_as(C.c_void_p)


class Tensor:
    """Owned (or wrapped) device tensor: ``CudaTensorF32`` of the reference."""

    def __init__(self, rt: "Runtime", handle: C.c_void_p):
        self.rt = rt
        self.handle = handle

    def __len__(self) -> int:
        return int(lib.vk_tensor_len(self.handle))

    @property
    def dtype(self) -> int:
        return int(lib.vk_tensor_dtype(self.handle))

    @property
    def device_ptr(self) -> int:
        return int(lib.vk_tensor_device_ptr(self.handle) or 0)

    def view(self, offset: int, length: int) -> "Tensor":
        """Non-owning view of elements [offset, offset + length), of this
        tensor's dtype; keeps this tensor alive while the view lives."""
        if offset < 0 or length < 0 or offset + length > len(self):
            raise VestraError(VK_ERR_INVALID, "view out of range")
        dt = self.dtype
        size = {VK_F32: 4, VK_F16: 2, VK_U8: 1, VK_I32: 4, VK_I64: 8}[dt]
        out = C.c_void_p()
        _check(lib.vk_tensor_wrap(self.rt.handle, dt, self.device_ptr + size * offset, length,
                                  C.byref(out)))
        t = Tensor(self.rt, out)
        t._base = self
        return t

    def numpy(self) -> np.ndarray:
        return self.rt.download_f32(self)

    def write(self, host: np.ndarray) -> None:
        if host.dtype == np.uint8:
            h = np.ascontiguousarray(host).reshape(-1)
            _check(lib.vk_write_u8(self.rt.handle, self.handle, _ptr(h), h.size))
        else:
            h = np.ascontiguousarray(host, dtype=np.float32).reshape(-1)
            _check(lib.vk_write_f32(self.rt.handle, self.handle, _ptr(h), h.size))

    def free(self) -> None:
        if self.handle:
            _check(lib.vk_tensor_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.handle:
                lib.vk_tensor_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def _h(t: Optional[Tensor]):
    return None if t is None else t.handle


class Linear:
    """``CudaLinearF32``: cached device weights, ``run(x, rows)``."""

    def __init__(self, rt: "Runtime", handle: C.c_void_p):
        self.rt = rt
        self.handle = handle

    def input_features(self) -> int:
        return int(lib.vk_linear_input_features(self.handle))

    def run(self, x: Tensor, rows: int) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_linear_run_f32(self.rt.handle, self.handle, x.handle, rows, C.byref(out)))
        return Tensor(self.rt, out)

    def run_into(self, x: Tensor, rows: int, out: Tensor) -> None:
        _check(lib.vk_linear_run_into_f32(self.rt.handle, self.handle, x.handle, rows, out.handle))

    def run_into_noalloc(self, x: Tensor, rows: int, out: Tensor) -> None:
        """run_into with split-K partial sums in the library's static device
        scratch: allocates nothing."""
        _check(lib.vk_linear_run_into_noalloc_f32(self.rt.handle, self.handle, x.handle, rows,
                                                  out.handle))

    def run_gelu(self, x: Tensor, rows: int, out: Tensor, exact_erf: bool = False) -> None:
        """FC1 + GELU: out = GELU(x W + b); A&S erf, or the device erff."""
        fn = lib.vk_linear_run_gelu_erf_f32 if exact_erf else lib.vk_linear_run_gelu_f32
        _check(fn(self.rt.handle, self.handle, x.handle, rows, out.handle))

    def run_qkv_hnd(self, x: Tensor, rows: int, heads: int, q: Tensor, k: Tensor,
                    v: Tensor, head_dim: int = 64) -> None:
        """QKV projection storing head-major Q, K, V [heads, rows, 64]."""
        _check(lib.vk_linear_run_qkv_hnd_f32(self.rt.handle, self.handle, x.handle, rows, heads,
                                             head_dim, q.handle, k.handle, v.handle))

    def run_hnd_into(self, hnd: Tensor, rows: int, heads: int, out: Tensor,
                     head_dim: int = 64) -> None:
        """Projection of a head-major input [heads, rows, 64]."""
        _check(lib.vk_linear_run_hnd_into_f32(self.rt.handle, self.handle, hnd.handle, rows,
                                              heads, head_dim, out.handle))

    def run_qkv_hnd_norm_rope(self, x: Tensor, rows: int, heads: int, q: Tensor, k: Tensor,
                              v: Tensor, q_gamma: Optional[Tensor], q_beta: Optional[Tensor],
                              k_gamma: Optional[Tensor], k_beta: Optional[Tensor],
                              n_special: int, gh: int, gw: int, view_count: int,
                              global_layer: bool, freq: float = 100.0,
                              eps: float = 1e-5, rope_mode: Optional[int] = None) -> None:
        """QKV projection storing head-major Q, K, V with Q/K-norm + RoPE fused;
        rope_mode None calls the default-convention entry point."""
        args = (self.rt.handle, self.handle, x.handle, rows, heads, 64, q.handle, k.handle,
                v.handle, _h(q_gamma), _h(q_beta), _h(k_gamma), _h(k_beta), n_special, gh, gw,
                view_count, 1 if global_layer else 0, freq, eps)
        if rope_mode is None:
            _check(lib.vk_linear_run_qkv_hnd_norm_rope_f32(*args))
        else:
            _check(lib.vk_linear_run_qkv_hnd_norm_rope_mode_f32(*args, rope_mode))

    def run_hnd_residual(self, hnd: Tensor, rows: int, heads: int, residual: Tensor,
                         head_dim: int = 64) -> None:
        """residual += (hnd as token rows) W + b [* gamma]."""
        _check(lib.vk_linear_run_hnd_residual_f32(self.rt.handle, self.handle, hnd.handle, rows,
                                                  heads, head_dim, residual.handle))

    def run_residual(self, x: Tensor, rows: int, residual: Tensor) -> None:
        """proj / FC2 + LayerScale + residual: residual += (x W + b) [* gamma]."""
        _check(lib.vk_linear_run_residual_f32(self.rt.handle, self.handle, x.handle, rows,
                                              residual.handle))

    def __del__(self):
        try:
            if self.handle:
                lib.vk_linear_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Event:
    def __init__(self, rt: "Runtime"):
        self.rt = rt
        h = C.c_void_p()
        _check(lib.vk_event_create(rt.handle, C.byref(h)))
        self.handle = h

    def record(self) -> None:
        _check(lib.vk_event_record(self.rt.handle, self.handle))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = C.c_float()
        _check(lib.vk_event_elapsed_ms(self.handle, stop.handle, C.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            lib.vk_event_destroy(self.handle)
        except Exception:
            pass


class Graph:
    def __init__(self, rt: "Runtime", handle: C.c_void_p):
        self.rt = rt
        self.handle = handle

    def launch(self) -> None:
        _check(lib.vk_graph_launch(self.rt.handle, self.handle))

    def __del__(self):
        try:
            lib.vk_graph_destroy(self.handle)
        except Exception:
            pass


class Runtime:
    """``vestra_kernels::cuda::CudaRuntime`` on one MI355X (one HIP stream)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib.vk_runtime_create(device, C.byref(h)))
        self.handle = h

    # -- runtime -------------------------------------------------------------
    def synchronize(self) -> None:
        _check(lib.vk_runtime_synchronize(self.handle))

    def cu_count(self) -> int:
        return int(lib.vk_runtime_cu_count(self.handle))

    def set_layernorm_order(self, order: int) -> None:
        """Summation order of every LayerNorm enqueued from now on:
        VK_LN_ORDER_TREE (default) or VK_LN_ORDER_SEQUENTIAL, the CPU
        kernel's left-to-right sums and its bits (layernorm_f32_cpu_order,
        vit_block.rs:528-537)."""
        _check(lib.vk_runtime_set_layernorm_order(self.handle, order))

    def layernorm_order(self) -> int:
        r = int(lib.vk_runtime_layernorm_order(self.handle))
        if r < 0:
            _check(r)
        return r

    def close(self) -> None:
        if self.handle:
            _check(lib.vk_runtime_destroy(self.handle))
            self.handle = None

    # -- tensors -------------------------------------------------------------
    def alloc_f32(self, n: int) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_tensor_alloc(self.handle, VK_F32, n, C.byref(out)))
        return Tensor(self, out)

    def upload_f32(self, host: np.ndarray) -> Tensor:
        h = np.ascontiguousarray(host, dtype=np.float32).reshape(-1)
        out = C.c_void_p()
        _check(lib.vk_upload_f32(self.handle, _ptr(h), h.size, C.byref(out)))
        return Tensor(self, out)

    def upload_f16(self, host: np.ndarray) -> Tensor:
        h = np.ascontiguousarray(host, dtype=np.float16).reshape(-1).view(np.uint16)
        out = C.c_void_p()
        _check(lib.vk_upload_f16(self.handle, _ptr(h), h.size, C.byref(out)))
        return Tensor(self, out)

    def upload_i32(self, host: np.ndarray) -> Tensor:
        h = np.ascontiguousarray(host, dtype=np.int32).reshape(-1)
        out = C.c_void_p()
        _check(lib.vk_upload_i32(self.handle, _ptr(h), h.size, C.byref(out)))
        return Tensor(self, out)

    def upload_i64(self, host: np.ndarray) -> Tensor:
        h = np.ascontiguousarray(host, dtype=np.int64).reshape(-1)
        out = C.c_void_p()
        _check(lib.vk_upload_i64(self.handle, _ptr(h), h.size, C.byref(out)))
        return Tensor(self, out)

    def upload_u8(self, host: np.ndarray) -> Tensor:
        h = np.ascontiguousarray(host, dtype=np.uint8).reshape(-1)
        out = C.c_void_p()
        _check(lib.vk_upload_u8(self.handle, _ptr(h), h.size, C.byref(out)))
        return Tensor(self, out)

    def download_u8(self, t: Tensor) -> np.ndarray:
        out = np.empty(len(t), dtype=np.uint8)
        _check(lib.vk_download_u8(self.handle, t.handle, _ptr(out), out.size))
        return out

    def download_f32(self, t: Tensor) -> np.ndarray:
        out = np.empty(len(t), dtype=np.float32)
        _check(lib.vk_download_f32(self.handle, t.handle, _ptr(out), out.size))
        return out

    def copy_f32(self, t: Tensor) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_copy_f32(self.handle, t.handle, C.byref(out)))
        return Tensor(self, out)

    def copy_segment_f32(self, t: Tensor, offset: int, length: int) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_copy_segment_f32(self.handle, t.handle, offset, length, C.byref(out)))
        return Tensor(self, out)

    def copy_segment_into_f32(self, dst: Tensor, dst_offset: int, src: Tensor,
                              src_offset: int, length: int) -> None:
        _check(lib.vk_copy_segment_into_f32(self.handle, dst.handle, dst_offset, src.handle,
                                            src_offset, length))

    def overwrite_prefix_f32(self, tokens: Tensor, prefix: Tensor, length: int) -> None:
        _check(lib.vk_overwrite_prefix_f32(self.handle, tokens.handle, prefix.handle, length))

    # -- fused per-token operations -----------------------------------------
    def layernorm_f32_cpu_order(self, x: Tensor, gamma: Tensor, beta: Tensor, rows: int,
                                cols: int, eps: float) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_layernorm_f32(self.handle, x.handle, gamma.handle, beta.handle, rows,
                                    cols, eps, C.byref(out)))
        return Tensor(self, out)

    def layernorm_into_f32(self, x: Tensor, gamma: Tensor, beta: Tensor, rows: int,
                           cols: int, eps: float, out: Tensor) -> None:
        _check(lib.vk_layernorm_into_f32(self.handle, x.handle, gamma.handle, beta.handle,
                                         rows, cols, eps, out.handle))

    def split_qkv_hnd_f32(self, qkv: Tensor, rows: int, heads: int, head_dim: int):
        """CudaRuntime::split_qkv_hnd_f32: returns head-major (q, k, v)."""
        q, k, v = C.c_void_p(), C.c_void_p(), C.c_void_p()
        _check(lib.vk_split_qkv_hnd_f32(self.handle, qkv.handle, rows, heads, head_dim,
                                        C.byref(q), C.byref(k), C.byref(v)))
        return Tensor(self, q), Tensor(self, k), Tensor(self, v)

    def split_qkv_hnd_into_f32(self, qkv: Tensor, rows: int, heads: int, head_dim: int,
                               q: Tensor, k: Tensor, v: Tensor) -> None:
        _check(lib.vk_split_qkv_hnd_into_f32(self.handle, qkv.handle, rows, heads, head_dim,
                                             q.handle, k.handle, v.handle))

    def hnd_to_token_f32(self, hnd: Tensor, rows: int, heads: int, head_dim: int) -> Tensor:
        """CudaRuntime::hnd_to_token_f32: head-major -> token-major rows."""
        out = C.c_void_p()
        _check(lib.vk_hnd_to_token_f32(self.handle, hnd.handle, rows, heads, head_dim,
                                       C.byref(out)))
        return Tensor(self, out)

    def hnd_to_token_into_f32(self, hnd: Tensor, rows: int, heads: int, head_dim: int,
                              out: Tensor) -> None:
        _check(lib.vk_hnd_to_token_into_f32(self.handle, hnd.handle, rows, heads, head_dim,
                                            out.handle))

    def capture_f32(self, local_x: Optional[Tensor], x: Tensor, n: int, n_special: int,
                    embed: int, view_count: int, norm_gamma: Tensor, norm_beta: Tensor,
                    eps: float, cat_token: bool, feat: Tensor, cam: Tensor) -> None:
        """Backbone::post_process_capture for view_count view-major views."""
        _check(lib.vk_capture_f32(self.handle, _h(local_x), x.handle, n, n_special, embed,
                                  view_count, norm_gamma.handle, norm_beta.handle, eps,
                                  1 if cat_token else 0, feat.handle, cam.handle))

    def token_to_chw_f32(self, tok: Tensor, n_tok: int, c: int, gamma: Optional[Tensor],
                         beta: Optional[Tensor], eps: float, out: Tensor) -> None:
        """token_major_to_chw_with_optional_layernorm: [n_tok, c] -> [c, n_tok]."""
        _check(lib.vk_token_to_chw_f32(self.handle, tok.handle, n_tok, c, _h(gamma), _h(beta),
                                       eps, out.handle))

    def alloc_u8(self, n: int) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_tensor_alloc(self.handle, 2, n, C.byref(out)))
        return Tensor(self, out)

    def resize_u8(self, src: Tensor, sh: int, sw: int, dst: Tensor, dh: int, dw: int,
                  mode: int) -> None:
        """resize_{bilinear,cubic,area}_u8 of preprocess.rs on the device."""
        need = int(lib.vk_resize_workspace_bytes(sh, sw, dh, dw, mode))
        ws = self.alloc_u8(need) if need else None
        _check(lib.vk_resize_u8(self.handle, src.handle, sh, sw, dst.handle, dh, dw, mode,
                                _h(ws)))
        # the workspace lives as long as the result (freeing a tensor waits for
        # the stream, which a graph capture in progress would not allow)
        dst._workspace = ws

    def preprocess_shape(self, h: int, w: int, image_size: int, patch: int,
                         upper_bound: bool = True):
        oh, ow = _sz(), _sz()
        _check(lib.vk_preprocess_shape(h, w, image_size, patch, 1 if upper_bound else 0,
                                       C.byref(oh), C.byref(ow)))
        return oh.value, ow.value

    def preprocess_resize_u8(self, src: Tensor, h: int, w: int, image_size: int, patch: int,
                             upper_bound: bool = True) -> Tensor:
        """preprocess's resize + patch snap: a new u8 [out_h, out_w, 3] tensor."""
        oh, ow = self.preprocess_shape(h, w, image_size, patch, upper_bound)
        out = self.alloc_u8(oh * ow * 3)
        need = int(lib.vk_preprocess_workspace_bytes(h, w, image_size, patch,
                                                     1 if upper_bound else 0))
        ws = self.alloc_u8(need) if need else None
        _check(lib.vk_preprocess_resize_u8(self.handle, src.handle, h, w, image_size, patch,
                                           1 if upper_bound else 0, _h(ws), out.handle))
        out._workspace = ws
        return out

    def normalize_u8_hwc_nchw_f32(self, src: Tensor, h: int, w: int, mean: Sequence[float],
                                  std: Sequence[float], out: Tensor) -> None:
        m = (C.c_float * 3)(*mean)
        s = (C.c_float * 3)(*std)
        _check(lib.vk_normalize_u8_hwc_nchw_f32(self.handle, src.handle, h, w, m, s, out.handle))

    def attention_online_f32(self, q: Tensor, k: Tensor, v: Tensor, heads: int, rows: int,
                             head_dim: int) -> Tensor:
        """CudaRuntime::attention_online_f32: softmax(Q K^T / sqrt(d)) V per head."""
        out = C.c_void_p()
        _check(lib.vk_attention_online_f32(self.handle, q.handle, k.handle, v.handle, heads,
                                           rows, head_dim, C.byref(out)))
        return Tensor(self, out)

    def attention_into_f32(self, q: Tensor, k: Tensor, v: Tensor, heads: int, rows: int,
                           head_dim: int, out: Tensor) -> None:
        _check(lib.vk_attention_into_f32(self.handle, q.handle, k.handle, v.handle, heads,
                                         rows, head_dim, out.handle))

    def gelu_f32_in_place(self, x: Tensor) -> None:
        _check(lib.vk_gelu_f32_inplace(self.handle, x.handle))

    def gelu_erf_f32_in_place(self, x: Tensor) -> None:
        _check(lib.vk_gelu_erf_f32_inplace(self.handle, x.handle))

    def add_f32_in_place(self, dst: Tensor, src: Tensor) -> None:
        _check(lib.vk_add_f32_inplace(self.handle, dst.handle, src.handle))

    def layerscale_f32_in_place(self, x: Tensor, gamma: Tensor, rows: int, cols: int) -> None:
        _check(lib.vk_layerscale_f32_inplace(self.handle, x.handle, gamma.handle, rows, cols))

    def layerscale_residual_f32(self, x: Tensor, y: Tensor, gamma: Optional[Tensor],
                                rows: int, cols: int) -> None:
        _check(lib.vk_layerscale_residual_f32(self.handle, x.handle, y.handle, _h(gamma),
                                              rows, cols))

    def layerscale_residual_layernorm_f32(self, x: Tensor, y: Tensor,
                                          ls_gamma: Optional[Tensor], ln_gamma: Tensor,
                                          ln_beta: Tensor, rows: int, cols: int, eps: float,
                                          ln_out: Tensor) -> None:
        _check(lib.vk_layerscale_residual_layernorm_f32(
            self.handle, x.handle, y.handle, _h(ls_gamma), ln_gamma.handle, ln_beta.handle,
            rows, cols, eps, ln_out.handle))

    def qk_norm_rope_f32_da3_base(self, q: Tensor, k: Tensor, q_gamma: Optional[Tensor],
                                  q_beta: Optional[Tensor], k_gamma: Optional[Tensor],
                                  k_beta: Optional[Tensor], positions: Tensor, heads: int,
                                  rows: int, freq: float = 100.0,
                                  eps: float = QK_NORM_EPS) -> None:
        _check(lib.vk_qk_norm_rope_f32(self.handle, q.handle, k.handle, _h(q_gamma),
                                       _h(q_beta), _h(k_gamma), _h(k_beta), positions.handle,
                                       heads, rows, freq, eps))

    def qk_norm_rope_mode_f32(self, q: Tensor, k: Tensor, q_gamma: Optional[Tensor],
                              q_beta: Optional[Tensor], k_gamma: Optional[Tensor],
                              k_beta: Optional[Tensor], positions: Tensor, heads: int,
                              rows: int, freq: float = 100.0, eps: float = QK_NORM_EPS,
                              rope_mode: int = VK_ROPE_DEFAULT) -> None:
        """qk_norm_rope_f32_da3_base with positions of dtype f32, i32 or i64
        and an explicit RoPE convention."""
        _check(lib.vk_qk_norm_rope_mode_f32(self.handle, q.handle, k.handle, _h(q_gamma),
                                            _h(q_beta), _h(k_gamma), _h(k_beta),
                                            positions.handle, heads, rows, freq, eps,
                                            rope_mode))

    def rope2d_f32(self, x: Tensor, positions: Tensor, heads: int, rows: int,
                   head_dim: int = 64, freq: float = 100.0,
                   rope_mode: int = VK_ROPE_DEFAULT) -> None:
        """vestra_kernels::rope2d in place on one head-major tensor."""
        _check(lib.vk_rope2d_f32(self.handle, x.handle, positions.handle, heads, rows,
                                 head_dim, freq, rope_mode))

    def qk_norm_rope_grid_f32(self, q: Tensor, k: Tensor, q_gamma: Optional[Tensor],
                              q_beta: Optional[Tensor], k_gamma: Optional[Tensor],
                              k_beta: Optional[Tensor], heads: int, head_dim: int,
                              n_special: int, gh: int, gw: int, view_count: int,
                              global_layer: bool, layout: int, freq: float = 100.0,
                              eps: float = QK_NORM_EPS,
                              rope_mode: Optional[int] = None) -> None:
        """Grid-position Q/K-norm + RoPE; rope_mode None calls the
        default-convention entry point."""
        args = (self.handle, q.handle, k.handle, _h(q_gamma), _h(q_beta), _h(k_gamma),
                _h(k_beta), heads, head_dim, n_special, gh, gw, view_count,
                1 if global_layer else 0, layout, freq, eps)
        if rope_mode is None:
            _check(lib.vk_qk_norm_rope_grid_f32(*args))
        else:
            _check(lib.vk_qk_norm_rope_grid_mode_f32(*args, rope_mode))

    def rope_positions_f32(self, n_special: int, gh: int, gw: int, view_count: int,
                           global_layer: bool) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_rope_positions_f32(self.handle, n_special, gh, gw, view_count,
                                         1 if global_layer else 0, C.byref(out)))
        return Tensor(self, out)

    # -- patch embedding -----------------------------------------------------
    def patchify_nchw_f32(self, img: Tensor, h: int, w: int, patch: int,
                          channels: int) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_patchify_nchw_f32(self.handle, img.handle, h, w, patch, channels,
                                        C.byref(out)))
        return Tensor(self, out)

    def prepare_linear_f32(self, in_features: int, out_features: int, weight: np.ndarray,
                           bias: np.ndarray, ls_gamma: Optional[np.ndarray] = None) -> Linear:
        w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
        b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
        g = None if ls_gamma is None else np.ascontiguousarray(ls_gamma, dtype=np.float32)
        out = C.c_void_p()
        _check(lib.vk_linear_prepare_f32(self.handle, in_features, out_features, _ptr(w),
                                         _ptr(b), None if g is None else _ptr(g),
                                         C.byref(out)))
        return Linear(self, out)

    def prepare_linear_oihw_f32(self, in_features: int, out_features: int,
                                weight_oihw: np.ndarray, bias: np.ndarray) -> Linear:
        w = np.ascontiguousarray(weight_oihw, dtype=np.float32).reshape(-1)
        b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
        out = C.c_void_p()
        _check(lib.vk_linear_prepare_oihw_f32(self.handle, in_features, out_features, _ptr(w),
                                              _ptr(b), C.byref(out)))
        return Linear(self, out)

    def prepare_linear_w16(self, in_features: int, out_features: int, weight_f16: np.ndarray,
                           bias: np.ndarray, ls_gamma: Optional[np.ndarray] = None) -> Linear:
        """prepare_linear_f32 from a GGUF F16 [in, out] weight, widened on the device."""
        w = np.ascontiguousarray(weight_f16, dtype=np.float16).reshape(-1).view(np.uint16)
        b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
        g = None if ls_gamma is None else np.ascontiguousarray(ls_gamma, dtype=np.float32)
        out = C.c_void_p()
        _check(lib.vk_linear_prepare_w16(self.handle, in_features, out_features, _ptr(w), _ptr(b),
                                         None if g is None else _ptr(g), C.byref(out)))
        return Linear(self, out)

    def prepare_linear_q8_0(self, in_features: int, out_features: int, blocks: np.ndarray,
                            bias: np.ndarray, ls_gamma: Optional[np.ndarray] = None) -> Linear:
        """prepare_linear_f32 from GGUF Q8_0 blocks of an [in, out] weight."""
        raw = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
        b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
        g = None if ls_gamma is None else np.ascontiguousarray(ls_gamma, dtype=np.float32)
        out = C.c_void_p()
        _check(lib.vk_linear_prepare_q8_0(self.handle, in_features, out_features, _ptr(raw),
                                          raw.size, _ptr(b), None if g is None else _ptr(g),
                                          C.byref(out)))
        return Linear(self, out)

    def prepare_linear_oihw_w16(self, in_features: int, out_features: int,
                                weight_oihw_f16: np.ndarray, bias: np.ndarray) -> Linear:
        w = np.ascontiguousarray(weight_oihw_f16, dtype=np.float16).reshape(-1).view(np.uint16)
        b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
        out = C.c_void_p()
        _check(lib.vk_linear_prepare_oihw_w16(self.handle, in_features, out_features, _ptr(w),
                                              _ptr(b), C.byref(out)))
        return Linear(self, out)

    def widen_f16_f32(self, src: Tensor, dst: Tensor) -> None:
        _check(lib.vk_widen_f16_f32(self.handle, src.handle, dst.handle))

    def dequantize_q8_0_f32(self, blocks: Tensor, n: int, dst: Tensor) -> None:
        _check(lib.vk_dequantize_q8_0_f32(self.handle, blocks.handle, n, dst.handle))

    def prepend_cls_add_pos_f32(self, patches: Tensor, cls: Tensor, pos: Tensor,
                                n_patches: int, embed: int) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_prepend_cls_add_pos_f32(self.handle, patches.handle, cls.handle,
                                              pos.handle, n_patches, embed, C.byref(out)))
        return Tensor(self, out)

    def pos_embed_bicubic_f32(self, pos_embed: Tensor, grid: int, embed: int, gh: int,
                              gw: int, interp_offset: float = 0.1) -> Tensor:
        out = C.c_void_p()
        _check(lib.vk_pos_embed_bicubic_f32(self.handle, pos_embed.handle, grid, embed, gh, gw,
                                            interp_offset, C.byref(out)))
        return Tensor(self, out)

    def patch_embed_u8(self, img_hwc: Tensor, h: int, w: int, patch: int,
                       mean: Sequence[float], std: Sequence[float], proj: Linear, cls: Tensor,
                       registers: Optional[Tensor], n_register: int, pos_table: Tensor,
                       out: Tensor) -> None:
        m = (C.c_float * 3)(*mean)
        s = (C.c_float * 3)(*std)
        _check(lib.vk_patch_embed_u8(self.handle, img_hwc.handle, h, w, patch,
                                     C.cast(m, C.c_void_p), C.cast(s, C.c_void_p),
                                     proj.handle, cls.handle, _h(registers), n_register,
                                     pos_table.handle, out.handle))

    def patch_embed_views_u8(self, images: Tensor, views: int, h: int, w: int, patch: int,
                             mean: Sequence[float], std: Sequence[float], proj: Linear,
                             cls: Tensor, registers: Optional[Tensor], n_register: int,
                             pos_table: Tensor, out: Tensor) -> None:
        """patch_embed_u8 of `views` images [views, h, w, 3] in one launch,
        into the view-major token buffer."""
        m = (C.c_float * 3)(*mean)
        s = (C.c_float * 3)(*std)
        _check(lib.vk_patch_embed_views_u8(self.handle, images.handle, views, h, w, patch,
                                           C.cast(m, C.c_void_p), C.cast(s, C.c_void_p),
                                           proj.handle, cls.handle, _h(registers), n_register,
                                           pos_table.handle, out.handle))

    # -- block sequence ------------------------------------------------------
    def vit_block_fused_ops(self, cfg: VitConfig, layer_idx: int, layer: VitLayer,
                            next_layer: Optional[VitLayer], act: VitActivations, gh: int,
                            gw: int, view_count: int, camera: Optional[Tensor],
                            flags: int = 0) -> None:
        _check(lib.vk_vit_block_fused_ops(
            self.handle, C.byref(cfg), layer_idx, C.byref(layer),
            None if next_layer is None else C.byref(next_layer), C.byref(act), gh, gw,
            view_count, _h(camera), flags))

    # -- timing / graphs -----------------------------------------------------
    def event(self) -> Event:
        return Event(self)

    def begin_capture(self) -> None:
        _check(lib.vk_graph_begin_capture(self.handle))

    def vit_block_forward_f32(self, cfg: VitConfig, layer_idx: int, weights: VitBlockWeights,
                              tokens: Tensor, gh: int, gw: int, view_count: int,
                              camera: Optional[Tensor], ws: VitBlockWorkspace) -> None:
        """run_tail_device: one whole block on the device, in place on tokens."""
        _check(lib.vk_vit_block_forward_f32(self.handle, C.byref(cfg), layer_idx,
                                            C.byref(weights), tokens.handle, gh, gw, view_count,
                                            _h(camera), C.byref(ws)))

    def backbone_forward_f32(self, cfg: VitConfig, blocks: Sequence[VitBlockWeights],
                             tokens: Tensor, gh: int, gw: int, view_count: int,
                             camera: Optional[Tensor], norm_gamma: Optional[Tensor],
                             norm_beta: Optional[Tensor], cat_token: bool,
                             out_layers: Sequence[int],
                             feats: Sequence[Tensor], cams: Sequence[Tensor],
                             ws: "BlockWorkspace", local_x: Optional[Tensor]) -> None:
        """Backbone::forward_multi_view_ordered: all blocks + captures on the device
        (norm_gamma / norm_beta are read by the captures only)."""
        arr = (VitBlockWeights * len(blocks))(*blocks)
        n = len(out_layers)
        layers = (C.c_int * max(n, 1))(*out_layers)
        fa = (_vp * max(n, 1))(*[f.handle.value for f in feats])
        ca = (_vp * max(n, 1))(*[c.handle.value for c in cams])
        _check(lib.vk_backbone_forward_f32(self.handle, C.byref(cfg), len(blocks), arr,
                                           tokens.handle, gh, gw, view_count, _h(camera),
                                           _h(norm_gamma), _h(norm_beta),
                                           1 if cat_token else 0, layers, n, fa, ca,
                                           C.byref(ws.struct), _h(local_x)))

    def block_workspace(self, rows: int, embed: int, mlp: int) -> "BlockWorkspace":
        return BlockWorkspace(self, rows, embed, mlp)

    def end_capture(self) -> Graph:
        out = C.c_void_p()
        _check(lib.vk_graph_end_capture(self.handle, C.byref(out)))
        return Graph(self, out)


def block_weights_struct(**handles) -> VitBlockWeights:
    """Builds a VitBlockWeights from named tensors and linears (missing: NULL)."""
    w = VitBlockWeights()
    for name, _ in VitBlockWeights._fields_:
        h = handles.get(name)
        setattr(w, name, None if h is None else h.handle.value)
    return w


class BlockWorkspace:
    """Owns the device scratch of vk_vit_block_forward_f32 for `rows` tokens."""

    def __init__(self, rt: "Runtime", rows: int, embed: int, mlp: int):
        self.tensors = {n: rt.alloc_f32(rows * embed) for n in ("ln", "q", "k", "v", "attn")}
        self.tensors["hidden"] = rt.alloc_f32(rows * mlp)
        self.struct = VitBlockWorkspace()
        for name, t in self.tensors.items():
            setattr(self.struct, name, t.handle.value)


def layer_struct(**tensors: Optional[Tensor]) -> VitLayer:
    """Builds a VitLayer from named tensors (missing names are NULL)."""
    lay = VitLayer()
    for name, _ in VitLayer._fields_:
        t = tensors.get(name)
        setattr(lay, name, None if t is None else t.handle.value)
    return lay


def activations_struct(**tensors: Tensor) -> VitActivations:
    act = VitActivations()
    for name, _ in VitActivations._fields_:
        t = tensors.get(name)
        setattr(act, name, None if t is None else t.handle.value)
    return act
