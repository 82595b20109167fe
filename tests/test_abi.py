"""CPU checks of the C ABI boundary: the built library exports every entry
point include/vestra_hip.h declares, the Python mirror binds all of them, and
the product package never reaches the oracle (no compute calls are made
here: there is no GPU in this environment)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vestra_hip.h")
LIB = os.path.join(ROOT, "vestra-engine_amd", "libvestra_hip.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_runtime_surface():
    names = declared_functions()
    for required in ("vk_runtime_create", "vk_upload_f32", "vk_download_f32", "vk_copy_f32",
                     "vk_copy_segment_f32", "vk_copy_segment_into_f32",
                     "vk_overwrite_prefix_f32", "vk_layernorm_f32", "vk_gelu_f32_inplace",
                     "vk_add_f32_inplace", "vk_layerscale_residual_f32",
                     "vk_qk_norm_rope_f32", "vk_patchify_nchw_f32", "vk_linear_prepare_f32",
                     "vk_linear_run_f32", "vk_prepend_cls_add_pos_f32",
                     "vk_pos_embed_bicubic_f32", "vk_patch_embed_u8",
                     "vk_vit_block_fused_ops", "vk_qk_norm_rope_mode_f32", "vk_rope2d_f32",
                     "vk_upload_i32", "vk_upload_i64"):
        assert required in names, required


@pytest.mark.skipif(not os.path.exists(LIB), reason="libvestra_hip.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="libvestra_hip.so not built")
def test_python_mirror_binds_every_declared_symbol():
    import vestra_hip
    missing = [n for n in declared_functions() if n not in vestra_hip._SIGS]
    assert not missing, missing
    assert vestra_hip.lib.vk_abi_version() == 2


@pytest.mark.skipif(not os.path.exists(LIB), reason="libvestra_hip.so not built")
def test_error_message_starts_empty_and_is_thread_local():
    import threading
    import vestra_hip
    seen = []
    t = threading.Thread(target=lambda: seen.append(vestra_hip.lib.vk_last_error()))
    t.start()
    t.join()
    assert seen == [b""]


@pytest.mark.skipif(not os.path.exists(LIB), reason="libvestra_hip.so not built")
def test_null_handles_are_rejected_without_a_device():
    # argument validation happens before any device call
    import vestra_hip
    assert vestra_hip.lib.vk_tensor_len(None) == 0
    assert vestra_hip.lib.vk_tensor_dtype(None) == -1
    assert vestra_hip.lib.vk_tensor_destroy(None) == 0
    assert vestra_hip.lib.vk_linear_destroy(None) == 0
    assert vestra_hip.lib.vk_runtime_create(0, None) == vestra_hip.VK_ERR_INVALID
    assert b"null" in vestra_hip.lib.vk_last_error()


def test_product_package_never_reaches_the_oracle():
    pkg = os.path.join(ROOT, "vestra-engine_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp", ".c")) or f == "Makefile":
                text = open(os.path.join(dirpath, f), errors="replace").read()
                assert "oracle" not in text.lower(), os.path.join(dirpath, f)
