"""GPU parity of the GGUF weight formats expanded on the device (Gguf::tensor_f32,
crates/da-gguf/src/reader.rs:279-349; q8_0.rs:24-51).

F16 widening and Q8_0 dequantisation are exact, so every check is bit-exact:
the flat conversions against the oracle's numpy restatement, and projections
prepared from the stored bytes against the f32 preparation of the oracle's
widened weights (same resident values -> same GEMM bits).
"""
import numpy as np
import pytest

import oracle
from test_gpu_patch_block import normals

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


def _same_bits(a, b):
    a, b = np.asarray(a, np.float32).reshape(-1), np.asarray(b, np.float32).reshape(-1)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(a[~nan].view(np.uint32),
                                                               b[~nan].view(np.uint32))


def test_widen_f16_all_bit_patterns(rt):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    src = rt.upload_f16(bits.view(np.float16))  # the bit patterns, not their values
    dst = rt.alloc_f32(bits.size)
    rt.widen_f16_f32(src, dst)
    assert _same_bits(dst.numpy(), oracle.f16_to_f32(bits))


@pytest.mark.parametrize("n", [32, 32 * 1000, 768 * 3072])
def test_dequantize_q8_0(rt, rng, n):
    raw = oracle.quantize_q8_0(normals(rng, n, scale=0.02))
    raw[2::34 * 7] = 0x80  # int8 -128 somewhere
    dst = rt.alloc_f32(n)
    rt.dequantize_q8_0_f32(rt.upload_u8(raw), n, dst)
    assert _same_bits(dst.numpy(), oracle.dequantize_q8_0(raw, n))


@pytest.mark.parametrize("rows,k,n,with_ls", [(866, 768, 2304, False), (97, 3072, 768, True),
                                               (40, 1024, 4096, False)])
def test_linear_from_f16_and_q8_0(rt, rng, rows, k, n, with_ls):
    x = rt.upload_f32(normals(rng, rows, k))
    b = normals(rng, n, scale=0.02)
    ls = rng.uniform(0, 0.1, n).astype(np.float32) if with_ls else None
    w32 = normals(rng, k, n, scale=0.02)
    w16 = w32.astype(np.float16)
    raw = oracle.quantize_q8_0(w32)
    cases = [(rt.prepare_linear_w16(k, n, w16, b, ls), w16.astype(np.float32)),
             (rt.prepare_linear_q8_0(k, n, raw, b, ls),
              oracle.dequantize_q8_0(raw, k * n).reshape(k, n))]
    for lin, widened in cases:
        ref = rt.prepare_linear_f32(k, n, widened, b, ls)
        got, want = rt.alloc_f32(rows * n), rt.alloc_f32(rows * n)
        lin.run_into(x, rows, got)
        ref.run_into(x, rows, want)
        assert np.array_equal(got.numpy(), want.numpy())


def test_patch_filter_from_f16(rt, rng):
    """ViT-L's F16 patch filter (1024 x 3x14x14): the fused patch embedding
    with the device-widened filter gives the bits of the f32 filter path."""
    h, w, embed = 28, 42, 1024
    img = rt.upload_u8(rng.integers(0, 256, (h, w, 3), dtype=np.uint8))
    wt16 = normals(rng, embed, 3, 14, 14, scale=0.02).astype(np.float16)
    b = normals(rng, embed, scale=0.02)
    cls, pos = rt.upload_f32(normals(rng, embed)), rt.upload_f32(normals(rng, 7, embed))
    mean, std = [0.485, 0.456, 0.406], [0.229, 0.224, 0.225]
    outs = []
    for proj in (rt.prepare_linear_oihw_w16(588, embed, wt16, b),
                 rt.prepare_linear_oihw_f32(588, embed, wt16.astype(np.float32), b)):
        out = rt.alloc_f32(7 * embed)
        rt.patch_embed_u8(img, h, w, 14, mean, std, proj, cls, None, 0, pos, out)
        outs.append(out.numpy())
    assert np.array_equal(outs[0], outs[1])


def test_weight_format_errors(rt, rng):
    b = np.zeros(64, np.float32)
    with pytest.raises(vh.VestraError):
        rt.prepare_linear_q8_0(3, 20, np.zeros(34 * 2, np.uint8), np.zeros(20, np.float32))
    with pytest.raises(vh.VestraError):
        rt.prepare_linear_q8_0(32, 64, np.zeros(34 * 63, np.uint8), b)   # byte count
    with pytest.raises(vh.VestraError):
        rt.dequantize_q8_0_f32(rt.upload_u8(np.zeros(34, np.uint8)), 33, rt.alloc_f32(33))
    with pytest.raises(vh.VestraError):
        rt.widen_f16_f32(rt.alloc_f32(4), rt.alloc_f32(4))               # not f16
