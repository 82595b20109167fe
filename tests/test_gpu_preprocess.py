"""GPU parity of the image preprocessing (crates/da-engine/src/preprocess.rs:236-482):
the three u8 resamplers, the aspect-preserving resize with the patch snap,
and the normalisation to NCHW f32.  All bit-exact against the oracle (u8
results after half-to-even rounding; the normalisation's f32 values)."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")

MODES = {"bilinear": 0, "cubic": 1, "area": 2}


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("shape", [(23, 31, 40, 57), (40, 57, 23, 31), (427, 640, 336, 504),
                                   (1080, 1920, 283, 504), (7, 5, 7, 13), (1, 1, 3, 2),
                                   (336, 504, 336, 504), (30, 20, 15, 40)])
def test_resize_bit_exact(rt, rng, mode, shape):
    sh, sw, dh, dw = shape
    img = rng.integers(0, 256, (sh, sw, 3), dtype=np.uint8)
    dst = rt.alloc_u8(dh * dw * 3)
    rt.resize_u8(rt.upload_u8(img), sh, sw, dst, dh, dw, MODES[mode])
    got = rt_download_u8(rt, dst, (dh, dw, 3))
    assert np.array_equal(got, oracle.resize_u8(img, dh, dw, mode))


def rt_download_u8(rt, t, shape):
    return rt.download_u8(t).reshape(shape)


@pytest.mark.parametrize("h,w,size,patch,upper", [
    (427, 640, 504, 14, True), (240, 320, 504, 14, True), (1080, 1920, 504, 14, True),
    (500, 700, 504, 14, True), (427, 640, 504, 14, False), (2, 2, 2, 2, True),
    (2, 2, 4, 2, True), (3, 3, 4, 2, True), (1008, 672, 1008, 14, True)])
def test_preprocess_resize_bit_exact(rt, rng, h, w, size, patch, upper):
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    want = oracle.preprocess_resize_u8(img, size, patch, upper)
    assert rt.preprocess_shape(h, w, size, patch, upper) == want.shape[:2]
    out = rt.preprocess_resize_u8(rt.upload_u8(img), h, w, size, patch, upper)
    got = rt_download_u8(rt, out, want.shape)
    assert np.array_equal(got, want)


def test_normalize_bit_exact(rt, rng):
    h, w = 336, 504
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    mean, std = [0.485, 0.456, 0.406], [0.229, 0.224, 0.225]
    out = rt.alloc_f32(3 * h * w)
    rt.normalize_u8_hwc_nchw_f32(rt.upload_u8(img), h, w, mean, std, out)
    want = oracle.normalize_u8_hwc(img, mean, std)
    assert np.array_equal(out.numpy().view(np.uint32), want.reshape(-1).view(np.uint32))


def test_preprocess_errors(rt):
    x = rt.alloc_u8(12)
    with pytest.raises(vh.VestraError):
        rt.resize_u8(x, 2, 2, rt.alloc_u8(12), 2, 2, 7)                 # mode
    with pytest.raises(vh.VestraError):
        rt.resize_u8(x, 2, 3, rt.alloc_u8(12), 2, 2, 0)                 # src size
    with pytest.raises(vh.UnsupportedShape):
        rt.preprocess_shape(0, 5, 504, 14)
