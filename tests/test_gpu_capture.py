"""GPU parity of the backbone capture (Backbone::post_process_capture,
backbone.rs:1139-1179) and the head's token -> CHW hand-off with LayerNorm
(token_major_to_chw_with_optional_layernorm, dpt_head.rs:260-301).

The copied parts (local_x rows, camera rows, the transpose) are bit-exact.
The LayerNorm'd parts must carry exactly the bits of vk_layernorm_into_f32 on
the same rows (the reference asserts the same identity between its fused
and materialised hand-off, dpt_head.rs:1038-1070) and match the oracle's
scalar LayerNorm within rtol 1e-5 / atol 1e-6 (tree vs sequential sums).
"""
import numpy as np
import pytest

import oracle
from conftest import F32_ATOL, F32_RTOL, assert_parity
from test_gpu_patch_block import normals

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


def _params(rng, D, f16):
    g, b = normals(rng, D, scale=0.02, shift=1), normals(rng, D, scale=0.02)
    if f16:
        g, b = g.astype(np.float16), b.astype(np.float16)
    return g, b


def _up(rt, a):
    return rt.upload_f16(a) if a.dtype == np.float16 else rt.upload_f32(a)


@pytest.mark.parametrize("D,gh,gw,views,cat,f16", [
    (768, 24, 36, 1, True, False), (768, 4, 6, 12, True, False), (1024, 3, 5, 2, True, True),
    (768, 4, 6, 2, False, False), (384, 2, 3, 3, True, False)])
def test_capture(rt, rng, D, gh, gw, views, cat, f16):
    ns, n_patch = 2, gh * gw
    n = ns + n_patch
    x, local = normals(rng, views * n, D), normals(rng, views * n, D)
    g, b = _params(rng, D, f16)
    W = 2 * D if cat else D
    feat, cam = rt.alloc_f32(views * n_patch * W), rt.alloc_f32(views * W)
    gd, bd = _up(rt, g), _up(rt, b)
    rt.capture_f32(rt.upload_f32(local) if cat else None, rt.upload_f32(x), n, ns, D, views,
                   gd, bd, 1e-6, cat, feat, cam)
    f = feat.numpy().reshape(views, n_patch, W)
    c = cam.numpy().reshape(views, W)
    rf, rc = oracle.capture(local, x, n, ns, D, views, g, b, 1e-6, cat)
    assert np.array_equal(c, rc)
    if cat:
        assert np.array_equal(f[..., :D], rf[..., :D])
    ln_part = f[..., D:] if cat else f
    assert_parity(ln_part, rf[..., D:] if cat else rf, F32_ATOL, F32_RTOL, "capture LN")
    # the same bits as the block LayerNorm on the gathered patch rows
    rows = x.reshape(views, n, D)[:, ns:].reshape(-1, D)
    ln = rt.alloc_f32(rows.size)
    rt.layernorm_into_f32(rt.upload_f32(rows), gd, bd, rows.shape[0], D, 1e-6, ln)
    assert np.array_equal(ln_part.reshape(-1), ln.numpy())


@pytest.mark.parametrize("n_tok,c,norm,f16", [
    (864, 1536, True, False), (3456, 2048, True, True), (100, 768, True, False),
    (864, 1536, False, False), (35, 16, True, False), (1, 4, True, False)])
def test_token_to_chw(rt, rng, n_tok, c, norm, f16):
    tok = normals(rng, n_tok, c)
    g, b = _params(rng, c, f16) if norm else (None, None)
    out = rt.alloc_f32(n_tok * c)
    td = rt.upload_f32(tok)
    gd = _up(rt, g) if norm else None
    bd = _up(rt, b) if norm else None
    rt.token_to_chw_f32(td, n_tok, c, gd, bd, 1e-5, out)
    got = out.numpy().reshape(c, n_tok)
    ref = oracle.token_to_chw(tok, n_tok, c, g, b, 1e-5)
    if not norm:
        assert np.array_equal(got, ref)
        return
    assert_parity(got, ref, F32_ATOL, F32_RTOL, f"token_to_chw {n_tok}x{c}")
    ln = rt.alloc_f32(n_tok * c)
    rt.layernorm_into_f32(td, gd, bd, n_tok, c, 1e-5, ln)
    assert np.array_equal(got, ln.numpy().reshape(n_tok, c).T)


def test_token_to_chw_reference_vectors(rt):
    """The reference's own hand-off vectors (dpt_head.rs:1041-1048): 35 tokens
    of a 5x7 grid, 16 channels, exact binary inputs."""
    n_tok, c = 35, 16
    tok = ((np.arange(n_tok * c) * 37 % 251).astype(np.float32) - 125.0) * 0.0078125
    g = (0.5 + np.arange(c) * 0.03125).astype(np.float32)
    b = (-0.25 + np.arange(c) * 0.015625).astype(np.float32)
    out = rt.alloc_f32(n_tok * c)
    rt.token_to_chw_f32(rt.upload_f32(tok), n_tok, c, rt.upload_f32(g), rt.upload_f32(b), 1e-5,
                        out)
    assert_parity(out.numpy(), oracle.token_to_chw(tok, n_tok, c, g, b, 1e-5), F32_ATOL, F32_RTOL,
                  "reference vectors")


def test_capture_and_chw_errors(rt, rng):
    D = 768
    g, b = rt.upload_f32(np.ones(D, np.float32)), rt.upload_f32(np.zeros(D, np.float32))
    x = rt.alloc_f32(6 * D)
    with pytest.raises(vh.VestraError):
        rt.capture_f32(None, x, 6, 2, D, 1, g, b, 1e-6, True, rt.alloc_f32(8 * D),
                       rt.alloc_f32(2 * D))                       # cat without local_x
    with pytest.raises(vh.VestraError):
        rt.capture_f32(None, x, 6, 2, D, 1, g, b, 1e-6, False, rt.alloc_f32(3 * D),
                       rt.alloc_f32(D))                           # feat size
    with pytest.raises(vh.UnsupportedShape):
        rt.token_to_chw_f32(rt.alloc_f32(10 * 6), 10, 6, None, None, 1e-5, rt.alloc_f32(60))
    t = rt.alloc_f32(8 * 16)
    with pytest.raises(vh.VestraError):
        rt.token_to_chw_f32(t, 8, 16, None, None, 1e-5, t)        # aliasing
    rt.token_to_chw_f32(rt.alloc_f32(0), 0, 16, None, None, 1e-5, rt.alloc_f32(0))


def test_chw_work_buffer_capture_rules(rng):
    """The hand-off's row statistics live in the runtime's work buffer:
    the first use inside a stream capture is refused (the buffer cannot be
    allocated there), a graph captured after an eager call replays
    correctly, and it still does after a larger call has replaced the
    buffer (the old one is kept until the runtime ends)."""
    import gc
    rt = vh.Runtime(0)  # fresh runtime: no work buffer yet
    _work_buffer_case(rt, rng)
    gc.collect()  # every tensor and graph of the case is gone
    rt.close()    # (left open when the case fails: its tensors may live on)


def _work_buffer_case(rt, rng):
    import gc
    n_tok, c = 100, 768
    tok = normals(rng, n_tok, c)
    g, b = _params(rng, c, False)
    td, gd, bd = rt.upload_f32(tok), rt.upload_f32(g), rt.upload_f32(b)
    out = rt.alloc_f32(n_tok * c)

    def step():
        rt.token_to_chw_f32(td, n_tok, c, gd, bd, 1e-5, out)

    rt.synchronize()
    gc.disable()
    try:
        rt.begin_capture()
        with pytest.raises(vh.VestraError, match="before stream capture"):
            step()
        rt.end_capture()
    finally:
        gc.enable()
    step()
    want = out.numpy()
    ln = rt.alloc_f32(n_tok * c)
    rt.layernorm_into_f32(td, gd, bd, n_tok, c, 1e-5, ln)
    assert np.array_equal(want.reshape(c, n_tok), ln.numpy().reshape(n_tok, c).T)
    rt.synchronize()
    gc.disable()
    try:
        rt.begin_capture()
        step()
        graph = rt.end_capture()
    finally:
        gc.enable()
    # 4.5 M tokens x 4 channels: 9 M floats of statistics, more than the
    # first allocation (8 Mi floats), so the buffer is replaced
    nb, cb = 4_500_000, 4
    big = normals(rng, nb, cb)
    gb, bb = _params(rng, cb, False)
    big_d, gbd, bbd = rt.upload_f32(big), rt.upload_f32(gb), rt.upload_f32(bb)
    big_out = rt.alloc_f32(nb * cb)
    rt.token_to_chw_f32(big_d, nb, cb, gbd, bbd, 1e-5, big_out)
    big_ln = rt.alloc_f32(nb * cb)
    rt.layernorm_into_f32(big_d, gbd, bbd, nb, cb, 1e-5, big_ln)
    assert np.array_equal(big_out.numpy().reshape(cb, nb), big_ln.numpy().reshape(nb, cb).T)
    for _ in range(3):
        out.write(np.zeros(n_tok * c, np.float32))
        graph.launch()
        rt.synchronize()
        assert np.array_equal(out.numpy(), want)
