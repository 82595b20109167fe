"""GPU parity of patch embedding, the runtime surface and the block sequence.

Patch projection runs on F32 MFMA with a different accumulation order than
the oracle's sequential sum, so it is compared within rtol 1e-5 / atol 1e-6
(F32 weights) or rtol 2e-3 / atol 2e-3 (F16-stored weights); everything
without a reduction (patchify, bicubic table, token assembly, copies) is
bit-exact.
"""
import numpy as np
import pytest

import oracle
from conftest import F32_ATOL, F32_RTOL, assert_parity, record_margin

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")

MEAN = [0.485, 0.456, 0.406]
STD = [0.229, 0.224, 0.225]


def normals(rng, *shape, scale=1.0, shift=0.0):
    return (shift + scale * rng.standard_normal(shape)).astype(np.float32)


def assert_dot_parity(got, ref, scale, k, label):
    """Parity for K-long f32 dot products accumulated in different orders
    (sequential in the oracle, MFMA on the GPU): rtol 1e-5 / atol 1e-6 plus
    the probabilistic rounding bound of either sum, sqrt(K) * 2^-24 *
    sum_k |a_k w_k| per output, counted twice (both sides round)."""
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    scale = np.asarray(scale, np.float64).reshape(-1)
    bound = F32_ATOL + F32_RTOL * np.abs(ref) + 2.0 * np.sqrt(k) * 2.0 ** -24 * scale
    err = np.abs(got - ref)
    record_margin("f32 dot products (projections, patch embedding)", got, ref, tol=bound,
                  label=label)
    worst = int(np.argmax(err / bound))
    assert np.all(err <= bound), (f"[{label}] worst@{worst} got={got[worst]!r} "
                                  f"ref={ref[worst]!r} err={err[worst]:.3e} "
                                  f"bound={bound[worst]:.3e}")


# ---------------------------------------------------------------- runtime
def test_runtime_copies(rt, rng):
    x = normals(rng, 3 * 768)
    t = rt.upload_f32(x)
    assert np.array_equal(rt.copy_f32(t).numpy(), x)
    seg = rt.copy_segment_f32(t, 768, 768)
    assert np.array_equal(seg.numpy(), x[768:1536])
    dst = rt.upload_f32(np.zeros(4 * 768, np.float32))
    rt.copy_segment_into_f32(dst, 768, t, 0, 3 * 768)
    expect = np.zeros(4 * 768, np.float32)
    expect[768:] = x
    assert np.array_equal(dst.numpy(), expect)
    cam = normals(rng, 768)
    rt.overwrite_prefix_f32(t, rt.upload_f32(cam), 768)
    assert np.array_equal(t.numpy()[:768], cam) and np.array_equal(t.numpy()[768:], x[768:])
    with pytest.raises(vh.VestraError) as e:
        rt.copy_segment_f32(t, 3 * 768, 1)
    assert "outside" in e.value.message


# 16-byte copies run in chunks of 192 float4 per wave, two chunks per wave
# between 24 and 48 waves per CU, and the last workgroup copies what is left
# after the whole chunks; other alignments take the element loop.
@pytest.mark.parametrize("float4s", ["short", "one_chunk_plus", "two_per_wave", "one_per_wave"])
def test_device_copy_sizes(rt, rng, float4s):
    cu = rt.cu_count()
    n16 = {"short": 100, "one_chunk_plus": 192 * 5 + 40,
           "two_per_wave": 192 * (24 * cu + 7) + 37,
           "one_per_wave": 192 * (48 * cu + 3) + 191}[float4s]
    x = normals(rng, 4 * n16)
    t = rt.upload_f32(x)
    assert np.array_equal(rt.copy_f32(t).numpy(), x)
    dst = rt.upload_f32(np.full(4 * n16 + 8, -1.0, np.float32))
    rt.copy_segment_into_f32(dst, 4, t, 0, 4 * n16)          # 16-byte aligned
    expect = np.full(4 * n16 + 8, -1.0, np.float32)
    expect[4:4 + 4 * n16] = x
    assert np.array_equal(dst.numpy(), expect)
    rt.copy_segment_into_f32(dst, 1, t, 3, 4 * n16 - 5)      # 4-byte aligned
    expect[1:4 * n16 - 4] = x[3:4 * n16 - 2]
    assert np.array_equal(dst.numpy(), expect)


def test_events_and_graph_replays(rt, rng):
    rows, cols = 866, 768
    x, y = normals(rng, rows, cols), normals(rng, rows, cols)
    g = rng.uniform(0, 0.1, cols).astype(np.float32)
    tx, ty, tg = rt.upload_f32(x), rt.upload_f32(y), rt.upload_f32(g)
    rt.synchronize()
    rt.begin_capture()
    rt.layerscale_residual_f32(tx, ty, tg, rows, cols)
    graph = rt.end_capture()
    expect = x.copy()
    for _ in range(3):
        graph.launch()
        rt.synchronize()
        expect = oracle.layerscale_residual(expect, y, g)
        assert np.array_equal(tx.numpy().reshape(rows, cols), expect)
        # eager work between replays
        rt.add_f32_in_place(tx, ty)
        expect = oracle.add(expect, y)
    e0, e1 = rt.event(), rt.event()
    e0.record()
    graph.launch()
    e1.record()
    assert e0.elapsed_ms(e1) >= 0.0


def test_graph_of_copies_replays(rt, rng):
    """Segment copies and the prefix (camera-slot) write are kernels: a
    captured sequence of them replays with the eager bits, replay after
    replay, with eager work in between."""
    D, rows = 768, 30
    x = normals(rng, rows, D)
    cam = normals(rng, 2 * D)
    tokens, camera, snap = rt.upload_f32(x), rt.upload_f32(cam), rt.alloc_f32(rows * D)
    ones_h = np.ones((rows, D), np.float32)
    ones = rt.upload_f32(ones_h)
    odd = rt.alloc_f32(5)

    def step():
        rt.copy_segment_into_f32(snap, 0, tokens, 0, rows * D)
        rt.copy_segment_into_f32(odd, 0, tokens, 3, 5)  # 4-byte aligned only
        rt.overwrite_prefix_f32(tokens, camera, D)      # the camera-slot write

    expect = x.copy()
    rt.synchronize()
    rt.begin_capture()
    step()
    graph = rt.end_capture()
    for r in range(3):
        graph.launch()
        rt.synchronize()
        snap_want = expect.copy()
        expect[0] = cam[:D]
        assert np.array_equal(snap.numpy().reshape(rows, D), snap_want), f"replay {r}"
        assert np.array_equal(odd.numpy(), snap_want.reshape(-1)[3:8]), f"replay {r}"
        assert np.array_equal(tokens.numpy().reshape(rows, D), expect), f"replay {r}"
        rt.add_f32_in_place(tokens, ones)
        expect = oracle.add(expect, ones_h)


def test_graph_lifetime_rules(rng):
    """A graph launches only on the runtime it was captured on, not after
    that runtime was destroyed, and its destroy is clean afterwards."""
    a, b = vh.Runtime(0), vh.Runtime(0)
    x, y = normals(rng, 4096), normals(rng, 4096)
    t, u = a.upload_f32(x), a.upload_f32(y)
    a.synchronize()
    a.begin_capture()
    try:
        a.add_f32_in_place(t, u)
    finally:
        graph = a.end_capture()
    graph.launch()
    a.synchronize()
    assert np.array_equal(t.numpy(), x + y)
    with pytest.raises(vh.VestraError, match="another runtime"):
        vh._check(vh.lib.vk_graph_launch(b.handle, graph.handle))
    handle = a.handle
    a.close()
    with pytest.raises(vh.VestraError, match="destroyed"):
        vh._check(vh.lib.vk_graph_launch(handle, graph.handle))
    del graph, t, u  # the graph and the tensors release the runtime
    b.close()


# ---------------------------------------------------------------- patch embedding pieces
def test_patchify_bit_exact(rt, rng):
    img = normals(rng, 3, 336, 504)
    out = rt.patchify_nchw_f32(rt.upload_f32(img), 336, 504, 14, 3).numpy()
    assert np.array_equal(out.reshape(864, 588), oracle.patchify_nchw(img, 14))


def test_linear_patch_kats(rt):
    # patch_embed.rs:280-339 through the split CUDA-shaped path:
    # patchify -> linear (OIHW filter) -> tokens.  embed padded to 4 columns.
    img = np.zeros((3, 4, 4), np.float32)
    img[0] = np.arange(16, dtype=np.float32).reshape(4, 4)
    w = np.zeros((4, 3, 2, 2), np.float32)
    w[0, 0] = 1.0
    lin = rt.prepare_linear_oihw_f32(12, 4, w, np.zeros(4, np.float32))
    rows = rt.patchify_nchw_f32(rt.upload_f32(img), 4, 4, 2, 3)
    out = lin.run(rows, 4).numpy().reshape(4, 4)
    assert out[:, 0].tolist() == [10.0, 18.0, 42.0, 50.0]
    lin0 = rt.prepare_linear_oihw_f32(12, 4, np.zeros((4, 3, 2, 2), np.float32),
                                      np.array([1, 2, 3, 4], np.float32))
    out0 = lin0.run(rt.patchify_nchw_f32(rt.upload_f32(np.ones((3, 4, 4), np.float32)), 4, 4, 2,
                                         3), 4).numpy().reshape(4, 4)
    assert (out0 == np.array([1, 2, 3, 4], np.float32)).all()


@pytest.mark.parametrize("m,k,n,with_ls", [(864, 588, 768, False), (865, 768, 768, True),
                                           (5, 13, 8, False), (3456, 588, 1024, False),
                                           (865, 3072, 768, True), (2000, 768, 700, False)])
def test_linear_matches_oracle(rt, rng, m, k, n, with_ls):
    """The plan model picks tile shape and split count by shape: 64 x 64
    unsplit with a K tail (864 x 588 x 768), 64 x 64 split 3 (865 x 768 x
    768), 128 x 128 unsplit with a K tail (3456 x 588 x 1024), 128 x 128
    split 6 (865 x 3072 x 768), 64 x 64 split 2 with partial row and column
    tiles (2000 x 768 x 700); K = 13 takes the narrow kernel."""
    x = normals(rng, m, k)
    w = normals(rng, k, n, scale=0.02)
    b = normals(rng, n, scale=0.02)
    ls = rng.uniform(0, 0.1, n).astype(np.float32) if with_ls else None
    lin = rt.prepare_linear_f32(k, n, w, b, ls)
    assert lin.input_features() == k
    out = lin.run(rt.upload_f32(x), m).numpy().reshape(m, n)
    ref = oracle.linear(x, w, b)
    if with_ls:
        ref = oracle.layerscale(ref, ls)
    scale = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64)
    if with_ls:
        scale = scale * ls
    assert_dot_parity(out, ref, scale, k, f"linear {m}x{k}x{n}")


# ---------------------------------------------------------------- fused linear epilogues
@pytest.mark.parametrize("m,k,n", [(97, 192, 136), (48, 13, 8), (865, 768, 3072), (865, 3072, 768)])
def test_linear_into_matches_run(rt, rng, m, k, n):
    x = rt.upload_f32(normals(rng, m, k))
    lin = rt.prepare_linear_f32(k, n, normals(rng, k, n, scale=0.02), normals(rng, n, scale=0.02))
    out = rt.alloc_f32(m * n)
    lin.run_into(x, m, out)
    assert np.array_equal(out.numpy(), lin.run(x, m).numpy())


@pytest.mark.parametrize("m,k,n", [(97, 192, 136), (48, 13, 8), (865, 768, 3072)])
@pytest.mark.parametrize("exact_erf", [False, True])
def test_linear_gelu_fused_is_the_unfused_sequence(rt, rng, m, k, n, exact_erf):
    # FC1 + GELU (vit_block.rs:578,642): bit-identical to linear then the GELU
    # stream on the GPU, and within the composed bound of the oracle
    xh, w, b = normals(rng, m, k), normals(rng, k, n, scale=0.05), normals(rng, n, scale=0.02)
    x = rt.upload_f32(xh)
    lin = rt.prepare_linear_f32(k, n, w, b)
    fused, plain = rt.alloc_f32(m * n), rt.alloc_f32(m * n)
    lin.run_gelu(x, m, fused, exact_erf=exact_erf)
    lin.run_into(x, m, plain)
    (rt.gelu_erf_f32_in_place if exact_erf else rt.gelu_f32_in_place)(plain)
    got = fused.numpy()
    assert np.array_equal(got, plain.numpy())
    if m * k * n <= 4_000_000:
        pre = oracle.linear(xh, w, b)
        ref = (oracle.gelu_erff if exact_erf else oracle.gelu)(pre)
        scale = np.abs(xh).astype(np.float64) @ np.abs(w).astype(np.float64)
        # |GELU'| <= 1.13: the dot-product bound carries through, then GELU's own
        bound = (1.13 * (F32_ATOL + F32_RTOL * np.abs(pre) + 2 * np.sqrt(k) * 2.0 ** -24 * scale)
                 + F32_ATOL + F32_RTOL * np.abs(ref))
        err = np.abs(got.reshape(m, n).astype(np.float64) - ref)
        assert np.all(err <= bound), float(np.max(err / bound))


@pytest.mark.parametrize("m,k,n,with_ls", [(97, 192, 136, True), (48, 13, 8, False),
                                           (865, 768, 768, True), (865, 3072, 768, True)])
def test_linear_residual_fused_is_the_unfused_sequence(rt, rng, m, k, n, with_ls):
    # proj/FC2 + LayerScale + residual (vit_block.rs:214-222,563-564,580)
    xh, w, b = normals(rng, m, k), normals(rng, k, n, scale=0.02), normals(rng, n, scale=0.02)
    ls = rng.uniform(0, 0.1, n).astype(np.float32) if with_ls else None
    res = normals(rng, m, n)
    x = rt.upload_f32(xh)
    lin = rt.prepare_linear_f32(k, n, w, b, ls)
    fused = rt.upload_f32(res)
    lin.run_residual(x, m, fused)
    plain, y = rt.upload_f32(res), rt.alloc_f32(m * n)
    lin.run_into(x, m, y)
    rt.add_f32_in_place(plain, y)
    got = fused.numpy()
    assert np.array_equal(got, plain.numpy())
    if m * k * n <= 4_000_000:
        t = oracle.linear(xh, w, b)
        if with_ls:
            t = oracle.layerscale(t, ls)
        ref = oracle.add(res, t)
        scale = np.abs(xh).astype(np.float64) @ np.abs(w).astype(np.float64)
        if with_ls:
            scale = scale * ls
        assert_dot_parity(got, ref, scale, k, f"linear+residual {m}x{k}x{n}")


def test_linear_fused_entry_points_reject_bad_arguments(rt, rng):
    x = rt.upload_f32(normals(rng, 4, 8))
    with_ls = rt.prepare_linear_f32(8, 4, normals(rng, 8, 4), normals(rng, 4),
                                    rng.uniform(0, 0.1, 4).astype(np.float32))
    with pytest.raises(vh.VestraError):
        with_ls.run_gelu(x, 4, rt.alloc_f32(16))      # GELU after a LayerScale: not a reference op
    plain = rt.prepare_linear_f32(8, 8, normals(rng, 8, 8), normals(rng, 8))
    with pytest.raises(vh.VestraError):
        plain.run_residual(x, 4, x)                   # residual overlapping the input
    with pytest.raises(vh.VestraError):
        plain.run_into(x, 4, rt.alloc_f32(31))        # wrong output size
    empty = rt.alloc_f32(0)
    plain.run_into(rt.alloc_f32(0), 0, empty)         # zero rows: nothing launched


def test_pos_embed_bicubic_bit_exact(rt, rng):
    M, E = 37, 768
    pe = normals(rng, M * M + 1, E, scale=0.02)
    out = rt.pos_embed_bicubic_f32(rt.upload_f32(pe), M, E, 24, 36, 0.1).numpy()
    assert np.array_equal(out.reshape(-1, E), oracle.pos_embed_bicubic(pe, M, E, 24, 36, 0.1))


def test_prepend_cls_add_pos_bit_exact(rt, rng):
    np_, E = 864, 768
    patches, cls, pos = normals(rng, np_, E), normals(rng, E), normals(rng, np_ + 1, E)
    out = rt.prepend_cls_add_pos_f32(rt.upload_f32(patches), rt.upload_f32(cls),
                                     rt.upload_f32(pos), np_, E).numpy()
    assert np.array_equal(out.reshape(-1, E), oracle.assemble_tokens(patches, 24, 36, cls, None, pos))


# ---------------------------------------------------------------- fused patch embedding
@pytest.mark.parametrize("h,w,embed,n_register", [(336, 504, 768, 1), (336, 504, 768, 0),
                                                  (28, 42, 16, 0), (672, 1008, 1024, 1)])
def test_patch_embed_u8_matches_oracle(rt, rng, h, w, embed, n_register):
    gh, gw = h // 14, w // 14
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    wt = normals(rng, embed, 3, 14, 14, scale=0.02)
    b = normals(rng, embed, scale=0.02)
    cls = normals(rng, embed, scale=0.02)
    regs = normals(rng, n_register, embed, scale=0.02) if n_register else None
    pos = normals(rng, 1 + gh * gw, embed, scale=0.02)
    proj = rt.prepare_linear_oihw_f32(588, embed, wt, b)
    out = rt.alloc_f32((1 + n_register + gh * gw) * embed)
    rt.patch_embed_u8(rt.upload_u8(img), h, w, 14, MEAN, STD, proj, rt.upload_f32(cls),
                      rt.upload_f32(regs) if regs is not None else None, n_register,
                      rt.upload_f32(pos), out)
    ref = oracle.patch_embed_u8(img, 14, MEAN, STD, wt, b, cls, regs, pos)
    got = out.numpy().reshape(ref.shape)
    # special rows involve no reduction: bit-exact
    assert np.array_equal(got[:1 + n_register], ref[:1 + n_register])
    a = np.abs(oracle.patchify_nchw(oracle.normalize_u8_hwc(img, MEAN, STD), 14)).astype(np.float64)
    scale = a @ np.abs(wt.reshape(embed, -1)).astype(np.float64).T
    assert_dot_parity(got[1 + n_register:], ref[1 + n_register:], scale, 588,
                      f"patch_embed {h}x{w}")


def test_patch_embed_u8_several_rounds_partial_tiles(rt, rng):
    """700x840 (3,000 patches: the last 32-patch tile holds 24) with 200
    outputs (the last 96-column tile holds 8): 94 x 3 = 282 tiles, more
    than one round of CUs, so the gathered kernel runs with u16 table
    addresses; rows and columns past the tile edges are computed on clamped
    data and never stored."""
    h, w, embed, n_register = 700, 840, 200, 2
    gh, gw = h // 14, w // 14
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    wt = normals(rng, embed, 3, 14, 14, scale=0.02)
    b = normals(rng, embed, scale=0.02)
    cls = normals(rng, embed, scale=0.02)
    regs = normals(rng, n_register, embed, scale=0.02)
    pos = normals(rng, 1 + gh * gw, embed, scale=0.02)
    proj = rt.prepare_linear_oihw_f32(588, embed, wt, b)
    out = rt.upload_f32(np.full((1 + n_register + gh * gw) * embed, np.nan, np.float32))
    rt.patch_embed_u8(rt.upload_u8(img), h, w, 14, MEAN, STD, proj, rt.upload_f32(cls),
                      rt.upload_f32(regs), n_register, rt.upload_f32(pos), out)
    ref = oracle.patch_embed_u8(img, 14, MEAN, STD, wt, b, cls, regs, pos)
    got = out.numpy().reshape(ref.shape)
    assert np.array_equal(got[:1 + n_register], ref[:1 + n_register])
    a = np.abs(oracle.patchify_nchw(oracle.normalize_u8_hwc(img, MEAN, STD), 14)).astype(np.float64)
    scale = a @ np.abs(wt.reshape(embed, -1)).astype(np.float64).T
    assert_dot_parity(got[1 + n_register:], ref[1 + n_register:], scale, 588,
                      "patch_embed 700x840, 200 outputs")


@pytest.mark.parametrize("h,w,embed", [(336, 504, 768), (672, 1008, 1024)])
def test_patch_embed_graph_replays(rt, rng, h, w, embed):
    """The fused patch embedding captured in a HIP graph (one round of tiles:
    u32 table addresses; several: u16) replays with the eager bits, replay
    after replay, with eager work on the same stream in between."""
    gh, gw = h // 14, w // 14
    rows = 1 + 1 + gh * gw
    img = rt.upload_u8(rng.integers(0, 256, (h, w, 3), dtype=np.uint8))
    proj = rt.prepare_linear_oihw_f32(588, embed, normals(rng, embed, 3, 14, 14, scale=0.02),
                                      normals(rng, embed, scale=0.02))
    cls = rt.upload_f32(normals(rng, embed, scale=0.02))
    regs = rt.upload_f32(normals(rng, embed, scale=0.02))
    pos = rt.upload_f32(normals(rng, 1 + gh * gw, embed, scale=0.02))
    eager = rt.alloc_f32(rows * embed)
    rt.patch_embed_u8(img, h, w, 14, MEAN, STD, proj, cls, regs, 1, pos, eager)
    want = eager.numpy()
    out = rt.alloc_f32(rows * embed)
    rt.synchronize()
    rt.begin_capture()
    try:
        rt.patch_embed_u8(img, h, w, 14, MEAN, STD, proj, cls, regs, 1, pos, out)
    finally:
        graph = rt.end_capture()
    junk = rt.upload_f32(np.ones(rows * embed, np.float32))
    for r in range(3):
        graph.launch()
        rt.synchronize()
        assert np.array_equal(out.numpy(), want), f"replay {r}"
        rt.add_f32_in_place(out, junk)  # eager work between the replays


def test_patch_embed_f16_filter_vitl_matches_oracle(rt, rng):
    """ViT-L at 1008x672 with the patch filter stored as F16 (GGUF F16
    element layout) and widened on the device: the oracle runs on the same
    filter widened on the host, which is exact (reader.rs:303-318)."""
    h, w, embed, n_register = 672, 1008, 1024, 1
    gh, gw = h // 14, w // 14
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    wt16 = normals(rng, embed, 3, 14, 14, scale=0.02).astype(np.float16)
    wt = wt16.astype(np.float32)
    b = normals(rng, embed, scale=0.02)
    cls = normals(rng, embed, scale=0.02)
    regs = normals(rng, n_register, embed, scale=0.02)
    pos = normals(rng, 1 + gh * gw, embed, scale=0.02)
    proj = rt.prepare_linear_oihw_w16(588, embed, wt16, b)
    out = rt.alloc_f32((1 + n_register + gh * gw) * embed)
    rt.patch_embed_u8(rt.upload_u8(img), h, w, 14, MEAN, STD, proj, rt.upload_f32(cls),
                      rt.upload_f32(regs), n_register, rt.upload_f32(pos), out)
    ref = oracle.patch_embed_u8(img, 14, MEAN, STD, wt, b, cls, regs, pos)
    got = out.numpy().reshape(ref.shape)
    assert np.array_equal(got[:1 + n_register], ref[:1 + n_register])
    a = np.abs(oracle.patchify_nchw(oracle.normalize_u8_hwc(img, MEAN, STD), 14)).astype(np.float64)
    scale = a @ np.abs(wt.reshape(embed, -1)).astype(np.float64).T
    assert_dot_parity(got[1 + n_register:], ref[1 + n_register:], scale, 588,
                      "patch_embed 672x1008 f16 filter")


@pytest.mark.parametrize("h,w,embed,views,n_register", [(336, 504, 768, 12, 1),
                                                        (336, 504, 768, 2, 1),
                                                        (28, 42, 16, 5, 0),
                                                        (28, 42, 80, 300, 2),
                                                        (112, 168, 768, 2, 1),
                                                        (672, 1008, 1024, 2, 1)])
def test_patch_embed_views_match_single_views(rt, rng, h, w, embed, views, n_register):
    """All views of one processed shape in one launch (the per-view loop of
    prepare_multi_view, engine.rs:573-626): every view's tokens carry the
    bits of its own vk_patch_embed_u8 call.  Launches of more 32-patch tiles
    than CUs take the pipelined kernel (persistent workgroups of two to 16
    tiles here, partial tiles in M and N at 28x42 with 80 outputs); the
    others and every single view take the gathered kernel, with u32
    addresses for one round of tiles (two 112x168 views: 48 tiles, view by
    view) and u16 for several (one 672x1008 view: 1,188 tiles)."""
    gh, gw = h // 14, w // 14
    tpv = 1 + n_register + gh * gw
    imgs = rng.integers(0, 256, (views, h, w, 3), dtype=np.uint8)
    proj = rt.prepare_linear_oihw_f32(588, embed, normals(rng, embed, 3, 14, 14, scale=0.02),
                                      normals(rng, embed, scale=0.02))
    cls = rt.upload_f32(normals(rng, embed, scale=0.02))
    regs = rt.upload_f32(normals(rng, n_register, embed, scale=0.02)) if n_register else None
    pos = rt.upload_f32(normals(rng, 1 + gh * gw, embed, scale=0.02))
    out = rt.alloc_f32(views * tpv * embed)
    rt.patch_embed_views_u8(rt.upload_u8(imgs), views, h, w, 14, MEAN, STD, proj, cls, regs,
                            n_register, pos, out)
    got = out.numpy().reshape(views, tpv, embed)
    for v in range(views):
        one = rt.alloc_f32(tpv * embed)
        rt.patch_embed_u8(rt.upload_u8(imgs[v]), h, w, 14, MEAN, STD, proj, cls, regs,
                          n_register, pos, one)
        assert np.array_equal(got[v], one.numpy().reshape(tpv, embed)), f"view {v}"


def test_patch_embed_views_need_aligned_views(rt, rng):
    # 14 x 14 x 3 = 588 bytes per view: the second view starts 4-byte aligned
    imgs = rt.upload_u8(rng.integers(0, 256, (2, 14, 14, 3), dtype=np.uint8))
    proj = rt.prepare_linear_oihw_f32(588, 16, normals(rng, 16, 3, 14, 14), normals(rng, 16))
    cls, pos = rt.upload_f32(normals(rng, 16)), rt.upload_f32(normals(rng, 2, 16))
    with pytest.raises(vh.UnsupportedShape):
        rt.patch_embed_views_u8(imgs, 2, 14, 14, 14, MEAN, STD, proj, cls, None, 0, pos,
                                rt.alloc_f32(2 * 2 * 16))
    with pytest.raises(vh.VestraError):  # image count
        rt.patch_embed_views_u8(imgs, 3, 14, 14, 14, MEAN, STD, proj, cls, None, 0, pos,
                                rt.alloc_f32(3 * 2 * 16))


def test_patch_embed_rejects_unqualified_patch(rt, rng):
    img = rt.upload_u8(rng.integers(0, 256, (32, 32, 3), dtype=np.uint8))
    proj = rt.prepare_linear_oihw_f32(3 * 16 * 16, 8, normals(rng, 8, 3, 16, 16), normals(rng, 8))
    with pytest.raises(vh.UnsupportedShape):
        rt.patch_embed_u8(img, 32, 32, 16, MEAN, STD, proj, rt.upload_f32(normals(rng, 8)), None,
                          0, rt.upload_f32(normals(rng, 5, 8)), rt.alloc_f32(5 * 8))


# ---------------------------------------------------------------- block sequence
def make_block(rt, rng, D, H, M, rows, with_ls=True, with_qkn=True):
    host = {
        "norm1_gamma": normals(rng, D, scale=0.02, shift=1.0),
        "norm1_beta": normals(rng, D, scale=0.02),
        "norm2_gamma": normals(rng, D, scale=0.02, shift=1.0),
        "norm2_beta": normals(rng, D, scale=0.02),
    }
    if with_qkn:
        host.update({"qnorm_gamma": normals(rng, 64, scale=0.02, shift=1.0),
                     "qnorm_beta": normals(rng, 64, scale=0.02),
                     "knorm_gamma": normals(rng, 64, scale=0.02, shift=1.0),
                     "knorm_beta": normals(rng, 64, scale=0.02)})
    if with_ls:
        host["ls1"] = rng.uniform(0, 0.1, D).astype(np.float32)
        host["ls2"] = rng.uniform(0, 0.1, D).astype(np.float32)
    dev = {k: rt.upload_f32(v) for k, v in host.items()}
    return host, dev


@pytest.mark.parametrize("views,layer_idx,flags", [
    (1, 0, 0), (1, 4, vh.VK_BLOCK_FUSE_LS_LN), (3, 5, vh.VK_BLOCK_FUSE_LS_LN),
    (3, 6, vh.VK_BLOCK_FUSE_LS_LN), (12, 7, vh.VK_BLOCK_FUSE_LS_LN)])
def test_block_fused_ops_matches_oracle(rt, rng, views, layer_idx, flags):
    D, H, M, nreg, gh, gw = 768, 12, 3072, 1, 24, 36
    tpv = 1 + nreg + gh * gw
    rows = tpv * views
    cfg = dict(embed_dim=D, num_heads=H, head_dim=64, mlp_hidden=M, num_register=nreg,
               ln_eps=1e-6, qk_norm_eps=1e-5, rope_freq=100.0, rope_start=0, qknorm_start=0,
               alt_start=4)
    host, dev = make_block(rt, rng, D, H, M, rows)
    tokens = normals(rng, rows, D)
    q, k = normals(rng, rows * D), normals(rng, rows * D)
    attn, mlp = normals(rng, rows, D), normals(rng, rows, D)
    hidden = normals(rng, rows, M)
    camera = normals(rng, 2 * D, scale=0.02)
    act_t = {"tokens": rt.upload_f32(tokens), "ln1": rt.alloc_f32(rows * D),
             "q": rt.upload_f32(q), "k": rt.upload_f32(k), "attn_proj": rt.upload_f32(attn),
             "ln2": rt.alloc_f32(rows * D), "hidden": rt.upload_f32(hidden),
             "mlp_out": rt.upload_f32(mlp)}
    rt.vit_block_fused_ops(vh.VitConfig(**cfg), layer_idx, vh.layer_struct(**dev), None,
                           vh.activations_struct(**act_t), gh, gw, views,
                           rt.upload_f32(camera), flags)
    ref = oracle.block_fused_ops(tokens, q, k, attn, hidden, mlp, host, cfg, layer_idx, gh, gw,
                                 views, camera)
    for name in ("tokens", "ln1", "q", "k", "ln2", "hidden"):
        assert_parity(act_t[name].numpy(), ref[name], F32_ATOL, F32_RTOL,
                      f"block {name} views={views} layer={layer_idx}")


def test_block_gating_matches_reference_semantics(rt, rng):
    # vit_block.rs:1403-1453: below qknorm_start/rope_start the Q/K path is
    # untouched; ls absent -> unscaled residual (1368-1401).
    D, H, M, gh, gw = 768, 12, 3072, 2, 3
    rows = 1 + gh * gw
    cfg = dict(embed_dim=D, num_heads=H, head_dim=64, mlp_hidden=M, num_register=0,
               ln_eps=1e-6, qk_norm_eps=1e-5, rope_freq=100.0, rope_start=1, qknorm_start=1,
               alt_start=-1)
    host, dev = make_block(rt, rng, D, H, M, rows, with_ls=False)
    tokens, q, k = normals(rng, rows, D), normals(rng, rows * D), normals(rng, rows * D)
    attn, mlp, hidden = normals(rng, rows, D), normals(rng, rows, D), normals(rng, rows, M)
    for layer_idx in (0, 1):
        act_t = {"tokens": rt.upload_f32(tokens), "ln1": rt.alloc_f32(rows * D),
                 "q": rt.upload_f32(q), "k": rt.upload_f32(k), "attn_proj": rt.upload_f32(attn),
                 "ln2": rt.alloc_f32(rows * D), "hidden": rt.upload_f32(hidden),
                 "mlp_out": rt.upload_f32(mlp)}
        rt.vit_block_fused_ops(vh.VitConfig(**cfg), layer_idx, vh.layer_struct(**dev), None,
                               vh.activations_struct(**act_t), gh, gw, 1, None, 0)
        ref = oracle.block_fused_ops(tokens, q, k, attn, hidden, mlp, host, cfg, layer_idx, gh,
                                     gw, 1)
        got_q = act_t["q"].numpy()
        if layer_idx == 0:
            assert np.array_equal(got_q, q)
        else:
            assert not np.allclose(got_q, q)
        assert_parity(got_q, ref["q"], F32_ATOL, F32_RTOL, f"gated q layer {layer_idx}")
        assert np.array_equal(act_t["tokens"].numpy().reshape(rows, D), ref["tokens"])


def test_block_chain_with_cross_block_fusion(rt, rng):
    # three consecutive blocks, LS2+res fused with the next block's LN1
    D, H, M, nreg, gh, gw, views = 768, 12, 3072, 1, 24, 36, 2
    tpv = 1 + nreg + gh * gw
    rows = tpv * views
    cfg = dict(embed_dim=D, num_heads=H, head_dim=64, mlp_hidden=M, num_register=nreg,
               ln_eps=1e-6, qk_norm_eps=1e-5, rope_freq=100.0, rope_start=0, qknorm_start=0,
               alt_start=4)
    layers = [make_block(rt, rng, D, H, M, rows) for _ in range(3)]
    tokens = normals(rng, rows, D)
    q, k = normals(rng, rows * D), normals(rng, rows * D)
    attn, mlp, hidden = normals(rng, rows, D), normals(rng, rows, D), normals(rng, rows, M)
    camera = normals(rng, 2 * D, scale=0.02)
    act_t = {"tokens": rt.upload_f32(tokens), "ln1": rt.alloc_f32(rows * D),
             "q": rt.upload_f32(q), "k": rt.upload_f32(k), "attn_proj": rt.upload_f32(attn),
             "ln2": rt.alloc_f32(rows * D), "hidden": rt.upload_f32(hidden),
             "mlp_out": rt.upload_f32(mlp)}
    act = vh.activations_struct(**act_t)
    cam_t = rt.upload_f32(camera)
    x, qq, kk, hh = tokens, q, k, hidden
    for i, layer_idx in enumerate((3, 4, 5)):
        flags = vh.VK_BLOCK_FUSE_LS_LN
        nxt = None
        if i > 0:
            flags |= vh.VK_BLOCK_SKIP_LN1
        if i < 2:
            flags |= vh.VK_BLOCK_FUSE_NEXT_LN1
            nxt = vh.layer_struct(**layers[i + 1][1])
        rt.vit_block_fused_ops(vh.VitConfig(**cfg), layer_idx, vh.layer_struct(**layers[i][1]),
                               nxt, act, gh, gw, views, cam_t, flags)
        ref = oracle.block_fused_ops(x, qq, kk, attn, hh, mlp, layers[i][0], cfg, layer_idx, gh,
                                     gw, views, camera)
        x, qq, kk, hh = ref["tokens"], ref["q"], ref["k"], ref["hidden"]
    got = act_t["tokens"].numpy()
    assert_parity(got, x, F32_ATOL, F32_RTOL, "chained tokens")
    assert_parity(act_t["ln1"].numpy(), ref["ln1"], F32_ATOL, F32_RTOL, "chained ln1")
    assert_parity(act_t["ln2"].numpy(), ref["ln2"], F32_ATOL, F32_RTOL, "chained ln2")
    assert_parity(act_t["q"].numpy(), qq, F32_ATOL, F32_RTOL, "chained q")
    assert_parity(act_t["hidden"].numpy(), hh, F32_ATOL, F32_RTOL, "chained hidden")
