"""The runtime's sequential LayerNorm order (VK_LN_ORDER_SEQUENTIAL) against
the oracle, bit for bit.

The reference's device method is layernorm_f32_cpu_order (vit_block.rs:
528-537, 567-576, 627-636): the CPU kernel's order, mean and biased two-pass
variance summed left to right (the sums of dpt_head.rs:272-296), then
1/sqrtf(var + eps).  In that order every LayerNorm of the path must give the
oracle's bits: block LayerNorm (in and out of place, f32 and f16
parameters), the fused LayerScale + residual + LayerNorm (and its camera-slot
form inside the block sequence), the per-(head, token) Q/K LayerNorm with
its rotation (standalone, explicit and grid positions, every RoPE
convention), the capture and the token -> CHW hand-off.  The benchmark's
12-view sequence is re-run in this order with tokens, LN1, LN2, Q and K
bit-identical to the oracle after every block (GELU keeps its F32 bar).
Whole blocks (projections and attention on F32 MFMA) are compared with the
oracle's envelope, and the LayerNorm parts of their outputs with the oracle's
LayerNorm of the device's own inputs, bit for bit.
"""
import numpy as np
import pytest

import oracle
from block_twin import backbone_f64, config, is_global, make_params, normals
from conftest import F32_ATOL, F32_RTOL, assert_parity

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")
import bench  # noqa: E402
from test_gpu_block_forward import DeviceBlock, assert_envelope  # noqa: E402
from test_gpu_headline_sequence import run_chain  # noqa: E402


@pytest.fixture(scope="module")
def srt():
    """A runtime of its own in the sequential order (the session's runtime
    keeps the default)."""
    r = vh.Runtime(0)
    r.set_layernorm_order(vh.VK_LN_ORDER_SEQUENTIAL)
    yield r
    r.synchronize()


def test_order_switch(rt):
    r = vh.Runtime(0)
    assert r.layernorm_order() == vh.VK_LN_ORDER_TREE
    r.set_layernorm_order(vh.VK_LN_ORDER_SEQUENTIAL)
    assert r.layernorm_order() == vh.VK_LN_ORDER_SEQUENTIAL
    with pytest.raises(vh.VestraError):
        r.set_layernorm_order(2)
    assert r.layernorm_order() == vh.VK_LN_ORDER_SEQUENTIAL
    assert rt.layernorm_order() == vh.VK_LN_ORDER_TREE
    r.close()


@pytest.mark.parametrize("rows,cols,f16", [(866, 768, False), (10392, 768, False),
                                           (3458, 1024, True), (5, 8, False), (37, 64, False),
                                           (3, 1300, False), (2, 8192, True), (1, 768, False)])
def test_layernorm_bit_exact(srt, rng, rows, cols, f16):
    x = normals(rng, rows, cols)
    g = normals(rng, cols, scale=0.02, shift=1.0)
    b = normals(rng, cols, scale=0.02)
    up = srt.upload_f16 if f16 else srt.upload_f32
    if f16:
        g, b = g.astype(np.float16), b.astype(np.float16)
    out = srt.layernorm_f32_cpu_order(srt.upload_f32(x), up(g), up(b), rows, cols, 1e-6)
    ref = oracle.layernorm(x, g, b, 1e-6)
    assert np.array_equal(out.numpy().reshape(rows, cols), ref)
    # in place, as scalar::layernorm runs (vit_block.rs:712)
    t = srt.upload_f32(x)
    srt.layernorm_into_f32(t, up(g), up(b), rows, cols, 1e-6, t)
    assert np.array_equal(t.numpy().reshape(rows, cols), ref)


@pytest.mark.parametrize("rows,cols,with_ls,f16", [(10392, 768, True, False),
                                                   (866, 768, False, False),
                                                   (3458, 1024, True, True), (7, 12, True, False)])
def test_layerscale_residual_layernorm_bit_exact(srt, rng, rows, cols, with_ls, f16):
    x, y = normals(rng, rows, cols), normals(rng, rows, cols)
    ls = rng.uniform(0, 0.1, cols).astype(np.float32)
    g = normals(rng, cols, scale=0.02, shift=1.0)
    b = normals(rng, cols, scale=0.02)
    pdt = np.float16 if f16 else np.float32
    up = srt.upload_f16 if f16 else srt.upload_f32
    ls, g, b = ls.astype(pdt), g.astype(pdt), b.astype(pdt)
    tx, out = srt.upload_f32(x), srt.alloc_f32(rows * cols)
    srt.layerscale_residual_layernorm_f32(tx, srt.upload_f32(y), up(ls) if with_ls else None,
                                          up(g), up(b), rows, cols, 1e-6, out)
    want_x = oracle.layerscale_residual(x, y, ls if with_ls else None)
    assert np.array_equal(tx.numpy().reshape(rows, cols), want_x)
    assert np.array_equal(out.numpy().reshape(rows, cols), oracle.layernorm(want_x, g, b, 1e-6))


@pytest.mark.parametrize("mode", oracle.ROPE_MODES)
@pytest.mark.parametrize("f16", [False, True])
def test_qk_norm_rope_reference_form_bit_exact(srt, rng, mode, f16):
    heads, n_special, gh, gw = 12, 2, 24, 36
    n = n_special + gh * gw
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    prm = [normals(rng, 64, scale=0.02, shift=1.0 if i % 2 == 0 else 0.0) for i in range(4)]
    if f16:
        prm = [p.astype(np.float16) for p in prm]
    up = srt.upload_f16 if f16 else srt.upload_f32
    pos = oracle.rope_positions(n_special, gh, gw, 1, False)
    tq, tk = srt.upload_f32(q), srt.upload_f32(k)
    srt.qk_norm_rope_mode_f32(tq, tk, *[up(p) for p in prm], srt.upload_i64(pos.astype(np.int64)),
                              heads, n, 100.0, 1e-5, mode)
    rq, rk = oracle.qk_norm_rope(q, k, *prm, pos, heads, n, mode=mode)
    assert np.array_equal(tq.numpy().reshape(rq.shape), rq)
    assert np.array_equal(tk.numpy().reshape(rk.shape), rk)


@pytest.mark.parametrize("glob", [False, True], ids=["local", "global"])
def test_qk_norm_rope_grid_12_views_bit_exact(srt, rng, glob):
    heads, n_special, gh, gw, views = 12, 2, 24, 36, 12
    tpv = n_special + gh * gw
    rows = tpv * views
    q, k = normals(rng, rows * heads * 64), normals(rng, rows * heads * 64)
    prm = [normals(rng, 64, scale=0.02, shift=1.0 if i % 2 == 0 else 0.0) for i in range(4)]
    layout = vh.VK_QK_HEADS_OUTER if glob else vh.VK_QK_VIEWS_OUTER
    tq, tk = srt.upload_f32(q), srt.upload_f32(k)
    srt.qk_norm_rope_grid_f32(tq, tk, *[srt.upload_f32(p) for p in prm], heads, 64, n_special,
                              gh, gw, views, glob, layout)
    pos = oracle.rope_positions(n_special, gh, gw, views, glob)
    if glob:
        rq, rk = oracle.qk_norm_rope(q, k, *prm, pos, heads, rows)
    else:
        rq = q.reshape(views, heads, tpv, 64).copy()
        rk = k.reshape(views, heads, tpv, 64).copy()
        for v in range(views):
            rq[v], rk[v] = [a.reshape(heads, tpv, 64) for a in oracle.qk_norm_rope(
                rq[v], rk[v], *prm, pos[v * tpv:(v + 1) * tpv], heads, tpv)]
    assert np.array_equal(tq.numpy().reshape(-1), rq.reshape(-1))
    assert np.array_equal(tk.numpy().reshape(-1), rk.reshape(-1))


@pytest.mark.parametrize("views,cat", [(1, True), (3, False), (2, True)])
def test_capture_bit_exact(srt, rng, views, cat):
    D, ns, gh, gw = 768, 2, 24, 36
    n = ns + gh * gw
    x, lx = normals(rng, views * n, D), normals(rng, views * n, D)
    g, b = normals(rng, D, scale=0.02, shift=1.0), normals(rng, D, scale=0.02)
    W = 2 * D if cat else D
    f, c = srt.alloc_f32(views * gh * gw * W), srt.alloc_f32(views * W)
    srt.capture_f32(srt.upload_f32(lx) if cat else None, srt.upload_f32(x), n, ns, D, views,
                    srt.upload_f32(g), srt.upload_f32(b), 1e-6, cat, f, c)
    wf, wc = oracle.capture(lx, x, n, ns, D, views, g, b, 1e-6, cat)
    assert np.array_equal(f.numpy().reshape(wf.shape), wf)
    assert np.array_equal(c.numpy().reshape(wc.shape), wc)


@pytest.mark.parametrize("n_tok,c", [(864, 1536), (864, 768), (37, 64)])
def test_token_to_chw_bit_exact(srt, rng, n_tok, c):
    tok = normals(rng, n_tok, c)
    g, b = normals(rng, c, scale=0.02, shift=1.0), normals(rng, c, scale=0.02)
    out = srt.alloc_f32(n_tok * c)
    srt.token_to_chw_f32(srt.upload_f32(tok), n_tok, c, srt.upload_f32(g), srt.upload_f32(b),
                         1e-5, out)
    assert np.array_equal(out.numpy().reshape(c, n_tok), oracle.token_to_chw(tok, n_tok, c, g, b))


def test_vitb_12_views_12_blocks_bits(srt, rng):
    """The benchmark's sequence in the sequential order: the residual stream,
    LN1, LN2, Q and K are the oracle's bits after every block."""
    model = run_chain(srt, rng, 12, bench.VITB, f16=False, exact=("ln1", "ln2", "q", "k"))
    assert model.rows == 10392


def test_vitl_24_blocks_f16_parameters_bits(srt, rng):
    run_chain(srt, rng, 1, bench.VITL, f16=True, exact=("ln1", "ln2", "q", "k"))


@pytest.mark.parametrize("gh,gw,views,depth,alt,outs", [
    (3, 4, 2, 4, 1, [3, 1]),
    (24, 36, 1, 3, 1, [2]),
])
def test_backbone_sequential_order(srt, rng, gh, gw, views, depth, alt, outs):
    """Whole blocks and the capture in the sequential order: within the
    oracle's envelope, and the capture's LayerNorm half is the oracle's
    LayerNorm of the device's own final tokens, bit for bit.  At 24 x 36 the
    FC2 projections run split-K, whose sum pass writes the next LN1 in the
    tree order: in the sequential order the projection and the LayerNorm are
    two launches, and the loop's bits equal the per-block entry's."""
    D, H, M = 768, 12, 3072
    cfg = config(D, H, M, alt=alt)
    ns = 1 + cfg["num_register"]
    n = ns + gh * gw
    rows = n * views
    params = [make_params(rng, D, M) for _ in range(depth)]
    devs = [DeviceBlock(srt, p, D, M) for p in params]
    x0, cam = normals(rng, rows, D), normals(rng, 2 * D)
    ng, nb = normals(rng, D, scale=0.02, shift=1), normals(rng, D, scale=0.02)
    cam_d, ng_d, nb_d = srt.upload_f32(cam), srt.upload_f32(ng), srt.upload_f32(nb)
    vcfg = vh.VitConfig(**cfg)
    tokens, ws, local = srt.upload_f32(x0), srt.block_workspace(rows, D, M), srt.alloc_f32(rows * D)
    feats = [srt.alloc_f32(views * gh * gw * 2 * D) for _ in outs]
    cams = [srt.alloc_f32(views * 2 * D) for _ in outs]
    srt.backbone_forward_f32(vcfg, [d.struct for d in devs], tokens, gh, gw, views, cam_d, ng_d,
                             nb_d, True, outs, feats, cams, ws, local)
    t2, ws2 = srt.upload_f32(x0), srt.block_workspace(rows, D, M)
    for layer, dev in enumerate(devs):
        srt.vit_block_forward_f32(vcfg, layer, dev.struct, t2, gh, gw, views, cam_d, ws2.struct)
    assert np.array_equal(tokens.numpy(), t2.numpy())
    xo, caps = oracle.backbone_forward(x0, params, cfg, gh, gw, views, cam, ng, nb, True, outs)
    x64, caps64 = backbone_f64(x0, params, cfg, gh, gw, views, cam, ng, nb, True, outs)
    assert_envelope(tokens.numpy(), xo, x64, "tokens")
    last = outs.index(depth - 1)
    got = feats[last].numpy().reshape(views, gh * gw, 2 * D)[:, :, D:]
    xt = tokens.numpy().reshape(views, n, D)[:, ns:]
    want = np.stack([oracle.layernorm(xt[v], ng, nb, 1e-6) for v in range(views)])
    assert np.array_equal(got, want)
    for i, o in enumerate(outs):
        assert_envelope(feats[i].numpy(), caps[i][0], caps64[i][0], f"feat {o}")
