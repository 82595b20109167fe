"""GPU parity of the whole device-resident block, vk_vit_block_forward_f32
(run_tail_device, vit_block.rs:489-582; block order vit_block.rs:1019-1139).

Two checks per case:

1. Composition: the block must give exactly the bits of the individual entry
   points called in the reference order (LN1, QKV storing head-major, Q/K-norm
   + RoPE, attention, head-major projection + LayerScale + residual, LN2,
   FC1 + GELU, FC2 + LayerScale + residual).  Each of those has its own parity
   test against the oracle; this pins the wiring (gating, global vs local
   attention, camera slot, buffer reuse).
2. Parity: against the oracle's composition of the same block.  After several
   K-long dot products no per-element closed form is practical, so the bound
   is the f32 rounding envelope of the oracle itself: with e = max |oracle -
   f64| (f64 = the same block in float64, A&S GELU and the oracle's f32
   rotation angles), every element must satisfy
   |gpu - oracle| <= 1e-6 + 1e-5*|f64| + 4*e.
   A wiring mistake (a skipped or misplaced step, a wrong scale, attention
   across views) moves results by 1e-2 or more.
"""
import numpy as np
import pytest

import oracle
from block_twin import block_f64, config, is_global, make_params, normals

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


class DeviceBlock:
    """Uploads one block's parameters and prepares its four projections."""

    def __init__(self, rt, p, D, M):
        self.vec = {k: rt.upload_f32(v) for k, v in p.items() if not k.endswith(("_w", "_b"))}
        self.qkv = rt.prepare_linear_f32(D, 3 * D, p["qkv_w"], p["qkv_b"])
        self.proj = rt.prepare_linear_f32(D, D, p["proj_w"], p["proj_b"], p.get("ls1"))
        self.fc1 = rt.prepare_linear_f32(D, M, p["fc1_w"], p["fc1_b"])
        self.fc2 = rt.prepare_linear_f32(M, D, p["fc2_w"], p["fc2_b"], p.get("ls2"))
        self.struct = vh.block_weights_struct(qkv=self.qkv, proj=self.proj, fc1=self.fc1,
                                              fc2=self.fc2, **self.vec)


def assert_envelope(got, ora, f64, label):
    got, ora, f64 = (np.asarray(a, np.float64).reshape(-1) for a in (got, ora, f64))
    e = np.max(np.abs(ora - f64))
    tol = 1e-6 + 1e-5 * np.abs(f64) + 4 * e
    d = np.abs(got - ora)
    i = int(np.argmax(d / tol))
    assert d[i] <= tol[i], (f"[{label}] |gpu-oracle|={d[i]:.3e} > tol={tol[i]:.3e} "
                            f"(oracle envelope {e:.3e}) at {i}")


# ---------------------------------------------------------------- the unfused GPU sequence
def unfused_block(rt, dev, cfg, layer, tokens, gh, gw, views, camera):
    D, H, M = cfg["embed_dim"], cfg["num_heads"], cfg["mlp_hidden"]
    ns = 1 + cfg["num_register"]
    tpv = ns + gh * gw
    rows = tpv * views
    glob = is_global(cfg, layer)
    if cfg["alt_start"] >= 0 and layer == cfg["alt_start"]:
        for v in range(views):
            rt.copy_segment_into_f32(tokens, v * tpv * D, camera, (1 if v else 0) * D, D)
    ln = rt.alloc_f32(rows * D)
    rt.layernorm_into_f32(tokens, dev.vec["norm1_gamma"], dev.vec["norm1_beta"], rows, D,
                          cfg["ln_eps"], ln)
    q, k, v = (rt.alloc_f32(rows * D) for _ in range(3))
    dev.qkv.run_qkv_hnd(ln, rows, H, q, k, v)
    use_qkn = cfg["qknorm_start"] >= 0 and layer >= cfg["qknorm_start"] and \
        "qnorm_gamma" in dev.vec
    if cfg["rope_start"] >= 0 and layer >= cfg["rope_start"]:
        g = [dev.vec[n] if use_qkn else None
             for n in ("qnorm_gamma", "qnorm_beta", "knorm_gamma", "knorm_beta")]
        rt.qk_norm_rope_grid_f32(q, k, *g, H, 64, ns, gh, gw, views, glob,
                                 vh.VK_QK_HEADS_OUTER, cfg["rope_freq"], cfg["qk_norm_eps"],
                                 rope_mode=cfg.get("rope_mode", 0))
    elif use_qkn:
        rt.layernorm_into_f32(q, dev.vec["qnorm_gamma"], dev.vec["qnorm_beta"], rows * H, 64,
                              cfg["qk_norm_eps"], q)
        rt.layernorm_into_f32(k, dev.vec["knorm_gamma"], dev.vec["knorm_beta"], rows * H, 64,
                              cfg["qk_norm_eps"], k)
    attn = rt.alloc_f32(rows * D)
    rt.attention_into_f32(q, k, v, H if glob else H * views, rows if glob else tpv, 64, attn)
    dev.proj.run_hnd_residual(attn, rows, H, tokens)
    rt.layernorm_into_f32(tokens, dev.vec["norm2_gamma"], dev.vec["norm2_beta"], rows, D,
                          cfg["ln_eps"], ln)
    hidden = rt.alloc_f32(rows * M)
    dev.fc1.run_gelu(ln, rows, hidden)
    dev.fc2.run_residual(hidden, rows, tokens)
    return {"q": q, "k": k, "v": v, "attn": attn, "ln2": ln, "hidden": hidden}


CASES = [
    # (D, H, M, gh, gw, views, layer, cfg overrides)
    pytest.param(768, 12, 3072, 4, 6, 1, 0, {}, id="vitb-1view-local"),
    pytest.param(768, 12, 3072, 4, 6, 3, 2, {}, id="vitb-3views-local"),
    pytest.param(768, 12, 3072, 4, 6, 3, 5, {}, id="vitb-3views-global"),
    pytest.param(768, 12, 3072, 4, 6, 2, 4, {}, id="vitb-2views-camera"),
    pytest.param(768, 12, 3072, 3, 5, 2, 1, dict(rope_start=-1), id="vitb-qknorm-no-rope"),
    pytest.param(768, 12, 3072, 3, 5, 2, 3, dict(qknorm_start=-1, alt=-1), id="vitb-rope-no-qknorm"),
    pytest.param(1024, 16, 4096, 3, 4, 2, 7, {}, id="vitl-2views-global"),
    pytest.param(768, 12, 3072, 24, 36, 1, 0, {}, id="vitb-504x336-local"),
    pytest.param(768, 12, 3072, 4, 6, 3, 2, dict(rope_mode=1), id="vitb-3views-local-interleaved"),
    pytest.param(768, 12, 3072, 4, 6, 3, 5, dict(rope_mode=3),
                 id="vitb-3views-global-interleaved-exphead"),
    pytest.param(768, 12, 3072, 24, 36, 1, 0, dict(rope_mode=2), id="vitb-504x336-exphead"),
]


@pytest.mark.parametrize("D,H,M,gh,gw,views,layer,over", CASES)
def test_block_forward(rt, rng, D, H, M, gh, gw, views, layer, over):
    cfg = config(D, H, M, **over)
    rows = (2 + gh * gw) * views
    p = make_params(rng, D, M)
    dev = DeviceBlock(rt, p, D, M)
    x0 = normals(rng, rows, D)
    camera = normals(rng, 2 * D)
    cam_dev = rt.upload_f32(camera)

    tokens = rt.upload_f32(x0)
    ws = rt.block_workspace(rows, D, M)
    rt.vit_block_forward_f32(vh.VitConfig(**cfg), layer, dev.struct, tokens, gh, gw, views,
                             cam_dev, ws.struct)
    got = {"tokens": tokens.numpy()}
    got.update({n: ws.tensors[n].numpy() for n in ("q", "k", "v", "attn", "hidden")})
    got["ln2"] = ws.tensors["ln"].numpy()

    # 1. the same bits as the unfused GPU sequence
    t2 = rt.upload_f32(x0)
    parts = unfused_block(rt, dev, cfg, layer, t2, gh, gw, views, cam_dev)
    assert np.array_equal(got["tokens"], t2.numpy()), "tokens differ from the unfused sequence"
    for n, t in parts.items():
        assert np.array_equal(got[n], t.numpy()), f"{n} differs from the unfused sequence"

    # 2. parity with the oracle inside its own rounding envelope
    ora = oracle.block_forward(x0, p, cfg, layer, gh, gw, views, camera)
    ref = block_f64(x0, p, cfg, layer, gh, gw, views, camera)
    for n in ("q", "k", "v", "attn", "ln2", "hidden", "tokens"):
        assert_envelope(got[n], ora[n], ref[n], f"{n} layer {layer}")


def test_block_forward_chained_blocks_reuse_workspace(rt, rng):
    """Four blocks in a row (local, global, camera slot at alt_start 2) share
    one workspace; the residual stream stays on the device throughout."""
    D, H, M, gh, gw, views = 768, 12, 3072, 3, 4, 2
    cfg = config(D, H, M, alt=2)
    rows = (2 + gh * gw) * views
    params = [make_params(rng, D, M) for _ in range(4)]
    devs = [DeviceBlock(rt, p, D, M) for p in params]
    x0 = normals(rng, rows, D)
    camera = normals(rng, 2 * D)
    tokens, ws, cam = rt.upload_f32(x0), rt.block_workspace(rows, D, M), rt.upload_f32(camera)
    ora, ref = x0, x0.astype(np.float64)
    for layer, (p, dev) in enumerate(zip(params, devs)):
        rt.vit_block_forward_f32(vh.VitConfig(**cfg), layer, dev.struct, tokens, gh, gw, views,
                                 cam, ws.struct)
        ora = oracle.block_forward(ora, p, cfg, layer, gh, gw, views, camera)["tokens"]
        ref = block_f64(ref, p, cfg, layer, gh, gw, views, camera)["tokens"]
    assert_envelope(tokens.numpy(), ora, ref, "4 chained blocks")


def test_block_forward_errors(rt, rng):
    D, H, M = 768, 12, 3072
    cfg = vh.VitConfig(**config(D, H, M))
    dev = DeviceBlock(rt, make_params(rng, D, M), D, M)
    rows = (2 + 2 * 3) * 1
    ws = rt.block_workspace(rows, D, M)
    with pytest.raises(vh.VestraError):
        rt.vit_block_forward_f32(cfg, 0, dev.struct, rt.alloc_f32(rows * D + 1), 2, 3, 1, None,
                                 ws.struct)                      # token count
    small = rt.block_workspace(rows - 1, D, M)
    with pytest.raises(vh.VestraError):
        rt.vit_block_forward_f32(cfg, 0, dev.struct, rt.alloc_f32(rows * D), 2, 3, 1, None,
                                 small.struct)                   # workspace size
    with pytest.raises(vh.VestraError):
        rt.vit_block_forward_f32(cfg, 4, dev.struct, rt.alloc_f32(rows * D), 2, 3, 1, None,
                                 ws.struct)                      # camera missing at alt_start
    swapped = vh.block_weights_struct(qkv=dev.fc1, proj=dev.proj, fc1=dev.qkv, fc2=dev.fc2,
                                      **dev.vec)
    with pytest.raises(vh.VestraError):
        rt.vit_block_forward_f32(cfg, 0, swapped, rt.alloc_f32(rows * D), 2, 3, 1, None,
                                 ws.struct)                      # projection shapes


def test_block_forward_graph_replays(rt, rng):
    """Two whole blocks (one split-K single view of 4x6 patches, so every
    projection takes the two-pass path) captured into a HIP graph after one
    eager pass: every replay, with eager work and synchronisation between
    replays, gives the bits of the eager sequence."""
    import gc
    D, H, M, gh, gw, views = 768, 12, 3072, 4, 6, 1
    cfg = vh.VitConfig(**config(D, H, M, alt=1))
    rows = (2 + gh * gw) * views
    devs = [DeviceBlock(rt, make_params(rng, D, M), D, M) for _ in range(2)]
    x0 = normals(rng, rows, D)
    cam = rt.upload_f32(normals(rng, 2 * D))
    tokens, ws = rt.upload_f32(x0), rt.block_workspace(rows, D, M)

    def step():
        for layer, dev in enumerate(devs):
            rt.vit_block_forward_f32(cfg, layer, dev.struct, tokens, gh, gw, views, cam, ws.struct)

    step()  # eager: RoPE table and split-K buffer exist before capture
    want = tokens.numpy()
    rt.synchronize()
    gc.disable()
    try:
        rt.begin_capture()
        step()
        graph = rt.end_capture()
    finally:
        gc.enable()
    for _ in range(3):
        tokens.write(x0)
        graph.launch()
        rt.synchronize()
        assert np.array_equal(tokens.numpy(), want)
        scratch = rt.upload_f32(normals(rng, rows, D))  # eager work between replays
        rt.layernorm_into_f32(scratch, devs[0].vec["norm1_gamma"], devs[0].vec["norm1_beta"],
                              rows, D, 1e-6, scratch)
        rt.synchronize()
