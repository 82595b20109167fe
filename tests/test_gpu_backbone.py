"""GPU parity of the backbone's block loop on the device, vk_backbone_forward_f32
(Backbone::forward_multi_view_ordered, backbone.rs:688-877; captures
backbone.rs:1139-1179).

1. Composition: the bits of the per-block entry (vk_vit_block_forward_f32)
   and vk_capture_f32 called in the reference's order, with the snapshot of
   the last local layer for captures at global layers.
2. Parity: the oracle's composition within its own f32 rounding envelope
   against a float64 twin (as for the single block):
   |gpu - oracle| <= 1e-6 + 1e-5*|f64| + 4*max|oracle - f64|.
"""
import numpy as np
import pytest

import oracle
from block_twin import backbone_f64, config, is_global, make_params, normals
from test_gpu_block_forward import DeviceBlock, assert_envelope

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


@pytest.mark.parametrize("D,H,M,gh,gw,views,depth,alt,outs,cat", [
    (768, 12, 3072, 3, 4, 2, 6, 2, [5, 1, 3, 4], True),
    (768, 12, 3072, 3, 4, 1, 4, -1, [3, 0], True),
    (1024, 16, 4096, 2, 3, 3, 4, 1, [3, 2], False),
])
def test_backbone_forward(rt, rng, D, H, M, gh, gw, views, depth, alt, outs, cat):
    cfg = config(D, H, M, alt=alt)
    n = 2 + gh * gw
    rows = n * views
    W = 2 * D if cat else D
    params = [make_params(rng, D, M) for _ in range(depth)]
    devs = [DeviceBlock(rt, p, D, M) for p in params]
    x0, cam = normals(rng, rows, D), normals(rng, 2 * D)
    ng, nb = normals(rng, D, scale=0.02, shift=1), normals(rng, D, scale=0.02)
    cam_d, ng_d, nb_d = rt.upload_f32(cam), rt.upload_f32(ng), rt.upload_f32(nb)
    vcfg = vh.VitConfig(**cfg)

    tokens, ws, local = rt.upload_f32(x0), rt.block_workspace(rows, D, M), rt.alloc_f32(rows * D)
    feats = [rt.alloc_f32(views * gh * gw * W) for _ in outs]
    cams = [rt.alloc_f32(views * W) for _ in outs]
    rt.backbone_forward_f32(vcfg, [d.struct for d in devs], tokens, gh, gw, views, cam_d, ng_d,
                            nb_d, cat, outs, feats, cams, ws, local)

    # 1. the per-block entry and the capture in the reference's order
    t2, ws2 = rt.upload_f32(x0), rt.block_workspace(rows, D, M)
    snap = rt.upload_f32(x0)
    want = {}
    for layer, dev in enumerate(devs):
        rt.vit_block_forward_f32(vcfg, layer, dev.struct, t2, gh, gw, views, cam_d, ws2.struct)
        glob = is_global(cfg, layer)
        for i, o in enumerate(outs):
            if o == layer:
                f, c = rt.alloc_f32(views * gh * gw * W), rt.alloc_f32(views * W)
                rt.capture_f32((snap if glob else t2) if cat else None, t2, n, 2, D, views, ng_d,
                               nb_d, 1e-6, cat, f, c)
                want[i] = (f.numpy(), c.numpy())
        if not glob:
            snap = rt.copy_f32(t2)
    assert np.array_equal(tokens.numpy(), t2.numpy())
    for i in range(len(outs)):
        assert np.array_equal(feats[i].numpy(), want[i][0]), f"feat of out layer {outs[i]}"
        assert np.array_equal(cams[i].numpy(), want[i][1]), f"cam of out layer {outs[i]}"

    # 2. parity with the oracle
    xo, caps = oracle.backbone_forward(x0, params, cfg, gh, gw, views, cam, ng, nb, cat, outs)
    x64, caps64 = backbone_f64(x0, params, cfg, gh, gw, views, cam, ng, nb, cat, outs)
    assert_envelope(tokens.numpy(), xo, x64, "tokens")
    for i in range(len(outs)):
        assert_envelope(feats[i].numpy(), caps[i][0], caps64[i][0], f"feat {outs[i]}")
        assert_envelope(cams[i].numpy(), caps[i][1], caps64[i][1], f"cam {outs[i]}")


@pytest.mark.parametrize("D,H,M,gh,gw,f16", [
    pytest.param(768, 12, 3072, 24, 36, False, id="vitb-504x336"),
    pytest.param(1024, 16, 4096, 48, 72, True, id="vitl-1008x672-f16-params"),
])
def test_backbone_block_loop_full_size(rt, rng, D, H, M, gh, gw, f16):
    """One image at full size through the block loop, where FC2 runs split-K
    and its sum pass also writes the next block's LN1: the bits of the
    per-block entry called block by block.  Four blocks with alt_start 2:
    blocks 0 and 2 hand LN1 on, block 1 precedes the camera write and block
    3 is the last."""
    cfg = config(D, H, M, alt=2)
    rows = 2 + gh * gw
    devs = []
    for _ in range(4):
        p = make_params(rng, D, M)
        dev = DeviceBlock(rt, p, D, M)
        if f16:
            dev.vec = {k: rt.upload_f16(v) for k, v in p.items()
                       if not k.endswith(("_w", "_b"))}
            dev.struct = vh.block_weights_struct(qkv=dev.qkv, proj=dev.proj, fc1=dev.fc1,
                                                 fc2=dev.fc2, **dev.vec)
        devs.append(dev)
    x0 = normals(rng, rows, D)
    cam = rt.upload_f32(normals(rng, 2 * D))
    vcfg = vh.VitConfig(**cfg)

    tokens, ws = rt.upload_f32(x0), rt.block_workspace(rows, D, M)
    rt.backbone_forward_f32(vcfg, [d.struct for d in devs], tokens, gh, gw, 1, cam, None, None,
                            False, [], [], [], ws, None)
    t2, ws2 = rt.upload_f32(x0), rt.block_workspace(rows, D, M)
    for layer, dev in enumerate(devs):
        rt.vit_block_forward_f32(vcfg, layer, dev.struct, t2, gh, gw, 1, cam, ws2.struct)
    assert np.array_equal(tokens.numpy(), t2.numpy())
    for name in ("ln", "q", "k", "v", "attn", "hidden"):
        assert np.array_equal(ws.tensors[name].numpy(), ws2.tensors[name].numpy()), name


def test_backbone_forward_errors(rt, rng):
    D, H, M = 768, 12, 3072
    cfg = vh.VitConfig(**config(D, H, M))
    dev = DeviceBlock(rt, make_params(rng, D, M), D, M)
    rows = 2 + 2 * 3
    ws = rt.block_workspace(rows, D, M)
    g, b = rt.upload_f32(np.ones(D, np.float32)), rt.upload_f32(np.zeros(D, np.float32))
    f, c = rt.alloc_f32(6 * 2 * D), rt.alloc_f32(2 * D)
    with pytest.raises(vh.VestraError):   # out layer never reached (backbone.rs:1333-1343)
        rt.backbone_forward_f32(cfg, [dev.struct], rt.alloc_f32(rows * D), 2, 3, 1, None, g, b,
                                True, [1], [f], [c], ws, rt.alloc_f32(rows * D))
