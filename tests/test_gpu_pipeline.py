"""GPU parity of the whole image-to-head-input path, end to end through the C
ABI: u8 camera frames -> preprocess resize + patch snap -> fused patch
embedding with the bicubic position table -> backbone blocks with captures
-> the head's LayerNorm + token -> CHW hand-off.

The resize is bit-exact (u8); everything after it is compared with the
oracle's composition of the same steps inside the oracle's own f32 rounding
envelope against a float64 twin: |gpu - oracle| <= 1e-6 + 1e-5*|f64| +
4*max|oracle - f64| (as for one block).  The twin takes the oracle's resized
frames and position table (both pinned separately, the table bit-exactly).
"""
import numpy as np
import pytest

import oracle
from block_twin import _ln64, backbone_f64, config, make_params, normals
from test_gpu_block_forward import DeviceBlock, assert_envelope

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")

MEAN, STD = [0.485, 0.456, 0.406], [0.229, 0.224, 0.225]


def _patch_embed_f64(img, wt, b, cls, reg, pos):
    """float64 twin of the fused patch embedding (preprocess.rs:484-500,
    patch_embed.rs:53-130, pos_embed.rs:254-306)."""
    h, w, _ = img.shape
    x = (img.astype(np.float64) / 255.0 - np.array(MEAN)) / np.array(STD)  # HWC
    gh, gw = h // 14, w // 14
    patches = x.reshape(gh, 14, gw, 14, 3).transpose(0, 2, 4, 1, 3).reshape(gh * gw, 588)
    proj = patches @ wt.reshape(wt.shape[0], 588).astype(np.float64).T + b
    pos64 = pos.astype(np.float64)
    rows = [cls.astype(np.float64) + pos64[0], reg.astype(np.float64)]
    return np.concatenate([np.stack(rows), proj + pos64[1:]])


@pytest.mark.parametrize("views,depth,alt,outs", [(1, 3, -1, [2, 0]), (3, 4, 1, [1, 3])])
def test_image_to_head_input(rt, rng, views, depth, alt, outs):
    D, H, M = 768, 12, 3072
    fh, fw = 61, 85                                   # -> 42 x 56 after the 56-bound resize
    oh, ow = rt.preprocess_shape(fh, fw, 56, 14)
    gh, gw = oh // 14, ow // 14
    n, n_patch = 2 + gh * gw, gh * gw
    cfg = config(D, H, M, alt=alt)
    params = [make_params(rng, D, M) for _ in range(depth)]
    devs = [DeviceBlock(rt, p, D, M) for p in params]
    wt, b = normals(rng, D, 3, 14, 14, scale=0.02), normals(rng, D, scale=0.02)
    cls, reg = normals(rng, D, scale=0.02), normals(rng, D, scale=0.02)
    grid_tab = normals(rng, 37 * 37 + 1, D, scale=0.02)
    cam = normals(rng, 2 * D, scale=0.02)
    vg, vb = normals(rng, D, scale=0.02, shift=1), normals(rng, D, scale=0.02)
    hg, hb = normals(rng, 2 * D, scale=0.02, shift=1), normals(rng, 2 * D, scale=0.02)
    frames = [rng.integers(0, 256, (fh, fw, 3), dtype=np.uint8) for _ in range(views)]

    # device path
    proj = rt.prepare_linear_oihw_f32(588, D, wt, b)
    pos = rt.pos_embed_bicubic_f32(rt.upload_f32(grid_tab), 37, D, gh, gw)
    tokens = rt.alloc_f32(views * n * D)
    resized = []
    for v, f in enumerate(frames):
        r = rt.preprocess_resize_u8(rt.upload_u8(f), fh, fw, 56, 14)
        resized.append(r)
        rt.patch_embed_u8(r, oh, ow, 14, MEAN, STD, proj, rt.upload_f32(cls), rt.upload_f32(reg),
                          1, pos, tokens.view(v * n * D, n * D))
    ws = rt.block_workspace(views * n, D, M)
    feats = [rt.alloc_f32(views * n_patch * 2 * D) for _ in outs]
    cams = [rt.alloc_f32(views * 2 * D) for _ in outs]
    rt.backbone_forward_f32(vh.VitConfig(**cfg), [d.struct for d in devs], tokens, gh, gw, views,
                            rt.upload_f32(cam), rt.upload_f32(vg), rt.upload_f32(vb), True, outs,
                            feats, cams, ws, rt.alloc_f32(views * n * D))
    hg_d, hb_d = rt.upload_f32(hg), rt.upload_f32(hb)
    chw = []
    for f in feats:
        per_view = []
        for v in range(views):
            out = rt.alloc_f32(n_patch * 2 * D)
            rt.token_to_chw_f32(f.view(v * n_patch * 2 * D, n_patch * 2 * D), n_patch, 2 * D,
                                hg_d, hb_d, 1e-5, out)
            per_view.append(out.numpy().reshape(2 * D, n_patch))
        chw.append(np.stack(per_view))

    # oracle path and float64 twin
    o_frames = [oracle.preprocess_resize_u8(f, 56, 14) for f in frames]
    for r, want in zip(resized, o_frames):
        assert np.array_equal(rt.download_u8(r).reshape(want.shape), want)
    o_pos = oracle.pos_embed_bicubic(grid_tab, 37, D, gh, gw)
    assert np.array_equal(pos.numpy().reshape(o_pos.shape), o_pos)
    o_tok = np.concatenate([oracle.patch_embed_u8(f, 14, MEAN, STD, wt, b, cls, reg, o_pos)
                            for f in o_frames])
    t64 = np.concatenate([_patch_embed_f64(f, wt, b, cls, reg, o_pos) for f in o_frames])
    _, o_caps = oracle.backbone_forward(o_tok, params, cfg, gh, gw, views, cam, vg, vb, True,
                                        outs)
    _, caps64 = backbone_f64(t64, params, cfg, gh, gw, views, cam, vg, vb, True, outs)
    for i, o in enumerate(outs):
        o_chw = np.stack([oracle.token_to_chw(o_caps[i][0][v], n_patch, 2 * D, hg, hb, 1e-5)
                          for v in range(views)])
        chw64 = np.stack([_ln64(caps64[i][0][v], hg, hb, 1e-5).T for v in range(views)])
        assert_envelope(chw[i], o_chw, chw64, f"head input of out layer {o}")
        assert_envelope(cams[i].numpy(), o_caps[i][1], caps64[i][1], f"camera of out layer {o}")
