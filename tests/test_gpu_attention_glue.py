"""GPU parity of the attention block's layout glue and the head-major linears.

The split of the QKV output into head-major Q, K, V and the attention output's
way back to token-major rows are pure permutations: bit-exact against the
oracle (vit_block.rs:818-833).  The fused forms (the QKV projection storing
Q, K, V head-major; the output projection reading the head-major input) must
give the bits of the projection plus the separate permutation, and match the
oracle within the dot-product bound of the projection.
"""
import numpy as np
import pytest

import oracle
from test_gpu_patch_block import assert_dot_parity, normals

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


@pytest.mark.parametrize("rows,heads,hd", [(866, 12, 64), (5, 3, 8), (3458, 16, 64)])
def test_split_qkv_hnd_bit_exact(rt, rng, rows, heads, hd):
    qkv = normals(rng, rows, 3 * heads * hd)
    q, k, v = rt.split_qkv_hnd_f32(rt.upload_f32(qkv), rows, heads, hd)
    rq, rk, rv = oracle.split_qkv_hnd(qkv, rows, heads, hd)
    assert np.array_equal(q.numpy(), rq.reshape(-1))
    assert np.array_equal(k.numpy(), rk.reshape(-1))
    assert np.array_equal(v.numpy(), rv.reshape(-1))


@pytest.mark.parametrize("rows,heads,hd", [(866, 12, 64), (7, 2, 12)])
def test_hnd_to_token_bit_exact_and_round_trip(rt, rng, rows, heads, hd):
    hnd = normals(rng, heads, rows, hd)
    tok = rt.hnd_to_token_f32(rt.upload_f32(hnd), rows, heads, hd).numpy()
    assert np.array_equal(tok, oracle.hnd_to_token(hnd, rows, heads, hd).reshape(-1))
    qkv = rt.upload_f32(np.concatenate([tok.reshape(rows, -1)] * 3, axis=1))
    q, k, v = (rt.alloc_f32(rows * heads * hd) for _ in range(3))
    rt.split_qkv_hnd_into_f32(qkv, rows, heads, hd, q, k, v)
    assert np.array_equal(q.numpy(), hnd.reshape(-1)) and np.array_equal(v.numpy(), hnd.reshape(-1))


def test_layout_glue_edges_and_errors(rt, rng):
    empty = rt.alloc_f32(0)
    rt.split_qkv_hnd_into_f32(empty, 0, 12, 64, rt.alloc_f32(0), rt.alloc_f32(0), rt.alloc_f32(0))
    rt.hnd_to_token_into_f32(empty, 0, 12, 64, rt.alloc_f32(0))
    with pytest.raises(vh.UnsupportedShape):
        rt.hnd_to_token_f32(rt.alloc_f32(2 * 3 * 6), 3, 2, 6)      # head_dim not a multiple of 4
    x = rt.alloc_f32(4 * 3 * 2 * 8)
    with pytest.raises(vh.VestraError):
        rt.split_qkv_hnd_f32(x, 5, 2, 8)                             # size mismatch
    y = rt.alloc_f32(4 * 2 * 8)
    with pytest.raises(vh.VestraError):
        rt.hnd_to_token_into_f32(y, 4, 2, 8, y)                      # overlap


@pytest.mark.parametrize("rows,embed,heads", [(97, 768, 12), (866, 768, 12), (130, 1024, 16)])
def test_qkv_hnd_projection_is_linear_then_split(rt, rng, rows, embed, heads):
    xh = normals(rng, rows, embed)
    w, b = normals(rng, embed, 3 * embed, scale=0.02), normals(rng, 3 * embed, scale=0.02)
    x = rt.upload_f32(xh)
    lin = rt.prepare_linear_f32(embed, 3 * embed, w, b)
    q, k, v = (rt.alloc_f32(rows * embed) for _ in range(3))
    lin.run_qkv_hnd(x, rows, heads, q, k, v)
    plain = rt.alloc_f32(rows * 3 * embed)
    lin.run_into(x, rows, plain)
    pq, pk, pv = rt.split_qkv_hnd_f32(plain, rows, heads, 64)
    for got, want in ((q, pq), (k, pk), (v, pv)):
        assert np.array_equal(got.numpy(), want.numpy())
    if rows <= 130:
        ref = oracle.split_qkv_hnd(oracle.linear(xh, w, b), rows, heads, 64)
        scale = oracle.split_qkv_hnd(
            (np.abs(xh).astype(np.float64) @ np.abs(w).astype(np.float64)).astype(np.float32),
            rows, heads, 64)
        for got, r, sc in zip((q, k, v), ref, scale):
            assert_dot_parity(got.numpy(), r, sc, embed, f"qkv_hnd {rows}x{embed}")


@pytest.mark.parametrize("rows,heads,with_ls", [(97, 12, True), (866, 12, True), (130, 16, False)])
def test_hnd_projection_is_token_then_linear(rt, rng, rows, heads, with_ls):
    embed = heads * 64
    hnd_h = normals(rng, heads, rows, 64)
    w, b = normals(rng, embed, embed, scale=0.02), normals(rng, embed, scale=0.02)
    ls = rng.uniform(0, 0.1, embed).astype(np.float32) if with_ls else None
    res = normals(rng, rows, embed)
    hnd = rt.upload_f32(hnd_h)
    lin = rt.prepare_linear_f32(embed, embed, w, b, ls)
    tok = rt.hnd_to_token_f32(hnd, rows, heads, 64)
    # store form
    got, want = rt.alloc_f32(rows * embed), rt.alloc_f32(rows * embed)
    lin.run_hnd_into(hnd, rows, heads, got)
    lin.run_into(tok, rows, want)
    assert np.array_equal(got.numpy(), want.numpy())
    # residual form
    fused, plain = rt.upload_f32(res), rt.upload_f32(res)
    lin.run_hnd_residual(hnd, rows, heads, fused)
    lin.run_residual(tok, rows, plain)
    out = fused.numpy()
    assert np.array_equal(out, plain.numpy())
    if rows <= 130:
        xt = oracle.hnd_to_token(hnd_h, rows, heads, 64)
        t = oracle.linear(xt, w, b)
        if with_ls:
            t = oracle.layerscale(t, ls)
        scale = np.abs(xt).astype(np.float64) @ np.abs(w).astype(np.float64)
        if with_ls:
            scale = scale * ls
        assert_dot_parity(out, oracle.add(res, t), scale, embed, f"hnd_residual {rows}x{embed}")


def test_head_major_linears_reject_unqualified_shapes(rt, rng):
    x = rt.upload_f32(normals(rng, 4, 96))
    lin = rt.prepare_linear_f32(96, 288, normals(rng, 96, 288), normals(rng, 288))
    q, k, v = (rt.alloc_f32(4 * 96) for _ in range(3))
    with pytest.raises(vh.UnsupportedShape):
        lin.run_qkv_hnd(x, 4, 3, q, k, v, head_dim=32)             # head_dim 32: not qualified
    wrong = rt.prepare_linear_f32(96, 96, normals(rng, 96, 96), normals(rng, 96))
    with pytest.raises(vh.VestraError):
        wrong.run_qkv_hnd(x, 4, 1, q, k, v)                         # out_features != 3*heads*64
    with_ls = rt.prepare_linear_f32(64, 192, normals(rng, 64, 192), normals(rng, 192),
                                    rng.uniform(0, 0.1, 192).astype(np.float32))
    x64 = rt.upload_f32(normals(rng, 4, 64))
    q1, k1, v1 = (rt.alloc_f32(4 * 64) for _ in range(3))
    with pytest.raises(vh.VestraError):
        with_ls.run_qkv_hnd(x64, 4, 1, q1, k1, v1)                  # QKV carries no LayerScale


@pytest.mark.parametrize("embed,heads,gh,gw,views,glob,f16,norm", [
    (768, 12, 24, 36, 1, False, False, True),     # one 504x336 image: 64 x 64 tiles
    (768, 12, 24, 36, 1, False, True, True),      # the same, f16 parameters
    (768, 12, 24, 36, 1, True, False, False),     # the same, RoPE only, global layer
    (768, 12, 24, 36, 12, True, False, True),     # 12-view global layer
    (768, 12, 24, 36, 12, False, False, True),    # 12-view local layer
    (1024, 16, 4, 8, 2, False, True, True),       # ViT-L, f16 parameters
    (768, 12, 3, 5, 3, True, False, False),       # RoPE only
])
def test_qkv_norm_rope_epilogue_is_the_separate_pass(rt, rng, embed, heads, gh, gw, views, glob,
                                                     f16, norm):
    """QKV + Q/K-norm + RoPE in one kernel gives the bits of the QKV projection
    followed by the Q/K kernel on the head-major layout."""
    rows = views * (2 + gh * gw)
    x = rt.upload_f32(normals(rng, rows, embed))
    lin = rt.prepare_linear_f32(embed, 3 * embed, normals(rng, embed, 3 * embed, scale=0.02),
                                normals(rng, 3 * embed, scale=0.02))
    par = [None] * 4
    if norm:
        host = [normals(rng, 64, scale=0.02, shift=s) for s in (1, 0, 1, 0)]
        par = [rt.upload_f16(h.astype(np.float16)) if f16 else rt.upload_f32(h) for h in host]
    fused = [rt.alloc_f32(rows * embed) for _ in range(3)]
    lin.run_qkv_hnd_norm_rope(x, rows, heads, *fused, *par, 2, gh, gw, views, glob)
    sep = [rt.alloc_f32(rows * embed) for _ in range(3)]
    lin.run_qkv_hnd(x, rows, heads, *sep)
    rt.qk_norm_rope_grid_f32(sep[0], sep[1], *par, heads, 64, 2, gh, gw, views, glob,
                             vh.VK_QK_HEADS_OUTER, 100.0, 1e-5)
    for name, a, b in zip("qkv", fused, sep):
        assert np.array_equal(a.numpy(), b.numpy()), f"{name} differs from the separate pass"
