"""GPU parity of every 2D RoPE convention (VK_ROPE_* flags) against the oracle.

The rotation's pairing (rotate-half (j, j+16) or interleaved (2i, 2i+1)
inside each 32-wide half) and its frequency exponent (2j/32 or 2j/64) are
fixed only inside the reference's absent kernel crate, so the library takes
them as a parameter (vit_block.rs:343-357, 543-557, 911-948).  Each
convention is compared with the oracle's restatement of the same
convention:

  * the reference-signature form (explicit positions, f32 / i32 / i64) at
    866 tokens, 12 heads, the 24 x 36 grid, with one and two special tokens;
  * the rotation alone (rope2d) bit for bit, and beyond the cos/sin table;
  * the grid form over 12 views x 866 tokens, local (views-outer) and global
    (one flattened sequence) layers;
  * the QKV projection's fused epilogue, bit-identical to the projection
    followed by the separate pass;
  * the block's fused-op sequence with the convention in vk_vit_config.

Bars: rtol 1e-5 / atol 1e-6 where a LayerNorm reduces in another order,
bit-exact for the rotation alone.
"""
import numpy as np
import pytest

import oracle
from conftest import F32_ATOL, F32_RTOL, assert_parity

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")

MODES = [pytest.param(m, id=f"mode{m}") for m in oracle.ROPE_MODES]


def normals(rng, *shape, scale=1.0, shift=0.0):
    return (shift + scale * rng.standard_normal(shape)).astype(np.float32)


def qk_params(rng):
    return [normals(rng, 64, scale=0.02, shift=1.0 if i % 2 == 0 else 0.0) for i in range(4)]


def upload_positions(rt, pos, dtype):
    if dtype == "f32":
        return rt.upload_f32(pos.astype(np.float32))
    if dtype == "i32":
        return rt.upload_i32(pos.astype(np.int32))
    return rt.upload_i64(pos.astype(np.int64))


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("n_special", [1, 2])
@pytest.mark.parametrize("pos_dtype", ["f32", "i32", "i64"])
def test_reference_form_each_convention(rt, rng, mode, n_special, pos_dtype):
    heads, gh, gw = 12, 24, 36
    n = n_special + gh * gw
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    qg, qb, kg, kb = qk_params(rng)
    pos = oracle.rope_positions(n_special, gh, gw, 1, False)
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_mode_f32(tq, tk, *[rt.upload_f32(a) for a in (qg, qb, kg, kb)],
                             upload_positions(rt, pos, pos_dtype), heads, n, 100.0, 1e-5, mode)
    rq, rk = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, n, mode=mode)
    assert_parity(tq.numpy(), rq, F32_ATOL, F32_RTOL, f"q mode {mode}")
    assert_parity(tk.numpy(), rk, F32_ATOL, F32_RTOL, f"k mode {mode}")


@pytest.mark.parametrize("mode", MODES)
def test_default_entry_is_mode_zero(rt, rng, mode):
    # the reference-signature entry point equals the mode entry with mode 0,
    # and differs from every other convention
    heads, n = 12, 866
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    pos = rt.upload_f32(oracle.rope_positions(2, 24, 36, 1, False))
    a = [rt.upload_f32(q), rt.upload_f32(k)]
    b = [rt.upload_f32(q), rt.upload_f32(k)]
    rt.qk_norm_rope_f32_da3_base(*a, None, None, None, None, pos, heads, n)
    rt.qk_norm_rope_mode_f32(*b, None, None, None, None, pos, heads, n, rope_mode=mode)
    same = np.array_equal(a[0].numpy(), b[0].numpy()) and np.array_equal(a[1].numpy(),
                                                                         b[1].numpy())
    assert same == (mode == 0)


@pytest.mark.parametrize("mode", MODES)
def test_rope2d_alone_bit_exact(rt, rng, mode):
    # one tensor, no LayerNorm: no reduction, the oracle's bits exactly
    heads, n_special, gh, gw = 12, 2, 24, 36
    n = n_special + gh * gw
    x = normals(rng, heads, n, 64)
    pos = oracle.rope_positions(n_special, gh, gw, 1, False).astype(np.int64)
    t = rt.upload_f32(x)
    rt.rope2d_f32(t, rt.upload_i64(pos), heads, n, rope_mode=mode)
    assert np.array_equal(t.numpy().reshape(heads, n, 64),
                          oracle.rope2d(x, heads, n, 64, pos, 100.0, mode))


@pytest.mark.parametrize("mode", MODES)
def test_rope2d_beyond_the_table(rt, rng, mode):
    heads, n = 2, 7
    x = normals(rng, heads, n, 64)
    pos = np.array([[0, 0], [1, 1], [1023, 5], [1024, 1100], [2000, 7], [5, 4096], [-3, 2]],
                   np.int64)
    t = rt.upload_f32(x)
    rt.rope2d_f32(t, rt.upload_i32(pos), heads, n, rope_mode=mode)
    ref = oracle.rope2d(x, heads, n, 64, pos, 100.0, mode)
    assert_parity(t.numpy(), ref, F32_ATOL, F32_RTOL, f"rope2d large positions mode {mode}")


@pytest.mark.parametrize("mode", [0, 1])
def test_rope2d_positions_beyond_32_bits(rt, rng, mode):
    """i64 coordinates past the int32 range, and f32 ones past it or NaN,
    rotate by (float)p * inv_freq as the CPU kernel converts its i64
    positions (no narrowing to 32 bits on the way): 2^32 + 5 is the angle
    of (float)(2^32 + 5), not of 5."""
    heads, n = 2, 6
    x = normals(rng, heads, n, 64)
    pos = np.array([[2 ** 32 + 5, 7], [3, -(2 ** 33) + 1], [2 ** 40 + 3, 2 ** 31],
                    [2 ** 31 - 1, -(2 ** 31) - 1], [5, 2 ** 32 + 5], [-(2 ** 62), 1]], np.int64)
    t = rt.upload_f32(x)
    rt.rope2d_f32(t, rt.upload_i64(pos), heads, n, rope_mode=mode)
    ref = oracle.rope2d(x, heads, n, 64, pos, 100.0, mode)
    assert_parity(t.numpy(), ref, F32_ATOL, F32_RTOL, f"rope2d i64 positions mode {mode}")
    # the same rows with positions narrowed to 32 bits rotate differently
    narrowed = oracle.rope2d(x, heads, n, 64, pos.astype(np.int32).astype(np.int64), 100.0, mode)
    assert not np.allclose(t.numpy().reshape(-1), narrowed.reshape(-1), rtol=1e-3, atol=1e-3)
    # f32 positions: truncated toward zero like `value as i64`, NaN as 0
    fpos = np.array([[3.0e9, 7.9], [-2.5e10, 1.0], [np.nan, 2.0], [1e12, -0.5], [4.5, 6.0],
                     [0.0, np.nan]], np.float32)
    ipos = np.where(np.isnan(fpos), 0, np.trunc(fpos.astype(np.float64))).astype(np.int64)
    t = rt.upload_f32(x)
    rt.rope2d_f32(t, rt.upload_f32(fpos), heads, n, rope_mode=mode)
    ref = oracle.rope2d(x, heads, n, 64, ipos, 100.0, mode)
    assert_parity(t.numpy(), ref, F32_ATOL, F32_RTOL, f"rope2d f32 positions mode {mode}")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("glob", [False, True], ids=["local", "global"])
def test_grid_form_12_views(rt, rng, mode, glob):
    heads, n_special, gh, gw, views = 12, 2, 24, 36, 12
    tpv = n_special + gh * gw
    rows = tpv * views
    q, k = normals(rng, rows * heads * 64), normals(rng, rows * heads * 64)
    qg, qb, kg, kb = qk_params(rng)
    layout = vh.VK_QK_HEADS_OUTER if glob else vh.VK_QK_VIEWS_OUTER
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_grid_f32(tq, tk, *[rt.upload_f32(a) for a in (qg, qb, kg, kb)], heads, 64,
                             n_special, gh, gw, views, glob, layout, rope_mode=mode)
    pos = oracle.rope_positions(n_special, gh, gw, views, glob)
    if glob:
        rq, rk = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, rows, mode=mode)
    else:
        rq = q.reshape(views, heads, tpv, 64).copy()
        rk = k.reshape(views, heads, tpv, 64).copy()
        for v in range(views):
            rq[v], rk[v] = [a.reshape(heads, tpv, 64) for a in oracle.qk_norm_rope(
                rq[v], rk[v], qg, qb, kg, kb, pos[v * tpv:(v + 1) * tpv], heads, tpv,
                mode=mode)]
    assert_parity(tq.numpy(), rq, F32_ATOL, F32_RTOL, f"q 12 views mode {mode}")
    assert_parity(tk.numpy(), rk, F32_ATOL, F32_RTOL, f"k 12 views mode {mode}")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("views,glob", [(1, False), (12, True)], ids=["1view", "12views-global"])
def test_qkv_epilogue_equals_separate_pass(rt, rng, mode, views, glob):
    D, H, n_special, gh, gw = 768, 12, 2, 24, 36
    rows = (n_special + gh * gw) * views
    x = rt.upload_f32(normals(rng, rows, D))
    lin = rt.prepare_linear_f32(D, 3 * D, normals(rng, D, 3 * D, scale=0.02),
                                normals(rng, 3 * D, scale=0.02))
    params = [rt.upload_f32(a) for a in qk_params(rng)]
    fused = [rt.alloc_f32(rows * D) for _ in range(3)]
    lin.run_qkv_hnd_norm_rope(x, rows, H, *fused, *params, n_special, gh, gw, views, glob,
                              rope_mode=mode)
    sep = [rt.alloc_f32(rows * D) for _ in range(3)]
    lin.run_qkv_hnd(x, rows, H, *sep)
    rt.qk_norm_rope_grid_f32(sep[0], sep[1], *params, H, 64, n_special, gh, gw, views, glob,
                             vh.VK_QK_HEADS_OUTER, rope_mode=mode)
    for name, a, b in zip("qkv", fused, sep):
        assert np.array_equal(a.numpy(), b.numpy()), f"{name} differs (mode {mode})"


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("layer", [2, 5], ids=["local", "global"])
def test_block_fused_ops_12_views(rt, rng, mode, layer):
    D, H, M, nreg, gh, gw, views = 768, 12, 3072, 1, 24, 36, 12
    tpv = 2 + gh * gw
    rows = tpv * views
    cfg = dict(embed_dim=D, num_heads=H, head_dim=64, mlp_hidden=M, num_register=nreg,
               ln_eps=1e-6, qk_norm_eps=1e-5, rope_freq=100.0, rope_start=0, qknorm_start=0,
               alt_start=4, rope_mode=mode)
    host = {"norm1_gamma": normals(rng, D, scale=0.02, shift=1),
            "norm1_beta": normals(rng, D, scale=0.02),
            "qnorm_gamma": normals(rng, 64, scale=0.02, shift=1),
            "qnorm_beta": normals(rng, 64, scale=0.02),
            "knorm_gamma": normals(rng, 64, scale=0.02, shift=1),
            "knorm_beta": normals(rng, 64, scale=0.02),
            "ls1": rng.uniform(0, 0.1, D).astype(np.float32),
            "norm2_gamma": normals(rng, D, scale=0.02, shift=1),
            "norm2_beta": normals(rng, D, scale=0.02),
            "ls2": rng.uniform(0, 0.1, D).astype(np.float32)}
    dev = {k_: rt.upload_f32(v) for k_, v in host.items()}
    tokens, q, k = normals(rng, rows, D), normals(rng, rows * D), normals(rng, rows * D)
    attn, mlp, hidden = normals(rng, rows, D), normals(rng, rows, D), normals(rng, rows, M)
    act = {"tokens": rt.upload_f32(tokens), "ln1": rt.alloc_f32(rows * D),
           "q": rt.upload_f32(q), "k": rt.upload_f32(k), "attn_proj": rt.upload_f32(attn),
           "ln2": rt.alloc_f32(rows * D), "hidden": rt.upload_f32(hidden),
           "mlp_out": rt.upload_f32(mlp)}
    rt.vit_block_fused_ops(vh.VitConfig(**cfg), layer, vh.layer_struct(**dev), None,
                           vh.activations_struct(**act), gh, gw, views, None,
                           vh.VK_BLOCK_FUSE_LS_LN)
    ref = oracle.block_fused_ops(tokens, q, k, attn, hidden, mlp, host, cfg, layer, gh, gw,
                                 views)
    for name in ("q", "k", "tokens", "ln1", "ln2"):
        assert_parity(act[name].numpy(), ref[name], F32_ATOL, F32_RTOL,
                      f"{name} layer {layer} mode {mode}")


def test_rejects_unknown_convention_and_position_dtype(rt, rng):
    heads, n = 2, 5
    q, k = rt.upload_f32(normals(rng, heads * n * 64)), rt.upload_f32(normals(rng, heads * n * 64))
    pos = rt.upload_f32(np.zeros((n, 2), np.float32))
    with pytest.raises(vh.VestraError, match="convention"):
        rt.qk_norm_rope_mode_f32(q, k, None, None, None, None, pos, heads, n, rope_mode=4)
    with pytest.raises(vh.VestraError, match="convention"):
        rt.qk_norm_rope_grid_f32(q, k, None, None, None, None, heads, 64, 1, 2, 2, 1, False,
                                 vh.VK_QK_HEADS_OUTER, rope_mode=8)
    with pytest.raises(vh.VestraError, match="positions"):
        rt.qk_norm_rope_mode_f32(q, k, None, None, None, None,
                                 rt.upload_u8(np.zeros(2 * n, np.uint8)), heads, n)
    with pytest.raises(vh.VestraError, match="f32"):
        # the reference-signature entry keeps the CUDA runtime's f32 positions
        rt.qk_norm_rope_f32_da3_base(q, k, None, None, None, None,
                                     rt.upload_i32(np.zeros((n, 2), np.int32)), heads, n)
