"""GPU parity of the fused per-token operations against the oracle.

Every test calls the HIP kernels through the C ABI (vestra_hip ->
libvestra_hip.so) on seeded inputs and compares with the scalar CPU oracle:
  * bit-exact where the operation order is the same (LayerScale+residual,
    residual add, LayerScale, RoPE positions, bicubic table, patchify,
    token assembly, RoPE of already-normalised rows);
  * |got - ref| <= atol + rtol*|ref| with rtol 1e-5 / atol 1e-6 for F32
    where the GPU reduces in a different order (LayerNorm mean/variance) or
    uses the device exp / erf, and rtol 2e-3 / atol 2e-3 for F16-stored
    parameters with F32 accumulation.
"""
import numpy as np
import pytest

import oracle
from conftest import F32_ATOL, F32_RTOL, W16_ATOL, W16_RTOL, assert_parity, record_margin

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


def normals(rng, *shape, scale=1.0, shift=0.0):
    return (shift + scale * rng.standard_normal(shape)).astype(np.float32)


# ---------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("rows,cols", [(5, 8), (1, 768), (866, 768), (865, 768),
                                       (10392, 768), (3458, 1024), (37, 64), (3, 1300)])
def test_layernorm_matches_oracle(rt, rng, rows, cols):
    x = normals(rng, rows, cols)
    g = normals(rng, cols, scale=0.02, shift=1.0)
    b = normals(rng, cols, scale=0.02)
    out = rt.layernorm_f32_cpu_order(rt.upload_f32(x), rt.upload_f32(g), rt.upload_f32(b),
                                     rows, cols, 1e-6).numpy()
    ref = oracle.layernorm(x, g, b, 1e-6)
    assert_parity(out, ref, F32_ATOL, F32_RTOL, f"ln {rows}x{cols}")
    record_margin("layernorm (tree order)", out, ref, atol=F32_ATOL, rtol=F32_RTOL,
                  label=f"{rows}x{cols}")


def test_layernorm_in_place_and_f16_params(rt, rng):
    rows, cols = 3458, 1024
    x = normals(rng, rows, cols)
    g = normals(rng, cols, scale=0.02, shift=1.0).astype(np.float16)
    b = normals(rng, cols, scale=0.02).astype(np.float16)
    t = rt.upload_f32(x)
    rt.layernorm_into_f32(t, rt.upload_f16(g), rt.upload_f16(b), rows, cols, 1e-6, t)
    ref = oracle.layernorm(x, g, b, 1e-6)
    assert_parity(t.numpy(), ref, F32_ATOL, F32_RTOL, "ln in place f16 params")
    assert_parity(t.numpy(), ref, W16_ATOL, W16_RTOL, "ln f16 bar")


def test_layernorm_rejects_bad_shapes(rt, rng):
    x = rt.upload_f32(normals(rng, 4, 6))
    g = rt.upload_f32(np.ones(6, np.float32))
    with pytest.raises(vh.UnsupportedShape):
        rt.layernorm_f32_cpu_order(x, g, g, 4, 6, 1e-6)   # cols % 4 != 0
    with pytest.raises(vh.VestraError) as e:
        rt.layernorm_f32_cpu_order(x, g, g, 5, 6, 1e-6)   # size mismatch
    assert e.value.code == vh.VK_ERR_INVALID and "rows*cols" in e.value.message


def test_layernorm_empty_rows(rt):
    g = rt.upload_f32(np.ones(8, np.float32))
    out = rt.layernorm_f32_cpu_order(rt.alloc_f32(0), g, g, 0, 8, 1e-6)
    assert len(out) == 0


# ---------------------------------------------------------------- GELU
@pytest.mark.parametrize("n", [866 * 3072, 1, 2, 3, 5, 4099, 3458 * 4096])
def test_gelu_matches_oracle(rt, rng, n):
    x = normals(rng, n)
    if n > 8:
        x[:8] = [0.0, -0.0, 10.0, -10.0, 1e-30, -5.5, 30.0, -30.0]
    t = rt.upload_f32(x)
    rt.gelu_f32_in_place(t)
    assert_parity(t.numpy(), oracle.gelu(x), F32_ATOL, F32_RTOL, f"gelu n={n}")
    record_margin("gelu (A&S erf, v_rcp/v_exp)", t.numpy(), oracle.gelu(x), atol=F32_ATOL,
                  rtol=F32_RTOL, label=f"n={n}")


def test_gelu_erf_variant_matches_oracle(rt, rng):
    x = normals(rng, 866 * 3072, scale=2.0)
    t = rt.upload_f32(x)
    rt.gelu_erf_f32_in_place(t)
    assert_parity(t.numpy(), oracle.gelu_erff(x), F32_ATOL, F32_RTOL, "gelu erff")


def test_gelu_empty(rt):
    t = rt.alloc_f32(0)
    rt.gelu_f32_in_place(t)


# ---------------------------------------------------------------- LayerScale / residual
@pytest.mark.parametrize("rows,cols", [(866, 768), (10392, 768), (3458, 1024), (3, 4), (7, 12)])
def test_layerscale_residual_bit_exact(rt, rng, rows, cols):
    x = normals(rng, rows, cols)
    y = normals(rng, rows, cols)
    g = rng.uniform(0, 0.1, cols).astype(np.float32)
    t = rt.upload_f32(x)
    rt.layerscale_residual_f32(t, rt.upload_f32(y), rt.upload_f32(g), rows, cols)
    assert np.array_equal(t.numpy().reshape(rows, cols), oracle.layerscale_residual(x, y, g))


def test_layerscale_residual_f16_gamma_and_absent_gamma(rt, rng):
    rows, cols = 3458, 1024
    x, y = normals(rng, rows, cols), normals(rng, rows, cols)
    g16 = rng.uniform(0, 0.1, cols).astype(np.float16)
    t = rt.upload_f32(x)
    rt.layerscale_residual_f32(t, rt.upload_f32(y), rt.upload_f16(g16), rows, cols)
    assert np.array_equal(t.numpy().reshape(rows, cols), oracle.layerscale_residual(x, y, g16))
    t2 = rt.upload_f32(x)
    rt.layerscale_residual_f32(t2, rt.upload_f32(y), None, rows, cols)
    assert np.array_equal(t2.numpy().reshape(rows, cols), oracle.add(x, y))


def test_add_and_layerscale_bit_exact(rt, rng):
    x, y = normals(rng, 1001), normals(rng, 1001)   # odd length: scalar tail
    t = rt.upload_f32(x)
    rt.add_f32_in_place(t, rt.upload_f32(y))
    assert np.array_equal(t.numpy(), oracle.add(x, y))
    x2 = normals(rng, 6, 8)
    g = normals(rng, 8)
    t2 = rt.upload_f32(x2)
    rt.layerscale_f32_in_place(t2, rt.upload_f32(g), 6, 8)
    assert np.array_equal(t2.numpy().reshape(6, 8), oracle.layerscale(x2, g))


def test_add_rejects_aliasing_and_mismatch(rt, rng):
    t = rt.upload_f32(normals(rng, 16))
    with pytest.raises(vh.VestraError):
        rt.add_f32_in_place(t, t)
    with pytest.raises(vh.VestraError):
        rt.add_f32_in_place(t, rt.upload_f32(normals(rng, 15)))


@pytest.mark.parametrize("with_ls", [True, False])
def test_fused_layerscale_residual_layernorm(rt, rng, with_ls):
    rows, cols = 10392, 768
    x, y = normals(rng, rows, cols), normals(rng, rows, cols)
    ls = rng.uniform(0, 0.1, cols).astype(np.float32)
    g = normals(rng, cols, scale=0.02, shift=1.0)
    b = normals(rng, cols, scale=0.02)
    tx = rt.upload_f32(x)
    out = rt.alloc_f32(rows * cols)
    rt.layerscale_residual_layernorm_f32(tx, rt.upload_f32(y), rt.upload_f32(ls) if with_ls else None,
                                         rt.upload_f32(g), rt.upload_f32(b), rows, cols, 1e-6, out)
    x_ref = oracle.layerscale_residual(x, y, ls if with_ls else None)
    assert np.array_equal(tx.numpy().reshape(rows, cols), x_ref)
    assert_parity(out.numpy(), oracle.layernorm(x_ref, g, b, 1e-6), F32_ATOL, F32_RTOL,
                  "ls+res+ln")


# Row counts at the edges of the row kernels' launch regimes, from the CU count
# as the launchers see it: stores are serialised from 8 rows per CU, and a
# wave takes two rows when the rows exceed 24 waves per CU but not twice that
# (an odd count leaves the last wave one row).
ROW_REGIMES = {
    "below_serialised": lambda cu: 8 * cu - 1,
    "first_serialised": lambda cu: 8 * cu,
    "two_per_wave_first": lambda cu: 24 * cu + 1,
    "two_per_wave_odd_last": lambda cu: 48 * cu - 1,
    "one_per_wave_again": lambda cu: 48 * cu + 1,
}


@pytest.mark.parametrize("regime", sorted(ROW_REGIMES))
def test_layernorm_row_regimes(rt, rng, regime):
    rows, cols = ROW_REGIMES[regime](rt.cu_count()), 768
    x = normals(rng, rows, cols, shift=0.5)
    g = normals(rng, cols, scale=0.02, shift=1.0)
    b = normals(rng, cols, scale=0.02)
    out = rt.layernorm_f32_cpu_order(rt.upload_f32(x), rt.upload_f32(g), rt.upload_f32(b),
                                     rows, cols, 1e-6).numpy()
    assert_parity(out, oracle.layernorm(x, g, b, 1e-6), F32_ATOL, F32_RTOL,
                  f"ln {regime} {rows}x{cols}")


def test_layernorm_two_per_wave_ragged_cols(rt, rng):
    """640 columns (not a multiple of 256) in the two-rows-per-wave regime."""
    rows, cols = 48 * rt.cu_count() - 1, 640
    x = normals(rng, rows, cols)
    g = normals(rng, cols, scale=0.02, shift=1.0)
    b = normals(rng, cols, scale=0.02)
    out = rt.layernorm_f32_cpu_order(rt.upload_f32(x), rt.upload_f32(g), rt.upload_f32(b),
                                     rows, cols, 1e-6).numpy()
    assert_parity(out, oracle.layernorm(x, g, b, 1e-6), F32_ATOL, F32_RTOL,
                  f"ln ragged {rows}x{cols}")


@pytest.mark.parametrize("regime", sorted(ROW_REGIMES))
def test_fused_layerscale_residual_layernorm_row_regimes(rt, rng, regime):
    """x bit-exact; the LayerNorm output equals the separate LayerNorm of the
    updated x bit for bit (both reduce a row in the same order)."""
    rows, cols = ROW_REGIMES[regime](rt.cu_count()), 768
    x, y = normals(rng, rows, cols), normals(rng, rows, cols)
    ls = rng.uniform(0, 0.1, cols).astype(np.float32)
    g = normals(rng, cols, scale=0.02, shift=1.0)
    b = normals(rng, cols, scale=0.02)
    tx, tg, tb = rt.upload_f32(x), rt.upload_f32(g), rt.upload_f32(b)
    out = rt.alloc_f32(rows * cols)
    rt.layerscale_residual_layernorm_f32(tx, rt.upload_f32(y), rt.upload_f32(ls), tg, tb,
                                         rows, cols, 1e-6, out)
    x_ref = oracle.layerscale_residual(x, y, ls)
    assert np.array_equal(tx.numpy().reshape(rows, cols), x_ref)
    fused = out.numpy()
    assert_parity(fused, oracle.layernorm(x_ref, g, b, 1e-6), F32_ATOL, F32_RTOL,
                  f"ls+res+ln {regime} {rows}x{cols}")
    alone = rt.layernorm_f32_cpu_order(tx, tg, tb, rows, cols, 1e-6).numpy()
    assert np.array_equal(fused, alone)


# ---------------------------------------------------------------- Q/K norm + RoPE
def qk_params(rng, dtype=np.float32):
    return [normals(rng, 64, scale=0.02, shift=1.0 if i % 2 == 0 else 0.0).astype(dtype)
            for i in range(4)]


@pytest.mark.parametrize("n_special,gh,gw,glob", [(2, 24, 36, False), (1, 24, 36, False),
                                                  (2, 24, 36, True), (1, 2, 2, False),
                                                  (2, 48, 72, False)])
def test_qk_norm_rope_reference_form(rt, rng, n_special, gh, gw, glob):
    heads = 12
    n = n_special + gh * gw
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    qg, qb, kg, kb = qk_params(rng)
    pos = oracle.rope_positions(n_special, gh, gw, 1, glob)
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_f32_da3_base(tq, tk, rt.upload_f32(qg), rt.upload_f32(qb),
                                 rt.upload_f32(kg), rt.upload_f32(kb), rt.upload_f32(pos),
                                 heads, n, 100.0, 1e-5)
    rq, rk = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, n)
    assert_parity(tq.numpy(), rq, F32_ATOL, F32_RTOL, "q")
    assert_parity(tk.numpy(), rk, F32_ATOL, F32_RTOL, "k")
    for name, got, ref in (("q", tq.numpy(), rq), ("k", tk.numpy(), rk)):
        record_margin("qk_norm_rope (tree order)", got, ref, atol=F32_ATOL, rtol=F32_RTOL,
                      label=f"{name} {n_special}+{gh}x{gw}{' global' if glob else ''}")


@pytest.mark.parametrize("heads,n_special,gh,gw", [(3, 1, 2, 3), (1, 2, 1, 3), (5, 2, 1, 1)])
def test_qk_norm_rope_odd_row_counts(rt, rng, heads, n_special, gh, gw):
    # an odd heads * tokens leaves the last (Q row, K row) pair group and
    # the grid's tail groups past the end: only real rows may be written
    n = n_special + gh * gw
    assert heads * n % 2 == 1
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    qg, qb, kg, kb = qk_params(rng)
    pos = oracle.rope_positions(n_special, gh, gw, 1, False)
    pad = normals(rng, 64)
    tq = rt.upload_f32(np.concatenate([q.reshape(-1), pad]))
    tk = rt.upload_f32(np.concatenate([k.reshape(-1), pad]))
    rt.qk_norm_rope_f32_da3_base(tq.view(0, heads * n * 64), tk.view(0, heads * n * 64),
                                 rt.upload_f32(qg), rt.upload_f32(qb), rt.upload_f32(kg),
                                 rt.upload_f32(kb), rt.upload_f32(pos), heads, n, 100.0, 1e-5)
    rq, rk = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, n)
    got_q, got_k = tq.numpy(), tk.numpy()
    assert_parity(got_q[:heads * n * 64], rq, F32_ATOL, F32_RTOL, "q")
    assert_parity(got_k[:heads * n * 64], rk, F32_ATOL, F32_RTOL, "k")
    assert np.array_equal(got_q[heads * n * 64:], pad) and np.array_equal(got_k[heads * n * 64:], pad)


def test_rope_alone_is_bit_exact(rt, rng):
    # without the LayerNorm the rotation itself has no reduction: the GPU
    # must equal the oracle bit for bit (shared cos/sin rounding, no FMA)
    heads, n_special, gh, gw = 12, 2, 24, 36
    n = n_special + gh * gw
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_grid_f32(tq, tk, None, None, None, None, heads, 64, n_special, gh, gw, 1,
                             False, vh.VK_QK_HEADS_OUTER)
    pos = oracle.rope_positions(n_special, gh, gw, 1, False).astype(np.int64)
    assert np.array_equal(tq.numpy().reshape(heads, n, 64), oracle.rope2d(q, heads, n, 64, pos))
    assert np.array_equal(tk.numpy().reshape(heads, n, 64), oracle.rope2d(k, heads, n, 64, pos))


def test_rope_positions_beyond_the_table(rt, rng):
    heads, n = 2, 6
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    pos = np.array([[0, 0], [1, 1], [1023, 5], [1024, 1100], [2000, 7], [5, 4096]], np.float32)
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_f32_da3_base(tq, tk, None, None, None, None, rt.upload_f32(pos), heads, n)
    ref = oracle.rope2d(q, heads, n, 64, pos.astype(np.int64))
    assert_parity(tq.numpy(), ref, F32_ATOL, F32_RTOL, "rope large positions")


@pytest.mark.parametrize("glob", [False, True])
def test_qk_grid_multi_view_layouts(rt, rng, glob):
    heads, n_special, gh, gw, views = 12, 2, 24, 36, 3
    tpv = n_special + gh * gw
    rows = tpv * views
    q, k = normals(rng, rows * heads * 64), normals(rng, rows * heads * 64)
    qg, qb, kg, kb = qk_params(rng)
    layout = vh.VK_QK_HEADS_OUTER if glob else vh.VK_QK_VIEWS_OUTER
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_grid_f32(tq, tk, *[rt.upload_f32(a) for a in (qg, qb, kg, kb)], heads, 64,
                             n_special, gh, gw, views, glob, layout)
    pos = oracle.rope_positions(n_special, gh, gw, views, glob)
    if glob:
        rq, rk = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, rows)
    else:
        rq, rk = q.reshape(views, heads, tpv, 64).copy(), k.reshape(views, heads, tpv, 64).copy()
        for v in range(views):
            rq[v], rk[v] = [a.reshape(heads, tpv, 64) for a in oracle.qk_norm_rope(
                rq[v], rk[v], qg, qb, kg, kb, pos[v * tpv:(v + 1) * tpv], heads, tpv)]
    assert_parity(tq.numpy(), rq, F32_ATOL, F32_RTOL, "q multi-view")
    assert_parity(tk.numpy(), rk, F32_ATOL, F32_RTOL, "k multi-view")


def test_qk_single_view_layouts_agree(rt, rng):
    heads, n_special, gh, gw = 12, 2, 6, 9
    n = n_special + gh * gw
    q, k = normals(rng, heads * n * 64), normals(rng, heads * n * 64)
    params = [rt.upload_f32(a) for a in qk_params(rng)]
    outs = []
    for layout in (vh.VK_QK_HEADS_OUTER, vh.VK_QK_VIEWS_OUTER):
        tq, tk = rt.upload_f32(q), rt.upload_f32(k)
        rt.qk_norm_rope_grid_f32(tq, tk, *params, heads, 64, n_special, gh, gw, 1, False, layout)
        outs.append((tq.numpy(), tk.numpy()))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_qk_f16_params_vit_l(rt, rng):
    heads, n_special, gh, gw = 16, 2, 48, 72
    n = n_special + gh * gw
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    qg, qb, kg, kb = qk_params(rng, np.float16)
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_grid_f32(tq, tk, *[rt.upload_f16(a) for a in (qg, qb, kg, kb)], heads, 64,
                             n_special, gh, gw, 1, False, vh.VK_QK_HEADS_OUTER)
    pos = oracle.rope_positions(n_special, gh, gw, 1, False)
    rq, rk = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, n)
    assert_parity(tq.numpy(), rq, F32_ATOL, F32_RTOL, "q f16 params")
    assert_parity(tk.numpy(), rk, F32_ATOL, F32_RTOL, "k f16 params")


def test_qk_rejects_unqualified_head_dim(rt, rng):
    t1, t2 = rt.upload_f32(normals(rng, 2 * 5 * 32)), rt.upload_f32(normals(rng, 2 * 5 * 32))
    with pytest.raises(vh.UnsupportedShape):
        rt.qk_norm_rope_grid_f32(t1, t2, None, None, None, None, 2, 32, 1, 2, 2, 1, False,
                                 vh.VK_QK_HEADS_OUTER)


def test_rope_positions_bit_exact(rt):
    for args in ((2, 24, 36, 12, False), (2, 24, 36, 12, True), (1, 3, 5, 2, False)):
        got = rt.rope_positions_f32(*args).numpy().reshape(-1, 2)
        assert np.array_equal(got, oracle.rope_positions(*args))


def test_rope_table_growth_keeps_captured_graphs_valid(rt, rng):
    """A grid wider than the default table (1,100 patches) grows the runtime's
    cos/sin table; a graph captured before the growth still reads the table
    it was captured with (kept alive until the runtime ends), and the wide
    grid's rotation matches the oracle bit for bit."""
    import gc
    heads, n_special = 2, 2
    small = (3, 5)
    n = n_special + small[0] * small[1]
    q, k = normals(rng, heads, n, 64), normals(rng, heads, n, 64)
    tq, tk = rt.upload_f32(q), rt.upload_f32(k)

    def small_step():
        rt.qk_norm_rope_grid_f32(tq, tk, None, None, None, None, heads, 64, n_special, *small, 1,
                                 False, vh.VK_QK_HEADS_OUTER)

    small_step()
    want = tq.numpy()
    rt.synchronize()
    gc.disable()
    try:
        rt.begin_capture()
        small_step()
        graph = rt.end_capture()
    finally:
        gc.enable()
    gh, gw = 1, 1100
    nw = n_special + gh * gw
    qw, kw = normals(rng, heads, nw, 64), normals(rng, heads, nw, 64)
    twq, twk = rt.upload_f32(qw), rt.upload_f32(kw)
    rt.qk_norm_rope_grid_f32(twq, twk, None, None, None, None, heads, 64, n_special, gh, gw, 1,
                             False, vh.VK_QK_HEADS_OUTER)
    pos = oracle.rope_positions(n_special, gh, gw, 1, False).astype(np.int64)
    assert np.array_equal(twq.numpy().reshape(heads, nw, 64), oracle.rope2d(qw, heads, nw, 64, pos))
    tq.write(q)
    graph.launch()
    rt.synchronize()
    assert np.array_equal(tq.numpy(), want)


def test_runtime_destroy_before_its_objects(rng):
    """Objects may outlive their runtime's handle: after vk_runtime_destroy
    the handle takes no new work, and the tensors, linears and events made
    on it are still destroyed cleanly (the runtime goes with the last)."""
    import ctypes
    import gc
    rt = vh.Runtime(0)
    h = rt.handle
    x = rng.standard_normal(4096).astype(np.float32)
    t = rt.upload_f32(x)
    assert np.array_equal(t.numpy(), x)
    lin = rt.prepare_linear_f32(16, 8, rng.standard_normal((16, 8)).astype(np.float32),
                                np.zeros(8, np.float32))
    ev = rt.event()
    ev.record()
    rt.close()
    out = ctypes.c_void_p()
    with pytest.raises(vh.VestraError, match="destroyed"):
        vh._check(vh.lib.vk_tensor_alloc(h, vh.VK_F32, 4, ctypes.byref(out)))
    with pytest.raises(vh.VestraError, match="destroyed"):
        vh._check(vh.lib.vk_runtime_synchronize(h))
    t.free()
    del lin, ev
    gc.collect()  # the last object releases the runtime
