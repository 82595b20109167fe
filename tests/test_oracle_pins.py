"""Pins the oracle (CPU restatement) before it is trusted as the GPU checker.

Each oracle function is checked against the reference's own known-answer data
(tests/golden/reference_kats.json), float64 library twins (tests/golden/
twins.npz, written by torch), float64 brute force, and invariants chosen so
that a plausible mistake (dropped term, wrong sign or index, transposed
operand, wrong epsilon) fails one of them.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle
from conftest import assert_parity, parity_report

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def twins():
    return dict(np.load(os.path.join(GOLDEN, "twins.npz")))


# ---------------------------------------------------------------- comparator
def test_compare_semantics_match_reference(kats):
    for case in kats["compare_semantics"]["cases"]:
        ok, max_abs, worst = parity_report(case["got"], case["ref"], case["atol"], case["rtol"])
        assert ok == case["ok"]
        if "worst" in case:
            assert worst == case["worst"]
            assert abs(max_abs - case["max_abs"]) < 1e-9


def test_compare_rejects_nan_and_size_mismatch():
    # stricter than the reference on NaN (its `d > tol` lets one pass)
    assert not parity_report([1.0, float("nan")], [1.0, 1.0], 1.0, 1.0)[0]
    assert not parity_report([1.0, 1.0], [1.0, float("nan")], 1.0, 1.0)[0]
    assert not parity_report([1.0, 2.0], [1.0], 1.0, 1.0)[0]


# ---------------------------------------------------------------- f16
def test_f16_widening_is_exact_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ---------------------------------------------------------------- LayerNorm
def test_layernorm_kat_zero_mean(kats):
    k = kats["layernorm_kat"]
    y = oracle.layernorm(np.array([k["x"]], np.float32), np.ones(4, np.float32),
                         np.zeros(4, np.float32), k["eps"])
    assert abs(float(y.mean())) < k["mean_tol"]


def test_layernorm_matches_torch_twin_768(twins):
    y = oracle.layernorm(twins["ln768_x"], twins["ln768_g"], twins["ln768_b"], 1e-6)
    assert_parity(y, twins["ln768_y64"], 1e-6, 1e-5, "ln768 vs torch f64")


def test_layernorm_matches_torch_twin_qk64(twins):
    y = oracle.layernorm(twins["ln64_x"], twins["ln64_g"], twins["ln64_b"], 1e-5)
    assert_parity(y, twins["ln64_y64"], 1e-6, 1e-5, "ln64 vs torch f64")


def test_layernorm_float64_brute_force_and_wrong_variants(rng):
    x = (rng.standard_normal((33, 1024)) * 2 + 0.3).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(1024)).astype(np.float32)
    b = (0.02 * rng.standard_normal(1024)).astype(np.float32)
    y = oracle.layernorm(x, g, b, 1e-6)
    xd = x.astype(np.float64)
    m = xd.mean(-1, keepdims=True)
    v = ((xd - m) ** 2).mean(-1, keepdims=True)
    ref = (xd - m) / np.sqrt(v + 1e-6) * g + b
    assert_parity(y, ref, 1e-6, 1e-5, "ln brute force")
    # an unbiased variance or a gamma/beta swap must not pass
    v_unb = ((xd - m) ** 2).sum(-1, keepdims=True) / (1024 - 1)
    wrong = (xd - m) / np.sqrt(v_unb + 1e-6) * g + b
    assert not parity_report(y, wrong, 1e-6, 1e-5)[0]
    wrong2 = (xd - m) / np.sqrt(v + 1e-6) * b + g
    assert not parity_report(y, wrong2, 1e-6, 1e-5)[0]


def test_layernorm_sequential_sum_order():
    # A row whose sequential f32 sum differs from its pairwise sum: the
    # oracle must follow the reference's left-to-right order.
    row = np.array([1e8, 1.0, -1e8, 1.0] * 16, np.float32)
    seq = np.float32(0)
    for v in row:
        seq = np.float32(seq + v)
    y = oracle.layernorm(row[None], np.ones(64, np.float32), np.zeros(64, np.float32), 1e-5)
    mean = np.float32(seq / np.float32(64))
    d = (row - mean).astype(np.float32)
    sq = np.float32(0)
    for v in d:
        sq = np.float32(sq + np.float32(v * v))
    inv = np.float32(1) / np.sqrt(np.float32(sq / np.float32(64)) + np.float32(1e-5))
    expect = ((row - mean) * inv).astype(np.float32)
    assert np.array_equal(y[0], expect)


def test_qk_norm_eps_discriminator(rng):
    # attention_and_layerscale_op.rs:91-196: near-constant rows make eps 1e-5
    # and 1e-6 distinguishable.
    heads, n, hd = 2, 2, 4
    q = np.zeros((heads * n, hd), np.float32)
    for r in range(heads * n):
        q[r] = 100.0 + r + rng.uniform(-1e-3, 1e-3, hd)
    g, b = np.ones(hd, np.float32), np.zeros(hd, np.float32)
    y5 = oracle.layernorm(q, g, b, 1e-5)
    y6 = oracle.layernorm(q, g, b, 1e-6)
    assert np.max(np.abs(y5 - y6)) > 1e-8


# ---------------------------------------------------------------- GELU
AS_BOUND = 1.5e-7 + 6 * 2.0 ** -24


def test_gelu_kats(kats):
    k = kats["gelu_kat"]
    y = oracle.gelu(np.array(k["x"], np.float32))
    for got, exp, tol in zip(y, k["expected"], k["tol"]):
        assert abs(float(got) - exp) < tol


def test_erf_as7126_error_bound():
    xs = np.linspace(-6, 6, 4001)
    err = max(abs(oracle.erf_as7126(float(np.float32(x))) - math.erf(float(np.float32(x))))
              for x in xs)
    # A&S 7.1.26 bound 1.5e-7 plus f32 evaluation: the cancellation in
    # 1 - p*t*exp(-a^2) costs up to ~6 ulp(1) = 6 * 2^-24
    assert err < AS_BOUND
    # a wrong coefficient is far outside that bound
    assert err > 0


def test_gelu_within_as7126_bound_of_exact_twin(twins):
    x = twins["gelu_x"]
    y = oracle.gelu(x).astype(np.float64)
    exact = twins["gelu_y64"]
    bound = 0.5 * np.abs(x.astype(np.float64)) * AS_BOUND + 2 * np.spacing(
        np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(y - exact) <= bound + 1e-30)


def test_gelu_erff_variant_matches_exact_twin(twins):
    y = oracle.gelu_erff(twins["gelu_x"])
    assert_parity(y, twins["gelu_y64"], 1e-6, 1e-5, "gelu(erff) vs torch f64")


# ---------------------------------------------------------------- LayerScale / residual
def test_layerscale_op_values(kats):
    k = kats["layerscale_op"]
    x = np.array(k["x"], np.float32).reshape(k["rows"], k["cols"])
    y = oracle.layerscale(x, np.array(k["gamma"], np.float32))
    assert np.array_equal(y.reshape(-1), np.array(k["expected"], np.float32))


def test_layerscale_residual_two_roundings(rng):
    x = rng.standard_normal((5, 8)).astype(np.float32)
    y = rng.standard_normal((5, 8)).astype(np.float32)
    g = rng.uniform(0, 0.1, 8).astype(np.float32)
    out = oracle.layerscale_residual(x, y, g)
    expect = (x + (y * g).astype(np.float32)).astype(np.float32)
    assert np.array_equal(out, expect)
    assert np.array_equal(oracle.layerscale_residual(x, y, None), (x + y).astype(np.float32))
    # an FMA (single rounding) differs on some elements of a larger draw
    xb = rng.standard_normal(4096).astype(np.float32)
    yb = rng.standard_normal(4096).astype(np.float32)
    gb = np.full(4096, np.float32(0.0731))
    two = oracle.layerscale_residual(xb[None], yb[None], gb)[0]
    fma = (xb.astype(np.float64) + yb.astype(np.float64) * gb.astype(np.float64)).astype(np.float32)
    assert np.array_equal(two, (xb + (yb * gb).astype(np.float32)).astype(np.float32))
    assert not np.array_equal(two, fma)


def test_layerscale_residual_w16_equals_widened(rng):
    x = rng.standard_normal((3, 16)).astype(np.float32)
    y = rng.standard_normal((3, 16)).astype(np.float32)
    g16 = rng.uniform(0, 0.1, 16).astype(np.float16)
    assert np.array_equal(oracle.layerscale_residual(x, y, g16),
                          oracle.layerscale_residual(x, y, g16.astype(np.float32)))


# ---------------------------------------------------------------- RoPE
def test_rope_positions_layout():
    # n_special 2, grid 2x3, two views: specials (0,0) per view, patches
    # (row+1, col+1) locally, (1,1) globally (vit_block.rs:841-881).
    loc = oracle.rope_positions(2, 2, 3, 2, False)
    one_view = [[0, 0], [0, 0], [1, 1], [1, 2], [1, 3], [2, 1], [2, 2], [2, 3]]
    assert loc.tolist() == one_view * 2
    glob = oracle.rope_positions(2, 2, 3, 2, True)
    assert glob.tolist() == ([[0, 0], [0, 0]] + [[1, 1]] * 6) * 2


def test_rope_identity_at_origin(rng):
    x = rng.standard_normal((2, 3, 64)).astype(np.float32)
    pos = np.zeros((3, 2), np.int64)
    assert np.array_equal(oracle.rope2d(x, 2, 3, 64, pos), x)


def test_rope_i64_position_beyond_32_bits():
    # A coordinate of 2^32 + 5 turns by the angle of its f32 conversion,
    # (float)(2^32 + 5) = 2^32, as `p as f32 * inv_freq` reads an i64: not by
    # 5 (its low 32 bits).  Frequency 0 turns by exactly that many radians.
    theta = float(np.float32(2 ** 32 + 5))
    assert theta == 2.0 ** 32
    for half, pos in ((0, [2 ** 32 + 5, 0]), (32, [0, 2 ** 32 + 5])):
        x = np.zeros((1, 1, 64), np.float32)
        x[0, 0, half] = 1.0
        y = oracle.rope2d(x, 1, 1, 64, np.array([pos], np.int64), 100.0, 0)[0, 0]
        assert abs(float(y[half]) - math.cos(theta)) < 2e-6
        assert abs(float(y[half + 16]) - math.sin(theta)) < 2e-6
        assert abs(math.cos(theta) - math.cos(5.0)) > 0.1  # the narrowed angle differs


def _pairs(mode):
    """Element pairs (a, b) of one 32-wide half under a RoPE convention:
    rotate-half (j, j+16) or interleaved (2j, 2j+1), in frequency order j."""
    if mode & oracle.ROPE_INTERLEAVED:
        return [(2 * j, 2 * j + 1) for j in range(16)]
    return [(j, j + 16) for j in range(16)]


@pytest.mark.parametrize("mode", oracle.ROPE_MODES)
def test_rope_preserves_pair_norms(rng, mode):
    x = rng.standard_normal((3, 5, 64)).astype(np.float32)
    pos = rng.integers(0, 80, (5, 2))
    y = oracle.rope2d(x, 3, 5, 64, pos, 100.0, mode).astype(np.float64)
    xd = x.astype(np.float64)
    for half in (0, 32):
        for a, b in _pairs(mode):
            n0 = xd[..., half + a] ** 2 + xd[..., half + b] ** 2
            n1 = y[..., half + a] ** 2 + y[..., half + b] ** 2
            assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("mode", oracle.ROPE_MODES)
def test_rope_complex_twin(rng, mode):
    # float64 twin written as complex multiplication: pair (a, b) of half h
    # is z = x_a + i x_b, rotated to z * exp(i p_h w_j) with
    # w_j = base^(-2j / denom), denom = 32 (exponent over the half) or 64
    # (over the head); the y half takes the row coordinate, the x half the
    # column.  The oracle rounds the angle once in f32, so the bound grows
    # with the angle.
    heads, n, base = 2, 9, 100.0
    x = rng.standard_normal((heads, n, 64)).astype(np.float32)
    pos = rng.integers(0, 60, (n, 2))
    pos[0] = (0, 0)
    got = oracle.rope2d(x, heads, n, 64, pos, base, mode).astype(np.float64)
    denom = 64.0 if mode & oracle.ROPE_EXP_HEAD else 32.0
    w = base ** (-2.0 * np.arange(16) / denom)
    expect = np.empty_like(got)
    for half, coord in ((0, 0), (32, 1)):
        for j, (a, b) in enumerate(_pairs(mode)):
            z = x[..., half + a].astype(np.float64) + 1j * x[..., half + b]
            z = z * np.exp(1j * pos[:, coord] * w[j])
            expect[..., half + a] = z.real
            expect[..., half + b] = z.imag
    mag = np.abs(x).astype(np.float64).max()
    bound = 4e-7 * mag * (1.0 + pos.max())
    assert np.max(np.abs(got - expect)) < bound


@pytest.mark.parametrize("mode", oracle.ROPE_MODES)
def test_rope_closed_form_angles(mode):
    # Textbook values: frequency 0 turns by exactly p radians; with base 100,
    # frequency 8 turns by p * 100^(-16/32) = p/10 (exponent over the half)
    # or p * 100^(-16/64) = p/sqrt(10) (over the head).  A unit vector at the
    # pair's first element lands on (cos t, sin t) in (first, second).
    pairs = _pairs(mode)
    slow = 1.0 / math.sqrt(10.0) if mode & oracle.ROPE_EXP_HEAD else 0.1
    for j, p, theta in ((0, 1, 1.0), (0, 3, 3.0), (8, 10, 10 * slow), (8, 7, 7 * slow)):
        for half, pos in ((0, [p, 0]), (32, [0, p])):
            a, b = pairs[j]
            x = np.zeros((1, 1, 64), np.float32)
            x[0, 0, half + a] = 1.0
            y = oracle.rope2d(x, 1, 1, 64, np.array([pos], np.int64), 100.0, mode)[0, 0]
            assert abs(float(y[half + a]) - math.cos(theta)) < 2e-6
            assert abs(float(y[half + b]) - math.sin(theta)) < 2e-6
            others = np.delete(y, [half + a, half + b])
            assert not others.any()


def test_rope_relative_position_property(rng):
    # <R(p)q, R(p')k> depends only on p - p' (per coordinate)
    q = rng.standard_normal((1, 1, 64)).astype(np.float32)
    k = rng.standard_normal((1, 1, 64)).astype(np.float32)

    def dot(pq, pk):
        a = oracle.rope2d(q, 1, 1, 64, np.array([pq], np.int64)).astype(np.float64)
        b = oracle.rope2d(k, 1, 1, 64, np.array([pk], np.int64)).astype(np.float64)
        return float((a * b).sum())

    base = dot((3, 5), (1, 2))
    for shift in ((1, 0), (0, 4), (7, 9)):
        s = dot((3 + shift[0], 5 + shift[1]), (1 + shift[0], 2 + shift[1]))
        assert abs(s - base) < 1e-4 * max(1.0, abs(base))
    assert abs(dot((4, 5), (1, 2)) - base) > 1e-3


@pytest.mark.parametrize("mode", oracle.ROPE_MODES)
def test_rope_recovered_angles_and_pairing(mode):
    # a unit vector at the first element of pair j of a half rotates inside
    # that pair only, by pos * base^(-2j/denom): y half by the row
    # coordinate, x half by the column.
    py, px = 7, 3
    denom = 64.0 if mode & oracle.ROPE_EXP_HEAD else 32.0
    for half, p in ((0, py), (32, px)):
        for j, (a, b) in enumerate(_pairs(mode)):
            x = np.zeros((1, 1, 64), np.float32)
            x[0, 0, half + a] = 1.0
            y = oracle.rope2d(x, 1, 1, 64, np.array([[py, px]], np.int64), 100.0, mode)[0, 0]
            nz = np.flatnonzero(np.abs(y) > 1e-7)
            assert set(nz.tolist()) <= {half + a, half + b}
            theta = math.atan2(float(y[half + b]), float(y[half + a]))
            expect = p * 100.0 ** (-2.0 * j / denom)
            d = (theta - expect + math.pi) % (2 * math.pi) - math.pi
            assert abs(d) < 2e-5 * max(1.0, expect)


def test_rope_conventions_differ(rng):
    # the four conventions are four different functions of the same input
    x = rng.standard_normal((1, 4, 64)).astype(np.float32)
    pos = np.array([[0, 0], [3, 5], [2, 7], [11, 4]], np.int64)
    outs = [oracle.rope2d(x, 1, 4, 64, pos, 100.0, m) for m in oracle.ROPE_MODES]
    for i in range(len(outs)):
        assert np.array_equal(outs[i][:, 0], x[:, 0])
        for j in range(i):
            assert np.max(np.abs(outs[i][:, 1:] - outs[j][:, 1:])) > 1e-3


def test_rope_changes_output(kats):
    k = kats["rope_changes_output"]
    rng = np.random.default_rng(0x12345678)
    x = rng.standard_normal((k["heads"], k["n"], k["head_dim"])).astype(np.float32)
    pos = np.array(k["pos_yx"], np.int64).reshape(k["n"], 2)
    y = oracle.rope2d(x, k["heads"], k["n"], k["head_dim"], pos, k["freq"])
    assert np.array_equal(y[:, 0], x[:, 0])  # token at (0,0) unchanged
    assert np.max(np.abs(y[:, 1] - x[:, 1])) > 1e-4


@pytest.mark.parametrize("mode", oracle.ROPE_MODES)
def test_qk_norm_rope_is_norm_then_rope(rng, mode):
    heads, n = 3, 7
    q = rng.standard_normal((heads, n, 64)).astype(np.float32)
    k = rng.standard_normal((heads, n, 64)).astype(np.float32)
    qg, qb, kg, kb = [(1 + 0.02 * rng.standard_normal(64)).astype(np.float32) for _ in range(4)]
    pos = oracle.rope_positions(1, 2, 3, 1, False)
    qo, ko = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, n, mode=mode)
    pi = pos.astype(np.int64)
    q_ref = oracle.rope2d(oracle.layernorm(q, qg, qb, 1e-5), heads, n, 64, pi, 100.0, mode)
    k_ref = oracle.rope2d(oracle.layernorm(k, kg, kb, 1e-5), heads, n, 64, pi, 100.0, mode)
    assert np.array_equal(qo, q_ref) and np.array_equal(ko, k_ref)
    if mode:
        return
    # rope-then-norm is a different function
    wrong = oracle.layernorm(oracle.rope2d(q, heads, n, 64, pos.astype(np.int64)), qg, qb, 1e-5)
    assert not np.allclose(qo, wrong, atol=1e-4)


# ---------------------------------------------------------------- patch embed
def test_patch_embed_kats(kats):
    for name in ("patch_embed_bias_broadcast", "patch_embed_row_major"):
        k = kats[name]
        img = np.array(k["image_nchw"], np.float32).reshape(3, k["h"], k["w"])
        w = np.array(k["weight_oihw"], np.float32).reshape(k["embed"], 3, k["patch"], k["patch"])
        out = oracle.patch_project_oihw(img, k["patch"], w, np.array(k["bias"], np.float32))
        assert out.tolist() == k["expected_tokens"], name


def test_patch_projection_matches_conv2d_twin(twins):
    out = oracle.patch_project_oihw(twins["conv_img"], 14, twins["conv_w"], twins["conv_b"])
    assert_parity(out, twins["conv_y64"], 1e-6, 1e-5, "patch conv vs torch f64")
    # the split path (patchify -> linear with W^T) is the same projection
    rows = oracle.patchify_nchw(twins["conv_img"], 14)
    wt = twins["conv_w"].reshape(16, -1).T.copy()
    lin = oracle.linear(rows, wt, twins["conv_b"])
    assert_parity(lin, twins["conv_y64"], 1e-6, 1e-5, "patchify+linear vs torch f64")


def test_normalize_kat(kats):
    k = kats["normalize"]
    img = np.array(k["hwc_u8"], np.uint8).reshape(k["h"], k["w"], 3)
    out = oracle.normalize_u8_hwc(img, k["mean"], k["std"])
    for c in range(3):
        for y in range(k["h"]):
            for x in range(k["w"]):
                v = int(img[y, x, c])
                expect = (np.float32(v) / np.float32(255.0) - np.float32(k["mean"][c])) / np.float32(k["std"][c])
                assert abs(float(out[c, y, x]) - float(expect)) < k["tolerance"]
                f64 = (v / 255.0 - k["mean"][c]) / k["std"][c]
                assert abs(float(out[c, y, x]) - f64) < 1e-5


def test_pos_embed_kats(kats):
    k = kats["pos_embed_tokens"]
    pe = np.array(k["pos_embed"], np.float32)
    table = oracle.pos_embed_bicubic(pe, k["grid"], k["embed"], k["gh"], k["gw"])
    patches = np.zeros((k["gh"] * k["gw"], k["embed"]), np.float32)
    toks = oracle.assemble_tokens(patches, k["gh"], k["gw"], np.array(k["cls"], np.float32), None,
                                  table)
    assert toks[0].tolist() == k["expected_row0"]
    native = oracle.pos_embed_bicubic(pe, 3, 2, 3, 3)
    assert native[0].tolist() == k["native_grid_cls_row"]


def test_pos_embed_bicubic_matches_torch_twin(twins):
    pe = twins["pe_src"]
    for gh, gw in ((24, 36), (5, 7)):
        out = oracle.pos_embed_bicubic(pe, 37, 8, gh, gw, 0.1)
        assert np.array_equal(out[0], pe[0])
        assert_parity(out[1:], twins[f"pe_{gh}x{gw}_y64"], 1e-6, 1e-4, f"bicubic {gh}x{gw}")


def test_pos_embed_partition_of_unity():
    # a constant grid resizes to the same constant (Keys weights sum to 1)
    pe = np.full((37 * 37 + 1, 4), 0.25, np.float32)
    out = oracle.pos_embed_bicubic(pe, 37, 4, 24, 36)
    assert np.allclose(out, 0.25, atol=1e-6)


def test_assemble_tokens_registers_get_no_position(rng):
    embed, gh, gw = 8, 2, 3
    patches = rng.standard_normal((gh * gw, embed)).astype(np.float32)
    cls = rng.standard_normal(embed).astype(np.float32)
    regs = rng.standard_normal((1, embed)).astype(np.float32)
    pos = rng.standard_normal((1 + gh * gw, embed)).astype(np.float32)
    toks = oracle.assemble_tokens(patches, gh, gw, cls, regs, pos)
    assert np.array_equal(toks[0], cls + pos[0])
    assert np.array_equal(toks[1], regs[0])
    assert np.array_equal(toks[2:], patches + pos[1:])


def test_patch_embed_u8_composes_the_three_steps(rng):
    h, w, embed = 28, 42, 16
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    mean, std = [0.485, 0.456, 0.406], [0.229, 0.224, 0.225]
    wt = (0.02 * rng.standard_normal((embed, 3, 14, 14))).astype(np.float32)
    b = (0.02 * rng.standard_normal(embed)).astype(np.float32)
    cls = rng.standard_normal(embed).astype(np.float32)
    pos = rng.standard_normal((1 + 6, embed)).astype(np.float32)
    full = oracle.patch_embed_u8(img, 14, mean, std, wt, b, cls, None, pos)
    chw = oracle.normalize_u8_hwc(img, mean, std)
    proj = oracle.patch_project_oihw(chw, 14, wt, b)
    assert np.array_equal(full, oracle.assemble_tokens(proj, 2, 3, cls, None, pos))


# ---------------------------------------------------------------- QKV layout glue
def test_split_qkv_hnd_matches_the_documented_reshape(rng):
    # vit_block.rs:38-43: columns Q | K | V, each [heads, head_dim] head-major,
    # i.e. ggml_reshape_4d(qkv, D, H, 3, tok); the pack loop (vit_block.rs:818-833)
    # moves it to [heads, n, head_dim]
    n, heads, hd = 7, 3, 8
    qkv = rng.standard_normal((n, 3 * heads * hd)).astype(np.float32)
    q, k, v = oracle.split_qkv_hnd(qkv, n, heads, hd)
    want = qkv.reshape(n, 3, heads, hd).transpose(1, 2, 0, 3)
    assert np.array_equal(q, want[0]) and np.array_equal(k, want[1]) and np.array_equal(v, want[2])
    # one element by hand: token 5, K block, head 2, dim 3
    assert k[2, 5, 3] == qkv[5, heads * hd + 2 * hd + 3]
    # a transposed read (heads and tokens swapped) would not match
    assert not np.array_equal(q, qkv[:, :heads * hd].reshape(heads, n, hd))


def test_hnd_to_token_inverts_the_split(rng):
    n, heads, hd = 5, 4, 16
    hnd = rng.standard_normal((heads, n, hd)).astype(np.float32)
    tok = oracle.hnd_to_token(hnd, n, heads, hd)
    assert np.array_equal(tok, hnd.transpose(1, 0, 2).reshape(n, heads * hd))
    qkv = np.concatenate([tok, tok + 1, tok + 2], axis=1)
    q, k, v = oracle.split_qkv_hnd(qkv, n, heads, hd)
    assert np.array_equal(q, hnd) and np.array_equal(k, hnd + 1) and np.array_equal(v, hnd + 2)


# ---------------------------------------------------------------- attention core
def _attention_f64(q, k, v):
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) / np.sqrt(q.shape[-1])
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return np.einsum("bij,bjd->bid", p / p.sum(axis=-1, keepdims=True), v.astype(np.float64))


def test_attention_matches_float64_brute_force(rng):
    b, n, d = 3, 37, 64
    q, k, v = (rng.standard_normal((b, n, d)).astype(np.float32) for _ in range(3))
    got = oracle.attention(q, k, v, b, n, d)
    ref = _attention_f64(q, k, v)
    assert np.max(np.abs(got - ref)) < 2e-6
    # dropping the 1/sqrt(d) scale is a different function
    wrong = _attention_f64(q * np.sqrt(d).astype(np.float32), k, v)
    assert np.max(np.abs(got - wrong)) > 1e-2


def test_attention_matches_torch_sdpa_twin(rng):
    torch = pytest.importorskip("torch")
    b, n, d = 2, 50, 64
    q, k, v = (rng.standard_normal((b, n, d)).astype(np.float32) for _ in range(3))
    twin = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(a).double() for a in (q, k, v))).numpy()
    assert np.max(np.abs(oracle.attention(q, k, v, b, n, d) - twin)) < 2e-6


def test_attention_invariants(rng):
    n, d = 20, 64
    q, k, v = (rng.standard_normal((1, n, d)).astype(np.float32) for _ in range(3))
    # one key far ahead of the others selects its value row
    k2 = k.copy()
    k2[0, 7] = q[0, 3] * 40
    assert np.allclose(oracle.attention(q, k2, v, 1, n, d)[0, 3], v[0, 7], atol=1e-6)
    # identical value rows come back unchanged (up to rounding)
    vc = np.repeat(v[:, :1], n, axis=1)
    assert np.allclose(oracle.attention(q, k, vc, 1, n, d), vc, rtol=0, atol=2e-6)
    # permuting keys and values together changes nothing but rounding
    perm = rng.permutation(n)
    assert np.allclose(oracle.attention(q, k[:, perm], v[:, perm], 1, n, d),
                       oracle.attention(q, k, v, 1, n, d), rtol=0, atol=2e-6)


# ---------------------------------------------------------------- whole block
def test_block_forward_matches_float64_twin(rng):
    """The oracle's whole-block composition (vit_block.rs:1019-1139) against an
    independent float64 composition of the same steps (tests/block_twin.py):
    local layer with 3 views, global layer, and the camera slot at alt_start."""
    from block_twin import block_f64, config, make_params, normals
    D, H, M, gh, gw, views = 768, 12, 3072, 4, 6, 3
    cfg = config(D, H, M)
    rows = (2 + gh * gw) * views
    for layer in (2, 4, 5):
        p = make_params(rng, D, M)
        x0, cam = normals(rng, rows, D), normals(rng, 2 * D)
        got = oracle.block_forward(x0, p, cfg, layer, gh, gw, views, cam)
        ref = block_f64(x0, p, cfg, layer, gh, gw, views, cam)
        for name in ("tokens", "q", "k", "v", "attn", "ln2", "hidden"):
            d = np.abs(got[name].astype(np.float64).reshape(-1) - ref[name].reshape(-1)).max()
            assert d < 2e-5, (layer, name, d)
        if layer == 2:
            # attending across views (the global rule on a local layer) is a
            # different function
            wrong = block_f64(x0, p, dict(cfg, alt_start=1), 3, gh, gw, views, cam)
            assert np.abs(got["attn"] - wrong["attn"]).max() > 1e-2
            # a missing LayerScale is a different function
            nols = {k: v for k, v in p.items() if k not in ("ls1", "ls2")}
            wrong = block_f64(x0, nols, cfg, layer, gh, gw, views, cam)
            assert np.abs(got["tokens"] - wrong["tokens"]).max() > 1e-2


# ---------------------------------------------------------------- capture / head hand-off
def test_capture_layout_rules(rng):
    """backbone.rs:1287-1372: cat_token -> feat [n_patch, 2*embed] and cam
    [2*embed]; without it -> [n_patch, embed] and [embed]; the normalised half
    is the scalar LayerNorm of the patch rows."""
    D, n, ns = 8, 5, 1  # 1 CLS + 2x2 patch grid, as the reference's tests
    x, local = rng.standard_normal((n, D)).astype(np.float32), \
        rng.standard_normal((n, D)).astype(np.float32)
    g, b = np.ones(D, np.float32), np.zeros(D, np.float32)
    feat, cam = oracle.capture(local, x, n, ns, D, 1, g, b, 1e-6, True)
    assert feat.shape == (1, 4, 2 * D) and cam.shape == (1, 2 * D)
    assert np.array_equal(feat[0, :, :D], local[1:]) and np.array_equal(cam[0, :D], local[0])
    assert np.array_equal(cam[0, D:], x[0])
    normed = feat[0, :, D:].astype(np.float64)
    assert np.allclose(normed.mean(axis=1), 0, atol=1e-6)
    assert np.allclose(normed.var(axis=1), 1, atol=1e-4)
    feat1, cam1 = oracle.capture(None, x, n, ns, D, 1, g, b, 1e-6, False)
    assert feat1.shape == (1, 4, D) and np.array_equal(feat1[0], feat[0, :, D:])
    assert np.array_equal(cam1[0], x[0])


def test_token_to_chw_reference_vectors_and_layout():
    """dpt_head.rs:1041-1070 vectors: exact binary inputs; out[ch, t] is the
    LayerNorm'd tok[t, ch] (eps HEAD_NORM_EPS = 1e-5, dpt_head.rs:101)."""
    n_tok, c = 35, 16
    tok = ((np.arange(n_tok * c) * 37 % 251).astype(np.float32) - 125.0) * 0.0078125
    g = (0.5 + np.arange(c) * 0.03125).astype(np.float32)
    b = (-0.25 + np.arange(c) * 0.015625).astype(np.float32)
    out = oracle.token_to_chw(tok, n_tok, c, g, b, 1e-5)
    t64 = tok.reshape(n_tok, c).astype(np.float64)
    m = t64.mean(axis=1, keepdims=True)
    ref = ((t64 - m) / np.sqrt(((t64 - m) ** 2).mean(axis=1, keepdims=True) + 1e-5) * g + b).T
    assert out.shape == (c, n_tok)
    assert np.max(np.abs(out - ref)) < 1e-5
    assert np.array_equal(oracle.token_to_chw(tok, n_tok, c), tok.reshape(n_tok, c).T)


# ---------------------------------------------------------------- GGUF Q8_0 weights
def test_q8_0_reference_block():
    """crates/da-gguf/tests/q8_0_roundtrip.rs: d = 0.5, q = -16..15 -> d*q."""
    blk = np.empty(34, np.uint8)
    blk[:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    out = oracle.dequantize_q8_0(blk, 32)
    assert np.array_equal(out, 0.5 * (np.arange(32) - 16).astype(np.float32))


def test_q8_0_layout_and_round_trip(rng):
    """Wire layout (little-endian f16 scale, then int8, 34 bytes per block;
    q8_0.rs:36-51) and the quantise/dequantise round trip within d/2."""
    x = rng.standard_normal(32 * 40).astype(np.float32) * 0.02
    raw = oracle.quantize_q8_0(x)
    assert raw.size == 40 * 34
    back = oracle.dequantize_q8_0(raw, x.size)
    d = np.frombuffer(raw.reshape(40, 34)[:, :2].tobytes(), "<f2").astype(np.float64)
    assert np.all(np.abs(back - x).reshape(40, 32) <= d[:, None] / 2 + 1e-12)
    # a byte-swapped scale is a different tensor
    swapped = raw.reshape(40, 34).copy()
    swapped[:, [0, 1]] = swapped[:, [1, 0]]
    assert not np.array_equal(oracle.dequantize_q8_0(swapped, x.size), back)
    with pytest.raises(ValueError):
        oracle.dequantize_q8_0(raw, x.size + 32)


# ---------------------------------------------------------------- preprocessing resize
def test_preprocess_shape_reference_cases():
    """preprocess.rs:541-612: 2x2 at image_size 4 / patch 2 -> 4x4; identity at
    2; 427x640 at 504 / patch 14 -> 336x504 (upper bound); "lower*" modes
    bound the short side."""
    assert oracle.preprocess_shape(2, 2, 4, 2)[2:4] == (4, 4)
    assert oracle.preprocess_shape(2, 2, 2, 2) == (2, 2, 2, 2, False)
    assert oracle.preprocess_shape(427, 640, 504, 14)[2:4] == (336, 504)
    assert oracle.preprocess_shape(3, 3, 4, 2)[2:4] == (4, 4)
    bh, bw, oh, ow, _ = oracle.preprocess_shape(427, 640, 504, 14, upper_bound=False)
    assert bh == 504 and (oh, ow) == (504, 756)
    # ties of the boundary size round to even, snaps prefer the larger multiple
    assert oracle.preprocess_shape(10, 5, 4, 1)[:2] == (4, 2)
    assert oracle.preprocess_shape(7, 7, 7, 2)[2:4] == (8, 8)


def test_preprocess_identity_is_a_copy(rng):
    img = rng.integers(0, 256, (2, 2, 3), dtype=np.uint8)
    assert np.array_equal(oracle.preprocess_resize_u8(img, 2, 2), img)


@pytest.mark.parametrize("mode", ["bilinear", "cubic", "area"])
def test_resize_constant_image_stays_constant(mode):
    for (sh, sw, dh, dw) in ((5, 7, 13, 9), (40, 30, 7, 11), (336, 504, 336, 504)):
        img = np.full((sh, sw, 3), (17, 128, 254), np.uint8)
        out = oracle.resize_u8(img, dh, dw, mode)
        assert np.array_equal(out, np.broadcast_to(img[:1, :1], out.shape)), (mode, sh, sw)


def _torch_resize(img, dh, dw, mode):
    torch = pytest.importorskip("torch")
    t = torch.from_numpy(img.astype(np.float64)).permute(2, 0, 1)[None]
    kw = {} if mode == "area" else {"align_corners": False}
    r = torch.nn.functional.interpolate(t, size=(dh, dw), mode=mode, **kw)
    return r[0].permute(1, 2, 0).numpy()


@pytest.mark.parametrize("mode,torch_mode,shape", [
    ("bilinear", "bilinear", (23, 31, 40, 57)), ("bilinear", "bilinear", (40, 57, 23, 31)),
    ("cubic", "bicubic", (23, 31, 40, 57)), ("cubic", "bicubic", (48, 64, 36, 50)),
    ("area", "area", (48, 60, 12, 20))])
def test_resize_matches_torch_twins(rng, mode, torch_mode, shape):
    """Half-pixel centres, clamp-to-edge taps, Keys a = -0.75 (torch's bicubic
    uses the same kernel), and the box filter at integer factors: within one
    u8 step of torch's float64 result (the reference rounds from f32)."""
    sh, sw, dh, dw = shape
    img = rng.integers(0, 256, (sh, sw, 3), dtype=np.uint8)
    got = oracle.resize_u8(img, dh, dw, mode).astype(np.float64)
    twin = np.clip(np.rint(_torch_resize(img, dh, dw, torch_mode)), 0, 255)
    assert np.max(np.abs(got - twin)) <= 1.0


def test_resize_area_matches_exact_box_integral(rng):
    """Non-integer downscale: the area taps approximate the exact overlap
    integral of each destination cell (preprocess.rs:347-382)."""
    sh, sw, dh, dw = 37, 53, 10, 14
    img = rng.integers(0, 256, (sh, sw, 3), dtype=np.uint8).astype(np.float64)

    def box(n_src, n_dst):
        m = np.zeros((n_dst, n_src))
        s = n_src / n_dst
        for d in range(n_dst):
            a, b = d * s, (d + 1) * s
            for i in range(int(np.floor(a)), min(n_src, int(np.ceil(b)))):
                m[d, i] = max(0.0, min(b, i + 1) - max(a, i)) / s
        return m

    exact = np.einsum("yi,xj,ijc->yxc", box(sh, dh), box(sw, dw), img)
    got = oracle.resize_u8(img.astype(np.uint8), dh, dw, "area").astype(np.float64)
    assert np.max(np.abs(got - np.rint(exact))) <= 1.0


# ---------------------------------------------------------------- backbone loop
def test_backbone_captures_follow_the_reference_rules(rng):
    """backbone.rs:1287-1372: captures in the requested (not execution) order,
    widths 2*embed (cat_token) or embed, n_patch rows, finite, distinct per
    layer; global layers pair the stream with the snapshot of the last local
    layer (backbone.rs:816-830); matches the float64 twin."""
    from block_twin import backbone_f64, config, make_params, normals
    D, H, M, gh, gw, views = 64, 1, 128, 2, 2, 2
    cfg = config(D, H, M, alt=2)
    blocks = [make_params(rng, D, M) for _ in range(6)]
    n = 2 + gh * gw
    x0, cam = normals(rng, views * n, D), normals(rng, 2 * D)
    ng, nb = normals(rng, D, scale=0.02, shift=1), normals(rng, D, scale=0.02)
    outs = [3, 1, 5]
    x, caps = oracle.backbone_forward(x0, blocks, cfg, gh, gw, views, cam, ng, nb, True, outs)
    for feat, c in caps:
        assert feat.shape == (views, gh * gw, 2 * D) and c.shape == (views, 2 * D)
        assert np.isfinite(feat).all() and np.isfinite(c).all()
    assert not np.array_equal(caps[0][0], caps[1][0])
    assert not np.array_equal(caps[1][0], caps[2][0])
    # layer 3 is global: its local half is the stream after layer 2
    x2 = x0.reshape(-1, D)
    for layer in range(3):
        x2 = oracle.block_forward(x2, blocks[layer], cfg, layer, gh, gw, views, cam)["tokens"]
    assert np.array_equal(caps[0][0][:, :, :D], x2.reshape(views, n, D)[:, 2:])
    # the float64 twin
    x64, caps64 = backbone_f64(x0, blocks, cfg, gh, gw, views, cam, ng, nb, True, outs)
    assert np.max(np.abs(x - x64)) < 1e-5
    for (f, c), (f64, c64) in zip(caps, caps64):
        assert np.max(np.abs(f - f64)) < 2e-5 and np.max(np.abs(c - c64)) < 1e-5
    # without cat_token: single width, the camera row of the stream
    _, caps1 = oracle.backbone_forward(x0, blocks, cfg, gh, gw, views, cam, ng, nb, False, [4])
    assert caps1[0][0].shape == (views, gh * gw, D) and caps1[0][1].shape == (views, D)
