"""GPU parity of the attention core, `attention_online_f32` (vit_block.rs:363, 559;
CPU `vestra_kernels::attention`, vit_block.rs:952), through the C ABI.

The GPU computes every score and every probability-weighted sum as an F32
MFMA dot product and the softmax online (one pass over 64-key blocks), the
oracle sequentially in f32.  Both are compared with a bound derived from the
float64 result of the same inputs:

  |gpu - oracle| <= 1e-6 + 1e-5*|ref| + E * A + (2*sqrt(n) + nb + 4) * u * B

with u = 2^-24, nb the number of 64-key blocks, E = 8*u*max_j S_j + 4*u the
relative error of a probability (S_j = sum_d |q_d k_jd| / 8 is the size of a
score's terms: a 64-term dot product's rounding is about sqrt(64)*u of it;
4u covers expf and the subtraction), A = sum_j p_j |v_jd - o_d| (how much an
error in the weights moves the weighted mean) and B = sum_j p_j |v_jd| (the
size of the terms of the value sum and of its rescales).  A dropped scale, a
missed rescale or a mis-masked key moves results by 1e-2 or more, far above
this bound (about 1e-5 at n = 866).
"""
import numpy as np
import pytest

import oracle
from conftest import record_margin
from test_gpu_patch_block import normals

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")

U = 2.0 ** -24


def _reference_and_bound(q, k, v, rows=None):
    """float64 attention of one sequence [n, 64] (query rows `rows` only) and
    the parity bound above for those rows."""
    n = q.shape[0]
    qr = q if rows is None else q[rows]
    q64, k64, v64 = (x.astype(np.float64) for x in (qr, k, v))
    s = q64 @ k64.T / 8.0
    sabs = np.abs(q64) @ np.abs(k64).T / 8.0
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    o = p @ v64
    a = np.stack([p[i] @ np.abs(v64 - o[i]) for i in range(len(o))])
    b = p @ np.abs(v64)
    e = 8 * U * sabs.max(axis=1) + 4 * U
    nb = (n + 63) // 64
    return o, e[:, None] * a + (2 * np.sqrt(n) + nb + 4) * U * b


def _assert_attention(got, want, bound, label):
    tol = 1e-6 + 1e-5 * np.abs(want) + bound
    record_margin("attention", got, want, tol=tol, label=label)
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    worst = np.unravel_index(np.argmax(d / tol), d.shape)
    assert np.all(d <= tol), (f"[{label}] |d|={d[worst]:.3e} > tol={tol[worst]:.3e} at {worst} "
                              f"got={got[worst]!r} want={want[worst]!r}")


def _run(rt, q, k, v, seqs, n):
    return rt.attention_online_f32(rt.upload_f32(q), rt.upload_f32(k), rt.upload_f32(v), seqs,
                                   n, 64).numpy().reshape(seqs, n, 64)


@pytest.mark.parametrize("seqs,n", [(1, 1), (3, 37), (2, 64), (2, 65), (1, 129), (12, 866),
                                    (2, 1000), (1, 3000)])
def test_attention_matches_oracle(rt, rng, seqs, n):
    """Grids of fewer than two 64-query workgroups per CU split each tile's
    key blocks over workgroups: 12 x 866 in 3 splits, 2 x 1000 in 8 splits
    of 2 blocks, 1 x 3000 in 8 splits of 5-6 blocks (ending in the partial
    block); the others run one workgroup per tile."""
    q, k, v = (normals(rng, seqs, n, 64) for _ in range(3))
    got = _run(rt, q, k, v, seqs, n)
    want = oracle.attention(q, k, v, seqs, n, 64)
    for s in range(seqs):
        _, bound = _reference_and_bound(q[s], k[s], v[s])
        _assert_attention(got[s], want[s], bound, f"seq {s} n={n}")


def test_attention_local_layer_views_outer(rt, rng):
    """A local layer's batch [views, heads, tokens, 64] is views*heads
    sequences of one view each: no key of another view is attended."""
    views, heads, tpv = 3, 12, 866
    q, k, v = (normals(rng, views * heads, tpv, 64) for _ in range(3))
    got = _run(rt, q, k, v, views * heads, tpv)
    want = oracle.attention(q, k, v, views * heads, tpv, 64)
    for s in (0, heads - 1, heads, 2 * heads + 5, views * heads - 1):
        _, bound = _reference_and_bound(q[s], k[s], v[s])
        _assert_attention(got[s], want[s], bound, f"view {s // heads} head {s % heads}")


def test_attention_large_scores_and_selection(rt, rng):
    """Post-LayerNorm magnitudes (scores up to ~50) and one key that wins by a
    wide margin: its value row comes back."""
    n = 300
    q, k, v = (normals(rng, 1, n, 64) for _ in range(3))
    q *= 3.0
    k[0, 250] = q[0, 17] * 4.0  # block 3 holds the maximum of query 17
    got = _run(rt, q, k, v, 1, n)
    want = oracle.attention(q, k, v, 1, n, 64)
    _, bound = _reference_and_bound(q[0], k[0], v[0])
    _assert_attention(got[0], want[0], bound, "large scores")
    assert np.allclose(got[0, 17], v[0, 250], rtol=0, atol=1e-6)


@pytest.mark.parametrize("heads,n", [(12, 10392), (16, 3458), (12, 13856), (12, 20784)])
def test_attention_full_size_sampled_rows(rt, rng, heads, n):
    """Global layer of the 12-view ViT-B sequence (12 heads over 10,392 rows,
    each query tile's key blocks in three splits), the ViT-L 1008x672 image
    (16 heads over 3,458 rows, two splits) and the global layers of 16 and 24
    views (13,856 and 20,784 rows: five and four splits): every head, 48
    sampled query rows (first, last, the special tokens, view boundaries)
    against float64 with the bound above."""
    q, k, v = (normals(rng, heads, n, 64) for _ in range(3))
    got = _run(rt, q, k, v, heads, n)
    assert np.isfinite(got).all()
    fixed = [0, 1, 2, 865, 866, 867, n - 2, n - 1]
    for h in range(heads):
        rows = np.unique(np.concatenate([fixed, rng.integers(0, n, 40)]))
        ref, bound = _reference_and_bound(q[h], k[h], v[h], rows)
        # the oracle's own rounding sits inside the same bound
        _assert_attention(got[h][rows], ref.astype(np.float32), 2 * bound, f"head {h}")


def test_attention_into_and_key_permutation(rt, rng):
    """The `into` form writes a caller tensor; permuting keys together with
    their values changes the result by rounding only."""
    n = 200
    q, k, v = (normals(rng, 2, n, 64) for _ in range(3))
    out = rt.alloc_f32(2 * n * 64)
    rt.attention_into_f32(rt.upload_f32(q), rt.upload_f32(k), rt.upload_f32(v), 2, n, 64, out)
    a = out.numpy().reshape(2, n, 64)
    assert np.array_equal(a, _run(rt, q, k, v, 2, n))
    perm = rng.permutation(n)
    b = _run(rt, q, k[:, perm], v[:, perm], 2, n)
    _, bound = _reference_and_bound(q[0], k[0], v[0])
    _assert_attention(b[0], a[0], 2 * bound, "permuted keys")


def test_attention_edges_and_errors(rt):
    empty = rt.alloc_f32(0)
    rt.attention_into_f32(empty, empty, empty, 12, 0, 64, rt.alloc_f32(0))
    rt.attention_into_f32(empty, empty, empty, 0, 866, 64, rt.alloc_f32(0))
    x = rt.alloc_f32(2 * 5 * 32)
    with pytest.raises(vh.UnsupportedShape):
        rt.attention_online_f32(x, x, x, 2, 5, 32)            # head_dim 32
    y = rt.alloc_f32(2 * 5 * 64)
    with pytest.raises(vh.VestraError):
        rt.attention_online_f32(y, y, y, 2, 6, 64)            # size mismatch
    with pytest.raises(vh.VestraError):
        rt.attention_into_f32(y, y, y, 2, 5, 64, y)           # out overlaps q


def test_attention_key_split_capture_rules(rng):
    """One image's attention (12 x 866: three key splits per query tile)
    keeps its partial results in the runtime's work buffer: the first call
    inside a stream capture is refused, a graph captured after an eager call
    replays the eager result bit for bit."""
    import gc
    rt = vh.Runtime(0)  # fresh runtime: no work buffer yet
    _key_split_case(rt, rng)
    gc.collect()
    rt.close()


def _key_split_case(rt, rng):
    import gc
    seqs, n = 12, 866
    q, k, v = (rt.upload_f32(normals(rng, seqs, n, 64)) for _ in range(3))
    out = rt.alloc_f32(seqs * n * 64)

    def step():
        rt.attention_into_f32(q, k, v, seqs, n, 64, out)

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
    rt.synchronize()
    gc.disable()
    try:
        rt.begin_capture()
        step()
        graph = rt.end_capture()
    finally:
        gc.enable()
    for _ in range(3):
        out.write(np.zeros(seqs * n * 64, np.float32))
        graph.launch()
        rt.synchronize()
        assert np.array_equal(out.numpy(), want)
