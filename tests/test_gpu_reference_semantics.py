"""Device counterparts of the reference's own semantic tests of this path.

* Q/K-norm eps discriminator (crates/da-graph/tests/attention_and_layerscale_op.rs:91-196):
  on rows whose variance is of the order of the two candidate eps values, the
  device Q/K LayerNorm must match eps = 1e-5 (QK_NORM_EPS, vit_block.rs:681-686)
  and must not match eps = 1e-6 (the model's ln_eps).
* Global attention couples the views, local attention does not
  (backbone.rs:1421-1443): after a global block, changing one view's tokens
  changes the other views' outputs; after a local block the other views keep
  their bits.
"""
import numpy as np
import pytest

import oracle
from block_twin import config, is_global, make_params, normals
from conftest import F32_ATOL, F32_RTOL, assert_parity, parity_report
from test_gpu_block_forward import DeviceBlock

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


def test_qk_norm_eps_discriminator(rt, rng):
    heads, n, hd = 12, 866, 64
    # zero-mean rows with a standard deviation of 1e-3: variance 1e-6, so
    # 1/sqrt(var + eps) is about 302 for eps 1e-5 and 707 for eps 1e-6
    q = rng.normal(0.0, 1e-3, (heads * n, hd)).astype(np.float32)
    k = rng.normal(0.0, 1e-3, (heads * n, hd)).astype(np.float32)
    qg, qb = normals(rng, hd, scale=0.02, shift=1), normals(rng, hd, scale=0.02)
    kg, kb = normals(rng, hd, scale=0.02, shift=1), normals(rng, hd, scale=0.02)
    # every position (0, 0): the rotation is the identity, exactly
    pos = np.zeros(n * 2, np.float32)
    qd, kd = rt.upload_f32(q), rt.upload_f32(k)
    rt.qk_norm_rope_f32_da3_base(qd, kd, rt.upload_f32(qg), rt.upload_f32(qb),
                                 rt.upload_f32(kg), rt.upload_f32(kb), rt.upload_f32(pos),
                                 heads, n, 100.0, 1e-5)
    for name, got, x, g, b in (("q", qd, q, qg, qb), ("k", kd, k, kg, kb)):
        y = got.numpy().reshape(heads * n, hd)
        assert_parity(y, oracle.layernorm(x, g, b, 1e-5), F32_ATOL, F32_RTOL,
                      f"{name}: eps 1e-5")
        ok, max_abs, _ = parity_report(y, oracle.layernorm(x, g, b, 1e-6), F32_ATOL, F32_RTOL)
        assert not ok and max_abs > 0.1, f"{name}: indistinguishable from eps 1e-6"


@pytest.mark.parametrize("layer", [1, 3])
def test_global_layers_couple_views(rt, rng, layer):
    D, H, M, gh, gw, views = 768, 12, 3072, 4, 6, 2
    cfg = config(D, H, M, alt=2)  # layer 1 local, layer 3 global
    glob = is_global(cfg, layer)
    assert glob == (layer == 3)
    tpv = 2 + gh * gw
    dev = DeviceBlock(rt, make_params(rng, D, M), D, M)
    cam = rt.upload_f32(normals(rng, 2 * D))
    x0 = normals(rng, views * tpv, D)
    x1 = x0.copy()
    x1[tpv + 2:] += normals(rng, tpv - 2, D)  # view 1's patch tokens only
    outs = []
    for x in (x0, x1):
        t, ws = rt.upload_f32(x), rt.block_workspace(views * tpv, D, M)
        rt.vit_block_forward_f32(vh.VitConfig(**cfg), layer, dev.struct, t, gh, gw, views, cam,
                                 ws.struct)
        outs.append(t.numpy().reshape(views, tpv, D))
    assert not np.array_equal(outs[0][1], outs[1][1]), "view 1 must change"
    if glob:
        assert np.max(np.abs(outs[0][0] - outs[1][0])) > 1e-4, \
            "a global layer must carry view 1's change into view 0"
    else:
        assert np.array_equal(outs[0][0], outs[1][0]), \
            "a local layer must leave view 0 untouched"
