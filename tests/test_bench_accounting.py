"""The benchmark line's byte accounting, restated independently.

value = algorithmic bytes of one step / step time, so the step's byte count
is checked here against the per-operation formulas (each tensor read or
written once, f32 activations, parameter vectors of w bytes per element),
summed over the launches the block plan issues: 12 ViT-B blocks over 12
views of 866 tokens, LayerScale + residual fused with the following
LayerNorm, the camera slot written inside the pass before alt_start.
"""
import numpy as np
import pytest

vh = pytest.importorskip("vestra_hip")
import bench  # noqa: E402

D, H, M, HD = 768, 12, 3072, 64


def ln(n, w=4):
    return 2 * n * D * 4 + 2 * D * w                 # x read, y written, gamma, beta


def ls_res(n, w=4):
    return 3 * n * D * 4 + D * w                     # x read and written, branch read, gamma


def ls_res_ln(n, w=4):
    return 4 * n * D * 4 + 3 * D * w                 # + LN output written, LN gamma/beta


def qk(n, w=4):
    return 2 * (2 * H * n * HD * 4) + 4 * HD * w     # Q and K read and written in place


def gelu(n):
    return 2 * n * M * 4


def test_block_plan_flags():
    plan = bench.block_plan(12, 4)
    base = vh.VK_BLOCK_FUSE_LS_LN
    assert plan[0] == base | vh.VK_BLOCK_FUSE_NEXT_LN1
    assert plan[4] == (base | vh.VK_BLOCK_SKIP_LN1 | vh.VK_BLOCK_CAMERA_WRITTEN
                       | vh.VK_BLOCK_FUSE_NEXT_LN1)
    assert plan[11] == base | vh.VK_BLOCK_SKIP_LN1
    for i in (1, 2, 3, 5, 10):
        assert plan[i] == base | vh.VK_BLOCK_SKIP_LN1 | vh.VK_BLOCK_FUSE_NEXT_LN1


@pytest.mark.parametrize("views", [1, 12])
def test_step_bytes_match_the_launches(views):
    n = views * 866
    want = ln(n)                                     # block 0's LN1
    for i in range(12):
        want += qk(n) + ls_res_ln(n) + gelu(n)       # Q/K, LS1+res+LN2, GELU
        want += ls_res_ln(n) if i < 11 else ls_res(n)
    want += views * D * 4                            # the camera token read into each view's slot
    assert bench.step_bytes(n, views, bench.block_plan(12, 4)) == want


def test_step_bytes_without_the_camera_fusion():
    # the unfused order: LS2+res before the camera layer, then the camera
    # copy (read and write of each view's slot) and LN1 at alt_start
    n = 12 * 866
    plan = bench.block_plan(12, 4)
    plan[3] &= ~vh.VK_BLOCK_FUSE_NEXT_LN1
    plan[4] &= ~(vh.VK_BLOCK_SKIP_LN1 | vh.VK_BLOCK_CAMERA_WRITTEN)
    fused = bench.step_bytes(n, 12, bench.block_plan(12, 4))
    unfused = bench.step_bytes(n, 12, plan)
    assert unfused - fused == (ls_res(n) + 2 * 12 * D * 4 + ln(n)) - (ls_res_ln(n) + 12 * D * 4)
    assert unfused == 7725969408   # the headline's bytes per step before the fusion


def test_step_launches_and_the_dominant_kernel():
    plan = bench.block_plan(12, 4)
    n = bench.step_launches(plan)
    # LN1 of block 0; LS1+res+LN2 in every block and LS2+res+LN1 (next) in
    # all but the last, whose LS2+res stands alone; the camera slot inside
    # the fused pass before alt_start
    assert n == {"layernorm": 1, "qk_norm_rope": 12, "layerscale_residual_layernorm": 23,
                 "gelu": 12, "layerscale_residual": 1, "camera_copy": 0}

    def entry(us, nbytes):
        return {"us": us, "bytes": nbytes, "GB_s": nbytes / us / 1e3}

    # per-launch times of the committed headline profile: the fused
    # LayerScale + LayerNorm dominates (23 x 23.2 us against 12 x 39.7 us)
    ops = {"layernorm": entry(12.9, ln(10392)), "qk_norm_rope": entry(22.1, qk(10392)),
           "layerscale_residual_layernorm": entry(23.2, ls_res_ln(10392)),
           "gelu": entry(39.7, gelu(10392)), "layerscale_residual": entry(16.8, ls_res(10392))}
    r = bench.roofline_entry(ops, plan)
    assert r["kernel"].startswith("ls_residual_layernorm_rows")
    assert r["launches_per_step"] == 23
    assert r["frac"] == round(ls_res_ln(10392) / 23.2e-6 / 8e12, 4)
    assert r["next"]["kernel"].startswith("gelu_kernel")
    assert abs(sum(r["share_of_op_time"].values()) - 1) < 1e-2
    # a slower GELU takes the roofline over
    ops["gelu"] = entry(50.0, gelu(10392))
    assert bench.roofline_entry(ops, plan)["kernel"].startswith("gelu_kernel")


def test_record_margin_shapes():
    from conftest import _MARGINS, record_margin
    got = np.ones((3, 4))
    ref = got + 1e-7
    r = record_margin("_selftest", got, ref, tol=np.full((3, 4), 2e-7))
    assert abs(r["bound_used"] - 0.5) < 1e-6 and r["max_abs"] > 0
    r = record_margin("_selftest", got.ravel(), ref, atol=1e-6, rtol=0.0)
    assert abs(r["bound_used"] - 0.1) < 1e-6
    assert abs(r["max_rel_ref_ge_1e-3"] - 1e-7) < 1e-9
    _MARGINS.pop("_selftest")
