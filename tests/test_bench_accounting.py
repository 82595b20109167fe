"""The benchmark line's byte accounting, restated independently.

value = algorithmic bytes of one step / step time, so the step's byte count
is checked here against the per-operation formulas (each tensor read or
written once, f32 activations, parameter vectors of w bytes per element),
summed over the launches the block plan issues: 12 ViT-B blocks over 12
views of 866 tokens, LayerScale + residual fused with the following
LayerNorm, the camera slot written inside the pass before alt_start.
"""
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
