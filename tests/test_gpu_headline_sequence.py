"""The benchmark's timed sequences compared with the oracle, block by block.

bench.py times the fused-op sequence of every block as bench.Model issues it
(block_plan: LayerScale + residual fused with LN2, the LS2 residual fused with
the next block's LN1 -- before the camera-slot layer alt_start that pass also
writes the camera slot -- global layers on the flattened views and local ones
in the views-outer Q/K layout).  These tests issue the same Model block by block and
chain the oracle's block_fused_ops beside it (the reference order of
vit_block.rs:1019-1139 over the multi-view batch of backbone.rs:688-877),
checking every output after every block at rtol 1e-5 / atol 1e-6:

  * ViT-B 504x336, 12 views x 866 tokens = 10,392 rows, 12 blocks (the
    headline workload), f32 parameters;
  * ViT-L 1008x672, 3,458 rows, 24 blocks, parameter vectors stored as F16
    (GGUF F16 element layout, widened exactly; reader.rs:303-318).

The projections' and attention's outputs between the operations are the
seeded tensors the benchmark holds: q, k and hidden are the same buffers for
every block and are transformed in place again by each one (in the model
each block gets fresh ones from its projections).  Per block the oracle
therefore takes the device's q, k and hidden as the block found them, and
every output must meet the bar; the residual stream carries no reduction
(LayerScale + residual, the camera write), so the device tokens must stay
bit-identical to the oracle's chained tokens through all blocks, and LN1 /
LN2 of them meet the bar.  Besides, a free-running oracle chain of q, k and
hidden (twelve or twenty-four re-normalisations and GELUs of the same
buffers, each adding its rounding differences) is compared at the end
within atol 1e-5.  After a block whose LS2 residual is fused with the next
LN1, the LN1 buffer holds the next block's LN1 of the new tokens (with the
camera slot written when the next block is alt_start).
"""
import numpy as np
import pytest

import oracle
from conftest import F32_ATOL, F32_RTOL, assert_parity

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")
import bench  # noqa: E402


CHAIN_ATOL = 1e-5  # free-running q/k/hidden chain: accumulated over every block


def with_camera(tokens, camera, views):
    """tokens [rows, D] with row 0 of every view replaced by the camera
    token: slot 0 for view 0, slot 1 for the others (backbone.rs:746-768)."""
    out = tokens.copy()
    D = out.shape[1]
    tpv = out.shape[0] // views
    cam = np.asarray(camera, np.float32).reshape(-1)
    for v in range(views):
        out[v * tpv] = cam[D:2 * D] if v > 0 else cam[:D]
    return out


def run_chain(rt, rng, views, shape, f16, exact=()):
    """Issue the benchmark's blocks one by one beside the oracle's chain;
    outputs named in `exact` must equal the oracle's bits (the rest meet
    the F32 bar)."""
    model = bench.Model(rt, rng, views=views, shape=shape, f16=f16)
    host = model.host_act
    tokens = host["tokens"].copy()
    free = {n: host[n].copy() for n in ("q", "k", "hidden")}
    dev_prev = {n: host[n].copy() for n in ("q", "k", "hidden")}
    eps = model.cfg_dict["ln_eps"]
    for i, flags in enumerate(model.plan):
        print(f"block {i} flags {flags} rows {model.rows}", flush=True)

        def ora(q, k, hidden):
            return oracle.block_fused_ops(tokens, q, k, host["attn_proj"], hidden,
                                          host["mlp_out"], model.host_layers[i], model.cfg_dict,
                                          i, shape.gh, shape.gw, views, model.camera_host)

        ref = ora(dev_prev["q"], dev_prev["k"], dev_prev["hidden"])
        free_ref = ora(free["q"], free["k"], free["hidden"])
        model.enqueue_block(i)
        got = {n: model.act[n].numpy() for n in ("tokens", "ln1", "ln2", "q", "k", "hidden")}
        want_tokens = ref["tokens"]
        if flags & vh.VK_BLOCK_FUSE_NEXT_LN1:
            if i + 1 == shape.alt:  # the camera slot, written by this block's last pass
                want_tokens = with_camera(want_tokens, model.camera_host, views)
            nl = model.host_layers[i + 1]
            ln1 = oracle.layernorm(want_tokens, nl["norm1_gamma"], nl["norm1_beta"], eps)
        else:
            ln1 = ref["ln1"]
        assert np.array_equal(got["tokens"].reshape(want_tokens.shape), want_tokens), \
            f"tokens after block {i} differ from the oracle's chained residual stream"
        expect = {"ln1": ln1, "ln2": ref["ln2"], "q": ref["q"], "k": ref["k"],
                  "hidden": ref["hidden"]}
        for name, want in expect.items():
            if name in exact:
                assert np.array_equal(got[name].reshape(-1), np.asarray(want).reshape(-1)), \
                    f"{name} after block {i} differs from the oracle's bits"
            else:
                assert_parity(got[name], want, F32_ATOL, F32_RTOL, f"{name} after block {i}")
        tokens = ref["tokens"]
        dev_prev = {n: got[n] for n in ("q", "k", "hidden")}
        free = {n: free_ref[n] for n in ("q", "k", "hidden")}
    for name in ("q", "k", "hidden"):
        assert_parity(dev_prev[name], free[name], CHAIN_ATOL, F32_RTOL,
                      f"{name} after {len(model.plan)} chained blocks")
    return model


def test_vitb_12_views_12_blocks_as_benchmarked(rt, rng):
    model = run_chain(rt, rng, 12, bench.VITB, f16=False)
    assert model.rows == 10392
    # the camera slot was written before alt_start by the previous block's
    # fused pass: row 0 of view 0 from slot 0, row 0 of the other views from
    # slot 1, then carried by the residual adds
    assert model.plan[bench.ALT] & vh.VK_BLOCK_CAMERA_WRITTEN
    assert model.plan[bench.ALT - 1] & vh.VK_BLOCK_FUSE_NEXT_LN1


def test_vitl_3458_rows_24_blocks_f16_parameters(rt, rng):
    model = run_chain(rt, rng, 1, bench.VITL, f16=True)
    assert model.rows == 3458
    assert all(v.dtype == np.float16 for v in model.host_layers[0].values())


@pytest.mark.parametrize("views", [1, 3])
def test_camera_write_fused_into_the_previous_pass(rt, rng, views):
    """The block before alt_start fusing its LS2 residual with the next LN1
    also writes the camera slot (VK_BLOCK_FUSE_NEXT_LN1 with a camera token),
    and the block at alt_start then skips the write and its LN1
    (VK_BLOCK_SKIP_LN1 | VK_BLOCK_CAMERA_WRITTEN): every output after both
    blocks is bit-identical to the unfused order (LS2 residual; camera write
    and LN1 in the block at alt_start)."""
    outs = []
    for fused in (False, True):
        r = np.random.default_rng(7)
        model = bench.Model(rt, r, views=views)
        alt = bench.ALT
        for i in range(alt + 1):
            flags = model.plan[i]
            if not fused and i == alt - 1:
                flags &= ~vh.VK_BLOCK_FUSE_NEXT_LN1
            if not fused and i == alt:
                flags &= ~(vh.VK_BLOCK_SKIP_LN1 | vh.VK_BLOCK_CAMERA_WRITTEN)
            nxt = model.structs[i + 1]
            model.rt.vit_block_fused_ops(model.cfg, i, model.structs[i], nxt, model.act_struct,
                                         model.shape.gh, model.shape.gw, views, model.camera,
                                         flags)
        outs.append({n: model.act[n].numpy() for n in ("tokens", "ln1", "ln2", "q", "k",
                                                          "hidden")})
    for n in outs[0]:
        assert np.array_equal(outs[0][n], outs[1][n]), n


@pytest.mark.parametrize("layer,flags", [
    (bench.ALT, vh.VK_BLOCK_CAMERA_WRITTEN),                          # without SKIP_LN1
    (bench.ALT, vh.VK_BLOCK_CAMERA_WRITTEN | vh.VK_BLOCK_FUSE_LS_LN),
    (bench.ALT + 1, vh.VK_BLOCK_CAMERA_WRITTEN | vh.VK_BLOCK_SKIP_LN1),  # not at alt_start
    (0, vh.VK_BLOCK_CAMERA_WRITTEN | vh.VK_BLOCK_SKIP_LN1),
])
def test_camera_written_flag_rejected_out_of_place(rt, rng, layer, flags):
    """VK_BLOCK_CAMERA_WRITTEN is taken only together with VK_BLOCK_SKIP_LN1
    at layer alt_start; any other use is an argument error raised before
    anything is enqueued (the tokens stay as they were)."""
    model = bench.Model(rt, rng, views=1)
    before = model.act["tokens"].numpy()
    with pytest.raises(vh.VestraError, match="CAMERA_WRITTEN"):
        model.rt.vit_block_fused_ops(model.cfg, layer, model.structs[layer],
                                     model.structs[layer + 1], model.act_struct,
                                     model.shape.gh, model.shape.gw, 1, model.camera, flags)
    assert np.array_equal(model.act["tokens"].numpy(), before)
