"""Writes the golden fixtures the oracle is pinned against.

Run from the repository root:  python tests/golden/make_golden.py

Two files:

* reference_kats.json -- the known-answer data held by the reference's own
  tests for this path (inputs and expected outputs transcribed as data):
    crates/da-engine/src/patch_embed.rs:280-339      patch projection KATs
    crates/da-engine/src/pos_embed.rs:326-442        pos-embed table + CLS KAT
    crates/da-engine/src/preprocess.rs:549-583       normalisation KAT
    crates/da-graph/tests/attention_and_layerscale_op.rs:5-31  LayerScale op
    da-parity/tests/compare_semantics.rs             comparator semantics
    docs/plans/2026-07-18-rust-engine-v1.md:776-791  GELU / LayerNorm KATs

* twins.npz -- float64 outputs of library routines computing the same
  mathematics independently of the oracle (torch on the CPU):
    torch.nn.functional.layer_norm   (block LN 768, Q/K LN 64)
    torch.nn.functional.gelu(approximate="none")   exact-erf GELU
    torch.nn.functional.interpolate(mode="bicubic", align_corners=False,
        scale_factor=((gh+0.1)/M, (gw+0.1)/M))      DINOv2 pos-embed resize
    torch.nn.functional.conv2d                       patch projection
  on small seeded inputs.
"""
import json
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
SEED = 20260812


def kats():
    img = np.zeros((3, 4, 4), np.float32)
    img[0] = np.arange(16, dtype=np.float32).reshape(4, 4)
    return {
        "patch_embed_bias_broadcast": {
            "source": "crates/da-engine/src/patch_embed.rs:280-303",
            "h": 4, "w": 4, "patch": 2, "embed": 3,
            "image_nchw": np.ones((3, 4, 4), np.float32).reshape(-1).tolist(),
            "weight_oihw": [0.0] * 36, "bias": [1.0, 2.0, 3.0],
            "expected_tokens": [[1.0, 2.0, 3.0]] * 4,
        },
        "patch_embed_row_major": {
            "source": "crates/da-engine/src/patch_embed.rs:305-339",
            "h": 4, "w": 4, "patch": 2, "embed": 1,
            "image_nchw": img.reshape(-1).tolist(),
            "weight_oihw": [1.0] * 4 + [0.0] * 8, "bias": [0.0],
            "expected_tokens": [[10.0], [18.0], [42.0], [50.0]],
        },
        "pos_embed_tokens": {
            "source": "crates/da-engine/src/pos_embed.rs:326-340,420-441",
            "grid": 3, "embed": 2,
            "pos_embed": [[float(r), -float(r)] for r in range(10)],
            "cls": [100.0, -100.0],
            "gh": 2, "gw": 2,
            "expected_row0": [100.0, -100.0],
            "native_grid_cls_row": [0.0, -0.0],
        },
        "normalize": {
            "source": "crates/da-engine/src/preprocess.rs:549-583",
            "h": 2, "w": 2,
            "hwc_u8": [255, 0, 0, 0, 255, 0, 0, 0, 255, 128, 128, 128],
            "mean": [0.485, 0.456, 0.406], "std": [0.229, 0.224, 0.225],
            "tolerance": 1e-6,
        },
        "layerscale_op": {
            "source": "crates/da-graph/tests/attention_and_layerscale_op.rs:5-31",
            "rows": 2, "cols": 3,
            "x": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "gamma": [10.0, -1.0, 0.5],
            "expected": [10.0, -2.0, 1.5, 40.0, -5.0, 3.0],
        },
        "compare_semantics": {
            "source": "da-parity/tests/compare_semantics.rs",
            "cases": [
                {"got": [1.0, 2.0, 3.0], "ref": [1.001, 1.999, 3.0], "atol": 2e-3, "rtol": 2e-3,
                 "ok": True},
                {"got": [1.0, 2.0, 5.0], "ref": [1.0, 2.0, 3.0], "atol": 2e-3, "rtol": 2e-3,
                 "ok": False, "worst": 2, "max_abs": 2.0},
                {"got": [], "ref": [], "atol": 1.0, "rtol": 1.0, "ok": False},
            ],
        },
        "gelu_kat": {
            "source": "docs/plans/2026-07-18-rust-engine-v1.md:776-783",
            "x": [0.0, 10.0, -10.0], "expected": [0.0, 10.0, 0.0], "tol": [1e-6, 1e-3, 1e-3],
        },
        "layernorm_kat": {
            "source": "docs/plans/2026-07-18-rust-engine-v1.md:785-791",
            "x": [1.0, 2.0, 3.0, 4.0], "eps": 1e-5, "mean_tol": 1e-4,
        },
        "rope_changes_output": {
            "source": "crates/da-graph/tests/attention_and_layerscale_op.rs:202-260",
            "heads": 1, "n": 2, "head_dim": 4, "pos_yx": [0, 0, 1, 2], "freq": 100.0,
        },
    }


def twins():
    rng = np.random.default_rng(SEED)
    out = {}
    # block LayerNorm, 7 rows x 768, eps 1e-6 (DA3 ln_eps)
    x = rng.standard_normal((7, 768)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(768)).astype(np.float32)
    b = (0.02 * rng.standard_normal(768)).astype(np.float32)
    out["ln768_x"], out["ln768_g"], out["ln768_b"] = x, g, b
    out["ln768_y64"] = F.layer_norm(torch.from_numpy(x).double(), (768,),
                                    torch.from_numpy(g).double(), torch.from_numpy(b).double(),
                                    1e-6).numpy()
    # Q/K LayerNorm rows of 64, eps 1e-5
    xq = (3.0 * rng.standard_normal((9, 64)) + 0.5).astype(np.float32)
    gq = (1 + 0.02 * rng.standard_normal(64)).astype(np.float32)
    bq = (0.02 * rng.standard_normal(64)).astype(np.float32)
    out["ln64_x"], out["ln64_g"], out["ln64_b"] = xq, gq, bq
    out["ln64_y64"] = F.layer_norm(torch.from_numpy(xq).double(), (64,),
                                   torch.from_numpy(gq).double(), torch.from_numpy(bq).double(),
                                   1e-5).numpy()
    # exact-erf GELU on a ramp and on normals
    xg = np.concatenate([np.linspace(-8, 8, 2001), rng.standard_normal(2000) * 2]).astype(np.float32)
    out["gelu_x"] = xg
    out["gelu_y64"] = F.gelu(torch.from_numpy(xg).double(), approximate="none").numpy()
    # DINOv2 bicubic pos-embed resize: 37x37 grid, embed 8, to 24x36 and 5x7
    M, E = 37, 8
    pe = (0.02 * rng.standard_normal((M * M + 1, E))).astype(np.float32)
    out["pe_src"] = pe
    for gh, gw in ((24, 36), (5, 7)):
        grid = torch.from_numpy(pe[1:]).double().reshape(1, M, M, E).permute(0, 3, 1, 2)
        sy, sx = (gh + 0.1) / M, (gw + 0.1) / M
        res = F.interpolate(grid, scale_factor=(sy, sx), mode="bicubic", align_corners=False)
        assert res.shape[-2:] == (gh, gw), res.shape
        out[f"pe_{gh}x{gw}_y64"] = res.permute(0, 2, 3, 1).reshape(gh * gw, E).numpy()
    # patch projection: 3x28x42 image (2x3 patches of 14), embed 16
    img = rng.standard_normal((3, 28, 42)).astype(np.float32)
    w = (0.02 * rng.standard_normal((16, 3, 14, 14))).astype(np.float32)
    bias = (0.02 * rng.standard_normal(16)).astype(np.float32)
    conv = F.conv2d(torch.from_numpy(img).double()[None], torch.from_numpy(w).double(),
                    torch.from_numpy(bias).double(), stride=14)
    out["conv_img"], out["conv_w"], out["conv_b"] = img, w, bias
    out["conv_y64"] = conv[0].reshape(16, -1).T.numpy()  # token-major [6, 16]
    return out


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(kats(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "twins.npz"), **twins())
    print("wrote", os.path.join(HERE, "reference_kats.json"), os.path.join(HERE, "twins.npz"))


if __name__ == "__main__":
    main()
