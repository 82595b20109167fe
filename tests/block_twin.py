"""float64 twin of one whole DA3 ViT block and seeded block parameters.

Shared by the oracle pins (CPU) and the GPU block tests.  The twin follows the
same steps as the oracle's block composition (vit_block.rs:1019-1139):
LayerNorm with the two-pass biased variance, [in, out] projections, per
(head, token) Q/K LayerNorm, the 2D rotation with the oracle's f32 angles
(cos/sin in float64, unrounded), softmax attention per head (per view for
local layers), the A&S 7.1.26 GELU, LayerScale and residual adds -- all in
float64.
"""
import math

import numpy as np

import oracle


def normals(rng, *shape, scale=1.0, shift=0.0):
    return (shift + scale * rng.standard_normal(shape)).astype(np.float32)


def make_params(rng, D, M, with_qkn=True, with_ls=True):
    p = {"norm1_gamma": normals(rng, D, scale=0.02, shift=1), "norm1_beta": normals(rng, D, scale=0.02),
         "qkv_w": normals(rng, D, 3 * D, scale=0.02), "qkv_b": normals(rng, 3 * D, scale=0.02),
         "proj_w": normals(rng, D, D, scale=0.02), "proj_b": normals(rng, D, scale=0.02),
         "norm2_gamma": normals(rng, D, scale=0.02, shift=1), "norm2_beta": normals(rng, D, scale=0.02),
         "fc1_w": normals(rng, D, M, scale=0.02), "fc1_b": normals(rng, M, scale=0.02),
         "fc2_w": normals(rng, M, D, scale=0.02), "fc2_b": normals(rng, D, scale=0.02)}
    if with_qkn:
        p.update({"qnorm_gamma": normals(rng, 64, scale=0.02, shift=1),
                  "qnorm_beta": normals(rng, 64, scale=0.02),
                  "knorm_gamma": normals(rng, 64, scale=0.02, shift=1),
                  "knorm_beta": normals(rng, 64, scale=0.02)})
    if with_ls:
        p["ls1"] = rng.uniform(0, 0.1, D).astype(np.float32)
        p["ls2"] = rng.uniform(0, 0.1, D).astype(np.float32)
    return p


def config(D, H, M, nreg=1, alt=4, rope_start=0, qknorm_start=0, rope_mode=0):
    return dict(embed_dim=D, num_heads=H, head_dim=64, mlp_hidden=M, num_register=nreg,
                ln_eps=1e-6, qk_norm_eps=1e-5, rope_freq=100.0, rope_start=rope_start,
                qknorm_start=qknorm_start, alt_start=alt, rope_mode=rope_mode)


def is_global(cfg, layer):
    return cfg["alt_start"] >= 0 and layer >= cfg["alt_start"] and layer % 2 == 1


# ---------------------------------------------------------------- float64 twin
def _ln64(x, g, b, eps):
    m = x.mean(axis=-1, keepdims=True)
    var = ((x - m) ** 2).mean(axis=-1, keepdims=True)
    return (x - m) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)


def _gelu64(x):
    a = np.abs(x) / math.sqrt(2.0)
    t = 1.0 / (1.0 + 0.3275911 * a)
    poly = ((((1.0614054 * t - 1.4531520) * t + 1.4214137) * t - 0.28449674) * t
            + 0.25482959) * t
    erf = np.sign(x) * (1.0 - poly * np.exp(-a * a))
    return 0.5 * x * (1.0 + erf)


def _rope64(x, pos, inv_freq, mode=0):
    # pairs (j, j+16) of each half, or (2j, 2j+1) with the interleaved flag
    first = np.arange(16) * 2 if mode & oracle.ROPE_INTERLEAVED else np.arange(16)
    second = first + 1 if mode & oracle.ROPE_INTERLEAVED else first + 16
    out = x.copy()
    for base, coord in ((0, 0), (32, 1)):
        p = pos[:, coord].astype(np.float32)
        ang = (p[:, None] * inv_freq[None, :]).astype(np.float32).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        a, b = x[..., base + first], x[..., base + second]
        out[..., base + first] = a * c - b * s
        out[..., base + second] = b * c + a * s
    return out


def _attn64(q, k, v):
    s = q @ np.swapaxes(k, -1, -2) / 8.0
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(axis=-1, keepdims=True)) @ v


def block_f64(tokens, p, cfg, layer, gh, gw, views, camera=None):
    D, H = cfg["embed_dim"], cfg["num_heads"]
    ns = 1 + cfg["num_register"]
    tpv = ns + gh * gw
    rows = tpv * views
    glob = is_global(cfg, layer)
    f = {k: np.asarray(v, np.float64) for k, v in p.items()}
    x = tokens.astype(np.float64).reshape(rows, D).copy()
    if cfg["alt_start"] >= 0 and layer == cfg["alt_start"]:
        for v in range(views):
            x[v * tpv] = camera.reshape(-1)[(1 if v else 0) * D:((1 if v else 0) + 1) * D]
    qkv = _ln64(x, f["norm1_gamma"], f["norm1_beta"], cfg["ln_eps"]) @ f["qkv_w"] + f["qkv_b"]
    q, k, v = (qkv[:, i * D:(i + 1) * D].reshape(rows, H, 64).transpose(1, 0, 2)
               for i in range(3))
    if cfg["qknorm_start"] >= 0 and layer >= cfg["qknorm_start"] and "qnorm_gamma" in p:
        q = _ln64(q, f["qnorm_gamma"], f["qnorm_beta"], cfg["qk_norm_eps"])
        k = _ln64(k, f["knorm_gamma"], f["knorm_beta"], cfg["qk_norm_eps"])
    if cfg["rope_start"] >= 0 and layer >= cfg["rope_start"]:
        pos = oracle.rope_positions(ns, gh, gw, views, glob)
        mode = cfg.get("rope_mode", 0)
        inv = oracle.rope_inv_freq(64, cfg["rope_freq"], mode)
        q, k = _rope64(q, pos, inv, mode), _rope64(k, pos, inv, mode)
    if glob:
        attn = _attn64(q, k, v)
    else:
        sh = (H * views, tpv, 64)
        attn = _attn64(q.reshape(sh), k.reshape(sh), v.reshape(sh)).reshape(H, rows, 64)
    y = attn.transpose(1, 0, 2).reshape(rows, D) @ f["proj_w"] + f["proj_b"]
    x = x + (y * f["ls1"] if "ls1" in p else y)
    ln2 = _ln64(x, f["norm2_gamma"], f["norm2_beta"], cfg["ln_eps"])
    hidden = _gelu64(ln2 @ f["fc1_w"] + f["fc1_b"])
    y = hidden @ f["fc2_w"] + f["fc2_b"]
    x = x + (y * f["ls2"] if "ls2" in p else y)
    return {"tokens": x, "q": q, "k": k, "v": v, "attn": attn, "ln2": ln2, "hidden": hidden}




def backbone_f64(tokens, blocks, cfg, gh, gw, views, camera, norm_gamma, norm_beta, cat,
                 out_layers):
    """float64 twin of the backbone block loop with its captures
    (backbone.rs:688-877, 1139-1179)."""
    D = cfg["embed_dim"]
    ns = 1 + cfg["num_register"]
    n = ns + gh * gw
    x = tokens.astype(np.float64).reshape(n * views, D)
    local = x.copy()
    out = [None] * len(out_layers)
    for layer, p in enumerate(blocks):
        x = block_f64(x, p, cfg, layer, gh, gw, views, camera)["tokens"]
        glob = is_global(cfg, layer)
        for i, want in enumerate(out_layers):
            if want != layer:
                continue
            xv = x.reshape(views, n, D)
            lv = (local if glob else x).reshape(views, n, D)
            normed = _ln64(xv[:, ns:], norm_gamma.astype(np.float64),
                           norm_beta.astype(np.float64), cfg["ln_eps"])
            if cat:
                out[i] = (np.concatenate([lv[:, ns:], normed], axis=2),
                          np.concatenate([lv[:, 0], xv[:, 0]], axis=1))
            else:
                out[i] = (normed, xv[:, 0].copy())
        if not glob:
            local = x.copy()
    return x, out
