"""The oracle: numpy front end of the scalar CPU restatement (vestra_oracle.c).

TEST INFRASTRUCTURE ONLY.  This package is the checker that the HIP library
is compared against.  It is imported by tests/, by __graft_entry__.smoke() to
check one small GPU invocation, and by bench.py's cpu_baseline leg (which
times it as the reported CPU baseline).  The product path never imports it.

Each wrapper names the reference function it restates; the C source cites
file:line for every formula.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvestra_oracle.so")


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        build()
    return C.CDLL(LIB_PATH)


lib = _load()

_vp, _sz, _i, _f = C.c_void_p, C.c_size_t, C.c_int, C.c_float
_SIGS = {
    "ora_set_threads": ([_i], None),
    "ora_get_threads": ([], _i),
    "ora_f16_to_f32": ([C.c_uint16], _f),
    "ora_f16_to_f32_array": ([_vp, _vp, _sz], None),
    "ora_layernorm_f32": ([_vp, _vp, _sz, _sz, _vp, _vp, _f], None),
    "ora_layernorm_w16": ([_vp, _vp, _sz, _sz, _vp, _vp, _f], None),
    "ora_erf_as7126": ([_f], _f),
    "ora_gelu_f32": ([_vp, _sz], None),
    "ora_gelu_erff_f32": ([_vp, _sz], None),
    "ora_layerscale_f32": ([_vp, _sz, _sz, _vp], None),
    "ora_add_f32": ([_vp, _vp, _sz], None),
    "ora_layerscale_residual_f32": ([_vp, _vp, _vp, _sz, _sz], None),
    "ora_layerscale_residual_w16": ([_vp, _vp, _vp, _sz, _sz], None),
    "ora_rope_positions": ([_vp, _sz, _sz, _sz, _sz, _i], None),
    "ora_rope_inv_freq": ([_vp, _sz, _f], None),
    "ora_rope_inv_freq_mode": ([_vp, _sz, _f, C.c_uint], None),
    "ora_rope2d_f32": ([_vp, _sz, _sz, _sz, _vp, _f], None),
    "ora_rope2d_mode_f32": ([_vp, _sz, _sz, _sz, _vp, _f, C.c_uint], None),
    "ora_qk_norm_rope_f32": ([_vp] * 7 + [_sz, _sz, _sz, _f, _f], None),
    "ora_qk_norm_rope_mode_f32": ([_vp] * 7 + [_sz, _sz, _sz, _f, _f, C.c_uint], None),
    "ora_qk_norm_rope_w16": ([_vp] * 7 + [_sz, _sz, _sz, _f, _f, C.c_uint], None),
    "ora_normalize_u8_hwc": ([_vp, _vp, _sz, _sz, _vp, _vp], None),
    "ora_patchify_nchw": ([_vp, _vp, _sz, _sz, _sz, _sz], None),
    "ora_linear_f32": ([_vp, _vp, _vp, _vp, _sz, _sz, _sz], None),
    "ora_patch_project_oihw": ([_vp, _sz, _sz, _sz, _vp, _vp, _sz, _vp], None),
    "ora_pos_embed_bicubic": ([_vp, _sz, _sz, _sz, _sz, _f, _vp], None),
    "ora_assemble_tokens": ([_vp, _sz, _sz, _sz, _vp, _vp, _sz, _vp, _vp], None),
    "ora_patch_embed_u8": ([_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _sz, _vp, _vp, _sz, _vp,
                            _vp], None),
    "ora_overwrite_prefix_f32": ([_vp, _vp, _sz], None),
    "ora_split_qkv_hnd": ([_vp, _sz, _sz, _sz, _vp, _vp, _vp], None),
    "ora_hnd_to_token": ([_vp, _sz, _sz, _sz, _vp], None),
    "ora_attention_f32": ([_vp, _vp, _vp, _sz, _sz, _sz, _vp], None),
    "ora_resize_bilinear_u8": ([_vp, _sz, _sz, _vp, _sz, _sz], None),
    "ora_resize_cubic_u8": ([_vp, _sz, _sz, _vp, _sz, _sz], None),
    "ora_resize_area_u8": ([_vp, _sz, _sz, _vp, _sz, _sz], None),
    "ora_preprocess_shape": ([_sz, _sz, _sz, _sz, _i, _vp], _i),
    "ora_preprocess_resize_u8": ([_vp, _sz, _sz, _sz, _sz, _i, _vp], None),
}
for _n, (_a, _r) in _SIGS.items():
    _fn = getattr(lib, _n)
    _fn.argtypes = _a
    _fn.restype = _r


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    # data_as keeps a reference to the array alive as long as the pointer
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def set_threads(n: int) -> None:
    lib.ora_set_threads(int(n))


def f16_bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib.ora_f16_to_f32_array(_p(b), _p(out), b.size)
    return out


def layernorm(x, gamma, beta, eps: float) -> np.ndarray:
    """scalar::layernorm over the last axis (vit_block.rs:696-714)."""
    x = _f32(x)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty_like(x)
    if np.asarray(gamma).dtype == np.float16:
        g, b = f16_bits(gamma), f16_bits(beta)
        lib.ora_layernorm_w16(_p(x), _p(out), rows, cols, _p(g), _p(b), eps)
    else:
        g, b = _f32(gamma), _f32(beta)
        lib.ora_layernorm_f32(_p(x), _p(out), rows, cols, _p(g), _p(b), eps)
    return out


def gelu(x) -> np.ndarray:
    """Kernels::gelu with A&S 7.1.26 erf (plans:865-876), returns a copy."""
    y = _f32(x).copy()
    lib.ora_gelu_f32(_p(y), y.size)
    return y


def gelu_erff(x) -> np.ndarray:
    y = _f32(x).copy()
    lib.ora_gelu_erff_f32(_p(y), y.size)
    return y


def erf_as7126(x: float) -> float:
    return float(lib.ora_erf_as7126(float(x)))


def layerscale(x, gamma) -> np.ndarray:
    y = _f32(x).copy()
    cols = y.shape[-1]
    lib.ora_layerscale_f32(_p(y), y.size // cols, cols, _p(_f32(gamma)))
    return y


def add(dst, src) -> np.ndarray:
    d = _f32(dst).copy()
    s = _f32(src)
    lib.ora_add_f32(_p(d), _p(s), d.size)
    return d


def layerscale_residual(x, y, gamma) -> np.ndarray:
    """x + y*gamma with two roundings (vit_block.rs:755-758 then add_residual)."""
    out = _f32(x).copy()
    yv = _f32(y)
    cols = out.shape[-1]
    if gamma is None:
        lib.ora_add_f32(_p(out), _p(yv), out.size)
    elif np.asarray(gamma).dtype == np.float16:
        lib.ora_layerscale_residual_w16(_p(out), _p(yv), _p(f16_bits(gamma)), out.size // cols, cols)
    else:
        lib.ora_layerscale_residual_f32(_p(out), _p(yv), _p(_f32(gamma)), out.size // cols, cols)
    return out


def rope_positions(n_special: int, gh: int, gw: int, view_count: int, global_layer: bool) -> np.ndarray:
    """Position builder of vit_block.rs:841-881, [rows, 2] f32 (y, x)."""
    rows = (n_special + gh * gw) * view_count
    out = np.empty((rows, 2), np.float32)
    lib.ora_rope_positions(_p(out), n_special, gh, gw, view_count, 1 if global_layer else 0)
    return out


# RoPE convention flags (the device ABI's VK_ROPE_* bits); 0 is the default:
# rotate-half pairing (i, i+16) and exponent 2j/32 for head_dim 64
ROPE_INTERLEAVED = 1
ROPE_EXP_HEAD = 2
ROPE_MODES = (0, ROPE_INTERLEAVED, ROPE_EXP_HEAD, ROPE_INTERLEAVED | ROPE_EXP_HEAD)


def rope_inv_freq(head_dim: int, base: float = 100.0, mode: int = 0) -> np.ndarray:
    out = np.empty(head_dim // 4, np.float32)
    lib.ora_rope_inv_freq_mode(_p(out), head_dim, base, mode)
    return out


def rope2d(x, heads: int, n: int, head_dim: int, pos_yx, base: float = 100.0,
           mode: int = 0) -> np.ndarray:
    """vestra_kernels::rope2d on [heads, n, head_dim] (returns a copy)."""
    y = _f32(x).copy()
    pos = np.ascontiguousarray(pos_yx, dtype=np.int64)
    lib.ora_rope2d_mode_f32(_p(y), heads, n, head_dim, _p(pos), base, mode)
    return y


def qk_norm_rope(q, k, qg, qb, kg, kb, pos_yx, heads: int, n: int, head_dim: int = 64,
                 base: float = 100.0, eps: float = 1e-5, mode: int = 0):
    """qk_norm_rope_f32_da3_base (vit_block.rs:911-924), returns (q, k) copies."""
    qo, ko = _f32(q).copy(), _f32(k).copy()
    pos = _f32(pos_yx)
    if np.asarray(qg).dtype == np.float16:
        args = [f16_bits(a) for a in (qg, qb, kg, kb)]
        lib.ora_qk_norm_rope_w16(_p(qo), _p(ko), *[_p(a) for a in args], _p(pos), heads, n,
                                 head_dim, base, eps, mode)
    else:
        args = [_f32(a) for a in (qg, qb, kg, kb)]
        lib.ora_qk_norm_rope_mode_f32(_p(qo), _p(ko), *[_p(a) for a in args], _p(pos), heads,
                                      n, head_dim, base, eps, mode)
    return qo, ko


def normalize_u8_hwc(img, mean, std) -> np.ndarray:
    img = np.ascontiguousarray(img, dtype=np.uint8)
    h, w, _ = img.shape
    out = np.empty((3, h, w), np.float32)
    m, s = _f32(mean), _f32(std)
    lib.ora_normalize_u8_hwc(_p(img), _p(out), h, w, _p(m), _p(s))
    return out


def patchify_nchw(img, patch: int) -> np.ndarray:
    img = _f32(img)
    c, h, w = img.shape
    out = np.empty(((h // patch) * (w // patch), c * patch * patch), np.float32)
    lib.ora_patchify_nchw(_p(img), _p(out), h, w, patch, c)
    return out


def linear(x, w_kn, bias) -> np.ndarray:
    """run_linear without LayerScale: x @ W[k, n] + b, sequential k."""
    x, w = _f32(x), _f32(w_kn)
    m, k = x.shape
    n = w.shape[1]
    out = np.empty((m, n), np.float32)
    lib.ora_linear_f32(_p(x), _p(w), _p(_f32(bias)) if bias is not None else None, _p(out), m, k, n)
    return out


def patch_project_oihw(img_chw, patch: int, w_oihw, bias) -> np.ndarray:
    img = _f32(img_chw)
    _, h, w = img.shape
    wt = _f32(w_oihw)
    embed = wt.shape[0]
    out = np.empty(((h // patch) * (w // patch), embed), np.float32)
    lib.ora_patch_project_oihw(_p(img), h, w, patch, _p(wt), _p(_f32(bias)), embed, _p(out))
    return out


def pos_embed_bicubic(pos_embed, grid: int, embed: int, gh: int, gw: int,
                      interp_offset: float = 0.1) -> np.ndarray:
    """interpolate_pos_embed (pos_embed.rs:122-169)."""
    src = _f32(pos_embed)
    out = np.empty((1 + gh * gw, embed), np.float32)
    lib.ora_pos_embed_bicubic(_p(src), grid, embed, gh, gw, interp_offset, _p(out))
    return out


def split_qkv_hnd(qkv, n: int, heads: int, head_dim: int):
    """Token-major QKV [n, 3*heads*head_dim] -> head-major Q, K, V [heads, n, head_dim]."""
    a = _f32(qkv)
    q, k, v = (np.empty((heads, n, head_dim), np.float32) for _ in range(3))
    lib.ora_split_qkv_hnd(_p(a), n, heads, head_dim, _p(q), _p(k), _p(v))
    return q, k, v


def hnd_to_token(hnd, n: int, heads: int, head_dim: int) -> np.ndarray:
    """Head-major [heads, n, head_dim] -> token-major [n, heads*head_dim]."""
    out = np.empty((n, heads * head_dim), np.float32)
    lib.ora_hnd_to_token(_p(_f32(hnd)), n, heads, head_dim, _p(out))
    return out


def attention(q, k, v, batches: int, n: int, head_dim: int) -> np.ndarray:
    """softmax(Q K^T / sqrt(head_dim)) V over `batches` sequences [n, head_dim]."""
    out = np.empty((batches, n, head_dim), np.float32)
    lib.ora_attention_f32(_p(_f32(q)), _p(_f32(k)), _p(_f32(v)), batches, n, head_dim, _p(out))
    return out


def assemble_tokens(patch_tokens, gh: int, gw: int, cls, registers, pos_table) -> np.ndarray:
    pt = _f32(patch_tokens)
    embed = pt.shape[-1]
    nreg = 0 if registers is None else int(np.asarray(registers).size // embed)
    regs = None if registers is None else _f32(registers)
    out = np.empty((1 + nreg + gh * gw, embed), np.float32)
    lib.ora_assemble_tokens(_p(pt), gh, gw, embed, _p(_f32(cls)), _p(regs), nreg,
                            _p(_f32(pos_table)), _p(out))
    return out


def patch_embed_u8(img_hwc, patch: int, mean, std, w_oihw, bias, cls, registers,
                   pos_table) -> np.ndarray:
    img = np.ascontiguousarray(img_hwc, dtype=np.uint8)
    h, w, _ = img.shape
    wt = _f32(w_oihw)
    embed = wt.shape[0]
    nreg = 0 if registers is None else int(np.asarray(registers).size // embed)
    regs = None if registers is None else _f32(registers)
    out = np.empty((1 + nreg + (h // patch) * (w // patch), embed), np.float32)
    lib.ora_patch_embed_u8(_p(img), h, w, patch, _p(_f32(mean)), _p(_f32(std)), _p(wt),
                           _p(_f32(bias)), embed, _p(_f32(cls)), _p(regs), nreg,
                           _p(_f32(pos_table)), _p(out))
    return out


def block_fused_ops(tokens, q, k, attn_proj, hidden, mlp_out, layer: dict, cfg: dict,
                    layer_idx: int, gh: int, gw: int, view_count: int, camera=None):
    """One block's fused per-token sequence (vit_block.rs:1019-1139 order), on copies.

    layer: dict of numpy parameter vectors (norm1_gamma, ..., ls2; absent or
    None entries follow the reference's presence gating).  q/k layout: one
    head-major sequence for global layers, per-view head-major blocks for local
    ones.  Returns dict(tokens, ln1, q, k, ln2, hidden).
    """
    D = cfg["embed_dim"]
    H = cfg["num_heads"]
    hd = cfg["head_dim"]
    n_special = 1 + cfg["num_register"]
    tpv = n_special + gh * gw
    rows = tpv * view_count
    alt = cfg["alt_start"]
    glob = alt >= 0 and layer_idx >= alt and layer_idx % 2 == 1
    x = _f32(tokens).reshape(rows, D).copy()
    if alt >= 0 and layer_idx == alt:
        cam = _f32(camera).reshape(-1)
        for v in range(view_count):
            slot = 1 if v > 0 else 0
            x[v * tpv] = cam[slot * D:(slot + 1) * D]
    ln1 = layernorm(x, layer["norm1_gamma"], layer["norm1_beta"], cfg["ln_eps"])
    qo = _f32(q).copy()
    ko = _f32(k).copy()
    use_qkn = cfg["qknorm_start"] >= 0 and layer_idx >= cfg["qknorm_start"] and \
        layer.get("qnorm_gamma") is not None
    use_rope = cfg["rope_start"] >= 0 and layer_idx >= cfg["rope_start"]
    if use_rope or use_qkn:
        pos = rope_positions(n_special, gh, gw, view_count, glob)
        if glob:
            blocks = [(qo.reshape(H, rows, hd), ko.reshape(H, rows, hd), pos)]
        else:
            qv = qo.reshape(view_count, H, tpv, hd)
            kv = ko.reshape(view_count, H, tpv, hd)
            blocks = [(qv[v], kv[v], pos[v * tpv:(v + 1) * tpv]) for v in range(view_count)]
        for qb_, kb_, p in blocks:
            n = qb_.shape[1]
            if use_qkn:
                qb_[...] = layernorm(qb_, layer["qnorm_gamma"], layer["qnorm_beta"], cfg["qk_norm_eps"])
                kb_[...] = layernorm(kb_, layer["knorm_gamma"], layer["knorm_beta"], cfg["qk_norm_eps"])
            if use_rope:
                pi = p.astype(np.int64)
                mode = cfg.get("rope_mode", 0)
                qb_[...] = rope2d(qb_, H, n, hd, pi, cfg["rope_freq"], mode).reshape(qb_.shape)
                kb_[...] = rope2d(kb_, H, n, hd, pi, cfg["rope_freq"], mode).reshape(kb_.shape)
    x = layerscale_residual(x, _f32(attn_proj).reshape(rows, D), layer.get("ls1"))
    ln2 = layernorm(x, layer["norm2_gamma"], layer["norm2_beta"], cfg["ln_eps"])
    hid = gelu(hidden)
    x = layerscale_residual(x, _f32(mlp_out).reshape(rows, D), layer.get("ls2"))
    return {"tokens": x, "ln1": ln1, "q": qo, "k": ko, "ln2": ln2, "hidden": hid}


def block_forward(tokens, params: dict, cfg: dict, layer_idx: int, gh: int, gw: int,
                  view_count: int, camera=None) -> dict:
    """One whole DA3 ViT block (vit_block.rs:1019-1139; device order of
    run_tail_device, vit_block.rs:489-582), composed from the functions above.

    params: norm1/norm2 gamma+beta, qkv_w [D, 3D] + qkv_b, optional
    qnorm/knorm gamma+beta, proj_w [D, D] + proj_b + optional ls1, fc1_w
    [D, M] + fc1_b, fc2_w [M, D] + fc2_b + optional ls2 (weights in the
    reference's [in, out] layout).  Local layers attend within each view,
    global layers (backbone.rs:459-460) over all rows.  Returns dict(tokens,
    q, k, v, attn, ln2, hidden) with q/k/v/attn head-major [H, rows, 64].
    """
    D = cfg["embed_dim"]
    H = cfg["num_heads"]
    hd = cfg["head_dim"]
    n_special = 1 + cfg["num_register"]
    tpv = n_special + gh * gw
    rows = tpv * view_count
    alt = cfg["alt_start"]
    glob = alt >= 0 and layer_idx >= alt and layer_idx % 2 == 1
    x = _f32(tokens).reshape(rows, D).copy()
    if alt >= 0 and layer_idx == alt:
        cam = _f32(camera).reshape(-1)
        for v in range(view_count):
            slot = 1 if v > 0 else 0
            x[v * tpv] = cam[slot * D:(slot + 1) * D]
    ln1 = layernorm(x, params["norm1_gamma"], params["norm1_beta"], cfg["ln_eps"])
    q, k, v = split_qkv_hnd(linear(ln1, params["qkv_w"], params["qkv_b"]), rows, H, hd)
    use_qkn = cfg["qknorm_start"] >= 0 and layer_idx >= cfg["qknorm_start"] and \
        params.get("qnorm_gamma") is not None
    use_rope = cfg["rope_start"] >= 0 and layer_idx >= cfg["rope_start"]
    if use_qkn:
        # per (head, token) row: the view split does not matter
        q = layernorm(q, params["qnorm_gamma"], params["qnorm_beta"], cfg["qk_norm_eps"])
        k = layernorm(k, params["knorm_gamma"], params["knorm_beta"], cfg["qk_norm_eps"])
    if use_rope:
        pos = rope_positions(n_special, gh, gw, view_count, glob).astype(np.int64)
        mode = cfg.get("rope_mode", 0)
        q = rope2d(q, H, rows, hd, pos, cfg["rope_freq"], mode).reshape(H, rows, hd)
        k = rope2d(k, H, rows, hd, pos, cfg["rope_freq"], mode).reshape(H, rows, hd)
    if glob:
        attn = attention(q, k, v, H, rows, hd)
    else:
        # [H, rows, hd] holds head h of view v at rows (h*views + v)*tpv...
        attn = attention(q, k, v, H * view_count, tpv, hd)
    attn = attn.reshape(H, rows, hd)
    y = linear(hnd_to_token(attn, rows, H, hd).reshape(rows, D), params["proj_w"],
               params["proj_b"])
    x = layerscale_residual(x, y, params.get("ls1"))
    ln2 = layernorm(x, params["norm2_gamma"], params["norm2_beta"], cfg["ln_eps"])
    hidden = gelu(linear(ln2, params["fc1_w"], params["fc1_b"]))
    y = linear(hidden, params["fc2_w"], params["fc2_b"])
    x = layerscale_residual(x, y, params.get("ls2"))
    return {"tokens": x, "q": q.reshape(H, rows, hd), "k": k.reshape(H, rows, hd),
            "v": v.reshape(H, rows, hd), "attn": attn, "ln2": ln2, "hidden": hidden}


def capture(local_x, x, n: int, n_special: int, embed: int, view_count: int, norm_gamma,
            norm_beta, eps: float, cat_token: bool):
    """Backbone::post_process_capture (backbone.rs:1139-1179) per view of a
    view-major batch: returns (feat [views, n_patch, W], cam [views, W]) with
    W = 2*embed (cat_token: [local row | LN(x row)], cam [local row 0 | x
    row 0]) or embed (LN(x row), cam x row 0)."""
    xv = _f32(x).reshape(view_count, n, embed)
    feats, cams = [], []
    for v in range(view_count):
        normed = layernorm(xv[v, n_special:], norm_gamma, norm_beta, eps)
        if cat_token:
            lv = _f32(local_x).reshape(view_count, n, embed)[v]
            feats.append(np.concatenate([lv[n_special:], normed], axis=1))
            cams.append(np.concatenate([lv[0], xv[v, 0]]))
        else:
            feats.append(normed)
            cams.append(xv[v, 0].copy())
    return np.stack(feats), np.stack(cams)


def token_to_chw(tok, n_tok: int, c: int, gamma=None, beta=None, eps: float = 1e-5):
    """The head's materialised hand-off (dpt_head.rs:513-518): scalar
    LayerNorm of every token row (when gamma/beta are given), then
    tok_major_to_chw, out[ch, t] = tok[t, ch]."""
    t = _f32(tok).reshape(n_tok, c)
    if gamma is not None:
        t = layernorm(t, gamma, beta, eps)
    return np.ascontiguousarray(t.T)


Q8_0_BLOCK, Q8_0_BLOCK_BYTES = 32, 34


def dequantize_q8_0(blocks, n: int) -> np.ndarray:
    """q8_0::dequantize_q8_0 over read_blocks' wire layout (crates/da-gguf/src/
    q8_0.rs:24-51): per 34-byte block a little-endian f16 scale d, then 32
    int8 q; out[32*b + j] = f32(d) * f32(q_j) (exact in f32)."""
    raw = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, Q8_0_BLOCK_BYTES)
    if raw.shape[0] * Q8_0_BLOCK != n:
        raise ValueError(f"{raw.shape[0]} blocks do not hold {n} values")
    d = f16_to_f32(raw[:, :2].copy().view("<u2").reshape(-1))
    q = raw[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).astype(np.float32).reshape(-1)


def quantize_q8_0(x) -> np.ndarray:
    """Test-input helper: ggml's Q8_0 quantisation (d = amax/127 rounded to
    f16, q = round(x/d)) into the 34-byte wire layout."""
    v = _f32(x).reshape(-1, Q8_0_BLOCK).astype(np.float64)
    amax = np.abs(v).max(axis=1)
    d = (amax / 127.0).astype(np.float16)
    dd = d.astype(np.float64)
    inv = np.where(dd > 0, 1.0 / np.where(dd > 0, dd, 1.0), 0.0)
    q = np.clip(np.rint(v * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((v.shape[0], Q8_0_BLOCK_BYTES), np.uint8)
    out[:, :2] = d.view(np.uint16).astype("<u2").view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def resize_u8(img_hwc, dh: int, dw: int, mode: str) -> np.ndarray:
    """resize_{bilinear,cubic,area}_u8 (preprocess.rs:253-409) of a u8 HWC RGB image."""
    img = np.ascontiguousarray(img_hwc, dtype=np.uint8)
    sh, sw, _ = img.shape
    out = np.empty((dh, dw, 3), np.uint8)
    fn = {"bilinear": lib.ora_resize_bilinear_u8, "cubic": lib.ora_resize_cubic_u8,
          "area": lib.ora_resize_area_u8}[mode]
    fn(_p(img), sw, sh, _p(out), dw, dh)
    return out


def preprocess_shape(h: int, w: int, image_size: int, patch: int, upper_bound: bool = True):
    """(boundary_h, boundary_w, out_h, out_w, scaled) of preprocess (preprocess.rs:432-469)."""
    d = np.zeros(4, np.uint64)
    scaled = lib.ora_preprocess_shape(h, w, image_size, patch, 1 if upper_bound else 0, _p(d))
    return int(d[0]), int(d[1]), int(d[2]), int(d[3]), bool(scaled)


def preprocess_resize_u8(img_hwc, image_size: int, patch: int, upper_bound: bool = True):
    """preprocess's resize and patch snap (preprocess.rs:432-469): u8 HWC at the model size."""
    img = np.ascontiguousarray(img_hwc, dtype=np.uint8)
    h, w, _ = img.shape
    _, _, oh, ow, _ = preprocess_shape(h, w, image_size, patch, upper_bound)
    out = np.empty((oh, ow, 3), np.uint8)
    lib.ora_preprocess_resize_u8(_p(img), h, w, image_size, patch, 1 if upper_bound else 0,
                                 _p(out))
    return out


def backbone_forward(tokens, blocks: list, cfg: dict, gh: int, gw: int, view_count: int,
                     camera, norm_gamma, norm_beta, cat_token: bool, out_layers):
    """Backbone::forward_multi_view_ordered (backbone.rs:688-877) on the
    view-major token rows: block_forward per layer, the snapshot local_x
    after every local layer, post_process_capture at each out layer in the
    caller's order (global layers pair the stream with local_x).  Returns
    (tokens, [(feat, cam) per out layer])."""
    D = cfg["embed_dim"]
    n = 1 + cfg["num_register"] + gh * gw
    alt = cfg["alt_start"]
    x = _f32(tokens).reshape(n * view_count, D).copy()
    local_x = x.copy()
    out = [None] * len(out_layers)
    for layer, p in enumerate(blocks):
        x = block_forward(x, p, cfg, layer, gh, gw, view_count, camera)["tokens"]
        glob = alt >= 0 and layer >= alt and layer % 2 == 1
        for i, want in enumerate(out_layers):
            if want == layer:
                out[i] = capture(local_x if glob else x, x, n, 1 + cfg["num_register"], D,
                                 view_count, norm_gamma, norm_beta, cfg["ln_eps"], cat_token)
        if not glob:
            local_x = x.copy()
    if any(o is None for o in out):
        raise ValueError("an out layer was never reached")
    return x, out
