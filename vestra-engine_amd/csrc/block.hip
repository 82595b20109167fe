// One DA3 ViT block's fused per-token operations, enqueued on the runtime's
// stream in the reference order (run_tail_device, vit_block.rs:489-582, and
// vit_block_with_views, vit_block.rs:1019-1139).  The GEMMs and attention
// between the operations are the caller's; their products arrive in
// vk_vit_activations.
//
// Multi-view batches are handled MI355X-first: the residual stream of all
// views stays in one view-major device buffer for every layer.  Per-token
// operations are independent of view boundaries, so local and global layers
// both run as one launch over view_count * tokens_per_view rows; only the
// RoPE positions differ (per-view grid positions vs (1,1)) and the Q/K layout
// (per-view head-major blocks vs one head-major sequence).  The reference's
// flatten / split copies around global layers (backbone.rs:770-796,
// 990-1027) do not exist here.
#include "common.h"

namespace {

bool layer_uses_global(const vk_vit_config* cfg, size_t layer) {
  return cfg->alt_start >= 0 && static_cast<long long>(layer) >= cfg->alt_start && layer % 2 == 1;
}

int check_len(const vk_tensor* t, size_t len, const char* name) {
  VK_REQUIRE(t != nullptr, "activation %s is null", name);
  VK_REQUIRE(t->dtype == VK_F32, "activation %s must be f32", name);
  VK_REQUIRE(t->len == len, "activation %s holds %zu, expected %zu", name, t->len, len);
  return VK_OK;
}

}  // namespace

extern "C" int vk_vit_block_fused_ops(vk_runtime* rt, const vk_vit_config* cfg,
                                      size_t layer_idx, const vk_vit_layer* layer,
                                      const vk_vit_layer* next_layer,
                                      const vk_vit_activations* act, size_t gh, size_t gw,
                                      size_t view_count, const vk_tensor* camera,
                                      unsigned flags) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(cfg && layer && act, "null argument");
  VK_REQUIRE(view_count > 0 && gw > 0 && gh > 0, "empty grid or view count");
  const size_t D = cfg->embed_dim;
  const size_t H = cfg->num_heads;
  const size_t hd = cfg->head_dim;
  const size_t M = cfg->mlp_hidden;
  VK_REQUIRE(D > 0 && H > 0 && hd > 0 && M > 0, "empty model dimensions");
  VK_REQUIRE(H * hd == D, "num_heads*head_dim (%zu) must equal embed_dim (%zu)", H * hd, D);
  const size_t n_special = 1 + cfg->num_register;
  const size_t tpv = n_special + gh * gw;
  const size_t rows = tpv * view_count;
  VK_TRY(check_len(act->tokens, rows * D, "tokens"));
  VK_TRY(check_len(act->ln1, rows * D, "ln1"));
  VK_TRY(check_len(act->q, rows * D, "q"));
  VK_TRY(check_len(act->k, rows * D, "k"));
  VK_TRY(check_len(act->attn_proj, rows * D, "attn_proj"));
  VK_TRY(check_len(act->ln2, rows * D, "ln2"));
  VK_TRY(check_len(act->hidden, rows * M, "hidden"));
  VK_TRY(check_len(act->mlp_out, rows * D, "mlp_out"));
  VK_REQUIRE(!(flags & VK_BLOCK_FUSE_NEXT_LN1) || next_layer,
             "VK_BLOCK_FUSE_NEXT_LN1 needs next_layer");
  // The camera slot can only have been written by the previous block's fused
  // LS2 + residual + LN1 pass, which also produced this block's LN1: the flag
  // is meaningful only with VK_BLOCK_SKIP_LN1 and only at alt_start.
  if (flags & VK_BLOCK_CAMERA_WRITTEN) {
    VK_REQUIRE(flags & VK_BLOCK_SKIP_LN1,
               "VK_BLOCK_CAMERA_WRITTEN needs VK_BLOCK_SKIP_LN1 (the previous block's fused "
               "LS2+res+LN1 pass writes both)");
    VK_REQUIRE(cfg->alt_start >= 0 && layer_idx == static_cast<size_t>(cfg->alt_start),
               "VK_BLOCK_CAMERA_WRITTEN is valid only at layer alt_start=%d (layer %zu)",
               cfg->alt_start, layer_idx);
  }

  const bool global = layer_uses_global(cfg, layer_idx);

  // camera-token slot write before block alt_start (backbone.rs:446-457 for
  // one view; 746-768 per view: slot 0 for the reference view, slot 1 for the
  // source views).
  bool camera_written = false;
  if (cfg->alt_start >= 0 && layer_idx == static_cast<size_t>(cfg->alt_start) &&
      !(flags & VK_BLOCK_CAMERA_WRITTEN)) {
    VK_REQUIRE(camera != nullptr, "camera token required at alt_start=%d", cfg->alt_start);
    VK_REQUIRE(camera->dtype == VK_F32 && camera->len >= D, "camera token must hold >= %zu f32", D);
    VK_REQUIRE(view_count == 1 || camera->len >= 2 * D,
               "multi-view camera token must hold reference and source slots (2*%zu)", D);
    VK_TRY(vk::write_camera_rows(rt, static_cast<float*>(act->tokens->ptr),
                                 static_cast<const float*>(camera->ptr), view_count, tpv, D));
    camera_written = true;
  }

  // LN1 (skipped when the previous block already produced it, unless the
  // camera write changed the tokens since)
  if (!(flags & VK_BLOCK_SKIP_LN1) || camera_written) {
    VK_TRY(vk_layernorm_into_f32(rt, act->tokens, layer->norm1_gamma, layer->norm1_beta, rows, D,
                                 cfg->ln_eps, act->ln1));
  }

  // Q/K-norm + RoPE gating (vit_block.rs:835-838)
  const bool use_qknorm = cfg->qknorm_start >= 0 &&
                          static_cast<long long>(layer_idx) >= cfg->qknorm_start &&
                          layer->qnorm_gamma != nullptr;
  const bool use_rope =
      cfg->rope_start >= 0 && static_cast<long long>(layer_idx) >= cfg->rope_start;
  const vk_qk_layout layout = global ? VK_QK_HEADS_OUTER : VK_QK_VIEWS_OUTER;
  if (use_rope) {
    VK_TRY(vk_qk_norm_rope_grid_mode_f32(
        rt, act->q, act->k, use_qknorm ? layer->qnorm_gamma : nullptr,
        use_qknorm ? layer->qnorm_beta : nullptr, use_qknorm ? layer->knorm_gamma : nullptr,
        use_qknorm ? layer->knorm_beta : nullptr, H, hd, n_special, gh, gw, view_count,
        global ? 1 : 0, layout, cfg->rope_freq, cfg->qk_norm_eps, cfg->rope_mode));
  } else if (use_qknorm) {
    // Q/K-norm without RoPE: LayerNorm over every (head, token) row
    VK_TRY(vk_layernorm_into_f32(rt, act->q, layer->qnorm_gamma, layer->qnorm_beta, rows * H, hd,
                                 cfg->qk_norm_eps, act->q));
    VK_TRY(vk_layernorm_into_f32(rt, act->k, layer->knorm_gamma, layer->knorm_beta, rows * H, hd,
                                 cfg->qk_norm_eps, act->k));
  }

  // tokens += ls1 (.) attn_proj, then LN2
  if (flags & VK_BLOCK_FUSE_LS_LN) {
    VK_TRY(vk_layerscale_residual_layernorm_f32(rt, act->tokens, act->attn_proj, layer->ls1,
                                                layer->norm2_gamma, layer->norm2_beta, rows, D,
                                                cfg->ln_eps, act->ln2));
  } else {
    VK_TRY(vk_layerscale_residual_f32(rt, act->tokens, act->attn_proj, layer->ls1, rows, D));
    VK_TRY(vk_layernorm_into_f32(rt, act->tokens, layer->norm2_gamma, layer->norm2_beta, rows, D,
                                 cfg->ln_eps, act->ln2));
  }

  // GELU on the FC1 output
  VK_TRY(vk_gelu_f32_inplace(rt, act->hidden));

  // tokens += ls2 (.) mlp_out [, the camera-slot overwrite when the next
  // block is alt_start and the camera token is given, next block's LN1]
  if (flags & VK_BLOCK_FUSE_NEXT_LN1) {
    const bool camera_next = cfg->alt_start >= 0 &&
                             layer_idx + 1 == static_cast<size_t>(cfg->alt_start) &&
                             camera != nullptr;
    if (camera_next) {
      VK_REQUIRE(camera->dtype == VK_F32 && camera->len >= D,
                 "camera token must hold >= %zu f32", D);
      VK_REQUIRE(view_count == 1 || camera->len >= 2 * D,
                 "multi-view camera token must hold reference and source slots (2*%zu)", D);
    }
    VK_TRY(vk::ls_residual_layernorm_camera(
        rt, act->tokens, act->mlp_out, layer->ls2, next_layer->norm1_gamma,
        next_layer->norm1_beta, rows, D, cfg->ln_eps, act->ln1, camera_next ? camera : nullptr,
        tpv));
  } else {
    VK_TRY(vk_layerscale_residual_f32(rt, act->tokens, act->mlp_out, layer->ls2, rows, D));
  }
  return VK_OK;
}

// ---------------------------------------------------------------------------
// The whole block on the device (run_tail_device, vit_block.rs:489-582).
//
// Q, K, V and the attention output stay head-major [H, rows, 64] for local
// and global layers alike.  A local layer's attention is per view; in this
// layout head h of view v is the contiguous run of tpv rows starting at row
// h*rows + v*tpv = (h*view_count + v)*tpv, so the view-major batch is simply
// H*view_count sequences of tpv tokens -- no repacking between layer kinds.
// The QKV projection writes Q, K, V head-major from its epilogue and the
// output projection reads the attention output head-major, so the
// reference's split_qkv_hnd / hnd_to_token passes (vit_block.rs:539-541, 560)
// are not separate launches, and Q/K-norm + RoPE run in the QKV epilogue.
// 7 launches per block; in the backbone's block loop FC2 also writes the
// next block's LN1, one launch fewer wherever FC2 runs split-K.
// ---------------------------------------------------------------------------
namespace {

int check_linear(const vk_linear* l, size_t in, size_t out, const char* name) {
  VK_REQUIRE(l != nullptr, "block weight %s is null", name);
  VK_REQUIRE(l->in_features == in && l->out_features == out,
             "block weight %s is %zu -> %zu, expected %zu -> %zu", name, l->in_features,
             l->out_features, in, out);
  return VK_OK;
}

// One block.  next != NULL: FC2's residual pass also writes the next
// block's LN1 (next->norm1) into ws->ln, in its split-K sum pass when it has
// one (the bits of the separate LayerNorm); ln1_done: this block's LN1 is
// already in ws->ln, written so by the previous block.  Neither is used
// across alt_start, where the camera slot is overwritten before LN1.
int block_forward(vk_runtime* rt, const vk_vit_config* cfg, size_t layer_idx,
                  const vk_vit_block_weights* w, vk_tensor* tokens, size_t gh, size_t gw,
                  size_t view_count, const vk_tensor* camera, const vk_vit_block_workspace* ws,
                  const vk_vit_block_weights* next, bool ln1_done) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(cfg && w && tokens && ws, "null argument");
  VK_REQUIRE(view_count > 0 && gw > 0 && gh > 0, "empty grid or view count");
  const size_t D = cfg->embed_dim;
  const size_t H = cfg->num_heads;
  const size_t hd = cfg->head_dim;
  const size_t M = cfg->mlp_hidden;
  VK_REQUIRE(D > 0 && H > 0 && M > 0, "empty model dimensions");
  VK_UNSUPPORTED_IF(hd != 64, "block: head_dim=%zu (qualified: 64)", hd);
  VK_REQUIRE(H * hd == D, "num_heads*head_dim (%zu) must equal embed_dim (%zu)", H * hd, D);
  const size_t n_special = 1 + cfg->num_register;
  const size_t tpv = n_special + gh * gw;
  const size_t rows = tpv * view_count;
  VK_TRY(check_len(tokens, rows * D, "tokens"));
  VK_TRY(check_len(ws->ln, rows * D, "workspace ln"));
  VK_TRY(check_len(ws->q, rows * D, "workspace q"));
  VK_TRY(check_len(ws->k, rows * D, "workspace k"));
  VK_TRY(check_len(ws->v, rows * D, "workspace v"));
  VK_TRY(check_len(ws->attn, rows * D, "workspace attn"));
  VK_TRY(check_len(ws->hidden, rows * M, "workspace hidden"));
  VK_TRY(check_linear(w->qkv, D, 3 * D, "qkv"));
  VK_TRY(check_linear(w->proj, D, D, "proj"));
  VK_TRY(check_linear(w->fc1, D, M, "fc1"));
  VK_TRY(check_linear(w->fc2, M, D, "fc2"));

  const bool global = layer_uses_global(cfg, layer_idx);

  // camera-token slot write at alt_start (backbone.rs:446-457, 746-768)
  const bool at_alt = cfg->alt_start >= 0 && layer_idx == static_cast<size_t>(cfg->alt_start);
  VK_REQUIRE(!(ln1_done && at_alt), "block: LN1 cannot precede the camera write at alt_start");
  VK_REQUIRE(!(next && cfg->alt_start >= 0 && layer_idx + 1 == static_cast<size_t>(cfg->alt_start)),
             "block: the next block's LN1 follows its camera write at alt_start");
  if (at_alt) {
    VK_REQUIRE(camera != nullptr, "camera token required at alt_start=%d", cfg->alt_start);
    VK_REQUIRE(camera->dtype == VK_F32 && camera->len >= D, "camera token must hold >= %zu f32", D);
    VK_REQUIRE(view_count == 1 || camera->len >= 2 * D,
               "multi-view camera token must hold reference and source slots (2*%zu)", D);
    VK_TRY(vk::write_camera_rows(rt, static_cast<float*>(tokens->ptr),
                                 static_cast<const float*>(camera->ptr), view_count, tpv, D));
  }

  // LN1 -> QKV (head-major Q, K, V) with Q/K-norm + RoPE, gated as in
  // vk_vit_block_fused_ops (vit_block.rs:835-838); with RoPE on, both run
  // in the projection's epilogue (the bits of the separate pass)
  if (!ln1_done)
    VK_TRY(vk_layernorm_into_f32(rt, tokens, w->norm1_gamma, w->norm1_beta, rows, D,
                                 cfg->ln_eps, ws->ln));
  const bool use_qknorm = cfg->qknorm_start >= 0 &&
                          static_cast<long long>(layer_idx) >= cfg->qknorm_start &&
                          w->qnorm_gamma != nullptr;
  const bool use_rope =
      cfg->rope_start >= 0 && static_cast<long long>(layer_idx) >= cfg->rope_start;
  if (use_rope) {
    VK_TRY(vk_linear_run_qkv_hnd_norm_rope_mode_f32(
        rt, w->qkv, ws->ln, rows, H, hd, ws->q, ws->k, ws->v,
        use_qknorm ? w->qnorm_gamma : nullptr, use_qknorm ? w->qnorm_beta : nullptr,
        use_qknorm ? w->knorm_gamma : nullptr, use_qknorm ? w->knorm_beta : nullptr, n_special,
        gh, gw, view_count, global ? 1 : 0, cfg->rope_freq, cfg->qk_norm_eps, cfg->rope_mode));
  } else {
    VK_TRY(vk_linear_run_qkv_hnd_f32(rt, w->qkv, ws->ln, rows, H, hd, ws->q, ws->k, ws->v));
  }
  if (!use_rope && use_qknorm) {
    VK_TRY(vk_layernorm_into_f32(rt, ws->q, w->qnorm_gamma, w->qnorm_beta, rows * H, hd,
                                 cfg->qk_norm_eps, ws->q));
    VK_TRY(vk_layernorm_into_f32(rt, ws->k, w->knorm_gamma, w->knorm_beta, rows * H, hd,
                                 cfg->qk_norm_eps, ws->k));
  }

  // attention: global -> H sequences of all rows; local -> H*view_count
  // sequences of one view's tokens
  VK_TRY(vk_attention_into_f32(rt, ws->q, ws->k, ws->v, global ? H : H * view_count,
                               global ? rows : tpv, hd, ws->attn));

  // tokens += (attn @ Wproj + b) * ls1, then LN2 (in the projection's
  // split-K sum pass when it has one)
  VK_TRY(vk::linear_hnd_residual_layernorm(rt, w->proj, ws->attn, rows, H, hd, tokens,
                                           w->norm2_gamma, w->norm2_beta, cfg->ln_eps, ws->ln));

  // FC1 + GELU -> tokens += (hidden @ Wfc2 + b) * ls2 [-> next block's LN1]
  VK_TRY(vk_linear_run_gelu_f32(rt, w->fc1, ws->ln, rows, ws->hidden));
  if (next) {
    VK_REQUIRE(next->norm1_gamma && next->norm1_beta, "next block's norm1 is null");
    return vk::linear_residual_layernorm(rt, w->fc2, ws->hidden, rows, tokens,
                                         next->norm1_gamma, next->norm1_beta, cfg->ln_eps,
                                         ws->ln);
  }
  return vk_linear_run_residual_f32(rt, w->fc2, ws->hidden, rows, tokens);
}

}  // namespace

extern "C" int vk_vit_block_forward_f32(vk_runtime* rt, const vk_vit_config* cfg,
                                        size_t layer_idx, const vk_vit_block_weights* w,
                                        vk_tensor* tokens, size_t gh, size_t gw,
                                        size_t view_count, const vk_tensor* camera,
                                        const vk_vit_block_workspace* ws) {
  return block_forward(rt, cfg, layer_idx, w, tokens, gh, gw, view_count, camera, ws, nullptr,
                       false);
}

// ---------------------------------------------------------------------------
// The backbone's block loop on the device (Backbone::forward and
// forward_multi_view_ordered, backbone.rs:390-532, 688-877): every block on
// the view-major residual stream, the pre-alternation snapshot local_x kept
// after each local layer, and the capture (final LayerNorm + cat) at each
// requested layer, in the order the caller lists them.
// ---------------------------------------------------------------------------
extern "C" int vk_backbone_forward_f32(vk_runtime* rt, const vk_vit_config* cfg, size_t depth,
                                       const vk_vit_block_weights* blocks, vk_tensor* tokens,
                                       size_t gh, size_t gw, size_t view_count,
                                       const vk_tensor* camera, const vk_tensor* norm_gamma,
                                       const vk_tensor* norm_beta, int cat_token,
                                       const int* out_layers, size_t n_out,
                                       vk_tensor* const* feats, vk_tensor* const* cams,
                                       const vk_vit_block_workspace* ws, vk_tensor* local_x) {
  VK_TRY(vk::bind(rt));
  VK_REQUIRE(cfg && blocks && tokens && ws, "null argument");
  VK_REQUIRE(n_out == 0 || (out_layers && feats && cams), "null capture arrays");
  VK_REQUIRE(view_count > 0, "empty view count");
  const size_t D = cfg->embed_dim;
  const size_t n_special = 1 + cfg->num_register;
  const size_t n = n_special + gh * gw;
  const size_t rows = n * view_count;
  const size_t width = cat_token ? 2 * D : D;
  VK_TRY(check_len(tokens, rows * D, "tokens"));
  // every requested layer must be reached (backbone.rs:1085-1095 panics otherwise)
  bool any_global_capture = false;
  for (size_t i = 0; i < n_out; ++i) {
    VK_REQUIRE(out_layers[i] >= 0 && static_cast<size_t>(out_layers[i]) < depth,
               "out layer %d was never reached (depth %zu)", out_layers[i], depth);
    VK_REQUIRE(feats[i] && cams[i], "null capture tensor for out layer %d", out_layers[i]);
    VK_TRY(check_len(feats[i], view_count * (n - n_special) * width, "capture feat"));
    VK_TRY(check_len(cams[i], view_count * width, "capture cam"));
    any_global_capture = any_global_capture ||
                         layer_uses_global(cfg, static_cast<size_t>(out_layers[i]));
  }
  // the snapshot is read only by captures at global layers with cat_token
  const bool keep_local = cat_token && any_global_capture;
  if (keep_local) VK_TRY(check_len(local_x, rows * D, "local_x"));
  if (keep_local) VK_TRY(vk_copy_segment_into_f32(rt, local_x, 0, tokens, 0, rows * D));
  // each block but the last, and the one before alt_start, finishes with the
  // next block's LN1 (one launch fewer where FC2 runs split-K)
  bool ln1_done = false;
  for (size_t layer = 0; layer < depth; ++layer) {
    const bool fuse_next =
        layer + 1 < depth &&
        !(cfg->alt_start >= 0 && layer + 1 == static_cast<size_t>(cfg->alt_start));
    VK_TRY(block_forward(rt, cfg, layer, &blocks[layer], tokens, gh, gw, view_count, camera, ws,
                         fuse_next ? &blocks[layer + 1] : nullptr, ln1_done));
    ln1_done = fuse_next;
    const bool global = layer_uses_global(cfg, layer);
    for (size_t i = 0; i < n_out; ++i) {
      if (static_cast<size_t>(out_layers[i]) != layer) continue;
      // local layers capture against the current stream, global ones against
      // the snapshot of the last local layer (backbone.rs:816-830)
      const vk_tensor* local = cat_token ? (global ? local_x : tokens) : nullptr;
      VK_TRY(vk_capture_f32(rt, local, tokens, n, n_special, D, view_count, norm_gamma,
                            norm_beta, cfg->ln_eps, cat_token, feats[i], cams[i]));
    }
    if (keep_local && !global)
      VK_TRY(vk_copy_segment_into_f32(rt, local_x, 0, tokens, 0, rows * D));
  }
  return VK_OK;
}
