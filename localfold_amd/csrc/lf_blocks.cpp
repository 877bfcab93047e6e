// Block and stack composition: AF2 Evoformer block / stack and AF3 Pairformer block, as
// ordered calls of the op entry points with every residual written in place.
//   Evoformer order: webgpu/af2/evoformer/block.js:1536-1629 (encodeEvoformerBlock)
//   Stack:           webgpu/af2/evoformer/stack.js:44-160
//   Pairformer:      cpu/af3/trunk/pairformer.js:495-541 (pairformerBlock)
//   AF3 MSA module:  cpu/af3/trunk/msa.js:157-287 (msaAttention, msaBlock)
#include <cmath>

#include "lf_context.h"
#include "lf_ops.h"

namespace lf {

// The Evoformer block; with `global` the extra-MSA block (encodeExtraMsaBlock,
// webgpu/af2/evoformer/block.js:1715-1744), whose step 2 is the global column attention.
// With `pair_only` only steps 4-9 run, the MSA being read and not written
// (encodeEvoformerPairBlock, block.js:1663-1713).
static int evoformer_block(lf_context* ctx, const lf_evoformer_block_args& a, const lf_evoformer_weights& w,
                           const lf_global_attention_weights* global = nullptr, int global_heads = 0,
                           bool pair_only = false) {
  LF_REQUIRE(a.sequences > 0 && a.length > 0 && a.c_m > 0 && a.c_z > 0, "evoformer block dimensions must be positive");
  LF_REQUIRE(a.msa && a.pair && a.msa_mask && a.pair_mask, "evoformer block: NULL activation or mask");
  const float eps = a.epsilon > 0.f ? a.epsilon : 1e-5f;
  const long long chunk = 1LL << 30;   // transition hidden budget per chunk on a 288 GB device

  if (!pair_only) {  // 1. MSA row attention with pair bias
    lf_attention_args x{};
    x.batch = a.sequences;
    x.queries = a.length;
    x.channels = a.c_m;
    x.heads = w.row_heads;
    x.act_dtype = a.msa_dtype;
    x.act = a.msa;
    x.mask = a.msa_mask;
    x.out = a.msa;
    x.accumulate = 1;
    x.bias_mode = LF_BIAS_SEPARATE;
    x.pair_dtype = a.pair_dtype;
    x.pair = a.pair;
    x.pair_channels = a.c_z;
    x.epsilon = eps;
    x.w = &w.row_attention;
    StageScope stage(ctx, "row_attention");
    LF_TRY(attention(ctx, x));
  }
  if (pair_only) {
  } else if (global) {  // 2. global column attention (extra-MSA block)
    lf_global_attention_args x{};
    x.sequences = a.sequences;
    x.length = a.length;
    x.channels = a.c_m;
    x.heads = global_heads;
    x.act_dtype = a.msa_dtype;
    x.act = a.msa;
    x.mask = a.msa_mask;
    x.out = a.msa;
    x.accumulate = 1;
    x.epsilon = eps;
    x.w = global;
    StageScope stage(ctx, "global_column_attention");
    LF_TRY(global_attention(ctx, x));
  } else {  // 2. MSA column attention
    lf_attention_args x{};
    x.batch = a.length;
    x.queries = a.sequences;
    x.channels = a.c_m;
    x.heads = w.column_heads;
    x.transpose = 1;
    x.act_dtype = a.msa_dtype;
    x.act = a.msa;
    x.mask = a.msa_mask;
    x.out = a.msa;
    x.accumulate = 1;
    x.epsilon = eps;
    x.w = &w.column_attention;
    StageScope stage(ctx, "column_attention");
    LF_TRY(attention(ctx, x));
  }
  if (!pair_only) {  // 3. MSA transition
    lf_transition_args x{};
    x.kind = LF_TRANSITION_RELU;
    x.rows = a.sequences * a.length;
    x.channels = a.c_m;
    x.hidden = a.msa_hidden;
    x.act_dtype = a.msa_dtype;
    x.act = a.msa;
    x.out = a.msa;
    x.accumulate = 1;
    x.chunk_bytes = chunk;
    x.epsilon = eps;
    x.w = &w.msa_transition;
    StageScope stage(ctx, "msa_transition");
    LF_TRY(transition(ctx, x));
  }
  {  // 4. outer product mean into the pair
    lf_opm_args x{};
    x.sequences = a.sequences;
    x.length = a.length;
    x.c_m = a.c_m;
    x.c_outer = a.c_outer;
    x.c_z = a.c_z;
    x.msa_dtype = a.msa_dtype;
    x.msa = a.msa;
    x.mask = a.msa_mask;
    x.pair_dtype = a.pair_dtype;
    x.pair_in = a.pair;
    x.out = a.pair;
    x.accumulate = 1;
    x.epsilon = eps;
    x.norm_epsilon = 1e-3f;
    x.w = &w.outer_product_mean;
    StageScope stage(ctx, "outer_product_mean");
    LF_TRY(outer_product_mean(ctx, x));
  }
  for (int dir = 0; dir < 2; ++dir) {  // 5, 6. triangle multiplication outgoing, incoming
    lf_tri_mult_args x{};
    x.direction = dir == 0 ? LF_OUTGOING : LF_INCOMING;
    x.dialect = LF_AF2;
    x.length = a.length;
    x.c_z = a.c_z;
    x.c_hidden = a.tri_hidden;
    x.act_dtype = a.pair_dtype;
    x.z = a.pair;
    x.mask = a.pair_mask;
    x.out = a.pair;
    x.accumulate = 1;
    x.epsilon = eps;
    x.w = dir == 0 ? &w.tri_out : &w.tri_in;
    StageScope stage(ctx, dir == 0 ? "tri_mult_outgoing" : "tri_mult_incoming");
    LF_TRY(tri_mult(ctx, x));
  }
  for (int end = 0; end < 2; ++end) {  // 7, 8. triangle attention starting, ending
    lf_attention_args x{};
    x.batch = a.length;
    x.queries = a.length;
    x.channels = a.c_z;
    x.heads = end ? w.tri_att_end_heads : w.tri_att_start_heads;
    x.transpose = end;
    x.act_dtype = a.pair_dtype;
    x.act = a.pair;
    x.mask = a.pair_mask;
    x.out = a.pair;
    x.accumulate = 1;
    x.bias_mode = LF_BIAS_NORMALIZED_INPUT;
    x.epsilon = eps;
    x.w = end ? &w.tri_att_end : &w.tri_att_start;
    StageScope stage(ctx, end ? "tri_attention_ending" : "tri_attention_starting");
    LF_TRY(attention(ctx, x));
  }
  {  // 9. pair transition
    lf_transition_args x{};
    x.kind = LF_TRANSITION_RELU;
    x.rows = a.length * a.length;
    x.channels = a.c_z;
    x.hidden = a.pair_hidden;
    x.act_dtype = a.pair_dtype;
    x.act = a.pair;
    x.out = a.pair;
    x.accumulate = 1;
    x.chunk_bytes = chunk;
    x.epsilon = eps;
    x.w = &w.pair_transition;
    StageScope stage(ctx, "pair_transition");
    LF_TRY(transition(ctx, x));
  }
  return LF_OK;
}

static int pairformer_block(lf_context* ctx, const lf_pairformer_block_args& a) {
  LF_REQUIRE(a.w != nullptr, "pairformer block: weights are NULL");
  LF_REQUIRE(a.tokens > 0 && a.c_z > 0, "pairformer block dimensions must be positive");
  LF_REQUIRE(a.pair && a.pair_mask, "pairformer block: NULL pair or pair mask");
  const lf_pairformer_weights& w = *a.w;
  const float eps = a.epsilon > 0.f ? a.epsilon : 1e-5f;
  const long long chunk = a.transition_chunk_bytes > 0 ? a.transition_chunk_bytes : (1LL << 30);
  const int N = a.tokens;
  for (int dir = 0; dir < 2; ++dir) {
    lf_tri_mult_args x{};
    x.direction = dir == 0 ? LF_OUTGOING : LF_INCOMING;
    x.dialect = LF_AF3;
    x.divide_by_length = a.divide_by_length;
    x.length = N;
    x.c_z = a.c_z;
    x.c_hidden = a.c_z;
    x.act_dtype = a.pair_dtype;
    x.z = a.pair;
    x.mask = a.pair_mask;
    x.out = a.pair;
    x.accumulate = 1;
    x.epsilon = eps;
    x.w = dir == 0 ? &w.tri_out : &w.tri_in;
    StageScope stage(ctx, dir == 0 ? "tri_mult_outgoing" : "tri_mult_incoming");
    LF_TRY(tri_mult(ctx, x));
  }
  for (int end = 0; end < 2; ++end) {
    lf_attention_args x{};
    x.batch = N;
    x.queries = N;
    x.channels = a.c_z;
    x.heads = w.pair_heads;
    x.transpose = end;
    x.act_dtype = a.pair_dtype;
    x.act = a.pair;
    x.mask = a.pair_mask;
    x.out = a.pair;
    x.accumulate = 1;
    x.fast_variance = 1;
    x.bias_mode = LF_BIAS_NORMALIZED_INPUT;
    // the bias comes from the untransposed pair unless the dialect swaps it
    // (cpu/af3/trunk/pairformer.js:338-353); the library's swap is relative to the
    // transposed logical rows
    x.swap_bias = end && !a.swap_transposed_bias;
    x.epsilon = eps;
    x.w = end ? &w.att_end : &w.att_start;
    StageScope stage(ctx, end ? "tri_attention_ending" : "tri_attention_starting");
    LF_TRY(attention(ctx, x));
  }
  {
    lf_transition_args x{};
    x.kind = LF_TRANSITION_SWIGLU;
    x.rows = N * N;
    x.channels = a.c_z;
    x.hidden = 4 * a.c_z;
    x.act_dtype = a.pair_dtype;
    x.act = a.pair;
    x.out = a.pair;
    x.accumulate = 1;
    x.fast_variance = 1;
    x.chunk_bytes = chunk;
    x.epsilon = eps;
    x.w = &w.pair_transition;
    StageScope stage(ctx, "pair_transition");
    LF_TRY(transition(ctx, x));
  }
  if (!a.single) return LF_OK;
  LF_REQUIRE(a.seq_mask && a.c_s > 0, "pairformer block: single track needs seq_mask and c_s");
  {
    lf_attention_weights sw = w.single_attention;
    sw.pair_norm_scale = w.single_logits_norm_scale;
    sw.pair_norm_offset = w.single_logits_norm_offset;
    sw.wb = w.single_logits_projection;
    lf_attention_args x{};
    x.batch = 1;
    x.queries = N;
    x.channels = a.c_s;
    x.heads = w.single_heads;
    x.head_dim = w.single_head_dim;
    x.act_dtype = a.single_dtype;
    x.act = a.single;
    x.mask = a.seq_mask;
    x.out = a.single;
    x.accumulate = 1;
    x.fast_variance = 1;
    x.bias_mode = LF_BIAS_SEPARATE;
    x.pair_dtype = a.pair_dtype;
    x.pair = a.pair;
    x.pair_channels = a.c_z;
    x.epsilon = eps;
    x.w = &sw;
    StageScope stage(ctx, "single_attention");
    LF_TRY(attention(ctx, x));
  }
  {
    lf_transition_args x{};
    x.kind = LF_TRANSITION_SWIGLU;
    x.rows = N;
    x.channels = a.c_s;
    x.hidden = 4 * a.c_s;
    x.act_dtype = a.single_dtype;
    x.act = a.single;
    x.out = a.single;
    x.accumulate = 1;
    x.fast_variance = 1;
    x.chunk_bytes = chunk;
    x.epsilon = eps;
    x.w = &w.single_transition;
    StageScope stage(ctx, "single_transition");
    LF_TRY(transition(ctx, x));
  }
  return LF_OK;
}

// AF3 pair-weighted averaging (msaAttention, cpu/af3/trunk/msa.js:157-219) as gated attention
// whose logits are the pair bias alone (no queries, no keys) over one key mask shared by every
// sequence, the mask's maximum over the sequences (:177-186).  Both layer norms use the fast
// variance (cpu/af3/trunk/pairformer.js:70-87); there are no biases.
static int pair_weighted_averaging(lf_context* ctx, const lf_pair_averaging_args& a) {
  LF_REQUIRE(a.w != nullptr, "pair-weighted averaging: weights are NULL");
  LF_REQUIRE(a.sequences > 0 && a.tokens > 0 && a.c_m > 0 && a.c_z > 0 && a.heads > 0 && a.head_dim > 0,
             "pair-weighted averaging dimensions must be positive");
  LF_REQUIRE(a.msa && a.msa_mask && a.pair && a.out, "pair-weighted averaging: NULL msa, mask, pair or out");
  const lf_pair_averaging_weights& w = *a.w;
  lf_attention_weights aw{};
  aw.norm_scale = w.act_norm_scale;
  aw.norm_offset = w.act_norm_offset;
  aw.wv = w.wv;
  aw.wg = w.wg;
  aw.wo = w.wo;
  aw.pair_norm_scale = w.pair_norm_scale;
  aw.pair_norm_offset = w.pair_norm_offset;
  aw.wb = w.pair_logits;
  lf_attention_args x{};
  x.batch = a.sequences;
  x.queries = a.tokens;
  x.channels = a.c_m;
  x.heads = a.heads;
  x.head_dim = a.head_dim;
  x.act_dtype = a.msa_dtype;
  x.act = a.msa;
  x.mask = a.msa_mask;
  x.out = a.out;
  x.accumulate = a.accumulate;
  x.fast_variance = 1;
  x.bias_mode = LF_BIAS_SEPARATE;
  x.pair_dtype = a.pair_dtype;
  x.pair = a.pair;
  x.pair_channels = a.c_z;
  x.epsilon = a.epsilon > 0.f ? a.epsilon : 1e-5f;
  x.w = &aw;
  return attention(ctx, x, /*no_qk=*/true, /*shared_key_mask=*/true);
}

// One AF3 MSA-module block (msaBlock, cpu/af3/trunk/msa.js:233-287).
static int msa_module_block(lf_context* ctx, const lf_msa_block_args& a) {
  LF_REQUIRE(a.w != nullptr, "msa module block: weights are NULL");
  LF_REQUIRE(a.sequences > 0 && a.tokens > 0 && a.c_m > 0 && a.c_z > 0, "msa module block dimensions must be positive");
  LF_REQUIRE(a.msa && a.pair && a.msa_mask && a.pair_mask, "msa module block: NULL activation or mask");
  const lf_msa_module_weights& w = *a.w;
  const float eps = a.epsilon > 0.f ? a.epsilon : 1e-5f;
  const long long chunk = a.transition_chunk_bytes > 0 ? a.transition_chunk_bytes : (1LL << 30);
  auto opm = [&]() -> int {
    lf_opm_args x{};
    x.sequences = a.sequences;
    x.length = a.tokens;
    x.c_m = a.c_m;
    x.c_outer = w.c_outer;
    x.c_z = a.c_z;
    x.msa_dtype = a.msa_dtype;
    x.msa = a.msa;
    x.mask = a.msa_mask;
    x.pair_dtype = a.pair_dtype;
    x.pair_in = a.pair;
    x.out = a.pair;
    x.accumulate = 1;
    x.fast_variance = 1;
    x.epsilon = eps;
    x.norm_epsilon = 1e-3f;
    x.w = &w.outer_product_mean;
    StageScope stage(ctx, "outer_product_mean");
    return outer_product_mean(ctx, x);
  };
  // the MSA update: the averaging and the transition move together (msa.js:259-263)
  auto update = [&]() -> int {
    {
      lf_pair_averaging_args x{};
      x.sequences = a.sequences;
      x.tokens = a.tokens;
      x.c_m = a.c_m;
      x.c_z = a.c_z;
      x.heads = w.msa_heads;
      x.head_dim = w.msa_head_dim;
      x.msa_dtype = a.msa_dtype;
      x.msa = a.msa;
      x.msa_mask = a.msa_mask;
      x.pair_dtype = a.pair_dtype;
      x.pair = a.pair;
      x.out = a.msa;
      x.accumulate = 1;
      x.epsilon = eps;
      x.w = &w.msa_attention;
      StageScope stage(ctx, "pair_weighted_averaging");
      LF_TRY(pair_weighted_averaging(ctx, x));
    }
    lf_transition_args x{};
    x.kind = LF_TRANSITION_SWIGLU;
    x.rows = a.sequences * a.tokens;
    x.channels = a.c_m;
    x.hidden = 4 * a.c_m;
    x.act_dtype = a.msa_dtype;
    x.act = a.msa;
    x.out = a.msa;
    x.accumulate = 1;
    x.fast_variance = 1;
    x.chunk_bytes = chunk;
    x.epsilon = eps;
    x.w = &w.msa_transition;
    StageScope stage(ctx, "msa_transition");
    return transition(ctx, x);
  };
  if (a.msa_update_before_opm) {
    LF_TRY(update());
    LF_TRY(opm());
  } else {
    LF_TRY(opm());
    LF_TRY(update());
  }
  lf_pairformer_block_args p{};
  p.tokens = a.tokens;
  p.c_z = a.c_z;
  p.swap_transposed_bias = a.swap_transposed_bias;
  p.divide_by_length = a.divide_by_length;
  p.pair_dtype = a.pair_dtype;
  p.pair = a.pair;
  p.pair_mask = a.pair_mask;
  p.transition_chunk_bytes = a.transition_chunk_bytes;
  p.epsilon = eps;
  p.w = &w.pair;
  return pairformer_block(ctx, p);
}

}  // namespace lf

extern "C" {

int lf_msa_pair_weighted_averaging(lf_context* ctx, const lf_pair_averaging_args* args) {
  if (!ctx || !args) return lf::set_error(LF_ERR_INVALID, "lf_msa_pair_weighted_averaging: NULL argument");
  hipSetDevice(ctx->device);
  return lf::pair_weighted_averaging(ctx, *args);
}

int lf_af2_recycle(lf_context* ctx, const lf_af2_recycle_args* args) {
  if (!ctx || !args) return lf::set_error(LF_ERR_INVALID, "lf_af2_recycle: NULL argument");
  if (args->extra_block_count < 0 || args->main_block_count < 0 || (args->extra_block_count > 0 && !args->extra_blocks) ||
      (args->main_block_count > 0 && !args->main_blocks))
    return lf::set_error(LF_ERR_INVALID, "lf_af2_recycle: bad block list");
  const lf_af2_recycle_args& a = *args;
  if ((a.main_block_count > 0 && (a.main.pair != a.embed.pair || a.main.msa != a.embed.msa)) ||
      (a.extra_block_count > 0 && (a.extra.pair != a.embed.pair || a.extra.msa != a.embed.extra)))
    return lf::set_error(LF_ERR_INVALID, "lf_af2_recycle: the stacks must run on the embedder's outputs");
  hipSetDevice(ctx->device);
  {
    lf::StageScope stage(ctx, "input_embedder");
    LF_TRY(lf::input_embedder(ctx, a.embed));
  }
  lf::MaskScope masks(ctx);   // the stacks' masks are inputs: their derived tables, once
  for (int b = 0; b < a.extra_block_count; ++b)
    LF_TRY(lf::evoformer_block(ctx, a.extra, a.extra_blocks[b].base, &a.extra_blocks[b].column_global,
                               a.extra_blocks[b].column_global_heads));
  for (int b = 0; b < a.main_block_count; ++b) LF_TRY(lf::evoformer_block(ctx, a.main, a.main_blocks[b]));
  return LF_OK;
}

int lf_msa_module_block(lf_context* ctx, const lf_msa_block_args* args) {
  if (!ctx || !args) return lf::set_error(LF_ERR_INVALID, "lf_msa_module_block: NULL argument");
  hipSetDevice(ctx->device);
  return lf::msa_module_block(ctx, *args);
}

int lf_evoformer_block(lf_context* ctx, const lf_evoformer_block_args* args) {
  if (!ctx || !args || !args->w) return lf::set_error(LF_ERR_INVALID, "lf_evoformer_block: NULL argument");
  hipSetDevice(ctx->device);
  return lf::evoformer_block(ctx, *args, *args->w);
}

int lf_evoformer_stack(lf_context* ctx, const lf_evoformer_block_args* args, const lf_evoformer_weights* blocks,
                       int block_count) {
  if (!ctx || !args || (!blocks && block_count > 0)) return lf::set_error(LF_ERR_INVALID, "lf_evoformer_stack: NULL argument");
  if (block_count < 0) return lf::set_error(LF_ERR_INVALID, "lf_evoformer_stack: negative block count");
  hipSetDevice(ctx->device);
  lf::MaskScope masks(ctx);   // the masks' key-bias rows and OPM normalisers, once per stack
  for (int i = 0; i < block_count; ++i) LF_TRY(lf::evoformer_block(ctx, *args, blocks[i]));
  return LF_OK;
}

int lf_extra_msa_block(lf_context* ctx, const lf_evoformer_block_args* args, const lf_extra_msa_weights* w) {
  if (!ctx || !args || !w) return lf::set_error(LF_ERR_INVALID, "lf_extra_msa_block: NULL argument");
  hipSetDevice(ctx->device);
  return lf::evoformer_block(ctx, *args, w->base, &w->column_global, w->column_global_heads);
}

int lf_extra_msa_stack(lf_context* ctx, const lf_evoformer_block_args* args, const lf_extra_msa_weights* blocks,
                       int block_count) {
  if (!ctx || !args || (!blocks && block_count > 0)) return lf::set_error(LF_ERR_INVALID, "lf_extra_msa_stack: NULL argument");
  if (block_count < 0) return lf::set_error(LF_ERR_INVALID, "lf_extra_msa_stack: negative block count");
  hipSetDevice(ctx->device);
  lf::MaskScope masks(ctx);
  for (int b = 0; b < block_count; ++b)
    LF_TRY(lf::evoformer_block(ctx, *args, blocks[b].base, &blocks[b].column_global, blocks[b].column_global_heads));
  return LF_OK;
}

int lf_evoformer_pair_stack(lf_context* ctx, const lf_evoformer_block_args* args, const lf_evoformer_weights* blocks,
                            int block_count) {
  if (!ctx || !args || (!blocks && block_count > 0))
    return lf::set_error(LF_ERR_INVALID, "lf_evoformer_pair_stack: NULL argument");
  if (block_count < 0) return lf::set_error(LF_ERR_INVALID, "lf_evoformer_pair_stack: negative block count");
  hipSetDevice(ctx->device);
  lf::MaskScope masks(ctx);
  for (int b = 0; b < block_count; ++b) LF_TRY(lf::evoformer_block(ctx, *args, blocks[b], nullptr, 0, true));
  return LF_OK;
}

int lf_pairformer_block(lf_context* ctx, const lf_pairformer_block_args* args) {
  if (!ctx || !args) return lf::set_error(LF_ERR_INVALID, "lf_pairformer_block: NULL argument");
  hipSetDevice(ctx->device);
  return lf::pairformer_block(ctx, *args);
}

}  // extern "C"
