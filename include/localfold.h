/*
 * localfold.h - C ABI of the MI355X (gfx950) pair-stack library, liblocalfold.so.
 *
 * The reference (sokrypton/localfold) exposes this path as JavaScript classes over
 * WebGPU (webgpu/index.js:1-8): TriangleMultiplication{Outgoing,Incoming}Gpu, AttentionGpu,
 * OuterProductMeanGpu, TransitionGpu, EvoformerBlockGpu, EvoformerStackGpu, plus the AF3
 * trunk classes (webgpu/af3/trunk/).  Each entry point below is what a binding of one of
 * those classes' `run()` calls once its input has been validated and copied to the device;
 * the citation on each names the reference interface it replaces.
 *
 * Conventions
 *  - Every tensor pointer is a DEVICE pointer (hipMalloc'd, or a torch CUDA tensor's
 *    data_ptr); shapes are plain ints; work is enqueued on the context's stream and the
 *    call returns without waiting (lf_synchronize waits).
 *  - Activation dtype codes: LF_F32, LF_F16, LF_BF16.  Layer-norm scales/offsets, biases
 *    and masks are always float32 (the reference keeps them float32:
 *    tools/quantize_af3.py:57, KEEP_FLOAT32).
 *  - Weights are lf_weight records: float32/float16/bfloat16 values, or the reference's
 *    codecs decoded on the device - int8 symmetric (code*scale) and int5 asymmetric
 *    (code*scale+zero, LSB-first 5-bit codes, one slack byte), fp16 scale/zero tables
 *    (shared/weights/dtype.js:212-406) - inside the triangle-multiplication kernels and the
 *    weight-resident output projections as they stage them into LDS, and by one short
 *    per-call pass for the streaming projections, transitions and OPM.  `group` > 0 is the reference's flat group map
 *    (group index = flat stored index / group: 64 for int8, 32 for int5); `group` == 0
 *    is one group per output channel.
 *  - Return value: LF_OK, or an error code; lf_last_error() holds the message
 *    (thread-local).  Invalid shapes are rejected before anything is enqueued, the way
 *    the reference's validate() throws a RangeError (webgpu/kernels/triangle/types.js:13-48).
 *  - "accumulate" = 0 writes the op's update (what the reference's class returns);
 *    1 writes input + update into `out`, which may alias the input (the in-place residual
 *    of webgpu/af2/evoformer/block.js:1536-1629).
 */
#ifndef LOCALFOLD_H
#define LOCALFOLD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lf_context lf_context;

enum { LF_OK = 0, LF_ERR_INVALID = 1, LF_ERR_DEVICE = 2, LF_ERR_MEMORY = 3, LF_ERR_UNSUPPORTED = 4 };
enum { LF_F32 = 0, LF_F16 = 1, LF_BF16 = 2, LF_INT8 = 3, LF_INT5 = 4 };
enum { LF_IN_OUT = 0, LF_OUT_IN = 1 };
enum { LF_OUTGOING = 0, LF_INCOMING = 1 };
enum { LF_AF2 = 0, LF_AF3 = 1 };

/* One stored weight tensor: `rows` x `cols` in storage order.  LF_IN_OUT: rows = inputs,
 * cols = outputs (Haiku / AF3 layout).  LF_OUT_IN: rows = outputs, cols = inputs (the
 * (out,in) layout of webgpu/kernels/triangle/types.js:28-43). */
typedef struct {
  int dtype;            /* LF_F32 / LF_F16 / LF_BF16 / LF_INT8 / LF_INT5 */
  int layout;           /* LF_IN_OUT or LF_OUT_IN */
  int rows, cols;
  int group;            /* quantised only: flat group size, or 0 = per output channel */
  const void* data;     /* values, or codes; int5 codes must stay readable for 4 bytes past
                           the last code byte (the reference's records hold a slack byte and
                           the scale table there; the kernels fetch aligned word pairs) */
  const void* scales;   /* fp16, one per group (quantised) */
  const void* zeros;    /* fp16, one per group (int5) */
} lf_weight;

/* ---- context, memory, stream, timing ------------------------------------------------- */

/* Replaces the WebGPU device of webgpu/node.js:51-81 / webgpu/runtime/device.js:98. */
lf_context* lf_context_create(int device_ordinal);
void lf_context_destroy(lf_context* ctx);
/* Enqueue on an existing hipStream_t (e.g. torch's current stream); NULL is the HIP null stream.
 * A new context starts on a non-blocking stream of its own. */
int lf_context_set_stream(lf_context* ctx, void* hip_stream);
const char* lf_last_error(void);
const char* lf_version(void);

/* Device memory owned by the caller (webgpu/runtime/allocator.js:55 GpuBufferAllocator). */
int lf_malloc(lf_context* ctx, size_t bytes, void** out);
int lf_free(lf_context* ctx, void* ptr);
int lf_memcpy_htod(lf_context* ctx, void* dst, const void* src, size_t bytes);
int lf_memcpy_dtoh(lf_context* ctx, void* dst, const void* src, size_t bytes);
int lf_memset(lf_context* ctx, void* dst, int value, size_t bytes);
int lf_synchronize(lf_context* ctx);
/* {currentBytes, peakBytes, allocationCount} of webgpu/runtime/allocator.js:188-194,
 * counting caller allocations, the context's scratch workspace and its mask tables.  Not
 * counted: the library's static LF_TRI_NOALLOC_SCRATCH_BYTES array, which every device the
 * library loads on holds until the process ends (see lf_tri_mult_noalloc). */
int lf_memory_stats(lf_context* ctx, size_t* current_bytes, size_t* peak_bytes, size_t* allocation_count);

/* Per-kernel timestamps (webgpu/runtime/execution.js:673-727 readTimestampProfile):
 * when enabled, every kernel launch is bracketed by hipEvents on the context stream. */
typedef struct {
  char label[48];
  float ms;
} lf_kernel_timing;
int lf_profile_enable(lf_context* ctx, int enable);
/* Waits for the stream, copies up to `max` records, returns the count (and clears them). */
int lf_profile_read(lf_context* ctx, lf_kernel_timing* out, int max);

/* ---- triangle multiplicative update -------------------------------------------------- */

/* AF2 (dialect LF_AF2): the sixteen tensors of webgpu/kernels/triangle/types.js:28-43 with
 * projection weights ap, ag, bp, bg [cH x cZ], wz [cZ x cH], wg [cZ x cZ], usually LF_OUT_IN.
 * AF3 (dialect LF_AF3, cpu/af3/trunk/pairformer.js:213-300): no biases, fast-variance LN,
 * `ap` = fused projection [cZ x 2cZ] and `ag` = fused gate [cZ x 2cZ] (a = column 2c,
 * b = column 2c+1), wz = outputProjection, wg = gatingLinear; bp/bg unused. */
typedef struct {
  const float *ln_in_scale, *ln_in_offset;
  lf_weight ap, ag, bp, bg;
  const float *ap_bias, *ag_bias, *bp_bias, *bg_bias;
  const float *ln_out_scale, *ln_out_offset;
  lf_weight wz;
  const float* wz_bias;
  lf_weight wg;
  const float* wg_bias;
} lf_tri_mult_weights;

typedef struct {
  int direction;          /* LF_OUTGOING: x_ij = sum_k a_ik b_jk; LF_INCOMING: sum_k a_kj b_ki */
  int dialect;            /* LF_AF2 or LF_AF3 */
  int divide_by_length;   /* AF3 rf3 dialect: x /= N before the centre norm */
  int length, c_z, c_hidden;
  int act_dtype;
  const void* z;          /* [N, N, cZ] */
  const float* mask;      /* [N, N] */
  void* out;              /* [N, N, cZ], act_dtype */
  int accumulate;
  float epsilon;          /* 1e-5 in the reference */
  const lf_tri_mult_weights* w;
} lf_tri_mult_args;

/* Replaces TriangleMultiplication{Outgoing,Incoming}Gpu.run (webgpu/kernels/triangle/webgpu.js:38-169)
 * and encodeTriangleMultiplication (webgpu/af2/evoformer/block.js:1288-1535). */
int lf_tri_mult(lf_context* ctx, const lf_tri_mult_args* args);

/* No counterpart in the reference: lf_tri_mult for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as lf_tri_mult, but its scratch (the a, b and X planes,
 * 3 * c_hidden * N^2 f16, plus 8 * N^2 bytes of LayerNorm statistics with 2-byte activations
 * at c_z = c_hidden = 128; weights are decoded while being staged into LDS, so they take no
 * scratch) lives in a static per-device array of LF_TRI_NOALLOC_SCRATCH_BYTES (reserved on
 * every device the library loads on, used or not), looked up once per device by
 * lf_context_create; nothing is
 * allocated or freed.  Shapes needing more scratch are rejected with LF_ERR_INVALID (c_hidden
 * 128 fits N <= 415, or 417 with f32 activations).  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams, two threads, two contexts) race, so
 * serialise them. */
#define LF_TRI_NOALLOC_SCRATCH_BYTES (128u << 20)
int lf_tri_mult_noalloc(lf_context* ctx, const lf_tri_mult_args* args);

/* ---- gated attention (MSA row / column, triangle starting / ending, AF3 grid / single) -- */

enum { LF_BIAS_NONE = 0, LF_BIAS_SEPARATE = 1, LF_BIAS_NORMALIZED_INPUT = 2, LF_BIAS_LOGITS = 3 };

typedef struct {
  const float *norm_scale, *norm_offset;
  lf_weight wq, wk, wv, wg, wo;          /* [C x H*d] / [H*d x C] in either layout */
  const float *q_bias, *g_bias, *o_bias; /* optional (NULL = none) */
  /* pair bias: LF_BIAS_SEPARATE uses pair_norm_* and wb [Cpair x H];
   * LF_BIAS_NORMALIZED_INPUT uses wb [C x H] on the normalised attention input */
  const float *pair_norm_scale, *pair_norm_offset;
  lf_weight wb;
} lf_attention_weights;

typedef struct {
  int batch, queries, channels, heads;
  int head_dim;           /* 0: channels / heads (AF2) */
  int transpose;          /* logical row (b,q) is storage row (q,b); key mask at [k,b] */
  int act_dtype;
  const void* act;        /* storage [batch*queries, C] (or [queries*batch, C] when transposed) */
  const float* mask;      /* storage order, batch*queries */
  void* out;
  int accumulate;
  int fast_variance;      /* AF3 layer norms */
  int bias_mode;          /* LF_BIAS_* */
  int swap_bias;          /* AF3 openfold dialect: bias[h][i][j] read at [j][i] when transposed */
  int pair_dtype;
  const void* pair;       /* LF_BIAS_SEPARATE: [queries, queries, pair_channels] */
  int pair_channels;
  const float* bias_logits; /* LF_BIAS_LOGITS: [H, queries, queries] float32 */
  float epsilon;
  const lf_attention_weights* w;
} lf_attention_args;

/* Replaces AttentionGpu.run (webgpu/kernels/attention.js:2580-2739) and encodeAttention
 * (webgpu/af2/evoformer/block.js:647-952); AF3 gridSelfAttention / singleAttention
 * (cpu/af3/trunk/pairformer.js:322-485) through the same entry. */
int lf_attention(lf_context* ctx, const lf_attention_args* args);

/* ---- transition ----------------------------------------------------------------------- */

enum { LF_TRANSITION_RELU = 0, LF_TRANSITION_SWIGLU = 1 };

typedef struct {
  const float *norm_scale, *norm_offset;
  lf_weight w1;           /* RELU: [C x H]; SWIGLU: [C x 2H], gate half first (blocked split) */
  const float* b1;
  lf_weight w2;           /* [H x C] */
  const float* b2;
} lf_transition_weights;

typedef struct {
  int kind;               /* LF_TRANSITION_RELU (AF2) or LF_TRANSITION_SWIGLU (AF3) */
  int rows, channels, hidden;
  int act_dtype;
  const void* act;
  void* out;
  int accumulate;
  int fast_variance;
  long long chunk_bytes;  /* hidden-buffer budget per chunk; 0 = 32 MiB (transition.js:377) */
  float epsilon;
  const lf_transition_weights* w;
} lf_transition_args;

/* Replaces TransitionGpu.run (webgpu/kernels/transition.js:1009-1105), encodeTransition
 * (block.js:488-646) and AF3 transition (cpu/af3/trunk/pairformer.js:180-201). */
int lf_transition(lf_context* ctx, const lf_transition_args* args);

/* ---- outer product mean --------------------------------------------------------------- */

typedef struct {
  const float *norm_scale, *norm_offset;
  lf_weight wl, wr;        /* [cM x cOuter] */
  const float *bl, *br;    /* optional */
  lf_weight wo;            /* [cOuter*cOuter x cZ] */
  const float* bo;         /* optional */
} lf_opm_weights;

typedef struct {
  int sequences, length, c_m, c_outer, c_z;
  int msa_dtype;
  const void* msa;         /* [S, N, cM] */
  const float* mask;       /* [S, N] */
  int pair_dtype;
  const void* pair_in;     /* residual source when accumulate (may alias out) */
  void* out;               /* [N, N, cZ] */
  int accumulate;
  int fast_variance;
  float epsilon;           /* layer norm, 1e-5 */
  float norm_epsilon;      /* 1e-3 */
  const lf_opm_weights* w;
} lf_opm_args;

/* Replaces OuterProductMeanGpu.run (webgpu/kernels/outer-product-mean.js:1748-1907) and
 * AF3 outerProductMean (cpu/af3/trunk/msa.js:72-155). */
int lf_outer_product_mean(lf_context* ctx, const lf_opm_args* args);

/* ---- global column attention (AF2 extra-MSA stack) ---------------------------------- */

typedef struct {
  const float *norm_scale, *norm_offset;  /* queryNormScale / queryNormOffset */
  lf_weight wq;             /* [C x H*d] */
  lf_weight wk, wv;         /* [C x d]: one key/value head shared by every query head */
  lf_weight wg;             /* [C x H*d] */
  const float* g_bias;      /* [H*d] */
  lf_weight wo;             /* [H*d x C] */
  const float* o_bias;      /* [C], optional */
} lf_global_attention_weights;

typedef struct {
  int sequences, length, channels, heads;
  int head_dim;             /* 0: channels / heads */
  int act_dtype;
  const void* act;          /* [S, N, C] */
  const float* mask;        /* [S, N] */
  void* out;                /* [S, N, C], act_dtype; may alias act when accumulate */
  int accumulate;
  float epsilon;            /* layer norm, 1e-5 */
  const lf_global_attention_weights* w;
} lf_global_attention_args;

/* Replaces encodeGlobalAttention (webgpu/af2/evoformer/block.js:953-1030) and its kernels
 * (block.js:88-400): per residue column, attention of the masked-mean query over the
 * sequences (a masked sequence's logit is -1e9), gated per sequence, projected out. */
int lf_global_column_attention(lf_context* ctx, const lf_global_attention_args* args);

/* ---- blocks --------------------------------------------------------------------------- */

typedef struct {
  lf_attention_weights row_attention;     int row_heads;
  lf_attention_weights column_attention;  int column_heads;
  lf_transition_weights msa_transition;
  lf_opm_weights outer_product_mean;
  lf_tri_mult_weights tri_out, tri_in;
  lf_attention_weights tri_att_start;     int tri_att_start_heads;
  lf_attention_weights tri_att_end;       int tri_att_end_heads;
  lf_transition_weights pair_transition;
} lf_evoformer_weights;

typedef struct {
  int sequences, length, c_m, c_z, c_outer, tri_hidden, msa_hidden, pair_hidden;
  int msa_dtype;  void* msa;     /* [S, N, cM], updated in place */
  int pair_dtype; void* pair;    /* [N, N, cZ], updated in place */
  const float* msa_mask;         /* [S, N] */
  const float* pair_mask;        /* [N, N] */
  float epsilon;
  const lf_evoformer_weights* w;
} lf_evoformer_block_args;

/* Replaces EvoformerBlockGpu.run / encodeEvoformerBlock (webgpu/af2/evoformer/block.js:1536-1629,
 * 1783-1824): row attention with pair bias, column attention, MSA transition, OPM,
 * triangle multiplication out/in, triangle attention start/end, pair transition. */
int lf_evoformer_block(lf_context* ctx, const lf_evoformer_block_args* args);

/* Replaces EvoformerStackGpu.run (webgpu/af2/evoformer/stack.js:44-160): `blocks` blocks in order. */
int lf_evoformer_stack(lf_context* ctx, const lf_evoformer_block_args* args, const lf_evoformer_weights* blocks,
                       int block_count);

/* The extra-MSA block's weights: the Evoformer block's (column_attention and column_heads
 * unused) with the global column attention in its place. */
typedef struct {
  lf_evoformer_weights base;
  lf_global_attention_weights column_global;
  int column_global_heads;
} lf_extra_msa_weights;

/* Replaces encodeExtraMsaBlock (webgpu/af2/evoformer/block.js:1715-1744): row attention with
 * pair bias, global column attention, MSA transition, then the pair steps of
 * encodeEvoformerPairBlock (block.js:1663-1713).  args->w is not read. */
int lf_extra_msa_block(lf_context* ctx, const lf_evoformer_block_args* args, const lf_extra_msa_weights* w);

/* Replaces ExtraMsaStackGpu.run (webgpu/af2/evoformer/stack.js:249-330): `block_count`
 * extra-MSA blocks in order on the same msa and pair. */
int lf_extra_msa_stack(lf_context* ctx, const lf_evoformer_block_args* args, const lf_extra_msa_weights* blocks,
                       int block_count);

/* Replaces ExtraMsaPairStackGpu.run (webgpu/af2/evoformer/stack.js:163-247), whose blocks
 * are encodeEvoformerPairBlock (webgpu/af2/evoformer/block.js:1663-1713): per block the outer
 * product mean of the (unchanged) msa into the pair, triangle multiplication out/in, triangle
 * attention start/end and the pair transition.  The msa is read, never written; the weights'
 * MSA-side records (row/column attention, MSA transition) are not read. */
int lf_evoformer_pair_stack(lf_context* ctx, const lf_evoformer_block_args* args, const lf_evoformer_weights* blocks,
                            int block_count);

typedef struct {
  lf_tri_mult_weights tri_out, tri_in;
  lf_attention_weights att_start, att_end;  int pair_heads;
  lf_transition_weights pair_transition;
  const float *single_logits_norm_scale, *single_logits_norm_offset;
  lf_weight single_logits_projection;       /* [cZ x Hs] */
  lf_attention_weights single_attention;  int single_heads, single_head_dim;
  lf_transition_weights single_transition;
} lf_pairformer_weights;

typedef struct {
  int tokens, c_z, c_s;
  int swap_transposed_bias, divide_by_length;
  int pair_dtype; void* pair;    /* [N, N, cZ] in place */
  int single_dtype; void* single;/* [N, cS] in place, or NULL for a pair-only block */
  const float* pair_mask;        /* [N, N] */
  const float* seq_mask;         /* [N] */
  long long transition_chunk_bytes;
  float epsilon;
  const lf_pairformer_weights* w;
} lf_pairformer_block_args;

/* Replaces one block of Af3PairformerStackGpu.run (webgpu/af3/trunk/pairformer-block.js:246-308),
 * in pairformerBlock order (cpu/af3/trunk/pairformer.js:495-541). */
int lf_pairformer_block(lf_context* ctx, const lf_pairformer_block_args* args);

/* ---- AF2 input and recycling embedder -------------------------------------------------- */

/* All f32 on the device, (in,out) layout (InputEmbedderGpu's packWeights,
 * webgpu/af2/evoformer/input-embedder.js:9-26). */
typedef struct {
  const float *preprocess_1d_w, *preprocess_1d_b;     /* [Ct x cM], [cM] */
  const float *preprocess_msa_w, *preprocess_msa_b;   /* [Cf x cM], [cM] */
  const float *left_w, *left_b, *right_w, *right_b;   /* [Ct x cZ], [cZ] */
  const float *prev_pos_w, *prev_pos_b;               /* [15 x cZ], [cZ] */
  const float *prev_msa_norm_scale, *prev_msa_norm_offset;    /* [cM] */
  const float *prev_pair_norm_scale, *prev_pair_norm_offset;  /* [cZ] */
  const float *relpos_w, *relpos_b;                   /* [65 x cZ], [cZ] */
  const float *extra_w, *extra_b;                     /* [25 x cE], [cE] */
} lf_input_embedder_weights;

typedef struct {
  int length, msa_sequences, extra_sequences;
  int target_channels, msa_feature_channels;          /* 22, 49 in AF2 */
  int c_m, c_z, c_e;                                  /* 256, 128, 64 */
  const float* target_feat;       /* [L, Ct] */
  const float* msa_feat;          /* [S, L, Cf] */
  const float* extra_msa;         /* [Se, L] residue codes 0..22 as f32 */
  const float* extra_has_deletion;    /* [Se, L] */
  const float* extra_deletion_value;  /* [Se, L] */
  const float* residue_index;     /* [L] */
  const float* aatype;            /* [L] */
  const void* prev_msa_first_row; /* [L, cM], msa_dtype; NULL = zeros (recycle 0) */
  const void* prev_pair;          /* [L, L, cZ], pair_dtype; NULL = zeros */
  const float* prev_positions;    /* [L, 37, 3] atom37; NULL = zeros */
  int msa_dtype;   void* msa;     /* out [S, L, cM] */
  int pair_dtype;  void* pair;    /* out [L, L, cZ]; may alias prev_pair (read and written per row) */
  int extra_dtype; void* extra;   /* out [Se, L, cE] */
  float epsilon;                  /* 1e-5 */
  const lf_input_embedder_weights* w;
} lf_input_embedder_args;

/* Replaces InputEmbedderGpu.run / encodeInputEmbedder (webgpu/af2/evoformer/input-embedder.js:
 * 160-231): the MSA, pair (without templates) and extra-MSA embeddings of one recycle. */
int lf_input_embedder(lf_context* ctx, const lf_input_embedder_args* args);

/* One AF2 recycle of the trunk before the structure module: the input embedder, the
 * extra-MSA stack on the extra activations and the pair, the Evoformer stack on the msa and
 * the pair.  The carried state is the embedder's recycled inputs: point
 * embed.prev_msa_first_row at main.msa and embed.prev_pair at main.pair (they are read before
 * being overwritten) and the outputs of one call are the recycled inputs of the next.
 * extra.msa = embed.extra, extra.pair = main.pair = embed.pair; extra.w and main.w are not
 * read.  Templates and the structure module are out of scope: prev_positions is the
 * caller's (atom37 from its structure module, or NULL for zeros). */
typedef struct {
  lf_input_embedder_args embed;
  lf_evoformer_block_args extra;  const lf_extra_msa_weights* extra_blocks;  int extra_block_count;
  lf_evoformer_block_args main;   const lf_evoformer_weights* main_blocks;   int main_block_count;
} lf_af2_recycle_args;

/* Replaces one iteration of the recycle loop of AlphaFoldMonomerGpu (webgpu/af2/model/
 * monomer.js:182-330) up to the Evoformer stack's output. */
int lf_af2_recycle(lf_context* ctx, const lf_af2_recycle_args* args);

/* ---- AF3 MSA module ------------------------------------------------------------------- */

/* Pair-weighted averaging weights (`msaAttention1`, cpu/af3/trunk/msa.js:157-219), no biases. */
typedef struct {
  const float *act_norm_scale, *act_norm_offset;    /* [cM] */
  const float *pair_norm_scale, *pair_norm_offset;  /* [cZ] */
  lf_weight pair_logits;                            /* [cZ x H] */
  lf_weight wv, wg;                                 /* [cM x H*d] (vProjection, gatingQuery) */
  lf_weight wo;                                     /* [H*d x cM] (outputProjection) */
} lf_pair_averaging_weights;

typedef struct {
  int sequences, tokens, c_m, c_z, heads, head_dim;
  int msa_dtype;
  const void* msa;          /* [S, N, cM] */
  const float* msa_mask;    /* [S, N]; the key mask is its maximum over the sequences */
  int pair_dtype;
  const void* pair;         /* [N, N, cZ] */
  void* out;                /* [S, N, cM], msa_dtype; may alias msa when accumulate */
  int accumulate;
  float epsilon;            /* layer norms (fast variance), 1e-5 */
  const lf_pair_averaging_weights* w;
} lf_pair_averaging_args;

/* Replaces msaAttention (cpu/af3/trunk/msa.js:157-219): softmax over keys j of
 * LN(pair_ij) . pairLogits[:, h] + 1e9 (max_s mask[s, j] - 1), shared by every sequence,
 * averages x vProjection; gated by sigmoid(x gatingQuery), then outputProjection. */
int lf_msa_pair_weighted_averaging(lf_context* ctx, const lf_pair_averaging_args* args);

typedef struct {
  lf_opm_weights outer_product_mean;  int c_outer;   /* AF3 outer product mean */
  lf_pair_averaging_weights msa_attention;  int msa_heads, msa_head_dim;
  lf_transition_weights msa_transition;              /* SwiGLU, hidden 4 cM */
  lf_pairformer_weights pair;                        /* pair steps; the single fields are not read */
} lf_msa_module_weights;

typedef struct {
  int sequences, tokens, c_m, c_z;
  int msa_update_before_opm;     /* 0: AF3 (OPM of the incoming msa first); 1: OpenDDE / Boltz-2 */
  int swap_transposed_bias, divide_by_length;
  int msa_dtype; void* msa;      /* [S, N, cM] in place */
  int pair_dtype; void* pair;    /* [N, N, cZ] in place */
  const float* msa_mask;         /* [S, N] */
  const float* pair_mask;        /* [N, N] */
  long long transition_chunk_bytes;
  float epsilon;
  const lf_msa_module_weights* w;
} lf_msa_block_args;

/* Replaces msaBlock (cpu/af3/trunk/msa.js:233-287): outer product mean into the pair and the
 * MSA update (pair-weighted averaging, SwiGLU transition) in the dialect's order, then the
 * pair steps of a pair-only pairformer block (triangle multiplications, grid attentions,
 * pair transition). */
int lf_msa_module_block(lf_context* ctx, const lf_msa_block_args* args);

#ifdef __cplusplus
}
#endif
#endif /* LOCALFOLD_H */
