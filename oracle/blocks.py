"""Block and stack order for the AF2 Evoformer and AF3 Pairformer, composed from oracle.ops.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
import numpy as np

from . import ops

F64 = np.float64


def _add(x, delta):
    return (np.asarray(x, F64) + np.asarray(delta, F64)).astype(np.float32)


def evoformer_block_af2(msa, pair, msa_mask, pair_mask, w, eps=1e-5):
    """One AF2 Evoformer block in `encodeEvoformerBlock` order (`webgpu/af2/evoformer/block.js:1536-1629`).

    1 row attention with pair bias, 2 column attention, 3 MSA transition, 4 OPM (+residual),
    5 tri-mult outgoing, 6 incoming, 7 tri-attention starting, 8 ending, 9 pair transition;
    every residual written in place.  `w` is the `syntheticBlockWeights` structure.
    Returns (msa, pair).
    """
    row = w["msaRowAttention"]
    pb = dict(row["pairBias"], source="separate", activations=pair)
    msa = _add(msa, ops.attention_af2(msa, msa_mask, row["attention"], row["heads"], False, pb, eps))
    col = w["msaColumnAttention"]
    # column attention: batch = residues, queries = sequences, transposed storage [S, N, C]
    msa = _add(msa, ops.attention_af2(msa, msa_mask, col["attention"], col["heads"], True, None, eps))
    msa = _add(msa, ops.transition_af2(msa, w["msaTransition"], eps))
    return msa, _pair_steps(msa, pair, msa_mask, pair_mask, w, eps)


def extra_msa_block_af2(msa, pair, msa_mask, pair_mask, w, eps=1e-5):
    """One AF2 extra-MSA block (`encodeExtraMsaBlock`, `webgpu/af2/evoformer/block.js:1715-1744`):
    the Evoformer block with the column attention replaced by global column attention
    (`w["msaColumnGlobalAttention"]`), then `encodeEvoformerPairBlock` (`:1663-1713`).
    Returns (msa, pair)."""
    row = w["msaRowAttention"]
    pb = dict(row["pairBias"], source="separate", activations=pair)
    msa = _add(msa, ops.attention_af2(msa, msa_mask, row["attention"], row["heads"], False, pb, eps))
    g = w["msaColumnGlobalAttention"]
    msa = _add(msa, ops.global_column_attention_af2(msa, msa_mask, g["attention"], g["heads"], eps))
    msa = _add(msa, ops.transition_af2(msa, w["msaTransition"], eps))
    return msa, _pair_steps(msa, pair, msa_mask, pair_mask, w, eps)


def evoformer_pair_block_af2(msa, pair, msa_mask, pair_mask, w, eps=1e-5):
    """The pair half of an Evoformer block (`encodeEvoformerPairBlock`,
    `webgpu/af2/evoformer/block.js:1663-1713`), a block of `ExtraMsaPairStackGpu`
    (`webgpu/af2/evoformer/stack.js:163-247`): the msa is read, not updated.  Returns the pair."""
    return _pair_steps(msa, pair, msa_mask, pair_mask, w, eps)


def _pair_steps(msa, pair, msa_mask, pair_mask, w, eps):
    """OPM, triangle multiplication out/in, triangle attention start/end, pair transition."""
    pair = _add(pair, ops.outer_product_mean_af2(msa, msa_mask, w["outerProductMean"], eps))
    pair = _add(pair, ops.tri_mult_af2(pair, pair_mask, w["triangleMultiplicationOutgoing"], "outgoing", eps))
    pair = _add(pair, ops.tri_mult_af2(pair, pair_mask, w["triangleMultiplicationIncoming"], "incoming", eps))
    st = w["triangleAttentionStarting"]
    pair = _add(pair, ops.attention_af2(pair, pair_mask, st["attention"], st["heads"], False,
                                        dict(st["pairBias"], source="normalized-input"), eps))
    en = w["triangleAttentionEnding"]
    pair = _add(pair, ops.attention_af2(pair, pair_mask, en["attention"], en["heads"], True,
                                        dict(en["pairBias"], source="normalized-input"), eps))
    return _add(pair, ops.transition_af2(pair, w["pairTransition"], eps))


def pairformer_block_af3(pair, single, pair_mask, seq_mask, w, swap_transposed_bias=False,
                         divide_by_length=False, eps=1e-5):
    """One AF3 pairformer block (`cpu/af3/trunk/pairformer.js:495-541`). Returns (pair, single)."""
    n = pair.shape[0]
    pair = _add(pair, ops.tri_mult_af3(pair, pair_mask, w["triangleMultiplicationOutgoing"], "outgoing",
                                       divide_by_length, eps))
    pair = _add(pair, ops.tri_mult_af3(pair, pair_mask, w["triangleMultiplicationIncoming"], "incoming",
                                       divide_by_length, eps))
    pair = _add(pair, ops.grid_self_attention_af3(pair, pair_mask, w["pairAttention1"], False,
                                                  swap_transposed_bias, eps))
    pair = _add(pair, ops.grid_self_attention_af3(pair, pair_mask, w["pairAttention2"], True,
                                                  swap_transposed_bias, eps))
    pair = _add(pair, ops.transition_af3(pair, w["pairTransition"], eps=eps))
    if single is None:
        return pair, None
    src = ops.layer_norm(pair, w["singlePairLogitsNormScale"], w["singlePairLogitsNormOffset"], eps,
                         fast_variance=True)
    heads = w["singleAttention"]["heads"]
    flat = ops.linear(src, w["singlePairLogitsProjection"])                     # [N, N, H]
    logits = np.asarray(flat, F64).transpose(2, 0, 1).astype(np.float32)
    single = _add(single, ops.single_attention_af3(single, logits, seq_mask, w["singleAttention"], eps))
    single = _add(single, ops.transition_af3(single, w["singleTransition"], eps=eps))
    assert logits.shape == (heads, n, n)
    return pair, single


def msa_block_af3(msa, pair, msa_mask, pair_mask, w, msa_update_before_opm, swap_transposed_bias=False,
                  divide_by_length=False, eps=1e-5):
    """One AF3 MSA-module block, `msaBlock` (`cpu/af3/trunk/msa.js:233-287`): the outer product
    mean into the pair and the MSA update (pair-weighted averaging, then the SwiGLU transition)
    in the dialect's order, then the pair steps of a pair-only pairformer block.
    Returns (msa, pair)."""
    def opm(m, p):
        return _add(p, ops.outer_product_mean_af3(m, msa_mask, w["outerProductMean"], eps))

    def update(m, p):
        m = _add(m, ops.msa_pair_weighted_averaging_af3(m, msa_mask, p, w["msaAttention1"], eps))
        return _add(m, ops.transition_af3(m, w["msaTransition"], eps=eps))

    if msa_update_before_opm:
        msa = update(msa, pair)
        pair = opm(msa, pair)
    else:
        pair = opm(msa, pair)
        msa = update(msa, pair)
    pair, _ = pairformer_block_af3(pair, None, pair_mask, None, w, swap_transposed_bias, divide_by_length, eps)
    return msa, pair
