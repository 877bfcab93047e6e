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
    pair = _add(pair, ops.outer_product_mean_af2(msa, msa_mask, w["outerProductMean"], eps))
    pair = _add(pair, ops.tri_mult_af2(pair, pair_mask, w["triangleMultiplicationOutgoing"], "outgoing", eps))
    pair = _add(pair, ops.tri_mult_af2(pair, pair_mask, w["triangleMultiplicationIncoming"], "incoming", eps))
    st = w["triangleAttentionStarting"]
    pair = _add(pair, ops.attention_af2(pair, pair_mask, st["attention"], st["heads"], False,
                                        dict(st["pairBias"], source="normalized-input"), eps))
    en = w["triangleAttentionEnding"]
    pair = _add(pair, ops.attention_af2(pair, pair_mask, en["attention"], en["heads"], True,
                                        dict(en["pairBias"], source="normalized-input"), eps))
    pair = _add(pair, ops.transition_af2(pair, w["pairTransition"], eps))
    return msa, pair


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


def synthetic_pairformer_weights(c_z, c_s, heads_pair, heads_single, dim_single, seed=3, factor=4):
    """Random-init AF3 pairformer block weights (N(0, 1/fan_in) masters, LN scale ~1).

    The reference has no AF3 synthetic generator; this uses the same `generator(seed)`
    stream with Box-Muller normals (oracle.prng.Stream.normal).
    """
    from .prng import Stream
    s = Stream(seed)

    def lin(i, o):
        return s.normal(i * o, 1.0 / np.sqrt(i)).reshape(i, o)

    def ln(c):
        return s.values(c, 0.2, 1), s.values(c, 0.1)

    def tri():
        sc, of = ln(c_z)
        cs, co = ln(c_z)
        return {"leftNormInputScale": sc, "leftNormInputOffset": of,
                "projection": lin(c_z, 2 * c_z), "gate": lin(c_z, 2 * c_z),
                "centerNormScale": cs, "centerNormOffset": co,
                "outputProjection": lin(c_z, c_z), "gatingLinear": lin(c_z, c_z)}

    def grid(heads, dim):
        sc, of = ln(c_z)
        w = heads * dim
        return {"heads": heads, "dimension": dim, "actNormScale": sc, "actNormOffset": of,
                "pairBiasProjection": lin(c_z, heads),
                "qProjection": lin(c_z, w).T.copy(), "kProjection": lin(c_z, w).T.copy(),
                "vProjection": lin(c_z, w), "gatingQuery": lin(c_z, w).T.copy(),
                "outputProjection": lin(w, c_z)}

    def trans(c):
        sc, of = ln(c)
        return {"inputLayerNormScale": sc, "inputLayerNormOffset": of,
                "transition1": lin(c, 2 * factor * c), "transition2": lin(factor * c, c)}

    w = {"triangleMultiplicationOutgoing": tri(), "triangleMultiplicationIncoming": tri(),
         "pairAttention1": grid(heads_pair, c_z // heads_pair),
         "pairAttention2": grid(heads_pair, c_z // heads_pair),
         "pairTransition": trans(c_z)}
    sc, of = ln(c_z)
    w["singlePairLogitsNormScale"], w["singlePairLogitsNormOffset"] = sc, of
    w["singlePairLogitsProjection"] = lin(c_z, heads_single)
    sc, of = ln(c_s)
    hw = heads_single * dim_single
    w["singleAttention"] = {"heads": heads_single, "dimension": dim_single,
                            "layerNormScale": sc, "layerNormOffset": of,
                            "qProjection": lin(c_s, hw), "qBias": s.values(hw, 0.1),
                            "kProjection": lin(c_s, hw), "vProjection": lin(c_s, hw),
                            "gatingQuery": lin(c_s, hw), "outputProjection": lin(hw, c_s)}
    w["singleTransition"] = trans(c_s)
    return w
