"""Pins the AF3 oracle functions: the outer product mean, single attention, grid (triangle)
attention and the pairformer block order.

Each check is either a case with a hand-computed answer (the reference's own
`test/af3-msa.test.js:40-107` cases for the OPM), a per-element loop over the reference's
loop nest on tiny inputs (`cpu/af3/trunk/pairformer.js:322-485`), or a composition whose
order a mistake would change.
"""
import math

import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import blocks, ops

F64 = np.float64


# ---- AF3 outer product mean: the reference's hand-computed cases -------------------------
# test/af3-msa.test.js:21-37: a one-channel LayerNorm with scale 0 and offset 1 outputs
# exactly 1, so left = leftWeight and right = rightWeight for every covered token.

def _pinned_opm(left, right):
    return {"layerNormInputScale": np.array([0], np.float32),
            "layerNormInputOffset": np.array([1], np.float32),
            "leftProjection": np.array([[left]], np.float32),
            "rightProjection": np.array([[right]], np.float32),
            "outputW": np.array([[1]], np.float32), "outputB": np.array([0], np.float32)}


def test_opm_af3_sums_before_dividing():
    # test/af3-msa.test.js:40-52: each of 2 sequences adds 2*3, coverage 2 -> 12/(1e-3+2)
    out = ops.outer_product_mean_af3(np.zeros((2, 2, 1), np.float32), np.ones((2, 2), np.float32),
                                     _pinned_opm(2, 3))
    np.testing.assert_allclose(out[..., 0], np.full((2, 2), 12 / (1e-3 + 2)), atol=1e-4)


def test_opm_af3_divides_by_pair_coverage():
    # test/af3-msa.test.js:54-70: sequence 1 lacks token 1
    mask = np.array([[1, 1], [1, 0]], np.float32)
    out = ops.outer_product_mean_af3(np.zeros((2, 2, 1), np.float32), mask, _pinned_opm(2, 3))[..., 0]
    assert abs(out[0, 0] - 12 / (1e-3 + 2)) < 1e-4
    assert abs(out[1, 1] - 6 / (1e-3 + 1)) < 1e-4
    assert abs(out[0, 1] - 6 / (1e-3 + 1)) < 1e-4
    assert abs(out[1, 0] - 6 / (1e-3 + 1)) < 1e-4


def test_opm_af3_uncovered_pair_is_exactly_zero():
    # test/af3-msa.test.js:72-77
    out = ops.outer_product_mean_af3(np.zeros((1, 2, 1), np.float32), np.array([[1, 0]], np.float32),
                                     _pinned_opm(2, 3))
    assert out[1, 1, 0] == 0.0 and np.isfinite(out).all()


def test_opm_af3_is_not_symmetric():
    # test/af3-msa.test.js:79-106: one-hot tokens normalise to (+2,-1,-1)/sqrt2 and (-1,+2,-1)/sqrt2;
    # left takes channel 0 of token i, right channel 1 of token j
    w = {"layerNormInputScale": np.ones(3, np.float32), "layerNormInputOffset": np.zeros(3, np.float32),
         "leftProjection": np.array([[1], [0], [0]], np.float32),
         "rightProjection": np.array([[0], [1], [0]], np.float32),
         "outputW": np.array([[1]], np.float32), "outputB": np.array([0], np.float32)}
    msa = np.array([[[1, 0, 0], [0, 1, 0]]], np.float32)
    out = ops.outer_product_mean_af3(msa, np.ones((1, 2), np.float32), w)[..., 0]
    assert out[0, 1] != out[1, 0]
    assert abs(out[0, 1] - 2 / 1.001) < 1e-3
    assert abs(out[1, 0] - 0.5 / 1.001) < 1e-3


def test_opm_af3_channel_order_and_bias_before_divide():
    # Two outer channels: flat index a*c + b (left channel a, right channel b), and the output
    # bias is added before the /(1e-3 + count) (`cpu/af3/trunk/msa.js:130-150`).
    w = {"layerNormInputScale": np.zeros(1, np.float32), "layerNormInputOffset": np.ones(1, np.float32),
         "leftProjection": np.array([[2, 5]], np.float32), "rightProjection": np.array([[3, 7]], np.float32),
         "outputW": np.eye(4, dtype=np.float32), "outputB": np.array([1, 0, 0, 0], np.float32)}
    out = ops.outer_product_mean_af3(np.zeros((1, 1, 1), np.float32), np.ones((1, 1), np.float32), w)[0, 0]
    np.testing.assert_allclose(out, np.array([2 * 3 + 1, 2 * 7, 5 * 3, 5 * 7]) / 1.001, rtol=1e-6)


# ---- AF3 single attention -----------------------------------------------------------------

def _single_weights(c, heads, dim, seed):
    s = S.Stream(seed)
    hw = heads * dim
    return {"heads": heads, "dimension": dim,
            "layerNormScale": s.values(c, 0.2, 1), "layerNormOffset": s.values(c, 0.1),
            "qProjection": s.normal(c * hw, 0.5).reshape(c, hw), "qBias": s.values(hw, 0.3),
            "kProjection": s.normal(c * hw, 0.5).reshape(c, hw),
            "vProjection": s.normal(c * hw, 0.5).reshape(c, hw),
            "gatingQuery": s.normal(c * hw, 0.5).reshape(c, hw),
            "outputProjection": s.normal(hw * c, 0.5).reshape(hw, c)}


def _brute_single(single, logits_hij, seq_mask, w, eps=1e-5):
    """The loop nest of `singleAttention` (`cpu/af3/trunk/pairformer.js:446-485`), element by
    element, with its own fast-variance LayerNorm and dense layers."""
    n, c = single.shape
    heads, dim = w["heads"], w["dimension"]
    width = heads * dim
    xs = np.asarray(single, F64)
    norm = np.zeros((n, c))
    for t in range(n):
        mean = sum(xs[t]) / c
        var = sum(v * v for v in xs[t]) / c - mean * mean
        for ch in range(c):
            norm[t, ch] = (xs[t, ch] - mean) / math.sqrt(var + eps) * w["layerNormScale"][ch] + w["layerNormOffset"][ch]

    def dense(x, W, bias=None):
        out = np.zeros((x.shape[0], W.shape[1]))
        for r in range(x.shape[0]):
            for o in range(W.shape[1]):
                acc = 0.0 if bias is None else float(bias[o])
                for i in range(W.shape[0]):
                    acc += x[r, i] * float(W[i, o])
                out[r, o] = acc
        return out

    q = dense(norm, w["qProjection"], w["qBias"])
    k = dense(norm, w["kProjection"])
    v = dense(norm, w["vProjection"])
    gathered = np.zeros((n, width))
    for h in range(heads):
        for i in range(n):
            lg = []
            for j in range(n):
                dot = sum(q[i, h * dim + d] * k[j, h * dim + d] for d in range(dim))
                lg.append(dot / math.sqrt(dim) + float(logits_hij[h, i, j]) + 1e9 * (float(seq_mask[j]) - 1))
            top = max(lg)
            e = [math.exp(x - top) for x in lg]
            tot = sum(e)
            for d in range(dim):
                gathered[i, h * dim + d] = sum(e[j] / tot * v[j, h * dim + d] for j in range(n))
    gate = dense(norm, w["gatingQuery"])
    gathered = gathered / (1 + np.exp(-gate))
    return dense(gathered, w["outputProjection"])


def test_single_attention_brute_force():
    n, c, heads, dim = 5, 6, 2, 3
    w = _single_weights(c, heads, dim, 11)
    s = S.Stream(12)
    single = s.normal(n * c).reshape(n, c)
    logits = s.normal(heads * n * n).reshape(heads, n, n)
    mask = np.array([1, 1, 0, 1, 0], np.float32)
    out = ops.single_attention_af3(single, logits, mask, w)
    ref = _brute_single(single, logits, mask, w)
    np.testing.assert_allclose(out, ref, atol=2e-5, rtol=1e-5)


def _two_token_weights(dim, q_bias):
    """Tokens (1, 0) and (0, 1) normalise (scale 1, offset 0) to +-(1, -1); q, k and v read
    channel 0 into every head dimension, so q_i = (+-1 + q_bias), k_j = v_j = +-1 per dimension."""
    first = np.zeros((2, dim), np.float32)
    first[0, :] = 1
    return {"heads": 1, "dimension": dim, "layerNormScale": np.ones(2, np.float32),
            "layerNormOffset": np.zeros(2, np.float32),
            "qProjection": first, "qBias": np.full(dim, q_bias, np.float32),
            "kProjection": first, "vProjection": first[:, :1].repeat(dim, 1) / dim,
            "gatingQuery": np.zeros((2, dim), np.float32),
            "outputProjection": np.hstack([np.ones((dim, 1)), np.zeros((dim, 1))]).astype(np.float32)}


@pytest.mark.parametrize("dim,q_bias,extra", [(4, 0.0, 0.0), (4, 0.5, 0.0), (9, 0.0, 0.7)])
def test_single_attention_closed_form(dim, q_bias, extra):
    # token 0's logits over keys (+1, -1): dim*(1 + q_bias)*(+-1)/sqrt(dim) (+ a pair logit on key 1);
    # values +-1 (spread over dim lanes, summed back by the output row), gate sigmoid(0) = 1/2.
    single = np.array([[1, 0], [0, 1]], np.float32)
    w = _two_token_weights(dim, q_bias)
    logits = np.zeros((1, 2, 2), np.float32)
    logits[0, 0, 1] = extra
    out = ops.single_attention_af3(single, logits, np.ones(2, np.float32), w)
    s = dim * (1 + q_bias) / math.sqrt(dim) * (1 - 2e-5)     # LN's eps: 0.5/sqrt(0.25+1e-5) = 1 - 2e-5
    l0, l1 = s, -s + extra
    expect = 0.5 * (math.exp(l0) - math.exp(l1)) / (math.exp(l0) + math.exp(l1))
    assert abs(out[0, 0] - expect) < 1e-4, (out[0, 0], expect)
    assert abs(out[0, 1]) < 1e-7


def test_single_attention_masked_key_invisible():
    n, c, heads, dim = 6, 8, 2, 4
    w = _single_weights(c, heads, dim, 21)
    s = S.Stream(22)
    single = s.normal(n * c).reshape(n, c)
    logits = s.normal(heads * n * n).reshape(heads, n, n)
    mask = np.array([1, 0, 1, 1, 0, 1], np.float32)
    base = ops.single_attention_af3(single, logits, mask, w)
    # change the masked tokens' pair logits (as keys) arbitrarily: unmasked rows' outputs do not move
    moved = logits.copy()
    moved[:, :, [1, 4]] += 50.0
    np.testing.assert_allclose(ops.single_attention_af3(single, moved, mask, w), base, atol=1e-6)
    # a row-constant shift of the logits is a softmax no-op
    np.testing.assert_allclose(ops.single_attention_af3(single, logits + 3.0, mask, w), base, atol=1e-5)
    # only one unmasked key: every row attends to that token's value
    one = np.zeros(n, np.float32)
    one[3] = 1
    out = ops.single_attention_af3(single, logits, one, w)
    x = ops.layer_norm(single, w["layerNormScale"], w["layerNormOffset"], fast_variance=True).astype(F64)
    v = x @ w["vProjection"]
    g = 1 / (1 + np.exp(-(x @ w["gatingQuery"])))
    np.testing.assert_allclose(out, (v[3][None] * g) @ w["outputProjection"], atol=1e-5)


# ---- AF3 grid (triangle) self-attention ---------------------------------------------------

def _brute_grid(pair, mask, w, transpose, swap, eps=1e-5):
    """The loop nest of `gridSelfAttention` (`cpu/af3/trunk/pairformer.js:322-431`) element by
    element: bias from the untransposed normalised pair (swapped for the ending node in the
    openfold3 dialect), q/k/gate (out,in), v/output (in,out), key mask mask[row, j] or
    mask[j, row], update restored to the input orientation."""
    n, _, c = pair.shape
    heads, dim = w["heads"], w["dimension"]
    width = heads * dim
    x = np.asarray(pair, F64)
    norm = np.zeros_like(x)
    for i in range(n):
        for j in range(n):
            mean = x[i, j].sum() / c
            var = (x[i, j] ** 2).sum() / c - mean * mean
            norm[i, j] = (x[i, j] - mean) / math.sqrt(var + eps) * w["actNormScale"] + w["actNormOffset"]
    raw = norm @ np.asarray(w["pairBiasProjection"], F64)             # [i, j, h]
    act = np.zeros_like(norm)
    for i in range(n):
        for j in range(n):
            act[i, j] = norm[j, i] if transpose else norm[i, j]
    q = act @ np.asarray(w["qProjection"], F64).T
    k = act @ np.asarray(w["kProjection"], F64).T
    v = act @ np.asarray(w["vProjection"], F64)
    gate = act @ np.asarray(w["gatingQuery"], F64).T
    gathered = np.zeros((n, n, width))
    for row in range(n):
        for h in range(heads):
            for i in range(n):
                lg = []
                for j in range(n):
                    dot = sum(q[row, i, h * dim + d] * k[row, j, h * dim + d] for d in range(dim))
                    b = raw[j, i, h] if (transpose and swap) else raw[i, j, h]
                    m = mask[j, row] if transpose else mask[row, j]
                    lg.append(dot / math.sqrt(dim) + b + (0.0 if m > 0 else -1e9))
                top = max(lg)
                e = [math.exp(t - top) for t in lg]
                tot = sum(e)
                for d in range(dim):
                    gathered[row, i, h * dim + d] = sum(e[j] / tot * v[row, j, h * dim + d] for j in range(n))
    out = (gathered / (1 + np.exp(-gate))) @ np.asarray(w["outputProjection"], F64)
    if transpose:
        out = out.transpose(1, 0, 2)
    return out


@pytest.mark.parametrize("transpose,swap", [(False, False), (True, False), (True, True)])
def test_grid_attention_brute_force(transpose, swap):
    n, c = 4, 8
    w = S.synthetic_pairformer_weights(c, 8, 2, 2, 4, seed=17)["pairAttention1"]
    s = S.Stream(18)
    pair = s.normal(n * n * c).reshape(n, n, c)
    mask = np.ones((n, n), np.float32)
    mask[1, 3] = mask[2, 0] = mask[3, 3] = 0      # asymmetric, so the transposed read matters
    out = ops.grid_self_attention_af3(pair, mask, w, transpose, swap_transposed_bias=swap)
    ref = _brute_grid(pair, mask, w, transpose, swap)
    np.testing.assert_allclose(out, ref, atol=2e-5, rtol=1e-5)


def test_grid_attention_scale_closed_form():
    # One head of width dim; every channel normalises to +-1 for tokens (1, 0) / (0, 1) along
    # the row; q and k read channel 0 in every dimension, v channel 0 once.  Row 0, query 0
    # sees logits (+dim, -dim)/sqrt(dim) over its two keys: out = tanh(sqrt(dim)) / 2.
    dim, n, c = 9, 2, 2
    w = {"heads": 1, "dimension": dim, "actNormScale": np.ones(c, np.float32),
         "actNormOffset": np.zeros(c, np.float32), "pairBiasProjection": np.zeros((c, 1), np.float32)}
    sel = np.zeros((dim, c), np.float32)
    sel[:, 0] = 1
    w["qProjection"] = sel
    w["kProjection"] = sel
    vsel = np.zeros((c, dim), np.float32)
    vsel[0, 0] = 1
    w["vProjection"] = vsel
    w["gatingQuery"] = np.zeros((dim, c), np.float32)
    outp = np.zeros((dim, c), np.float32)
    outp[0, 0] = 1
    w["outputProjection"] = outp
    pair = np.array([[[1, 0], [0, 1]], [[1, 0], [0, 1]]], np.float32)
    out = ops.grid_self_attention_af3(pair, np.ones((n, n), np.float32), w, False)
    s = math.sqrt(dim) * (1 - 2e-5) ** 2
    assert abs(out[0, 0, 0] - 0.5 * math.tanh(s)) < 1e-4, out[0, 0, 0]
    # mask key 1 of row 0: query 0 takes key 0's value exactly (+1, times gate 1/2)
    m = np.ones((n, n), np.float32)
    m[0, 1] = 0
    out = ops.grid_self_attention_af3(pair, m, w, False)
    assert abs(out[0, 0, 0] - 0.5 * (1 - 2e-5)) < 1e-6 and abs(out[0, 1, 0] - 0.5 * (1 - 2e-5)) < 1e-6


# ---- pairformer block order ---------------------------------------------------------------

def test_pairformer_single_track_reads_final_pair():
    # `cpu/af3/trunk/pairformer.js:515-537`: the single track's pair logits come from the pair
    # AFTER the triangle updates, both attentions and the pair transition.
    n, cz, cs = 5, 8, 12
    w = S.synthetic_pairformer_weights(cz, cs, 2, 2, 4, seed=31)
    s = S.Stream(32)
    pair = s.normal(n * n * cz).reshape(n, n, cz)
    single = s.normal(n * cs).reshape(n, cs)
    pm = np.ones((n, n), np.float32)
    sm = np.array([1, 1, 1, 1, 0], np.float32)
    p_out, s_out = blocks.pairformer_block_af3(pair, single, pm, sm, w)

    def add(x, d):
        return (np.asarray(x, F64) + np.asarray(d, F64)).astype(np.float32)

    p = pair
    p = add(p, ops.tri_mult_af3(p, pm, w["triangleMultiplicationOutgoing"], "outgoing"))
    p = add(p, ops.tri_mult_af3(p, pm, w["triangleMultiplicationIncoming"], "incoming"))
    p = add(p, ops.grid_self_attention_af3(p, pm, w["pairAttention1"], False))
    p = add(p, ops.grid_self_attention_af3(p, pm, w["pairAttention2"], True))
    before_transition = p
    p = add(p, ops.transition_af3(p, w["pairTransition"]))
    np.testing.assert_array_equal(p_out, p)

    def single_from(src_pair):
        src = ops.layer_norm(src_pair, w["singlePairLogitsNormScale"], w["singlePairLogitsNormOffset"],
                             fast_variance=True)
        lg = np.asarray(ops.linear(src, w["singlePairLogitsProjection"]), F64).transpose(2, 0, 1)
        x = add(single, ops.single_attention_af3(single, lg.astype(np.float32), sm, w["singleAttention"]))
        return add(x, ops.transition_af3(x, w["singleTransition"]))

    np.testing.assert_allclose(s_out, single_from(p), atol=1e-6)
    # reading the pair one step early gives a measurably different single track
    assert np.abs(single_from(before_transition) - s_out).max() > 1e-3
