"""Pins the oracle: the reference's fixtures and tests, closed forms and brute force."""
import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import codec, ops, prng
from tests import helpers as H


# ---- triangle multiplication ------------------------------------------------------------

def test_openfold_fixture():
    # test/cpu-reference.test.js:18-27: mean < 1e-7, max < 1e-6
    f = H.load_fixture("openfold_triangle_small")
    assert f["meta"]["source"].startswith("OpenFold")
    m = H.metrics(ops.tri_mult_af2(f["z"], f["mask"], f["weights"], "outgoing", f["meta"]["epsilon"]), f["expected"])
    assert m["meanAbsoluteError"] < 1e-7 and m["maxAbsoluteError"] < 1e-6, m


@pytest.mark.parametrize("name", H.FIXTURES[1:])
def test_alphafold_fixtures(name):
    # test/triangle-multiplication-outgoing.gpu.test.js:41-48: mean < 1e-5, max < 1e-4
    f = H.load_fixture(name)
    m = H.metrics(ops.tri_mult_af2(f["z"], f["mask"], f["weights"], "outgoing", f["meta"]["epsilon"]), f["expected"])
    assert m["meanAbsoluteError"] < 1e-5 and m["maxAbsoluteError"] < 1e-4, m


def _brute_tri(z, mask, w, direction, eps=1e-5):
    """Element loops straight from the einsums 'ikc,jkc->ijc' / 'kjc,kic->ijc' on tiny inputs."""
    n = z.shape[0]
    zn = ops.layer_norm(z, w["layerNormInWeight"], w["layerNormInBias"], eps).astype(np.float64)
    sig = lambda x: 1 / (1 + np.exp(-x))
    lin = lambda x, W, b: x @ W.astype(np.float64).T + b
    a = lin(zn, w["linearAPWeight"], w["linearAPBias"]) * sig(lin(zn, w["linearAGWeight"], w["linearAGBias"])) * mask[..., None]
    b = lin(zn, w["linearBPWeight"], w["linearBPBias"]) * sig(lin(zn, w["linearBGWeight"], w["linearBGBias"])) * mask[..., None]
    x = np.zeros_like(a)
    for i in range(n):
        for j in range(n):
            for k in range(n):
                x[i, j] += a[i, k] * b[j, k] if direction == "outgoing" else a[k, j] * b[k, i]
    xn = ops.layer_norm(x, w["layerNormOutWeight"], w["layerNormOutBias"], eps)
    return lin(xn, w["linearZWeight"], w["linearZBias"]) * sig(lin(zn, w["linearGWeight"], w["linearGBias"]))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tri_brute_force(direction):
    inp = S.deterministic_triangle_input(5, 6, 4, 13)
    ref = _brute_tri(inp["z"], inp["mask"], inp["weights"], direction)
    out = ops.tri_mult_af2(inp["z"], inp["mask"], inp["weights"], direction)
    assert np.abs(out - ref).max() < 1e-5


@pytest.mark.parametrize("name", H.FIXTURES)
def test_incoming_is_transposed_outgoing(name):
    # incoming(z, mask) == transpose(outgoing(transpose(z), transpose(mask)))
    f = H.load_fixture(name)
    zt = f["z"].transpose(1, 0, 2).copy()
    inc = ops.tri_mult_af2(f["z"], f["mask"], f["weights"], "incoming")
    out_t = ops.tri_mult_af2(zt, f["mask"].T.copy(), f["weights"], "outgoing").transpose(1, 0, 2)
    assert np.abs(inc - out_t).max() < 1e-4 * max(1.0, np.abs(inc).max())


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_af3_reduces_to_af2(direction):
    # AF3 = AF2 with interleaved a/b columns, zero biases and fast variance.  With inputs whose
    # rows have zero mean the two variance formulas agree; compare on the AF2 restatement.
    c, n = 8, 6
    w3 = H.af3_tri_weights(c, 5)
    s = S.Stream(4)
    z = s.normal(n * n * c).reshape(n, n, c)
    mask = (s.uniform(n * n) > 0.2).astype(np.float32).reshape(n, n)
    w2 = {"layerNormInWeight": w3["leftNormInputScale"], "layerNormInBias": w3["leftNormInputOffset"],
          "linearAPWeight": w3["projection"][:, 0::2].T, "linearBPWeight": w3["projection"][:, 1::2].T,
          "linearAGWeight": w3["gate"][:, 0::2].T, "linearBGWeight": w3["gate"][:, 1::2].T,
          "layerNormOutWeight": w3["centerNormScale"], "layerNormOutBias": w3["centerNormOffset"],
          "linearZWeight": w3["outputProjection"].T, "linearGWeight": w3["gatingLinear"].T}
    for k in ["linearAPBias", "linearBPBias", "linearAGBias", "linearBGBias"]:
        w2[k] = np.zeros(c, np.float32)
    w2["linearZBias"] = np.zeros(c, np.float32)
    w2["linearGBias"] = np.zeros(c, np.float32)
    a3 = ops.tri_mult_af3(z, mask, w3, direction)
    a2 = ops.tri_mult_af2(z, mask, w2, direction)
    assert np.abs(a3 - a2).max() < 1e-4


def test_layer_norm_closed_forms():
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    y = ops.layer_norm(x, np.ones(4), np.zeros(4), eps=0.0)
    np.testing.assert_allclose(y, (x - 2.5) / np.sqrt(1.25), rtol=1e-6)
    y2 = ops.layer_norm(np.vstack([x, 10 * x]), np.ones(4), np.zeros(4))
    np.testing.assert_allclose(y2[0], y[0], atol=1e-4)          # rows independent
    yf = ops.layer_norm(x, np.ones(4), np.zeros(4), eps=0.0, fast_variance=True)
    np.testing.assert_allclose(yf, y, atol=1e-6)


def test_linear_transposed_weights():
    rng = np.random.default_rng(0)
    x, w = rng.normal(size=(3, 5)).astype(np.float32), rng.normal(size=(5, 7)).astype(np.float32)
    np.testing.assert_array_equal(ops.linear(x, w), ops.linear(x, w.T.copy(), transposed=True))


# ---- transitions --------------------------------------------------------------------------

def test_swiglu_blocked_split_and_swish():
    # test/af3-pairformer.test.js: swish(1)*3 through a transition whose gate half is the first half
    c = 2
    w = {"inputLayerNormScale": np.zeros(c, np.float32), "inputLayerNormOffset": np.ones(c, np.float32),
         "transition1": np.zeros((c, 2 * c), np.float32), "transition2": np.zeros((c, c), np.float32)}
    w["transition1"][0, 0] = 1.0      # gate channel 0 <- LN input 1
    w["transition1"][1, c] = 3.0      # value channel 0 <- 3 * LN input 1 (LN output is the offset: 1)
    w["transition2"][0, 0] = 1.0
    out = ops.transition_af3(np.array([[0.3, -0.7]], np.float32), w, factor=1)
    sw = 1.0 / (1.0 + np.exp(-1.0))
    # LN output is the offset (1, 1): gate = 1*1 + 0 = 1, value = 3*1 = 3 -> swish(1) * 3
    np.testing.assert_allclose(out[0, 0], sw * 3.0, rtol=1e-6)
    assert out[0, 1] == 0


def test_relu_transition_closed_form():
    c, h = 2, 3
    w = {"layerNormScale": np.zeros(c, np.float32), "layerNormOffset": np.array([1.0, -1.0], np.float32),
         "firstWeight": np.array([[1, -1, 2], [0, 0, 0]], np.float32), "firstBias": np.array([0, 0, -5], np.float32),
         "secondWeight": np.ones((h, c), np.float32), "secondBias": np.array([0.5, 0], np.float32)}
    out = ops.transition_af2(np.array([[3.0, 4.0]], np.float32), w)
    # hidden = relu([1, -1, 2 - 5]) = [1, 0, 0] -> out = [1 + 0.5, 1]
    np.testing.assert_allclose(out[0], [1.5, 1.0])


# ---- attention ----------------------------------------------------------------------------

def _attn_weights(c, heads, seed, pair_c=None):
    s = S.Stream(seed)
    r = 1 / np.sqrt(c)
    w = {"queryNormScale": s.values(c, 0.2, 1), "queryNormOffset": s.values(c, 0.1),
         "queryWeight": s.values(c * c, r).reshape(c, c), "keyWeight": s.values(c * c, r).reshape(c, c),
         "valueWeight": s.values(c * c, r).reshape(c, c), "gatingWeight": s.values(c * c, r).reshape(c, c),
         "gatingBias": s.values(c, 0.1, 1), "outputWeight": s.values(c * c, r).reshape(c, c),
         "outputBias": s.values(c, 0.05)}
    return w


def _brute_attention(act, mask, w, heads, transpose, bias):
    """Per-element loops of the WGSL flash semantics (attention.js:877-940)."""
    a = act.transpose(1, 0, 2) if transpose else act
    mk = mask.T if transpose else mask
    B, Q, Cc = a.shape
    d = Cc // heads
    x = ops.layer_norm(a, w["queryNormScale"], w["queryNormOffset"]).astype(np.float64)
    q = x @ w["queryWeight"] / np.sqrt(d)
    k = x @ w["keyWeight"]
    v = x @ w["valueWeight"]
    g = 1 / (1 + np.exp(-(x @ w["gatingWeight"] + w["gatingBias"])))
    o = np.zeros((B, Q, Cc))
    for b in range(B):
        for h in range(heads):
            sl = slice(h * d, (h + 1) * d)
            for i in range(Q):
                logits = []
                for j in range(Q):
                    l = float(q[b, i, sl] @ k[b, j, sl]) + 1e9 * (mk[b, j] - 1)
                    if bias is not None:
                        l += bias[h, i, j]
                    logits.append(min(max(l, -1e8), 1e8))
                logits = np.array(logits)
                p = np.exp(logits - logits.max())
                p /= p.sum()
                o[b, i, sl] = (p[:, None] * v[b, :, sl]).sum(0)
    o = o * g
    upd = o @ w["outputWeight"] + w["outputBias"]
    return upd.transpose(1, 0, 2) if transpose else upd


@pytest.mark.parametrize("transpose", [False, True])
def test_attention_brute_force(transpose):
    s = S.Stream(3)
    B, Q, c, heads = 3, 5, 8, 2
    act = s.values(B * Q * c, 1.5).reshape((Q, B, c) if transpose else (B, Q, c))
    mask = np.ones((Q, B) if transpose else (B, Q), np.float32)
    mask.flat[3] = 0
    w = _attn_weights(c, heads, 9)
    ref = _brute_attention(act, mask, w, heads, transpose, None)
    out = ops.attention_af2(act, mask, w, heads, transpose)
    assert np.abs(out - ref).max() < 1e-5


def test_attention_pair_bias_separate_brute_force():
    s = S.Stream(5)
    B, Q, c, heads, cz = 2, 4, 8, 2, 6
    act = s.values(B * Q * c, 1.5).reshape(B, Q, c)
    pair = s.values(Q * Q * cz, 1.5).reshape(Q, Q, cz)
    mask = np.ones((B, Q), np.float32)
    w = _attn_weights(c, heads, 2)
    pb = {"source": "separate", "activations": pair, "layerNormScale": s.values(cz, 0.2, 1),
          "layerNormOffset": s.values(cz, 0.1), "projectionWeight": s.values(cz * heads, 0.5).reshape(cz, heads)}
    bias = (ops.layer_norm(pair, pb["layerNormScale"], pb["layerNormOffset"]).astype(np.float64)
            @ pb["projectionWeight"]).transpose(2, 0, 1)
    ref = _brute_attention(act, mask, w, heads, False, bias)
    out = ops.attention_af2(act, mask, w, heads, False, pb)
    assert np.abs(out - ref).max() < 1e-5


def test_attention_single_unmasked_key_selects_value():
    s = S.Stream(8)
    B, Q, c, heads = 1, 6, 4, 1
    act = s.values(B * Q * c, 1.0).reshape(B, Q, c)
    mask = np.zeros((B, Q), np.float32)
    mask[0, 2] = 1
    w = _attn_weights(c, heads, 4)
    x = ops.layer_norm(act, w["queryNormScale"], w["queryNormOffset"]).astype(np.float64)
    v = x @ w["valueWeight"]
    g = 1 / (1 + np.exp(-(x @ w["gatingWeight"] + w["gatingBias"])))
    expect = (v[0, 2][None, :] * g[0]) @ w["outputWeight"] + w["outputBias"]
    out = ops.attention_af2(act, mask, w, heads)
    np.testing.assert_allclose(out[0], expect, atol=1e-5)


def test_grid_attention_transpose_identity():
    # ending-node attention == starting-node attention on the transposed pair (stock AF3 with the
    # bias NOT swapped is the only case where this needs the bias transposed: use swap=True)
    from localfold_amd.synthetic import synthetic_pairformer_weights
    n, c = 6, 16
    w = synthetic_pairformer_weights(c, 8, 2, 2, 4)["pairAttention1"]
    s = S.Stream(2)
    pair = s.normal(n * n * c).reshape(n, n, c)
    mask = (s.uniform(n * n) > 0.2).astype(np.float32).reshape(n, n)
    end = ops.grid_self_attention_af3(pair, mask, w, True, swap_transposed_bias=True)
    start_t = ops.grid_self_attention_af3(pair.transpose(1, 0, 2).copy(), mask.T.copy(), w, False)
    np.testing.assert_allclose(end, start_t.transpose(1, 0, 2), atol=1e-5)


# ---- outer product mean -------------------------------------------------------------------

def test_opm_single_sequence_closed_form():
    s = S.Stream(6)
    n, cm, co, cz = 4, 8, 3, 5
    msa = s.values(n * cm, 1.0).reshape(1, n, cm)
    mask = np.array([[1, 1, 0, 1]], np.float32)
    w = {"layerNormScale": s.values(cm, 0.2, 1), "layerNormOffset": s.values(cm, 0.1),
         "leftWeight": s.values(cm * co, 0.4).reshape(cm, co), "leftBias": s.values(co, 0.1),
         "rightWeight": s.values(cm * co, 0.4).reshape(cm, co), "rightBias": s.values(co, 0.1),
         "outputWeight": s.values(co * co * cz, 0.3).reshape(co * co, cz), "outputBias": s.values(cz, 0.05)}
    x = ops.layer_norm(msa[0], w["layerNormScale"], w["layerNormOffset"]).astype(np.float64)
    l = (x @ w["leftWeight"] + w["leftBias"]) * mask[0][:, None]
    r = (x @ w["rightWeight"] + w["rightBias"]) * mask[0][:, None]
    out = ops.outer_product_mean_af2(msa, mask, w)
    for i in range(n):
        for j in range(n):
            o = np.outer(l[i], r[j]).reshape(-1) @ w["outputWeight"] + w["outputBias"]
            np.testing.assert_allclose(out[i, j], o / (1e-3 + mask[0, i] * mask[0, j]), rtol=1e-5, atol=1e-5)


def _opm_weights(s, cm, co, cz):
    return {"layerNormScale": s.values(cm, 0.2, 1), "layerNormOffset": s.values(cm, 0.1),
            "leftWeight": s.values(cm * co, 0.4).reshape(cm, co), "leftBias": s.values(co, 0.1),
            "rightWeight": s.values(cm * co, 0.4).reshape(cm, co), "rightBias": s.values(co, 0.1),
            "outputWeight": s.values(co * co * cz, 0.3).reshape(co * co, cz), "outputBias": s.values(cz, 0.05)}


def test_opm_count_identity():
    """S = 5 with ragged masks.  With the LN scale 0, every normalised row is the offset
    beta, so l_si = m_si L and r_sj = m_sj R for fixed vectors L = beta Wl + bl and
    R = beta Wr + br; the sum over sequences is then count_ij (L outer R), with
    count_ij = sum_s m_si m_sj, and the update is ((count_ij vec(L outer R)) W + b) /
    (1e-3 + count_ij) (outer-product-mean.js:702-742: bias, then the divide).  This fixes
    the coverage denominator (not the sequence count, not the product of per-token counts),
    the a*c + b flattening (L != R) and the bias-before-divide order."""
    s = S.Stream(16)
    n, cm, co, cz, seqs = 5, 8, 3, 4, 5
    w = _opm_weights(s, cm, co, cz)
    w["layerNormScale"] = np.zeros(cm, np.float32)
    msa = s.values(seqs * n * cm, 1.0).reshape(seqs, n, cm)
    mask = np.array([[1, 1, 1, 1, 1], [1, 0, 1, 1, 0], [0, 1, 1, 0, 0], [1, 1, 0, 1, 0], [1, 0, 1, 1, 0]],
                    np.float32)
    beta = np.asarray(w["layerNormOffset"], np.float64)
    L = beta @ w["leftWeight"] + w["leftBias"]
    R = beta @ w["rightWeight"] + w["rightBias"]
    out = ops.outer_product_mean_af2(msa, mask, w)
    for i in range(n):
        for j in range(n):
            count = sum(mask[t, i] * mask[t, j] for t in range(seqs))
            o = (count * np.outer(L, R).reshape(-1)) @ w["outputWeight"] + w["outputBias"]
            np.testing.assert_allclose(out[i, j], o / (1e-3 + count), rtol=1e-5, atol=1e-6)
    # the pairs (0, 4), (4, 4) ... are covered by one sequence, (1, 2) by two, (0, 0) by four
    assert {float(sum(mask[:, i] * mask[:, j])) for i in range(n) for j in range(n)} >= {1.0, 2.0, 4.0}


def test_opm_per_element_loop_several_sequences():
    """S = 4, ragged masks, general LN: the oracle against an element-by-element loop over
    sequences, channel pairs (a, b) and outputs."""
    s = S.Stream(17)
    n, cm, co, cz, seqs = 4, 6, 3, 5, 4
    w = _opm_weights(s, cm, co, cz)
    msa = s.values(seqs * n * cm, 1.0).reshape(seqs, n, cm)
    mask = np.array([[1, 1, 0, 1], [0, 1, 1, 1], [1, 1, 1, 0], [1, 0, 1, 1]], np.float32)
    x = ops.layer_norm(msa, w["layerNormScale"], w["layerNormOffset"]).astype(np.float64)
    out = ops.outer_product_mean_af2(msa, mask, w)
    for i in range(n):
        for j in range(n):
            acc = np.zeros(co * co)
            count = 0.0
            for t in range(seqs):
                count += mask[t, i] * mask[t, j]
                for a in range(co):
                    la = mask[t, i] * (sum(x[t, i, k] * w["leftWeight"][k, a] for k in range(cm)) + w["leftBias"][a])
                    for b in range(co):
                        rb = mask[t, j] * (sum(x[t, j, k] * w["rightWeight"][k, b] for k in range(cm))
                                           + w["rightBias"][b])
                        acc[a * co + b] += la * rb
            for z in range(cz):
                v = w["outputBias"][z] + sum(acc[q] * w["outputWeight"][q, z] for q in range(co * co))
                np.testing.assert_allclose(out[i, j, z], v / (1e-3 + count), rtol=1e-5, atol=1e-6)


# ---- codecs -------------------------------------------------------------------------------

def _int5_record(codes_by_group, scales, zeros):
    codes = np.array(codes_by_group, np.uint8)
    return {"dtype": "int5", "shape": [codes.size], "data": S.pack_bits(codes, 5),
            "scales": np.array(scales, np.float16), "zeros": np.array(zeros, np.float16), "block": 32}


def test_int5_every_code_position():
    # test/int5-tensor.test.js: codes 0..31 in one group decode to themselves
    out = codec.decode(_int5_record([list(range(32))], [1], [0]))
    np.testing.assert_array_equal(out, np.arange(32))


def test_int5_groups_independent():
    out = codec.decode(_int5_record([[31] * 32, [0] * 32], [1, 1], [0, 0]))
    assert (out[:32] == 31).all() and (out[32:] == 0).all()


def test_int5_scale_and_zero():
    out = codec.decode(_int5_record([[0] * 32, [31] * 32], [0.5, 2], [-4, 10]))
    assert out[0] == -4 and out[32] == 31 * 2 + 10


def test_int5_group_is_20_bytes():
    assert S.pack_bits(np.zeros((3, 32), np.uint8), 5).size == 3 * 20 + 1


@pytest.mark.parametrize("dtype,tol", [("int8", 0.01), ("int5", 0.05)])
def test_quantise_round_trip(dtype, tol):
    rng = np.random.default_rng(1)
    w = rng.normal(size=(64, 96)).astype(np.float32)
    for rec in (S.make_record(w, dtype), S.make_record(w, dtype, channel_axis=1)):
        dec = codec.decode(rec)
        rel = np.abs(dec - w).max() / np.abs(w).max()
        assert rel < tol, rel


def test_int8_decode_is_code_times_scale():
    rec = {"dtype": "int8", "shape": [128], "data": np.arange(-64, 64).astype(np.int8),
           "scales": np.array([0.5, 0.25], np.float16), "block": 64}
    out = codec.decode(rec)
    np.testing.assert_array_equal(out[:64], np.arange(-64, 0) * 0.5)
    np.testing.assert_array_equal(out[64:], np.arange(0, 64) * 0.25)


# ---- generator ----------------------------------------------------------------------------

@pytest.mark.parametrize("seed", [0, 7, 1000 + 384, 0xFFFFFFFF])
def test_generator_counter_form(seed):
    np.testing.assert_array_equal(S.uniform_stream(seed, 257), prng.uniform_sequential(seed, 257))


def test_error_metrics_exact():
    # test/cpu-reference.test.js:35-41
    m = ops.error_metrics(np.array([1, 3], np.float32), np.array([2, 1], np.float32))
    assert m["meanAbsoluteError"] == 1.5 and m["maxAbsoluteError"] == 2
    assert m["rootMeanSquareError"] == np.sqrt(2.5)
