"""AF3 MSA module: pair-weighted averaging (`msaAttention`, cpu/af3/trunk/msa.js:157-219) and
the MSA-module block (`msaBlock`, :233-287).

CPU: the oracle against what the reference's semantics fix (one token, uniform logits, the
key mask as the maximum over the sequences, a token no sequence covers is the same as a
deleted token, sequences do not mix, both block orderings move both outputs as
test/opendde-branches.test.js:135-230 asserts, and equal ones when the outer product's output
is zero).  GPU: the C ABI against the oracle."""
import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import blocks, ops
from tests import helpers as H


def _avg_inputs(s, n, cm, cz, heads, dim, seed):
    w = S.synthetic_msa_module_weights(c_m=cm, c_z=cz, heads=heads, dim=dim, heads_pair=2, c_outer=8,
                                       seed=seed)["msaAttention1"]
    st = S.Stream(seed + 7)
    msa = st.normal(s * n * cm).reshape(s, n, cm).astype(np.float32)
    pair = st.normal(n * n * cz).reshape(n, n, cz).astype(np.float32)
    mask = np.ones((s, n), np.float32)
    return w, msa, pair, mask


def _values_gate(msa, w):
    x = np.asarray(ops.layer_norm(msa, w["actNormScale"], w["actNormOffset"], 1e-5, fast_variance=True), np.float64)
    return x @ w["vProjection"], ops.sigmoid(x @ w["gatingQuery"])


def test_oracle_single_token_closed_form():
    """One token: every softmax is 1, the update is (v * sigmoid(g)) Wo whatever the pair."""
    w, msa, pair, mask = _avg_inputs(4, 1, 32, 16, 4, 8, 1)
    got = ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    v, g = _values_gate(msa, w)
    np.testing.assert_allclose(got, (v * g) @ w["outputProjection"], rtol=2e-5, atol=2e-5)
    got2 = ops.msa_pair_weighted_averaging_af3(msa, mask, pair * 3 + 1, w)
    np.testing.assert_allclose(got2, got, rtol=1e-6, atol=1e-6)


def test_oracle_zero_logits_average_the_covered_tokens():
    """pairLogits = 0: each head averages the values of the tokens some sequence covers,
    uniformly; a token masked in only some sequences still counts (maximum over sequences)."""
    w, msa, pair, mask = _avg_inputs(3, 6, 32, 16, 4, 8, 2)
    w = dict(w, pairLogits=np.zeros_like(w["pairLogits"]))
    mask[:, 4] = 0          # no sequence covers token 4
    mask[0, 1] = 0          # token 1 is covered by sequences 1 and 2
    got = ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    v, g = _values_gate(msa, w)
    keep = [0, 1, 2, 3, 5]
    mean = v[:, keep].mean(1, keepdims=True)                      # [S, 1, H*d]
    np.testing.assert_allclose(got, (mean * g) @ w["outputProjection"], rtol=2e-5, atol=2e-5)


def test_oracle_uncovered_token_equals_deleted_token():
    """A token no sequence covers is out of every softmax: the other tokens' updates equal
    those of the problem with that token's msa column and pair row and column deleted."""
    w, msa, pair, mask = _avg_inputs(3, 7, 32, 16, 4, 8, 3)
    mask[:, 2] = 0
    mask[1, 5] = 0
    got = ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    keep = [0, 1, 3, 4, 5, 6]
    ref = ops.msa_pair_weighted_averaging_af3(msa[:, keep], mask[:, keep], pair[keep][:, keep], w)
    np.testing.assert_allclose(got[:, keep], ref, rtol=2e-5, atol=2e-5)


def test_oracle_every_key_masked_is_uniform():
    """No token covered: the f32 logits are all -1e9 and each head averages every token."""
    w, msa, pair, mask = _avg_inputs(2, 5, 32, 16, 4, 8, 5)
    mask[:] = 0
    got = ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    v, g = _values_gate(msa, w)
    np.testing.assert_allclose(got, (v.mean(1, keepdims=True) * g) @ w["outputProjection"], rtol=2e-5, atol=2e-5)


def test_oracle_sequences_do_not_mix():
    """The weights come from the pair alone: a sequence's update depends on its own row only,
    so permuting sequences permutes updates and changing one row leaves the others."""
    w, msa, pair, mask = _avg_inputs(5, 6, 32, 16, 4, 8, 4)
    a = ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    perm = np.array([2, 4, 0, 1, 3])
    b = ops.msa_pair_weighted_averaging_af3(msa[perm], mask[perm], pair, w)
    np.testing.assert_allclose(b, a[perm], rtol=1e-6, atol=1e-6)
    msa2 = msa.copy()
    msa2[3] = S.Stream(99).normal(6 * 32).reshape(6, 32)
    c = ops.msa_pair_weighted_averaging_af3(msa2, mask, pair, w)
    np.testing.assert_allclose(c[[0, 1, 2, 4]], a[[0, 1, 2, 4]], rtol=1e-6, atol=1e-6)


def _block_inputs(s, n, seed, cm=32, cz=16):
    w = S.synthetic_msa_module_weights(c_m=cm, c_z=cz, heads=4, dim=8, heads_pair=2, c_outer=8, seed=seed)
    act = S.synthetic_activations(s, n, cm, cz, seed=seed + 50)
    return w, act


def test_oracle_block_orderings_differ():
    """Both orderings over one set of weights move both the msa and the pair
    (test/opendde-branches.test.js:213-224)."""
    w, act = _block_inputs(3, 5, 5)
    a = blocks.msa_block_af3(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w, False)
    b = blocks.msa_block_af3(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w, True)
    for x, y in zip(a, b):
        assert np.sqrt(np.mean((x - y) ** 2)) / np.sqrt(np.mean(x ** 2)) > 1e-6


def test_oracle_block_orderings_agree_without_outer_product():
    """With the outer product's output zeroed the two orderings are one function, and with the
    MSA update's outputs zeroed as well the msa passes through and the pair is the pair-only
    pairformer block's."""
    w, act = _block_inputs(3, 5, 6)
    opm = dict(w["outerProductMean"], outputW=np.zeros_like(w["outerProductMean"]["outputW"]),
               outputB=np.zeros_like(w["outerProductMean"]["outputB"]))
    w0 = dict(w, outerProductMean=opm)
    a = blocks.msa_block_af3(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w0, False)
    b = blocks.msa_block_af3(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w0, True)
    for x, y in zip(a, b):
        np.testing.assert_allclose(x, y, rtol=1e-6, atol=1e-6)
    att = dict(w["msaAttention1"], outputProjection=np.zeros_like(w["msaAttention1"]["outputProjection"]))
    tr = dict(w["msaTransition"], transition2=np.zeros_like(w["msaTransition"]["transition2"]))
    w1 = dict(w0, msaAttention1=att, msaTransition=tr)
    m, p = blocks.msa_block_af3(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w1, False)
    np.testing.assert_array_equal(m, act["msa"])
    rp, _ = blocks.pairformer_block_af3(act["pair"], None, act["pairMask"], None, w1)
    np.testing.assert_allclose(p, rp, rtol=1e-6, atol=1e-6)


def _dev(ctx, x, dt=None):
    import torch
    t = torch.as_tensor(np.ascontiguousarray(x)).to(ctx.device)
    return t.to(dt) if dt is not None else t


@pytest.mark.gpu
@pytest.mark.parametrize("s,n,cm,cz,heads,dim,dt", [(4, 9, 32, 16, 4, 8, "float32"),
                                                    (40, 70, 64, 128, 8, 8, "bfloat16"),
                                                    (7, 130, 64, 32, 2, 32, "float16"),
                                                    (3, 5, 16, 16, 2, 4, "float32"),
                                                    (6, 70, 16, 16, 4, 6, "bfloat16"),
                                                    (256, 200, 64, 128, 8, 8, "bfloat16")])
def test_pair_weighted_averaging(ctx, s, n, cm, cz, heads, dim, dt):
    """The op (update only) against the oracle; ragged token counts (keys past one 64-key
    chunk), a token masked in some sequences, a token no sequence covers; head widths that are
    multiples of 4 run the softmax + GEMM path, 6 the flash path."""
    import torch
    from localfold_amd import device as D
    w, msa, pair, mask = _avg_inputs(s, n, cm, cz, heads, dim, s + n)
    mask[0, 1] = 0
    mask[:, n - 2] = 0
    dw = D.DeviceWeights(ctx.device)
    ws = D.pair_averaging_weights(dw, w)
    x, p = _dev(ctx, msa, getattr(torch, dt)), _dev(ctx, pair, getattr(torch, dt))
    out = D.msa_pair_weighted_averaging(ctx, x, _dev(ctx, mask), p, ws, heads, dim)
    torch.cuda.synchronize()
    ref = ops.msa_pair_weighted_averaging_af3(x.float().cpu().numpy(), mask, p.float().cpu().numpy(), w)
    H.assert_close(out.float().cpu().numpy(), ref, label=f"pwa {s}x{n} {dt}")


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [8, 6])
def test_pair_weighted_averaging_every_key_masked(ctx, dim):
    """Every token masked in every sequence: the reference's f32 softmax is uniform over the
    tokens.  Head dim 8 takes the softmax + GEMM path, head dim 6 the flash path, whose
    +-1e8 clamp leaves the row uniform as well; both are held to the oracle."""
    import torch
    from localfold_amd import device as D
    w, msa, pair, mask = _avg_inputs(3, 20, 32, 16, 4, dim, 17)
    mask[:] = 0
    dw = D.DeviceWeights(ctx.device)
    ws = D.pair_averaging_weights(dw, w)
    out = D.msa_pair_weighted_averaging(ctx, _dev(ctx, msa), _dev(ctx, mask), _dev(ctx, pair), ws, 4, dim)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    H.assert_close(out.cpu().numpy(), ref, label=f"pwa every key masked, head dim {dim}")


@pytest.mark.gpu
def test_pair_weighted_averaging_in_place(ctx):
    import torch
    from localfold_amd import device as D
    w, msa, pair, mask = _avg_inputs(6, 20, 64, 32, 8, 8, 11)
    dw = D.DeviceWeights(ctx.device)
    ws = D.pair_averaging_weights(dw, w)
    x = _dev(ctx, msa)
    D.msa_pair_weighted_averaging(ctx, x, _dev(ctx, mask), _dev(ctx, pair), ws, 8, 8, out=x, accumulate=True)
    torch.cuda.synchronize()
    ref = msa.astype(np.float64) + ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    H.assert_close(x.cpu().numpy(), ref, label="pwa in place")


@pytest.mark.gpu
@pytest.mark.parametrize("s,n,before", [(5, 12, False), (5, 12, True), (33, 40, False)])
def test_msa_module_block(ctx, s, n, before):
    import torch
    from localfold_amd import device as D
    w, act = _block_inputs(s, n, 7 + n, cm=64, cz=32)
    dw = D.DeviceWeights(ctx.device)
    ws = D.msa_module_weights(dw, w)
    msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
    D.msa_module_block(ctx, msa, pair, _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"]), ws, before)
    torch.cuda.synchronize()
    rm, rp = blocks.msa_block_af3(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w, before)
    H.assert_close(msa.cpu().numpy(), rm, label=f"msa module msa before={before}")
    H.assert_close(pair.cpu().numpy(), rp, label=f"msa module pair before={before}")


def _fast_ln_loop(row, scale, offset, eps=1e-5):
    """AF3 layerNorm of one row with the fast variance E[x^2] - E[x]^2
    (cpu/af3/trunk/pairformer.js:68-87), element by element."""
    c = len(row)
    mean = sum(float(v) for v in row) / c
    var = sum(float(v) * float(v) for v in row) / c - mean * mean
    inv = 1.0 / np.sqrt(var + eps)
    return [(float(row[k]) - mean) * inv * float(scale[k]) + float(offset[k]) for k in range(c)]


def _msa_attention_loop(msa, mask, pair, w):
    """`msaAttention` (cpu/af3/trunk/msa.js:157-219) element by element: logits
    flat[(i*N + j)*H + h] into weightsByHead[h][i][j] plus 1e9 (keyMask[j] - 1), softmax over
    j, then averaged[s][i][h*d + e] = sum_j weightsByHead[h][i][j] v[s][j][h*d + e], gated and
    projected."""
    s_, n, c = msa.shape
    cz = pair.shape[-1]
    heads, d = w["heads"], w["dimension"]
    hd = heads * d
    x = [[_fast_ln_loop(msa[s, t], w["actNormScale"], w["actNormOffset"]) for t in range(n)] for s in range(s_)]
    pn = [[_fast_ln_loop(pair[i, j], w["pairNormScale"], w["pairNormOffset"]) for j in range(n)] for i in range(n)]
    pl = np.asarray(w["pairLogits"], np.float64)
    flat = [0.0] * (n * n * heads)
    for i in range(n):
        for j in range(n):
            for h in range(heads):
                flat[(i * n + j) * heads + h] = sum(pn[i][j][k] * pl[k, h] for k in range(cz))
    key_mask = [max([0.0] + [float(mask[s, t]) for s in range(s_)]) for t in range(n)]
    weights = np.zeros((heads, n, n))
    for h in range(heads):
        for i in range(n):
            row = [flat[(i * n + j) * heads + h] + 1e9 * (key_mask[j] - 1) for j in range(n)]
            top = max(row)
            e = [np.exp(v - top) for v in row]
            tot = sum(e)
            weights[h, i] = [v / tot for v in e]
    vp, gq, op = (np.asarray(w[k], np.float64) for k in ("vProjection", "gatingQuery", "outputProjection"))
    out = np.zeros((s_, n, c))
    for s in range(s_):
        values = [[sum(x[s][t][k] * vp[k, o] for k in range(c)) for o in range(hd)] for t in range(n)]
        for i in range(n):
            gated = []
            for h in range(heads):
                for e in range(d):
                    tot = sum(weights[h, i, j] * values[j][h * d + e] for j in range(n))
                    g = sum(x[s][i][k] * gq[k, h * d + e] for k in range(c))
                    gated.append(tot / (1.0 + np.exp(-g)))
            for o in range(c):
                out[s, i, o] = sum(gated[q] * op[q, o] for q in range(hd))
    return out


def test_oracle_per_element_loop_asymmetric_logits():
    """The oracle against a per-element loop of msaAttention on an asymmetric pair (so that
    the logits' [h][i][j] orientation matters: swapping i and j fails), with logits scaled up
    so the softmax is far from uniform, a token covered by one sequence only and one covered
    by none."""
    w, msa, pair, mask = _avg_inputs(3, 5, 12, 6, 2, 3, 11)
    w = dict(w, pairLogits=(w["pairLogits"] * 4).astype(np.float32))
    st = S.Stream(99)
    pair = (pair + 2.0 * np.triu(st.normal(25).reshape(5, 5))[..., None]).astype(np.float32)
    mask[:, 3] = 0
    mask[1:, 1] = 0
    got = ops.msa_pair_weighted_averaging_af3(msa, mask, pair, w)
    ref = _msa_attention_loop(msa, mask, pair, w)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)
    # the orientation is pinned: the transposed pair gives a different answer
    swapped = ops.msa_pair_weighted_averaging_af3(msa, mask, pair.transpose(1, 0, 2).copy(), w)
    assert np.abs(swapped - ref).max() > 1e-2
