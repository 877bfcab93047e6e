"""Global column attention and the AF2 extra-MSA block (`encodeGlobalAttention`,
`encodeExtraMsaBlock`, webgpu/af2/evoformer/block.js:88-400, 953-1030, 1715-1744).

CPU: the oracle against properties the reference's semantics fix (sequence permutation
equivariance, masked sequences invisible to the others, the one-sequence and all-masked
closed forms).  GPU: the C ABI against the oracle (op, block, two-block stack)."""
import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import blocks, ops
from tests import helpers as H


def _inputs(s, n, c, heads, seed, masked=True):
    g = S.synthetic_global_attention_weights(c, heads, seed)
    st = S.Stream(seed + 1)
    msa = st.normal(s * n * c).reshape(s, n, c).astype(np.float32)
    mask = np.ones((s, n), np.float32)
    if masked and s > 2:
        mask[1, ::3] = 0
        mask[-1, 2:] = 0
    return g, msa, mask


def test_oracle_permutation_equivariance():
    """Permuting the sequences (msa rows and mask rows together) permutes the update rows."""
    g, msa, mask = _inputs(7, 5, 64, 8, 3)
    perm = np.array([3, 0, 6, 1, 5, 2, 4])
    a = ops.global_column_attention_af2(msa, mask, g["attention"], 8)
    b = ops.global_column_attention_af2(msa[perm], mask[perm], g["attention"], 8)
    np.testing.assert_allclose(b, a[perm], rtol=1e-5, atol=1e-6)


def test_oracle_masked_sequences_do_not_reach_the_others():
    """A masked sequence is out of the query mean and its logit is -1e9: changing its
    activations leaves every unmasked sequence's update unchanged."""
    g, msa, mask = _inputs(6, 4, 64, 8, 4, masked=False)
    mask[2, :] = 0
    a = ops.global_column_attention_af2(msa, mask, g["attention"], 8)
    msa2 = msa.copy()
    msa2[2] = S.Stream(9).normal(4 * 64).reshape(4, 64)
    b = ops.global_column_attention_af2(msa2, mask, g["attention"], 8)
    keep = [0, 1, 3, 4, 5]
    np.testing.assert_allclose(b[keep], a[keep], rtol=1e-5, atol=1e-6)


def _closed_form(x_row, attended, w, heads):
    gate = ops.sigmoid(np.asarray(x_row, np.float64) @ w["gatingWeight"] + w["gatingBias"])
    return (gate * np.tile(attended, heads)) @ w["outputWeight"] + w["outputBias"]


def test_oracle_single_sequence_closed_form():
    """One unmasked sequence: the softmax is 1, so every head attends to that sequence's value
    row; the update is (sigmoid(x Wg + bg) * [v]*H) Wo + bo."""
    g, msa, mask = _inputs(1, 3, 64, 8, 5, masked=False)
    w = g["attention"]
    got = ops.global_column_attention_af2(msa, mask, w, 8)
    x = ops.layer_norm(msa, w["queryNormScale"], w["queryNormOffset"])
    for i in range(3):
        v = np.asarray(x[0, i], np.float64) @ w["valueWeight"]
        np.testing.assert_allclose(got[0, i], _closed_form(x[0, i], v, w, 8), rtol=2e-5, atol=2e-5)


def test_oracle_fully_masked_column_is_uniform():
    """Every sequence of a column masked: all logits are -1e9, the softmax is uniform and each
    head attends to the mean value row (what the reference's replace-by--1e9 gives)."""
    g, msa, mask = _inputs(5, 2, 64, 8, 6, masked=False)
    mask[:, 1] = 0
    w = g["attention"]
    got = ops.global_column_attention_af2(msa, mask, w, 8)
    x = ops.layer_norm(msa, w["queryNormScale"], w["queryNormOffset"])
    vmean = (np.asarray(x[:, 1], np.float64) @ w["valueWeight"]).mean(0)
    for s in range(5):
        np.testing.assert_allclose(got[s, 1], _closed_form(x[s, 1], vmean, w, 8), rtol=2e-5, atol=2e-5)


def _dev(ctx, x, dt=None):
    import torch
    t = torch.as_tensor(np.ascontiguousarray(x)).to(ctx.device)
    return t.to(dt) if dt is not None else t


@pytest.mark.gpu
@pytest.mark.parametrize("s,n,c,heads,dt", [(5, 7, 64, 8, "float32"), (37, 20, 64, 8, "bfloat16"),
                                            (300, 9, 64, 8, "float16"), (9, 11, 64, 4, "float32"),
                                            (6, 13, 64, 2, "bfloat16")])
def test_global_column_attention(ctx, s, n, c, heads, dt):
    """The op (update only) against the oracle; 300 sequences give each thread of a column
    more than one; head widths 8, 16 and 32."""
    import torch
    from localfold_amd import device as D
    g, msa, mask = _inputs(s, n, c, heads, s + n)
    dw = D.DeviceWeights(ctx.device)
    ws = D.global_attention_weights(dw, g["attention"])
    x = _dev(ctx, msa, getattr(torch, dt))
    out = D.global_column_attention(ctx, x, _dev(ctx, mask), ws, heads)
    torch.cuda.synchronize()
    ref = ops.global_column_attention_af2(x.float().cpu().numpy(), mask, g["attention"], heads)
    H.assert_close(out.float().cpu().numpy(), ref, label=f"global {s}x{n} {dt}")


@pytest.mark.gpu
def test_global_column_attention_in_place(ctx):
    import torch
    from localfold_amd import device as D
    g, msa, mask = _inputs(12, 10, 64, 8, 21)
    dw = D.DeviceWeights(ctx.device)
    ws = D.global_attention_weights(dw, g["attention"])
    x = _dev(ctx, msa)
    D.global_column_attention(ctx, x, _dev(ctx, mask), ws, 8, out=x, accumulate=True)
    torch.cuda.synchronize()
    ref = msa.astype(np.float64) + ops.global_column_attention_af2(msa, mask, g["attention"], 8)
    H.assert_close(x.cpu().numpy(), ref, label="global in place")


def _extra_inputs(s, n, seed):
    w = S.synthetic_extra_msa_block_weights(c_m=64, c_z=32, c_outer=8, heads_msa=8, heads_pair=2, tri_hidden=32,
                                            msa_hidden=256, pair_hidden=128, seed=seed)
    act = S.synthetic_activations(s, n, 64, 32, seed=seed + 50)
    return w, act


@pytest.mark.gpu
@pytest.mark.parametrize("s,n", [(5, 12), (40, 17)])
def test_extra_msa_block(ctx, s, n):
    import torch
    from localfold_amd import device as D
    w, act = _extra_inputs(s, n, 2)
    dw = D.DeviceWeights(ctx.device)
    ws = D.extra_msa_weights(dw, w)
    msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
    D.extra_msa_block(ctx, msa, pair, _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"]), ws, w)
    torch.cuda.synchronize()
    rm, rp = blocks.extra_msa_block_af2(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w)
    H.assert_close(msa.cpu().numpy(), rm, label="extra msa")
    H.assert_close(pair.cpu().numpy(), rp, label="extra pair")


@pytest.mark.gpu
def test_extra_msa_stack_two_blocks(ctx):
    import torch
    from localfold_amd import device as D
    w0, act = _extra_inputs(6, 10, 3)
    w1, _ = _extra_inputs(6, 10, 4)
    dw = D.DeviceWeights(ctx.device)
    wss = [D.extra_msa_weights(dw, w0), D.extra_msa_weights(dw, w1)]
    msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
    D.extra_msa_stack(ctx, msa, pair, _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"]), wss, w0)
    torch.cuda.synchronize()
    rm, rp = act["msa"], act["pair"]
    for w in (w0, w1):
        rm, rp = blocks.extra_msa_block_af2(rm, rp, act["msaMask"], act["pairMask"], w)
    H.assert_close(msa.cpu().numpy(), rm, label="extra stack msa")
    H.assert_close(pair.cpu().numpy(), rp, label="extra stack pair")


def _ln_loop(row, scale, offset, eps=1e-5):
    """Two-pass layer norm of one row, element by element (the WGSL normalise)."""
    c = len(row)
    mean = sum(float(v) for v in row) / c
    var = sum((float(v) - mean) ** 2 for v in row) / c
    inv = 1.0 / np.sqrt(var + eps)
    return [(float(row[k]) - mean) * inv * float(scale[k]) + float(offset[k]) for k in range(c)]


def _global_loop(msa, mask, w, heads):
    """The kernels of `webgpu/af2/evoformer/block.js:101-400`, element by element: keys and
    values (one shared head of width d, `:101-146`), the column's masked mean over the
    sequences and its projection onto the heads times inverseSqrt(d) (`:166-226`), a per-lane
    online softmax merged across 64 lanes with -1e9 for masked sequences (`:240-300`), and
    the gated output projection (`:329-400`)."""
    s_, n, c = msa.shape
    hd = len(w["gatingBias"])
    d = hd // heads
    wq, wk, wv = (np.asarray(w[k], np.float64) for k in ("queryWeight", "keyWeight", "valueWeight"))
    wg, wo = np.asarray(w["gatingWeight"], np.float64), np.asarray(w["outputWeight"], np.float64)
    x = [[_ln_loop(msa[s, i], w["queryNormScale"], w["queryNormOffset"]) for i in range(n)] for s in range(s_)]
    out = np.zeros((s_, n, c))
    for i in range(n):
        key = [[sum(x[s][i][k] * wk[k, e] for k in range(c)) for e in range(d)] for s in range(s_)]
        val = [[sum(x[s][i][k] * wv[k, e] for k in range(c)) for e in range(d)] for s in range(s_)]
        count = sum(float(mask[s, i]) for s in range(s_))
        den = 1e-10 + count
        means = [sum(x[s][i][k] * float(mask[s, i]) for s in range(s_)) / den for k in range(c)]
        attended = [0.0] * hd
        for h in range(heads):
            q = [sum(means[k] * wq[k, h * d + e] for k in range(c)) / np.sqrt(d) for e in range(d)]
            lanes = []
            for lane in range(64):
                mx, dn, acc = -1e30, 0.0, [0.0] * d
                for s in range(lane, s_, 64):
                    logit = sum(q[e] * key[s][e] for e in range(d))
                    if mask[s, i] == 0:
                        logit = -1e9
                    nm = max(mx, logit)
                    ps, wt = np.exp(mx - nm), np.exp(logit - nm)
                    dn = dn * ps + wt
                    acc = [acc[e] * ps + wt * val[s][e] for e in range(d)]
                    mx = nm
                lanes.append((mx, dn, acc))
            top = max(t[0] for t in lanes)
            tot = sum(t[1] * np.exp(t[0] - top) for t in lanes)
            for e in range(d):
                attended[h * d + e] = sum(t[2][e] * np.exp(t[0] - top) for t in lanes) / tot
        for s in range(s_):
            gated = [attended[g] / (1.0 + np.exp(-(float(w["gatingBias"][g]) +
                                                   sum(x[s][i][k] * wg[k, g] for k in range(c)))))
                     for g in range(hd)]
            for o in range(c):
                out[s, i, o] = float(w["outputBias"][o]) + sum(gated[g] * wo[g, o] for g in range(hd))
    return out


@pytest.mark.parametrize("s,heads,seed", [(5, 2, 61), (70, 4, 62)])
def test_oracle_per_element_loop(s, heads, seed):
    """The oracle against the kernels' own element-by-element semantics, with a masked
    sequence, a partly masked column and (at 70 sequences) lanes holding more than one
    sequence; non-trivial LN scale and offset."""
    n, c = 3, 16
    g = S.synthetic_global_attention_weights(c, heads, seed)
    w = dict(g["attention"])
    st = S.Stream(seed + 3)
    w["queryNormScale"] = (1.0 + 0.3 * st.normal(c)).astype(np.float32)
    w["queryNormOffset"] = (0.2 * st.normal(c)).astype(np.float32)
    msa = st.normal(s * n * c).reshape(s, n, c).astype(np.float32)
    mask = np.ones((s, n), np.float32)
    mask[1, :] = 0
    mask[::3, 2] = 0
    got = ops.global_column_attention_af2(msa, mask, w, heads)
    ref = _global_loop(msa, mask, w, heads)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)


def _two_sequence_case(d, masked_second):
    """Two sequences, one residue, one head, C = 2.  A row (u, -u) normalises to (r, -r) with
    r = u / sqrt(u^2 + eps), so with unit LN scale and offset beta: x1 = (r, -r) + beta and
    x2 = (-r, r) + beta.  Hand-picked weights make every intermediate a short sum."""
    u, eps = 3.0, 1e-5
    r = u / np.sqrt(u * u + eps)
    beta = np.array([0.5, -0.25])
    w = {
        "queryNormScale": np.ones(2, np.float32), "queryNormOffset": beta.astype(np.float32),
        "queryWeight": np.zeros((2, d), np.float32), "keyWeight": np.zeros((2, d), np.float32),
        "valueWeight": np.zeros((2, d), np.float32), "gatingWeight": np.zeros((2, d), np.float32),
        "gatingBias": np.zeros(d, np.float32), "outputWeight": np.zeros((d, 2), np.float32),
        "outputBias": np.array([0.125, -0.5], np.float32),
    }
    w["queryWeight"][0, 0], w["queryWeight"][1, 0] = 4.0, 2.0      # q0 = 4 m0 + 2 m1
    w["keyWeight"][0, 0], w["keyWeight"][1, 0] = 1.0, -1.0         # k0 = x0 - x1
    w["valueWeight"][0, 0], w["valueWeight"][1, 1 % d] = 1.0, 1.0  # v0 = x0, v1 = x1
    w["gatingBias"][:] = 0.0                                       # gate = sigmoid(0) = 1/2 ...
    w["gatingWeight"][0, 0] = 1.0                                  # ... except channel 0: sigmoid(x0)
    w["outputWeight"][0, 0], w["outputWeight"][1 % d, 1] = 1.0, 2.0
    msa = np.array([[[u, -u]], [[-u, u]]], np.float32)
    mask = np.array([[1.0], [0.0 if masked_second else 1.0]], np.float32)
    x1, x2 = np.array([r, -r]) + beta, np.array([-r, r]) + beta
    m = x1 if masked_second else (x1 + x2) * (2.0 / (2.0 + 1e-10)) / 2.0
    q0 = (4.0 * m[0] + 2.0 * m[1]) / np.sqrt(d)                     # the 1/sqrt(d) scale
    l1, l2 = q0 * (x1[0] - x1[1]), q0 * (x2[0] - x2[1])
    p1 = 1.0 if masked_second else 1.0 / (1.0 + np.exp(l2 - l1))
    att = p1 * np.array([x1[0], x1[1]]) + (1.0 - p1) * np.array([x2[0], x2[1]])
    expect = []
    for x in (x1, x2):
        g0 = 1.0 / (1.0 + np.exp(-x[0]))
        if d == 1:   # v0 and v1 share the one slot: channel 0 takes x0 + x1 of the attended rows
            a0 = att[0] + att[1]
            expect.append([0.125 + g0 * a0, -0.5 + 2.0 * g0 * a0])
        else:
            expect.append([0.125 + g0 * att[0], -0.5 + 2.0 * 0.5 * att[1]])
    return msa, mask, w, np.array(expect)[:, None, :]


@pytest.mark.parametrize("d", [1, 2, 8])
@pytest.mark.parametrize("masked_second", [False, True])
def test_oracle_two_sequence_closed_form(d, masked_second):
    """Fixes the q scale 1/sqrt(d) (1/d or none changes the softmax), the masked MEAN for the
    query (a masked sum doubles q), and the -1e9 for a masked sequence (its p is 0 and the
    unmasked sequence attends only to itself)."""
    msa, mask, w, expect = _two_sequence_case(d, masked_second)
    got = ops.global_column_attention_af2(msa, mask, w, 1)
    np.testing.assert_allclose(got, expect, rtol=1e-5, atol=1e-6)


def test_oracle_two_sequence_closed_form_is_sensitive():
    """The closed form is not blind: a doubled q (a sum, not a mean) moves the result."""
    msa, mask, w, expect = _two_sequence_case(2, False)
    w2 = dict(w, queryWeight=w["queryWeight"] * 2)
    got = ops.global_column_attention_af2(msa, mask, w2, 1)
    assert np.abs(got - expect).max() > 1e-2


@pytest.mark.gpu
def test_evoformer_pair_stack_two_blocks(ctx):
    """lf_evoformer_pair_stack (ExtraMsaPairStackGpu): two pair halves against the oracle;
    the msa is read and left bit-identical."""
    import torch
    from localfold_amd import device as D
    w0, act = _extra_inputs(7, 11, 5)
    w1, _ = _extra_inputs(7, 11, 6)
    dw = D.DeviceWeights(ctx.device)
    wss = [D.evoformer_weights(dw, w0), D.evoformer_weights(dw, w1)]
    msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
    D.evoformer_pair_stack(ctx, msa, pair, _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"]), wss, w0)
    torch.cuda.synchronize()
    rp = act["pair"]
    for w in (w0, w1):
        rp = blocks.evoformer_pair_block_af2(act["msa"], rp, act["msaMask"], act["pairMask"], w)
    np.testing.assert_array_equal(msa.cpu().numpy(), act["msa"])
    H.assert_close(pair.cpu().numpy(), rp, label="pair stack pair")
