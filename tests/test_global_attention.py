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
