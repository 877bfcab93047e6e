"""AF2 input and recycling embedder (`InputEmbedderGpu.run`, webgpu/af2/evoformer/input-embedder.js).

The reference's own test (test/input-embedder.gpu.test.js) compares with a fixture whose weights
and expected tensors are not committed (only its feature files are), so the oracle is pinned by
what the shaders fix: distogram bins worked by hand, glycine's CA as its pseudo-beta, the
relative-position clip, one-hot features selecting weight rows, the recycled rows entering only
where they should.  GPU: the C ABI against the oracle."""
import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import ops
from tests import helpers as H

KEYS = ("targetFeatures", "msaFeatures", "extraMsa", "extraHasDeletion", "extraDeletionValue", "residueIndex",
        "aatype", "previousMsaFirstRow", "previousPair", "previousPositions")


def _oracle(f, w):
    return ops.input_embedder_af2(*(f[k] for k in KEYS), w)


def test_dgram_bins_by_hand():
    """Bins are 1.25 A wide from 3.25 A; at or below 3.25 A no bin, past 20.75 A the last."""
    d = np.array([0.0, 3.25, 4.0, 5.0, 19.0, 20.0, 25.0])
    got = ops.dgram_bins(d * d)
    want = [None, None, 0, 1, 12, 13, 14]
    for row, b in zip(got, want):
        if b is None:
            assert row.sum() == 0
        else:
            assert row.sum() == 1 and row[b] == 1


def test_pseudo_beta_glycine_uses_ca():
    pos = np.zeros((2, 37, 3), np.float32)
    pos[:, 1] = [1, 2, 3]     # CA
    pos[:, 3] = [7, 8, 9]     # CB
    got = ops.pseudo_beta(pos, np.array([7, 0]))
    np.testing.assert_array_equal(got, [[1, 2, 3], [7, 8, 9]])


def _zero_weights(w):
    return {k: np.zeros_like(v) for k, v in w.items()}


def test_relative_position_clip():
    """With only Wrel[k] = k set, pair[i, j] = clip(ri - rj + 32, 0, 64): 32 on the diagonal,
    0 / 64 across the chain gap of 200."""
    w, f = S.synthetic_input_embedder(8, 2, 1, c_m=64, c_z=64, c_e=64)
    z = _zero_weights(w)
    z["relativePositionWeight"] = np.repeat(np.arange(65, dtype=np.float32)[:, None], 64, 1)
    _, pair, _ = _oracle(f, z)
    ri = f["residueIndex"].astype(int)
    want = np.clip(ri[:, None] - ri[None, :] + 32, 0, 64)
    np.testing.assert_array_equal(pair[..., 5], want)
    assert pair[0, 7, 0] == 0 and pair[7, 0, 0] == 64 and pair[3, 3, 0] == 32


def test_one_hot_features_select_weight_rows():
    """One-hot target features and msa features pick weight rows; the extra code picks its
    row, deletion features add rows 23 and 24; the recycled first row enters sequence 0 only
    and a zero recycled row normalises to the offset."""
    w, f = S.synthetic_input_embedder(6, 3, 2, c_m=64, c_z=64, c_e=64)
    f = dict(f, previousMsaFirstRow=np.zeros_like(f["previousMsaFirstRow"]))
    f["msaFeatures"][:] = 0
    f["msaFeatures"][1, 2, 5] = 1
    msa, _, extra = _oracle(f, w)
    aa = f["aatype"].astype(int)
    base = w["preprocess1dBias"] + w["preprocessMsaBias"]
    np.testing.assert_allclose(msa[2, 4], w["preprocess1dWeight"][aa[4] + 1] + base, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(msa[1, 2], w["preprocess1dWeight"][aa[2] + 1] + base + w["preprocessMsaWeight"][5],
                               rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(msa[0, 4], w["preprocess1dWeight"][aa[4] + 1] + base + w["previousMsaNormOffset"],
                               rtol=1e-6, atol=1e-6)
    code = int(f["extraMsa"][1, 3])
    want = (w["extraMsaBias"] + w["extraMsaWeight"][code] + f["extraHasDeletion"][1, 3] * w["extraMsaWeight"][23]
            + f["extraDeletionValue"][1, 3] * w["extraMsaWeight"][24])
    np.testing.assert_allclose(extra[1, 3], want, rtol=1e-6, atol=1e-6)


def test_pair_distogram_term():
    """Only Wpos set: pair[i, j] is Wpos of the bin of |cb_i - cb_j| (none on the diagonal)."""
    w, f = S.synthetic_input_embedder(9, 1, 1, c_m=64, c_z=64, c_e=64)
    z = _zero_weights(w)
    z["previousPositionWeight"] = np.repeat(np.arange(1, 16, dtype=np.float32)[:, None], 64, 1)
    _, pair, _ = _oracle(f, z)
    cb = ops.pseudo_beta(f["previousPositions"], f["aatype"])
    for i in range(9):
        for j in range(9):
            d = np.linalg.norm(cb[i] - cb[j])
            b = 0 if d <= 3.25 else min(int((d - 3.25) // 1.25) + 1, 15)
            assert pair[i, j, 0] == b, (i, j, d)


def _dev(ctx, f):
    import torch
    return {k: torch.as_tensor(np.ascontiguousarray(v, np.float32)).to(ctx.device) for k, v in f.items()}


@pytest.mark.gpu
@pytest.mark.parametrize("L,s,se,cm,cz,ce,dt", [(13, 3, 5, 256, 128, 64, "float32"),
                                                (70, 9, 17, 256, 128, 64, "bfloat16"),
                                                (33, 2, 0, 64, 96, 32, "float16")])
def test_input_embedder(ctx, L, s, se, cm, cz, ce, dt):
    import torch
    from localfold_amd import device as D
    w, f = S.synthetic_input_embedder(L, s, se, c_m=cm, c_z=cz, c_e=ce, seed=L)
    dw = D.DeviceWeights(ctx.device)
    ws = D.input_embedder_weights(dw, w)
    fd = _dev(ctx, f)
    tdt = getattr(torch, dt)
    prev_msa = fd["previousMsaFirstRow"].to(tdt)
    prev_pair = fd["previousPair"].to(tdt)
    msa, pair, extra = D.input_embedder(ctx, fd, ws, cm, cz, ce, tdt, prev_msa, prev_pair, fd["previousPositions"])
    torch.cuda.synchronize()
    f2 = dict(f, previousMsaFirstRow=prev_msa.float().cpu().numpy(), previousPair=prev_pair.float().cpu().numpy())
    rm, rp, re = _oracle(f2, w)
    H.assert_close(msa.float().cpu().numpy(), rm, label=f"embed msa {dt}")
    H.assert_close(pair.float().cpu().numpy(), rp, label=f"embed pair {dt}")
    if se:
        H.assert_close(extra.float().cpu().numpy(), re, label=f"embed extra {dt}")


@pytest.mark.gpu
def test_input_embedder_recycle_zero_and_in_place(ctx):
    """NULL recycled tensors are zeros (recycle 0); the pair may be written over the recycled
    pair it reads."""
    import torch
    from localfold_amd import device as D
    w, f = S.synthetic_input_embedder(21, 4, 6, seed=5)
    dw = D.DeviceWeights(ctx.device)
    ws = D.input_embedder_weights(dw, w)
    fd = _dev(ctx, f)
    msa, pair, extra = D.input_embedder(ctx, fd, ws)
    torch.cuda.synchronize()
    z = dict(f, previousMsaFirstRow=np.zeros_like(f["previousMsaFirstRow"]),
             previousPair=np.zeros_like(f["previousPair"]), previousPositions=np.zeros_like(f["previousPositions"]))
    rm, rp, re = _oracle(z, w)
    H.assert_close(msa.cpu().numpy(), rm, label="embed recycle 0 msa")
    H.assert_close(pair.cpu().numpy(), rp, label="embed recycle 0 pair")
    prev = fd["previousPair"].clone()
    _, pair2, _ = D.input_embedder(ctx, fd, ws, prev_msa=fd["previousMsaFirstRow"], prev_pair=prev,
                                   prev_positions=fd["previousPositions"], pair_out=prev)
    torch.cuda.synchronize()
    _, rp2, _ = _oracle(f, w)
    H.assert_close(pair2.cpu().numpy(), rp2, label="embed pair in place")


@pytest.mark.gpu
def test_af2_recycle_two_recycles(ctx):
    """Two recycles of embed -> extra-MSA block -> Evoformer block through lf_af2_recycle, the
    second embedding the first's msa row 0 and pair (monomer.js:182-330 up to the stack's
    output), against the oracle's composition of the same steps."""
    import torch
    from localfold_amd import device as D
    from oracle import blocks
    L, s_, se, cm, cz, ce = 14, 3, 6, 64, 32, 64
    w, f = S.synthetic_input_embedder(L, s_, se, c_m=cm, c_z=cz, c_e=ce, seed=8)
    wx = S.synthetic_extra_msa_block_weights(c_m=ce, c_z=cz, c_outer=8, heads_msa=8, heads_pair=2, tri_hidden=32,
                                             msa_hidden=4 * ce, pair_hidden=4 * cz, seed=21)
    wm = S.synthetic_block_weights(c_m=cm, c_z=cz, c_outer=8, heads_msa=4, heads_pair=2, tri_hidden=32,
                                   msa_hidden=4 * cm, pair_hidden=4 * cz, seed=22)
    rng = np.random.default_rng(3)
    masks = {"msa": (rng.random((s_, L)) > 0.1).astype(np.float32),
             "extra": (rng.random((se, L)) > 0.2).astype(np.float32), "pair": np.ones((L, L), np.float32)}
    dw = D.DeviceWeights(ctx.device)
    ews = D.input_embedder_weights(dw, w)
    xws, mws = [D.extra_msa_weights(dw, wx)], [D.evoformer_weights(dw, wm)]
    fd = _dev(ctx, f)
    md = {k: torch.as_tensor(v).to(ctx.device) for k, v in masks.items()}
    state = D.af2_recycle_state(fd, cm, cz, ce, torch.float32)
    pos = [None, fd["previousPositions"]]
    rm = rp = None
    for r in range(2):
        D.af2_recycle(ctx, fd, state, md, ews, xws, wx, mws, wm, first=(r == 0), prev_positions=pos[r])
        prev = dict(f, previousMsaFirstRow=np.zeros((L, cm), np.float32) if r == 0 else rm[0],
                    previousPair=np.zeros((L, L, cz), np.float32) if r == 0 else rp,
                    previousPositions=np.zeros_like(f["previousPositions"]) if r == 0 else f["previousPositions"])
        rm, rp, re = _oracle(prev, w)
        re, rp = blocks.extra_msa_block_af2(re, rp, masks["extra"], masks["pair"], wx)
        rm, rp = blocks.evoformer_block_af2(rm, rp, masks["msa"], masks["pair"], wm)
    torch.cuda.synchronize()
    H.assert_close(state["msa"].cpu().numpy(), rm, label="recycle msa")
    H.assert_close(state["pair"].cpu().numpy(), rp, label="recycle pair")
