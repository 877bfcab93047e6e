"""AF2 Evoformer block / stack and AF3 Pairformer block on the GPU through the C ABI, against
the oracle's block composition; the CPU-path block (N_res = 64, N_seq = 1) at full size."""
import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import blocks, ops
from tests import helpers as H

pytestmark = pytest.mark.gpu


def _dev(ctx, x, dt=None):
    import torch
    t = torch.as_tensor(np.ascontiguousarray(x)).to(ctx.device)
    return t.to(dt) if dt is not None else t


def _evo_inputs(s, n, seed):
    w = S.synthetic_block_weights(c_m=256, c_z=128, c_outer=32, heads_msa=8, heads_pair=4, tri_hidden=128,
                                  msa_hidden=1024, pair_hidden=512, seed=seed)
    act = S.synthetic_activations(s, n, 256, 128, seed=seed + 100)
    return w, act


@pytest.mark.parametrize("s,n", [(4, 24), (6, 37)])
def test_evoformer_block(ctx, s, n):
    import torch
    from localfold_amd import device as D
    w, act = _evo_inputs(s, n, 1)
    dw = D.DeviceWeights(ctx.device)
    ws = D.evoformer_weights(dw, w)
    msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
    D.evoformer_block(ctx, msa, pair, _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"]), ws, w)
    torch.cuda.synchronize()
    rm, rp = blocks.evoformer_block_af2(act["msa"], act["pair"], act["msaMask"], act["pairMask"], w)
    H.assert_close(msa.cpu().numpy(), rm, label="evoformer msa")
    H.assert_close(pair.cpu().numpy(), rp, label="evoformer pair")


def test_evoformer_block_from_bundle(ctx, tmp_path):
    """A block whose weights come from an int8 bundle in the reference's manifest + shard layout
    (stacked haiku, codes uploaded as stored, triangle projections in their [in][out] storage)
    matches the oracle block run on those weights' decoded values."""
    import torch
    from localfold_amd import bundle as B, device as D
    from oracle import codec
    w, act = _evo_inputs(3, 28, 5)
    tensors, section, _ = H.af2_stack_bundle_tensors([w], "int8", 64)
    store = B.FileTensorStore.open(H.write_bundle(str(tmp_path), tensors, section))
    wb = B.af2_main_stack_weights(store)[0]

    def decoded(v):
        if isinstance(v, dict) and "dtype" in v:
            return codec.decode(v)
        return {k: decoded(u) for k, u in v.items()} if isinstance(v, dict) else v

    wf = decoded(wb)
    for key in ("triangleMultiplicationOutgoing", "triangleMultiplicationIncoming"):   # oracle: (out,in)
        for name in ("linearAPWeight", "linearAGWeight", "linearBPWeight", "linearBGWeight", "linearZWeight", "linearGWeight"):
            wf[key][name] = wf[key][name].T.copy()
    dw = D.DeviceWeights(ctx.device)
    ws = D.evoformer_weights(dw, wb)
    msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
    D.evoformer_block(ctx, msa, pair, _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"]), ws, wb)
    torch.cuda.synchronize()
    rm, rp = blocks.evoformer_block_af2(act["msa"], act["pair"], act["msaMask"], act["pairMask"], wf)
    H.assert_close(msa.cpu().numpy(), rm, label="bundle block msa")
    H.assert_close(pair.cpu().numpy(), rp, label="bundle block pair")


def test_evoformer_stack_two_blocks(ctx):
    import torch
    from localfold_amd import device as D
    s, n = 4, 20
    w1, act = _evo_inputs(s, n, 2)
    w2, _ = _evo_inputs(s, n, 3)
    dw = D.DeviceWeights(ctx.device)
    ws = [D.evoformer_weights(dw, w1), D.evoformer_weights(dw, w2)]
    msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
    D.evoformer_stack(ctx, msa, pair, _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"]), ws, w1)
    torch.cuda.synchronize()
    rm, rp = act["msa"], act["pair"]
    for w in (w1, w2):
        rm, rp = blocks.evoformer_block_af2(rm, rp, act["msaMask"], act["pairMask"], w)
    H.assert_close(msa.cpu().numpy(), rm, label="stack msa")
    H.assert_close(pair.cpu().numpy(), rp, label="stack pair")


def test_evoformer_stack_mask_tables_follow_the_masks(ctx):
    """A stack call computes its mask tables (key-bias rows, OPM normalisers) in the first block
    and reuses them: two stacks in a row on the same mask buffers with different contents (the
    second masks the last residues and sequences) must each equal block-by-block calls, which
    compute every table afresh -- bit for bit, the kernels being the same."""
    import torch
    from localfold_amd import device as D
    s, n = 5, 24
    w1, act = _evo_inputs(s, n, 4)
    w2, _ = _evo_inputs(s, n, 5)
    dw = D.DeviceWeights(ctx.device)
    ws = [D.evoformer_weights(dw, w1), D.evoformer_weights(dw, w2)]
    mm, pm = _dev(ctx, act["msaMask"]), _dev(ctx, act["pairMask"])
    for variant in range(2):
        if variant == 1:   # new contents in the same buffers
            mm[-1, :] = 0
            mm[:, -3:] = 0
            pm[-3:, :] = 0
            pm[:, -3:] = 0
        msa, pair = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
        D.evoformer_stack(ctx, msa, pair, mm, pm, ws, w1)
        msa2, pair2 = _dev(ctx, act["msa"]), _dev(ctx, act["pair"])
        for wsk, w in zip(ws, (w1, w2)):
            D.evoformer_block(ctx, msa2, pair2, mm, pm, wsk, w)
        torch.cuda.synchronize()
        assert torch.equal(msa, msa2), f"variant {variant}: stack msa differs from its blocks"
        assert torch.equal(pair, pair2), f"variant {variant}: stack pair differs from its blocks"
        rm, rp = act["msa"], act["pair"]
        for w in (w1, w2):
            rm, rp = blocks.evoformer_block_af2(rm, rp, mm.cpu().numpy(), pm.cpu().numpy(), w)
        H.assert_close(msa.cpu().numpy(), rm, label=f"stack msa, masks {variant}")
        H.assert_close(pair.cpu().numpy(), rp, label=f"stack pair, masks {variant}")


def test_config1_af2_block_full_size(ctx):
    """The CPU-path workload: one AF2 block, N_res=64, N_seq=1, c_m 256, c_z 128, fp32 weights
    ~N(0, 1/fan_in), activations ~N(0, 1), seed 0."""
    import torch
    from localfold_amd import device as D
    w, msa0, pair0 = S.config1_inputs(seed=0)
    n = pair0.shape[0]
    msa_mask = np.ones((1, n), np.float32)
    pair_mask = np.ones((n, n), np.float32)
    dw = D.DeviceWeights(ctx.device)
    ws = D.evoformer_weights(dw, w)
    msa, pair = _dev(ctx, msa0), _dev(ctx, pair0)
    D.evoformer_block(ctx, msa, pair, _dev(ctx, msa_mask), _dev(ctx, pair_mask), ws, w)
    torch.cuda.synchronize()
    rm, rp = blocks.evoformer_block_af2(msa0, pair0, msa_mask, pair_mask, w)
    H.assert_close(msa.cpu().numpy(), rm, label="config1 msa")
    H.assert_close(pair.cpu().numpy(), rp, label="config1 pair")


@pytest.mark.parametrize("swap,divide", [(False, False), (True, True)])
def test_pairformer_block(ctx, swap, divide):
    import torch
    from localfold_amd import device as D
    n, cz, cs = 32, 128, 384
    w = S.synthetic_pairformer_weights(cz, cs, 4, 16, 24, seed=9)
    st = S.Stream(10)
    pair0 = st.normal(n * n * cz).reshape(n, n, cz)
    single0 = st.normal(n * cs).reshape(n, cs)
    seq_mask = np.ones(n, np.float32)
    seq_mask[-4:] = 0
    pair_mask = np.outer(seq_mask, seq_mask).astype(np.float32)
    dw = D.DeviceWeights(ctx.device)
    ws = D.pairformer_weights(dw, w)
    pair, single = _dev(ctx, pair0), _dev(ctx, single0)
    D.pairformer_block(ctx, pair, single, _dev(ctx, pair_mask), _dev(ctx, seq_mask), ws,
                       swap_transposed_bias=swap, divide_by_length=divide)
    torch.cuda.synchronize()
    rp, rs = blocks.pairformer_block_af3(pair0, single0, pair_mask, seq_mask, w, swap, divide)
    H.assert_close(pair.cpu().numpy(), rp, label="pairformer pair")
    H.assert_close(single.cpu().numpy(), rs, label="pairformer single")
