"""The smallest shapes each entry point accepts, through the C ABI against the oracle: length 1
and 2 triangle multiplication and triangle attention, one MSA sequence of one residue, a single
transition row and a one-sequence OPM over one and two residues.  The reference's validators
accept every positive size (webgpu/kernels/triangle/types.js:13-48); these are the cases where
every tile, chunk and key block of the kernels is mostly padding."""
import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import ops
from tests import helpers as H

pytestmark = pytest.mark.gpu


def _dev(ctx, x, dt=None):
    import torch
    t = torch.as_tensor(np.ascontiguousarray(x)).to(ctx.device)
    return t.to(dt) if dt is not None else t


@pytest.fixture(scope="module")
def blockw():
    return S.synthetic_block_weights(c_m=256, c_z=128, c_outer=32, heads_msa=8, heads_pair=4, tri_hidden=128,
                                     msa_hidden=1024, pair_hidden=512, seed=1)


@pytest.mark.parametrize("n", [1, 2])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("act", ["float32", "bfloat16"])
def test_tri_mult_tiny(ctx, n, direction, act):
    import torch
    from localfold_amd import device as D
    inp = S.deterministic_triangle_input(n, 128, 128, 5 + n)
    dw = D.DeviceWeights(ctx.device)
    ws = D.tri_mult_weights(dw, inp["weights"])
    z = _dev(ctx, inp["z"]).to(getattr(torch, act))
    out = D.tri_mult(ctx, z, _dev(ctx, np.asarray(inp["mask"], np.float32)), ws, direction)
    torch.cuda.synchronize()
    ref = ops.tri_mult_af2(z.float().cpu().numpy(), inp["mask"], inp["weights"], direction)
    H.assert_close(out.float().cpu().numpy(), ref, max_abs=2e-2, label=f"tri {n} {direction} {act}")


@pytest.mark.parametrize("n", [1, 2])
@pytest.mark.parametrize("ending", [False, True])
def test_triangle_attention_tiny(ctx, blockw, n, ending):
    import torch
    from localfold_amd import capi, device as D
    act = S.synthetic_activations(1, n, 256, 128, seed=40 + n)
    key = "triangleAttentionEnding" if ending else "triangleAttentionStarting"
    tw = blockw[key]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, tw["attention"], tw["pairBias"])
    out = D.attention(ctx, _dev(ctx, act["pair"]), _dev(ctx, act["pairMask"]), ws, 4, ending,
                      capi.LF_BIAS_NORMALIZED_INPUT, None)
    torch.cuda.synchronize()
    ref = ops.attention_af2(act["pair"], act["pairMask"], tw["attention"], 4, ending,
                            dict(tw["pairBias"], source="normalized-input"))
    H.assert_close(out.cpu().numpy(), ref, label=f"tri-att {n} {ending}")


def test_msa_row_attention_one_sequence_one_residue(ctx, blockw):
    import torch
    from localfold_amd import capi, device as D
    act = S.synthetic_activations(1, 1, 256, 128, seed=44)
    row = blockw["msaRowAttention"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, row["attention"], row["pairBias"])
    out = D.attention(ctx, _dev(ctx, act["msa"]), _dev(ctx, act["msaMask"]), ws, 8, False,
                      capi.LF_BIAS_SEPARATE, _dev(ctx, act["pair"]))
    torch.cuda.synchronize()
    pb = dict(row["pairBias"], source="separate", activations=act["pair"])
    ref = ops.attention_af2(act["msa"], act["msaMask"], row["attention"], 8, False, pb)
    H.assert_close(out.cpu().numpy(), ref, label="row 1x1")


@pytest.mark.parametrize("which", ["pairTransition", "msaTransition"])
def test_transition_one_row(ctx, blockw, which):
    import torch
    from localfold_amd import device as D
    w = blockw[which]
    c, hid = w["firstWeight"].shape
    x = S.Stream(9).values(c, 1.5).reshape(1, 1, c)
    dw = D.DeviceWeights(ctx.device)
    out = D.transition(ctx, _dev(ctx, x), D.transition_weights(dw, w), hid)
    torch.cuda.synchronize()
    H.assert_close(out.cpu().numpy(), ops.transition_af2(x, w), label=f"{which} one row")


@pytest.mark.parametrize("s,n", [(1, 1), (1, 2), (2, 1)])
def test_opm_tiny(ctx, blockw, s, n):
    import torch
    from localfold_amd import device as D
    act = S.synthetic_activations(s, n, 256, 128, seed=50 + s * 3 + n)
    w = blockw["outerProductMean"]
    dw = D.DeviceWeights(ctx.device)
    pair = _dev(ctx, act["pair"])
    D.outer_product_mean(ctx, _dev(ctx, act["msa"]), _dev(ctx, act["msaMask"]), D.opm_weights(dw, w), 32, 128,
                         pair=pair, out=pair, accumulate=True)
    torch.cuda.synchronize()
    ref = act["pair"].astype(np.float64) + ops.outer_product_mean_af2(act["msa"], act["msaMask"], w)
    H.assert_close(pair.cpu().numpy(), ref, label=f"opm {s}x{n}")
