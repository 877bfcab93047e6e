"""Transitions (AF2 ReLU, AF3 SwiGLU, row chunking) and outer product mean (AF2, AF3) on the GPU
through the C ABI, against the oracle."""
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


@pytest.mark.parametrize("rows_shape,which,chunk", [((37, 37), "pairTransition", 0), ((6, 45), "msaTransition", 0),
                                                    ((64, 64), "pairTransition", 128 * 1024)])
def test_transition_relu(ctx, blockw, rows_shape, which, chunk):
    import torch
    from localfold_amd import device as D
    w = blockw[which]
    c = w["firstWeight"].shape[0]
    hid = w["firstWeight"].shape[1]
    x = S.Stream(5).values(int(np.prod(rows_shape)) * c, 1.5).reshape(*rows_shape, c)
    dw = D.DeviceWeights(ctx.device)
    ws = D.transition_weights(dw, w)
    out = D.transition(ctx, _dev(ctx, x), ws, hid, chunk_bytes=chunk)
    torch.cuda.synchronize()
    ref = ops.transition_af2(x, w)
    H.assert_close(out.cpu().numpy(), ref, label=f"{which} {rows_shape} chunk={chunk}")


@pytest.mark.parametrize("c,hidden", [(128, 96), (256, 96), (128, 32)])
def test_transition_fused_odd_chunk_count(ctx, c, hidden):
    """Hidden widths of 3 and 1 chunks of 32: the fused kernel stages its weight chunks two to
    an LDS buffer, so a count that is not a multiple of two ends on a half-used buffer."""
    import torch
    from localfold_amd import device as D
    st = S.Stream(c + hidden)
    w = {"layerNormScale": st.values(c, 0.2, 1), "layerNormOffset": st.values(c, 0.1),
         "firstWeight": st.normal(c * hidden, 1 / np.sqrt(c)).reshape(c, hidden), "firstBias": st.values(hidden, 0.1),
         "secondWeight": st.normal(hidden * c, 1 / np.sqrt(hidden)).reshape(hidden, c),
         "secondBias": st.values(c, 0.05)}
    x = st.values(600 * c, 1.5).reshape(600, c)
    dw = D.DeviceWeights(ctx.device)
    out = D.transition(ctx, _dev(ctx, x), D.transition_weights(dw, w), hidden)
    torch.cuda.synchronize()
    H.assert_close(out.cpu().numpy(), ops.transition_af2(x, w), label=f"c={c} hidden={hidden}")


@pytest.mark.parametrize("which,dt", [("pairTransition", "bfloat16"), ("msaTransition", "bfloat16"),
                                      ("msaTransition", "float16")])
def test_transition_fused_dtypes(ctx, blockw, which, dt):
    """16-bit activations, 700 rows (a partial 256-row block); the update alone is compared, so
    the output rounding is that of the update's magnitude."""
    import torch
    from localfold_amd import device as D
    w = blockw[which]
    c, hid = w["firstWeight"].shape
    x = S.Stream(11).values(700 * c, 1.5).reshape(700, c)
    xt = _dev(ctx, x, getattr(torch, dt))
    x16 = xt.float().cpu().numpy()
    dw = D.DeviceWeights(ctx.device)
    ws = D.transition_weights(dw, w)
    out = D.transition(ctx, xt, ws, hid)
    torch.cuda.synchronize()
    H.assert_close(out.float().cpu().numpy(), ops.transition_af2(x16, w), label=f"{which} {dt}")


@pytest.mark.parametrize("c,n", [(128, 40), (384, 50)])
def test_transition_swiglu(ctx, c, n):
    import torch
    from localfold_amd import capi, device as D
    pw = S.synthetic_pairformer_weights(128, 384, 4, 16, 24, seed=6)
    w = pw["pairTransition"] if c == 128 else pw["singleTransition"]
    rows = n * n if c == 128 else n
    x = S.Stream(8).normal(rows * c).reshape(rows, c)
    dw = D.DeviceWeights(ctx.device)
    ws = D.transition_weights(dw, w, capi.LF_TRANSITION_SWIGLU)
    xt = _dev(ctx, x)
    D.transition(ctx, xt, ws, 4 * c, capi.LF_TRANSITION_SWIGLU, out=xt, accumulate=True, fast_variance=True)
    torch.cuda.synchronize()
    ref = x.astype(np.float64) + ops.transition_af3(x, w)
    H.assert_close(xt.cpu().numpy(), ref, label=f"swiglu {c}")


@pytest.mark.parametrize("s,n", [(1, 16), (5, 37), (16, 64), (64, 96), (128, 64)])
def test_opm_af2(ctx, blockw, s, n):
    import torch
    from localfold_amd import device as D
    act = S.synthetic_activations(s, n, 256, 128, seed=s * 7 + n)
    mask = act["msaMask"].copy()
    if s > 2:
        mask[2, ::3] = 0
    w = blockw["outerProductMean"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.opm_weights(dw, w)
    pair = _dev(ctx, act["pair"])
    D.outer_product_mean(ctx, _dev(ctx, act["msa"]), _dev(ctx, mask), ws, 32, 128, pair=pair, out=pair,
                         accumulate=True)
    torch.cuda.synchronize()
    ref = act["pair"].astype(np.float64) + ops.outer_product_mean_af2(act["msa"], mask, w)
    H.assert_close(pair.cpu().numpy(), ref, label=f"opm {s}x{n}")


@pytest.mark.parametrize("dt,accumulate", [("bfloat16", True), ("float16", False), ("float32", False)])
def test_opm_fused_output(ctx, blockw, dt, accumulate):
    """c_outer 32, c_z 128 with whole 256-row outer tiles (N = 64, S = 64) takes the fused kernel:
    the output GEMM, the /den and the residual run on the outer-product tile in LDS.  Pair in
    each activation dtype, accumulated in place or written to a separate output."""
    import torch
    from localfold_amd import device as D
    s_, n = 64, 64
    act = S.synthetic_activations(s_, n, 256, 128, seed=91)
    mask = act["msaMask"].copy()
    mask[3, ::4] = 0
    mask[:, -3:] = 0
    w = blockw["outerProductMean"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.opm_weights(dw, w)
    tdt = getattr(torch, dt)
    pair_in = _dev(ctx, act["pair"]).to(tdt)
    before = pair_in.float().cpu().numpy().astype(np.float64)   # the stored input, before the update
    out = pair_in if accumulate else torch.full_like(pair_in, 7.0)
    D.outer_product_mean(ctx, _dev(ctx, act["msa"]), _dev(ctx, mask), ws, 32, 128, pair=pair_in, out=out,
                         accumulate=accumulate)
    torch.cuda.synchronize()
    upd = ops.outer_product_mean_af2(act["msa"], mask, w)
    ref = (before + upd) if accumulate else upd
    # the result is stored in the pair dtype: add one rounding of the largest value to the
    # bound (half an ulp, at most 2^-8 of the value for bf16's 8 significant bits, 2^-11 for f16)
    half_ulp = {"bfloat16": 2.0 ** -8, "float16": 2.0 ** -11, "float32": 0.0}[dt]
    H.assert_close(out.float().cpu().numpy(), ref, max_abs=H.MAX_ABS + half_ulp * float(np.abs(ref).max()),
                   label=f"opm fused {dt} accumulate={accumulate}")


def test_opm_af3(ctx):
    import torch
    from localfold_amd import capi, device as D
    s_, n, cm, co, cz = 6, 30, 64, 32, 128
    st = S.Stream(4)
    msa = st.normal(s_ * n * cm).reshape(s_, n, cm)
    mask = (st.uniform(s_ * n) > 0.2).astype(np.float32).reshape(s_, n)
    w = {"layerNormInputScale": st.values(cm, 0.2, 1), "layerNormInputOffset": st.values(cm, 0.1),
         "leftProjection": st.normal(cm * co, 1 / np.sqrt(cm)).reshape(cm, co),
         "rightProjection": st.normal(cm * co, 1 / np.sqrt(cm)).reshape(cm, co),
         "outputW": st.normal(co * co * cz, 1 / co).reshape(co * co, cz), "outputB": st.values(cz, 0.05)}
    dw = D.DeviceWeights(ctx.device)
    ws = D.opm_weights(dw, w, capi.LF_AF3)
    out = D.outer_product_mean(ctx, _dev(ctx, msa), _dev(ctx, mask), ws, co, cz, fast_variance=True)
    torch.cuda.synchronize()
    ref = ops.outer_product_mean_af3(msa, mask, w)
    H.assert_close(out.cpu().numpy(), ref, label="opm af3")
