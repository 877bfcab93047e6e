"""Gated attention on the GPU through the C ABI against the oracle: MSA row attention with a
separate pair bias, column attention, triangle attention (starting / ending, bias from the
normalised input), AF3 grid and single attention; activation and weight dtypes; full-size
N = 512 workload (checked on a sample of batch rows)."""
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


def _run(ctx, act, mask, ws, heads, transpose=False, bias_mode=0, pair=None, act_dt=None, **kw):
    import torch
    from localfold_amd import device as D
    a = _dev(ctx, act, act_dt)
    m = _dev(ctx, np.asarray(mask, np.float32))
    p = _dev(ctx, pair, act_dt) if pair is not None else None
    out = D.attention(ctx, a, m, ws, heads, transpose, bias_mode, p, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), a.float().cpu().numpy(), (p.float().cpu().numpy() if p is not None else None)


@pytest.fixture(scope="module")
def blockw():
    return S.synthetic_block_weights(c_m=256, c_z=128, c_outer=32, heads_msa=8, heads_pair=4, tri_hidden=128,
                                     msa_hidden=1024, pair_hidden=512, seed=1)


@pytest.mark.parametrize("s,n", [(5, 40), (3, 37), (8, 64)])
def test_msa_row_attention_pair_bias(ctx, blockw, s, n):
    from localfold_amd import capi, device as D
    act = S.synthetic_activations(s, n, 256, 128, seed=s + n)
    row = blockw["msaRowAttention"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, row["attention"], row["pairBias"])
    out, _, _ = _run(ctx, act["msa"], act["msaMask"], ws, 8, False, capi.LF_BIAS_SEPARATE, act["pair"])
    pb = dict(row["pairBias"], source="separate", activations=act["pair"])
    ref = ops.attention_af2(act["msa"], act["msaMask"], row["attention"], 8, False, pb)
    H.assert_close(out, ref, label=f"row {s}x{n}")


@pytest.mark.parametrize("c,heads", [(64, 8), (64, 4), (48, 4), (40, 8), (64, 2)])
@pytest.mark.parametrize("n", [40, 64])
def test_row_attention_head_widths(ctx, c, heads, n):
    """Head dims 8, 16, 12, 5 and 32 over whole (64) and ragged (40) key chunks: the 16-wide
    (d <= 16) and 32-wide kernels, with and without zeroing the unwritten head dims and keys."""
    from localfold_amd import capi, device as D
    w = S.synthetic_block_weights(c_m=c, c_z=32, c_outer=8, heads_msa=heads, heads_pair=2, tri_hidden=32,
                                  msa_hidden=2 * c, pair_hidden=64, seed=heads + c)
    act = S.synthetic_activations(3, n, c, 32, seed=n + c)
    row = w["msaRowAttention"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, row["attention"], row["pairBias"])
    out, _, _ = _run(ctx, act["msa"], act["msaMask"], ws, heads, False, capi.LF_BIAS_SEPARATE, act["pair"])
    pb = dict(row["pairBias"], source="separate", activations=act["pair"])
    ref = ops.attention_af2(act["msa"], act["msaMask"], row["attention"], heads, False, pb)
    assert np.isfinite(out).all()
    H.assert_close(out, ref, label=f"row c={c} heads={heads} n={n}")


@pytest.mark.parametrize("n", [24, 101])
def test_triangle_attention_256_channels(ctx, n):
    """256-channel triangle attention, 8 heads of 32: 17 projection chunks of 64 columns (q, k,
    v, g and the bias), which the 256-wide projection kernel stages two to an LDS buffer, over
    column ranges of one chunk (N = 24) and of two with an odd remainder (N = 101)."""
    from localfold_amd import capi, device as D
    w = S.synthetic_block_weights(c_m=64, c_z=256, c_outer=8, heads_msa=2, heads_pair=8, tri_hidden=32,
                                  msa_hidden=64, pair_hidden=64, seed=n)
    tw = w["triangleAttentionStarting"]
    act = S.synthetic_activations(1, n, 64, 256, seed=n + 1)
    mask = act["pairMask"].copy()
    mask[:, -2:] = 0
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, tw["attention"], tw["pairBias"])
    out, _, _ = _run(ctx, act["pair"], mask, ws, 8, False, capi.LF_BIAS_NORMALIZED_INPUT)
    ref = ops.attention_af2(act["pair"], mask, tw["attention"], 8, False,
                            dict(tw["pairBias"], source="normalized-input"))
    H.assert_close(out, ref, label=f"tri-att c=256 n={n}")


def test_row_attention_keys_over_one_stage(ctx, blockw):
    """600 keys (padded to 640): the kernel stages 512 keys in LDS at a time, so the second
    stage (128 keys, the last ones masked) runs after a block-wide reload."""
    from localfold_amd import capi, device as D
    s, n = 2, 600
    act = S.synthetic_activations(s, n, 256, 128, seed=6)
    mask = np.ones((s, n), np.float32)
    mask[:, -40:] = 0
    mask[1, 100:130] = 0
    row = blockw["msaRowAttention"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, row["attention"], row["pairBias"])
    out, _, _ = _run(ctx, act["msa"], mask, ws, 8, False, capi.LF_BIAS_SEPARATE, act["pair"])
    pb = dict(row["pairBias"], source="separate", activations=act["pair"])
    ref = ops.attention_af2(act["msa"], mask, row["attention"], 8, False, pb)
    H.assert_close(out, ref, label=f"row {s}x{n}")


@pytest.mark.parametrize("s,n", [(5, 40), (33, 17)])
def test_msa_column_attention(ctx, blockw, s, n):
    from localfold_amd import device as D
    act = S.synthetic_activations(s, n, 256, 128, seed=3)
    col = blockw["msaColumnAttention"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, col["attention"])
    out, _, _ = _run(ctx, act["msa"], act["msaMask"], ws, 8, True)
    ref = ops.attention_af2(act["msa"], act["msaMask"], col["attention"], 8, True)
    H.assert_close(out, ref, label=f"column {s}x{n}")


@pytest.mark.parametrize("n", [24, 37, 70, 130])
@pytest.mark.parametrize("ending", [False, True])
def test_triangle_attention(ctx, blockw, n, ending):
    from localfold_amd import capi, device as D
    act = S.synthetic_activations(1, n, 256, 128, seed=n)
    mask = act["pairMask"].copy()
    mask[:, -3:] = 0
    key = "triangleAttentionEnding" if ending else "triangleAttentionStarting"
    tw = blockw[key]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, tw["attention"], tw["pairBias"])
    out, _, _ = _run(ctx, act["pair"], mask, ws, 4, ending, capi.LF_BIAS_NORMALIZED_INPUT)
    ref = ops.attention_af2(act["pair"], mask, tw["attention"], 4, ending,
                            dict(tw["pairBias"], source="normalized-input"))
    H.assert_close(out, ref, label=f"tri-att {n} {ending}")


@pytest.mark.parametrize("act_dt,wdt", [("bfloat16", "int8"), ("float16", "int5"), ("float32", "float16")])
def test_dtypes(ctx, blockw, act_dt, wdt):
    import torch
    from localfold_amd import capi, device as D
    n = 48
    act = S.synthetic_activations(1, n, 256, 128, seed=7)
    tw = blockw["triangleAttentionStarting"]
    names = ["queryWeight", "keyWeight", "valueWeight", "gatingWeight", "outputWeight"]
    rec, dec = H.quantise_weights(tw["attention"], names, wdt, False, 1)
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, rec, tw["pairBias"])
    out, ain, _ = _run(ctx, act["pair"], act["pairMask"], ws, 4, False, capi.LF_BIAS_NORMALIZED_INPUT,
                       act_dt=getattr(torch, act_dt))
    ref = ops.attention_af2(ain, act["pairMask"], dec, 4, False, dict(tw["pairBias"], source="normalized-input"))
    H.assert_close(out, ref, label=f"{act_dt}/{wdt}")


@pytest.mark.parametrize("wdt,ending", [("int8", False), ("int5", True), ("float16", False)])
def test_output_projection_decoded_in_kernel(ctx, blockw, wdt, ending):
    """N = 192 gives 36,864 rows, enough 16-row tiles for the weight-resident output projection,
    which then decodes the stored output weights itself (no expansion of them)."""
    from localfold_amd import capi, device as D
    n = 192
    act = S.synthetic_activations(1, n, 256, 128, seed=13)
    key = "triangleAttentionEnding" if ending else "triangleAttentionStarting"
    tw = blockw[key]
    names = ["queryWeight", "keyWeight", "valueWeight", "gatingWeight", "outputWeight"]
    rec, dec = H.quantise_weights(tw["attention"], names, wdt, False, 1)
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, rec, tw["pairBias"])
    out, _, _ = _run(ctx, act["pair"], act["pairMask"], ws, 4, ending, capi.LF_BIAS_NORMALIZED_INPUT)
    ref = ops.attention_af2(act["pair"], act["pairMask"], dec, 4, ending, dict(tw["pairBias"], source="normalized-input"))
    H.assert_close(out, ref, label=f"in-kernel output decode {wdt}")


def test_msa_row_attention_output_decoded_in_kernel(ctx, blockw):
    """c_m = 256 (K = N = 256 output projection) over 36,864 rows, int8 weights in groups of 64."""
    from localfold_amd import capi, device as D
    s_, n = 192, 192
    act = S.synthetic_activations(s_, n, 256, 128, seed=17)
    row = blockw["msaRowAttention"]
    names = ["queryWeight", "keyWeight", "valueWeight", "gatingWeight", "outputWeight"]
    rec, dec = H.quantise_weights(row["attention"], names, "int8", False, 1)
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, rec, row["pairBias"])
    out, _, _ = _run(ctx, act["msa"], act["msaMask"], ws, 8, False, capi.LF_BIAS_SEPARATE, act["pair"])
    pb = dict(row["pairBias"], source="separate", activations=act["pair"])
    ref = ops.attention_af2(act["msa"], act["msaMask"], dec, 8, False, pb)
    H.assert_close(out, ref, label="row attention, in-kernel output decode")


def test_accumulate_in_place_transposed(ctx, blockw):
    import torch
    from localfold_amd import capi, device as D
    n = 40
    act = S.synthetic_activations(1, n, 256, 128, seed=11)
    tw = blockw["triangleAttentionEnding"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, tw["attention"], tw["pairBias"])
    z = _dev(ctx, act["pair"])
    m = _dev(ctx, act["pairMask"])
    D.attention(ctx, z, m, ws, 4, True, capi.LF_BIAS_NORMALIZED_INPUT, out=z, accumulate=True)
    torch.cuda.synchronize()
    ref = act["pair"].astype(np.float64) + ops.attention_af2(act["pair"], act["pairMask"], tw["attention"], 4, True,
                                                             dict(tw["pairBias"], source="normalized-input"))
    H.assert_close(z.cpu().numpy(), ref)


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("act_dt", ["float32", "bfloat16"])
def test_output_projection_many_rows(ctx, blockw, transpose, act_dt):
    """131 x 257 = 33667 rows (above 8 waves x 16 rows per CU, and not a multiple of 16): the
    output projection runs as the weight-resident row GEMM and ends on a partial tile; the
    update is accumulated in place, through the transposed row map for column attention."""
    import torch
    from localfold_amd import device as D
    s, n = 131, 257
    act = S.synthetic_activations(s, n, 256, 128, seed=21)
    mask = act["msaMask"].copy()
    mask[:, -5:] = 0
    col = blockw["msaColumnAttention"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, col["attention"])
    x = _dev(ctx, act["msa"], getattr(torch, act_dt))
    ain = x.float().cpu().numpy()
    D.attention(ctx, x, _dev(ctx, mask), ws, 8, transpose, out=x, accumulate=True)
    torch.cuda.synchronize()
    ref = ain.astype(np.float64) + ops.attention_af2(ain, mask, col["attention"], 8, transpose)
    m = H.metrics(x.float().cpu().numpy(), ref)
    print(f"{act_dt} transpose={transpose}: {m}", flush=True)
    if act_dt == "float32":
        H.assert_close(x.cpu().numpy(), ref, label=f"many rows {act_dt} {transpose}")
    else:   # bf16 storage of the result: its rounding (|x| ~ 4, 2^-9 relative) on top of the bound
        H.assert_close(x.float().cpu().numpy(), ref, max_abs=H.MAX_ABS + float(np.abs(ref).max()) * 2.0 ** -8,
                       label=f"many rows {act_dt} {transpose}")


@pytest.mark.parametrize("transpose,swap", [(False, False), (True, False), (True, True)])
def test_af3_grid_attention(ctx, transpose, swap):
    from localfold_amd import capi, device as D
    n, c = 36, 128
    w = S.synthetic_pairformer_weights(c, 384, 4, 16, 24, seed=5)["pairAttention1"]
    s = S.Stream(12)
    pair = s.normal(n * n * c).reshape(n, n, c)
    mask = np.ones((n, n), np.float32)
    mask[-4:, :] = 0
    mask[:, -4:] = 0
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af3_grid(dw, w)
    # stock AF3 keeps the untransposed bias for the ending node: the library's swap flag
    # transposes relative to the logical (transposed) rows, so it is set when the dialect is not
    lib_swap = transpose and not swap
    out, _, _ = _run(ctx, pair, mask, ws, 4, transpose, capi.LF_BIAS_NORMALIZED_INPUT,
                     fast_variance=True, swap_bias=lib_swap)
    ref = ops.grid_self_attention_af3(pair, mask, w, transpose, swap_transposed_bias=swap)
    H.assert_close(out, ref, label=f"af3 grid {transpose} {swap}")


def test_af3_single_attention(ctx):
    from localfold_amd import capi, device as D
    n, cz, cs = 40, 128, 384
    pw = S.synthetic_pairformer_weights(cz, cs, 4, 16, 24, seed=8)
    s = S.Stream(3)
    pair = s.normal(n * n * cz).reshape(n, n, cz)
    single = s.normal(n * cs).reshape(n, cs)
    seq_mask = np.ones(n, np.float32)
    seq_mask[-5:] = 0
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af3_single(dw, pw["singleAttention"], pw["singlePairLogitsNormScale"],
                                        pw["singlePairLogitsNormOffset"], pw["singlePairLogitsProjection"])
    out, _, _ = _run(ctx, single[None], seq_mask[None], ws, 16, False, capi.LF_BIAS_SEPARATE, pair,
                     head_dim=24, fast_variance=True)
    src = ops.layer_norm(pair, pw["singlePairLogitsNormScale"], pw["singlePairLogitsNormOffset"], fast_variance=True)
    logits = np.asarray(ops.linear(src, pw["singlePairLogitsProjection"]), np.float64).transpose(2, 0, 1)
    ref = ops.single_attention_af3(single, logits.astype(np.float32), seq_mask, pw["singleAttention"])
    H.assert_close(out[0], ref, label="af3 single")


def test_fully_masked_row_is_finite(ctx, blockw):
    from localfold_amd import capi, device as D
    n = 20
    act = S.synthetic_activations(1, n, 256, 128, seed=2)
    mask = np.ones((n, n), np.float32)
    mask[3, :] = 0          # every key of batch row 3 masked: uniform softmax (logits clamp at -1e8)
    tw = blockw["triangleAttentionStarting"]
    dw = D.DeviceWeights(ctx.device)
    ws = D.attention_weights_af2(dw, tw["attention"], tw["pairBias"])
    out, _, _ = _run(ctx, act["pair"], mask, ws, 4, False, capi.LF_BIAS_NORMALIZED_INPUT)
    ref = ops.attention_af2(act["pair"], mask, tw["attention"], 4, False, dict(tw["pairBias"], source="normalized-input"))
    assert np.isfinite(out).all()
    H.assert_close(out, ref, label="masked row")


def test_config3_full_size_sampled(ctx):
    """The triangle-attention workload: N=512, c_z=128, 4x32 heads, fp16 pair ~N(0,1), fp16 weights, last 26
    residues masked; starting then ending node, checked on 3 batch rows each."""
    import torch
    from localfold_amd import capi, device as D
    n, c = 512, 128
    s = S.Stream(33)
    pair = s.normal(n * n * c).reshape(n, n, c)
    mask = np.ones((n, n), np.float32)
    mask[:, n - 26:] = 0
    mask[n - 26:, :] = 0
    for ending, seed in ((False, 41), (True, 42)):
        w = S.config3_attention_weights(c, 4, seed)
        rec = S.quantise_records(w["attention"], ["queryWeight", "keyWeight", "valueWeight", "gatingWeight",
                                                  "outputWeight"], "float16", False, 1)
        dw = D.DeviceWeights(ctx.device)
        ws = D.attention_weights_af2(dw, rec, w["pairBias"])
        out, pin, _ = _run(ctx, pair, mask, ws, 4, ending, capi.LF_BIAS_NORMALIZED_INPUT, act_dt=torch.float16)
        rows = [0, 255, n - 1]
        ref = ops.attention_af2(pin, mask, H.decoded(rec), 4, ending, dict(w["pairBias"], source="normalized-input"),
                                batch_rows=rows)
        got = out.transpose(1, 0, 2)[rows] if ending else out[rows]
        H.assert_close(got, ref, label=f"config3 ending={ending}")
