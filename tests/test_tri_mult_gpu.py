"""Triangle multiplication on the GPU through the C ABI, against the oracle and the
reference's committed fixtures (test/triangle-multiplication-outgoing.gpu.test.js:31-69,
test/evoformer-triangle-incoming.gpu.test.js:36-85)."""
import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import ops
from tests import helpers as H

pytestmark = pytest.mark.gpu


def _run(ctx, z, mask, w, direction="outgoing", dialect=0, act=None, accumulate=False, divide=False):
    import torch
    from localfold_amd import device as D
    act = act or torch.float32
    dw = D.DeviceWeights(ctx.device)
    ws = D.tri_mult_weights(dw, w, dialect)
    zt = torch.as_tensor(z).to(ctx.device).to(act)
    mt = torch.as_tensor(np.asarray(mask, np.float32)).to(ctx.device)
    out = D.tri_mult(ctx, zt, mt, ws, direction, dialect, accumulate=accumulate, divide_by_length=divide)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), zt.float().cpu().numpy()


@pytest.mark.parametrize("name", H.FIXTURES)
def test_fixture_outgoing(ctx, name):
    f = H.load_fixture(name)
    out, _ = _run(ctx, f["z"], f["mask"], f["weights"])
    m = H.metrics(out, f["expected"])
    print(name, m)
    # the reference's f16 bounds on the same fixtures (mean < 1e-3, max < 1e-2)
    assert m["meanAbsoluteError"] < 1e-3 and m["maxAbsoluteError"] < 1e-2, m


@pytest.mark.parametrize("name", H.FIXTURES)
def test_fixture_incoming_vs_oracle(ctx, name):
    f = H.load_fixture(name)
    out, _ = _run(ctx, f["z"], f["mask"], f["weights"], "incoming")
    ref = ops.tri_mult_af2(f["z"], f["mask"], f["weights"], "incoming", f["meta"]["epsilon"])
    m = H.metrics(out, ref)
    assert m["meanAbsoluteError"] < 1e-3 and m["maxAbsoluteError"] < 1e-2, m


@pytest.mark.parametrize("n,cz,ch,seed", [(3, 4, 5, 42), (37, 64, 32, 5), (37, 128, 128, 3), (64, 128, 128, 7),
                                         (130, 128, 128, 11), (24, 256, 128, 17), (20, 256, 256, 19),
                                         (12, 128, 128, 23)])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_deterministic_input(ctx, n, cz, ch, seed, direction):
    inp = S.deterministic_triangle_input(n, cz, ch, seed)
    out, _ = _run(ctx, inp["z"], inp["mask"], inp["weights"], direction)
    ref = ops.tri_mult_af2(inp["z"], inp["mask"], inp["weights"], direction)
    H.assert_close(out, ref, label=f"{n}/{cz}/{ch}/{direction}")


@pytest.mark.parametrize("dtype,per_channel", [("float16", False), ("int8", False), ("int5", False),
                                               ("int8", True), ("int5", True)])
@pytest.mark.parametrize("act", ["float32", "bfloat16", "float16"])
def test_quantised_weights_and_activation_dtypes(ctx, dtype, per_channel, act):
    import torch
    inp = S.deterministic_triangle_input(48, 128, 128, 3)
    rec, dec = H.quantise_weights(inp["weights"], H.TRI_MATS, dtype, per_channel, 0)
    tdt = getattr(torch, act)
    for direction in ("outgoing", "incoming"):
        out, zin = _run(ctx, inp["z"], inp["mask"], rec, direction, act=tdt)
        ref = ops.tri_mult_af2(zin, inp["mask"], dec, direction)
        # the update is stored in the activation dtype: add its rounding to the bound
        H.assert_close(out, ref, max_abs=2e-2, label=f"{dtype}/{per_channel}/{act}/{direction}")


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("divide", [False, True])
@pytest.mark.parametrize("n", [256, 64, 40, 12])
def test_af3_dialect(ctx, direction, divide, n):
    """n = 256, 64 and 40: the resident kernels (interleaved tensors split in LDS), at 256 and
    64 with the direct-to-LDS contraction (N a multiple of 64: 128-row tiles at 256, 96-row
    tiles at 64, as at 384); n = 12: the chunked kernels (the interleaved columns decoded
    weight by weight)."""
    c = 128
    w = H.af3_tri_weights(c, 21)
    s = S.Stream(77)
    z = s.normal(n * n * c).reshape(n, n, c)
    mask = np.ones((n, n), np.float32)
    mask[-4:, :] = 0
    mask[:, -4:] = 0
    out, _ = _run(ctx, z, mask, w, direction, dialect=1, divide=divide)
    assert out.shape == (n, n, c)
    ref = ops.tri_mult_af3(z, mask, w, direction, divide_by_length=divide)
    H.assert_close(out, ref, label=f"af3/{direction}/{divide}")


def test_af3_dialect_large_contraction_tiles(ctx):
    """AF3 at N = 768 (incoming, divided by the length, bf16 pair): the split projection of
    the interleaved tensors feeding the 256 x 256-tile contraction; against the oracle."""
    import torch
    n, c = 768, 128
    w = H.af3_tri_weights(c, 23)
    z = S.Stream(79).normal(n * n * c).reshape(n, n, c)
    mask = np.ones((n, n), np.float32)
    mask[-8:, :] = 0
    mask[:, -8:] = 0
    out, zin = _run(ctx, z, mask, w, "incoming", dialect=1, act=torch.bfloat16, divide=True)
    ref = ops.tri_mult_af3(zin, mask, w, "incoming", divide_by_length=True)
    H.assert_close(out, ref, max_abs=2e-2, label="af3/768/incoming")


def test_accumulate_in_place(ctx):
    import torch
    from localfold_amd import device as D
    inp = S.deterministic_triangle_input(33, 128, 128, 9)
    dw = D.DeviceWeights(ctx.device)
    ws = D.tri_mult_weights(dw, inp["weights"])
    z = torch.as_tensor(inp["z"]).to(ctx.device)
    m = torch.as_tensor(inp["mask"]).to(ctx.device)
    D.tri_mult(ctx, z, m, ws, "outgoing", out=z, accumulate=True)
    torch.cuda.synchronize()
    ref = inp["z"].astype(np.float64) + ops.tri_mult_af2(inp["z"], inp["mask"], inp["weights"], "outgoing")
    H.assert_close(z.cpu().numpy(), ref)


def test_config2_full_size(ctx):
    """The headline workload at full size: N=384, int5 per-output-channel weights, bf16 pair,
    last 16 residues masked; outgoing then incoming, each against the oracle."""
    import torch
    c2 = H.config2_inputs()
    out1, zin = _run(ctx, c2["z"], c2["mask"], c2["rec_out"], "outgoing", act=torch.bfloat16)
    ref1 = ops.tri_mult_af2(zin, c2["mask"], c2["dec_out"], "outgoing")
    H.assert_close(out1, ref1, label="config2/outgoing")
    out2, zin2 = _run(ctx, c2["z"], c2["mask"], c2["rec_in"], "incoming", act=torch.bfloat16)
    ref2 = ops.tri_mult_af2(zin2, c2["mask"], c2["dec_in"], "incoming")
    H.assert_close(out2, ref2, label="config2/incoming")
    assert np.isfinite(out1).all() and np.isfinite(out2).all()


@pytest.mark.parametrize("n,direction", [(768, "outgoing"), (768, "incoming"), (960, "outgoing")])
def test_large_contraction_tiles(ctx, n, direction):
    """N = 768 and 960: the contraction runs on 256 x 256 tiles (8 waves of 128 x 64); at 960
    the last tile row and column are clamped (64 rows past N); against the oracle."""
    import torch
    inp = S.deterministic_triangle_input(n, 128, 128, 29)
    out, zin = _run(ctx, inp["z"], inp["mask"], inp["weights"], direction, act=torch.bfloat16)
    ref = ops.tri_mult_af2(zin, inp["mask"], inp["weights"], direction)
    H.assert_close(out, ref, label=f"{n}/{direction}")


def test_invalid_shapes_rejected(ctx):
    import torch
    from localfold_amd import capi, device as D
    inp = S.deterministic_triangle_input(4, 8, 8, 1)
    dw = D.DeviceWeights(ctx.device)
    ws = D.tri_mult_weights(dw, inp["weights"])
    z = torch.zeros(4, 4, 9, device=ctx.device)       # cZ 9 against weights of 8
    m = torch.ones(4, 4, device=ctx.device)
    with pytest.raises(capi.LocalfoldError, match="inputs"):
        D.tri_mult(ctx, z, m, ws)


def _tri_records(w, dtype, layout):
    """The six matrices as `dtype` records stored (out,in) or, transposed, (in,out); returns
    (records, the (out,in) float32 matrices the oracle takes)."""
    recs, dec = dict(w), dict(w)
    for name in H.TRI_MATS:
        m = np.asarray(w[name], np.float32)
        stored = m if layout == "out_in" else np.ascontiguousarray(m.T)
        rec = S.make_record(stored, dtype)
        rec["layout"] = layout
        recs[name] = rec
        d = H.decoded({"x": rec})["x"]
        dec[name] = d if layout == "out_in" else np.ascontiguousarray(d.T)
    return recs, dec


def _shift_codes(dw, wt, rec, offset):
    """Rebinds wt.data to a copy of the record's stored bytes that starts `offset` bytes past
    an aligned address, so that the kernels cannot load the weights in aligned runs."""
    import torch
    dt = rec["dtype"]
    host = (np.asarray(rec["data"], np.float32) if dt == "float32" else
            np.asarray(rec["data"], np.float32).astype(np.float16) if dt == "float16" else np.asarray(rec["data"]))
    raw = np.ascontiguousarray(host).view(np.uint8).reshape(-1)
    buf = torch.zeros(raw.size + 64, dtype=torch.uint8, device=dw.device)
    buf[offset:offset + raw.size] = torch.from_numpy(raw.copy()).to(dw.device)
    dw.keep.append(buf)
    wt.data = buf.data_ptr() + offset


@pytest.mark.parametrize("dtype", ["float32", "float16", "int8", "int5"])
@pytest.mark.parametrize("mode", ["in_out", "misaligned"])
def test_weight_storage_paths(ctx, dtype, mode):
    """The kernels decode the stored weights themselves, three ways: runs of 8 along k
    ((out,in) storage, the other tests), runs along n ((in,out) storage: 8 columns per load,
    written down the LDS rows), and weight by weight when the codes' address is not aligned
    for the run loads (here 4 bytes past alignment: f32 and f16 runs need 16, int8 8; int5
    1 byte past, against 4)."""
    import torch
    from localfold_amd import device as D
    inp = S.deterministic_triangle_input(40, 128, 128, 13)
    layout = "in_out" if mode == "in_out" else "out_in"
    recs, dec = _tri_records(inp["weights"], dtype, layout)
    dw = D.DeviceWeights(ctx.device)
    ws = D.tri_mult_weights(dw, recs)
    if mode == "misaligned":
        off = 1 if dtype == "int5" else 4
        for field, name in zip(("ap", "ag", "bp", "bg", "wz", "wg"), H.TRI_MATS):
            _shift_codes(dw, getattr(ws, field), recs[name], off)
    zt = torch.as_tensor(inp["z"]).to(ctx.device)
    mt = torch.as_tensor(inp["mask"]).to(ctx.device)
    for direction in ("outgoing", "incoming"):
        out = D.tri_mult(ctx, zt, mt, ws, direction)
        torch.cuda.synchronize()
        ref = ops.tri_mult_af2(inp["z"], inp["mask"], dec, direction)
        H.assert_close(out.cpu().numpy(), ref, label=f"{dtype}/{mode}/{direction}")


def test_weights_from_a_temporary_upload_stay_valid(ctx):
    """A weight struct built from a DeviceWeights nobody else holds keeps those device buffers
    alive (the struct points into them)."""
    import gc
    import torch
    from localfold_amd import device as D
    inp = S.deterministic_triangle_input(40, 128, 128, 9)
    ws = D.tri_mult_weights(D.DeviceWeights(ctx.device), inp["weights"])
    gc.collect()
    # fresh allocations that would reuse freed weight memory
    junk = [torch.full((1 << 20,), float("nan"), device=ctx.device) for _ in range(8)]
    z = torch.as_tensor(inp["z"]).to(ctx.device)
    out = D.tri_mult(ctx, z, torch.as_tensor(np.asarray(inp["mask"], np.float32)).to(ctx.device), ws, "outgoing")
    torch.cuda.synchronize()
    del junk
    H.assert_close(out.cpu().numpy(), ops.tri_mult_af2(inp["z"], inp["mask"], inp["weights"], "outgoing"),
                   label="temporary DeviceWeights")
