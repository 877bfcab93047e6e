"""Shared test helpers: fixtures, synthetic inputs, quantised-weight builders, metrics."""
import json
from pathlib import Path

import numpy as np

from oracle import codec, ops, prng

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURES = ["openfold_triangle_small", "af2_single_short9", "af2_single_model1_59", "af2_a3m_model1_59"]

# north_star tolerance on pair / MSA activations per op or block
MAX_ABS = 2e-2
REL_FRO = 5e-3


def load_fixture(name):
    f = np.load(GOLDEN / f"{name}.npz")
    meta = json.loads(str(f["meta"]))
    w = {k: f[k] for k in f.files if k not in ("z", "mask", "expected", "meta")}
    return {"z": f["z"], "mask": f["mask"], "expected": f["expected"], "weights": w, "meta": meta}


def metrics(actual, expected):
    return ops.error_metrics(actual, expected)


def assert_close(actual, expected, max_abs=MAX_ABS, rel_fro=REL_FRO, label=""):
    m = metrics(actual, expected)
    assert m["maxAbsoluteError"] <= max_abs and m["relativeFrobenius"] <= rel_fro, f"{label}: {m}"
    return m


def quantise_weights(w: dict, names, dtype: str, per_channel: bool, out_axis: int):
    """Returns (records for the kernels, decoded float32 arrays for the oracle)."""
    recs, dec = dict(w), dict(w)
    for name in names:
        if dtype == "float32":
            continue
        if dtype in ("float16",):
            rec = codec.make_record(w[name], "float16")
        elif per_channel:
            rec = codec.make_record(w[name], dtype, channel_axis=out_axis)
        else:
            rec = codec.make_record(w[name], dtype)
        recs[name] = rec
        dec[name] = codec.decode(rec)
    return recs, dec


TRI_MATS = ["linearAPWeight", "linearAGWeight", "linearBPWeight", "linearBGWeight", "linearZWeight", "linearGWeight"]
TRI3_MATS = ["projection", "gate", "outputProjection", "gatingLinear"]


def af3_tri_weights(c, seed):
    s = prng.Stream(seed)
    r = 1.0 / np.sqrt(c)
    return {"leftNormInputScale": s.values(c, 0.2, 1), "leftNormInputOffset": s.values(c, 0.1),
            "projection": s.normal(c * 2 * c, r).reshape(c, 2 * c), "gate": s.normal(c * 2 * c, r).reshape(c, 2 * c),
            "centerNormScale": s.values(c, 0.2, 1), "centerNormOffset": s.values(c, 0.1),
            "outputProjection": s.normal(c * c, r).reshape(c, c), "gatingLinear": s.normal(c * c, r).reshape(c, c)}


def config2_inputs(n=384, c=128, seed=2, masked_tail=16):
    """z ~N(0,1), weights N(0,1/fan_in) masters quantised int5 per output channel,
    mask ones except the last `masked_tail` residues (rows and columns)."""
    s = prng.Stream(seed)
    z = s.normal(n * n * c).reshape(n, n, c)
    mask = np.ones((n, n), np.float32)
    if masked_tail:
        mask[n - masked_tail:, :] = 0
        mask[:, n - masked_tail:] = 0

    def tri(seed_off):
        t = prng.Stream(seed + 100 + seed_off)
        rz = 1.0 / np.sqrt(c)
        return {"layerNormInWeight": t.values(c, 0.2, 1), "layerNormInBias": t.values(c, 0.1),
                "linearAPWeight": t.normal(c * c, rz).reshape(c, c), "linearAPBias": t.values(c, 0.03),
                "linearAGWeight": t.normal(c * c, rz).reshape(c, c), "linearAGBias": t.values(c, 0.03, 1),
                "linearBPWeight": t.normal(c * c, rz).reshape(c, c), "linearBPBias": t.values(c, 0.03),
                "linearBGWeight": t.normal(c * c, rz).reshape(c, c), "linearBGBias": t.values(c, 0.03, 1),
                "layerNormOutWeight": t.values(c, 0.2, 1), "layerNormOutBias": t.values(c, 0.1),
                "linearZWeight": t.normal(c * c, rz).reshape(c, c), "linearZBias": t.values(c, 0.03),
                "linearGWeight": t.normal(c * c, rz).reshape(c, c), "linearGBias": t.values(c, 0.03, 1)}
    w_out, w_in = tri(0), tri(1)
    rec_out, dec_out = quantise_weights(w_out, TRI_MATS, "int5", True, 0)
    rec_in, dec_in = quantise_weights(w_in, TRI_MATS, "int5", True, 0)
    return {"z": z, "mask": mask, "rec_out": rec_out, "dec_out": dec_out, "rec_in": rec_in, "dec_in": dec_in}
