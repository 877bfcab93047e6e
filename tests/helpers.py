"""Shared test helpers: fixtures, synthetic inputs, quantised-weight builders, metrics."""
import json
from pathlib import Path

import numpy as np

from localfold_amd import synthetic as S
from oracle import codec, ops

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


def decoded(recs: dict) -> dict:
    """Oracle view of a weight dict: every codec record decoded to float32."""
    return {k: (codec.decode(v) if isinstance(v, dict) and "dtype" in v else v) for k, v in recs.items()}


def quantise_weights(w: dict, names, dtype: str, per_channel: bool, out_axis: int):
    """Returns (records for the kernels, decoded float32 arrays for the oracle)."""
    recs = S.quantise_records(w, names, dtype, per_channel, out_axis)
    return recs, decoded(recs)


TRI_MATS = S.TRI_MATS
TRI3_MATS = S.TRI3_MATS
af3_tri_weights = S.af3_tri_weights


def config2_inputs(*a, **k):
    c2 = S.config2_inputs(*a, **k)
    c2["dec_out"] = decoded(c2["rec_out"])
    c2["dec_in"] = decoded(c2["rec_in"])
    return c2
