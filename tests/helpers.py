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


# ---------------------------------------------------------------------------------------
# Weight bundles in the reference's manifest + shard layout (shared/weights/dtype.js)
# ---------------------------------------------------------------------------------------

def write_bundle(dirpath, tensors: dict, sections: dict = None, shard: str = "weights.bin") -> str:
    """Writes `tensors` (name -> record as synthetic.make_record returns) to one shard and a
    manifest.json beside it: every tensor starts on a 4-byte boundary; int8 codes are followed
    by their fp16 scales (2-byte aligned, absolute scaleOffset); packed codes (slack byte
    included) by fp16 scales, then fp16 zeros.  Returns the manifest path."""
    import json
    import os
    buf = bytearray()
    table = {}

    def align(a):
        buf.extend(b"\0" * ((-len(buf)) % a))

    for name, rec in tensors.items():
        align(4)
        entry = {"file": shard, "shape": list(rec["shape"]), "dtype": rec["dtype"], "byteOffset": len(buf)}
        dt = rec["dtype"]
        if dt == "float32":
            buf += np.asarray(rec["data"], "<f4").tobytes()
        elif dt == "float16":
            buf += np.asarray(rec["data"], np.float32).astype("<f2").tobytes()
        else:
            buf += np.asarray(rec["data"]).tobytes()
            align(2)
            entry["block"] = int(rec["block"])
            entry["scaleOffset"] = len(buf)
            buf += np.asarray(rec["scales"], np.float16).astype("<f2").tobytes()
            if dt != "int8":
                entry["zeroOffset"] = len(buf)
                buf += np.asarray(rec["zeros"], np.float16).astype("<f2").tobytes()
        table[name] = entry
    os.makedirs(dirpath, exist_ok=True)
    with open(os.path.join(dirpath, shard), "wb") as f:
        f.write(bytes(buf))
    manifest = {"formatVersion": 1, "tensors": table}
    manifest.update(sections or {})
    path = os.path.join(dirpath, "manifest.json")
    with open(path, "w") as f:
        json.dump(manifest, f)
    return path


def af2_stack_bundle_tensors(blocks_w: list, dtype: str, block: int = None):
    """The evoformerStack section of an AF2 bundle (stacked haiku: one tensor per parameter,
    block index leading, AlphaFold's parameter shapes) for the per-block weight dicts of
    synthetic.synthetic_block_weights.  Matrices are quantised to `dtype` as one stacked
    tensor (flat groups); vectors stay float32.  Returns (tensors, evoformerStack section,
    the stacked float arrays by tensor name)."""
    from localfold_amd import synthetic as S

    def attn(key, heads):
        def get(w):
            a = w[key]["attention"]
            c = a["queryWeight"].shape[0]
            hd = a["queryWeight"].shape[1]
            d = hd // heads
            return {
                ("attention", "query_w"): a["queryWeight"].reshape(c, heads, d),
                ("attention", "key_w"): a["keyWeight"].reshape(c, heads, d),
                ("attention", "value_w"): a["valueWeight"].reshape(c, heads, d),
                ("attention", "gating_w"): a["gatingWeight"].reshape(c, heads, d),
                ("attention", "gating_b"): a["gatingBias"].reshape(heads, d),
                ("attention", "output_w"): a["outputWeight"].reshape(heads, d, -1),
                ("attention", "output_b"): a["outputBias"],
                ("query_norm", "scale"): a["queryNormScale"],
                ("query_norm", "offset"): a["queryNormOffset"],
            }
        return get

    def tri(key):
        def get(w):
            t = w[key]
            return {
                ("layer_norm_input", "scale"): t["layerNormInWeight"], ("layer_norm_input", "offset"): t["layerNormInBias"],
                ("center_layer_norm", "scale"): t["layerNormOutWeight"], ("center_layer_norm", "offset"): t["layerNormOutBias"],
                ("left_projection", "weights"): t["linearAPWeight"].T, ("left_projection", "bias"): t["linearAPBias"],
                ("left_gate", "weights"): t["linearAGWeight"].T, ("left_gate", "bias"): t["linearAGBias"],
                ("right_projection", "weights"): t["linearBPWeight"].T, ("right_projection", "bias"): t["linearBPBias"],
                ("right_gate", "weights"): t["linearBGWeight"].T, ("right_gate", "bias"): t["linearBGBias"],
                ("output_projection", "weights"): t["linearZWeight"].T, ("output_projection", "bias"): t["linearZBias"],
                ("gating_linear", "weights"): t["linearGWeight"].T, ("gating_linear", "bias"): t["linearGBias"],
            }
        return get

    def trans(key):
        def get(w):
            t = w[key]
            return {("input_layer_norm", "scale"): t["layerNormScale"], ("input_layer_norm", "offset"): t["layerNormOffset"],
                    ("transition1", "weights"): t["firstWeight"], ("transition1", "bias"): t["firstBias"],
                    ("transition2", "weights"): t["secondWeight"], ("transition2", "bias"): t["secondBias"]}
        return get

    def opm(w):
        o = w["outerProductMean"]
        co = o["leftWeight"].shape[1]
        return {("layer_norm_input", "scale"): o["layerNormScale"], ("layer_norm_input", "offset"): o["layerNormOffset"],
                ("left_projection", "weights"): o["leftWeight"], ("left_projection", "bias"): o["leftBias"],
                ("right_projection", "weights"): o["rightWeight"], ("right_projection", "bias"): o["rightBias"],
                (None, "output_w"): o["outputWeight"].reshape(co, co, -1), (None, "output_b"): o["outputBias"]}

    w0 = blocks_w[0]
    roots = [
        ("msa_row_attention_with_pair_bias", attn("msaRowAttention", w0["msaRowAttention"]["heads"])),
        ("msa_column_attention", attn("msaColumnAttention", w0["msaColumnAttention"]["heads"])),
        ("triangle_attention_starting_node", attn("triangleAttentionStarting", w0["triangleAttentionStarting"]["heads"])),
        ("triangle_attention_ending_node", attn("triangleAttentionEnding", w0["triangleAttentionEnding"]["heads"])),
        ("triangle_multiplication_outgoing", tri("triangleMultiplicationOutgoing")),
        ("triangle_multiplication_incoming", tri("triangleMultiplicationIncoming")),
        ("msa_transition", trans("msaTransition")),
        ("pair_transition", trans("pairTransition")),
        ("outer_product_mean", opm),
    ]
    extra = lambda w: {
        ("msa_row_attention_with_pair_bias", "feat_2d_weights"): w["msaRowAttention"]["pairBias"]["projectionWeight"],
        ("msa_row_attention_with_pair_bias/feat_2d_norm", "scale"): w["msaRowAttention"]["pairBias"]["layerNormScale"],
        ("msa_row_attention_with_pair_bias/feat_2d_norm", "offset"): w["msaRowAttention"]["pairBias"]["layerNormOffset"],
        ("triangle_attention_starting_node", "feat_2d_weights"): w["triangleAttentionStarting"]["pairBias"]["projectionWeight"],
        ("triangle_attention_ending_node", "feat_2d_weights"): w["triangleAttentionEnding"]["pairBias"]["projectionWeight"],
    }
    per_block = []
    for w in blocks_w:
        entries = {}
        for root, get in roots:
            for (sub, key), v in get(w).items():
                entries[(root if sub is None else f"{root}/{sub}", key)] = np.asarray(v, np.float32)
        entries.update({k: np.asarray(v, np.float32) for k, v in extra(w).items()})
        per_block.append(entries)
    tensors, parameters, stacked = {}, {}, {}
    for i, key in enumerate(per_block[0]):
        name = f"stack_haiku_{i:04d}"
        arr = np.stack([b[key] for b in per_block])
        stacked[name] = arr
        matrix = arr.ndim >= 3 and key[1] not in ("gating_b",)
        tensors[name] = S.make_record(arr, dtype if matrix else "float32", block=block)
        parameters.setdefault(key[0], {})[key[1]] = name
    section = {"evoformerStack": {"blocks": len(blocks_w), "parameterFormat": "stacked-haiku",
                                  "parameters": parameters}}
    return tensors, section, stacked
