"""The weight-bundle reader (localfold_amd/bundle.py) on bundles written in the reference's
manifest + shard layout, and on the reference's own committed fixture manifests when the
reference checkout is present."""
import json
import os

import numpy as np
import pytest

from localfold_amd import bundle as B
from localfold_amd import synthetic as S
from oracle import codec
from tests import helpers as H

REF_FIXTURES = "/root/reference/test/fixtures"


def _small_blocks(n=2):
    return [S.synthetic_block_weights(c_m=64, c_z=32, c_outer=8, heads_msa=4, heads_pair=2, tri_hidden=32,
                                      msa_hidden=256, pair_hidden=128, seed=10 + b) for b in range(n)]


@pytest.mark.parametrize("dtype,block", [("int8", 64), ("int5", 32), ("float32", None)])
def test_af2_stack_round_trip(tmp_path, dtype, block):
    """Every matrix of every block comes back as the stored codes of its block's slice (decoded
    values equal the stacked tensor's decode at those indices); vectors come back exactly."""
    blocks_w = _small_blocks()
    tensors, section, stacked = H.af2_stack_bundle_tensors(blocks_w, dtype, block)
    path = H.write_bundle(str(tmp_path), tensors, section)
    store = B.FileTensorStore.open(path)
    got = B.af2_main_stack_weights(store, msa_channels=64, pair_channels=32)
    assert len(got) == 2
    params = section["evoformerStack"]["parameters"]
    full = {name: codec.decode(rec).reshape(2, -1) for name, rec in tensors.items()}
    for b, w in enumerate(got):
        # matrices: the record decodes to the stacked tensor's block-b values
        checks = [
            (w["msaRowAttention"]["attention"]["queryWeight"], params["msa_row_attention_with_pair_bias/attention"]["query_w"]),
            (w["msaColumnAttention"]["attention"]["outputWeight"], params["msa_column_attention/attention"]["output_w"]),
            (w["msaTransition"]["secondWeight"], params["msa_transition/transition2"]["weights"]),
            (w["outerProductMean"]["outputWeight"], params["outer_product_mean"]["output_w"]),
            (w["triangleMultiplicationIncoming"]["linearZWeight"], params["triangle_multiplication_incoming/output_projection"]["weights"]),
            (w["triangleAttentionEnding"]["pairBias"]["projectionWeight"], params["triangle_attention_ending_node"]["feat_2d_weights"]),
            (w["msaRowAttention"]["pairBias"]["projectionWeight"], params["msa_row_attention_with_pair_bias"]["feat_2d_weights"]),
        ]
        for rec, name in checks:
            assert rec["layout"] == "in_out" and rec["dtype"] == tensors[name]["dtype"]
            np.testing.assert_array_equal(codec.decode(rec).reshape(-1), full[name][b], err_msg=name)
        # vectors
        np.testing.assert_array_equal(w["msaRowAttention"]["attention"]["gatingBias"],
                                      stacked[params["msa_row_attention_with_pair_bias/attention"]["gating_b"]][b].reshape(-1))
        np.testing.assert_array_equal(w["pairTransition"]["firstBias"],
                                      stacked[params["pair_transition/transition1"]["bias"]][b])
        assert w["msaRowAttention"]["heads"] == 4 and w["triangleAttentionStarting"]["heads"] == 2
        # the triangle projections are the transposes of the (out,in) dict entries
        tw = blocks_w[b]["triangleMultiplicationOutgoing"]
        rec = w["triangleMultiplicationOutgoing"]["linearAPWeight"]
        assert rec["shape"] == [32, 32]
        if dtype == "float32":
            np.testing.assert_array_equal(codec.decode(rec), tw["linearAPWeight"].T)


def test_values_decode_any_range(tmp_path):
    """values() decodes an arbitrary element range (not group-aligned) the way readTensorRange
    does: the same numbers as decoding the whole tensor and slicing."""
    vals = S.Stream(3).normal(1000).astype(np.float32)
    tensors = {"q8": S.make_record(vals, "int8", block=64), "q5": S.make_record(vals[:992], "int5", block=32),
               "f16": S.make_record(vals, "float16")}
    store = B.FileTensorStore.open(H.write_bundle(str(tmp_path), tensors))
    for name in tensors:
        whole = codec.decode(tensors[name]).reshape(-1)
        for first, count in [(0, 7), (37, 100), (64, 64), (900, len(whole) - 900)]:
            np.testing.assert_array_equal(store.values(name, first, count), whole[first:first + count])


def test_group_misaligned_record_is_refused(tmp_path):
    vals = S.Stream(4).normal(256).astype(np.float32)
    store = B.FileTensorStore.open(H.write_bundle(str(tmp_path), {"q": S.make_record(vals, "int8", block=64)}))
    with pytest.raises(ValueError, match="quantisation group"):
        store.record("q", 10, 64)


def test_manifest_errors(tmp_path):
    vals = S.Stream(5).normal(64).astype(np.float32)
    path = H.write_bundle(str(tmp_path), {"x": S.make_record(vals, "float32")})
    store = B.FileTensorStore.open(path)
    with pytest.raises(KeyError, match="manifest contains no tensor named y"):
        store.record("y")
    m = json.load(open(path))
    m["tensors"]["x"]["byteOffset"] = 1024
    json.dump(m, open(path, "w"))
    with pytest.raises(ValueError, match="points outside"):
        B.FileTensorStore.open(path).record("x")
    del m["tensors"]
    json.dump(m, open(path, "w"))
    with pytest.raises(ValueError, match="has no tensor table"):
        B.FileTensorStore.open(path)
    assert B.packed_bits("int5") == 5 and B.packed_bits("int8") is None and B.packed_bits("float16") is None


@pytest.mark.skipif(not os.path.isdir(REF_FIXTURES), reason="the reference checkout is not present")
@pytest.mark.parametrize("fixture,golden", [("openfold-triangle-small", "openfold_triangle_small"),
                                            ("alphafold-single-sequence/short-9", "af2_single_short9")])
def test_reference_fixture_manifests(fixture, golden):
    """The reference's committed fixture manifests read through the store give the tensors the
    committed golden files hold."""
    store = B.FileTensorStore.open(os.path.join(REF_FIXTURES, fixture, "manifest.json"))
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", golden + ".npz"))
    for name in ("z", "mask", "expected", "linearAPWeight", "layerNormOutBias"):
        np.testing.assert_array_equal(store.values(name).reshape(g[name].shape), g[name])
