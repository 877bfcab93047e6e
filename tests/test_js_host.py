"""The Node host (localfold_amd/js): CPU checks here, GPU parity through the JS classes on the
reference's fixture format and oracle cases (written to a temp directory by this test)."""
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import ops
from tests import helpers as H

ROOT = Path(__file__).resolve().parent.parent
JS = ROOT / "localfold_amd" / "js"
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _run_node(script, arg, timeout=240):
    r = subprocess.run([NODE, str(JS / "test" / script), str(arg)], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    print(r.stderr[-3000:])
    return r


def test_js_cpu_suite(tmp_path):
    if not (ROOT / "localfold_amd" / "lib" / "localfold_napi.node").exists():
        pytest.skip("addon not built")
    cases = [{"seed": s, "values": S.uniform_stream(s, 300).tolist()} for s in (0, 7, 1000 + 384, 0xFFFFFFFF)]
    p = tmp_path / "gen.json"
    p.write_text(json.dumps(cases))
    r = _run_node("cpu.test.js", p)
    assert r.returncode == 0 and "FAIL" not in r.stdout


def _write_fixture_dir(name, out: Path):
    f = H.load_fixture(name)
    d = out / name
    d.mkdir()
    tensors = {}
    for key in ["z", "mask", "expected"] + list(f["weights"].keys()):
        arr = f[key] if key in ("z", "mask", "expected") else f["weights"][key]
        np.asarray(arr, "<f4").tofile(d / f"{key}.f32.bin")
        tensors[key] = {"file": f"{key}.f32.bin", "shape": list(np.shape(arr)), "dtype": "float32"}
    meta = f["meta"]
    (d / "manifest.json").write_text(json.dumps({"formatVersion": 1, "operator": meta["operator"], "source": meta["source"],
                                                 "shape": meta["shape"], "epsilon": meta["epsilon"], "tensors": tensors}))
    return f


@pytest.mark.gpu
def test_js_gpu_suite(tmp_path):
    cases = {"fixtures": H.FIXTURES}
    for name in H.FIXTURES:
        f = _write_fixture_dir(name, tmp_path)
    # incoming on the a3m capture, expected from the oracle
    f = H.load_fixture("af2_a3m_model1_59")
    ops.tri_mult_af2(f["z"], f["mask"], f["weights"], "incoming").astype("<f4").tofile(tmp_path / "incoming.expected.f32.bin")
    cases["incoming"] = {"fixture": "af2_a3m_model1_59", "expected": "incoming.expected.f32.bin"}

    w = S.synthetic_block_weights(c_m=256, c_z=128, c_outer=32, heads_msa=8, heads_pair=4, tri_hidden=128,
                                  msa_hidden=1024, pair_hidden=512, seed=1)
    act = S.synthetic_activations(3, 30, 256, 128, seed=5)
    en = w["triangleAttentionEnding"]
    for k, v in en["attention"].items():
        np.asarray(v, "<f4").tofile(tmp_path / f"attention.{k}.f32.bin")
    np.asarray(en["pairBias"]["projectionWeight"], "<f4").tofile(tmp_path / "attention.pairProjection.f32.bin")
    np.asarray(act["pair"], "<f4").tofile(tmp_path / "attention.act.f32.bin")
    np.asarray(act["pairMask"], "<f4").tofile(tmp_path / "attention.mask.f32.bin")
    ref = ops.attention_af2(act["pair"], act["pairMask"], en["attention"], 4, True,
                            dict(en["pairBias"], source="normalized-input"))
    np.asarray(ref, "<f4").tofile(tmp_path / "attention.expected.f32.bin")
    cases["attention"] = {"batch": 30, "queries": 30, "channels": 128, "heads": 4, "transpose": True,
                          "names": list(en["attention"].keys())}

    tw = w["pairTransition"]
    for k, v in tw.items():
        np.asarray(v, "<f4").tofile(tmp_path / f"transition.{k}.f32.bin")
    np.asarray(act["pair"], "<f4").tofile(tmp_path / "transition.act.f32.bin")
    np.asarray(ops.transition_af2(act["pair"], tw), "<f4").tofile(tmp_path / "transition.expected.f32.bin")
    cases["transition"] = {"rows": 900, "channels": 128, "hidden": 512, "names": list(tw.keys())}

    ow = w["outerProductMean"]
    for k, v in ow.items():
        np.asarray(v, "<f4").tofile(tmp_path / f"opm.{k}.f32.bin")
    np.asarray(act["msa"], "<f4").tofile(tmp_path / "opm.act.f32.bin")
    np.asarray(act["msaMask"], "<f4").tofile(tmp_path / "opm.mask.f32.bin")
    np.asarray(ops.outer_product_mean_af2(act["msa"], act["msaMask"], ow), "<f4").tofile(tmp_path / "opm.expected.f32.bin")
    cases["opm"] = {"sequences": 3, "length": 30, "cM": 256, "cOuter": 32, "cZ": 128, "names": list(ow.keys())}

    (tmp_path / "cases.json").write_text(json.dumps(cases))
    r = _run_node("gpu.test.js", tmp_path)
    assert r.returncode == 0 and "FAIL" not in r.stdout
