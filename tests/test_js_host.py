"""The Node host (localfold_amd/js): CPU checks here, GPU parity through the JS classes on the
reference's fixture format and oracle cases (written to a temp directory by this test)."""
import json
import os
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
    fx = tmp_path / "fixtures"
    fx.mkdir()
    for name in H.FIXTURES:
        _write_fixture_dir(name, fx)
    r = subprocess.run([NODE, str(JS / "test" / "cpu.test.js"), str(p), str(fx)], capture_output=True, text=True,
                       timeout=240)
    print(r.stdout)
    print(r.stderr[-3000:])
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


def _dump_tree(node, out: Path, prefix: str):
    """JSON-able copy of a nested weight/input dict with arrays written as float32 files."""
    if isinstance(node, dict):
        return {k: _dump_tree(v, out, f"{prefix}.{k}") for k, v in node.items()}
    if isinstance(node, (list, tuple)):
        return [_dump_tree(v, out, f"{prefix}.{i}") for i, v in enumerate(node)]
    if isinstance(node, np.ndarray):
        np.ascontiguousarray(node, "<f4").tofile(out / f"{prefix}.f32.bin")
        return {"$f32": f"{prefix}.f32.bin"}
    if isinstance(node, (np.integer,)):
        return int(node)
    if isinstance(node, (np.floating,)):
        return float(node)
    return node


def test_js_f16_conversion_matches_numpy(tmp_path):
    """The JS host's f16 storage conversion (float32ToFloat16Bits) against numpy's float32 ->
    float16 cast (IEEE round to nearest, ties to even) on values over the whole f16 range,
    subnormals, overflow and exact ties included."""
    rng = np.random.default_rng(3)
    mant = rng.integers(0, 1 << 23, 60000, dtype=np.uint32)
    expo = rng.integers(100, 145, 60000, dtype=np.uint32)     # 2^-27 .. 2^17
    sign = rng.integers(0, 2, 60000, dtype=np.uint32) << 31
    vals = ((expo << 23) | mant | sign).view(np.float32)
    ties = (np.arange(1, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24)   # halfway cases
    vals = np.concatenate([vals, ties, ties * 1024, np.float32([65504, 65519.99, 65520, 1e-8, 0, -0.0])])
    src = tmp_path / "v.f32"
    vals.astype("<f4").tofile(src)
    code = ("const lf=require(process.argv[1]);const fs=require('fs');const b=fs.readFileSync(process.argv[2]);"
            "const v=new Float32Array(b.buffer.slice(b.byteOffset,b.byteOffset+b.byteLength));"
            "fs.writeFileSync(process.argv[3],Buffer.from(lf.float32ToFloat16Bits(v).buffer));")
    dst = tmp_path / "h.u16"
    r = subprocess.run([NODE, "-e", code, str(JS / "index.js"), str(src), str(dst)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.fromfile(dst, "<u2")
    with np.errstate(over="ignore"):   # values past 65520 overflow to infinity, as intended
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]


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

    # EvoformerBlockGpu (the reference test's input fields, test/evoformer-block.gpu.test.js:144-156)
    from oracle import blocks
    ew = S.synthetic_block_weights(c_m=256, c_z=128, c_outer=32, heads_msa=8, heads_pair=4, tri_hidden=128,
                                   msa_hidden=1024, pair_hidden=512, seed=4)
    ea = S.synthetic_activations(4, 21, 256, 128, seed=6)
    rm, rp = blocks.evoformer_block_af2(ea["msa"], ea["pair"], ea["msaMask"], ea["pairMask"], ew)
    ev = {"input": {"msa": ea["msa"], "pair": ea["pair"], "msaMask": ea["msaMask"], "pairMask": ea["pairMask"],
                    "sequences": 4, "length": 21, "cM": 256, "cZ": 128, "cOuter": 32, "triangleHidden": 128,
                    "weights": ew},
          "expectedMsa": rm, "expectedPair": rp}
    (tmp_path / "evoformer.json").write_text(json.dumps(_dump_tree(ev, tmp_path, "evo")))

    # ExtraMsaStackGpu: two extra-MSA blocks (webgpu/af2/evoformer/stack.js:249-330, input.blockWeights)
    xws = [S.synthetic_extra_msa_block_weights(c_m=64, c_z=32, c_outer=8, heads_msa=8, heads_pair=2, tri_hidden=32,
                                               msa_hidden=256, pair_hidden=128, seed=s_) for s_ in (31, 32)]
    xa = S.synthetic_activations(5, 14, 64, 32, seed=33)
    xm, xp = xa["msa"], xa["pair"]
    for xw in xws:
        xm, xp = blocks.extra_msa_block_af2(xm, xp, xa["msaMask"], xa["pairMask"], xw)
    ex = {"input": {"msa": xa["msa"], "pair": xa["pair"], "msaMask": xa["msaMask"], "pairMask": xa["pairMask"],
                    "sequences": 5, "length": 14, "cM": 64, "cZ": 32, "cOuter": 8, "triangleHidden": 32,
                    "blockWeights": xws},
          "expectedMsa": xm, "expectedPair": xp}
    xp2 = xa["pair"]
    for xw in xws:
        xp2 = blocks.evoformer_pair_block_af2(xa["msa"], xp2, xa["msaMask"], xa["pairMask"], xw)
    ex["expectedPairOnly"] = xp2
    (tmp_path / "extra.json").write_text(json.dumps(_dump_tree(ex, tmp_path, "ex")))

    # Af3PairformerStackGpu: two blocks
    n, cz, cs = 24, 128, 384
    pws = [S.synthetic_pairformer_weights(cz, cs, 4, 16, 24, seed=s_) for s_ in (21, 22)]
    st = S.Stream(23)
    pair0 = st.normal(n * n * cz).reshape(n, n, cz)
    single0 = st.normal(n * cs).reshape(n, cs)
    seq_mask = np.ones(n, np.float32)
    seq_mask[-3:] = 0
    pair_mask = np.outer(seq_mask, seq_mask).astype(np.float32)
    rp, rs = pair0, single0
    for pw in pws:
        rp, rs = blocks.pairformer_block_af3(rp, rs, pair_mask, seq_mask, pw, False, False)
    pf = {"state": {"pair": pair0, "single": single0, "pairMask": pair_mask, "seqMask": seq_mask, "tokens": n},
          "blocks": pws, "expectedPair": rp, "expectedSingle": rs}
    (tmp_path / "pairformer.json").write_text(json.dumps(_dump_tree(pf, tmp_path, "pf")))

    # Af3MsaStackGpu: two MSA-module blocks, AF3 order (webgpu/af3/trunk/msa-stack.js:67-140)
    mws = [S.synthetic_msa_module_weights(c_m=64, c_z=32, heads=8, dim=8, heads_pair=2, c_outer=8, seed=s_)
           for s_ in (41, 42)]
    ma = S.synthetic_activations(6, 16, 64, 32, seed=43)
    mm, mp = ma["msa"], ma["pair"]
    for mw in mws:
        mm, mp = blocks.msa_block_af3(mm, mp, ma["msaMask"], ma["pairMask"], mw, False)
    ms = {"state": {"msa": ma["msa"], "pair": ma["pair"], "msaMask": ma["msaMask"], "pairMask": ma["pairMask"],
                    "tokens": 16, "sequences": 6},
          "blocks": [dict(w, msaChannels=64, pairChannels=32) for w in mws], "expectedMsa": mm, "expectedPair": mp}
    (tmp_path / "msastack.json").write_text(json.dumps(_dump_tree(ms, tmp_path, "ms")))

    # InputEmbedderGpu (the reference test's input fields, test/input-embedder.gpu.test.js:56-77)
    iw, fe = S.synthetic_input_embedder(19, 3, 7, seed=44)
    rm_, rp_, re_ = ops.input_embedder_af2(fe["targetFeatures"], fe["msaFeatures"], fe["extraMsa"],
                                           fe["extraHasDeletion"], fe["extraDeletionValue"], fe["residueIndex"],
                                           fe["aatype"], fe["previousMsaFirstRow"], fe["previousPair"],
                                           fe["previousPositions"], iw)
    em = {"input": dict({k: np.asarray(v, np.float32).reshape(-1) for k, v in fe.items()}, length=19,
                        msaSequences=3, extraSequences=7, targetChannels=22, msaFeatureChannels=49, msaChannels=256,
                        pairChannels=128, extraMsaChannels=64, weights=iw),
          "expectedMsa": rm_, "expectedPair": rp_, "expectedExtra": re_}
    (tmp_path / "embed.json").write_text(json.dumps(_dump_tree(em, tmp_path, "em")))

    (tmp_path / "cases.json").write_text(json.dumps(cases))
    r = _run_node("gpu.test.js", tmp_path)
    assert r.returncode == 0 and "FAIL" not in r.stdout
    # the addon's calls went to the in-tree HIP library, not another copy
    loaded = [l.split(" ", 1)[1] for l in r.stdout.splitlines() if l.startswith("native-library ")]
    lib = os.path.realpath(os.path.join(os.path.dirname(__file__), "..", "localfold_amd", "lib", "liblocalfold.so"))
    assert loaded == [lib], (loaded, lib)
