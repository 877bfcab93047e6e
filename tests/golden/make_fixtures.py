"""Convert the reference's committed triangle-multiplication fixtures into npz files.

The four fixtures are data the reference's own tests hold
(`test/fixtures/openfold-triangle-small/`, `test/fixtures/alphafold-single-sequence/short-9/`,
`test/fixtures/alphafold-single-sequence/model1-reference-59/`,
`test/fixtures/alphafold-a3m/model1-reference-59/`; loaded there by
`shared/bundles/node.js:11-40` and checked in `test/cpu-reference.test.js:18-27` and
`test/triangle-multiplication-outgoing.gpu.test.js:31-69`).  Each holds `z`, `mask`, the
sixteen (out,in) weights of `TriangleMultiplicationOutgoing` and the reference `expected`
update (without the residual).  This script copies the float32 tensors verbatim into one
compressed npz per fixture, plus the manifest's shape/epsilon/source.  It reads the
reference tree only when run by hand; the tests read the npz files.

    python tests/golden/make_fixtures.py /root/reference
"""
import json
import sys
from pathlib import Path

import numpy as np

FIXTURES = {
    "openfold_triangle_small": "test/fixtures/openfold-triangle-small",
    "af2_single_short9": "test/fixtures/alphafold-single-sequence/short-9",
    "af2_single_model1_59": "test/fixtures/alphafold-single-sequence/model1-reference-59",
    "af2_a3m_model1_59": "test/fixtures/alphafold-a3m/model1-reference-59",
}


def convert(root: Path, out: Path) -> None:
    for name, rel in FIXTURES.items():
        directory = root / rel
        manifest = json.loads((directory / "manifest.json").read_text())
        arrays = {}
        for tensor, record in manifest["tensors"].items():
            assert record["dtype"] == "float32"
            raw = np.fromfile(directory / record["file"], dtype="<f4")
            assert raw.size == int(np.prod(record["shape"])), tensor
            arrays[tensor] = raw.reshape(record["shape"])
        meta = {"source": manifest["source"], "shape": manifest["shape"],
                "epsilon": manifest["epsilon"], "operator": manifest["operator"]}
        np.savez_compressed(out / f"{name}.npz", meta=np.array(json.dumps(meta)), **arrays)
        print(name, {k: v.shape for k, v in arrays.items() if k in ("z", "expected")})


if __name__ == "__main__":
    convert(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"), Path(__file__).parent)
