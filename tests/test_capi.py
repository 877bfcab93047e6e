"""CPU-side checks of the boundary: the library loads, exports every function the header
declares, and the ctypes mirror matches the header (no compute: there is no GPU here)."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "localfold.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(lf_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ["lf_context_create", "lf_tri_mult", "lf_attention", "lf_transition", "lf_outer_product_mean",
              "lf_evoformer_block", "lf_evoformer_stack", "lf_pairformer_block", "lf_last_error"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    from localfold_amd import capi
    lib = capi.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_mirror_covers_header():
    from localfold_amd import capi
    bound = {name for name, _, _ in capi.PROTOTYPES}
    assert set(declared_functions()) == bound


def test_context_create_without_gpu_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from localfold_amd import capi
    lib = capi.load()
    assert not lib.lf_context_create(0)
    assert b"device" in lib.lf_last_error()


def test_struct_sizes_match_c_layout():
    """Compile a tiny C program against the header and compare sizeof/offsetof with ctypes."""
    import ctypes as C
    import subprocess
    import tempfile
    from localfold_amd import capi
    structs = ["lf_weight", "lf_tri_mult_weights", "lf_tri_mult_args", "lf_attention_weights", "lf_attention_args",
               "lf_transition_weights", "lf_transition_args", "lf_opm_weights", "lf_opm_args",
               "lf_evoformer_weights", "lf_evoformer_block_args", "lf_pairformer_weights",
               "lf_pairformer_block_args", "lf_kernel_timing", "lf_global_attention_weights",
               "lf_global_attention_args", "lf_extra_msa_weights", "lf_input_embedder_weights",
               "lf_input_embedder_args", "lf_af2_recycle_args", "lf_pair_averaging_weights",
               "lf_pair_averaging_args", "lf_msa_module_weights", "lf_msa_block_args"]
    src = "#include <stdio.h>\n#include \"localfold.h\"\nint main(){\n" + "".join(
        f'printf("{s} %zu\\n", sizeof({s}));\n' for s in structs) + "return 0;}\n"
    with tempfile.TemporaryDirectory() as d:
        c = Path(d) / "s.c"
        c.write_text(src)
        exe = Path(d) / "s"
        subprocess.run(["gcc", "-I", str(ROOT / "include"), str(c), "-o", str(exe)], check=True)
        out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    sizes = dict(line.split() for line in out.strip().splitlines())
    for s in structs:
        assert C.sizeof(getattr(capi, s)) == int(sizes[s]), s
