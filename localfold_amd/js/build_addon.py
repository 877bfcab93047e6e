"""Builds localfold_amd/lib/localfold_napi.node (the N-API binding of liblocalfold.so) with g++.

    python localfold_amd/js/build_addon.py

Compiles addon.cc against the installed Node headers (/usr/include/node); N-API symbols
resolve from the node binary at load time, liblocalfold.so through an $ORIGIN rpath.
"""
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE.parent / "lib"
NODE_INCLUDE = Path(os.environ.get("NODE_INCLUDE", "/usr/include/node"))


def build() -> Path:
    out = LIB / "localfold_napi.node"
    if not (NODE_INCLUDE / "node_api.h").exists():
        raise RuntimeError(f"node_api.h not found under {NODE_INCLUDE}")
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wno-unused-parameter",
           f"-I{NODE_INCLUDE}", "-DNODE_GYP_MODULE_NAME=localfold_napi", str(HERE / "addon.cc"),
           "-o", str(out), f"-L{LIB}", "-llocalfold", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"addon build failed:\n{r.stderr}")
    print(f"built {out}", file=sys.stderr)
    return out


if __name__ == "__main__":
    build()
