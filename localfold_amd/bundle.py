"""Weight bundles in the reference's manifest + shard format, read for the device.

A bundle is a JSON manifest whose ``tensors`` table maps a name to
``{file, shape, dtype, byteOffset?, block?, scaleOffset?, zeroOffset?}`` inside shard files
beside it (shared/bundles/tensor-store.js:5-58).  The stored forms are those of
shared/weights/dtype.js:24-406:

- ``float32`` / ``float16``: little-endian values;
- ``int8``: one code per element at ``byteOffset``, then an fp16 scale per ``block`` elements
  at the *absolute* ``scaleOffset`` (symmetric: value = code * scale);
- ``intN`` (N < 8, e.g. ``int5``): codes packed LSB-first, ``block * N / 8`` bytes per group
  plus one slack byte at the end, fp16 scales at ``scaleOffset`` and fp16 zero points at
  ``zeroOffset`` (asymmetric: value = code * scale + zero).

Quantised tensors stay quantised here: :meth:`FileTensorStore.record` hands back the codes and
tables as stored (sliced to one block of a stacked tensor), which the kernels decode on the
device; only vectors (biases, LayerNorm parameters) are decoded on the host, as
:meth:`FileTensorStore.values`.  :func:`af2_main_stack_weights` maps an AF2 bundle's
stacked-haiku parameter table to the per-block weight dictionaries the block entry points take
(shared/bundles/alphafold-fixture.js:41-270, ``mainStackWeights``).
"""
import json
import math
import os
import re

import numpy as np

__all__ = ["FileTensorStore", "af2_main_stack_weights", "packed_bits", "tensor_elements", "tensor_byte_length"]

_BYTES = {"float32": 4, "float16": 2, "int8": 1}


def packed_bits(dtype: str):
    """Width of a sub-byte packed integer dtype (int1..int7), else None (dtype.js:43-48)."""
    m = re.fullmatch(r"int([1-9])", dtype)
    if m is None:
        return None
    bits = int(m.group(1))
    return bits if bits < 8 else None


def tensor_elements(rec: dict) -> int:
    return int(np.prod(rec["shape"], dtype=np.int64)) if len(rec["shape"]) else 1


def tensor_byte_length(rec: dict) -> int:
    """Bytes one tensor spans from its byteOffset (dtype.js:127-149): for quantised tensors the
    codes, any padding and the trailing fp16 tables (one for int8, two for packed widths)."""
    bits = packed_bits(rec["dtype"])
    if rec["dtype"] not in _BYTES and bits is None:
        raise ValueError(f"unsupported tensor dtype {rec['dtype']}")
    n = tensor_elements(rec)
    if rec["dtype"] != "int8" and bits is None:
        return n * _BYTES[rec["dtype"]]
    block, scale_offset = rec.get("block"), rec.get("scaleOffset")
    if not isinstance(block, int) or block <= 0:
        raise ValueError(f"{rec['dtype']} tensor has no block size")
    if not isinstance(scale_offset, int):
        raise ValueError(f"{rec['dtype']} tensor has no scale offset")
    groups = -(-n // block)
    trailing = groups * 2 if bits is None else groups * 4
    return (scale_offset - rec.get("byteOffset", 0)) + trailing


class FileTensorStore:
    """A manifest's tensor table over memory-mapped shards (tensor-store.js:5-58)."""

    def __init__(self, manifest_path: str):
        self.manifest_path = os.path.abspath(manifest_path)
        with open(self.manifest_path, encoding="utf8") as f:
            self.manifest = json.load(f)
        if "tensors" not in self.manifest:
            raise ValueError(f"{self.manifest_path} has no tensor table")
        self._dir = os.path.dirname(self.manifest_path)
        self._shards = {}

    @classmethod
    def open(cls, manifest_path: str) -> "FileTensorStore":
        return cls(manifest_path)

    def _record(self, name: str) -> dict:
        rec = self.manifest["tensors"].get(name)
        if rec is None:
            raise KeyError(f"manifest contains no tensor named {name}")
        if "dtype" not in rec:
            # a missing dtype is a manifest this reader does not understand, not float32
            raise ValueError(f"{name} has no dtype")
        return rec

    def shape(self, name: str):
        return list(self._record(name)["shape"])

    def _shard(self, name: str, rec: dict) -> np.ndarray:
        buf = self._shards.get(rec["file"])
        if buf is None:
            path = os.path.join(self._dir, rec["file"])
            buf = np.memmap(path, dtype=np.uint8, mode="r") if os.path.getsize(path) else np.zeros(0, np.uint8)
            self._shards[rec["file"]] = buf
        start = rec.get("byteOffset", 0)
        if not isinstance(start, int) or start < 0 or start + tensor_byte_length(rec) > buf.size:
            raise ValueError(f"{name} points outside {rec['file']}")
        return buf

    def _range(self, rec: dict, first: int, count):
        n = tensor_elements(rec)
        count = n - first if count is None else count
        if first < 0 or count < 0 or first + count > n:
            raise IndexError(f"range {first}:{count} lies outside a tensor of {n}")
        return count

    def record(self, name: str, first: int = 0, count: int = None, shape=None) -> dict:
        """Elements [first, first + count) as a device weight record: codes and tables as
        stored for quantised dtypes (the range must start on a quantisation group and, for
        packed widths, on a byte), values for float dtypes.  ``shape`` (default: the range as
        one row) is the logical 2-D shape the record carries."""
        rec = self._record(name)
        count = self._range(rec, first, count)
        buf = self._shard(name, rec)
        base = rec.get("byteOffset", 0)
        out = {"shape": list(shape) if shape is not None else [count], "source": name}
        dt = rec["dtype"]
        if dt == "float32":
            out.update(dtype="float32", data=np.frombuffer(buf, np.float32, count, base + 4 * first).copy())
            return out
        if dt == "float16":
            out.update(dtype="float16", data=np.frombuffer(buf, np.float16, count, base + 2 * first).astype(np.float32))
            return out
        block = rec["block"]
        if first % block:
            raise ValueError(f"{name}: range {first}:{count} does not start on a quantisation group of {block}")
        g0, g1 = first // block, -(-(first + count) // block)
        scale_at = rec["scaleOffset"]
        scales = np.frombuffer(buf, np.uint16, g1 - g0, scale_at + 2 * g0).copy()
        if dt == "int8":
            codes = np.frombuffer(buf, np.int8, count, base + first).copy()
            out.update(dtype="int8", data=codes, scales=scales.view(np.float16), block=block)
            return out
        bits = packed_bits(dt)
        if bits is None:
            raise ValueError(f"unsupported tensor dtype {dt}")
        if (first * bits) % 8 or (block * bits) % 8:
            raise ValueError(f"{name}: {dt} at group {block} does not split into whole bytes at {first}")
        if not isinstance(rec.get("zeroOffset"), int):
            raise ValueError(f"{dt} tensor has no zero offset; it is asymmetric")
        nbytes = -(-count * bits // 8) + 1   # the codes plus the slack byte the decoder may touch
        start = base + first * bits // 8
        codes = np.frombuffer(buf, np.uint8, min(nbytes, buf.size - start), start).copy()
        if codes.size < nbytes:
            codes = np.concatenate([codes, np.zeros(nbytes - codes.size, np.uint8)])
        zeros = np.frombuffer(buf, np.uint16, g1 - g0, rec["zeroOffset"] + 2 * g0).copy()
        out.update(dtype=dt, data=codes, scales=scales.view(np.float16), zeros=zeros.view(np.float16), block=block)
        return out

    def values(self, name: str, first: int = 0, count: int = None) -> np.ndarray:
        """Elements [first, first + count) decoded to float32 on the host, as readTensorRange
        does (dtype.js:212-406): code * scale for int8, code * scale + zero for packed widths,
        computed in float64 and rounded once."""
        rec = self._record(name)
        count = self._range(rec, first, count)
        if rec["dtype"] in ("float32", "float16"):
            return self.record(name, first, count)["data"].astype(np.float32)
        block = rec["block"]
        g0 = first // block
        lo = g0 * block
        r = self.record(name, lo, count + (first - lo))
        n = count + (first - lo)
        groups = np.arange(n) // block
        scale = r["scales"].astype(np.float64)[groups]
        if r["dtype"] == "int8":
            v = r["data"].astype(np.float64) * scale
        else:
            bits = packed_bits(r["dtype"])
            codes = r["data"].astype(np.uint32)
            bit = np.arange(n, dtype=np.int64) * bits
            pair = codes[bit >> 3] | (codes[(bit >> 3) + 1] << 8)
            v = ((pair >> (bit & 7).astype(np.uint32)) & ((1 << bits) - 1)).astype(np.float64) * scale \
                + r["zeros"].astype(np.float64)[groups]
        return v[first - lo:].astype(np.float32)


# ---------------------------------------------------------------------------------------
# AF2 main-stack parameters (stacked haiku) -> per-block weight dictionaries
# ---------------------------------------------------------------------------------------

class _Stacked:
    def __init__(self, store: FileTensorStore, parameters: dict, blocks: int, block: int):
        self.store, self.parameters, self.blocks, self.block = store, parameters, blocks, block

    def _name(self, module: str, key: str) -> str:
        name = self.parameters.get(module, {}).get(key)
        if name is None:
            raise KeyError(f"missing {module}/{key}")
        return name

    def _slice(self, name: str):
        n = tensor_elements(self.store._record(name))
        if n % self.blocks:
            raise ValueError(f"{name}: {n} elements do not split into {self.blocks} blocks")
        per = n // self.blocks
        return self.block * per, per

    def shape(self, module: str, key: str):
        return self.store.shape(self._name(module, key))[1:]

    def vector(self, module: str, key: str) -> np.ndarray:
        name = self._name(module, key)
        first, count = self._slice(name)
        return self.store.values(name, first, count)

    def matrix(self, module: str, key: str, rows: int) -> dict:
        """One block's [in][out] matrix as a device record (layout in,out: haiku stores every
        linear as [input][output], with head axes flattened in order)."""
        name = self._name(module, key)
        first, count = self._slice(name)
        if count % rows:
            raise ValueError(f"{module}/{key}: {count} elements are not {rows} rows")
        rec = self.store.record(name, first, count, shape=[rows, count // rows])
        rec["layout"] = "in_out"
        return rec


def _attention(p: _Stacked, root: str, c: int) -> dict:
    a = f"{root}/attention"
    return {
        "heads": int(p.shape(a, "gating_b")[0]),
        "attention": {
            "queryNormScale": p.vector(f"{root}/query_norm", "scale"),
            "queryNormOffset": p.vector(f"{root}/query_norm", "offset"),
            "queryWeight": p.matrix(a, "query_w", c),
            "keyWeight": p.matrix(a, "key_w", c),
            "valueWeight": p.matrix(a, "value_w", c),
            "gatingWeight": p.matrix(a, "gating_w", c),
            "gatingBias": p.vector(a, "gating_b"),
            "outputWeight": p.matrix(a, "output_w", int(np.prod(p.shape(a, "output_w")[:-1]))),
            "outputBias": p.vector(a, "output_b"),
        },
    }


def _transition(p: _Stacked, root: str, c: int) -> dict:
    hidden = int(p.shape(f"{root}/transition1", "bias")[0])
    return {
        "layerNormScale": p.vector(f"{root}/input_layer_norm", "scale"),
        "layerNormOffset": p.vector(f"{root}/input_layer_norm", "offset"),
        "firstWeight": p.matrix(f"{root}/transition1", "weights", c),
        "firstBias": p.vector(f"{root}/transition1", "bias"),
        "secondWeight": p.matrix(f"{root}/transition2", "weights", hidden),
        "secondBias": p.vector(f"{root}/transition2", "bias"),
    }


def _triangle(p: _Stacked, root: str, cz: int) -> dict:
    hidden = int(p.shape(f"{root}/left_projection", "bias")[0])
    out = {
        "layerNormInWeight": p.vector(f"{root}/layer_norm_input", "scale"),
        "layerNormInBias": p.vector(f"{root}/layer_norm_input", "offset"),
        "layerNormOutWeight": p.vector(f"{root}/center_layer_norm", "scale"),
        "layerNormOutBias": p.vector(f"{root}/center_layer_norm", "offset"),
    }
    for name, module, rows in (("linearAP", "left_projection", cz), ("linearAG", "left_gate", cz),
                               ("linearBP", "right_projection", cz), ("linearBG", "right_gate", cz),
                               ("linearZ", "output_projection", hidden), ("linearG", "gating_linear", cz)):
        # stored [in][out]; the kernels read either layout, so the codes go up untransposed
        out[name + "Weight"] = p.matrix(f"{root}/{module}", "weights", rows)
        out[name + "Bias"] = p.vector(f"{root}/{module}", "bias")
    return out


def af2_main_stack_weights(store: FileTensorStore, msa_channels: int = 256, pair_channels: int = 128):
    """One weight dictionary per Evoformer block from an AF2 bundle's ``evoformerStack``
    section, in the structure of ``EvoformerStackGpu``'s ``input.blocks``
    (alphafold-fixture.js:222-270).  Matrices are device records of the stored codes."""
    section = store.manifest.get("evoformerStack")
    if section is None or section.get("parameterFormat") != "stacked-haiku":
        raise ValueError("bundle has no stacked-haiku evoformerStack section")
    blocks, parameters = int(section["blocks"]), section["parameters"]
    cm, cz = msa_channels, pair_channels
    result = []
    for block in range(blocks):
        p = _Stacked(store, parameters, blocks, block)
        row = _attention(p, "msa_row_attention_with_pair_bias", cm)
        row["pairBias"] = {
            "layerNormScale": p.vector("msa_row_attention_with_pair_bias/feat_2d_norm", "scale"),
            "layerNormOffset": p.vector("msa_row_attention_with_pair_bias/feat_2d_norm", "offset"),
            "projectionWeight": p.matrix("msa_row_attention_with_pair_bias", "feat_2d_weights", cz),
        }
        tri_start = _attention(p, "triangle_attention_starting_node", cz)
        tri_start["pairBias"] = {"projectionWeight": p.matrix("triangle_attention_starting_node", "feat_2d_weights", cz)}
        tri_end = _attention(p, "triangle_attention_ending_node", cz)
        tri_end["pairBias"] = {"projectionWeight": p.matrix("triangle_attention_ending_node", "feat_2d_weights", cz)}
        c_outer = int(p.shape("outer_product_mean/left_projection", "bias")[0])
        result.append({
            "msaRowAttention": row,
            "msaColumnAttention": _attention(p, "msa_column_attention", cm),
            "msaTransition": _transition(p, "msa_transition", cm),
            "outerProductMean": {
                "layerNormScale": p.vector("outer_product_mean/layer_norm_input", "scale"),
                "layerNormOffset": p.vector("outer_product_mean/layer_norm_input", "offset"),
                "leftWeight": p.matrix("outer_product_mean/left_projection", "weights", cm),
                "leftBias": p.vector("outer_product_mean/left_projection", "bias"),
                "rightWeight": p.matrix("outer_product_mean/right_projection", "weights", cm),
                "rightBias": p.vector("outer_product_mean/right_projection", "bias"),
                "outputWeight": p.matrix("outer_product_mean", "output_w", c_outer * c_outer),
                "outputBias": p.vector("outer_product_mean", "output_b"),
            },
            "triangleMultiplicationOutgoing": _triangle(p, "triangle_multiplication_outgoing", cz),
            "triangleMultiplicationIncoming": _triangle(p, "triangle_multiplication_incoming", cz),
            "triangleAttentionStarting": tri_start,
            "triangleAttentionEnding": tri_end,
            "pairTransition": _transition(p, "pair_transition", cz),
        })
    return result
