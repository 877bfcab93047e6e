"""Weight codec DECODER: the reference's readTensorRange, restated in numpy (the checker).

The encoders (quantisers, bit packer) that write the records live in
localfold_amd/synthetic.py; this module only reads records back, independently.

* int8, symmetric, one float16 scale per `block` (64) consecutive elements of the flattened
  stored tensor: `tools/quantize_model.py:103-117` (quantise), `shared/weights/dtype.js:227-250`
  (decode `code * scale`).
* intN (N<8, int5 in practice), asymmetric, float16 scale and zero per `block` (32)
  consecutive elements, codes packed least-significant-bit first, one slack byte:
  `tools/quantize_af3.py:59-97` (quantise, pack), `shared/weights/dtype.js:259-292,294-389`
  (decode `code * scale + zero`).
* float16: `shared/weights/dtype.js:391-395`.

Besides the reference's flat-group map (group = flat_index // block) this module also
builds the per-output-channel map that the headline triangle workload uses ("per-output-channel fp16
scales"): group = output column.  Both decode with the same `code*scale(+zero)`.

The decoder computes `code*scale + zero` exactly and rounds once to float32, as the
reference does (JS float64 arithmetic stored into a Float32Array).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
import numpy as np


def unpack_bits(packed: np.ndarray, count: int, bits: int) -> np.ndarray:
    """Code `i` starts at bit `i*bits`; read two bytes and mask (`dtype.js:279-286`)."""
    idx = np.arange(count, dtype=np.int64)
    bit = idx * bits
    byte = bit >> 3
    pair = packed[byte].astype(np.uint32) | (packed[byte + 1].astype(np.uint32) << 8)
    return ((pair >> (bit & 7).astype(np.uint32)) & ((1 << bits) - 1)).astype(np.uint8)


def decode(record: dict) -> np.ndarray:
    """Decode a weight record to float32 in its stored shape.

    record: {dtype: "float32"|"float16"|"int8"|"int5"|"intN", shape, data, scales?, zeros?,
             block (flat group) | channel_axis (per-output-channel map)}.
    Follows `readTensorRange` (`shared/weights/dtype.js:212-406`); the per-channel map uses
    the same arithmetic with group = index along `channel_axis`.
    """
    shape = tuple(record["shape"])
    n = int(np.prod(shape))
    dt = record["dtype"]
    if dt == "float32":
        return np.asarray(record["data"], np.float32).reshape(shape)
    if dt == "float16":
        return np.asarray(record["data"], np.float16).astype(np.float32).reshape(shape)
    if "channel_axis" in record:
        ax = record["channel_axis"]
        grid = np.indices(shape)[ax].reshape(-1)
    else:
        grid = np.arange(n) // record["block"]
    scales = np.asarray(record["scales"], np.float16).astype(np.float64)[grid]
    if dt == "int8":
        codes = np.asarray(record["data"], np.int8).reshape(-1)[:n].astype(np.float64)
        return (codes * scales).astype(np.float32).reshape(shape)
    bits = int(dt[3:])
    if "channel_axis" in record and record.get("packed", True) is False:
        codes = np.asarray(record["data"], np.uint8).reshape(-1)[:n]
    else:
        codes = unpack_bits(np.asarray(record["data"], np.uint8), n, bits)
    zeros = np.asarray(record["zeros"], np.float16).astype(np.float64)[grid]
    return (codes.astype(np.float64) * scales + zeros).astype(np.float32).reshape(shape)


