"""Weight codecs: the reference's on-disk quantisers and decoder, restated in numpy.

* int8, symmetric, one float16 scale per `block` (64) consecutive elements of the flattened
  stored tensor: `tools/quantize_model.py:103-117` (quantise), `shared/weights/dtype.js:227-250`
  (decode `code * scale`).
* intN (N<8, int5 in practice), asymmetric, float16 scale and zero per `block` (32)
  consecutive elements, codes packed least-significant-bit first, one slack byte:
  `tools/quantize_af3.py:59-97` (quantise, pack), `shared/weights/dtype.js:259-292,294-389`
  (decode `code * scale + zero`).
* float16: `shared/weights/dtype.js:391-395`.

Besides the reference's flat-group map (group = flat_index // block) this module also
builds the per-output-channel map that BASELINE config 2 names ("per-output-channel fp16
scales"): group = output column.  Both decode with the same `code*scale(+zero)`.

The decoder computes `code*scale + zero` exactly and rounds once to float32, as the
reference does (JS float64 arithmetic stored into a Float32Array).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
import numpy as np


def quantise_int8(values: np.ndarray, block: int = 64):
    """Symmetric per-block int8 (`tools/quantize_model.py:103-117`). Returns (codes int8, scales f16)."""
    flat = np.asarray(values, np.float32).reshape(-1)
    pad = (-flat.size) % block
    grid = np.concatenate([flat, np.zeros(pad, np.float32)]).reshape(-1, block)
    amax = np.abs(grid).max(1, keepdims=True)
    scale = (amax / 127.0).astype("<f2").astype(np.float32)
    safe = np.where(scale == 0, 1.0, scale)
    codes = np.clip(np.rint(grid / safe), -127, 127).astype(np.int8)
    return codes.reshape(-1)[:flat.size], scale.reshape(-1).astype("<f2")


def quantise_asym(values: np.ndarray, block: int = 32, bits: int = 5):
    """Asymmetric per-group codes (`tools/quantize_af3.py:59-80`). Returns (codes u8, scales f16, zeros f16)."""
    levels = 2 ** bits - 1
    flat = np.asarray(values, np.float32).reshape(-1)
    pad = (-flat.size) % block
    grid = np.concatenate([flat, np.zeros(pad, np.float32)]).reshape(-1, block)
    low = grid.min(1, keepdims=True).astype(np.float32)
    high = grid.max(1, keepdims=True).astype(np.float32)
    zeros = low.astype(np.float16)
    scales = ((high - low) / levels).astype(np.float16)
    safe = scales.astype(np.float32)
    safe[safe == 0] = 1.0
    codes = np.clip(np.rint((grid - zeros.astype(np.float32)) / safe), 0, levels).astype(np.uint8)
    return codes, scales.reshape(-1), zeros.reshape(-1)


def pack_bits(codes: np.ndarray, bits: int = 5) -> np.ndarray:
    """LSB-first packing of a (groups, group) code grid plus one slack byte (`quantize_af3.py:83-101`)."""
    groups, group = codes.shape
    if (group * bits) % 8:
        raise ValueError(f"group {group} of {bits} bits does not pack into whole bytes")
    unpacked = np.unpackbits(codes[:, :, None].astype(np.uint8), axis=2, count=bits, bitorder="little")
    stream = unpacked.reshape(groups, group * bits)
    packed = np.packbits(stream, axis=1, bitorder="little").astype(np.uint8).reshape(-1)
    return np.concatenate([packed, np.zeros(1, np.uint8)])


def quantise_per_channel(values: np.ndarray, out_axis: int, bits: int, symmetric: bool):
    """Per-output-channel quantisation: one group per output column.

    Same rounding rules as the flat quantisers (scale/zero rounded to f16 before the codes
    are chosen).  Returns codes in the stored (flattened) order and per-channel tables.
    """
    w = np.asarray(values, np.float32)
    moved = np.moveaxis(w, out_axis, 0).reshape(w.shape[out_axis], -1)   # [out, in]
    if symmetric:
        amax = np.abs(moved).max(1, keepdims=True)
        levels = 2 ** (bits - 1) - 1
        scale = (amax / levels).astype("<f2").astype(np.float32)
        safe = np.where(scale == 0, 1.0, scale)
        codes = np.clip(np.rint(moved / safe), -levels, levels).astype(np.int8)
        zeros = None
    else:
        levels = 2 ** bits - 1
        low = moved.min(1, keepdims=True)
        high = moved.max(1, keepdims=True)
        zeros16 = low.astype(np.float16)
        scale16 = ((high - low) / levels).astype(np.float16)
        safe = scale16.astype(np.float32)
        safe[safe == 0] = 1.0
        codes = np.clip(np.rint((moved - zeros16.astype(np.float32)) / safe), 0, levels).astype(np.uint8)
        scale = scale16.astype(np.float32)
        zeros = zeros16.reshape(-1)
    codes_stored = np.moveaxis(codes.reshape([w.shape[out_axis]] + [s for i, s in enumerate(w.shape) if i != out_axis]),
                               0, out_axis).reshape(-1)
    return codes_stored, scale.reshape(-1).astype("<f2"), zeros


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


def make_record(values: np.ndarray, dtype: str, block: int = None, channel_axis: int = None) -> dict:
    """Quantise `values` (stored shape) into a record `decode` and the HIP loaders read."""
    values = np.asarray(values, np.float32)
    shape = list(values.shape)
    if dtype == "float32":
        return {"dtype": dtype, "shape": shape, "data": values.copy()}
    if dtype == "float16":
        return {"dtype": dtype, "shape": shape, "data": values.astype(np.float16)}
    if dtype == "int8":
        if channel_axis is not None:
            codes, scales, _ = quantise_per_channel(values, channel_axis, 8, True)
            return {"dtype": dtype, "shape": shape, "data": codes.astype(np.int8), "scales": scales,
                    "channel_axis": channel_axis}
        codes, scales = quantise_int8(values, block or 64)
        return {"dtype": dtype, "shape": shape, "data": codes, "scales": scales, "block": block or 64}
    if dtype.startswith("int"):
        bits = int(dtype[3:])
        if channel_axis is not None:
            codes, scales, zeros = quantise_per_channel(values, channel_axis, bits, False)
            n = codes.size
            pad = (-n) % 8
            packed = pack_bits(np.concatenate([codes, np.zeros(pad, np.uint8)]).reshape(1, -1), bits)
            return {"dtype": dtype, "shape": shape, "data": packed, "scales": scales, "zeros": zeros,
                    "channel_axis": channel_axis}
        block = block or 32
        codes, scales, zeros = quantise_asym(values, block, bits)
        return {"dtype": dtype, "shape": shape, "data": pack_bits(codes, bits), "scales": scales,
                "zeros": zeros, "block": block}
    raise ValueError(dtype)
