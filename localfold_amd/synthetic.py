"""Synthetic inputs: the reference's deterministic generator, its synthetic weight builders,
its weight quantisers, and the benchmark workload definitions.

This is the equivalent of the reference's testing/tooling surface
(`webgpu/testing/deterministic-input.js`, `tools/gpu/af2-synthetic-block.js`,
`tools/quantize_model.py`, `tools/quantize_af3.py`): it writes inputs and weight records,
it computes nothing on the hot path.

`generator(seed)` (`webgpu/testing/deterministic-input.js:1-10`, identical copy in
`tools/gpu/af2-synthetic-block.js:20-29`) is a mulberry32-style integer mixer whose
state advances by the constant 0x6d2b79f5 before every draw.  Draw `i` (0-based) therefore
depends only on `seed + (i+1)*0x6d2b79f5 mod 2^32`, so a whole stream is one vectorised
uint32 computation.  `Math.imul` is the low 32 bits of a product, `>>>` a logical shift,
and the JS `value + imul(...)` followed by `^` wraps mod 2^32 - all of which uint32
numpy arithmetic reproduces bit for bit.
"""
import numpy as np

_INC = np.uint32(0x6D2B79F5)


def uniform_stream(seed: int, count: int, start: int = 0) -> np.ndarray:
    """Draws `start .. start+count-1` of `generator(seed)` as float64 in [0, 1).

    Follows `deterministic-input.js:1-10` line by line, vectorised over the counter.
    """
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        state = ((np.uint64(seed & 0xFFFFFFFF) + idx * np.uint64(0x6D2B79F5)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        v = state
        v = (v ^ (v >> np.uint32(15))) * (v | np.uint32(1))                       # imul(v ^ v>>>15, v|1)
        v = v ^ (v + (v ^ (v >> np.uint32(7))) * (v | np.uint32(61)))           # v ^= v + imul(v ^ v>>>7, v|61)
        v = v ^ (v >> np.uint32(14))
    return v.astype(np.float64) / 4294967296.0


class Stream:
    """A cursor over one generator, drawing blocks in order like the JS closures do."""

    def __init__(self, seed: int):
        self.seed = seed
        self.pos = 0

    def uniform(self, count: int) -> np.ndarray:
        out = uniform_stream(self.seed, count, self.pos)
        self.pos += count
        return out

    def values(self, count: int, scale: float, center: float = 0.0) -> np.ndarray:
        """`center + (random()*2 - 1)*scale` stored as float32 (`deterministic-input.js:14-18`)."""
        return (center + (self.uniform(count) * 2.0 - 1.0) * scale).astype(np.float32)

    def normal(self, count: int, std: float = 1.0) -> np.ndarray:
        """Box-Muller over consecutive draw pairs: z = sqrt(-2 ln(1-u1)) cos(2 pi u2).

        The reference has no normal sampler; this is the transform the benchmark workloads
        (`~N(0, s)`) are generated with here, stated so a fixture can be reproduced.
        """
        pairs = self.uniform(2 * count).reshape(count, 2)
        r = np.sqrt(-2.0 * np.log1p(-pairs[:, 0]))
        return (r * np.cos(2.0 * np.pi * pairs[:, 1]) * std).astype(np.float32)


TRIANGLE_WEIGHT_NAMES = [
    "layerNormInWeight", "layerNormInBias", "linearAPWeight", "linearAPBias",
    "linearAGWeight", "linearAGBias", "linearBPWeight", "linearBPBias",
    "linearBGWeight", "linearBGBias", "layerNormOutWeight", "layerNormOutBias",
    "linearZWeight", "linearZBias", "linearGWeight", "linearGBias",
]


def deterministic_triangle_input(length: int, c_z: int, c_hidden: int, seed: int = 7) -> dict:
    """`createDeterministicTriangleInput` (`webgpu/testing/deterministic-input.js:12-45`)."""
    s = Stream(seed)
    v = s.values
    rz, rh = 1.0 / np.sqrt(c_z), 1.0 / np.sqrt(c_hidden)
    w = {}
    w["layerNormInWeight"] = v(c_z, 0.1, 1)
    w["layerNormInBias"] = v(c_z, 0.05)
    w["linearAPWeight"] = v(c_hidden * c_z, 0.15 * rz).reshape(c_hidden, c_z)
    w["linearAPBias"] = v(c_hidden, 0.03)
    w["linearAGWeight"] = v(c_hidden * c_z, 0.15 * rz).reshape(c_hidden, c_z)
    w["linearAGBias"] = v(c_hidden, 0.03, 1)
    w["linearBPWeight"] = v(c_hidden * c_z, 0.15 * rz).reshape(c_hidden, c_z)
    w["linearBPBias"] = v(c_hidden, 0.03)
    w["linearBGWeight"] = v(c_hidden * c_z, 0.15 * rz).reshape(c_hidden, c_z)
    w["linearBGBias"] = v(c_hidden, 0.03, 1)
    w["layerNormOutWeight"] = v(c_hidden, 0.1, 1)
    w["layerNormOutBias"] = v(c_hidden, 0.05)
    w["linearZWeight"] = v(c_z * c_hidden, 0.15 * rh).reshape(c_z, c_hidden)
    w["linearZBias"] = v(c_z, 0.03)
    w["linearGWeight"] = v(c_z * c_z, 0.15 * rz).reshape(c_z, c_z)
    w["linearGBias"] = v(c_z, 0.03, 1)
    pairs = length * length
    mask = (s.uniform(pairs) > 0.15).astype(np.float32).reshape(length, length)
    z = v(pairs * c_z, 1).reshape(length, length, c_z)
    return {"shape": {"length": length, "cZ": c_z, "cHidden": c_hidden}, "z": z, "mask": mask,
            "weights": w}


def synthetic_block_weights(c_m: int, c_z: int, c_outer: int, heads_msa: int, heads_pair: int,
                            tri_hidden: int, msa_hidden: int, pair_hidden: int, seed: int = 1) -> dict:
    """`syntheticBlockWeights` (`tools/gpu/af2-synthetic-block.js:36-138`), AF2 main block.

    The reference uses one `heads` for every attention; here the MSA (row/column) and pair
    (triangle) head counts are separate because AF2 uses 8 and 4.  Draw order follows
    the reference's object literal order.  Attention, transition and OPM weights are
    (in,out); triangle weights are (out,in) as `webgpu/kernels/triangle/types.js:28-43` reads them.
    """
    s = Stream(seed)
    noise = s.values

    def attention_group(channels, heads):
        r = 1.0 / np.sqrt(channels)
        return {"heads": heads, "attention": {
            "queryNormScale": noise(channels, 0.2, 1),
            "queryNormOffset": noise(channels, 0.1),
            "queryWeight": noise(channels * channels, r).reshape(channels, channels),
            "keyWeight": noise(channels * channels, r).reshape(channels, channels),
            "valueWeight": noise(channels * channels, r).reshape(channels, channels),
            "gatingWeight": noise(channels * channels, r).reshape(channels, channels),
            "gatingBias": noise(channels, 0.1, 1),
            "outputWeight": noise(channels * channels, r).reshape(channels, channels),
            "outputBias": noise(channels, 0.05),
        }}

    def transition_group(channels, hidden):
        return {
            "layerNormScale": noise(channels, 0.2, 1),
            "layerNormOffset": noise(channels, 0.1),
            "firstWeight": noise(channels * hidden, 1 / np.sqrt(channels)).reshape(channels, hidden),
            "firstBias": noise(hidden, 0.1),
            "secondWeight": noise(hidden * channels, 1 / np.sqrt(hidden)).reshape(hidden, channels),
            "secondBias": noise(channels, 0.05),
        }

    def triangle_group():
        rz, rh = 0.15 / np.sqrt(c_z), 0.15 / np.sqrt(tri_hidden)
        return {
            "layerNormInWeight": noise(c_z, 0.2, 1),
            "layerNormInBias": noise(c_z, 0.1),
            "linearAPWeight": noise(tri_hidden * c_z, rz).reshape(tri_hidden, c_z),
            "linearAPBias": noise(tri_hidden, 0.03),
            "linearAGWeight": noise(tri_hidden * c_z, rz).reshape(tri_hidden, c_z),
            "linearAGBias": noise(tri_hidden, 0.03, 1),
            "linearBPWeight": noise(tri_hidden * c_z, rz).reshape(tri_hidden, c_z),
            "linearBPBias": noise(tri_hidden, 0.03),
            "linearBGWeight": noise(tri_hidden * c_z, rz).reshape(tri_hidden, c_z),
            "linearBGBias": noise(tri_hidden, 0.03, 1),
            "layerNormOutWeight": noise(tri_hidden, 0.2, 1),
            "layerNormOutBias": noise(tri_hidden, 0.1),
            "linearZWeight": noise(c_z * tri_hidden, rh).reshape(c_z, tri_hidden),
            "linearZBias": noise(c_z, 0.03),
            "linearGWeight": noise(c_z * c_z, rz).reshape(c_z, c_z),
            "linearGBias": noise(c_z, 0.03, 1),
        }

    w = {}
    row = attention_group(c_m, heads_msa)
    row["pairBias"] = {
        "layerNormScale": noise(c_z, 0.2, 1),
        "layerNormOffset": noise(c_z, 0.1),
        "projectionWeight": noise(c_z * heads_msa, 1 / np.sqrt(c_z)).reshape(c_z, heads_msa),
    }
    w["msaRowAttention"] = row
    w["msaTransition"] = transition_group(c_m, msa_hidden)
    w["outerProductMean"] = {
        "layerNormScale": noise(c_m, 0.2, 1),
        "layerNormOffset": noise(c_m, 0.1),
        "leftWeight": noise(c_m * c_outer, 1 / np.sqrt(c_m)).reshape(c_m, c_outer),
        "leftBias": noise(c_outer, 0.1),
        "rightWeight": noise(c_m * c_outer, 1 / np.sqrt(c_m)).reshape(c_m, c_outer),
        "rightBias": noise(c_outer, 0.1),
        "outputWeight": noise(c_outer * c_outer * c_z, 1 / c_outer).reshape(c_outer * c_outer, c_z),
        "outputBias": noise(c_z, 0.05),
    }
    w["triangleMultiplicationOutgoing"] = triangle_group()
    w["triangleMultiplicationIncoming"] = triangle_group()
    start = attention_group(c_z, heads_pair)
    start["pairBias"] = {"projectionWeight": noise(c_z * heads_pair, 1 / np.sqrt(c_z)).reshape(c_z, heads_pair)}
    w["triangleAttentionStarting"] = start
    end = attention_group(c_z, heads_pair)
    end["pairBias"] = {"projectionWeight": noise(c_z * heads_pair, 1 / np.sqrt(c_z)).reshape(c_z, heads_pair)}
    w["triangleAttentionEnding"] = end
    w["pairTransition"] = transition_group(c_z, pair_hidden)
    w["msaColumnAttention"] = attention_group(c_m, heads_msa)
    return w


def synthetic_global_attention_weights(c_m: int, heads: int, seed: int = 5) -> dict:
    """Global column attention weights in the layout `encodeGlobalAttention` uploads
    (`webgpu/af2/evoformer/block.js:963-980`): queryWeight [C, H*d], key/value [C, d] with
    d = C / heads, gating [C, H*d] + bias, output [H*d, C] + bias, all (in,out)."""
    s = Stream(seed)
    noise = s.values
    d = c_m // heads
    r = 1.0 / np.sqrt(c_m)
    return {"heads": heads, "attention": {
        "queryNormScale": noise(c_m, 0.2, 1),
        "queryNormOffset": noise(c_m, 0.1),
        "queryWeight": noise(c_m * heads * d, r).reshape(c_m, heads * d),
        "keyWeight": noise(c_m * d, r).reshape(c_m, d),
        "valueWeight": noise(c_m * d, r).reshape(c_m, d),
        "gatingWeight": noise(c_m * heads * d, r).reshape(c_m, heads * d),
        "gatingBias": noise(heads * d, 0.1, 1),
        "outputWeight": noise(heads * d * c_m, 1 / np.sqrt(heads * d)).reshape(heads * d, c_m),
        "outputBias": noise(c_m, 0.05),
    }}


def synthetic_extra_msa_block_weights(c_m: int = 64, c_z: int = 128, c_outer: int = 32, heads_msa: int = 8,
                                      heads_pair: int = 4, tri_hidden: int = 128, msa_hidden: int = 256,
                                      pair_hidden: int = 512, seed: int = 11) -> dict:
    """An AF2 extra-MSA block (`encodeExtraMsaBlock`, `webgpu/af2/evoformer/block.js:1715-1744`):
    the main block's weights with `msaColumnGlobalAttention` in place of `msaColumnAttention`
    (AF2 extra MSA: c_m 64, 8 heads of 8)."""
    w = synthetic_block_weights(c_m, c_z, c_outer, heads_msa, heads_pair, tri_hidden, msa_hidden, pair_hidden, seed)
    del w["msaColumnAttention"]
    w["msaColumnGlobalAttention"] = synthetic_global_attention_weights(c_m, heads_msa, seed + 1000)
    return w


def synthetic_activations(sequences: int, length: int, c_m: int, c_z: int, seed: int = 9) -> dict:
    """`syntheticActivations` (`tools/gpu/af2-synthetic-block.js:141-162`)."""
    s = Stream(seed)
    msa_mask = np.ones((sequences, length), np.float32)
    if sequences > 1 and length > 1:
        msa_mask[sequences - 1, 1] = 0
    pair_mask = np.ones(length * length, np.float32)
    if length > 1:
        pair_mask[2 % (length * length)] = 0
        pair_mask[max(length * length - 3, 0)] = 0
    msa = s.values(sequences * length * c_m, 1.5).reshape(sequences, length, c_m)
    pair = s.values(length * length * c_z, 1.5).reshape(length, length, c_z)
    return {"msa": msa, "pair": pair, "msaMask": msa_mask, "pairMask": pair_mask.reshape(length, length)}


# ---------------------------------------------------------------------------------------
# Weight quantisers (writers of the codec records shared/weights/dtype.js reads)
# ---------------------------------------------------------------------------------------

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
    """Per-output-channel quantisation (the headline triangle workload's): one group per output column.

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


def quantise_records(w: dict, names, dtype: str, per_channel: bool, out_axis: int) -> dict:
    """A copy of `w` with the named matrices replaced by codec records of `dtype`."""
    recs = dict(w)
    for name in names:
        if dtype == "float32":
            continue
        if dtype == "float16":
            recs[name] = make_record(w[name], "float16")
        elif per_channel:
            recs[name] = make_record(w[name], dtype, channel_axis=out_axis)
        else:
            recs[name] = make_record(w[name], dtype)
    return recs


TRI_MATS = ["linearAPWeight", "linearAGWeight", "linearBPWeight", "linearBGWeight", "linearZWeight", "linearGWeight"]
TRI3_MATS = ["projection", "gate", "outputProjection", "gatingLinear"]


def af3_tri_weights(c, seed):
    s = Stream(seed)
    r = 1.0 / np.sqrt(c)
    return {"leftNormInputScale": s.values(c, 0.2, 1), "leftNormInputOffset": s.values(c, 0.1),
            "projection": s.normal(c * 2 * c, r).reshape(c, 2 * c), "gate": s.normal(c * 2 * c, r).reshape(c, 2 * c),
            "centerNormScale": s.values(c, 0.2, 1), "centerNormOffset": s.values(c, 0.1),
            "outputProjection": s.normal(c * c, r).reshape(c, c), "gatingLinear": s.normal(c * c, r).reshape(c, c)}


def config2_inputs(n=384, c=128, seed=2, masked_tail=16):
    """Headline triangle workload: z ~N(0,1), weights N(0,1/fan_in) masters quantised int5 per output channel,
    mask ones except the last `masked_tail` residues (rows and columns)."""
    s = Stream(seed)
    z = s.normal(n * n * c).reshape(n, n, c)
    mask = np.ones((n, n), np.float32)
    if masked_tail:
        mask[n - masked_tail:, :] = 0
        mask[:, n - masked_tail:] = 0

    def tri(seed_off):
        t = Stream(seed + 100 + seed_off)
        rz = 1.0 / np.sqrt(c)
        return {"layerNormInWeight": t.values(c, 0.2, 1), "layerNormInBias": t.values(c, 0.1),
                "linearAPWeight": t.normal(c * c, rz).reshape(c, c), "linearAPBias": t.values(c, 0.03),
                "linearAGWeight": t.normal(c * c, rz).reshape(c, c), "linearAGBias": t.values(c, 0.03, 1),
                "linearBPWeight": t.normal(c * c, rz).reshape(c, c), "linearBPBias": t.values(c, 0.03),
                "linearBGWeight": t.normal(c * c, rz).reshape(c, c), "linearBGBias": t.values(c, 0.03, 1),
                "layerNormOutWeight": t.values(c, 0.2, 1), "layerNormOutBias": t.values(c, 0.1),
                "linearZWeight": t.normal(c * c, rz).reshape(c, c), "linearZBias": t.values(c, 0.03),
                "linearGWeight": t.normal(c * c, rz).reshape(c, c), "linearGBias": t.values(c, 0.03, 1)}
    w_out, w_in = tri(0), tri(1)
    return {"z": z, "mask": mask, "w_out": w_out, "w_in": w_in,
            "rec_out": quantise_records(w_out, TRI_MATS, "int5", True, 0),
            "rec_in": quantise_records(w_in, TRI_MATS, "int5", True, 0)}


def synthetic_pairformer_weights(c_z, c_s, heads_pair, heads_single, dim_single, seed=3, factor=4):
    """Random-init AF3 pairformer block weights (N(0, 1/fan_in) masters, LN scale ~1).

    The reference has no AF3 synthetic generator; this uses the same `generator(seed)`
    stream with Box-Muller normals (Stream.normal).
    """
    s = Stream(seed)

    def lin(i, o):
        return s.normal(i * o, 1.0 / np.sqrt(i)).reshape(i, o)

    def ln(c):
        return s.values(c, 0.2, 1), s.values(c, 0.1)

    def tri():
        sc, of = ln(c_z)
        cs, co = ln(c_z)
        return {"leftNormInputScale": sc, "leftNormInputOffset": of,
                "projection": lin(c_z, 2 * c_z), "gate": lin(c_z, 2 * c_z),
                "centerNormScale": cs, "centerNormOffset": co,
                "outputProjection": lin(c_z, c_z), "gatingLinear": lin(c_z, c_z)}

    def grid(heads, dim):
        sc, of = ln(c_z)
        w = heads * dim
        return {"heads": heads, "dimension": dim, "actNormScale": sc, "actNormOffset": of,
                "pairBiasProjection": lin(c_z, heads),
                "qProjection": lin(c_z, w).T.copy(), "kProjection": lin(c_z, w).T.copy(),
                "vProjection": lin(c_z, w), "gatingQuery": lin(c_z, w).T.copy(),
                "outputProjection": lin(w, c_z)}

    def trans(c):
        sc, of = ln(c)
        return {"inputLayerNormScale": sc, "inputLayerNormOffset": of,
                "transition1": lin(c, 2 * factor * c), "transition2": lin(factor * c, c)}

    w = {"triangleMultiplicationOutgoing": tri(), "triangleMultiplicationIncoming": tri(),
         "pairAttention1": grid(heads_pair, c_z // heads_pair),
         "pairAttention2": grid(heads_pair, c_z // heads_pair),
         "pairTransition": trans(c_z)}
    sc, of = ln(c_z)
    w["singlePairLogitsNormScale"], w["singlePairLogitsNormOffset"] = sc, of
    w["singlePairLogitsProjection"] = lin(c_z, heads_single)
    sc, of = ln(c_s)
    hw = heads_single * dim_single
    w["singleAttention"] = {"heads": heads_single, "dimension": dim_single,
                            "layerNormScale": sc, "layerNormOffset": of,
                            "qProjection": lin(c_s, hw), "qBias": s.values(hw, 0.1),
                            "kProjection": lin(c_s, hw), "vProjection": lin(c_s, hw),
                            "gatingQuery": lin(c_s, hw), "outputProjection": lin(hw, c_s)}
    w["singleTransition"] = trans(c_s)
    return w


def synthetic_msa_module_weights(c_m: int = 64, c_z: int = 128, heads: int = 8, dim: int = 8,
                                 heads_pair: int = 4, c_outer: int = 32, seed: int = 13, factor: int = 4) -> dict:
    """Random-init AF3 MSA-module block weights (`msaBlock`, `cpu/af3/trunk/msa.js:233-287`): the
    pair-only pairformer block's, plus `msaAttention1` (`msaAttention`, `:157-219`), the SwiGLU
    `msaTransition` and the AF3 `outerProductMean` (`:72-155`); all (in,out), N(0, 1/fan_in)."""
    w = synthetic_pairformer_weights(c_z, 32, heads_pair, 2, 16, seed=seed, factor=factor)
    for key in ("singlePairLogitsNormScale", "singlePairLogitsNormOffset", "singlePairLogitsProjection",
                "singleAttention", "singleTransition"):
        del w[key]
    st = Stream(seed + 1000)

    def lin(i, o):
        return st.normal(i * o, 1.0 / np.sqrt(i)).reshape(i, o)

    hw = heads * dim
    w["msaAttention1"] = {"heads": heads, "dimension": dim,
                          "actNormScale": st.values(c_m, 0.2, 1), "actNormOffset": st.values(c_m, 0.1),
                          "pairNormScale": st.values(c_z, 0.2, 1), "pairNormOffset": st.values(c_z, 0.1),
                          "pairLogits": lin(c_z, heads), "vProjection": lin(c_m, hw),
                          "gatingQuery": lin(c_m, hw), "outputProjection": lin(hw, c_m)}
    w["msaTransition"] = {"inputLayerNormScale": st.values(c_m, 0.2, 1), "inputLayerNormOffset": st.values(c_m, 0.1),
                          "transition1": lin(c_m, 2 * factor * c_m), "transition2": lin(factor * c_m, c_m)}
    w["outerProductMean"] = {"layerNormInputScale": st.values(c_m, 0.2, 1), "layerNormInputOffset": st.values(c_m, 0.1),
                             "leftProjection": lin(c_m, c_outer), "rightProjection": lin(c_m, c_outer),
                             "outputW": st.normal(c_outer * c_outer * c_z, 1.0 / c_outer).reshape(c_outer * c_outer, c_z),
                             "outputB": st.values(c_z, 0.05)}
    return w


def config3_attention_weights(c: int, heads: int, seed: int) -> dict:
    """Triangle-attention workload weights: N(0, 1/fan_in) masters, LN scale ~1."""
    s = Stream(seed)
    r = 1.0 / np.sqrt(c)
    att = {"queryNormScale": s.values(c, 0.2, 1), "queryNormOffset": s.values(c, 0.1),
           "queryWeight": s.normal(c * c, r).reshape(c, c), "keyWeight": s.normal(c * c, r).reshape(c, c),
           "valueWeight": s.normal(c * c, r).reshape(c, c), "gatingWeight": s.normal(c * c, r).reshape(c, c),
           "gatingBias": s.values(c, 0.1, 1), "outputWeight": s.normal(c * c, r).reshape(c, c),
           "outputBias": s.values(c, 0.05)}
    return {"heads": heads, "attention": att,
            "pairBias": {"projectionWeight": s.normal(c * heads, r).reshape(c, heads)}}


def config1_inputs(seed: int = 0, n: int = 64, c_m: int = 256, c_z: int = 128):
    """CPU-path workload: one AF2 Evoformer block, N_res=64, N_seq=1, fp32 weights ~N(0,1/fan_in)
    (LN scales/offsets as `syntheticBlockWeights`), msa/pair ~N(0,1).  Returns (weights, msa, pair)."""
    w = synthetic_block_weights(c_m=c_m, c_z=c_z, c_outer=32, heads_msa=8, heads_pair=4, tri_hidden=128,
                                msa_hidden=4 * c_m, pair_hidden=4 * c_z, seed=seed + 1)
    s = Stream(seed)

    def renorm(d):
        for k, v in list(d.items()):
            if isinstance(v, dict):
                renorm(v)
            elif isinstance(v, np.ndarray) and v.ndim == 2:
                fan_in = v.shape[1] if k.startswith("linear") else v.shape[0]   # triangle weights are (out,in)
                d[k] = s.normal(v.size, 1.0 / np.sqrt(fan_in)).reshape(v.shape)
    renorm(w)
    msa = s.normal(n * c_m).reshape(1, n, c_m)
    pair = s.normal(n * n * c_z).reshape(n, n, c_z)
    return w, msa, pair


def quantise_tree(w: dict, dtype: str, block: int = 64) -> dict:
    """Every 2-D matrix in a nested block-weight dict replaced by a flat-group codec record."""
    out = {}
    for k, v in w.items():
        if isinstance(v, dict):
            out[k] = quantise_tree(v, dtype, block)
        elif isinstance(v, np.ndarray) and v.ndim == 2:
            out[k] = make_record(v, dtype, block=block)
        else:
            out[k] = v
    return out


def config3_inputs(n: int = 512, c: int = 128, heads: int = 4, seed: int = 33):
    """Triangle-attention workload: fp16 pair ~N(0,1), fp16 weights ~N(0,1/fan_in) for starting and ending
    node attention, key padding with the last 5% of residues masked (rows and columns)."""
    s = Stream(seed)
    pair = s.normal(n * n * c).reshape(n, n, c)
    masked = int(round(0.05 * n))
    mask = np.ones((n, n), np.float32)
    mask[:, n - masked:] = 0
    mask[n - masked:, :] = 0
    mats = ["queryWeight", "keyWeight", "valueWeight", "gatingWeight", "outputWeight"]
    weights = []
    for seed_w in (seed + 8, seed + 9):
        w = config3_attention_weights(c, heads, seed_w)
        weights.append(dict(w, attention=quantise_records(w["attention"], mats, "float16", False, 1),
                            pairBias={"projectionWeight": make_record(w["pairBias"]["projectionWeight"], "float16")}))
    return {"pair": pair, "mask": mask, "starting": weights[0], "ending": weights[1], "masked": masked}


def config4_inputs(n: int = 384, sequences: int = 512, c_m: int = 256, c_z: int = 128, seed: int = 4,
                   block: int = 64):
    """AF2 Evoformer workload, one block's inputs: an MSA of random tokens over 21 classes (gap
    probability 0.2, the first row the gap-free query) embedded through a random N(0,1) table,
    pair ~N(0,1), block weights ~N(0,1/fan_in) quantised to int8 with fp16 scales (flat groups
    of `block`).  Masks are all ones (no padding)."""
    w, _, _ = config1_inputs(seed=seed, n=1, c_m=c_m, c_z=c_z)
    s = Stream(seed + 50)
    u = s.uniform(sequences * n).reshape(sequences, n)
    aa = np.minimum((s.uniform(sequences * n) * 20).astype(np.int64), 19).reshape(sequences, n)
    tokens = np.where(u < 0.2, 20, aa)
    tokens[0] = aa[0]
    table = s.normal(21 * c_m).reshape(21, c_m).astype(np.float32)
    msa = table[tokens]
    pair = s.normal(n * n * c_z).reshape(n, n, c_z)
    return {"weights": quantise_tree(w, "int8", block), "msa": msa, "pair": pair, "tokens": tokens,
            "msa_mask": np.ones((sequences, n), np.float32), "pair_mask": np.ones((n, n), np.float32)}


def synthetic_input_embedder(length: int, msa_sequences: int, extra_sequences: int, c_m: int = 256,
                             c_z: int = 128, c_e: int = 64, target_channels: int = 22,
                             msa_feature_channels: int = 49, seed: int = 17) -> tuple:
    """Random-init AF2 input-embedder weights (`InputEmbedderGpu`, webgpu/af2/evoformer/
    input-embedder.js:9-26, all (in,out) f32) and features of the shapes it reads: one-hot
    target features, msa features, extra codes 0..22 with deletion features, residue indices
    with a chain gap, aatype and atom37 positions.  Returns (weights, features)."""
    st = Stream(seed)

    def lin(i, o):
        return st.normal(i * o, 1.0 / np.sqrt(i)).reshape(i, o).astype(np.float32)

    w = {"preprocess1dWeight": lin(target_channels, c_m), "preprocess1dBias": st.values(c_m, 0.1),
         "preprocessMsaWeight": lin(msa_feature_channels, c_m), "preprocessMsaBias": st.values(c_m, 0.1),
         "leftSingleWeight": lin(target_channels, c_z), "leftSingleBias": st.values(c_z, 0.1),
         "rightSingleWeight": lin(target_channels, c_z), "rightSingleBias": st.values(c_z, 0.1),
         "previousPositionWeight": lin(15, c_z), "previousPositionBias": st.values(c_z, 0.1),
         "previousMsaNormScale": st.values(c_m, 0.2, 1), "previousMsaNormOffset": st.values(c_m, 0.1),
         "previousPairNormScale": st.values(c_z, 0.2, 1), "previousPairNormOffset": st.values(c_z, 0.1),
         "relativePositionWeight": lin(65, c_z), "relativePositionBias": st.values(c_z, 0.1),
         "extraMsaWeight": lin(25, c_e), "extraMsaBias": st.values(c_e, 0.1)}
    rng = np.random.default_rng(seed)
    aatype = rng.integers(0, 20, length)
    target = np.zeros((length, target_channels), np.float32)
    target[np.arange(length), aatype + 1] = 1
    msa_feat = (rng.random((msa_sequences, length, msa_feature_channels)) < 0.1).astype(np.float32)
    msa_feat[..., 48] = rng.random((msa_sequences, length))
    residue_index = np.arange(length, dtype=np.float32)
    residue_index[length // 2:] += 200            # a chain break: offsets past +-32 clip
    positions = np.cumsum(rng.normal(0, 2.2, (length, 37, 3)), axis=0).astype(np.float32)
    f = {"targetFeatures": target, "msaFeatures": msa_feat,
         "extraMsa": rng.integers(0, 23, (extra_sequences, length)).astype(np.float32),
         "extraHasDeletion": (rng.random((extra_sequences, length)) < 0.2).astype(np.float32),
         "extraDeletionValue": rng.random((extra_sequences, length)).astype(np.float32),
         "residueIndex": residue_index, "aatype": aatype.astype(np.float32),
         "previousMsaFirstRow": rng.normal(0, 1, (length, c_m)).astype(np.float32),
         "previousPair": rng.normal(0, 1, (length, length, c_z)).astype(np.float32),
         "previousPositions": positions}
    return w, f
