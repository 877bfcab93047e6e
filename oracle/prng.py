"""The reference's deterministic generator and synthetic inputs, restated in numpy.

`generator(seed)` (`webgpu/testing/deterministic-input.js:1-10`, identical copy in
`tools/gpu/af2-synthetic-block.js:20-29`) is a mulberry32-style integer mixer whose
state advances by the constant 0x6d2b79f5 before every draw.  Draw `i` (0-based) therefore
depends only on `seed + (i+1)*0x6d2b79f5 mod 2^32`, so a whole stream is one vectorised
uint32 computation.  `Math.imul` is the low 32 bits of a product, `>>>` a logical shift,
and the JS `value + imul(...)` followed by `^` wraps mod 2^32 - all of which uint32
numpy arithmetic reproduces bit for bit.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
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


def uniform_sequential(seed: int, count: int) -> np.ndarray:
    """The same stream, one draw at a time in plain Python integers (cross-check only)."""
    state = seed & 0xFFFFFFFF
    out = np.empty(count)
    m = 0xFFFFFFFF
    for i in range(count):
        state = (state + 0x6D2B79F5) & m
        v = state
        v = ((v ^ (v >> 15)) * (v | 1)) & m
        v = (v ^ ((v + (((v ^ (v >> 7)) * (v | 61)) & m)) & m)) & m
        out[i] = ((v ^ (v >> 14)) & m) / 4294967296.0
    return out


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

        The reference has no normal sampler; this is the transform the BASELINE configs
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
