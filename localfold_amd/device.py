"""Python host over the C ABI, with torch as the device-memory plumbing.

torch supplies device tensors and the stream; every computation goes through
liblocalfold.so.  The op helpers mirror the reference classes' inputs
(`webgpu/kernels/triangle/types.js`, `webgpu/kernels/attention.js:15-57`,
`webgpu/kernels/transition.js:445-460`, `webgpu/kernels/outer-product-mean.js:38-70`):
numpy weight dicts keyed by the reference's names, uploaded once into DeviceWeights.

A weight value is either a numpy array (float32 values) or a record dict
{dtype: "float32"|"float16"|"bfloat16"|"int8"|"int5", shape, data, scales?, zeros?,
 block | channel_axis} (the codec records of shared/weights/dtype.js).
"""
import ctypes as C
import functools

import numpy as np
import torch

from . import capi
from .capi import check

_DTYPE_CODE = {"float32": capi.LF_F32, "float16": capi.LF_F16, "bfloat16": capi.LF_BF16,
               "int8": capi.LF_INT8, "int5": capi.LF_INT5}
_TORCH_ACT = {torch.float32: capi.LF_F32, torch.float16: capi.LF_F16, torch.bfloat16: capi.LF_BF16}


def act_code(t: torch.Tensor) -> int:
    if t.dtype not in _TORCH_ACT:
        raise TypeError(f"activation dtype {t.dtype} is not float32/float16/bfloat16")
    return _TORCH_ACT[t.dtype]


def _owned(build):
    """The struct a weight builder returns points into its DeviceWeights' device buffers: it
    keeps that DeviceWeights alive (weights built from a temporary stay valid)."""
    @functools.wraps(build)
    def wrapped(dw, *args, **kwargs):
        struct = build(dw, *args, **kwargs)
        struct._owner = dw
        return struct
    return wrapped


def ptr(t) -> int:
    return None if t is None else t.data_ptr()


class Context:
    """An lf_context bound to torch's current stream on `device`."""

    def __init__(self, device: int = 0):
        self.lib = capi.load()
        if not torch.cuda.is_available():
            raise capi.LocalfoldError("no GPU: liblocalfold needs a HIP device (there is no CPU fallback)")
        self.device = torch.device("cuda", device)
        torch.cuda.set_device(self.device)
        h = self.lib.lf_context_create(device)
        if not h:
            raise capi.LocalfoldError(self.lib.lf_last_error().decode())
        self.handle = C.c_void_p(h)
        self.bind_stream()

    def bind_stream(self, stream=None):
        s = stream or torch.cuda.current_stream(self.device)
        check(self.lib.lf_context_set_stream(self.handle, C.c_void_p(s.cuda_stream)))

    def close(self):
        if getattr(self, "handle", None):
            self.lib.lf_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        check(self.lib.lf_synchronize(self.handle))

    def profile(self, enable: bool = True):
        check(self.lib.lf_profile_enable(self.handle, int(enable)))

    def read_profile(self, max_records: int = 4096):
        buf = (capi.lf_kernel_timing * max_records)()
        n = self.lib.lf_profile_read(self.handle, buf, max_records)
        if n < 0:
            check(-n)
        return [(buf[i].label.decode(), float(buf[i].ms)) for i in range(n)]

    def memory_stats(self):
        cur, peak, cnt = C.c_size_t(), C.c_size_t(), C.c_size_t()
        check(self.lib.lf_memory_stats(self.handle, C.byref(cur), C.byref(peak), C.byref(cnt)))
        return {"currentBytes": cur.value, "peakBytes": peak.value, "allocationCount": cnt.value}


class DeviceWeights:
    """Uploads weight records / vectors and keeps the tensors alive while structs point at them."""

    def __init__(self, device):
        self.device = device
        self.keep = []

    def vec(self, x):
        if x is None:
            return None
        t = torch.as_tensor(np.ascontiguousarray(np.asarray(x, np.float32)).reshape(-1)).to(self.device)
        self.keep.append(t)
        return t.data_ptr()

    def _tensor(self, arr, dtype=None):
        a = np.ascontiguousarray(arr)
        t = torch.from_numpy(a.view(np.uint8).copy() if dtype is None else a).to(self.device)
        self.keep.append(t)
        return t.data_ptr()

    def weight(self, value, layout: int, dtype_override: str = None) -> capi.lf_weight:
        """lf_weight for a numpy array (float32) or a codec record, in the given stored layout."""
        rec = value if isinstance(value, dict) else {"dtype": "float32", "data": np.asarray(value, np.float32),
                                                     "shape": list(np.shape(value))}
        if dtype_override and rec["dtype"] == "float32":
            rec = dict(rec, dtype=dtype_override)
        shape = list(rec["shape"])
        if len(shape) != 2:
            raise ValueError(f"weights must be 2-D, got shape {shape}")
        if "layout" in rec:   # a record that names its stored layout (a bundle's [in][out] codes)
            layout = {"in_out": capi.LF_IN_OUT, "out_in": capi.LF_OUT_IN}[rec["layout"]]
        w = capi.lf_weight()
        w.dtype = _DTYPE_CODE[rec["dtype"]]
        w.layout = layout
        w.rows, w.cols = shape
        dt = rec["dtype"]
        if dt == "float32":
            w.data = self._tensor(np.asarray(rec["data"], np.float32))
        elif dt == "float16":
            w.data = self._tensor(np.asarray(rec["data"], np.float32).astype(np.float16))
        elif dt == "bfloat16":
            t = torch.as_tensor(np.asarray(rec["data"], np.float32)).to(torch.bfloat16).to(self.device)
            self.keep.append(t)
            w.data = t.data_ptr()
        else:
            codes = np.asarray(rec["data"])
            if dt == "int5":   # the kernels' aligned word-pair fetch reads <= 3 bytes past the codes
                codes = np.concatenate([codes.view(np.uint8).reshape(-1), np.zeros(4, np.uint8)])
            w.data = self._tensor(codes)
            w.scales = self._tensor(np.asarray(rec["scales"], np.float16))
            if rec.get("zeros") is not None:
                w.zeros = self._tensor(np.asarray(rec["zeros"], np.float16))
            if "channel_axis" in rec:
                out_axis = 1 if layout == capi.LF_IN_OUT else 0
                if rec["channel_axis"] != out_axis:
                    raise ValueError("per-channel quantisation must be along the output axis")
                w.group = 0
            else:
                w.group = int(rec["block"])
        return w


# ---------------------------------------------------------------------------------------
# Triangle multiplication
# ---------------------------------------------------------------------------------------

@_owned
def tri_mult_weights(dw: DeviceWeights, w: dict, dialect: int = capi.LF_AF2) -> capi.lf_tri_mult_weights:
    """Struct for the reference's weight names.

    AF2: the sixteen (out,in) tensors of `webgpu/kernels/triangle/types.js:28-43`.
    AF3: leftNormInputScale/Offset, projection, gate, centerNormScale/Offset,
    outputProjection, gatingLinear (all (in,out), `cpu/af3/trunk/pairformer.js:213-300`).
    """
    s = capi.lf_tri_mult_weights()
    if dialect == capi.LF_AF2:
        s.ln_in_scale, s.ln_in_offset = dw.vec(w["layerNormInWeight"]), dw.vec(w["layerNormInBias"])
        s.ap = dw.weight(w["linearAPWeight"], capi.LF_OUT_IN)
        s.ag = dw.weight(w["linearAGWeight"], capi.LF_OUT_IN)
        s.bp = dw.weight(w["linearBPWeight"], capi.LF_OUT_IN)
        s.bg = dw.weight(w["linearBGWeight"], capi.LF_OUT_IN)
        s.ap_bias, s.ag_bias = dw.vec(w["linearAPBias"]), dw.vec(w["linearAGBias"])
        s.bp_bias, s.bg_bias = dw.vec(w["linearBPBias"]), dw.vec(w["linearBGBias"])
        s.ln_out_scale, s.ln_out_offset = dw.vec(w["layerNormOutWeight"]), dw.vec(w["layerNormOutBias"])
        s.wz = dw.weight(w["linearZWeight"], capi.LF_OUT_IN)
        s.wz_bias = dw.vec(w["linearZBias"])
        s.wg = dw.weight(w["linearGWeight"], capi.LF_OUT_IN)
        s.wg_bias = dw.vec(w["linearGBias"])
    else:
        s.ln_in_scale, s.ln_in_offset = dw.vec(w["leftNormInputScale"]), dw.vec(w["leftNormInputOffset"])
        s.ap = dw.weight(w["projection"], capi.LF_IN_OUT)
        s.ag = dw.weight(w["gate"], capi.LF_IN_OUT)
        s.ln_out_scale, s.ln_out_offset = dw.vec(w["centerNormScale"]), dw.vec(w["centerNormOffset"])
        s.wz = dw.weight(w["outputProjection"], capi.LF_IN_OUT)
        s.wg = dw.weight(w["gatingLinear"], capi.LF_IN_OUT)
    return s


def tri_mult(ctx: Context, z: torch.Tensor, mask: torch.Tensor, wstruct: capi.lf_tri_mult_weights,
             direction: str = "outgoing", dialect: int = capi.LF_AF2, out: torch.Tensor = None,
             accumulate: bool = False, epsilon: float = 1e-5, divide_by_length: bool = False,
             noalloc: bool = False) -> torch.Tensor:
    """One triangle multiplicative update through lf_tri_mult, or, with noalloc, through
    lf_tri_mult_noalloc (the library's static scratch; `out` must then be given by callers
    that cannot allocate)."""
    n, n2, cz = z.shape
    if n != n2 or tuple(mask.shape) != (n, n) or mask.dtype != torch.float32:
        raise ValueError("z must be [N, N, cZ] and mask [N, N] float32")
    if out is None:
        out = torch.empty_like(z)
    a = capi.lf_tri_mult_args()
    a.direction = capi.LF_OUTGOING if direction == "outgoing" else capi.LF_INCOMING
    a.dialect = dialect
    a.divide_by_length = int(divide_by_length)
    a.length, a.c_z = n, cz
    a.c_hidden = wstruct.wz.cols if wstruct.wz.layout == capi.LF_OUT_IN else wstruct.wz.rows
    a.act_dtype = act_code(z)
    a.z, a.mask, a.out = ptr(z), ptr(mask), ptr(out)
    a.accumulate = int(accumulate)
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    fn = ctx.lib.lf_tri_mult_noalloc if noalloc else ctx.lib.lf_tri_mult
    check(fn(ctx.handle, C.byref(a)))
    return out


# ---------------------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------------------

@_owned
def attention_weights_af2(dw: DeviceWeights, w: dict, pair_bias: dict = None) -> capi.lf_attention_weights:
    """AF2 gated attention (`webgpu/kernels/attention.js:15-57`): (in,out) weights;
    pair_bias: {layerNormScale, layerNormOffset, projectionWeight} (separate pair tensor) or
    {projectionWeight} (bias from the normalised input)."""
    s = capi.lf_attention_weights()
    s.norm_scale, s.norm_offset = dw.vec(w["queryNormScale"]), dw.vec(w["queryNormOffset"])
    s.wq = dw.weight(w["queryWeight"], capi.LF_IN_OUT)
    s.wk = dw.weight(w["keyWeight"], capi.LF_IN_OUT)
    s.wv = dw.weight(w["valueWeight"], capi.LF_IN_OUT)
    s.wg = dw.weight(w["gatingWeight"], capi.LF_IN_OUT)
    s.wo = dw.weight(w["outputWeight"], capi.LF_IN_OUT)
    s.g_bias, s.o_bias = dw.vec(w["gatingBias"]), dw.vec(w["outputBias"])
    if pair_bias is not None:
        s.wb = dw.weight(pair_bias["projectionWeight"], capi.LF_IN_OUT)
        if "layerNormScale" in pair_bias:
            s.pair_norm_scale = dw.vec(pair_bias["layerNormScale"])
            s.pair_norm_offset = dw.vec(pair_bias["layerNormOffset"])
    return s


@_owned
def attention_weights_af3_grid(dw: DeviceWeights, w: dict) -> capi.lf_attention_weights:
    """AF3 grid attention (`cpu/af3/trunk/pairformer.js:322-431`): q/k/gate (out,in), v/output (in,out)."""
    s = capi.lf_attention_weights()
    s.norm_scale, s.norm_offset = dw.vec(w["actNormScale"]), dw.vec(w["actNormOffset"])
    s.wq = dw.weight(w["qProjection"], capi.LF_OUT_IN)
    s.wk = dw.weight(w["kProjection"], capi.LF_OUT_IN)
    s.wv = dw.weight(w["vProjection"], capi.LF_IN_OUT)
    s.wg = dw.weight(w["gatingQuery"], capi.LF_OUT_IN)
    s.wo = dw.weight(w["outputProjection"], capi.LF_IN_OUT)
    s.g_bias = dw.vec(w.get("gatingQueryBias"))
    s.o_bias = dw.vec(w.get("outputProjectionBias"))
    s.wb = dw.weight(w["pairBiasProjection"], capi.LF_IN_OUT)
    return s


@_owned
def attention_weights_af3_single(dw: DeviceWeights, w: dict, norm_scale, norm_offset, projection) -> capi.lf_attention_weights:
    """AF3 single attention (`cpu/af3/trunk/pairformer.js:446-485`) with the pair-logits LN and
    projection of `pairformerBlock` (`:516-537`) as a separate pair bias."""
    s = capi.lf_attention_weights()
    s.norm_scale, s.norm_offset = dw.vec(w["layerNormScale"]), dw.vec(w["layerNormOffset"])
    s.wq = dw.weight(w["qProjection"], capi.LF_IN_OUT)
    s.wk = dw.weight(w["kProjection"], capi.LF_IN_OUT)
    s.wv = dw.weight(w["vProjection"], capi.LF_IN_OUT)
    s.wg = dw.weight(w["gatingQuery"], capi.LF_IN_OUT)
    s.wo = dw.weight(w["outputProjection"], capi.LF_IN_OUT)
    s.q_bias = dw.vec(w["qBias"])
    s.pair_norm_scale, s.pair_norm_offset = dw.vec(norm_scale), dw.vec(norm_offset)
    s.wb = dw.weight(projection, capi.LF_IN_OUT)
    return s


def attention(ctx: Context, act: torch.Tensor, mask: torch.Tensor, wstruct: capi.lf_attention_weights, heads: int,
              transpose: bool = False, bias_mode: int = capi.LF_BIAS_NONE, pair: torch.Tensor = None,
              head_dim: int = 0, fast_variance: bool = False, swap_bias: bool = False, out: torch.Tensor = None,
              accumulate: bool = False, epsilon: float = 1e-5, bias_logits: torch.Tensor = None) -> torch.Tensor:
    """act: storage [batch, queries, C] ([queries, batch, C] when transpose); mask: storage [.., ..]."""
    d0, d1, c = act.shape
    batch, queries = (d1, d0) if transpose else (d0, d1)
    if tuple(mask.shape) != (d0, d1) or mask.dtype != torch.float32:
        raise ValueError("mask must be float32 with the activation's storage shape")
    if out is None:
        out = torch.empty_like(act)
    a = capi.lf_attention_args()
    a.batch, a.queries, a.channels, a.heads, a.head_dim = batch, queries, c, heads, head_dim
    a.transpose = int(transpose)
    a.act_dtype = act_code(act)
    a.act, a.mask, a.out = ptr(act), ptr(mask), ptr(out)
    a.accumulate = int(accumulate)
    a.fast_variance = int(fast_variance)
    a.bias_mode = bias_mode
    a.swap_bias = int(swap_bias)
    if pair is not None:
        a.pair_dtype = act_code(pair)
        a.pair = ptr(pair)
        a.pair_channels = pair.shape[-1]
    a.bias_logits = ptr(bias_logits)
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_attention(ctx.handle, C.byref(a)))
    return out


# ---------------------------------------------------------------------------------------
# Transition and outer product mean
# ---------------------------------------------------------------------------------------

@_owned
def transition_weights(dw: DeviceWeights, w: dict, kind: int = capi.LF_TRANSITION_RELU) -> capi.lf_transition_weights:
    """AF2 (`webgpu/kernels/transition.js:445-460`): layerNormScale/Offset, firstWeight [C,H],
    firstBias, secondWeight [H,C], secondBias.  AF3 SwiGLU (`cpu/af3/trunk/pairformer.js:180-201`):
    inputLayerNormScale/Offset, transition1 [C,2H], transition2 [H,C]."""
    s = capi.lf_transition_weights()
    if kind == capi.LF_TRANSITION_RELU:
        s.norm_scale, s.norm_offset = dw.vec(w["layerNormScale"]), dw.vec(w["layerNormOffset"])
        s.w1, s.b1 = dw.weight(w["firstWeight"], capi.LF_IN_OUT), dw.vec(w["firstBias"])
        s.w2, s.b2 = dw.weight(w["secondWeight"], capi.LF_IN_OUT), dw.vec(w["secondBias"])
    else:
        s.norm_scale, s.norm_offset = dw.vec(w["inputLayerNormScale"]), dw.vec(w["inputLayerNormOffset"])
        s.w1 = dw.weight(w["transition1"], capi.LF_IN_OUT)
        s.w2 = dw.weight(w["transition2"], capi.LF_IN_OUT)
    return s


def transition(ctx: Context, x: torch.Tensor, wstruct: capi.lf_transition_weights, hidden: int,
               kind: int = capi.LF_TRANSITION_RELU, out: torch.Tensor = None, accumulate: bool = False,
               fast_variance: bool = False, chunk_bytes: int = 0, epsilon: float = 1e-5) -> torch.Tensor:
    if out is None:
        out = torch.empty_like(x)
    a = capi.lf_transition_args()
    a.kind = kind
    a.channels = x.shape[-1]
    a.rows = x.numel() // a.channels
    a.hidden = hidden
    a.act_dtype = act_code(x)
    a.act, a.out = ptr(x), ptr(out)
    a.accumulate = int(accumulate)
    a.fast_variance = int(fast_variance)
    a.chunk_bytes = chunk_bytes
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_transition(ctx.handle, C.byref(a)))
    return out


@_owned
def opm_weights(dw: DeviceWeights, w: dict, dialect: int = capi.LF_AF2) -> capi.lf_opm_weights:
    """AF2 (`webgpu/kernels/outer-product-mean.js:38-85`): layerNormScale/Offset, leftWeight,
    leftBias, rightWeight, rightBias, outputWeight [c*c, cZ], outputBias.  AF3
    (`cpu/af3/trunk/msa.js:72-155`): layerNormInputScale/Offset, leftProjection,
    rightProjection, outputW, outputB."""
    s = capi.lf_opm_weights()
    if dialect == capi.LF_AF2:
        s.norm_scale, s.norm_offset = dw.vec(w["layerNormScale"]), dw.vec(w["layerNormOffset"])
        s.wl, s.bl = dw.weight(w["leftWeight"], capi.LF_IN_OUT), dw.vec(w["leftBias"])
        s.wr, s.br = dw.weight(w["rightWeight"], capi.LF_IN_OUT), dw.vec(w["rightBias"])
        s.wo, s.bo = dw.weight(w["outputWeight"], capi.LF_IN_OUT), dw.vec(w["outputBias"])
    else:
        s.norm_scale, s.norm_offset = dw.vec(w["layerNormInputScale"]), dw.vec(w["layerNormInputOffset"])
        s.wl = dw.weight(w["leftProjection"], capi.LF_IN_OUT)
        s.wr = dw.weight(w["rightProjection"], capi.LF_IN_OUT)
        s.wo, s.bo = dw.weight(w["outputW"], capi.LF_IN_OUT), dw.vec(w.get("outputB"))
    return s


def outer_product_mean(ctx: Context, msa: torch.Tensor, mask: torch.Tensor, wstruct: capi.lf_opm_weights,
                       c_outer: int, c_z: int, pair: torch.Tensor = None, out: torch.Tensor = None,
                       accumulate: bool = False, fast_variance: bool = False, epsilon: float = 1e-5,
                       norm_epsilon: float = 1e-3) -> torch.Tensor:
    s_, n, cm = msa.shape
    if out is None:
        out = torch.empty((n, n, c_z), dtype=pair.dtype if pair is not None else msa.dtype, device=msa.device)
    a = capi.lf_opm_args()
    a.sequences, a.length, a.c_m, a.c_outer, a.c_z = s_, n, cm, c_outer, c_z
    a.msa_dtype = act_code(msa)
    a.msa, a.mask = ptr(msa), ptr(mask)
    a.pair_dtype = act_code(out)
    a.pair_in = ptr(pair)
    a.out = ptr(out)
    a.accumulate = int(accumulate)
    a.fast_variance = int(fast_variance)
    a.epsilon, a.norm_epsilon = epsilon, norm_epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_outer_product_mean(ctx.handle, C.byref(a)))
    return out


@_owned
def global_attention_weights(dw: DeviceWeights, w: dict) -> capi.lf_global_attention_weights:
    """Global column attention (`encodeGlobalAttention`, `webgpu/af2/evoformer/block.js:963-980`):
    queryNorm, queryWeight [C, H*d], keyWeight / valueWeight [C, d], gatingWeight [C, H*d] +
    gatingBias, outputWeight [H*d, C] + outputBias, all (in,out)."""
    s = capi.lf_global_attention_weights()
    s.norm_scale, s.norm_offset = dw.vec(w["queryNormScale"]), dw.vec(w["queryNormOffset"])
    s.wq = dw.weight(w["queryWeight"], capi.LF_IN_OUT)
    s.wk = dw.weight(w["keyWeight"], capi.LF_IN_OUT)
    s.wv = dw.weight(w["valueWeight"], capi.LF_IN_OUT)
    s.wg = dw.weight(w["gatingWeight"], capi.LF_IN_OUT)
    s.g_bias = dw.vec(w["gatingBias"])
    s.wo = dw.weight(w["outputWeight"], capi.LF_IN_OUT)
    s.o_bias = dw.vec(w.get("outputBias"))
    return s


def global_column_attention(ctx: Context, msa: torch.Tensor, mask: torch.Tensor,
                            wstruct: capi.lf_global_attention_weights, heads: int, out: torch.Tensor = None,
                            accumulate: bool = False, head_dim: int = 0, epsilon: float = 1e-5) -> torch.Tensor:
    """msa [S, N, C], mask [S, N]: the update (or msa + update with accumulate) into `out`."""
    s_, n, c = msa.shape
    if out is None:
        out = torch.empty_like(msa)
    a = capi.lf_global_attention_args()
    a.sequences, a.length, a.channels, a.heads, a.head_dim = s_, n, c, heads, head_dim
    a.act_dtype, a.act, a.mask, a.out = act_code(msa), ptr(msa), ptr(mask), ptr(out)
    a.accumulate = int(accumulate)
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_global_column_attention(ctx.handle, C.byref(a)))
    return out


# ---------------------------------------------------------------------------------------
# Blocks
# ---------------------------------------------------------------------------------------

@_owned
def evoformer_weights(dw: DeviceWeights, w: dict) -> capi.lf_evoformer_weights:
    """lf_evoformer_weights from the `syntheticBlockWeights` / AlphaFoldFixture structure
    (`tools/gpu/af2-synthetic-block.js:36-138`)."""
    s = capi.lf_evoformer_weights()
    row = w["msaRowAttention"]
    s.row_attention = attention_weights_af2(dw, row["attention"], row["pairBias"])
    s.row_heads = row["heads"]
    col = w.get("msaColumnAttention")   # absent in an extra-MSA block (global attention instead)
    if col is not None:
        s.column_attention = attention_weights_af2(dw, col["attention"])
        s.column_heads = col["heads"]
    s.msa_transition = transition_weights(dw, w["msaTransition"])
    s.outer_product_mean = opm_weights(dw, w["outerProductMean"])
    s.tri_out = tri_mult_weights(dw, w["triangleMultiplicationOutgoing"])
    s.tri_in = tri_mult_weights(dw, w["triangleMultiplicationIncoming"])
    st, en = w["triangleAttentionStarting"], w["triangleAttentionEnding"]
    s.tri_att_start = attention_weights_af2(dw, st["attention"], st["pairBias"])
    s.tri_att_start_heads = st["heads"]
    s.tri_att_end = attention_weights_af2(dw, en["attention"], en["pairBias"])
    s.tri_att_end_heads = en["heads"]
    s.pair_transition = transition_weights(dw, w["pairTransition"])
    return s


def evoformer_block_args(msa: torch.Tensor, pair: torch.Tensor, msa_mask: torch.Tensor, pair_mask: torch.Tensor,
                         w: dict, epsilon: float = 1e-5) -> capi.lf_evoformer_block_args:
    s_, n, cm = msa.shape
    a = capi.lf_evoformer_block_args()
    a.sequences, a.length, a.c_m, a.c_z = s_, n, cm, pair.shape[-1]
    a.c_outer = np.shape(_plain(w["outerProductMean"]["leftWeight"]))[1]
    a.tri_hidden = _out_dim(w["triangleMultiplicationOutgoing"]["linearAPWeight"], out_axis=0)
    a.msa_hidden = np.shape(_plain(w["msaTransition"]["firstWeight"]))[1]
    a.pair_hidden = np.shape(_plain(w["pairTransition"]["firstWeight"]))[1]
    a.msa_dtype, a.msa = act_code(msa), ptr(msa)
    a.pair_dtype, a.pair = act_code(pair), ptr(pair)
    a.msa_mask, a.pair_mask = ptr(msa_mask), ptr(pair_mask)
    a.epsilon = epsilon
    return a


def _plain(v):
    return np.zeros(v["shape"]) if isinstance(v, dict) else v


def _out_dim(v, out_axis: int) -> int:
    """Output width of a weight whose arrays are stored with the output on `out_axis`; a record
    naming its own layout (a bundle's [in][out] codes) says where its output axis is."""
    shape = np.shape(_plain(v))
    if isinstance(v, dict) and "layout" in v:
        out_axis = 1 if v["layout"] == "in_out" else 0
    return shape[out_axis]


def evoformer_block(ctx: Context, msa, pair, msa_mask, pair_mask, wstruct, w: dict, epsilon: float = 1e-5):
    """One AF2 Evoformer block, msa and pair updated in place."""
    a = evoformer_block_args(msa, pair, msa_mask, pair_mask, w, epsilon)
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_evoformer_block(ctx.handle, C.byref(a)))


def evoformer_stack(ctx: Context, msa, pair, msa_mask, pair_mask, wstructs, w0: dict, epsilon: float = 1e-5):
    """`len(wstructs)` blocks in order (EvoformerStackGpu.run), msa and pair updated in place."""
    a = evoformer_block_args(msa, pair, msa_mask, pair_mask, w0, epsilon)
    arr = (capi.lf_evoformer_weights * len(wstructs))(*wstructs)
    check(ctx.lib.lf_evoformer_stack(ctx.handle, C.byref(a), arr, len(wstructs)))


def evoformer_pair_stack(ctx: Context, msa, pair, msa_mask, pair_mask, wstructs, w0: dict, epsilon: float = 1e-5):
    """`len(wstructs)` pair halves of Evoformer blocks (ExtraMsaPairStackGpu.run): OPM of the
    unchanged msa, triangle multiplication out/in, triangle attention start/end, pair
    transition; the pair is updated in place, the msa is only read."""
    a = evoformer_block_args(msa, pair, msa_mask, pair_mask, w0, epsilon)
    arr = (capi.lf_evoformer_weights * len(wstructs))(*wstructs)
    check(ctx.lib.lf_evoformer_pair_stack(ctx.handle, C.byref(a), arr, len(wstructs)))


@_owned
def extra_msa_weights(dw: DeviceWeights, w: dict) -> capi.lf_extra_msa_weights:
    """An extra-MSA block's weights: the Evoformer structure with `msaColumnGlobalAttention`."""
    s = capi.lf_extra_msa_weights()
    s.base = evoformer_weights(dw, w)
    g = w["msaColumnGlobalAttention"]
    s.column_global = global_attention_weights(dw, g["attention"])
    s.column_global_heads = g["heads"]
    return s


def extra_msa_block(ctx: Context, msa, pair, msa_mask, pair_mask, wstruct, w: dict, epsilon: float = 1e-5):
    """One AF2 extra-MSA block (`encodeExtraMsaBlock`), msa and pair updated in place."""
    a = evoformer_block_args(msa, pair, msa_mask, pair_mask, w, epsilon)
    check(ctx.lib.lf_extra_msa_block(ctx.handle, C.byref(a), C.byref(wstruct)))


def extra_msa_stack(ctx: Context, msa, pair, msa_mask, pair_mask, wstructs, w0: dict, epsilon: float = 1e-5):
    """`len(wstructs)` extra-MSA blocks in order (ExtraMsaStackGpu.run), in place."""
    a = evoformer_block_args(msa, pair, msa_mask, pair_mask, w0, epsilon)
    arr = (capi.lf_extra_msa_weights * len(wstructs))(*wstructs)
    check(ctx.lib.lf_extra_msa_stack(ctx.handle, C.byref(a), arr, len(wstructs)))


@_owned
def pairformer_weights(dw: DeviceWeights, w: dict) -> capi.lf_pairformer_weights:
    """From the AF3 block structure of `cpu/af3/trunk/pairformer.js:495-541`."""
    s = capi.lf_pairformer_weights()
    s.tri_out = tri_mult_weights(dw, w["triangleMultiplicationOutgoing"], capi.LF_AF3)
    s.tri_in = tri_mult_weights(dw, w["triangleMultiplicationIncoming"], capi.LF_AF3)
    s.att_start = attention_weights_af3_grid(dw, w["pairAttention1"])
    s.att_end = attention_weights_af3_grid(dw, w["pairAttention2"])
    s.pair_heads = w["pairAttention1"]["heads"]
    s.pair_transition = transition_weights(dw, w["pairTransition"], capi.LF_TRANSITION_SWIGLU)
    s.single_logits_norm_scale = dw.vec(w["singlePairLogitsNormScale"])
    s.single_logits_norm_offset = dw.vec(w["singlePairLogitsNormOffset"])
    s.single_logits_projection = dw.weight(w["singlePairLogitsProjection"], capi.LF_IN_OUT)
    sa = w["singleAttention"]
    s.single_attention = attention_weights_af3_single(dw, sa, None, None, w["singlePairLogitsProjection"])
    s.single_heads, s.single_head_dim = sa["heads"], sa["dimension"]
    s.single_transition = transition_weights(dw, w["singleTransition"], capi.LF_TRANSITION_SWIGLU)
    return s


def pairformer_block(ctx: Context, pair, single, pair_mask, seq_mask, wstruct, swap_transposed_bias=False,
                     divide_by_length=False, transition_chunk_bytes=0, epsilon=1e-5):
    a = capi.lf_pairformer_block_args()
    a.tokens, a.c_z = pair.shape[0], pair.shape[-1]
    a.c_s = single.shape[-1] if single is not None else 0
    a.swap_transposed_bias, a.divide_by_length = int(swap_transposed_bias), int(divide_by_length)
    a.pair_dtype, a.pair = act_code(pair), ptr(pair)
    if single is not None:
        a.single_dtype, a.single = act_code(single), ptr(single)
    a.pair_mask, a.seq_mask = ptr(pair_mask), ptr(seq_mask)
    a.transition_chunk_bytes = transition_chunk_bytes
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_pairformer_block(ctx.handle, C.byref(a)))


@_owned
def pair_averaging_weights(dw: DeviceWeights, w: dict) -> capi.lf_pair_averaging_weights:
    """AF3 `msaAttention1` (`cpu/af3/trunk/msa.js:157-219`): actNorm / pairNorm, pairLogits
    [cZ, H], vProjection / gatingQuery [cM, H*d], outputProjection [H*d, cM], all (in,out)."""
    s = capi.lf_pair_averaging_weights()
    s.act_norm_scale, s.act_norm_offset = dw.vec(w["actNormScale"]), dw.vec(w["actNormOffset"])
    s.pair_norm_scale, s.pair_norm_offset = dw.vec(w["pairNormScale"]), dw.vec(w["pairNormOffset"])
    s.pair_logits = dw.weight(w["pairLogits"], capi.LF_IN_OUT)
    s.wv = dw.weight(w["vProjection"], capi.LF_IN_OUT)
    s.wg = dw.weight(w["gatingQuery"], capi.LF_IN_OUT)
    s.wo = dw.weight(w["outputProjection"], capi.LF_IN_OUT)
    return s


def msa_pair_weighted_averaging(ctx: Context, msa: torch.Tensor, mask: torch.Tensor, pair: torch.Tensor,
                                wstruct: capi.lf_pair_averaging_weights, heads: int, head_dim: int,
                                out: torch.Tensor = None, accumulate: bool = False,
                                epsilon: float = 1e-5) -> torch.Tensor:
    """msa [S, N, cM], mask [S, N], pair [N, N, cZ]: the update (or msa + update) into `out`."""
    s_, n, c = msa.shape
    if out is None:
        out = torch.empty_like(msa)
    a = capi.lf_pair_averaging_args()
    a.sequences, a.tokens, a.c_m, a.c_z = s_, n, c, pair.shape[-1]
    a.heads, a.head_dim = heads, head_dim
    a.msa_dtype, a.msa, a.msa_mask = act_code(msa), ptr(msa), ptr(mask)
    a.pair_dtype, a.pair, a.out = act_code(pair), ptr(pair), ptr(out)
    a.accumulate = int(accumulate)
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_msa_pair_weighted_averaging(ctx.handle, C.byref(a)))
    return out


@_owned
def msa_module_weights(dw: DeviceWeights, w: dict) -> capi.lf_msa_module_weights:
    """One AF3 MSA-module block (`msaBlock`, `cpu/af3/trunk/msa.js:233-287`): outerProductMean,
    msaAttention1, msaTransition and the pair weights of a pairformer block."""
    s = capi.lf_msa_module_weights()
    s.outer_product_mean = opm_weights(dw, w["outerProductMean"], capi.LF_AF3)
    left = w["outerProductMean"]["leftProjection"]   # an array, or a stored record (quantised)
    s.c_outer = left["shape"][-1] if isinstance(left, dict) else np.shape(left)[-1]
    s.msa_attention = pair_averaging_weights(dw, w["msaAttention1"])
    s.msa_heads, s.msa_head_dim = w["msaAttention1"]["heads"], w["msaAttention1"]["dimension"]
    s.msa_transition = transition_weights(dw, w["msaTransition"], capi.LF_TRANSITION_SWIGLU)
    p = s.pair
    p.tri_out = tri_mult_weights(dw, w["triangleMultiplicationOutgoing"], capi.LF_AF3)
    p.tri_in = tri_mult_weights(dw, w["triangleMultiplicationIncoming"], capi.LF_AF3)
    p.att_start = attention_weights_af3_grid(dw, w["pairAttention1"])
    p.att_end = attention_weights_af3_grid(dw, w["pairAttention2"])
    p.pair_heads = w["pairAttention1"]["heads"]
    p.pair_transition = transition_weights(dw, w["pairTransition"], capi.LF_TRANSITION_SWIGLU)
    return s


def msa_module_block(ctx: Context, msa, pair, msa_mask, pair_mask, wstruct, msa_update_before_opm: bool,
                     swap_transposed_bias=False, divide_by_length=False, transition_chunk_bytes=0, epsilon=1e-5):
    """One AF3 MSA-module block, msa and pair updated in place."""
    a = capi.lf_msa_block_args()
    a.sequences, a.tokens, a.c_m = msa.shape
    a.c_z = pair.shape[-1]
    a.msa_update_before_opm = int(msa_update_before_opm)
    a.swap_transposed_bias, a.divide_by_length = int(swap_transposed_bias), int(divide_by_length)
    a.msa_dtype, a.msa, a.pair_dtype, a.pair = act_code(msa), ptr(msa), act_code(pair), ptr(pair)
    a.msa_mask, a.pair_mask = ptr(msa_mask), ptr(pair_mask)
    a.transition_chunk_bytes = transition_chunk_bytes
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_msa_module_block(ctx.handle, C.byref(a)))


_EMBED_WEIGHTS = {"preprocess_1d_w": "preprocess1dWeight", "preprocess_1d_b": "preprocess1dBias",
                  "preprocess_msa_w": "preprocessMsaWeight", "preprocess_msa_b": "preprocessMsaBias",
                  "left_w": "leftSingleWeight", "left_b": "leftSingleBias", "right_w": "rightSingleWeight",
                  "right_b": "rightSingleBias", "prev_pos_w": "previousPositionWeight",
                  "prev_pos_b": "previousPositionBias", "prev_msa_norm_scale": "previousMsaNormScale",
                  "prev_msa_norm_offset": "previousMsaNormOffset", "prev_pair_norm_scale": "previousPairNormScale",
                  "prev_pair_norm_offset": "previousPairNormOffset", "relpos_w": "relativePositionWeight",
                  "relpos_b": "relativePositionBias", "extra_w": "extraMsaWeight", "extra_b": "extraMsaBias"}


@_owned
def input_embedder_weights(dw: DeviceWeights, w: dict) -> capi.lf_input_embedder_weights:
    """InputEmbedderGpu's weights (`webgpu/af2/evoformer/input-embedder.js:9-26`), f32 (in,out)."""
    s = capi.lf_input_embedder_weights()
    for field, key in _EMBED_WEIGHTS.items():
        setattr(s, field, dw.vec(np.asarray(w[key], np.float32).reshape(-1)))
    return s


def input_embedder(ctx: Context, f: dict, wstruct: capi.lf_input_embedder_weights, c_m: int = 256, c_z: int = 128,
                   c_e: int = 64, dtype=torch.float32, prev_msa=None, prev_pair=None, prev_positions=None,
                   pair_out: torch.Tensor = None, epsilon: float = 1e-5):
    """One recycle's embeddings from device features `f` (InputEmbedderGpu.run input names, f32
    tensors): returns (msa [S, L, cM], pair [L, L, cZ], extra [Se, L, cE]) in `dtype`."""
    L, ct = f["targetFeatures"].shape
    s_, _, cf = f["msaFeatures"].shape
    se = f["extraMsa"].shape[0]
    dev = f["targetFeatures"].device
    msa = torch.empty(s_, L, c_m, device=dev, dtype=dtype)
    pair = pair_out if pair_out is not None else torch.empty(L, L, c_z, device=dev, dtype=dtype)
    extra = torch.empty(se, L, c_e, device=dev, dtype=dtype)
    a = capi.lf_input_embedder_args()
    a.length, a.msa_sequences, a.extra_sequences, a.target_channels, a.msa_feature_channels = L, s_, se, ct, cf
    a.c_m, a.c_z, a.c_e = c_m, c_z, c_e
    a.target_feat, a.msa_feat = ptr(f["targetFeatures"]), ptr(f["msaFeatures"])
    a.extra_msa, a.extra_has_deletion = ptr(f["extraMsa"]), ptr(f["extraHasDeletion"])
    a.extra_deletion_value = ptr(f["extraDeletionValue"])
    a.residue_index, a.aatype = ptr(f["residueIndex"]), ptr(f["aatype"])
    a.prev_msa_first_row = ptr(prev_msa) if prev_msa is not None else None
    a.prev_pair = ptr(prev_pair) if prev_pair is not None else None
    a.prev_positions = ptr(prev_positions) if prev_positions is not None else None
    a.msa_dtype, a.msa = act_code(msa), ptr(msa)
    a.pair_dtype, a.pair = act_code(pair), ptr(pair)
    a.extra_dtype, a.extra = act_code(extra), ptr(extra)
    a.epsilon = epsilon
    a.w = C.pointer(wstruct)
    check(ctx.lib.lf_input_embedder(ctx.handle, C.byref(a)))
    return msa, pair, extra


def af2_recycle_state(f: dict, c_m: int = 256, c_z: int = 128, c_e: int = 64, dtype=torch.bfloat16) -> dict:
    """Device buffers carried across recycles: msa [S, L, cM], pair [L, L, cZ], extra [Se, L, cE]."""
    L = f["targetFeatures"].shape[0]
    dev = f["targetFeatures"].device
    return {"msa": torch.zeros(f["msaFeatures"].shape[0], L, c_m, device=dev, dtype=dtype),
            "pair": torch.zeros(L, L, c_z, device=dev, dtype=dtype),
            "extra": torch.zeros(f["extraMsa"].shape[0], L, c_e, device=dev, dtype=dtype)}


def af2_recycle(ctx: Context, f: dict, state: dict, masks: dict, embed_ws, extra_wss, extra_w0: dict, main_wss,
                main_w0: dict, first: bool, prev_positions: torch.Tensor = None, epsilon: float = 1e-5):
    """One recycle (lf_af2_recycle): embed from the carried state (zeros when `first`), the
    extra-MSA stack, the Evoformer stack; `state` holds the result, which is the next recycle's
    carried state.  masks: msa [S, L], extra [Se, L], pair [L, L] (f32)."""
    msa, pair, extra = state["msa"], state["pair"], state["extra"]
    L, ct = f["targetFeatures"].shape
    a = capi.lf_af2_recycle_args()
    e = a.embed
    e.length, e.msa_sequences, e.extra_sequences = L, msa.shape[0], extra.shape[0]
    e.target_channels, e.msa_feature_channels = ct, f["msaFeatures"].shape[2]
    e.c_m, e.c_z, e.c_e = msa.shape[2], pair.shape[2], extra.shape[2]
    e.target_feat, e.msa_feat = ptr(f["targetFeatures"]), ptr(f["msaFeatures"])
    e.extra_msa, e.extra_has_deletion = ptr(f["extraMsa"]), ptr(f["extraHasDeletion"])
    e.extra_deletion_value = ptr(f["extraDeletionValue"])
    e.residue_index, e.aatype = ptr(f["residueIndex"]), ptr(f["aatype"])
    e.prev_msa_first_row = None if first else ptr(msa)
    e.prev_pair = None if first else ptr(pair)
    e.prev_positions = ptr(prev_positions)
    e.msa_dtype, e.msa, e.pair_dtype, e.pair = act_code(msa), ptr(msa), act_code(pair), ptr(pair)
    e.extra_dtype, e.extra = act_code(extra), ptr(extra)
    e.epsilon = epsilon
    e.w = C.pointer(embed_ws)
    if extra_wss:
        a.extra = evoformer_block_args(extra, pair, masks["extra"], masks["pair"], extra_w0, epsilon)
        arr_e = (capi.lf_extra_msa_weights * len(extra_wss))(*extra_wss)
        a.extra_blocks, a.extra_block_count = arr_e, len(extra_wss)
    if main_wss:
        a.main = evoformer_block_args(msa, pair, masks["msa"], masks["pair"], main_w0, epsilon)
        arr_m = (capi.lf_evoformer_weights * len(main_wss))(*main_wss)
        a.main_blocks, a.main_block_count = arr_m, len(main_wss)
    else:
        a.main.msa, a.main.pair = ptr(msa), ptr(pair)
    check(ctx.lib.lf_af2_recycle(ctx.handle, C.byref(a)))
    return state
