"""The pair-stack operators, restated in numpy (float64 compute, float32 storage).

Every function returns what the reference's function or GPU class returns for the same
input: the UPDATE (delta) of an op, never the residual sum, unless it says otherwise.
Array layouts are the reference's flat layouts reshaped: pair [N, N, C], msa [S, N, C],
masks [N, N] / [S, N], triangle weights (out,in), everything else (in,out).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

F32 = np.float32
F64 = np.float64


def _parallel(fn, items):
    """Runs fn over independent items on host threads (numpy releases the GIL in its array
    loops and BLAS calls); each item writes a disjoint slice of its output."""
    items = list(items)
    workers = min(len(items), int(os.environ.get("LOCALFOLD_ORACLE_THREADS", min(16, os.cpu_count() or 1))))
    if workers <= 1:
        for it in items:
            fn(it)
        return
    from threadpoolctl import threadpool_limits
    with threadpool_limits(1), ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(fn, items))


def _f32(x):
    return np.asarray(x, F64).astype(F32)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, F64)))


# ---------------------------------------------------------------------------------------
# Layer norm and dense layers
# ---------------------------------------------------------------------------------------

def layer_norm(x, scale, offset, eps=1e-5, fast_variance=False):
    """LayerNorm over the last axis.

    two-pass: `normalizeRows` (`webgpu/kernels/triangle/cpu-reference.js:5-29`) and the WGSL
    normalise (`webgpu/kernels/attention.js:189-257`): mean, then mean of squared deviations.
    fast_variance: AF3's E[x^2]-E[x]^2 (`cpu/af3/trunk/pairformer.js:68-87`).
    """
    x = np.asarray(x, F64)
    c = x.shape[-1]
    mean = x.sum(-1, keepdims=True) / c
    if fast_variance:
        var = (x * x).sum(-1, keepdims=True) / c - mean * mean
    else:
        d = x - mean
        var = (d * d).sum(-1, keepdims=True) / c
    inv = 1.0 / np.sqrt(var + eps)
    return _f32((x - mean) * inv * np.asarray(scale, F64) + np.asarray(offset, F64))


def linear(x, w, bias=None, transposed=False):
    """rows x in -> rows x out with a float64 accumulator, rounded once.

    (in,out) weights: `linear` (`cpu/af3/trunk/pairformer.js:100-150`); (out,in) weights
    (`transposed`): `project` (`webgpu/kernels/triangle/cpu-reference.js:31-50`).
    """
    x = np.asarray(x, F64)
    w = np.asarray(w, F64)
    y = x @ (w.T if transposed else w)
    if bias is not None:
        y = y + np.asarray(bias, F64)
    return _f32(y)


# ---------------------------------------------------------------------------------------
# Triangle multiplication
# ---------------------------------------------------------------------------------------

def _contract(a, b, direction):
    """a, b: [N, N, H] (pair-major).  outgoing x_ij = sum_k a_ik b_jk; incoming sum_k a_kj b_ki.

    `cpu-reference.js:76-88` (outgoing, f64 accumulator) and `pairformer.js:247-258` (both).
    """
    a = np.ascontiguousarray(np.asarray(a, F64).transpose(2, 0, 1))   # [H, N, N]
    b = np.ascontiguousarray(np.asarray(b, F64).transpose(2, 0, 1))
    if direction == "outgoing":
        x = np.matmul(a, np.ascontiguousarray(b.transpose(0, 2, 1)))    # [H, i, j] = sum_k a[h,i,k] b[h,j,k]
    elif direction == "incoming":
        x = np.matmul(np.ascontiguousarray(b.transpose(0, 2, 1)), a)    # [H, i, j] = sum_k b[h,k,i] a[h,k,j]
    else:
        raise ValueError(direction)
    return x.transpose(1, 2, 0)                # [i, j, H]


def tri_mult_af2(z, mask, w, direction="outgoing", eps=1e-5):
    """AF2 triangle multiplicative update, returning the update (no residual).

    Follows `triangleMultiplicationOutgoingReference` (`webgpu/kernels/triangle/cpu-reference.js:55-99`):
    two-pass LN, five (out,in) projections with biases, a = ap*sigmoid(ag)*mask (and b),
    contraction, centre LN over channels, output projection gated by sigmoid(LN(z) Wg + bg).
    `direction="incoming"` contracts a_kj*b_ki (`pairformer.js:252-257`, AF2's incoming).
    """
    n = z.shape[0]
    zn = layer_norm(z, w["layerNormInWeight"], w["layerNormInBias"], eps)
    ap = linear(zn, w["linearAPWeight"], w["linearAPBias"], transposed=True)
    ag = linear(zn, w["linearAGWeight"], w["linearAGBias"], transposed=True)
    bp = linear(zn, w["linearBPWeight"], w["linearBPBias"], transposed=True)
    bg = linear(zn, w["linearBGWeight"], w["linearBGBias"], transposed=True)
    m = np.asarray(mask, F64).reshape(n, n, 1)
    a = _f32(np.asarray(ap, F64) * sigmoid(ag) * m)
    b = _f32(np.asarray(bp, F64) * sigmoid(bg) * m)
    x = _f32(_contract(a, b, direction))
    xn = layer_norm(x, w["layerNormOutWeight"], w["layerNormOutBias"], eps)
    out = linear(xn, w["linearZWeight"], w["linearZBias"], transposed=True)
    gate = linear(zn, w["linearGWeight"], w["linearGBias"], transposed=True)
    return _f32(np.asarray(out, F64) * sigmoid(gate))


def tri_mult_af3(z, mask, w, direction="outgoing", divide_by_length=False, eps=1e-5):
    """AF3 triangle multiplication (`cpu/af3/trunk/pairformer.js:213-300`).

    No biases, fast-variance LN, fused (in, 2c) projection and gate split INTERLEAVED
    (a = column 2c, b = column 2c+1), optional rf3 division by the length before the centre
    norm.  Weights: leftNormInputScale/Offset, projection [c,2c], gate [c,2c],
    centerNormScale/Offset, outputProjection [c,c], gatingLinear [c,c] (all (in,out)).
    """
    n, _, c = z.shape
    zn = layer_norm(z, w["leftNormInputScale"], w["leftNormInputOffset"], eps, fast_variance=True)
    proj = np.asarray(linear(zn, w["projection"]), F64)
    gate = np.asarray(linear(zn, w["gate"]), F64)
    m = np.asarray(mask, F64).reshape(n, n, 1)
    a = _f32(proj[..., 0::2] * (m * sigmoid(gate[..., 0::2])))
    b = _f32(proj[..., 1::2] * m * sigmoid(gate[..., 1::2]))
    x = _contract(a, b, direction)
    if divide_by_length:
        x = x / n
    x = _f32(x)
    xn = layer_norm(x, w["centerNormScale"], w["centerNormOffset"], eps, fast_variance=True)
    out = linear(xn, w["outputProjection"])
    g = linear(zn, w["gatingLinear"])
    return _f32(np.asarray(out, F64) * sigmoid(g))


# ---------------------------------------------------------------------------------------
# Gated attention (AF2 WGSL semantics) and AF3 grid / single attention
# ---------------------------------------------------------------------------------------

def _softmax_attend(q, k, v, logit_bias):
    """q,k,v: [B, H, Q, D] f64; logit_bias broadcastable to [B, H, Q, K]. Returns [B, H, Q, D]."""
    logits = q @ k.transpose(0, 1, 3, 2) + logit_bias
    logits = logits - logits.max(-1, keepdims=True)
    p = np.exp(logits)
    p = p / p.sum(-1, keepdims=True)
    return p @ v


def attention_af2(activations, mask, w, heads, transpose=False, pair_bias=None, eps=1e-5,
                  batch_chunk=None, batch_rows=None):
    """AF2 gated self-attention, the semantics of `AttentionGpu.run` (`webgpu/kernels/attention.js:2580-2739`).

    activations: [batch, queries, C] in the (untransposed) storage layout when
    `transpose=False`; with `transpose=True` the storage is [queries, batch, C] and
    logical row (b, q) reads storage row (q, b) (`attention.js:163-168`), the key mask is
    read at [k, b] (`attention.js:906-909`) and the update is stored back transposed.
      x = LN(row) (two-pass, eps)                          `attention.js:189-257`
      q = x Wq / sqrt(d); k = x Wk; v = x Wv; g = sigmoid(x Wg + bg)   `attention.js:482-507`
      logit = q.k + 1e9 (mask_k - 1) + bias[h, q, k], clamped to +-1e8  `attention.js:917-921`
      o = softmax(logit) v * g;  update = o Wo + bo
    pair_bias: None | {"source": "separate", "activations": pair [Q,Q,Cz], "layerNormScale",
    "layerNormOffset", "projectionWeight" [Cz, H]} | {"source": "normalized-input",
    "projectionWeight" [C, H]}  (`attention.js:695-783`: bias[h][i][j] = LN(z_ij) . W[:, h]).
    Weights are (in,out).  Returns the update in the storage layout.
    `batch_rows` restricts the result to those logical batch rows (returned as
    [len(batch_rows), queries, C], logical order) - batch rows are independent given the
    bias, so a large case can be checked on a sample.
    """
    act = np.asarray(activations, F32)
    if transpose:
        act = act.transpose(1, 0, 2)          # logical [batch, queries, C]
        msk = np.asarray(mask, F64).T         # storage [queries, batch] -> [batch, queries]
    else:
        msk = np.asarray(mask, F64)
    bsz, nq, c = act.shape
    d = c // heads
    x = layer_norm(act, w["queryNormScale"], w["queryNormOffset"], eps)
    bias = None
    if pair_bias is not None:
        if pair_bias["source"] == "separate":
            pn = layer_norm(pair_bias["activations"], pair_bias["layerNormScale"],
                            pair_bias["layerNormOffset"], eps)
            bias = linear(pn, pair_bias["projectionWeight"])          # [Q, Q, H]
        else:
            # bias[h][i][j] from the normalised logical row (i, j) of the attention input itself
            # (`block.js:1592-1610`, source "normalized-input"; batch == queries there)
            bias = linear(x.reshape(bsz * nq, c), pair_bias["projectionWeight"]).reshape(bsz, nq, heads)
        bias = np.asarray(bias, F64).transpose(2, 0, 1)              # [H, Q, K]
    if batch_rows is not None:
        x = x[np.asarray(batch_rows)]
        msk = msk[np.asarray(batch_rows)]
        bsz = x.shape[0]
    qs = 1.0 / np.sqrt(d)
    q = _f32(np.asarray(linear(x, w["queryWeight"]), F64) * qs)
    kk = linear(x, w["keyWeight"])
    v = linear(x, w["valueWeight"])
    g = _f32(sigmoid(linear(x, w["gatingWeight"], w["gatingBias"])))

    def heads_of(t):
        return np.asarray(t, F64).reshape(t.shape[0], nq, heads, d).transpose(0, 2, 1, 3)

    out = np.empty((bsz, nq, heads, d), F64)
    step = batch_chunk or max(1, int(2 ** 22 // max(1, heads * nq * nq)))

    def rows(b0):
        b1 = min(bsz, b0 + step)
        mb = (1e9 * (msk[b0:b1] - 1.0))[:, None, None, :]
        lb = mb if bias is None else mb + bias[None]
        qh, kh, vh = heads_of(q[b0:b1]), heads_of(kk[b0:b1]), heads_of(v[b0:b1])
        logits = qh @ kh.transpose(0, 1, 3, 2)
        logits += lb
        np.clip(logits, -1e8, 1e8, out=logits)
        logits -= logits.max(-1, keepdims=True)
        np.exp(logits, out=logits)
        logits /= logits.sum(-1, keepdims=True)
        out[b0:b1] = (logits @ vh).transpose(0, 2, 1, 3)

    _parallel(rows, range(0, bsz, step))
    o = _f32(out.reshape(bsz, nq, c) * np.asarray(g, F64))
    upd = linear(o, w["outputWeight"], w["outputBias"])
    if batch_rows is not None:
        return upd
    return upd.transpose(1, 0, 2).copy() if transpose else upd


def grid_self_attention_af3(pair, mask, w, transpose, swap_transposed_bias=False, eps=1e-5):
    """AF3 triangle ("grid") attention (`cpu/af3/trunk/pairformer.js:322-431`).

    Fast-variance LN of the untransposed pair; bias from that (optionally swapped), the
    activation transposed for the ending node; q/k/gate weights are (out,in) ("transposed"),
    v and output (in,out); optional gate/output biases (rf3); key mask at [row, j] or
    [j, row]; update restored to the original orientation.
    """
    n, _, c = pair.shape
    heads, dim = w["heads"], w["dimension"]
    xn = layer_norm(pair, w["actNormScale"], w["actNormOffset"], eps, fast_variance=True)
    raw = np.asarray(linear(xn, w["pairBiasProjection"]), F64)      # [i, j, H]
    if transpose and swap_transposed_bias:
        raw = raw.transpose(1, 0, 2)
    bias = _f32(raw).astype(F64).transpose(2, 0, 1)                 # [H, i, j]
    act = xn.transpose(1, 0, 2) if transpose else xn
    q = linear(act, w["qProjection"], transposed=True)
    k = linear(act, w["kProjection"], transposed=True)
    v = linear(act, w["vProjection"])
    msk = np.asarray(mask, F64)
    if transpose:
        msk = msk.T                                                 # key mask of row r: mask[j, r]
    qh = np.asarray(q, F64).reshape(n, n, heads, dim).transpose(0, 2, 1, 3)
    kh = np.asarray(k, F64).reshape(n, n, heads, dim).transpose(0, 2, 1, 3)
    vh = np.asarray(v, F64).reshape(n, n, heads, dim).transpose(0, 2, 1, 3)
    logits = (qh @ kh.transpose(0, 1, 3, 2)) / np.sqrt(dim) + bias[None] \
        + np.where(msk > 0, 0.0, -1e9)[:, None, None, :]
    logits = _f32(logits).astype(F64)
    logits -= logits.max(-1, keepdims=True)
    p = np.exp(logits)
    p /= p.sum(-1, keepdims=True)
    p = _f32(p).astype(F64)
    o = _f32((p @ vh).transpose(0, 2, 1, 3).reshape(n, n, heads * dim))
    g = np.asarray(linear(act, w["gatingQuery"], transposed=True), F64)
    if w.get("gatingQueryBias") is not None:
        g = g + np.asarray(w["gatingQueryBias"], F64)
    o = _f32(np.asarray(o, F64) * sigmoid(_f32(g)))
    out = linear(o, w["outputProjection"], w.get("outputProjectionBias"))
    return out.transpose(1, 0, 2).copy() if transpose else out


def single_attention_af3(single, pair_logits, seq_mask, w, eps=1e-5):
    """AF3 single-track attention with pair logits (`cpu/af3/trunk/pairformer.js:446-485`).

    pair_logits: [H, N, N].  q has a bias; no gate bias; key mask 1e9*(m-1).
    """
    n, c = single.shape
    heads, dim = w["heads"], w["dimension"]
    x = layer_norm(single, w["layerNormScale"], w["layerNormOffset"], eps, fast_variance=True)
    q = linear(x, w["qProjection"], w["qBias"])
    k = linear(x, w["kProjection"])
    v = linear(x, w["vProjection"])
    qh = np.asarray(q, F64).reshape(n, heads, dim).transpose(1, 0, 2)
    kh = np.asarray(k, F64).reshape(n, heads, dim).transpose(1, 0, 2)
    vh = np.asarray(v, F64).reshape(n, heads, dim).transpose(1, 0, 2)
    logits = (qh @ kh.transpose(0, 2, 1)) / np.sqrt(dim) + np.asarray(pair_logits, F64) \
        + (1e9 * (np.asarray(seq_mask, F64) - 1.0))[None, None, :]
    logits = _f32(logits).astype(F64)
    logits -= logits.max(-1, keepdims=True)
    p = np.exp(logits)
    p /= p.sum(-1, keepdims=True)
    p = _f32(p).astype(F64)
    o = _f32((p @ vh).transpose(1, 0, 2).reshape(n, heads * dim))
    g = linear(x, w["gatingQuery"])
    o = _f32(np.asarray(o, F64) * sigmoid(g))
    return linear(o, w["outputProjection"])


def global_column_attention_af2(msa, mask, w, heads, eps=1e-5):
    """AF2 extra-MSA global column attention, the semantics of `encodeGlobalAttention`
    (`webgpu/af2/evoformer/block.js:953-1030`) and its kernels (`:88-400`).  Per residue
    column i, over the sequences s:

      x = LN(msa) with queryNorm (two-pass, eps);
      k_si = x_si Wk, v_si = x_si Wv        (one shared head of width d, `:101-146`);
      q_ih = (sum_s m_si x_si / (1e-10 + sum_s m_si)) Wq_h / sqrt(d)      (`:166-226`);
      logit_sih = q_ih . k_si, replaced by -1e9 where m_si = 0; softmax over s   (`:240-300`);
      o_sih = sigmoid(x_si Wg + bg)_h * sum_s softmax v_s              (`:329-400`);
      update_si = o_si Wo + bo.
    Weights (in,out): queryWeight [C, H*d], keyWeight/valueWeight [C, d], gatingWeight
    [C, H*d], gatingBias [H*d], outputWeight [H*d, C], outputBias [C]; d = len(gatingBias)/heads.
    Every intermediate buffer is rounded to float32 as the reference stores it.
    Returns the msa update [S, N, C].
    """
    s_, n, c = msa.shape
    d = len(w["gatingBias"]) // heads
    x = layer_norm(msa, w["queryNormScale"], w["queryNormOffset"], eps)
    m = np.asarray(mask, F64)
    keys = np.asarray(linear(x, w["keyWeight"]), F64)            # [S, N, d]
    values = np.asarray(linear(x, w["valueWeight"]), F64)
    den = 1e-10 + m.sum(0)                                       # [N]
    means = _f32((np.asarray(x, F64) * m[..., None]).sum(0) / den[:, None])   # [N, C]
    q = np.asarray(_f32(np.asarray(means, F64) @ np.asarray(w["queryWeight"], F64).reshape(c, heads * d)
                        / np.sqrt(d)), F64).reshape(n, heads, d)
    logits = np.einsum("nhd,snd->nhs", q, keys)
    logits = np.where((m.T == 0)[:, None, :], -1e9, logits)
    logits = logits - logits.max(-1, keepdims=True)
    p = np.exp(logits)
    p = p / p.sum(-1, keepdims=True)
    attended = np.asarray(_f32(np.einsum("nhs,snd->nhd", p, values)), F64).reshape(n, heads * d)
    gate = sigmoid(np.asarray(linear(x, w["gatingWeight"], w["gatingBias"]), F64))
    gated = _f32(gate * attended[None])
    return linear(gated, w["outputWeight"], w["outputBias"])


def msa_pair_weighted_averaging_af3(msa, mask, pair, w, eps=1e-5):
    """AF3 MSA pair-weighted averaging, `msaAttention` (`cpu/af3/trunk/msa.js:157-219`):
    fast-variance LN of the msa (actNorm) and of the pair (pairNorm); logits
    LN(pair) . pairLogits [cZ, H] (no bias); the key mask is the maximum of the MSA mask over
    the sequences (`:177-186`), added as 1e9 (keyMask - 1); softmax over j per (h, i), shared by
    every sequence; averaged = softmax . (x vProjection), times sigmoid(x gatingQuery), then
    outputProjection.  All weights (in,out), no biases.  Returns the msa update [S, N, C]."""
    s_, n, c = msa.shape
    heads, d = w["heads"], w["dimension"]
    x = layer_norm(msa, w["actNormScale"], w["actNormOffset"], eps, fast_variance=True)
    pn = layer_norm(pair, w["pairNormScale"], w["pairNormOffset"], eps, fast_variance=True)
    flat = np.asarray(linear(pn, w["pairLogits"]), F64)                # [N, N, H]
    key_mask = np.asarray(mask, F64).max(0)                           # [N]
    # stored as f32 (weightsByHead is a Float32Array, :188-193): with every key masked the 1e9
    # term swamps the logits and the row is uniform
    logits = np.asarray(_f32(flat.transpose(2, 0, 1) + 1e9 * (key_mask[None, None, :] - 1.0)), F64)
    logits = logits - logits.max(-1, keepdims=True)
    p = np.exp(logits)
    p = np.asarray(_f32(p / p.sum(-1, keepdims=True)), F64)          # [H, N, N]
    values = np.asarray(linear(x, w["vProjection"]), F64).reshape(s_, n, heads, d)
    averaged = np.einsum("hij,sjhd->sihd", p, values).reshape(s_, n, heads * d)
    gate = sigmoid(np.asarray(linear(x, w["gatingQuery"]), F64))
    return linear(_f32(averaged * gate), w["outputProjection"])


# ---------------------------------------------------------------------------------------
# Outer product mean and transitions
# ---------------------------------------------------------------------------------------

def _outer_sum(left, right):
    """outer[i, j, a*c + b] = sum_s left[s, i, a] * right[s, j, b] (the einsum 'sia,sjb->ijab'),
    as one float64 GEMM over the sequences."""
    s, n, co = left.shape
    l2 = np.asarray(left, F64).reshape(s, n * co)
    r2 = np.asarray(right, F64).reshape(s, n * co)
    return (l2.T @ r2).reshape(n, co, n, co).transpose(0, 2, 1, 3).reshape(n, n, co * co)


def outer_product_mean_af2(msa, mask, w, eps=1e-5, norm_eps=1e-3):
    """AF2 OPM, the semantics of `OuterProductMeanGpu` (`webgpu/kernels/outer-product-mean.js`).

    l = mask * (LN(msa) Wl + bl), r likewise (`:395-416`);
    update_ij = (sum_s sum_ab l_sia r_sjb W[(a*c+b), z] + b_z) / (norm_eps + sum_s m_si m_sj)
    (`:595-610` index order, `:702-742` bias-then-divide).  Returns the pair update.
    """
    s, n, _ = msa.shape
    co = w["leftWeight"].shape[1]
    x = layer_norm(msa, w["layerNormScale"], w["layerNormOffset"], eps)
    m = np.asarray(mask, F64)[..., None]
    left = _f32(np.asarray(linear(x, w["leftWeight"], w["leftBias"]), F64) * m)
    right = _f32(np.asarray(linear(x, w["rightWeight"], w["rightBias"]), F64) * m)
    outer = _outer_sum(left, right)
    upd = outer @ np.asarray(w["outputWeight"], F64) + np.asarray(w["outputBias"], F64)
    count = np.asarray(mask, F64).T @ np.asarray(mask, F64)          # [i, j] = sum_s m_si m_sj
    return _f32(upd / (norm_eps + count)[..., None])


def outer_product_mean_af3(msa, mask, w, eps=1e-5, norm_eps=1e-3):
    """AF3 OPM (`cpu/af3/trunk/msa.js:72-155`): fast-variance LN, no biases, /(eps + count)."""
    s, n, _ = msa.shape
    co = w["leftProjection"].shape[1]
    x = layer_norm(msa, w["layerNormInputScale"], w["layerNormInputOffset"], eps, fast_variance=True)
    m = np.asarray(mask, F64)[..., None]
    left = _f32(np.asarray(linear(x, w["leftProjection"]), F64) * m)
    right = _f32(np.asarray(linear(x, w["rightProjection"]), F64) * m)
    outer = _outer_sum(left, right)
    upd = outer @ np.asarray(w["outputW"], F64)
    if w.get("outputB") is not None:
        upd = upd + np.asarray(w["outputB"], F64)
    count = np.asarray(mask, F64).T @ np.asarray(mask, F64)
    return _f32(upd / (norm_eps + count)[..., None])


def transition_af2(x, w, eps=1e-5):
    """AF2 transition `ReLU(LN(x) W1 + b1) W2 + b2` (`webgpu/kernels/transition.js:745-766,1080-1085`)."""
    xn = layer_norm(x, w["layerNormScale"], w["layerNormOffset"], eps)
    h = linear(xn, w["firstWeight"], w["firstBias"])
    h = np.maximum(h, F32(0))
    return linear(h, w["secondWeight"], w["secondBias"])


def transition_af3(x, w, factor=4, eps=1e-5):
    """AF3 SwiGLU transition, BLOCKED split (`cpu/af3/trunk/pairformer.js:180-201`)."""
    c = x.shape[-1]
    inter = c * factor
    xn = layer_norm(x, w["inputLayerNormScale"], w["inputLayerNormOffset"], eps, fast_variance=True)
    wide = np.asarray(linear(xn, w["transition1"]), F64)
    a, b = wide[..., :inter], wide[..., inter:]
    gated = _f32(a * sigmoid(a) * b)
    return linear(gated, w["transition2"])


def chunk_rows(rows, channels, hidden, budget_bytes=32 * 1024 * 1024, tile_rows=64):
    """Rows per transition chunk so the f32 hidden buffer stays within `budget_bytes`.

    Restates the capacity rule of `transitionChunkRows` (`webgpu/kernels/transition.js:411-442`)
    without WebGPU's binding-offset alignment (HIP has none): all rows when they fit,
    else the largest multiple of `tile_rows` that fits.
    """
    row_bytes = max(channels, hidden) * 4
    if rows * row_bytes <= budget_bytes:
        return rows
    cap = budget_bytes // row_bytes
    if cap < tile_rows:
        raise ValueError("budget cannot hold one tile of transition rows")
    return min(rows, (cap // tile_rows) * tile_rows)


def error_metrics(actual, expected):
    """`errorMetrics` (`webgpu/kernels/triangle/types.js:50-69`) plus relative Frobenius."""
    a = np.asarray(actual, F64).reshape(-1)
    e = np.asarray(expected, F64).reshape(-1)
    if a.size != e.size or a.size == 0:
        raise ValueError("error metrics require equally sized, non-empty arrays")
    d = np.abs(a - e)
    return {"meanAbsoluteError": float(d.mean()), "maxAbsoluteError": float(d.max()),
            "rootMeanSquareError": float(np.sqrt((d * d).mean())),
            "relativeFrobenius": float(np.sqrt((d * d).sum()) / max(np.sqrt((e * e).sum()), 1e-30))}


# ---------------------------------------------------------------------------------------
# AF2 input and recycling embedder
# ---------------------------------------------------------------------------------------

EMBED_DGRAM_BINS, EMBED_MIN_BIN, EMBED_MAX_BIN, EMBED_MAX_RELATIVE = 15, 3.25, 20.75, 32


def pseudo_beta(positions, aatype):
    """CB of each residue from atom37 positions [L, 37, 3], CA (atom 1) for glycine (aatype 7)
    (`PAIR_SHADER` pseudo_beta_coordinate, `webgpu/af2/evoformer/input-embedder.js:105-108`)."""
    atom = np.where(np.asarray(aatype).astype(np.int64) == 7, 1, 3)
    return np.asarray(positions, F64).reshape(-1, 37, 3)[np.arange(len(atom)), atom]


def dgram_bins(d2):
    """One-hot [.., 15] of squared distances: bin b covers (lower_b^2, upper_b^2) with
    lower_b = 3.25 + b w, w = 17.5 / 14, upper the next lower, the last bin unbounded above
    (`input-embedder.js:121-128`).  Squared distances at or below 3.25^2 fall in no bin."""
    w = np.float32((EMBED_MAX_BIN - EMBED_MIN_BIN) / (EMBED_DGRAM_BINS - 1))
    b = np.arange(EMBED_DGRAM_BINS)
    lower = (np.float32(EMBED_MIN_BIN) + b.astype(np.float32) * w).astype(F64)
    upper = np.append(lower[1:], np.inf)
    d2 = np.asarray(d2, F64)[..., None]
    return ((d2 > lower * lower) & (d2 < upper * upper)).astype(F64)


def input_embedder_af2(target_feat, msa_feat, extra_msa, extra_has_deletion, extra_deletion_value,
                       residue_index, aatype, prev_msa_first_row, prev_pair, prev_positions, w, eps=1e-5):
    """AF2 input + recycling embedder before the template branch, `InputEmbedderGpu.run` /
    `encodeInputEmbedder` (`webgpu/af2/evoformer/input-embedder.js:160-231`):
      msa[s, r]   = target[r] W1d + b1d + msa_feat[s, r] Wmsa + bmsa (+ LN(prev_msa[r]) on s = 0)
                    (MSA_SHADER, :61-83)
      pair[i, j]  = target[i] Wl + bl + target[j] Wr + br + bpos + Wpos[dgram bin of the
                    pseudo-beta distance] + LN(prev_pair[i, j]) + brel + Wrel[clip(ri - rj + 32,
                    0, 64)]  (PAIR_SHADER, :99-137)
      extra[s, r] = bext + Wext[code] + has_deletion Wext[23] + deletion_value Wext[24]
                    (EXTRA_SHADER, :85-97)
    Layer norms: two-pass, eps 1e-5 (`createAttentionNormParameters`, :197-204).
    Returns (msa [S, L, cM], pair [L, L, cZ], extra [Se, L, cE])."""
    tf = np.asarray(target_feat, F64)
    n = tf.shape[0]
    single = tf @ w["preprocess1dWeight"] + w["preprocess1dBias"]
    msa = np.asarray(msa_feat, F64) @ w["preprocessMsaWeight"] + w["preprocessMsaBias"] + single[None]
    msa[0] += layer_norm(prev_msa_first_row, w["previousMsaNormScale"], w["previousMsaNormOffset"], eps)
    left = tf @ w["leftSingleWeight"] + w["leftSingleBias"]
    right = tf @ w["rightSingleWeight"] + w["rightSingleBias"]
    pair = left[:, None] + right[None, :] + w["previousPositionBias"]
    cb = pseudo_beta(prev_positions, aatype)
    d2 = ((cb[:, None] - cb[None, :]) ** 2).sum(-1)
    pair += dgram_bins(d2) @ w["previousPositionWeight"]
    pair += layer_norm(prev_pair, w["previousPairNormScale"], w["previousPairNormOffset"], eps)
    ri = np.asarray(residue_index).astype(np.int64)
    rel = np.clip(ri[:, None] - ri[None, :] + EMBED_MAX_RELATIVE, 0, 2 * EMBED_MAX_RELATIVE)
    pair += w["relativePositionBias"] + np.asarray(w["relativePositionWeight"], F64)[rel]
    we = np.asarray(w["extraMsaWeight"], F64)
    codes = np.asarray(extra_msa).astype(np.int64)
    extra = (w["extraMsaBias"] + we[codes] + np.asarray(extra_has_deletion, F64)[..., None] * we[23]
             + np.asarray(extra_deletion_value, F64)[..., None] * we[24])
    assert pair.shape[:2] == (n, n)
    return _f32(msa), _f32(pair), _f32(extra)
