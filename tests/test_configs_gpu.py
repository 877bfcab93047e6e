"""The Evoformer (N_res = 384, N_seq = 512) and Pairformer (N = 1024) workloads on the GPU through
the C ABI, against the oracle.

Config 4: one AF2 Evoformer block at full size (N_res = 384, N_seq = 512, int8 weights in
groups of 64), and the 48-block stack at a reduced shape (48 distinct int8 weight sets).
Config 5: one AF3 Pairformer block with int5 weights (groups of 32) and the last 32 tokens
padded, against the oracle at N = 256, and at the full N = 1024 through the padding
invariance (padded tokens cannot reach unpadded outputs).

The residual stream is checked in two storage types:

* f32: the north-star bound as it stands, max abs <= 2e-2 and relative Frobenius <= 5e-3;
* bf16 (one block): the relative Frobenius bound only.  bf16 storage cannot meet the max-abs
  bound: pair values reach |x| ~ 9.5 after one config-4 block, where rounding the exact result
  to bf16 once is already off by 0.03, and every in-place write of the residual rounds again.
  The f32 residual stream is therefore the configuration whose parity is claimed (and the one
  the stack runs in: over 48 blocks bf16 storage drifts to a relative Frobenius error of 1.6e-2).
"""
import time

import numpy as np
import pytest

from localfold_amd import synthetic as S
from oracle import blocks, codec, ops
from tests import helpers as H

pytestmark = pytest.mark.gpu


def _decoded(v):
    if isinstance(v, dict) and "dtype" in v:
        return codec.decode(v)
    return {k: _decoded(u) for k, u in v.items()} if isinstance(v, dict) else v


def _bf16_round(x):
    import torch
    return torch.as_tensor(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def _dev(ctx, x, dt=None):
    import torch
    t = torch.as_tensor(np.ascontiguousarray(x)).to(ctx.device)
    return t.to(dt) if dt is not None else t


def assert_close_storage(actual, expected, storage, label):
    """The north-star bound for f32 storage; the relative Frobenius bound alone for bf16."""
    m = H.metrics(actual, expected)
    print(f"{label} [{storage}]: {m}", flush=True)
    if storage == "f32":
        H.assert_close(actual, expected, label=f"{label} [f32]")
    else:
        assert m["relativeFrobenius"] <= H.REL_FRO, f"{label} [{storage}]: {m}"


# ---- config 4: one block at full size -----------------------------------------------------

@pytest.fixture(scope="module")
def config4():
    c4 = S.config4_inputs()
    c4["decoded"] = _decoded(c4["weights"])
    # both storage types start from the same values: the inputs rounded to bf16
    c4["msa"] = _bf16_round(c4["msa"])
    c4["pair"] = _bf16_round(c4["pair"])
    t = time.perf_counter()
    c4["expect"] = blocks.evoformer_block_af2(c4["msa"], c4["pair"], c4["msa_mask"], c4["pair_mask"],
                                              c4["decoded"])
    print(f"config 4 oracle block: {time.perf_counter() - t:.1f} s", flush=True)
    return c4


@pytest.mark.parametrize("storage", ["f32", "bf16"])
def test_config4_block_full_size(ctx, config4, storage):
    import torch
    from localfold_amd import device as D
    dt = torch.float32 if storage == "f32" else torch.bfloat16
    dw = D.DeviceWeights(ctx.device)
    ws = D.evoformer_weights(dw, config4["weights"])
    msa, pair = _dev(ctx, config4["msa"], dt), _dev(ctx, config4["pair"], dt)
    D.evoformer_block(ctx, msa, pair, _dev(ctx, config4["msa_mask"]), _dev(ctx, config4["pair_mask"]), ws,
                      config4["weights"])
    torch.cuda.synchronize()
    rm, rp = config4["expect"]
    assert_close_storage(msa.float().cpu().numpy(), rm, storage, "config4 block msa")
    assert_close_storage(pair.float().cpu().numpy(), rp, storage, "config4 block pair")


# ---- config 4: the 48-block stack at a reduced shape --------------------------------------

@pytest.fixture(scope="module")
def stack48():
    n, s_ = 48, 16
    c4 = S.config4_inputs(n=n, sequences=s_, seed=6)
    weights = [c4["weights"]] + [S.quantise_tree(S.config1_inputs(seed=200 + k, n=1)[0], "int8", 64)
                                 for k in range(47)]
    states = [(_bf16_round(c4["msa"]), _bf16_round(c4["pair"]))]
    t = time.perf_counter()
    for w in weights:
        states.append(blocks.evoformer_block_af2(*states[-1], c4["msa_mask"], c4["pair_mask"], _decoded(w)))
    print(f"48 oracle blocks at N={n}, S={s_}: {time.perf_counter() - t:.1f} s", flush=True)
    return {"weights": weights, "states": states, "msa_mask": c4["msa_mask"], "pair_mask": c4["pair_mask"]}


def test_config4_stack_per_block_bound(ctx, stack48):
    """The north-star bound holds for every one of the 48 blocks (int8, f32 residual stream):
    each block starts from the oracle's state after the block before and is compared with the
    oracle's state after it."""
    import torch
    from localfold_amd import device as D
    dw = D.DeviceWeights(ctx.device)
    mm, pm = _dev(ctx, stack48["msa_mask"]), _dev(ctx, stack48["pair_mask"])
    worst = {"msa": 0.0, "pair": 0.0}
    for b, w in enumerate(stack48["weights"]):
        m0, p0 = stack48["states"][b]
        rm, rp = stack48["states"][b + 1]
        msa, pair = _dev(ctx, m0), _dev(ctx, p0)
        D.evoformer_block(ctx, msa, pair, mm, pm, D.evoformer_weights(dw, w), w)
        torch.cuda.synchronize()
        for name, got, ref in (("msa", msa, rm), ("pair", pair, rp)):
            m = H.assert_close(got.cpu().numpy(), ref, label=f"stack block {b} {name}")
            worst[name] = max(worst[name], m["maxAbsoluteError"])
    print(f"worst per-block max abs over 48 blocks: {worst}", flush=True)


def test_config4_stack_48_blocks(ctx, stack48):
    """The whole stack through lf_evoformer_stack (48 distinct int8 weight sets, f32 residual
    stream) against 48 chained oracle blocks: relative Frobenius <= 5e-3, and max abs <= 2e-2
    times the rms of the expected activations.

    The max-abs bound scales because the stack amplifies absolute differences as the
    activations grow (rms 1 -> ~12 for the pair over 48 random-init blocks): the oracle itself
    moves by rms 1.1e-3 at its output when its input moves by rms 1e-4, while relative errors
    do not grow.  Each block's own error stays inside the unscaled bound (the test above)."""
    import torch
    from localfold_amd import device as D
    dw = D.DeviceWeights(ctx.device)
    ws = [D.evoformer_weights(dw, w) for w in stack48["weights"]]
    m0, p0 = stack48["states"][0]
    msa, pair = _dev(ctx, m0), _dev(ctx, p0)
    D.evoformer_stack(ctx, msa, pair, _dev(ctx, stack48["msa_mask"]), _dev(ctx, stack48["pair_mask"]), ws,
                      stack48["weights"][0])
    torch.cuda.synchronize()
    rm, rp = stack48["states"][-1]
    for name, got, ref in (("msa", msa, rm), ("pair", pair, rp)):
        rms = float(np.sqrt(np.mean(np.square(ref, dtype=np.float64))))
        m = H.assert_close(got.cpu().numpy(), ref, max_abs=H.MAX_ABS * rms, label=f"48-block stack {name}")
        print(f"48-block stack {name}: rms(expected) {rms:.2f} {m}", flush=True)


# ---- config 4: later blocks of the full-shape stack ----------------------------------------

@pytest.mark.parametrize("k", [23, 47])
def test_config4_full_shape_stack_block_k(ctx, config4, k):
    """The 48-block stack at the full config-4 shape (N_res = 384, N_seq = 512, 48 distinct
    int8 weight sets, f32 residual stream): the GPU stack runs blocks 0 .. k-1, and block k
    then runs once on the GPU and once in the oracle from that same GPU state, held to the
    unscaled north-star bound (max abs <= 2e-2, relative Frobenius <= 5e-3).  Block k sees
    activations grown by k blocks (pair rms ~ 6-12), which the block-0 test does not."""
    import torch
    from localfold_amd import device as D
    weights = [config4["weights"]] + [S.quantise_tree(S.config1_inputs(seed=300 + b, n=1)[0], "int8", 64)
                                      for b in range(k)]
    dw = D.DeviceWeights(ctx.device)
    ws = [D.evoformer_weights(dw, w) for w in weights]
    mm, pm = _dev(ctx, config4["msa_mask"]), _dev(ctx, config4["pair_mask"])
    msa, pair = _dev(ctx, config4["msa"]), _dev(ctx, config4["pair"])
    D.evoformer_stack(ctx, msa, pair, mm, pm, ws[:k], weights[0])
    torch.cuda.synchronize()
    m0, p0 = msa.cpu().numpy(), pair.cpu().numpy()
    assert np.isfinite(m0).all() and np.isfinite(p0).all()
    D.evoformer_block(ctx, msa, pair, mm, pm, ws[k], weights[k])
    torch.cuda.synchronize()
    t = time.perf_counter()
    rm, rp = blocks.evoformer_block_af2(m0, p0, config4["msa_mask"], config4["pair_mask"], _decoded(weights[k]))
    print(f"config 4 oracle block {k}: {time.perf_counter() - t:.1f} s; input pair rms "
          f"{float(np.sqrt(np.mean(np.square(p0, dtype=np.float64)))):.2f}", flush=True)
    for name, got, ref in (("msa", msa, rm), ("pair", pair, rp)):
        print(f"full-shape stack block {k} {name}: {H.metrics(got.cpu().numpy(), ref)}", flush=True)
        H.assert_close(got.cpu().numpy(), ref, label=f"full-shape stack block {k} {name}")


# ---- config 5: the AF3 Pairformer block ---------------------------------------------------

def _config5(n, seed=21, padded=32):
    cz, cs = 128, 384
    w = S.quantise_tree(S.synthetic_pairformer_weights(cz, cs, 4, 16, 24, seed=seed), "int5", 32)
    st = S.Stream(seed + 1)
    pair = _bf16_round(st.normal(n * n * cz).reshape(n, n, cz))
    single = _bf16_round(st.normal(n * cs).reshape(n, cs))
    seq_mask = np.ones(n, np.float32)
    seq_mask[n - padded:] = 0
    return w, pair, single, seq_mask, np.outer(seq_mask, seq_mask).astype(np.float32)


@pytest.fixture(scope="module")
def config5_n256():
    w, pair, single, sm, pm = _config5(256)
    t = time.perf_counter()
    expect = blocks.pairformer_block_af3(pair, single, pm, sm, _decoded(w))
    print(f"config 5 oracle block at N=256: {time.perf_counter() - t:.1f} s", flush=True)
    return w, pair, single, sm, pm, expect


@pytest.mark.parametrize("storage", ["f32", "bf16"])
def test_config5_block_int5_padded(ctx, config5_n256, storage):
    import torch
    from localfold_amd import device as D
    w, pair0, single0, sm, pm, (rp, rs) = config5_n256
    dt = torch.float32 if storage == "f32" else torch.bfloat16
    dw = D.DeviceWeights(ctx.device)
    ws = D.pairformer_weights(dw, w)
    pair, single = _dev(ctx, pair0, dt), _dev(ctx, single0, dt)
    D.pairformer_block(ctx, pair, single, _dev(ctx, pm), _dev(ctx, sm), ws)
    torch.cuda.synchronize()
    assert_close_storage(pair.float().cpu().numpy(), rp, storage, "config5 N=256 pair")
    assert_close_storage(single.float().cpu().numpy(), rs, storage, "config5 N=256 single")


def test_config5_block_full_size_padding_invariance(ctx):
    """Config 5 at N = 1024, bf16: outputs finite, and the 32 padded tokens' activations (their
    pair rows and columns and their single rows) cannot reach any unpadded output: changing
    them leaves every unpadded pair entry and single row bit-identical."""
    import torch
    from localfold_amd import device as D
    n, pad = 1024, 32
    w, pair0, single0, sm, pm = _config5(n)
    dw = D.DeviceWeights(ctx.device)
    ws = D.pairformer_weights(dw, w)
    bf = torch.bfloat16
    pair_a, single_a = _dev(ctx, pair0, bf), _dev(ctx, single0, bf)
    pair_b, single_b = pair_a.clone(), single_a.clone()
    g = torch.Generator(device=ctx.device).manual_seed(5)
    k = n - pad
    pair_b[k:, :] = (3 * torch.randn(pad, n, 128, device=ctx.device, generator=g)).to(bf)
    pair_b[:, k:] = (3 * torch.randn(n, pad, 128, device=ctx.device, generator=g)).to(bf)
    single_b[k:] = (3 * torch.randn(pad, 384, device=ctx.device, generator=g)).to(bf)
    smd, pmd = _dev(ctx, sm), _dev(ctx, pm)
    D.pairformer_block(ctx, pair_a, single_a, pmd, smd, ws)
    D.pairformer_block(ctx, pair_b, single_b, pmd, smd, ws)
    torch.cuda.synchronize()
    assert torch.isfinite(pair_a).all() and torch.isfinite(single_a).all()
    assert torch.isfinite(pair_b).all() and torch.isfinite(single_b).all()
    assert torch.equal(pair_a[:k, :k], pair_b[:k, :k])
    assert torch.equal(single_a[:k], single_b[:k])
    # the padded inputs did change and the block did move the unpadded outputs
    assert not torch.equal(pair_a[k:], pair_b[k:])
    assert not torch.equal(pair_a[:k, :k], _dev(ctx, pair0, bf)[:k, :k])
