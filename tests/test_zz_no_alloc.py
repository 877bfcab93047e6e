"""lf_tri_mult_noalloc (the allocation-free triangle multiplication) against lf_tri_mult through
the C ABI: identical results on two calls in a row, the second smaller, and a clear rejection of
shapes whose scratch exceeds the static array."""
import numpy as np
import pytest

from localfold_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _run(ctx, n, direction, noalloc, seed):
    import torch
    from localfold_amd import device as D
    c2 = S.config2_inputs(n, 128, seed=seed, masked_tail=max(1, n // 24))
    dw = D.DeviceWeights(ctx.device)
    w = D.tri_mult_weights(dw, c2["rec_out" if direction == "outgoing" else "rec_in"])
    z = torch.as_tensor(c2["z"]).to(ctx.device).to(torch.bfloat16)
    mask = torch.as_tensor(c2["mask"]).to(ctx.device)
    out = torch.empty_like(z)
    D.tri_mult(ctx, z, mask, w, direction, out=out, accumulate=True, noalloc=noalloc)
    torch.cuda.synchronize()
    return out, dw


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_noalloc_matches_allocating_entry_point(ctx, direction):
    import torch
    for n, seed in ((384, 2), (100, 3)):          # the second call is smaller
        print(f"noalloc {direction} N={n}", flush=True)
        ref, _ = _run(ctx, n, direction, False, seed)
        got, _ = _run(ctx, n, direction, True, seed)
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), (n, (got.float() - ref.float()).abs().max().item())


def _noalloc_rc(ctx, n, dtype):
    import ctypes as C
    import torch
    from localfold_amd import capi, device as D
    dw = D.DeviceWeights(ctx.device)   # holds the weight buffers: alive until the call is done
    w = D.tri_mult_weights(dw, S.config2_inputs(16, 128, seed=1)["rec_out"])
    z = torch.zeros(n, n, 128, dtype=dtype, device=ctx.device)
    mask = torch.ones(n, n, device=ctx.device)
    out = torch.empty_like(z)
    a = capi.lf_tri_mult_args()
    a.direction, a.dialect, a.length, a.c_z, a.c_hidden = capi.LF_OUTGOING, capi.LF_AF2, n, 128, 128
    a.act_dtype = D.act_code(z)
    a.z, a.mask, a.out = D.ptr(z), D.ptr(mask), D.ptr(out)
    a.epsilon = 1e-5
    a.w = C.pointer(w)
    rc = ctx.lib.lf_tri_mult_noalloc(ctx.handle, C.byref(a))
    torch.cuda.synchronize()
    del dw
    return rc, out


def test_noalloc_rejects_oversized_shape(ctx):
    from localfold_amd import capi
    import torch
    rc, _ = _noalloc_rc(ctx, 420, torch.bfloat16)   # 3 * 128 * 420^2 f16 planes exceed the 128 MiB array
    assert rc == capi.LF_ERR_INVALID
    assert b"static scratch" in ctx.lib.lf_last_error()


def test_noalloc_scratch_boundary(ctx):
    """At N = 416 the three planes fit (132.9 MB) but not with the 8-byte LayerNorm statistics
    per pair that the 2-byte-activation kernels hand from project to output (134.3 MB); f32
    activations recompute them and fit."""
    import torch
    from localfold_amd import capi
    rc, _ = _noalloc_rc(ctx, 416, torch.bfloat16)
    assert rc == capi.LF_ERR_INVALID and b"static scratch" in ctx.lib.lf_last_error()
    rc, out = _noalloc_rc(ctx, 412, torch.bfloat16)
    assert rc == capi.LF_OK and torch.isfinite(out.float()).all()
    rc, out = _noalloc_rc(ctx, 416, torch.float32)
    assert rc == capi.LF_OK and torch.isfinite(out).all()
