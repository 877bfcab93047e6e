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


def test_noalloc_rejects_oversized_shape(ctx):
    import ctypes as C
    import torch
    from localfold_amd import capi, device as D
    n = 420                       # 3 * 128 * 420^2 f16 planes exceed the 128 MiB array
    w = D.tri_mult_weights(D.DeviceWeights(ctx.device), S.config2_inputs(16, 128, seed=1)["rec_out"])
    z = torch.zeros(n, n, 128, dtype=torch.bfloat16, device=ctx.device)
    mask = torch.ones(n, n, device=ctx.device)
    a = capi.lf_tri_mult_args()
    a.direction, a.dialect, a.length, a.c_z, a.c_hidden = capi.LF_OUTGOING, capi.LF_AF2, n, 128, 128
    a.act_dtype = D.act_code(z)
    a.z, a.mask, a.out = D.ptr(z), D.ptr(mask), D.ptr(z)
    a.epsilon = 1e-5
    a.w = C.pointer(w)
    rc = ctx.lib.lf_tri_mult_noalloc(ctx.handle, C.byref(a))
    assert rc == capi.LF_ERR_INVALID
    assert b"static scratch" in ctx.lib.lf_last_error()
