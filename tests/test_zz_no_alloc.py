"""wa_bsa_fwd_noalloc (the block-sparse forward whose workspace is the library's static device array)
against wa_bsa_fwd with a caller-allocated workspace: outputs and log-sum-exps bit-identical, on two
calls in a row (the second smaller, so it runs on what the first left in the array), with rows
long enough to be cut into several split units (the partials and arrival counters that live in
the array are used). Also: a launch that needs more than the array is rejected before it runs, and
a caller-supplied workspace is refused."""
import ctypes

import pytest
import torch

from worldattention_amd import _lib
from worldattention_amd.hsa.block_sparse import bsa_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, b, h, lq, lkv, width, bs=128, d=128):
    g = torch.Generator().manual_seed(seed)
    nq, nkv = -(-lq // bs), -(-lkv // bs)
    q = torch.randn(b, lq, h, d, generator=g).bfloat16().to(DEV)
    k = torch.randn(b, lkv, h, d, generator=g).bfloat16().to(DEV)
    v = torch.randn(b, lkv, h, d, generator=g).bfloat16().to(DEV)
    index = torch.stack([torch.randperm(nkv, generator=g)[:width] for _ in range(b * h * nq)])
    index = index.view(b, h, nq, width).int().to(DEV)
    num = torch.randint(0, width + 1, (b, h, nq), generator=g, dtype=torch.int32)
    num.view(-1)[0] = width            # at least one row cut into the most split units
    num.view(-1)[1] = 0                # an empty row
    return q, k, v, index, num.to(DEV), lq, lkv, bs


def _both(case, heads=None):
    q, k, v, index, num, lq, lkv, bs = case
    res = []
    for noalloc in (False, True):
        out = torch.full(q.shape, float("nan"), dtype=torch.float32, device=DEV)
        _, lse = bsa_forward(q, k, v, index=index, num=num, block_size=bs, layout="blhd", heads=heads, out=out,
                             lq=lq, lkv=lkv, want_lse=True, noalloc=noalloc)
        res.append((out, lse))
    torch.cuda.synchronize()
    return res


def test_noalloc_forward_equals_the_workspace_forward_on_two_calls():
    big = _case(1, b=1, h=3, lq=1000, lkv=8000, width=40)      # up to 3 split units per row
    small = _case(2, b=1, h=2, lq=500, lkv=3000, width=20)     # smaller: reuses the array
    for name, case, heads in (("first", big, None), ("second", small, torch.tensor([1], dtype=torch.int32))):
        if heads is not None:
            heads = heads.to(DEV)
        (ref, ref_lse), (got, got_lse) = _both(case, heads)
        hs = list(range(case[0].shape[2])) if heads is None else heads.tolist()
        assert torch.isfinite(got[:, :, hs]).all(), f"{name} call: unwritten output"
        assert torch.equal(got[:, :, hs], ref[:, :, hs]), f"{name} call: outputs differ"
        assert torch.equal(got_lse[:, hs], ref_lse[:, hs]), f"{name} call: log-sum-exps differ"
    # and the first shape once more after the smaller one
    (ref, ref_lse), (got, got_lse) = _both(big)
    assert torch.equal(got, ref) and torch.equal(got_lse, ref_lse)


def test_noalloc_rejects_oversized_launches_and_workspaces():
    q, k, v, index, num, lq, lkv, bs = _case(3, b=1, h=1, lq=256, lkv=1024, width=8)
    args = _lib.BsaFwdArgs(
        q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3], v.data_ptr(), *v.stride()[:3],
        q.data_ptr(), *q.stride()[:3], _lib.WA_BF16, None,
        index.data_ptr(), num.data_ptr(), 64, None, None, 0,
        1, 64, 40000, 40000, 128, 128, 0.0, _lib.WA_EPI_PLAIN,
        None, 0, 0, 0, 0, None, None, 0, 0, 0,
        None, None, 0, 64, 16, None)
    # 64 heads x 313 query blocks x 4 split units of partials: far beyond the static array; the
    # size check rejects it before any launch, so the small tensors are never read
    need = _lib.lib().wa_bsa_fwd_workspace_bytes(64 * 313, 64, 16, 128, 128)
    assert need > _lib.BSA_FWD_NOALLOC_SCRATCH_BYTES
    rc = _lib.lib().wa_bsa_fwd_noalloc(ctypes.byref(args), ctypes.c_void_p(_lib.stream_ptr(q.device)))
    assert rc == _lib.WA_ERR_ARG and b"static scratch" in _lib.lib().wa_last_error()
    args.workspace = q.data_ptr()
    rc = _lib.lib().wa_bsa_fwd_noalloc(ctypes.byref(args), ctypes.c_void_p(_lib.stream_ptr(q.device)))
    assert rc == _lib.WA_ERR_ARG and b"must be NULL" in _lib.lib().wa_last_error()
