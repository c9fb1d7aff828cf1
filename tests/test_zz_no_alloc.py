"""wa_bsa_fwd_noalloc (the block-sparse forward whose workspace is the library's static device array)
against wa_bsa_fwd with a caller-allocated workspace: outputs and log-sum-exps bit-identical, on two
calls in a row (the second smaller, so it runs on what the first left in the array), with rows
long enough to be cut into several split units (the partials and arrival counters that live in
the array are used). Its argument rejections (a launch needing more than the array, a caller
workspace) are host-side checks, tested without a GPU in test_capi.py."""
import pytest
import torch

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
