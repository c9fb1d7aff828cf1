"""GPU parity of the fused QKV epilogue and the in-place cache roll against the cache-write oracle.

Tolerances: values, and roped queries / keys without the RMSNorm, bit-exact (the rotation uses
the oracle's fp64 products and roundings). With the RMSNorm, the sum of squares is formed in
torch's CPU fp32 order but the factor is the correctly rounded 1 / sqrt, while torch's CPU rsqrt
(MKL) differs from that in the last fp32 bit for ~0.65% of inputs: a normed element may then sit
one bf16 ulp away, so roped q / k are checked to within one bf16 ulp of the larger element of their
rotation pair, with at most 0.1% of elements off at all (fp32: four fp32 ulps, at most 2% off).
Coarse slots within
1e-2 max-abs / 1e-3 mean-abs (compression: fp32 sums in another order, one bf16 rounding); cache
indices and attention windows equal; routing from the kept key block sums equal to pooling the
window's keys.
"""
import math

import pytest
import torch

from oracle import cache as OC
from oracle import hkv as OK
from worldattention_amd import _lib
from worldattention_amd import hsa as W
from worldattention_amd.hsa import kvcache as KV
from worldattention_amd.hsa.routing import _route, block_counts, pool_blhd_many, pool_for_routing

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, want, max_abs, mean_abs, what):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    assert got.shape == want.shape, f"{what}: {tuple(got.shape)} vs {tuple(want.shape)}"
    diff = (got - want).abs()
    assert diff.max().item() <= max_abs and diff.mean().item() <= mean_abs, (
        f"{what}: max {diff.max().item():.3e} mean {diff.mean().item():.3e}")


def _within_pair_ulp(got, want, what):
    """|got - want| <= one bf16 ulp (2^-7 relative) of max(|want| over its RoPE pair), at most 0.1%
    of elements off; fp32: four fp32 ulps (2^-20), at most 2% off (an rsqrt bit moves a whole row,
    with no bf16 rounding to absorb it)."""
    fp32 = want.dtype == torch.float32
    rel, max_frac = (2.0 ** -20, 2e-2) if fp32 else (2.0 ** -7, 1e-3)
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    assert got.shape == want.shape, f"{what}: {tuple(got.shape)} vs {tuple(want.shape)}"
    pair = want.reshape(*want.shape[:-1], -1, 2).abs().amax(-1, keepdim=True).expand(*want.shape[:-1], -1, 2)
    pair = pair.reshape(want.shape)
    diff = (got - want).abs()
    assert (diff <= rel * pair + 1e-30).all(), f"{what}: max excess {(diff - rel * pair).max().item():.3e}"
    off = (diff > 0).float().mean().item()
    assert off <= max_frac, f"{what}: {off:.2%} of elements differ"


def _equal(got, want, what):
    got, want = got.detach().cpu(), want.detach().cpu()
    assert got.shape == want.shape, f"{what}: {tuple(got.shape)} vs {tuple(want.shape)}"
    if not torch.equal(got, want):
        bad = (got.float() != want.float()).sum().item()
        raise AssertionError(f"{what}: {bad} of {got.numel()} elements differ")


@pytest.mark.parametrize("dtype,w_dtype,d", [(torch.bfloat16, torch.bfloat16, 128), (torch.bfloat16, torch.float32, 64),
                                             (torch.float32, torch.float32, 64), (torch.bfloat16, None, 128)])
def test_qkv_epilogue_matches_oracle(dtype, w_dtype, d):
    """Norm + RoPE of every query token, norm + RoPE + insert of the written key tokens and the
    value copy, with a source offset (the reference's recompute write), tokens past the grid
    (unrotated), a start frame and a batch of two."""
    torch.manual_seed(d)
    b, h, grid = 2, 3, (3, 4, 6)
    n = 3 * 4 * 6 + 5
    cap, ws, so = 400, 77, 9
    wl = n - so
    q, k, v = (torch.randn(b, n, h, d).to(dtype) * 3 for _ in range(3))
    wq = wk = None
    if w_dtype is not None:
        wq, wk = (torch.rand(h * d).to(w_dtype) + 0.5 for _ in range(2))
    freqs = OK.rope_freqs(1024, d)
    cache = {"k": torch.full((b, cap, h, d), 5.0, dtype=dtype, device=DEV),
             "v": torch.full((b, cap, h, d), -5.0, dtype=dtype, device=DEV)}
    got_q = KV.qkv_epilogue(q.to(DEV), k.to(DEV), v.to(DEV), cache, grid_sizes=torch.tensor([list(grid)] * b),
                            freqs=freqs, start_frame=11, write_start=ws, src_offset=so, write_len=wl,
                            norm_q=None if wq is None else wq.to(DEV), norm_k=None if wk is None else wk.to(DEV),
                            eps=1e-6, block_size=64)
    shape = (b, n, h * d)
    nq = OC.rms_norm(q.reshape(shape), wq, 1e-6).reshape(b, n, h, d)
    nk = OC.rms_norm(k.reshape(shape), wk, 1e-6).reshape(b, n, h, d)
    want_q = OC.causal_rope(nq, grid, freqs, 11).to(dtype)
    want_k = OC.causal_rope(nk, grid, freqs, 11).to(dtype)
    same = _equal if w_dtype is None else _within_pair_ulp
    same(got_q, want_q, "roped q")
    same(cache["k"][:, ws:ws + wl], want_k[:, so:], "cache k")
    _equal(cache["v"][:, ws:ws + wl], v[:, so:], "cache v")
    assert (cache["k"][:, :ws] == 5).all() and (cache["k"][:, ws + wl:] == 5).all(), "writes outside the slot"
    # the written blocks' sums: block means of the cache's first ws + wl tokens
    L = ws + wl
    sums = cache["k_block_sums"]
    _, pad, _, nkv = block_counts(L, L, 64)
    first = ws // 64
    (means,) = pool_blhd_many([(cache["k"], L, nkv)], 64)
    real = torch.full((nkv,), 64.0, device=DEV)
    real[-1] = L - (nkv - 1) * 64
    got_means = sums[:, :, first:nkv] / real[first:].view(1, 1, -1, 1)
    if dtype == torch.float32 and L % 64:
        _close(got_means, means[:, :, first:], 1e-5, 1e-6, "block sums / count")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qkv_epilogue_with_one_grid_per_sample_matches_oracle(dtype):
    """grid_sizes with a grid of its own per sample (``causal_model.py:43`` loops over them): three
    samples, the first two sharing a grid (one launch) and the third with another (a second
    launch); each sample's tokens past its grid pass through unrotated. No norm: bit-exact."""
    torch.manual_seed(7)
    b, h, d, n = 3, 2, 64, 80
    grids = [[2, 4, 8], [2, 4, 8], [3, 5, 5]]   # 64, 64 and 75 tokens
    q, k, v = (torch.randn(b, n, h, d).to(dtype) * 3 for _ in range(3))
    freqs = OK.rope_freqs(64, d)
    cache = {"k": torch.zeros(b, 128, h, d, dtype=dtype, device=DEV),
             "v": torch.zeros(b, 128, h, d, dtype=dtype, device=DEV)}
    got_q = KV.qkv_epilogue(q.to(DEV), k.to(DEV), v.to(DEV), cache, grid_sizes=torch.tensor(grids), freqs=freqs,
                            start_frame=5, write_start=20, src_offset=0, write_len=n)
    _equal(got_q, OC.causal_rope(q, grids, freqs, 5).to(dtype), "roped q, per-sample grids")
    _equal(cache["k"][:, 20:20 + n], OC.causal_rope(k, grids, freqs, 5).to(dtype), "cache k, per-sample grids")
    _equal(cache["v"][:, 20:20 + n], v, "cache v")


def test_qkv_epilogue_rejects_bad_arguments():
    d, h = 64, 2
    q = torch.randn(1, 10, h, d, device=DEV).bfloat16()
    cache = {"k": torch.zeros(1, 16, h, d, dtype=torch.bfloat16, device=DEV),
             "v": torch.zeros(1, 16, h, d, dtype=torch.bfloat16, device=DEV)}
    freqs = OK.rope_freqs(8, d)
    with pytest.raises(ValueError, match="does not fit"):
        KV.qkv_epilogue(q, q, q, cache, grid_sizes=(1, 2, 5), freqs=freqs, start_frame=0, write_start=10)
    with pytest.raises(ValueError, match="rows of the RoPE table"):
        KV.qkv_epilogue(q, q, q, cache, grid_sizes=(1, 2, 5), freqs=freqs, start_frame=8, write_start=0)
    with pytest.raises(ValueError, match="grids for a batch"):
        KV.qkv_epilogue(q, q, q, cache, grid_sizes=[[1, 2, 5], [2, 1, 5]], freqs=freqs, start_frame=0,
                        write_start=0)
    q2 = torch.randn(2, 10, h, d, device=DEV).bfloat16()
    cache2 = {n: torch.zeros(2, 16, h, d, dtype=torch.bfloat16, device=DEV) for n in ("k", "v")}
    with pytest.raises(ValueError, match="rows of the RoPE table"):  # checked for every sample
        KV.qkv_epilogue(q2, q2, q2, cache2, grid_sizes=[[1, 2, 5], [1, 1, 9]], freqs=freqs, start_frame=0,
                        write_start=0)
    with pytest.raises(ValueError, match="both RMSNorm"):
        KV.qkv_epilogue(q, q, q, cache, grid_sizes=(1, 2, 5), freqs=freqs, start_frame=0, write_start=0,
                        norm_q=torch.ones(h * d, device=DEV))


@pytest.mark.parametrize("evicted", [8, 100, 700])
def test_kv_roll_in_place_equals_clone_and_shift(evicted):
    """Shifts shorter and longer than the moved range (launch chunking), bf16, with the coarse rows."""
    torch.manual_seed(evicted)
    b, cap, h, d, sink = 2, 1024, 3, 64, 40
    rolled = cap - sink - evicted - 13
    k = torch.randn(b, cap, h, d, device=DEV).bfloat16()
    v = torch.randn(b, cap, h, d, device=DEV).bfloat16()
    want_k, want_v = k.clone(), v.clone()
    want_k[:, sink:sink + rolled] = k[:, sink + evicted:sink + evicted + rolled].clone()
    want_v[:, sink:sink + rolled] = v[:, sink + evicted:sink + evicted + rolled].clone()
    cache = {"k": k, "v": v}
    KV.kv_roll(cache, sink_tokens=sink, num_evicted=evicted, num_rolled=rolled, block_size=64)
    _equal(cache["k"], want_k, "rolled k")
    _equal(cache["v"], want_v, "rolled v")


def _module(h, d, seg, bs=64):
    m = W.HSAAttention(h, d, block_size=bs, proj_segment_len=seg, routing="topk", topk=[4] * h).to(DEV)
    torch.manual_seed(1)
    with torch.no_grad():
        m.k_proj_mat.copy_((torch.rand(m.proj_rank, seg) / 16).bfloat16())
        m.v_proj_mat.copy_((torch.rand(m.proj_rank, seg) / 16).bfloat16())
    return m


@pytest.mark.parametrize("sink_size,max_frames", [(1, 7), (0, 7), (1, 5)])
def test_cache_step_sequence_matches_oracle(sink_size, max_frames):
    """Six chunks of three frames through a seven-frame cache (inserts, then rolls) and a
    recompute of the last chunk, with RMSNorm, the coarse tier and the key block sums: every
    step's roped queries, attention window and cache equal the oracle's; the coarse slots match
    within tolerance; routing over the window from the kept sums equals pooling its keys."""
    torch.manual_seed(7 + sink_size + max_frames)
    b, h, d, gh, gw = 1, 2, 64, 4, 32
    fs = gh * gw
    grid = (3, gh, gw)
    chunk, cap = 3 * fs, 7 * fs
    m = _module(h, d, fs)
    rank = m.proj_rank
    lc = m.coarse_cache_size(cap)
    freqs = OK.rope_freqs(1024, d)
    wq, wk = (torch.rand(h * d) + 0.5).bfloat16(), (torch.rand(h * d) + 0.5).bfloat16()
    gpu = {"k": torch.zeros(b, cap, h, d, dtype=torch.bfloat16, device=DEV),
           "v": torch.zeros(b, cap, h, d, dtype=torch.bfloat16, device=DEV),
           "k_coarse": torch.zeros(b, lc, h, d, dtype=torch.bfloat16, device=DEV),
           "v_coarse": torch.zeros(b, lc, h, d, dtype=torch.bfloat16, device=DEV),
           "global_end_index": torch.tensor([0], device=DEV), "local_end_index": torch.tensor([0], device=DEV)}
    cpu = {key: t.cpu().clone() for key, t in gpu.items()}
    proj = (m.k_proj_mat.detach().cpu(), m.v_proj_mat.detach().cpu(), fs, 64)
    kw = dict(grid_sizes=grid, sink_size=sink_size, local_attn_size=max_frames, max_attention_size=max_frames * fs,
              eps=1e-6)
    starts = [i * chunk for i in range(6)] + [5 * chunk]
    for step, start in enumerate(starts):
        q, k, v = (torch.randn(b, chunk, h, d).bfloat16() for _ in range(3))
        rq, ak, av, akc, avc, info = KV.cache_step(gpu, q.to(DEV), k.to(DEV), v.to(DEV), freqs=freqs,
                                                   current_start=start, norm_q=wq.to(DEV), norm_k=wk.to(DEV),
                                                   hsa_module=m, block_size=64, **kw)
        oq, ok_, ov, okc, ovc, oinfo = OC.cache_step(cpu, q, k, v, freqs=freqs, current_start=start, norm_q=wq,
                                                     norm_k=wk, proj=proj, **{k2: v2 for k2, v2 in kw.items()
                                                                              if k2 != "grid_sizes"}, grid=grid)
        what = f"step {step} (start {start})"
        for key in ("action", "write_start_index", "write_end_index", "local_end_index", "is_recompute",
                    "num_evicted_tokens"):
            assert info[key] == oinfo[key], f"{what}: {key} {info[key]} vs {oinfo[key]}"
        _within_pair_ulp(rq, oq, f"{what}: roped q")
        _within_pair_ulp(ak, ok_, f"{what}: window k")
        _equal(av, ov, f"{what}: window v")
        _within_pair_ulp(gpu["k"], cpu["k"], f"{what}: cache k")
        _equal(gpu["v"], cpu["v"], f"{what}: cache v")
        assert int(gpu["global_end_index"]) == int(cpu["global_end_index"])
        assert int(gpu["local_end_index"]) == int(cpu["local_end_index"])
        le = int(cpu["local_end_index"])
        _close(gpu["k_coarse"][:, :le // fs * rank], cpu["k_coarse"][:, :le // fs * rank], 1e-2, 1e-3,
               f"{what}: k_coarse")
        _close(gpu["v_coarse"][:, :le // fs * rank], cpu["v_coarse"][:, :le // fs * rank], 1e-2, 1e-3,
               f"{what}: v_coarse")
        if akc is not None:
            _close(akc, okc, 1e-2, 1e-3, f"{what}: window k_coarse")
        sums = info["k_block_sums"]
        if sums is not None:
            L = ak.shape[1]
            _, _, nq, nkv = block_counts(rq.shape[1], L, 64)
            qp, kp = pool_blhd_many([(rq, rq.shape[1], nq), (ak, L, nkv)], 64)
            qp2, held, key_args = pool_for_routing(rq, ak, rq.shape[1], L, 64, k_block_sums=sums)
            _, p_want = _route(None, qp, kp, mode=_lib.WA_ROUTE_TOPK, head_k=[4] * h, want_probs=True)
            _, p_got = _route(None, qp2, held, mode=_lib.WA_ROUTE_TOPK, head_k=[4] * h, want_probs=True,
                              **key_args)
            _equal(p_got, p_want, f"{what}: routing from the kept sums")


def test_cache_step_with_one_grid_per_sample_matches_oracle():
    """A batch of two whose samples have their own grids (the second holds two frames of the
    three-frame chunk, so its last frame's tokens pass through unrotated): four chunks through a
    five-frame cache with a one-frame sink (inserts, then rolls), with RMSNorm; the frame length and
    the cache indices come from sample 0, as the reference's step takes them."""
    torch.manual_seed(21)
    b, h, d, gh, gw = 2, 2, 64, 4, 32
    fs = gh * gw
    grids = [[3, gh, gw], [2, gh, gw]]
    chunk, cap = 3 * fs, 5 * fs
    freqs = OK.rope_freqs(1024, d)
    wq, wk = (torch.rand(h * d) + 0.5).bfloat16(), (torch.rand(h * d) + 0.5).bfloat16()
    gpu = {"k": torch.zeros(b, cap, h, d, dtype=torch.bfloat16, device=DEV),
           "v": torch.zeros(b, cap, h, d, dtype=torch.bfloat16, device=DEV),
           "global_end_index": torch.tensor([0], device=DEV), "local_end_index": torch.tensor([0], device=DEV)}
    cpu = {key: t.cpu().clone() for key, t in gpu.items()}
    kw = dict(sink_size=1, local_attn_size=5, max_attention_size=5 * fs, eps=1e-6)
    for step, start in enumerate(i * chunk for i in range(4)):
        q, k, v = (torch.randn(b, chunk, h, d).bfloat16() for _ in range(3))
        rq, ak, av, _, _, info = KV.cache_step(gpu, q.to(DEV), k.to(DEV), v.to(DEV), grid_sizes=torch.tensor(grids),
                                               freqs=freqs, current_start=start, norm_q=wq.to(DEV),
                                               norm_k=wk.to(DEV), **kw)
        oq, ok_, ov, _, _, oinfo = OC.cache_step(cpu, q, k, v, grid=grids, freqs=freqs, current_start=start,
                                                 norm_q=wq, norm_k=wk, **kw)
        what = f"step {step} (start {start})"
        for key in ("write_start_index", "write_end_index", "local_end_index", "num_evicted_tokens"):
            assert info[key] == oinfo[key], f"{what}: {key} {info[key]} vs {oinfo[key]}"
        _within_pair_ulp(rq, oq, f"{what}: roped q")
        _within_pair_ulp(ak, ok_, f"{what}: window k")
        _equal(av, ov, f"{what}: window v")
        _within_pair_ulp(gpu["k"], cpu["k"], f"{what}: cache k")
        _equal(gpu["v"], cpu["v"], f"{what}: cache v")
