"""GPU parity of the cache-write side: ``kv_append`` against slice assignment, the block sums it
keeps against the oracle's block pooling, the coarse slots it fills against ``oracle.compress_kv``,
and HSA calls that read the cached sums against calls that pool the keys.

Tolerances: cache writes bit-exact; routing from cached sums bit-exact against routing from pooled
keys (the same means are formed, so probabilities, orders and counts are equal); block sums / real
count within fp32 summation-order noise (1e-5 relative) of the oracle's fp32 block means; coarse
rows within 1e-2 max-abs / 1e-3 mean-abs of the oracle (one bf16 rounding of fp32 sums in another
order); HSA outputs with cached sums identical to the outputs without.
"""
import math

import pytest
import torch

from oracle import hsa as O
from worldattention_amd import hsa as W
from worldattention_amd import _lib
from worldattention_amd.hsa import attention as WA
from worldattention_amd.hsa.routing import _route, block_counts, pool_blhd_many, pool_for_routing

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _assert_close(got, want, max_abs, mean_abs, what):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(want.shape)}"
    diff = (got - want).abs()
    assert diff.max().item() <= max_abs, f"{what}: max-abs {diff.max().item():.3e}"
    assert diff.mean().item() <= mean_abs, f"{what}: mean-abs {diff.mean().item():.3e}"


def _empty_cache(b, cap, h, d, dtype):
    # non-zero garbage, so a write that misses its slot shows
    return {"k": torch.full((b, cap, h, d), 7.0, dtype=dtype, device=DEV),
            "v": torch.full((b, cap, h, d), -3.0, dtype=dtype, device=DEV)}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bs", [64, 128])
def test_kv_append_writes_and_block_sums(dtype, bs):
    """Ragged chunks appended in turn (partial blocks completed by the next chunk), a strided
    (non-contiguous) source, and a head subset for the sums on the last append."""
    torch.manual_seed(11)
    b, cap, h, d = 2, 1000, 3, 128
    cache = _empty_cache(b, cap, h, d, dtype)
    want_k, want_v = cache["k"].clone(), cache["v"].clone()
    start = 0
    for n in (100, 37, 1, 250, 64, 300):
        k_new = torch.randn(b, n, h, d, device=DEV).to(dtype)
        v_new = torch.randn(b, h, n, d, device=DEV).to(dtype).transpose(1, 2)  # BLHD view of BHLD memory
        info = W.kv_append(cache, k_new, v_new, write_start=start, block_size=bs)
        want_k[:, start:start + n] = k_new
        want_v[:, start:start + n] = v_new
        assert torch.equal(cache["k"], want_k) and torch.equal(cache["v"], want_v), f"cache after [{start}, +{n})"
        assert info["write_start_index"] == start and info["write_end_index"] == start + n
        start += n
        # every written block: sums / real == the oracle's fp32 means of the first `start` tokens
        _, pad, _, nkv = block_counts(start, start, bs)
        kf = torch.zeros(b, h, pad, d)
        kf[:, :, :start] = want_k[:, :start].float().transpose(1, 2).cpu()
        want_mean = O.block_mean_pool(kf, start, nkv, bs)  # fp32 input: no rounding, means of real tokens
        real = torch.full((nkv,), float(bs))
        real[-1] = start - (nkv - 1) * bs
        got_mean = cache["k_block_sums"][:, :, :nkv].cpu() / real.view(1, 1, nkv, 1)
        torch.testing.assert_close(got_mean, want_mean, rtol=1e-5, atol=1e-6)
        assert not cache["k_block_sums"][:, :, nkv:].any(), "blocks past the written tokens"
    # sums of a head subset: the other heads keep their previous sums
    before = cache["k_block_sums"].clone()
    cache["k"][:, :start] += 1  # change every key, so recomputed sums differ
    W.kv_append(cache, cache["k"][:, start - 10:start].clone(), cache["v"][:, start - 10:start].clone(),
                write_start=start - 10, block_size=bs, heads=[0, 2])
    last = (start - 1) // bs
    after = cache["k_block_sums"]
    assert torch.equal(after[:, 1], before[:, 1])
    assert torch.equal(after[:, [0, 2], :last], before[:, [0, 2], :last])
    assert not torch.equal(after[:, [0, 2], last], before[:, [0, 2], last])


def test_kv_append_rejects_bad_ranges():
    cache = _empty_cache(1, 300, 2, 64, torch.bfloat16)
    k_new = torch.randn(1, 50, 2, 64, device=DEV).bfloat16()
    with pytest.raises(ValueError, match="do not fit"):
        W.kv_append(cache, k_new, k_new, write_start=260, block_size=64)
    with pytest.raises(ValueError, match="new k / v"):
        W.kv_append(cache, k_new[:, :, :1], k_new[:, :, :1], write_start=0, block_size=64)
    W.kv_append(cache, k_new, k_new, write_start=0, block_size=64)
    with pytest.raises(ValueError, match="block_size"):
        W.kv_append(cache, k_new, k_new, write_start=50)


@pytest.mark.parametrize("kv_len", [4000, 3968, 130])
def test_routing_from_cached_sums_equals_pooled_keys(kv_len):
    """Bit-exact: probabilities (the general route kernel), top-k and Gini selections (the wave
    kernel / the general kernel) from the cached sums equal those from pooling the keys, with the
    cache longer than the routed keys (sums read in place, row stride of the whole cache)."""
    torch.manual_seed(kv_len)
    b, cap, h, d, bs = 1, 4608, 4, 128, 64
    cache = _empty_cache(b, cap, h, d, torch.bfloat16)
    base = torch.randn(b, cap, h, d, device=DEV).bfloat16()
    for s0 in range(0, kv_len, 1560):
        n = min(1560, kv_len - s0)
        W.kv_append(cache, base[:, s0:s0 + n], base[:, s0:s0 + n], write_start=s0, block_size=bs)
    q = torch.randn(b, 700, h, d, device=DEV).bfloat16()
    k = cache["k"][:, :kv_len]
    _, _, nq, nkv = block_counts(700, kv_len, bs)
    qp, kp = pool_blhd_many([(q, 700, nq), (k, kv_len, nkv)], bs)
    qp2, held, key_args = pool_for_routing(q, k, 700, kv_len, bs, k_block_sums=cache["k_block_sums"])
    assert held.data_ptr() == cache["k_block_sums"].data_ptr() and held.shape[2] == cap // bs
    assert torch.equal(qp, qp2)
    _, p_want = _route(None, qp, kp, mode=_lib.WA_ROUTE_TOPK, head_k=[8] * h, want_probs=True)
    r_got, p_got = _route(None, qp2, held, mode=_lib.WA_ROUTE_TOPK, head_k=[8] * h, want_probs=True, **key_args)
    assert torch.equal(p_got, p_want)
    ks = [4, 8, 16, 60]
    r_want, _ = _route(None, qp, kp, mode=_lib.WA_ROUTE_TOPK, head_k=ks)
    r_got, _ = _route(None, qp2, held, mode=_lib.WA_ROUTE_TOPK, head_k=ks, **key_args)
    assert torch.equal(r_got.num, r_want.num)
    for hh, kk in enumerate(ks):
        kk = min(kk, nkv)
        assert torch.equal(r_got.index[:, hh, :, :kk], r_want.index[:, hh, :, :kk])
    g_want, _ = _route(None, qp, kp, mode=_lib.WA_ROUTE_GINI, tau_min=0.35, tau_max=1.0)
    g_got, _ = _route(None, qp2, held, mode=_lib.WA_ROUTE_GINI, tau_min=0.35, tau_max=1.0, **key_args)
    assert torch.equal(g_got.thresholds, g_want.thresholds) and torch.equal(g_got.num, g_want.num)
    assert torch.equal(g_got.index, g_want.index)
    # against the oracle: the routed probabilities of the keys the cache holds
    qf = torch.zeros(b, h, nq * bs, d, dtype=torch.bfloat16)
    qf[:, :, :700] = q.transpose(1, 2).cpu()
    kf = torch.zeros(b, h, nkv * bs, d, dtype=torch.bfloat16)
    kf[:, :, :kv_len] = k.transpose(1, 2).cpu()
    want = O.block_attention_map(O.block_mean_pool(qf, 700, nq, bs), O.block_mean_pool(kf, kv_len, nkv, bs))
    _assert_close(p_got, want, 1e-5, 1e-7, "routing probabilities vs oracle")


def _module(h, d, bs, seg=1560):
    m = W.HSAAttention(h, d, block_size=bs, proj_segment_len=seg, routing="topk", topk=[8, 16, 4, 32][:h],
                       head_modes=["both", "sparse", "linear", "both"][:h]).to(DEV)
    torch.manual_seed(5)
    with torch.no_grad():
        m.k_proj_mat.copy_((torch.rand(m.proj_rank, seg) / 40).bfloat16())
        m.v_proj_mat.copy_(O.init_projection(m.proj_rank, seg, bs))
        m.gate_lin.weight.copy_(torch.randn(d, d) * 0.02)
        m.gate_lin.bias.copy_(torch.randn(d) * 0.02)
    return m


def test_kv_append_fills_coarse_cache_like_the_oracle():
    """Three segment-aligned chunks (one, two and one 1560-token segments): each chunk's coarse
    rows land at ``token_range_to_coarse`` and match ``oracle.compress_kv`` of the chunk; an
    unaligned range is refused before anything is written."""
    torch.manual_seed(2)
    b, h, d, bs, seg = 1, 4, 128, 64, 1560
    m = _module(h, d, bs, seg)
    cap = 5 * seg
    cache = _empty_cache(b, cap, h, d, torch.bfloat16)
    lc = m.coarse_cache_size(cap)
    cache["k_coarse"] = torch.zeros(b, lc, h, d, dtype=torch.bfloat16, device=DEV)
    cache["v_coarse"] = torch.zeros(b, lc, h, d, dtype=torch.bfloat16, device=DEV)
    start = 0
    for n_seg in (1, 2, 1):
        n = n_seg * seg
        k_new = torch.randn(b, n, h, d, device=DEV).bfloat16()
        v_new = torch.randn(b, n, h, d, device=DEV).bfloat16()
        info = W.kv_append(cache, k_new, v_new, write_start=start, block_size=bs, hsa_module=m)
        c0, c1 = O.token_range_to_coarse(start, start + n, seg, m.proj_rank)
        assert info["new_k_coarse"].shape[1] == c1 - c0
        wk, wv = O.compress_kv(k_new.transpose(1, 2).cpu(), v_new.transpose(1, 2).cpu(), segment_len=seg,
                               k_proj_mat=m.k_proj_mat.detach().cpu(), v_proj_mat=m.v_proj_mat.detach().cpu(),
                               block_size=bs)
        _assert_close(cache["k_coarse"][:, c0:c1].transpose(1, 2), wk, 1e-2, 1e-3, f"k_coarse [{c0}, {c1})")
        _assert_close(cache["v_coarse"][:, c0:c1].transpose(1, 2), wv, 1e-2, 1e-3, f"v_coarse [{c0}, {c1})")
        start += n
    assert not cache["k_coarse"][:, start // seg * m.proj_rank:].any(), "the unwritten segment's slots"
    snap = {key: t.clone() for key, t in cache.items() if isinstance(t, torch.Tensor)}
    with pytest.raises(ValueError, match="segment-aligned"):
        W.kv_append(cache, k_new[:, :100], v_new[:, :100], write_start=0, block_size=bs, hsa_module=m)
    for key, t in snap.items():
        assert torch.equal(cache[key], t), f"{key} changed by a refused append"


@pytest.mark.parametrize("routing", ["topk", "gini"])
def test_hsa_with_cached_sums_equals_pooling_the_keys(routing):
    """A decode-style sequence: chunks appended, then an HSA call over the cache prefix, with and
    without the cached sums (and with ``k_pooled`` means), at a length that ends mid-block and one
    that ends on a block boundary."""
    torch.manual_seed(7)
    b, h, d, bs, seg = 1, 4, 128, 64, 1560
    m = _module(h, d, bs, seg)
    m.routing = routing
    cap = 3 * seg
    cache = _empty_cache(b, cap, h, d, torch.bfloat16)
    start = 0
    for n in (1560, 1560, 1520):  # 3120 = 48.75 blocks, 4640 = 72.5 blocks, then 4680
        k_new = torch.randn(b, n, h, d, device=DEV).bfloat16()
        v_new = torch.randn(b, n, h, d, device=DEV).bfloat16()
        W.kv_append(cache, k_new, v_new, write_start=start, block_size=bs)
        start += n
        q = torch.randn(b, 1560, h, d, device=DEV).bfloat16()
        k, v = cache["k"][:, :start], cache["v"][:, :start]
        with torch.no_grad():
            want = m(q, k, v)
            got = m(q, k, v, k_block_sums=cache["k_block_sums"])
            nkv = math.ceil(start / bs)
            (kp,) = pool_blhd_many([(k, start, nkv)], bs)
            got_p = m(q, k, v, k_pooled=kp)
        assert torch.equal(got, want), f"cached sums, {start} tokens"
        assert torch.equal(got_p, want), f"k_pooled, {start} tokens"
    with pytest.raises(ValueError, match="not both"):
        with torch.no_grad():
            m(q, k, v, k_block_sums=cache["k_block_sums"], k_pooled=kp)
