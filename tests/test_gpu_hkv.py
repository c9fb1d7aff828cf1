"""GPU parity of the HKV tier (libworldattention_amd via worldattention_amd.hkv) against the CPU
oracle (oracle/hkv.py).

Tolerances: page selections are bit-exact given the kernel's own scores (checked against the
oracle's stable top-k of those scores); scores and summaries are fp32 means / dot products whose
summation order differs from torch's: |diff| <= 1e-5 * scale-of-data + 1e-6. Re-rotated keys are
fp32 complex products rounded to the key dtype: fp32 within 2e-6, bf16 within one bf16 ulp of the
oracle (the rounding boundary can fall differently when the product is contracted into an FMA).
Values and un-rotated channels are copied bit-exactly.
"""
import math

import pytest
import torch

from oracle import hkv as O
from worldattention_amd import hkv as W
from worldattention_amd.hkv import _ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def freq_table(pairs, positions=64):
    inv = 1.0 / (10000.0 ** (torch.arange(0, pairs, dtype=torch.float64) / pairs))
    return torch.polar(torch.ones(positions, pairs, dtype=torch.float64),
                       torch.outer(torch.arange(positions, dtype=torch.float64), inv))


def close(got, want, rtol=1e-5, atol=1e-6, what=""):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    lim = atol + rtol * want.abs().max().item()
    diff = (got - want).abs().max().item() if got.numel() else 0.0
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(want.shape)}"
    assert diff <= lim, f"{what}: max-abs {diff:.3e} > {lim:.3e}"


def within_one_bf16_ulp(got, want, what=""):
    g, w = got.detach().cpu().float(), want.detach().cpu().float()
    ulp = torch.where(w == 0, torch.full_like(w, 2.0 ** -133), w.abs() * 2.0 ** -7)
    bad = (g - w).abs() > ulp
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one bf16 ulp"
    frac = (g != w).float().mean().item()
    assert frac < 0.01, f"{what}: {frac:.3%} of elements differ"


# ---------------------------------------------------------------------------------------------
# page summaries / query and prompt indices
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,d,b,heads", [(torch.bfloat16, 128, 1, 12), (torch.float32, 24, 2, 2),
                                             (torch.bfloat16, 64, 2, 3), (torch.float32, 128, 1, 4)])
def test_page_key_index_matches_oracle(dtype, d, b, heads):
    torch.manual_seed(d + b)
    fsl, frames, start = 50, 7, 11
    tokens = fsl * frames - 17                    # partial last frame and page
    band = O.temporal_band(O.rope_freqs(1024, d), d)
    keys = torch.randn(b, tokens, heads, d).to(dtype)
    spans = O.page_spans(tokens, 2 * fsl)
    want = O.page_key_index(keys, spans, frame_seq_length=fsl, start_frame=start, temporal_freqs=band)
    got = W.page_key_index(keys.to(DEV), spans, frame_seq_length=fsl, start_frame=start,
                           temporal_freqs=band.to(DEV))
    close(got, want, rtol=2e-3 if dtype == torch.bfloat16 else 1e-5, what=f"summary {dtype} d={d}")
    irregular = [(0, 30), (30, 31), (31, tokens)]      # explicit-span path
    want = O.page_key_index(keys, irregular, frame_seq_length=fsl, start_frame=start, temporal_freqs=band)
    got = W.page_key_index(keys.to(DEV), irregular, frame_seq_length=fsl, start_frame=start, temporal_freqs=band)
    close(got, want, rtol=2e-3 if dtype == torch.bfloat16 else 1e-5, what="irregular spans")


def test_page_key_index_is_start_frame_invariant_on_gpu():
    """The reference's content-space property (tests/test_hkv_retrieval.py:101-137)."""
    torch.manual_seed(0)
    d, heads, ft, frames = 24, 2, 6, 4
    tokens = ft * frames
    band = O.temporal_band(freq_table(d // 2), d)
    content = torch.randn(1, tokens, heads, d)
    out = []
    for start in (0, 9):
        ids = start + torch.arange(tokens) // ft
        rot = torch.view_as_complex(content.double().reshape(1, tokens, heads, d // 2, 2)).clone()
        rot[..., :band.shape[1]] *= band[ids].view(1, tokens, 1, -1)
        stored = torch.view_as_real(rot).reshape(content.shape).float().to(DEV)
        out.append(W.page_key_index(stored, [(0, 12), (12, 24)], frame_seq_length=ft, start_frame=start,
                                    temporal_freqs=band))
    assert out[0].shape == (2, heads * d)
    close(out[0], out[1], atol=1e-3, rtol=0)
    assert W.page_key_index(torch.randn(1, 8, 1, 8, device=DEV), [], frame_seq_length=4, start_frame=0,
                            temporal_freqs=torch.ones(4, 2, dtype=torch.complex64)) is None


@pytest.mark.parametrize("dim", [32, 33, 1536, 4096])
def test_query_and_prompt_index_match_oracle(dim):
    torch.manual_seed(dim)
    q = torch.randn(2, 37, dim)
    close(W.query_index(q.to(DEV)), O.query_index(q), what="query_index")
    close(W.query_index(q.bfloat16().to(DEV)), O.query_index(q.bfloat16()), what="query_index bf16")
    e = torch.randn(1, 11, dim) * 3
    p = W.prompt_index(e.to(DEV))
    close(p, O.prompt_index(e), what="prompt_index")
    assert abs(p.norm().item() - 1.0) < 1e-5
    close(W.prompt_index(e[:, torch.randperm(11)].to(DEV)), p, atol=1e-6, rtol=0, what="token order")


# ---------------------------------------------------------------------------------------------
# scoring and selection
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("pages,dim,k", [(120, 1536, 8), (1, 64, 1), (4096, 256, 33), (777, 100, 777)])
def test_score_topk_matches_oracle(pages, dim, k):
    torch.manual_seed(pages)
    index, q = torch.randn(pages, dim), torch.randn(dim)
    scale = math.sqrt(dim)
    sel, sel_scores, scores = _ops.score_topk(index.to(DEV), q.to(DEV), k, scale=scale, want_scores=True)
    close(scores, O.score_pages(q, index), what="scores")
    s = scores.cpu()
    assert sel.cpu().tolist() == O.stable_topk(s, k)            # bit-exact given identical scores
    assert torch.equal(sel_scores.cpu(), s[sel.cpu().long()])
    assert sel.cpu().tolist() == O.stable_topk(O.score_pages(q, index), k)   # tie-free data


def test_selection_beyond_one_launch_matches_the_oracle():
    """More rows than one selection launch takes: runs of 4096 rows merged, ties across runs to
    the lowest row, masked rows skipped, the full score vector returned."""
    torch.manual_seed(9)
    n, dim, k = 9000, 64, 12
    index = torch.randn(n, dim)
    index[8100] = index[100]          # exact ties in different runs
    index[5000] = index[100]
    q = torch.randn(dim)
    mask = torch.zeros(n, dtype=torch.uint8)
    mask[7:40] = 1
    sel, vals, scores = _ops.score_topk(index.to(DEV), q.to(DEV), k, scale=8.0, mask=mask.to(DEV), want_scores=True)
    want_scores = O.score_pages(q, index, scale=8.0)
    close(scores, want_scores, what="scores")
    masked = scores.cpu().clone()
    masked[mask.bool()] = -float("inf")
    order = torch.sort(masked, descending=True, stable=True).indices[:k]
    assert sel.cpu().tolist() == order.tolist()
    close(vals, masked[order], what="selected scores")


def test_selection_ties_mask_and_empty_slots():
    torch.manual_seed(0)
    base = torch.randn(6, 64)
    index = torch.stack([base[0], base[1], base[0], base[2], base[1], base[0]])  # duplicate rows
    q = base[0].clone()
    sel, _, scores = _ops.score_topk(index.to(DEV), q.to(DEV), 6, want_scores=True)
    assert sel.cpu().tolist() == O.stable_topk(scores.cpu(), 6)
    assert sel.cpu().tolist()[:3] == [0, 2, 5]                   # equal scores: lowest index first
    mask = torch.tensor([1, 0, 0, 1, 0, 1], dtype=torch.uint8)
    sel, sel_scores, _ = _ops.score_topk(index.to(DEV), q.to(DEV), 5, mask=mask.to(DEV))
    sel = sel.cpu().tolist()
    free = [i for i in O.stable_topk(scores.cpu(), 6) if not mask[i]]
    assert sel[:3] == free and sel[3:] == [-1, -1]
    assert torch.isinf(sel_scores[3:].cpu()).all()


def test_stage_functions_match_oracle():
    torch.manual_seed(0)
    bank = torch.nn.functional.normalize(torch.randn(6, 32), dim=1)
    assert W.select_top_chunks(bank[4].clone().to(DEV), bank.to(DEV), 1) == [4]
    assert W.select_top_chunks(bank[4].to(DEV), bank.to(DEV), 6) == O.select_top_chunks(bank[4], bank, 6)
    assert W.select_top_chunks(bank[0].to(DEV), bank.to(DEV), 0) == []
    assert W.select_top_chunks(bank[0].to(DEV), torch.zeros(0, 32, device=DEV), 2) == []
    assert len(W.select_top_chunks(bank[0].to(DEV), bank.to(DEV), 99)) == 6
    cands = [(c, p, torch.randn(32)) for c in range(3) for p in range(4)]
    q = torch.randn(32)
    got = W.select_topk_pages(q.to(DEV), [(c, p, v.to(DEV)) for c, p, v in cands], 4)
    want = O.select_topk_pages(q, cands, 4)
    assert [g[:2] for g in got] == [w[:2] for w in want]
    assert all(abs(g[2] - w[2]) <= 1e-5 for g, w in zip(got, want))
    assert W.select_topk_pages(q.to(DEV), [], 4) == []
    close(W.score_pages(q.to(DEV), torch.stack([c[2] for c in cands]).to(DEV)),
          O.score_pages(q, torch.stack([c[2] for c in cands])), what="score_pages")
    assert W.score_pages(q.to(DEV), torch.zeros(0, 32, device=DEV)).numel() == 0


# ---------------------------------------------------------------------------------------------
# re-rotation
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,d", [(torch.float32, 24), (torch.bfloat16, 128), (torch.float32, 128),
                                     (torch.bfloat16, 30)])
def test_shift_and_derope_match_oracle(dtype, d):
    torch.manual_seed(d)
    band = O.temporal_band(O.rope_freqs(256, d), d)
    k = (torch.randn(2, 90, 3, d) * 2).to(dtype)
    for new, orig in ((40, 3), (3, 40), (7, 7), (300, 0)):
        want = O.shift_temporal_rope(k, band, new, orig)
        got = W.shift_temporal_rope(k.to(DEV), band, new, orig)
        if dtype == torch.bfloat16:
            within_one_bf16_ulp(got, want, what=f"shift {new}<-{orig}")
        else:
            close(got, want, atol=2e-6, rtol=0, what=f"shift {new}<-{orig}")
        nt = O.temporal_complex_dims(d)
        assert torch.equal(got.cpu()[..., 2 * nt:], k[..., 2 * nt:])      # only the band moves
    ids = 5 + torch.arange(90) // 13
    want = O.derope_temporal(k, band, ids)
    got = W.derope_temporal(k.to(DEV), band.to(DEV), ids.to(DEV))
    if dtype == torch.bfloat16:
        within_one_bf16_ulp(got, want, what="derope")
    else:
        close(got, want, atol=2e-6, rtol=0, what="derope")


def test_in_place_rotation_by_rows_touches_only_the_range():
    torch.manual_seed(1)
    d, nt = 128, O.temporal_complex_dims(128)
    band = O.temporal_band(O.rope_freqs(64, d), d)
    k = torch.randn(1, 40, 2, d).bfloat16()
    kd = k.to(DEV)
    factors = _ops.factor_table(band, torch.tensor([9, 20]), torch.tensor([1, 2]), kd.device)
    rows = torch.tensor([0] * 10 + [1] * 15, dtype=torch.int32, device=DEV)
    _ops.rotate_temporal(kd, factors, rows=rows, t0=5, t1=30)
    want = k.clone()
    want[:, 5:15] = O.shift_temporal_rope(k[:, 5:15], band, 9, 1)
    want[:, 15:30] = O.shift_temporal_rope(k[:, 15:30], band, 20, 2)
    within_one_bf16_ulp(kd, want, what="rows")
    assert torch.equal(kd.cpu()[:, :5], k[:, :5]) and torch.equal(kd.cpu()[:, 30:], k[:, 30:])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gather_rotate_equals_copy_then_rerope(dtype):
    """The fused install (pinned pages read by the kernel, re-rope on the way) against DMA copies
    followed by the in-place rotation: bit-identical keys, 40 pages (two launches), pages of
    unequal length out of order, and untouched tokens outside the pages; without factors it is
    a plain copy. Pageable pages are refused."""
    torch.manual_seed(3)
    d, h, b = 128, 3, 2
    nt = O.temporal_complex_dims(d)
    band = O.temporal_band(O.rope_freqs(128, d), d)
    blob = torch.randn(b, 900, h, d).to(dtype).pin_memory()
    spans = [(i * 20 + (i % 3), i * 20 + (i % 3) + 7 + (i % 5)) for i in range(40)]
    spans.reverse()
    pages, off = [], 0
    for s0, s1 in spans:
        pages.append((blob[:, s0:s1], off))
        off += s1 - s0
    factors = _ops.factor_table(band, torch.arange(40) + 50, torch.arange(40), torch.device(DEV))
    cap = off + 9
    got = torch.full((b, cap, h, d), 3.0, dtype=dtype, device=DEV)
    _ops.gather_rotate(pages, got, factors)
    want = torch.full((b, cap, h, d), 3.0, dtype=dtype, device=DEV)
    rows = []
    for i, (src, o) in enumerate(pages):
        want[:, o:o + src.shape[1]] = src.to(DEV)
        rows += [i] * src.shape[1]
    _ops.rotate_temporal(want, factors, rows=torch.tensor(rows, dtype=torch.int32, device=DEV), t0=0, t1=off)
    assert torch.equal(got.cpu(), want.cpu())
    plain = torch.zeros_like(got)
    _ops.gather_rotate(pages, plain, None)
    for src, o in pages:
        assert torch.equal(plain[:, o:o + src.shape[1]].cpu(), src)
    with pytest.raises(ValueError, match="pinned"):
        _ops.gather_rotate([(blob[:, :4].clone(), 0)], got, None)


# ---------------------------------------------------------------------------------------------
# host-tier copies
# ---------------------------------------------------------------------------------------------
def test_pinned_store_and_gather_round_trip_and_pageable_is_rejected():
    torch.manual_seed(2)
    src = torch.randn(2, 64, 3, 8, device=DEV).bfloat16()
    host = torch.empty(2, 40, 3, 8, dtype=torch.bfloat16, pin_memory=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    done = torch.cuda.Event()
    es, row = 2, 3 * 8 * 2
    cp = _ops.PageCopy(src[:, 10:50].data_ptr(), src.stride(0) * es, host.data_ptr(), 40 * row, 40 * row, 2)
    _ops.copy_pages([cp], to_device=False, stream=side, done=done)
    done.synchronize()
    assert torch.equal(host, src[:, 10:50].cpu())
    back = torch.zeros(2, 64, 3, 8, dtype=torch.bfloat16, device=DEV)
    pages = [_ops.PageCopy(host[:, s:s + 8].data_ptr(), 40 * row, back[:, 20 + s:28 + s].data_ptr(),
                           back.stride(0) * es, 8 * row, 2) for s in range(0, 40, 8)]
    issued = _ops.copy_pages(pages, to_device=True, stream=side, done=done)
    assert issued == 1                                            # adjacent pages merge
    torch.cuda.current_stream().wait_event(done)
    torch.cuda.synchronize()
    assert torch.equal(back[:, 20:60], src[:, 10:50]) and back[:, :20].abs().sum() == 0
    pageable = torch.empty(2, 40, 3, 8, dtype=torch.bfloat16)
    bad = _ops.PageCopy(pageable.data_ptr(), 40 * row, back.data_ptr(), back.stride(0) * es, 8 * row, 2)
    with pytest.raises(ValueError, match="pinned"):
        _ops.copy_pages([bad], to_device=True, stream=side)


# ---------------------------------------------------------------------------------------------
# HKVCache end to end (the reference's tests/test_hkv_cache.py scenarios, GPU-resident cache)
# ---------------------------------------------------------------------------------------------
FRAME_TOKENS, PAGE_FRAMES = 4, 2
PAGE_TOKENS = FRAME_TOKENS * PAGE_FRAMES
CAPACITY, BLOCKS, HEADS, HEAD_DIM, PROMPT_DIM = 16, 2, 1, 32, 8
STALE = -999.0
FREQS = O.temporal_band(freq_table(HEAD_DIM // 2, 128), HEAD_DIM)


def hsa_modules():
    from worldattention_amd.hsa import HSAAttention
    mods = []
    for block in range(BLOCKS):
        m = HSAAttention(num_heads=HEADS, head_dim=HEAD_DIM, block_size=64, proj_segment_len=FRAME_TOKENS,
                         backend="torch").to(DEV)
        with torch.no_grad():
            m.k_proj_mat.fill_(0.0)
            m.k_proj_mat[0, :] = (block + 1) / FRAME_TOKENS
            m.v_proj_mat.fill_(0.0)
            m.v_proj_mat[0, :] = (block + 1) / FRAME_TOKENS
        mods.append(m)
    return mods


def make_cache(mods, with_coarse=True, stale=False):
    slots = mods[0].coarse_cache_size(CAPACITY)
    cache = []
    for _ in range(BLOCKS):
        blk = {"k": torch.zeros(1, CAPACITY, HEADS, HEAD_DIM, device=DEV),
               "v": torch.zeros(1, CAPACITY, HEADS, HEAD_DIM, device=DEV),
               "global_end_index": torch.zeros([], dtype=torch.long, device=DEV),
               "local_end_index": torch.zeros([], dtype=torch.long, device=DEV)}
        if with_coarse:
            blk["k_coarse"] = torch.full((1, slots, HEADS, HEAD_DIM), STALE if stale else 0.0, device=DEV)
            blk["v_coarse"] = torch.full((1, slots, HEADS, HEAD_DIM), STALE if stale else 0.0, device=DEV)
        cache.append(blk)
    return cache


def fill(cache, valid, tag):
    for bi, blk in enumerate(cache):
        vals = tag * 1000 + bi * 100 + torch.arange(valid, dtype=torch.float32, device=DEV)
        blk["k"][0, :valid, 0, :] = vals[:, None]
        blk["v"][0, :valid, 0, :] = -vals[:, None]
        blk["local_end_index"].fill_(valid)


def prompt(seed):
    torch.manual_seed(seed)
    return torch.randn(1, 3, PROMPT_DIM, device=DEV)


def bank(topk_pages=2, stage1=2, rerope=False, **kw):
    return W.HKVCache(frame_seq_length=FRAME_TOKENS, page_size_frames=PAGE_FRAMES, topk_pages=topk_pages,
                      stage1_topk_chunks=stage1, rerope=rerope, **kw)


def seed_chunks(bk, mods, count=2):
    for tag in range(1, count + 1):
        c = make_cache(mods)
        fill(c, CAPACITY, tag)
        bk.store(c, prompt_embeds=prompt(tag), current_start_frame=tag * 10, temporal_freqs=FREQS)
    return bk


def test_store_pages_index_and_pinned_blobs():
    mods = hsa_modules()
    bk = bank()
    c = make_cache(mods)
    fill(c, CAPACITY, 1)
    assert bk.store(c, prompt_embeds=prompt(1), current_start_frame=10, temporal_freqs=FREQS) == 0
    ch = bk.chunks[0]
    assert ch["valid_tokens"] == CAPACITY and ch["page_spans"] == [(0, 8), (8, 16)]
    assert ch["start_frame"] == 10 - CAPACITY // FRAME_TOKENS
    assert ch["page_index"].shape == (2, HEADS * HEAD_DIM) and bk.tier.location(0) == "cpu"
    want = O.page_key_index(c[0]["k"].cpu(), ch["page_spans"], frame_seq_length=FRAME_TOKENS,
                            start_frame=ch["start_frame"], temporal_freqs=FREQS)
    close(ch["page_index"], want, what="store page index")
    blob = bk.tier.get(0)
    for bi in range(BLOCKS):
        assert blob["k"][bi].is_pinned() and torch.equal(blob["k"][bi], c[bi]["k"].cpu())
        assert torch.equal(blob["v"][bi], c[bi]["v"].cpu())
    c2 = make_cache(mods)
    fill(c2, 12, 1)
    bk.store(c2, prompt_embeds=prompt(1), current_start_frame=10, temporal_freqs=FREQS)
    assert bk.chunks[1]["page_spans"] == [(0, 8), (8, 12)]
    assert bk.store(make_cache(mods), prompt_embeds=prompt(1), current_start_frame=0, temporal_freqs=FREQS) == -1
    bk.reset()
    assert len(bk) == 0 and bk.tier.location(0) == "absent"


def test_retrieve_matches_the_oracle_pipeline():
    mods = hsa_modules()
    bk = seed_chunks(bank(topk_pages=4, stage1=2), mods)
    assert bank().retrieve(prompt_embeds=prompt(1), query_vec=torch.randn(HEADS * HEAD_DIM)) == []
    target = (1, 1)
    q = bk.chunks[1]["page_index"][1].clone()
    one = bank(topk_pages=1)
    seed_chunks(one, mods)
    assert one.retrieve(prompt_embeds=prompt(2), query_vec=one.chunks[1]["page_index"][1].clone()) == [target]
    torch.manual_seed(5)
    q = torch.randn(HEADS * HEAD_DIM)
    sel = bk.retrieve(prompt_embeds=prompt(1), query_vec=q.to(DEV))
    # oracle: stage 1 over the prompt bank, stage 2 over the pooled pages, chronological order
    bank_cpu = torch.stack([p.cpu() for p in bk.prompt_bank])
    cands = O.select_top_chunks(O.prompt_index(prompt(1).cpu()), bank_cpu, 2)
    pool = [(c, p, bk.chunks[c]["page_index"][p].cpu()) for c in cands for p in range(2)]
    chosen = [(c, p) for c, p, _ in O.select_topk_pages(q, pool, 4)]
    starts = {i: ch["start_frame"] for i, ch in enumerate(bk.chunks)}
    spans = {i: ch["page_spans"] for i, ch in enumerate(bk.chunks)}
    assert sel == O.chronological(chosen, starts, spans)
    assert len(sel) == 4 and len({c for c, _ in sel}) == 2
    with pytest.raises(ValueError):
        bk.retrieve(prompt_embeds=prompt(1), query_vec=torch.randn(5))


def test_apply_installs_pages_verbatim_and_sets_end_indices():
    mods = hsa_modules()
    bk = seed_chunks(bank(topk_pages=1), mods)
    c = make_cache(mods)
    assert bk.apply(c, [(1, 1)], current_start_frame=30, temporal_freqs=FREQS, hsa_modules=mods) == PAGE_TOKENS
    s, e = bk.chunks[1]["page_spans"][1]
    for bi, blk in enumerate(c):
        want = (2 * 1000 + bi * 100 + torch.arange(s, e, dtype=torch.float32))[:, None].expand(-1, HEAD_DIM)
        assert torch.equal(blk["k"][0, :PAGE_TOKENS, 0].cpu(), want)
        assert (blk["k"][0, PAGE_TOKENS:] == 0).all()
        assert int(blk["local_end_index"]) == PAGE_TOKENS and int(blk["global_end_index"]) == 30 * FRAME_TOKENS


def test_apply_refreshes_kept_key_block_sums():
    """A cache that keeps key block sums for routing gets them recomputed for the installed pages."""
    from worldattention_amd.hsa.kvcache import kv_append
    mods = hsa_modules()
    bk = seed_chunks(bank(topk_pages=1), mods)
    c = make_cache(mods)
    torch.manual_seed(4)
    for blk in c:
        x = torch.randn(1, CAPACITY, HEADS, HEAD_DIM, device=DEV)
        kv_append(blk, x, x, write_start=0, block_size=4)
    n = bk.apply(c, [(1, 1)], current_start_frame=30, temporal_freqs=FREQS, hsa_modules=mods)
    for blk in c:
        k = blk["k"][0, :n, 0].cpu().double()
        want = k.reshape(n // 4, 4, HEAD_DIM).sum(1)
        got = blk["k_block_sums"][0, 0, : n // 4].cpu().double()
        assert torch.allclose(got, want, rtol=1e-6, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_apply_reropes_keys_like_the_oracle(dtype):
    mods = hsa_modules()
    bk = bank(topk_pages=2, rerope=True)
    torch.manual_seed(9)
    for tag in (1, 2):
        c = make_cache(mods)
        for blk in c:
            blk["k"] = torch.randn(1, CAPACITY, HEADS, HEAD_DIM, device=DEV).to(dtype)
            blk["v"] = torch.randn(1, CAPACITY, HEADS, HEAD_DIM, device=DEV).to(dtype)
            blk["local_end_index"].fill_(CAPACITY)
        bk.store(c, prompt_embeds=prompt(tag), current_start_frame=tag * 10, temporal_freqs=FREQS)
    c = make_cache(mods)
    for blk in c:
        blk["k"], blk["v"] = blk["k"].to(dtype), blk["v"].to(dtype)
    for blk in c:
        del blk["k_coarse"], blk["v_coarse"]
    selected = [(0, 1), (1, 0)]
    total = bk.apply(c, selected, current_start_frame=30, temporal_freqs=FREQS.to(DEV))
    assert total == 2 * PAGE_TOKENS
    entries = [(cid, *bk.chunks[cid]["page_spans"][pid]) for cid, pid in selected]
    starts = {i: ch["start_frame"] for i, ch in enumerate(bk.chunks)}
    installed, moves = O.install_plan(entries, CAPACITY, 30, FRAME_TOKENS, starts)
    for bi, blk in enumerate(c):
        off = 0
        for (cid, s, e), (orig, new) in zip(installed, moves):
            src = bk.tier.get(cid)
            want = O.shift_temporal_rope(src["k"][bi][:, s:e], FREQS, new, orig)
            got = blk["k"][:, off:off + e - s]
            if dtype == torch.bfloat16:
                within_one_bf16_ulp(got, want, what=f"layer {bi} page {cid}:{s}")
            else:
                close(got, want, atol=2e-6, rtol=0, what=f"layer {bi} page {cid}:{s}")
            assert torch.equal(blk["v"][:, off:off + e - s].cpu(), src["v"][bi][:, s:e])
            off += e - s


def test_apply_truncates_noops_skips_and_requires_modules():
    mods = hsa_modules()
    bk = seed_chunks(bank(topk_pages=4, stage1=2), mods)
    sel = bk.retrieve(prompt_embeds=prompt(1), query_vec=torch.randn(HEADS * HEAD_DIM, device=DEV))
    c = make_cache(mods)
    assert bk.apply(c, sel, current_start_frame=30, temporal_freqs=FREQS, hsa_modules=mods) == CAPACITY
    assert int(c[0]["local_end_index"]) == CAPACITY
    c = make_cache(mods)
    fill(c, CAPACITY, 7)
    assert bk.apply(c, [], current_start_frame=30, temporal_freqs=FREQS, hsa_modules=mods) == 0
    assert c[0]["k"].abs().sum() > 0
    c = make_cache(mods)
    assert bk.apply(c, [(99, 0), (0, 99), (0, 0)], current_start_frame=30, temporal_freqs=FREQS,
                    hsa_modules=mods) == PAGE_TOKENS
    with pytest.raises(ValueError):
        bk.apply(make_cache(mods, stale=True), [(0, 0)], current_start_frame=30, temporal_freqs=FREQS)
    c = make_cache(mods, with_coarse=False)
    assert bk.apply(c, [(0, 0)], current_start_frame=30, temporal_freqs=FREQS) == PAGE_TOKENS
    assert all("k_coarse" not in blk for blk in c)


def test_apply_rebuilds_the_compressed_tier_per_layer():
    mods = hsa_modules()
    bk = seed_chunks(bank(topk_pages=2, stage1=2), mods)
    sel = bk.retrieve(prompt_embeds=prompt(1), query_vec=torch.randn(HEADS * HEAD_DIM, device=DEV))
    c = make_cache(mods, stale=True)
    n = bk.apply(c, sel, current_start_frame=30, temporal_freqs=FREQS, hsa_modules=mods)
    for bi, blk in enumerate(c):
        assert not (blk["k_coarse"] == STALE).any() and not (blk["v_coarse"] == STALE).any()
        lk, lv = blk["k"][:, :n], blk["v"][:, :n]
        # known answer: rank-1 projection rows of (block+1)/4 average each 4-token segment x (block+1)
        want_k = lk.reshape(1, n // 4, 4, HEADS, HEAD_DIM).mean(dim=2) * (bi + 1)
        close(blk["k_coarse"][:, :n // 4], want_k, rtol=1e-2, what="coarse k")
        with torch.no_grad():
            ek, ev = mods[bi].compress_kv_cache(lk, lv)
        close(blk["k_coarse"][:, :ek.shape[1]], ek, atol=1e-4, rtol=0, what="coarse k == compress")
        close(blk["v_coarse"][:, :ev.shape[1]], ev, atol=1e-4, rtol=0, what="coarse v == compress")
        assert (blk["k_coarse"][:, ek.shape[1]:] == 0).all()


def test_pages_survive_an_nvme_round_trip(tmp_path):
    mods = hsa_modules()
    bk = seed_chunks(bank(topk_pages=1, nvme_enabled=True, nvme_dir=str(tmp_path), cpu_max_chunks=1), mods)
    assert bk.tier.location(0) == "nvme"
    c = make_cache(mods)
    assert bk.apply(c, [(0, 0)], current_start_frame=30, temporal_freqs=FREQS, hsa_modules=mods) == PAGE_TOKENS
    assert bk.tier.stats()["n_loads"] >= 1
    assert torch.equal(c[0]["k"][0, 0, 0].cpu(), torch.full((HEAD_DIM,), 1000.0))


def test_per_layer_events_let_attention_start_before_the_last_layer():
    mods = hsa_modules()
    bk = seed_chunks(bank(topk_pages=2), mods)
    c = make_cache(mods)
    n = bk.apply(c, [(0, 0), (1, 1)], current_start_frame=30, temporal_freqs=FREQS, hsa_modules=mods, wait=False)
    assert len(bk.layer_events) == BLOCKS
    for bi in range(BLOCKS):
        bk.wait_layer(bi)
        got = c[bi]["k"][0, :n, 0, 0].clone()
        assert got[0].item() == 1000 + bi * 100 and got[PAGE_TOKENS].item() == 2000 + bi * 100 + 8
