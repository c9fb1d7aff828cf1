"""Pins the CPU HKV oracle (oracle/hkv.py) against the reference tests' known answers
(tests/test_hkv_rope.py, test_hkv_retrieval.py, test_hkv_cache.py) and against independent
formulations: a full three-band RoPE applied from scratch, fp64 brute-force means, torch.topk on
tie-free scores and hand-derived page plans."""
import math

import pytest
import torch

from oracle import hkv as O

HEAD_DIM, HEADS = 24, 2
FRAMES, LAT_H, LAT_W = 4, 2, 3
FRAME_TOKENS = LAT_H * LAT_W
MAX_POS = 64


def freq_table(pairs, positions=MAX_POS):
    inv = 1.0 / (10000.0 ** (torch.arange(0, pairs, dtype=torch.float64) / pairs))
    return torch.polar(torch.ones(positions, pairs, dtype=torch.float64),
                       torch.outer(torch.arange(positions, dtype=torch.float64), inv))


def full_rope(x, freqs, start_frame, temporal_at_zero=False):
    """All three bands rotated from scratch for tokens laid out (frame, h, w): the independent
    statement the band-only shift / de-rope must agree with."""
    tokens, heads, d = x.shape
    pairs = d // 2
    t_band, h_band, w_band = freqs.split([pairs - 2 * (pairs // 3), pairs // 3, pairs // 3], dim=1)
    out = torch.view_as_complex(x.double().reshape(tokens, heads, pairs, 2)).clone()
    for tok in range(tokens):
        f, rem = divmod(tok, LAT_H * LAT_W)
        hh, ww = divmod(rem, LAT_W)
        pos = torch.cat([t_band[0 if temporal_at_zero else start_frame + f], h_band[hh], w_band[ww]])
        out[tok] = out[tok] * pos
    return torch.view_as_real(out).reshape(tokens, heads, d).to(x.dtype)


def setup():
    torch.manual_seed(0)
    x = torch.randn(FRAMES * FRAME_TOKENS, HEADS, HEAD_DIM)
    freqs = freq_table(HEAD_DIM // 2)
    return x, freqs, O.temporal_band(freqs, HEAD_DIM)


def test_temporal_band_width_matches_the_wan_rope_split():
    for d in range(2, 258, 2):
        assert O.temporal_complex_dims(d) == (d - 4 * (d // 6)) // 2   # model.py:29-36 split
    assert O.temporal_complex_dims(128) == 22
    assert O.rope_freqs(8, 128).shape == (8, 64)


def test_shift_equals_encoding_at_the_new_frame():
    x, freqs, band = setup()
    enc = full_rope(x, freqs, 3)
    shifted = O.shift_temporal_rope(enc.unsqueeze(0), band, 11, 3).squeeze(0)
    assert torch.allclose(shifted, full_rope(x, freqs, 11), atol=1e-4)


def test_shift_by_zero_and_inverse():
    x, freqs, band = setup()
    enc = full_rope(x, freqs, 5)
    assert torch.allclose(O.shift_temporal_rope(enc.unsqueeze(0), band, 5, 5).squeeze(0), enc, atol=1e-5)
    there = O.shift_temporal_rope(enc.unsqueeze(0), band, 9, 5)
    assert torch.allclose(O.shift_temporal_rope(there, band, 5, 9).squeeze(0), enc, atol=1e-4)


def test_derope_equals_spatial_only_encoding_and_is_position_free():
    x, freqs, band = setup()
    spatial = full_rope(x, freqs, 0, temporal_at_zero=True)
    for start in (0, 6, 21):
        ids = start + torch.arange(FRAMES * FRAME_TOKENS) // FRAME_TOKENS
        out = O.derope_temporal(full_rope(x, freqs, start).unsqueeze(0), band, ids).squeeze(0)
        assert torch.allclose(out, spatial, atol=1e-4)


def test_positions_beyond_the_table_are_clamped():
    x, _, band = setup()
    out = O.shift_temporal_rope(x.unsqueeze(0), band, MAX_POS + 100, 0)
    assert torch.isfinite(out).all()
    same = O.shift_temporal_rope(x.unsqueeze(0), band, MAX_POS - 1, 0)
    assert torch.equal(out, same)


def test_rope_apply_3d_matches_the_per_token_rotation():
    torch.manual_seed(1)
    d, heads, frames, hgt, wid = 24, 2, 3, 2, 2
    freqs = O.rope_freqs(32, d)
    x = torch.randn(1, frames * hgt * wid, heads, d)
    got = O.rope_apply_3d(x, freqs, frames, hgt, wid, start_frame=4)
    pairs = d // 2
    ft, fh, fw = freqs.split([pairs - 2 * (pairs // 3), pairs // 3, pairs // 3], dim=1)
    want = torch.view_as_complex(x.double().reshape(1, -1, heads, pairs, 2)).clone()
    for tok in range(frames * hgt * wid):
        f, rem = divmod(tok, hgt * wid)
        hh, ww = divmod(rem, wid)
        want[0, tok] *= torch.cat([ft[4 + f], fh[hh], fw[ww]])
    assert torch.allclose(got, torch.view_as_real(want).reshape(x.shape).float(), atol=1e-5)


def test_page_key_index_is_content_space_and_a_brute_force_mean():
    torch.manual_seed(0)
    d, heads, ft, frames = 24, 2, 6, 4
    tokens = ft * frames
    band = O.temporal_band(freq_table(d // 2), d)
    content = torch.randn(2, tokens, heads, d)
    spans = [(0, 10), (10, tokens)]
    idx = []
    for start in (0, 9):
        ids = start + torch.arange(tokens) // ft
        rot = torch.view_as_complex(content.double().reshape(2, tokens, heads, d // 2, 2)).clone()
        rot[..., :band.shape[1]] *= band[ids].view(1, tokens, 1, -1)
        stored = torch.view_as_real(rot).reshape(content.shape).float()
        idx.append(O.page_key_index(stored, spans, frame_seq_length=ft, start_frame=start, temporal_freqs=band))
    assert idx[0].shape == (2, heads * d)
    assert torch.allclose(idx[0], idx[1], atol=1e-3)
    brute = torch.zeros(2, heads * d, dtype=torch.float64)
    flat = content.double().reshape(2, tokens, heads * d)
    for p, (s, e) in enumerate(spans):
        for b in range(2):
            acc = torch.zeros(heads * d, dtype=torch.float64)
            for t in range(s, e):
                acc += flat[b, t]
            brute[p] += acc / (e - s) / 2
    assert torch.allclose(idx[0].double(), brute, atol=1e-4)
    assert O.page_key_index(torch.randn(1, 8, 1, 8), [], frame_seq_length=4, start_frame=0,
                            temporal_freqs=torch.ones(4, 2, dtype=torch.complex64)) is None


def test_query_and_prompt_index():
    torch.manual_seed(0)
    q = torch.randn(2, 5, 32)
    assert torch.allclose(O.query_index(q), q.double().sum(dim=(0, 1)).float() / 10, atol=1e-6)
    e = torch.randn(2, 7, 32)
    p = O.prompt_index(e)
    assert abs(p.norm().item() - 1.0) < 1e-5
    assert torch.allclose(p, O.prompt_index(e[:, torch.randperm(7)]), atol=1e-6)


def test_scores_use_the_sqrt_dim_scale_and_topk_agrees_with_torch_on_distinct_scores():
    torch.manual_seed(0)
    q, pages = torch.randn(32), torch.randn(5, 32)
    assert torch.allclose(O.score_pages(q, pages), pages @ q / math.sqrt(32), atol=1e-5)
    assert torch.allclose(O.score_pages(q, pages, scale=0.0), pages @ q)
    assert O.score_pages(q, torch.zeros(0, 32)).numel() == 0
    for seed in range(5):
        torch.manual_seed(seed)
        s = torch.randn(300)
        assert O.stable_topk(s, 17) == torch.topk(s, 17).indices.tolist()


def test_stable_topk_breaks_ties_by_lowest_index():
    s = torch.tensor([1.0, 3.0, 3.0, 2.0, 3.0, 2.0])
    assert O.stable_topk(s, 4) == [1, 2, 4, 3]
    assert O.stable_topk(s, 0) == [] and O.stable_topk(s, 99) == [1, 2, 4, 3, 5, 0]


def test_stage1_and_stage2_selection():
    torch.manual_seed(0)
    bank = torch.nn.functional.normalize(torch.randn(6, 32), dim=1)
    assert O.select_top_chunks(bank[4].clone(), bank, 1) == [4]
    scores = (bank @ bank[4]).tolist()
    assert O.select_top_chunks(bank[4], bank, 6) == sorted(range(6), key=lambda i: -scores[i])
    assert O.select_top_chunks(bank[0], bank, 0) == [] and len(O.select_top_chunks(bank[0], bank, 99)) == 6
    cands = [(c, p, torch.randn(32)) for c in range(3) for p in range(4)]
    q = torch.randn(32)
    sel = O.select_topk_pages(q, cands, 4)
    want = torch.topk(torch.stack([c[2] for c in cands]) @ q / math.sqrt(32), 4).indices.tolist()
    assert [cands.index(next(c for c in cands if c[0] == a and c[1] == b)) for a, b, _ in sel] == want
    assert O.select_topk_pages(cands[9][2].clone(), cands, 1)[0][:2] == (2, 1)


def test_page_bookkeeping_known_answers():
    """Page spans, chronological order and the install / re-rope plan of the reference cache tests
    (tests/test_hkv_cache.py: 4-token frames, 2-frame pages, 16-token capacity)."""
    assert O.page_spans(16, 8) == [(0, 8), (8, 16)]
    assert O.page_spans(12, 8) == [(0, 8), (8, 12)]
    assert O.page_spans(0, 8) == []
    start_frames = {0: 10 - 16 // 4, 1: 20 - 16 // 4}
    spans = {0: [(0, 8), (8, 16)], 1: [(0, 8), (8, 16)]}
    assert O.chronological([(1, 0), (0, 1), (1, 1), (0, 0)], start_frames, spans) == [(0, 0), (0, 1), (1, 0), (1, 1)]
    installed, moves = O.install_plan([(1, 8, 16)], 16, 30, 4, start_frames)
    assert installed == [(1, 8, 16)] and moves == [(16 + 8 // 4, 30 - 8 // 4)]
    installed, moves = O.install_plan([(0, 0, 8), (0, 8, 16), (1, 0, 8), (1, 8, 16)], 16, 30, 4, start_frames)
    assert installed == [(0, 0, 8), (0, 8, 16)]
    assert moves == [(6, 26), (8, 28)]
    installed, _ = O.install_plan([(0, 0, 8), (1, 8, 12)], 10, 30, 4, start_frames)
    assert installed == [(0, 0, 8), (1, 8, 10)]
