"""Pins of the cache-write oracle (``oracle/cache.py``) on the CPU: the RMSNorm against an fp64
brute force and a known answer, the 3-D RoPE against a per-element rotation built from the angle
formula, and the cache step's contents against the sliding-window invariant."""
import math

import pytest
import torch

from oracle import cache as OC
from oracle import hkv as OK
from oracle import hsa as OH


def test_rms_norm_matches_fp64_and_a_constant_row():
    torch.manual_seed(0)
    x = torch.randn(2, 5, 96)
    w = torch.randn(96)
    got = OC.rms_norm(x, w, 1e-6)
    xd = x.double()
    want = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    torch.testing.assert_close(got.double(), want, rtol=1e-6, atol=1e-6)
    c = torch.full((1, 1, 64), -3.0)
    out = OC.rms_norm(c, torch.full((64,), 2.0), 0.0)
    assert torch.equal(out, torch.full((1, 1, 64), -2.0))
    assert OC.rms_norm(x, None, 1e-6) is x


def _brute_rope(x, frames, height, width, start_frame, theta=10000.0):
    """a cos t - b sin t, a sin t + b cos t per complex pair, t from the band's angle formula."""
    b, length, heads, d = x.shape
    half = d // 2
    ct, ch = half - 2 * (half // 3), half // 3
    dims = (2 * ct, 2 * ch, 2 * ch)
    out = x.clone()
    for s in range(length):
        f, r = divmod(s, height * width)
        hh, ww = divmod(r, width)
        for c in range(half):
            if c < ct:
                pos, j, dim = start_frame + f, c, dims[0]
            elif c < ct + ch:
                pos, j, dim = hh, c - ct, dims[1]
            else:
                pos, j, dim = ww, c - ct - ch, dims[2]
            t = pos / theta ** (2 * j / dim)
            a, bb = x[:, s, :, 2 * c], x[:, s, :, 2 * c + 1]
            out[:, s, :, 2 * c] = a * math.cos(t) - bb * math.sin(t)
            out[:, s, :, 2 * c + 1] = a * math.sin(t) + bb * math.cos(t)
    return out


@pytest.mark.parametrize("d", [64, 128])
def test_causal_rope_matches_a_per_element_rotation(d):
    torch.manual_seed(d)
    x = torch.randn(1, 2 * 3 * 4 + 5, 2, d, dtype=torch.float64)
    freqs = OK.rope_freqs(64, d)
    got = OC.causal_rope(x, (2, 3, 4), freqs, start_frame=7)
    want = _brute_rope(x[:, :24], 2, 3, 4, 7)
    torch.testing.assert_close(got[:, :24], want, rtol=1e-12, atol=1e-12)
    assert torch.equal(got[:, 24:], x[:, 24:])  # past the grid: unrotated


def test_causal_rope_with_one_grid_per_sample_matches_a_per_element_rotation():
    """A batch whose samples have different grids (``causal_model.py:43`` loops over them): each
    sample rotates by its own grid and passes the tokens past it through."""
    torch.manual_seed(3)
    d = 64
    x = torch.randn(2, 30, 2, d, dtype=torch.float64)
    freqs = OK.rope_freqs(64, d)
    grids = [(2, 3, 4), (1, 5, 5)]
    got = OC.causal_rope(x, grids, freqs, start_frame=3)
    for i, (f, h, w) in enumerate(grids):
        seq = f * h * w
        want = _brute_rope(x[i:i + 1, :seq], f, h, w, 3)
        torch.testing.assert_close(got[i:i + 1, :seq], want, rtol=1e-12, atol=1e-12)
        assert torch.equal(got[i, seq:], x[i, seq:])


def _ids(n, h, d, start):
    """Tokens whose every channel holds the token's global index (exact in fp32)."""
    t = torch.arange(start, start + n, dtype=torch.float32).view(1, n, 1, 1)
    return t.expand(1, n, h, d).clone()


def test_cache_step_keeps_sink_frames_then_the_latest_frames():
    """Chunks of 3 frames into a 7-frame cache with a 1-frame sink: after every step the values
    are the sink's tokens followed by the most recent tokens, in order; a recompute step rewrites
    its chunk but not the sink, and leaves the indices where they were."""
    fs, h, d = 8, 2, 16                      # tokens per frame (grid 1 x 2 x 4), heads, head dim
    grid = (3, 2, 4)
    chunk, cap, sink = 3 * fs, 7 * fs, fs
    freqs = OK.rope_freqs(256, d)
    cache = {"k": torch.zeros(1, cap, h, d), "v": torch.zeros(1, cap, h, d),
             "global_end_index": torch.tensor([0]), "local_end_index": torch.tensor([0])}
    for step in range(5):
        start = step * chunk
        x = _ids(chunk, h, d, start)
        _, ak, av, _, _, info = OC.cache_step(cache, x, x, x, grid=grid, freqs=freqs, current_start=start,
                                              sink_size=1, local_attn_size=7, max_attention_size=cap)
        end = start + chunk
        le = int(cache["local_end_index"])
        assert int(cache["global_end_index"]) == end and le == min(end, cap)
        ids = cache["v"][0, :le, 0, 0]
        recent = torch.arange(end - (le - sink), end, dtype=torch.float32)
        want = torch.cat([torch.arange(sink, dtype=torch.float32), recent]) if end > cap else torch.arange(end, dtype=torch.float32)
        assert torch.equal(ids, want), f"step {step}: {ids.tolist()}"
        assert torch.equal(av[0, :, 0, 0], want)
        assert info["action"] == ("roll_and_insert" if end > cap else "direct_insert")
    # recompute the last chunk with new values: the sink survives, the indices stay
    before = cache["v"].clone()
    start = 4 * chunk
    x = _ids(chunk, h, d, start) + 0.5
    _, _, _, _, _, info = OC.cache_step(cache, x, x, x, grid=grid, freqs=freqs, current_start=start,
                                        sink_size=1, local_attn_size=7, max_attention_size=cap)
    assert info["is_recompute"] and int(cache["global_end_index"]) == 5 * chunk
    ws = info["write_start_index"]
    assert torch.equal(cache["v"][:, :ws], before[:, :ws])
    assert torch.equal(cache["v"][0, ws:cap, 0, 0], torch.arange(start, start + chunk, dtype=torch.float32)[-(cap - ws):] + 0.5)


def test_cache_step_coarse_tier_equals_compressing_the_window():
    """With a coarse tier (one segment per frame), the coarse slots of the cached frames equal
    compressing the cached tokens segment by segment, after inserts and rolls."""
    torch.manual_seed(3)
    fs, h, d, bs = 16, 2, 16, 64
    grid = (2, 4, 4)
    chunk, cap, sink = 2 * fs, 6 * fs, fs
    rank = math.ceil(fs / bs)
    kp, vp = torch.rand(rank, fs) / 8, OH.init_projection(rank, fs, bs, dtype=torch.float32)
    freqs = OK.rope_freqs(256, d)
    lc = OH.coarse_cache_size(cap, fs, rank)
    cache = {"k": torch.zeros(1, cap, h, d), "v": torch.zeros(1, cap, h, d), "k_coarse": torch.zeros(1, lc, h, d),
             "v_coarse": torch.zeros(1, lc, h, d), "global_end_index": torch.tensor([0]),
             "local_end_index": torch.tensor([0])}
    for step in range(5):
        x = torch.randn(1, chunk, h, d)
        OC.cache_step(cache, x, x, x, grid=grid, freqs=freqs, current_start=step * chunk, sink_size=1,
                      local_attn_size=6, max_attention_size=cap, proj=(kp, vp, fs, bs))
        le = int(cache["local_end_index"])
        wk, wv = OH.compress_kv(cache["k"][:, :le].transpose(1, 2), cache["v"][:, :le].transpose(1, 2),
                                segment_len=fs, k_proj_mat=kp, v_proj_mat=vp, block_size=bs)
        assert torch.equal(cache["k_coarse"][:, :le // fs * rank].transpose(1, 2), wk)
        assert torch.equal(cache["v_coarse"][:, :le // fs * rank].transpose(1, 2), wv)
