"""GPU parity at the benchmark geometries that the unit tests only cover in pieces: cfg 4 (one
H = 40 layer call of the Wan-14B stack) and cfg 3 (the HKV tier at its real page geometry, through
``HKVCache.store -> retrieve -> apply`` and an HSA call over the page pool).

Tolerances: attention outputs max-abs <= 2e-2 and mean-abs <= 2e-3 against the fp32 oracle; routing
and page selections bit-exact given identical scores; page summaries within fp32 reduction-order
noise; installed keys within one bf16 ulp (plus the fp32 product error where a rotation cancels)
of the oracle's re-rope, values bit-exact.
"""
import pytest
import torch

from oracle import hkv as OK
from oracle import hsa as O
from worldattention_amd import hkv as WK
from worldattention_amd import hsa as W
from worldattention_amd import workloads
from worldattention_amd.hsa import attention as WA

pytestmark = pytest.mark.gpu
DEV = "cuda"


def assert_close(got, want, max_abs=2e-2, mean_abs=2e-3, what=""):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(want.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    diff = (got - want).abs()
    assert diff.max().item() <= max_abs, f"{what}: max-abs {diff.max().item():.3e} > {max_abs}"
    assert diff.mean().item() <= mean_abs, f"{what}: mean-abs {diff.mean().item():.3e} > {mean_abs}"


def check_topk_routing(route, parts, ks, heads, what, tie_rel=1e-5, max_tie_rows=0.01):
    """The fused route kernel scores the pooled blocks itself, in its own fp32 summation order, so
    two blocks whose oracle probabilities agree to ~1e-7 may trade places. Every listed position must
    hold the oracle's block, or a block whose oracle probability is within ``tie_rel`` of it; rows
    with such swaps must be rare. Separately, the selection from identical scores (the oracle's own
    map through the GPU top-k) must equal the oracle's exactly."""
    amap = parts["attn_map"]
    want = parts["routing"]
    got_idx, got_num = route.index.cpu(), route.num.cpu()
    rows, swapped = 0, 0
    for h in heads:
        k = ks[h]
        assert torch.equal(got_num[:, h], want.num[:, h]), f"{what}: num of head {h}"
        g, r = got_idx[0, h, :, :k], want.index[0, h, :, :k]
        p = amap[0, h]
        for i in range(g.shape[0]):
            rows += 1
            if torch.equal(g[i], r[i]):
                continue
            swapped += 1
            for m in torch.nonzero(g[i] != r[i]).flatten().tolist():
                pg, pr = p[i, g[i, m]].item(), p[i, r[i, m]].item()
                assert abs(pg - pr) <= tie_rel * pr, (
                    f"{what}: head {h} row {i} slot {m}: block {int(g[i, m])} (p={pg:.9g}) vs oracle "
                    f"{int(r[i, m])} (p={pr:.9g})")
    assert swapped <= max_tie_rows * rows, f"{what}: {swapped} of {rows} rows differ by near-ties"
    same_scores = W.build_topk_routing(amap.to(DEV), ks)
    for h in heads:
        k = ks[h]
        assert torch.equal(same_scores.index.cpu()[:, h, :, :k], want.index[:, h, :, :k]), f"{what}: head {h}"
        assert torch.equal(same_scores.num.cpu()[:, h], want.num[:, h])
    return swapped


def within_bf16_of_rotation(got, want, what):
    """Rotated bf16 keys: both sides form the fp32 complex product of a key pair and a unit factor
    (error up to ~2^-21 of the pair's magnitude, depending on how each side fuses the products) and
    round it to bf16, so they may differ by one bf16 ulp of the value plus that fp32 error (which
    dominates where the product cancels to near zero)."""
    g, w = got.detach().cpu().float(), want.detach().cpu().float()
    pair = w.reshape(*w.shape[:-1], w.shape[-1] // 2, 2).norm(dim=-1)
    mag = pair.repeat_interleave(2, dim=-1)
    tol = w.abs() * 2.0 ** -7 + mag * 2.0 ** -20
    bad = (g - w).abs() > tol
    if bad.any():
        i = torch.nonzero(bad)[0].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} elements beyond one bf16 ulp (first {i}: "
                             f"{g[tuple(i)].item():.6g} vs {w[tuple(i)].item():.6g}, pair magnitude "
                             f"{mag[tuple(i)].item():.4g})")
    frac = (g != w).float().mean().item()
    assert frac < 0.01, f"{what}: {frac:.3%} of elements differ"


def hsa_both(q, k, v, cfg, gate_w=None, gate_b=None):
    """(GPU output, GPU routing, oracle output, oracle parts) of one head-adaptive HSA call."""
    d = q.shape[-1]
    kw = dict(block_size=cfg["block_size"], routing="topk", topk=cfg["topk"], head_modes=cfg["head_modes"],
              linear_mode=cfg["linear_mode"], proj_segment_len=cfg.get("proj_segment_len", 1560))
    gate_w = torch.zeros(d, d) if gate_w is None else gate_w
    gate_b = torch.zeros(d) if gate_b is None else gate_b
    want, parts = O.hsa_attention(q.cpu(), k.cpu(), v.cpu(), gate_weight=gate_w, gate_bias=gate_b,
                                  return_parts=True, **kw)
    lin = torch.nn.Linear(d, d).to(DEV)
    with torch.no_grad():
        lin.weight.copy_(gate_w)
        lin.bias.copy_(gate_b)
    save = {}
    with torch.no_grad():
        got = WA.hsa_forward(q.to(DEV), k.to(DEV), v.to(DEV), k_coarse=None, v_coarse=None, k_proj_mat=None,
                             v_proj_mat=None, gate_lin=lin, tau_min=0.35, tau_max=1.0, save=save, **kw)
    return got, save["route"], want, parts


# ----------------------------------------------------------------------------------------------
# cfg 4: one H = 40 layer call (30 sparse heads at top-16, 10 elu1 heads), 4,680 vs 32,760 tokens
# ----------------------------------------------------------------------------------------------
def test_cfg4_h40_layer_call_matches_oracle():
    cfg = workloads.cfg4_layer(seed=0)
    q, k, v = cfg["q"], cfg["k"], cfg["v"]
    assert q.shape == (1, 4680, 40, 128) and k.shape == (1, 32760, 40, 128) and q.dtype == torch.bfloat16
    g = torch.Generator().manual_seed(4)
    gate_w, gate_b = torch.randn(128, 128, generator=g) * 0.02, torch.zeros(128)
    got, route, want, parts = hsa_both(q, k, v, cfg, gate_w, gate_b)
    sparse = [h for h, m in enumerate(cfg["head_modes"]) if m == "sparse"]
    assert len(sparse) == 30 and route.num.shape == (1, 40, 37)
    check_topk_routing(route, parts, cfg["topk"], sparse, "cfg4")
    linear = [h for h, m in enumerate(cfg["head_modes"]) if m == "linear"]
    assert_close(got[:, :, linear], want[:, :, linear], what="cfg4 elu1 heads")
    assert_close(got, want, what="cfg4 H=40 call")


# ----------------------------------------------------------------------------------------------
# cfg 3: 120 one-frame pages of 1,560 tokens, H = 12, D = 128, bf16; frames 0..113 banked as 19
# six-frame chunks (pinned host tier), frames 114..119 resident; top-8 pages installed in front of
# the resident frames and re-roped to frames 106..113; HSA over the 21,840-token pool.
# ----------------------------------------------------------------------------------------------
def test_cfg3_hkv_page_geometry_through_the_cache_api():
    cfg = workloads.cfg3(DEV, seed=0, layers=1)
    ft, hist, hf, nres, nret = (cfg[n] for n in ("frame_tokens", "history_frames", "host_frames",
                                                 "resident_frames", "retrieved"))
    heads, d = cfg["q"].shape[2], cfg["q"].shape[3]
    assert (ft, hist, hf, nres, nret, heads, d) == (1560, 120, 114, 6, 8, 12, 128)
    band = OK.temporal_band(cfg["freqs"], d)            # [positions, 22] complex128 on the device
    band_cpu = band.cpu()
    keys0 = cfg["keys0"]                                 # layer-0 roped keys of all 120 frames
    host_k, host_v = cfg["host_k"][0], cfg["host_v"][0]  # frames 0..113, pinned
    dev_v = host_v.to(DEV)

    chunk_frames = 6
    n_chunks = hf // chunk_frames
    bank = WK.HKVCache(frame_seq_length=ft, page_size_frames=1, topk_pages=nret, stage1_topk_chunks=n_chunks,
                       cpu_max_chunks=64, rerope=True)
    gp = torch.Generator().manual_seed(3)
    for c in range(n_chunks):
        s, e = c * chunk_frames * ft, (c + 1) * chunk_frames * ft
        blk = {"k": keys0[:, s:e], "v": dev_v[:, s:e],
               "local_end_index": torch.tensor(e - s, device=DEV), "global_end_index": torch.tensor(e, device=DEV)}
        assert bank.store([blk], prompt_embeds=torch.randn(1, 4, 64, generator=gp),
                          current_start_frame=(c + 1) * chunk_frames, temporal_freqs=band) == c
    torch.cuda.synchronize()
    del dev_v

    # page summaries of every chunk against the oracle's de-roped means
    for c in range(n_chunks):
        ch = bank.chunks[c]
        assert ch["start_frame"] == c * chunk_frames and len(ch["page_spans"]) == chunk_frames
        s = c * chunk_frames * ft
        want = OK.page_key_index(keys0[:, s:s + chunk_frames * ft].cpu(), ch["page_spans"], frame_seq_length=ft,
                                 start_frame=c * chunk_frames, temporal_freqs=band_cpu)
        got = ch["page_index"].cpu()
        lim = 1e-6 + 1e-5 * want.abs().max().item()
        assert (got - want).abs().max().item() <= lim, f"chunk {c} page summaries"

    # retrieval: the oracle's stage 2 over the same summaries, chronological; the planted frames
    qvec = WK.query_index(cfg["q_content"])
    pairs = bank.retrieve(prompt_embeds=torch.randn(1, 4, 64, generator=gp), query_vec=qvec)
    cands = [(c, p, bank.chunks[c]["page_index"][p].cpu()) for c in range(n_chunks) for p in range(chunk_frames)]
    chosen = OK.select_topk_pages(OK.query_index(cfg["q_content"].cpu()), cands, nret)
    starts = {c: bank.chunks[c]["start_frame"] for c in range(n_chunks)}
    spans = {c: bank.chunks[c]["page_spans"] for c in range(n_chunks)}
    assert pairs == OK.chronological([(c, p) for c, p, _ in chosen], starts, spans)
    frames = [c * chunk_frames + p for c, p in pairs]
    assert frames == sorted(cfg["truth"])
    scores = OK.score_pages(OK.query_index(cfg["q_content"].cpu()), torch.stack([x[2] for x in cands]))
    top = torch.sort(scores, descending=True).values
    assert (top[nret - 1] - top[nret]).item() > 1e-3 * top[nret - 1].abs().item(), "selection boundary is a near-tie"

    # install into the online cache: the first 8 frame slots of the pool, in front of the resident
    # frames (which the cache view does not cover, so apply leaves them alone)
    pool_k, pool_v = cfg["pool_k"][0], cfg["pool_v"][0]
    resident_k = pool_k[:, nret * ft:].clone()
    pool_k[:, : nret * ft].fill_(7.0)                   # stale contents the install must overwrite
    pool_v[:, : nret * ft].fill_(7.0)
    cache = [{"k": pool_k[:, : nret * ft], "v": pool_v[:, : nret * ft],
              "global_end_index": torch.zeros([], dtype=torch.long, device=DEV),
              "local_end_index": torch.zeros([], dtype=torch.long, device=DEV)}]
    base = hist - nres                                   # the resident frames start here
    n = bank.apply(cache, pairs, current_start_frame=base, temporal_freqs=band, wait=False)
    bank.wait_layer(0)
    assert n == nret * ft
    assert int(cache[0]["local_end_index"]) == n and int(cache[0]["global_end_index"]) == base * ft
    assert torch.equal(pool_k[:, nret * ft:], resident_k)
    got_k, got_v = pool_k[:, :n].cpu(), pool_v[:, :n].cpu()
    for i, f in enumerate(frames):
        src_k = host_k[:, f * ft:(f + 1) * ft]
        want_k = OK.shift_temporal_rope(src_k, band_cpu, base - nret + i, f)
        within_bf16_of_rotation(got_k[:, i * ft:(i + 1) * ft], want_k, f"page {f}: re-roped keys")
        assert torch.equal(got_v[:, i * ft:(i + 1) * ft], host_v[:, f * ft:(f + 1) * ft]), f"page {f}: values"

    # the HSA call over the 21,840-token pool (171 key blocks, the last with 80 real tokens)
    assert pool_k.shape[1] == 21840
    cfg3 = dict(block_size=cfg["block_size"], topk=cfg["topk"], head_modes=cfg["head_modes"],
                linear_mode=cfg["linear_mode"], proj_segment_len=ft)
    got, route, want, parts = hsa_both(cfg["q"], pool_k, pool_v, cfg3)
    sparse = [h for h, m in enumerate(cfg["head_modes"]) if m == "sparse"]
    assert route.index.shape[-1] == 171
    check_topk_routing(route, parts, cfg["topk"], sparse, "cfg3")
    assert_close(got, want, what="cfg3 HSA over the page pool")
