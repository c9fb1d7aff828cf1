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


def ulps_apart(a: float, b: float) -> int:
    """Distance of two positive fp32 values in units in the last place."""
    ia = torch.tensor([a], dtype=torch.float32).view(torch.int32).item()
    ib = torch.tensor([b], dtype=torch.float32).view(torch.int32).item()
    return abs(ia - ib)


def check_near_ties(got_idx, want_idx, lengths, amap, heads, what, max_ulps=2, max_tie_rows=0.05):
    """Each row's first ``lengths`` listed blocks: the GPU's routing kernels score the pooled blocks
    themselves, in their own fp32 summation order, so their map can differ from the oracle's in the
    last bit (at the reference mode's shape, 37% of entries differ, by at most 7e-10), and two
    blocks the oracle scores within an ulp or two of each other (or exactly equal) may then trade
    places. Every listed position must hold the oracle's block or one whose oracle probability is
    within ``max_ulps`` fp32 ulps of it, and at most ``max_tie_rows`` of the rows may show such a
    swap. Returns (rows with a swap, rows)."""
    rows = swapped = 0
    for h in heads:
        p = amap[0, h]
        for i in range(got_idx.shape[2]):
            n = int(lengths[0, h, i])
            g, r = got_idx[0, h, i, :n], want_idx[0, h, i, :n]
            rows += 1
            if torch.equal(g, r):
                continue
            swapped += 1
            for m in torch.nonzero(g != r).flatten().tolist():
                pg, pr = p[i, g[m]].item(), p[i, r[m]].item()
                assert ulps_apart(pg, pr) <= max_ulps, (
                    f"{what}: head {h} row {i} slot {m}: block {int(g[m])} (p={pg:.9g}) vs oracle "
                    f"{int(r[m])} (p={pr:.9g})")
    assert swapped <= max_tie_rows * rows, f"{what}: {swapped} of {rows} rows differ by near-ties"
    print(f"{what}: {swapped} of {rows} rows hold near-tie swaps (<= {max_ulps} ulp)")
    return swapped, rows


def check_topk_routing(route, parts, ks, heads, what):
    """The selection from identical scores (the oracle's own map through the GPU top-k) must equal
    the oracle's exactly; the end-to-end routing (the fused kernel scoring the pooled blocks itself)
    may differ from it only by near-ties (:func:`check_near_ties`)."""
    amap = parts["attn_map"]
    want = parts["routing"]
    got_idx, got_num = route.index.cpu(), route.num.cpu()
    for h in heads:
        assert torch.equal(got_num[:, h], want.num[:, h]), f"{what}: num of head {h}"
    lengths = torch.zeros_like(want.num)
    for h in heads:
        lengths[:, h] = ks[h]
    swapped, _ = check_near_ties(got_idx, want.index, lengths, amap, heads, what)
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


def test_reference_default_mode_at_the_wan_shape():
    """The reference's own configuration (block 64, Gini routing, low-rank branch, both branches on
    every head; causal_model.py:100-107) on the cfg 2 chunk through HSAAttention. Routing
    (thresholds, counts and each row's selected blocks) equals the oracle's bit for bit on all 12
    heads x 74 query blocks from the oracle's own map, and end to end up to near-ties (blocks the
    oracle scores within 2 ulp of each other); outputs of sampled query blocks (first, middle, partial last) of three
    heads are within the bf16 tolerance of the oracle's per-row attention + low-rank branch + gate."""
    import torch.nn.functional as F
    from worldattention_amd import _lib
    from worldattention_amd.hsa import routing as WR
    cfg = workloads.cfg2_reference_mode(device=DEV, seed=0)
    q, k, v, mod = cfg["q"], cfg["k"], cfg["v"], cfg["module"]
    b, lq, h, d = q.shape
    lkv, bs = k.shape[1], mod.block_size
    save = {}
    with torch.no_grad():
        got = WA.hsa_forward(q, k, v, k_coarse=None, v_coarse=None, k_proj_mat=mod.k_proj_mat,
                             v_proj_mat=mod.v_proj_mat, gate_lin=mod.gate_lin, block_size=bs, tau_min=mod.tau_min,
                             tau_max=mod.tau_max, proj_segment_len=mod.proj_segment_len, routing="gini", topk=None,
                             head_modes=None, linear_mode="lowrank", save=save)
        assert torch.equal(got, mod(q, k, v))              # the module call is the same path
    torch.cuda.synchronize()
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    qpl, kpl, nq, nkv = O.block_counts(lq, lkv, bs)
    q_p = O.pad_to_len(qc, qpl).transpose(1, 2).contiguous()
    k_p = O.pad_to_len(kc, kpl).transpose(1, 2).contiguous()
    v_p = O.pad_to_len(vc, kpl).transpose(1, 2).contiguous()
    amap = O.block_attention_map(O.block_mean_pool(q_p, lq, nq, bs), O.block_mean_pool(k_p, lkv, nkv, bs))
    want_route = O.build_block_routing(amap, mod.tau_min, mod.tau_max)
    # from identical scores (the oracle's map), the GPU's Gini routing is the oracle's bit for bit
    same, _ = WR._route(amap.to(DEV), None, None, mode=_lib.WA_ROUTE_GINI, tau_min=mod.tau_min, tau_max=mod.tau_max)
    assert torch.equal(same.thresholds.cpu(), want_route.thresholds)
    assert torch.equal(same.num.cpu(), want_route.num)
    assert torch.equal(same.index.cpu(), want_route.index)
    # end to end (the routing kernel scores the pooled blocks itself): the same thresholds and
    # counts, and the same lists up to near-ties
    route = save["route"]
    assert torch.equal(route.thresholds.cpu(), want_route.thresholds)
    assert torch.equal(route.num.cpu(), want_route.num)
    check_near_ties(route.index.cpu(), want_route.index, want_route.num, amap, range(h), "reference mode")
    sizes = O.variable_block_sizes(lkv, kpl, bs)
    kcomp, vcomp = O.compress_kv(kc.transpose(1, 2), vc.transpose(1, 2), segment_len=mod.proj_segment_len,
                                 k_proj_mat=mod.k_proj_mat.cpu(), v_proj_mat=mod.v_proj_mat.cpu(), block_size=bs)
    w, bias = mod.gate_lin.weight.cpu(), mod.gate_lin.bias.cpu()
    for hh in (0, 5, 11):
        for i in (0, nq // 2, nq - 1):
            rows = slice(i * bs, min((i + 1) * bs, lq))
            sparse = O.block_sparse_attention(q_p[:, hh:hh + 1, i * bs:(i + 1) * bs], k_p[:, hh:hh + 1],
                                              v_p[:, hh:hh + 1], want_route.index[:, hh:hh + 1, i:i + 1],
                                              want_route.num[:, hh:hh + 1, i:i + 1], sizes, bs)
            sparse = sparse[0, 0, :rows.stop - rows.start]
            lin = O.linear_branch_lowrank(qc[:, rows, hh].unsqueeze(1), kcomp[:, hh:hh + 1], vcomp[:, hh:hh + 1])[0, 0]
            gate = torch.sigmoid(F.linear(qc[0, rows, hh].to(w.dtype), w, bias)).to(lin.dtype)
            want = torch.addcmul(sparse.to(lin.dtype), lin, gate).to(q.dtype)
            assert_close(got[0, rows, hh], want, what=f"head {hh} query block {i}")
