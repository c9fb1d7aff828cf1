"""Pins the HSA oracle (CPU): golden vectors written from the reference module, the reference's own
known answers re-expressed (tests/test_hsa_routing.py, tests/test_hsa_attention.py), and closed
forms for the north-star extensions. Runs on CPU."""
import math
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import hsa as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ----------------------------------------------------------------------------------------------
# golden vectors from the reference implementation itself
# ----------------------------------------------------------------------------------------------
def test_routing_matches_reference_golden_vectors_bit_exactly():
    cases = torch.load(os.path.join(GOLDEN, "routing_gini.pt"), weights_only=True)
    assert len(cases) >= 6
    for c in cases:
        r = O.build_block_routing(c["block_attn"], c["tau_min"], c["tau_max"], return_mask=True)
        assert torch.equal(r.thresholds, c["thresholds"])
        assert torch.equal(r.num, c["num"])
        assert torch.equal(r.index, c["index"])
        assert torch.equal(r.mask, c["mask"])


def _f32_ulp(x: float) -> float:
    return 2.0 ** (math.frexp(abs(x))[1] - 24)


def test_routing_matches_reference_boundary_goldens():
    """Rows whose exclusive prefix lies -3..+3 fp32 ulp from the head threshold (crafted with the
    reference itself): num there depends on the threshold's last bits, and the oracle reproduces
    the reference's count on every row."""
    cases = torch.load(os.path.join(GOLDEN, "routing_boundary.pt"), weights_only=True)
    assert len(cases) == 2
    for c in cases:
        r = O.build_block_routing(c["block_attn"], c["tau_min"], c["tau_max"], return_mask=True)
        assert torch.equal(r.thresholds, c["thresholds"])
        assert torch.equal(r.num, c["num"]) and torch.equal(r.index, c["index"]) and torch.equal(r.mask, c["mask"])
        # the fixture does what it claims: the listed slots sit within 3 ulp of the threshold
        h = int(c["boundary_head"])
        tau = float(c["thresholds"][h])
        sp, _ = torch.sort(c["block_attn"].float(), dim=-1, descending=True)
        excl = torch.cumsum(sp, dim=-1) - sp
        for row, slot, ulps in zip(c["boundary_rows"].tolist(), c["boundary_slots"].tolist(),
                                   c["boundary_ulps"].tolist()):
            off = (float(excl[0, h, row, slot]) - tau) / _f32_ulp(tau)
            assert abs(off) <= 3 and round(off) == ulps
            # num is the first slot whose exclusive prefix reaches the threshold
            assert (int(c["num"][0, h, row]) > slot) == (off < 0)


def test_hsa_attention_matches_reference_golden_vectors():
    """Same routing and rounding points as the reference: at least 99.9% of output elements are
    bit-identical; the rest differ by one rounding step of the output dtype (the sparse matmuls
    sum in a different order than the reference's batched gather)."""
    cases = torch.load(os.path.join(GOLDEN, "hsa_attention.pt"), weights_only=True)
    assert {c["q"].dtype for c in cases} == {torch.float32, torch.bfloat16}
    for c in cases:
        out, parts = O.hsa_attention(c["q"], c["k"], c["v"], k_proj_mat=c["k_proj_mat"],
                                     v_proj_mat=c["v_proj_mat"], gate_weight=c["gate_weight"],
                                     gate_bias=c["gate_bias"], block_size=c["block_size"], tau_min=c["tau_min"],
                                     tau_max=c["tau_max"], proj_segment_len=c["proj_segment_len"],
                                     return_parts=True)
        want = c["out"]
        assert out.dtype == want.dtype
        same = (out == want).float().mean().item()
        assert same >= 0.999, same
        if out.dtype == torch.bfloat16:
            assert torch.allclose(out.float(), want.float(), rtol=2.0 ** -7, atol=2e-4)
        else:
            assert torch.allclose(out, want, rtol=1e-6, atol=1e-6)


# ----------------------------------------------------------------------------------------------
# routing: independent loop transcription and known answers (reference test_hsa_routing.py)
# ----------------------------------------------------------------------------------------------
def _loop_routing(block_attn, tau_min, tau_max):
    """Plain-Python transcription of the Gini / threshold / minimal-k definition."""
    bsz, heads, nq, nkv = block_attn.shape
    ginis = torch.zeros(bsz, heads, nq, dtype=torch.float64)
    orders = {}
    for b in range(bsz):
        for h in range(heads):
            for i in range(nq):
                row = block_attn[b, h, i].tolist()
                order = sorted(range(nkv), key=lambda j: (-row[j], j))
                orders[b, h, i] = order
                ginis[b, h, i] = sum((nkv - 2 * (m + 1) + 1) * row[order[m]] for m in range(nkv)) / nkv
    thr = tau_min + ginis.mean(dim=(0, 2)) * (tau_max - tau_min)
    counts = torch.zeros(bsz, heads, nq, dtype=torch.int32)
    for (b, h, i), order in orders.items():
        acc, k = 0.0, 0
        while k < nkv:
            acc += block_attn[b, h, i, order[k]].item()
            k += 1
            if acc >= thr[h].item():
                break
        counts[b, h, i] = k
    return thr, counts, orders


def test_gini_threshold_and_selection_match_the_definition():
    torch.manual_seed(0)
    attn = torch.softmax(torch.randn(2, 4, 5, 16) * 2.0, dim=-1)
    r = O.build_block_routing(attn, 0.35, 1.0, return_mask=True)
    thr, counts, orders = _loop_routing(attn, 0.35, 1.0)
    assert torch.allclose(r.thresholds.double(), thr, atol=1e-6)
    assert torch.equal(r.num, counts)
    for (b, h, i), order in orders.items():
        assert r.index[b, h, i].tolist() == order
        sel = set(order[: counts[b, h, i]])
        assert set(torch.nonzero(r.mask[b, h, i]).flatten().tolist()) == sel


def test_gini_spans_uniform_to_one_hot():
    n = 16
    uniform = torch.full((1, 1, 1, n), 1.0 / n)
    one_hot = torch.zeros(1, 1, 1, n)
    one_hot[..., 3] = 1.0
    assert abs(O.build_block_routing(uniform, 0.0, 1.0).thresholds.item()) < 1e-6
    assert abs(O.build_block_routing(one_hot, 0.0, 1.0).thresholds.item() - (n - 1) / n) < 1e-6


def test_thresholds_are_per_head():
    n = 16
    attn = torch.stack([torch.full((1, 1, n), 1.0 / n), F.one_hot(torch.tensor([[0]]), n).float()], dim=1)
    thr = O.build_block_routing(attn, 0.35, 1.0).thresholds
    assert thr.shape == (2,) and thr[1] > thr[0] + 0.5


def test_block_mean_pool_partial_block_known_answer():
    x = torch.zeros(1, 1, 12, 2)
    x[0, 0, :10] = 1.0
    pooled = O.block_mean_pool(x, 10, 3, 4)
    assert torch.allclose(pooled[0, 0, 2], torch.ones(2))


def test_block_mean_pool_matches_brute_force_and_reference_dtypes():
    torch.manual_seed(3)
    for dtype in (torch.float32, torch.bfloat16):
        for logical in (256, 230):
            x = torch.randn(1, 2, 256, 8).to(dtype)
            x[:, :, logical:] = 0
            got = O.block_mean_pool(x, logical, 4, 64)
            for blk in range(4):
                real = min(64, logical - blk * 64)
                want = x[0, 1, blk * 64: blk * 64 + real].double().mean(dim=0)
                assert torch.allclose(got[0, 1, blk].double(), want, atol=2e-2 if dtype == torch.bfloat16 else 1e-6)
            assert got.dtype == (dtype if logical % 64 == 0 else torch.float32)


def test_routing_invariants_end_to_end():
    torch.manual_seed(0)
    q, k = torch.randn(1, 3, 256, 16), torch.randn(1, 3, 256, 16)
    attn = O.block_attention_map(O.block_mean_pool(q, 256, 4, 64), O.block_mean_pool(k, 256, 4, 64))
    assert torch.allclose(attn.sum(-1), torch.ones(1, 3, 4), atol=1e-5)
    want = torch.softmax(torch.einsum("bhid,bhjd->bhij", O.block_mean_pool(q, 256, 4, 64).double(),
                                      O.block_mean_pool(k, 256, 4, 64).double()) / 4.0, -1)
    assert torch.allclose(attn.double(), want, atol=1e-6)
    r = O.build_block_routing(attn, 0.35, 1.0, return_mask=True)
    assert r.num.min() >= 1 and r.num.max() <= 4
    assert torch.equal(r.mask.sum(-1).to(torch.int32), r.num)


def test_topk_routing_matches_torch_topk_and_lowest_index_ties():
    torch.manual_seed(1)
    attn = torch.softmax(torch.randn(1, 3, 6, 40) * 3, -1)
    r = O.build_topk_routing(attn, [4, 8, 0], return_mask=True)
    assert r.num[0, :, 0].tolist() == [4, 8, 0]
    for h, kk in enumerate([4, 8]):
        for i in range(6):
            want = torch.topk(attn[0, h, i], kk).indices.tolist()
            assert r.index[0, h, i, :kk].tolist() == want
    tied = torch.tensor([0.1, 0.3, 0.1, 0.3, 0.2]).view(1, 1, 1, 5)
    r = O.build_topk_routing(tied, 3)
    assert r.index[0, 0, 0].tolist() == [1, 3, 4, 0, 2]


def test_map_to_index_is_ascending_and_padded():
    m = torch.tensor([[[[0, 1, 0, 1, 1], [0, 0, 0, 0, 0]]]], dtype=torch.bool)
    idx, num = O.map_to_index(m)
    assert num.tolist() == [[[3, 0]]]
    assert idx[0, 0, 0].tolist() == [1, 3, 4, -1, -1] and idx[0, 0, 1].tolist() == [-1] * 5


# ----------------------------------------------------------------------------------------------
# block-sparse attention (reference test_hsa_routing.py:97-193)
# ----------------------------------------------------------------------------------------------
def _sdpa(q, k, v):
    return F.scaled_dot_product_attention(q.double(), k.double(), v.double()).float()


def test_sparse_full_selection_is_dense_attention():
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 128, 16) for _ in range(3))
    index = torch.arange(2, dtype=torch.int32).view(1, 1, 1, 2).expand(1, 2, 2, 2).contiguous()
    num = torch.full((1, 2, 2), 2, dtype=torch.int32)
    got = O.block_sparse_attention(q, k, v, index, num, O.variable_block_sizes(128, 128, 64), 64)
    assert torch.allclose(got, _sdpa(q, k, v), atol=1e-5)


def test_sparse_single_block_and_partial_tail_and_empty_rows():
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 1, 128, 16) for _ in range(3))
    index = torch.zeros(1, 1, 2, 2, dtype=torch.int32)
    got = O.block_sparse_attention(q, k, v, index, torch.ones(1, 1, 2, dtype=torch.int32),
                                   O.variable_block_sizes(128, 128, 64), 64)
    assert torch.allclose(got, _sdpa(q, k[:, :, :64], v[:, :, :64]), atol=1e-5)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 96:] = 0
    v2[:, :, 96:] = 0
    index = torch.tensor([0, 1], dtype=torch.int32).view(1, 1, 1, 2)
    got = O.block_sparse_attention(q[:, :, :64], k2, v2, index, torch.full((1, 1, 1), 2, dtype=torch.int32),
                                   O.variable_block_sizes(96, 128, 64), 64)
    assert torch.allclose(got, _sdpa(q[:, :, :64], k2[:, :, :96], v2[:, :, :96]), atol=1e-5)
    out = O.block_sparse_attention(q, k, v, torch.zeros(1, 1, 2, 2, dtype=torch.int32),
                                   torch.tensor([[[0, 1]]], dtype=torch.int32), O.variable_block_sizes(128, 128, 64), 64)
    assert torch.count_nonzero(out[:, :, :64]) == 0 and torch.count_nonzero(out[:, :, 64:]) > 0


def test_sparse_ignores_slots_past_num_and_counts_duplicates():
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 256, 16) for _ in range(3))
    index = torch.arange(4, dtype=torch.int32).view(1, 1, 1, 4).expand(1, 2, 4, 4).contiguous()
    num = torch.randint(1, 5, (1, 2, 4), dtype=torch.int32)
    sizes = O.variable_block_sizes(256, 256, 64)
    base = O.block_sparse_attention(q, k, v, index, num, sizes, 64)
    scrambled = index.clone()
    for h in range(2):
        for i in range(4):
            kept = int(num[0, h, i])
            scrambled[0, h, i, kept:] = torch.randint(0, 4, (4 - kept,), dtype=torch.int32)
    assert torch.allclose(base, O.block_sparse_attention(q, k, v, scrambled, num, sizes, 64), atol=1e-6)
    # a block listed twice counts twice: equals dense attention over [K0, K0]
    dup = torch.zeros(1, 1, 1, 2, dtype=torch.int32)
    got = O.block_sparse_attention(q[:1, :1, :64], k[:1, :1, :64], v[:1, :1, :64], dup,
                                   torch.full((1, 1, 1), 2, dtype=torch.int32), O.variable_block_sizes(64, 64, 64), 64)
    kk = torch.cat([k[:1, :1, :64]] * 2, 2)
    vv = torch.cat([v[:1, :1, :64]] * 2, 2)
    assert torch.allclose(got, _sdpa(q[:1, :1, :64], kk, vv), atol=1e-5)


def test_sparse_lse_is_log_sum_exp_of_scaled_logits():
    torch.manual_seed(5)
    q, k, v = (torch.randn(1, 1, 64, 16) for _ in range(3))
    _, lse = O.block_sparse_attention(q, k, v, torch.zeros(1, 1, 1, 1, dtype=torch.int32),
                                      torch.ones(1, 1, 1, dtype=torch.int32), O.variable_block_sizes(64, 64, 64), 64,
                                      return_lse=True)
    want = torch.logsumexp((q[0, 0] @ k[0, 0].T).double() / 4.0, -1)
    assert torch.allclose(lse[0, 0].double(), want, atol=1e-5)


# ----------------------------------------------------------------------------------------------
# linear branches and composition (reference test_hsa_attention.py)
# ----------------------------------------------------------------------------------------------
def test_compress_kv_is_the_projection_closed_form():
    torch.manual_seed(0)
    k, v = torch.randn(1, 3, 200, 16), torch.randn(1, 3, 200, 16)
    proj = O.init_projection(1, 50, 64)
    kc, vc = O.compress_kv(k, v, segment_len=50, k_proj_mat=proj, v_proj_mat=proj, block_size=64)
    assert kc.shape == (1, 3, 4, 16)
    assert torch.allclose(kc[0, 0, 0], proj[0].float() @ k[0, 0, :50], atol=1e-5)
    assert torch.allclose(kc[0, 2, 3], k[0, 2, 150:200].mean(0), atol=1e-3)


def test_lowrank_linear_branch_is_sdpa_over_the_compressed_keys():
    torch.manual_seed(0)
    q, kc, vc = torch.randn(1, 2, 50, 16), torch.randn(1, 2, 7, 16), torch.randn(1, 2, 7, 16)
    assert torch.allclose(O.linear_branch_lowrank(q, kc, vc), _sdpa(q, kc, vc), atol=1e-5)


def test_elu1_linear_branch_matches_quadratic_form_and_loop():
    torch.manual_seed(0)
    q, k, v = torch.randn(1, 2, 9, 8), torch.randn(1, 2, 13, 8), torch.randn(1, 2, 13, 8)
    got = O.linear_branch_elu1(q, k, v, compute_dtype=torch.float64)
    fq, fk = F.elu(q.double()) + 1, F.elu(k.double()) + 1
    att = fq @ fk.transpose(-1, -2)
    want = (att @ v.double()) / att.sum(-1, keepdim=True)
    assert torch.allclose(got.double(), want, atol=1e-6)
    # per-token loop on one head
    for t in range(9):
        w = [(fq[0, 1, t] @ fk[0, 1, s]).item() for s in range(13)]
        o = sum(wi * v[0, 1, s].double() for s, wi in enumerate(w)) / sum(w)
        assert torch.allclose(got[0, 1, t].double(), o, atol=1e-6)
    # phi is elu+1: positive, identity+1 above zero, exp below
    x = torch.tensor([-2.0, 0.0, 3.0])
    assert torch.allclose(O.elu1(x), torch.tensor([math.exp(-2.0), 1.0, 4.0]))


def _inputs(lq=100, lkv=200, h=3, d=16, seed=1, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(1, n, h, d, generator=g).to(dtype) for n in (lq, lkv, lkv))


def test_output_is_the_gated_sum_of_the_branches_and_split_modes_restrict_it():
    q, k, v = _inputs()
    proj = O.init_projection(1, 50, 64)
    w, b = torch.randn(16, 16) * 0.1, torch.full((16,), 0.3)
    out, parts = O.hsa_attention(q, k, v, k_proj_mat=proj, v_proj_mat=proj, gate_weight=w, gate_bias=b,
                                 block_size=64, proj_segment_len=50, return_parts=True)
    gate = torch.sigmoid(q @ w.T + b)
    assert torch.allclose(out, parts["sparse"] + parts["linear"] * gate, atol=1e-6)
    modes = ["sparse", "linear", "both"]
    out2, parts2 = O.hsa_attention(q, k, v, k_proj_mat=proj, v_proj_mat=proj, gate_weight=w, gate_bias=b,
                                   block_size=64, proj_segment_len=50, head_modes=modes, return_parts=True)
    assert torch.allclose(out2[:, :, 0], parts["sparse"][:, :, 0], atol=1e-6)
    assert torch.allclose(out2[:, :, 1], (parts["linear"] * gate)[:, :, 1], atol=1e-6)
    assert torch.allclose(out2[:, :, 2], out[:, :, 2], atol=1e-6)
    assert int(parts2["routing"].num[0, 1].max()) == 0


def test_coarse_cache_equals_inline_compression():
    q, k, v = _inputs()
    proj = O.init_projection(1, 50, 64)
    inline = O.hsa_attention(q, k, v, k_proj_mat=proj, v_proj_mat=proj, block_size=64, proj_segment_len=50)
    kc, vc = O.compress_kv(k.transpose(1, 2), v.transpose(1, 2), segment_len=50, k_proj_mat=proj, v_proj_mat=proj,
                           block_size=64)
    cached = O.hsa_attention(q, k, v, k_coarse=kc.transpose(1, 2), v_coarse=vc.transpose(1, 2), k_proj_mat=proj,
                             v_proj_mat=proj, block_size=64, proj_segment_len=50)
    assert torch.allclose(inline, cached, atol=1e-5)


def test_init_projection_rows_average_one_block():
    proj = O.init_projection(25, 1560, 64)
    assert int((proj[0] != 0).sum()) == 64 and abs(proj[0, 0].item() - 1 / 64) < 1e-3
    assert int((proj[24] != 0).sum()) == 1560 - 24 * 64
    assert O.coarse_cache_size(0, 50, 1) == 0 and O.coarse_cache_size(200, 50, 1) == 4
    assert O.token_range_to_coarse(50, 150, 50, 1) == (1, 3)
    with pytest.raises(ValueError):
        O.token_range_to_coarse(0, 51, 50, 1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_vectorized_sparse_equals_the_per_row_loop(dtype):
    torch.manual_seed(21)
    b, h, nq, nkv, bs, d = 2, 3, 4, 6, 16, 8
    q, k, v = (torch.randn(b, h, n * bs, d).to(dtype) for n in (nq, nkv, nkv))
    index = torch.stack([torch.randperm(nkv) for _ in range(b * h * nq)]).view(b, h, nq, nkv).int()
    num = torch.randint(0, nkv + 1, (b, h, nq), dtype=torch.int32)
    num[0, 1, 2] = 0
    index[1, 0, 3, :3] = torch.tensor([2, 2, 9])     # duplicate and out-of-range (clamped) ids
    num[1, 0, 3] = 3
    sizes = torch.tensor([16, 16, 16, 16, 16, 5], dtype=torch.int32)
    loop = O.block_sparse_attention(q, k, v, index, num, sizes, bs)
    vec = O.block_sparse_attention_gather(q, k, v, index, num, sizes, bs)
    assert vec.dtype == loop.dtype
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    assert torch.allclose(vec.float(), loop.float(), atol=tol, rtol=tol)
    qr, kr, vr = (t.double().requires_grad_() for t in (q, k, v))
    ql, kl, vl = (t.double().requires_grad_() for t in (q, k, v))
    g = torch.randn(q.shape, dtype=torch.float64)
    O.block_sparse_attention_gather(qr, kr, vr, index, num, sizes, bs).backward(g)
    O.block_sparse_attention(ql, kl, vl, index, num, sizes, bs).backward(g)
    for a, c in ((qr, ql), (kr, kl), (vr, vl)):
        assert torch.allclose(a.grad, c.grad, atol=1e-10)
