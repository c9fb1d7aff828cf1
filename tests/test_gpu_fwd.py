"""GPU parity of the forward path against the CPU oracle (and the reference's own golden outputs).

Tolerances: integer/index outputs bit-exact; attention outputs max-abs <= 2e-2 and mean-abs <= 2e-3
against the fp32 oracle (the north-star bf16 tolerance)."""
import os

import pytest
import torch

from oracle import hsa as O
from worldattention_amd import hsa as W
from worldattention_amd import workloads
from worldattention_amd.hsa import attention as WA
from worldattention_amd.hsa import routing as WR

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def assert_close(got, want, max_abs=2e-2, mean_abs=2e-3, what=""):
    diff = (got.detach().float().cpu() - want.detach().float().cpu()).abs()
    assert torch.isfinite(got.float()).all(), f"{what}: non-finite output"
    assert diff.max().item() <= max_abs, f"{what}: max-abs {diff.max().item():.3e} > {max_abs}"
    assert diff.mean().item() <= mean_abs, f"{what}: mean-abs {diff.mean().item():.3e} > {mean_abs}"


# ----------------------------------------------------------------------------------------------
# routing
# ----------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("logical", [512, 470])
def test_block_mean_pool_matches_oracle(dtype, logical):
    torch.manual_seed(0)
    x = (torch.randn(2, 3, 512, 64) * 2).to(dtype)
    x[:, :, logical:] = 0
    want = O.block_mean_pool(x, logical, 4, 128)
    got = W.block_mean_pool(x.to(DEV), logical, 4, 128)
    assert got.dtype == want.dtype
    if dtype == torch.bfloat16:
        # the reference rounds the bf16 block mean (or block sum); the kernel reproduces it
        assert (got.cpu() == want).float().mean().item() >= 0.999
        assert torch.allclose(got.cpu().float(), want.float(), rtol=2 ** -7, atol=0)
    else:
        assert torch.allclose(got.cpu(), want, atol=1e-5, rtol=1e-5)


def test_pooling_jobs_in_one_launch_equal_separate_launches():
    """wa_block_mean_pool_n (query + key tensors of one call, plus an fp32 job that needs its own
    launch) writes exactly what one wa_block_mean_pool call per tensor writes."""
    from worldattention_amd.hsa.routing import pool_blhd, pool_blhd_many
    torch.manual_seed(3)
    heads = torch.tensor([4, 0, 2], dtype=torch.int32, device=DEV)
    q = torch.randn(2, 300, 5, 128, device=DEV).bfloat16()
    k = torch.randn(2, 1000, 5, 128, device=DEV).bfloat16()
    x = torch.randn(2, 256, 5, 64, device=DEV)
    jobs = [(q, 300, 3), (k, 1000, 8), (x, 256, 2)]
    got = pool_blhd_many(jobs, 128, heads=heads)
    for (t, n, nb), g in zip(jobs, got):
        want = pool_blhd(t, n, nb, 128, heads=heads)
        assert torch.equal(g[:, heads.long()], want[:, heads.long()])


@pytest.mark.parametrize("fixture", ["routing_gini.pt", "routing_boundary.pt"])
def test_gini_routing_is_bit_exact_on_reference_golden_maps(fixture):
    """Thresholds, counts, permutations and masks equal the reference's bit for bit, including the
    rows whose exclusive prefix sits within 3 fp32 ulp of the threshold (the row Gini sums and the
    head mean follow torch's CPU fp32 summation order)."""
    for c in torch.load(os.path.join(GOLDEN, fixture), weights_only=True):
        r = W.build_block_routing(c["block_attn"].to(DEV), c["tau_min"], c["tau_max"], return_mask=True)
        assert torch.equal(r.thresholds.cpu(), c["thresholds"])
        assert torch.equal(r.index.cpu(), c["index"])
        assert torch.equal(r.num.cpu(), c["num"])
        assert torch.equal(r.mask.cpu(), c["mask"])


@pytest.mark.parametrize("shape", [(1, 12, 37, 256), (3, 2, 9, 40), (2, 1, 11, 16), (5, 9, 1, 64), (6, 3, 1, 17),
                                   (17, 33, 1, 16), (5, 6, 1, 16), (1, 3, 5, 1000)])
def test_gini_thresholds_equal_torch_fp32_reductions(shape):
    """Thresholds equal the reference formula evaluated by torch on the CPU (fp32 sum over blocks,
    fp32 mean over batch and query blocks), over shapes that take each reduction path: contiguous
    runs of >= 8 and < 8 elements, a single head, a single query block with heads grouped by 4 /
    32 or not."""
    torch.manual_seed(sum(shape))
    attn = torch.softmax(torch.randn(shape) * 3, -1)
    b, h, nq, n = shape
    sp, _ = torch.sort(attn, dim=-1, descending=True)
    ranks = torch.arange(1, n + 1, dtype=torch.float32)
    gini = torch.sum((n + 1 - 2 * ranks) * sp, dim=-1) / n
    want = 0.35 + gini.mean(dim=(0, 2)) * (1.0 - 0.35)
    got = W.build_block_routing(attn.to(DEV), 0.35, 1.0).thresholds.cpu()
    assert torch.equal(got, want)


@pytest.mark.parametrize("nkv", [16, 37, 256, 512, 1100])
def test_routing_is_bit_exact_given_identical_maps_with_ties(nkv):
    torch.manual_seed(nkv)
    attn = torch.softmax(torch.randn(2, 3, 9, nkv) * 3, -1)
    # inject exact ties: quantize one head's weights
    attn[:, 1] = (attn[:, 1] * 64).round() / 64
    want_g = O.build_block_routing(attn, 0.35, 1.0, return_mask=True)
    got_g = W.build_block_routing(attn.to(DEV), 0.35, 1.0, return_mask=True)
    assert torch.equal(got_g.index.cpu(), want_g.index)
    assert torch.equal(got_g.num.cpu(), want_g.num)
    assert torch.equal(got_g.mask.cpu(), want_g.mask)
    ks = [3, min(17, nkv), 0]
    want_t = O.build_topk_routing(attn, ks, return_mask=True)
    got_t = W.build_topk_routing(attn.to(DEV), ks, return_mask=True)
    assert torch.equal(got_t.index.cpu(), want_t.index)
    assert torch.equal(got_t.num.cpu(), want_t.num)
    assert torch.equal(got_t.mask.cpu(), want_t.mask)


def test_block_attention_map_matches_oracle():
    torch.manual_seed(2)
    qp, kp = torch.randn(1, 4, 37, 128), torch.randn(1, 4, 256, 128)
    got = W.block_attention_map(qp.to(DEV), kp.to(DEV)).cpu()
    want = O.block_attention_map(qp, kp)
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-7)


def test_map_to_index_matches_oracle():
    torch.manual_seed(4)
    m = torch.rand(2, 3, 5, 200) < 0.3
    idx, num = W.map_to_index(m.to(DEV))
    widx, wnum = O.map_to_index(m)
    assert torch.equal(idx.cpu(), widx) and torch.equal(num.cpu(), wnum)


# ----------------------------------------------------------------------------------------------
# block-sparse forward
# ----------------------------------------------------------------------------------------------
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("bs", [64, 128])
def test_block_sparse_attention_matches_oracle(d, bs):
    torch.manual_seed(d + bs)
    nq, nkv = 5, 9
    lkv = nkv * bs - bs // 3          # partial trailing key block
    q = torch.randn(2, 3, nq * bs, d).bfloat16()
    k = torch.randn(2, 3, nkv * bs, d).bfloat16()
    v = torch.randn(2, 3, nkv * bs, d).bfloat16()
    k[:, :, lkv:] = 0
    v[:, :, lkv:] = 0
    index = torch.stack([torch.randperm(nkv) for _ in range(2 * 3 * nq)]).view(2, 3, nq, nkv).int()
    num = torch.randint(0, nkv + 1, (2, 3, nq), dtype=torch.int32)
    num[0, 0, 0] = 0                   # empty row -> 0
    index[1, 2, 1, :3] = torch.tensor([4, 4, 4])   # duplicates count
    num[1, 2, 1] = 3
    index[1, 1, 2, 0] = 99             # out of range -> clamped
    sizes = O.variable_block_sizes(lkv, nkv * bs, bs)
    want, lse_want = O.block_sparse_attention(q, k, v, index, num, sizes, bs, return_lse=True)
    got = W.block_sparse_attention_reference(q.to(DEV), k.to(DEV), v.to(DEV), index.to(DEV), num.to(DEV),
                                             sizes.to(DEV), bs)
    assert got.dtype == torch.bfloat16
    assert_close(got, want, what=f"bsa d={d} bs={bs}")
    assert torch.count_nonzero(got[0, 0, :bs]) == 0
    from worldattention_amd.hsa.block_sparse import bsa_forward
    from worldattention_amd import _lib
    _, lse = bsa_forward(q.to(DEV), k.to(DEV), v.to(DEV), index=index.to(DEV), num=num.to(DEV), block_size=bs,
                         block_sizes=sizes.to(DEV), want_lse=True)
    finite = torch.isfinite(lse_want)
    assert torch.equal(torch.isfinite(lse.cpu()), finite)
    assert torch.allclose(lse.cpu()[finite], lse_want[finite].float(), atol=2e-2)


def test_full_selection_is_dense_attention():
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 256, 64).bfloat16() for _ in range(3))
    index = torch.arange(4, dtype=torch.int32).view(1, 1, 1, 4).expand(1, 2, 4, 4).contiguous()
    num = torch.full((1, 2, 4), 4, dtype=torch.int32)
    got = W.block_sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), block_sizes=torch.full((4,), 64, device=DEV),
                                   q2k_index=index.to(DEV), q2k_num=num.to(DEV))
    want = torch.nn.functional.scaled_dot_product_attention(q.double(), k.double(), v.double())
    assert_close(got, want, what="dense")


# ----------------------------------------------------------------------------------------------
# linear branches
# ----------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_compress_kv_matches_oracle(dtype):
    torch.manual_seed(1)
    k, v = torch.randn(1, 3, 3200, 128).to(dtype), torch.randn(1, 3, 3200, 128).to(dtype)
    pk = (torch.rand(25, 1560) / 40).bfloat16()
    pv = O.init_projection(25, 1560, 64)
    wk, wv = O.compress_kv(k, v, segment_len=1560, k_proj_mat=pk, v_proj_mat=pv, block_size=64)
    gk, gv = W.compress_kv(k.to(DEV), v.to(DEV), segment_len=1560, k_proj_mat=pk.to(DEV), v_proj_mat=pv.to(DEV),
                           block_size=64)
    assert gk.shape == wk.shape == (1, 3, 25 + 25 + 2, 128)
    assert_close(gk, wk, max_abs=1e-2, mean_abs=1e-3, what="compress k")
    assert_close(gv, wv, max_abs=1e-2, mean_abs=1e-3, what="compress v")


@pytest.mark.parametrize("d", [64, 128])
def test_dense_distillation_teacher_matches_oracle(d):
    """The distillation teacher (the dense flash kernel) against fp32 softmax attention (the
    oracle's dense attention, pinned by SDPA in fp64), and the recorded loss against the MSE to it."""
    from worldattention_amd.hsa import distill
    torch.manual_seed(d)
    q, k, v = torch.randn(2, 700, 3, d), torch.randn(2, 2000, 3, d), torch.randn(2, 2000, 3, d)
    want = O.linear_branch_lowrank(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
    qg, kg, vg = (t.to(DEV).bfloat16() for t in (q, k, v))
    got = distill.dense_attention(qg, kg, vg)
    assert got.dtype == torch.bfloat16
    assert_close(got, want, what="dense teacher")
    got32 = distill.dense_attention(qg.float(), kg.float(), vg.float())
    assert got32.dtype == torch.float32
    assert_close(got32, want, what="dense teacher, fp32 result")
    hsa_out = (want + 0.05 * torch.randn_like(want)).to(DEV).requires_grad_(True)
    distill.enable_distill(True)
    try:
        distill.record_against_dense(hsa_out, qg.float(), kg.float(), vg.float())
        (loss,) = distill.pop_distill_losses()
    finally:
        distill.enable_distill(False)
    want_loss = ((hsa_out.detach().cpu() - want) ** 2).mean()
    assert abs(loss.item() - want_loss.item()) <= 2e-2 * want_loss.item()
    loss.backward()
    assert hsa_out.grad is not None and torch.isfinite(hsa_out.grad).all()


def test_lowrank_linear_branch_matches_oracle():
    torch.manual_seed(3)
    q, kc, vc = torch.randn(1, 2, 300, 64), torch.randn(1, 2, 77, 64), torch.randn(1, 2, 77, 64)
    got = WA._linear_branch(q.to(DEV), kc.to(DEV), vc.to(DEV))
    assert_close(got, O.linear_branch_lowrank(q, kc, vc), what="lowrank")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128])
def test_elu1_linear_branch_matches_oracle(d, dtype):
    torch.manual_seed(d)
    q, k, v = (torch.randn(1, n, 4, d).to(dtype) for n in (700, 5000, 5000))
    heads = torch.tensor([0, 2, 3], dtype=torch.int32, device=DEV)
    s, z = WA.elu1_state(k.to(DEV), v.to(DEV), heads)
    out = torch.zeros(1, 700, 4, d, dtype=torch.float32, device=DEV)
    WA.elu1_readout(q.to(DEV), s, z, heads, out)
    want = O.linear_branch_elu1(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                compute_dtype=torch.float64).transpose(1, 2)
    for h in (0, 2, 3):
        assert_close(out[:, :, h], want[:, :, h], max_abs=1e-2, mean_abs=1e-3, what=f"elu1 head {h}")
    assert torch.count_nonzero(out[:, :, 1]) == 0


def test_empty_head_lists_launch_nothing():
    """An empty head list writes nothing (the library reads a missing list as every head, so the
    wrappers never pass an empty one down)."""
    from worldattention_amd.hsa._bwd import bsa_backward
    from worldattention_amd.hsa.block_sparse import bsa_forward
    torch.manual_seed(5)
    b, h, lq, lkv, d = 1, 3, 300, 700, 128
    q, k, v = (torch.randn(b, n, h, d, device=DEV).bfloat16() for n in (lq, lkv, lkv))
    empty = torch.zeros(0, dtype=torch.int32, device=DEV)
    out, _ = bsa_forward(q, k, v, index=None, num=None, block_size=128, layout="blhd", heads=empty,
                         out=torch.zeros(b, lq, h, d, dtype=torch.bfloat16, device=DEV))
    assert torch.count_nonzero(out) == 0
    s, z = WA.elu1_state(k, v, empty)
    assert s.shape == (b, 0, d, d) and z.shape == (b, 0, d)
    o2 = torch.zeros(b, lq, h, d, device=DEV)
    WA.elu1_readout(q, s, z, empty, o2)
    assert torch.count_nonzero(o2) == 0
    lse = torch.zeros(b, h, lq, device=DEV)
    dq, dk, dv = bsa_backward(q, k, v, o2, lse, o2, index=None, num=None, block_size=128, layout="blhd",
                              heads=empty, dq=torch.zeros(b, lq, h, d, device=DEV),
                              dk=torch.zeros(b, lkv, h, d, device=DEV), dv=torch.zeros(b, lkv, h, d, device=DEV))
    assert not dq.any() and not dk.any() and not dv.any()


# ----------------------------------------------------------------------------------------------
# hsa_attention end to end
# ----------------------------------------------------------------------------------------------
def test_hsa_attention_matches_reference_golden_outputs():
    """The reference module's own outputs (Gini routing, low-rank branch, trained-looking gate)."""
    for c in torch.load(os.path.join(GOLDEN, "hsa_attention.pt"), weights_only=True):
        gate = torch.nn.Linear(c["q"].shape[-1], c["q"].shape[-1]).to(c["q"].dtype)
        with torch.no_grad():
            gate.weight.copy_(c["gate_weight"])
            gate.bias.copy_(c["gate_bias"])
        with torch.no_grad():
            got = W.hsa_attention(c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), k_proj_mat=c["k_proj_mat"].to(DEV),
                                  v_proj_mat=c["v_proj_mat"].to(DEV), gate_lin=gate.to(DEV), block_size=c["block_size"],
                                  tau_min=c["tau_min"], tau_max=c["tau_max"], proj_segment_len=c["proj_segment_len"])
        assert got.dtype == c["out"].dtype and got.shape == c["out"].shape
        assert_close(got, c["out"], what=f"golden {tuple(c['q'].shape)} {c['q'].dtype}")


def _run_both(cfg, oracle_kwargs=None, gate=None):
    q, k, v = cfg["q"], cfg["k"], cfg["v"]
    kw = dict(block_size=cfg["block_size"], routing=cfg["routing"], topk=cfg["topk"], head_modes=cfg["head_modes"],
              linear_mode=cfg["linear_mode"], proj_segment_len=cfg["proj_segment_len"])
    d = q.shape[-1]
    rank = -(-cfg["proj_segment_len"] // cfg["block_size"])
    proj = O.init_projection(rank, cfg["proj_segment_len"], cfg["block_size"])
    w = torch.zeros(d, d) if gate is None else gate[0]
    b = torch.zeros(d) if gate is None else gate[1]
    want, parts = O.hsa_attention(q.cpu(), k.cpu(), v.cpu(), k_proj_mat=proj, v_proj_mat=proj, gate_weight=w,
                                  gate_bias=b, return_parts=True, **kw)
    lin = torch.nn.Linear(d, d).to(DEV)
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(b)
    save = {}
    with torch.no_grad():
        got = WA.hsa_forward(q.to(DEV), k.to(DEV), v.to(DEV), k_coarse=None, v_coarse=None, k_proj_mat=proj.to(DEV),
                             v_proj_mat=proj.to(DEV), gate_lin=lin, tau_min=0.35, tau_max=1.0, save=save, **kw)
    return got, want, parts, save


def test_hsa_cfg1_split_heads_match_oracle():
    cfg = workloads.cfg1()
    got, want, parts, save = _run_both(cfg, gate=(torch.randn(64, 64) * 0.1, torch.full((64,), 0.2)))
    r = save["route"]
    assert torch.equal(r.num.cpu()[:, 0], parts["routing"].num[:, 0])
    assert torch.equal(r.index.cpu()[:, 0, :, :4], parts["routing"].index[:, 0, :, :4])
    assert_close(got, want, what="cfg1")


def test_hsa_cfg2_wan_chunk_matches_oracle():
    cfg = workloads.cfg2()
    got, want, parts, save = _run_both(cfg)
    sparse = [h for h, m in enumerate(cfg["head_modes"]) if m == "sparse"]
    r = save["route"]
    for h in sparse:
        assert torch.equal(r.num.cpu()[:, h], parts["routing"].num[:, h])
        kk = cfg["topk"][h]
        same = (r.index.cpu()[:, h, :, :kk] == parts["routing"].index[:, h, :, :kk]).all(-1).float().mean()
        assert same.item() == 1.0, f"head {h}: {same.item()}"
    assert_close(got, want, what="cfg2")


@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float32])
def test_hsa_gated_linear_heads_match_oracle(gate_dtype):
    """bf16 head-adaptive call whose linear heads take the gated readout with real gate weights,
    from a bf16 gate layer (pre-activation rounded to bf16) and from an fp32 one."""
    torch.manual_seed(11)
    q = torch.randn(1, 700, 4, 128).bfloat16()
    k = torch.randn(1, 3000, 4, 128).bfloat16()
    v = torch.randn(1, 3000, 4, 128).bfloat16()
    w, b = torch.randn(128, 128) * 0.1, torch.randn(128) * 0.2
    kw = dict(block_size=128, routing="topk", topk=[4, 0, 0, 8], head_modes=["sparse", "linear", "linear", "sparse"],
              linear_mode="elu1", proj_segment_len=1000)
    want = O.hsa_attention(q, k, v, gate_weight=w.to(gate_dtype), gate_bias=b.to(gate_dtype), **kw)
    lin = torch.nn.Linear(128, 128).to(device=DEV, dtype=gate_dtype)
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(b)
        got = WA.hsa_forward(q.to(DEV), k.to(DEV), v.to(DEV), k_coarse=None, v_coarse=None, k_proj_mat=None,
                             v_proj_mat=None, gate_lin=lin, tau_min=0.35, tau_max=1.0, **kw)
    for h in (1, 2):
        assert_close(got[:, :, h], want[:, :, h], what=f"gated linear head {h} ({gate_dtype})")
    assert_close(got, want, what=f"gated head-adaptive call ({gate_dtype})")


def test_hsa_reference_mode_bf16_matches_oracle():
    torch.manual_seed(7)
    q = torch.randn(1, 1000, 4, 128).bfloat16()
    k = torch.randn(1, 3000, 4, 128).bfloat16()
    v = torch.randn(1, 3000, 4, 128).bfloat16()
    proj = (torch.rand(8, 1000) / 100).bfloat16()
    gate = torch.nn.Linear(128, 128).bfloat16()
    with torch.no_grad():
        want = O.hsa_attention(q, k, v, k_proj_mat=proj, v_proj_mat=proj, gate_weight=gate.weight, gate_bias=gate.bias,
                               block_size=128, proj_segment_len=1000)
        got = W.hsa_attention(q.to(DEV), k.to(DEV), v.to(DEV), k_proj_mat=proj.to(DEV), v_proj_mat=proj.to(DEV),
                              gate_lin=gate.to(DEV), block_size=128, proj_segment_len=1000)
    assert_close(got, want, what="reference mode bf16")


def test_coarse_cache_equals_inline_compression_on_gpu():
    torch.manual_seed(9)
    hsa = W.HSAAttention(num_heads=2, head_dim=64, block_size=64, proj_segment_len=100).to(DEV)
    from worldattention_amd.hsa_stage import init_hsa_parameters
    init_hsa_parameters(hsa)
    q, k, v = (torch.randn(1, n, 2, 64, device=DEV) for n in (150, 400, 400))
    with torch.no_grad():
        inline = hsa(q, k, v)
        kc, vc = hsa.compress_kv_cache(k, v)
        cached = hsa(q, k, v, k_coarse=kc, v_coarse=vc)
    assert torch.allclose(inline, cached, atol=1e-5)


@pytest.mark.parametrize("use_visits", [False, True])
@pytest.mark.parametrize("split", [1, 3, 8])
def test_bsa_head_subset_split_units_match_oracle(use_visits, split):
    """A launch over a subset of heads (rows numbered by head slot) with lists cut into several
    split units; index / num are laid out by global head, as the routing writes them."""
    from worldattention_amd.hsa.block_sparse import bsa_forward
    torch.manual_seed(split)
    bs, d, b, h, nq, nkv = 128, 128, 2, 4, 3, 11
    lq, lkv = nq * bs - 50, nkv * bs - 70
    q = torch.randn(b, lq, h, d).bfloat16()
    k = torch.randn(b, lkv, h, d).bfloat16()
    v = torch.randn(b, lkv, h, d).bfloat16()
    index = torch.stack([torch.randperm(nkv) for _ in range(b * h * nq)]).view(b, h, nq, nkv).int()
    ks = [0, 5, 0, 11]
    num = torch.tensor(ks, dtype=torch.int32).view(1, h, 1).expand(b, h, nq).contiguous()
    heads = torch.tensor([3, 1], dtype=torch.int32)
    out = torch.zeros(b, lq, h, d, dtype=torch.float32, device=DEV)
    bsa_forward(q.to(DEV), k.to(DEV), v.to(DEV), index=index.to(DEV), num=num.to(DEV), block_size=bs,
                layout="blhd", heads=heads.to(DEV), out=out, lq=lq, lkv=lkv, split=split,
                visits=[ks[3], ks[1]] if use_visits else None)
    qp = O.pad_to_len(q, nq * bs).transpose(1, 2)
    kp, vp = (O.pad_to_len(t, nkv * bs).transpose(1, 2) for t in (k, v))
    sizes = O.variable_block_sizes(lkv, nkv * bs, bs)
    want = O.block_sparse_attention(qp.float(), kp.float(), vp.float(), index, num, sizes, bs).transpose(1, 2)[:, :lq]
    for hh in (1, 3):
        assert_close(out[:, :, hh], want[:, :, hh], what=f"head {hh} split {split}")
    assert torch.count_nonzero(out[:, :, 0]) == 0 and torch.count_nonzero(out[:, :, 2]) == 0


@pytest.mark.parametrize("use_visits", [False, True])
def test_bsa_arrival_counters_and_empty_rows(use_visits):
    """Multi-unit rows are merged by their last unit: with caller-provided arrival counters the
    output is bit for bit the one of a launch that clears its own, the counters are zero again
    afterwards (a second launch on them agrees too), and rows with no visits (a launched head
    whose top-k is 0, and single empty rows) are written as zero rows."""
    from worldattention_amd.hsa.block_sparse import bsa_forward
    torch.manual_seed(5)
    bs, d, b, h, nq, nkv = 128, 128, 1, 3, 4, 9
    lq, lkv = nq * bs, nkv * bs - 30
    q = torch.randn(b, lq, h, d).bfloat16()
    k = torch.randn(b, lkv, h, d).bfloat16()
    v = torch.randn(b, lkv, h, d).bfloat16()
    index = torch.stack([torch.randperm(nkv) for _ in range(b * h * nq)]).view(b, h, nq, nkv).int()
    ks = [7, 0, 9]
    num = torch.tensor(ks, dtype=torch.int32).view(1, h, 1).expand(b, h, nq).contiguous()
    if not use_visits:
        num[0, 0, 2] = 0                  # one empty row inside a routed head
    args = dict(index=index.to(DEV), num=num.to(DEV), block_size=bs, layout="blhd", lq=lq, lkv=lkv, split=2,
                visits=ks if use_visits else None)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    ref = torch.full((b, lq, h, d), 7.0, dtype=torch.float32, device=DEV)
    bsa_forward(qd, kd, vd, out=ref, **args)
    arrivals = torch.zeros(b * h * nq, dtype=torch.int32, device=DEV)
    for _ in range(2):
        got = torch.full((b, lq, h, d), 7.0, dtype=torch.float32, device=DEV)
        bsa_forward(qd, kd, vd, out=got, arrivals=arrivals, **args)
        assert torch.equal(got, ref)
        assert torch.count_nonzero(arrivals) == 0
    qp = O.pad_to_len(q, nq * bs).transpose(1, 2)
    kp, vp = (O.pad_to_len(t, nkv * bs).transpose(1, 2) for t in (k, v))
    sizes = O.variable_block_sizes(lkv, nkv * bs, bs)
    want = O.block_sparse_attention(qp.float(), kp.float(), vp.float(), index, num, sizes, bs).transpose(1, 2)[:, :lq]
    assert_close(ref, want, what="split rows")
    assert torch.count_nonzero(ref[:, :, 1]) == 0
    if not use_visits:
        assert torch.count_nonzero(ref[:, 2 * bs:3 * bs, 0]) == 0


@pytest.mark.parametrize("order", ["rising", "falling"])
@pytest.mark.parametrize("split", [2, 16])
def test_bsa_large_logits_rescale_matches_oracle(order, split):
    """Logits up to ~170 (log2 units) whose maxima rise (or fall) by ~15 per key block along the
    visit order (ascending block id): the forward's running max lags the scores, and the sum check
    must move it (rescaling the accumulators) on the first step and on most later ones, or never
    after the first when the scores fall. Split rows merge partials whose log-sum-exps differ by
    far more than fp32 exponents of the raw scores could hold."""
    from worldattention_amd.hsa.block_sparse import bsa_forward
    torch.manual_seed(11)
    bs, d, b, h, nq, nkv = 128, 128, 1, 2, 2, 12
    lq, lkv = nq * bs, nkv * bs - 50
    q = torch.randn(b, lq, h, d) * 2
    grow = torch.arange(nkv, dtype=torch.float32) * 2 + 1
    if order == "falling":
        grow = grow.flip(0)
    k = torch.randn(b, nkv * bs, h, d) * grow.repeat_interleave(bs).view(1, -1, 1, 1)
    k = k[:, :lkv]
    v = torch.randn(b, lkv, h, d)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    index = torch.stack([torch.randperm(nkv) for _ in range(b * h * nq)]).view(b, h, nq, nkv).int()
    num = torch.full((b, h, nq), nkv, dtype=torch.int32)
    num[0, 1, 1] = 5
    got, _ = bsa_forward(q.to(DEV), k.to(DEV), v.to(DEV), index=index.to(DEV), num=num.to(DEV), block_size=bs,
                         layout="blhd", lq=lq, lkv=lkv, split=split, out_dtype=torch.float32)
    qp = O.pad_to_len(q, nq * bs).transpose(1, 2)
    kp, vp = (O.pad_to_len(t, nkv * bs).transpose(1, 2) for t in (k, v))
    sizes = O.variable_block_sizes(lkv, nkv * bs, bs)
    want = O.block_sparse_attention(qp.float(), kp.float(), vp.float(), index, num, sizes, bs).transpose(1, 2)[:, :lq]
    assert torch.isfinite(got).all()
    assert_close(got, want, what=f"{order} logits, split {split}")


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("split", [32, 64])
@pytest.mark.parametrize("logits", ["plain", "rising"])
def test_bsa_key_split_long_rows_match_oracle(d, split, logits):
    """64-key blocks with units of at least 32 visits run the key-split kernel (two waves per query
    tile, one per 32-key half of every step, merged in LDS): rows of 0 to 90 visits (several units
    per row past `split`, each unit's slice visited in block order), a partial last key block whose
    real keys end inside the first half of its step, a partial last query block, duplicates, and
    logits that rise along the blocks so the halves' running maxima differ when they merge."""
    from worldattention_amd.hsa.block_sparse import bsa_forward
    torch.manual_seed(d + split)
    bs, b, h, nq, nkv = 64, 1, 2, 3, 90
    lq, lkv = nq * bs - 20, nkv * bs - 40
    q = torch.randn(b, lq, h, d)
    k = torch.randn(b, nkv * bs, h, d)
    if logits == "rising":
        q = q * 2
        k = k * (torch.arange(nkv, dtype=torch.float32) * 0.25 + 1).repeat_interleave(bs).view(1, -1, 1, 1)
    k = k[:, :lkv]
    v = torch.randn(b, lkv, h, d)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    index = torch.stack([torch.randperm(nkv) for _ in range(b * h * nq)]).view(b, h, nq, nkv).int()
    num = torch.tensor([[90, 0, 33], [64, 71, 20]], dtype=torch.int32).view(b, h, nq)
    index[0, 1, 0, 10:13] = 17              # duplicates count
    got, _ = bsa_forward(q.to(DEV), k.to(DEV), v.to(DEV), index=index.to(DEV), num=num.to(DEV), block_size=bs,
                         layout="blhd", lq=lq, lkv=lkv, split=split, out_dtype=torch.float32)
    qp = O.pad_to_len(q, nq * bs).transpose(1, 2)
    kp, vp = (O.pad_to_len(t, nkv * bs).transpose(1, 2) for t in (k, v))
    sizes = O.variable_block_sizes(lkv, nkv * bs, bs)
    want = O.block_sparse_attention(qp.float(), kp.float(), vp.float(), index, num, sizes, bs).transpose(1, 2)[:, :lq]
    assert torch.isfinite(got).all()
    assert_close(got, want, what=f"key split d={d} split={split} {logits}")
    assert torch.count_nonzero(got[0, bs:2 * bs, 0]) == 0


def test_hsa_forward_graph_replays_equal_eager_calls():
    """The cfg 2 call captured in a HIP graph (as bench.py times it): every replay, with eager work
    and synchronizations between replays, equals the eager call bit for bit."""
    cfg = workloads.cfg2(device=DEV, seed=3)
    q, k, v = cfg["q"], cfg["k"], cfg["v"]
    kw = dict(k_coarse=None, v_coarse=None, k_proj_mat=None, v_proj_mat=None, gate_lin=None,
              block_size=cfg["block_size"], tau_min=0.35, tau_max=1.0, proj_segment_len=cfg["proj_segment_len"],
              routing=cfg["routing"], topk=cfg["topk"], head_modes=cfg["head_modes"], linear_mode=cfg["linear_mode"])

    def call():
        with torch.no_grad():
            return WA.hsa_forward(q, k, v, **kw)

    want = call().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = call()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from the eager call"
        other = call()                    # eager work between replays
        assert torch.equal(other, want)
        torch.cuda.synchronize()


def test_native_split_forward_equals_the_python_orchestration():
    """hsa_forward of split heads (top-k sparse, elu1 linear, bf16) runs as one library call
    (wa_hsa_fwd). With a trained gate it gives, bit for bit, the output and routing of the same
    entry points called one by one from Python (pooling, routing, the sparse launch, the elu1
    state and the gated readout)."""
    from worldattention_amd import _lib
    from worldattention_amd.hsa.block_sparse import bsa_forward
    cfg = workloads.cfg2(device=DEV, seed=6)
    q, k, v = cfg["q"], cfg["k"], cfg["v"]
    b, lq, h, d = q.shape
    lkv, bs = k.shape[1], cfg["block_size"]
    gate = torch.nn.Linear(d, d).to(DEV)
    with torch.no_grad():
        gate.weight.normal_(0, 0.05)
        gate.bias.normal_(0, 0.05)
    kw = dict(k_coarse=None, v_coarse=None, k_proj_mat=None, v_proj_mat=None, gate_lin=gate,
              block_size=bs, tau_min=0.35, tau_max=1.0, proj_segment_len=cfg["proj_segment_len"],
              routing=cfg["routing"], topk=cfg["topk"], head_modes=cfg["head_modes"], linear_mode=cfg["linear_mode"])
    save = {}
    with torch.no_grad():
        got = WA.hsa_forward(q, k, v, save=save, **kw)

    plan = WA.HeadPlan(h, cfg["head_modes"], DEV)
    spec = WA.GateSpec(gate, v.dtype)
    ks = WA._per_head_k(cfg["topk"], h)
    _, _, nq, nkv = WR.block_counts(lq, lkv, bs)
    want = torch.empty_like(got)
    with torch.no_grad():
        qp, kp, key_args = WR.pool_for_routing(q, k, lq, lkv, bs, plan.t["sparse"])
        arrivals = torch.empty(b * len(plan.sparse_only) * nq, dtype=torch.int32, device=DEV)
        route, _ = WR._route(None, qp, kp, mode=_lib.WA_ROUTE_TOPK, head_k=ks, heads=plan.t["sparse"],
                             clear=arrivals, **key_args)
        bsa_forward(q, k, v, index=route.index, num=route.num, block_size=bs, layout="blhd",
                    heads=plan.t["sparse_only"], out=want, lq=lq, lkv=lkv, attn_round_bf16=True,
                    visits=[min(ks[i], nkv) for i in plan.sparse_only], arrivals=arrivals)
        s, z = WA.elu1_state(k, v, plan.t["linear_only"])
        WA.elu1_readout(q, s, z, plan.t["linear_only"], want, epilogue=_lib.WA_EPI_GATED, lin_round_bf16=True,
                        **spec.kwargs())
    assert torch.equal(got, want)
    sparse = plan.sparse_only
    assert torch.equal(save["route"].index[:, sparse], route.index[:, sparse])
    assert torch.equal(save["route"].num[:, sparse], route.num[:, sparse])


def _split_kw(cfg, gate):
    return dict(k_coarse=None, v_coarse=None, k_proj_mat=None, v_proj_mat=None, gate_lin=gate,
                block_size=cfg["block_size"], tau_min=0.35, tau_max=1.0, proj_segment_len=cfg["proj_segment_len"],
                routing=cfg["routing"], topk=cfg["topk"], head_modes=cfg["head_modes"],
                linear_mode=cfg["linear_mode"])


def _trained_gate(d, seed):
    gen = torch.Generator().manual_seed(seed)
    gate = torch.nn.Linear(d, d)
    with torch.no_grad():
        gate.weight.copy_(torch.randn(d, d, generator=gen) * 0.05)
        gate.bias.copy_(torch.randn(d, generator=gen) * 0.05)
    return gate.to(DEV)


def test_native_split_forward_concurrent_streams_equal_serial():
    """Two threads call the one-call forward (wa_hsa_fwd) at the same time, each on its own stream
    (so each gets its own side stream and fork / join events and nothing is shared between the
    calls): every result equals the same call made alone."""
    import threading
    cfgs = [workloads.cfg2(device=DEV, seed=s) for s in (7, 8)]
    gates = [_trained_gate(c["q"].shape[-1], 20 + i) for i, c in enumerate(cfgs)]
    with torch.no_grad():
        want = [WA.hsa_forward(c["q"], c["k"], c["v"], **_split_kw(c, g)) for c, g in zip(cfgs, gates)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in cfgs]
    got = [[None] * 4 for _ in cfgs]
    errors = []
    barrier = threading.Barrier(len(cfgs))

    def worker(i):
        try:
            c = cfgs[i]
            with torch.no_grad(), torch.cuda.stream(streams[i]):
                barrier.wait()
                for r in range(4):
                    got[i][r] = WA.hsa_forward(c["q"], c["k"], c["v"], **_split_kw(c, gates[i]))
        except Exception as e:  # reported below, from the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cfgs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(len(cfgs)):
        for r in range(4):
            assert torch.equal(got[i][r], want[i]), f"thread {i} call {r} differs from the serial call"


def test_native_split_forward_without_side_stream_is_identical(monkeypatch):
    """wa_hsa_fwd with a NULL side stream runs both branches on the caller's stream, with the same
    output bit for bit as the forked call."""
    cfg = workloads.cfg2(device=DEV, seed=9)
    gate = _trained_gate(cfg["q"].shape[-1], 30)
    with torch.no_grad():
        forked = WA.hsa_forward(cfg["q"], cfg["k"], cfg["v"], **_split_kw(cfg, gate))
    monkeypatch.setattr(WA, "_fork_join", lambda dev, main: (None, None, None))
    with torch.no_grad():
        single = WA.hsa_forward(cfg["q"], cfg["k"], cfg["v"], **_split_kw(cfg, gate))
    torch.cuda.synchronize()
    assert torch.equal(single, forked)
