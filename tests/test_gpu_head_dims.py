"""Head dims other than 64 and 128 on the GPU against the CPU oracle.

The reference's functional API and module take any head dim (its own module tests run
``head_dim=16``, ``tests/test_hsa_attention.py:30-49``); the kernels take 64 and 128, so other head
dims run padded (queries / values / gate with zeros, keys with ``PAD_KEY_VALUE``) at the original
``head_dim ** -0.5``. The oracle is the same dimension-generic restatement the 64 / 128 tests use.

Tolerances as the other forward / backward tests: outputs max-abs <= 2e-2, mean-abs <= 2e-3 against
the fp32 oracle; input gradients the same; gate-parameter gradients (sums over tokens) 0.1 / 1e-2.
"""
import pytest
import torch

from oracle import hsa as O
from worldattention_amd import hsa as W
from worldattention_amd.hsa import attention as WA
from worldattention_amd.hsa import distill
from worldattention_amd.hsa_stage import init_hsa_parameters

pytestmark = pytest.mark.gpu
DEV = "cuda"


def assert_close(got, want, max_abs=2e-2, mean_abs=2e-3, what=""):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    assert got.shape == want.shape, f"{what}: {tuple(got.shape)} vs {tuple(want.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    diff = (got - want).abs()
    assert diff.max().item() <= max_abs, f"{what}: max-abs {diff.max().item():.3e} > {max_abs}"
    assert diff.mean().item() <= mean_abs, f"{what}: mean-abs {diff.mean().item():.3e} > {mean_abs}"


def _inputs(d, h=3, lq=100, lkv=300, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, lq, h, d, generator=g)
    k = torch.randn(1, lkv, h, d, generator=g) + torch.randn(1, lkv // 50 + 1, h, d, generator=g).repeat_interleave(
        50, dim=1)[:, :lkv]
    v = torch.randn(1, lkv, h, d, generator=g)
    w = torch.randn(d, d, generator=g) * 0.1
    b = torch.randn(d, generator=g) * 0.1
    return q, k, v, w, b


def _gate(w, b):
    lin = torch.nn.Linear(w.shape[1], w.shape[0]).to(DEV)
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(b)
    return lin


MODES = {
    # the reference's default: Gini routing, low-rank linear branch, both branches on every head
    "reference": dict(block_size=64, routing="gini", linear_mode="lowrank", proj_segment_len=100),
    # the north star's head-adaptive mode: top-k sparse heads and elu(x)+1 linear heads
    "split": dict(block_size=64, routing="topk", topk=[2, 0, 3], head_modes=["sparse", "linear", "sparse"],
                  linear_mode="elu1", proj_segment_len=100),
}


@pytest.mark.parametrize("mode", ["reference", "split"])
@pytest.mark.parametrize("d", [16, 32, 96])
def test_hsa_attention_at_other_head_dims_matches_oracle(d, mode):
    q, k, v, w, b = _inputs(d, seed=d)
    kw = MODES[mode]
    proj = O.init_projection(-(-kw["proj_segment_len"] // kw["block_size"]), kw["proj_segment_len"], 64)
    want = O.hsa_attention(q, k, v, k_proj_mat=proj, v_proj_mat=proj, gate_weight=w, gate_bias=b, **kw)
    with torch.no_grad():
        got = W.hsa_attention(q.to(DEV), k.to(DEV), v.to(DEV), k_proj_mat=proj.to(DEV), v_proj_mat=proj.to(DEV),
                              gate_lin=_gate(w, b), **kw)
    assert got.shape == (1, 100, 3, d) and got.is_contiguous()
    assert_close(got, want, what=f"{mode} d={d}")


@pytest.mark.parametrize("mode,d", [("reference", 16), ("split", 96)])
def test_gradients_at_other_head_dims_match_oracle(mode, d):
    """dQ, dK, dV and the gate's dW, db through the padding (fp32 inputs, fp32 oracle autograd)."""
    q, k, v, w, b = _inputs(d, seed=d + 1)
    kw = MODES[mode]
    proj = O.init_projection(-(-kw["proj_segment_len"] // kw["block_size"]), kw["proj_segment_len"], 64)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(5))
    ref = [t.clone().requires_grad_() for t in (q, k, v, w, b)]
    O.hsa_attention(*ref[:3], k_proj_mat=proj, v_proj_mat=proj, gate_weight=ref[3], gate_bias=ref[4],
                    **kw).backward(do)
    qg, kg, vg = (t.to(DEV).requires_grad_() for t in (q, k, v))
    gate = _gate(w, b)
    out = W.hsa_attention(qg, kg, vg, k_proj_mat=proj.to(DEV), v_proj_mat=proj.to(DEV), gate_lin=gate, **kw)
    out.backward(do.to(DEV))
    for name, got, r in (("dq", qg.grad, ref[0].grad), ("dk", kg.grad, ref[1].grad), ("dv", vg.grad, ref[2].grad)):
        assert got.shape == r.shape
        assert_close(got, r, what=f"{mode} d={d} {name}")
    assert_close(gate.weight.grad, ref[3].grad, 0.1, 1e-2, what=f"{mode} d={d} dW")
    assert_close(gate.bias.grad, ref[4].grad, 0.1, 1e-2, what=f"{mode} d={d} db")


def test_module_at_head_dim_16_as_the_reference_tests_it():
    """HSAAttention(num_heads=3, head_dim=16, block_size=64, proj_segment_len=50), initialized by the
    block-averaging rule, on 100 queries over 200 keys: the output equals the oracle's, and a
    backward reaches q, k, v and the gate with finite gradients of the right shapes."""
    torch.manual_seed(0)
    m = WA.HSAAttention(num_heads=3, head_dim=16, block_size=64, tau_min=0.35, tau_max=1.0, proj_segment_len=50)
    init_hsa_parameters(m)
    with torch.no_grad():
        m.gate_lin.bias.fill_(0.3)
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, n, 3, 16, generator=g) for n in (100, 200, 200))
    want = O.hsa_attention(q, k, v, k_proj_mat=m.k_proj_mat.detach(), v_proj_mat=m.v_proj_mat.detach(),
                           gate_weight=m.gate_lin.weight.detach(), gate_bias=m.gate_lin.bias.detach(), block_size=64,
                           proj_segment_len=50)
    m = m.to(DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = m(qg, kg, vg)
    assert_close(out, want, what="module head_dim 16")
    out.square().sum().backward()
    for t in (qg, kg, vg, m.gate_lin.weight, m.gate_lin.bias):
        assert t.grad is not None and t.grad.shape == t.shape and torch.isfinite(t.grad).all()


@pytest.mark.parametrize("d", [16, 96])
def test_building_blocks_at_other_head_dims_match_oracle(d):
    """block_sparse_attention_reference, compress_kv, the low-rank branch and the dense teacher."""
    torch.manual_seed(d)
    bs, nq, nkv = 64, 3, 5
    lkv = nkv * bs - 20
    q, k, v = (torch.randn(1, 2, n * bs, d).bfloat16() for n in (nq, nkv, nkv))
    k[:, :, lkv:] = 0
    v[:, :, lkv:] = 0
    index = torch.stack([torch.randperm(nkv) for _ in range(2 * nq)]).view(1, 2, nq, nkv).int()
    num = torch.randint(1, nkv + 1, (1, 2, nq), dtype=torch.int32)
    sizes = O.variable_block_sizes(lkv, nkv * bs, bs)
    want = O.block_sparse_attention(q, k, v, index, num, sizes, bs)
    got = W.block_sparse_attention_reference(q.to(DEV), k.to(DEV), v.to(DEV), index.to(DEV), num.to(DEV),
                                             sizes.to(DEV), bs)
    assert_close(got, want, what=f"block-sparse d={d}")

    kk, vv = torch.randn(1, 2, 700, d), torch.randn(1, 2, 700, d)
    proj = O.init_projection(4, 200, 64)
    wk, wv = O.compress_kv(kk, vv, segment_len=200, k_proj_mat=proj, v_proj_mat=proj, block_size=64)
    gk, gv = W.compress_kv(kk.to(DEV), vv.to(DEV), segment_len=200, k_proj_mat=proj.to(DEV), v_proj_mat=proj.to(DEV),
                           block_size=64)
    assert_close(gk, wk, 1e-2, 1e-3, what=f"compress k d={d}")
    assert_close(gv, wv, 1e-2, 1e-3, what=f"compress v d={d}")

    qq = torch.randn(1, 2, 150, d)
    assert_close(WA._linear_branch(qq.to(DEV), wk.to(DEV), wv.to(DEV)), O.linear_branch_lowrank(qq, wk, wv),
                 what=f"low-rank branch d={d}")

    qd, kd, vd = torch.randn(1, 300, 2, d), torch.randn(1, 500, 2, d), torch.randn(1, 500, 2, d)
    want_t = O.linear_branch_lowrank(qd.transpose(1, 2), kd.transpose(1, 2), vd.transpose(1, 2)).transpose(1, 2)
    assert_close(distill.dense_attention(qd.to(DEV), kd.to(DEV), vd.to(DEV)), want_t, what=f"dense teacher d={d}")
