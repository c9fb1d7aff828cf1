"""Host-side behaviour of the product API that needs no GPU: validation errors raised before any
kernel call (mirroring the reference's), parameter bookkeeping, the distillation registry, and the
absence of any CPU fallback."""
import pytest
import torch

from worldattention_amd import hsa as W
from worldattention_amd.hsa import attention as WA
from worldattention_amd.hsa import distill
from worldattention_amd.hsa_stage import init_hsa_parameters


def _module(**kw):
    torch.manual_seed(0)
    return W.HSAAttention(num_heads=3, head_dim=64, block_size=64, proj_segment_len=50, backend="torch", **kw)


def test_backend_resolution_accepts_reference_names_and_rejects_others():
    assert W.resolve_backend("torch") == "torch"
    assert W.resolve_backend("triton") == "triton"
    assert W.resolve_backend("auto") in ("torch", "triton")
    with pytest.raises(ValueError):
        W.resolve_backend("nope")


def test_block_size_is_validated():
    with pytest.raises(ValueError):
        W.HSAAttention(num_heads=1, head_dim=64, block_size=32)
    assert W.HSAAttention(num_heads=1, head_dim=64, block_size=128).proj_rank == 13
    with pytest.raises(ValueError):
        W.HSAAttention(num_heads=2, head_dim=64, head_modes=["both", "nope"])
    with pytest.raises(ValueError):
        W.HSAAttention(num_heads=2, head_dim=64, linear_mode="nope")


def test_parameters_start_at_zero_and_checkpoint_keys_match_the_reference():
    hsa = _module()
    assert hsa.k_proj_mat.shape == (1, 50) and hsa.k_proj_mat.dtype == torch.bfloat16
    for p in (hsa.k_proj_mat, hsa.v_proj_mat, hsa.gate_lin.weight, hsa.gate_lin.bias):
        assert torch.count_nonzero(p) == 0
    assert sorted(W.hsa_parameter_names(hsa)) == ["gate_lin.bias", "gate_lin.weight", "k_proj_mat", "v_proj_mat"]
    W.require_trained_hsa([], "ckpt.pt")
    W.require_trained_hsa(["blocks.0.self_attn.q.weight"])
    with pytest.raises(RuntimeError, match="HSA training"):
        W.require_trained_hsa(["blocks.0.self_attn.hsa_attention.k_proj_mat"], "ckpt.pt")


def test_training_initialization_gives_block_pooling():
    hsa = _module()
    assert init_hsa_parameters(hsa) == 1
    row = hsa.k_proj_mat[0]
    assert int((row != 0).sum()) == 50 and abs(row[0].item() - 1 / 50) < 1e-3
    wide = W.HSAAttention(num_heads=1, head_dim=64, block_size=128, proj_segment_len=1560)
    init_hsa_parameters(wide)
    assert int((wide.k_proj_mat[12] != 0).sum()) == 1560 - 12 * 128


def test_coarse_cache_sizing_and_alignment():
    hsa = _module()
    assert hsa.coarse_cache_size(0) == 0
    assert hsa.coarse_cache_size(50) == hsa.proj_rank
    assert hsa.coarse_cache_size(200) == 4 * hsa.proj_rank
    assert hsa.token_range_to_coarse(50, 150) == (1, 3)
    with pytest.raises(ValueError):
        hsa.token_range_to_coarse(0, 51)
    assert WA.coarse_length(32760, 1560, 13, 128) == 21 * 13
    assert WA.coarse_length(200, 50, 1, 64) == 4


def test_argument_validation_matches_the_reference():
    q = torch.zeros(1, 4, 2, 64)
    kv = torch.zeros(1, 8, 2, 64)
    proj = torch.zeros(1, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="together"):
        W.hsa_attention(q, kv, kv, k_coarse=kv, k_proj_mat=proj, v_proj_mat=proj)
    with pytest.raises(ValueError, match="positive"):
        W.hsa_attention(q[:, :0], kv, kv, k_proj_mat=proj, v_proj_mat=proj)
    with pytest.raises(ValueError, match="k_coarse"):
        W.hsa_attention(q, kv, kv, k_coarse=torch.zeros(1, 2, 3, 64), v_coarse=torch.zeros(1, 2, 3, 64),
                        k_proj_mat=proj, v_proj_mat=proj)
    with pytest.raises(ValueError, match="same shape"):
        W.compress_kv(kv, kv, segment_len=8, k_proj_mat=proj, v_proj_mat=torch.zeros(2, 8), block_size=64)


def test_cpu_tensors_are_rejected_there_is_no_fallback():
    hsa = _module()
    q, k = torch.randn(1, 64, 3, 64), torch.randn(1, 128, 3, 64)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm GPU"):
        hsa(q, k, k)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        W.build_block_routing(torch.rand(1, 1, 2, 4), 0.35, 1.0)


def test_distillation_registry():
    assert distill.pop_distill_losses() == []
    distill.enable_distill(True)
    try:
        distill.record_distill_loss(torch.tensor(1.0))
        assert len(distill.pop_distill_losses()) == 1
        assert distill.pop_distill_losses() == []
    finally:
        distill.enable_distill(False)
    assert not distill.distill_enabled()


def test_gate_kernel_copies_follow_the_parameter_object():
    """The bf16 / fp32 copies handed to the fusion kernels live on the parameter itself: a new
    module never sees another module's copy (even at a reused address), and an in-place update
    refreshes the copy."""
    from worldattention_amd.hsa.attention import GateSpec
    a, b = torch.nn.Linear(8, 8), torch.nn.Linear(8, 8)
    with torch.no_grad():
        b.weight.copy_(a.weight * 3)
    wa = GateSpec(a, torch.float32).w
    wb = GateSpec(b, torch.float32).w
    assert torch.equal(wa.float(), a.weight.detach().bfloat16().float())
    assert torch.equal(wb.float(), b.weight.detach().bfloat16().float())
    assert GateSpec(a, torch.float32).w is wa                      # unchanged parameter: reused
    with torch.no_grad():
        a.weight.add_(1.0)
    assert torch.equal(GateSpec(a, torch.float32).w.float(), a.weight.detach().bfloat16().float())


def test_empty_head_lists_are_refused_at_the_c_boundary():
    """A missing head list means every head to the library, so an empty one (whose data pointer
    can be NULL) is refused before any call; a list of heads passes through."""
    from worldattention_amd import _lib
    with pytest.raises(ValueError, match="empty head list"):
        _lib.heads_arg(torch.zeros(0, dtype=torch.int32))
    assert _lib.heads_arg(None) == (None, 0)
    t = torch.tensor([1, 3], dtype=torch.int32)
    assert _lib.heads_arg(t) == (t.data_ptr(), 2)
