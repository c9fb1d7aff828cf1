"""Write golden vectors for the two functions no closed form pins bit-exactly.

Run once, in the build container (the reference tree is not present on GPU boxes):

    python tests/golden/make_golden.py /root/reference

It loads the reference's HSA leaf package ``wan/modules/hsa`` by file path under a private package
name (so the heavy ``wan/__init__.py`` is never executed) and records, on seeded tie-free inputs:

* ``routing_gini.pt`` — ``build_block_routing`` (Gini thresholds, counts, permutation): the fp32
  rounding of the Gini mean/threshold and the double ``cumsum`` decide ``num`` near boundaries;
* ``hsa_attention.pt`` — ``hsa_attention`` end to end (torch backend, fp32 and bf16 inputs, padded
  lengths, a trained-looking gate): the composed cast sequence of ``attention.py:184-259``;
* ``routing_boundary.pt`` — ``build_block_routing`` on maps crafted so that some rows' exclusive
  prefix lies -3..+3 fp32 ulp from the head threshold: where ``num`` turns on the threshold's
  last bits.

Only inputs and outputs are written; no reference source is copied.
"""
from __future__ import annotations

import importlib.util
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference_hsa(ref_root: str):
    # the reference tree is read-only: importing it must not leave __pycache__ directories there
    sys.dont_write_bytecode = True
    pkg_dir = os.path.join(ref_root, "wan", "modules", "hsa")
    spec = importlib.util.spec_from_file_location(
        "_reference_hsa", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    module = importlib.util.module_from_spec(spec)
    sys.modules["_reference_hsa"] = module
    spec.loader.exec_module(module)
    return module


def routing_cases(ref):
    cases = []
    g = torch.Generator().manual_seed(1234)
    for shape, temp in (((2, 3, 5, 40), 2.0), ((1, 4, 7, 64), 4.0), ((1, 2, 37, 256), 3.0)):
        attn = torch.softmax(torch.randn(shape, generator=g) * temp, dim=-1)
        for tau_min, tau_max in ((0.35, 1.0), (0.1, 0.9)):
            r = ref.build_block_routing(attn, tau_min, tau_max, return_mask=True)
            cases.append(dict(block_attn=attn, tau_min=tau_min, tau_max=tau_max, index=r.index,
                              num=r.num, mask=r.mask, thresholds=r.thresholds))
    return cases


def _ulp(x: float) -> float:
    import math
    m, e = math.frexp(abs(x))
    return 2.0 ** (e - 24)


def routing_boundary_cases(ref):
    """Maps with rows whose exclusive prefix sits a few fp32 ulp from the head threshold.

    For head 0 of each map, target rows get their largest weight nudged (iterating, since every row
    moves the head's Gini mean) until the reference's exclusive prefix at a chosen slot lands
    ``delta`` ulp from the reference's threshold: there ``num`` depends on the last bits of the
    fp32 Gini mean. Each case records, per target row, the slot and the offset actually reached
    (measured with the reference's own outputs)."""
    cases = []
    g = torch.Generator().manual_seed(777)
    for shape, temp in (((1, 2, 12, 16), 2.0), ((1, 2, 37, 256), 3.0)):
        attn = torch.softmax(torch.randn(shape, generator=g) * temp, dim=-1)
        deltas = [-3, -2, -1, 0, 1, 2, 3]
        rows = list(range(len(deltas)))
        slots = {}
        for _ in range(60):
            r = ref.build_block_routing(attn, 0.35, 1.0)
            tau = float(r.thresholds[0])
            sp, si = torch.sort(attn.float(), dim=-1, descending=True)
            excl = torch.cumsum(sp, dim=-1) - sp
            done = True
            for row, delta in zip(rows, deltas):
                e = excl[0, 0, row]
                if row not in slots:
                    slots[row] = int(torch.argmin((e[1:] - tau).abs())) + 1
                m = slots[row]
                want = tau + delta * _ulp(tau)
                err = want - float(e[m])
                if abs(err) > 0.25 * _ulp(tau):
                    done = False
                    top = int(si[0, 0, row, 0])
                    attn[0, 0, row, top] = float(attn[0, 0, row, top]) + err
            if done:
                break
        r = ref.build_block_routing(attn, 0.35, 1.0, return_mask=True)
        tau = float(r.thresholds[0])
        sp, _ = torch.sort(attn.float(), dim=-1, descending=True)
        excl = torch.cumsum(sp, dim=-1) - sp
        reached = [round((float(excl[0, 0, row, slots[row]]) - tau) / _ulp(tau)) for row in rows]
        cases.append(dict(block_attn=attn.clone(), tau_min=0.35, tau_max=1.0, index=r.index, num=r.num, mask=r.mask,
                          thresholds=r.thresholds, boundary_head=0, boundary_rows=torch.tensor(rows),
                          boundary_slots=torch.tensor([slots[row] for row in rows]),
                          boundary_ulps=torch.tensor(reached)))
    return cases


def attention_cases(ref):
    cases = []
    g = torch.Generator().manual_seed(4321)
    specs = [
        # (B, Lq, Lkv, H, D, seg, dtype, gate_bias)
        (1, 100, 300, 2, 64, 100, torch.float32, 0.0),
        (1, 128, 512, 2, 64, 128, torch.float32, 0.7),
        (1, 100, 300, 2, 64, 100, torch.bfloat16, -0.4),
        (1, 150, 450, 2, 128, 150, torch.bfloat16, 0.2),
    ]
    for b, lq, lkv, h, d, seg, dtype, bias in specs:
        hsa = ref.HSAAttention(num_heads=h, head_dim=d, block_size=64, tau_min=0.35, tau_max=1.0,
                               proj_segment_len=seg, backend="torch")
        with torch.no_grad():
            for proj in (hsa.k_proj_mat, hsa.v_proj_mat):
                proj.copy_((torch.rand(proj.shape, generator=g) / seg).to(proj.dtype))
            hsa.gate_lin.weight.copy_(torch.randn(d, d, generator=g) * 0.1)
            hsa.gate_lin.bias.fill_(bias)
        if dtype != torch.float32:
            hsa = hsa.to(dtype)
        q = torch.randn(b, lq, h, d, generator=g).to(dtype)
        k = (torch.randn(b, lkv, h, d, generator=g)
             + torch.randn(b, lkv // 50 + 1, h, d, generator=g).repeat_interleave(50, dim=1)[:, :lkv]).to(dtype)
        v = torch.randn(b, lkv, h, d, generator=g).to(dtype)
        with torch.no_grad():
            out = hsa(q, k, v)
        cases.append(dict(q=q, k=k, v=v, k_proj_mat=hsa.k_proj_mat.detach().clone(),
                          v_proj_mat=hsa.v_proj_mat.detach().clone(),
                          gate_weight=hsa.gate_lin.weight.detach().clone(),
                          gate_bias=hsa.gate_lin.bias.detach().clone(),
                          block_size=64, proj_segment_len=seg, tau_min=0.35, tau_max=1.0, out=out))
    return cases


WRITERS = {
    "routing_gini.pt": routing_cases,
    "hsa_attention.pt": attention_cases,
    "routing_boundary.pt": routing_boundary_cases,
}


def main(ref_root: str, only=None) -> None:
    ref = load_reference_hsa(ref_root)
    for name, make in WRITERS.items():
        if only and name not in only:
            continue
        torch.save(make(ref), os.path.join(HERE, name))
        print("wrote", name)


if __name__ == "__main__":
    # python tests/golden/make_golden.py [reference root] [file names to write (default: all)]
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", sys.argv[2:])
