"""CPU oracle for the HSA + HKV attention path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU (fp32, or fp64 where asked), the semantics of the
reference's attention path:

* ``oracle.hsa`` — routing, block-sparse attention, low-rank compression, both linear-branch modes,
  gated fusion and the full ``hsa_attention`` composition
  (reference: ``wan/modules/hsa/{routing,block_sparse_torch,attention}.py``,
  ``trainer/hsa_stage.py``);
* ``oracle.hkv`` — page summaries, temporal re-rotation, two-stage retrieval, install planning and
  the LRU tier (reference: ``pipeline/hkv/{retrieval,rope,cache,tiering}.py``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker or the reported CPU baseline. The product package
``worldattention_amd`` never imports it and has no CPU fallback.

Pinning status of each function is listed in its docstring ("pinned by: ..."). Functions whose
results have no independent check say "parity unpinned".
"""
