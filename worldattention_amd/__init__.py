"""worldattention_amd — MI355X-native Hybrid Sparse Attention (HSA) + Hierarchical KV cache (HKV).

``worldattention_amd.hsa`` mirrors ``wan.modules.hsa`` and ``worldattention_amd.hkv`` mirrors
``pipeline.hkv`` of alibaba-damo-academy/WorldAttention; both run hand-written gfx950 HIP kernels
from ``libworldattention_amd.so`` through its C ABI (``include/worldattention_amd.h``).
"""

__version__ = "0.1.0"
