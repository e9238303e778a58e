"""sophia_amd: the Kimi Delta Attention (KDA) mixer hot path of Arain119/Sophia,
rebuilt for AMD MI355X (gfx950).

* ``sophia_amd.kda``    -- ``SophiaKDA`` / ``CausalDepthwiseConv1d`` /
  ``set_pad_mask``: drop-ins for ml/runtime/model/attention.py.
* ``sophia_amd.ops``    -- torch-facing kernel entry points, including the
  flash-linear-attention signatures ``chunk_kda`` / ``fused_recurrent_kda``.
* ``sophia_amd._native``-- ctypes binding of the C ABI (include/sophia_kda.h)
  exported by ``sophia_amd/_lib/libsophia_kda.so``.
* ``sophia_amd.build``  -- hipcc build of that library.
"""

from .config import ModelArgs
from .state import LayerCacheSnapshot, RuntimeCacheSnapshot

__all__ = ["ModelArgs", "LayerCacheSnapshot", "RuntimeCacheSnapshot"]
