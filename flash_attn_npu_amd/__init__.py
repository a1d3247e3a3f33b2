"""FlashAttention forward for AMD Instinct MI355X (gfx950).

`flash_attn_npu_amd.flash_attention_forward` is the drop-in module for the
reference's flash_attention_forward.py; its `attention` (alias
`flash_attention_forward`) launches the hand-written HIP kernel in
libfa_mi355x.so through the C ABI of include/fa_fwd.h.
"""

from . import flash_attention_forward  # noqa: F401  (the drop-in module)
from .flash_attention_forward import DEVICE, PROFILE_OP_NAME, attention  # noqa: F401
