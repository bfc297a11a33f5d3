"""fna2_amd — FlashNaylisAttention-2 forward/backward for AMD MI355X (gfx950).

The hot path is ``flash_naylis_attn`` (module ``flash_naylis_attn``), backed by
hand-written HIP kernels in ``csrc/`` behind the C ABI of ``include/fna2.h``.
``attention_fna2`` holds the ``NaylisAttention`` caller with the reference's
constructor and forward signatures.  Around the path: ``rope.rope_varlen``
(varlen rotary embedding, optionally with the QK RMSNorm) and
``decode.flash_naylis_decode`` (one-token decode against a KV cache).
``ops`` registers the path as the custom operators ``fna2::fwd`` /
``fna2::bwd`` (fake and autograd registrations), which ``flash_naylis_attn``
calls, so that ``torch.compile`` traces it.
"""
from .decode import flash_naylis_decode  # noqa: F401
from .flash_naylis_attn import (  # noqa: F401
    BLOCK_M,
    BLOCK_N,
    BLOCK_R,
    FlashNaylisAttnFunc,
    flash_naylis_attn,
)
from .rope import rope_varlen  # noqa: F401
from . import ops  # noqa: F401,E402  (registers the fna2::fwd / fna2::bwd custom ops)

__all__ = ["BLOCK_M", "BLOCK_N", "BLOCK_R", "FlashNaylisAttnFunc", "flash_naylis_attn",
           "flash_naylis_decode", "rope_varlen"]
