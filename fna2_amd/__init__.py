"""fna2_amd — FlashNaylisAttention-2 forward/backward for AMD MI355X (gfx950).

The hot path is ``flash_naylis_attn`` (module ``flash_naylis_attn``), backed by
hand-written HIP kernels in ``csrc/`` behind the C ABI of ``include/fna2.h``.
``attention_fna2`` holds the ``NaylisAttention`` caller with the reference's
constructor and forward signatures.
"""
from .flash_naylis_attn import (  # noqa: F401
    BLOCK_M,
    BLOCK_N,
    BLOCK_R,
    FlashNaylisAttnFunc,
    flash_naylis_attn,
)

__all__ = ["BLOCK_M", "BLOCK_N", "BLOCK_R", "FlashNaylisAttnFunc", "flash_naylis_attn"]
