"""Python call surface of the gfx950 attention kernels (same names as the reference's kernels/)."""
from .flash_attention import flash_attention_forward
from .flash_attention_backward import flash_attention
from .flash_attention_varlen import flash_attention_varlen_forward

__all__ = ["flash_attention_forward", "flash_attention", "flash_attention_varlen_forward"]
