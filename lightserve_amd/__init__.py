"""MI355X-native FlashAttention for lightserve's attention hot path.

Public entry points (mirroring the reference's kernels/ package):
    lightserve_amd.kernels.flash_attention.flash_attention_forward
    lightserve_amd.kernels.flash_attention_backward.flash_attention
    lightserve_amd.kernels.flash_attention_varlen.flash_attention_varlen_forward
Importing the package loads no native code; the gfx950 library
(liblsfa_gfx950.so) is loaded on the first kernel call.
"""
__version__ = "0.1.0"
