"""The allocation-free backward entry point (lsfa_bwd_noalloc) against
lsfa_bwd on the same arguments.

lsfa_bwd_noalloc takes lsfa_bwd's arguments but ignores the workspace: it
runs lsfa_bwd's default kernels with the library's own device scratch array,
so its gradients must equal lsfa_bwd's bit for bit. Two calls in a row, the
second with a smaller problem (the array keeps the first call's contents),
and the split-phase timing mode through the same array.
"""
import pytest
import torch

from lightserve_amd import _lib
from lightserve_amd.kernels.flash_attention_backward import _backward_args, _flash_attention_forward_lse

pytestmark = pytest.mark.gpu


def _inputs(B, H, N, D, seed, device):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(B, H, N, D, generator=g) * 0.5).to(torch.bfloat16).to(device) for _ in range(4)]


def test_noalloc_matches_bwd(gpu):
    stream = _lib.current_stream(gpu)
    for B, H, N, D, causal in ((2, 4, 600, 128, True), (1, 3, 150, 64, False)):
        print(f"case bwd_noalloc {B}x{H}x{N}x{D} causal={causal}", flush=True)
        q, k, v, do = _inputs(B, H, N, D, N, gpu)
        o, L = _flash_attention_forward_lse(q, k, v, causal)
        args, keep = _backward_args(do, q, k, v, o, L, causal)
        outs = keep[3]
        _lib.bwd(args, stream)
        ref = [t.clone() for t in outs]
        for t in outs:
            t.fill_(float("nan"))
        args.workspace, args.workspace_bytes = None, 0
        _lib.bwd_noalloc(args, stream)
        torch.cuda.synchronize()
        for name, got, want in zip(("dq", "dk", "dv"), outs, ref):
            assert torch.equal(got, want), name
        # the two kernels one at a time, sharing the library's array
        for t in outs:
            t.fill_(float("nan"))
        for f in (_lib.BWD_ONLY_DQ, _lib.BWD_ONLY_DKDV):
            args.flags = f
            _lib.bwd_noalloc(args, stream)
        args.flags = 0
        torch.cuda.synchronize()
        for name, got, want in zip(("dq", "dk", "dv"), outs, ref):
            assert torch.equal(got, want), f"phases {name}"
