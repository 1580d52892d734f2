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


def test_noalloc_under_graph_capture(gpu):
    """lsfa_bwd_noalloc captured in a HIP graph (the callers it is for): after
    an eager warm-up call, the captured call replays three times, with eager
    work and synchronizations between the replays, and every replay gives
    lsfa_bwd's gradients bit for bit."""
    stream = torch.cuda.Stream(device=gpu)
    q, k, v, do = _inputs(2, 4, 700, 128, 77, gpu)
    o, L = _flash_attention_forward_lse(q, k, v, True)
    args, keep = _backward_args(do, q, k, v, o, L, True)
    outs = keep[3]
    _lib.bwd(args, _lib.current_stream(gpu))
    torch.cuda.synchronize()
    ref = [t.clone() for t in outs]
    args.workspace, args.workspace_bytes = None, 0
    with torch.cuda.stream(stream):
        _lib.bwd_noalloc(args, stream.cuda_stream)  # warm-up: resolves the array's address on this device
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _lib.bwd_noalloc(args, stream.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"case bwd_noalloc graph replay {rep}", flush=True)
        for t in outs:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(("dq", "dk", "dv"), outs, ref):
            assert torch.equal(got, want), f"replay {rep} {name}"


def test_noalloc_varlen_gqa(gpu):
    """A packed varlen batch with GQA (8 query heads over 2 KV heads, ragged
    and empty sequences) through lsfa_bwd_noalloc and lsfa_bwd on the same
    arguments: equal bit for bit, twice in a row."""
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward
    lens_q, lens_k = [300, 0, 77, 513], [300, 40, 200, 513]
    Hq, Hkv, D = 8, 2, 128
    g = torch.Generator().manual_seed(11)
    q, do = ((torch.randn(sum(lens_q), Hq, D, generator=g) * 0.5).bfloat16().to(gpu) for _ in range(2))
    k, v = ((torch.randn(sum(lens_k), Hkv, D, generator=g) * 0.5).bfloat16().to(gpu) for _ in range(2))
    cu = lambda ls: torch.tensor([0] + list(torch.tensor(ls).cumsum(0)), dtype=torch.int32, device=gpu)  # noqa: E731
    cu_q, cu_k = cu(lens_q), cu(lens_k)
    o, lse = flash_attention_varlen_forward(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), True)
    grads = [torch.empty_like(t) for t in (q, k, v)]
    th = _lib.strides_thd
    args = _lib.BwdArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o.data_ptr(), dout=do.data_ptr(), lse=lse.data_ptr(),
        dq=grads[0].data_ptr(), dk=grads[1].data_ptr(), dv=grads[2].data_ptr(), workspace=None, workspace_bytes=0,
        q_stride=th(q), k_stride=th(k), v_stride=th(v), o_stride=th(o), do_stride=th(do), dq_stride=th(grads[0]),
        dk_stride=th(grads[1]), dv_stride=th(grads[2]), lse_stride=_lib._i64x3(0, lse.stride(0), lse.stride(1)),
        cu_seqlens_q=cu_q.data_ptr(), cu_seqlens_k=cu_k.data_ptr(), dtype=_lib.TORCH_TO_LSFA[torch.bfloat16],
        batch=len(lens_q), heads_q=Hq, heads_kv=Hkv, seqlen_q=max(lens_q), seqlen_k=max(lens_k), head_dim=D,
        causal=1, sm_scale=D ** -0.5, flags=0)
    stream = _lib.current_stream(gpu)
    n = _lib.bwd_workspace_size(args)
    ws = torch.empty(n, device=gpu, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = ws.data_ptr(), n
    _lib.bwd(args, stream)
    torch.cuda.synchronize()
    ref = [t.clone() for t in grads]
    args.workspace, args.workspace_bytes = None, 0
    for rep in range(2):
        print(f"case bwd_noalloc varlen gqa call {rep}", flush=True)
        for t in grads:
            t.fill_(float("nan"))
        _lib.bwd_noalloc(args, stream)
        torch.cuda.synchronize()
        for name, got, want in zip(("dq", "dk", "dv"), grads, ref):
            assert torch.equal(got, want), f"call {rep} {name}"
