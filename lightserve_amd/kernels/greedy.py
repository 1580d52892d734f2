"""Greedy next token of a decode step on MI355X.

    greedy_next_token(logits, out=None, seq_lens=None) -> tokens (int64)

tokens[r] = logits[r].argmax() with torch's comparison (NaN beats every
number, ties go to the lower index), as the reference takes it after each
step (model/cuda_graph_decode.py:114, :145); seq_lens, when given, is advanced
by one in the same launch (lsfa_greedy).
"""
import torch

from .. import _lib


def greedy_next_token(logits: torch.Tensor, out: torch.Tensor = None, seq_lens: torch.Tensor = None):
    assert logits.ndim == 2 and logits.is_cuda and logits.stride(1) == 1, "logits [rows, cols] on the GPU"
    assert logits.dtype in _lib.TORCH_TO_LSFA, f"unsupported dtype {logits.dtype}"
    rows, cols = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    assert out.dtype == torch.int64 and out.shape == (rows,) and out.is_contiguous(), "out: int64 [rows]"
    if seq_lens is not None:
        assert seq_lens.dtype == torch.int32 and seq_lens.shape == (rows,) and seq_lens.is_contiguous(), (
            "seq_lens: int32 [rows]")
    if rows == 0:
        return out
    args = _lib.GreedyArgs(logits=logits.data_ptr(), tokens=out.data_ptr(),
                           seq_lens=seq_lens.data_ptr() if seq_lens is not None else None,
                           logits_stride=logits.stride(0), dtype=_lib.TORCH_TO_LSFA[logits.dtype], rows=rows,
                           cols=cols)
    with torch.cuda.device(logits.device):
        _lib.greedy(args, _lib.current_stream(logits.device))
    return out
