"""GPU parity of the greedy next-token kernel (lsfa_greedy) with torch's
argmax, which the reference takes after each decode step
(model/cuda_graph_decode.py:114, :145): vocabulary-sized rows in all three
dtypes, the 16-byte and the scalar scan, ties and NaNs (torch's rule: NaN
beats every number, the lower index wins a tie), rows of -inf, and the
sequence-length update."""
import pytest
import torch

from lightserve_amd.kernels.greedy import greedy_next_token

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,cols", [(1, 128256), (8, 32000), (3, 4097), (5, 1), (2, 8)])
def test_greedy_matches_torch_argmax(rows, cols, dtype):
    print(f"case greedy rows={rows} cols={cols} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows * cols)
    x = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    assert torch.equal(greedy_next_token(x), x.argmax(dim=-1))
    # ties: the maximum repeated at several columns
    x2 = torch.round(torch.randn(rows, cols, device="cuda", generator=g) * 2).to(dtype)
    assert torch.equal(greedy_next_token(x2), x2.argmax(dim=-1))


def test_greedy_nan_inf_and_strided_rows():
    print("case greedy nan/inf/strided", flush=True)
    x = torch.randn(6, 1000, device="cuda", dtype=torch.bfloat16)
    x[1, 700] = float("nan")
    x[2, 10] = float("nan")
    x[2, 5] = float("nan")
    x[3] = float("-inf")
    x[4, 999] = float("inf")
    x[5, 3] = float("inf")
    x[5, 4] = float("inf")
    ref = x.float().argmax(dim=-1)
    assert torch.equal(greedy_next_token(x), ref)
    big = torch.randn(4, 3000, device="cuda", dtype=torch.bfloat16)
    for view in (big[:, 8:2008], big[:, 3:2003]):   # aligned (16-byte scan) and misaligned (scalar scan)
        assert torch.equal(greedy_next_token(view), view.argmax(dim=-1))


def test_greedy_advances_seq_lens_in_place():
    print("case greedy seq_lens", flush=True)
    x = torch.randn(4, 5000, device="cuda", dtype=torch.bfloat16)
    out = torch.full((4,), -1, dtype=torch.int64, device="cuda")
    lens = torch.tensor([0, 7, 100, 3], dtype=torch.int32, device="cuda")
    res = greedy_next_token(x, out=out, seq_lens=lens)
    assert res.data_ptr() == out.data_ptr() and torch.equal(out, x.argmax(dim=-1))
    assert lens.tolist() == [1, 8, 101, 4]
