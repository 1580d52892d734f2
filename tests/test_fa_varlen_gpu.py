"""GPU parity of the packed varlen GQA forward (config 5: chunked prefill over
a cached prefix) against oracle.attention.varlen_reference."""
import pytest
import torch

from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward
from oracle.attention import attention_reference, varlen_reference
from lightserve_amd.workloads import make_varlen_inputs
from tests.gates import assert_gate, assert_lse

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("causal", [True, False])
def test_varlen_small(gpu, dtype, causal):
    inp = make_varlen_inputs(device=gpu, batch=3, chunk=70, prefix=(100, 300), heads=(8, 2), D=128)
    q, k, v = (inp[n].to(dtype) for n in ("q", "k", "v"))
    o, lse = flash_attention_varlen_forward(q, k, v, inp["cu_seqlens_q"], inp["cu_seqlens_k"],
                                            inp["max_seqlen_q"], inp["max_seqlen_k"], causal=causal)
    o_ref, lse_ref = varlen_reference(q.cpu(), k.cpu(), v.cpu(), inp["cu_seqlens_q"].cpu(),
                                      inp["cu_seqlens_k"].cpu(), causal=causal)
    if dtype == torch.float32:
        torch.testing.assert_close(o.cpu().double(), o_ref, atol=1e-3, rtol=1e-3)
    else:
        assert_gate(o.cpu(), o_ref, f"varlen {dtype} causal={causal}")
    assert_lse(lse.cpu(), lse_ref, "varlen")


def test_varlen_ragged_and_empty_sequences(gpu):
    """Sequences of length 0, 1 and not a multiple of the tile, including a
    chunk longer than its key range (rows that see no key: o=0, lse=-inf)."""
    torch.manual_seed(3)
    lens_q = [5, 0, 1, 130, 64]
    lens_k = [17, 3, 1, 200, 40]
    cu_q = torch.tensor([0] + list(torch.tensor(lens_q).cumsum(0)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(lens_k).cumsum(0)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), 4, 64, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(int(cu_k[-1]), 1, 64, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(int(cu_k[-1]), 1, 64, device=gpu, dtype=torch.bfloat16)
    o, lse = flash_attention_varlen_forward(q, k, v, cu_q.to(gpu), cu_k.to(gpu), max(lens_q), max(lens_k))
    o_ref, lse_ref = varlen_reference(q.cpu(), k.cpu(), v.cpu(), cu_q, cu_k, causal=True)
    assert_gate(o.cpu(), o_ref, "ragged varlen")
    assert_lse(lse.cpu(), lse_ref, "ragged varlen")


def test_varlen_config5_full_size(gpu):
    """Config 5 at full size (B=8, 32 q heads over 8 kv heads, 512-token
    chunks after 1024-8192-token prefixes); oracle in fp32 on the GPU."""
    inp = make_varlen_inputs(device=gpu)
    q, k, v = inp["q"], inp["k"], inp["v"]
    cu_q, cu_k = inp["cu_seqlens_q"], inp["cu_seqlens_k"]
    o, lse = flash_attention_varlen_forward(q, k, v, cu_q, cu_k, inp["max_seqlen_q"], inp["max_seqlen_k"])
    cq, ck = cu_q.tolist(), cu_k.tolist()
    group = q.shape[1] // k.shape[1]
    for b in range(len(cq) - 1):
        qb = q[cq[b]:cq[b + 1]].transpose(0, 1)
        kb = k[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(group, 0)
        vb = v[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(group, 0)
        ob, lb = attention_reference(qb, kb, vb, True, dtype=torch.float32)
        assert_gate(o[cq[b]:cq[b + 1]].transpose(0, 1), ob, f"config 5 seq {b}")
        assert_lse(lse[:, cq[b]:cq[b + 1]], lb, f"config 5 seq {b}")
