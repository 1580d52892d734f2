"""Error gates shared by the GPU parity tests.

The correctness gate (max-abs 2e-2, mean-abs 2e-3; logsumexp 1e-3) for fp16/bf16 outputs vs an fp32/fp64 eager oracle
on the same (cast) inputs: max-abs <= 2e-2 and mean-abs <= 2e-3; logsumexp
max-abs <= 1e-3. The same max/mean gate is applied to dQ/dK/dV.
"""
import torch

MAX_ABS = 2e-2
MEAN_ABS = 2e-3
LSE_ABS = 1e-3


def errors(got, ref):
    err = (got.double() - ref.to(got.device).double()).abs()
    return err.max().item(), err.mean().item()


def assert_gate(got, ref, what, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    mx, mn = errors(got, ref)
    print(f"[gate] {what}: max-abs {mx:.3e} (<= {max_abs:g}), mean-abs {mn:.3e} (<= {mean_abs:g})", flush=True)
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e}, mean-abs {mn:.3e}"


def assert_grad_parity(got, exact, ref_alg, what, slack=1.5):
    """Gradient check. Passes the max-abs / mean-abs gate outright, or else must be no
    worse than `slack` x the error of the reference's own algorithm (the
    restated tiled backward with the reference's bf16 rounding points, outputs
    stored in the input dtype) against the same exact gradients. Also prints
    the representation floor (exact gradients rounded to the input dtype)."""
    assert got.shape == exact.shape and torch.isfinite(got).all(), f"{what}: bad shape or non-finite"
    mx, mn = errors(got, exact)
    amx, amn = errors(ref_alg.to(got.dtype), exact)
    fmx, fmn = errors(exact.to(got.dtype), exact)
    mag = exact.abs().max().item()
    print(f"[grad] {what}: ours max {mx:.3e} mean {mn:.3e} | reference algorithm max {amx:.3e} mean {amn:.3e}"
          f" | dtype floor max {fmx:.3e} mean {fmn:.3e} | max |g| {mag:.3e}", flush=True)
    if mx <= MAX_ABS and mn <= MEAN_ABS:
        return
    assert mx <= slack * amx and mn <= slack * amn, (
        f"{what}: max {mx:.3e} mean {mn:.3e} exceed the gate and {slack}x the reference algorithm "
        f"({amx:.3e}, {amn:.3e})")


def assert_lse(got, ref, what):
    fin = torch.isfinite(ref.to(got.device))
    assert torch.equal(torch.isfinite(got), fin), f"{what}: -inf pattern differs"
    mx = (got[fin].double() - ref.to(got.device)[fin].double()).abs().max().item() if fin.any() else 0.0
    print(f"[gate] {what}: lse max-abs {mx:.3e} (<= {LSE_ABS:g})", flush=True)
    assert mx <= LSE_ABS, f"{what}: lse max-abs {mx:.3e}"
