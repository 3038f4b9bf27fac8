"""Helpers shared by the tests: torch <-> oracle array conversion and checks."""
import numpy as np
import torch

from oracle import fa_oracle as orc

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}   # out max-abs vs the fp32 golden
LSE_RTOL = 1e-4


def odt(dtype):
    return orc.BF16 if dtype == torch.bfloat16 else orc.FP16


def bits(t):
    """16-bit tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a, dtype, device="cpu"):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype).to(device)


def randn(shape, dtype, gen, device):
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype).to(device)


# Half an ulp of the 16-bit type, relative: the oracle's output is itself
# rounded to that type, so a kernel result within TOL of the exact value can
# round to the neighbouring 16-bit value (one ulp away from the oracle's) when
# the two fp32 values straddle a rounding boundary. That matters for outputs of
# magnitude >= 2 in bf16 (ulp 2^-6 there), e.g. with strongly local ALiBi.
HALF_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def assert_close_out(out, ref_bits, dtype, tol=None):
    tol = TOL[dtype] if tol is None else tol
    got = out.detach().float().cpu().numpy()
    ref = orc.from_bits(ref_bits, odt(dtype)).reshape(got.shape)
    err = np.abs(got - ref)
    mx = float(np.nanmax(err)) if err.size else 0.0
    assert not np.isnan(got).any(), "NaN in output"
    excess = err - (tol + np.abs(ref) * HALF_ULP[dtype])
    assert not (excess > 0).any(), f"out max-abs {mx:.3e} > {tol:.1e} + half an ulp of the reference value"
    return mx


def assert_close_lse(lse, ref, rtol=LSE_RTOL):
    got = lse.detach().float().cpu().numpy()
    ref = np.asarray(ref, dtype=np.float32).reshape(got.shape)
    inf_ref = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf_ref), "LSE +inf pattern differs"
    if (~inf_ref).any():
        g, r = got[~inf_ref], ref[~inf_ref]
        rel = np.abs(g - r) / np.maximum(np.abs(r), 1.0)
        assert float(rel.max()) <= rtol, f"LSE rel {float(rel.max()):.3e} > {rtol:.0e}"
        return float(rel.max())
    return 0.0
