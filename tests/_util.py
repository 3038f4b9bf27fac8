"""Helpers shared by the tests: torch <-> oracle array conversion and checks."""
import numpy as np
import torch

from oracle import fa_oracle as orc

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}   # out max-abs vs the fp32 golden
LSE_RTOL = 1e-4
# Absolute floor of the LSE check, for |LSE| < 0.1 only (below that the 1e-4
# relative bound is under 1e-5): a row's LSE is formed from fp32 dot products
# of bf16 / fp16 values summed in a different order than the golden's, which
# leaves errors of a few 1e-7 in absolute terms whatever the LSE's size, so a
# purely relative bound cannot hold for an LSE near zero (e.g. one visible key
# with a score near 0).
LSE_ATOL = 1e-5


def odt(dtype):
    return orc.BF16 if dtype == torch.bfloat16 else orc.FP16


def bits(t):
    """16-bit tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a, dtype, device="cpu"):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype).to(device)


def randn(shape, dtype, gen, device):
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype).to(device)


# One ulp of the 16-bit type, relative (an upper bound: 2^-7 |x| for bf16,
# 2^-10 |x| for fp16). Both the kernel's output and the oracle's are rounded
# to that type from their fp32 values, each by up to half an ulp, so two fp32
# results within TOL of each other can come out one ulp apart when they
# straddle a rounding boundary. That matters for outputs of magnitude >= 2 in
# bf16 (ulp 2^-6 and more there): strongly local ALiBi, or inputs uniform in
# [-5, 5) as the reference's own tests draw them (one ulp is 2^-5 for outputs
# in [4, 8)). The bar stays tighter than the reference tests' own
# rtol = atol = 1e-2 (tests/test_flash_attn_npu_v3.py:517-521).
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def assert_close_out(out, ref_bits, dtype, tol=None, rtol=0.0):
    """|got - ref| <= tol + rtol * |ref| + one ulp of ref, elementwise; returns
    the largest |got - ref|. rtol is 0 for the north-star bar."""
    tol = TOL[dtype] if tol is None else tol
    got = out.detach().float().cpu().numpy()
    ref = orc.from_bits(ref_bits, odt(dtype)).reshape(got.shape)
    err = np.abs(got - ref)
    mx = float(np.nanmax(err)) if err.size else 0.0
    assert not np.isnan(got).any(), "NaN in output"
    excess = err - (tol + np.abs(ref) * (rtol + ULP[dtype]))
    assert not (excess > 0).any(), (f"out max-abs {mx:.3e} > {tol:.1e} + {rtol:.0e} relative + one ulp of the "
                                    f"reference value")
    return mx


def assert_close_lse(lse, ref, rtol=LSE_RTOL, atol=LSE_ATOL):
    """|got - ref| <= rtol * |ref| + atol per row (+inf rows must match);
    returns the largest relative error |got - ref| / |ref|."""
    got = lse.detach().float().cpu().numpy()
    ref = np.asarray(ref, dtype=np.float32).reshape(got.shape)
    inf_ref = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf_ref), "LSE +inf pattern differs"
    if (~inf_ref).any():
        g, r = got[~inf_ref].astype(np.float64), ref[~inf_ref].astype(np.float64)
        err = np.abs(g - r)
        bad = err > rtol * np.abs(r) + atol
        assert not bad.any(), (f"LSE off by {float(err[bad].max()):.3e} at |ref| = {float(np.abs(r[bad]).min()):.3e} "
                               f"(bound {rtol:.0e} relative + {atol:.0e})")
        return float((err / np.maximum(np.abs(r), 1e-30)).max())
    return 0.0
