"""Pins the oracle's FP8 (e4m3) front before it is trusted as the checker of
the FP8 path. CPU only.

The reference rejects FP8 inputs (q_descale / k_descale / v_descale,
csrc/arch22/flash_attn_npu_v3/flash_api.cpp:154-156), so the semantics are
the v3 API's: scores scaled by softmax_scale * q_descale * k_descale, the
output by v_descale, descales of shape (batch, nheads_k). The byte decoding is
checked against torch's own float8_e4m3fn conversion (a separate
implementation) and the OCP specification's named values; the descale
placement against the float64 brute force with the factors applied by hand.
"""
import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests.golden import brute


def test_e4m3_decoding_matches_torch_for_every_byte():
    codes = np.arange(256, dtype=np.uint8)
    mine = orc.from_bits(orc.e4m3_to_bf16_bits(codes), orc.BF16)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert (np.isnan(mine) == nan).all()
    assert np.array_equal(mine[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # also tells -0 from +0


def test_e4m3_named_values():
    # OCP 8-bit FP spec, E4M3: max normal 448, min normal 2^-6, min subnormal 2^-9, NaN S.1111.111
    v = lambda c: float(orc.from_bits(orc.e4m3_to_bf16_bits(np.array([c], np.uint8)), orc.BF16)[0])
    assert v(0x7E) == 448.0 and v(0xFE) == -448.0
    assert v(0x08) == 2.0 ** -6 and v(0x01) == 2.0 ** -9 and v(0x07) == 7 * 2.0 ** -9
    assert v(0x38) == 1.0 and v(0xB8) == -1.0 and v(0x3C) == 1.5
    assert np.isnan(v(0x7F)) and np.isnan(v(0xFF))
    assert np.signbit(v(0x80)) and v(0x80) == 0.0


def _q8(rng, shape, amp):
    return torch.from_numpy((rng.standard_normal(shape) * amp).astype(np.float32)).to(torch.float8_e4m3fn) \
        .view(torch.uint8).numpy()


@pytest.mark.parametrize("causal,window,softcap", [(True, (-1, -1), 0.0), (False, (3, 2), 0.0), (False, (-1, -1), 5.0)])
def test_attention_fp8_descales_vs_fp64_brute_force(causal, window, softcap):
    rng = np.random.default_rng(7)
    B, Sq, Sk, H, Hk, D = 2, 5, 9, 4, 2, 16
    q8, k8, v8 = _q8(rng, (B, Sq, H, D), 2.0), _q8(rng, (B, Sk, Hk, D), 2.0), _q8(rng, (B, Sk, Hk, D), 3.0)
    qd = rng.uniform(0.2, 1.5, (B, Hk)).astype(np.float32)
    kd = rng.uniform(0.2, 1.5, (B, Hk)).astype(np.float32)
    vd = rng.uniform(0.2, 1.5, (B, Hk)).astype(np.float32)
    scale = D ** -0.5
    out, lse = orc.attention_fp8(q8, k8, v8, scale=scale, q_descale=qd, k_descale=kd, v_descale=vd, causal=causal,
                                 window=window, softcap=softcap)
    deq = lambda x: orc.from_bits(orc.e4m3_to_bf16_bits(x), orc.BF16).astype(np.float64)
    qf, kf, vf = deq(q8), deq(k8), deq(v8)
    g = H // Hk
    for b in range(B):
        for h in range(H):
            hk = h // g
            # descales applied by hand: q and k scaled before the product, v after the softmax
            o_ref, l_ref = brute.attention(qf[b, :, h:h + 1] * qd[b, hk], kf[b, :, hk:hk + 1] * kd[b, hk],
                                           vf[b, :, hk:hk + 1], scale, causal=causal, window=window, softcap=softcap)
            np.testing.assert_allclose(out[b, :, h], o_ref[:, 0] * vd[b, hk], atol=6e-2 * vd[b, hk], rtol=2e-2)
            np.testing.assert_allclose(lse[b, h], l_ref[0], rtol=1e-4, atol=1e-4)
