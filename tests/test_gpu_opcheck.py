"""torch.library.opcheck on every fa_mi355x operator: the schemas (mutation
and aliasing declarations: the kvcache ops write k_cache / v_cache,
fwd_combine_out writes out), the fake (meta) implementations against the real
outputs (shapes, dtypes, FP8 giving bf16), and tracing under AOT dispatch."""
import pytest
import torch

from fa_mi355x import ops
from tests._util import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
UTILS = ("test_schema", "test_autograd_registration", "test_faketensor", "test_aot_dispatch_dynamic")


# torch implements no arithmetic on float8_e4m3fn tensors, which the schema
# and AOT checks perform on the op's inputs; FP8 calls get the fake-tensor
# check, which compares the fake's shapes and dtypes (bf16 out) with the op's
UTILS_FP8 = ("test_faketensor",)


def _chk(op, args, kwargs=None):
    fp8 = any(isinstance(x, torch.Tensor) and x.dtype == torch.float8_e4m3fn for x in args)
    torch.library.opcheck(op, args, kwargs or {}, test_utils=UTILS_FP8 if fp8 else UTILS)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float8_e4m3fn])
def test_opcheck_fwd_kvcache(dt):
    print(f"case opcheck fwd_kvcache {dt}", flush=True)
    g = torch.Generator().manual_seed(800)
    mk = lambda *s: randn(s, torch.float32, g, DEV).to(dt)
    q, kc, vc = mk(2, 1, 8, 128), mk(2, 64, 2, 128), mk(2, 64, 2, 128)
    kn, vn = mk(2, 1, 2, 128), mk(2, 1, 2, 128)
    sl = torch.tensor([10, 40], dtype=torch.int32, device=DEV)
    _chk(ops.fwd_kvcache, (q, kc, vc, kn, vn, sl, None, None, None, None, None, None, 0.088, True, -1, 0, 0.0, True,
                           0))
    _chk(ops.fwd_kvcache_v3, (q, kc, vc, kn, vn, sl, None, None, None, None, None, None, None, None, 0, None, 0.088,
                              True, -1, 0, 0, 0.0, True, 0))


def test_opcheck_fwd_and_varlen():
    print("case opcheck fwd / varlen_fwd", flush=True)
    g = torch.Generator().manual_seed(801)
    q, k, v = randn((2, 40, 8, 128), torch.float16, g, DEV), randn((2, 50, 2, 128), torch.float16, g, DEV), \
        randn((2, 50, 2, 128), torch.float16, g, DEV)
    _chk(ops.fwd, (q, k, v, None, 0.0, 0.088, True, -1, 0, 0.0))
    _chk(ops.fwd, (q, k, v, None, 0.0, 0.088, False, 16, 4, 20.0), dict(attention_chunk=32, num_splits=2))
    cu = torch.tensor([0, 30, 80], dtype=torch.int32, device=DEV)
    qv, kv = randn((80, 8, 128), torch.float16, g, DEV), randn((80, 2, 128), torch.float16, g, DEV)
    _chk(ops.varlen_fwd, (qv, kv, kv, cu, cu, None, None, None, 50, 50, 0.0, 0.088, True, -1, 0, 0.0))


def test_opcheck_fwd_fp8():
    print("case opcheck fwd fp8", flush=True)
    g = torch.Generator().manual_seed(802)
    mk = lambda *s: randn(s, torch.float32, g, DEV).to(torch.float8_e4m3fn)
    q, k = mk(2, 40, 8, 128), mk(2, 50, 2, 128)
    ds = torch.full((2, 2), 0.5, device=DEV)
    _chk(ops.fwd, (q, k, k, None, 0.0, 0.088, True, -1, 0, 0.0), dict(q_descale=ds, k_descale=ds, v_descale=ds))


def test_opcheck_combine():
    print("case opcheck combine", flush=True)
    g = torch.Generator().manual_seed(803)
    op = torch.randn((3, 2, 5, 4, 128), generator=g).to(DEV)
    lp = torch.randn((3, 2, 5, 4), generator=g).to(DEV)
    _chk(ops.fwd_combine, (op, lp, torch.bfloat16))
    _chk(ops.fwd_combine_out, (op, lp, torch.empty((2, 5, 4, 128), device=DEV)))


def test_opcheck_bwd():
    print("case opcheck bwd / varlen_bwd", flush=True)
    g = torch.Generator().manual_seed(804)
    q, k, v = (randn(s, torch.bfloat16, g, DEV) for s in ((2, 40, 8, 64), (2, 50, 2, 64), (2, 50, 2, 64)))
    out, lse = ops.fwd(q, k, v, None, 0.0, 0.125, True, -1, 0, 0.0)
    do = randn((2, 40, 8, 64), torch.bfloat16, g, DEV)
    _chk(ops.bwd, (do, q, k, v, out, lse, None, 0.0, 0.125, True, -1, 0, 0.0, False))
    cu = torch.tensor([0, 30, 80], dtype=torch.int32, device=DEV)
    qv, kv = randn((80, 8, 64), torch.bfloat16, g, DEV), randn((80, 2, 64), torch.bfloat16, g, DEV)
    ov, lv = ops.varlen_fwd(qv, kv, kv, cu, cu, None, None, None, 50, 50, 0.0, 0.125, True, -1, 0, 0.0)
    _chk(ops.varlen_bwd, (randn((80, 8, 64), torch.bfloat16, g, DEV), qv, kv, kv, ov, lv, cu, cu, None, 50, 50, 0.0,
                          0.125, True, -1, 0, 0.0, False))


def test_opcheck_fwd_with_metadata_workspace():
    """The workspace a scheduler_metadata buffer brings in is written by the
    kernels (split partials, the plan), so the schemas declare it mutable."""
    from flash_attn_npu_v3 import interface as v3
    print("case opcheck fwd / varlen_fwd / fwd_kvcache_v3 with a metadata workspace", flush=True)
    g = torch.Generator().manual_seed(805)
    q, k, v = randn((2, 40, 8, 128), torch.float16, g, DEV), randn((2, 50, 2, 128), torch.float16, g, DEV), \
        randn((2, 50, 2, 128), torch.float16, g, DEV)
    sl = torch.tensor([50, 50], dtype=torch.int32, device=DEV)
    md = v3.get_scheduler_metadata(2, 40, 50, 8, 2, 128, sl, qkv_dtype=torch.float16, causal=True, num_splits=2)
    ws = md[256:].clone()
    _chk(ops.fwd, (q, k, v, None, 0.0, 0.088, True, -1, 0, 0.0), dict(num_splits=2, workspace=ws))
    cu = torch.tensor([0, 30, 80], dtype=torch.int32, device=DEV)
    qv, kv = randn((80, 8, 128), torch.float16, g, DEV), randn((80, 2, 128), torch.float16, g, DEV)
    _chk(ops.varlen_fwd, (qv, kv, kv, cu, cu, None, None, None, 50, 50, 0.0, 0.088, True, -1, 0, 0.0),
         dict(num_splits=2, workspace=ws))
    kc, vc = randn((2, 64, 2, 128), torch.float16, g, DEV), randn((2, 64, 2, 128), torch.float16, g, DEV)
    q1 = randn((2, 1, 8, 128), torch.float16, g, DEV)
    # the call's split count is the metadata's (2), as the v3 interface passes it
    _chk(ops.fwd_kvcache_v3, (q1, kc, vc, None, None, sl, None, None, None, None, None, None, None, None, 0, None,
                              0.088, True, -1, 0, 0, 0.0, True, 2), dict(workspace=ws))
