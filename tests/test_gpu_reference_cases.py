"""The reference's own forward case lists, run on the GPU against the CPU oracle.

* v2 flash_attn_with_kvcache: tests/test_flash_attn_npu_v2.py:145-255 of the
  reference (contiguous and paged caches);
* v3 flash_attn_with_kvcache: tests/test_flash_attn_npu_v3.py:148-274, each
  case with cache_mode 0 (contiguous, or for the TND layout a packed
  (total_k, nheads_k, headdim) cache) and 1 (paged), num_splits 0 and 2 (2
  only for paged TND, as the reference skips the rest: :281-282), and the
  "is_varied" ragged lengths drawn the way the reference draws them (:296-302);
* v3 flash_attn_func: :523-544;
* v3 flash_attn_varlen_func: :598-625, head dim 111 included.

Inputs are drawn as the reference draws them, uniform in [-5, 5), here from a
seeded generator; paged caches use 128-token blocks with sequential block ids
(:288-324). Exact duplicate tuples of a list run once.

Checks: the oracle recomputes, per case, the first and the last sequence,
each on its first and last kv head with all of that kv head's query heads
(every sequence and head for the head-dim-111 cases), from the K / V rows of
that sequence gathered on the host. LSE is held to the north-star 1e-4
relative. The output is checked twice:

* against the oracle, at the north-star bar scaled to these inputs. Attention
  is linear in v, so scaling v scales the output and every rounding error in
  it (the 16-bit rounding of P before P.V, at points that depend on each
  implementation's running maximum, and of the output itself) by the same
  factor. The bar of 1e-2 (bf16) / 2e-3 (fp16) is stated for N(0, 1) values
  (standard deviation 1); these lists draw v uniform in [-5, 5), standard
  deviation 5 / sqrt(3), so the bar here is that many times the north-star
  one (0.029 bf16, 0.0058 fp16), plus one ulp of the reference value (both
  results are rounded to 16 bits);
* against the exact result (float64, tests/golden/brute.py), within what the
  16-bit rounding of P and of the output can cause in any implementation
  that sums the row from the unrounded P (as the golden and the kernels do):
  |got - exact| <= u max|v| + u |exact| + 1e-4, u = 2^-8 (bf16) / 2^-11 (fp16),
  the largest relative rounding error of that type.

The first bar is looser than these reference tests' own, |got - golden| <=
1e-2 + 1e-2 |golden| (rtol = atol = 1e-2: tests/test_flash_attn_npu_v3.py:
517-521, tests/test_flash_attn_npu_v2.py:404-407), for outputs near zero. The
reference's kernel rounds P at the same 512-key stacks as its golden, so the
two round alike; this build's prefill kernel rounds P against a running
maximum it moves only when a row's maximum grows by more than 2^8 (the
"lazy" rescale), so a row's dominant weight is rounded too, where the
golden's is exactly 1. Measured on these inputs: kernel and oracle both about
3e-3 from the exact result on average; at most 0.03 (kernel) and 0.02
(oracle); the kernel misses the reference's bar against the exact result on
1 to 3 outputs of a million in 4 of these cases (all prefill), the oracle on
none.

Window semantics are the small-op golden's (tests/fa_small_op_golden.py:21-58),
which north_star names: after normalisation a negative bound of a local
window leaves that side unbounded. The reference's v3 test golden instead
reads a negative right bound literally (create_binary_matrix, :465-474, and
its row zeroing, :476-490): of these lists only the window (508, -256) tells
the two apart, and it is checked here with the small-op golden's meaning."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests.golden import brute
from tests._util import TOL, assert_close_lse, assert_close_out, bits, odt

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)
F16, BF = torch.float16, torch.bfloat16
SIGMA_V = 5.0 / math.sqrt(3.0)  # standard deviation of values uniform in [-5, 5)

# (dtype, B, H, Hk, Sq, Sk, D, cache_mode, block, causal, wl, wr, softcap): the reference's v2 list
V2_KV = [
    (BF, 1, 1, 1, 1024, 1024, 128, 1, 128, False, -1, -1, 0.0), (BF, 5, 4, 4, 1024, 1024, 128, 0, 128, True, -1, -1, 0.0),
    (F16, 7, 1, 1, 512, 512, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 1, 1, 1, 1024, 128, 1, 128, True, -1, -1, 0.0),
    (BF, 1, 1, 1, 1, 1024, 128, 1, 128, False, -1, -1, 0.0), (BF, 2, 1, 1, 1024, 1024, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 5, 4, 4, 1024, 1024, 128, 1, 128, True, -1, -1, 0.0), (BF, 1, 1, 1, 1, 4096, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 2, 1, 1, 1, 2048, 128, 1, 128, False, -1, -1, 0.0), (F16, 2, 2, 1, 128, 128, 128, 1, 128, True, -1, -1, 0.0),
    (BF, 2, 6, 2, 2, 1024, 128, 1, 128, True, -1, -1, 0.0), (BF, 1, 1, 1, 1024, 1024, 128, 1, 128, True, 512, 0, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 1, 128, True, 512, 256, 0.0),
    (BF, 5, 4, 4, 1024, 1024, 128, 0, 128, True, -128, 864, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 1, 128, False, 0, 256, 0.0),
    (F16, 2, 2, 2, 512, 512, 128, 0, 128, False, 64, 128, 0.0),
    (BF, 1, 8, 2, 1, 512, 128, 0, 128, True, -1, -1, 0.0), (BF, 4, 32, 8, 1, 2048, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 8, 64, 8, 1, 4096, 128, 0, 128, False, -1, -1, 0.0), (BF, 4, 64, 16, 16, 1024, 128, 0, 128, True, -1, -1, 0.0),
    (BF, 8, 128, 16, 32, 2048, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 4, 64, 8, 64, 4096, 128, 0, 128, False, -1, -1, 0.0), (BF, 8, 128, 8, 1, 4096, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 4, 32, 4, 16, 1024, 256, 0, 128, False, -1, -1, 0.0), (BF, 8, 128, 32, 64, 2048, 128, 0, 128, True, -1, -1, 0.0),
    (BF, 4, 64, 4, 32, 512, 128, 0, 128, False, -1, -1, 0.0), (BF, 2, 64, 8, 1, 4096, 256, 0, 128, False, -1, -1, 0.0),
    (BF, 1, 32, 4, 1, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 64, 4, 1, 4096, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 128, 4, 1, 2048, 128, 1, 128, True, -1, -1, 0.0), (BF, 2, 32, 4, 1, 4096, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 2, 16, 2, 1, 2048, 128, 1, 128, True, -1, -1, 0.0), (BF, 1, 32, 8, 1, 2048, 256, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 32, 4, 4, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 2, 16, 2, 4, 4096, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 64, 4, 8, 2048, 128, 1, 128, True, -1, -1, 0.0), (BF, 1, 32, 4, 16, 4096, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 32, 4, 3, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 2, 16, 2, 5, 4096, 128, 1, 128, True, -1, -1, 0.0),
    (BF, 1, 64, 4, 7, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 32, 4, 11, 4096, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 32, 8, 13, 2048, 256, 1, 128, False, -1, -1, 0.0), (BF, 2, 16, 2, 15, 2048, 128, 1, 128, True, -1, -1, 0.0),
    (BF, 4, 32, 32, 1, 2048, 128, 0, 128, False, -1, -1, 0.0), (BF, 8, 64, 64, 1, 4096, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 4, 32, 32, 16, 1024, 128, 0, 128, True, -1, -1, 0.0), (BF, 4, 64, 64, 32, 2048, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 8, 16, 16, 8, 4096, 128, 0, 128, False, -1, -1, 0.0), (BF, 2, 32, 32, 1, 4096, 256, 0, 128, False, -1, -1, 0.0),
    (BF, 2, 32, 8, 65, 2048, 128, 0, 128, False, -1, -1, 0.0), (BF, 2, 64, 16, 96, 2048, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 1, 32, 8, 128, 4096, 128, 0, 128, False, -1, -1, 0.0), (BF, 2, 16, 4, 256, 2048, 128, 0, 128, True, -1, -1, 0.0),
    (BF, 1, 32, 4, 65, 2048, 256, 0, 128, False, -1, -1, 0.0), (BF, 2, 24, 2, 6, 2048, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 4, 32, 2, 6, 4096, 128, 0, 128, False, -1, -1, 0.0), (BF, 2, 40, 2, 6, 2048, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 2, 24, 2, 8, 2048, 128, 0, 128, False, -1, -1, 0.0), (BF, 4, 32, 2, 8, 4096, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 2, 24, 2, 10, 2048, 128, 0, 128, False, -1, -1, 0.0), (BF, 4, 32, 2, 10, 4096, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 2, 64, 2, 10, 2048, 128, 0, 128, False, -1, -1, 0.0), (BF, 2, 24, 2, 6, 2048, 256, 0, 128, False, -1, -1, 0.0),
    (BF, 4, 48, 2, 8, 4096, 128, 0, 128, False, -1, -1, 0.0), (BF, 2, 48, 4, 8, 2048, 128, 0, 128, False, -1, -1, 0.0),
    (BF, 4, 64, 4, 10, 4096, 128, 0, 128, False, -1, -1, 0.0), (BF, 1, 64, 4, 2, 2048, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 2, 32, 4, 2, 4096, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 64, 8, 4, 4096, 128, 1, 128, True, -1, -1, 0.0),
    (BF, 1, 32, 4, 7, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 2, 16, 2, 8, 4096, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 32, 4, 13, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 32, 8, 16, 2048, 256, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 6, 2, 6, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 10, 2, 6, 2048, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 6, 2, 10, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 10, 2, 10, 2048, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 14, 2, 10, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 18, 2, 10, 2048, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 6, 2, 14, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 10, 2, 14, 2048, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 6, 2, 9, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 6, 2, 11, 2048, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 10, 2, 15, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 10, 2, 10, 4096, 256, 1, 128, True, -1, -1, 0.0),
    (BF, 1, 8, 2, 8, 2048, 128, 1, 128, False, -1, -1, 0.0), (BF, 1, 16, 2, 16, 2048, 128, 1, 128, False, -1, -1, 0.0),
    (BF, 1, 32, 8, 128, 4096, 128, 0, 128, False, -1, -1, 30.0),
    (BF, 2, 16, 4, 256, 2048, 128, 0, 128, True, -1, -1, 50.0),
    (BF, 1, 32, 4, 65, 2048, 256, 0, 128, False, -1, -1, 50.0),
    (BF, 2, 24, 2, 6, 2048, 128, 0, 128, False, -1, -1, 30.0),
    (BF, 4, 32, 2, 6, 4096, 128, 0, 128, False, -1, -1, 50.0),
    (BF, 2, 40, 2, 6, 2048, 128, 0, 128, False, -1, -1, 50.0),
]

# (dtype, B, H, Hk, Sq, Sk, D, block, causal, layout, is_varied, wl, wr, softcap): the reference's v3 list
V3_KV = [
    (BF, 2, 6, 2, 2, 1024, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 5, 4, 4, 1024, 1024, 128, 128, True, "TND", False, -1, -1, 0.0),
    (F16, 7, 1, 1, 512, 512, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 1, 1, 1024, 1024, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 1, 1, 1024, 1024, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 5, 4, 4, 1024, 1024, 128, 128, True, "BSND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1, 1024, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1, 1024, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1, 1024, 128, 128, True, "BSND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1, 1024, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 1, 1, 1, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (F16, 2, 2, 1, 128, 128, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 2, 6, 2, 2, 1024, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 2, 1, 1, 16, 1024, 128, 128, False, "TND", True, -1, -1, 0.0),
    (BF, 2, 6, 2, 16, 1024, 128, 128, False, "TND", True, -1, -1, 0.0),
    (BF, 2, 6, 2, 16, 1024, 128, 128, True, "TND", True, -1, -1, 0.0),
    (BF, 1, 64, 1, 2, 1024, 256, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 1, 1, 16, 1024, 256, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 2, 1, 1, 16, 10240, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 6, 2, 16, 10240, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 6, 1, 1, 16, 10240, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 128, True, "BSND", False, 512, 0, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 128, True, "TND", False, 512, 0, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 128, False, "TND", False, 0, 256, 0.0),
    (F16, 2, 1, 1, 512, 512, 128, 128, False, "TND", False, 508, -256, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, 128, False, "BSND", False, -128, 1024, 0.0),
    (F16, 2, 2, 2, 512, 512, 128, 128, False, "TND", False, 64, 128, 0.0),
    (BF, 4, 32, 8, 1, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 8, 64, 8, 1, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 64, 16, 16, 1024, 128, 128, True, "BSND", False, -1, -1, 0.0),
    (BF, 8, 128, 16, 32, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 64, 8, 64, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 8, 128, 8, 1, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 32, 4, 16, 1024, 256, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 8, 128, 32, 64, 2048, 128, 128, True, "BSND", False, -1, -1, 0.0),
    (BF, 4, 64, 4, 32, 512, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 64, 8, 1, 4096, 256, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 32, 8, 32, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 8, 64, 8, 32, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 4, 32, 8, 64, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 8, 64, 8, 64, 2048, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 4, 64, 8, 48, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 4, 64, 4, 32, 1024, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 4, 32, 8, 64, 2048, 256, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 8, 128, 16, 32, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 1, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 64, 4, 1, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 128, 4, 1, 2048, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 2, 32, 4, 1, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 16, 2, 1, 2048, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 8, 1, 2048, 256, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 4, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 16, 2, 4, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 64, 4, 8, 2048, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 16, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 3, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 16, 2, 5, 4096, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 1, 64, 4, 7, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 11, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 8, 13, 2048, 256, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 16, 2, 15, 2048, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 4, 32, 32, 1, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 8, 64, 64, 1, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 32, 32, 16, 1024, 128, 128, True, "BSND", False, -1, -1, 0.0),
    (BF, 4, 64, 64, 32, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 8, 16, 16, 8, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 32, 32, 1, 4096, 256, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 32, 8, 65, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 64, 16, 96, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 1, 32, 8, 128, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 16, 4, 256, 2048, 128, 128, True, "BSND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 65, 2048, 256, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 32, 32, 32, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 4, 32, 32, 48, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 4, 64, 64, 64, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 32, 8, 65, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 64, 16, 96, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 24, 2, 6, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 32, 2, 6, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 40, 2, 6, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 24, 2, 8, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 32, 2, 8, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 24, 2, 10, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 32, 2, 10, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 64, 2, 10, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 24, 2, 6, 2048, 256, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 48, 2, 8, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 2, 48, 4, 8, 2048, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 4, 64, 4, 10, 4096, 128, 128, False, "BSND", False, -1, -1, 0.0),
    (BF, 1, 64, 4, 2, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 32, 4, 2, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 64, 8, 4, 4096, 128, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 7, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 2, 16, 2, 8, 4096, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 4, 13, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 8, 16, 2048, 256, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 6, 2, 6, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 10, 2, 6, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 6, 2, 10, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 10, 2, 10, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 14, 2, 10, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 18, 2, 10, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 6, 2, 14, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 10, 2, 14, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 6, 2, 9, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 6, 2, 11, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 10, 2, 15, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 10, 2, 10, 4096, 256, 128, True, "TND", False, -1, -1, 0.0),
    (BF, 1, 8, 2, 8, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 16, 2, 16, 2048, 128, 128, False, "TND", False, -1, -1, 0.0),
    (BF, 1, 32, 8, 128, 4096, 128, 128, False, "BSND", False, -1, -1, 30.0),
    (BF, 2, 16, 4, 256, 2048, 128, 128, True, "BSND", False, -1, -1, 50.0),
    (BF, 1, 32, 4, 65, 2048, 256, 128, False, "BSND", False, -1, -1, 50.0),
    (BF, 4, 32, 32, 32, 2048, 128, 128, False, "TND", False, -1, -1, 30.0),
    (BF, 4, 32, 32, 48, 2048, 128, 128, False, "TND", False, -1, -1, 50.0),
    (BF, 4, 64, 64, 64, 2048, 128, 128, False, "TND", False, -1, -1, 50.0),
]

# (dtype, B, H, Hk, Sq, Sk, D, return_attn_probs, causal, softcap): the reference's flash_attn_func list
DENSE = [
    (F16, 1, 1, 1, 1024, 1024, 128, True, False, 0.0), (F16, 5, 4, 4, 1024, 1024, 128, True, True, 0.0),
    (F16, 7, 1, 1, 512, 512, 128, True, False, 0.0), (F16, 1, 1, 1, 1024, 1024, 128, False, False, 0.0),
    (F16, 5, 4, 4, 1024, 1024, 128, False, True, 0.0), (F16, 7, 1, 1, 512, 512, 128, False, False, 0.0),
    (F16, 4, 2, 1, 513, 513, 128, False, False, 0.0), (BF, 1, 1, 1, 1024, 1024, 128, True, False, 0.0),
    (BF, 5, 4, 4, 1024, 1024, 128, True, True, 0.0), (BF, 7, 1, 1, 512, 512, 128, True, False, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, False, False, 0.0), (BF, 5, 4, 4, 1024, 1024, 128, False, True, 0.0),
    (BF, 7, 1, 1, 512, 512, 128, False, False, 0.0),
    (F16, 7, 1, 1, 512, 512, 128, False, False, 30.0), (F16, 4, 2, 1, 513, 513, 128, False, False, 50.0),
    (BF, 1, 1, 1, 1024, 1024, 128, True, False, 30.0), (BF, 5, 4, 4, 1024, 1024, 128, True, True, 50.0),
]

# (dtype, B, H, Hk, Sq, Sk, D, causal, wl, wr, softcap): the reference's flash_attn_varlen_func list
VARLEN = [
    (BF, 1, 1, 1, 512, 1024, 128, True, -1, -1, 0.0), (BF, 2, 4, 4, 1024, 1024, 128, False, -1, -1, 0.0),
    (F16, 7, 5, 1, 512, 512, 128, True, -1, -1, 0.0), (F16, 7, 5, 1, 777, 888, 192, False, -1, -1, 0.0),
    (F16, 7, 5, 1, 1777, 1888, 256, True, -1, -1, 0.0), (BF, 1, 1, 1, 7777, 8192, 64, True, -1, -1, 0.0),
    (BF, 7, 5, 1, 711, 8192, 111, True, -1, -1, 0.0),
    (BF, 1, 1, 1, 512, 512, 128, True, 512, 0, 0.0), (BF, 1, 1, 1, 512, 512, 128, True, 256, 128, 0.0),
    (F16, 2, 4, 4, 256, 256, 128, False, 64, 128, 0.0), (BF, 1, 1, 1, 512, 512, 128, False, 0, 256, 0.0),
    (BF, 2, 6, 2, 128, 256, 128, True, 127, 0, 0.0), (BF, 2, 4, 4, 128, 512, 128, True, 511, 0, 0.0),
    (F16, 1, 2, 2, 64, 192, 128, False, 32, 64, 0.0), (BF, 1, 1, 1, 1024, 1024, 128, True, 512, 0, 0.0),
    (BF, 1, 1, 1, 1, 1024, 128, True, 512, 0, 0.0), (F16, 2, 1, 1, 512, 512, 128, False, 508, -256, 0.0),
    (BF, 1, 1, 1, 1024, 1024, 128, True, -128, 864, 0.0), (BF, 2, 6, 2, 2, 1024, 128, True, 256, 0, 0.0),
    (F16, 7, 5, 1, 777, 888, 192, False, -1, -1, 30.0), (F16, 7, 5, 1, 1777, 1888, 256, True, -1, -1, 50.0),
    (BF, 1, 1, 1, 7777, 8192, 64, True, -1, -1, 30.0), (BF, 7, 5, 1, 711, 8192, 111, True, -1, -1, 50.0),
]


def _uniq(xs):
    return list(dict.fromkeys(xs))


def _id(case):
    return "-".join("bf16" if x is BF else "fp16" if x is F16 else str(x) for x in case)


def _unif(shape, dtype, gen):
    """uniform in [-5, 5) as the reference draws its inputs, on the device"""
    return (torch.rand(shape, generator=gen, device=DEV, dtype=torch.float32) * 10.0 - 5.0).to(dtype)


def _check(out_rows, lse_rows, q_rows, k_rows, v_rows, dtype, scale, causal, window, softcap):
    """One (sequence, kv head): out_rows (Sq, g, Dv) and lse_rows (g, Sq) from
    the GPU against the oracle and the exact result on q_rows (Sq, g, D),
    k_rows / v_rows (Lk, D)."""
    qh = bits(q_rows)[None]
    kh, vh = bits(k_rows)[None, :, None], bits(v_rows)[None, :, None]
    ro, rl = orc.attention(qh, kh, vh, dtype=odt(dtype), scale=scale, softcap=softcap, causal=causal,
                           window=window, nthreads=NT)
    mx = assert_close_out(out_rows[None], ro, dtype, tol=TOL[dtype] * SIGMA_V)
    rel = assert_close_lse(lse_rows[None], rl) if lse_rows is not None else 0.0
    ex, _ = brute.attention(q_rows.float().cpu().numpy(), k_rows.float().cpu().numpy()[:, None],
                            v_rows.float().cpu().numpy()[:, None], scale, causal=causal, window=window,
                            softcap=softcap)
    got = out_rows.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ex)
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    vmax = float(v_rows.abs().max()) if v_rows.numel() else 0.0
    bad = err > u * vmax + u * np.abs(ex) + 1e-4
    assert not bad.any(), (f"{int(bad.sum())} outputs beyond the 16-bit rounding envelope of the float64 result "
                           f"(max err {err.max():.3e})")
    return mx, rel


def _picks(n, every):
    return list(range(n)) if every else sorted({0, n - 1})


def _check_all(seqs, kv_heads, g, get, dtype, scale, causal, window, softcap):
    """get(b, hk) -> (out_rows, lse_rows or None, q_rows, k_rows, v_rows)."""
    worst = [0.0, 0.0]
    for b in seqs:
        for hk in kv_heads:
            o, l, qr, kr, vr = get(b, hk)
            if qr.shape[0] == 0:
                continue
            mx, rel = _check(o, l, qr, kr, vr, dtype, scale, causal, window, softcap)
            worst = [max(worst[0], mx), max(worst[1], rel)]
    return worst


# ---- v2 flash_attn_with_kvcache ------------------------------------------------------------------
@pytest.mark.parametrize("case", _uniq(V2_KV), ids=_id)
def test_reference_v2_kvcache(case):
    import flash_attn_npu_v2
    dtype, B, H, Hk, Sq, Sk, D, cache_mode, _, causal, wl, wr, softcap = case
    print(f"case v2 kvcache {_id(case)}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(7000 + V2_KV.index(case))
    block = 128
    q = _unif((B, Sq, H, D), dtype, gen)
    nper = (Sk + block - 1) // block
    if cache_mode == 1:
        nblocks = max(64, nper * B)
        kc, vc = _unif((nblocks, block, Hk, D), dtype, gen), _unif((nblocks, block, Hk, D), dtype, gen)
        bt = torch.arange(B * nper, dtype=torch.int32, device=DEV).view(B, nper)
    else:
        kc, vc = _unif((B, Sk, Hk, D), dtype, gen), _unif((B, Sk, Hk, D), dtype, gen)
        bt = None
    seqlens = torch.full((B,), Sk, dtype=torch.int32, device=DEV)
    out, lse = flash_attn_npu_v2.flash_attn_with_kvcache(q, kc, vc, None, None, cache_seqlens=seqlens,
                                                         block_table=bt, causal=causal, window_size=[wl, wr],
                                                         softcap=softcap, rotary_interleaved=False,
                                                         return_softmax_lse=True)
    torch.cuda.synchronize()
    g = H // Hk
    keys = (lambda c, b: c[bt[b].long()].reshape(-1, Hk, D)[:Sk]) if bt is not None else (lambda c, b: c[b, :Sk])

    def get(b, hk):
        hs = slice(hk * g, (hk + 1) * g)
        return out[b, :, hs], lse[b, hs], q[b, :, hs], keys(kc, b)[:, hk], keys(vc, b)[:, hk]

    mx, rel = _check_all(_picks(B, False), _picks(Hk, False), g, get, dtype, D ** -0.5, causal, (wl, wr), softcap)
    print(f"  out max-abs {mx:.2e}, lse rel {rel:.1e}", flush=True)


# ---- v3 flash_attn_with_kvcache ------------------------------------------------------------------
def _v3_runs():
    runs = []
    for case in _uniq(V3_KV):
        layout, varied = case[9], case[10]
        for cache_mode in (0, 1):
            for ns in (0, 2):
                if ns > 1 and not (cache_mode == 1 and layout == "TND"):
                    continue
                if varied and layout != "TND":
                    continue
                runs.append((case, cache_mode, ns))
    return runs


@pytest.mark.parametrize("run", _v3_runs(), ids=lambda r: f"{_id(r[0])}-cache{r[1]}-splits{r[2]}")
def test_reference_v3_kvcache(run):
    import flash_attn_npu_v3
    case, cache_mode, num_splits = run
    dtype, B, H, Hk, q_seqlen, kv_seqlen, D, _, causal, layout, varied, wl, wr, softcap = case
    print(f"case v3 kvcache {_id(case)} cache_mode {cache_mode} num_splits {num_splits}", flush=True)
    seed = 8000 + V3_KV.index(case) * 4 + cache_mode * 2 + (num_splits > 0)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    block = 128
    if varied:
        # per-batch q in [1, q_seqlen], kv in [q, kv_seqlen] (the reference's draw, :296-302)
        gl = torch.Generator().manual_seed(1234)
        q_lens = torch.randint(low=1, high=q_seqlen + 1, size=(B,), generator=gl).tolist()
        kv_lens = [int(torch.randint(low=q, high=kv_seqlen + 1, size=(1,), generator=gl)) for q in q_lens]
    else:
        q_lens, kv_lens = [q_seqlen] * B, [kv_seqlen] * B
    tnd = layout == "TND"
    q = _unif((sum(q_lens), H, D) if tnd else (B, q_seqlen, H, D), dtype, gen)
    nper = (kv_seqlen + block - 1) // block
    bt = None
    cu_k = None
    if cache_mode == 1:
        nblocks = max(64, nper * B)
        kc, vc = _unif((nblocks, block, Hk, D), dtype, gen), _unif((nblocks, block, Hk, D), dtype, gen)
        bt = torch.arange(B * nper, dtype=torch.int32, device=DEV).view(B, nper)
    elif tnd:
        kc, vc = _unif((sum(kv_lens), Hk, D), dtype, gen), _unif((sum(kv_lens), Hk, D), dtype, gen)
        cu_k = np.concatenate([[0], np.cumsum(kv_lens)])
    else:
        kc, vc = _unif((B, kv_seqlen, Hk, D), dtype, gen), _unif((B, kv_seqlen, Hk, D), dtype, gen)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)])
    seqlens = torch.tensor(kv_lens, dtype=torch.int32, device=DEV)
    out, lse, *_ = flash_attn_npu_v3.flash_attn_with_kvcache(
        q, kc, vc, None, None, None, cache_seqlens=seqlens, page_table=bt,
        cu_seqlens_q=torch.from_numpy(cu_q).to(torch.int32).to(DEV) if tnd else None,
        max_seqlen_q=q_seqlen, causal=causal, window_size=[wl, wr], softcap=softcap, rotary_interleaved=False,
        num_splits=num_splits, return_softmax_lse=True)
    torch.cuda.synchronize()
    g = H // Hk

    def keys(c, b):
        if bt is not None:
            return c[bt[b].long()].reshape(-1, Hk, D)[:kv_lens[b]]
        if cu_k is not None:
            return c[cu_k[b]:cu_k[b + 1]]
        return c[b, :kv_lens[b]]

    def get(b, hk):
        hs = slice(hk * g, (hk + 1) * g)
        if tnd:
            rows = slice(int(cu_q[b]), int(cu_q[b + 1]))
            return out[rows, hs], lse[hs, rows], q[rows, hs], keys(kc, b)[:, hk], keys(vc, b)[:, hk]
        return out[b, :, hs], lse[b, hs], q[b, :, hs], keys(kc, b)[:, hk], keys(vc, b)[:, hk]

    mx, rel = _check_all(_picks(B, False), _picks(Hk, False), g, get, dtype, D ** -0.5, causal, (wl, wr), softcap)
    print(f"  out max-abs {mx:.2e}, lse rel {rel:.1e}", flush=True)


# ---- v3 flash_attn_func ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", _uniq(DENSE), ids=_id)
def test_reference_v3_dense(case):
    import flash_attn_npu_v3
    dtype, B, H, Hk, Sq, Sk, D, ret, causal, softcap = case
    print(f"case v3 dense {_id(case)}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(9000 + DENSE.index(case))
    q, k, v = _unif((B, Sq, H, D), dtype, gen), _unif((B, Sk, Hk, D), dtype, gen), _unif((B, Sk, Hk, D), dtype, gen)
    scale = 1.0 / math.sqrt(D)
    res = flash_attn_npu_v3.flash_attn_func(q, k, v, softmax_scale=scale, causal=causal, window_size=[-1, -1],
                                            softcap=softcap, return_attn_probs=ret)
    out, lse = (res[0], res[1]) if ret else (res, None)
    torch.cuda.synchronize()
    g = H // Hk

    def get(b, hk):
        hs = slice(hk * g, (hk + 1) * g)
        return out[b, :, hs], None if lse is None else lse[b, hs], q[b, :, hs], k[b, :, hk], v[b, :, hk]

    mx, rel = _check_all(_picks(B, False), _picks(Hk, False), g, get, dtype, scale, causal, (-1, -1), softcap)
    print(f"  out max-abs {mx:.2e}, lse rel {rel:.1e}", flush=True)


# ---- v3 flash_attn_varlen_func --------------------------------------------------------------------
@pytest.mark.parametrize("case", _uniq(VARLEN), ids=_id)
def test_reference_v3_varlen(case):
    import flash_attn_npu_v3
    dtype, B, H, Hk, Sq, Sk, D, causal, wl, wr, softcap = case
    print(f"case v3 varlen {_id(case)}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(9500 + VARLEN.index(case))
    q, k, v = _unif((B * Sq, H, D), dtype, gen), _unif((B * Sk, Hk, D), dtype, gen), _unif((B * Sk, Hk, D), dtype, gen)
    cu_q = torch.arange(B + 1, dtype=torch.int32, device=DEV) * Sq
    cu_k = torch.arange(B + 1, dtype=torch.int32, device=DEV) * Sk
    scale = 1.0 / math.sqrt(D)
    out, lse = flash_attn_npu_v3.flash_attn_varlen_func(q, k, v, cu_q, cu_k, Sq, Sk, softmax_scale=scale,
                                                        causal=causal, window_size=(wl, wr), softcap=softcap,
                                                        return_attn_probs=True)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (B * Sq, H, D) and tuple(lse.shape) == (H, B * Sq)
    g = H // Hk

    def get(b, hk):
        hs, rows, keys = slice(hk * g, (hk + 1) * g), slice(b * Sq, (b + 1) * Sq), slice(b * Sk, (b + 1) * Sk)
        return out[rows, hs], lse[hs, rows], q[rows, hs], k[keys, hk], v[keys, hk]

    every = D % 8 != 0  # the head dims the v3 API pads: every sequence
    mx, rel = _check_all(_picks(B, every), _picks(Hk, every), g, get, dtype, scale, causal, (wl, wr), softcap)
    print(f"  out max-abs {mx:.2e}, lse rel {rel:.1e}", flush=True)
