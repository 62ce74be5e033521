"""GPU parity of the fast decode kernels at group sizes other than 1, 2, 4 and 8: Hq / Hkv = 3,
5, 6, 7 and 16 run the matrix-core kernel (paged_decode_mfma, q rows G..15 of its 16-row MFMA
blocks zero), as in Llama-3.2-3B (24 / 8), Qwen2.5-7B (28 / 4) or Qwen3-235B-A22B (64 / 4).
The reference's decode step for them is the same torch path as for any other head ratio
(src/plastic_infer/exec/attention.py:151-190, src/plastic_infer/exec/runner_paged.py:112-129,
251-255).

Bars: the pools after an append call bit-exact against the oracle's write (the new tokens'
slots hold NaN / Inf before the call); outputs within 2e-2 (bf16) / 5e-3 (fp16) of the oracle.
"""

from __future__ import annotations

import pytest
import torch

import oracle.paged_kv as OP
from plastic_infer.kernel import paged_decode_attention
from test_gpu_append_decode import _case, _check

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3}


@pytest.mark.parametrize("dtype,G", [(torch.bfloat16, 3), (torch.bfloat16, 5),
                                     (torch.bfloat16, 6), (torch.bfloat16, 7),
                                     (torch.bfloat16, 16), (torch.float16, 3),
                                     (torch.float16, 7), (torch.float16, 16)])
def test_append_decode_other_group_sizes(dev, dtype, G):
    """Lengths around page (16) and step (128) boundaries, two kv heads; the append call
    against the oracle and against kv_scatter + paged_decode_attention."""
    Hkv = 2
    lens = [1, 15, 16, 17, 127, 128, 129, 511, 512, 513, 1024, 1100]
    q, kp, vp, bt, lens_t, kn, vn = _case(300 + G, lens, Hkv * G, Hkv, 700, dtype=dtype)
    _check(dev, q, kp, vp, bt, lens_t, kn, vn, 16, tol=TOL[dtype])


@pytest.mark.parametrize("G,lens", [
    (3, [8192]),                 # one segment per kv head, cut over many waves and merged
    (7, [0, 4097, 0, 129, 0]),
    (16, [8192, 3]),
    (16, [0, 4097, 0, 129, 0]),
])
def test_decode_other_group_sizes_split_over_waves(dev, G, lens):
    Hkv = 4
    q, kp, vp, bt, lens_t, _, _ = _case(320 + G, lens, Hkv * G, Hkv, 1100)
    out = paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                 lens_t.to(dev)).cpu()
    live = lens_t > 0
    assert not out[~live].any()
    ref = OP.decode_batch(q[live], kp, vp, bt[live].clamp(min=0), lens_t[live], 16)
    err = (out[live].float() - ref.float()).abs().max().item()
    assert err <= TOL[torch.bfloat16], err
