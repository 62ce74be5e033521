"""pia_paged_decode_attention_noalloc (the library-scratch decode entry point) against
pia_paged_decode_attention (caller workspace), both called through the C-ABI.

Both run the same kernels with the same split of the batch over the same wave count, so their
outputs must agree bit for bit; the oracle bounds both within 2e-2 (the bf16 attention bar).
Each case makes two no-alloc calls in a row on the shared scratch, the second on a smaller
batch, so stale partials of the first call are present when the second runs.
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle.paged_kv as OP
from plastic_infer import _native as N
from plastic_infer.kernel import decode_workspace_bytes

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _case(seed: int, lens: list[int], Hq: int, Hkv: int, D: int, num_pages: int, dtype):
    g = torch.Generator().manual_seed(seed)
    n_pages = [(L + 15) // 16 for L in lens]
    maxp = max(1, max(n_pages))
    perm = torch.randperm(num_pages, generator=g)
    bt = torch.full((len(lens), maxp), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(n_pages):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    kp = torch.randn(num_pages, Hkv, D, 16, generator=g).to(dtype)
    vp = torch.randn(num_pages, Hkv, D, 16, generator=g).to(dtype)
    q = torch.randn(len(lens), Hq, D, generator=g).to(dtype)
    return q, kp, vp, bt, torch.tensor(lens, dtype=torch.int32)


def _call(name: str, dev, q, kp, vp, bt, lens, ws=None):
    B, Hq, D = q.shape
    num_pages, Hkv = kp.shape[0], kp.shape[1]
    out = torch.full((B, Hq, D), float("nan"), dtype=q.dtype, device=dev)
    args = [out.data_ptr(), q.data_ptr(), q.stride(0), kp.data_ptr(), vp.data_ptr(),
            bt.data_ptr(), bt.shape[1], lens.data_ptr(), B, Hq, Hkv, D, 16, num_pages,
            1.0 / math.sqrt(D), N.dtype_code(q.dtype)]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    N.call(name, *args, N.stream_of(dev))
    return out


@pytest.mark.parametrize("G,Hkv,D,dtype", [(4, 8, 128, torch.bfloat16),
                                           (8, 4, 128, torch.bfloat16),
                                           (1, 2, 128, torch.bfloat16),
                                           (16, 2, 128, torch.bfloat16),
                                           (4, 8, 128, torch.float16),
                                           (7, 2, 128, torch.float16),
                                           (2, 2, 64, torch.float16)])   # general kernel
def test_noalloc_matches_workspace_entry_point(dev, G, Hkv, D, dtype):
    g = torch.Generator().manual_seed(900 + G)
    first = torch.randint(1, 600, (300,), generator=g).tolist()
    first[7] = 0
    first[11] = 5000
    second = torch.randint(1, 900, (37,), generator=g).tolist()
    Hq = G * Hkv
    for i, lens in enumerate((first, second)):
        q, kp, vp, bt, lt = _case(910 + 10 * G + i, lens, Hq, Hkv, D, 7000, dtype)
        qd, kd, vd, btd, ld = (t.to(dev) for t in (q, kp, vp, bt, lt))
        need = decode_workspace_bytes(len(lens), Hq, Hkv, D, 16, bt.shape[1])
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        ref_dev = _call("pia_paged_decode_attention", dev, qd, kd, vd, btd, ld, ws).cpu()
        got = _call("pia_paged_decode_attention_noalloc", dev, qd, kd, vd, btd, ld).cpu()
        torch.cuda.synchronize(dev)
        assert torch.equal(got, ref_dev), f"call {i}: no-alloc differs from the workspace path"
        ref = OP.decode_batch(q, kp, vp, bt.clamp(min=0), lt, 16)
        err = (got.float() - ref.float()).abs().max().item()
        assert err <= BF16_TOL, (i, err)


def test_noalloc_batch_over_one_launch_then_smaller(dev):
    """1100 sequences (two launches sharing the scratch inside one call), then 5 sequences."""
    g = torch.Generator().manual_seed(950)
    for i, lens in enumerate((torch.randint(0, 200, (1100,), generator=g).tolist(),
                              [4097, 1, 16, 17, 0])):
        q, kp, vp, bt, lt = _case(951 + i, lens, 32, 8, 128, 16000, torch.bfloat16)
        qd, kd, vd, btd, ld = (t.to(dev) for t in (q, kp, vp, bt, lt))
        need = decode_workspace_bytes(len(lens), 32, 8, 128, 16, bt.shape[1])
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        ref_dev = _call("pia_paged_decode_attention", dev, qd, kd, vd, btd, ld, ws).cpu()
        got = _call("pia_paged_decode_attention_noalloc", dev, qd, kd, vd, btd, ld).cpu()
        assert torch.equal(got, ref_dev), f"call {i}"


def test_noalloc_scratch_size_and_limit():
    """The scratch a launch needs (meta ints, then two partial slots per wave) fits the
    library's 32 MiB for every supported group size."""
    lib = N.load()
    for G in (1, 2, 3, 4, 5, 6, 7, 8, 16):
        need = lib.pia_paged_decode_noalloc_scratch_bytes(8 * G, 8)
        assert 0 < need <= 32 << 20, (G, need)
    assert lib.pia_paged_decode_noalloc_scratch_bytes(72, 8) == 0   # G = 9: general kernel
