"""The HBM read probe behind bench.py --workload hbm-read (a measurement aid with no
counterpart in the reference): both access patterns run on a small buffer and return success,
tile ids outside the buffer are skipped by the kernel's own bounds check, and malformed sizes
are refused before any launch."""

from __future__ import annotations

import pytest
import torch

from plastic_infer import _native as N

pytestmark = pytest.mark.gpu


def test_hbm_read_probe_patterns(dev):
    buf = torch.randint(0, 255, (1 << 20,), dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    st = N.stream_of(dev)
    N.call("pia_hbm_read_probe", buf.data_ptr(), buf.numel(), None, 0, sink.data_ptr(), st)
    ids = torch.tensor([0, 255, 7, -1, 256, 1 << 30, 3], dtype=torch.int32, device=dev)
    N.call("pia_hbm_read_probe", buf.data_ptr(), buf.numel(), ids.data_ptr(), ids.numel(),
           sink.data_ptr(), st)
    torch.cuda.synchronize(dev)
    with pytest.raises(N.NativeError):
        N.call("pia_hbm_read_probe", buf.data_ptr(), 100, None, 0, sink.data_ptr(), st)


@pytest.mark.parametrize("row_bytes,rows_per_load", [(1536, 16), (1536, 1), (4096, 8),
                                                     (4096, 2), (1024, 4)])
def test_hbm_read_rows_probe_shapes(dev, row_bytes, rows_per_load):
    """Every load shape reads whole 16-row blocks of the buffer (the tail past the last whole
    block is not read) and returns success."""
    buf = torch.randint(0, 255, ((1 << 20) + 4096,), dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    N.call("pia_hbm_read_rows_probe", buf.data_ptr(), buf.numel(), row_bytes, rows_per_load,
           sink.data_ptr(), N.stream_of(dev))
    torch.cuda.synchronize(dev)
