"""The C-ABI library loads and exports exactly what include/plastic_infer_amd.h declares
(CPU: no compute call is made; argument validation returns before any device work)."""

from __future__ import annotations

import ctypes
import pathlib
import re
import subprocess

import pytest

from plastic_infer import _native as N

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "plastic_infer_amd.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pia_[a-z0-9_]+)\s*\(", text)))


def test_library_exists_and_loads():
    assert N.LIB_PATH.exists(), "build the library first (plastic-infer_amd/csrc/build.py)"
    lib = N.load()
    assert lib.pia_abi_version() == N.EXPECTED_ABI


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 15
    lib = ctypes.CDLL(str(N.LIB_PATH))
    for name in names:
        assert hasattr(lib, name), f"{name} declared but not exported"
    assert set(names) == set(N._SIGNATURES), "ctypes bindings drift from the header"


def test_exports_are_c_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(declared_functions()) <= exported


def test_invalid_arguments_are_rejected_without_device_work():
    lib = N.load()
    rc = lib.pia_kv_scatter(None, None, None, None, None, 4, 8, 8, 2, 4, 16, 10, 3, None)
    assert rc == -1 and b"elem_bytes" in lib.pia_last_error()
    rc = lib.pia_paged_attention(None, None, None, None, None, 1, None, None, None, 1, 1,
                                 3, 2, 16, 16, 10, 1.0, 2, None)
    assert rc == -1 and b"num_heads % num_kv_heads" in lib.pia_last_error()
    rc = lib.pia_moe_topk(None, None, None, 0, 4, 8, 9, 1, 0, -1, None)
    assert rc == -1
    # the workspace is the decode scratch layout at 4096 waves, independent of the batch
    for hq in (8, 16, 32, 64):
        off, total = ctypes.c_int64(), ctypes.c_int64()
        assert lib.pia_paged_decode_scratch_layout(hq, 8, 4096, ctypes.byref(off),
                                                   ctypes.byref(total)) == 0
        for b, bt in ((256, 512), (1, 4)):
            assert N.query("pia_paged_decode_workspace_bytes", b, hq, 8, 128, 16, bt) == \
                total.value
    # general kernel (head_dim 64, or G = 9): no workspace; G = 3 runs a fast kernel
    assert N.query("pia_paged_decode_workspace_bytes", 4, 4, 4, 64, 16, 8) == 0
    assert N.query("pia_paged_decode_workspace_bytes", 4, 72, 8, 128, 16, 8) == 0
    assert N.query("pia_paged_decode_workspace_bytes", 4, 24, 8, 128, 16, 8) > 0
    with pytest.raises(N.NativeError):
        N.call("pia_moe_sum_reduce", None, None, 1, 0, 4, 2, None)
    # the read probe checks its arguments before any launch
    with pytest.raises(N.NativeError):
        N.call("pia_hbm_read_probe", None, 4096, None, 0, None, None)
    # the rows probe too: a shape it does not take, a row it cannot split, no whole block
    fake = 1 << 20  # never dereferenced: every call below fails its checks first
    for row_bytes, r, nbytes in ((1536, 3, 1 << 20), (1088, 2, 1 << 20), (96, 16, 1 << 20),
                                 (4096, 16, 4096)):
        with pytest.raises(N.NativeError):
            N.call("pia_hbm_read_rows_probe", fake, nbytes, row_bytes, r, fake, None)


@pytest.mark.parametrize("group", [1, 2, 3, 4, 5, 6, 7, 8, 16])
def test_decode_scratch_layout(group):
    """The one layout every decode entry point uses: the arrival counters (one 8-byte word per
    wave, starting at the first 8-byte boundary of a buffer that is only 4-byte aligned) end
    before the partials, which are exactly two slots of `group` rows x (128 + 2) fp32 per wave
    and end at the total. A layout whose counters follow partial slots sized for another group
    (a past fault of this kind) breaks the first or the last assertion."""
    lib = N.load()
    prev_total = 0
    for waves in (2, 6, 256, 1024, 2048, 4094, 4096):
        off, total = ctypes.c_int64(), ctypes.c_int64()
        assert lib.pia_paged_decode_scratch_layout(8 * group, 8, waves, ctypes.byref(off),
                                                   ctypes.byref(total)) == 0
        assert off.value % 256 == 0
        assert 4 + 8 * waves <= off.value, "counters overrun the partials"
        assert total.value - off.value == waves * 2 * group * (128 + 2) * 4
        assert total.value > prev_total
        prev_total = total.value
    off, total = ctypes.c_int64(), ctypes.c_int64()
    assert lib.pia_paged_decode_scratch_layout(72, 8, 64, ctypes.byref(off),
                                               ctypes.byref(total)) == -2
    assert lib.pia_paged_decode_scratch_layout(32, 8, 4097, ctypes.byref(off),
                                               ctypes.byref(total)) == -1
