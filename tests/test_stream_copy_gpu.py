"""ember_stream_copy, the benchmark's bandwidth reference: a bit-exact copy at sizes from one
16-byte unit to tens of MB, and EMBER_EINVAL for sizes or pointers it does not take."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib, ops  # noqa: E402

DEV = "cuda"


@pytest.mark.parametrize("n", [4, 256, 1028, 33 * 2 ** 20 // 4 + 4])
def test_stream_copy_is_exact(n):
    g = torch.Generator(device=DEV)
    g.manual_seed(n)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), generator=g, device=DEV, dtype=torch.int32)
    dst = torch.full_like(src, 7)
    ops.stream_copy_hip(src, dst)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)


def test_stream_copy_rejects_what_it_does_not_take():
    lib = _lib.load()
    a = torch.zeros(64, dtype=torch.int32, device=DEV)
    b = torch.zeros(64, dtype=torch.int32, device=DEV)
    assert lib.ember_stream_copy(a.data_ptr(), b.data_ptr(), 12, None) == 1        # not a multiple of 16
    assert lib.ember_stream_copy(a.data_ptr() + 4, b.data_ptr(), 16, None) == 1    # unaligned
    assert lib.ember_stream_copy(a.data_ptr(), b.data_ptr(), 0, None) == 0
    with pytest.raises(ValueError):
        ops.stream_copy_hip(a[1:], b[1:])
