"""GPU parity of transfers and view packing against the reference's raw
byte contract (tests/fixtures/transfer_contract.php, transcribed into
tests/golden/transfer_contract.json; the checks follow
tests/cuda_transfer_contract.phpt:21-61 and host_array_transfer_layout.phpt:
14-47).  Thirteen storage dtypes, eight elements each, including NaN
payloads, signed zeros, infinities and subnormal bit patterns: every view
layout must download exactly the bytes of its logical elements, so the
device pack kernel has to move bits, never values."""
import gc
import json
import os

import pytest

from phptensors import CudaArray

pytestmark = pytest.mark.gpu

FIX = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "transfer_contract.json")))

# the fixture's view recipes, restated with this package's view methods
VIEWS = {
    "contiguous": lambda x: x,
    "offset": lambda x: x.select(0, 1),                              # $x->slice(1)
    "transpose": lambda x: x.transpose(),
    "stepped": lambda x: x.slice(":, 1:4:2"),
    "offset-stepped": lambda x: x.slice(1, [1, 4, 2]),
    "broadcast": lambda x: x.select(0, 1).broadcastTo([3, 4]),
    "scalar": lambda x: x.select(0, 1).select(0, 2),                 # $x->slice(1, 2)
    "empty": lambda x: x.slice([0, 0]),
    "singleton": lambda x: x.reshape([1, 2, 4]),
}


def expected_bytes(raw, width, indices):
    return b"".join(raw[i * width:(i + 1) * width] for i in indices)


@pytest.mark.parametrize("dtype", sorted(FIX["patterns"]))
def test_view_layouts_download_exact_bytes(dtype):
    raw = bytes.fromhex(FIX["patterns"][dtype])
    width = len(raw) // 8
    assert width * 8 == len(raw)
    device = CudaArray.fromBuffer(raw, [2, 4], dtype)
    assert device.toBuffer() == raw
    kept = []
    for name, spec in FIX["layouts"].items():
        view = VIEWS[name](device)
        want = expected_bytes(raw, width, spec["indices"])
        assert view.getShape() == spec["shape"] and view.getDtype() == dtype, name
        assert view.toBuffer() == want, name
        copy = view.copy()
        assert copy.getShape() == spec["shape"] and copy.toBuffer() == want, name
        # a second upload of the downloaded bytes gives the same bytes
        if spec["shape"] and 0 not in spec["shape"]:
            again = CudaArray.fromBuffer(want, spec["shape"], dtype)
            assert again.toBuffer() == want, name
        kept.append((view, copy, want))
    # views and copies keep their storage after the source handle is gone
    del device, view, copy
    gc.collect()
    for view, copy, want in kept:
        assert view.toBuffer() == want
        assert copy.toBuffer() == want


@pytest.mark.parametrize("dtype", sorted(FIX["patterns"]))
def test_large_transpose_and_sparse_column_pack_on_device(dtype):
    raw = bytes.fromhex(FIX["patterns"][dtype])
    width = len(raw) // 8
    large = CudaArray.fromBuffer(raw * 8192, [8192, 8], dtype)
    want = b"".join(raw[i * width:(i + 1) * width] * 8192 for i in range(8))
    assert large.transpose().toBuffer() == want
    assert large.transpose().copy().toBuffer() == want
    col = large.select(1, 3)                                        # $large->slice(':, 3')
    assert col.getShape() == [8192]
    assert col.toBuffer() == raw[3 * width:4 * width] * 8192
