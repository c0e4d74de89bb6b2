"""The allocation-free row selection (``chroma_hip_rows_topk_static``, scratch in a static device array)
against the workspace entry point (``chroma_hip_rows_topk``) through the C ABI, on two calls in a row, the
second smaller, and against the reference GPU top-k order on the host."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import numpy_of
from tests.test_hip_runtime import host_topk, rows_topk, selection_rows

pytestmark = pytest.mark.gpu


def test_static_scratch_selection_matches_workspace_entry_point():
    from chroma_amd._src import native

    lib = native.library()
    cases = [(8, 201088, 40, True, torch.float32), (3, 100003, 5, False, torch.bfloat16)]  # the second needs less scratch
    for rows, width, k, largest, dtype in cases:
        x = selection_rows(rows, width, dtype, 17 * rows + k)
        device = x.cuda()
        values, ids = rows_topk(lib, device, k, largest, entry="static")
        want_values, want_ids = rows_topk(lib, device, k, largest, entry="workspace")
        np.testing.assert_array_equal(ids.numpy(), want_ids.numpy())
        np.testing.assert_array_equal(numpy_of(values).view(np.uint8), numpy_of(want_values).view(np.uint8))
        host = numpy_of(x)
        for r in range(rows):
            np.testing.assert_array_equal(ids[r].numpy(), host_topk(host[r], k, largest))
    # a selection needing more than the static array holds is refused before anything runs
    rows, width, k = 2048, 201088, 64
    assert lib.chroma_hip_rows_topk_workspace(rows, width, k) > (4 << 20)
    small = torch.zeros(8, device="cuda")
    error = ctypes.create_string_buffer(256)
    status = lib.chroma_hip_rows_topk_static(small.data_ptr(), native.FLOAT32, rows, width, k, 1, small.data_ptr(), small.data_ptr(),
                                             None, error, len(error))
    assert status == native.RUNTIME_ERROR and b"static scratch" in error.value
