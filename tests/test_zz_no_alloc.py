"""kh_qmatmul_static: the product without a workspace argument (its scratch a
device array of the library), against kh_qmatmul with a workspace of the
caller, through the C ABI: bitwise equal on two calls in a row, the second
smaller, for the decode, small-M and many-row kernels; a call needing more
than the array is refused before any launch."""

import numpy as np
import pytest
import torch

import kapel_amd as ka
from kapel_amd import synth

pytestmark = pytest.mark.gpu

LIMIT = 32 << 20  # KH_STATIC_SCRATCH_BYTES


def weights(specs, seed):
    ws = []
    for i, (fmt, group, n, k) in enumerate(specs):
        data = ka.quantize(fmt, group, synth.normal(seed + i, n * k, 0.02))
        ws.append(ka.QuantizedTensor(torch.from_numpy(data).to("cuda:0"), fmt, group, n, k))
    return ws


def call(ws, x, flags, static):
    lib = ka.lib()
    arr = (ka._Weight * len(ws))(*[w.weight() for w in ws])
    rows, k = x.shape
    out = torch.full((rows, sum(w.n for w in ws)), float("nan"), device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    if static:
        status = lib.kh_qmatmul_static(arr, len(ws), k, ka.F32, x.data_ptr(), rows, ka.F32,
                                       out.data_ptr(), flags, stream)
    else:
        size = lib.kh_qmatmul_workspace(arr, len(ws), k, rows, flags)
        ws_ = torch.zeros(size, dtype=torch.uint8, device="cuda:0")
        status = lib.kh_qmatmul(arr, len(ws), k, ka.F32, x.data_ptr(), rows, ka.F32, out.data_ptr(),
                                flags, ws_.data_ptr(), size, stream)
    torch.cuda.synchronize()
    return status, out.cpu().numpy()


@pytest.mark.parametrize("flags", [0, ka.BYTE_ACTIVATIONS_ALL_ROWS])
@pytest.mark.parametrize("case", [
    # (weights, rows of the first call, rows of the second call)
    ([(ka.Q4K, 0, 1024, 3072), (ka.Q4K, 0, 512, 3072)], 1, 1),
    ([(ka.Q6K, 0, 300, 2048)], 40, 3),
    ([(ka.Q8_0, 0, 700, 4096)], 130, 17),
])
def test_static_scratch_matches_the_workspace_entry(case, flags):
    specs, rows1, rows2 = case
    ws = weights(specs, 11)
    k = specs[0][3]
    for i, rows in enumerate((rows1, rows2)):
        x = torch.from_numpy(synth.normal(40 + i, rows * k, 1.0).reshape(rows, k)).to("cuda:0")
        s1, want = call(ws, x, flags, static=False)
        s2, got = call(ws, x, flags, static=True)
        assert s1 == ka.KH_OK and s2 == ka.KH_OK
        assert not np.isnan(got).any()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (specs, rows)


def test_static_scratch_refuses_what_does_not_fit():
    ws = weights([(ka.Q8_0, 0, 64, 8192)], 3)
    arr = (ka._Weight * 1)(ws[0].weight())
    rows = 4096  # the prepared activations alone exceed the array
    assert ka.lib().kh_qmatmul_workspace(arr, 1, 8192, rows, 0) > LIMIT
    x = torch.zeros((rows, 8192), device="cuda:0")
    out = torch.zeros((rows, 64), device="cuda:0")
    status = ka.lib().kh_qmatmul_static(arr, 1, 8192, ka.F32, x.data_ptr(), rows, ka.F32, out.data_ptr(),
                                        0, torch.cuda.current_stream().cuda_stream)
    assert status == ka.KH_ERR_WORKSPACE
    assert ka.lib().kh_error_string(status)
