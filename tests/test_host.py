"""CPU checks of the product library: it loads, exports what the header
declares, agrees with the oracle on geometry and on the load-time quantizers,
and refuses what QuantizedMatmul::infer refuses (kapel-ops/src/matmul.rs:105-150),
before any device work."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import kapel_amd as ka
import oracle as ko
from kapel_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "kapel_hip.h")).read()
    return sorted(set(re.findall(r"^[a-z_0-9 \*]*?\b(kh_[a-z_0-9]+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    declared = header_symbols()
    assert len(declared) >= 11
    assert sorted(ka.SYMBOLS) == declared
    L = ka.lib()
    for name in declared:
        assert hasattr(L, name), name
    assert L.kh_version().startswith(b"kapel_hip")


FORMATS = [(ka.INT8, 32), (ka.INT8, 40), (ka.INT8, 64), (ka.INT8, 128), (ka.INT4, 32),
           (ka.INT4, 40), (ka.INT4, 64), (ka.Q8_0, 0), (ka.Q4_0, 0), (ka.Q4_1, 0), (ka.Q5_0, 0),
           (ka.Q5_1, 0), (ka.Q2K, 0), (ka.Q3K, 0), (ka.Q4K, 0), (ka.Q5K, 0), (ka.Q6K, 0),
           (ka.IQ4_NL, 0), (ka.IQ4_XS, 0), (ka.IQ3_S, 0)]


@pytest.mark.parametrize("fmt,group", FORMATS)
def test_geometry_matches_the_oracle(fmt, group):
    assert ka.block_len(fmt, group) == ko.block_len(fmt, group)
    assert ka.block_bytes(fmt, group) == ko.block_bytes(fmt, group)


def test_unknown_formats_have_no_geometry():
    assert ka.block_len(99, 0) == 0 and ka.block_bytes(15, 0) == 0
    assert ka.block_len(ka.INT4, 7) == 0  # odd int4 groups (dtype.rs:119-128)
    assert ka.block_len(ka.INT8, 0) == 0


REFERENCE_QUANTIZERS = [(ka.INT8, 32), (ka.INT8, 64), (ka.INT4, 32), (ka.INT4, 64), (ka.INT4, 40),
                        (ka.Q8_0, 0), (ka.Q4_0, 0), (ka.Q4_1, 0)]


@pytest.mark.parametrize("fmt,group", REFERENCE_QUANTIZERS)
def test_host_quantizer_writes_the_reference_bytes(fmt, group):
    """Two independent implementations of dtype.rs:565-841 (the oracle's C
    and the library's C++) give the same bytes, on normal data, on edge
    blocks (zeros, ties, a single spike) and on the dtype.rs test ramp."""
    length = ko.block_len(fmt, group)
    x = synth.normal(3, 64 * length, 0.02)
    x[:length] = 0.0
    x[length:2 * length] = np.arange(length, dtype=np.float32) - length / 2 + 0.5
    x[2 * length:3 * length] = 0.0
    x[2 * length + 3] = -1.0
    ramp = np.array([(i - 31.5) / 10.0 for i in range(64)], dtype=np.float32)
    x = np.concatenate([x, np.resize(ramp, (64 // length + 1) * length)[:length * max(1, 64 // length)]])
    x = x[: x.size // length * length]
    ours = ka.quantize(fmt, group, x, threads=3)
    theirs = ko.quantize(fmt, group, x)
    assert np.array_equal(ours, theirs)


KQUANTS = [(ka.Q2K, 3), (ka.Q3K, 7), (ka.Q4K, 15), (ka.Q5K, 31), (ka.Q6K, 63), (ka.Q5_0, 31),
           (ka.Q5_1, 31)]


@pytest.mark.parametrize("fmt,levels", KQUANTS)
def test_library_encoders_round_trip(fmt, levels):
    """The library's own encoders (no reference counterpart) write valid
    blocks: decoded by the oracle's restatement of dtype.rs:342-520, every
    value is within about a step of its source, and the error shrinks with
    the number of levels."""
    length = ko.block_len(fmt)
    x = synth.normal(11, 64 * 256, 0.02)
    back = ko.dequantize(fmt, 0, ka.quantize(fmt, 0, x))
    err = np.abs(back - x.astype(np.float64))
    # Per group of 16, the step is at most the group's range / levels, and
    # the sub-scale rounding adds at most a few percent of the block's step.
    span = np.ptp(x.reshape(-1, 16), axis=1).max() if fmt != ka.Q6K else 2 * np.abs(x).max()
    assert err.max() <= 1.5 * span / levels + 1e-6, (err.max(), span / levels)
    rel = np.sqrt((err ** 2).mean()) / x.std()
    assert rel < {3: 0.35, 7: 0.2, 15: 0.1, 31: 0.05, 63: 0.025}[levels], rel
    # Zeros stay zeros.
    zeros = ko.dequantize(fmt, 0, ka.quantize(fmt, 0, np.zeros(length, np.float32)))
    assert np.all(zeros == 0.0)


def test_quantizer_refuses_partial_blocks():
    with pytest.raises(ka.BlockMisaligned):
        ka.quantize(ka.Q4K, 0, np.zeros(100, np.float32))
    with pytest.raises(ka.UnsupportedDType):
        ka.quantize(ka.IQ3_S, 0, np.zeros(256, np.float32))


def weight_struct(fmt, group, n, k, data=4096):
    size = 0 if ka.block_len(fmt, group) == 0 else k // max(1, ka.block_len(fmt, group)) * ka.block_bytes(fmt, group) * n
    return ka._Weight(fmt, group, data, size, n)


def qmatmul(weights, k, rows, x=4096, out=4096, kind=ka.F32, flags=0, ws=4096, ws_bytes=1 << 40):
    """Fake, aligned addresses: every call here is refused or empty before any access."""
    arr = (ka._Weight * max(1, len(weights)))(*weights)
    return ka.lib().kh_qmatmul(arr, len(weights), k, kind, x, rows, kind, out, flags, ws,
                               ws_bytes, None)


def test_the_abi_refuses_what_infer_refuses():
    """Status codes, returned before any device call (no GPU needed)."""
    w = weight_struct(ka.Q4K, 0, 4, 512)
    assert qmatmul([], 512, 1) == ka.KH_ERR_ARITY
    assert qmatmul([weight_struct(99, 0, 4, 512)], 512, 1) == ka.KH_ERR_DTYPE
    assert qmatmul([weight_struct(ka.Q4K, 0, 4, 512)], 500, 1) == ka.KH_ERR_MISALIGNED
    bad = ka._Weight(ka.Q4K, 0, 4096, 7, 4)
    assert qmatmul([bad], 512, 1) == ka.KH_ERR_SHAPE
    assert qmatmul([w], 512, 1, kind=7) == ka.KH_ERR_DTYPE
    assert qmatmul([w], 512, 1, ws=None) == ka.KH_ERR_WORKSPACE
    assert qmatmul([w], 512, 1, ws_bytes=16) == ka.KH_ERR_WORKSPACE
    assert qmatmul([w], 512, 1, ws=4096 + 64) == ka.KH_ERR_WORKSPACE  # 256-byte alignment
    assert qmatmul([weight_struct(ka.Q4K, 0, 4, 512, data=4098)], 512, 1) == ka.KH_ERR_SHAPE
    huge = ka._Weight(ka.Q4K, 0, 4096, (1 << 33) * 144, 1 << 33)
    assert qmatmul([huge], 256, 1) == ka.KH_ERR_OVERFLOW
    assert qmatmul([w], 512, 1, x=None) == ka.KH_ERR_NULL
    # Nothing to do: no rows, or no weight rows.
    assert qmatmul([w], 512, 0) == ka.KH_OK
    assert qmatmul([weight_struct(ka.Q4K, 0, 0, 512)], 512, 3) == ka.KH_OK
    assert ka.lib().kh_error_string(ka.KH_ERR_MISALIGNED).startswith(b"quantized_matmul")


def test_workspace_grows_with_rows_and_covers_the_split():
    w = weight_struct(ka.Q4K, 0, 8192, 3072)
    arr = (ka._Weight * 1)(w)
    one = ka.lib().kh_qmatmul_workspace(arr, 1, 3072, 1, 0)
    many = ka.lib().kh_qmatmul_workspace(arr, 1, 3072, 64, ka.BYTE_ACTIVATIONS)
    assert 0 < one < many
    assert ka.lib().kh_qmatmul_workspace(arr, 1, 3000, 1, 0) == 0  # refused: misaligned
    # K = 0 (conformity.rs's [5, 0] case): the call plans no launch (the
    # outputs are zero-filled), at every row count and activation kind; the
    # workspace is still sized.
    empty = (ka._Weight * 1)(weight_struct(ka.Q4K, 0, 8, 0))
    for rows in (1, 3, 17, 64):
        for flags in (0, ka.BYTE_ACTIVATIONS, ka.BYTE_ACTIVATIONS_ALL_ROWS):
            assert ka.lib().kh_qmatmul_workspace(empty, 1, 0, rows, flags) > 0


def test_workspace_of_a_launch_of_many_rounds_without_a_device():
    """A launch of many rounds of the CUs (the 151936 x 4096 Q6_K table)
    plans the streamed decode kernel, whose plan asks the runtime for its
    occupancy: with no device the query fails and the plan falls back to its
    own count; sizing the workspace (which plans f32 and bf16 activations
    alike) still succeeds, at one row and at three rows in bytes."""
    arr = (ka._Weight * 1)(weight_struct(ka.Q6K, 0, 151936, 4096))
    assert ka.lib().kh_qmatmul_workspace(arr, 1, 4096, 1, 0) > 0
    assert ka.lib().kh_qmatmul_workspace(arr, 1, 4096, 3, ka.BYTE_ACTIVATIONS) > 0


def test_infer_mirrors_the_reference():
    """QuantizedMatmul::infer (kapel-ops/src/matmul.rs:105-150) on host tensors."""
    op = ka.QuantizedMatmul()
    w = ka.quantized(synth.normal(1, 5 * 256, 0.02).reshape(5, 256), ka.Q4K)
    x = torch.zeros((2, 3, 256))
    assert op.infer([x, w]) == ((2, 3, 5), torch.float32)
    w2 = ka.quantized(synth.normal(2, 3 * 256, 0.02).reshape(3, 256), ka.Q8_0)
    assert op.infer([x, w, w2]) == ((2, 3, 8), torch.float32)
    with pytest.raises(ka.Arity):
        op.infer([x])
    with pytest.raises(ka.InvalidArgument):
        op.infer([torch.zeros((2, 128)), w])
    with pytest.raises(ka.UnsupportedDType):
        op.infer([torch.zeros((2, 256), dtype=torch.int32), w])
    with pytest.raises(ka.UnsupportedDType):
        op.infer([x, torch.zeros((5, 256))])
    bad = ka.QuantizedTensor(w.data, ka.Q4K, 0, 5, 200)
    with pytest.raises(ka.BlockMisaligned):
        op.infer([torch.zeros((1, 200)), bad])


def expert_call(w, experts, k, tokens, topk, per_route=0, kind=ka.F32, x=8192, idx=8192, out=8192):
    return ka.lib().kh_expert_matmul(ctypes.byref(w), experts, k, kind, x, tokens, topk, per_route,
                                     idx, ka.F32, out, 0, None, 0, None)


def test_the_experts_abi_refuses_what_infer_refuses():
    """kapel-ops/src/experts.rs:166-225, as status codes before any device call."""
    w = weight_struct(ka.Q4K, 0, 4 * 7, 512)
    assert expert_call(weight_struct(99, 0, 28, 512), 4, 512, 5, 3) == ka.KH_ERR_DTYPE
    assert expert_call(w, 0, 512, 5, 3) == ka.KH_ERR_SHAPE            # no experts
    assert expert_call(w, 3, 512, 5, 3) == ka.KH_ERR_SHAPE            # 28 rows for 3
    assert expert_call(weight_struct(ka.Q4K, 0, 28, 500), 4, 500, 5, 3) == ka.KH_ERR_MISALIGNED
    assert expert_call(w, 4, 512, 5, 3, kind=9) == ka.KH_ERR_DTYPE
    assert expert_call(w, 4, 512, 5, 3, idx=None) == ka.KH_ERR_NULL
    assert expert_call(w, 4, 512, 5, 3, x=None) == ka.KH_ERR_NULL
    # Misaligned activations need the workspace (none given).
    assert expert_call(w, 4, 512, 5, 3, x=8196) == ka.KH_ERR_WORKSPACE
    huge = ka._Weight(ka.Q4K, 0, 4096, (1 << 24) * 144 * 2, 1 << 24)
    assert expert_call(huge, 1, 512, 1, 1) == ka.KH_ERR_OVERFLOW      # 4.8 GB an expert
    # Nothing to do.
    assert expert_call(w, 4, 512, 0, 3) == ka.KH_OK
    assert expert_call(weight_struct(ka.Q4K, 0, 0, 512), 4, 512, 5, 3) == ka.KH_OK
    size = ka.lib().kh_expert_matmul_workspace(ctypes.byref(w), 4, 512, 5, 3, 1, ka.F32, 0)
    assert size >= 5 * 3 * 512 * 4
    assert ka.lib().kh_expert_matmul_workspace(ctypes.byref(w), 3, 512, 5, 3, 1, ka.F32, 0) == 0


def test_expert_infer_mirrors_the_reference():
    op = ka.ExpertMatmul(4)
    w = ka.quantized(synth.normal(3, 28 * 256, 0.02).reshape(28, 256), ka.Q8_0)
    idx = torch.zeros((5, 3), dtype=torch.int64)
    assert op.infer([torch.zeros((5, 256)), w, idx]) == ((5, 3, 7), torch.float32)
    assert op.infer([torch.zeros((5, 3, 256), dtype=torch.bfloat16), w, idx]) == ((5, 3, 7), torch.bfloat16)
    with pytest.raises(ka.Arity):
        op.infer([torch.zeros((5, 256)), w])
    with pytest.raises(ka.InvalidArgument):
        op.infer([torch.zeros((4, 256)), w, idx])
    with pytest.raises(ka.InvalidArgument):
        ka.ExpertMatmul(3).infer([torch.zeros((5, 256)), w, idx])
    with pytest.raises(ka.InvalidArgument):
        op.infer([torch.zeros((5, 256)), w, idx.float()])
    with pytest.raises(ka.UnsupportedDType):
        op.infer([torch.zeros((5, 256)), torch.zeros((28, 256)), idx])
    with pytest.raises(ka.IndexOutOfRange):
        op.check([0, 3, 4])
    op.check([0, 3, 1])
