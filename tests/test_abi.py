"""The C ABI library on the CPU: exported symbols, argument checks, host-side bookkeeping.

No kernel runs here; every call below returns before touching a device (or reports that
none is present).
"""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "qmsg.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(qmsg_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(os.path.join(ROOT, "large_model_amd", "libqmsg.so"))
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


def create(q, E, X, K, F, layers=1, tmax=4):
    cfg = q._Cfg(E, X, K, F)
    h = ctypes.c_void_p()
    st = q.lib.qmsg_create(ctypes.byref(h), 0, ctypes.byref(cfg), layers, tmax)
    return st, h, q.lib.qmsg_last_error(None).decode()


@pytest.mark.parametrize("shape", [(0, 16, 4, 128), (256, 16, 0, 128), (256, 4, 8, 128), (256, 16, 4, -1)])
def test_create_rejects_bad_shapes(q, shape):
    st, h, msg = create(q, *shape)
    assert st == -1 and not h.value and "bad shape" in msg


@pytest.mark.parametrize("shape", [(300, 16, 4, 128), (256, 16, 4, 80), (256, 512, 8, 128), (256, 80, 72, 128)])
def test_create_reports_unsupported_shapes(q, shape):
    """Rows that are not whole 32-blocks (n_embd 300, n_ff_exp 80: no qms_matmul int8 path,
    src/quant.c:134-136), more than 256 experts or more than 64 of them per token."""
    st, h, msg = create(q, *shape)
    assert st == -2 and not h.value and "unsupported" in msg


@pytest.mark.parametrize("shape", [(256, 8, 2, 128), (256, 20, 4, 128), (1024, 60, 4, 256), (96, 8, 2, 96),
                                   (256, 16, 4, 96), (2080, 64, 8, 352)])
def test_create_takes_any_expert_count(q, shape):
    """Expert counts that are not a multiple of 16 (Mixtral's 8, 60) and rows of whole 32-blocks
    off the integer kernels' grid (n_embd % 256 != 0, n_ff_exp = 32 x odd) pass the shape gate;
    here, without a device, creation then fails on the device, not on the shape."""
    st, h, msg = create(q, *shape)
    assert st != -2 and "unsupported" not in msg
    if st == 0:
        q.lib.qmsg_destroy(h)


def test_create_null_and_destroy_null(q):
    assert q.lib.qmsg_create(None, 0, None, 1, 1) == -1
    q.lib.qmsg_destroy(None)
    assert q.lib.qmsg_moe(None, 0, None, None, 1, None) == -1
    assert q.lib.qmsg_set_path(None, 0) == -1


def test_create_without_a_device(q):
    from conftest_gpu import gpu_available
    if gpu_available():
        pytest.skip("a GPU is present")
    st, h, msg = create(q, 256, 16, 4, 128)
    assert st == -4 and "not available" in msg


def test_row_bytes_match_gguf():
    """qms_row_bytes (src/gguf.c:85-96) in the binding and the oracle."""
    import oracle as orc
    from large_model_amd.qmsg import row_bytes
    for t in (0, 1, 2, 3, 8, 14):
        for n in (32, 96, 256, 4096, 1536, 300):
            assert row_bytes(t, n) == orc.row_bytes(t, n)


def test_q8_record_layout(q):
    import oracle as orc
    assert q.Q8_DTYPE == orc.Q8_DTYPE and q.Q8_DTYPE.itemsize == 44


def test_workload_byte_counts():
    from large_model_amd.workloads import WORKLOADS
    w = WORKLOADS["q235b_decode_t1"]
    assert w.gate_bytes == 3_538_944 and w.expert_bytes == 10_616_832
    assert w.layer_bytes(8) == 87_064_576
    assert WORKLOADS["q30b_decode_t1"].layer_bytes(8) == 22_298_624
    assert WORKLOADS["tiny"].layer_bytes(4) == 239_616
    assert WORKLOADS["q235b_prefill_t512"].int8_ops() == 154_618_822_656


def test_zipf_targets_and_bias():
    from large_model_amd.workloads import zipf_bias, zipf_targets
    c = zipf_targets(128, 8, 512)
    assert abs(c.sum() - 4096) < 1e-6 and c.max() <= 512 and np.all(np.diff(c) <= 1e-9)
    b1, b2 = zipf_bias(128, 8, 512, 4096), zipf_bias(128, 8, 512, 4096)
    assert np.array_equal(b1, b2) and b1.dtype == np.float32 and b1.max() == 0.0
