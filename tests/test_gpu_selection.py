"""What an int4 product launches is what its plan says: for every shape the
parity tests run, the device's last selection after the product
(accel_hip_last_selection, recorded as the kernels are launched) equals the
selection planned without running (accel_int4_select on the same device and
the same addresses), kernel names, grids, reason and rejections alike.  The
planned routes themselves are pinned on the CPU (tests/test_selection.py)."""
import numpy as np
import pytest

import accel_amd as A
from accel_amd import BF16, F32
from test_gpu_int4 import SHAPES_BF16, SHAPES_F32

pytestmark = pytest.mark.gpu


def _zero_weights(dev, K, N):
    n = K * N
    return dev.upload_int4(np.zeros((n + 7) // 8, np.uint32),
                           np.zeros((n + 127) // 128, np.uint16),
                           np.zeros((n + 127) // 128, np.uint16), n)


def _same(got, want):
    assert got.op == want.op
    assert got.kernel == want.kernel
    assert got.reason == want.reason
    assert got.rejected == want.rejected


def _check(dev, M, K, N, dtype, a_off=0):
    w = _zero_weights(dev, K, N)
    esz = 4 if dtype == F32 else 2
    base = dev.alloc((M * K + 16,), dtype)
    a = A.Buffer(dev, base.ptr + a_off, M * K * esz, dtype, (M, K) if M > 1 else (K,))
    out = dev.alloc((M, N) if M > 1 else (N,), dtype)
    if M == 1 and dtype == F32:
        dev.Int4MatVec(a, w, out)
    else:
        a.shape = (M, K)
        out.shape = (M, N)
        dev.Int4MatMul(a, w, out)
    dev.sync()
    got = dev.last_selection()
    want = A.select(M, K, N, dtype, a=a.ptr, codes=w.codes.ptr,
                    op="Int4MatVec" if (M == 1 and dtype == F32) else "Int4MatMul",
                    dev=dev.index)
    _same(got, want)
    assert got.launches, got
    base.free()
    out.free()
    w.free()
    return got


@pytest.mark.parametrize("M,K,N", SHAPES_F32)
def test_f32_launches_are_the_plan(dev, M, K, N):
    _check(dev, M, K, N, F32)


@pytest.mark.parametrize("M,K,N", SHAPES_BF16)
def test_bf16_launches_are_the_plan(dev, M, K, N):
    _check(dev, M, K, N, BF16)


def test_unaligned_bf16_rows_run_the_per_element_kernel(dev):
    sel = _check(dev, 64, 256, 256, BF16, a_off=2)
    assert sel.launches == ["int4_generic_bf16_kernel"]


def test_sets_and_noalloc_report_their_launches(dev):
    K = 4096
    ws = [_zero_weights(dev, K, n) for n in (4096, 1024, 1024)]
    a = dev.upload(np.zeros(K, np.float32))
    outs = [dev.alloc((n,), F32) for n in (4096, 1024, 1024)]
    dev.Int4MatVecSet(a, ws, outs)
    dev.sync()
    sel = dev.last_selection()
    assert sel.op == "Int4MatVecSet"
    assert all(k.startswith("int4_decode_set_kernel<") for k in sel.launches), sel
    dev.Int4MatVecNoAlloc(a, ws[0], outs[0])
    dev.sync()
    sel = dev.last_selection()
    want = A.select(1, K, 4096, F32, a=a.ptr, codes=ws[0].codes.ptr, op="Int4MatVecNoAlloc",
                    dev=dev.index)
    _same(sel, want)
    for b in outs + [a]:
        b.free()
    for w in ws:
        w.free()
