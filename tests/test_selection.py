"""The selection report (accel_int4_select / accel_hip_last_selection), the
analogue of the reference's KernelSelection{Op, Kernel, Reason, Rejected}
(tensor/compile.go:36-42) as Plan.Selections reports it (tensor/plan.go:36-41).

On the CPU: every shape the GPU parity tests run (SHAPES_F32, SHAPES_BF16) is
planned for the modelled MI355X without a GPU, and the launches it becomes are
checked against the route each shape is in those lists to exercise, written
out here by hand; the alignment fallbacks (bf16 rows that are not 16-byte
aligned, f32 rows the matrix cores cannot load) are named as such; a choice
says what it turned down (tensor/quantized_test.go:353-365 holds the reference
to the same).  The GPU test (tests/test_gpu_selection.py) checks that what a
product launches is what the plan says."""
import re

import pytest

import accel_amd as A
from test_gpu_int4 import SHAPES_BF16, SHAPES_F32

ALIGNED = 1 << 20

DEC1 = "int4_decode_f32_kernel"
MF = "int4_decode_mfma_kernel"

# (M, K, N) -> the launches, by kernel name with template arguments, in order
F32_ROUTES = {
    (1, 4096, 4096): [f"{DEC1}<1, 256, 32, false, float>"],
    (1, 128, 128): [f"{DEC1}<1, 128, 32, false, float>"],
    (1, 200, 20): ["int4_generic_f32_kernel"],
    (1, 256, 4): ["int4_generic_f32_kernel"],
    (1, 4096, 14336): [f"{DEC1}<1, 512, 32, false, float>"],
    (1, 1000, 384): [f"{DEC1}<1, 128, 32, false, float>"],
    (2, 512, 1024): [f"{MF}<1, 8, float>"],
    (3, 256, 640): [f"{MF}<1, 8, float>"],
    (5, 200, 20): ["int4_generic_f32_kernel"],
    (7, 384, 256): [f"{MF}<1, 8, float>"],
    (8, 4096, 1024): [f"{MF}<1, 8, float>"],
    (13, 200, 20): ["int4_generic_f32_kernel"],
    (16, 4096, 14336): [f"{MF}<2, 8, float>"],
    (17, 256, 512): ["int4_gemm_f32x3_kernel"],
    (64, 512, 256): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
    (65, 320, 384): ["int4_gemm_f32x3_kernel"],
    (3, 200, 640): [f"{DEC1}<3, 128, 16, false, float>"],
    (6, 100, 1024): [f"{DEC1}<6, 256, 8, false, float>"],
    (12, 72, 512): [f"{DEC1}<8, 256, 8, false, float>", f"{DEC1}<4, 256, 16, false, float>"],
    (2, 4100, 1024): [f"{DEC1}<2, 256, 32, false, float>"],
    (1, 4096, 640): [f"{DEC1}<1, 128, 32, false, float>"],
    (2, 4096, 14336): [f"{MF}<2, 8, float>"],
    (2, 1024, 640): [f"{MF}<1, 8, float>"],
    (17, 1024, 8192): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
    (18, 2048, 4096): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
    (40, 8192, 4096): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
    (1, 16640, 256): [f"{DEC1}<1, 256, 32, true, float>"],
    (2, 33000, 128): [f"{DEC1}<2, 128, 32, true, float>"],
    (1, 14336, 4096): [f"{DEC1}<1, 256, 32, false, float>"],
    (1, 2048, 8192): [f"{DEC1}<1, 512, 32, false, float>"],
    (1, 9000, 8704): [f"{DEC1}<1, 512, 32, true, float>"],
    (4, 4096, 4096): [f"{MF}<2, 8, float>"],
    (9, 1024, 384): [f"{MF}<1, 8, float>"],
    (11, 2048, 768): [f"{MF}<1, 8, float>"],
    (15, 14336, 4096): [f"{MF}<1, 8, float>"],
    (16, 96, 256): [f"{MF}<1, 8, float>"],
    (6, 32, 128): [f"{MF}<1, 8, float>"],
    (10, 4096, 1024): [f"{MF}<1, 8, float>"],
    (8, 4096, 4096): [f"{MF}<1, 8, float>"],
    (8, 14336, 4096): [f"{MF}<1, 8, float>"],
    (257, 64, 128): ["int4_gemm_f32x3_kernel"],
    (128, 1024, 512): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
    (300, 2048, 1024): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
    (40, 96, 256): ["int4_gemm_f32_kernel"],
    (64, 4096, 4096): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
    (33, 1088, 256): ["int4_gemm_f32x3_kernel", "int4_gemm_reduce_kernel"],
}

BF = "int4_gemm_bf16_kernel"
SK = "int4_gemm_bf16_splitk_kernel"
RED = "int4_gemm_reduce_kernel"
BF16_ROUTES = {
    (1, 64, 128): [f"{DEC1}<1, 128, 32, false, unsigned short>"],
    (64, 256, 256): [f"{BF}<2, false>"],
    (100, 512, 384): [f"{SK}<4>", RED],
    (128, 128, 128): [f"{BF}<4, false>"],
    (1, 4096, 14336): [f"{DEC1}<1, 512, 32, false, unsigned short>"],
    (2, 4096, 14336): [f"{MF}<2, 8, unsigned short>"],
    (8, 1024, 640): [f"{MF}<1, 8, unsigned short>"],
    (16, 2048, 4096): [f"{MF}<1, 8, unsigned short>"],
    (5, 96, 256): [f"{MF}<1, 8, unsigned short>"],
    (257, 1024, 640): [f"{SK}<8>", f"{SK}<1>", RED],
    (512, 2048, 1024): [f"{SK}<8>", RED],
    (300, 64, 128): [f"{BF}<8, false>", f"{BF}<2, false>"],
    (256, 192, 384): [f"{BF}<8, false>"],
    (511, 320, 256): [f"{BF}<8, false>", f"{BF}<8, false>"],
    (832, 128, 256): [f"{BF}<8, false>", f"{BF}<2, false>"],
    (97, 64, 256): [f"{BF}<4, false>"],
    (200, 256, 128): [f"{BF}<7, false>"],
    (480, 128, 128): [f"{BF}<8, false>", f"{BF}<7, false>"],
    (64, 4096, 4096): [f"{SK}<2>", RED],
    (17, 4096, 1024): [f"{SK}<1>", RED],
    (96, 1088, 256): [f"{SK}<3>", RED],
}


def _names(sel):
    return [re.sub(r" \[.*\]$", "", k) for k in sel.launches]


def test_every_gpu_shape_has_an_expected_route():
    assert set(F32_ROUTES) == set(SHAPES_F32)
    assert set(BF16_ROUTES) == set(SHAPES_BF16)


@pytest.mark.parametrize("M,K,N", SHAPES_F32)
def test_f32_routes(M, K, N):
    sel = A.select(M, K, N, A.F32, a=ALIGNED, codes=ALIGNED)
    assert _names(sel) == F32_ROUTES[(M, K, N)], sel
    assert sel.op == ("Int4MatVec" if M == 1 else "Int4MatMul")
    assert sel.reason


@pytest.mark.parametrize("M,K,N", SHAPES_BF16)
def test_bf16_routes(M, K, N):
    sel = A.select(M, K, N, A.BF16, a=ALIGNED, codes=ALIGNED)
    assert _names(sel) == BF16_ROUTES[(M, K, N)], sel
    assert sel.reason


def test_unaligned_bf16_rows_take_the_per_element_kernel_and_say_why():
    sel = A.select(2048, 4096, 4096, A.BF16, a=ALIGNED + 2, codes=ALIGNED)
    assert _names(sel) == ["int4_generic_bf16_kernel"]
    assert any("not 16-byte aligned" in r for r in sel.rejected), sel
    # aligned, the same product is the matrix-core tiles
    assert _names(A.select(2048, 4096, 4096, A.BF16, a=ALIGNED)) == [f"{BF}<8, false>"]


def test_unaligned_f32_rows_leave_the_matrix_cores():
    # 2..16 rows: the VALU decode kernel instead of the matrix-core one
    sel = A.select(8, 4096, 4096, A.F32, a=ALIGNED + 4)
    assert _names(sel) == [f"{DEC1}<8, 256, 8, true, float>"]   # two batches a slice
    assert "not 16-byte aligned" in sel.reason
    # more rows: the fp32 VALU tiles, naming the matrix-core tiles' condition
    sel = A.select(2048, 4096, 4096, A.F32, a=ALIGNED + 4)
    assert _names(sel) == ["int4_gemm_f32_kernel"]
    assert any("f32 matrix-core tiles" in r and "aligned" in r for r in sel.rejected), sel


def test_unaligned_codes_leave_the_decode_kernels():
    sel = A.select(1, 4096, 4096, A.F32, codes=ALIGNED + 4)
    assert _names(sel) == ["int4_generic_f32_kernel"]
    assert any("decode kernels" in r for r in sel.rejected), sel


def test_a_choice_names_what_it_turned_down():
    # a decode product of several rows turned down the prefill tiles
    sel = A.select(16, 4096, 14336)
    assert any("matrix-core tiles" in r for r in sel.rejected), sel
    # a prefill turned down the decode kernels
    sel = A.select(2048, 4096, 4096)
    assert any("decode kernels" in r for r in sel.rejected), sel


def test_the_grid_is_reported():
    sel = A.select(1, 4096, 4096)
    assert sel.launches == [f"{DEC1}<1, 256, 32, false, float> [16 tiles x 16 K slices]"]
    sel = A.select(2048, 4096, 4096, A.BF16)
    assert sel.launches == [f"{BF}<8, false> [256 tiles]"]


def test_the_fused_linear_bias_is_in_the_kernel_name():
    sel = A.select(2048, 4096, 4096, A.BF16, op="Int4Linear", flags=A.SELECT_BIAS)
    assert sel.op == "Int4Linear"
    assert _names(sel) == [f"{BF}<8, true>"]


def test_noalloc_answers_before_a_capture():
    sel = A.select(1, 4096, 14336, op="Int4MatVecNoAlloc")
    assert _names(sel) == [f"{DEC1}<1, 512, 32, false, float>"]
    # the LM head's split-K sums (16 slices x 128256 columns) exceed the static scratch
    with pytest.raises(A.Refused, match="static scratch holds"):
        A.select(1, 4096, 128256, op="Int4MatVecNoAlloc")


def test_empty_products_launch_nothing():
    sel = A.select(0, 4096, 4096)
    assert sel.launches == [] and "empty" in sel.reason


PR = "int4_panel_rows_kernel"


@pytest.mark.parametrize("M,K,names", [
    (1, 4096, ["int4_panel_matvec_kernel<4, false, true, true, false>"]),
    (2, 4096, [f"{PR}<2, 2, true, false>"]),
    (3, 4096, [f"{PR}<4, 2, true, false>"]),
    (8, 14336, [f"{PR}<8, 2, true, false>"]),
    (8, 1002, [f"{PR}<8, 2, false, false>"]),
    (17, 4096, [f"{PR}<8, 2, true, false>"] * 2 + [f"{PR}<2, 2, true, false>"]),
])
def test_prepared_rows_routes(M, K, names):
    """Int4MatMulPrepared: one row on the one-row panel kernel, 2..8 rows in
    one launch of the rows kernel (rows rounded up to 2, 4 or 8), more in
    passes of eight."""
    sel = A.select(M, K, 4096, A.F32, a=ALIGNED, op="Int4MatMulPrepared")
    assert _names(sel) == names, sel
    assert sel.op == "Int4MatMulPrepared" and sel.reason and sel.rejected


def test_prepared_rows_need_even_k_and_aligned_rows():
    with pytest.raises(A.Refused, match="K even"):
        A.select(2, 1001, 4096, A.F32, a=ALIGNED, op="Int4MatMulPrepared")
    with pytest.raises(A.Refused, match="K even"):
        A.select(2, 4096, 4096, A.F32, a=ALIGNED + 4, op="Int4MatMulPrepared")
