"""The ``ops_sparse`` / ``ops_sparse_test`` operators on the GPU: the known-answer cases of the
reference's bridge test (torch_npu/test_spmv_npu.py:37-113), on a ROCm device."""
import pytest
import torch

import ops_sparse  # noqa: F401  (defines the operators)

pytestmark = pytest.mark.gpu


def _csr(dtype, dev):
    row_ptr = torch.tensor([0, 2, 3], dtype=torch.int32, device=dev)
    col_ind = torch.tensor([0, 2, 1], dtype=torch.int32, device=dev)
    values = torch.tensor([2, 3, 4], dtype=dtype, device=dev)
    return torch.sparse_csr_tensor(row_ptr, col_ind, values, size=(2, 3), device=dev), row_ptr, col_ind, values


@pytest.mark.parametrize("entry", ["mv", "spmv"])
def test_csr_times_vector(entry, dev):
    matrix, _, _, _ = _csr(torch.float32, dev)
    vector = torch.tensor([1.0, 2.0, 3.0], device=dev)
    fn = torch.mv if entry == "mv" else torch.ops.ops_sparse.spmv
    result = fn(matrix, vector)
    assert result.is_cuda
    torch.testing.assert_close(result.cpu(), torch.tensor([11.0, 8.0]), rtol=0, atol=0)


@pytest.mark.parametrize("length", [2, 4])
@pytest.mark.parametrize("entry", ["mv", "spmv"])
def test_rejects_short_and_long_vectors(length, entry, dev):
    matrix, _, _, _ = _csr(torch.float32, dev)
    vector = torch.arange(1, length + 1, dtype=torch.float32, device=dev)
    fn = torch.mv if entry == "mv" else torch.ops.ops_sparse.spmv
    with pytest.raises(RuntimeError, match="SpMV matrix columns must equal vector length"):
        fn(matrix, vector)


def test_hook_updates_y_in_place(dev):
    _, row_ptr, col_ind, values = _csr(torch.float32, dev)
    x = torch.tensor([1.0, 2.0, 3.0], device=dev)
    y = torch.tensor([5.0, 6.0], device=dev)
    returned = torch.ops.ops_sparse_test.spmv_npu(row_ptr, col_ind, values, x, y, 2.0, 3.0, "N", 0)
    assert returned.data_ptr() == y.data_ptr()
    torch.testing.assert_close(y.cpu(), torch.tensor([37.0, 34.0]), rtol=0, atol=0)


def test_fp16_csr(dev):
    matrix, _, _, _ = _csr(torch.float16, dev)
    vector = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float16, device=dev)
    result = torch.mv(matrix, vector)
    assert result.dtype == torch.float16
    torch.testing.assert_close(result.cpu().float(), torch.tensor([11.0, 8.0]), rtol=0, atol=0)


def test_complex_conjugate_transpose_hook(dev):
    row_ptr = torch.tensor([0, 2, 3], dtype=torch.int32, device=dev)
    col_ind = torch.tensor([0, 1, 1], dtype=torch.int32, device=dev)
    values = torch.tensor([1 + 2j, 3 - 1j, 2 + 4j], dtype=torch.complex64, device=dev)
    x = torch.tensor([1 - 1j, 2 + 3j], dtype=torch.complex64, device=dev)
    y = torch.empty(2, dtype=torch.complex64, device=dev)
    result = torch.ops.ops_sparse_test.spmv_npu(row_ptr, col_ind, values, x, y, 1 + 0j, 0 + 0j, "H", 0)
    assert result.data_ptr() == y.data_ptr()
    torch.testing.assert_close(result.cpu(), torch.tensor([-1 - 3j, 20 - 4j], dtype=torch.complex64), rtol=0, atol=0)


@pytest.mark.parametrize("base,ptrs,indices,expected", [
    (0, [0, 3, 5], [2, 0, 2, 1, 0], [-10.25, 4.25, 9.0]),
    (1, [1, 4, 6], [1, 3, 3, 1, 2], [6.0, -14.5, 11.5]),
])
def test_transpose_unsorted_and_duplicate_columns(base, ptrs, indices, expected, dev):
    values = torch.tensor([1.0, 2.0, 3.0, -1.0, 4.0], device=dev)
    x = torch.tensor([2.0, -3.0], device=dev)
    row_ptr = torch.tensor(ptrs, dtype=torch.int32, device=dev)
    col_ind = torch.tensor(indices, dtype=torch.int32, device=dev)
    y = torch.tensor([0.5, -1.0, 2.0], device=dev)
    returned = torch.ops.ops_sparse_test.spmv_npu(row_ptr, col_ind, values, x, y, 1.25, -0.5, "T", base)
    assert returned.data_ptr() == y.data_ptr()
    torch.testing.assert_close(y.cpu(), torch.tensor(expected), rtol=0.0, atol=1e-6)


def test_hook_rejects_int64_indices(dev):
    _, row_ptr, col_ind, values = _csr(torch.float32, dev)
    x = torch.ones(3, device=dev)
    y = torch.zeros(2, device=dev)
    with pytest.raises(RuntimeError, match="int32"):
        torch.ops.ops_sparse_test.spmv_npu(row_ptr.long(), col_ind, values, x, y, 1.0, 0.0, "N", 0)


@pytest.mark.parametrize("dtype", [torch.float64, torch.int64, torch.complex128])
@pytest.mark.parametrize("entry", ["mv", "spmv"])
def test_unsupported_dtypes_raise_runtime_error(dtype, entry, dev):
    """ToAclDataType (torch_npu/spmv_npu.cpp:286-297) rejects every other dtype; importing the
    package replaces PyTorch's CSR mv, so such a call raises instead of computing."""
    matrix, _, _, _ = _csr(dtype, dev)
    vector = torch.tensor([1, 2, 3], dtype=dtype, device=dev)
    fn = torch.mv if entry == "mv" else torch.ops.ops_sparse.spmv
    with pytest.raises(RuntimeError, match="unsupported A5 SpMV tensor dtype"):
        fn(matrix, vector)


def test_hook_rejects_non_integral_and_out_of_range_int32_scalars(dev):
    """MakeScalars (torch_npu/spmv_npu.cpp:108-124): INT32 SpMV takes integral scalars that fit int32."""
    _, row_ptr, col_ind, _ = _csr(torch.float32, dev)
    values = torch.tensor([2, 3, 4], dtype=torch.int8, device=dev)
    x = torch.tensor([1, 2, 3], dtype=torch.int8, device=dev)
    y = torch.tensor([5, 6], dtype=torch.int32, device=dev)
    hook = torch.ops.ops_sparse_test.spmv_npu
    with pytest.raises(RuntimeError, match="must be integral scalars"):
        hook(row_ptr, col_ind, values, x, y, 2.5, 1, "N", 0)
    with pytest.raises(RuntimeError, match="must be integral scalars"):
        hook(row_ptr, col_ind, values, x, y, 2, 1.0, "N", 0)
    with pytest.raises(RuntimeError, match="must fit int32"):
        hook(row_ptr, col_ind, values, x, y, 2**31, 1, "N", 0)
    torch.testing.assert_close(y.cpu(), torch.tensor([5, 6], dtype=torch.int32))  # untouched
    hook(row_ptr, col_ind, values, x, y, 2, 3, "N", 0)
    torch.testing.assert_close(y.cpu(), torch.tensor([2 * 11 + 15, 2 * 8 + 18], dtype=torch.int32))


def test_hook_rejects_complex_scalars_for_real_compute(dev):
    _, row_ptr, col_ind, values = _csr(torch.float32, dev)
    x = torch.tensor([1.0, 2.0, 3.0], device=dev)
    y = torch.tensor([5.0, 6.0], device=dev)
    with pytest.raises(RuntimeError, match="real SpMV compute type cannot use a complex scalar"):
        torch.ops.ops_sparse_test.spmv_npu(row_ptr, col_ind, values, x, y, complex(2, 1), 3.0, "N", 0)
