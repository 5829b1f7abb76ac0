"""GPU parity of aclsparseSpMV (through the C ABI) against the CPU oracle and the reference KATs."""
import ctypes
import json
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close, host_bits, oracle_result
from ops_sparse import _lib, spmv_npu
from ops_sparse._lib import DataType, IndexBase, Operation, PointerMode, SpMVAlg, Status
from ops_sparse.spmv import CsrDescr, CsrSpMV, DnVecDescr, Handle, HostScalar
from ops_sparse import workloads as wl

pytestmark = pytest.mark.gpu

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
ALG = {"DEFAULT": SpMVAlg.DEFAULT, "CSR_ALG1": SpMVAlg.CSR_ALG1, "CSR_ALG2": SpMVAlg.CSR_ALG2}
OP = {"N": Operation.NON_TRANSPOSE, "T": Operation.TRANSPOSE, "H": Operation.CONJUGATE_TRANSPOSE}


def run_workload(w, dev, alg=SpMVAlg.DEFAULT, preprocess=True):
    w = w.to(dev)
    y = w.y0.to(w.out_dtype).clone()
    op = OP[w.trans]
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=op, alg=alg)
    if preprocess:
        plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    return w, y, plan


def t(data, dtype, dev):
    return torch.tensor(data, dtype=dtype, device=dev)


# --------------------------- reference KATs ---------------------------------

@pytest.mark.parametrize("case", KATS["csv_cases"], ids=lambda c: c["name"])
def test_reference_csv_three_stage_and_reexecute(case, dev):
    rp = t(case["row_ptr"], torch.int32, dev)
    ci = t(case["col_ind"], torch.int32, dev)
    va = t(case["values"], torch.float32, dev)
    x = t(case["x"], torch.float32, dev)
    y = t(case["y"], torch.float32, dev)
    op = OP[case["op"]]
    plan = CsrSpMV(case["rows"], case["cols"], rp, ci, va, x, y, case["alpha"], case["beta"], op=op,
                   base=case["base"], alg=ALG[case["alg"]])
    assert plan.buffer_size >= 64 and plan.buffer_size % 64 == 0
    if case["pointer_mode"] == "DEVICE":
        plan.handle.set_pointer_mode(PointerMode.DEVICE)
        da = t([case["alpha"]], torch.float32, dev)
        db = t([case["beta"]], torch.float32, dev)
        plan.alpha = type("P", (), {"ptr": ctypes.c_void_p(da.data_ptr())})()
        plan.beta = type("P", (), {"ptr": ctypes.c_void_p(db.data_ptr())})()
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), case["expected_first"], atol=case["tolerance"], rtol=0)
    plan.run()  # same pattern and workspace: still valid for a second call
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), case["expected_second"], atol=case["tolerance"], rtol=0)


def test_reference_zero_nnz_beta_and_misaligned_workspace(dev):
    k = KATS["zero_nnz_beta"]
    rp = t(k["row_ptr"], torch.int32, dev)
    x = t(k["x"], torch.float32, dev)
    y = t(k["y"], torch.float32, dev)
    empty_i = torch.empty(0, dtype=torch.int32, device=dev)
    empty_f = torch.empty(0, dtype=torch.float32, device=dev)
    plan = CsrSpMV(k["rows"], k["cols"], rp, empty_i, empty_f, x, y, k["alpha"], k["beta"])
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), k["expected"])
    lib = _lib.lib()
    st = lib.aclsparseSpMV(plan.handle.h, 0, plan.alpha.ptr, plan.mat.d, plan.x.d, plan.beta.ptr, plan.y.d,
                           int(DataType.FLOAT), 0, ctypes.c_void_p(plan.workspace.data_ptr() + 1))
    assert st == Status.INVALID_VALUE


def test_reference_repeated_coordinates(dev):
    k = KATS["repeated_coordinates"]
    y = t(k["y"], torch.float32, dev)
    plan = CsrSpMV(1, 1, t(k["row_ptr"], torch.int32, dev), t(k["col_ind"], torch.int32, dev),
                   t(k["values"], torch.float32, dev), t(k["x"], torch.float32, dev), y, k["alpha"], k["beta"],
                   alg=ALG[k["alg"]])
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    assert y.item() == k["expected"][0]


@pytest.mark.parametrize("alg", ["DEFAULT", "CSR_ALG1", "CSR_ALG2"])
@pytest.mark.parametrize("mode", ["HOST", "DEVICE"])
def test_reference_golden_precision_on_the_device(alg, mode, dev):
    """{2^24, 1, -2^24} . {1, 1, 1} = 1 exactly (test/spmv/arch22/spmv_test.cpp:350-361).  A plain fp32
    sum gives 0; the reference device sums matrices of at most 64 rows with Kahan compensation and an
    FMA product residual (sparse/spmv/arch35/spmv_kernel.cpp:448-499), and so does this build."""
    k = KATS["golden_precision"]
    y = t([7.0], torch.float32, dev)
    plan = CsrSpMV(1, 3, t(k["row_ptr"], torch.int32, dev), t(k["col_ind"], torch.int32, dev),
                   t(k["values"], torch.float32, dev), t(k["x"], torch.float32, dev), y, 1.0, 0.0,
                   alg=ALG[alg])
    if mode == "DEVICE":
        plan.handle.set_pointer_mode(PointerMode.DEVICE)
        da, db = t([1.0], torch.float32, dev), t([0.0], torch.float32, dev)
        plan.alpha = type("P", (), {"ptr": ctypes.c_void_p(da.data_ptr())})()
        plan.beta = type("P", (), {"ptr": ctypes.c_void_p(db.data_ptr())})()
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    assert y.item() == k["expected"]


@pytest.mark.parametrize("rows", [1, 33, 64, 65])
def test_small_fp32_rows_compensated_up_to_64(rows, dev):
    """Each row holds {2^24, 1, -2^24} (and a tail of ordinary values): up to 64 rows every row comes
    out exact, as on the reference device; from 65 rows on the row kernels run (plain fp32 sums, within
    the 1e-5 row-scaled tolerance).  beta != 0 reads y; a non-finite product takes the plain sum."""
    per = [16777216.0, 1.0, -16777216.0, 0.5]
    rp = torch.arange(0, 4 * rows + 1, 4, dtype=torch.int32)
    ci = torch.tensor([0, 1, 2, 3] * rows, dtype=torch.int32)
    va = torch.tensor(per * rows, dtype=torch.float32)
    x = torch.tensor([1.0, 1.0, 1.0, 2.0])
    y0 = torch.arange(rows, dtype=torch.float32)
    if rows == 33:
        va[4 * 5 + 3] = float("inf")  # row 5: inf * 2 -> the plain sum, inf
    y = y0.to(dev).clone()
    plan = CsrSpMV(rows, 4, rp.to(dev), ci.to(dev), va.to(dev), x.to(dev), y, 2.0, 0.5)
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    got = y.cpu()
    exact = 2.0 * 2.0 + 0.5 * y0  # alpha * (1 + 0.5*2) + beta * y
    if rows <= 64:
        want = exact.clone()
        if rows == 33:
            want[5] = float("inf")
        assert torch.equal(got, want)
    else:
        scale = 2.0 * (2 * 16777216.0 + 2.0) + 0.5 * y0.abs()
        assert float(((got - exact).abs() / scale).max()) <= 1e-5


@pytest.mark.parametrize("op", ["N", "T", "H"])
@pytest.mark.parametrize("alg", ["DEFAULT", "CSR_ALG2"])
@pytest.mark.parametrize("rows", [2, 4096])
def test_reference_int8_saturation(op, alg, rows, dev):
    k = KATS["int8_saturation"]
    rp = [0, 1] + [2] * (rows - 1)
    transpose = op != "N"
    x = torch.full((rows if transpose else 2,), 127, dtype=torch.int8, device=dev)
    y = torch.zeros(2 if transpose else rows, dtype=torch.int32, device=dev)
    plan = CsrSpMV(rows, 2, t(rp, torch.int32, dev), t(k["col_ind"], torch.int32, dev),
                   t(k["values"], torch.int8, dev), x, y, k["alpha"], k["beta"], op=OP[op], alg=ALG[alg])
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert list(got[:2]) == k["expected_head"]
    assert np.all(got[2:] == 0)


def test_reference_fp16_round_half_even(dev):
    k = KATS["fp16_halfway"]
    h = lambda bits: torch.tensor(np.array(bits, dtype=np.uint16).view(np.int16), device=dev).view(torch.float16)
    y = h(k["y_bits"]).clone()
    plan = CsrSpMV(2, 2, t(k["row_ptr"], torch.int32, dev), t(k["col_ind"], torch.int32, dev), h(k["values_bits"]),
                   h(k["x_bits"]), y, k["alpha"], k["beta"])
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    assert list(host_bits(y)) == k["expected_bits"]


def test_reference_complex_conjugate_transpose(dev):
    k = KATS["complex_conj_transpose"]
    c = lambda v: torch.tensor([complex(a, b) for a, b in v], dtype=torch.complex64, device=dev)
    y = c(k["y"])
    plan = CsrSpMV(2, 2, t(k["row_ptr"], torch.int32, dev), t(k["col_ind"], torch.int32, dev), c(k["values"]),
                   c(k["x"]), y, complex(*k["alpha"]), complex(*k["beta"]), op=Operation.CONJUGATE_TRANSPOSE,
                   alg=ALG[k["alg"]])
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), [complex(a, b) for a, b in k["expected"]], atol=1e-6)


def _strided_fixture(rows, is_sorted):
    rp, ci, va = [1], [], []
    for r in range(rows):
        if r % 2 == 0:
            ci += [1, 3] if is_sorted else [3, 1]
            va += [2.0, 3.0] if is_sorted else [3.0, 2.0]
        else:
            ci.append(2)
            va.append(4.0)
        rp.append(len(va) + 1)
    return rp, ci, va


def _with_stride(vals, stride, sentinel):
    out = [sentinel] * (len(vals) * stride)
    out[::stride] = vals
    return out


@pytest.mark.parametrize("case", KATS["strided"]["cases"], ids=lambda c: f"{c['op']}{c['rows']}{c['alg']}{c['sorted']}")
def test_reference_strided_storage_preserves_padding(case, dev):
    k = KATS["strided"]
    s = k["strides"]
    rows, op = case["rows"], case["op"]
    transpose = op != "N"
    rp, ci, va = _strided_fixture(rows, case["sorted"])
    xl = [1.0] * rows if transpose else [1.0, 2.0, 3.0]
    out_len = 3 if transpose else rows
    sent = k["sentinel"]
    d_rp = t(_with_stride(rp, s["row"], k["index_sentinel"]), torch.int32, dev)
    d_ci = t(_with_stride(ci, s["col"], k["index_sentinel"]), torch.int32, dev)
    d_va = t(_with_stride(va, s["val"], sent), torch.float32, dev)
    d_x = t(_with_stride(xl, s["x"], sent), torch.float32, dev)
    y_init = _with_stride([k["y_init"]] * out_len, s["y"], sent)
    d_y = t(y_init, torch.float32, dev)
    lib = _lib.lib()
    h = Handle(torch.cuda.current_stream().cuda_stream or _lib.HIP_NULL_STREAM)
    mat = CsrDescr(rows, 3, d_rp, d_ci, d_va, base=1)
    mat.set_strides(s["row"], s["col"], s["val"])
    vx = DnVecDescr(len(xl), d_x)
    vx.set_stride(s["x"])
    vy = DnVecDescr(out_len, d_y)
    vy.set_stride(s["y"])
    a, b = HostScalar(k["alpha"], DataType.FLOAT), HostScalar(k["beta"], DataType.FLOAT)
    size = ctypes.c_size_t()
    opv, algv = int(OP[op]), int(ALG[case["alg"]])
    assert lib.aclsparseSpMVGetBufferSize(h.h, opv, a.ptr, mat.d, vx.d, b.ptr, vy.d, 0, algv,
                                          ctypes.byref(size)) == 0
    ws = torch.empty(size.value, dtype=torch.uint8, device=dev)
    even, odd = (rows + 1) // 2, rows // 2
    for preprocess in (False, True):
        d_y.copy_(t(y_init, torch.float32, dev))
        if preprocess:
            assert lib.aclsparseSpMVPreprocess(h.h, opv, a.ptr, mat.d, vx.d, b.ptr, vy.d, 0, algv,
                                               ctypes.c_void_p(ws.data_ptr())) == 0
        assert lib.aclsparseSpMV(h.h, opv, a.ptr, mat.d, vx.d, b.ptr, vy.d, 0, algv,
                                 ctypes.c_void_p(ws.data_ptr())) == 0
        torch.cuda.synchronize()
        got = d_y.cpu().numpy()
        texp = [4.0 * even + 15.0, 8.0 * odd + 15.0, 6.0 * even + 15.0]
        for i, v in enumerate(got):
            logical = i // s["y"]
            if i % s["y"]:
                exp = sent
            elif transpose:
                exp = texp[logical]
            else:
                exp = k["expected_n"]["even_row"] if logical % 2 == 0 else k["expected_n"]["odd_row"]
            assert v == pytest.approx(exp, rel=1e-6), (i, v, exp, preprocess)


# --------------------------- workload parity --------------------------------

@pytest.mark.parametrize("name,scale", [("c1", 1), ("c2", 64), ("c3", 64), ("c5", 64)])
def test_config_parity_scaled(name, scale, dev):
    w, y, _ = run_workload(wl.config(name, "cpu", scale), dev)
    print(f"{w.name}: rows={w.rows} nnz={w.nnz} err={assert_close(w, y):.3e}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_config4_lowp_parity_scaled(dtype, dev):
    w, y, _ = run_workload(wl.config("c4", "cpu", 256, dtype=dtype), dev)
    assert_close(w, y)


@pytest.mark.parametrize("name", ["c2", "c3", "c5"])
def test_config_parity_full_size(name, dev):
    w = wl.config(name, dev, 1)
    w, y, _ = run_workload(w, dev)
    print(f"{w.name}: rows={w.rows} nnz={w.nnz} err={assert_close(w.to('cpu'), y):.3e}")


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_config_parity_full_size_reference_sized_workspace(name, dev):
    """CSR_ALG1 on the reference-sized workspace: the row kernels (c3) and the atomic scatter into a
    cols-long accumulator (c5, opA = T), at full size against the oracle."""
    w = wl.config(name, dev, 1)
    w, y, plan = run_workload(w, dev, alg=SpMVAlg.CSR_ALG1)
    rb = 4
    ref = (192 + (w.rows + 1) * rb + 63) // 64 * 64 + (w.cols * 4 if w.trans != "N" else 0)
    assert plan.buffer_size <= 2 * ref
    print(f"{w.name} ALG1: workspace {plan.buffer_size} B (reference formula {ref} B) "
          f"err={assert_close(w.to('cpu'), y):.3e}")


@pytest.mark.parametrize("name,scale,i64", [("c3", 64, False), ("c2", 16, False), ("c5", 64, False),
                                            ("c3", 64, True)])
def test_partition_metadata_bit_exact(name, scale, i64, dev):
    w = wl.config(name, "cpu", scale)
    if i64:
        w.row_ptr = w.row_ptr.to(torch.int64)
    w, y, plan = run_workload(w, dev)
    ws = plan.workspace.cpu().numpy()
    hdr = np.frombuffer(ws[:192].tobytes(), dtype=np.uint64)
    nb, rp_off, bl_off, bn_off = int(hdr[5]), int(hdr[6]), int(hdr[7]), int(hdr[8])
    norm_ref, blocks_ref, bnnz_ref = oracle.partition(w.row_ptr.cpu().numpy(), w.nnz)
    assert nb == oracle.num_blocks(w.rows, w.nnz) and int(hdr[4]) == oracle.items_per_block(w.rows, w.nnz)
    rdt = np.int64 if i64 else np.int32
    rb = 8 if i64 else 4
    norm = np.frombuffer(ws[rp_off:rp_off + rb * (w.rows + 1)].tobytes(), dtype=rdt)
    blocks = np.frombuffer(ws[bl_off:bl_off + 4 * (nb + 1)].tobytes(), dtype=np.int32)
    bnnz = np.frombuffer(ws[bn_off:bn_off + rb * (nb + 1)].tobytes(), dtype=rdt)
    np.testing.assert_array_equal(norm, norm_ref)
    np.testing.assert_array_equal(blocks, blocks_ref)
    np.testing.assert_array_equal(bnnz, bnnz_ref)
    assert np.all(np.diff(blocks) <= 511)
    ts_off, tb_off, max_tasks, long_chunks = int(hdr[13]), int(hdr[14]), int(hdr[15]), int(hdr[12] >> 32)
    if w.trans == "N" and w.values.dtype == torch.float32:
        # the long-block task table (fp32 non-transpose plans)
        start_ref, tblock_ref = oracle.task_table(bnnz_ref, long_chunks)
        assert ts_off and tb_off and long_chunks >= 1 and tblock_ref.size <= max_tasks
        start = np.frombuffer(ws[ts_off:ts_off + 4 * (nb + 1)].tobytes(), dtype=np.int32)
        tblock = np.frombuffer(ws[tb_off:tb_off + 4 * tblock_ref.size].tobytes(), dtype=np.int32)
        np.testing.assert_array_equal(start, start_ref)
        np.testing.assert_array_equal(tblock, tblock_ref)
        if name == "c3":
            assert tblock_ref.size > 0  # power-law rows do produce long blocks
    else:
        assert ts_off == 0 and tb_off == 0


def test_beta_zero_never_reads_y(dev):
    w = wl.config("c2", "cpu", 256)
    w.beta = 0.0
    w.y0 = torch.full_like(w.y0, float("nan"))
    w2, y, _ = run_workload(w, dev)
    w.y0 = torch.zeros_like(w.y0)
    assert_close(w, y)


def test_long_rows_and_empty_rows(dev):
    # one 100k-entry row among short and empty rows: spans many LDS chunks
    lengths = torch.tensor([3, 0, 100000, 0, 0, 7] + [1] * 5000 + [0] * 3000 + [5000], dtype=torch.int64)
    g = torch.Generator().manual_seed(7)
    rp, col = wl.csr_from_lengths(lengths, 200000, g, "cpu")
    n = col.numel()
    w = wl.Workload("long_rows", lengths.numel(), 200000, rp.to(torch.int32), col,
                    torch.rand(n, generator=g) * 2 - 1, torch.rand(200000, generator=g) * 2 - 1,
                    torch.rand(lengths.numel(), generator=g) * 2 - 1, 1.25, -0.75)
    for pre in (True, False):
        w2, y, _ = run_workload(w, dev, preprocess=pre)
        assert_close(w, y)


def test_int64_row_offsets_fp32(dev):
    w = wl.config("c3", "cpu", 128)
    w.row_ptr = w.row_ptr.to(torch.int64)
    w2, y, _ = run_workload(w, dev)
    assert_close(w, y)


def test_no_preprocess_matches_preprocess(dev):
    w = wl.config("c3", "cpu", 128)
    _, y1, _ = run_workload(w, dev, preprocess=False)
    _, y2, _ = run_workload(w, dev, preprocess=True)
    assert torch.equal(y1, y2)


def test_spmv_npu_mirror_and_mv(dev):
    w = wl.config("c1", "cpu")
    d = w.to(dev)
    y = spmv_npu(d.row_ptr, d.col_ind, d.values, d.x, d.y0, w.alpha, w.beta)
    torch.cuda.synchronize()
    assert_close(w, y)
    from ops_sparse import mv
    a = torch.sparse_csr_tensor(d.row_ptr.to(torch.int64), d.col_ind.to(torch.int64), d.values,
                                size=(w.rows, w.cols))
    y2 = mv(a, d.x)
    torch.cuda.synchronize()
    assert torch.equal(y2, y)


def test_torch_mv_dispatches_here(dev):
    # torch.mv(csr, vec) on the GPU runs ops_sparse.mv (aten::mv, SparseCsrCUDA),
    # as the reference's package routes it for the NPU (torch_extension/spmv.py:43-46)
    import ops_sparse  # noqa: F401  (the import registers the kernel)
    w = wl.config("c1", "cpu")
    d = w.to(dev)
    a = torch.sparse_csr_tensor(d.row_ptr.to(torch.int64), d.col_ind.to(torch.int64), d.values,
                                size=(w.rows, w.cols))
    y = torch.mv(a, d.x)
    torch.cuda.synchronize()
    assert torch.equal(y, ops_sparse.mv(a, d.x))
    w0 = wl.Workload(w.name, w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, w.y0, 1.0, 0.0)
    assert_close(w0, y)
    # int8 values: SpMvCsr accumulates and returns int32, which PyTorch's own kernel does not offer
    g = torch.Generator().manual_seed(5)
    v8 = torch.randint(-128, 128, (w.col_ind.numel(),), generator=g, dtype=torch.int8)
    x8 = torch.randint(-128, 128, (w.cols,), generator=g, dtype=torch.int8)
    a8 = torch.sparse_csr_tensor(d.row_ptr.to(torch.int64), d.col_ind.to(torch.int64), v8.to(dev),
                                 size=(w.rows, w.cols))
    y8 = torch.mv(a8, x8.to(dev))
    torch.cuda.synchronize()
    assert y8.dtype == torch.int32
    ref = torch.zeros(w.rows, dtype=torch.int64)
    rp = w.row_ptr.to(torch.int64)
    prod = v8.to(torch.int64) * x8.to(torch.int64)[w.col_ind.to(torch.int64)]
    ref.index_add_(0, torch.repeat_interleave(torch.arange(w.rows), rp[1:] - rp[:-1]), prod)
    assert torch.equal(y8.cpu(), ref.to(torch.int32))


@pytest.mark.parametrize("nnz", [1, 2, 3, 5, 7])
def test_tiny_nnz_counts(nnz, dev):
    # fewer non-zeros than one 16-byte group, and nnz % 4 != 0 tails
    rows, cols = 3, 4
    lengths = torch.tensor([nnz, 0, 0], dtype=torch.int64)
    g = torch.Generator().manual_seed(nnz)
    rp, col = wl.csr_from_lengths(lengths, cols, g, "cpu", distinct=False)
    w = wl.Workload("tiny", rows, cols, rp.to(torch.int32), col, torch.rand(col.numel(), generator=g),
                    torch.rand(cols, generator=g), torch.rand(rows, generator=g), 2.0, 0.5)
    _, y, _ = run_workload(w, dev)
    assert_close(w, y)


@pytest.mark.parametrize("shift", [0, 1, 2, 3])
@pytest.mark.parametrize("tail", [0, 1, 2, 3])
def test_chunk_edges_at_every_alignment(shift, tail, dev):
    """Loads and gathers stop at each chunk's last non-zero: blocks and chunks that start and end at
    every offset within a 16-byte group, multi-chunk blocks, and nnz % 4 tail entries must all be read."""
    g = torch.Generator().manual_seed(100 + 4 * shift + tail)
    body = torch.randint(0, 12, (3000,), generator=g)
    body[::97] = torch.randint(500, 1600, (body[::97].numel(),), generator=g)  # blocks of 1-4 chunks
    lengths = torch.cat([torch.tensor([shift], dtype=torch.int64), body.to(torch.int64)])
    extra = (tail - int(lengths.sum()) % 4) % 4
    lengths = torch.cat([lengths, torch.tensor([extra + 1], dtype=torch.int64)])
    cols = 4096
    rp, col = wl.csr_from_lengths(lengths, cols, g, "cpu", distinct=False)  # exact lengths (repeats allowed)
    n = col.numel()
    assert n % 4 == (tail + 1) % 4
    w = wl.Workload("edges", lengths.numel(), cols, rp.to(torch.int32), col,
                    torch.rand(n, generator=g) * 2 - 1, torch.rand(cols, generator=g) * 2 - 1,
                    torch.rand(lengths.numel(), generator=g) * 2 - 1, -0.5, 1.25)
    _, y, _ = run_workload(w, dev)
    assert_close(w, y)


def test_long_last_row_with_beta(dev):
    # the last row spans many partition windows, so trailing blocks start at row == rows
    lengths = torch.tensor([2] * 300 + [60000], dtype=torch.int64)
    g = torch.Generator().manual_seed(11)
    rp, col = wl.csr_from_lengths(lengths, 100000, g, "cpu")
    n = col.numel()
    w = wl.Workload("long_last", lengths.numel(), 100000, rp.to(torch.int32), col,
                    torch.rand(n, generator=g) * 2 - 1, torch.rand(100000, generator=g) * 2 - 1,
                    torch.rand(lengths.numel(), generator=g) * 2 - 1, 1.0, 3.0)
    norm, blocks, _ = oracle.partition(rp.numpy(), n)
    assert (blocks[:-1] == lengths.numel()).any(), "fixture must produce blocks that start at row == rows"
    _, y, _ = run_workload(w, dev)
    assert_close(w, y)


@pytest.mark.parametrize("op", ["T", "H"])
def test_transpose_by_columns_is_deterministic(op, dev):
    """The column-gather transpose sums every column in a fixed order: two runs agree bit for bit,
    also with a different algorithm id and without Preprocess (reference CSR_ALG2 semantics)."""
    w = wl.config("c5", "cpu", 32)
    if op == "H":
        g = torch.Generator().manual_seed(3)
        w.values = torch.complex(w.values, torch.rand(w.nnz, generator=g) - 0.5)
        w.x = torch.complex(w.x, torch.rand(w.x.numel(), generator=g) - 0.5)
        w.y0 = torch.complex(w.y0, torch.zeros_like(w.y0))
        w.out_dtype = torch.complex64
    w.trans = op
    outs = []
    for alg, pre in ((SpMVAlg.DEFAULT, True), (SpMVAlg.CSR_ALG2, True), (SpMVAlg.DEFAULT, False)):
        _, y, _ = run_workload(w, dev, alg=alg, preprocess=pre)
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    if op == "T":
        assert_close(w, outs[0].to(dev))
    else:
        rp = w.row_ptr.numpy().astype(np.int64)
        z = oracle.spmv_c64(rp, w.col_ind.numpy(), w.values.numpy(), w.x.numpy(), w.y0.numpy(), w.cols, 2,
                            w.alpha, w.beta)
        np.testing.assert_allclose(outs[0].numpy(), z, rtol=1e-4, atol=1e-4)


def test_transpose_skips_entries_outside_the_rows(dev):
    """Row offsets that start past 0 (base 1 with rowPtr[0] = 3): entries before the first row and
    after the last are not part of the matrix."""
    rp = t([3, 5, 6], torch.int32, dev)          # base 1: rows own entries 2..4 (0-based 2,3 and 4)
    ci = t([1, 2, 1, 3, 2, 3], torch.int32, dev)  # entries 0, 1 and 5 are outside the rows
    va = t([100.0, 100.0, 2.0, 3.0, 4.0, 100.0], torch.float32, dev)
    x = t([1.0, 10.0], torch.float32, dev)
    y = t([0.0, 0.0, 0.0], torch.float32, dev)
    plan = CsrSpMV(2, 3, rp, ci, va, x, y, 1.0, 0.0, op=Operation.TRANSPOSE, base=1)
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), [2.0, 40.0, 3.0])


@pytest.mark.parametrize("i64,dtype,beta", [(False, torch.float32, 0.5), (True, torch.float32, 0.0),
                                             (False, torch.float16, 1.0), (True, torch.bfloat16, -0.25)])
def test_long_rows_split_into_tasks(i64, dtype, beta, dev):
    """Rows of thousands of entries are reduced by many waves (one task per chunk) and combined by the
    block's last task; neighbouring short, empty and medium rows inside the same blocks stay exact."""
    g = torch.Generator().manual_seed(11)
    pattern = [0, 3, 60000, 0, 2, 2500, 1, 0, 0, 4097, 5, 130000, 7, 0, 2049, 2048, 2047] + [3] * 3000 + [70000]
    lengths = torch.tensor(pattern, dtype=torch.int64)
    cols = 150000
    rp, col = wl.csr_from_lengths(lengths, cols, g, "cpu")
    n = col.numel()
    vals = (torch.rand(n, generator=g) * 2 - 1).to(dtype)
    x = (torch.rand(cols, generator=g) * 2 - 1).to(dtype)
    w = wl.Workload("tasks", lengths.numel(), cols, rp.to(torch.int64 if i64 else torch.int32), col, vals, x,
                    (torch.rand(lengths.numel(), generator=g) * 2 - 1), 1.5, beta, out_dtype=dtype)
    for pre in (True, False):
        _, y, plan = run_workload(w, dev, preprocess=pre)
        assert_close(w, y)
    # more calls on the same plan and workspace: the arrival counters are reset by each block's last task
    d = w.to(dev)
    for _ in range(3):
        y.copy_(d.y0.to(dtype))
        plan.run()
        torch.cuda.synchronize()
        assert_close(w, y)


def _mixed_lengths(seed, tail):
    """Short, medium, empty and multi-chunk rows, nnz % 4 == tail (exact lengths, repeats allowed)."""
    g = torch.Generator().manual_seed(seed)
    body = torch.randint(0, 10, (6000,), generator=g)
    body[::211] = torch.randint(300, 2500, (body[::211].numel(),), generator=g)
    lengths = torch.cat([body.to(torch.int64), torch.tensor([0, 1, 5000, 3], dtype=torch.int64)])
    extra = (tail - int(lengths.sum()) % 4) % 4
    lengths[-1] += extra
    cols = 3000
    rp, col = wl.csr_from_lengths(lengths, cols, g, "cpu", distinct=False)
    assert col.numel() % 4 == tail
    return g, lengths.numel(), cols, rp, col


@pytest.mark.parametrize("tail", [0, 3])
@pytest.mark.parametrize("i64", [False, True])
def test_int8_stream_rows_bit_exact(tail, i64, dev):
    """int8 values and x, int32 output (int64 accumulation, saturating epilogue) on the row-block
    stream kernel: bit-exact against the oracle, including alpha/beta and int32 saturation."""
    g, rows, cols, rp, col = _mixed_lengths(40 + tail, tail)
    n = col.numel()
    v8 = torch.randint(-128, 128, (n,), generator=g, dtype=torch.int8)
    x8 = torch.randint(-128, 128, (cols,), generator=g, dtype=torch.int8)
    y0 = torch.randint(-2 ** 31, 2 ** 31 - 1, (rows,), generator=g, dtype=torch.int64).to(torch.int32)
    for alpha, beta in ((3, -2), (70000, 1), (1, 0)):
        y = y0.to(dev).clone()
        plan = CsrSpMV(rows, cols, rp.to(torch.int64 if i64 else torch.int32).to(dev), col.to(dev), v8.to(dev),
                       x8.to(dev), y, alpha, beta)
        plan.preprocess()
        plan.run()
        torch.cuda.synchronize()
        ref = oracle.spmv_i8(rp.numpy(), col.numpy(), v8.numpy(), x8.numpy(), y0.numpy(), alpha, beta, cols=cols)
        np.testing.assert_array_equal(y.cpu().numpy(), ref)


@pytest.mark.parametrize("tail", [1, 2])
def test_complex64_stream_rows(tail, dev):
    """complex64 values, x and y on the row-block stream kernel, against the fp64 oracle."""
    g, rows, cols, rp, col = _mixed_lengths(50 + tail, tail)
    n = col.numel()
    cplx = lambda k: torch.complex(torch.rand(k, generator=g) * 2 - 1, torch.rand(k, generator=g) * 2 - 1)
    v, x, y0 = cplx(n), cplx(cols), cplx(rows)
    alpha, beta = complex(1.5, -0.25), complex(0.5, 0.75)
    y = y0.to(dev).clone()
    plan = CsrSpMV(rows, cols, rp.to(torch.int32).to(dev), col.to(dev), v.to(dev), x.to(dev), y, alpha, beta)
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    ref = oracle.spmv_c64(rp.numpy(), col.numpy(), v.numpy(), x.numpy(), y0.numpy(), cols, 0, alpha, beta)
    # row scale |alpha| * sum |a||x| + |beta y|
    rpn = rp.numpy()
    absprod = np.abs(v.numpy()) * np.abs(x.numpy())[col.numpy()]
    scale = abs(alpha) * np.add.reduceat(np.append(absprod, 0.0), rpn[:-1]) * (np.diff(rpn) > 0) + \
        abs(beta) * np.abs(y0.numpy())
    err = np.abs(y.cpu().numpy().astype(np.complex128) - ref) / np.maximum(scale, 1e-30)
    assert err.max() <= 1e-5, float(err.max())


def test_int8_to_fp32_stream_rows(dev):
    """int8 values and x with fp32 compute and output (exact int products, fp32 sums)."""
    g, rows, cols, rp, col = _mixed_lengths(61, 2)
    n = col.numel()
    v8 = torch.randint(-128, 128, (n,), generator=g, dtype=torch.int8)
    x8 = torch.randint(-128, 128, (cols,), generator=g, dtype=torch.int8)
    y0 = torch.rand(rows, generator=g) * 2 - 1
    y = y0.to(dev).clone()
    plan = CsrSpMV(rows, cols, rp.to(torch.int32).to(dev), col.to(dev), v8.to(dev), x8.to(dev), y, 1.5, 0.5)
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    rpn = rp.numpy()
    prod = v8.numpy().astype(np.float64) * x8.numpy().astype(np.float64)[col.numpy()]
    seg = np.add.reduceat(np.append(prod, 0.0), rpn[:-1]) * (np.diff(rpn) > 0)
    absseg = np.add.reduceat(np.append(np.abs(prod), 0.0), rpn[:-1]) * (np.diff(rpn) > 0)
    golden = 1.5 * seg + 0.5 * y0.numpy().astype(np.float64)
    scale = 1.5 * absseg + 0.5 * np.abs(y0.numpy())
    err = np.abs(y.cpu().numpy().astype(np.float64) - golden) / np.maximum(scale, 1e-30)
    assert err.max() <= 1e-5, float(err.max())


def test_real_matrix_complex_output_stream_rows(dev):
    """fp32 values and x with complex64 y and complex alpha/beta, against the fp64 oracle."""
    g, rows, cols, rp, col = _mixed_lengths(62, 1)
    n = col.numel()
    v = torch.rand(n, generator=g) * 2 - 1
    x = torch.rand(cols, generator=g) * 2 - 1
    y0 = torch.complex(torch.rand(rows, generator=g) * 2 - 1, torch.rand(rows, generator=g) * 2 - 1)
    alpha, beta = complex(0.75, 1.25), complex(-0.5, 0.25)
    y = y0.to(dev).clone()
    plan = CsrSpMV(rows, cols, rp.to(torch.int32).to(dev), col.to(dev), v.to(dev), x.to(dev), y, alpha, beta)
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    ref = oracle.spmv_c64(rp.numpy(), col.numpy(), v.numpy(), x.numpy(), y0.numpy(), cols, 0, alpha, beta,
                          val_is_real=True)
    rpn = rp.numpy()
    absprod = np.abs(v.numpy()) * np.abs(x.numpy())[col.numpy()]
    scale = abs(alpha) * np.add.reduceat(np.append(absprod, 0.0), rpn[:-1]) * (np.diff(rpn) > 0) + \
        abs(beta) * np.abs(y0.numpy())
    err = np.abs(y.cpu().numpy().astype(np.complex128) - ref) / np.maximum(scale, 1e-30)
    assert err.max() <= 1e-5, float(err.max())


@pytest.mark.parametrize("per", [9, 12, 16, 17])
def test_rows_of_nine_to_sixteen_entries(per, dev):
    """Blocks of many rows of 9-16 entries take the 16-read one-lane-per-row path (17: the
    whole-wave path); mixed with shorter rows in the same blocks."""
    g = torch.Generator().manual_seed(per)
    lengths = torch.full((20000,), per, dtype=torch.int64)
    lengths[::7] = torch.randint(0, 9, (lengths[::7].numel(),), generator=g)
    rp, col = wl.csr_from_lengths(lengths, 30000, g, "cpu", distinct=False)
    n = col.numel()
    w = wl.Workload("mid_rows", lengths.numel(), 30000, rp.to(torch.int32), col, torch.rand(n, generator=g) * 2 - 1,
                    torch.rand(30000, generator=g) * 2 - 1, torch.rand(lengths.numel(), generator=g) * 2 - 1,
                    1.5, -0.5)
    _, y, _ = run_workload(w, dev)
    assert_close(w, y)
    w.trans = "T"
    w.y0 = torch.rand(30000, generator=g) * 2 - 1
    _, y, _ = run_workload(w, dev)
    assert_close(w, y)


@pytest.mark.parametrize("name,trans", [("c2", "N"), ("c3", "N"), ("c5", "T")])
def test_hip_graph_capture_and_replay(name, trans, dev):
    """aclsparseSpMV enqueues only kernels (no memsets or copies), so a caller can capture it in a
    HIP graph; every replay, with eager work and synchronisations in between, matches eager runs
    bit for bit (long-row task counters are reset by each block's last task)."""
    w = wl.config(name, "cpu", 64)
    w.trans = trans
    d = w.to(dev)
    s = torch.cuda.Stream()
    y = d.y0.clone()
    torch.cuda.synchronize()  # the inputs were written on the default stream
    with torch.cuda.stream(s):
        plan = CsrSpMV(w.rows, w.cols, d.row_ptr, d.col_ind, d.values, d.x, y, w.alpha, w.beta, op=OP[trans])
        plan.preprocess()
    torch.cuda.synchronize()
    y.copy_(d.y0)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        plan.run()
    torch.cuda.synchronize()
    eager = y.clone()
    assert_close(w, eager)
    g = torch.cuda.CUDAGraph()
    y.copy_(d.y0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        plan.run()
    for _ in range(3):
        y.copy_(d.y0)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        with torch.cuda.stream(s):  # eager work between replays
            plan.run()
        torch.cuda.synchronize()


@pytest.mark.parametrize("op", ["N", "T"])
def test_strided_operands_mid_size(op, dev):
    """Strided row offsets, col_ind, values, x and y (the general kernel) on a matrix with short,
    empty and multi-chunk rows: results match the oracle and padding elements are untouched."""
    g = torch.Generator().manual_seed(77)
    lengths = torch.randint(0, 12, (3000,), generator=g)
    lengths[::250] = 1500
    rows, cols = lengths.numel(), 2500
    rp, col = wl.csr_from_lengths(lengths.to(torch.int64), cols, g, "cpu")
    n = col.numel()
    val = torch.rand(n, generator=g) * 2 - 1
    xlen, ylen = (rows, cols) if op == "T" else (cols, rows)
    x = torch.rand(xlen, generator=g) * 2 - 1
    y0 = torch.rand(ylen, generator=g) * 2 - 1
    sr, sc, sv, sx, sy = 2, 3, 2, 2, 3
    sent = -777.0

    def spread(v, s, fill):
        out = torch.full((v.numel() * s,), fill, dtype=v.dtype)
        out[::s] = v
        return out.to(dev)

    d_rp = spread(rp.to(torch.int32), sr, -1)
    d_col = spread(col, sc, -1)
    d_val, d_x, d_y = spread(val, sv, sent), spread(x, sx, sent), spread(y0, sy, sent)
    h = Handle(torch.cuda.current_stream().cuda_stream or _lib.HIP_NULL_STREAM)
    mat = CsrDescr(rows, cols, d_rp[::sr], d_col[::sc], d_val[::sv])
    mat.set_strides(sr, sc, sv)
    vx, vy = DnVecDescr(xlen, d_x[::sx]), DnVecDescr(ylen, d_y[::sy])
    vx.set_stride(sx)
    vy.set_stride(sy)
    a, b = HostScalar(1.25, DataType.FLOAT), HostScalar(-0.5, DataType.FLOAT)
    lib = _lib.lib()
    size = ctypes.c_size_t()
    opv = int(OP[op])
    assert lib.aclsparseSpMVGetBufferSize(h.h, opv, a.ptr, mat.d, vx.d, b.ptr, vy.d, 0, 0, ctypes.byref(size)) == 0
    ws = torch.empty(size.value, dtype=torch.uint8, device=dev)
    assert lib.aclsparseSpMVPreprocess(h.h, opv, a.ptr, mat.d, vx.d, b.ptr, vy.d, 0, 0,
                                       ctypes.c_void_p(ws.data_ptr())) == 0
    assert lib.aclsparseSpMV(h.h, opv, a.ptr, mat.d, vx.d, b.ptr, vy.d, 0, 0, ctypes.c_void_p(ws.data_ptr())) == 0
    torch.cuda.synchronize()
    got = d_y.cpu()
    pad = torch.ones(got.numel(), dtype=torch.bool)
    pad[::sy] = False
    assert torch.all(got[pad] == sent)
    w = wl.Workload("strided", rows, cols, rp.to(torch.int32), col, val, x, y0, 1.25, -0.5, trans=op)
    assert_close(w, got[::sy].contiguous())


@pytest.mark.parametrize("dtype", [torch.float32, torch.complex64])
def test_transpose_groups_spanning_many_rows(dtype, dev):
    """The transpose's product pass reads rows as 8-bit deltas per 256-entry group; groups that
    span more than 255 rows (runs of empty rows) fall back to the int32 row table and per-entry x
    reads. Mixed in one matrix: dense stretches, sparse stretches, a block of empty rows."""
    g = torch.Generator().manual_seed(5)
    lengths = torch.zeros(120000, dtype=torch.int64)
    lengths[:20000] = torch.randint(0, 9, (20000,), generator=g)      # narrow groups
    lengths[20000:80000:397] = 1                                      # one entry per 397 rows
    lengths[80000:80300] = 3
    lengths[100000::1000] = torch.randint(1, 300, (20,), generator=g)  # long rows far apart
    rp, col = wl.csr_from_lengths(lengths, 5000, g, "cpu", distinct=False)
    n = col.numel()
    u = lambda k: torch.rand(k, generator=g) * 2 - 1
    if dtype == torch.complex64:
        val, x, y0 = torch.complex(u(n), u(n)), torch.complex(u(120000), u(120000)), torch.complex(u(5000), u(5000))
        got = _run_complex_t(rp, col, val, x, y0, dev)
        ref = oracle.spmv_c64(rp.numpy(), col.numpy(), val.numpy(), x.numpy(), y0.numpy(), 5000, 1, 1.5, 0.5)
        np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=1e-4 * max(1.0, float(np.abs(ref).max())))
        return
    w = wl.Workload("span", lengths.numel(), 5000, rp.to(torch.int32), col, u(n), u(120000), u(5000), 1.5, -0.5,
                    trans="T")
    _, y, _ = run_workload(w, dev)
    assert_close(w, y)


def _run_complex_t(rp, col, val, x, y0, dev):
    y = y0.to(dev).clone()
    plan = CsrSpMV(rp.numel() - 1, y0.numel(), rp.to(torch.int32).to(dev), col.to(dev), val.to(dev), x.to(dev), y,
                   complex(1.5, 0), complex(0.5, 0), op=OP["T"])
    plan.run()
    torch.cuda.synchronize()
    return y.cpu()


def test_fp16_output_rounding_edges(dev):
    """fp16 y: alpha * (a * x) with a = 1, x = 2 hits chosen fp32 values exactly; each must round to the
    nearest fp16, ties to even: overflow to inf at 65520, the largest half below it, subnormal halves,
    a tie at half the smallest subnormal (to zero) and just above it (to the smallest subnormal)."""
    targets = np.array([70000.0, 65519.0, 65520.0, -65536.0, 1.0e-6, -3.0e-6, 2.0 ** -25, 2.0 ** -25 * 1.0000001,
                        6.0e-5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 0.0], dtype=np.float32)
    n = targets.size
    x = torch.full((n,), 2.0, dtype=torch.float16, device=dev)
    for tv in targets:
        assert np.float32(np.float32(tv / 2) * 2) == tv  # alpha * 2 is exact in fp32
    for i, tv in enumerate(targets):
        y = torch.zeros(n, dtype=torch.float16, device=dev)
        rp = torch.arange(n + 1, dtype=torch.int32, device=dev)
        col = torch.arange(n, dtype=torch.int32, device=dev)
        # one non-zero in row i only: y_i = alpha * 1 * 2
        vals = torch.zeros(n, dtype=torch.float16, device=dev)
        vals[i] = 1.0
        plan = CsrSpMV(n, n, rp, col, vals, x, y, float(np.float32(tv / 2)), 0.0)
        plan.preprocess()
        plan.run()
        torch.cuda.synchronize()
        got = host_bits(y)[i]
        want = np.array([tv], dtype=np.float32).astype(np.float16).view(np.uint16)[0]
        assert got == want, f"{tv!r}: got {got:#06x} want {want:#06x}"


def _complex_laplacian(n, seed, far=0, every=1):
    """The 5-point Laplacian of an n x n grid with complex64 values (plus, with far > 0, one entry `far`
    columns off the diagonal in every `every`-th row)."""
    m = n * n
    i = torch.arange(m, dtype=torch.int64)
    offs = [-n, -1, 0, 1, n]
    r = torch.cat([i] * len(offs) + ([i[::every]] if far else []))
    c = torch.cat([i + o for o in offs] + ([i[::every] + far] if far else []))
    ok = (c >= 0) & (c < m)
    key = torch.unique(r[ok] * m + c[ok])
    r, c = key // m, key % m
    row_ptr = torch.zeros(m + 1, dtype=torch.int64)
    row_ptr[1:] = torch.cumsum(torch.bincount(r, minlength=m), 0)
    g = torch.Generator().manual_seed(seed)
    cplx = lambda k: torch.complex(torch.rand(k, generator=g) * 2 - 1, torch.rand(k, generator=g) * 2 - 1)
    return m, row_ptr, c.to(torch.int32), cplx(c.numel()), cplx(m), cplx(m)


@pytest.mark.parametrize("op,far,every,flag", [(Operation.CONJUGATE_TRANSPOSE, 0, 1, 6), (Operation.TRANSPOSE, 0, 1, 6),
                                                (Operation.TRANSPOSE, 40000, 8, 2),
                                                (Operation.CONJUGATE_TRANSPOSE, 200000, 1, 0)])
def test_complex_banded_transpose_one_pass(op, far, every, flag, dev):
    """complex64 T / H after Preprocess: a banded matrix takes the one-pass kernel over the CSC pattern
    (values gathered by CSR position, x by row, conjugated for H) on rows and positions packed as 16-bit
    offsets (path flag 6); one entry 40 000 columns off the diagonal in every eighth row keeps it banded
    but out of 16-bit reach (flag 2: the 32-bit rows and positions); an entry per row 200 000 columns off
    keeps the product and column passes (flag 0). Each against the fp64 oracle, and bit-identical to the
    same SpMV without Preprocess (the two-pass path: same products, same order)."""
    m, row_ptr, col, v, x, y0 = _complex_laplacian(700, 5 + far, far, every)
    alpha, beta = complex(1.25, -0.5), complex(0.5, 0.25)
    outs = []
    for pre in (True, False):
        y = y0.to(dev).clone()
        plan = CsrSpMV(m, m, row_ptr.to(torch.int32).to(dev), col.to(dev), v.to(dev), x.to(dev), y, alpha, beta,
                       op=op)
        if pre:
            plan.preprocess()
            torch.cuda.synchronize()
            h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
            assert int(h[16] & 0xFFFFFFFF) == flag
        plan.run()  # after Preprocess synchronised: on the host's copy of the choice
        torch.cuda.synchronize()
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1])
    mode = 2 if op == Operation.CONJUGATE_TRANSPOSE else 1
    z = oracle.spmv_c64(row_ptr.numpy(), col.numpy(), v.numpy(), x.numpy(), y0.numpy(), m, mode, alpha, beta)
    np.testing.assert_allclose(outs[0].numpy(), z, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("kind", ["int8", "real_complex"])
def test_banded_transpose_one_pass_other_types(kind, dev):
    """int8 -> int32 and fp32 values with complex64 y (real A, complex compute) under opA = T after
    Preprocess: the one-pass banded kernel on packed 16-bit offsets (path flag 6), bit-identical to the
    product and column passes (the same SpMV without Preprocess) and equal to the exact result (int8) or
    within fp32 error of the fp64 oracle (complex)."""
    m, row_ptr, col, _, _, _ = _complex_laplacian(600, 13)
    g = torch.Generator().manual_seed(13)
    nnz = col.numel()
    if kind == "int8":
        v = torch.randint(-128, 128, (nnz,), generator=g, dtype=torch.int8)
        x = torch.randint(-128, 128, (m,), generator=g, dtype=torch.int8)
        y0 = torch.randint(-1000, 1000, (m,), generator=g, dtype=torch.int32)
        alpha, beta = 2, 3
    else:
        v = torch.rand(nnz, generator=g) * 2 - 1
        x = torch.rand(m, generator=g) * 2 - 1
        y0 = torch.complex(torch.rand(m, generator=g) * 2 - 1, torch.rand(m, generator=g) * 2 - 1)
        alpha, beta = complex(0.75, 1.25), complex(-0.5, 0.25)
    outs = []
    for pre in (True, False):
        y = y0.to(dev).clone()
        plan = CsrSpMV(m, m, row_ptr.to(torch.int32).to(dev), col.to(dev), v.to(dev), x.to(dev), y, alpha, beta,
                       op=Operation.TRANSPOSE)
        if pre:
            plan.preprocess()
            torch.cuda.synchronize()
            h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
            assert int(h[16] & 0xFFFFFFFF) == 6
        plan.run()
        torch.cuda.synchronize()
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1])
    rp = row_ptr.numpy()
    rows = np.repeat(np.arange(m), np.diff(rp))
    if kind == "int8":
        acc = np.zeros(m, np.int64)
        np.add.at(acc, col.numpy().astype(np.int64), v.numpy().astype(np.int64) * x.numpy().astype(np.int64)[rows])
        want = np.clip(alpha * acc + beta * y0.numpy().astype(np.int64), -2**31, 2**31 - 1)
        np.testing.assert_array_equal(outs[0].numpy().astype(np.int64), want)
    else:
        z = oracle.spmv_c64(rp, col.numpy(), v.numpy(), x.numpy(), y0.numpy(), m, 1, alpha, beta, val_is_real=True)
        np.testing.assert_allclose(outs[0].numpy(), z, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("kind,rdtype", [("c64", torch.int32), ("c64", torch.int64), ("int8_fp32", torch.int32),
                                         ("real_c64", torch.int32)])
def test_gen_rows_on_narrow_columns(kind, rdtype, dev):
    """The stream kernel of non-fp32 accumulators (complex64; int8 values and x with fp32 y; fp32 values
    and x with complex64 y) after Preprocess on a matrix of 2.4 M entries: the narrow column copy on the
    merge-path blocks (path flag 3; these kinds have no entry-aligned variant), bit-identical to the same
    SpMV on col_ind (without Preprocess) and within fp32 error of the oracle."""
    m, row_ptr, col, v, x, y0 = _complex_laplacian(700, 29)
    alpha, beta = complex(0.5, -1.25), complex(1.5, 0.5)
    g = torch.Generator().manual_seed(31)
    if kind == "int8_fp32":
        v = torch.randint(-128, 128, (col.numel(),), generator=g, dtype=torch.int8)
        x = torch.randint(-128, 128, (m,), generator=g, dtype=torch.int8)
        y0 = torch.rand(m, generator=g) * 2 - 1
        alpha, beta = 1.5, 0.5
    elif kind == "real_c64":
        v = torch.rand(col.numel(), generator=g) * 2 - 1
        x = torch.rand(m, generator=g) * 2 - 1
    outs = []
    for pre in (True, False):
        y = y0.to(dev).clone()
        plan = CsrSpMV(m, m, row_ptr.to(rdtype).to(dev), col.to(dev), v.to(dev), x.to(dev), y, alpha, beta)
        if pre:
            plan.preprocess()
            torch.cuda.synchronize()
            h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
            assert int(h[16] & 0xFFFFFFFF) == 3
        plan.run()
        torch.cuda.synchronize()
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1])
    rp = row_ptr.numpy()
    if kind == "int8_fp32":
        rows = np.repeat(np.arange(m), np.diff(rp))
        seg = np.zeros(m)
        np.add.at(seg, rows, v.numpy().astype(np.float64) * x.numpy().astype(np.float64)[col.numpy()])
        want = alpha * seg + beta * y0.numpy().astype(np.float64)
        np.testing.assert_allclose(outs[0].numpy(), want, rtol=1e-5, atol=1e-3)
    else:
        z = oracle.spmv_c64(rp, col.numpy(), v.numpy(), x.numpy(), y0.numpy(), m, 0, alpha, beta,
                            val_is_real=kind == "real_c64")
        np.testing.assert_allclose(outs[0].numpy(), z, rtol=1e-4, atol=1e-4)

@pytest.mark.parametrize("kind", ["fp32", "c64"])
def test_banded_transpose_values_updated_in_place(kind, dev):
    """Preprocess keeps the pattern only: after values are overwritten in place (same pointer), the next
    SpMV of the one-pass banded transpose (fp32 flag 4, complex64 flag 6) uses the new values."""
    m, row_ptr, col, v, x, y0 = _complex_laplacian(1100, 41)
    if kind == "fp32":
        v, x, y0 = v.real.contiguous(), x.real.contiguous(), y0.real.contiguous()
        alpha, beta, flag = 1.25, -0.5, 4
    else:
        alpha, beta, flag = complex(1.25, 0.5), complex(-0.5, 0.25), 6
    dv = v.to(dev)
    y = y0.to(dev).clone()
    plan = CsrSpMV(m, m, row_ptr.to(torch.int32).to(dev), col.to(dev), dv, x.to(dev), y, alpha, beta,
                   op=Operation.TRANSPOSE)
    plan.preprocess()
    torch.cuda.synchronize()
    h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
    assert int(h[16] & 0xFFFFFFFF) == flag
    plan.run()
    g = torch.Generator().manual_seed(42)
    if kind == "fp32":
        v2 = torch.rand(v.shape, generator=g) * 4 - 2
    else:
        v2 = torch.complex(torch.rand(v.numel(), generator=g) * 4 - 2, torch.rand(v.numel(), generator=g) * 4 - 2)
    dv.copy_(v2.to(dev))
    y.copy_(y0.to(dev))
    plan.run()
    torch.cuda.synchronize()
    rp = row_ptr.numpy()
    if kind == "fp32":
        z = oracle.spmv_c64(rp, col.numpy(), v2.numpy(), x.numpy(), y0.to(torch.complex64).numpy(), m, 1,
                            alpha, beta, val_is_real=True).real
    else:
        z = oracle.spmv_c64(rp, col.numpy(), v2.numpy(), x.numpy(), y0.numpy(), m, 1, alpha, beta)
    np.testing.assert_allclose(y.cpu().numpy(), z, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("op", ["N", "H"])
def test_complex_graph_capture_on_chosen_paths(op, dev):
    """complex64 SpMV captured in a HIP graph once Preprocess's choice is on the host: N on the narrow
    column copy (flag 3), H on the banded one-pass kernel (flag 6); every replay, with eager work between,
    matches the eager result bit for bit."""
    m, row_ptr, col, v, x, y0 = _complex_laplacian(700, 53)
    alpha, beta = complex(1.25, -0.5), complex(0.5, 0.75)
    o = Operation.NON_TRANSPOSE if op == "N" else Operation.CONJUGATE_TRANSPOSE
    s = torch.cuda.Stream()
    dy0 = y0.to(dev)
    y = dy0.clone()
    torch.cuda.synchronize()  # the inputs were written on the default stream
    with torch.cuda.stream(s):
        plan = CsrSpMV(m, m, row_ptr.to(torch.int32).to(dev), col.to(dev), v.to(dev), x.to(dev), y, alpha, beta,
                       op=o)
        plan.preprocess()
    torch.cuda.synchronize()
    h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
    assert int(h[16] & 0xFFFFFFFF) == (3 if op == "N" else 6)
    with torch.cuda.stream(s):
        plan.run()
    torch.cuda.synchronize()
    y.copy_(dy0)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        plan.run()
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    y.copy_(dy0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        plan.run()
    for _ in range(3):
        y.copy_(dy0)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        with torch.cuda.stream(s):
            plan.run()
        torch.cuda.synchronize()
