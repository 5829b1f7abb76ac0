"""Writes reference_kats.json: the known-answer cases held by the reference's own SpMV tests.

Every case is data transcribed from the cited reference test (inputs and the
expected outputs that test asserts); nothing here runs reference code.  Paths
are relative to the reference repository.

Run: python tests/golden/make_fixtures.py
"""
import json
import os

H = os.path.dirname(os.path.abspath(__file__))


def csv_cases():
    # test/spmv/arch35/spmv_test.csv (7 lines) with the 2x3 fixture of
    # test/spmv/arch35/spmv_test.cpp:69-86 and the second-execution golden :144-154.
    rows = [
        ("fp32_n_base0_default", "N", 0, "DEFAULT", "HOST", 2.0, 3.0),
        ("fp32_n_base1_alg1", "N", 1, "CSR_ALG1", "HOST", 2.0, 3.0),
        ("fp32_t_base0_default", "T", 0, "DEFAULT", "HOST", 1.0, 2.0),
        ("fp32_t_base1_alg1", "T", 1, "CSR_ALG1", "HOST", 1.0, 2.0),
        ("fp32_t_base0_alg2", "T", 0, "CSR_ALG2", "HOST", 1.0, 2.0),
        ("fp32_n_device_scalar", "N", 0, "DEFAULT", "DEVICE", 2.0, 3.0),
    ]
    out = []
    for name, op, base, alg, mode, a, b in rows:
        if op == "N":
            x, y = [1.0, 2.0, 3.0], [5.0, 6.0]
            first = [a * (2 * x[0] + 3 * x[2]) + b * y[0], a * (4 * x[1]) + b * y[1]]
            product = [11.0, 8.0]
        else:
            x, y = [10.0, 20.0], [7.0, 8.0, 9.0]
            first = [a * (2 * x[0]) + b * y[0], a * (4 * x[1]) + b * y[1], a * (3 * x[0]) + b * y[2]]
            product = [20.0, 80.0, 30.0]
        second = [a * p + b * f for p, f in zip(product, first)]
        out.append(dict(name=name, op=op, base=base, alg=alg, pointer_mode=mode, alpha=a, beta=b,
                        rows=2, cols=3, row_ptr=[base, base + 2, base + 3], col_ind=[base, base + 2, base + 1],
                        values=[2.0, 3.0, 4.0], x=x, y=y, expected_first=first, expected_second=second,
                        tolerance=1e-5, source="test/spmv/arch35/spmv_test.cpp:69-86,144-154,159-212"))
    return out


def fixtures():
    return {
        "csv_cases": csv_cases(),
        # test/spmv/arch35/spmv_test.cpp:474-506
        "zero_nnz_beta": dict(rows=2, cols=3, row_ptr=[0, 0, 0], x=[1.0, 2.0, 3.0], y=[4.0, 5.0], alpha=1.0,
                              beta=2.0, expected=[8.0, 10.0], source="test/spmv/arch35/spmv_test.cpp:474-506"),
        # test/spmv/arch35/spmv_test.cpp:508-541
        "repeated_coordinates": dict(rows=1, cols=1, row_ptr=[0, 2], col_ind=[0, 0], values=[2.0, 3.0], x=[4.0],
                                     y=[9.0], alpha=1.0, beta=0.0, alg="CSR_ALG2", expected=[20.0],
                                     source="test/spmv/arch35/spmv_test.cpp:508-541"),
        # test/spmv/arch35/spmv_test.cpp:617-663: values {127,-127}, x all 127,
        # alpha INT32_MAX, beta 0 -> y[0]=INT32_MAX, y[1]=INT32_MIN, rest 0
        "int8_saturation": dict(values=[127, -127], col_ind=[0, 1], alpha=2147483647, beta=0,
                                row_counts=[2, 4096], ops=["N", "T", "H"], algs=["DEFAULT", "CSR_ALG2"],
                                expected_head=[2147483647, -2147483648],
                                source="test/spmv/arch35/spmv_test.cpp:617-663"),
        # test/spmv/arch35/spmv_test.cpp:665-697: fp16 bits, RNE halfway
        "fp16_halfway": dict(rows=2, cols=2, row_ptr=[0, 2, 4], col_ind=[0, 1, 0, 1],
                             values_bits=[0x3C00, 0x1000, 0xBC00, 0x9000], x_bits=[0x3C00, 0x3C00],
                             y_bits=[0, 0], alpha=1.0, beta=0.0, expected_bits=[0x3C00, 0xBC00],
                             source="test/spmv/arch35/spmv_test.cpp:665-697"),
        # test/spmv/arch35/spmv_test.cpp:699-734: complex64, op=H, ALG2
        "complex_conj_transpose": dict(rows=2, cols=2, row_ptr=[0, 2, 3], col_ind=[0, 1, 1],
                                       values=[[1.0, 2.0], [3.0, -1.0], [2.0, 4.0]], x=[[1.0, -1.0], [2.0, 3.0]],
                                       y=[[9.0, 8.0], [7.0, 6.0]], alpha=[1.0, 0.0], beta=[0.0, 0.0],
                                       alg="CSR_ALG2", expected=[[-1.0, -3.0], [20.0, -4.0]],
                                       source="test/spmv/arch35/spmv_test.cpp:699-734"),
        # test/spmv/arch35/spmv_test.cpp:255-374: base-1 CSR, strides row 2,
        # col 3, values 4, x 5, y 6, sentinel padding; alpha 2 beta 3, y0 = 5
        "strided": dict(strides=dict(row=2, col=3, val=4, x=5, y=6), sentinel=-1234.0, index_sentinel=-999,
                        alpha=2.0, beta=3.0, y_init=5.0,
                        cases=[dict(rows=2, op="N", alg="DEFAULT", sorted=True),
                               dict(rows=65, op="N", alg="DEFAULT", sorted=True),
                               dict(rows=2, op="T", alg="DEFAULT", sorted=True),
                               dict(rows=2, op="T", alg="DEFAULT", sorted=False),
                               dict(rows=2, op="H", alg="CSR_ALG2", sorted=True),
                               dict(rows=4096, op="T", alg="DEFAULT", sorted=True)],
                        expected_n=dict(even_row=37.0, odd_row=31.0),
                        expected_t="[4*evenRows+15, 8*oddRows+15, 6*evenRows+15]",
                        source="test/spmv/arch35/spmv_test.cpp:255-374"),
        # test/spmv/arch22/spmv_test.cpp:350-361: the fp32 golden must be
        # computed in double: {2^24, 1, -2^24} . {1,1,1} = 1
        "golden_precision": dict(row_ptr=[0, 3], col_ind=[0, 1, 2], values=[16777216.0, 1.0, -16777216.0],
                                 x=[1.0, 1.0, 1.0], expected=1.0,
                                 source="test/spmv/arch22/spmv_test.cpp:350-361"),
        # test/spmv/arch22/spmv_test_verification.h:111-165: verifier self-tests
        "verifier": dict(
            cases=[
                dict(golden=[1.0] * 100, actual=[1.005] + [1.0] * 99, tol="float32", passed=True),
                dict(golden=[1.0] * 100, actual=["nan"] + [1.0] * 99, tol="float32", passed=False),
                dict(golden=[1.0] * 100, actual=["inf"] + [1.0] * 99, tol="float32", passed=False),
                dict(golden=[1.0 + 2e-8], actual=[1.0], tol="exact_float", passed=False),
                dict(golden=[1.0], actual=[1.0], tol="float32", passed=True),
                dict(golden=[1.0], actual=[2.0], tol="float32", passed=False),
                dict(golden=[1.0], actual=["nan"], tol="float32", passed=False),
                dict(golden=["inf"], actual=[1.0], tol="float32", passed=False),
                dict(golden=[16777217], actual=[16777216], tol="int32", passed=False),
                dict(golden=[16777217], actual=[16777217], tol="int32", passed=True),
            ],
            diagnostics=dict(golden_head=[1000.0, 0.0], actual_head=[1000.02, 0.005], n=100,
                             passed=False, ratio=0.99),
            source="test/spmv/arch22/spmv_test_verification.h:111-165"),
    }


if __name__ == "__main__":
    path = os.path.join(H, "reference_kats.json")
    with open(path, "w") as f:
        json.dump(fixtures(), f, indent=1)
    print(path)
