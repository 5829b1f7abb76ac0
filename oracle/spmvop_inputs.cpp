// spmvop_inputs.cpp — the inputs of the reference's SpMVOp tests, drawn with
// this toolchain's C++ standard library exactly as those tests draw them.
//
// TEST INFRASTRUCTURE ONLY (loaded by tests/ as an input generator; the
// product never links it).  What it restates (paths relative to the reference
// repository):
//   BuildCsr        test/spmv_op/arch35/spmv_op_test.cpp:50-67 ("diag",
//                   "empty" and "random" patterns, values in [-5, 5])
//   RandomCsr       test/frame/fill.h:71-123 (SparseFillGenerator::generateCsr:
//                   per row an optional empty-row draw, a binomial row length,
//                   distinct uniform column draws with a 4x attempt budget,
//                   completion from the unused columns by std::shuffle, sorted
//                   columns, then one value draw per entry)
//   ShuffleRows     test/spmv_op/arch35/spmv_op_npu_wrapper.h:26-44 (std::shuffle
//                   of each row's (column, value) pairs with mt19937(seed + 999))
//   DenseFloat      test/frame/fill.h:133-141,211-215 (uniform_real<float> draws)
//   X and Y         spmv_op_test.cpp:98-101 (seeds + 1 and + 2, range [-3, 3])
// The draws are the ones libstdc++ makes for these distributions; the
// reference's tests use the same standard-library calls in the same order.
#include <algorithm>
#include <cstdint>
#include <random>
#include <utility>
#include <vector>

namespace {

struct Csr {
    std::vector<int32_t> rp, col;
    std::vector<float> val;
};

Csr RandomCsr(int64_t rows, int64_t cols, double sparsity, double emptyProb, uint32_t seed, double lo, double hi)
{
    Csr out;
    out.rp.assign(static_cast<size_t>(rows) + 1, 0);
    if (rows <= 0 || cols <= 0) return out;
    std::mt19937 rng(seed);
    sparsity = std::clamp(sparsity, 0.0, 1.0);
    emptyProb = std::clamp(emptyProb, 0.0, 1.0);
    std::uniform_real_distribution<float> emptyDist(0.0f, 1.0f);
    std::uniform_real_distribution<float> valDist(static_cast<float>(lo), static_cast<float>(hi));
    std::binomial_distribution<int> lenDist(static_cast<int>(cols), 1.0 - sparsity);
    std::vector<int> seen(static_cast<size_t>(cols), -1);
    std::vector<int> picked;
    int64_t nnz = 0;
    for (int64_t i = 0; i < rows; ++i) {
        out.rp[static_cast<size_t>(i)] = static_cast<int32_t>(nnz);
        if (emptyProb > 0.0 && emptyDist(rng) < static_cast<float>(emptyProb)) continue;
        int want = std::min(lenDist(rng), static_cast<int>(cols));
        if (want <= 0) continue;
        for (int tries = 0; static_cast<int>(picked.size()) < want && tries < want * 4; ++tries) {
            std::uniform_int_distribution<int32_t> colDist(0, static_cast<int32_t>(cols) - 1);
            const int32_t c = colDist(rng);
            if (seen[static_cast<size_t>(c)] != static_cast<int>(i)) {
                seen[static_cast<size_t>(c)] = static_cast<int>(i);
                picked.push_back(c);
            }
        }
        if (static_cast<int>(picked.size()) < want) {
            const size_t drawn = picked.size();
            for (int32_t c = 0; c < cols; ++c) {
                if (seen[static_cast<size_t>(c)] != static_cast<int>(i)) picked.push_back(c);
            }
            std::shuffle(picked.begin() + static_cast<std::ptrdiff_t>(drawn), picked.end(), rng);
            picked.resize(static_cast<size_t>(want));
        }
        std::sort(picked.begin(), picked.end());
        for (int32_t c : picked) {
            out.col.push_back(c);
            out.val.push_back(valDist(rng));
            ++nnz;
        }
        picked.clear();
    }
    out.rp[static_cast<size_t>(rows)] = static_cast<int32_t>(nnz);
    return out;
}

void ShuffleRows(Csr& a, int64_t rows, uint32_t seed)
{
    std::mt19937 rng(seed + 999);
    std::vector<std::pair<int32_t, float>> row;
    for (int64_t i = 0; i < rows; ++i) {
        const int32_t b = a.rp[static_cast<size_t>(i)], e = a.rp[static_cast<size_t>(i) + 1];
        if (e - b <= 1) continue;
        row.clear();
        for (int32_t j = b; j < e; ++j) row.emplace_back(a.col[static_cast<size_t>(j)], a.val[static_cast<size_t>(j)]);
        std::shuffle(row.begin(), row.end(), rng);
        for (int32_t j = b; j < e; ++j) {
            a.col[static_cast<size_t>(j)] = row[static_cast<size_t>(j - b)].first;
            a.val[static_cast<size_t>(j)] = row[static_cast<size_t>(j - b)].second;
        }
    }
}

std::vector<float> DenseFloat(int64_t n, double lo, double hi, uint32_t seed)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(static_cast<float>(lo), static_cast<float>(hi));
    std::vector<float> out(static_cast<size_t>(n > 0 ? n : 0));
    for (auto& v : out) v = dist(rng);
    return out;
}

}  // namespace

extern "C" {

// pattern: 0 random, 1 diag, 2 empty.  Fills rp[m+1] always; col/val (capacity
// cap), x[k] and y[m] when non-null.  Returns nnz (col/val are written only
// when cap >= nnz).
int64_t oracle_spmvop_inputs(int64_t m, int64_t k, double sparsity, double emptyProb, uint32_t seed, int pattern,
                             int unsorted, int32_t* rp, int32_t* col, float* val, int64_t cap, float* x, float* y)
{
    Csr a;
    if (pattern == 1) {  // makeDiagCsr(m): an m x m identity pattern of ones
        a.rp.resize(static_cast<size_t>(m) + 1);
        for (int64_t i = 0; i <= m; ++i) a.rp[static_cast<size_t>(i)] = static_cast<int32_t>(i);
        for (int64_t i = 0; i < m; ++i) {
            a.col.push_back(static_cast<int32_t>(i));
            a.val.push_back(1.0f);
        }
    } else if (pattern == 2 || m <= 0 || k <= 0) {
        a.rp.assign(static_cast<size_t>(m > 0 ? m : 0) + 1, 0);
    } else {
        a = RandomCsr(m, k, sparsity, emptyProb, seed, -5.0, 5.0);
        if (unsorted) ShuffleRows(a, m, seed);
    }
    const int64_t nnz = static_cast<int64_t>(a.col.size());
    std::copy(a.rp.begin(), a.rp.end(), rp);
    if (col != nullptr && val != nullptr && cap >= nnz) {
        std::copy(a.col.begin(), a.col.end(), col);
        std::copy(a.val.begin(), a.val.end(), val);
    }
    if (x != nullptr && k > 0) {
        const std::vector<float> v = DenseFloat(k, -3.0, 3.0, seed + 1);
        std::copy(v.begin(), v.end(), x);
    }
    if (y != nullptr && m > 0) {
        const std::vector<float> v = DenseFloat(m, -3.0, 3.0, seed + 2);
        std::copy(v.begin(), v.end(), y);
    }
    return nnz;
}

}  // extern "C"
