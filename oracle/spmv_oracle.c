/*
 * spmv_oracle.c — CPU restatement of the reference's SpMV host golden.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product (libaclsparse_hip.so and the
 * ops_sparse package) never links, imports or calls it.
 *
 * What each function restates (paths relative to the reference repository):
 *   oracle_half_from_float / oracle_float_from_half
 *       host `half` conversion, test/spmv/arch22/spmv_test.cpp:39-126
 *   oracle_bf16_from_float / oracle_float_from_bf16
 *       host `bfloat16_t` conversion, test/spmv/arch22/spmv_test.cpp:128-157
 *   oracle_spmv_f64        SpmvCpu<double,float,double> as BuildSpmvGolden
 *                          calls it for pure fp32 (spmv_test.cpp:258-279,311-337)
 *   oracle_spmv_trans_f64  SpmvTransCpu<double,...> (spmv_test.cpp:283-307)
 *   oracle_spmv_lowp       SpmvCpu<float, half|bf16, half|bf16|float>:
 *                          fp32 accumulation of upcast products, one RNE cast
 *   oracle_spmv_trans_lowp SpmvTransCpu<float, half|bf16, ...>
 *   oracle_spmv_i8         int8 -> int32 path: exact int64 sum, saturating
 *                          alpha/beta epilogue (sparse/spmv/arch35/spmv_kernel.cpp:341-376)
 *   oracle_spmv_c64        complex64 path in double (conjugate for op=H)
 *   oracle_row_scale       |alpha|*sum|a_ij*x_j| + |beta*y_i| per output row,
 *                          the scale of the north-star tolerance
 *   oracle_items_per_block / oracle_spmv_partition
 *                          this build's row-block partition (no reference
 *                          counterpart; restated from its definition:
 *                          block b starts at the first row r with
 *                          16*r + rowOffset[r] >= b*T)
 *   oracle_spmvop_tables   SpMVOp ALG2 reorder / scratch / bin_edge
 *                          (sparse/spmv_op/arch35/spmv_op_kernel.cpp:425-540)
 *   oracle_verify_mere_mare MERE/MARE check, test/frame/verify.h:126-175
 *   oracle_verify_mixed    Verification() mixed tolerance,
 *                          test/spmv/arch22/spmv_test_verification.h:23-101
 *
 * CSR inputs are base 0 and contiguous (the reference golden also runs on
 * base-0 data: spmv_test.cpp ShiftCsrIndexBase); row offsets are int64.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------ 16-bit floats ----------------------------- */

float oracle_float_from_half(uint16_t bits)
{
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exp = (bits >> 10) & 0x1Fu;
    uint32_t mant = bits & 0x3FFu;
    uint32_t u;
    if (exp == 0) {
        if (mant == 0) {
            u = sign;
        } else {
            /* subnormal: normalise the mantissa, adjusting the exponent */
            exp = 113;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                exp--;
            }
            u = sign | (exp << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7F800000u | (mant << 13);
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

uint16_t oracle_half_from_float(float v)
{
    uint32_t u;
    memcpy(&u, &v, sizeof u);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {
        uint16_t payload = (uint16_t)((a & 0x007FFFFFu) >> 13);
        return (uint16_t)(sign | 0x7C00u | payload | (payload == 0 && a != 0x7F800000u ? 1 : 0));
    }
    int32_t exponent = (int32_t)((a >> 23) & 0xFFu) - 127 + 15;
    uint32_t mantissa = a & 0x007FFFFFu;
    if (exponent >= 31) return (uint16_t)(sign | 0x7C00u);
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        mantissa |= 0x00800000u;
        uint32_t shift = (uint32_t)(14 - exponent);
        uint32_t rounded = (mantissa + ((1u << (shift - 1)) - 1u) + ((mantissa >> shift) & 1u)) >> shift;
        return (uint16_t)(sign | rounded);
    }
    uint32_t rm = mantissa + 0x00000FFFu + ((mantissa >> 13) & 1u);
    if ((rm & 0x00800000u) != 0) {
        rm = 0;
        ++exponent;
        if (exponent >= 31) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)exponent << 10) | (rm >> 13));
}

float oracle_float_from_bf16(uint16_t bits)
{
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

uint16_t oracle_bf16_from_float(float f)
{
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7F800000u) == 0x7F800000u) {
        uint16_t b = (uint16_t)(u >> 16);
        if ((u & 0x007FFFFFu) != 0) b |= 0x0040u; /* every NaN stays a NaN */
        return b;
    }
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* value kinds of the low-precision paths */
enum { K_F32 = 0, K_F16 = 1, K_BF16 = 2 };

static float load_lowp(const void *p, int64_t i, int kind)
{
    if (kind == K_F16) return oracle_float_from_half(((const uint16_t *)p)[i]);
    if (kind == K_BF16) return oracle_float_from_bf16(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

static void store_lowp(void *p, int64_t i, float v, int kind)
{
    if (kind == K_F16) ((uint16_t *)p)[i] = oracle_half_from_float(v);
    else if (kind == K_BF16) ((uint16_t *)p)[i] = oracle_bf16_from_float(v);
    else ((float *)p)[i] = v;
}

/* ------------------------------ fp32 golden ------------------------------- */

/* z_i = alpha * sum_j a_ij x_j + beta * y_i, accumulated in double. */
void oracle_spmv_f64(int64_t rows, const int64_t *rp, const int32_t *col, const float *val, const float *x,
                     const float *y, double alpha, double beta, double *z)
{
    for (int64_t i = 0; i < rows; ++i) {
        double sum = 0.0;
        for (int64_t p = rp[i]; p < rp[i + 1]; ++p) sum += (double)val[p] * (double)x[col[p]];
        z[i] = alpha * sum + beta * (double)y[i];
    }
}

/* The same product split over nthreads POSIX threads by row ranges (this
 * build's parallel restatement, used only as a labelled CPU baseline; the
 * reference's host golden is the serial loop above). */
struct oracle_par_arg {
    int64_t r0, r1;
    const int64_t *rp;
    const int32_t *col;
    const float *val, *x, *y;
    double alpha, beta;
    double *z;
};

static void *oracle_par_run(void *p)
{
    const struct oracle_par_arg *a = (const struct oracle_par_arg *)p;
    for (int64_t i = a->r0; i < a->r1; ++i) {
        double sum = 0.0;
        for (int64_t q = a->rp[i]; q < a->rp[i + 1]; ++q) sum += (double)a->val[q] * (double)a->x[a->col[q]];
        a->z[i] = a->alpha * sum + a->beta * (double)a->y[i];
    }
    return NULL;
}

int oracle_spmv_f64_threads(int64_t rows, const int64_t *rp, const int32_t *col, const float *val, const float *x,
                            const float *y, double alpha, double beta, double *z, int nthreads)
{
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    struct oracle_par_arg args[256];
    for (int t = 0; t < nthreads; ++t) {
        args[t].r0 = rows * t / nthreads;
        args[t].r1 = rows * (t + 1) / nthreads;
        args[t].rp = rp;
        args[t].col = col;
        args[t].val = val;
        args[t].x = x;
        args[t].y = y;
        args[t].alpha = alpha;
        args[t].beta = beta;
        args[t].z = z;
        if (pthread_create(&th[t], NULL, oracle_par_run, &args[t]) != 0) {
            for (int u = 0; u < t; ++u) pthread_join(th[u], NULL);
            return -1;
        }
    }
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    return 0;
}

/* z_j = beta*y_j + sum_i alpha*x_i*a_ij, rows with alpha*x_i == 0 skipped. */
void oracle_spmv_trans_f64(int64_t rows, int64_t cols, const int64_t *rp, const int32_t *col, const float *val,
                           const float *x, const float *y, double alpha, double beta, double *z)
{
    for (int64_t j = 0; j < cols; ++j) z[j] = beta * (double)y[j];
    for (int64_t i = 0; i < rows; ++i) {
        const double xv = alpha * (double)x[i];
        if (xv == 0.0) continue;
        for (int64_t p = rp[i]; p < rp[i + 1]; ++p) z[col[p]] = z[col[p]] + xv * (double)val[p];
    }
}

/* Per-output scale |alpha|*sum|a*x| + |beta*y| (non-transpose / transpose). */
void oracle_row_scale(int64_t rows, int64_t cols, const int64_t *rp, const int32_t *col, const void *val,
                      const void *x, const void *y, int kind, int yKind, int transpose, double alpha, double beta,
                      double *scale)
{
    const int64_t n = transpose ? cols : rows;
    for (int64_t j = 0; j < n; ++j) scale[j] = fabs(beta * (double)load_lowp(y, j, yKind));
    for (int64_t i = 0; i < rows; ++i) {
        for (int64_t p = rp[i]; p < rp[i + 1]; ++p) {
            const int64_t o = transpose ? col[p] : i;
            const int64_t xi = transpose ? i : col[p];
            scale[o] += fabs(alpha * (double)load_lowp(val, p, kind) * (double)load_lowp(x, xi, kind));
        }
    }
}

/* ------------------------ fp16 / bf16, fp32 compute ----------------------- */

void oracle_spmv_lowp(int64_t rows, const int64_t *rp, const int32_t *col, const void *val, const void *x,
                      const void *y, int kind, int yKind, float alpha, float beta, void *z)
{
    for (int64_t i = 0; i < rows; ++i) {
        float sum = 0.0f;
        for (int64_t p = rp[i]; p < rp[i + 1]; ++p) sum += load_lowp(val, p, kind) * load_lowp(x, col[p], kind);
        store_lowp(z, i, alpha * sum + beta * load_lowp(y, i, yKind), yKind);
    }
}

/* oracle_spmv_lowp split over nthreads POSIX threads by row ranges (this
 * build's parallel restatement for the labelled CPU baseline; every row is
 * summed in the serial loop's order, so the results are bit-identical). */
struct oracle_lowp_arg {
    int64_t r0, r1;
    const int64_t *rp;
    const int32_t *col;
    const void *val, *x, *y;
    int kind, yKind;
    float alpha, beta;
    void *z;
};

static void *oracle_lowp_run(void *p)
{
    const struct oracle_lowp_arg *a = (const struct oracle_lowp_arg *)p;
    for (int64_t i = a->r0; i < a->r1; ++i) {
        float sum = 0.0f;
        for (int64_t q = a->rp[i]; q < a->rp[i + 1]; ++q) {
            sum += load_lowp(a->val, q, a->kind) * load_lowp(a->x, a->col[q], a->kind);
        }
        store_lowp(a->z, i, a->alpha * sum + a->beta * load_lowp(a->y, i, a->yKind), a->yKind);
    }
    return NULL;
}

int oracle_spmv_lowp_threads(int64_t rows, const int64_t *rp, const int32_t *col, const void *val, const void *x,
                             const void *y, int kind, int yKind, float alpha, float beta, void *z, int nthreads)
{
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    struct oracle_lowp_arg args[256];
    for (int t = 0; t < nthreads; ++t) {
        struct oracle_lowp_arg a = {rows * t / nthreads, rows * (t + 1) / nthreads, rp, col, val, x, y,
                                    kind, yKind, alpha, beta, z};
        args[t] = a;
        if (pthread_create(&th[t], NULL, oracle_lowp_run, &args[t]) != 0) {
            for (int u = 0; u < t; ++u) pthread_join(th[u], NULL);
            return -1;
        }
    }
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    return 0;
}

void oracle_spmv_trans_lowp(int64_t rows, int64_t cols, const int64_t *rp, const int32_t *col, const void *val,
                            const void *x, const void *y, int kind, int yKind, float alpha, float beta, float *acc,
                            void *z)
{
    for (int64_t j = 0; j < cols; ++j) acc[j] = beta * load_lowp(y, j, yKind);
    for (int64_t i = 0; i < rows; ++i) {
        const float xv = alpha * load_lowp(x, i, kind);
        if (xv == 0.0f) continue;
        for (int64_t p = rp[i]; p < rp[i + 1]; ++p) acc[col[p]] = acc[col[p]] + xv * load_lowp(val, p, kind);
    }
    for (int64_t j = 0; j < cols; ++j) store_lowp(z, j, acc[j], yKind);
}

/* ------------------------------ int8 -> int32 ----------------------------- */

static int64_t sat32(int64_t v) { return v > 2147483647LL ? 2147483647LL : v < -2147483648LL ? -2147483648LL : v; }

static int32_t scaled_i32(int64_t sum, int64_t alpha, int64_t beta, int64_t oldY)
{
    const int64_t betaTerm = beta * oldY;
    if (alpha == 0) return (int32_t)sat32(betaTerm);
    /* exact: |sum| < 2^45 and |alpha| < 2^31, so use 128-bit arithmetic */
    __int128 r = (__int128)sum * alpha + betaTerm;
    if (r > 2147483647) return 2147483647;
    if (r < -2147483648LL) return (int32_t)-2147483648LL;
    return (int32_t)r;
}

void oracle_spmv_i8(int64_t rows, int64_t cols, const int64_t *rp, const int32_t *col, const int8_t *val,
                    const int8_t *x, const int32_t *y, int transpose, int32_t alpha, int32_t beta, int32_t *z,
                    int64_t *acc)
{
    const int64_t n = transpose ? cols : rows;
    for (int64_t j = 0; j < n; ++j) acc[j] = 0;
    for (int64_t i = 0; i < rows; ++i) {
        for (int64_t p = rp[i]; p < rp[i + 1]; ++p) {
            if (transpose) acc[col[p]] += (int64_t)val[p] * (int64_t)x[i];
            else acc[i] += (int64_t)val[p] * (int64_t)x[col[p]];
        }
    }
    for (int64_t j = 0; j < n; ++j) z[j] = scaled_i32(acc[j], alpha, beta, beta == 0 ? 0 : y[j]);
}

/* ------------------------------ complex64 --------------------------------- */

/* val/x/y/z interleaved (re, im); compute in double; op 0=N 1=T 2=H;
 * valIsReal: values and x are float (f32 -> c64 combination). */
void oracle_spmv_c64(int64_t rows, int64_t cols, const int64_t *rp, const int32_t *col, const float *val,
                     const float *x, const float *y, int valIsReal, int op, double ar, double ai, double br,
                     double bi, double *z)
{
    const int64_t n = op == 0 ? rows : cols;
    for (int64_t j = 0; j < 2 * n; ++j) z[j] = 0.0;
    for (int64_t i = 0; i < rows; ++i) {
        for (int64_t p = rp[i]; p < rp[i + 1]; ++p) {
            double vr = valIsReal ? val[p] : val[2 * p], vi = valIsReal ? 0.0 : val[2 * p + 1];
            if (op == 2) vi = -vi;
            const int64_t xi = op == 0 ? col[p] : i;
            const double xr = valIsReal ? x[xi] : x[2 * xi], xim = valIsReal ? 0.0 : x[2 * xi + 1];
            const int64_t o = op == 0 ? i : col[p];
            z[2 * o] += vr * xr - vi * xim;
            z[2 * o + 1] += vr * xim + vi * xr;
        }
    }
    for (int64_t j = 0; j < n; ++j) {
        const double sr = z[2 * j], si = z[2 * j + 1];
        const double yr = y[2 * j], yi = y[2 * j + 1];
        z[2 * j] = ar * sr - ai * si + br * yr - bi * yi;
        z[2 * j + 1] = ar * si + ai * sr + br * yi + bi * yr;
    }
}

/* ----------------------------- partition ---------------------------------- */

/* T = min(2032, 496 + floor(16*496*rows/nnz)) (2032 when nnz == 0);
 * blocks = ceil((16*rows + nnz) / T). */
int64_t oracle_items_per_block(int64_t rows, int64_t nnz)
{
    if (nnz == 0) return 2032;
    const uint64_t t = 496u + ((uint64_t)(16 * 496) * (uint64_t)rows) / (uint64_t)nnz;
    return t > 2032u ? 2032 : (int64_t)t;
}

int64_t oracle_num_blocks(int64_t rows, int64_t nnz)
{
    const int64_t t = oracle_items_per_block(rows, nnz);
    return (16 * rows + nnz + t - 1) / t;
}

/* norm[i] = clamp(rowPtr[i*stride] - base, 0, nnz) for i in [0, rows];
 * blocks[b] = first row r with 16*r + norm[r] >= b*T (b < B), blocks[B] = rows;
 * block_nnz[b] = norm[blocks[b]].  Computed by a forward sweep, independently
 * of the device's per-block binary search. */
void oracle_spmv_partition(int64_t rows, int64_t nnz, const int64_t *rowPtr, int64_t stride, int64_t base,
                           int64_t *norm, int32_t *blocks, int64_t *blockNnz)
{
    const int64_t t = oracle_items_per_block(rows, nnz);
    const int64_t nb = oracle_num_blocks(rows, nnz);
    for (int64_t i = 0; i <= rows; ++i) {
        int64_t v = rowPtr[i * stride] - base;
        norm[i] = v < 0 ? 0 : v > nnz ? nnz : v;
    }
    int64_t r = 0;
    for (int64_t b = 0; b < nb; ++b) {
        while (r < rows && 16 * r + norm[r] < b * t) ++r;
        blocks[b] = (int32_t)r;
        blockNnz[b] = norm[r];
    }
    blocks[nb] = (int32_t)rows;
    blockNnz[nb] = norm[rows];
}

/* ---------------------------- SpMVOp ALG2 ---------------------------------- */

/* Restates the reference's ALG2 tables (sparse/spmv_op/arch35/spmv_op_kernel.cpp:425-540)
 * for a given bin count: scratch[i] = rowPtr[i+1]-rowPtr[i], reorder = iota,
 * bottom-up merge sort descending by scratch taking the left run on ties,
 * then bin_edge by the running-sum loop.  tmp arrays: m entries each. */
void oracle_spmvop_tables(int32_t m, const int64_t *rowPtr, uint32_t numBlocks, int32_t *reorder, int32_t *scratch,
                          int32_t *tmpReorder, int32_t *tmpNnz, int32_t *binEdge)
{
    for (int32_t i = 0; i < m; ++i) {
        scratch[i] = (int32_t)(rowPtr[i + 1] - rowPtr[i]);
        reorder[i] = i;
    }
    for (int32_t width = 1; width < m; width *= 2) {
        for (int32_t i = 0; i < m; i += 2 * width) {
            const int32_t left = i;
            const int32_t mid = (i + width < m) ? (i + width) : m;
            const int32_t right = (i + 2 * width < m) ? (i + 2 * width) : m;
            int32_t a = left, b = mid, k = left;
            while (a < mid && b < right) {
                if (scratch[a] >= scratch[b]) { tmpReorder[k] = reorder[a]; tmpNnz[k] = scratch[a]; ++a; }
                else { tmpReorder[k] = reorder[b]; tmpNnz[k] = scratch[b]; ++b; }
                ++k;
            }
            while (a < mid) { tmpReorder[k] = reorder[a]; tmpNnz[k] = scratch[a]; ++a; ++k; }
            while (b < right) { tmpReorder[k] = reorder[b]; tmpNnz[k] = scratch[b]; ++b; ++k; }
            for (int32_t idx = left; idx < right; ++idx) {
                reorder[idx] = tmpReorder[idx];
                scratch[idx] = tmpNnz[idx];
            }
        }
    }
    int64_t total = 0;
    for (int32_t i = 0; i < m; ++i) total += scratch[i];
    const int64_t perBlock = (total > 0 && numBlocks > 0) ? (total + numBlocks - 1) / numBlocks : 0;
    binEdge[0] = 0;
    uint32_t bin = 1;
    int64_t running = 0;
    for (int32_t i = 0; i < m; ++i) {
        running += scratch[i];
        if (bin < numBlocks && running >= perBlock * (int64_t)bin) {
            binEdge[bin] = i + 1;
            ++bin;
        }
    }
    while (bin <= numBlocks) binEdge[bin++] = m;
}

/* MERE/MARE of test/frame/verify.h:126-175 (epsilon 2^-14 in the denominator);
 * returns 1 when MERE < threshold and MARE < multiplier*threshold and no
 * one-sided non-finite value. */
int oracle_verify_mere_mare(int64_t n, const float *golden, const float *actual, double threshold,
                            double multiplier, double *mereOut, double *mareOut)
{
    const double eps = 0.00006103515625;
    double sum = 0.0, mare = 0.0;
    int64_t mismatch = 0, skipped = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int oa = isnan(actual[i]) || isinf(actual[i]);
        const int ga = isnan(golden[i]) || isinf(golden[i]);
        if (oa && ga) { ++skipped; continue; }
        if (oa || ga) { ++mismatch; continue; }
        const double rel = fabs((double)actual[i] - (double)golden[i]) / (fabs((double)golden[i]) + eps);
        sum += rel;
        if (rel > mare) mare = rel;
    }
    const int64_t eff = n - skipped - mismatch;
    const double mere = eff > 0 ? sum / (double)eff : 0.0;
    *mereOut = mere;
    *mareOut = mare;
    return mismatch == 0 && mere < threshold && mare < multiplier * threshold;
}

/* ------------------------- mixed-tolerance verify -------------------------- */

/* Returns 0 on pass, 1 on fail; outputs the matched ratio and max abs error.
 * golden/actual are doubles (callers upcast); exact != 0 selects the int32
 * exact-match rule. */
int oracle_verify_mixed(int64_t n, const double *golden, const double *actual, double rtol, double atol,
                        double maxAbsLimit, double requiredRatio, int exact, double *ratioOut, double *maxAbsOut)
{
    int64_t pass = 0;
    double maxAbs = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const int finite = isfinite(actual[i]) && isfinite(golden[i]);
        const double err = finite ? fabs(actual[i] - golden[i]) : INFINITY;
        const double tol = atol + rtol * fabs(golden[i]);
        int matched = finite && err <= tol;
        if (exact) matched = actual[i] == golden[i];
        pass += matched ? 1 : 0;
        if (err > maxAbs) maxAbs = err;
    }
    const float ratio = n == 0 ? 1.0f : (float)pass / (float)n;
    *ratioOut = ratio;
    *maxAbsOut = maxAbs;
    if (exact) return ratio < (float)requiredRatio ? 1 : 0;
    return (ratio < (float)requiredRatio || maxAbs > maxAbsLimit) ? 1 : 0;
}
