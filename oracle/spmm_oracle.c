/*
 * spmm_oracle.c — CPU restatement of the reference's SpMMOp arithmetic and of
 * the random inputs its tests draw.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product never links, imports or calls it.
 *
 * What each function restates (paths relative to the reference repository):
 *   oracle_mt19937_fill     std::mt19937 (the 32-bit Mersenne Twister of
 *                           Matsumoto & Nishimura, seeded by init_genrand) as
 *                           the tests construct it: std::mt19937 rng(seed)
 *                           (test/spmm_op/spmm_op_golden.h:104-107,
 *                           test/spmm_op/arch35/spmm_op_test.cpp:121-133)
 *   oracle_uniform_real     std::uniform_real_distribution<double>(lo, hi)
 *                           over that engine as libstdc++ computes it:
 *                           generate_canonical<double, 53> draws two words,
 *                           S = w0 + w1 * 2^32 (in double), S / 2^64, then
 *                           u * (hi - lo) + lo
 *   oracle_spmm_f32         the SpMMOp kernel's fp32 steps per output element
 *                           (sparse/spmm_op/arch35/spmm_op_kernel.cpp:386-424
 *                           products and sums in CSR order, out-of-range
 *                           columns skipped; :529-547 Kahan for
 *                           ALG1_HIGH_PRECISION; :549-640 alpha then beta
 *                           epilogue; :89-127 fp16 clamp and ties-away cast;
 *                           :687-880 nnz == 0 -> beta * C)
 *   oracle_spmm_golden_f64  SpmmGolden, the tests' fp64 reference
 *                           (test/spmm_op/spmm_op_golden.h:140-226)
 *   oracle_half_from_float_away  fp32 -> fp16 round to nearest, ties away
 *                           from zero (RoundMode::CAST_ROUND)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------ Mersenne Twister ------------------------------ */

#define MT_N 624
#define MT_M 397

typedef struct {
    uint32_t s[MT_N];
    int i;
} Mt;

static void MtSeed(Mt *mt, uint32_t seed)
{
    mt->s[0] = seed;
    for (int i = 1; i < MT_N; ++i) {
        mt->s[i] = 1812433253u * (mt->s[i - 1] ^ (mt->s[i - 1] >> 30)) + (uint32_t)i;
    }
    mt->i = MT_N;
}

static uint32_t MtNext(Mt *mt)
{
    if (mt->i >= MT_N) {
        for (int k = 0; k < MT_N; ++k) {
            const uint32_t y = (mt->s[k] & 0x80000000u) | (mt->s[(k + 1) % MT_N] & 0x7FFFFFFFu);
            mt->s[k] = mt->s[(k + MT_M) % MT_N] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
        }
        mt->i = 0;
    }
    uint32_t y = mt->s[mt->i++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9D2C5680u;
    y ^= (y << 15) & 0xEFC60000u;
    y ^= y >> 18;
    return y;
}

void oracle_mt19937_fill(uint32_t seed, int64_t count, uint32_t *out)
{
    Mt mt;
    MtSeed(&mt, seed);
    for (int64_t i = 0; i < count; ++i) out[i] = MtNext(&mt);
}

void oracle_uniform_real(uint32_t seed, double lo, double hi, int64_t count, double *out)
{
    Mt mt;
    MtSeed(&mt, seed);
    const double r = 4294967296.0;
    for (int64_t i = 0; i < count; ++i) {
        double sum = (double)MtNext(&mt);
        sum += (double)MtNext(&mt) * r;
        double u = sum / (r * r);
        if (u >= 1.0) u = nextafter(1.0, 0.0);
        out[i] = u * (hi - lo) + lo;
    }
}

/* ------------------------------ fp16 ties-away cast ------------------------------ */

uint16_t oracle_half_from_float_away(float v)
{
    uint32_t x;
    memcpy(&x, &v, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    /* exponent of v as an fp16 and the value in units of the fp16 spacing there */
    const int e = (int)(a >> 23) - 127;
    if (e >= 16) return (uint16_t)(sign | 0x7C00u);
    if (e < -25) return (uint16_t)sign;
    const uint64_t mant = (a & 0x7FFFFFu) | 0x800000u;   /* value = mant * 2^(e-23) */
    const int unitExp = e >= -14 ? e - 10 : -24;          /* fp16 spacing at v */
    const int shift = unitExp - (e - 23);                 /* >= 13 */
    uint64_t q = mant >> shift;
    const uint64_t rem = mant & ((1ull << shift) - 1ull);
    if (rem >= (1ull << (shift - 1))) q += 1;             /* ties away from zero */
    /* q counts fp16 units of 2^unitExp: rebuild the bits */
    uint32_t bits;
    if (unitExp == -24) {
        bits = (uint32_t)q;                               /* subnormal (q may reach 0x400: smallest normal) */
    } else {
        bits = ((uint32_t)(e + 15) << 10) + (uint32_t)(q - 1024u);  /* q in [1024, 2048] */
    }
    if (bits >= 0x7C00u) bits = 0x7C00u;
    return (uint16_t)(sign | bits);
}

static float HalfRoundTrip(float v)
{
    const uint16_t h = oracle_half_from_float_away(v);
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    float f;
    if (exp == 0) {
        f = ldexpf((float)mant, -24);
    } else if (exp == 31) {
        const uint32_t u = 0x7F800000u | (mant << 13);
        memcpy(&f, &u, sizeof f);
    } else {
        f = ldexpf((float)(mant | 0x400u), (int)exp - 25);
    }
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    u |= sign;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* ------------------------------ SpMMOp arithmetic ------------------------------ */

/*
 * rowPtr/col carry the index base; val, b and c hold fp32 values (fp16 data
 * already widened, which is exact).  op(B)(t, j) = b[t*ldb + j] when bContig,
 * else b[j*ldb + t]; C(i, j) = c[i*ldc + j] when cRow, else c[j*ldc + i].
 * c is read (beta != 0) and overwritten with the values the kernel stores
 * (for fp16 output: the value of the stored fp16).
 */
void oracle_spmm_f32(int64_t m, int64_t k, int64_t n, const int64_t *rowPtr, const int32_t *col, const float *val,
                     int64_t nnz, int32_t base, const float *b, int64_t ldb, int32_t bContig, float *c, int64_t ldc,
                     int32_t cRow, float alpha, float beta, int32_t kahan, int32_t halfOut)
{
    const int betaZero = beta == 0.0f;
    /* op(B) rows contiguous: a k x n copy when B is stored the other way */
    float *bt = NULL;
    if (!bContig && k > 0 && n > 0) {
        bt = (float *)malloc((size_t)(k * n) * sizeof(float));
        for (int64_t j = 0; j < n; ++j)
            for (int64_t t = 0; t < k; ++t) bt[t * n + j] = b[j * ldb + t];
        b = bt;
        ldb = n;
        bContig = 1;
    }
    float *acc = (float *)calloc((size_t)(n > 0 ? n : 1), sizeof(float));
    float *comp = (float *)calloc((size_t)(n > 0 ? n : 1), sizeof(float));
    for (int64_t i = 0; i < m; ++i) {
        const int64_t rs = rowPtr[i] - base, re = rowPtr[i + 1] - base;
        for (int64_t j = 0; j < n; ++j) acc[j] = comp[j] = 0.0f;
        /* entry-major: every output column still sums its products in CSR order */
        for (int64_t p = (nnz == 0 ? re : rs); p < re; ++p) {
            const int64_t t = (int64_t)col[p] - base;
            if (t < 0 || t >= k) continue;
            const float v = val[p];
            const float *brow = b + t * ldb;
            for (int64_t j = 0; j < n; ++j) {
                const float prod = v * brow[j];
                if (kahan) {
                    const float y = prod - comp[j];
                    const float s = acc[j] + y;
                    comp[j] = (s - acc[j]) - y;
                    acc[j] = s;
                } else {
                    acc[j] = acc[j] + prod;
                }
            }
        }
        for (int64_t j = 0; j < n; ++j) {
            const int64_t ci = cRow ? i * ldc + j : j * ldc + i;
            float out;
            if (nnz == 0) {
                out = betaZero ? 0.0f : beta * c[ci];
            } else {
                out = alpha * acc[j];
                if (!betaZero) {
                    const float bc = beta * c[ci];
                    out = out + bc;
                }
            }
            if (halfOut) {
                out = out > 65504.0f ? 65504.0f : out;
                out = out < -65504.0f ? -65504.0f : out;
                out = HalfRoundTrip(out);
            }
            c[ci] = out;
        }
    }
    free(acc);
    free(comp);
    free(bt);
}

/* b and cInit in canonical row-major order of their logical shapes (k x n, or n x k when bTrans). */
void oracle_spmm_golden_f64(int64_t m, int64_t k, int64_t n, const int64_t *rowPtr, const int32_t *col,
                            const double *val, int32_t base, const double *b, int32_t bTrans, const double *cInit,
                            double alpha, double beta, double *out)
{
    double *dot = (double *)calloc((size_t)(n > 0 ? n : 1), sizeof(double));
    /* op(B) as k x n row-major (a copy when B is given n x k) */
    double *bt = NULL;
    const double *bk = b;
    if (bTrans && k > 0 && n > 0) {
        bt = (double *)malloc((size_t)(k * n) * sizeof(double));
        for (int64_t j = 0; j < n; ++j)
            for (int64_t t = 0; t < k; ++t) bt[t * n + j] = b[j * k + t];
        bk = bt;
    }
    for (int64_t i = 0; i < m; ++i) {
        const int64_t s = rowPtr[i] - base, e = rowPtr[i + 1] - base;
        for (int64_t j = 0; j < n; ++j) dot[j] = 0.0;
        for (int64_t p = s; p < e; ++p) {  /* each column's dot still runs over p in order */
            const int64_t t = (int64_t)col[p] - base;
            if (t < 0 || t >= k) continue;
            const double v = val[p];
            const double *brow = bk + t * n;
            for (int64_t j = 0; j < n; ++j) dot[j] += v * brow[j];
        }
        for (int64_t j = 0; j < n; ++j) out[i * n + j] = alpha * dot[j] + beta * cInit[i * n + j];
    }
    free(bt);
    free(dot);
}
