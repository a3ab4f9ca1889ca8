/*
 * cl3_oracle.c -- C restatement of the reference's CPU geometric matmul.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ as a checker and by bench.py's
 * cpu_baseline leg as the timed CPU path.  The product (yggdrasil_amd) never
 * links it.
 *
 * out[m, n] = sum_k gp(a[m, k], b[k, n]),  a: M x K, b: K x N, out: M x N,
 * every element a multivector of 8 contiguous floats in the basis order
 * 1, e1, e2, e3, e12, e13, e23, e123.
 *
 * Operation order restated from mjolnir/src/cpu/batch_ops.c:56-71 (zero
 * accumulator, k ascending, one full product per k then a component-wise
 * add) and mjolnir/src/cpu/geometric_product.c:17-56 (the 64 terms of one
 * product visited with the left operand's blade outer, the right operand's
 * blade inner, each term (sign * a_i) * b_j rounded before its add).  The
 * Cayley table is generated at first use from the blade bitmasks (product
 * blade = XOR of the masks, sign = parity of the transpositions needed to
 * sort the generators), not copied.
 *
 * Built with -ffp-contract=off so no multiply-add is fused: the results are
 * then bit-identical to the reference's NumPy path and to its compiled C.
 */
#include <stddef.h>
#include <stdint.h>

/* blade index (reference order) -> generator bitmask (bit0=e1, bit1=e2, bit2=e3) */
static const int kMask[8] = {0, 1, 2, 4, 3, 5, 6, 7};
static int g_idx[8][8];
static float g_sign[8][8];
static int g_ready = 0;

static int reorder_sign(int a, int b) {
    /* number of (x in a, y in b) with x > y: each is one transposition */
    int swaps = 0;
    for (int x = 0; x < 3; ++x)
        if (a & (1 << x))
            for (int y = 0; y < x; ++y)
                if (b & (1 << y)) ++swaps;
    return (swaps & 1) ? -1 : 1;
}

static void init_tables(void) {
    if (g_ready) return;
    int of_mask[8];
    for (int i = 0; i < 8; ++i) of_mask[kMask[i]] = i;
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 8; ++j) {
            g_idx[i][j] = of_mask[kMask[i] ^ kMask[j]];
            g_sign[i][j] = (float)reorder_sign(kMask[i], kMask[j]);
        }
    g_ready = 1;
}

void oracle_tables(int32_t *idx, float *sign) {
    init_tables();
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 8; ++j) {
            idx[i * 8 + j] = g_idx[i][j];
            sign[i * 8 + j] = g_sign[i][j];
        }
}

static inline void gp_acc(const float *a, const float *b, float *acc) {
    float t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 8; ++j) {
            float s = g_sign[i][j] * a[i];
            t[g_idx[i][j]] += s * b[j];
        }
    for (int r = 0; r < 8; ++r) acc[r] += t[r];
}

void oracle_geom_prod(const float *a, const float *b, float *out, size_t count) {
    init_tables();
    for (size_t n = 0; n < count; ++n) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        gp_acc(a + 8 * n, b + 8 * n, acc);
        for (int r = 0; r < 8; ++r) out[8 * n + r] = acc[r];
    }
}

static void matmul_rows(const float *a, const float *b, float *out, size_t m0, size_t m1, size_t K, size_t N) {
    for (size_t m = m0; m < m1; ++m)
        for (size_t n = 0; n < N; ++n) {
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (size_t k = 0; k < K; ++k) gp_acc(a + 8 * (m * K + k), b + 8 * (k * N + n), acc);
            for (int r = 0; r < 8; ++r) out[8 * (m * N + n) + r] = acc[r];
        }
}

/* Single-threaded, as the reference runs. */
void oracle_geom_matmul(const float *a, const float *b, float *out, size_t M, size_t K, size_t N) {
    init_tables();
    matmul_rows(a, b, out, 0, M, K, N);
}

/* OpenMP over output rows; every element keeps the serial operation order,
 * so the result is bit-identical to oracle_geom_matmul. */
void oracle_geom_matmul_omp(const float *a, const float *b, float *out, size_t M, size_t K, size_t N, int threads) {
    init_tables();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (long m = 0; m < (long)M; ++m) matmul_rows(a, b, out, (size_t)m, (size_t)m + 1, K, N);
}
