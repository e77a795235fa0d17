/*
 * CPU checker (test infrastructure only): the grouped GEMM of the oracle in
 * the HIP kernels' accumulation order, written in C so that whole expert
 * spans at the benchmark shapes (about 1e11 multiply-adds) take seconds.
 *
 * It computes exactly what oracle/moe_oracle.py:_mfma_order_matmul computes:
 *   c[r, j] = acc after the last group, where for each ascending group of
 *   `group` k indices  acc = (float)((double)acc + S),  S = the sum of the
 *   group's products a[r, k] * b[j, k] taken in double.
 * Inputs hold bf16 values (as float), so every product is exact in double and
 * so is the sum of a group of 8 for data of ordinary dynamic range; the only
 * rounding is the one to float per group. k is padded with zeros to a whole
 * number of groups. (The accumulation model itself follows the reference's
 * grouped GEMM contract, src/moe_dispatch/experts.py:21-35: fp32 accumulation,
 * bf16 inputs.)
 *
 * Build: gcc -O3 -fopenmp -mavx2 -mfma -ffp-contract=off -shared -fPIC
 *        oracle/mfma_gemm.c -o oracle/_build/libmoe_oracle.so   (see build() in __graft_entry__.py)
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define COLS 32 /* output columns per block: one block's accumulators stay in registers/L1 */

void moe_oracle_mfma_gemm(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                          int64_t group) {
    const int64_t groups = (k + group - 1) / group;
    const int64_t kpad = groups * group;
    const int64_t blocks = (n + COLS - 1) / COLS;
#pragma omp parallel
    {
        double* bt = (double*)malloc(sizeof(double) * (size_t)kpad * COLS); /* [kpad][COLS] */
#pragma omp for schedule(dynamic, 1)
        for (int64_t blk = 0; blk < blocks; ++blk) {
            const int64_t c0 = blk * COLS;
            const int64_t cn = n - c0 < COLS ? n - c0 : COLS;
            for (int64_t kk = 0; kk < kpad; ++kk)
                for (int64_t j = 0; j < COLS; ++j)
                    bt[kk * COLS + j] = (j < cn && kk < k) ? (double)b[(c0 + j) * k + kk] : 0.0;
            for (int64_t r = 0; r < m; ++r) {
                const float* ar = a + r * k;
                float acc[COLS];
                double s[COLS];
                for (int64_t j = 0; j < COLS; ++j) acc[j] = 0.0f;
                for (int64_t g = 0; g < groups; ++g) {
                    for (int64_t j = 0; j < COLS; ++j) s[j] = 0.0;
                    for (int64_t q = 0; q < group; ++q) {
                        const int64_t kk = g * group + q;
                        const double av = kk < k ? (double)ar[kk] : 0.0;
                        const double* brow = bt + kk * COLS;
                        for (int64_t j = 0; j < COLS; ++j) s[j] += av * brow[j];
                    }
                    for (int64_t j = 0; j < COLS; ++j) acc[j] = (float)((double)acc[j] + s[j]);
                }
                float* cr = c + r * n + c0;
                for (int64_t j = 0; j < cn; ++j) cr[j] = acc[j];
            }
        }
        free(bt);
    }
}
