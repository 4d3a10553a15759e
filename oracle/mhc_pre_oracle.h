/*
 * CPU oracle for the MhcPre operator.
 *
 * TEST INFRASTRUCTURE ONLY.  Only the test suite, the smoke check and the
 * benchmark's cpu_baseline leg may load this library, and only as the checker
 * (or, in the benchmark, as the timed CPU baseline).  The product path
 * (libmhcpre.so) never links, loads or calls it.
 *
 * It restates the reference AscendC kernel's arithmetic in plain C, in the
 * kernel's floating-point order:
 *   code/op_kernel/mhc_pre.cpp:393-520  PreprocessRows (cast, sumsq, gamma, invRms)
 *   code/op_kernel/mhc_pre.cpp:522-540  ProjectWithCube (mix = xg . phi_mem[M][K]^T)
 *   code/op_kernel/mhc_pre.cpp:542-555  Sigmoid
 *   code/op_kernel/mhc_pre.cpp:732-758  PostprocessRows epilogue
 *   code/op_kernel/mhc_pre.cpp:761-826  weighted stream reduction + CAST_RINT
 *   code/op_host/mhc_pre.cpp:11,94-95,152-157  tile 512, eps defaults, invFlatDim
 *   cloud_runner/runner.cpp:45-116      fp16 / bf16 conversion semantics
 *
 * Built with -ffp-contract=off and without fast-math: every binary operation
 * is one IEEE fp32 rounding, as in the reference's vector unit.
 */
#ifndef MHC_PRE_ORACLE_H
#define MHC_PRE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 / bf16 helpers (cloud_runner/runner.cpp:45-116, audit_group_vec.py:165-223) */
uint16_t oracle_f32_to_f16(float v);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float v);
float oracle_bf16_to_f32(uint16_t b);
/* Vector forms used by the tests (n elements). */
void oracle_f32_to_f16_n(const float *src, uint16_t *dst, int64_t n);
void oracle_f32_to_bf16_n(const float *src, uint16_t *dst, int64_t n);
void oracle_f16_to_f32_n(const uint16_t *src, float *dst, int64_t n);
void oracle_bf16_to_f32_n(const uint16_t *src, float *dst, int64_t n);

/*
 * Full operator on a set of rows.
 *   x      raw 16-bit patterns, [T][n][D] (row r at x + r*n*D)
 *   phi    fp32, memory [M][K] with K = n*D, M = n*n + 2n (phi_mem[j*K + k])
 *   alpha  fp32 [3] = {alphaPre, alphaPost, alphaRes}
 *   bias   fp32 [M]
 *   gamma  fp32 [K] or NULL (gamma off)
 *   rows   row indices to evaluate (NULL: rows 0..nrows-1)
 * Outputs are compact, indexed by the position in `rows`:
 *   hIn [nrows][D] (16-bit patterns), hPost [nrows][n], hRes [nrows][n*n],
 *   hPre [nrows][n] (may be NULL), mix [nrows][M] (raw GEMM, may be NULL),
 *   invRms [nrows] (may be NULL).
 * nthreads <= 0 uses every available core; rows are independent, so the
 * result does not depend on the thread count.
 * Returns 0 on success, nonzero on an invalid argument.
 */
int oracle_mhc_pre(const uint16_t *x, int is_bf16, int64_t T, int n, int64_t D,
                   const float *phi, const float *alpha, const float *bias,
                   const float *gamma, float norm_eps, float hc_eps,
                   const int64_t *rows, int64_t nrows,
                   uint16_t *h_in, float *h_post, float *h_res, float *h_pre,
                   float *mix, float *inv_rms, int nthreads);

/*
 * The weighted stream reduction alone, on given hPre weights:
 *   hIn[r][d] = RNE(sum_s fl(hPre[r][s] * x[r][s][d])), streams in order
 * (the same code path oracle_mhc_pre uses).  x [R][n][D] 16-bit patterns,
 * h_pre [R][n], h_in [R][D].  Lets a test check a device's hIn stage
 * bit-exactly from the device's own hPre.
 */
int oracle_weighted_stream_sum(const uint16_t *x, int is_bf16, int64_t R, int n, int64_t D,
                               const float *h_pre, uint16_t *h_in);

/* Number of threads oracle_mhc_pre uses for nthreads <= 0. */
int oracle_max_threads(void);

/*
 * The reference test harnesses' input generators, reproduced bit-for-bit with
 * glibc rand():
 *   cloud_runner/runner.cpp:368-382 (srand(42)) and
 *   cloud_runner/probe_e1e2.cpp:242-254 (srand(7)).
 * Fills x (as float, before the fp16/bf16 cast), phi [K*M], bias [M] and
 * gamma [K] in the harness's draw order.
 */
void oracle_reference_harness_inputs(unsigned seed, int64_t T, int n, int64_t D,
                                     float *x, float *phi, float *bias, float *gamma);

#ifdef __cplusplus
}
#endif

#endif
