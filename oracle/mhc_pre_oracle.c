/*
 * CPU oracle for the MhcPre operator -- TEST INFRASTRUCTURE ONLY.
 * See mhc_pre_oracle.h for who may use it and which reference lines each part
 * restates.  Compile with -ffp-contract=off and no fast-math.
 */
#include "mhc_pre_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Host tile length of the RMS pass: code/op_host/mhc_pre.cpp:11,152. */
#define ORACLE_SUMSQ_TILE 512

static uint32_t f32_bits(float v)
{
    uint32_t b;
    memcpy(&b, &v, 4);
    return b;
}

static float bits_f32(uint32_t b)
{
    float v;
    memcpy(&v, &b, 4);
    return v;
}

/* fp32 -> fp16, round-half-even, subnormals and overflow-to-inf as
 * cloud_runner/runner.cpp:59-100; NaN stays NaN as audit_group_vec.py:169-170. */
uint16_t oracle_f32_to_f16(float v)
{
    const uint32_t bits = f32_bits(v);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exp = (bits >> 23) & 0xFFu;
    const uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0xFFu) {
        return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    }
    int32_t exp16 = (int32_t)exp - 127 + 15;
    if (exp16 >= 0x1F) {
        return (uint16_t)(sign | 0x7C00u);
    }
    if (exp16 <= 0) {
        const uint32_t m = mant | 0x800000u;
        const int shift = 14 - exp16;
        if (shift >= 25) {
            return (uint16_t)sign;
        }
        uint32_t half = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t threshold = 1u << (shift - 1);
        if (rem > threshold || (rem == threshold && (half & 1u))) {
            half++;
        }
        /* A carry out of the subnormal range lands on the smallest normal. */
        return (uint16_t)(sign | half);
    }
    uint32_t mant16 = mant >> 13;
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (mant16 & 1u))) {
        mant16++;
        if (mant16 == 0x400u) {
            mant16 = 0;
            exp16++;
        }
    }
    if (exp16 >= 0x1F) {
        return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)exp16 << 10) | mant16);
}

/* Exact widening (cloud_runner/runner.cpp:45-57). */
float oracle_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (h >> 15) & 1u;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t mant = h & 0x3FFu;
    float mag;
    if (exp == 0x1Fu) {
        mag = mant ? NAN : INFINITY;
    } else if (exp == 0) {
        mag = ldexpf((float)mant, -24);
    } else {
        mag = ldexpf((float)(mant | 0x400u), (int)exp - 25);
    }
    return sign ? -mag : mag;
}

/* fp32 -> bf16, round-half-even (cloud_runner/runner.cpp:102-108); NaN is kept quiet. */
uint16_t oracle_f32_to_bf16(float v)
{
    const uint32_t bits = f32_bits(v);
    if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x7FFFFFu)) {
        return (uint16_t)((bits >> 16) | 0x40u);
    }
    const uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7FFFu + lsb) >> 16);
}

float oracle_bf16_to_f32(uint16_t b)
{
    return bits_f32((uint32_t)b << 16);
}

void oracle_f32_to_f16_n(const float *src, uint16_t *dst, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        dst[i] = oracle_f32_to_f16(src[i]);
    }
}

void oracle_f32_to_bf16_n(const float *src, uint16_t *dst, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        dst[i] = oracle_f32_to_bf16(src[i]);
    }
}

void oracle_f16_to_f32_n(const uint16_t *src, float *dst, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        dst[i] = oracle_f16_to_f32(src[i]);
    }
}

void oracle_bf16_to_f32_n(const uint16_t *src, float *dst, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        dst[i] = oracle_bf16_to_f32(src[i]);
    }
}

int oracle_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Sigmoid in the reference vector order (code/op_kernel/mhc_pre.cpp:542-555):
 * v*scale, +bias, *(-1), Exp, +1, 1/., +eps (the +eps only when eps != 0). */
static float oracle_sigmoid(float scaled, float bias, float eps)
{
    float v = scaled * 1.0f;
    v = v + bias;
    v = v * -1.0f;
    v = expf(v);
    v = v + 1.0f;
    v = 1.0f / v;
    if (eps != 0.0f) {
        v = v + eps;
    }
    return v;
}

/* hIn[d] = RNE(((hPre[0]*x0 + hPre[1]*x1) + ...) + hPre[n-1]*x_{n-1}) on raw x
 * (mhc_pre.cpp:787-813: broadcast multiply, stream-ordered add, CAST_RINT). */
static void stream_sum_row(const float *xf, int is_bf16, int n, int64_t D, const float *pre,
                           uint16_t *h_in)
{
    for (int64_t d = 0; d < D; ++d) {
        float a = pre[0] * xf[d];
        for (int s = 1; s < n; ++s) {
            const float p = pre[s] * xf[(int64_t)s * D + d];
            a = a + p;
        }
        h_in[d] = is_bf16 ? oracle_f32_to_bf16(a) : oracle_f32_to_f16(a);
    }
}

/* One row of the operator.  `phi_t` is phi transposed to [K][M] so the GEMM's
 * inner loop runs over the M independent accumulators; each accumulator still
 * sums its products in increasing k, one rounding per product and per add. */
static void oracle_row(const uint16_t *xrow, int is_bf16, int n, int64_t D,
                       const float *phi_t, const float *alpha, const float *bias,
                       const float *gamma, float norm_eps, float hc_eps,
                       float inv_flat, float *xf, float *acc,
                       uint16_t *h_in, float *h_post, float *h_res, float *h_pre,
                       float *mix_out, float *inv_rms_out)
{
    const int64_t K = (int64_t)n * D;
    const int M = n * n + 2 * n;

    /* Cast (mhc_pre.cpp:454, CAST_NONE: exact). */
    for (int64_t k = 0; k < K; ++k) {
        xf[k] = is_bf16 ? oracle_bf16_to_f32(xrow[k]) : oracle_f16_to_f32(xrow[k]);
    }

    /* Sum of squares: one partial per 512-element tile (mhc_pre.cpp:461-465),
     * partials added in tile order by the scalar unit (mhc_pre.cpp:484-497).
     * The order inside one tile belongs to the hardware ReduceSum; it is taken
     * as sequential here. */
    float sumsq = 0.0f;
    for (int64_t t0 = 0; t0 < K; t0 += ORACLE_SUMSQ_TILE) {
        const int64_t t1 = (t0 + ORACLE_SUMSQ_TILE < K) ? t0 + ORACLE_SUMSQ_TILE : K;
        float s = 0.0f;
        for (int64_t k = t0; k < t1; ++k) {
            const float sq = xf[k] * xf[k];
            s = s + sq;
        }
        sumsq = sumsq + s;
    }
    /* invRms = 1 / sqrt(sumsq * invFlatDim + normEps): Muls, Adds, Sqrt, then a
     * Div of a ones vector (mhc_pre.cpp:504-519) -- sqrt then divide. */
    float inv_rms = sumsq * inv_flat;
    inv_rms = inv_rms + norm_eps;
    inv_rms = sqrtf(inv_rms);
    inv_rms = 1.0f / inv_rms;

    /* Mixing GEMM on xg = x * gamma (squares were taken before gamma,
     * mhc_pre.cpp:461-468); fp32 products and fp32 accumulation. */
    for (int j = 0; j < M; ++j) {
        acc[j] = 0.0f;
    }
    for (int64_t k = 0; k < K; ++k) {
        const float xg = gamma ? xf[k] * gamma[k] : xf[k];
        const float *prow = phi_t + k * M;
        for (int j = 0; j < M; ++j) {
            const float p = xg * prow[j];
            acc[j] = acc[j] + p;
        }
    }

    /* Epilogue, scalars first (mhc_pre.cpp:735-758). */
    const float s_pre = inv_rms * alpha[0];
    const float s_post = inv_rms * alpha[1];
    const float s_res = inv_rms * alpha[2];
    float pre_local[8];
    for (int i = 0; i < n; ++i) {
        pre_local[i] = oracle_sigmoid(acc[i] * s_pre, bias[i], hc_eps);
        const float post = oracle_sigmoid(acc[n + i] * s_post, bias[n + i], 0.0f);
        h_post[i] = post * 2.0f;
        if (h_pre) {
            h_pre[i] = pre_local[i];
        }
    }
    for (int ij = 0; ij < n * n; ++ij) {
        const float scaled = acc[2 * n + ij] * s_res;
        h_res[ij] = scaled + bias[2 * n + ij];
    }

    stream_sum_row(xf, is_bf16, n, D, pre_local, h_in);

    if (mix_out) {
        memcpy(mix_out, acc, sizeof(float) * (size_t)M);
    }
    if (inv_rms_out) {
        *inv_rms_out = inv_rms;
    }
}

int oracle_mhc_pre(const uint16_t *x, int is_bf16, int64_t T, int n, int64_t D,
                   const float *phi, const float *alpha, const float *bias,
                   const float *gamma, float norm_eps, float hc_eps,
                   const int64_t *rows, int64_t nrows,
                   uint16_t *h_in, float *h_post, float *h_res, float *h_pre,
                   float *mix, float *inv_rms, int nthreads)
{
    if (!x || !phi || !alpha || !bias || !h_in || !h_post || !h_res) {
        return 1;
    }
    if (n < 1 || n > 8 || D <= 0 || T <= 0 || nrows < 0) {
        return 2;
    }
    const int64_t K = (int64_t)n * D;
    const int M = n * n + 2 * n;
    for (int64_t i = 0; i < nrows; ++i) {
        const int64_t r = rows ? rows[i] : i;
        if (r < 0 || r >= T) {
            return 3;
        }
    }
    /* invFlatDim = fl(1.0f / K), computed on the host (code/op_host/mhc_pre.cpp:154). */
    const float inv_flat = 1.0f / (float)K;

    float *phi_t = (float *)malloc(sizeof(float) * (size_t)K * (size_t)M);
    if (!phi_t) {
        return 4;
    }
    /* phi is read as [M][K] (code/op_kernel/mhc_pre.cpp:229,535, B transposed). */
    for (int j = 0; j < M; ++j) {
        for (int64_t k = 0; k < K; ++k) {
            phi_t[k * M + j] = phi[(int64_t)j * K + k];
        }
    }

    int err = 0;
#ifdef _OPENMP
    const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel num_threads(nt) reduction(| : err)
#endif
    {
        float *xf = (float *)malloc(sizeof(float) * (size_t)K);
        float *acc = (float *)malloc(sizeof(float) * (size_t)M);
        if (!xf || !acc) {
            err |= 4;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (int64_t i = 0; i < nrows; ++i) {
                const int64_t r = rows ? rows[i] : i;
                oracle_row(x + r * K, is_bf16, n, D, phi_t, alpha, bias, gamma,
                           norm_eps, hc_eps, inv_flat, xf, acc,
                           h_in + i * D, h_post + i * n, h_res + i * (int64_t)n * n,
                           h_pre ? h_pre + i * n : NULL, mix ? mix + i * M : NULL,
                           inv_rms ? inv_rms + i : NULL);
            }
        }
        free(xf);
        free(acc);
    }
    (void)nthreads;
    free(phi_t);
    return err;
}

/* The reference harnesses draw x, then phi, then bias, then gamma from one
 * glibc rand() stream (cloud_runner/runner.cpp:370-382;
 * cloud_runner/probe_e1e2.cpp:242-254). */
void oracle_reference_harness_inputs(unsigned seed, int64_t T, int n, int64_t D,
                                     float *x, float *phi, float *bias, float *gamma)
{
    const int64_t K = (int64_t)n * D;
    const int64_t M = (int64_t)n * n + 2 * n;
    srand(seed);
    for (int64_t i = 0; i < T * K; ++i) {
        x[i] = (float)(rand() % 2000) / 10000.0f - 0.1f;
    }
    for (int64_t i = 0; i < K * M; ++i) {
        phi[i] = (float)(rand() % 200) / 10000.0f - 0.01f;
    }
    for (int64_t i = 0; i < M; ++i) {
        bias[i] = (float)(rand() % 200) / 10000.0f - 0.01f;
    }
    for (int64_t i = 0; i < K; ++i) {
        gamma[i] = 1.0f + (float)(rand() % 200) / 10000.0f;
    }
}

int oracle_weighted_stream_sum(const uint16_t *x, int is_bf16, int64_t R, int n, int64_t D,
                               const float *h_pre, uint16_t *h_in)
{
    if (!x || !h_pre || !h_in || n < 1 || n > 8 || D <= 0 || R < 0) {
        return 1;
    }
    const int64_t K = (int64_t)n * D;
    float *xf = (float *)malloc(sizeof(float) * (size_t)K);
    if (!xf) {
        return 4;
    }
    for (int64_t r = 0; r < R; ++r) {
        for (int64_t k = 0; k < K; ++k) {
            xf[k] = is_bf16 ? oracle_bf16_to_f32(x[r * K + k]) : oracle_f16_to_f32(x[r * K + k]);
        }
        stream_sum_row(xf, is_bf16, n, D, h_pre + r * n, h_in + r * D);
    }
    free(xf);
    return 0;
}
