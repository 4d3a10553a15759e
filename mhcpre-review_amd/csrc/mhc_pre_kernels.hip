// MhcPre HIP kernels for gfx950 (CDNA4).
//
// Stages (reference: code/op_kernel/mhc_pre.cpp):
//   prep_b          gamma (.) phi split into bf16 hi + lo, laid out as MFMA B fragments
//   gemm_partial    split-K mixing GEMM on bf16 MFMA (fp32 accumulate) + sum of squares
//   epilogue_hin    fixed-order reduction of the partials, invRms, sigmoid / affine
//                   epilogue, weighted stream reduction with RNE stores
//
// Numerics.  x (bf16) is exact as an MFMA operand; fp16 x is split exactly into
// bf16 hi + lo.  B = gamma*phi (fp32) is split into bf16 hi + lo with a residual
// below 2^-17 |B|, and both halves go through the MFMA into fp32 accumulators,
// so the GEMM carries fp32-level accuracy at bf16 MFMA rate.  Everything after
// the GEMM is fp32 in the reference kernel's operation order (built with
// -ffp-contract=off: one rounding per product and per sum).

#include "mhc_pre_device.h"
#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace mhc {
namespace {

using namespace dev;

// ---------------------------------------------------------------------------
// prep_b: B operand fragments.
//
// Layout: [ks = K/32][ct = NT][lane 64] x 16 bytes.  Lane l of fragment
// (ks, ct) holds B[k = 32ks + 8(l/16) + e][c = 16ct + l%16] for e = 0..7,
// where column c < M is hi(gamma[k]*phi_mem[c*K + k]) and c >= M is the lo
// half of column c - M.  A wave loads one fragment as 1 KiB contiguous.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prep_b_kernel(const float *__restrict__ phi,
                                                     const float *__restrict__ gamma,
                                                     u32x4_t *__restrict__ bsplit, int64_t K,
                                                     int M, int NT, uint32_t *__restrict__ status)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx == 0 && status != nullptr) {
        *status = kDeviceOk;
    }
    const int64_t total = (K / 32) * NT * kWave;
    if (idx >= total) {
        return;
    }
    const int lane = (int)(idx % kWave);
    const int ct = (int)((idx / kWave) % NT);
    const int64_t ks = idx / ((int64_t)kWave * NT);
    const int c = 16 * ct + (lane & 15);
    const bool isLo = c >= M;
    const int j = isLo ? c - M : c;
    const int64_t k0 = ks * 32 + 8 * (lane >> 4);

    const f32x4_t *src = reinterpret_cast<const f32x4_t *>(phi + (int64_t)j * K + k0);
    const f32x4_t p0 = src[0], p1 = src[1];
    float b[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
    if (gamma != nullptr) {
        const f32x4_t *gs = reinterpret_cast<const f32x4_t *>(gamma + k0);
        const f32x4_t g0 = gs[0], g1 = gs[1];
        const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            b[e] = b[e] * g[e];
        }
    }
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float hi = bf16_bits_to_f32(f32_to_bf16_bits(b[e]));
        out[e] = isLo ? (b[e] - hi) : hi;
    }
    // Nontemporal: read by the next kernel (lines left in this XCD's L2 slow
    // its reads of B down).
    __builtin_nontemporal_store(pack8_bf16(out), &bsplit[idx]);
}

// ---------------------------------------------------------------------------
// split_b_from_prepared: the same fragments from prepared weights (layout of
// launch_prepare_b: per k-step, tile t < Q = M/16 holds hi of columns
// 16t + l%16, tile Q + t their lo, and when M % 16 == 8 tile 2Q holds hi
// (lanes l%16 < 8) and lo (the others) of column 16Q + l%8).  Every 16-byte
// fragment lane is copied from the prepared lane holding the same column
// half and k.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void split_b_from_prepared_kernel(const u32x4_t *__restrict__ src,
                                                                    u32x4_t *__restrict__ bsplit,
                                                                    int64_t K, int M, int NT,
                                                                    uint32_t *__restrict__ status)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx == 0 && status != nullptr) {
        *status = kDeviceOk;
    }
    const int64_t total = (K / 32) * NT * kWave;
    if (idx >= total) {
        return;
    }
    const int lane = (int)(idx % kWave);
    const int ct = (int)((idx / kWave) % NT);
    const int64_t ks = idx / ((int64_t)kWave * NT);
    const int c = 16 * ct + (lane & 15);
    const bool lo = c >= M;
    const int j = lo ? c - M : c;
    const int Q = M / 16;
    int tile, sl;
    if (j < 16 * Q) {
        tile = (lo ? Q : 0) + j / 16;
        sl = (j % 16) + 16 * (lane >> 4);
    } else {
        tile = 2 * Q;
        sl = (j - 16 * Q) + (lo ? 8 : 0) + 16 * (lane >> 4);
    }
    __builtin_nontemporal_store(src[(ks * NT + tile) * kWave + sl], &bsplit[idx]);
}

// ---------------------------------------------------------------------------
// gemm_partial: one workgroup = 4 waves = one 16-row tile x one K-slice.
// Waves interleave the slice's 32-wide k-steps; the workgroup reduces its
// waves through LDS in wave order and writes
//   partial[slice][row][j]  j < M : sum over the slice of xg . B (hi + lo)
//   partial[slice][row][M]        : sum over the slice of x^2
// A fragment (lane l): x[row0 + l%16][32ks + 8(l/16) .. +8], one 16-byte load.
// C fragment (lane l, reg i): C[4(l/16) + i][l%16].
// ---------------------------------------------------------------------------
template <int N, bool kBf16>
__global__ __launch_bounds__(256) void gemm_partial_kernel(const uint16_t *__restrict__ x,
                                                           const u32x4_t *__restrict__ bsplit,
                                                           float *__restrict__ partial, int64_t T,
                                                           int64_t K, int ksPerSlice)
{
    using S = Shape<N>;
    constexpr int M = S::M;
    constexpr int NT = S::NT;
    constexpr int LDW = 2 * M + 1;  // LDS row stride (floats): [hi | lo] columns + sumsq
    __shared__ float red[4][16][LDW];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int64_t row = (int64_t)blockIdx.x * 16 + (lane & 15);
    const bool rowOk = row < T;
    const int slice = blockIdx.y;
    const int64_t ksTotal = K / 32;
    const int64_t ksBegin = (int64_t)slice * ksPerSlice;
    const int64_t ksEnd = ksBegin + ksPerSlice < ksTotal ? ksBegin + ksPerSlice : ksTotal;

    f32x4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    float ss = 0.f;
    const uint16_t *xrow = x + (rowOk ? row : 0) * K + 8 * g;

    for (int64_t ks = ksBegin + wave; ks < ksEnd; ks += 4) {
        u32x4_t xa = u32x4_t{0u, 0u, 0u, 0u};
        if (rowOk) {
            xa = *reinterpret_cast<const u32x4_t *>(xrow + ks * 32);
        }
        u32x4_t bfrag[NT];
        const u32x4_t *bsrc = bsplit + (ks * NT) * kWave + lane;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            bfrag[t] = bsrc[t * kWave];
        }
        ss = sumsq8<kBf16>(xa, ss);
        if constexpr (kBf16) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                acc[t] = mfma16(xa, bfrag[t], acc[t]);
            }
        } else {
            float f[8];
            unpack8<kBf16>(xa, f);
            u32x4_t ahi, alo;
            split_f16_to_bf16(f, ahi, alo);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                acc[t] = mfma16(ahi, bfrag[t], acc[t]);
            }
#pragma unroll
            for (int t = 0; t < S::NTHI; ++t) {
                acc[t] = mfma16(alo, bfrag[t], acc[t]);
            }
        }
    }

    // Row sum of squares: the 4 lane groups of a row, fixed pairing order.
    ss = ss + __shfl_xor(ss, 16);
    ss = ss + __shfl_xor(ss, 32);

#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            red[wave][4 * g + i][16 * t + (lane & 15)] = acc[t][i];
        }
    }
    if (g == 0) {
        red[wave][lane & 15][2 * M] = ss;
    }
    __syncthreads();

    const int64_t rowBase = (int64_t)blockIdx.x * 16;
    float *dst = partial + ((int64_t)slice * T) * (M + 1);
    for (int idx = threadIdx.x; idx < 16 * (M + 1); idx += blockDim.x) {
        const int r = idx / (M + 1);
        const int j = idx % (M + 1);
        if (rowBase + r >= T) {
            continue;
        }
        float v;
        if (j < M) {
            v = (red[0][r][j] + red[0][r][M + j]);
            v = v + (red[1][r][j] + red[1][r][M + j]);
            v = v + (red[2][r][j] + red[2][r][M + j]);
            v = v + (red[3][r][j] + red[3][r][M + j]);
        } else {
            v = ((red[0][r][2 * M] + red[1][r][2 * M]) + red[2][r][2 * M]) + red[3][r][2 * M];
        }
        dst[(rowBase + r) * (M + 1) + j] = v;
    }
}

// ---------------------------------------------------------------------------
// epilogue_hin: one workgroup per row.  Reduces the split-K partials in slice
// order, then the epilogue (code/op_kernel/mhc_pre.cpp:735-758) and the
// weighted stream reduction with RNE stores (code/op_kernel/mhc_pre.cpp:761-826).
// ---------------------------------------------------------------------------
template <int N, bool kBf16>
__global__ __launch_bounds__(256) void epilogue_hin_kernel(
    const uint16_t *__restrict__ x, const float *__restrict__ partial, int S, int64_t T,
    int64_t D, int64_t row0, const float *__restrict__ alpha, const float *__restrict__ bias,
    float normEps, float hcEps, float invFlatDim, uint16_t *__restrict__ hIn,
    float *__restrict__ hPost, float *__restrict__ hRes, float *__restrict__ hPre)
{
    constexpr int M = Shape<N>::M;
    __shared__ float smix[M + 1];
    __shared__ float spre[N];
    const int64_t row = row0 + blockIdx.x;  // row0: first row of this launch
    const int tid = threadIdx.x;

    if (tid <= M) {
        float a = 0.f;
        for (int s = 0; s < S; ++s) {
            a = a + partial[((int64_t)s * T + row) * (M + 1) + tid];
        }
        smix[tid] = a;
    }
    __syncthreads();

    if (tid < M) {
        const float invRms = ref_inv_rms(smix[M], invFlatDim, normEps);
        const float mix = smix[tid];
        if (tid < N) {
            const float sP = invRms * alpha[0];
            const float v = ref_sigmoid(mix * sP, bias[tid], hcEps);
            spre[tid] = v;
            if (hPre != nullptr) {
                hPre[row * N + tid] = v;
            }
        } else if (tid < 2 * N) {
            const float sQ = invRms * alpha[1];
            const float v = ref_sigmoid(mix * sQ, bias[tid], 0.0f);
            hPost[row * N + (tid - N)] = v * 2.0f;
        } else {
            const float sR = invRms * alpha[2];
            const float v = mix * sR;
            hRes[row * (N * N) + (tid - 2 * N)] = v + bias[tid];
        }
    }
    __syncthreads();

    float pre[N];
#pragma unroll
    for (int s = 0; s < N; ++s) {
        pre[s] = spre[s];
    }
    const uint16_t *xr = x + row * (N * D);
    uint16_t *out = hIn + row * D;
    for (int64_t d8 = tid; d8 < D / 8; d8 += blockDim.x) {
        float acc[8];
        {
            float f[8];
            unpack8<kBf16>(*reinterpret_cast<const u32x4_t *>(xr + d8 * 8), f);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                acc[e] = pre[0] * f[e];
            }
        }
#pragma unroll
        for (int s = 1; s < N; ++s) {
            float f[8];
            unpack8<kBf16>(*reinterpret_cast<const u32x4_t *>(xr + s * D + d8 * 8), f);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float p = pre[s] * f[e];
                acc[e] = acc[e] + p;
            }
        }
        u32x4_t o;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            o[w] = pack2_x<kBf16>(acc[2 * w], acc[2 * w + 1]);
        }
        *reinterpret_cast<u32x4_t *>(out + d8 * 8) = o;
    }
}

template <int N, bool kBf16>
hipError_t launch_split_t(const Plan &p, void *workspace, hipStream_t stream)
{
    char *ws = static_cast<char *>(workspace);
    uint32_t *status = reinterpret_cast<uint32_t *>(ws);
    u32x4_t *bsplit = reinterpret_cast<u32x4_t *>(ws + p.wsBsplit);
    float *partial = reinterpret_cast<float *>(ws + p.wsPartial);

    const int64_t prepThreads = (p.K / 32) * p.NT * kWave;
    if (p.bprep != nullptr) {
        hipLaunchKernelGGL(split_b_from_prepared_kernel, dim3((unsigned)((prepThreads + 255) / 256)),
                           dim3(256), 0, stream, static_cast<const u32x4_t *>(p.bprep), bsplit, p.K,
                           p.M, p.NT, status);
    } else {
        hipLaunchKernelGGL(prep_b_kernel, dim3((unsigned)((prepThreads + 255) / 256)), dim3(256), 0,
                           stream, p.phi, p.hasGamma ? p.gamma : nullptr, bsplit, p.K, p.M, p.NT,
                           status);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    const unsigned rowTiles = (unsigned)((p.T + 15) / 16);
    hipLaunchKernelGGL((gemm_partial_kernel<N, kBf16>), dim3(rowTiles, (unsigned)p.splitS),
                       dim3(256), 0, stream, static_cast<const uint16_t *>(p.x), bsplit, partial,
                       p.T, p.K, p.ksPerSlice);
    err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    // One workgroup per row, kEpilogueRowsPerLaunch rows per launch.
    for (int64_t r0 = 0; r0 < p.T; r0 += kEpilogueRowsPerLaunch) {
        const dim3 grid((unsigned)std::min<int64_t>(kEpilogueRowsPerLaunch, p.T - r0));
        hipLaunchKernelGGL((epilogue_hin_kernel<N, kBf16>), grid, dim3(256), 0, stream,
                           static_cast<const uint16_t *>(p.x), partial, p.splitS, p.T, p.D, r0,
                           p.alpha, p.bias, p.normEps, p.hcEps, p.invFlatDim,
                           static_cast<uint16_t *>(p.hIn), p.hPost, p.hRes,
                           p.hasHPre ? p.hPre : nullptr);
        err = hipGetLastError();
        if (err != hipSuccess) {
            return err;
        }
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_split(const Plan &p, void *workspace, hipStream_t stream)
{
    switch (p.n) {
    case 4:
        return p.isBf16 ? launch_split_t<4, true>(p, workspace, stream)
                        : launch_split_t<4, false>(p, workspace, stream);
    case 6:
        return p.isBf16 ? launch_split_t<6, true>(p, workspace, stream)
                        : launch_split_t<6, false>(p, workspace, stream);
    case 8:
        return p.isBf16 ? launch_split_t<8, true>(p, workspace, stream)
                        : launch_split_t<8, false>(p, workspace, stream);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace mhc
