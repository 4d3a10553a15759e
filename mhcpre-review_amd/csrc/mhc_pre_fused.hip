// Fused MhcPre kernel for gfx950: x is read from HBM once and stays in VGPRs.
//
// Work decomposition.  D is cut into P slices of DW = 32*KS columns.  A unit
// is (16-row tile, slice p): the 16 rows x n streams x DW columns of x, held
// by one wave in VGPRs as the A fragments of v_mfma_f32_16x16x32_bf16.  A
// workgroup of W waves owns one slice for the whole launch and keeps that
// slice of the B operand (gamma*phi split into bf16 hi + lo) in LDS.  The P
// workgroups that own the slices of the same row tiles form a team; teams
// are XCD-local when the grid is a multiple of 8 (workgroup g runs on XCD
// g % 8 and team = g % numTeams).
//
// Per unit a wave:
//   1. multiplies its x block by the LDS B slice (MFMA, fp32 accumulate) and
//      sums x^2 from the same registers;
//   2. publishes the slice's partial sums (M mix columns + sumsq per row) and
//      counts itself in on the row tile's arrival counter;
//   3. the last of the P slices to arrive sums the hPre columns and sumsq
//      over all slices in a fixed order, evaluates invRms and hPre and
//      publishes hPre; then it sums the remaining columns and writes hPost /
//      hRes (and hPre when asked); every other slice polls the published hPre
//      of its rows;
//   4. computes hIn for its DW columns from the x still in its registers.
// The last-arriver rule needs no wave to wait for one that has not arrived,
// and the cooperative launch keeps every workgroup resident, so the waits
// always end; each is still bounded by a spin limit that records
// kDeviceTimeout in the status word instead of hanging.
//
// Exchange memory is accessed with device-scope (sc1) loads and stores, and a
// wave waits for its stores to complete (s_waitcnt) before the atomic that
// announces them; no agent-scope fence is used, because on a multi-L2 device
// each one writes back or invalidates a whole L2.

#include "mhc_pre_device.h"
#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace mhc {
namespace {

using namespace dev;

constexpr int kFusedWaves = 8;  // waves per workgroup (2 per SIMD)

struct FusedArgs {
    const uint16_t *x;
    const float *phi;
    const float *gamma;
    const float *alpha;
    const float *bias;
    uint16_t *hIn;
    float *hPost;
    float *hRes;
    float *hPre;
    float *partial;      // [RT][P] records of Rec<N>::FLOATS
    float *finalPre;     // [RT] blocks of Rec<N>::FIN
    uint32_t *arrive;    // [RT] counters, kCounterStride words apart
    uint32_t *status;
    int64_t T;
    int64_t D;
    int64_t K;
    int64_t RT;
    int P;
    int numTeams;
    float normEps;
    float hcEps;
    float invFlatDim;
    uint32_t spinLimit;
};

// Column slots of the [hi | lo] B operand, NT = 2M/16 tiles of 16 lanes:
// tiles [0,Q) hold hi of j = 16t + l, tiles [Q,2Q) lo of the same j, so hi and
// lo of a column meet in the same lane; when M % 16 == 8 the last tile holds
// hi (lanes 0-7) and lo (lanes 8-15) of j = 16Q + (l & 7).
template <int M>
struct ColLayout {
    static constexpr int Q = M / 16;
    static constexpr bool kHalfTile = (M % 16) == 8;
    static_assert(M % 16 == 0 || M % 16 == 8, "M = n*n + 2n is 24, 48 or 80");
    __device__ static void slot(int c, bool &lo, int &j)
    {
        const int t = c >> 4, l = c & 15;
        if (t < Q) {
            lo = false;
            j = 16 * t + l;
        } else if (t < 2 * Q) {
            lo = true;
            j = 16 * (t - Q) + l;
        } else {
            lo = l >= 8;
            j = 16 * Q + (l & 7);
        }
    }
    // Tiles whose columns include a hi half (fp16 x multiplies these by x_lo too).
    static constexpr bool has_hi(int t) { return t < Q || t == 2 * Q; }
};

// Exchange record of one (row tile, slice), column-major: column c holds its
// 16 rows contiguously (64 bytes).  Column N is the sum of squares; mix column
// j sits at column j (j < N, the hPre columns) or j + 1.  The column count is
// even, so a record is a whole number of 128-byte lines and no line is
// written by two slices.  A wave reads four columns of 16 rows -- one 256-byte
// span -- per load instruction.
template <int N>
struct Rec {
    static constexpr int M = N * N + 2 * N;
    static constexpr int RC = ((M + 1 + 1) / 2) * 2;
    static constexpr int FLOATS = RC * 16;
    // Per-tile broadcast block written by the last slice: hPre columns
    // 0..N-1 and invRms at column N, 16 rows each, padded to 128-byte lines.
    static constexpr int FIN = (((N + 1) * 16 + 31) / 32) * 32;
    __device__ static int col(int j) { return j < N ? j : j + 1; }
};

// Arrival counters are spaced one 256-byte line apart: device-scope atomics
// on one line serialize, and the tiles' counters are hit concurrently.
constexpr int kCounterStride = 64;  // uint32 words

// hPre slots not yet written hold this signalling-NaN pattern; arithmetic
// only ever produces quiet NaNs, so a computed hPre can never equal it.
constexpr uint32_t kPreSentinel = 0x7F80DEADu;

// Sum over slices q = 0..P-1, in that order, of the float at src + q*step;
// loads are issued 32 slices at a time so they are in flight together.
__device__ __forceinline__ float sum_over_slices(const float *src, int P, int step, bool active)
{
    float v = 0.f;
    for (int q0 = 0; q0 < P; q0 += 32) {
        float t[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            const int q = q0 + u;
            t[u] = (active && q < P) ? ld_dev(src + (int64_t)q * step) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            v = v + t[u];
        }
    }
    return v;
}

__global__ __launch_bounds__(256) void fused_reset_kernel(uint32_t *__restrict__ arrive,
                                                          uint32_t *__restrict__ finalPre,
                                                          int64_t RT, int64_t finalWords,
                                                          uint32_t *__restrict__ status)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < RT) {
        arrive[i * kCounterStride] = 0u;
    }
    if (i < finalWords) {
        finalPre[i] = kPreSentinel;
    }
    if (i == 0) {
        *status = kDeviceOk;
    }
}

template <int N, int KS, bool kBf16>
__global__ __launch_bounds__(kFusedWaves * 64) void fused_kernel(FusedArgs a)
{
    using S = Shape<N>;
    constexpr int M = S::M;
    constexpr int NT = S::NT;
    using CL = ColLayout<M>;
    using RC = Rec<N>;
    constexpr int W = kFusedWaves;
    constexpr int DW = 32 * KS;
    constexpr int Q = CL::Q;
    extern __shared__ u32x4_t bl[];  // [NFRAG][64] B fragments of this workgroup's slice

    const int P = a.P;
    const int numTeams = a.numTeams;
    const int g = blockIdx.x;
    if (g >= P * numTeams) {
        return;  // spare workgroup: the whole workgroup leaves together
    }
    const int team = g % numTeams;
    const int p = g / numTeams;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int grp = lane >> 4;
    const int rl = lane & 15;
    const int64_t d0 = (int64_t)p * DW;
    const int64_t stride = (int64_t)numTeams * W;
    int64_t rt = (int64_t)team * W + wave;

    u32x4_t xr[N][KS];
    auto load_x = [&](int64_t rtile) {
        const int64_t row = rtile * 16 + rl;
        const bool ok = row < a.T;
        const uint16_t *base = a.x + (ok ? row : 0) * a.K + d0 + 8 * grp;
#pragma unroll
        for (int s = 0; s < N; ++s) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                xr[s][ks] = ok ? *reinterpret_cast<const u32x4_t *>(base + s * a.D + 32 * ks)
                               : u32x4_t{0u, 0u, 0u, 0u};
            }
        }
    };
    if ((int64_t)team * W >= a.RT) {
        return;  // no row tile for any wave of this workgroup
    }
    if (rt < a.RT) {
        load_x(rt);  // in flight while the B slice is built
    }

    // B slice: fragment f = ((s*KS + ks)*NT + ct)*64 + l holds, for lane l,
    // B[k = s*D + d0 + 32ks + 8(l/16) + e][slot 16ct + l%16], e = 0..7.  A
    // thread builds all NT column tiles of one (s, ks, lane) item, so it reads
    // the item's gamma once; two items' loads are in flight together.
    constexpr int ITEMS = N * KS * 64;
    for (int it0 = tid; it0 < ITEMS; it0 += 2 * W * 64) {
        f32x4_t ph[2][NT][2];
        f32x4_t gm[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int it = it0 + h * W * 64;
            if (it < ITEMS) {
                const int fl = it & 63;
                const int sk = it >> 6;
                const int64_t k0 =
                    (sk / KS) * a.D + d0 + 32 * (sk % KS) + 8 * (fl >> 4);
#pragma unroll
                for (int ct = 0; ct < NT; ++ct) {
                    bool lo;
                    int j;
                    CL::slot(16 * ct + (fl & 15), lo, j);
                    const f32x4_t *src =
                        reinterpret_cast<const f32x4_t *>(a.phi + (int64_t)j * a.K + k0);
                    ph[h][ct][0] = src[0];
                    ph[h][ct][1] = src[1];
                }
                if (a.gamma != nullptr) {
                    const f32x4_t *gs = reinterpret_cast<const f32x4_t *>(a.gamma + k0);
                    gm[h][0] = gs[0];
                    gm[h][1] = gs[1];
                } else {
                    gm[h][0] = f32x4_t{1.f, 1.f, 1.f, 1.f};
                    gm[h][1] = f32x4_t{1.f, 1.f, 1.f, 1.f};
                }
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int it = it0 + h * W * 64;
            if (it < ITEMS) {
                const int fl = it & 63;
                const int sk = it >> 6;
#pragma unroll
                for (int ct = 0; ct < NT; ++ct) {
                    bool lo;
                    int j;
                    CL::slot(16 * ct + (fl & 15), lo, j);
                    float out[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        float b = ph[h][ct][e >> 2][e & 3];
                        if (a.gamma != nullptr) {
                            b = b * gm[h][e >> 2][e & 3];
                        }
                        const float hi = bf16_bits_to_f32(f32_to_bf16_bits(b));
                        out[e] = lo ? (b - hi) : hi;
                    }
                    bl[(sk * NT + ct) * 64 + fl] = pack8_bf16(out);
                }
            }
        }
    }
    __syncthreads();

    const float alphaPre = a.alpha[0];
    const float alphaPost = a.alpha[1];
    const float alphaRes = a.alpha[2];

    for (; rt < a.RT; rt += stride) {
        // 1. GEMM slice + sum of squares.
        f32x4_t acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        float ss = 0.f;
        // B fragments are read one k-step ahead of the MFMAs that use them;
        // the compiler barriers stop the scheduler from hoisting more reads
        // (the x block already holds most of the VGPRs).
        constexpr int STEPS = N * KS;
        u32x4_t bcur[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            bcur[t] = bl[t * 64 + lane];
        }
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            u32x4_t bnext[NT];
            if (st + 1 < STEPS) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    bnext[t] = bl[((st + 1) * NT + t) * 64 + lane];
                }
            }
            asm volatile("" ::: "memory");
            const u32x4_t av = xr[st / KS][st % KS];
            ss = sumsq8<kBf16>(av, ss);
            if constexpr (kBf16) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t] = mfma16(av, bcur[t], acc[t]);
                }
            } else {
                float f[8];
                unpack8<kBf16>(av, f);
                u32x4_t ahi, alo;
                split_f16_to_bf16(f, ahi, alo);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t] = mfma16(ahi, bcur[t], acc[t]);
                    if (CL::has_hi(t)) {
                        acc[t] = mfma16(alo, bcur[t], acc[t]);
                    }
                }
            }
            if (st + 1 < STEPS) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    bcur[t] = bnext[t];
                }
            }
        }
        ss = ss + __shfl_xor(ss, 16);
        ss = ss + __shfl_xor(ss, 32);

        // 2. Publish this slice's partials (C fragment: lane holds rows
        //    4*grp + i of column slot 16t + rl).
        float *rec = a.partial + (rt * P + p) * RC::FLOATS;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * grp + i;
#pragma unroll
            for (int t = 0; t < Q; ++t) {
                st_dev(rec + RC::col(16 * t + rl) * 16 + r, acc[t][i] + acc[Q + t][i]);
            }
            if constexpr (CL::kHalfTile) {
                const float other = __shfl_xor(acc[2 * Q][i], 8);
                if (rl < 8) {
                    st_dev(rec + RC::col(16 * Q + rl) * 16 + r, acc[2 * Q][i] + other);
                }
            }
        }
        if (grp == 0) {
            st_dev(rec + N * 16 + rl, ss);
        }
        wait_all_memory();  // the partials are visible device-wide before we count in
        uint32_t old = 0;
        if (lane == 0) {
            old = __hip_atomic_fetch_add(a.arrive + rt * kCounterStride, 1u, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        }
        old = __shfl(old, 0);
        const int64_t row = rt * 16 + rl;
        const bool rowOk = row < a.T;

        // 3. hPre and invRms of the tile's 16 rows.  Lane (rl, grp) owns hPre
        //    column grp of row rl.
        static_assert(N == 4, "the fused path maps the n = 4 hPre columns to the 4 lane groups");
        const float *tileRec = a.partial + rt * P * RC::FLOATS;
        float *fin = a.finalPre + rt * RC::FIN;
        uint32_t *finBits = reinterpret_cast<uint32_t *>(fin);
        float preC, invRms;
        if (old == (uint32_t)(P - 1)) {
            // Last slice in: sum over the slices (fixed order), evaluate, publish.
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            const float mixC = sum_over_slices(tileRec + grp * 16 + rl, P, RC::FLOATS, true);
            const float ssum = sum_over_slices(tileRec + N * 16 + rl, P, RC::FLOATS, grp == 0);
            invRms = ref_inv_rms(__shfl(ssum, rl), a.invFlatDim, a.normEps);
            preC = ref_sigmoid(mixC * (invRms * alphaPre), a.bias[grp], a.hcEps);
            __hip_atomic_store(finBits + grp * 16 + rl, __float_as_uint(preC), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            if (grp == 0) {
                __hip_atomic_store(finBits + N * 16 + rl, __float_as_uint(invRms),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (a.hPre != nullptr && rowOk) {
                a.hPre[row * N + grp] = preC;
            }
        } else {
            // Poll the published values (the reset kernel filled the block
            // with a signalling-NaN sentinel that no arithmetic produces).
            uint32_t spins = 0;
            uint32_t pb, ib;
            for (;;) {
                pb = __hip_atomic_load(finBits + grp * 16 + rl, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                ib = grp == 0 ? __hip_atomic_load(finBits + N * 16 + rl, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                              : 0u;
                if (__all(pb != kPreSentinel && ib != kPreSentinel)) {
                    break;
                }
                if (++spins > a.spinLimit) {
                    if (lane == 0) {
                        __hip_atomic_store(a.status, kDeviceTimeout, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    }
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            preC = __uint_as_float(pb);
            invRms = __shfl(__uint_as_float(ib), rl);
        }
        float pre[N];
#pragma unroll
        for (int s = 0; s < N; ++s) {
            pre[s] = __shfl(preC, 16 * s + rl);
        }

        // 3b. hPost / hRes: the M - N other columns in groups of four, group m
        //     done by slice m mod P (every partial is in: hPre exists).
        {
            constexpr int NG = (M - N + 3) / 4;
            const float sQ = invRms * alphaPost;
            const float sR = invRms * alphaRes;
            for (int m = p; m < NG; m += P) {
                const int jj = N + 4 * m + grp;
                const bool colOk = jj < M;
                const float v = sum_over_slices(tileRec + RC::col(colOk ? jj : 0) * 16 + rl, P,
                                                RC::FLOATS, colOk);
                if (colOk && rowOk) {
                    if (jj < 2 * N) {
                        const float sg = ref_sigmoid(v * sQ, a.bias[jj], 0.0f);
                        a.hPost[row * N + (jj - N)] = sg * 2.0f;
                    } else {
                        const float r = v * sR;
                        a.hRes[row * (N * N) + (jj - 2 * N)] = r + a.bias[jj];
                    }
                }
            }
        }

        // 4. hIn for this slice's columns from the registers.
        if (rowOk) {
            uint16_t *out = a.hIn + row * a.D + d0 + 8 * grp;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                // Unpack one k-step at a time (an empty asm that "rewrites"
                // the registers keeps the unpacking from being hoisted).
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    asm volatile("" : "+v"(xr[s][ks]));
                }
                float h[8];
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    float f[8];
                    unpack8<kBf16>(xr[s][ks], f);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float prod = pre[s] * f[e];
                        h[e] = (s == 0) ? prod : h[e] + prod;
                    }
                }
                u32x4_t o;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    o[w] = f32_to_x<kBf16>(h[2 * w]) | (f32_to_x<kBf16>(h[2 * w + 1]) << 16);
                }
                *reinterpret_cast<u32x4_t *>(out + 32 * ks) = o;
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (rt + stride < a.RT) {
            load_x(rt + stride);
        }
    }
}

template <int N, int KS, bool kBf16>
size_t fused_lds_bytes()
{
    return (size_t)N * KS * Shape<N>::NT * 64 * sizeof(u32x4_t);
}

template <int N, int KS, bool kBf16>
hipError_t fused_prepare_attr()
{
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        err = hipFuncSetAttribute(reinterpret_cast<const void *>(&fused_kernel<N, KS, kBf16>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)fused_lds_bytes<N, KS, kBf16>());
    });
    return err;
}

template <int N, int KS, bool kBf16>
int fused_coresident_t(int numCUs)
{
    if (fused_prepare_attr<N, KS, kBf16>() != hipSuccess) {
        return -1;
    }
    int perCU = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &perCU, reinterpret_cast<const void *>(&fused_kernel<N, KS, kBf16>),
            kFusedWaves * 64, fused_lds_bytes<N, KS, kBf16>()) != hipSuccess) {
        return -1;
    }
    return perCU * numCUs;
}

template <int N, int KS, bool kBf16>
hipError_t launch_fused_t(const Plan &p, void *workspace, hipStream_t stream)
{
    hipError_t err = fused_prepare_attr<N, KS, kBf16>();
    if (err != hipSuccess) {
        return err;
    }
    char *ws = static_cast<char *>(workspace);
    FusedArgs a;
    a.x = static_cast<const uint16_t *>(p.x);
    a.phi = p.phi;
    a.gamma = p.hasGamma ? p.gamma : nullptr;
    a.alpha = p.alpha;
    a.bias = p.bias;
    a.hIn = static_cast<uint16_t *>(p.hIn);
    a.hPost = p.hPost;
    a.hRes = p.hRes;
    a.hPre = p.hasHPre ? p.hPre : nullptr;
    a.status = reinterpret_cast<uint32_t *>(ws);
    a.arrive = reinterpret_cast<uint32_t *>(ws + p.wsCounters);
    a.finalPre = reinterpret_cast<float *>(ws + p.wsFinal);
    a.partial = reinterpret_cast<float *>(ws + p.wsFusedPartial);
    a.T = p.T;
    a.D = p.D;
    a.K = p.K;
    a.RT = p.fusedTiles;
    a.P = p.fusedP;
    a.numTeams = p.fusedTeams;
    a.normEps = p.normEps;
    a.hcEps = p.hcEps;
    a.invFlatDim = p.invFlatDim;
    a.spinLimit = 1u << 20;  // about a second of polling per wait

    const int64_t finalWords = p.fusedTiles * Rec<N>::FIN;
    hipLaunchKernelGGL(fused_reset_kernel, dim3((unsigned)((finalWords + 255) / 256)), dim3(256), 0,
                       stream, a.arrive, reinterpret_cast<uint32_t *>(a.finalPre),
                       (int64_t)p.fusedTiles, finalWords, a.status);
    err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    void *args[] = {&a};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&fused_kernel<N, KS, kBf16>),
                                      dim3((unsigned)p.fusedGrid), dim3(kFusedWaves * 64), args,
                                      (unsigned)fused_lds_bytes<N, KS, kBf16>(), stream);
}

}  // namespace

// Fused-path instantiations: n = 4 with KS in {8, 7, 4, 2, 1}.
#define MHC_FUSED_DISPATCH(FN, ...)                                            \
    switch (p.fusedDw / 32) {                                                  \
    case 8:                                                                    \
        return p.isBf16 ? FN<4, 8, true>(__VA_ARGS__) : FN<4, 8, false>(__VA_ARGS__); \
    case 7:                                                                    \
        return p.isBf16 ? FN<4, 7, true>(__VA_ARGS__) : FN<4, 7, false>(__VA_ARGS__); \
    case 4:                                                                    \
        return p.isBf16 ? FN<4, 4, true>(__VA_ARGS__) : FN<4, 4, false>(__VA_ARGS__); \
    case 2:                                                                    \
        return p.isBf16 ? FN<4, 2, true>(__VA_ARGS__) : FN<4, 2, false>(__VA_ARGS__); \
    case 1:                                                                    \
        return p.isBf16 ? FN<4, 1, true>(__VA_ARGS__) : FN<4, 1, false>(__VA_ARGS__); \
    default:                                                                   \
        break;                                                                 \
    }

hipError_t launch_fused(const Plan &p, void *workspace, hipStream_t stream)
{
    if (p.n != 4) {
        return hipErrorNotSupported;
    }
    MHC_FUSED_DISPATCH(launch_fused_t, p, workspace, stream)
    return hipErrorNotSupported;
}

int fused_max_coresident(const Plan &p, int numCUs)
{
    if (p.n != 4) {
        return -1;
    }
    MHC_FUSED_DISPATCH(fused_coresident_t, numCUs)
    return -1;
}

}  // namespace mhc
