// Fused MhcPre kernel for gfx950: x is read from HBM once and stays in VGPRs.
//
// Work decomposition.  D is cut into P slices of DW = 64*KP columns.  A unit
// is (16-row tile, slice p): the 16 rows x n streams x DW columns of x, held
// by one wave in VGPRs.  A workgroup of W = 8 waves (two per SIMD) owns one
// slice for the whole launch and keeps that slice of the B operand
// (gamma*phi split into bf16 hi + lo) in LDS.  The P workgroups that own the
// slices of the same row tiles form a team (team = workgroup % numTeams).
//
// Register layout of x.  A unit is loaded as whole 128-byte lines: register
// (s, kp, h) holds, in lane l, row 8h + (l & 7) and the 8 columns starting at
// 64kp + 8(l >> 4) + 32((l >> 3) & 1) of stream s, so the 8 lanes of a row
// read (and later write, for hIn) one full line.  The MFMA A operand wants
// lane l to hold row l & 15; one DPP row_ror:8 move with a bank mask per
// dword turns registers (kp, h = 0, 1) into the A fragments of k-steps 2kp
// and 2kp + 1.  x is read and hIn written with nontemporal buffer accesses.
//
// Per unit a wave:
//   1. multiplies its x block by the LDS B slice (MFMA, fp32 accumulate) and
//      forms the Gram matrix of its rows with the same fragments, whose
//      diagonal is the slice's sum of squares per row;
//   2. publishes the slice's partial sums (M mix columns + sumsq per row) as
//      tagged words (below) and, without waiting, finishes the hPost / hRes
//      columns it owns for its previous tile;
//   3. obtains hPre and invRms of its 16 rows: the tile's reducer (slice
//      tile mod P) polls the P records until every word carries this launch's
//      tag, sums the hPre columns and sumsq over the slices in a fixed order,
//      evaluates invRms and hPre and publishes them as tagged words; every
//      other slice polls that block;
//   4. computes hIn for its DW columns from the x still in its registers and,
//      as each register group is consumed, issues the loads of its next unit
//      into it.
//
// Exchange words.  Every exchanged value is one 8-byte word: the fp32 bits in
// the low half and a tag in the high half, written and read as single-copy
// atomic 64-bit accesses at device scope (sc1).  The tag is a hash of the
// word's position mixed with a per-launch epoch, so a word holds the current
// value exactly when its tag matches: no arrival counter, no release wait and
// no reset of the workspace between launches.  A reader accepts a block only
// when every word it read carries the expected tag; a block left over from an
// earlier launch (another epoch) or filled with any constant never does.  The
// epoch is kept in the workspace header (epoch_load / mark / publish), so the
// replays of a captured HIP graph get fresh epochs too.  Every wait is bounded
// by a spin limit; running out records kDeviceTimeout with the host launch id
// in the status word instead of hanging, and the values that wait was for are
// taken as NaN, so the affected outputs are NaN.  The grid is
// sized to the device's co-residency limit, so every workgroup is resident
// when nothing else runs on the device (a cooperative launch, on request,
// guarantees it even then); a reducer is then never waiting on a workgroup
// that has not started.

#include "mhc_pre_device.h"
#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace mhc {
namespace {

using namespace dev;

constexpr int kFusedWaves = 8;  // waves per workgroup (two per SIMD)

struct FusedArgs {
    const uint16_t *x;
    const float *phi;
    const float *gamma;
    const u32x4_t *bprep;  // prepared B fragments [K/32][NT][64] (kPrep only)
    const float *alpha;
    const float *bias;
    uint16_t *hIn;
    float *hPost;
    float *hRes;
    float *hPre;
    uint64_t *recs;      // [RT][P] records of Rec<N>::WORDS tagged words
    uint64_t *bcast;     // [RT] blocks of Rec<N>::BWORDS tagged words
    uint64_t *status;    // (launchId << 32) | kDeviceTimeout after a timeout
    char *hdr;           // workspace header (status word, exchange epoch)
    uint32_t *statusWord;  // the caller's sticky status word, or null
    int64_t T;
    int64_t D;
    int64_t K;
    int64_t RT;
    int P;
    int numTeams;
    float normEps;
    float hcEps;
    float invFlatDim;
    uint32_t launchId;
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
    __device__ __forceinline__ static void slot(int c, bool &lo, int &j)
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
// 16 rows as 16 consecutive tagged words (128 bytes).  Column N is the sum of
// squares; mix column j sits at column j (j < N, the hPre columns) or j + 1.
// The per-tile broadcast block holds hPre columns 0..N-1 and invRms at
// column N, 16 rows each.
template <int N>
struct Rec {
    static constexpr int M = N * N + 2 * N;
    static constexpr int COLS = M + 1;
    static constexpr int WORDS = COLS * 16;
    static constexpr int BWORDS = (N + 1) * 16;
    __device__ static int col(int j) { return j < N ? j : j + 1; }
};

// Tags: a multiplicative hash of the word's position (distinct for the
// records and the broadcast blocks) mixed with the launch epoch.
__device__ __forceinline__ uint32_t rec_tag(uint32_t pos, uint32_t epoch)
{
    return (pos * 0x9E3779B1u) ^ epoch;
}
__device__ __forceinline__ uint32_t bcast_tag(uint32_t pos, uint32_t epoch)
{
    return (pos * 0x85EBCA77u) ^ epoch ^ 0xC2B2AE3Du;
}

__device__ __forceinline__ uint64_t ld_word(const uint64_t *p)
{
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cache-policy operands of the buffer builtins.
constexpr int kCpolNt = 2;    // nontemporal: x and hIn are streamed once
constexpr int kCpolDev = 16;  // sc1: device-scope coherent

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, 0x00020000);
}

// Sums over the P slice records of a tile, for record columns c0 .. c0+NC-1
// and all 16 rows, checking every word's tag.  Lane l takes item
// it = l % (8 NC) (column c0 + it/8, rows 2(it%8) and 2(it%8) + 1, one 16-byte
// load per slice) and slice group sg = l / (8 NC), and adds slices sg,
// sg + NSG, ... in increasing order; the groups are then added in order
// 0, 1, ..., NSG-1, so the result is a fixed-order sum.  Loads are issued U
// slices per lane at a time.  Lanes it < 8 NC return the two row totals of
// their item; valid is true when every word read carried the expected tag.
template <int NC, int COLS, int U>
__device__ __forceinline__ float2 sum_records(__amdgpu_buffer_rsrc_t r, int c0, int P, int lane,
                                              uint32_t tileBase, uint32_t epoch, bool &valid)
{
    constexpr int NIT = 8 * NC;
    constexpr int NSG = 64 / NIT;
    static_assert(NSG >= 1, "at most 8 columns per call");
    const int it = lane % NIT;
    const int sg = lane / NIT;
    const bool act = sg < NSG;
    const int c = c0 + it / 8;
    const int row0 = 2 * (it % 8);
    float2 acc = make_float2(0.f, 0.f);
    bool ok = true;
    for (int q0 = 0; q0 < P; q0 += NSG * U) {
        u32x4_t t[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + sg + NSG * u;
            t[u] = (act && q < P)
                       ? __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                         r, ((q * COLS + c) * 16 + row0) * 8, 0,
                                                         kCpolDev))
                       : u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + sg + NSG * u;
            if (act && q < P) {
                const uint32_t pos = tileBase + (uint32_t)((q * COLS + c) * 16 + row0);
                ok = ok && t[u][1] == rec_tag(pos, epoch) && t[u][3] == rec_tag(pos + 1u, epoch);
                acc.x = acc.x + __uint_as_float(t[u][0]);
                acc.y = acc.y + __uint_as_float(t[u][2]);
            }
        }
    }
    float2 tot = acc;
#pragma unroll
    for (int k = 1; k < NSG; ++k) {
        tot.x = tot.x + __shfl(acc.x, it + k * NIT);
        tot.y = tot.y + __shfl(acc.y, it + k * NIT);
    }
    valid = __all(ok);
    return tot;
}

// A fragments of k-steps 2kp and 2kp + 1 from the line-layout registers r0
// (rows 0-7) and r1 (rows 8-15): lanes with bit 3 set take the other
// register's lane l ^ 8 (DPP row_ror:8 with banks 2-3 or 0-1 enabled).
__device__ __forceinline__ void lines_to_frags(const u32x4_t &r0, const u32x4_t &r1, u32x4_t &k0,
                                               u32x4_t &k1)
{
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        k0[w] = (uint32_t)__builtin_amdgcn_update_dpp((int)r0[w], (int)r1[w], 0x128, 0xF, 0xC, false);
        k1[w] = (uint32_t)__builtin_amdgcn_update_dpp((int)r1[w], (int)r0[w], 0x128, 0xF, 0x3, false);
    }
}

__device__ __forceinline__ f32x4_t mfma16_f16(const u32x4_t &a, const u32x4_t &b, const f32x4_t &c)
{
    typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ void record_timeout(const FusedArgs &a, int lane)
{
    if (lane == 0) {
        __hip_atomic_store(a.status, ((uint64_t)a.launchId << 32) | kDeviceTimeout, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        st_status_word(a.statusWord);
    }
}

template <int N, int KP, bool kBf16, bool kPrep>
__global__ __launch_bounds__(kFusedWaves * 64) void fused_kernel(FusedArgs a)
{
    using S = Shape<N>;
    constexpr int M = S::M;
    constexpr int NT = S::NT;
    using CL = ColLayout<M>;
    using RC = Rec<N>;
    constexpr int W = kFusedWaves;
    constexpr int KS = 2 * KP;  // 32-column MFMA k-steps per stream
    constexpr int DW = 64 * KP;
    constexpr int Q = CL::Q;
    extern __shared__ u32x4_t bl[];  // [N*KS][NT][64] B fragments, per-wave scratch, staging
    __shared__ uint32_t epochSh;     // the launch's exchange epoch, from thread 0 to every wave
    static_assert(N == 4, "the fused path maps the n = 4 hPre columns to the 4 lane groups");

    const int tid = threadIdx.x;
    // Thread 0 reads the epoch the previous launch on this workspace left.
    const uint32_t prevEpoch = tid == 0 ? epoch_load(a.hdr, kWsEpochOff) : 0u;
    const int P = a.P;
    const int numTeams = a.numTeams;
    const int g = blockIdx.x;
    if (g >= P * numTeams) {
        if (tid == 0) {
            epoch_mark(a.hdr, kWsSeenOff, epoch_next(prevEpoch), g);
        }
        return;  // spare workgroup: the whole workgroup leaves together
    }
    const int team = g % numTeams;
    const int p = g / numTeams;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t d0 = (int64_t)p * DW;
    const int64_t stride = (int64_t)numTeams * W;
    float *scratch = reinterpret_cast<float *>(bl + N * KS * NT * 64) + wave * RC::BWORDS;
    uint64_t *stage = reinterpret_cast<uint64_t *>(reinterpret_cast<float *>(bl + N * KS * NT * 64) +
                                                   W * RC::BWORDS) +
                      wave * RC::WORDS;
    int64_t rt = (int64_t)team * W + wave;

    u32x4_t xr[N][KP][2];
    // x and hIn of a tile go through buffer resources based at the tile's
    // first row and sized to its valid rows: loads past T read zero and
    // stores past T are dropped.
    auto tile_rows = [&](int64_t rtile) { return (int)min((int64_t)16, a.T - rtile * 16); };
    auto load_line = [&](__amdgpu_buffer_rsrc_t xrs, int xLane, int Ki, int Di, int d0i, int s,
                         int kp, int h) {
        const int so = (8 * h * Ki + s * Di + d0i) * 2;
        xr[s][kp][h] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xrs, xLane + 128 * kp, so, kCpolNt));
    };
    if ((int64_t)team * W >= a.RT) {
        if (tid == 0) {
            epoch_mark(a.hdr, kWsSeenOff, epoch_next(prevEpoch), g);
        }
        return;  // no row tile for any wave of this workgroup
    }
    // B slice: fragment f = ((s*KS + ks)*NT + ct)*64 + l holds, for lane l,
    // B[k = s*D + d0 + 32ks + 8(l/16) + e][slot 16ct + l%16], e = 0..7.  A
    // thread builds all NT column tiles of one (s, ks, lane) item, so it reads
    // the item's gamma once; two items' loads are in flight together.
    if constexpr (kPrep) {
        // Prepared weights: the fragments already have this layout; k-step ks
        // of stream s is the prepared k-step (s D + d0 + 32 ks) / 32.
        constexpr int FR = N * KS * NT * 64;
        for (int f = tid; f < FR; f += W * 64) {
            const int sk = f / (NT * 64);
            const int ct = (f / 64) % NT;
            const int64_t gks = ((sk / KS) * a.D + d0 + 32 * (sk % KS)) / 32;
            bl[f] = a.bprep[(gks * NT + ct) * 64 + (f & 63)];
        }
    } else {
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
    }
    if (rt < a.RT) {
        // The first unit's x, issued once the B slice is built: a wave stalls
        // at a load while the CU's memory queue is full, and these loads
        // issued first held the weights' loads (and the build) behind them
        // (n = 4, D = 8192, T = 8192: 186.0 -> 184.0 us).
        const int lrow = lane & 7;
        const int lineOff = 8 * (lane >> 4) + 32 * ((lane >> 3) & 1);
        const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x + rt * 16 * a.K, tile_rows(rt) * (int)a.K * 2);
#pragma unroll
        for (int s = 0; s < N; ++s) {
#pragma unroll
            for (int kp = 0; kp < KP; ++kp) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    load_line(xrs, (lrow * (int)a.K + lineOff) * 2, (int)a.K, (int)a.D, (int)d0, s,
                              kp, h);
                }
            }
        }
    }

    if (tid == 0) {
        epochSh = epoch_next(prevEpoch);
        epoch_mark(a.hdr, kWsSeenOff, epochSh, g);
    }
    __syncthreads();

    const float alphaPre = a.alpha[0];
    const float alphaPost = a.alpha[1];
    const float alphaRes = a.alpha[2];
    const uint32_t epoch = __builtin_amdgcn_readfirstlane(epochSh);

    // hPost / hRes columns (mix columns N .. M-1) of a finished tile: column
    // N + m is done by slice m mod P, from the records (every one of them is
    // complete once the tile's hPre exists, but the tags are checked anyway).
    auto post_res = [&](int64_t rtile, float invRmsLane, int Pi, int laneO) {
        const __amdgpu_buffer_rsrc_t tr =
            make_rsrc(a.recs + rtile * Pi * RC::WORDS, Pi * RC::WORDS * 8);
        const uint32_t tileBase = (uint32_t)(rtile * Pi * RC::WORDS);
        for (int m = p; m < M - N; m += Pi) {
            const int jj = N + m;
            float2 tot;
            bool valid = false;
            for (uint32_t spins = 0;; ++spins) {
                tot = sum_records<1, RC::COLS, 4>(tr, RC::col(jj), Pi, laneO, tileBase, epoch, valid);
                if (valid) {
                    break;
                }
                if (spins >= a.spinLimit) {
                    record_timeout(a, laneO);
                    tot = make_float2(poison(), poison());  // an expired wait: NaN outputs
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            const int r0 = 2 * (laneO % 8);
            const float ir0 = __shfl(invRmsLane, r0);
            const float ir1 = __shfl(invRmsLane, r0 + 1);
            if (laneO < 8) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int64_t row = rtile * 16 + r0 + e;
                    const float v = e == 0 ? tot.x : tot.y;
                    const float ir = e == 0 ? ir0 : ir1;
                    if (row < a.T) {
                        if (jj < 2 * N) {
                            const float sg = ref_sigmoid(v * (ir * alphaPost), a.bias[jj], 0.0f);
                            a.hPost[row * N + (jj - N)] = sg * 2.0f;
                        } else {
                            const float r = v * (ir * alphaRes);
                            a.hRes[row * (N * N) + (jj - 2 * N)] = r + a.bias[jj];
                        }
                    }
                }
            }
        }
    };

    int64_t prevTile = -1;
    float prevInvRms = 0.f;
    for (; rt < a.RT; rt += stride) {
        // Per-unit copies the compiler cannot see through: the offsets
        // derived from them are recomputed each unit (a few instructions)
        // instead of being hoisted out of the loop and held in registers.
        int laneO = lane;
        int Ki = (int)a.K;
        int Di = (int)a.D;
        int d0i = (int)d0;
        int Pi = P;
        asm volatile("" : "+v"(laneO), "+s"(Ki), "+s"(Di), "+s"(d0i), "+s"(Pi));
        const int grp = laneO >> 4;
        const int rl = laneO & 15;
        const int lrow = laneO & 7;
        const int lineOff = 8 * (laneO >> 4) + 32 * ((laneO >> 3) & 1);

        // 1. GEMM slice + Gram matrix (sum of squares on its diagonal).  The
        //    B fragments of the next k-step are read while this step's MFMAs
        //    run; the compiler barriers keep the scheduler from hoisting more.
        f32x4_t acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        f32x4_t gram = f32x4_t{0.f, 0.f, 0.f, 0.f};
        constexpr int STEPS = N * KS;
        u32x4_t bcur[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            bcur[t] = bl[t * 64 + laneO];
        }
        u32x4_t kf[2];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int s = st / KS;
            const int kp = (st % KS) >> 1;
            const int q = st & 1;
            u32x4_t bnext[NT];
            if (st + 1 < STEPS) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    bnext[t] = bl[((st + 1) * NT + t) * 64 + laneO];
                }
            }
            asm volatile("" ::: "memory");
            if (q == 0) {
                lines_to_frags(xr[s][kp][0], xr[s][kp][1], kf[0], kf[1]);
            }
            if constexpr (kBf16) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t] = mfma16(kf[q], bcur[t], acc[t]);
                }
                gram = mfma16(kf[q], kf[q], gram);
            } else {
                gram = mfma16_f16(kf[q], kf[q], gram);
                float f[8];
                unpack8<kBf16>(kf[q], f);
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
            __builtin_amdgcn_sched_barrier(0);
        }
        // Gram diagonal: row r sits in lane 16(r/4) + r, register r % 4.
        const bool diagLane = (rl >> 2) == grp;
        const int di = rl & 3;
        const float ss = di == 0 ? gram[0] : di == 1 ? gram[1] : di == 2 ? gram[2] : gram[3];

        // 2. Publish this slice's partials as tagged words.  The C fragment
        //    (lane holds rows 4*grp + i of column slot 16t + rl) is written to
        //    this wave's LDS staging record first, so that the device-scope
        //    stores go out as whole 128-byte lines (8 lanes x 16 bytes per
        //    column) instead of scattered 8-byte writes.
        {
            const uint32_t recBase = (uint32_t)((rt * Pi + p) * RC::WORDS);
            auto put = [&](int w, float v) {
                stage[w] = (uint64_t)__float_as_uint(v) | ((uint64_t)rec_tag(recBase + w, epoch) << 32);
            };
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * grp + i;
#pragma unroll
                for (int t = 0; t < Q; ++t) {
                    put(RC::col(16 * t + rl) * 16 + r, acc[t][i] + acc[Q + t][i]);
                }
                if constexpr (CL::kHalfTile) {
                    const float other = __shfl_xor(acc[2 * Q][i], 8);
                    if (rl < 8) {
                        put(RC::col(16 * Q + rl) * 16 + r, acc[2 * Q][i] + other);
                    }
                }
            }
            if (diagLane) {
                put(N * 16 + rl, ss);
            }
            // A wave's LDS accesses complete in order; the barrier keeps the
            // compiler from moving the reads below above the writes.
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            const __amdgpu_buffer_rsrc_t rr =
                make_rsrc(a.recs + (rt * Pi + p) * RC::WORDS, RC::WORDS * 8);
            constexpr int CHUNKS = RC::WORDS / 2;  // 16-byte chunks of the record
#pragma unroll
            for (int k = 0; k < (CHUNKS + 63) / 64; ++k) {
                const int j = laneO + 64 * k;
                if (j < CHUNKS) {
                    const u32x4_t v = *reinterpret_cast<const u32x4_t *>(stage + 2 * j);
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v), rr,
                        16 * j, 0, kCpolDev);
                }
            }
        }
        // The previous tile's hPost / hRes fill the time the other slices
        // need to publish.
        if (prevTile >= 0) {
            post_res(prevTile, prevInvRms, Pi, laneO);
        }

        // 3. hPre and invRms of the tile's 16 rows: lane (rl, grp) ends with
        //    hPre column grp and invRms of row rl.
        uint64_t *blk = a.bcast + rt * RC::BWORDS;
        const uint32_t blkBase = (uint32_t)(rt * RC::BWORDS);
        float preC, invRms;
        if (rt % Pi == p) {
            // Reducer: sum columns 0..N (hPre mix columns, sum of squares)
            // over the slices in a fixed order once every record is in.
            const __amdgpu_buffer_rsrc_t tr = make_rsrc(a.recs + rt * Pi * RC::WORDS, Pi * RC::WORDS * 8);
            const uint32_t tileBase = (uint32_t)(rt * Pi * RC::WORDS);
            float2 tot;
            bool valid = false;
            for (uint32_t spins = 0;; ++spins) {
                tot = sum_records<N + 1, RC::COLS, 14>(tr, 0, Pi, laneO, tileBase, epoch, valid);
                if (valid) {
                    break;
                }
                if (spins >= a.spinLimit) {
                    record_timeout(a, laneO);
                    tot = make_float2(poison(), poison());  // NaN hPre, invRms and outputs
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            constexpr int NIT = 8 * (N + 1);
            const int it = laneO % NIT;
            const int c = it / 8;
            const int r0 = 2 * (it % 8);
            // invRms of rows r0, r0 + 1 from the sum-of-squares lanes (c == N).
            float ir0 = ref_inv_rms(tot.x, a.invFlatDim, a.normEps);
            float ir1 = ref_inv_rms(tot.y, a.invFlatDim, a.normEps);
            ir0 = __shfl(ir0, 8 * N + it % 8);
            ir1 = __shfl(ir1, 8 * N + it % 8);
            if (laneO < NIT) {
                const float bc = c < N ? a.bias[c] : 0.f;
                u32x4_t wv;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float ir = e == 0 ? ir0 : ir1;
                    const float mix = e == 0 ? tot.x : tot.y;
                    const float v = c < N ? ref_sigmoid(mix * (ir * alphaPre), bc, a.hcEps) : ir;
                    const int idx = c * 16 + r0 + e;
                    scratch[idx] = v;
                    wv[2 * e] = __float_as_uint(v);
                    wv[2 * e + 1] = bcast_tag(blkBase + idx, epoch);
                    const int64_t row = rt * 16 + r0 + e;
                    if (c < N && a.hPre != nullptr && row < a.T) {
                        a.hPre[row * N + c] = v;
                    }
                }
                // Two tagged words (rows r0, r0 + 1) per lane: 8 lanes fill
                // a column's 128-byte line.
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, wv),
                    make_rsrc(blk, RC::BWORDS * 8), (c * 16 + r0) * 8, 0, kCpolDev);
            }
            preC = scratch[grp * 16 + rl];
            invRms = scratch[N * 16 + rl];
        } else {
            uint64_t pw = 0, iw = 0;
            for (uint32_t spins = 0;; ++spins) {
                pw = ld_word(blk + grp * 16 + rl);
                iw = ld_word(blk + N * 16 + rl);
                const bool ok = (uint32_t)(pw >> 32) == bcast_tag(blkBase + grp * 16 + rl, epoch) &&
                                (uint32_t)(iw >> 32) == bcast_tag(blkBase + N * 16 + rl, epoch);
                if (__all(ok)) {
                    break;
                }
                if (spins >= a.spinLimit) {
                    record_timeout(a, laneO);
                    pw = iw = (uint64_t)__float_as_uint(poison());  // NaN hIn, hPost, hRes
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            preC = __uint_as_float((uint32_t)pw);
            invRms = __uint_as_float((uint32_t)iw);
        }
        prevTile = rt;
        prevInvRms = invRms;

        // hPre of the two line-layout rows of this lane: 8h + (lane & 7).
        float pre[2][N];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int s = 0; s < N; ++s) {
                pre[h][s] = __shfl(preC, 16 * s + 8 * h + lrow);
            }
        }

        // 4. hIn for this slice's columns from the registers; each consumed
        //    register group is refilled with the next unit's x at once.
        const int64_t rtNext = rt + stride;
        const bool more = rtNext < a.RT;
        const __amdgpu_buffer_rsrc_t hrs = make_rsrc(a.hIn + rt * 16 * a.D, tile_rows(rt) * Di * 2);
        const __amdgpu_buffer_rsrc_t xrs =
            make_rsrc(a.x + (more ? rtNext : rt) * 16 * a.K, tile_rows(more ? rtNext : rt) * Ki * 2);
        const int hLane = (lrow * Di + lineOff) * 2;
        const int xLane = (lrow * Ki + lineOff) * 2;
#pragma unroll
        for (int kp = 0; kp < KP; ++kp) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // An empty asm that "rewrites" the registers keeps the
                // unpacking from being hoisted ahead of this group.
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    asm volatile("" : "+v"(xr[s][kp][h]));
                }
                float hv[8];
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    float f[8];
                    unpack8<kBf16>(xr[s][kp][h], f);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float prod = pre[h][s] * f[e];
                        hv[e] = (s == 0) ? prod : hv[e] + prod;
                    }
                }
                u32x4_t o;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    o[w] = pack2_x<kBf16>(hv[2 * w], hv[2 * w + 1]);
                }
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, o), hrs,
                    hLane + 128 * kp, (8 * h * Di + d0i) * 2, kCpolNt);
                if (more) {
#pragma unroll
                    for (int s = 0; s < N; ++s) {
                        load_line(xrs, xLane, Ki, Di, d0i, s, kp, h);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if (prevTile >= 0) {
        post_res(prevTile, prevInvRms, P, lane);
    }
    // Workgroup 0 (team 0, which always has a tile) advances the workspace's
    // epoch once every workgroup has taken this one.
    if (g == 0 && wave == 0) {
        if (!epoch_publish(a.hdr, kWsEpochOff, kWsSeenOff, epoch, (int)gridDim.x, a.spinLimit)) {
            record_timeout(a, lane);
        }
    }
}

template <int N, int KP, bool kBf16, bool kPrep>
size_t fused_lds_bytes()
{
    return (size_t)N * 2 * KP * Shape<N>::NT * 64 * sizeof(u32x4_t) +
           (size_t)kFusedWaves * Rec<N>::BWORDS * sizeof(float) +
           (size_t)kFusedWaves * Rec<N>::WORDS * sizeof(uint64_t);
}

template <int N, int KP, bool kBf16, bool kPrep>
hipError_t fused_prepare_attr()
{
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        err = hipFuncSetAttribute(reinterpret_cast<const void *>(&fused_kernel<N, KP, kBf16, kPrep>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)fused_lds_bytes<N, KP, kBf16, kPrep>());
    });
    return err;
}

template <int N, int KP, bool kBf16, bool kPrep>
int fused_coresident_t(int numCUs)
{
    if (fused_prepare_attr<N, KP, kBf16, kPrep>() != hipSuccess) {
        return -1;
    }
    int perCU = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &perCU, reinterpret_cast<const void *>(&fused_kernel<N, KP, kBf16, kPrep>),
            kFusedWaves * 64, fused_lds_bytes<N, KP, kBf16, kPrep>()) != hipSuccess) {
        return -1;
    }
    return perCU * numCUs;
}

template <int N, int KP, bool kBf16, bool kPrep>
hipError_t launch_fused_t(const Plan &p, void *workspace, uint32_t launchId, hipStream_t stream)
{
    hipError_t err = fused_prepare_attr<N, KP, kBf16, kPrep>();
    if (err != hipSuccess) {
        return err;
    }
    char *ws = static_cast<char *>(workspace);
    FusedArgs a;
    a.x = static_cast<const uint16_t *>(p.x);
    a.phi = p.phi;
    a.gamma = p.hasGamma ? p.gamma : nullptr;
    a.bprep = static_cast<const u32x4_t *>(p.bprep);
    a.alpha = p.alpha;
    a.bias = p.bias;
    a.hIn = static_cast<uint16_t *>(p.hIn);
    a.hPost = p.hPost;
    a.hRes = p.hRes;
    a.hPre = p.hasHPre ? p.hPre : nullptr;
    a.status = reinterpret_cast<uint64_t *>(ws);
    a.statusWord = p.statusWord;
    a.hdr = ws;
    a.bcast = reinterpret_cast<uint64_t *>(ws + p.wsFinal);
    a.recs = reinterpret_cast<uint64_t *>(ws + p.wsFusedPartial);
    a.T = p.T;
    a.D = p.D;
    a.K = p.K;
    a.RT = p.fusedTiles;
    a.P = p.fusedP;
    a.numTeams = p.fusedTeams;
    a.normEps = p.normEps;
    a.hcEps = p.hcEps;
    a.invFlatDim = p.invFlatDim;
    a.launchId = launchId;
    a.spinLimit = p.spinLimit;

    const unsigned lds = (unsigned)fused_lds_bytes<N, KP, kBf16, kPrep>();
    if (!p.fusedCooperative) {
        hipLaunchKernelGGL((fused_kernel<N, KP, kBf16, kPrep>), dim3((unsigned)p.fusedGrid),
                           dim3(kFusedWaves * 64), lds, stream, a);
        return hipGetLastError();
    }
    void *args[] = {&a};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&fused_kernel<N, KP, kBf16, kPrep>),
                                      dim3((unsigned)p.fusedGrid), dim3(kFusedWaves * 64), args,
                                      lds, stream);
}

}  // namespace

// Fused-path instantiations: n = 4 with KP in {4, 2, 1} (DW = 256, 128, 64),
// B built from phi and gamma or copied from prepared weights.
#define MHC_FUSED_DISPATCH_P(FN, PREP, ...)                                    \
    switch (p.fusedDw / 64) {                                                  \
    case 4:                                                                    \
        return p.isBf16 ? FN<4, 4, true, PREP>(__VA_ARGS__) : FN<4, 4, false, PREP>(__VA_ARGS__); \
    case 2:                                                                    \
        return p.isBf16 ? FN<4, 2, true, PREP>(__VA_ARGS__) : FN<4, 2, false, PREP>(__VA_ARGS__); \
    case 1:                                                                    \
        return p.isBf16 ? FN<4, 1, true, PREP>(__VA_ARGS__) : FN<4, 1, false, PREP>(__VA_ARGS__); \
    default:                                                                   \
        break;                                                                 \
    }
#define MHC_FUSED_DISPATCH(FN, ...)                                            \
    if (p.bprep != nullptr) {                                                  \
        MHC_FUSED_DISPATCH_P(FN, true, __VA_ARGS__)                            \
    } else {                                                                   \
        MHC_FUSED_DISPATCH_P(FN, false, __VA_ARGS__)                           \
    }

hipError_t launch_fused(const Plan &p, void *workspace, uint32_t launchId, hipStream_t stream)
{
    if (p.n != 4) {
        return hipErrorNotSupported;
    }
    MHC_FUSED_DISPATCH(launch_fused_t, p, workspace, launchId, stream)
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
