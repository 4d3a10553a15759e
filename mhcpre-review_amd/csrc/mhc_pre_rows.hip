// Row-block kernels for gfx950 (rows path, K % 128 == 0: n = 6 and 8, and small n = 4 batches).
//
// Why x is read twice here.  For n = 8 the B operand of the mixing GEMM
// (gamma * phi split into bf16 hi + lo, 2M = 160 columns) takes 320 bytes per
// element of K.  A slice of K whose B fits one CU's LDS is at most ~450
// elements wide, and the partial sums such a slice would have to hand to the
// other slices of a row (M + 1 = 81 floats) are then as large as its share of
// the row's x.  Keeping x on chip until hPre is known (as the persistent n = 4
// kernels do) would move more bytes between CUs than it saves; so this path
// runs a split-K GEMM that reads x once, and a second pass that reads x again
// for hIn.  Two launches:
//
//   rows_gemm      split-K GEMM over work items (256-row block, K-range).  A
//                  workgroup is 8 waves of 32 rows (two 16-row MFMA blocks).
//                  K is cut into stages of 2 k-steps (one 128-byte line of a
//                  row); K-range kr takes a contiguous run of stages.  x is
//                  read with nontemporal loads (measured on MI355X: 6.4 TB/s
//                  for this read pattern against 4.9 with default caching or
//                  with the ranges' stages interleaved).  Each stage's B goes
//                  through registers into an LDS ring: built from phi and
//                  gamma (256-byte runs of every mix column, split into bf16
//                  hi + lo rows), or copied from prepared weights (fragments
//                  in the order the MFMA reads them, as rows_prep_b writes
//                  them); its x goes into a register ring as whole 128-byte
//                  lines (8 lanes per row), both kAhead stages ahead of the
//                  MFMAs.  A DPP row_ror:8 turns two
//                  line registers into the A fragments of two k-steps.  hi and
//                  lo products accumulate into one fp32 accumulator per mix
//                  column; a Gram MFMA of the same fragments gives the sum of
//                  squares on its diagonal.  Writes the M+1 partial sums of
//                  each (row, K-range) (mix columns, then the sum of squares):
//                  K-range-major, or row-major when there are many K-ranges
//                  (each row's sums then one contiguous run for its epilogue).
//   rows_epilogue  one workgroup per row: the K-range partials summed in
//                  K-range order, invRms, the sigmoid / affine epilogue
//                  (code/op_kernel/mhc_pre.cpp:735-758), and hIn from a second
//                  read of x with round-half-even stores
//                  (code/op_kernel/mhc_pre.cpp:761-826).
//
// rows_prep_b (mhcPrePrepareWeights) writes the prepared fragments:
// [K/32 k-steps][NT tiles][64 lanes] x 16 bytes.  Tile t < Q holds hi of
// columns 16t + l%16 and tile Q + t their lo, in the same lanes; when
// M % 16 == 8 the last tile holds hi (lanes 0-7 of each 16) and lo (lanes
// 8-15) of the last 8 columns.  Lane l holds k = 32ks + 8(l/16) .. +8.
//
// Work items map to XCDs so that the workgroups of one XCD share K-ranges:
// workgroup g runs on XCD g mod X (round-robin dispatch) and takes item
// (g mod X) * C + g / X of the X*C item slots, items numbered row block
// fastest.  The phi runs (or prepared fragments) of an item's K-range are then
// read by the other row blocks of the same K-range from that XCD's L2.  The mapping affects
// speed only.

#include "mhc_pre_device.h"
#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>
#include <utility>

namespace mhc {
namespace {

using namespace dev;

constexpr int kRW = 8;                       // waves per GEMM workgroup (two per SIMD)
constexpr int kRowsWave = 32;                // rows per wave (two 16-row MFMA blocks)
constexpr int kRowBlock = kRW * kRowsWave;   // rows per work item
constexpr int kStageKs = 2;                  // k-steps per stage (kStageKs / 2 lines of a row)
constexpr int kAhead = 3;                    // stages of x loading ahead of the MFMAs
constexpr int kXSlots = kAhead + 1;          // x register ring
constexpr int kBSets = kAhead - 1;           // B staging register sets
// Small-batch GEMM: rows of a workgroup (n = 4 has 2 accumulator tiles per
// 16 rows, n = 6 and 8 have 3 and 5); the wide variant holds twice as many.
template <int N>
constexpr int small_rows() { return N == 4 ? 128 : 64; }
constexpr int kSmallWaves = 4;               // small-batch GEMM: waves building a K-range's B
// Small-batch GEMM: waves per workgroup.  Each multiplies one 16-row block
// by a share of the K-range: half of it in the narrow n = 6 and 8 variants
// (two waves per block), all of it otherwise.  Measured on MI355X (back to
// back, us, one wave / two waves per block): n = 8, D = 7168, T = 64 16.1 /
// 15.5; n = 8, D = 4096, T = 64 14.2 / 13.7; n = 4, D = 7168, T = 128
// 10.5 / 10.9 (16 waves of 89 VGPRs).
template <int N, bool kWide>
constexpr int small_split() { return (kWide || N == 4) ? 1 : 2; }
template <int N, bool kWide>
constexpr int small_waves() { return small_rows<N>() * (kWide ? 2 : 1) / 16 * small_split<N, kWide>(); }
constexpr int kSmallKs = 2;                  // small-batch GEMM: k-steps per wave

// Column tiles of the B operand and the accumulator tile each one adds into.
template <int N>
struct RowsCols {
    static constexpr int M = N * N + 2 * N;
    static constexpr int Q = M / 16;
    static constexpr bool kHalf = (M % 16) == 8;
    static constexpr int NT = 2 * Q + (kHalf ? 1 : 0);  // = 2M / 16
    static constexpr int NA = Q + (kHalf ? 1 : 0);      // accumulator tiles
    static_assert(M % 16 == 0 || M % 16 == 8, "M = n*n + 2n is 24, 48 or 80");
    static constexpr int acc(int t) { return t < Q ? t : (t < 2 * Q ? t - Q : Q); }
    static constexpr bool hi_tile(int t) { return t < Q || t == 2 * Q; }
};

constexpr int kCpolNt = 2;   // nontemporal: x is streamed
constexpr int kCpolDev = 16; // sc1: device scope, written through

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, 0x00020000);
}

template <int kCpol>
__device__ __forceinline__ u32x4_t load16(__amdgpu_buffer_rsrc_t r, int off)
{
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpol));
}

// Waits until at most `kOut` of this wave's vector-memory loads are still in
// flight (they complete in issue order), without waiting on LDS or exports.
template <int kOut>
__device__ __forceinline__ void wait_vm()
{
    static_assert(kOut >= 0 && kOut < 64, "vmcnt range");
    // s_waitcnt fields: vmcnt [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
    constexpr int imm = (kOut & 15) | ((kOut >> 4) << 14) | (7 << 4) | (15 << 8);
    __builtin_amdgcn_s_waitcnt(imm);
}

// Workgroup barrier that orders LDS only (no wait for outstanding global
// loads, which __syncthreads() would add).
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Calls f(std::integral_constant<int, i>{}) for i = 0 .. kCount-1.
template <typename F, int... kIs>
__device__ __forceinline__ void static_for_seq(F &&f, std::integer_sequence<int, kIs...>)
{
    (f(std::integral_constant<int, kIs>{}), ...);
}
template <int kCount, typename F>
__device__ __forceinline__ void static_for(F &&f)
{
    static_for_seq(f, std::make_integer_sequence<int, kCount>{});
}

// A fragments of k-steps 2q and 2q + 1 from line-layout registers r0 (rows
// 0-7) and r1 (rows 8-15).  In a line register lane l holds row l & 7 and the
// 8 columns at 8(l >> 4) + 32((l >> 3) & 1) of a 64-column line; the A
// fragment wants row l & 15 and columns 8(l >> 4) of its k-step, so lanes
// with bit 3 set take the other register's lane l ^ 8 (DPP row_ror:8 with
// banks 2-3 or 0-1 enabled).
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

// ---------------------------------------------------------------------------
// rows_prep_b: one thread per (k-step, accumulator tile, lane): reads 8 k of
// one phi column (and gamma), writes the hi and the lo fragment lanes.
// ---------------------------------------------------------------------------
template <int N>
__global__ __launch_bounds__(256) void rows_prep_b_kernel(const float *__restrict__ phi,
                                                          const float *__restrict__ gamma,
                                                          u32x4_t *__restrict__ bfrag, int64_t K,
                                                          uint32_t *__restrict__ status)
{
    using C = RowsCols<N>;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx == 0 && status != nullptr) {
        *status = kDeviceOk;
    }
    const int64_t total = (K / 32) * C::NA * kWave;
    if (idx >= total) {
        return;
    }
    const int lane = (int)(idx % kWave);
    const int ta = (int)((idx / kWave) % C::NA);
    const int64_t ks = idx / ((int64_t)kWave * C::NA);
    int j, thi, tlo, lhi, llo;
    if (ta < C::Q) {
        j = 16 * ta + (lane & 15);
        thi = ta;
        tlo = C::Q + ta;
        lhi = llo = lane;
    } else {
        if ((lane & 15) >= 8) {
            return;
        }
        j = 16 * C::Q + (lane & 7);
        thi = tlo = 2 * C::Q;
        lhi = lane;
        llo = lane + 8;
    }
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
    u32x4_t hi, lo;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t h, l;
        split2_bf16(b[2 * w], b[2 * w + 1], h, l);
        hi[w] = h;
        lo[w] = l;
    }
    // Nontemporal stores: with plain ones the block GEMM that reads B next
    // ran about 20 us slower at n = 8, D = 8192, T = 5472, for the same
    // bytes fetched from memory.
    u32x4_t *dst = bfrag + ks * C::NT * kWave;
    __builtin_nontemporal_store(hi, &dst[thi * kWave + lhi]);
    __builtin_nontemporal_store(lo, &dst[tlo * kWave + llo]);
}

// ---------------------------------------------------------------------------
// rows_gemm
// ---------------------------------------------------------------------------
struct RowsGemmArgs {
    const uint16_t *x;
    const u32x4_t *bfrag;   // prepared B fragments (kPhi false)
    const float *phi;       // phi [M][K] and gamma [K] or null (kPhi true)
    const float *gamma;
    float *partial;  // element (row, K-range, column) at row * rowStride + kr * rangeStride + column
    int64_t rowStride;
    int64_t rangeStride;
    int64_t T;
    int64_t K;
    int NS;          // stages of K (K / 32 / kStageKs)
    int S;           // K-ranges of ceil(NS / S) stages (the last may be shorter)
    int rowBlocks;   // 256-row blocks
    int perXcd;      // item slots per XCD
    int nXcd;
};

// kPhi: B of each stage is built here from phi and gamma (bit-identical to
// rows_prep_b's fragments: the same product and splits), so a launch needs no
// prep kernel.  The workgroup loads the stage's 64 values of K of every mix
// column as 256-byte runs (16 lanes per column, 4 values per lane, whole
// lines), multiplies by gamma, splits into bf16 hi and lo and writes them as
// rows of an LDS block: row j (hi of column j) and row M + j (its lo), each
// 64 values padded to kPhiPitch bytes, so that the 16 lanes of a fragment
// read phase (16 rows, pitch 144 bytes) hit distinct banks.  The MFMAs then
// read their fragments from those rows.  Without kPhi the stage's fragments
// come from the prepared buffer in fragment order.
constexpr int kPhiPitch = kStageKs * 32 * 2 + 16;

template <int N, bool kBf16, bool kPhi>
__global__ __launch_bounds__(kRW * 64) void rows_gemm_kernel(RowsGemmArgs a)
{
    using C = RowsCols<N>;
    constexpr int M = C::M;
    constexpr int NT = C::NT;
    constexpr int NA = C::NA;
    constexpr int Q = C::Q;
    constexpr int kLines = kStageKs / 2;      // 128-byte lines of a row per stage
    constexpr int SF = kStageKs * NT;         // B fragments per stage
    constexpr int NB = (SF + kRW - 1) / kRW;  // fragments each wave copies (some waves one fewer)
    constexpr int NP = (16 * M + kRW * kWave - 1) / (kRW * kWave);  // phi loads per lane and stage
    constexpr int kXLoads = 4 * kLines;       // x line loads per wave and stage
    constexpr int kBLoads = kPhi ? NP + 1 : NB;  // B loads per wave and stage (phi runs + gamma)
    constexpr int kUnroll = kXSlots;          // steps per loop trip: every ring index static
    static_assert(kUnroll % kBSets == 0 && kUnroll % 2 == 0, "static ring indices");
    static_assert(kStageKs == 2, "a stage is 64 values of K: 16 lanes x 4 per mix column");
    constexpr int kStageBytes = kPhi ? 2 * M * kPhiPitch : SF * kWave * 16;
    __shared__ __attribute__((aligned(16))) char bsh[2][kStageBytes];  // B of stages s and s + 1

    const int lane = threadIdx.x & 63;
    // Wave-uniform (scalar) wave index: the buffer resources built from it
    // stay in scalar registers.
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = blockIdx.x;
    const int f = (g % a.nXcd) * a.perXcd + g / a.nXcd;
    if (f >= a.rowBlocks * a.S) {
        return;
    }
    const int rb = f % a.rowBlocks;
    const int kr = f / a.rowBlocks;
    const int per = (a.NS + a.S - 1) / a.S;
    const int gs0 = kr * per;                 // first stage of this K-range
    const int nst = min(per, a.NS - gs0);     // its stages (at least one)

    // x of this wave's 32 rows, through a resource that covers the valid
    // rows only: loads of rows past T return zeros.
    const int64_t r0 = (int64_t)rb * kRowBlock + (int64_t)kRowsWave * w;
    const int vrows = (int)max((int64_t)0, min((int64_t)kRowsWave, a.T - r0));
    const int K2 = (int)(a.K * 2);  // row stride in bytes
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + (vrows > 0 ? r0 * a.K : 0), vrows * K2);
    const int xLane = (lane & 7) * K2 + 2 * (8 * (lane >> 4) + 32 * ((lane >> 3) & 1));
    const __amdgpu_buffer_rsrc_t br = make_rsrc(a.bfrag, kPhi ? 0 : a.NS * SF * kWave * 16);
    const bool hasGamma = a.gamma != nullptr;
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.phi, kPhi ? M * K2 * 2 : 0);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.gamma, kPhi && hasGamma ? K2 * 2 : 0);
    // kPhi: lane l of wave w loads, with its i-th phi load, the 4 values of K
    // at 4 (l & 15) of mix column pj(i) = 32 i + 4 w + (l >> 4) (none past M).
    const int pk = 4 * (lane & 15);
    auto pj = [&](int i) { return 32 * i + 4 * w + (lane >> 4); };

    u32x4_t xs[kXSlots][4][kLines];  // [slot][8-row group][line of the stage]
    u32x4_t bst[kBSets][kBLoads];    // B of a stage on its way to LDS

    // Per-lane offsets are loop-invariant registers and the stage's part of
    // each address is a scalar offset.
    const int bLane = w * (kWave * 16) + lane * 16;
    int xOff[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        xOff[h] = xLane + 8 * h * K2;
    }

    // Stage s's loads: its B fragments into staging set s mod kBSets, then
    // its x lines into ring slot s mod kXSlots.  Every stage issues the same
    // loads in the same order, live or not: stages past the K-range (and a
    // wave's fragment slots past SF) read through size-0 resources, so the
    // counter waits below stay exact.
    auto issue = [&](int s, u32x4_t(&bd)[kBLoads], u32x4_t(&xd)[4][kLines]) {
        const bool live = s < nst;
        const int gs = gs0 + s;  // stage of K
        if constexpr (kPhi) {
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const __amdgpu_buffer_rsrc_t pq = (live && 32 * i + 4 * w < M) ? pr : make_rsrc(a.phi, 0);
                bd[i] = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(pq, (pj(i) * (K2 / 2) + pk) * 4, gs * 256, 0));
            }
            bd[NP] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(live ? gr : make_rsrc(a.gamma, 0), pk * 4, gs * 256, 0));
        } else {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int fr = w + kRW * i;
                const __amdgpu_buffer_rsrc_t bq = (live && fr < SF) ? br : make_rsrc(a.bfrag, 0);
                bd[i] = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(bq, bLane, (gs * SF + kRW * i) * (kWave * 16), 0));
            }
        }
        // Keep the B loads ahead of the x lines in the (in-order) load
        // counter: waiting for them must not wait for this stage's x.
        __builtin_amdgcn_sched_barrier(0);
        const __amdgpu_buffer_rsrc_t xq = live ? xr : make_rsrc(a.x, 0);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
#pragma unroll
            for (int c = 0; c < kLines; ++c) {
                xd[h][c] = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xq, xOff[h] + 128 * c,
                                                                   gs * (kStageKs * 64), kCpolNt));
            }
        }
        // Stages stay in issue order in the load counter.
        __builtin_amdgcn_sched_barrier(0);
    };
    auto stash = [&](int sl, const u32x4_t(&bd)[kBLoads]) {
        if constexpr (kPhi) {
            const f32x4_t gv = __builtin_bit_cast(f32x4_t, bd[NP]);
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                if (32 * i + 4 * w < M) {  // (wave-uniform)
                    f32x4_t bv = __builtin_bit_cast(f32x4_t, bd[i]);
                    if (hasGamma) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            bv[e] = bv[e] * gv[e];
                        }
                    }
                    uint32_t h0, l0, h1, l1;  // bf16(B) and bf16(B - hi) of k pairs (pk, pk+1), (pk+2, pk+3)
                    split2_bf16(bv[0], bv[1], h0, l0);
                    split2_bf16(bv[2], bv[3], h1, l1);
                    char *row = &bsh[sl][pj(i) * kPhiPitch + 2 * pk];
                    *reinterpret_cast<uint2 *>(row) = make_uint2(h0, h1);
                    *reinterpret_cast<uint2 *>(row + M * kPhiPitch) = make_uint2(l0, l1);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int fr = w + kRW * i;
                if (fr < SF) {
                    reinterpret_cast<u32x4_t *>(bsh[sl])[fr * kWave + lane] = bd[i];
                }
            }
        }
    };
    // kPhi: the byte offset in a stage block of lane `lane`'s fragment of
    // tile t, k-step 0 (k-step ksl adds 64 bytes): tile t < Q holds hi of
    // columns 16 t + l % 16 (rows 16 t + l % 16), tile Q + t their lo (rows
    // M + ...); when M % 16 == 8, tile 2Q holds hi (lanes l % 16 < 8) and lo
    // (the others) of columns 16 Q + l % 8.  Lane l holds k = 8 (l / 16) ...
    const int fragBase = (lane & 15) * kPhiPitch + 16 * (lane >> 4);
    const int halfBase = (((lane & 15) < 8 ? 0 : M) + 16 * Q + (lane & 7)) * kPhiPitch + 16 * (lane >> 4);
    auto frag_off = [&](int t) {
        if (t < Q) {
            return fragBase + 16 * t * kPhiPitch;
        }
        if (t < 2 * Q) {
            return fragBase + (M + 16 * (t - Q)) * kPhiPitch;
        }
        return halfBase;
    };

    f32x4_t acc[2][NA];
    f32x4_t gram[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        gram[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < NA; ++t) {
            acc[r][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
    }

    // Prologue: stages 0 .. kAhead - 1 in flight, stage 0's B in LDS.
    issue(0, bst[0], xs[0]);
    wait_vm<kXLoads>();
    stash(0, bst[0]);
#pragma unroll
    for (int s = 1; s < kAhead; ++s) {
        issue(s, bst[s % kBSets], xs[s]);
    }

    // Step s: x of stage s and B of stage s + 1 have arrived once only the
    // loads issued after B(s + 1) -- x of stage s + 1 and stages s + 2 ..
    // s + kAhead - 1 -- may still be in flight.  The barrier makes every
    // wave's stash of B(s) visible and tells every wave that all reads of
    // LDS slot (s + 1) mod 2 (stage s - 1) are done; B(s + 1) goes there,
    // and stage s + kAhead's loads go out into the staging set and ring slot
    // just freed.  Loads of stages past the K-range read zeros for both x
    // and B.
    // One step, stage s0 + u, with u (the ring and staging slots) a
    // compile-time constant in every copy of the body.
    auto step = [&](int s0, auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
        const int s = s0 + u;
        const int sl = u % kXSlots;
        const int bl = u % 2;
        wait_vm<kXLoads + (kAhead - 2) * (kBLoads + kXLoads)>();
        lds_barrier();
        stash((u + 1) % 2, bst[(u + 1) % kBSets]);
        issue(s + kAhead, bst[(u + kAhead) % kBSets], xs[(u + kAhead) % kXSlots]);
        if (vrows > 0) {
            // All of the stage's B fragments are read before its MFMAs,
            // so the LDS latency is paid once per stage.
            u32x4_t bf[kStageKs][NT];
#pragma unroll
            for (int ksl = 0; ksl < kStageKs; ++ksl) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if constexpr (kPhi) {
                        bf[ksl][t] = *reinterpret_cast<const u32x4_t *>(&bsh[bl][frag_off(t) + 64 * ksl]);
                    } else {
                        bf[ksl][t] = reinterpret_cast<const u32x4_t *>(bsh[bl])[(ksl * NT + t) * kWave + lane];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < kLines; ++c) {
                u32x4_t af[2][2];  // [16-row block][k-step of the line]
                lines_to_frags(xs[sl][0][c], xs[sl][1][c], af[0][0], af[0][1]);
                lines_to_frags(xs[sl][2][c], xs[sl][3][c], af[1][0], af[1][1]);
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int ksl = 2 * c + kk;
                    if constexpr (kBf16) {
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            const u32x4_t b = bf[ksl][t];
                            acc[0][C::acc(t)] = mfma16(af[0][kk], b, acc[0][C::acc(t)]);
                            acc[1][C::acc(t)] = mfma16(af[1][kk], b, acc[1][C::acc(t)]);
                        }
                        gram[0] = mfma16(af[0][kk], af[0][kk], gram[0]);
                        gram[1] = mfma16(af[1][kk], af[1][kk], gram[1]);
                    } else {
                        // fp16 x = hi + lo exactly in bf16; x_lo meets the
                        // hi B columns only (x_lo * B_lo is below 2^-16 of
                        // the product).
                        u32x4_t xh[2], xl[2];
#pragma unroll
                        for (int r = 0; r < 2; ++r) {
                            float fx[8];
                            unpack8<false>(af[r][kk], fx);
                            split_f16_to_bf16(fx, xh[r], xl[r]);
                        }
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            const u32x4_t b = bf[ksl][t];
#pragma unroll
                            for (int r = 0; r < 2; ++r) {
                                acc[r][C::acc(t)] = mfma16(xh[r], b, acc[r][C::acc(t)]);
                                if (C::hi_tile(t)) {
                                    acc[r][C::acc(t)] = mfma16(xl[r], b, acc[r][C::acc(t)]);
                                }
                            }
                        }
                        gram[0] = mfma16_f16(af[0][kk], af[0][kk], gram[0]);
                        gram[1] = mfma16_f16(af[1][kk], af[1][kk], gram[1]);
                    }
                }
            }
        }
    };
    // Whole trips of kUnroll stages; then the last, partial trip as a second
    // copy of the body that skips the stages past the K-range (the same for
    // every wave of the workgroup), so that the branch stays out of the main
    // loop.
    int s0 = 0;
    for (; s0 + kUnroll <= nst; s0 += kUnroll) {
        static_for<kUnroll>([&](auto uc) __attribute__((always_inline)) { step(s0, uc); });
    }
    if (s0 < nst) {
        static_for<kUnroll>([&](auto uc) __attribute__((always_inline)) {
            if (s0 + decltype(uc)::value < nst) {
                step(s0, uc);
            }
        });
    }
    // Loads of the stages past the K-range may still be in flight.
    __builtin_amdgcn_s_waitcnt(0);
    if (vrows == 0) {
        return;
    }

    // C fragment: lane l, register e holds row 4(l >> 4) + e, column l & 15
    // of its 16 x 16 tile.
    float *dst = a.partial + (int64_t)r0 * a.rowStride + (int64_t)kr * a.rangeStride;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = 16 * r + 4 * (lane >> 4) + e;
            const bool ok = row < vrows;
            float *drow = dst + (int64_t)row * a.rowStride;
#pragma unroll
            for (int t = 0; t < Q; ++t) {
                if (ok) {
                    drow[16 * t + (lane & 15)] = acc[r][t][e];
                }
            }
            if constexpr (C::kHalf) {
                // hi in lanes 0-7 of each 16, lo of the same column 8 lanes up.
                const float v = acc[r][Q][e];
                const float lo = row_swap8(v);
                if (ok && (lane & 15) < 8) {
                    drow[16 * Q + (lane & 7)] = v + lo;
                }
            }
            // Diagonal of the Gram tile: the row's sum of squares.
            if (ok && (lane & 15) == 4 * (lane >> 4) + e) {
                drow[M] = gram[r][e];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// rows_small: decode-shaped batches (T <= small_rows(n), or twice that in
// the wide variant).  One workgroup per K-range of kSmallWaves * kSmallKs
// k-steps.  Each of the first kSmallWaves waves builds the B fragments of
// kSmallKs of them from phi and gamma (or copies them from the prepared
// buffer) into LDS; after one barrier every wave multiplies its 16-row block
// by its share of the K-range's fragments (the first or second half in the
// narrow n = 6 and 8 variants, whose two sums per block then meet in LDS in
// that order; all of them otherwise) and the block's partial sums go out
// from registers.  Rows past T read as zeros and are not written; a block that
// starts at or past T skips the products.
// ---------------------------------------------------------------------------
struct RowsSmallArgs {
    const uint16_t *x;
    const float *phi;
    const float *gamma;
    const u32x4_t *bprep;  // prepared B fragments [K/32][NT][64] (kPrep only)
    float *partial;    // element (row, K-range, column) at row * rowStride + kr * rangeStride + column
    uint32_t *status;  // low half of the device status word
    int64_t rowStride;
    int64_t rangeStride;
    int64_t T;
    int64_t K;
};

template <int N, bool kBf16, bool kPrep, bool kWide>
__global__ __launch_bounds__((small_waves<N, kWide>() * 64)) void rows_small_kernel(RowsSmallArgs a)
{
    using C = RowsCols<N>;
    constexpr int M = C::M;
    constexpr int NA = C::NA;
    constexpr int NT = C::NT;
    constexpr int Q = C::Q;
    constexpr int kKs = kSmallWaves * kSmallKs;          // k-steps per workgroup
    constexpr int kBlocks = small_rows<N>() * (kWide ? 2 : 1) / 16;  // 16-row blocks
    constexpr int kSplit = small_split<N, kWide>();      // waves per block
    constexpr int kKsW = kKs / kSplit;                   // k-steps per wave
    static_assert(kSmallKs == 2, "one 128-byte line of each row per k-step pair");
    static_assert(kKsW % 2 == 0, "whole k-step pairs per wave");
    static_assert(small_waves<N, kWide>() >= kSmallWaves, "every builder wave also multiplies");
    // LDS: one region per builder wave.  It first holds the wave's phi block in row
    // order (row pitch kPhiPitch floats: consecutive rows start 4 banks
    // apart), which the wave reads back in B-fragment order, then the
    // wave's fragments [kSmallKs][NT][64 lanes] (hi tiles, lo tiles, then
    // the half tile), in the order of the prepared buffer.
    constexpr int kPhiK = kSmallKs * 32;
    constexpr int kPhiPitch = kPhiK + 4;
    constexpr int kStageBytes = M * kPhiPitch * 4;
    constexpr int kFragBytes = kSmallKs * NT * kWave * 16;
    constexpr int kRegion = kStageBytes > kFragBytes ? kStageBytes : kFragBytes;
    __shared__ __attribute__((aligned(16))) char lds[kSmallWaves * kRegion];
    // After the products the second-half waves' sums pass through the same
    // LDS: [block][NA accumulator tiles + Gram tile][64 lanes].
    static_assert(kSplit == 1 || kBlocks * (NA + 1) * kWave * 16 <= kSmallWaves * kRegion,
                  "the half sums fit the fragment regions");

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool builder = w < kSmallWaves;  // wave-uniform
    const int wb = builder ? w : 0;
    char *const region = lds + wb * kRegion;
    float *const stage = reinterpret_cast<float *>(region);
    u32x4_t *const frags = reinterpret_cast<u32x4_t *>(region);
    const int kr = blockIdx.x;
    const int T = (int)a.T;
    if (kr == 0 && threadIdx.x == 0) {
        *a.status = kDeviceOk;
    }
    const int K2 = (int)(a.K * 2);
    const int64_t kg0 = (int64_t)kr * kKs;            // first k-step of the workgroup
    const int64_t ks0 = kg0 + (int64_t)wb * kSmallKs;  // first k-step this wave builds
    const int rb = w % kBlocks;                        // this wave's 16-row block
    const int half = w / kBlocks;                      // its share of the k-steps
    const int kw0 = half * kKsW;                       // first k-step (in the range) it multiplies

    // phi rows as whole 256-byte runs (the wave's 64 k of 4 rows per load),
    // into LDS in row order; read back below in B-fragment order.  Prepared
    // weights: the wave's NT fragments of each of its k-steps instead.
    constexpr int kPhiLoads = kPrep ? 1 : M / 4;
    static_assert(M % 4 == 0, "4 phi rows per load");
    f32x4_t phl[kPhiLoads];
    f32x4_t gm[kSmallKs][2];
    u32x4_t pf[kSmallKs][kPrep ? NT : 1];
    if (!builder) {
        // No B to build: straight to the barrier.
    } else if constexpr (kPrep) {
#pragma unroll
        for (int kk = 0; kk < kSmallKs; ++kk) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                pf[kk][t] = a.bprep[((ks0 + kk) * NT + t) * kWave + lane];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < kPhiLoads; ++i) {
            const int j = 4 * i + (lane >> 4);
            phl[i] = *reinterpret_cast<const f32x4_t *>(a.phi + (int64_t)j * a.K + ks0 * 32 + 4 * (lane & 15));
        }
#pragma unroll
        for (int kk = 0; kk < kSmallKs; ++kk) {
            const int64_t k0 = (ks0 + kk) * 32 + 8 * (lane >> 4);
            const f32x4_t *gsrc = reinterpret_cast<const f32x4_t *>(a.gamma != nullptr ? a.gamma + k0 : a.phi);
            gm[kk][0] = gsrc[0];
            gm[kk][1] = gsrc[1];
        }
    }
    // Every wave's weight loads are in the CU's memory queue before any x
    // load (a wave stalls at a load while the queue is full, so x issued
    // first held back the B build); every load is issued before any use:
    // one memory round trip.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // x as whole 128-byte lines (two k-steps of a row): for pair p, register
    // (p, h) holds, in lane l, row 16 rb + 8h + (l & 7) and the 8 k at
    // 8(l >> 4) + 32((l >> 3) & 1) of k-steps kg0 + kw0 + 2p and the next;
    // a DPP exchange turns each pair into the A fragments of the two.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, T * K2);
    constexpr int kPairs = kKsW / 2;
    u32x4_t xln[kPairs][2];
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            xln[p][h] = load16<kCpolNt>(xr, (16 * rb + 8 * h + (lane & 7)) * K2 +
                                                (int)((kg0 + kw0 + 2 * p) * 64) + 16 * (lane >> 4) +
                                                64 * ((lane >> 3) & 1));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    if (!builder) {
    } else if constexpr (kPrep) {
#pragma unroll
        for (int kk = 0; kk < kSmallKs; ++kk) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                frags[(kk * NT + t) * kWave + lane] = pf[kk][t];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < kPhiLoads; ++i) {
            *reinterpret_cast<f32x4_t *>(stage + (4 * i + (lane >> 4)) * kPhiPitch + 4 * (lane & 15)) = phl[i];
        }
        // B-fragment order: tile ta covers mix columns 16ta + (l & 15); the
        // half tile's lanes 8-15 hold the lo half of the column of lanes 0-7.
        // (The wave reads only its own region, which it wrote above, and
        // overwrites it with its fragments once every read has returned.)
        f32x4_t ph[kSmallKs][NA][2];
#pragma unroll
        for (int kk = 0; kk < kSmallKs; ++kk) {
#pragma unroll
            for (int ta = 0; ta < NA; ++ta) {
                const int j = ta < Q ? 16 * ta + (lane & 15) : 16 * Q + (lane & 7);
                const float *src = stage + j * kPhiPitch + 32 * kk + 8 * (lane >> 4);
                ph[kk][ta][0] = *reinterpret_cast<const f32x4_t *>(src);
                ph[kk][ta][1] = *reinterpret_cast<const f32x4_t *>(src + 4);
            }
        }
        const bool hasGamma = a.gamma != nullptr;
        u32x4_t fr[kSmallKs][NT];
#pragma unroll
        for (int kk = 0; kk < kSmallKs; ++kk) {
#pragma unroll
            for (int ta = 0; ta < NA; ++ta) {
                float b[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    b[e] = ph[kk][ta][e >> 2][e & 3];
                    if (hasGamma) {
                        b[e] = b[e] * gm[kk][e >> 2][e & 3];
                    }
                }
                u32x4_t bh, bl;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t h, l;
                    split2_bf16(b[2 * q], b[2 * q + 1], h, l);
                    bh[q] = h;
                    bl[q] = l;
                }
                if (ta < Q) {
                    fr[kk][ta] = bh;
                    fr[kk][Q + ta] = bl;
                } else if constexpr (C::kHalf) {
                    // Half tile: hi in lanes 0-7 of each 16, lo in lanes 8-15.
                    fr[kk][2 * Q] = (lane & 15) < 8 ? bh : bl;
                }
            }
        }
#pragma unroll
        for (int kk = 0; kk < kSmallKs; ++kk) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                frags[(kk * NT + t) * kWave + lane] = fr[kk][t];
            }
        }
    }
    lds_barrier();

    // Whether this wave's block holds rows below T (wave-uniform).
    const bool live = 16 * rb < T;
    f32x4_t acc[NA];
    f32x4_t gram = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NA; ++t) {
        acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (live) {
        u32x4_t xa[kKsW];
#pragma unroll
        for (int p = 0; p < kPairs; ++p) {
            lines_to_frags(xln[p][0], xln[p][1], xa[2 * p], xa[2 * p + 1]);
        }
        // This wave's k-steps in order: k-step kk's fragments were built by
        // wave kk / kSmallKs.
#pragma unroll
        for (int q = 0; q < kKsW; ++q) {
            const int kk = kw0 + q;
            const u32x4_t *src = reinterpret_cast<const u32x4_t *>(lds + (kk / kSmallKs) * kRegion) +
                                 (kk % kSmallKs) * NT * kWave + lane;
            u32x4_t bf[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                bf[t] = src[t * kWave];
            }
            u32x4_t xh, xl;
            if constexpr (!kBf16) {
                float fx[8];
                unpack8<false>(xa[q], fx);
                split_f16_to_bf16(fx, xh, xl);
            }
#pragma unroll
            for (int t = 0; t < Q; ++t) {
                if constexpr (kBf16) {
                    acc[t] = mfma16(xa[q], bf[t], acc[t]);
                    acc[t] = mfma16(xa[q], bf[Q + t], acc[t]);
                } else {
                    acc[t] = mfma16(xh, bf[t], acc[t]);
                    acc[t] = mfma16(xh, bf[Q + t], acc[t]);
                    acc[t] = mfma16(xl, bf[t], acc[t]);
                }
            }
            if constexpr (C::kHalf) {
                if constexpr (kBf16) {
                    acc[Q] = mfma16(xa[q], bf[2 * Q], acc[Q]);
                } else {
                    acc[Q] = mfma16(xh, bf[2 * Q], acc[Q]);
                    acc[Q] = mfma16(xl, bf[2 * Q], acc[Q]);
                }
            }
            if constexpr (kBf16) {
                gram = mfma16(xa[q], xa[q], gram);
            } else {
                gram = mfma16_f16(xa[q], xa[q], gram);
            }
        }
    }
    if constexpr (kSplit == 2) {
        // The second half's sums, added to the first half's in that order.
        // Every wave takes both barriers (the first: all fragment reads are
        // done before the regions are overwritten).
        f32x4_t *red = reinterpret_cast<f32x4_t *>(lds) + rb * (NA + 1) * kWave + lane;
        lds_barrier();
        if (half == 1 && live) {
#pragma unroll
            for (int t = 0; t < NA; ++t) {
                red[t * kWave] = acc[t];
            }
            red[NA * kWave] = gram;
        }
        lds_barrier();
        if (half == 1 || !live) {
            return;
        }
#pragma unroll
        for (int t = 0; t < NA; ++t) {
            acc[t] = acc[t] + red[t * kWave];
        }
        gram = gram + red[NA * kWave];
    } else if (!live) {
        return;
    }

    // Partial sums of this block's rows (C fragment: lane l, register e
    // holds row 4(l >> 4) + e, column l & 15 of its tile); read once, by the
    // epilogue.
    float *dst = a.partial + (int64_t)kr * a.rangeStride;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = 16 * rb + 4 * (lane >> 4) + e;
        const bool ok = row < T;
        float *drow = dst + (int64_t)row * a.rowStride;
#pragma unroll
        for (int t = 0; t < Q; ++t) {
            if (ok) {
                __builtin_nontemporal_store(acc[t][e], &drow[16 * t + (lane & 15)]);
            }
        }
        if constexpr (C::kHalf) {
            // hi in lanes 0-7 of each 16, lo of the same column 8 lanes up.
            const float v = acc[Q][e];
            const float lo = row_swap8(v);
            if (ok && (lane & 15) < 8) {
                __builtin_nontemporal_store(v + lo, &drow[16 * Q + (lane & 7)]);
            }
        }
        // Diagonal of the Gram tile: the row's sum of squares.
        if (ok && (lane & 15) == 4 * (lane >> 4) + e) {
            __builtin_nontemporal_store(gram[e], &drow[M]);
        }
    }
}

// ---------------------------------------------------------------------------
// rows_epilogue: one workgroup of 256 threads per row; each thread holds 4
// column octets of all n streams, so one row's x (up to D = 8192) is in
// flight at once and a CU keeps several rows in flight.
// ---------------------------------------------------------------------------
struct RowsEpiArgs {
    const uint16_t *x;
    const float *partial;  // element (row, K-range, column) at row * rowStride + kr * rangeStride + column
    int64_t rowStride;
    int64_t rangeStride;
    const float *alpha;
    const float *bias;
    uint16_t *hIn;
    float *hPost;
    float *hRes;
    float *hPre;
    int64_t T;
    int64_t D;
    int64_t row0;  // row of workgroup 0 (launches of kEpilogueRowsPerLaunch rows)
    int S;
    float normEps;
    float hcEps;
    float invFlatDim;
};

template <int N, bool kBf16, int kEpiThreads, int kEpiOct>
__global__ __launch_bounds__(kEpiThreads) void rows_epilogue_kernel(RowsEpiArgs a)
{
    constexpr int M = N * N + 2 * N;
    constexpr int COLS = M + 1;
    constexpr int G = kEpiThreads / COLS;  // partial-sum groups
    __shared__ float red[G][COLS];
    __shared__ float smix[COLS];
    __shared__ float spre[N];

    const int64_t row = a.row0 + blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t DO = a.D / 8;  // column octets
    // Part blockIdx.y of gridDim.y writes the hIn octets [oBeg, oEnd) of the
    // row; every part evaluates the row's sums, part 0 writes hPost, hRes
    // and hPre.
    const int64_t partOct = (DO + gridDim.y - 1) / gridDim.y;
    const int64_t oBeg = min(DO, (int64_t)blockIdx.y * partOct);
    const int64_t oEnd = min(DO, oBeg + partOct);
    const bool part0 = blockIdx.y == 0;
    const int Di2 = (int)(a.D * 2);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + row * N * a.D, N * Di2);
    const __amdgpu_buffer_rsrc_t hr = make_rsrc(a.hIn + row * a.D, Di2);
    const int xLane = (int)(oBeg + tid) * 16;

    // bias and alpha for this thread's output column, loaded up front so
    // that their round trip overlaps the others.
    const float biasJ = tid < M ? a.bias[tid] : 0.f;
    const float alphaJ = tid < N ? a.alpha[0] : (tid < 2 * N ? a.alpha[1] : a.alpha[2]);

    // The first pass of x loads, issued so that its round trip overlaps the
    // partial sums': before them in the narrow variant, after the first
    // batch of them in the wide one (a wave stalls at a load while the CU's
    // memory queue is full, and the sums are needed first).  In the wide
    // variant threads past the part's octets load nothing (with a row split
    // over parts, most of its threads: n = 8, D = 7168, T = 64 14.8 -> 14.1
    // us); the narrow one loads them (other columns' data or zeros,
    // size-bounded resource, not stored) rather than branch around its
    // loads (n = 8, D = 8192, T = 5472: 281.1 against 282.2 us).
    u32x4_t xv[kEpiOct][N];
    auto load_x = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int o = 0; o < kEpiOct; ++o) {
            if (kEpiThreads < 1024 || oBeg + tid + (int64_t)o * kEpiThreads < oEnd) {
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    xv[o][s] = load16<kCpolNt>(xr, xLane + o * (kEpiThreads * 16) + s * Di2);
                }
            } else {
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    xv[o][s] = u32x4_t{0u, 0u, 0u, 0u};
                }
            }
        }
    };

    // Partial sums: group q sums K-ranges [q*Sg, (q+1)*Sg) of column j in
    // order; the groups are then added in group order.
    const int q = tid / COLS;
    const int j = tid - q * COLS;
    const int Sg = (a.S + G - 1) / G;
    const int sBeg = q < G ? q * Sg : 0;
    const int sEnd = q < G ? min(a.S, sBeg + Sg) : 0;
    const float *src = a.partial + row * a.rowStride + (q < G ? j : 0);
    const int64_t stride = a.rangeStride;
    // Wide variant (small batches with many K-ranges; its use is set by
    // rows_epilogue_wide): up to kBatch are loaded before the first add (one
    // memory round trip, where a load per add costs one each), then added in
    // K-range order.  Slots past the group's range load nothing.
    constexpr int kBatch = 32;
    float t0[kEpiThreads >= 1024 ? kBatch : 1];
    if constexpr (kEpiThreads >= 1024) {
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            t0[i] = sBeg + i < sEnd ? src[(int64_t)(sBeg + i) * stride] : 0.f;
        }
    }
    load_x();
    if (q < G) {
        float v = 0.f;
        if constexpr (kEpiThreads >= 1024) {
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                if (sBeg + i < sEnd) {
                    v = v + t0[i];
                }
            }
            for (int sk = sBeg + kBatch; sk < sEnd; sk += kBatch) {
                float t[kBatch];
#pragma unroll
                for (int i = 0; i < kBatch; ++i) {
                    t[i] = sk + i < sEnd ? src[(int64_t)(sk + i) * stride] : 0.f;
                }
#pragma unroll
                for (int i = 0; i < kBatch; ++i) {
                    if (sk + i < sEnd) {
                        v = v + t[i];
                    }
                }
            }
        } else {
            int sk = sBeg;
            for (; sk + 8 <= sEnd; sk += 8) {
                float t[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    t[i] = src[(int64_t)(sk + i) * stride];
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    v = v + t[i];
                }
            }
            for (; sk < sEnd; ++sk) {
                v = v + src[(int64_t)sk * stride];
            }
        }
        red[q][j] = v;
    }
    __syncthreads();
    if (tid < COLS) {
        float v = red[0][tid];
#pragma unroll
        for (int i = 1; i < G; ++i) {
            v = v + red[i][tid];
        }
        smix[tid] = v;
    }
    __syncthreads();

    if (tid < M) {
        const float invRms = ref_inv_rms(smix[M], a.invFlatDim, a.normEps);
        const float mix = smix[tid];
        const float sc = invRms * alphaJ;
        if (tid < N) {
            const float v = ref_sigmoid(mix * sc, biasJ, a.hcEps);
            spre[tid] = v;
            if (a.hPre != nullptr && part0) {
                a.hPre[row * N + tid] = v;
            }
        } else if (part0) {
            if (tid < 2 * N) {
                const float v = ref_sigmoid(mix * sc, biasJ, 0.0f);
                a.hPost[row * N + (tid - N)] = v * 2.0f;
            } else {
                const float v = mix * sc;
                a.hRes[row * (N * N) + (tid - 2 * N)] = v + biasJ;
            }
        }
    }
    __syncthreads();

    float pre[N];
#pragma unroll
    for (int s = 0; s < N; ++s) {
        pre[s] = spre[s];
    }
    // hIn[d] = RNE(sum over s of pre[s] * x[s][d]), summed in stream order.
    for (int64_t base = 0; oBeg + base < oEnd; base += (int64_t)kEpiThreads * kEpiOct) {
        if (base > 0) {
#pragma unroll
            for (int o = 0; o < kEpiOct; ++o) {
                if (kEpiThreads < 1024 || oBeg + base + tid + (int64_t)o * kEpiThreads < oEnd) {
#pragma unroll
                    for (int s = 0; s < N; ++s) {
                        xv[o][s] = load16<kCpolNt>(xr, (int)(base * 16) + xLane + o * (kEpiThreads * 16) + s * Di2);
                    }
                }
            }
        }
#pragma unroll
        for (int o = 0; o < kEpiOct; ++o) {
            const int d8 = (int)(oBeg + base) + tid + kEpiThreads * o;
            float acc[8];
            {
                float f[8];
                unpack8<kBf16>(xv[o][0], f);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    acc[e] = pre[0] * f[e];
                }
            }
#pragma unroll
            for (int s = 1; s < N; ++s) {
                float f[8];
                unpack8<kBf16>(xv[o][s], f);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float p = pre[s] * f[e];
                    acc[e] = acc[e] + p;
                }
            }
            u32x4_t out;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                out[w] = pack2_x<kBf16>(acc[2 * w], acc[2 * w + 1]);
            }
            // hIn goes out with device-scope (write-through) stores: about
            // 3 us faster than nontemporal ones at n = 8, D = 8192, T = 5472.
            if (d8 < oEnd) {
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, out), hr,
                    d8 * 16, 0, kCpolDev);
            }
        }
    }
}

template <int N, bool kBf16>
hipError_t launch_rows_t(const Plan &p, void *workspace, int nXcd, hipStream_t stream)
{
    char *ws = static_cast<char *>(workspace);
    uint32_t *status = reinterpret_cast<uint32_t *>(ws);
    float *partial = reinterpret_cast<float *>(ws + p.wsRowsPartial);
    constexpr int64_t kCols = RowsCols<N>::M + 1;
    const int64_t rowStride = p.rowsRowMajor ? p.rowsS * kCols : kCols;
    const int64_t rangeStride = p.rowsRowMajor ? kCols : p.T * kCols;
    using C = RowsCols<N>;
    hipError_t err = hipSuccess;

    const u32x4_t *bprep = static_cast<const u32x4_t *>(p.bprep);
    if (p.rowsSmall) {
        RowsSmallArgs sa;
        sa.x = static_cast<const uint16_t *>(p.x);
        sa.phi = p.phi;
        sa.gamma = p.hasGamma ? p.gamma : nullptr;
        sa.bprep = bprep;
        sa.partial = partial;
        sa.rowStride = rowStride;
        sa.rangeStride = rangeStride;
        sa.status = status;
        sa.T = p.T;
        sa.K = p.K;
        // More rows than the narrow variant holds: the wide one.
        const dim3 grid((unsigned)p.rowsS);
        if (p.T > small_rows<N>()) {
            const dim3 block(small_waves<N, true>() * 64);
            if (bprep != nullptr) {
                hipLaunchKernelGGL((rows_small_kernel<N, kBf16, true, true>), grid, block, 0, stream, sa);
            } else {
                hipLaunchKernelGGL((rows_small_kernel<N, kBf16, false, true>), grid, block, 0, stream, sa);
            }
        } else {
            const dim3 block(small_waves<N, false>() * 64);
            if (bprep != nullptr) {
                hipLaunchKernelGGL((rows_small_kernel<N, kBf16, true, false>), grid, block, 0, stream, sa);
            } else {
                hipLaunchKernelGGL((rows_small_kernel<N, kBf16, false, false>), grid, block, 0, stream, sa);
            }
        }
    } else {
        // Without prepared weights the GEMM builds each stage's B from phi
        // and gamma itself (rowsBFromPhi) or reads fragments a prep launch
        // wrote to the workspace.
        u32x4_t *bfrag = reinterpret_cast<u32x4_t *>(ws + p.wsRowsB);
        const bool fromPhi = bprep == nullptr && p.rowsBFromPhi;
        if (bprep == nullptr && !fromPhi) {
            const int64_t prepThreads = (p.K / 32) * C::NA * kWave;
            hipLaunchKernelGGL((rows_prep_b_kernel<N>), dim3((unsigned)((prepThreads + 255) / 256)),
                               dim3(256), 0, stream, p.phi, p.hasGamma ? p.gamma : nullptr, bfrag, p.K,
                               status);
            err = hipGetLastError();
            if (err != hipSuccess) {
                return err;
            }
        }
        RowsGemmArgs g;
        g.x = static_cast<const uint16_t *>(p.x);
        g.bfrag = bprep != nullptr ? bprep : bfrag;
        g.phi = p.phi;
        g.gamma = p.hasGamma ? p.gamma : nullptr;
        g.partial = partial;
        g.rowStride = rowStride;
        g.rangeStride = rangeStride;
        g.T = p.T;
        g.K = p.K;
        g.NS = (int)(p.K / 32 / kStageKs);
        g.S = p.rowsS;
        g.rowBlocks = p.rowsBlocks;
        g.nXcd = nXcd;
        const int items = p.rowsBlocks * p.rowsS;
        g.perXcd = (items + nXcd - 1) / nXcd;
        if (!fromPhi) {
            hipLaunchKernelGGL((rows_gemm_kernel<N, kBf16, false>), dim3((unsigned)(g.perXcd * nXcd)),
                               dim3(kRW * 64), 0, stream, g);
        } else {
            hipLaunchKernelGGL((rows_gemm_kernel<N, kBf16, true>), dim3((unsigned)(g.perXcd * nXcd)),
                               dim3(kRW * 64), 0, stream, g);
        }
    }
    err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }

    RowsEpiArgs e;
    e.x = static_cast<const uint16_t *>(p.x);
    e.partial = partial;
    e.rowStride = rowStride;
    e.rangeStride = rangeStride;
    e.alpha = p.alpha;
    e.bias = p.bias;
    e.hIn = static_cast<uint16_t *>(p.hIn);
    e.hPost = p.hPost;
    e.hRes = p.hRes;
    e.hPre = p.hasHPre ? p.hPre : nullptr;
    e.T = p.T;
    e.D = p.D;
    e.S = p.rowsS;
    e.normEps = p.normEps;
    e.hcEps = p.hcEps;
    e.invFlatDim = p.invFlatDim;
    for (int64_t r0 = 0; r0 < p.T; r0 += kEpilogueRowsPerLaunch) {
        e.row0 = r0;
        const int64_t rows = std::min<int64_t>(kEpilogueRowsPerLaunch, p.T - r0);
        const bool wide = rows_epilogue_wide(N, p.rowsS, rows);
        // Fewer rows than a wave of workgroups (small batches): each row's
        // hIn is split over up to 8 workgroups of at least 128 column octets
        // each, so that more CUs share the x reads (each part sums the row's
        // partials itself; narrow rows gain nothing from a split).
        const int parts = (int)std::max<int64_t>(
            1, std::min<int64_t>(std::min<int64_t>(8, 256 / rows), p.D / 8 / 128));
        const dim3 grid((unsigned)rows, (unsigned)parts);
        if (wide) {
            hipLaunchKernelGGL((rows_epilogue_kernel<N, kBf16, 1024, 1>), grid, dim3(1024), 0, stream, e);
        } else {
            hipLaunchKernelGGL((rows_epilogue_kernel<N, kBf16, 256, 4>), grid, dim3(256), 0, stream, e);
        }
        err = hipGetLastError();
        if (err != hipSuccess) {
            return err;
        }
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_prepare_b(int n, const float *phi, const float *gamma, void *bfrag, int64_t K,
                            hipStream_t stream)
{
    int na = 0;
    switch (n) {
    case 4:
        na = RowsCols<4>::NA;
        break;
    case 6:
        na = RowsCols<6>::NA;
        break;
    case 8:
        na = RowsCols<8>::NA;
        break;
    default:
        return hipErrorInvalidValue;
    }
    const int64_t threads = (K / 32) * na * kWave;
    const dim3 grid((unsigned)((threads + 255) / 256));
    u32x4_t *dst = static_cast<u32x4_t *>(bfrag);
    if (n == 4) {
        hipLaunchKernelGGL((rows_prep_b_kernel<4>), grid, dim3(256), 0, stream, phi, gamma, dst, K,
                           static_cast<uint32_t *>(nullptr));
    } else if (n == 6) {
        hipLaunchKernelGGL((rows_prep_b_kernel<6>), grid, dim3(256), 0, stream, phi, gamma, dst, K,
                           static_cast<uint32_t *>(nullptr));
    } else {
        hipLaunchKernelGGL((rows_prep_b_kernel<8>), grid, dim3(256), 0, stream, phi, gamma, dst, K,
                           static_cast<uint32_t *>(nullptr));
    }
    return hipGetLastError();
}

// The epilogue's 1024-thread variant (12 groups of M + 1 threads at n = 8
// sum the K-range partials, one octet of x per thread) against the 256-thread
// one (3 groups, four octets per thread).  With few rows the partial sums are
// a large part of a row's work and more threads in flight win; from a few
// hundred rows on, x dominates and the 256-thread workgroups stream it faster.
// Measured on MI355X (us per launch back to back, 1024 / 256 threads): n = 8,
// D = 7168, T = 64 (224 K-ranges) 16.7 / 20.2; n = 8, D = 8192, T = 256 30.1 /
// 32.1; n = 4, D = 4096, T = 128 12.3 / 13.8; n = 6, D = 1024, T = 64 10.1 /
// 10.9; n = 4, D = 256, T = 128 (4 K-ranges) 12.4 / 11.8; n = 8, D = 8192,
// T = 512 43.7 / 43.1, T = 2048 129.1 / 123.1; n = 6, D = 4096, T = 512 28.9 /
// 26.2.  So: the 1024-thread variant for at most 256 rows when a 256-thread
// group would add at least 4 partials per column.
bool rows_epilogue_wide(int n, int S, int64_t rows)
{
    const int cols = n * n + 2 * n + 1;
    const int perGroup = (S + 256 / cols - 1) / (256 / cols);
    return rows <= 256 && perGroup >= 4;
}

int rows_block_rows() { return kRowBlock; }
int rows_gemm_threads() { return kRW * 64; }
int rows_small_rows(int n, bool wide)
{
    return (n == 4 ? small_rows<4>() : n == 6 ? small_rows<6>() : small_rows<8>()) * (wide ? 2 : 1);
}
int rows_small_ksteps() { return kSmallWaves * kSmallKs; }
int rows_stage_ksteps() { return kStageKs; }

hipError_t launch_rows(const Plan &p, void *workspace, int nXcd, hipStream_t stream)
{
    switch (p.n) {
    case 4:
        return p.isBf16 ? launch_rows_t<4, true>(p, workspace, nXcd, stream)
                        : launch_rows_t<4, false>(p, workspace, nXcd, stream);
    case 6:
        return p.isBf16 ? launch_rows_t<6, true>(p, workspace, nXcd, stream)
                        : launch_rows_t<6, false>(p, workspace, nXcd, stream);
    case 8:
        return p.isBf16 ? launch_rows_t<8, true>(p, workspace, nXcd, stream)
                        : launch_rows_t<8, false>(p, workspace, nXcd, stream);
    default:
        return hipErrorNotSupported;
    }
}

}  // namespace mhc
