// Strip kernel for gfx950 (n = 4, D % 32 == 0): x is read from HBM once,
// held in VGPRs in a ring of row tiles until its hIn is written, and the
// cross-workgroup exchange of the K-reduction runs in the shadow of the x
// stream.
//
// Teams.  The workgroups of one XCD form teams of P = ceil(D / 256) slice
// workgroups and R reducer workgroups (when D % 256 != 0, the lanes of the
// last slice whose columns lie past D load zeros and store nothing).  Workgroup g runs on XCD g mod X (the
// hardware dispatches workgroups round-robin over the X XCDs), so a team's
// exchange stays inside one XCD's L2.  Results do not depend on where a
// workgroup actually runs (one placed off its team's XCD writes through to
// memory); only the speed does.  Where P slices and two reducers do not fit
// one XCD, the host launches with X = 1: teams then span the device and
// every exchange store writes through to memory.  Team t owns row tiles t,
// t + numTeams, ... (16 rows each); its k-th tile is its "team step k".
//
// Slice workgroup p (8 waves, two per SIMD).  Wave w owns strip w mod 4, the
// 64 columns [256p + 64(w mod 4), +64) of every stream (256 values of K),
// and belongs to wave group w / 4; group g takes the team steps g, g + 2, ...
// (its "own steps"), so the two waves of a SIMD work on different tiles.  The
// B operand of each strip (gamma * phi split into bf16 hi + lo, 3 column
// tiles x 8 k-steps, 24 KB) is built once into LDS.  x of a tile is 16 rows
// x 4 streams x 64 columns = 8 KB per wave (32 VGPRs), loaded as whole
// 128-byte lines (register (s, h) holds, in lane l, row 8h + (l & 7) and the
// 8 columns at 8(l >> 4) + 32((l >> 3) & 1) of stream s) into a ring of L
// tiles.  Own step j of a wave:
//   1. hIn of own tile j - E from the ring, with hPre from the tile's
//      broadcast block, polled one own step earlier; the poll for the next
//      step; the hIn stores;
//   2. the MFMAs of own tile j against B (a DPP row_ror:8 turns a pair of
//      line registers into the A fragments of two k-steps) and a Gram MFMA
//      of the same fragments, whose diagonal is the sum of squares; after
//      each stream's MFMAs, the loads of that stream of own tile j - E + L go
//      out into the registers hIn freed;
//   3. the four strips' partials (M mix columns + sumsq, 16 rows) meet in LDS
//      and are summed in strip order into the slice's record, stored as
//      tagged words (below) in whole 128-byte lines.
// So L - E tiles are loading ahead of the MFMA while E tiles wait for hPre.
//
// Reducer workgroup r of a team takes the team steps r, r + R, ...: it polls
// the P records of the tile, sums them in slice order, evaluates invRms and
// hPre, publishes hPre as a broadcast block of tagged words, then writes the
// hPre, hPost and hRes outputs.
//
// Exchange words.  Every exchanged value is one 8-byte word: the fp32 bits in
// the low half and a tag in the high half, written and read as single-copy
// atomic accesses at device scope (sc1).  The tag is a hash of the word's
// position XOR a per-launch epoch, so a word holds the current value exactly
// when its tag matches: no arrival counter, no release wait, no reset of the
// workspace between launches.  The epoch is kept in the workspace header
// (epoch_load / epoch_mark / epoch_publish), so replays of a captured HIP graph get fresh
// epochs too.  Every wait is bounded by a spin limit; running out records
// kDeviceTimeout with the host launch id in the status word instead of
// hanging, and the rows the wave or workgroup could not finish get NaN
// outputs.  The grid is one workgroup per CU, all co-resident when nothing
// else occupies the device.

#include "mhc_pre_device.h"
#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>
#include <utility>

namespace mhc {
namespace {

using namespace dev;

constexpr int kGroups = 2;                   // wave groups per workgroup (waves per SIMD)
constexpr int kStrips = 4;                   // 64-column strips per slice
constexpr int kWaves = kGroups * kStrips;    // waves per workgroup
constexpr int kStripCols = 64;               // x columns of each stream per strip
constexpr int kSlice = kStrips * kStripCols; // columns per slice
constexpr int kRing = 5;                     // L: x tiles held per wave
constexpr int kLag = 3;                      // E: hIn of own tile j at own step j + E
static_assert(kLag < kRing, "ring geometry");
// Exchange ring: team step k uses record / broadcast slot k mod S, and the
// team has R reducers, R in {1, 2, 4} (reducer k mod R takes step k).  A
// slice of group h writes the record of step m (m = h mod 2) at the end of
// its own step m / 2, after its hIn of step m - 2E, that is after it has seen
// the broadcast block of step m - 2E.  That block's reducer publishes it
// after finishing (both phases of) its previous tile, step m - 2E - R, and
// every tile before.  The slot's previous occupant, step m - S, is among
// those when some step m - S + tR (t >= 1, tR even, so of the same group) is
// at most m - 2E: S = 2E + 4 does it for R = 1, 2 and 4.  The broadcast
// block of step m is written only after every slice has written the record
// of step m, hence after each has read the block of step m - S.
constexpr int kMaxReducers = 4;
constexpr int kRingSlots = 2 * kLag + kMaxReducers;
static_assert(kRingSlots >= (kLag + 1) * kGroups, "ring slots");
constexpr int kMaxSlices = 64;              // slice workgroups per team (the reducer loads are sized for it)
constexpr int kXccIdReg = (3 << 11) | 20;    // s_getreg operand: HW_REG_XCC_ID, bits [3:0]

struct StripArgs {
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
    uint64_t *recs;    // [team][ringSlots][P] records of Rec<N>::WORDS tagged words
    uint64_t *bcast;   // [team][ringSlots] blocks of Rec<N>::BWORDS tagged words
    char *hdr;         // workspace header: the status word ((launchId << 32) |
                       // kDeviceTimeout after a timeout) at 0, the exchange epoch
    uint32_t *statusWord;  // the caller's sticky status word, or null
    int64_t T;
    int64_t D;
    int64_t K;
    int64_t RT;
    int P;            // slice workgroups per team (ceil(D / 256))
    int R;            // reducer workgroups per team
    int nXcd;         // XCDs of the device
    int teamsPerXcd;  // teams formed from the workgroups of one XCD
    int numTeams;     // nXcd * teamsPerXcd
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
    static constexpr bool has_hi(int t) { return t < Q || t == 2 * Q; }
};

// Record of one (row tile, slice), column-major: column c holds its 16 rows
// as 16 consecutive tagged words (128 bytes).  Column N is the sum of
// squares; mix column j sits at column j (j < N, the hPre columns) or j + 1.
// The per-tile broadcast block holds hPre columns 0..N-1, 16 rows each.
template <int N>
struct Rec {
    static constexpr int M = N * N + 2 * N;
    static constexpr int COLS = M + 1;
    static constexpr int WORDS = COLS * 16;
    static constexpr int CHUNKS = WORDS / 2;  // 16-byte chunks
    static constexpr int BWORDS = N * 16;
    __device__ static int col(int j) { return j < N ? j : j + 1; }
};

// Word positions are uint32 and wrap modulo 2^32 for very large T.  That is
// harmless: a reader only ever finds, at a ring address, words of the same
// launch's earlier occupants of that slot, k * S * numTeams * (P * WORDS or
// BWORDS) positions apart (numTeams * P <= 256 CUs, so not a multiple of
// 2^32 for any k below 2^17, more slot reuses than T < 2^24 rows allow), or
// words of other launches (other epochs).
__device__ __forceinline__ uint32_t rec_tag(uint32_t pos, uint32_t epoch)
{
    return (pos * 0x9E3779B1u) ^ epoch;
}
__device__ __forceinline__ uint32_t bcast_tag(uint32_t pos, uint32_t epoch)
{
    return (pos * 0x85EBCA77u) ^ epoch ^ 0xC2B2AE3Du;
}

constexpr int kCpolNt = 2;    // nontemporal: x and hIn are streamed once
constexpr int kCpolDev = 16;  // sc1: device-scope coherent

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, 0x00020000);
}

// Every global access of the kernel is a buffer instruction, the exchange
// words and the status word included (aligned 8-byte accesses, performed as
// one access, sc1).  Atomics through generic pointers would compile to FLAT
// instructions, which count on both the vector-memory and the LDS counters:
// with one of them in flight, every later counter wait of the wave has to
// wait for zero, which drains the x ring at every step.
__device__ __forceinline__ uint64_t ld_word(__amdgpu_buffer_rsrc_t r, int off)
{
    return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCpolDev));
}
__device__ __forceinline__ void st_status(uint64_t *status, uint32_t launchId)
{
    const uint64_t v = ((uint64_t)launchId << 32) | kDeviceTimeout;
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned int, v),
                                          make_rsrc(status, 8), 0, 0, kCpolDev);
}

template <int kCpol>
__device__ __forceinline__ void store16(const u32x4_t &v, __amdgpu_buffer_rsrc_t r, int off)
{
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v), r, off, 0, kCpol);
}

__device__ __forceinline__ void record_timeout(const StripArgs &a, int lane)
{
    if (lane == 0) {
        st_status(reinterpret_cast<uint64_t *>(a.hdr), a.launchId);
        st_status_word(a.statusWord);
    }
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

// Workgroup barrier that orders LDS only.  __syncthreads() also makes every
// outstanding global load and store of the wave complete first.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Workgroup-wide AND of ok through LDS, with a barrier that orders LDS only
// (__syncthreads_and also waits for the workgroup's outstanding global
// stores).  The two halves of votes are used alternately: a wave writes one
// half again only after the barrier of the other half, which every wave
// reaches after reading this one.
__device__ __forceinline__ bool wg_all(bool ok, uint32_t *votes, uint32_t &parity)
{
    const int w = (int)(threadIdx.x >> 6);
    const bool waveOk = __all(ok) != 0;
    uint32_t *half = votes + parity * kWaves;
    parity ^= 1u;
    if ((threadIdx.x & 63) == 0) {
        half[w] = waveOk ? 1u : 0u;
    }
    const u32x4_t *v = reinterpret_cast<const u32x4_t *>(half);
    lds_barrier();
    const u32x4_t v0 = v[0];
    const u32x4_t v1 = v[1];
    return (v0[0] & v0[1] & v0[2] & v0[3] & v1[0] & v1[1] & v1[2] & v1[3]) != 0u;
}

// A fragments of k-steps 2q and 2q + 1 from the line-layout registers r0
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

// Reducer workgroup r of a team: the team's steps k = r, r + R, ..., one
// tile at a time with all its waves, in two phases.
//   Phase 1 reads record columns 0..N (the hPre mix columns and the sum of
//   squares): thread t takes item t % (8 (N+1)) (column item / 8, rows
//   2 (item % 8) and +1) and slice group t / (8 (N+1)), and sums the records
//   of slices sg, sg + SG1, ... in increasing order.  Every word read must
//   carry its tag; the whole workgroup retries until all do.  The groups are
//   then added in order in LDS, invRms and hPre are evaluated, and hPre is
//   published (the broadcast block).
//   Phase 2 then reads the hPost / hRes columns N+1 .. M the same way and
//   writes those outputs.
// Every sum has a fixed order.  The ring size (kRingSlots) keeps a slot from
// being rewritten before its reducer has finished both phases.
template <int N, int C0, int NC, int UMAX>
struct ColPoll {
    static constexpr int ITEMS = NC * 8;
    static constexpr int SG = (kWaves * 64) / ITEMS;
    static_assert(SG >= 1, "reducer layout");
    int c, r0, sg;
    bool act;
    u32x4_t t[UMAX];
    __device__ ColPoll(int tid)
    {
        const int item = tid % ITEMS;
        sg = tid / ITEMS;
        act = sg < SG;
        c = C0 + (item >> 3);
        r0 = 2 * (item & 7);
    }
    // Issues the loads of this thread's slices sg, sg + SG, ... (at most UMAX).
    __device__ void issue(__amdgpu_buffer_rsrc_t tr, int P)
    {
#pragma unroll
        for (int u = 0; u < UMAX; ++u) {
            const int q = sg + SG * u;
            t[u] = (act && q < P) ? __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                                    tr, ((q * Rec<N>::COLS + c) * 16 + r0) * 8, 0,
                                                                    kCpolDev))
                                  : u32x4_t{0u, 0u, 0u, 0u};
        }
    }
    // Sums the loaded words in slice order; false if a tag does not match.
    __device__ bool sum(uint32_t tileBase, uint32_t epoch, int P, float2 &acc) const
    {
        bool ok = true;
        acc = make_float2(0.f, 0.f);
#pragma unroll
        for (int u = 0; u < UMAX; ++u) {
            const int q = sg + SG * u;
            if (act && q < P) {
                const uint32_t pos = tileBase + (uint32_t)((q * Rec<N>::COLS + c) * 16 + r0);
                ok = ok && t[u][1] == rec_tag(pos, epoch) && t[u][3] == rec_tag(pos + 1u, epoch);
                acc.x = acc.x + __uint_as_float(t[u][0]);
                acc.y = acc.y + __uint_as_float(t[u][2]);
            }
        }
        return ok;
    }
};

template <int N, int MaxS>
__device__ __forceinline__ void reducer_wg(const StripArgs &a, int team, int ntiles, int r, int R,
                                           bool local, float *lds, uint32_t prevEpoch,
                                           uint32_t *epochSh)
{
    using RC = Rec<N>;
    constexpr int COLS = RC::COLS;
    constexpr int kSg1 = (kWaves * 64) / ((N + 1) * 8);
    constexpr int kSg2 = (kWaves * 64) / ((COLS - N - 1) * 8);
    using Poll1 = ColPoll<N, 0, N + 1, (MaxS + kSg1 - 1) / kSg1>;
    using Poll2 = ColPoll<N, N + 1, COLS - N - 1, (MaxS + kSg2 - 1) / kSg2>;
    constexpr int kSums = Poll1::SG * Poll1::ITEMS > Poll2::SG * Poll2::ITEMS ? Poll1::SG * Poll1::ITEMS
                                                                              : Poll2::SG * Poll2::ITEMS;
    float *sums = lds;                // [SG][ITEMS][2] of the current phase
    float *irs = lds + 2 * kSums;     // [16] invRms per row
    uint32_t *votes = reinterpret_cast<uint32_t *>(lds + 2 * kSums + 16);  // [2][kWaves]
    static_assert((2 * kSums + 16) % 4 == 0, "vote words 16-byte aligned");
    static_assert(kWaves == 8, "wg_all reads two 16-byte vote vectors");
    static_assert(8 * (N + 1) <= 64, "phase 1 is finished by one wave");
    uint32_t voteParity = 0;
    const int tid = threadIdx.x;
    const int P = a.P;
    // The launch's exchange epoch: read by thread 0 from the workspace header
    // (prevEpoch), handed to every wave through LDS.
    if (tid == 0) {
        *epochSh = epoch_next(prevEpoch);
        epoch_mark(a.hdr, kWsSeenOff, *epochSh, blockIdx.x);
    }
    lds_barrier();
    const uint32_t epoch = __builtin_amdgcn_readfirstlane(*epochSh);
    const float alphaPre = a.alpha[0];
    const float alphaPost = a.alpha[1];
    const float alphaRes = a.alpha[2];
    Poll1 p1(tid);
    Poll2 p2(tid);
    // The bias of this thread's column in each phase, loaded once.
    const float bias1 = a.bias[p1.c < N ? p1.c : 0];
    const float bias2 = a.bias[p2.c - 1];
    bool timedOut = false;
    for (int k = r; k < ntiles; k += R) {
        const int rt = team + a.numTeams * k;
        const uint32_t slot = (uint32_t)(team * kRingSlots + k % kRingSlots);
        const __amdgpu_buffer_rsrc_t tr = make_rsrc(a.recs + (uint64_t)slot * P * RC::WORDS, P * RC::WORDS * 8);
        const uint32_t tileBase = (uint32_t)rt * (uint32_t)P * (uint32_t)RC::WORDS;

        // Phase 1: hPre columns and sum of squares.  Once a wait of this
        // workgroup has expired, its rows get NaN outputs (and a NaN hPre
        // broadcast, so the slices' hIn of those rows is NaN too).
        float2 acc;
        bool got = false;  // every word of this tile's columns carried its tag
        for (uint32_t spins = 0;; ++spins) {
            p1.issue(tr, P);
            const bool ok = p1.sum(tileBase, epoch, P, acc);
            if (wg_all(ok, votes, voteParity)) {
                got = true;
                break;
            }
            if (timedOut) {
                break;  // an earlier wait expired: no more waiting in this launch
            }
            if (spins >= a.spinLimit) {
                record_timeout(a, tid);
                timedOut = true;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (!got) {
            acc = make_float2(poison(), poison());
        }
        if (p1.act) {
            sums[(p1.sg * Poll1::ITEMS + tid % Poll1::ITEMS) * 2] = acc.x;
            sums[(p1.sg * Poll1::ITEMS + tid % Poll1::ITEMS) * 2 + 1] = acc.y;
        }
        lds_barrier();
        // Wave 0 finishes phase 1 (its lanes 0 .. 8(N+1)-1 are the items):
        // the groups' sums in order, invRms in the lanes of column N (lane
        // 8N + i has rows 2i, 2i + 1), handed to the hPre lanes of the same
        // rows by a shuffle and to phase 2 through LDS (read after the next
        // barrier).
        if (tid < 64) {
            float2 gs[Poll1::SG];
#pragma unroll
            for (int g = 0; g < Poll1::SG; ++g) {
                gs[g] = tid < Poll1::ITEMS ? *reinterpret_cast<const float2 *>(&sums[(g * Poll1::ITEMS + tid) * 2])
                                           : make_float2(0.f, 0.f);
            }
            float2 tot = make_float2(0.f, 0.f);
#pragma unroll
            for (int g = 0; g < Poll1::SG; ++g) {
                tot.x = tot.x + gs[g].x;
                tot.y = tot.y + gs[g].y;
            }
            float ir2[2] = {0.f, 0.f};
            if (tid < Poll1::ITEMS && p1.c == N) {  // sum of squares: invRms of rows r0, r0 + 1
                ir2[0] = ref_inv_rms(tot.x, a.invFlatDim, a.normEps);
                ir2[1] = ref_inv_rms(tot.y, a.invFlatDim, a.normEps);
                irs[p1.r0] = ir2[0];
                irs[p1.r0 + 1] = ir2[1];
            }
            ir2[0] = __shfl(ir2[0], 8 * N + (tid & 7));
            ir2[1] = __shfl(ir2[1], 8 * N + (tid & 7));
            if (tid < Poll1::ITEMS && p1.c < N) {
            // hPre column c: broadcast words (rows r0, r0 + 1) and the
            // optional hPre output.
            const int c = p1.c;
            u32x4_t wv;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float ir = ir2[e];
                const float mix = e == 0 ? tot.x : tot.y;
                const float v = ref_sigmoid(mix * (ir * alphaPre), bias1, a.hcEps);
                const int idx = c * 16 + p1.r0 + e;
                wv[2 * e] = __float_as_uint(v);
                wv[2 * e + 1] = bcast_tag((uint32_t)rt * (uint32_t)RC::BWORDS + (uint32_t)idx, epoch);
                const int row = rt * 16 + p1.r0 + e;
                if (a.hPre != nullptr && row < a.T) {
                    a.hPre[(int64_t)row * N + c] = v;
                }
            }
            const __amdgpu_buffer_rsrc_t br = make_rsrc(a.bcast + (uint64_t)slot * RC::BWORDS, RC::BWORDS * 8);
            if (local) {
                store16<0>(wv, br, (c * 16 + p1.r0) * 8);
            } else {
                store16<kCpolDev>(wv, br, (c * 16 + p1.r0) * 8);
            }
            }
        }

        // Phase 2: hPost / hRes columns.
        got = false;
        for (uint32_t spins = 0;; ++spins) {
            p2.issue(tr, P);
            const bool ok = p2.sum(tileBase, epoch, P, acc);
            if (wg_all(ok, votes, voteParity)) {
                got = true;
                break;
            }
            if (timedOut) {
                break;
            }
            if (spins >= a.spinLimit) {
                record_timeout(a, tid);
                timedOut = true;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (!got) {
            acc = make_float2(poison(), poison());
        }
        if (p2.act) {
            sums[(p2.sg * Poll2::ITEMS + tid % Poll2::ITEMS) * 2] = acc.x;
            sums[(p2.sg * Poll2::ITEMS + tid % Poll2::ITEMS) * 2 + 1] = acc.y;
        }
        lds_barrier();
        if (tid < Poll2::ITEMS) {
            float2 gs[Poll2::SG];
#pragma unroll
            for (int g = 0; g < Poll2::SG; ++g) {
                gs[g] = *reinterpret_cast<const float2 *>(&sums[(g * Poll2::ITEMS + tid) * 2]);
            }
            float2 tot = make_float2(0.f, 0.f);
#pragma unroll
            for (int g = 0; g < Poll2::SG; ++g) {
                tot.x = tot.x + gs[g].x;
                tot.y = tot.y + gs[g].y;
            }
            // Mix column j = c - 1 (N .. M-1): hPost or hRes.
            const int jj = p2.c - 1;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int row = rt * 16 + p2.r0 + e;
                const float v = e == 0 ? tot.x : tot.y;
                const float ir = irs[p2.r0 + e];
                if (row < a.T) {
                    if (jj < 2 * N) {
                        const float sgm = ref_sigmoid(v * (ir * alphaPost), bias2, 0.0f);
                        a.hPost[(int64_t)row * N + (jj - N)] = sgm * 2.0f;
                    } else {
                        const float rr = v * (ir * alphaRes);
                        a.hRes[(int64_t)row * (N * N) + (jj - 2 * N)] = rr + bias2;
                    }
                }
            }
        }
        lds_barrier();  // sums / irs are reused by the next tile
    }
}

template <int N, bool kBf16, bool kPrep>
__global__ __launch_bounds__(kWaves * 64) void strip_kernel(StripArgs a)
{
    using S = Shape<N>;
    constexpr int M = S::M;
    constexpr int NT = S::NT;
    using CL = ColLayout<M>;
    using RC = Rec<N>;
    constexpr int Q = CL::Q;
    constexpr int L = kRing;
    constexpr int E = kLag;
    constexpr int KS = 2 * N;  // 32-column k-steps per strip (two per stream)
    static_assert(N == 4, "the strip path is built for n = 4");
    // Partials of the four strips of each group, double-buffered by own step:
    // column c of a strip's partial at c * kColPitch floats.  The pitch (20,
    // not 16) puts the 16-byte writes of 8 consecutive lanes (consecutive
    // columns) on distinct LDS banks.
    constexpr int kColPitch = 20;
    __shared__ __attribute__((aligned(16))) float part[kGroups][2][kStrips][RC::COLS * kColPitch];
    // B operand of each strip, in MFMA fragment order (24 KB per strip).
    __shared__ u32x4_t bsh[kStrips][KS][NT][64];
    // Second staging area of the B build (rows of 256 values of K padded to
    // kStagePitch bytes, hi then lo).
    constexpr int kStagePitch = kSlice * 2 + 16;
    __shared__ __attribute__((aligned(16))) char stage2[kPrep ? 16 : 2 * M * kStagePitch];
    // Per-group count of partials written (4 per own step).
    __shared__ uint32_t arrived[kGroups];
    // The launch's exchange epoch, handed from thread 0 to every wave.
    __shared__ uint32_t epochSh;

    const int tid = threadIdx.x;
    // Thread 0 reads the epoch the previous launch on this workspace left; the
    // load is waited for only where the epoch is first needed.
    const uint32_t prevEpoch = tid == 0 ? epoch_load(a.hdr, kWsEpochOff) : 0u;
    const int g = blockIdx.x;
    const int xcd = g % a.nXcd;
    const int j = g / a.nXcd;
    const int teamSize = a.P + a.R;
    const int tj = j / teamSize;
    if (tj >= a.teamsPerXcd) {
        // Spare workgroup: the whole workgroup leaves together.
        if (tid == 0) {
            epoch_mark(a.hdr, kWsSeenOff, epoch_next(prevEpoch), g);
        }
        return;
    }
    const int team = xcd + a.nXcd * tj;
    const int role = j % teamSize;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) wave index
    const int64_t numTeams = a.numTeams;
    const int64_t ntiles = team < a.RT ? (a.RT - team + numTeams - 1) / numTeams : 0;
    // Exchange stores stay in this XCD's L2 (plain stores, which the readers'
    // device-scope loads see there) when the workgroup runs on the XCD its
    // team belongs to; a workgroup placed on another XCD writes through to
    // memory (sc1).  The hardware dispatches workgroup g to XCD g mod X, so
    // in practice every store is local.
    const bool local = a.nXcd > 1 && (int)(__builtin_amdgcn_s_getreg(kXccIdReg) & 15) == xcd;

    if (role >= a.P) {
        // A reducer instance whose unrolled record loads cover the team and
        // little more: every poll round runs all of them, predicated, and the
        // round is on the team's critical path (sized for 64 slices, the
        // reducers of 30-slice teams ran 13% slower, MI355X, D = 7680, T =
        // 8192).
        float *lds = &part[0][0][0][0];
        const int rr = role - a.P;
        if (a.P <= 8) {
            reducer_wg<N, 8>(a, team, (int)ntiles, rr, a.R, local, lds, prevEpoch, &epochSh);
        } else if (a.P <= 16) {
            reducer_wg<N, 16>(a, team, (int)ntiles, rr, a.R, local, lds, prevEpoch, &epochSh);
        } else if (a.P <= 32) {
            reducer_wg<N, 32>(a, team, (int)ntiles, rr, a.R, local, lds, prevEpoch, &epochSh);
        } else {
            reducer_wg<N, kMaxSlices>(a, team, (int)ntiles, rr, a.R, local, lds, prevEpoch, &epochSh);
        }
        return;
    }

    // ---- slice workgroup ----
    // Wave w: strip w % 4 of the slice, group w / 4.  Group g takes the
    // team's steps k = g, g + G, g + 2G, ... (its own steps jj = 0, 1, ...),
    // so the G waves on a SIMD work on different tiles and one computes while
    // the others wait for the memory queue.
    const int p = role;
    const int strip = w & 3;
    const int half = w >> 2;  // the wave's group
    const int Ki = (int)a.K;
    const int Di = (int)a.D;
    const int col0 = p * kSlice + strip * kStripCols;
    // A strip past D (the last slice when D % 256 != 0) holds no columns:
    // its x reads zeros through size-0 resources, its B is zero and it
    // stores no hIn, so it adds nothing to the slice's partial sums.
    const bool stripLive = col0 < Di;
    const int lrow = lane & 7;
    const int lineOff = 8 * (lane >> 4) + 32 * ((lane >> 3) & 1);
    // A lane whose 8 columns lie past D (the last slice when D % 64 != 0)
    // loads and stores nothing: its offsets are past every resource's end.
    constexpr int kPastEnd = 0x40000000;
    const bool colLive = col0 + lineOff < Di;
    const int xLane = colLive ? (lrow * Ki + col0 + lineOff) * 2 : kPastEnd;
    const int hLane = colLive ? (lrow * Di + col0 + lineOff) * 2 : kPastEnd;
    const int rl = lane & 15;
    const int grp = lane >> 4;
    if (tid < kGroups) {
        arrived[tid] = 0;
    }
    if (ntiles == 0) {
        if (tid == 0) {
            epoch_mark(a.hdr, kWsSeenOff, epoch_next(prevEpoch), g);
        }
        return;
    }
    // 32-bit tile and row indices (the launch validates T < 2^31 / 16);
    // byte offsets of a tile are formed in 64 bits from them.
    const int T32 = (int)a.T;
    // The kernel arguments the loop uses, as independent scalars: the
    // compiler otherwise keeps the argument block as one 16-register tuple
    // and spills and reloads it whole.
    const char *xBase = reinterpret_cast<const char *>(a.x);
    char *hBase = reinterpret_cast<char *>(a.hIn);
    uint64_t *recsBase = a.recs;
    uint64_t *bcastBase = a.bcast;
    uint64_t *statusW = reinterpret_cast<uint64_t *>(a.hdr);
    int P32 = a.P;
    uint32_t spinLimit = a.spinLimit;
    uint32_t launchId = a.launchId;
    asm volatile("" : "+s"(xBase), "+s"(hBase), "+s"(recsBase), "+s"(bcastBase), "+s"(statusW),
                 "+s"(P32), "+s"(spinLimit), "+s"(launchId));
    const int nt32 = (int)ntiles;
    const int nmine = (nt32 - half + kGroups - 1) / kGroups;
    const int teamI = team;
    const int nTeams = (int)numTeams;
    const uint32_t xTileBytes = 16u * (uint32_t)Ki * 2u;
    const uint32_t hTileBytes = 16u * (uint32_t)Di * 2u;
    // Team tile of own step jj, and its valid rows (0 past the last one).
    auto tile_of = [&](int jj) { return teamI + nTeams * (kGroups * jj + half); };
    auto rows_of = [&](int jj) {
        return (jj >= 0 && jj < nmine) ? min(16, T32 - tile_of(jj) * 16) : 0;
    };
    auto x_tile = [&](int jj) {
        return xBase + (uint64_t)(uint32_t)tile_of(jj) * xTileBytes;
    };
    auto h_tile = [&](int jj) {
        return hBase + (uint64_t)(uint32_t)tile_of(jj) * hTileBytes;
    };

    // x of a tile goes through a buffer resource based at the tile's first
    // row and sized to its valid rows: loads past T (or of a step past the
    // last tile, size 0) read zero without touching memory.  The whole
    // offset is in the VGPR operand, which the range check covers.
    u32x4_t xb[L][N][2];
#pragma unroll
    for (int b = 0; b < L; ++b) {
#pragma unroll
        for (int s = 0; s < N; ++s) {
            xb[b][s][0] = u32x4_t{0u, 0u, 0u, 0u};
            xb[b][s][1] = u32x4_t{0u, 0u, 0u, 0u};
        }
    }
    // B operand of each strip, in LDS for the whole launch: fragment (ks, ct)
    // holds, for lane l, B[k = s*D + col0 + 32q + 8(l/16) + e][slot 16ct +
    // l%16], e = 0..7, with ks = 2s + q.  All of a wave's weight loads are
    // issued before their first use, so the build costs one memory round
    // trip; the first x tiles are loaded behind them.
    u32x4_t (*bfr)[NT][64] = bsh[strip];
    constexpr int KW = KS / kGroups;  // k-steps copied per wave (prepared weights)
    // Without prepared weights, wave w loads mix columns CPW w .. CPW w +
    // CPW - 1 of phi: for each stream one 1 KB run of a column (the slice's
    // 256 values of K, lane l holding 4 consecutive ones), and gamma of the
    // same runs; they become fragments through LDS below.  (Loads in
    // fragment order touch 16 columns x 64 bytes each; at n = 4, D = 4096,
    // T = 1024 a launch took 22.4 us with those and 21.5 us with the runs.)
    constexpr int CPW = M / kWaves;
    static_assert(M % kWaves == 0, "mix columns per wave");
    const bool hasGamma = a.gamma != nullptr;
    f32x4_t pv[N][CPW];
    f32x4_t gv[N];
    // Prepared weights (kPrep): the fragments already have this layout; k-step
    // ks of the strip is the prepared k-step (s D + col0 + 32 q) / 32, and the
    // G waves of a strip share its k-steps (the wave of group g copies ks =
    // g, g + G, ...); they are copied into LDS below, behind the x loads.
    u32x4_t pf[kPrep ? KW : 1][kPrep ? NT : 1];
    if constexpr (kPrep) {
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            const int ks = half + kGroups * i;
            const int64_t gks = ((int64_t)(ks >> 1) * a.D + col0 + 32 * (ks & 1)) / 32;
            const bool ksLive = col0 + 32 * (ks & 1) < Di;  // the k-step's 32 columns are within D
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                pf[i][t] = ksLive ? a.bprep[(gks * NT + t) * 64 + lane] : u32x4_t{0u, 0u, 0u, 0u};
            }
        }
    } else {
        const __amdgpu_buffer_rsrc_t phiR = make_rsrc(a.phi, M * Ki * 4);
        const __amdgpu_buffer_rsrc_t gamR = make_rsrc(a.gamma, hasGamma ? Ki * 4 : 0);
        // Lanes whose 4 values of K lie past D read zeros (offsets past the
        // resources' ends).
        const bool laneLive = p * kSlice + 4 * lane < Di;
#pragma unroll
        for (int s = 0; s < N; ++s) {
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                pv[s][c] = __builtin_bit_cast(
                    f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                 phiR, laneLive ? ((CPW * w + c) * Ki + s * Di + p * kSlice) * 4 + 16 * lane : M * Ki * 4,
                                 0, 0));
            }
            gv[s] = __builtin_bit_cast(
                f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             gamR, laneLive ? (s * Di + p * kSlice) * 4 + 16 * lane : Ki * 4, 0, 0));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // Every wave's weight loads are in the CU's memory queue before any
    // wave's x loads.  A wave stalls at a load while the queue is full, and
    // with each wave's loads in program order, the last waves' weights came
    // in behind the other waves' first tiles and held the B build (and every
    // step after it).
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // The ring: slot jj mod L holds own tile jj; tiles 0 .. L-E-1 are loaded
    // before the first step, and step jj loads tile jj - E + L.  The first
    // tiles' loads go out in four parts (tile 0 streams 0-1, tile 0 streams
    // 2-3, then tile 1's), so that a wave stalled at a full memory queue
    // holds back no more of the B build than one part: with prepared weights
    // all here, without them one part after each stream's rows are staged
    // in the B build below (measured at n = 4, D = 7168, T = 8192: the
    // barrier above ~0.5 us faster per launch, the four parts ~0.7 us more).
    auto load_x_part = [&](auto pc) __attribute__((always_inline)) {
        constexpr int part = decltype(pc)::value;
        constexpr int b = part / 2;
        const __amdgpu_buffer_rsrc_t r = make_rsrc(x_tile(b), stripLive ? rows_of(b) * Ki * 2 : 0);
#pragma unroll
        for (int s = 2 * (part % 2); s < 2 * (part % 2) + 2; ++s) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                xb[b][s][h] = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, xLane + (8 * h * Ki + s * Di) * 2,
                                                                   0, kCpolNt));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    static_assert(L - E == 2 && N == 4, "the first tiles' loads go out in four parts");
    if constexpr (kPrep) {
        static_for<4>(load_x_part);
    }
    if constexpr (kPrep) {
#pragma unroll
        for (int i = 0; i < KW; ++i) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                bfr[half + kGroups * i][t][lane] = pf[i][t];
            }
        }
    } else {
        // One round per stream s, through two staging areas used in turn
        // (the partials buffer, idle until the first step, and stage2): each
        // wave writes its columns' products gamma * phi as bf16 hi and lo
        // rows (row j: the slice's 256 values of K, padded to kStagePitch
        // bytes so that the 8 lanes of a read phase hit distinct banks), then
        // builds 3 of the stream's 24 fragments (4 strips x 2 k-steps x NT
        // tiles) from them.  Round s + 1's rows are written while round s's
        // fragments are read, so the rounds take one barrier each.
        static_assert(2 * M * kStagePitch <= (int)sizeof(part), "staging fits the partials buffer");
        static_assert(kStrips * 2 * NT == 3 * kWaves, "fragments per wave and round");
        char *const areas[2] = {reinterpret_cast<char *>(&part[0][0][0][0]), stage2};
        auto write_rows = [&](int s) __attribute__((always_inline)) {
            char *stHi = areas[s & 1];
            char *stLo = stHi + M * kStagePitch;
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                float bv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    bv[e] = pv[s][c][e];
                    if (hasGamma) {
                        bv[e] = bv[e] * gv[s][e];
                    }
                }
                uint32_t h0, l0, h1, l1;  // bf16(B) and bf16(B - hi), k pairs (4l, 4l+1), (4l+2, 4l+3)
                split2_bf16(bv[0], bv[1], h0, l0);
                split2_bf16(bv[2], bv[3], h1, l1);
                const int off = (CPW * w + c) * kStagePitch + 8 * lane;
                *reinterpret_cast<uint2 *>(stHi + off) = make_uint2(h0, h1);
                *reinterpret_cast<uint2 *>(stLo + off) = make_uint2(l0, l1);
            }
        };
        write_rows(0);
        __builtin_amdgcn_sched_barrier(0);
        load_x_part(std::integral_constant<int, 0>{});
        lds_barrier();
#pragma unroll
        for (int s = 0; s < N; ++s) {
            if (s + 1 < N) {
                write_rows(s + 1);  // the other area: its last reader was round s - 1
                __builtin_amdgcn_sched_barrier(0);
                static_for<3>([&](auto pc) __attribute__((always_inline)) {
                    if (decltype(pc)::value == s) {
                        load_x_part(std::integral_constant<int, decltype(pc)::value + 1>{});
                    }
                });
            }
            const char *stHi = areas[s & 1];
            const char *stLo = stHi + M * kStagePitch;
#pragma unroll
            for (int f0 = 0; f0 < 3; ++f0) {
                const int f = 3 * w + f0;  // (strip, q, t) = (f / (2 NT), (f / NT) % 2, f % NT)
                const int fs = f / (2 * NT);
                const int fq = (f / NT) % 2;
                const int ft = f % NT;
                bool lo;
                int jc;
                CL::slot(16 * ft + rl, lo, jc);
                const int k = 64 * fs + 32 * fq + 8 * grp;
                bsh[fs][2 * s + fq][ft][lane] =
                    *reinterpret_cast<const u32x4_t *>((lo ? stLo : stHi) + jc * kStagePitch + 2 * k);
            }
            if (s + 1 < N) {
                lds_barrier();  // round s + 1's rows written, round s's area free again
            }
        }
    }
    if (tid == 0) {
        epochSh = epoch_next(prevEpoch);
        epoch_mark(a.hdr, kWsSeenOff, epochSh, g);
    }
    lds_barrier();
    const uint32_t epoch = __builtin_amdgcn_readfirstlane(epochSh);

    // Every step of the main loop issues the same memory operations in the
    // same order (two hIn stores, one broadcast poll, eight x loads, one
    // record store per lane), whatever the step: out-of-range tiles go
    // through size-0 resources and polls of out-of-range tiles re-read the
    // team's first block and are ignored.  With no data-dependent branch
    // around a memory operation, the compiler's wait counts stay exact and no
    // wait drains the ring.  The poll of step jj serves the hIn of step
    // jj + 1; the x loads and the record store of step jj are behind it.
    // The drain steps, past the last tile, only write hIn.
    uint64_t pr[L];  // broadcast polls: slot j mod L for own tile j's hIn
#pragma unroll
    for (int b = 0; b < L; ++b) {
        pr[b] = 0;
    }
    const __amdgpu_buffer_rsrc_t bcastAll =
        make_rsrc(bcastBase, a.numTeams * kRingSlots * RC::BWORDS * 8);
    // Exchange ring slot of own step jj (team step G jj + group).
    auto slot_of = [&](int jj) { return teamI * kRingSlots + (kGroups * jj + half) % kRingSlots; };
    bool timedOut = false;

    // Meeting count of the other group once it has run all its steps (the
    // meetings are in the steps with a tile, own steps 0 .. nmine - 1).
    const int nmineOther = (nt32 - (half ^ 1) + kGroups - 1) / kGroups;
    const uint32_t otherCount = 4u * (uint32_t)nmineOther;

    // One step of the pipeline: own step j0 + b, ring slot b mod L (a
    // compile-time constant in every copy of the body).  A drain step (kFull
    // false: own steps nmine .. nmine + E - 1, which have no tile of their
    // own) runs part 1 only, the hIn of own tile jj - E.
    auto step = [&](int j0, auto bc, auto fullc) __attribute__((always_inline)) {
        constexpr int b = decltype(bc)::value;
        constexpr bool kFull = decltype(fullc)::value;
        static_assert(!kFull || b < L, "a step with a tile uses ring slot b");
        // The step index is recomputed from an opaque copy, so that the
        // per-step addresses are derived in each step rather than
        // precomputed for all L unrolled steps and held in registers.
        int jj = j0 + b;
        asm volatile("" : "+s"(jj));
        const int rt = tile_of(jj);
        const int jh = jj - E;
        const int hb = (b - E + 2 * L) % L;  // ring slot of own tile jh (static after unrolling)
        static_assert(b - E + 2 * L >= 0, "ring slot");
        const bool liveH = jh >= 0 && jh < nmine;
        const int rth = tile_of(jh);

        // 1. hIn of own tile jh = jj - E from ring slot hb, with hPre
        //    from the poll issued in the previous step (first the
        //    fast path: the poll already carries every tag).
        uint64_t wv = pr[hb];
        const uint32_t want = bcast_tag((uint32_t)rth * (uint32_t)RC::BWORDS + (uint32_t)lane, epoch);
        if (liveH && !timedOut && !__all((uint32_t)(wv >> 32) == want)) {
            const int blkOff = (slot_of(jh) * RC::BWORDS + lane) * 8;
            for (uint32_t spins = 0;; ++spins) {
                __builtin_amdgcn_s_sleep(1);
                wv = ld_word(bcastAll, blkOff);
                if (__all((uint32_t)(wv >> 32) == want)) {
                    break;
                }
                if (spins >= spinLimit) {
                    if (lane == 0) {
                        st_status(statusW, launchId);
                    }
                    timedOut = true;
                    break;
                }
            }
        }
        // Lane l holds hPre column l/16 of row l%16.  Once a wait of this
        // wave has expired its hPre is taken as NaN, so the hIn of those
        // rows is NaN rather than a value from a missing broadcast.
        const float preC = timedOut ? poison() : __uint_as_float((uint32_t)wv);
        float pre[2][N];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int s = 0; s < N; ++s) {
                pre[h][s] = __shfl(preC, 16 * s + 8 * h + lrow);
            }
        }
        u32x4_t hout[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float hv[8];
#pragma unroll
            for (int s = 0; s < N; ++s) {
                float f[8];
                unpack8<kBf16>(xb[hb][s][h], f);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float prod = pre[h][s] * f[e];
                    hv[e] = (s == 0) ? prod : hv[e] + prod;
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                hout[h][q] = pack2_x<kBf16>(hv[2 * q], hv[2 * q + 1]);
            }
        }
        //    Poll for the hIn of the next step (own tile jh + 1; the
        //    team's first tile when that does not exist), issued before
        //    the hIn stores so that the next step's wait for it does not
        //    also wait for them.
        {
            const int jp = jh + 1;
            const int jpc = (jp >= 0 && jp < nmine) ? jp : 0;
            pr[(hb + 1) % L] = __builtin_bit_cast(
                uint64_t, __builtin_amdgcn_raw_buffer_load_b64(
                              bcastAll, (slot_of(jpc) * RC::BWORDS + lane) * 8, 0, kCpolDev));
        }
        {
            const __amdgpu_buffer_rsrc_t hr = make_rsrc(h_tile(jh), liveH && stripLive ? rows_of(jh) * Di * 2 : 0);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                store16<kCpolNt>(hout[h], hr, hLane + 8 * h * Di * 2);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!kFull) {
            return;
        }
        // Ring slot of own tile jj (drain copies, with b >= L, return above;
        // the clamp keeps their discarded remainder in bounds).
        constexpr int bx = b < L ? b : 0;

        // 2. GEMM of own tile jj (zeros past the last tile) and its Gram
        //    matrix, one stream at a time; after each stream's MFMAs the
        //    two loads of that stream of own tile jh + L go out into the
        //    slot hIn just consumed.  This part runs at raised wave
        //    priority: of the two waves on a SIMD, the one issuing its
        //    next tiles' loads goes first, which keeps the CU's memory
        //    queue fuller (measured at n = 4, D = 7168, T = 8192,
        //    interleaved on two MI355X boxes: 108.5 -> 108.0 and 108.0 ->
        //    107.4 us per launch; the hIn part raised instead: +0.7 us).
        __builtin_amdgcn_s_setprio(1);
        const int jn = jh + L;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(x_tile(jn), stripLive ? rows_of(jn) * Ki * 2 : 0);
        f32x4_t acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        f32x4_t gram = f32x4_t{0.f, 0.f, 0.f, 0.f};
        // B fragments come from LDS, those of the next k-step read while
        // this k-step's MFMAs run.
        u32x4_t bcur[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            bcur[t] = bfr[0][t][lane];
        }
#pragma unroll
        for (int s = 0; s < N; ++s) {
            u32x4_t kf[2];
            lines_to_frags(xb[bx][s][0], xb[bx][s][1], kf[0], kf[1]);
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int ks = 2 * s + q;
                u32x4_t bnext[NT];
                if (ks + 1 < KS) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        bnext[t] = bfr[ks + 1][t][lane];
                    }
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
                if (ks + 1 < KS) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        bcur[t] = bnext[t];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                xb[hb][s][h] = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                 xr, xLane + (8 * h * Ki + s * Di) * 2, 0, kCpolNt));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // Gram diagonal: row r sits in lane 16(r/4) + r, register r % 4.
        const int di = rl & 3;
        const float ss = di == 0 ? gram[0] : di == 1 ? gram[1] : di == 2 ? gram[2] : gram[3];

        __builtin_amdgcn_s_setprio(0);
        // 3. This wave's partials into LDS, [column][row]: the C fragment
        //    gives lane (rl, grp) rows 4grp .. 4grp+3 of column slot 16t + rl.
        float *mine = &part[half][jj & 1][strip][0];
#pragma unroll
        for (int t = 0; t < Q; ++t) {
            const f32x4_t v = acc[t] + acc[Q + t];
            *reinterpret_cast<f32x4_t *>(mine + RC::col(16 * t + rl) * kColPitch + 4 * grp) = v;
        }
        if constexpr (CL::kHalfTile) {
            f32x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[i] = __shfl_xor(acc[2 * Q][i], 8);
            }
            if (rl < 8) {
                *reinterpret_cast<f32x4_t *>(mine + RC::col(16 * Q + rl) * kColPitch + 4 * grp) =
                    acc[2 * Q] + o;
            }
        }
        if ((rl >> 2) == grp) {
            mine[N * kColPitch + rl] = ss;
        }
        //    The four strips of this group meet through an LDS counter
        //    (the other group keeps running): each adds one after its
        //    partials, then waits for 4 (jj + 1).  A strip writes this
        //    buffer again two steps later, after the next meeting, by
        //    which time every strip has read it.  The wait also holds a
        //    group that is a step ahead of the other (count below 4 jj):
        //    the SIMDs favour the older waves, and a group left to run
        //    ahead finishes early and leaves the other to run the last
        //    steps alone.  The wait for the other group is capped at
        //    its final count, so it always ends.
        {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (lane == 0) {  // one count per wave
                __hip_atomic_fetch_add(&arrived[half], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            const uint32_t target = 4u * (uint32_t)(jj + 1);
            const uint32_t otherTarget = min(target - 4u, otherCount);
            while (__hip_atomic_load(&arrived[half], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target ||
                   __hip_atomic_load(&arrived[half ^ 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <
                       otherTarget) {
                __builtin_amdgcn_s_sleep(1);
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
        // 4. The slice's record: 16-byte chunk c2 = 64 strip + lane
        //    (column c2/8, rows 2(c2%8), +1), the four strips summed in
        //    strip order; 8 lanes fill one column's 128-byte line.  Lanes
        //    past the record and steps past the last tile store out of
        //    range (dropped).
        {
            const int c2 = strip * 64 + lane;
            const int ch = c2 < RC::CHUNKS ? c2 : 0;
            const int c = ch >> 3;
            const int r0 = 2 * (ch & 7);
            const float *pb = &part[half][jj & 1][0][0];
            float2 v = *reinterpret_cast<const float2 *>(pb + c * kColPitch + r0);
#pragma unroll
            for (int st = 1; st < kStrips; ++st) {
                const float2 u =
                    *reinterpret_cast<const float2 *>(pb + st * RC::COLS * kColPitch + c * kColPitch + r0);
                v.x = v.x + u.x;
                v.y = v.y + u.y;
            }
            const uint32_t pos = ((uint32_t)rt * (uint32_t)P32 + (uint32_t)p) * (uint32_t)RC::WORDS +
                                 (uint32_t)(c * 16 + r0);
            u32x4_t recw;
            recw[0] = __float_as_uint(v.x);
            recw[1] = rec_tag(pos, epoch);
            recw[2] = __float_as_uint(v.y);
            recw[3] = rec_tag(pos + 1u, epoch);
            const __amdgpu_buffer_rsrc_t rr = make_rsrc(
                recsBase + ((uint64_t)(uint32_t)slot_of(jj) * (uint32_t)P32 + (uint32_t)p) * RC::WORDS,
                jj < nmine ? RC::WORDS * 8 : 0);
            const int off = c2 < RC::CHUNKS ? 16 * c2 : RC::WORDS * 8;
            if (local) {
                store16<0>(recw, rr, off);
            } else {
                store16<kCpolDev>(recw, rr, off);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // Whole rounds of L steps with a tile; then a separate copy of the body
    // (so that its branches do not reach the main loop) for the last, partial
    // round of steps with a tile (fewer than L) and the E drain steps.
    using Full = std::integral_constant<bool, true>;
    using Drain = std::integral_constant<bool, false>;
    int j0 = 0;
    for (; j0 + L <= nmine; j0 += L) {
        static_for<L>([&](auto bc) __attribute__((always_inline)) { step(j0, bc, Full{}); });
    }
    static_for<L + E - 1>([&](auto bc) __attribute__((always_inline)) {
        constexpr int b = decltype(bc)::value;
        if (j0 + b < nmine) {
            if constexpr (b < L) {
                step(j0, bc, Full{});
            }
        } else if (j0 + b < nmine + E) {
            step(j0, bc, Drain{});
        }
    });
    // A wave whose wait expired also marks the caller's status word, once,
    // outside the loop.
    if (timedOut && lane == 0) {
        st_status_word(a.statusWord);
    }
    // Workgroup 0 (always a slice workgroup of team 0) advances the
    // workspace's epoch once every workgroup has taken this one.
    if (g == 0 && w == 0) {
        if (!epoch_publish(a.hdr, kWsEpochOff, kWsSeenOff, epoch, (int)gridDim.x, spinLimit) &&
            lane == 0) {
            st_status(statusW, launchId);
            st_status_word(a.statusWord);
        }
    }
}

template <int N, bool kBf16, bool kPrep>
int strip_coresident_t(int numCUs)
{
    int perCU = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &perCU, reinterpret_cast<const void *>(&strip_kernel<N, kBf16, kPrep>), kWaves * 64, 0) !=
        hipSuccess) {
        return -1;
    }
    return perCU * numCUs;
}

template <int N, bool kBf16, bool kPrep>
hipError_t launch_strip_t(const Plan &p, void *workspace, uint32_t launchId, hipStream_t stream)
{
    char *ws = static_cast<char *>(workspace);
    StripArgs a;
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
    a.hdr = ws;
    a.statusWord = p.statusWord;
    a.bcast = reinterpret_cast<uint64_t *>(ws + p.wsStripBcast);
    a.recs = reinterpret_cast<uint64_t *>(ws + p.wsStripRecs);
    a.T = p.T;
    a.D = p.D;
    a.K = p.K;
    a.RT = p.fusedTiles;
    a.P = p.stripP;
    a.R = p.stripR;
    a.nXcd = p.stripXcds;
    a.teamsPerXcd = p.stripTeamsPerXcd;
    a.numTeams = p.stripXcds * p.stripTeamsPerXcd;
    a.normEps = p.normEps;
    a.hcEps = p.hcEps;
    a.invFlatDim = p.invFlatDim;
    a.launchId = launchId;
    a.spinLimit = p.spinLimit;
    if (!p.fusedCooperative) {
        hipLaunchKernelGGL((strip_kernel<N, kBf16, kPrep>), dim3((unsigned)p.stripGrid), dim3(kWaves * 64), 0,
                           stream, a);
        return hipGetLastError();
    }
    // Cooperative launch (MHCPRE_LAUNCH=cooperative): co-residency of the
    // whole grid is guaranteed even next to concurrent work.
    void *args[] = {&a};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&strip_kernel<N, kBf16, kPrep>),
                                      dim3((unsigned)p.stripGrid), dim3(kWaves * 64), args, 0,
                                      stream);
}

}  // namespace

hipError_t launch_strip(const Plan &p, void *workspace, uint32_t launchId, hipStream_t stream)
{
    if (p.n != 4) {
        return hipErrorNotSupported;
    }
    if (p.bprep != nullptr) {
        return p.isBf16 ? launch_strip_t<4, true, true>(p, workspace, launchId, stream)
                        : launch_strip_t<4, false, true>(p, workspace, launchId, stream);
    }
    return p.isBf16 ? launch_strip_t<4, true, false>(p, workspace, launchId, stream)
                    : launch_strip_t<4, false, false>(p, workspace, launchId, stream);
}

int strip_ring_slots() { return kRingSlots; }

int strip_record_words() { return Rec<4>::WORDS; }

int strip_bcast_words() { return Rec<4>::BWORDS; }

int strip_teams_per_xcd(int P, int cusPerXcd)
{
    // Teams of two or more slices get at least two reducers; a single-slice
    // team keeps one, which leaves room for more teams.
    int t = cusPerXcd / (P + (P >= 2 ? 2 : 1));
    if (t < 1) {
        t = cusPerXcd / (P + 1);
    }
    return t;
}

int strip_max_slices() { return kMaxSlices; }

int strip_reducers(int available)
{
    return available >= 4 ? 4 : available >= 2 ? 2 : available;
}

int strip_max_coresident(const Plan &p, int numCUs)
{
    if (p.n != 4) {
        return -1;
    }
    if (p.bprep != nullptr) {
        return p.isBf16 ? strip_coresident_t<4, true, true>(numCUs)
                        : strip_coresident_t<4, false, true>(numCUs);
    }
    return p.isBf16 ? strip_coresident_t<4, true, false>(numCUs)
                    : strip_coresident_t<4, false, false>(numCUs);
}

}  // namespace mhc
