// Internal launch plan shared by the host library and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace mhc {

// Kernel paths an executor can launch.
enum class Path : int {
    kSplit = 0,   // prep B, split-K MFMA GEMM + sumsq partials, epilogue + hIn (x read twice)
    kFused = 1,   // one persistent kernel: x read once, kept in registers
    kStrip = 2,   // one persistent kernel: XCD-local teams, B in LDS, x in a register ring
    kRows = 3,    // prep B, split-K GEMM over 256-row blocks (B through an LDS ring), epilogue + hIn
};

// Device status word (first 8 bytes of the workspace): the low half holds a
// code, the high half the host launch id of the launch that wrote it.  The
// strip and fused kernels write (launch id, kDeviceTimeout) only when a wait
// runs out; the split path's first kernel writes kDeviceOk into the low half.
constexpr uint32_t kDeviceOk = 0u;
constexpr uint32_t kDeviceTimeout = 0x7107u;

// Bytes reserved at the head of the workspace: the status word at 0, and the
// exchange epoch of the strip and fused kernels.  The epoch lives in device
// memory, not in the kernel arguments, so that a launch captured in a HIP
// graph still gets a fresh epoch on every replay: every workgroup reads the
// word at kWsEpochOff, uses one more than it and records the epoch it uses in
// its own slot of the array at kWsSeenOff; workgroup 0, at its end, stores
// the new epoch once every slot of the grid holds it (no workgroup reads the
// word after that).
constexpr size_t kWsEpochOff = 64;            // uint32: epoch of the latest strip / fused launch
constexpr size_t kWsSeenOff = 256;            // uint32 [kMaxEpochGrid]: epoch each workgroup uses
constexpr int kMaxEpochGrid = 2048;           // largest strip / fused grid
constexpr size_t kWsHeaderBytes = kWsSeenOff + 4 * kMaxEpochGrid;

struct Plan {
    Path path = Path::kSplit;

    // Problem shape.
    int n = 0;        // streams
    int M = 0;        // n*n + 2n
    int NT = 0;       // 16-wide column tiles of the [hi | lo] B operand: 2M / 16
    int64_t T = 0;    // rows (tokens)
    int64_t D = 0;    // per-stream width
    int64_t K = 0;    // n * D
    bool isBf16 = true;
    bool hasGamma = false;
    bool hasHPre = false;
    // Strip and fused path launch.  By default a plain launch of a grid sized
    // to the device's co-residency limit: every workgroup is resident as long
    // as no other kernel occupies the device, and the kernels' bounded waits
    // turn any other case into a reported timeout rather than a hang.
    // MHCPRE_LAUNCH=cooperative selects a cooperative launch, which
    // guarantees co-residency next to concurrent work at the cost of a
    // slower dispatch (about 20 us per launch on MI355X).
    bool fusedCooperative = false;
    // Polls of a strip or fused wait before it records kDeviceTimeout and
    // gives up (about a second).  MHCPRE_SPIN_LIMIT at phase 1 overrides it,
    // for tests of the timeout path.
    uint32_t spinLimit = 1u << 20;
    float normEps = 1e-6f;
    float hcEps = 1e-6f;
    float invFlatDim = 0.f;  // fl(1.0f / K), as code/op_host/mhc_pre.cpp:154

    // Split path: K-slices of the GEMM and k-steps (32 wide) per slice.
    int splitS = 1;
    int ksPerSlice = 0;

    // Fused path parameters (fusedGrid / fusedTeams are filled per launch
    // from the device's co-residency limit).
    int fusedDw = 0;          // x columns per slice (32 * k-steps)
    int fusedP = 0;           // slices per row tile = D / fusedDw
    int fusedGrid = 0;        // workgroups in the cooperative grid
    int fusedTeams = 0;       // teams of fusedP workgroups
    int64_t fusedTiles = 0;   // 16-row tiles

    // Strip path (n = 4, D % 32 == 0 from D = 192): P = ceil(D / 256) slice
    // workgroups of 256 columns and R reducer workgroups per team, teams
    // formed inside one XCD or across the device.  stripR, stripXcds,
    // stripTeamsPerXcd and stripGrid are filled per launch from the device.
    int stripP = 0;
    int stripMaxTeams = 0;  // teams the workspace's exchange rings are sized for (those of the
                            // device phase 1 planned for)
    int stripR = 0;
    int stripXcds = 0;
    int stripTeamsPerXcd = 0;
    int stripGrid = 0;

    // Rows path (K % 128 == 0): rowsS K-ranges (contiguous runs of
    // rows_stage_ksteps()-k-step stages) over rowsBlocks blocks of
    // rows_block_rows() rows.
    int rowsS = 0;
    int rowsBlocks = 0;
    // The block GEMM builds B from phi and gamma itself (no prep launch);
    // otherwise a prep kernel writes B fragments to the workspace first.
    bool rowsBFromPhi = false;
    // Small batches (T <= rows_small_rows(n, false), or up to twice that with
    // K >= 16384): one GEMM workgroup per K-range of rows_small_ksteps()
    // k-steps, B built from phi by the workgroup itself, no prep launch.
    bool rowsSmall = false;
    // Partial sums stored row-major, [T][rowsS][M+1] (each row's sums
    // contiguous for its epilogue), instead of [rowsS][T][M+1].
    bool rowsRowMajor = false;

    // Workspace layout (byte offsets).  The paths' regions overlap: a
    // workspace holds one launch at a time.
    size_t wsBsplit = 0;      // split: B fragments
    size_t wsPartial = 0;     // split: [S][T][M+1] partials
    size_t wsFinal = 0;       // fused: per-tile hPre / invRms blocks (tagged words)
    size_t wsFusedPartial = 0;// fused: per-(tile, slice) exchange records (tagged words)
    size_t wsFusedEnd = 0;    // fused: end of its layout (0: no fused layout)
    size_t wsSplitEnd = 0;    // split: end of its layout
    size_t wsStripBcast = 0;  // strip: per-team rings of broadcast blocks (tagged words)
    size_t wsStripRecs = 0;   // strip: per-team rings of P exchange records (tagged words)
    size_t wsRowsB = 0;       // rows (prep launch): B fragments [K/32][NT][64 lanes] x 16 bytes
    size_t wsRowsPartial = 0; // rows: partials, [rowsS][T][M+1] or [T][rowsS][M+1]
    size_t wsTotal = 0;

    // Bound device pointers (caller memory).
    uint32_t *statusWord = nullptr;  // strip / fused launches: the caller's sticky status word
    const void *x = nullptr;
    const float *phi = nullptr;
    const float *alpha = nullptr;
    const float *bias = nullptr;
    const float *gamma = nullptr;
    void *hIn = nullptr;
    float *hPost = nullptr;
    float *hRes = nullptr;
    float *hPre = nullptr;
    // Prepared B operand (mhcPrePrepareWeights), or null: the kernels then
    // build B from phi and gamma.  Layout of launch_prepare_b.
    const void *bprep = nullptr;
};

// Built-in workspace of mhcPreNoAlloc (mhc_pre_noalloc.hip): kScratchBytes
// per device, in the library's device code object.  scratch_address gives the
// current device's copy (the caller makes `device` current).
constexpr size_t kScratchBytes = size_t{64} << 20;
hipError_t scratch_address(int device, void **ptr);

// Kernel launchers (mhc_pre_kernels.hip).  Each returns the first HIP error.
hipError_t launch_split(const Plan &plan, void *workspace, hipStream_t stream);
// launchId: host-side id of the launch, written with kDeviceTimeout into the
// status word when a bounded wait expires (the exchange epoch itself comes
// from the workspace header).
hipError_t launch_fused(const Plan &plan, void *workspace, uint32_t launchId, hipStream_t stream);

hipError_t launch_strip(const Plan &plan, void *workspace, uint32_t launchId, hipStream_t stream);

// Prepared B operand (mhc_pre_rows.hip): B = gamma (.) phi (gamma may be
// null) split into bf16 hi + lo MFMA fragments, [K/32 k-steps][2M/16 column
// tiles][64 lanes] x 16 bytes.  Lane l of fragment (ks, t) holds k = 32 ks +
// 8 (l / 16) .. + 7 of one column: tile t < Q = M/16 the hi half of column
// 16 t + l % 16, tile Q + t the lo half of the same column; when M % 16 == 8
// tile 2Q holds column 16 Q + l % 8, hi in lanes l % 16 < 8 and lo in the
// others.  The strip and fused kernels keep B in LDS in this same column
// order, and the rows path's GEMM reads it as it is.
hipError_t launch_prepare_b(int n, const float *phi, const float *gamma, void *bfrag, int64_t K,
                            hipStream_t stream);

// Rows path (mhc_pre_rows.hip); nXcd: XCDs of the device (work placement
// only).
hipError_t launch_rows(const Plan &plan, void *workspace, int nXcd, hipStream_t stream);
// Row blocks up to which the block GEMM builds B from phi itself (see
// mhc_pre_rows.hip); above it a prep launch writes B fragments first.
constexpr int64_t kRowsPhiMaxBlocks = 16;
// Whether the rows-path epilogue of `rows` rows over S K-ranges runs its
// 1024-thread variant (mhc_pre_rows.hip).
bool rows_epilogue_wide(int n, int S, int64_t rows);
// Rows per work item, k-steps per stage and work-items per workgroup of the
// rows-path GEMM.
int rows_block_rows();
int rows_stage_ksteps();
int rows_gemm_threads();
// Largest batch of the small-batch GEMM and k-steps per workgroup there.
// Rows the small-batch GEMM holds (the wide variant: twice as many).
int rows_small_rows(int n, bool wide);
int rows_small_ksteps();

// Stream probe (mhc_pre_stream.hip): reads readBytes (a multiple of 4096) from
// src and writes writeBytes (a multiple of 1024) to dst in the best-served
// access pattern, with `workgroups` workgroups of 512 threads.
hipError_t launch_stream_probe(const void *src, int64_t readBytes, void *dst, int64_t writeBytes,
                               int workgroups, hipStream_t stream);

// Workgroups of the strip kernel that can be resident per CU (x numCUs), or
// -1 if the plan has no strip kernel.
int strip_max_coresident(const Plan &plan, int numCUs);

// Exchange ring slots per team of the strip kernel, and the tagged 8-byte
// words of one exchange record (per slice) and of one broadcast block.
int strip_ring_slots();
int strip_record_words();
int strip_bcast_words();
// Teams of P slices (plus their reducers) that cusPerXcd CUs of one XCD
// hold; 0 when not even one fits.
int strip_teams_per_xcd(int P, int cusPerXcd);
// Largest number of slice workgroups per team the strip kernel supports.
int strip_max_slices();
// Reducer workgroups per team the strip kernel uses when `available` (>= 1)
// workgroups per team are left over after the slices (1, 2 or 4; the ring
// size depends on it).
int strip_reducers(int available);

// Rows per launch of the one-workgroup-per-row epilogue kernels (rows and
// split paths): a grid's work-items must stay below 2^32, so larger batches
// take several launches.
constexpr int64_t kEpilogueRowsPerLaunch = int64_t{1} << 20;

// Largest number of fused-path workgroups that can be co-resident on a device
// with numCUs compute units, or -1 if the plan has no fused kernel.
int fused_max_coresident(const Plan &plan, int numCUs);

// Fused-path workspace geometry for n streams, in 8-byte tagged words: one
// exchange record of M + 1 columns x 16 rows per (row tile, slice), and one
// broadcast block of n + 1 columns x 16 rows per row tile.
inline int fused_record_words(int n) { return (n * n + 2 * n + 1) * 16; }
inline int fused_bcast_words(int n) { return (n + 1) * 16; }

}  // namespace mhc
