// MhcPre host library: validation, launch plan, workspace sizing and launch.
//
// Mirrors the reference host op (code/op_host/mhc_pre.cpp): the acceptance
// rules of TilingFunc (:57-79,126-130), the output shapes and types of
// InferShape / InferDataType (:217-257), the attribute defaults (:297-298) and
// the gamma-presence rule (:90).  The Ascend tiling (row partition over 48 AIV
// cores, Cube M64 tiling, UB budgeting) has no counterpart: the GPU plan is a
// grid shape and a workspace layout.  Unlike the reference's process-global
// tiling cache (:36-51,99-121), nothing here is shared between calls, so
// concurrent phase-1 calls are safe.

#include "mhc_pre.h"
#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <map>
#include <tuple>
#include <unordered_map>

// Prepared weights: B = gamma (.) phi as bf16 hi + lo MFMA fragments in a
// caller-owned device buffer (layout of mhc::launch_prepare_b).
struct mhcPreWeights {
    int n = 0;
    int M = 0;
    int64_t K = 0;
    void *buffer = nullptr;
    uint64_t version = 0;
    int device = -1;  // device holding the buffer (-1: unknown)
};

namespace {

// Prepared buffers in use: the (n, K) layout each holds and how many weights
// handles and executors refer to it.  Preparing a buffer again with another
// layout while any of them lives would make them read fragments in the wrong
// order, so it is refused; once none is left the buffer is free again.
struct BufferLayout {
    int n;
    int64_t K;
    int refs;
};
std::mutex g_buffersMu;
std::unordered_map<const void *, BufferLayout> g_buffers;

bool buffer_acquire(const void *buffer, int n, int64_t K)
{
    std::lock_guard<std::mutex> lock(g_buffersMu);
    auto it = g_buffers.find(buffer);
    if (it == g_buffers.end()) {
        g_buffers.emplace(buffer, BufferLayout{n, K, 1});
        return true;
    }
    if (it->second.n != n || it->second.K != K) {
        return false;
    }
    ++it->second.refs;
    return true;
}

void buffer_release(const void *buffer)
{
    std::lock_guard<std::mutex> lock(g_buffersMu);
    auto it = g_buffers.find(buffer);
    if (it != g_buffers.end() && --it->second.refs <= 0) {
        g_buffers.erase(it);
    }
}

}  // namespace

struct mhcPreExecutor {
    mhc::Plan plan;
    // Device that holds x (-1: the runtime could not tell, e.g. no device is
    // visible at phase 1); launches must have it current.
    int device = -1;
    // Host id of this executor's latest launch; the device status word only
    // reports a timeout written under it.
    std::atomic<uint32_t> lastLaunchId{0};
    // Workgroups of the strip / fused kernel the device holds at once
    // (occupancy query, made once per executor: at phase 1 when the current
    // device holds x, else at the first launch); -2 until known.
    std::atomic<int> stripCoresident{-2};
    std::atomic<int> fusedCoresident{-2};
    // The caller's sticky device status word (mhcPreExecutorSetStatusWord),
    // or null.
    std::atomic<uint32_t *> statusWord{nullptr};
    // Prepared-weights buffer this executor reads (registered), or null.
    const void *preparedBuffer = nullptr;
};

namespace {

// Largest row count (B*S) and per-stream width D a launch plan accepts: the
// split path's GEMM grid has T/16 workgroups of 256 work-items in its x
// dimension, which must stay below 2^32; D <= 2^24 keeps K = n*D and every
// byte offset formed from T and K far inside 64 bits.
constexpr int64_t kMaxRows = int64_t{1} << 28;
constexpr int64_t kMaxWidth = int64_t{1} << 24;

// Product of the dims, or -1 if it does not fit in 62 bits (a tensor that
// large fits no device); 0 if a dim is 0.  Negative dims give a negative or
// meaningless product, which every caller rejects with dims_positive.
int64_t numel(const mhcTensor &t)
{
    int64_t n = 1;
    for (int i = 0; i < t.ndim; ++i) {
        if (__builtin_mul_overflow(n, t.dims[i], &n) || n > (int64_t{1} << 62)) {
            return -1;
        }
    }
    return n;
}

bool dims_positive(const mhcTensor &t)
{
    if (t.ndim < 0 || t.ndim > MHC_MAX_DIMS) {
        return false;
    }
    for (int i = 0; i < t.ndim; ++i) {
        if (t.dims[i] <= 0) {
            return false;
        }
    }
    return true;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Compute units and XCDs of the current device, cached per device.
struct DeviceShape {
    int cus = 0;
    int xcds = 0;
};

// CUs and XCDs of `device` (cached per device).
bool device_shape_of(int device, DeviceShape &out)
{
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static DeviceShape cache[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) {
        return false;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (cache[device].cus == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) !=
                hipSuccess ||
            cus <= 0) {
            return false;
        }
        int xcds = 0;
        if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, device) != hipSuccess ||
            xcds <= 0 || cus % xcds != 0) {
            (void)hipGetLastError();
            xcds = 1;
        }
        cache[device].cus = cus;
        cache[device].xcds = xcds;
    }
    out = cache[device];
    return true;
}

// The current device and its shape.
bool device_shape(int &device, DeviceShape &out)
{
    if (hipGetDevice(&device) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return device_shape_of(device, out);
}

// MI355X: 256 CUs in 8 XCDs.  Phase 1 plans a strip executor's exchange rings
// for the device that holds x, or for this shape when the runtime cannot
// tell which device that is.
constexpr DeviceShape kPlanShapeDefault{256, 8};

// Where the strip kernel's teams live on a device: inside each XCD (the
// exchange then stays in the XCD's L2), or across the whole device, its CUs
// taken as one group (the kernel then stores its exchange words through to
// memory, device scope), with four reducers per team.  The x stream's rate
// follows the number of CUs that hold slices, so the teams go across XCDs
// where that puts at least 15% more CUs on slices, or where a team with two
// reducers does not fit an XCD.  Measured on MI355X (bf16, gamma, back to
// back, us, in an XCD / across XCDs): T = 8192: D = 2048 (8 slices) 38.1 /
// 44.4, 2304 (9) 50.2 / 47.4, 2560 (10) 56.5 / 55.3, 3328 (13) 55.1 / 61.0,
// 4096 (16) 89.9 / 72.5, 5120 (20) 99.8 / 92.4, 5632 (22) 101.6 / 99.9,
// 6144 (24) 99.9 / 103.3, 7168 (28) 105.7 / 117.3, 7680 (30) 116.3 / 129.9;
// T = 1024: D = 2560 14.7 / 15.2, 4096 19.2 / 17.6, 6144 20.6 / 20.7.
// Across XCDs, four reducers even where two would leave room for one more
// team (T = 8192, two / four: D = 10240 (40 slices) 214.7 / 180.7 us, D =
// 12288 (48) 269.7 / 221.0 us).
struct StripGeometry {
    int groups;    // XCDs, or 1
    int perGroup;  // CUs of a group
    int teams;     // teams per group
};
StripGeometry strip_geometry(int P, const DeviceShape &s)
{
    const int perXcd = s.cus / s.xcds;
    if (s.xcds == 1) {
        return {1, s.cus, mhc::strip_teams_per_xcd(P, s.cus)};
    }
    const int teamsLocal = P + 2 <= perXcd ? mhc::strip_teams_per_xcd(P, perXcd) : 0;
    const int teamsAcross = s.cus / (P + 4);
    if (teamsLocal > 0 && teamsAcross * 100 < teamsLocal * s.xcds * 115) {
        return {s.xcds, perXcd, teamsLocal};
    }
    return {1, s.cus, teamsAcross >= 1 ? teamsAcross : mhc::strip_teams_per_xcd(P, s.cus)};
}

// Phase-1 knobs for tests and measurement sweeps (MHCPRE_FORCE_PATH,
// MHCPRE_SPIN_LIMIT, MHCPRE_ROWS_B, MHCPRE_ROWS_PARTIALS) are read only when
// MHCPRE_TESTING=1: a stray one in a production environment changes nothing.
const char *test_env(const char *name)
{
    const char *gate = std::getenv("MHCPRE_TESTING");
    if (gate == nullptr || std::strcmp(gate, "1") != 0) {
        return nullptr;
    }
    return std::getenv(name);
}

// Device that holds the device memory at `p`, or -1 when the runtime cannot
// tell (host memory, an address no allocation covers, no device visible).
int device_of(const void *p)
{
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    return attr.type == hipMemoryTypeDevice ? attr.device : -1;
}

// Launch ids (written into the status word with a timeout): process-wide,
// strictly increasing from a start that differs between processes (time and
// address mixed), skipping 0 and ~0.
uint32_t next_launch_id()
{
    static std::atomic<uint32_t> counter{[] {
        const uint64_t t = static_cast<uint64_t>(
            std::chrono::high_resolution_clock::now().time_since_epoch().count());
        const uint64_t a = reinterpret_cast<uintptr_t>(&counter);
        uint64_t h = (t ^ (a << 17)) * 0x9E3779B97F4A7C15ull;
        return static_cast<uint32_t>(h >> 32);
    }()};
    for (;;) {
        const uint32_t e = counter.fetch_add(1u, std::memory_order_relaxed);
        if (e != 0u && e != 0xFFFFFFFFu) {
            return e;
        }
    }
}

// Trailing dims of `t` must be `tail` and its element count `count`.
bool shape_matches(const mhcTensor &t, int64_t count, const int64_t *tail, int ntail)
{
    if (!dims_positive(t) || t.ndim < ntail || numel(t) != count) {
        return false;
    }
    for (int i = 0; i < ntail; ++i) {
        if (t.dims[t.ndim - ntail + i] != tail[i]) {
            return false;
        }
    }
    return true;
}

// Phase-1 plan cache (the reference caches its tiling per shape,
// code/op_host/mhc_pre.cpp:36-51,99-121, in an unlocked global): the plan of
// a shape, without its tensor pointers, keyed by everything the plan depends
// on, under a lock.  The test knobs bypass it (MHCPRE_TESTING=1).
struct PlanKey {
    int64_t T;
    int64_t D;
    int n;
    int xdtype;
    int device;
    uint32_t normEps;
    uint32_t hcEps;
    bool hasGamma;
    bool hasHPre;
    bool cooperative;
    bool operator==(const PlanKey &o) const
    {
        return T == o.T && D == o.D && n == o.n && xdtype == o.xdtype && device == o.device &&
               normEps == o.normEps && hcEps == o.hcEps && hasGamma == o.hasGamma &&
               hasHPre == o.hasHPre && cooperative == o.cooperative;
    }
};
struct PlanKeyHash {
    size_t operator()(const PlanKey &k) const
    {
        uint64_t h = 0x9E3779B97F4A7C15ull;
        const uint64_t parts[] = {static_cast<uint64_t>(k.T), static_cast<uint64_t>(k.D),
                                  static_cast<uint64_t>(k.n) | (static_cast<uint64_t>(k.xdtype) << 8) |
                                      (static_cast<uint64_t>(static_cast<uint32_t>(k.device)) << 16),
                                  (static_cast<uint64_t>(k.normEps) << 32) | k.hcEps,
                                  static_cast<uint64_t>(k.hasGamma) | (static_cast<uint64_t>(k.hasHPre) << 1) |
                                      (static_cast<uint64_t>(k.cooperative) << 2)};
        for (uint64_t v : parts) {
            h = (h ^ v) * 0xBF58476D1CE4E5B9ull;
            h ^= h >> 31;
        }
        return static_cast<size_t>(h);
    }
};
constexpr size_t kPlanCacheEntries = 1024;  // cleared when full

std::mutex &plan_cache_mutex()
{
    static std::mutex mu;
    return mu;
}
std::unordered_map<PlanKey, mhc::Plan, PlanKeyHash> &plan_cache()
{
    static std::unordered_map<PlanKey, mhc::Plan, PlanKeyHash> cache;
    return cache;
}

bool testing_knobs() { return test_env("MHCPRE_TESTING") != nullptr; }

int validate_and_plan(const mhcTensor *x, const mhcTensor *phi, const mhcTensor *alpha,
                      const mhcTensor *bias, const mhcTensor *gamma, float normEps, float hcEps,
                      const mhcTensor *hIn, const mhcTensor *hPost, const mhcTensor *hRes,
                      const mhcTensor *hPre, mhc::Plan &p)
{
    if (x == nullptr || phi == nullptr || alpha == nullptr || bias == nullptr || hIn == nullptr ||
        hPost == nullptr || hRes == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    // x must be 4-D [B, S, n, D] (code/op_host/mhc_pre.cpp:67-70); 3-D [T, n, D]
    // is accepted as an extension.
    if (x->ndim != 4 && x->ndim != 3) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    int64_t T = 1;
    for (int i = 0; i + 2 < x->ndim; ++i) {
        if (x->dims[i] <= 0) {
            return MHC_STATUS_INVALID_SHAPE;
        }
        if (__builtin_mul_overflow(T, x->dims[i], &T) || T >= kMaxRows) {
            return MHC_STATUS_UNSUPPORTED_SHAPE;
        }
    }
    const int64_t n64 = x->dims[x->ndim - 2];
    const int64_t D = x->dims[x->ndim - 1];
    if (D <= 0) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    if (D > kMaxWidth) {
        return MHC_STATUS_UNSUPPORTED_SHAPE;
    }
    // Supported stream counts and alignments (code/op_host/mhc_pre.cpp:76-79,126-128).
    if (n64 != 4 && n64 != 6 && n64 != 8) {
        return MHC_STATUS_UNSUPPORTED_SHAPE;
    }
    const int n = static_cast<int>(n64);
    const int64_t K = n64 * D;
    const int M = n * n + 2 * n;
    if (M > 80 || (K % 8) != 0 || (D % 16) != 0) {
        return MHC_STATUS_UNSUPPORTED_SHAPE;
    }

    // Types (code/op_host/mhc_pre.cpp:265-296; InferDataType :251-257).
    if (x->dtype != MHC_DTYPE_FLOAT16 && x->dtype != MHC_DTYPE_BF16) {
        return MHC_STATUS_INVALID_DTYPE;
    }
    const bool hasGamma = gamma != nullptr && numel(*gamma) > 0 && gamma->ndim > 0;
    if (phi->dtype != MHC_DTYPE_FLOAT || alpha->dtype != MHC_DTYPE_FLOAT ||
        bias->dtype != MHC_DTYPE_FLOAT || hPost->dtype != MHC_DTYPE_FLOAT ||
        hRes->dtype != MHC_DTYPE_FLOAT || hIn->dtype != x->dtype ||
        (hasGamma && gamma->dtype != MHC_DTYPE_FLOAT) ||
        (hPre != nullptr && hPre->dtype != MHC_DTYPE_FLOAT)) {
        return MHC_STATUS_INVALID_DTYPE;
    }

    // Element counts.  The reference never checks these (only x is
    // shape-checked); reading past a short phi would be silent there.
    if (!dims_positive(*phi) || numel(*phi) != K * M || !dims_positive(*alpha) ||
        numel(*alpha) != 3 || !dims_positive(*bias) || numel(*bias) != M) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    if (hasGamma && (!dims_positive(*gamma) || numel(*gamma) != K)) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    // Output shapes as InferShape: hIn [.., D], hPost [.., n], hRes [.., n, n].
    const int64_t tailD[1] = {D};
    const int64_t tailN[1] = {n64};
    const int64_t tailNN[2] = {n64, n64};
    if (!shape_matches(*hIn, T * D, tailD, 1) || !shape_matches(*hPost, T * n64, tailN, 1) ||
        !shape_matches(*hRes, T * n64 * n64, tailNN, 2) ||
        (hPre != nullptr && !shape_matches(*hPre, T * n64, tailN, 1))) {
        return MHC_STATUS_INVALID_SHAPE;
    }

    // Device addresses.
    if (x->data == nullptr || phi->data == nullptr || alpha->data == nullptr ||
        bias->data == nullptr || hIn->data == nullptr || hPost->data == nullptr ||
        hRes->data == nullptr || (hasGamma && gamma->data == nullptr) ||
        (hPre != nullptr && hPre->data == nullptr)) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (!aligned(x->data, 16) || !aligned(hIn->data, 16) || !aligned(phi->data, 16) ||
        (hasGamma && !aligned(gamma->data, 16)) || !aligned(alpha->data, 4) ||
        !aligned(bias->data, 4) || !aligned(hPost->data, 4) || !aligned(hRes->data, 4) ||
        (hPre != nullptr && !aligned(hPre->data, 4))) {
        return MHC_STATUS_MISALIGNED;
    }

    p = mhc::Plan{};
    p.n = n;
    p.M = M;
    p.NT = (2 * M) / 16;
    p.T = T;
    p.D = D;
    p.K = K;
    p.isBf16 = x->dtype == MHC_DTYPE_BF16;
    p.hasGamma = hasGamma;
    p.hasHPre = hPre != nullptr;
    p.normEps = normEps;
    p.hcEps = hcEps;
    p.invFlatDim = 1.0f / static_cast<float>(K);
    p.x = x->data;
    p.phi = static_cast<const float *>(phi->data);
    p.alpha = static_cast<const float *>(alpha->data);
    p.bias = static_cast<const float *>(bias->data);
    p.gamma = hasGamma ? static_cast<const float *>(gamma->data) : nullptr;
    p.hIn = hIn->data;
    p.hPost = static_cast<float *>(hPost->data);
    p.hRes = static_cast<float *>(hRes->data);
    p.hPre = hPre != nullptr ? static_cast<float *>(hPre->data) : nullptr;

    // A cached plan of the same shape: the tensor pointers are this call's.
    const int planDevice = device_of(p.x);
    const char *launchEnv = std::getenv("MHCPRE_LAUNCH");
    PlanKey key{T, D, n, x->dtype, planDevice, 0u, 0u, hasGamma, hPre != nullptr,
                launchEnv != nullptr && std::strcmp(launchEnv, "cooperative") == 0};
    std::memcpy(&key.normEps, &normEps, 4);
    std::memcpy(&key.hcEps, &hcEps, 4);
    const bool useCache = !testing_knobs();
    if (useCache) {
        std::lock_guard<std::mutex> lock(plan_cache_mutex());
        const auto it = plan_cache().find(key);
        if (it != plan_cache().end()) {
            const mhc::Plan bound = p;
            p = it->second;
            p.x = bound.x;
            p.phi = bound.phi;
            p.alpha = bound.alpha;
            p.bias = bound.bias;
            p.gamma = bound.gamma;
            p.hIn = bound.hIn;
            p.hPost = bound.hPost;
            p.hRes = bound.hRes;
            p.hPre = bound.hPre;
            return MHC_STATUS_SUCCESS;
        }
    }

    // Split path plan: enough (row tile, K-slice) workgroups to fill the chip,
    // at least 16 k-steps (4 per wave) per slice.
    const int64_t rowTiles = (T + 15) / 16;
    const int64_t ksTotal = K / 32;
    const int64_t maxSlices = std::max<int64_t>(1, ksTotal / 16);
    int64_t S = std::min<int64_t>(maxSlices, std::max<int64_t>(1, (2048 + rowTiles - 1) / rowTiles));
    const int64_t ksPer = (ksTotal + S - 1) / S;
    S = (ksTotal + ksPer - 1) / ksPer;
    p.splitS = static_cast<int>(S);
    p.ksPerSlice = static_cast<int>(ksPer);

    // Fused path (n = 4): slices of DW = 64*KP columns, the widest of 256,
    // 128, 64 that divides D (a wider slice reads longer runs of each row
    // and needs fewer exchange records per tile).
    p.fusedTiles = rowTiles;
    if (n == 4 && (D % 64) == 0) {
        for (int kp : {4, 2, 1}) {
            if (D % (64 * kp) == 0) {
                p.fusedDw = 64 * kp;
                p.fusedP = static_cast<int>(D / (64 * kp));
                break;
            }
        }
    }
    // Strip path (n = 4, D % 32 == 0 from D = 192): slices of 256 columns
    // (the last one narrower when D % 256 != 0: whole 64-column strips past
    // D and, when D % 64 == 32, the upper half of the last live strip load
    // and store nothing), at most strip_max_slices() of them; its tile and
    // row indices are 32-bit, which bounds T.  Measured on MI355X (bf16,
    // gamma, back to back, us, strip / rows / split): T = 8192: D = 7104
    // 107.4 / 167.5 / 264.6, 7072 122.4 / 168.1 / 261.9 (its odd streams'
    // rows start half a cache line off), 4160 75.3 / 109.0 / 144.2, 2112
    // 47.1 / 65.1 / 65.7, 1216 29.9 / 48.3 / 44.6, 320 19.3 / 34.4 / 21.6,
    // 224 17.4 / 32.8 / 18.5, 192 16.6 / 31.9 / 17.7; T = 2048: D = 7104
    // 33.8 / 50.7 / 61.1, 7072 37.1 / 50.9 / 60.9, 1216 14.4 / 21.4 / 19.1,
    // 192 10.2 / 13.7 / 11.7; T = 1024: D = 7072 22.6 / 29.9 / 40.6, 224
    // 10.3 / 10.7 / 12.0.  One slice of one or two strips gains nothing on
    // the split path (D = 64, T = 8192 16.0 / 27.3 / 15.0; D = 128 16.2 /
    // 31.8 / 15.9).
    if (n == 4 && (D % 32) == 0 && D >= 192 && (D + 255) / 256 <= mhc::strip_max_slices() &&
        T < (int64_t{1} << 24)) {
        p.stripP = static_cast<int>((D + 255) / 256);
    }
    // Rows path (any n, K % 128 == 0): rows_block_rows()-row blocks x S
    // K-ranges of contiguous stages (the last range may be shorter).  S balances whole waves of 256
    // workgroups (one per CU of an MI355X; S only affects speed) against the
    // partial traffic: cost ~ rounds * (x bytes of one item) + partial bytes
    // written and read.  32-bit buffer offsets bound K and the B bytes.
    const int64_t rowsNT = (2 * M) / 16;
    if ((K % 128) == 0 && K < (int64_t{1} << 25) &&
        (K / 32) * rowsNT * 1024 < (int64_t{1} << 31)) {
        const int64_t blockRows = mhc::rows_block_rows();
        const int64_t blocks = (T + blockRows - 1) / blockRows;
        const int64_t NS = K / 32 / mhc::rows_stage_ksteps();
        const int64_t stageBytes = 32 * 2 * mhc::rows_stage_ksteps();
        constexpr int64_t kSlotsPerRound = 256;
        double best = -1.0;
        for (int64_t S = 1; S <= NS; ++S) {
            const int64_t perItem = (NS + S - 1) / S;
            if (S > 1 && (NS + S - 2) / (S - 1) == perItem) {
                continue;  // same stages per item with fewer ranges; this
                           // also keeps every range non-empty
            }
            if ((blocks * S + 255) * mhc::rows_gemm_threads() >= (int64_t{1} << 32)) {
                break;  // the GEMM grid's work-items must stay below 2^32
            }
            const int64_t rounds = (blocks * S + kSlotsPerRound - 1) / kSlotsPerRound;
            const double cost = static_cast<double>(rounds) * static_cast<double>(std::min(T, blockRows)) *
                                    static_cast<double>(perItem * stageBytes) * kSlotsPerRound +
                                2.0 * static_cast<double>(S) * static_cast<double>(T) * (M + 1) * 4.0;
            if (best < 0.0 || cost < best) {
                best = cost;
                p.rowsS = static_cast<int>(S);
            }
        }
        p.rowsBlocks = static_cast<int>(blocks);
        // n = 8 with fp16 x takes the prep launch at every batch: its block
        // GEMM building B itself needs more registers than two waves per
        // SIMD have (a 40-byte private segment) and ran slower (MI355X, back
        // to back, us, in-GEMM / prep: D = 7168, T = 2048 130.4 / 120.1; D =
        // 8192, T = 1024 82.3 / 80.4, T = 2048 144.7 / 141.5, T = 4096 264.6
        // / 255.7; D = 4096, T = 2048 89.2 / 83.4; bf16, D = 8192, T = 2048
        // 122.4 / 133.5 keeps the in-GEMM build).
        p.rowsBFromPhi = blocks <= mhc::kRowsPhiMaxBlocks && !(n == 8 && !p.isBf16);
        if (const char *phiEnv = test_env("MHCPRE_ROWS_B")) {
            if (std::strcmp(phiEnv, "phi") == 0) {
                p.rowsBFromPhi = true;
            } else if (std::strcmp(phiEnv, "prep") == 0) {
                p.rowsBFromPhi = false;
            }
        }
        // Small batches: one K-range per workgroup of the small-batch GEMM,
        // which builds B from phi itself (each element of B is used once).
        // Its wide variant (twice the rows and waves) takes the next band of
        // T when the rows are long: measured on MI355X (back to back, us,
        // small-batch / block GEMM): n = 4, D = 7168, T = 160 11.8 / 12.6,
        // T = 256 13.1 / 14.6; D = 4096, T = 256 12.3 / 13.6; n = 8, D = 7168,
        // T = 128 19.9 / 22.4; D = 2048 (K = 16384), T = 128 13.8 / 14.4;
        // n = 6, D = 4096, T = 128 12.7 / 14.0; but D = 1024, T = 256 10.9 /
        // 10.2 and fp16 D = 2048, T = 256 13.4 / 11.4 (K < 16384).  Its x
        // offsets (every row it holds, past T too) stay below 2^31.
        const int64_t smallKs = mhc::rows_small_ksteps();
        const bool wide = T > mhc::rows_small_rows(n, false);
        if (T <= mhc::rows_small_rows(n, wide) && (!wide || K >= 16384) && ((K / 32) % smallKs) == 0 &&
            mhc::rows_small_rows(n, wide) * K * 2 < (int64_t{1} << 31)) {
            p.rowsSmall = true;
            p.rowsS = static_cast<int>((K / 32) / smallKs);
        }
        // The epilogue addresses the partials with 32-bit offsets.
        if (static_cast<int64_t>(p.rowsS) * T * (M + 1) * 4 >= (int64_t{1} << 31)) {
            p.rowsS = 0;
        }
        // Many K-ranges: partials row-major, so that each epilogue workgroup
        // reads its row's sums as one run.  Measured on MI355X (back to back,
        // us, K-range-major / row-major): n = 8, D = 7168, T = 64 (S = 224)
        // 16.8 / 16.0; n = 8, D = 8192, T = 256 30.2 / 28.9, T = 2048 123.3 /
        // 122.0; n = 6, D = 4096, T = 512 26.5 / 24.9; with few K-ranges the
        // GEMM's scattered short writes cost more (n = 4, D = 256, T = 128,
        // S = 4: 10.1 / 10.6; n = 8, D = 8192, T = 5472, S = 11: 280.2 /
        // 282.0).
        p.rowsRowMajor = p.rowsS >= 32;
        if (const char *layoutEnv = test_env("MHCPRE_ROWS_PARTIALS")) {
            if (std::strcmp(layoutEnv, "rows") == 0) {
                p.rowsRowMajor = true;
            } else if (std::strcmp(layoutEnv, "ranges") == 0) {
                p.rowsRowMajor = false;
            }
        }
    }
    if (n == 4) {
        // The strip kernel where it applies (D % 32 == 0, D >= 192), except small
        // batches: its fixed cost (every workgroup builds its B slice) is
        // ~11-12 us whatever the shape, while the rows path's two short
        // launches grow with K and T.  Measured on MI355X (back to back, us,
        // bf16 with gamma unless noted, rows / strip): T <= 128 rows at every
        // width (D = 7168: T = 128 10.2 / 11.6; D = 4096, T = 128 9.8 / 11.5;
        // fp16 without gamma, D = 7168, T = 128 10.8 / 12.4); T = 160 rows
        // up to D = 6144 (11.3 / 11.9); up to T = 256 rows on the wide
        // small-batch GEMM at 31 or more slices (their few teams span the
        // XCDs: D = 7936, T = 256 13.9 / 14.9; D = 8192, T = 256 14.8 / 14.7;
        // D = 10240, T = 192 14.1 / 15.5; D = 16384, T = 256 20.0 / 20.7;
        // strip from T = 384: D = 8192 19.0 / 15.4) and below them while T *
        // D <= 9 * 2^17 (D = 4096, T = 256 12.0 /
        // 12.3; D = 5120, T = 224 12.2 / 12.8; D = 6144, T = 192 12.0 / 12.1;
        // D = 7168, T = 160 12.0 / 12.0; strip above: D = 5120, T = 256 12.8
        // / 12.3; D = 6144, T = 224 12.7 / 11.6; D = 7168, T = 192 12.4 /
        // 12.3, T = 256 13.5 / 12.3; fp16 without gamma, D = 7168, T = 256
        // 15.2 / 13.7) and below while T * D <= 2^19 (D = 2048, T = 256 11.0
        // / 10.9; D = 3072, T = 192 12.1 / 12.3 stays strip); up to T = 1024
        // while T * D <= 3 * 2^17 (D = 768, T = 512 10.7 / 10.9; D = 256, T =
        // 768 10.1 / 10.6; D = 256, T = 1024 10.8 / 10.6, D = 512, T = 1024
        // 11.9 / 10.9 and D = 1024, T = 512 11.7 / 11.0 stay strip).
        //
        // Other widths take the rows path, or the split path for short rows
        // (K <= 8704) from T = 2048, whose 16-row tiles then beat the rows
        // path's reread of x; the fused kernel was slower than one of the
        // two at every shape measured (rows / split / fused: D = 7104, T =
        // 8192 166 / 264 / 754; D = 4160, T = 8192 107 / 144 / 374; D =
        // 4160, T = 1024 24.1 / 30.7 / 64.7; D = 2112, T = 1024 17.7 / 19.8
        // / 32.0; D = 2112, T = 8192 68.5 / 66.0 / 131; D = 1216, T = 2048
        // 21.4 / 19.0 / 29.1; D = 384, T = 4096 24.6 / 15.5 / 25.0; D = 192,
        // T = 8192 35.2 / 17.5 / 21.5) and stays the fallback of shapes the
        // rows path cannot hold.
        if (p.stripP > 0) {
            // Single-slice teams (D = 256) included: the strip kernel also
            // beats the split path there (strip / split, us: T = 4096 11.8 /
            // 13.3, 8192 17.1 / 20.2, 32768 42.7 / 49.6).
            p.path = mhc::Path::kStrip;
            const int64_t td = T * D;
            if (p.rowsS > 0 &&
                (T <= 128 || (T <= 160 && D <= 6144) ||
                 (T <= 256 && ((p.rowsSmall && (td <= 9 * (int64_t{1} << 17) || p.stripP >= 31)) ||
                               td <= (int64_t{1} << 19))) ||
                 (T <= 1024 && td <= 3 * (int64_t{1} << 17)))) {
                p.path = mhc::Path::kRows;
            }
        } else if (p.rowsS > 0) {
            p.path = mhc::Path::kRows;
            if (!p.rowsSmall && K <= 8704 && T >= 2048) {
                p.path = mhc::Path::kSplit;
            }
        } else {
            p.path = p.fusedP > 0 ? mhc::Path::kFused : mhc::Path::kSplit;
        }
    } else {
        p.path = p.rowsS > 0 ? mhc::Path::kRows : mhc::Path::kSplit;
        // Short rows (K <= 9216) from a thousand rows: the rows path reads x
        // twice and adds many partial sums per row, while the split path's
        // 16-row tiles stream x once per kernel with few partials.  Measured
        // on MI355X, back to back (rows / split, us): n = 6, D = 512: T =
        // 2048 28.4 / 17.1, 4096 43.7 / 26.2, 8192 64.7 / 39.2; n = 6, D =
        // 1024: T = 512 14.8 / 16.2, 1024 22.2 / 18.8, 4096 49.4 / 39.7, 8192
        // 76.7 / 62.0; n = 6, D = 1536: T = 1024 24.3 / 24.6, 2048 37.2 /
        // 33.4, 8192 89.5 / 86.3; n = 8, D = 512: T = 1024 24.4 / 17.9, 8192
        // 80.4 / 58.8; n = 8, D = 1024: T = 512 21.8 / 21.0, 1024 31.7 /
        // 28.4, 4096 63.6 / 60.4, 8192 101.9 / 99.1.  From K = 12288 the rows
        // path is as fast or faster (n = 6, D = 2048: T = 1024 28.7 / 29.1,
        // 2048 40.9 / 40.3, 8192 108.9 / 110.9; n = 8, D = 1536: T = 1024
        // 32.5 / 35.9, 2048 46.5 / 51.3, 8192 126.1 / 142.7).
        if (p.path == mhc::Path::kRows && !p.rowsSmall && K <= 9216 &&
            (T >= 1024 || (T >= 512 && n == 8 && K <= 8192))) {
            p.path = mhc::Path::kSplit;
        }
    }
    const char *force = test_env("MHCPRE_FORCE_PATH");
    if (force != nullptr) {
        if (std::strcmp(force, "split") == 0) {
            p.path = mhc::Path::kSplit;
        } else if (std::strcmp(force, "fused") == 0 && p.fusedP > 0) {
            p.path = mhc::Path::kFused;
        } else if (std::strcmp(force, "rows") == 0 && p.rowsS > 0) {
            p.path = mhc::Path::kRows;
        } else if (std::strcmp(force, "strip") == 0 && p.stripP > 0) {
            p.path = mhc::Path::kStrip;
        }
    }
    if (const char *launch = std::getenv("MHCPRE_LAUNCH")) {
        p.fusedCooperative = std::strcmp(launch, "cooperative") == 0;
    }
    if (const char *spin = test_env("MHCPRE_SPIN_LIMIT")) {
        char *end = nullptr;
        const unsigned long v = std::strtoul(spin, &end, 10);
        if (end != spin && *end == '\0' && v <= 0xFFFFFFFFul) {
            p.spinLimit = static_cast<uint32_t>(v);
        }
    }

    // Strip teams: those the device that holds x runs (MI355X's shape when
    // the runtime cannot tell), at most one per row tile.  A device that
    // cannot hold one team, inside an XCD or across them, takes the fused
    // path (or the split path).
    if (p.stripP > 0) {
        DeviceShape shape = kPlanShapeDefault;
        const int dev = planDevice;
        if (dev < 0 || !device_shape_of(dev, shape)) {
            (void)hipGetLastError();
            shape = kPlanShapeDefault;
        }
        const StripGeometry geo = strip_geometry(p.stripP, shape);
        const int teamsPerXcd = geo.teams;
        const int teams = teamsPerXcd * geo.groups;
        p.stripMaxTeams = static_cast<int>(std::min<int64_t>(rowTiles, teams));
        if (teams < 1 && p.path == mhc::Path::kStrip) {
            p.path = p.fusedP > 0 ? mhc::Path::kFused : mhc::Path::kSplit;
        }
    }

    // Workspace: the header, then the layout of the path the plan takes (a
    // workspace holds one launch at a time).  The split layout holds B
    // fragments and [S][T][M+1] partials; the fused layout a broadcast block
    // and P records per row tile; the strip layout only per-team rings of
    // them, so its size does not grow with T.  A fused plan also covers the
    // split layout, its fallback on a device that cannot co-schedule a fused
    // team; a strip executor runs a fallback only where its workspace holds
    // that layout (phase 2 checks).
    const size_t splitBsplit = mhc::kWsHeaderBytes;
    const size_t splitPartial =
        align_up(splitBsplit + static_cast<size_t>(K) * static_cast<size_t>(2 * M) * 2, 256);
    const size_t splitEnd =
        align_up(splitPartial + static_cast<size_t>(S) * static_cast<size_t>(T) * (M + 1) * 4, 256);
    p.wsBsplit = splitBsplit;
    p.wsPartial = splitPartial;
    p.wsSplitEnd = splitEnd;
    if (p.fusedP > 0) {
        const size_t tiles = static_cast<size_t>(rowTiles);
        p.wsFinal = mhc::kWsHeaderBytes;
        p.wsFusedPartial = align_up(p.wsFinal + tiles * mhc::fused_bcast_words(n) * 8, 256);
        p.wsFusedEnd = align_up(
            p.wsFusedPartial + tiles * p.fusedP * mhc::fused_record_words(n) * 8, 256);
    }
    size_t stripEnd = 0;
    if (p.stripP > 0) {
        const size_t ring = static_cast<size_t>(p.stripMaxTeams) * mhc::strip_ring_slots();
        p.wsStripBcast = mhc::kWsHeaderBytes;
        p.wsStripRecs = align_up(p.wsStripBcast + ring * mhc::strip_bcast_words() * 8, 256);
        stripEnd = align_up(p.wsStripRecs + ring * p.stripP * mhc::strip_record_words() * 8, 256);
    }
    size_t rowsEnd = 0;
    if (p.rowsS > 0) {
        p.wsRowsB = mhc::kWsHeaderBytes;
        p.wsRowsPartial = p.wsRowsB;
        if (!p.rowsSmall && !p.rowsBFromPhi) {
            p.wsRowsPartial =
                align_up(p.wsRowsB + static_cast<size_t>(K / 32) * static_cast<size_t>(p.NT) * 1024, 256);
        }
        rowsEnd = align_up(p.wsRowsPartial + static_cast<size_t>(p.rowsS) * static_cast<size_t>(T) *
                                                 static_cast<size_t>(M + 1) * 4,
                           256);
    }
    switch (p.path) {
    case mhc::Path::kStrip:
        p.wsTotal = stripEnd;
        break;
    case mhc::Path::kFused:
        p.wsTotal = std::max(p.wsFusedEnd, splitEnd);
        break;
    case mhc::Path::kRows:
        p.wsTotal = rowsEnd;
        break;
    default:
        p.wsTotal = splitEnd;
        break;
    }
    if (useCache) {
        std::lock_guard<std::mutex> lock(plan_cache_mutex());
        if (plan_cache().size() >= kPlanCacheEntries) {
            plan_cache().clear();
        }
        plan_cache().emplace(key, p);
    }
    return MHC_STATUS_SUCCESS;
}

void prime_coresident(mhcPreExecutor *ex);

// Shape and type rules of weights to prepare: those phase 1 applies to phi
// and gamma (element counts: phi K*M, gamma K or none), with K taken from
// phi's element count and D = K / n a multiple of 16.
int weights_shape(const mhcTensor *phi, const mhcTensor *gamma, int32_t n, int &M, int64_t &K,
                  bool &hasGamma)
{
    if (phi == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (n != 4 && n != 6 && n != 8) {
        return MHC_STATUS_UNSUPPORTED_SHAPE;
    }
    M = n * n + 2 * n;
    hasGamma = gamma != nullptr && numel(*gamma) > 0 && gamma->ndim > 0;
    if (phi->dtype != MHC_DTYPE_FLOAT || (hasGamma && gamma->dtype != MHC_DTYPE_FLOAT)) {
        return MHC_STATUS_INVALID_DTYPE;
    }
    const int64_t count = numel(*phi);
    if (!dims_positive(*phi) || count <= 0 || count % M != 0) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    K = count / M;
    if (K % n != 0 || (K / n) % 16 != 0 || K / n > kMaxWidth) {
        return MHC_STATUS_UNSUPPORTED_SHAPE;
    }
    if (hasGamma && (!dims_positive(*gamma) || numel(*gamma) != K)) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    return MHC_STATUS_SUCCESS;
}

uint64_t prepared_bytes(int M, int64_t K) { return static_cast<uint64_t>(K) * static_cast<uint64_t>(2 * M) * 2; }

int get_workspace(const mhcTensor *x, const mhcTensor *phi, const mhcTensor *alpha,
                  const mhcTensor *bias, const mhcTensor *gamma, float normEps, float hcEps,
                  const mhcTensor *hIn, const mhcTensor *hPost, const mhcTensor *hRes,
                  const mhcTensor *hPre, uint64_t *workspaceSize, mhcPreExecutor **executor)
{
    if (workspaceSize == nullptr || executor == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    *executor = nullptr;
    mhc::Plan plan;
    const int st = validate_and_plan(x, phi, alpha, bias, gamma, normEps, hcEps, hIn, hPost, hRes, hPre,
                               plan);
    if (st != MHC_STATUS_SUCCESS) {
        return st;
    }
    mhcPreExecutor *ex = new (std::nothrow) mhcPreExecutor;
    if (ex == nullptr) {
        return MHC_STATUS_HIP_ERROR;
    }
    ex->plan = plan;
    ex->device = device_of(plan.x);
    prime_coresident(ex);
    *workspaceSize = plan.wsTotal;
    *executor = ex;
    return MHC_STATUS_SUCCESS;
}

// Co-resident workgroups of the executor's strip or fused kernel on the
// current device: the occupancy query runs once per process, device and
// kernel instance (n, x dtype, prepared weights, fused slice width), and its
// result is kept in the executor too.
int cached_coresident(std::atomic<int> &slot, int (*query)(const mhc::Plan &, int),
                      const mhc::Plan &p, int cus)
{
    int v = slot.load(std::memory_order_relaxed);
    if (v != -2) {
        return v;
    }
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess) {
        (void)hipGetLastError();
        return query(p, cus);
    }
    using Key = std::tuple<uintptr_t, int, int, bool, bool, int, int>;
    static std::mutex mu;
    static std::map<Key, int> known;
    const Key key{reinterpret_cast<uintptr_t>(query), device, p.n, p.isBf16, p.bprep != nullptr,
                  p.fusedDw, cus};
    {
        std::lock_guard<std::mutex> lock(mu);
        const auto it = known.find(key);
        if (it != known.end()) {
            v = it->second;
        }
    }
    if (v == -2) {
        v = query(p, cus);
        std::lock_guard<std::mutex> lock(mu);
        known.emplace(key, v);
    }
    slot.store(v, std::memory_order_relaxed);
    return v;
}

// Phase 2 after the workspace checks: the device check, the path choice for
// this device and the kernel launches.
int launch_on(void *workspace, mhcPreExecutor *executor, hipStream_t stream)
{
    const mhc::Plan &p = executor->plan;
    // The kernels run on the current device and address the executor's
    // tensors directly: it must be the device that holds them.
    if (executor->device >= 0) {
        int current = -1;
        if (hipGetDevice(&current) != hipSuccess) {
            (void)hipGetLastError();
            return MHC_STATUS_HIP_ERROR;
        }
        if (current != executor->device) {
            return MHC_STATUS_DEVICE_MISMATCH;
        }
    }
    hipError_t err = hipSuccess;
    bool done = false;
    int device = -1;
    DeviceShape shape;
    // The launches' status is read back with hipGetLastError: first clear an
    // error an earlier call of the process may have left there (the split
    // path makes no other HIP call before its first launch).
    (void)hipGetLastError();
    if (p.path != mhc::Path::kSplit && !device_shape(device, shape)) {
        return MHC_STATUS_HIP_ERROR;
    }
    const uint32_t launchId = next_launch_id();
    executor->lastLaunchId.store(launchId, std::memory_order_relaxed);
    if (p.path == mhc::Path::kStrip) {
        // One workgroup per CU, all co-resident; each XCD's CUs hold at least
        // one team of stripP slice workgroups and one reducer workgroup.
        // Teams of two or more slices get at least two reducers: with one,
        // the reducer paces the team (measured on MI355X at T = 8192: 43 ->
        // 32 us at D = 1024, 74 -> 54 us at D = 2304); a single-slice team
        // keeps one, which leaves room for more teams.
        const StripGeometry geo = strip_geometry(p.stripP, shape);
        const int perXcd = geo.perGroup;
        int teamsPerXcd = geo.teams;
        // Teams beyond the rings' capacity would have no slots of their own
        // (teams without tiles write nothing).
        if (teamsPerXcd * geo.groups > p.stripMaxTeams && p.stripMaxTeams < p.fusedTiles) {
            teamsPerXcd = p.stripMaxTeams / geo.groups;
        }
        if (teamsPerXcd >= 1 && shape.cus <= mhc::kMaxEpochGrid &&
            cached_coresident(executor->stripCoresident, mhc::strip_max_coresident, p, shape.cus) >=
                shape.cus) {
            mhc::Plan lp = p;
            lp.statusWord = executor->statusWord.load(std::memory_order_relaxed);
            lp.stripXcds = geo.groups;
            lp.stripTeamsPerXcd = teamsPerXcd;
            // Workgroups of a team beyond the slices and reducers leave at once.
            lp.stripR = mhc::strip_reducers(perXcd / teamsPerXcd - p.stripP);
            lp.stripGrid = shape.cus;
            err = mhc::launch_strip(lp, workspace, launchId, stream);
            done = true;
        }
    }
    // A strip executor whose device cannot hold its teams (not the device
    // phase 1 planned for) falls back only to a layout its workspace holds.
    const auto fallbackOk = [&](size_t end) { return p.path != mhc::Path::kStrip || end <= p.wsTotal; };
    if (!done && p.path == mhc::Path::kStrip && !fallbackOk(p.wsFusedEnd) && !fallbackOk(p.wsSplitEnd)) {
        return MHC_STATUS_UNSUPPORTED_SHAPE;
    }
    if (!done && p.fusedP > 0 && (p.path == mhc::Path::kFused || p.path == mhc::Path::kStrip) &&
        fallbackOk(p.wsFusedEnd)) {
        // The fused path, or the strip path's fallback on a device too small
        // for a strip team.  Teams of fusedP workgroups must be co-resident; a
        // device too small for one team runs the split path instead.
        const int coresident =
            cached_coresident(executor->fusedCoresident, mhc::fused_max_coresident, p, shape.cus);
        if (coresident >= p.fusedP) {
            mhc::Plan lp = p;
            lp.statusWord = executor->statusWord.load(std::memory_order_relaxed);
            lp.fusedTeams = std::min(coresident, mhc::kMaxEpochGrid) / p.fusedP;
            lp.fusedGrid = lp.fusedTeams * p.fusedP;
            err = mhc::launch_fused(lp, workspace, launchId, stream);
            done = true;
        }
    }
    if (!done && p.path == mhc::Path::kRows) {
        err = mhc::launch_rows(p, workspace, shape.xcds, stream);
        done = true;
    }
    if (!done) {
        if (!fallbackOk(p.wsSplitEnd)) {
            return MHC_STATUS_UNSUPPORTED_SHAPE;
        }
        err = mhc::launch_split(p, workspace, stream);
    }
    return err == hipSuccess ? MHC_STATUS_SUCCESS : MHC_STATUS_HIP_ERROR;
}

// The occupancy queries of a new executor and the address of the device's
// built-in workspace (mhcPreNoAlloc), when the current device is the one
// that holds its tensors (otherwise its first launch makes them): so that a
// later launch, one under stream capture included, makes neither call.
void prime_coresident(mhcPreExecutor *ex)
{
    const mhc::Plan &p = ex->plan;
    int device = -1;
    DeviceShape shape;
    if (ex->device < 0) {
        return;
    }
    if (!device_shape(device, shape) || device != ex->device) {
        (void)hipGetLastError();
        return;
    }
    void *scratch = nullptr;
    if (mhc::scratch_address(device, &scratch) != hipSuccess) {
        (void)hipGetLastError();
    }
    if (p.path != mhc::Path::kStrip && p.path != mhc::Path::kFused) {
        return;
    }
    if (p.path == mhc::Path::kStrip) {
        (void)cached_coresident(ex->stripCoresident, mhc::strip_max_coresident, p, shape.cus);
    }
    if (p.fusedP > 0) {
        (void)cached_coresident(ex->fusedCoresident, mhc::fused_max_coresident, p, shape.cus);
    }
}

}  // namespace

extern "C" {

int mhcPreGetWorkspaceSize(const mhcTensor *x, const mhcTensor *phi, const mhcTensor *alpha,
                           const mhcTensor *bias, const mhcTensor *gamma, float normEps,
                           float hcEps, const mhcTensor *hIn, const mhcTensor *hPost,
                           const mhcTensor *hRes, uint64_t *workspaceSize,
                           mhcPreExecutor **executor)
{
    return get_workspace(x, phi, alpha, bias, gamma, normEps, hcEps, hIn, hPost, hRes, nullptr,
                         workspaceSize, executor);
}

int mhcPreGetWorkspaceSizeWithHPre(const mhcTensor *x, const mhcTensor *phi,
                                   const mhcTensor *alpha, const mhcTensor *bias,
                                   const mhcTensor *gamma, float normEps, float hcEps,
                                   const mhcTensor *hIn, const mhcTensor *hPost,
                                   const mhcTensor *hRes, const mhcTensor *hPre,
                                   uint64_t *workspaceSize, mhcPreExecutor **executor)
{
    return get_workspace(x, phi, alpha, bias, gamma, normEps, hcEps, hIn, hPost, hRes, hPre,
                         workspaceSize, executor);
}

int mhcPre(void *workspace, uint64_t workspaceSize, mhcPreExecutor *executor, hipStream_t stream)
{
    if (executor == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (workspace == nullptr || workspaceSize < executor->plan.wsTotal) {
        return MHC_STATUS_WORKSPACE_TOO_SMALL;
    }
    if (!aligned(workspace, 256)) {
        return MHC_STATUS_WORKSPACE_TOO_SMALL;
    }
    return launch_on(workspace, executor, stream);
}

int mhcPrePrepareWeightsSize(const mhcTensor *phi, const mhcTensor *gamma, int32_t n,
                             uint64_t *bytes)
{
    if (bytes == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    int M = 0;
    int64_t K = 0;
    bool hasGamma = false;
    const int st = weights_shape(phi, gamma, n, M, K, hasGamma);
    if (st != MHC_STATUS_SUCCESS) {
        return st;
    }
    *bytes = prepared_bytes(M, K);
    return MHC_STATUS_SUCCESS;
}

int mhcPrePrepareWeights(const mhcTensor *phi, const mhcTensor *gamma, int32_t n, void *buffer,
                         uint64_t bytes, uint64_t version, hipStream_t stream,
                         mhcPreWeights **weights)
{
    if (weights == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    *weights = nullptr;
    int M = 0;
    int64_t K = 0;
    bool hasGamma = false;
    const int st = weights_shape(phi, gamma, n, M, K, hasGamma);
    if (st != MHC_STATUS_SUCCESS) {
        return st;
    }
    if (buffer == nullptr || phi->data == nullptr || (hasGamma && gamma->data == nullptr)) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (bytes < prepared_bytes(M, K)) {
        return MHC_STATUS_WORKSPACE_TOO_SMALL;
    }
    if (!aligned(buffer, 256) || !aligned(phi->data, 16) || (hasGamma && !aligned(gamma->data, 16))) {
        return MHC_STATUS_MISALIGNED;
    }
    // The preparation runs on the current device, which must hold the buffer.
    const int device = device_of(buffer);
    if (device >= 0) {
        int current = -1;
        if (hipGetDevice(&current) != hipSuccess) {
            (void)hipGetLastError();
            return MHC_STATUS_HIP_ERROR;
        }
        if (current != device) {
            return MHC_STATUS_DEVICE_MISMATCH;
        }
    }
    mhcPreWeights *w = new (std::nothrow) mhcPreWeights;
    if (w == nullptr) {
        return MHC_STATUS_HIP_ERROR;
    }
    // A buffer that live handles or executors read with another layout.
    if (!buffer_acquire(buffer, n, K)) {
        delete w;
        return MHC_STATUS_INVALID_SHAPE;
    }
    // The launch's status is read back with hipGetLastError: first clear an
    // error an earlier call of the process may have left there.
    (void)hipGetLastError();
    if (mhc::launch_prepare_b(n, static_cast<const float *>(phi->data),
                              hasGamma ? static_cast<const float *>(gamma->data) : nullptr, buffer, K,
                              stream) != hipSuccess) {
        (void)hipGetLastError();
        buffer_release(buffer);
        delete w;
        return MHC_STATUS_HIP_ERROR;
    }
    w->n = n;
    w->M = M;
    w->K = K;
    w->buffer = buffer;
    w->version = version;
    w->device = device;
    *weights = w;
    return MHC_STATUS_SUCCESS;
}

int mhcPreWeightsVersion(const mhcPreWeights *weights, uint64_t *version)
{
    if (weights == nullptr || version == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    *version = weights->version;
    return MHC_STATUS_SUCCESS;
}

int mhcPreWeightsDestroy(mhcPreWeights *weights)
{
    if (weights == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    buffer_release(weights->buffer);
    delete weights;
    return MHC_STATUS_SUCCESS;
}

int mhcPreGetWorkspaceSizePrepared(const mhcTensor *x, const mhcPreWeights *weights,
                                   const mhcTensor *alpha, const mhcTensor *bias, float normEps,
                                   float hcEps, const mhcTensor *hIn, const mhcTensor *hPost,
                                   const mhcTensor *hRes, const mhcTensor *hPre,
                                   uint64_t *workspaceSize, mhcPreExecutor **executor)
{
    if (weights == nullptr || workspaceSize == nullptr || executor == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    *executor = nullptr;
    // phi stands in for the prepared buffer in phase 1's checks (element
    // count K*M, fp32, aligned); gamma is folded into the prepared B.
    mhcTensor phiD{};
    phiD.data = weights->buffer;
    phiD.dtype = MHC_DTYPE_FLOAT;
    phiD.ndim = 2;
    phiD.dims[0] = weights->K;
    phiD.dims[1] = weights->M;
    mhc::Plan plan;
    const int st = validate_and_plan(x, &phiD, alpha, bias, nullptr, normEps, hcEps, hIn, hPost, hRes,
                                     hPre, plan);
    if (st != MHC_STATUS_SUCCESS) {
        return st;
    }
    if (plan.n != weights->n || plan.K != weights->K) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    const int device = device_of(plan.x);
    if (device >= 0 && weights->device >= 0 && device != weights->device) {
        return MHC_STATUS_DEVICE_MISMATCH;
    }
    plan.bprep = weights->buffer;
    plan.phi = nullptr;
    plan.gamma = nullptr;
    plan.hasGamma = false;
    mhcPreExecutor *ex = new (std::nothrow) mhcPreExecutor;
    if (ex == nullptr) {
        return MHC_STATUS_HIP_ERROR;
    }
    if (!buffer_acquire(weights->buffer, weights->n, weights->K)) {
        delete ex;
        return MHC_STATUS_INVALID_SHAPE;
    }
    ex->preparedBuffer = weights->buffer;
    ex->plan = plan;
    ex->device = device;
    prime_coresident(ex);
    *workspaceSize = plan.wsTotal;
    *executor = ex;
    return MHC_STATUS_SUCCESS;
}

int mhcPreNoAlloc(mhcPreExecutor *executor, hipStream_t stream)
{
    if (executor == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    // The built-in workspace has a fixed size: larger plans are rejected
    // before any HIP call.
    if (executor->plan.wsTotal > mhc::kScratchBytes) {
        return MHC_STATUS_SCRATCH_TOO_SMALL;
    }
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess) {
        (void)hipGetLastError();
        return MHC_STATUS_HIP_ERROR;
    }
    void *ws = nullptr;
    if (mhc::scratch_address(device, &ws) != hipSuccess) {
        (void)hipGetLastError();
        return MHC_STATUS_HIP_ERROR;
    }
    return launch_on(ws, executor, stream);
}

int mhcPreExecutorSetStatusWord(mhcPreExecutor *executor, uint32_t *deviceWord)
{
    if (executor == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (!aligned(deviceWord, 4)) {
        return MHC_STATUS_MISALIGNED;
    }
    executor->statusWord.store(deviceWord, std::memory_order_relaxed);
    return MHC_STATUS_SUCCESS;
}

int mhcPreExecutorDestroy(mhcPreExecutor *executor)
{
    if (executor == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (executor->preparedBuffer != nullptr) {
        buffer_release(executor->preparedBuffer);
    }
    delete executor;
    return MHC_STATUS_SUCCESS;
}

int mhcPreQueryDeviceStatus(void *workspace, uint64_t workspaceSize,
                            const mhcPreExecutor *executor, hipStream_t stream)
{
    if (executor == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (workspace == nullptr && workspaceSize == 0) {
        // The launches of mhcPreNoAlloc: the current device's built-in array.
        int device = -1;
        if (hipGetDevice(&device) != hipSuccess || mhc::scratch_address(device, &workspace) != hipSuccess) {
            (void)hipGetLastError();
            return MHC_STATUS_HIP_ERROR;
        }
        workspaceSize = mhc::kScratchBytes;
    }
    if (workspace == nullptr || workspaceSize < executor->plan.wsTotal) {
        return MHC_STATUS_WORKSPACE_TOO_SMALL;
    }
    if (hipStreamSynchronize(stream) != hipSuccess) {
        return MHC_STATUS_HIP_ERROR;
    }
    uint64_t word = 0;
    if (hipMemcpy(&word, workspace, sizeof(word), hipMemcpyDeviceToHost) != hipSuccess) {
        return MHC_STATUS_HIP_ERROR;
    }
    const uint32_t code = static_cast<uint32_t>(word);
    const uint32_t epoch = static_cast<uint32_t>(word >> 32);
    const bool timedOut = code == mhc::kDeviceTimeout &&
                          epoch == executor->lastLaunchId.load(std::memory_order_relaxed);
    return timedOut ? MHC_STATUS_DEVICE_TIMEOUT : MHC_STATUS_SUCCESS;
}

const char *mhcPreStatusString(int status)
{
    switch (status) {
    case MHC_STATUS_SUCCESS:
        return "success";
    case MHC_STATUS_NULL_ARGUMENT:
        return "null argument";
    case MHC_STATUS_INVALID_SHAPE:
        return "invalid shape";
    case MHC_STATUS_UNSUPPORTED_SHAPE:
        return "unsupported shape";
    case MHC_STATUS_INVALID_DTYPE:
        return "invalid dtype";
    case MHC_STATUS_WORKSPACE_TOO_SMALL:
        return "workspace too small";
    case MHC_STATUS_HIP_ERROR:
        return "HIP error";
    case MHC_STATUS_DEVICE_MISMATCH:
        return "device mismatch";
    case MHC_STATUS_DEVICE_TIMEOUT:
        return "device timeout";
    case MHC_STATUS_MISALIGNED:
        return "misaligned device pointer";
    case MHC_STATUS_SCRATCH_TOO_SMALL:
        return "workspace larger than the built-in scratch";
    default:
        return "unknown status";
    }
}

int mhcPreExecutorPath(const mhcPreExecutor *executor, const char **name)
{
    if (executor == nullptr || name == nullptr) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    switch (executor->plan.path) {
    case mhc::Path::kStrip:
        *name = "strip";
        break;
    case mhc::Path::kFused:
        *name = "fused";
        break;
    case mhc::Path::kRows:
        *name = "rows";
        break;
    default:
        *name = "split";
        break;
    }
    return MHC_STATUS_SUCCESS;
}

int mhcPreStreamProbe(const void *src, uint64_t readBytes, void *dst, uint64_t writeBytes,
                      int32_t workgroups, hipStream_t stream)
{
    if ((readBytes > 0 && src == nullptr) || (writeBytes > 0 && dst == nullptr)) {
        return MHC_STATUS_NULL_ARGUMENT;
    }
    if (readBytes % 4096 != 0 || writeBytes % 1024 != 0 || readBytes >= (uint64_t{1} << 42) ||
        writeBytes >= (uint64_t{1} << 40) || workgroups < 0 || workgroups > 65536) {
        return MHC_STATUS_INVALID_SHAPE;
    }
    if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0) {
        return MHC_STATUS_MISALIGNED;
    }
    if (readBytes == 0 && writeBytes == 0) {
        return MHC_STATUS_SUCCESS;
    }
    int wg = workgroups;
    if (wg == 0) {
        int device = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&device) != hipSuccess || hipGetDeviceProperties(&prop, device) != hipSuccess) {
            return MHC_STATUS_HIP_ERROR;
        }
        wg = prop.multiProcessorCount;
    }
    (void)hipGetLastError();  // a stale error from an earlier call is not this launch's
    return mhc::launch_stream_probe(src, static_cast<int64_t>(readBytes), dst, static_cast<int64_t>(writeBytes), wg,
                                    stream) == hipSuccess
               ? MHC_STATUS_SUCCESS
               : MHC_STATUS_HIP_ERROR;
}

}  // extern "C"
