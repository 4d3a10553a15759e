// Internal launch plan shared by the host library and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace mhc {

// Kernel paths an executor can launch.
enum class Path : int {
    kSplit = 0,   // prep B, split-K MFMA GEMM + sumsq partials, epilogue + hIn (x read twice)
    kFused = 1,   // prep B, one persistent kernel: x read once, kept in registers
};

// Device status word values (first 4 bytes of the workspace).
constexpr uint32_t kDeviceOk = 0u;
constexpr uint32_t kDeviceTimeout = 0x7107u;

// Bytes reserved at the head of the workspace for the status word and the
// fused path's team counters header.
constexpr size_t kWsHeaderBytes = 256;

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
    float normEps = 1e-6f;
    float hcEps = 1e-6f;
    float invFlatDim = 0.f;  // fl(1.0f / K), as code/op_host/mhc_pre.cpp:154

    // Split path: K-slices of the GEMM and k-steps (32 wide) per slice.
    int splitS = 1;
    int ksPerSlice = 0;

    // Fused path parameters.
    int fusedDw = 0;          // d-columns per wave slice
    int fusedP = 0;           // waves (slices) per 16-row tile team
    int fusedWaves = 0;       // waves per workgroup
    int fusedGrid = 0;        // workgroups (cooperative grid)
    int fusedTeams = 0;       // teams of fusedP slices
    int64_t fusedTiles = 0;   // 16-row tiles

    // Workspace layout (byte offsets).
    size_t wsBsplit = 0;
    size_t wsPartial = 0;
    size_t wsCounters = 0;
    size_t wsTotal = 0;

    // Bound device pointers (caller memory).
    const void *x = nullptr;
    const float *phi = nullptr;
    const float *alpha = nullptr;
    const float *bias = nullptr;
    const float *gamma = nullptr;
    void *hIn = nullptr;
    float *hPost = nullptr;
    float *hRes = nullptr;
    float *hPre = nullptr;
};

// Kernel launchers (mhc_pre_kernels.hip).  Each returns the first HIP error.
hipError_t launch_split(const Plan &plan, void *workspace, hipStream_t stream);
hipError_t launch_fused(const Plan &plan, void *workspace, hipStream_t stream);

// Largest number of fused-path workgroups that can be co-resident on the
// current device for a plan with the given wave count, or a negative HIP error.
int fused_max_coresident(const Plan &plan, int numCUs);

}  // namespace mhc
