// Stream probe: a measured bandwidth ceiling for a given read/write byte mix.
//
// The kernel reads `readBytes` and writes `writeBytes` with the access pattern
// HBM serves best on MI355X: every wave takes 4 KB read blocks and 1 KB write
// blocks, grid-strided, each read block as four whole 1 KB wavefront loads
// (nontemporal, like the operator's x stream) and each write block as one
// 1 KB wavefront store; four blocks are in flight per wave.  The written data
// is derived from the read data, so no load can be dropped.  It computes
// nothing else: its rate is what the operator's own byte mix (x in, hIn out)
// could reach with no arithmetic, no exchange and no access-pattern
// constraint, which bench.py reports beside the operator's rate.

#include "mhc_pre_device.h"
#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace mhc {
namespace {

using dev::u32x4_t;

constexpr int kProbeWaves = 8;
constexpr int kProbeUnroll = 4;
constexpr int kReadBlock = 4096;
constexpr int kWriteBlock = 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t probe_rsrc(const void *base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, 0x00020000);
}

template <typename F, int... kIs>
__device__ __forceinline__ void probe_for_seq(F &&f, std::integer_sequence<int, kIs...>)
{
    (f(std::integral_constant<int, kIs>{}), ...);
}

__global__ __launch_bounds__(kProbeWaves * 64) void stream_probe_kernel(const char *src, int64_t nRead,
                                                                        char *dst, int64_t nWrite,
                                                                        int64_t iters)
{
    const int lane = threadIdx.x & 63;
    const int64_t V = (int64_t)gridDim.x * kProbeWaves;
    const int64_t v = (int64_t)blockIdx.x * kProbeWaves + (threadIdx.x >> 6);
    for (int64_t i = 0; i < iters; i += kProbeUnroll) {
        u32x4_t d[kProbeUnroll][4];
        probe_for_seq(
            [&](auto uc) {
                constexpr int u = decltype(uc)::value;
                const int64_t b = v + V * (i + u);
                const bool live = b < nRead;
                const __amdgpu_buffer_rsrc_t r =
                    probe_rsrc(src + (live ? b : 0) * kReadBlock, live ? kReadBlock : 0);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    d[u][k] = __builtin_bit_cast(
                        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, k * 1024 + lane * 16, 0, 2));
                }
            },
            std::make_integer_sequence<int, kProbeUnroll>{});
        probe_for_seq(
            [&](auto uc) {
                constexpr int u = decltype(uc)::value;
                const int64_t b = v + V * (i + u);
                const bool live = b < nWrite;
                const u32x4_t o = d[u][0] ^ d[u][1] ^ d[u][2] ^ d[u][3];
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, o),
                    probe_rsrc(dst + (live ? b : 0) * kWriteBlock, live ? kWriteBlock : 0), lane * 16, 0, 2);
            },
            std::make_integer_sequence<int, kProbeUnroll>{});
    }
}

}  // namespace

hipError_t launch_stream_probe(const void *src, int64_t readBytes, void *dst, int64_t writeBytes,
                               int workgroups, hipStream_t stream)
{
    const int64_t nRead = readBytes / kReadBlock;
    const int64_t nWrite = writeBytes / kWriteBlock;
    const int64_t V = (int64_t)workgroups * kProbeWaves;
    const int64_t blocks = nRead > nWrite ? nRead : nWrite;
    const int64_t iters = (blocks + V - 1) / V;
    hipLaunchKernelGGL(stream_probe_kernel, dim3((unsigned)workgroups), dim3(kProbeWaves * 64), 0, stream,
                       static_cast<const char *>(src), nRead, static_cast<char *>(dst), nWrite, iters);
    return hipGetLastError();
}

}  // namespace mhc
