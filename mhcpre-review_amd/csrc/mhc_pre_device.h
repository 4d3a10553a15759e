// Device helpers shared by the MhcPre kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mhc_pre.h"

namespace mhc {
namespace dev {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

template <int N>
struct Shape {
    static constexpr int M = N * N + 2 * N;     // mix columns
    static constexpr int NT = (2 * M) / 16;     // [hi | lo] column tiles
    static constexpr int NTHI = (M + 15) / 16;  // tiles holding a hi column
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Round-half-even conversions (v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

template <bool kBf16>
__device__ __forceinline__ float x_to_f32(uint32_t bits)
{
    return kBf16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

template <bool kBf16>
__device__ __forceinline__ uint32_t f32_to_x(float f)
{
    return kBf16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Two floats to a packed pair (a in the low half), round-half-even: one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32, where two scalar conversions cost two
// conversions, a shift and an or.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

__device__ __forceinline__ uint32_t pack2_f16(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}

template <bool kBf16>
__device__ __forceinline__ uint32_t pack2_x(float a, float b)
{
    return kBf16 ? pack2_bf16(a, b) : pack2_f16(a, b);
}

// Packed bf16 hi + lo of two floats: hi = bf16(v), lo = bf16(v - hi), both
// round-half-even (v - hi is exact in fp32).
__device__ __forceinline__ void split2_bf16(float a, float b, uint32_t &hi, uint32_t &lo)
{
    hi = pack2_bf16(a, b);
    lo = pack2_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

// Unpack 8 16-bit values held in a u32x4 (element e in half e&1 of word e>>1).
template <bool kBf16>
__device__ __forceinline__ void unpack8(const u32x4_t &v, float (&f)[8])
{
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        f[2 * w] = x_to_f32<kBf16>(v[w] & 0xFFFFu);
        f[2 * w + 1] = x_to_f32<kBf16>(v[w] >> 16);
    }
}

__device__ __forceinline__ u32x4_t pack8_bf16(const float (&f)[8])
{
    u32x4_t r;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        r[w] = pack2_bf16(f[2 * w], f[2 * w + 1]);
    }
    return r;
}

// acc + sum of the squares of 8 packed 16-bit values, one fp32 FMA per value
// (unpacking a bf16 pair is one shift and one mask).
template <bool kBf16>
__device__ __forceinline__ float sumsq8(const u32x4_t &v, float acc)
{
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        float lo, hi;
        if constexpr (kBf16) {
            lo = __uint_as_float(v[w] << 16);
            hi = __uint_as_float(v[w] & 0xFFFF0000u);
        } else {
            lo = f16_bits_to_f32(v[w] & 0xFFFFu);
            hi = f16_bits_to_f32(v[w] >> 16);
        }
        acc = __builtin_fmaf(lo, lo, acc);
        acc = __builtin_fmaf(hi, hi, acc);
    }
    return acc;
}

// Device-scope (cross-XCD coherent) accesses for data exchanged between
// workgroups inside one launch: global_store / global_load with the sc1
// scope bit.  They write through / read past the per-XCD L2 without the
// whole-cache write-back and invalidate that an agent-scope fence costs.
__device__ __forceinline__ void st_dev(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float ld_dev(const float *p)
{
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until every memory access this wave issued has completed (stores
// acknowledged at their scope), and keeps the compiler from moving memory
// accesses across the wait.  Placed between the device-scope data stores and
// the atomic that publishes them.
__device__ __forceinline__ void wait_all_memory()
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The value of lane l ^ 8 within each row of 16 lanes (DPP row_ror:8): a VALU
// move, where a shuffle would take an LDS round trip and a wait.
__device__ __forceinline__ float row_swap8(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t &v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4_t mfma16(const u32x4_t &a, const u32x4_t &b, const f32x4_t &c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// fp16 x -> exact bf16 pair: x = hi + lo (an fp16 significand has 11 bits).
__device__ __forceinline__ void split_f16_to_bf16(const float (&f)[8], u32x4_t &hi, u32x4_t &lo)
{
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t h, l;
        split2_bf16(f[2 * w], f[2 * w + 1], h, l);
        hi[w] = h;
        lo[w] = l;
    }
}

// Exchange epoch of a strip or fused launch, kept in the workspace header.
// One thread of every workgroup reads the epoch the previous launch on the
// workspace stored (epoch_load); the launch uses epoch_next of it, so
// consecutive launches on a workspace, graph replays included, never share an
// epoch.  Each workgroup records the epoch it uses in its own slot
// (epoch_mark); one wave of workgroup 0 stores the new epoch at its end, once
// every workgroup's slot holds it (epoch_publish), so no workgroup can read
// the advanced value.  No workgroup contends for a word, and a workspace left
// with any contents by other use needs no reset.
__device__ __forceinline__ uint32_t epoch_next(uint32_t prev)
{
    const uint32_t e = prev + 1u;
    return (e == 0u || e == 0xFFFFFFFFu) ? 1u : e;  // 0 and ~0 never tag a word
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t header_rsrc(void *ws, size_t off, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(static_cast<char *>(ws) + off, (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ uint32_t epoch_load(void *ws, size_t epochOff)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(header_rsrc(ws, epochOff, 4), 0, 0, 16 /* sc1 */);
}

__device__ __forceinline__ void epoch_mark(void *ws, size_t seenOff, uint32_t epoch, int g)
{
    __builtin_amdgcn_raw_buffer_store_b32(epoch, header_rsrc(ws, seenOff, 4 * (g + 1)), 4 * g, 0,
                                          16 /* sc1 */);
}

// One whole wave: waits (bounded by spinLimit polls) until the slots of all
// `grid` workgroups hold `epoch`, then stores it as the header's epoch.
// Returns false if the wait expired (the epoch is stored anyway, so that the
// next launch cannot reuse it).
__device__ __forceinline__ bool epoch_publish(void *ws, size_t epochOff, size_t seenOff, uint32_t epoch,
                                              int grid, uint32_t spinLimit)
{
    const int lane = (int)(threadIdx.x & 63);
    const __amdgpu_buffer_rsrc_t seen = header_rsrc(ws, seenOff, 4 * grid);
    bool done = false;
    for (uint32_t spins = 0;; ++spins) {
        bool ok = true;
        for (int i = lane; i < grid; i += 64) {
            ok = ok && (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(seen, 4 * i, 0, 16) == epoch;
        }
        if (__all(ok)) {
            done = true;
            break;
        }
        if (spins >= spinLimit) {
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(epoch, header_rsrc(ws, epochOff, 4), 0, 0, 16);
    }
    return done;
}

// Quiet NaN written into the outputs of rows whose exchange wait expired.
__device__ __forceinline__ float poison() { return __uint_as_float(0x7FC00000u); }

// The caller's sticky status word (mhcPreExecutorSetStatusWord), if set: a
// workgroup whose bounded wait expired stores the public timeout status in
// it (a buffer store, device scope); nothing else writes it.
__device__ __forceinline__ void st_status_word(uint32_t *w)
{
    if (w != nullptr) {
        __builtin_amdgcn_raw_buffer_store_b32(
            (uint32_t)MHC_STATUS_DEVICE_TIMEOUT,
            __builtin_amdgcn_make_buffer_rsrc(w, (short)0, 4, 0x00020000), 0, 0, 16 /* sc1 */);
    }
}

// Sigmoid in the reference vector order (code/op_kernel/mhc_pre.cpp:542-555):
// scale, +bias, negate, exp, +1, reciprocal, +eps (only when eps != 0).
__device__ __forceinline__ float ref_sigmoid(float scaled, float bias, float eps)
{
    float v = scaled + bias;
    v = -v;
    v = expf(v);
    v = v + 1.0f;
    v = 1.0f / v;
    if (eps != 0.0f) {
        v = v + eps;
    }
    return v;
}

// invRms = 1 / sqrt(sumsq * invFlatDim + normEps) (code/op_kernel/mhc_pre.cpp:504-519).
__device__ __forceinline__ float ref_inv_rms(float sumsq, float invFlatDim, float normEps)
{
    float v = sumsq * invFlatDim;
    v = v + normEps;
    v = sqrtf(v);
    return 1.0f / v;
}

}  // namespace dev
}  // namespace mhc
