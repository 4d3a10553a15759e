// Device helpers shared by the MhcPre kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {
namespace dev {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

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
        r[w] = f32_to_bf16_bits(f[2 * w]) | (f32_to_bf16_bits(f[2 * w + 1]) << 16);
    }
    return r;
}

// acc + sum of the squares of 8 packed 16-bit values, two per v_dot2 (the
// products of two 16-bit floats are exact in fp32).
template <bool kBf16>
__device__ __forceinline__ float sumsq8(const u32x4_t &v, float acc)
{
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if constexpr (kBf16) {
            const bf16x2_t p = __builtin_bit_cast(bf16x2_t, v[w]);
            acc = __builtin_amdgcn_fdot2_f32_bf16(p, p, acc, false);
        } else {
            const f16x2_t p = __builtin_bit_cast(f16x2_t, v[w]);
            acc = __builtin_amdgcn_fdot2(p, p, acc, false);
        }
    }
    return acc;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t &v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4_t mfma16(const u32x4_t &a, const u32x4_t &b, const f32x4_t &c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// fp16 x -> exact bf16 pair: x = hi + lo (an fp16 significand has 11 bits).
__device__ __forceinline__ void split_f16_to_bf16(const float (&f)[8], u32x4_t &hi, u32x4_t &lo)
{
    float h[8], l[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        h[e] = bf16_bits_to_f32(f32_to_bf16_bits(f[e]));
        l[e] = f[e] - h[e];
    }
    hi = pack8_bf16(h);
    lo = pack8_bf16(l);
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
