// Shared device and host helpers of the gfx950 kernel set.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "muyo_hip.h"

namespace muyo
{
// ------------------------------------------------------------------------------------------------
// Host-side error reporting: every C entry point returns a status and leaves a message here.

void SetLastError(const char* format, ...);
void ClearLastError();

/// Record `code` with a formatted message and return it (for `return Fail(...)`).
int Fail(int code, const char* format, ...);

/// Translate a HIP failure into the C ABI's positive status.
int HipStatus(hipError_t status, const char* what);

#define MUYO_HIP_CHECK(expr)                                  \
    do                                                        \
    {                                                         \
        const hipError_t muyo_status_ = (expr);               \
        if (muyo_status_ != hipSuccess)                       \
        {                                                     \
            return ::muyo::HipStatus(muyo_status_, #expr);    \
        }                                                     \
    } while (0)

/// Status of the most recent launch on this thread.
inline int LaunchStatus(const char* kernel)
{
    const hipError_t status = hipGetLastError();
    return status == hipSuccess ? MUYO_OK : HipStatus(status, kernel);
}

inline hipStream_t AsStream(void* stream) { return static_cast<hipStream_t>(stream); }

inline bool Aligned16(const void* pointer) { return (reinterpret_cast<uintptr_t>(pointer) & 15u) == 0; }

inline uint32_t CeilDiv(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

/// ggml's fastdiv magic for divisor d: (mulhi(n, mp) + n) >> L == n / d for every 32-bit n
/// (src/Swiglu.cpp:46-54, src/FullModel.cpp:367-375 reproduce the host side of it).
inline void FastDivMagic(uint32_t d, uint32_t& mp, uint32_t& l)
{
    l = 0;
    while (l < 32 && (uint32_t{1} << l) < d)
    {
        ++l;
    }
    mp = static_cast<uint32_t>((uint64_t{1} << 32) * ((uint64_t{1} << l) - d) / d + 1);
}

// ------------------------------------------------------------------------------------------------
// Device helpers. Wavefronts are 64 lanes on CDNA4.

constexpr int kWave = 64;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float HalfBitsToFloat(uint16_t bits)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ uint16_t FloatToHalfBits(float value)
{
    // v_cvt_f16_f32 rounds to nearest even in the default mode.
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(value));
}

/// Sum across groups of `kWidth` consecutive lanes; every lane of a group gets the group's sum.
template <int kWidth>
__device__ __forceinline__ float GroupSum(float value)
{
#pragma unroll
    for (int offset = kWidth / 2; offset > 0; offset >>= 1)
    {
        value += __shfl_xor(value, offset, kWave);
    }
    return value;
}

template <int kWidth>
__device__ __forceinline__ float GroupMax(float value)
{
#pragma unroll
    for (int offset = kWidth / 2; offset > 0; offset >>= 1)
    {
        value = fmaxf(value, __shfl_xor(value, offset, kWave));
    }
    return value;
}

/// (value, index) maximum with ties to the lower index, across groups of kWidth lanes.
template <int kWidth>
__device__ __forceinline__ void GroupArgMax(float& value, int32_t& index)
{
#pragma unroll
    for (int offset = kWidth / 2; offset > 0; offset >>= 1)
    {
        const float other = __shfl_xor(value, offset, kWave);
        const int32_t otherIndex = __shfl_xor(index, offset, kWave);
        if (other > value || (other == value && otherIndex < index))
        {
            value = other;
            index = otherIndex;
        }
    }
}

/// 16-byte global load of 8 halves widened to f32 (exact).
__device__ __forceinline__ void LoadHalf8(const uint16_t* __restrict__ source, float out[8])
{
    const half8 h = *reinterpret_cast<const half8*>(source);
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        out[i] = static_cast<float>(h[i]);
    }
}
}  // namespace muyo
