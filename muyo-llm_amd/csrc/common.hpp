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

/// The value held by a lane of the other half of this lane's group of 2*kStep consecutive lanes.
/// Meant for butterfly reductions in which, before step kStep, every lane of each kStep-lane
/// half already holds the same value: the partner lane then need not be lane ^ kStep, so the
/// steps inside a 16-lane row use DPP (quad permutes, then the half-row and row mirrors). The
/// steps across rows and across the wave's halves are lane ^ 16 and lane ^ 32 exchanges
/// (v_permlane16_swap, v_permlane32_swap): VALU operations, where an LDS swizzle or two lane
/// reads would wait on the LDS pipe or a scalar register.
template <int kStep>
__device__ __forceinline__ int PartnerLane(int value)
{
    static_assert(kStep == 1 || kStep == 2 || kStep == 4 || kStep == 8 || kStep == 16 || kStep == 32, "step");
    if constexpr (kStep == 1)
    {
        return __builtin_amdgcn_update_dpp(value, value, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    }
    else if constexpr (kStep == 2)
    {
        return __builtin_amdgcn_update_dpp(value, value, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    }
    else if constexpr (kStep == 4)
    {
        return __builtin_amdgcn_update_dpp(value, value, 0x141, 0xF, 0xF, false);  // row_half_mirror
    }
    else if constexpr (kStep == 8)
    {
        return __builtin_amdgcn_update_dpp(value, value, 0x140, 0xF, 0xF, false);  // row_mirror
    }
    else if constexpr (kStep == 16)
    {
        // Rows 2r and 2r + 1 exchange: the pair holds (even row's, odd row's) value per lane.
        const auto rows = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(value), static_cast<unsigned>(value),
                                                           false, false);
        return static_cast<int>((__lane_id() & 16u) != 0 ? rows[0] : rows[1]);
    }
    else
    {
        // The wave's halves exchange: the pair holds (low half's, high half's) value per lane.
        const auto halves = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(value),
                                                             static_cast<unsigned>(value), false, false);
        return static_cast<int>((__lane_id() & 32u) != 0 ? halves[0] : halves[1]);
    }
}

template <int kStep>
__device__ __forceinline__ float PartnerLane(float value)
{
    return __int_as_float(PartnerLane<kStep>(__float_as_int(value)));
}

/// Sum across groups of `kWidth` consecutive lanes; every lane of a group gets the group's sum,
/// bit-identical on every lane (each step adds the same two values in either order).
template <int kWidth>
__device__ __forceinline__ float GroupSum(float value)
{
    static_assert(kWidth >= 1 && kWidth <= kWave && (kWidth & (kWidth - 1)) == 0, "width");
    if constexpr (kWidth >= 2) value += PartnerLane<1>(value);
    if constexpr (kWidth >= 4) value += PartnerLane<2>(value);
    if constexpr (kWidth >= 8) value += PartnerLane<4>(value);
    if constexpr (kWidth >= 16) value += PartnerLane<8>(value);
    if constexpr (kWidth >= 32) value += PartnerLane<16>(value);
    if constexpr (kWidth >= 64) value += PartnerLane<32>(value);
    return value;
}

/// GroupSum of N independent values, level by level: each lane permute reads a register written
/// N instructions earlier, so the chain needs no wait states between its steps.
template <int kWidth, int N>
__device__ __forceinline__ void GroupSumN(float (&v)[N])
{
    static_assert(kWidth >= 1 && kWidth <= kWave && (kWidth & (kWidth - 1)) == 0, "width");
#define MUYO_GROUP_SUM_LEVEL(step)                   \
    if constexpr (kWidth >= 2 * (step))              \
    {                                                \
        float other[N];                              \
        _Pragma("unroll") for (int i = 0; i < N; ++i) \
        {                                            \
            other[i] = PartnerLane<step>(v[i]);      \
        }                                            \
        _Pragma("unroll") for (int i = 0; i < N; ++i) \
        {                                            \
            v[i] += other[i];                        \
        }                                            \
    }
    MUYO_GROUP_SUM_LEVEL(1)
    MUYO_GROUP_SUM_LEVEL(2)
    MUYO_GROUP_SUM_LEVEL(4)
    MUYO_GROUP_SUM_LEVEL(8)
    MUYO_GROUP_SUM_LEVEL(16)
    MUYO_GROUP_SUM_LEVEL(32)
#undef MUYO_GROUP_SUM_LEVEL
}

template <int kCtrl>
__device__ __forceinline__ float DppMove(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), kCtrl, 0xF, 0xF, false));
}

/// Sums eight values over each octet of lanes (lanes 8o .. 8o + 7), leaving lane L the octet's
/// total of value L & 7: a reduce-scatter of three halving exchanges, 7 lane permutes where eight
/// separate octet sums take 24.
__device__ __forceinline__ float OctetScatter8(const float (&v)[8])
{
    const uint32_t lane = __lane_id();
    // Partner L ^ 7 (row_half_mirror): lanes with bit 2 set keep values 4..7, the others 0..3.
    const bool b2 = (lane & 4u) != 0;
    float u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const float keep = b2 ? v[i + 4] : v[i];
        const float send = b2 ? v[i] : v[i + 4];
        u[i] = keep + DppMove<0x141>(send);
    }
    // Partner L ^ 2 (quad_perm [2,3,0,1]), split by bit 1.
    const bool b1 = (lane & 2u) != 0;
    float t[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
    {
        const float keep = b1 ? u[i + 2] : u[i];
        const float send = b1 ? u[i] : u[i + 2];
        t[i] = keep + DppMove<0x4E>(send);
    }
    // Partner L ^ 1 (quad_perm [1,0,3,2]), split by bit 0.
    const bool b0 = (lane & 1u) != 0;
    return (b0 ? t[1] : t[0]) + DppMove<0xB1>(b0 ? t[0] : t[1]);
}

/// Sums eight values over the 64 lanes of a wave, leaving lane L the total of value L & 7: the
/// octet reduce-scatter, then three full exchanges (L ^ 8, L ^ 16, L ^ 32). About a third of the
/// lane permutes of eight separate sums.
__device__ __forceinline__ float ScatterSum8(const float (&v)[8])
{
    float r = OctetScatter8(v);
    r += DppMove<0x128>(r);  // row_ror:8
    const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(r), __float_as_uint(r), false, false);
    r = __uint_as_float(rows[0]) + __uint_as_float(rows[1]);
    const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(r), __float_as_uint(r), false, false);
    return __uint_as_float(halves[0]) + __uint_as_float(halves[1]);
}

template <int kWidth>
__device__ __forceinline__ float GroupMax(float value)
{
    static_assert(kWidth >= 1 && kWidth <= kWave && (kWidth & (kWidth - 1)) == 0, "width");
    if constexpr (kWidth >= 2) value = fmaxf(value, PartnerLane<1>(value));
    if constexpr (kWidth >= 4) value = fmaxf(value, PartnerLane<2>(value));
    if constexpr (kWidth >= 8) value = fmaxf(value, PartnerLane<4>(value));
    if constexpr (kWidth >= 16) value = fmaxf(value, PartnerLane<8>(value));
    if constexpr (kWidth >= 32) value = fmaxf(value, PartnerLane<16>(value));
    if constexpr (kWidth >= 64) value = fmaxf(value, PartnerLane<32>(value));
    return value;
}

template <int kStep>
__device__ __forceinline__ void ArgMaxStep(float& value, int32_t& index)
{
    const float other = PartnerLane<kStep>(value);
    const int32_t otherIndex = PartnerLane<kStep>(index);
    if (other > value || (other == value && otherIndex < index))
    {
        value = other;
        index = otherIndex;
    }
}

/// (value, index) maximum with ties to the lower index, across groups of kWidth lanes.
template <int kWidth>
__device__ __forceinline__ void GroupArgMax(float& value, int32_t& index)
{
    static_assert(kWidth >= 1 && kWidth <= kWave && (kWidth & (kWidth - 1)) == 0, "width");
    if constexpr (kWidth >= 2) ArgMaxStep<1>(value, index);
    if constexpr (kWidth >= 4) ArgMaxStep<2>(value, index);
    if constexpr (kWidth >= 8) ArgMaxStep<4>(value, index);
    if constexpr (kWidth >= 16) ArgMaxStep<8>(value, index);
    if constexpr (kWidth >= 32) ArgMaxStep<16>(value, index);
    if constexpr (kWidth >= 64) ArgMaxStep<32>(value, index);
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
