// Portable seeded generator for synthetic weights and inputs.
//
// Counter-based, so every element is computed independently (no sequential state) and the same
// bits come out on the host and on any GPU: the only operations are 64-bit integer arithmetic,
// exact int->double conversion, one correctly rounded multiply and add in double, and
// round-to-nearest-even narrowing to f32 and fp16.
//   word(seed, i) = mix64(mix64(seed) + i), mix64 = SplitMix64's output function
//   normal(i)     = (sum of the 12 32-bit halves of word(6i+0..6i+5)) * 2^-32 - 6
// The Irwin-Hall sum of 12 uniforms has mean 0 and variance 1 (support +-6).
#include "common.hpp"

// Every multiply and add below is rounded on its own (no fused multiply-add), so the device
// reproduces the host generator bit for bit.
#pragma clang fp contract(off)

namespace muyo
{
namespace
{
__host__ __device__ __forceinline__ uint64_t Mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ double IrwinHall(uint64_t key, uint64_t i)
{
    uint64_t sum = 0;
#pragma unroll
    for (uint64_t k = 0; k < 6; ++k)
    {
        const uint64_t w = Mix64(key + 6u * i + k);
        sum += (w >> 32) + (w & 0xFFFFFFFFull);
    }
    return static_cast<double>(sum) * 0x1p-32 - 6.0;
}

constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void FillNormalF32(float* __restrict__ out, uint64_t count, uint64_t key,
                                                        double mean, double stddev)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride)
    {
        out[i] = static_cast<float>(mean + stddev * IrwinHall(key, i));
    }
}

__global__ __launch_bounds__(kBlock) void FillNormalF16(uint16_t* __restrict__ out, uint64_t count, uint64_t key,
                                                        double mean, double stddev)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride)
    {
        const float value = static_cast<float>(mean + stddev * IrwinHall(key, i));
        out[i] = FloatToHalfBits(value);
    }
}

__global__ __launch_bounds__(kBlock) void FillUniformF32(float* __restrict__ out, uint64_t count, uint64_t key)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride)
    {
        const uint64_t w = Mix64(key + i);
        out[i] = static_cast<float>(w >> 40) * 0x1p-23f - 1.0f;
    }
}

uint32_t FillGrid(uint64_t count)
{
    const uint64_t blocks = (count + kBlock - 1) / kBlock;
    return static_cast<uint32_t>(blocks < 1 ? 1 : (blocks > 16384 ? 16384 : blocks));
}
}  // namespace
}  // namespace muyo

using namespace muyo;

extern "C" uint64_t muyo_tensor_seed(uint64_t seed, uint32_t kind, uint32_t layer)
{
    return Mix64(seed ^ ((static_cast<uint64_t>(kind) << 40) | (static_cast<uint64_t>(layer) << 8) | 0x5Aull));
}

extern "C" int muyo_fill_normal_f16(void* d, uint64_t count, uint64_t seed, double mean, double stddev, void* stream)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "fill_normal_f16: destination is NULL");
    }
    if (count == 0)
    {
        return MUYO_OK;
    }
    hipLaunchKernelGGL(FillNormalF16, dim3(FillGrid(count)), dim3(kBlock), 0, AsStream(stream),
                       static_cast<uint16_t*>(d), count, Mix64(seed), mean, stddev);
    return LaunchStatus("fill_normal_f16");
}

extern "C" int muyo_fill_normal_f32(float* d, uint64_t count, uint64_t seed, double mean, double stddev, void* stream)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "fill_normal_f32: destination is NULL");
    }
    if (count == 0)
    {
        return MUYO_OK;
    }
    hipLaunchKernelGGL(FillNormalF32, dim3(FillGrid(count)), dim3(kBlock), 0, AsStream(stream), d, count, Mix64(seed),
                       mean, stddev);
    return LaunchStatus("fill_normal_f32");
}

extern "C" int muyo_fill_uniform_f32(float* d, uint64_t count, uint64_t seed, void* stream)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "fill_uniform_f32: destination is NULL");
    }
    if (count == 0)
    {
        return MUYO_OK;
    }
    hipLaunchKernelGGL(FillUniformF32, dim3(FillGrid(count)), dim3(kBlock), 0, AsStream(stream), d, count,
                       Mix64(seed));
    return LaunchStatus("fill_uniform_f32");
}
