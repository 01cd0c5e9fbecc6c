// Elementwise and broadcast ops: add_f32, swiglu_f32, rope_neox_f32, get_rows_{f16,f32}_f32,
// cpy_f32_f32.
//
// Each op has a contiguous fast path (flat float4 streams, one read and one write per element)
// and a general path that evaluates the contract's index math element by element. Where the
// shader divides with fastdiv magic words, the host decodes each (mp, L) pair back to the
// divisor it encodes and the kernel divides by that (exactly, for every index); a pair that
// encodes no divisor at all, such as a zeroed block, is rejected.
#include <algorithm>
#include <cmath>

#include "common.hpp"

namespace muyo
{
namespace
{
constexpr int kBlock = 256;

/// Element `idx` of a `(1, y, z)` dispatch over the `z*262144 + y*512 + x` index space.
__device__ __forceinline__ bool Covered(uint64_t idx, uint32_t gy, uint32_t gz)
{
    return (idx % 262144u) < 512ull * gy && idx / 262144u < gz;
}

/// Upper bound of the covered prefix, for sizing the launch.
uint64_t CoveredLimit(uint64_t n, uint32_t gy, uint32_t gz)
{
    if (gy >= 512)
    {
        return std::min<uint64_t>(n, 262144ull * gz);
    }
    return std::min<uint64_t>(n, 262144ull * (gz - 1) + 512ull * gy);
}

// ------------------------------------------------------------------------------------------------
// add (shaders/llama/add.comp:23-46, generic_binary_head.glsl:43-65)

struct AddArgs
{
    uint64_t n;
    uint32_t ne00, ne01, ne02, ne03;
    uint32_t nb00, nb01, nb02, nb03;
    uint32_t ne10, ne11, ne12, ne13;
    uint32_t nb10, nb11, nb12, nb13;
    uint32_t nb20, nb21, nb22, nb23;
    uint32_t aoff, boff, doff;
    uint32_t norepeat;
    uint32_t gy, gz;
};

// The flat paths stream with non-temporal loads and stores: nothing they touch is read again by
// the same launch, and keeping it out of L2 lifts a 44 MB add from 55 % to 63 % of 8 TB/s.
__global__ __launch_bounds__(kBlock) void AddFlat4(const float4v* __restrict__ a, const float4v* __restrict__ b,
                                                   float4v* __restrict__ d, uint64_t n4)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride)
    {
        const float4v x = __builtin_nontemporal_load(a + i);
        const float4v y = __builtin_nontemporal_load(b + i);
        __builtin_nontemporal_store(x + y, d + i);
    }
}

__global__ __launch_bounds__(kBlock) void AddGeneral(const float* __restrict__ a, const float* __restrict__ b,
                                                     float* __restrict__ d, AddArgs p)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; idx < p.n; idx += stride)
    {
        if (!Covered(idx, p.gy, p.gz))
        {
            continue;
        }
        const uint64_t s012 = static_cast<uint64_t>(p.ne02) * p.ne01 * p.ne00;
        const uint64_t s01 = static_cast<uint64_t>(p.ne01) * p.ne00;
        const uint64_t i03 = idx / s012;
        const uint64_t r3 = idx - i03 * s012;
        const uint64_t i02 = r3 / s01;
        const uint64_t r2 = r3 - i02 * s01;
        const uint64_t i01 = r2 / p.ne00;
        const uint64_t i00 = r2 - i01 * p.ne00;
        const uint64_t src0 = i03 * p.nb03 + i02 * p.nb02 + i01 * p.nb01 + i00 * p.nb00;
        uint64_t src1;
        if (p.norepeat)
        {
            src1 = i03 * p.nb13 + i02 * p.nb12 + i01 * p.nb11 + i00 * p.nb10;
        }
        else
        {
            src1 = (i03 % p.ne13) * p.nb13 + (i02 % p.ne12) * p.nb12 + (i01 % p.ne11) * p.nb11 +
                   (i00 % p.ne10) * p.nb10;
        }
        const uint64_t dst = i03 * p.nb23 + i02 * p.nb22 + i01 * p.nb21 + i00 * p.nb20;
        d[p.doff + dst] = a[p.aoff + src0] + b[p.boff + src1];
    }
}

/// True when element (i0, i1, i2, i3) of a tensor with these extents and strides sits at
/// i0 + ne0 * (i1 + ne1 * (i2 + ne2 * i3)); a dimension of extent 1 has no say in that.
bool Contiguous(uint32_t ne0, uint32_t ne1, uint32_t ne2, uint32_t ne3, uint32_t nb0, uint32_t nb1, uint32_t nb2,
                uint32_t nb3)
{
    const uint64_t s1 = ne0;
    const uint64_t s2 = s1 * ne1;
    const uint64_t s3 = s2 * ne2;
    return (ne0 <= 1 || nb0 == 1) && (ne1 <= 1 || nb1 == s1) && (ne2 <= 1 || nb2 == s2) && (ne3 <= 1 || nb3 == s3);
}

uint32_t GridFor(uint64_t items)
{
    return static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>((items + kBlock - 1) / kBlock, 8192)));
}

// ------------------------------------------------------------------------------------------------
// swiglu (shaders/llama/swiglu.comp, glu_main.glsl:1-35)

__device__ __forceinline__ float SwiGlu(float a, float b) { return a / (1.0f + expf(-a)) * b; }

struct GluArgs
{
    uint64_t n;
    uint32_t div[3];  // divisors of ne2_012mp, ne2_01mp, ne2_0mp
    uint32_t ne00, ne20, ne21, ne22;
    uint32_t mode;
    uint32_t nb00, nb01, nb02, nb03;
    uint32_t nb10, nb11, nb12, nb13;
    uint32_t nb20, nb21, nb22, nb23;
    uint32_t aoff, boff, doff;
    uint32_t gy, gz;
};

__global__ __launch_bounds__(kBlock) void SwiGluFlat4(const float4v* __restrict__ a, const float4v* __restrict__ b,
                                                      float4v* __restrict__ d, uint64_t n4)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride)
    {
        const float4v g = __builtin_nontemporal_load(a + i);
        const float4v u = __builtin_nontemporal_load(b + i);
        const float4v o = {SwiGlu(g.x, u.x), SwiGlu(g.y, u.y), SwiGlu(g.z, u.z), SwiGlu(g.w, u.w)};
        __builtin_nontemporal_store(o, d + i);
    }
}

__global__ __launch_bounds__(kBlock) void SwiGluGeneral(const float* __restrict__ a, const float* __restrict__ b,
                                                        float* __restrict__ d, GluArgs p)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < p.n; i += stride)
    {
        if (!Covered(i, p.gy, p.gz))
        {
            continue;
        }
        // glu_main.glsl:9-16: quotients by the encoded divisors, offsets by the shape.
        const uint64_t s012 = static_cast<uint64_t>(p.ne22) * p.ne21 * p.ne20;
        const uint64_t s01 = static_cast<uint64_t>(p.ne21) * p.ne20;
        const uint64_t i23 = i / p.div[0];
        if (i23 * s012 > i)
        {
            continue;
        }
        const uint64_t r3 = i - i23 * s012;
        const uint64_t i22 = r3 / p.div[1];
        if (i22 * s01 > r3)
        {
            continue;
        }
        const uint64_t r2 = r3 - i22 * s01;
        const uint64_t i21 = r2 / p.div[2];
        if (i21 * p.ne20 > r2)
        {
            continue;
        }
        const uint64_t i20 = r2 - i21 * p.ne20;
        const uint64_t srcA = p.aoff + i23 * p.nb03 + i22 * p.nb02 + i21 * p.nb01 + i20 * p.nb00;
        const uint64_t srcB = p.boff + i23 * p.nb13 + i22 * p.nb12 + i21 * p.nb11 + i20 * p.nb10;
        const uint64_t dst = p.doff + i23 * p.nb23 + i22 * p.nb22 + i21 * p.nb21 + i20 * p.nb20;
        const uint64_t half = static_cast<uint64_t>(p.ne00 / 2) * p.nb00;
        float value;
        if (p.mode == LLAMA_GLU_MODE_DEFAULT_HALVES)
        {
            value = SwiGlu(a[srcA], a[srcA + half]);
        }
        else if (p.mode == LLAMA_GLU_MODE_SWAPPED_HALVES)
        {
            value = SwiGlu(a[srcA + half], a[srcA]);
        }
        else
        {
            value = SwiGlu(a[srcA], b[srcB]);
        }
        d[dst] = value;
    }
}

// ------------------------------------------------------------------------------------------------
// rope_neox (shaders/llama/rope_neox.comp:6-17, rope_funcs.glsl:17-35,76-114)

constexpr uint32_t kRopeTablePairs = 256;

struct RopeArgs
{
    LlamaRopePushConstants pc;
    uint32_t gx, gy, gz;
    uint32_t pairs;  // per row: min(256*gy, ceil(ne00/2))
};

__device__ __forceinline__ float YarnRamp(float low, float high, uint32_t i0)
{
    const float y = (static_cast<float>(i0 / 2) - low) / fmaxf(0.001f, high - low);
    return 1.0f - fminf(1.0f, fmaxf(0.0f, y));
}

/// cos and sin of pair iw's angle at position `pos`, scaled by mscale (rope_funcs.glsl:17-35's
/// rope_yarn); `power` is thetaScale^(iw / 2). Both rope kernels use it, so they agree bit for bit.
__device__ __forceinline__ void RopeAngleWith(const LlamaRopePushConstants& p, float freqFactor, uint32_t iw,
                                              float power, int32_t pos, float& c, float& s)
{
    const float thetaBase = static_cast<float>(pos) * power;
    const float thetaExtrap = thetaBase / freqFactor;
    float mscale = p.attnFactor;
    const float thetaInterp = p.freqScale * thetaExtrap;
    float theta = thetaInterp;
    if (p.extFactor != 0.0f)
    {
        const float rampMix = YarnRamp(p.corrDims[0], p.corrDims[1], iw) * p.extFactor;
        theta = thetaInterp * (1.0f - rampMix) + thetaExtrap * rampMix;
        mscale *= 1.0f + 0.1f * logf(1.0f / p.freqScale);
    }
    if (p.isBack != 0)
    {
        theta = -theta;
    }
    float cs;
    float sn;
    sincosf(theta, &sn, &cs);  // one range reduction for both
    c = cs * mscale;
    s = sn * mscale;
}

__device__ __forceinline__ void RopeAngle(const LlamaRopePushConstants& p, const float* __restrict__ ff, uint32_t iw,
                                          float power, int32_t pos, float& c, float& s)
{
    RopeAngleWith(p, p.hasFf != 0 ? ff[iw / 2] : 1.0f, iw, power, pos, c, s);
}

/// The rotation of one pair, with its fused multiply-adds written out so that both rope kernels
/// round identically: (x0 c - x1 s, x0 s + x1 c).
__device__ __forceinline__ void RopeRotate(float x0, float x1, float c, float s, float& y0, float& y1)
{
    y0 = fmaf(x0, c, -(x1 * s));
    y1 = fmaf(x0, s, x1 * c);
}

/// Heads of one token a RopeNeoxRows thread rotates with the same angles.
constexpr uint32_t kRopeHeadsPerThread = 4;

/// The common case as a stream: every row rotated whole (nOffs 0, nDims = ne00), rows and
/// offsets on 16-byte boundaries, no set_rows, whole tokens. Thread t takes quad q (pairs
/// 4q..4q+3: four floats from each half of a row) of up to four heads of one token, so each
/// angle's cos and sin serve four rows; rows are loaded and stored 16 bytes at a time with
/// non-temporal hints. The position and frequency factors are requested before the rows (loads
/// complete in order, so the angles would otherwise wait for the rows), and the table of powers
/// and the angles are computed while the rows are in flight.
__global__ __launch_bounds__(kBlock) void RopeNeoxRows(const float* __restrict__ x, const int32_t* __restrict__ positions,
                                                       const float* __restrict__ ff, float* __restrict__ d,
                                                       LlamaRopePushConstants p, uint32_t tokens)
{
    __shared__ float thetaPow[kRopeTablePairs];
    const uint32_t half = p.nDims / 2;
    const uint32_t quads = half / 4;
    const uint32_t groups = (p.ne01 + kRopeHeadsPerThread - 1) / kRopeHeadsPerThread;
    const uint32_t item = blockIdx.x * kBlock + threadIdx.x;
    const bool live = item < tokens * groups * quads;
    const uint32_t q = item % quads;
    const uint32_t tg = min(item / quads, tokens * groups - 1);
    const uint32_t token = tg / groups;
    const uint32_t h0 = (tg - token * groups) * kRopeHeadsPerThread;
    const uint32_t i3 = token / p.ne02;
    const uint32_t i2 = token - i3 * p.ne02;
    const uint64_t xRow = p.aOffset + static_cast<uint64_t>(i3) * p.nb03 + static_cast<uint64_t>(i2) * p.nb02 + 4u * q;
    const uint64_t dRow = p.dOffset + static_cast<uint64_t>(i3) * p.nb13 + static_cast<uint64_t>(i2) * p.nb12 + 4u * q;
    const int32_t pos = positions[i2];
    float freq[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
    {
        freq[e] = p.hasFf != 0 ? ff[4u * q + static_cast<uint32_t>(e)] : 1.0f;
    }
    float4v lo[kRopeHeadsPerThread];
    float4v hi[kRopeHeadsPerThread];
#pragma unroll
    for (uint32_t k = 0; k < kRopeHeadsPerThread; ++k)
    {
        const uint32_t h = min(h0 + k, p.ne01 - 1);
        const float* row = x + xRow + static_cast<uint64_t>(h) * p.nb01;
        lo[k] = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(row));
        hi[k] = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(row + half));
    }
    for (uint32_t j = threadIdx.x; j < half; j += kBlock)
    {
        thetaPow[j] = powf(p.thetaScale, static_cast<float>(j));
    }
    __syncthreads();
    if (!live)
    {
        return;
    }
    float c[4];
    float sn[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
    {
        const uint32_t j = 4u * q + static_cast<uint32_t>(e);
        RopeAngleWith(p, freq[e], 2u * j, thetaPow[j], pos, c[e], sn[e]);
    }
#pragma unroll
    for (uint32_t k = 0; k < kRopeHeadsPerThread; ++k)
    {
        if (h0 + k < p.ne01)
        {
            float4v outLo, outHi;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                float y0, y1;
                RopeRotate(lo[k][e], hi[k][e], c[e], sn[e], y0, y1);
                outLo[e] = y0;
                outHi[e] = y1;
            }
            float* row = d + dRow + static_cast<uint64_t>(h0 + k) * p.nb11;
            __builtin_nontemporal_store(outLo, reinterpret_cast<float4v*>(row));
            __builtin_nontemporal_store(outHi, reinterpret_cast<float4v*>(row + half));
        }
    }
}

__global__ __launch_bounds__(kBlock) void RopeNeox(const float* __restrict__ x, const int32_t* __restrict__ positions,
                                                   const float* __restrict__ ff, float* __restrict__ d,
                                                   const uint32_t* __restrict__ setRows, RopeArgs args)
{
    const LlamaRopePushConstants& p = args.pc;
    // thetaScale^j depends only on the pair index within the rotated span: computed once per
    // workgroup (the shader's pow(theta_scale, i0 / 2) at each j).
    __shared__ float thetaPow[kRopeTablePairs];
    const uint32_t tablePairs = min(p.nDims / 2, kRopeTablePairs);
    for (uint32_t j = threadIdx.x; j < tablePairs; j += kBlock)
    {
        thetaPow[j] = powf(p.thetaScale, static_cast<float>(j));
    }
    __syncthreads();
    // The host keeps nrows * pairs below 2^32.
    const uint32_t item = blockIdx.x * kBlock + threadIdx.x;
    if (item >= p.nrows * args.pairs)
    {
        return;
    }
    const uint32_t row = item / args.pairs;
    const uint32_t i0 = 2u * (item - row * args.pairs);
    // row = x + 32768 * z over the dispatched workgroups.
    const bool rowCovered = args.gz == 1 ? row < args.gx : ((row % 32768u) < args.gx && row / 32768u < args.gz);
    if (!rowCovered || i0 >= p.ne00)
    {
        return;
    }
    const uint32_t i3 = row / (p.ne01 * p.ne02);
    const uint32_t i2 = (row - i3 * p.ne01 * p.ne02) / p.ne01;
    const uint32_t i1 = row - i3 * p.ne01 * p.ne02 - i2 * p.ne01;

    uint64_t idst = i0 / 2 + static_cast<uint64_t>(i1) * p.nb11 + static_cast<uint64_t>(i2) * p.nb12 +
                    static_cast<uint64_t>(i3) * p.nb13;
    const uint64_t ix = p.aOffset + static_cast<uint64_t>(i3) * p.nb03 + static_cast<uint64_t>(i2) * p.nb02 +
                        static_cast<uint64_t>(i1) * p.nb01 + i0 / 2;
    if (p.setRowsStride != 0)
    {
        idst = static_cast<uint64_t>(i1) * p.nb11 + i0 / 2;
        idst += static_cast<uint64_t>(setRows[2 * i2]) * p.setRowsStride;
    }
    idst += p.dOffset;

    if (i0 < p.nOffs || i0 >= p.nOffs + p.nDims)
    {
        d[idst + i0 / 2 + 0] = x[ix + i0 / 2 + 0];
        d[idst + i0 / 2 + 1] = x[ix + i0 / 2 + 1];
        return;
    }
    const uint32_t iw = i0 - p.nOffs;
    const float power = (iw & 1u) == 0 && iw / 2 < tablePairs ? thetaPow[iw / 2]
                                                               : powf(p.thetaScale, static_cast<float>(iw) / 2.0f);
    float c, s;
    RopeAngle(p, ff, iw, power, positions[i2], c, s);
    const float x0 = x[ix + p.nOffs / 2];
    const float x1 = x[ix + p.nOffs / 2 + p.nDims / 2];
    float y0, y1;
    RopeRotate(x0, x1, c, s, y0, y1);
    d[idst + p.nOffs / 2] = y0;
    d[idst + p.nOffs / 2 + p.nDims / 2] = y1;
}

// ------------------------------------------------------------------------------------------------
// get_rows (shaders/llama/get_rows.comp:8-42)

struct GetRowsArgs
{
    uint32_t ne00, ne01, ne10, ne11, ne12;
    uint32_t nb01, nb02, nb03;
    uint32_t nb10, nb11, nb12;
    uint32_t nb21, nb22, nb23;
    uint32_t aoff, boff, doff;
    uint32_t width;  // min(ne00, 512 * dispatch x)
};

template <typename AT>
__device__ __forceinline__ float Widen(AT v);

template <>
__device__ __forceinline__ float Widen<uint16_t>(uint16_t v)
{
    return HalfBitsToFloat(v);
}

template <>
__device__ __forceinline__ float Widen<float>(float v)
{
    return v;
}

template <typename AT>
__global__ __launch_bounds__(kBlock) void GetRows(const AT* __restrict__ a, const int32_t* __restrict__ b,
                                                  float* __restrict__ d, GetRowsArgs p)
{
    // blockIdx.y enumerates (i10, i11, i12); blockIdx.x * kBlock + threadIdx.x is i00.
    const uint32_t i00 = blockIdx.x * kBlock + threadIdx.x;
    if (i00 >= p.width)
    {
        return;
    }
    const uint64_t outer = static_cast<uint64_t>(p.ne10) * p.ne11 * p.ne12;
    for (uint64_t o = blockIdx.y; o < outer; o += gridDim.y)
    {
        const uint32_t i10 = static_cast<uint32_t>(o % p.ne10);
        const uint32_t gz = static_cast<uint32_t>(o / p.ne10);  // i11 * ne12 + i12
        const uint32_t i11 = gz / p.ne12;
        const uint32_t i12 = gz % p.ne12;
        const int32_t i01 = b[p.boff + static_cast<uint64_t>(i10) * p.nb10 + static_cast<uint64_t>(i11) * p.nb11 +
                              static_cast<uint64_t>(i12) * p.nb12];
        const uint64_t dOff = p.doff + static_cast<uint64_t>(i10) * p.nb21 + static_cast<uint64_t>(i11) * p.nb22 +
                              static_cast<uint64_t>(i12) * p.nb23;
        if (i01 < 0 || static_cast<uint32_t>(i01) >= p.ne01)
        {
            d[dOff + i00] = 0.0f;
            continue;
        }
        const uint64_t aOff = p.aoff + static_cast<uint64_t>(i01) * p.nb01 + static_cast<uint64_t>(i11) * p.nb02 +
                              static_cast<uint64_t>(i12) * p.nb03;
        d[dOff + i00] = Widen<AT>(a[aOff + i00]);
    }
}

template <typename AT>
int LaunchGetRows(const char* name, const LlamaAddPushConstants* pc, const AT* a, const int32_t* b, float* d,
                  uint32_t gx, uint32_t gy, uint32_t gz, void* stream)
{
    if (pc == nullptr || a == nullptr || b == nullptr || d == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: push constants, A, B and D are required", name);
    }
    if (gx == 0 || gy == 0 || gz == 0 || pc->ne00 == 0 || pc->ne10 == 0 || pc->ne11 == 0 || pc->ne12 == 0)
    {
        return MUYO_OK;
    }
    GetRowsArgs p{};
    p.ne00 = pc->ne00;
    p.ne01 = pc->ne01;
    p.ne10 = pc->ne10;
    p.ne11 = pc->ne11;
    p.ne12 = pc->ne12;
    p.nb01 = pc->nb01;
    p.nb02 = pc->nb02;
    p.nb03 = pc->nb03;
    p.nb10 = pc->nb10;
    p.nb11 = pc->nb11;
    p.nb12 = pc->nb12;
    p.nb21 = pc->nb21;
    p.nb22 = pc->nb22;
    p.nb23 = pc->nb23;
    p.aoff = pc->misalignOffsets >> 16;
    p.boff = (pc->misalignOffsets >> 8) & 0xFFu;
    p.doff = pc->misalignOffsets & 0xFFu;
    p.width = static_cast<uint32_t>(std::min<uint64_t>(pc->ne00, 512ull * gx));
    const uint64_t outer = static_cast<uint64_t>(pc->ne10) * pc->ne11 * pc->ne12;
    const dim3 grid(CeilDiv(p.width, kBlock), static_cast<uint32_t>(std::min<uint64_t>(outer, 65535)), 1);
    hipLaunchKernelGGL((GetRows<AT>), grid, dim3(kBlock), 0, AsStream(stream), a, b, d, p);
    return LaunchStatus(name);
}

// ------------------------------------------------------------------------------------------------
// cpy (shaders/llama/copy.comp:8-25, generic_unary_head.glsl:34-55)

struct CopyArgs
{
    uint64_t n;  // covered elements: min(ne, 512 * max(x, y))
    uint32_t div0[3];  // divisors of ne0_012mp, ne0_01mp, ne0_0mp
    uint32_t div1[3];  // divisors of ne1_012mp, ne1_01mp, ne1_0mp
    uint32_t ne00, ne01, ne02;
    uint32_t nb00, nb01, nb02, nb03;
    uint32_t ne10, ne11, ne12;
    uint32_t nb10, nb11, nb12, nb13;
    uint32_t aoff, doff;
};

/// src0_idx / dst_idx of generic_unary_head.glsl:34-55: quotients by the encoded divisors,
/// offsets by the shape. Returns false where the shader's unsigned arithmetic would wrap.
__device__ __forceinline__ bool UnaryIndex(uint64_t idx, const uint32_t* div, uint32_t ne0, uint32_t ne1, uint32_t ne2,
                                           uint32_t nb0, uint32_t nb1, uint32_t nb2, uint32_t nb3, uint64_t& out)
{
    const uint64_t p012 = static_cast<uint64_t>(ne2) * ne1 * ne0;
    const uint64_t p01 = static_cast<uint64_t>(ne1) * ne0;
    const uint64_t i3 = idx / div[0];
    if (i3 * p012 > idx)
    {
        return false;
    }
    const uint64_t r3 = idx - i3 * p012;
    const uint64_t i2 = r3 / div[1];
    if (i2 * p01 > r3)
    {
        return false;
    }
    const uint64_t r2 = r3 - i2 * p01;
    const uint64_t i1 = r2 / div[2];
    if (i1 * ne0 > r2)
    {
        return false;
    }
    const uint64_t i0 = r2 - i1 * ne0;
    out = i3 * nb3 + i2 * nb2 + i1 * nb1 + i0 * nb0;
    return true;
}

__global__ __launch_bounds__(kBlock) void CopyStrided(const float* __restrict__ a, float* __restrict__ d, CopyArgs p)
{
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (idx >= p.n)
    {
        return;
    }
    uint64_t src, dst;
    if (!UnaryIndex(idx, p.div0, p.ne00, p.ne01, p.ne02, p.nb00, p.nb01, p.nb02, p.nb03, src) ||
        !UnaryIndex(idx, p.div1, p.ne10, p.ne11, p.ne12, p.nb10, p.nb11, p.nb12, p.nb13, dst))
    {
        return;
    }
    d[p.doff + dst] = a[p.aoff + src];
}

/// The divisor d whose init_fastdiv_values are (mp, l), if there is one. The shader divides by
/// whatever divisor the words encode (src/FullModel.cpp:398-401 encodes ne11 where
/// src/KvCache.cpp:214-216 encodes ne10), so the kernels use the decoded divisor, not the shape.
bool DecodeFastDiv(uint32_t mp, uint32_t l, uint32_t& divisor)
{
    if (l > 32)
    {
        return false;
    }
    // mp - 1 = floor(2^32 (2^l - d) / d), so d ~= 2^(32+l) / (2^32 + mp - 1); try the neighbours.
    const unsigned __int128 numerator = static_cast<unsigned __int128>(1) << (32 + l);
    const uint64_t denominator = (uint64_t{1} << 32) + mp - 1;
    const uint64_t guess = static_cast<uint64_t>(numerator / denominator);
    for (uint64_t d = guess > 2 ? guess - 2 : 1; d <= guess + 2; ++d)
    {
        if (d == 0 || d > 0xFFFFFFFFull)
        {
            continue;
        }
        uint32_t wantMp, wantL;
        FastDivMagic(static_cast<uint32_t>(d), wantMp, wantL);
        if (wantMp == mp && wantL == l)
        {
            divisor = static_cast<uint32_t>(d);
            return true;
        }
    }
    return false;
}

}  // namespace
}  // namespace muyo

using namespace muyo;

extern "C" int muyo_add_f32(const LlamaAddPushConstants* pc, uint32_t norepeat, const float* a, const float* b,
                            float* d, float* /*partial_sums*/, uint32_t dispatch_x, uint32_t dispatch_y,
                            uint32_t dispatch_z, void* stream)
{
    const char* name = "add_f32";
    if (pc == nullptr || a == nullptr || b == nullptr || d == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: push constants, A, B and D are required", name);
    }
    if (dispatch_x == 0 || dispatch_y == 0 || dispatch_z == 0 || pc->ne == 0)
    {
        return MUYO_OK;
    }
    if (dispatch_x != 1)
    {
        return Fail(MUYO_E_DISPATCH, "%s: x must be 1 (the shader's 256 threads x 2 cover a 512-element y block)",
                    name);
    }
    if (pc->ne00 == 0 || pc->ne01 == 0 || pc->ne02 == 0 || pc->ne03 == 0 ||
        (!norepeat && (pc->ne10 == 0 || pc->ne11 == 0 || pc->ne12 == 0 || pc->ne13 == 0)))
    {
        return Fail(MUYO_E_CONTRACT, "%s: every ne0x (and ne1x when repeating) must be >= 1", name);
    }
    const uint64_t limit = CoveredLimit(pc->ne, dispatch_y, dispatch_z);
    const bool sameShape = pc->ne00 == pc->ne10 && pc->ne01 == pc->ne11 && pc->ne02 == pc->ne12 &&
                           pc->ne03 == pc->ne13;
    const bool flat =
        limit == pc->ne && pc->misalignOffsets == 0 && (pc->ne & 3u) == 0 &&
        static_cast<uint64_t>(pc->ne00) * pc->ne01 * pc->ne02 * pc->ne03 == pc->ne &&
        Contiguous(pc->ne00, pc->ne01, pc->ne02, pc->ne03, pc->nb00, pc->nb01, pc->nb02, pc->nb03) &&
        Contiguous(pc->ne00, pc->ne01, pc->ne02, pc->ne03, pc->nb20, pc->nb21, pc->nb22, pc->nb23) &&
        (norepeat || sameShape) &&
        Contiguous(pc->ne00, pc->ne01, pc->ne02, pc->ne03, pc->nb10, pc->nb11, pc->nb12, pc->nb13) &&
        Aligned16(a) && Aligned16(b) && Aligned16(d);
    const hipStream_t s = AsStream(stream);
    if (flat)
    {
        const uint64_t n4 = pc->ne / 4;
        hipLaunchKernelGGL(AddFlat4, dim3(GridFor(n4)), dim3(kBlock), 0, s, reinterpret_cast<const float4v*>(a),
                           reinterpret_cast<const float4v*>(b), reinterpret_cast<float4v*>(d), n4);
        return LaunchStatus(name);
    }
    AddArgs p{};
    p.n = limit;
    p.ne00 = pc->ne00;
    p.ne01 = pc->ne01;
    p.ne02 = pc->ne02;
    p.ne03 = pc->ne03;
    p.nb00 = pc->nb00;
    p.nb01 = pc->nb01;
    p.nb02 = pc->nb02;
    p.nb03 = pc->nb03;
    p.ne10 = pc->ne10;
    p.ne11 = pc->ne11;
    p.ne12 = pc->ne12;
    p.ne13 = pc->ne13;
    p.nb10 = pc->nb10;
    p.nb11 = pc->nb11;
    p.nb12 = pc->nb12;
    p.nb13 = pc->nb13;
    p.nb20 = pc->nb20;
    p.nb21 = pc->nb21;
    p.nb22 = pc->nb22;
    p.nb23 = pc->nb23;
    p.aoff = pc->misalignOffsets >> 16;
    p.boff = (pc->misalignOffsets >> 8) & 0xFFu;
    p.doff = pc->misalignOffsets & 0xFFu;
    p.norepeat = norepeat ? 1u : 0u;
    p.gy = dispatch_y;
    p.gz = dispatch_z;
    hipLaunchKernelGGL(AddGeneral, dim3(GridFor(limit)), dim3(kBlock), 0, s, a, b, d, p);
    return LaunchStatus(name);
}

extern "C" int muyo_swiglu_f32(const LlamaGluPushConstants* pc, const float* a, const float* b, float* d,
                               uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    const char* name = "swiglu_f32";
    if (pc == nullptr || a == nullptr || d == nullptr || (pc->mode == LLAMA_GLU_MODE_SPLIT && b == nullptr))
    {
        return Fail(MUYO_E_NULL, "%s: push constants, A, D (and B in split mode) are required", name);
    }
    if (pc->mode > LLAMA_GLU_MODE_SPLIT)
    {
        return Fail(MUYO_E_CONTRACT, "%s: mode %u is not 0, 1 or 2", name, pc->mode);
    }
    if (dispatch_x == 0 || dispatch_y == 0 || dispatch_z == 0 || pc->N == 0)
    {
        return MUYO_OK;
    }
    if (dispatch_x != 1)
    {
        return Fail(MUYO_E_DISPATCH, "%s: x must be 1 (512-thread workgroups are laid along y)", name);
    }
    uint32_t div[3];
    if (!DecodeFastDiv(pc->ne2_012mp, pc->ne2_012L, div[0]) || !DecodeFastDiv(pc->ne2_01mp, pc->ne2_01L, div[1]) ||
        !DecodeFastDiv(pc->ne2_0mp, pc->ne2_0L, div[2]))
    {
        return Fail(MUYO_E_CONTRACT,
                    "%s: an ne2_* fastdiv pair is not init_fastdiv_values of any divisor (zeroed magic would send "
                    "every element to row 0's address)",
                    name);
    }
    const uint64_t d012 = static_cast<uint64_t>(pc->ne22) * pc->ne21 * pc->ne20;
    const bool canonicalDivisors =
        div[0] == d012 && div[1] == static_cast<uint64_t>(pc->ne21) * pc->ne20 && div[2] == pc->ne20;
    const uint64_t limit = CoveredLimit(pc->N, dispatch_y, dispatch_z);
    const bool flat = limit == pc->N && canonicalDivisors && pc->mode == LLAMA_GLU_MODE_SPLIT && pc->misalignOffsets == 0 &&
                      (pc->N & 3u) == 0 && d012 >= pc->N &&  // so every element has i23 = 0
                      Contiguous(pc->ne20, pc->ne21, pc->ne22, 1, pc->nb00, pc->nb01, pc->nb02, pc->nb03) &&
                      Contiguous(pc->ne20, pc->ne21, pc->ne22, 1, pc->nb10, pc->nb11, pc->nb12, pc->nb13) &&
                      Contiguous(pc->ne20, pc->ne21, pc->ne22, 1, pc->nb20, pc->nb21, pc->nb22, pc->nb23) &&
                      Aligned16(a) && Aligned16(b) && Aligned16(d);
    const hipStream_t s = AsStream(stream);
    if (flat)
    {
        const uint64_t n4 = pc->N / 4;
        hipLaunchKernelGGL(SwiGluFlat4, dim3(GridFor(n4)), dim3(kBlock), 0, s, reinterpret_cast<const float4v*>(a),
                           reinterpret_cast<const float4v*>(b), reinterpret_cast<float4v*>(d), n4);
        return LaunchStatus(name);
    }
    GluArgs p{};
    p.n = limit;
    p.div[0] = div[0];
    p.div[1] = div[1];
    p.div[2] = div[2];
    p.ne00 = pc->ne00;
    p.ne20 = pc->ne20;
    p.ne21 = pc->ne21;
    p.ne22 = pc->ne22;
    p.mode = pc->mode;
    p.nb00 = pc->nb00;
    p.nb01 = pc->nb01;
    p.nb02 = pc->nb02;
    p.nb03 = pc->nb03;
    p.nb10 = pc->nb10;
    p.nb11 = pc->nb11;
    p.nb12 = pc->nb12;
    p.nb13 = pc->nb13;
    p.nb20 = pc->nb20;
    p.nb21 = pc->nb21;
    p.nb22 = pc->nb22;
    p.nb23 = pc->nb23;
    p.aoff = pc->misalignOffsets >> 16;
    p.boff = (pc->misalignOffsets >> 8) & 0xFFu;
    p.doff = pc->misalignOffsets & 0xFFu;
    p.gy = dispatch_y;
    p.gz = dispatch_z;
    hipLaunchKernelGGL(SwiGluGeneral, dim3(GridFor(limit)), dim3(kBlock), 0, s, a, b, d, p);
    return LaunchStatus(name);
}

extern "C" int muyo_rope_neox_f32(const LlamaRopePushConstants* pc, const float* x, const int32_t* positions,
                                  const float* ff, float* d, const uint32_t* set_rows, uint32_t dispatch_x,
                                  uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    const char* name = "rope_neox_f32";
    if (pc == nullptr || x == nullptr || positions == nullptr || d == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: push constants, X, Y (positions) and D are required", name);
    }
    if ((pc->hasFf != 0 && ff == nullptr) || (pc->setRowsStride != 0 && set_rows == nullptr))
    {
        return Fail(MUYO_E_NULL, "%s: Z (hasFf) or I (setRowsStride) binding is NULL", name);
    }
    if (dispatch_x == 0 || dispatch_y == 0 || dispatch_z == 0 || pc->nrows == 0 || pc->ne00 == 0)
    {
        return MUYO_OK;
    }
    if (pc->ne01 == 0 || pc->ne02 == 0)
    {
        return Fail(MUYO_E_CONTRACT, "%s: ne01 and ne02 must be >= 1", name);
    }
    if (dispatch_x > 32768 && dispatch_z > 1)
    {
        return Fail(MUYO_E_DISPATCH, "%s: x must be <= 32768 when z > 1", name);
    }
    RopeArgs args{};
    args.pc = *pc;
    args.gx = dispatch_x;
    args.gy = dispatch_y;
    args.gz = dispatch_z;
    args.pairs = static_cast<uint32_t>(std::min<uint64_t>(256ull * dispatch_y, (pc->ne00 + 1) / 2));
    const uint64_t total = static_cast<uint64_t>(pc->nrows) * args.pairs;
    if (total >= 0xFFFFFFFFull - kBlock)
    {
        return Fail(MUYO_E_RANGE, "%s: %llu (row, pair) items exceed the 32-bit index space", name,
                    static_cast<unsigned long long>(total));
    }
    // Whole rows, 16-byte aligned rows and offsets, every pair dispatched: the streaming kernel.
    const uint32_t half = pc->nDims / 2;
    const bool aligned = Aligned16(x) && Aligned16(d) &&
                         ((pc->aOffset | pc->dOffset | pc->nb01 | pc->nb02 | pc->nb03 | pc->nb11 | pc->nb12 |
                           pc->nb13) & 3u) == 0;
    const uint32_t rows = std::min(pc->nrows, dispatch_x);
    if (pc->nOffs == 0 && pc->nDims == pc->ne00 && half % 4 == 0 && half <= kRopeTablePairs &&
        pc->setRowsStride == 0 && dispatch_z == 1 && args.pairs == half && aligned && rows % pc->ne01 == 0)
    {
        const uint32_t tokens = rows / pc->ne01;
        const uint64_t groups = (pc->ne01 + kRopeHeadsPerThread - 1) / kRopeHeadsPerThread;
        const uint64_t items = static_cast<uint64_t>(tokens) * groups * (half / 4);
        hipLaunchKernelGGL(RopeNeoxRows, dim3(CeilDiv(items, kBlock)), dim3(kBlock), 0, AsStream(stream), x,
                           positions, ff, d, *pc, tokens);
        return LaunchStatus(name);
    }
    hipLaunchKernelGGL(RopeNeox, dim3(CeilDiv(total, kBlock)), dim3(kBlock), 0, AsStream(stream), x, positions, ff, d,
                       set_rows, args);
    return LaunchStatus(name);
}

extern "C" int muyo_get_rows_f16_f32(const LlamaAddPushConstants* pc, const void* a, const int32_t* b, float* d,
                                     uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    return LaunchGetRows<uint16_t>("get_rows_f16_f32", pc, static_cast<const uint16_t*>(a), b, d, dispatch_x,
                                   dispatch_y, dispatch_z, stream);
}

extern "C" int muyo_get_rows_f32(const LlamaAddPushConstants* pc, const float* a, const int32_t* b, float* d,
                                 uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    return LaunchGetRows<float>("get_rows_f32", pc, a, b, d, dispatch_x, dispatch_y, dispatch_z, stream);
}

extern "C" int muyo_cpy_f32_f32(const LlamaCopyPushConstants* pc, const float* a, float* d, uint32_t dispatch_x,
                                uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    const char* name = "cpy_f32_f32";
    if (pc == nullptr || a == nullptr || d == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: push constants, A and D are required", name);
    }
    if (dispatch_x == 0 || dispatch_y == 0 || dispatch_z == 0 || pc->ne == 0)
    {
        return MUYO_OK;
    }
    if (dispatch_z != 1 || (dispatch_x > 1 && dispatch_y > 1))
    {
        return Fail(MUYO_E_DISPATCH, "%s: dispatch must be (n, 1, 1) or (1, n, 1)", name);
    }
    CopyArgs p{};
    const bool words0 = DecodeFastDiv(pc->ne0_012mp, pc->ne0_Ls & 0x3Fu, p.div0[0]) &&
                        DecodeFastDiv(pc->ne0_01mp, (pc->ne0_Ls >> 8) & 0x3Fu, p.div0[1]) &&
                        DecodeFastDiv(pc->ne0_0mp, (pc->ne0_Ls >> 16) & 0x3Fu, p.div0[2]);
    const bool words1 = DecodeFastDiv(pc->ne1_012mp, pc->ne1_Ls & 0x3Fu, p.div1[0]) &&
                        DecodeFastDiv(pc->ne1_01mp, (pc->ne1_Ls >> 8) & 0x3Fu, p.div1[1]) &&
                        DecodeFastDiv(pc->ne1_0mp, (pc->ne1_Ls >> 16) & 0x3Fu, p.div1[2]);
    if (!words0 || !words1)
    {
        return Fail(MUYO_E_CONTRACT,
                    "%s: a fastdiv (mp, L) pair is not init_fastdiv_values of any divisor (a zeroed or corrupted "
                    "block; shifts are packed outermost divisor first)",
                    name);
    }
    p.n = std::min<uint64_t>(pc->ne, 512ull * std::max(dispatch_x, dispatch_y));
    p.ne00 = pc->ne00;
    p.ne01 = pc->ne01;
    p.ne02 = pc->ne02;
    p.nb00 = pc->nb00;
    p.nb01 = pc->nb01;
    p.nb02 = pc->nb02;
    p.nb03 = pc->nb03;
    p.ne10 = pc->ne10;
    p.ne11 = pc->ne11;
    p.ne12 = pc->ne12;
    p.nb10 = pc->nb10;
    p.nb11 = pc->nb11;
    p.nb12 = pc->nb12;
    p.nb13 = pc->nb13;
    p.aoff = pc->misalignOffsets >> 16;
    p.doff = pc->misalignOffsets & 0xFFFFu;
    hipLaunchKernelGGL(CopyStrided, dim3(CeilDiv(p.n, kBlock)), dim3(kBlock), 0, AsStream(stream), a, d, p);
    return LaunchStatus(name);
}
