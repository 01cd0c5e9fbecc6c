// C++ node factories over the muyo_hip C ABI.
//
// A reference node (src/MatVec.cpp:112-159 and the *Execute lambdas of src/FullModel.cpp:133-484)
// is a push-constant block, buffers in descriptor-binding order and a dispatch. Each node here
// holds exactly those and launches the matching gfx950 kernel on a stream, so a render-graph
// node's execute callback becomes `node.Execute(stream)`. The Make* functions fill the push
// constants the way the reference's node factories do.
#pragma once

#include <cmath>
#include <cstdint>
#include <initializer_list>

#include "muyo/LlamaContracts.h"
#include "muyo_hip.h"

namespace muyo_llm
{
namespace hip
{
/// ggml's init_fastdiv_values: the (multiplier, shift) pair the shaders' fastdiv consumes
/// (src/Swiglu.cpp:46-54).
inline void InitFastDiv(uint32_t d, uint32_t& mp, uint32_t& shift)
{
    shift = 0;
    while (shift < 32 && (uint32_t{1} << shift) < d)
    {
        ++shift;
    }
    mp = static_cast<uint32_t>((uint64_t{1} << 32) * ((uint64_t{1} << shift) - d) / d + 1);
}

/// MatVecExecute's fill (src/FullModel.cpp:133-175) for `rows` outputs of `ncols` each.
inline LlamaMatVecPushConstants MakeMatVec(uint32_t ncols, uint32_t rows, uint32_t fusionFlags = 0)
{
    LlamaMatVecPushConstants pc{};
    pc.ncols = ncols;
    pc.strideA = ncols;
    pc.strideB = ncols;
    pc.strideD = rows;
    pc.fusionFlags = fusionFlags;
    pc.ne02 = 1;
    pc.ne12 = 1;
    pc.broadcast2 = 1;
    pc.broadcast3 = 1;
    return pc;
}

/// RmsNormExecute / MakeAddPushConstants (src/FullModel.cpp:215-284, src/ElementwiseAdd.cpp:59-88)
/// for `rows` contiguous rows of `length`; the second operand has `length` elements per row.
inline LlamaAddPushConstants MakeRows(uint32_t length, uint32_t rows = 1, float eps = 0.0F)
{
    LlamaAddPushConstants pc{};
    pc.ne = length * rows;
    pc.ne00 = length;
    pc.ne01 = rows;
    pc.ne02 = 1;
    pc.ne03 = 1;
    pc.nb00 = 1;
    pc.nb01 = length;
    pc.nb02 = length * rows;
    pc.nb03 = length * rows;
    pc.ne10 = length;
    pc.ne11 = 1;
    pc.ne12 = 1;
    pc.ne13 = 1;
    pc.nb10 = 1;
    pc.nb11 = length;
    pc.nb12 = length;
    pc.nb13 = length;
    pc.ne20 = length;
    pc.ne21 = rows;
    pc.ne22 = 1;
    pc.ne23 = 1;
    pc.nb20 = 1;
    pc.nb21 = length;
    pc.nb22 = length * rows;
    pc.nb23 = length * rows;
    pc.param1 = eps;
    return pc;
}

/// The same block for an element-wise add over a [rows][length] tensor (B of the same shape).
inline LlamaAddPushConstants MakeAdd(uint32_t length, uint32_t rows = 1)
{
    LlamaAddPushConstants pc = MakeRows(length, rows);
    pc.ne11 = rows;
    pc.nb12 = length * rows;
    pc.nb13 = length * rows;
    return pc;
}

/// SwigluExecute's fill (src/FullModel.cpp:287-327): split mode over `count` elements.
inline LlamaGluPushConstants MakeSwiglu(uint32_t count)
{
    LlamaGluPushConstants pc{};
    pc.N = count;
    pc.ne00 = count;
    pc.ne20 = count;
    pc.mode = LLAMA_GLU_MODE_SPLIT;
    for (uint32_t* nb : {&pc.nb00, &pc.nb10, &pc.nb20})
    {
        nb[0] = 1;
        nb[1] = count;
        nb[2] = count;
        nb[3] = count;
    }
    pc.ne21 = 1;
    pc.ne22 = 1;
    InitFastDiv(count, pc.ne2_012mp, pc.ne2_012L);
    InitFastDiv(count, pc.ne2_01mp, pc.ne2_01L);
    InitFastDiv(count, pc.ne2_0mp, pc.ne2_0L);
    return pc;
}

/// RopeExecute's fill (src/FullModel.cpp:179-212): NeoX rope of `rows` heads of `headDim`, the
/// output rows `outputRowStride` apart starting `dOffset` elements in (a cache row when the
/// stride is headDim * maxSeq).
inline LlamaRopePushConstants MakeRopeNeox(uint32_t rows, uint32_t headDim, float freqBase,
                                           uint32_t outputRowStride = 0, uint32_t dOffset = 0)
{
    LlamaRopePushConstants pc{};
    pc.ropeMode = LLAMA_ROPE_MODE_NEOX;
    pc.nrows = rows;
    pc.nDims = headDim;
    pc.freqScale = 1.0F;
    pc.freqBase = freqBase;
    pc.extFactor = 0.0F;
    pc.attnFactor = 1.0F;
    pc.thetaScale = std::pow(freqBase, -2.0F / static_cast<float>(headDim));
    pc.ne00 = headDim;
    pc.ne01 = rows;
    pc.ne02 = 1;
    const uint32_t out = outputRowStride != 0 ? outputRowStride : headDim;
    pc.nb01 = headDim;
    pc.nb02 = headDim * rows;
    pc.nb03 = headDim * rows;
    pc.nb11 = out;
    pc.nb12 = out * rows;
    pc.nb13 = out * rows;
    pc.dOffset = dOffset;
    return pc;
}

/// SoftMaxExecute's fill (src/FullModel.cpp:331-349): `rows` rows of `columns`, scaled.
inline LlamaSoftMaxPushConstants MakeSoftMax(uint32_t rows, uint32_t columns, float scale)
{
    LlamaSoftMaxPushConstants pc{};
    pc.KX = columns;
    pc.ne00 = columns;
    pc.ne01 = rows;
    pc.ne02 = 1;
    pc.ne12 = 1;
    pc.ne13 = 1;
    pc.scale = scale;
    pc.nrowsX = rows;
    return pc;
}

/// ArgmaxExecute's fill (src/FullModel.cpp:461-484).
inline LlamaGenericHeadPushConstants MakeArgmax(uint32_t columns, uint32_t rows = 1)
{
    LlamaGenericHeadPushConstants pc{};
    pc.KX = columns;
    pc.KY = rows;
    return pc;
}

/// GetRowsExecute's fill (src/FullModel.cpp:424-458): `count` rows of a [vocab][dim] table.
inline LlamaAddPushConstants MakeGetRows(uint32_t dim, uint32_t vocab, uint32_t count = 1)
{
    LlamaAddPushConstants pc{};
    pc.ne = dim * vocab;
    pc.ne00 = dim;
    pc.ne01 = vocab;
    pc.ne02 = 1;
    pc.ne03 = 1;
    pc.nb00 = 1;
    pc.nb01 = dim;
    pc.nb02 = dim * vocab;
    pc.nb03 = dim * vocab;
    pc.ne10 = count;
    pc.ne11 = 1;
    pc.ne12 = 1;
    pc.ne13 = 1;
    pc.nb10 = 1;
    pc.nb11 = count;
    pc.nb12 = count;
    pc.nb13 = count;
    pc.ne20 = dim;
    pc.ne21 = count;
    pc.ne22 = 1;
    pc.ne23 = 1;
    pc.nb20 = 1;
    pc.nb21 = dim;
    pc.nb22 = dim * count;
    pc.nb23 = dim * count;
    return pc;
}

/// CopyValueColumnExecute's fill (src/FullModel.cpp:353-420, src/KvCache.cpp:184-225): value
/// vector v[kvDim] into column `position` of the transposed cache [kvDim / headDim][headDim][maxSeq].
inline LlamaCopyPushConstants MakeValueColumn(uint32_t kvDim, uint32_t headDim, uint32_t maxSeq, uint32_t position)
{
    LlamaCopyPushConstants pc{};
    pc.ne = kvDim;
    pc.ne00 = kvDim;
    pc.ne01 = 1;
    pc.ne02 = 1;
    pc.ne03 = 1;
    pc.nb00 = 1;
    pc.ne10 = headDim;
    pc.ne11 = maxSeq;
    pc.ne12 = 1;
    pc.ne13 = 1;
    pc.nb10 = maxSeq;
    pc.nb11 = headDim * maxSeq;
    pc.misalignOffsets = position;
    uint32_t l0 = 0;
    uint32_t l1 = 0;
    uint32_t l2 = 0;
    InitFastDiv(pc.ne11, pc.ne1_0mp, l0);
    InitFastDiv(pc.ne11 * pc.ne10, pc.ne1_01mp, l1);
    InitFastDiv(pc.ne12 * pc.ne11 * pc.ne10, pc.ne1_012mp, l2);
    pc.ne1_Ls = l2 | (l1 << 8) | (l0 << 16);
    InitFastDiv(pc.ne00, pc.ne0_0mp, l0);
    InitFastDiv(pc.ne01 * pc.ne00, pc.ne0_01mp, l1);
    InitFastDiv(pc.ne02 * pc.ne01 * pc.ne00, pc.ne0_012mp, l2);
    pc.ne0_Ls = l2 | (l1 << 8) | (l0 << 16);
    return pc;
}

/// The value-column copy fill of src/KvCache.cpp:190-220: v[kvDim] into column `position` of a
/// transposed cache [kvDim][maxSeq] (channel stride maxSeq, position stride 1), divisors
/// including the innermost dimension.
inline LlamaCopyPushConstants MakeCacheValueColumn(uint32_t kvDim, uint32_t maxSeq, uint32_t position)
{
    LlamaCopyPushConstants pc{};
    pc.ne = kvDim;
    pc.ne00 = kvDim;
    pc.ne01 = 1;
    pc.ne02 = 1;
    pc.ne03 = 1;
    pc.nb00 = 1;
    pc.ne10 = kvDim;
    pc.ne11 = maxSeq;
    pc.ne12 = 1;
    pc.ne13 = 1;
    pc.nb10 = maxSeq;
    pc.nb11 = 1;
    pc.misalignOffsets = position;
    uint32_t l0 = 0;
    uint32_t l1 = 0;
    uint32_t l2 = 0;
    InitFastDiv(pc.ne12 * pc.ne11 * pc.ne10, pc.ne1_012mp, l2);
    InitFastDiv(pc.ne11 * pc.ne10, pc.ne1_01mp, l1);
    InitFastDiv(pc.ne10, pc.ne1_0mp, l0);
    pc.ne1_Ls = l2 | (l1 << 8) | (l0 << 16);
    InitFastDiv(pc.ne02 * pc.ne01 * pc.ne00, pc.ne0_012mp, l2);
    InitFastDiv(pc.ne01 * pc.ne00, pc.ne0_01mp, l1);
    InitFastDiv(pc.ne00, pc.ne0_0mp, l0);
    pc.ne0_Ls = l2 | (l1 << 8) | (l0 << 16);
    return pc;
}

struct Dispatch
{
    uint32_t x = 1;
    uint32_t y = 1;
    uint32_t z = 1;
};

/// add.comp's canonical dispatch for `count` elements: (1, ceil(count / 512)), past 512
/// y-blocks split into z.
inline Dispatch ElementDispatch(uint32_t count)
{
    const uint32_t y = (count + 511) / 512;
    return y > 512 ? Dispatch{1, 512, (y + 511) / 512} : Dispatch{1, y, 1};
}

/// One workgroup per row (row = z * 262144 + y * 512 + x).
inline Dispatch RowDispatch(uint32_t rows)
{
    if (rows <= 512)
    {
        return {rows, 1, 1};
    }
    const uint32_t y = (rows + 511) / 512;
    return y <= 512 ? Dispatch{512, y, 1} : Dispatch{512, 512, (rows + 262143) / 262144};
}

// ------------------------------------------------------------------------------------------------
// Nodes: push constants + bindings (in descriptor order) + dispatch.

struct MatVecF16Node
{
    LlamaMatVecPushConstants pc{};
    MuyoMatVecSpec spec{32, 1, 1};
    const void* a = nullptr;  // fp16 weights
    const float* b = nullptr;
    float* d = nullptr;
    const float* fuse0 = nullptr;
    const float* fuse1 = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_mul_mat_vec_f16_f32_f32(&pc, &spec, a, b, d, fuse0, fuse1, dispatch.x, dispatch.y, dispatch.z,
                                            stream);
    }
};

struct MatVecF32Node
{
    LlamaMatVecPushConstants pc{};
    MuyoMatVecSpec spec{32, 1, 1};
    const float* a = nullptr;
    const float* b = nullptr;
    float* d = nullptr;
    const float* fuse0 = nullptr;
    const float* fuse1 = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_mul_mat_vec_f32_f32_f32(&pc, &spec, a, b, d, fuse0, fuse1, dispatch.x, dispatch.y, dispatch.z,
                                            stream);
    }
};

struct RmsNormNode
{
    LlamaAddPushConstants pc{};
    uint32_t doMultiply = 1;
    const float* a = nullptr;
    const float* b = nullptr;  // weight row
    float* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_rms_norm_f32(&pc, doMultiply, a, b, d, nullptr, dispatch.x, dispatch.y, dispatch.z, stream);
    }
};

struct AddNode
{
    LlamaAddPushConstants pc{};
    uint32_t norepeat = 1;
    const float* a = nullptr;
    const float* b = nullptr;
    float* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_add_f32(&pc, norepeat, a, b, d, nullptr, dispatch.x, dispatch.y, dispatch.z, stream);
    }
};

struct SwigluNode
{
    LlamaGluPushConstants pc{};
    const float* a = nullptr;  // gate
    const float* b = nullptr;  // up
    float* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_swiglu_f32(&pc, a, b, d, dispatch.x, dispatch.y, dispatch.z, stream);
    }
};

struct RopeNode
{
    LlamaRopePushConstants pc{};
    const float* x = nullptr;
    const int32_t* positions = nullptr;
    const float* ff = nullptr;
    float* d = nullptr;
    const uint32_t* setRows = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_rope_neox_f32(&pc, x, positions, ff, d, setRows, dispatch.x, dispatch.y, dispatch.z, stream);
    }
};

struct SoftMaxNode
{
    LlamaSoftMaxPushConstants pc{};
    const float* x = nullptr;
    const float* mask = nullptr;
    const float* sinks = nullptr;
    float* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_soft_max_f32(&pc, x, mask, sinks, d, dispatch.x, dispatch.y, dispatch.z, stream);
    }
};

struct ArgmaxNode
{
    LlamaGenericHeadPushConstants pc{};
    const float* a = nullptr;
    int32_t* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const { return muyo_argmax_f32(&pc, a, d, dispatch.x, dispatch.y, dispatch.z, stream); }
};

struct GetRowsF16Node
{
    LlamaAddPushConstants pc{};
    const void* a = nullptr;  // fp16 table
    const int32_t* b = nullptr;
    float* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_get_rows_f16_f32(&pc, a, b, d, dispatch.x, dispatch.y, dispatch.z, stream);
    }
};

struct GetRowsF32Node
{
    LlamaAddPushConstants pc{};
    const float* a = nullptr;
    const int32_t* b = nullptr;
    float* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const
    {
        return muyo_get_rows_f32(&pc, a, b, d, dispatch.x, dispatch.y, dispatch.z, stream);
    }
};

struct CopyNode
{
    LlamaCopyPushConstants pc{};
    const float* a = nullptr;
    float* d = nullptr;
    Dispatch dispatch;
    int Execute(void* stream) const { return muyo_cpy_f32_f32(&pc, a, d, dispatch.x, dispatch.y, dispatch.z, stream); }
};
}  // namespace hip
}  // namespace muyo_llm
