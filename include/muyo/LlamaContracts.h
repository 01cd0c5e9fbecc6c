/*
 * Op contracts of the decode-step kernel set, as plain C structs.
 *
 * Each struct carries, field for field and in the same order, the push-constant block the
 * reference fills for one op (src/LlamaContracts.h:22-294 in muyo-llm, plus the unary `copy`
 * block declared privately in src/FullModel.cpp:353-365 and src/KvCache.cpp:47-56). Keeping the
 * layout identical is what makes every node a drop-in: a caller that already fills these blocks
 * passes the same bytes to the HIP launchers in muyo_hip.h.
 *
 * Conventions that carry over unchanged:
 *   - every `ne*` is an element count and every `nb*` an element stride (never bytes);
 *   - dimension 0 is the fastest-varying one;
 *   - `misalignOffsets` packs per-operand element offsets (binary ops: A<<16 | B<<8 | D,
 *     unary copy: A<<16 | D in the low 16 bits).
 *
 * The structs are C so that cgo/ctypes/JNI bindings can declare them without a C++ compiler.
 * The size checks below are the same ones the reference keeps; the launchers additionally
 * validate the fields at run time and return an error instead of mis-indexing.
 */
#ifndef MUYO_LLAMA_CONTRACTS_H
#define MUYO_LLAMA_CONTRACTS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* add / rms_norm / get_rows: the binary head (src/LlamaContracts.h:22-38). 29 words. */
typedef struct LlamaAddPushConstants
{
    uint32_t ne;

    uint32_t ne00, ne01, ne02, ne03;
    uint32_t nb00, nb01, nb02, nb03;
    uint32_t ne10, ne11, ne12, ne13;
    uint32_t nb10, nb11, nb12, nb13;
    uint32_t ne20, ne21, ne22, ne23;
    uint32_t nb20, nb21, nb22, nb23;

    uint32_t misalignOffsets;

    float param1; /* rms_norm: epsilon */
    float param2;
    int32_t param3;
} LlamaAddPushConstants;

/* mul_mat_vec (src/LlamaContracts.h:66-84). 13 words. `strideD` is also the row bound. */
typedef struct LlamaMatVecPushConstants
{
    uint32_t ncols;
    uint32_t strideA;
    uint32_t strideB;
    uint32_t strideD;

    uint32_t batchStrideA;
    uint32_t batchStrideB;
    uint32_t batchStrideD;

    uint32_t fusionFlags;

    uint32_t baseWorkGroupY;
    uint32_t ne02;
    uint32_t ne12;
    uint32_t broadcast2;
    uint32_t broadcast3;
} LlamaMatVecPushConstants;

/* rope (src/LlamaContracts.h:125-153). 30 words. */
typedef struct LlamaRopePushConstants
{
    uint32_t ropeMode;
    uint32_t nrows;
    uint32_t nDims;
    uint32_t nOffs;
    float freqScale;
    float freqBase;
    float extFactor;
    float attnFactor;
    float corrDims[2];
    float thetaScale;
    uint32_t hasFf;
    int32_t sections[4];
    uint32_t isImrope;
    uint32_t isBack;
    uint32_t setRowsStride;
    uint32_t ne00;
    uint32_t ne01;
    uint32_t ne02;
    uint32_t nb01;
    uint32_t nb02;
    uint32_t nb03;
    uint32_t nb11;
    uint32_t nb12;
    uint32_t nb13;
    uint32_t aOffset;
    uint32_t dOffset;
} LlamaRopePushConstants;

/* GLU family, swiglu among them (src/LlamaContracts.h:182-199). 27 words. */
typedef struct LlamaGluPushConstants
{
    uint32_t N;
    uint32_t ne00;
    uint32_t ne20;
    uint32_t mode;
    float alpha;
    float limit;
    uint32_t nb00, nb01, nb02, nb03;
    uint32_t nb10, nb11, nb12, nb13;
    uint32_t nb20, nb21, nb22, nb23;
    uint32_t ne21;
    uint32_t ne22;
    uint32_t misalignOffsets;
    uint32_t ne2_012mp, ne2_012L;
    uint32_t ne2_01mp, ne2_01L;
    uint32_t ne2_0mp, ne2_0L;
} LlamaGluPushConstants;

/* Generic head, argmax among its users (src/LlamaContracts.h:224-232). 6 words. */
typedef struct LlamaGenericHeadPushConstants
{
    uint32_t KX; /* row length */
    uint32_t KY; /* row count */
    float param1;
    float param2;
    float param3;
    float param4;
} LlamaGenericHeadPushConstants;

/* soft_max (src/LlamaContracts.h:255-274). 17 words. */
typedef struct LlamaSoftMaxPushConstants
{
    uint32_t KX;
    uint32_t KY;
    uint32_t ne00;
    uint32_t ne01;
    uint32_t ne02;
    uint32_t ne12;
    uint32_t ne13;
    uint32_t nb11;
    uint32_t nb12;
    uint32_t nb13;
    float scale;
    float maxBias;
    float m0;
    float m1;
    uint32_t nHeadLog2;
    uint32_t nrowsX;
    uint32_t hasSinks;
} LlamaSoftMaxPushConstants;

/* Unary head used by the strided copy that appends a value column to the cache
 * (src/FullModel.cpp:353-365, src/KvCache.cpp:47-56). 30 words. The `*_Ls` words pack three
 * fastdiv shifts, outermost divisor in the low byte. */
typedef struct LlamaCopyPushConstants
{
    uint32_t ne;
    uint32_t ne00, ne01, ne02, ne03, nb00, nb01, nb02, nb03;
    uint32_t ne10, ne11, ne12, ne13, nb10, nb11, nb12, nb13;
    uint32_t misalignOffsets;
    float param1, param2, param3, param4;
    uint32_t ne0_012mp, ne0_01mp, ne0_0mp, ne0_Ls;
    uint32_t ne1_012mp, ne1_01mp, ne1_0mp, ne1_Ls;
} LlamaCopyPushConstants;

/* Descriptor-binding order of each op (src/LlamaContracts.h:46-52, 92-99, 160-167, 206-211,
 * 239-243, 282-288). The launchers take their buffers in exactly this order. */
enum
{
    LLAMA_ADD_BINDING_A = 0,
    LLAMA_ADD_BINDING_B = 1,
    LLAMA_ADD_BINDING_D = 2,
    LLAMA_ADD_BINDING_PARTIAL_SUMS = 3,

    LLAMA_MAT_VEC_BINDING_A = 0,
    LLAMA_MAT_VEC_BINDING_B = 1,
    LLAMA_MAT_VEC_BINDING_D = 2,
    LLAMA_MAT_VEC_BINDING_FUSE0 = 3,
    LLAMA_MAT_VEC_BINDING_FUSE1 = 4,

    LLAMA_ROPE_BINDING_X = 0,
    LLAMA_ROPE_BINDING_Y = 1,
    LLAMA_ROPE_BINDING_Z = 2,
    LLAMA_ROPE_BINDING_D = 3,
    LLAMA_ROPE_BINDING_I = 4,

    LLAMA_GLU_BINDING_A = 0,
    LLAMA_GLU_BINDING_B = 1,
    LLAMA_GLU_BINDING_D = 2,

    LLAMA_ARGMAX_BINDING_A = 0,
    LLAMA_ARGMAX_BINDING_D = 1,

    LLAMA_SOFT_MAX_BINDING_X = 0,
    LLAMA_SOFT_MAX_BINDING_Y = 1,
    LLAMA_SOFT_MAX_BINDING_Z = 2,
    LLAMA_SOFT_MAX_BINDING_D = 3
};

/* mul_mat_vec `fusionFlags` bits (src/LlamaContracts.h:112-118). */
enum
{
    LLAMA_MAT_VEC_FUSION_BIAS0 = 0x1,
    LLAMA_MAT_VEC_FUSION_BIAS1 = 0x2,
    LLAMA_MAT_VEC_FUSION_SCALE0 = 0x4,
    LLAMA_MAT_VEC_FUSION_SCALE1 = 0x8
};

/* rope modes (src/LlamaContracts.h:170-174) and GLU modes (src/LlamaContracts.h:215-220). */
enum
{
    LLAMA_ROPE_MODE_NORMAL = 0,
    LLAMA_ROPE_MODE_NEOX = 2
};

enum
{
    LLAMA_GLU_MODE_DEFAULT_HALVES = 0,
    LLAMA_GLU_MODE_SWAPPED_HALVES = 1,
    LLAMA_GLU_MODE_SPLIT = 2
};

#ifdef __cplusplus
} /* extern "C" */

static_assert(sizeof(LlamaAddPushConstants) == 29 * sizeof(uint32_t), "add/rms_norm/get_rows block is 29 words");
static_assert(sizeof(LlamaMatVecPushConstants) == 13 * sizeof(uint32_t), "mul_mat_vec block is 13 words");
static_assert(sizeof(LlamaRopePushConstants) == 30 * sizeof(uint32_t), "rope block is 30 words");
static_assert(sizeof(LlamaGluPushConstants) == 27 * sizeof(uint32_t), "glu block is 27 words");
static_assert(sizeof(LlamaGenericHeadPushConstants) == 6 * sizeof(uint32_t), "generic head is 6 words");
static_assert(sizeof(LlamaSoftMaxPushConstants) == 17 * sizeof(uint32_t), "soft_max block is 17 words");
static_assert(sizeof(LlamaCopyPushConstants) == 30 * sizeof(uint32_t), "unary copy block is 30 words");

/* The reference spells these as namespaced constants (src/LlamaContracts.h:46-58, 92-118,
 * 160-174, 206-220, 239-249, 282-294); the same names are kept for C++ callers. */
namespace muyo_llm
{
using ::LlamaAddPushConstants;
using ::LlamaCopyPushConstants;
using ::LlamaGenericHeadPushConstants;
using ::LlamaGluPushConstants;
using ::LlamaMatVecPushConstants;
using ::LlamaRopePushConstants;
using ::LlamaSoftMaxPushConstants;

namespace llama_add_bindings
{
constexpr uint32_t A = LLAMA_ADD_BINDING_A;
constexpr uint32_t B = LLAMA_ADD_BINDING_B;
constexpr uint32_t D = LLAMA_ADD_BINDING_D;
constexpr uint32_t PARTIAL_SUMS = LLAMA_ADD_BINDING_PARTIAL_SUMS;
}  // namespace llama_add_bindings
namespace llama_add_spec_constants
{
constexpr uint32_t NOREPEAT = 0;
}
namespace llama_mat_vec_bindings
{
constexpr uint32_t A = LLAMA_MAT_VEC_BINDING_A;
constexpr uint32_t B = LLAMA_MAT_VEC_BINDING_B;
constexpr uint32_t D = LLAMA_MAT_VEC_BINDING_D;
constexpr uint32_t FUSE0 = LLAMA_MAT_VEC_BINDING_FUSE0;
constexpr uint32_t FUSE1 = LLAMA_MAT_VEC_BINDING_FUSE1;
}  // namespace llama_mat_vec_bindings
namespace llama_mat_vec_spec_constants
{
constexpr uint32_t BLOCK_SIZE = 0;
constexpr uint32_t NUM_ROWS = 1;
constexpr uint32_t NUM_COLS = 2;
}  // namespace llama_mat_vec_spec_constants
namespace llama_mat_vec_fusion
{
constexpr uint32_t BIAS0 = LLAMA_MAT_VEC_FUSION_BIAS0;
constexpr uint32_t BIAS1 = LLAMA_MAT_VEC_FUSION_BIAS1;
constexpr uint32_t SCALE0 = LLAMA_MAT_VEC_FUSION_SCALE0;
constexpr uint32_t SCALE1 = LLAMA_MAT_VEC_FUSION_SCALE1;
}  // namespace llama_mat_vec_fusion
namespace llama_rope_bindings
{
constexpr uint32_t X = LLAMA_ROPE_BINDING_X;
constexpr uint32_t Y = LLAMA_ROPE_BINDING_Y;
constexpr uint32_t Z = LLAMA_ROPE_BINDING_Z;
constexpr uint32_t D = LLAMA_ROPE_BINDING_D;
constexpr uint32_t I = LLAMA_ROPE_BINDING_I;
}  // namespace llama_rope_bindings
namespace llama_rope_modes
{
constexpr uint32_t NORMAL = LLAMA_ROPE_MODE_NORMAL;
constexpr uint32_t NEOX = LLAMA_ROPE_MODE_NEOX;
}  // namespace llama_rope_modes
namespace llama_glu_bindings
{
constexpr uint32_t A = LLAMA_GLU_BINDING_A;
constexpr uint32_t B = LLAMA_GLU_BINDING_B;
constexpr uint32_t D = LLAMA_GLU_BINDING_D;
}  // namespace llama_glu_bindings
namespace llama_glu_modes
{
constexpr uint32_t DEFAULT_HALVES = LLAMA_GLU_MODE_DEFAULT_HALVES;
constexpr uint32_t SWAPPED_HALVES = LLAMA_GLU_MODE_SWAPPED_HALVES;
constexpr uint32_t SPLIT = LLAMA_GLU_MODE_SPLIT;
}  // namespace llama_glu_modes
namespace llama_argmax_bindings
{
constexpr uint32_t A = LLAMA_ARGMAX_BINDING_A;
constexpr uint32_t D = LLAMA_ARGMAX_BINDING_D;
}  // namespace llama_argmax_bindings
namespace llama_argmax_spec_constants
{
constexpr uint32_t BLOCK_SIZE = 0;
}
namespace llama_soft_max_bindings
{
constexpr uint32_t X = LLAMA_SOFT_MAX_BINDING_X;
constexpr uint32_t Y = LLAMA_SOFT_MAX_BINDING_Y;
constexpr uint32_t Z = LLAMA_SOFT_MAX_BINDING_Z;
constexpr uint32_t D = LLAMA_SOFT_MAX_BINDING_D;
}  // namespace llama_soft_max_bindings
namespace llama_soft_max_spec_constants
{
constexpr uint32_t BLOCK_SIZE = 0;
}
}  // namespace muyo_llm
#else
_Static_assert(sizeof(LlamaAddPushConstants) == 29 * sizeof(uint32_t), "add/rms_norm/get_rows block is 29 words");
_Static_assert(sizeof(LlamaMatVecPushConstants) == 13 * sizeof(uint32_t), "mul_mat_vec block is 13 words");
_Static_assert(sizeof(LlamaRopePushConstants) == 30 * sizeof(uint32_t), "rope block is 30 words");
_Static_assert(sizeof(LlamaGluPushConstants) == 27 * sizeof(uint32_t), "glu block is 27 words");
_Static_assert(sizeof(LlamaGenericHeadPushConstants) == 6 * sizeof(uint32_t), "generic head is 6 words");
_Static_assert(sizeof(LlamaSoftMaxPushConstants) == 17 * sizeof(uint32_t), "soft_max block is 17 words");
_Static_assert(sizeof(LlamaCopyPushConstants) == 30 * sizeof(uint32_t), "unary copy block is 30 words");
#endif

#endif /* MUYO_LLAMA_CONTRACTS_H */
