/*
 * muyo_hip: the C ABI of the MI355X (gfx950) decode-step kernel set.
 *
 * Every entry point takes plain pointers and sizes: no HIP, torch or C++ types appear in the
 * signatures, so the library binds from C, C++, ctypes, cgo or JNI alike. Device pointers are
 * HIP device addresses; `stream` is a `hipStream_t` passed as `void*` (NULL = the default
 * stream). Launches are asynchronous on `stream` unless stated otherwise.
 *
 * Per-op launchers. Each replaces one reference graph node: the node declared a shader, a
 * push-constant block (muyo/LlamaContracts.h), its buffers in descriptor-binding order and a
 * `vkCmdDispatch(x, y, z)`. The launcher takes exactly those, in that order, and computes what
 * the node computed over the work domain that dispatch covered. The reference's shader
 * workgroup shape is NOT reproduced: the kernels pick their own gfx950 geometry.
 *
 * Return value: 0 on success; a negative MUYO_E_* when the arguments break the contract (nothing
 * is launched); a positive hipError_t when HIP rejects the launch. `muyo_last_error()` gives the
 * message of the most recent failure on the calling thread.
 *
 * Ownership: the caller owns every buffer passed to a launcher; launchers do not retain
 * pointers beyond the call. The decoder (below) owns the buffers it allocates.
 *
 * Threads and devices: launchers may be called from several host threads, on any device; each
 * launches on the calling thread's current device. What they cache on the host (a device's CU
 * count, a kernel's occupancy and its LDS opt-in) is kept per device and filled on first use
 * under a lock. A decoder belongs to the device that was current when it was created and must
 * be used with that device current, from one thread at a time.
 */
#ifndef MUYO_HIP_H
#define MUYO_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "muyo/LlamaContracts.h"

#ifdef __cplusplus
extern "C" {
#endif

enum
{
    MUYO_OK = 0,
    MUYO_E_NULL = -1,        /* a required pointer is NULL */
    MUYO_E_CONTRACT = -2,    /* a push-constant field is inconsistent (stride, fastdiv magic, ...) */
    MUYO_E_DISPATCH = -3,    /* the dispatch shape is not one the op's shader accepts */
    MUYO_E_UNSUPPORTED = -4, /* a feature of the contract this build does not implement */
    MUYO_E_RANGE = -5,       /* a size or position is out of range */
    MUYO_E_NOMEM = -6,       /* device allocation failed */
    MUYO_E_STATE = -7        /* the object is not in a state that allows the call */
};

/* Message describing the last failure on this thread ("" if none). */
const char* muyo_last_error(void);

/* Library version string. */
const char* muyo_version(void);

/* ---------------------------------------------------------------------------------------------
 * Per-op launchers (one per reference shader variant).
 * ------------------------------------------------------------------------------------------- */

/* Specialisation constants of mul_mat_vec (src/LlamaContracts.h:102-107). blockSize is accepted
 * and ignored (the kernel picks its own wave geometry); numRows scales the dispatch into rows;
 * numCols must be 1 (one B column, the decode case). */
typedef struct MuyoMatVecSpec
{
    uint32_t blockSize;
    uint32_t numRows;
    uint32_t numCols;
} MuyoMatVecSpec;

/* mul_mat_vec_f16_f32_f32 (CMakeLists.txt:168-172; shaders/llama/mul_mat_vec.comp:248-264).
 * Replaces the GEMV node of src/MatVec.cpp:112-159 and the projection nodes (QKV, o, gate, up,
 * down, LM head) that src/FullModel.cpp builds with MatVecSpec/MatVecExecute (:133-175).
 *   d[batch][row] = sum_k f32(A[batchA][row*ncols + k]) * B[batch][k]
 *                   (+ FUSE0[...] if BIAS0) (+ FUSE1[...] if BIAS1)
 * Rows computed: [0, min(numRows*x*z, strideD)); batches: y. As in the shader, the A row stride
 * is `ncols` (strideA is not used for rows), batchA follows ne12/broadcast2/broadcast3, and the
 * SCALE flags have no effect outside the expert-indexed variant. spec may be NULL (32/1/1). */
int muyo_mul_mat_vec_f16_f32_f32(const LlamaMatVecPushConstants* pc, const MuyoMatVecSpec* spec, const void* a,
                                 const float* b, float* d, const float* fuse0, const float* fuse1, uint32_t dispatch_x,
                                 uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* mul_mat_vec_f32_f32_f32 (CMakeLists.txt:174-178): same contract with F32 A. This is the
 * GQA-batched attention GEMV of src/FullModel.cpp:793-812 (scores over the key cache with
 * dispatch x = position + 1) and :825-844 (values over the transposed value cache). */
int muyo_mul_mat_vec_f32_f32_f32(const LlamaMatVecPushConstants* pc, const MuyoMatVecSpec* spec, const float* a,
                                 const float* b, float* d, const float* fuse0, const float* fuse1, uint32_t dispatch_x,
                                 uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* rms_norm_f32 (CMakeLists.txt:117-121; shaders/llama/rms_norm.comp:53-151). Replaces
 * src/RmsNorm.cpp:91-154 and src/FullModel.cpp:215-247. One output row per dispatched
 * workgroup (x = rows, y = channels, z = samples):
 *   d = x * rsqrt(mean(x^2) + param1) [* w]   (w when do_multiply != 0)
 * `partial_sums` is the shader's declared-but-unread binding 3 and may be NULL. */
int muyo_rms_norm_f32(const LlamaAddPushConstants* pc, uint32_t do_multiply, const float* a, const float* b, float* d,
                      float* partial_sums, uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z,
                      void* stream);

/* The same op with an fp16 weight row (the reference reads F32 norm weights; fp16 is the storage
 * the decode workloads here use). The weight is widened exactly to f32 before the multiply. */
int muyo_rms_norm_f32_f16w(const LlamaAddPushConstants* pc, uint32_t do_multiply, const float* a, const void* b,
                           float* d, float* partial_sums, uint32_t dispatch_x, uint32_t dispatch_y,
                           uint32_t dispatch_z, void* stream);

/* add_f32 (CMakeLists.txt:110-115; shaders/llama/add.comp:23-46). Replaces
 * src/ElementwiseAdd.cpp:123-162 and src/FullModel.cpp:250-284. d = a + b over the dispatched
 * element range, B broadcast by modulo unless norepeat != 0. ADD_RMS is off (as compiled by the
 * reference), so partial_sums is not written and may be NULL. Canonical dispatch: (1, ceil(ne/512), z). */
int muyo_add_f32(const LlamaAddPushConstants* pc, uint32_t norepeat, const float* a, const float* b, float* d,
                 float* partial_sums, uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* swiglu_f32 (CMakeLists.txt:130-134; shaders/llama/swiglu.comp + glu_main.glsl). Replaces
 * src/Swiglu.cpp:94-145 and src/FullModel.cpp:287-327. d = silu(a) * b in the mode of
 * `pc->mode`. Index quotients use the divisors the ne2_* fastdiv words encode (as the shader
 * does); a word pair that is init_fastdiv_values of no divisor (e.g. zeroed) is MUYO_E_CONTRACT. */
int muyo_swiglu_f32(const LlamaGluPushConstants* pc, const float* a, const float* b, float* d, uint32_t dispatch_x,
                    uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* rope_neox_f32 (CMakeLists.txt:123-128; shaders/llama/rope_neox.comp, rope_funcs.glsl:76-114).
 * Replaces src/Rope.cpp:96-153 and src/FullModel.cpp:179-212 (q rope, and the k rope of
 * :771-784 that writes into the key cache through nb11/dOffset). Positions are int32 per i2; `ff` is read only when
 * hasFf != 0 and `set_rows` (uint32 pairs) only when setRowsStride != 0. */
int muyo_rope_neox_f32(const LlamaRopePushConstants* pc, const float* x, const int32_t* positions, const float* ff,
                       float* d, const uint32_t* set_rows, uint32_t dispatch_x, uint32_t dispatch_y,
                       uint32_t dispatch_z, void* stream);

/* soft_max_f32 (CMakeLists.txt:161-163; shaders/llama/soft_max.comp:41-172). Replaces
 * src/SoftMax.cpp:85-128 and src/FullModel.cpp:331-349. Row r = z*262144 + y*512 + x of the
 * dispatch, bounded by nrowsX: d = softmax(x*scale + slope*mask [, sink]). */
int muyo_soft_max_f32(const LlamaSoftMaxPushConstants* pc, const float* x, const float* mask, const float* sinks,
                      float* d, uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* argmax_f32 (CMakeLists.txt:148-150; shaders/llama/argmax.comp:20-60). Replaces
 * src/Argmax.cpp:74-106 and src/FullModel.cpp:461-484. d[row] = index of the largest of the KX
 * values of row `row` (< KY). Ties resolve to the LOWEST index, which is the rule of the host
 * greedy scan the reference actually samples with (src/Sampler.cpp:32-43). */
int muyo_argmax_f32(const LlamaGenericHeadPushConstants* pc, const float* a, int32_t* d, uint32_t dispatch_x,
                    uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* get_rows_f16_f32 / get_rows_f32 (CMakeLists.txt:136-146; shaders/llama/get_rows.comp:8-42).
 * Replace src/GetRows.cpp:84-139 and src/FullModel.cpp:424-458: d[i10][:] = f32(A[idx[i10]][:]).
 * A row index outside [0, ne01) gives a zero row instead of an out-of-bounds read. */
int muyo_get_rows_f16_f32(const LlamaAddPushConstants* pc, const void* a, const int32_t* b, float* d,
                          uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z, void* stream);
int muyo_get_rows_f32(const LlamaAddPushConstants* pc, const float* a, const int32_t* b, float* d, uint32_t dispatch_x,
                      uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* cpy_f32_f32 (CMakeLists.txt:156-159; shaders/llama/copy.comp + generic_unary_head.glsl).
 * Replaces the value-column append of src/FullModel.cpp:353-420 and src/KvCache.cpp:184-225:
 * d[doff + dst_idx(i)] = a[aoff + src0_idx(i)], i < ne. As in the shader, the quotients of
 * src0_idx/dst_idx use the divisors the fastdiv words encode (shifts packed outermost divisor
 * first) and the offsets use the shapes; a pair that encodes no divisor is MUYO_E_CONTRACT and
 * an index whose unsigned arithmetic would wrap is skipped. */
int muyo_cpy_f32_f32(const LlamaCopyPushConstants* pc, const float* a, float* d, uint32_t dispatch_x,
                     uint32_t dispatch_y, uint32_t dispatch_z, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Decode-step attention over an fp16 KV cache (no single reference node: it replaces the
 * attn_scores, attn_softmax and attn_values nodes of src/FullModel.cpp:793-844 for one layer;
 * the reference computes the same with f32 caches, src/Attention.cpp:253-294).
 * Layout: kcache/vcache are [kv_heads][max_seq][head_dim] fp16; q is [heads][head_dim] f32.
 * For every query head h (kv head h / (heads/kv_heads)):
 *   out[h] = sum_{j<=pos} softmax_j(scale * q[h].k[j]) * v[j]
 * `position` is a device int32 (the cache row of the current token; keys 0..pos are read).
 * The caller appends k/v of the current token before this call (muyo_rope_append_f16kv).
 * max_seq <= 32768; q and the caches 16-byte aligned.
 * `workspace` is caller-owned device memory (16-byte aligned) of at least
 * muyo_attention_decode_f16kv_workspace_bytes(heads, kv_heads, head_dim, max_seq) bytes for the
 * chunk partials; it needs no clearing. Calls that overlap in time (other streams) need their
 * own workspaces. The call allocates nothing, so it may be captured into a graph.
 * ------------------------------------------------------------------------------------------- */
size_t muyo_attention_decode_f16kv_workspace_bytes(uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                                                   uint32_t max_seq); /* 0: unsupported shape */
int muyo_attention_decode_f16kv(const float* q, const void* kcache, const void* vcache, float* out,
                                const int32_t* position, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                                uint32_t max_seq, float scale, void* workspace, uint64_t workspace_bytes,
                                void* stream);

/* muyo_attention_decode_f16kv without a workspace and without any allocation. It has no
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * graph capture, serving loops that forbid hipMalloc). The chunk partials live in a fixed
 * 512 KiB device array per GPU, held until the process ends; shapes whose partials
 * (kv_heads * chunks * (heads / kv_heads) * (head_dim + 2) floats, chunks = min(16,
 * ceil(max_seq * head_dim / 2048))) exceed it are MUYO_E_UNSUPPORTED. Every call on one GPU
 * shares that array: calls that overlap in time on one GPU (other streams, other threads) race. */
int muyo_attention_decode_f16kv_static(const float* q, const void* kcache, const void* vcache, float* out,
                                       const int32_t* position, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                                       uint32_t max_seq, float scale, void* stream);

/* Rope k (NeoX, theta = pos * theta_scale^j) and append k and v of the current token, as fp16,
 * at row `*position` of the [kv_heads][max_seq][head_dim] caches; q is roped into q_out. This
 * is the q rope + k rope + v copy node trio of src/FullModel.cpp:756-795 for an fp16 cache. */
int muyo_rope_append_f16kv(const float* q, const float* k, const float* v, float* q_out, void* kcache, void* vcache,
                           const int32_t* position, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                           uint32_t max_seq, float theta_scale, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Decoder: the composed decode step (RunFullModel's graph, src/FullModel.cpp:685-998, plus its
 * feedToken/sampleNext loop, :1096-1117, minus GGUF loading and tokenisation). Device memory is owned by the
 * decoder; the step is captured once into a hipGraph and replayed per token with the token and
 * position held in device memory.
 * ------------------------------------------------------------------------------------------- */

typedef struct MuyoQwen2Config
{
    uint32_t layers;
    uint32_t hidden;
    uint32_t feedForward;
    uint32_t heads;
    uint32_t kvHeads;
    uint32_t headDim;
    uint32_t vocab;
    uint32_t maxSeq;
    float rmsEps;
    float ropeBase;
    uint32_t untiedOutput; /* 0: the LM head is TOKEN_EMBD (tied); 1: a separate OUTPUT tensor */
} MuyoQwen2Config;

typedef struct MuyoDecoder MuyoDecoder;

/* Tensor kinds a caller may address (per layer where noted). Shapes, row-major:
 *   TOKEN_EMBD   fp16 [vocab][hidden]   (also the LM head unless untiedOutput)
 *   OUTPUT       fp16 [vocab][hidden]   (the LM head when untiedOutput; absent otherwise)
 *   OUTPUT_NORM  f32  [hidden]
 *   ATTN_NORM    f32  [hidden]                               per layer
 *   ATTN_QKV     fp16 [heads*hd + 2*kvHeads*hd][hidden]      per layer (q rows, then k, then v)
 *   ATTN_QKV_B   f32  [heads*hd + 2*kvHeads*hd]              per layer
 *   ATTN_OUTPUT  fp16 [hidden][heads*hd]                     per layer
 *   FFN_NORM     f32  [hidden]                               per layer
 *   FFN_GATE     fp16 [feedForward][hidden]                  per layer
 *   FFN_UP       fp16 [feedForward][hidden]                  per layer
 *   FFN_DOWN     fp16 [hidden][feedForward]                  per layer
 *   KCACHE       fp16 [kvHeads][maxSeq][hd]                  per layer
 *   VCACHE       fp16 [kvHeads][maxSeq][hd]                  per layer
 *   LOGITS       f32  [vocab]                                (output of the last step) */
enum
{
    MUYO_TENSOR_TOKEN_EMBD = 0,
    MUYO_TENSOR_OUTPUT_NORM = 1,
    MUYO_TENSOR_ATTN_NORM = 2,
    MUYO_TENSOR_ATTN_QKV = 3,
    MUYO_TENSOR_ATTN_QKV_B = 4,
    MUYO_TENSOR_ATTN_OUTPUT = 5,
    MUYO_TENSOR_FFN_NORM = 6,
    MUYO_TENSOR_FFN_GATE = 7,
    MUYO_TENSOR_FFN_UP = 8,
    MUYO_TENSOR_FFN_DOWN = 9,
    MUYO_TENSOR_KCACHE = 10,
    MUYO_TENSOR_VCACHE = 11,
    MUYO_TENSOR_LOGITS = 12,
    MUYO_TENSOR_OUTPUT = 13
};

/* Allocate a decoder for `config` on the current HIP device. Caches are zeroed. */
int muyo_decoder_create(const MuyoQwen2Config* config, MuyoDecoder** out);
void muyo_decoder_destroy(MuyoDecoder* decoder);
/* The configuration the decoder was created with. */
int muyo_decoder_config(const MuyoDecoder* decoder, MuyoQwen2Config* out);

/* Device address and byte size of one tensor. A request for MUYO_TENSOR_FFN_DOWN's address
 * makes the next step rebuild the decoder's transposed copy of that matrix (decoders that run
 * the feed-forward block as one launch): writes through an address requested before a step
 * are seen by later steps only after another request or an upload. */
int muyo_decoder_tensor(MuyoDecoder* decoder, uint32_t kind, uint32_t layer, void** device_ptr, uint64_t* bytes);

/* Synchronous host<->device copies of a whole tensor (bytes must equal the tensor's size). */
int muyo_decoder_upload(MuyoDecoder* decoder, uint32_t kind, uint32_t layer, const void* host, uint64_t bytes);
int muyo_decoder_download(MuyoDecoder* decoder, uint32_t kind, uint32_t layer, void* host, uint64_t bytes);

/* Fill every weight from the portable seeded generator (muyo_fill_normal_f16/f32 below):
 * matrices and the embedding N(0, 0.02), biases N(0, 0.02), norm weights N(1, 0.1). Tensor t of
 * layer l uses stream seed muyo_tensor_seed(seed, t, l). Caches are zeroed. */
int muyo_decoder_fill_random(MuyoDecoder* decoder, uint64_t seed);

/* Fill cache rows [0, positions) of every layer with N(0, 1) (seeded like fill_random, kinds
 * KCACHE/VCACHE), and zero the rest. */
int muyo_decoder_fill_kv_random(MuyoDecoder* decoder, uint32_t positions, uint64_t seed);

/* One decode step, synchronous: feed `token` at cache row `position`, return the greedy next
 * token (ties to the lowest index). Logits are left in the LOGITS tensor. */
int muyo_decoder_step(MuyoDecoder* decoder, int32_t token, int32_t position, int32_t* next_token);

/* Greedy generation fully on the device: feeds `token` at `position`, then feeds back each
 * greedy token, for `count` steps, with no host round trip between steps (one hipGraph launch
 * per step). ids[i] receives the i-th generated token. Synchronises `stream` before returning. */
int muyo_decoder_generate(MuyoDecoder* decoder, int32_t token, int32_t position, uint32_t count, int32_t* ids,
                          void* stream);

/* Enqueue `count` greedy steps on `stream` without synchronising (for timing); the ids stay on
 * the device and are fetched with muyo_decoder_generated_ids. */
int muyo_decoder_generate_async(MuyoDecoder* decoder, int32_t token, int32_t position, uint32_t count, void* stream);
int muyo_decoder_generated_ids(MuyoDecoder* decoder, int32_t* ids, uint32_t count);

/* Number of kernel launches one step enqueues (for reporting). */
uint32_t muyo_decoder_launches_per_step(const MuyoDecoder* decoder);

/* Kernels of one step, for per-kernel timing and profiling. */
enum
{
    MUYO_KERNEL_EMBED = 0,     /* previous step's greedy id, step bookkeeping, token row -> hidden f32
                                  (advances the state) */
    MUYO_KERNEL_QKV = 1,       /* rms_norm + q|k|v GEMV + bias + rope + cache append */
    MUYO_KERNEL_ATTENTION = 2, /* GQA attention over cache rows 0..position (chunk partials, and their
                                  merge when o_proj does not merge them) */
    MUYO_KERNEL_O_PROJ = 3,    /* [attention merge +] o_proj GEMV + residual */
    MUYO_KERNEL_GATE_UP = 4,   /* rms_norm + gate/up GEMV + swiglu */
    MUYO_KERNEL_DOWN = 5,      /* down GEMV + residual */
    MUYO_KERNEL_LM_HEAD = 6,   /* rms_norm + tied LM head + per-workgroup argmax partials */
    MUYO_KERNEL_FFN = 7        /* rms_norm + gate/up + swiglu + down in one launch, on decoders with a
                                  hidden size of at most 1024 and layers other than the last (the
                                  step's own feed-forward launch there; GATE_UP and DOWN still run
                                  the two-launch form) */
};

/* Set the device-side token and position (stream-ordered) without running a step. */
int muyo_decoder_set_state(MuyoDecoder* decoder, int32_t token, int32_t position, void* stream);

/* Enqueue exactly one kernel of the step for `layer` (ignored for EMBED and LM_HEAD) on
 * `stream`, with the decoder's buffers and current device state. */
int muyo_decoder_enqueue_kernel(MuyoDecoder* decoder, uint32_t kernel, uint32_t layer, void* stream);

/* The reference's node self-tests (`int RunX()` of src/{MatVec,RmsNorm,Rope,SoftMax,Argmax,
 * ElementwiseAdd,Swiglu,GetRows,KvCache,Attention}.cpp, C++ declarations in include/muyo/) by
 * the reference CLI's mode names (src/main.cpp:246-248): "--add", "--matvec", "--rmsnorm", "--rope",
 * "--swiglu", "--getrows", "--argmax", "--softmax", "--attention", "--kvcache", or "--smoke" for
 * all. Runs on the current device, synchronously. Returns 0 when every selected test matches its
 * CPU reference, 1 when one does not, MUYO_E_RANGE for an unknown mode. */
int muyo_self_test(const char* mode);

/* ---------------------------------------------------------------------------------------------
 * GGUF model files. Replaces the reference's GgufReader (src/Gguf.h:40-103, src/Gguf.cpp:155-373)
 * and its model load (src/FullModel.cpp:85-108 config, :582-600 tensors, :1022-1032 upload).
 *
 * muyo_gguf_open maps the file read-only and parses the header, metadata and tensor table
 * (MUYO_E_CONTRACT for a bad magic or a truncated table). The lookups convert as GgufReader's do:
 * *_uint_or and *_float_or cast any numeric or boolean scalar (fallback when absent or not
 * scalar), *_string_or returns a string value, *_string_array_size the length of a string array
 * (0 otherwise). Returned strings live until the next string lookup or the close. The data
 * section starts at the header's end rounded up to general.alignment (32 when absent).
 * muyo_gguf_tensor_data points into the mapping at an F32 or F16 tensor's bytes
 * (MUYO_E_UNSUPPORTED for other types, MUYO_E_RANGE past the end of the file).
 *
 * muyo_gguf_qwen2_config reads the qwen2.* dimensions and the vocabulary (the length of
 * tokenizer.ggml.tokens) as the reference does, with headDim = hidden / heads, maxSeq = max_seq,
 * and untiedOutput = 1 when the file has output.weight. muyo_decoder_load_gguf uploads every
 * weight of such a file into a decoder of that configuration: token_embd, output_norm, output
 * (if untied) and per layer attn_norm, attn_q|k|v (stacked into ATTN_QKV), their biases
 * (ATTN_QKV_B), attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down. Weights must be F16 and norms
 * and biases F32 with the configuration's dimensions (else MUYO_E_CONTRACT, or
 * MUYO_E_UNSUPPORTED for quantised types).
 * ------------------------------------------------------------------------------------------- */
typedef struct MuyoGguf MuyoGguf;

int muyo_gguf_open(const char* path, MuyoGguf** out);
void muyo_gguf_close(MuyoGguf* gguf);
uint32_t muyo_gguf_version(const MuyoGguf* gguf);
uint64_t muyo_gguf_data_offset(const MuyoGguf* gguf);
uint64_t muyo_gguf_metadata_count(const MuyoGguf* gguf);
uint64_t muyo_gguf_tensor_count(const MuyoGguf* gguf);
/* Entry `index` of the tensor table: name (valid until close), ggml type, dimension count and
 * dims[0..3] (fastest-varying first, unused ones 1), offset from the data section. */
int muyo_gguf_tensor_info(const MuyoGguf* gguf, uint64_t index, const char** name, uint32_t* type, uint32_t* n_dims,
                          uint64_t* dims, uint64_t* offset);
int muyo_gguf_has(const MuyoGguf* gguf, const char* key);
uint64_t muyo_gguf_uint_or(const MuyoGguf* gguf, const char* key, uint64_t fallback);
double muyo_gguf_float_or(const MuyoGguf* gguf, const char* key, double fallback);
const char* muyo_gguf_string_or(MuyoGguf* gguf, const char* key, const char* fallback);
uint64_t muyo_gguf_string_array_size(const MuyoGguf* gguf, const char* key);
const char* muyo_gguf_string_array_at(MuyoGguf* gguf, const char* key, uint64_t index);
int muyo_gguf_tensor_data(const MuyoGguf* gguf, const char* name, const void** data, uint64_t* bytes);
int muyo_gguf_qwen2_config(const MuyoGguf* gguf, uint32_t max_seq, MuyoQwen2Config* out);
int muyo_decoder_load_gguf(MuyoDecoder* decoder, const MuyoGguf* gguf);

/* ---------------------------------------------------------------------------------------------
 * Tokenizer. Replaces the reference's muyo_llm::Tokenizer (src/Tokenizer.h:22-88,
 * src/Tokenizer.cpp:89-345): GPT-2/Qwen2 byte-level BPE built from a GGUF file's
 * tokenizer.ggml.tokens, .merges, .token_type and .pre. Host code; no device is needed.
 *
 * muyo_tokenizer_create is Tokenizer(const GgufReader&) (MUYO_E_CONTRACT when the file has no
 * tokens array); the tokenizer keeps no reference to the file. muyo_tokenizer_encode is
 * Encode(text, parse_special): CONTROL/USER_DEFINED tokens are matched as units first when
 * parse_special is nonzero, the text between them is split by Qwen2's pattern (pre "qwen2",
 * "stablelm2", "hunyuan", "solar-open") or GPT-2's (any other) and merged by rank. It sets *count to
 * the number of ids and writes them when they fit in `capacity` (else MUYO_E_RANGE; 3 ids per
 * byte of text always fit); a code point above U+10FFFF in the text is MUYO_E_RANGE, as the
 * reference throws on one. muyo_tokenizer_decode is Decode (ids out of range are skipped),
 * muyo_tokenizer_token_bytes is TokenBytes, both reporting the byte length in *length and
 * copying when it fits. muyo_tokenizer_token_text is TokenFor ("" out of range, valid until
 * destroy), muyo_tokenizer_is_special IsSpecial, muyo_tokenizer_vocab_size VocabSize.
 * ------------------------------------------------------------------------------------------- */
typedef struct MuyoTokenizer MuyoTokenizer;

int muyo_tokenizer_create(const MuyoGguf* gguf, MuyoTokenizer** out);
void muyo_tokenizer_destroy(MuyoTokenizer* tokenizer);
uint64_t muyo_tokenizer_vocab_size(const MuyoTokenizer* tokenizer);
const char* muyo_tokenizer_token_text(const MuyoTokenizer* tokenizer, uint64_t id);
int muyo_tokenizer_is_special(const MuyoTokenizer* tokenizer, int32_t id);
int muyo_tokenizer_encode(const MuyoTokenizer* tokenizer, const char* text, uint64_t length, int parse_special,
                          int32_t* ids, uint64_t capacity, uint64_t* count);
int muyo_tokenizer_decode(const MuyoTokenizer* tokenizer, const int32_t* ids, uint64_t n, char* text,
                          uint64_t capacity, uint64_t* length);
int muyo_tokenizer_token_bytes(const MuyoTokenizer* tokenizer, int32_t id, char* bytes, uint64_t capacity,
                               uint64_t* length);

/* ---------------------------------------------------------------------------------------------
 * Batched prefill. The reference feeds a prompt one token at a time, a full decode step per
 * token (feedToken inside runTurn, src/FullModel.cpp:1096-1108,1162-1170), and names batched
 * prefill with mul_mm and flash_attn as deferred work (docs/Plan.md:277, README.md:120-121,
 * shaders/llama/mul_mm.comp). muyo_decoder_prefill is that feed done at once: the prompt's rows go
 * through each layer as GEMMs on the matrix cores and one causal attention, the K/V rows land in
 * the cache as the steps would have written them, and the last position's logits give the next
 * token as sampleNext would (greedy, or the decoder's sampler over the whole history).
 *
 * Activations reach the matrix cores as split planes: hi = f16(x), lo = f16(x - hi), two uint16
 * arrays of the same shape; W.hi + W.lo accumulated in f32 keeps ~22 bits of every activation,
 * so results agree with the f32 token-by-token path to f32 rounding. Every activation must stay
 * below 65504 in magnitude (f16's range).
 * ------------------------------------------------------------------------------------------- */

/* Feed tokens[0..count) at cache rows position..position+count-1 (in passes of at most 2048 rows)
 * and return the next token, as `count` calls of muyo_decoder_step would (their K/V rows, the
 * token history, the LOGITS of the last position). Synchronous; continue with
 * muyo_decoder_generate(next_token, position + count, ...). */
int muyo_decoder_prefill(MuyoDecoder* decoder, const int32_t* tokens, uint32_t count, int32_t position,
                         int32_t* next_token);

/* The prefill's kernels, on device memory, enqueued on `stream`. Planes and f16 weights are
 * uint16 arrays; every buffer 16-byte aligned. */
/* hi/lo planes of x[0..count), count % 4 == 0. */
int muyo_split_f32_f16x2(const float* x, uint64_t count, void* hi, void* lo, void* stream);
/* rms_norm (x * rsqrt(mean(x^2) + eps)) * w of each row of x [rows][cols] into planes, cols % 4 == 0. */
int muyo_rms_norm_split_f16x2(const float* x, const float* w, uint32_t rows, uint32_t cols, float eps, void* hi,
                              void* lo, void* stream);
/* out[m][n] = sum_k (a_hi + a_lo)[m][k] * w[n][k] (+ bias[n]) (+ residual[m][n]); a planes
 * [rows][k], w fp16 [n][k], out/residual f32 [rows][n]; bias and residual may be NULL;
 * n % 4 == 0, k % 8 == 0. */
int muyo_gemm_split_f16(const void* a_hi, const void* a_lo, const void* w, const float* bias, const float* residual,
                        float* out, uint32_t rows, uint32_t n, uint32_t k, void* stream);
/* h[m][f] = silu(g) * u, g and u the split products with w_gate[f] and w_up[f] (fp16 [ffn][k]),
 * written as planes [rows][ffn]; ffn % 4 == 0, k % 8 == 0. */
int muyo_gemm_swiglu_split_f16(const void* a_hi, const void* a_lo, const void* w_gate, const void* w_up, void* h_hi,
                               void* h_lo, uint32_t rows, uint32_t ffn, uint32_t k, void* stream);
/* From qkv [rows][(heads + 2 kv_heads) * head_dim] (q rows, k rows, v rows, bias included):
 * rope_neox at positions pos0 + m with angles pos * rope_pow[j] (rope_pow: device f32
 * [head_dim / 2], theta_scale^j), q into planes [rows][heads * head_dim], k and v as fp16 into
 * the caches [kv_heads][max_seq][head_dim] at rows pos0 + m. */
int muyo_rope_split_append_f16kv(const float* qkv, uint32_t rows, int32_t pos0, uint32_t heads, uint32_t kv_heads,
                                 uint32_t head_dim, uint32_t max_seq, const float* rope_pow, void* q_hi, void* q_lo,
                                 void* kcache, void* vcache, void* stream);
/* Causal GQA attention of the queries at positions pos0 + m (q planes [rows][heads * head_dim])
 * over cache rows 0..pos0 + m: softmax(scale * K q) . V into planes [rows][heads * head_dim].
 * head_dim 64 or 128, heads / kv_heads <= 8. */
int muyo_prefill_attention_f16kv(const void* q_hi, const void* q_lo, const void* kcache, const void* vcache,
                                 void* out_hi, void* out_lo, uint32_t rows, int32_t pos0, uint32_t heads,
                                 uint32_t kv_heads, uint32_t head_dim, uint32_t max_seq, float scale, void* stream);
/* muyo_prefill_attention_f16kv with a caller-owned workspace (16-byte aligned, at least
 * muyo_prefill_attention_workspace_bytes(rows, heads, head_dim) bytes, no clearing needed): query
 * tiles (32 queries) whose causal range is longer than 512 keys are split into key chunks run by
 * separate workgroups, and a second kernel combines their softmax partials. The same results to
 * f32 rounding. A prompt whose chunks would exceed 512 work items (past about 4096 queries)
 * runs unsplit. muyo_decoder_prefill runs this path.
 * Calls that overlap in time need their own workspaces. */
size_t muyo_prefill_attention_workspace_bytes(uint32_t rows, uint32_t heads, uint32_t head_dim); /* 0: unsupported */
int muyo_prefill_attention_f16kv_ws(const void* q_hi, const void* q_lo, const void* kcache, const void* vcache,
                                    void* out_hi, void* out_lo, uint32_t rows, int32_t pos0, uint32_t heads,
                                    uint32_t kv_heads, uint32_t head_dim, uint32_t max_seq, float scale,
                                    void* workspace, uint64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Token sampling on the device. Replaces the reference's host sampler, muyo_llm::Sampler
 * (src/Sampler.h:16-42, src/Sampler.cpp:10-100), which its decode loop calls on the mapped
 * logits after every step (src/FullModel.cpp:1111-1117).
 *
 * MuyoSamplerParams mirrors SamplerParams (src/Sampler.h:16-23) field for field; `reserved` pads
 * the seed to 8 bytes. The engine is the reference's std::mt19937_64(seed), kept on the device in
 * an opaque state of muyo_sampler_state_bytes() bytes; one uniform double is drawn per token
 * sampled with temperature > 0, as uniform_real_distribution<double>(0, 1) of libstdc++ draws it
 * (one 64-bit word / 2^64).
 *
 * muyo_sample_f32 is Sampler::Sample on device memory: the repetition penalty over the last
 * repeat_last_n entries of history[0..history_count) (each occurrence applies it once; negative
 * means all), temperature <= 0 as greedy (lowest index on ties), else division by the
 * temperature, top-k, top-p and one draw. It modifies `logits` in place as the reference does.
 * Among exactly equal logits the top-k order puts the lower index first (the reference leaves it
 * to std::partial_sort). With temperature > 0 the device keeps at most 1024 candidates: top_k must
 * be 1..1024, or <= 0 with vocab <= 1024 (else MUYO_E_UNSUPPORTED). `workspace` is device memory
 * of muyo_sample_workspace_bytes(vocab, params) bytes, zero-filled before its first use (each
 * call leaves it so). The call enqueues a few kernels on `stream` and writes the token to device
 * memory at `token`.
 * ------------------------------------------------------------------------------------------- */
typedef struct MuyoSamplerParams
{
    float temperature;     /* <= 0: greedy */
    int32_t top_k;         /* <= 0: the whole vocabulary */
    float top_p;
    float repeat_penalty;  /* 1: off */
    int32_t repeat_last_n; /* negative: the whole history */
    uint32_t reserved;
    uint64_t seed;
} MuyoSamplerParams;

/* The decoder's next-token rule: Sampler::Sample with these parameters after every step, on the
 * device, seeded now with params->seed (NULL: greedy, the default). Greedy without a penalty keeps
 * the LM head's own argmax; anything else runs the sampler on a copy of the logits (the LOGITS
 * tensor stays as the LM head wrote it). The penalty's history is the token embedded at each
 * position: the steps record theirs, and muyo_decoder_set_history supplies earlier ones (a
 * prompt). Takes effect from the next step; the step's graph is recorded again. */
int muyo_decoder_set_sampler(MuyoDecoder* decoder, const MuyoSamplerParams* params);
/* tokens[0..count) as the history of positions 0..count-1 (count <= maxSeq). */
int muyo_decoder_set_history(MuyoDecoder* decoder, const int32_t* tokens, uint32_t count);

size_t muyo_sampler_state_bytes(void);
/* std::mt19937_64(seed) into `state` (device memory), stream-ordered. */
int muyo_sampler_seed(void* state, uint64_t seed, void* stream);
size_t muyo_sample_workspace_bytes(uint32_t vocab, const MuyoSamplerParams* params);
int muyo_sample_f32(float* logits, uint32_t vocab, const int32_t* history, uint32_t history_count,
                    const MuyoSamplerParams* params, void* state, void* workspace, int32_t* token, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Synthetic-input helpers (portable seeded generator; bit-identical on host and device).
 *   word(seed, i)   = mix64(mix64(seed) + i)            mix64 = SplitMix64's finaliser
 *   uniform(i)      = (word >> 40) * 2^-23 - 1          in [-1, 1), exact in f32
 *   normal(i)       = sum of the 12 32-bit halves of word(6i .. 6i+5) * 2^-32 - 6
 *                     (Irwin-Hall: mean 0, variance 1), then mean + std * normal in double,
 *                     rounded to f32 and (for f16) on to fp16, both round-to-nearest-even.
 * ------------------------------------------------------------------------------------------- */
int muyo_fill_normal_f16(void* d, uint64_t count, uint64_t seed, double mean, double std, void* stream);
int muyo_fill_normal_f32(float* d, uint64_t count, uint64_t seed, double mean, double std, void* stream);
int muyo_fill_uniform_f32(float* d, uint64_t count, uint64_t seed, void* stream);
uint64_t muyo_tensor_seed(uint64_t seed, uint32_t kind, uint32_t layer);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MUYO_HIP_H */
