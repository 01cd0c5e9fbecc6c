/*
 * CPU oracle for the decode-step kernel set — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker the HIP kernels are compared against. Only tests/, the smoke
 * check of __graft_entry__.py and the cpu_baseline leg of bench.py may load it; the product
 * library (libmuyo_hip.so) never links or calls it.
 *
 * Every op restates the reference's own CPU reference loop (muyo-llm, src/ *.cpp), cited per
 * function. The decode step restates tools/reference_qwen2.py:100-166 in the node order of
 * src/FullModel.cpp:726-993, with double accumulation for the GEMV/attention sums so that
 * greedy ids are robust to summation order.
 *
 * Pins (how each function is checked independently of its own formula) are listed in the
 * test files that exercise them: the reference's known-answer tests (src/MatVec.cpp:70-80,
 * RmsNorm.cpp:60-72, Rope.cpp:55-64, SoftMax.cpp:49-53, Argmax.cpp:51-56, ElementwiseAdd.cpp:95-99,
 * Swiglu.cpp:61-67, GetRows.cpp:49-56, KvCache.cpp:356-400, Attention.cpp:253-294,
 * TransformerLayer.cpp:242-286), closed forms and invariants, float64 library routines (numpy,
 * torch) and brute force on small inputs.
 */
#ifndef MUYO_ORACLE_H
#define MUYO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32. float->half rounds to nearest, ties to even. */
float oracle_half_to_float(uint16_t h);
uint16_t oracle_float_to_half(float f);
void oracle_halves_to_floats(const uint16_t* h, float* f, uint64_t n);
void oracle_floats_to_halves(const float* f, uint16_t* h, uint64_t n);

/* Portable seeded generator (same definition as the product's synthetic-input helpers). */
uint64_t oracle_mix64(uint64_t z);
void oracle_fill_normal_f16(uint16_t* out, uint64_t count, uint64_t seed, double mean, double std);
void oracle_fill_normal_f32(float* out, uint64_t count, uint64_t seed, double mean, double std);
void oracle_fill_uniform_f32(float* out, uint64_t count, uint64_t seed);
uint64_t oracle_tensor_seed(uint64_t seed, uint32_t kind, uint32_t layer);

/* Threads used by the row-parallel loops (results do not depend on it). Returns the count set. */
int oracle_set_threads(int n);

/* y[r] = sum_c f32(A[r*row_stride + c]) * x[c], f32 running sum in column order
 * (src/MatVec.cpp:52-60 HostMatVec; src/TransformerLayer.cpp:209-223 Gemv). */
void oracle_mat_vec_f16(const uint16_t* a, const float* x, float* y, uint32_t rows, uint32_t cols,
                        uint64_t row_stride);
void oracle_mat_vec_f32(const float* a, const float* x, float* y, uint32_t rows, uint32_t cols, uint64_t row_stride);

/* Same product with a double running sum, rounded once to f32 (the accumulation the decode step
 * uses; reference_qwen2.py:112-114,138,149-152,163 compute these with numpy matmul). */
void oracle_mat_vec_f16_f64acc(const uint16_t* a, const float* x, float* y, uint32_t rows, uint32_t cols,
                               uint64_t row_stride);

/* y = x * f32(1/sqrt(sum_double(x^2)/cols + eps)) * w, per row (src/RmsNorm.cpp:194-216,
 * src/TransformerLayer.cpp:225-239). w may be NULL (no multiply). */
void oracle_rms_norm(const float* x, const float* w, float* y, uint32_t rows, uint32_t cols, float eps);
void oracle_rms_norm_f16w(const float* x, const uint16_t* w, float* y, uint32_t rows, uint32_t cols, float eps);

/* Per row: v = x*scale (f32), m = max v, y = f32(exp(v - m) / sum_double(exp(v - m)))
 * (src/SoftMax.cpp:164-191). */
void oracle_soft_max(const float* x, float* y, uint32_t rows, uint32_t cols, float scale);

/* Greedy scan, strict '>' so ties go to the lowest index (src/Sampler.cpp:32-43). */
int32_t oracle_argmax(const float* x, uint32_t n);
void oracle_argmax_rows(const float* x, int32_t* out, uint32_t rows, uint32_t cols);

/* d = a + b (src/ElementwiseAdd.cpp:208). */
void oracle_add(const float* a, const float* b, float* d, uint64_t n);

/* d = g / (1 + exp(-g)) * u in f32 (src/Swiglu.cpp:56,187). */
void oracle_swiglu(const float* g, const float* u, float* d, uint64_t n);

/* NeoX rope of `rows` heads of `head_dim` channels, rotating the first n_dims channels in pairs
 * (j, j + n_dims/2) by theta = pos * powf(theta_scale, j) (src/Rope.cpp:48-51,191-203;
 * src/KvCache.cpp:78-91). Channels past n_dims are copied. */
void oracle_rope_neox(const float* x, float* y, uint32_t rows, uint32_t head_dim, uint32_t n_dims, int32_t pos,
                      float theta_scale);

/* d[i] = f32(table[index*dim + i]) (src/GetRows.cpp:179-182, src/Embedding.cpp:69-85). */
void oracle_get_rows_f16(const uint16_t* table, int32_t index, float* d, uint32_t dim);

/* One decode-step attention over fp16 caches [kv_heads][max_seq][head_dim], keys 0..pos, in
 * double (src/KvCache.cpp:356-400, src/Attention.cpp:253-294; GQA head h reads kv head
 * h / (heads/kv_heads) as reference_qwen2.py:133-137 repeats them). */
void oracle_attention_f16kv(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                            uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t max_seq, int32_t pos,
                            float scale);

/* Qwen2-shaped model held in host memory, the same tensor layout the product decoder uses. */
typedef struct OracleQwen2
{
    uint32_t layers, hidden, ffn, heads, kv_heads, head_dim, vocab, max_seq;
    float rms_eps, rope_base;
    const uint16_t* token_embd;      /* [vocab][hidden], also the tied LM head */
    const float* output_norm;        /* [hidden] */
    const float* const* attn_norm;   /* [layers] -> [hidden] */
    const uint16_t* const* attn_qkv; /* [layers] -> [(heads+2*kv_heads)*head_dim][hidden] */
    const float* const* attn_qkv_b;  /* [layers] -> [(heads+2*kv_heads)*head_dim] */
    const uint16_t* const* attn_out; /* [layers] -> [hidden][heads*head_dim] */
    const float* const* ffn_norm;    /* [layers] -> [hidden] */
    const uint16_t* const* ffn_gate; /* [layers] -> [ffn][hidden] */
    const uint16_t* const* ffn_up;   /* [layers] -> [ffn][hidden] */
    const uint16_t* const* ffn_down; /* [layers] -> [hidden][ffn] */
    uint16_t* const* kcache;         /* [layers] -> [kv_heads][max_seq][head_dim] */
    uint16_t* const* vcache;         /* [layers] -> [kv_heads][max_seq][head_dim] */
    const uint16_t* output;          /* [vocab][hidden] untied LM head (output.weight), or NULL: token_embd */
} OracleQwen2;

/* One decode step: embed `token`, run every layer at cache row `pos` (appending k/v as fp16),
 * final norm, LM head (output, or the tied token_embd). Writes `logits` [vocab]; returns the greedy id; top2 (optional)
 * receives the largest two logits. Returns -1 on bad arguments. */
int32_t oracle_decode_step(const OracleQwen2* m, int32_t token, int32_t pos, float* logits, float* top2);
/* The same step as the reference's CPU path computes it: every sum an f32 running sum in index
 * order (HostMatVec for each projection and the LM head, src/MatVec.cpp:52-60), softmax and
 * rms_norm as src/SoftMax.cpp:164-191 and src/RmsNorm.cpp:194-216. Appends the cache row like
 * oracle_decode_step. The CPU baseline that bench.py times; not a checker. */
int32_t oracle_decode_step_f32(const OracleQwen2* m, int32_t token, int32_t pos, float* logits);

/* One transformer layer on an f32 hidden vector (used to check the composition at small
 * shapes): out = layer(x) at cache row pos. Same arithmetic as inside oracle_decode_step. */
void oracle_decode_layer(const OracleQwen2* m, uint32_t layer, const float* x, int32_t pos, float* out);

#ifdef __cplusplus
}
#endif

#endif /* MUYO_ORACLE_H */
