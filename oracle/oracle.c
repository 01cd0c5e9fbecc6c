/*
 * CPU oracle for the decode-step kernel set — TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Never linked into, or called by, the product library.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* binary16                                                                                    */

float oracle_half_to_float(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    uint32_t mantissa = h & 0x3FFu;
    uint32_t bits;
    if (exponent == 0)
    {
        if (mantissa == 0)
        {
            bits = sign;
        }
        else
        {
            /* Subnormal: normalise. value = mantissa * 2^-24. */
            int e = -1;
            do
            {
                ++e;
                mantissa <<= 1;
            } while ((mantissa & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mantissa & 0x3FFu) << 13);
        }
    }
    else if (exponent == 0x1F)
    {
        bits = sign | 0x7F800000u | (mantissa << 13);
    }
    else
    {
        bits = sign | ((exponent + 127 - 15) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

uint16_t oracle_float_to_half(float f)
{
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u)
    {
        /* Inf stays Inf; NaN stays a quiet NaN with the top payload bits. */
        return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? (0x200u | ((absx >> 13) & 0x3FFu)) : 0u));
    }
    if (absx >= 0x47800000u)
    {
        return (uint16_t)(sign | 0x7C00u); /* >= 65536 */
    }
    if (absx < 0x38800000u)
    {
        /* Result is a half subnormal (or zero): q = round(value / 2^-24). */
        if (absx < 0x33000000u)
        {
            return (uint16_t)sign; /* below 2^-25: rounds to zero (2^-25 itself ties to even 0) */
        }
        const uint32_t e = absx >> 23;
        const uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
        const uint32_t s = 126u - e; /* 14..24 */
        uint32_t q = m >> s;
        const uint32_t rem = m & ((1u << s) - 1u);
        const uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (q & 1u)))
        {
            ++q;
        }
        return (uint16_t)(sign | q);
    }
    const uint32_t e = (absx >> 23) - 127u + 15u;
    const uint32_t m = absx & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
    {
        ++h; /* a carry into the exponent is the correct next binade, up to Inf */
    }
    return (uint16_t)(sign | h);
}

void oracle_halves_to_floats(const uint16_t* h, float* f, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i)
    {
        f[i] = oracle_half_to_float(h[i]);
    }
}

void oracle_floats_to_halves(const float* f, uint16_t* h, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i)
    {
        h[i] = oracle_float_to_half(f[i]);
    }
}

/* A table for the hot half->float widening in the GEMVs. */
static float g_half_table[65536];
static int g_half_table_ready = 0;

static void ensure_half_table(void)
{
    if (!g_half_table_ready)
    {
        for (uint32_t i = 0; i < 65536u; ++i)
        {
            g_half_table[i] = oracle_half_to_float((uint16_t)i);
        }
        g_half_table_ready = 1;
    }
}

/* ------------------------------------------------------------------------------------------ */
/* Generator                                                                                   */

uint64_t oracle_mix64(uint64_t z)
{
    /* SplitMix64 (Steele, Lea, Flood 2014), one step from state z. */
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double irwin_hall_normal(uint64_t key, uint64_t i)
{
    uint64_t sum = 0;
    for (uint64_t k = 0; k < 6; ++k)
    {
        const uint64_t w = oracle_mix64(key + 6u * i + k);
        sum += (w >> 32) + (w & 0xFFFFFFFFull);
    }
    return (double)sum * 0x1p-32 - 6.0;
}

void oracle_fill_normal_f32(float* out, uint64_t count, uint64_t seed, double mean, double std)
{
    const uint64_t key = oracle_mix64(seed);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i)
    {
        out[i] = (float)(mean + std * irwin_hall_normal(key, (uint64_t)i));
    }
}

void oracle_fill_normal_f16(uint16_t* out, uint64_t count, uint64_t seed, double mean, double std)
{
    const uint64_t key = oracle_mix64(seed);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i)
    {
        out[i] = oracle_float_to_half((float)(mean + std * irwin_hall_normal(key, (uint64_t)i)));
    }
}

void oracle_fill_uniform_f32(float* out, uint64_t count, uint64_t seed)
{
    const uint64_t key = oracle_mix64(seed);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i)
    {
        const uint64_t w = oracle_mix64(key + (uint64_t)i);
        out[i] = (float)(w >> 40) * 0x1p-23f - 1.0f;
    }
}

uint64_t oracle_tensor_seed(uint64_t seed, uint32_t kind, uint32_t layer)
{
    return oracle_mix64(seed ^ (((uint64_t)kind << 40) | ((uint64_t)layer << 8) | 0x5Aull));
}

int oracle_set_threads(int n)
{
#ifdef _OPENMP
    if (n > 0)
    {
        omp_set_num_threads(n);
    }
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ------------------------------------------------------------------------------------------ */
/* Ops                                                                                         */

void oracle_mat_vec_f16(const uint16_t* a, const float* x, float* y, uint32_t rows, uint32_t cols,
                        uint64_t row_stride)
{
    ensure_half_table();
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
    {
        const uint16_t* row = a + (uint64_t)r * row_stride;
        float sum = 0.0f;
        for (uint32_t c = 0; c < cols; ++c)
        {
            sum += g_half_table[row[c]] * x[c];
        }
        y[r] = sum;
    }
}

void oracle_mat_vec_f32(const float* a, const float* x, float* y, uint32_t rows, uint32_t cols, uint64_t row_stride)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
    {
        const float* row = a + (uint64_t)r * row_stride;
        float sum = 0.0f;
        for (uint32_t c = 0; c < cols; ++c)
        {
            sum += row[c] * x[c];
        }
        y[r] = sum;
    }
}

void oracle_mat_vec_f16_f64acc(const uint16_t* a, const float* x, float* y, uint32_t rows, uint32_t cols,
                               uint64_t row_stride)
{
    ensure_half_table();
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
    {
        const uint16_t* row = a + (uint64_t)r * row_stride;
        double sum = 0.0;
        for (uint32_t c = 0; c < cols; ++c)
        {
            sum += (double)g_half_table[row[c]] * (double)x[c];
        }
        y[r] = (float)sum;
    }
}

static void rms_norm_row(const float* x, const float* w32, const uint16_t* w16, float* y, uint32_t cols, float eps)
{
    double sum_squares = 0.0;
    for (uint32_t c = 0; c < cols; ++c)
    {
        sum_squares += (double)x[c] * (double)x[c];
    }
    const float scale = (float)(1.0 / sqrt(sum_squares / cols + eps));
    for (uint32_t c = 0; c < cols; ++c)
    {
        float value = x[c] * scale;
        if (w32 != NULL)
        {
            value *= w32[c];
        }
        else if (w16 != NULL)
        {
            value *= oracle_half_to_float(w16[c]);
        }
        y[c] = value;
    }
}

void oracle_rms_norm(const float* x, const float* w, float* y, uint32_t rows, uint32_t cols, float eps)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
    {
        rms_norm_row(x + (uint64_t)r * cols, w, NULL, y + (uint64_t)r * cols, cols, eps);
    }
}

void oracle_rms_norm_f16w(const float* x, const uint16_t* w, float* y, uint32_t rows, uint32_t cols, float eps)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
    {
        rms_norm_row(x + (uint64_t)r * cols, NULL, w, y + (uint64_t)r * cols, cols, eps);
    }
}

static void soft_max_row(const float* in, float* out, uint32_t cols, float scale)
{
    float max_scaled = -1e30f;
    for (uint32_t c = 0; c < cols; ++c)
    {
        const float v = in[c] * scale;
        max_scaled = v > max_scaled ? v : max_scaled;
    }
    double sum_exp = 0.0;
    for (uint32_t c = 0; c < cols; ++c)
    {
        sum_exp += expf(in[c] * scale - max_scaled);
    }
    for (uint32_t c = 0; c < cols; ++c)
    {
        out[c] = (float)(expf(in[c] * scale - max_scaled) / sum_exp);
    }
}

void oracle_soft_max(const float* x, float* y, uint32_t rows, uint32_t cols, float scale)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
    {
        soft_max_row(x + (uint64_t)r * cols, y + (uint64_t)r * cols, cols, scale);
    }
}

int32_t oracle_argmax(const float* x, uint32_t n)
{
    int32_t best = 0;
    for (uint32_t i = 1; i < n; ++i)
    {
        if (x[i] > x[best])
        {
            best = (int32_t)i;
        }
    }
    return best;
}

void oracle_argmax_rows(const float* x, int32_t* out, uint32_t rows, uint32_t cols)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
    {
        out[r] = oracle_argmax(x + (uint64_t)r * cols, cols);
    }
}

void oracle_add(const float* a, const float* b, float* d, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i)
    {
        d[i] = a[i] + b[i];
    }
}

void oracle_swiglu(const float* g, const float* u, float* d, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i)
    {
        d[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
    }
}

void oracle_rope_neox(const float* x, float* y, uint32_t rows, uint32_t head_dim, uint32_t n_dims, int32_t pos,
                      float theta_scale)
{
    const uint32_t half = n_dims / 2;
    for (uint32_t r = 0; r < rows; ++r)
    {
        const float* in = x + (uint64_t)r * head_dim;
        float* out = y + (uint64_t)r * head_dim;
        for (uint32_t j = 0; j < half; ++j)
        {
            const float theta = (float)pos * powf(theta_scale, (float)j);
            const float c = cosf(theta);
            const float s = sinf(theta);
            const float x0 = in[j];
            const float x1 = in[j + half];
            out[j] = x0 * c - x1 * s;
            out[j + half] = x0 * s + x1 * c;
        }
        for (uint32_t j = n_dims; j < head_dim; ++j)
        {
            out[j] = in[j];
        }
    }
}

void oracle_get_rows_f16(const uint16_t* table, int32_t index, float* d, uint32_t dim)
{
    const uint16_t* row = table + (uint64_t)index * dim;
    for (uint32_t i = 0; i < dim; ++i)
    {
        d[i] = oracle_half_to_float(row[i]);
    }
}

void oracle_attention_f16kv(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                            uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t max_seq, int32_t pos,
                            float scale)
{
    ensure_half_table();
    const uint32_t group = heads / kv_heads;
    const uint32_t keys = (uint32_t)pos + 1u;
    double* weights = (double*)malloc(sizeof(double) * keys);
    double* acc = (double*)malloc(sizeof(double) * head_dim);
    for (uint32_t h = 0; h < heads; ++h)
    {
        const uint32_t g = h / group;
        const float* qh = q + (uint64_t)h * head_dim;
        const uint16_t* kbase = kcache + (uint64_t)g * max_seq * head_dim;
        const uint16_t* vbase = vcache + (uint64_t)g * max_seq * head_dim;
        double max_score = -1e300;
        for (uint32_t j = 0; j < keys; ++j)
        {
            double dot = 0.0;
            for (uint32_t c = 0; c < head_dim; ++c)
            {
                dot += (double)qh[c] * (double)g_half_table[kbase[(uint64_t)j * head_dim + c]];
            }
            weights[j] = dot * (double)scale;
            max_score = weights[j] > max_score ? weights[j] : max_score;
        }
        double sum = 0.0;
        for (uint32_t j = 0; j < keys; ++j)
        {
            weights[j] = exp(weights[j] - max_score);
            sum += weights[j];
        }
        for (uint32_t c = 0; c < head_dim; ++c)
        {
            acc[c] = 0.0;
        }
        for (uint32_t j = 0; j < keys; ++j)
        {
            const double p = weights[j] / sum;
            for (uint32_t c = 0; c < head_dim; ++c)
            {
                acc[c] += p * (double)g_half_table[vbase[(uint64_t)j * head_dim + c]];
            }
        }
        for (uint32_t c = 0; c < head_dim; ++c)
        {
            out[(uint64_t)h * head_dim + c] = (float)acc[c];
        }
    }
    free(weights);
    free(acc);
}

/* ------------------------------------------------------------------------------------------ */
/* Decode step: tools/reference_qwen2.py:107-166 in the node order of src/FullModel.cpp:726-993. */

void oracle_decode_layer(const OracleQwen2* m, uint32_t l, const float* x, int32_t pos, float* out)
{
    const uint32_t hd = m->head_dim;
    const uint32_t qdim = m->heads * hd;
    const uint32_t kvdim = m->kv_heads * hd;
    const uint32_t qkv_rows = qdim + 2u * kvdim;
    const float theta_scale = powf(m->rope_base, -2.0f / (float)hd); /* src/FullModel.cpp:201 */
    const float attn_scale = 1.0f / sqrtf((float)hd);                /* src/FullModel.cpp:184 */

    float* xn = (float*)malloc(sizeof(float) * m->hidden);
    float* qkv = (float*)malloc(sizeof(float) * qkv_rows);
    float* qr = (float*)malloc(sizeof(float) * qdim);
    float* kr = (float*)malloc(sizeof(float) * kvdim);
    float* attn = (float*)malloc(sizeof(float) * qdim);
    float* o = (float*)malloc(sizeof(float) * m->hidden);
    float* x1 = (float*)malloc(sizeof(float) * m->hidden);
    float* gate = (float*)malloc(sizeof(float) * m->ffn);
    float* up = (float*)malloc(sizeof(float) * m->ffn);
    float* act = (float*)malloc(sizeof(float) * m->ffn);
    float* down = (float*)malloc(sizeof(float) * m->hidden);

    /* pre_norm -> q/k/v projections with bias (reference_qwen2.py:111-114). */
    oracle_rms_norm(x, m->attn_norm[l], xn, 1, m->hidden, m->rms_eps);
    oracle_mat_vec_f16_f64acc(m->attn_qkv[l], xn, qkv, qkv_rows, m->hidden, m->hidden);
    for (uint32_t r = 0; r < qkv_rows; ++r)
    {
        qkv[r] += m->attn_qkv_b[l][r];
    }
    /* q_rope, k_rope into the cache row, v append (reference_qwen2.py:120-130). */
    oracle_rope_neox(qkv, qr, m->heads, hd, hd, pos, theta_scale);
    oracle_rope_neox(qkv + qdim, kr, m->kv_heads, hd, hd, pos, theta_scale);
    for (uint32_t g = 0; g < m->kv_heads; ++g)
    {
        for (uint32_t c = 0; c < hd; ++c)
        {
            const uint64_t slot = ((uint64_t)g * m->max_seq + (uint64_t)pos) * hd + c;
            m->kcache[l][slot] = oracle_float_to_half(kr[g * hd + c]);
            m->vcache[l][slot] = oracle_float_to_half(qkv[qdim + kvdim + g * hd + c]);
        }
    }
    /* GQA attention over keys 0..pos (reference_qwen2.py:132-137). */
    oracle_attention_f16kv(qr, m->kcache[l], m->vcache[l], attn, m->heads, m->kv_heads, hd, m->max_seq, pos,
                           attn_scale);
    /* o_proj + residual (reference_qwen2.py:138,145). */
    oracle_mat_vec_f16_f64acc(m->attn_out[l], attn, o, m->hidden, qdim, qdim);
    oracle_add(x, o, x1, m->hidden);
    /* post_norm, gate/up, swiglu, down, residual (reference_qwen2.py:148-157). */
    oracle_rms_norm(x1, m->ffn_norm[l], xn, 1, m->hidden, m->rms_eps);
    oracle_mat_vec_f16_f64acc(m->ffn_gate[l], xn, gate, m->ffn, m->hidden, m->hidden);
    oracle_mat_vec_f16_f64acc(m->ffn_up[l], xn, up, m->ffn, m->hidden, m->hidden);
    oracle_swiglu(gate, up, act, m->ffn);
    oracle_mat_vec_f16_f64acc(m->ffn_down[l], act, down, m->hidden, m->ffn, m->ffn);
    oracle_add(x1, down, out, m->hidden);

    free(xn);
    free(qkv);
    free(qr);
    free(kr);
    free(attn);
    free(o);
    free(x1);
    free(gate);
    free(up);
    free(act);
    free(down);
}

int32_t oracle_decode_step(const OracleQwen2* m, int32_t token, int32_t pos, float* logits, float* top2)
{
    if (m == NULL || logits == NULL || token < 0 || (uint32_t)token >= m->vocab || pos < 0 ||
        (uint32_t)pos >= m->max_seq || m->heads % m->kv_heads != 0)
    {
        return -1;
    }
    float* h = (float*)malloc(sizeof(float) * m->hidden);
    float* next = (float*)malloc(sizeof(float) * m->hidden);
    float* hn = (float*)malloc(sizeof(float) * m->hidden);

    oracle_get_rows_f16(m->token_embd, token, h, m->hidden); /* embed */
    for (uint32_t l = 0; l < m->layers; ++l)
    {
        oracle_decode_layer(m, l, h, pos, next);
        memcpy(h, next, sizeof(float) * m->hidden);
    }
    oracle_rms_norm(h, m->output_norm, hn, 1, m->hidden, m->rms_eps);               /* final_norm */
    /* LM head: output.weight when the model has one (src/FullModel.cpp:583), else the tied table. */
    const uint16_t* head = m->output != NULL ? m->output : m->token_embd;
    oracle_mat_vec_f16_f64acc(head, hn, logits, m->vocab, m->hidden, m->hidden);
    const int32_t best = oracle_argmax(logits, m->vocab);
    if (top2 != NULL)
    {
        float second = -INFINITY;
        for (uint32_t i = 0; i < m->vocab; ++i)
        {
            if ((int32_t)i != best && logits[i] > second)
            {
                second = logits[i];
            }
        }
        top2[0] = logits[best];
        top2[1] = second;
    }
    free(h);
    free(next);
    free(hn);
    return best;
}

/* ------------------------------------------------------------------------------------------ */
/* The reference's CPU path as written: every sum an f32 running sum in index order, as the
 * host references compute them (src/MatVec.cpp:52-60 HostMatVec for every projection and the LM
 * head, src/RmsNorm.cpp:194-216, src/SoftMax.cpp:164-191, src/Swiglu.cpp:56, src/Rope.cpp:48-51,
 * src/Sampler.cpp:32-43), composed into tools/reference_qwen2.py:100-166's step. This is the
 * timed CPU baseline; the double-accumulating oracle_decode_step above stays the checker. */

static void attention_f32(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out, uint32_t heads,
                          uint32_t kv_heads, uint32_t head_dim, uint32_t max_seq, int32_t pos, float scale)
{
    const uint32_t group = heads / kv_heads;
    const uint32_t keys = (uint32_t)pos + 1u;
#pragma omp parallel for schedule(static)
    for (int64_t hh = 0; hh < (int64_t)heads; ++hh)
    {
        const uint32_t h = (uint32_t)hh;
        const uint32_t g = h / group;
        const float* qh = q + (uint64_t)h * head_dim;
        const uint16_t* kbase = kcache + (uint64_t)g * max_seq * head_dim;
        const uint16_t* vbase = vcache + (uint64_t)g * max_seq * head_dim;
        float* scores = (float*)malloc(sizeof(float) * keys);
        float* probs = (float*)malloc(sizeof(float) * keys);
        for (uint32_t j = 0; j < keys; ++j)
        {
            float dot = 0.0f;
            for (uint32_t c = 0; c < head_dim; ++c)
            {
                dot += qh[c] * g_half_table[kbase[(uint64_t)j * head_dim + c]];
            }
            scores[j] = dot;
        }
        soft_max_row(scores, probs, keys, scale);
        for (uint32_t c = 0; c < head_dim; ++c)
        {
            float acc = 0.0f;
            for (uint32_t j = 0; j < keys; ++j)
            {
                acc += probs[j] * g_half_table[vbase[(uint64_t)j * head_dim + c]];
            }
            out[(uint64_t)h * head_dim + c] = acc;
        }
        free(scores);
        free(probs);
    }
}

int32_t oracle_decode_step_f32(const OracleQwen2* m, int32_t token, int32_t pos, float* logits)
{
    if (m == NULL || logits == NULL || token < 0 || (uint32_t)token >= m->vocab || pos < 0 ||
        (uint32_t)pos >= m->max_seq || m->heads % m->kv_heads != 0)
    {
        return -1;
    }
    ensure_half_table();
    const uint32_t hd = m->head_dim;
    const uint32_t qdim = m->heads * hd;
    const uint32_t kvdim = m->kv_heads * hd;
    const uint32_t qkv_rows = qdim + 2u * kvdim;
    const float theta_scale = powf(m->rope_base, -2.0f / (float)hd);
    const float attn_scale = 1.0f / sqrtf((float)hd);
    const uint32_t widest = m->ffn > qkv_rows ? m->ffn : qkv_rows;
    float* h = (float*)malloc(sizeof(float) * m->hidden);
    float* xn = (float*)malloc(sizeof(float) * m->hidden);
    float* x1 = (float*)malloc(sizeof(float) * m->hidden);
    float* o = (float*)malloc(sizeof(float) * m->hidden);
    float* qkv = (float*)malloc(sizeof(float) * widest);
    float* qr = (float*)malloc(sizeof(float) * qdim);
    float* kr = (float*)malloc(sizeof(float) * kvdim);
    float* attn = (float*)malloc(sizeof(float) * qdim);
    float* gate = (float*)malloc(sizeof(float) * m->ffn);
    float* up = (float*)malloc(sizeof(float) * m->ffn);

    oracle_get_rows_f16(m->token_embd, token, h, m->hidden);
    for (uint32_t l = 0; l < m->layers; ++l)
    {
        oracle_rms_norm(h, m->attn_norm[l], xn, 1, m->hidden, m->rms_eps);
        oracle_mat_vec_f16(m->attn_qkv[l], xn, qkv, qkv_rows, m->hidden, m->hidden);
        for (uint32_t r = 0; r < qkv_rows; ++r)
        {
            qkv[r] += m->attn_qkv_b[l][r];
        }
        oracle_rope_neox(qkv, qr, m->heads, hd, hd, pos, theta_scale);
        oracle_rope_neox(qkv + qdim, kr, m->kv_heads, hd, hd, pos, theta_scale);
        for (uint32_t g = 0; g < m->kv_heads; ++g)
        {
            for (uint32_t c = 0; c < hd; ++c)
            {
                const uint64_t slot = ((uint64_t)g * m->max_seq + (uint64_t)pos) * hd + c;
                m->kcache[l][slot] = oracle_float_to_half(kr[g * hd + c]);
                m->vcache[l][slot] = oracle_float_to_half(qkv[qdim + kvdim + g * hd + c]);
            }
        }
        attention_f32(qr, m->kcache[l], m->vcache[l], attn, m->heads, m->kv_heads, hd, m->max_seq, pos, attn_scale);
        oracle_mat_vec_f16(m->attn_out[l], attn, o, m->hidden, qdim, qdim);
        oracle_add(h, o, x1, m->hidden);
        oracle_rms_norm(x1, m->ffn_norm[l], xn, 1, m->hidden, m->rms_eps);
        oracle_mat_vec_f16(m->ffn_gate[l], xn, gate, m->ffn, m->hidden, m->hidden);
        oracle_mat_vec_f16(m->ffn_up[l], xn, up, m->ffn, m->hidden, m->hidden);
        oracle_swiglu(gate, up, qkv, m->ffn);
        oracle_mat_vec_f16(m->ffn_down[l], qkv, o, m->hidden, m->ffn, m->ffn);
        oracle_add(x1, o, h, m->hidden);
    }
    oracle_rms_norm(h, m->output_norm, xn, 1, m->hidden, m->rms_eps);
    const uint16_t* head = m->output != NULL ? m->output : m->token_embd;
    oracle_mat_vec_f16(head, xn, logits, m->vocab, m->hidden, m->hidden);
    const int32_t best = oracle_argmax(logits, m->vocab);
    free(h);
    free(xn);
    free(x1);
    free(o);
    free(qkv);
    free(qr);
    free(kr);
    free(attn);
    free(gate);
    free(up);
    return best;
}
