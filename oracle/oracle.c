/*
 * oracle.c - CPU restatement of toklet's scalar attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for tests/, smoke() and the
 * cpu_baseline leg of bench.py.  The product never links or calls it.
 *
 * Each function names the reference function it restates (file:line under
 * the toklet source tree).  Loop order, FP32/FP64 precision and the order of
 * validation checks follow the reference so that outputs and error codes are
 * comparable with its frozen fixtures.  Rust `usize` checked arithmetic is
 * restated with __builtin_*_overflow on size_t (both are 64-bit here).
 *
 * Parity pinning (which check fixes each function) is listed in the test
 * modules under tests/ that import this library.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* ---- error helpers: src/cpu/mod.rs:84-127 ---- */

static uint32_t fail(orc_error *err, uint32_t code, const char *tensor, size_t index,
                     size_t expected, size_t actual) {
    if (err) {
        err->code = code;
        err->tensor = tensor;
        err->index = index;
        err->expected = expected;
        err->actual = actual;
    }
    return code;
}

static uint32_t ok(orc_error *err) { return fail(err, ORC_OK, NULL, 0, 0, 0); }

#define TRY(expr)                        \
    do {                                 \
        uint32_t _rc = (expr);           \
        if (_rc != ORC_OK) return _rc;   \
    } while (0)

/* nonzero (src/cpu/mod.rs:84-90) */
static uint32_t nonzero(size_t value, const char *name, orc_error *err) {
    if (value == 0) return fail(err, ORC_ZERO_DIMENSION, name, 0, 0, 0);
    return ORC_OK;
}

/* product (src/cpu/mod.rs:92-94) */
static uint32_t product(size_t a, size_t b, size_t *out, orc_error *err) {
    if (__builtin_mul_overflow(a, b, out)) return fail(err, ORC_SIZE_OVERFLOW, NULL, 0, 0, 0);
    return ORC_OK;
}

static uint32_t checked_add(size_t a, size_t b, size_t *out, orc_error *err) {
    if (__builtin_add_overflow(a, b, out)) return fail(err, ORC_SIZE_OVERFLOW, NULL, 0, 0, 0);
    return ORC_OK;
}

/* length (src/cpu/mod.rs:96-106) */
static uint32_t length(const char *tensor, size_t actual, size_t expected, orc_error *err) {
    if (actual != expected) return fail(err, ORC_LENGTH, tensor, 0, expected, actual);
    return ORC_OK;
}

/* finite (src/cpu/mod.rs:108-114) */
static uint32_t finite(const char *tensor, const float *values, size_t len, orc_error *err) {
    for (size_t i = 0; i < len; ++i)
        if (!isfinite(values[i])) return fail(err, ORC_NON_FINITE, tensor, i, 0, 0);
    return ORC_OK;
}

static uint32_t invalid(const char *name, orc_error *err) {
    return fail(err, ORC_INVALID_PARAMETER, name, 0, 0, 0);
}

static uint32_t non_finite(const char *tensor, size_t index, orc_error *err) {
    return fail(err, ORC_NON_FINITE, tensor, index, 0, 0);
}

/* ---- rotary: src/cpu/attention.rs:10-64 ---- */

uint32_t orc_rotary(const float *input, size_t input_len, float *output, size_t output_len,
                    size_t tokens, size_t heads, size_t head_dim, size_t offset, float theta,
                    orc_error *err) {
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(heads, "heads", err));
    TRY(nonzero(head_dim, "head_dim", err));
    if (head_dim % 2 != 0) return invalid("rotary head_dim must be even", err);
    if (!isfinite(theta) || theta <= 0.0f) return invalid("theta must be finite and positive", err);
    size_t last;
    TRY(checked_add(offset, tokens - 1, &last, err));
    if ((unsigned __int128)last > ((unsigned __int128)1 << 53))
        return invalid("rotary positions must be at most 2^53", err);
    size_t token_stride, count;
    TRY(product(heads, head_dim, &token_stride, err));
    TRY(product(tokens, token_stride, &count, err));
    TRY(length("rotary input", input_len, count, err));
    TRY(length("rotary output", output_len, count, err));
    TRY(finite("rotary input", input, input_len, err));
    size_t half = head_dim / 2;
    for (size_t feature = 0; feature < half; ++feature) {
        double frequency = pow((double)theta, -(2.0 * (double)feature) / (double)head_dim);
        for (size_t token = 0; token < tokens; ++token) {
            double angle = (double)(offset + token) * frequency;
            float s = (float)sin(angle), c = (float)cos(angle);
            for (size_t head = 0; head < heads; ++head) {
                size_t first = token * token_stride + head * head_dim + feature;
                size_t second = first + half;
                float x = input[first] * c - input[second] * s;
                float y = input[second] * c + input[first] * s;
                if (!isfinite(x) || !isfinite(y))
                    return non_finite("rotary output", !isfinite(x) ? first : second, err);
                output[first] = x;
                output[second] = y;
            }
        }
    }
    return ok(err);
}

/* ---- proportional rotary: src/cpu/proportional_rotary.rs:32-91 ---- */

uint32_t orc_proportional_rotary(const float *input, size_t input_len, float *output,
                                 size_t output_len, size_t tokens, size_t heads,
                                 size_t head_dim, size_t rotated_dims, size_t offset,
                                 float base, float factor, orc_error *err) {
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(heads, "heads", err));
    TRY(nonzero(head_dim, "head_dim", err));
    if (head_dim % 2 != 0 || rotated_dims % 2 != 0 || rotated_dims > head_dim)
        return invalid("proportional rotary dimensions", err);
    if (!isfinite(base) || base <= 0.0f || !isfinite(factor) || factor <= 0.0f)
        return invalid("proportional rotary base/factor", err);
    size_t last;
    TRY(checked_add(offset, tokens - 1, &last, err));
    if ((unsigned __int128)last > ((unsigned __int128)1 << 53))
        return invalid("rotary positions must be at most 2^53", err);
    size_t stride, count;
    TRY(product(heads, head_dim, &stride, err));
    TRY(product(tokens, stride, &count, err));
    TRY(length("proportional rotary input", input_len, count, err));
    TRY(length("proportional rotary output", output_len, count, err));
    TRY(finite("proportional rotary input", input, input_len, err));
    memcpy(output, input, count * sizeof(float));
    for (size_t pair = 0; pair < rotated_dims / 2; ++pair) {
        double inverse =
            pow((double)base, -(2.0 * (double)pair) / (double)head_dim) / (double)factor;
        for (size_t token = 0; token < tokens; ++token) {
            double angle = (double)(offset + token) * inverse;
            float s = (float)sin(angle), c = (float)cos(angle);
            for (size_t head = 0; head < heads; ++head) {
                size_t first = token * stride + head * head_dim + pair;
                size_t second = first + head_dim / 2;
                float a = input[first] * c - input[second] * s;
                float b = input[second] * c + input[first] * s;
                if (!isfinite(a) || !isfinite(b))
                    return non_finite("proportional rotary output",
                                      !isfinite(a) ? first : second, err);
                output[first] = a;
                output[second] = b;
            }
        }
    }
    return ok(err);
}

/* ---- Llama 3 rotary: src/cpu/llama3_rotary.rs:13-146 ---- */

/* Llama3Scaling::new (src/cpu/llama3_rotary.rs:14-37): the FP32 parameters are
 * widened to FP64 once. */
uint32_t orc_llama3_scaling(float factor, float low, float high, size_t original,
                            orc_llama3 *out, orc_error *err) {
    if (!isfinite(factor) || factor < 1.0f || !isfinite(low) || low <= 0.0f ||
        !isfinite(high) || high <= low || original == 0 ||
        (unsigned __int128)original > ((unsigned __int128)1 << 53))
        return invalid("Llama3 rotary scaling", err);
    out->factor = (double)factor;
    out->low = (double)low;
    out->high = (double)high;
    out->original = (double)original;
    return ok(err);
}

/* Llama3Scaling::inverse_frequency (src/cpu/llama3_rotary.rs:44-61), in FP64:
 * wavelengths below original/high keep the ordinary frequency, those above
 * original/low divide it by factor, and the closed band between blends the two
 * linearly in original/wavelength. */
uint32_t orc_llama3_inverse_frequency(const orc_llama3 *s, double ordinary, double *out,
                                      orc_error *err) {
    if (!isfinite(ordinary) || ordinary <= 0.0) return invalid("Llama3 inverse frequency", err);
    const double wavelength = 6.283185307179586 / ordinary;  /* 2*pi in FP64 */
    double result;
    if (s->factor == 1.0 || wavelength < s->original / s->high) {
        result = ordinary;
    } else if (wavelength > s->original / s->low) {
        result = ordinary / s->factor;
    } else {
        const double smooth = (s->original / wavelength - s->low) / (s->high - s->low);
        result = (1.0 - smooth) * ordinary / s->factor + smooth * ordinary;
    }
    if (!isfinite(result) || result <= 0.0)
        return invalid("Llama3 scaled frequency underflow", err);
    *out = result;
    return ok(err);
}

/* llama3_rotary (src/cpu/llama3_rotary.rs:87-146): split-half pairs over the
 * whole head, frequency theta^(-2j/D) scaled as above, angle and sine/cosine
 * in FP64, rounded to FP32, FP32 rotation. */
uint32_t orc_llama3_rotary(const float *input, size_t input_len, float *output,
                           size_t output_len, size_t tokens, size_t heads, size_t head_dim,
                           size_t offset, float theta, const orc_llama3 *scaling,
                           orc_error *err) {
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(heads, "heads", err));
    TRY(nonzero(head_dim, "head_dim", err));
    if (head_dim % 2 != 0) return invalid("Llama3 rotary head_dim must be even", err);
    if (!isfinite(theta) || theta <= 0.0f) return invalid("theta must be finite and positive", err);
    size_t last;
    TRY(checked_add(offset, tokens - 1, &last, err));
    if ((unsigned __int128)last > ((unsigned __int128)1 << 53))
        return invalid("rotary positions must be at most 2^53", err);
    size_t stride, count;
    TRY(product(heads, head_dim, &stride, err));
    TRY(product(tokens, stride, &count, err));
    TRY(length("Llama3 rotary input", input_len, count, err));
    TRY(length("Llama3 rotary output", output_len, count, err));
    TRY(finite("Llama3 rotary input", input, input_len, err));
    for (size_t pair = 0; pair < head_dim / 2; ++pair) {
        const double ordinary = pow((double)theta, -(2.0 * (double)pair) / (double)head_dim);
        double inverse;
        TRY(orc_llama3_inverse_frequency(scaling, ordinary, &inverse, err));
        for (size_t token = 0; token < tokens; ++token) {
            const double angle = (double)(offset + token) * inverse;
            const float s = (float)sin(angle), c = (float)cos(angle);
            for (size_t head = 0; head < heads; ++head) {
                const size_t first = token * stride + head * head_dim + pair;
                const size_t second = first + head_dim / 2;
                const float a = input[first] * c - input[second] * s;
                const float b = input[second] * c + input[first] * s;
                if (!isfinite(a) || !isfinite(b))
                    return non_finite("Llama3 rotary output", !isfinite(a) ? first : second, err);
                output[first] = a;
                output[second] = b;
            }
        }
    }
    return ok(err);
}

/* ---- rmsnorm: src/cpu/reductions.rs:8-49 ---- */

uint32_t orc_rmsnorm(const float *input, size_t input_len, const float *weight,
                     size_t weight_len, float *output, size_t output_len, size_t tokens,
                     size_t hidden, float epsilon, orc_error *err) {
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(hidden, "hidden", err));
    size_t count;
    TRY(product(tokens, hidden, &count, err));
    TRY(length("input", input_len, count, err));
    TRY(length("output", output_len, count, err));
    TRY(length("norm weight", weight_len, hidden, err));
    if (!isfinite(epsilon) || epsilon <= 0.0f)
        return invalid("epsilon must be finite and positive", err);
    TRY(finite("input", input, input_len, err));
    TRY(finite("norm weight", weight, weight_len, err));
    for (size_t row = 0; row < tokens; ++row) {
        const float *source = input + row * hidden;
        float *destination = output + row * hidden;
        double squares = 0.0;
        for (size_t column = 0; column < hidden; ++column) {
            double x = (double)source[column];
            squares += x * x;
        }
        double denominator = sqrt(squares / (double)hidden + (double)epsilon);
        for (size_t column = 0; column < hidden; ++column) {
            float value = (float)((double)source[column] / denominator * (double)weight[column]);
            if (!isfinite(value)) return non_finite("output", row * hidden + column, err);
            destination[column] = value;
        }
    }
    return ok(err);
}

/* ---- softmax: src/cpu/reductions.rs:57-106 ---- */

uint32_t orc_softmax(const float *scores, size_t scores_len, const uint8_t *mask,
                     size_t mask_len, float *output, size_t output_len, size_t rows,
                     size_t columns, orc_error *err) {
    TRY(nonzero(rows, "rows", err));
    TRY(nonzero(columns, "columns", err));
    size_t count;
    TRY(product(rows, columns, &count, err));
    TRY(length("scores", scores_len, count, err));
    TRY(length("output", output_len, count, err));
    TRY(finite("scores", scores, scores_len, err));
    if (mask) {
        TRY(length("mask", mask_len, count, err));
        for (size_t row = 0; row < rows; ++row) {
            int any = 0;
            for (size_t c = 0; c < columns; ++c) any |= mask[row * columns + c] != 0;
            if (!any) return fail(err, ORC_FULLY_MASKED, NULL, row, 0, 0);
        }
    }
    for (size_t row = 0; row < rows; ++row) {
        const float *source = scores + row * columns;
        float *destination = output + row * columns;
        const uint8_t *row_mask = mask ? mask + row * columns : NULL;
        double maximum = -INFINITY;
        for (size_t c = 0; c < columns; ++c)
            if (!row_mask || row_mask[c]) maximum = fmax(maximum, (double)source[c]);
        double sum = 0.0;
        for (size_t c = 0; c < columns; ++c)
            if (!row_mask || row_mask[c]) sum += exp((double)source[c] - maximum);
        for (size_t c = 0; c < columns; ++c)
            destination[c] =
                (!row_mask || row_mask[c]) ? (float)(exp((double)source[c] - maximum) / sum) : 0.0f;
    }
    return ok(err);
}

/* ---- full-prefix attention: src/cpu/attention.rs:85-178 ---- */

uint32_t orc_attention(const float *q, size_t q_len, const float *k, size_t k_len,
                       const float *v, size_t v_len, float *context, size_t context_len,
                       float *scores, size_t scores_len, float *probabilities,
                       size_t probabilities_len, const orc_attention_shape *shape,
                       orc_error *err) {
    size_t tokens = shape->tokens, query_heads = shape->query_heads;
    size_t kv_heads = shape->kv_heads, head_dim = shape->head_dim;
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(query_heads, "query_heads", err));
    TRY(nonzero(kv_heads, "kv_heads", err));
    TRY(nonzero(head_dim, "head_dim", err));
    if (query_heads % kv_heads != 0) return invalid("query_heads must be divisible by kv_heads", err);
    size_t q_stride, kv_stride, q_count, kv_count, score_count, tmp;
    TRY(product(query_heads, head_dim, &q_stride, err));
    TRY(product(kv_heads, head_dim, &kv_stride, err));
    TRY(product(tokens, q_stride, &q_count, err));
    TRY(product(tokens, kv_stride, &kv_count, err));
    TRY(product(query_heads, tokens, &tmp, err));
    TRY(product(tmp, tokens, &score_count, err));
    TRY(length("q", q_len, q_count, err));
    TRY(length("k", k_len, kv_count, err));
    TRY(length("v", v_len, kv_count, err));
    TRY(length("attention context", context_len, q_count, err));
    TRY(length("attention scores", scores_len, score_count, err));
    TRY(length("attention probabilities", probabilities_len, score_count, err));
    TRY(finite("q", q, q_len, err));
    TRY(finite("k", k, k_len, err));
    TRY(finite("v", v, v_len, err));
    size_t group = query_heads / kv_heads;
    float denominator = sqrtf((float)head_dim);
    for (size_t head = 0; head < query_heads; ++head) {
        size_t kv_head = head / group;
        for (size_t query = 0; query < tokens; ++query) {
            size_t q_start = query * q_stride + head * head_dim;
            size_t row_start = (head * tokens + query) * tokens;
            for (size_t key = 0; key < tokens; ++key) {
                size_t k_start = key * kv_stride + kv_head * head_dim;
                float dot = 0.0f;
                for (size_t f = 0; f < head_dim; ++f) dot += q[q_start + f] * k[k_start + f];
                float score = dot / denominator;
                if (!isfinite(score)) return non_finite("attention scores", row_start + key, err);
                scores[row_start + key] = score;
            }
        }
    }
    for (size_t head = 0; head < query_heads; ++head) {
        size_t kv_head = head / group;
        for (size_t query = 0; query < tokens; ++query) {
            size_t row_start = (head * tokens + query) * tokens;
            size_t included_end = row_start + query + 1;
            TRY(orc_softmax(scores + row_start, query + 1, NULL, 0, probabilities + row_start,
                            query + 1, 1, query + 1, err));
            for (size_t i = included_end; i < row_start + tokens; ++i) probabilities[i] = 0.0f;
            size_t context_start = query * q_stride + head * head_dim;
            for (size_t f = 0; f < head_dim; ++f) {
                float value = 0.0f;
                for (size_t key = 0; key <= query; ++key)
                    value += probabilities[row_start + key] * v[key * kv_stride + kv_head * head_dim + f];
                if (!isfinite(value)) return non_finite("attention context", context_start + f, err);
                context[context_start + f] = value;
            }
        }
    }
    return ok(err);
}

/* ---- cached chunk attention: src/cpu/attention.rs:201-296 ---- */

uint32_t orc_attention_cached(const float *q, size_t q_len, const float *k, size_t k_len,
                              const float *v, size_t v_len, float *context,
                              size_t context_len, float *scores, size_t scores_len,
                              float *probabilities, size_t probabilities_len,
                              const orc_cached_shape *shape, orc_error *err) {
    size_t tokens = shape->tokens, query_heads = shape->query_heads;
    size_t kv_heads = shape->kv_heads, head_dim = shape->head_dim;
    size_t capacity = shape->capacity, offset = shape->offset;
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(query_heads, "query_heads", err));
    TRY(nonzero(kv_heads, "kv_heads", err));
    TRY(nonzero(head_dim, "head_dim", err));
    TRY(nonzero(capacity, "cache capacity", err));
    if (query_heads % kv_heads != 0) return invalid("query_heads must be divisible by kv_heads", err);
    size_t end;
    TRY(checked_add(offset, tokens, &end, err));
    if (end > capacity) return invalid("cache capacity exceeded", err);
    size_t q_stride, q_count, head_stride, kv_count;
    TRY(product(query_heads, head_dim, &q_stride, err));
    TRY(product(tokens, q_stride, &q_count, err));
    TRY(product(capacity, head_dim, &head_stride, err));
    TRY(product(kv_heads, head_stride, &kv_count, err));
    TRY(length("q", q_len, q_count, err));
    TRY(length("k cache", k_len, kv_count, err));
    TRY(length("v cache", v_len, kv_count, err));
    TRY(length("attention context", context_len, q_count, err));
    TRY(length("attention scores", scores_len, capacity, err));
    TRY(length("attention probabilities", probabilities_len, capacity, err));
    TRY(finite("q", q, q_len, err));
    for (size_t head = 0; head < kv_heads; ++head) {
        size_t start = head * head_stride;
        TRY(finite("k cache prefix", k + start, end * head_dim, err));
        TRY(finite("v cache prefix", v + start, end * head_dim, err));
    }
    size_t group = query_heads / kv_heads;
    float denominator = sqrtf((float)head_dim);
    for (size_t head = 0; head < query_heads; ++head) {
        size_t kv_start = (head / group) * head_stride;
        for (size_t query = 0; query < tokens; ++query) {
            size_t visible = offset + query + 1;
            size_t q_start = query * q_stride + head * head_dim;
            for (size_t key = 0; key < visible; ++key) {
                size_t start = kv_start + key * head_dim;
                float dot = 0.0f;
                for (size_t f = 0; f < head_dim; ++f) dot += q[q_start + f] * k[start + f];
                scores[key] = dot / denominator;
                if (!isfinite(scores[key])) return non_finite("attention scores", key, err);
            }
            TRY(orc_softmax(scores, visible, NULL, 0, probabilities, visible, 1, visible, err));
            for (size_t f = 0; f < head_dim; ++f) {
                float value = 0.0f;
                for (size_t key = 0; key < visible; ++key)
                    value += probabilities[key] * v[kv_start + key * head_dim + f];
                if (!isfinite(value)) return non_finite("attention context", q_start + f, err);
                context[q_start + f] = value;
            }
        }
    }
    return ok(err);
}

/* Score softcap used inside window/span attention (this build's extension of
 * src/cpu/softcap.rs:16-29 to attention scores): FP64 divide/tanh/multiply of
 * the stored FP32 score, one rounding back to FP32. */
static float capped(float score, float softcap) {
    if (softcap == 0.0f) return score;
    double cap = (double)softcap;
    return (float)(tanh((double)score / cap) * cap);
}

/* First visible key of `position` (absolute), as in window_attention.rs:105-107. */
static size_t first_visible(size_t key_start, size_t position, int has_window, size_t window) {
    if (!has_window) return key_start;
    size_t lower = position >= window - 1 ? position - (window - 1) : 0;
    return key_start > lower ? key_start : lower;
}

/* ---- window attention: src/cpu/window_attention.rs:36-168 ---- */

uint32_t orc_window_attention(const float *q, size_t q_len, const float *k, size_t k_len,
                              const float *v, size_t v_len, float *context,
                              size_t context_len, float *scores, size_t scores_len,
                              float *probabilities, size_t probabilities_len,
                              const orc_window_shape *s, orc_error *err) {
    TRY(nonzero(s->queries, "queries", err));
    TRY(nonzero(s->keys, "keys", err));
    TRY(nonzero(s->query_heads, "query_heads", err));
    TRY(nonzero(s->kv_heads, "kv_heads", err));
    TRY(nonzero(s->head_dim, "head_dim", err));
    if (s->keys > s->capacity || s->query_heads % s->kv_heads != 0)
        return invalid("attention capacity/head mapping", err);
    if ((s->has_window && s->window == 0) || !isfinite(s->scale) || s->scale <= 0.0f)
        return invalid("attention window/scale", err);
    if (s->softcap != 0.0f && (!isfinite(s->softcap) || s->softcap < 0.0f))
        return invalid("attention score softcap", err);
    size_t key_end, query_last;
    TRY(checked_add(s->key_start, s->keys - 1, &key_end, err));
    TRY(checked_add(s->query_start, s->queries - 1, &query_last, err));
    size_t query_stride, query_count, kv_stride, kv_count, used_kv, tmp, scratch_count;
    TRY(product(s->query_heads, s->head_dim, &query_stride, err));
    TRY(product(s->queries, query_stride, &query_count, err));
    TRY(product(s->capacity, s->head_dim, &kv_stride, err));
    TRY(product(s->kv_heads, kv_stride, &kv_count, err));
    TRY(product(s->keys, s->head_dim, &used_kv, err));
    TRY(product(s->query_heads, s->queries, &tmp, err));
    TRY(product(tmp, s->keys, &scratch_count, err));
    TRY(length("attention query", q_len, query_count, err));
    TRY(length("attention key", k_len, kv_count, err));
    TRY(length("attention value", v_len, kv_count, err));
    TRY(length("attention context", context_len, query_count, err));
    TRY(length("attention scores", scores_len, scratch_count, err));
    TRY(length("attention probabilities", probabilities_len, scratch_count, err));
    TRY(finite("attention query", q, q_len, err));
    for (size_t head = 0; head < s->kv_heads; ++head) {
        size_t start = head * kv_stride;
        for (size_t i = 0; i < used_kv; ++i)
            if (!isfinite(k[start + i])) return non_finite("attention key", start + i, err);
        for (size_t i = 0; i < used_kv; ++i)
            if (!isfinite(v[start + i])) return non_finite("attention value", start + i, err);
    }
    for (size_t query = 0; query < s->queries; ++query) {
        size_t position = s->query_start + query;
        size_t first = first_visible(s->key_start, position, s->has_window, s->window);
        size_t last = key_end < position ? key_end : position;
        if (first > last) return fail(err, ORC_FULLY_MASKED, NULL, query, 0, 0);
    }
    size_t group = s->query_heads / s->kv_heads;
    for (size_t head = 0; head < s->query_heads; ++head) {
        size_t kv_base = (head / group) * kv_stride;
        for (size_t query = 0; query < s->queries; ++query) {
            size_t q_base = query * query_stride + head * s->head_dim;
            size_t row = (head * s->queries + query) * s->keys;
            for (size_t key = 0; key < s->keys; ++key) {
                size_t k_base = kv_base + key * s->head_dim;
                double sum = 0.0;
                for (size_t f = 0; f < s->head_dim; ++f)
                    sum += (double)q[q_base + f] * (double)k[k_base + f];
                float score = capped((float)(sum * (double)s->scale), s->softcap);
                if (!isfinite(score)) return non_finite("attention scores", row + key, err);
                scores[row + key] = score;
            }
            size_t position = s->query_start + query;
            size_t first = first_visible(s->key_start, position, s->has_window, s->window) - s->key_start;
            size_t last = (key_end < position ? key_end : position) - s->key_start;
            float maximum = -INFINITY;
            for (size_t key = first; key <= last; ++key)
                maximum = fmaxf(maximum, scores[row + key]);
            double denominator = 0.0;
            for (size_t key = first; key <= last; ++key)
                denominator += exp((double)scores[row + key] - (double)maximum);
            for (size_t key = 0; key < s->keys; ++key) probabilities[row + key] = 0.0f;
            for (size_t key = first; key <= last; ++key)
                probabilities[row + key] =
                    (float)(exp((double)scores[row + key] - (double)maximum) / denominator);
            for (size_t f = 0; f < s->head_dim; ++f) {
                double sum = 0.0;
                for (size_t key = first; key <= last; ++key)
                    sum += (double)probabilities[row + key] * (double)v[kv_base + key * s->head_dim + f];
                float value = (float)sum;
                if (!isfinite(value)) return non_finite("attention context", q_base + f, err);
                context[q_base + f] = value;
            }
        }
    }
    return ok(err);
}

/* ---- span attention: src/cpu/span_attention.rs:42-220 ---- */

uint32_t orc_span_attention(const float *q, size_t q_len, const orc_segment segments[3],
                            float *context, size_t context_len, float *scores,
                            size_t scores_len, float *probabilities, size_t probabilities_len,
                            const orc_span_shape *s, orc_error *err) {
    TRY(nonzero(s->queries, "queries", err));
    TRY(nonzero(s->keys, "keys", err));
    TRY(nonzero(s->query_heads, "query_heads", err));
    TRY(nonzero(s->kv_heads, "kv_heads", err));
    TRY(nonzero(s->head_dim, "head_dim", err));
    if (s->query_heads % s->kv_heads != 0 || (s->has_window && s->window == 0) ||
        !isfinite(s->scale) || s->scale <= 0.0f)
        return invalid("segmented attention heads/window/scale", err);
    if (s->softcap != 0.0f && (!isfinite(s->softcap) || s->softcap < 0.0f))
        return invalid("attention score softcap", err);
    size_t key_end, query_last;
    TRY(checked_add(s->key_start, s->keys - 1, &key_end, err));
    TRY(checked_add(s->query_start, s->queries - 1, &query_last, err));
    size_t query_stride, query_count, tmp, scratch_count;
    TRY(product(s->query_heads, s->head_dim, &query_stride, err));
    TRY(product(s->queries, query_stride, &query_count, err));
    TRY(product(s->query_heads, s->queries, &tmp, err));
    TRY(product(tmp, s->keys, &scratch_count, err));
    TRY(length("attention query", q_len, query_count, err));
    TRY(length("attention context", context_len, query_count, err));
    TRY(length("attention scores", scores_len, scratch_count, err));
    TRY(length("attention probabilities", probabilities_len, scratch_count, err));
    size_t keys = 0;
    for (int i = 0; i < 3; ++i) {
        const orc_segment *seg = &segments[i];
        size_t rows, expected = 0;
        TRY(product(seg->keys, s->head_dim, &rows, err));
        if (seg->keys != 0) {
            if (seg->head_stride < rows) return invalid("attention segment heads overlap", err);
            size_t start;
            TRY(checked_add(s->key_start, keys, &start, err));
            if (seg->key_start != start) return invalid("attention segment logical origin", err);
            size_t heads_part;
            TRY(product(s->kv_heads - 1, seg->head_stride, &heads_part, err));
            TRY(checked_add(heads_part, rows, &expected, err));
        }
        TRY(length("attention segment key", seg->k_len, expected, err));
        TRY(length("attention segment value", seg->v_len, expected, err));
        TRY(checked_add(keys, seg->keys, &keys, err));
    }
    TRY(length("attention segment keys", keys, s->keys, err));
    TRY(finite("attention query", q, q_len, err));
    for (int i = 0; i < 3; ++i) {
        const orc_segment *seg = &segments[i];
        if (seg->keys == 0) continue;
        size_t rows = seg->keys * s->head_dim;
        for (size_t head = 0; head < s->kv_heads; ++head) {
            size_t start = head * seg->head_stride;
            for (size_t j = 0; j < rows; ++j)
                if (!isfinite(seg->k[start + j]))
                    return non_finite("attention segment key", start + j, err);
            for (size_t j = 0; j < rows; ++j)
                if (!isfinite(seg->v[start + j]))
                    return non_finite("attention segment value", start + j, err);
        }
    }
    for (size_t query = 0; query < s->queries; ++query) {
        size_t position = s->query_start + query;
        size_t first = first_visible(s->key_start, position, s->has_window, s->window);
        size_t last = key_end < position ? key_end : position;
        if (first > last) return fail(err, ORC_FULLY_MASKED, NULL, query, 0, 0);
    }
    size_t group = s->query_heads / s->kv_heads;
    for (size_t head = 0; head < s->query_heads; ++head) {
        size_t kv_head = head / group;
        for (size_t query = 0; query < s->queries; ++query) {
            size_t q_base = query * query_stride + head * s->head_dim;
            size_t row = (head * s->queries + query) * s->keys;
            size_t logical = 0;
            for (int i = 0; i < 3; ++i) {
                const orc_segment *seg = &segments[i];
                if (seg->keys == 0) continue;
                size_t base = kv_head * seg->head_stride;
                for (size_t key = 0; key < seg->keys; ++key) {
                    size_t k_base = base + key * s->head_dim;
                    double sum = 0.0;
                    for (size_t f = 0; f < s->head_dim; ++f)
                        sum += (double)q[q_base + f] * (double)seg->k[k_base + f];
                    float score = capped((float)(sum * (double)s->scale), s->softcap);
                    if (!isfinite(score))
                        return non_finite("attention scores", row + logical + key, err);
                    scores[row + logical + key] = score;
                }
                logical += seg->keys;
            }
            size_t position = s->query_start + query;
            size_t first = first_visible(s->key_start, position, s->has_window, s->window) - s->key_start;
            size_t last = (key_end < position ? key_end : position) - s->key_start;
            float maximum = -INFINITY;
            for (size_t key = first; key <= last; ++key)
                maximum = fmaxf(maximum, scores[row + key]);
            double denominator = 0.0;
            for (size_t key = first; key <= last; ++key)
                denominator += exp((double)scores[row + key] - (double)maximum);
            for (size_t key = 0; key < s->keys; ++key) probabilities[row + key] = 0.0f;
            for (size_t key = first; key <= last; ++key)
                probabilities[row + key] =
                    (float)(exp((double)scores[row + key] - (double)maximum) / denominator);
            for (size_t f = 0; f < s->head_dim; ++f) {
                double sum = 0.0;
                size_t logical2 = 0;
                for (int i = 0; i < 3; ++i) {
                    const orc_segment *seg = &segments[i];
                    if (seg->keys == 0) continue;
                    size_t begin = first > logical2 ? first - logical2 : 0;
                    if (begin > seg->keys) begin = seg->keys;
                    size_t stop = last + 1 > logical2 ? last + 1 - logical2 : 0;
                    if (stop > seg->keys) stop = seg->keys;
                    size_t base = kv_head * seg->head_stride;
                    for (size_t key = begin; key < stop; ++key)
                        sum += (double)probabilities[row + logical2 + key] *
                               (double)seg->v[base + key * s->head_dim + f];
                    logical2 += seg->keys;
                }
                float value = (float)sum;
                if (!isfinite(value)) return non_finite("attention context", q_base + f, err);
                context[q_base + f] = value;
            }
        }
    }
    return ok(err);
}

/* ---- logit softcap: src/cpu/softcap.rs:16-29 ---- */

uint32_t orc_logit_softcap(float *logits, size_t len, float cap, orc_error *err) {
    TRY(nonzero(len, "logit softcap width", err));
    if (!isfinite(cap) || cap <= 0.0f) return invalid("logit softcap", err);
    TRY(finite("logits", logits, len, err));
    double c = (double)cap;
    for (size_t i = 0; i < len; ++i) logits[i] = (float)(tanh((double)logits[i] / c) * c);
    return ok(err);
}

/* ---- ring geometry: src/model/window_rows.rs:24-88 ---- */

size_t orc_view_start(size_t offset, int has_window, size_t window) {
    if (!has_window) return 0;
    return offset >= window - 1 ? offset - (window - 1) : 0;
}

void orc_old_spans(size_t capacity, size_t offset, int has_window, size_t window,
                   size_t out[6]) {
    size_t start = orc_view_start(offset, has_window, window);
    size_t old = offset - start;
    size_t slot = start % capacity;
    size_t first = old < capacity - slot ? old : capacity - slot;
    out[0] = start;
    out[1] = slot;
    out[2] = first;
    out[3] = start + first;
    out[4] = 0;
    out[5] = old - first;
}

void orc_copy_runs(size_t capacity, size_t offset, size_t tokens, int sliding, size_t out[6]) {
    size_t first_new = sliding ? (tokens > capacity ? tokens - capacity : 0) : 0;
    /* (offset + first_new) % capacity, computed without wrapping near SIZE_MAX */
    size_t slot = sliding ? (offset % capacity + first_new % capacity) % capacity : offset;
    size_t count = tokens - first_new;
    size_t first = count < capacity - slot ? count : capacity - slot;
    out[0] = first_new;
    out[1] = slot;
    out[2] = first;
    out[3] = first_new + first;
    out[4] = 0;
    out[5] = count - first;
}

/* ---- greedy argmax: src/sampling.rs:5-18 ---- */

/* ---- matmul: src/cpu/mod.rs:140-158, 183-247 (the FP32 path) ---- */

uint32_t orc_matmul(const float *input, size_t input_len, const float *weights,
                    size_t weights_len, const float *bias, size_t bias_len, float *output,
                    size_t output_len, size_t tokens, size_t in_features, size_t out_features,
                    orc_error *err) {
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(in_features, "in_features", err));
    TRY(nonzero(out_features, "out_features", err));
    size_t count;
    TRY(product(tokens, in_features, &count, err));
    TRY(length("input", input_len, count, err));
    TRY(product(out_features, in_features, &count, err));
    TRY(length("weights", weights_len, count, err));
    TRY(product(tokens, out_features, &count, err));
    TRY(length("output", output_len, count, err));
    if (bias) {
        TRY(length("bias", bias_len, out_features, err));
        TRY(finite("bias", bias, bias_len, err));
    }
    TRY(finite("input", input, input_len, err));
    TRY(finite("weights", weights, weights_len, err));
    for (size_t token = 0; token < tokens; ++token) {
        const float *row = input + token * in_features;
        for (size_t feature = 0; feature < out_features; ++feature) {
            const float *w = weights + feature * in_features;
            float sum = 0.0f;
            for (size_t i = 0; i < in_features; ++i) sum += row[i] * w[i];
            if (bias) sum += bias[feature];
            if (!isfinite(sum)) return non_finite("output", token * out_features + feature, err);
            output[token * out_features + feature] = sum;
        }
    }
    return ok(err);
}

uint32_t orc_greedy(const float *logits, size_t len, uint32_t *token, orc_error *err) {
    TRY(nonzero(len, "vocabulary", err));
    if (len - 1 > (size_t)UINT32_MAX) return invalid("vocabulary IDs must fit u32", err);
    TRY(finite("logits", logits, len, err));
    size_t best = 0;
    for (size_t i = 1; i < len; ++i)
        if (logits[i] > logits[best]) best = i;
    *token = (uint32_t)best;
    return ok(err);
}
