/*
 * oracle.h - CPU restatement of toklet's scalar attention operators.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libtokhip, the
 * toklet_amd package) links, loads or calls this library.  It is the parity
 * checker used by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg, and nothing else.
 *
 * Every function restates one reference function with the same loop order,
 * the same FP32/FP64 precision mix and the same validation order, so that its
 * error codes and outputs can be compared with the reference's frozen
 * fixtures.  Build with -O2 -ffp-contract=off (no FMA contraction, as Rust
 * does not contract) and glibc libm (Rust's f64::exp/tanh/sin/cos/powf call
 * the platform libm on Linux).
 *
 * Error codes mirror toklet::cpu::Error (src/cpu/mod.rs:47-68).
 */
#ifndef TOKLET_ORACLE_H
#define TOKLET_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_ZERO_DIMENSION = 1,
    ORC_SIZE_OVERFLOW = 2,
    ORC_LENGTH = 3,
    ORC_TOKEN = 4,
    ORC_NON_FINITE = 5,
    ORC_INVALID_PARAMETER = 6,
    ORC_FULLY_MASKED = 7,
};

/* One error value: code plus the payload of the matching Rust variant. */
typedef struct orc_error {
    uint32_t code;
    const char *tensor;   /* Length/NonFinite tensor, ZeroDimension/InvalidParameter name */
    size_t index;         /* NonFinite index, FullyMasked row */
    size_t expected;      /* Length */
    size_t actual;        /* Length */
} orc_error;

/* src/cpu/attention.rs:67-72 */
typedef struct orc_attention_shape {
    size_t tokens, query_heads, kv_heads, head_dim;
} orc_attention_shape;

/* src/cpu/attention.rs:181-189 */
typedef struct orc_cached_shape {
    size_t tokens, query_heads, kv_heads, head_dim, capacity, offset;
} orc_cached_shape;

/* src/cpu/window_attention.rs:6-17.  Option<usize> window is (has_window, window).
 * softcap is this build's score-softcap extension: 0 disables it. */
typedef struct orc_window_shape {
    size_t queries, keys, capacity, query_heads, kv_heads, head_dim;
    size_t query_start, key_start;
    int has_window;
    size_t window;
    float scale;
    float softcap;
} orc_window_shape;

/* src/cpu/span_attention.rs:9-16 (slices are pointer + element length). */
typedef struct orc_segment {
    const float *k;
    size_t k_len;
    const float *v;
    size_t v_len;
    size_t keys, head_stride, key_start;
} orc_segment;

/* src/cpu/span_attention.rs:18-28, plus the softcap extension. */
typedef struct orc_span_shape {
    size_t queries, keys, query_heads, kv_heads, head_dim;
    size_t query_start, key_start;
    int has_window;
    size_t window;
    float scale;
    float softcap;
} orc_span_shape;

uint32_t orc_rotary(const float *input, size_t input_len, float *output, size_t output_len,
                    size_t tokens, size_t heads, size_t head_dim, size_t offset, float theta,
                    orc_error *err);

uint32_t orc_proportional_rotary(const float *input, size_t input_len, float *output,
                                 size_t output_len, size_t tokens, size_t heads,
                                 size_t head_dim, size_t rotated_dims, size_t offset,
                                 float base, float factor, orc_error *err);

/* Llama3Scaling (src/cpu/llama3_rotary.rs:6-11): parameters widened to FP64. */
typedef struct orc_llama3 {
    double factor, low, high, original;
} orc_llama3;

uint32_t orc_llama3_scaling(float factor, float low, float high, size_t original,
                            orc_llama3 *out, orc_error *err);

uint32_t orc_llama3_inverse_frequency(const orc_llama3 *s, double ordinary, double *out,
                                      orc_error *err);

uint32_t orc_llama3_rotary(const float *input, size_t input_len, float *output,
                           size_t output_len, size_t tokens, size_t heads, size_t head_dim,
                           size_t offset, float theta, const orc_llama3 *scaling,
                           orc_error *err);

uint32_t orc_rmsnorm(const float *input, size_t input_len, const float *weight,
                     size_t weight_len, float *output, size_t output_len, size_t tokens,
                     size_t hidden, float epsilon, orc_error *err);

/* mask: NULL or `rows*columns` bytes, nonzero = included. */
uint32_t orc_softmax(const float *scores, size_t scores_len, const uint8_t *mask,
                     size_t mask_len, float *output, size_t output_len, size_t rows,
                     size_t columns, orc_error *err);

uint32_t orc_attention(const float *q, size_t q_len, const float *k, size_t k_len,
                       const float *v, size_t v_len, float *context, size_t context_len,
                       float *scores, size_t scores_len, float *probabilities,
                       size_t probabilities_len, const orc_attention_shape *shape,
                       orc_error *err);

uint32_t orc_attention_cached(const float *q, size_t q_len, const float *k, size_t k_len,
                              const float *v, size_t v_len, float *context,
                              size_t context_len, float *scores, size_t scores_len,
                              float *probabilities, size_t probabilities_len,
                              const orc_cached_shape *shape, orc_error *err);

uint32_t orc_window_attention(const float *q, size_t q_len, const float *k, size_t k_len,
                              const float *v, size_t v_len, float *context,
                              size_t context_len, float *scores, size_t scores_len,
                              float *probabilities, size_t probabilities_len,
                              const orc_window_shape *shape, orc_error *err);

uint32_t orc_span_attention(const float *q, size_t q_len, const orc_segment segments[3],
                            float *context, size_t context_len, float *scores,
                            size_t scores_len, float *probabilities, size_t probabilities_len,
                            const orc_span_shape *shape, orc_error *err);

uint32_t orc_logit_softcap(float *logits, size_t len, float cap, orc_error *err);

/* src/model/window_rows.rs:8-88: ring geometry (spans are {position, slot, rows},
 * copy runs are {source_row, slot, rows}). has_window selects Option<usize>. */
size_t orc_view_start(size_t offset, int has_window, size_t window);
void orc_old_spans(size_t capacity, size_t offset, int has_window, size_t window,
                   size_t out[6]);
void orc_copy_runs(size_t capacity, size_t offset, size_t tokens, int sliding, size_t out[6]);

/* Greedy argmax with the lowest index on ties (src/sampling.rs:5-18). */
uint32_t orc_matmul(const float *input, size_t input_len, const float *weights,
                    size_t weights_len, const float *bias, size_t bias_len, float *output,
                    size_t output_len, size_t tokens, size_t in_features, size_t out_features,
                    orc_error *err);
uint32_t orc_greedy(const float *logits, size_t len, uint32_t *token, orc_error *err);

#ifdef __cplusplus
}
#endif
#endif
