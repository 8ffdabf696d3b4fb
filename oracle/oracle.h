/*
 * CPU oracle for the Qwen3 batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's CPU engine
 * (metal_infrence_engine/src/cpu_inference.rs): the HIP engine's results are compared against
 * it, and it is timed as the CPU baseline. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. The product path never calls it.
 *
 * Every function cites the reference line it restates. Op order is kept exactly: separate
 * f32 multiply and add (built with -ffp-contract=off, no fast-math), the 8-accumulator fold
 * of dot_bf16, sequential iterator sums, (x*s)*w in rmsnorm, divide-by-sum in softmax, and
 * glibc powf/sinf/cosf/expf, which are what Rust's f32 methods call on Linux.
 */
#ifndef QE_ORACLE_H
#define QE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* cpu_inference.rs:20-33 (Config; the subset of config.json the forward pass reads) */
typedef struct {
  uint64_t hidden_size;
  uint64_t intermediate_size;
  uint64_t num_hidden_layers;
  uint64_t num_attention_heads;
  uint64_t num_key_value_heads;
  uint64_t head_dim;
  uint64_t vocab_size;
  float rms_norm_eps;
  float rope_theta;
  uint32_t eos_token_id;
} or_config;

typedef struct or_model or_model;
typedef struct or_kvcache or_kvcache;

/* status codes */
enum {
  OR_OK = 0,
  OR_ERR_IO = 1,        /* file missing / unreadable (io::Error) */
  OR_ERR_FORMAT = 2,    /* bad safetensors header or config.json (serde error / assert) */
  OR_ERR_TENSOR = 3,    /* missing tensor, wrong dtype, or size mismatch (Model::weight panics) */
  OR_ERR_POS = 4,       /* pos != number of cached positions (the reference indexes out of bounds) */
  OR_ERR_ARG = 5
};

/* cpu_inference.rs:58-84 Model::load_model. On error returns NULL and writes a message. */
or_model* or_load_model(const char* path, int* status, char* err, size_t errlen);
void or_free_model(or_model* m);
void or_get_config(const or_model* m, or_config* out);
/* number of tensors in the header and the name/offsets of tensor i (for the byte formula) */
size_t or_num_tensors(const or_model* m);
int or_tensor_info(const or_model* m, size_t i, const char** name, const char** dtype,
                   int64_t* off0, int64_t* off1);

/* cpu_inference.rs:50-55 KVCache::new */
or_kvcache* or_kv_new(const or_model* m);
/* The same cache, but every appended K/V element is rounded to bf16 (nearest, ties to even) and
 * attention reads the rounded values: the semantics of a bf16 KV cache, which the reference has
 * only as an experiment (README.md:23,90). */
or_kvcache* or_kv_new_bf16(const or_model* m);
/* f32 -> nearest bf16 (ties to even), widened back to f32; NaN stays a quiet NaN */
float or_round_bf16(float f);
void or_kv_free(or_kvcache* c);
size_t or_kv_len(const or_kvcache* c);

/* cpu_inference.rs:98-179 Model::forward. logits_out has vocab_size floats. */
int or_forward(const or_model* m, uint32_t token, size_t pos, or_kvcache* c, float* logits_out);

/* main.rs:37-42 argmax: first maximum wins (strict >), starting from index 0 */
uint32_t or_argmax(const float* x, size_t n);

/* bench.rs:106-116 / tests/mbu.rs:19-30 and bench.rs:118-119 */
uint64_t or_weight_bytes_per_token(const or_model* m);
uint64_t or_kv_bytes_at(const or_config* c, uint64_t pos);

/* threads used by or_matvec (cpu_inference.rs:231 available_parallelism); 0 = detect */
void or_set_threads(int n);
int or_get_threads(void);

/* primitives, exposed for unit tests (cpu_inference.rs:182-257) */
float or_bf16_to_f32(uint16_t x);
float or_dot(const float* a, const float* b, size_t n);
float or_dot_bf16(const uint16_t* w, const float* x, size_t n);
float or_silu(float x);
void or_rmsnorm(float* out, const float* x, const uint16_t* w, size_t n, float eps);
void or_rmsnorm_inplace(float* x, const uint16_t* w, size_t n, float eps);
void or_rope(float* x, size_t n, size_t pos, float theta);
void or_softmax(float* x, size_t n);
void or_matvec(float* out, const uint16_t* w, const float* x, size_t rows, size_t cols);

/* metal_inference.rs:140-154 rope_table: [max_seq][head_dim/2] of (cos, sin) */
void or_rope_table(float* out, size_t max_seq, size_t head_dim, float theta);

/*
 * The attention loop of cpu_inference.rs:144-162 for one token, on its own: q is
 * [n_heads*head_dim] (after q-norm and RoPE), k/v are the cache of one layer laid out
 * [n_pos][n_kv_heads*head_dim] (position-major, as KVCache stores it), out is
 * [n_heads*head_dim]. Attends positions 0..n_pos-1.
 */
void or_attention(const float* q, const float* k, const float* v, size_t n_pos, size_t n_heads,
                  size_t n_kv_heads, size_t head_dim, float* out);

#ifdef __cplusplus
}
#endif
#endif
