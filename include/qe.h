/*
 * qe.h -- C ABI of the MI355X-native Qwen3 batch-1 decode engine (libqe.so).
 *
 * The engine API of the reference's Rust crate, flattened to plain C so that a Rust `-sys`
 * crate (or ctypes, or C++) can bind it without any GPU types in the signatures. Every entry
 * point returns an int status (QE_OK == 0) and never aborts; qe_last_error() gives the message
 * of the last failure on the calling thread. A model handle and the caches made from it are
 * single-threaded: calls on one model must not overlap (the reference's MetalModel shares its
 * scratch buffers the same way, metal_inference.rs:85-98).
 *
 * Reference interfaces replaced (paths relative to the reference root):
 *   metal_infrence_engine/src/cpu_inference.rs, metal_infrence_engine/src/metal_inference.rs,
 *   metal_infrence_engine/src/bin/bench.rs, metal_infrence_engine/tests/read_bandwidth.rs.
 */
#ifndef QE_H
#define QE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define QE_OK 0
#define QE_ERR_IO 1          /* file missing or unreadable (io::Error in the reference) */
#define QE_ERR_FORMAT 2      /* bad safetensors header / config.json / alignment */
#define QE_ERR_TENSOR 3      /* missing tensor, non-BF16 dtype, or shape mismatch */
#define QE_ERR_POS 4         /* pos >= max_seq, or pos beyond the cached length */
#define QE_ERR_ARG 5         /* invalid argument (null pointer, token >= vocab, ...) */
#define QE_ERR_UNSUPPORTED 6 /* a shape the kernels do not handle (head_dim != 128, ...) */
#define QE_ERR_HIP 7         /* a HIP runtime call failed */
#define QE_ERR_NO_DEVICE 8   /* no usable gfx950 device */
#define QE_ERR_KERNEL 9      /* a kernel reported a failure through its error word */

/* KV cache element types */
#define QE_KV_F32 0
#define QE_KV_BF16 1

/* Subset of config.json the forward pass reads. Replaces `Config`, cpu_inference.rs:20-33. */
typedef struct qe_config {
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
} qe_config;

typedef struct qe_model qe_model;
typedef struct qe_kv qe_kv;

/* Called once per finished decode step with that step's greedy token, in order. */
typedef void (*qe_on_token)(void* user, uint32_t token);

/* Message of the last failed call on this thread ("" if none). Valid until the next call. */
const char* qe_last_error(void);

/* ---- model: MetalModel::load_model (metal_inference.rs:157-168), which reads the file with
 *      Model::load_model (cpu_inference.rs:58-84) and the sibling config.json. Weights are
 *      copied once into a device arena on the current HIP device. ---- */
int qe_model_load(const char* safetensors_path, qe_model** out);
void qe_model_free(qe_model* model);
/* MetalModel::config (metal_inference.rs:170) */
int qe_model_config(const qe_model* model, qe_config* out);
/* The HIP stream (hipStream_t) every call on this model is ordered on, so a caller can time
 * it with its own events. No reference counterpart: the Metal engine keeps its queue private. */
void* qe_model_stream(const qe_model* model);
/* bench.rs:106-116 (tests/mbu.rs:19-30): every tensor's bytes except the embedding table,
 * plus one embedding row */
uint64_t qe_weight_bytes_per_token(const qe_model* model);
/* bench.rs:118-119: K and V bytes read at position pos (f32 as in the reference; bf16 halves) */
uint64_t qe_kv_bytes_at(const qe_model* model, uint64_t pos, int kv_dtype);
/* How this model's decode step runs its layers: 2 = all of them in one persistent launch, 1 = two
 * launches per layer (attention block, MLP block), 0 = one launch per stage. 1 and 2 serve one KV
 * head per XCD and need the Qwen3-0.6B shape on a device that deals a launch's workgroups to its
 * XCDs round-robin; QE_FUSED=0, 1 or 2 at model load caps the choice. No reference counterpart:
 * the Metal engine encodes one dispatch per stage (metal_inference.rs:318-387). */
int qe_model_fused_layers(const qe_model* model);

/* ---- KV cache: MetalKVCache::new (metal_inference.rs:129-137). One cache per sequence,
 *      tied to the model it was made from; holds the RoPE table for max_seq positions. ---- */
int qe_kv_new(qe_model* model, uint64_t max_seq, int kv_dtype, qe_kv** out);
void qe_kv_free(qe_kv* kv);
uint64_t qe_kv_max_seq(const qe_kv* kv);
/* positions cached so far (the next forward must use pos <= this) */
uint64_t qe_kv_len(const qe_kv* kv);

/* ---- one token: MetalModel::forward (metal_inference.rs:284-291) == Model::forward
 *      (cpu_inference.rs:98-179). Runs `token` at `pos`, writes its K/V into the cache and
 *      returns the vocab_size logits in logits_out (host memory). Requires pos < max_seq and
 *      pos <= qe_kv_len(kv); afterwards qe_kv_len(kv) == pos + 1. ---- */
int qe_forward(qe_model* model, uint32_t token, uint64_t pos, qe_kv* kv, float* logits_out);

/* ---- prefill: the prompt loop of bench.rs:174-176 (one forward per token). Writes the last
 *      position's logits to last_logits (nullable). n = 0 does nothing: last_logits and the
 *      cache are left as they were. ---- */
int qe_prefill(qe_model* model, const uint32_t* ids, uint64_t n, uint64_t start_pos, qe_kv* kv,
               float* last_logits);

/* ---- greedy decode: MetalModel::decode (metal_inference.rs:293-316). `first` goes in at
 *      start_pos; each step's GPU argmax (lowest index on ties, main.rs:37-42) feeds the next
 *      step on the device. on_token (nullable) is called with each step's token as the step
 *      finishes. If logits_per_step is not NULL it receives steps*vocab_size floats (slower:
 *      one device-to-host copy per step; meant for parity tests). steps = 0 does nothing. ---- */
int qe_decode(qe_model* model, uint32_t first, uint64_t start_pos, uint64_t steps, qe_kv* kv,
              qe_on_token on_token, void* user, float* logits_per_step);

/* ---- multi-token forward on the matrix cores (no reference counterpart: the reference's
 *      prompt loop calls forward once per token, bench.rs:174-176) ---- */
/* Chunked prefill: runs ids[0..n) at positions start_pos.. through the model in chunks of up to
 * `chunk` tokens (0 = 512, at most 2048): one bf16 MFMA GEMM per projection and chunk, f32
 * activations split into two bf16 halves (about 16 mantissa bits), causal attention over the
 * cache and the chunk. Appends the K/V of every position and writes the last token's logits
 * (nullable). Same position contract as qe_prefill; logits agree with it within 1e-2, not bit for
 * bit. The model's chunk buffers are allocated on first use. Consecutive chunks of more than 32
 * tokens run on two streams (the model's and one it creates on first use, with a second set of
 * chunk buffers), each chunk's attention ordered after the earlier chunks' K/V rows of the same
 * layer; the call returns once every stream is done. n = 0 does nothing. */
int qe_prefill_batch(qe_model* model, const uint32_t* ids, uint64_t n, uint64_t start_pos, qe_kv* kv,
                     uint32_t chunk, float* last_logits);
/* Verify k (1..64) tokens at positions start_pos.. in one pass (the k-token check of speculative
 * decoding): appends their K/V and writes all k logit rows, logits_out [k][vocab_size]. */
int qe_verify(qe_model* model, const uint32_t* ids, uint64_t k, uint64_t start_pos, qe_kv* kv,
              float* logits_out);
/* qe_verify with each row's greedy token taken on the device (the decode step's argmax rule):
 * tokens_out[i] = the token after ids[i]. */
int qe_verify_greedy(qe_model* model, const uint32_t* ids, uint64_t k, uint64_t start_pos, qe_kv* kv,
                     uint32_t* tokens_out);

/* ---- speculative greedy decode by prompt lookup (no reference counterpart: README.md:109-111
 *      names it as the next step). Same contract and same greedy tokens as qe_decode(first,
 *      start_pos, steps): each pass drafts up to k_max tokens that followed an earlier
 *      occurrence of the history's last g tokens (g = ngram .. 1; history = context[0..n_context)
 *      + first + the tokens emitted so far; the most recent occurrence with k_max followers, else
 *      the earliest) and checks them with one verify pass; drafts are
 *      accepted while they equal the greedy token of the row before, and that pass adds one
 *      greedy token of its own. With no draft a pass is one decode step. on_token gets every
 *      token in order. k_max 1..63, ngram >= 1. ---- */
typedef struct {
  uint64_t passes;        /* verify passes */
  uint64_t drafted;       /* draft tokens checked */
  uint64_t accepted;      /* draft tokens accepted */
  uint64_t single_steps;  /* decode steps taken when no draft was found */
  uint64_t plain_steps;   /* decode steps taken in plain blocks while drafting did not pay */
} qe_lookup_stats;
/* Adaptive (on unless QE_LOOKUP_ADAPTIVE=0 when the model was loaded): the host times the passes
 * as they run; once they average under 2 tokens each it also times one block of 16 pipelined
 * decode steps, and while the passes emit fewer tokens per second than those steps, it decodes
 * plain blocks of 16 steps with one pass after each (plain_steps). The tokens do not change. */
int qe_decode_lookup(qe_model* model, const uint32_t* context, uint64_t n_context, uint32_t first, uint64_t start_pos,
                     uint64_t steps, qe_kv* kv, uint32_t k_max, uint32_t ngram, qe_on_token on_token, void* user,
                     qe_lookup_stats* stats);
/* A draft source: writes up to k_max tokens that are to follow history[0..n) (context, first and
 * the tokens emitted so far) to draft_out and returns their count (0: no draft), or
 * QE_DRAFT_ERROR when it fails: the decode then stops before another pass and returns QE_ERR_ARG,
 * with the tokens emitted so far delivered and the cache valid up to the next position. */
#define QE_DRAFT_ERROR 0xFFFFFFFFu
typedef uint32_t (*qe_draft_fn)(void* user, const uint32_t* history, uint64_t n, uint32_t k_max, uint32_t* draft_out);
/* qe_decode_lookup with the drafts of `draft` (a draft model, another lookup rule, ...) instead
 * of prompt lookup, and the adaptive rule on when adaptive != 0. No reference counterpart. */
int qe_decode_drafted(qe_model* model, const uint32_t* context, uint64_t n_context, uint32_t first, uint64_t start_pos,
                      uint64_t steps, qe_kv* kv, uint32_t k_max, qe_draft_fn draft, void* draft_user, int adaptive,
                      qe_on_token on_token, void* user, qe_lookup_stats* stats);
/* The draft rule alone (host code, no device): writes the draft qe_decode_lookup would check
 * after history[0..n) (at most k_max tokens) to draft_out and returns its length. */
uint64_t qe_lookup_draft(const uint32_t* history, uint64_t n, uint32_t ngram, uint32_t k_max, uint32_t* draft_out);

/* ---- per-stage kernel timing: runs `token` at `pos` like qe_forward, then times each stage
 *      of the step (qkv, attention, o_proj, gate_up, down, lm_head, argmax) as a graph of that
 *      stage's launches only (28 per-layer launches, or one; past 1024 positions o_proj is 56:
 *      the attention merge and o_proj), replayed 8 times between two HIP
 *      events, each stage from the step state of `pos`. Writes, per stage, the mean duration of
 *      one launch in microseconds to us_out, the launches per decode step to launches_out
 *      (nullable) and the stage name (a static string) to names_out (nullable); *n_out = stages
 *      written. The stage "qkv+attention" times each layer's q|k|v and attention launches together
 *      (2 per layer), so that the attention's time behind its producer is that minus the "qkv"
 *      stage's; the stages "qkv+attention+o_proj", ... up to
 *      "qkv+attention+o_proj+gate_up+down+lm_head" time the step's prefixes the same way, so that
 *      differences of consecutive prefixes (duration x launches) are the stages' costs inside the
 *      step (the argmax, the last launch, is timed alone only: its replays advance the step
 *      state). A cache of fewer than 9 positions skips the argmax stage (its replays advance the
 *      token ring). With two launches per layer (qe_model_fused_layers() == 1) the stages are
 *      attn_block, mlp_block, final_reduce, lm_head and argmax, their prefixes and "step" (the
 *      whole step's graph); then "in_step:attn_block" and "in_step:mlp_block", each layer
 *      launch's share of the whole step (its first workgroup's start to the next layer launch's
 *      first start, from per-workgroup clock stamps of a compilation of the same kernels that
 *      writes them; launches_out counts the launches with a successor), and "in_exec:attn_block",
 *      "in_exec:mlp_block", first start to last workgroup exit. Afterwards the step is run once
 *      more, so the cache holds what qe_forward(token, pos) leaves; a kernel error raised by any
 *      replay is returned as QE_ERR_KERNEL. No reference counterpart: the reference timed kernels
 *      by removing them by hand (README.md:64-71). ---- */
int qe_profile_step(qe_model* model, uint32_t token, uint64_t pos, qe_kv* kv, float* us_out,
                    uint32_t* launches_out, const char** names_out, uint32_t max_stages, uint32_t* n_out);

/* ---- synthetic inputs (the reference loads a real checkpoint; this build writes a seeded
 *      random-init one with the same tensor names, shapes and file format) ---- */
/* Writes <dir>/model.safetensors and <dir>/config.json: every matrix bf16 ~ N(0, 0.02) from
 * `seed`, norm gains 1.0, lm_head.weight a byte copy of model.embed_tokens.weight. */
int qe_write_random_checkpoint(const char* dir, uint64_t seed, const qe_config* cfg);
/* n token ids uniform in [0, vocab) from `seed` */
void qe_random_prompt(uint64_t seed, uint64_t n, uint32_t vocab, uint32_t* out);

/* ---- isolated device ops on caller-owned device memory (HIP device pointers; stream may be
 *      NULL for the default stream). For the isolated benchmarks and kernel parity tests. ---- */
/* out[r] = sum_c bf16(w[r*cols + c]) * x[c], f32 accumulate; matvec_bf16,
 * inference.metal:143-186 / cpu_inference.rs:225-257. cols % 8 == 0, w 16-byte aligned. */
int qe_op_matvec_bf16(const void* w, const float* x, float* out, uint64_t rows, uint64_t cols,
                      void* stream);
/* c[i][j] = sum_k a[i][k] bf16(w[j][k]): the chunked prefill's GEMM (a f32 [m][k] split into two
 * bf16 halves, w bf16 [n][k], f32 accumulate on the matrix cores). n even, k % 32 == 0,
 * a and w 16-byte aligned. No reference counterpart (the reference has no batched path). */
int qe_op_gemm_bf16(const float* a, const void* w, float* c, uint64_t m, uint64_t n, uint64_t k,
                    void* stream);
/* One decode step of GQA attention (cpu_inference.rs:144-162, inference.metal:234-296) for
 * head_dim 128: q [n_heads*128] (post q-norm and RoPE), k/v caches laid out
 * [n_kv_heads][kv_stride][128] f32, attending positions 0..n_pos-1; out [n_heads*128].
 * The positions are split into n_splits runs (1..128; 0 picks runs of 64 positions), each
 * attended by one workgroup per KV head, and a second kernel merges the runs' partial softmax
 * sums. `work` (partials, overwritten by every call) must hold qe_op_attention_work_bytes(...)
 * bytes of device memory. */
uint64_t qe_op_attention_work_bytes(uint64_t n_heads, uint64_t n_kv_heads, uint64_t n_pos);
int qe_op_attention(const float* q, const float* k, const float* v, float* out, uint64_t n_pos,
                    uint64_t kv_stride, uint64_t n_heads, uint64_t n_kv_heads, uint32_t n_splits,
                    void* work, void* stream);
/* qe_op_attention with no work buffer and no allocation: the partial sums go to a 1 MiB array in
 * device memory that the library holds on each GPU it runs on until the process ends. No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops that forbid hipMalloc). Same arguments and results as
 * qe_op_attention; calls with n_heads x runs above 2048 (runs = n_splits, or n_pos / 64 rounded
 * up, at most 128) are refused with QE_ERR_ARG. Every call on one GPU shares that GPU's array, so
 * calls that overlap on one GPU (two streams or two threads) race. The first call on each device
 * looks up the array's device address (hipGetSymbolAddress, which may load the library's device
 * code): make it outside stream capture; later calls may be captured into a graph. */
int qe_op_attention_static(const float* q, const float* k, const float* v, float* out, uint64_t n_pos,
                           uint64_t kv_stride, uint64_t n_heads, uint64_t n_kv_heads, uint32_t n_splits,
                           void* stream);
/* Greedy token of each of `rows` logit rows of n floats (device memory, row-major): the argmax
 * of main.rs:37-42 -- the first maximum wins (lowest index on ties, -0.0 ties +0.0), NaN entries
 * never win, a NaN at index 0 gives 0, and a row with nothing above -inf gives 0. tokens_out:
 * `rows` uint32 in device memory. The verify pass's device argmax (qe_verify_greedy) runs this
 * kernel. */
int qe_op_argmax(const float* logits, uint64_t rows, uint64_t n, uint32_t* tokens_out, void* stream);
/* Streaming read of n floats (n % 4 == 0): the read_sum kernel of tests/read_bandwidth.rs:16-54,
 * writing one partial sum per block to partial[grid]. grid == 0 picks a default. */
int qe_op_read_sum(const float* src, uint64_t n, float* partial, uint32_t grid, void* stream);
/* The same sum with non-temporal loads (not allocated in the MALL), block b reading the contiguous
 * quarter-float4 range [n/4 b / grid, n/4 (b + 1) / grid): on gfx950 this streaming form reads
 * faster than the strided one, so the read ceiling is the better of the two. It replaces nothing
 * in the reference, whose read_bandwidth.rs kernel has one form (tests/read_bandwidth.rs:16-54). */
int qe_op_read_sum_nt(const float* src, uint64_t n, float* partial, uint32_t grid, void* stream);

#ifdef __cplusplus
}
#endif
#endif
