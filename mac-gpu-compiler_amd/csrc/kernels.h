// Device-side data structures and launch wrappers of the decode step (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qe {

constexpr int kHeadDim = 128;        // head dimension the attention kernels are written for
constexpr int kAttnMaxSplits = 128;  // most position runs per KV head (isolated attention op)

// Per-sequence device state, advanced by the last kernel of each step so a captured step can
// be replayed without host writes: step i reads tokens[tok_idx] at position pos and writes its
// greedy token to tokens[tok_idx + 1].
struct StepState {
  uint32_t pos;
  uint32_t tok_idx;
  uint32_t max_seq;
  uint32_t tok_cap;  // entries in the token ring
};

// Error bits a kernel sets in the model's error word instead of faulting.
enum : uint32_t {
  kErrPos = 1u,       // pos >= max_seq seen on the device
  kErrToken = 2u,     // input token >= vocab
  kErrRing = 4u,      // token ring full
  kErrShape = 8u,     // the decode step's attention runs do not cover pos (a host-side mistake)
  kErrSync = 16u,     // a fused layer's wait for the workgroups of its XCD ran out of spins
  kErrPlace = 32u,    // a fused layer's workgroup read an XCD id past the 8 XCDs
};

// Per-workgroup greedy candidate (value, index); NaN is never a candidate.
struct ArgCand {
  float v;
  uint32_t i;
};

// Weight chunks that a later kernel of the step reads, loaded ahead into the L2 of the XCD that
// will read them. Consumer workgroup j of launch_matvec_wide reads the 16-byte chunks
// [j * cw_chunks, (j + 1) * cw_chunks) of its matrix and runs on XCD j % 8 (workgroups are
// dispatched round-robin over the 8 XCDs).
struct L2Prefetch {
  const uint16_t* w;   // bf16 matrix
  uint32_t n_chunks;   // 16-byte chunks in the matrix
  uint32_t cw_chunks;  // chunks one consumer workgroup reads
  uint32_t n_cwg;      // consumer workgroups
};
constexpr int kMaxPrefetch = 2;

struct MatvecParams {
  const uint16_t* w;     // bf16 [rows][cols] row-major
  const float* x;        // [cols] input
  const uint16_t* nw;    // bf16 [cols] RMSNorm gain (prologues kNorm, kEmbedNorm)
  float eps;
  uint32_t rows, cols;
  float* out;            // [rows] (store / residual add), [rows/2] (silu pairs)
  ArgCand* cand;         // per-workgroup argmax candidates (epilogue kLogits)
  // prologue kEmbedNorm: x is row tokens[state->tok_idx] of the bf16 table `embed`
  const uint16_t* embed;
  const uint32_t* tokens;
  const StepState* state;
  uint32_t vocab;
  float* x_out;          // the embedding row is also written here (the residual stream)
  uint32_t* err;
  // prologue kAttnMerge: x[h*128 + d] is merged from attention split partials
  const float* attn_part;  // [n_kv][attn_splits][group][kPartStride]
  uint32_t attn_splits, attn_group;
};

enum Prologue { kCopy = 0, kNorm = 1, kEmbedNorm = 2, kAttnMerge = 3 };
enum Epilogue { kStore = 0, kResAdd = 1, kSiluPair = 2, kLogits = 3 };

struct AttnParams {
  const float* qkv;        // raw projections [n_heads*D | n_kv*D | n_kv*D]
  const uint16_t* q_norm;  // bf16 [D]
  const uint16_t* k_norm;  // bf16 [D]
  const float* rope;       // [max_seq][D/2][2] (cos, sin)
  const float* rope_cur;   // [D/2][2]: the rope row of state->pos (split kernel)
  void* k_cache;          // layer base, [n_kv][max_seq][D], f32 or bf16
  void* v_cache;
  float* partial;          // [n_kv][splits][group][kPartStride]
  const StepState* state;
  uint32_t* err;
  uint32_t n_heads, n_kv, max_seq;
  float eps, scale;
  int kv_bf16;
  uint32_t n_pos_fixed;    // isolated op: attend positions 0..n_pos_fixed-1 with a final q
  // rows of several tokens (launch_attention_rows): the G' = n_heads / n_kv rows of KV head g are
  // tok_heads q heads of each of G' / tok_heads consecutive tokens; row r is token r / tok_heads,
  // head g * tok_heads + r % tok_heads, its q at r / tok_heads * q_tok_stride + head * 128 (and
  // its output there too), and it sees positions up to n_pos_fixed - tokens + token (causal).
  // tok_heads = 0: one token (the rows are the G' heads of g)
  uint32_t tok_heads, q_tok_stride;
  // rows of several tokens: the G' rows of a KV head are served by row_split workgroups of
  // G' / row_split rows each (0 or 1: one workgroup), all reading the same K/V runs
  uint32_t row_split;
  uint32_t splits;         // runs per KV head (set by the launchers)
  uint32_t run;            // decode: positions per run (a multiple of 64) chosen by the host for
                           // the step's position; 0: derived from pos on the device
  // decode only: 8 * pf_slots extra workgroups load these matrices into L2 while the attention
  // runs (pf_slots = 0: none), at positions below pf_max_pos
  L2Prefetch pf[kMaxPrefetch];
  uint32_t pf_slots;
  uint32_t pf_max_pos;
};

// --- launch wrappers (kernels.hip) ---
hipError_t launch_matvec(const MatvecParams& p, int prologue, int epilogue, hipStream_t s);
uint32_t matvec_num_blocks(uint32_t rows, uint32_t cols, int epilogue);
// the per-layer projections: ~1000 workgroups, x read per chunk from global memory
hipError_t launch_matvec_wide(const MatvecParams& p, int prologue, int epilogue, hipStream_t s);
// Decode-step attention: grid (n_kv, splits); at each step the n = pos + 1 cached positions are
// cut into `splits` runs of a whole number of 64-position tiles, each workgroup writes its (m, l,
// acc) partials (runs past pos write empty ones), and the o_proj matvec merges them in its
// prologue (kAttnMerge, up to kAttnMaxMergeSplits runs). Long contexts use up to
// kAttnMaxWideSplits runs, merged by launch_attention_merge before a plain o_proj.
constexpr int kAttnMaxMergeSplits = 16;
constexpr int kAttnMaxWideSplits = 64;
// one split partial per q head: m, l, 2 pad floats, acc[128] (16-byte aligned rows)
constexpr int kPartStride = 4 + kHeadDim;
hipError_t launch_attention_split(const AttnParams& p, uint32_t splits, hipStream_t s);
// out [n_heads][128] = the merge of the `splits` partials per q head that launch_attention_split
// wrote to p.partial (splits <= kAttnMaxSplits)
hipError_t launch_attention_merge(const AttnParams& p, uint32_t splits, float* out, hipStream_t s);
// The L2 prefetch of a matrix that launch_matvec_wide(rows x cols, prologue, epilogue) will read.
L2Prefetch l2_prefetch_target(const uint16_t* w, uint32_t rows, uint32_t cols, int prologue, int epilogue);
// Prefetch workgroups per XCD for these targets (each loads at most 16 chunks per thread).
uint32_t l2_prefetch_slots(const L2Prefetch* pf, int n);
// The isolated op: final q [n_heads][D], complete K/V [n_kv][max_seq][D] (f32), positions
// 0..n_pos_fixed-1 in `splits` runs (<= kAttnMaxSplits), partials merged into out [n_heads][D].
hipError_t launch_attention_op(const AttnParams& p, uint32_t splits, float* out, hipStream_t s);
// Attention of T tokens at positions n_pos_fixed - T .. n_pos_fixed - 1 over positions
// 0..n_pos_fixed-1 of a cache that already holds their K/V (f32 or bf16), causal among them, with
// the same kernels: q [T][heads][128] final (normalized, rotated), out [T][heads][128]. The T
// tokens' q heads of a KV head share one read of its K/V: p.n_heads = n_kv * T * tok_heads must
// give 1, 2, 4 or 8 rows per KV head. partial: n_kv * splits * (rows per KV head) * kPartStride floats.
// out = nullptr: the partials only (a consumer merges them, launch_mv_rows_merge).
hipError_t launch_attention_rows(const AttnParams& p, uint32_t splits, float* out, hipStream_t s);
// Greedy token from the lm_head candidates; advances the step state and, with `rope`, copies the
// RoPE row of the next position ([half] (cos, sin) pairs) to rope_cur for the next step.
hipError_t launch_argmax(const ArgCand* cand, uint32_t n_cand, const float* logits, StepState* st,
                         uint32_t* tokens, uint32_t* host_tokens, uint32_t* err, const float* rope,
                         float* rope_cur, uint32_t half, hipStream_t s);
// nt: the non-temporal form, one contiguous range of the buffer per workgroup
hipError_t launch_read_sum(const float* src, uint64_t n, float* partial, uint32_t grid, bool nt, hipStream_t s);

// ---- fused decode layer (fused.hip): two launches per layer for the Qwen3-0.6B shape ----
// One KV head per XCD: the 256 workgroups of a launch are 8 XCDs x 32 slots (workgroup i runs
// on XCD (start + i) % 8, the start varying from launch to launch; a workgroup reads its XCD from
// HW_REG_XCC_ID and takes slot i / 8). The stages of a launch hand data to each other only inside
// one XCD, through its L2, as (value, tag) pairs; what crosses XCDs (the o_proj and down outputs,
// split over the XCDs' column slices) goes to the next launch as 8 partial vectors that it adds
// to the residual stream.
constexpr uint32_t kFusedXcds = 8;
constexpr uint32_t kFusedSlots = 32;     // workgroups per XCD
constexpr uint32_t kFusedMaxRuns = 32;   // attention runs per KV head (one per slot)
constexpr uint32_t kFusedH = 1024, kFusedI = 3072, kFusedHeads = 16, kFusedKv = 8;
// generation words: one per XCD, each on its own 128-byte line
constexpr uint32_t kFusedLineWords = 32;
constexpr size_t kFusedSyncWords = size_t(kFusedXcds) * kFusedLineWords;
// exchange buffers, in (value, tag) pairs
constexpr size_t kFusedQkvPairs = size_t(kFusedHeads + 2 * kFusedKv) * kHeadDim;
// ... followed by the merged attention output of each XCD ([8][G * 128] pairs) of a 32-run step
constexpr size_t kFusedAttPairs = size_t(kFusedHeads) * kHeadDim;
constexpr size_t kFusedPartPairs = size_t(kFusedKv) * kFusedMaxRuns * (kFusedHeads / kFusedKv) * kPartStride;
constexpr size_t kFusedHPairs = kFusedI;
// token rows of a fused launch: 1 (decode step) or 2 (verify pass); every exchange buffer, the
// residual and the partials hold kFusedMaxRows rows, row r at r times the one-row size
constexpr uint32_t kFusedMaxRows = 2;
constexpr size_t kFusedQkvRowPairs = kFusedQkvPairs + kFusedAttPairs;

// A region of weights that extra workgroups of a launch load into the L2 of each XCD for a later
// launch: on XCD x the rows [0, rows) of row_bytes bytes at base + x * xcd_bytes + r * stride.
struct FusedPrefetch {
  const uint8_t* base;
  uint32_t xcd_bytes, row_bytes, stride, rows;
};
constexpr int kFusedMaxPrefetch = 4;

struct FusedLayerParams {
  // attention block
  const uint16_t* w_in;     // input_layernorm gain [H]
  const uint16_t* w_qkv;    // q_proj | k_proj | v_proj rows [QD + 2 KD][H]
  const uint16_t* q_norm;   // [D]
  const uint16_t* k_norm;   // [D]
  const uint16_t* w_o;      // [H][QD]
  // MLP block
  const uint16_t* w_post;   // post_attention_layernorm gain [H]
  const uint16_t* w_gu;     // gate/up rows interleaved [2I][H]
  const uint16_t* w_down;   // [H][I]
  // residual stream: x = res_in + sum_x part_in[x] (layer 0 of the attention block: x = the
  // embedding row of the step's token)
  const float* res_in;
  const float* part_in;     // [8][H]
  float* res_out;           // x, written by workgroup 0 for the next launch
  float* part_out;          // [8][H]: this launch's o_proj (or down) output, one slice per XCD
  // exchanged inside one XCD during a launch, as (value bits, tag) pairs
  uint2* qkv;               // [kFusedQkvPairs] raw projections, then [kFusedAttPairs] merged heads
  uint2* attn_part;         // [kFusedPartPairs]: [8][kFusedMaxRuns][G][kPartStride]
  uint2* h;                 // [kFusedHPairs] silu(gate) * up
  const uint16_t* embed;
  const uint32_t* tokens;
  uint32_t vocab;
  const StepState* state;
  void* k_cache;            // layer base [8][max_seq][D], f32 or bf16
  void* v_cache;
  int kv_bf16;
  uint32_t max_seq;
  const float* rope_cur;    // [D/2][2]
  uint32_t splits, run;     // attention runs per KV head (<= 32) and positions per run
  float eps, scale;
  uint32_t* sync;           // kFusedSyncWords generation words, zeroed once
  uint32_t* err;
  // pf_wgs extra workgroups per XCD load the pf regions into its L2 (at positions below
  // pf_max_pos; pf_wgs = 0: none)
  FusedPrefetch pf[kFusedMaxPrefetch];
  uint32_t pf_wgs, pf_max_pos;
  // the attention block's slots without a run or o_proj rows load the pf regions once their
  // q|k|v rows are out
  int pf_idle;
  // the workgroups of the runs load pf region 1 once their partials are out
  int pf_run;
  // MLP block: the next layer's q|k|v rows [QD + 2 KD][H] (null: none); workgroup (x, s) loads
  // the rows that slot s of the next attention block reads into XCD x's L2
  const uint16_t* qkv_next;
  // clock stamps, read by the *_timed launchers only (null: none): layer workgroup b stores the
  // 100 MHz real-time clock at its start to ts[2 b] and at its exit to ts[2 b + 1]
  uint64_t* ts;
  // token rows (1 or kFusedMaxRows) at positions state->pos .. + rows - 1: tokens[state->tok_idx + r]
  // in layer 0; rows > 1 (up to 16 single-tile runs): rope_cur is the RoPE table [max_seq][D]
  // and row r takes row pos + r
  uint32_t rows;
};

// layer l's attention block: [embedding | residual + partials] -> RMSNorm -> q|k|v ->
// q/k RMSNorm + RoPE + K/V append + attention (split runs) -> merge -> o_proj slice partial
hipError_t launch_fused_attn(const FusedLayerParams& p, bool first_layer, hipStream_t s);
// layer l's MLP block: residual + partials -> RMSNorm -> gate|up + silu -> down slice partial
hipError_t launch_fused_mlp(const FusedLayerParams& p, hipStream_t s);
// the same two blocks compiled with the clock stamps of FusedLayerParams::ts (fused_timed.hip),
// for timing the layer launches inside a whole step
hipError_t launch_fused_attn_timed(const FusedLayerParams& p, bool first_layer, hipStream_t s);
hipError_t launch_fused_mlp_timed(const FusedLayerParams& p, hipStream_t s);
// x = res + sum of the 8 partials (the last layer's output, before the final norm)
// gain: x = the final RMSNorm of each row's sum, with that gain and eps
hipError_t launch_fused_reduce(const float* res, const float* part, float* x, uint32_t rows, const uint16_t* gain,
                               float eps, hipStream_t s);
// ---- the decode step's layers in one persistent launch (persist.hip), same shape ----
struct PersistParams {
  // layer 0's tensors; layer l's are layer_stride bytes further on
  const uint16_t *w_in, *w_qkv, *q_norm, *k_norm, *w_o, *w_post, *w_gu, *w_down;
  uint64_t layer_stride;
  uint32_t n_layers;       // at most 32
  const uint16_t* embed;
  const uint32_t* tokens;
  uint32_t vocab;
  const StepState* state;
  void* k_cache;           // layer 0's [8][max_seq][D], f32 or bf16; layer l at + l * layer_kv elements
  void* v_cache;
  uint64_t layer_kv;
  int kv_bf16;
  uint32_t max_seq;
  const float* rope_cur;   // [D/2][2]
  uint32_t splits, run;    // attention runs per KV head (4, 8, 16 of 64 positions, or 32) and their length
  float eps, scale;
  float* x_out;            // [H] the last layer's output (the residual stream before the final norm)
  // (value, tag) pairs: inside an XCD
  uint2* qkv;              // [kFusedQkvPairs]
  uint2* attn_part;        // [kFusedPartPairs]
  uint2* h;                // [kFusedHPairs]
  uint2* xa;               // [8][H] each XCD's gathered residual stream after the attention
  uint2* xm;               // [8][H] ... after the MLP
  // across XCDs
  uint2* part_a;           // [8][H] o_proj partials
  uint2* part_m;           // [8][H] down partials
  uint32_t* gen;           // one word, zeroed once
  uint32_t* err;
};
hipError_t launch_decode_persist(const PersistParams& p, hipStream_t s);

// Runs a 256-workgroup kernel whose workgroup i writes the XCD it runs on to dev_ids[i] (256
// words), copies them to host_ids (pinned, 256 words); *ok = the workgroups were dealt to the 8
// XCDs round-robin (workgroup i on XCD (start + i) % 8 for some start).
hipError_t fused_placement_check(uint32_t* dev_ids, uint32_t* host_ids, bool* ok, hipStream_t s);

}  // namespace qe
