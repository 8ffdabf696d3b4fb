// Launch wrappers of the multi-token (chunked prefill / verify) kernels, gfx950 bf16 MFMA.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace qe {

// kGemmPartial: split over K; split z writes its partial sums to C + z M ldc (launch_gemm_split)
// kGemmQkRope (launch_gemm_qk_rope): the q|k|v projection of a chunk with the per-head q/k
// RMSNorm, RoPE and the K/V append of k_qk_rope in its epilogue
enum GemmEpilogue { kGemmStore = 0, kGemmResAdd = 1, kGemmSiluPair = 2, kGemmPartial = 3, kGemmQkRope = 4 };

// most key runs the causal attention of a chunk is split into (partials merged after)
constexpr int kBatchMaxRuns = 32;

// C[m][n] (=, +=) sum_k A'[m][k] W[n][k] for m < M, n < N; A' = A, or A x rowscale[m] x gain[k]
// (an RMSNorm) when the launch asks for the norm. kGemmSiluPair: W rows 2i / 2i+1 are gate_i /
// up_i and C[m][i] = silu(gate) * up. N even, K % 32 == 0, lda % 4 == 0.
// Up to kGemmSkinnyMaxM rows run on the skinny kernel, which computes the norm's row scales
// itself (rowscale unused, eps used); more rows need rowscale filled by launch_rownorm.
struct GemmParams {
  const float* A;
  uint32_t lda;
  const float* rowscale;  // [M]
  const uint16_t* gain;   // bf16 [K]
  const uint16_t* W;      // bf16 [N][K]
  uint32_t M, N, K;
  float* C;
  uint32_t ldc;
  float eps;
};

constexpr uint32_t kGemmSkinnyMaxM = 32;
// Between kGemmSkinnyMaxM and kGemmTileMinM rows, 64 x 64 tiles (k_gemm_lds). Above, up to
// kGemmRowsMaxM rows (K a multiple of 64), the 64-row eight-wave kernel (k_gemm_rows8), then
// 128-row tiles (k_gemm_tile): the faster at each size measured (128, 256, 512, 1024, 2048 rows).
constexpr uint32_t kGemmTileMinM = 64;
constexpr uint32_t kGemmRowsMaxM = 1024;

// Verify passes and chunks of up to kMvRowsMaxM tokens run the projections as a matvec over their
// token rows: out[m][.] for m < M from x [M][cols] (see launch_mv_rows). Each further row adds its
// own products and lane reductions to every wave of that matvec, so past 4 rows the skinny GEMM
// on the matrix cores is faster (measured at 5, 8 and 9 rows).
constexpr uint32_t kMvRowsMaxM = 4;
struct MvRowsParams {
  const uint16_t* w;     // bf16 [rows][cols], row-major
  const float* x;        // [M][cols]
  const uint16_t* gain;  // bf16 [cols]: the RMSNorm gain (norm launches only)
  float* out;            // [M][ldo]
  uint32_t M, rows, cols, ldo;
  float eps;
  // launch_mv_rows_merge only: x is the attention output merged from the split kernel's
  // partials [n_kv][attn_splits][rows per KV head][kPartStride] (launch_attention_rows layout:
  // row j of KV head g is token j / tok_heads, q head g tok_heads + j % tok_heads)
  const float* attn_part = nullptr;
  uint32_t attn_splits = 0, tok_heads = 0;
  // launch_lm_head_rows only (null: none): each workgroup's greedy candidate of each token row,
  // cand[v * workgroups + workgroup] (the decode step's kLogits rule)
  ArgCand* cand = nullptr;
};

// Weights of the next GEMM that a short launch loads into the L2 of the XCDs that will read them
// (8 x slots extra workgroups; slots = 0: none)
struct TilePrefetch {
  L2Prefetch pf[kMaxPrefetch];
  uint32_t slots;
};

struct BatchAttnParams {
  const float* qkv;        // [M][n_heads + 2 n_kv][128] raw projections
  float* q;                // [M][n_heads][128] normalized + rotated q
  float* att;              // [M][n_heads][128] attention output
  float* part;             // [M][n_heads][runs][kPartStride] partials (several key runs)
  const uint16_t* q_norm;  // bf16 [128]
  const uint16_t* k_norm;
  const float* rope;       // [max_seq][64](cos, sin)
  void* k_cache;           // layer base [n_kv][max_seq][128]
  void* v_cache;
  uint32_t M, start, max_seq, n_heads, n_kv;
  uint32_t key_run;        // positions per key run (set by launch_attn_causal)
  float eps, scale;
  int kv_bf16;
  uint32_t runs;           // key runs (set by launch_attn_causal)
  TilePrefetch pf;         // launch_attn_causal: weights its launch also loads into L2
};

hipError_t launch_rownorm(const float* x, uint32_t M, uint32_t K, float eps, float* s, hipStream_t st);
// The L2 prefetch of W [N][K] for the unsplit skinny GEMM (M <= 16): workgroup j reads rows
// 16 j .. 16 j + 15.
L2Prefetch skinny_prefetch_target(const uint16_t* W, uint32_t N, uint32_t K);
hipError_t launch_gemm(const GemmParams& p, bool norm, int epi, hipStream_t st);
// K splits for a split GEMM: enough workgroups to fill the chip, each split a multiple of the
// kernel's k step deep (1 when K does not split)
uint32_t gemm_splits(uint32_t M, uint32_t N, uint32_t K);
// partial sums of `splits` K ranges (no norm): C[z][m][n], z < splits, ldc = N
hipError_t launch_gemm_split(const GemmParams& p, uint32_t splits, hipStream_t st);
// The prefetch target of the weights of launch_gemm / launch_gemm_qk_rope (epi) or
// launch_gemm_split (kGemmPartial) at M rows on the 64-row kernel: column tile j, every row tile
// and K split of which runs on XCD j % 8, reads W rows [bn j, bn (j + 1)). w = nullptr where
// another kernel serves the shape or a column tile's workgroups do not stay on one XCD.
L2Prefetch gemm_prefetch_target(const uint16_t* W, uint32_t M, uint32_t N, uint32_t K, int epi);
// the slots that cover these targets (at most 64)
uint32_t tile_prefetch_slots(const L2Prefetch* pf, int n);
// x[m][n] += sum_z part[z][m][n] (z in order), then s[m] = 1 / sqrt(mean_n x[m][n]^2 + eps):
// the residual add of a split GEMM fused with the next RMSNorm's row scale. N % 4 == 0.
hipError_t launch_resadd_partials(float* x, const float* part, uint32_t splits, uint32_t M, uint32_t N, float eps,
                                  float* s, hipStream_t st);
// out[m][r] (=, +=) sum_c W[r][c] x'[m][c] for m < M (kGemmStore / kGemmResAdd), or
// out[m][i] = silu(gate_i) * up_i over the interleaved gate/up rows (kGemmSiluPair, ldo >= rows/2);
// x' = x, or RMSNorm(x_m) * gain with `norm`. f32 FMA on bf16 weights, as the decode matvec.
// cols % 8 == 0, cols <= 4096, 1 <= M <= kMvRowsMaxM; out must not alias x.
hipError_t launch_mv_rows(const MvRowsParams& p, bool norm, int epi, hipStream_t st);
// final RMSNorm (gain) + lm_head of M <= kMvRowsMaxM token rows: out[m][row], each row's logits
// equal to the decode step's lm_head's for that hidden state (its layout and summation order).
// hipErrorNotSupported past 1024 columns.
hipError_t launch_lm_head_rows(const MvRowsParams& p, hipStream_t st);
// o_proj + residual of a short pass with the attention merge in its prologue (as the decode step
// does): x[m][h*128 + d] = sum_s e_s acc_s / sum_s e_s l_s over the attn_splits partials of
// token m, q head h (every workgroup merges its chunks of every row). hipErrorNotSupported
// unless mv_rows_merge_fits(M, splits) and cols is whole heads of 128 with cols / 8 <= 256.
hipError_t launch_mv_rows_merge(const MvRowsParams& p, hipStream_t st);
// the merge slots a thread loads per token row (4, 8 or 16 for up to 4, 8, 16 runs) times the
// token rows stay within 16
bool mv_rows_merge_fits(uint32_t M, uint32_t splits);
hipError_t launch_qk_rope(const BatchAttnParams& p, hipStream_t st);
// The q|k|v GEMM of a chunk (A = x with the input RMSNorm, W = [q | k | v] rows, N = (n_heads +
// 2 n_kv) 128) with k_qk_rope's work in its epilogue: q rows normalized and rotated to a.q, k and
// v rows (k normalized and rotated) appended to the cache at positions a.start + m. Returns
// hipErrorNotSupported where the 64-row kernel does not serve the shape (the caller then runs
// launch_gemm and launch_qk_rope).
hipError_t launch_gemm_qk_rope(const GemmParams& g, const BatchAttnParams& a, hipStream_t st);
// causal attention of a chunk over `runs` (1..kBatchMaxRuns) key runs, merged into att; p.pf:
// weights the launch also loads into L2 (whole planes of workgroups after the runs')
hipError_t launch_attn_causal(const BatchAttnParams& p, uint32_t runs, hipStream_t st);
// key runs for a chunk of M tokens at positions start.. : at least 4, more while the chunk has
// under 512 workgroups, and at most one per 128 keys
uint32_t attn_causal_runs(uint32_t M, uint32_t start, uint32_t n_heads, uint32_t n_kv);
// tokens[r] = greedy token of row r of logits [rows][V] (the decode step's argmax rule);
// cand: rows * kArgParts candidates of scratch (device memory); rows <= 65535; err_in / err_out
// (optional): the device error word, copied to err_out once the tokens are written
constexpr uint32_t kArgParts = 64;
// tokens[r] = the greedy token of row r from its n_cand candidates cand[r n_cand ..] (written by
// launch_lm_head_rows) and the first logit of the row (logits [rows][V]); err as launch_row_argmax
hipError_t launch_cand_argmax(const ArgCand* cand, uint32_t n_cand, const float* logits, uint32_t rows, uint32_t V,
                              uint32_t* tokens, hipStream_t st, const uint32_t* err_in, uint32_t* err_out);
// workgroups of launch_lm_head_rows for `rows` logit rows (its candidates per token row)
uint32_t lm_head_rows_workgroups(uint32_t rows);
hipError_t launch_row_argmax(const float* logits, uint32_t rows, uint32_t V, uint32_t* tokens, ArgCand* cand,
                             hipStream_t st, const uint32_t* err_in = nullptr, uint32_t* err_out = nullptr);
hipError_t launch_embed_rows(const uint16_t* table, const uint32_t* ids, uint32_t M, uint32_t H, float* x,
                             hipStream_t st);
// The ids of a short pass (M <= kIdsByValue) as a kernel argument: no host-to-device copy.
constexpr uint32_t kIdsByValue = 64;
struct TokenIds {
  uint32_t id[kIdsByValue];
};
hipError_t launch_embed_rows(const uint16_t* table, const TokenIds& ids, uint32_t M, uint32_t H, float* x,
                             hipStream_t st);

}  // namespace qe
