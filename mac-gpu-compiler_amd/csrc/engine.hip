// Host engine behind the C ABI of include/qe.h: device weight arena, per-sequence KV cache with
// its RoPE table and step state, one decode step captured as a hipGraph per cache and replayed.
//
// Reference: metal_infrence_engine/src/metal_inference.rs (MetalModel, MetalKVCache, forward,
// decode, commit_step) and cpu_inference.rs (the loader contract and the byte formula).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/qe.h"
#include "batch.h"
#include "checkpoint.h"
#include "kernels.h"
#include "status.h"

using qe::ArgCand;
using qe::AttnParams;
using qe::FusedLayerParams;
using qe::MatvecParams;
using qe::StepState;

namespace {

thread_local std::string g_err;

int vfail(int code, const char* fmt, va_list ap) {
  char buf[1024];
  vsnprintf(buf, sizeof(buf), fmt, ap);
  g_err = buf;
  return code;
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vfail(code, fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace

namespace qe {
int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vfail(code, fmt, ap);
  va_end(ap);
  return code;
}
}  // namespace qe

namespace {

#define HIP_TRY(expr)                                                                       \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess) return fail(QE_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

struct Layer {
  const uint16_t* w_in;    // input_layernorm [H]
  const uint16_t* w_qkv;   // q_proj | k_proj | v_proj rows, [QD + 2 KD][H]
  const uint16_t* q_norm;  // [D]
  const uint16_t* k_norm;  // [D]
  const uint16_t* w_o;     // [H][QD]
  const uint16_t* w_post;  // post_attention_layernorm [H]
  const uint16_t* w_gu;    // gate/up rows interleaved: row 2i = gate_i, row 2i+1 = up_i, [2I][H]
  const uint16_t* w_down;  // [H][I]
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

constexpr uint32_t kBatchDefaultChunk = 512;  // tokens per chunk of qe_prefill_batch (chunk = 0)
constexpr uint32_t kBatchMaxChunk = 2048;
constexpr uint32_t kVerifyMaxTokens = 64;  // tokens of one qe_verify call
static_assert(kVerifyMaxTokens <= qe::kIdsByValue, "verify ids travel in a kernel argument");

}  // namespace

// The chunk buffers, stream and per-layer K/V events of one of the extra streams of a chunked
// prefill (the first stream is the model's own, with its batch buffers).
struct ChunkBufs {
  uint8_t* mem = nullptr;
  uint32_t cap = 0;
  hipStream_t stream = nullptr;
  float *bx = nullptr, *bs = nullptr, *bqkv = nullptr, *bq = nullptr, *batt = nullptr, *bh = nullptr;
  float *bpart = nullptr, *bsplit = nullptr;
  std::vector<hipEvent_t> kv_ev;
};
constexpr int kMaxPrefillStreams = 4;

struct qe_model {
  qe::Checkpoint ckpt;
  qe_config cfg{};
  int device = 0;
  hipStream_t stream = nullptr;
  uint8_t* arena = nullptr;
  size_t arena_bytes = 0;
  const uint16_t* embed = nullptr;
  const uint16_t* lm_head = nullptr;
  const uint16_t* final_norm = nullptr;
  std::vector<Layer> layers;
  // activations
  float* x = nullptr;
  float* qkv = nullptr;
  float* att = nullptr;
  float* h = nullptr;
  float* logits = nullptr;
  ArgCand* cand = nullptr;
  uint32_t n_cand = 0;
  float* attn_part = nullptr;
  uint32_t* err = nullptr;  // device error word
  // two launches per layer (fused.hip) for the Qwen3-0.6B shape, when a launch deals its
  // workgroups to the XCDs round-robin (checked at load; QE_FUSED=0 keeps one launch per
  // stage): residual stream
  // ping-pong buffers, the 8 per-XCD partials of o_proj and of down, and the XCD sync words
  int fused = 0;  // 0: one launch per stage, 1: two launches per layer, 2: one persistent launch
  float *res0 = nullptr, *res1 = nullptr, *part_attn = nullptr, *part_mlp = nullptr;
  // the persistent launch's exchange buffers (pairs): each XCD's gathered residual stream after
  // the attention and after the MLP, and the per-XCD o_proj and down partials; its generation word
  uint2 *pxa = nullptr, *pxm = nullptr, *ppa = nullptr, *ppm = nullptr;
  uint32_t* pgen = nullptr;
  uint64_t layer_stride = 0;  // bytes between consecutive layers' tensors in the arena
  uint2 *fqkv = nullptr, *fh = nullptr;  // (value, tag) pairs exchanged inside an XCD
  uint32_t* fsync = nullptr;
  // a two-row verify pass through the two launches per layer: its step state {pos, 0, ..} and its
  // two token ids (res0 .. fh hold kFusedMaxRows rows)
  StepState* vstate = nullptr;
  uint32_t* vtokens = nullptr;
  hipEvent_t vstage_ev = nullptr;  // recorded after the copy of the pass's staging words
  ArgCand* vcand = nullptr;        // the pass's lm_head candidates, kFusedMaxRows x lm_head workgroups
  uint32_t* place_word = nullptr;
  // extra workgroups per XCD of each attention block that load the layer's MLP weights into the
  // L2 of their XCD (QE_FUSED_PF_ATTN), and of each MLP block that load the next layer's q|k|v
  // and o_proj weights (QE_FUSED_PF_MLP)
  uint32_t fused_pf_attn = 0, fused_pf_mlp = 0;
  // the attention block's slots without a run or o_proj rows load part of the layer's gate|up
  // rows into L2 for the MLP block (QE_FUSED_PF_IDLE=0: off)
  bool fused_pf_idle = true;
  // ... and the run workgroups the rest of them once their partials are out (QE_FUSED_PF_RUN=0: off)
  bool fused_pf_run = true;
  // attention runs of 32 positions up to this many cached positions (QE_FUSED_RUN32; a multiple
  // of 64, at most 512: 16 runs)
  uint64_t fused_run32 = 256;
  // each MLP block's workgroups load the next layer's q|k|v rows that their slot of the next
  // attention block reads into their XCD's L2 (QE_FUSED_PF_QKV=0: off)
  bool fused_pf_qkv = true;
  // the attention block's o_proj workgroups load the MLP block's down columns of their XCD into
  // its L2 while the runs work (QE_FUSED_PF_DOWN=0: off)
  bool fused_pf_down = true;
  uint8_t* scratch = nullptr;
  // qe_profile_step's in-step timing: while ts_buf is set, the i-th two-launch-layer launch that
  // enqueue_step_fused makes stamps its workgroups' start and end clocks at ts_buf + i *
  // kTsPerLaunch, and ts_stage[i] names its stage
  uint64_t* ts_buf = nullptr;
  const char** ts_stage = nullptr;
  uint32_t n_ts = 0, ts_cap = 0;
  // pinned host staging
  float* h_logits = nullptr;
  uint32_t* h_small = nullptr;  // [0..3] state staging, [8] token, [12] error word, [16..21] verify staging
  uint64_t weight_bytes = 0;
  // decode attention launches also load the next weights into L2 (QE_L2_PREFETCH=0 turns it off)
  bool l2_prefetch = true;
  // verify passes and chunks of up to kMvRowsMaxM tokens run their projections as multi-row
  // matvecs (QE_MV_ROWS=0: on the skinny GEMM)
  bool mv_rows = true;
  // passes of at most 8 / (q heads per KV head) tokens (a verify of up to 4 rows) attend on the
  // decode step's split kernel, all their q heads of a KV head sharing one read of its K/V
  // (QE_ROWS_SPLIT_ATTN=0: on the causal matrix-core kernel)
  bool rows_split_attn = true;
  // and their o_proj merges those runs in its prologue when they are few (QE_MV_MERGE=0: a
  // merge launch of its own)
  bool mv_merge = true;
  // chunks on the 64-row GEMM: the causal attention launch also loads o_proj's weights into the
  // L2 of the XCDs that will read them (QE_PREFILL_PREFETCH=0 turns it off)
  bool prefill_prefetch = true;
  // ... and their lm_head is the decode step's matvec over all their rows, each row's logits
  // equal to a decode step's (QE_LM_HEAD_ROWS=0: the skinny GEMM; a 2-row pass 0.83 -> 0.80 ms)
  bool lm_head_rows = true;
  // two-row verify passes through the two launches per layer (QE_VERIFY_FUSED=0: the batch path)
  bool verify_fused = true;
  // the decode step's final reduce applies the final norm (QE_LM_PRENORM=0: the lm_head does)
  bool lm_prenorm = true;
  // qe_decode_lookup decodes plain blocks while its verify passes emit tokens more slowly than
  // plain steps (QE_LOOKUP_ADAPTIVE=0: always drafts)
  bool lookup_adaptive = true;
  // its last timing of a plain decode step (seconds per step) and the position it was taken at
  double plain_step_s = 0;
  uint64_t plain_step_pos = 0;
  // multi-token (chunked prefill / verify) buffers, grown on first use: up to batch_cap tokens
  uint8_t* batch_mem = nullptr;
  uint32_t batch_cap = 0, batch_logit_rows = 0;
  float *bx = nullptr, *bs = nullptr, *bqkv = nullptr, *bq = nullptr, *batt = nullptr, *bh = nullptr;
  float* bpart = nullptr;   // causal attention partials
  float* bsplit = nullptr;  // split GEMM partial sums [splits][cap][hidden]
  // a chunked prefill on prefill_streams streams (QE_PREFILL_STREAMS, 1 to 4): the extra streams
  // with their chunk buffers and, per stream, one event per layer recorded once the chunk's K/V
  // rows of that layer are in the cache. 2048 tokens in chunks of 512: 10.8-11.2 ms on two
  // streams vs 12.5-12.8 on one (three streams: the same as two; four: slower). Once the process
  // has a second stream, eager launches on the first are slightly slower (a k = 4 verify
  // 1.22-1.23 vs 1.195-1.205 ms; 1.21 with the stream created but never used; destroying it
  // after each prefill does not help); graph-replayed decode steps are not.
  int prefill_streams = 2;
  ChunkBufs extra[kMaxPrefillStreams - 1];
  std::vector<hipEvent_t> kv_ev0;  // the first stream's per-layer K/V events
  hipEvent_t start_ev = nullptr;
  ArgCand* bcand = nullptr;  // row argmax candidates of a verify pass [kVerifyMaxTokens][kArgParts]
  float* blogits = nullptr;
  uint32_t* ids_dev = nullptr;  // the token ids of one qe_prefill_batch / qe_verify call
  uint64_t ids_cap = 0;

  ~qe_model() {  // teardown errors have nowhere to go; the handle is gone either way
    if (stream) (void)hipStreamSynchronize(stream);
    if (arena) (void)hipFree(arena);
    if (scratch) (void)hipFree(scratch);
    if (batch_mem) (void)hipFree(batch_mem);
    for (ChunkBufs& b : extra) {
      if (b.stream) (void)hipStreamSynchronize(b.stream);
      if (b.mem) (void)hipFree(b.mem);
      for (hipEvent_t e : b.kv_ev) (void)hipEventDestroy(e);
      if (b.stream) (void)hipStreamDestroy(b.stream);
    }
    for (hipEvent_t e : kv_ev0) (void)hipEventDestroy(e);
    if (start_ev) (void)hipEventDestroy(start_ev);
    if (vstage_ev) (void)hipEventDestroy(vstage_ev);
    if (ids_dev) (void)hipFree(ids_dev);
    if (h_logits) (void)hipHostFree(h_logits);
    if (h_small) (void)hipHostFree(h_small);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

struct qe_kv {
  qe_model* model = nullptr;
  uint64_t max_seq = 0;
  int dtype = QE_KV_F32;
  uint8_t* mem = nullptr;  // K, V, rope table, state, token ring
  void* k = nullptr;       // [L][n_kv][max_seq][D]
  void* v = nullptr;
  float* rope = nullptr;   // [max_seq][D/2][2]
  float* rope_cur = nullptr;  // [D/2][2]: the row of the current position (split attention)
  StepState* state = nullptr;
  uint32_t* tokens = nullptr;       // device token ring [tok_cap]
  uint32_t* host_tokens = nullptr;  // pinned, written by the argmax kernel
  uint32_t tok_cap = 0;
  uint32_t attn_splits = 1;     // the most attention runs per KV head a step uses
  // past 64 kAttnMaxMergeSplits positions, up to kAttnMaxWideSplits runs per KV head, merged by a
  // launch of their own before a plain o_proj (QE_WIDE_ATTN=0: kAttnMaxMergeSplits runs of more
  // tiles, merged in the o_proj prologue)
  bool wide_attn = true;
  // the attention shape enqueue_step records: runs per KV head and positions per run
  uint32_t step_splits = 1, step_run = 64;
  bool eager = false;           // launch the step kernel by kernel instead of replaying a graph
  // one captured step per attention shape (splits, run); launch_step picks it by position
  struct StepGraph {
    uint32_t splits, run;
    hipGraph_t graph;
    hipGraphExec_t exec;
  };
  std::vector<StepGraph> graphs;
  // two-row verify passes (verify_fused): one graph per attention shape and batch logits buffer
  struct VerifyGraph {
    uint32_t splits, run;
    const void* logits;
    const void* cand;
    hipGraph_t graph;
    hipGraphExec_t exec;
  };
  std::vector<VerifyGraph> vgraphs;
  std::vector<hipEvent_t> events;
  uint64_t len = 0;

  ~qe_kv() {
    if (model && model->stream) (void)hipStreamSynchronize(model->stream);
    for (auto& g : graphs) {
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
      if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    for (auto& g : vgraphs) {
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
      if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    for (auto e : events) (void)hipEventDestroy(e);
    if (mem) (void)hipFree(mem);
    if (host_tokens) (void)hipHostFree(host_tokens);
  }
};

namespace {

int check_device(int& dev) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(QE_ERR_NO_DEVICE, "no HIP device is visible");
  HIP_TRY(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, dev));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(QE_ERR_NO_DEVICE, "device %d is %s; this build targets gfx950 (MI355X)", dev, prop.gcnArchName);
  return QE_OK;
}

int validate_config(const qe_config& c) {
  if (c.head_dim != qe::kHeadDim) return fail(QE_ERR_UNSUPPORTED, "head_dim %llu: the kernels need 128", (unsigned long long)c.head_dim);
  if (!c.num_key_value_heads || c.num_attention_heads % c.num_key_value_heads)
    return fail(QE_ERR_UNSUPPORTED, "num_attention_heads must be a multiple of num_key_value_heads");
  uint64_t g = c.num_attention_heads / c.num_key_value_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8) return fail(QE_ERR_UNSUPPORTED, "q heads per KV head must be 1, 2, 4 or 8");
  const uint64_t H = c.hidden_size, I = c.intermediate_size, QD = c.num_attention_heads * c.head_dim;
  if (!H || !I || !c.num_hidden_layers || !c.vocab_size) return fail(QE_ERR_UNSUPPORTED, "zero dimension in config");
  if (H % 8 || I % 8 || QD % 8) return fail(QE_ERR_UNSUPPORTED, "hidden/intermediate/q sizes must be multiples of 8");
  if (H > 4096 || I > 4096 || QD > 4096) return fail(QE_ERR_UNSUPPORTED, "matvec input widths above 4096 are not supported");
  if (c.vocab_size >= 0xFFFFFFFFull) return fail(QE_ERR_UNSUPPORTED, "vocab too large");
  return QE_OK;
}

}  // namespace

extern "C" {

const char* qe_last_error(void) { return g_err.c_str(); }

int qe_model_load(const char* path, qe_model** out) {
  if (!path || !out) return fail(QE_ERR_ARG, "null argument");
  *out = nullptr;
  std::unique_ptr<qe_model> m(new qe_model());
  std::string err;
  int rc = m->ckpt.open(path, err);
  if (rc != QE_OK) return fail(rc, "%s", err.c_str());
  m->cfg = m->ckpt.config();
  if (const char* pf = getenv("QE_L2_PREFETCH")) m->l2_prefetch = strcmp(pf, "0") != 0;
  if (const char* mr = getenv("QE_MV_ROWS")) m->mv_rows = strcmp(mr, "0") != 0;
  if (const char* ra = getenv("QE_ROWS_SPLIT_ATTN")) m->rows_split_attn = strcmp(ra, "0") != 0;
  if (const char* mm = getenv("QE_MV_MERGE")) m->mv_merge = strcmp(mm, "0") != 0;
  if (const char* lh = getenv("QE_LM_HEAD_ROWS")) m->lm_head_rows = strcmp(lh, "0") != 0;
  if (const char* vf = getenv("QE_VERIFY_FUSED")) m->verify_fused = strcmp(vf, "0") != 0;
  if (const char* pn = getenv("QE_LM_PRENORM")) m->lm_prenorm = strcmp(pn, "0") != 0;
  if (const char* la = getenv("QE_LOOKUP_ADAPTIVE")) m->lookup_adaptive = strcmp(la, "0") != 0;
  if (const char* ps = getenv("QE_PREFILL_STREAMS"))
    m->prefill_streams = std::min(std::max(atoi(ps), 1), kMaxPrefillStreams);
  if (const char* pp = getenv("QE_PREFILL_PREFETCH")) m->prefill_prefetch = strcmp(pp, "0") != 0;
  const qe_config& c = m->cfg;
  const uint64_t H = c.hidden_size, I = c.intermediate_size, L = c.num_hidden_layers, V = c.vocab_size;
  const uint64_t D = c.head_dim, QD = c.num_attention_heads * D, KD = c.num_key_value_heads * D;

  // resolve every tensor on the host first, so a bad file fails before any device work
  struct Src { const uint16_t* p; uint64_t n; };
  auto get = [&](const std::string& name, uint64_t numel, Src& s) -> bool {
    s.p = m->ckpt.bf16(name, numel, err);
    s.n = numel;
    return s.p != nullptr;
  };
  Src embed, lm, fnorm;
  if (!get("model.embed_tokens.weight", V * H, embed) || !get("lm_head.weight", V * H, lm) ||
      !get("model.norm.weight", H, fnorm))
    return fail(QE_ERR_TENSOR, "%s", err.c_str());
  struct LSrc { Src in, q, k, v, qn, kn, o, post, g, u, d; };
  std::vector<LSrc> ls(L);
  for (uint64_t l = 0; l < L; l++) {
    LSrc& s = ls[l];
    if (!get(qe::layer_tensor(l, "input_layernorm.weight"), H, s.in) ||
        !get(qe::layer_tensor(l, "self_attn.q_proj.weight"), QD * H, s.q) ||
        !get(qe::layer_tensor(l, "self_attn.k_proj.weight"), KD * H, s.k) ||
        !get(qe::layer_tensor(l, "self_attn.v_proj.weight"), KD * H, s.v) ||
        !get(qe::layer_tensor(l, "self_attn.q_norm.weight"), D, s.qn) ||
        !get(qe::layer_tensor(l, "self_attn.k_norm.weight"), D, s.kn) ||
        !get(qe::layer_tensor(l, "self_attn.o_proj.weight"), H * QD, s.o) ||
        !get(qe::layer_tensor(l, "post_attention_layernorm.weight"), H, s.post) ||
        !get(qe::layer_tensor(l, "mlp.gate_proj.weight"), I * H, s.g) ||
        !get(qe::layer_tensor(l, "mlp.up_proj.weight"), I * H, s.u) ||
        !get(qe::layer_tensor(l, "mlp.down_proj.weight"), H * I, s.d))
      return fail(QE_ERR_TENSOR, "%s", err.c_str());
  }
  if ((rc = validate_config(c)) != QE_OK) return rc;
  if ((rc = check_device(m->device)) != QE_OK) return rc;
  m->weight_bytes = m->ckpt.weight_bytes_per_token();

  // arena layout (256-byte aligned tensors)
  size_t off = 0;
  auto take = [&](uint64_t elems) { size_t o = off; off = align_up(off + elems * 2, 256); return o; };
  const size_t o_embed = take(V * H), o_lm = take(V * H), o_fnorm = take(H);
  struct LOff { size_t in, qkv, qn, kn, o, post, gu, d; };
  std::vector<LOff> lo(L);
  for (uint64_t l = 0; l < L; l++) {
    lo[l].in = take(H);
    lo[l].qkv = take((QD + 2 * KD) * H);
    lo[l].qn = take(D);
    lo[l].kn = take(D);
    lo[l].o = take(H * QD);
    lo[l].post = take(H);
    lo[l].gu = take(2 * I * H);
    lo[l].d = take(H * I);
  }
  m->arena_bytes = off;
  HIP_TRY(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
  HIP_TRY(hipMalloc(&m->arena, m->arena_bytes));

  // upload through a pinned staging buffer; relayout q|k|v and gate/up on the host
  const size_t stage_bytes = size_t(64) << 20;
  uint8_t* stage = nullptr;
  HIP_TRY(hipHostMalloc(&stage, stage_bytes, hipHostMallocDefault));
  auto upload = [&](size_t dst_off, const void* src, size_t bytes) -> int {
    const uint8_t* s = static_cast<const uint8_t*>(src);
    for (size_t done = 0; done < bytes; done += stage_bytes) {
      size_t n = std::min(stage_bytes, bytes - done);
      memcpy(stage, s + done, n);
      hipError_t e = hipMemcpyAsync(m->arena + dst_off + done, stage, n, hipMemcpyHostToDevice, m->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
      if (e != hipSuccess) return fail(QE_ERR_HIP, "weight upload failed: %s", hipGetErrorString(e));
    }
    return QE_OK;
  };
  auto upload_rows_interleaved = [&](size_t dst_off, const uint16_t* a, const uint16_t* b, uint64_t rows, uint64_t cols) -> int {
    // row 2i <- a[i], row 2i+1 <- b[i]
    const uint64_t row_bytes = cols * 2;
    const uint64_t rows_per = std::max<uint64_t>(1, stage_bytes / (2 * row_bytes));
    for (uint64_t r0 = 0; r0 < rows; r0 += rows_per) {
      uint64_t nr = std::min(rows_per, rows - r0);
      for (uint64_t i = 0; i < nr; i++) {
        memcpy(stage + (2 * i) * row_bytes, a + (r0 + i) * cols, row_bytes);
        memcpy(stage + (2 * i + 1) * row_bytes, b + (r0 + i) * cols, row_bytes);
      }
      hipError_t e = hipMemcpyAsync(m->arena + dst_off + 2 * r0 * row_bytes, stage, 2 * nr * row_bytes, hipMemcpyHostToDevice, m->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
      if (e != hipSuccess) return fail(QE_ERR_HIP, "weight upload failed: %s", hipGetErrorString(e));
    }
    return QE_OK;
  };
  rc = upload(o_embed, embed.p, V * H * 2);
  if (rc == QE_OK) rc = upload(o_lm, lm.p, V * H * 2);
  if (rc == QE_OK) rc = upload(o_fnorm, fnorm.p, H * 2);
  for (uint64_t l = 0; l < L && rc == QE_OK; l++) {
    const LSrc& s = ls[l];
    rc = upload(lo[l].in, s.in.p, H * 2);
    if (rc == QE_OK) rc = upload(lo[l].qkv, s.q.p, QD * H * 2);
    if (rc == QE_OK) rc = upload(lo[l].qkv + QD * H * 2, s.k.p, KD * H * 2);
    if (rc == QE_OK) rc = upload(lo[l].qkv + (QD + KD) * H * 2, s.v.p, KD * H * 2);
    if (rc == QE_OK) rc = upload(lo[l].qn, s.qn.p, D * 2);
    if (rc == QE_OK) rc = upload(lo[l].kn, s.kn.p, D * 2);
    if (rc == QE_OK) rc = upload(lo[l].o, s.o.p, H * QD * 2);
    if (rc == QE_OK) rc = upload(lo[l].post, s.post.p, H * 2);
    if (rc == QE_OK) rc = upload_rows_interleaved(lo[l].gu, s.g.p, s.u.p, I, H);
    if (rc == QE_OK) rc = upload(lo[l].d, s.d.p, H * I * 2);
  }
  (void)hipHostFree(stage);
  if (rc != QE_OK) return rc;

  auto at = [&](size_t o) { return reinterpret_cast<const uint16_t*>(m->arena + o); };
  m->embed = at(o_embed);
  m->lm_head = at(o_lm);
  m->final_norm = at(o_fnorm);
  m->layers.resize(L);
  for (uint64_t l = 0; l < L; l++)
    m->layers[l] = Layer{at(lo[l].in), at(lo[l].qkv), at(lo[l].qn), at(lo[l].kn),
                         at(lo[l].o), at(lo[l].post), at(lo[l].gu), at(lo[l].d)};

  // activations and reduction scratch
  const uint32_t G = uint32_t(c.num_attention_heads / c.num_key_value_heads);
  m->n_cand = qe::matvec_num_blocks(uint32_t(V), uint32_t(H), qe::kLogits);
  size_t so = 0;
  auto stake = [&](size_t bytes) { size_t o = so; so = align_up(so + bytes, 256); return o; };
  constexpr size_t FR = qe::kFusedMaxRows;
  const size_t s_x = stake(FR * H * 4), s_qkv = stake((QD + 2 * KD) * 4), s_att = stake(QD * 4), s_h = stake(I * 4),
               s_logits = stake(V * 4), s_cand = stake(size_t(m->n_cand) * sizeof(ArgCand)),
               s_part = stake(std::max(size_t(c.num_key_value_heads) * qe::kAttnMaxWideSplits * G * qe::kPartStride * 4,
                                       FR * qe::kFusedPartPairs * 8)),
               s_err = stake(4), s_res0 = stake(FR * H * 4), s_res1 = stake(FR * H * 4),
               s_pa = stake(FR * qe::kFusedXcds * H * 4), s_pm = stake(FR * qe::kFusedXcds * H * 4),
               s_sync = stake(qe::kFusedSyncWords * 4), s_place = stake(qe::kFusedXcds * qe::kFusedSlots * 4),
               s_fqkv = stake(FR * qe::kFusedQkvRowPairs * 8), s_fh = stake(FR * qe::kFusedHPairs * 8),
               s_vstate = stake(sizeof(StepState) + FR * 4),
               s_vcand = stake(FR * qe::lm_head_rows_workgroups(uint32_t(V)) * sizeof(ArgCand)),
               s_pxa = stake(qe::kFusedXcds * H * 8), s_pxm = stake(qe::kFusedXcds * H * 8),
               s_ppa = stake(qe::kFusedXcds * H * 8), s_ppm = stake(qe::kFusedXcds * H * 8), s_pgen = stake(256);
  static_assert(qe::kFusedPartPairs * 8 <= size_t(qe::kFusedKv) * qe::kAttnMaxWideSplits * 2 * qe::kPartStride * 4,
                "fused attention partial pairs fit attn_part");
  HIP_TRY(hipMalloc(&m->scratch, so));
  HIP_TRY(hipMemset(m->scratch, 0, so));
  m->x = reinterpret_cast<float*>(m->scratch + s_x);
  m->qkv = reinterpret_cast<float*>(m->scratch + s_qkv);
  m->att = reinterpret_cast<float*>(m->scratch + s_att);
  m->h = reinterpret_cast<float*>(m->scratch + s_h);
  m->logits = reinterpret_cast<float*>(m->scratch + s_logits);
  m->cand = reinterpret_cast<ArgCand*>(m->scratch + s_cand);
  m->attn_part = reinterpret_cast<float*>(m->scratch + s_part);
  m->err = reinterpret_cast<uint32_t*>(m->scratch + s_err);
  m->res0 = reinterpret_cast<float*>(m->scratch + s_res0);
  m->res1 = reinterpret_cast<float*>(m->scratch + s_res1);
  m->part_attn = reinterpret_cast<float*>(m->scratch + s_pa);
  m->part_mlp = reinterpret_cast<float*>(m->scratch + s_pm);
  m->fsync = reinterpret_cast<uint32_t*>(m->scratch + s_sync);
  m->place_word = reinterpret_cast<uint32_t*>(m->scratch + s_place);
  m->fqkv = reinterpret_cast<uint2*>(m->scratch + s_fqkv);
  m->fh = reinterpret_cast<uint2*>(m->scratch + s_fh);
  m->vstate = reinterpret_cast<StepState*>(m->scratch + s_vstate);
  m->vtokens = reinterpret_cast<uint32_t*>(m->scratch + s_vstate + sizeof(StepState));
  m->vcand = reinterpret_cast<ArgCand*>(m->scratch + s_vcand);
  m->pxa = reinterpret_cast<uint2*>(m->scratch + s_pxa);
  m->pxm = reinterpret_cast<uint2*>(m->scratch + s_pxm);
  m->ppa = reinterpret_cast<uint2*>(m->scratch + s_ppa);
  m->ppm = reinterpret_cast<uint2*>(m->scratch + s_ppm);
  m->pgen = reinterpret_cast<uint32_t*>(m->scratch + s_pgen);
  if (const char* v = getenv("QE_FUSED_PF_ATTN")) m->fused_pf_attn = uint32_t(std::min(std::max(atoi(v), 0), 64));
  if (const char* v = getenv("QE_FUSED_PF_MLP")) m->fused_pf_mlp = uint32_t(std::min(std::max(atoi(v), 0), 64));
  if (const char* v = getenv("QE_FUSED_PF_IDLE")) m->fused_pf_idle = strcmp(v, "0") != 0;
  if (const char* v = getenv("QE_FUSED_PF_RUN")) m->fused_pf_run = strcmp(v, "0") != 0;
  if (const char* v = getenv("QE_FUSED_PF_QKV")) m->fused_pf_qkv = strcmp(v, "0") != 0;
  if (const char* v = getenv("QE_FUSED_PF_DOWN")) m->fused_pf_down = strcmp(v, "0") != 0;
  if (const char* v = getenv("QE_FUSED_RUN32")) m->fused_run32 = uint64_t(std::min(std::max(atoi(v), 0), 512)) / 64 * 64;
  // the layers' tensors sit at one stride in the arena (the persistent launch finds layer l's from
  // layer 0's)
  m->layer_stride = L > 1 ? lo[1].in - lo[0].in : 0;
  bool strided = true;
  for (uint64_t l = 0; l < L; l++) {
    const LOff& a = lo[l];
    const size_t d = l * m->layer_stride;
    strided = strided && a.in == lo[0].in + d && a.qkv == lo[0].qkv + d && a.qn == lo[0].qn + d &&
              a.kn == lo[0].kn + d && a.o == lo[0].o + d && a.post == lo[0].post + d && a.gu == lo[0].gu + d &&
              a.d == lo[0].d + d;
  }
  const char* fz = getenv("QE_FUSED");
  // default: two launches per layer (measured 1781-1800 tok/s on the 128-step bench against
  // 1766 for the persistent launch and 1598 for one launch per stage)
  const int want_mode = fz ? std::min(std::max(atoi(fz), 0), 2) : 1;
  if (want_mode > 0 && H == qe::kFusedH && I == qe::kFusedI && D == qe::kHeadDim &&
      c.num_attention_heads == qe::kFusedHeads && c.num_key_value_heads == qe::kFusedKv) {
    bool ok = false;
    uint32_t* host_ids = nullptr;
    HIP_TRY(hipHostMalloc(&host_ids, qe::kFusedXcds * qe::kFusedSlots * 4, hipHostMallocDefault));
    hipError_t pe = qe::fused_placement_check(m->place_word, host_ids, &ok, m->stream);
    if (getenv("QE_FUSED_DEBUG")) {
      fprintf(stderr, "qe: workgroup -> XCD placement (%s):", ok ? "round-robin" : "NOT round-robin");
      for (uint32_t i = 0; i < qe::kFusedXcds * qe::kFusedSlots; i++) fprintf(stderr, " %u", host_ids[i]);
      fprintf(stderr, "\n");
    }
    (void)hipHostFree(host_ids);
    HIP_TRY(pe);
    if (ok) m->fused = want_mode == 2 && strided && L <= 32 ? 2 : 1;
  }
  HIP_TRY(hipHostMalloc(&m->h_logits, V * 4, hipHostMallocDefault));
  HIP_TRY(hipHostMalloc(&m->h_small, 128, hipHostMallocDefault));
  *out = m.release();
  return QE_OK;
}

void qe_model_free(qe_model* model) { delete model; }

int qe_model_config(const qe_model* model, qe_config* out) {
  if (!model || !out) return fail(QE_ERR_ARG, "null argument");
  *out = model->cfg;
  return QE_OK;
}

uint64_t qe_weight_bytes_per_token(const qe_model* model) { return model ? model->weight_bytes : 0; }

int qe_model_fused_layers(const qe_model* model) { return model ? model->fused : 0; }

void* qe_model_stream(const qe_model* model) { return model ? static_cast<void*>(model->stream) : nullptr; }

uint64_t qe_kv_bytes_at(const qe_model* model, uint64_t pos, int kv_dtype) {
  if (!model) return 0;
  const qe_config& c = model->cfg;
  const uint64_t el = kv_dtype == QE_KV_BF16 ? 2 : 4;
  return 2 * c.num_hidden_layers * (pos + 1) * c.num_key_value_heads * c.head_dim * el;
}

}  // extern "C"

namespace {

// Enqueue one decode step (reads tokens[tok_idx] at state.pos) on the model stream.
// Timing marks for qe_profile_step: an event recorded before each kernel launch (and one after
// the last), with the stage name of the kernel that follows it.
// Enqueues one decode step on the model's stream. With `only` set, just the kernels of that
// stage are enqueued (qe_profile_step times each stage this way); `launches` counts them.
int enqueue_step_fused(qe_model* m, qe_kv* kv, const char* only, uint32_t* launches, uint32_t rows = 1);
// timing-buffer words per launch: a start and an end stamp for each of the layer workgroups
// (the prefetch workgroups beyond them stamp nothing)
constexpr size_t kTsPerLaunch = 2 * size_t(qe::kFusedXcds) * qe::kFusedSlots;
int enqueue_step_persist(qe_model* m, qe_kv* kv, const char* only, uint32_t* launches);

int enqueue_step(qe_model* m, qe_kv* kv, const char* only = nullptr, uint32_t* launches = nullptr) {
  // the persistent launch addresses a head's K/V region through 32-bit buffer offsets: caches of
  // more than 2^22 positions take the two-launch step
  if (m->fused == 2 && kv->max_seq <= (uint64_t(1) << 22)) return enqueue_step_persist(m, kv, only, launches);
  if (m->fused == 1) return enqueue_step_fused(m, kv, only, launches);
  const qe_config& c = m->cfg;
  const uint32_t H = uint32_t(c.hidden_size), I = uint32_t(c.intermediate_size), V = uint32_t(c.vocab_size);
  const uint32_t D = uint32_t(c.head_dim), QD = uint32_t(c.num_attention_heads) * D, KD = uint32_t(c.num_key_value_heads) * D;
  const size_t el = kv->dtype == QE_KV_BF16 ? 2 : 4;
  const size_t layer_kv = size_t(c.num_key_value_heads) * kv->max_seq * D * el;
  hipStream_t s = m->stream;
  // `only` names one stage or several joined by '+', e.g. "qkv+attention" for each layer's q|k|v
  // and attention launches (the attention then runs behind its producer, as in the step)
  auto want = [&](const char* name) {
    bool w = !only;
    const size_t n = strlen(name);
    for (const char* t = only; t && !w; t = strchr(t, '+') ? strchr(t, '+') + 1 : nullptr)
      w = strncmp(t, name, n) == 0 && (t[n] == '+' || t[n] == '\0');
    if (w && launches) ++*launches;
    return w;
  };
  auto matvec = [&](const MatvecParams& p, int pro, int epi) { return qe::launch_matvec_wide(p, pro, epi, s); };
  for (uint64_t l = 0; l < c.num_hidden_layers; l++) {
    const Layer& w = m->layers[l];
    MatvecParams p{};
    p.eps = c.rms_norm_eps;
    // [layer 0: embedding row (cpu_inference.rs:109-111)] input_layernorm + q|k|v projections
    // (cpu_inference.rs:129-132)
    p.w = w.w_qkv; p.x = m->x; p.nw = w.w_in; p.rows = QD + 2 * KD; p.cols = H; p.out = m->qkv;
    p.embed = m->embed; p.tokens = kv->tokens; p.state = kv->state; p.vocab = V; p.x_out = m->x; p.err = m->err;
    if (want("qkv")) HIP_TRY(matvec(p, l == 0 ? qe::kEmbedNorm : qe::kNorm, qe::kStore));
    // q/k norm + RoPE, K/V append, attention (cpu_inference.rs:134-162)
    AttnParams a{};
    a.qkv = m->qkv; a.q_norm = w.q_norm; a.k_norm = w.k_norm; a.rope = kv->rope; a.rope_cur = kv->rope_cur;
    a.k_cache = static_cast<uint8_t*>(kv->k) + l * layer_kv;
    a.v_cache = static_cast<uint8_t*>(kv->v) + l * layer_kv;
    a.partial = m->attn_part; a.state = kv->state; a.err = m->err;
    a.n_heads = uint32_t(c.num_attention_heads); a.n_kv = uint32_t(c.num_key_value_heads);
    a.max_seq = uint32_t(kv->max_seq); a.eps = c.rms_norm_eps; a.scale = 1.0f / sqrtf(float(D));
    a.kv_bf16 = kv->dtype == QE_KV_BF16;
    if (m->l2_prefetch) {
      // the attention is latency-bound: extra workgroups of its launch pull this layer's gate/up
      // and down weights into the L2 of the XCDs whose workgroups will read them (measured
      // against o_proj + gate/up, down alone and adding the next layer's q|k|v: this pair is
      // fastest)
      a.pf[0] = qe::l2_prefetch_target(w.w_gu, 2 * I, H, qe::kNorm, qe::kSiluPair);
      a.pf[1] = qe::l2_prefetch_target(w.w_down, H, I, qe::kCopy, qe::kResAdd);
      a.pf_slots = qe::l2_prefetch_slots(a.pf, qe::kMaxPrefetch);
      // once the layer's own K/V stream reaches half the prefetched bytes the attention is no
      // longer idle on HBM and the prefetch costs more than it saves (measured crossover:
      // ~1150 positions with an f32 cache, ~2300-2700 with bf16)
      const double pf_bytes = double(3 * I * H) * 2.0, kv_bytes_per_pos = double(2 * c.num_key_value_heads * D * el);
      a.pf_max_pos = uint32_t(std::min(0.5 * pf_bytes / kv_bytes_per_pos, double(kv->max_seq)));
    }
    p = MatvecParams{};
    p.w = w.w_o; p.x = m->att; p.rows = H; p.cols = QD; p.out = m->x;
    a.run = kv->step_run;
    if (want("attention")) HIP_TRY(qe::launch_attention_split(a, kv->step_splits, s));
    // merge the attention partials, then o_proj + residual (cpu_inference.rs:163-164): in the
    // o_proj prologue, or for more runs than it takes, in a launch of its own
    if (kv->step_splits > uint32_t(qe::kAttnMaxMergeSplits)) {
      if (want("o_proj")) {
        if (launches) ++*launches;  // the stage is two launches here
        HIP_TRY(qe::launch_attention_merge(a, kv->step_splits, m->att, s));
        HIP_TRY(qe::launch_matvec_wide(p, qe::kCopy, qe::kResAdd, s));
      }
    } else {
      p.attn_part = m->attn_part; p.attn_splits = kv->step_splits;
      p.attn_group = uint32_t(c.num_attention_heads / c.num_key_value_heads);
      if (want("o_proj")) HIP_TRY(qe::launch_matvec_wide(p, qe::kAttnMerge, qe::kResAdd, s));
    }
    // post_attention_layernorm + gate/up + silu*up (cpu_inference.rs:167-170)
    p = MatvecParams{};
    p.eps = c.rms_norm_eps;
    p.w = w.w_gu; p.x = m->x; p.nw = w.w_post; p.rows = 2 * I; p.cols = H; p.out = m->h;
    if (want("gate_up")) HIP_TRY(matvec(p, qe::kNorm, qe::kSiluPair));
    // down_proj + residual (cpu_inference.rs:171-172)
    p = MatvecParams{};
    p.w = w.w_down; p.x = m->h; p.rows = H; p.cols = I; p.out = m->x;
    if (want("down")) HIP_TRY(matvec(p, qe::kCopy, qe::kResAdd));
  }
  // final norm + lm_head + greedy candidates (cpu_inference.rs:175-178), then argmax
  MatvecParams p{};
  p.eps = c.rms_norm_eps;
  p.w = m->lm_head; p.x = m->x; p.nw = m->final_norm; p.rows = V; p.cols = H; p.out = m->logits; p.cand = m->cand;
  if (want("lm_head")) HIP_TRY(qe::launch_matvec(p, qe::kNorm, qe::kLogits, s));
  if (want("argmax")) {
    HIP_TRY(qe::launch_argmax(m->cand, m->n_cand, m->logits, kv->state, kv->tokens, kv->host_tokens, m->err,
                              kv->rope, kv->rope_cur, D / 2, s));
  }
  return QE_OK;
}

// The decode step as two launches per layer (fused.hip): each layer's attention block, then its
// MLP block; the final reduction of the last layer's partials, the lm_head and the argmax.
// `only` / `launches` as in enqueue_step, with the stages attn_block, mlp_block, final_reduce,
// lm_head and argmax.
// rows = 2: the layers of a two-row verify pass (m->vstate, m->vtokens; RoPE rows from the table), ending with the
// final residual rows in m->x; the caller runs the lm_head and the argmax over both rows.
int enqueue_step_fused(qe_model* m, qe_kv* kv, const char* only, uint32_t* launches, uint32_t rows) {
  const qe_config& c = m->cfg;
  const uint32_t V = uint32_t(c.vocab_size), D = uint32_t(c.head_dim);
  const size_t el = kv->dtype == QE_KV_BF16 ? 2 : 4;
  const size_t layer_kv = size_t(c.num_key_value_heads) * kv->max_seq * D * el;
  hipStream_t s = m->stream;
  auto want = [&](const char* name) {
    bool w = !only;
    const size_t n = strlen(name);
    for (const char* t = only; t && !w; t = strchr(t, '+') ? strchr(t, '+') + 1 : nullptr)
      w = strncmp(t, name, n) == 0 && (t[n] == '+' || t[n] == '\0');
    if (w && launches) ++*launches;
    return w;
  };
  // qe_profile_step's stamps: the next launch's slot of the timing buffer, or none
  auto ts_slot = [&](const char* stage) -> uint64_t* {
    if (!m->ts_buf || m->n_ts >= m->ts_cap) return nullptr;
    m->ts_stage[m->n_ts] = stage;
    return m->ts_buf + size_t(m->n_ts++) * kTsPerLaunch;
  };
  FusedLayerParams f{};
  f.rows = rows;
  f.qkv = m->fqkv; f.attn_part = reinterpret_cast<uint2*>(m->attn_part); f.h = m->fh;
  f.embed = m->embed; f.tokens = kv->tokens; f.vocab = V; f.state = kv->state;
  f.kv_bf16 = kv->dtype == QE_KV_BF16; f.max_seq = uint32_t(kv->max_seq); f.rope_cur = kv->rope_cur;
  f.splits = kv->step_splits; f.run = kv->step_run;
  if (rows > 1) {
    f.state = m->vstate; f.tokens = m->vtokens; f.rope_cur = kv->rope;
  }
  f.eps = c.rms_norm_eps; f.scale = 1.0f / sqrtf(float(D));
  f.sync = m->fsync; f.err = m->err;
  const uint32_t H = uint32_t(c.hidden_size), I = uint32_t(c.intermediate_size), NX = qe::kFusedXcds;
  const uint32_t QD = uint32_t(c.num_attention_heads) * D, KD = uint32_t(c.num_key_value_heads) * D;
  auto bytes = [](const uint16_t* w) { return reinterpret_cast<const uint8_t*>(w); };
  // prefetch only while a layer's K/V history is under half the prefetched bytes (past that the
  // attention itself streams from HBM)
  const double kv_pos_bytes = double(2 * c.num_key_value_heads * D * el);
  for (uint64_t l = 0; l < c.num_hidden_layers; l++) {
    const Layer& w = m->layers[l];
    f.w_in = w.w_in; f.w_qkv = w.w_qkv; f.q_norm = w.q_norm; f.k_norm = w.k_norm; f.w_o = w.w_o;
    f.w_post = w.w_post; f.w_gu = w.w_gu; f.w_down = w.w_down;
    f.k_cache = static_cast<uint8_t*>(kv->k) + l * layer_kv;
    f.v_cache = static_cast<uint8_t*>(kv->v) + l * layer_kv;
    // attention block: x = res0 + the previous layer's down partials (layer 0: the embedding);
    // its extra workgroups load this layer's gate|up rows and down columns of each XCD
    f.res_in = m->res0; f.part_in = m->part_mlp; f.res_out = m->res1; f.part_out = m->part_attn;
    for (auto& r : f.pf) r = qe::FusedPrefetch{};
    f.pf_wgs = m->fused_pf_attn;
    f.pf_idle = 0;
    f.pf_run = 0;
    f.qkv_next = nullptr;
    if (f.pf_wgs) {
      f.pf[0] = qe::FusedPrefetch{bytes(w.w_gu), 2 * I / NX * H * 2, 2 * I / NX * H * 2, 0, 1};
      f.pf[1] = qe::FusedPrefetch{bytes(w.w_down), I / NX * 2, I / NX * 2, I * 2, H};
    } else if (m->fused_pf_idle && f.splits < 16) {
      // the 16 - splits slots without a run each pull ~128 KB into L2 while the runs and o_proj
      // are latency-bound (a CU takes in ~30 GB/s; more would hold up the launch's end): the
      // first 2 (16 - splits) of each MLP slot's 24 gate|up rows, all 24 with 4 runs, 16 with 8
      // (measured at 130..257 positions: 1948 -> 2101 tok/s; all 24 rows with 8 runs: 1935 -> 1852)
      const uint32_t rows = std::min(2 * (16 - f.splits), 24u);
      f.pf[0] = qe::FusedPrefetch{bytes(w.w_gu), 2 * I / NX * H * 2, rows * H * 2, 24 * H * 2, qe::kFusedSlots};
      f.pf_idle = 1;
      if (rows < 24 && m->fused_pf_run) {
        // the run workgroups finish ~2 us before the launch does (the merge and o_proj follow
        // them): they load the rest of each MLP slot's rows, 8 of 24 with 8 runs
        f.pf[1] = qe::FusedPrefetch{bytes(w.w_gu) + size_t(rows) * H * 2, 2 * I / NX * H * 2, (24 - rows) * H * 2,
                                    24 * H * 2, qe::kFusedSlots};
        f.pf_run = 1;
      }
    }
    if (!f.pf_wgs && m->fused_pf_down)
      f.pf[2] = qe::FusedPrefetch{bytes(w.w_down), I / NX * 2, I / NX * 2, I * 2, H};
    f.pf_max_pos = uint32_t(std::min(0.5 * double(3 * I * H * 2) / kv_pos_bytes, double(kv->max_seq)));
    if (want("attn_block")) {
      f.ts = ts_slot("attn_block");
      HIP_TRY(f.ts ? qe::launch_fused_attn_timed(f, l == 0, s) : qe::launch_fused_attn(f, l == 0, s));
    }
    // MLP block: x = res1 + the o_proj partials; its extra workgroups load the next layer's q|k|v
    // rows and o_proj columns of each XCD
    f.res_in = m->res1; f.part_in = m->part_attn; f.res_out = m->res0; f.part_out = m->part_mlp;
    for (auto& r : f.pf) r = qe::FusedPrefetch{};
    f.pf_idle = 0;
    f.pf_run = 0;
    f.pf_wgs = l + 1 < c.num_hidden_layers ? m->fused_pf_mlp : 0;
    f.qkv_next = l + 1 < c.num_hidden_layers && m->fused_pf_qkv ? m->layers[l + 1].w_qkv : nullptr;
    if (f.pf_wgs) {
      const Layer& n = m->layers[l + 1];
      const uint32_t G = QD / KD;
      f.pf[0] = qe::FusedPrefetch{bytes(n.w_qkv), G * D * H * 2, G * D * H * 2, 0, 1};
      f.pf[1] = qe::FusedPrefetch{bytes(n.w_qkv) + size_t(QD) * H * 2, D * H * 2, D * H * 2, 0, 1};
      f.pf[2] = qe::FusedPrefetch{bytes(n.w_qkv) + size_t(QD + KD) * H * 2, D * H * 2, D * H * 2, 0, 1};
      f.pf[3] = qe::FusedPrefetch{bytes(n.w_o), G * D * 2, G * D * 2, QD * 2, H};
      f.pf_max_pos = uint32_t(std::min(0.5 * double((QD + 2 * KD + QD) * H * 2) / kv_pos_bytes, double(kv->max_seq)));
    }
    if (want("mlp_block")) {
      f.ts = ts_slot("mlp_block");
      HIP_TRY(f.ts ? qe::launch_fused_mlp_timed(f, s) : qe::launch_fused_mlp(f, s));
    }
  }
  // the reduce also applies the final norm, and the lm_head copies x as it is (a verify pass's
  // lm_head over its rows always)
  const bool prenorm = rows > 1 || m->lm_prenorm;
  if (want("final_reduce"))
    HIP_TRY(qe::launch_fused_reduce(m->res0, m->part_mlp, m->x, rows, prenorm ? m->final_norm : nullptr,
                                    c.rms_norm_eps, s));
  if (rows > 1) return QE_OK;
  MatvecParams p{};
  p.eps = c.rms_norm_eps;
  p.w = m->lm_head; p.x = m->x; p.nw = m->final_norm; p.rows = V; p.cols = uint32_t(c.hidden_size);
  p.out = m->logits; p.cand = m->cand;
  if (want("lm_head")) HIP_TRY(qe::launch_matvec(p, prenorm ? qe::kCopy : qe::kNorm, qe::kLogits, s));
  if (want("argmax")) {
    HIP_TRY(qe::launch_argmax(m->cand, m->n_cand, m->logits, kv->state, kv->tokens, kv->host_tokens, m->err,
                              kv->rope, kv->rope_cur, D / 2, s));
  }
  return QE_OK;
}

// The decode step as one persistent launch for all layers (persist.hip), then the lm_head and the
// argmax. `only` / `launches` as in enqueue_step, with the stages layers, lm_head and argmax.
int enqueue_step_persist(qe_model* m, qe_kv* kv, const char* only, uint32_t* launches) {
  const qe_config& c = m->cfg;
  const uint32_t V = uint32_t(c.vocab_size), D = uint32_t(c.head_dim);
  hipStream_t s = m->stream;
  auto want = [&](const char* name) {
    bool w = !only;
    const size_t n = strlen(name);
    for (const char* t = only; t && !w; t = strchr(t, '+') ? strchr(t, '+') + 1 : nullptr)
      w = strncmp(t, name, n) == 0 && (t[n] == '+' || t[n] == '\0');
    if (w && launches) ++*launches;
    return w;
  };
  const Layer& w = m->layers[0];
  qe::PersistParams q{};
  q.w_in = w.w_in; q.w_qkv = w.w_qkv; q.q_norm = w.q_norm; q.k_norm = w.k_norm; q.w_o = w.w_o;
  q.w_post = w.w_post; q.w_gu = w.w_gu; q.w_down = w.w_down;
  q.layer_stride = m->layer_stride; q.n_layers = uint32_t(c.num_hidden_layers);
  q.embed = m->embed; q.tokens = kv->tokens; q.vocab = V; q.state = kv->state;
  q.k_cache = kv->k; q.v_cache = kv->v; q.layer_kv = uint64_t(c.num_key_value_heads) * kv->max_seq * D;
  q.kv_bf16 = kv->dtype == QE_KV_BF16; q.max_seq = uint32_t(kv->max_seq); q.rope_cur = kv->rope_cur;
  q.splits = kv->step_splits; q.run = kv->step_run;
  q.eps = c.rms_norm_eps; q.scale = 1.0f / sqrtf(float(D));
  q.x_out = m->x;
  q.qkv = m->fqkv; q.attn_part = reinterpret_cast<uint2*>(m->attn_part); q.h = m->fh;
  q.xa = m->pxa; q.xm = m->pxm; q.part_a = m->ppa; q.part_m = m->ppm; q.gen = m->pgen; q.err = m->err;
  if (want("layers")) HIP_TRY(qe::launch_decode_persist(q, s));
  MatvecParams p{};
  p.eps = c.rms_norm_eps;
  p.w = m->lm_head; p.x = m->x; p.nw = m->final_norm; p.rows = V; p.cols = uint32_t(c.hidden_size);
  p.out = m->logits; p.cand = m->cand;
  if (want("lm_head")) HIP_TRY(qe::launch_matvec(p, qe::kNorm, qe::kLogits, s));
  if (want("argmax")) {
    HIP_TRY(qe::launch_argmax(m->cand, m->n_cand, m->logits, kv->state, kv->tokens, kv->host_tokens, m->err,
                              kv->rope, kv->rope_cur, D / 2, s));
  }
  return QE_OK;
}

// Multi-token buffers for up to `cap` tokens and `logit_rows` full logit rows.
int ensure_batch(qe_model* m, uint32_t cap, uint32_t logit_rows) {
  if (m->batch_mem && cap <= m->batch_cap && logit_rows <= m->batch_logit_rows) return QE_OK;
  cap = std::max(cap, m->batch_cap);
  logit_rows = std::max(logit_rows, m->batch_logit_rows);
  const qe_config& c = m->cfg;
  const size_t H = c.hidden_size, I = c.intermediate_size, D = c.head_dim;
  const size_t QD = c.num_attention_heads * D, KD = c.num_key_value_heads * D;
  size_t off = 0;
  auto take = [&](size_t b) { size_t o = off; off = align_up(off + b, 256); return o; };
  const size_t ox = take(cap * H * 4), os = take(cap * 4), oqkv = take(cap * (QD + 2 * KD) * 4),
               oq = take(cap * QD * 4), oatt = take(cap * QD * 4), oh = take(cap * I * 4),
               ologit = take(size_t(logit_rows) * c.vocab_size * 4);
  // attention partials: the most (tokens x key runs) any chunk of up to cap tokens asks for
  size_t part_rows = 0;
  for (uint32_t M = 1; M <= cap; M++)
    part_rows = std::max(part_rows, size_t(M) * qe::attn_causal_runs(M, 1u << 30, uint32_t(c.num_attention_heads),
                                                                     uint32_t(c.num_key_value_heads)));
  // the split kernel's partials for passes of up to 8 tokens: tokens x runs rows per q head
  part_rows = std::max(part_rows, size_t(std::min<uint32_t>(cap, 8)) * qe::kAttnMaxSplits);
  const size_t opart = take(part_rows * c.num_attention_heads * qe::kPartStride * 4);
  const size_t osplit = take(size_t(8) * cap * H * 4);  // gemm_splits returns at most 8
  const size_t ocand = take(size_t(kVerifyMaxTokens) * qe::kArgParts * sizeof(ArgCand));
  HIP_TRY(hipStreamSynchronize(m->stream));
  if (m->batch_mem) HIP_TRY(hipFree(m->batch_mem));
  m->batch_mem = nullptr;
  HIP_TRY(hipMalloc(&m->batch_mem, off));
  m->batch_cap = cap;
  m->batch_logit_rows = logit_rows;
  m->bx = reinterpret_cast<float*>(m->batch_mem + ox);
  m->bs = reinterpret_cast<float*>(m->batch_mem + os);
  m->bqkv = reinterpret_cast<float*>(m->batch_mem + oqkv);
  m->bq = reinterpret_cast<float*>(m->batch_mem + oq);
  m->batt = reinterpret_cast<float*>(m->batch_mem + oatt);
  m->bh = reinterpret_cast<float*>(m->batch_mem + oh);
  m->blogits = reinterpret_cast<float*>(m->batch_mem + ologit);
  m->bpart = reinterpret_cast<float*>(m->batch_mem + opart);
  m->bsplit = reinterpret_cast<float*>(m->batch_mem + osplit);
  m->bcand = reinterpret_cast<ArgCand*>(m->batch_mem + ocand);
  return QE_OK;
}

// The extra streams of a chunked prefill on `streams` streams: their chunk buffers for up to
// `cap` tokens (those of ensure_batch without the logit rows), and the per-layer K/V events.
int ensure_streams(qe_model* m, uint32_t cap, int streams) {
  const qe_config& c = m->cfg;
  const size_t L = c.num_hidden_layers;
  auto events = [&](std::vector<hipEvent_t>& v) -> int {
    while (v.size() < L) {
      hipEvent_t e;
      HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
      v.push_back(e);
    }
    return QE_OK;
  };
  if (!m->start_ev) HIP_TRY(hipEventCreateWithFlags(&m->start_ev, hipEventDisableTiming));
  if (int rc = events(m->kv_ev0)) return rc;
  const size_t H = c.hidden_size, I = c.intermediate_size, D = c.head_dim;
  const size_t QD = c.num_attention_heads * D, KD = c.num_key_value_heads * D;
  for (int i = 0; i + 1 < streams; i++) {
    ChunkBufs& b = m->extra[i];
    if (!b.stream) HIP_TRY(hipStreamCreateWithFlags(&b.stream, hipStreamNonBlocking));
    if (int rc = events(b.kv_ev)) return rc;
    if (b.mem && cap <= b.cap) continue;
    const uint32_t bcap = std::max(cap, b.cap);
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off = align_up(off + n, 256); return o; };
    const size_t ox = take(bcap * H * 4), os = take(bcap * 4), oqkv = take(bcap * (QD + 2 * KD) * 4),
                 oq = take(bcap * QD * 4), oatt = take(bcap * QD * 4), oh = take(bcap * I * 4);
    size_t part_rows = 0;
    for (uint32_t M = 1; M <= bcap; M++)
      part_rows = std::max(part_rows, size_t(M) * qe::attn_causal_runs(M, 1u << 30, uint32_t(c.num_attention_heads),
                                                                       uint32_t(c.num_key_value_heads)));
    part_rows = std::max(part_rows, size_t(std::min<uint32_t>(bcap, 8)) * qe::kAttnMaxSplits);
    const size_t opart = take(part_rows * c.num_attention_heads * qe::kPartStride * 4);
    const size_t osplit = take(size_t(8) * bcap * H * 4);
    HIP_TRY(hipStreamSynchronize(b.stream));
    if (b.mem) HIP_TRY(hipFree(b.mem));
    b.mem = nullptr;
    HIP_TRY(hipMalloc(&b.mem, off));
    b.cap = bcap;
    b.bx = reinterpret_cast<float*>(b.mem + ox);
    b.bs = reinterpret_cast<float*>(b.mem + os);
    b.bqkv = reinterpret_cast<float*>(b.mem + oqkv);
    b.bq = reinterpret_cast<float*>(b.mem + oq);
    b.batt = reinterpret_cast<float*>(b.mem + oatt);
    b.bh = reinterpret_cast<float*>(b.mem + oh);
    b.bpart = reinterpret_cast<float*>(b.mem + opart);
    b.bsplit = reinterpret_cast<float*>(b.mem + osplit);
  }
  return QE_OK;
}

// Copies n token ids to the device (in stream order, before the kernels that read them).
int upload_ids(qe_model* m, const uint32_t* ids, uint64_t n) {
  if (n > m->ids_cap) {
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (m->ids_dev) HIP_TRY(hipFree(m->ids_dev));
    m->ids_dev = nullptr;
    m->ids_cap = 0;
    HIP_TRY(hipMalloc(&m->ids_dev, n * 4));
    m->ids_cap = n;
  }
  HIP_TRY(hipMemcpyAsync(m->ids_dev, ids, n * 4, hipMemcpyHostToDevice, m->stream));
  return QE_OK;
}

enum BatchLogits { kNoLogits, kLastLogits, kAllLogits };

// A chunk of a multi-stream prefill, on stream `set` (0: the model's, with its batch buffers; i > 0:
// extra[i - 1]): its layer-l attention waits for wait_kv[l] (the previous chunk's event, on another
// stream), and kv_done[l] is recorded after that wait and this chunk's layer-l K/V rows.
struct ChunkStream {
  int set;
  hipEvent_t* kv_done;
  hipEvent_t* wait_kv;
};

// One chunk of M tokens at positions start..start+M-1 through every layer, appending their K/V.
// The ids are device memory (ids), or for a short pass the kernel argument ids_v (ids null).
// kAllLogits: logits of every row to m->blogits [M][V]; kLastLogits: the last row's logits to
// m->logits (the decode step's buffer); kNoLogits: none (an inner chunk). cs: a chunk of a
// multi-stream prefill (its buffers, stream and events), else the model's stream and buffers.
int enqueue_batch(qe_model* m, qe_kv* kv, uint32_t M, uint32_t start, const uint32_t* ids, BatchLogits logits,
                  const qe::TokenIds* ids_v = nullptr, const ChunkStream* cs = nullptr) {
  const ChunkBufs* xb = cs && cs->set > 0 ? &m->extra[cs->set - 1] : nullptr;
  float* const bx = xb ? xb->bx : m->bx;
  float* const bs = xb ? xb->bs : m->bs;
  float* const bqkv = xb ? xb->bqkv : m->bqkv;
  float* const bq = xb ? xb->bq : m->bq;
  float* const batt = xb ? xb->batt : m->batt;
  float* const bh = xb ? xb->bh : m->bh;
  float* const bpart = xb ? xb->bpart : m->bpart;
  float* const bsplit = xb ? xb->bsplit : m->bsplit;
  const qe_config& c = m->cfg;
  const uint32_t H = uint32_t(c.hidden_size), I = uint32_t(c.intermediate_size), V = uint32_t(c.vocab_size);
  const uint32_t D = uint32_t(c.head_dim), QD = uint32_t(c.num_attention_heads) * D, KD = uint32_t(c.num_key_value_heads) * D;
  const size_t el = kv->dtype == QE_KV_BF16 ? 2 : 4;
  const size_t layer_kv = size_t(c.num_key_value_heads) * kv->max_seq * D * el;
  hipStream_t s = xb ? xb->stream : m->stream;
  const float eps = c.rms_norm_eps;
  // Up to kGemmSkinnyMaxM rows the skinny GEMM computes each norm's row scales itself and adds
  // residuals in its epilogue. Past that, bs holds the row scales of the current norm input:
  // from a rownorm launch for layer 0, then from the reduction that finishes each split o_proj /
  // down (residual add + the next norm's scales in one pass).
  // Up to kMvRowsMaxM rows the projections are matvecs over the M token rows: each weight is
  // loaded once per pass, the norm is computed per row in the kernel and the residual is added in
  // its epilogue (the lm_head of a verify stays on the skinny GEMM).
  const bool skinny = M <= qe::kGemmSkinnyMaxM;
  const bool mv = m->mv_rows && M <= qe::kMvRowsMaxM;
  auto gemm = [&](const float* A, uint32_t lda, const uint16_t* gain, const uint16_t* W, uint32_t N, uint32_t K,
                  float* C, uint32_t ldc, int epi) -> int {
    // gate|up (the widest projection) at 4 rows is faster on the skinny GEMM: 1.405 vs 1.431 ms
    // per k = 4 verify (at 3 rows the matvec still wins)
    if (mv && lda == K && W != m->lm_head && !(epi == qe::kGemmSiluPair && M >= 4)) {
      qe::MvRowsParams r{W, A, gain, C, M, N, K, ldc, eps};
      HIP_TRY(qe::launch_mv_rows(r, gain != nullptr, epi, s));
      return QE_OK;
    }
    qe::GemmParams g{A, lda, bs, gain, W, M, N, K, C, ldc, eps};
    HIP_TRY(qe::launch_gemm(g, gain != nullptr, epi, s));
    return QE_OK;
  };
  // x += A W^T, then bs = the row scales of the updated x
  auto gemm_resadd = [&](const float* A, uint32_t lda, const uint16_t* W, uint32_t K) -> int {
    if (mv || (skinny && qe::gemm_splits(M, H, K) == 1)) return gemm(A, lda, nullptr, W, H, K, bx, H, qe::kGemmResAdd);
    if (!skinny && K % 64) {  // no split: residual epilogue, then the row scales
      if (int rc2 = gemm(A, lda, nullptr, W, H, K, bx, H, qe::kGemmResAdd)) return rc2;
      HIP_TRY(qe::launch_rownorm(bx, M, H, eps, bs, s));
      return QE_OK;
    }
    const uint32_t z = qe::gemm_splits(M, H, K);
    qe::GemmParams g{A, lda, nullptr, nullptr, W, M, H, K, bsplit, H, eps};
    HIP_TRY(qe::launch_gemm_split(g, z, s));
    HIP_TRY(qe::launch_resadd_partials(bx, bsplit, z, M, H, eps, bs, s));
    return QE_OK;
  };
  int rc;
  if (ids_v) HIP_TRY(qe::launch_embed_rows(m->embed, *ids_v, M, H, bx, s));
  else HIP_TRY(qe::launch_embed_rows(m->embed, ids, M, H, bx, s));
  if (!skinny) HIP_TRY(qe::launch_rownorm(bx, M, H, eps, bs, s));
  for (uint64_t l = 0; l < c.num_hidden_layers; l++) {
    const Layer& w = m->layers[l];
    // q/k norm + RoPE, K/V append, causal attention (cpu_inference.rs:134-162)
    qe::BatchAttnParams a{};
    a.qkv = bqkv; a.q = bq; a.att = batt; a.q_norm = w.q_norm; a.k_norm = w.k_norm; a.rope = kv->rope;
    a.k_cache = static_cast<uint8_t*>(kv->k) + l * layer_kv;
    a.v_cache = static_cast<uint8_t*>(kv->v) + l * layer_kv;
    a.M = M; a.start = start; a.max_seq = uint32_t(kv->max_seq);
    a.n_heads = uint32_t(c.num_attention_heads); a.n_kv = uint32_t(c.num_key_value_heads);
    a.eps = eps; a.scale = 1.0f / sqrtf(float(D)); a.kv_bf16 = kv->dtype == QE_KV_BF16;
    // input_layernorm + q|k|v (cpu_inference.rs:129-132); chunks on the 64-row GEMM do the q/k
    // norm, RoPE and K/V append in its epilogue, the others in k_qk_rope
    hipError_t fused = hipErrorNotSupported;
    if (!mv && !skinny) {
      const qe::GemmParams g{bx, H, bs, w.w_in, w.w_qkv, M, QD + 2 * KD, H, bqkv, QD + 2 * KD, eps};
      fused = qe::launch_gemm_qk_rope(g, a, s);
      if (fused != hipSuccess && fused != hipErrorNotSupported) HIP_TRY(fused);
    }
    if (fused != hipSuccess) {
      if ((rc = gemm(bx, H, w.w_in, w.w_qkv, QD + 2 * KD, H, bqkv, QD + 2 * KD, qe::kGemmStore))) return rc;
      HIP_TRY(qe::launch_qk_rope(a, s));
    }
    // multi-stream prefill: the attention reads the previous chunks' K/V rows of this layer,
    // appended on other streams. The event is recorded after this chunk's own wait, so that it
    // stands for the K/V rows of this chunk and of every chunk before it (chunk i waits for
    // chunk i-1 only, whatever the number of streams).
    if (cs && cs->wait_kv) HIP_TRY(hipStreamWaitEvent(s, cs->wait_kv[l], 0));
    if (cs && cs->kv_done) HIP_TRY(hipEventRecord(cs->kv_done[l], s));
    const uint32_t rows_per_kv = (a.n_heads / a.n_kv) * M;
    uint32_t merge_splits = 0;  // > 0: o_proj merges this many attention runs in its prologue
    if (m->rows_split_attn && (rows_per_kv == 1 || rows_per_kv == 2 || rows_per_kv == 4 || rows_per_kv == 8)) {
      // few tokens: the split kernel, the q heads of all M tokens of a KV head over one read of
      // its K/V, each token causal (positions up to its own), runs of 64 positions
      AttnParams r{};
      r.qkv = bq; r.k_cache = a.k_cache; r.v_cache = a.v_cache; r.partial = bpart;
      r.n_kv = a.n_kv; r.n_heads = a.n_kv * rows_per_kv; r.max_seq = a.max_seq; r.scale = a.scale;
      r.kv_bf16 = a.kv_bf16; r.n_pos_fixed = start + M; r.tok_heads = a.n_heads / a.n_kv; r.q_tok_stride = QD;
      // 8 rows (4 tokens): two workgroups of 4 rows per KV head halve each one's score and
      // P.V work for a second read of the K/V runs, mostly from L2 (verify of 4 tokens at
      // position 2048: 1.321 -> 1.261 ms; 4 workgroups of 2 rows: 1.399 ms; 4 rows: no change)
      if (rows_per_kv == 8) r.row_split = 2;
      if (m->l2_prefetch && mv) {
        // as in the decode step: the attention is latency-bound, so extra workgroups load this
        // layer's gate|up (the skinny GEMM's rows at 4 tokens, else the multi-row matvec's) and
        // down weights into the L2 of the XCDs that will read them
        r.pf[0] = M >= 4 ? qe::skinny_prefetch_target(w.w_gu, 2 * I, H)
                         : qe::l2_prefetch_target(w.w_gu, 2 * I, H, qe::kNorm, qe::kSiluPair);
        r.pf[1] = qe::l2_prefetch_target(w.w_down, H, I, qe::kCopy, qe::kResAdd);
        r.pf_slots = qe::l2_prefetch_slots(r.pf, qe::kMaxPrefetch);
      }
      const uint32_t splits = std::min<uint32_t>(qe::kAttnMaxSplits, (start + M + 63) / 64);
      // with few runs the multi-row o_proj merges them in its prologue, as the decode step's does
      if (mv && m->mv_merge && qe::mv_rows_merge_fits(M, splits) && QD % D == 0 && QD / 8 <= 256)
        merge_splits = splits;
      HIP_TRY(qe::launch_attention_rows(r, splits, merge_splits ? nullptr : batt, s));
    } else {
      a.part = bpart;
      if (m->prefill_prefetch && !skinny) {
        // the attention is latency-bound: extra workgroups load o_proj's weights (a split GEMM)
        // into L2
        a.pf.pf[0] = qe::gemm_prefetch_target(w.w_o, M, H, QD, qe::kGemmPartial);
        a.pf.slots = qe::tile_prefetch_slots(a.pf.pf, qe::kMaxPrefetch);
      }
      HIP_TRY(qe::launch_attn_causal(a, qe::attn_causal_runs(M, start, a.n_heads, a.n_kv), s));
    }
    // o_proj + residual (cpu_inference.rs:163-164)
    if (merge_splits) {
      qe::MvRowsParams r{w.w_o, nullptr, nullptr, bx, M, H, QD, H, eps};
      r.attn_part = bpart; r.attn_splits = merge_splits; r.tok_heads = a.n_heads / a.n_kv;
      HIP_TRY(qe::launch_mv_rows_merge(r, s));
    } else if ((rc = gemm_resadd(batt, QD, w.w_o, QD))) {
      return rc;
    }
    // post_attention_layernorm + gate/up + silu*up, down + residual (cpu_inference.rs:167-172)
    if ((rc = gemm(bx, H, w.w_post, w.w_gu, 2 * I, H, bh, I, qe::kGemmSiluPair))) return rc;
    if ((rc = gemm_resadd(bh, I, w.w_down, I))) return rc;
  }
  // final norm + lm_head (cpu_inference.rs:175-178)
  if (logits == kAllLogits) {
    hipError_t lh = hipErrorNotSupported;
    if (mv && m->lm_head_rows) {
      const qe::MvRowsParams r{m->lm_head, bx, m->final_norm, m->blogits, M, V, H, V, eps};
      lh = qe::launch_lm_head_rows(r, s);
      if (lh != hipSuccess && lh != hipErrorNotSupported) HIP_TRY(lh);
    }
    if (lh != hipSuccess &&
        (rc = gemm(bx, H, m->final_norm, m->lm_head, V, H, m->blogits, V, qe::kGemmStore)))
      return rc;
  } else if (logits == kLastLogits) {
    MatvecParams p{};
    p.eps = eps; p.w = m->lm_head; p.x = bx + size_t(M - 1) * H; p.nw = m->final_norm;
    p.rows = V; p.cols = H; p.out = m->logits; p.cand = m->cand;
    HIP_TRY(qe::launch_matvec(p, qe::kNorm, qe::kLogits, s));
  }
  return QE_OK;
}

// host -> device: state {pos, tok_idx = 0} and tokens[0] = token, through pinned staging; the
// RoPE row of pos becomes rope_cur (k_argmax advances it with pos after every step)
int set_state(qe_model* m, qe_kv* kv, uint32_t token, uint64_t pos) {
  HIP_TRY(hipStreamSynchronize(m->stream));
  StepState st{uint32_t(pos), 0u, uint32_t(kv->max_seq), kv->tok_cap};
  memcpy(m->h_small, &st, sizeof(st));
  m->h_small[8] = token;
  const size_t D = m->cfg.head_dim;
  HIP_TRY(hipMemcpyAsync(kv->state, m->h_small, sizeof(st), hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipMemcpyAsync(kv->tokens, m->h_small + 8, 4, hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipMemcpyAsync(kv->rope_cur, kv->rope + pos * D, D * 4, hipMemcpyDeviceToDevice, m->stream));
  return QE_OK;
}

// The attention shape of a decode step at position pos: runs of `run` positions (a multiple of
// 64, the least that covers pos + 1 positions in kv->attn_splits runs) and `splits` runs per KV
// head. Runs of 64 come in 4, 8 or attn_splits, so that a short context in a large cache does
// not launch (and o_proj does not merge) empty runs; longer runs always use attn_splits. The
// host knows every step's position, so each step replays the graph of its shape and the
// attention kernel starts its first K/V tile load at launch instead of after reading pos.
void step_shape(const qe_kv* kv, uint64_t pos, uint32_t& splits, uint32_t& run) {
  const uint64_t n = pos + 1, S = kv->attn_splits;
  if (kv->model->fused) {
    // one run per slot of an XCD: up to fused_run32 positions runs of 32 in 4, 8 or 16 (half the
    // K/V and the work per run of a 64-position tile); then runs of 64 in 4, 8, 16 or 32 up to
    // 64 x 32 positions, then 32 runs of a whole number of tiles
    if (kv->model->fused == 1 && n <= kv->model->fused_run32) {  // (the persistent launch takes runs of 64)
      run = 32;
      const uint64_t active = (n + 31) / 32;
      splits = uint32_t(active <= 4 ? 4 : active <= 8 ? 8 : 16);
      return;
    }
    const uint64_t R = qe::kFusedMaxRuns;
    run = uint32_t(64 * ((n + 64 * R - 1) / (64 * R)));
    const uint64_t active = (n + run - 1) / run;
    splits = uint32_t(run > 64 ? R : active <= 4 ? 4 : active <= 8 ? 8 : active <= 16 ? 16 : R);
    return;
  }
  if (kv->wide_attn && n > 64 * uint64_t(qe::kAttnMaxMergeSplits)) {
    // long context: runs of whole tiles over up to kAttnMaxWideSplits workgroups per KV head,
    // their count rounded up to a multiple of 8 (fewer step graphs; the extra runs are empty).
    // Against 16 runs of 128..256 positions merged in o_proj, at 4096 steps from a 130-token
    // prompt: 1288 vs 1218 tok/s (f32 cache; 1158 vs 1054 over the last 512 steps), 1339 vs
    // 1306 (bf16 cache).
    const uint64_t W = qe::kAttnMaxWideSplits;
    run = uint32_t(64 * ((n + 64 * W - 1) / (64 * W)));
    const uint64_t active = (n + run - 1) / run;
    splits = uint32_t(std::min<uint64_t>(W, 8 * ((active + 7) / 8)));
    return;
  }
  run = uint32_t(64 * ((n + 64 * S - 1) / (64 * S)));
  const uint64_t active = (n + run - 1) / run;
  splits = uint32_t(run == 64 ? (active <= 4 ? std::min<uint64_t>(4, S) : active <= 8 ? std::min<uint64_t>(8, S) : S) : S);
}

// capture one decode step with attention shape (splits, run)
int capture_step(qe_model* m, qe_kv* kv, uint32_t splits, uint32_t run) {
  HIP_TRY(hipStreamSynchronize(m->stream));
  kv->step_splits = splits;
  kv->step_run = run;
  HIP_TRY(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
  int rc = enqueue_step(m, kv);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(m->stream, &g);
  if (rc != QE_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return fail(QE_ERR_HIP, "graph capture failed: %s", hipGetErrorString(e));
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return fail(QE_ERR_HIP, "graph instantiation failed: %s", hipGetErrorString(e));
  }
  kv->graphs.push_back({splits, run, g, ex});
  return QE_OK;
}

// one decode step at position pos on the model stream: a replay of the graph of its attention
// shape (captured here the first time a shape is needed), or eager launches
int launch_step(qe_model* m, qe_kv* kv, uint64_t pos) {
  uint32_t splits, run;
  step_shape(kv, pos, splits, run);
  if (kv->eager) {
    kv->step_splits = splits;
    kv->step_run = run;
    return enqueue_step(m, kv);
  }
  for (const auto& g : kv->graphs)
    if (g.splits == splits && g.run == run) {
      kv->step_splits = splits;
      kv->step_run = run;
      HIP_TRY(hipGraphLaunch(g.exec, m->stream));
      return QE_OK;
    }
  int rc = capture_step(m, kv, splits, run);
  if (rc) return rc;
  HIP_TRY(hipGraphLaunch(kv->graphs.back().exec, m->stream));
  return QE_OK;
}

// read and clear the device error word
int check_err(qe_model* m) {
  HIP_TRY(hipMemcpyAsync(m->h_small + 12, m->err, 4, hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  uint32_t e = m->h_small[12];
  if (e) {
    HIP_TRY(hipMemsetAsync(m->err, 0, 4, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return fail(QE_ERR_KERNEL,
                "kernel error bits 0x%x (1: pos >= max_seq, 2: token >= vocab, 4: token ring full, "
                "8: attention runs do not cover pos)", e);
  }
  return QE_OK;
}

}  // namespace

extern "C" {

int qe_kv_new(qe_model* model, uint64_t max_seq, int kv_dtype, qe_kv** out) {
  if (!model || !out) return fail(QE_ERR_ARG, "null argument");
  *out = nullptr;
  if (max_seq == 0 || max_seq > (1u << 24)) return fail(QE_ERR_ARG, "max_seq must be in 1..2^24");
  if (kv_dtype != QE_KV_F32 && kv_dtype != QE_KV_BF16) return fail(QE_ERR_ARG, "kv_dtype must be QE_KV_F32 or QE_KV_BF16");
  const qe_config& c = model->cfg;
  std::unique_ptr<qe_kv> kv(new qe_kv());
  kv->model = model;
  kv->max_seq = max_seq;
  kv->dtype = kv_dtype;
  kv->tok_cap = uint32_t(max_seq + 2);
  const size_t el = kv_dtype == QE_KV_BF16 ? 2 : 4;
  const size_t D = c.head_dim;
  const size_t kv_bytes = c.num_hidden_layers * c.num_key_value_heads * max_seq * D * el;
  const size_t rope_bytes = max_seq * D * 4;
  size_t off = 0;
  auto take = [&](size_t b) { size_t o = off; off = align_up(off + b, 256); return o; };
  const size_t ok_ = take(kv_bytes), ov = take(kv_bytes), orope = take(rope_bytes), ocur = take(D * 4),
               ost = take(sizeof(StepState)), otok = take(size_t(kv->tok_cap) * 4);
  HIP_TRY(hipSetDevice(model->device));
  HIP_TRY(hipMalloc(&kv->mem, off));
  HIP_TRY(hipMemsetAsync(kv->mem, 0, off, model->stream));
  kv->k = kv->mem + ok_;
  kv->v = kv->mem + ov;
  kv->rope = reinterpret_cast<float*>(kv->mem + orope);
  kv->rope_cur = reinterpret_cast<float*>(kv->mem + ocur);
  kv->state = reinterpret_cast<StepState*>(kv->mem + ost);
  kv->tokens = reinterpret_cast<uint32_t*>(kv->mem + otok);
  HIP_TRY(hipHostMalloc(&kv->host_tokens, size_t(kv->tok_cap) * 4, hipHostMallocDefault));
  memset(kv->host_tokens, 0, size_t(kv->tok_cap) * 4);

  // RoPE table, same expressions as rope_table (metal_inference.rs:140-154) and rope
  // (cpu_inference.rs:203-215): freq_i = theta^(-2i/D) via powf, then sin/cos of pos*freq
  std::vector<float> table(max_seq * D);
  const size_t half = D / 2;
  std::vector<float> freqs(half);
  for (size_t i = 0; i < half; i++) freqs[i] = powf(c.rope_theta, -2.0f * float(i) / float(D));
  for (size_t pos = 0; pos < max_seq; pos++)
    for (size_t i = 0; i < half; i++) {
      const float ang = float(pos) * freqs[i];
      table[(pos * half + i) * 2] = cosf(ang);
      table[(pos * half + i) * 2 + 1] = sinf(ang);
    }
  HIP_TRY(hipMemcpyAsync(kv->rope, table.data(), rope_bytes, hipMemcpyHostToDevice, model->stream));
  HIP_TRY(hipStreamSynchronize(model->stream));

  // the most attention runs (workgroups) per KV head a step uses: one per 64 cached positions,
  // at most kAttnMaxMergeSplits (the o_proj prologue merges that many partials per q head);
  // step_shape picks each step's runs within this
  kv->attn_splits = uint32_t(std::min<uint64_t>((max_seq + 63) / 64, qe::kAttnMaxMergeSplits));
  if (const char* e = getenv("QE_WIDE_ATTN")) kv->wide_attn = strcmp(e, "0") != 0;

  // QE_LAUNCH=eager launches each step kernel by kernel (for tools that do not follow graph
  // replays, such as counter collection); otherwise one decode step is captured and replayed
  const char* launch = getenv("QE_LAUNCH");
  kv->eager = launch && strcmp(launch, "eager") == 0;
  kv->events.resize(4);
  for (auto& ev : kv->events) HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  if (kv->eager) {
    *out = kv.release();
    return QE_OK;
  }
  // capture every attention shape up front when there are few (caches up to ~60 K positions);
  // larger caches capture the rest as decoding first reaches them
  std::vector<std::pair<uint32_t, uint32_t>> shapes;
  for (uint64_t pos = 0; pos < max_seq && shapes.size() <= 64;) {
    uint32_t splits, run;
    step_shape(kv.get(), pos, splits, run);
    if (shapes.empty() || shapes.back() != std::make_pair(splits, run)) shapes.push_back({splits, run});
    // the next position whose shape can differ: the end of this run length's range (runs merged
    // in o_proj), else the next multiple of 64 (wide runs change their count every 8 runs and
    // their length every 64 kAttnMaxWideSplits positions)
    const bool wide = splits > uint32_t(qe::kAttnMaxMergeSplits);
    pos = run == 64 || wide || model->fused ? (pos / 64 + 1) * 64 : uint64_t(run) * kv->attn_splits;
  }
  if (shapes.size() <= 64) {
    for (const auto& sh : shapes) {
      int rc = capture_step(model, kv.get(), sh.first, sh.second);
      if (rc) return rc;
    }
  }
  *out = kv.release();
  return QE_OK;
}

void qe_kv_free(qe_kv* kv) { delete kv; }
uint64_t qe_kv_max_seq(const qe_kv* kv) { return kv ? kv->max_seq : 0; }
uint64_t qe_kv_len(const qe_kv* kv) { return kv ? kv->len : 0; }

int qe_forward(qe_model* model, uint32_t token, uint64_t pos, qe_kv* kv, float* logits_out) {
  if (!model || !kv || !logits_out) return fail(QE_ERR_ARG, "null argument");
  if (kv->model != model) return fail(QE_ERR_ARG, "cache belongs to another model");
  if (pos >= kv->max_seq) return fail(QE_ERR_POS, "pos %llu exceeds KV cache size %llu", (unsigned long long)pos, (unsigned long long)kv->max_seq);
  if (pos > kv->len) return fail(QE_ERR_POS, "pos %llu is past the %llu cached positions", (unsigned long long)pos, (unsigned long long)kv->len);
  if (token >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "token %u >= vocab %llu", token, (unsigned long long)model->cfg.vocab_size);
  int rc = set_state(model, kv, token, pos);
  if (rc) return rc;
  if ((rc = launch_step(model, kv, pos))) return rc;
  const size_t V = model->cfg.vocab_size;
  HIP_TRY(hipMemcpyAsync(model->h_logits, model->logits, V * 4, hipMemcpyDeviceToHost, model->stream));
  if ((rc = check_err(model))) return rc;
  memcpy(logits_out, model->h_logits, V * 4);
  kv->len = pos + 1;
  return QE_OK;
}

int qe_profile_step(qe_model* model, uint32_t token, uint64_t pos, qe_kv* kv, float* us_out, uint32_t* launches_out,
                    const char** names_out, uint32_t max_stages, uint32_t* n_out) {
  if (!model || !kv || !us_out || !n_out) return fail(QE_ERR_ARG, "null argument");
  if (kv->model != model) return fail(QE_ERR_ARG, "cache belongs to another model");
  if (pos >= kv->max_seq) return fail(QE_ERR_POS, "pos %llu exceeds KV cache size %llu", (unsigned long long)pos, (unsigned long long)kv->max_seq);
  if (pos > kv->len) return fail(QE_ERR_POS, "pos %llu is past the %llu cached positions", (unsigned long long)pos, (unsigned long long)kv->len);
  if (token >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "token %u >= vocab", token);
  // the full step first, so that every stage reads the activations of a real step
  int rc = set_state(model, kv, token, pos);
  if (rc) return rc;
  if ((rc = launch_step(model, kv, pos))) return rc;
  if ((rc = check_err(model))) return rc;
  kv->len = pos + 1;
  // then each stage alone: a graph of its launches (28 per-layer launches, or the one lm_head /
  // argmax), replayed kReps times between two events. Every stage starts from the step state of
  // `pos` (set_state), so its replays run at that position as the step did; the argmax replays
  // each advance the token ring by one, which a cache of fewer than kReps + 2 positions cannot
  // hold, so such a cache skips the argmax stage.
  // Each stage alone, then the step's prefixes (each adding the next stage, as the step orders
  // them) up to the lm_head, whose differences are the stages' in-step costs. The argmax, the
  // step's last launch, is not in a prefix: it advances the step state, which the attention
  // launches of a replayed prefix would then follow past the captured position.
  static const char* const kStageList[] = {"qkv",
                                           "attention",
                                           "qkv+attention",
                                           "o_proj",
                                           "gate_up",
                                           "down",
                                           "lm_head",
                                           "argmax",
                                           "qkv+attention+o_proj",
                                           "qkv+attention+o_proj+gate_up",
                                           "qkv+attention+o_proj+gate_up+down",
                                           "qkv+attention+o_proj+gate_up+down+lm_head",
                                           nullptr};
  // the two-launch layers (fused.hip): per layer an attention block and an MLP block
  static const char* const kFusedStageList[] = {"attn_block",
                                                "mlp_block",
                                                "final_reduce",
                                                "lm_head",
                                                "argmax",
                                                "attn_block+mlp_block",
                                                "attn_block+mlp_block+final_reduce",
                                                "attn_block+mlp_block+final_reduce+lm_head",
                                                nullptr};
  // one persistent launch for all layers (persist.hip)
  static const char* const kPersistStageList[] = {"layers", "lm_head", "argmax", "layers+lm_head", nullptr};
  // and last the whole step ("step"): the argmax's cost in the step is the step minus the prefix
  // that ends with the lm_head (it advances the step state, so it cannot end a shorter prefix)
  std::vector<const char*> kStages;
  for (const char* const* st = model->fused == 2 ? kPersistStageList : model->fused ? kFusedStageList : kStageList; *st;
       st++)
    kStages.push_back(*st);
  kStages.push_back("step");
  constexpr int kReps = 8;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  HIP_TRY(hipEventCreate(&e0));
  hipError_t he = hipEventCreate(&e1);
  uint32_t n = 0;
  for (const char* stage : kStages) {
    if (he != hipSuccess || rc != QE_OK) break;
    const bool full = strcmp(stage, "step") == 0;
    if ((full || strcmp(stage, "argmax") == 0) && kv->tok_cap < uint32_t(kReps + 3)) continue;
    if (full) {
      // its replays run the captured attention shape at positions pos .. pos + kReps
      uint32_t s0, r0, s1, r1;
      step_shape(kv, pos, s0, r0);
      step_shape(kv, std::min<uint64_t>(pos + kReps, kv->max_seq - 1), s1, r1);
      if (s0 != s1 || r0 != r1 || pos + kReps >= kv->max_seq) continue;
    }
    if ((rc = set_state(model, kv, token, pos)) != QE_OK) break;
    uint32_t launches = 0;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    if ((he = hipStreamBeginCapture(model->stream, hipStreamCaptureModeThreadLocal)) != hipSuccess) break;
    rc = enqueue_step(model, kv, full ? nullptr : stage, &launches);
    he = hipStreamEndCapture(model->stream, &g);
    if (rc == QE_OK && he == hipSuccess && launches > 0) {
      he = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
      if (he == hipSuccess) he = hipGraphLaunch(ge, model->stream);  // warm-up replay
      if (he == hipSuccess) he = hipEventRecord(e0, model->stream);
      for (int r = 0; r < kReps && he == hipSuccess; r++) he = hipGraphLaunch(ge, model->stream);
      if (he == hipSuccess) he = hipEventRecord(e1, model->stream);
      if (he == hipSuccess) he = hipEventSynchronize(e1);
      float ms = 0.f;
      if (he == hipSuccess) he = hipEventElapsedTime(&ms, e0, e1);
      if (he == hipSuccess && n < max_stages) {
        us_out[n] = ms * 1e3f / float(kReps * launches);
        if (launches_out) launches_out[n] = launches;
        if (names_out) names_out[n] = stage;
      }
      if (he == hipSuccess) n++;
    }
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
  }
  (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (rc != QE_OK) return rc;
  if (he != hipSuccess) return fail(QE_ERR_HIP, "stage timing failed: %s", hipGetErrorString(he));
  // Last, the two-launch layers' launches inside the whole step: a graph of the step whose layer
  // launches are the clock-stamping compilation of the same kernels (FusedLayerParams::ts),
  // replayed kReps times at pos .. pos + kReps - 1 (one attention shape, as for "step"). Per
  // stage: "in_step:<stage>", a launch's share of the step, from its first workgroup's start to
  // the next layer launch's first start (dispatch and drain included, as a kernel trace counts
  // them; the step's last launch has no successor and is left out), and "in_exec:<stage>", its
  // first workgroup's start to its last workgroup's exit.
  uint32_t s0, r0, s1, r1;
  step_shape(kv, pos, s0, r0);
  step_shape(kv, std::min<uint64_t>(pos + kReps, kv->max_seq - 1), s1, r1);
  if (model->fused == 1 && s0 == s1 && r0 == r1 && pos + kReps < kv->max_seq && kv->tok_cap >= uint32_t(kReps + 3)) {
    const uint32_t cap = 2 * uint32_t(model->cfg.num_hidden_layers);
    std::vector<const char*> ts_stage(cap, nullptr);
    std::vector<uint64_t> host(size_t(cap) * kTsPerLaunch);
    uint64_t* dts = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipError_t me = hipMalloc(&dts, host.size() * 8);
    int mrc = QE_OK;
    if (me == hipSuccess) me = hipMemsetAsync(dts, 0, host.size() * 8, model->stream);
    if (me == hipSuccess) mrc = set_state(model, kv, token, pos);
    if (me == hipSuccess && mrc == QE_OK) {
      model->ts_buf = dts;
      model->ts_stage = ts_stage.data();
      model->n_ts = 0;
      model->ts_cap = cap;
      me = hipStreamBeginCapture(model->stream, hipStreamCaptureModeThreadLocal);
      if (me == hipSuccess) {
        mrc = enqueue_step(model, kv);
        const hipError_t ce = hipStreamEndCapture(model->stream, &g);
        if (me == hipSuccess) me = ce;
      }
      model->ts_buf = nullptr;
      model->ts_stage = nullptr;
    }
    const uint32_t nl = model->n_ts;
    model->n_ts = 0;
    double sum[2][2] = {{0.0, 0.0}, {0.0, 0.0}};  // [share, window][attn, mlp]
    uint32_t cnt[2][2] = {{0, 0}, {0, 0}};
    if (me == hipSuccess && mrc == QE_OK && nl > 0) me = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (me == hipSuccess && mrc == QE_OK && nl > 0) {
      me = hipGraphLaunch(ge, model->stream);  // warm-up replay
      const uint32_t nwg = qe::kFusedXcds * qe::kFusedSlots;  // the stamping workgroups
      for (int r = 0; r < kReps && me == hipSuccess; r++) {
        me = hipGraphLaunch(ge, model->stream);
        if (me == hipSuccess) me = hipMemcpyAsync(host.data(), dts, size_t(nl) * kTsPerLaunch * 8, hipMemcpyDeviceToHost, model->stream);
        if (me == hipSuccess) me = hipStreamSynchronize(model->stream);
        std::vector<uint64_t> first(nl, UINT64_MAX), last(nl, 0);
        for (uint32_t i = 0; i < nl && me == hipSuccess; i++) {
          const uint64_t* t = host.data() + size_t(i) * kTsPerLaunch;
          for (uint32_t b = 0; b < nwg; b++) {
            first[i] = std::min(first[i], t[2 * b]);
            last[i] = std::max(last[i], t[2 * b + 1]);
          }
        }
        for (uint32_t i = 0; i < nl && me == hipSuccess; i++) {
          const int k = strcmp(ts_stage[i], "attn_block") == 0 ? 0 : 1;
          if (i + 1 < nl && first[i + 1] > first[i]) {
            sum[0][k] += double(first[i + 1] - first[i]) * 0.01;  // 100 MHz clock: 10 ns per tick
            cnt[0][k]++;
          }
          if (last[i] > first[i]) {
            sum[1][k] += double(last[i] - first[i]) * 0.01;
            cnt[1][k]++;
          }
        }
      }
    }
    static const char* const kInStep[2][2] = {{"in_step:attn_block", "in_step:mlp_block"},
                                              {"in_exec:attn_block", "in_exec:mlp_block"}};
    for (int w = 0; w < 2; w++)
      for (int k = 0; k < 2 && me == hipSuccess && mrc == QE_OK; k++) {
        if (cnt[w][k] && n < max_stages) {
          us_out[n] = float(sum[w][k] / cnt[w][k]);
          if (launches_out) launches_out[n] = cnt[w][k] / kReps;
          if (names_out) names_out[n] = kInStep[w][k];
          n++;
        }
      }
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    (void)hipStreamSynchronize(model->stream);
    if (dts) (void)hipFree(dts);
    if (mrc != QE_OK) return mrc;
    if (me != hipSuccess) return fail(QE_ERR_HIP, "in-step timing failed: %s", hipGetErrorString(me));
  }
  // a kernel error raised by any of the replays is reported like one of a step
  if ((rc = check_err(model))) return rc;
  // the stage replays ran on the activations the step left behind, so the K/V they wrote at pos
  // are not the step's: run the step once more, which leaves the cache as qe_forward would
  if ((rc = set_state(model, kv, token, pos))) return rc;
  if ((rc = launch_step(model, kv, pos))) return rc;
  if ((rc = check_err(model))) return rc;
  *n_out = n;
  return QE_OK;
}

int qe_prefill(qe_model* model, const uint32_t* ids, uint64_t n, uint64_t start_pos, qe_kv* kv, float* last_logits) {
  if (!model || !kv || (!ids && n)) return fail(QE_ERR_ARG, "null argument");
  if (kv->model != model) return fail(QE_ERR_ARG, "cache belongs to another model");
  if (n == 0) return QE_OK;
  if (start_pos > kv->len) return fail(QE_ERR_POS, "start_pos %llu is past the %llu cached positions", (unsigned long long)start_pos, (unsigned long long)kv->len);
  if (start_pos + n > kv->max_seq) return fail(QE_ERR_POS, "prompt end %llu exceeds KV cache size %llu", (unsigned long long)(start_pos + n), (unsigned long long)kv->max_seq);
  for (uint64_t i = 0; i < n; i++)
    if (ids[i] >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "token %u at %llu >= vocab", ids[i], (unsigned long long)i);
  // each step reads tokens[tok_idx]; stage the whole prompt into the ring in one copy, then
  // replay the step n times (the argmax write to tokens[k+1] is overwritten by the next id)
  int rc = set_state(model, kv, ids[0], start_pos);
  if (rc) return rc;
  for (uint64_t i = 0; i < n; i++) {
    if (i > 0) {
      // overwrite the slot the previous step's argmax wrote with the next prompt id
      HIP_TRY(hipMemcpyAsync(kv->tokens + i, ids + i, 4, hipMemcpyHostToDevice, model->stream));
    }
    if ((rc = launch_step(model, kv, start_pos + i))) return rc;
  }
  if (last_logits) {
    HIP_TRY(hipMemcpyAsync(model->h_logits, model->logits, model->cfg.vocab_size * 4, hipMemcpyDeviceToHost, model->stream));
  }
  if ((rc = check_err(model))) return rc;
  if (last_logits) memcpy(last_logits, model->h_logits, model->cfg.vocab_size * 4);
  kv->len = start_pos + n;
  return QE_OK;
}

int qe_prefill_batch(qe_model* model, const uint32_t* ids, uint64_t n, uint64_t start_pos, qe_kv* kv, uint32_t chunk,
                     float* last_logits) {
  if (!model || !kv || (!ids && n)) return fail(QE_ERR_ARG, "null argument");
  if (kv->model != model) return fail(QE_ERR_ARG, "cache belongs to another model");
  if (n == 0) return QE_OK;
  if (chunk == 0) chunk = kBatchDefaultChunk;
  if (chunk > kBatchMaxChunk) return fail(QE_ERR_ARG, "chunk %u above %u", chunk, kBatchMaxChunk);
  if (start_pos > kv->len) return fail(QE_ERR_POS, "start_pos %llu is past the %llu cached positions", (unsigned long long)start_pos, (unsigned long long)kv->len);
  if (start_pos + n > kv->max_seq) return fail(QE_ERR_POS, "prompt end %llu exceeds KV cache size %llu", (unsigned long long)(start_pos + n), (unsigned long long)kv->max_seq);
  for (uint64_t i = 0; i < n; i++)
    if (ids[i] >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "token %u at %llu >= vocab", ids[i], (unsigned long long)i);
  int rc = ensure_batch(model, chunk, 0);
  if (rc) return rc;
  // chunks of more than kGemmSkinnyMaxM tokens go round-robin over up to prefill_streams streams
  // and buffer sets: chunk i's layer-l attention waits for chunk i-1's layer-l K/V rows, and
  // otherwise the chunks' launches overlap (each chunk runs the same kernels as on one stream)
  const uint64_t n_chunks = (n + chunk - 1) / chunk;
  const int S = chunk > qe::kGemmSkinnyMaxM ? int(std::min<uint64_t>(model->prefill_streams, n_chunks)) : 1;
  if (S > 1 && (rc = ensure_streams(model, chunk, S))) return rc;
  if ((rc = upload_ids(model, ids, n))) return rc;
  auto stream_of = [&](int set) { return set ? model->extra[set - 1].stream : model->stream; };
  auto events_of = [&](int set) { return set ? model->extra[set - 1].kv_ev.data() : model->kv_ev0.data(); };
  if (S > 1) {  // the extra streams start after everything queued so far (ids, earlier steps)
    HIP_TRY(hipEventRecord(model->start_ev, model->stream));
    for (int j = 1; j < S; j++) HIP_TRY(hipStreamWaitEvent(stream_of(j), model->start_ev, 0));
  }
  int last_set = 0;
  for (uint64_t done = 0, i = 0; done < n; i++) {
    const uint32_t M = uint32_t(std::min<uint64_t>(chunk, n - done));
    const BatchLogits lg = done + M == n && last_logits ? kLastLogits : kNoLogits;
    const int set = int(i % uint64_t(S));
    ChunkStream cs{set, nullptr, nullptr};
    if (S > 1) {
      cs.kv_done = events_of(set);
      cs.wait_kv = i > 0 ? events_of(int((i - 1) % uint64_t(S))) : nullptr;
    }
    last_set = set;
    if ((rc = enqueue_batch(model, kv, M, uint32_t(start_pos + done), model->ids_dev + done, lg, nullptr,
                            S > 1 ? &cs : nullptr))) {
      // nothing queued may outlive the call (the caller may free the cache next)
      for (int j = 0; j < S; j++) (void)hipStreamSynchronize(stream_of(j));
      return rc;
    }
    done += M;
  }
  for (int j = 1; j < S; j++) HIP_TRY(hipStreamSynchronize(stream_of(j)));
  if (last_logits) {
    HIP_TRY(hipMemcpyAsync(model->h_logits, model->logits, model->cfg.vocab_size * 4, hipMemcpyDeviceToHost,
                           stream_of(last_set)));
    HIP_TRY(hipStreamSynchronize(stream_of(last_set)));
  }
  HIP_TRY(hipStreamSynchronize(model->stream));
  if (last_logits) memcpy(last_logits, model->h_logits, model->cfg.vocab_size * 4);
  kv->len = start_pos + n;
  return QE_OK;
}

namespace {

int check_verify_args(qe_model* model, const uint32_t* ids, uint64_t k, uint64_t start_pos, qe_kv* kv) {
  if (!model || !kv || !ids) return fail(QE_ERR_ARG, "null argument");
  if (kv->model != model) return fail(QE_ERR_ARG, "cache belongs to another model");
  if (k == 0 || k > kVerifyMaxTokens) return fail(QE_ERR_ARG, "k must be 1..%u", kVerifyMaxTokens);
  if (start_pos > kv->len) return fail(QE_ERR_POS, "start_pos %llu is past the %llu cached positions", (unsigned long long)start_pos, (unsigned long long)kv->len);
  if (start_pos + k > kv->max_seq) return fail(QE_ERR_POS, "verify end %llu exceeds KV cache size %llu", (unsigned long long)(start_pos + k), (unsigned long long)kv->max_seq);
  for (uint64_t i = 0; i < k; i++)
    if (ids[i] >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "token %u at %llu >= vocab", ids[i], (unsigned long long)i);
  return QE_OK;
}

constexpr int kNotFused = -1;
constexpr uint32_t kTokPending = 0xFFFFFFFFu;  // a pinned token slot not yet written

// A two-row verify pass (positions pos, pos + 1) through the two launches per layer, every weight
// read once for both rows; the lm_head over both rows and the device argmax of each row follow.
// kNotFused when the pass's attention needs more than 16 runs (the batch path takes it).
// tokens: the greedy token of each row, or null; logits_out: host [R][V] logits, or null.
int verify_fused(qe_model* m, const uint32_t* ids, uint32_t R, uint64_t pos, qe_kv* kv, uint32_t* tokens,
                 float* logits_out) {
  uint32_t splits, run;
  step_shape(kv, pos + R - 1, splits, run);  // the runs cover positions 0 .. pos + R - 1
  if (R != qe::kFusedMaxRows || splits > 16) return kNotFused;
  const qe_config& c = m->cfg;
  const size_t V = c.vocab_size;
  // the staging words are free once the previous pass's copy of them is done
  if (!m->vstage_ev) HIP_TRY(hipEventCreateWithFlags(&m->vstage_ev, hipEventDisableTiming));
  else HIP_TRY(hipEventSynchronize(m->vstage_ev));
  const StepState st{uint32_t(pos), 0u, uint32_t(kv->max_seq), R};
  memcpy(m->h_small + 16, &st, sizeof(st));
  std::copy(ids, ids + R, m->h_small + 20);
  HIP_TRY(hipMemcpyAsync(m->vstate, m->h_small + 16, sizeof(st) + R * 4, hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipEventRecord(m->vstage_ev, m->stream));
  // the pass: the layers, the lm_head over both rows, each row's argmax into pinned memory
  uint32_t* host_tok = reinterpret_cast<uint32_t*>(m->h_logits);
  auto enqueue = [&]() -> int {
    const uint32_t ks = kv->step_splits, kr = kv->step_run;
    kv->step_splits = splits;
    kv->step_run = run;
    int rc = enqueue_step_fused(m, kv, nullptr, nullptr, R);
    kv->step_splits = ks;
    kv->step_run = kr;
    if (rc) return rc;
    // (x comes normalized from the final reduce); each workgroup's candidates, then one
    // reduction per row
    qe::MvRowsParams r{m->lm_head, m->x, nullptr, m->blogits, R, uint32_t(V), uint32_t(c.hidden_size),
                       uint32_t(V), c.rms_norm_eps};
    r.cand = m->vcand;
    HIP_TRY(qe::launch_lm_head_rows(r, m->stream));
    HIP_TRY(qe::launch_cand_argmax(m->vcand, qe::lm_head_rows_workgroups(uint32_t(V)), m->blogits, R, uint32_t(V),
                                   host_tok, m->stream, m->err, host_tok + R));
    return QE_OK;
  };
  // the host waits for the tokens and the error word in pinned memory (every slot pending first)
  // instead of synchronizing the stream, whose wake-up costs more than a spin on these words
  for (uint32_t r = 0; r <= R; r++) __atomic_store_n(&host_tok[r], kTokPending, __ATOMIC_RELAXED);
  int rc = QE_OK;
  if (kv->eager) {
    if ((rc = enqueue())) return rc;
  } else {
    // one graph per attention shape (the launches are ~60, so a pass replayed from the host
    // would wait on its launch calls)
    qe_kv::VerifyGraph* vg = nullptr;
    for (auto& g : kv->vgraphs)
      if (g.splits == splits && g.run == run && g.logits == m->blogits && g.cand == m->bcand) vg = &g;
    if (!vg) {
      HIP_TRY(hipStreamSynchronize(m->stream));
      HIP_TRY(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
      rc = enqueue();
      hipGraph_t g = nullptr;
      const hipError_t e = hipStreamEndCapture(m->stream, &g);
      if (rc != QE_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
      }
      if (e != hipSuccess) return fail(QE_ERR_HIP, "verify graph capture failed: %s", hipGetErrorString(e));
      hipGraphExec_t ex = nullptr;
      const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
      if (ie != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(QE_ERR_HIP, "verify graph instantiation failed: %s", hipGetErrorString(ie));
      }
      kv->vgraphs.push_back({splits, run, m->blogits, m->bcand, g, ex});
      vg = &kv->vgraphs.back();
    }
    HIP_TRY(hipGraphLaunch(vg->exec, m->stream));
  }
  if (logits_out) {
    HIP_TRY(hipMemcpyAsync(logits_out, m->blogits, size_t(R) * V * 4, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
  } else {
    // spin until every slot is written; a stream that has failed or finished without writing them
    // ends the wait (checked every 4096 spins)
    for (uint32_t spins = 1;; spins++) {
      bool done = true;
      for (uint32_t r = 0; r <= R; r++) done = done && __atomic_load_n(&host_tok[r], __ATOMIC_ACQUIRE) != kTokPending;
      if (done) break;
      if (spins % 4096 == 0 && hipStreamQuery(m->stream) != hipErrorNotReady) {
        HIP_TRY(hipStreamSynchronize(m->stream));
        for (uint32_t r = 0; r <= R; r++)
          if (__atomic_load_n(&host_tok[r], __ATOMIC_ACQUIRE) == kTokPending)
            return fail(QE_ERR_KERNEL, "verify pass ended without its tokens");
        break;
      }
    }
  }
  if (__atomic_load_n(&host_tok[R], __ATOMIC_ACQUIRE) && (rc = check_err(m))) return rc;
  if (tokens) memcpy(tokens, host_tok, size_t(R) * 4);
  kv->len = std::max<uint64_t>(kv->len, pos + R);
  return QE_OK;
}

// verify pass with the argmax on the device: tokens[i] = greedy token of row i
int verify_greedy(qe_model* model, const uint32_t* ids, uint32_t k, uint64_t start_pos, qe_kv* kv, uint32_t* tokens) {
  int rc = ensure_batch(model, k, k);
  if (rc) return rc;
  if (k == qe::kFusedMaxRows && model->fused == 1 && model->verify_fused) {
    rc = verify_fused(model, ids, k, start_pos, kv, tokens, nullptr);
    if (rc != kNotFused) return rc;
  }
  qe::TokenIds tv{};  // k <= kVerifyMaxTokens = kIdsByValue: the ids travel in the kernel argument
  std::copy(ids, ids + k, tv.id);
  if ((rc = enqueue_batch(model, kv, k, uint32_t(start_pos), nullptr, kAllLogits, &tv))) return rc;
  // the greedy tokens go straight to pinned host memory (h_logits is idle here: no decode step
  // is in flight on this stream)
  uint32_t* host_tok = reinterpret_cast<uint32_t*>(model->h_logits);
  HIP_TRY(qe::launch_row_argmax(model->blogits, k, uint32_t(model->cfg.vocab_size), host_tok, model->bcand,
                                model->stream));
  HIP_TRY(hipStreamSynchronize(model->stream));
  memcpy(tokens, host_tok, size_t(k) * 4);
  kv->len = std::max<uint64_t>(kv->len, start_pos + k);
  return QE_OK;
}

// Prompt lookup (Saxena, "Prompt Lookup Decoding", 2023): the draft is what followed an earlier
// occurrence of the history's last g tokens, g from ngram down to 1, at most kd tokens: the most
// recent occurrence followed by kd tokens, else the earliest (whose continuation is the longest);
// empty when no suffix recurs.
void lookup_draft(const std::vector<uint32_t>& h, uint32_t ngram, uint32_t kd, std::vector<uint32_t>& draft) {
  draft.clear();
  const size_t n = h.size();
  if (kd == 0 || n < 2) return;
  for (size_t g = std::min<size_t>(ngram, n - 1); g >= 1; g--) {
    size_t earliest = n;
    for (size_t i = n - g; i-- > 0;) {  // candidate starts, most recent first; i + g <= n - 1
      if (!std::equal(h.begin() + i, h.begin() + i + g, h.end() - g)) continue;
      earliest = i;
      if (i + g + kd <= n) break;  // a full-length continuation
    }
    if (earliest < n) {
      const size_t from = earliest + g, to = std::min(n, from + kd);
      draft.assign(h.begin() + from, h.begin() + to);
      return;
    }
  }
}

}  // namespace

int qe_verify(qe_model* model, const uint32_t* ids, uint64_t k, uint64_t start_pos, qe_kv* kv, float* logits_out) {
  if (!logits_out) return fail(QE_ERR_ARG, "null argument");
  if (int rc = check_verify_args(model, ids, k, start_pos, kv)) return rc;
  int rc = ensure_batch(model, uint32_t(k), uint32_t(k));
  if (rc) return rc;
  if (k == qe::kFusedMaxRows && model->fused == 1 && model->verify_fused) {
    rc = verify_fused(model, ids, uint32_t(k), start_pos, kv, nullptr, logits_out);
    if (rc != kNotFused) return rc;
  }
  qe::TokenIds tv{};
  std::copy(ids, ids + k, tv.id);
  if ((rc = enqueue_batch(model, kv, uint32_t(k), uint32_t(start_pos), nullptr, kAllLogits, &tv))) return rc;
  HIP_TRY(hipMemcpyAsync(logits_out, model->blogits, size_t(k) * model->cfg.vocab_size * 4, hipMemcpyDeviceToHost,
                         model->stream));
  HIP_TRY(hipStreamSynchronize(model->stream));
  kv->len = std::max<uint64_t>(kv->len, start_pos + k);
  return QE_OK;
}

uint64_t qe_lookup_draft(const uint32_t* history, uint64_t n, uint32_t ngram, uint32_t k_max, uint32_t* draft_out) {
  if (!history || !draft_out) return 0;
  std::vector<uint32_t> h(history, history + n), d;
  lookup_draft(h, ngram, k_max, d);
  std::copy(d.begin(), d.end(), draft_out);
  return d.size();
}

int qe_verify_greedy(qe_model* model, const uint32_t* ids, uint64_t k, uint64_t start_pos, qe_kv* kv,
                     uint32_t* tokens_out) {
  if (!tokens_out) return fail(QE_ERR_ARG, "null argument");
  if (int rc = check_verify_args(model, ids, k, start_pos, kv)) return rc;
  return verify_greedy(model, ids, uint32_t(k), start_pos, kv, tokens_out);
}

}  // extern "C"

namespace {

// The speculative loop of qe_decode_lookup / qe_decode_drafted. Each pass asks `draft` for up to
// k tokens after the history and checks them with one verify pass (accepted while they equal the
// greedy token of the row before, plus that pass's own token); with no draft it takes one decode
// step. Adaptive: the host times the passes as they run (their mean seconds and tokens so far).
// Once kAdaptMinPasses passes average under kAdaptMarginal tokens, one pipelined block of plain
// decode steps is timed as well, unless the model holds such a timing from within
// kAdaptStepReuse positions of this one; from then on, while even the passes' optimistic rate (mean
// tokens plus one standard error, over their mean seconds) is below the plain steps' rate, the
// loop decodes plain blocks of kAdaptBlock steps and tries one pass after each. The tokens are
// the greedy ones whatever the loop does.
constexpr double kAdaptMarginal = 2.0;
constexpr uint64_t kAdaptBlock = 16;
constexpr int kAdaptMinPasses = 6;
constexpr uint64_t kAdaptStepReuse = 1024;

template <class Draft>
int decode_drafted(qe_model* model, const uint32_t* context, uint64_t n_context, uint32_t first, uint64_t start_pos,
                   uint64_t steps, qe_kv* kv, uint32_t k_max, Draft&& draft, bool adaptive, qe_on_token on_token,
                   void* user, qe_lookup_stats* stats) {
  if (!model || !kv || (!context && n_context)) return fail(QE_ERR_ARG, "null argument");
  if (kv->model != model) return fail(QE_ERR_ARG, "cache belongs to another model");
  if (k_max == 0 || k_max >= kVerifyMaxTokens) return fail(QE_ERR_ARG, "k_max must be 1..%u", kVerifyMaxTokens - 1);
  if (start_pos > kv->len) return fail(QE_ERR_POS, "start_pos %llu is past the %llu cached positions", (unsigned long long)start_pos, (unsigned long long)kv->len);
  if (start_pos + steps > kv->max_seq) return fail(QE_ERR_POS, "decode end %llu exceeds KV cache size %llu", (unsigned long long)(start_pos + steps), (unsigned long long)kv->max_seq);
  if (first >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "token %u >= vocab", first);
  for (uint64_t i = 0; i < n_context; i++)
    if (context[i] >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "context token %u at %llu >= vocab", context[i], (unsigned long long)i);
  using clock = std::chrono::steady_clock;
  auto secs = [](clock::time_point a, clock::time_point b) { return std::chrono::duration<double>(b - a).count(); };
  qe_lookup_stats st{};
  std::vector<uint32_t> h(context, context + n_context), d(kVerifyMaxTokens), ids, got(kVerifyMaxTokens), blk;
  h.push_back(first);
  uint32_t cur = first;
  uint64_t pos = start_pos, emitted = 0;
  // sums over the timed passes (seconds, tokens, tokens^2); the mean seconds of a plain step
  double sum_s = 0, sum_tok = 0, sum_tok2 = 0, step_s = 0;
  int passes_seen = 0;
  if (adaptive && model->plain_step_s > 0 &&
      std::max(start_pos, model->plain_step_pos) - std::min(start_pos, model->plain_step_pos) <= kAdaptStepReuse)
    step_s = model->plain_step_s;
  bool plain = false;  // the next iteration decodes a plain block
  auto emit = [&](uint32_t tok) {
    h.push_back(tok);
    if (on_token) on_token(user, tok);
  };
  int rc;
  while (emitted < steps) {
    if (plain) {
      const uint64_t nb = std::min(kAdaptBlock, steps - emitted);
      blk.clear();
      auto keep = [](void* u, uint32_t t) { static_cast<std::vector<uint32_t>*>(u)->push_back(t); };
      const auto t0 = clock::now();
      if ((rc = qe_decode(model, cur, pos, nb, kv, keep, &blk, nullptr))) return rc;
      const double per = secs(t0, clock::now()) / double(nb);
      step_s = step_s > 0 ? 0.5 * (step_s + per) : per;
      model->plain_step_s = step_s;
      model->plain_step_pos = pos;
      for (uint32_t t : blk) emit(t);
      st.plain_steps += nb;
      cur = blk.back();
      pos += nb;
      emitted += nb;
      plain = false;  // then one pass, which decides again
      continue;
    }
    // a pass emits accepted drafts + 1 token, so it never runs past `steps`
    const uint32_t kk = uint32_t(std::min<uint64_t>(k_max, steps - emitted - 1));
    const uint32_t nr = kk ? draft(h, kk, d.data()) : 0u;
    if (nr == QE_DRAFT_ERROR) {
      kv->len = pos;  // positions before pos hold the emitted sequence; the next one is cur's
      return fail(QE_ERR_ARG, "the draft function reported an error after %llu tokens", (unsigned long long)emitted);
    }
    const uint32_t nd = std::min(nr, kk);
    if (nd == 0) {  // nothing to verify: one decode step
      uint32_t tok = 0;
      auto keep = [](void* u, uint32_t t) { *static_cast<uint32_t*>(u) = t; };
      if ((rc = qe_decode(model, cur, pos, 1, kv, keep, &tok, nullptr))) return rc;
      st.single_steps++;
      emit(tok);
      cur = tok;
      pos++;
      emitted++;
      continue;
    }
    for (uint32_t i = 0; i < nd; i++)
      if (d[i] >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "draft token %u >= vocab", d[i]);
    ids.assign(1, cur);
    ids.insert(ids.end(), d.begin(), d.begin() + nd);
    const auto t0 = clock::now();
    if ((rc = verify_greedy(model, ids.data(), uint32_t(ids.size()), pos, kv, got.data()))) return rc;
    // row i is the greedy token after ids[i]: drafts are accepted while they equal it, and the
    // row after the last accepted one adds a token of its own
    uint32_t j = 0;
    while (j < nd && got[j] == d[j]) j++;
    st.passes++;
    st.drafted += nd;
    st.accepted += j;
    for (uint32_t i = 0; i <= j; i++) emit(i < j ? d[i] : got[j]);
    cur = got[j];
    pos += j + 1;
    emitted += j + 1;
    if (adaptive) {
      sum_s += secs(t0, clock::now());
      sum_tok += double(j + 1);
      sum_tok2 += double(j + 1) * double(j + 1);
      if (++passes_seen >= kAdaptMinPasses) {
        const double n = passes_seen, mean = sum_tok / n;
        if (step_s > 0) {
          const double upper = mean + std::sqrt(std::max(0.0, sum_tok2 / n - mean * mean) / n);
          plain = upper / (sum_s / n) < 1.0 / step_s;
        } else {
          plain = mean < kAdaptMarginal;  // time a plain block to compare
        }
      }
    }
  }
  kv->len = start_pos + steps;  // positions past the accepted tokens hold rejected drafts
  if (stats) *stats = st;
  return QE_OK;
}

}  // namespace

extern "C" {

int qe_decode_lookup(qe_model* model, const uint32_t* context, uint64_t n_context, uint32_t first, uint64_t start_pos,
                     uint64_t steps, qe_kv* kv, uint32_t k_max, uint32_t ngram, qe_on_token on_token, void* user,
                     qe_lookup_stats* stats) {
  if (ngram == 0) return fail(QE_ERR_ARG, "ngram must be >= 1");
  std::vector<uint32_t> tmp;
  auto lookup = [&](const std::vector<uint32_t>& h, uint32_t k, uint32_t* out) -> uint32_t {
    lookup_draft(h, ngram, k, tmp);
    std::copy(tmp.begin(), tmp.end(), out);
    return uint32_t(tmp.size());
  };
  return decode_drafted(model, context, n_context, first, start_pos, steps, kv, k_max, lookup,
                        model && model->lookup_adaptive, on_token, user, stats);
}

int qe_decode_drafted(qe_model* model, const uint32_t* context, uint64_t n_context, uint32_t first, uint64_t start_pos,
                      uint64_t steps, qe_kv* kv, uint32_t k_max, qe_draft_fn draft, void* draft_user, int adaptive,
                      qe_on_token on_token, void* user, qe_lookup_stats* stats) {
  if (!draft) return fail(QE_ERR_ARG, "null draft function");
  auto source = [&](const std::vector<uint32_t>& h, uint32_t k, uint32_t* out) -> uint32_t {
    return draft(draft_user, h.data(), h.size(), k, out);
  };
  return decode_drafted(model, context, n_context, first, start_pos, steps, kv, k_max, source, adaptive != 0,
                        on_token, user, stats);
}

int qe_decode(qe_model* model, uint32_t first, uint64_t start_pos, uint64_t steps, qe_kv* kv, qe_on_token on_token,
              void* user, float* logits_per_step) {
  if (!model || !kv) return fail(QE_ERR_ARG, "null argument");
  if (kv->model != model) return fail(QE_ERR_ARG, "cache belongs to another model");
  if (steps == 0) return QE_OK;
  if (start_pos > kv->len) return fail(QE_ERR_POS, "start_pos %llu is past the %llu cached positions", (unsigned long long)start_pos, (unsigned long long)kv->len);
  if (start_pos + steps > kv->max_seq) return fail(QE_ERR_POS, "decode end %llu exceeds KV cache size %llu", (unsigned long long)(start_pos + steps), (unsigned long long)kv->max_seq);
  if (first >= model->cfg.vocab_size) return fail(QE_ERR_ARG, "token %u >= vocab", first);
  int rc = set_state(model, kv, first, start_pos);
  if (rc) return rc;
  const size_t V = model->cfg.vocab_size;
  const size_t nev = kv->events.size();
  // step i runs while the host waits for step i-1 (metal_inference.rs:297-316)
  for (uint64_t i = 0; i <= steps; i++) {
    if (i < steps) {
      if (i >= nev) HIP_TRY(hipEventSynchronize(kv->events[i % nev]));  // ring slot free
      if ((rc = launch_step(model, kv, start_pos + i))) return rc;
      if (logits_per_step) {
        HIP_TRY(hipMemcpyAsync(model->h_logits, model->logits, V * 4, hipMemcpyDeviceToHost, model->stream));
      }
      HIP_TRY(hipEventRecord(kv->events[i % nev], model->stream));
      if (logits_per_step) {
        HIP_TRY(hipEventSynchronize(kv->events[i % nev]));
        memcpy(logits_per_step + i * V, model->h_logits, V * 4);
      }
    }
    if (i >= 1) {
      HIP_TRY(hipEventSynchronize(kv->events[(i - 1) % nev]));
      if (on_token) on_token(user, __atomic_load_n(&kv->host_tokens[i], __ATOMIC_ACQUIRE));
    }
  }
  if ((rc = check_err(model))) return rc;
  kv->len = start_pos + steps;
  return QE_OK;
}

// ---- synthetic inputs ----
int qe_write_random_checkpoint(const char* dir, uint64_t seed, const qe_config* cfg) {
  if (!dir || !cfg) return fail(QE_ERR_ARG, "null argument");
  std::string err;
  int rc = qe::write_random_checkpoint(dir, seed, *cfg, err);
  if (rc) return fail(rc, "%s", err.c_str());
  return QE_OK;
}

void qe_random_prompt(uint64_t seed, uint64_t n, uint32_t vocab, uint32_t* out) {
  if (out && vocab) qe::random_prompt(seed, n, vocab, out);
}

// ---- isolated ops ----
int qe_op_matvec_bf16(const void* w, const float* x, float* out, uint64_t rows, uint64_t cols, void* stream) {
  if (!w || !x || !out) return fail(QE_ERR_ARG, "null argument");
  if (cols % 8 || rows == 0 || cols == 0 || rows > 0xFFFFFFFFull || cols > 0xFFFFFFFFull)
    return fail(QE_ERR_ARG, "rows must be > 0 and cols a positive multiple of 8");
  if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(x) % 16)
    return fail(QE_ERR_ARG, "w and x must be 16-byte aligned");
  MatvecParams p{};
  p.w = static_cast<const uint16_t*>(w); p.x = x; p.rows = uint32_t(rows); p.cols = uint32_t(cols); p.out = out;
  // the kernel the engine uses for this shape: per-layer projections take the wide layout,
  // vocabulary-sized matrices (the lm_head) the LDS-staged one
  const bool wide = cols / 8 <= 512 && rows <= 16384;
  HIP_TRY(wide ? qe::launch_matvec_wide(p, qe::kCopy, qe::kStore, static_cast<hipStream_t>(stream))
               : qe::launch_matvec(p, qe::kCopy, qe::kStore, static_cast<hipStream_t>(stream)));
  return QE_OK;
}

int qe_op_gemm_bf16(const float* a, const void* w, float* c, uint64_t m, uint64_t n, uint64_t k, void* stream) {
  if (!a || !w || !c) return fail(QE_ERR_ARG, "null argument");
  if (m == 0 || n == 0 || k == 0 || n % 2 || k % 32 || m > 0xFFFFFFFFull || n > 0xFFFFFFFFull || k > 0xFFFFFFFFull)
    return fail(QE_ERR_ARG, "need m > 0, n even, k a multiple of 32");
  if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w) % 16)
    return fail(QE_ERR_ARG, "a and w must be 16-byte aligned");
  qe::GemmParams g{a, uint32_t(k), nullptr, nullptr, static_cast<const uint16_t*>(w), uint32_t(m), uint32_t(n),
                   uint32_t(k), c, uint32_t(n), 0.f};
  HIP_TRY(qe::launch_gemm(g, false, qe::kGemmStore, static_cast<hipStream_t>(stream)));
  return QE_OK;
}

uint64_t qe_op_attention_work_bytes(uint64_t n_heads, uint64_t n_kv_heads, uint64_t n_pos) {
  (void)n_pos;  // the partials are sized for the most runs, kAttnMaxSplits per KV head
  if (!n_kv_heads || n_heads % n_kv_heads) return 0;
  const uint64_t G = n_heads / n_kv_heads;
  return align_up(n_kv_heads * qe::kAttnMaxSplits * G * qe::kPartStride * 4, 256);
}

int qe_op_attention(const float* q, const float* k, const float* v, float* out, uint64_t n_pos, uint64_t kv_stride,
                    uint64_t n_heads, uint64_t n_kv_heads, uint32_t n_splits, void* work, void* stream) {
  if (!q || !k || !v || !out || !work) return fail(QE_ERR_ARG, "null argument");
  if (n_pos == 0 || n_pos > kv_stride || kv_stride > 0xFFFFFFFFull) return fail(QE_ERR_ARG, "need 0 < n_pos <= kv_stride");
  if (!n_kv_heads || n_heads % n_kv_heads) return fail(QE_ERR_ARG, "n_heads must be a multiple of n_kv_heads");
  const uint64_t G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail(QE_ERR_UNSUPPORTED, "q heads per KV head must be 1, 2, 4 or 8");
  if (n_splits > qe::kAttnMaxSplits) return fail(QE_ERR_ARG, "n_splits above %d", qe::kAttnMaxSplits);
  AttnParams a{};
  a.qkv = q; a.k_cache = const_cast<float*>(k); a.v_cache = const_cast<float*>(v);
  a.partial = static_cast<float*>(work);
  a.n_heads = uint32_t(n_heads); a.n_kv = uint32_t(n_kv_heads); a.max_seq = uint32_t(kv_stride);
  a.scale = 1.0f / sqrtf(float(qe::kHeadDim)); a.n_pos_fixed = uint32_t(n_pos);
  // default: runs of 64 positions (one tile each), at most kAttnMaxSplits of them
  uint64_t splits = n_splits ? n_splits : (n_pos + 63) / 64;
  splits = std::min<uint64_t>(std::max<uint64_t>(splits, 1), qe::kAttnMaxSplits);
  HIP_TRY(qe::launch_attention_op(a, uint32_t(splits), out, static_cast<hipStream_t>(stream)));
  return QE_OK;
}

int qe_op_argmax(const float* logits, uint64_t rows, uint64_t n, uint32_t* tokens_out, void* stream) {
  if (!logits || !tokens_out) return fail(QE_ERR_ARG, "null argument");
  if (rows == 0 || n == 0 || rows > 0x7FFFFFFFull || n > 0x7FFFFFFFull) return fail(QE_ERR_ARG, "need 0 < rows, n < 2^31");
  // candidate scratch from the stream-ordered allocator, in batches of at most 65535 rows
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t batch = std::min<uint64_t>(rows, 65535);
  ArgCand* cand = nullptr;
  HIP_TRY(hipMallocAsync(reinterpret_cast<void**>(&cand), batch * qe::kArgParts * sizeof(ArgCand), st));
  for (uint64_t r0 = 0; r0 < rows; r0 += batch) {
    const uint32_t nr = uint32_t(std::min<uint64_t>(batch, rows - r0));
    const hipError_t e = qe::launch_row_argmax(logits + r0 * n, nr, uint32_t(n), tokens_out + r0, cand, st);
    if (e != hipSuccess) {
      (void)hipFreeAsync(cand, st);
      return fail(QE_ERR_HIP, "row argmax: %s", hipGetErrorString(e));
    }
  }
  HIP_TRY(hipFreeAsync(cand, st));
  return QE_OK;
}

int qe_op_read_sum(const float* src, uint64_t n, float* partial, uint32_t grid, void* stream) {
  if (!src || !partial) return fail(QE_ERR_ARG, "null argument");
  if (n % 4) return fail(QE_ERR_ARG, "n must be a multiple of 4");
  HIP_TRY(qe::launch_read_sum(src, n, partial, grid ? grid : 2048, false, static_cast<hipStream_t>(stream)));
  return QE_OK;
}

int qe_op_read_sum_nt(const float* src, uint64_t n, float* partial, uint32_t grid, void* stream) {
  if (!src || !partial) return fail(QE_ERR_ARG, "null argument");
  if (n % 4) return fail(QE_ERR_ARG, "n must be a multiple of 4");
  HIP_TRY(qe::launch_read_sum(src, n, partial, grid ? grid : 2048, true, static_cast<hipStream_t>(stream)));
  return QE_OK;
}

}  // extern "C"
