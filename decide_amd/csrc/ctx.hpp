// Library-internal state of a dn_ctx and the helpers shared by the C ABI
// translation units (api.cpp: context, weights, forward; train.cpp: training).
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/decide_hip.h"
#include "common.hpp"

struct DevBuf {
  void *p = nullptr;
  size_t cap = 0;
};

// Per-tensor training state, in the slot's stored layout (Wi rows interleaved).
struct ParamTrain {
  DevBuf master;   // fp32 weights when the slot holds bf16 (projections in bf16 mode)
  DevBuf grad, m, v;
  DevBuf wt;       // projections: transposed operand copy [in x out] for the input-gradient GEMMs
  bool wt_valid = false;
};

struct TensorSlot {
  DevBuf buf;
  int64_t n = 0;     // float32 elements expected
  int rank = 1;      // rank of the reference tensor (model.go:51-84)
  bool proj = false; // projection matrix: stored in the operand precision
  bool wi = false;   // Wi: rows interleaved for the GeGLU epilogue
  bool set = false;
  ParamTrain train;  // allocated by the training entry points
};

struct Config {
  int hidden = 0, inter = 0, heads = 0, layers = 0, vocab = 0;
  float eps = 1e-5f;
  int half_window = 64;
  double theta_g = 160000, theta_l = 10000;
  std::vector<uint8_t> sliding;
  int precision = DN_PRECISION_BF16;
  // Geometry outside the MFMA kernels' shapes (head_dim != 64, hidden % 256,
  // intermediate % 64): any-shape GEMM and attention kernels, Wi stored in its
  // natural layout, no training.
  bool generic = false;
  // Small-M GEMMs on 32 x 32 tiles (16-bit): operands straight into registers
  // instead of through LDS (dn_set_small_m_loads; the same results).
  bool skinny_regs = false;
};

// Activations of one layer kept by a training forward (the reference's
// layerCache, internal/nn/forward.go:65-73, without the n x n probabilities:
// the backward recomputes them from lse).
struct LayerSave {
  DevBuf hs, h1;                      // fp32 [T x H]: layer input, residual after attention
  DevBuf n1, qkv, ctx, n2, wi, act;   // operand type: QKV input, un-rotated qkv, ctx, Wi input, Wi output, GeGLU
  DevBuf lse;                         // fp32 [T x heads]
  DevBuf mean1, rstd1, mean2, rstd2;  // fp32 [T]: attn_norm and mlp_norm row statistics
};

struct TrainState {
  bool enabled = false;
  int train_from = 0;
  bool train_emb = true;
  int adam_step = 0;
  std::vector<LayerSave> layers;
  bool have_forward = false;  // the activations of the last dn_forward_train are intact
  int T = 0, R = 0;
  std::vector<int32_t> ids;   // token ids of the last training forward
  DevBuf emb_mean, emb_rstd;  // emb norm row statistics of the last training forward
  // dh1, dwi and dqkv alternate by layer parity: the weight-gradient stream
  // transposes them while the main stream works on the next layer. dop_out /
  // dop_h1: bf16 copies of dout and dh1 (the input-gradient GEMMs' operands).
  DevBuf dcur, dprev, dh1[2], dact, dwi[2], dn2, dctx, dqkv[2], dn1, dop_out, dop_h1, dsum, part, lnpart, dE, dl,
      contrib;
  DevBuf emb_order, emb_seg, emb_id, sq_part, sq_out;
  DevBuf mt;                        // optimizer tensor table (device copy of mt_host)
  std::vector<MTensor> mt_host;
  // Weight-gradient GEMMs run on a second stream: per layer parity, the
  // transposed operands of the layer's four GEMMs, and the events that order
  // them against the main stream (operands ready / arena free again).
  DevBuf opT[2];
  hipStream_t side = nullptr;
  hipEvent_t ev_ready[2] = {nullptr, nullptr}, ev_done[2] = {nullptr, nullptr};
  hipEvent_t ev_trans[2] = {nullptr, nullptr};  // the layer's gradient transposes are done
};

// Inference batches of at most kSmallSplitMaxTokens tokens split the residual
// GEMMs (Wo, MlpWo) over K across workgroups, into at most kSmallSplitParts
// parts and kSplitMaxWorkgroups workgroups; the LayerNorm after each sums
// the parts into the residual stream.
constexpr int kSmallSplitMaxTokens = 128, kSmallSplitParts = 6, kSplitMaxWorkgroups = 256;

// Device memory one forward works in beyond the weights: the activations,
// the batch layout and the head's scratch. forward_core takes it from the
// context's own buffers unless a caller hands one in
// (dn_forward_device_noalloc points it into the library's static scratch array).
struct Workspace {
  float *h = nullptr;                                   // fp32 [T x H] residual stream
  void *xn = nullptr, *qkv = nullptr, *ctx = nullptr, *act = nullptr;  // operand type
  int *kinfo = nullptr;                                 // [T]
  float *head_s1 = nullptr, *head_d = nullptr;          // [R x H], [R x H/2]
  // [kSmallSplitParts x T x H] split-K partial products of the residual
  // GEMMs for batches of at most kSmallSplitMaxTokens tokens; null otherwise.
  float *part = nullptr;
  // Folded LayerNorm (bf16 / fp16, more than 1024 tokens): per row the residual
  // GEMM's (mean, M2) pairs over each 192 columns ([T x H/192]), and the
  // row means of a layer's attn_norm and mlp_norm ([T] each); null: no fold.
  float *lpart = nullptr;
  float *lmean1 = nullptr, *lmean2 = nullptr;
  int *seq_off = nullptr, *seq_len = nullptr, *chunk_off = nullptr, *first = nullptr;
  int4 *chunk_desc = nullptr, *work = nullptr;
  ChunkInfo *chunks = nullptr;
  uint32_t *codes = nullptr;
  // Global-layer work items of ATTN_QUERIES_GLOBAL queries (inference), their
  // tile codes and first tiles (inside the arrays above, after the
  // ATTN_QUERIES items' sections).
  int4 *work2 = nullptr;
  uint32_t *codes2 = nullptr;
  int *first2 = nullptr;
  int nwork2 = 0;
  int T = 0, nchunks = 0, nwork = 0;
  int nseq = 0, max_len = 0;
};

// The batch layout on the host: token offset and 32-token chunk offset of
// each sequence, the chunks (first token, length) and the attention work
// items (sequence, first query).
struct HostLayout {
  std::vector<int> seq_off, chunk_off;
  std::vector<int4> chunk_desc, work, work2;  // work2: ATTN_QUERIES_GLOBAL-query items
};

// One part of a forward split over two streams: its sequences' layout and
// device layout arrays (the activation buffers are the context's, at the
// part's token offset).
struct PartLayout {
  std::vector<int> len;
  HostLayout hl;
  DevBuf d_seq_off, d_seq_len, d_chunk_off, d_chunk_desc, d_chunks, d_work, d_codes, d_first;
  int T = 0, nchunks = 0, nwork = 0, nwork2 = 0;
};
constexpr int kMaxParts = 2;

struct dn_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipStream_t own_stream = nullptr;
  std::string err;
  bool configured = false;
  Config cfg;
  std::map<std::string, TensorSlot> w;
  DevBuf inv_freq;  // 32 doubles global theta, 32 local
  // workspace
  DevBuf h, xn, qkv, ctxb, act, kinfo, logits, err_flag, head_s1, head_d, smallpart;
  // A host batch (dn_forward, dn_forward_train) arrives as one copy: the
  // token ids, positions, option ids and mask-row tokens packed in `io`, with
  // these views into it (valid until the next staged batch), from a pinned
  // host buffer that also receives the logits and the error flag.
  DevBuf io;
  const int32_t *d_ids = nullptr, *d_pos = nullptr, *d_opt = nullptr, *d_rowtok = nullptr;
  void *pin = nullptr;
  size_t pin_cap = 0;
  bool pin_pending = false;  // a copy out of `pin` may be in flight (a call failed before its final sync)
  // RoPE cos/sin per position 0..65535 (global theta, then local), built once
  // per configuration at the first forward.
  DevBuf rope;
  bool rope_ready = false;
  DevBuf gA, gB, gC;  // dn_gemm_f32 staging
  DevBuf calib;       // dn_mfma_calibrate's result sink
  void *scratch = nullptr;  // this device's static scratch array (noalloc.cpp), from hipGetSymbolAddress
  // Folded LayerNorm (dn_set_ln_fold): the column sums of the LayerNorm-
  // weighted QKV and Wi weights per layer ([L x (3H + 2I)] floats, allocated
  // by dn_set_config), rebuilt when the weights' generation (bumped by every
  // upload and optimizer step) has moved; the forwards' statistics buffers.
  DevBuf fold_cs, fold_part, fold_mean;
  uint64_t wgen = 1, fold_gen = 0;
  bool ln_fold = true;
  // Forwards of large batches run in two parts of whole sequences, one per
  // stream (the context's and aux_stream, created on first use at the
  // default priority), so the kernels of one part overlap the other's.
  PartLayout parts[kMaxParts];
  hipStream_t aux_stream = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  int split_min_tokens = 8192;  // batches from this many tokens (and >= 2 sequences) are split
  int tail_min_tokens = 2048;   // from this many tokens the last layer's tail runs on the head's rows
  // batch layout cache
  std::vector<int> lay_len;
  HostLayout hlay;
  DevBuf d_seq_off, d_seq_len, d_chunk_off, d_chunk_desc, d_work, d_chunks;
  DevBuf d_codes, d_first;  // attention tile classes per work item: [global | local]
  int lay_T = 0, lay_nchunks = 0, lay_nwork = 0, lay_nwork2 = 0;
  // kernel probe: events[2*k], events[2*k+1] bracket launch k of one forward
  int probe_layer = -1;
  std::vector<hipEvent_t> probe_pool;  // 10 events per recorded forward
  int probe_used = 0;                  // forwards recorded
  std::vector<hipEvent_t> probe_bwd_pool;  // 6 events per recorded backward
  int probe_bwd_used = 0;
  TrainState tr;
  // Certified argmax (dn_set_certify, certify.cpp): an fp32 twin holding the
  // same weights recomputes the sequences whose two best logits are closer
  // than the margin; counters of sequences checked / recomputed; the twin's
  // compact batch and logits for dn_forward_device.
  dn_ctx *exact = nullptr;
  float certify_margin = 0.0f;
  int64_t cert_checked = 0, cert_recomputed = 0;
  DevBuf cert_in, cert_out;
};

namespace dnh {

constexpr int kPositions = 65536;  // RoPE table rows: positions are validated / flagged to this range

int fail(dn_ctx *c, int code, const std::string &msg);
int hip_fail(dn_ctx *c, const char *op, hipError_t e);
hipError_t ensure(DevBuf &b, size_t bytes);
void release(DevBuf &b);
void release_slot(TensorSlot &t);
void release_train(TrainState &tr);
uint16_t f32_to_bf16_rne(float f);
std::string layer_prefix(int l);
const void *W(dn_ctx *c, const std::string &name);
int check_ready(dn_ctx *c);
int64_t wi_src_row(int64_t r, int64_t I);
// Validates a host batch as dn_forward does and stages it on the device
// (ids, pos, opt, row_tok); *R receives the number of option rows.
int stage_batch(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
                const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, int logits_cap, int *R,
                int64_t *T);
// The forward on device-resident token arrays; with train, the activations of
// layers >= c->tr.train_from are kept in c->tr.layers.
// ws: the workspace to run in (inference only); null = the context's buffers.
int forward_core(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *d_ids, const int32_t *d_pos,
                 const int32_t *d_opt, int R, const int32_t *d_row_tok, float *d_logits, bool train,
                 const Workspace *ws = nullptr);
// The batch layout of nseq sequences on the host; *T and *nchunks receive
// the token and 32-token chunk counts.
void host_layout(HostLayout &hl, int nseq, const int32_t *seq_len, int *T, int *nchunks);
// Copies a host layout into w's device arrays on stream s.
int upload_layout(dn_ctx *c, const HostLayout &hl, const Workspace &w, int nseq, const int32_t *seq_len,
                  hipStream_t s);
// RoPE tables of the configured thetas and the device error flag: built at
// set-up (dn_set_config), so forwards allocate neither.
int ensure_rope(dn_ctx *c);
// Points the global-layer (ATTN_QUERIES_GLOBAL) work-item fields of w into
// its work / codes / first arrays, after the ATTN_QUERIES items' sections.
void set_work2(Workspace &w, int nwork2);
int ensure_err_flag(dn_ctx *c);
// Folded LayerNorm: whether a forward of T tokens on this context takes it,
// and the column sums brought up to date with the weights (a kernel per
// projection on stream s when they changed; no allocation).
bool fold_eligible(const dn_ctx *c, int T);
int ensure_fold_cs(dn_ctx *c, hipStream_t s);
// Bytes of the folded LayerNorm's per-token statistics (0 when the context
// never folds).
size_t fold_bytes_per_token(const dn_ctx *c);
// Fills in the context's own scratch pointer for its device (noalloc.cpp;
// called by dn_open with the device current).
int noalloc_init(dn_ctx *c);
// Finishes a host-array forward: logits to the host and the device error flag.
int finish_forward(dn_ctx *c, int R, float *logits);
// Certified argmax (certify.cpp): near-tie sequences of a finished forward
// recomputed on the fp32 twin (no-ops without dn_set_certify).
int certify_host(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
                 const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, float *logits);
int certify_device(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *d_ids, const int32_t *d_pos,
                   const int32_t *d_opt, int R, const int32_t *d_row_tok, float *d_logits);
void close_certify(dn_ctx *c);

}  // namespace dnh

#define HIPCHK(c, op, expr)                                     \
  do {                                                          \
    hipError_t e_ = (expr);                                     \
    if (e_ != hipSuccess) return dnh::hip_fail(c, op, e_);      \
  } while (0)
