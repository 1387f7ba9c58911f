// C ABI of libdecide_hip.so: context, weights, batch layout and the forward
// orchestration. Declarations and the reference interfaces each entry point
// replaces are in include/decide_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "ctx.hpp"

namespace {
thread_local std::string g_err;  // errors without a context
}  // namespace

int set_host_error(int code, const std::string &msg) {
  g_err = msg;
  return code;
}

using namespace dnh;

namespace dnh {

int fail(dn_ctx *c, int code, const std::string &msg) {
  if (c)
    c->err = msg;
  else
    g_err = msg;
  return code;
}

int hip_fail(dn_ctx *c, const char *op, hipError_t e) {
  const int code = e == hipErrorOutOfMemory ? DN_OUT_OF_MEMORY : DN_DEVICE_ERROR;
  return fail(c, code, std::string("hip: ") + op + " failed: " + hipGetErrorString(e) + " [code " +
                           std::to_string((int)e) + "]");
}

hipError_t ensure(DevBuf &b, size_t bytes) {
  if (bytes == 0) bytes = 16;
  if (bytes <= b.cap) return hipSuccess;
  if (b.p) {
    hipError_t e = hipFree(b.p);
    if (e != hipSuccess) return e;
  }
  b.p = nullptr;
  b.cap = 0;
  bytes = (bytes + 255) & ~(size_t)255;
  hipError_t e = hipMalloc(&b.p, bytes);
  if (e != hipSuccess) {
    b.p = nullptr;
    return e;
  }
  b.cap = bytes;
  return hipSuccess;
}

void release(DevBuf &b) {
  if (b.p) (void)hipFree(b.p);
  b.p = nullptr;
  b.cap = 0;
}

void release_slot(TensorSlot &t) {
  DevBuf *bufs[] = {&t.buf, &t.train.master, &t.train.grad, &t.train.m, &t.train.v, &t.train.wt};
  for (DevBuf *b : bufs) release(*b);
}

void release_train(TrainState &tr) {
  for (LayerSave &S : tr.layers) {
    DevBuf *bufs[] = {&S.hs, &S.h1, &S.n1, &S.qkv, &S.ctx, &S.n2, &S.wi, &S.act, &S.lse,
                      &S.mean1, &S.rstd1, &S.mean2, &S.rstd2};
    for (DevBuf *b : bufs) release(*b);
  }
  tr.layers.clear();
  DevBuf *bufs[] = {&tr.dcur, &tr.dprev, &tr.dh1[0], &tr.dh1[1], &tr.dact, &tr.dwi[0], &tr.dwi[1], &tr.dn2,
                    &tr.dctx, &tr.dqkv[0], &tr.dqkv[1], &tr.dn1, &tr.dop_out, &tr.dop_h1, &tr.dsum, &tr.part,
                    &tr.lnpart, &tr.dE, &tr.dl, &tr.contrib, &tr.emb_order, &tr.emb_seg, &tr.emb_id, &tr.sq_part,
                    &tr.sq_out, &tr.opT[0], &tr.opT[1], &tr.emb_mean, &tr.emb_rstd, &tr.mt};
  if (tr.side) (void)hipStreamSynchronize(tr.side);
  for (DevBuf *b : bufs) release(*b);
  for (int i = 0; i < 2; i++) {
    if (tr.ev_ready[i]) (void)hipEventDestroy(tr.ev_ready[i]);
    if (tr.ev_done[i]) (void)hipEventDestroy(tr.ev_done[i]);
    if (tr.ev_trans[i]) (void)hipEventDestroy(tr.ev_trans[i]);
    tr.ev_ready[i] = tr.ev_done[i] = tr.ev_trans[i] = nullptr;
  }
  if (tr.side) (void)hipStreamDestroy(tr.side);
  tr.side = nullptr;
  tr.have_forward = false;
}

uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Nearest-even binary16 bits of f (the compiler's conversion: subnormals
// kept, |f| >= 65520 to infinity). bf16 values with 2^-17 <= |f| <= 65504
// convert exactly.
uint16_t f32_to_f16_rne(float f) {
  const _Float16 h = (_Float16)f;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

// Whether a finite f lies outside binary16's range (it would become infinite).
bool f16_overflows(float f) { return std::isfinite(f) && std::fabs(f) >= 65520.0f; }

std::string layer_prefix(int l) { return "model.layers." + std::to_string(l) + "."; }

void define_tensors(dn_ctx *c) {
  const Config &g = c->cfg;
  const int64_t H = g.hidden, I = g.inter;
  auto add = [&](const std::string &name, int64_t n, int rank, bool proj = false, bool wi = false) {
    TensorSlot s;
    s.n = n;
    s.rank = rank;
    s.proj = proj;
    s.wi = wi;
    c->w[name] = s;
  };
  add("model.embeddings.tok_embeddings.weight", (int64_t)g.vocab * H, 2);
  add("model.embeddings.norm.weight", H, 1);
  for (int l = 0; l < g.layers; l++) {
    const std::string p = layer_prefix(l);
    if (l > 0) add(p + "attn_norm.weight", H, 1);
    add(p + "attn.Wqkv.weight", 3 * H * H, 2, true);
    add(p + "attn.Wo.weight", H * H, 2, true);
    add(p + "mlp_norm.weight", H, 1);
    add(p + "mlp.Wi.weight", 2 * I * H, 2, true, !g.generic);  // interleaved for the MFMA GeGLU epilogue
    add(p + "mlp.Wo.weight", H * I, 2, true);
  }
  add("model.final_norm.weight", H, 1);
  add("scorer.input_norm.weight", H, 1);
  add("scorer.input_norm.bias", H, 1);
  add("scorer.dense.weight", H / 2 * H, 2);
  add("scorer.dense.bias", H / 2, 1);
  add("scorer.norm.weight", H / 2, 1);
  add("scorer.norm.bias", H / 2, 1);
  add("scorer.out_proj.weight", H / 2, 2);
  add("scorer.out_proj.bias", 1, 1);
}

// Device pointer of an uploaded weight (check_ready has verified that every
// tensor of the configured model is set; a name outside the model is a bug
// here, not an input error, and gives a null pointer rather than a new slot).
const void *W(dn_ctx *c, const std::string &name) {
  auto it = c->w.find(name);
  return it == c->w.end() ? nullptr : it->second.buf.p;
}

// The global-layer work items (ATTN_QUERIES_GLOBAL queries) follow the
// ATTN_QUERIES ones in the work array; their tile codes and first tiles
// follow the two sections (global, local) of the ATTN_QUERIES items.
void set_work2(Workspace &w, int nwork2) {
  w.nwork2 = nwork2;
  w.work2 = w.work + w.nwork;
  w.codes2 = w.codes + (size_t)2 * w.nwork * ATTN_MAXKT;
  w.first2 = w.first + 2 * w.nwork;
}

// Batch layout: sequence offsets, 32-token chunks and ATTN_QUERIES-query work items.
void host_layout(HostLayout &hl, int nseq, const int32_t *seq_len, int *T_out, int *nch_out) {
  hl.seq_off.assign(nseq + 1, 0);
  hl.chunk_off.assign(nseq + 1, 0);
  hl.chunk_desc.clear();
  hl.work.clear();
  hl.work2.clear();
  int T = 0, nch = 0;
  for (int s = 0; s < nseq; s++) {
    const int n = seq_len[s];
    hl.seq_off[s] = T;
    hl.chunk_off[s] = nch;
    for (int i = 0; i < n; i += 32) hl.chunk_desc.push_back(make_int4(T + i, std::min(32, n - i), 0, 0));
    // Work item: (sequence, first query, sequence offset, sequence length).
    for (int q = 0; q < n; q += ATTN_QUERIES) hl.work.push_back(make_int4(s, q, T, n));
    for (int q = 0; q < n; q += ATTN_QUERIES_GLOBAL) hl.work2.push_back(make_int4(s, q, T, n));
    nch += (n + 31) / 32;
    T += n;
  }
  hl.seq_off[nseq] = T;
  hl.chunk_off[nseq] = nch;
  *T_out = T;
  *nch_out = nch;
}

int upload_layout(dn_ctx *c, const HostLayout &hl, const Workspace &w, int nseq, const int32_t *seq_len,
                  hipStream_t s) {
  HIPCHK(c, "hipMemcpyAsync",
         hipMemcpyAsync(w.seq_off, hl.seq_off.data(), sizeof(int) * (nseq + 1), hipMemcpyHostToDevice, s));
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(w.seq_len, seq_len, sizeof(int) * nseq, hipMemcpyHostToDevice, s));
  HIPCHK(c, "hipMemcpyAsync",
         hipMemcpyAsync(w.chunk_off, hl.chunk_off.data(), sizeof(int) * (nseq + 1), hipMemcpyHostToDevice, s));
  if (!hl.chunk_desc.empty())
    HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(w.chunk_desc, hl.chunk_desc.data(), sizeof(int4) * hl.chunk_desc.size(),
                                               hipMemcpyHostToDevice, s));
  if (!hl.work.empty())
    HIPCHK(c, "hipMemcpyAsync",
           hipMemcpyAsync(w.work, hl.work.data(), sizeof(int4) * hl.work.size(), hipMemcpyHostToDevice, s));
  if (!hl.work2.empty())
    HIPCHK(c, "hipMemcpyAsync",
           hipMemcpyAsync(w.work2, hl.work2.data(), sizeof(int4) * hl.work2.size(), hipMemcpyHostToDevice, s));
  return DN_OK;
}

// The context's own workspace: layout arrays (re-uploaded only when the batch
// layout changes) and activation buffers for T tokens and R rows.
// Folded LayerNorm: attn_norm and mlp_norm of the large-batch bf16 forward
// run inside the GEMMs around them (LnFold, the EPI_*_LN forms): the residual GEMM
// before the norm writes its operand and row statistics, the GEMM after it
// applies the row and column terms, and the LayerNorm launch disappears.
bool fold_geometry(const dn_ctx *c) {
  const Config &g = c->cfg;
  return !g.generic && gemm_ln_fold_ok(g.precision, 1025, g.hidden, g.inter);
}

bool fold_eligible(const dn_ctx *c, int T) {
  const Config &g = c->cfg;
  return c->ln_fold && c->fold_cs.p && !g.generic && gemm_ln_fold_ok(g.precision, T, g.hidden, g.inter);
}

size_t fold_bytes_per_token(const dn_ctx *c) {
  if (!fold_geometry(c)) return 0;
  return sizeof(float) * 2 * (c->cfg.hidden / kLnPartCols) + sizeof(float) * 2;
}

// The consumer GEMMs' column sums of layer l: QKV's (attn_norm, layers >= 1)
// at fold_cs + l * (3H + 2I), Wi's (mlp_norm) 3H further.
float *fold_cs_qkv(dn_ctx *c, int l) {
  const Config &g = c->cfg;
  return (float *)c->fold_cs.p + (size_t)l * (3 * g.hidden + 2 * g.inter);
}
float *fold_cs_wi(dn_ctx *c, int l) { return fold_cs_qkv(c, l) + 3 * c->cfg.hidden; }

int ensure_fold_cs(dn_ctx *c, hipStream_t s) {
  if (!c->fold_cs.p || c->fold_gen == c->wgen) return DN_OK;
  const Config &g = c->cfg;
  const int H = g.hidden, I = g.inter;
  for (int l = 0; l < g.layers; l++) {
    const std::string pf = layer_prefix(l);
    if (l > 0)
      HIPCHK(c, "fold_colsum", launch_fold_colsum(g.precision, W(c, pf + "attn.Wqkv.weight"), 3 * H, H,
                                                  (const float *)W(c, pf + "attn_norm.weight"), fold_cs_qkv(c, l), s));
    HIPCHK(c, "fold_colsum", launch_fold_colsum(g.precision, W(c, pf + "mlp.Wi.weight"), 2 * I, H,
                                                (const float *)W(c, pf + "mlp_norm.weight"), fold_cs_wi(c, l), s));
  }
  c->fold_gen = c->wgen;
  return DN_OK;
}

// The folded LayerNorm's statistics buffers for T tokens (none when this
// context never folds).
int ensure_fold_buffers(dn_ctx *c, size_t T) {
  if (!fold_geometry(c) || !c->ln_fold) return DN_OK;
  HIPCHK(c, "hipMalloc", ensure(c->fold_part, sizeof(float) * 2 * (c->cfg.hidden / kLnPartCols) * T));
  HIPCHK(c, "hipMalloc", ensure(c->fold_mean, sizeof(float) * 2 * T));
  return DN_OK;
}

int ctx_workspace(dn_ctx *c, int nseq, const int32_t *seq_len, int R, Workspace *w) {
  std::vector<int> len(seq_len, seq_len + nseq);
  const bool same = len == c->lay_len && c->d_seq_off.p;
  if (!same) {
    HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));  // old host staging may be in flight
    c->lay_len.clear();
    int T = 0, nch = 0;
    host_layout(c->hlay, nseq, seq_len, &T, &nch);
    const size_t nw = c->hlay.work.size(), nw2 = c->hlay.work2.size();
    HIPCHK(c, "hipMalloc", ensure(c->d_seq_off, sizeof(int) * (nseq + 1)));
    HIPCHK(c, "hipMalloc", ensure(c->d_seq_len, sizeof(int) * (nseq + 1)));
    HIPCHK(c, "hipMalloc", ensure(c->d_chunk_off, sizeof(int) * (nseq + 1)));
    HIPCHK(c, "hipMalloc", ensure(c->d_chunk_desc, sizeof(int4) * (nch + 1)));
    HIPCHK(c, "hipMalloc", ensure(c->d_chunks, sizeof(ChunkInfo) * (nch + 1)));
    HIPCHK(c, "hipMalloc", ensure(c->d_work, sizeof(int4) * (nw + nw2 + 1)));
    HIPCHK(c, "hipMalloc", ensure(c->d_codes, sizeof(uint32_t) * ATTN_MAXKT * (2 * nw + nw2 + 1)));
    HIPCHK(c, "hipMalloc", ensure(c->d_first, sizeof(int) * (2 * nw + nw2 + 1)));
    c->lay_len = len;
    c->lay_T = T;
    c->lay_nchunks = nch;
    c->lay_nwork = (int)nw;
    c->lay_nwork2 = (int)nw2;
  }
  Workspace &o = *w;
  o.seq_off = (int *)c->d_seq_off.p;
  o.seq_len = (int *)c->d_seq_len.p;
  o.chunk_off = (int *)c->d_chunk_off.p;
  o.chunk_desc = (int4 *)c->d_chunk_desc.p;
  o.chunks = (ChunkInfo *)c->d_chunks.p;
  o.work = (int4 *)c->d_work.p;
  o.codes = (uint32_t *)c->d_codes.p;
  o.first = (int *)c->d_first.p;
  o.T = c->lay_T;
  o.nchunks = c->lay_nchunks;
  o.nwork = c->lay_nwork;
  set_work2(o, c->lay_nwork2);
  o.nseq = (int)c->lay_len.size();
  o.max_len = c->lay_len.empty() ? 0 : *std::max_element(c->lay_len.begin(), c->lay_len.end());
  if (!same) {
    int rc = upload_layout(c, c->hlay, o, nseq, c->lay_len.data(), c->stream);
    if (rc) return rc;
  }
  const Config &g = c->cfg;
  const size_t es = prec16(g.precision) ? 2 : 4, T = (size_t)o.T, H = g.hidden;
  HIPCHK(c, "hipMalloc", ensure(c->h, sizeof(float) * T * H));
  HIPCHK(c, "hipMalloc", ensure(c->xn, es * T * H));
  HIPCHK(c, "hipMalloc", ensure(c->qkv, es * T * 3 * H));
  HIPCHK(c, "hipMalloc", ensure(c->ctxb, es * T * H));
  HIPCHK(c, "hipMalloc", ensure(c->act, es * T * g.inter));
  HIPCHK(c, "hipMalloc", ensure(c->kinfo, sizeof(int) * T));
  HIPCHK(c, "hipMalloc", ensure(c->head_s1, sizeof(float) * (size_t)std::max(R, 1) * H));
  HIPCHK(c, "hipMalloc", ensure(c->head_d, sizeof(float) * (size_t)std::max(R, 1) * (H / 2)));
  if (T <= (size_t)kSmallSplitMaxTokens)
    HIPCHK(c, "hipMalloc", ensure(c->smallpart, sizeof(float) * kSmallSplitParts * T * H));
  o.part = T <= (size_t)kSmallSplitMaxTokens ? (float *)c->smallpart.p : nullptr;
  if (fold_eligible(c, (int)T)) {
    const int rc = ensure_fold_buffers(c, T);
    if (rc) return rc;
    o.lpart = (float *)c->fold_part.p;
    o.lmean1 = (float *)c->fold_mean.p;
    o.lmean2 = (float *)c->fold_mean.p + T;
  }
  o.h = (float *)c->h.p;
  o.xn = c->xn.p;
  o.qkv = c->qkv.p;
  o.ctx = c->ctxb.p;
  o.act = c->act.p;
  o.kinfo = (int *)c->kinfo.p;
  o.head_s1 = (float *)c->head_s1.p;
  o.head_d = (float *)c->head_d.p;
  return DN_OK;
}

int ensure_rope(dn_ctx *c) {
  if (c->rope_ready) return DN_OK;
  HIPCHK(c, "hipMalloc", ensure(c->rope, sizeof(float) * kPositions * 32 * 4));
  float *r = (float *)c->rope.p;
  const double *inv = (const double *)c->inv_freq.p;
  HIPCHK(c, "rope_tables", launch_rope_tables(nullptr, kPositions, inv, inv + 32, r, r + (size_t)kPositions * 32,
                                              r + (size_t)2 * kPositions * 32, r + (size_t)3 * kPositions * 32,
                                              c->stream));
  c->rope_ready = true;
  return DN_OK;
}

// The device-side error flag: allocated and zeroed once per context.
int ensure_err_flag(dn_ctx *c) {
  if (c->err_flag.p) return DN_OK;
  HIPCHK(c, "hipMalloc", ensure(c->err_flag, sizeof(int)));
  HIPCHK(c, "hipMemsetAsync", hipMemsetAsync(c->err_flag.p, 0, sizeof(int), c->stream));
  return DN_OK;
}

int check_ready(dn_ctx *c) {
  if (!c->configured) return fail(c, DN_INVALID_ARG, "decide_hip: dn_set_config has not been called");
  if (!dn_weights_ready(c)) {
    for (auto &kv : c->w)
      if (!kv.second.set) return fail(c, DN_INVALID_ARG, "decide_hip: weight " + kv.first + " not uploaded");
  }
  return DN_OK;
}

// Returns the event pair slot for launch k of the current forward, or null
// when the probe is off for this layer.
hipEvent_t *probe_slot(dn_ctx *c, int l) {
  if (c->probe_layer != l) return nullptr;
  const size_t need = (size_t)(c->probe_used + 1) * 10;
  while (c->probe_pool.size() < need) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    c->probe_pool.push_back(e);
  }
  return &c->probe_pool[(size_t)c->probe_used * 10];
}

#define PROBED(slot, k, op, call)                                              \
  do {                                                                         \
    if (slot) HIPCHK(c, "hipEventRecord", hipEventRecord((slot)[2 * (k)], s)); \
    HIPCHK(c, op, call);                                                       \
    if (slot) HIPCHK(c, "hipEventRecord", hipEventRecord((slot)[2 * (k) + 1], s)); \
  } while (0)

// The tokens one stream works on: a workspace (for one part of a split
// forward, a view at the part's token offset into the context's buffers),
// those tokens' ids / positions / option ids, and the stream.
struct Pass {
  // Global layers on ATTN_QUERIES_GLOBAL work items (the two-stream forward of
  // a large batch); every other forward, training included, uses ATTN_QUERIES
  // items for all layers.
  bool wide_global = false;
  // The folded LayerNorm (the workspace has its buffers and the pass more
  // than 1024 tokens).
  bool fold = false;
  Workspace w;
  const int32_t *ids, *pos, *opt;
  hipStream_t s;
};

// Token info, 32-token chunk summaries, attention tile classes of both layer
// types, and the embedding gather + emb norm into cur (fp32) and xn0.
int enqueue_prologue(dn_ctx *c, const Pass &p, float *cur, void *xn0, float *emb_mean, float *emb_rstd) {
  const Config &g = c->cfg;
  const Workspace &w = p.w;
  hipStream_t s = p.s;
  // Token info, chunk summaries and the embedding gather + emb norm in one
  // launch, then the tile classes (which need the chunk summaries).
  HIPCHK(c, "prologue",
         launch_prologue(g.precision, p.pos, p.opt, w.chunk_desc, w.nchunks, w.kinfo, w.chunks, p.ids, w.T,
                         (const float *)W(c, "model.embeddings.tok_embeddings.weight"), g.vocab,
                         (const float *)W(c, "model.embeddings.norm.weight"), g.eps, g.hidden, cur, xn0,
                         (int *)c->err_flag.p, s, emb_mean, emb_rstd));
  const size_t nw = (size_t)w.nwork;
  // Local layers use the ATTN_QUERIES items; global layers too (both types
  // in one launch), or the ATTN_QUERIES_GLOBAL ones in the two-stream forward.
  if (p.wide_global)
    HIPCHK(c, "tile_codes", launch_tile_codes(w.chunks, w.work, w.seq_len, w.chunk_off, w.nwork, 1, g.half_window,
                                              w.codes + nw * ATTN_MAXKT, w.first + nw, s));
  else
    HIPCHK(c, "tile_codes", launch_tile_codes(w.chunks, w.work, w.seq_len, w.chunk_off, w.nwork, -1, g.half_window,
                                              w.codes, w.first, s));
  if (p.wide_global)
    HIPCHK(c, "tile_codes", launch_tile_codes(w.chunks, w.work2, w.seq_len, w.chunk_off, w.nwork2, 0, g.half_window,
                                              w.codes2, w.first2, s, ATTN_WAVES * ATTN_QT_GLOBAL));
  return DN_OK;
}

// Split-K parts of a small batch's residual GEMM (32 x 32 tiles): the most,
// among the counts launch_ln_parts sums, that keep tiles x parts within
// kSplitMaxWorkgroups and give every part a whole number of K groups (1: no
// split).
int small_split_parts(int precision, int T, int N, int K) {
  const int tiles = (N / 32) * ((T + 31) / 32), kt = prec16(precision) ? 64 : 32;
  for (int p : {6, 4, 3, 2})
    if (p <= kSmallSplitParts && tiles * p <= kSplitMaxWorkgroups && K % (p * kt) == 0) return p;
  return 1;
}

// A projection GEMM of the model: the MFMA kernels, or the any-shape kernel
// for geometries they do not tile.
hipError_t layer_gemm(const Config &g, int epi, const GemmArgs &a0, hipStream_t s, const LnFold *ln = nullptr) {
  GemmArgs a = a0;
  a.skinny_regs = g.skinny_regs ? 1 : 0;
  return g.generic ? launch_gemm_generic(g.precision, epi, a, s) : launch_gemm(g.precision, epi, a, s, ln);
}

// The launches of encoder layer l over the pass's tokens: the residual stream
// enters in `in`, leaves the attention half in h1 and the layer in out (the
// same buffer unless training keeps them apart); x1 is the QKV input of layer
// 0 (the embedding output; later layers normalise `in` into the workspace).
// S (training) receives the layer's activations; ev brackets the five probed
// launches. attn_only: stop after attention (enqueue_rows_tail finishes the
// layer for the head's rows). Small inference batches (w.part set, the
// residual stream updated in place): Wo runs split over K and mlp_norm sums
// its parts into the residual; in_parts > 0: `in` still lacks the previous
// layer's MlpWo parts, which attn_norm adds; mo_parts non-null: this layer's
// MlpWo may leave its parts for the next layer's attn_norm the same way and
// stores their count (0: the residual stream is complete). With the folded
// LayerNorm (p.fold): fold_in, the previous layer's MlpWo left attn_norm's
// operand in the workspace's xn and its statistics (this layer's QKV applies
// the norm); mlp_norm is folded into Wo and Wi; fold_out, this layer's
// MlpWo leaves the next layer's attn_norm operand the same way.
int enqueue_layer(dn_ctx *c, const Pass &p, int l, float *in, float *h1, float *out, void *x1, LayerSave *S,
                  hipEvent_t *ev, bool attn_only = false, int in_parts = 0, int *mo_parts = nullptr,
                  bool fold_in = false, bool fold_out = false) {
  const Config &g = c->cfg;
  const int H = g.hidden, I = g.inter, prec = g.precision;
  const Workspace &w = p.w;
  const int T = w.T;
  hipStream_t s = p.s;
  const std::string pf = layer_prefix(l);
  const bool sliding = g.sliding[l] != 0;
  const bool split = w.part && !S && !g.generic && h1 == in && out == in;
  const bool fold = p.fold && w.lpart && !S && !split && !g.generic && h1 == in && out == in;
  fold_in = fold_in && fold && l > 0;
  fold_out = fold_out && fold && l + 1 < g.layers;
  const int lparts = H / kLnPartCols;
  if (l > 0) {
    x1 = S ? S->n1.p : w.xn;
    if (fold_in) {
      // the previous layer's MlpWo wrote x1 and the row statistics
    } else if (in_parts > 0 && split)
      HIPCHK(c, "ln(attn_norm)", launch_ln_parts(prec, in, w.part, in_parts, T, H,
                                                 (const float *)W(c, pf + "attn_norm.weight"), g.eps, x1, s));
    else
      HIPCHK(c, "ln(attn_norm)",
             launch_ln(prec, in, T, H, (const float *)W(c, pf + "attn_norm.weight"), g.eps, x1, s,
                       S ? (float *)S->mean1.p : nullptr, S ? (float *)S->rstd1.p : nullptr));
  }
  GemmArgs q{};
  q.A = x1;
  q.lda = H;
  q.B = W(c, pf + "attn.Wqkv.weight");
  q.ldb = H;
  q.C = S ? S->qkv.p : w.qkv;
  q.ldc = 3 * H;
  q.M = T;
  q.N = 3 * H;
  q.K = H;
  q.n_store = 3 * H;
  LnFold qf{};
  if (fold_in) {
    qf.lpart = w.lpart;
    qf.lparts = lparts;
    qf.mprev = w.lmean2;  // what the previous MlpWo subtracted: its layer's mlp_norm means
    qf.mean_out = w.lmean1;
    qf.lcs = fold_cs_qkv(c, l);
    qf.eps = g.eps;
  }
  PROBED(ev, DN_PROBE_QKV, "gemm(Wqkv)", layer_gemm(g, fold_in ? EPI_STORE_LN : EPI_STORE, q, s, &qf));

  const float *rope = (const float *)c->rope.p;
  const size_t tab = (size_t)kPositions * 32;
  AttnArgs at{};
  at.kinfo = w.kinfo;
  at.work = w.work;
  at.seq_off = w.seq_off;
  at.seq_len = w.seq_len;
  at.nwork = w.nwork;
  at.H = H;
  at.heads = g.heads;
  at.half_window = g.half_window;
  at.scale_log2 = (float)(1.0 / std::sqrt(64.0)) * 1.44269504088896340736f;
  at.qkv = q.C;
  at.ctx = S ? S->ctx.p : w.ctx;
  at.lse = S ? (float *)S->lse.p : nullptr;
  at.sliding = sliding ? 1 : 0;
  at.codes = w.codes + (sliding ? (size_t)w.nwork * ATTN_MAXKT : 0);
  at.first = w.first + (sliding ? w.nwork : 0);
  at.qt = ATTN_QT;
  if (!sliding && p.wide_global && w.nwork2 > 0) {  // global layer of the two-stream forward: 256-query items
    at.work = w.work2;
    at.nwork = w.nwork2;
    at.codes = w.codes2;
    at.first = w.first2;
    at.qt = ATTN_QT_GLOBAL;
  }
  at.cos_t = rope + (sliding ? 2 : 0) * tab;  // the layer type picks the table (forward.go:297-301)
  at.sin_t = rope + (sliding ? 3 : 1) * tab;
  at.nseq = w.nseq;
  at.max_len = w.max_len;
  at.head_dim = H / g.heads;
  at.scale = (float)(1.0 / std::sqrt((double)at.head_dim));  // forward.go:351
  PROBED(ev, DN_PROBE_ATTENTION, "attention",
         g.generic ? launch_attention_generic(prec, at, s) : launch_attention(prec, at, s));
  if (attn_only) return DN_OK;

  GemmArgs o{};
  o.A = at.ctx;
  o.lda = H;
  o.B = W(c, pf + "attn.Wo.weight");
  o.ldb = H;
  o.C = h1;
  o.res = h1 == in ? nullptr : in;
  o.ldc = H;
  o.M = T;
  o.N = H;
  o.K = H;
  o.n_store = H;
  o.accumulate = 1;
  void *x2 = S ? S->n2.p : w.xn;
  // The row value the folded mlp_norm's operand is taken relative to: this
  // layer's attn_norm means when its QKV folded too (0 otherwise).
  float *const mlp_mprev = fold_in ? w.lmean1 : nullptr;
  const int wo_parts = split ? small_split_parts(prec, T, H, H) : 1;
  if (wo_parts > 1) {
    o.skinny_regs = g.skinny_regs ? 1 : 0;
    PROBED(ev, DN_PROBE_WO, "gemm(Wo)", launch_gemm_small_split(prec, o, wo_parts, w.part, s));
    HIPCHK(c, "ln(mlp_norm)", launch_ln_parts(prec, h1, w.part, wo_parts, T, H,
                                              (const float *)W(c, pf + "mlp_norm.weight"), g.eps, x2, s));
  } else if (fold) {
    LnFold of{};
    of.fx = x2;
    of.lw = (const float *)W(c, pf + "mlp_norm.weight");
    of.lpart = w.lpart;
    of.lparts = lparts;
    of.mprev = mlp_mprev;
    PROBED(ev, DN_PROBE_WO, "gemm(Wo)", layer_gemm(g, EPI_F32_LN, o, s, &of));
  } else {
    PROBED(ev, DN_PROBE_WO, "gemm(Wo)", layer_gemm(g, EPI_F32, o, s));
    HIPCHK(c, "ln(mlp_norm)", launch_ln(prec, h1, T, H, (const float *)W(c, pf + "mlp_norm.weight"), g.eps, x2, s,
                                        S ? (float *)S->mean2.p : nullptr, S ? (float *)S->rstd2.p : nullptr));
  }

  GemmArgs wi{};
  wi.A = x2;
  wi.lda = H;
  wi.B = W(c, pf + "mlp.Wi.weight");
  wi.ldb = H;
  wi.M = T;
  wi.N = 2 * I;
  wi.K = H;
  wi.n_store = 2 * I;
  if (S) {  // training keeps the pre-activation as well as the GeGLU output
    wi.C = S->wi.p;
    wi.ldc = 2 * I;
    wi.C2 = S->act.p;
    wi.ldc2 = I;
    PROBED(ev, DN_PROBE_WI, "gemm(Wi)", layer_gemm(g, EPI_GEGLU_KEEP, wi, s));
  } else {
    wi.C = w.act;
    wi.ldc = I;
    LnFold wf{};
    if (fold) {
      wf.lpart = w.lpart;
      wf.lparts = lparts;
      wf.mprev = mlp_mprev;
      wf.mean_out = w.lmean2;
      wf.lcs = fold_cs_wi(c, l);
      wf.eps = g.eps;
    }
    PROBED(ev, DN_PROBE_WI, "gemm(Wi)", layer_gemm(g, fold ? EPI_GEGLU_LN : EPI_GEGLU, wi, s, &wf));
  }

  GemmArgs mo{};
  mo.A = S ? S->act.p : w.act;
  mo.lda = I;
  mo.B = W(c, pf + "mlp.Wo.weight");
  mo.ldb = I;
  mo.C = out;
  mo.res = out == h1 ? nullptr : h1;
  mo.ldc = H;
  mo.M = T;
  mo.N = H;
  mo.K = I;
  mo.n_store = H;
  mo.accumulate = 1;
  const int parts = split && mo_parts ? small_split_parts(prec, T, H, I) : 1;
  if (mo_parts) *mo_parts = parts > 1 ? parts : 0;
  mo.skinny_regs = g.skinny_regs ? 1 : 0;
  LnFold mf{};
  if (fold_out) {
    mf.fx = w.xn;
    mf.lw = (const float *)W(c, layer_prefix(l + 1) + "attn_norm.weight");
    mf.lpart = w.lpart;
    mf.lparts = lparts;
    mf.mprev = w.lmean2;
  }
  if (parts > 1)
    PROBED(ev, DN_PROBE_MLPWO, "gemm(MlpWo)", launch_gemm_small_split(prec, mo, parts, w.part, s));
  else
    PROBED(ev, DN_PROBE_MLPWO, "gemm(MlpWo)", layer_gemm(g, fold_out ? EPI_F32_LN : EPI_F32, mo, s, &mf));
  return DN_OK;
}

// Whether the last layer carries only the head's R rows past attention
// (dn_set_row_tail): an inference forward of at least tail_min_tokens tokens
// with at most a quarter of them head rows, unless the probe times the last
// layer's launches. Everything after attention in a layer is row-wise, and
// the head reads only its rows of the last layer's output.
bool tail_on_rows(const dn_ctx *c, int T, int R, bool train) {
  return !train && R > 0 && c->tail_min_tokens > 0 && T >= c->tail_min_tokens && 4LL * R <= T &&
         c->probe_layer != c->cfg.layers - 1;
}

// Layer l after its attention, for the R rows row_tok (indices into the
// T_total tokens) only: their attention output (ctx) and residual (h) rows
// are gathered, then Wo + residual, mlp_norm, Wi + GeGLU and MlpWo +
// residual run on R rows. The buffers are those the layer no longer reads
// once its attention has run: h_r (fp32 [R x H]) and the mlp_norm output at
// the start of qkv_buf, the gathered ctx rows in xn_buf, the GeGLU output in
// act_buf. *h_out receives h_r, whose row r is token row_tok[r]'s output.
int enqueue_rows_tail(dn_ctx *c, int l, const void *ctx, const float *h, int T_total, const int32_t *row_tok, int R,
                      void *qkv_buf, void *xn_buf, void *act_buf, float **h_out, hipStream_t s) {
  const Config &g = c->cfg;
  const int H = g.hidden, I = g.inter, prec = g.precision;
  const std::string pf = layer_prefix(l);
  float *h_r = (float *)qkv_buf;
  void *xn_r = (char *)qkv_buf + sizeof(float) * (size_t)R * H;
  void *ctx_r = xn_buf, *act_r = act_buf;
  HIPCHK(c, "gather_rows",
         launch_gather_rows(prec, ctx, h, row_tok, R, T_total, H, ctx_r, h_r, (int *)c->err_flag.p, s));
  GemmArgs o{};
  o.A = ctx_r;
  o.lda = H;
  o.B = W(c, pf + "attn.Wo.weight");
  o.ldb = H;
  o.C = h_r;
  o.ldc = H;
  o.M = R;
  o.N = H;
  o.K = H;
  o.n_store = H;
  o.accumulate = 1;
  HIPCHK(c, "gemm(Wo)", layer_gemm(g, EPI_F32, o, s));
  HIPCHK(c, "ln(mlp_norm)", launch_ln(prec, h_r, R, H, (const float *)W(c, pf + "mlp_norm.weight"), g.eps, xn_r, s));
  GemmArgs wi{};
  wi.A = xn_r;
  wi.lda = H;
  wi.B = W(c, pf + "mlp.Wi.weight");
  wi.ldb = H;
  wi.C = act_r;
  wi.ldc = I;
  wi.M = R;
  wi.N = 2 * I;
  wi.K = H;
  wi.n_store = 2 * I;
  HIPCHK(c, "gemm(Wi)", layer_gemm(g, EPI_GEGLU, wi, s));
  GemmArgs mo{};
  mo.A = act_r;
  mo.lda = I;
  mo.B = W(c, pf + "mlp.Wo.weight");
  mo.ldb = I;
  mo.C = h_r;
  mo.ldc = H;
  mo.M = R;
  mo.N = H;
  mo.K = I;
  mo.n_store = H;
  mo.accumulate = 1;
  HIPCHK(c, "gemm(MlpWo)", layer_gemm(g, EPI_F32, mo, s));
  *h_out = h_r;
  return DN_OK;
}

// Whether the last layer of a row-tail forward also runs its attention and
// its Q projection on the option rows (enqueue_rows_layer): the MFMA
// geometry, at most ROW_ITEMS_MAXSEQ sequences, and room for the row buffers
// in the buffers that layer leaves free (h_r in ctx; the gathered QKV input,
// Q and attention rows in act; the GeGLU rows in xn).
bool rows_layer_fits(const dn_ctx *c, int T, int R, int nseq) {
  const Config &g = c->cfg;
  if (g.generic || nseq > ROW_ITEMS_MAXSEQ) return false;
  const size_t es = prec16(g.precision) ? 2 : 4, H = g.hidden, I = g.inter, t = T, r = R;
  return 4 * r * H <= es * t * H && 3 * es * r * H <= es * t * I && es * r * I <= es * t * H;
}

// Bytes the option-row attention's work list takes in head_s1: nit int4
// items, R row slots and the item count.
size_t row_items_bytes(int nit, int R) { return sizeof(int4) * (size_t)nit + sizeof(int) * ((size_t)R + 1); }

// Layer l (the last) for the R option rows row_tok only, over the batch
// layout and buffers of w: attn_norm of every token (l > 0; x1 is layer 0's
// input otherwise), K and V of every token (rows H..3H of Wqkv into qkv's k
// and v columns), the rows' QKV input and residual gathered, their Q, the
// option-row attention (launch_row_items groups the rows by sequence), then
// Wo + residual, mlp_norm, Wi + GeGLU and MlpWo + residual on R rows. Every
// row's result is what the full layer gives that token: attention rows are
// independent queries over the same keys, and the rest is row-wise.
// *h_out receives h_r (row r: token row_tok[r]).
int enqueue_rows_layer(dn_ctx *c, const Workspace &w, int l, const float *h, const void *x1,
                       const int32_t *row_tok, int R, float **h_out, hipStream_t s) {
  const Config &g = c->cfg;
  const int H = g.hidden, I = g.inter, prec = g.precision, T = w.T;
  const size_t es = prec16(prec) ? 2 : 4;
  const std::string pf = layer_prefix(l);
  if (l > 0) {
    HIPCHK(c, "ln(attn_norm)", launch_ln(prec, h, T, H, (const float *)W(c, pf + "attn_norm.weight"), g.eps, w.xn, s));
    x1 = w.xn;
  }
  float *h_r = (float *)w.ctx;
  char *A = (char *)w.act;
  void *xn_r = A, *q_r = A + es * R * H, *ctx_r = A + 2 * es * R * H, *act_r = w.xn;
  HIPCHK(c, "gather_rows", launch_gather_rows(prec, x1, h, row_tok, R, T, H, xn_r, h_r, (int *)c->err_flag.p, s));
  const char *wqkv = (const char *)W(c, pf + "attn.Wqkv.weight");
  GemmArgs kv{};
  kv.A = x1;
  kv.lda = H;
  kv.B = wqkv + es * H * H;
  kv.ldb = H;
  kv.C = (char *)w.qkv + es * H;
  kv.ldc = 3 * H;
  kv.M = T;
  kv.N = 2 * H;
  kv.K = H;
  kv.n_store = 2 * H;
  HIPCHK(c, "gemm(Wqkv k, v)", layer_gemm(g, EPI_STORE, kv, s));
  GemmArgs q{};
  q.A = xn_r;
  q.lda = H;
  q.B = wqkv;
  q.ldb = H;
  q.C = q_r;
  q.ldc = H;
  q.M = R;
  q.N = H;
  q.K = H;
  q.n_store = H;
  HIPCHK(c, "gemm(Wqkv q)", layer_gemm(g, EPI_STORE, q, s));
  // Work items in head_s1 (free until the head): items, then slots, then the
  // count. Only sequences that hold rows make items, at most one per row, and
  // a sequence's rows split into ceil(r/128) items, so min(nseq, R) +
  // ceil(R/128) bounds the count whatever the rows' distribution.
  const int nit = std::min(w.nseq, R) + (R + ATTN_QUERIES - 1) / ATTN_QUERIES;
  if (row_items_bytes(nit, R) > sizeof(float) * (size_t)R * H)
    return fail(c, DN_DEVICE_ERROR, "decide_hip: row work items exceed the head scratch");
  int4 *items = (int4 *)w.head_s1;
  int *rows = (int *)(items + nit), *nitems = rows + R;
  HIPCHK(c, "row_items", launch_row_items(row_tok, R, w.seq_off, w.nseq, T, items, rows, nitems, s));
  const bool sliding = g.sliding[l] != 0;
  const float *rope = (const float *)c->rope.p;
  const size_t tab = (size_t)kPositions * 32;
  AttnArgs at{};
  at.qkv = w.qkv;
  at.ctx = ctx_r;
  at.kinfo = w.kinfo;
  at.cos_t = rope + (sliding ? 2 : 0) * tab;
  at.sin_t = rope + (sliding ? 3 : 1) * tab;
  at.seq_off = w.seq_off;
  at.seq_len = w.seq_len;
  at.nwork = nit;
  at.H = H;
  at.heads = g.heads;
  at.sliding = sliding ? 1 : 0;
  at.half_window = g.half_window;
  at.scale_log2 = (float)(1.0 / std::sqrt(64.0)) * 1.44269504088896340736f;
  at.qt = ATTN_QT;
  at.items = items;
  at.nitems = nitems;
  at.rows = rows;
  at.row_tok = row_tok;
  at.q_rows = q_r;
  HIPCHK(c, "attention(rows)", launch_attention_rows(prec, at, s));
  GemmArgs o{};
  o.A = ctx_r;
  o.lda = H;
  o.B = W(c, pf + "attn.Wo.weight");
  o.ldb = H;
  o.C = h_r;
  o.ldc = H;
  o.M = R;
  o.N = H;
  o.K = H;
  o.n_store = H;
  o.accumulate = 1;
  HIPCHK(c, "gemm(Wo)", layer_gemm(g, EPI_F32, o, s));
  HIPCHK(c, "ln(mlp_norm)", launch_ln(prec, h_r, R, H, (const float *)W(c, pf + "mlp_norm.weight"), g.eps, xn_r, s));
  GemmArgs wi{};
  wi.A = xn_r;
  wi.lda = H;
  wi.B = W(c, pf + "mlp.Wi.weight");
  wi.ldb = H;
  wi.C = act_r;
  wi.ldc = I;
  wi.M = R;
  wi.N = 2 * I;
  wi.K = H;
  wi.n_store = 2 * I;
  HIPCHK(c, "gemm(Wi)", layer_gemm(g, EPI_GEGLU, wi, s));
  GemmArgs mo{};
  mo.A = act_r;
  mo.lda = I;
  mo.B = W(c, pf + "mlp.Wo.weight");
  mo.ldb = I;
  mo.C = h_r;
  mo.ldc = H;
  mo.M = R;
  mo.N = H;
  mo.K = I;
  mo.n_store = H;
  mo.accumulate = 1;
  HIPCHK(c, "gemm(MlpWo)", layer_gemm(g, EPI_F32, mo, s));
  *h_out = h_r;
  return DN_OK;
}

// The scorer head over the R option rows (row_tok: indices into the T_total
// tokens of h; null: rows 0 .. R-1 of h, T_total = R).
int enqueue_head(dn_ctx *c, const float *h, int T_total, const int32_t *row_tok, int R, float *logits, float *s1,
                 float *d, hipStream_t s) {
  const Config &g = c->cfg;
  HeadArgs ha{};
  ha.h = h;
  ha.row_tok = row_tok;
  ha.R = R;
  ha.T = T_total;
  ha.H = g.hidden;
  ha.eps = g.eps;
  ha.final_norm = (const float *)W(c, "model.final_norm.weight");
  ha.in_w = (const float *)W(c, "scorer.input_norm.weight");
  ha.in_b = (const float *)W(c, "scorer.input_norm.bias");
  ha.dense_w = (const float *)W(c, "scorer.dense.weight");
  ha.dense_b = (const float *)W(c, "scorer.dense.bias");
  ha.norm_w = (const float *)W(c, "scorer.norm.weight");
  ha.norm_b = (const float *)W(c, "scorer.norm.bias");
  ha.out_w = (const float *)W(c, "scorer.out_proj.weight");
  ha.out_b = (const float *)W(c, "scorer.out_proj.bias");
  ha.logits = logits;
  ha.err_flag = (int *)c->err_flag.p;
  HIPCHK(c, "head", launch_head(ha, s1, d, s, g.generic));
  return DN_OK;
}

// The layout arrays of part k (sequences seq_len[0..nseq)), rebuilt and
// uploaded on stream s only when its sequence lengths change; fills the
// layout fields of w.
int part_layout(dn_ctx *c, int k, int nseq, const int32_t *seq_len, hipStream_t s, Workspace *w) {
  PartLayout &P = c->parts[k];
  std::vector<int> len(seq_len, seq_len + nseq);
  const bool same = len == P.len && P.d_seq_off.p;
  if (!same) {
    int T = 0, nch = 0;
    host_layout(P.hl, nseq, seq_len, &T, &nch);
    const size_t nw = P.hl.work.size(), nw2 = P.hl.work2.size();
    HIPCHK(c, "hipMalloc", ensure(P.d_seq_off, sizeof(int) * (nseq + 1)));
    HIPCHK(c, "hipMalloc", ensure(P.d_seq_len, sizeof(int) * (nseq + 1)));
    HIPCHK(c, "hipMalloc", ensure(P.d_chunk_off, sizeof(int) * (nseq + 1)));
    HIPCHK(c, "hipMalloc", ensure(P.d_chunk_desc, sizeof(int4) * (nch + 1)));
    HIPCHK(c, "hipMalloc", ensure(P.d_chunks, sizeof(ChunkInfo) * (nch + 1)));
    HIPCHK(c, "hipMalloc", ensure(P.d_work, sizeof(int4) * (nw + nw2 + 1)));
    HIPCHK(c, "hipMalloc", ensure(P.d_codes, sizeof(uint32_t) * ATTN_MAXKT * (2 * nw + nw2 + 1)));
    HIPCHK(c, "hipMalloc", ensure(P.d_first, sizeof(int) * (2 * nw + nw2 + 1)));
    P.len = len;
    P.T = T;
    P.nchunks = nch;
    P.nwork = (int)nw;
    P.nwork2 = (int)nw2;
  }
  w->seq_off = (int *)P.d_seq_off.p;
  w->seq_len = (int *)P.d_seq_len.p;
  w->chunk_off = (int *)P.d_chunk_off.p;
  w->chunk_desc = (int4 *)P.d_chunk_desc.p;
  w->chunks = (ChunkInfo *)P.d_chunks.p;
  w->work = (int4 *)P.d_work.p;
  w->codes = (uint32_t *)P.d_codes.p;
  w->first = (int *)P.d_first.p;
  w->T = P.T;
  w->nchunks = P.nchunks;
  w->nwork = P.nwork;
  set_work2(*w, P.nwork2);
  w->nseq = nseq;
  w->max_len = len.empty() ? 0 : *std::max_element(len.begin(), len.end());
  if (!same) return upload_layout(c, P.hl, *w, nseq, P.len.data(), s);
  return DN_OK;
}

// Inference forward of a large batch in two parts of whole sequences (about
// half the tokens each), the first on the context's stream and the second on
// aux_stream, layer by layer in alternation, so that one part's kernels fill
// the GPU around the other's (a residual GEMM's HBM-bound epilogue beside a
// projection GEMM's MFMA-bound main loop). Every kernel sees exactly the
// tokens it would see in the single-stream forward, so the logits are the
// same; the head runs once over all rows after the join.
// The sequence index that cuts a batch nearest half of its tokens (both
// parts non-empty); *first_tokens receives the first part's token count.
int split_point(int nseq, const int32_t *seq_len, int T_total, int *first_tokens) {
  int cut = 1, acc = seq_len[0];
  while (cut < nseq - 1 && 2 * (acc + seq_len[cut]) <= T_total) acc += seq_len[cut++];
  if (cut < nseq - 1 && std::abs(2 * (acc + seq_len[cut]) - T_total) < std::abs(2 * acc - T_total))
    acc += seq_len[cut++];
  *first_tokens = acc;
  return cut;
}

// Smallest part of a split forward: above it every GEMM of a part runs the
// tiled kernels of the single-stream forward (small M runs the small-M
// kernels, whose summation order differs), so the logits are identical.
constexpr int kMinPartTokens = 1025;

int forward_split(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *d_ids, const int32_t *d_pos,
                  const int32_t *d_opt, int R, const int32_t *d_row_tok, float *d_logits, int T_total, int cut,
                  int acc, const Workspace *wfull) {
  const Config &g = c->cfg;
  const int H = g.hidden, I = g.inter, L = g.layers;
  const size_t es = prec16(g.precision) ? 2 : 4;
  const int cnt[2] = {cut, nseq - cut}, tok0[2] = {0, acc};
  if (!c->aux_stream) {
    HIPCHK(c, "hipStreamCreate", hipStreamCreateWithFlags(&c->aux_stream, hipStreamNonBlocking));
    HIPCHK(c, "hipEventCreate", hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming));
    HIPCHK(c, "hipEventCreate", hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming));
  }
  const hipStream_t st[2] = {c->stream, c->aux_stream};
  // Shared activation buffers for all tokens; each part works at its offset.
  const size_t T = (size_t)T_total;
  HIPCHK(c, "hipMalloc", ensure(c->h, sizeof(float) * T * H));
  HIPCHK(c, "hipMalloc", ensure(c->xn, es * T * H));
  HIPCHK(c, "hipMalloc", ensure(c->qkv, es * T * 3 * H));
  HIPCHK(c, "hipMalloc", ensure(c->ctxb, es * T * H));
  HIPCHK(c, "hipMalloc", ensure(c->act, es * T * I));
  HIPCHK(c, "hipMalloc", ensure(c->kinfo, sizeof(int) * T));
  HIPCHK(c, "hipMalloc", ensure(c->head_s1, sizeof(float) * (size_t)std::max(R, 1) * H));
  HIPCHK(c, "hipMalloc", ensure(c->head_d, sizeof(float) * (size_t)std::max(R, 1) * (H / 2)));
  int rc = ensure_err_flag(c);
  if (rc) return rc;
  rc = ensure_rope(c);
  if (rc) return rc;
  // Each part's GEMMs fold when the part has more than 1024 tokens, as the
  // single-stream forward of the whole batch does (kMinPartTokens).
  const bool fold = fold_eligible(c, std::min(acc, T_total - acc));
  if (fold) {
    rc = ensure_fold_buffers(c, T);
    if (rc) return rc;
    rc = ensure_fold_cs(c, st[0]);  // before the fork: both streams read the column sums
    if (rc) return rc;
  }
  // The aux stream starts after everything already queued on the context's
  // stream (the caller's uploads of the token arrays among it).
  HIPCHK(c, "hipEventRecord", hipEventRecord(c->ev_fork, st[0]));
  HIPCHK(c, "hipStreamWaitEvent", hipStreamWaitEvent(st[1], c->ev_fork, 0));
  Pass ps[2];
  for (int k = 0; k < 2; k++) {
    const int32_t *sl = seq_len + (k ? cut : 0);
    const bool changed = c->parts[k].len != std::vector<int>(sl, sl + cnt[k]);
    if (changed) HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(st[k]));  // host staging may be in flight
    rc = part_layout(c, k, cnt[k], sl, st[k], &ps[k].w);
    if (rc) return rc;
    const size_t t0 = (size_t)tok0[k];
    Workspace &w = ps[k].w;
    w.h = (float *)c->h.p + t0 * H;
    w.xn = (char *)c->xn.p + es * t0 * H;
    w.qkv = (char *)c->qkv.p + es * t0 * 3 * H;
    w.ctx = (char *)c->ctxb.p + es * t0 * H;
    w.act = (char *)c->act.p + es * t0 * I;
    w.kinfo = (int *)c->kinfo.p + t0;
    if (fold) {
      w.lpart = (float *)c->fold_part.p + t0 * 2 * (H / kLnPartCols);
      w.lmean1 = (float *)c->fold_mean.p + t0;
      w.lmean2 = (float *)c->fold_mean.p + T + t0;
    }
    ps[k].fold = fold;
    ps[k].ids = d_ids + t0;
    ps[k].pos = d_pos + t0;
    ps[k].opt = d_opt ? d_opt + t0 : nullptr;
    ps[k].s = st[k];
    ps[k].wide_global = true;
    rc = enqueue_prologue(c, ps[k], w.h, w.xn, nullptr, nullptr);
    if (rc) return rc;
  }
  const bool rows_tail = tail_on_rows(c, T_total, R, false);
  const bool rows_layer = rows_tail && rows_layer_fits(c, T_total, R, nseq);
  const int nfull = rows_layer ? L - 1 : L;
  for (int l = 0; l < nfull; l++)
    for (int k = 0; k < 2; k++) {
      rc = enqueue_layer(c, ps[k], l, ps[k].w.h, ps[k].w.h, ps[k].w.h, ps[k].w.xn, nullptr, nullptr,
                         rows_tail && l == L - 1, 0, nullptr, l > 0, l + 1 < nfull);
      if (rc) return rc;
    }
  HIPCHK(c, "hipEventRecord", hipEventRecord(c->ev_join, st[1]));
  HIPCHK(c, "hipStreamWaitEvent", hipStreamWaitEvent(st[0], c->ev_join, 0));
  if (rows_layer) {  // the last layer over the whole batch: its layout from ctx_workspace (taken before the fork)
    float *h_r = nullptr;
    rc = enqueue_rows_layer(c, *wfull, L - 1, (const float *)c->h.p, L == 1 ? c->xn.p : nullptr, d_row_tok, R, &h_r,
                            st[0]);
    if (rc) return rc;
    return enqueue_head(c, h_r, R, nullptr, R, d_logits, (float *)c->head_s1.p, (float *)c->head_d.p, st[0]);
  }
  if (rows_tail) {  // the parts' buffers are views into the shared ones: row_tok indexes them directly
    float *h_r = nullptr;
    rc = enqueue_rows_tail(c, L - 1, c->ctxb.p, (const float *)c->h.p, T_total, d_row_tok, R, c->qkv.p, c->xn.p,
                           c->act.p, &h_r, st[0]);
    if (rc) return rc;
    return enqueue_head(c, h_r, R, nullptr, R, d_logits, (float *)c->head_s1.p, (float *)c->head_d.p, st[0]);
  }
  return enqueue_head(c, (const float *)c->h.p, T_total, d_row_tok, R, d_logits, (float *)c->head_s1.p,
                      (float *)c->head_d.p, st[0]);
}

int forward_core(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *d_ids, const int32_t *d_pos,
                 const int32_t *d_opt, int R, const int32_t *d_row_tok, float *d_logits, bool train,
                 const Workspace *ws) {
  const Config &g = c->cfg;
  const int H = g.hidden, I = g.inter, L = g.layers;
  const size_t es = prec16(g.precision) ? 2 : 4;
  TrainState &tr = c->tr;
  tr.have_forward = false;  // any forward replaces the layout and the encoder output
  if (!ws && !train && c->probe_layer < 0 && nseq >= 2 && c->split_min_tokens > 0) {
    long long T_total = 0;
    for (int i = 0; i < nseq; i++) T_total += seq_len[i];
    if (T_total >= c->split_min_tokens) {
      int first = 0;
      const int cut = split_point(nseq, seq_len, (int)T_total, &first);
      if (first >= kMinPartTokens && T_total - first >= kMinPartTokens) {
        // The option-row last layer runs over the whole batch: its layout comes
        // from the context's workspace (uploaded here, before the fork, when it
        // changes).
        Workspace wf;
        if (tail_on_rows(c, (int)T_total, R, false) && rows_layer_fits(c, (int)T_total, R, nseq)) {
          const int rc = ctx_workspace(c, nseq, seq_len, R, &wf);
          if (rc) return rc;
        }
        return forward_split(c, nseq, seq_len, d_ids, d_pos, d_opt, R, d_row_tok, d_logits, (int)T_total, cut,
                             first, &wf);
      }
    }
  }
  Workspace w;
  int rc = DN_OK;
  if (ws) {
    w = *ws;
  } else {
    rc = ctx_workspace(c, nseq, seq_len, R, &w);
    if (rc) return rc;
  }
  const int T = w.T;
  // The split-K residual GEMMs (partials summed by the next LayerNorm) are an
  // inference path: a training forward's frozen layers keep the whole-K
  // kernels, the summation order of its trainable ones.
  if (train) w.part = nullptr;
  if (train) {
    tr.layers.resize(L);
    for (int l = tr.train_from; l < L; l++) {
      LayerSave &S = tr.layers[l];
      HIPCHK(c, "hipMalloc", ensure(S.hs, sizeof(float) * T * H));
      HIPCHK(c, "hipMalloc", ensure(S.h1, sizeof(float) * T * H));
      HIPCHK(c, "hipMalloc", ensure(S.n1, es * T * H));
      HIPCHK(c, "hipMalloc", ensure(S.qkv, es * T * 3 * H));
      HIPCHK(c, "hipMalloc", ensure(S.ctx, es * T * H));
      HIPCHK(c, "hipMalloc", ensure(S.n2, es * T * H));
      HIPCHK(c, "hipMalloc", ensure(S.wi, es * T * 2 * I));
      HIPCHK(c, "hipMalloc", ensure(S.act, es * T * I));
      HIPCHK(c, "hipMalloc", ensure(S.lse, sizeof(float) * T * g.heads));
      for (DevBuf *b : {&S.mean1, &S.rstd1, &S.mean2, &S.rstd2}) HIPCHK(c, "hipMalloc", ensure(*b, sizeof(float) * T));
    }
    HIPCHK(c, "hipMalloc", ensure(tr.emb_mean, sizeof(float) * T));
    HIPCHK(c, "hipMalloc", ensure(tr.emb_rstd, sizeof(float) * T));
  }
  if (ws && (!c->rope_ready || !c->err_flag.p))
    return fail(c, DN_INVALID_ARG, "decide_hip: set-up incomplete (dn_set_config builds the RoPE tables)");
  rc = ensure_err_flag(c);
  if (rc) return rc;
  rc = ensure_rope(c);
  if (rc) return rc;

  Pass ps;
  ps.w = w;
  ps.ids = d_ids;
  ps.pos = d_pos;
  ps.opt = d_opt;
  ps.s = c->stream;
  ps.fold = !train && w.lpart && fold_eligible(c, T);
  if (ps.fold) {
    rc = ensure_fold_cs(c, ps.s);
    if (rc) return rc;
  }
  // Training keeps each saved layer's input in its own buffer (LayerSave::hs)
  // and its post-attention residual in LayerSave::h1: the residual GEMMs read
  // one and write the next, so the residual stream moves through the saved
  // buffers without copies; unsaved layers update the workspace's h in place.
  auto saved = [&](int l) -> LayerSave * { return train && l >= tr.train_from && l < L ? &tr.layers[l] : nullptr; };
  float *h = w.h;
  float *cur = saved(0) ? (float *)saved(0)->hs.p : h;  // the residual stream entering layer 0
  void *xn0 = saved(0) ? saved(0)->n1.p : w.xn;         // layer 0's QKV input (no attn_norm)
  rc = enqueue_prologue(c, ps, cur, xn0, train ? (float *)tr.emb_mean.p : nullptr,
                        train ? (float *)tr.emb_rstd.p : nullptr);
  if (rc) return rc;
  bool probed = false;
  const bool rows_tail = tail_on_rows(c, T, R, train);
  const bool rows_layer = rows_tail && rows_layer_fits(c, T, R, w.nseq);
  const int nfull = rows_layer ? L - 1 : L;  // layers enqueue_layer runs
  int pending = 0;                           // MlpWo parts not yet in the residual stream
  for (int l = 0; l < nfull; l++) {
    hipEvent_t *ev = ws ? nullptr : probe_slot(c, l);  // the probe creates events: not in a caller's workspace
    probed |= ev != nullptr;
    // Training keeps this layer's activations (layers >= train_from).
    LayerSave *S = saved(l);
    float *in = cur;                                              // this layer's input (S->hs when saved)
    float *h1 = S ? (float *)S->h1.p : in;                        // residual after attention
    float *out = saved(l + 1) ? (float *)saved(l + 1)->hs.p : h;  // the layer's output
    // The last layer's MlpWo completes the residual stream itself (the head
    // or the option-row layer reads it).
    int parts = 0;
    rc = enqueue_layer(c, ps, l, in, h1, out, xn0, S, ev, rows_tail && l == L - 1, pending,
                       !train && l + 1 < nfull ? &parts : nullptr, l > 0, l + 1 < nfull);
    if (rc) return rc;
    pending = parts;
    cur = out;
  }
  if (probed) c->probe_used++;
  if (rows_layer) {
    float *h_r = nullptr;
    rc = enqueue_rows_layer(c, w, L - 1, cur, L == 1 ? xn0 : nullptr, d_row_tok, R, &h_r, ps.s);
    if (rc) return rc;
    rc = enqueue_head(c, h_r, R, nullptr, R, d_logits, w.head_s1, w.head_d, ps.s);
  } else if (rows_tail) {
    float *h_r = nullptr;
    rc = enqueue_rows_tail(c, L - 1, w.ctx, h, T, d_row_tok, R, w.qkv, w.xn, w.act, &h_r, ps.s);
    if (rc) return rc;
    rc = enqueue_head(c, h_r, R, nullptr, R, d_logits, w.head_s1, w.head_d, ps.s);
  } else {
    rc = enqueue_head(c, h, T, d_row_tok, R, d_logits, w.head_s1, w.head_d, ps.s);
  }
  if (rc) return rc;
  if (train) {
    tr.have_forward = true;
    tr.T = T;
    tr.R = R;
  }
  return DN_OK;
}

// The tensor slot `name` when it exists and expects n values; else fails.
int find_slot(dn_ctx *c, const char *name, const void *data, int64_t n, TensorSlot **out) {
  if (!c->configured) return fail(c, DN_INVALID_ARG, "decide_hip: dn_set_config has not been called");
  if (!name || !data) return fail(c, DN_INVALID_ARG, "decide_hip: dn_upload_tensor: NULL argument");
  auto it = c->w.find(name);
  if (it == c->w.end()) return fail(c, DN_INVALID_ARG, std::string("decide_hip: unknown tensor ") + name);
  TensorSlot &t = it->second;
  if (n != t.n)
    return fail(c, DN_INVALID_ARG, std::string("nn: ") + name + " has " + std::to_string(n) +
                                       " values, model expects " + std::to_string(t.n));
  *out = &t;
  return DN_OK;
}

// Wi's value rows [0,I) and gate rows [I,2I) are interleaved in groups of 32:
// stored row 64g+r is value row 32g+r (r < 32) or gate row I+32g+r-32
// (r >= 32).
int64_t wi_src_row(int64_t r, int64_t I) {
  const int64_t g = r / 64, k = r % 64;
  return k < 32 ? 32 * g + k : I + 32 * g + (k - 32);
}

int upload_f32(dn_ctx *c, TensorSlot &t, const float *data, int64_t n) {
  (void)hipSetDevice(c->device);
  const bool bf = t.proj && prec16(c->cfg.precision);
  const bool half = c->cfg.precision == DN_PRECISION_FP16;
  if (bf && half)
    for (int64_t i = 0; i < n; i++)
      if (f16_overflows(data[i]))
        return fail(c, DN_UNSUPPORTED, "decide_hip: a projection weight is outside the fp16 range (|w| >= 65520)");
  uint16_t (*to16)(float) = half ? f32_to_f16_rne : f32_to_bf16_rne;
  const size_t bytes = (size_t)n * (bf ? 2 : 4);
  HIPCHK(c, "hipMalloc", ensure(t.buf, bytes));
  const int64_t H = c->cfg.hidden, I = c->cfg.inter;
  auto src_row = [&](int64_t r) -> int64_t { return t.wi ? wi_src_row(r, I) : r; };
  const int64_t rows = t.wi ? 2 * I : 0;
  t.train.wt_valid = false;
  if (bf) {
    std::vector<uint16_t> tmp((size_t)n);
    std::vector<float> master(c->tr.enabled ? (size_t)n : 0);
    if (t.wi) {
      for (int64_t r = 0; r < rows; r++) {
        const float *s = data + src_row(r) * H;
        for (int64_t k = 0; k < H; k++) tmp[r * H + k] = to16(s[k]);
        if (!master.empty()) std::memcpy(&master[r * H], s, sizeof(float) * H);
      }
    } else {
      for (int64_t i = 0; i < n; i++) tmp[i] = to16(data[i]);
      if (!master.empty()) std::memcpy(master.data(), data, sizeof(float) * n);
    }
    HIPCHK(c, "hipMemcpy", hipMemcpy(t.buf.p, tmp.data(), bytes, hipMemcpyHostToDevice));
    if (!master.empty()) {  // training keeps the fp32 weights the bf16 copy is rounded from
      HIPCHK(c, "hipMalloc", ensure(t.train.master, sizeof(float) * n));
      HIPCHK(c, "hipMemcpy", hipMemcpy(t.train.master.p, master.data(), sizeof(float) * n, hipMemcpyHostToDevice));
    }
  } else if (t.wi) {
    std::vector<float> tmp((size_t)n);
    for (int64_t r = 0; r < rows; r++) std::memcpy(&tmp[r * H], data + src_row(r) * H, sizeof(float) * H);
    HIPCHK(c, "hipMemcpy", hipMemcpy(t.buf.p, tmp.data(), bytes, hipMemcpyHostToDevice));
  } else {
    HIPCHK(c, "hipMemcpy", hipMemcpy(t.buf.p, data, bytes, hipMemcpyHostToDevice));
  }
  t.set = true;
  c->wgen++;
  return DN_OK;
}
// Validation (forward.go:142-196) and staging of a host batch.
int stage_batch(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
                const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, int logits_cap, int *R_out,
                int64_t *T_out) {
  if (nseq < 0 || (nseq > 0 && (!seq_len || !ids || !pos || !nmask)))
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_forward: NULL argument");
  const Config &g = c->cfg;
  // Validation, forward.go:142-196.
  std::vector<int32_t> row_tok;
  int64_t T = 0, mp = 0;
  for (int si = 0; si < nseq; si++) {
    const int n = seq_len[si];
    if (n <= 0) return fail(c, DN_INVALID_ARG, "nn: malformed sequence " + std::to_string(si));
    if (n > 8192) return fail(c, DN_UNSUPPORTED, "decide_hip: sequence " + std::to_string(si) + " is longer than 8192 tokens");
    if (nmask[si] <= 0) return fail(c, DN_INVALID_ARG, "nn: sequence " + std::to_string(si) + " has no options");
    for (int k = 0; k < nmask[si]; k++) {
      const int m = mask_pos[mp + k];
      if (m < 0 || m >= n)
        return fail(c, DN_INVALID_ARG, "nn: sequence " + std::to_string(si) + " mask position " +
                                           std::to_string(m) + " out of range");
      row_tok.push_back((int32_t)(T + m));
    }
    mp += nmask[si];
    T += n;
  }
  if (T > (1 << 30)) return fail(c, DN_UNSUPPORTED, "decide_hip: batch too large");
  for (int64_t t = 0; t < T; t++)
    if (ids[t] < 0 || ids[t] >= g.vocab)
      return fail(c, DN_INVALID_ARG, "nn: token id " + std::to_string(ids[t]) + " out of range");
  // The attention kernel packs (option id + 1, position) into 16 bits each.
  for (int64_t t = 0; t < T; t++) {
    if (pos[t] < 0 || pos[t] > 0xffff)
      return fail(c, DN_UNSUPPORTED, "decide_hip: position id " + std::to_string(pos[t]) + " outside [0, 65535]");
    if (opt_id && (opt_id[t] < -1 || opt_id[t] > 32766))
      return fail(c, DN_UNSUPPORTED, "decide_hip: option id " + std::to_string(opt_id[t]) + " outside [-1, 32766]");
  }
  const int R = (int)row_tok.size();
  *R_out = R;
  if (logits_cap < R) return fail(c, DN_INVALID_ARG, "decide_hip: logits buffer holds fewer than " +
                                                         std::to_string(R) + " values");
  *T_out = T;
  if (T == 0) return DN_OK;
  (void)hipSetDevice(c->device);
  hipStream_t s = c->stream;
  // One pinned staging buffer and one copy for the whole batch: [ids | pos |
  // opt | rowtok] (opt only when given). A call that staged ends by
  // synchronizing its stream (finish_forward); one that failed before that
  // leaves pin_pending set, and the buffer is not rewritten before its copy
  // has finished.
  if (c->pin_pending) {
    HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
    c->pin_pending = false;
  }
  const size_t nin = (size_t)(opt_id ? 3 : 2) * T + R, in_bytes = sizeof(int32_t) * nin;
  const size_t pin_bytes = std::max(in_bytes, sizeof(float) * R + sizeof(int));
  if (c->pin_cap < pin_bytes) {
    if (c->pin) (void)hipHostFree(c->pin);
    c->pin = nullptr;
    c->pin_cap = 0;
    const size_t cap = std::max<size_t>(pin_bytes + pin_bytes / 2, 64 << 10);
    HIPCHK(c, "hipHostMalloc", hipHostMalloc(&c->pin, cap, hipHostMallocDefault));
    c->pin_cap = cap;
  }
  HIPCHK(c, "hipMalloc", ensure(c->io, in_bytes));
  HIPCHK(c, "hipMalloc", ensure(c->logits, sizeof(float) * std::max(R, 1)));
  int rc = ensure_err_flag(c);
  if (rc) return rc;
  int32_t *hp = (int32_t *)c->pin, *dp = (int32_t *)c->io.p;
  std::memcpy(hp, ids, sizeof(int32_t) * T);
  std::memcpy(hp + T, pos, sizeof(int32_t) * T);
  c->d_ids = dp;
  c->d_pos = dp + T;
  size_t off = 2 * (size_t)T;
  c->d_opt = nullptr;
  if (opt_id) {
    std::memcpy(hp + off, opt_id, sizeof(int32_t) * T);
    c->d_opt = dp + off;
    off += T;
  }
  std::memcpy(hp + off, row_tok.data(), sizeof(int32_t) * R);
  c->d_rowtok = dp + off;
  HIPCHK(c, "hipMemsetAsync", hipMemsetAsync(c->err_flag.p, 0, sizeof(int), s));
  c->pin_pending = true;
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(c->io.p, c->pin, in_bytes, hipMemcpyHostToDevice, s));
  return DN_OK;
}

int finish_forward(dn_ctx *c, int R, float *logits) {
  hipStream_t s = c->stream;
  // Logits and the error flag come back through the pinned staging buffer
  // (the batch's copy out of it precedes these on the stream).
  char *hp = (char *)c->pin;
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(hp, c->logits.p, sizeof(float) * R, hipMemcpyDeviceToHost, s));
  HIPCHK(c, "hipMemcpyAsync",
         hipMemcpyAsync(hp + sizeof(float) * R, c->err_flag.p, sizeof(int), hipMemcpyDeviceToHost, s));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
  c->pin_pending = false;
  int flag = 0;
  std::memcpy(&flag, hp + sizeof(float) * R, sizeof(int));
  if (R > 0) std::memcpy(logits, hp, sizeof(float) * R);
  if (flag) return fail(c, DN_DEVICE_ERROR, "decide_hip: device saw an out-of-range index after validation");
  return DN_OK;
}

}  // namespace dnh

extern "C" {

int dn_abi_version(void) { return DN_ABI_VERSION; }

const char *dn_status_string(int status) {
  switch (status) {
    case DN_OK: return "ok";
    case DN_NO_GPU: return "no GPU";
    case DN_INVALID_ARG: return "invalid argument";
    case DN_OUT_OF_MEMORY: return "out of memory";
    case DN_DEVICE_ERROR: return "device error";
    case DN_UNSUPPORTED: return "unsupported";
  }
  return "unknown status";
}

int dn_open(int device, dn_ctx **out) {
  if (!out) return fail(nullptr, DN_INVALID_ARG, "decide_hip: dn_open: out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(nullptr, DN_NO_GPU, std::string("decide_hip: no GPU (") +
                                        (e != hipSuccess ? hipGetErrorString(e) : "0 devices") + ")");
  if (device < 0 || device >= count)
    return fail(nullptr, DN_INVALID_ARG, "decide_hip: device " + std::to_string(device) + " out of range");
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(nullptr, "hipSetDevice", e);
  dn_ctx *c = new dn_ctx;
  c->device = device;
  e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(nullptr, "hipStreamCreate", e);
  }
  c->stream = c->own_stream;
  int rc = noalloc_init(c);
  if (rc) {
    (void)hipStreamDestroy(c->own_stream);
    delete c;
    return rc;
  }
  *out = c;
  return DN_OK;
}

void dn_close(dn_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  close_certify(c);
  for (auto &kv : c->w) release_slot(kv.second);
  release_train(c->tr);
  for (hipEvent_t e : c->probe_pool) (void)hipEventDestroy(e);
  for (hipEvent_t e : c->probe_bwd_pool) (void)hipEventDestroy(e);
  DevBuf *bufs[] = {&c->inv_freq, &c->h,     &c->xn,       &c->qkv,         &c->ctxb,     &c->act,
                    &c->rope,     &c->kinfo, &c->io,
                    &c->logits,   &c->err_flag, &c->gA,    &c->gB,          &c->gC,       &c->d_seq_off, &c->head_s1, &c->head_d,
                    &c->d_seq_len, &c->d_chunk_off, &c->d_chunk_desc, &c->d_work, &c->d_chunks,
                    &c->d_codes,   &c->d_first, &c->calib, &c->smallpart, &c->fold_cs, &c->fold_part,
                    &c->fold_mean};
  for (DevBuf *b : bufs) release(*b);
  if (c->pin) (void)hipHostFree(c->pin);
  for (PartLayout &P : c->parts)
    for (DevBuf *b : {&P.d_seq_off, &P.d_seq_len, &P.d_chunk_off, &P.d_chunk_desc, &P.d_chunks, &P.d_work,
                      &P.d_codes, &P.d_first})
      release(*b);
  if (c->aux_stream) (void)hipStreamSynchronize(c->aux_stream);
  if (c->aux_stream) (void)hipStreamDestroy(c->aux_stream);
  if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
  if (c->ev_join) (void)hipEventDestroy(c->ev_join);
  if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
  delete c;
}

const char *dn_last_error(const dn_ctx *c) { return c ? c->err.c_str() : g_err.c_str(); }

int dn_set_stream(dn_ctx *c, void *stream) {
  if (!c) return DN_INVALID_ARG;
  c->stream = (hipStream_t)stream;
  return DN_OK;
}

int dn_set_config(dn_ctx *c, int hidden, int inter, int heads, int layers, int vocab, float eps, int half_window,
                  double theta_global, double theta_local, const uint8_t *layer_is_sliding, int precision) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (hidden <= 0 || inter <= 0 || heads <= 0 || layers <= 0 || vocab <= 0 || !layer_is_sliding ||
      hidden % heads != 0 || hidden % 2 != 0)
    return fail(c, DN_INVALID_ARG, "nn: incomplete or inconsistent config");
  if (precision != DN_PRECISION_FP32 && precision != DN_PRECISION_BF16 && precision != DN_PRECISION_FP16)
    return fail(c, DN_INVALID_ARG, "decide_hip: unknown precision " + std::to_string(precision));
  close_certify(c);  // a new configuration starts without certification (and its twin)
  // The MFMA kernels take head_dim 64 with hidden % 256 == 0 and intermediate
  // % 64 == 0 (ModernBERT-base); other geometries up to hidden 1024 with head
  // widths 8, 16, 32 or 64 (the reference's own test models among them) run
  // the any-shape GEMM and attention kernels.
  const int hd = hidden / heads;
  const bool fast = hd == 64 && hidden % 256 == 0 && inter % 64 == 0 && hidden <= 1024;
  const bool generic_ok = (hd == 8 || hd == 16 || hd == 32 || hd == 64) && hidden % 8 == 0 && hidden <= 1024;
  if (!fast && !generic_ok)
    return fail(c, DN_UNSUPPORTED, "decide_hip: this build implements hidden <= 1024 with hidden % 8 == 0 and "
                                   "head_dim 8, 16, 32 or 64");
  (void)hipSetDevice(c->device);
  for (auto &kv : c->w) release_slot(kv.second);
  c->w.clear();
  release_train(c->tr);
  c->tr = TrainState();
  Config &g = c->cfg;
  g.hidden = hidden;
  g.inter = inter;
  g.heads = heads;
  g.layers = layers;
  g.vocab = vocab;
  g.eps = eps == 0 ? 1e-5f : eps;
  g.half_window = half_window == 0 ? 64 : half_window;
  g.theta_g = theta_global;
  g.theta_l = theta_local;
  g.sliding.assign(layer_is_sliding, layer_is_sliding + layers);
  g.precision = precision;
  g.generic = !fast;
  define_tensors(c);
  // inv_freq_i = 1 / theta^(2i/D), model.go:244-247, for the D/2 rotation
  // pairs (tables keep 32 columns; narrower heads use the first D/2).
  double inv[64];
  for (int i = 0; i < 32; i++) {
    inv[i] = i < hd / 2 ? 1.0 / std::pow(theta_global, (double)(2 * i) / (double)hd) : 0.0;
    inv[32 + i] = i < hd / 2 ? 1.0 / std::pow(theta_local, (double)(2 * i) / (double)hd) : 0.0;
  }
  HIPCHK(c, "hipMalloc", ensure(c->inv_freq, sizeof(inv)));
  HIPCHK(c, "hipMemcpy", hipMemcpy(c->inv_freq.p, inv, sizeof(inv), hipMemcpyHostToDevice));
  c->rope_ready = false;
  c->configured = true;
  // The folded LayerNorm's column sums (filled from the weights at the first
  // forward that folds, and again after they change).
  release(c->fold_cs);
  c->fold_gen = 0;
  if (fold_geometry(c))
    HIPCHK(c, "hipMalloc", ensure(c->fold_cs, sizeof(float) * (size_t)layers * (3 * hidden + 2 * inter)));
  // Set-up work that forwards would otherwise do on first use: the RoPE
  // tables of these thetas and the device error flag.
  int rc = ensure_rope(c);
  if (rc) return rc;
  rc = ensure_err_flag(c);
  if (rc) return rc;
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  return DN_OK;
}

static int upload_bf16_impl(dn_ctx *c, const char *name, const uint16_t *bits, int64_t n) {
  TensorSlot *t = nullptr;
  int rc = find_slot(c, name, bits, n, &t);
  if (rc) return rc;
  if (!(t->proj && c->cfg.precision == DN_PRECISION_BF16)) {
    // Stored as float32 (widened exactly, safetensors.go:113-124) or, in
    // fp16 mode, as binary16 from the widened values: exact for bf16 values
    // of magnitude 2^-17 .. 65504, nearest-even below that.
    std::vector<float> f((size_t)n);
    for (int64_t i = 0; i < n; i++) {
      const uint32_t u = (uint32_t)bits[i] << 16;
      std::memcpy(&f[i], &u, 4);
    }
    return upload_f32(c, *t, f.data(), n);
  }
  if (c->tr.enabled) {
    // Training keeps fp32 masters: widen exactly and take the float path.
    std::vector<float> f((size_t)n);
    for (int64_t i = 0; i < n; i++) {
      const uint32_t u = (uint32_t)bits[i] << 16;
      std::memcpy(&f[i], &u, 4);
    }
    return upload_f32(c, *t, f.data(), n);
  }
  (void)hipSetDevice(c->device);
  t->train.wt_valid = false;
  HIPCHK(c, "hipMalloc", ensure(t->buf, (size_t)n * 2));
  if (t->wi) {
    const int64_t H = c->cfg.hidden, I = c->cfg.inter;
    std::vector<uint16_t> tmp((size_t)n);
    for (int64_t r = 0; r < 2 * I; r++) std::memcpy(&tmp[r * H], bits + wi_src_row(r, I) * H, 2 * H);
    HIPCHK(c, "hipMemcpy", hipMemcpy(t->buf.p, tmp.data(), (size_t)n * 2, hipMemcpyHostToDevice));
  } else {
    HIPCHK(c, "hipMemcpy", hipMemcpy(t->buf.p, bits, (size_t)n * 2, hipMemcpyHostToDevice));
  }
  t->set = true;
  c->wgen++;
  return DN_OK;
}

int dn_upload_tensor_bf16(dn_ctx *c, const char *name, const uint16_t *bits, int64_t n) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = upload_bf16_impl(c, name, bits, n);
  if (rc || !c->exact) return rc;
  rc = dn_upload_tensor_bf16(c->exact, name, bits, n);  // the certification twin widens to float32
  return rc ? fail(c, rc, c->exact->err) : DN_OK;
}

int dn_upload_tensor(dn_ctx *c, const char *name, const float *data, int64_t n) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  TensorSlot *t = nullptr;
  int rc = find_slot(c, name, data, n, &t);
  if (rc) return rc;
  rc = upload_f32(c, *t, data, n);
  if (rc || !c->exact) return rc;
  rc = dn_upload_tensor(c->exact, name, data, n);  // the certification twin keeps float32
  return rc ? fail(c, rc, c->exact->err) : DN_OK;
}

int dn_weights_ready(const dn_ctx *c) {
  if (!c || !c->configured) return 0;
  for (auto &kv : c->w)
    if (!kv.second.set) return 0;
  return !c->exact || dn_weights_ready(c->exact);
}

int dn_forward(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
               const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, float *logits, int logits_cap) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = check_ready(c);
  if (rc) return rc;
  int R = 0;
  int64_t T = 0;
  rc = stage_batch(c, nseq, seq_len, ids, pos, opt_id, nmask, mask_pos, logits_cap, &R, &T);
  if (rc || T == 0) return rc;
  rc = forward_core(c, nseq, seq_len, c->d_ids, c->d_pos, c->d_opt, R, c->d_rowtok, (float *)c->logits.p, false);
  if (rc) return rc;
  rc = finish_forward(c, R, logits);
  if (rc) return rc;
  return certify_host(c, nseq, seq_len, ids, pos, opt_id, nmask, mask_pos, logits);
}

int dn_forward_device(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *d_ids, const int32_t *d_pos,
                      const int32_t *d_opt_id, int nrows, const int32_t *d_row_tok, float *d_logits) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = check_ready(c);
  if (rc) return rc;
  if (nseq <= 0 || !seq_len || !d_ids || !d_pos || nrows < 0 || (nrows > 0 && (!d_row_tok || !d_logits)))
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_forward_device: bad argument");
  for (int s = 0; s < nseq; s++) {
    if (seq_len[s] <= 0) return fail(c, DN_INVALID_ARG, "nn: malformed sequence " + std::to_string(s));
    if (seq_len[s] > 8192)
      return fail(c, DN_UNSUPPORTED, "decide_hip: sequence " + std::to_string(s) + " is longer than 8192 tokens");
  }
  (void)hipSetDevice(c->device);
  int rc2 = forward_core(c, nseq, seq_len, d_ids, d_pos, d_opt_id, nrows, d_row_tok, d_logits, false);
  if (rc2) return rc2;
  return certify_device(c, nseq, seq_len, d_ids, d_pos, d_opt_id, nrows, d_row_tok, d_logits);
}

int dn_check_device_errors(dn_ctx *c) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (!c->err_flag.p) return DN_OK;
  int flag = 0;
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(&flag, c->err_flag.p, sizeof(int), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  if (flag) {
    HIPCHK(c, "hipMemsetAsync", hipMemsetAsync(c->err_flag.p, 0, sizeof(int), c->stream));
    HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
    if (flag & 4) return fail(c, DN_UNSUPPORTED, "decide_hip: position outside [0, 65535] or option id outside [-1, 32766]");
    return fail(c, DN_INVALID_ARG, (flag & 1) ? "nn: token id out of range" : "nn: mask position out of range");
  }
  return DN_OK;
}

int dn_gemm_f32(dn_ctx *c, int transA, int transB, int M, int N, int K, const float *A, int lda, const float *B,
                int ldb, float *C, int ldc, int accumulate) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (M < 0 || N < 0 || K < 0) return fail(c, DN_INVALID_ARG, "decide_hip: negative GEMM dimension");
  if (M == 0 || N == 0) return DN_OK;
  if (!C || ldc < N) return fail(c, DN_INVALID_ARG, "decide_hip: bad C / ldc");
  if (K > 0) {
    if (!A || !B) return fail(c, DN_INVALID_ARG, "decide_hip: NULL operand");
    if (lda < (transA ? M : K) || ldb < (transB ? K : N))
      return fail(c, DN_INVALID_ARG, "decide_hip: leading dimension too small");
  }
  (void)hipSetDevice(c->device);
  hipStream_t s = c->stream;
  const int Kp = K == 0 ? 32 : (K + 31) / 32 * 32;
  const int Np = (N + 127) / 128 * 128;
  // Stage op(A) as M x Kp and op(B) as Np x Kp (zero padded), the device
  // counterpart of packA/packB (gemm.go:147-195).
  const size_t a_rows = transA ? K : M, a_cols = transA ? M : K;
  const size_t b_rows = transB ? N : K, b_cols = transB ? K : N;
  const size_t a_span = K ? (a_rows - 1) * lda + a_cols : 0, b_span = K ? (b_rows - 1) * ldb + b_cols : 0;
  HIPCHK(c, "hipMalloc", ensure(c->gA, sizeof(float) * (a_span + (size_t)M * Kp)));
  HIPCHK(c, "hipMalloc", ensure(c->gB, sizeof(float) * (b_span + (size_t)Np * Kp)));
  HIPCHK(c, "hipMalloc", ensure(c->gC, sizeof(float) * (size_t)M * N));
  float *rawA = (float *)c->gA.p, *Ap = rawA + a_span;
  float *rawB = (float *)c->gB.p, *Bp = rawB + b_span;
  float *Cd = (float *)c->gC.p;
  if (K) {
    HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(rawA, A, sizeof(float) * a_span, hipMemcpyHostToDevice, s));
    HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(rawB, B, sizeof(float) * b_span, hipMemcpyHostToDevice, s));
  }
  // op(A) is M x K: element (i,k) = transA ? A[k*lda+i] : A[i*lda+k].
  HIPCHK(c, "pack(A)", launch_pack(rawA, transA, M, K, lda, Ap, M, Kp, s));
  // B operand rows are output columns: row j = op(B)[:, j], element (j,k) =
  // transB ? B[j*ldb+k] : B[k*ldb+j].
  HIPCHK(c, "pack(B)", launch_pack(rawB, !transB, N, K, ldb, Bp, Np, Kp, s));
  if (accumulate) {
    HIPCHK(c, "hipMemcpy2DAsync", hipMemcpy2DAsync(Cd, sizeof(float) * N, C, sizeof(float) * ldc,
                                                   sizeof(float) * N, M, hipMemcpyHostToDevice, s));
  }
  GemmArgs a{};
  a.A = Ap;
  a.lda = Kp;
  a.B = Bp;
  a.ldb = Kp;
  a.C = Cd;
  a.ldc = N;
  a.M = M;
  a.N = Np;
  a.K = Kp;
  a.n_store = N;
  a.accumulate = accumulate ? 1 : 0;
  HIPCHK(c, "gemm", launch_gemm(DN_PRECISION_FP32, EPI_F32, a, s));
  HIPCHK(c, "hipMemcpy2DAsync", hipMemcpy2DAsync(C, sizeof(float) * ldc, Cd, sizeof(float) * N, sizeof(float) * N,
                                                 M, hipMemcpyDeviceToHost, s));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
  return DN_OK;
}

int dn_gemm_device(dn_ctx *c, int precision, int M, int N, int K, const void *d_A, const void *d_B, float *d_C,
                   int accumulate) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (precision != DN_PRECISION_FP32 && precision != DN_PRECISION_BF16 && precision != DN_PRECISION_FP16)
    return fail(c, DN_INVALID_ARG, "decide_hip: unknown precision");
  if (M < 0 || !d_A || !d_B || !d_C) return fail(c, DN_INVALID_ARG, "decide_hip: dn_gemm_device: bad argument");
  if (!gemm_shape_ok(precision, N, K))
    return fail(c, DN_UNSUPPORTED, "decide_hip: dn_gemm_device needs N % 128 == 0 and K % 64 (bf16, fp16) / 32 (fp32)");
  (void)hipSetDevice(c->device);
  GemmArgs a{};
  a.A = d_A;
  a.lda = K;
  a.B = d_B;
  a.ldb = K;
  a.C = d_C;
  a.ldc = N;
  a.M = M;
  a.N = N;
  a.K = K;
  a.n_store = N;
  a.accumulate = accumulate ? 1 : 0;
  HIPCHK(c, "gemm", launch_gemm(precision, EPI_F32, a, c->stream));
  return DN_OK;
}

int dn_gemm_device_store(dn_ctx *c, int precision, int M, int N, int K, const void *d_A, const void *d_B, void *d_C) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (precision != DN_PRECISION_BF16 && precision != DN_PRECISION_FP16)
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_gemm_device_store takes 16-bit operands (bf16, fp16)");
  if (M < 0 || !d_A || !d_B || !d_C)
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_gemm_device_store: bad argument");
  if (!gemm_shape_ok(precision, N, K))
    return fail(c, DN_UNSUPPORTED, "decide_hip: dn_gemm_device_store needs N % 128 == 0 and K % 64 == 0");
  (void)hipSetDevice(c->device);
  GemmArgs a{};
  a.A = d_A;
  a.lda = K;
  a.B = d_B;
  a.ldb = K;
  a.C = d_C;
  a.ldc = N;
  a.M = M;
  a.N = N;
  a.K = K;
  a.n_store = N;
  a.skinny_regs = c->cfg.skinny_regs ? 1 : 0;
  HIPCHK(c, "gemm", launch_gemm(precision, EPI_STORE, a, c->stream));
  return DN_OK;
}

int dn_set_stream_split(dn_ctx *c, int min_tokens) {
  if (!c || min_tokens < 0) return DN_INVALID_ARG;
  c->err.clear();
  c->split_min_tokens = min_tokens;
  return DN_OK;
}

int dn_set_small_m_loads(dn_ctx *c, int mode) {
  if (!c || (mode != 0 && mode != 1)) return DN_INVALID_ARG;
  c->cfg.skinny_regs = mode == 0;
  return DN_OK;
}

int dn_set_row_tail(dn_ctx *c, int min_tokens) {
  if (!c || min_tokens < 0) return DN_INVALID_ARG;
  c->err.clear();
  c->tail_min_tokens = min_tokens;
  return DN_OK;
}

int dn_set_ln_fold(dn_ctx *c, int on) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  c->ln_fold = on != 0;
  return DN_OK;
}

int dn_synchronize(dn_ctx *c) {
  if (!c) return DN_INVALID_ARG;
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  return DN_OK;
}

int dn_set_probe(dn_ctx *c, int layer) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (c->probe_used || c->probe_bwd_used) HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  c->probe_layer = layer;
  c->probe_used = 0;
  c->probe_bwd_used = 0;
  // Events for the next kProbeForwards forwards and backwards are created
  // here, so that the calls being timed create none (more grow on demand).
  constexpr size_t kProbeForwards = 128;
  for (auto pool : {std::make_pair(&c->probe_pool, (size_t)10), std::make_pair(&c->probe_bwd_pool, (size_t)6)})
    while (layer >= 0 && pool.first->size() < kProbeForwards * pool.second) {
      hipEvent_t e;
      HIPCHK(c, "hipEventCreate", hipEventCreate(&e));
      pool.first->push_back(e);
    }
  return DN_OK;
}

int dn_read_probe_backward(dn_ctx *c, double *ms, int *count) {
  if (!c || !ms || !count) return DN_INVALID_ARG;
  c->err.clear();
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  if (c->tr.side) HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->tr.side));
  for (int f = 0; f < c->probe_bwd_used; f++)
    for (int k = 0; k < 3; k++) {
      float t = 0;
      HIPCHK(c, "hipEventElapsedTime", hipEventElapsedTime(&t, c->probe_bwd_pool[(size_t)f * 6 + 2 * k],
                                                           c->probe_bwd_pool[(size_t)f * 6 + 2 * k + 1]));
      ms[k] += t;
    }
  *count += c->probe_bwd_used;
  c->probe_bwd_used = 0;
  return DN_OK;
}

int dn_read_probe(dn_ctx *c, double *ms, int *count) {
  if (!c || !ms || !count) return DN_INVALID_ARG;
  c->err.clear();
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  for (int f = 0; f < c->probe_used; f++)
    for (int k = 0; k < 5; k++) {
      float t = 0;
      HIPCHK(c, "hipEventElapsedTime",
             hipEventElapsedTime(&t, c->probe_pool[(size_t)f * 10 + 2 * k], c->probe_pool[(size_t)f * 10 + 2 * k + 1]));
      ms[k] += t;
    }
  *count += c->probe_used;
  c->probe_used = 0;
  return DN_OK;
}

int dn_mfma_calibrate(dn_ctx *c, int mode, double *tflops) {
  if (!c || !tflops || mode < 0 || mode > 5) return DN_INVALID_ARG;
  c->err.clear();
  (void)hipSetDevice(c->device);
  int cus = 0;
  HIPCHK(c, "hipDeviceGetAttribute", hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->device));
  HIPCHK(c, "hipMalloc", ensure(c->calib, 256 * sizeof(float)));
  hipEvent_t e0, e1;
  HIPCHK(c, "hipEventCreate", hipEventCreate(&e0));
  hipError_t err = hipEventCreate(&e1);
  if (err != hipSuccess) {
    (void)hipEventDestroy(e0);
    return hip_fail(c, "hipEventCreate", err);
  }
  // Two 4-wave blocks per CU (two waves per SIMD, as the GEMMs run); a short
  // launch first so the timed one starts at the loaded clock.
  const int blocks = 2 * cus, iters = 6000;
  float ms = 0;
  err = launch_mfma_calibrate(mode, blocks, iters / 4, (float *)c->calib.p, c->stream);
  if (err == hipSuccess) err = hipEventRecord(e0, c->stream);
  if (err == hipSuccess) err = launch_mfma_calibrate(mode, blocks, iters, (float *)c->calib.p, c->stream);
  if (err == hipSuccess) err = hipEventRecord(e1, c->stream);
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (err != hipSuccess) return hip_fail(c, "mfma_calibrate", err);
  *tflops = ms > 0 ? mfma_calibrate_flop(mode, blocks, iters) / (ms * 1e-3) / 1e12 : 0.0;
  return DN_OK;
}

int dn_build_sequence(const int32_t *ids, int n, int32_t mask_id, int independent, int32_t *pos, int32_t *opt_id,
                      int32_t *mask_pos, int *has_opt) {
  if (n < 0 || (n > 0 && (!ids || !pos || !mask_pos)) || !has_opt) return -1;
  int nm = 0;
  for (int i = 0; i < n; i++) {
    pos[i] = i;
    if (ids[i] == mask_id) mask_pos[nm++] = i;
  }
  *has_opt = 0;
  if (!independent || nm == 0) return nm;
  if (!opt_id) return -1;
  // The trailing token (the final [SEP]) belongs to no option; options
  // restart their positions right after the prefix (forward.go:39-54).
  const int last = n - 1, prefix = mask_pos[0];
  for (int i = 0; i < n; i++) opt_id[i] = -1;
  for (int k = 0; k < nm; k++) {
    const int start = mask_pos[k], end = k + 1 < nm ? mask_pos[k + 1] : last;
    for (int i = start; i < end; i++) {
      opt_id[i] = k;
      pos[i] = prefix + i - start;
    }
  }
  *has_opt = 1;
  return nm;
}

double dn_round(double x, int places) {
  const double p = std::pow(10.0, (double)places);
  return std::nearbyint(x * p) / p;
}

int dn_answer(const double *logits, int k, double temperature, double *probs, int *choice, double *confidence) {
  if (k <= 0 || !logits || !probs || !choice || !confidence) return DN_INVALID_ARG;
  // calibrated + softmax (local.go:206-232).
  const double t = std::fmax(temperature, 1e-4);
  double maxv = -INFINITY;
  for (int i = 0; i < k; i++) maxv = std::fmax(maxv, logits[i] / t);
  double sum = 0;
  for (int i = 0; i < k; i++) {
    probs[i] = std::exp(logits[i] / t - maxv);
    sum += probs[i];
  }
  for (int i = 0; i < k; i++) probs[i] /= sum;
  // argmax of raw logits, first index wins ties (local.go:254-262).
  int best = 0;
  for (int i = 0; i < k; i++)
    if (logits[i] > logits[best]) best = i;
  *choice = best;
  // marginConfidence (local.go:241-252).
  if (k <= 1) {
    *confidence = 1.0;
  } else {
    double pmax = 0;
    for (int i = 0; i < k; i++) pmax = std::fmax(pmax, probs[i]);
    const double cf = ((double)k * pmax - 1) / (double)(k - 1);
    *confidence = dn_round(std::fmax(0.0, std::fmin(1.0, cf)), 3);
  }
  return DN_OK;
}

int dn_evaluate(dn_ctx *c, int nq, const int32_t *kind, const int32_t *n_opt, const int32_t *q_len,
                const int32_t *ids, const double *temperature, int32_t mask_id, int independent, double *probs,
                int32_t *choice, double *confidence, double *value) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (nq < 0 || (nq > 0 && (!kind || !n_opt || !q_len || !temperature || !choice || !confidence || !value)))
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_evaluate: NULL argument");
  // Pass 1, in question order as Local.Evaluate walks them (local.go:126-150):
  // the checks of rawLogits (local.go:185-192) and the batch layout.
  std::vector<int32_t> seq_len, bpos, bopt, nmask, mpos, bids;
  std::vector<int> fwd_q;  // question of each forwarded sequence
  int64_t off = 0, nprob = 0;
  for (int q = 0; q < nq; q++) {
    const int k = n_opt[q], kd = kind[q], n = q_len[q];
    const std::string where = "decide: question " + std::to_string(q) + ": ";
    if (kd < DN_KIND_CHOICE || kd > DN_KIND_NOUL) return fail(c, DN_INVALID_ARG, where + "unsupported question kind");
    if (k < 0 || n < 0) return fail(c, DN_INVALID_ARG, where + "negative option or token count");
    if (kd == DN_KIND_NOUL && k != 2) return fail(c, DN_INVALID_ARG, where + "a Noul has exactly two options");
    if (n > 0 && !ids) return fail(c, DN_INVALID_ARG, "decide_hip: dn_evaluate: NULL argument");
    if (kd == DN_KIND_NOUL || k >= 2) {  // k <= 1 skips the model (local.go:285-287, :310-312)
      if (n > 8192)
        return fail(c, DN_INVALID_ARG, where + "input is " + std::to_string(n) + " tokens; the limit is 8192");
      const size_t t0 = bpos.size(), m0 = mpos.size();
      bpos.resize(t0 + n);
      bopt.resize(t0 + n, -1);
      mpos.resize(m0 + n);
      int has_opt = 0;
      const int nm = dn_build_sequence(ids + off, n, mask_id, independent, bpos.data() + t0, bopt.data() + t0,
                                       mpos.data() + m0, &has_opt);
      if (nm != k) return fail(c, DN_INVALID_ARG, where + "input contains the reserved [MASK] token");
      mpos.resize(m0 + nm);
      bids.insert(bids.end(), ids + off, ids + off + n);
      seq_len.push_back(n);
      nmask.push_back(nm);
      fwd_q.push_back(q);
    }
    off += n;
    nprob += k;
  }
  if (nprob > 0 && !probs) return fail(c, DN_INVALID_ARG, "decide_hip: dn_evaluate: NULL argument");
  // One forward for every question that needs the model.
  std::vector<float> logits(mpos.size());
  if (!seq_len.empty()) {
    const int rc = dn_forward(c, (int)seq_len.size(), seq_len.data(), bids.data(), bpos.data(),
                              independent ? bopt.data() : nullptr, nmask.data(), mpos.data(), logits.data(),
                              (int)logits.size());
    if (rc) return rc;
  }
  // Pass 2: evalChoice / evalScore / evalNoul after the forward
  // (local.go:264-356), logits widened to float64 (local.go:199-203).
  std::vector<int64_t> lg_off((size_t)nq, -1);
  for (size_t i = 0, r = 0; i < fwd_q.size(); r += nmask[i], i++) lg_off[fwd_q[i]] = (int64_t)r;
  std::vector<double> lg, pr;
  for (int q = 0, po = 0; q < nq; po += n_opt[q], q++) {
    const int k = n_opt[q], kd = kind[q];
    double *pq = probs ? probs + po : nullptr;
    choice[q] = -1;
    confidence[q] = 0;
    value[q] = 0;
    if (k == 0) continue;  // empty answer
    pr.assign((size_t)k, 1.0);
    int ch = 0;
    double cf = 1.0;
    if (lg_off[q] >= 0) {
      lg.assign(logits.begin() + lg_off[q], logits.begin() + lg_off[q] + k);
      dn_answer(lg.data(), k, temperature[q], pr.data(), &ch, &cf);
    }
    if (kd == DN_KIND_CHOICE) {
      choice[q] = ch;
      confidence[q] = cf;
    } else if (kd == DN_KIND_SCORE) {
      double expect = 0;
      for (int i = 0; i < k; i++) expect += (double)i * pr[i];
      value[q] = dn_round(expect, 2);
      confidence[q] = cf;
    } else {
      value[q] = dn_round(std::fmax(0.0, std::fmin(1.0, pr[0])), 4);
    }
    for (int i = 0; i < k; i++) pq[i] = dn_round(pr[i], 4);
  }
  return DN_OK;
}

}  // extern "C"
