// C ABI of the training path: the device half of the reference's gpunn
// engine (internal/gpunn/model.go) with the scorer head on the device too,
// following nn.(*Model).Backward (internal/nn/backward.go:19-115) step for
// step, and AdamW (internal/train/optim.go). Declarations and the reference
// interfaces each entry point replaces are in include/decide_hip.h.
//
// Per layer, from the top (dout = gradient of the layer output, fp32):
//   dact = dout . MlpWo            gMlpWo += dout^T . act
//   dwi  = GeGLU'(dact, wi)        gWi    += dwi^T . n2       dn2 = dwi . Wi
//          (in the dact GEMM's epilogue, dact is never stored)
//   dh1  = dout + LNbwd(dn2)       (mlp_norm)
//   dctx = dh1 . Wo                gWo    += dh1^T . ctx
//   dqkv = attention backward (RoPE inverse on dq, dk)
//   gWqkv += dqkv^T . n1           dn1 = dqkv . Wqkv
//   dprev = dh1 + LNbwd(dn1)       (attn_norm; layer 0: dh1 + dn1)
// Input-gradient GEMMs run on the forward GEMM kernel with a transposed copy
// of the weights; weight-gradient GEMMs (a reduction over tokens) run split-K
// on transposed operand copies, with partial products summed in split order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <numeric>
#include <string>
#include <vector>

#include "ctx.hpp"

using namespace dnh;

namespace {

const char *kTok = "model.embeddings.tok_embeddings.weight";
const char *kEmbNorm = "model.embeddings.norm.weight";

// Frozen tensors (SetTrainable, internal/gpunn/model.go:155-171; NewAdamW,
// internal/train/optim.go:36-53).
bool frozen(const TrainState &tr, const std::string &name) {
  if (name == kTok) return !tr.train_emb || tr.train_from > 0;
  if (name == kEmbNorm) return tr.train_from > 0;
  if (name.rfind("model.layers.", 0) == 0) {
    int l = 0;
    for (size_t i = 13; i < name.size() && name[i] >= '0' && name[i] <= '9'; i++) l = l * 10 + (name[i] - '0');
    return l < tr.train_from;
  }
  return false;
}

bool bf16_slot(const dn_ctx *c, const TensorSlot &t) { return t.proj && c->cfg.precision == DN_PRECISION_BF16; }

// fp32 weights of a slot: the master copy for bf16 projections, else the slot.
float *param(dn_ctx *c, TensorSlot &t) { return (float *)(bf16_slot(c, t) ? t.train.master.p : t.buf.p); }

int alloc_zero(dn_ctx *c, DevBuf &b, size_t bytes) {
  if (b.p && b.cap >= bytes) return DN_OK;
  release(b);
  HIPCHK(c, "hipMalloc", ensure(b, bytes));
  HIPCHK(c, "hipMemsetAsync", hipMemsetAsync(b.p, 0, bytes, c->stream));
  return DN_OK;
}

int ensure_param_state(dn_ctx *c) {
  for (auto &kv : c->w) {
    ParamTrain &p = kv.second.train;
    const size_t bytes = sizeof(float) * kv.second.n;
    int rc = alloc_zero(c, p.grad, bytes);
    if (!rc) rc = alloc_zero(c, p.m, bytes);
    if (!rc) rc = alloc_zero(c, p.v, bytes);
    if (rc) return rc;
    if (bf16_slot(c, kv.second) && !p.master.p)
      return fail(c, DN_INVALID_ARG, "decide_hip: " + kv.first + " was uploaded before dn_enable_training");
  }
  return DN_OK;
}

// Input width of a projection (its stored layout is [out x in]).
int64_t proj_in(const dn_ctx *c, const std::string &name) {
  const size_t n = name.size(), k = std::string("mlp.Wo.weight").size();
  return n >= k && name.compare(n - k, k, "mlp.Wo.weight") == 0 ? c->cfg.inter : c->cfg.hidden;
}

// The transposed operand copy [in x out] of a projection, from its fp32 weights.
int refresh_wt(dn_ctx *c, const std::string &name, TensorSlot &t) {
  if (t.train.wt_valid) return DN_OK;
  const int prec = c->cfg.precision;
  const int64_t in = proj_in(c, name), out = t.n / in;
  HIPCHK(c, "hipMalloc", ensure(t.train.wt, (size_t)t.n * (prec == DN_PRECISION_BF16 ? 2 : 4)));
  HIPCHK(c, "transpose(W)", launch_transpose(0, prec, param(c, t), (int)out, (int)in, (int)in, t.train.wt.p,
                                             (int)out, (int)out, nullptr, c->stream));
  t.train.wt_valid = true;
  return DN_OK;
}

// Splits of the token (K) dimension for a weight-gradient GEMM: about 200
// workgroups of 64 x 128 (bf16) or 512 of 128 x 128 (fp32) in all, while each
// split keeps at least 512 tokens of K; the partial outputs cost splits x M x N
// floats of extra traffic. (Isolated bf16 launches at 3840 tokens: dWqkv
// 36.7 us as 128 x 128 tiles x 4 splits, 24.8 us as 64 x 128 tiles unsplit.)
int split_count(int prec, int M, int N, int Tp) {
  const bool bf = prec == DN_PRECISION_BF16;
  const int tiles = ((M + (bf ? 63 : 127)) / (bf ? 64 : 128)) * (N / 128);
  const int target = bf ? 200 : 512;
  const int kb = Tp / 64;
  int s = std::min({16, std::max(1, (target + tiles - 1) / tiles), std::max(1, kb / 8)});
  while (s > 1 && kb % s) s--;
  return s;
}

#define RCX(expr)         \
  do {                    \
    int rcx_ = (expr);    \
    if (rcx_) return rcx_; \
  } while (0)

struct Bwd {
  dn_ctx *c;
  int prec, T, Tp, H, I, heads;
  size_t es;
  hipStream_t s;

  // C[M x N] (epi) = A[M x K] . B[N x K]^T on the forward GEMM kernel.
  int gemm(int epi, int M, int N, int K, const void *A, int lda, const void *B, int ldb, void *C, int ldc) {
    GemmArgs a{};
    a.A = A;
    a.lda = lda;
    a.B = B;
    a.ldb = ldb;
    a.C = C;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    a.n_store = N;
    HIPCHK(c, "gemm", launch_gemm(prec, epi, a, s));
    return DN_OK;
  }
  // G[M x N] += A^T . B over the tokens, from the transposed copies At [M x Tp]
  // and Bt [N x Tp], on stream ws.
  int wgrad(int M, int N, const void *At, const void *Bt, float *G, hipStream_t ws) {
    GemmArgs a{};
    a.A = At;
    a.lda = Tp;
    a.B = Bt;
    a.ldb = Tp;
    a.C = G;
    a.M = M;
    a.N = N;
    a.K = Tp;
    a.accumulate = 1;
    const int sp = split_count(prec, M, N, Tp);
    if (sp == 1) {  // one split: accumulate straight into the gradient
      a.ldc = N;
      a.n_store = N;
      HIPCHK(c, "gemm", launch_gemm(prec, EPI_F32, a, ws));
      return DN_OK;
    }
    HIPCHK(c, "gemm(split-K)", launch_gemm_splitk(prec, a, sp, (float *)c->tr.part.p, ws));
    return DN_OK;
  }
  // dst [cols x Tp] = src[T x cols]^T in the operand type (zero past T); with
  // copy, also the operand-type copy of an fp32 src.
  int transpose(int prec_in, const void *src, int cols, void *dst, void *copy = nullptr, hipStream_t ts = nullptr) {
    HIPCHK(c, "transpose", launch_transpose(prec_in, prec, src, T, cols, cols, dst, Tp, Tp, copy, ts ? ts : s));
    return DN_OK;
  }
  // Several such transposes {prec_in, src, cols, dst} in one launch when
  // every width is a multiple of 64, else one launch each.
  struct Job {
    int prec_in;
    const void *src;
    int cols;
    void *dst;
  };
  int transposes(std::initializer_list<Job> jobs, hipStream_t ts) {
    bool batch = jobs.size() <= (size_t)TB_MAX;
    for (const Job &j : jobs) batch = batch && j.cols % 64 == 0;
    if (!batch) {
      for (const Job &j : jobs) RCX(transpose(j.prec_in, j.src, j.cols, j.dst, nullptr, ts));
      return DN_OK;
    }
    TransposeBatch tb{};
    for (const Job &j : jobs) tb.job[tb.n++] = TransposeJob{j.src, j.dst, j.cols, j.prec_in == 0 ? 1 : 0, 0};
    tb.rows = T;
    tb.rows_pad = Tp;
    tb.ldt = Tp;
    HIPCHK(c, "transpose(batch)", launch_transpose_batch(tb, prec, ts));
    return DN_OK;
  }
};

#define RC(expr)              \
  do {                        \
    int rc_ = (expr);         \
    if (rc_) return rc_;      \
  } while (0)

// Event pair slots for the backward probe of layer l (null when not probed).
hipEvent_t *probe_bwd_slot(dn_ctx *c, int l) {
  if (c->probe_layer != l) return nullptr;
  const size_t need = (size_t)(c->probe_bwd_used + 1) * 6;
  while (c->probe_bwd_pool.size() < need) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    c->probe_bwd_pool.push_back(e);
  }
  return &c->probe_bwd_pool[(size_t)c->probe_bwd_used * 6];
}

int backward_impl(dn_ctx *c, const float *dlogits) {
  const Config &g = c->cfg;
  TrainState &tr = c->tr;
  const int H = g.hidden, I = g.inter, L = g.layers, T = tr.T, R = tr.R;
  const int prec = g.precision;
  const size_t es = prec == DN_PRECISION_BF16 ? 2 : 4;
  const int Tp = (T + 63) / 64 * 64;
  hipStream_t s = c->stream;
  Bwd b{c, prec, T, Tp, H, I, g.heads, es, s};
  auto grad = [&](const std::string &name) { return (float *)c->w.at(name).train.grad.p; };
  auto wt = [&](const std::string &name) -> const void * { return c->w.at(name).train.wt.p; };

  // Workspace.
  const size_t TH = (size_t)T * H;
  HIPCHK(c, "hipMalloc", ensure(tr.dcur, 4 * TH));
  HIPCHK(c, "hipMalloc", ensure(tr.dprev, 4 * TH));
  for (int q = 0; q < 2; q++) {
    HIPCHK(c, "hipMalloc", ensure(tr.dh1[q], 4 * TH));
    HIPCHK(c, "hipMalloc", ensure(tr.dwi[q], es * T * 2 * I));
    HIPCHK(c, "hipMalloc", ensure(tr.dqkv[q], es * T * 3 * H));
  }
  HIPCHK(c, "hipMalloc", ensure(tr.dn2, 4 * TH));
  HIPCHK(c, "hipMalloc", ensure(tr.dn1, 4 * TH));
  // dact only when the GeGLU backward cannot run in the GEMM's epilogue.
  if (!gemm_epi_ok(prec, EPI_GEGLU_BWD, T)) HIPCHK(c, "hipMalloc", ensure(tr.dact, 4 * (size_t)T * I));
  HIPCHK(c, "hipMalloc", ensure(tr.dctx, es * TH));
  HIPCHK(c, "hipMalloc", ensure(tr.dop_out, es * TH));
  HIPCHK(c, "hipMalloc", ensure(tr.dop_h1, es * TH));
  // Transposed operands of one layer's weight-gradient GEMMs: dout, act, dwi,
  // n2, dh1, ctx, dqkv, n1 (rows of Tp tokens), one arena per layer parity.
  const size_t opT_rows = (size_t)8 * H + 3 * I;
  for (int q = 0; q < 2; q++) HIPCHK(c, "hipMalloc", ensure(tr.opT[q], es * opT_rows * Tp));
  if (!tr.side) {
    HIPCHK(c, "hipStreamCreate", hipStreamCreateWithFlags(&tr.side, hipStreamNonBlocking));
    for (int q = 0; q < 2; q++) {
      HIPCHK(c, "hipEventCreate", hipEventCreateWithFlags(&tr.ev_ready[q], hipEventDisableTiming));
      HIPCHK(c, "hipEventCreate", hipEventCreateWithFlags(&tr.ev_done[q], hipEventDisableTiming));
      HIPCHK(c, "hipEventCreate", hipEventCreateWithFlags(&tr.ev_trans[q], hipEventDisableTiming));
    }
  }
  // Nothing of an earlier call may still use the arenas, buffers or partials.
  for (int q = 0; q < 2; q++) {
    HIPCHK(c, "hipEventRecord", hipEventRecord(tr.ev_done[q], tr.side));
    HIPCHK(c, "hipEventRecord", hipEventRecord(tr.ev_trans[q], tr.side));
  }
  HIPCHK(c, "hipMalloc", ensure(tr.dsum, 4 * (size_t)T * g.heads));
  // split-K partials: weight gradients (<= 16 splits) and input gradients (<= 4 splits of T x max(H, I))
  HIPCHK(c, "hipMalloc", ensure(tr.part, 4 * std::max((size_t)16 * std::max({(size_t)3 * H * H, (size_t)2 * I * H,
                                                                             (size_t)H * I}),
                                                        (size_t)4 * T * std::max(H, I))));
  // LayerNorm weight-gradient partials: one slot per (layer parity, norm);
  // their column sums run on the weight-gradient stream.
  const size_t lnslot = (size_t)ln_bwd_blocks(std::max(T, R)) * H;
  HIPCHK(c, "hipMalloc", ensure(tr.lnpart, 4 * 4 * lnslot));
  HIPCHK(c, "hipMalloc", ensure(tr.dl, 4 * (size_t)std::max(R, 1)));
  HIPCHK(c, "hipMalloc", ensure(tr.contrib, 4 * (size_t)std::max(R, 1) * 5 * H));
  for (int l = tr.train_from; l < L; l++) {
    const std::string p = layer_prefix(l);
    for (const char *w : {"attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight"})
      RC(refresh_wt(c, p + w, c->w.at(p + w)));
  }

  // Head (HeadBackward, backward.go:161-196) into the [MASK] rows of dcur.
  float *dcur = (float *)tr.dcur.p, *dprev = (float *)tr.dprev.p;
  HIPCHK(c, "hipMemsetAsync", hipMemsetAsync(dcur, 0, 4 * TH, s));
  HIPCHK(c, "hipMemcpyAsync",
         hipMemcpyAsync(tr.dl.p, dlogits, sizeof(float) * R, hipMemcpyHostToDevice, s));
  const float *hw[7] = {(const float *)W(c, "model.final_norm.weight"), (const float *)W(c, "scorer.input_norm.weight"),
                        (const float *)W(c, "scorer.dense.weight"),     (const float *)W(c, "scorer.dense.bias"),
                        (const float *)W(c, "scorer.norm.weight"),      (const float *)W(c, "scorer.norm.bias"),
                        (const float *)W(c, "scorer.out_proj.weight")};
  float *hg[9] = {grad("scorer.out_proj.weight"), grad("scorer.norm.weight"),  grad("scorer.norm.bias"),
                  grad("scorer.dense.bias"),      grad("scorer.dense.weight"), grad("scorer.input_norm.weight"),
                  grad("scorer.input_norm.bias"), grad("model.final_norm.weight"), grad("scorer.out_proj.bias")};
  HIPCHK(c, "head_bwd", launch_head_bwd((const float *)c->h.p, c->d_rowtok, (const float *)c->head_s1.p,
                                        (const float *)c->head_d.p, (const float *)tr.dl.p, R, H, g.eps, hw, dcur,
                                        (float *)tr.contrib.p, hg, s));

  const float *rope = (const float *)c->rope.p;
  const size_t nw = (size_t)c->lay_nwork;
  float *dn2 = (float *)tr.dn2.p, *dn1 = (float *)tr.dn1.p, *dact = (float *)tr.dact.p;
  const bool bf = prec == DN_PRECISION_BF16;
  const bool fuse_geglu = gemm_epi_ok(prec, EPI_GEGLU_BWD, T);
  float *lnpart = (float *)tr.lnpart.p;
  for (int l = L - 1; l >= tr.train_from && l >= 0; l--) {
    const std::string p = layer_prefix(l);
    const LayerSave &S = tr.layers[l];
    const bool sliding = g.sliding[l] != 0;
    const int par = l & 1;
    hipEvent_t *ev = probe_bwd_slot(c, l);
    auto mark = [&](int k, int end, hipStream_t st) -> int {
      if (ev) HIPCHK(c, "hipEventRecord", hipEventRecord(ev[2 * k + end], st));
      return DN_OK;
    };
    // This parity's gradient buffers and LayerNorm partials are free once
    // the weight-gradient stream has read layer l+2's; that stream alone
    // writes the arenas after the top layer (whose arena write is ordered by
    // the records at entry).
    HIPCHK(c, "hipStreamWaitEvent", hipStreamWaitEvent(s, tr.ev_trans[par], 0));
    char *arena = (char *)tr.opT[par].p;
    size_t row0 = 0;
    auto slice = [&](int rows) {
      void *q = arena + es * row0 * Tp;
      row0 += rows;
      return q;
    };
    void *doutT = slice(H), *actT = slice(I), *dwiT = slice(2 * I), *n2T = slice(H), *dh1T = slice(H),
         *ctxT = slice(H), *dqkvT = slice(3 * H), *n1T = slice(H);
    float *dh1 = (float *)tr.dh1[par].p;
    void *dwi = tr.dwi[par].p, *dqkv = tr.dqkv[par].p;
    const bool top = l == L - 1;
    // dout (fp32) as an operand: in bf16 its rounded copy, written by the
    // layer above's LN backward (for the top layer, by this transpose, which
    // also gives its transposed copy; lower layers' transposes run on the
    // weight-gradient stream).
    if (top) RC(b.transpose(0, dcur, H, doutT, bf ? tr.dop_out.p : nullptr));
    const void *dout_op = bf ? tr.dop_out.p : (const void *)dcur;

    // MLP: out = h1 + MlpWo(act)
    if (fuse_geglu) {  // dwi straight from the GEMM's epilogue
      GemmArgs ga{};
      ga.A = dout_op;
      ga.lda = H;
      ga.B = wt(p + "mlp.Wo.weight");
      ga.ldb = H;
      ga.C = dwi;
      ga.ldc = 2 * I;
      ga.M = T;
      ga.N = I;
      ga.K = H;
      ga.n_store = I;
      ga.gin = S.wi.p;
      HIPCHK(c, "gemm(geglu_bwd)", launch_gemm(prec, EPI_GEGLU_BWD, ga, s));
    } else {
      RC(b.gemm(EPI_F32, T, I, H, dout_op, H, wt(p + "mlp.Wo.weight"), H, dact, I));
      HIPCHK(c, "geglu_bwd", launch_geglu_bwd(prec, dact, S.wi.p, dwi, T, I, s));
    }
    RC(b.gemm(EPI_F32, T, H, 2 * I, dwi, 2 * I, wt(p + "mlp.Wi.weight"), 2 * I, dn2, H));
    float *lnp_mlp = lnpart + (size_t)(2 * par) * lnslot, *lnp_attn = lnp_mlp + lnslot;
    HIPCHK(c, "ln_bwd(mlp_norm)", launch_ln_bwd(dh1, dcur, dn2, (const float *)S.h1.p, nullptr,
                                                (const float *)S.mean2.p, (const float *)S.rstd2.p,
                                                (const float *)W(c, p + "mlp_norm.weight"), g.eps, T, H, lnp_mlp,
                                                nullptr, s, bf ? tr.dop_h1.p : nullptr));

    // Attention: h1 = in + Wo(ctx)
    const void *dh1_op = bf ? tr.dop_h1.p : (const void *)dh1;
    RC(b.gemm(EPI_STORE, T, H, H, dh1_op, H, wt(p + "attn.Wo.weight"), H, tr.dctx.p, H));

    AttnBwdArgs at{};
    at.qkv = S.qkv.p;
    at.ctx = S.ctx.p;
    at.dctx = tr.dctx.p;
    at.lse = (const float *)S.lse.p;
    at.dsum = (float *)tr.dsum.p;
    at.dqkv = dqkv;
    at.kinfo = (const int *)c->kinfo.p;
    at.cos_t = rope + (size_t)(sliding ? 2 : 0) * kPositions * 32;
    at.sin_t = rope + (size_t)(sliding ? 3 : 1) * kPositions * 32;
    at.work = (const int4 *)c->d_work.p;
    at.codes = (const uint32_t *)c->d_codes.p + (sliding ? nw * ATTN_MAXKT : 0);
    at.first = (const int *)c->d_first.p + (sliding ? nw : 0);
    at.seq_off = (const int *)c->d_seq_off.p;
    at.seq_len = (const int *)c->d_seq_len.p;
    at.chunks = (const ChunkInfo *)c->d_chunks.p;
    at.chunk_off = (const int *)c->d_chunk_off.p;
    at.nwork = c->lay_nwork;
    at.H = H;
    at.heads = g.heads;
    at.sliding = sliding ? 1 : 0;
    at.half_window = g.half_window;
    at.scale = (float)(1.0 / std::sqrt(64.0));
    at.scale_log2 = at.scale * 1.44269504088896340736f;
    RC(mark(DN_PROBE_BWD_ATTENTION, 0, s));
    HIPCHK(c, "attention_bwd", launch_attention_bwd(prec, at, s));
    RC(mark(DN_PROBE_BWD_ATTENTION, 1, s));

    RC(mark(DN_PROBE_BWD_DGRAD_QKV, 0, s));
    RC(b.gemm(EPI_F32, T, H, 3 * H, dqkv, 3 * H, wt(p + "attn.Wqkv.weight"), 3 * H, dn1, H));
    RC(mark(DN_PROBE_BWD_DGRAD_QKV, 1, s));
    // dprev held the layer above's dout: its transpose must be done.
    HIPCHK(c, "hipStreamWaitEvent", hipStreamWaitEvent(s, tr.ev_trans[par ^ 1], 0));
    if (l > 0) {
      HIPCHK(c, "ln_bwd(attn_norm)", launch_ln_bwd(dprev, dh1, dn1, (const float *)S.hs.p, nullptr,
                                                   (const float *)S.mean1.p, (const float *)S.rstd1.p,
                                                   (const float *)W(c, p + "attn_norm.weight"), g.eps, T, H, lnp_attn,
                                                   nullptr, s, bf ? tr.dop_out.p : nullptr));
    } else {
      HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(dprev, dh1, 4 * TH, hipMemcpyDeviceToDevice, s));
      HIPCHK(c, "add", launch_add(dprev, dn1, TH, s));
    }
    // The layer's weight gradients on the side stream, overlapping the next
    // layer's input-gradient chain.
    HIPCHK(c, "hipEventRecord", hipEventRecord(tr.ev_ready[par], s));
    HIPCHK(c, "hipStreamWaitEvent", hipStreamWaitEvent(tr.side, tr.ev_ready[par], 0));
    // The gradients' transposes and the LayerNorm weight gradients (their
    // buffers alternate by layer parity; ev_trans releases them and dout),
    // then the saved activations' transposes.
    if (top)
      RC(b.transposes({{prec, dwi, 2 * I, dwiT}, {0, dh1, H, dh1T}, {prec, dqkv, 3 * H, dqkvT}}, tr.side));
    else
      RC(b.transposes({{0, dcur, H, doutT}, {prec, dwi, 2 * I, dwiT}, {0, dh1, H, dh1T}, {prec, dqkv, 3 * H, dqkvT}},
                      tr.side));
    HIPCHK(c, "colsum(norms)", launch_ln_bwd_colsum(lnp_mlp, T, H, grad(p + "mlp_norm.weight"), tr.side,
                                                    l > 0 ? lnp_attn : nullptr,
                                                    l > 0 ? grad(p + "attn_norm.weight") : nullptr));
    HIPCHK(c, "hipEventRecord", hipEventRecord(tr.ev_trans[par], tr.side));
    RC(b.transposes(
        {{prec, S.act.p, I, actT}, {prec, S.n2.p, H, n2T}, {prec, S.ctx.p, H, ctxT}, {prec, S.n1.p, H, n1T}}, tr.side));
    RC(b.wgrad(H, I, doutT, actT, grad(p + "mlp.Wo.weight"), tr.side));
    RC(b.wgrad(2 * I, H, dwiT, n2T, grad(p + "mlp.Wi.weight"), tr.side));
    RC(b.wgrad(H, H, dh1T, ctxT, grad(p + "attn.Wo.weight"), tr.side));
    RC(mark(DN_PROBE_BWD_WGRAD_QKV, 0, tr.side));
    RC(b.wgrad(3 * H, H, dqkvT, n1T, grad(p + "attn.Wqkv.weight"), tr.side));
    RC(mark(DN_PROBE_BWD_WGRAD_QKV, 1, tr.side));
    if (ev) c->probe_bwd_used++;
    HIPCHK(c, "hipEventRecord", hipEventRecord(tr.ev_done[par], tr.side));
    std::swap(dcur, dprev);
  }
  // Every weight gradient is in place before the call returns.
  HIPCHK(c, "hipStreamWaitEvent", hipStreamWaitEvent(s, tr.ev_done[0], 0));
  HIPCHK(c, "hipStreamWaitEvent", hipStreamWaitEvent(s, tr.ev_done[1], 0));

  // Embeddings (backward.go:96-109): LN backward of the emb norm from the
  // gathered rows, then the rows added into dTok in token order.
  if (tr.train_emb && tr.train_from == 0) {
    HIPCHK(c, "hipMalloc", ensure(tr.dE, 4 * TH));
    HIPCHK(c, "hipMemsetAsync", hipMemsetAsync(tr.dE.p, 0, 4 * TH, s));
    HIPCHK(c, "ln_bwd(emb)", launch_ln_bwd((float *)tr.dE.p, nullptr, dcur, (const float *)W(c, kTok),
                                           c->d_ids, (const float *)tr.emb_mean.p,
                                           (const float *)tr.emb_rstd.p, (const float *)W(c, kEmbNorm), g.eps, T, H,
                                           lnpart,
                                           grad(kEmbNorm), s));
    std::vector<int> order(T);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b2) { return tr.ids[a] < tr.ids[b2]; });
    std::vector<int> seg_start, seg_id;
    for (int k = 0; k < T; k++)
      if (k == 0 || tr.ids[order[k]] != tr.ids[order[k - 1]]) {
        seg_start.push_back(k);
        seg_id.push_back(tr.ids[order[k]]);
      }
    const int nseg = (int)seg_id.size();
    seg_start.push_back(T);
    HIPCHK(c, "hipMalloc", ensure(tr.emb_order, sizeof(int) * T));
    HIPCHK(c, "hipMalloc", ensure(tr.emb_seg, sizeof(int) * (nseg + 1)));
    HIPCHK(c, "hipMalloc", ensure(tr.emb_id, sizeof(int) * std::max(nseg, 1)));
    HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(tr.emb_order.p, order.data(), sizeof(int) * T, hipMemcpyHostToDevice, s));
    HIPCHK(c, "hipMemcpyAsync",
           hipMemcpyAsync(tr.emb_seg.p, seg_start.data(), sizeof(int) * (nseg + 1), hipMemcpyHostToDevice, s));
    HIPCHK(c, "hipMemcpyAsync",
           hipMemcpyAsync(tr.emb_id.p, seg_id.data(), sizeof(int) * nseg, hipMemcpyHostToDevice, s));
    HIPCHK(c, "embed_bwd", launch_embed_bwd((const float *)tr.dE.p, (const int *)tr.emb_order.p,
                                            (const int *)tr.emb_seg.p, (const int *)tr.emb_id.p, nseg, H, grad(kTok), s));
    // the host vectors above are read by the copies: wait before they go
    HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
  }
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
  return DN_OK;
}

// Copies between a slot's stored layout and the reference layout (Wi rows
// interleaved in groups of 32 value / 32 gate rows).
void to_reference_layout(const dn_ctx *c, const TensorSlot &t, const float *stored, float *out) {
  if (!t.wi) {
    std::memcpy(out, stored, sizeof(float) * t.n);
    return;
  }
  const int64_t H = c->cfg.hidden, I = c->cfg.inter;
  for (int64_t r = 0; r < 2 * I; r++) std::memcpy(out + wi_src_row(r, I) * H, stored + r * H, sizeof(float) * H);
}
void to_stored_layout(const dn_ctx *c, const TensorSlot &t, const float *ref, float *out) {
  if (!t.wi) {
    std::memcpy(out, ref, sizeof(float) * t.n);
    return;
  }
  const int64_t H = c->cfg.hidden, I = c->cfg.inter;
  for (int64_t r = 0; r < 2 * I; r++) std::memcpy(out + r * H, ref + wi_src_row(r, I) * H, sizeof(float) * H);
}

int training_ready(dn_ctx *c) {
  if (!c->tr.enabled) return fail(c, DN_INVALID_ARG, "decide_hip: dn_enable_training has not been called");
  return check_ready(c);
}

}  // namespace

extern "C" {

int dn_enable_training(dn_ctx *c) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (!c->configured) return fail(c, DN_INVALID_ARG, "decide_hip: dn_set_config has not been called");
  if (c->tr.enabled) return DN_OK;
  if (c->cfg.generic)
    return fail(c, DN_UNSUPPORTED, "decide_hip: training needs head_dim 64, hidden % 256 == 0 and "
                                   "intermediate % 64 == 0");
  if (c->cfg.precision == DN_PRECISION_FP16)
    return fail(c, DN_UNSUPPORTED, "decide_hip: training runs in fp32 or bf16 (fp16 is inference only)");
  for (auto &kv : c->w)
    if (kv.second.set && bf16_slot(c, kv.second))
      return fail(c, DN_INVALID_ARG, "decide_hip: dn_enable_training must precede the weight uploads");
  c->tr.enabled = true;
  return DN_OK;
}

int dn_set_trainable(dn_ctx *c, int train_from, int train_emb) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (train_from < 0) return fail(c, DN_INVALID_ARG, "decide_hip: negative train_from");
  c->tr.train_from = std::min(train_from, c->cfg.layers);
  c->tr.train_emb = train_emb != 0;
  c->tr.have_forward = false;  // the kept activations depend on train_from
  return DN_OK;
}

int dn_forward_train(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
                     const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, float *logits,
                     int logits_cap) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = training_ready(c);
  if (rc) return rc;
  (void)hipSetDevice(c->device);
  rc = ensure_param_state(c);
  if (rc) return rc;
  int R = 0;
  int64_t T = 0;
  rc = stage_batch(c, nseq, seq_len, ids, pos, opt_id, nmask, mask_pos, logits_cap, &R, &T);
  if (rc) return rc;
  c->tr.have_forward = false;
  if (T == 0) return DN_OK;
  rc = forward_core(c, nseq, seq_len, c->d_ids, c->d_pos, c->d_opt, R, c->d_rowtok, (float *)c->logits.p, true);
  if (rc) return rc;
  c->tr.ids.assign(ids, ids + T);
  return finish_forward(c, R, logits);
}

int dn_backward(dn_ctx *c, const float *dlogits, int nrows) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = training_ready(c);
  if (rc) return rc;
  if (!c->tr.have_forward)
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_backward needs the activations of a dn_forward_train");
  if (nrows != c->tr.R || (nrows > 0 && !dlogits))
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_backward: expected " + std::to_string(c->tr.R) + " logits");
  (void)hipSetDevice(c->device);
  return backward_impl(c, dlogits);
}

// Uploads the optimizer table: every trainable tensor (or, with all, every
// tensor that has a gradient), in the model's tensor order, with its workgroup
// ranges; AdamW's rate and weight decay (optim.go:118-141) are filled in
// when given. The host copy stays alive until the caller's synchronize.
int mt_upload(dn_ctx *c, bool all, float lr, float head_lr, float weight_decay, int *nt, int *chunks, int *parts) {
  TrainState &tr = c->tr;
  tr.mt_host.clear();
  int nc = 0, np = 0;
  for (auto &kv : c->w) {
    TensorSlot &t = kv.second;
    if (all ? !t.train.grad.p : frozen(tr, kv.first)) continue;
    MTensor e{};
    e.p = param(c, t);
    e.g = (float *)t.train.grad.p;
    e.m = (float *)t.train.m.p;
    e.v = (float *)t.train.v.p;
    e.wq = bf16_slot(c, t) ? (bf16 *)t.buf.p : nullptr;
    e.n = (size_t)t.n;
    const bool head = kv.first.rfind("scorer.", 0) == 0;
    e.rate = head ? head_lr : lr;
    const bool decay = t.rank == 2 && kv.first != kTok;
    e.wd = decay ? weight_decay * e.rate : 0.0f;
    e.first_chunk = nc;
    e.first_part = np;
    e.nparts = sumsq_blocks(e.n);
    nc += mt_chunks(e.n);
    np += e.nparts;
    tr.mt_host.push_back(e);
  }
  *nt = (int)tr.mt_host.size();
  *chunks = nc;
  *parts = np;
  if (tr.mt_host.empty()) return DN_OK;
  const size_t bytes = sizeof(MTensor) * tr.mt_host.size();
  HIPCHK(c, "hipMalloc", ensure(tr.mt, bytes));
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(tr.mt.p, tr.mt_host.data(), bytes, hipMemcpyHostToDevice, c->stream));
  return DN_OK;
}

int dn_zero_grad(dn_ctx *c) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  (void)hipSetDevice(c->device);
  int nt = 0, chunks = 0, parts = 0;
  int rc = mt_upload(c, true, 0.0f, 0.0f, 0.0f, &nt, &chunks, &parts);
  if (rc) return rc;
  HIPCHK(c, "zero_grad", launch_zero_multi((const MTensor *)c->tr.mt.p, nt, chunks, c->stream));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  return DN_OK;
}

int dn_grad_sumsq(dn_ctx *c, double *out) {
  if (!c || !out) return DN_INVALID_ARG;
  c->err.clear();
  int rc = training_ready(c);
  if (rc) return rc;
  (void)hipSetDevice(c->device);
  rc = ensure_param_state(c);
  if (rc) return rc;
  TrainState &tr = c->tr;
  int nt = 0, chunks = 0, nparts = 0;
  rc = mt_upload(c, false, 0.0f, 0.0f, 0.0f, &nt, &chunks, &nparts);
  if (rc) return rc;
  HIPCHK(c, "hipMalloc", ensure(tr.sq_part, sizeof(double) * std::max(nparts, 1)));
  HIPCHK(c, "hipMalloc", ensure(tr.sq_out, sizeof(double)));
  if (nparts == 0) HIPCHK(c, "hipMemsetAsync", hipMemsetAsync(tr.sq_part.p, 0, sizeof(double), c->stream));
  HIPCHK(c, "sumsq", launch_sumsq_multi((const MTensor *)tr.mt.p, nt, nparts, (double *)tr.sq_part.p, c->stream));
  HIPCHK(c, "sum", launch_sum_doubles((const double *)tr.sq_part.p, nparts, (double *)tr.sq_out.p, c->stream));
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(out, tr.sq_out.p, sizeof(double), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  return DN_OK;
}

int dn_adamw_step(dn_ctx *c, float lr, float head_lr, float weight_decay, float grad_scale) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = training_ready(c);
  if (rc) return rc;
  (void)hipSetDevice(c->device);
  rc = ensure_param_state(c);
  if (rc) return rc;
  TrainState &tr = c->tr;
  tr.adam_step++;
  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
  const double b1c = 1 - std::pow((double)b1, (double)tr.adam_step);
  const double b2c = 1 - std::pow((double)b2, (double)tr.adam_step);
  const float step_size = (float)(1 / b1c), inv_sqrt_b2c = (float)(1 / std::sqrt(b2c));
  int nt = 0, chunks = 0, parts = 0;
  rc = mt_upload(c, false, lr, head_lr, weight_decay, &nt, &chunks, &parts);
  if (rc) return rc;
  HIPCHK(c, "adamw", launch_adamw_multi((const MTensor *)tr.mt.p, nt, chunks, b1, b2, eps, grad_scale, step_size,
                                        inv_sqrt_b2c, c->stream));
  for (auto &kv : c->w)
    if (!frozen(tr, kv.first)) kv.second.train.wt_valid = false;
  c->wgen++;  // the folded LayerNorm's column sums follow the new weights
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  return DN_OK;
}

int dn_download_tensor(dn_ctx *c, const char *name, int which, float *out, int64_t n) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (!name || !out) return fail(c, DN_INVALID_ARG, "decide_hip: dn_download_tensor: NULL argument");
  auto it = c->w.find(name);
  if (it == c->w.end()) return fail(c, DN_INVALID_ARG, std::string("decide_hip: unknown tensor ") + name);
  TensorSlot &t = it->second;
  if (n != t.n) return fail(c, DN_INVALID_ARG, std::string("decide_hip: ") + name + " has " + std::to_string(t.n) + " values");
  (void)hipSetDevice(c->device);
  std::vector<float> tmp((size_t)n);
  const void *src = nullptr;
  if (which == DN_STATE_WEIGHT) {
    if (!t.set) return fail(c, DN_INVALID_ARG, std::string("decide_hip: weight ") + name + " not uploaded");
    if (bf16_slot(c, t) && !t.train.master.p) {  // inference copy only: widen the bf16 operand
      std::vector<uint16_t> bits((size_t)n);
      HIPCHK(c, "hipMemcpy", hipMemcpy(bits.data(), t.buf.p, 2 * (size_t)n, hipMemcpyDeviceToHost));
      for (int64_t i = 0; i < n; i++) {
        const uint32_t u = (uint32_t)bits[i] << 16;
        std::memcpy(&tmp[i], &u, 4);
      }
      to_reference_layout(c, t, tmp.data(), out);
      return DN_OK;
    }
    src = bf16_slot(c, t) ? t.train.master.p : t.buf.p;
  } else if (which == DN_STATE_GRAD || which == DN_STATE_M || which == DN_STATE_V) {
    const DevBuf &b = which == DN_STATE_GRAD ? t.train.grad : which == DN_STATE_M ? t.train.m : t.train.v;
    if (!b.p) return fail(c, DN_INVALID_ARG, "decide_hip: no training state (dn_enable_training, dn_forward_train)");
    src = b.p;
  } else {
    return fail(c, DN_INVALID_ARG, "decide_hip: unknown state " + std::to_string(which));
  }
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  HIPCHK(c, "hipMemcpy", hipMemcpy(tmp.data(), src, sizeof(float) * (size_t)n, hipMemcpyDeviceToHost));
  to_reference_layout(c, t, tmp.data(), out);
  return DN_OK;
}

int dn_upload_state(dn_ctx *c, const char *name, int which, const float *data, int64_t n) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = training_ready(c);
  if (rc) return rc;
  if (!name || !data) return fail(c, DN_INVALID_ARG, "decide_hip: dn_upload_state: NULL argument");
  auto it = c->w.find(name);
  if (it == c->w.end()) return fail(c, DN_INVALID_ARG, std::string("decide_hip: unknown tensor ") + name);
  TensorSlot &t = it->second;
  if (n != t.n) return fail(c, DN_INVALID_ARG, std::string("decide_hip: ") + name + " has " + std::to_string(t.n) + " values");
  if (which != DN_STATE_GRAD && which != DN_STATE_M && which != DN_STATE_V)
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_upload_state takes DN_STATE_GRAD, DN_STATE_M or DN_STATE_V");
  (void)hipSetDevice(c->device);
  rc = ensure_param_state(c);
  if (rc) return rc;
  std::vector<float> tmp((size_t)n);
  to_stored_layout(c, t, data, tmp.data());
  DevBuf &b = which == DN_STATE_GRAD ? t.train.grad : which == DN_STATE_M ? t.train.m : t.train.v;
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  HIPCHK(c, "hipMemcpy", hipMemcpy(b.p, tmp.data(), sizeof(float) * (size_t)n, hipMemcpyHostToDevice));
  return DN_OK;
}

int dn_set_adam_step(dn_ctx *c, int step) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (step < 0) return fail(c, DN_INVALID_ARG, "decide_hip: negative step");
  c->tr.adam_step = step;
  return DN_OK;
}

}  // extern "C"
