// Certified argmax for the 16-bit modes (dn_set_certify).
//
// The reference answers a Choice question with the argmax of its options'
// float32 logits (local.go:254-262, :291). A 16-bit forward moves each logit
// by a small rounding error, so a question whose two best options lie closer
// than that error may come out the other way. With certification on, every
// forward checks each sequence's logits (one sequence holds one question in
// the Choice and SystemOne layouts dn_evaluate builds): when its two largest
// logits are less than `margin` apart, or any of its logits is not finite,
// the sequence is run again on an fp32 twin of the context (same geometry,
// the uploaded weights in float32, fp32 MFMA everywhere: the validation
// mode, whose logits match the reference to ~1e-7) and its logits are
// replaced by the twin's. Every other sequence keeps its 16-bit logits,
// whose order the margin certifies as long as the margin bounds the 16-bit
// error of a logit difference.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "ctx.hpp"

using namespace dnh;

namespace {

// Whether logits lg[0..k) need the exact path: two of them within margin of
// the best, or a non-finite value.
bool near_tie(const float *lg, int k, float margin) {
  float top1 = -INFINITY, top2 = -INFINITY;
  for (int i = 0; i < k; i++) {
    const float v = lg[i];
    if (!std::isfinite(v)) return true;
    if (v > top1) {
      top2 = top1;
      top1 = v;
    } else if (v > top2) {
      top2 = v;
    }
  }
  return k >= 2 && top1 - top2 < margin;
}

int child_fail(dn_ctx *c, int rc) {
  return fail(c, rc, "decide_hip: certification (fp32 recompute): " + c->exact->err);
}

}  // namespace

namespace dnh {

void close_certify(dn_ctx *c) {
  if (c->exact) dn_close(c->exact);
  c->exact = nullptr;
  c->certify_margin = 0.0f;
  release(c->cert_in);
  release(c->cert_out);
}

// Host-array forward: logits (host, R of them, sequence by sequence as
// nmask says) are final 16-bit logits; near-tie sequences are recomputed by
// the fp32 twin through its own dn_forward.
int certify_host(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
                 const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, float *logits) {
  if (!c->exact) return DN_OK;
  std::vector<int32_t> sl, sid, spos, sopt, snm, smp;
  std::vector<int> dst;  // logit index of each recomputed row
  int64_t toff = 0, roff = 0;
  for (int s = 0; s < nseq; s++) {
    const int n = seq_len[s], k = nmask[s];
    c->cert_checked++;
    if (near_tie(logits + roff, k, c->certify_margin)) {
      sl.push_back(n);
      sid.insert(sid.end(), ids + toff, ids + toff + n);
      spos.insert(spos.end(), pos + toff, pos + toff + n);
      if (opt_id) sopt.insert(sopt.end(), opt_id + toff, opt_id + toff + n);
      snm.push_back(k);
      smp.insert(smp.end(), mask_pos + roff, mask_pos + roff + k);
      for (int i = 0; i < k; i++) dst.push_back((int)(roff + i));
    }
    toff += n;
    roff += k;
  }
  if (sl.empty()) return DN_OK;
  c->cert_recomputed += (int64_t)sl.size();
  std::vector<float> sub(dst.size());
  c->exact->stream = c->stream;
  const int rc = dn_forward(c->exact, (int)sl.size(), sl.data(), sid.data(), spos.data(),
                            opt_id ? sopt.data() : nullptr, snm.data(), smp.data(), sub.data(), (int)sub.size());
  if (rc) return child_fail(c, rc);
  for (size_t j = 0; j < dst.size(); j++) logits[dst[j]] = sub[j];
  return DN_OK;
}

// Device-array forward (dn_forward_device): the logits and row tokens are
// read back, rows are assigned to sequences by their token index, and the
// near-tie sequences' tokens are copied into a compact batch that the fp32
// twin runs; its logits replace the rows' in d_logits. Synchronous.
int certify_device(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *d_ids, const int32_t *d_pos,
                   const int32_t *d_opt, int R, const int32_t *d_row_tok, float *d_logits) {
  if (!c->exact || R <= 0) return DN_OK;
  hipStream_t s = c->stream;
  std::vector<float> lg((size_t)R);
  std::vector<int32_t> rt((size_t)R);
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(lg.data(), d_logits, sizeof(float) * R, hipMemcpyDeviceToHost, s));
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(rt.data(), d_row_tok, sizeof(int32_t) * R, hipMemcpyDeviceToHost, s));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
  std::vector<int64_t> off((size_t)nseq + 1, 0);
  for (int i = 0; i < nseq; i++) off[i + 1] = off[i] + seq_len[i];
  // Rows of each sequence in row order (an index outside the batch is the
  // forward's own error, flagged on the device; such rows are left alone).
  std::vector<std::vector<int>> rows((size_t)nseq);
  for (int r = 0; r < R; r++) {
    const int64_t t = rt[r];
    if (t < 0 || t >= off[nseq]) continue;
    const int si = (int)(std::upper_bound(off.begin(), off.end(), t) - off.begin()) - 1;
    rows[si].push_back(r);
  }
  std::vector<int> pick;
  std::vector<float> tmp;
  for (int i = 0; i < nseq; i++) {
    if (rows[i].empty()) continue;
    c->cert_checked++;
    tmp.clear();
    for (int r : rows[i]) tmp.push_back(lg[r]);
    if (near_tie(tmp.data(), (int)tmp.size(), c->certify_margin)) pick.push_back(i);
  }
  if (pick.empty()) return DN_OK;
  c->cert_recomputed += (int64_t)pick.size();
  std::vector<int32_t> sl, srt;
  std::vector<int> dst;
  int64_t T2 = 0;
  for (int i : pick) {
    for (int r : rows[i]) {
      srt.push_back((int32_t)(rt[r] - off[i] + T2));
      dst.push_back(r);
    }
    sl.push_back(seq_len[i]);
    T2 += seq_len[i];
  }
  const int R2 = (int)dst.size();
  const size_t nin = (size_t)(d_opt ? 3 : 2) * T2 + R2;
  HIPCHK(c, "hipMalloc", ensure(c->cert_in, sizeof(int32_t) * nin));
  HIPCHK(c, "hipMalloc", ensure(c->cert_out, sizeof(float) * R2));
  int32_t *ids2 = (int32_t *)c->cert_in.p, *pos2 = ids2 + T2, *opt2 = d_opt ? pos2 + T2 : nullptr;
  int32_t *rt2 = pos2 + (d_opt ? 2 : 1) * T2;
  int64_t o = 0;
  for (int i : pick) {
    const size_t b = sizeof(int32_t) * seq_len[i];
    HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(ids2 + o, d_ids + off[i], b, hipMemcpyDeviceToDevice, s));
    HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(pos2 + o, d_pos + off[i], b, hipMemcpyDeviceToDevice, s));
    if (d_opt) HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(opt2 + o, d_opt + off[i], b, hipMemcpyDeviceToDevice, s));
    o += seq_len[i];
  }
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(rt2, srt.data(), sizeof(int32_t) * R2, hipMemcpyHostToDevice, s));
  c->exact->stream = s;
  int rc = check_ready(c->exact);
  if (!rc) rc = forward_core(c->exact, (int)pick.size(), sl.data(), ids2, pos2, opt2, R2, rt2, (float *)c->cert_out.p,
                             false);
  if (rc) return child_fail(c, rc);
  std::vector<float> sub((size_t)R2);
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(sub.data(), c->cert_out.p, sizeof(float) * R2, hipMemcpyDeviceToHost, s));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
  for (int j = 0; j < R2; j++) lg[dst[j]] = sub[j];
  HIPCHK(c, "hipMemcpyAsync", hipMemcpyAsync(d_logits, lg.data(), sizeof(float) * R, hipMemcpyHostToDevice, s));
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(s));
  return DN_OK;
}

}  // namespace dnh

extern "C" {

int dn_set_certify(dn_ctx *c, float margin) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  if (!c->configured) return fail(c, DN_INVALID_ARG, "decide_hip: dn_set_config has not been called");
  if (!(margin >= 0.0f) || !std::isfinite(margin))
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_set_certify: margin must be finite and >= 0");
  if (margin == 0.0f) {
    close_certify(c);
    return DN_OK;
  }
  if (c->cfg.precision == DN_PRECISION_FP32)
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_set_certify: the fp32 mode is already the exact path");
  if (c->tr.enabled) return fail(c, DN_UNSUPPORTED, "decide_hip: dn_set_certify: not for training contexts");
  if (!c->exact) {
    for (auto &kv : c->w)
      if (kv.second.set)
        return fail(c, DN_INVALID_ARG, "decide_hip: dn_set_certify must precede the weight uploads");
    dn_ctx *x = nullptr;
    int rc = dn_open(c->device, &x);
    if (rc) return fail(c, rc, "decide_hip: dn_set_certify: opening the fp32 twin failed");
    const Config &g = c->cfg;
    rc = dn_set_config(x, g.hidden, g.inter, g.heads, g.layers, g.vocab, g.eps, g.half_window, g.theta_g, g.theta_l,
                       g.sliding.data(), DN_PRECISION_FP32);
    if (rc) {
      const std::string why = x->err;
      dn_close(x);
      return fail(c, rc, "decide_hip: dn_set_certify: " + why);
    }
    c->exact = x;
  }
  c->certify_margin = margin;
  return DN_OK;
}

int dn_read_certify(dn_ctx *c, int64_t *checked, int64_t *recomputed) {
  if (!c || !checked || !recomputed) return DN_INVALID_ARG;
  *checked = c->cert_checked;
  *recomputed = c->cert_recomputed;
  c->cert_checked = c->cert_recomputed = 0;
  return DN_OK;
}

}  // extern "C"
