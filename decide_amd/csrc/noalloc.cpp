// dn_forward_device_noalloc: the forward of dn_forward_device for callers
// that cannot allocate device memory (tight serving loops, harnesses that
// forbid hipMalloc). It synchronises the context's stream before uploading
// the batch layout, so it refuses a capturing stream (DN_UNSUPPORTED).
// Every buffer the forward works in beyond the weights and the caller's
// inputs and outputs (the activations, the batch layout, the head's
// scratch) is carved out of one static device array per GPU, `scratch`, of
// kScratchBytes. The call makes no hipMalloc / hipFree and uses no
// allocating library routine; the RoPE tables, the error flag and the
// folded LayerNorm's column-sum array come from set-up (dn_set_config; the
// column sums are refilled by a kernel when the weights have changed).
//
// Every call on a GPU shares that GPU's array and it keeps the last call's
// contents: calls that overlap on one GPU (two contexts, two streams) race.
// Nothing in it needs to start at zero: each forward writes every element it
// reads (embedding + LayerNorm write the residual stream before the residual
// GEMMs accumulate into it; the layout is uploaded by every call).
#include <algorithm>
#include <mutex>

#include "ctx.hpp"

using namespace dnh;

namespace {

constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) char scratch[kScratchBytes];

// Device address of `scratch` on each device, looked up once per device with
// that device current. In host code `scratch` itself is only a host-side
// stand-in for the symbol, never a device address.
void *g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

}  // namespace

namespace dnh {

int noalloc_init(dn_ctx *c) {
  if (c->device < 0 || c->device >= kMaxDevices) return DN_OK;  // no scratch: the entry point reports it
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[c->device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(nullptr, "hipGetSymbolAddress(scratch)", e);
    g_scratch[c->device] = p;
  }
  c->scratch = g_scratch[c->device];
  return DN_OK;
}

}  // namespace dnh

extern "C" int dn_forward_device_noalloc(dn_ctx *c, int nseq, const int32_t *seq_len, const int32_t *d_ids,
                                         const int32_t *d_pos, const int32_t *d_opt_id, int nrows,
                                         const int32_t *d_row_tok, float *d_logits) {
  if (!c) return DN_INVALID_ARG;
  c->err.clear();
  int rc = check_ready(c);
  if (rc) return rc;
  if (nseq <= 0 || !seq_len || !d_ids || !d_pos || nrows < 0 || (nrows > 0 && (!d_row_tok || !d_logits)))
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_forward_device_noalloc: bad argument");
  for (int s = 0; s < nseq; s++) {
    if (seq_len[s] <= 0) return fail(c, DN_INVALID_ARG, "nn: malformed sequence " + std::to_string(s));
    if (seq_len[s] > 8192)
      return fail(c, DN_UNSUPPORTED, "decide_hip: sequence " + std::to_string(s) + " is longer than 8192 tokens");
  }
  if (!c->scratch) return fail(c, DN_DEVICE_ERROR, "decide_hip: no scratch array on this device");
  (void)hipSetDevice(c->device);
  // The host layout vectors are rewritten below: an earlier call's copies
  // out of them must have finished. A capturing stream cannot be waited for
  // (and a captured copy would read those vectors at replay), so capture is
  // refused before anything is enqueued.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIPCHK(c, "hipStreamIsCapturing", hipStreamIsCapturing(c->stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(c, DN_UNSUPPORTED, "decide_hip: dn_forward_device_noalloc cannot run under stream capture");
  HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
  int T = 0, nch = 0;
  host_layout(c->hlay, nseq, seq_len, &T, &nch);
  const int nwork = (int)c->hlay.work.size(), nwork2 = (int)c->hlay.work2.size();
  const Config &g = c->cfg;
  const size_t es = prec16(g.precision) ? 2 : 4, H = g.hidden, I = g.inter, Tz = T;
  const size_t R1 = (size_t)(nrows > 0 ? nrows : 1);
  // Carve the workspace (256-byte aligned pieces) before touching anything.
  size_t off = 0;
  char *base = (char *)c->scratch;
  auto take = [&](size_t bytes) -> void * {
    void *p = base + off;
    off += (bytes + 255) & ~(size_t)255;
    return p;
  };
  Workspace w;
  w.h = (float *)take(sizeof(float) * Tz * H);
  w.xn = take(es * Tz * H);
  w.qkv = take(es * Tz * 3 * H);
  w.ctx = take(es * Tz * H);
  w.act = take(es * Tz * I);
  w.kinfo = (int *)take(sizeof(int) * Tz);
  w.head_s1 = (float *)take(sizeof(float) * R1 * H);
  w.head_d = (float *)take(sizeof(float) * R1 * (H / 2));
  if (T <= kSmallSplitMaxTokens) w.part = (float *)take(sizeof(float) * kSmallSplitParts * Tz * H);
  if (fold_eligible(c, T)) {  // the folded LayerNorm's statistics, as dn_forward_device has them
    w.lpart = (float *)take(sizeof(float) * 2 * (H / kLnPartCols) * Tz);
    w.lmean1 = (float *)take(sizeof(float) * Tz);
    w.lmean2 = (float *)take(sizeof(float) * Tz);
  }
  w.seq_off = (int *)take(sizeof(int) * (nseq + 1));
  w.seq_len = (int *)take(sizeof(int) * (nseq + 1));
  w.chunk_off = (int *)take(sizeof(int) * (nseq + 1));
  w.chunk_desc = (int4 *)take(sizeof(int4) * (nch + 1));
  w.chunks = (ChunkInfo *)take(sizeof(ChunkInfo) * (nch + 1));
  w.work = (int4 *)take(sizeof(int4) * (nwork + nwork2 + 1));
  w.codes = (uint32_t *)take(sizeof(uint32_t) * ATTN_MAXKT * (2 * nwork + nwork2 + 1));
  w.first = (int *)take(sizeof(int) * (2 * nwork + nwork2 + 1));
  if (off > kScratchBytes) {
    const size_t per_token = sizeof(float) * H + es * (5 * H + I) + sizeof(int) + fold_bytes_per_token(c);
    return fail(c, DN_INVALID_ARG, "decide_hip: dn_forward_device_noalloc: this batch (" + std::to_string(T) +
                                       " tokens, " + std::to_string(nrows) + " rows) needs " + std::to_string(off) +
                                       " bytes of scratch; the maximum is " + std::to_string(kScratchBytes) +
                                       " (about " + std::to_string(kScratchBytes / per_token) +
                                       " tokens at this configuration)");
  }
  w.T = T;
  w.nchunks = nch;
  w.nwork = nwork;
  set_work2(w, nwork2);
  w.nseq = nseq;
  w.max_len = *std::max_element(seq_len, seq_len + nseq);
  rc = upload_layout(c, c->hlay, w, nseq, seq_len, c->stream);
  if (rc) return rc;
  return forward_core(c, nseq, seq_len, d_ids, d_pos, d_opt_id, nrows, d_row_tok, d_logits, false, &w);
}
