// CPU oracle: a C++ restatement of the reference's pure-Go encoder forward.
//
// TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP
// library and the CPU baseline timed by bench.py. Only tests/, the smoke
// entry and bench.py's cpu_baseline leg load it; the product path never does.
//
// What it restates (paths relative to the reference checkout):
//   internal/blas/gemm.go:13-220     Sgemm / Sgemm1: blocking mr=6 nr=16 kc=256
//                                    mc=96, packA/packB, dynamic job queue
//   internal/blas/kern_amd64.s:5-81  6x16 AVX2/FMA micro-kernel (acc := 0,
//                                    acc = fma(a,b,acc) over one kc block in
//                                    increasing k, then C += acc)
//   internal/nn/ops.go:13-44         parallelFor (4*workers dynamic chunks)
//   internal/nn/ops.go:63-92         layerNormFwd (f64 two-pass statistics)
//   internal/nn/ops.go:140-142       gelu (exact erf form, erf in f64)
//   internal/nn/ops.go:155-175       applyRope (rotate-half)
//   internal/nn/model.go:242-258     ropeTables (angle rounded to f32 first)
//   internal/nn/forward.go:28-56     BuildSequence
//   internal/nn/forward.go:129-245   Forward (layout, masks, layers, rows)
//   internal/nn/forward.go:250-282   HeadForward
//   internal/nn/forward.go:284-343   layerFwd
//   internal/nn/forward.go:347-409   attnFwd + softmaxMasked
//   local.go:206-262                 softmax, calibrated, round, marginConfidence, argmax
//
// Go evaluates float32 expressions in IEEE single precision without
// contracting a*b+c on amd64, so everything outside the explicit FMA
// micro-kernel is compiled with -ffp-contract=off and written with Go's
// left-to-right association.
//
// Parity pins (tests/test_oracle.py): the reference's own PyTorch fixture
// (tiny_ref.safetensors: logits, hidden.0-3, l1.n1, l1.attn), naive float64
// GEMM on the reference test's shape list with all transposes, accumulate and
// padded leading dimensions, order invariance, and closed forms for LN, RoPE,
// GELU and the answer post-processing.
#include <immintrin.h>

#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// Worker pool: stands in for goroutines. run(w, body) executes body on w
// threads (the caller included); work distribution inside body is the
// reference's atomic-counter queue.
class Pool {
 public:
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu_);
      stop_ = true;
      gen_++;
    }
    cv_.notify_all();
    for (auto &t : th_) t.join();
  }
  void run(int w, const std::function<void()> &body) {
    if (w <= 1) {
      body();
      return;
    }
    ensure(w - 1);
    {
      std::lock_guard<std::mutex> g(mu_);
      body_ = &body;
      active_ = w - 1;
      pending_ = w - 1;
      gen_++;
    }
    cv_.notify_all();
    body();
    std::unique_lock<std::mutex> g(mu_);
    done_.wait(g, [&] { return pending_ == 0; });
    body_ = nullptr;
  }

 private:
  void ensure(int n) {
    while ((int)th_.size() < n) {
      int id = (int)th_.size();
      // The thread starts from the current generation: work published after
      // this point (gen_ incremented by run) is seen as new.
      const uint64_t g0 = gen_;
      th_.emplace_back([this, id, g0] { loop(id, g0); });
    }
  }
  void loop(int id, uint64_t seen) {
    for (;;) {
      const std::function<void()> *b = nullptr;
      {
        std::unique_lock<std::mutex> g(mu_);
        cv_.wait(g, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
        if (id >= active_) continue;
        b = body_;
      }
      (*b)();
      {
        std::lock_guard<std::mutex> g(mu_);
        if (--pending_ == 0) done_.notify_all();
      }
    }
  }
  std::vector<std::thread> th_;
  std::mutex mu_;
  std::condition_variable cv_, done_;
  const std::function<void()> *body_ = nullptr;
  uint64_t gen_ = 0;
  int active_ = 0, pending_ = 0;
  bool stop_ = false;
};

Pool &pool() {
  static Pool p;
  return p;
}

int g_workers = 1;  // runtime.GOMAXPROCS(0) / blas.Workers

// Emulated operand rounding (not part of the reference's arithmetic): each bit
// rounds one stage's values to bfloat16 (nearest even) where a bf16 device
// path stores or multiplies them, so that the effect of each stage on the
// logits can be measured on the CPU. 0 (the default) is the reference.
int g_round = 0;
int g_round_lo = 0, g_round_hi = 1 << 30;  // layers [lo, hi) round; the others are exact
int g_round_now = 0;                         // the current layer's switches
enum : int {
  RND_XN = 1,     // LayerNorm outputs feeding QKV and Wi (and layer 0's emb-norm output)
  RND_QKV = 2,    // the QKV GEMM's stored output, before RoPE
  RND_QK = 4,     // q and k after RoPE (score MFMA operands)
  RND_P = 8,      // attention probabilities before P.V
  RND_CTX = 16,   // attention output (Wo's operand)
  RND_ACT = 32,   // GeGLU output (MlpWo's operand)
  RND_FP16 = 128, // round the stages above to IEEE binary16 instead of bfloat16
  RND_XFOLD = 256, // LayerNorm folded into the GEMM after it: the LayerNorm input x rounded,
                   // the statistics taken from the unrounded x, the output not rounded
  RND_XFOLDC = 512, // as RND_XFOLD, x less the previous LayerNorm's row mean rounded
};
inline float bf16_round(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7F800000u) == 0x7F800000u) return x;
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  std::memcpy(&x, &u, 4);
  return x;
}
// Nearest-even binary16 value of x (subnormals kept, overflow to infinity).
inline float fp16_round(float x) {
  float a = std::fabs(x);
  if (!(a < 65520.0f)) return a != a ? x : std::copysign(INFINITY, x);
  if (a < 6.103515625e-05f) return std::nearbyint(x * 16777216.0f) / 16777216.0f;  // quantum 2^-24
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u = (u + 0xFFFu + ((u >> 13) & 1u)) & 0xFFFFE000u;
  std::memcpy(&x, &u, 4);
  return x;
}
void round_if(int bit, float *x, size_t n) {
  if (!(g_round_now & bit)) return;
  if (g_round_now & RND_FP16)
    for (size_t i = 0; i < n; i++) x[i] = fp16_round(x[i]);
  else
    for (size_t i = 0; i < n; i++) x[i] = bf16_round(x[i]);
}

// RND_XFOLD: y = (round(x) - mean) * rstd * w with the statistics of the
// unrounded rows, as a device path that multiplies the rounded residual
// stream by w-scaled weights and subtracts mean * (column sums) afterwards
// computes it.
void fold_if(float *y, const float *x, int rows, int dim, const float *w, const float *mean, const float *rstd,
             const float *prev_mean) {
  if (!(g_round_now & (RND_XFOLD | RND_XFOLDC))) return;
  const bool centred = (g_round_now & RND_XFOLDC) != 0;
  for (int r = 0; r < rows; r++) {
    const float mp = centred && prev_mean ? prev_mean[r] : 0.0f;
    for (int i = 0; i < dim; i++) {
      float v = x[(size_t)r * dim + i] - mp;
      v = (g_round_now & RND_FP16) ? fp16_round(v) : bf16_round(v);
      y[(size_t)r * dim + i] = (v - (mean[r] - mp)) * rstd[r] * w[i];
    }
  }
}

// parallelFor, internal/nn/ops.go:13-44.
void parallel_for(int n, const std::function<void(int, int)> &fn) {
  int workers = g_workers;
  if (n <= 0) return;
  if (workers > n) workers = n;
  if (workers <= 1) {
    fn(0, n);
    return;
  }
  int chunk = std::max(1, (n + 4 * workers - 1) / (4 * workers));
  int chunks = (n + chunk - 1) / chunk;
  std::atomic<int> next{0};
  pool().run(std::min(workers, chunks), [&] {
    for (;;) {
      int c = next.fetch_add(1);
      if (c >= chunks) return;
      int lo = c * chunk;
      fn(lo, std::min(lo + chunk, n));
    }
  });
}

// ---------------------------------------------------------------------------
// SGEMM, internal/blas/gemm.go.
constexpr int MR = 6, NR = 16, KC = 256, MC = 96;

struct Scratch {
  std::vector<float> a, b;
  float tmp[MR * NR];
};

// kern6x16, kern_amd64.s:5-81. 12 accumulators start at zero, one FMA per
// (k, i, j) in increasing k, then C += acc.
void kern6x16(int k, const float *a, const float *b, float *c, int ldc) {
  __m256 c00 = _mm256_setzero_ps(), c01 = _mm256_setzero_ps();
  __m256 c10 = _mm256_setzero_ps(), c11 = _mm256_setzero_ps();
  __m256 c20 = _mm256_setzero_ps(), c21 = _mm256_setzero_ps();
  __m256 c30 = _mm256_setzero_ps(), c31 = _mm256_setzero_ps();
  __m256 c40 = _mm256_setzero_ps(), c41 = _mm256_setzero_ps();
  __m256 c50 = _mm256_setzero_ps(), c51 = _mm256_setzero_ps();
  for (int p = 0; p < k; p++) {
    __m256 b0 = _mm256_loadu_ps(b), b1 = _mm256_loadu_ps(b + 8);
    __m256 a0 = _mm256_broadcast_ss(a + 0), a1 = _mm256_broadcast_ss(a + 1);
    c00 = _mm256_fmadd_ps(b0, a0, c00);
    c01 = _mm256_fmadd_ps(b1, a0, c01);
    c10 = _mm256_fmadd_ps(b0, a1, c10);
    c11 = _mm256_fmadd_ps(b1, a1, c11);
    a0 = _mm256_broadcast_ss(a + 2);
    a1 = _mm256_broadcast_ss(a + 3);
    c20 = _mm256_fmadd_ps(b0, a0, c20);
    c21 = _mm256_fmadd_ps(b1, a0, c21);
    c30 = _mm256_fmadd_ps(b0, a1, c30);
    c31 = _mm256_fmadd_ps(b1, a1, c31);
    a0 = _mm256_broadcast_ss(a + 4);
    a1 = _mm256_broadcast_ss(a + 5);
    c40 = _mm256_fmadd_ps(b0, a0, c40);
    c41 = _mm256_fmadd_ps(b1, a0, c41);
    c50 = _mm256_fmadd_ps(b0, a1, c50);
    c51 = _mm256_fmadd_ps(b1, a1, c51);
    a += MR;
    b += NR;
  }
  auto st = [&](float *row, __m256 x0, __m256 x1) {
    _mm256_storeu_ps(row, _mm256_add_ps(x0, _mm256_loadu_ps(row)));
    _mm256_storeu_ps(row + 8, _mm256_add_ps(x1, _mm256_loadu_ps(row + 8)));
  };
  st(c + 0 * ldc, c00, c01);
  st(c + 1 * ldc, c10, c11);
  st(c + 2 * ldc, c20, c21);
  st(c + 3 * ldc, c30, c31);
  st(c + 4 * ldc, c40, c41);
  st(c + 5 * ldc, c50, c51);
}

// packA, gemm.go:147-170.
void pack_a(Scratch &s, bool trans, const float *A, int lda, int i0, int p0, int mb, int kb) {
  int panels = (mb + MR - 1) / MR;
  s.a.resize((size_t)panels * MR * kb);
  float *dst = s.a.data();
  for (int pi = 0; pi < panels; pi++) {
    size_t base = (size_t)pi * MR * kb;
    int rows = std::min(MR, mb - pi * MR);
    for (int p = 0; p < kb; p++) {
      float *d = dst + base + (size_t)p * MR;
      if (!trans) {
        for (int i = 0; i < rows; i++) d[i] = A[(size_t)(i0 + pi * MR + i) * lda + p0 + p];
      } else {
        const float *src = A + (size_t)(p0 + p) * lda + i0 + pi * MR;
        std::memcpy(d, src, sizeof(float) * rows);
      }
      for (int i = rows; i < MR; i++) d[i] = 0;
    }
  }
}

// packB, gemm.go:172-195.
void pack_b(Scratch &s, bool trans, const float *B, int ldb, int p0, int j0, int kb, int nb) {
  int panels = (nb + NR - 1) / NR;
  s.b.resize((size_t)panels * NR * kb);
  float *dst = s.b.data();
  for (int pj = 0; pj < panels; pj++) {
    size_t base = (size_t)pj * NR * kb;
    int cols = std::min(NR, nb - pj * NR);
    for (int p = 0; p < kb; p++) {
      float *d = dst + base + (size_t)p * NR;
      if (!trans) {
        const float *src = B + (size_t)(p0 + p) * ldb + j0 + pj * NR;
        std::memcpy(d, src, sizeof(float) * cols);
      } else {
        for (int j = 0; j < cols; j++) d[j] = B[(size_t)(j0 + pj * NR + j) * ldb + p0 + p];
      }
      for (int j = cols; j < NR; j++) d[j] = 0;
    }
  }
}

// macro, gemm.go:197-220.
void macro(Scratch &s, float *C, int ldc, int mb, int nb, int kb) {
  for (int jr = 0; jr < nb; jr += NR) {
    const float *bp = s.b.data() + (size_t)(jr / NR) * NR * kb;
    int cols = std::min(NR, nb - jr);
    for (int ir = 0; ir < mb; ir += MR) {
      const float *ap = s.a.data() + (size_t)(ir / MR) * MR * kb;
      int rows = std::min(MR, mb - ir);
      if (rows == MR && cols == NR) {
        kern6x16(kb, ap, bp, C + (size_t)ir * ldc + jr, ldc);
        continue;
      }
      std::memset(s.tmp, 0, sizeof(s.tmp));
      kern6x16(kb, ap, bp, s.tmp, NR);
      for (int i = 0; i < rows; i++) {
        float *dst = C + (size_t)(ir + i) * ldc + jr;
        for (int j = 0; j < cols; j++) dst[j] += s.tmp[i * NR + j];
      }
    }
  }
}

int round_up(int x, int m) { return (x + m - 1) / m * m; }

// sgemm, gemm.go:71-138.
void sgemm(int workers, bool transA, bool transB, int M, int N, int K, const float *A, int lda,
           const float *B, int ldb, float *C, int ldc, bool accumulate) {
  if (M == 0 || N == 0) return;
  if (!accumulate)
    for (int i = 0; i < M; i++) std::memset(C + (size_t)i * ldc, 0, sizeof(float) * N);
  if (K == 0) return;
  if ((int64_t)M * N * K < (1 << 15)) workers = 1;
  int mBlk = std::min(MC, round_up(M, MR));
  int mBlocks = (M + mBlk - 1) / mBlk;
  int nBlk = round_up(N, NR);
  int want = (2 * workers + mBlocks - 1) / mBlocks;
  if (want > 1) nBlk = std::min(nBlk, std::max(NR, round_up((N + want - 1) / want, NR)));
  nBlk = std::min(nBlk, 256);
  int nBlocks = (N + nBlk - 1) / nBlk;
  int jobs = mBlocks * nBlocks;
  auto run = [&](int job, Scratch &s) {
    int ic = (job % mBlocks) * mBlk;
    int jc = (job / mBlocks) * nBlk;
    int mb = std::min(mBlk, M - ic);
    int nb = std::min(nBlk, N - jc);
    for (int pc = 0; pc < K; pc += KC) {
      int kb = std::min(KC, K - pc);
      pack_a(s, transA, A, lda, ic, pc, mb, kb);
      pack_b(s, transB, B, ldb, pc, jc, kb, nb);
      macro(s, C + (size_t)ic * ldc + jc, ldc, mb, nb, kb);
    }
  };
  if (workers == 1 || jobs == 1) {
    thread_local Scratch s;
    for (int j = 0; j < jobs; j++) run(j, s);
    return;
  }
  std::atomic<int> next{0};
  pool().run(std::min(workers, jobs), [&] {
    thread_local Scratch s;
    for (;;) {
      int j = next.fetch_add(1);
      if (j >= jobs) break;
      run(j, s);
    }
  });
}

// ---------------------------------------------------------------------------
// Model, internal/nn/model.go + config.go.
struct Config {
  int hidden, inter, heads, layers, vocab;
  float eps;
  int half_window;
  double theta_g, theta_l;
  std::vector<uint8_t> sliding;
};

struct TrainCache;

struct Model {
  Config cfg;
  std::shared_ptr<TrainCache> tc;  // activations of the last training forward
  std::map<std::string, std::vector<float>> w;
  const float *get(const std::string &name) const {
    auto it = w.find(name);
    return it == w.end() ? nullptr : it->second.data();
  }
};

// layerNormFwd, ops.go:63-92.
// mean / rstd (when non-null) receive the row statistics, as the reference
// records them for the backward pass.
void layer_norm(float *y, const float *x, int rows, int dim, const float *w, const float *b, float eps,
                float *mean = nullptr, float *rstd = nullptr) {
  parallel_for(rows, [&](int lo, int hi) {
    for (int r = lo; r < hi; r++) {
      const float *row = x + (size_t)r * dim;
      double sum = 0;
      for (int i = 0; i < dim; i++) sum += (double)row[i];
      double mu = sum / (double)dim;
      double vs = 0;
      for (int i = 0; i < dim; i++) {
        double d = (double)row[i] - mu;
        vs += d * d;
      }
      float rs = (float)(1.0 / std::sqrt(vs / (double)dim + (double)eps));
      float m = (float)mu;
      if (mean) mean[r] = m;
      if (rstd) rstd[r] = rs;
      float *o = y + (size_t)r * dim;
      if (b) {
        for (int i = 0; i < dim; i++) o[i] = (row[i] - m) * rs * w[i] + b[i];
      } else {
        for (int i = 0; i < dim; i++) o[i] = (row[i] - m) * rs * w[i];
      }
    }
  });
}

// gelu, ops.go:140-142.
inline float gelu(float x) {
  const double sqrt2 = 1.41421356237309504880168872420969808;
  return 0.5f * x * (1.0f + (float)std::erf((double)x * sqrt2 / 2.0));
}

// ropeTables, model.go:242-258.
void rope_tables(const std::vector<int32_t> &pos, int headDim, double theta, std::vector<float> &cs,
                 std::vector<float> &sn) {
  int half = headDim / 2;
  std::vector<double> inv(half);
  for (int i = 0; i < half; i++) inv[i] = 1.0 / std::pow(theta, (double)(2 * i) / (double)headDim);
  cs.assign(pos.size() * half, 0);
  sn.assign(pos.size() * half, 0);
  for (size_t s = 0; s < pos.size(); s++)
    for (int i = 0; i < half; i++) {
      double f = (double)(float)((double)pos[s] * inv[i]);
      cs[s * half + i] = (float)std::cos(f);
      sn[s * half + i] = (float)std::sin(f);
    }
}

// geluGrad, ops.go:145-150: d gelu(x) / dx with erf and exp in float64.
inline float gelu_grad(float x) {
  const double sqrt2 = 1.41421356237309504880168872420969808;
  const double pi = 3.14159265358979323846264338327950288;
  double xf = (double)x;
  double cdf = 0.5 * (1 + std::erf(xf * sqrt2 / 2));
  double pdf = std::exp(-0.5 * xf * xf) / std::sqrt(2 * pi);
  return (float)(cdf + xf * pdf);
}

// applyRope, ops.go:155-175; inverse transposes the rotation (backward pass).
void apply_rope(float *qkv, int T, int H, int heads, int D, const float *cs, const float *sn, bool inverse = false) {
  int half = D / 2, stride = 3 * H;
  parallel_for(T, [&](int lo, int hi) {
    for (int t = lo; t < hi; t++)
      for (int hd = 0; hd < heads; hd++)
        for (int off : {hd * D, H + hd * D}) {
          float *v = qkv + (size_t)t * stride + off;
          for (int i = 0; i < half; i++) {
            float c = cs[(size_t)t * half + i], s = sn[(size_t)t * half + i];
            if (inverse) s = -s;
            float a = v[i], b = v[i + half];
            v[i] = a * c - b * s;
            v[i + half] = b * c + a * s;
          }
        }
  });
}

// softmaxMasked, forward.go:382-409.
void softmax_masked(float *P, int n, float scale, const uint8_t *mask) {
  for (int i = 0; i < n; i++) {
    float *row = P + (size_t)i * n;
    float maxv = -INFINITY;
    for (int j = 0; j < n; j++) {
      if (mask && mask[(size_t)i * n + j] == 0) continue;
      float v = row[j] * scale;
      if (v > maxv) maxv = v;
    }
    double sum = 0;
    for (int j = 0; j < n; j++) {
      if (mask && mask[(size_t)i * n + j] == 0) {
        row[j] = 0;
        continue;
      }
      float e = (float)std::exp((double)(row[j] * scale - maxv));
      row[j] = e;
      sum += (double)e;
    }
    float inv = (float)(1.0 / sum);
    for (int j = 0; j < n; j++) row[j] *= inv;
  }
}

struct SeqInfo {
  int off, n;
  size_t pOff = 0;  // offset of this sequence's kept attention probabilities
  std::vector<uint8_t> full, slide;  // full empty == nil (all allowed)
};

struct Debug {
  float *hs;    // (L+1) x T x H : input of each layer, then the encoder output
  float *n1;    // L x T x H     : attention input (attn_norm output, layer 0: identity)
  float *attn;  // L x T x H     : Wo . ctx, before the residual add
};

void linear(float *y, const float *x, int T, int K, const float *w, int N) {
  sgemm(g_workers, false, true, T, N, K, x, K, w, K, y, N, false);
}

// attnFwd, forward.go:347-378. With pkeep (training) the probabilities are
// kept there, n x n per (sequence, head) at pOff + head*n*n; otherwise P is
// per-item scratch.
void attn_fwd(const Config &cfg, const std::vector<SeqInfo> &seqs, float *ctx, const float *qkv, bool sliding,
              float *pkeep = nullptr) {
  int H = cfg.hidden, heads = cfg.heads, D = H / heads, stride = 3 * H;
  float scale = (float)(1.0 / std::sqrt((double)D));
  int items = (int)seqs.size() * heads;
  parallel_for(items, [&](int lo, int hi) {
    std::vector<float> P;
    for (int it = lo; it < hi; it++) {
      int si = it / heads, hd = it % heads;
      const SeqInfo &s = seqs[si];
      int n = s.n;
      float *Pp;
      if (pkeep) {
        Pp = pkeep + s.pOff + (size_t)hd * n * n;
      } else {
        P.resize((size_t)n * n);
        Pp = P.data();
      }
      const float *q = qkv + (size_t)s.off * stride + hd * D;
      const float *k = qkv + (size_t)s.off * stride + H + hd * D;
      const float *v = qkv + (size_t)s.off * stride + 2 * H + hd * D;
      sgemm(1, false, true, n, n, D, q, stride, k, stride, Pp, n, false);
      const uint8_t *mask = sliding ? s.slide.data() : (s.full.empty() ? nullptr : s.full.data());
      softmax_masked(Pp, n, scale, mask);
      round_if(RND_P, Pp, (size_t)n * n);
      sgemm(1, false, false, n, D, n, Pp, n, v, stride, ctx + (size_t)s.off * H + hd * D, H, false);
    }
  });
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI used by tests/ and bench.py through ctypes.
extern "C" {

void orc_set_workers(int n) { g_workers = n < 1 ? 1 : n; }

// Stage rounding switches (RND_* bits above); 0 restores the reference.
void orc_set_rounding(int mask) { g_round = mask; }
// Restricts the stage rounding to encoder layers [lo, hi).
void orc_set_rounding_layers(int lo, int hi) {
  g_round_lo = lo;
  g_round_hi = hi;
}
int orc_get_workers(void) { return g_workers; }

// blas.Sgemm (gemm.go:61) with an explicit worker count (Sgemm1 == workers 1).
void orc_sgemm(int workers, int transA, int transB, int M, int N, int K, const float *A, int lda, const float *B,
               int ldb, float *C, int ldc, int accumulate) {
  sgemm(workers, transA != 0, transB != 0, M, N, K, A, lda, B, ldb, C, ldc, accumulate != 0);
}

// The same summation order written per element (no blocking): C (=0 unless
// accumulate); for each 256-wide k block: acc = 0; acc = fma(a,b,acc) in
// increasing k; C += acc. Used to pin orc_sgemm bit-for-bit.
void orc_sgemm_ref(int transA, int transB, int M, int N, int K, const float *A, int lda, const float *B, int ldb,
                   float *C, int ldc, int accumulate) {
  for (int i = 0; i < M; i++)
    for (int j = 0; j < N; j++) {
      float c = accumulate ? C[(size_t)i * ldc + j] : 0.0f;
      for (int pc = 0; pc < K; pc += KC) {
        float acc = 0.0f;
        for (int k = pc; k < std::min(K, pc + KC); k++) {
          float a = transA ? A[(size_t)k * lda + i] : A[(size_t)i * lda + k];
          float b = transB ? B[(size_t)j * ldb + k] : B[(size_t)k * ldb + j];
          acc = std::fma(a, b, acc);
        }
        c = c + acc;
      }
      C[(size_t)i * ldc + j] = c;
    }
}

// BuildSequence, forward.go:28-56. Returns the number of mask positions
// written to mask_pos (capacity n). *has_opt is 1 when OptID is non-nil.
int orc_build_sequence(const int32_t *ids, int n, int32_t mask_id, int independent, int32_t *pos, int32_t *opt,
                       int32_t *mask_pos, int *has_opt) {
  int nm = 0;
  for (int i = 0; i < n; i++) {
    pos[i] = i;
    if (ids[i] == mask_id) mask_pos[nm++] = i;
  }
  *has_opt = 0;
  if (!independent || nm == 0) return nm;
  int last = n - 1;
  *has_opt = 1;
  for (int i = 0; i < n; i++) opt[i] = -1;
  int prefix = mask_pos[0];
  for (int k = 0; k < nm; k++) {
    int start = mask_pos[k];
    int end = k + 1 < nm ? mask_pos[k + 1] : last;
    for (int i = start; i < end; i++) {
      opt[i] = k;
      pos[i] = prefix + i - start;
    }
  }
  return nm;
}

void *orc_model_new(int hidden, int inter, int heads, int layers, int vocab, float eps, int half_window,
                    double theta_g, double theta_l, const uint8_t *sliding) {
  Model *m = new Model;
  m->cfg = Config{hidden, inter, heads, layers, vocab, eps, half_window, theta_g, theta_l,
                  std::vector<uint8_t>(sliding, sliding + layers)};
  return m;
}

void orc_model_free(void *m) { delete (Model *)m; }

void orc_model_set(void *mp, const char *name, const float *data, int64_t n) {
  Model *m = (Model *)mp;
  m->w[name].assign(data, data + n);
}

}  // extern "C"

namespace {

// Per-layer activations a training forward keeps (layerCache, forward.go:65-73).
struct LayerCache {
  std::vector<float> n1, mean1, rstd1, qkv, ctx, h1, n2, mean2, rstd2, wi, act, P;
};

// The parts of nn.Cache (forward.go:77-110) that Backward reads.
struct TrainCache {
  int trainFrom = 0, T = 0, R = 0;
  std::vector<SeqInfo> seqs;
  std::vector<int32_t> ids;
  std::vector<float> cosG, sinG, cosL, sinL;
  std::vector<float> embX, embMean, embRstd;
  std::vector<std::vector<float>> hs;  // hs[l] = input of layer l (kept for l >= trainFrom), hs[L] = output
  std::vector<LayerCache> lc;
  std::vector<int> rowTok;
  std::vector<float> fN, fMean, fRstd, s1, m1, r1, d, ge, s2, m2, r2;
};

// Model.Forward (forward.go:129-245) + layerFwd (:284-343) + HeadForward
// (:250-282). Sequences are concatenated: seq_len[nseq], ids/pos/opt[T];
// has_opt[s] = 0 means OptID nil for that sequence. mask_pos holds each
// sequence's mask positions (local indices), nmask[s] of them. With tc
// (training) the activations of layers >= trainFrom, the attention
// probabilities and the head's intermediates are kept there; layers below
// trainFrom keep nothing (forward.go:226-236). Returns 0, or a negative code
// mirroring the reference's validation errors:
//   -1 malformed sequence, -2 no options, -3 mask position out of range,
//   -4 token id out of range, -5 missing weight.
int forward_impl(const Model &m, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos_in,
                 const int32_t *opt_in, const uint8_t *has_opt, const int32_t *nmask, const int32_t *mask_pos,
                 float *logits, float *dbg_hs, float *dbg_n1, float *dbg_attn, TrainCache *tc, int trainFrom) {
  const Config &cfg = m.cfg;
  int H = cfg.hidden, I = cfg.inter, D = H / cfg.heads, L = cfg.layers;
  if (tc) trainFrom = std::min(std::max(trainFrom, 0), L + 1);
  else trainFrom = L + 1;
  std::vector<SeqInfo> seqs;
  std::vector<int32_t> pos;
  std::vector<int> rowTok;
  int T = 0, mp_off = 0;
  size_t pTotal = 0;
  for (int si = 0; si < nseq; si++) {
    int n = seq_len[si];
    if (n <= 0) return -1;
    if (nmask[si] == 0) return -2;
    SeqInfo info;
    info.off = T;
    info.n = n;
    info.pOff = pTotal;
    const int32_t *op = opt_in + T;
    const int32_t *ps = pos_in + T;
    if (has_opt[si]) {
      info.full.assign((size_t)n * n, 0);
      for (int i = 0; i < n; i++) {
        int oi = op[i];
        for (int j = 0; j < n; j++) {
          int oj = op[j];
          if ((oi == -1 && oj == -1) || (oi != -1 && (oj == -1 || oi == oj))) info.full[(size_t)i * n + j] = 1;
        }
      }
    }
    info.slide.assign((size_t)n * n, 0);
    int w = cfg.half_window;
    for (int i = 0; i < n; i++)
      for (int j = 0; j < n; j++) {
        int d = ps[i] - ps[j];
        if (d < 0) d = -d;
        if (d <= w && (info.full.empty() || info.full[(size_t)i * n + j] == 1)) info.slide[(size_t)i * n + j] = 1;
      }
    seqs.push_back(std::move(info));
    pos.insert(pos.end(), ps, ps + n);
    for (int k = 0; k < nmask[si]; k++) {
      int mpos = mask_pos[mp_off + k];
      if (mpos < 0 || mpos >= n) return -3;
      rowTok.push_back(T + mpos);
    }
    mp_off += nmask[si];
    T += n;
    pTotal += (size_t)n * n * cfg.heads;
  }
  for (int t = 0; t < T; t++)
    if (ids[t] < 0 || ids[t] >= cfg.vocab) return -4;
  int R = (int)rowTok.size();

  TrainCache scratch;
  TrainCache &c = tc ? *tc : scratch;
  c.trainFrom = trainFrom;
  c.T = T;
  c.R = R;
  c.ids.assign(ids, ids + T);
  c.rowTok = rowTok;
  rope_tables(pos, D, cfg.theta_g, c.cosG, c.sinG);
  rope_tables(pos, D, cfg.theta_l, c.cosL, c.sinL);

  const float *tok = m.get("model.embeddings.tok_embeddings.weight");
  const float *embNorm = m.get("model.embeddings.norm.weight");
  if (!tok || !embNorm) return -5;
  c.embX.assign((size_t)T * H, 0);
  c.embMean.assign(T, 0);
  c.embRstd.assign(T, 0);
  parallel_for(T, [&](int lo, int hi) {
    for (int t = lo; t < hi; t++) std::memcpy(&c.embX[(size_t)t * H], tok + (size_t)ids[t] * H, sizeof(float) * H);
  });
  c.hs.assign(L + 1, {});
  c.lc.assign(L, {});
  for (int l = 0; l <= L; l++)
    if (l >= trainFrom || l == L) c.hs[l].assign((size_t)T * H, 0);
  std::vector<float> ping((size_t)T * H), pong((size_t)T * H);
  float *cur = trainFrom == 0 ? c.hs[0].data() : ping.data();
  layer_norm(cur, c.embX.data(), T, H, embNorm, nullptr, cfg.eps, c.embMean.data(), c.embRstd.data());
  std::vector<float> x0r;  // layer 0's QKV operand when rounded (the residual stays exact)
  if (dbg_hs) std::memcpy(dbg_hs, cur, sizeof(float) * T * H);

  LayerCache frozen;
  std::vector<float> tmp((size_t)T * H);
  std::vector<float> fold_prev;  // RND_XFOLDC: the previous LayerNorm's row means
  for (int l = 0; l < L; l++) {
    std::string p = "model.layers." + std::to_string(l) + ".";
    const float *attnNorm = m.get(p + "attn_norm.weight");
    const float *Wqkv = m.get(p + "attn.Wqkv.weight");
    const float *Wo = m.get(p + "attn.Wo.weight");
    const float *mlpNorm = m.get(p + "mlp_norm.weight");
    const float *Wi = m.get(p + "mlp.Wi.weight");
    const float *MlpWo = m.get(p + "mlp.Wo.weight");
    if (!Wqkv || !Wo || !mlpNorm || !Wi || !MlpWo || (l > 0 && !attnNorm)) return -5;
    float *out;
    if (l + 1 >= trainFrom || l + 1 == L) out = c.hs[l + 1].data();
    else out = cur == ping.data() ? pong.data() : ping.data();
    const bool keep = l >= trainFrom;
    LayerCache &lc = keep ? c.lc[l] : frozen;
    bool sliding = cfg.sliding[l] != 0;
    // layerFwd, forward.go:284-343.
    g_round_now = l >= g_round_lo && l < g_round_hi ? g_round : 0;
    const float *in = cur;
    const float *x1 = in;
    if (l > 0) {  // layer 0 has no attn_norm (model.go:13-14, forward.go:289-294)
      lc.n1.resize((size_t)T * H);
      lc.mean1.resize(T);
      lc.rstd1.resize(T);
      layer_norm(lc.n1.data(), in, T, H, attnNorm, nullptr, cfg.eps, lc.mean1.data(), lc.rstd1.data());
      x1 = lc.n1.data();
      round_if(RND_XN, lc.n1.data(), (size_t)T * H);
      fold_if(lc.n1.data(), in, T, H, attnNorm, lc.mean1.data(), lc.rstd1.data(),
              fold_prev.empty() ? nullptr : fold_prev.data());
    } else if (g_round_now & RND_XN) {
      x0r.assign(in, in + (size_t)T * H);
      round_if(RND_XN, x0r.data(), x0r.size());
      x1 = x0r.data();
    }
    if (dbg_n1) std::memcpy(dbg_n1 + (size_t)l * T * H, x1, sizeof(float) * T * H);
    lc.qkv.resize((size_t)T * 3 * H);
    linear(lc.qkv.data(), x1, T, H, Wqkv, 3 * H);
    round_if(RND_QKV, lc.qkv.data(), (size_t)T * 3 * H);
    apply_rope(lc.qkv.data(), T, H, cfg.heads, D, sliding ? c.cosL.data() : c.cosG.data(),
               sliding ? c.sinL.data() : c.sinG.data());
    if (g_round_now & RND_QK)
      for (int t = 0; t < T; t++) round_if(RND_QK, &lc.qkv[(size_t)t * 3 * H], (size_t)2 * H);
    lc.ctx.resize((size_t)T * H);
    if (keep) lc.P.assign(pTotal, 0);
    attn_fwd(cfg, seqs, lc.ctx.data(), lc.qkv.data(), sliding, keep ? lc.P.data() : nullptr);
    round_if(RND_CTX, lc.ctx.data(), (size_t)T * H);
    linear(tmp.data(), lc.ctx.data(), T, H, Wo, H);
    if (dbg_attn) std::memcpy(dbg_attn + (size_t)l * T * H, tmp.data(), sizeof(float) * T * H);
    lc.h1.resize((size_t)T * H);
    parallel_for(T * H, [&](int lo, int hi) {
      for (int i = lo; i < hi; i++) lc.h1[i] = in[i] + tmp[i];
    });
    lc.n2.resize((size_t)T * H);
    lc.mean2.resize(T);
    lc.rstd2.resize(T);
    layer_norm(lc.n2.data(), lc.h1.data(), T, H, mlpNorm, nullptr, cfg.eps, lc.mean2.data(), lc.rstd2.data());
    round_if(RND_XN, lc.n2.data(), (size_t)T * H);
    fold_if(lc.n2.data(), lc.h1.data(), T, H, mlpNorm, lc.mean2.data(), lc.rstd2.data(),
            l > 0 ? lc.mean1.data() : nullptr);
    fold_prev = lc.mean2;
    lc.wi.resize((size_t)T * 2 * I);
    linear(lc.wi.data(), lc.n2.data(), T, H, Wi, 2 * I);
    lc.act.resize((size_t)T * I);
    parallel_for(T, [&](int lo, int hi) {
      for (int t = lo; t < hi; t++) {
        const float *row = &lc.wi[(size_t)t * 2 * I];
        float *a = &lc.act[(size_t)t * I];
        for (int i = 0; i < I; i++) a[i] = gelu(row[i]) * row[I + i];
      }
    });
    round_if(RND_ACT, lc.act.data(), (size_t)T * I);
    linear(tmp.data(), lc.act.data(), T, I, MlpWo, H);
    parallel_for(T * H, [&](int lo, int hi) {
      for (int i = lo; i < hi; i++) out[i] = lc.h1[i] + tmp[i];
    });
    cur = out;
    if (dbg_hs) std::memcpy(dbg_hs + (size_t)(l + 1) * T * H, cur, sizeof(float) * T * H);
  }
  c.seqs = std::move(seqs);
  std::vector<float> rows((size_t)R * H);
  for (int r = 0; r < R; r++) std::memcpy(&rows[(size_t)r * H], &cur[(size_t)rowTok[r] * H], sizeof(float) * H);

  // HeadForward, forward.go:250-282.
  const float *finalNorm = m.get("model.final_norm.weight");
  const float *inW = m.get("scorer.input_norm.weight"), *inB = m.get("scorer.input_norm.bias");
  const float *denseW = m.get("scorer.dense.weight"), *denseB = m.get("scorer.dense.bias");
  const float *normW = m.get("scorer.norm.weight"), *normB = m.get("scorer.norm.bias");
  const float *outW = m.get("scorer.out_proj.weight"), *outB = m.get("scorer.out_proj.bias");
  if (!finalNorm || !inW || !inB || !denseW || !denseB || !normW || !normB || !outW || !outB) return -5;
  int half = H / 2;
  c.fN.assign((size_t)R * H, 0);
  c.fMean.assign(R, 0);
  c.fRstd.assign(R, 0);
  c.s1.assign((size_t)R * H, 0);
  c.m1.assign(R, 0);
  c.r1.assign(R, 0);
  c.d.assign((size_t)R * half, 0);
  c.ge.assign((size_t)R * half, 0);
  c.s2.assign((size_t)R * half, 0);
  c.m2.assign(R, 0);
  c.r2.assign(R, 0);
  layer_norm(c.fN.data(), rows.data(), R, H, finalNorm, nullptr, cfg.eps, c.fMean.data(), c.fRstd.data());
  layer_norm(c.s1.data(), c.fN.data(), R, H, inW, inB, 1e-5f, c.m1.data(), c.r1.data());
  linear(c.d.data(), c.s1.data(), R, H, denseW, half);
  for (int r = 0; r < R; r++)
    for (int i = 0; i < half; i++) {
      c.d[(size_t)r * half + i] += denseB[i];
      c.ge[(size_t)r * half + i] = gelu(c.d[(size_t)r * half + i]);
    }
  layer_norm(c.s2.data(), c.ge.data(), R, half, normW, normB, 1e-5f, c.m2.data(), c.r2.data());
  for (int r = 0; r < R; r++) {
    float s = 0;
    for (int i = 0; i < half; i++) s += c.s2[(size_t)r * half + i] * outW[i];
    logits[r] = s + outB[0];
  }
  return 0;
}

// layerNormBwd, ops.go:94-135: ADDS the input gradient into dx and
// accumulates dw (and db when non-null); per-chunk partial sums are merged
// under a lock as the reference does.
void layer_norm_bwd(float *dx, const float *dy, const float *x, int rows, int dim, const float *w, const float *mean,
                    const float *rstd, float *dw, float *db) {
  std::mutex mu;
  parallel_for(rows, [&](int lo, int hi) {
    std::vector<float> pw(dim, 0.0f), pb(db ? dim : 0, 0.0f), xh(dim);
    for (int r = lo; r < hi; r++) {
      const float *row = x + (size_t)r * dim;
      const float *g = dy + (size_t)r * dim;
      float m = mean[r], rs = rstd[r];
      double s1 = 0, s2 = 0;
      for (int i = 0; i < dim; i++) {
        xh[i] = (row[i] - m) * rs;
        float gw = g[i] * w[i];
        s1 += (double)gw;
        s2 += (double)(gw * xh[i]);
        pw[i] += g[i] * xh[i];
        if (db) pb[i] += g[i];
      }
      float a = (float)(s1 / (double)dim), b = (float)(s2 / (double)dim);
      float *o = dx + (size_t)r * dim;
      for (int i = 0; i < dim; i++) o[i] += rs * (g[i] * w[i] - a - xh[i] * b);
    }
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < dim; i++) dw[i] += pw[i];
    if (db)
      for (int i = 0; i < dim; i++) db[i] += pb[i];
  });
}

// attnBwd, backward.go:117-159: dqkv (before the RoPE inverse) from dctx,
// the rotated qkv and the kept probabilities.
void attn_bwd(const Config &cfg, const std::vector<SeqInfo> &seqs, float *dqkv, const float *dctx, const float *qkv,
              const float *P) {
  int H = cfg.hidden, D = H / cfg.heads, heads = cfg.heads, stride = 3 * H;
  float scale = (float)(1.0 / std::sqrt((double)D));
  int items = (int)seqs.size() * heads;
  parallel_for(items, [&](int lo, int hi) {
    std::vector<float> dP;
    for (int it = lo; it < hi; it++) {
      int si = it / heads, hd = it % heads;
      const SeqInfo &s = seqs[si];
      int n = s.n;
      const float *p = P + s.pOff + (size_t)hd * n * n;
      dP.assign((size_t)n * n, 0);
      const float *q = qkv + (size_t)s.off * stride + hd * D;
      const float *k = qkv + (size_t)s.off * stride + H + hd * D;
      const float *v = qkv + (size_t)s.off * stride + 2 * H + hd * D;
      const float *dc = dctx + (size_t)s.off * H + hd * D;
      sgemm(1, false, true, n, n, D, dc, H, v, stride, dP.data(), n, false);  // dP = dctx . V^T
      for (int i = 0; i < n; i++) {
        const float *pr = p + (size_t)i * n;
        float *dr = dP.data() + (size_t)i * n;
        float dot = 0;
        for (int j = 0; j < n; j++) dot += pr[j] * dr[j];
        for (int j = 0; j < n; j++) dr[j] = pr[j] * (dr[j] - dot) * scale;
      }
      float *dq = dqkv + (size_t)s.off * stride + hd * D;
      float *dk = dqkv + (size_t)s.off * stride + H + hd * D;
      float *dv = dqkv + (size_t)s.off * stride + 2 * H + hd * D;
      sgemm(1, true, false, n, D, n, p, n, dc, H, dv, stride, false);         // dV = P^T . dctx
      sgemm(1, false, false, n, D, n, dP.data(), n, k, stride, dq, stride, false);  // dQ = dS . K
      sgemm(1, true, false, n, D, n, dP.data(), n, q, stride, dk, stride, false);   // dK = dS^T . Q
    }
  });
}

float *grad_of(Model &g, const std::string &name) {
  auto it = g.w.find(name);
  return it == g.w.end() ? nullptr : it->second.data();
}

// HeadBackward, backward.go:161-196: dlogits through the scorer head and the
// final norm; returns dRows (R x H).
std::vector<float> head_backward(const Model &m, const TrainCache &c, const float *rows, const float *dlogits,
                                 Model &g) {
  const Config &cfg = m.cfg;
  int H = cfg.hidden, R = c.R, half = H / 2;
  const float *outW = m.get("scorer.out_proj.weight"), *denseW = m.get("scorer.dense.weight");
  std::vector<float> ds2((size_t)R * half);
  float *gOutB = grad_of(g, "scorer.out_proj.bias"), *gOutW = grad_of(g, "scorer.out_proj.weight");
  for (int r = 0; r < R; r++) {
    float dl = dlogits[r];
    gOutB[0] += dl;
    const float *row = &c.s2[(size_t)r * half];
    for (int i = 0; i < half; i++) {
      gOutW[i] += dl * row[i];
      ds2[(size_t)r * half + i] = dl * outW[i];
    }
  }
  std::vector<float> dge((size_t)R * half, 0.0f);
  layer_norm_bwd(dge.data(), ds2.data(), c.ge.data(), R, half, m.get("scorer.norm.weight"), c.m2.data(), c.r2.data(),
                 grad_of(g, "scorer.norm.weight"), grad_of(g, "scorer.norm.bias"));
  std::vector<float> dd((size_t)R * half);
  float *gDenseB = grad_of(g, "scorer.dense.bias");
  for (int r = 0; r < R; r++)
    for (int i = 0; i < half; i++) {
      float v = dge[(size_t)r * half + i] * gelu_grad(c.d[(size_t)r * half + i]);
      dd[(size_t)r * half + i] = v;
      gDenseB[i] += v;
    }
  sgemm(g_workers, true, false, half, H, R, dd.data(), half, c.s1.data(), H, grad_of(g, "scorer.dense.weight"), H,
        true);
  std::vector<float> ds1((size_t)R * H);
  sgemm(g_workers, false, false, R, H, half, dd.data(), half, denseW, H, ds1.data(), H, false);
  std::vector<float> dfN((size_t)R * H, 0.0f);
  layer_norm_bwd(dfN.data(), ds1.data(), c.fN.data(), R, H, m.get("scorer.input_norm.weight"), c.m1.data(),
                 c.r1.data(), grad_of(g, "scorer.input_norm.weight"), grad_of(g, "scorer.input_norm.bias"));
  std::vector<float> dRows((size_t)R * H, 0.0f);
  layer_norm_bwd(dRows.data(), dfN.data(), rows, R, H, m.get("model.final_norm.weight"), c.fMean.data(),
                 c.fRstd.data(), grad_of(g, "model.final_norm.weight"), nullptr);
  return dRows;
}

// Model.Backward, backward.go:19-115: accumulates into g the gradient of a
// loss whose derivative with respect to the option logits is dlogits.
void backward_impl(const Model &m, const TrainCache &c, const float *dlogits, Model &g, bool trainEmb) {
  const Config &cfg = m.cfg;
  int H = cfg.hidden, I = cfg.inter, D = H / cfg.heads, L = cfg.layers;
  int T = c.T, R = c.R;
  const float *hL = c.hs[L].data();
  std::vector<float> rows((size_t)R * H);
  for (int r = 0; r < R; r++) std::memcpy(&rows[(size_t)r * H], hL + (size_t)c.rowTok[r] * H, sizeof(float) * H);
  std::vector<float> dRows = head_backward(m, c, rows.data(), dlogits, g);
  std::vector<float> dcur((size_t)T * H, 0.0f);
  for (int r = 0; r < R; r++)
    std::memcpy(&dcur[(size_t)c.rowTok[r] * H], &dRows[(size_t)r * H], sizeof(float) * H);

  std::vector<float> dh1((size_t)T * H), dact((size_t)T * I), dwi((size_t)T * 2 * I), dn2((size_t)T * H, 0.0f),
      dctx((size_t)T * H), dqkv((size_t)T * 3 * H), dn1((size_t)T * H), dprev((size_t)T * H);
  for (int l = L - 1; l >= c.trainFrom && l >= 0; l--) {
    std::string p = "model.layers." + std::to_string(l) + ".";
    const LayerCache &lc = c.lc[l];
    const float *in = c.hs[l].data();
    const float *dout = dcur.data();
    const float *attnNorm = m.get(p + "attn_norm.weight");

    // MLP: out = h1 + Wo(act)
    sgemm(g_workers, false, false, T, I, H, dout, H, m.get(p + "mlp.Wo.weight"), I, dact.data(), I, false);
    sgemm(g_workers, true, false, H, I, T, dout, H, lc.act.data(), I, grad_of(g, p + "mlp.Wo.weight"), I, true);
    parallel_for(T, [&](int lo, int hi) {
      for (int t = lo; t < hi; t++) {
        const float *row = &lc.wi[(size_t)t * 2 * I];
        const float *da = &dact[(size_t)t * I];
        float *dw = &dwi[(size_t)t * 2 * I];
        for (int i = 0; i < I; i++) {
          float a = row[i], gt = row[I + i];
          dw[i] = da[i] * gt * gelu_grad(a);
          dw[I + i] = da[i] * gelu(a);
        }
      }
    });
    sgemm(g_workers, true, false, 2 * I, H, T, dwi.data(), 2 * I, lc.n2.data(), H, grad_of(g, p + "mlp.Wi.weight"), H,
          true);
    sgemm(g_workers, false, false, T, H, 2 * I, dwi.data(), 2 * I, m.get(p + "mlp.Wi.weight"), H, dn2.data(), H,
          false);
    dh1 = dcur;  // residual path
    layer_norm_bwd(dh1.data(), dn2.data(), lc.h1.data(), T, H, m.get(p + "mlp_norm.weight"), lc.mean2.data(),
                   lc.rstd2.data(), grad_of(g, p + "mlp_norm.weight"), nullptr);

    // Attention: h1 = in + Wo(ctx)
    sgemm(g_workers, false, false, T, H, H, dh1.data(), H, m.get(p + "attn.Wo.weight"), H, dctx.data(), H, false);
    sgemm(g_workers, true, false, H, H, T, dh1.data(), H, lc.ctx.data(), H, grad_of(g, p + "attn.Wo.weight"), H, true);
    attn_bwd(cfg, c.seqs, dqkv.data(), dctx.data(), lc.qkv.data(), lc.P.data());
    const bool sliding = cfg.sliding[l] != 0;
    apply_rope(dqkv.data(), T, H, cfg.heads, D, sliding ? c.cosL.data() : c.cosG.data(),
               sliding ? c.sinL.data() : c.sinG.data(), true);
    const float *n1 = attnNorm ? lc.n1.data() : in;
    sgemm(g_workers, true, false, 3 * H, H, T, dqkv.data(), 3 * H, n1, H, grad_of(g, p + "attn.Wqkv.weight"), H, true);
    sgemm(g_workers, false, false, T, H, 3 * H, dqkv.data(), 3 * H, m.get(p + "attn.Wqkv.weight"), H, dn1.data(), H,
          false);
    dprev = dh1;  // residual path
    if (attnNorm) {
      layer_norm_bwd(dprev.data(), dn1.data(), in, T, H, attnNorm, lc.mean1.data(), lc.rstd1.data(),
                     grad_of(g, p + "attn_norm.weight"), nullptr);
    } else {
      parallel_for(T * H, [&](int lo, int hi) {
        for (int i = lo; i < hi; i++) dprev[i] += dn1[i];
      });
    }
    std::swap(dcur, dprev);
    std::fill(dn2.begin(), dn2.end(), 0.0f);
  }

  // Embeddings.
  if (trainEmb && c.trainFrom == 0) {
    std::vector<float> dE((size_t)T * H, 0.0f);
    layer_norm_bwd(dE.data(), dcur.data(), c.embX.data(), T, H, m.get("model.embeddings.norm.weight"),
                   c.embMean.data(), c.embRstd.data(), grad_of(g, "model.embeddings.norm.weight"), nullptr);
    float *gTok = grad_of(g, "model.embeddings.tok_embeddings.weight");
    for (int t = 0; t < T; t++) {
      float *dst = gTok + (size_t)c.ids[t] * H;
      const float *src = &dE[(size_t)t * H];
      for (int i = 0; i < H; i++) dst[i] += src[i];
    }
  }
}

// Tensor order and shapes of nn.Model.Tensors() (model.go:51-84): name,
// element count, rank.
struct TensorDesc {
  std::string name;
  size_t n;
  int rank;
};
std::vector<TensorDesc> tensor_list(const Config &cfg) {
  size_t H = cfg.hidden, I = cfg.inter;
  std::vector<TensorDesc> t = {{"model.embeddings.tok_embeddings.weight", (size_t)cfg.vocab * H, 2},
                               {"model.embeddings.norm.weight", H, 1}};
  for (int l = 0; l < cfg.layers; l++) {
    std::string p = "model.layers." + std::to_string(l) + ".";
    if (l > 0) t.push_back({p + "attn_norm.weight", H, 1});
    t.push_back({p + "attn.Wqkv.weight", 3 * H * H, 2});
    t.push_back({p + "attn.Wo.weight", H * H, 2});
    t.push_back({p + "mlp_norm.weight", H, 1});
    t.push_back({p + "mlp.Wi.weight", 2 * I * H, 2});
    t.push_back({p + "mlp.Wo.weight", H * I, 2});
  }
  t.push_back({"model.final_norm.weight", H, 1});
  t.push_back({"scorer.input_norm.weight", H, 1});
  t.push_back({"scorer.input_norm.bias", H, 1});
  t.push_back({"scorer.dense.weight", H / 2 * H, 2});
  t.push_back({"scorer.dense.bias", H / 2, 1});
  t.push_back({"scorer.norm.weight", H / 2, 1});
  t.push_back({"scorer.norm.bias", H / 2, 1});
  t.push_back({"scorer.out_proj.weight", H / 2, 2});
  t.push_back({"scorer.out_proj.bias", 1, 1});
  return t;
}

// AdamW, internal/train/optim.go:11-145.
struct AdamW {
  float beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f, weightDecay = 0;
  Model *model = nullptr, *grads = nullptr;
  std::vector<TensorDesc> list;
  std::vector<std::vector<float>> m, v;
  std::vector<bool> frozen, head, decay;
  int step = 0;
};

// NewAdamW, optim.go:31-65.
AdamW *adamw_new(Model *model, Model *grads, float wd, int trainFrom, bool trainEmb, bool headOnly) {
  AdamW *o = new AdamW;
  o->weightDecay = wd;
  o->model = model;
  o->grads = grads;
  o->list = tensor_list(model->cfg);
  for (const TensorDesc &t : o->list) {
    bool frozen = false, head = t.name.rfind("scorer.", 0) == 0, decay = t.rank == 2;
    if (t.name == "model.embeddings.tok_embeddings.weight") {
      frozen = !trainEmb || trainFrom > 0;
      decay = false;
    } else if (t.name == "model.embeddings.norm.weight") {
      frozen = trainFrom > 0;
    } else if (t.name.rfind("model.layers.", 0) == 0) {
      int l = 0;
      for (size_t i = 13; i < t.name.size() && t.name[i] >= '0' && t.name[i] <= '9'; i++) l = l * 10 + (t.name[i] - '0');
      frozen = l < trainFrom;
    }
    if (headOnly && (t.name.rfind("model.embeddings.", 0) == 0 || t.name.rfind("model.layers.", 0) == 0))
      frozen = true;
    o->frozen.push_back(frozen);
    o->head.push_back(head);
    o->decay.push_back(decay);
    o->m.emplace_back(t.n, 0.0f);
    o->v.emplace_back(t.n, 0.0f);
  }
  return o;
}

// GradNorm, optim.go:68-90 (per-tensor float64 sums of squares).
double adamw_grad_norm(const AdamW &o) {
  double total = 0;
  for (size_t i = 0; i < o.list.size(); i++) {
    if (o.frozen[i]) continue;
    const std::vector<float> &d = o.grads->w.at(o.list[i].name);
    double s = 0;
    for (float v : d) s += (double)v * (double)v;
    total += s;
  }
  return std::sqrt(total);
}

// Update, optim.go:94-145.
void adamw_update(AdamW &o, float lr, float headLR, float gradScale) {
  o.step++;
  double b1c = 1 - std::pow((double)o.beta1, (double)o.step);
  double b2c = 1 - std::pow((double)o.beta2, (double)o.step);
  float stepSize = (float)(1 / b1c);
  float invSqrtB2c = (float)(1 / std::sqrt(b2c));
  for (size_t i = 0; i < o.list.size(); i++) {
    if (o.frozen[i]) continue;
    float rate = o.head[i] ? headLR : lr;
    float wd = o.decay[i] ? o.weightDecay * rate : 0.0f;
    std::vector<float> &p = o.model->w.at(o.list[i].name);
    const std::vector<float> &g = o.grads->w.at(o.list[i].name);
    std::vector<float> &m = o.m[i], &v = o.v[i];
    parallel_for((int)p.size(), [&](int lo, int hi) {
      for (int k = lo; k < hi; k++) {
        float gr = g[k] * gradScale;
        m[k] = o.beta1 * m[k] + (1 - o.beta1) * gr;
        v[k] = o.beta2 * v[k] + (1 - o.beta2) * gr * gr;
        float den = (float)std::sqrt((double)v[k]) * invSqrtB2c + o.eps;
        p[k] -= rate * stepSize * m[k] / den + wd * p[k];
      }
    });
  }
}

}  // namespace

extern "C" {

// Inference forward (Forward with trainFrom >= Layers); the dbg_* arrays, when
// non-null, receive each layer's input, attention input and Wo output.
int orc_forward(void *mp, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos_in,
                const int32_t *opt_in, const uint8_t *has_opt, const int32_t *nmask, const int32_t *mask_pos,
                float *logits, float *dbg_hs, float *dbg_n1, float *dbg_attn) {
  return forward_impl(*(Model *)mp, nseq, seq_len, ids, pos_in, opt_in, has_opt, nmask, mask_pos, logits, dbg_hs,
                      dbg_n1, dbg_attn, nullptr, 0);
}

// Training forward: Forward(c, batch, trainFrom) with the model's own cache.
int orc_forward_train(void *mp, int trainFrom, int nseq, const int32_t *seq_len, const int32_t *ids,
                      const int32_t *pos_in, const int32_t *opt_in, const uint8_t *has_opt, const int32_t *nmask,
                      const int32_t *mask_pos, float *logits) {
  Model &m = *(Model *)mp;
  if (!m.tc) m.tc = std::make_shared<TrainCache>();
  return forward_impl(m, nseq, seq_len, ids, pos_in, opt_in, has_opt, nmask, mask_pos, logits, nullptr, nullptr,
                      nullptr, m.tc.get(), trainFrom);
}

// Backward of the last orc_forward_train into the gradient model g (a model
// of the same configuration whose tensors accumulate). Returns -1 without a
// training forward.
int orc_backward(void *mp, const float *dlogits, void *gp, int trainEmb) {
  Model &m = *(Model *)mp;
  if (!m.tc) return -1;
  backward_impl(m, *m.tc, dlogits, *(Model *)gp, trainEmb != 0);
  return 0;
}

// NewLike + Zero (model.go:123-130): every tensor of the configuration, zeroed.
void orc_model_zero_like(void *dst, void *src) {
  Model &d = *(Model *)dst;
  for (const TensorDesc &t : tensor_list(((Model *)src)->cfg)) d.w[t.name].assign(t.n, 0.0f);
}

// Copies tensor name into out (n values); -1 if absent or of another size.
int orc_model_get(void *mp, const char *name, float *out, int64_t n) {
  Model &m = *(Model *)mp;
  auto it = m.w.find(name);
  if (it == m.w.end() || (int64_t)it->second.size() != n) return -1;
  std::memcpy(out, it->second.data(), sizeof(float) * n);
  return 0;
}

void *orc_adamw_new(void *model, void *grads, float wd, int trainFrom, int trainEmb, int headOnly) {
  return adamw_new((Model *)model, (Model *)grads, wd, trainFrom, trainEmb != 0, headOnly != 0);
}
void orc_adamw_free(void *o) { delete (AdamW *)o; }
double orc_adamw_grad_norm(void *o) { return adamw_grad_norm(*(AdamW *)o); }
void orc_adamw_update(void *o, float lr, float headLR, float gradScale) {
  adamw_update(*(AdamW *)o, lr, headLR, gradScale);
}
// Moment tensor (which 0 = m, 1 = v) of name; -1 if absent.
int orc_adamw_get(void *op, const char *name, int which, float *out, int64_t n) {
  AdamW &o = *(AdamW *)op;
  for (size_t i = 0; i < o.list.size(); i++)
    if (o.list[i].name == name) {
      const std::vector<float> &src = which ? o.v[i] : o.m[i];
      if ((int64_t)src.size() != n) return -1;
      std::memcpy(out, src.data(), sizeof(float) * n);
      return 0;
    }
  return -1;
}

// Pieces exposed for closed-form checks.
void orc_layer_norm(float *y, const float *x, int rows, int dim, const float *w, const float *b, float eps) {
  layer_norm(y, x, rows, dim, w, b, eps);
}
float orc_gelu(float x) { return gelu(x); }
float orc_gelu_grad(float x) { return gelu_grad(x); }
void orc_apply_rope_inverse(float *qkv, int T, int H, int heads, int D, const float *cs, const float *sn) {
  apply_rope(qkv, T, H, heads, D, cs, sn, true);
}
void orc_rope_tables(const int32_t *pos, int n, int headDim, double theta, float *cs, float *sn) {
  std::vector<int32_t> p(pos, pos + n);
  std::vector<float> c, s;
  rope_tables(p, headDim, theta, c, s);
  std::memcpy(cs, c.data(), sizeof(float) * c.size());
  std::memcpy(sn, s.data(), sizeof(float) * s.size());
}
void orc_apply_rope(float *qkv, int T, int H, int heads, int D, const float *cs, const float *sn) {
  apply_rope(qkv, T, H, heads, D, cs, sn);
}
void orc_softmax_masked(float *P, int n, float scale, const uint8_t *mask) { softmax_masked(P, n, scale, mask); }

// local.go:206-262 answer post-processing, float64.
// calibrated (local.go:225-232): p = softmax(logit / max(T, 1e-4)).
void orc_calibrated(const double *logits, int k, double temperature, double *probs) {
  double t = std::max(temperature, 1e-4);
  double maxv = -INFINITY;
  std::vector<double> sc(k);
  for (int i = 0; i < k; i++) {
    sc[i] = logits[i] / t;
    maxv = std::max(maxv, sc[i]);
  }
  double sum = 0;
  for (int i = 0; i < k; i++) {
    probs[i] = std::exp(sc[i] - maxv);
    sum += probs[i];
  }
  for (int i = 0; i < k; i++) probs[i] /= sum;
}
// round (local.go:234-237): RoundToEven(x * 10^places) / 10^places.
double orc_round(double x, int places) {
  double p = std::pow(10.0, (double)places);
  return std::nearbyint(x * p) / p;
}
// marginConfidence (local.go:241-252).
double orc_margin_confidence(const double *probs, int n) {
  if (n <= 1) return 1.0;
  double pmax = 0;
  for (int i = 0; i < n; i++) pmax = std::max(pmax, probs[i]);
  double c = ((double)n * pmax - 1) / (double)(n - 1);
  return orc_round(std::max(0.0, std::min(1.0, c)), 3);
}
// argmax (local.go:254-262): first index wins ties.
int orc_argmax(const double *x, int n) {
  int best = 0;
  for (int i = 0; i < n; i++)
    if (x[i] > x[best]) best = i;
  return best;
}

}  // extern "C"
