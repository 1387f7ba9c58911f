// Training kernels other than attention and the GEMMs: the GeGLU forward
// that keeps the Wi pre-activation, the backward of GeGLU, LayerNorm, the
// embedding gather and the scoring head, operand transposes for the
// weight-gradient GEMMs, gradient sums of squares and AdamW.
//
// Reference (internal/nn/backward.go, ops.go; internal/train/optim.go):
//   geglu backward  backward.go:49-61   dwi = [da*gate*gelu'(a) | da*gelu(a)]
//   layerNormBwd    ops.go:94-135        dx += rs*(g*w - mean(g*w) - xh*mean(g*w*xh)), dw += sum g*xh (+ db)
//   embeddings      backward.go:96-109   dTok[id] += LN backward of the emb norm, in token order
//   HeadBackward    backward.go:161-196
//   GradNorm        optim.go:68-90       float64 sums of squares
//   Update          optim.go:94-145      AdamW with decoupled weight decay
// Reductions over rows are two-stage with fixed order (per-block partials,
// then a sum in block order), so results do not depend on scheduling.
#include "common.hpp"

namespace {

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <class T>
__device__ __forceinline__ float ld_elem(const T *p) {
  return (float)*p;
}

// ---------------------------------------------------------------------------
// 64 x 64 tiles through LDS: dstT[c][r] = src[r][c] for r < rows_pad (zero
// for r >= rows), converted to TO; when copy is set also copy[r][c] = src[r][c]
// (r < rows) in TO. Grid (cols/64, rows_pad/64), 256 threads.
template <class TI, class TO>
__global__ __launch_bounds__(256) void transpose_kernel(const TI *src, int rows, int cols, int lds, TO *dstT, int ldt,
                                                        int rows_pad, TO *copy) {
  __shared__ float tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
#pragma unroll 4
  for (int j = 0; j < 16; j++) {
    const int r = r0 + ty + 4 * j, c = c0 + tx;
    float v = 0.0f;
    if (r < rows && c < cols) {
      v = ld_elem(src + (size_t)r * lds + c);
      if (copy) copy[(size_t)r * cols + c] = (TO)v;
    }
    tile[ty + 4 * j][tx] = v;
  }
  __syncthreads();
#pragma unroll 4
  for (int j = 0; j < 16; j++) {
    const int c = c0 + ty + 4 * j, r = r0 + tx;
    if (c < cols && r < rows_pad) dstT[(size_t)c * ldt + r] = (TO)tile[tx][ty + 4 * j];
  }
}

// The same with 8-element vectors (16 bytes of bf16, 32 of fp32) on both
// sides: needs cols, lds and ldt multiples of 8 and rows_pad a multiple of 64.
template <class TI, class TO>
__device__ __forceinline__ void transpose8_tile(float (&tile)[64][65], const TI *src, int rows, int cols, int lds,
                                                TO *dstT, int ldt, int rows_pad, TO *copy, int c0, int r0) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int it = tid + 256 * j, r = it >> 3, cg = (it & 7) * 8;
    float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (r0 + r < rows && c0 + cg < cols) {
      Vec8<TI>::load(src + (size_t)(r0 + r) * lds + c0 + cg, v);
      if (copy) Vec8<TO>::store(copy + (size_t)(r0 + r) * cols + c0 + cg, v);
    }
#pragma unroll
    for (int u = 0; u < 8; u++) tile[r][cg + u] = v[u];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int it = tid + 256 * j, c = it >> 3, rg = (it & 7) * 8;
    if (c0 + c >= cols || r0 + rg >= rows_pad) continue;
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = tile[rg + u][c];
    Vec8<TO>::store(dstT + (size_t)(c0 + c) * ldt + r0 + rg, v);
  }
}

template <class TI, class TO>
__global__ __launch_bounds__(256) void transpose8_kernel(const TI *src, int rows, int cols, int lds, TO *dstT,
                                                         int ldt, int rows_pad, TO *copy) {
  __shared__ float tile[64][65];
  transpose8_tile<TI, TO>(tile, src, rows, cols, lds, dstT, ldt, rows_pad, copy, blockIdx.x * 64, blockIdx.y * 64);
}

// Several transposes in one launch (TransposeBatch): each job owns a run of
// (cols/64) x (rows_pad/64) consecutive blocks; its input is fp32 or bf16.
template <class TO>
__global__ __launch_bounds__(256) void transpose8_batch_kernel(TransposeBatch b) {
  __shared__ float tile[64][65];
  int e = 0;
#pragma unroll
  for (int i = 1; i < TB_MAX; i++)
    if (i < b.n && (int)blockIdx.x >= b.job[i].first_block) e = i;
  const TransposeJob &J = b.job[e];
  const int blk = blockIdx.x - J.first_block, nbx = J.cols / 64;
  const int c0 = (blk % nbx) * 64, r0 = (blk / nbx) * 64;
  if (J.f32_in)
    transpose8_tile<float, TO>(tile, (const float *)J.src, b.rows, J.cols, J.cols, (TO *)J.dst, b.ldt, b.rows_pad,
                               (TO *)nullptr, c0, r0);
  else
    transpose8_tile<bf16, TO>(tile, (const bf16 *)J.src, b.rows, J.cols, J.cols, (TO *)J.dst, b.ldt, b.rows_pad,
                              (TO *)nullptr, c0, r0);
}

// GeGLU on the stored Wi output (rows interleaved in 64-column groups: 32
// value columns, then the 32 matching gate columns): act[t][32g+r] =
// gelu(wi[t][64g+r]) * wi[t][64g+32+r] (forward.go:327-336).
template <class T>
__global__ void geglu_fwd_kernel(const T *wi, T *act, int rows, int I) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)rows * I) return;
  const size_t t = idx / I;
  const int i = (int)(idx % I), g = i >> 5, r = i & 31;
  const T *row = wi + t * 2 * I + 64 * g;
  act[idx] = (T)(gelu_erf<T>(ld_elem(row + r)) * ld_elem(row + 32 + r));
}

// GeGLU backward (backward.go:49-61) in the interleaved layout: each thread
// takes 8 consecutive act columns (16-byte bf16 / 32-byte fp32 accesses).
template <class T>
__global__ void geglu_bwd_kernel(const float *dact, const T *wi, T *dwi, int rows, int I) {
  const size_t idx = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (idx >= (size_t)rows * I) return;
  const size_t t = idx / I;
  const int i = (int)(idx % I), g = i >> 5, r = i & 31;  // r is a multiple of 8
  const T *row = wi + t * 2 * I + 64 * g;
  T *out = dwi + t * 2 * I + 64 * g;
  float a[8], gt[8], da[8], dv[8], dg[8];
  Vec8<T>::load(row + r, a);
  Vec8<T>::load(row + 32 + r, gt);
  Vec8<float>::load(dact + idx, da);
#pragma unroll
  for (int u = 0; u < 8; u++) {
    dv[u] = da[u] * gt[u] * gelu_grad<T>(a[u]);
    dg[u] = da[u] * gelu_erf<T>(a[u]);
  }
  Vec8<T>::store(out + r, dv);
  Vec8<T>::store(out + 32 + r, dg);
}

// ---------------------------------------------------------------------------
// LayerNorm backward (layerNormBwd, ops.go:94-135) for bias-free norms over
// rows of dim = 64*NE: one wave per row, RPW rows per wave with their loads
// issued together; dx = res + ... (res given) or dx += ...; this block's
// partial of dw (sum over its rows of dy*xh) goes to part[block]. mean and
// rstd are the forward's statistics (when null they are recomputed from x
// as the forward computes them, f64). x rows are x[r] or, with ids, the
// embedding row tok[ids[r]].
constexpr int LNB_WAVES = 4, LNB_RPW = 4;
template <int NE>
__global__ __launch_bounds__(256) void ln_bwd_kernel(float *dx, const float *res, const float *dy, const float *x,
                                                     const int *ids, const float *mean, const float *rstd,
                                                     const float *w, float eps, int rows, float *part, bf16 *dx_op) {
  constexpr int dim = 64 * NE;
  __shared__ float sw[LNB_WAVES][dim];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float wv[NE], pw[NE];
#pragma unroll
  for (int j = 0; j < NE; j++) {
    wv[j] = w[lane + 64 * j];
    pw[j] = 0.0f;
  }
  constexpr int RB = LNB_WAVES * LNB_RPW;  // rows per block and pass
  for (int r0 = blockIdx.x * RB + wave * LNB_RPW; r0 < rows; r0 += gridDim.x * RB) {
    float xv[LNB_RPW][NE], gv[LNB_RPW][NE], bv[LNB_RPW][NE], m[LNB_RPW], rs[LNB_RPW];
#pragma unroll
    for (int q = 0; q < LNB_RPW; q++) {
      const int r = min(r0 + q, rows - 1);
      const float *xr = ids ? x + (size_t)ids[r] * dim : x + (size_t)r * dim;
      const float *br = (res ? res : dx) + (size_t)r * dim;  // dx = res + ... or dx += ...
#pragma unroll
      for (int j = 0; j < NE; j++) {
        xv[q][j] = xr[lane + 64 * j];
        gv[q][j] = dy[(size_t)r * dim + lane + 64 * j];
        bv[q][j] = br[lane + 64 * j];
      }
      if (mean) {
        m[q] = mean[r];
        rs[q] = rstd[r];
      }
    }
    if (!mean) {
#pragma unroll
      for (int q = 0; q < LNB_RPW; q++) {
        double s = 0;
#pragma unroll
        for (int j = 0; j < NE; j++) s += (double)xv[q][j];
        const double mu = wave_sum_d(s) / (double)dim;
        double v = 0;
#pragma unroll
        for (int j = 0; j < NE; j++) {
          const double d = (double)xv[q][j] - mu;
          v += d * d;
        }
        rs[q] = (float)(1.0 / sqrt(wave_sum_d(v) / (double)dim + (double)eps));
        m[q] = (float)mu;
      }
    }
#pragma unroll
    for (int q = 0; q < LNB_RPW; q++) {
      const int r = r0 + q;
      double s1 = 0, s2 = 0;
#pragma unroll
      for (int j = 0; j < NE; j++) {
#pragma clang fp contract(off)
        const float xh = (xv[q][j] - m[q]) * rs[q];
        const float gw = gv[q][j] * wv[j];
        s1 += (double)gw;
        s2 += (double)(gw * xh);
        if (r < rows) pw[j] += gv[q][j] * xh;
        xv[q][j] = xh;
      }
      const float a = (float)(wave_sum_d(s1) / (double)dim), b = (float)(wave_sum_d(s2) / (double)dim);
      if (r >= rows) continue;
      float *o = dx + (size_t)r * dim;
#pragma unroll
      for (int j = 0; j < NE; j++) {
#pragma clang fp contract(off)
        const float v = bv[q][j] + rs[q] * (gv[q][j] * wv[j] - a - xv[q][j] * b);
        o[lane + 64 * j] = v;
        if (dx_op) dx_op[(size_t)r * dim + lane + 64 * j] = (bf16)v;  // the next GEMM's bf16 operand
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NE; j++) sw[wave][lane + 64 * j] = pw[j];
  __syncthreads();
  for (int i = threadIdx.x; i < dim; i += 256) {
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < LNB_WAVES; q++) acc += sw[q][i];
    part[(size_t)blockIdx.x * dim + i] = acc;
  }
}

// Column sums of part [nparts x n] in two launches with a fixed order:
// colsum_kernel: block (x, y) sums rows y*per .. y*per+per-1 of columns
// 64x .. 64x+63 (each wave every 4th row, 4 independent loads in flight per
// lane, then the 4 waves in order) into part2[y][col]; colsum_final_kernel
// adds the NG partial rows, in order, into out.
constexpr int COLSUM_NG = 16;
__global__ __launch_bounds__(256) void colsum_kernel(const float *part_a, const float *part_b, int nparts, int n,
                                                     float *part2_a, float *part2_b) {
  const float *part = blockIdx.z ? part_b : part_a;
  float *part2 = blockIdx.z ? part2_b : part2_a;
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int per = (nparts + COLSUM_NG - 1) / COLSUM_NG;
  const int p0 = blockIdx.y * per, p1 = min(nparts, p0 + per);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (c < n) {
    int p = p0 + wave;
    for (; p + 12 < p1; p += 16) {
#pragma unroll
      for (int u = 0; u < 4; u++) acc[u] += part[(size_t)(p + 4 * u) * n + c];
    }
    for (; p < p1; p += 4) acc[0] += part[(size_t)p * n + c];
  }
  red[wave][lane] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (wave == 0 && c < n) part2[(size_t)blockIdx.y * n + c] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

__global__ void colsum_final_kernel(const float *part2_a, const float *part2_b, int n, float *out_a, float *out_b) {
  const float *part2 = blockIdx.y ? part2_b : part2_a;
  float *out = blockIdx.y ? out_b : out_a;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float acc = 0.0f;
#pragma unroll
  for (int y = 0; y < COLSUM_NG; y++) acc += part2[(size_t)y * n + i];
  out[i] += acc;
}

// dst[i] += src[i].
__global__ void add_kernel(float *dst, const float *src, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] += src[i];
}

// Embedding gradient: one block per distinct token id; the rows of dE whose
// token has that id are added to dTok[id] in token order (backward.go:102-108).
__global__ __launch_bounds__(256) void embed_bwd_kernel(const float *dE, const int *order, const int *seg_start,
                                                        const int *seg_id, int dim, float *gtok) {
  const int sgi = blockIdx.x;
  const int b = seg_start[sgi], e = seg_start[sgi + 1];
  float *dst = gtok + (size_t)seg_id[sgi] * dim;
  for (int i = threadIdx.x; i < dim; i += 256) {
    float acc = dst[i];
    for (int k = b; k < e; k++) acc += dE[(size_t)order[k] * dim + i];
    dst[i] = acc;
  }
}

// ---------------------------------------------------------------------------
// HeadBackward (backward.go:161-196), fp32. One 256-thread block per row r:
// recomputes final_norm (fN), the input_norm statistics, gelu and the scorer
// norm from the encoder row and the forward's s1 and d (dense output before
// its bias), then back-propagates dl = dlogits[r]:
//   ds2 = dl*OutW; dge = LNbwd(ds2); dd = dge*gelu'(d+b); ds1 = dd.DenseW;
//   dfN = LNbwd(ds1); dRows = LNbwd(dfN) -> dcur[rowTok[r]].
// Per-row parameter-gradient terms go to contrib (summed over rows by
// head_param_kernel): [dl*s2 | ds2*xh2 | ds2 | dd | ds1*xh1 | ds1 | dfN*xhF].
struct HeadBwdArgs {
  const float *h;         // encoder output [T x H]
  const int *row_tok;     // [R]
  const float *s1, *d;    // forward's input_norm output [R x H] and dense output [R x H/2]
  const float *dlogits;   // [R]
  int R, H;
  float eps;
  const float *final_norm, *in_w, *dense_w, *dense_b, *norm_w, *norm_b, *out_w;
  float *dcur;            // [T x H], zero except the rows written here
  float *contrib;         // [R x (4*half + 3*H)]
};

__device__ __forceinline__ double block_sum(double v, double *red) {
  v = wave_sum_d(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// LN backward of one row held 3 (or 2 for half rows) elements per thread:
// returns dx (no accumulate), with xh the normalized input and w the weight.
template <int E>
__device__ __forceinline__ void row_ln_bwd(const float (&g)[E], const float (&xh)[E], const float (&w)[E],
                                           const bool (&ok)[E], float rs, int dim, double *red, float (&dx)[E]) {
  double s1 = 0, s2 = 0;
#pragma unroll
  for (int j = 0; j < E; j++)
    if (ok[j]) {
#pragma clang fp contract(off)
      const float gw = g[j] * w[j];
      s1 += (double)gw;
      s2 += (double)(gw * xh[j]);
    }
  const float a = (float)(block_sum(s1, red) / (double)dim);
  const float b = (float)(block_sum(s2, red) / (double)dim);
#pragma unroll
  for (int j = 0; j < E; j++) {
#pragma clang fp contract(off)
    dx[j] = ok[j] ? rs * (g[j] * w[j] - a - xh[j] * b) : 0.0f;
  }
}

template <int E>
__device__ __forceinline__ void row_stats_block(const float (&x)[E], const bool (&ok)[E], int dim, float eps,
                                                double *red, float &mean, float &rstd) {
  double s = 0;
#pragma unroll
  for (int j = 0; j < E; j++)
    if (ok[j]) s += (double)x[j];
  const double mu = block_sum(s, red) / (double)dim;
  double v = 0;
#pragma unroll
  for (int j = 0; j < E; j++)
    if (ok[j]) {
      const double d = (double)x[j] - mu;
      v += d * d;
    }
  rstd = (float)(1.0 / sqrt(block_sum(v, red) / (double)dim + (double)eps));
  mean = (float)mu;
}

__global__ __launch_bounds__(256) void head_bwd_row_kernel(HeadBwdArgs a) {
  constexpr int EH = 4;  // H <= 1024
  constexpr int EF = 2;  // half <= 512
  __shared__ double red[4];
  __shared__ float sdd[512];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int H = a.H, half = H / 2;
  const int t = a.row_tok[r];
  const float dl = a.dlogits[r];
  const size_t cw = (size_t)4 * half + 3 * H;
  float *ct = a.contrib + (size_t)r * cw;
  // Half rows: gelu input, scorer norm.
  float dv[EF], ge[EF], nw[EF], xh2[EF], ds2[EF];
  bool okf[EF];
#pragma unroll
  for (int j = 0; j < EF; j++) {
    const int i = tid + 256 * j;
    okf[j] = i < half;
    dv[j] = okf[j] ? a.d[(size_t)r * half + i] + a.dense_b[i] : 0.0f;
    ge[j] = okf[j] ? gelu_erf<float>(dv[j]) : 0.0f;
    nw[j] = okf[j] ? a.norm_w[i] : 0.0f;
  }
  float m2, r2;
  row_stats_block(ge, okf, half, 1e-5f, red, m2, r2);
#pragma unroll
  for (int j = 0; j < EF; j++) {
    const int i = tid + 256 * j;
    float s2;
    {
#pragma clang fp contract(off)
      xh2[j] = (ge[j] - m2) * r2;
      s2 = xh2[j] * nw[j] + (okf[j] ? a.norm_b[i] : 0.0f);  // the forward's s2, unfused (ops.go:83)
    }
    ds2[j] = okf[j] ? dl * a.out_w[i] : 0.0f;
    if (okf[j]) {
      ct[i] = dl * s2;  // OutW: dl * s2
      ct[half + i] = ds2[j] * xh2[j];               // norm weight
      ct[2 * half + i] = ds2[j];                    // norm bias
    }
  }
  float dge[EF];
  row_ln_bwd(ds2, xh2, nw, okf, r2, half, red, dge);
#pragma unroll
  for (int j = 0; j < EF; j++) {
    const int i = tid + 256 * j;
    if (okf[j]) {
      const float v = dge[j] * gelu_grad<float>(dv[j]);
      sdd[i] = v;
      ct[3 * half + i] = v;  // dense bias (and, with s1, the dense weight)
    }
  }
  __syncthreads();
  // Full rows: ds1 = dd . DenseW, input_norm and final_norm backward.
  float x[EH], fn[EH], xhF[EH], xh1[EH], wF[EH], wI[EH], ds1[EH];
  bool ok[EH];
#pragma unroll
  for (int j = 0; j < EH; j++) {
    const int i = tid + 256 * j;
    ok[j] = i < H;
    x[j] = ok[j] ? a.h[(size_t)t * H + i] : 0.0f;
    wF[j] = ok[j] ? a.final_norm[i] : 0.0f;
    wI[j] = ok[j] ? a.in_w[i] : 0.0f;
    float acc = 0.0f;
    if (ok[j])
      for (int k = 0; k < half; k++) acc += sdd[k] * a.dense_w[(size_t)k * H + i];
    ds1[j] = acc;
  }
  float mF, rF;
  row_stats_block(x, ok, H, a.eps, red, mF, rF);
#pragma unroll
  for (int j = 0; j < EH; j++) {
    {
#pragma clang fp contract(off)
      xhF[j] = (x[j] - mF) * rF;
    }
    fn[j] = ok[j] ? xhF[j] * wF[j] : 0.0f;
  }
  float m1, r1;
  row_stats_block(fn, ok, H, 1e-5f, red, m1, r1);
#pragma unroll
  for (int j = 0; j < EH; j++) {
    const int i = tid + 256 * j;
    {
#pragma clang fp contract(off)
      xh1[j] = (fn[j] - m1) * r1;
    }
    if (ok[j]) {
      ct[4 * half + i] = ds1[j] * xh1[j];  // input_norm weight
      ct[4 * half + H + i] = ds1[j];       // input_norm bias
    }
  }
  float dfN[EH], dRow[EH];
  row_ln_bwd(ds1, xh1, wI, ok, r1, H, red, dfN);
  row_ln_bwd(dfN, xhF, wF, ok, rF, H, red, dRow);
  // Rows that share a token: the reference copies dRows into dcur in row
  // order, so the last such row's gradient stands (backward.go:30-33). This
  // block writes dcur only if no later row names the same token.
  bool last = true;
  for (int r2 = r + 1; r2 < a.R; r2++) last = last && a.row_tok[r2] != t;
#pragma unroll
  for (int j = 0; j < EH; j++) {
    const int i = tid + 256 * j;
    if (ok[j]) {
      ct[4 * half + 2 * H + i] = dfN[j] * xhF[j];  // final_norm weight
      if (last) a.dcur[(size_t)t * H + i] = dRow[j];
    }
  }
}

// Head parameter gradients from the per-row terms, summed over rows in row
// order: thread i < half*H is DenseW[i/H][i%H] += sum_r dd[r][i/H]*s1[r][i%H];
// the rest add the column sums of contrib and the out_proj bias.
__global__ void head_param_kernel(HeadBwdArgs a, float *g_outw, float *g_normw, float *g_normb, float *g_denseb,
                                  float *g_densew, float *g_inw, float *g_inb, float *g_final, float *g_outb) {
  const int H = a.H, half = H / 2;
  const size_t cw = (size_t)4 * half + 3 * H;
  const size_t nd = (size_t)half * H;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < nd) {
    const int k = (int)(idx / H), i = (int)(idx % H);
    float acc = 0.0f;
    for (int r = 0; r < a.R; r++) acc += a.contrib[(size_t)r * cw + 3 * half + k] * a.s1[(size_t)r * H + i];
    g_densew[idx] += acc;
    return;
  }
  const size_t c = idx - nd;
  if (c < cw) {
    float acc = 0.0f;
    for (int r = 0; r < a.R; r++) acc += a.contrib[(size_t)r * cw + c];
    float *dst;
    size_t off;
    if (c < (size_t)half) dst = g_outw, off = c;
    else if (c < (size_t)2 * half) dst = g_normw, off = c - half;
    else if (c < (size_t)3 * half) dst = g_normb, off = c - 2 * half;
    else if (c < (size_t)4 * half) dst = g_denseb, off = c - 3 * half;
    else if (c < (size_t)4 * half + H) dst = g_inw, off = c - 4 * half;
    else if (c < (size_t)4 * half + 2 * H) dst = g_inb, off = c - 4 * half - H;
    else dst = g_final, off = c - 4 * half - 2 * H;
    dst[off] += acc;
    return;
  }
  if (c == cw) {
    float acc = 0.0f;
    for (int r = 0; r < a.R; r++) acc += a.dlogits[r];
    g_outb[0] += acc;
  }
}

// ---------------------------------------------------------------------------
// Sum of squares in float64: block partials (fixed grid), then one sum in
// partial order.
// The table entry owning workgroup b: the last one whose first workgroup
// (field FIRST) is <= b (binary search; the table is in ascending order).
template <int MTensor::*FIRST>
__device__ __forceinline__ int mt_find(const MTensor *t, int nt, int b) {
  int lo = 0, hi = nt - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t[mid].*FIRST <= b) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Partial j of a tensor: the f64 sum of g^2 over i = 256*j + thread, strided
// by 256*nparts, threads then waves in a fixed order.
__global__ __launch_bounds__(256) void sumsq_multi_kernel(const MTensor *tab, int nt, double *part) {
  __shared__ double red[4];
  const int ti = mt_find<&MTensor::first_part>(tab, nt, blockIdx.x);
  const MTensor &t = tab[ti];
  const int j = blockIdx.x - t.first_part;
  double s = 0;
  for (size_t i = (size_t)j * 256 + threadIdx.x; i < t.n; i += (size_t)t.nparts * 256) {
    const double v = (double)t.g[i];
    s += v * v;
  }
  s = wave_sum_d(s);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void zero_multi_kernel(const MTensor *tab, int nt) {
  const MTensor &t = tab[mt_find<&MTensor::first_chunk>(tab, nt, blockIdx.x)];
  const size_t k0 = (size_t)(blockIdx.x - t.first_chunk) * MT_CHUNK;
  for (size_t k = k0 + threadIdx.x; k < t.n && k < k0 + MT_CHUNK; k += 256) t.g[k] = 0.0f;
}

// One block of 256 threads: strided per-thread sums, then the 256 sums in a
// fixed tree order.
__global__ __launch_bounds__(256) void sum_doubles_kernel(const double *part, int n, double *out) {
  __shared__ double red[256];
  double s = 0;
  for (int i = threadIdx.x; i < n; i += 256) s += part[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = red[0];
}

// AdamW (Update, optim.go:118-141), written unfused as the reference
// evaluates it. With wq (bf16 projections) the new weight is also stored in
// the operand copy, rounded to nearest even.
__global__ __launch_bounds__(256) void adamw_multi_kernel(const MTensor *tab, int nt, float b1, float b2, float eps,
                                                          float scale, float step_size, float inv_sqrt_b2c) {
  const MTensor &t = tab[mt_find<&MTensor::first_chunk>(tab, nt, blockIdx.x)];
  const size_t k0 = (size_t)(blockIdx.x - t.first_chunk) * MT_CHUNK;
  float *p = t.p, *m = t.m, *v = t.v;
  const float *g = t.g;
  bf16 *wq = t.wq;
  const float lr = t.rate, wd = t.wd;
  for (size_t k = k0 + threadIdx.x; k < t.n && k < k0 + MT_CHUNK; k += 256) {
#pragma clang fp contract(off)
    const float gr = g[k] * scale;
    const float mk = b1 * m[k] + (1 - b1) * gr;
    const float vk = b2 * v[k] + (1 - b2) * gr * gr;
    m[k] = mk;
    v[k] = vk;
    const float den = (float)sqrt((double)vk) * inv_sqrt_b2c + eps;
    const float pk = p[k] - (lr * step_size * mk / den + wd * p[k]);
    p[k] = pk;
    if (wq) wq[k] = (bf16)pk;
  }
}

__global__ void widen_bf16_kernel(const bf16 *src, float *dst, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = (float)src[i];
}

inline unsigned blocks(size_t n, int per = 256) { return (unsigned)((n + per - 1) / per); }

}  // namespace

hipError_t launch_transpose_batch(const TransposeBatch &b0, int precision_out, hipStream_t s) {
  if (b0.n <= 0 || b0.rows_pad <= 0) return hipSuccess;
  if (b0.n > TB_MAX || b0.rows_pad % 64 || b0.ldt % 8) return hipErrorInvalidValue;
  TransposeBatch b = b0;
  int blocks_total = 0;
  for (int i = 0; i < b.n; i++) {
    if (b.job[i].cols <= 0 || b.job[i].cols % 64) return hipErrorInvalidValue;
    if (!b.job[i].f32_in && precision_out != 1) return hipErrorInvalidValue;
    b.job[i].first_block = blocks_total;
    blocks_total += (b.job[i].cols / 64) * (b.rows_pad / 64);
  }
  if (precision_out == 1)
    hipLaunchKernelGGL(transpose8_batch_kernel<bf16>, dim3(blocks_total), dim3(256), 0, s, b);
  else
    hipLaunchKernelGGL(transpose8_batch_kernel<float>, dim3(blocks_total), dim3(256), 0, s, b);
  return hipGetLastError();
}

hipError_t launch_transpose(int precision_in, int precision_out, const void *src, int rows, int cols, int lds,
                            void *dstT, int ldt, int rows_pad, void *copy, hipStream_t s) {
  if (rows_pad <= 0 || cols <= 0) return hipSuccess;
  const dim3 grid((cols + 63) / 64, (rows_pad + 63) / 64), block(256);
  if (cols % 8 == 0 && lds % 8 == 0 && ldt % 8 == 0 && rows_pad % 64 == 0) {
    if (precision_in == 0 && precision_out == 1)
      hipLaunchKernelGGL((transpose8_kernel<float, bf16>), grid, block, 0, s, (const float *)src, rows, cols, lds,
                         (bf16 *)dstT, ldt, rows_pad, (bf16 *)copy);
    else if (precision_in == 0 && precision_out == 0)
      hipLaunchKernelGGL((transpose8_kernel<float, float>), grid, block, 0, s, (const float *)src, rows, cols, lds,
                         (float *)dstT, ldt, rows_pad, (float *)copy);
    else if (precision_in == 1 && precision_out == 1)
      hipLaunchKernelGGL((transpose8_kernel<bf16, bf16>), grid, block, 0, s, (const bf16 *)src, rows, cols, lds,
                         (bf16 *)dstT, ldt, rows_pad, (bf16 *)copy);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (precision_in == 0 && precision_out == 1)
    hipLaunchKernelGGL((transpose_kernel<float, bf16>), grid, block, 0, s, (const float *)src, rows, cols, lds,
                       (bf16 *)dstT, ldt, rows_pad, (bf16 *)copy);
  else if (precision_in == 0 && precision_out == 0)
    hipLaunchKernelGGL((transpose_kernel<float, float>), grid, block, 0, s, (const float *)src, rows, cols, lds,
                       (float *)dstT, ldt, rows_pad, (float *)copy);
  else if (precision_in == 1 && precision_out == 1)
    hipLaunchKernelGGL((transpose_kernel<bf16, bf16>), grid, block, 0, s, (const bf16 *)src, rows, cols, lds,
                       (bf16 *)dstT, ldt, rows_pad, (bf16 *)copy);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_geglu_fwd(int precision, const void *wi, void *act, int rows, int I, hipStream_t s) {
  const size_t n = (size_t)rows * I;
  if (n == 0) return hipSuccess;
  if (precision == 1)
    hipLaunchKernelGGL(geglu_fwd_kernel<bf16>, dim3(blocks(n)), dim3(256), 0, s, (const bf16 *)wi, (bf16 *)act, rows, I);
  else
    hipLaunchKernelGGL(geglu_fwd_kernel<float>, dim3(blocks(n)), dim3(256), 0, s, (const float *)wi, (float *)act, rows,
                       I);
  return hipGetLastError();
}

hipError_t launch_geglu_bwd(int precision, const float *dact, const void *wi, void *dwi, int rows, int I,
                            hipStream_t s) {
  const size_t n = (size_t)rows * I;
  if (n == 0) return hipSuccess;
  if (I % 32 != 0) return hipErrorInvalidValue;
  if (precision == 1)
    hipLaunchKernelGGL(geglu_bwd_kernel<bf16>, dim3(blocks(n / 8)), dim3(256), 0, s, dact, (const bf16 *)wi,
                       (bf16 *)dwi, rows, I);
  else
    hipLaunchKernelGGL(geglu_bwd_kernel<float>, dim3(blocks(n / 8)), dim3(256), 0, s, dact, (const float *)wi,
                       (float *)dwi, rows, I);
  return hipGetLastError();
}

int ln_bwd_blocks(int rows) {
  constexpr int RB = LNB_WAVES * LNB_RPW;
  return std::max(1, std::min(1024, (rows + RB - 1) / RB)) + COLSUM_NG;
}

hipError_t launch_ln_bwd(float *dx, const float *res, const float *dy, const float *x, const int *ids,
                         const float *mean, const float *rstd, const float *w, float eps, int rows, int dim,
                         float *part, float *dw, hipStream_t s, void *dx_bf16) {
  if (rows <= 0) return hipSuccess;
  const int nb = ln_bwd_blocks(rows) - COLSUM_NG;
  switch (dim) {
#define LNB_CASE(NE)                                                                                               \
  case 64 * NE:                                                                                                    \
    hipLaunchKernelGGL(ln_bwd_kernel<NE>, dim3(nb), dim3(256), 0, s, dx, res, dy, x, ids, mean, rstd, w, eps, rows, \
                       part, (bf16 *)dx_bf16);                                                                     \
    break;
    LNB_CASE(4)
    LNB_CASE(6)
    LNB_CASE(8)
    LNB_CASE(12)
    LNB_CASE(16)
#undef LNB_CASE
    default:
      return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !dw) return e;
  return launch_ln_bwd_colsum(part, rows, dim, dw, s);
}

hipError_t launch_ln_bwd_colsum(float *part, int rows, int dim, float *dw, hipStream_t s, float *part_b,
                                float *dw_b) {
  if (rows <= 0) return hipSuccess;
  const int nb = ln_bwd_blocks(rows) - COLSUM_NG;
  const int two = part_b && dw_b ? 2 : 1;
  float *part2 = part + (size_t)nb * dim, *part2_b = two == 2 ? part_b + (size_t)nb * dim : part2;
  hipLaunchKernelGGL(colsum_kernel, dim3((dim + 63) / 64, COLSUM_NG, two), dim3(256), 0, s, part,
                     two == 2 ? part_b : part, nb, dim, part2, part2_b);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(colsum_final_kernel, dim3(blocks(dim), two), dim3(256), 0, s, part2, part2_b, dim, dw,
                     two == 2 ? dw_b : dw);
  return hipGetLastError();
}

hipError_t launch_add(float *dst, const float *src, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(add_kernel, dim3(blocks(n)), dim3(256), 0, s, dst, src, n);
  return hipGetLastError();
}

hipError_t launch_embed_bwd(const float *dE, const int *order, const int *seg_start, const int *seg_id, int nseg,
                            int dim, float *gtok, hipStream_t s) {
  if (nseg <= 0) return hipSuccess;
  hipLaunchKernelGGL(embed_bwd_kernel, dim3(nseg), dim3(256), 0, s, dE, order, seg_start, seg_id, dim, gtok);
  return hipGetLastError();
}

hipError_t launch_head_bwd(const float *h, const int *row_tok, const float *s1, const float *d, const float *dlogits,
                           int R, int H, float eps, const float *const *w, float *dcur, float *contrib,
                           float *const *g, hipStream_t s) {
  if (R <= 0) return hipSuccess;
  if (H > 1024 || H % 256 != 0) return hipErrorInvalidValue;
  // w: final_norm, in_w, dense_w, dense_b, norm_w, norm_b, out_w
  HeadBwdArgs a{h, row_tok, s1, d, dlogits, R, H, eps, w[0], w[1], w[2], w[3], w[4], w[5], w[6], dcur, contrib};
  hipLaunchKernelGGL(head_bwd_row_kernel, dim3(R), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // g: out_w, norm_w, norm_b, dense_b, dense_w, in_w, in_b, final_norm, out_b
  const size_t n = (size_t)(H / 2) * H + (size_t)4 * (H / 2) + 3 * H + 1;
  hipLaunchKernelGGL(head_param_kernel, dim3(blocks(n)), dim3(256), 0, s, a, g[0], g[1], g[2], g[3], g[4], g[5], g[6],
                     g[7], g[8]);
  return hipGetLastError();
}

int sumsq_blocks(size_t n) { return (int)std::max<size_t>(1, std::min<size_t>(256, (n + 4095) / 4096)); }

hipError_t launch_sumsq_multi(const MTensor *t, int nt, int total_parts, double *part, hipStream_t s) {
  if (nt <= 0 || total_parts <= 0) return hipSuccess;
  hipLaunchKernelGGL(sumsq_multi_kernel, dim3(total_parts), dim3(256), 0, s, t, nt, part);
  return hipGetLastError();
}

hipError_t launch_zero_multi(const MTensor *t, int nt, int total_chunks, hipStream_t s) {
  if (nt <= 0 || total_chunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_multi_kernel, dim3(total_chunks), dim3(256), 0, s, t, nt);
  return hipGetLastError();
}

hipError_t launch_sum_doubles(const double *part, int n, double *out, hipStream_t s) {
  hipLaunchKernelGGL(sum_doubles_kernel, dim3(1), dim3(256), 0, s, part, n, out);
  return hipGetLastError();
}

hipError_t launch_adamw_multi(const MTensor *t, int nt, int total_chunks, float b1, float b2, float eps, float scale,
                              float step_size, float inv_sqrt_b2c, hipStream_t s) {
  if (nt <= 0 || total_chunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(adamw_multi_kernel, dim3(total_chunks), dim3(256), 0, s, t, nt, b1, b2, eps, scale, step_size,
                     inv_sqrt_b2c);
  return hipGetLastError();
}

hipError_t launch_widen_bf16(const void *src, float *dst, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(widen_bf16_kernel, dim3(blocks(n)), dim3(256), 0, s, (const bf16 *)src, dst, n);
  return hipGetLastError();
}
