// Row-wise kernels: embedding gather + LayerNorm, LayerNorm, RoPE tables,
// the scoring head, and the operand packer used by the general GEMM entry.
//
// All are HBM-bound; rows are handled one wavefront per row with 128-bit
// loads, and LayerNorm statistics are reduced in double as the reference's
// layerNormFwd does (internal/nn/ops.go:63-92): mean = sum/dim, two-pass
// variance, rs = f32(1/sqrt(var + eps)), y = ((x - f32(mean)) * rs) * w (+ b).
#include "common.hpp"

namespace {

// Butterfly sums over the 64 lanes, v + v[lane ^ o] for o = 32, 16, ..., 1,
// without LDS round trips: the lane-32 and lane-16 exchanges are
// v_permlane32_swap / v_permlane16_swap (swapping a copy of v with itself
// leaves v[l] in one result and v[l ^ o] in the other, so their sum is the
// exchange sum), the others DPP moves: row_ror:8 is lane ^ 8 within a row of
// 16; row_ror:4 reads lane (l +- 4) mod 16, which after the three steps
// above holds the same value as lane l ^ 4 (each lane's value depends on
// l % 8 only); quad_perm [2,3,0,1] and [1,0,3,2] are lane ^ 2 and lane ^ 1.
// Floating-point addition is commutative, so every lane ends with the same
// bits as the shuffle butterfly v += __shfl_xor(v, o).
template <int CTRL>
__device__ __forceinline__ unsigned dpp_u32(unsigned x) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long u = __double_as_longlong(v);
  const unsigned lo = dpp_u32<CTRL>((unsigned)u), hi = dpp_u32<CTRL>((unsigned)(u >> 32));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double wave_sum(double v) {
  {
    const unsigned long long u = __double_as_longlong(v);
    const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)u, (unsigned)u, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)(u >> 32), (unsigned)(u >> 32), false, false);
    v = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0])) +
        __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
  }
  {
    const unsigned long long u = __double_as_longlong(v);
    const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)u, (unsigned)u, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)(u >> 32), (unsigned)(u >> 32), false, false);
    v = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0])) +
        __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
  }
  v += dpp_f64<0x128>(v);  // row_ror:8
  v += dpp_f64<0x124>(v);  // row_ror:4
  v += dpp_f64<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f64<0xB1>(v);   // quad_perm [1,0,3,2]
  return v;
}
__device__ __forceinline__ float wave_sumf(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

constexpr int MAXV = 4;  // float4 vectors per lane: rows up to 64*4*4 = 1024 wide

// One row of `dim` floats (dim % 4 == 0, dim <= 1024) held as float4 in
// registers; returns mean and rstd with the reference's f64 statistics.
__device__ __forceinline__ void row_stats(const float4 (&x)[MAXV], int nvec, int lane, int dim, float eps,
                                          float &mean, float &rstd) {
  double s = 0;
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) s += (double)x[j].x + (double)x[j].y + (double)x[j].z + (double)x[j].w;
  const double mu = wave_sum(s) / (double)dim;
  double v = 0;
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) {
      const double a = (double)x[j].x - mu, b = (double)x[j].y - mu, c = (double)x[j].z - mu,
                   d = (double)x[j].w - mu;
      v += a * a + b * b + c * c + d * d;
    }
  const double var = wave_sum(v) / (double)dim;
  rstd = (float)(1.0 / sqrt(var + (double)eps));
  mean = (float)mu;
}

template <class T>
__device__ __forceinline__ void store4(T *p, float4 v);
template <>
__device__ __forceinline__ void store4<float>(float *p, float4 v) {
  *(float4 *)p = v;
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16 *p, float4 v) {
  *(uint2 *)p = make_uint2(pack16<bf16>(v.x, v.y), pack16<bf16>(v.z, v.w));
}
template <>
__device__ __forceinline__ void store4<f16>(f16 *p, float4 v) {
  *(uint2 *)p = make_uint2(pack16<f16>(v.x, v.y), pack16<f16>(v.z, v.w));
}

// Token info and 32-token chunk summaries in one launch: 32 lanes per chunk
// (desc = (first token, length)), lane i packing token i's info
// (((opt+1) << 16) | pos; a position outside [0, 65535] or an option id
// outside [-1, 32766] sets bit 4 of the error flag, the packed form and the
// per-position RoPE tables covering that range only) and the chunk's summary
// reduced over the lanes (integer min / max / counts, exact in any order).
// Chunk c = (256-thread block b) * 8 + threadIdx.x / 32.
__device__ __forceinline__ void token_chunk(int b, const int *pos, const int *opt, const int4 *desc, int nchunks,
                                            int *kinfo, ChunkInfo *out, int *err_flag) {
  const int c = (b * 256 + (int)threadIdx.x) >> 5, i = threadIdx.x & 31;
  if (c >= nchunks) return;  // whole 32-lane groups leave together
  const int4 d = desc[c];
  int pmin = 0x7fffffff, pmax = -0x7fffffff, omin = 0x7fffffff, omax = -1, npre = 0, nopt = 0;
  if (i < d.y) {
    const int t = d.x + i;
    const int o = opt ? opt[t] : -1, p = pos[t];
    if (p < 0 || p > 65535 || o < -1 || o > 32766) atomicOr(err_flag, 4);
    const int v = ((o + 1) << 16) | (p & 0xffff);
    kinfo[t] = v;
    const int ov = (v >> 16) - 1, pv = v & 0xffff;
    pmin = pv;
    pmax = pv;
    if (ov < 0) {
      npre = 1;
    } else {
      nopt = 1;
      omin = ov;
      omax = ov;
    }
  }
#pragma unroll
  for (int m = 16; m > 0; m >>= 1) {
    pmin = min(pmin, __shfl_xor(pmin, m, 32));
    pmax = max(pmax, __shfl_xor(pmax, m, 32));
    omin = min(omin, __shfl_xor(omin, m, 32));
    omax = max(omax, __shfl_xor(omax, m, 32));
    npre += __shfl_xor(npre, m, 32);
    nopt += __shfl_xor(nopt, m, 32);
  }
  if (i == 0) out[c] = ChunkInfo{pmin, pmax, omin, omax, npre, nopt, d.y, 0};
}

// Embedding gather (forward.go:204-209) + emb norm (forward.go:220). Writes the
// fp32 residual stream h and its GEMM-operand copy xn (layer 0 has no
// attn_norm, so its QKV input is h itself).
// Rows 4b .. 4b+3 (256-thread block b), one wave per row.
template <class T>
__device__ __forceinline__ void embed_ln(int b, const int *ids, int Tn, const float *tok, int vocab, const float *w,
                                         float eps, int dim, float *h, T *xn, int *err, float *mean_out,
                                         float *rstd_out) {
  const int lane = threadIdx.x & 63;
  const int t = b * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  int id = ids[t];
  if (id < 0 || id >= vocab) {
    if (lane == 0) atomicOr(err, 1);
    id = 0;
  }
  const int nvec = dim / 4;
  const float4 *src = (const float4 *)(tok + (size_t)id * dim);
  float4 x[MAXV], wv[MAXV];
  const float4 *w4 = (const float4 *)w;
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) x[j] = src[lane + 64 * j];
#pragma unroll
  for (int j = 0; j < MAXV; j++)  // the weights with the row, not after its statistics
    if (lane + 64 * j < nvec) wv[j] = w4[lane + 64 * j];
  float mean, rs;
  row_stats(x, nvec, lane, dim, eps, mean, rs);
  if (mean_out && lane == 0) {  // training keeps the statistics (forward.go:220, layerNormFwd's mean/rstd)
    mean_out[t] = mean;
    rstd_out[t] = rs;
  }
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) {
      const float4 ww = wv[j];
      float4 y;
      y.x = (x[j].x - mean) * rs * ww.x;
      y.y = (x[j].y - mean) * rs * ww.y;
      y.z = (x[j].z - mean) * rs * ww.z;
      y.w = (x[j].w - mean) * rs * ww.w;
      ((float4 *)(h + (size_t)t * dim))[lane + 64 * j] = y;
      store4<T>(xn + (size_t)t * dim + 4 * (lane + 64 * j), y);
    }
}

// The forward's prologue in one launch: blocks [0, nb_tc) pack the token info
// and summarise the 32-token chunks, the rest gather the embeddings and
// apply the embedding norm (independent work, one launch boundary fewer).
template <class T>
__global__ __launch_bounds__(256) void prologue_kernel(const int *pos, const int *opt, const int4 *desc, int nchunks,
                                                       int *kinfo, ChunkInfo *chunks, int nb_tc, const int *ids,
                                                       int Tn, const float *tok, int vocab, const float *w,
                                                       float eps, int dim, float *h, T *xn, int *err,
                                                       float *mean_out, float *rstd_out) {
  const int b = blockIdx.x;
  if (b < nb_tc)
    token_chunk(b, pos, opt, desc, nchunks, kinfo, chunks, err);
  else
    embed_ln<T>(b - nb_tc, ids, Tn, tok, vocab, w, eps, dim, h, xn, err, mean_out, rstd_out);
}


// Bias-free LayerNorm of the fp32 residual stream into the GEMM operand type
// (attn_norm forward.go:289-294, mlp_norm forward.go:324).
// RPW rows per wave (their loads and reductions interleave). NPART > 0: the
// row is xin + (p0 + p1 + ... ) over the NPART split-K partial products at
// part + k * pstride (the residual GEMM's C = res + A.B^T), stored to xout
// before it is normalised.
// WPB waves per workgroup.
template <class T, int RPW, int NPART = 0, int WPB = 4>
__global__ __launch_bounds__(64 * WPB) void ln_kernel(const float *xin, int rows, int dim, const float *w, float eps,
                                                      T *y, float *mean_out, float *rstd_out,
                                                      const float *part = nullptr, size_t pstride = 0,
                                                      float *xout = nullptr) {
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * WPB + (threadIdx.x >> 6)) * RPW;
  const int nvec = dim / 4;
  float4 x[RPW][MAXV];
#pragma unroll
  for (int rr = 0; rr < RPW; rr++) {
    const float4 *src = (const float4 *)(xin + (size_t)min(r0 + rr, rows - 1) * dim);
#pragma unroll
    for (int j = 0; j < MAXV; j++)
      if (lane + 64 * j < nvec) x[rr][j] = src[lane + 64 * j];
  }
  // The weights are loaded with the row (and before the partial
  // products), not after its statistics.
  const float4 *w4 = (const float4 *)w;
  float4 wv[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) wv[j] = w4[lane + 64 * j];
  if constexpr (NPART > 0) {
    float4 p[RPW][NPART][MAXV];
#pragma unroll
    for (int rr = 0; rr < RPW; rr++)
#pragma unroll
      for (int k = 0; k < NPART; k++) {
        const float4 *src = (const float4 *)(part + k * pstride + (size_t)min(r0 + rr, rows - 1) * dim);
#pragma unroll
        for (int j = 0; j < MAXV; j++)
          if (lane + 64 * j < nvec) p[rr][k][j] = src[lane + 64 * j];
      }
#pragma unroll
    for (int rr = 0; rr < RPW; rr++)
#pragma unroll
      for (int j = 0; j < MAXV; j++)
        if (lane + 64 * j < nvec) {
          float4 a = p[rr][0][j];
#pragma unroll
          for (int k = 1; k < NPART; k++)
            a = make_float4(a.x + p[rr][k][j].x, a.y + p[rr][k][j].y, a.z + p[rr][k][j].z, a.w + p[rr][k][j].w);
          x[rr][j] = make_float4(x[rr][j].x + a.x, x[rr][j].y + a.y, x[rr][j].z + a.z, x[rr][j].w + a.w);
        }
    // Stored after every sum: a store between them makes the next sum wait
    // for it (the wait counter counts stores too).
#pragma unroll
    for (int rr = 0; rr < RPW; rr++)
#pragma unroll
      for (int j = 0; j < MAXV; j++)
        if (lane + 64 * j < nvec && r0 + rr < rows)
          *(float4 *)(xout + (size_t)(r0 + rr) * dim + 4 * (lane + 64 * j)) = x[rr][j];
  }
#pragma unroll
  for (int rr = 0; rr < RPW; rr++) {
    const int r = r0 + rr;
    float mean, rs;
    row_stats(x[rr], nvec, lane, dim, eps, mean, rs);
    if (r >= rows) continue;
    if (mean_out && lane == 0) {
      mean_out[r] = mean;
      rstd_out[r] = rs;
    }
#pragma unroll
    for (int j = 0; j < MAXV; j++)
      if (lane + 64 * j < nvec) {
        const float4 ww = wv[j];
        float4 o;
        o.x = (x[rr][j].x - mean) * rs * ww.x;
        o.y = (x[rr][j].y - mean) * rs * ww.y;
        o.z = (x[rr][j].z - mean) * rs * ww.z;
        o.w = (x[rr][j].w - mean) * rs * ww.w;
        store4<T>(y + (size_t)r * dim + 4 * (lane + 64 * j), o);
      }
  }
}

// ropeTables (internal/nn/model.go:242-258): angle = f32(pos * inv_freq[i])
// widened back to f64, then f32(cos), f32(sin). One thread per (row, i); row
// t is token t's position, or position t itself when pos is null (the
// per-position tables the QKV epilogue indexes).
__global__ void rope_tables_kernel(const int *pos, int Tn, const double *inv_g, const double *inv_l, float *cg,
                                   float *sg, float *cl, float *sl) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= Tn * 32) return;
  const int t = idx >> 5, i = idx & 31;
  const double p = (double)(pos ? pos[t] : t);
  const double fg = (double)(float)(p * inv_g[i]);
  const double fl = (double)(float)(p * inv_l[i]);
  cg[idx] = (float)cos(fg);
  sg[idx] = (float)sin(fg);
  cl[idx] = (float)cos(fl);
  sl[idx] = (float)sin(fl);
}

// Scoring head (HeadForward, forward.go:250-282), in three launches:
//   head_pre  : gather the [MASK] rows of the encoder output, final_norm, then
//               input_norm (+bias, eps 1e-5) -> s1 [R x H]            (one wave per row)
//   GEMM      : d = s1 . dense^T [R x H/2] on fp32 MFMA (the reference's linearFwd)
//   head_post : +bias, gelu, norm (+bias, eps 1e-5), dot with out_proj, +bias
//                                                                     (one wave per row)
__global__ __launch_bounds__(256) void head_pre_kernel(HeadArgs a, float *s1) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.R) return;
  const int dim = a.H, nvec = dim / 4;
  int t = a.row_tok ? a.row_tok[r] : r;
  if (t < 0 || t >= a.T) {
    if (lane == 0) atomicOr(a.err_flag, 2);
    t = 0;
  }
  const float4 *src = (const float4 *)(a.h + (size_t)t * dim);
  float4 x[MAXV], fwv[MAXV], iwv[MAXV], ibv[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) x[j] = src[lane + 64 * j];
  // Both norms' weights with the row, not after its statistics.
  const float4 *fw = (const float4 *)a.final_norm, *iw = (const float4 *)a.in_w, *ib = (const float4 *)a.in_b;
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) {
      fwv[j] = fw[lane + 64 * j];
      iwv[j] = iw[lane + 64 * j];
      ibv[j] = ib[lane + 64 * j];
    }
  float mean, rs;
  row_stats(x, nvec, lane, dim, a.eps, mean, rs);
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) {
      const float4 ww = fwv[j];
      x[j].x = (x[j].x - mean) * rs * ww.x;
      x[j].y = (x[j].y - mean) * rs * ww.y;
      x[j].z = (x[j].z - mean) * rs * ww.z;
      x[j].w = (x[j].w - mean) * rs * ww.w;
    }
  row_stats(x, nvec, lane, dim, 1e-5f, mean, rs);
#pragma unroll
  for (int j = 0; j < MAXV; j++)
    if (lane + 64 * j < nvec) {
      const float4 ww = iwv[j], bb = ibv[j];
      float4 y;
      y.x = (x[j].x - mean) * rs * ww.x + bb.x;
      y.y = (x[j].y - mean) * rs * ww.y + bb.y;
      y.z = (x[j].z - mean) * rs * ww.z + bb.z;
      y.w = (x[j].w - mean) * rs * ww.w + bb.w;
      ((float4 *)(s1 + (size_t)r * dim))[lane + 64 * j] = y;
    }
}

__global__ __launch_bounds__(256) void head_post_kernel(HeadArgs a, const float *d) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.R) return;
  const int half = a.H / 2;
  constexpr int MAXE = 8;  // half <= 512
  float g[MAXE], nw[MAXE], nb[MAXE], ow[MAXE];
#pragma unroll
  for (int j = 0; j < MAXE; j++) {  // the norm and output weights with the row, not after its statistics
    const int i = lane + 64 * j;
    if (i < half) {
      g[j] = d[(size_t)r * half + i] + a.dense_b[i];
      nw[j] = a.norm_w[i];
      nb[j] = a.norm_b[i];
      ow[j] = a.out_w[i];
    }
  }
  double s = 0;
#pragma unroll
  for (int j = 0; j < MAXE; j++) {
    const int i = lane + 64 * j;
    if (i < half) {
      g[j] = gelu_erf<float>(g[j]);
      s += (double)g[j];
    } else {
      g[j] = 0.0f;
    }
  }
  const double mu = wave_sum(s) / (double)half;
  double v = 0;
#pragma unroll
  for (int j = 0; j < MAXE; j++)
    if (lane + 64 * j < half) {
      const double dd = (double)g[j] - mu;
      v += dd * dd;
    }
  const double var = wave_sum(v) / (double)half;
  const float rs = (float)(1.0 / sqrt(var + 1e-5));
  const float m = (float)mu;
  float dot = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXE; j++) {
    const int i = lane + 64 * j;
    if (i < half) dot += ((g[j] - m) * rs * nw[j] + nb[j]) * ow[j];
  }
  dot = wave_sumf(dot);
  if (lane == 0) a.logits[r] = dot + a.out_b[0];
}

// Rows row_tok[r] of the attention output ctx (operand type) and of the
// residual stream h (fp32) copied to row r of ctx_r / h_r: the inputs of the
// last layer's row-wise tail when only the head's rows are carried past
// attention. One wave per row; a row index outside [0, T) raises error flag 2
// (as head_pre does) and copies row 0.
template <class T>
__global__ __launch_bounds__(256) void gather_rows_kernel(const T *ctx, const float *h, const int *row_tok, int R,
                                                          int Tn, int H, T *ctx_r, float *h_r, int *err_flag) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  int t = row_tok[r];
  if (t < 0 || t >= Tn) {
    if (lane == 0) atomicOr(err_flag, 2);
    t = 0;
  }
  const float4 *hs = (const float4 *)(h + (size_t)t * H);
  float4 *hd = (float4 *)(h_r + (size_t)r * H);
  for (int j = lane; j < H / 4; j += 64) hd[j] = hs[j];
  // 16-byte chunks of the operand row (H * sizeof(T) is a multiple of 16)
  const uint4 *cs = (const uint4 *)(ctx + (size_t)t * H);
  uint4 *cd = (uint4 *)(ctx_r + (size_t)r * H);
  for (int j = lane; j < (int)(H * sizeof(T) / 16); j += 64) cd[j] = cs[j];
}

// dst[dst_rows x dst_cols] (row-major, zero padded) = op(src) where op(src)
// is rows x cols; src is row-major with leading dimension ld, stored
// transposed (cols x rows) when trans is set.
__global__ void pack_kernel(const float *src, int trans, int rows, int cols, int ld, float *dst, int dst_rows,
                            int dst_cols) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)dst_rows * dst_cols) return;
  const int r = idx / dst_cols, c = idx % dst_cols;
  float v = 0.0f;
  if (r < rows && c < cols) v = trans ? src[(size_t)c * ld + r] : src[(size_t)r * ld + c];
  dst[idx] = v;
}

}  // namespace


hipError_t launch_prologue(int precision, const int *pos, const int *opt, const int4 *chunk_desc, int nchunks,
                           int *kinfo, ChunkInfo *chunks, const int *ids, int Tn, const float *tok, int vocab,
                           const float *w, float eps, int H, float *h, void *xn, int *err, hipStream_t s,
                           float *mean, float *rstd) {
  if (Tn <= 0) return hipSuccess;
  const int nb_tc = (nchunks + 7) / 8, nb_emb = (Tn + 3) / 4;
  dim3 grid(nb_tc + nb_emb), block(256);
  if (precision == PREC_BF16)
    hipLaunchKernelGGL(prologue_kernel<bf16>, grid, block, 0, s, pos, opt, chunk_desc, nchunks, kinfo, chunks, nb_tc,
                       ids, Tn, tok, vocab, w, eps, H, h, (bf16 *)xn, err, mean, rstd);
  else if (precision == PREC_F16)
    hipLaunchKernelGGL(prologue_kernel<f16>, grid, block, 0, s, pos, opt, chunk_desc, nchunks, kinfo, chunks, nb_tc,
                       ids, Tn, tok, vocab, w, eps, H, h, (f16 *)xn, err, mean, rstd);
  else
    hipLaunchKernelGGL(prologue_kernel<float>, grid, block, 0, s, pos, opt, chunk_desc, nchunks, kinfo, chunks,
                       nb_tc, ids, Tn, tok, vocab, w, eps, H, h, (float *)xn, err, mean, rstd);
  return hipGetLastError();
}

// cs[n] = sum_k lw[k] * B[n][k] (B bf16 or fp16, N x K), summed in fp64 and rounded
// to float: the column sums of the LayerNorm-weighted projection that a
// folded LayerNorm's consumer GEMM subtracts. One wave per row n.
template <class T>
__global__ __launch_bounds__(256) void fold_colsum_kernel(const T *B, int N, int K, const float *lw, float *cs) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (n >= N) return;
  const T *b = B + (size_t)n * K;
  double acc = 0;
  for (int k = lane; k < K; k += 64) acc += (double)lw[k] * (double)(float)b[k];
  acc = wave_sum(acc);
  if (lane == 0) cs[n] = (float)acc;
}

hipError_t launch_fold_colsum(int precision, const void *B, int N, int K, const float *lw, float *cs,
                              hipStream_t s) {
  if (N <= 0) return hipSuccess;
  if (precision == PREC_BF16)
    hipLaunchKernelGGL(fold_colsum_kernel<bf16>, dim3((N + 3) / 4), dim3(256), 0, s, (const bf16 *)B, N, K, lw, cs);
  else if (precision == PREC_F16)
    hipLaunchKernelGGL(fold_colsum_kernel<f16>, dim3((N + 3) / 4), dim3(256), 0, s, (const f16 *)B, N, K, lw, cs);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_ln(int precision, const float *x, int rows, int H, const float *w, float eps, void *y,
                     hipStream_t s, float *mean, float *rstd) {
  if (rows <= 0) return hipSuccess;
  constexpr int RPW = 1;
  dim3 grid((rows + 4 * RPW - 1) / (4 * RPW)), block(256);
  if (precision == PREC_BF16)
    hipLaunchKernelGGL((ln_kernel<bf16, RPW>), grid, block, 0, s, x, rows, H, w, eps, (bf16 *)y, mean, rstd);
  else if (precision == PREC_F16)
    hipLaunchKernelGGL((ln_kernel<f16, RPW>), grid, block, 0, s, x, rows, H, w, eps, (f16 *)y, mean, rstd);
  else
    hipLaunchKernelGGL((ln_kernel<float, RPW>), grid, block, 0, s, x, rows, H, w, eps, (float *)y, mean, rstd);
  return hipGetLastError();
}

hipError_t launch_ln_parts(int precision, float *x, const float *part, int nparts, int rows, int H, const float *w,
                           float eps, void *y, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  // One row per workgroup: a CU streams a burst of loads at only ~50 GB/s,
  // so the row's (1 + nparts) x H floats are spread over as many CUs as rows.
  dim3 grid(rows), block(64);
  const size_t ps = (size_t)rows * H;
#define LN_PARTS(N)                                                                                               \
  if (nparts == N) {                                                                                              \
    if (precision == PREC_BF16)                                                                                   \
      hipLaunchKernelGGL((ln_kernel<bf16, 1, N, 1>), grid, block, 0, s, x, rows, H, w, eps, (bf16 *)y, nullptr,   \
                         nullptr, part, ps, x);                                                                   \
    else if (precision == PREC_F16)                                                                               \
      hipLaunchKernelGGL((ln_kernel<f16, 1, N, 1>), grid, block, 0, s, x, rows, H, w, eps, (f16 *)y, nullptr,     \
                         nullptr, part, ps, x);                                                                   \
    else                                                                                                          \
      hipLaunchKernelGGL((ln_kernel<float, 1, N, 1>), grid, block, 0, s, x, rows, H, w, eps, (float *)y, nullptr, \
                         nullptr, part, ps, x);                                                                   \
    return hipGetLastError();                                                                                     \
  }
  LN_PARTS(2)
  LN_PARTS(3)
  LN_PARTS(4)
  LN_PARTS(6)
#undef LN_PARTS
  return hipErrorInvalidValue;
}

hipError_t launch_rope_tables(const int *pos, int Tn, const double *inv_g, const double *inv_l, float *cos_g,
                              float *sin_g, float *cos_l, float *sin_l, hipStream_t s) {
  if (Tn <= 0) return hipSuccess;
  const int n = Tn * 32;
  hipLaunchKernelGGL(rope_tables_kernel, dim3((n + 255) / 256), dim3(256), 0, s, pos, Tn, inv_g, inv_l, cos_g, sin_g,
                     cos_l, sin_l);
  return hipGetLastError();
}

hipError_t launch_head(const HeadArgs &a, float *s1, float *d, hipStream_t s, bool generic) {
  if (a.R <= 0) return hipSuccess;
  if (a.H > 1024 || a.H % 8 != 0) return hipErrorInvalidValue;
  const dim3 grid((a.R + 3) / 4), block(256);
  hipLaunchKernelGGL(head_pre_kernel, grid, block, 0, s, a, s1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  GemmArgs g{};
  g.A = s1;
  g.lda = a.H;
  g.B = a.dense_w;
  g.ldb = a.H;
  g.C = d;
  g.ldc = a.H / 2;
  g.M = a.R;
  g.N = a.H / 2;
  g.K = a.H;
  g.n_store = a.H / 2;
  e = generic ? launch_gemm_generic(0, EPI_F32, g, s) : launch_gemm(0, EPI_F32, g, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(head_post_kernel, grid, block, 0, s, a, d);
  return hipGetLastError();
}

hipError_t launch_gather_rows(int precision, const void *ctx, const float *h, const int *row_tok, int R, int T,
                              int H, void *ctx_r, float *h_r, int *err_flag, hipStream_t s) {
  if (R <= 0) return hipSuccess;
  if (H % 8 != 0) return hipErrorInvalidValue;
  const dim3 grid((R + 3) / 4), block(256);
  if (precision == PREC_BF16)
    hipLaunchKernelGGL(gather_rows_kernel<bf16>, grid, block, 0, s, (const bf16 *)ctx, h, row_tok, R, T, H,
                       (bf16 *)ctx_r, h_r, err_flag);
  else if (precision == PREC_F16)
    hipLaunchKernelGGL(gather_rows_kernel<f16>, grid, block, 0, s, (const f16 *)ctx, h, row_tok, R, T, H,
                       (f16 *)ctx_r, h_r, err_flag);
  else
    hipLaunchKernelGGL(gather_rows_kernel<float>, grid, block, 0, s, (const float *)ctx, h, row_tok, R, T, H,
                       (float *)ctx_r, h_r, err_flag);
  return hipGetLastError();
}

hipError_t launch_pack(const float *src, int trans, int rows, int cols, int ld, float *dst, int dst_rows,
                       int dst_cols, hipStream_t s) {
  const size_t n = (size_t)dst_rows * dst_cols;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, trans, rows, cols, ld,
                     dst, dst_rows, dst_cols);
  return hipGetLastError();
}
