// Shared device-side definitions for the gfx950 encoder kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

// Records msg as the error of calls made without a context (dn_last_error(NULL))
// and returns code.
int set_host_error(int code, const std::string &msg);

typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(bf16))));
typedef bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(bf16))));
typedef bf16 bf16x2_t __attribute__((__vector_size__(2 * sizeof(bf16))));
// IEEE binary16: the operand type of the fp16 mode (11-bit significand where
// bf16 has 8, the same MFMA rate and bytes).
typedef _Float16 f16;
typedef f16 f16x8 __attribute__((__vector_size__(8 * sizeof(f16))));
typedef f16 f16x2_t __attribute__((__vector_size__(2 * sizeof(f16))));

// Precision codes of the launchers: 0 fp32, 1 bf16, 2 fp16 (operand type of
// the GEMM / attention operands and the activations stored between kernels).
enum { PREC_F32 = 0, PREC_BF16 = 1, PREC_F16 = 2 };
inline bool prec16(int precision) { return precision != PREC_F32; }
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

// Per-element-type MFMA shape. Both element types use the 32x32 output
// layout (16 fp32 accumulators per lane): lane l owns output column l%32 and
// rows 8*(i/4) + 4*(l/32) + i%4 for accumulator i. Operand layout: lane l
// feeds row (A) / column (B) l%32 with SLOTS consecutive k values starting at
// (l/32)*SLOTS inside each KSTEP-wide k step.
template <class T>
struct Mfma;

template <>
struct Mfma<bf16> {
  static constexpr int KSTEP = 16;  // v_mfma_f32_32x32x16_bf16
  static constexpr int SLOTS = 8;
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<f16> {
  static constexpr int KSTEP = 16;  // v_mfma_f32_32x32x16_f16
  static constexpr int SLOTS = 8;
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// The 16 x 16 x 32 form of the 16-bit MFMAs (4 accumulators per lane: lane l
// owns column l%16 and rows 4*(l/16) .. +3; operand lane l feeds row l%16
// with 8 consecutive k values from 8*(l/16)).
template <class T>
__device__ __forceinline__ f32x4 mma16x16(typename Mfma<T>::frag a, typename Mfma<T>::frag b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mma16x16<bf16>(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mma16x16<f16>(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <>
struct Mfma<float> {
  static constexpr int KSTEP = 2;  // v_mfma_f32_32x32x2_f32
  static constexpr int SLOTS = 1;
  typedef float frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// Row (M) index inside a 32x32 MFMA output tile of accumulator i on this lane.
__device__ __forceinline__ int mfma_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

template <class T>
__device__ __forceinline__ T to_elem(float x);
template <>
__device__ __forceinline__ float to_elem<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 to_elem<bf16>(float x) { return (bf16)x; }
template <>
__device__ __forceinline__ f16 to_elem<f16>(float x) { return (f16)x; }

// Two 16-bit elements in one 32-bit word (element 0 in bits 0..15): widen
// one of them, or round a pair to nearest even and pack it.
template <class T>
__device__ __forceinline__ float lo16(uint32_t w);
template <class T>
__device__ __forceinline__ float hi16(uint32_t w);
template <class T>
__device__ __forceinline__ uint32_t pack16(float lo, float hi);
template <>
__device__ __forceinline__ float lo16<bf16>(uint32_t w) { return __uint_as_float(w << 16); }
template <>
__device__ __forceinline__ float hi16<bf16>(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
template <>
__device__ __forceinline__ uint32_t pack16<bf16>(float lo, float hi) {
  bf16x2_t v = {(bf16)lo, (bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ __forceinline__ float lo16<f16>(uint32_t w) { return (float)__builtin_bit_cast(f16, (uint16_t)w); }
template <>
__device__ __forceinline__ float hi16<f16>(uint32_t w) { return (float)__builtin_bit_cast(f16, (uint16_t)(w >> 16)); }
template <>
__device__ __forceinline__ uint32_t pack16<f16>(float lo, float hi) {
  f16x2_t v = {(f16)lo, (f16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// GELU, exact erf form: 0.5*x*(1 + erf(x/sqrt2)) (internal/nn/ops.go:140-142).
// The fp32 validation build evaluates erf in double as the reference does.
template <class T>
__device__ __forceinline__ float gelu_erf(float x);
template <>
__device__ __forceinline__ float gelu_erf<float>(float x) {
  return 0.5f * x * (1.0f + (float)erf((double)x * 1.41421356237309504880 / 2.0));
}
// erf(x) for the bf16 path, whose result is rounded to bf16 (2^-9 relative)
// anyway: the rational approximation 7.1.26 of Abramowitz & Stegun,
// |error| <= 1.5e-7, evaluated with one exp2 and one hardware reciprocal
// (v_rcp_f32, 1 ulp: a correctly rounded one compiles to the ten-instruction
// IEEE division sequence, for an error far below the formula's own).
__device__ __forceinline__ float erf_as(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * ax);
  const float p = t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  const float y = 1.0f - p * exp2f(-ax * ax * 1.44269504088896341f);
  return copysignf(y, x);
}
template <>
__device__ __forceinline__ float gelu_erf<bf16>(float x) {
  return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752440f));
}
// fp16 results are rounded to 2^-11 relative: the same approximation.
template <>
__device__ __forceinline__ float gelu_erf<f16>(float x) {
  return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752440f));
}

// d gelu(x)/dx = Phi(x) + x phi(x) (geluGrad, ops.go:145-150): float64 in the
// fp32 build; the bf16 build uses the same erf approximation as its forward.
template <class T>
__device__ __forceinline__ float gelu_grad(float x);
template <>
__device__ __forceinline__ float gelu_grad<float>(float x) {
  const double xf = (double)x;
  const double cdf = 0.5 * (1 + erf(xf * 1.41421356237309504880 / 2));
  const double pdf = exp(-0.5 * xf * xf) / sqrt(2 * 3.14159265358979323846);
  return (float)(cdf + xf * pdf);
}
template <>
__device__ __forceinline__ float gelu_grad<bf16>(float x) {
  const float cdf = 0.5f * (1.0f + erf_as(x * 0.70710678118654752440f));
  const float pdf = exp2f(-0.5f * x * x * 1.44269504088896341f) * 0.39894228040143267794f;
  return cdf + x * pdf;
}

// Eight consecutive elements as floats: 16 bytes of bf16 or 32 of fp32.
template <class T>
struct Vec8;
template <>
struct Vec8<bf16> {
  static __device__ __forceinline__ void load(const bf16 *p, float (&v)[8]) {
    const uint4 u = *(const uint4 *)p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void store(bf16 *p, const float (&v)[8]) {
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = (bf16)v[i];
    *(bf16x8 *)p = o;
  }
};
template <>
struct Vec8<f16> {
  static __device__ __forceinline__ void load(const f16 *p, float (&v)[8]) {
    const uint4 u = *(const uint4 *)p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = lo16<f16>(w[i]);
      v[2 * i + 1] = hi16<f16>(w[i]);
    }
  }
  static __device__ __forceinline__ void store(f16 *p, const float (&v)[8]) {
    *(uint4 *)p = make_uint4(pack16<f16>(v[0], v[1]), pack16<f16>(v[2], v[3]), pack16<f16>(v[4], v[5]),
                             pack16<f16>(v[6], v[7]));
  }
};
template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float *p, float (&v)[8]) {
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float *p, const float (&v)[8]) {
    *(float4 *)p = make_float4(v[0], v[1], v[2], v[3]);
    *(float4 *)(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};

// Summary of up to 32 consecutive tokens of one sequence, used by the
// attention kernel to skip (or fast-path) whole key tiles.
struct ChunkInfo {
  int pmin, pmax;  // position range
  int omin, omax;  // option-id range over option tokens (omin > omax if none)
  int nprefix;     // tokens with opt == -1
  int nopt;        // tokens with opt >= 0
  int len;         // valid tokens in the chunk
  int pad;
};

// Host-side launchers (implemented in the .hip files, called by api.cpp).
struct GemmArgs {
  const void *A;  // M x K, row stride lda (elements)
  const void *B;  // N x K, row stride ldb (weights, PyTorch (out,in) layout)
  void *C;        // output
  int M, N, K, lda, ldb, ldc;
  int n_store;    // columns actually stored (fp32 epilogue)
  int accumulate; // fp32 epilogue: C += result
  int ngroups;    // N-tile groups per XCD sweep (set by launch_gemm)
  int order;      // workgroup -> tile order (0: XCD-aware groups)
  size_t c_split; // split-K: elements between the partial outputs of blockIdx.y (0: one split)
  const float *res; // EPI_F32 with accumulate: C = res + result (res has C's layout); null: C += result
  void *C2;         // EPI_GEGLU_KEEP: the GeGLU output (ldc2), C receives the plain product
  int ldc2;
  const void *gin;  // EPI_GEGLU_BWD: the GeGLU input (the Wi output, M x 2N, row stride ldc)
  int skinny_regs;  // small-M kernel, 16-bit 32 x 32 tiles: operands loaded straight into registers
                    // (0: whole 128-byte rows through LDS by global->LDS DMA)
};

// LayerNorm folded into the GEMMs on either side of it (16-bit inference),
// the EPI_*_LN forms' second kernel argument (GemmArgs stays at its size:
// larger kernel arguments cost every launch ~0.6 us, which the small-batch
// forwards' ~160 launches feel). The residual GEMM (EPI_F32_LN) also writes
// fx = (x - mprev[row]) * lw[col] in the operand type, of the new residual x (row stride
// ldc) and, per row and 192-column N-tile, the tile's (mean, M2) of x to
// lpart (lparts float pairs per row). The GEMM that takes fx as A (EPI_STORE_LN,
// EPI_GEGLU_LN) merges them into the row's mean and rstd = 1/sqrt(M2/K +
// eps) and computes rstd * (A.B^T - (mean - mprev[row]) * lcs[col]) with
// lcs[n] = sum_k lw[k] B[n][k], i.e. LayerNorm(x).B^T with the LayerNorm
// weight in lcs and in fx; its tiles at n0 = 0 write the row mean to
// mean_out. mprev null: 0.
struct LnFold {
  void *fx;
  const float *lw, *lcs, *mprev;
  float *lpart;
  float *mean_out;
  int lparts;
  float eps;
};

// GEMM epilogues: fp32 store / accumulate, store in the operand type, GeGLU of
// value/gate column pairs, and (training) both the plain product and its
// GeGLU, or the GeGLU backward: the product is the gradient of the GeGLU
// output (M x N), and C (M x 2N, operand type, the interleaved Wi layout)
// receives the gradients of its value and gate inputs, read from gin.
enum { EPI_F32 = 0, EPI_STORE = 1, EPI_GEGLU = 2, EPI_GEGLU_KEEP = 3, EPI_GEGLU_BWD = 4 };
// The folded-LayerNorm forms (LnFold; bf16 or fp16, M > 1024): the
// residual GEMM that produces the LayerNorm's input, and the store / GeGLU
// GEMMs that consume its output.
enum { EPI_F32_LN = 5, EPI_STORE_LN = 6, EPI_GEGLU_LN = 7 };
// Columns per LayerNorm statistics part written by EPI_F32_LN.
constexpr int kLnPartCols = 192;
// Whether the folded LayerNorm runs for a 16-bit model of this geometry at M
// rows (the configurations launch_gemm tiles for EPI_*_LN).
bool gemm_ln_fold_ok(int precision, int M, int hidden, int inter);

hipError_t launch_gemm(int precision, int epi, const GemmArgs &a, hipStream_t s, const LnFold *ln = nullptr);
// Any-shape GEMM for model geometries the MFMA kernels do not tile: one thread
// per output element, an fp32 dot product over K in order. EPI_F32,
// EPI_STORE and EPI_GEGLU, the last over the natural Wi layout (value rows
// [0, N/2), gate rows [N/2, N); output N/2 columns).
hipError_t launch_gemm_generic(int precision, int epi, const GemmArgs &a, hipStream_t s);
// Whether launch_gemm takes this epilogue at M rows (EPI_GEGLU_BWD needs the
// tiled kernel: M > 128 in bf16, M > 1024 in fp32).
bool gemm_epi_ok(int precision, int epi, int M);
// Split-K fp32-output GEMM: `splits` (1..16) partial products, each over a.K / splits
// of K (a.K % (splits * 64) == 0), written to partial + split * M * N
// (row-major, ldc = N), then summed in split order into C (M x N, ldc = N;
// added to C when a.accumulate, else stored). partial holds splits * M * N floats.
hipError_t launch_gemm_splitk(int precision, const GemmArgs &a, int splits, float *partial, hipStream_t s);
// Small M (<= 128) split-K on the whole-K kernel, no reduction: workgroup z of
// a tile multiplies K elements [z*K/splits, (z+1)*K/splits) and stores its
// fp32 partial product at partial + z * M * N (row-major, ldc = N); a.C,
// a.res and a.accumulate are ignored. The consumer sums the splits
// (launch_ln's partial inputs). a.K % (splits * 64) == 0 (bf16) / 32 (fp32).
hipError_t launch_gemm_small_split(int precision, const GemmArgs &a, int splits, float *partial, hipStream_t s);
bool gemm_shape_ok(int precision, int N, int K);

// Attention work item: 32 * QT * ATTN_WAVES queries of one sequence (each
// wave owns QT tiles of 32 queries), for every head. QT = 1 (128 queries, 3
// waves per SIMD) everywhere except the global layers of the two-stream
// forward of a large batch, which take QT = 2 (256 queries, 2 waves per SIMD:
// alone it is no faster, cfg3 125 -> 123 us and cfg4 317 -> 360 us per global
// layer, but beside the other stream's kernels the whole forward gains, cfg3
// +1%, cfg4 +2%). Local layers with QT = 2: 86 -> 104 us.
constexpr int ATTN_WAVES = 4;
constexpr int ATTN_QT = 1;
constexpr int ATTN_QUERIES = 32 * ATTN_QT * ATTN_WAVES;
constexpr int ATTN_QT_GLOBAL = 2;
constexpr int ATTN_QUERIES_GLOBAL = 32 * ATTN_QT_GLOBAL * ATTN_WAVES;
// Key tiles (64 keys) per sequence: sequences up to 8192 tokens.
constexpr int ATTN_MAXKT = 128;

struct AttnArgs {
  const void *qkv;
  void *ctx;
  const int *kinfo;   // per token: ((opt+1) << 16) | pos
  const float *cos_t, *sin_t;  // RoPE tables [65536 x 32] of this layer's theta, row = position
  const int4 *work;   // (seq, q0, seq offset, seq length) per workgroup
  const uint32_t *codes;  // [nwork][ATTN_MAXKT] tile classes of this layer type (tile_codes_kernel)
  const int *first;       // [nwork] first tile with an allowed pair
  const int *seq_off, *seq_len;
  int nwork, H, heads, sliding, half_window;
  float scale_log2;   // softmax scale * log2(e)
  float *lse;         // training: per (token, head) log2 of the softmax denominator of the
                      // scaled scores, lse[t*heads + head] = max*scale_log2 + log2(sum); null otherwise
  int qt;                       // query tiles per wave of the work items (ATTN_QT or ATTN_QT_GLOBAL)
  int nseq, max_len, head_dim;  // the any-geometry kernel: sequences, longest one, head width,
  float scale;                  // and the softmax scale float32(1 / sqrt(head_dim))
  // Option-row attention (launch_attention_rows): work items and slots from
  // launch_row_items (nwork: an upper bound on the items, nseq + ceil(R /
  // ATTN_QUERIES)); Q of row r at q_rows + r * H (rotated by the kernel);
  // ctx row r receives row r's output.
  const int4 *items;
  const int *nitems, *rows, *row_tok;
  const void *q_rows;
};
hipError_t launch_attention(int precision, const AttnArgs &a, hipStream_t s);
// Attention of the option rows only (the last layer past which only they are
// used): the queries are rows r of row_tok grouped into a.items.
hipError_t launch_attention_rows(int precision, const AttnArgs &a, hipStream_t s);
// items / rows / nitems for launch_attention_rows from row_tok[R] and the
// batch's seq_off (nseq + 1 entries); nseq <= ROW_ITEMS_MAXSEQ. items needs
// nseq + ceil(R / ATTN_QUERIES) entries, rows R.
constexpr int ROW_ITEMS_MAXSEQ = 1024;
hipError_t launch_row_items(const int *row_tok, int R, const int *seq_off, int nseq, int T, int4 *items, int *rows,
                            int *nitems, hipStream_t s);
// Attention for model geometries the MFMA kernel does not take (head width 8,
// 16 or 32; the reference's own small test models): one thread per query,
// the reference's two-pass masked softmax (attnFwd + softmaxMasked,
// forward.go:347-409, ops.go), fp32 arithmetic. Same inputs and output.
hipError_t launch_attention_generic(int precision, const AttnArgs &a, hipStream_t s);

// Attention backward (the reference's attnBwd + the RoPE inverse,
// backward.go:117-159 and :77-81): dqkv from dctx, the un-rotated qkv, ctx and
// the forward's lse. The batch layout fields are the forward's.
struct AttnBwdArgs {
  const void *qkv;     // [T x 3H] un-rotated, operand type
  const void *ctx;     // [T x H] forward output O, operand type
  const void *dctx;    // [T x H] dO, operand type
  const float *lse;    // [T x heads] from the forward
  float *dsum;         // [T x heads] scratch: D = rowsum(dO * O)
  void *dqkv;          // [T x 3H] out (dq, dk after the RoPE inverse; dv), operand type
  const int *kinfo;
  const float *cos_t, *sin_t;
  const int4 *work;
  const uint32_t *codes;
  const int *first;
  const int *seq_off, *seq_len;
  const ChunkInfo *chunks;
  const int *chunk_off;
  int nwork, H, heads, sliding, half_window;
  float scale;         // 1/sqrt(64)
  float scale_log2;    // scale * log2(e)
};
hipError_t launch_attention_bwd(int precision, const AttnBwdArgs &a, hipStream_t s);

// Tile classes of work items of 32 * nc queries (nc = ATTN_WAVES * QT);
// sliding 0: global layers, 1: sliding-window layers, -1: both in one launch
// (the sliding-window codes and first tiles one section of nwork items after
// the global ones).
hipError_t launch_tile_codes(const ChunkInfo *chunks, const int4 *work, const int *seq_len, const int *chunk_off,
                             int nwork, int sliding, int half_window, uint32_t *codes, int *first, hipStream_t s,
                             int nc = ATTN_WAVES * ATTN_QT);
hipError_t launch_rope_tables(const int *pos, int T, const double *inv_g, const double *inv_l, float *cos_g,
                              float *sin_g, float *cos_l, float *sin_l, hipStream_t s);
// The forward's prologue in one launch: per token kinfo = ((opt+1) << 16) |
// pos (a position outside [0, 65535] or an option id outside [-1, 32766]
// sets bit 4 of err: the packed form and the per-position RoPE tables cover
// that range only); per 32-token chunk (chunk_desc = (first token, length),
// the chunks covering every token) its ChunkInfo summary; and the embedding
// gather (an id outside [0, vocab) sets bit 1 of err and reads row 0) + emb
// norm into h (fp32) and xn (operand type), with the row statistics in
// mean / rstd when given (training).
hipError_t launch_prologue(int precision, const int *pos, const int *opt, const int4 *chunk_desc, int nchunks,
                           int *kinfo, ChunkInfo *chunks, const int *ids, int Tn, const float *tok, int vocab,
                           const float *w, float eps, int H, float *h, void *xn, int *err, hipStream_t s,
                           float *mean = nullptr, float *rstd = nullptr);
// Column sums of a LayerNorm-weighted bf16 or fp16 projection for the folded
// LayerNorm: cs[n] = sum_k lw[k] * B[n][k] (fp64 sums), B N x K.
hipError_t launch_fold_colsum(int precision, const void *B, int N, int K, const float *lw, float *cs,
                              hipStream_t s);
// LayerNorm launchers; mean / rstd (optional, [rows]) receive the row statistics.
hipError_t launch_ln(int precision, const float *x, int rows, int H, const float *w, float eps, void *y, hipStream_t s,
                     float *mean = nullptr, float *rstd = nullptr);
// LayerNorm of x + (p0 + p1 + ... + p{nparts-1}) (the split-K partial
// products of the residual GEMM before it, summed left to right, then added
// to x), the sum stored back into x first: the residual update
// C = res + A.B^T and the norm that reads it in one launch. part holds
// nparts slices of rows x H floats; nparts 4 or 6.
hipError_t launch_ln_parts(int precision, float *x, const float *part, int nparts, int rows, int H, const float *w,
                           float eps, void *y, hipStream_t s);
struct HeadArgs {
  const float *h;
  const int *row_tok;  // the rows of h the head reads; null: rows 0 .. R-1
  int R, T, H;
  float eps;
  const float *final_norm, *in_w, *in_b, *dense_w, *dense_b, *norm_w, *norm_b, *out_w, *out_b;
  float *logits;
  int *err_flag;
};
// generic: the dense layer's GEMM on the any-shape kernel (geometries the
// MFMA GEMMs do not tile).
hipError_t launch_head(const HeadArgs &a, float *s1, float *d, hipStream_t s, bool generic = false);
hipError_t launch_pack(const float *src, int trans, int rows, int cols, int ld, float *dst, int dst_rows,
                       int dst_cols, hipStream_t s);
// ctx_r[r] = ctx[row_tok[r]] (operand type), h_r[r] = h[row_tok[r]] (fp32), H
// columns, r < R; an index outside [0, T) sets bit 2 of *err_flag.
hipError_t launch_gather_rows(int precision, const void *ctx, const float *h, const int *row_tok, int R, int T,
                              int H, void *ctx_r, float *h_r, int *err_flag, hipStream_t s);

// Training kernels (backward.hip). Precision codes: 0 fp32, 1 bf16.
hipError_t launch_transpose(int precision_in, int precision_out, const void *src, int rows, int cols, int lds,
                            void *dstT, int ldt, int rows_pad, void *copy, hipStream_t s);
// Up to TB_MAX transposes dst[cols x ldt] = src[rows x cols]^T (zero for rows
// .. rows_pad) in one launch; each src is fp32 or (bf16 output only) bf16,
// cols a multiple of 64, rows_pad of 64. first_block is set by the launcher.
constexpr int TB_MAX = 4;
struct TransposeJob {
  const void *src;
  void *dst;
  int cols, f32_in, first_block;
};
struct TransposeBatch {
  TransposeJob job[TB_MAX];
  int n, rows, rows_pad, ldt;
};
hipError_t launch_transpose_batch(const TransposeBatch &b, int precision_out, hipStream_t s);
hipError_t launch_geglu_fwd(int precision, const void *wi, void *act, int rows, int I, hipStream_t s);
hipError_t launch_geglu_bwd(int precision, const float *dact, const void *wi, void *dwi, int rows, int I,
                            hipStream_t s);
// LayerNorm backward: dx = res + LNbwd(dy) when res is given, else dx += LNbwd(dy);
// dw += the weight gradient (part holds ln_bwd_blocks(rows) x dim floats of scratch).
// mean / rstd: the forward's row statistics (recomputed from x when null);
// dx_bf16 (optional) receives dx rounded to bf16 (the next GEMM's operand).
int ln_bwd_blocks(int rows);
hipError_t launch_ln_bwd(float *dx, const float *res, const float *dy, const float *x, const int *ids,
                         const float *mean, const float *rstd, const float *w, float eps, int rows, int dim,
                         float *part, float *dw, hipStream_t s, void *dx_bf16 = nullptr);
// The weight-gradient half alone (launch_ln_bwd with dw null leaves it out):
// dw += the column sums of the per-block partials in part, in a fixed order.
// With part_b and dw_b, a second norm's partials and gradient in the same launches.
hipError_t launch_ln_bwd_colsum(float *part, int rows, int dim, float *dw, hipStream_t s, float *part_b = nullptr,
                                float *dw_b = nullptr);
hipError_t launch_add(float *dst, const float *src, size_t n, hipStream_t s);
hipError_t launch_embed_bwd(const float *dE, const int *order, const int *seg_start, const int *seg_id, int nseg,
                            int dim, float *gtok, hipStream_t s);
// w: final_norm, in_w, dense_w, dense_b, norm_w, norm_b, out_w;
// g: out_w, norm_w, norm_b, dense_b, dense_w, in_w, in_b, final_norm, out_b.
// contrib holds R x (2H + 3H) floats.
hipError_t launch_head_bwd(const float *h, const int *row_tok, const float *s1, const float *d, const float *dlogits,
                           int R, int H, float eps, const float *const *w, float *dcur, float *contrib,
                           float *const *g, hipStream_t s);
// Optimizer work over many tensors in one launch: a device table of the
// tensors, each owning a run of consecutive workgroups.
struct MTensor {
  float *p;        // fp32 parameters (the master copy of a bf16 projection)
  float *g, *m, *v;
  bf16 *wq;        // bf16 operand copy to refresh, or null
  size_t n;
  float rate, wd;  // learning rate; decoupled weight decay (times the rate), 0 if none
  int first_chunk; // first workgroup of the elementwise kernels (MT_CHUNK elements each)
  int first_part;  // first workgroup / partial of the sum of squares
  int nparts;      // sumsq_blocks(n)
};
constexpr int MT_CHUNK = 4096;
int sumsq_blocks(size_t n);
inline int mt_chunks(size_t n) { return (int)((n + MT_CHUNK - 1) / MT_CHUNK); }
// part[first_part + j] = the j-th of nparts strided partial sums of g^2 (f64), per tensor.
hipError_t launch_sumsq_multi(const MTensor *t, int nt, int total_parts, double *part, hipStream_t s);
hipError_t launch_sum_doubles(const double *part, int n, double *out, hipStream_t s);
// g = 0 over every tensor of the table.
hipError_t launch_zero_multi(const MTensor *t, int nt, int total_chunks, hipStream_t s);
// AdamW (optim.go:118-141) over every tensor of the table.
hipError_t launch_adamw_multi(const MTensor *t, int nt, int total_chunks, float b1, float b2, float eps, float scale,
                              float step_size, float inv_sqrt_b2c, hipStream_t s);
hipError_t launch_widen_bf16(const void *src, float *dst, size_t n, hipStream_t s);
// Register-only bf16 MFMA loop (calibrate.hip): mode 0 operands rotated every
// iteration, mode 1 constant; mfma_calibrate_flop gives the work of a launch.
hipError_t launch_mfma_calibrate(int mode, int blocks, int iters, float *sink, hipStream_t s);
double mfma_calibrate_flop(int mode, int blocks, int iters);
