// Projection GEMMs: C[M x N] = A[M x K] . B[N x K]^T on MFMA (fp32 accumulate).
//
// Replaces the reference's linearFwd -> blas.Sgemm(false, true, ...)
// (internal/nn/forward.go:122-124, internal/blas/gemm.go:61-138) for the four
// per-layer projections, with the elementwise work that follows each of them
// fused into the epilogue:
//   EPI_QKV   : RoPE on the q/k columns (internal/nn/ops.go:155-175), store qkv
//   EPI_F32   : store fp32, optionally C += (the residual adds, forward.go:318-322, 338-342)
//   EPI_GEGLU : act = gelu(value) * gate (forward.go:327-336); the Wi rows are
//               interleaved at upload so each 64-column group holds 32 value
//               rows followed by the 32 matching gate rows
//
// Both operands are K-contiguous (token-major activations, (out,in) weights),
// so each lane's MFMA operand is one contiguous LDS read. Tiles of BM x BN x
// (128 bytes of K) are staged through LDS, double buffered, with 16 bytes of
// padding per 128-byte row so the 32 rows read by one MFMA operand land in
// distinct bank groups.
#include "common.hpp"

namespace {

constexpr int ROWB = 144;  // bytes per LDS tile row: 128 of K + 16 padding

template <class T, int BM, int BN, int WAVES_M, int WAVES_N, int EPI>
__global__ __launch_bounds__(WAVES_M *WAVES_N * 64) void gemm_nt_kernel(GemmArgs g) {
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int KT = 128 / sizeof(T);  // K elements per stage
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_CH = BM * 8 / NT, B_CH = BN * 8 / NT;  // 16-byte chunks per thread
  static_assert(A_CH * NT == BM * 8 && B_CH * NT == BN * 8, "tile/thread mismatch");
  static_assert(EPI == EPI_F32 || TN % 2 == 0, "paired epilogues need 64-column wave tiles");

  __shared__ __attribute__((aligned(16))) char smem[2][(BM + BN) * ROWB];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int lr = lane & 31, lh = lane >> 5;

  // XCD-aware tile order: consecutive workgroups go round-robin over the 8
  // XCDs; give each XCD a contiguous range of tiles (N fastest) so an A row
  // panel is reused out of that XCD's L2.
  const int tiles_n = g.N / BN;
  const int ntiles = gridDim.x;
  int bid = blockIdx.x;
  int tile = (ntiles % 8 == 0) ? (bid % 8) * (ntiles / 8) + bid / 8 : bid;
  const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;

  const char *Ab = (const char *)g.A;
  const char *Bb = (const char *)g.B;
  const size_t lda_b = (size_t)g.lda * sizeof(T), ldb_b = (size_t)g.ldb * sizeof(T);

  // Global -> register staging of one K stage (16-byte chunks; 8 threads per
  // 128-byte row), then register -> LDS. Rows past M re-read row M-1 (their
  // results are never stored).
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 ra[A_CH], rb[B_CH];
  const char *a_src[A_CH];
  const char *b_src[B_CH];
  int a_dst[A_CH], b_dst[B_CH];
#pragma unroll
  for (int i = 0; i < A_CH; i++) {
    const int c = tid + i * NT, r = c >> 3, cc = c & 7;
    a_src[i] = Ab + (size_t)min(m0 + r, g.M - 1) * lda_b + cc * 16;
    a_dst[i] = r * ROWB + cc * 16;
  }
#pragma unroll
  for (int i = 0; i < B_CH; i++) {
    const int c = tid + i * NT, r = c >> 3, cc = c & 7;
    b_src[i] = Bb + (size_t)(n0 + r) * ldb_b + cc * 16;
    b_dst[i] = (BM + r) * ROWB + cc * 16;
  }
#define GEMM_GLOAD(k0)                                                                       \
  do {                                                                                       \
    const size_t kb_ = (size_t)(k0) * sizeof(T);                                             \
    _Pragma("unroll") for (int i = 0; i < A_CH; i++) ra[i] = *(const u32x4 *)(a_src[i] + kb_); \
    _Pragma("unroll") for (int i = 0; i < B_CH; i++) rb[i] = *(const u32x4 *)(b_src[i] + kb_); \
  } while (0)
#define GEMM_SSTORE(buf)                                                                        \
  do {                                                                                          \
    _Pragma("unroll") for (int i = 0; i < A_CH; i++) *(u32x4 *)(smem[buf] + a_dst[i]) = ra[i]; \
    _Pragma("unroll") for (int i = 0; i < B_CH; i++) *(u32x4 *)(smem[buf] + b_dst[i]) = rb[i]; \
  } while (0)

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  const int nk = g.K / KT;
  GEMM_GLOAD(0);
  GEMM_SSTORE(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) GEMM_GLOAD((kt + 1) * KT);
    const char *sa = smem[buf] + (wm * WM + lr) * ROWB;
    const char *sb = smem[buf] + (BM + wn * WN + lr) * ROWB;
#pragma unroll
    for (int ks = 0; ks < KT / MF::KSTEP; ks++) {
      const int kof = (ks * MF::KSTEP + lh * MF::SLOTS) * (int)sizeof(T);
      frag a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) a[i] = *(const frag *)(sa + i * 32 * ROWB + kof);
#pragma unroll
      for (int j = 0; j < TN; j++) b[j] = *(const frag *)(sb + j * 32 * ROWB + kof);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = MF::mma(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < nk) GEMM_SSTORE(buf ^ 1);
    __syncthreads();
  }

#undef GEMM_GLOAD
#undef GEMM_SSTORE

  // Epilogue.
  const int row_base = m0 + wm * WM;
  const int col_base = n0 + wn * WN;
  if constexpr (EPI == EPI_F32) {
    float *C = (float *)g.C;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int col = col_base + j * 32 + lr;
        if (col >= g.n_store) continue;
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int row = row_base + i * 32 + mfma_row(e, lane);
          if (row < g.M) {
            float *p = C + (size_t)row * g.ldc + col;
            *p = g.accumulate ? *p + acc[i][j][e] : acc[i][j][e];
          }
        }
      }
  } else if constexpr (EPI == EPI_QKV) {
    T *C = (T *)g.C;
#pragma unroll
    for (int jp = 0; jp < TN / 2; jp++) {
      const int c0 = col_base + jp * 64;  // start of one 64-wide head slice
      const bool rot = c0 < g.rope_cols;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int row = row_base + i * 32 + mfma_row(e, lane);
          float a = acc[i][2 * jp][e], b = acc[i][2 * jp + 1][e];
          if (rot) {
            const int tr = min(row, g.M - 1);
            const float c = g.cos_t[(size_t)tr * 32 + lr], s = g.sin_t[(size_t)tr * 32 + lr];
            const float a2 = a * c - b * s;
            const float b2 = b * c + a * s;
            a = a2;
            b = b2;
          }
          if (row < g.M) {
            T *p = C + (size_t)row * g.ldc + c0 + lr;
            p[0] = to_elem<T>(a);
            p[32] = to_elem<T>(b);
          }
        }
    }
  } else {  // EPI_GEGLU
    T *C = (T *)g.C;
#pragma unroll
    for (int jp = 0; jp < TN / 2; jp++) {
      const int oc = (col_base + jp * 64) / 2 + lr;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int row = row_base + i * 32 + mfma_row(e, lane);
          const float v = acc[i][2 * jp][e], gt = acc[i][2 * jp + 1][e];
          if (row < g.M) C[(size_t)row * g.ldc + oc] = to_elem<T>(gelu_erf<T>(v) * gt);
        }
    }
  }
}

template <class T, int BM, int BN, int WM_, int WN_>
hipError_t launch_cfg(int epi, const GemmArgs &a, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
  dim3 grid(tiles), block(WM_ * WN_ * 64);
  switch (epi) {
    case EPI_F32:
      hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, WM_, WN_, EPI_F32>), grid, block, 0, s, a);
      break;
    case EPI_QKV:
      hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, WM_, WN_, EPI_QKV>), grid, block, 0, s, a);
      break;
    default:
      hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, WM_, WN_, EPI_GEGLU>), grid, block, 0, s, a);
      break;
  }
  return hipGetLastError();
}

}  // namespace

// All tile configs use BN = 128 and stage 128 bytes of K per step.
bool gemm_shape_ok(int precision, int N, int K) {
  const int kt = precision == 1 ? 64 : 32;
  return N > 0 && K > 0 && N % 128 == 0 && K % kt == 0;
}

hipError_t launch_gemm(int precision, int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  const bool small = a.M <= 1024;
  if (precision == 1) {
    if (small) return launch_cfg<bf16, 64, 128, 1, 2>(epi, a, s);
    return launch_cfg<bf16, 256, 128, 2, 2>(epi, a, s);
  }
  if (small) return launch_cfg<float, 64, 128, 1, 2>(epi, a, s);
  return launch_cfg<float, 256, 128, 2, 2>(epi, a, s);
}
