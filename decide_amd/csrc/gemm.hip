// Projection GEMMs: C[M x N] = A[M x K] . B[N x K]^T on MFMA (fp32 accumulate).
//
// Replaces the reference's linearFwd -> blas.Sgemm(false, true, ...)
// (internal/nn/forward.go:122-124, internal/blas/gemm.go:61-138) for the four
// per-layer projections, with the elementwise work that follows each of them
// fused into the epilogue:
//   EPI_STORE : store in the operand type (qkv; RoPE is applied by the
//               attention kernel as it loads q and k)
//   EPI_F32   : store fp32, optionally C += (the residual adds, forward.go:318-322, 338-342)
//   EPI_GEGLU : act = gelu(value) * gate (forward.go:327-336); the Wi rows are
//               interleaved at upload so each 64-column group holds 32 value
//               rows followed by the 32 matching gate rows
//
// Design (gfx950):
//   * Both operands are K-contiguous (token-major activations, (out,in)
//     weights): every MFMA operand is one contiguous 16-byte LDS read.
//   * K is staged 128 bytes at a time through an NSTAGE-deep ring of LDS
//     buffers filled by direct global->LDS loads (global_load_lds_dwordx4), so
//     NSTAGE-1 stages are in flight while one is consumed and no registers are
//     spent on staging. Each wave-wide load writes 1 KB = 8 tile rows.
//   * LDS rows are 128 bytes with the 16-byte chunks XOR-swizzled by
//     (row >> 1) & 7, so the 16 rows read by a quarter-wave fall in distinct
//     banks (the swizzle is applied on the global side of the DMA).
//   * Workgroup -> tile order is XCD-aware: consecutive workgroup ids go
//     round-robin over the 8 XCDs; each XCD owns a contiguous range of M
//     panels and sweeps the N tiles in groups small enough that the group's
//     slice of B stays in that XCD's 4 MB L2 while its A panels stream.
//   * The epilogue stages the finished tile through LDS so global stores are
//     full 16-byte-per-lane rows.
#include <type_traits>

#include "common.hpp"

namespace {


// XOR swizzle of the 16-byte chunks of an LDS tile row: with RB-byte rows,
// the 16 rows read by a quarter-wave at one logical chunk land in 16
// distinct 4-bank groups.
template <int RB>
__device__ __forceinline__ int swz(int row) {
  return RB == 128 ? (row >> 1) & 7 : (row >> 2) & 3;
}

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gbl_void;

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Eight 16-byte LDS reads and the wait for them (s_waitcnt lgkmcnt(0)) in
// one statement, so the outputs hold the data when the statement ends (an
// asm output counts as written at the end of its statement; were the wait a
// separate statement, a register copy the compiler placed in between would
// read a value not yet landed). The compiler does not see these as reads of
// memory that global->LDS DMA writes, so it adds no vmcnt wait of its own:
// the caller waits for the DMA explicitly.
__device__ __forceinline__ void lds_read8x16(const char *const (&p)[8], uint4 (&o)[8]) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  uint32_t a[8];
#pragma unroll
  for (int i = 0; i < 8; i++) a[i] = (uint32_t)(size_t)(const __attribute__((address_space(3))) char *)p[i];
  i32x4 v0, v1, v2, v3, v4, v5, v6, v7;
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %9\n\t"
      "ds_read_b128 %2, %10\n\t"
      "ds_read_b128 %3, %11\n\t"
      "ds_read_b128 %4, %12\n\t"
      "ds_read_b128 %5, %13\n\t"
      "ds_read_b128 %6, %14\n\t"
      "ds_read_b128 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(v4), "=&v"(v5), "=&v"(v6), "=&v"(v7)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7])
      : "memory");
  o[0] = __builtin_bit_cast(uint4, v0), o[1] = __builtin_bit_cast(uint4, v1);
  o[2] = __builtin_bit_cast(uint4, v2), o[3] = __builtin_bit_cast(uint4, v3);
  o[4] = __builtin_bit_cast(uint4, v4), o[5] = __builtin_bit_cast(uint4, v5);
  o[6] = __builtin_bit_cast(uint4, v6), o[7] = __builtin_bit_cast(uint4, v7);
}

template <int BM, int BN>
struct TileOrder {
  int m0, n0;
  __device__ __forceinline__ TileOrder(int bid, int tiles_m, int tiles_n, int ngroups, int order) {
    int tm, tn;
    const int nt = tiles_m * tiles_n;
    if (order != 1 && tiles_m % 8 == 0 && tiles_n % ngroups == 0 && nt == (int)gridDim.x) {
      const int xcd = order == 2 ? bid / (nt / 8) : bid % 8, j = order == 2 ? bid % (nt / 8) : bid / 8;
      const int pm = tiles_m / 8, gn = tiles_n / ngroups;
      const int grp = j / (pm * gn), rem = j % (pm * gn);
      tm = xcd * pm + rem / gn;
      tn = grp * gn + rem % gn;
    } else {
      tm = bid / tiles_n;
      tn = bid % tiles_n;
    }
    m0 = tm * BM;
    n0 = tn * BN;
  }
};

// Copies a staged tile (BM rows of V 16-byte vectors, LD elements apart in
// LDS) to rows m0.. of C (row stride ldc, from column c0), rows past M
// skipped. The LDS reads go in batches of eight ahead of their stores, so a
// thread waits for LDS once per batch rather than once per vector.
template <class T, int BM, int V, int NT, int LD>
__device__ __forceinline__ void store_staged(const T *st, T *C, int ldc, int m0, int c0, int M, int tid) {
  constexpr int EPV = 16 / sizeof(T), ITER = BM * V / NT;
  static_assert(ITER * NT == BM * V, "staged tile shape");
  if constexpr (ITER % 8 == 0) {
    // One asm statement reads the batch and waits for it (lds_read8x16), so
    // the compiler cannot sink each read into its store's row guard.
#pragma unroll
    for (int b0 = 0; b0 < ITER; b0 += 8) {
      const char *p[8];
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = tid + (b0 + u) * NT;
        p[u] = (const char *)(st + (c / V) * LD + (c % V) * EPV);
      }
      lds_read8x16(p, v);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = tid + (b0 + u) * NT, row = m0 + c / V;
        if (row < M) *(uint4 *)(C + (size_t)row * ldc + c0 + (c % V) * EPV) = v[u];
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < ITER; u++) {
      const int c = tid + u * NT, row = m0 + c / V;
      if (row < M) *(uint4 *)(C + (size_t)row * ldc + c0 + (c % V) * EPV) = *(const uint4 *)(st + (c / V) * LD + (c % V) * EPV);
    }
  }
}

// Folded LayerNorm, consumer side. ln_fold_load fetches row `row`'s
// per-part (mean, M2) pairs (fp32: each of a row block's N-tiles reads
// them, so their bytes pass the memory path many times) and mprev (issued
// before the first stages' DMA,
// whose issue is not delayed by them); ln_fold_merge combines the pairs by
// the pairwise update of Chan, Golub and LeVeque for equal counts (the mean
// of the part means; M2 = the parts' M2 plus the count times the squared
// deviations of the part means), in fp64 like the LayerNorm kernel's
// two-pass statistics, and returns (rstd, mean - mprev) with mean and rstd
// rounded to float as that kernel rounds them; write_mean also stores the
// row's mean.
constexpr int kLnMaxParts = 8;  // launch_gemm checks lparts <= 8
__device__ __forceinline__ void ln_fold_load(const GemmArgs &g, const LnFold &lf, int row, float2 (&v)[kLnMaxParts],
                                             float &mp) {
  const int rr = min(row, g.M - 1), np = lf.lparts;
  const float2 *pp = (const float2 *)lf.lpart + (size_t)rr * np;
#pragma unroll
  for (int t = 0; t < kLnMaxParts; t++)
    if (t < np) v[t] = pp[t];
  mp = lf.mprev ? lf.mprev[rr] : 0.0f;
}
__device__ __forceinline__ float2 ln_fold_merge(const GemmArgs &g, const LnFold &lf, int row,
                                                const float2 (&v)[kLnMaxParts], float mp, bool write_mean) {
  const int np = lf.lparts;
  double sum = 0;
#pragma unroll
  for (int t = 0; t < kLnMaxParts; t++)
    if (t < np) sum += (double)v[t].x;
  const double mu = sum / np;
  double m2 = 0;
#pragma unroll
  for (int t = 0; t < kLnMaxParts; t++)
    if (t < np) {
      const double d = (double)v[t].x - mu;
      m2 += (double)v[t].y + (double)kLnPartCols * d * d;
    }
  const float mean = (float)mu;
  if (write_mean && row < g.M) lf.mean_out[row] = mean;
  return make_float2((float)(1.0 / sqrt(m2 / (double)g.K + (double)lf.eps)), mean - mp);
}

// WGM x WGN waves tile the BM x BN block; each wave owns a WM x WN sub-tile.
// The body of gemm_nt_kernel and gemm_nt_ln_kernel (lf: the folded
// LayerNorm's arguments, used by the EPI_*_LN forms only).
template <class T, int BM, int BN, int RB, int NSTAGE, int EPI, int WPE, int WGM, int WGN>
__device__ __forceinline__ void gemm_nt_tile(const GemmArgs &g, const LnFold &lf) {
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  constexpr int NW = WGM * WGN, NT = 64 * NW;
  constexpr int KT = RB / sizeof(T);   // K elements per stage (RB-byte rows)
  constexpr int CPR = RB / 16;         // 16-byte chunks per row
  constexpr int RPI = 1024 / RB;       // rows per wave-wide DMA instruction
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = (BM + BN) * RB;
  constexpr int LOADS = (BM + BN) * CPR / NT;  // 16-byte DMA loads per thread per stage
  static_assert(LOADS * NT == (BM + BN) * CPR, "tile rows must fill whole DMA instructions");
  static_assert(EPI == EPI_F32 || EPI == EPI_F32_LN || EPI == EPI_GEGLU_BWD || TN % 2 == 0,
                "paired epilogues need 64-column wave tiles");
  constexpr bool F32OUT = EPI == EPI_F32 || EPI == EPI_F32_LN;
  constexpr bool GATED = EPI == EPI_GEGLU || EPI == EPI_GEGLU_LN;
  constexpr bool LNC = EPI == EPI_STORE_LN || EPI == EPI_GEGLU_LN;  // folded LayerNorm consumer
  static_assert(NSTAGE >= 2 && LOADS * (NSTAGE - 2) < 64, "pipeline depth");
  // fp32 epilogue staged in WGM passes of WM rows; the others in one pass.
  constexpr int EPI_BYTES = (F32OUT || EPI == EPI_GEGLU_BWD) ? WM * (BN + 4) * 4
                                                            : BM * ((GATED ? BN / 2 : BN) + 8) * (int)sizeof(T);
  constexpr int SMEM_RING = NSTAGE * STAGE > EPI_BYTES ? NSTAGE * STAGE : EPI_BYTES;
  // The folded LayerNorm consumer's row statistics and column sums follow
  // the ring in the same array: a second LDS object would make the compiler
  // wait for every DMA (vmcnt(0)) before the main loop's fragment reads.
  constexpr int LN_BYTES = LNC ? BM * 8 + BN * 4 : 0;
  __shared__ __attribute__((aligned(1024))) char smem[SMEM_RING + LN_BYTES];

  // The wave index is uniform: readfirstlane keeps it (and every LDS-DMA
  // destination, which goes through M0) in scalar registers.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int lr = lane & 31, lh = lane >> 5;

  const TileOrder<BM, BN> to(blockIdx.x, (g.M + BM - 1) / BM, g.N / BN, g.ngroups, g.order);
  const int m0 = to.m0, n0 = to.n0;
  // Folded LayerNorm consumer: thread t < BM takes block row t's statistics
  // and thread t < BN column n0 + t's lcs (loaded here; merged after the
  // main loop, when they have landed with the last stage, so the first
  // stages start without waiting for them); the epilogue reads (rstd, mean -
  // mprev) of its rows from ln_st and its columns' lcs from ln_cs.
  float2 *const ln_st = (float2 *)(smem + SMEM_RING);
  float *const ln_cs = (float *)(smem + SMEM_RING + BM * 8);
  float2 ln_v[LNC ? kLnMaxParts : 1];
  float ln_mp = 0.0f, ln_c = 0.0f;
  if constexpr (LNC) {
    if (threadIdx.x < BM) ln_fold_load(g, lf, m0 + (int)threadIdx.x, ln_v, ln_mp);
    if (threadIdx.x < BN) ln_c = lf.lcs[n0 + threadIdx.x];
  }
  // Split-K: blockIdx.y takes K elements [y*K, (y+1)*K) of A and B and writes
  // its own partial output.
  const size_t koff = (size_t)blockIdx.y * g.K;
  const T *gA = (const T *)g.A + koff, *gB = (const T *)g.B + koff;
  char *gC = (char *)g.C + (size_t)blockIdx.y * g.c_split * (F32OUT ? 4 : sizeof(T));

  // DMA sources: load i of this wave fills tile rows RPI*(wave + NW*i) .. +RPI-1;
  // lane l writes row RPI*(wave+NW*i) + l/CPR, LDS chunk slot l%CPR, which
  // holds the row's logical 16-byte chunk (l%CPR) ^ swz(row).
  const char *src[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; i++) {
    const int r = RPI * (wave + NW * i) + lane / CPR;
    const int c = (lane % CPR) ^ swz<RB>(r);
    if (r < BM)
      src[i] = (const char *)gA + (size_t)min(m0 + r, g.M - 1) * g.lda * sizeof(T) + c * 16;
    else
      src[i] = (const char *)gB + (size_t)(n0 + r - BM) * g.ldb * sizeof(T) + c * 16;
  }
  auto issue_part = [&](int stage, int k0, int i0, int i1) {
    char *dst = smem + stage * STAGE + wave * 1024;
    const size_t kb = (size_t)k0 * sizeof(T);
#pragma unroll
    for (int i = i0; i < i1; i++)
      __builtin_amdgcn_global_load_lds((gbl_void *)(src[i] + kb), (lds_void *)(dst + i * NW * 1024), 16, 0, 0);
  };
  auto issue = [&](int stage, int k0) { issue_part(stage, k0, 0, LOADS); };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  const int rw = wm * WM, cw = wn * WN;  // wave tile origin inside the block tile

  // Every stage issues the same number of DMA loads (past the end of K the
  // last stage is re-read into a ring slot nothing reads again), so the
  // vmcnt arithmetic below is exact and no branch surrounds a DMA issue.
  const int nk = g.K / KT;
#pragma unroll
  for (int s = 0; s < NSTAGE - 1; s++) issue(s, min(s, nk - 1) * KT);

  constexpr int NKS = KT / MF::KSTEP;                  // MFMA k steps per stage
  constexpr int PER_KS = (LOADS + NKS - 1) / NKS;      // next-stage loads issued per k step
  static_assert(NKS % 2 == 0, "operand double buffering alternates per k step");

  // MFMA operands are double buffered across k steps: the fragments of step
  // ks+1 (or of the next stage's step 0) are read from LDS while the MFMAs of
  // step ks run. The next stage's readiness (vmcnt + barrier) is established
  // at the end of each stage, after the last MFMAs of the stage are issued.
  frag fa[2][TM], fb[2][TN];
  auto load_frags = [&](int buf, int stage, int ks) {
    const char *sa = smem + stage * STAGE;
    const char *sb = sa + BM * RB;
    const int ke = ks * MF::KSTEP + lh * MF::SLOTS;  // first k element of this lane's operand
    const int chunk = ke * (int)sizeof(T) / 16, within = ke * (int)sizeof(T) % 16;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int r = wm * WM + i * 32 + lr;
      fa[buf][i] = *(const frag *)(sa + r * RB + ((chunk ^ swz<RB>(r)) << 4) + within);
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int r = wn * WN + j * 32 + lr;
      fb[buf][j] = *(const frag *)(sb + r * RB + ((chunk ^ swz<RB>(r)) << 4) + within);
    }
  };
  // Waits until stage kt has landed for every wave: NSTAGE-2 later stages'
  // loads may still be in flight.
  auto stage_ready = [&]() {
    wait_vmcnt<LOADS * (NSTAGE - 2)>();
    __builtin_amdgcn_s_barrier();
  };

  stage_ready();
  load_frags(0, 0, 0);
  for (int kt = 0; kt < nk; kt++) {
    // Refill the buffer of stage kt-1 (every wave finished reading it before
    // the barrier that made stage kt visible) with stage kt + NSTAGE - 1.
    const int rstage = (kt + NSTAGE - 1) % NSTAGE, rk = min(kt + NSTAGE - 1, nk - 1) * KT;
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const int cur = ks & 1;
      // Program order: next step's operand reads, this step's share of the
      // DMA refill (the DMA writes LDS, so reads placed after it could not be
      // hoisted above it), then this step's MFMAs.
      if (ks + 1 < NKS) load_frags(cur ^ 1, kt % NSTAGE, ks + 1);
      {
        const int i0 = ks * PER_KS < LOADS ? ks * PER_KS : LOADS;
        const int i1 = (ks + 1) * PER_KS < LOADS ? (ks + 1) * PER_KS : LOADS;
        issue_part(rstage, rk, i0, i1);
      }
      // B is the MFMA's first operand: acc[i][j] holds the transposed
      // 32x32 block, so lane l owns token row l%32 and four runs of four
      // consecutive output columns (vector stores in the epilogue).
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = MF::mma(fb[cur][j], fa[cur][i], acc[i][j]);
      // One MFMA, then all of the next step's operand reads (they get the
      // rest of the step to land), then the DMA issues, then the MFMAs.
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (ks + 1 < NKS) __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, PER_KS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - 2, 0);
      if (ks + 1 == NKS && kt + 1 < nk) {
        stage_ready();
        load_frags(cur ^ 1, (kt + 1) % NSTAGE, 0);
      }
    }
  }
  // All waves done with the ring and every DMA landed: reuse it for the epilogue.
  wait_vmcnt<0>();
  if constexpr (LNC) {
    // The folded LayerNorm's row statistics (loaded at the start, landed
    // with the last stage) and column sums, for every wave's epilogue: the
    // barrier must also wait for these LDS writes.
    if (threadIdx.x < BM) ln_st[threadIdx.x] = ln_fold_merge(g, lf, m0 + (int)threadIdx.x, ln_v, ln_mp, n0 == 0);
    if (threadIdx.x < BN) ln_cs[threadIdx.x] = ln_c;
    __syncthreads();
  } else {
    __builtin_amdgcn_s_barrier();
  }
  // fp32 staging of the rows of wave row `pass` (LD floats per row).
  auto stage_f32 = [&](float *st, int LD, int pass) {
    if (wm == pass) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int q = 0; q < 4; q++)
            *(float4 *)(st + (i * 32 + lr) * LD + cw + j * 32 + mfma_row(4 * q, lane)) =
                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
    }
  };
  if constexpr (EPI == EPI_GEGLU_BWD) {
    // The product is dact (the GeGLU output's gradient, fp32, as the
    // reference's backward holds it); each thread takes 8 consecutive
    // columns of one row (inside one 32-column group), reads the matching
    // value and gate inputs and writes their gradients (backward.go:49-61).
    // Output column n of the product is value column 64*(n/32) + n%32 of the
    // interleaved layout, so the tile's outputs are 2*BN contiguous columns.
    constexpr int LD = BN + 4, HM = WM, U = BN / 8;
    constexpr int ITER = HM * U / NT;
    constexpr int BATCH = ITER <= 4 ? ITER : ITER % 4 == 0 ? 4 : ITER % 3 == 0 ? 3 : 2;
    static_assert(ITER * NT == HM * U && ITER % BATCH == 0, "GeGLU backward epilogue shape");
    float *st = (float *)smem;
    const T *Wg = (const T *)g.gin;
    T *D = (T *)gC;
#pragma unroll
    for (int pass = 0; pass < WGM; pass++) {
      stage_f32(st, LD, pass);
      __syncthreads();
      for (int b0 = 0; b0 < ITER; b0 += BATCH) {
        float a[BATCH][8], gt[BATCH][8];
#pragma unroll
        for (int u = 0; u < BATCH; u++) {
          const int c = tid + (b0 + u) * NT, r = c / U, cu = (c % U) * 8;
          const int row = min(m0 + pass * HM + r, g.M - 1);
          const size_t o = (size_t)row * g.ldc + 2 * n0 + 64 * (cu >> 5) + (cu & 31);
          Vec8<T>::load(Wg + o, a[u]);
          Vec8<T>::load(Wg + o + 32, gt[u]);
        }
#pragma unroll
        for (int u = 0; u < BATCH; u++) {
          const int c = tid + (b0 + u) * NT, r = c / U, cu = (c % U) * 8;
          const int row = m0 + pass * HM + r;
          if (row >= g.M) continue;
          const size_t o = (size_t)row * g.ldc + 2 * n0 + 64 * (cu >> 5) + (cu & 31);
          const float4 d0 = *(const float4 *)(st + r * LD + cu), d1 = *(const float4 *)(st + r * LD + cu + 4);
          const float da[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
          float dv[8], dg[8];
#pragma unroll
          for (int e = 0; e < 8; e++) {
            dv[e] = da[e] * gt[u][e] * gelu_grad<T>(a[u][e]);
            dg[e] = da[e] * gelu_erf<T>(a[u][e]);
          }
          Vec8<T>::store(D + o, dv);
          Vec8<T>::store(D + o + 32, dg);
        }
      }
      if (pass + 1 < WGM) __syncthreads();
    }
  } else if constexpr (F32OUT) {
    constexpr bool LN = EPI == EPI_F32_LN;  // also the folded LayerNorm's operand and statistics
    constexpr int LD = BN + 4;  // floats per staged row
    constexpr int HM = WM;      // rows per pass: the waves with wm == pass stage theirs
    float *st = (float *)smem;
    float *C = (float *)gC;
    const float *R = g.res ? g.res : C;  // residual input of the accumulate
    constexpr int V = BN / 4;  // float4 per row
    constexpr int ITER = HM * V / NT;
    static_assert(ITER * NT == HM * V, "epilogue shape");
    // Folded LayerNorm: TPR threads per row of a pass (8 on 256-row tiles).
    constexpr int TPR = NT / HM, CW = 4 * TPR;
    static_assert(!LN || (BN == kLnPartCols && TPR * HM == NT && (TPR == 4 || TPR == 8) && BN % CW == 0),
                  "LayerNorm statistics: 4 or 8 threads per 192-column row");
    const bool vec = (g.ldc & 3) == 0;
    // The residual loads of a pass are issued together (one HBM round trip
    // per pass): pass 0's before its staging, so that their latency overlaps
    // it; each later pass's right after the previous pass's stores, before
    // its staging barrier. Loads and stores of an element are made by the
    // same thread; the rows of different passes are disjoint.
    float4 old[ITER];
    auto load_old = [&](int pass) {
#pragma unroll
      for (int u = 0; u < ITER; u++) {
        const int c = tid + u * NT, r = c / V, c4 = (c % V) * 4;
        const int row = m0 + pass * HM + r, col = n0 + c4;
        old[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (g.accumulate && vec && row < g.M && col + 4 <= g.n_store)
          old[u] = *(const float4 *)(R + (size_t)row * g.ldc + col);
      }
    };
    load_old(0);
    // Folded LayerNorm: thread (row tid / TPR of the pass, part tid % TPR)
    // takes the 4-column chunks 4 part + CW q (q < NQ) of the row, so that
    // the TPR threads of a row store 8 TPR contiguous bytes of the bf16
    // operand per instruction; the LayerNorm weight at them.
    constexpr int NQ = BN / CW;
    float4 lw4[LN ? NQ : 1];
    if constexpr (LN) {
#pragma unroll
      for (int q = 0; q < NQ; q++) lw4[q] = *(const float4 *)(lf.lw + n0 + 4 * (tid % TPR) + CW * q);
    }
#pragma unroll
    for (int pass = 0; pass < WGM; pass++) {
      float ln_mp = 0.0f;
      if constexpr (LN)
        if (lf.mprev) ln_mp = lf.mprev[min(m0 + pass * HM + tid / TPR, g.M - 1)];
      stage_f32(st, LD, pass);
      __syncthreads();
#pragma unroll
      for (int u = 0; u < ITER; u++) {
        const int c = tid + u * NT, r = c / V, c4 = (c % V) * 4;
        const int row = m0 + pass * HM + r, col = n0 + c4;
        if (row >= g.M || col >= g.n_store) continue;
        const float4 v = *(const float4 *)(st + r * LD + c4);
        float *p = C + (size_t)row * g.ldc + col;
        if (vec && col + 4 <= g.n_store) {
          const float4 x = make_float4(v.x + old[u].x, v.y + old[u].y, v.z + old[u].z, v.w + old[u].w);
          *(float4 *)p = x;
          if constexpr (LN)  // read back below (launch_gemm guarantees vec and n_store == N for this form)
            *(float4 *)(st + r * LD + c4) = x;
        } else {
          const float vv[4] = {v.x, v.y, v.z, v.w};
          const float *pr = R + (size_t)row * g.ldc + col;
          for (int q = 0; q < 4 && col + q < g.n_store; q++) p[q] = g.accumulate ? pr[q] + vv[q] : vv[q];
        }
      }
      if constexpr (LN) {
        // The pass's rows from the staging area: TPR threads per row, the
        // chunks above. The next LayerNorm's operand (x - mprev) * w in T,
        // one 8-byte store per chunk; the statistics over this tile's 192
        // columns: fp32 partial sums, the TPR reduced in fp64 in a fixed
        // order, then the squared deviations from the tile mean the same way,
        // stored as an fp32 pair (their fp32 rounding, ~1e-6 relative, is far
        // below the bf16 operand's).
        __syncthreads();
        const int r = tid / TPR, part = tid % TPR;
        float4 xv[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) xv[q] = *(const float4 *)(st + r * LD + 4 * part + CW * q);
        {
          const int row = m0 + pass * HM + r;
          if (row < g.M) {
            T *f = (T *)lf.fx + (size_t)row * g.ldc + n0 + 4 * part;
#pragma unroll
            for (int q = 0; q < NQ; q++) {
              const float4 a = xv[q], wa = lw4[q];
              *(uint2 *)(f + CW * q) = make_uint2(pack16<T>((a.x - ln_mp) * wa.x, (a.y - ln_mp) * wa.y),
                                                  pack16<T>((a.z - ln_mp) * wa.z, (a.w - ln_mp) * wa.w));
            }
          }
        }
        float s32 = 0.0f;
#pragma unroll
        for (int q = 0; q < NQ; q++) s32 += (xv[q].x + xv[q].y) + (xv[q].z + xv[q].w);
        double sum = s32;
#pragma unroll
        for (int o = 1; o < TPR; o <<= 1) sum += __shfl_xor(sum, o);
        const double mu = sum / BN;
        const float muf = (float)mu;
        float q32 = 0.0f;
#pragma unroll
        for (int q = 0; q < NQ; q++) {
          const float a = xv[q].x - muf, b = xv[q].y - muf, c = xv[q].z - muf, d = xv[q].w - muf;
          q32 += (a * a + b * b) + (c * c + d * d);
        }
        double m2 = q32;
#pragma unroll
        for (int o = 1; o < TPR; o <<= 1) m2 += __shfl_xor(m2, o);
        const int row = m0 + pass * HM + r;
        if (part == 0 && row < g.M)
          ((float2 *)lf.lpart)[(size_t)row * lf.lparts + n0 / BN] = make_float2((float)mu, (float)m2);
      }
      if (pass + 1 < WGM) {
        load_old(pass + 1);
        __syncthreads();
      }
    }
  } else {
    // Operand-type epilogue: the plain product (gated false) or the GeGLU of
    // each value/gate column pair (gated true), staged in LDS and stored as
    // 16-byte rows. EPI_GEGLU_KEEP writes both (training keeps the Wi output).
    auto emit = [&](auto gated, T *Cout, int ldo) {
      constexpr bool G = decltype(gated)::value;
      constexpr int OC = G ? BN / 2 : BN;  // output columns of the block tile
      constexpr int LD = OC + 8;           // staged row length (elements)
      typedef T T4 __attribute__((ext_vector_type(4)));
      T *st = (T *)smem;
      // Folded LayerNorm consumer: lcs at this lane's columns (block j, run
      // q: the 4 columns from cw + 32 j + mfma_row(4 q)).
      float cs[LNC ? TN : 1][16];
      if constexpr (LNC) {
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const float4 c4 = *(const float4 *)(ln_cs + cw + j * 32 + mfma_row(4 * q, lane));
            cs[j][4 * q] = c4.x, cs[j][4 * q + 1] = c4.y, cs[j][4 * q + 2] = c4.z, cs[j][4 * q + 3] = c4.w;
          }
      }
      // rstd * (product - (mean - mprev) * lcs) for the folded LayerNorm
      // (ln_st and ln_cs were written before the epilogue's barrier).
      float ln_rs[LNC ? TM : 1], ln_dm[LNC ? TM : 1];
      if constexpr (LNC) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const float2 t = ln_st[rw + 32 * i + lr];
          ln_rs[i] = t.x, ln_dm[i] = t.y;
        }
      }
      auto fin = [&](float v, int i, int j, int e) -> float {
        if constexpr (LNC) {
          float r = __builtin_fmaf(-ln_dm[i], cs[j][e], v) * ln_rs[i];
          // fp16: the compiler would fuse this product into the conversion
          // for some outputs (v_fma_mixlo_f16, one rounding instead of two)
          // and not others, so results would depend on the tile shape; the
          // empty asm keeps every output a rounded fp32 product.
          if constexpr (std::is_same<T, f16>::value) asm("" : "+v"(r));
          return r;
        } else {
          return v;
        }
      };
#pragma unroll
      for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int jp = 0; jp < TN / 2; jp++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const int r = rw + i * 32 + lr, c = mfma_row(4 * q, lane);  // 4 consecutive columns from c
            const f32x16 &a = acc[i][2 * jp], &b = acc[i][2 * jp + 1];
            const int ja = 2 * jp, jb = 2 * jp + 1;
            if constexpr (!G) {
              *(T4 *)(st + r * LD + cw + jp * 64 + c) =
                  T4{to_elem<T>(fin(a[4 * q], i, ja, 4 * q)), to_elem<T>(fin(a[4 * q + 1], i, ja, 4 * q + 1)),
                     to_elem<T>(fin(a[4 * q + 2], i, ja, 4 * q + 2)), to_elem<T>(fin(a[4 * q + 3], i, ja, 4 * q + 3))};
              *(T4 *)(st + r * LD + cw + jp * 64 + 32 + c) =
                  T4{to_elem<T>(fin(b[4 * q], i, jb, 4 * q)), to_elem<T>(fin(b[4 * q + 1], i, jb, 4 * q + 1)),
                     to_elem<T>(fin(b[4 * q + 2], i, jb, 4 * q + 2)), to_elem<T>(fin(b[4 * q + 3], i, jb, 4 * q + 3))};
            } else {
              T4 o;
#pragma unroll
              for (int t = 0; t < 4; t++)
                o[t] = to_elem<T>(gelu_erf<T>(fin(a[4 * q + t], i, ja, 4 * q + t)) * fin(b[4 * q + t], i, jb, 4 * q + t));
              *(T4 *)(st + r * LD + (cw + jp * 64) / 2 + c) = o;
            }
          }
      }
      __syncthreads();
      const int oc0 = G ? n0 / 2 : n0;
      constexpr int EPV = 16 / sizeof(T);  // elements per 16-byte vector
      constexpr int V = OC / EPV;
      store_staged<T, BM, V, NT, LD>(st, Cout, ldo, m0, oc0, g.M, tid);
    };
    if constexpr (EPI == EPI_STORE || EPI == EPI_STORE_LN) {
      emit(std::false_type{}, (T *)gC, g.ldc);
    } else if constexpr (GATED) {
      emit(std::true_type{}, (T *)gC, g.ldc);
    } else {
      emit(std::false_type{}, (T *)gC, g.ldc);
      __syncthreads();  // the staging area is reused
      emit(std::true_type{}, (T *)g.C2, g.ldc2);
    }
  }
}

template <class T, int BM, int BN, int RB, int NSTAGE, int EPI, int WPE, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(WPE))) void gemm_nt_kernel(GemmArgs g) {
  static_assert(EPI < EPI_F32_LN, "the folded-LayerNorm forms run as gemm_nt_ln_kernel");
  gemm_nt_tile<T, BM, BN, RB, NSTAGE, EPI, WPE, WGM, WGN>(g, LnFold{});
}
template <class T, int BM, int BN, int RB, int NSTAGE, int EPI, int WPE, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(WPE))) void gemm_nt_ln_kernel(GemmArgs g,
                                                                                                            LnFold lf) {
  static_assert(EPI >= EPI_F32_LN, "plain forms run as gemm_nt_kernel");
  gemm_nt_tile<T, BM, BN, RB, NSTAGE, EPI, WPE, WGM, WGN>(g, lf);
}

template <class T, int BM, int BN, int RB, int NSTAGE, int WPE, int WGM = 2, int WGN = 2>
hipError_t launch_cfg(int epi, const GemmArgs &a, hipStream_t s, int splits = 1) {
  const int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
  dim3 grid(tiles, splits), block(64 * WGM * WGN);
  // bf16 256-row tiles serve only the operand-type epilogues (the fp32 ones
  // take 128 x 192 or 128 x 128 tiles): the fp32 epilogue is not built there.
  constexpr bool f32_epi = !(sizeof(T) == 2 && BM == 256);
  // The fp16 mode is inference only: no training epilogues.
  constexpr bool train_epi = !std::is_same<T, f16>::value;
  if (!train_epi && (epi == EPI_GEGLU_BWD || epi == EPI_GEGLU_KEEP)) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_F32:
      if constexpr (f32_epi)
        hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, RB, NSTAGE, EPI_F32, WPE, WGM, WGN>), grid, block, 0, s, a);
      else
        return hipErrorInvalidValue;
      break;
    case EPI_STORE:
      hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, RB, NSTAGE, EPI_STORE, WPE, WGM, WGN>), grid, block, 0, s, a);
      break;
    case EPI_GEGLU:
      hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, RB, NSTAGE, EPI_GEGLU, WPE, WGM, WGN>), grid, block, 0, s, a);
      break;
    case EPI_GEGLU_BWD:
      if constexpr (train_epi)
        hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, RB, NSTAGE, EPI_GEGLU_BWD, WPE, WGM, WGN>), grid, block, 0, s, a);
      break;
    default:
      if constexpr (train_epi)
        hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, RB, NSTAGE, EPI_GEGLU_KEEP, WPE, WGM, WGN>), grid, block, 0, s, a);
      break;
  }
  return hipGetLastError();
}

// One epilogue alone (the fp32 one or the GeGLU backward), for tiles whose
// wave columns (BN / 2 = 96) do not pair up for the operand-type epilogues.
// WGM rows of waves (64-row wave tiles when BM = 256 and WGM = 4).
template <class T, int BM, int BN, int RB, int NSTAGE, int WPE, int EPI = EPI_F32, int WGM = 2>
hipError_t launch_cfg_one(const GemmArgs &a, hipStream_t s, int splits = 1, const LnFold *ln = nullptr) {
  static_assert(EPI == EPI_F32 || EPI == EPI_F32_LN || EPI == EPI_GEGLU_BWD, "epilogues that take 96-column wave tiles");
  constexpr int WGN = BN / 96;  // 96-column wave tiles: 2 x 2 waves for 192 columns, 2 x 4 for 384
  static_assert(WGN * 96 == BN && (WGN == 2 || WGN == 4), "96-column wave tiles");
  static_assert(WGM * WGN <= 8, "at most 8 waves per workgroup");
  const int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
  if constexpr (EPI == EPI_F32_LN)
    hipLaunchKernelGGL((gemm_nt_ln_kernel<T, BM, BN, RB, NSTAGE, EPI, WPE, WGM, WGN>), dim3(tiles, splits),
                       dim3(64 * WGM * WGN), 0, s, a, *ln);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, RB, NSTAGE, EPI, WPE, WGM, WGN>), dim3(tiles, splits),
                       dim3(64 * WGM * WGN), 0, s, a);
  return hipGetLastError();
}

// Small-M GEMM (M <= 128 in bf16: one request; M <= 1024 in fp32: the
// scorer's dense layer over every [MASK] row of a batch). Such
// launches are bound by streaming the weights and by latency, and the
// 128-wide tiles above would give only N/128 workgroups. Here a workgroup
// owns a TR x TC output tile (TR = 32*MB rows, TC = 32*NB columns) and all
// of K:
//   * K is walked in groups of GK elements (four 16-byte loads per lane and
//     operand row); the W waves take the groups round-robin and load their
//     MFMA operands straight from global memory into registers (every
//     operand is used by one wave only, so LDS staging buys nothing),
//     prefetching the next group while the current one is multiplied.
//   * The waves' partial tiles are summed through LDS in a fixed order, so
//     results do not depend on timing, by the threads that store the
//     result (one barrier). Splitting K across workgroups of one launch
//     would need a device-scope release/acquire per workgroup (an L2
//     writeback + invalidate on gfx950); instead launch_gemm_small_split
//     gives each K slice its own fp32 partial tile and the kernel that
//     follows (the next LayerNorm, launch_ln_parts) sums the slices.
// Operand layout: in load j of a group, lane l reads the 16 bytes of row
// l%32 at group offset 2*VPL*j + VPL*(l/32); for bf16 that is exactly the
// k step j operand of v_mfma_f32_32x32x16_bf16, for fp32 the four values
// feed four v_mfma_f32_32x32x2f32 (A and B use the same k order).
template <int V>
using fvec = float __attribute__((ext_vector_type(V)));

// Sum of the NP partial tiles (TE floats apart) at float index idx (a
// multiple of V): (p0 + p4) + (p1 + p5) + (p2 + p6) + (p3 + p7) for eight,
// p0 + p1 + p2 + p3 for four.
template <int V, int NP, int TE>
__device__ __forceinline__ fvec<V> partial_sum(const float *red, int idx) {
  const fvec<V> *p = (const fvec<V> *)(red + idx);
  constexpr int S = TE / V;
  fvec<V> v;
  if constexpr (NP == 8) {
    v = p[0] + p[4 * S];
#pragma unroll
    for (int w = 1; w < 4; w++) v = v + (p[w * S] + p[(w + 4) * S]);
  } else {
    v = p[0];
#pragma unroll
    for (int w = 1; w < 4; w++) v = v + p[w * S];
  }
  return v;
}

template <class T, int MB, int NB, int EPI, int W, bool F16 = false, bool DMA = false>
__global__ __launch_bounds__(64 * W) void gemm_skinny_kernel(GemmArgs g) {
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  static_assert(!F16 || sizeof(T) == 2, "16 x 16 blocks: 16-bit operands");
  static_assert(!DMA || (F16 && MB == 1 && NB == 1 && W == 8), "LDS operand path: 16-bit 32 x 32 tiles, 8 waves");
  // DMA: each wave stages its K groups through a private two-slot LDS slab.
  // A group's 32 A rows and 32 B rows (128 bytes each) arrive by eight
  // wave-wide global->LDS loads, lane l carrying 16 bytes of row 8j + l/8, so
  // every row is read as one whole 128-byte segment (the register path's
  // lanes read 64-byte pieces of 16 rows per instruction); the fragments are
  // then read from LDS in the same layout the register path loads them in,
  // so both paths feed the MFMAs the same operands in the same order.
  constexpr int SLAB = 64 * 128;  // bytes of one group (64 rows x 128 bytes)
  // F16: the tile as 16 x 16 blocks of the 16 x 16 x 32 MFMA, whose operand
  // lanes read 64 contiguous bytes of a row (four lanes x 16 bytes) where the
  // 32 x 32 x 16 form reads 32 (two lanes): half the cache-line sectors per
  // load instruction.
  constexpr int BW = F16 ? 16 : 32;                  // block width
  constexpr int RB = 32 * MB / BW, CB = 32 * NB / BW;  // row / column blocks
  constexpr int NS = F16 ? 2 : 4;                    // MFMA k steps per 64-element group
  constexpr int NE = F16 ? 4 : 16;                   // accumulator elements per lane
  typedef float accv __attribute__((__vector_size__(NE * sizeof(float))));
  constexpr int NT = 64 * W;
  constexpr int VPL = 16 / (int)sizeof(T);  // elements per 16-byte load
  constexpr int GK = 8 * VPL;               // k elements per group
  constexpr int TR = 32 * MB, TC = 32 * NB, TE = TR * TC;
  static_assert(EPI != EPI_GEGLU_KEEP || NB == 2, "the kept pre-activation tile is 32 value + 32 gate columns");
  static_assert(EPI != EPI_GEGLU || NB <= 2, "GeGLU tiles");
  static_assert(W == 4 || W == 8, "wave count");
  // Partial tiles held in LDS at once: all W when they fit in 64 KB.
  constexpr bool FOLD = W == 8 && 8 * TE * 4 > 65536;
  constexpr int NP = FOLD ? 4 : W;
  // The fp32 epilogue works on items of FV floats, two when that gives every
  // thread one item; NQ items per thread.
  constexpr int FV = TE <= 2 * NT ? 2 : 4, TEV = TE / FV, NQ = (TEV + NT - 1) / NT;
  // The partial tiles; in DMA mode the same memory first holds the waves'
  // slabs (W x 2 groups), and a barrier separates the two uses.
  constexpr int RED = DMA && W * 2 * SLAB / 4 > NP * TE ? W * 2 * SLAB / 4 : NP * TE;
  __shared__ __attribute__((aligned(1024))) float red[RED];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, lh = lane >> 5;
  const int n0 = blockIdx.x * TC, m0 = blockIdx.y * TR;
  // Split-K (fp32 epilogue): blockIdx.z takes K elements [z*K, (z+1)*K) of A
  // and B and writes its own partial output, c_split elements further on.
  const int kz = blockIdx.z * g.K;

  // This lane's row (column) within a block and its first k element.
  const int brow = F16 ? (lane & 15) : lr, bk = F16 ? (lane >> 4) * VPL : lh * VPL;
  const T *ap[RB], *bp[CB];
#pragma unroll
  for (int i = 0; i < RB; i++) ap[i] = (const T *)g.A + (size_t)min(m0 + BW * i + brow, g.M - 1) * g.lda + kz + bk;
#pragma unroll
  for (int j = 0; j < CB; j++) {
    const int cc = BW * j + brow;  // tile column
    // GeGLU on 32-column tiles: the 64-row group n0 / 64 of the interleaved
    // weights holds 32 value rows then their 32 gate rows; tile half
    // (n0 / 32) % 2 takes value rows 16h .. 16h+15 as columns 0..15 and the
    // matching gate rows as columns 16..31, so the tile's outputs are the 16
    // columns n0 / 2 .. n0 / 2 + 15.
    const int row = (EPI == EPI_GEGLU && NB == 1)
                        ? (n0 & ~63) + (cc < 16 ? 0 : 32) + ((n0 >> 5) & 1) * 16 + (cc & 15)
                        : n0 + cc;
    bp[j] = (const T *)g.B + (size_t)row * g.ldb + kz + bk;
  }

  accv acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; i++)
#pragma unroll
    for (int j = 0; j < CB; j++)
#pragma unroll
      for (int e = 0; e < NE; e++) acc[i][j][e] = 0.0f;
  // Tile element (row-major TR x TC) of accumulator element e of block (i, j).
  auto tile_at = [&](int i, int j, int e) {
    if constexpr (F16) return (BW * i + 4 * (lane >> 4) + e) * TC + BW * j + (lane & 15);
    else return (32 * i + mfma_row(e, lane)) * TC + 32 * j + lr;
  };

#define SKINNY_LOAD(XA, XB, GRP)                                                                   \
  do {                                                                                             \
    const int k_ = (GRP) * GK;                                                                     \
    _Pragma("unroll") for (int i = 0; i < RB; i++) _Pragma("unroll") for (int q = 0; q < NS; q++) \
        XA[i][q] = *(const uint4 *)(ap[i] + k_ + (GK / NS) * q);                                   \
    _Pragma("unroll") for (int j = 0; j < CB; j++) _Pragma("unroll") for (int q = 0; q < NS; q++) \
        XB[j][q] = *(const uint4 *)(bp[j] + k_ + (GK / NS) * q);                                   \
  } while (0)

  const int ngrp = g.K / GK;
  uint4 la[RB][NS], lb[CB][NS];
  int grp = wave;
  if (!DMA && grp < ngrp) SKINNY_LOAD(la, lb, grp);
  // The fp32 epilogue's residual input, loaded now (behind the first operand
  // group) so its latency overlaps the main loop instead of following the
  // reduction; each element is read and then written by this thread only.
  fvec<FV> pre[NQ];
  const bool vec = (g.ldc & (FV - 1)) == 0;
  if constexpr (EPI == EPI_F32) {
    const float *R = g.res ? g.res : (const float *)g.C;
#pragma unroll
    for (int k = 0; k < NQ; k++) {
      pre[k] = 0.0f;
      const int q = tid + NT * k;
      const int r = q / (TC / FV), col = n0 + (q % (TC / FV)) * FV;
      if (g.accumulate && vec && q < TEV && m0 + r < g.M && col + FV <= g.n_store)
        pre[k] = *(const fvec<FV> *)(R + (size_t)(m0 + r) * g.ldc + col);
    }
  }
  if constexpr (DMA) {
    // Slab row r < 32 is A row m0 + r, r >= 32 the B row of tile column
    // r - 32 (the mapping of bp above). DMA load j of a group fills slab
    // rows 8j .. 8j+7; lane l brings the 16-byte chunk (l % 8) ^ swz(row) of
    // row 8j + l / 8 into LDS slot l % 8 of that row, so a row's logical
    // chunk c sits in slot c ^ swz(row) (the XOR swizzle spreads the 16 rows
    // a quarter-wave reads over distinct banks).
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const char *dsrc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int r = 8 * j + (lane >> 3);
      const int c = (lane & 7) ^ swz<128>(r);
      const T *row;
      if (r < 32) {
        row = (const T *)g.A + (size_t)min(m0 + r, g.M - 1) * g.lda;
      } else {
        const int cc = r - 32;
        const int br = EPI == EPI_GEGLU ? (n0 & ~63) + (cc < 16 ? 0 : 32) + ((n0 >> 5) & 1) * 16 + (cc & 15) : n0 + cc;
        row = (const T *)g.B + (size_t)br * g.ldb;
      }
      dsrc[j] = (const char *)(row + kz) + c * 16;
    }
    // The LDS reads are opaque to the compiler (lds_read8x16), so it adds no
    // waits of its own for the DMA: the vmcnt waits below are the only ones.
    auto issue = [&](int gi, int slot) {
      char *dst = (char *)red + (wv * 2 + slot) * SLAB;
      const size_t kb = (size_t)gi * GK * sizeof(T);
#pragma unroll
      for (int j = 0; j < 8; j++)
        __builtin_amdgcn_global_load_lds((gbl_void *)(dsrc[j] + kb), (lds_void *)(dst + j * 1024), 16, 0, 0);
    };
    // This wave's groups: wv, wv + W, ... (the register path's order).
    const int myn = wv < ngrp ? (ngrp - 1 - wv) / W + 1 : 0;
    if (myn > 0) issue(wv, 0);
    if (myn > 1) issue(wv + W, 1);
    for (int i = 0; i < myn; i++) {
      // Group i has landed once at most the next group's eight loads are
      // outstanding (the residual loads above are older and count as done).
      if (i + 1 < myn) wait_vmcnt<8>();
      else wait_vmcnt<0>();
      const char *sl = (const char *)red + (wv * 2 + (i & 1)) * SLAB;
      const char *fp[8];
      uint4 fr[8];
#pragma unroll
      for (int q = 0; q < NS; q++) {
        const int c = (lane >> 4) + 4 * q;  // the register path's k chunk for this lane
#pragma unroll
        for (int b = 0; b < 2; b++) {
          const int ra = 16 * b + (lane & 15), rb = 32 + ra;
          fp[4 * q + b] = sl + ra * 128 + ((c ^ swz<128>(ra)) << 4);
          fp[4 * q + 2 + b] = sl + rb * 128 + ((c ^ swz<128>(rb)) << 4);
        }
      }
      // The fragments are in registers when this returns: the MFMAs may use
      // them and the slot can be refilled with group i + 2.
      lds_read8x16(fp, fr);
#pragma unroll
      for (int q = 0; q < NS; q++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
          la[b][q] = fr[4 * q + b];
          lb[b][q] = fr[4 * q + 2 + b];
        }
      if (i + 2 < myn) issue(wv + (i + 2) * W, i & 1);
#pragma unroll
      for (int q = 0; q < NS; q++)
#pragma unroll
        for (int a = 0; a < RB; a++)
#pragma unroll
          for (int b = 0; b < CB; b++)
            acc[a][b] = mma16x16<T>(__builtin_bit_cast(frag, la[a][q]), __builtin_bit_cast(frag, lb[b][q]), acc[a][b]);
    }
    // Every load has landed and every wave is done with its slab before the
    // partial tiles reuse the memory.
    wait_vmcnt<0>();
    __syncthreads();
    grp = ngrp;  // the register loop below does nothing
  }
  for (; grp < ngrp; grp += W) {
    uint4 na[RB][NS], nb[CB][NS];
    const bool more = grp + W < ngrp;
    if (more) SKINNY_LOAD(na, nb, grp + W);
#pragma unroll
    for (int q = 0; q < NS; q++) {
      if constexpr (F16) {
#pragma unroll
        for (int i = 0; i < RB; i++)
#pragma unroll
          for (int j = 0; j < CB; j++)
            acc[i][j] = mma16x16<T>(__builtin_bit_cast(frag, la[i][q]), __builtin_bit_cast(frag, lb[j][q]), acc[i][j]);
      } else if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < NB; j++)
            acc[i][j] = MF::mma(__builtin_bit_cast(frag, la[i][q]), __builtin_bit_cast(frag, lb[j][q]), acc[i][j]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
          for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) {
              const uint4 a4 = la[i][q], b4 = lb[j][q];
              const unsigned ua = e == 0 ? a4.x : e == 1 ? a4.y : e == 2 ? a4.z : a4.w;
              const unsigned ub = e == 0 ? b4.x : e == 1 ? b4.y : e == 2 ? b4.z : b4.w;
              acc[i][j] = MF::mma(__builtin_bit_cast(frag, ua), __builtin_bit_cast(frag, ub), acc[i][j]);
            }
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < RB; i++)
#pragma unroll
        for (int q = 0; q < NS; q++) la[i][q] = na[i][q];
#pragma unroll
      for (int j = 0; j < CB; j++)
#pragma unroll
        for (int q = 0; q < NS; q++) lb[j][q] = nb[j][q];
    }
  }
#undef SKINNY_LOAD

  // Reduce the W partial tiles (row-major TR x TC) in a fixed order:
  // (p0 + p4) + (p1 + p5) + (p2 + p6) + (p3 + p7) with 8 waves, p0 + p1 + p2 +
  // p3 with 4. When the eight partials fit in LDS every wave stores its own
  // and one barrier follows; otherwise waves 4..7 fold theirs into waves 0..3
  // first. Each epilogue thread then sums only the elements it stores.
  if constexpr (FOLD) {
    if (wave >= 4) {
      float *mine = red + (wave - 4) * TE;
#pragma unroll
      for (int i = 0; i < RB; i++)
#pragma unroll
        for (int j = 0; j < CB; j++)
#pragma unroll
          for (int e = 0; e < NE; e++) mine[tile_at(i, j, e)] = acc[i][j][e];
    }
    __syncthreads();
    if (wave < 4) {
      const float *theirs = red + wave * TE;
#pragma unroll
      for (int i = 0; i < RB; i++)
#pragma unroll
        for (int j = 0; j < CB; j++)
#pragma unroll
          for (int e = 0; e < NE; e++) acc[i][j][e] += theirs[tile_at(i, j, e)];
    }
    __syncthreads();
  }
  if (wave < NP) {
    float *mine = red + wave * TE;
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
      for (int j = 0; j < CB; j++)
#pragma unroll
        for (int e = 0; e < NE; e++) mine[tile_at(i, j, e)] = acc[i][j][e];
  }
  __syncthreads();
  if constexpr (EPI == EPI_F32) {
    float *C = (float *)g.C + blockIdx.z * g.c_split;
#pragma unroll
    for (int k = 0; k < NQ; k++) {
      const int q = tid + NT * k;
      if (q >= TEV) break;
      const int r = q / (TC / FV), c = (q % (TC / FV)) * FV, col = n0 + c;
      if (m0 + r >= g.M || col >= g.n_store) continue;
      const fvec<FV> v = partial_sum<FV, NP, TE>(red, r * TC + c);
      float *p = C + (size_t)(m0 + r) * g.ldc + col;
      if (vec && col + FV <= g.n_store) {
        *(fvec<FV> *)p = pre[k] + v;
      } else {
        const float *pr = (g.res ? g.res : C) + (size_t)(m0 + r) * g.ldc + col;  // residual input
        for (int u = 0; u < FV && col + u < g.n_store; u++) p[u] = g.accumulate ? pr[u] + v[u] : v[u];
      }
    }
  } else {
    auto emit = [&](auto gated, T *C, int ldo) {
      constexpr bool G = decltype(gated)::value;
      constexpr int OC = G ? TC / 2 : TC;  // output columns of the tile
      // Elements per thread item: 16-bit types down to 2 (a 4-byte store) so
      // that every thread has an item; fp32 4 (16 bytes).
      constexpr int EPV = sizeof(T) == 4 ? 4 : TR * OC >= 8 * NT ? 8 : TR * OC >= 4 * NT ? 4 : 2;
      constexpr int RV = EPV > 4 ? 4 : EPV;  // partial-sum vector width
      const int oc0 = G ? n0 / 2 : n0;
      for (int q = tid; q < TR * (OC / EPV); q += NT) {
        const int r = q / (OC / EPV), c = (q % (OC / EPV)) * EPV;
        if (m0 + r >= g.M) continue;
        float val[EPV], gate[EPV];
#pragma unroll
        for (int h = 0; h < EPV / RV; h++) {
          const fvec<RV> v = partial_sum<RV, NP, TE>(red, r * TC + c + RV * h);
#pragma unroll
          for (int u = 0; u < RV; u++) val[RV * h + u] = v[u];
          if constexpr (G) {
            const fvec<RV> x = partial_sum<RV, NP, TE>(red, r * TC + TC / 2 + c + RV * h);
#pragma unroll
            for (int u = 0; u < RV; u++) gate[RV * h + u] = x[u];
          }
        }
        float o[EPV];
#pragma unroll
        for (int u = 0; u < EPV; u++) {
          if constexpr (!G) {
            o[u] = val[u];
          } else {
            o[u] = gelu_erf<T>(val[u]) * gate[u];
          }
        }
        T *dst = C + (size_t)(m0 + r) * ldo + oc0 + c;
        if constexpr (sizeof(T) == 2) {
          unsigned w[EPV / 2];
#pragma unroll
          for (int u = 0; u < EPV / 2; u++) w[u] = pack16<T>(o[2 * u], o[2 * u + 1]);
          if constexpr (EPV == 8) *(uint4 *)dst = make_uint4(w[0], w[1], w[2], w[3]);
          else if constexpr (EPV == 4) *(uint2 *)dst = make_uint2(w[0], w[1]);
          else *(unsigned *)dst = w[0];
        } else {
          *(float4 *)dst = make_float4(o[0], o[1], o[2], o[3]);
        }
      }
    };
    if constexpr (EPI == EPI_STORE) {
      emit(std::false_type{}, (T *)g.C, g.ldc);
    } else if constexpr (EPI == EPI_GEGLU) {
      emit(std::true_type{}, (T *)g.C, g.ldc);
    } else {
      emit(std::false_type{}, (T *)g.C, g.ldc);
      emit(std::true_type{}, (T *)g.C2, g.ldc2);
    }
  }
}

// bf16 32 x 32 tiles run as 16 x 16 x 32 MFMA blocks (cfg5 0.7165 -> 0.7055
// ms); the 64-row and 64-column tiles of 112-row batches were slower that
// way (0.860 -> 0.868 ms) and keep 32 x 32 x 16.
template <class T, int MB, int NB, int W>
hipError_t launch_skinny_cfg(int epi, const GemmArgs &a, hipStream_t s, int splits = 1) {
  constexpr bool F = sizeof(T) == 2 && MB == 1 && NB == 1;
  constexpr bool D = F && W == 8;  // the LDS operand path exists for these tiles
  dim3 grid(a.N / (32 * NB), (a.M + 32 * MB - 1) / (32 * MB), splits), block(64 * W);
  const bool dma = D && !a.skinny_regs;
#define SKINNY_LAUNCH(E)                                                                        \
  do {                                                                                          \
    if (dma)                                                                                    \
      hipLaunchKernelGGL((gemm_skinny_kernel<T, MB, NB, E, W, F, D>), grid, block, 0, s, a);   \
    else                                                                                        \
      hipLaunchKernelGGL((gemm_skinny_kernel<T, MB, NB, E, W, F>), grid, block, 0, s, a);      \
  } while (0)
  switch (epi) {
    case EPI_F32:
      SKINNY_LAUNCH(EPI_F32);
      break;
    case EPI_STORE:
      SKINNY_LAUNCH(EPI_STORE);
      break;
    case EPI_GEGLU:
      SKINNY_LAUNCH(EPI_GEGLU);
      break;
    default:
      if constexpr (NB == 2 && !std::is_same<T, f16>::value)
        hipLaunchKernelGGL((gemm_skinny_kernel<T, MB, 2, EPI_GEGLU_KEEP, W, F>), grid, block, 0, s, a);
      else return hipErrorInvalidValue;
      break;
  }
#undef SKINNY_LAUNCH
  return hipGetLastError();
}

// Tile choice, 8 waves: 32-row tiles up to 128 rows while the grid fits one
// workgroup per CU (more workgroups for the few rows: cfg5 1.10 -> 0.92 ms,
// cfg2 1.18 -> 1.06 ms against 64-row tiles everywhere), 64-row tiles
// otherwise; 32 columns, or for GeGLU 32 (16 value + 16 gate rows) or 64
// (32 + 32; training's kept pre-activation always).
template <class T>
hipError_t launch_skinny(int epi, const GemmArgs &a, hipStream_t s) {
  if (epi == EPI_GEGLU || epi == EPI_GEGLU_KEEP) {
    // Inference GeGLU on 32-column tiles (16 outputs each) while their grid
    // fits one workgroup per CU (MI355X: 256): twice the workgroups of the
    // 64-column tiles, a third less operand traffic per workgroup (cfg5
    // 0.809 -> 0.789 ms; at 112 rows, 288 workgroups, 0.932 -> 0.951 ms).
    if (a.M <= 128 && epi == EPI_GEGLU && (a.N / 32) * ((a.M + 31) / 32) <= 256)
      return launch_skinny_cfg<T, 1, 1, 8>(epi, a, s);
    if (a.M <= 128) return launch_skinny_cfg<T, 1, 2, 8>(epi, a, s);
    // fp32 inference GeGLU above 128 rows also on 32-row tiles (one 512-token
    // fp32 forward 3.92 -> 3.80 ms against 64 x 64, bit-identical).
    if (std::is_same<T, float>::value && epi == EPI_GEGLU) return launch_skinny_cfg<T, 1, 2, 8>(epi, a, s);
    return launch_skinny_cfg<T, 2, 2, 8>(epi, a, s);
  }
  // 32-row tiles while their grid fits one workgroup per CU, else 64-row
  // tiles (QKV at 112 rows: 288 -> 144 workgroups, cfg2 0.917 -> 0.901 ms).
  if (a.M <= 128 && (a.N / 32) * ((a.M + 31) / 32) <= 256) return launch_skinny_cfg<T, 1, 1, 8>(epi, a, s);
  // fp32 above 128 rows (the validation GEMM, the certification twin's
  // forward): 32 x 32 tiles for outputs of 2048 columns or more, two
  // workgroups per CU (512 x 2304 x 768: 39.6 -> 33.5 us; 1024 rows: 64.1 ->
  // 55.6 us; bit-identical, the same K split over eight waves); the 768-wide
  // outputs keep 64-row tiles (their 32 x 32 grid: 14.2 -> 15.4 us).
  if (std::is_same<T, float>::value && a.M > 128 && a.N >= 2048) return launch_skinny_cfg<T, 1, 1, 8>(epi, a, s);
  return launch_skinny_cfg<T, 2, 1, 8>(epi, a, s);
}

// Small-M split-K: a workgroup's time grows with the K it streams (~3.4 ns
// per K element at M = 64 on top of ~2.1 us, whatever the grid), so K is
// split over `splits` workgroups per tile, each writing an fp32 partial tile
// into partial[z][M x N]; the consumer sums them.
template <class T>
hipError_t launch_skinny_split(const GemmArgs &a0, int splits, float *partial, hipStream_t s) {
  GemmArgs a = a0;
  a.K = a0.K / splits;
  a.C = partial;
  a.res = nullptr;
  a.ldc = a0.N;
  a.n_store = a0.N;
  a.accumulate = 0;
  a.c_split = (size_t)a0.M * a0.N;
  return launch_skinny_cfg<T, 1, 1, 8>(EPI_F32, a, s, splits);
}

// C (+)= sum over splits of part[s * n + i], in split order; four
// consecutive elements per thread (n % 4 == 0), every split's load issued
// before the sum.
__global__ void splitk_reduce_kernel(const float *part, int splits, size_t n, float *C, int accumulate) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  constexpr int MAXS = 16;
  float4 p[MAXS];
#pragma unroll
  for (int s = 0; s < MAXS; s++)
    if (s < splits) p[s] = *(const float4 *)(part + (size_t)s * n + i);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int s = 0; s < MAXS; s++)
    if (s < splits) acc = make_float4(acc.x + p[s].x, acc.y + p[s].y, acc.z + p[s].z, acc.w + p[s].w);
  if (accumulate) {
    const float4 c = *(const float4 *)(C + i);
    acc = make_float4(c.x + acc.x, c.y + acc.y, c.z + acc.z, c.w + acc.w);
  }
  *(float4 *)(C + i) = acc;
}

}  // namespace

hipError_t launch_gemm_splitk(int precision, const GemmArgs &a0, int splits, float *partial, hipStream_t s) {
  if (a0.M <= 0) return hipSuccess;
  if (precision == PREC_F16) return hipErrorInvalidValue;  // training only
  if (splits < 1 || splits > 16 || a0.K % (splits * 64) != 0 || a0.N % 128 != 0) return hipErrorInvalidValue;
  GemmArgs a = a0;
  a.K = a0.K / splits;
  a.C = partial;
  a.ldc = a0.N;
  a.n_store = a0.N;
  a.accumulate = 0;
  a.c_split = (size_t)a0.M * a0.N;
  a.ngroups = 1;
  a.order = 1;  // row-major tile order: the grid is (tiles, splits)
  // bf16: 64 x 128 tiles with 128-byte K stages (the long-K weight-gradient
  // shapes run best on them, unsplit or lightly split).
  hipError_t e = precision == 1 ? launch_cfg<bf16, 64, 128, 128, 4, 1>(EPI_F32, a, s, splits)
                                : launch_cfg<float, 128, 128, 128, 3, 1>(EPI_F32, a, s, splits);
  if (e != hipSuccess) return e;
  const size_t n = (size_t)a0.M * a0.N;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, partial, splits,
                     n, (float *)a0.C, a0.accumulate);
  return hipGetLastError();
}

hipError_t launch_gemm_small_split(int precision, const GemmArgs &a, int splits, float *partial, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  const int kt = prec16(precision) ? 64 : 32;
  if (a.M > 128 || splits < 1 || a.K % (splits * kt) != 0 || a.N % 128 != 0) return hipErrorInvalidValue;
  return precision == PREC_BF16  ? launch_skinny_split<bf16>(a, splits, partial, s)
         : precision == PREC_F16 ? launch_skinny_split<f16>(a, splits, partial, s)
                                 : launch_skinny_split<float>(a, splits, partial, s);
}

// All tile configs use BN = 128; K is staged 64 or 128 bytes per step.
bool gemm_shape_ok(int precision, int N, int K) {
  const int kt = prec16(precision) ? 64 : 32;
  return N > 0 && K > 0 && N % 128 == 0 && K % kt == 0;
}

bool gemm_epi_ok(int precision, int epi, int M) {
  if (epi >= EPI_F32_LN) return prec16(precision) && M > 1024;
  if (epi != EPI_GEGLU_BWD) return true;
  return prec16(precision) ? M > 128 : M > 1024;
}

bool gemm_ln_fold_ok(int precision, int M, int hidden, int inter) {
  return prec16(precision) && M > 1024 && hidden % kLnPartCols == 0 && hidden / kLnPartCols <= 8 &&
         3 * hidden > 1024 && (3 * hidden) % 128 == 0 && (2 * inter) % 128 == 0 && inter % 64 == 0;
}

// Any-shape GEMM (model geometries the MFMA kernels do not tile): thread n of
// block (x, m) computes output element (m, 256 x + n) as an fp32 dot product
// over K in order, then the epilogue. Performance is not its purpose.
template <class T, int EPI>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmArgs g) {
  const int m = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
  const int ncols = EPI == EPI_GEGLU ? g.N / 2 : g.N;
  if (m >= g.M || n >= ncols) return;
  const T *a = (const T *)g.A + (size_t)m * g.lda;
  auto dot = [&](int row) {
    const T *b = (const T *)g.B + (size_t)row * g.ldb;
    float acc = 0.0f;
    for (int k = 0; k < g.K; k++) acc = fmaf((float)a[k], (float)b[k], acc);
    return acc;
  };
  if constexpr (EPI == EPI_F32) {
    if (n >= g.n_store) return;
    const float v = dot(n);
    float *C = (float *)g.C + (size_t)m * g.ldc + n;
    const float *R = g.res ? g.res + (size_t)m * g.ldc + n : C;
    *C = g.accumulate ? *R + v : v;
  } else if constexpr (EPI == EPI_STORE) {
    ((T *)g.C)[(size_t)m * g.ldc + n] = to_elem<T>(dot(n));
  } else {
    const float v = dot(n), gate = dot(ncols + n);
    ((T *)g.C)[(size_t)m * g.ldc + n] = to_elem<T>(gelu_erf<T>(v) * gate);
  }
}

template <class T>
hipError_t launch_gemm_generic_t(int epi, const GemmArgs &a, hipStream_t s) {
  const int ncols = epi == EPI_GEGLU ? a.N / 2 : a.N;
  const dim3 grid((ncols + 255) / 256, a.M), block(256);
  switch (epi) {
    case EPI_F32: hipLaunchKernelGGL((gemm_generic_kernel<T, EPI_F32>), grid, block, 0, s, a); break;
    case EPI_STORE: hipLaunchKernelGGL((gemm_generic_kernel<T, EPI_STORE>), grid, block, 0, s, a); break;
    case EPI_GEGLU: hipLaunchKernelGGL((gemm_generic_kernel<T, EPI_GEGLU>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemm_generic(int precision, int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.N <= 0 || a.K <= 0 || (epi == EPI_GEGLU && a.N % 2)) return hipErrorInvalidValue;
  return precision == PREC_BF16  ? launch_gemm_generic_t<bf16>(epi, a, s)
         : precision == PREC_F16 ? launch_gemm_generic_t<f16>(epi, a, s)
                                 : launch_gemm_generic_t<float>(epi, a, s);
}

// The tiled kernel's configuration for 16-bit operands (bf16 or fp16; the
// same tiles, measured on bf16).
template <class T>
hipError_t launch_gemm16(int epi, const GemmArgs &a, hipStream_t s, const LnFold *ln);

hipError_t launch_gemm(int precision, int epi, const GemmArgs &a0, hipStream_t s, const LnFold *ln) {
  if (a0.M <= 0) return hipSuccess;
  if (!gemm_epi_ok(precision, epi, a0.M) || (epi == EPI_GEGLU_BWD && (!a0.gin || a0.ldc % 8))) return hipErrorInvalidValue;
  // Small M goes to the whole-K kernel (grid: N/32 x M/64 workgroups). In
  // fp32 (the scorer's dense layer over all [MASK] rows, the fp32 validation
  // build) that pays up to M = 1024: the 64 x 128 tiles below would leave
  // most CUs idle with a 24-step fp32 K loop each.
  if (a0.M <= 128)
    return precision == PREC_BF16  ? launch_skinny<bf16>(epi, a0, s)
           : precision == PREC_F16 ? launch_skinny<f16>(epi, a0, s)
                                   : launch_skinny<float>(epi, a0, s);
  if (precision == PREC_F32 && a0.M <= 1024) return launch_skinny<float>(epi, a0, s);
  GemmArgs a = a0;
  // N groups per XCD sweep: keep the group's slice of B (N/groups rows of
  // K elements) within about 2 MB of L2.
  const size_t b_bytes = (size_t)a.N * a.K * (prec16(precision) ? 2 : 4);
  const int tiles_n = a.N / 128;
  int groups = 1;
  while (b_bytes / groups > (2u << 20) && groups < tiles_n) {
    groups++;
    while (tiles_n % groups) groups++;
  }
  a.ngroups = groups;
  a.order = 0;
  // Tile configs (measured on cfg3 shapes, 2304- and 768-wide outputs):
  //  * M <= 1024: 64 x 128, 128-byte K stages, 4 stages, 1 workgroup per CU;
  //  * paired / store epilogues (N = 2304): 256 x 128, 64-byte stages x 3
  //    (72 KB LDS), two workgroups per CU so one tile's epilogue and DMA
  //    stalls overlap the other's MFMAs;
  //  * fp32 epilogue with N a multiple of 192 (the 768-wide Wo / MlpWo and
  //    dX GEMMs): 192-column tiles (below); other fp32 outputs and the GeGLU
  //    backward (training): 128 x 128, 64-byte stages x 3 (48 KB), three
  //    workgroups per CU.
  //  * medium M (the trainer's micro-batches: a few thousand rows) has too
  //    few large tiles to fill 256 CUs: up to 4096 rows the fp32 and the
  //    narrow (N <= 1024) store epilogues take 64 x 128 tiles and the wide
  //    store 128 x 128; the GeGLU epilogues keep 128 x 128 up to 8192 rows
  //    (isolated launches on the training shapes, 3840 rows: Wi + GeGLU 36.4
  //    -> 31.3 us, dX GEMMs N = 768 K = 2304 32.3 -> 30.4 us, dctx 16.0 ->
  //    12.6 us).
  if (precision == PREC_BF16) return launch_gemm16<bf16>(epi, a, s, ln);
  if (precision == PREC_F16) return launch_gemm16<f16>(epi, a, s, ln);
  if (a.M <= 1024) return launch_cfg<float, 64, 128, 128, 4, 1>(epi, a, s);
  return launch_cfg<float, 256, 128, 128, 3, 1>(epi, a, s);
}

// The folded-LayerNorm forms on the tiles launch_gemm16 gives their plain
// counterparts at M > 1024 (the 192-column residual tiles; the store and
// GeGLU tiles of N > 1024).
template <class T, int BM, int BN, int RB, int NSTAGE, int WPE, int EPI>
hipError_t launch_fold_cfg(const GemmArgs &a, const LnFold &ln, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
  hipLaunchKernelGGL((gemm_nt_ln_kernel<T, BM, BN, RB, NSTAGE, EPI, WPE, 2, 2>), dim3(tiles), dim3(256), 0, s, a, ln);
  return hipGetLastError();
}

template <class T>
hipError_t launch_gemm_fold(int epi, const GemmArgs &a, const LnFold *ln, hipStream_t s) {
  const bool medium = a.M <= 4096;
  if (!ln) return hipErrorInvalidValue;
  if (epi == EPI_F32_LN) {
    if (a.N % kLnPartCols || ln->lparts != a.N / kLnPartCols || !a.accumulate || a.ldc % 4 || a.n_store != a.N ||
        !ln->fx || !ln->lw || !ln->lpart)
      return hipErrorInvalidValue;
    if (medium) return launch_cfg_one<T, 64, 192, 128, 4, 1, EPI_F32_LN>(a, s, 1, ln);
    return launch_cfg_one<T, 256, 192, 128, 2, 2, EPI_F32_LN, 4>(a, s, 1, ln);
  }
  if (ln->lparts < 1 || ln->lparts > 8 || ln->lparts * kLnPartCols != a.K || !ln->lpart || !ln->lcs ||
      !ln->mean_out || (epi == EPI_STORE_LN && a.N <= 1024))
    return hipErrorInvalidValue;
  if (epi == EPI_STORE_LN) {
    if (medium) return launch_fold_cfg<T, 128, 128, 64, 3, 3, EPI_STORE_LN>(a, *ln, s);
    return launch_fold_cfg<T, 256, 128, 64, 3, 2, EPI_STORE_LN>(a, *ln, s);
  }
  if (a.M <= 8192) return launch_fold_cfg<T, 128, 128, 64, 3, 3, EPI_GEGLU_LN>(a, *ln, s);
  return launch_fold_cfg<T, 256, 128, 64, 3, 2, EPI_GEGLU_LN>(a, *ln, s);
}

template <class T>
hipError_t launch_gemm16(int epi, const GemmArgs &a, hipStream_t s, const LnFold *ln) {
  if (epi >= EPI_F32_LN) return launch_gemm_fold<T>(epi, a, ln, s);
  const bool small = a.M <= 1024;
  {
    if (small) return launch_cfg<T, 64, 128, 128, 4, 1>(epi, a, s);
    const bool medium = a.M <= 4096;
    if (epi == EPI_F32 && a.N % 192 == 0) {
      // 768-wide outputs in 192-column tiles: 3,840 rows make 240 tiles of
      // 64 x 192 for 256 CUs where 64 x 128 made 360 (dX GEMM N = 768,
      // K = 2304: 30.6 -> 24.2 us isolated; Wo 16.2 -> 12.7 us). Above 4096
      // rows, 256 x 192 tiles of 8 waves (64 x 96 each) at one workgroup per
      // CU (112 KB of LDS: 2 stages of 64 K elements). These GEMMs are bound
      // by the vector memory path (TA/TD), not by HBM or the matrix cores:
      // every byte staged into LDS and every fp32 residual byte passes it.
      // Per output element the main loop stages (1/BN + 1/BM) K operand
      // elements: 0.0091 K for 256 x 192 against 0.0104 K for 128 x 384
      // (-12.5%), and the residual read + write is the same. Alternating
      // runs on one box, cfg3: Wo 80.7 -> 75.7 us, MlpWo 90.5 -> 83.8 us per
      // launch, forward 2.80 -> 2.82M tokens/s; TA busy 0.64 -> 0.38, TD
      // 0.77 -> 0.71 (128 x 384 tiles of 8 waves with 3 stages of 32 K
      // elements before; 128 x 192 at two workgroups per CU was 2-4% slower
      // still).
      if (medium) return launch_cfg_one<T, 64, 192, 128, 4, 1>(a, s);
      return launch_cfg_one<T, 256, 192, 128, 2, 2, EPI_F32, 4>(a, s);
    }
    // GeGLU backward (N = 1152) at medium M: 64 x 192 at two workgroups per
    // CU (3840 rows: 30.2 -> 25.8 us isolated). Training only (bf16).
    if constexpr (!std::is_same<T, f16>::value)
      if (epi == EPI_GEGLU_BWD && medium && a.N % 192 == 0)
        return launch_cfg_one<T, 64, 192, 64, 4, 2, EPI_GEGLU_BWD>(a, s);
    if (epi == EPI_F32 || (epi == EPI_STORE && a.N <= 1024 && a.M <= 16384)) {
      if (medium) return launch_cfg<T, 64, 128, 128, 4, 1>(epi, a, s);
      return launch_cfg<T, 128, 128, 64, 3, 3>(epi, a, s);
    }
    if (epi == EPI_GEGLU_BWD || (epi == EPI_STORE && medium) ||
        ((epi == EPI_GEGLU || epi == EPI_GEGLU_KEEP) && a.M <= 8192))
      return launch_cfg<T, 128, 128, 64, 3, 3>(epi, a, s);
    return launch_cfg<T, 256, 128, 64, 3, 2>(epi, a, s);
  }
}
