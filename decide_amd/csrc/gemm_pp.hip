// Large-M bf16 projection GEMMs on a persistent, ping-pong scheduled kernel:
// C[M x N] = A[M x K] . B[N x K]^T, fp32 accumulate, with the forward's
// fused epilogues (EPI_STORE: the qkv projection, forward.go:296; EPI_GEGLU:
// the Wi projection + GeGLU, forward.go:326-336). Same arithmetic as
// gemm_nt_kernel (k steps in increasing order into one fp32 accumulator per
// element, B as the MFMA's first operand), so the outputs are identical.
//
// Schedule (gfx950, one 512-thread workgroup per CU, 256 x 192 output tiles):
//   * K is staged 32 elements (64-byte LDS rows) at a time, filled by direct
//     global->LDS loads. Waves 0-3 (group 0) load the A rows of each stage
//     into an NSA-slot ring, waves 4-7 (group 1) the B rows into an NSB-slot
//     ring. vmcnt counts each wave's own loads in issue order, so the two
//     streams run at their own depths: A (activations, streamed from HBM)
//     NSA-1 stages ahead, B (weights, resident in L2) NSB-1 stages ahead.
//   * Each SIMD holds one wave of each group. The groups alternate between a
//     memory phase (read this stage's MFMA operands from LDS into registers,
//     issue the DMA of a later stage) and a compute phase (the stage's
//     12 MFMAs from registers); group 1 runs one phase behind group 0, and
//     every phase ends at a workgroup barrier. So while one wave of a SIMD
//     issues MFMAs back to back, the other does its memory work, and the
//     matrix core never waits for an LDS read or a DMA issue.
//   * The workgroup walks its tiles as one stream of stages: the ring keeps
//     loading the next tile's first stages while the current tile's epilogue
//     runs. Epilogues store straight from registers (a lane swap pairs
//     the 8-byte column runs of lanes l and l+32 into 16-byte stores), so LDS
//     holds only the ring.
//   * Tiles are ordered per XCD (workgroup b runs on XCD b % 8): each XCD
//     owns a contiguous range of M panels and sweeps them N group by N group.
#include "common.hpp"

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gbl_void;

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// s_waitcnt lgkmcnt(0).
__device__ __forceinline__ void lgkm_wait0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// A workgroup barrier that the compiler schedules nothing across.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

constexpr int BM = 256, BN = 192;
constexpr int RB = 64;                   // bytes per LDS row per stage
constexpr int KT = RB / 2;               // K elements per stage
constexpr int ASLOT = BM * RB;           // A ring slot: 16 KB
constexpr int BSLOT = BN * RB;           // B ring slot: 12 KB
constexpr int LA = BM / 64, LB = BN / 64;  // 1 KB DMA instructions per wave and stage: group 0 (A), group 1 (B)
constexpr int TM = 2, TN = 3;            // 32 x 32 MFMA tiles per wave: 64 rows x 96 columns
#ifndef PP_NSA
#define PP_NSA 7  // A ring slots
#endif
#ifndef PP_NSB
#define PP_NSB 3  // B ring slots
#endif

// 16-byte chunk swizzle of a 64-byte LDS row: the 16 rows a quarter-wave
// reads at one logical chunk fall in distinct bank groups.
__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  bf16x2_t v = {(bf16)lo, (bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Lanes l < 32 keep x and receive y of lane l + 32 in its place; lanes
// l >= 32 receive x of lane l - 32 in place of theirs and keep y
// (v_permlane32_swap: x[32..63] <-> y[0..31]).
__device__ __forceinline__ void swap32(uint32_t &x, uint32_t &y) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  x = r[0];
  y = r[1];
}

// Stores issued per wave by one tile's epilogue (they count in vmcnt).
template <int EPI>
constexpr int epi_stores() {
  return EPI == EPI_STORE ? 2 * TM * TN : TM * TN;
}

template <int EPI, int NSA, int NSB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_pp_kernel(GemmArgs g) {
  static_assert(EPI == EPI_STORE || EPI == EPI_GEGLU, "epilogues of the ping-pong kernel");
  static_assert(NSA >= 3 && NSB >= 3 && LA * (NSA - 2) + epi_stores<EPI>() < 64 &&
                    LB * (NSB - 2) + epi_stores<EPI>() < 64, "ring depths");
  __shared__ __attribute__((aligned(1024))) char smem[NSA * ASLOT + NSB * BSLOT];
  char *const bring = smem + NSA * ASLOT;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wig = wave & 3;
  const int NS = grp ? NSB : NSA;  // ring depth of this wave's own DMA stream
  const int lr = lane & 31, lh = lane >> 5;
  const int rw = 128 * grp + 64 * (wig >> 1);  // wave tile origin inside the block tile
  const int cw = 96 * (wig & 1);

  // ---- this workgroup's tiles
  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = g.N / BN;
  const int nwg = gridDim.x, wg = blockIdx.x;
  const int gn = g.ngroups > 0 && tiles_n % g.ngroups == 0 ? tiles_n / g.ngroups : tiles_n;
  const bool xcd = tiles_m % 8 == 0 && nwg % 8 == 0;
  int count;
  if (xcd) {
    const int per = (tiles_m / 8) * tiles_n, c = wg / 8, w8 = nwg / 8;
    count = c < per ? (per - c + w8 - 1) / w8 : 0;
  } else {
    const int total = tiles_m * tiles_n;
    count = wg < total ? (total - wg + nwg - 1) / nwg : 0;
  }
  if (count == 0) return;
  auto tile = [&](int t, int &m0, int &n0) {
    int tm, tn;
    if (xcd) {
      const int P = tiles_m / 8, x = wg % 8, j = wg / 8 + t * (nwg / 8);
      const int grp_n = j / (P * gn), rem = j % (P * gn);
      tm = x * P + rem / gn;
      tn = grp_n * gn + rem % gn;
    } else {
      const int j = wg + t * nwg;
      tm = j / tiles_n;
      tn = j % tiles_n;
    }
    m0 = tm * BM;
    n0 = tn * BN;
  };

  // ---- DMA stream: the stage after the last one of this workgroup reloads
  // the last tile's data into a slot nobody reads again, so every stage
  // issues the same number of loads and the vmcnt arithmetic is exact.
  const char *src[LA];
  auto set_src = [&](int m0, int n0) {
#pragma unroll
    for (int i = 0; i < LA; i++) {
      const int r = 16 * (wig + 4 * i) + (lane >> 2);  // tile row written by this lane
      const int c = (lane & 3) ^ swz(r);               // logical 16-byte chunk it holds
      if (grp == 0) {
        src[i] = (const char *)g.A + ((size_t)min(m0 + r, g.M - 1) * g.lda) * 2 + c * 16;
      } else if (i < LB) {
        int wrow = n0 + r;
        if constexpr (EPI == EPI_GEGLU) {
          // B row r of the tile: 32-row MFMA tile j = r / 32 holds the value
          // rows (t < 16) then the gate rows (t >= 16) of GeGLU features
          // f0 + 16 j + t % 16. The weights are stored interleaved in 64-row
          // groups (32 value rows, then the matching 32 gate rows).
          const int t = r & 31, f = n0 / 2 + 16 * (r >> 5) + (t & 15);
          wrow = 64 * (f >> 5) + (f & 31) + (t >= 16 ? 32 : 0);
        }
        src[i] = (const char *)g.B + ((size_t)wrow * g.ldb) * 2 + c * 16;
      }
    }
  };
  const int nk = g.K / KT;
  const int nq = count * nk;  // stages of this workgroup
  int d_t = 0, d_k = 0;       // tile and k stage of the next DMA
  {
    int m0, n0;
    tile(0, m0, n0);
    set_src(m0, n0);
  }
  auto issue = [&](int slot) {
    char *dst = (grp ? bring + slot * BSLOT : smem + slot * ASLOT) + wig * 1024;
    const size_t kb = (size_t)d_k * RB;
#pragma unroll
    for (int i = 0; i < LA; i++)
      if (grp == 0 || i < LB)
        __builtin_amdgcn_global_load_lds((gbl_void *)(src[i] + kb), (lds_void *)(dst + i * 4096), 16, 0, 0);
    if (++d_k == nk) {
      d_k = 0;
      d_t++;
      int m0, n0;
      tile(min(d_t, count - 1), m0, n0);
      set_src(m0, n0);
    }
  };

  bf16x8 fa[2][TM], fb[2][TN];
  auto read_frags = [&](int sla, int slb) {
    const char *sa = smem + sla * ASLOT, *sb = bring + slb * BSLOT;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const int chunk = 2 * ks + lh;
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = rw + 32 * i + lr;
        fa[ks][i] = *(const bf16x8 *)(sa + r * RB + ((chunk ^ swz(r)) << 4));
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int r = cw + 32 * j + lr;
        fb[ks][j] = *(const bf16x8 *)(sb + r * RB + ((chunk ^ swz(r)) << 4));
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};

  // Waits until this wave's own DMA of the stage after the current one has
  // landed: NS-2 later stages of its loads may still be in flight, plus the
  // stores of an epilogue issued after that DMA.
  int last_epi = -NSA - NSB;
  auto dma_wait = [&](int q) {
    const bool stores = last_epi >= q + 2 - NS && last_epi <= q - 1;
    if (grp == 0) {
      if (stores) vm_wait<LA * (NSA - 2) + epi_stores<EPI>()>();
      else vm_wait<LA * (NSA - 2)>();
    } else {
      if (stores) vm_wait<LB * (NSB - 2) + epi_stores<EPI>()>();
      else vm_wait<LB * (NSB - 2)>();
    }
  };

  int cm0, cn0;  // tile whose accumulators are being built
  tile(0, cm0, cn0);

  auto epilogue = [&]() {
    const size_t ldc = g.ldc;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int row = cm0 + rw + 32 * i + lr;  // this lane's token row
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const f32x16 &a = acc[i][j];
        // Lane (lr, lh) holds columns 8q + 4lh + (0..3) of the 32-column
        // MFMA tile j for q = 0..3.
        if constexpr (EPI == EPI_STORE) {
          uint32_t p[4][2];
#pragma unroll
          for (int q = 0; q < 4; q++) {
            p[q][0] = pack_bf16(a[4 * q], a[4 * q + 1]);
            p[q][1] = pack_bf16(a[4 * q + 2], a[4 * q + 3]);
          }
          // After the swaps lane (lr, 0) holds columns 0-7 and 16-23, lane
          // (lr, 1) columns 8-15 and 24-31.
          swap32(p[0][0], p[1][0]);
          swap32(p[0][1], p[1][1]);
          swap32(p[2][0], p[3][0]);
          swap32(p[2][1], p[3][1]);
          if (row < g.M) {
            bf16 *o = (bf16 *)g.C + row * ldc + cn0 + cw + 32 * j + 8 * lh;
            *(uint4 *)o = make_uint4(p[0][0], p[0][1], p[1][0], p[1][1]);
            *(uint4 *)(o + 16) = make_uint4(p[2][0], p[2][1], p[3][0], p[3][1]);
          }
        } else {
          // Columns 0-15 of the MFMA tile are values, 16-31 the gates of the
          // same 16 features: accumulator e pairs with e + 8.
          uint32_t p[2][2];
#pragma unroll
          for (int q = 0; q < 2; q++) {
            float o4[4];
#pragma unroll
            for (int t = 0; t < 4; t++) o4[t] = gelu_erf<bf16>(a[4 * q + t]) * a[8 + 4 * q + t];
            p[q][0] = pack_bf16(o4[0], o4[1]);
            p[q][1] = pack_bf16(o4[2], o4[3]);
          }
          // After the swaps lane (lr, 0) holds features 0-7, lane (lr, 1) 8-15.
          swap32(p[0][0], p[1][0]);
          swap32(p[0][1], p[1][1]);
          if (row < g.M) {
            bf16 *o = (bf16 *)g.C + row * ldc + (cn0 + cw) / 2 + 16 * j + 8 * lh;
            *(uint4 *)o = make_uint4(p[0][0], p[0][1], p[1][0], p[1][1]);
          }
        }
      }
    }
  };

  // ---- prologue: NS-1 stages of each stream in flight, the first one
  // visible to all waves.
  for (int s = 0; s < NS - 1; s++) issue(s);
  // Ring slots: of stage q in A and B, and of this wave's next DMA.
  int sla = 0, slb = 0, sld = NS - 1;
  if (grp == 0) vm_wait<LA * (NSA - 2)>();
  else vm_wait<LB * (NSB - 2)>();
  phase_barrier();
  if (grp == 1) phase_barrier();  // group 1 runs one phase behind

  for (int q = 0; q < nq; q++) {
    // memory phase: this stage's operands, the DMA of stage q + NS - 1 of
    // this wave's stream into the slot of stage q - 1 (both groups finished
    // reading it before the previous barrier)
    read_frags(sla, slb);
    issue(sld);
    sla = sla + 1 == NSA ? 0 : sla + 1;
    slb = slb + 1 == NSB ? 0 : slb + 1;
    sld = sld + 1 == NS ? 0 : sld + 1;
    lgkm_wait0();
    if (grp == 1) dma_wait(q);  // group 0 reads stage q + 1 right after the next barrier
    phase_barrier();
    // compute phase
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = Mfma<bf16>::mma(fb[ks][j], fa[ks][i], acc[i][j]);
    if (grp == 0) dma_wait(q);
    if (q % nk == nk - 1) {
      epilogue();
      last_epi = q;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};
      tile(q / nk + 1 < count ? q / nk + 1 : q / nk, cm0, cn0);
    }
    phase_barrier();
  }
  if (grp == 0) phase_barrier();
  vm_wait<0>();  // no LDS DMA may land after the workgroup ends
}

// Compute units of the current device (the persistent grid: one workgroup per CU).
int cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || n <= 0)
    return 256;
  return n;
}

template <int EPI>
hipError_t launch_pp(const GemmArgs &a, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
  const int cus = cu_count();
  const int grid = tiles < cus ? tiles : cus;
  hipLaunchKernelGGL((gemm_pp_kernel<EPI, PP_NSA, PP_NSB>), dim3(grid), dim3(512), 0, s, a);
  return hipGetLastError();
}

}  // namespace

bool gemm_pp_ok(int precision, int epi, const GemmArgs &a) {
  return precision == 1 && (epi == EPI_STORE || epi == EPI_GEGLU) && a.M >= 8192 && a.N % BN == 0 && a.K % KT == 0 &&
         a.K >= KT;
}

hipError_t launch_gemm_pp(int epi, const GemmArgs &a0, hipStream_t s) {
  GemmArgs a = a0;
  // N groups per XCD sweep: keep the group's slice of B within about 2 MB of L2.
  const int tiles_n = a.N / BN;
  const size_t b_bytes = (size_t)a.N * a.K * 2;
  int groups = 1;
  while (b_bytes / groups > (2u << 20) && groups < tiles_n) {
    groups++;
    while (tiles_n % groups) groups++;
  }
  a.ngroups = groups;
  return epi == EPI_STORE ? launch_pp<EPI_STORE>(a, s) : launch_pp<EPI_GEGLU>(a, s);
}
