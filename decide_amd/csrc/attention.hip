// Fused masked multi-head attention (forward only).
//
// Replaces the reference's per-(sequence, head) attnFwd
// (internal/nn/forward.go:347-378): Sgemm1 Q.K^T, softmaxMasked
// (forward.go:382-409), Sgemm1 P.V; and its dense n x n uint8 masks
// (forward.go:152-176). Here nothing n x n is materialised:
//   * the mask is evaluated per element from each token's (option id,
//     position): allowed(i,j) = block(opt_i, opt_j) && (global || |pos_i-pos_j| <= W),
//     block(a,b) = (a == -1 && b == -1) || (a != -1 && (b == -1 || a == b));
//   * 32-token chunk summaries let a workgroup skip key tiles with no allowed
//     pair and drop the per-element test on tiles where every pair is allowed;
//   * softmax is the online (running max / running sum) form in fp32.
//
// Work decomposition: one workgroup = 4 waves = 128 queries of one
// (sequence, head); wave w owns queries q0+32w .. q0+32w+31, one per lane
// pair (lane l and l^32 share query l%32). Scores are computed transposed,
// S^T = K . Q^T, so that each lane holds 16 keys of ONE query per 32x32
// tile: the row max and row sum are in-register plus one exchange with the
// partner lane. The same register layout is directly the B operand of
// O^T = V^T . P^T (keys permuted consistently in both operands), so P never
// leaves registers. V is staged transposed in LDS for that product.
#include "common.hpp"

namespace {

constexpr int KTILE = 64;   // keys per tile
constexpr int D = 64;       // head dim

__device__ __forceinline__ int tile_class(const ChunkInfo &q, const ChunkInfo &k, int sliding, int W) {
  // 0: no allowed pair; 1: every pair allowed; 2: test per element.
  const bool qp = q.nprefix > 0, qo = q.nopt > 0, kp = k.nprefix > 0, ko = k.nopt > 0;
  const bool any_block = (kp && (qp || qo)) || (qo && ko && !(q.omax < k.omin || k.omax < q.omin));
  if (!any_block) return 0;
  if (sliding && (q.pmin - k.pmax > W || k.pmin - q.pmax > W)) return 0;
  const bool block_full = !ko || (!qp && q.omin == q.omax && k.omin == k.omax && q.omin == k.omin);
  const bool win_full = !sliding || max(q.pmax - k.pmin, k.pmax - q.pmin) <= W;
  return (block_full && win_full && k.len == 32) ? 1 : 2;
}

__device__ __forceinline__ int combine(int a, int b) {
  if (a == 0 && b == 0) return 0;
  if (a == 1 && b == 1) return 1;
  return 2;
}

template <class T>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  constexpr int ROWK = D * sizeof(T) + 16;       // K tile row bytes (key-major)
  constexpr int ROWV = KTILE * sizeof(T) + 16;   // V^T tile row bytes (d-major)
  __shared__ __attribute__((aligned(16))) char sK[KTILE * ROWK];
  __shared__ __attribute__((aligned(16))) char sV[D * ROWV];
  __shared__ __attribute__((aligned(16))) int sInfo[KTILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lh = lane >> 5;
  const int4 wk = a.work[blockIdx.x];
  const int s = wk.x, q0 = wk.y, head = blockIdx.y;
  const int n = a.seq_len[s], base = a.seq_off[s], cbase = a.chunk_off[s];
  const int nch = (n + 31) / 32;
  const int H = a.H, ld = 3 * H;
  const T *qkv = (const T *)a.qkv;

  ChunkInfo empty = {0, 0, 1, 0, 0, 0, 0, 0};
  ChunkInfo qc[4];
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const int c = q0 / 32 + w;
    qc[w] = c < nch ? a.chunks[cbase + c] : empty;
  }

  // This lane's query.
  const int q = q0 + wave * 32 + lr;
  const bool qvalid = q < n;
  const int qq = qvalid ? q : n - 1;
  const int qinfo = a.kinfo[base + qq];
  const int qopt = (qinfo >> 16) - 1, qpos = qinfo & 0xffff;

  // Q^T operand fragments (B operand: column = query, k = head dim).
  constexpr int NKS = D / MF::KSTEP;
  frag qf[NKS];
  {
    const T *qrow = qkv + (size_t)(base + qq) * ld + head * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) qf[ks] = *(const frag *)(qrow + ks * MF::KSTEP + lh * MF::SLOTS);
  }

  f32x16 ot[2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) ot[i][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  const int nkt = (n + KTILE - 1) / KTILE;
  for (int kt = 0; kt < nkt; kt++) {
    const int k0 = kt * KTILE;
    const ChunkInfo kc0 = a.chunks[cbase + 2 * kt];
    const ChunkInfo kc1 = (2 * kt + 1 < nch) ? a.chunks[cbase + 2 * kt + 1] : empty;
    int cls[4];
    bool need = false;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      cls[w] = combine(tile_class(qc[w], kc0, a.sliding, a.half_window),
                       tile_class(qc[w], kc1, a.sliding, a.half_window));
      need |= cls[w] != 0;
    }
    if (!need) continue;  // uniform over the workgroup

    __syncthreads();  // previous tile fully consumed
    // Stage K (key-major) and V^T (d-major) for keys k0..k0+63; zero beyond n.
    constexpr int CPR = D * sizeof(T) / 16;  // 16-byte chunks per key row
    constexpr int EPC = 16 / sizeof(T);      // elements per chunk
#pragma unroll
    for (int c = tid; c < KTILE * CPR; c += 256) {
      const int key = c / CPR, cc = c % CPR;
      uint4 kv = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
      if (k0 + key < n) {
        const T *row = qkv + (size_t)(base + k0 + key) * ld + head * D + cc * EPC;
        kv = *(const uint4 *)(row + H);
        vv = *(const uint4 *)(row + 2 * H);
      }
      *(uint4 *)(sK + key * ROWK + cc * 16) = kv;
      const T *ve = (const T *)&vv;
#pragma unroll
      for (int e = 0; e < EPC; e++) *(T *)(sV + (cc * EPC + e) * ROWV + key * sizeof(T)) = ve[e];
    }
    if (tid < KTILE) sInfo[tid] = (k0 + tid < n) ? a.kinfo[base + k0 + tid] : 0;
    __syncthreads();

    const int mycls = cls[wave];
    if (mycls == 0) continue;

    // S^T = K . Q^T for 64 keys x 32 queries (two 32x32 tiles).
    f32x16 st[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) st[i][e] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const int kof = (ks * MF::KSTEP + lh * MF::SLOTS) * (int)sizeof(T);
#pragma unroll
      for (int i = 0; i < 2; i++) {
        frag kf = *(const frag *)(sK + (i * 32 + lr) * ROWK + kof);
        st[i] = MF::mma(kf, qf[ks], st[i]);
      }
    }

    // Scale, mask, running max.
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int kl = i * 32 + 8 * g + 4 * lh;  // 4 consecutive keys kl..kl+3
        int4 inf4 = {0, 0, 0, 0};
        if (mycls == 2) inf4 = *(const int4 *)(sInfo + kl);
        const int *inf = (const int *)&inf4;
#pragma unroll
        for (int u = 0; u < 4; u++) {
          float x = st[i][4 * g + u] * a.scale_log2;
          if (mycls == 2) {
            const int ko = (inf[u] >> 16) - 1, kp = inf[u] & 0xffff;
            bool ok = k0 + kl + u < n;
            ok = ok && (qopt == -1 ? ko == -1 : (ko == -1 || ko == qopt));
            ok = ok && (!a.sliding || abs(qpos - kp) <= a.half_window);
            x = ok ? x : -INFINITY;
          }
          st[i][4 * g + u] = x;
          mx = fmaxf(mx, x);
        }
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float p = exp2f(st[i][e] - m_use);
        st[i][e] = p;
        psum += p;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) ot[i][e] *= alpha;

    // O^T += V^T . P^T. k step ks covers accumulator registers
    // [ks*SLOTS, ks*SLOTS + SLOTS) of the flattened S^T tiles; accumulator r
    // of tile i on lane half lh is key 32*i + 8*((r%16)/4) + 4*lh + r%4.
    constexpr int NPV = KTILE / MF::KSTEP;
#pragma unroll
    for (int ks = 0; ks < NPV; ks++) {
      frag pf;
      if constexpr (sizeof(T) == 2) {
        const int ti = ks >> 1, r0 = (ks & 1) * 8;
#pragma unroll
        for (int u = 0; u < 8; u++) pf[u] = (bf16)st[ti][r0 + u];
      } else {
        pf = st[ks >> 4][ks & 15];
      }
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const char *vrow = sV + (i * 32 + lr) * ROWV;
        frag vf;
        if constexpr (sizeof(T) == 2) {
          const int kb = 32 * (ks >> 1) + 16 * (ks & 1) + 4 * lh;
          bf16x4 lo = *(const bf16x4 *)(vrow + kb * 2);
          bf16x4 hi = *(const bf16x4 *)(vrow + (kb + 8) * 2);
          vf = (bf16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
          const int r = ks & 15;
          const int key = 32 * (ks >> 4) + 8 * (r >> 2) + 4 * lh + (r & 3);
          vf = *(const float *)(vrow + key * 4);
        }
        ot[i] = MF::mma(vf, pf, ot[i]);
      }
    }
  }

  // Normalise and store ctx[token][head*64 + d].
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (qvalid) {
    T *out = (T *)a.ctx + (size_t)(base + q) * H + head * D;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int d0 = i * 32 + 8 * g + 4 * lh;
#pragma unroll
        for (int u = 0; u < 4; u++) out[d0 + u] = to_elem<T>(ot[i][4 * g + u] * inv);
      }
  }
}

__global__ void token_info_kernel(const int *pos, const int *opt, int *kinfo, int T) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < T) kinfo[t] = (((opt ? opt[t] : -1) + 1) << 16) | (pos[t] & 0xffff);
}

__global__ void chunk_summary_kernel(const int *kinfo, const int4 *desc, ChunkInfo *out, int nchunks) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= nchunks) return;
  const int4 d = desc[c];  // (first token, length)
  ChunkInfo ci = {0x7fffffff, -0x7fffffff, 0x7fffffff, -1, 0, 0, d.y, 0};
  for (int i = 0; i < d.y; i++) {
    const int v = kinfo[d.x + i];
    const int o = (v >> 16) - 1, p = v & 0xffff;
    ci.pmin = min(ci.pmin, p);
    ci.pmax = max(ci.pmax, p);
    if (o < 0) {
      ci.nprefix++;
    } else {
      ci.nopt++;
      ci.omin = min(ci.omin, o);
      ci.omax = max(ci.omax, o);
    }
  }
  out[c] = ci;
}

}  // namespace

hipError_t launch_attention(int precision, const AttnArgs &a, hipStream_t s) {
  if (a.nwork <= 0) return hipSuccess;
  dim3 grid(a.nwork, a.heads), block(256);
  if (precision == 1)
    hipLaunchKernelGGL(attention_kernel<bf16>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(attention_kernel<float>, grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_token_info(const int *pos, const int *opt, int *kinfo, int T, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(token_info_kernel, dim3((T + 255) / 256), dim3(256), 0, s, pos, opt, kinfo, T);
  return hipGetLastError();
}

hipError_t launch_chunk_summary(const int *kinfo, const int4 *desc, ChunkInfo *out, int nchunks, hipStream_t s) {
  if (nchunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(chunk_summary_kernel, dim3((nchunks + 127) / 128), dim3(128), 0, s, kinfo, desc, out, nchunks);
  return hipGetLastError();
}
