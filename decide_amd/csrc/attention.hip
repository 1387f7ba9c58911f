// Fused masked multi-head attention (forward only), with RoPE applied to q
// and k on the way in.
//
// Replaces the reference's per-(sequence, head) attnFwd
// (internal/nn/forward.go:347-378): Sgemm1 Q.K^T, softmaxMasked
// (forward.go:382-409), Sgemm1 P.V; its dense n x n uint8 masks
// (forward.go:152-176); and applyRope on q and k (internal/nn/ops.go:155-175,
// forward.go:297-301). Nothing n x n is materialised:
//   * the mask is evaluated per element from each token's (option id,
//     position): allowed(i,j) = block(opt_i, opt_j) && (global || |pos_i-pos_j| <= W),
//     block(a,b) = (a == -1 && b == -1) || (a != -1 && (b == -1 || a == b));
//   * 32-token chunk summaries classify each (32-query chunk, 32-key half
//     tile) pair as empty, full or mixed: a wave skips the MFMAs, softmax and
//     P.V of empty halves, and the per-element test of full ones;
//   * softmax is the online (running max / running sum) form in fp32.
//
// Work decomposition: one workgroup = ATTN_WAVES (4) waves = 128 queries of one
// (sequence, head); wave w owns queries q0+32w .. q0+32w+31, one per lane
// pair (lane l and l^32 share query l%32). Scores are computed transposed,
// S^T = K . Q^T, so that each lane holds 16 keys of ONE query per 32x32
// tile: the row max and row sum are in-register plus one exchange with the
// partner lane. The same register layout is directly the B operand of
// O^T = V^T . P^T (keys permuted consistently in both operands), so P never
// leaves registers.
//
// Key tiles (64 keys) are visited in a list of the tiles some wave needs; the
// next tile's K, V and RoPE factors are loaded into registers while the
// current one is computed. K is rotated and stored key-major; V is stored
// transposed (d-major) with two keys packed per 32-bit word so each wave's
// LDS writes are contiguous.
#include "common.hpp"

namespace {

constexpr int KTILE = 64;   // keys per tile
constexpr int D = 64;       // head dim
static_assert(ATTN_MAXKT * KTILE == 8192, "tile codes cover sequences up to 8192 tokens");

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

// 16-bit types (bf16, fp16): each of a thread's R items is one (key, 16-byte
// chunk pair (c, c+4)) of K with its RoPE factors and one (key pair, 8-d
// group) of V; the workgroup's threads cover the tile's 256 K items and 256
// V items.
template <class T, int R>
struct Staging {
  uint4 k_lo[R], k_hi[R], v0[R], v1[R];
  float4 c_lo[R], c_hi[R], s_lo[R], s_hi[R];
  uint32_t valid;  // bit j: K item j's key, 8+j / 16+j: V item j's two keys exist (zeroed at the store)
  int info;
};

// fp32: 512 (key, 16-byte chunk pair) K items and 1024 (key, 4-d group) V
// items per tile.
template <int R>
struct Staging<float, R> {
  uint4 k_lo[2 * R], k_hi[2 * R], v[4 * R];
  float4 c[2 * R], s[2 * R];
  uint32_t valid;  // bit j: K item j's key, 8+j: V item j's key exists (zeroed at the store)
  int info;
};

// ok ? v : 0, per component (a select of the whole vector can end up as an
// indexed scratch access).
__device__ __forceinline__ uint4 keep_if(bool ok, uint4 v) {
  return make_uint4(ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u);
}

// The per-token info (((opt+1) << 16) | pos) a thread needs to stage a key
// tile: the positions of its K items' keys (they index the RoPE tables) and,
// for the first 64 threads, key k0 + tid (the tile's mask info). Loaded one
// tile ahead of the K / V / RoPE loads, so that the position-dependent table
// loads issue at once instead of waiting for a dependent load every tile.
template <class T, int R>
struct KeyInfo {
  static constexpr int KI = sizeof(T) == 2 ? R : 2 * R;  // K items per thread
  int pk[KI];
  int pi;
};

template <class T, int R>
__device__ __forceinline__ void key_info_load(KeyInfo<T, R> &f, const int *kinfo, int base, int n, int k0, int tid) {
  constexpr int NT = 256 / R, SH = sizeof(T) == 2 ? 2 : 3;  // K item it -> key it >> SH
#pragma unroll
  for (int j = 0; j < KeyInfo<T, R>::KI; j++) {
    const int key = (tid + NT * j) >> SH;
    f.pk[j] = kinfo[base + min(k0 + key, n - 1)];
  }
  // Key k0 + (tid % 64)'s info, clamped to the last key; stage_load replaces
  // it for keys past the end. No select here: a register write after this
  // load would have to wait for every load still in flight to that register,
  // and in the tile loop that wait also covered the tile just issued.
  f.pi = kinfo[base + min(k0 + (tid & (KTILE - 1)), n - 1)];
}

// Loads one key tile (keys k0 .. k0+63) into registers; NT threads, R = 256/NT.
template <class T, int R>
__device__ __forceinline__ void stage_load(Staging<T, R> &st, const T *qkv, int ld, int H, int head, int base, int n,
                                           int k0, const float *cos_t, const float *sin_t,
                                           const KeyInfo<T, R> &ki, int tid) {
  constexpr int NT = 256 / R;
  // Keys past the sequence end read the last key's row (in bounds) and are
  // zeroed; their RoPE factors are whatever that row has (results unused).
  // The RoPE tables are indexed by position (low 16 bits of the key's info).
  // The loaded values are not touched here (a select on them would wait for
  // the loads): keys past the sequence end are zeroed by stage_store.
  st.valid = 0;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int j = 0; j < R; j++) {  // K: key = it / 4, chunk c = it % 4 (elements 8c..8c+7 and 32+8c..)
      const int it = tid + NT * j, key = it >> 2, c = it & 3;
      st.valid |= (k0 + key < n ? 1u : 0u) << j;
      // Token indices are non-negative: zero-extended, the row offset is one
      // 32 x 32 -> 64-bit multiply-add.
      const size_t tok = (unsigned)(base + min(k0 + key, n - 1));
      const T *row = qkv + tok * (unsigned)ld + H + head * D;
      st.k_lo[j] = *(const uint4 *)(row + 8 * c);
      st.k_hi[j] = *(const uint4 *)(row + 32 + 8 * c);
      const size_t p = (size_t)(ki.pk[j] & 0xffff);
      st.c_lo[j] = *(const float4 *)(cos_t + p * 32 + 8 * c);
      st.c_hi[j] = *(const float4 *)(cos_t + p * 32 + 8 * c + 4);
      st.s_lo[j] = *(const float4 *)(sin_t + p * 32 + 8 * c);
      st.s_hi[j] = *(const float4 *)(sin_t + p * 32 + 8 * c + 4);
    }
#pragma unroll
    for (int j = 0; j < R; j++) {  // V: key pair p = it % 32, d group g = it / 32
      const int it = tid + NT * j, p = it & 31, g = it >> 5;
      const int k = k0 + 2 * p;
      st.v0[j] = *(const uint4 *)(qkv + (size_t)(unsigned)(base + min(k, n - 1)) * (unsigned)ld + 2 * H + head * D + 8 * g);
      st.v1[j] = *(const uint4 *)(qkv + (size_t)(unsigned)(base + min(k + 1, n - 1)) * (unsigned)ld + 2 * H + head * D +
                                  8 * g);
      st.valid |= ((k < n ? 1u : 0u) << (8 + j)) | ((k + 1 < n ? 1u : 0u) << (16 + j));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2 * R; j++) {  // K: (key, chunk c in 0..7) = item tid + NT j
      const int it = tid + NT * j, key = it >> 3, c = it & 7;
      st.valid |= (k0 + key < n ? 1u : 0u) << j;
      const size_t tok = (size_t)(base + min(k0 + key, n - 1));
      const T *row = qkv + tok * ld + H + head * D;
      st.k_lo[j] = *(const uint4 *)(row + 4 * c);
      st.k_hi[j] = *(const uint4 *)(row + 32 + 4 * c);
      const size_t p = (size_t)(ki.pk[j] & 0xffff);
      st.c[j] = *(const float4 *)(cos_t + p * 32 + 4 * c);
      st.s[j] = *(const float4 *)(sin_t + p * 32 + 4 * c);
    }
#pragma unroll
    for (int j = 0; j < 4 * R; j++) {  // V: key = it % 64, d group g = it / 64
      const int it = tid + NT * j, key = it & 63, g = it >> 6;
      st.v[j] = *(const uint4 *)(qkv + (size_t)(base + min(k0 + key, n - 1)) * ld + 2 * H + head * D + 4 * g);
      st.valid |= (k0 + key < n ? 1u : 0u) << (8 + j);
    }
  }
  // Keys past the sequence end get option field 0xffff (option id -2, which
  // neither the prefix (-1) nor any query's own option matches).
  st.info = k0 + tid < n ? ki.pi : (int)0xffff0000u;
}

// RoPE of one (a, b) pair, unfused like applyRope (ops.go:169-170).
__device__ __forceinline__ void rope1(float &a, float &b, float c, float s) {
#pragma clang fp contract(off)
  const float x = a * c - b * s;
  const float y = b * c + a * s;
  a = x;
  b = y;
}

template <class T, int R>
__device__ __forceinline__ void stage_store(const Staging<T, R> &st, char *sK, char *sV, int *sKo, int *sKw,
                                            int half_window, int tid, int ROWK, int ROWV) {
  constexpr int NT = 256 / R;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int it = tid + NT * j, key = it >> 2, c = it & 3;
      const bool ok = (st.valid >> j) & 1;
      const uint4 kl = keep_if(ok, st.k_lo[j]), kh = keep_if(ok, st.k_hi[j]);
      const uint32_t klo[4] = {kl.x, kl.y, kl.z, kl.w};
      const uint32_t khi[4] = {kh.x, kh.y, kh.z, kh.w};
      const float cs[8] = {st.c_lo[j].x, st.c_lo[j].y, st.c_lo[j].z, st.c_lo[j].w,
                           st.c_hi[j].x, st.c_hi[j].y, st.c_hi[j].z, st.c_hi[j].w};
      const float sn[8] = {st.s_lo[j].x, st.s_lo[j].y, st.s_lo[j].z, st.s_lo[j].w,
                           st.s_hi[j].x, st.s_hi[j].y, st.s_hi[j].z, st.s_hi[j].w};
      uint32_t po[4], ph[4];
#pragma unroll
      for (int w = 0; w < 4; w++) {
        float a0 = lo16<T>(klo[w]), a1 = hi16<T>(klo[w]), b0 = lo16<T>(khi[w]), b1 = hi16<T>(khi[w]);
        rope1(a0, b0, cs[2 * w], sn[2 * w]);
        rope1(a1, b1, cs[2 * w + 1], sn[2 * w + 1]);
        po[w] = pack16<T>(a0, a1);
        ph[w] = pack16<T>(b0, b1);
      }
      *(uint4 *)(sK + key * ROWK + 16 * c) = make_uint4(po[0], po[1], po[2], po[3]);
      *(uint4 *)(sK + key * ROWK + 64 + 16 * c) = make_uint4(ph[0], ph[1], ph[2], ph[3]);
    }
    // V^T: row d = 8g + e holds key pairs (2p, 2p+1), one per 32-bit word.
    // Within each 16-key group the 4-key runs are stored in the order
    // 0-3, 8-11, 4-7, 12-15: the eight keys one lane feeds to a P.V step
    // (runs 4lh.. and 8+4lh.., the S^T accumulator order) are then one
    // contiguous 16-byte read.
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int it = tid + NT * j, p = it & 31, g = it >> 5;
      const int lp = p & 7, q4 = lp >> 1;
      const int pw = (p & ~7) + ((((q4 & 1) << 1) | (q4 >> 1)) << 1) + (lp & 1);
      const uint4 v0 = keep_if((st.valid >> (8 + j)) & 1, st.v0[j]), v1 = keep_if((st.valid >> (16 + j)) & 1, st.v1[j]);
      const uint32_t va[4] = {v0.x, v0.y, v0.z, v0.w};
      const uint32_t vb[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int w = 0; w < 4; w++) {
        // Byte permutes: (va & 0xffff) | (vb << 16) and (va >> 16) | (vb & 0xffff0000).
        *(uint32_t *)(sV + (8 * g + 2 * w) * ROWV + 4 * pw) = __builtin_amdgcn_perm(vb[w], va[w], 0x05040100u);
        *(uint32_t *)(sV + (8 * g + 2 * w + 1) * ROWV + 4 * pw) = __builtin_amdgcn_perm(vb[w], va[w], 0x07060302u);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2 * R; j++) {
      const int it = tid + NT * j, key = it >> 3, c = it & 7;
      const bool ok = (st.valid >> j) & 1;
      const uint4 kl = keep_if(ok, st.k_lo[j]), kh = keep_if(ok, st.k_hi[j]);
      float4 lo = *(const float4 *)&kl, hi = *(const float4 *)&kh;
      const float4 cs = st.c[j], sn = st.s[j];
      rope1(lo.x, hi.x, cs.x, sn.x);
      rope1(lo.y, hi.y, cs.y, sn.y);
      rope1(lo.z, hi.z, cs.z, sn.z);
      rope1(lo.w, hi.w, cs.w, sn.w);
      *(float4 *)(sK + key * ROWK + 16 * c) = lo;
      *(float4 *)(sK + key * ROWK + 128 + 16 * c) = hi;
    }
#pragma unroll
    for (int j = 0; j < 4 * R; j++) {
      const int it = tid + NT * j, key = it & 63, g = it >> 6;
      const uint4 v = keep_if((st.valid >> (8 + j)) & 1, st.v[j]);
      *(uint32_t *)(sV + (4 * g + 0) * ROWV + 4 * key) = v.x;
      *(uint32_t *)(sV + (4 * g + 1) * ROWV + 4 * key) = v.y;
      *(uint32_t *)(sV + (4 * g + 2) * ROWV + 4 * key) = v.z;
      *(uint32_t *)(sV + (4 * g + 3) * ROWV + 4 * key) = v.w;
    }
  }
  // Each key's mask fields, decoded once: option id (-1 prefix, -2 past the
  // sequence end) and position + half window.
  if (tid < KTILE) {
    sKo[tid] = (st.info >> 16) - 1;
    sKw[tid] = (st.info & 0xffff) + half_window;
  }
}

// LOCAL: a sliding-window layer (the window test is compiled in).
// LIST: the queries are the option rows of a.items (row_items_kernel): Q
// read from a.q_rows and the output written at row r, every key tile tested
// per element.
// fp32 four-wave workgroups run at two waves per SIMD: at three they spilled
// 44-62 VGPRs (one 512-token fp32 forward 3.81 -> 3.52 ms without the spills).
template <class T, int QW, int QT, bool LOCAL, bool LIST = false>
__global__ __launch_bounds__(64 * QW)
__attribute__((amdgpu_waves_per_eu(sizeof(T) == 4 && QW == ATTN_WAVES ? 2 : QT == 1 ? 3 : 2))) void attention_kernel(
    AttnArgs a) {
  // R staging items per thread; with more than 4 waves only the first 256
  // threads stage. Each wave owns QT 32-query tiles.
  constexpr int NT = 64 * QW, R = QW >= 4 ? 1 : 4 / QW;
  static_assert(QW == 1 || QW == 2 || QW == 4 || QW == 8, "waves per workgroup");
  static_assert(QT * QW <= 8, "tile codes hold 8 query chunks");
  // Workgroups of fewer than ATTN_WAVES waves (fp32 batches of few work
  // items) take ATTN_WAVES / QW turns at one work item of ATTN_WAVES 32-query
  // chunks: part `sub` of the item computes chunks sub * QW .. sub * QW + QW - 1.
  constexpr int SUB = LIST ? 1 : ATTN_WAVES / QW;
  static_assert(SUB * QW == ATTN_WAVES || SUB == 1, "work item parts");
  static_assert(SUB == 1 || QT == 1, "parted work items have one query tile per wave");
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  constexpr int ROWK = D * sizeof(T) + 16;       // K tile row bytes (key-major)
  constexpr int ROWV = KTILE * sizeof(T) + 16;   // V^T tile row bytes (d-major)
  // 16-bit: two buffers, tile t is computed from one while tile t+1 is stored
  // into the other, with one barrier per tile. fp32 (the validation mode,
  // twice the bytes) keeps one buffer and a second barrier.
  constexpr int NBUF = sizeof(T) == 2 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) char sK[NBUF][KTILE * ROWK];
  __shared__ __attribute__((aligned(16))) char sV[NBUF][D * ROWV];
  // Per staged key: option id (-1 prefix, -2 past the sequence end) and
  // position + half window, the fields the per-element mask tests.
  __shared__ __attribute__((aligned(16))) int sKo[NBUF][KTILE];
  __shared__ __attribute__((aligned(16))) int sKw[NBUF][KTILE];
  // Per key tile: for each 32-query chunk c of the work item, the 2-bit class
  // of each 32-key half (bits 4c..4c+1 keys 0-31, 4c+2..4c+3 keys 32-63).
  __shared__ uint32_t sCode[ATTN_MAXKT];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  // Linear grid, XCD-aware: workgroup ids go round-robin over the 8 XCDs, so
  // XCD x gets the contiguous range [x*per, (x+1)*per) of the logical order
  // (work item, head) with the q blocks of one sequence and its 12 heads
  // adjacent: the K/V rows, RoPE factors and chunk summaries they share are
  // reused out of that XCD's L2.
  const int total = a.nwork * a.heads * SUB;
  const int bid = blockIdx.x;
  int logical = bid;
  if (total % 8 == 0) logical = (bid % 8) * (total / 8) + bid / 8;
  const int sub = logical % SUB;
  logical /= SUB;
  const int wi = logical / a.heads, head = logical % a.heads;
  const int wq = sub * QW + wave;  // this wave's chunk of the work item (QT query tiles each)
  int s, q0 = 0, slot0 = 0, cnt = 0, n, base;
  if constexpr (LIST) {
    if (wi >= *a.nitems) return;  // the grid is sized by an upper bound on the items
    const int4 it = a.items[wi];
    s = it.x, slot0 = it.y, cnt = it.z;
    n = a.seq_len[s], base = a.seq_off[s];
  } else {
    // (sequence, first query, offset, length): no dependent load for the
    // sequence's extent before the key info and staging loads.
    const int4 wk = a.work[wi];
    s = wk.x, q0 = wk.y, base = wk.z, n = wk.w;
  }
  const int H = a.H, ld = 3 * H;
  const T *qkv = (const T *)a.qkv;
  const int nkt = (n + KTILE - 1) / KTILE;

  // This work item's tile classes (computed once per forward and layer type
  // by tile_codes_kernel) and its first needed tile: the first tile's loads
  // are issued before the classes reach LDS.
  int kt;
  if constexpr (LIST) {
    // Class 2 (per element) for both halves of every tile, for the waves
    // that hold rows.
    uint32_t all = 0;
    for (int w = 0; w < QW * QT; w++)
      if (32 * w < cnt) all |= 0xAu << (4 * w);
    for (int k = tid; k < nkt; k += NT) sCode[k] = all;
    kt = 0;
  } else {
    const uint32_t *codes = a.codes + (size_t)wi * ATTN_MAXKT;
    for (int k = tid; k < nkt; k += NT) sCode[k] = codes[k];
    kt = a.first[wi];
  }
  Staging<T, R> st;
  KeyInfo<T, R> ki;
  const bool stager = tid < 256;
  if (kt < nkt && stager) {
    key_info_load<T, R>(ki, a.kinfo, base, n, kt * KTILE, tid);
    stage_load<T, R>(st, qkv, ld, H, head, base, n, kt * KTILE, a.cos_t, a.sin_t, ki, tid);
  }

  // This lane's queries (one per query tile), their RoPE factors and the
  // rotated Q^T operands (B operand: column = query, k = head dim).
  constexpr int NKS = D / MF::KSTEP;
  frag qf[QT][NKS];
  int qopt[QT], qpos[QT], qrow_r[QT];
  bool qvalid[QT];
#pragma unroll
  for (int t = 0; t < QT; t++) {
    int qq;
    const T *qrow;
    if constexpr (LIST) {
      const int idx = (wq * QT + t) * 32 + lr;
      qvalid[t] = idx < cnt;
      const int r = a.rows[slot0 + (qvalid[t] ? idx : 0)];
      qrow_r[t] = r;
      // a row token outside the sequence (flagged by the row gather) reads an in-bounds query
      qq = min(max(a.row_tok[r] - base, 0), n - 1);
      qrow = (const T *)a.q_rows + (size_t)r * H + head * D;
    } else {
      const int q = q0 + (wq * QT + t) * 32 + lr;
      qvalid[t] = q < n;
      qq = qvalid[t] ? q : n - 1;
      qrow = qkv + (size_t)(base + qq) * ld + head * D;
    }
    const int qinfo = a.kinfo[base + qq];
    qopt[t] = (qinfo >> 16) - 1;
    qpos[t] = qinfo & 0xffff;
    const float *cq = a.cos_t + (size_t)qpos[t] * 32, *sq = a.sin_t + (size_t)qpos[t] * 32;
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) qf[t][ks] = *(const frag *)(qrow + ks * MF::KSTEP + lh * MF::SLOTS);
    // Pairs (i, i+32): step ks holds i = ks*KSTEP + lh*SLOTS + u, its partner
    // is in step ks + NKS/2 at the same slot.
#pragma unroll
    for (int ks = 0; ks < NKS / 2; ks++)
#pragma unroll
      for (int u = 0; u < MF::SLOTS; u++) {
#pragma clang fp contract(off)
        const int i = ks * MF::KSTEP + lh * MF::SLOTS + u;
        const float c = cq[i], sn = sq[i];
        float x, y;
        if constexpr (sizeof(T) == 2) {
          x = (float)qf[t][ks][u];
          y = (float)qf[t][ks + NKS / 2][u];
        } else {
          x = qf[t][ks];
          y = qf[t][ks + NKS / 2];
        }
        const float x2 = x * c - y * sn, y2 = y * c + x * sn;
        if constexpr (sizeof(T) == 2) {
          qf[t][ks][u] = to_elem<T>(x2);
          qf[t][ks + NKS / 2][u] = to_elem<T>(y2);
        } else {
          qf[t][ks] = x2;
          qf[t][ks + NKS / 2] = y2;
        }
      }
  }

  f32x16 ot[QT][2];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int t = 0; t < QT; t++) {
    m_run[t] = -INFINITY;
    l_run[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) ot[t][i][e] = 0.0f;
  }

  __syncthreads();  // sCode visible
  auto next_tile = [&](int kt) {
    while (kt < nkt && sCode[kt] == 0) kt++;
    return kt;
  };

  // Pipeline: the first tile is stored, the second one's loads are issued
  // and the third one's key info; then per tile: compute it from buffer b,
  // store the next tile (loaded during the compute) into buffer b^1, issue
  // the loads of the one after (its key info arrived during the compute) and
  // the key info of the one after that, one barrier.
  int kn = nkt, kn_next = nkt, b = 0;
  if (kt < nkt) {
    if (stager) stage_store<T, R>(st, sK[0], sV[0], sKo[0], sKw[0], a.half_window, tid, ROWK, ROWV);
    kn = next_tile(kt + 1);
    if (kn < nkt) {
      if (stager) {
        key_info_load<T, R>(ki, a.kinfo, base, n, kn * KTILE, tid);
        stage_load<T, R>(st, qkv, ld, H, head, base, n, kn * KTILE, a.cos_t, a.sin_t, ki, tid);
      }
      kn_next = next_tile(kn + 1);
      if (kn_next < nkt && stager) key_info_load<T, R>(ki, a.kinfo, base, n, kn_next * KTILE, tid);
    }
    __syncthreads();
  }
  const unsigned win2 = (unsigned)(2 * a.half_window);
  while (kt < nkt) {
    const char *sKb = sK[b], *sVb = sV[b];
    const int *sKob = sKo[b], *sKwb = sKw[b];
    // This wave's classes: per query tile t and 32-key half i (uniform
    // across the wave).
    const int mycode =
        __builtin_amdgcn_readfirstlane((sCode[kt] >> (4 * QT * wq)) & ((1u << (4 * QT)) - 1));
    int hcls[QT][2];
#pragma unroll
    for (int t = 0; t < QT; t++) {
      hcls[t][0] = (mycode >> (4 * t)) & 3;
      hcls[t][1] = (mycode >> (4 * t + 2)) & 3;
    }

    if (mycode != 0) {
      // S^T = K . Q^T per query tile for 64 keys (two 32x32 tiles); a K
      // fragment read from LDS feeds every query tile that needs its half.
      // A half with no allowed pair (class 0) is neither computed nor read
      // below; the others start from a zero accumulator operand (no
      // per-tile register initialisation).
      f32x16 sT[QT][2];
      const f32x16 zero = {};
#pragma unroll
      for (int i = 0; i < 2; i++) {
        int any = 0;
#pragma unroll
        for (int t = 0; t < QT; t++) any |= hcls[t][i];
        if (any == 0) continue;
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
          const int kof = (ks * MF::KSTEP + lh * MF::SLOTS) * (int)sizeof(T);
          frag kf = *(const frag *)(sKb + (i * 32 + lr) * ROWK + kof);
#pragma unroll
          for (int t = 0; t < QT; t++)
            if (hcls[t][i]) sT[t][i] = MF::mma(kf, qf[t][ks], ks == 0 ? zero : sT[t][i]);
        }
      }

      // Per query tile: mask and running max on the raw scores; the softmax
      // scale (times log2 e, > 0) is applied inside the exponent:
      // p = 2^(s*c - m*c). The per-element test is branch-free (bitwise and +
      // select).
#pragma unroll
      for (int t = 0; t < QT; t++) {
        if ((hcls[t][0] | hcls[t][1]) == 0) continue;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          if (hcls[t][i] != 2) continue;
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const int kl = i * 32 + 8 * g + 4 * lh;  // 4 consecutive keys kl..kl+3
            const int4 ko4 = *(const int4 *)(sKob + kl), kw4 = *(const int4 *)(sKwb + kl);
            const int kos[4] = {ko4.x, ko4.y, ko4.z, ko4.w}, kws[4] = {kw4.x, kw4.y, kw4.z, kw4.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
              // Block mask: a prefix query sees prefix keys; an option query
              // sees prefix keys and its own option, i.e. ko in {-1, qopt}
              // (keys past the sequence end carry -2 and match neither).
              // Window: |kpos - qpos| <= W on local layers.
              bool ok = (kos[u] == -1) | (kos[u] == qopt[t]);
              if constexpr (LOCAL) ok = ok & ((unsigned)(kws[u] - qpos[t]) <= win2);
              sT[t][i][4 * g + u] = ok ? sT[t][i][4 * g + u] : -INFINITY;
            }
          }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          if (hcls[t][i] == 0) continue;
#pragma unroll
          for (int e = 0; e < 16; e++) mx = fmaxf(mx, sT[t][i][e]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run[t], mx);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float c = a.scale_log2, mc = -m_use * c;
        const float alpha = __builtin_amdgcn_exp2f((m_run[t] - m_use) * c);
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          if (hcls[t][i] == 0) continue;  // all -inf: p = 0, and P.V skips the half
#pragma unroll
          for (int e = 0; e < 16; e++) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sT[t][i][e], c, mc));
            sT[t][i][e] = p;
            psum += p;
          }
        }
        l_run[t] = l_run[t] * alpha + psum;
        m_run[t] = m_new;
        if (__ballot(alpha != 1.0f)) {  // no lane's maximum moved: nothing to rescale
#pragma unroll
          for (int i = 0; i < 2; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) ot[t][i][e] *= alpha;
        }
      }

      // O^T += V^T . P^T. k step ks covers accumulator registers
      // [ks*SLOTS, ks*SLOTS + SLOTS) of the flattened S^T tiles; accumulator r
      // of tile i on lane half lh is key 32*i + 8*((r%16)/4) + 4*lh + r%4. A V
      // fragment read from LDS feeds every query tile that needs its half.
      constexpr int NPV = KTILE / MF::KSTEP;
#pragma unroll
      for (int ks = 0; ks < NPV; ks++) {
        const int half = ks / (NPV / 2);
        int any = 0;
#pragma unroll
        for (int t = 0; t < QT; t++) any |= hcls[t][half];
        if (any == 0) continue;
        frag pf[QT];
#pragma unroll
        for (int t = 0; t < QT; t++) {
          if constexpr (sizeof(T) == 2) {
            const int ti = ks >> 1, r0 = (ks & 1) * 8;
#pragma unroll
            for (int u = 0; u < 8; u++) pf[t][u] = to_elem<T>(sT[t][ti][r0 + u]);
          } else {
            pf[t] = sT[t][ks >> 4][ks & 15];
          }
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const char *vrow = sVb + (i * 32 + lr) * ROWV;
          frag vf;
          if constexpr (sizeof(T) == 2) {
            vf = *(const frag *)(vrow + 32 * ks + 16 * lh);  // keys 16ks + {4lh..4lh+3, 8+4lh..8+4lh+3}
          } else {
            const int r = ks & 15;
            const int key = 32 * (ks >> 4) + 8 * (r >> 2) + 4 * lh + (r & 3);
            vf = *(const float *)(vrow + key * 4);
          }
#pragma unroll
          for (int t = 0; t < QT; t++)
            if (hcls[t][half]) ot[t][i] = MF::mma(vf, pf[t], ot[t][i]);
        }
      }
    }
    int kn2 = nkt;
    if (kn < nkt) {
      const int nb = NBUF == 2 ? b ^ 1 : 0;
      if constexpr (NBUF == 1) __syncthreads();  // every wave is done with the one buffer
      if (stager) stage_store<T, R>(st, sK[nb], sV[nb], sKo[nb], sKw[nb], a.half_window, tid, ROWK, ROWV);
      kn2 = kn_next;  // == next_tile(kn + 1); ki holds its key info
      if (kn2 < nkt) {
        if (stager) stage_load<T, R>(st, qkv, ld, H, head, base, n, kn2 * KTILE, a.cos_t, a.sin_t, ki, tid);
        kn_next = next_tile(kn2 + 1);
        if (kn_next < nkt && stager) key_info_load<T, R>(ki, a.kinfo, base, n, kn_next * KTILE, tid);
      }
    }
    __syncthreads();  // the next tile's buffer is complete; buffer b is free
    kt = kn;
    kn = kn2;
    b = NBUF == 2 ? b ^ 1 : 0;
  }

  // Normalise and store ctx[token][head*64 + d]; in training also the
  // softmax denominator in log2 form (the backward recomputes P from it).
#pragma unroll
  for (int t = 0; t < QT; t++) {
    const float l_tot = l_run[t] + __shfl_xor(l_run[t], 32);
    const float inv = 1.0f / l_tot;
    if (!LIST && a.lse && qvalid[t] && lh == 0) {
      const int q = q0 + (wq * QT + t) * 32 + lr;
      a.lse[(size_t)(base + q) * a.heads + head] = m_run[t] * a.scale_log2 + log2f(l_tot);
    }
    if (qvalid[t]) {
      const int q = q0 + (wq * QT + t) * 32 + lr;
      T *out = (T *)a.ctx + (size_t)(LIST ? qrow_r[t] : base + q) * H + head * D;
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d0 = i * 32 + 8 * g + 4 * lh;
          if constexpr (sizeof(T) == 2) {
            *(uint2 *)(out + d0) = make_uint2(pack16<T>(ot[t][i][4 * g] * inv, ot[t][i][4 * g + 1] * inv),
                                              pack16<T>(ot[t][i][4 * g + 2] * inv, ot[t][i][4 * g + 3] * inv));
          } else {
            *(float4 *)(out + d0) = make_float4(ot[t][i][4 * g] * inv, ot[t][i][4 * g + 1] * inv,
                                                ot[t][i][4 * g + 2] * inv, ot[t][i][4 * g + 3] * inv);
          }
        }
    }
  }
}

// Work items of the option-row attention (attention_kernel<..., LIST>): the
// rows r < R (row_tok[r] a token of the batch) grouped by sequence, each
// sequence's rows in chunks of up to ATTN_QUERIES, item = (sequence, first
// slot in rows[], row count). One workgroup of 1024 threads, thread j owning
// sequence j (nseq <= ROW_ITEMS_MAXSEQ):
//   1. every row's sequence (binary search of seq_off), counted per sequence;
//   2. exclusive scans of the counts (first slot) and of the chunk counts
//      (first item);
//   3. every row placed in a slot of its sequence (in atomic order: a row's
//      result does not depend on its slot) and the items written.
// A row token outside [0, T) counts as sequence 0 (the row gather flags it).
__device__ __forceinline__ int block_excl_scan(int v, int *wsum) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int w = 0; w < 16; w++) {
      const int t = wsum[w];
      wsum[w] = acc;
      acc += t;
    }
    wsum[16] = acc;
  }
  __syncthreads();
  return x - v + wsum[wave];
}

__global__ __launch_bounds__(1024) void row_items_kernel(const int *row_tok, int R, const int *seq_off, int nseq,
                                                         int T, int4 *items, int *rows, int *nitems) {
  __shared__ int cnt[ROW_ITEMS_MAXSEQ], fill[ROW_ITEMS_MAXSEQ], wsum[17];
  const int j = threadIdx.x;
  cnt[j] = 0;
  fill[j] = 0;
  __syncthreads();
  auto seq_of = [&](int r) {
    const int t = row_tok[r];
    if (t < 0 || t >= T) return 0;
    int lo = 0, hi = nseq - 1;  // last sequence whose offset is <= t
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (seq_off[mid] <= t) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  };
  for (int r = j; r < R; r += 1024) atomicAdd(&cnt[seq_of(r)], 1);
  __syncthreads();
  const int c = j < nseq ? cnt[j] : 0, nch = (c + ATTN_QUERIES - 1) / ATTN_QUERIES;
  const int slot0 = block_excl_scan(c, wsum);
  const int item0 = block_excl_scan(nch, wsum);
  if (j == 0) *nitems = wsum[16];
  for (int k = 0; k < nch; k++) items[item0 + k] = make_int4(j, slot0 + k * ATTN_QUERIES, min(ATTN_QUERIES, c - k * ATTN_QUERIES), 0);
  cnt[j] = slot0;  // reused: first slot of sequence j
  __syncthreads();
  for (int r = j; r < R; r += 1024) {
    const int sq = seq_of(r);
    rows[cnt[sq] + atomicAdd(&fill[sq], 1)] = r;
  }
}

// Tile classes of one work item (32 * NC queries of one sequence) for one
// layer type: for every 64-key tile and 32-query chunk c, the 2-bit class (0
// none, 1 all, 2 per-element) of each 32-key half against the chunk, packed
// as bits 4c..4c+3; and the first tile with any allowed pair (nkt if none).
// The classes depend only on the batch layout and the layer type, so every
// layer of that type reuses them.
template <int NC>
__global__ __launch_bounds__(64) void tile_codes_kernel(const ChunkInfo *chunks, const int4 *work, const int *seq_len,
                                                        const int *chunk_off, int sliding, int half_window,
                                                        uint32_t *codes, int *first) {
  static_assert(NC <= 8, "32-bit codes");
  __shared__ int s_first;
  const int wi = blockIdx.x, tid = threadIdx.x;
  // sliding < 0: both layer types in one launch, blockIdx.y = 1 for the
  // sliding-window one, its codes and first tiles one section (gridDim.x
  // items) after the global ones.
  if (sliding < 0) {
    sliding = blockIdx.y;
    codes += (size_t)sliding * gridDim.x * ATTN_MAXKT;
    first += sliding * gridDim.x;
  }
  const int4 wk = work[wi];
  const int s = wk.x, q0 = wk.y;
  const int n = seq_len[s], cbase = chunk_off[s];
  const int nch = (n + 31) / 32, nkt = (n + KTILE - 1) / KTILE;
  if (tid == 0) s_first = nkt;
  __syncthreads();
  const ChunkInfo empty = {0, 0, 1, 0, 0, 0, 0, 0};
  ChunkInfo qc[NC];
#pragma unroll
  for (int w = 0; w < NC; w++) {
    const int c = q0 / 32 + w;
    qc[w] = c < nch ? chunks[cbase + c] : empty;
  }
  for (int kt = tid; kt < nkt; kt += 64) {
    const ChunkInfo kc0 = chunks[cbase + 2 * kt];
    const ChunkInfo kc1 = (2 * kt + 1 < nch) ? chunks[cbase + 2 * kt + 1] : empty;
    uint32_t code = 0;
#pragma unroll
    for (int w = 0; w < NC; w++)
      code |= (uint32_t)(tile_class(qc[w], kc0, sliding, half_window) |
                         (tile_class(qc[w], kc1, sliding, half_window) << 2))
              << (4 * w);
    codes[(size_t)wi * ATTN_MAXKT + kt] = code;
    if (code) atomicMin(&s_first, kt);
  }
  __syncthreads();
  if (tid == 0) first[wi] = s_first;
}




// ---------------------------------------------------------------------------
// Attention backward: the reference's attnBwd (backward.go:117-159) with the
// RoPE inverse (backward.go:77-81), recomputing P instead of keeping it:
//   P = 2^(s*c - lse) (c = scale*log2 e; lse from the forward), masked -> 0
//   dP = dO . V^T,  D = rowsum(dO * O) (= sum_j P dP),  dS = P * (dP - D) * scale
//   dQ = dS . K,    dK = dS^T . Q,    dV = P^T . dO
// Two kernels, neither with atomics:
//   * attn_bwd_dq_kernel is query-major (the forward's work items, tile list
//     and tile classes): S^T = K.Q^T and dP^T = V.dO^T put one query per lane
//     pair, so lse and D are per-lane scalars; dQ^T += K^T . dS^T uses dS^T
//     straight from registers (keys permuted in the staged K^T, as the forward
//     does for V^T). It also writes D for the second kernel.
//   * attn_bwd_dkdv_kernel is key-major (128 keys of one (sequence, head) per
//     workgroup, one key per lane pair): S = Q.K^T and dP = dO.V^T put one key
//     per lane, and dV^T += dO^T . P, dK^T += Q^T . dS take P and dS from
//     registers. Query tiles with no allowed pair for any wave are skipped by
//     the same chunk classes as the forward.
// Every tile is staged row-major (RoPE applied to q and k), and the
// transposed, key-permuted copy an MFMA operand needs is built from it in LDS.


// One 64-row x 64-d tile of rows r0.. of a row-major [tokens x ld] array, in
// registers between load and store. Item it of the 256 threads is (row,
// 16-byte chunk c and its RoPE partner c + 32 elements): bf16 4 chunks per
// half row, fp32 8.
template <class T>
struct RowStage {
  static constexpr int NI = sizeof(T) == 2 ? 1 : 2;
  uint4 lo[NI], hi[NI];
  float4 c0[NI], c1[NI], s0[NI], s1[NI];
};

template <class T, bool ROT>
__device__ __forceinline__ void rows_load(RowStage<T> &st, const T *src, int ld, int base, int r0, int n,
                                          const float *cos_t, const float *sin_t, const int *kinfo, int tid) {
  constexpr int EL = 16 / sizeof(T), CPH = 32 / EL;  // elements per chunk, chunks per half row
#pragma unroll
  for (int j = 0; j < RowStage<T>::NI; j++) {
    const int it = tid + 256 * j, row = it / CPH, c = it % CPH;
    const bool ok = r0 + row < n;
    const size_t tok = (size_t)(base + min(r0 + row, n - 1));
    const T *p = src + tok * ld;
    st.lo[j] = keep_if(ok, *(const uint4 *)(p + EL * c));
    st.hi[j] = keep_if(ok, *(const uint4 *)(p + 32 + EL * c));
    if constexpr (ROT) {
      const size_t pos = (size_t)(kinfo[tok] & 0xffff);
      st.c0[j] = *(const float4 *)(cos_t + pos * 32 + EL * c);
      st.s0[j] = *(const float4 *)(sin_t + pos * 32 + EL * c);
      if constexpr (sizeof(T) == 2) {
        st.c1[j] = *(const float4 *)(cos_t + pos * 32 + EL * c + 4);
        st.s1[j] = *(const float4 *)(sin_t + pos * 32 + EL * c + 4);
      }
    }
  }
}

// Stores the tile row-major: row r at dst + r*ROW, d-contiguous.
template <class T, bool ROT>
__device__ __forceinline__ void rows_store(const RowStage<T> &st, char *dst, int tid) {
  constexpr int EL = 16 / sizeof(T), CPH = 32 / EL, ROW = D * sizeof(T) + 16;
#pragma unroll
  for (int j = 0; j < RowStage<T>::NI; j++) {
    const int it = tid + 256 * j, row = it / CPH, c = it % CPH;
    uint4 lo = st.lo[j], hi = st.hi[j];
    if constexpr (ROT) {
      if constexpr (sizeof(T) == 2) {
        const uint32_t l[4] = {lo.x, lo.y, lo.z, lo.w}, h[4] = {hi.x, hi.y, hi.z, hi.w};
        const float cs[8] = {st.c0[j].x, st.c0[j].y, st.c0[j].z, st.c0[j].w,
                             st.c1[j].x, st.c1[j].y, st.c1[j].z, st.c1[j].w};
        const float sn[8] = {st.s0[j].x, st.s0[j].y, st.s0[j].z, st.s0[j].w,
                             st.s1[j].x, st.s1[j].y, st.s1[j].z, st.s1[j].w};
        uint32_t po[4], ph[4];
#pragma unroll
        for (int w = 0; w < 4; w++) {
          float a0 = lo16<T>(l[w]), a1 = hi16<T>(l[w]), b0 = lo16<T>(h[w]), b1 = hi16<T>(h[w]);
          rope1(a0, b0, cs[2 * w], sn[2 * w]);
          rope1(a1, b1, cs[2 * w + 1], sn[2 * w + 1]);
          po[w] = pack16<T>(a0, a1);
          ph[w] = pack16<T>(b0, b1);
        }
        lo = make_uint4(po[0], po[1], po[2], po[3]);
        hi = make_uint4(ph[0], ph[1], ph[2], ph[3]);
      } else {
        float4 a = *(const float4 *)&lo, b = *(const float4 *)&hi;
        rope1(a.x, b.x, st.c0[j].x, st.s0[j].x);
        rope1(a.y, b.y, st.c0[j].y, st.s0[j].y);
        rope1(a.z, b.z, st.c0[j].z, st.s0[j].z);
        rope1(a.w, b.w, st.c0[j].w, st.s0[j].w);
        lo = *(const uint4 *)&a;
        hi = *(const uint4 *)&b;
      }
    }
    *(uint4 *)(dst + row * ROW + 16 * c) = lo;
    *(uint4 *)(dst + row * ROW + (32 * sizeof(T)) + 16 * c) = hi;
  }
}

// Builds the transposed copy TT[d][row] of a row-major tile R (both with
// D*sizeof(T)+16-byte rows). bf16: rows (2p, 2p+1) share a 32-bit word, and
// within each 16-row group the 4-row runs are in the order 0-3, 8-11, 4-7,
// 12-15 (the order one lane feeds a k step from the S^T / S accumulators).
// fp32: plain row order; the reader permutes per k step.
template <class T>
__device__ __forceinline__ void build_transposed(const char *R, char *TT, int tid) {
  constexpr int ROW = D * sizeof(T) + 16;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int it = tid + 256 * j, p = it & 31, d = it >> 5;
      const uint32_t lo = *(const uint16_t *)(R + (2 * p) * ROW + 2 * d);
      const uint32_t hi = *(const uint16_t *)(R + (2 * p + 1) * ROW + 2 * d);
      const int lp = p & 7, q4 = lp >> 1;
      const int pw = (p & ~7) + ((((q4 & 1) << 1) | (q4 >> 1)) << 1) + (lp & 1);
      *(uint32_t *)(TT + d * ROW + 4 * pw) = lo | (hi << 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int it = tid + 256 * j, r = it & 63, d = it >> 6;
      *(float *)(TT + d * ROW + 4 * r) = *(const float *)(R + r * ROW + 4 * d);
    }
  }
}

// MFMA operand of k step ks from the row-major tile (row `row`, k = d).
template <class T>
__device__ __forceinline__ typename Mfma<T>::frag row_frag(const char *R, int row, int ks, int lh) {
  using MF = Mfma<T>;
  constexpr int ROW = D * sizeof(T) + 16;
  return *(const typename MF::frag *)(R + row * ROW + (ks * MF::KSTEP + lh * MF::SLOTS) * (int)sizeof(T));
}

// MFMA operand of k step ks (over the 64 tile rows) from the transposed tile
// (row d), matching the register order of an S^T / S accumulator pair.
template <class T>
__device__ __forceinline__ typename Mfma<T>::frag t_frag(const char *TT, int d, int ks, int lh) {
  using MF = Mfma<T>;
  constexpr int ROW = D * sizeof(T) + 16;
  const char *row = TT + d * ROW;
  if constexpr (sizeof(T) == 2) {
    return *(const typename MF::frag *)(row + 32 * ks + 16 * lh);
  } else {
    const int r = ks & 15;
    return *(const float *)(row + 4 * (32 * (ks >> 4) + 8 * (r >> 2) + 4 * lh + (r & 3)));
  }
}

// The B operand of k step ks taken from a pair of 32x32 accumulators (the 64
// tile rows of the k dimension).
template <class T>
__device__ __forceinline__ typename Mfma<T>::frag acc_frag(const f32x16 (&x)[2], int ks) {
  typename Mfma<T>::frag f;
  if constexpr (sizeof(T) == 2) {
    const int ti = ks >> 1, r0 = (ks & 1) * 8;
#pragma unroll
    for (int u = 0; u < 8; u++) f[u] = to_elem<T>(x[ti][r0 + u]);
  } else {
    f = x[ks >> 4][ks & 15];
  }
  return f;
}

// Writes a lane's 64-d row (two 32-d accumulator blocks of one token, d =
// 32*blk + mfma_row(e)) to dst[d], with the inverse RoPE rotation of the
// token's position when cs is given (pairs (d, d+32) are the same register
// of the two blocks).
template <class T>
__device__ __forceinline__ void store_row64(f32x16 (&x)[2], T *dst, const float *cs, const float *sn, int lh) {
  if (cs) {
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int d = 8 * (e >> 2) + 4 * lh + (e & 3);
      float u = x[0][e], v = x[1][e];
      rope1(u, v, cs[d], -sn[d]);
      x[0][e] = u;
      x[1][e] = v;
    }
  }
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d0 = b * 32 + 8 * g + 4 * lh;
      if constexpr (sizeof(T) == 2) {
        *(uint2 *)(dst + d0) = make_uint2(pack16<T>(x[b][4 * g], x[b][4 * g + 1]), pack16<T>(x[b][4 * g + 2], x[b][4 * g + 3]));
      } else {
        *(float4 *)(dst + d0) = make_float4(x[b][4 * g], x[b][4 * g + 1], x[b][4 * g + 2], x[b][4 * g + 3]);
      }
    }
}

template <class T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_bwd_dq_kernel(AttnBwdArgs a) {
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  constexpr int ROW = D * sizeof(T) + 16, NKS = D / MF::KSTEP, NPV = KTILE / MF::KSTEP;
  __shared__ __attribute__((aligned(16))) char sK[KTILE * ROW];
  __shared__ __attribute__((aligned(16))) char sV[KTILE * ROW];
  __shared__ __attribute__((aligned(16))) char sKT[D * ROW];
  __shared__ __attribute__((aligned(16))) int sInfo[KTILE];
  __shared__ uint32_t sCode[ATTN_MAXKT];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int total = a.nwork * a.heads, bid = blockIdx.x;
  const int logical = total % 8 == 0 ? (bid % 8) * (total / 8) + bid / 8 : bid;
  const int wi = logical / a.heads, head = logical % a.heads;
  const int4 wk = a.work[wi];
  const int s = wk.x, q0 = wk.y;
  const int n = a.seq_len[s], base = a.seq_off[s];
  const int H = a.H, ld = 3 * H;
  const T *qkv = (const T *)a.qkv;
  const int nkt = (n + KTILE - 1) / KTILE;
  const uint32_t *codes = a.codes + (size_t)wi * ATTN_MAXKT;
  for (int kt = tid; kt < nkt; kt += 256) sCode[kt] = codes[kt];

  // The lane's query: rotated Q^T and dO^T operands, lse, D.
  const int q = q0 + wave * 32 + lr;
  const bool qvalid = q < n;
  const size_t qtok = (size_t)(base + (qvalid ? q : n - 1));
  const int qinfo = a.kinfo[qtok], qopt = (qinfo >> 16) - 1, qpos = qinfo & 0xffff;
  const float *cq = a.cos_t + (size_t)qpos * 32, *sq = a.sin_t + (size_t)qpos * 32;
  frag qf[NKS], dof[NKS];
  float dsum = 0.0f;
  {
    const T *qrow = qkv + qtok * ld + head * D;
    const T *orow = (const T *)a.ctx + qtok * H + head * D;
    const T *drow = (const T *)a.dctx + qtok * H + head * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const int k0 = ks * MF::KSTEP + lh * MF::SLOTS;
      qf[ks] = *(const frag *)(qrow + k0);
      dof[ks] = *(const frag *)(drow + k0);
      const frag of = *(const frag *)(orow + k0);
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int u = 0; u < 8; u++) dsum += (float)dof[ks][u] * (float)of[u];
      } else {
        dsum += dof[ks] * of;
      }
    }
#pragma unroll
    for (int ks = 0; ks < NKS / 2; ks++)
#pragma unroll
      for (int u = 0; u < MF::SLOTS; u++) {
        const int i = ks * MF::KSTEP + lh * MF::SLOTS + u;
        float x, y;
        if constexpr (sizeof(T) == 2) {
          x = (float)qf[ks][u];
          y = (float)qf[ks + NKS / 2][u];
        } else {
          x = qf[ks];
          y = qf[ks + NKS / 2];
        }
        rope1(x, y, cq[i], sq[i]);
        if constexpr (sizeof(T) == 2) {
          qf[ks][u] = to_elem<T>(x);
          qf[ks + NKS / 2][u] = to_elem<T>(y);
        } else {
          qf[ks] = x;
          qf[ks + NKS / 2] = y;
        }
      }
  }
  dsum += __shfl_xor(dsum, 32);
  if (qvalid && lh == 0) a.dsum[qtok * a.heads + head] = dsum;
  const float lse = a.lse[qtok * a.heads + head];
  const float c = a.scale_log2;

  f32x16 dq[2];
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int e = 0; e < 16; e++) dq[b][e] = 0.0f;

  __syncthreads();  // sCode
  const unsigned win2 = a.sliding ? (unsigned)(2 * a.half_window) : 0xffffffffu;
  for (int kt = a.first[wi]; kt < nkt; kt++) {
    if (sCode[kt] == 0) continue;
    const int k0 = kt * KTILE;
    {
      RowStage<T> sk, sv;
      rows_load<T, true>(sk, qkv + H + head * D, ld, base, k0, n, a.cos_t, a.sin_t, a.kinfo, tid);
      rows_load<T, false>(sv, qkv + 2 * H + head * D, ld, base, k0, n, nullptr, nullptr, nullptr, tid);
      const int info = (tid < KTILE && k0 + tid < n) ? a.kinfo[base + k0 + tid] : 0;
      __syncthreads();  // the previous tile's reads are done
      rows_store<T, true>(sk, sK, tid);
      rows_store<T, false>(sv, sV, tid);
      if (tid < KTILE) sInfo[tid] = info;
    }
    __syncthreads();
    build_transposed<T>(sK, sKT, tid);
    __syncthreads();

    const int mycode = __builtin_amdgcn_readfirstlane((sCode[kt] >> (4 * wave)) & 15);
    if (mycode == 0) continue;
    const int hcls[2] = {mycode & 3, (mycode >> 2) & 3};
    f32x16 sT[2], dpT[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        sT[i][e] = 0.0f;
        dpT[i][e] = 0.0f;
      }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (hcls[i] == 0) continue;
#pragma unroll
      for (int ks = 0; ks < NKS; ks++) {
        sT[i] = MF::mma(row_frag<T>(sK, i * 32 + lr, ks, lh), qf[ks], sT[i]);
        dpT[i] = MF::mma(row_frag<T>(sV, i * 32 + lr, ks, lh), dof[ks], dpT[i]);
      }
    }
    // P^T and dS^T in place of sT (per element: key 32i + 8(e/4) + 4lh + e%4).
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (hcls[i] == 0) continue;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int kl = i * 32 + 8 * g + 4 * lh;
        const int4 inf4 = *(const int4 *)(sInfo + kl);
        const int inf[4] = {inf4.x, inf4.y, inf4.z, inf4.w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int ko = (inf[u] >> 16) - 1, kp = inf[u] & 0xffff;
          const bool ok = qvalid & (k0 + kl + u < n) & ((ko == -1) | (ko == qopt)) &
                          ((unsigned)(kp - qpos + a.half_window) <= win2);
          const int e = 4 * g + u;
          const float p = ok ? __builtin_amdgcn_exp2f(fmaf(sT[i][e], c, -lse)) : 0.0f;
          sT[i][e] = p * (dpT[i][e] - dsum) * a.scale;
        }
      }
    }
    // dQ^T += K^T . dS^T
#pragma unroll
    for (int ks = 0; ks < NPV; ks++) {
      if (hcls[ks / (NPV / 2)] == 0) continue;
      const frag df = acc_frag<T>(sT, ks);
#pragma unroll
      for (int b = 0; b < 2; b++) dq[b] = MF::mma(t_frag<T>(sKT, b * 32 + lr, ks, lh), df, dq[b]);
    }
  }
  if (qvalid) store_row64<T>(dq, (T *)a.dqkv + qtok * ld + head * D, cq, sq, lh);
}

template <class T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_bwd_dkdv_kernel(AttnBwdArgs a) {
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  constexpr int ROW = D * sizeof(T) + 16, NKS = D / MF::KSTEP, NPV = KTILE / MF::KSTEP;
  __shared__ __attribute__((aligned(16))) char sQ[KTILE * ROW];
  __shared__ __attribute__((aligned(16))) char sQT[D * ROW];
  __shared__ __attribute__((aligned(16))) char sO[KTILE * ROW];
  __shared__ __attribute__((aligned(16))) char sOT[D * ROW];
  __shared__ __attribute__((aligned(16))) int sInfo[KTILE];
  __shared__ __attribute__((aligned(16))) float sL[KTILE], sD[KTILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int total = a.nwork * a.heads, bid = blockIdx.x;
  const int logical = total % 8 == 0 ? (bid % 8) * (total / 8) + bid / 8 : bid;
  const int wi = logical / a.heads, head = logical % a.heads;
  const int4 wk = a.work[wi];
  const int s = wk.x, kw0 = wk.y;  // this workgroup's 128 keys start at kw0
  const int n = a.seq_len[s], base = a.seq_off[s];
  const int H = a.H, ld = 3 * H;
  const T *qkv = (const T *)a.qkv;
  const int nch = (n + 31) / 32, cbase = a.chunk_off[s];

  // The lane's key: rotated K and V operands (B operands: column = key).
  const int k = kw0 + wave * 32 + lr;
  const bool kvalid = k < n;
  const size_t ktok = (size_t)(base + (kvalid ? k : n - 1));
  const int kinfo = a.kinfo[ktok], kopt = (kinfo >> 16) - 1, kpos = kinfo & 0xffff;
  const float *ck = a.cos_t + (size_t)kpos * 32, *sk = a.sin_t + (size_t)kpos * 32;
  frag kf[NKS], vf[NKS];
  {
    const T *krow = qkv + ktok * ld + H + head * D;
    const T *vrow = qkv + ktok * ld + 2 * H + head * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const int k0 = ks * MF::KSTEP + lh * MF::SLOTS;
      kf[ks] = *(const frag *)(krow + k0);
      vf[ks] = *(const frag *)(vrow + k0);
    }
#pragma unroll
    for (int ks = 0; ks < NKS / 2; ks++)
#pragma unroll
      for (int u = 0; u < MF::SLOTS; u++) {
        const int i = ks * MF::KSTEP + lh * MF::SLOTS + u;
        float x, y;
        if constexpr (sizeof(T) == 2) {
          x = (float)kf[ks][u];
          y = (float)kf[ks + NKS / 2][u];
        } else {
          x = kf[ks];
          y = kf[ks + NKS / 2];
        }
        rope1(x, y, ck[i], sk[i]);
        if constexpr (sizeof(T) == 2) {
          kf[ks][u] = to_elem<T>(x);
          kf[ks + NKS / 2][u] = to_elem<T>(y);
        } else {
          kf[ks] = x;
          kf[ks + NKS / 2] = y;
        }
      }
  }
  // Key chunk of each wave (empty past the sequence end).
  const ChunkInfo empty = {0, 0, 1, 0, 0, 0, 0, 0};
  ChunkInfo kc[4];
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const int ch = kw0 / 32 + w;
    kc[w] = ch < nch ? a.chunks[cbase + ch] : empty;
  }

  f32x16 dk[2], dv[2];
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      dk[b][e] = 0.0f;
      dv[b][e] = 0.0f;
    }
  const float c = a.scale_log2;
  const unsigned win2 = a.sliding ? (unsigned)(2 * a.half_window) : 0xffffffffu;
  const int nqt = (n + KTILE - 1) / KTILE;
  for (int qt = 0; qt < nqt; qt++) {
    const int q0 = qt * KTILE;
    const ChunkInfo qc0 = a.chunks[cbase + 2 * qt];
    const ChunkInfo qc1 = 2 * qt + 1 < nch ? a.chunks[cbase + 2 * qt + 1] : empty;
    int any = 0, hcls[2] = {0, 0};
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const int c0 = tile_class(qc0, kc[w], a.sliding, a.half_window);
      const int c1 = tile_class(qc1, kc[w], a.sliding, a.half_window);
      any |= c0 | c1;
      if (w == wave) {
        hcls[0] = c0;
        hcls[1] = c1;
      }
    }
    if (any == 0) continue;
    // Staged one operand at a time after the barrier (fewer live registers:
    // two workgroups per CU hide the load latency).
    __syncthreads();  // the previous tile's reads are done
    {
      RowStage<T> sq;
      rows_load<T, true>(sq, qkv + head * D, ld, base, q0, n, a.cos_t, a.sin_t, a.kinfo, tid);
      rows_store<T, true>(sq, sQ, tid);
    }
    {
      RowStage<T> so;
      rows_load<T, false>(so, (const T *)a.dctx + head * D, H, base, q0, n, nullptr, nullptr, nullptr, tid);
      rows_store<T, false>(so, sO, tid);
    }
    if (tid < KTILE) {
      int info = 0;
      float lse = INFINITY, dd = 0.0f;  // rows past the end: P = 2^-inf = 0
      if (q0 + tid < n) {
        const size_t t = (size_t)(base + q0 + tid);
        info = a.kinfo[t];
        lse = a.lse[t * a.heads + head];
        dd = a.dsum[t * a.heads + head];
      }
      sInfo[tid] = info;
      sL[tid] = lse;
      sD[tid] = dd;
    }
    __syncthreads();
    build_transposed<T>(sQ, sQT, tid);
    build_transposed<T>(sO, sOT, tid);
    __syncthreads();
    if ((hcls[0] | hcls[1]) == 0) continue;

    // One 32-query half at a time (fewer live accumulators): S = Q.K^T and
    // dP = dO.V^T, then P and dS in place, then that half's k steps of
    // dV^T += dO^T . P and dK^T += Q^T . dS. Element e of the half's
    // accumulators is query 32i + 8(e/4) + 4lh + e%4.
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (hcls[i] == 0) continue;
      f32x16 sc, dp;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        sc[e] = 0.0f;
        dp[e] = 0.0f;
      }
#pragma unroll
      for (int ks = 0; ks < NKS; ks++) {
        sc = MF::mma(row_frag<T>(sQ, i * 32 + lr, ks, lh), kf[ks], sc);
        dp = MF::mma(row_frag<T>(sO, i * 32 + lr, ks, lh), vf[ks], dp);
      }
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int ql = i * 32 + 8 * g + 4 * lh;
        const int4 inf4 = *(const int4 *)(sInfo + ql);
        const float4 l4 = *(const float4 *)(sL + ql), d4 = *(const float4 *)(sD + ql);
        const int inf[4] = {inf4.x, inf4.y, inf4.z, inf4.w};
        const float lq[4] = {l4.x, l4.y, l4.z, l4.w}, dq4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int qo = (inf[u] >> 16) - 1, qp = inf[u] & 0xffff;
          const bool ok = kvalid & (q0 + ql + u < n) & ((kopt == -1) | (kopt == qo)) &
                          ((unsigned)(kpos - qp + a.half_window) <= win2);
          const int e = 4 * g + u;
          const float p = ok ? __builtin_amdgcn_exp2f(fmaf(sc[e], c, -lq[u])) : 0.0f;
          sc[e] = p;
          dp[e] = p * (dp[e] - dq4[u]) * a.scale;
        }
      }
#pragma unroll
      for (int kl = 0; kl < NPV / 2; kl++) {
        const int ks = i * (NPV / 2) + kl;
        frag pf, df;
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int u = 0; u < 8; u++) {
            pf[u] = to_elem<T>(sc[kl * 8 + u]);
            df[u] = to_elem<T>(dp[kl * 8 + u]);
          }
        } else {
          pf = sc[kl];
          df = dp[kl];
        }
#pragma unroll
        for (int b = 0; b < 2; b++) {
          dv[b] = MF::mma(t_frag<T>(sOT, b * 32 + lr, ks, lh), pf, dv[b]);
          dk[b] = MF::mma(t_frag<T>(sQT, b * 32 + lr, ks, lh), df, dk[b]);
        }
      }
    }
  }
  if (kvalid) {
    T *row = (T *)a.dqkv + ktok * ld + head * D;
    store_row64<T>(dk, row + H, ck, sk, lh);
    store_row64<T>(dv, row + 2 * H, nullptr, nullptr, lh);
  }
}

}  // namespace

// Attention for head widths other than 64 (the reference's small test
// models): thread = one query of one (sequence, head). The reference's attnFwd
// + softmaxMasked (forward.go:347-409, ops.go) in three passes over the
// sequence's allowed keys, scores recomputed each time: the maximum of the
// scaled scores; the f64 sum of e_j = float32(exp(s_j * scale - max)); ctx =
// sum_j p_j v_j with p_j = e_j * float32(1 / sum). q and k are rotated as
// applyRope does, in fp32, from the un-rotated qkv.
template <class T, int D>
__global__ __launch_bounds__(64) void attention_generic_kernel(AttnArgs a) {
  constexpr int HALF = D / 2;
  const int sq = blockIdx.y, head = blockIdx.z;
  const int n = a.seq_len[sq], base = a.seq_off[sq];
  const int qi = blockIdx.x * 64 + threadIdx.x;
  if (qi >= n) return;
  const int H = a.H, ld = 3 * H;
  const T *qkv = (const T *)a.qkv;
  const int qinf = a.kinfo[base + qi];
  const int qopt = (qinf >> 16) - 1, qpos = qinf & 0xffff;
  auto rotate = [&](float (&x)[D], int pos) {
#pragma unroll
    for (int i = 0; i < HALF; i++) rope1(x[i], x[i + HALF], a.cos_t[(size_t)pos * 32 + i], a.sin_t[(size_t)pos * 32 + i]);
  };
  float q[D];
  {
    const T *src = qkv + (size_t)(base + qi) * ld + head * D;
#pragma unroll
    for (int d = 0; d < D; d++) q[d] = (float)src[d];
    rotate(q, qpos);
  }
  const float scale = a.scale;
  // Score of key j (raw, unscaled) if the mask allows it.
  auto score = [&](int j, float &sc) -> bool {
    const int inf = a.kinfo[base + j], ko = (inf >> 16) - 1, kp = inf & 0xffff;
    if (ko != -1 && ko != qopt) return false;
    if (a.sliding && abs(kp - qpos) > a.half_window) return false;
    float k[D];
    const T *src = qkv + (size_t)(base + j) * ld + H + head * D;
#pragma unroll
    for (int d = 0; d < D; d++) k[d] = (float)src[d];
    rotate(k, kp);
    float acc = 0.0f;
#pragma unroll
    for (int d = 0; d < D; d++) acc = fmaf(q[d], k[d], acc);
    sc = acc;
    return true;
  };
  float maxv = -INFINITY;
  for (int j = 0; j < n; j++) {
    float sc;
    if (score(j, sc)) maxv = fmaxf(maxv, sc * scale);
  }
  double sum = 0.0;
  for (int j = 0; j < n; j++) {
    float sc;
    if (score(j, sc)) sum += (double)(float)exp((double)(sc * scale - maxv));
  }
  const float inv = (float)(1.0 / sum);
  float o[D];
#pragma unroll
  for (int d = 0; d < D; d++) o[d] = 0.0f;
  for (int j = 0; j < n; j++) {
    float sc;
    if (!score(j, sc)) continue;
    const float p = (float)exp((double)(sc * scale - maxv)) * inv;
    const T *v = qkv + (size_t)(base + j) * ld + 2 * H + head * D;
#pragma unroll
    for (int d = 0; d < D; d++) o[d] = fmaf(p, (float)v[d], o[d]);
  }
  T *out = (T *)a.ctx + (size_t)(base + qi) * H + head * D;
#pragma unroll
  for (int d = 0; d < D; d++) out[d] = to_elem<T>(o[d]);
}

template <class T>
hipError_t launch_attention_generic_t(const AttnArgs &a, hipStream_t s) {
  const dim3 grid((a.max_len + 63) / 64, a.nseq, a.heads), block(64);
  switch (a.head_dim) {
    case 8: hipLaunchKernelGGL((attention_generic_kernel<T, 8>), grid, block, 0, s, a); break;
    case 16: hipLaunchKernelGGL((attention_generic_kernel<T, 16>), grid, block, 0, s, a); break;
    case 32: hipLaunchKernelGGL((attention_generic_kernel<T, 32>), grid, block, 0, s, a); break;
    case 64: hipLaunchKernelGGL((attention_generic_kernel<T, 64>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attention_generic(int precision, const AttnArgs &a, hipStream_t s) {
  if (a.nseq <= 0 || a.max_len <= 0) return hipSuccess;
  return precision == PREC_BF16  ? launch_attention_generic_t<bf16>(a, s)
         : precision == PREC_F16 ? launch_attention_generic_t<f16>(a, s)
                                 : launch_attention_generic_t<float>(a, s);
}

template <class T>
void launch_attention_t(const AttnArgs &a, hipStream_t s) {
  // fp32 launches of at most 256 (work item, head) pairs (the certification
  // twin's few sequences, fp32 validation of small requests) leave most CUs
  // idle: each work item runs as two workgroups of two waves (the same
  // per-query arithmetic; one 512-token fp32 forward 3.81 -> 3.37 ms, bit-
  // identical; one-wave parts measured the same).
  if constexpr (std::is_same<T, float>::value) {
    if (a.qt == ATTN_QT && a.nwork * a.heads <= 256) {
      dim3 grid(a.nwork * a.heads * (ATTN_WAVES / 2)), block(128);
      if (a.sliding) hipLaunchKernelGGL((attention_kernel<T, 2, ATTN_QT, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((attention_kernel<T, 2, ATTN_QT, false>), grid, block, 0, s, a);
      return;
    }
  }
  dim3 grid(a.nwork * a.heads), block(64 * ATTN_WAVES);
  if (a.sliding)
    hipLaunchKernelGGL((attention_kernel<T, ATTN_WAVES, ATTN_QT, true>), grid, block, 0, s, a);
  else if (a.qt == ATTN_QT_GLOBAL)
    hipLaunchKernelGGL((attention_kernel<T, ATTN_WAVES, ATTN_QT_GLOBAL, false>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((attention_kernel<T, ATTN_WAVES, ATTN_QT, false>), grid, block, 0, s, a);
}

template <class T>
void launch_attention_rows_t(const AttnArgs &a, hipStream_t s) {
  dim3 grid(a.nwork * a.heads), block(64 * ATTN_WAVES);
  if (a.sliding)
    hipLaunchKernelGGL((attention_kernel<T, ATTN_WAVES, ATTN_QT, true, true>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((attention_kernel<T, ATTN_WAVES, ATTN_QT, false, true>), grid, block, 0, s, a);
}

hipError_t launch_attention(int precision, const AttnArgs &a, hipStream_t s) {
  if (a.nwork <= 0) return hipSuccess;
  // Sliding-window layers take ATTN_QT; global layers ATTN_QT or (their
  // inference layout) ATTN_QT_GLOBAL.
  if (a.qt != ATTN_QT && (a.sliding || a.qt != ATTN_QT_GLOBAL)) return hipErrorInvalidValue;
  if (precision == PREC_BF16) launch_attention_t<bf16>(a, s);
  else if (precision == PREC_F16) launch_attention_t<f16>(a, s);
  else launch_attention_t<float>(a, s);
  return hipGetLastError();
}

hipError_t launch_attention_rows(int precision, const AttnArgs &a, hipStream_t s) {
  if (a.nwork <= 0) return hipSuccess;
  if (a.qt != ATTN_QT) return hipErrorInvalidValue;
  if (precision == PREC_BF16) launch_attention_rows_t<bf16>(a, s);
  else if (precision == PREC_F16) launch_attention_rows_t<f16>(a, s);
  else launch_attention_rows_t<float>(a, s);
  return hipGetLastError();
}

hipError_t launch_row_items(const int *row_tok, int R, const int *seq_off, int nseq, int T, int4 *items, int *rows,
                            int *nitems, hipStream_t s) {
  if (nseq <= 0 || nseq > ROW_ITEMS_MAXSEQ || R <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(row_items_kernel, dim3(1), dim3(1024), 0, s, row_tok, R, seq_off, nseq, T, items, rows, nitems);
  return hipGetLastError();
}

hipError_t launch_tile_codes(const ChunkInfo *chunks, const int4 *work, const int *seq_len, const int *chunk_off,
                             int nwork, int sliding, int half_window, uint32_t *codes, int *first, hipStream_t s,
                             int nc) {
  if (nwork <= 0) return hipSuccess;
  const dim3 grid(nwork, sliding < 0 ? 2 : 1);
  if (nc == ATTN_WAVES * ATTN_QT)
    hipLaunchKernelGGL(tile_codes_kernel<ATTN_WAVES * ATTN_QT>, grid, dim3(64), 0, s, chunks, work, seq_len,
                       chunk_off, sliding, half_window, codes, first);
  else if (nc == ATTN_WAVES * ATTN_QT_GLOBAL)
    hipLaunchKernelGGL(tile_codes_kernel<ATTN_WAVES * ATTN_QT_GLOBAL>, grid, dim3(64), 0, s, chunks, work,
                       seq_len, chunk_off, sliding, half_window, codes, first);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}




hipError_t launch_attention_bwd(int precision, const AttnBwdArgs &a, hipStream_t s) {
  if (a.nwork <= 0) return hipSuccess;
  static_assert(ATTN_QUERIES == 128 && ATTN_WAVES == 4, "backward kernels use 4-wave, 128-token work items");
  dim3 grid(a.nwork * a.heads), block(256);
  if (precision == PREC_F16) return hipErrorInvalidValue;  // training: fp32 and bf16
  if (precision == PREC_BF16) {
    hipLaunchKernelGGL(attn_bwd_dq_kernel<bf16>, grid, block, 0, s, a);
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel<bf16>, grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL(attn_bwd_dq_kernel<float>, grid, block, 0, s, a);
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel<float>, grid, block, 0, s, a);
  }
  return hipGetLastError();
}
