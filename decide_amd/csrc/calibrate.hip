// Attainable bf16 MFMA rate on this GPU for the data the projection GEMMs
// multiply. A register-only loop of v_mfma_f32_32x32x16_bf16 in the GEMMs'
// wave pattern (2 x 3 accumulator tiles, 2 k steps, B as the first operand),
// two waves per SIMD on every CU, no memory traffic. The operands are drawn
// like the forward's: activations ~ N(0, 1) against weights ~ N(0, 0.02).
// With mode 0 they are rotated one lane every iteration, so each MFMA sees
// new values with the same statistics, as in a real GEMM; mode 1 keeps them
// constant. The matrix core's rate depends on how much its inputs toggle
// (power), so mode 0 is the ceiling a real GEMM can approach and mode 1
// the rate quoted by register-only benchmarks.
#include "common.hpp"

namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Roughly N(0, sd): the sum of four uniform bytes (Irwin-Hall), centred.
__device__ __forceinline__ bf16 normalish(uint32_t &state, float sd) {
  state = mix32(state + 0x9e3779b9u);
  const float s = (float)(state & 255) + (float)((state >> 8) & 255) + (float)((state >> 16) & 255) +
                  (float)(state >> 24);
  return (bf16)((s - 510.0f) * (sd / 147.8f));
}

__device__ __forceinline__ bf16x8 rotate_lanes(bf16x8 v) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 w = __builtin_bit_cast(i32x4, v);
#pragma unroll
  for (int e = 0; e < 4; e++) w[e] = __builtin_amdgcn_mov_dpp(w[e], 0x121, 0xf, 0xf, false);  // row_ror:1
  return __builtin_bit_cast(bf16x8, w);
}

template <int MODE>
__global__ __launch_bounds__(256) void mfma_calibrate_kernel(int iters, uint32_t seed, float *sink) {
  uint32_t st = mix32(seed ^ (blockIdx.x * 256u + threadIdx.x));
  bf16x8 a[2][2][2], b[2][2][3];  // [operand set][k step][tile]
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 8; e++) a[0][ks][i][e] = normalish(st, 1.0f);
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
      for (int e = 0; e < 8; e++) b[0][ks][j][e] = normalish(st, 0.02f);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
#pragma unroll
    for (int i = 0; i < 2; i++) a[1][ks][i] = a[0][ks][i];
#pragma unroll
    for (int j = 0; j < 3; j++) b[1][ks][j] = b[0][ks][j];
  }
  f32x16 acc[2][3];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 3; j++) acc[i][j] = f32x16{};
  // Two operand sets: the MFMAs of one iteration read set p while the next
  // iteration's operands are rotated into set p ^ 1.
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int p = 0; p < 2; p++) {
#pragma unroll
      for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
          for (int j = 0; j < 3; j++) acc[i][j] = Mfma<bf16>::mma(b[p][ks][j], a[p][ks][i], acc[i][j]);
      if constexpr (MODE == 0) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
#pragma unroll
          for (int i = 0; i < 2; i++) a[p ^ 1][ks][i] = rotate_lanes(a[p][ks][i]);
#pragma unroll
          for (int j = 0; j < 3; j++) b[p ^ 1][ks][j] = rotate_lanes(b[p][ks][j]);
        }
      }
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) s += acc[i][j][e];
  if (s == 1234.5f) sink[threadIdx.x] = s;  // keeps the accumulators live; never true in practice
}

}  // namespace

// MFMAs per thread-block iteration: 2 operand sets x 12 per wave, 4 waves.
double mfma_calibrate_flop(int blocks, int iters) { return (double)blocks * 4 * iters * 24 * 32768.0; }

hipError_t launch_mfma_calibrate(int mode, int blocks, int iters, float *sink, hipStream_t s) {
  if (mode == 0)
    hipLaunchKernelGGL(mfma_calibrate_kernel<0>, dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
  else
    hipLaunchKernelGGL(mfma_calibrate_kernel<1>, dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
  return hipGetLastError();
}
