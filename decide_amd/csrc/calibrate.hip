// Attainable MFMA rate on this GPU for the data the projection GEMMs
// multiply. A register-only loop of v_mfma_f32_32x32x16_bf16 (bf16),
// v_mfma_f32_32x32x16_f16 (fp16) or v_mfma_f32_32x32x2_f32 (fp32, the
// validation mode and dn_gemm_f32) in the
// GEMMs' wave pattern (2 x 3 accumulator tiles, 2 k steps, B as the first
// operand), two waves per SIMD on every CU, no memory traffic. The operands are drawn
// like the forward's: activations ~ N(0, 1) against weights ~ N(0, 0.02).
// With mode 0 (bf16), 2 (fp32) and 4 (fp16) they are rotated one lane every
// iteration, so each MFMA sees new values with the same statistics, as in a
// real GEMM; modes 1, 3 and 5 keep them constant. The matrix core's rate depends on how much its inputs toggle
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
__device__ __forceinline__ float normalish(uint32_t &state, float sd) {
  state = mix32(state + 0x9e3779b9u);
  const float s = (float)(state & 255) + (float)((state >> 8) & 255) + (float)((state >> 16) & 255) +
                  (float)(state >> 24);
  return (s - 510.0f) * (sd / 147.8f);
}

// One MFMA operand of normalish values.
__device__ __forceinline__ void fill(bf16x8 &v, uint32_t &st, float sd) {
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = (bf16)normalish(st, sd);
}
__device__ __forceinline__ void fill(f16x8 &v, uint32_t &st, float sd) {
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = (f16)normalish(st, sd);
}
__device__ __forceinline__ void fill(float &v, uint32_t &st, float sd) { v = normalish(st, sd); }

__device__ __forceinline__ int ror1(int w) { return __builtin_amdgcn_mov_dpp(w, 0x121, 0xf, 0xf, false); }  // row_ror:1
template <class V>
__device__ __forceinline__ V rotate_lanes(V v) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  static_assert(sizeof(V) == sizeof(i32x4), "8 x 16-bit operand");
  i32x4 w = __builtin_bit_cast(i32x4, v);
#pragma unroll
  for (int e = 0; e < 4; e++) w[e] = ror1(w[e]);
  return __builtin_bit_cast(V, w);
}
__device__ __forceinline__ float rotate_lanes(float v) { return __int_as_float(ror1(__float_as_int(v))); }

template <int MODE, class T>
__global__ __launch_bounds__(256) void mfma_calibrate_kernel(int iters, uint32_t seed, float *sink) {
  using MF = Mfma<T>;
  typedef typename MF::frag frag;
  uint32_t st = mix32(seed ^ (blockIdx.x * 256u + threadIdx.x));
  frag a[2][2][2], b[2][2][3];  // [operand set][k step][tile]
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
#pragma unroll
    for (int i = 0; i < 2; i++) fill(a[0][ks][i], st, 1.0f);
#pragma unroll
    for (int j = 0; j < 3; j++) fill(b[0][ks][j], st, 0.02f);
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
          for (int j = 0; j < 3; j++) acc[i][j] = MF::mma(b[p][ks][j], a[p][ks][i], acc[i][j]);
      if constexpr (MODE % 2 == 0) {
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

// MFMAs per thread-block iteration: 2 operand sets x 12 per wave, 4 waves;
// 32x32x16 (bf16, modes 0 and 1; fp16, modes 4 and 5) or 32x32x2 (fp32,
// modes 2 and 3) each.
double mfma_calibrate_flop(int mode, int blocks, int iters) {
  return (double)blocks * 4 * iters * 24 * (mode == 2 || mode == 3 ? 4096.0 : 32768.0);
}

hipError_t launch_mfma_calibrate(int mode, int blocks, int iters, float *sink, hipStream_t s) {
  switch (mode) {
    case 0:
      hipLaunchKernelGGL((mfma_calibrate_kernel<0, bf16>), dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
      break;
    case 1:
      hipLaunchKernelGGL((mfma_calibrate_kernel<1, bf16>), dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
      break;
    case 2:
      hipLaunchKernelGGL((mfma_calibrate_kernel<2, float>), dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
      break;
    case 3:
      hipLaunchKernelGGL((mfma_calibrate_kernel<3, float>), dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
      break;
    case 4:
      hipLaunchKernelGGL((mfma_calibrate_kernel<4, f16>), dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
      break;
    default:
      hipLaunchKernelGGL((mfma_calibrate_kernel<5, f16>), dim3(blocks), dim3(256), 0, s, iters, 12345u, sink);
      break;
  }
  return hipGetLastError();
}
