// Sustained MFMA rate of this GPU, for the roofline context of bench.py (--probe peak): not part of the
// libkh C ABI. Each wave issues 32 independent-accumulator v_mfma_f32_32x32x16_f16 per iteration on
// operands held in registers (no memory traffic in the loop). With `vary` set, the operands are random
// fp16 values from `ops` and their mantissas flip every iteration, as the operands of a real GEMM change
// from one MFMA to the next; otherwise every MFMA sees the same operands. The two rates differ by the
// data-dependent power the MFMA units draw, which sets the clock the chip sustains.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int THREADS = 512;

// ops: n_slots x THREADS x 8 16-byte operands; workgroup g reads slot g % n_slots
__global__ __launch_bounds__(THREADS) void mfma_rate_kernel(const u32x4* __restrict__ ops, int n_slots, int iters,
                                                            int vary, float* __restrict__ sink) {
  const u32x4* src = ops + ((size_t)(blockIdx.x % n_slots) * THREADS + threadIdx.x) * 8;
  u32x4 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[i] = src[i];
    b[i] = src[4 + i];
  }
  const uint32_t flip = vary ? 0x01ff01ffu : 0u;
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = (f32x16){};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int i = 0; i < 8; i++)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[(i + r) & 3]),
                                                        __builtin_bit_cast(f16x8, b[(i + 2 * r + 1) & 3]), acc[i], 0,
                                                        0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) a[i] ^= flip;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) s += acc[i][0] + acc[i][15];
  if (s == 1234567.0f) sink[threadIdx.x] = s;  // keeps the loop live; practically never taken
}

}  // namespace

extern "C" {

// Launches `grid` workgroups of 512 threads, each running `iters` x 32 MFMAs (32 x 32 x 16 f16: 32768 FLOP
// each) on `stream`. ops: n_slots x 512 x 8 16-byte operands; sink: 512 floats. Returns a hipError_t.
int kh_probe_mfma_rate(void* stream, const void* ops, int n_slots, int grid, int iters, int vary, float* sink) {
  if (!ops || !sink || n_slots <= 0 || grid <= 0 || iters <= 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(grid), dim3(THREADS), 0, (hipStream_t)stream, (const u32x4*)ops, n_slots,
                     iters, vary, sink);
  return (int)hipGetLastError();
}

}  // extern "C"
