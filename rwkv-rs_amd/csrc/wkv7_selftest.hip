// Self-test of two bf16 building blocks whose results rest on how this
// toolchain lowers them, run on the device exactly as the kernels run them:
//
// - chunk::split2 (wkv7_chunk.hpp): an fp32 value as bf16 hi and lo parts,
//   hi = RNE(x), lo = RNE(x - hi), the residual from one bf16 dot product
//   with the constant pair (-1, -0). The chunked kernels form every product
//   of two fp32 operands from these parts. Encoded as the inline constant
//   -1.0, the pair would be read as another 16-bit value.
// - add_rb (wkv7_device.hpp): RNE(x) + RNE(p) as an fp32 value, by one
//   packed conversion and a bf16 dot product with (1, 1). The bf16-state
//   decode forms each rounded sum with it and rounds the result to bf16.
//
// The test that calls this (tests/test_gpu_selftest.py) holds the split
// bit for bit to fp32 subtraction, and the sum's bf16 rounding bit for bit
// to that of the fp32 addition, on edge values.
#include "wkv7_chunk.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

__global__ __launch_bounds__(256) void bf16_ops_selftest_kernel(const float* a, const float* b,
                                                                int64_t n, uint32_t* split,
                                                                float* sum) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t hi, lo;
  chunk::split2(a[i], b[i], hi, lo);
  split[2 * i] = hi;
  split[2 * i + 1] = lo;
  sum[i] = add_rb(a[i], b[i]);
}

}  // namespace

hipError_t launch_bf16_ops_selftest(const float* a, const float* b, int64_t n, uint32_t* split,
                                    float* sum, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(bf16_ops_selftest_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a, b,
                     n, split, sum);
  return hipGetLastError();
}

}  // namespace wkv7
