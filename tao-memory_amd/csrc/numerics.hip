// Numerics self-test: evaluates the library's bf16 exp / log (tao_common.h)
// on caller-given bf16 inputs, so tests can check them exhaustively (every
// call site in the kernels rounds its argument to bf16 first, so the 65536
// bf16 bit patterns are the whole input domain), and its two 64-lane fp32
// fold sums on caller-given groups.
#include "tao_launch.h"
#include "tao_common.h"

namespace tao {
namespace {

__global__ __launch_bounds__(kThreads) void numerics_kernel(int op, const bf16_t* x, bf16_t* y,
                                                            int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const float v = bf2f(x[i]);
  y[i] = f2bf(op == 0 ? exp_bf(v) : log_bf(v));
}

// One wave per 64 fp32 values: op 2 = wave_fold_sum on the bit-reversed
// layout, op 3 = wave_sum_fold on the natural layout.
__global__ __launch_bounds__(64) void fold_test_kernel(int op, const float* x, float* y) {
  const int lane = threadIdx.x;
  const float* g = x + (int64_t)blockIdx.x * 64;
  const float r = op == 2 ? wave_fold_sum(g[fold_lane(lane)]) : wave_sum_fold(g[lane]);
  if (lane == 0) y[blockIdx.x] = r;
}

}  // namespace
}  // namespace tao

extern "C" int tao_numerics_selftest(int32_t op, const void* x, void* y, int64_t n, void* stream) {
  if (op < 0 || op > 3 || n < 0 || (n && (!x || !y)) || (op >= 2 && n % 64)) {
    tao::set_error("numerics self-test: op 0 (exp) or 1 (log) on bf16, 2 or 3 (64-lane fold "
                   "sums) on fp32 groups of 64, with non-null buffers");
    return TAO_E_ARGUMENT;
  }
  if (n == 0) return TAO_OK;
  if (op >= 2) {
    if (n / 64 > 0x7FFFFFFF) {
      tao::set_error("numerics self-test: too many groups");
      return TAO_E_ARGUMENT;
    }
    hipLaunchKernelGGL(tao::fold_test_kernel, dim3((unsigned)(n / 64)), dim3(64), 0,
                       (hipStream_t)stream, op, (const float*)x, (float*)y);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      tao::set_error(hipGetErrorString(e));
      return (int)e;
    }
    return TAO_OK;
  }
  const int64_t blocks = (n + tao::kThreads - 1) / tao::kThreads;
  if (blocks > 0x7FFFFFFF) {
    tao::set_error("numerics self-test: too many elements");
    return TAO_E_ARGUMENT;
  }
  hipLaunchKernelGGL(tao::numerics_kernel, dim3((unsigned)blocks), dim3(tao::kThreads), 0,
                     (hipStream_t)stream, op, (const bf16_t*)x, (bf16_t*)y, n);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    tao::set_error(hipGetErrorString(e));
    return (int)e;
  }
  return TAO_OK;
}
