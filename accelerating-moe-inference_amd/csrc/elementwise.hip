// Elementwise ops of the expert MLP (the reference's tensor_ops::silu and
// tensor_ops::mul, src/tensor.cu:163-173).  The grouped expert GEMM fuses
// both into its epilogue; these standalone kernels serve the drop-in
// tensor_ops API.  HBM-bound: grid-stride, one element per lane per step.
#include "common.hpp"

namespace moe {
namespace {

__global__ __launch_bounds__(256) void silu_kernel(const float* x, float* y, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        const float v = x[i];
        y[i] = v / (1.0f + static_cast<float>(exp(-static_cast<double>(v))));
    }
}

__global__ __launch_bounds__(256) void mul_kernel(const float* a, const float* b, float* c,
                                                  int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        c[i] = a[i] * b[i];
}

unsigned grid_for(int64_t n) {
    const int64_t blocks = ceil_div(n, 256);
    return static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
}

}  // namespace

void launch_silu(const float* x, float* y, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(silu_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, y, n);
}

void launch_mul(const float* a, const float* b, float* c, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(mul_kernel, dim3(grid_for(n)), dim3(256), 0, s, a, b, c, n);
}

}  // namespace moe
