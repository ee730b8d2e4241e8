#include "born_launch.h"
namespace qdl {
hipError_t bwd_launch_bf16(const BwdArgs&, hipStream_t) { return hipErrorNotSupported; }
hipError_t bwd_launch_f16(const BwdArgs&, hipStream_t) { return hipErrorNotSupported; }
hipError_t bwd_launch_f32(const BwdArgs&, hipStream_t) { return hipErrorNotSupported; }
}
namespace qdl {
__global__ void zero_fill_kernel(float* p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0.f;
}
hipError_t zero_fill(float* p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int blocks = (int)((n + 255) / 256); if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, s, p, n);
    return hipGetLastError();
}
}
