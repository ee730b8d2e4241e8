// Non-template backward kernels: the deterministic dscale reduction and the
// zero fill used for empty problems.
#include "born_bwd.h"
#include "born_launch.h"

namespace qdl {

// dscale[out] = (2 / s) * eps * sum delta / Z over the rows of that output,
// in a fixed order (double accumulation, fixed tree).
__global__ __launch_bounds__(256) void born_bwd_dscale_kernel(BwdArgs p) {
    __shared__ double red[256];
    const int out = blockIdx.x;
    const int tid = threadIdx.x;
    double acc = 0.0;
    if (p.per_head_scale) {
        const int64_t n = (int64_t)p.B * p.T;
        for (int64_t j = tid; j < n; j += 256) {
            const int64_t b = j / p.T, i = j % p.T;
            acc += (double)p.delta_z[(b * p.H + out) * p.T + i];
        }
    } else {
        const int64_t n = (int64_t)p.B * p.H * p.T;
        for (int64_t j = tid; j < n; j += 256) acc += (double)p.delta_z[j];
    }
    red[tid] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] += red[tid + w];
        __syncthreads();
    }
    if (tid == 0) {
        const float s = p.scale[out];
        p.dscale[out] = (s == 0.f) ? 0.f : (float)(2.0 / (double)s * (double)p.eps * red[0]);
    }
}

__global__ void born_zero_fill_kernel(float* __restrict__ x, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        x[i] = 0.f;
}

hipError_t launch_bwd_common_post(const BwdArgs& a, hipStream_t st) {
    const int nout = a.per_head_scale ? a.H : 1;
    hipLaunchKernelGGL(born_bwd_dscale_kernel, dim3(nout), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t zero_fill(float* p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(born_zero_fill_kernel, dim3(blocks), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

}  // namespace qdl
