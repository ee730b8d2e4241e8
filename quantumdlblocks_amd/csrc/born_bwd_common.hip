// Non-template backward kernels: the deterministic dscale reduction and the
// zero fill used for empty problems.
#include "born_bwd.h"
#include "born_launch.h"

namespace qdl {

// dscale[out] = (2 / s) * eps * sum delta / Z over the rows of that output.
// Two fixed-order stages (no atomics, so the result is bitwise reproducible):
// stage 1 sums DSCALE_CHUNKS contiguous chunks of each output's rows into
// double partials, stage 2 adds the partials in order.
__global__ __launch_bounds__(256) void born_bwd_dscale_partial_kernel(BwdArgs p, double* part) {
    __shared__ double red[256];
    const int out = blockIdx.y;
    const int chunk = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t n = p.per_head_scale ? (int64_t)p.B * p.T : (int64_t)p.B * p.H * p.T;
    const int64_t len = (n + DSCALE_CHUNKS - 1) / DSCALE_CHUNKS;
    const int64_t lo = chunk * len;
    const int64_t hi = lo + len < n ? lo + len : n;
    double acc = 0.0;
    for (int64_t j = lo + tid; j < hi; j += 256) {
        int64_t idx = j;
        if (p.per_head_scale) {
            const int64_t b = j / p.T, i = j % p.T;
            idx = (b * p.H + out) * p.T + i;
        }
        acc += (double)p.delta_z[idx];
    }
    red[tid] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] += red[tid + w];
        __syncthreads();
    }
    if (tid == 0) part[out * DSCALE_CHUNKS + chunk] = red[0];
}

__global__ __launch_bounds__(64) void born_bwd_dscale_final_kernel(BwdArgs p, const double* part) {
    const int out = blockIdx.x;
    if (threadIdx.x != 0) return;
    double acc = 0.0;
    for (int c = 0; c < DSCALE_CHUNKS; ++c) acc += part[out * DSCALE_CHUNKS + c];
    const float s = p.scale[out];
    p.dscale[out] = (s == 0.f) ? 0.f : (float)(2.0 / (double)s * (double)p.eps * acc);
}

__global__ void born_zero_fill_kernel(float* __restrict__ x, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        x[i] = 0.f;
}

hipError_t launch_bwd_common_post(const BwdArgs& a, hipStream_t st) {
    const int nout = a.per_head_scale ? a.H : 1;
    hipLaunchKernelGGL(born_bwd_dscale_partial_kernel, dim3(DSCALE_CHUNKS, nout), dim3(256), 0, st, a,
                       a.dscale_part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(born_bwd_dscale_final_kernel, dim3(nout), dim3(64), 0, st, a,
                       (const double*)a.dscale_part);
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
