// Kernel argument block of the purified-Born kernels (purified.h).
#pragma once

#include <stdint.h>

namespace qdl {

struct PurArgs {
    const void* q;
    const void* k;
    const void* v;
    float* o;            // forward: (B, H, T, D) fp32 output
    float* z;            // forward: (B, H, T) fp32, Z = sum p + eps
    const float* o_in;   // backward: the forward's fp32 output
    const void* dout;    // backward: upstream gradient, input dtype
    const float* z_in;   // backward: the forward's Z
    const float* scale;  // gamma: 1 or H values
    const float* tau;    // tau: 1 or H values
    const int32_t* doc;  // (B, T) or nullptr
    void* dq;
    void* dk;
    void* dv;
    float* dscale;       // n_scale outputs
    float* dtau;         // n_tau outputs
    float* ndelta;       // workspace (B, H, T): -delta
    float* zinv;         // workspace (B, H, T): 1 / Z
    float* part;         // workspace: 2 x (dK/dV workgroups) partial sums
    int per_head_scale;
    int per_head_tau;
    int B, H, T, D;
    int is_causal;
    int window;
    float eps;
    float eps_base;
};

}  // namespace qdl
