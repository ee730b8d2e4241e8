// Fused Q/K prologue: unitary RoPE then L2 normalisation, one pass per row,
// forward and backward (C ABI declared in include/qdl_flash_born.h).
//
// Reference: SubspaceProjectorBornAttention.forward, attention.py:573-589;
// apply_unitary_rope, functional.py:104-121; l2_normalize and its
// memory-efficient autograd function, functional.py:36-80.
//
// HBM-bound streaming kernels.  A row (one (b, h, t) of q or k) is handled by
// a group of LPR consecutive lanes (a power of two); lane j of the group owns
// column chunks j, j + LPR, ... of the first half (VEC elements each) and the
// matching chunks of the second half, i.e. both members of every rotation pair
// it touches.  The row's fp32 sum is reduced across the group with xor
// shuffles.  Rows of one (b, h) are consecutive in the grid, so a workgroup
// reads 256 / LPR consecutive rows of the rotary table.
//
// Rounding.  For bf16 / fp16 every intermediate the reference materialises as
// a 16-bit tensor is rounded to the dtype here too (round to nearest even):
// the table entries (cos.to(x.dtype)), each product, each sum or difference,
// the rotated row, the normalised row; the backward rounds the L2 gradient and
// each product and sum of the transposed rotation the way autograd's 16-bit
// ops do.  The reference rounds each tensor op separately, so no product and
// sum may be contracted into one fused operation: contraction is off for the
// arithmetic written in this file (the pragma below; operations inside
// library helpers carry their own contraction flags, so none are used here),
// which also keeps the compiler from fusing the native fp16 ops it narrows
// "fp32 op on fp16 values, then round to fp16" into.
#include <math.h>
#include <stdint.h>

#include "../../include/qdl_flash_born.h"
#include "born_common.h"

#pragma clang fp contract(off)

namespace qdl {
namespace {

// An fp32 value materialised in a register.  Rounding it to fp16 afterwards
// is then two roundings (fp32 op, then fp16), as in the reference; without
// it the compiler may fold "fp32 multiply, round to fp16" into one
// mixed-precision instruction that rounds the exact product once.
__device__ __forceinline__ float as_f32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

template <class E>
struct RowIO;

template <>
struct RowIO<BF16> {
    static constexpr int kBytes = 2;
    __device__ __forceinline__ static float rnd(float x) { return BF16::lo(BF16::pack(x, 0.f)); }
    __device__ __forceinline__ static void rnd2(float& x, float& y) {
        const uint32_t u = BF16::pack(x, y);
        x = BF16::lo(u);
        y = BF16::hi(u);
    }
    __device__ __forceinline__ static void load(const void* p, int n, float* v) {
        if (n == 8) {
            const u32x4 u = ldg16(p);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = BF16::lo(u[i]);
                v[2 * i + 1] = BF16::hi(u[i]);
            }
        } else {
            v[0] = __uint_as_float((uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
        }
    }
    __device__ __forceinline__ static void store(void* p, int n, const float* v) {
        if (n == 8) {
            u32x4 u;
#pragma unroll
            for (int i = 0; i < 4; ++i) u[i] = BF16::pack(v[2 * i], v[2 * i + 1]);
            *reinterpret_cast<u32x4*>(p) = u;
        } else {
            *reinterpret_cast<uint16_t*>(p) = (uint16_t)(BF16::pack(v[0], 0.f) & 0xffffu);
        }
    }
};

template <>
struct RowIO<F16> {
    static constexpr int kBytes = 2;
    __device__ __forceinline__ static float rnd(float x) { return F16::lo(F16::pack(as_f32(x), 0.f)); }
    __device__ __forceinline__ static void rnd2(float& x, float& y) {
        const uint32_t u = F16::pack(as_f32(x), as_f32(y));
        x = F16::lo(u);
        y = F16::hi(u);
    }
    __device__ __forceinline__ static void load(const void* p, int n, float* v) {
        if (n == 8) {
            const u32x4 u = ldg16(p);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = F16::lo(u[i]);
                v[2 * i + 1] = F16::hi(u[i]);
            }
        } else {
            v[0] = (float)*reinterpret_cast<const _Float16*>(p);
        }
    }
    __device__ __forceinline__ static void store(void* p, int n, const float* v) {
        if (n == 8) {
            u32x4 u;
#pragma unroll
            for (int i = 0; i < 4; ++i) u[i] = F16::pack(as_f32(v[2 * i]), as_f32(v[2 * i + 1]));
            *reinterpret_cast<u32x4*>(p) = u;
        } else {
            *reinterpret_cast<uint16_t*>(p) = (uint16_t)(F16::pack(as_f32(v[0]), 0.f) & 0xffffu);
        }
    }
};

struct F32Tag {};

template <>
struct RowIO<F32Tag> {
    static constexpr int kBytes = 4;
    __device__ __forceinline__ static float rnd(float x) { return x; }
    __device__ __forceinline__ static void rnd2(float&, float&) {}
    __device__ __forceinline__ static void load(const void* p, int n, float* v) {
        if (n == 4) {
            const f32x4 u = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = u[i];
        } else {
            v[0] = *reinterpret_cast<const float*>(p);
        }
    }
    __device__ __forceinline__ static void store(void* p, int n, const float* v) {
        if (n == 4) {
            const f32x4 u = {v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(p) = u;
        } else {
            *reinterpret_cast<float*>(p) = v[0];
        }
    }
};

struct RowRef {
    const void* p;
    int64_t sb, sh, st;  // element strides
};

struct PrologueArgs {
    // Forward: src = q / k (strided), dst = q_out / k_out (contiguous).
    // Backward: src = dq_out / dk_out, aux = q_out / k_out (both contiguous),
    //           dst = dq / dk (strided).
    RowRef src[2];
    RowRef aux[2];
    RowRef dst[2];
    float* rinv_out[2];
    const float* rinv_in[2];
    const float* cos;
    const float* sin;
    int64_t ld;
    int nfreq;
    int B, H, T, D;
    int lpr;      // lanes per row (power of two, <= 64)
    int tab_vec;  // table rows can be read 16 bytes at a time
    float eps;
};

// Position of grid row `row`: rows run in (b, h, t) order, so the rows of a
// workgroup are consecutive time steps of one head.  (A (b, t, h) order for
// the projection layout, reading its rows contiguously, measured no faster.)
struct RowPos {
    int b, h, t;
    int lin;  // (b H + h) T + t: index into the contiguous tensors and 1/norm
};

__device__ __forceinline__ RowPos row_pos(const PrologueArgs& p, int row) {
    RowPos r;
    r.t = row % p.T;
    const int bh = row / p.T;
    r.h = bh % p.H;
    r.b = bh / p.H;
    r.lin = row;
    return r;
}

__device__ __forceinline__ int64_t row_off(const RowRef& r, const RowPos& q) {
    return (int64_t)q.b * r.sb + (int64_t)q.h * r.sh + (int64_t)q.t * r.st;
}

// cos / sin of pairs i0 .. i0 + n - 1 of table row t, rounded to the dtype;
// pairs past nfreq rotate by angle 0.
template <class IO, int VEC>
__device__ __forceinline__ void load_table(const PrologueArgs& p, int t, int i0, float* c, float* s) {
    const float* cr = p.cos + (int64_t)t * p.ld + i0;
    const float* sr = p.sin + (int64_t)t * p.ld + i0;
    if (VEC % 4 == 0 && p.tab_vec && i0 + VEC <= p.nfreq) {
#pragma unroll
        for (int v = 0; v < VEC; v += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(cr + v);
            const f32x4 b = *reinterpret_cast<const f32x4*>(sr + v);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                c[v + i] = a[i];
                s[v + i] = b[i];
            }
        }
    } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            const bool in = i0 + v < p.nfreq;
            c[v] = in ? cr[v] : 1.f;
            s[v] = in ? sr[v] : 0.f;
        }
    }
#pragma unroll
    for (int v = 0; v < VEC; v += 2) {
        if (VEC == 1) {
            c[0] = IO::rnd(c[0]);
            s[0] = IO::rnd(s[0]);
        } else {
            IO::rnd2(c[v], c[v + 1]);
            IO::rnd2(s[v], s[v + 1]);
        }
    }
}

__device__ __forceinline__ float group_sum(float v, int lpr) {
    for (int m = 1; m < lpr; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Forward.  grid (ceil(rows / (256 / lpr)), 2): y = 0 for q, 1 for k.
// MAXC = column chunks per lane at most; ROPE = rotate (tables given).  The
// rotation is a template switch so that the table loads issue straight after
// the row loads (a runtime test measured ~9% slower at D = 64).
template <class IO, int VEC, int MAXC, bool ROPE>
__global__ __launch_bounds__(256) void qk_prologue_fwd_kernel(PrologueArgs p) {
    const int which = blockIdx.y;
    if (p.src[which].p == nullptr) return;
    const int lpr = p.lpr;
    const int rows = p.B * p.H * p.T;
    const int row = blockIdx.x * (256 / lpr) + threadIdx.x / lpr;
    const int j0 = threadIdx.x & (lpr - 1);
    if (row >= rows) return;  // whole row groups leave together
    const int half = p.D >> 1;
    const int nch = half / VEC;
    const RowPos pos = row_pos(p, row);
    const int t = pos.t;
    const char* src = static_cast<const char*>(p.src[which].p) + row_off(p.src[which], pos) * IO::kBytes;

    float y1[MAXC][VEC], y2[MAXC][VEC];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int j = j0 + c * lpr;
        if (j < nch) {
            float x1[VEC], x2[VEC];
            IO::load(src + (int64_t)j * VEC * IO::kBytes, VEC, x1);
            IO::load(src + (int64_t)(half + j * VEC) * IO::kBytes, VEC, x2);
            if (ROPE) {
                float cs[VEC], sn[VEC];
                load_table<IO, VEC>(p, t, j * VEC, cs, sn);
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    const float a = IO::rnd(x1[v] * cs[v]);
                    const float b = IO::rnd(x2[v] * sn[v]);
                    const float e = IO::rnd(x1[v] * sn[v]);
                    const float f = IO::rnd(x2[v] * cs[v]);
                    y1[c][v] = IO::rnd(a - b);
                    y2[c][v] = IO::rnd(e + f);
                }
            } else {
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    y1[c][v] = x1[v];
                    y2[c][v] = x2[v];
                }
            }
#pragma unroll
            for (int v = 0; v < VEC; ++v) ss = fmaf(y1[c][v], y1[c][v], fmaf(y2[c][v], y2[c][v], ss));
        }
    }
    ss = group_sum(ss, lpr);
    // 1 / sqrt(sum + eps): the sum plus eps rounded to fp32 as the reference's
    // fp32 tensor add rounds it, the reciprocal root correctly rounded.
    const float se = ss + p.eps;
    const float rinv = (float)(1.0 / sqrt((double)se));

    char* dst = static_cast<char*>(const_cast<void*>(p.dst[which].p)) + row_off(p.dst[which], pos) * IO::kBytes;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int j = j0 + c * lpr;
        if (j < nch) {
            float o1[VEC], o2[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                o1[v] = y1[c][v] * rinv;
                o2[v] = y2[c][v] * rinv;
            }
            IO::store(dst + (int64_t)j * VEC * IO::kBytes, VEC, o1);
            IO::store(dst + (int64_t)(half + j * VEC) * IO::kBytes, VEC, o2);
        }
    }
    if (j0 == 0 && p.rinv_out[which] != nullptr) p.rinv_out[which][pos.lin] = rinv;
}

// Backward.  Same grid and lane mapping as the forward.
template <class IO, int VEC, int MAXC, bool ROPE>
__global__ __launch_bounds__(256) void qk_prologue_bwd_kernel(PrologueArgs p) {
    const int which = blockIdx.y;
    if (p.src[which].p == nullptr) return;
    const int lpr = p.lpr;
    const int rows = p.B * p.H * p.T;
    const int row = blockIdx.x * (256 / lpr) + threadIdx.x / lpr;
    const int j0 = threadIdx.x & (lpr - 1);
    if (row >= rows) return;
    const int half = p.D >> 1;
    const int nch = half / VEC;
    const RowPos pos = row_pos(p, row);
    const int t = pos.t;
    const char* gp = static_cast<const char*>(p.src[which].p) + row_off(p.src[which], pos) * IO::kBytes;
    const char* yp = static_cast<const char*>(p.aux[which].p) + row_off(p.aux[which], pos) * IO::kBytes;
    const float rinv = p.rinv_in[which][pos.lin];

    float g1[MAXC][VEC], g2[MAXC][VEC], y1[MAXC][VEC], y2[MAXC][VEC];
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int j = j0 + c * lpr;
        if (j < nch) {
            IO::load(gp + (int64_t)j * VEC * IO::kBytes, VEC, g1[c]);
            IO::load(gp + (int64_t)(half + j * VEC) * IO::kBytes, VEC, g2[c]);
            IO::load(yp + (int64_t)j * VEC * IO::kBytes, VEC, y1[c]);
            IO::load(yp + (int64_t)(half + j * VEC) * IO::kBytes, VEC, y2[c]);
#pragma unroll
            for (int v = 0; v < VEC; ++v) dot = fmaf(g1[c][v], y1[c][v], fmaf(g2[c][v], y2[c][v], dot));
        }
    }
    dot = group_sum(dot, lpr);

    char* dst = static_cast<char*>(const_cast<void*>(p.dst[which].p)) + row_off(p.dst[which], pos) * IO::kBytes;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int j = j0 + c * lpr;
        if (j < nch) {
            float d1[VEC], d2[VEC];
            // L2 backward: ((g - dot y) rinv), rounded to the dtype.
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                d1[v] = IO::rnd((g1[c][v] - dot * y1[c][v]) * rinv);
                d2[v] = IO::rnd((g2[c][v] - dot * y2[c][v]) * rinv);
            }
            if (ROPE) {
                float cs[VEC], sn[VEC];
                load_table<IO, VEC>(p, t, j * VEC, cs, sn);
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    const float a = IO::rnd(d1[v] * cs[v]);
                    const float b = IO::rnd(d2[v] * sn[v]);
                    const float e = IO::rnd(d2[v] * cs[v]);
                    const float f = IO::rnd(d1[v] * sn[v]);
                    d1[v] = (a + b);
                    d2[v] = (e - f);
                }
            }
            IO::store(dst + (int64_t)j * VEC * IO::kBytes, VEC, d1);
            IO::store(dst + (int64_t)(half + j * VEC) * IO::kBytes, VEC, d2);
        }
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int pow2_at_least(int n) {
    int v = 1;
    while (v < n) v <<= 1;
    return v;
}

// Vector width usable for every row tensor of the call (elements of 16 bytes),
// else 1.
bool vec_ok(const PrologueArgs& a, int vec) {
    const int half = a.D / 2;
    if (half % vec) return false;
    for (int w = 0; w < 2; ++w) {
        const RowRef* refs[3] = {&a.src[w], &a.aux[w], &a.dst[w]};
        for (const RowRef* r : refs) {
            if (!r->p) continue;
            if (!aligned16(r->p) || r->sb % vec || r->sh % vec || r->st % vec) return false;
        }
    }
    return true;
}

template <class IO, bool FWD, int VEC, int MAXC>
void launch_kernel(const PrologueArgs& a, dim3 grid, hipStream_t st) {
    if (FWD) {
        if (a.cos)
            hipLaunchKernelGGL((qk_prologue_fwd_kernel<IO, VEC, MAXC, true>), grid, dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((qk_prologue_fwd_kernel<IO, VEC, MAXC, false>), grid, dim3(256), 0, st, a);
    } else {
        if (a.cos)
            hipLaunchKernelGGL((qk_prologue_bwd_kernel<IO, VEC, MAXC, true>), grid, dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((qk_prologue_bwd_kernel<IO, VEC, MAXC, false>), grid, dim3(256), 0, st, a);
    }
}

template <class IO, bool FWD>
hipError_t launch_prologue(PrologueArgs a, hipStream_t st) {
    constexpr int V16 = 16 / IO::kBytes;
    const int half = a.D / 2;
    const bool vec = vec_ok(a, V16);
    const int nch = vec ? half / V16 : half;
    a.lpr = pow2_at_least(nch) < 64 ? pow2_at_least(nch) : 64;
    a.tab_vec = a.cos && aligned16(a.cos) && aligned16(a.sin) && (a.ld % 4 == 0);
    const int rows = a.B * a.H * a.T;
    const int rpb = 256 / a.lpr;
    const dim3 grid((unsigned)((rows + rpb - 1) / rpb), 2);
    if (vec) {
        // half <= 128: at most 16 (bf16 / fp16) or 32 (fp32) chunks, one per lane.
        launch_kernel<IO, FWD, V16, 1>(a, grid, st);
    } else {
        // Scalar columns: half <= 128 chunks over at most 64 lanes.
        launch_kernel<IO, FWD, 1, 2>(a, grid, st);
    }
    return hipGetLastError();
}

template <bool FWD>
hipError_t dispatch(int dtype, const PrologueArgs& a, hipStream_t st) {
    switch (dtype) {
        case QDL_BORN_DTYPE_BF16: return launch_prologue<RowIO<BF16>, FWD>(a, st);
        case QDL_BORN_DTYPE_F16: return launch_prologue<RowIO<F16>, FWD>(a, st);
        default: return launch_prologue<RowIO<F32Tag>, FWD>(a, st);
    }
}

int check_shape(int dtype, int64_t B, int64_t H, int64_t T, int64_t D) {
    if (dtype != QDL_BORN_DTYPE_F32 && dtype != QDL_BORN_DTYPE_F16 && dtype != QDL_BORN_DTYPE_BF16)
        return QDL_BORN_E_DTYPE;
    if (B < 0 || H < 0 || T < 0) return QDL_BORN_E_SHAPE;
    if (B * H * T > ((int64_t)1 << 31) - 256) return QDL_BORN_E_SHAPE;
    if (D < 2 || D > 256 || (D & 1)) return QDL_BORN_E_ROPEDIM;
    return QDL_BORN_OK;
}

int check_table(const float* c, const float* s, int64_t nfreq, int64_t ld, int64_t D) {
    if (!c) return QDL_BORN_OK;
    if (!s) return QDL_BORN_E_NULL;
    if (nfreq < 0 || nfreq > D / 2 || ld < nfreq) return QDL_BORN_E_TABLE;
    return QDL_BORN_OK;
}

RowRef ref(const void* p, const int64_t* strides, int64_t H, int64_t T, int64_t D) {
    RowRef r;
    r.p = p;
    if (strides) {
        r.sb = strides[0];
        r.sh = strides[1];
        r.st = strides[2];
    } else {
        r.st = D;
        r.sh = T * D;
        r.sb = H * T * D;
    }
    return r;
}

int hip_status(hipError_t e) { return e == hipSuccess ? QDL_BORN_OK : (int)e; }

}  // namespace
}  // namespace qdl

extern "C" {

int qdl_flash_born_qk_prologue_fwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                                   const void* q, const int64_t* q_strides, const void* k,
                                   const int64_t* k_strides, const float* cos_table,
                                   const float* sin_table, int64_t n_freq, int64_t table_ld,
                                   double eps, void* q_out, void* k_out, float* q_rinv,
                                   float* k_rinv, qdl_stream_t stream) {
    using namespace qdl;
    int rc = check_shape(dtype, B, H, T, D);
    if (rc != QDL_BORN_OK) return rc;
    rc = check_table(cos_table, sin_table, n_freq, table_ld, D);
    if (rc != QDL_BORN_OK) return rc;
    if (!(eps >= 0.0)) return QDL_BORN_E_SHAPE;
    if (B * H * T == 0 || (!q && !k)) return QDL_BORN_OK;
    if (q && (!q_strides || !q_out)) return QDL_BORN_E_NULL;
    if (k && (!k_strides || !k_out)) return QDL_BORN_E_NULL;
    PrologueArgs a = {};
    a.src[0] = ref(q, q_strides, H, T, D);
    a.src[1] = ref(k, k_strides, H, T, D);
    a.dst[0] = ref(q ? q_out : nullptr, nullptr, H, T, D);
    a.dst[1] = ref(k ? k_out : nullptr, nullptr, H, T, D);
    a.aux[0] = ref(nullptr, nullptr, H, T, D);
    a.aux[1] = ref(nullptr, nullptr, H, T, D);
    a.rinv_out[0] = q_rinv;
    a.rinv_out[1] = k_rinv;
    a.cos = cos_table;
    a.sin = sin_table;
    a.nfreq = (int)n_freq;
    a.ld = table_ld;
    a.B = (int)B;
    a.H = (int)H;
    a.T = (int)T;
    a.D = (int)D;
    a.eps = (float)eps;
    return hip_status(dispatch<true>(dtype, a, reinterpret_cast<hipStream_t>(stream)));
}

int qdl_flash_born_qk_prologue_bwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                                   const void* dq_out, const void* dk_out, const void* q_out,
                                   const void* k_out, const float* q_rinv, const float* k_rinv,
                                   const float* cos_table, const float* sin_table, int64_t n_freq,
                                   int64_t table_ld, void* dq, const int64_t* dq_strides, void* dk,
                                   const int64_t* dk_strides, qdl_stream_t stream) {
    using namespace qdl;
    int rc = check_shape(dtype, B, H, T, D);
    if (rc != QDL_BORN_OK) return rc;
    rc = check_table(cos_table, sin_table, n_freq, table_ld, D);
    if (rc != QDL_BORN_OK) return rc;
    if (B * H * T == 0 || (!dq_out && !dk_out)) return QDL_BORN_OK;
    if (dq_out && (!q_out || !q_rinv || !dq || !dq_strides)) return QDL_BORN_E_NULL;
    if (dk_out && (!k_out || !k_rinv || !dk || !dk_strides)) return QDL_BORN_E_NULL;
    PrologueArgs a = {};
    a.src[0] = ref(dq_out, nullptr, H, T, D);
    a.src[1] = ref(dk_out, nullptr, H, T, D);
    a.aux[0] = ref(dq_out ? q_out : nullptr, nullptr, H, T, D);
    a.aux[1] = ref(dk_out ? k_out : nullptr, nullptr, H, T, D);
    a.dst[0] = ref(dq_out ? dq : nullptr, dq_strides, H, T, D);
    a.dst[1] = ref(dk_out ? dk : nullptr, dk_strides, H, T, D);
    a.rinv_in[0] = q_rinv;
    a.rinv_in[1] = k_rinv;
    a.cos = cos_table;
    a.sin = sin_table;
    a.nfreq = (int)n_freq;
    a.ld = table_ld;
    a.B = (int)B;
    a.H = (int)H;
    a.T = (int)T;
    a.D = (int)D;
    return hip_status(dispatch<false>(dtype, a, reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"
