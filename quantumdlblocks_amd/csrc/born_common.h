// Shared device helpers for the gfx950 flash-Born kernels.
//
// Layout conventions (all tensors contiguous):
//   q, k, v, o, do, dq, dk, dv : (B, H, T, D), element type E
//   z, delta                   : (B, H, T) fp32
//   doc_ids                    : (B, T) int32
//
// MFMA lane layouts used throughout (wave64, lane l, c = l % 32, g = l / 32):
//   v_mfma_f32_32x32x16_{bf16,f16}
//     A (32x16): lane holds A[c][8g .. 8g+7]       (8 x 16-bit = 4 dwords)
//     B (16x32): lane holds B[8g .. 8g+7][c]
//     C (32x32): lane holds C[row(r)][c], r = 0..15,
//                row(r) = 8*(r/4) + 4*g + (r%4)
//   v_mfma_f32_32x32x2_f32
//     A (32x2):  lane holds A[c][g]; B (2x32): lane holds B[g][c]; C as above.
// Only A/B consistency matters for a contraction, so the kernels permute the
// contraction index freely; the C layout is what the score -> probability ->
// next-operand handoff relies on.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>
#include <type_traits>

namespace qdl {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

// Row of a 32x32 MFMA accumulator register r for lane half g.
__device__ __forceinline__ constexpr int acc_row(int r, int g) {
    return 8 * (r >> 2) + 4 * g + (r & 3);
}

// Packed 16-bit ReLU: bf16 and fp16 are sign-magnitude, so a signed 16-bit
// integer max against zero clears every negative value (including -0).
__device__ __forceinline__ uint32_t relu_pk16(uint32_t u) {
    i16x2 x = __builtin_bit_cast(i16x2, u);
    i16x2 zero = {0, 0};
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(x, zero));
}

// Where the scale enters the 16-bit weights.  bf16 keeps fp32's exponent
// range, so the scale is folded out of the tile loop (p' = r|r| from the
// unscaled overlap r, p = s^2 p', restored once per row in the epilogue).
// fp16 (kScaleInSquare) runs the reference's own arithmetic: the forward
// squares c r with c = |s|, i.e. p = relu(s r)^2 in fp32, and rounds it to
// fp16 only as the P.V operand (flash_born.py:166-183), so a weight flushes
// or overflows exactly where the reference's does; the backward scales by
// c = 2|s|, so its dS operand is the reference's 2 a dP (flash_born.py:
// 305-311) and its p/Z operand 4 p/Z (at most 4: it flushes later and never
// overflows).  The epilogues divide c back out.
struct BF16 {
    static constexpr int kDtype = 2;
    static constexpr bool kScaleInSquare = false;
    __device__ __forceinline__ static f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    // Round-to-nearest-even fp32 pair -> packed 16-bit pair; the vector
    // conversion maps to one v_cvt_pk_bf16_f32 (element-wise casts do not).
    __device__ __forceinline__ static uint32_t pack(float x, float y) {
        const f32x2 f = {x, y};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
    }
    // acc + u.lo + u.hi in fp32 (v_dot2c_f32_bf16 against (1, 1)).
    __device__ __forceinline__ static float sum2(uint32_t u, float acc) {
        const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u), one, acc, false);
    }
    __device__ __forceinline__ static float lo(uint32_t u) { return __uint_as_float(u << 16); }
    __device__ __forceinline__ static float hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
};

struct F16 {
    static constexpr int kDtype = 1;
    static constexpr bool kScaleInSquare = true;
    __device__ __forceinline__ static f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    __device__ __forceinline__ static uint32_t pack(float x, float y) {
        const f32x2 f = {x, y};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
    }
    __device__ __forceinline__ static float sum2(uint32_t u, float acc) {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, u), one, acc, false);
    }
    __device__ __forceinline__ static float lo(uint32_t u) {
        return (float)__builtin_bit_cast(f16x2, u)[0];
    }
    __device__ __forceinline__ static float hi(uint32_t u) {
        return (float)__builtin_bit_cast(f16x2, u)[1];
    }
};

__device__ __forceinline__ float relu_f32(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// Whether a (query, key) pair at offset d = query - key is masked by
// causality (d < 0) and/or a sliding window (d >= W); causal with a window
// as one unsigned compare, (unsigned)d >= W, which keeps fewer condition
// registers live than the two signed tests.
template <bool CAUS, bool WIN>
__device__ __forceinline__ bool pair_cut(int d, int W) {
    if constexpr (CAUS && WIN) return (uint32_t)d >= (uint32_t)W;
    else if constexpr (CAUS) return d < 0;
    else if constexpr (WIN) return d >= W;
    else return false;
}

// One pair of Born weights of a tile, packed for the P.V product, added to
// the row's running sum z.  x0, x1: the overlaps r' (fp32; the sign of the
// scale folded into Q, masked elements already zero); c: the fp16 scale |s|.
//   bf16: p' = relu(r')|r'|, rounded to bf16 (the scale goes back in per row
//         in the epilogue); z adds the rounded weights (one v_dot2c).
//   fp16: p = relu(c r')^2 = relu(s r)^2 in fp32, the reference's weight
//         (flash_born.py:166-182), rounded to fp16 only as the P.V operand
//         (:183); z adds the fp32 weights, as the reference's z_acc does.
template <class E>
__device__ __forceinline__ uint32_t born_weight_pair(float x0, float x1, float c, float& z) {
    if constexpr (E::kScaleInSquare) {
        const float a0 = relu_f32(x0 * c), a1 = relu_f32(x1 * c);
        const float p0 = a0 * a0, p1 = a1 * a1;
        z = (z + p0) + p1;
        return E::pack(p0, p1);
    } else {
        const uint32_t u = relu_pk16(E::pack(x0 * fabsf(x0), x1 * fabsf(x1)));
        z = E::sum2(u, z);
        return u;
    }
}

// An fp16 pair as two bf16 pairs that sum to it exactly (the purified
// forward's fp16 V operand, whose products with the split fp32 weights run on
// the bf16 MFMA): hi = each value's fp32 form truncated to bf16, lo = the
// remainder, which holds at most the 3 low bits of fp16's 11-bit significand
// (or of a subnormal's 10) and so is exact in bf16 and truncates exactly.
__device__ __forceinline__ void f16_pair_to_bf16_hi_lo(uint32_t u, uint32_t& hi, uint32_t& lo) {
    const float a = F16::lo(u), b = F16::hi(u);
    const uint32_t ab = __float_as_uint(a) & 0xffff0000u, bb = __float_as_uint(b) & 0xffff0000u;
    hi = (ab >> 16) | bb;
    const float ra = a - __uint_as_float(ab), rb = b - __uint_as_float(bb);
    lo = (__float_as_uint(ra) >> 16) | (__float_as_uint(rb) & 0xffff0000u);
}

// O^T += V^T P for the purified forward: bf16 V times the split weights
// (hi, lo: two bf16 MFMAs), or fp16 V split exactly into bf16 hi + lo times
// them (three: the lo x lo term, below 2^-17 of the product, is left out).
template <class E>
__device__ __forceinline__ f32x16 pur_pv(u32x4 v, u32x4 ph, u32x4 pl, f32x16 acc) {
    if constexpr (std::is_same<E, F16>::value) {
        u32x4 vh, vl;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t h, l;
            f16_pair_to_bf16_hi_lo(v[w], h, l);
            vh[w] = h;
            vl[w] = l;
        }
        acc = BF16::mfma(vh, ph, acc);
        acc = BF16::mfma(vh, pl, acc);
        return BF16::mfma(vl, ph, acc);
    } else {
        acc = BF16::mfma(v, ph, acc);
        return BF16::mfma(v, pl, acc);
    }
}

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ds_read_b64_tr_b16 (gfx950): within each 16-lane group, lane i receives
// element (i % 4) of the 4 x 16-bit chunks addressed by lanes i/4, 4 + i/4,
// 8 + i/4 and 12 + i/4.  With those four lanes pointing at 4 consecutive rows
// of a row-major tile, lane i gets 4 consecutive rows of one column.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// XOR swizzle of the 16-byte chunks of a 128-byte LDS tile row r: chunk c is
// stored at c ^ lds_swz(r).  LDS serves 64 banks x 4 bytes per cycle; a
// ds_read_b128 is served 16 lanes at a time and a ds_read_b64(_tr_b16) 32 at
// a time.  With rows of 128 bytes, two rows of equal parity share their banks,
// so a row read (lanes on 16 consecutive rows, one logical chunk) is
// conflict-free when lds_swz takes 8 distinct values on the 8 rows of each
// parity, and a transposed read (lanes on rows r0..r0+3, r0 % 4 == 0, an
// aligned group of 4 chunks) when lds_swz(r) ^ lds_swz(r + 2) has bit 2 set
// for r % 4 in {0, 1}.  Both hold here (2 (r & 3) | ((r >> 2) & 1) meets only
// the second, r & 7 neither).
__device__ __forceinline__ int lds_swz(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ u32x4 ldg16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

// Kernel argument block shared by the forward kernels.
struct FwdArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* z;
    const float* scale;
    const int32_t* doc;  // (B, T) or nullptr
    int per_head_scale;
    int B, H, T, D;
    int is_causal;
    int window;
    float eps;
};

// Forward with the Q prologue folded into the query-block load (bf16,
// D = 64): the FwdArgs fields, with q holding the raw query rows (unit stride
// along D, element strides q_sb / q_sh / q_st for b, h, t) and k the keys
// already normalised (contiguous), plus the rotary tables and the outputs
// the backward needs: the normalised query rows and 1/norm per row.
struct FwdProArgs : FwdArgs {
    int64_t q_sb, q_sh, q_st;
    const float* cos;  // (T, ld) fp32, or nullptr: no rotation
    const float* sin;
    int ld, nfreq;
    float norm_eps;
    void* q_out;       // (B, H, T, D) contiguous
    float* q_rinv;     // (B, H, T)
};

// Kernel argument block shared by the backward kernels.
struct BwdArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* dout;
    const float* z;
    const float* scale;
    const int32_t* doc;
    void* dq;
    void* dk;
    void* dv;
    float* ndelta;         // (B, H, T) workspace: -(dO . O) per row
    float* delta_z;        // (B, H, T) workspace: dO . O / Z per row
    float* zinv;           // (B, H, T) workspace: 1 / Z per row
    double* dscale_part;   // workspace: dscale partial sums (per chunk of rows, or per workgroup)
    float* dscale;         // n_scale outputs
    int per_head_scale;
    int B, H, T, D;
    int is_causal;
    int window;
    float eps;
};

// Fixed number of partial sums per dscale output (deterministic reduction).
constexpr int DSCALE_CHUNKS = 128;

// Mask modes compiled into the kernels.
enum MaskMode : int {
    kDense = 0,    // non-causal, no window, no documents
    kCausal = 1,   // causal only
    kGeneral = 2,  // runtime causal flag + window + document ids
    kWindow = 3,   // causal with a sliding window (the tuned kernels)
    kWindowNC = 4, // sliding window without causality (the D = 64 fast kernels)
};

// Row i sees keys j with i - j < window (flash_born.py:173-174), and j <= i
// under causality: kWindowNC keeps every key after the row as well.
constexpr bool mode_window(int m) { return m == kWindow || m == kWindowNC; }
constexpr bool mode_causal(int m) { return m == kCausal || m == kWindow; }

// Document ids: the span of candidate tiles a block has to visit.  The
// block's stationary rows r0 .. r1-1 hold ids in [dlo, dhi]; candidate tile t
// (t_lo <= t <= t_hi) covers rows t TS .. min(T, t TS + TS) - 1 of the
// streamed operand.  Returns the first (x) and last (y) candidate whose id
// range meets [dlo, dhi], x > y when none does.  A visible pair needs equal
// ids, so no tile outside the span has one: the span is exact for sorted ids
// (compute_document_ids output) and a superset for any others, and the tiles
// inside keep their per-element masks.  Every thread of the block calls it
// (three barriers); red is four ints of LDS.
template <int TS>
__device__ int2 doc_tile_span(const int32_t* __restrict__ docb, int T, int r0, int r1, int t_lo, int t_hi,
                              int32_t* red) {
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63;
    auto wave_min = [](int x) {
        for (int o = 1; o < 64; o <<= 1) x = min(x, __shfl_xor(x, o));
        return x;
    };
    auto wave_max = [](int x) {
        for (int o = 1; o < 64; o <<= 1) x = max(x, __shfl_xor(x, o));
        return x;
    };
    if (tid == 0) {
        red[0] = INT_MAX;
        red[1] = INT_MIN;
        red[2] = INT_MAX;
        red[3] = INT_MIN;
    }
    __syncthreads();
    int lo = INT_MAX, hi = INT_MIN;
    for (int r = r0 + tid; r < r1; r += nt) {
        const int d = docb[r];
        lo = min(lo, d);
        hi = max(hi, d);
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0) {
        atomicMin(&red[0], lo);
        atomicMax(&red[1], hi);
    }
    __syncthreads();
    const int dlo = red[0], dhi = red[1];
    const bool vec = (reinterpret_cast<uintptr_t>(docb) & 15) == 0;
    int first = INT_MAX, last = INT_MIN;
    for (int t = t_lo + tid; t <= t_hi; t += nt) {
        const int k0 = t * TS, k1 = min(T, k0 + TS);
        int a = INT_MAX, z = INT_MIN;
        if (vec && k1 - k0 == TS) {
#pragma unroll 8
            for (int j = 0; j < TS / 4; ++j) {
                const int4 x = *reinterpret_cast<const int4*>(docb + k0 + 4 * j);
                a = min(a, min(min(x.x, x.y), min(x.z, x.w)));
                z = max(z, max(max(x.x, x.y), max(x.z, x.w)));
            }
        } else {
            for (int k = k0; k < k1; ++k) {
                const int d = docb[k];
                a = min(a, d);
                z = max(z, d);
            }
        }
        if (z >= dlo && a <= dhi) {
            first = min(first, t);
            last = max(last, t);
        }
    }
    first = wave_min(first);
    last = wave_max(last);
    if (lane == 0) {
        atomicMin(&red[2], first);
        atomicMax(&red[3], last);
    }
    __syncthreads();
    return make_int2(red[2], red[3]);
}

// Documents: whether the n ids of the staged tile (in LDS) and the ids a and
// b of this lane's stationary rows are all one document, so that the tile
// needs no per-element document test.  Uniform per wave.
__device__ __forceinline__ bool one_document(const int32_t* ids, int n, int a, int b) {
    const int d0 = ids[0];
    bool same = (a == d0) && (b == d0);
    for (int i = threadIdx.x & 63; i < n; i += 64) same = same && (ids[i] == d0);
    return __ballot(!same) == 0;
}

}  // namespace qdl
