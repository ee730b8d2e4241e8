// The Q prologue (unitary RoPE, then L2 normalisation: attention.py:583-589,
// functional.py:59-84,104-121) folded into an attention kernel's query-row
// load, with the rounding of the standalone prologue kernel (qk_prologue.hip)
// so the rows are bit-identical to its output: each table entry, product,
// sum and difference rounded to bf16, the fp32 sum of squares accumulated
// pair by pair and then across the row's four 8-pair chunks as
// ((c0 + c1) + (c2 + c3)), 1/norm = 1/sqrt(sum + eps) correctly rounded from
// double.
//
// Lane layout shared by the kernels that use it: a row of D = 64 bf16 values
// is eight 16-byte chunks; chunk c (columns 8c .. 8c+7) rotates against
// chunk c + 4 (pair i = column i with column i + 32).  A lane holds chunks
// g, 2 + g (its operands ks = 0, 1) and their partners 4 + g, 6 + g
// (ks = 2, 3); the lane 32 apart holds the rest of the row.
#pragma once

#include "born_common.h"

namespace qdl {

// Table entries of 8 consecutive pairs i0 .. i0+7 of one row.
struct RotRow {
    float c[8], s[8];
};

// Rotary table entries of row t (clamped to T - 1: rows past T hold zeros, so
// any table row gives zeros) for pairs i0 .. i0+7; pairs at or past nfreq
// rotate by angle 0.  vec: 16-byte loads (tables 16-byte aligned, ld a
// multiple of 4 and every pair of the head dim inside the table).
__device__ __forceinline__ void rot_load(const float* cos, const float* sin, int ld, int nfreq, int T, int t, int i0,
                                         bool vec, RotRow& r) {
    const int tt = min(t, T - 1);
    const float* cr = cos + (size_t)tt * ld;
    const float* sr = sin + (size_t)tt * ld;
    if (vec) {
#pragma unroll
        for (int v = 0; v < 8; v += 4) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(cr + i0 + v);
            const f32x4 y = *reinterpret_cast<const f32x4*>(sr + i0 + v);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                r.c[v + e] = x[e];
                r.s[v + e] = y[e];
            }
        }
    } else {
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const int idx = min(i0 + v, nfreq - 1);
            const float x = cr[idx], y = sr[idx];
            r.c[v] = (i0 + v < nfreq) ? x : 1.f;
            r.s[v] = (i0 + v < nfreq) ? y : 0.f;
        }
    }
}

// Rotate the 8 pairs (a[v], b[v]) of one row by the table entries r (rot: a
// table was given; r is rounded to bf16 in place); returns the pairs' sum of
// squares.  ya, yb: the rotated (bf16-exact) values.
__device__ __forceinline__ float rope8(const u32x4& a, const u32x4& b, RotRow& r, bool rot, u32x4& ya, u32x4& yb) {
#pragma clang fp contract(off)
    float ss = 0.f;
    if (rot) {
#pragma unroll
        for (int v = 0; v < 8; v += 2) {
            const uint32_t uc = BF16::pack(r.c[v], r.c[v + 1]), us = BF16::pack(r.s[v], r.s[v + 1]);
            r.c[v] = BF16::lo(uc);
            r.c[v + 1] = BF16::hi(uc);
            r.s[v] = BF16::lo(us);
            r.s[v + 1] = BF16::hi(us);
        }
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        float y1[2], y2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float x1 = e ? BF16::hi(a[w]) : BF16::lo(a[w]);
            const float x2 = e ? BF16::hi(b[w]) : BF16::lo(b[w]);
            if (rot) {
                const int v = 2 * w + e;
                const float r0 = BF16::lo(BF16::pack(x1 * r.c[v], 0.f));
                const float r1 = BF16::lo(BF16::pack(x2 * r.s[v], 0.f));
                const float r2 = BF16::lo(BF16::pack(x1 * r.s[v], 0.f));
                const float r3 = BF16::lo(BF16::pack(x2 * r.c[v], 0.f));
                y1[e] = BF16::lo(BF16::pack(r0 - r1, 0.f));
                y2[e] = BF16::lo(BF16::pack(r2 + r3, 0.f));
            } else {
                y1[e] = x1;
                y2[e] = x2;
            }
            ss = fmaf(y1[e], y1[e], fmaf(y2[e], y2[e], ss));
        }
        ya[w] = BF16::pack(y1[0], y1[1]);
        yb[w] = BF16::pack(y2[0], y2[1]);
    }
    return ss;
}

// 1/norm of a row from its sum of squares.
__device__ __forceinline__ float rot_rinv(float ss, float norm_eps) {
    const float se = ss + norm_eps;
    return (float)(1.0 / sqrt((double)se));
}

// A rotated chunk times 1/norm, rounded to bf16.
__device__ __forceinline__ void rot_scale(u32x4& y, float rinv) {
#pragma unroll
    for (int w = 0; w < 4; ++w) y[w] = BF16::pack(BF16::lo(y[w]) * rinv, BF16::hi(y[w]) * rinv);
}

// One row's four operands (chunks g, 2 + g, 4 + g, 6 + g: x[0..3]) -> q' in
// place, with the table entries of pairs 8g .. 8g+7 (r0) and 8(2+g) ..
// 8(2+g)+7 (r1); the row's other half sits in the lane 32 apart, which runs
// this in step.  Returns 1/norm.
__device__ __forceinline__ float rot_normalise_row(u32x4 (&x)[4], RotRow& r0, RotRow& r1, bool rot, float norm_eps) {
    u32x4 y0, y1, y2, y3;
    const float pa = rope8(x[0], x[2], r0, rot, y0, y2);
    const float pb = rope8(x[1], x[3], r1, rot, y1, y3);
    const float s01 = pa + __shfl_xor(pa, 32);
    const float s23 = pb + __shfl_xor(pb, 32);
    const float rinv = rot_rinv(s01 + s23, norm_eps);
    rot_scale(y0, rinv);
    rot_scale(y1, rinv);
    rot_scale(y2, rinv);
    rot_scale(y3, rinv);
    x[0] = y0;
    x[1] = y1;
    x[2] = y2;
    x[3] = y3;
    return rinv;
}

}  // namespace qdl
