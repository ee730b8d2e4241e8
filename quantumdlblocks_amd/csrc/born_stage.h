// Global -> LDS staging of 16-bit row tiles, optionally transposed.
//
// A tile is R consecutive rows (tokens) x DP columns (head dims) of a
// contiguous (T x D) matrix.  Each thread moves "pair chunks": 8 columns of 2
// consecutive rows (2 x 16 bytes), so that the transposed copy can be written
// as packed (row 2k, row 2k+1) 32-bit words: column c of the tile becomes a
// row of the transposed copy.  Rows >= T and columns >= D are zero-filled.
#pragma once

#include "born_common.h"

namespace qdl {

template <int R, int DP, int NT>
struct PairStager {
    static_assert(R % 2 == 0 && DP % 8 == 0, "tile shape");
    static constexpr int CPR = DP / 8;             // chunks per row
    static constexpr int CH = (R / 2) * CPR;       // pair chunks per tile
    static constexpr int PT = (CH + NT - 1) / NT;  // pair chunks per thread
    u32x4 x[PT][2];

    // Loads rows r0 .. r0+R-1.  If `rdiv` is given, each row is divided by
    // rdiv[row] (fp32) and re-rounded to the element type E.
    template <class E>
    __device__ __forceinline__ void load(const uint16_t* __restrict__ src, int r0, int T, int D,
                                         int tid, const float* __restrict__ rdiv = nullptr) {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 8;
                const int row = r0 + 2 * (idx / CPR);
                u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
                if (col < D) {
                    if (row < T) a = ldg16(src + (size_t)row * D + col);
                    if (row + 1 < T) b = ldg16(src + (size_t)(row + 1) * D + col);
                }
                if (rdiv != nullptr) {
                    const float sa = row < T ? 1.0f / rdiv[row] : 0.f;
                    const float sb = row + 1 < T ? 1.0f / rdiv[row + 1] : 0.f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        a[j] = E::pack(E::lo(a[j]) * sa, E::hi(a[j]) * sa);
                        b[j] = E::pack(E::lo(b[j]) * sb, E::hi(b[j]) * sb);
                    }
                }
                x[i][0] = a;
                x[i][1] = b;
            }
        }
    }

    // Row-major copy: lds_row[r * RS + c].
    template <int RS>
    __device__ __forceinline__ void store_rows(uint16_t* lds_row, int tid) const {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 8;
                const int row = 2 * (idx / CPR);
                *reinterpret_cast<u32x4*>(&lds_row[row * RS + col]) = x[i][0];
                *reinterpret_cast<u32x4*>(&lds_row[(row + 1) * RS + col]) = x[i][1];
            }
        }
    }

    // Transposed copy: lds_trn[c * TS + r].
    template <int TS>
    __device__ __forceinline__ void store_trans(uint16_t* lds_trn, int tid) const {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 8;
                const int row = 2 * (idx / CPR);
                const u32x4 a = x[i][0], b = x[i][1];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t even = (a[j] & 0xffffu) | (b[j] << 16);
                    const uint32_t odd = (a[j] >> 16) | (b[j] & 0xffff0000u);
                    *reinterpret_cast<uint32_t*>(&lds_trn[(col + 2 * j) * TS + row]) = even;
                    *reinterpret_cast<uint32_t*>(&lds_trn[(col + 2 * j + 1) * TS + row]) = odd;
                }
            }
        }
    }
};

// 16-byte-chunk staging of a row tile (no transpose).
template <int R, int DP, int NT>
struct RowStager {
    static constexpr int CPR = DP / 8;
    static constexpr int CH = R * CPR;
    static constexpr int PT = (CH + NT - 1) / NT;
    u32x4 x[PT];

    __device__ __forceinline__ void load(const uint16_t* __restrict__ src, int r0, int T, int D, int tid) {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 8;
                const int row = r0 + idx / CPR;
                u32x4 a = {0u, 0u, 0u, 0u};
                if (row < T && col < D) a = ldg16(src + (size_t)row * D + col);
                x[i] = a;
            }
        }
    }

    template <int RS>
    __device__ __forceinline__ void store_rows(uint16_t* lds_row, int tid) const {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 8;
                const int row = idx / CPR;
                *reinterpret_cast<u32x4*>(&lds_row[row * RS + col]) = x[i];
            }
        }
    }
};

// fp32 row tile staging (16-byte chunks of 4 floats).
template <int R, int DP, int NT>
struct RowStager32 {
    static constexpr int CPR = DP / 4;
    static constexpr int CH = R * CPR;
    static constexpr int PT = (CH + NT - 1) / NT;
    f32x4 x[PT];

    __device__ __forceinline__ void load(const float* __restrict__ src, int r0, int T, int D, int tid) {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 4;
                const int row = r0 + idx / CPR;
                f32x4 a = {0.f, 0.f, 0.f, 0.f};
                if (row < T && col < D) a = *reinterpret_cast<const f32x4*>(src + (size_t)row * D + col);
                x[i] = a;
            }
        }
    }

    template <int RS>
    __device__ __forceinline__ void store_rows(float* lds_row, int tid) const {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 4;
                const int row = idx / CPR;
                *reinterpret_cast<f32x4*>(&lds_row[row * RS + col]) = x[i];
            }
        }
    }
};

}  // namespace qdl
