// Flash-Born backward for head dim D == 64, dense or causal, with or without
// document ids (no window): the C5 and document-masked training hot paths.  Same arithmetic as born_bwd_dq16_kernel
// (born_bwd.h); the tiles move and the instruction stream is laid out the way
// born_fwd_fast.h does it.
//
// dQ kernel (queries stationary), one 256-row query block per workgroup, rows
// dealt to waves in 16-row slices as in the forward (two MFMA column blocks
// per wave):
//   * Q and dO rows go straight from HBM into registers (B operands of S^T
//     and dP^T); 1/Z_i and delta_i / Z_i are per-lane scalars.
//   * K and V tiles of 64 keys go global -> LDS with buffer_load ... lds
//     through a ring of three stages (tile u+2 issued right after the barrier
//     that starts tile u).  Each 16-byte chunk c of row r sits at chunk
//     c ^ f(r) of its LDS row:
//       K: f(r) = 2 (r & 3) | ((r >> 2) & 1)  -> conflict-free both for the
//          8-row ds_read_b128 of S^T = K Q^T and for the 4-row
//          ds_read_b64_tr_b16 of dQ^T = K^T U
//       V: f(r) = r & 7                        -> 8-row ds_read_b128 of dP^T
//     (32 banks x 4 bytes).
//   * Per 32-key half: S^T, T^T MFMAs (raised wave priority), the elementwise
//     pass U = relu(S^T) (T^T / Z - delta / Z), then dQ^T += K^T U.  The two
//     workgroups sharing each SIMD overlap one's MFMAs with the other's VALU.
//   * Under causality the block's four diagonal tiles are masked per element
//     (column block 0 in all four, block 1 in the last two).
//   * The finished dQ rows are scaled, packed, staged in the idle ring and
//     written back 16 bytes per lane (8 whole rows per store instruction).
//
// DOC (document ids, no window; flash_born.py:145-147, 175-177 and the
// backward's HAS_DOC_IDS branches): the same kernels visit only the tiles
// whose document-id range meets the block's (screened in chunks of candidate
// tiles into a list in LDS, as the document forward does), and a tile's
// column block is masked per element when it is on the causal diagonal or its
// tile spans several documents, per lane when the tile is one document that
// not all of the column block's rows (keys) belong to.
#pragma once

#include <climits>

#include "born_fwd_fast.h"

namespace qdl {

// Tile-list entries: tile index, plus this bit when all of the tile's rows
// belong to one document.
constexpr int kDocOne = 1 << 30;

// Runs of a wave's tiles t = 0 .. n-1 (tile t holds rows lo + 64 t ..
// lo + 64 t + 63 of the other side): [0, ta) invisible, [ta, tf) masked,
// [tf, tg) full, [tg, tv) masked, [tv, n) invisible, for a wave that may see
// rows [v0, v1] and sees all of them in full in rows [f0, f1].
struct WaveRuns {
    int ta, tf, tg, tv;
    __device__ __forceinline__ WaveRuns(int lo, int n, int v0, int v1, int f0, int f1) {
        auto rel = [&](int t) { return min(max(t, 0), n); };
        ta = rel(v0 >= lo ? (v0 - lo) / 64 : 0);
        tv = max(rel(v1 >= lo ? (v1 - lo) / 64 + 1 : 0), ta);
        tf = min(max(rel(f0 > lo ? (f0 - lo + 63) / 64 : 0), ta), tv);
        tg = min(max(rel(f1 + 1 >= lo ? (f1 - lo + 1) / 64 : 0), tf), tv);
    }
};

constexpr int kRunsBig = 1 << 29;  // "no bound" for WaveRuns

// Document-id range of rows r0 .. r1-1 of one batch row's ids.
__device__ __forceinline__ void doc_rows_range(const int32_t* __restrict__ docb, int r0, int r1, int n, bool vec,
                                               int& lo, int& hi) {
    lo = INT_MAX;
    hi = INT_MIN;
    if (vec && r1 - r0 == n) {
        // Eight 16-byte loads in flight per round trip.
#pragma unroll 8
        for (int j = 0; j < n / 4; ++j) {
            const int4 x = *reinterpret_cast<const int4*>(docb + r0 + 4 * j);
            lo = min(lo, min(min(x.x, x.y), min(x.z, x.w)));
            hi = max(hi, max(max(x.x, x.y), max(x.z, x.w)));
        }
    } else {
        for (int r = r0; r < r1; ++r) {
            const int d = docb[r];
            lo = min(lo, d);
            hi = max(hi, d);
        }
    }
}

// Screens candidate tiles c0 .. c0+nc-1 (nc <= block size; tile t holds rows
// row0 + TS t .. row0 + TS t + TS - 1, clipped to T) of one batch row's ids:
// a tile is kept when its [min, max] id range meets [lo, hi] (exact for
// sorted ids, a superset for any others, whose tiles keep the per-element
// test).  Writes the kept tiles in ascending order to list (index | kDocOne
// when the tile is one document) and that document to ldoc; returns how many.
// Every thread of the block calls it; keep / tdoc are nc-entry
// scratch arrays, list / ldoc nc entries, count one int, all in LDS.
template <int TS>
__device__ int screen_doc_tiles(const int32_t* __restrict__ docb, int T, int row0, int c0, int nc, int lo, int hi,
                                int32_t* keep, int32_t* tdoc, int32_t* list, int32_t* ldoc, int32_t* count) {
    const int tid = threadIdx.x, lane = tid & 63;
    const bool vec = ((reinterpret_cast<uintptr_t>(docb) | (uintptr_t)(row0 * 4)) & 15) == 0;
    if (tid < nc) {
        const int r0 = row0 + (c0 + tid) * TS;
        int a, z;
        doc_rows_range(docb, r0, min(r0 + TS, T), TS, vec, a, z);
        keep[tid] = (z >= lo && a <= hi) ? (a == z ? 3 : 1) : 0;
        tdoc[tid] = a;
    }
    __syncthreads();
    if (tid < 64) {
        int n = 0;
        for (int b0 = 0; b0 < nc; b0 += 64) {
            const int i = b0 + lane;
            const int kf = i < nc ? keep[i] : 0;
            const uint64_t m = __ballot(kf != 0);
            const int pos = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            if (kf != 0) {
                list[pos] = (c0 + i) | ((kf & 2) ? kDocOne : 0);
                ldoc[pos] = tdoc[i];
            }
            n += __popcll(m);
        }
        if (lane == 0) *count = n;
    }
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(*count);
}

// PUR: purified-Born gradients (flash_born.py:950-1061): with r the raw
// overlap, u = relu(gamma (r - tau)), b = relu(r) (zero where masked),
// dR = (4 gamma u^3 + 2 eps_base b) dP rounded to bf16 as the reference's
// `.to(k.dtype)` rounds it; O is the forward's fp32 output.  The dscale
// closed form is Born's only: the purified dgamma / dtau come from the dK/dV
// kernel.
// PAD (purified only): a head dim D < 64 (a multiple of 8), as in the
// forward: chunks past D load as zeros and are not stored.
// NW (documents only): 2 waves over 128-row blocks, four workgroups per CU
// and a two-stage ring, as the document forward (fewer blocks straddle a
// document edge); otherwise 4 waves over 256-row blocks.
template <class E, int DP, int MODE, bool PUR = false, bool DOC = false, bool PAD = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void born_bwd16_dq_fast_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    static_assert(DP == 64, "tuned for D = 64");
    static_assert(!PAD || (PUR && !DOC), "narrow head dims: purified");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified gradients: 16-bit");
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    static_assert(NW == 4 || (NW == 2 && DOC), "128-row blocks: the document variant");
    constexpr int NQB = 2, BN = 64, NST = NW == 4 ? 3 : 2, BM = NW * 32 * NQB;
    constexpr int KS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    constexpr int CAP = 64 * NW;           // documents: candidate tiles screened per pass
    constexpr int KDW = BN / NW;           // documents: key ids loaded per wave per tile
    // Loads per wave per tile: K, V (and a slice of the key document ids).
    constexpr int kTileLoads = 2 * LPW + (DOC ? 1 : 0);
    static_assert(TB % (1024 * NW) == 0 && BM * RB <= 2 * NST * TB, "tile split / staging fits the ring");
    static_assert(BM == NW * BN, "NW 64-row slices per block");
    // kWindow: causal, row i sees keys i - window + 1 .. i (kWindowNC: up to
    // T - 1) (flash_born.py:394,
    // 415-416): the block visits the key tiles from its window's first key on.
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);

    // One buffer: the K/V ring during the tile loop, the output staging
    // (BM rows x 128 bytes) once the loop is done.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * NST * TB];
    // Documents: key document ids per stage, the kept-tile list and screening scratch.
    __shared__ __attribute__((aligned(16))) int32_t kd_lds[DOC ? NST * BN : 1];
    __shared__ int32_t t_list[DOC ? CAP : 1], t_doc[DOC ? CAP : 1], t_keep[DOC ? CAP : 1], t_tdoc[DOC ? CAP : 1];
    __shared__ int32_t s_rng[2 * NW + 1];
    uint8_t* const k_lds = smem;
    uint8_t* const v_lds = smem + NST * TB;

    const int T = p.T;
    const int BH = p.B * p.H;
    const int nmb = (T + BM - 1) / BM;
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    // Under causality the longest key ranges go first.
    const int mb = kCaus ? (nmb - 1 - bid / BH) : (bid / BH);
    const int h = bh % p.H;
    const int R = mb * BM;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, g = lane >> 5;
    // Rows: column c of block qb -> row R + (BM/2) qb + (BM/4) (c / 16) +
    // 16 wave + c % 16.
    const int lrow = (BM / 4) * (c >> 4) + 16 * wave + (c & 15);

    // Head dim in HBM: DP, or (PAD) D < DP with CG 16-byte chunks per row.
    const int D = PAD ? p.D : DP;
    const int CG = D / 8;
    const size_t base = (size_t)bh * T * D;
    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (!PUR && sc < 0.f) ? 0x80008000u : 0u;
    // fp16 scales the overlap by c = 2|s|, so the dS operand is the
    // reference's 2 a dP (see E::kScaleInSquare); the epilogue divides c out.
    const float sq_pre = (E::kScaleInSquare && sc != 0.f) ? 2.f * fabsf(sc) : 1.f;
    // Purified: t = gamma r - gamma tau; dR / dP = 4 gamma u^3 + 2 eps_base b.
    float pg = 0.f, pgt = 0.f, p4g = 0.f, p2e = 0.f;
    if constexpr (PUR) {
        pg = sc;
        pgt = -sc * p.tau[p.per_head_tau ? h : 0];
        p4g = 4.f * sc;
        p2e = 2.f * p.eps_base;
    }

    // Stationary operands: sign-flipped Q and dO rows of this lane's queries.
    // delta_i = dO_i . O_i is formed here from the stored O (each lane holds
    // half a row; the other half is in lane ^ 32), and the per-row -delta,
    // 1/Z and delta/Z the dK/dV kernel and the dscale reduction read are
    // written to the workspace.
    int qrow[NQB];
    u32x4 qr[NQB][KS], dr[NQB][KS];
    float zinv[NQB], nd[NQB];
    // Documents: each row's document id (INT_MIN past T; such rows are not
    // stored), kept in LDS (r_doc, by row of the block) for the tile loop,
    // whose registers are all taken.
    int qdoc[NQB];
    __shared__ int32_t r_doc[DOC ? BM : 1];
    const int32_t* __restrict__ docb = nullptr;
    if constexpr (DOC) docb = p.doc + (size_t)(bh / p.H) * T;
    {
        const uint16_t* __restrict__ Qg = reinterpret_cast<const uint16_t*>(p.q) + base;
        const uint16_t* __restrict__ dOg = reinterpret_cast<const uint16_t*>(p.dout) + base;
        const uint16_t* __restrict__ Og = nullptr;
        const float* __restrict__ Og32 = nullptr;
        if constexpr (PUR)
            Og32 = p.o_in + base;
        else
            Og = reinterpret_cast<const uint16_t*>(p.o) + base;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            qrow[qb] = R + (BM / 2) * qb + lrow;
            const int qi = qrow[qb];
            const bool ok = qi < T;
            if constexpr (DOC) {
                qdoc[qb] = ok ? docb[qi] : INT_MIN;
                if (g == 0) r_doc[(BM / 2) * qb + lrow] = qdoc[qb];
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
                if (ok && (!PAD || 2 * ks + g < CG)) {
                    x = ldg16(Qg + (size_t)qi * D + (2 * ks + g) * 8);
                    y = ldg16(dOg + (size_t)qi * D + (2 * ks + g) * 8);
                }
                qr[qb][ks] = x ^ flip;
                dr[qb][ks] = y;
            }
            float dl = 0.f;
            if (ok) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    if (PAD && 2 * ks + g >= CG) continue;  // dO is zero there
                    if constexpr (PUR) {
                        const f32x4 oa = *reinterpret_cast<const f32x4*>(Og32 + (size_t)qi * D + (2 * ks + g) * 8);
                        const f32x4 ob = *reinterpret_cast<const f32x4*>(Og32 + (size_t)qi * D + (2 * ks + g) * 8 + 4);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float o0 = j < 2 ? oa[2 * j] : ob[2 * j - 4];
                            const float o1 = j < 2 ? oa[2 * j + 1] : ob[2 * j - 3];
                            dl += o0 * E::lo(dr[qb][ks][j]) + o1 * E::hi(dr[qb][ks][j]);
                        }
                    } else {
                        const u32x4 o = ldg16(Og + (size_t)qi * D + (2 * ks + g) * 8);
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            dl += E::lo(o[j]) * E::lo(dr[qb][ks][j]) + E::hi(o[j]) * E::hi(dr[qb][ks][j]);
                    }
                }
            }
            dl += __shfl_xor(dl, 32);
            const size_t row = (size_t)bh * T + qi;
            float zr = 1.f;
            if (ok) {
                if constexpr (PUR)
                    zr = p.z_in[row];
                else
                    zr = p.z[row];
            }
            zinv[qb] = ok ? 1.0f / zr : 0.f;
            nd[qb] = ok ? -(dl / zr) : 0.f;
            if (ok && g == 0) {
                p.ndelta[row] = -dl;
                p.zinv[row] = zinv[qb];
                if constexpr (!PUR) p.delta_z[row] = dl / zr;
            }
        }
    }
    // This workgroup's part of dscale = (2/s) eps sum delta / Z (closed form):
    // its rows' sum, in a fixed order (lanes, then waves), one double per
    // workgroup.
    if constexpr (!PUR) {
        __shared__ float s_dz[NW];
        float dz = (g == 0) ? -(nd[0] + nd[1]) : 0.f;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) dz += __shfl_xor(dz, off);
        if (lane == 0) s_dz[wave] = dz;
        __syncthreads();
        if (tid == 0) {
            double acc = 0.0;
#pragma unroll
            for (int w = 0; w < NW; ++w) acc += (double)s_dz[w];
            p.dscale_part[bid] = acc;
        }
    }

    // Key tiles tb .. tb+ntiles-1 (tb: the window's first key tile, else 0;
    // documents: the candidates, screened below), counted from tb.
    const int W = kWin ? p.window : 0;
    const int tb = kWin ? max(0, R - W + 1) / BN : 0;
    const int ntiles = (kCaus ? (min(T, R + BM) + BN - 1) / BN : (T + BN - 1) / BN) - tb;
    const int t0 = kCaus ? min(R / BN - tb, ntiles) : ntiles;  // first diagonal tile
    // Window: tiles before te hold keys older than the window of some row (the
    // block's last row sees keys from R + BM - W on).
    const int te = kWin ? min(max((R + BM - W + BN - 1) / BN - tb, 0), t0) : 0;

    const uint32_t nrec = (uint32_t)T * (uint32_t)(2 * D);
    const i32x4 rk = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.k) + base, nrec);
    const i32x4 rv = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.v) + base, nrec);
    const i32x4 rdoc = buffer_rsrc(docb, DOC ? (uint32_t)T * 4u : 0u);
    auto kswz = [](int r) __attribute__((always_inline)) { return ((r & 3) << 1) | ((r >> 2) & 1); };

    // Tile u (documents: kept tile u of the list) -> stage u % NST:
    // wave-instruction i writes LDS slots (wave * LPW + i) * 64 + lane,
    // slot = row * CPR + chunk'; documents: also this wave's KDW key document
    // ids (lanes 0 .. KDW/4 - 1, 16 bytes each).
    auto issue = [&](int u) __attribute__((always_inline)) {
        const int st = u % NST;
        int key0 = (tb + u) * BN;
        if constexpr (DOC) key0 = (tb + (__builtin_amdgcn_readfirstlane(t_list[u]) & ~kDocOne)) * BN;
        uint8_t* kb = k_lds + st * TB;
        uint8_t* vb = v_lds + st * TB;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int slot = (wave * LPW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int off = (key0 + row) * (2 * D);
            const int kc = pc ^ kswz(row), vc = pc ^ (row & 7);
            dma_load16(rk, lds_addr(kb + (wave * LPW + i) * 1024), (PAD && kc >= CG) ? kBufOOB : off + (kc << 4));
            dma_load16(rv, lds_addr(vb + (wave * LPW + i) * 1024), (PAD && vc >= CG) ? kBufOOB : off + (vc << 4));
        }
        if constexpr (DOC)
            if (lane < KDW / 4)
                dma_load16(rdoc, lds_addr(kd_lds + st * BN + wave * KDW), (key0 + wave * KDW + lane * 4) * 4);
    };

    // Operand reads.  Rows: K/V row nb * 32 + c (A operands of S^T, dP^T);
    // K^T: keys nb * 32 + hh * 16 + 4 g + (lane & 15) / 4 (+8), d columns
    // db * 32 + 16 ((lane >> 4) & 1) + 4 (lane & 3): the key order of the
    // accumulator layout of U (as P in the forward).
    const int trow_l = 4 * g + ((lane & 15) >> 2);
    const int tcol_l = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    auto k_row = [&](const uint8_t* kb, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + c;
        return *reinterpret_cast<const u32x4*>(kb + row * RB + (((2 * ks + g) ^ kswz(row)) << 4));
    };
    auto v_row = [&](const uint8_t* vb, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + c;
        return *reinterpret_cast<const u32x4*>(vb + row * RB + (((2 * ks + g) ^ (row & 7)) << 4));
    };
    auto k_tr = [&](const uint8_t* kb, int nb, int hh, int db) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + hh * 16 + trow_l;
        const int col = db * 32 + tcol_l;
        const uint8_t* b0 = kb + row * RB + (((col >> 3) ^ kswz(row)) << 4) + (col & 7) * 2;
        const u32x2 x = lds_read_tr16(reinterpret_cast<const uint16_t*>(b0));
        const u32x2 y = lds_read_tr16(reinterpret_cast<const uint16_t*>(b0 + 8 * RB));
        const u32x4 a = {x[0], x[1], y[0], y[1]};
        return a;
    };

    f32x16 acc[DB][NQB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) acc[db][qb] = zero16();

    // One 32-key half nb of a tile:
    //   S^T = K Q^T, T^T = V dO^T       (A = K, V rows; B = Q^T, dO^T)
    //   U = relu(S^T) (T^T / Z - delta / Z), masked keys zeroed
    //   dQ^T += K^T U                     (A = K^T, B = U)
    // MFMAs at raised wave priority, the elementwise pass at normal priority:
    // the two workgroups sharing a SIMD overlap one's MFMAs with the other's
    // VALU work.  (Interleaving the column blocks' phases within the wave
    // measured slower.)  relu is an integer max on the float bits (no NaN
    // canonicalisation).  The causal mask of column block qb is applied
    // under mk[qb]: uniform runtime flags on the diagonal and window-edge
    // tiles (one body for all of them; two bodies under one branch cost more
    // registers than the wave has), compile-time false on the plain tiles,
    // whose body has no mask code and runs in a loop of its own.
    // Documents, per tile: column block qb is tested per element (dm) or not
    // at all; kdp: this stage's key document ids.
    bool dm[NQB] = {false, false};
    const int32_t* kdp = kd_lds;
    auto half = [&](const uint8_t* kb, const uint8_t* vb, int nb, int kbase, const auto& mk, auto skip0)
        __attribute__((always_inline)) {
        // skip0: column block 0 sees none of the tile (diagonal tiles 2 and
        // 3 under causality): its MFMAs and elementwise pass are left out.
        constexpr int Q0 = decltype(skip0)::value ? 1 : 0;
        f32x16 s[NQB], t[NQB];
        uint32_t pk[NQB][8];
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int qb = Q0; qb < NQB; ++qb) s[qb] = zero16(), t[qb] = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 ko = k_row(kb, nb, ks);
            const u32x4 vo = v_row(vb, nb, ks);
#pragma unroll
            for (int qb = Q0; qb < NQB; ++qb) {
                s[qb] = E::mfma(ko, qr[qb][ks], s[qb]);
                t[qb] = E::mfma(vo, dr[qb][ks], t[qb]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        if constexpr (PUR) {
#pragma unroll
            for (int qb = Q0; qb < NQB; ++qb) {
                const int lim = qrow[qb] - kbase;
                // Documents: the row's id (read only where the tile is tested).
                int rd = 0;
                if constexpr (DOC)
                    if (dm[qb]) rd = r_doc[(BM / 2) * qb + (BM / 4) * (c >> 4) + 16 * wave + (c & 15)];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float w[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int r = 2 * j + e;
                        const int off = 8 * (r >> 2) + (r & 3);
                        const float x = s[qb][r];
                        const float u = __int_as_float(max(__float_as_int(fmaf(x, pg, pgt)), 0));
                        const float bb = __int_as_float(max(__float_as_int(x), 0));
                        const float f = fmaf(p4g, u * u * u, p2e * bb);
                        float dr_ = f * fmaf(t[qb][r], zinv[qb], nd[qb]);
                        // A masked pair weighs zero even where its overlap is
                        // zero (u = relu(-gamma tau) > 0 for tau < 0).
                        if constexpr (DOC) {
                            const bool cut = kWin ? pair_cut<kCaus, kWin>(lim - off, W) : (kCaus && off > lim);
                            if (dm[qb] && (cut || kdp[nb * 32 + 4 * g + off] != rd)) dr_ = 0.f;
                        } else {
                            // Causal with a window: one unsigned compare.
                            const bool cut = (kCaus && kWin) ? pair_cut<kCaus, kWin>(lim - off, W)
                                                             : ((kCaus && off > lim) || (kWin && off < lim - W + 1));
                            if (mk[qb] && cut) dr_ = 0.f;
                        }
                        w[e] = dr_;
                    }
                    pk[qb][j] = E::pack(w[0], w[1]);
                }
            }
        } else {
#pragma unroll
        for (int qb = Q0; qb < NQB; ++qb) {
            if constexpr (DOC) {
                // Key kbase + 8 (r / 4) + r % 4 of register r is masked past
                // the lane's row (causal) or in another document.
                if (dm[qb]) {
                    // Last visible key offset (causal); with a window the
                    // two bounds as one unsigned compare (causal alone keeps
                    // the plain test, which compiles shorter here).
                    const int lim = kCaus ? qrow[qb] - kbase : INT_MAX;
                    const int rd = r_doc[(BM / 2) * qb + (BM / 4) * (c >> 4) + 16 * wave + (c & 15)];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int4 d4 = *reinterpret_cast<const int4*>(kdp + nb * 32 + 4 * g + 8 * i);
                        const int dk[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int off = 8 * i + k;
                            const bool cut = kWin ? pair_cut<kCaus, kWin>(lim - off, W) : off > lim;
                            if (cut || dk[k] != rd) s[qb][4 * i + k] = 0.f;
                        }
                    }
                }
            } else if (mk[qb]) {
                // Masked past the lane's row, and (window) before its first key.
                const int lim = qrow[qb] - kbase;
                const int wlo = kWin ? lim - W + 1 : 0;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int off = 8 * (r >> 2) + (r & 3);
                    if ((kCaus && off > lim) || (kWin && off < wlo)) s[qb][r] = 0.f;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float x0 = s[qb][2 * j], x1 = s[qb][2 * j + 1];
                if constexpr (E::kScaleInSquare) x0 *= sq_pre, x1 *= sq_pre;
                const float a0 = __int_as_float(max(__float_as_int(x0), 0));
                const float a1 = __int_as_float(max(__float_as_int(x1), 0));
                pk[qb][j] = E::pack(a0 * fmaf(t[qb][2 * j], zinv[qb], nd[qb]), a1 * fmaf(t[qb][2 * j + 1], zinv[qb], nd[qb]));
            }
        }
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const u32x4 a = k_tr(kb, nb, hh, db);
#pragma unroll
                for (int qb = Q0; qb < NQB; ++qb) {
                    const u32x4 bq = {pk[qb][4 * hh], pk[qb][4 * hh + 1], pk[qb][4 * hh + 2], pk[qb][4 * hh + 3]};
                    acc[db][qb] = E::mfma(a, bq, acc[db][qb]);
                }
            }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };
    auto tile = [&](const uint8_t* kb, const uint8_t* vb, int key0, const auto& mk, auto skip0)
        __attribute__((always_inline)) {
        half(kb, vb, 0, key0 + 4 * g, mk, skip0);
        half(kb, vb, 1, key0 + 32 + 4 * g, mk, skip0);
    };
    using NoSkip = std::integral_constant<bool, false>;
    using Skip0 = std::integral_constant<bool, true>;
    // Mask flags of a plain tile: known false at compile time.
    struct NoMask {
        constexpr bool operator[](int) const { return false; }
    };

    // Pipeline: tiles 0 and 1 issued up front (tile 1 after the stationary
    // loads have landed, so the compiler's wait for them does not also wait
    // for tile 1), tile u+2 right after the barrier that starts step u; at
    // that barrier each wave has waited for its share of tile u (loads return
    // in order: only tile u+1's may still be in flight).
    if constexpr (DOC) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qr[qb][ks]), "+v"(dr[qb][ks]));
            asm volatile("" : "+v"(zinv[qb]), "+v"(nd[qb]));
        }
        // Document range of each column block's valid rows (uniform per
        // wave; qone: all of them in document qsd) and of the whole block.
        int qsd[NQB];
        bool qone[NQB];
        int wlo = INT_MAX, whi = INT_MIN;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            int lo = qrow[qb] < T ? qdoc[qb] : INT_MAX, hi = qrow[qb] < T ? qdoc[qb] : INT_MIN;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                lo = min(lo, __shfl_xor(lo, off));
                hi = max(hi, __shfl_xor(hi, off));
            }
            lo = __builtin_amdgcn_readfirstlane(lo);
            hi = __builtin_amdgcn_readfirstlane(hi);
            qsd[qb] = lo;
            qone[qb] = lo == hi;
            wlo = min(wlo, lo);
            whi = max(whi, hi);
        }
        if (lane == 0) {
            s_rng[2 * wave] = wlo;
            s_rng[2 * wave + 1] = whi;
        }
        __syncthreads();
        int bq_lo = INT_MAX, bq_hi = INT_MIN;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            bq_lo = min(bq_lo, s_rng[2 * w]);
            bq_hi = max(bq_hi, s_rng[2 * w + 1]);
        }
        // The kept tiles of each chunk of candidates through the same pipeline.
        for (int c0 = 0; c0 < ntiles; c0 += CAP) {
            const int n = screen_doc_tiles<BN>(docb, T, tb * BN, c0, min(CAP, ntiles - c0), bq_lo, bq_hi, t_keep, t_tdoc,
                                               t_list, t_doc, &s_rng[2 * NW]);
            // Tiles 0 .. NST-2 up front, tile u+NST-1 after the barrier of
            // step u (into the stage of tile u-1).
            if (n > 0) issue(0);
            if (NST == 3 && n > 1) issue(1);
            for (int u = 0; u < n; ++u) {
                if (NST == 3 && u + 1 < n)
                    wait_vmcnt<kTileLoads>();
                else
                    wait_vmcnt<0>();
                __syncthreads();
                if (u + NST - 1 < n) issue(u + NST - 1);
                int soff = (u % NST) * TB;
                asm volatile("" : "+s"(soff));
                const uint8_t* kb = k_lds + soff;
                const uint8_t* vb = v_lds + soff;
                kdp = kd_lds + (soff / TB) * BN;
                const int e = __builtin_amdgcn_readfirstlane(t_list[u]);
                const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
                const int ti = e & ~kDocOne;
                const bool one = (e & kDocOne) != 0;
                // A column block is tested per element on the causal diagonal
                // (block 1 from tile t0 + BM/128 on; window: block 1 on every
                // diagonal tile, both on the tiles before te) and unless the
                // tile's keys and all of its rows are one and the same
                // document.
                const bool mk[NQB] = {ti >= t0 || (kWin && ti < te),
                                      ti >= t0 + BM / 128 || (kWin && (ti < te || ti >= t0))};
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) dm[qb] = mk[qb] || !(one && qone[qb] && td == qsd[qb]);
                tile(kb, vb, (tb + ti) * BN, mk, NoSkip{});
            }
            __syncthreads();  // the list and the ring are reused by the next chunk
        }
    } else {
    if (ntiles > 0) issue(0);
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qr[qb][ks]), "+v"(dr[qb][ks]));
        asm volatile("" : "+v"(zinv[qb]), "+v"(nd[qb]));
    }
    if (ntiles > 1) issue(1);
    int u = 0;
    auto step = [&](const uint8_t*& kb, const uint8_t*& vb) __attribute__((always_inline)) {
        if (u + 1 < ntiles)
            wait_vmcnt<kTileLoads>();
        else
            wait_vmcnt<0>();
        __syncthreads();
        if (u + 2 < ntiles) issue(u + 2);
        int soff = (u % NST) * TB;
        asm volatile("" : "+s"(soff));
        kb = k_lds + soff;
        vb = v_lds + soff;
    };
    // Window: the tiles before te, both blocks tested per element.
    for (; u < te; ++u) {
        const uint8_t *kb, *vb;
        step(kb, vb);
        const bool mk[NQB] = {true, true};
        tile(kb, vb, (tb + u) * BN, mk, NoSkip{});
    }
    // Plain tiles: no mask.
    for (; u < t0; ++u) {
        const uint8_t *kb, *vb;
        step(kb, vb);
        tile(kb, vb, (tb + u) * BN, NoMask{}, NoSkip{});
    }
    // Diagonal tiles t0, t0+1: block 0 cut by the mask, block 1 fully
    // visible; t0+2, t0+3: block 0 sees none of the tile (left out), block 1
    // cut.  Window: both blocks tested on the diagonal tiles.
    for (; u < ntiles; ++u) {
        const uint8_t *kb, *vb;
        step(kb, vb);
        const bool mk[NQB] = {true, u >= t0 + 2 || kWin};
        if (kCaus && u >= t0 + 2)
            tile(kb, vb, (tb + u) * BN, mk, Skip0{});
        else
            tile(kb, vb, (tb + u) * BN, mk, NoSkip{});
    }
    }

    // Epilogue: scale, pack, stage this wave's rows in the idle ring (row r at
    // smem + 128 r, chunks XOR-swizzled by r & 7), read them back 16 bytes
    // per lane and store 8 whole rows per instruction.
    __syncthreads();  // every wave is done with the ring
    uint16_t* __restrict__ dQ = reinterpret_cast<uint16_t*>(p.dq) + base;
    const float f = PUR ? 1.f : E::kScaleInSquare ? sc : 2.f * sc * fabsf(sc);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int lr = (BM / 4) * ((ln & 31) >> 4) + 16 * wave + (ln & 15);
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const int row = (BM / 2) * qb + lr;
        uint8_t* rb = smem + row * RB;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x16& o = acc[db][qb];
                u32x2 w;
                w[0] = E::pack(o[4 * j] * f, o[4 * j + 1] * f);
                w[1] = E::pack(o[4 * j + 2] * f, o[4 * j + 3] * f);
                const int chunk = 4 * db + j;
                *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 7)) << 4) + 8 * (ln >> 5)) = w;
            }
    }
    const int chunk = ln & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = (BM / 4) * (i >> 1) + 16 * wave + 8 * (i & 1) + (ln >> 3);
        const u32x4 x = *reinterpret_cast<const u32x4*>(smem + row * RB + ((chunk ^ (row & 7)) << 4));
        const int q = R + row;
        if (q < T && (!PAD || chunk < CG))
            __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dQ + (size_t)q * D + chunk * 8));
    }
}

// dscale from the dQ kernel's per-workgroup sums: output o adds, in a fixed
// order, the partials of the workgroups whose head it covers.
// (A template, so the translation units of several dtypes can each hold it.)
template <int kUnused = 0>
__global__ __launch_bounds__(256) void born_bwd_dscale_groups_kernel(BwdArgs p, int nwg) {
    __shared__ double red[256];
    const int o = blockIdx.x;
    const int BH = p.B * p.H;
    double acc = 0.0;
    // Eight independent loads in flight per thread; each thread still adds
    // its partials in index order (i, i + 256, i + 512, ...).
    for (int i0 = threadIdx.x; i0 < nwg; i0 += 8 * 256) {
        double v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j * 256;
            const bool take = i < nwg && (!p.per_head_scale || ((i % BH) % p.H) == o);
            v[j] = take ? p.dscale_part[i] : 0.0;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += v[j];
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float s = p.scale[o];
        p.dscale[o] = (s == 0.f) ? 0.f : (float)(2.0 / (double)s * (double)p.eps * red[0]);
    }
}

// Workgroups of the D = 64 dQ launch (each writes one dscale partial):
// 256-row blocks, 128-row blocks with documents.
inline int bwd16_dq_fast_groups(int B, int H, int T, bool doc) {
    const int BM = doc ? 128 : 256;
    return ((T + BM - 1) / BM) * B * H;
}

template <class E, int DP, int MODE, bool DOC = false>
hipError_t launch_bwd16_dq_fast(const BwdArgs& a, hipStream_t st) {
    constexpr int NW = DOC ? 2 : 4;
    const dim3 grid((unsigned)bwd16_dq_fast_groups(a.B, a.H, a.T, DOC));
    hipLaunchKernelGGL((born_bwd16_dq_fast_kernel<E, DP, MODE, false, DOC, false, NW>), grid, dim3(64 * NW), 0, st, a);
    return hipGetLastError();
}

// dK / dV kernel (keys stationary), one 128-key block per workgroup, wave w
// owning keys 32 w .. 32 w + 31 (one MFMA column block):
//   * Sign-flipped K and V rows of the wave's keys go straight from HBM into
//     registers (B operands of S = Q K'^T and dP = dO V^T).
//   * Query tiles of 64 rows stream through a three-stage LDS ring: Q and dO
//     (buffer_load ... lds, chunks XOR-swizzled as K in the dQ kernel, so
//     both the row reads of S / dP and the transposed reads of dK / dV are
//     conflict-free), plus -delta and 1/Z of the tile's rows (16 lanes each).
//   * Per 32-query half, in the accumulator layout (one key per lane, 16
//     queries per lane):
//       S   = Q K'^T                    (A = Q rows)
//       dPz = dO V^T - delta            (A = dO rows, accumulator
//                                        initialised with -delta from LDS)
//       t = relu(S) / Z_i, W = t relu(S), U = t dPz   (masked queries zeroed)
//       dV^T += dO^T W,  dK^T += Q^T U  (A = dO^T, Q^T transposed reads)
//   * The finished dK, dV rows are scaled, packed, staged in the idle ring and
//     written back 16 bytes per lane.
// PUR: purified-Born gradients (flash_born.py:812-948): W = p / Z and
// dR = (4 gamma u^3 + 2 eps_base b) dP, both rounded to bf16 before their
// contractions as in the reference; each workgroup also writes its partial
// sums of dgamma = 4 sum u^3 dP (r - tau) and dtau = -4 gamma sum u^3 dP
// (PurArgs::part; reduced per output in a fixed order afterwards).  Keys
// past T are left out of those sums (their zero K row still weighs
// relu(-gamma tau) when tau < 0); queries past T have 1/Z = 0 from the
// workspace read, so they add nothing.
template <class E, int DP, int MODE, bool PUR = false, bool DOC = false, bool PAD = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((PUR && (DOC || mode_window(MODE))) ? 2 : 3,
                                                                     (PUR && (DOC || mode_window(MODE))) ? 2 : 3)))
void born_bwd16_dkdv_fast_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    static_assert(DP == 64, "tuned for D = 64");
    static_assert(!PAD || (PUR && !DOC), "narrow head dims: purified");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified gradients: 16-bit");
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    constexpr int NW = 4, BQ = 64, NST = 3, BK = NW * 32;
    constexpr int KS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BQ * RB;            // bytes per Q or dO tile
    // Bytes per stage: Q, dO, -delta, 1/Z (documents: and the query document ids).
    constexpr int NROWV = DOC ? 3 : 2;
    constexpr int SB = 2 * TB + NROWV * BQ * 4;
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of Q, dO)
    // Documents: candidate tiles screened per pass (three workgroups per CU
    // leave room for 128-entry lists).
    constexpr int CAP = 128;
    static_assert(TB % (1024 * NW) == 0 && BQ * 4 == 256 && 2 * BK * RB <= NST * SB, "tile split / staging");
    // kWindow: causal, key j is seen by queries j .. j + window - 1 (kWindowNC:
    // queries 0 .. j + window - 1): the block visits the query tiles up to
    // its last key's window.
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);

    __shared__ __attribute__((aligned(1024))) uint8_t smem[NST * SB];
    __shared__ int32_t t_list[DOC ? CAP : 1], t_doc[DOC ? CAP : 1], t_keep[DOC ? CAP : 1], t_tdoc[DOC ? CAP : 1];
    __shared__ int32_t s_rng[2 * NW + 1];

    const int T = p.T;
    const int BH = p.B * p.H;
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    // Key blocks in ascending order: under causality the first sees the most
    // queries; kWindowNC: descending, the last sees the most.
    const int kblk = MODE == kWindowNC ? (T + BK - 1) / BK - 1 - bid / BH : bid / BH;
    const int h = bh % p.H;
    const int K0 = kblk * BK;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, g = lane >> 5;
    const int kw0 = K0 + 32 * wave;  // first key of this wave
    const int key = kw0 + c;         // this lane's key

    // Head dim in HBM: DP, or (PAD) D < DP with CG 16-byte chunks per row.
    const int D = PAD ? p.D : DP;
    const int CG = D / 8;
    const size_t base = (size_t)bh * T * D;
    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (!PUR && sc < 0.f) ? 0x80008000u : 0u;
    const float sq_pre = (E::kScaleInSquare && sc != 0.f) ? 2.f * fabsf(sc) : 1.f;
    float pg = 0.f, pgt = 0.f, ptau = 0.f, p4g = 0.f, p2e = 0.f, pe = 0.f;
    if constexpr (PUR) {
        ptau = p.tau[p.per_head_tau ? h : 0];
        pg = sc;
        pgt = -sc * ptau;
        p4g = 4.f * sc;
        p2e = 2.f * p.eps_base;
        pe = p.eps_base;
    }
    float dg_acc = 0.f, dt_acc = 0.f;  // purified: sum u^3 dP (r - tau), sum u^3 dP

    // Stationary operands: sign-flipped K and V rows of this lane's key.
    u32x4 kr[KS], vr[KS];
    {
        const uint16_t* __restrict__ Kg = reinterpret_cast<const uint16_t*>(p.k) + base;
        const uint16_t* __restrict__ Vg = reinterpret_cast<const uint16_t*>(p.v) + base;
        const bool ok = key < T;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
            if (ok && (!PAD || 2 * ks + g < CG)) {
                x = ldg16(Kg + (size_t)key * D + (2 * ks + g) * 8);
                y = ldg16(Vg + (size_t)key * D + (2 * ks + g) * 8);
            }
            kr[ks] = x ^ flip;
            vr[ks] = y;
        }
    }
    // Documents: this lane's key's document id (INT_MIN past T; such keys
    // have zero K and V rows and are not stored).
    const int32_t* __restrict__ docb = nullptr;
    int kdoc = INT_MIN;
    if constexpr (DOC) {
        docb = p.doc + (size_t)(bh / p.H) * T;
        if (key < T) kdoc = docb[key];
    }

    // Query tiles q_lo + BQ u (documents: the candidates, screened below;
    // window: up to the last query that sees the block's last key).
    const int W = kWin ? p.window : 0;
    const int q_lo = kCaus ? K0 : 0;
    const int q_hi = kWin ? (int)min((int64_t)T, (int64_t)K0 + BK - 1 + W) : T;
    const int ntiles = (K0 < T) ? (q_hi - q_lo + BQ - 1) / BQ : 0;

    const uint32_t nrec = (uint32_t)T * (uint32_t)(2 * D);
    const i32x4 rq = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.q) + base, nrec);
    const i32x4 rd = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.dout) + base, nrec);
    const i32x4 rdl = buffer_rsrc(p.ndelta + (size_t)bh * T, (uint32_t)T * 4u);
    const i32x4 rzi = buffer_rsrc(p.zinv + (size_t)bh * T, (uint32_t)T * 4u);
    const i32x4 rdoc = buffer_rsrc(docb, DOC ? (uint32_t)T * 4u : 0u);
    auto swz = [](int r) __attribute__((always_inline)) { return ((r & 3) << 1) | ((r >> 2) & 1); };

    // Tile u (documents: kept tile u of the list) -> stage u % NST.  Waves 0
    // and 1 (documents: and 2) also bring the tile's -delta, 1/Z (and query
    // document ids), lanes 0-15, 16 bytes each: one more load per tile.
    const int kTileLoadsW = 2 * LPW + (wave < NROWV ? 1 : 0);
    auto tile_row0 = [&](int u) __attribute__((always_inline)) -> int {
        if constexpr (DOC) return q_lo + (__builtin_amdgcn_readfirstlane(t_list[u]) & ~kDocOne) * BQ;
        return q_lo + u * BQ;
    };
    auto issue = [&](int u) __attribute__((always_inline)) {
        uint8_t* sb = smem + (u % NST) * SB;
        const int i0 = tile_row0(u);
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int slot = (wave * LPW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int ch = pc ^ swz(row);
            const int off = (PAD && ch >= CG) ? kBufOOB : (i0 + row) * (2 * D) + (ch << 4);
            dma_load16(rq, lds_addr(sb + (wave * LPW + i) * 1024), off);
            dma_load16(rd, lds_addr(sb + TB + (wave * LPW + i) * 1024), off);
        }
        if (lane < 16) {
            const uint32_t la = lds_addr(sb + 2 * TB + wave * BQ * 4);
            if (wave == 0)
                dma_load16(rdl, la, (i0 + 4 * lane) * 4);
            else if (wave == 1)
                dma_load16(rzi, la, (i0 + 4 * lane) * 4);
            else if (DOC && wave == 2)
                dma_load16(rdoc, la, (i0 + 4 * lane) * 4);
        }
    };

    const int trow_l = 4 * g + ((lane & 15) >> 2);
    const int tcol_l = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    // Row reads (A of S and dPz): query row nb * 32 + c, chunk 2 ks + g.
    auto row_op = [&](const uint8_t* tb, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + c;
        return *reinterpret_cast<const u32x4*>(tb + row * RB + (((2 * ks + g) ^ swz(row)) << 4));
    };
    // Transposed reads (A of dV^T, dK^T): queries nb * 32 + hh * 16 + 4 g +
    // (lane & 15) / 4 (+8), d columns db * 32 + 16 ((lane >> 4) & 1) + 4 (lane & 3).
    auto tr_op = [&](const uint8_t* tb, int nb, int hh, int db) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + hh * 16 + trow_l;
        const int col = db * 32 + tcol_l;
        const uint8_t* b0 = tb + row * RB + (((col >> 3) ^ swz(row)) << 4) + (col & 7) * 2;
        const u32x2 x = lds_read_tr16(reinterpret_cast<const uint16_t*>(b0));
        const u32x2 y = lds_read_tr16(reinterpret_cast<const uint16_t*>(b0 + 8 * RB));
        const u32x4 a = {x[0], x[1], y[0], y[1]};
        return a;
    };

    f32x16 acc_v[DB], acc_k[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_v[db] = zero16(), acc_k[db] = zero16();

    // Documents, per tile: the wave's keys are tested per element (xm) or
    // not at all.
    bool xm = false;
    // One 32-query half nb of a tile (rows i0 + nb * 32 + 8 (r / 4) + 4 g +
    // r % 4 for register r).  One instantiation for every tile; the causal
    // mask (key past the query) applies under the uniform flag mk.
    auto half = [&](const uint8_t* sb, int nb, int qbase, auto mk) __attribute__((always_inline)) {
        const uint8_t* qt = sb;
        const uint8_t* dt = sb + TB;
        const float* dl = reinterpret_cast<const float*>(sb + 2 * TB);
        const float* zl = reinterpret_cast<const float*>(sb + 2 * TB + BQ * 4);
        f32x16 s = zero16(), dp;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dl + nb * 32 + 8 * i + 4 * g);
#pragma unroll
            for (int k = 0; k < 4; ++k) dp[4 * i + k] = d4[k];
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s = E::mfma(row_op(qt, nb, ks), kr[ks], s);
            dp = E::mfma(row_op(dt, nb, ks), vr[ks], dp);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        uint32_t w2[8], u2[8];
        if constexpr (PUR) {
            const int lim = qbase - key;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 z4 = *reinterpret_cast<const f32x4*>(zl + nb * 32 + 8 * i + 4 * g);
#pragma unroll
                for (int k = 0; k < 4; k += 2) {
                    float ww[2], uu[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int r = 4 * i + k + e;
                        const float x = s[r];
                        float u = __int_as_float(max(__float_as_int(fmaf(x, pg, pgt)), 0));
                        float bb = __int_as_float(max(__float_as_int(x), 0));
                        const int off = 8 * (r >> 2) + (r & 3);
                        if constexpr (DOC) {
                            const int32_t* qd = reinterpret_cast<const int32_t*>(sb + 2 * TB + 2 * BQ * 4);
                            if (xm && (pair_cut<kCaus, kWin>(off + lim, W) || qd[nb * 32 + 4 * g + off] != kdoc))
                                u = bb = 0.f;
                        } else {
                            if (mk && pair_cut<kCaus, kWin>(off + lim, W)) u = bb = 0.f;
                        }
                        const float u2_ = u * u;
                        const float dpz = dp[r] * z4[k + e];
                        const float a = u2_ * u * dpz;
                        dg_acc = fmaf(a, x - ptau, dg_acc);
                        dt_acc += a;
                        ww[e] = fmaf(u2_, u2_, pe * bb * bb) * z4[k + e];
                        uu[e] = fmaf(p4g, u2_ * u, p2e * bb) * dpz;
                    }
                    w2[(4 * i + k) >> 1] = E::pack(ww[0], ww[1]);
                    u2[(4 * i + k) >> 1] = E::pack(uu[0], uu[1]);
                }
            }
        } else {
        if constexpr (DOC) {
            // Query qbase + 8 (r / 4) + r % 4 of register r is masked before
            // the lane's key (causal) or in another document.
            if (xm) {
                const int lim = qbase - key;  // query - key of register 0
                const int32_t* qd = reinterpret_cast<const int32_t*>(sb + 2 * TB + 2 * BQ * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int4 d4 = *reinterpret_cast<const int4*>(qd + nb * 32 + 8 * i + 4 * g);
                    const int dq[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (pair_cut<kCaus, kWin>(8 * i + k + lim, W) || dq[k] != kdoc) s[4 * i + k] = 0.f;
                }
            }
        } else if (mk) {
            // Register r (query qbase + off) is masked before the lane's key
            // (off + lim < 0) and (window) past its window (off + lim >= W).
            const int lim = qbase - key;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                if ((kCaus && off + lim < 0) || (kWin && off + lim >= W)) s[r] = 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 z4 = *reinterpret_cast<const f32x4*>(zl + nb * 32 + 8 * i + 4 * g);
#pragma unroll
            for (int k = 0; k < 4; k += 2) {
                const int r = 4 * i + k;
                float x0 = s[r], x1 = s[r + 1];
                if constexpr (E::kScaleInSquare) x0 *= sq_pre, x1 *= sq_pre;
                const float a0 = __int_as_float(max(__float_as_int(x0), 0));
                const float a1 = __int_as_float(max(__float_as_int(x1), 0));
                const float t0 = a0 * z4[k], t1 = a1 * z4[k + 1];
                w2[r >> 1] = E::pack(t0 * a0, t1 * a1);
                u2[r >> 1] = E::pack(t0 * dp[r], t1 * dp[r + 1]);
            }
        }
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const u32x4 bw = {w2[4 * hh], w2[4 * hh + 1], w2[4 * hh + 2], w2[4 * hh + 3]};
            const u32x4 bu = {u2[4 * hh], u2[4 * hh + 1], u2[4 * hh + 2], u2[4 * hh + 3]};
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                acc_v[db] = E::mfma(tr_op(dt, nb, hh, db), bw, acc_v[db]);
                acc_k[db] = E::mfma(tr_op(qt, nb, hh, db), bu, acc_k[db]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };

    // Pipeline as in the dQ kernel: tiles 0 and 1 issued up front, tile u+2
    // right after the barrier that starts step u.
    if constexpr (DOC) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kr[ks]), "+v"(vr[ks]));
        // Document range of the wave's valid keys (uniform; kone: all of them
        // in document ksd) and of the whole block.
        int lo = key < T ? kdoc : INT_MAX, hi = key < T ? kdoc : INT_MIN;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            lo = min(lo, __shfl_xor(lo, off));
            hi = max(hi, __shfl_xor(hi, off));
        }
        lo = __builtin_amdgcn_readfirstlane(lo);
        hi = __builtin_amdgcn_readfirstlane(hi);
        const int ksd = lo;
        const bool kone = lo == hi;
        if (lane == 0) {
            s_rng[2 * wave] = lo;
            s_rng[2 * wave + 1] = hi;
        }
        __syncthreads();
        int bk_lo = INT_MAX, bk_hi = INT_MIN;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            bk_lo = min(bk_lo, s_rng[2 * w]);
            bk_hi = max(bk_hi, s_rng[2 * w + 1]);
        }
        for (int c0 = 0; c0 < ntiles; c0 += CAP) {
            const int n = screen_doc_tiles<BQ>(docb, T, q_lo, c0, min(CAP, ntiles - c0), bk_lo, bk_hi, t_keep, t_tdoc,
                                               t_list, t_doc, &s_rng[2 * NW]);
            if (n > 0) issue(0);
            if (n > 1) issue(1);
            for (int u = 0; u < n; ++u) {
                if (u + 1 < n) {
                    if (wave < NROWV)
                        wait_vmcnt<2 * LPW + 1>();
                    else
                        wait_vmcnt<2 * LPW>();
                } else {
                    wait_vmcnt<0>();
                }
                __syncthreads();
                if (u + 2 < n) issue(u + 2);
                const int e = __builtin_amdgcn_readfirstlane(t_list[u]);
                const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
                const int i0 = q_lo + (e & ~kDocOne) * BQ;
                if (kCaus && i0 + BQ - 1 < kw0) continue;  // every query before every key
                if (kWin && i0 > kw0 + 31 + W - 1) continue;  // every query past every key's window
                int soff = (u % NST) * SB;
                asm volatile("" : "+s"(soff));
                const uint8_t* sb = smem + soff;
                const bool mk = (kCaus && i0 < kw0 + 31) || (kWin && i0 + BQ - 1 >= kw0 + W);
                // Tested per element on the causal diagonal, at a window's
                // end, and unless the tile's queries and all of the wave's
                // keys are one and the same document.
                xm = mk || !((e & kDocOne) != 0 && kone && td == ksd);
                half(sb, 0, i0 + 4 * g, mk);
                half(sb, 1, i0 + 32 + 4 * g, mk);
            }
            __syncthreads();  // the list and the ring are reused by the next chunk
        }
    } else {
    if (ntiles > 0) issue(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kr[ks]), "+v"(vr[ks]));
    if (ntiles > 1) issue(1);
    // This wave's keys kw0 .. kw0 + 31 are seen by queries [kw0, kw0 + 31 +
    // W - 1] (causal, window), all of them by queries [kw0 + 31, kw0 + W - 1]:
    // its query tiles split into runs, the masked and the unmasked tile bodies
    // each in a loop of its own (one body with a runtime mask flag computes
    // the mask's compares and selects on every tile).
    static_assert(BQ == 64, "WaveRuns counts 64-row tiles");
    const WaveRuns runs(q_lo, ntiles, kCaus ? kw0 : 0, kWin ? kw0 + 31 + W - 1 : kRunsBig, kCaus ? kw0 + 31 : 0,
                        kWin ? kw0 + W - 1 : kRunsBig);
    int u = 0;
    auto step = [&]() __attribute__((always_inline)) {
        if (u + 1 < ntiles) {
            if (wave < 2)
                wait_vmcnt<2 * LPW + 1>();
            else
                wait_vmcnt<2 * LPW>();
        } else {
            wait_vmcnt<0>();
        }
        __syncthreads();
        if (u + 2 < ntiles) issue(u + 2);
    };
    auto run = [&](int tend, auto mk) __attribute__((always_inline)) {
        for (; u < tend; ++u) {
            step();
            int soff = (u % NST) * SB;
            asm volatile("" : "+s"(soff));
            const uint8_t* sb = smem + soff;
            const int i0 = q_lo + u * BQ;
            half(sb, 0, i0 + 4 * g, mk);
            half(sb, 1, i0 + 32 + 4 * g, mk);
        }
    };
    for (; u < runs.ta; ++u) step();
    run(runs.tf, std::true_type{});
    run(runs.tg, std::false_type{});
    run(runs.tv, std::true_type{});
    for (; u < ntiles; ++u) step();
    }
    (void)kTileLoadsW;

    // Epilogue: dK = 2 s|s| / c acc_k, dV = (s / c)^2 acc_v (c = sq_pre: 1,
    // or 2|s| for fp16, where the factors are s and 1/4;
    // purified: the accumulators as they are), packed, staged in the idle
    // ring (rows: dK at 0, dV at 128 rows) and stored 16 bytes per lane.
    __syncthreads();
    const float fk = PUR ? 1.f : E::kScaleInSquare ? sc : 2.f * sc * fabsf(sc);
    const float fv = PUR ? 1.f : E::kScaleInSquare ? (sc != 0.f ? 0.25f : 0.f) : sc * sc;
    if constexpr (PUR) {
        // Workgroup partials of dgamma and dtau in a fixed order (lanes, then
        // waves); keys past T excluded.
        float a = key < T ? 4.f * dg_acc : 0.f;
        float t2 = key < T ? -4.f * sc * dt_acc : 0.f;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            a += __shfl_xor(a, off);
            t2 += __shfl_xor(t2, off);
        }
        float* red = reinterpret_cast<float*>(smem + 2 * BK * RB);
        if (lane == 0) red[wave] = a, red[NW + wave] = t2;
        __syncthreads();
        if (tid == 0) {
            float sa = 0.f, st = 0.f;
            for (int w = 0; w < NW; ++w) sa += red[w], st += red[NW + w];
            p.part[bid] = sa;
            p.part[gridDim.x + bid] = st;
        }
    }
    int ln = lane;
    asm volatile("" : "+v"(ln));
    {
        const int row = 32 * wave + (ln & 31);
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            uint8_t* rb = smem + (which * BK + row) * RB;
            const float f = which ? fv : fk;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x16& o = which ? acc_v[db] : acc_k[db];
                    u32x2 w;
                    w[0] = E::pack(o[4 * j] * f, o[4 * j + 1] * f);
                    w[1] = E::pack(o[4 * j + 2] * f, o[4 * j + 3] * f);
                    const int chunk = 4 * db + j;
                    *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 7)) << 4) + 8 * (ln >> 5)) = w;
                }
        }
    }
    uint16_t* __restrict__ dK = reinterpret_cast<uint16_t*>(p.dk) + base;
    uint16_t* __restrict__ dV = reinterpret_cast<uint16_t*>(p.dv) + base;
    const int chunk = ln & 7;
#pragma unroll
    for (int which = 0; which < 2; ++which)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 32 * wave + 8 * i + (ln >> 3);
            const u32x4 x = *reinterpret_cast<const u32x4*>(smem + (which * BK + row) * RB + ((chunk ^ (row & 7)) << 4));
            const int kk = K0 + row;
            if (kk < T && (!PAD || chunk < CG))
                __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>((which ? dV : dK) + (size_t)kk * D + chunk * 8));
        }
}

template <class E, int DP, int MODE, bool DOC = false>
hipError_t launch_bwd16_dkdv_fast(const BwdArgs& a, hipStream_t st) {
    constexpr int BK = 128;
    const dim3 grid((unsigned)((a.T + BK - 1) / BK) * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_bwd16_dkdv_fast_kernel<E, DP, MODE, false, DOC>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace qdl
