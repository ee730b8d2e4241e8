// Flash-Born backward specialised for head dim D == 128 (no padding): dense,
// causal, or causal with a sliding window; Born weights, no document ids.
// Same arithmetic as the D == 64 kernels (born_bwd_fast.h), the same two
// launches (dQ first: it also forms delta and fills the workspace), with the
// register split the wider rows need:
//   * dQ (queries stationary): 8 waves over a 256-row query block, wave w
//     owning rows 32w .. 32w+31 (one MFMA column block: its Q and dO operands
//     are 64 VGPRs and its dQ accumulators 64).
//   * dK/dV (keys stationary): 8 waves over a 256-key block, wave w owning
//     keys 32w .. 32w+31 (K and V operands 64 VGPRs, dK and dV accumulators
//     128).
//   * Tiles of 64 rows (K, V for dQ; Q, dO plus -delta and 1/Z for dK/dV) go
//     global -> LDS with buffer_load ... lds through a ring of three stages,
//     one workgroup per CU.  Rows are 256 bytes, so every row starts on bank
//     0; 16-byte chunk c of row r sits at chunk c ^ swz256(r), conflict-free
//     both for the row reads (ds_read_b128 quarter-waves: 16 consecutive
//     rows of one chunk) and the transposed reads (ds_read_b64_tr_b16
//     half-waves: rows r0 .. r0+3, r0 % 4 == 0, of an aligned group of four
//     chunks).
//   * Each wave's tiles split into runs as in the D == 128 forward: tiles
//     none of its pairs see (no work, only the barrier), tiles its diagonal
//     or window edge cuts (masked per element), and tiles all of its pairs
//     see (no mask), each run in a loop of its own.
// PUR: the purified-Born gradients (flash_born.py:812-1061) as in the D == 64
// kernels' purified mode (bf16, dense or causal): dR = (4 gamma u^3 +
// 2 eps_base b) dP and W = p / Z rounded to bf16 before their contractions,
// O read in fp32, and the dK/dV kernel's workgroups writing their partial
// sums of dgamma and dtau (reduced per output afterwards in a fixed order).
// PAD: a head dim D < 128 (a multiple of 8) as in the D == 128 forward: the
// tile loads of chunks past D return zeros, the stationary rows are zero
// there, and the output chunks past D are not stored.
#pragma once

#include "born_bwd_fast.h"
#include "born_fwd_d128.h"
#include "purified_args.h"

namespace qdl {

__device__ __forceinline__ int swz256(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

struct BwdD128Cfg {
    static constexpr int DP = 128;
    static constexpr int NW = 8;    // waves per workgroup, two per SIMD
    static constexpr int BM = 256;  // dQ: query rows per block (32 per wave)
    static constexpr int NWK = 4;   // dK/dV: waves per workgroup, one per SIMD
    static constexpr int BK = 128;  // dK/dV: keys per block (32 per wave)
};

// NW (documents only): 4 waves over 128-row blocks, two workgroups per CU and
// a two-stage ring, as the document forward; otherwise 8 waves over 256-row
// blocks.
template <class E, int MODE, bool PUR = false, bool PAD = false, bool DOC = false, int NW = 8>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void born_bwd16_dq_d128_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    static_assert(MODE != kWindowNC || !DOC, "windows without causality: no documents");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified gradients: 16-bit");

    static_assert(NW == 8 || (NW == 4 && DOC), "128-row blocks: the document mode");
    constexpr int DP = 128, BN = 64, NST = NW == 8 ? 3 : 2, BM = 32 * NW;
    constexpr int KS = DP / 16, DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    constexpr int CAP = 256;               // documents: candidate tiles screened per pass
    constexpr int KDW = BN / NW;           // documents: key ids loaded per wave per tile
    // Loads per wave per tile: K, V (documents: and KDW of the key document ids).
    constexpr int kTileLoads = 2 * LPW + (DOC ? 1 : 0);
    static_assert(TB % (1024 * NW) == 0 && BM * RB <= 2 * NST * TB && BM == 32 * NW, "tile split / staging");
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);

    // The K/V ring during the tile loop, the output staging afterwards.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * NST * TB];
    __shared__ float s_dz[NW];
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
    const int qrow = R + 32 * wave + c;  // this lane's query row

    // Head dim in HBM: DP, or (PAD) D < DP with CG 16-byte chunks per row.
    const int D = PAD ? p.D : DP;
    const int CG = D / 8;
    const size_t base = (size_t)bh * T * D;
    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (!PUR && sc < 0.f) ? 0x80008000u : 0u;
    const float sq_pre = (E::kScaleInSquare && sc != 0.f) ? 2.f * fabsf(sc) : 1.f;
    // Purified: t = gamma r - gamma tau; dR / dP = 4 gamma u^3 + 2 eps_base b.
    float pg = 0.f, pgt = 0.f, p4g = 0.f, p2e = 0.f;
    if constexpr (PUR) {
        pg = sc;
        pgt = -sc * p.tau[p.per_head_tau ? h : 0];
        p4g = 4.f * sc;
        p2e = 2.f * p.eps_base;
    }

    // Stationary operands (sign-flipped Q, dO: B operands of S^T and T^T),
    // delta_i = dO_i . O_i from the stored O (each lane holds half a row, the
    // other half is in lane ^ 32), and the workspace rows -delta, 1/Z,
    // delta/Z for the dK/dV kernel and the dscale reduction.
    u32x4 qr[KS], dr[KS];
    float zinv, nd;
    {
        const uint16_t* __restrict__ Qg = reinterpret_cast<const uint16_t*>(p.q) + base;
        const uint16_t* __restrict__ dOg = reinterpret_cast<const uint16_t*>(p.dout) + base;
        const bool ok = qrow < T;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
            if (ok && (!PAD || 2 * ks + g < CG)) {
                x = ldg16(Qg + (size_t)qrow * D + (2 * ks + g) * 8);
                y = ldg16(dOg + (size_t)qrow * D + (2 * ks + g) * 8);
            }
            qr[ks] = x ^ flip;
            dr[ks] = y;
        }
        float dl = 0.f;
        if (ok) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if (PAD && 2 * ks + g >= CG) continue;  // dO is zero there
                if constexpr (PUR) {
                    const float* o32 = p.o_in + base + (size_t)qrow * D + (2 * ks + g) * 8;
                    const f32x4 oa = *reinterpret_cast<const f32x4*>(o32);
                    const f32x4 ob = *reinterpret_cast<const f32x4*>(o32 + 4);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float o0 = j < 2 ? oa[2 * j] : ob[2 * j - 4];
                        const float o1 = j < 2 ? oa[2 * j + 1] : ob[2 * j - 3];
                        dl += o0 * E::lo(dr[ks][j]) + o1 * E::hi(dr[ks][j]);
                    }
                } else {
                    const uint16_t* Og = reinterpret_cast<const uint16_t*>(p.o) + base;
                    const u32x4 o = ldg16(Og + (size_t)qrow * D + (2 * ks + g) * 8);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        dl += E::lo(o[j]) * E::lo(dr[ks][j]) + E::hi(o[j]) * E::hi(dr[ks][j]);
                }
            }
        }
        dl += __shfl_xor(dl, 32);
        const size_t row = (size_t)bh * T + qrow;
        float zr = 1.f;
        if (ok) {
            if constexpr (PUR)
                zr = p.z_in[row];
            else
                zr = p.z[row];
        }
        zinv = ok ? 1.0f / zr : 0.f;
        nd = ok ? -(dl / zr) : 0.f;
        if (ok && g == 0) {
            p.ndelta[row] = -dl;
            p.zinv[row] = zinv;
            if constexpr (!PUR) p.delta_z[row] = dl / zr;
        }
    }
    // This workgroup's part of dscale = (2/s) eps sum delta / Z (closed form):
    // its rows' sum in a fixed order (lanes, then waves), one double.
    if constexpr (!PUR) {
        float dz = (g == 0) ? -nd : 0.f;
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

    // Key tiles tb .. tb+ntiles-1 (tb: the window's first key tile, else 0).
    const int W = kWin ? p.window : 0;
    const int tb = kWin ? max(0, R - W + 1) / BN : 0;
    const int ntiles = (kCaus ? (min(T, R + BM) + BN - 1) / BN : (T + BN - 1) / BN) - tb;
    // This wave's rows rw .. rw + 31 see keys [rw - W + 1, rw + 31] (causal,
    // window) and all of them see keys [rw + 32 - W, rw].
    const int rw = R + 32 * wave;
    const WaveRuns runs(tb * BN, ntiles, kWin ? max(0, rw - W + 1) : 0, kCaus ? rw + 31 : kRunsBig,
                        kWin ? max(0, rw + 32 - W) : 0, kCaus ? rw : kRunsBig);

    const uint32_t nrec = (uint32_t)T * (uint32_t)(2 * D);
    const i32x4 rk = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.k) + base, nrec);
    const i32x4 rv = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.v) + base, nrec);
    const int32_t* __restrict__ docb = nullptr;
    if constexpr (DOC) docb = p.doc + (size_t)(bh / p.H) * T;
    const i32x4 rdoc = buffer_rsrc(docb, DOC ? (uint32_t)T * 4u : 0u);

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
            const int ch = pc ^ swz256(row);
            const int off = (PAD && ch >= CG) ? kBufOOB : (key0 + row) * (2 * D) + (ch << 4);
            dma_load16(rk, lds_addr(kb + (wave * LPW + i) * 1024), off);
            dma_load16(rv, lds_addr(vb + (wave * LPW + i) * 1024), off);
        }
        if constexpr (DOC)
            if (lane < KDW / 4)
                dma_load16(rdoc, lds_addr(kd_lds + st * BN + wave * KDW), (key0 + wave * KDW + lane * 4) * 4);
    };

    // Operand reads.  Rows: K/V row nb * 32 + c (A operands of S^T, T^T);
    // K^T: keys nb * 32 + hh * 16 + 4 g + (lane & 15) / 4 (+8), d columns
    // db * 32 + 16 ((lane >> 4) & 1) + 4 (lane & 3): the key order of the
    // accumulator layout of U.
    const int trow_l = 4 * g + ((lane & 15) >> 2);
    const int tcol_l = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    auto row_rd = [&](const uint8_t* tb_, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + c;
        return *reinterpret_cast<const u32x4*>(tb_ + row * RB + (((2 * ks + g) ^ swz256(row)) << 4));
    };
    auto tr_rd = [&](const uint8_t* tb_, int nb, int hh, int db) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + hh * 16 + trow_l;
        const int col = db * 32 + tcol_l;
        const uint8_t* b0 = tb_ + row * RB + (((col >> 3) ^ swz256(row)) << 4) + (col & 7) * 2;
        const uint8_t* b1 = tb_ + (row + 8) * RB + (((col >> 3) ^ swz256(row + 8)) << 4) + (col & 7) * 2;
        const u32x2 x = lds_read_tr16(reinterpret_cast<const uint16_t*>(b0));
        const u32x2 y = lds_read_tr16(reinterpret_cast<const uint16_t*>(b1));
        const u32x4 a = {x[0], x[1], y[0], y[1]};
        return a;
    };

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = zero16();

    constexpr int kFull = 1, kMasked = 2, kDocm = 3;
    using Full = std::integral_constant<int, kFull>;
    using Masked = std::integral_constant<int, kMasked>;
    using Docm = std::integral_constant<int, kDocm>;
    // Documents: the row's document id (INT_MIN past T); per tile, whether
    // this wave tests it per element (dmw) and the stage's key ids (kdp).
    const int qdoc = (DOC && qrow < T) ? docb[qrow] : INT_MIN;
    bool dmw = true;
    const int32_t* kdp = kd_lds;
    // One 32-key half nb of a tile:
    //   S^T = K Q^T, T^T = V dO^T      (A = K, V rows; B = Q^T, dO^T)
    //   U = relu(S^T) (T^T / Z - delta / Z), masked keys zeroed
    //   dQ^T += K^T U                    (A = K^T, B = U)
    // MFMAs at raised wave priority, the elementwise pass at normal priority.
    auto half = [&](const uint8_t* kb, const uint8_t* vb, int nb, int kbase, auto m) __attribute__((always_inline)) {
        f32x16 s = zero16(), t = zero16();
        uint32_t pk[8];
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s = E::mfma(row_rd(kb, nb, ks), qr[ks], s);
            t = E::mfma(row_rd(vb, nb, ks), dr[ks], t);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        if constexpr (PUR) {
            // A masked pair weighs zero even where its overlap is zero (u =
            // relu(-gamma tau) > 0 for tau < 0).  Keys past T need no mask
            // here: their K rows (zero) multiply U.
            const int lim = qrow - kbase;  // query - key of register 0
            const int wlo = kWin ? lim - W + 1 : 0;  // window: first visible key
            // Documents: bit r set for a register masked by the diagonal
            // (causal), the window or another document.
            uint32_t dmask = 0;
            if constexpr (decltype(m)::value == kDocm) {
                if (dmw) {
                    const int dlim = kCaus ? lim : INT_MAX;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int4 d4 = *reinterpret_cast<const int4*>(kdp + nb * 32 + 4 * g + 8 * i);
                        const int dk[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (8 * i + k > dlim || (kWin && 8 * i + k < wlo) || dk[k] != qdoc)
                                dmask |= 1u << (4 * i + k);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float w[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int r = 2 * j + e;
                    const float x = s[r];
                    const float uu = __int_as_float(max(__float_as_int(fmaf(x, pg, pgt)), 0));
                    const float bb = __int_as_float(max(__float_as_int(x), 0));
                    const float f = fmaf(p4g, uu * uu * uu, p2e * bb);
                    float d = f * fmaf(t[r], zinv, nd);
                    if constexpr (decltype(m)::value == kMasked) {
                        const int off = 8 * (r >> 2) + (r & 3);
                        // Causal with a window: one unsigned compare.
                        const bool cut = (kCaus && kWin) ? pair_cut<kCaus, kWin>(lim - off, W)
                                                         : ((kCaus && off > lim) || (kWin && off < wlo));
                        if (cut) d = 0.f;
                    }
                    if constexpr (decltype(m)::value == kDocm)
                        if ((dmask >> r) & 1u) d = 0.f;
                    w[e] = d;
                }
                pk[j] = E::pack(w[0], w[1]);
            }
        } else {
        if constexpr (decltype(m)::value == kMasked) {
            // Key kbase + 8 (r / 4) + r % 4 of register r: masked past the
            // lane's row, and (window) before its first key.
            const int lim = qrow - kbase;
            const int wlo = kWin ? lim - W + 1 : 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                if ((kCaus && off > lim) || (kWin && off < wlo)) s[r] = 0.f;
            }
        }
        if constexpr (decltype(m)::value == kDocm) {
            // Masked past the lane's row (causal) or in another document.
            if (dmw) {
                const int lim = kCaus ? qrow - kbase : INT_MAX;
                const int wlo = kWin ? lim - W + 1 : 0;  // window: first visible key
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int4 d4 = *reinterpret_cast<const int4*>(kdp + nb * 32 + 4 * g + 8 * i);
                    const int dk[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (8 * i + k > lim || (kWin && 8 * i + k < wlo) || dk[k] != qdoc) s[4 * i + k] = 0.f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float x0 = s[2 * j], x1 = s[2 * j + 1];
            if constexpr (E::kScaleInSquare) x0 *= sq_pre, x1 *= sq_pre;
            const float a0 = __int_as_float(max(__float_as_int(x0), 0));
            const float a1 = __int_as_float(max(__float_as_int(x1), 0));
            pk[j] = E::pack(a0 * fmaf(t[2 * j], zinv, nd), a1 * fmaf(t[2 * j + 1], zinv, nd));
        }
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const u32x4 bq = {pk[4 * hh], pk[4 * hh + 1], pk[4 * hh + 2], pk[4 * hh + 3]};
                acc[db] = E::mfma(tr_rd(kb, nb, hh, db), bq, acc[db]);
            }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };

    // Pipeline: tiles 0 and 1 issued up front (tile 1 after the stationary
    // loads have landed), tile u+2 right after the barrier that starts step
    // u; at that barrier each wave has waited for its share of tile u.
    if constexpr (DOC) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qr[ks]), "+v"(dr[ks]));
        asm volatile("" : "+v"(zinv), "+v"(nd));
        // Document range of this wave's valid rows (uniform; wone: one
        // document) and of the whole block.
        int wlo = qrow < T ? qdoc : INT_MAX, whi = qrow < T ? qdoc : INT_MIN;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            wlo = min(wlo, __shfl_xor(wlo, off));
            whi = max(whi, __shfl_xor(whi, off));
        }
        wlo = __builtin_amdgcn_readfirstlane(wlo);
        whi = __builtin_amdgcn_readfirstlane(whi);
        const bool wone = wlo == whi;
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
        // The kept tiles of each chunk of candidates through the same
        // pipeline.  Per tile and wave: nothing to do when the tile lies past
        // the wave's rows or is one document none of them belongs to; no
        // per-element test when it is before the wave's first row and one
        // document that all of them belong to.
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
                const int key0 = (tb + (e & ~kDocOne)) * BN;
                const bool one = (e & kDocOne) != 0;
                // Window: as in the forward.
                const bool vis = !(kCaus && key0 > rw + 31) && !(kWin && key0 + BN - 1 < rw - W + 1) &&
                                 !(one && (td < wlo || td > whi));
                dmw = (kCaus && key0 + BN - 1 > rw) || (kWin && key0 < rw + 32 - W) || !(one && wone && td == wlo);
                if (vis) {
                    half(kb, vb, 0, key0 + 4 * g, Docm{});
                    half(kb, vb, 1, key0 + 32 + 4 * g, Docm{});
                }
            }
            __syncthreads();  // the list and the ring are reused by the next chunk
        }
    } else {
    if (ntiles > 0) issue(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qr[ks]), "+v"(dr[ks]));
    asm volatile("" : "+v"(zinv), "+v"(nd));
    if (ntiles > 1) issue(1);
    int u = 0;
    auto step = [&]() __attribute__((always_inline)) {
        if (u + 1 < ntiles)
            wait_vmcnt<kTileLoads>();
        else
            wait_vmcnt<0>();
        __syncthreads();
        if (u + 2 < ntiles) issue(u + 2);
    };
    auto run = [&](int tend, auto m) __attribute__((always_inline)) {
        for (; u < tend; ++u) {
            step();
            int soff = (u % NST) * TB;
            asm volatile("" : "+s"(soff));
            const uint8_t* kb = k_lds + soff;
            const uint8_t* vb = v_lds + soff;
            const int key0 = (tb + u) * BN;
            half(kb, vb, 0, key0 + 4 * g, m);
            half(kb, vb, 1, key0 + 32 + 4 * g, m);
        }
    };
    for (; u < runs.ta; ++u) step();
    if constexpr (MODE == kDense) {
        // Nothing to mask (keys past T have zero K rows): one loop.
        run(ntiles, Full{});
    } else {
        run(runs.tf, Masked{});
        run(runs.tg, Full{});
        run(runs.tv, Masked{});
    }
    for (; u < ntiles; ++u) step();
    }

    // Epilogue: scale, pack, stage this wave's rows in the idle ring (row r
    // at smem + RB r, chunks XOR-swizzled by r & 15), read them back 16
    // bytes per lane and store 4 whole rows per instruction.
    __syncthreads();  // every wave is done with the ring
    uint16_t* __restrict__ dQ = reinterpret_cast<uint16_t*>(p.dq) + base;
    const float f = PUR ? 1.f : E::kScaleInSquare ? sc : 2.f * sc * fabsf(sc);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    {
        const int row = 32 * wave + (ln & 31);
        uint8_t* rb = smem + row * RB;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                u32x2 w;
                w[0] = E::pack(acc[db][4 * j] * f, acc[db][4 * j + 1] * f);
                w[1] = E::pack(acc[db][4 * j + 2] * f, acc[db][4 * j + 3] * f);
                const int chunk = 4 * db + j;
                *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 15)) << 4) + 8 * (ln >> 5)) = w;
            }
    }
    const int chunk = ln & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = 32 * wave + 4 * i + (ln >> 4);
        const u32x4 x = *reinterpret_cast<const u32x4*>(smem + row * RB + ((chunk ^ (row & 15)) << 4));
        const int q = R + row;
        if (q < T && (!PAD || chunk < CG))
            __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dQ + (size_t)q * D + chunk * 8));
    }
}

// NW (documents only): 2 waves over 64-key blocks and a two-stage ring, so
// that two workgroups share a CU (still one wave per SIMD) and one's
// start-up overlaps the other's tiles; otherwise 4 waves over 128 keys.
template <class E, int MODE, bool PUR = false, bool PAD = false, bool DOC = false, int NW = BwdD128Cfg::NWK>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(1, 1)))
void born_bwd16_dkdv_d128_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    static_assert(MODE != kWindowNC || !DOC, "windows without causality: no documents");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified gradients: 16-bit");
    static_assert(NW == 4 || (NW == 2 && DOC), "64-key blocks: the document mode");

    constexpr int DP = 128, BQ = 64, NST = NW == 4 ? 3 : 2, BK = 32 * NW;
    constexpr int KS = DP / 16, DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BQ * RB;            // bytes per Q or dO tile
    // Bytes per stage: Q, dO, -delta, 1/Z (documents: and the query document ids).
    constexpr int SB = 2 * TB + (DOC ? 3 : 2) * BQ * 4;
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of Q, dO)
    constexpr int CAP = 64 * NW;           // documents: candidate tiles screened per pass (one per thread)
    static_assert(TB % (1024 * NW) == 0 && BQ * 4 == 256 && BK * RB <= NST * SB && BK == 32 * NW,
                  "tile split / staging");
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

    // Query tiles q_lo + BQ u up to q_hi (window: the last query that sees
    // the block's last key).
    const int W = kWin ? p.window : 0;
    const int q_lo = kCaus ? K0 : 0;
    const int q_hi = kWin ? (int)min((int64_t)T, (int64_t)K0 + BK - 1 + W) : T;
    const int ntiles = (q_hi - q_lo + BQ - 1) / BQ;
    // This wave's keys kw0 .. kw0 + 31 are seen by queries [kw0, kw0 + 31 +
    // W - 1] (causal, window), all of them by queries [kw0 + 31, kw0 + W - 1].
    const WaveRuns runs(q_lo, ntiles, kCaus ? kw0 : 0, kWin ? kw0 + 31 + W - 1 : kRunsBig, kCaus ? kw0 + 31 : 0,
                        kWin ? kw0 + W - 1 : kRunsBig);

    const uint32_t nrec = (uint32_t)T * (uint32_t)(2 * D);
    const i32x4 rq = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.q) + base, nrec);
    const i32x4 rd = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.dout) + base, nrec);
    const i32x4 rdl = buffer_rsrc(p.ndelta + (size_t)bh * T, (uint32_t)T * 4u);
    const i32x4 rzi = buffer_rsrc(p.zinv + (size_t)bh * T, (uint32_t)T * 4u);
    const int32_t* __restrict__ docb = nullptr;
    if constexpr (DOC) docb = p.doc + (size_t)(bh / p.H) * T;
    const i32x4 rdoc = buffer_rsrc(docb, DOC ? (uint32_t)T * 4u : 0u);

    // Tile u (documents: kept tile u of the list) -> stage u % NST.  The
    // tile's -delta, 1/Z and (documents) query document ids (rows 0, 1, 2 of
    // 64 values after the Q and dO tiles) come in one load each (lanes 0-15,
    // 16 bytes each), row r from wave r % NW.
    constexpr int kRowLoaders = DOC ? 3 : 2;
    auto issue = [&](int u) __attribute__((always_inline)) {
        uint8_t* sb = smem + (u % NST) * SB;
        int i0 = q_lo + u * BQ;
        if constexpr (DOC) i0 = q_lo + (__builtin_amdgcn_readfirstlane(t_list[u]) & ~kDocOne) * BQ;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int slot = (wave * LPW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int ch = pc ^ swz256(row);
            const int off = (PAD && ch >= CG) ? kBufOOB : (i0 + row) * (2 * D) + (ch << 4);
            dma_load16(rq, lds_addr(sb + (wave * LPW + i) * 1024), off);
            dma_load16(rd, lds_addr(sb + TB + (wave * LPW + i) * 1024), off);
        }
        if (lane < 16) {
#pragma unroll
            for (int r = 0; r < kRowLoaders; ++r)
                if (wave == r % NW)
                    dma_load16(r == 0 ? rdl : r == 1 ? rzi : rdoc, lds_addr(sb + 2 * TB + r * BQ * 4),
                               (i0 + 4 * lane) * 4);
        }
    };

    // Operand reads.  Rows (A of S and dPz): query row nb * 32 + c, chunk
    // 2 ks + g.  Transposed (A of dV^T, dK^T): queries nb * 32 + hh * 16 +
    // 4 g + (lane & 15) / 4 (+8), d columns db * 32 + 16 ((lane >> 4) & 1) +
    // 4 (lane & 3).  swz256 is unchanged by the row steps of 8, 16 and 32, so
    // a lane's byte offsets within a stage are the 8 + 8 below plus
    // constants: each tile adds its stage base to them once and every read
    // takes its constant part as the instruction's immediate offset.
    int roff[KS], toff[DB][2];
    {
        const int trow_l = 4 * g + ((lane & 15) >> 2);
        const int tcol_l = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) roff[ks] = c * RB + (((2 * ks + g) ^ swz256(c)) << 4);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int row = trow_l + 8 * e;
                const int col = db * 32 + tcol_l;
                toff[db][e] = row * RB + (((col >> 3) ^ swz256(row)) << 4) + (col & 7) * 2;
            }
    }
    struct Bases {
        const uint8_t* r[KS];
        const uint8_t* t[DB][2];
    };
    auto bases_of = [&](const uint8_t* sb) __attribute__((always_inline)) -> Bases {
        Bases b;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) b.r[ks] = sb + roff[ks];
#pragma unroll
        for (int db = 0; db < DB; ++db) b.t[db][0] = sb + toff[db][0], b.t[db][1] = sb + toff[db][1];
        return b;
    };
    // which: 0 = Q, 1 = dO (the second tile of the stage).
    auto row_rd = [&](const Bases& b, int which, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        return *reinterpret_cast<const u32x4*>(b.r[ks] + which * TB + nb * 32 * RB);
    };
    auto tr_rd = [&](const Bases& b, int which, int nb, int hh, int db) __attribute__((always_inline)) -> u32x4 {
        const int k = which * TB + (nb * 32 + hh * 16) * RB;
        const u32x2 x = lds_read_tr16(reinterpret_cast<const uint16_t*>(b.t[db][0] + k));
        const u32x2 y = lds_read_tr16(reinterpret_cast<const uint16_t*>(b.t[db][1] + k));
        const u32x4 a = {x[0], x[1], y[0], y[1]};
        return a;
    };

    f32x16 acc_v[DB], acc_k[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_v[db] = zero16(), acc_k[db] = zero16();

    constexpr int kFull = 1, kMasked = 2, kDocm = 3;
    using Full = std::integral_constant<int, kFull>;
    using Masked = std::integral_constant<int, kMasked>;
    using Docm = std::integral_constant<int, kDocm>;
    // Documents: the lane's key document id (INT_MIN past T); per tile,
    // whether this wave tests it per element.
    const int kdoc = (DOC && key < T) ? docb[key] : INT_MIN;
    bool dmw = true;
    // Per 32-query half nb of a tile (queries i0 + nb * 32 + 8 (r / 4) +
    // 4 g + r % 4 for register r; one key per lane):
    //   S   = Q K'^T                  (A = Q rows)
    //   dPz = dO V^T - delta          (A = dO rows, accumulator initialised
    //                                  with -delta from LDS)
    //   t = relu(S) / Z_i, W = t relu(S), U = t dPz   (masked queries zeroed)
    //   dV^T += dO^T W,  dK^T += Q^T U   (A = dO^T, Q^T transposed reads)
    // One wave per SIMD leaves nothing to hide a wave's LDS latency behind
    // but its own work, so a tile runs as four fenced phases with every
    // phase's operands read one phase earlier (the first phase's right after
    // the tile's barrier):
    //   1: S, dPz of half 0                         reads rows of half 1
    //   2: S, dPz of half 1 | elementwise(half 0)   reads Q^T, dO^T of half 0
    //   3: dV, dK += half 0 | elementwise(half 1)   reads Q^T, dO^T of half 1
    //   4: dV, dK += half 1
    auto read_rows = [&](const Bases& b, int which, int nb, u32x4 (&dst)[KS]) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) dst[ks] = row_rd(b, which, nb, ks);
    };
    auto read_tr = [&](const Bases& b, int which, int nb, u32x4 (&dst)[2][DB]) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db) dst[hh][db] = tr_rd(b, which, nb, hh, db);
    };
    auto sdp = [&](const u32x4 (&aq)[KS], const u32x4 (&ad)[KS], f32x16& s, f32x16& dp) __attribute__((always_inline)) {
        s = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s = E::mfma(aq[ks], kr[ks], s);
            dp = E::mfma(ad[ks], vr[ks], dp);
        }
    };
    auto init_dp = [&](const uint8_t* sb, int nb, f32x16& dp) __attribute__((always_inline)) {
        const float* dl = reinterpret_cast<const float*>(sb + 2 * TB);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dl + nb * 32 + 8 * i + 4 * g);
#pragma unroll
            for (int k = 0; k < 4; ++k) dp[4 * i + k] = d4[k];
        }
    };
    auto elementwise = [&](const uint8_t* sb, int nb, int qbase, f32x16& s, const f32x16& dp, uint32_t (&w2)[8],
                           uint32_t (&u2)[8], auto m) __attribute__((always_inline)) {
        const float* zl = reinterpret_cast<const float*>(sb + 2 * TB + BQ * 4);
        if constexpr (PUR) {
            // Masked pairs (query before the lane's key; documents: in
            // another document) weigh zero; queries past T have 1/Z = 0 from
            // the workspace read.
            const int lim = qbase - key;
            uint32_t dmask = 0;
            if constexpr (decltype(m)::value == kDocm) {
                if (dmw) {
                    const int32_t* qd = reinterpret_cast<const int32_t*>(sb + 2 * TB + 2 * BQ * 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int4 d4 = *reinterpret_cast<const int4*>(qd + nb * 32 + 8 * i + 4 * g);
                        const int dq[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (pair_cut<kCaus, kWin>(8 * i + k + lim, W) || dq[k] != kdoc)
                                dmask |= 1u << (4 * i + k);
                    }
                }
            }
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
                        if constexpr (decltype(m)::value == kMasked) {
                            const int off = 8 * (r >> 2) + (r & 3);
                            if (pair_cut<kCaus, kWin>(off + lim, W)) u = bb = 0.f;
                        }
                        if constexpr (decltype(m)::value == kDocm)
                            if ((dmask >> r) & 1u) u = bb = 0.f;
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
            return;
        }
        if constexpr (decltype(m)::value == kDocm) {
            // Masked before the lane's key (causal) or in another document.
            if (dmw) {
                const int lim = kCaus ? qbase - key : INT_MAX / 2;
                const int32_t* qd = reinterpret_cast<const int32_t*>(sb + 2 * TB + 2 * BQ * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int4 d4 = *reinterpret_cast<const int4*>(qd + nb * 32 + 8 * i + 4 * g);
                    const int dq[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (8 * i + k + lim < 0 || (kWin && 8 * i + k + lim >= W) || dq[k] != kdoc) s[4 * i + k] = 0.f;
                }
            }
        }
        if constexpr (decltype(m)::value == kMasked) {
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
    };
    auto dvdk = [&](const u32x4 (&td)[2][DB], const u32x4 (&tq)[2][DB], const uint32_t (&w2)[8],
                    const uint32_t (&u2)[8]) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const u32x4 bw = {w2[4 * hh], w2[4 * hh + 1], w2[4 * hh + 2], w2[4 * hh + 3]};
            const u32x4 bu = {u2[4 * hh], u2[4 * hh + 1], u2[4 * hh + 2], u2[4 * hh + 3]};
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                acc_v[db] = E::mfma(td[hh][db], bw, acc_v[db]);
                acc_k[db] = E::mfma(tq[hh][db], bu, acc_k[db]);
            }
        }
    };
    // VALU instructions interleaved per MFMA (the purified elementwise pass
    // is about three times the Born one).
    constexpr int VE = PUR ? 14 : 5;
    auto tile = [&](const uint8_t* sb, int i0, auto m) __attribute__((always_inline)) {
        const Bases bs = bases_of(sb);
        u32x4 rq0[KS], rd0[KS], rq1[KS], rd1[KS];
        u32x4 tq0[2][DB], td0[2][DB], tq1[2][DB], td1[2][DB];
        f32x16 s0, dp0, s1, dp1;
        uint32_t w0[8], u0[8], w1[8], u1[8];
        read_rows(bs, 0, 0, rq0);
        read_rows(bs, 1, 0, rd0);
        init_dp(sb, 0, dp0);
        init_dp(sb, 1, dp1);
        // 1
        __builtin_amdgcn_s_setprio(1);
        read_rows(bs, 0, 1, rq1);
        read_rows(bs, 1, 1, rd1);
        sdp(rq0, rd0, s0, dp0);
        __builtin_amdgcn_sched_barrier(0);
        // 2
        __builtin_amdgcn_s_setprio(0);
        read_tr(bs, 0, 0, tq0);
        read_tr(bs, 1, 0, td0);
        sdp(rq1, rd1, s1, dp1);
        elementwise(sb, 0, i0 + 4 * g, s0, dp0, w0, u0, m);
#pragma unroll
        for (int i = 0; i < 2 * KS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, VE, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
        }
        __builtin_amdgcn_sched_barrier(0);
        // 3
        read_tr(bs, 0, 1, tq1);
        read_tr(bs, 1, 1, td1);
        dvdk(td0, tq0, w0, u0);
        elementwise(sb, 1, i0 + 32 + 4 * g, s1, dp1, w1, u1, m);
#pragma unroll
        for (int i = 0; i < 4 * DB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x002, VE, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        // 4
        __builtin_amdgcn_s_setprio(1);
        dvdk(td1, tq1, w1, u1);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };

    // Pipeline as in the dQ kernel.  The stationary operands are pinned in
    // AGPRs (MFMA reads its A/B operands from either file), leaving the
    // VGPRs to the phases' operand buffers.
    if constexpr (DOC) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+a"(kr[ks]), "+a"(vr[ks]));
        // Document range of this wave's valid keys (uniform; kone: one
        // document) and of the whole block.
        int klo = key < T ? kdoc : INT_MAX, khi = key < T ? kdoc : INT_MIN;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            klo = min(klo, __shfl_xor(klo, off));
            khi = max(khi, __shfl_xor(khi, off));
        }
        klo = __builtin_amdgcn_readfirstlane(klo);
        khi = __builtin_amdgcn_readfirstlane(khi);
        const bool kone = klo == khi;
        if (lane == 0) {
            s_rng[2 * wave] = klo;
            s_rng[2 * wave + 1] = khi;
        }
        __syncthreads();
        int bk_lo = INT_MAX, bk_hi = INT_MIN;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            bk_lo = min(bk_lo, s_rng[2 * w]);
            bk_hi = max(bk_hi, s_rng[2 * w + 1]);
        }
        // The kept query tiles of each chunk of candidates through the same
        // pipeline.  Per tile and wave: nothing to do when the tile ends
        // before the wave's first key or is one document none of its keys
        // belongs to; no per-element test when it starts after the wave's
        // last key and is one document that all of them belong to.
        for (int c0 = 0; c0 < ntiles; c0 += CAP) {
            const int n = screen_doc_tiles<BQ>(docb, T, q_lo, c0, min(CAP, ntiles - c0), bk_lo, bk_hi, t_keep, t_tdoc,
                                               t_list, t_doc, &s_rng[2 * NW]);
            // Tiles 0 .. NST-2 up front, tile u+NST-1 after the barrier of
            // step u (into the stage of tile u-1).
            if (n > 0) issue(0);
            if (NST == 3 && n > 1) issue(1);
            for (int u = 0; u < n; ++u) {
                if (NST == 3 && u + 1 < n) {
                    if (wave < kRowLoaders)
                        wait_vmcnt<2 * LPW + 1>();
                    else
                        wait_vmcnt<2 * LPW>();
                } else {
                    wait_vmcnt<0>();
                }
                __syncthreads();
                if (u + NST - 1 < n) issue(u + NST - 1);
                int soff = (u % NST) * SB;
                asm volatile("" : "+s"(soff));
                const int e = __builtin_amdgcn_readfirstlane(t_list[u]);
                const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
                const int i0 = q_lo + (e & ~kDocOne) * BQ;
                const bool one = (e & kDocOne) != 0;
                // Window: the tile is past every key's window when it starts
                // after the last key's, and cut by one when it ends after
                // the first key's.
                const bool vis = !(kCaus && i0 + BQ - 1 < kw0) && !(kWin && i0 > kw0 + 31 + W - 1) &&
                                 !(one && (td < klo || td > khi));
                dmw = (kCaus && i0 < kw0 + 31) || (kWin && i0 + BQ - 1 >= kw0 + W) || !(one && kone && td == klo);
                if (vis) tile(smem + soff, i0, Docm{});
            }
            __syncthreads();  // the list and the ring are reused by the next chunk
        }
    } else {
    if (ntiles > 0) issue(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+a"(kr[ks]), "+a"(vr[ks]));
    if (ntiles > 1) issue(1);
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
    auto run = [&](int tend, auto m) __attribute__((always_inline)) {
        for (; u < tend; ++u) {
            step();
            int soff = (u % NST) * SB;
            asm volatile("" : "+s"(soff));
            tile(smem + soff, q_lo + u * BQ, m);
        }
    };
    for (; u < runs.ta; ++u) step();
    run(runs.tf, Masked{});
    run(runs.tg, Full{});
    run(runs.tv, Masked{});
    for (; u < ntiles; ++u) step();
    }

    // Epilogue: dK = 2 s|s| / c acc_k, dV = (s / c)^2 acc_v (c = sq_pre: 1,
    // or 2|s| for fp16, where the factors are s and 1/4),
    // packed and staged, one output at a time, in this wave's own 32 rows of
    // the idle ring (row r at smem + RB r, chunks XOR-swizzled by r & 15),
    // then read back 16 bytes per lane and stored 4 whole rows per
    // instruction.
    __syncthreads();  // every wave is done with the ring
    const float fk = PUR ? 1.f : E::kScaleInSquare ? sc : 2.f * sc * fabsf(sc);
    const float fv = PUR ? 1.f : E::kScaleInSquare ? (sc != 0.f ? 0.25f : 0.f) : sc * sc;
    if constexpr (PUR) {
        // Workgroup partials of dgamma and dtau in a fixed order (lanes, then
        // waves), past the output staging; keys past T excluded (their zero
        // K row still weighs relu(-gamma tau) when tau < 0).
        float a = key < T ? 4.f * dg_acc : 0.f;
        float t2 = key < T ? -4.f * sc * dt_acc : 0.f;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            a += __shfl_xor(a, off);
            t2 += __shfl_xor(t2, off);
        }
        float* red = reinterpret_cast<float*>(smem + BK * RB);
        if (lane == 0) red[wave] = a, red[NW + wave] = t2;
        __syncthreads();
        if (tid == 0) {
            float sa = 0.f, st = 0.f;
            for (int w = 0; w < NW; ++w) sa += red[w], st += red[NW + w];
            p.part[bid] = sa;
            p.part[gridDim.x + bid] = st;
        }
    }
    uint16_t* __restrict__ dK = reinterpret_cast<uint16_t*>(p.dk) + base;
    uint16_t* __restrict__ dV = reinterpret_cast<uint16_t*>(p.dv) + base;
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int which = 0; which < 2; ++which) {
        const int row = 32 * wave + (ln & 31);
        uint8_t* rb = smem + row * RB;
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
                *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 15)) << 4) + 8 * (ln >> 5)) = w;
            }
        const int chunk = ln & 15;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r2 = 32 * wave + 4 * i + (ln >> 4);
            const u32x4 x = *reinterpret_cast<const u32x4*>(smem + r2 * RB + ((chunk ^ (r2 & 15)) << 4));
            const int kk = K0 + r2;
            if (kk < T && (!PAD || chunk < CG))
                __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>((which ? dV : dK) + (size_t)kk * D + chunk * 8));
        }
    }
}

// The D == 128 backward: dQ (and the workspace), dK/dV, then dscale from the
// dQ kernel's per-workgroup sums.
// DOC: document ids (no window) on the same kernels' document mode.
template <class E, int MODE, bool PAD = false, bool DOC = false>
hipError_t launch_bwd16_d128(const BwdArgs& a, hipStream_t st) {
    const unsigned BH = (unsigned)(a.B * a.H);
    // dQ: 256-row blocks of 8 waves, 128-row blocks of 4 with documents (one
    // dscale partial per workgroup either way).
    constexpr int NWQ = DOC ? 4 : BwdD128Cfg::NW, BMQ = 32 * NWQ;
    // dK/dV: 128-key blocks of 4 waves, 64-key blocks of 2 with documents.
    constexpr int NWK = DOC ? 2 : BwdD128Cfg::NWK, BKK = 32 * NWK;
    const unsigned nq = (unsigned)((a.T + BMQ - 1) / BMQ);
    const unsigned nk = (unsigned)((a.T + BKK - 1) / BKK);
    hipLaunchKernelGGL((born_bwd16_dq_d128_kernel<E, MODE, false, PAD, DOC, NWQ>), dim3(nq * BH), dim3(NWQ * 64), 0,
                       st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((born_bwd16_dkdv_d128_kernel<E, MODE, false, PAD, DOC, NWK>), dim3(nk * BH), dim3(NWK * 64), 0,
                       st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(born_bwd_dscale_groups_kernel<0>, dim3((unsigned)(a.per_head_scale ? a.H : 1)), dim3(256), 0,
                       st, a, (int)(nq * BH));
    return hipGetLastError();
}

// The purified D == 128 backward (bf16 or fp16): dQ (and the workspace),
// dK/dV (and the dgamma / dtau partials); the caller reduces the partials (one
// per dK/dV workgroup: B H ceil(T / 128), with documents B H ceil(T / 64)).
template <int MODE, bool PAD = false, bool DOC = false, class E = BF16>
hipError_t launch_purified_bwd_d128(const PurArgs& a, hipStream_t st) {
    const unsigned BH = (unsigned)(a.B * a.H);
    constexpr int NWQ = DOC ? 4 : BwdD128Cfg::NW, BMQ = 32 * NWQ;
    constexpr int NWK = DOC ? 2 : BwdD128Cfg::NWK, BKK = 32 * NWK;
    const unsigned nq = (unsigned)((a.T + BMQ - 1) / BMQ);
    const unsigned nk = (unsigned)((a.T + BKK - 1) / BKK);
    hipLaunchKernelGGL((born_bwd16_dq_d128_kernel<E, MODE, true, PAD, DOC, NWQ>), dim3(nq * BH), dim3(NWQ * 64), 0,
                       st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((born_bwd16_dkdv_d128_kernel<E, MODE, true, PAD, DOC, NWK>), dim3(nk * BH), dim3(NWK * 64), 0,
                       st, a);
    return hipGetLastError();
}

}  // namespace qdl
