// Flash-Born backward for head dims 128 < D <= 256 (bf16 / fp16): dense,
// causal, or a sliding window with or without causality; Born weights, no
// document ids.  The arithmetic and the two launches of the D == 128 kernels
// (born_bwd_d128.h: dQ first, forming delta and the workspace; then dK/dV;
// then dscale from the dQ workgroups' sums), with the register split that
// 512-byte rows force:
//   * dQ (queries stationary): a wave's 32 query rows need 64 VGPRs of Q and
//     64 of dO operands and 128 registers of dQ accumulators, so the kernel
//     runs one wave per SIMD (4 waves over a 128-row block) with the
//     accumulators in AGPRs.
//   * dK/dV (keys stationary): a wave's 32 keys need 128 VGPRs of K and V
//     operands and 256 registers of dK and dV accumulators: one wave per
//     SIMD (4 waves over a 128-key block), every AGPR an accumulator.
//   * Tiles of 64 rows (K, V for dQ; Q, dO plus -delta and 1/Z for dK/dV)
//     go global -> LDS with buffer_load ... lds through a ring of two stages
//     (32 KiB per tile), one workgroup per CU.  Rows are 512 bytes; 16-byte
//     chunk c of row r sits at chunk c ^ swz256(r) (the swizzle touches the
//     low four bits of the chunk index, which select the bank group), so the
//     row reads and the transposed reads are conflict-free as at D == 128.
//   * With one wave per SIMD no second wave hides a wave's LDS latency, so
//     each 32-row half of a tile runs as fenced phases (overlaps and products;
//     elementwise; accumulation) whose operand reads the scheduler issues a
//     few MFMAs ahead inside the phase.
// Each MFMA takes one operand from LDS (the other is stationary in
// registers): the kernels are bound by LDS bandwidth and MFMA issue together.
// PAD: 128 < D < 256 (a multiple of 8) on the same kernels: the loads of the
// chunks past D return zeros, the stationary rows are zero there, and the
// output chunks past D are not stored.
// PUR: the purified-Born gradients (flash_born.py:812-1061) as in the D == 128
// kernels' purified mode: dR = (4 gamma u^3 + 2 eps_base b) dP and W = p / Z
// rounded to the input dtype before their contractions, O read in fp32, and
// the dK/dV workgroups writing their partial sums of dgamma and dtau (reduced
// per output afterwards in a fixed order).
// DOC: document ids (with or without a causal window) as in the D == 128
// kernels' document mode: each block screens its candidate tiles (key tiles
// for dQ, query tiles for dK/dV) by document-id range into a list in LDS,
// loads each kept tile's 64 ids with it, skips a tile per wave that lies on
// the invisible side of its diagonal or window or is one document none of
// its rows (keys) belongs to, and tests the rest per element unless document
// and diagonal allow none.
#pragma once

#include "born_bwd_d128.h"

namespace qdl {

struct BwdD256Cfg {
    static constexpr int DP = 256;
    static constexpr int NW = 4;    // waves per workgroup, one per SIMD
    static constexpr int BM = 128;  // dQ: query rows per block (32 per wave)
    static constexpr int BK = 128;  // dK/dV: keys per block (32 per wave)
    static constexpr int LEAD = 4;  // operand reads in flight ahead of the MFMAs
};

// A lane's LDS byte offsets into the two-stage ring of 64-row tiles of
// 512-byte rows (chunk c of row r at chunk c ^ swz256(r)).  swz256 reads bits
// 0-3 of the row and changes bits 0-3 of the chunk, so steps of 16 rows and
// of 16 chunks move every offset by a constant: 8 offsets serve the row reads
// (row 32 nb + c, chunk 2 ks + g: r[ks & 7] + 256 (ks >> 3) + 32 RB nb) and 8
// the transposed reads (rows 32 nb + 16 hh + 4 g + (lane & 15) / 4 + 8 e,
// columns 32 db + 16 ((lane >> 4) & 1) + 4 (lane & 3): t[db & 3][e] + 256
// (db >> 2) + RB (32 nb + 16 hh)), the rest being instruction immediates
// (below 64 KiB).  Stage st's two tiles start at 64 KiB st, so moving to the
// other stage flips bit 16 of every offset in place (flip()): the 16 VGPRs are
// the kernel's only LDS addresses.
struct RingOffs512 {
    int r[8], t[4][2];
    __device__ __forceinline__ RingOffs512(int lane) {
        constexpr int RB = 512;
        const int c = lane & 31, g = lane >> 5;
        const int trow = 4 * g + ((lane & 15) >> 2);
        const int tcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = c * RB + (((2 * j + g) ^ swz256(c)) << 4);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int row = trow + 8 * e;
                t[j][e] = row * RB + (((4 * j + (tcol >> 3)) ^ swz256(row)) << 4) + (tcol & 7) * 2;
            }
    }
    __device__ __forceinline__ void flip() {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            r[j] ^= 0x10000;
            asm volatile("" : "+v"(r[j]));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                t[j][e] ^= 0x10000;
                asm volatile("" : "+v"(t[j][e]));
            }
    }
    // which: the first (0) or second (1) tile of the stage.
    __device__ __forceinline__ u32x4 row(const uint8_t* lds, int which, int nb, int ks) const {
        return *reinterpret_cast<const u32x4*>(lds + r[ks & 7] + which * 32768 + nb * 32 * RB_ + (ks >> 3) * 256);
    }
    __device__ __forceinline__ u32x4 tr(const uint8_t* lds, int which, int nb, int hh, int db) const {
        const int k = which * 32768 + (nb * 32 + hh * 16) * RB_ + (db >> 2) * 256;
        const u32x2 x = lds_read_tr16(reinterpret_cast<const uint16_t*>(lds + t[db & 3][0] + k));
        const u32x2 y = lds_read_tr16(reinterpret_cast<const uint16_t*>(lds + t[db & 3][1] + k));
        const u32x4 a = {x[0], x[1], y[0], y[1]};
        return a;
    }
    static constexpr int RB_ = 512;
};

template <class E, int MODE, bool PAD = false, bool PUR = false, bool DOC = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void born_bwd16_dq_d256_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified gradients: 16-bit");
    static_assert(MODE != kWindowNC || !DOC, "windows without causality: no documents");
    constexpr int DP = 256, NW = BwdD256Cfg::NW, BN = 64, NST = 2, BM = BwdD256Cfg::BM;
    constexpr int KS = DP / 16, DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    static_assert(TB % (1024 * NW) == 0 && BM * RB <= 2 * NST * TB && BM == 32 * NW, "tile split / staging");
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);

    // The K/V ring during the tile loop (stage st: K tile at smem + 2 TB st,
    // V tile right after it), the output staging afterwards.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * NST * TB];
    __shared__ float s_dz[NW];
    // Documents: key document ids per stage, the kept-tile list and screening scratch.
    constexpr int CAP = 64 * NW;  // candidate tiles screened per pass (one per thread)
    constexpr int KDW = BN / NW;  // key ids loaded per wave per tile
    __shared__ __attribute__((aligned(16))) int32_t kd_lds[DOC ? NST * BN : 1];
    __shared__ int32_t t_list[DOC ? CAP : 1], t_doc[DOC ? CAP : 1], t_keep[DOC ? CAP : 1], t_tdoc[DOC ? CAP : 1];
    __shared__ int32_t s_rng[DOC ? 2 * NW + 1 : 1];

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
    // delta = dO . O from the stored O (each lane holds half a row, the other
    // half is in lane ^ 32; purified: the fp32 O), and the workspace rows
    // -delta, 1/Z (Born: and delta/Z).
    u32x4 qr[KS], dr[KS];
    float zinv, nd;
    {
        const uint16_t* __restrict__ Qg = reinterpret_cast<const uint16_t*>(p.q) + base;
        const uint16_t* __restrict__ dOg = reinterpret_cast<const uint16_t*>(p.dout) + base;
        const bool ok = qrow < T;
        float dl = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
            const bool in = ok && (!PAD || 2 * ks + g < CG);
            if (in) {
                x = ldg16(Qg + (size_t)qrow * D + (2 * ks + g) * 8);
                y = ldg16(dOg + (size_t)qrow * D + (2 * ks + g) * 8);
            }
            qr[ks] = x ^ flip;
            dr[ks] = y;
            if constexpr (PUR) {
                if (in) {
                    const float* o32 = p.o_in + base + (size_t)qrow * D + (2 * ks + g) * 8;
                    const f32x4 oa = *reinterpret_cast<const f32x4*>(o32);
                    const f32x4 ob = *reinterpret_cast<const f32x4*>(o32 + 4);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float o0 = j < 2 ? oa[2 * j] : ob[2 * j - 4];
                        const float o1 = j < 2 ? oa[2 * j + 1] : ob[2 * j - 3];
                        dl += o0 * E::lo(y[j]) + o1 * E::hi(y[j]);
                    }
                }
            } else {
                u32x4 o = {0u, 0u, 0u, 0u};
                if (in) o = ldg16(reinterpret_cast<const uint16_t*>(p.o) + base + (size_t)qrow * D + (2 * ks + g) * 8);
#pragma unroll
                for (int j = 0; j < 4; ++j) dl += E::lo(o[j]) * E::lo(y[j]) + E::hi(o[j]) * E::hi(y[j]);
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
    // wave-instruction i writes LDS slots (wave * LPW + i) * 64 + lane, slot =
    // row * CPR + chunk'; documents: also this wave's KDW of the tile's key
    // ids (lanes 0 .. KDW/4 - 1, 16 bytes each).
    auto issue = [&](int u) __attribute__((always_inline)) {
        const int st = u % NST;
        int key0 = (tb + u) * BN;
        if constexpr (DOC) key0 = (tb + (__builtin_amdgcn_readfirstlane(t_list[u]) & ~kDocOne)) * BN;
        uint8_t* kb = smem + st * 2 * TB;
        uint8_t* vb = kb + TB;
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

    // Operand reads (rows: A operands of S^T, T^T; K^T, transposed: A of
    // dQ^T, in the key order of the accumulator layout of U) through the
    // ring's lane offsets (current stage); which = 0 (K) or 1 (V).
    static_assert(2 * TB == 0x10000, "stages 64 KiB apart");
    RingOffs512 ro(lane);
    constexpr int LEAD = BwdD256Cfg::LEAD;

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        acc[db] = zero16();
        asm volatile("" : "+a"(acc[db]));
    }

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
    // Each phase's operand reads run LEAD MFMAs ahead of their use.
    auto half = [&](int nb, int kbase, auto m) __attribute__((always_inline)) {
        f32x16 s = zero16(), t = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s = E::mfma(ro.row(smem, 0, nb, ks), qr[ks], s);
            t = E::mfma(ro.row(smem, 1, nb, ks), dr[ks], t);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 0);  // DS read
#pragma unroll
        for (int i = 0; i < 2 * KS - LEAD; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, LEAD, 0);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t pk[8];
        if constexpr (PUR) {
            // A masked pair weighs zero even where its overlap is zero (u =
            // relu(-gamma tau) > 0 for tau < 0).  Keys past T need no mask
            // here: their K rows (zero) multiply U.
            const int lim = qrow - kbase;
            const int wlo = kWin ? lim - W + 1 : 0;
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
                        if ((kCaus && off > lim) || (kWin && off < wlo)) d = 0.f;
                    }
                    if constexpr (decltype(m)::value == kDocm)
                        if ((dmask >> r) & 1u) d = 0.f;
                    w[e] = d;
                }
                pk[j] = E::pack(w[0], w[1]);
            }
        } else {
            if constexpr (decltype(m)::value == kDocm) {
                // Masked past the lane's row (causal), before its window or
                // in another document.
                if (dmw) {
                    const int lim = kCaus ? qrow - kbase : INT_MAX;
                    const int wlo = kWin ? lim - W + 1 : 0;
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
            if constexpr (decltype(m)::value == kMasked) {
                // Key kbase + 8 (r / 4) + r % 4 of register r: masked past
                // the lane's row, and (window) before its first key.
                const int lim = qrow - kbase;
                const int wlo = kWin ? lim - W + 1 : 0;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int off = 8 * (r >> 2) + (r & 3);
                    if ((kCaus && off > lim) || (kWin && off < wlo)) s[r] = 0.f;
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
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const u32x4 bq = {pk[4 * hh], pk[4 * hh + 1], pk[4 * hh + 2], pk[4 * hh + 3]};
                acc[db] = E::mfma(ro.tr(smem, 0, nb, hh, db), bq, acc[db]);
            }
        // Two transposed reads per operand.
        __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 1);
#pragma unroll
        for (int i = 0; i < 2 * DB - LEAD / 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, LEAD / 2, 1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // Pipeline: tile 0 issued before the stationary loads land; at the top of
    // step u, once tile u has landed (each wave waits for its own share) and
    // the barrier has made it visible and freed tile u-1's stage, tile u+1
    // goes out into that stage.
    if constexpr (!DOC) issue(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qr[ks]), "+v"(dr[ks]));
    asm volatile("" : "+v"(zinv), "+v"(nd));
    int u = 0;
    auto step_n = [&](int n) __attribute__((always_inline)) {
        wait_vmcnt<0>();
        __syncthreads();
        if (u + 1 < n) issue(u + 1);
    };
    auto step = [&]() __attribute__((always_inline)) { step_n(ntiles); };
    auto run = [&](int tend, auto m) __attribute__((always_inline)) {
        for (; u < tend; ++u) {
            step();
            const int key0 = (tb + u) * BN;
            half(0, key0 + 4 * g, m);
            half(1, key0 + 32 + 4 * g, m);
            ro.flip();
        }
    };
    if constexpr (DOC) {
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
        // The kept tiles of each chunk of candidates through the ring.  Per
        // tile and wave: nothing to do when the tile lies past the wave's
        // rows (or before their windows) or is one document none of them
        // belongs to; no per-element test when it is before the wave's first
        // row and one document that all of them belong to.
        for (int c0 = 0; c0 < ntiles; c0 += CAP) {
            const int n = screen_doc_tiles<BN>(docb, T, tb * BN, c0, min(CAP, ntiles - c0), bq_lo, bq_hi, t_keep, t_tdoc,
                                               t_list, t_doc, &s_rng[2 * NW]);
            if (n > 0) issue(0);
            for (u = 0; u < n; ++u) {
                step_n(n);
                kdp = kd_lds + (u % NST) * BN;
                const int e = __builtin_amdgcn_readfirstlane(t_list[u]);
                const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
                const int key0 = (tb + (e & ~kDocOne)) * BN;
                const bool one = (e & kDocOne) != 0;
                const bool vis = !(kCaus && key0 > rw + 31) && !(kWin && key0 + BN - 1 < rw - W + 1) &&
                                 !(one && (td < wlo || td > whi));
                dmw = (kCaus && key0 + BN - 1 > rw) || (kWin && key0 < rw + 32 - W) || !(one && wone && td == wlo);
                if (vis) {
                    half(0, key0 + 4 * g, Docm{});
                    half(1, key0 + 32 + 4 * g, Docm{});
                }
                ro.flip();
            }
            if (n & 1) ro.flip();  // the next chunk starts on stage 0
            __syncthreads();       // the list and the ring are reused by the next chunk (or the output)
        }
    } else {
    // (ro follows the stage of tile u: flipped after every tile, idle or not.)
    for (; u < runs.ta; ++u) {
        step();
        ro.flip();
    }
    if constexpr (MODE == kDense) {
        // Nothing to mask (the rows past T contribute zero): one loop.
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
    // bytes per lane and store 2 whole rows per instruction.
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
    const int chunk = ln & 31;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = 32 * wave + 2 * i + (ln >> 5);
        const u32x4 x = *reinterpret_cast<const u32x4*>(smem + row * RB + ((chunk ^ (row & 15)) << 4));
        const int q = R + row;
        if (q < T && (!PAD || chunk < CG))
            __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dQ + (size_t)q * D + chunk * 8));
    }
}

// dK/dV (keys stationary).  Every MFMA here accumulates in AGPRs: a wave's
// dK and dV accumulators for 32 keys fill all 256, so with the S and dPz
// accumulators the compiler keeps two accumulator blocks in VGPRs and moves
// them through the AGPRs around their MFMAs (about 110 register moves per 64
// MFMAs of a 32-query half), with no scratch spills.  Splitting a key block
// into a dV and a dK workgroup (each fits the AGPRs, but S is formed twice:
// five contractions per pair instead of four) measured 15% slower for the
// step (B16 H4 T2048 D256: 529 against 623 TFLOP/s).
template <class E, int MODE, bool PAD = false, bool PUR = false, bool DOC = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void born_bwd16_dkdv_d256_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified gradients: 16-bit");
    static_assert(MODE != kWindowNC || !DOC, "windows without causality: no documents");
    constexpr int DP = 256, NW = BwdD256Cfg::NW, BQ = 64, NST = 2, BK = BwdD256Cfg::BK;
    constexpr int KS = DP / 16, DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BQ * RB;            // bytes per Q or dO tile
    constexpr int NROWS = DOC ? 3 : 2;     // -delta, 1/Z (documents: and the query ids)
    constexpr int RW = NROWS * BQ * 4;     // those rows of a stage
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of Q, dO)
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);
    static_assert(2 * TB == 0x10000 && BK * RB <= 2 * NST * TB, "stages 64 KiB apart / staging");

    // Stage st: Q and dO tiles at 2 TB st; -delta, 1/Z (and the query
    // document ids) at 2 NST TB + RW st.  Afterwards the output staging.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * NST * TB + NST * RW];
    // Documents: the kept-tile list and screening scratch.
    constexpr int CAP = 64 * NW;  // candidate tiles screened per pass (one per thread)
    __shared__ int32_t t_list[DOC ? CAP : 1], t_doc[DOC ? CAP : 1], t_keep[DOC ? CAP : 1], t_tdoc[DOC ? CAP : 1];
    __shared__ int32_t s_rng[DOC ? 2 * NW + 1 : 1];

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

    // Tile u (documents: kept tile u of the list) -> stage u % NST (Q and dO
    // tiles at 2 TB st, the rows at 2 NST TB + RW st).  Row r of the tile's
    // -delta, 1/Z and (documents) query ids comes from wave r (lanes 0-15, 16
    // bytes each).
    auto issue = [&](int u) __attribute__((always_inline)) {
        uint8_t* sb = smem + (u % NST) * 2 * TB;
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
            const uint32_t la = lds_addr(smem + 2 * NST * TB + (u % NST) * RW + wave * BQ * 4);
            if (wave == 0)
                dma_load16(rdl, la, (i0 + 4 * lane) * 4);
            else if (wave == 1)
                dma_load16(rzi, la, (i0 + 4 * lane) * 4);
            else if (DOC && wave == 2)
                dma_load16(rdoc, la, (i0 + 4 * lane) * 4);
        }
    };

    // Operand reads (rows: A of S and dPz; transposed: A of dV^T, dK^T)
    // through the ring's lane offsets (current stage); which = 0 (Q) or 1 (dO).
    RingOffs512 ro(lane);
    constexpr int LEAD = PUR ? 2 : BwdD256Cfg::LEAD;  // purified: more registers in the elementwise pass

    f32x16 acc_v[DB], acc_k[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_v[db] = zero16(), acc_k[db] = zero16();

    constexpr int kFull = 1, kMasked = 2, kDocm = 3;
    using Full = std::integral_constant<int, kFull>;
    using Masked = std::integral_constant<int, kMasked>;
    using Docm = std::integral_constant<int, kDocm>;
    // Query at offset d = query - key masked by causality (d < 0) or the
    // window (d >= W): with both, one unsigned compare; documents under
    // causality take the unsigned form too (|d| < T), which measured fewer
    // spilled registers with padded head dims.
    auto cut = [&](int d) __attribute__((always_inline)) -> bool {
        if constexpr (kCaus && kWin) return (uint32_t)d >= (uint32_t)W;
        if constexpr (kCaus && DOC) return (uint32_t)d >= 0x7fffffffu;
        return (kCaus && d < 0) || (kWin && d >= W);
    };
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
    // Each phase's operand reads run LEAD MFMAs ahead of their use.
    auto half = [&](const uint8_t* rw, int nb, int qbase, auto m) __attribute__((always_inline)) {
        const float* dl = reinterpret_cast<const float*>(rw);
        const float* zl = reinterpret_cast<const float*>(rw + BQ * 4);
        f32x16 s = zero16(), dp;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dl + nb * 32 + 8 * i + 4 * g);
#pragma unroll
            for (int k = 0; k < 4; ++k) dp[4 * i + k] = d4[k];
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s = E::mfma(ro.row(smem, 0, nb, ks), kr[ks], s);
            dp = E::mfma(ro.row(smem, 1, nb, ks), vr[ks], dp);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, LEAD + 4, 0);  // DS read (and the -delta rows)
#pragma unroll
        for (int i = 0; i < 2 * KS - LEAD; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, LEAD, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!PUR && decltype(m)::value == kDocm) {
            // Masked before the lane's key (causal), past its window or in
            // another document.
            if (dmw) {
                const int lim = kCaus ? qbase - key : INT_MAX / 2;
                const int32_t* qd = reinterpret_cast<const int32_t*>(rw + 2 * BQ * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int4 d4 = *reinterpret_cast<const int4*>(qd + nb * 32 + 8 * i + 4 * g);
                    const int dq[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (cut(8 * i + k + lim) || dq[k] != kdoc) s[4 * i + k] = 0.f;
                }
            }
        }
        if constexpr (!PUR && decltype(m)::value == kMasked) {
            // Register r (query qbase + off) is masked before the lane's key
            // (off + lim < 0) and (window) past its window (off + lim >= W).
            const int lim = qbase - key;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                if (cut(off + lim)) s[r] = 0.f;
            }
        }
        uint32_t w2[8], u2[8];
        if constexpr (PUR) {
            // Masked pairs (query before the lane's key, or past its window;
            // documents: in another document) weigh zero; queries past T
            // have 1/Z = 0 from the workspace read.
            const int lim = qbase - key;
            uint32_t dmask = 0;
            if constexpr (decltype(m)::value == kDocm) {
                if (dmw) {
                    const int32_t* qd = reinterpret_cast<const int32_t*>(rw + 2 * BQ * 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int4 d4 = *reinterpret_cast<const int4*>(qd + nb * 32 + 8 * i + 4 * g);
                        const int dq[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (cut(8 * i + k + lim) || dq[k] != kdoc)
                                dmask |= 1u << (4 * i + k);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 z4 = *reinterpret_cast<const f32x4*>(zl + nb * 32 + 8 * i + 4 * g);
#pragma unroll
                for (int k = 0; k < 4; k += 2) {
                    float ww[2], uv[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int r = 4 * i + k + e;
                        const float x = s[r];
                        float uu = __int_as_float(max(__float_as_int(fmaf(x, pg, pgt)), 0));
                        float bb = __int_as_float(max(__float_as_int(x), 0));
                        if constexpr (decltype(m)::value == kMasked) {
                            const int off = 8 * (r >> 2) + (r & 3);
                            if (cut(off + lim)) uu = bb = 0.f;
                        }
                        if constexpr (decltype(m)::value == kDocm)
                            if ((dmask >> r) & 1u) uu = bb = 0.f;
                        const float u2_ = uu * uu;
                        const float dpz = dp[r] * z4[k + e];
                        const float a = u2_ * uu * dpz;
                        dg_acc = fmaf(a, x - ptau, dg_acc);
                        dt_acc += a;
                        ww[e] = fmaf(u2_, u2_, pe * bb * bb) * z4[k + e];
                        uv[e] = fmaf(p4g, u2_ * uu, p2e * bb) * dpz;
                    }
                    w2[(4 * i + k) >> 1] = E::pack(ww[0], ww[1]);
                    u2[(4 * i + k) >> 1] = E::pack(uv[0], uv[1]);
                }
            }
        } else {
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
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const u32x4 bw = {w2[4 * hh], w2[4 * hh + 1], w2[4 * hh + 2], w2[4 * hh + 3]};
            const u32x4 bu = {u2[4 * hh], u2[4 * hh + 1], u2[4 * hh + 2], u2[4 * hh + 3]};
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                acc_v[db] = E::mfma(ro.tr(smem, 1, nb, hh, db), bw, acc_v[db]);
                acc_k[db] = E::mfma(ro.tr(smem, 0, nb, hh, db), bu, acc_k[db]);
            }
        }
        // Two transposed reads per operand.
        __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 1);
#pragma unroll
        for (int i = 0; i < 4 * DB - LEAD / 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, LEAD / 2, 1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // Pipeline as in the dQ kernel (two stages).
    if constexpr (!DOC) issue(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kr[ks]), "+v"(vr[ks]));
    int u = 0;
    auto step_n = [&](int n) __attribute__((always_inline)) {
        wait_vmcnt<0>();
        __syncthreads();
        if (u + 1 < n) issue(u + 1);
    };
    auto step = [&]() __attribute__((always_inline)) { step_n(ntiles); };
    auto run = [&](int tend, auto m) __attribute__((always_inline)) {
        for (; u < tend; ++u) {
            step();
            int roff = (u % NST) * RW;
            asm volatile("" : "+s"(roff));
            const uint8_t* rw = smem + 2 * NST * TB + roff;
            const int i0 = q_lo + u * BQ;
            half(rw, 0, i0 + 4 * g, m);
            half(rw, 1, i0 + 32 + 4 * g, m);
            ro.flip();
        }
    };
    if constexpr (DOC) {
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
        // The kept query tiles of each chunk of candidates through the ring.
        // Per tile and wave: nothing to do when the tile ends before the
        // wave's first key (or starts past its keys' windows) or is one
        // document none of its keys belongs to; no per-element test when it
        // starts after the wave's last key and is one document that all of
        // them belong to.
        for (int c0 = 0; c0 < ntiles; c0 += CAP) {
            const int n = screen_doc_tiles<BQ>(docb, T, q_lo, c0, min(CAP, ntiles - c0), bk_lo, bk_hi, t_keep, t_tdoc,
                                               t_list, t_doc, &s_rng[2 * NW]);
            if (n > 0) issue(0);
            for (u = 0; u < n; ++u) {
                step_n(n);
                int roff = (u % NST) * RW;
                asm volatile("" : "+s"(roff));
                const uint8_t* rw = smem + 2 * NST * TB + roff;
                const int e = __builtin_amdgcn_readfirstlane(t_list[u]);
                const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
                const int i0 = q_lo + (e & ~kDocOne) * BQ;
                const bool one = (e & kDocOne) != 0;
                const bool vis = !(kCaus && i0 + BQ - 1 < kw0) && !(kWin && i0 > kw0 + 31 + W - 1) &&
                                 !(one && (td < klo || td > khi));
                dmw = (kCaus && i0 < kw0 + 31) || (kWin && i0 + BQ - 1 >= kw0 + W) || !(one && kone && td == klo);
                if (vis) {
                    half(rw, 0, i0 + 4 * g, Docm{});
                    half(rw, 1, i0 + 32 + 4 * g, Docm{});
                }
                ro.flip();
            }
            if (n & 1) ro.flip();  // the next chunk starts on stage 0
            __syncthreads();       // the list and the ring are reused by the next chunk (or the output)
        }
    } else {
    // (ro follows the stage of tile u: flipped after every tile, idle or not.)
    for (; u < runs.ta; ++u) {
        step();
        ro.flip();
    }
    if constexpr (MODE == kDense) {
        // Nothing to mask (the rows past T contribute zero): one loop.
        run(ntiles, Full{});
    } else {
        run(runs.tf, Masked{});
        run(runs.tg, Full{});
        run(runs.tv, Masked{});
    }
    for (; u < ntiles; ++u) step();
    }

    // Epilogue: dK = 2 s|s| / c acc, dV = (s / c)^2 acc (c = sq_pre: 1, or
    // 2|s| for fp16, where the factors are s and 1/4), packed and staged in
    // this wave's own 32 rows of the idle ring (row r at smem + RB r, chunks
    // XOR-swizzled by r & 15), then read back 16 bytes per lane and stored 2
    // whole rows per instruction.
    __syncthreads();  // every wave is done with the ring
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
    int ln = lane;
    asm volatile("" : "+v"(ln));
    auto put = [&](const f32x16 (&acc)[DB], float f, void* dst) __attribute__((always_inline)) {
        uint16_t* __restrict__ out = reinterpret_cast<uint16_t*>(dst) + base;
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
        const int chunk = ln & 31;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r2 = 32 * wave + 2 * i + (ln >> 5);
            const u32x4 x = *reinterpret_cast<const u32x4*>(smem + r2 * RB + ((chunk ^ (r2 & 15)) << 4));
            const int kk = K0 + r2;
            if (kk < T && (!PAD || chunk < CG))
                __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(out + (size_t)kk * D + chunk * 8));
        }
    };
    put(acc_k, PUR ? 1.f : E::kScaleInSquare ? sc : 2.f * sc * fabsf(sc), p.dk);
    put(acc_v, PUR ? 1.f : E::kScaleInSquare ? (sc != 0.f ? 0.25f : 0.f) : sc * sc, p.dv);
}

// The purified backward at 128 < D <= 256 (bf16 or fp16): dQ (and the
// workspace), dK/dV (and the dgamma / dtau partials); the caller reduces the
// partials (one per dK/dV workgroup).
template <class E, int MODE, bool PAD, bool DOC = false>
hipError_t launch_purified_bwd_d256(const PurArgs& a, hipStream_t st) {
    using C = BwdD256Cfg;
    const unsigned BH = (unsigned)(a.B * a.H);
    const unsigned nq = (unsigned)((a.T + C::BM - 1) / C::BM);
    const unsigned nk = (unsigned)((a.T + C::BK - 1) / C::BK);
    hipLaunchKernelGGL((born_bwd16_dq_d256_kernel<E, MODE, PAD, true, DOC>), dim3(nq * BH), dim3(C::NW * 64), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((born_bwd16_dkdv_d256_kernel<E, MODE, PAD, true, DOC>), dim3(nk * BH), dim3(C::NW * 64), 0,
                       st, a);
    return hipGetLastError();
}

// The 128 < D <= 256 backward: dQ (and the workspace), dK/dV, then dscale
// from the dQ kernel's per-workgroup sums.
template <class E, int MODE, bool PAD, bool DOC = false>
hipError_t launch_bwd16_d256(const BwdArgs& a, hipStream_t st) {
    using C = BwdD256Cfg;
    const unsigned BH = (unsigned)(a.B * a.H);
    const unsigned nq = (unsigned)((a.T + C::BM - 1) / C::BM);
    const unsigned nk = (unsigned)((a.T + C::BK - 1) / C::BK);
    hipLaunchKernelGGL((born_bwd16_dq_d256_kernel<E, MODE, PAD, false, DOC>), dim3(nq * BH), dim3(C::NW * 64), 0, st,
                       a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((born_bwd16_dkdv_d256_kernel<E, MODE, PAD, false, DOC>), dim3(nk * BH), dim3(C::NW * 64), 0,
                       st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(born_bwd_dscale_groups_kernel<0>, dim3((unsigned)(a.per_head_scale ? a.H : 1)), dim3(256), 0,
                       st, a, (int)(nq * BH));
    return hipGetLastError();
}

}  // namespace qdl
