// Flash-Born forward with document ids, head dim D == 64: the C4 path
// (causal or not; WIN: causal with a sliding window too).
//
// Same arithmetic, row layout and four-phase tile as born_fwd16_fast_kernel
// (born_fwd_fast.h).  What differs is the set of key tiles a query block
// visits, which depends on the document ids:
//   * One 256-row query block per workgroup (two workgroups per CU), or
//     128 rows (four per CU: the Born launch, see NW below), the blocks of
//     the longest key ranges launched first.  Q goes straight from
//     HBM into registers, so LDS holds only the K/V ring (three stages of a
//     K tile, a V tile and the tile's 64 key document ids) and the tile list.
//   * Candidate key tiles (up to the block's last row under causality) are
//     screened 256 at a time, one thread per tile: a tile is kept when the
//     [min, max] range of its key document ids meets the block's query range
//     (exact for sorted ids, i.e. compute_document_ids output; conservative,
//     still correct, for any others).  Wave 0 compacts the kept tiles, with
//     their single document id (or "mixed"), into a list in LDS.
//   * The kept tiles go through the same DMA ring and barrier pipeline as the
//     fast kernel (tiles of step u+2 issued after the barrier that starts
//     step u); each stage also receives the tile's key document ids.
//   * Per wave and column block the tile is unmasked when its keys and the
//     block's 32 rows all belong to one and the same document and it is off
//     the causal diagonal; otherwise every element is tested (key > row under
//     causality, or key document != row document).  Column block 0 is fully
//     masked in diagonal tiles 2 and 3 (computed anyway: a single tile
//     instantiation keeps the register count within two waves per SIMD).
//   * A finished block's rows are staged in the (then idle) ring and written
//     back 16 bytes per lane, 8 whole rows per store instruction.
#pragma once

#include <climits>
#include <type_traits>

#include "born_fwd_fast.h"

namespace qdl {

// PUR: purified-Born weights (flash_born.py:696-811) as in the fast forward:
// p = relu(gamma (r - tau))^4 + eps_base relu(r)^2 in fp32, each weight split
// into two bf16 terms for the P V contraction, Z summed in fp32, the output
// in fp32.  A masked pair (or a key past T) weighs zero even where its
// overlap is zero, so the masks zero the weights, not the overlaps.
// WIN: a causal sliding window with the documents (flash_born.py:173-174):
// candidate tiles start at the block's first row's window, tiles that start
// before the block's last row's window are tested per element, and the test
// also drops keys before the row's window.
//
// NW: waves per workgroup, 4 (256-row blocks, two workgroups per CU, a ring
// of three stages) or 2 (128-row blocks, four workgroups per CU, a ring of
// two stages: 40 KiB of LDS each).  Every wave holds two 32-row column blocks
// either way; 128-row blocks straddle fewer document edges and cut the
// causal diagonal finer (C4's documents: 1.28x the visible pairs executed
// against 1.53x for 256-row blocks).
//
// PRO: the Q prologue folded into the Q load (bf16 Born): q holds the raw
// query rows (element strides q_sb, q_sh, q_st), each lane rotates and
// normalises its rows' operands in registers as the standalone prologue
// kernel would (born_qk_fold.h), and, when a backward follows (q_rinv set),
// writes the normalised rows and their 1/norm.
template <class E, int DP, bool PUR = false, bool WIN = false, int NW = 4, bool PRO = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void born_fwd16_doc_kernel(
    typename std::conditional<PUR, PurArgs, typename std::conditional<PRO, FwdProArgs, FwdArgs>::type>::type p) {
    static_assert(DP == 64, "tuned for D = 64");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified: 16-bit inputs");
    static_assert(!PRO || (std::is_same<E, BF16>::value && !PUR), "the fused prologue is bf16 Born only");
    static_assert(NW == 4 || NW == 2, "256- or 128-row blocks");
    constexpr int NQB = 2, BN = 64, NST = NW == 4 ? 3 : 2, BM = 64 * NW;
    constexpr int KS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    constexpr int CAP = 64 * NW;           // candidate tiles screened per pass (one per thread)
    constexpr int KDW = BN / NW;           // key document ids loaded per wave per tile
    // Loads per wave per tile: K, V and a slice of the key document ids.
    constexpr int kTileLoads = 2 * LPW + 1;
    static_assert(TB % (1024 * NW) == 0 && BN == 64 && KDW % 4 == 0, "tile split");

    // One buffer: the K/V ring during the tile loop, the output staging
    // (BM rows x 128 bytes) once the loop is done.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * NST * TB];
    __shared__ __attribute__((aligned(16))) int32_t kd_lds[NST * BN];  // key document ids per stage
    __shared__ int32_t t_list[CAP];                                   // kept tiles, ascending
    __shared__ int32_t t_doc[CAP];                                    // their document id or INT_MIN
    __shared__ int32_t t_keep[CAP];
    __shared__ int32_t t_tdoc[CAP];
    __shared__ int32_t s_qrng[2 * NW];
    __shared__ int32_t s_count;
    uint8_t* const k_lds = smem;
    uint8_t* const v_lds = smem + NST * TB;

    const int T = p.T;
    const int BH = p.B * p.H;
    const int nmb = (T + BM - 1) / BM;
    const bool causal = WIN || p.is_causal != 0;
    const int W = WIN ? p.window : 0;
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    const int mb = causal ? (nmb - 1 - bid / BH) : (bid / BH);
    const int b = bh / p.H, h = bh % p.H;
    const int R = mb * BM;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, g = lane >> 5;

    const size_t base = (size_t)bh * T * DP;
    const uint16_t* __restrict__ Qg = reinterpret_cast<const uint16_t*>(p.q) + base;
    const int32_t* __restrict__ docb = p.doc + (size_t)b * T;
    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (!PUR && sc < 0.f) ? 0x80008000u : 0u;  // sign of the scale folded into Q
    // fp16: the reference's weights relu(s r)^2 (born_weight_pair).
    const float sq_pre = E::kScaleInSquare ? fabsf(sc) : 1.f;
    // Purified weights: t = gamma r - gamma tau, b' = sqrt(eps_base) relu(r).
    float pg = 0.f, pgt = 0.f, pse = 0.f;
    if constexpr (PUR) {
        pg = sc;
        pgt = -sc * p.tau[p.per_head_tau ? h : 0];
        pse = sqrtf(p.eps_base);
    }

    const uint32_t nrec = (uint32_t)T * (uint32_t)RB;
    const i32x4 rk = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.k) + base, nrec);
    const i32x4 rv = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.v) + base, nrec);
    const i32x4 rd = buffer_rsrc(docb, (uint32_t)T * 4u);

    // Rows: column c of block qb -> row R + (BM/2) qb + (BM/4) (c / 16) +
    // 16 wave + c % 16: every wave has 16-row pieces of each quarter.
    const int lrow = (BM / 4) * (c >> 4) + 16 * wave + (c & 15);
    int qrow[NQB], qdoc[NQB];
    u32x4 qr[NQB][KS];
    if constexpr (PRO) {
        // Raw rows, the table entries of every row of the lane first (one
        // memory round trip), then q' in registers.
        const uint16_t* Qraw = reinterpret_cast<const uint16_t*>(p.q) + (size_t)b * p.q_sb + (size_t)h * p.q_sh;
        const bool rot = p.cos != nullptr;
        const bool vec = rot && ((reinterpret_cast<uintptr_t>(p.cos) | reinterpret_cast<uintptr_t>(p.sin)) & 15) == 0 &&
                         (p.ld & 3) == 0 && p.nfreq >= DP / 2;
        RotRow rt[NQB][2];
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            qrow[qb] = R + (BM / 2) * qb + lrow;
            const bool ok = qrow[qb] < T;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 x = {0u, 0u, 0u, 0u};
                if (ok) x = ldg16(Qraw + (size_t)qrow[qb] * p.q_st + (2 * ks + g) * 8);
                qr[qb][ks] = x;
            }
            if (rot) {
                rot_load(p.cos, p.sin, p.ld, p.nfreq, T, qrow[qb], 8 * g, vec, rt[qb][0]);
                rot_load(p.cos, p.sin, p.ld, p.nfreq, T, qrow[qb], 8 * (2 + g), vec, rt[qb][1]);
            }
            qdoc[qb] = ok ? docb[qrow[qb]] : INT_MIN;
        }
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const float rinv = rot_normalise_row(qr[qb], rt[qb][0], rt[qb][1], rot, p.norm_eps);
            // The normalised rows and their 1/norm, for the backward (not
            // written when no backward follows: q_rinv null).
            if (qrow[qb] < T && p.q_rinv != nullptr) {
                uint16_t* qo = reinterpret_cast<uint16_t*>(p.q_out) + base + (size_t)qrow[qb] * DP;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    __builtin_nontemporal_store(qr[qb][ks], reinterpret_cast<u32x4*>(qo + 8 * (2 * ks + g)));
                if (g == 0) __builtin_nontemporal_store(rinv, p.q_rinv + (size_t)bh * T + qrow[qb]);
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) qr[qb][ks] ^= flip;
        }
    } else {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            qrow[qb] = R + (BM / 2) * qb + lrow;
            const bool ok = qrow[qb] < T;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 x = {0u, 0u, 0u, 0u};
                if (ok) x = ldg16(Qg + (size_t)qrow[qb] * DP + (2 * ks + g) * 8);
                qr[qb][ks] = x ^ flip;
            }
            qdoc[qb] = ok ? docb[qrow[qb]] : INT_MIN;
        }
    }

    const int kv_hi = causal ? min(T, R + BM) : T;
    // Window: candidates from the tile of the block's first row's first key.
    const int tb = WIN ? max(0, R - W + 1) / BN : 0;
    const int ncand = (kv_hi + BN - 1) / BN - tb;
    const int t0 = causal ? R / BN : INT_MAX;  // first diagonal tile
    // Window: tiles starting before this key are cut by some row's window.
    const int kwin = WIN ? R + BM - W : 0;

    // Document-id range of candidate tile `tid` of the first screening chunk,
    // loaded here so its latency overlaps the Q loads'.  All loads of a
    // thread are independent (one memory latency).
    const bool doc_vec = (reinterpret_cast<uintptr_t>(docb) & 15) == 0;
    auto tile_range = [&](int tile, int& lo, int& hi) __attribute__((always_inline)) {
        const int key0 = tile * BN;
        const int kend = min(key0 + BN, T);
        lo = INT_MAX;
        hi = INT_MIN;
        if (doc_vec && kend - key0 == BN) {
#pragma unroll 8
            for (int j = 0; j < BN / 4; ++j) {
                const int4 x = *reinterpret_cast<const int4*>(docb + key0 + 4 * j);
                lo = min(lo, min(min(x.x, x.y), min(x.z, x.w)));
                hi = max(hi, max(max(x.x, x.y), max(x.z, x.w)));
            }
        } else {
            for (int key = key0; key < kend; ++key) {
                const int d = docb[key];
                lo = min(lo, d);
                hi = max(hi, d);
            }
        }
    };
    int tlo0 = INT_MAX, thi0 = INT_MIN;
    if (tid < min(CAP, ncand)) tile_range(tb + tid, tlo0, thi0);

    // Document range of each column block's valid rows (uniform per wave):
    // qsd[qb] is the one document of all 32 rows, or INT_MIN + 1 when they
    // span several (never equal to a tile's document id, or to "mixed").
    int qsd[NQB];
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
        qsd[qb] = (lo == hi) ? lo : INT_MIN + 1;
        wlo = min(wlo, lo);
        whi = max(whi, hi);
    }
    if (lane == 0) {
        s_qrng[2 * wave] = wlo;
        s_qrng[2 * wave + 1] = whi;
    }
    __syncthreads();
    int bq_lo = INT_MAX, bq_hi = INT_MIN;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        bq_lo = min(bq_lo, s_qrng[2 * w]);
        bq_hi = max(bq_hi, s_qrng[2 * w + 1]);
    }

    // Screen candidate tiles c0 .. c0+nc-1 into t_list / t_doc; returns the
    // number kept (the first chunk's ranges were loaded up front).
    auto screen = [&](int c0, int nc) -> int {
        if (tid < nc) {
            int lo = tlo0, hi = thi0;
            if (c0 > 0) tile_range(tb + c0 + tid, lo, hi);
            t_keep[tid] = (hi >= bq_lo && lo <= bq_hi) ? 1 : 0;
            t_tdoc[tid] = (lo == hi) ? lo : INT_MIN;
        }
        __syncthreads();
        if (wave == 0) {
            int count = 0;
            for (int base0 = 0; base0 < nc; base0 += 64) {
                const int i = base0 + lane;
                const bool keep = i < nc && t_keep[i] != 0;
                const uint64_t m = __ballot(keep);
                const int pos = count + (int)__builtin_amdgcn_mbcnt_hi(
                                            (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                if (keep) {
                    t_list[pos] = c0 + i;
                    t_doc[pos] = t_tdoc[i];
                }
                count += __popcll(m);
            }
            if (lane == 0) s_count = count;
        }
        __syncthreads();
        return __builtin_amdgcn_readfirstlane(s_count);
    };

    // Kept tile u -> stage u % NST: K, V (wave-instruction i writes LDS slots
    // (wave * LPW + i) * 64 + lane, slot = row * CPR + chunk') and this
    // wave's 16 key document ids (lanes 0-3, 16 bytes each).
    auto issue = [&](int u) __attribute__((always_inline)) {
        const int st = u % NST;
        const int key0 = (tb + __builtin_amdgcn_readfirstlane(t_list[u])) * BN;
        uint8_t* kb = k_lds + st * TB;
        uint8_t* vb = v_lds + st * TB;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int slot = (wave * LPW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int off = (key0 + row) * RB;
            dma_load16(rk, lds_addr(kb + (wave * LPW + i) * 1024), off + ((pc ^ (row & 7)) << 4));
            dma_load16(rv, lds_addr(vb + (wave * LPW + i) * 1024), off + ((pc ^ ((row & 3) << 1)) << 4));
        }
        if (lane < KDW / 4) dma_load16(rd, lds_addr(kd_lds + st * BN + wave * KDW), (key0 + wave * KDW + lane * 4) * 4);
    };

    f32x16 oacc[DB][NQB];
    float zacc[NQB][2];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) oacc[db][qb] = zero16();
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) zacc[qb][0] = zacc[qb][1] = 0.f;

    const int vrow_l = 4 * g + ((lane & 15) >> 2);
    const int vcol_l = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    auto k_operand = [&](const uint8_t* kb, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + c;
        const int pc = (2 * ks + g) ^ (row & 7);
        return *reinterpret_cast<const u32x4*>(kb + row * RB + pc * 16);
    };
    auto v_operand = [&](const uint8_t* vb, int nb, int hh, int db) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + hh * 16 + vrow_l;
        const int col = db * 32 + vcol_l;
        const int pc = (col >> 3) ^ ((row & 3) << 1);
        const uint8_t* b0 = vb + row * RB + pc * 16 + (col & 7) * 2;
        const uint8_t* b1 = vb + (row + 8) * RB + pc * 16 + (col & 7) * 2;
        const u32x2 x = lds_read_tr16(reinterpret_cast<const uint16_t*>(b0));
        const u32x2 y = lds_read_tr16(reinterpret_cast<const uint16_t*>(b1));
        const u32x4 a = {x[0], x[1], y[0], y[1]};
        return a;
    };

    // Elementwise pass over one 32-key half of S^T: p' = relu(x|x|) packed,
    // z += p'.
    auto elementwise = [&](f32x16 (&s)[NQB], uint32_t (&pk)[NQB][8]) __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                pk[qb][j] = born_weight_pair<E>(s[qb][2 * j], s[qb][2 * j + 1], sq_pre, zacc[qb][j & 1]);
            }
        }
    };
    // Zero the masked elements of column block qb in one 32-key half: key
    // key0h + 4 g + 8 i + k (register 4 i + k) is masked when it lies past
    // the lane's row (causal) or belongs to another document (kd: this
    // stage's key document ids).
    // A tile of a single document (single, uniform) needs no id compare: the
    // lane's row sees its keys iff it is in that document (vis), folded into
    // the causal limit.
    auto apply_mask = [&](f32x16& s, int qb, int key0h, const int32_t* kd, bool single, bool vis)
        __attribute__((always_inline)) {
        // Last visible key offset (causal; WIN: the window's first is W - 1
        // before it, both tested as one unsigned compare).
        int lim = causal ? qrow[qb] - (key0h + 4 * g) : INT_MAX;
        if (single) {
            if (!vis) lim = -1;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                if (WIN ? pair_cut<true, true>(lim - off, W) : off > lim) s[r] = 0.f;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int4 d4 = *reinterpret_cast<const int4*>(kd + 4 * g + 8 * i);
                const int dk[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if ((WIN ? pair_cut<true, true>(lim - (8 * i + k), W) : 8 * i + k > lim) || dk[k] != qdoc[qb]) s[4 * i + k] = 0.f;
            }
        }
    };

    // Zero the column of every lane whose row is outside the tile's single
    // document (the tile is off the causal diagonal).
    auto apply_lane = [&](f32x16& s, bool vis) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = vis ? s[r] : 0.f;
    };

    u32x4 kop[KS];
    auto read_k = [&](u32x4 (&dst)[KS], const uint8_t* kb, int nb) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) dst[ks] = k_operand(kb, nb, ks);
    };
    auto read_v = [&](u32x4 (&dst)[2][DB], const uint8_t* vb, int nb) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db) dst[hh][db] = v_operand(vb, nb, hh, db);
    };
    auto qk_op = [&](const u32x4 (&ops)[KS], f32x16 (&s)[NQB]) __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) s[qb] = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) s[qb] = E::mfma(ops[ks], qr[qb][ks], s[qb]);
    };
    constexpr int PW = PUR ? 8 : 1;  // packed low parts of the purified weights
    auto pv_op = [&](const u32x4 (&ops)[2][DB], const uint32_t (&pk)[NQB][8], const uint32_t (&pl)[NQB][PW])
        __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    const u32x4 bq = {pk[qb][4 * hh], pk[qb][4 * hh + 1], pk[qb][4 * hh + 2], pk[qb][4 * hh + 3]};
                    if constexpr (PUR) {
                        const u32x4 bl = {pl[qb][4 * hh % PW], pl[qb][(4 * hh + 1) % PW], pl[qb][(4 * hh + 2) % PW],
                                          pl[qb][(4 * hh + 3) % PW]};
                        oacc[db][qb] = pur_pv<E>(ops[hh][db], bq, bl, oacc[db][qb]);
                    } else {
                        oacc[db][qb] = E::mfma(ops[hh][db], bq, oacc[db][qb]);
                    }
                }
    };
    // Purified weights of one 32-key half (keys key0h + 4 g + 8 (r / 4) +
    // r % 4), the masked ones zeroed: per element where the column block is
    // tested (mm: causal bound, or T - 1 without causality, and the key id;
    // a tile of one document tests only the bound, all of it when the lane's
    // row is in another document), per lane (ll: rows outside the tile's one
    // document), or not at all.  Z in fp32, each weight split hi + lo.
    auto elementwise_pur = [&](f32x16 (&s)[NQB], uint32_t (&pk)[NQB][8], uint32_t (&pl)[NQB][PW], int key0h,
                               const int32_t* kd, bool mm0, bool mm1, bool ll0, bool ll1, bool vv0, bool vv1,
                               bool single) __attribute__((always_inline)) {
        const bool mm[NQB] = {mm0, mm1}, ll[NQB] = {ll0, ll1}, vv[NQB] = {vv0, vv1};
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            int lim = (causal ? qrow[qb] : T - 1) - (key0h + 4 * g);
            if (single && !vv[qb]) lim = -1;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float w[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int r = 2 * j + e;
                    const int off = 8 * (r >> 2) + (r & 3);
                    const float x = s[qb][r];
                    const float t = fmaf(x, pg, pgt);
                    const float u = __int_as_float(max(__float_as_int(t), 0));
                    const float bq = __int_as_float(max(__float_as_int(x * pse), 0));
                    const float u2 = u * u;
                    float pw = fmaf(u2, u2, bq * bq);
                    bool masked = false;
                    if (mm[qb]) {
                        masked = WIN ? pair_cut<true, true>(lim - off, W) : off > lim;
                        if (!single) masked = masked || kd[4 * g + off] != qdoc[qb];
                    } else if (ll[qb]) {
                        masked = !vv[qb];
                    }
                    w[e] = masked ? 0.f : pw;
                }
                zacc[qb][0] += w[0] + w[1];
                const uint32_t hi = BF16::pack(w[0], w[1]);
                pk[qb][j] = hi;
                pl[qb][j % PW] = BF16::pack(w[0] - BF16::lo(hi), w[1] - BF16::hi(hi));
            }
        }
    };
    // The fast kernel's four phases (see born_fwd_fast.h), MFMA-only phases at
    // raised wave priority.  One instantiation for every tile (a second one in
    // the loop costs more registers than the wave has): the masks are applied
    // between phases under uniform flags (m0, m1: column block 0 / 1 masked).
    auto tile = [&](const uint8_t* kb, const uint8_t* vb, const int32_t* kd, int key0, bool m0, bool m1, bool l0,
                    bool l1, bool v0, bool v1, bool single) __attribute__((always_inline)) {
        f32x16 s0[NQB], s1[NQB];
        uint32_t pk0[NQB][8], pk1[NQB][8];
        u32x4 kop1[KS], vop0[2][DB], vop1[2][DB];
        if constexpr (PUR) {
            // Purified: masks applied to the weights; PV issues twice the
            // MFMAs (hi and lo parts); V of keys 32-63 is read at the start
            // of the last phase (keeps the tile within the register budget).
            uint32_t pl0[NQB][PW], pl1[NQB][PW];
            __builtin_amdgcn_s_setprio(1);
            read_k(kop1, kb, 1);
            qk_op(kop, s0);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
            read_v(vop0, vb, 0);
            qk_op(kop1, s1);
            elementwise_pur(s0, pk0, pl0, key0, kd, m0, m1, l0, l1, v0, v1, single);
#pragma unroll
            for (int i = 0; i < KS * NQB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 40, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            pv_op(vop0, pk0, pl0);
            elementwise_pur(s1, pk1, pl1, key0 + 32, kd + 32, m0, m1, l0, l1, v0, v1, single);
#pragma unroll
            for (int i = 0; i < (std::is_same<E, F16>::value ? 6 : 4) * DB * NQB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                __builtin_amdgcn_sched_group_barrier(0x002, 20, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            read_v(vop1, vb, 1);
            pv_op(vop1, pk1, pl1);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
            return;
        }
        const uint32_t plx[NQB][PW] = {};  // (Born: no low parts)
        __builtin_amdgcn_s_setprio(1);
        read_k(kop1, kb, 1);
        qk_op(kop, s0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        if (m0) apply_mask(s0[0], 0, key0, kd, single, v0);
        else if (l0) apply_lane(s0[0], v0);
        if (m1) apply_mask(s0[1], 1, key0, kd, single, v1);
        else if (l1) apply_lane(s0[1], v1);
        __builtin_amdgcn_sched_barrier(0);
        read_v(vop0, vb, 0);
        qk_op(kop1, s1);
        elementwise(s0, pk0);
#pragma unroll
        for (int i = 0; i < KS * NQB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (m0) apply_mask(s1[0], 0, key0 + 32, kd + 32, single, v0);
        else if (l0) apply_lane(s1[0], v0);
        if (m1) apply_mask(s1[1], 1, key0 + 32, kd + 32, single, v1);
        else if (l1) apply_lane(s1[1], v1);
        __builtin_amdgcn_sched_barrier(0);
        read_v(vop1, vb, 1);
        pv_op(vop0, pk0, plx);
        elementwise(s1, pk1);
#pragma unroll
        for (int i = 0; i < 2 * DB * NQB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x002, 10, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        pv_op(vop1, pk1, plx);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };

    // Pipeline over the kept tiles of each screened chunk: tiles 0 .. NST-2
    // issued up front, tile u+NST-1 right after the barrier that starts step
    // u (the stage of tile u-1, which every wave has left by then); at that
    // barrier each wave has waited for its share of tile u (loads return in
    // order: only the later tiles' may still be in flight).
    for (int c0 = 0; c0 < ncand; c0 += CAP) {
        const int n = screen(c0, min(CAP, ncand - c0));
        if (n > 0) issue(0);
        if (NST == 3 && n > 1) issue(1);
        for (int u = 0; u < n; ++u) {
            if (NST == 3 && u + 1 < n)
                wait_vmcnt<kTileLoads>();
            else
                wait_vmcnt<0>();
            __syncthreads();
            if (u + NST - 1 < n) issue(u + NST - 1);
            // Stage offset opaque to the optimiser (addresses formed per tile).
            int soff = (u % NST) * TB;
            asm volatile("" : "+s"(soff));
            const uint8_t* kb = k_lds + soff;
            const uint8_t* vb = v_lds + soff;
            const int32_t* kd = kd_lds + (soff / TB) * BN;
            const int ti = tb + __builtin_amdgcn_readfirstlane(t_list[u]);
            const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
            read_k(kop, kb, 0);
            // A column block needs the element test on the causal diagonal
            // (256-row blocks: tiles t0 .. t0+3, block 0 in all four, block 1
            // in the last two; 128-row blocks: t0, t0+1 and t0+1)
            // and where the tile's keys span several documents.  Off the
            // diagonal, keys of one document are visible to the rows of that
            // document and to no other: unless all 32 rows are in it, a
            // per-lane select clears the other rows' columns.
            const int rel = ti - t0;  // t0 is INT_MAX without causality
            const bool mixed = td == INT_MIN;
            // Purified: a tile holding keys past T is tested per element (the
            // zero rows of those keys still weigh relu(-gamma tau)).
            const bool tail = PUR && (ti + 1) * BN > T;
            // Window: both blocks tested where a row's window starts.
            const bool cut = WIN && ti * BN < kwin;
            const bool m0 = rel >= 0 || mixed || tail || cut;
            const bool m1 = rel >= BM / 128 || mixed || tail || cut;
            tile(kb, vb, kd, ti * BN, m0, m1, td != qsd[0], td != qsd[1], qdoc[0] == td, qdoc[1] == td, !mixed);
        }
        __syncthreads();  // the list and the ring are reused by the next chunk
    }

    float* __restrict__ Zp = p.z + (size_t)bh * T;
    if constexpr (PUR) {
        // Purified: O = acc / (Z + eps) in fp32, stored from the accumulators.
        float* __restrict__ O32 = p.o + base;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const float zl = zacc[qb][0] + zacc[qb][1];
            const float zd = zl + __shfl_xor(zl, 32) + p.eps;
            const int qi = R + (BM / 2) * qb + lrow;
            if (qi < T) {
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x16& o = oacc[db][qb];
                        const f32x4 w = {o[4 * j] / zd, o[4 * j + 1] / zd, o[4 * j + 2] / zd, o[4 * j + 3] / zd};
                        // plain store: L2 merges each row's 32-byte pieces into whole lines
                        *reinterpret_cast<f32x4*>(O32 + (size_t)qi * DP + db * 32 + 8 * j + 4 * g) = w;
                    }
                if (g == 0) __builtin_nontemporal_store(zd, Zp + qi);
            }
        }
        return;
    }
    // Epilogue: normalise, stage this wave's rows in the idle ring (row r at
    // smem + 128 r, chunks XOR-swizzled by r & 7), read them back 16 bytes
    // per lane and store 8 whole rows per instruction (non-temporal).
    uint16_t* __restrict__ O = reinterpret_cast<uint16_t*>(p.o) + base;
    const float s2 = (sq_pre > 0.f) ? (sc / sq_pre) * (sc / sq_pre) : 0.f;
    const float eps_s = (p.eps == 0.f) ? 0.f : p.eps / s2;
    // (The lane index goes through an empty asm so these addresses are formed
    // here rather than hoisted and kept live across the tile loop.)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int lr = (BM / 4) * ((ln & 31) >> 4) + 16 * wave + (ln & 15);
    const int gg = ln >> 5;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const float zl = zacc[qb][0] + zacc[qb][1];
        const float zt = zl + __shfl_xor(zl, 32);
        const float rcp = 1.0f / (zt + eps_s);
        const int row = (BM / 2) * qb + lr;
        uint8_t* rb = smem + row * RB;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x16& o = oacc[db][qb];
                u32x2 w;
                w[0] = E::pack(o[4 * j] * rcp, o[4 * j + 1] * rcp);
                w[1] = E::pack(o[4 * j + 2] * rcp, o[4 * j + 3] * rcp);
                const int chunk = 4 * db + j;
                *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 7)) << 4) + 8 * gg) = w;
            }
        if (gg == 0 && R + row < T) __builtin_nontemporal_store(s2 * zt + p.eps, Zp + R + row);
    }
    const int chunk = ln & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = (BM / 4) * (i >> 1) + 16 * wave + 8 * (i & 1) + (ln >> 3);
        const u32x4 x = *reinterpret_cast<const u32x4*>(smem + row * RB + ((chunk ^ (row & 7)) << 4));
        const int qi = R + row;
        if (qi < T) __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(O + (size_t)qi * DP + chunk * 8));
    }
}

// Born with documents: 128-row blocks (the document ids live on the device,
// so the host cannot look at their lengths).  Against 256-row blocks, on
// B4 H16 T8192 bf16 (one box, best of 5 x 50 launches): geometric documents
// of mean 128 / 512 / 2048 tokens 103.7 -> 83.7, 150.9 -> 142.9, 312.4 ->
// 313.1 us; one document per row 519.5 -> 548.2 us.
template <class E, int DP, bool WIN = false>
hipError_t launch_fwd16_doc(const FwdArgs& a, hipStream_t st) {
    constexpr int NW = 2, BM = 64 * NW;
    const dim3 grid((unsigned)((a.T + BM - 1) / BM) * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd16_doc_kernel<E, DP, false, WIN, NW>), grid, dim3(64 * NW), 0, st, a);
    return hipGetLastError();
}

// Born forward with document ids and the Q prologue folded into the Q load
// (bf16, D = 64; WIN: with a causal sliding window); the keys arrive
// normalised.  Same grid as launch_fwd16_doc.
template <bool WIN = false>
hipError_t launch_fwd16_doc_prologue(const FwdProArgs& a, hipStream_t st) {
    constexpr int NW = 2, BM = 64 * NW;
    const dim3 grid((unsigned)((a.T + BM - 1) / BM) * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd16_doc_kernel<BF16, 64, false, WIN, NW, true>), grid, dim3(64 * NW), 0, st, a);
    return hipGetLastError();
}

// Purified-Born forward with document ids (bf16, D = 64; WIN: with a causal
// sliding window), 128-row blocks as the Born launch (p4b 220 -> 227,
// pwc4b 155 -> 166 TFLOP/s for the step on one box, 4 VGPRs spilled).
template <bool WIN = false, class E = BF16>
hipError_t launch_purified_fwd_doc(const PurArgs& a, hipStream_t st) {
    constexpr int NW = 2, BM = 64 * NW;
    const dim3 grid((unsigned)((a.T + BM - 1) / BM) * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd16_doc_kernel<E, 64, true, WIN, NW>), grid, dim3(64 * NW), 0, st, a);
    return hipGetLastError();
}

}  // namespace qdl
