// Flash-Born forward specialised for head dim D == 128 (no padding): dense,
// causal, or causal with a sliding window.
//
// Same arithmetic and load pipeline as the D == 64 kernel (born_fwd_fast.h):
// LDS-DMA K/V ring of three 64-key stages, one barrier per tile, two 256-row
// query blocks per workgroup under causality (mb and nmb-1-mb), Q block and
// output rows staged through LDS.  What changes with the wider rows:
//   * Registers: a wave holds one 32-row MFMA column block (its Q operands
//     are 32 VGPRs and its O accumulators 64 at D == 128; two column blocks
//     would not fit two waves per SIMD).  The workgroup is 8 waves (two per
//     SIMD) over a 256-row block, wave w owning rows 32w .. 32w+31, so every
//     K/V tile in LDS feeds 256 query rows.
//   * LDS: 3 x (16 + 16) KiB ring + 64 KiB Q block = 160 KiB, one workgroup
//     per CU.  Rows are 256 bytes, so every row starts on bank 0 and the
//     16-byte chunks are XOR-swizzled per row:
//       K, Q: chunk' = chunk ^ (row & 15)       -> 16 consecutive rows of one
//             chunk (a ds_read_b128 quarter-wave) hit 16 distinct chunks;
//       V:    chunk' = chunk ^ 4 (row & 3)      -> the 4 rows x 64 bytes of a
//             ds_read_b64_tr_b16 half-wave hit 4 distinct 64-byte groups.
//   * Masks per wave: with contiguous rows, each wave's tiles split into
//     runs that are fully visible to all of its rows (no mask), cut by its
//     diagonal or its window edge (both bounds tested per element), or
//     invisible to it (no work; it only joins the barrier).  Under causality
//     the four diagonal tiles of a block then cost the busier SIMD 2, 2, 1
//     and 1 wave-tiles instead of 2 each.
// Per tile the wave runs the D == 64 kernel's four fenced phases: QK(keys
// 0-31); QK(keys 32-63) | elementwise(0-31); PV(0-31) | elementwise(32-63);
// PV(32-63), each phase's LDS operands read one phase ahead.
//
// PUR: the purified-Born weights (flash_born.py:696-811) as in the D == 64
// fast forward: p = relu(gamma (r - tau))^4 + eps_base relu(r)^2 in fp32,
// each weight split into bf16 hi + lo terms for the P V contraction (two
// MFMAs), Z summed in fp32, O and Z stored in fp32 straight from the
// accumulators.  Masks zero the weights (a zero overlap still weighs
// relu(-gamma tau)^4 when tau < 0), so without causality the keys past T
// are masked in the last tile too.
//
// PAD: a head dim D < 128 (a multiple of 8) on the same kernel.  The rows in
// HBM are 2 D bytes; the loads of the 16-byte chunks past D are sent out of
// the buffer's range, so they land in LDS as zeros, and the output chunks
// past D are not stored.  The arithmetic is that of D == 128 with zero
// columns (which add nothing to any overlap).
//
// DOC: document ids (no window; flash_born.py:145-147, 175-177; also with
// PAD), one 256-row block per workgroup.  The block's candidate key tiles are screened by
// document-id range into a list in LDS (as the D == 64 document kernels do)
// and only the kept tiles go through the ring, each with its 64 key ids.  Per
// tile a wave skips the work when the tile lies past its rows or is one
// document none of its rows belongs to, and tests the tile per element
// (document and causal) unless the tile is before its first row and one
// document all of its rows belong to.  Q goes straight from HBM into
// registers, and the output rows are staged in the idle ring, so the 64 KiB
// Q block is not needed.
#pragma once

#include <type_traits>

#include "born_bwd_fast.h"
#include "born_common.h"
#include "born_fwd_fast.h"
#include "purified_args.h"

namespace qdl {

struct FwdD128Cfg {
    static constexpr int DP = 128;
    static constexpr int NW = 8;    // waves per workgroup, two per SIMD
    static constexpr int BM = 256;  // query rows per block, 32 per wave
    static constexpr int BN = 64;   // keys per tile
    static constexpr int NST = 3;   // K/V ring stages
};

// NW (documents only): 4 waves over 128-row blocks, two workgroups per CU
// and a two-stage ring (fewer blocks straddle a document edge, and two
// workgroups per CU overlap one's start-up with the other's tiles);
// otherwise 8 waves over 256-row blocks.
template <class E, int MODE, bool PUR = false, bool PAD = false, bool DOC = false, int NW = 8>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void born_fwd16_d128_kernel(typename std::conditional<PUR, PurArgs, FwdArgs>::type p) {
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    static_assert(MODE != kWindowNC || !DOC, "windows without causality: no documents");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified: 16-bit inputs");
    static_assert(NW == 8 || (NW == 4 && DOC), "128-row blocks: the document mode");
    using C = FwdD128Cfg;
    constexpr int DP = C::DP, BM = 32 * NW, BN = C::BN, NST = NW == 8 ? C::NST : 2;
    constexpr int KDW = BN / NW;  // documents: key ids loaded per wave per tile
    constexpr int KS = DP / 16;            // 16-wide contraction steps of QK
    constexpr int DB = DP / 32;            // 32-column blocks of O
    constexpr int RB = DP * 2;             // bytes per row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int QB = BM * RB;            // bytes per Q block
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    constexpr int LQW = QB / (1024 * NW);  // 1-KiB loads per wave per Q block
    static_assert(TB % (1024 * NW) == 0 && QB % (1024 * NW) == 0, "tile split");
    static_assert(LQW * 1024 == 32 * RB, "each wave's Q loads land on its own 32 rows");
    // kWindow: causal with a window; kWindowNC: a window without causality
    // (row i sees keys i - W + 1 .. T - 1).
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);

    __shared__ __attribute__((aligned(1024))) uint8_t k_lds[NST * TB];
    __shared__ __attribute__((aligned(1024))) uint8_t v_lds[NST * TB];
    __shared__ __attribute__((aligned(1024))) uint8_t q_lds[DOC ? 16 : QB];
    // Documents: key document ids per stage, the kept-tile list and screening scratch.
    constexpr int CAP = 256;  // candidate tiles screened per pass
    __shared__ __attribute__((aligned(16))) int32_t kd_lds[DOC ? NST * BN : 1];
    __shared__ int32_t t_list[DOC ? CAP : 1], t_doc[DOC ? CAP : 1], t_keep[DOC ? CAP : 1], t_tdoc[DOC ? CAP : 1];
    __shared__ int32_t s_rng[DOC ? 2 * NW + 1 : 1];

    const int T = p.T;
    const int BH = p.B * p.H;
    const int nmb = fast_fwd_nmb(T, BM);
    const int bid = blockIdx.x;
    // Paired launch: item 0 is query block nmb-1-pr, item 1 block pr when
    // that is a different block.  Unpaired: one block per workgroup, the
    // longest key ranges first (kWindowNC: the first blocks).
    const bool paired = gridDim.x < (unsigned)(nmb * BH);
    const int bh = bid % BH;
    const int pr = bid / BH;
    const int h = bh % p.H;
    const int mb_a = (MODE == kWindowNC && !paired) ? pr : nmb - 1 - pr, mb_b = paired ? pr : mb_a;
    const int nitems = (mb_a != mb_b) ? 2 : 1;
    const int W = kWin ? p.window : 0;
    // First key tile of a block (its first row's window start) and its tile count.
    auto item_t0 = [&](int mb) -> int { return kWin ? max(0, mb * BM - W + 1) / BN : 0; };
    auto item_tiles = [&](int mb) -> int {
        const int kv_hi = kCaus ? min(T, (mb + 1) * BM) : T;
        return (kv_hi + BN - 1) / BN - item_t0(mb);
    };
    const int nt_a = item_tiles(mb_a);
    const int ntot = nt_a + (nitems == 2 ? item_tiles(mb_b) : 0);
    const int tb_a = item_t0(mb_a), tb_b = item_t0(mb_b);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const int c = lane & 31, g = lane >> 5;

    // Head dim in HBM: DP, or (PAD) D < DP with CG 16-byte chunks per row.
    const int D = PAD ? p.D : DP;
    const int RBG = 2 * D;
    const int CG = D / 8;
    const size_t base = (size_t)bh * T * D;
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

    const uint32_t nrec = (uint32_t)T * (uint32_t)RBG;
    const i32x4 rq = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.q) + base, nrec);
    const i32x4 rk = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.k) + base, nrec);
    const i32x4 rv = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.v) + base, nrec);

    // Tile u of the workgroup's sequence -> stage st: wave-instruction i
    // writes LDS slots (wave * LPW + i) * 64 + lane, slot = row * CPR + chunk'.
    const int32_t* __restrict__ docb = nullptr;
    if constexpr (DOC) docb = p.doc + (size_t)(bh / p.H) * T;
    const i32x4 rdoc = buffer_rsrc(docb, DOC ? (uint32_t)T * 4u : 0u);
    auto issue = [&](int u, int st) __attribute__((always_inline)) {
        int key0 = (u < nt_a ? tb_a + u : tb_b + (u - nt_a)) * BN;
        if constexpr (DOC) key0 = (tb_a + (__builtin_amdgcn_readfirstlane(t_list[u]) & ~kDocOne)) * BN;
        uint8_t* kb = k_lds + st * TB;
        uint8_t* vb = v_lds + st * TB;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int slot = (wave * LPW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int off = (key0 + row) * RBG;
            const int kc = pc ^ (row & 15), vc = pc ^ ((row & 3) << 2);
            dma_load16(rk, lds_addr(kb + (wave * LPW + i) * 1024), (PAD && kc >= CG) ? kBufOOB : off + (kc << 4));
            dma_load16(rv, lds_addr(vb + (wave * LPW + i) * 1024), (PAD && vc >= CG) ? kBufOOB : off + (vc << 4));
        }
        // Documents: this wave's KDW of the tile's key ids (lanes 0 .. KDW/4 - 1).
        if constexpr (DOC)
            if (lane < KDW / 4)
                dma_load16(rdoc, lds_addr(kd_lds + st * BN + wave * KDW), (key0 + wave * KDW + lane * 4) * 4);
    };
    auto issue_q = [&](int mb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < LQW; ++i) {
            const int slot = (wave * LQW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int qc = pc ^ (row & 15);
            dma_load16<true>(rq, lds_addr(q_lds + (wave * LQW + i) * 1024),
                             (PAD && qc >= CG) ? kBufOOB : (mb * BM + row) * RBG + (qc << 4));
        }
    };

    int qrow = 0;  // this lane's query row (current item)
    u32x4 qr[KS];
    f32x16 oacc[DB];
    float zacc[2];

    // Per-lane V offsets (transposed read): row kc + 4 g + (lane & 15) / 4
    // (+8), column db*32 + 16 ((lane >> 4) & 1) + 4 (lane & 3).
    const int vrow_l = 4 * g + ((lane & 15) >> 2);
    const int vcol_l = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    // K (A operand of S^T = K Q^T): key row nb*32 + c, chunk 2 ks + g.
    auto k_operand = [&](const uint8_t* kb, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + c;
        const int pc = (2 * ks + g) ^ (row & 15);
        return *reinterpret_cast<const u32x4*>(kb + row * RB + pc * 16);
    };
    auto v_operand = [&](const uint8_t* vb, int nb, int hh, int db) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + hh * 16 + vrow_l;
        const int col = db * 32 + vcol_l;
        const int pc = (col >> 3) ^ ((row & 3) << 2);  // rows r and r + 8 share the swizzle
        const uint8_t* b0 = vb + row * RB + pc * 16 + (col & 7) * 2;
        const uint8_t* b1 = b0 + 8 * RB;
        const u32x2 x = lds_read_tr16(reinterpret_cast<const uint16_t*>(b0));
        const u32x2 y = lds_read_tr16(reinterpret_cast<const uint16_t*>(b1));
        const u32x4 a = {x[0], x[1], y[0], y[1]};
        return a;
    };

    // Tile forms, passed as integral constants: kFull (no mask) or kMasked
    // (key past the row, or before its window, zeroed per element).
    constexpr int kFull = 1, kMasked = 2, kDocm = 3;
    using Full = std::integral_constant<int, kFull>;
    using Masked = std::integral_constant<int, kMasked>;
    using Docm = std::integral_constant<int, kDocm>;
    // Documents: the row's id (INT_MIN past T); per tile, whether this wave
    // tests it per element (dmw), its first key and the stage's key ids.
    int qdoc = INT_MIN;
    bool dmw = true;
    int dkey0 = 0;
    const int32_t* kdp = kd_lds;

    // Elementwise pass over one 32-key half of S^T (lane: query c, keys
    // kbase + 8 (r / 4) + r % 4): p' = relu(x|x|) packed, z += p'.  Masked
    // keys (past the row, or before its window) are zeroed first.
    constexpr int PW = PUR ? 8 : 1;  // packed low parts of the purified weights
    auto elementwise = [&](f32x16& s, uint32_t (&pk)[8], uint32_t (&pl)[PW], auto m, int kbase)
        __attribute__((always_inline)) {
        if constexpr (PUR) {
            // Weights zeroed past the row (causal) or past T (dense), before
            // the row's window, and (documents) in another document: bit r of
            // dmask for register r.
            const int lim = (kCaus ? qrow : T - 1) - kbase;
            const int wlo = kWin ? qrow - kbase - W + 1 : 0;
            uint32_t dmask = 0;
            if constexpr (decltype(m)::value == kDocm) {
                if (dmw) {
                    const int32_t* kd = kdp + (kbase - dkey0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int4 d4 = *reinterpret_cast<const int4*>(kd + 8 * i);
                        const int dk[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (((kCaus && kWin) ? pair_cut<true, true>(lim - (8 * i + k), W) : (8 * i + k > lim || (kWin && 8 * i + k < wlo))) ||
                                dk[k] != qdoc)
                                dmask |= 1u << (4 * i + k);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float w[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float x = s[2 * j + e];
                    const float t = fmaf(x, pg, pgt);
                    const float u = __int_as_float(max(__float_as_int(t), 0));
                    const float bq = __int_as_float(max(__float_as_int(x * pse), 0));
                    const float u2 = u * u;
                    float pw = fmaf(u2, u2, bq * bq);
                    if constexpr (decltype(m)::value == kMasked) {
                        const int r = 2 * j + e, off = 8 * (r >> 2) + (r & 3);
                        if ((kCaus && kWin) ? pair_cut<true, true>(lim - off, W) : (off > lim || (kWin && off < wlo))) pw = 0.f;
                    }
                    if constexpr (decltype(m)::value == kDocm)
                        if ((dmask >> (2 * j + e)) & 1u) pw = 0.f;
                    w[e] = pw;
                }
                zacc[0] += w[0] + w[1];
                const uint32_t hi = BF16::pack(w[0], w[1]);
                pk[j] = hi;
                pl[j % PW] = BF16::pack(w[0] - BF16::lo(hi), w[1] - BF16::hi(hi));
            }
            return;
        }
        if constexpr (decltype(m)::value == kMasked) {
            const int lim = qrow - kbase;
            const int wlo = kWin ? lim - W + 1 : 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                if ((kCaus && kWin) ? pair_cut<true, true>(lim - off, W) : ((kCaus && off > lim) || (kWin && off < wlo))) s[r] = 0.f;
            }
        }
        if constexpr (decltype(m)::value == kDocm) {
            // Masked past the row (causal) or in another document.
            if (dmw) {
                const int lim = kCaus ? qrow - kbase : INT_MAX;
                const int wlo = kWin ? lim - W + 1 : 0;  // window: first visible key
                const int32_t* kd = kdp + (kbase - dkey0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int4 d4 = *reinterpret_cast<const int4*>(kd + 8 * i);
                    const int dk[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (((kCaus && kWin) ? pair_cut<true, true>(lim - (8 * i + k), W) : (8 * i + k > lim || (kWin && 8 * i + k < wlo))) ||
                            dk[k] != qdoc)
                            s[4 * i + k] = 0.f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            pk[j] = born_weight_pair<E>(s[2 * j], s[2 * j + 1], sq_pre, zacc[j & 1]);
        }
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
    auto qk_op = [&](const u32x4 (&ops)[KS], f32x16& s) __attribute__((always_inline)) {
        s = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s = E::mfma(ops[ks], qr[ks], s);
    };
    auto pv_op = [&](const u32x4 (&ops)[2][DB], const uint32_t (&pk)[8], const uint32_t (&pl)[PW])
        __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const u32x4 bq = {pk[4 * hh], pk[4 * hh + 1], pk[4 * hh + 2], pk[4 * hh + 3]};
                if constexpr (PUR) {
                    const u32x4 bl = {pl[4 * hh % PW], pl[(4 * hh + 1) % PW], pl[(4 * hh + 2) % PW],
                                      pl[(4 * hh + 3) % PW]};
                    oacc[db] = pur_pv<E>(ops[hh][db], bq, bl, oacc[db]);
                } else {
                    oacc[db] = E::mfma(ops[hh][db], bq, oacc[db]);
                }
            }
    };
    // One tile, four fenced phases (kop: K of keys 0-31, read after the
    // tile's barrier):
    //   1: S0 = QK(kop)                           reads K(keys 32-63) -> kop1
    //   2: S1 = QK(kop1) | elementwise(S0) -> P0  reads V(keys 0-31)  -> vop0
    //   3: O += PV(vop0, P0) | elementwise(S1)    reads V(keys 32-63) -> vop1
    //   4: O += PV(vop1, P1)
    // Purified: twice the PV MFMAs and about four times the elementwise
    // VALU work per weight; V of keys 32-63 is read at the start of phase 4
    // instead (keeps the tile within the register budget).
    constexpr int V2 = PUR ? 20 : 6, V3 = PUR ? 10 : 6;
    auto tile = [&](const uint8_t* kb, const uint8_t* vb, int key0, auto m) __attribute__((always_inline)) {
        f32x16 s0, s1;
        uint32_t pk0[8], pk1[8], pl0[PW], pl1[PW];
        u32x4 kop1[KS], vop0[2][DB], vop1[2][DB];
        // 1
        __builtin_amdgcn_s_setprio(1);
        read_k(kop1, kb, 1);
        qk_op(kop, s0);
        __builtin_amdgcn_sched_barrier(0);
        // 2
        __builtin_amdgcn_s_setprio(0);
        read_v(vop0, vb, 0);
        qk_op(kop1, s1);
        elementwise(s0, pk0, pl0, m, key0 + 4 * g);
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, V2, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // DS read
        }
        __builtin_amdgcn_sched_barrier(0);
        // 3
        if constexpr (!PUR) read_v(vop1, vb, 1);
        pv_op(vop0, pk0, pl0);
        elementwise(s1, pk1, pl1, m, key0 + 32 + 4 * g);
#pragma unroll
        for (int i = 0; i < (PUR ? (std::is_same<E, F16>::value ? 6 : 4) : 2) * DB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x002, V3, 1);
            if constexpr (!PUR) __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        // 4
        __builtin_amdgcn_s_setprio(1);
        if constexpr (PUR) read_v(vop1, vb, 1);
        pv_op(vop1, pk1, pl1);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };

    // This wave's 32 rows of the Q block in LDS -> B operands of S^T, the
    // sign of the scale folded in; the asm pins them in registers.
    auto load_q = [&]() __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int row = 32 * wave + (ln & 31);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int pc = (2 * ks + (ln >> 5)) ^ (row & 15);
            qr[ks] = *reinterpret_cast<const u32x4*>(q_lds + row * RB + pc * 16);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            qr[ks] ^= flip;
            asm volatile("" : "+v"(qr[ks]));
        }
    };

    uint16_t* __restrict__ O = reinterpret_cast<uint16_t*>(p.o) + base;
    float* __restrict__ O32 = reinterpret_cast<float*>(p.o) + base;  // purified: fp32 rows
    float* __restrict__ Zp = p.z + (size_t)bh * T;
    const float s2 = (sq_pre > 0.f) ? (sc / sq_pre) * (sc / sq_pre) : 0.f;
    const float eps_s = (p.eps == 0.f) ? 0.f : p.eps / s2;

    // Normalise and store a finished item's rows: pack() turns the
    // accumulators into 16-bit pairs, put_lds() writes them into this wave's
    // own rows of the Q block (their Q is in registers by then), flush()
    // reads them back 16 bytes per lane (4 whole rows per store instruction)
    // and stores them and the row sums, non-temporal.
    u32x2 opk[DB][4];
    float ztot = 0.f;
    auto pack = [&]() __attribute__((always_inline)) {
        const float zl = zacc[0] + zacc[1];
        ztot = zl + __shfl_xor(zl, 32);
        const float rcp = 1.0f / (ztot + eps_s);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x16& o = oacc[db];
                opk[db][j][0] = E::pack(o[4 * j] * rcp, o[4 * j + 1] * rcp);
                opk[db][j][1] = E::pack(o[4 * j + 2] * rcp, o[4 * j + 3] * rcp);
            }
    };
    // Output staging: this wave's rows of the Q block (documents: its 32 rows
    // of the idle ring, waves 0-3 in the K ring, 4-7 in the V ring).
    static_assert(!DOC || NST * BN >= 4 * 32, "documents: four waves' rows fit one ring");
    uint8_t* const stg = DOC ? (wave < 4 ? k_lds : v_lds) + 32 * (wave & 3) * RB : q_lds + 32 * wave * RB;
    auto put_lds = [&]() __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int row = ln & 31;  // of the wave's 32 (row & 15 as for the block row)
        const int gg = ln >> 5;
        uint8_t* rb = stg + row * RB;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int chunk = 4 * db + j;  // columns 32 db + 8 j + 4 gg .. +3
                *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 15)) << 4) + 8 * gg) = opk[db][j];
            }
    };
    auto flush = [&](int mb) __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int qz = mb * BM + 32 * wave + (ln & 31);
        if ((ln >> 5) == 0 && qz < T) __builtin_nontemporal_store(s2 * ztot + p.eps, Zp + qz);
        const int chunk = ln & 15;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = 4 * i + (ln >> 4);
            const u32x4 x = *reinterpret_cast<const u32x4*>(stg + row * RB + ((chunk ^ (row & 15)) << 4));
            const int qi = mb * BM + 32 * wave + row;
            if (qi < T && (!PAD || chunk < CG))
                __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(O + (size_t)qi * D + chunk * 8));
        }
    };
    // Purified: O = acc / (Z + eps) and Z + eps, fp32, straight from the
    // accumulators (lane: one query row, 4 consecutive columns per store).
    // Plain stores for O: an instruction writes 32 bytes of each row, and L2
    // merges a row's pieces into whole lines before they reach HBM
    // (non-temporal stores wrote them partial, 2.3x the output bytes).
    auto store_pur = [&](int mb) __attribute__((always_inline)) {
        const float zl = zacc[0] + zacc[1];
        const float zd = zl + __shfl_xor(zl, 32) + p.eps;
        const int qi = mb * BM + 32 * wave + c;
        if (qi < T) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x16& o = oacc[db];
                    const f32x4 w = {o[4 * j] / zd, o[4 * j + 1] / zd, o[4 * j + 2] / zd, o[4 * j + 3] / zd};
                    const int col = db * 32 + 8 * j + 4 * g;
                    if (!PAD || col < D)
                        *reinterpret_cast<f32x4*>(O32 + (size_t)qi * D + col) = w;
                }
            if (g == 0) __builtin_nontemporal_store(zd, Zp + qi);
        }
    };
    auto start_item = [&](int mb) __attribute__((always_inline)) {
        qrow = mb * BM + 32 * wave + c;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db] = zero16();
        zacc[0] = zacc[1] = 0.f;
    };

    // Load pipeline (as in the D == 64 kernel): Q of item 0 and tiles 0, 1
    // up front; at the top of step u, after the barrier, tile u+2 (and at
    // u == uq the second item's Q block, ahead of tile uq+2).  Each wave waits
    // for its share of tile u (everything issued before tile u+1), then the
    // barrier makes the whole tile visible and frees tile u-1's stage.  The
    // first item's rows are staged in LDS in the second item's first step and
    // stored at the top of its second step (purified: stored from registers
    // in its first step); the next step drains them.
    constexpr int kTileLoads = 2 * LPW, kQLoads = LQW;
    const bool early_q = (nitems == 2);
    const int uq = max(1, nt_a - 4);
    auto top = [&](int u) __attribute__((always_inline)) {
        const bool stores_out = (nitems == 2) && (u == nt_a + (PUR ? 1 : 2));
        const int after = stores_out ? 0 : ((u == uq + 1 && early_q) ? kQLoads : 0) + (u + 1 < ntot ? kTileLoads : 0);
        if (after >= kQLoads + kTileLoads)
            wait_vmcnt<kQLoads + kTileLoads>();
        else if (after >= kTileLoads)
            wait_vmcnt<kTileLoads>();
        else
            wait_vmcnt<0>();
        __syncthreads();
        if (u == uq && early_q) issue_q(mb_b);
        if (u + 2 < ntot) issue(u + 2, (u + 2) % NST);
        if (!PUR && nitems == 2 && u == nt_a + 1) flush(mb_a);
        // The waits above cover the second item's Q block from step uq + 2
        // on.  A first item of one or two tiles (a short last block under a
        // window: uq = 1 and the second item starts at step 1 or 2) starts
        // the second item before that, so its Q block is drained here, and
        // the barrier makes every wave's share visible before any reads it.
        if (early_q && u == nt_a && nt_a < uq + 2) {
            wait_vmcnt<0>();
            __syncthreads();
        }
    };

    if constexpr (DOC) {
        // One block (unpaired launch).  The rows' documents first: the
        // screening needs them; Q (straight into registers, the sign of the
        // scale folded in) is loaded after the first chunk's first two tiles
        // are issued, so its loads overlap theirs.
        start_item(mb_a);
        if (qrow < T) qdoc = docb[qrow];
        auto load_q_regs = [&]() __attribute__((always_inline)) {
            const uint16_t* __restrict__ Qg = reinterpret_cast<const uint16_t*>(p.q) + base;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 x = {0u, 0u, 0u, 0u};
                if (qrow < T && (!PAD || 2 * ks + g < CG)) x = ldg16(Qg + (size_t)qrow * D + (2 * ks + g) * 8);
                qr[ks] = x ^ flip;
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qr[ks]));
        };
        // Document range of this wave's valid rows (uniform; wone: one
        // document) and of the whole block.
        const int rw = mb_a * BM + 32 * wave;
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
        constexpr int kDocTileLoads = 2 * LPW + 1;  // K, V and the wave's key ids
        const int ncand = nt_a;
        for (int c0 = 0; c0 < ncand; c0 += CAP) {
            const int n = screen_doc_tiles<BN>(docb, T, tb_a * BN, c0, min(CAP, ncand - c0), bq_lo, bq_hi, t_keep, t_tdoc,
                                               t_list, t_doc, &s_rng[2 * NW]);
            // Tiles 0 .. NST-2 up front, tile u+NST-1 after the barrier of
            // step u (into the stage of tile u-1).
            if (n > 0) issue(0, 0);
            if (NST == 3 && n > 1) issue(1, 1);
            if (c0 == 0) load_q_regs();
            for (int u = 0; u < n; ++u) {
                if (NST == 3 && u + 1 < n)
                    wait_vmcnt<kDocTileLoads>();
                else
                    wait_vmcnt<0>();
                __syncthreads();
                if (u + NST - 1 < n) issue(u + NST - 1, (u + NST - 1) % NST);
                int soff = (u % NST) * TB;  // opaque: operand addresses formed per tile
                asm volatile("" : "+s"(soff));
                const uint8_t* kb = k_lds + soff;
                const uint8_t* vb = v_lds + soff;
                kdp = kd_lds + (soff / TB) * BN;
                const int e = __builtin_amdgcn_readfirstlane(t_list[u]);
                const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
                dkey0 = (tb_a + (e & ~kDocOne)) * BN;
                const bool one = (e & kDocOne) != 0;
                // Window: the tile is past every row's window when it ends
                // before the first row's, and cut by one when it starts
                // before the last row's.
                const bool vis = !(kCaus && dkey0 > rw + 31) && !(kWin && dkey0 + BN - 1 < rw - W + 1) &&
                                 !(one && (td < wlo || td > whi));
                dmw = (kCaus && dkey0 + BN - 1 > rw) || (kWin && dkey0 < rw + 32 - W) ||
                      !(one && wone && td == wlo) || (PUR && dkey0 + BN > T);
                if (vis) {
                    read_k(kop, kb, 0);
                    tile(kb, vb, dkey0, Docm{});
                }
            }
            __syncthreads();  // the list and the ring are reused by the next chunk (or the output)
        }
        if constexpr (PUR) {
            store_pur(mb_a);
        } else {
            pack();
            put_lds();
            flush(mb_a);
        }
        return;
    }

    issue_q(mb_a);
    issue(0, 0);
    if (ntot > 1) issue(1, 1);

    int u = 0;
    for (int it = 0; it < nitems; ++it) {
        const int mb = it ? mb_b : mb_a;
        const int nt = it ? ntot - nt_a : nt_a;
        const int tb = it ? tb_b : tb_a;
        top(u);
        if constexpr (PUR) {
            if (it > 0) store_pur(mb_a);
            load_q();
        } else if (it > 0) {
            pack();
            load_q();  // before the previous item's rows overwrite this wave's Q rows
            put_lds();
        } else {
            load_q();
        }
        start_item(mb);
        // This wave's rows are rw .. rw + 31: the keys it may see are
        // [kv0, kv1] and the keys all of its rows see [kf0, kf1].  Its tiles
        // (counted from the item's first, tb) fall into five runs: [0, ta)
        // nothing visible, [ta, tf) masked, [tf, tg) full, [tg, tv) masked,
        // [tv, nt) nothing visible (causal: tg is the tile holding the
        // wave's diagonal, tv the one after it).  One loop per run keeps the
        // masked and full tile bodies out of a common branch (two tile bodies
        // in one branch exceed the register budget).  The barriers and loads
        // of every step run in every wave.  Purified, non-causal: the keys
        // past T are masked (the last tile is masked when T % BN != 0).
        constexpr int kBig = 1 << 29;
        const int rw = mb * BM + 32 * wave;
        const int kv0 = kWin ? max(0, rw - W + 1) : 0;
        const int kv1 = kCaus ? rw + 31 : (PUR ? T - 1 : kBig);
        const int kf0 = kWin ? max(0, rw + 32 - W) : 0;
        const int kf1 = kCaus ? rw : (PUR ? T - 1 : kBig);
        auto rel = [&](int kt) -> int { return min(max(kt - tb, 0), nt); };
        const int ta = rel(kv0 / BN);
        const int tv = max(rel(kv1 / BN + 1), ta);
        const int tf = min(max(rel((kf0 + BN - 1) / BN), ta), tv);
        const int tg = min(max(rel((kf1 + 1) / BN), tf), tv);
        auto stage = [&](int uu, const uint8_t*& kb, const uint8_t*& vb) __attribute__((always_inline)) {
            int soff = (uu % NST) * TB;  // opaque: operand addresses formed per tile
            asm volatile("" : "+s"(soff));
            kb = k_lds + soff;
            vb = v_lds + soff;
        };
        int t = 0;
        bool at_top = true;  // top(u) already done for the current step
        auto idle_run = [&](int tend) __attribute__((always_inline)) {
            for (; t < tend; ++t, ++u) {
                if (!at_top) top(u);
                at_top = false;
            }
        };
        auto masked_run = [&](int tend) __attribute__((always_inline)) {
            for (; t < tend; ++t, ++u) {
                if (!at_top) top(u);
                at_top = false;
                const uint8_t *kb, *vb;
                stage(u, kb, vb);
                read_k(kop, kb, 0);
                tile(kb, vb, (tb + t) * BN, Masked{});
            }
        };
        idle_run(ta);
        masked_run(tf);
        for (; t < tg; ++t, ++u) {
            if (!at_top) top(u);
            at_top = false;
            const uint8_t *kb, *vb;
            stage(u, kb, vb);
            read_k(kop, kb, 0);
            tile(kb, vb, (tb + t) * BN, Full{});
        }
        masked_run(tv);
        idle_run(nt);
    }
    if constexpr (PUR) {
        store_pur(nitems == 2 ? mb_b : mb_a);
    } else {
        if (nitems == 2 && ntot == nt_a + 1) flush(mb_a);  // a one-tile second item: no later step
        pack();
        put_lds();
        flush(nitems == 2 ? mb_b : mb_a);
    }
}

// One workgroup per CU (160 KiB of LDS), so the launch runs in rounds of 256
// workgroups.  Paired or unpaired, by the estimated finishing time of each in
// tile steps: paired workgroups all carry about the same work (causal: a pair
// (mb, nmb-1-mb) holds 4 (nmb + 1) tiles; dense: 2 nt) and finish in whole
// rounds; unpaired blocks go out longest first, so the CUs' loads even out
// to about the average plus one short block.  Paired when that is no later
// (it overlaps the second block's start-up with the first's tail): d3, d5
// (one and two full rounds) pair; B8 H10 T2048 (320 pairs, 1.25 rounds)
// does not.
inline bool d128_fwd_paired(int B, int H, int T, bool causal) {
    constexpr int64_t S = 256;  // CUs
    const int64_t BH = (int64_t)B * H;
    const int64_t nmb = (T + 255) / 256, nt = (T + 63) / 64;
    const int64_t rounds = (BH * ((nmb + 1) / 2) + S - 1) / S;
    if (causal) {
        const int64_t total = BH * 2 * nmb * (nmb + 1);  // sum over blocks of 4 (mb + 1)
        return rounds * 4 * (nmb + 1) <= (total + S - 1) / S + 4;
    }
    return rounds * 2 * nt <= (BH * nmb + S - 1) / S * nt;
}

// Documents (with or without a causal window): one block per workgroup, the
// longest key ranges first under causality.
template <class E, int MODE, bool PAD = false>
hipError_t launch_fwd16_d128_doc(const FwdArgs& a, hipStream_t st) {
    using C = FwdD128Cfg;
    // 128-row blocks of 4 waves, two workgroups per CU.
    constexpr int NW = 4, BM = 32 * NW;
    const dim3 grid((unsigned)fast_fwd_nmb(a.T, BM) * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd16_d128_kernel<E, MODE, false, PAD, true, NW>), grid, dim3(NW * 64), 0, st, a);
    return hipGetLastError();
}

template <class E, int MODE, bool PAD = false>
hipError_t launch_fwd16_d128(const FwdArgs& a, hipStream_t st) {
    using C = FwdD128Cfg;
    // Windows: never paired.
    const unsigned BH = (unsigned)(a.B * a.H);
    const unsigned npair = (unsigned)fast_fwd_npair(a.T, C::BM) * BH;
    const unsigned nsingle = (unsigned)fast_fwd_nmb(a.T, C::BM) * BH;
    const bool pair = !mode_window(MODE) && d128_fwd_paired(a.B, a.H, a.T, MODE == kCausal);
    const dim3 grid(pair ? npair : nsingle);
    hipLaunchKernelGGL((born_fwd16_d128_kernel<E, MODE, false, PAD>), grid, dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

// Purified-Born forward with document ids (bf16, D == 128; with or without a
// causal window).
template <int MODE, class E = BF16, bool PAD = false>
hipError_t launch_purified_fwd_d128_doc(const PurArgs& a, hipStream_t st) {
    using C = FwdD128Cfg;
    constexpr int NW = 4, BM = 32 * NW;
    const dim3 grid((unsigned)fast_fwd_nmb(a.T, BM) * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd16_d128_kernel<E, MODE, true, PAD, true, NW>), grid, dim3(NW * 64), 0, st, a);
    return hipGetLastError();
}

// Purified-Born forward through the same kernel (bf16, 64 < D <= 128, dense,
// causal or causal window, no documents); the Born launch's grid, except that
// window blocks (about equal work each) are paired too when two rounds of
// pairs take no longer than the rounds of single blocks: the second block's
// loads then overlap the first block's fp32 output stores (B16 H8 T2048,
// window 384: step 632 -> 620 us; the Born window forward gains nothing).
template <int MODE, bool PAD = false, class E = BF16>
hipError_t launch_purified_fwd_d128(const PurArgs& a, hipStream_t st) {
    using C = FwdD128Cfg;
    const unsigned BH = (unsigned)(a.B * a.H);
    const unsigned npair = (unsigned)fast_fwd_npair(a.T, C::BM) * BH;
    const unsigned nsingle = (unsigned)fast_fwd_nmb(a.T, C::BM) * BH;
    constexpr unsigned kCUs = 256;
    const bool pair = mode_window(MODE) ? 2 * ((npair + kCUs - 1) / kCUs) <= (nsingle + kCUs - 1) / kCUs
                                        : d128_fwd_paired(a.B, a.H, a.T, MODE == kCausal);
    const dim3 grid(pair ? npair : nsingle);
    hipLaunchKernelGGL((born_fwd16_d128_kernel<E, MODE, true, PAD>), grid, dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

}  // namespace qdl
