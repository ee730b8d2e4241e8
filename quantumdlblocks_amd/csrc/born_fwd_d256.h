// Flash-Born forward for head dims 128 < D <= 256 (bf16 / fp16): dense,
// causal, or a sliding window with or without causality; no document ids.
// The arithmetic of the D == 64 and D == 128 forwards (born_fwd_fast.h,
// born_fwd_d128.h: S^T = K Q^T on the 16-bit MFMA, p' = relu(x|x|) packed,
// Z from the packed weights, O^T += V^T P, O = acc / (Z + eps / s^2)) with
// the register split and load pipeline of the wide-row backward
// (born_bwd_d256.h):
//   * A wave's 32 query rows need 64 VGPRs of Q operands and 128 registers
//     of O accumulators (which the MFMAs keep in AGPRs), so the kernel runs
//     one wave per SIMD: 4 waves over a 128-row block, wave w owning rows
//     32 w .. 32 w + 31, Q loaded straight from HBM into registers.
//   * K/V tiles of 64 keys (32 KiB each) go global -> LDS with buffer_load
//     ... lds through a ring of two stages 64 KiB apart, one workgroup per
//     CU; chunks swizzled by swz256 (row reads of K, transposed reads of V,
//     both conflict-free), the lane offsets flipped in place between stages.
//   * Per 32-key half: S^T (16 MFMAs, K rows), the elementwise pass, O^T
//     (16 MFMAs, V transposed), each phase's LDS operand reads issued a few
//     MFMAs ahead.  Each MFMA takes one operand from LDS.
//   * Each wave's tiles split into runs (nothing visible / cut by its
//     diagonal or window edge / fully visible), one loop per run.
// PAD: 128 < D < 256 (a multiple of 8): the loads of the chunks past D return
// zeros, Q is zero there, and the output chunks past D are not stored.
// PUR: the purified-Born weights (flash_born.py:696-811) as in the D == 64 and
// D == 128 forwards: p = relu(gamma (r - tau))^4 + eps_base relu(r)^2 in
// fp32, each weight split into bf16 hi + lo terms for P V (fp16 V split
// exactly into two bf16 terms: pur_pv), Z summed in fp32, O and Z stored in
// fp32 straight from the accumulators; masks zero the weights, so without
// causality the keys past T are masked in the last tile too.
// DOC: document ids (with or without a causal window) as in the D == 128
// kernel's document mode: the block's candidate key tiles screened by
// document-id range into a list in LDS (screen_doc_tiles), each kept tile
// loaded with its 64 key ids; per tile a wave skips the work when the tile
// lies past its rows (or its window) or is one document none of its rows
// belongs to, and tests it per element unless the tile is before its first
// row and one document all of its rows belong to.
#pragma once

#include "born_bwd_d256.h"

namespace qdl {

template <class E, int MODE, bool PAD = false, bool PUR = false, bool DOC = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void born_fwd16_d256_kernel(typename std::conditional<PUR, PurArgs, FwdArgs>::type p) {
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "mask modes");
    static_assert(MODE != kWindowNC || !DOC, "windows without causality: no documents");
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified: 16-bit inputs");
    constexpr int DP = 256, NW = 4, BN = 64, NST = 2, BM = 32 * NW;
    constexpr int KS = DP / 16, DB = DP / 32;
    constexpr int RB = DP * 2;             // bytes per row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    static_assert(TB % (1024 * NW) == 0 && 2 * TB == 0x10000 && BM * RB <= 2 * NST * TB,
                  "tile split / stages 64 KiB apart / staging");
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);

    // Stage st: K tile at 2 TB st, V tile right after it; afterwards the
    // output staging.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * NST * TB];
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
    // The longest key ranges first (causal: the last blocks).
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

    // Key tiles tb .. tb+ntiles-1 (tb: the window's first key tile, else 0).
    const int W = kWin ? p.window : 0;
    const int tb = kWin ? max(0, R - W + 1) / BN : 0;
    const int ntiles = (kCaus ? (min(T, R + BM) + BN - 1) / BN : (T + BN - 1) / BN) - tb;
    // This wave's rows rw .. rw + 31 see keys [rw - W + 1, rw + 31] (causal,
    // window) and all of them see keys [rw + 32 - W, rw]; purified without
    // causality: keys up to T - 1, so a partial last tile is masked.
    const int rw = R + 32 * wave;
    const int vis_hi = kCaus ? rw + 31 : (PUR ? T - 1 : kRunsBig);
    const int all_hi = kCaus ? rw : (PUR ? T - 1 : kRunsBig);
    const WaveRuns runs(tb * BN, ntiles, kWin ? max(0, rw - W + 1) : 0, vis_hi, kWin ? max(0, rw + 32 - W) : 0, all_hi);

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
        int key0 = (tb + u) * BN;
        if constexpr (DOC) key0 = (tb + (__builtin_amdgcn_readfirstlane(t_list[u]) & ~kDocOne)) * BN;
        uint8_t* kb = smem + (u % NST) * 2 * TB;
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
                dma_load16(rdoc, lds_addr(kd_lds + (u % NST) * BN + wave * KDW), (key0 + wave * KDW + lane * 4) * 4);
    };

    // This lane's Q row chunks 2 ks + g (B operands of S^T), the sign of the
    // scale folded in.
    u32x4 qr[KS];
    auto load_q = [&]() __attribute__((always_inline)) {
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
    // Tile 0 goes out before the Q rows are loaded, so the two overlap
    // (documents: Q first, during the screening, below).
    if constexpr (!DOC) {
        issue(0);
        load_q();
    }

    // Operand reads through the ring's lane offsets (current stage):
    // which = 0 (K rows: A of S^T) or 1 (V transposed: A of O^T).
    RingOffs512 ro(lane);
    constexpr int LEAD = BwdD256Cfg::LEAD;

    f32x16 oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = zero16();
    float zacc[2] = {0.f, 0.f};

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
    // One 32-key half nb of a tile (lane: query c, keys kbase + 8 (r / 4) +
    // r % 4 of register r):
    //   S^T = K Q^T                 (A = K rows, B = Q^T)
    //   p' = relu(x|x|) packed, z += p'   (masked keys zeroed first)
    //   O^T += V^T P                (A = V^T, B = P)
    auto half = [&](int nb, int kbase, auto m) __attribute__((always_inline)) {
        f32x16 s = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s = E::mfma(ro.row(smem, 0, nb, ks), qr[ks], s);
        __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 0);  // DS read
#pragma unroll
        for (int i = 0; i < KS - LEAD; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, LEAD, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(m)::value == kMasked) {
            // Masked past the lane's row (causal) and before its window.
            const int lim = qrow - kbase;
            const int wlo = kWin ? lim - W + 1 : 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                if ((kCaus && off > lim) || (kWin && off < wlo)) s[r] = 0.f;
            }
        }
        constexpr int PW = PUR ? 8 : 1;  // packed low parts of the purified weights
        uint32_t pk[8], pl[PW];
        if constexpr (PUR) {
            // Weights zeroed past the row (causal) or past T (dense), and
            // before the row's window.
            const int lim = (kCaus ? qrow : T - 1) - kbase;
            const int wlo = kWin ? qrow - kbase - W + 1 : 0;
            // Documents: bit r set for a register masked by the diagonal
            // (causal), T, the window or another document.
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
                            if (8 * i + k > lim || (kWin && 8 * i + k < wlo) || dk[k] != qdoc)
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
                    const float uu = __int_as_float(max(__float_as_int(t), 0));
                    const float bq = __int_as_float(max(__float_as_int(x * pse), 0));
                    const float u2 = uu * uu;
                    float pw = fmaf(u2, u2, bq * bq);
                    if constexpr (decltype(m)::value == kMasked) {
                        const int r = 2 * j + e, off = 8 * (r >> 2) + (r & 3);
                        if (off > lim || (kWin && off < wlo)) pw = 0.f;
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
        } else {
            if constexpr (decltype(m)::value == kDocm) {
                // Masked past the row (causal), before its window or in
                // another document.
                if (dmw) {
                    const int lim = kCaus ? qrow - kbase : INT_MAX;
                    const int wlo = kWin ? lim - W + 1 : 0;
                    const int32_t* kd = kdp + (kbase - dkey0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int4 d4 = *reinterpret_cast<const int4*>(kd + 8 * i);
                        const int dk[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (8 * i + k > lim || (kWin && 8 * i + k < wlo) || dk[k] != qdoc) s[4 * i + k] = 0.f;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) pk[j] = born_weight_pair<E>(s[2 * j], s[2 * j + 1], sq_pre, zacc[j & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const u32x4 bq = {pk[4 * hh], pk[4 * hh + 1], pk[4 * hh + 2], pk[4 * hh + 3]};
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                if constexpr (PUR) {
                    const u32x4 bl = {pl[4 * hh % PW], pl[(4 * hh + 1) % PW], pl[(4 * hh + 2) % PW],
                                      pl[(4 * hh + 3) % PW]};
                    oacc[db] = pur_pv<E>(ro.tr(smem, 1, nb, hh, db), bq, bl, oacc[db]);
                } else {
                    oacc[db] = E::mfma(ro.tr(smem, 1, nb, hh, db), bq, oacc[db]);
                }
            }
        }
        // Two transposed reads per operand (purified: two or three MFMAs).
        constexpr int MPO = PUR ? (std::is_same<E, F16>::value ? 3 : 2) : 1;
        __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 1);
#pragma unroll
        for (int i = 0; i < 2 * DB - LEAD / 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, MPO, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, MPO * LEAD / 2, 1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // Pipeline: at the top of step u, once tile u has landed (each wave waits
    // for its own share) and the barrier has made it visible and freed tile
    // u-1's stage, tile u+1 goes out into that stage.
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
        // The rows' documents (the screening needs them), then the Q rows,
        // whose transfer overlaps the screening: this wave's range of ids
        // (uniform; wone: one document) and the block's.
        if (qrow < T) qdoc = docb[qrow];
        load_q();
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
        // The kept tiles of each chunk of candidates through the ring.
        for (int c0 = 0; c0 < ntiles; c0 += CAP) {
            const int n = screen_doc_tiles<BN>(docb, T, tb * BN, c0, min(CAP, ntiles - c0), bq_lo, bq_hi, t_keep, t_tdoc,
                                               t_list, t_doc, &s_rng[2 * NW]);
            if (n > 0) issue(0);
            for (u = 0; u < n; ++u) {
                step_n(n);
                kdp = kd_lds + (u % NST) * BN;
                const int e = __builtin_amdgcn_readfirstlane(t_list[u]);
                const int td = __builtin_amdgcn_readfirstlane(t_doc[u]);
                dkey0 = (tb + (e & ~kDocOne)) * BN;
                const bool one = (e & kDocOne) != 0;
                // Window: the tile is past every row's window when it ends
                // before the first row's, and cut by one when it starts
                // before the last row's.
                const bool vis = !(kCaus && dkey0 > rw + 31) && !(kWin && dkey0 + BN - 1 < rw - W + 1) &&
                                 !(one && (td < wlo || td > whi));
                dmw = (kCaus && dkey0 + BN - 1 > rw) || (kWin && dkey0 < rw + 32 - W) ||
                      !(one && wone && td == wlo) || (PUR && dkey0 + BN > T);
                if (vis) {
                    half(0, dkey0 + 4 * g, Docm{});
                    half(1, dkey0 + 32 + 4 * g, Docm{});
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
    run(runs.tf, Masked{});
    run(runs.tg, Full{});
    run(runs.tv, Masked{});
    for (; u < ntiles; ++u) step();
    }

    // Epilogue: Z = s^2 z + eps and O = acc / (z + eps / s^2) (c = sq_pre
    // folded into the weights), packed and staged in this wave's own 32 rows
    // of the idle ring (row r at smem + RB r, chunks XOR-swizzled by r & 15),
    // read back 16 bytes per lane and stored 2 whole rows per instruction.
    if constexpr (PUR) {
        // O = acc / (Z + eps) and Z + eps, fp32, straight from the
        // accumulators (lane: one query row, 4 consecutive columns per store;
        // plain stores, which L2 merges into whole lines).
        const float zl = zacc[0] + zacc[1];
        const float zd = zl + __shfl_xor(zl, 32) + p.eps;
        if (qrow < T) {
            float* __restrict__ O32 = p.o + base;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 w = {oacc[db][4 * j] / zd, oacc[db][4 * j + 1] / zd, oacc[db][4 * j + 2] / zd,
                                     oacc[db][4 * j + 3] / zd};
                    const int col = db * 32 + 8 * j + 4 * g;
                    if (!PAD || col < D) *reinterpret_cast<f32x4*>(O32 + (size_t)qrow * D + col) = w;
                }
            if (g == 0) __builtin_nontemporal_store(zd, p.z + (size_t)bh * T + qrow);
        }
        return;
    }
    __syncthreads();  // every wave is done with the ring
    const float s2 = (sq_pre > 0.f) ? (sc / sq_pre) * (sc / sq_pre) : 0.f;
    const float eps_s = (p.eps == 0.f) ? 0.f : p.eps / s2;
    const float zl = zacc[0] + zacc[1];
    const float ztot = zl + __shfl_xor(zl, 32);
    const float rcp = 1.0f / (ztot + eps_s);
    uint16_t* __restrict__ O = reinterpret_cast<uint16_t*>(p.o) + base;
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
                w[0] = E::pack(oacc[db][4 * j] * rcp, oacc[db][4 * j + 1] * rcp);
                w[1] = E::pack(oacc[db][4 * j + 2] * rcp, oacc[db][4 * j + 3] * rcp);
                const int chunk = 4 * db + j;  // columns 32 db + 8 j + 4 g .. +3
                *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 15)) << 4) + 8 * (ln >> 5)) = w;
            }
    }
    if (g == 0 && qrow < T) __builtin_nontemporal_store(s2 * ztot + p.eps, p.z + (size_t)bh * T + qrow);
    const int chunk = ln & 31;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = 32 * wave + 2 * i + (ln >> 5);
        const u32x4 x = *reinterpret_cast<const u32x4*>(smem + row * RB + ((chunk ^ (row & 15)) << 4));
        const int qi = R + row;
        if (qi < T && (!PAD || chunk < CG))
            __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(O + (size_t)qi * D + chunk * 8));
    }
}

// One 128-row block per workgroup, one workgroup per CU (128 KiB of LDS),
// the longest key ranges first.
template <class E, int MODE, bool PAD, bool PUR = false, bool DOC = false, class A>
hipError_t launch_fwd16_d256(const A& a, hipStream_t st) {
    const unsigned nmb = (unsigned)((a.T + 127) / 128);
    hipLaunchKernelGGL((born_fwd16_d256_kernel<E, MODE, PAD, PUR, DOC>), dim3(nmb * (unsigned)(a.B * a.H)), dim3(256),
                       0, st, a);
    return hipGetLastError();
}

}  // namespace qdl
