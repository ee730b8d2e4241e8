// Flash-Born forward, specialised for head dim D == 64 (no padding), non-causal
// or causal without window/document masks: the C2/C3/C5 hot path.
//
// Same arithmetic as born_fwd16_kernel (born_fwd.h); what changes is how the
// tiles move, how work is spread over workgroups and waves, and how the
// wave's instruction stream is laid out:
//   * Q, K and V tiles go global -> LDS with buffer_load_dwordx4 ... lds (no
//     staging registers, no staging VALU).  Each wave instruction writes 1 KiB
//     of LDS contiguously (lane l at base + 16 l), so tiles are dense in LDS
//     and 16-byte chunks are XOR-swizzled within each row instead of padded:
//       K:    chunk' = chunk ^ lds_swz(row) -> row reads conflict-free
//       Q:    chunk' = chunk ^ (row & 7)    (read once per query block)
//       V:    chunk' = chunk ^ 2 (row & 3)  -> 4-row ds_read_b64_tr_b16 conflict-free
//     (32 banks x 4 bytes).  Each lane picks the global chunk that belongs in
//     its fixed LDS slot.  Rows >= T lie beyond the buffer's num_records and
//     arrive as zeros.
//   * A workgroup handles one 256-row query block, or (the paired launch)
//     two blocks of one (batch, head), mb and nmb-1-mb, the second block's Q
//     and first K/V tiles loaded while the first block finishes.  Dense
//     launches pair when that still gives every CU two workgroups; causal
//     ones when a head has at most four blocks (fast_fwd_causal_paired).
//     Otherwise one block per workgroup, longest key ranges first: the
//     dispatcher then gives each CU's freed slot the next block.
//   * K/V tiles of both blocks form one sequence through a ring of three LDS
//     stages: tile u+2 is issued right after the barrier that starts tile u,
//     and tile u is waited for only at that barrier, so every load has two
//     tiles of compute to land.  One barrier per tile.
//   * A finished block's rows are normalised, packed to 16 bits, staged in
//     the wave's own rows of the Q buffer and written back 16 bytes per lane
//     (8 whole rows per store instruction), right after a barrier, so they
//     have a full tile of compute to drain before the next wait.
//   * Per tile the wave runs QK(keys 0-31), then QK(keys 32-63) interleaved
//     with the first half's elementwise pass, then PV(first half) interleaved
//     with the second half's elementwise pass, then PV(second half); the
//     interleave is pinned with sched_group_barrier so MFMA and VALU co-issue.
//     Every phase's LDS operands are read one phase earlier (the tile's first
//     K operands right after its barrier).
//   * Rows are dealt to waves so that every wave has work in every tile: the
//     256-row block is four 64-row slices, and wave w owns rows 16w..16w+15 of
//     each slice.  Its MFMA column block 0 holds slices 0 and 1, block 1
//     slices 2 and 3 (column c -> slice 2 qb + c / 16, row 16 w + c % 16).
//     Under causality the block's four diagonal tiles then cost every wave
//     2, 2, 1 and 1 column blocks (block 0 is fully masked past diagonal tile
//     1), instead of one wave carrying all four tiles while the others wait
//     at the barrier.  Diagonal tiles apply the per-element causal mask to
//     the column blocks they cut.
#pragma once

#include <type_traits>

#include "born_common.h"
#include "born_qk_fold.h"
#include "purified_args.h"

namespace qdl {

// s_waitcnt vmcnt(N) leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef __attribute__((address_space(3))) void lds_void;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer descriptor (gfx9 family): 48-bit base, stride 0, num_records in
// bytes; loads at offsets >= num_records return zeros.
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t nbytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    const i32x4 r = {(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), (int)nbytes, 0x00020000};
    return r;
}

// Offset sent to a buffer load that must return zeros (past every range).
constexpr int kBufOOB = 0x7ffffff0;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(size_t)(lds_void*)(p);
}

// 16 bytes per lane, global (buffer) -> LDS at m0 + 16 * lane.  Issued as
// inline asm so the compiler does not treat it as an LDS store it must wait
// for before every LDS read; completion is tracked by the explicit vmcnt waits
// and barriers of the pipeline instead.  m0 is saved and restored.
template <bool kStream = false>
__device__ __forceinline__ void dma_load16(i32x4 rsrc, uint32_t lds_base, int voffset) {
    int saved;
    if constexpr (kStream) {  // read once: streaming (non-temporal) cache policy
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %2\n\t"
            "buffer_load_dwordx4 %1, %3, 0 offen nt lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "v"(voffset), "s"(lds_base), "s"(rsrc)
            : "memory");
    } else {
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %2\n\t"
            "buffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "v"(voffset), "s"(lds_base), "s"(rsrc)
            : "memory");
    }
}

template <int DP>
struct FastFwdCfg {
    static_assert(DP == 64, "tuned for D = 64");
    static constexpr int NW = 4;
    static constexpr int NQB = 2;
    static constexpr int BN = 64;
    static constexpr int NST = 3;
    static constexpr int BM = NW * 32 * NQB;
};

// Query blocks per (batch, head) and workgroups per (batch, head).
__host__ __device__ inline int fast_fwd_nmb(int T, int BM) { return (T + BM - 1) / BM; }
__host__ __device__ inline int fast_fwd_npair(int T, int BM) { return (fast_fwd_nmb(T, BM) + 1) / 2; }

// PUR selects the purified-Born weights (flash_born.py:696-811): with r the
// raw overlap, p = relu(gamma (r - tau))^4 + eps_base relu(r)^2 in fp32,
// Z = sum p + eps in fp32, O = sum p v / Z written in fp32.  The reference
// contracts P V in fp32; here each weight is split into two bf16 terms,
// p = hi + lo with hi = bf16(p), lo = bf16(p - hi) (|p - hi - lo| <= 2^-17 p),
// and both go through the bf16 MFMA against the exact bf16 V, so the product
// keeps ~16 bits of each weight at bf16 MFMA rate.  Masked and out-of-range
// pairs have their weight zeroed (a zero overlap still weighs
// relu(-gamma tau)^4 when tau < 0).  Output rows are stored straight from the
// accumulators.
// PAD (purified only): a head dim D < 64 (a multiple of 8); the rows in HBM
// are 2 D bytes, the chunks past D are loaded from outside the buffer's range
// (zeros in LDS) and the output columns past D are not stored.
template <class E, int DP, int MODE, bool PUR = false, bool PRO = false, bool PAD = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void born_fwd16_fast_kernel(
    typename std::conditional<PUR, PurArgs, typename std::conditional<PRO, FwdProArgs, FwdArgs>::type>::type p) {
    static_assert(MODE == kDense || MODE == kCausal || mode_window(MODE), "no document masks here");
    // Purified: the weights are split into bf16 terms (fp32's exponent range)
    // whatever the input dtype; fp16 V is split exactly into two bf16 terms.
    static_assert(!PUR || std::is_same<E, BF16>::value || std::is_same<E, F16>::value, "purified: 16-bit inputs");
    static_assert(!PRO || (std::is_same<E, BF16>::value && !PUR), "the fused prologue is bf16 Born only");
    static_assert(!mode_window(MODE) || !PRO, "sliding windows: no fused prologue");
    static_assert(!PAD || PUR, "narrow head dims: purified");
    using C = FastFwdCfg<DP>;
    constexpr int NW = C::NW, NQB = C::NQB, BN = C::BN, NST = C::NST, BM = C::BM;
    constexpr int KS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int QB = BM * RB;            // bytes per Q block
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    constexpr int LQW = QB / (1024 * NW);  // 1-KiB loads per wave per Q block
    static_assert(TB % (1024 * NW) == 0 && QB % (1024 * NW) == 0, "tile split");
    static_assert(NST == 3, "vmcnt bookkeeping below assumes a three-stage ring");
    // kWindow: causal, and row i sees keys i - window + 1 .. i
    // (flash_born.py:152, 173-174); kWindowNC: not causal, row i sees keys
    // i - window + 1 .. T - 1.  Launched unpaired (one block per workgroup);
    // each block visits the key tiles from its window's first key on.
    constexpr bool kWin = mode_window(MODE);
    constexpr bool kCaus = mode_causal(MODE);

    // The DMA loads are issued as inline asm, so the compiler never waits on
    // them; their completion is tracked by the pipeline's own vmcnt waits and
    // barriers.  80 KiB in all: two workgroups per CU.
    __shared__ __attribute__((aligned(1024))) uint8_t k_lds[NST * TB];
    __shared__ __attribute__((aligned(1024))) uint8_t v_lds[NST * TB];
    __shared__ __attribute__((aligned(1024))) uint8_t q_lds[QB];

    const int T = p.T;
    const int BH = p.B * p.H;
    const int nmb = fast_fwd_nmb(T, BM);
    const int bid = blockIdx.x;
    // Paired launch (fast_fwd_npair blocks per head): item 0 is query block
    // nmb-1-pr (the longer key range under causality), item 1 block pr when
    // that is a different block.  Unpaired launch (nmb blocks per head, for
    // problems too small to give every CU two paired workgroups): one block
    // per workgroup, the longest key ranges first, except that with 257 to
    // 512 workgroups the second 256 take theirs in ascending length:
    // workgroups k and k + 256 share a CU (the dispatcher deals workgroups to
    // the 8 XCDs in turn and fills each XCD's 32 CUs in order), so every CU
    // pairs a long block with a short one.
    const bool paired = gridDim.x < (unsigned)(nmb * BH);
    const int item = (!paired && kCaus && bid >= 256 && gridDim.x <= 512u) ? (int)gridDim.x + 255 - bid : bid;
    const int bh = item % BH;
    const int pr = item / BH;
    const int h = bh % p.H;
    // kWindowNC: the first blocks see the most keys, so they go first.
    const int mb_a = (MODE == kWindowNC && !paired) ? pr : nmb - 1 - pr, mb_b = paired ? pr : mb_a;
    const int nitems = (mb_a != mb_b) ? 2 : 1;
    const int W = kWin ? p.window : 0;
    // First key tile of a block (its window's first key), and its tile count.
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
    // Purified weights: t = gamma r - gamma tau, b' = sqrt(eps_base) relu(r).
    float pg = 0.f, pgt = 0.f, pse = 0.f;
    if constexpr (PUR) {
        pg = sc;
        pgt = -sc * p.tau[p.per_head_tau ? h : 0];
        pse = sqrtf(p.eps_base);
    }
    // fp16: the weights are the reference's relu(s r)^2 (c = |s| times the
    // sign-folded overlap; born_weight_pair); bf16: s^2 goes back in per row.
    const float sq_pre = E::kScaleInSquare ? fabsf(sc) : 1.f;

    const uint32_t nrec = (uint32_t)T * (uint32_t)RBG;
    // Bytes between consecutive Q / K rows: 2 D, or the raw rows' time stride
    // when the prologue is fused (the host keeps (T + 256) rows of it within
    // 32-bit offsets).
    uint32_t qrow_b = RBG;
    size_t qbase = base;
    if constexpr (PRO) {
        qrow_b = (uint32_t)p.q_st * 2u;
        qbase = (size_t)(bh / p.H) * p.q_sb + (size_t)h * p.q_sh;
    }
    const i32x4 rq = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.q) + qbase, (uint32_t)T * qrow_b);
    const i32x4 rk = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.k) + base, nrec);
    const i32x4 rv = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.v) + base, nrec);

    // Tile u of the block's sequence -> stage st: wave-instruction i writes
    // LDS slots (wave * LPW + i) * 64 + lane, slot = row * CPR + chunk'.
    auto issue = [&](int u, int st) __attribute__((always_inline)) {
        const int key0 = (u < nt_a ? tb_a + u : tb_b + (u - nt_a)) * BN;
        uint8_t* kb = k_lds + st * TB;
        uint8_t* vb = v_lds + st * TB;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int slot = (wave * LPW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int off = (key0 + row) * RBG;
            const int kc = pc ^ lds_swz(row), vc = pc ^ ((row & 3) << 1);
            dma_load16(rk, lds_addr(kb + (wave * LPW + i) * 1024), (PAD && kc >= CG) ? kBufOOB : off + (kc << 4));
            dma_load16(rv, lds_addr(vb + (wave * LPW + i) * 1024), (PAD && vc >= CG) ? kBufOOB : off + (vc << 4));
        }
    };
    auto issue_q = [&](int mb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < LQW; ++i) {
            const int slot = (wave * LQW + i) * 64 + lane;
            const int row = slot / CPR, pc = slot % CPR;
            const int qc = pc ^ (row & 7);
            dma_load16<true>(rq, lds_addr(q_lds + (wave * LQW + i) * 1024),
                             (PAD && qc >= CG) ? kBufOOB : (mb * BM + row) * (int)qrow_b + (qc << 4));
        }
    };

    static_assert(NQB == 2 && BM == 4 * BN && BN == 64, "two column blocks over four 64-row slices");
    // Row of MFMA column c within a block: slice 2 qb + c / 16, row 16 w + c % 16.
    const int lrow = 64 * (c >> 4) + 16 * wave + (c & 15);
    int qrow[NQB];  // query row of this lane's column in block qb (current item)
    int mlim[NQB];  // last visible key of a masked column block: the query row (causal) or T - 1
    u32x4 qr[NQB][KS];
    f32x16 oacc[DB][NQB];
    float zacc[NQB][2];

    // Per-lane LDS byte offsets that do not depend on the tile.
    // K (A operand of S^T = K Q^T): row nb*32 + c, chunk 2 ks + g.
    // V (transposed read): row kc + 4 g + (lane & 15) / 4 (+8), column
    // db*32 + 16 ((lane >> 4) & 1) + 4 (lane & 3).
    const int vrow_l = 4 * g + ((lane & 15) >> 2);
    const int vcol_l = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    auto k_operand = [&](const uint8_t* kb, int nb, int ks) __attribute__((always_inline)) -> u32x4 {
        const int row = nb * 32 + c;
        const int pc = (2 * ks + g) ^ lds_swz(row);
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

    // Column-block modes of a tile, passed as integral constants:
    // kSkip (no visible key: no MFMA, no VALU), kFull, kMasked (causal
    // mask applied per element).
    constexpr int kSkip = 0, kFull = 1, kMasked = 2;
    using Skip = std::integral_constant<int, kSkip>;
    using Full = std::integral_constant<int, kFull>;
    using Masked = std::integral_constant<int, kMasked>;

    // Elementwise pass over one 32-key block of S^T: p' = relu(x|x|) packed,
    // z += p'.  Masked keys (key > query row) are zeroed first.
    constexpr int PW = PUR ? 8 : 1;  // packed low parts of the purified weights
    auto elementwise = [&](f32x16 (&s)[NQB], uint32_t (&pk)[NQB][8], uint32_t (&pl)[NQB][PW], auto m0, auto m1,
                           int kbase) __attribute__((always_inline)) {
        constexpr int M[NQB] = {decltype(m0)::value, decltype(m1)::value};
        if constexpr (PUR) {
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                if (M[qb] == kSkip) continue;
                const int lim = mlim[qb] - kbase;
                const int wlo = kWin ? qrow[qb] - kbase - W + 1 : 0;  // window: first visible key
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float w[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float x = s[qb][2 * j + e];
                        const float t = fmaf(x, pg, pgt);
                        const float u = __int_as_float(max(__float_as_int(t), 0));
                        const float bq = __int_as_float(max(__float_as_int(x * pse), 0));
                        const float u2 = u * u;
                        float pw = fmaf(u2, u2, bq * bq);
                        if (M[qb] == kMasked) {
                            const int r = 2 * j + e;
                            const int off = 8 * (r >> 2) + (r & 3);
                            if (off > lim || (kWin && off < wlo)) pw = 0.f;
                        }
                        w[e] = pw;
                    }
                    zacc[qb][0] += w[0] + w[1];
                    const uint32_t hi = BF16::pack(w[0], w[1]);
                    pk[qb][j] = hi;
                    pl[qb][j] = BF16::pack(w[0] - BF16::lo(hi), w[1] - BF16::hi(hi));
                }
            }
            return;
        }
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            if (M[qb] == kSkip) continue;
            if (M[qb] == kMasked) {
                // Key kbase + 8 (r / 4) + r % 4 of register r: masked past the
                // lane's row (causal), and (window) before the row's first key.
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
                pk[qb][j] = born_weight_pair<E>(s[qb][2 * j], s[qb][2 * j + 1], sq_pre, zacc[qb][j & 1]);
            }
        }
    };

    // One tile, four phases, fenced so the scheduler cannot pull a later
    // phase's work (and registers) into an earlier one:
    //   1: S0 = QK(keys 0-31, operands kop)         reads K(keys 32-63) -> kop1
    //   2: S1 = QK(kop1) | elementwise(S0) -> P0    reads V(keys 0-31)  -> vop0
    //   3: O += PV(vop0, P0) | elementwise(S1) -> P1 reads V(keys 32-63) -> vop1
    //   4: O += PV(vop1, P1)
    // kop (K of keys 0-31) is read after the tile's barrier, so a tile only
    // has to be resident from its own step on.
    static_assert(NB == 2, "two 32-key halves per tile");
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
    auto qk_op = [&](const u32x4 (&ops)[KS], f32x16 (&s)[NQB], auto m0, auto m1) __attribute__((always_inline)) {
        constexpr int M[NQB] = {decltype(m0)::value, decltype(m1)::value};
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
            if (M[qb] != kSkip) s[qb] = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb)
                if (M[qb] != kSkip) s[qb] = E::mfma(ops[ks], qr[qb][ks], s[qb]);
    };
    auto pv_op = [&](const u32x4 (&ops)[2][DB], const uint32_t (&pk)[NQB][8], const uint32_t (&pl)[NQB][PW],
                     auto m0, auto m1) __attribute__((always_inline)) {
        constexpr int M[NQB] = {decltype(m0)::value, decltype(m1)::value};
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    if (M[qb] == kSkip) continue;
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
    auto tile = [&](const uint8_t* kb, const uint8_t* vb, int key0, auto m0, auto m1)
        __attribute__((always_inline)) {
        constexpr int NA = (decltype(m0)::value != kSkip) + (decltype(m1)::value != kSkip);
        f32x16 s0[NQB], s1[NQB];
        uint32_t pk0[NQB][8], pk1[NQB][8];
        uint32_t pl0[NQB][PW], pl1[NQB][PW];
        // VALU instructions interleaved per MFMA (the purified weights cost
        // about four times the Born ones, and PV issues twice the MFMAs).
        constexpr int V2 = PUR ? 40 : 10, V3 = PUR ? 20 : 10;
        u32x4 kop1[KS], vop0[2][DB], vop1[2][DB];
        // 1 (MFMA only: issued at raised wave priority, so the two
        // workgroups sharing a SIMD hand the matrix pipe back and forth
        // instead of the older one running ahead)
        __builtin_amdgcn_s_setprio(1);
        read_k(kop1, kb, 1);
        qk_op(kop, s0, m0, m1);
        __builtin_amdgcn_sched_barrier(0);
        // 2
        __builtin_amdgcn_s_setprio(0);
        read_v(vop0, vb, 0);
        qk_op(kop1, s1, m0, m1);
        elementwise(s0, pk0, pl0, m0, m1, key0 + 4 * g);
#pragma unroll
        for (int i = 0; i < KS * NA; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, V2, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
        }
        __builtin_amdgcn_sched_barrier(0);
        // 3 (purified: V of keys 32-63 is read at the start of 4 instead,
        // which keeps the phase within the register budget)
        if constexpr (!PUR) read_v(vop1, vb, 1);
        pv_op(vop0, pk0, pl0, m0, m1);
        elementwise(s1, pk1, pl1, m0, m1, key0 + 32 + 4 * g);
#pragma unroll
        for (int i = 0; i < (PUR ? (std::is_same<E, F16>::value ? 6 : 4) : 2) * DB * NA; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x002, V3, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        // 4 (MFMA only)
        __builtin_amdgcn_s_setprio(1);
        if constexpr (PUR) read_v(vop1, vb, 1);
        pv_op(vop1, pk1, pl1, m0, m1);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };

    // Q prologue folded into the query-block load (PRO): the raw query rows
    // come in through the Q block's LDS staging as usual, and each lane turns
    // its rows' operands into q' = l2_normalize(rope(q)) in registers
    // (born_qk_fold.h: bit-identical to the standalone prologue kernel).  The
    // keys arrive normalised (the prologue kernel runs on K alone first):
    // normalising each K tile in LDS here measured slower than the two
    // separate launches (every key tile is staged by ~2.5 workgroups, and the
    // tile loop is bound by instruction issue).
    // The prologue's parameters are re-read from the kernel argument segment
    // where they are used (scalar loads), rather than held in registers
    // through the tile loop, whose scalar and vector registers are all taken.
    typedef const __attribute__((address_space(4))) FwdProArgs* KargPtr;
    auto pro_args = [&]() __attribute__((always_inline)) -> KargPtr {
        KargPtr ka = (KargPtr)(__builtin_amdgcn_kernarg_segment_ptr());
        asm volatile("" : "+s"(ka));
        return ka;
    };
    // This wave's rows of the Q block in LDS -> B operands of S^T.  The sign
    // of the scale is folded into Q; the asm pins the result in registers so
    // it is not recomputed inside the tile loop.
    auto load_q = [&](int mb) __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int lr = 64 * ((ln & 31) >> 4) + 16 * wave + (ln & 15);
        // The Q prologue: every table entry this lane needs, for both of its
        // rows, before any is used.
        RotRow rtab[PRO ? NQB : 1][2];
        bool rot = false;
        if constexpr (PRO) {
            KargPtr ka = pro_args();
            rot = ka->cos != nullptr;
            // One branch around all four row loads, so they form one batch.
            auto load_all = [&](bool vec) __attribute__((always_inline)) {
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    const int t = mb * BM + 128 * qb + lr;
                    KargPtr kt = pro_args();
                    rot_load(kt->cos, kt->sin, kt->ld, kt->nfreq, T, t, 8 * (ln >> 5), vec, rtab[qb][0]);
                    rot_load(kt->cos, kt->sin, kt->ld, kt->nfreq, T, t, 8 * (2 + (ln >> 5)), vec, rtab[qb][1]);
                }
            };
            if (rot) {
                const bool vec = ((reinterpret_cast<uintptr_t>(ka->cos) | reinterpret_cast<uintptr_t>(ka->sin)) & 15) == 0 &&
                                 (ka->ld & 3) == 0 && ka->nfreq >= DP / 2;
                if (vec)
                    load_all(true);
                else
                    load_all(false);
            }
        }
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int row = 128 * qb + lr;
                const int pc = (2 * ks + (ln >> 5)) ^ (row & 7);
                qr[qb][ks] = *reinterpret_cast<const u32x4*>(q_lds + row * RB + pc * 16);
            }
            if constexpr (PRO) {
                // The lane holds chunks g, 2 + g (ks 0, 1) and their partners
                // 4 + g, 6 + g (ks 2, 3); the other half-wave the rest of the row.
                const int gg = ln >> 5;
                const int t = mb * BM + 128 * qb + lr;
                const float rinv = rot_normalise_row(qr[qb], rtab[qb][0], rtab[qb][1], rot, pro_args()->norm_eps);
                // The normalised rows and their 1/norm, for the backward
                // (not written when no backward follows: q_rinv null).
                if (t < T && pro_args()->q_rinv != nullptr) {
                    KargPtr ka = pro_args();
                    uint16_t* qo = reinterpret_cast<uint16_t*>(ka->q_out) + ((size_t)bh * T + t) * DP;
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks)
                        __builtin_nontemporal_store(qr[qb][ks], reinterpret_cast<u32x4*>(qo + 8 * (2 * ks + gg)));
                    if (gg == 0) __builtin_nontemporal_store(rinv, ka->q_rinv + (size_t)bh * T + t);
                }
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                qr[qb][ks] ^= flip;
                asm volatile("" : "+v"(qr[qb][ks]));
            }
        }
    };

    uint16_t* __restrict__ O = reinterpret_cast<uint16_t*>(p.o) + base;
    float* __restrict__ O32 = reinterpret_cast<float*>(p.o) + base;  // purified: fp32 rows
    float* __restrict__ Zp = p.z + (size_t)bh * T;
    const float s2 = (sq_pre > 0.f) ? (sc / sq_pre) * (sc / sq_pre) : 0.f;
    const float eps_s = (p.eps == 0.f) ? 0.f : p.eps / s2;

    // Normalise and store the finished item's rows, in parts so the next
    // item's Q can be read in between: pack() normalises the accumulators
    // into 16-bit pairs (the accumulators die there); put_lds() writes them
    // into this wave's own rows of the Q block in LDS (their Q is already in
    // registers); flush() reads them back 16 bytes per lane, so each store
    // instruction writes 8 whole rows (1 KiB contiguous), and stores the row
    // sums.  Outputs are stored non-temporal: nothing in this kernel reads
    // them, and dirty lines left in L2 would have to be written back when it
    // ends.
    u32x2 opk[NQB][DB][4];
    float ztot[NQB];
    auto pack = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const float zl = zacc[qb][0] + zacc[qb][1];
            ztot[qb] = zl + __shfl_xor(zl, 32);
            const float rcp = 1.0f / (ztot[qb] + eps_s);
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x16& o = oacc[db][qb];
                    opk[qb][db][j][0] = E::pack(o[4 * j] * rcp, o[4 * j + 1] * rcp);
                    opk[qb][db][j][1] = E::pack(o[4 * j + 2] * rcp, o[4 * j + 3] * rcp);
                }
        }
    };
    auto put_lds = [&]() __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int lr = 64 * ((ln & 31) >> 4) + 16 * wave + (ln & 15);
        const int gg = ln >> 5;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const int row = 128 * qb + lr;
            uint8_t* rb = q_lds + row * RB;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int chunk = 4 * db + j;
                    *reinterpret_cast<u32x2*>(rb + ((chunk ^ (row & 7)) << 4) + 8 * gg) = opk[qb][db][j];
                }
        }
    };
    auto flush = [&](int mb) __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int lr = 64 * ((ln & 31) >> 4) + 16 * wave + (ln & 15);
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const int qi = mb * BM + 128 * qb + lr;
            if ((ln >> 5) == 0 && qi < T) __builtin_nontemporal_store(s2 * ztot[qb] + p.eps, Zp + qi);
        }
        const int chunk = ln & 7;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = 64 * (i >> 1) + 16 * wave + 8 * (i & 1) + (ln >> 3);
            const u32x4 x = *reinterpret_cast<const u32x4*>(q_lds + row * RB + ((chunk ^ (row & 7)) << 4));
            const int qi = mb * BM + row;
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
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const float zl = zacc[qb][0] + zacc[qb][1];
            const float zd = zl + __shfl_xor(zl, 32) + p.eps;
            const int qi = mb * BM + 128 * qb + lrow;
            if (qi < T) {
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x16& o = oacc[db][qb];
                        const f32x4 w = {o[4 * j] / zd, o[4 * j + 1] / zd, o[4 * j + 2] / zd, o[4 * j + 3] / zd};
                        const int col = db * 32 + 8 * j + 4 * g;
                        if (!PAD || col < D)
                            *reinterpret_cast<f32x4*>(O32 + (size_t)qi * D + col) = w;
                    }
                if (g == 0) __builtin_nontemporal_store(zd, Zp + qi);
            }
        }
    };
    auto start_item = [&](int mb) __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) qrow[qb] = mb * BM + 128 * qb + lrow;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) mlim[qb] = kCaus ? qrow[qb] : T - 1;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) oacc[db][qb] = zero16();
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) zacc[qb][0] = zacc[qb][1] = 0.f;
    };

    // Load pipeline.  Issue order: Q of item 0, tiles 0 and 1 (prologue);
    // then at the top of step u, after the barrier, tile u+2 (and at u == uq
    // the second item's Q block, ahead of tile uq+2).  At the top of step u
    // each wave waits until its share of tile u has landed (everything
    // issued before tile u+1), then the barrier makes the whole tile visible
    // and frees the stage of tile u-1.  Loads return in order.  The first
    // item's rows are written to LDS in the second item's first step and
    // stored at the top of its second step (after that step's loads are
    // issued); the only stores before the last step, they are drained by
    // the wait one step later.
    // The second item's Q block is issued at the top of step uq, four steps
    // before that item starts (away from the start-up burst).  With two
    // items T > 256, so the first item has at least 5 tiles and 1 <= uq;
    // every wave read the first item's Q at step 0, and the Q block is
    // resident from step uq + 2 on.
    constexpr int kTileLoads = 2 * LPW, kQLoads = LQW;
    const bool early_q = (nitems == 2);
    const int uq = max(1, nt_a - 4);
    auto top = [&](int u) __attribute__((always_inline)) {
        // The first item's rows are stored at step nt_a + 1 (Born, from LDS)
        // or nt_a (purified, from registers); the next step drains them.
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
    };

    issue_q(mb_a);
    issue(0, 0);
    if (ntot > 1) issue(1, 1);

    int u = 0;
    for (int it = 0; it < nitems; ++it) {
        const int mb = it ? mb_b : mb_a;
        const int nt = it ? ntot - nt_a : nt_a;
        // Tiles are counted from the item's first key tile tb (0 but for
        // windows).  Purified, non-causal, T not a multiple of the tile: the
        // last tile masks the keys past T.
        const int tb = it ? tb_b : tb_a;
        const int t0 = kCaus ? min(mb * (BM / BN) - tb, nt) : ((PUR && T % BN) ? nt - 1 : nt);
        // Window: tiles before te hold keys older than some row's window (the
        // block's last row R + 255 sees keys from R + 256 - W on): both
        // column blocks tested per element there.
        const int te = kWin ? min(max((mb * BM + BM - W + BN - 1) / BN - tb, 0), t0) : 0;
        // The item's first step: the previous item's rows go out right
        // after this barrier, a full step before the next wait.
        top(u);
        if constexpr (PUR) {
            if (it > 0) store_pur(mb_a);
            load_q(mb);
        } else if (it > 0) {
            pack();
            load_q(mb);  // before the previous item's rows overwrite this wave's Q rows
            put_lds();
        } else {
            load_q(mb);
        }
        start_item(mb);
        bool at_top = true;  // top(u) already done for the current step
        auto stage = [&](int uu, const uint8_t*& kb, const uint8_t*& vb) __attribute__((always_inline)) {
            // The stage offset is opaque to the optimiser, so it forms each
            // operand address from it per tile instead of keeping addresses
            // for all three stages live in registers.
            int soff = (uu % NST) * TB;
            asm volatile("" : "+s"(soff));
            kb = k_lds + soff;
            vb = v_lds + soff;
        };
        int t = 0;
        if constexpr (kWin) {
            for (; t < te; ++t, ++u) {
                if (!at_top) top(u);
                at_top = false;
                const uint8_t *kb, *vb;
                stage(u, kb, vb);
                read_k(kop, kb, 0);
                tile(kb, vb, (tb + t) * BN, Masked{}, Masked{});
            }
        }
        for (; t < t0; ++t, ++u) {
            if (!at_top) top(u);
            at_top = false;
            const uint8_t *kb, *vb;
            stage(u, kb, vb);
            read_k(kop, kb, 0);
            tile(kb, vb, (tb + t) * BN, Full{}, Full{});
        }
        if constexpr (kCaus) {
            // Diagonal tiles 0 and 1: block 0 cut by the mask, block 1 fully
            // visible (window: tested too, it may start inside the tile);
            // tiles 2 and 3: block 0 fully masked, block 1 cut.
            for (; t < nt; ++t, ++u) {
                if (!at_top) top(u);
                at_top = false;
                const uint8_t *kb, *vb;
                stage(u, kb, vb);
                read_k(kop, kb, 0);
                if (t - t0 < 2) {
                    if constexpr (kWin)
                        tile(kb, vb, (tb + t) * BN, Masked{}, Masked{});
                    else
                        tile(kb, vb, (tb + t) * BN, Masked{}, Full{});
                } else {
                    tile(kb, vb, (tb + t) * BN, Skip{}, Masked{});
                }
            }
        } else if constexpr (PUR) {
            // Not causal: the last tile holds the keys past T (tile counted
            // from tb, the window's first key tile).
            for (; t < nt; ++t, ++u) {
                if (!at_top) top(u);
                at_top = false;
                const uint8_t *kb, *vb;
                stage(u, kb, vb);
                read_k(kop, kb, 0);
                tile(kb, vb, (tb + t) * BN, Masked{}, Masked{});
            }
        }
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

// Causal launches pair blocks (mb, nmb-1-mb) when a head has at most four
// query blocks and the pairs still give every CU two workgroups: unpaired,
// such a launch runs as two rounds of workgroups (the longest blocks, then
// the shortest), and the second round's Q blocks and first tiles are all
// loaded at once mid-kernel; paired, each workgroup loads its second block
// while it finishes the first (C3: 48.1 -> 45.0 us per launch, bit-identical
// outputs).  Longer rows run one block per workgroup, longest first (four or
// more rounds, where the two launches measure the same).
inline bool fast_fwd_causal_paired(int B, int H, int T) {
    const int64_t nmb = (T + 255) / 256;
    return nmb >= 2 && nmb <= 4 && (int64_t)B * H * ((nmb + 1) / 2) >= 512;
}

template <class E, int DP, int MODE>
hipError_t launch_fwd16_fast(const FwdArgs& a, hipStream_t st) {
    using C = FastFwdCfg<DP>;
    // Dense: pair query blocks unless that leaves fewer than two workgroups
    // per CU (256 CUs); then one block per workgroup.  Causal: as
    // fast_fwd_causal_paired decides; windows: one block per workgroup.
    const unsigned BH = (unsigned)(a.B * a.H);
    const unsigned npair = (unsigned)fast_fwd_npair(a.T, C::BM) * BH;
    const unsigned nsingle = (unsigned)fast_fwd_nmb(a.T, C::BM) * BH;
    const bool pair = MODE == kDense ? npair >= 512u : (MODE == kCausal && fast_fwd_causal_paired(a.B, a.H, a.T));
    const dim3 grid(pair ? npair : nsingle);
    hipLaunchKernelGGL((born_fwd16_fast_kernel<E, DP, MODE>), grid, dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

// Born forward with the Q/K prologue fused into the loads (bf16, D == 64,
// dense or causal, no window / documents); same grid as launch_fwd16_fast.
template <int MODE>
hipError_t launch_fwd16_fast_prologue(const FwdProArgs& a, hipStream_t st) {
    using C = FastFwdCfg<64>;
    const unsigned BH = (unsigned)(a.B * a.H);
    const unsigned npair = (unsigned)fast_fwd_npair(a.T, C::BM) * BH;
    const unsigned nsingle = (unsigned)fast_fwd_nmb(a.T, C::BM) * BH;
    const dim3 grid((npair < 512u || MODE == kCausal) ? nsingle : npair);
    hipLaunchKernelGGL((born_fwd16_fast_kernel<BF16, 64, MODE, false, true>), grid, dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

// Purified-Born forward through the same kernel (bf16 or fp16, D == 64,
// dense, causal or a sliding window; no documents).
template <int MODE, bool PAD = false, class E = BF16>
hipError_t launch_purified_fwd_fast(const PurArgs& a, hipStream_t st) {
    using C = FastFwdCfg<64>;
    const unsigned BH = (unsigned)(a.B * a.H);
    const unsigned npair = (unsigned)fast_fwd_npair(a.T, C::BM) * BH;
    const unsigned nsingle = (unsigned)fast_fwd_nmb(a.T, C::BM) * BH;
    const dim3 grid((npair < 512u || MODE != kDense) ? nsingle : npair);
    hipLaunchKernelGGL((born_fwd16_fast_kernel<E, 64, MODE, true, false, PAD>), grid, dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

}  // namespace qdl
