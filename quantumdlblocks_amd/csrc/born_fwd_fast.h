// Flash-Born forward, specialised for head dim D == 64 (no padding), non-causal
// or causal without window/document masks: the C2/C3/C5 hot path.
//
// Same arithmetic as born_fwd16_kernel (born_fwd.h); what changes is how the
// tiles move and how the wave's instruction stream is laid out:
//   * K and V tiles go global -> LDS with buffer_load_dwordx4 ... lds (no
//     staging registers, no staging VALU).  Each wave instruction writes 1 KiB
//     of LDS contiguously (lane l at base + 16 l), so tiles are dense in LDS
//     and 16-byte chunks are XOR-swizzled within each row instead of padded:
//       K: chunk' = chunk ^ (row & 7)       -> 8-row ds_read_b128 conflict-free
//       V: chunk' = chunk ^ 2 (row & 3)     -> 4-row ds_read_b64_tr_b16 conflict-free
//     (32 banks x 4 bytes).  Each lane picks the global chunk that belongs in
//     its fixed LDS slot.  Keys >= T lie beyond the buffer's num_records and
//     arrive as zeros.
//   * Four LDS stages: loads run three tiles ahead and are waited for one
//     tile ahead, so tile t+1 is resident while tile t is computed.  One
//     barrier per tile.
//   * Per tile the wave runs QK(keys 0-31), then QK(keys 32-63) interleaved
//     with the first half's elementwise pass, then PV(first half) interleaved
//     with the second half's elementwise pass, then PV(second half); the
//     interleave is pinned with sched_group_barrier so MFMA and VALU co-issue.
//     Every phase's LDS operands are read one phase earlier (the next tile's
//     first K operands during the last PV), so no MFMA waits on an LDS read.
//   * Each wave owns 32*NQB consecutive query rows; under causality a wave
//     skips the tiles past its last row and masks exactly one diagonal tile
//     (the same code path with the causal mask applied).
#pragma once

#include <type_traits>

#include "born_common.h"

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

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(size_t)(lds_void*)(p);
}

// 16 bytes per lane, global (buffer) -> LDS at m0 + 16 * lane.  Issued as
// inline asm so the compiler does not treat it as an LDS store it must wait
// for before every LDS read; completion is tracked by the explicit vmcnt waits
// and barriers of the pipeline instead.  m0 is saved and restored.
__device__ __forceinline__ void dma_load16(i32x4 rsrc, uint32_t lds_base, int voffset) {
    int saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "buffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voffset), "s"(lds_base), "s"(rsrc)
        : "memory");
}

template <int DP>
struct FastFwdCfg {
    static_assert(DP == 64, "tuned for D = 64");
    static constexpr int NW = 4;
    static constexpr int NQB = 2;
    static constexpr int BN = 64;
    static constexpr int NST = 4;
    static constexpr int BM = NW * 32 * NQB;
};

template <class E, int DP, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void born_fwd16_fast_kernel(FwdArgs p) {
    static_assert(MODE == kDense || MODE == kCausal, "no window / document masks here");
    using C = FastFwdCfg<DP>;
    constexpr int NW = C::NW, NQB = C::NQB, BN = C::BN, NST = C::NST, BM = C::BM;
    constexpr int KS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int RB = DP * 2;             // bytes per tile row
    constexpr int CPR = RB / 16;           // 16-byte chunks per row
    constexpr int TB = BN * RB;            // bytes per K or V tile
    constexpr int LPW = TB / (1024 * NW);  // 1-KiB loads per wave per tile (each of K, V)
    static_assert(TB % (1024 * NW) == 0, "tile split");
    constexpr bool kCaus = (MODE == kCausal);

    // Ring of NST stages.  The DMA loads are issued as inline asm, so the
    // compiler never waits on them; their completion is tracked by the
    // pipeline's own vmcnt waits and barriers.
    __shared__ __attribute__((aligned(1024))) uint8_t k_lds[NST * TB];
    __shared__ __attribute__((aligned(1024))) uint8_t v_lds[NST * TB];

    const int T = p.T;
    const int BH = p.B * p.H;
    const int nmb = (T + BM - 1) / BM;
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    const int mb = kCaus ? (nmb - 1 - bid / BH) : (bid / BH);
    const int h = bh % p.H;
    const int m0 = mb * BM;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const int c = lane & 31, g = lane >> 5;

    // Query rows of block qb of this wave.
    int qrow0[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) qrow0[qb] = m0 + 32 * (NQB * wave + qb);
    const int q_lo = qrow0[0];

    const size_t base = (size_t)bh * T * DP;
    const uint16_t* __restrict__ Q = reinterpret_cast<const uint16_t*>(p.q) + base;
    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (sc < 0.f) ? 0x80008000u : 0u;

    u32x4 qr[NQB][KS];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const int row = qrow0[qb] + c;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 x = {0u, 0u, 0u, 0u};
            if (row < T) x = ldg16(Q + (size_t)row * DP + ks * 16 + g * 8);
            qr[qb][ks] = x ^ flip;
        }
    }

    const int kv_hi = kCaus ? min(T, m0 + BM) : T;
    const int ntiles = (kv_hi + BN - 1) / BN;

    const uint32_t nrec = (uint32_t)T * (uint32_t)RB;
    const i32x4 rk = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.k) + base, nrec);
    const i32x4 rv = buffer_rsrc(reinterpret_cast<const uint16_t*>(p.v) + base, nrec);

    // Tile `t` -> stage `st`: wave-instruction i writes LDS slots
    // (wave * LPW + i) * 64 + lane, slot = row * CPR + chunk'.
    auto issue = [&](int t, int st) __attribute__((always_inline)) {
        const int key0 = t * BN;
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
    };

    f32x16 oacc[DB][NQB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) oacc[db][qb] = zero16();
    float zacc[NQB][2];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) zacc[qb][0] = zacc[qb][1] = 0.f;

    // Per-lane LDS byte offsets that do not depend on the tile.
    // K (A operand of S^T = K Q^T): row nb*32 + c, chunk 2 ks + g.
    // V (transposed read): row kc + 4 g + (lane & 15) / 4 (+8), column
    // db*32 + 16 ((lane >> 4) & 1) + 4 (lane & 3).
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

    // Elementwise pass over one 32-key block of S^T: p' = relu(x|x|) packed,
    // z += p'.  Masked keys (causal) are zeroed first when `lim` says so.
    auto elementwise = [&](f32x16 (&s)[NQB], uint32_t (&pk)[NQB][8], auto masked_c, int kbase)
        __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            if constexpr (decltype(masked_c)::value) {
                const int lim = qrow0[qb] + c - kbase;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (8 * (r >> 2) + (r & 3) > lim) s[qb][r] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x0 = s[qb][2 * j], x1 = s[qb][2 * j + 1];
                uint32_t u = relu_pk16(E::pack(x0 * fabsf(x0), x1 * fabsf(x1)));
                zacc[qb][j & 1] = E::sum2(u, zacc[qb][j & 1]);
                pk[qb][j] = u;
            }
        }
    };

    // One tile, four phases, fenced so the scheduler cannot pull a later
    // phase's work (and registers) into an earlier one:
    //   1: S0 = QK(keys 0-31, operands kop)         reads K(keys 32-63) -> kop1
    //   2: S1 = QK(kop1) | elementwise(S0) -> P0    reads V(keys 0-31)  -> vop0
    //   3: O += PV(vop0, P0) | elementwise(S1) -> P1 reads V(keys 32-63) -> vop1
    //   4: O += PV(vop1, P1)                         reads next tile's K(keys 0-31) -> kop
    // `msk` applies the causal mask (the wave's diagonal tile).
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
    auto qk_op = [&](const u32x4 (&ops)[KS], f32x16 (&s)[NQB]) __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) s[qb] = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) s[qb] = E::mfma(ops[ks], qr[qb][ks], s[qb]);
    };
    auto pv_op = [&](const u32x4 (&ops)[2][DB], const uint32_t (&pk)[NQB][8]) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    const u32x4 bq = {pk[qb][4 * hh], pk[qb][4 * hh + 1], pk[qb][4 * hh + 2], pk[qb][4 * hh + 3]};
                    oacc[db][qb] = E::mfma(ops[hh][db], bq, oacc[db][qb]);
                }
    };
    auto tile = [&](const uint8_t* kb, const uint8_t* vb, const uint8_t* kb_next, auto msk, int key0)
        __attribute__((always_inline)) {
        f32x16 s0[NQB], s1[NQB];
        uint32_t pk0[NQB][8], pk1[NQB][8];
        u32x4 kop1[KS], vop0[2][DB], vop1[2][DB];
        // 1
        read_k(kop1, kb, 1);
        qk_op(kop, s0);
        __builtin_amdgcn_sched_barrier(0);
        // 2
        read_v(vop0, vb, 0);
        qk_op(kop1, s1);
        elementwise(s0, pk0, msk, key0 + 4 * g);
#pragma unroll
        for (int i = 0; i < KS * NQB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
        }
        __builtin_amdgcn_sched_barrier(0);
        // 3
        read_v(vop1, vb, 1);
        pv_op(vop0, pk0);
        elementwise(s1, pk1, msk, key0 + 32 + 4 * g);
#pragma unroll
        for (int i = 0; i < 2 * DB * NQB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x002, 10, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        // 4
        read_k(kop, kb_next, 0);
        pv_op(vop1, pk1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // Tile t lives in stage t % NST.  Loads run three tiles ahead; tile t+1
    // is waited for at the top of iteration t, so it is resident while tile
    // t is computed and its first K operands can be read in tile t's last phase.
    for (int t = 0; t < 3 && t < ntiles; ++t) issue(t, t);
    if (ntiles > 2)
        wait_vmcnt<2 * LPW>();
    else
        wait_vmcnt<0>();
    __syncthreads();
    read_k(kop, k_lds, 0);
    int st = 0;  // stage of tile t
    // Top of iteration t: tile t+1 resident for everyone, tile t-1 consumed;
    // then tile t+3 is issued into the stage tile t-1 held.
    auto advance = [&](int t) __attribute__((always_inline)) {
        if (t > 0) {
            if (t + 2 < ntiles)
                wait_vmcnt<2 * LPW>();  // this wave's loads of tile t+1 landed
            else
                wait_vmcnt<0>();
            __syncthreads();
        }
        if (t + 3 < ntiles) issue(t + 3, (st + 3) & (NST - 1));
    };
    // Unmasked tiles first, then (causal) the wave's diagonal tile and the
    // tiles past its rows, which it only keeps in step with the barriers.
    const int t_diag = kCaus ? min(q_lo / BN, ntiles) : ntiles;
    int t = 0;
    for (; t < t_diag; ++t) {
        advance(t);
        const int st1 = (st + 1) & (NST - 1);
        tile(k_lds + st * TB, v_lds + st * TB, k_lds + st1 * TB, std::false_type{}, t * BN);
        st = st1;
    }
    if constexpr (kCaus) {
        static_assert(BN == 64 && NQB == 2, "one diagonal tile per wave");
        for (; t < ntiles; ++t) {
            advance(t);
            const int st1 = (st + 1) & (NST - 1);
            if (t == t_diag) tile(k_lds + st * TB, v_lds + st * TB, k_lds + st1 * TB, std::true_type{}, t * BN);
            st = st1;
        }
    }

    // Epilogue: one query per lane.
    uint16_t* __restrict__ O = reinterpret_cast<uint16_t*>(p.o) + base;
    float* __restrict__ Zp = p.z + (size_t)bh * T;
    const float s2 = sc * sc;
    const float eps_s = (p.eps == 0.f) ? 0.f : p.eps / s2;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const float zl = zacc[qb][0] + zacc[qb][1];
        const float zt = zl + __shfl_xor(zl, 32);
        const float rcp = 1.0f / (zt + eps_s);
        const int qi = qrow0[qb] + c;
        if (qi < T) {
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int d = db * 32 + 8 * j + 4 * g;
                    const f32x16& o = oacc[db][qb];
                    u32x2 w;
                    w[0] = E::pack(o[4 * j] * rcp, o[4 * j + 1] * rcp);
                    w[1] = E::pack(o[4 * j + 2] * rcp, o[4 * j + 3] * rcp);
                    *reinterpret_cast<u32x2*>(O + (size_t)qi * DP + d) = w;
                }
            }
            if (g == 0) Zp[qi] = s2 * zt + p.eps;
        }
    }
}

template <class E, int DP, int MODE>
hipError_t launch_fwd16_fast(const FwdArgs& a, hipStream_t st) {
    using C = FastFwdCfg<DP>;
    const int nmb = (a.T + C::BM - 1) / C::BM;
    const dim3 grid((unsigned)nmb * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd16_fast_kernel<E, DP, MODE>), grid, dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

}  // namespace qdl
