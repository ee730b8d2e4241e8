// Flash-Born forward kernels for gfx950.
//
// Replaces the reference's `_flash_born_fwd_kernel`
// (src/qdlblocks/kernels/flash_born.py:81-192).  One workgroup owns BM = NW*QW
// query rows of one (b, h); each wave owns QW = 32*NQB of them.  K/V tiles of
// BN keys are staged through LDS (double buffered, one barrier per tile) and
// consumed by every wave of the workgroup.
//
// Per tile and wave (16-bit inputs):
//   S^T = K * Q^T        v_mfma_f32_32x32x16, A = K from LDS, B = Q^T held in
//                        registers for the whole kernel
//   p'  = relu(r * |r|)  fp32 -> packed 16-bit, relu on the packed value; the
//                        scale is folded out: relu(s r)^2 = s^2 relu(sign(s) r)^2,
//                        sign(s) is applied to Q once, s^2 at the end
//   z  += p'_lo + p'_hi  v_dot2c_f32 against (1, 1): z sums exactly the
//                        rounded weights the PV product uses
//   O^T += V^T * P^T     A = V^T read from the row-major V tile with
//                        ds_read_b64_tr_b16 (transpose on read), B = P^T
//                        straight from the S^T accumulator registers: the
//                        32x32 C layout gives each lane one query and 8 keys
//                        per 16-key chunk, which is the B layout up to a
//                        permutation of keys that the V^T read applies too.
// LDS rows are padded for the 32-bank LDS: K rows by 16 bytes (conflict-free
// 16-byte reads of 8 consecutive rows), V rows to 32 mod 128 bytes (the four
// rows a 16-lane transpose read touches fall in distinct banks).
// At the end each lane owns one query: z is completed with one cross-half
// shuffle, O = O^T / (z + eps / s^2), Z = s^2 z + eps.
//
// PUR: the purified-Born forward (flash_born.py:696-811) on the same tiles,
// as the fast kernels run it: p = relu(gamma (r - tau))^4 + eps_base relu(r)^2
// in fp32, Z = sum p + eps in fp32, masked pairs and keys past T weighing
// zero, each weight split into two bf16 terms for P.V (fp16 V split exactly
// into two bf16 terms, pur_pv), O = sum p v / Z written in fp32.  Used for the
// head dims above 128.
#pragma once

#include <type_traits>

#include "born_common.h"
#include "purified_args.h"

namespace qdl {

// ---------------------------------------------------------------------------
// 16-bit (bf16 / fp16) forward.
// ---------------------------------------------------------------------------
template <class E, int DP, int NQB, int NW, int BN, int MODE, int WPE, bool PUR = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void born_fwd16_kernel(typename std::conditional<PUR, PurArgs, FwdArgs>::type p) {
    static_assert(DP % 32 == 0 && DP <= 256, "padded head dim");
    static_assert(BN % 32 == 0, "key tile");
    constexpr int QW = 32 * NQB;
    constexpr int BM = NW * QW;
    constexpr int KS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int NT = NW * 64;
    constexpr int KSTR = DP + 8;   // K row stride in LDS (elements)
    constexpr int VSTR = DP + 16;  // V row stride in LDS (elements)
    constexpr int KCH = BN * DP / 8;          // 16-byte chunks per K or V tile
    constexpr int KPT = (KCH + NT - 1) / NT;
    constexpr bool kDoc = (MODE == kGeneral);

    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][BN * KSTR];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][BN * VSTR];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[kDoc ? 2 : 1][kDoc ? BN : 1];
    // Document-aware tile list (doc_ids given): candidate key tiles are
    // screened CAP at a time; a tile is kept when its [min, max] document id
    // range meets the workgroup's query range.  Exact skipping for sorted ids
    // (compute_document_ids output), conservative for any others.
    constexpr int CAP = kDoc ? 256 : 1;
    __shared__ int32_t t_keep[CAP];
    __shared__ int32_t t_list[CAP];
    __shared__ int2 t_rng[CAP];
    __shared__ int2 t_rng_c[CAP];
    __shared__ int32_t s_qrng[2 * NW];
    __shared__ int32_t s_count;

    const int T = p.T, D = p.D;
    const int BH = p.B * p.H;
    const int nmb = (T + BM - 1) / BM;
    const bool causal = (MODE == kCausal) || (MODE == kGeneral && p.is_causal);
    const int window = (MODE == kGeneral) ? p.window : 0;
    const bool has_doc = kDoc && p.doc != nullptr;

    // Heaviest query blocks first under causality; consecutive blocks share
    // nothing, blocks BH apart share (b, h) and, with BH a multiple of 8, land
    // on the same XCD.
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    const int mb = causal ? (nmb - 1 - bid / BH) : (bid / BH);
    const int b = bh / p.H, h = bh % p.H;
    const int m0 = mb * BM;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, g = lane >> 5;
    const int q0 = m0 + wave * QW;

    const size_t base = (size_t)bh * T * D;
    const uint16_t* __restrict__ Q = reinterpret_cast<const uint16_t*>(p.q) + base;
    const uint16_t* __restrict__ K = reinterpret_cast<const uint16_t*>(p.k) + base;
    const uint16_t* __restrict__ V = reinterpret_cast<const uint16_t*>(p.v) + base;
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;

    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (!PUR && sc < 0.f) ? 0x80008000u : 0u;  // sign of the scale folded into Q
    // fp16: the weights are the reference's relu(s r)^2 (c = |s| times the
    // sign-folded overlap; born_weight_pair); bf16: s^2 goes back in per row.
    const float sq_pre = E::kScaleInSquare ? fabsf(sc) : 1.f;
    // Purified weights: t = gamma r - gamma tau, b' = sqrt(eps_base) relu(r).
    float pg = 0.f, pgt = 0.f, pse = 0.f;
    if constexpr (PUR) {
        pg = sc;
        pgt = -sc * p.tau[p.per_head_tau ? h : 0];
        pse = sqrtf(p.eps_base);
    }

    // Q^T operand, resident for the whole kernel.
    u32x4 qr[NQB][KS];
    const bool q_full = (q0 + QW <= T) && (D == DP);
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const int row = q0 + qb * 32 + c;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + g * 8;
            u32x4 x = {0u, 0u, 0u, 0u};
            if (q_full || (row < T && d < D)) x = ldg16(Q + (size_t)row * D + d);
            x ^= flip;
            qr[qb][ks] = x;
        }
    }
    int qdoc[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const int row = q0 + qb * 32 + c;
        qdoc[qb] = (has_doc && row < T) ? docb[row] : -1;
    }
    // Document-id range of this wave's valid query rows, and of the workgroup's.
    int wq_lo = INT_MAX, wq_hi = INT_MIN, bq_lo = INT_MAX, bq_hi = INT_MIN;
    if (kDoc && has_doc) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            if (q0 + qb * 32 + c < T) {
                wq_lo = min(wq_lo, qdoc[qb]);
                wq_hi = max(wq_hi, qdoc[qb]);
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            wq_lo = min(wq_lo, __shfl_xor(wq_lo, off));
            wq_hi = max(wq_hi, __shfl_xor(wq_hi, off));
        }
        if (lane == 0) {
            s_qrng[2 * wave] = wq_lo;
            s_qrng[2 * wave + 1] = wq_hi;
        }
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            bq_lo = min(bq_lo, s_qrng[2 * w]);
            bq_hi = max(bq_hi, s_qrng[2 * w + 1]);
        }
    }

    // Key range of this workgroup (flash_born.py:152-154).
    int kv_lo = 0;
    int kv_hi = causal ? min(T, m0 + BM) : T;
    if (window > 0) kv_lo = max(0, m0 - window + 1) & ~(BN - 1);
    const int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + BN - 1) / BN : 0;

    // Staged tile in registers: 16-byte K and V row chunks, the tile's doc ids.
    struct Regs {
        u32x4 k[KPT];
        u32x4 v[KPT];
        int d;
    };
    // Interior tiles (all keys < T, D == DP) load without bounds checks.
    auto load_tile = [&](Regs& r, int key0) {
        const bool full = (key0 + BN <= T) && (D == DP);
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int idx = tid + i * NT;
            if (KCH % NT == 0 || idx < KCH) {
                const int row = idx / (DP / 8);
                const int col = (idx % (DP / 8)) * 8;
                const int key = key0 + row;
                u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
                if (full || (key < T && col < D)) {
                    x = ldg16(K + (size_t)key * D + col);
                    y = ldg16(V + (size_t)key * D + col);
                }
                r.k[i] = x;
                r.v[i] = y;
            }
        }
        if (kDoc && has_doc && tid < BN) {
            const int key = key0 + tid;
            r.d = key < T ? docb[key] : -2;
        }
    };
    auto store_tile = [&](const Regs& r, int buf) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int idx = tid + i * NT;
            if (KCH % NT == 0 || idx < KCH) {
                const int row = idx / (DP / 8);
                const int col = (idx % (DP / 8)) * 8;
                *reinterpret_cast<u32x4*>(&k_lds[buf][row * KSTR + col]) = r.k[i];
                *reinterpret_cast<u32x4*>(&v_lds[buf][row * VSTR + col]) = r.v[i];
            }
        }
        if (kDoc && has_doc && tid < BN) doc_lds[buf][tid] = r.d;
    };

    f32x16 oacc[DB][NQB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) oacc[db][qb] = zero16();
    float zacc[NQB][2];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) zacc[qb][0] = zacc[qb][1] = 0.f;

    auto compute = [&](int buf, int key0, int2 drng) {
        // Which of this wave's (query, key) pairs can be visible in the tile.
        bool active = q0 < T;
        if (kDoc && has_doc) active = active && drng.y >= wq_lo && drng.x <= wq_hi;
        // The document test is needed unless the tile's keys and the wave's
        // queries all belong to one and the same document.
        const bool doc_mask = kDoc && has_doc && !(drng.x == drng.y && wq_lo == wq_hi && drng.x == wq_lo);
        bool need_mask = doc_mask;
        if (causal) {
            active = active && (key0 <= q0 + QW - 1);
            need_mask = need_mask || (key0 + BN - 1 > q0);
        }
        if (window > 0) {
            active = active && (key0 + BN - 1 > q0 - window);
            need_mask = need_mask || (key0 <= q0 + QW - 1 - window);
        }
        // Purified: a key past T (zero K row) still weighs relu(-gamma tau)^4.
        if (PUR) need_mask = need_mask || (key0 + BN > T);
        if (!active) return;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            f32x16 s[NQB];
            uint32_t vis_bits[NQB];  // purified: bit r set for a visible register r
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) vis_bits[qb] = 0xffffu;
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) s[qb] = zero16();
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const u32x4 a = *reinterpret_cast<const u32x4*>(
                    &k_lds[buf][(nb * 32 + c) * KSTR + ks * 16 + g * 8]);
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) s[qb] = E::mfma(a, qr[qb][ks], s[qb]);
            }
            if (need_mask) {
                const int kbase = key0 + nb * 32 + 4 * g;
                // Document ids of this lane's 16 keys: 4 runs of 4 consecutive keys.
                int kd[16];
                if (kDoc && doc_mask) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int4 x = *reinterpret_cast<const int4*>(&doc_lds[buf][nb * 32 + 4 * g + 8 * j]);
                        kd[4 * j] = x.x;
                        kd[4 * j + 1] = x.y;
                        kd[4 * j + 2] = x.z;
                        kd[4 * j + 3] = x.w;
                    }
                }
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    // key = kbase + off(r); visible iff off(r) <= qi - kbase
                    // (causal) and off(r) > qi - kbase - window.
                    const int lim = q0 + qb * 32 + c - kbase;
                    const int hi = causal ? lim : (PUR ? T - 1 - kbase : INT_MAX);
                    const int lo = window > 0 ? lim - window : INT_MIN;
                    uint32_t bits = 0;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int off = 8 * (r >> 2) + (r & 3);
                        bool vis = (off <= hi) && (off > lo);
                        if (kDoc && doc_mask) vis = vis && (kd[r] == qdoc[qb]);
                        if constexpr (PUR)
                            bits |= vis ? (1u << r) : 0u;
                        else if (!vis)
                            s[qb][r] = 0.f;
                    }
                    vis_bits[qb] = bits;
                }
            }
            uint32_t pk[NQB][8];
            uint32_t pl[NQB][PUR ? 8 : 1];
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if constexpr (PUR) {
                        float w[2];
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const float x = s[qb][2 * j + e];
                            const float u = relu_f32(fmaf(x, pg, pgt));
                            const float bq = relu_f32(x * pse);
                            const float u2 = u * u;
                            const float pw = fmaf(u2, u2, bq * bq);
                            w[e] = ((vis_bits[qb] >> (2 * j + e)) & 1u) ? pw : 0.f;
                        }
                        zacc[qb][0] += w[0] + w[1];
                        const uint32_t hi = BF16::pack(w[0], w[1]);
                        pk[qb][j] = hi;
                        pl[qb][j] = BF16::pack(w[0] - BF16::lo(hi), w[1] - BF16::hi(hi));
                    } else {
                        pk[qb][j] = born_weight_pair<E>(s[qb][2 * j], s[qb][2 * j + 1], sq_pre, zacc[qb][j & 1]);
                    }
                }
            }
            // V^T operand of the 16-key chunk (nb, hh): lane group G = lane / 16
            // reads rows key + 4 (G / 2) + i / 4 (and +8), columns
            // 16 (G % 2) + 4 (i % 4) of each 32-wide d block.
            const int vr = nb * 32 + 4 * (lane >> 5) + ((lane & 15) >> 2);
            const int vc = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const uint16_t* vp = &v_lds[buf][(vr + hh * 16) * VSTR + db * 32 + vc];
                    const u32x2 lo = lds_read_tr16(vp);
                    const u32x2 hi = lds_read_tr16(vp + 8 * VSTR);
                    const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                    for (int qb = 0; qb < NQB; ++qb) {
                        const u32x4 bq = {pk[qb][4 * hh], pk[qb][4 * hh + 1], pk[qb][4 * hh + 2],
                                          pk[qb][4 * hh + 3]};
                        if constexpr (PUR) {
                            const u32x4 bl = {pl[qb][4 * hh], pl[qb][4 * hh + 1], pl[qb][4 * hh + 2],
                                              pl[qb][4 * hh + 3]};
                            oacc[db][qb] = pur_pv<E>(a, bq, bl, oacc[db][qb]);
                        } else {
                            oacc[db][qb] = E::mfma(a, bq, oacc[db][qb]);
                        }
                    }
                }
            }
        }
    };

    // Screen candidate tiles c0 .. c0+nc-1 (document ids given): one tile per
    // thread, its ids read as 16-byte vectors when aligned (all loads of a
    // thread independent, so a screening pass costs about one memory
    // latency); then wave 0 compacts the kept tiles into t_list.
    static_assert(!kDoc || CAP == NT, "one candidate tile per thread");
    const bool doc_vec = kDoc && has_doc && ((reinterpret_cast<uintptr_t>(docb) & 15) == 0);
    auto screen = [&](int c0, int nc) -> int {
        if (tid < nc) {
            const int key0 = kv_lo + (c0 + tid) * BN;
            const int kend = min(key0 + BN, T);
            int lo = INT_MAX, hi = INT_MIN;
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
            t_rng[tid] = make_int2(lo, hi);
            t_keep[tid] = (hi >= bq_lo && lo <= bq_hi) ? 1 : 0;
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
                    t_rng_c[pos] = t_rng[i];
                }
                count += __popcll(m);
            }
            if (lane == 0) s_count = count;
        }
        __syncthreads();
        return s_count;
    };
    const bool listed = kDoc && has_doc;
    auto tile_key = [&](int t) -> int { return kv_lo + (listed ? t_list[t] : t) * BN; };
    auto tile_rng = [&](int t) -> int2 { return listed ? t_rng_c[t] : make_int2(0, 0); };

    // Software pipeline, prefetch distance 2: while tile t is consumed from
    // LDS buffer t%2, register set (t+1)%2 holds tile t+1 and tile t+2 is in
    // flight into the other set; each load has two tiles of compute to land.
    // With a tile list the pipeline runs once per screened chunk.
    const int chunk = listed ? CAP : max(ntiles, 1);
    for (int c0 = 0; c0 < ntiles; c0 += chunk) {
        const int n = listed ? screen(c0, min(CAP, ntiles - c0)) : ntiles;
        Regs ra, rb;
        if (n > 0) {
            load_tile(ra, tile_key(0));
            store_tile(ra, 0);
        }
        if (n > 1) load_tile(rb, tile_key(1));
        __syncthreads();
        for (int t = 0; t < n; t += 2) {
            if (t + 2 < n) load_tile(ra, tile_key(t + 2));
            compute(0, tile_key(t), tile_rng(t));
            if (t + 1 < n) store_tile(rb, 1);
            __syncthreads();
            if (t + 1 >= n) break;
            if (t + 3 < n) load_tile(rb, tile_key(t + 3));
            compute(1, tile_key(t + 1), tile_rng(t + 1));
            if (t + 2 < n) store_tile(ra, 0);
            __syncthreads();
        }
    }

    // Epilogue: one query per lane.
    float* __restrict__ Zp = p.z + (size_t)bh * T;
    if constexpr (PUR) {
        // O = acc / (Z + eps) and Z + eps in fp32.
        float* __restrict__ O32 = p.o + base;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const float zl = zacc[qb][0] + zacc[qb][1];
            const float zd = zl + __shfl_xor(zl, 32) + p.eps;
            const int qi = q0 + qb * 32 + c;
            if (qi < T) {
#pragma unroll
                for (int db = 0; db < DB; ++db) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int d = db * 32 + 8 * j + 4 * g;
                        if (d < D) {
                            const f32x16& o = oacc[db][qb];
                            const f32x4 w = {o[4 * j] / zd, o[4 * j + 1] / zd, o[4 * j + 2] / zd, o[4 * j + 3] / zd};
                            *reinterpret_cast<f32x4*>(O32 + (size_t)qi * D + d) = w;
                        }
                    }
                }
                if (g == 0) Zp[qi] = zd;
            }
        }
        return;
    }
    uint16_t* __restrict__ O = reinterpret_cast<uint16_t*>(p.o) + base;
    const float s2 = (sq_pre > 0.f) ? (sc / sq_pre) * (sc / sq_pre) : 0.f;
    const float eps_s = (p.eps == 0.f) ? 0.f : p.eps / s2;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const float zl = zacc[qb][0] + zacc[qb][1];
        const float zt = zl + __shfl_xor(zl, 32);
        const float rcp = 1.0f / (zt + eps_s);
        const int qi = q0 + qb * 32 + c;
        if (qi < T) {
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int d = db * 32 + 8 * j + 4 * g;
                    if (d < D) {
                        const f32x16& o = oacc[db][qb];
                        u32x2 w;
                        w[0] = E::pack(o[4 * j] * rcp, o[4 * j + 1] * rcp);
                        w[1] = E::pack(o[4 * j + 2] * rcp, o[4 * j + 3] * rcp);
                        *reinterpret_cast<u32x2*>(O + (size_t)qi * D + d) = w;
                    }
                }
            }
            if (g == 0) Zp[qi] = s2 * zt + p.eps;
        }
    }
}

// ---------------------------------------------------------------------------
// fp32 forward: v_mfma_f32_32x32x2_f32, no reduced-precision operands
// (the reference runs its fp32 dots with allow_tf32=False).
// ---------------------------------------------------------------------------
template <int DP, int NW, int BN, int MODE, int WPE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void born_fwd32_kernel(FwdArgs p) {
    static_assert(DP % 32 == 0 && DP <= 256, "padded head dim");
    constexpr int QW = 32;
    constexpr int BM = NW * QW;
    constexpr int KQ = DP / 8;     // float4 pairs of contraction steps
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int NT = NW * 64;
    constexpr int KSTR = DP + 4;   // floats
    constexpr int VSTR = DP + 4;
    constexpr int CH = BN * DP / 4;    // 16-byte chunks per tile
    constexpr int CPT = (CH + NT - 1) / NT;
    constexpr bool kDoc = (MODE == kGeneral);

    __shared__ __attribute__((aligned(16))) float k_lds[2][BN * KSTR];
    __shared__ __attribute__((aligned(16))) float v_lds[2][BN * VSTR];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[kDoc ? 2 : 1][kDoc ? BN : 1];

    const int T = p.T, D = p.D;
    const int BH = p.B * p.H;
    const int nmb = (T + BM - 1) / BM;
    const bool causal = (MODE == kCausal) || (MODE == kGeneral && p.is_causal);
    const int window = (MODE == kGeneral) ? p.window : 0;
    const bool has_doc = kDoc && p.doc != nullptr;

    const int bid = blockIdx.x;
    const int bh = bid % BH;
    const int mb = causal ? (nmb - 1 - bid / BH) : (bid / BH);
    const int b = bh / p.H, h = bh % p.H;
    const int m0 = mb * BM;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, g = lane >> 5;
    const int q0 = m0 + wave * QW;

    const size_t base = (size_t)bh * T * D;
    const float* __restrict__ Q = reinterpret_cast<const float*>(p.q) + base;
    const float* __restrict__ K = reinterpret_cast<const float*>(p.k) + base;
    const float* __restrict__ V = reinterpret_cast<const float*>(p.v) + base;
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;

    const float sc = p.scale[p.per_head_scale ? h : 0];
    const float sgn = (sc < 0.f) ? -1.f : 1.f;

    // Contraction step t of the QK product uses dim 8*(t/4) + 4*g + (t%4), so
    // each lane reads 4 consecutive dims at once.
    f32x4 qr[KQ];
    {
        const int row = q0 + c;
#pragma unroll
        for (int u = 0; u < KQ; ++u) {
            const int d = 8 * u + 4 * g;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if (row < T && d < D) x = *reinterpret_cast<const f32x4*>(Q + (size_t)row * D + d);
            qr[u] = x * sgn;
        }
    }
    const int qi = q0 + c;
    const int qdoc = (has_doc && qi < T) ? docb[qi] : -1;

    int kv_lo = 0;
    int kv_hi = causal ? min(T, m0 + BM) : T;
    if (window > 0) kv_lo = max(0, m0 - window + 1) & ~(BN - 1);
    const int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + BN - 1) / BN : 0;

    f32x4 kreg[CPT], vreg[CPT];
    int dreg = -2;
    auto load_tile = [&](int key0) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int row = idx / (DP / 4);
                const int col = (idx % (DP / 4)) * 4;
                const int key = key0 + row;
                f32x4 xk = {0.f, 0.f, 0.f, 0.f}, xv = {0.f, 0.f, 0.f, 0.f};
                if (key < T && col < D) {
                    xk = *reinterpret_cast<const f32x4*>(K + (size_t)key * D + col);
                    xv = *reinterpret_cast<const f32x4*>(V + (size_t)key * D + col);
                }
                kreg[i] = xk;
                vreg[i] = xv;
            }
        }
        if (kDoc && has_doc && tid < BN) {
            const int key = key0 + tid;
            dreg = key < T ? docb[key] : -2;
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int row = idx / (DP / 4);
                const int col = (idx % (DP / 4)) * 4;
                *reinterpret_cast<f32x4*>(&k_lds[buf][row * KSTR + col]) = kreg[i];
                *reinterpret_cast<f32x4*>(&v_lds[buf][row * VSTR + col]) = vreg[i];
            }
        }
        if (kDoc && has_doc && tid < BN) doc_lds[buf][tid] = dreg;
    };

    f32x16 oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = zero16();
    float zacc = 0.f;

    if (ntiles > 0) {
        load_tile(kv_lo);
        store_tile(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int key0 = kv_lo + t * BN;
        const int buf = t & 1;
        const bool more = (t + 1) < ntiles;
        if (more) load_tile(key0 + BN);

        bool active = q0 < T;
        bool need_mask = has_doc;
        if (causal) {
            active = active && (key0 <= q0 + QW - 1);
            need_mask = need_mask || (key0 + BN - 1 > q0);
        }
        if (window > 0) {
            active = active && (key0 + BN - 1 > q0 - window);
            need_mask = need_mask || (key0 <= q0 + QW - 1 - window);
        }
        if (active) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                f32x16 s = zero16();
#pragma unroll
                for (int u = 0; u < KQ; ++u) {
                    const f32x4 a = *reinterpret_cast<const f32x4*>(
                        &k_lds[buf][(nb * 32 + c) * KSTR + 8 * u + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) s = mfma_f32(a[e], qr[u][e], s);
                }
                if (need_mask) {
                    const int kbase = key0 + nb * 32 + 4 * g;
                    const int lim = qi - kbase;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int off = 8 * (r >> 2) + (r & 3);
                        bool vis = true;
                        if (causal) vis = vis && (off <= lim);
                        if (window > 0) vis = vis && (off > lim - window);
                        if (kDoc && has_doc) vis = vis && (doc_lds[buf][kbase - key0 + off] == qdoc);
                        if (!vis) s[r] = 0.f;
                    }
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float x = fmaxf(s[r], 0.f);
                    const float pr = x * x;
                    zacc += pr;
                    s[r] = pr;
                }
                // O^T += V^T P^T: step r contracts key acc_row(r, g) of this block.
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int krow = nb * 32 + acc_row(r, g);
#pragma unroll
                    for (int db = 0; db < DB; ++db)
                        oacc[db] = mfma_f32(v_lds[buf][krow * VSTR + db * 32 + c], s[r], oacc[db]);
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    float* __restrict__ O = reinterpret_cast<float*>(p.o) + base;
    float* __restrict__ Zp = p.z + (size_t)bh * T;
    const float s2 = sc * sc;
    const float eps_s = (p.eps == 0.f) ? 0.f : p.eps / s2;
    const float zt = zacc + __shfl_xor(zacc, 32);
    const float rcp = 1.0f / (zt + eps_s);
    if (qi < T) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = db * 32 + 8 * j + 4 * g;
                if (d < D) {
                    f32x4 w = {oacc[db][4 * j] * rcp, oacc[db][4 * j + 1] * rcp,
                               oacc[db][4 * j + 2] * rcp, oacc[db][4 * j + 3] * rcp};
                    *reinterpret_cast<f32x4*>(O + (size_t)qi * D + d) = w;
                }
            }
        }
        if (g == 0) Zp[qi] = s2 * zt + p.eps;
    }
}

// Tile configuration per padded head dim (16-bit inputs).  The D <= 64
// configuration can be overridden at build time (QDL_FWD64_*) for tuning.
#ifndef QDL_FWD64_NQB
#define QDL_FWD64_NQB 2
#endif
#ifndef QDL_FWD64_NW
#define QDL_FWD64_NW 4
#endif
#ifndef QDL_FWD64_BN
#define QDL_FWD64_BN 64
#endif
#ifndef QDL_FWD64_WPE
#define QDL_FWD64_WPE 2
#endif
template <int DP>
struct Fwd16Cfg {
    static constexpr int NQB = DP <= 64 ? QDL_FWD64_NQB : 1;
    static constexpr int NW = DP <= 64 ? QDL_FWD64_NW : 4;
    static constexpr int BN = DP <= 64 ? QDL_FWD64_BN : (DP <= 128 ? 64 : 32);
    static constexpr int WPE = DP <= 64 ? QDL_FWD64_WPE : (DP <= 128 ? 2 : 1);
    static constexpr int BM = NW * 32 * NQB;
};

template <int DP>
struct Fwd32Cfg {
    static constexpr int NW = 4;
    static constexpr int BN = 32;
    static constexpr int WPE = DP <= 128 ? 2 : 1;
    static constexpr int BM = NW * 32;
};

template <class E, int DP, int MODE>
hipError_t launch_fwd16(const FwdArgs& a, hipStream_t st) {
    using C = Fwd16Cfg<DP>;
    const int nmb = (a.T + C::BM - 1) / C::BM;
    const dim3 grid((unsigned)nmb * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd16_kernel<E, DP, C::NQB, C::NW, C::BN, MODE, C::WPE>), grid,
                       dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

// 128 < D <= 256 (documents with a causal window or none), 16-bit inputs:
// the DMA-ring kernel of born_fwd_d256.h (instantiated in born_fwd_d256.hip).
template <class E>
hipError_t launch_fwd16_wide(const FwdArgs& a, hipStream_t st);

template <int DP, int MODE>
hipError_t launch_fwd32(const FwdArgs& a, hipStream_t st) {
    using C = Fwd32Cfg<DP>;
    const int nmb = (a.T + C::BM - 1) / C::BM;
    const dim3 grid((unsigned)nmb * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((born_fwd32_kernel<DP, C::NW, C::BN, MODE, C::WPE>), grid, dim3(C::NW * 64),
                       0, st, a);
    return hipGetLastError();
}

}  // namespace qdl
