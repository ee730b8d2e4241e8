// Flash-Born backward kernels for gfx950.
//
// Replaces the reference's `_flash_born_bwd_kernel` (dK, dV, dscale) and
// `_flash_born_bwd_dq_kernel` (src/qdlblocks/kernels/flash_born.py:195-430).
//
// With Z_i = sum_j p_ij + eps, delta_i = dO_i . O_i and s the (per-head) scale:
//   dP_ij = (dO_i . v_j - delta_i) / Z_i
//   dS_ij = 2 a_ij dP_ij,   a_ij = |s| relu(r'_ij),  r' = sign(s) q . k
//   dq_i  = s sum_j dS_ij k_j = 2 s|s| sum_j relu(r'_ij) dP_ij k_j
//   dk_j  = s sum_i dS_ij q_i = 2 s|s| sum_i relu(r'_ij) dP_ij q_i
//   dv_j  = sum_i p_ij / Z_i dO_i = s^2 sum_i relu(r'_ij)^2 / Z_i dO_i
//   dscale = sum dS_ij r_ij = (2/s) sum_ij p_ij dP_ij = (2/s) eps sum_i delta_i / Z_i
// delta is taken from the stored forward output O, as the reference does
// (flash_born.py:277, 302).  dO . v_j - delta_i cancels strongly in rows with
// few visible keys, and 2 a dP / Z amplifies it by 1/a there, so it is always
// formed in fp32 from the unscaled bf16/fp16 dO (the dP accumulator starts at
// -delta_i) before 1/Z_i is applied.
// The last identity (sum_j p_ij dP_ij = delta_i eps / Z_i) makes dscale a
// per-row closed form, reduced in a fixed order: deterministic, and free of
// the cancellation of an O(T^2) sum whose true value is O(eps).
//
// Launch sequence: delta pre-pass (delta and delta / Z per row) -> dK/dV
// kernel (keys stationary in registers, query tiles of Q and dO staged in LDS
// in row and transposed layouts) -> dQ kernel (queries stationary, K staged in
// both layouts, V row-major) -> dscale reduction.
#pragma once

#include "born_bwd_d128.h"
#include "born_bwd_fast.h"
#include "born_common.h"
#include "born_stage.h"

namespace qdl {

// ---------------------------------------------------------------------------
// Pre-pass: -delta_i = -(dO_i . O_i), delta_i / Z_i and 1 / Z_i, one group of
// G lanes per row.
// ---------------------------------------------------------------------------
template <class E, bool F32>
__global__ __launch_bounds__(256) void born_bwd_delta_kernel(BwdArgs p, int G) {
    const int per_block = 256 / G;
    const int64_t nrows = (int64_t)p.B * p.H * p.T;
    const int64_t row = (int64_t)blockIdx.x * per_block + threadIdx.x / G;
    const int sub = threadIdx.x % G;
    const int D = p.D;
    float acc = 0.f;
    if (row < nrows) {
        if constexpr (F32) {
            const float* o = reinterpret_cast<const float*>(p.o) + row * D;
            const float* d = reinterpret_cast<const float*>(p.dout) + row * D;
            for (int c = sub * 4; c < D; c += G * 4) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(o + c);
                const f32x4 b = *reinterpret_cast<const f32x4*>(d + c);
                acc += a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
            }
        } else {
            const uint16_t* o = reinterpret_cast<const uint16_t*>(p.o) + row * D;
            const uint16_t* d = reinterpret_cast<const uint16_t*>(p.dout) + row * D;
            for (int c = sub * 8; c < D; c += G * 8) {
                const u32x4 a = ldg16(o + c);
                const u32x4 b = ldg16(d + c);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc += E::lo(a[j]) * E::lo(b[j]) + E::hi(a[j]) * E::hi(b[j]);
            }
        }
    }
    for (int off = G >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (row < nrows && sub == 0) {
        const float zi = 1.0f / p.z[row];
        p.ndelta[row] = -acc;
        p.delta_z[row] = acc / p.z[row];
        p.zinv[row] = zi;
    }
}

// Visibility of (query i, key j) under the kernel's mask mode.
template <int MODE>
__device__ __forceinline__ bool visible(int i, int j, bool causal, int window, bool has_doc, int doc_i,
                                        int doc_j) {
    bool v = true;
    if (causal) v = v && (j <= i);
    if (MODE == kGeneral) {
        if (window > 0) v = v && (i - j < window);
        if (has_doc) v = v && (doc_i == doc_j);
    }
    return v;
}

// ---------------------------------------------------------------------------
// dQ, 16-bit.  Queries stationary (like the forward).  Per key tile and wave:
//   S^T  = K Q'^T          (A = K rows from LDS, B = sign-flipped Q^T in registers)
//   dP^T = V dO^T          (A = V rows from LDS, B = dO^T in registers)
//   u    = relu(S^T) * (dP^T / Z_i - delta'_i)   one query per lane
//   dQ^T += K^T u          (A = K^T from the transposed LDS copy, B = u from
//                           the accumulator registers, as P in the forward)
// PUR: the purified gradient (flash_born.py:1035-1058) in place of u:
// dR = (4 gamma u^3 + 2 eps_base b) dP / Z with u = relu(gamma (r - tau)),
// b = relu(r), zero where masked, rounded to the input dtype as the
// reference's .to(k.dtype); -delta and 1/Z come from the workspace.
// ---------------------------------------------------------------------------
template <class E, int DP, int NQB, int NW, int BN, int MODE, int WPE, bool PUR = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void born_bwd_dq16_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    constexpr int QW = 32 * NQB;
    constexpr int BM = NW * QW;
    constexpr int KS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int NT = NW * 64;
    constexpr int RS = DP + 8;
    constexpr int TS = BN + 4;
    constexpr bool kDoc = (MODE == kGeneral);
    using KStage = PairStager<BN, DP, NT>;
    using VStage = RowStager<BN, DP, NT>;

    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) uint16_t kt_lds[2][DP * TS];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[kDoc ? 2 : 1][kDoc ? BN : 1];
    __shared__ int32_t span_red[kDoc ? 4 : 1];

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
    const uint16_t* __restrict__ Q = reinterpret_cast<const uint16_t*>(p.q) + base;
    const uint16_t* __restrict__ K = reinterpret_cast<const uint16_t*>(p.k) + base;
    const uint16_t* __restrict__ V = reinterpret_cast<const uint16_t*>(p.v) + base;
    const uint16_t* __restrict__ dO = reinterpret_cast<const uint16_t*>(p.dout) + base;
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;

    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (!PUR && sc < 0.f) ? 0x80008000u : 0u;
    // fp16 scales the overlap by c = 2|s|, so the dS operand is the
    // reference's 2 a dP (see E::kScaleInSquare); the epilogue divides c out.
    const float sq_pre = (E::kScaleInSquare && sc != 0.f) ? 2.f * fabsf(sc) : 1.f;
    auto pre = [&](float x) __attribute__((always_inline)) {
        if constexpr (E::kScaleInSquare) return x * sq_pre;
        else return x;
    };
    float pg = 0.f, pgt = 0.f, p4g = 0.f, p2e = 0.f;
    if constexpr (PUR) {
        pg = sc;
        pgt = -sc * p.tau[p.per_head_tau ? h : 0];
        p4g = 4.f * sc;
        p2e = 2.f * p.eps_base;
    }

    u32x4 qr[NQB][KS], dr[NQB][KS];
    float zinv[NQB], nd[NQB];
    int qdoc[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const int row = q0 + qb * 32 + c;
        const bool ok = row < T;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + g * 8;
            u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
            if (ok && d < D) {
                x = ldg16(Q + (size_t)row * D + d);
                y = ldg16(dO + (size_t)row * D + d);
            }
            qr[qb][ks] = x ^ flip;
            dr[qb][ks] = y;
        }
        if constexpr (PUR) {
            zinv[qb] = ok ? p.zinv[(size_t)bh * T + row] : 0.f;
            nd[qb] = ok ? p.ndelta[(size_t)bh * T + row] * zinv[qb] : 0.f;
        } else {
            zinv[qb] = ok ? 1.0f / p.z[(size_t)bh * T + row] : 0.f;
            nd[qb] = ok ? -p.delta_z[(size_t)bh * T + row] : 0.f;
        }
        qdoc[qb] = (has_doc && ok) ? docb[row] : -1;
    }

    int kv_lo = 0;
    int kv_hi = causal ? min(T, m0 + BM) : T;
    if (window > 0) kv_lo = max(0, m0 - window + 1) & ~(BN - 1);
    int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + BN - 1) / BN : 0;

    KStage kst;
    VStage vst;
    int dreg = -2;
    auto load_tile = [&](int key0) {
        kst.template load<E>(K, key0, T, D, tid);
        vst.load(V, key0, T, D, tid);
        if (kDoc && has_doc && tid < BN) dreg = (key0 + tid < T) ? docb[key0 + tid] : -2;
    };
    auto store_tile = [&](int buf) {
        kst.template store_rows<RS>(k_lds[buf], tid);
        kst.template store_trans<TS>(kt_lds[buf], tid);
        vst.template store_rows<RS>(v_lds[buf], tid);
        if (kDoc && has_doc && tid < BN) doc_lds[buf][tid] = dreg;
    };

    f32x16 acc[DB][NQB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) acc[db][qb] = zero16();

    // Documents: visit only the span of key tiles whose ids meet the block's
    // rows'.  Under causality the span ends at the block's diagonal tile (its
    // last row sees its own key): the span is walked from there downwards,
    // so the first tile's loads go out before the screening and overlap it.
    int kstep = BN;
    bool first_issued = false;
    if constexpr (kDoc) {
        if (has_doc && ntiles > 0) {
            const int t_top = kv_lo / BN + ntiles - 1;
            if (causal) {
                load_tile(t_top * BN);
                first_issued = true;
            }
            const int2 sp = doc_tile_span<BN>(docb, T, m0, min(T, m0 + BM), kv_lo / BN, t_top, span_red);
            if (causal) {
                ntiles = sp.x <= sp.y ? t_top - sp.x + 1 : 0;
                kv_lo = t_top * BN;
                kstep = -BN;
            } else {
                ntiles = sp.x <= sp.y ? sp.y - sp.x + 1 : 0;
                if (ntiles > 0) kv_lo = sp.x * BN;
            }
        }
    }
    if (ntiles > 0) {
        if (!first_issued) load_tile(kv_lo);
        store_tile(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int key0 = kv_lo + t * kstep;
        const int buf = t & 1;
        const bool more = (t + 1) < ntiles;
        if (more) load_tile(key0 + kstep);

        bool active = q0 < T;
        bool need_mask = false;
        if constexpr (kDoc) need_mask = has_doc && !one_document(doc_lds[buf], BN, qdoc[0], qdoc[NQB - 1]);
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
                f32x16 s[NQB], tt[NQB];
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    s[qb] = zero16();
                    tt[qb] = zero16();
                }
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const u32x4 ak = *reinterpret_cast<const u32x4*>(
                        &k_lds[buf][(nb * 32 + c) * RS + ks * 16 + g * 8]);
                    const u32x4 av = *reinterpret_cast<const u32x4*>(
                        &v_lds[buf][(nb * 32 + c) * RS + ks * 16 + g * 8]);
#pragma unroll
                    for (int qb = 0; qb < NQB; ++qb) {
                        s[qb] = E::mfma(ak, qr[qb][ks], s[qb]);
                        tt[qb] = E::mfma(av, dr[qb][ks], tt[qb]);
                    }
                }
                uint32_t vis_bits[NQB];  // purified: bit r set for a visible register r
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) vis_bits[qb] = 0xffffu;
                if (need_mask) {
                    const int kbase = key0 + nb * 32 + 4 * g;
#pragma unroll
                    for (int qb = 0; qb < NQB; ++qb) {
                        const int qi = q0 + qb * 32 + c;
                        uint32_t bits = 0;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int key = kbase + 8 * (r >> 2) + (r & 3);
                            const int kd = (kDoc && has_doc) ? doc_lds[buf][key - key0] : 0;
                            const bool vis = visible<MODE>(qi, key, causal, window, has_doc, qdoc[qb], kd);
                            if constexpr (PUR)
                                bits |= vis ? (1u << r) : 0u;
                            else if (!vis)
                                s[qb][r] = 0.f;
                        }
                        vis_bits[qb] = bits;
                    }
                }
                uint32_t pk[NQB][8];
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if constexpr (PUR) {
                            // A masked pair weighs zero even where its overlap is zero.
                            float w[2];
#pragma unroll
                            for (int e = 0; e < 2; ++e) {
                                const int r = 2 * j + e;
                                const float x = s[qb][r];
                                const float u = relu_f32(fmaf(x, pg, pgt));
                                const float f = fmaf(p4g, u * u * u, p2e * relu_f32(x));
                                const float d = f * fmaf(tt[qb][r], zinv[qb], nd[qb]);
                                w[e] = ((vis_bits[qb] >> r) & 1u) ? d : 0.f;
                            }
                            pk[qb][j] = E::pack(w[0], w[1]);
                        } else {
                            const float u0 = fmaxf(pre(s[qb][2 * j]), 0.f) * fmaf(tt[qb][2 * j], zinv[qb], nd[qb]);
                            const float u1 =
                                fmaxf(pre(s[qb][2 * j + 1]), 0.f) * fmaf(tt[qb][2 * j + 1], zinv[qb], nd[qb]);
                            pk[qb][j] = E::pack(u0, u1);
                        }
                    }
                }
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        const uint16_t* kr =
                            &kt_lds[buf][(db * 32 + c) * TS + nb * 32 + hh * 16 + g * 4];
                        const u32x2 lo = *reinterpret_cast<const u32x2*>(kr);
                        const u32x2 hi = *reinterpret_cast<const u32x2*>(kr + 8);
                        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                        for (int qb = 0; qb < NQB; ++qb) {
                            const u32x4 bq = {pk[qb][4 * hh], pk[qb][4 * hh + 1], pk[qb][4 * hh + 2],
                                              pk[qb][4 * hh + 3]};
                            acc[db][qb] = E::mfma(a, bq, acc[db][qb]);
                        }
                    }
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    uint16_t* __restrict__ dQ = reinterpret_cast<uint16_t*>(p.dq) + base;
    const float f = PUR ? 1.f : E::kScaleInSquare ? sc : 2.f * sc * fabsf(sc);
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const int qi = q0 + qb * 32 + c;
        if (qi < T) {
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int d = db * 32 + 8 * j + 4 * g;
                    if (d < D) {
                        const f32x16& o = acc[db][qb];
                        u32x2 w;
                        w[0] = E::pack(o[4 * j] * f, o[4 * j + 1] * f);
                        w[1] = E::pack(o[4 * j + 2] * f, o[4 * j + 3] * f);
                        *reinterpret_cast<u32x2*>(dQ + (size_t)qi * D + d) = w;
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dK / dV, 16-bit.  Keys stationary: each wave owns 32 keys, their K (sign
// flipped) and V rows held in registers as MFMA B operands.  Query tiles of
// BQ rows stream through LDS: Q and dO, each in row-major and transposed
// copies, plus -delta and 1/Z per query.  Per tile and wave:
//   S   = Q K'^T          (C layout: one key per lane, 16 queries per block)
//   dPz = dO V^T - delta  (accumulator initialised with -delta)
//   t = relu(S) / Z_i;  dV^T += dO^T (t relu(S)),  dK^T += Q^T (t dPz)
// CS column splits: with CS == 2 two workgroups share a key block, each
// forming S and dPz over the whole head dim but accumulating dK, dV for half
// of its columns (the wide head dims' full accumulators and stationary rows
// exceed even one wave's 512 registers).
// PUR: the purified gradients (flash_born.py:896-947): W = p / Z and
// dR = (4 gamma u^3 + 2 eps_base b) dP / Z, each rounded to the input dtype
// as the reference does, zero where masked; each key block's first column
// split also writes its partial sums of dgamma = 4 sum u^3 dP (r - tau) and
// dtau = -4 gamma sum u^3 dP (keys past T left out), reduced per output in a
// fixed order afterwards.
// ---------------------------------------------------------------------------
template <class E, int DP, int NW, int BQ, int MODE, int WPE, int CS = 1, bool PUR = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void born_bwd_dkdv16_kernel(typename std::conditional<PUR, PurArgs, BwdArgs>::type p) {
    constexpr int BK = NW * 32;
    constexpr int KS = DP / 16;
    constexpr int DBF = DP / 32;                // column blocks of the head dim
    constexpr int DB = (DBF + CS - 1) / CS;     // column blocks accumulated here (at most)
    constexpr int NQ = BQ / 32;
    constexpr int NT = NW * 64;
    constexpr int RS = DP + 8;
    constexpr int TS = BQ + 4;
    constexpr bool kDoc = (MODE == kGeneral);
    using Stage = PairStager<BQ, DP, NT>;

    __shared__ __attribute__((aligned(16))) uint16_t q_lds[2][BQ * RS];
    __shared__ __attribute__((aligned(16))) uint16_t qt_lds[2][DP * TS];
    __shared__ __attribute__((aligned(16))) uint16_t d_lds[2][BQ * RS];
    __shared__ __attribute__((aligned(16))) uint16_t dt_lds[2][DP * TS];
    __shared__ __attribute__((aligned(16))) float nd_lds[2][BQ];
    __shared__ __attribute__((aligned(16))) float zi_lds[2][BQ];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[kDoc ? 2 : 1][kDoc ? BQ : 1];
    __shared__ int32_t span_red[kDoc ? 4 : 1];

    const int T = p.T, D = p.D;
    const int BH = p.B * p.H;
    const bool causal = (MODE == kCausal) || (MODE == kGeneral && p.is_causal);
    const int window = (MODE == kGeneral) ? p.window : 0;
    const bool has_doc = kDoc && p.doc != nullptr;

    // Key blocks in ascending order: under causality the first sees the most
    // queries.  Column split: workgroups bid and bid + 1 share a key block.
    const int cs = (CS > 1) ? (int)(blockIdx.x % CS) : 0;
    const int bid = blockIdx.x / CS;
    const int bh = bid % BH;
    const int kb = bid / BH;
    const int db0 = cs * DB;  // first column block accumulated here
    const int b = bh / p.H, h = bh % p.H;
    const int k0 = kb * BK;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, g = lane >> 5;
    const int kw0 = k0 + wave * 32;
    const int key = kw0 + c;

    const size_t base = (size_t)bh * T * D;
    const uint16_t* __restrict__ Q = reinterpret_cast<const uint16_t*>(p.q) + base;
    const uint16_t* __restrict__ K = reinterpret_cast<const uint16_t*>(p.k) + base;
    const uint16_t* __restrict__ V = reinterpret_cast<const uint16_t*>(p.v) + base;
    const uint16_t* __restrict__ dO = reinterpret_cast<const uint16_t*>(p.dout) + base;
    const float* __restrict__ NDl = p.ndelta + (size_t)bh * T;
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;

    const float sc = p.scale[p.per_head_scale ? h : 0];
    const uint32_t flip = (!PUR && sc < 0.f) ? 0x80008000u : 0u;
    // fp16 scales the overlap by c = 2|s|, so the dS operand is the
    // reference's 2 a dP (see E::kScaleInSquare); the epilogue divides c out.
    const float sq_pre = (E::kScaleInSquare && sc != 0.f) ? 2.f * fabsf(sc) : 1.f;
    auto pre = [&](float x) __attribute__((always_inline)) {
        if constexpr (E::kScaleInSquare) return x * sq_pre;
        else return x;
    };
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

    u32x4 kr[KS], vr[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d = ks * 16 + g * 8;
        u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
        if (key < T && d < D) {
            x = ldg16(K + (size_t)key * D + d);
            y = ldg16(V + (size_t)key * D + d);
        }
        kr[ks] = x ^ flip;
        vr[ks] = y;
    }
    const int kdoc = (has_doc && key < T) ? docb[key] : -2;

    // Query range (flash_born.py:264-265): causal starts at the block's first
    // key; a window ends W past its last key.
    int q_lo = causal ? (k0 & ~(BQ - 1)) : 0;
    int q_hi = T;
    if (window > 0) q_hi = min(T, k0 + BK - 1 + window);
    int ntiles = (q_hi > q_lo && k0 < T) ? (q_hi - q_lo + BQ - 1) / BQ : 0;

    Stage qst, dst;
    float ndreg = 0.f, zireg = 0.f;
    int dreg = -1;
    auto load_tile = [&](int i0) {
        qst.template load<E>(Q, i0, T, D, tid);
        dst.template load<E>(dO, i0, T, D, tid);
        if (tid < BQ) {
            const int i = i0 + tid;
            ndreg = i < T ? NDl[i] : 0.f;
            if constexpr (PUR)
                zireg = i < T ? p.zinv[(size_t)bh * T + i] : 0.f;
            else
                zireg = i < T ? 1.0f / p.z[(size_t)bh * T + i] : 0.f;
            if (kDoc && has_doc) dreg = i < T ? docb[i] : -1;
        }
    };
    auto store_tile = [&](int buf) {
        qst.template store_rows<RS>(q_lds[buf], tid);
        qst.template store_trans<TS>(qt_lds[buf], tid);
        dst.template store_rows<RS>(d_lds[buf], tid);
        dst.template store_trans<TS>(dt_lds[buf], tid);
        if (tid < BQ) {
            nd_lds[buf][tid] = ndreg;
            zi_lds[buf][tid] = zireg;
            if (kDoc && has_doc) doc_lds[buf][tid] = dreg;
        }
    };

    f32x16 dv[DB], dk[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        dv[db] = zero16();
        dk[db] = zero16();
    }

    // Documents: visit only the span of query tiles whose ids meet the
    // block's keys'.  Under causality the span starts at q_lo (the query tile
    // holding key k0 sees it), so that tile's loads go out before the
    // screening and overlap it.
    bool first_issued = false;
    if constexpr (kDoc) {
        if (has_doc && ntiles > 0) {
            if (causal) {
                load_tile(q_lo);
                first_issued = true;
            }
            const int2 sp = doc_tile_span<BQ>(docb, T, k0, min(T, k0 + BK), q_lo / BQ, q_lo / BQ + ntiles - 1,
                                              span_red);
            if (causal) {
                ntiles = sp.x <= sp.y ? sp.y - q_lo / BQ + 1 : 0;
            } else {
                ntiles = sp.x <= sp.y ? sp.y - sp.x + 1 : 0;
                if (ntiles > 0) q_lo = sp.x * BQ;
            }
        }
    }
    if (ntiles > 0) {
        if (!first_issued) load_tile(q_lo);
        store_tile(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int i0 = q_lo + t * BQ;
        const int buf = t & 1;
        const bool more = (t + 1) < ntiles;
        if (more) load_tile(i0 + BQ);

        bool active = kw0 < T;
        bool need_mask = false;
        if constexpr (kDoc) need_mask = has_doc && !one_document(doc_lds[buf], BQ, kdoc, kdoc);
        if (causal) {
            active = active && (i0 + BQ - 1 >= kw0);
            need_mask = need_mask || (i0 < kw0 + 31);
        }
        if (window > 0) {
            active = active && (i0 - (kw0 + 31) < window);
            need_mask = need_mask || (i0 + BQ - 1 - kw0 >= window);
        }
        if (active) {
#pragma unroll
            for (int qs = 0; qs < NQ; ++qs) {
                f32x16 s = zero16();
                f32x16 dp, zi;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 n4 = *reinterpret_cast<const f32x4*>(&nd_lds[buf][qs * 32 + 8 * j + 4 * g]);
                    const f32x4 z4 = *reinterpret_cast<const f32x4*>(&zi_lds[buf][qs * 32 + 8 * j + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dp[4 * j + e] = n4[e];
                        zi[4 * j + e] = z4[e];
                    }
                }
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const u32x4 aq = *reinterpret_cast<const u32x4*>(
                        &q_lds[buf][(qs * 32 + c) * RS + ks * 16 + g * 8]);
                    const u32x4 ad = *reinterpret_cast<const u32x4*>(
                        &d_lds[buf][(qs * 32 + c) * RS + ks * 16 + g * 8]);
                    s = E::mfma(aq, kr[ks], s);
                    dp = E::mfma(ad, vr[ks], dp);
                }
                uint32_t vis_bits = 0xffffu;  // purified: bit r set for a visible register r
                if (need_mask) {
                    const int ibase = i0 + qs * 32 + 4 * g;
                    uint32_t bits = 0;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int qi = ibase + 8 * (r >> 2) + (r & 3);
                        const int qd = (kDoc && has_doc) ? doc_lds[buf][qi - i0] : 0;
                        const bool vis = visible<MODE>(qi, key, causal, window, has_doc, qd, kdoc);
                        if constexpr (PUR)
                            bits |= vis ? (1u << r) : 0u;
                        else if (!vis)
                            s[r] = 0.f;
                    }
                    vis_bits = bits;
                }
                uint32_t w2[8], u2[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if constexpr (PUR) {
                        // Masked pairs weigh zero; queries past T have 1/Z = 0.
                        float ww[2], uu[2];
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const int r = 2 * j + e;
                            const float x = s[r];
                            float u = relu_f32(fmaf(x, pg, pgt));
                            float bb = relu_f32(x);
                            if (!((vis_bits >> r) & 1u)) u = bb = 0.f;
                            const float u2_ = u * u;
                            const float dpz = dp[r] * zi[r];
                            const float a = u2_ * u * dpz;
                            dg_acc = fmaf(a, x - ptau, dg_acc);
                            dt_acc += a;
                            ww[e] = fmaf(u2_, u2_, pe * bb * bb) * zi[r];
                            uu[e] = fmaf(p4g, u2_ * u, p2e * bb) * dpz;
                        }
                        w2[j] = E::pack(ww[0], ww[1]);
                        u2[j] = E::pack(uu[0], uu[1]);
                    } else {
                        const float a0 = fmaxf(pre(s[2 * j]), 0.f), a1 = fmaxf(pre(s[2 * j + 1]), 0.f);
                        const float t0 = a0 * zi[2 * j], t1 = a1 * zi[2 * j + 1];
                        w2[j] = E::pack(t0 * a0, t1 * a1);
                        u2[j] = E::pack(t0 * dp[2 * j], t1 * dp[2 * j + 1]);
                    }
                }
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const u32x4 bw = {w2[4 * hh], w2[4 * hh + 1], w2[4 * hh + 2], w2[4 * hh + 3]};
                    const u32x4 bu = {u2[4 * hh], u2[4 * hh + 1], u2[4 * hh + 2], u2[4 * hh + 3]};
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        if (DBF % CS != 0 && db0 + db >= DBF) break;  // the last split's short share
                        const int off = ((db0 + db) * 32 + c) * TS + qs * 32 + hh * 16 + g * 4;
                        const u32x2 dlo = *reinterpret_cast<const u32x2*>(&dt_lds[buf][off]);
                        const u32x2 dhi = *reinterpret_cast<const u32x2*>(&dt_lds[buf][off + 8]);
                        const u32x2 qlo = *reinterpret_cast<const u32x2*>(&qt_lds[buf][off]);
                        const u32x2 qhi = *reinterpret_cast<const u32x2*>(&qt_lds[buf][off + 8]);
                        const u32x4 ad = {dlo[0], dlo[1], dhi[0], dhi[1]};
                        const u32x4 aq = {qlo[0], qlo[1], qhi[0], qhi[1]};
                        dv[db] = E::mfma(ad, bw, dv[db]);
                        dk[db] = E::mfma(aq, bu, dk[db]);
                    }
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    if constexpr (PUR) {
        // Workgroup partials of dgamma and dtau in a fixed order (lanes, then
        // waves), from the first column split of the key block only (the
        // others form the same sums); keys past T excluded.
        __shared__ float red[2 * NW];
        float a = key < T ? 4.f * dg_acc : 0.f;
        float t2 = key < T ? -4.f * sc * dt_acc : 0.f;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            a += __shfl_xor(a, off);
            t2 += __shfl_xor(t2, off);
        }
        if (lane == 0) red[wave] = a, red[NW + wave] = t2;
        __syncthreads();
        if (cs == 0 && tid == 0) {
            float sa = 0.f, st = 0.f;
            for (int w = 0; w < NW; ++w) sa += red[w], st += red[NW + w];
            const int nwg = (int)(gridDim.x / CS);
            p.part[bid] = sa;
            p.part[nwg + bid] = st;
        }
    }
    if (key < T) {
        uint16_t* __restrict__ dK = reinterpret_cast<uint16_t*>(p.dk) + base;
        uint16_t* __restrict__ dV = reinterpret_cast<uint16_t*>(p.dv) + base;
        const float fk = PUR ? 1.f : E::kScaleInSquare ? sc : 2.f * sc * fabsf(sc);
        const float fv = PUR ? 1.f : E::kScaleInSquare ? (sc != 0.f ? 0.25f : 0.f) : sc * sc;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = (db0 + db) * 32 + 8 * j + 4 * g;
                if (d < D) {
                    u32x2 wk, wv;
                    wk[0] = E::pack(dk[db][4 * j] * fk, dk[db][4 * j + 1] * fk);
                    wk[1] = E::pack(dk[db][4 * j + 2] * fk, dk[db][4 * j + 3] * fk);
                    wv[0] = E::pack(dv[db][4 * j] * fv, dv[db][4 * j + 1] * fv);
                    wv[1] = E::pack(dv[db][4 * j + 2] * fv, dv[db][4 * j + 3] * fv);
                    *reinterpret_cast<u32x2*>(dK + (size_t)key * D + d) = wk;
                    *reinterpret_cast<u32x2*>(dV + (size_t)key * D + d) = wv;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dQ, fp32 (v_mfma_f32_32x32x2_f32).  Same structure as the 16-bit kernel;
// fp32 operands need no transposed copies: the contraction over keys reads
// K[key][d] with d across lanes.
// ---------------------------------------------------------------------------
template <int DP, int NW, int BN, int MODE, int WPE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void born_bwd_dq32_kernel(BwdArgs p) {
    constexpr int QW = 32;
    constexpr int BM = NW * QW;
    constexpr int KQ = DP / 8;
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int NT = NW * 64;
    constexpr int RS = DP + 4;
    constexpr bool kDoc = (MODE == kGeneral);
    using Stage = RowStager32<BN, DP, NT>;

    __shared__ __attribute__((aligned(16))) float k_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) float v_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[kDoc ? 2 : 1][kDoc ? BN : 1];
    __shared__ int32_t span_red[kDoc ? 4 : 1];

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
    const int qi = q0 + c;

    const size_t base = (size_t)bh * T * D;
    const float* __restrict__ Q = reinterpret_cast<const float*>(p.q) + base;
    const float* __restrict__ K = reinterpret_cast<const float*>(p.k) + base;
    const float* __restrict__ V = reinterpret_cast<const float*>(p.v) + base;
    const float* __restrict__ dO = reinterpret_cast<const float*>(p.dout) + base;
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;

    const float sc = p.scale[p.per_head_scale ? h : 0];
    const float sgn = (sc < 0.f) ? -1.f : 1.f;

    f32x4 qr[KQ], dr[KQ];
#pragma unroll
    for (int u = 0; u < KQ; ++u) {
        const int d = 8 * u + 4 * g;
        f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
        if (qi < T && d < D) {
            x = *reinterpret_cast<const f32x4*>(Q + (size_t)qi * D + d);
            y = *reinterpret_cast<const f32x4*>(dO + (size_t)qi * D + d);
        }
        qr[u] = x * sgn;
        dr[u] = y;
    }
    const bool qok = qi < T;
    const float zinv = qok ? 1.0f / p.z[(size_t)bh * T + qi] : 0.f;
    const float nd = qok ? -p.delta_z[(size_t)bh * T + qi] : 0.f;
    const int qdoc = (has_doc && qok) ? docb[qi] : -1;

    int kv_lo = 0;
    int kv_hi = causal ? min(T, m0 + BM) : T;
    if (window > 0) kv_lo = max(0, m0 - window + 1) & ~(BN - 1);
    int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + BN - 1) / BN : 0;

    Stage kst, vst;
    int dreg = -2;
    auto load_tile = [&](int key0) {
        kst.load(K, key0, T, D, tid);
        vst.load(V, key0, T, D, tid);
        if (kDoc && has_doc && tid < BN) dreg = (key0 + tid < T) ? docb[key0 + tid] : -2;
    };
    auto store_tile = [&](int buf) {
        kst.template store_rows<RS>(k_lds[buf], tid);
        vst.template store_rows<RS>(v_lds[buf], tid);
        if (kDoc && has_doc && tid < BN) doc_lds[buf][tid] = dreg;
    };

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = zero16();

    // Documents: visit only the span of key tiles whose ids meet the block's
    // rows'.  Under causality the span ends at the block's diagonal tile (its
    // last row sees its own key): the span is walked from there downwards,
    // so the first tile's loads go out before the screening and overlap it.
    int kstep = BN;
    bool first_issued = false;
    if constexpr (kDoc) {
        if (has_doc && ntiles > 0) {
            const int t_top = kv_lo / BN + ntiles - 1;
            if (causal) {
                load_tile(t_top * BN);
                first_issued = true;
            }
            const int2 sp = doc_tile_span<BN>(docb, T, m0, min(T, m0 + BM), kv_lo / BN, t_top, span_red);
            if (causal) {
                ntiles = sp.x <= sp.y ? t_top - sp.x + 1 : 0;
                kv_lo = t_top * BN;
                kstep = -BN;
            } else {
                ntiles = sp.x <= sp.y ? sp.y - sp.x + 1 : 0;
                if (ntiles > 0) kv_lo = sp.x * BN;
            }
        }
    }
    if (ntiles > 0) {
        if (!first_issued) load_tile(kv_lo);
        store_tile(0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int key0 = kv_lo + t * kstep;
        const int buf = t & 1;
        const bool more = (t + 1) < ntiles;
        if (more) load_tile(key0 + kstep);
        bool active = q0 < T;
        bool need_mask = false;
        if constexpr (kDoc) need_mask = has_doc && !one_document(doc_lds[buf], BN, qdoc, qdoc);
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
                f32x16 s = zero16(), tt = zero16();
#pragma unroll
                for (int u = 0; u < KQ; ++u) {
                    const f32x4 ak = *reinterpret_cast<const f32x4*>(&k_lds[buf][(nb * 32 + c) * RS + 8 * u + 4 * g]);
                    const f32x4 av = *reinterpret_cast<const f32x4*>(&v_lds[buf][(nb * 32 + c) * RS + 8 * u + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s = mfma_f32(ak[e], qr[u][e], s);
                        tt = mfma_f32(av[e], dr[u][e], tt);
                    }
                }
                const int kbase = key0 + nb * 32 + 4 * g;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float x = fmaxf(s[r], 0.f);
                    if (need_mask) {
                        const int kk = kbase + 8 * (r >> 2) + (r & 3);
                        const int kd = (kDoc && has_doc) ? doc_lds[buf][kk - key0] : 0;
                        if (!visible<MODE>(qi, kk, causal, window, has_doc, qdoc, kd)) x = 0.f;
                    }
                    s[r] = x * fmaf(tt[r], zinv, nd);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int krow = nb * 32 + acc_row(r, g);
#pragma unroll
                    for (int db = 0; db < DB; ++db)
                        acc[db] = mfma_f32(k_lds[buf][krow * RS + db * 32 + c], s[r], acc[db]);
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }
    if (qok) {
        float* __restrict__ dQ = reinterpret_cast<float*>(p.dq) + base;
        const float f = 2.f * sc * fabsf(sc);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = db * 32 + 8 * j + 4 * g;
                if (d < D) {
                    f32x4 w = {acc[db][4 * j] * f, acc[db][4 * j + 1] * f, acc[db][4 * j + 2] * f,
                               acc[db][4 * j + 3] * f};
                    *reinterpret_cast<f32x4*>(dQ + (size_t)qi * D + d) = w;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dK / dV, fp32.  Keys stationary; K' and V rows of the wave's 32 keys are
// B operands, in registers (KV_LDS = false) or, for wide heads, read from a
// per-workgroup LDS copy (KV_LDS = true, one wave per workgroup).  Same
// arithmetic as the 16-bit kernel; fp32 operands need no transposed copies.
// CS column splits as in the 16-bit kernel: with CS == 2 two workgroups share
// a key block, each accumulating dK, dV for half of the head dim's columns.
// ---------------------------------------------------------------------------
template <int DP, int NW, int BQ, int MODE, int WPE, bool KV_LDS, int CS = 1>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void born_bwd_dkdv32_kernel(BwdArgs p) {
    constexpr int BK = NW * 32;
    constexpr int KQ = DP / 8;
    constexpr int DBF = DP / 32;             // column blocks of the head dim
    constexpr int DB = (DBF + CS - 1) / CS;  // column blocks accumulated here (at most)
    constexpr int NQ = BQ / 32;
    constexpr int NT = NW * 64;
    constexpr int RS = DP + 4;
    constexpr int NBUF = KV_LDS ? 1 : 2;
    constexpr bool kDoc = (MODE == kGeneral);
    using Stage = RowStager32<BQ, DP, NT>;
    static_assert(!KV_LDS || NW == 1, "LDS-resident K/V uses one wave per workgroup");

    __shared__ __attribute__((aligned(16))) float q_lds[NBUF][BQ * RS];
    __shared__ __attribute__((aligned(16))) float d_lds[NBUF][BQ * RS];
    __shared__ __attribute__((aligned(16))) float kv_lds[KV_LDS ? 2 : 1][KV_LDS ? 32 * RS : 4];
    __shared__ __attribute__((aligned(16))) float nd_lds[NBUF][BQ];
    __shared__ __attribute__((aligned(16))) float zi_lds[NBUF][BQ];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[kDoc ? NBUF : 1][kDoc ? BQ : 1];
    __shared__ int32_t span_red[kDoc ? 4 : 1];

    const int T = p.T, D = p.D;
    const int BH = p.B * p.H;
    const bool causal = (MODE == kCausal) || (MODE == kGeneral && p.is_causal);
    const int window = (MODE == kGeneral) ? p.window : 0;
    const bool has_doc = kDoc && p.doc != nullptr;

    const int cs = (CS > 1) ? (int)(blockIdx.x % CS) : 0;
    const int bid = blockIdx.x / CS;
    const int db0 = cs * DB;  // first column block accumulated here
    const int bh = bid % BH;
    const int kb = bid / BH;
    const int b = bh / p.H, h = bh % p.H;
    const int k0 = kb * BK;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, g = lane >> 5;
    const int kw0 = k0 + wave * 32;
    const int key = kw0 + c;

    const size_t base = (size_t)bh * T * D;
    const float* __restrict__ Q = reinterpret_cast<const float*>(p.q) + base;
    const float* __restrict__ K = reinterpret_cast<const float*>(p.k) + base;
    const float* __restrict__ V = reinterpret_cast<const float*>(p.v) + base;
    const float* __restrict__ dO = reinterpret_cast<const float*>(p.dout) + base;
    const float* __restrict__ Zr = p.z + (size_t)bh * T;
    const float* __restrict__ NDl = p.ndelta + (size_t)bh * T;
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;

    const float sc = p.scale[p.per_head_scale ? h : 0];
    const float sgn = (sc < 0.f) ? -1.f : 1.f;

    // B operands: K'[key][d(t, g)], V[key][d(t, g)] with d(t, g) = 8(t/4) + 4g + t%4.
    f32x4 kr[KV_LDS ? 1 : KQ], vr[KV_LDS ? 1 : KQ];
    if constexpr (KV_LDS) {
        for (int idx = tid; idx < 32 * (DP / 4); idx += NT) {
            const int row = idx / (DP / 4), col = (idx % (DP / 4)) * 4;
            const int kk = kw0 + row;
            f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
            if (kk < T && col < D) {
                x = *reinterpret_cast<const f32x4*>(K + (size_t)kk * D + col) * sgn;
                y = *reinterpret_cast<const f32x4*>(V + (size_t)kk * D + col);
            }
            *reinterpret_cast<f32x4*>(&kv_lds[0][row * RS + col]) = x;
            *reinterpret_cast<f32x4*>(&kv_lds[1][row * RS + col]) = y;
        }
    } else {
#pragma unroll
        for (int u = 0; u < KQ; ++u) {
            const int d = 8 * u + 4 * g;
            f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
            if (key < T && d < D) {
                x = *reinterpret_cast<const f32x4*>(K + (size_t)key * D + d);
                y = *reinterpret_cast<const f32x4*>(V + (size_t)key * D + d);
            }
            kr[u] = x * sgn;
            vr[u] = y;
        }
    }
    const int kdoc = (has_doc && key < T) ? docb[key] : -2;

    int q_lo = causal ? (k0 & ~(BQ - 1)) : 0;
    int q_hi = T;
    if (window > 0) q_hi = min(T, k0 + BK - 1 + window);
    int ntiles = (q_hi > q_lo && k0 < T) ? (q_hi - q_lo + BQ - 1) / BQ : 0;

    Stage qst, dst;
    float ndreg = 0.f, zireg = 0.f;
    int dreg = -1;
    auto load_tile = [&](int i0) {
        qst.load(Q, i0, T, D, tid);
        dst.load(dO, i0, T, D, tid);
        if (tid < BQ) {
            const int i = i0 + tid;
            ndreg = i < T ? NDl[i] : 0.f;
            zireg = i < T ? 1.0f / Zr[i] : 0.f;
            if (kDoc && has_doc) dreg = i < T ? docb[i] : -1;
        }
    };
    auto store_tile = [&](int buf) {
        qst.template store_rows<RS>(q_lds[buf], tid);
        dst.template store_rows<RS>(d_lds[buf], tid);
        if (tid < BQ) {
            nd_lds[buf][tid] = ndreg;
            zi_lds[buf][tid] = zireg;
            if (kDoc && has_doc) doc_lds[buf][tid] = dreg;
        }
    };

    f32x16 dv[DB], dk[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        dv[db] = zero16();
        dk[db] = zero16();
    }

    // Documents: visit only the span of query tiles whose ids meet the
    // block's keys'.  Under causality the span starts at q_lo (the query tile
    // holding key k0 sees it), so that tile's loads go out before the
    // screening and overlap it.
    bool first_issued = false;
    if constexpr (kDoc) {
        if (has_doc && ntiles > 0) {
            if (causal) {
                load_tile(q_lo);
                first_issued = true;
            }
            const int2 sp = doc_tile_span<BQ>(docb, T, k0, min(T, k0 + BK), q_lo / BQ, q_lo / BQ + ntiles - 1,
                                              span_red);
            if (causal) {
                ntiles = sp.x <= sp.y ? sp.y - q_lo / BQ + 1 : 0;
            } else {
                ntiles = sp.x <= sp.y ? sp.y - sp.x + 1 : 0;
                if (ntiles > 0) q_lo = sp.x * BQ;
            }
        }
    }
    if (ntiles > 0) {
        if (!first_issued) load_tile(q_lo);
        store_tile(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int i0 = q_lo + t * BQ;
        const int buf = (NBUF == 2) ? (t & 1) : 0;
        const bool more = (t + 1) < ntiles;
        if (NBUF == 2 && more) load_tile(i0 + BQ);

        bool active = kw0 < T;
        bool need_mask = false;
        if constexpr (kDoc) need_mask = has_doc && !one_document(doc_lds[buf], BQ, kdoc, kdoc);
        if (causal) {
            active = active && (i0 + BQ - 1 >= kw0);
            need_mask = need_mask || (i0 < kw0 + 31);
        }
        if (window > 0) {
            active = active && (i0 - (kw0 + 31) < window);
            need_mask = need_mask || (i0 + BQ - 1 - kw0 >= window);
        }
        if (active) {
#pragma unroll
            for (int qs = 0; qs < NQ; ++qs) {
                f32x16 s = zero16(), dp, zi;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 n4 = *reinterpret_cast<const f32x4*>(&nd_lds[buf][qs * 32 + 8 * j + 4 * g]);
                    const f32x4 z4 = *reinterpret_cast<const f32x4*>(&zi_lds[buf][qs * 32 + 8 * j + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dp[4 * j + e] = n4[e];
                        zi[4 * j + e] = z4[e];
                    }
                }
#pragma unroll
                for (int u = 0; u < KQ; ++u) {
                    const f32x4 aq = *reinterpret_cast<const f32x4*>(&q_lds[buf][(qs * 32 + c) * RS + 8 * u + 4 * g]);
                    const f32x4 ad = *reinterpret_cast<const f32x4*>(&d_lds[buf][(qs * 32 + c) * RS + 8 * u + 4 * g]);
                    f32x4 bk, bv;
                    if constexpr (KV_LDS) {
                        bk = *reinterpret_cast<const f32x4*>(&kv_lds[0][c * RS + 8 * u + 4 * g]);
                        bv = *reinterpret_cast<const f32x4*>(&kv_lds[1][c * RS + 8 * u + 4 * g]);
                    } else {
                        bk = kr[u];
                        bv = vr[u];
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s = mfma_f32(aq[e], bk[e], s);
                        dp = mfma_f32(ad[e], bv[e], dp);
                    }
                }
                const int ibase = i0 + qs * 32 + 4 * g;
                f32x16 w, uu;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float a = fmaxf(s[r], 0.f);
                    if (need_mask) {
                        const int qi = ibase + 8 * (r >> 2) + (r & 3);
                        const int qd = (kDoc && has_doc) ? doc_lds[buf][qi - i0] : 0;
                        if (!visible<MODE>(qi, key, causal, window, has_doc, qd, kdoc)) a = 0.f;
                    }
                    const float t = a * zi[r];
                    w[r] = t * a;
                    uu[r] = t * dp[r];
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int qrow = qs * 32 + acc_row(r, g);
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        if (DBF % CS != 0 && db0 + db >= DBF) break;  // the last split's short share
                        dv[db] = mfma_f32(d_lds[buf][qrow * RS + (db0 + db) * 32 + c], w[r], dv[db]);
                        dk[db] = mfma_f32(q_lds[buf][qrow * RS + (db0 + db) * 32 + c], uu[r], dk[db]);
                    }
                }
            }
        }
        if (NBUF == 2) {
            if (more) store_tile(buf ^ 1);
            __syncthreads();
        } else {
            __syncthreads();
            if (more) {
                load_tile(i0 + BQ);
                store_tile(0);
            }
            __syncthreads();
        }
    }

    if (key < T) {
        float* __restrict__ dK = reinterpret_cast<float*>(p.dk) + base;
        float* __restrict__ dV = reinterpret_cast<float*>(p.dv) + base;
        const float fk = 2.f * sc * fabsf(sc);
        const float fv = sc * sc;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = (db0 + db) * 32 + 8 * j + 4 * g;
                if (d < D) {
                    f32x4 wk = {dk[db][4 * j] * fk, dk[db][4 * j + 1] * fk, dk[db][4 * j + 2] * fk,
                                dk[db][4 * j + 3] * fk};
                    f32x4 wv = {dv[db][4 * j] * fv, dv[db][4 * j + 1] * fv, dv[db][4 * j + 2] * fv,
                                dv[db][4 * j + 3] * fv};
                    *reinterpret_cast<f32x4*>(dK + (size_t)key * D + d) = wk;
                    *reinterpret_cast<f32x4*>(dV + (size_t)key * D + d) = wv;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Launch configuration and sequence.
// ---------------------------------------------------------------------------
template <int DP>
struct Bwd16Cfg {
    static constexpr int DQ_NQB = DP <= 64 ? 2 : 1;
    static constexpr int DQ_BN = DP <= 128 ? 64 : 32;
    static constexpr int DQ_WPE = DP <= 64 ? 2 : 1;
    static constexpr int KV_BQ = DP <= 64 ? 64 : 32;
    static constexpr int KV_WPE = DP <= 64 ? 2 : 1;
    // dK/dV column splits: at DP >= 192 (64-305 spills unsplit; B8 T2048:
    // D = 256 step 1914 -> 1098 us, D = 192 1414 -> 1202); DP = 160 spills
    // little unsplit and runs faster so (1088 against 1379 us).
    static constexpr int KV_CS = DP >= 192 ? 2 : 1;
    static constexpr int NW = 4;
};

template <int DP>
struct Bwd32Cfg {
    static constexpr int DQ_WPE = DP <= 64 ? 2 : 1;
    static constexpr bool KV_LDS = DP > 128;
    static constexpr int KV_NW = KV_LDS ? 1 : 4;
    static constexpr int KV_WPE = DP <= 64 ? 2 : 1;
    // dK/dV column splits: dense launches at D = 192 and 256 (each split
    // forms S and dP again, which outweighs the spills it removes elsewhere:
    // B4 H2 T2048 backward D = 256 dense 6917 -> 5034 us, D = 192 dense
    // 3901 -> 3695, but causal D = 256 3146 -> 3227 and D = 160 1489 -> 1913).
    template <int MODE>
    static constexpr int kv_cs() { return (MODE == kDense && (DP == 192 || DP == 256)) ? 2 : 1; }
    static constexpr int BQ = 32;
    static constexpr int NW = 4;
    static constexpr int BN = 32;
};

inline int delta_group(int D, int per_chunk) {
    int n = (D + per_chunk - 1) / per_chunk, g = 1;
    while (g < n && g < 32) g <<= 1;
    return g;
}

template <class E, bool F32>
hipError_t launch_bwd_common_pre(const BwdArgs& a, hipStream_t st) {
    const int G = delta_group(a.D, F32 ? 4 : 8);
    const int64_t rows = (int64_t)a.B * a.H * a.T;
    const int per_block = 256 / G;
    const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
    hipLaunchKernelGGL((born_bwd_delta_kernel<E, F32>), grid, dim3(256), 0, st, a, G);
    return hipGetLastError();
}

// dscale reduction (defined in born_bwd_common.hip).
hipError_t launch_bwd_common_post(const BwdArgs& a, hipStream_t st);

// 128 < D <= 256 (documents with a causal window or none), 16-bit inputs:
// the DMA-ring kernels of born_bwd_d256.h (instantiated in born_bwd_d256.hip).
template <class E>
hipError_t launch_bwd16_wide(const BwdArgs& a, hipStream_t st);

template <class E, int DP, int MODE>
hipError_t launch_bwd16(const BwdArgs& a, hipStream_t st) {
    using C = Bwd16Cfg<DP>;
    hipError_t e = hipSuccess;
    const unsigned BH = (unsigned)(a.B * a.H);
    // D == 64, dense or causal, per-head slice addressable with 32-bit buffer
    // offsets: the fast dQ kernel (which also forms delta and fills the
    // workspace, so no pre-pass) and then the fast dK/dV kernel
    // (born_bwd_fast.h).
    const bool addr32 = ((int64_t)a.T + 256) * a.D * 2 < ((int64_t)1 << 31);
    const bool fast = DP == 64 && a.D == 64 && MODE != kGeneral && addr32;
    // Sliding window without documents: the two fast kernels' window modes
    // (kWindow causal, kWindowNC not).
    if constexpr (DP == 64 && MODE == kGeneral) {
        if (a.D == 64 && a.doc == nullptr && a.window > 0 && addr32) {
            if (a.is_causal) {
                if ((e = launch_bwd16_dq_fast<E, 64, kWindow>(a, st)) != hipSuccess) return e;
                if ((e = launch_bwd16_dkdv_fast<E, 64, kWindow>(a, st)) != hipSuccess) return e;
            } else {
                if ((e = launch_bwd16_dq_fast<E, 64, kWindowNC>(a, st)) != hipSuccess) return e;
                if ((e = launch_bwd16_dkdv_fast<E, 64, kWindowNC>(a, st)) != hipSuccess) return e;
            }
            const int nwg = ((a.T + 255) / 256) * a.B * a.H;
            hipLaunchKernelGGL(born_bwd_dscale_groups_kernel<0>, dim3((unsigned)(a.per_head_scale ? a.H : 1)), dim3(256),
                               0, st, a, nwg);
            return hipGetLastError();
        }
    }
    // Documents (with or without a causal window): the same two fast
    // kernels' document variants (tile lists screened by document range).
    if constexpr (DP == 64 && MODE == kGeneral) {
        if (a.D == 64 && a.doc != nullptr && addr32 && (a.window == 0 || a.is_causal)) {
            if (a.window > 0) {
                e = launch_bwd16_dq_fast<E, 64, kWindow, true>(a, st);
                if (e != hipSuccess) return e;
                e = launch_bwd16_dkdv_fast<E, 64, kWindow, true>(a, st);
            } else {
                e = a.is_causal ? launch_bwd16_dq_fast<E, 64, kCausal, true>(a, st)
                                : launch_bwd16_dq_fast<E, 64, kDense, true>(a, st);
                if (e != hipSuccess) return e;
                e = a.is_causal ? launch_bwd16_dkdv_fast<E, 64, kCausal, true>(a, st)
                                : launch_bwd16_dkdv_fast<E, 64, kDense, true>(a, st);
            }
            if (e != hipSuccess) return e;
            const int nwg = bwd16_dq_fast_groups(a.B, a.H, a.T, true);
            hipLaunchKernelGGL(born_bwd_dscale_groups_kernel<0>, dim3((unsigned)(a.per_head_scale ? a.H : 1)), dim3(256),
                               0, st, a, nwg);
            return hipGetLastError();
        }
    }
    // D == 128, dense, causal or a sliding window with or without causality
    // (no documents): the D == 128 kernels (born_bwd_d128.h); 64 < D < 128 on
    // the same kernels with the columns past D zero.
    if constexpr (DP == 128) {
        if (a.D == 128 && a.doc == nullptr && addr32) {
            if (MODE == kGeneral && a.window > 0 && a.is_causal) return launch_bwd16_d128<E, kWindow>(a, st);
            if (MODE == kGeneral && a.window > 0 && !a.is_causal) return launch_bwd16_d128<E, kWindowNC>(a, st);
            if (MODE == kDense || MODE == kCausal) return launch_bwd16_d128<E, MODE == kCausal ? kCausal : kDense>(a, st);
        }
    }
    // D == 128 with document ids (and a causal window): the same kernels'
    // document mode.
    if constexpr (DP == 128 && MODE == kGeneral) {
        if (a.D == 128 && a.doc != nullptr && addr32 && (a.window == 0 || a.is_causal)) {
            if (a.window > 0) return launch_bwd16_d128<E, kWindow, false, true>(a, st);
            return a.is_causal ? launch_bwd16_d128<E, kCausal, false, true>(a, st)
                               : launch_bwd16_d128<E, kDense, false, true>(a, st);
        }
    }
    // 128 < D <= 256, dense, causal or a sliding window with or without
    // causality (documents: with a causal window or none): the DMA-ring
    // kernels for wide rows.
    if constexpr (DP > 128) {
        if (a.D > 128 && addr32 && (a.doc == nullptr || a.window == 0 || a.is_causal))
            return launch_bwd16_wide<E>(a, st);
    }
    // 64 < D < 128 with documents: the same kernels' document mode with zero
    // columns past D.
    if constexpr ((DP == 96 || DP == 128) && MODE == kGeneral) {
        if (a.D > 64 && a.D < 128 && a.doc != nullptr && addr32 && (a.window == 0 || a.is_causal)) {
            if (a.window > 0) return launch_bwd16_d128<E, kWindow, true, true>(a, st);
            return a.is_causal ? launch_bwd16_d128<E, kCausal, true, true>(a, st)
                               : launch_bwd16_d128<E, kDense, true, true>(a, st);
        }
    }
    if constexpr (DP == 96 || DP == 128) {
        if (a.D > 64 && a.D < 128 && a.doc == nullptr && addr32) {
            if (MODE == kGeneral && a.window > 0 && a.is_causal) return launch_bwd16_d128<E, kWindow, true>(a, st);
            if (MODE == kGeneral && a.window > 0 && !a.is_causal) return launch_bwd16_d128<E, kWindowNC, true>(a, st);
            if (MODE == kDense || MODE == kCausal)
                return launch_bwd16_d128<E, MODE == kCausal ? kCausal : kDense, true>(a, st);
        }
    }
    if constexpr (DP == 64 && MODE != kGeneral) {
        if (fast) {
            if ((e = launch_bwd16_dq_fast<E, 64, MODE>(a, st)) != hipSuccess) return e;
            if ((e = launch_bwd16_dkdv_fast<E, 64, MODE>(a, st)) != hipSuccess) return e;
            const int nwg = ((a.T + 255) / 256) * a.B * a.H;
            hipLaunchKernelGGL(born_bwd_dscale_groups_kernel<0>, dim3((unsigned)(a.per_head_scale ? a.H : 1)), dim3(256),
                               0, st, a, nwg);
            return hipGetLastError();
        }
    }
    if (!fast && (e = launch_bwd_common_pre<E, false>(a, st)) != hipSuccess) return e;
    if (!fast) {
        constexpr int BK = C::NW * 32;
        const dim3 grid((unsigned)((a.T + BK - 1) / BK) * BH * C::KV_CS);
        hipLaunchKernelGGL((born_bwd_dkdv16_kernel<E, DP, C::NW, C::KV_BQ, MODE, C::KV_WPE, C::KV_CS>), grid,
                           dim3(C::NW * 64), 0, st, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (!fast && MODE == kGeneral && a.doc != nullptr && C::DQ_NQB == 2) {
        // Documents: 128-row query blocks straddle fewer document edges
        // than 256-row ones, so fewer of their tiles are partly visible.
        constexpr int BM = C::NW * 32;
        const dim3 grid((unsigned)((a.T + BM - 1) / BM) * BH);
        hipLaunchKernelGGL((born_bwd_dq16_kernel<E, DP, 1, C::NW, C::DQ_BN, MODE, C::DQ_WPE>), grid,
                           dim3(C::NW * 64), 0, st, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    } else if (!fast) {
        constexpr int BM = C::NW * 32 * C::DQ_NQB;
        const dim3 grid((unsigned)((a.T + BM - 1) / BM) * BH);
        hipLaunchKernelGGL((born_bwd_dq16_kernel<E, DP, C::DQ_NQB, C::NW, C::DQ_BN, MODE, C::DQ_WPE>),
                           grid, dim3(C::NW * 64), 0, st, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return launch_bwd_common_post(a, st);
}

template <int DP, int MODE>
hipError_t launch_bwd32(const BwdArgs& a, hipStream_t st) {
    using C = Bwd32Cfg<DP>;
    hipError_t e = launch_bwd_common_pre<BF16, true>(a, st);
    if (e != hipSuccess) return e;
    const unsigned BH = (unsigned)(a.B * a.H);
    {
        constexpr int BK = C::KV_NW * 32;
        constexpr int CS = C::template kv_cs<MODE>();
        const dim3 grid((unsigned)((a.T + BK - 1) / BK) * BH * CS);
        hipLaunchKernelGGL((born_bwd_dkdv32_kernel<DP, C::KV_NW, C::BQ, MODE, C::KV_WPE, C::KV_LDS, CS>), grid,
                           dim3(C::KV_NW * 64), 0, st, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    {
        constexpr int BM = C::NW * 32;
        const dim3 grid((unsigned)((a.T + BM - 1) / BM) * BH);
        hipLaunchKernelGGL((born_bwd_dq32_kernel<DP, C::NW, C::BN, MODE, C::DQ_WPE>), grid,
                           dim3(C::NW * 64), 0, st, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return launch_bwd_common_post(a, st);
}

}  // namespace qdl
