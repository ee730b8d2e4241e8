// Flash purified-Born attention for gfx950: the reference's
// `_flash_purified_born_fwd_kernel`, `_flash_purified_born_bwd_kernel` and
// `_flash_purified_born_bwd_dq_kernel` (src/qdlblocks/kernels/flash_born.py:
// 696-1061).
//
// Per (b, h), with r_ij = q_i . k_j (unscaled), gamma = scale_h, tau = tau_h:
//   u_ij = max(0, gamma (r_ij - tau)) M_ij,  b_ij = max(0, r_ij) M_ij,
//   p_ij = u_ij^4 + eps_base b_ij^2,  Z_i = sum_j p_ij + eps,
//   O_i  = sum_j p_ij v_j / Z_i                        (O and Z in fp32)
// Backward with delta_i = dO_i . O_i (from the fp32 O):
//   dP_ij = (dO_i . v_j - delta_i) / Z_i,   du_ij = 4 u_ij^3 dP_ij,
//   dR_ij = gamma du_ij + 2 eps_base b_ij dP_ij,
//   dq_i = sum_j dR_ij k_j,  dk_j = sum_i dR_ij q_i,  dv_j = sum_i p_ij / Z_i dO_i,
//   dgamma = sum du_ij (r_ij - tau),  dtau = -gamma sum du_ij.
//
// The reference contracts P V as an fp32 dot (v cast to fp32) and keeps p,
// Z and O in fp32, so every contraction here runs on v_mfma_f32_32x32x2_f32
// with operands converted to fp32 as they are staged into LDS (bf16 and fp16
// values convert exactly).  As in the reference, the backward rounds the
// weights p/Z and dR to the input dtype before their contractions.  The
// masks (causal, sliding window, document ids) are the Born kernels'
// (flash_born.py:783-794, 906-917).  dgamma and dtau are reduced in a fixed
// order (per-workgroup partials, then one pass per output): deterministic,
// unlike the reference's float atomics.
#pragma once

#include "born_common.h"
#include "purified_args.h"

namespace qdl {

// Input element access: 4 consecutive elements <-> f32x4, and rounding to
// the input dtype (what the reference's `.to(q.dtype)` before a dot does).
template <class IN>
struct PurIO;
template <>
struct PurIO<float> {
    static constexpr int kBytes = 4;
    static __device__ __forceinline__ f32x4 load4(const void* base, size_t idx) {
        return *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + idx);
    }
    static __device__ __forceinline__ void store4(void* base, size_t idx, f32x4 x) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(base) + idx) = x;
    }
    static __device__ __forceinline__ float round(float x) { return x; }
};
template <class E>
struct PurIO16 {
    static constexpr int kBytes = 2;
    static __device__ __forceinline__ f32x4 load4(const void* base, size_t idx) {
        const u32x2 u = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(base) + idx);
        const f32x4 x = {E::lo(u[0]), E::hi(u[0]), E::lo(u[1]), E::hi(u[1])};
        return x;
    }
    static __device__ __forceinline__ void store4(void* base, size_t idx, f32x4 x) {
        const u32x2 u = {E::pack(x[0], x[1]), E::pack(x[2], x[3])};
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(base) + idx) = u;
    }
    static __device__ __forceinline__ float round(float x) { return E::lo(E::pack(x, 0.f)); }
};
template <>
struct PurIO<BF16> : PurIO16<BF16> {};
template <>
struct PurIO<F16> : PurIO16<F16> {};

// Visibility of (query i, key j) under the runtime masks.
__device__ __forceinline__ bool pur_visible(int i, int j, bool causal, int window, bool has_doc, int doc_i,
                                            int doc_j) {
    bool v = true;
    if (causal) v = v && (j <= i);
    if (window > 0) v = v && (i - j < window);
    if (has_doc) v = v && (doc_i == doc_j);
    return v;
}

// R rows x DP columns of an input-dtype tile, staged through registers as fp32.
template <class IN, int R, int DP, int NT>
struct PurStager {
    static constexpr int CPR = DP / 4;
    static constexpr int CH = R * CPR;
    static constexpr int PT = (CH + NT - 1) / NT;
    f32x4 x[PT];
    __device__ __forceinline__ void load(const void* src, int r0, int T, int D, int tid) {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) {
                const int col = (idx % CPR) * 4;
                const int row = r0 + idx / CPR;
                f32x4 a = {0.f, 0.f, 0.f, 0.f};
                if (row < T && col < D) a = PurIO<IN>::load4(src, (size_t)row * D + col);
                x[i] = a;
            }
        }
    }
    template <int RS>
    __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int idx = tid + i * NT;
            if (CH % NT == 0 || idx < CH) *reinterpret_cast<f32x4*>(&lds[(idx / CPR) * RS + (idx % CPR) * 4]) = x[i];
        }
    }
};

template <int DP>
struct PurCfg {
    static constexpr int NW = 4;
    static constexpr int BN = 32;  // keys per forward / dQ tile
    static constexpr int BQ = 32;  // queries per dK/dV tile
    static constexpr int FWD_WPE = DP <= 128 ? 2 : 1;
    static constexpr int DQ_WPE = DP <= 64 ? 2 : 1;
    static constexpr int KV_WPE = DP <= 64 ? 2 : 1;
    static constexpr bool KV_LDS = DP > 128;  // dK/dV: K, V rows from LDS (one wave per workgroup)
    static constexpr int KV_NW = KV_LDS ? 1 : 4;
};

// ---------------------------------------------------------------------------
// Forward (flash_born.py:696-811).  Queries stationary: wave w owns 32 query
// rows; K/V tiles of BN keys double-buffered in LDS.
//   S^T = K Q^T (accumulator: one query per lane, 16 keys), p in fp32,
//   O^T += V^T P^T with the weights as fp32 B operands.
// ---------------------------------------------------------------------------
template <class IN, int DP, int NW, int BN, int WPE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void purified_fwd_kernel(PurArgs p) {
    static_assert(DP % 32 == 0 && DP <= 256, "padded head dim");
    constexpr int QW = 32;
    constexpr int BM = NW * QW;
    constexpr int KQ = DP / 8;
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int NT = NW * 64;
    constexpr int RS = DP + 4;
    using Stage = PurStager<IN, BN, DP, NT>;

    __shared__ __attribute__((aligned(16))) float k_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) float v_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[2][BN];
    __shared__ int32_t span_red[4];

    const int T = p.T, D = p.D;
    const int BH = p.B * p.H;
    const int nmb = (T + BM - 1) / BM;
    const bool causal = p.is_causal != 0;
    const int window = p.window;
    const bool has_doc = p.doc != nullptr;

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
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;
    const float gam = p.scale[p.per_head_scale ? h : 0];
    const float tau = p.tau[p.per_head_tau ? h : 0];
    const float eb = p.eps_base;

    // Contraction step t of the QK product uses dim 8 (t/4) + 4 g + t%4.
    f32x4 qr[KQ];
#pragma unroll
    for (int u = 0; u < KQ; ++u) {
        const int d = 8 * u + 4 * g;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (qi < T && d < D) x = PurIO<IN>::load4(p.q, base + (size_t)qi * D + d);
        qr[u] = x;
    }
    const int qdoc = (has_doc && qi < T) ? docb[qi] : -1;

    // Key range (flash_born.py:767-769).
    int kv_lo = 0;
    const int kv_hi = causal ? min(T, m0 + BM) : T;
    if (window > 0) kv_lo = max(0, m0 - window + 1) & ~(BN - 1);
    int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + BN - 1) / BN : 0;
    if (has_doc && ntiles > 0) {
        const int2 sp = doc_tile_span<BN>(docb, T, m0, min(T, m0 + BM), kv_lo / BN, kv_lo / BN + ntiles - 1,
                                          span_red);
        ntiles = sp.x <= sp.y ? sp.y - sp.x + 1 : 0;
        if (ntiles > 0) kv_lo = sp.x * BN;
    }

    Stage kst, vst;
    int dreg = -2;
    auto load_tile = [&](int key0) {
        kst.load(reinterpret_cast<const char*>(p.k) + base * PurIO<IN>::kBytes, key0, T, D, tid);
        vst.load(reinterpret_cast<const char*>(p.v) + base * PurIO<IN>::kBytes, key0, T, D, tid);
        if (has_doc && tid < BN) dreg = (key0 + tid < T) ? docb[key0 + tid] : -2;
    };
    auto store_tile = [&](int buf) {
        kst.template store<RS>(k_lds[buf], tid);
        vst.template store<RS>(v_lds[buf], tid);
        if (has_doc && tid < BN) doc_lds[buf][tid] = dreg;
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
        bool need_mask = (has_doc && !one_document(doc_lds[buf], BN, qdoc, qdoc)) || key0 + BN > T;
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
                    const f32x4 a = *reinterpret_cast<const f32x4*>(&k_lds[buf][(nb * 32 + c) * RS + 8 * u + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) s = mfma_f32(a[e], qr[u][e], s);
                }
                const int kbase = key0 + nb * 32 + 4 * g;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float x = s[r];
                    float uu = fmaxf(gam * (x - tau), 0.f);
                    float bb = fmaxf(x, 0.f);
                    if (need_mask) {
                        const int kk = kbase + 8 * (r >> 2) + (r & 3);
                        const int kd = has_doc ? doc_lds[buf][kk - key0] : 0;
                        if (kk >= T || !pur_visible(qi, kk, causal, window, has_doc, qdoc, kd)) uu = bb = 0.f;
                    }
                    const float u2 = uu * uu;
                    const float pr = u2 * u2 + eb * (bb * bb);
                    zacc += pr;
                    s[r] = pr;
                }
                // O^T += V^T P^T: step r contracts key acc_row(r, g) of this block.
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int krow = nb * 32 + acc_row(r, g);
#pragma unroll
                    for (int db = 0; db < DB; ++db) oacc[db] = mfma_f32(v_lds[buf][krow * RS + db * 32 + c], s[r], oacc[db]);
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    const float zd = zacc + __shfl_xor(zacc, 32) + p.eps;
    if (qi < T) {
        float* __restrict__ O = p.o + base;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = db * 32 + 8 * j + 4 * g;
                if (d < D) {
                    const f32x4 w = {oacc[db][4 * j] / zd, oacc[db][4 * j + 1] / zd, oacc[db][4 * j + 2] / zd,
                                     oacc[db][4 * j + 3] / zd};
                    *reinterpret_cast<f32x4*>(O + (size_t)qi * D + d) = w;
                }
            }
        if (g == 0) p.z[(size_t)bh * T + qi] = zd;
    }
}

// ---------------------------------------------------------------------------
// Pre-pass: -delta_i = -(dO_i . O_i) with O in fp32, and 1 / Z_i.  One group
// of G lanes per row.
// ---------------------------------------------------------------------------
template <class IN>
__global__ __launch_bounds__(256) void purified_delta_kernel(PurArgs p, int G) {
    const int per_block = 256 / G;
    const int64_t nrows = (int64_t)p.B * p.H * p.T;
    const int64_t row = (int64_t)blockIdx.x * per_block + threadIdx.x / G;
    const int sub = threadIdx.x % G;
    const int D = p.D;
    float acc = 0.f;
    if (row < nrows) {
        for (int c = sub * 4; c < D; c += G * 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(p.o_in + row * D + c);
            const f32x4 b = PurIO<IN>::load4(p.dout, (size_t)row * D + c);
            acc += a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
        }
    }
    for (int off = G >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (row < nrows && sub == 0) {
        p.ndelta[row] = -acc;
        p.zinv[row] = 1.0f / p.z_in[row];
    }
}

// Element of the backward shared by the dK/dV and dQ kernels: from the raw
// overlap x and dpz = dP (already divided by Z), the gradient dR of the
// overlap and the weight's gamma-derivative factor du = 4 u^3 dP.
struct PurGrad {
    float dr, du;
};
__device__ __forceinline__ PurGrad pur_grad(float x, float dpz, float gam, float tau, float eb, bool vis) {
    float uu = fmaxf(gam * (x - tau), 0.f);
    float bb = fmaxf(x, 0.f);
    if (!vis) uu = bb = 0.f;
    const float du = 4.0f * (uu * uu * uu) * dpz;
    PurGrad r;
    r.du = du;
    r.dr = du * gam + 2.0f * eb * bb * dpz;
    return r;
}

// ---------------------------------------------------------------------------
// dK, dV, dgamma and dtau partials (flash_born.py:814-947).  Keys stationary:
// each wave owns 32 keys, their K and V rows held as B operands (registers,
// or LDS for wide heads with one wave per workgroup).  Query tiles of BQ rows
// stream through LDS with their -delta and 1/Z.  Per tile:
//   S = Q K^T, dP = dO V^T - delta (accumulator initialised with -delta),
//   w = round(p / Z), dR = round(gamma du + 2 eps_base b dP / Z),
//   dV^T += dO^T w, dK^T += Q^T dR.
// ---------------------------------------------------------------------------
template <class IN, int DP, int NW, int BQ, int WPE, bool KV_LDS>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void purified_dkdv_kernel(PurArgs p) {
    constexpr int BK = NW * 32;
    constexpr int KQ = DP / 8;
    constexpr int DB = DP / 32;
    constexpr int NQ = BQ / 32;
    constexpr int NT = NW * 64;
    constexpr int RS = DP + 4;
    constexpr int NBUF = KV_LDS ? 1 : 2;
    using Stage = PurStager<IN, BQ, DP, NT>;
    static_assert(!KV_LDS || NW == 1, "LDS-resident K/V uses one wave per workgroup");

    __shared__ __attribute__((aligned(16))) float q_lds[NBUF][BQ * RS];
    __shared__ __attribute__((aligned(16))) float d_lds[NBUF][BQ * RS];
    __shared__ __attribute__((aligned(16))) float kv_lds[KV_LDS ? 2 : 1][KV_LDS ? 32 * RS : 4];
    __shared__ __attribute__((aligned(16))) float nd_lds[NBUF][BQ];
    __shared__ __attribute__((aligned(16))) float zi_lds[NBUF][BQ];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[NBUF][BQ];
    __shared__ int32_t span_red[4];
    __shared__ float red[2][NW];

    const int T = p.T, D = p.D;
    const int BH = p.B * p.H;
    const bool causal = p.is_causal != 0;
    const int window = p.window;
    const bool has_doc = p.doc != nullptr;

    const int bid = blockIdx.x;
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
    const char* Qb = reinterpret_cast<const char*>(p.q) + base * PurIO<IN>::kBytes;
    const char* dOb = reinterpret_cast<const char*>(p.dout) + base * PurIO<IN>::kBytes;
    const float* __restrict__ NDl = p.ndelta + (size_t)bh * T;
    const float* __restrict__ ZIl = p.zinv + (size_t)bh * T;
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;
    const float gam = p.scale[p.per_head_scale ? h : 0];
    const float tau = p.tau[p.per_head_tau ? h : 0];
    const float eb = p.eps_base;

    // B operands: K[key][d(t, g)], V[key][d(t, g)] with d(t, g) = 8 (t/4) + 4 g + t%4.
    f32x4 kr[KV_LDS ? 1 : KQ], vr[KV_LDS ? 1 : KQ];
    if constexpr (KV_LDS) {
        for (int idx = tid; idx < 32 * (DP / 4); idx += NT) {
            const int row = idx / (DP / 4), col = (idx % (DP / 4)) * 4;
            const int kk = kw0 + row;
            f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
            if (kk < T && col < D) {
                x = PurIO<IN>::load4(p.k, base + (size_t)kk * D + col);
                y = PurIO<IN>::load4(p.v, base + (size_t)kk * D + col);
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
                x = PurIO<IN>::load4(p.k, base + (size_t)key * D + d);
                y = PurIO<IN>::load4(p.v, base + (size_t)key * D + d);
            }
            kr[u] = x;
            vr[u] = y;
        }
    }
    const int kdoc = (has_doc && key < T) ? docb[key] : -2;

    // Query range (flash_born.py:885-886; with a window no query past the
    // block's last key + window - 1 sees it, causal or not).
    int q_lo = causal ? (k0 & ~(BQ - 1)) : 0;
    int q_hi = T;
    if (window > 0) q_hi = min(T, k0 + BK - 1 + window);
    int ntiles = (q_hi > q_lo && k0 < T) ? (q_hi - q_lo + BQ - 1) / BQ : 0;
    if (has_doc && ntiles > 0) {
        const int2 sp = doc_tile_span<BQ>(docb, T, k0, min(T, k0 + BK), q_lo / BQ, q_lo / BQ + ntiles - 1,
                                          span_red);
        ntiles = sp.x <= sp.y ? sp.y - sp.x + 1 : 0;
        if (ntiles > 0) q_lo = sp.x * BQ;
    }

    Stage qst, dst;
    float ndreg = 0.f, zireg = 0.f;
    int dreg = -1;
    auto load_tile = [&](int i0) {
        qst.load(Qb, i0, T, D, tid);
        dst.load(dOb, i0, T, D, tid);
        if (tid < BQ) {
            const int i = i0 + tid;
            ndreg = i < T ? NDl[i] : 0.f;
            zireg = i < T ? ZIl[i] : 0.f;
            if (has_doc) dreg = i < T ? docb[i] : -1;
        }
    };
    auto store_tile = [&](int buf) {
        qst.template store<RS>(q_lds[buf], tid);
        dst.template store<RS>(d_lds[buf], tid);
        if (tid < BQ) {
            nd_lds[buf][tid] = ndreg;
            zi_lds[buf][tid] = zireg;
            if (has_doc) doc_lds[buf][tid] = dreg;
        }
    };

    f32x16 dv[DB], dk[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) dv[db] = zero16(), dk[db] = zero16();
    float ds_acc = 0.f, dt_acc = 0.f;

    if (ntiles > 0) {
        load_tile(q_lo);
        store_tile(0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int i0 = q_lo + t * BQ;
        const int buf = (NBUF == 2) ? (t & 1) : 0;
        const bool more = (t + 1) < ntiles;
        if (NBUF == 2 && more) load_tile(i0 + BQ);
        bool active = kw0 < T;
        bool need_mask = (has_doc && !one_document(doc_lds[buf], BQ, kdoc, kdoc)) || key >= T || i0 + BQ > T;
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
                    for (int e = 0; e < 4; ++e) dp[4 * j + e] = n4[e], zi[4 * j + e] = z4[e];
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
                f32x16 w, dr;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float x = s[r];
                    bool vis = true;
                    if (need_mask) {
                        const int qq = ibase + 8 * (r >> 2) + (r & 3);
                        const int qd = has_doc ? doc_lds[buf][qq - i0] : 0;
                        vis = qq < T && key < T && pur_visible(qq, key, causal, window, has_doc, qd, kdoc);
                    }
                    float uu = fmaxf(gam * (x - tau), 0.f);
                    float bb = fmaxf(x, 0.f);
                    if (!vis) uu = bb = 0.f;
                    const float u2 = uu * uu;
                    const float pr = u2 * u2 + eb * (bb * bb);
                    w[r] = PurIO<IN>::round(pr * zi[r]);
                    const float dpz = dp[r] * zi[r];
                    const float du = 4.0f * (u2 * uu) * dpz;
                    dr[r] = PurIO<IN>::round(du * gam + 2.0f * eb * bb * dpz);
                    ds_acc += du * (x - tau);
                    dt_acc -= du * gam;
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int qrow = qs * 32 + acc_row(r, g);
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        dv[db] = mfma_f32(d_lds[buf][qrow * RS + db * 32 + c], w[r], dv[db]);
                        dk[db] = mfma_f32(q_lds[buf][qrow * RS + db * 32 + c], dr[r], dk[db]);
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
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = db * 32 + 8 * j + 4 * g;
                if (d < D) {
                    const f32x4 wk = {dk[db][4 * j], dk[db][4 * j + 1], dk[db][4 * j + 2], dk[db][4 * j + 3]};
                    const f32x4 wv = {dv[db][4 * j], dv[db][4 * j + 1], dv[db][4 * j + 2], dv[db][4 * j + 3]};
                    PurIO<IN>::store4(p.dk, base + (size_t)key * D + d, wk);
                    PurIO<IN>::store4(p.dv, base + (size_t)key * D + d, wv);
                }
            }
    }

    // Workgroup partials of dgamma and dtau, in a fixed order.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        ds_acc += __shfl_xor(ds_acc, off);
        dt_acc += __shfl_xor(dt_acc, off);
    }
    if (lane == 0) red[0][wave] = ds_acc, red[1][wave] = dt_acc;
    __syncthreads();
    if (tid == 0) {
        float a = 0.f, t2 = 0.f;
        for (int w2 = 0; w2 < NW; ++w2) a += red[0][w2], t2 += red[1][w2];
        p.part[bid] = a;
        p.part[gridDim.x + bid] = t2;
    }
}

// ---------------------------------------------------------------------------
// dQ (flash_born.py:950-1061).  Queries stationary (Q and dO rows in
// registers, -delta and 1/Z per lane); K/V tiles of BN keys in LDS.
//   S^T = K Q^T, dP^T = V dO^T, dR^T as above, dQ^T += K^T dR^T.
// ---------------------------------------------------------------------------
template <class IN, int DP, int NW, int BN, int WPE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void purified_dq_kernel(PurArgs p) {
    constexpr int QW = 32;
    constexpr int BM = NW * QW;
    constexpr int KQ = DP / 8;
    constexpr int DB = DP / 32;
    constexpr int NB = BN / 32;
    constexpr int NT = NW * 64;
    constexpr int RS = DP + 4;
    using Stage = PurStager<IN, BN, DP, NT>;

    __shared__ __attribute__((aligned(16))) float k_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) float v_lds[2][BN * RS];
    __shared__ __attribute__((aligned(16))) int32_t doc_lds[2][BN];
    __shared__ int32_t span_red[4];

    const int T = p.T, D = p.D;
    const int BH = p.B * p.H;
    const int nmb = (T + BM - 1) / BM;
    const bool causal = p.is_causal != 0;
    const int window = p.window;
    const bool has_doc = p.doc != nullptr;

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
    const int32_t* __restrict__ docb = has_doc ? p.doc + (size_t)b * T : nullptr;
    const float gam = p.scale[p.per_head_scale ? h : 0];
    const float tau = p.tau[p.per_head_tau ? h : 0];
    const float eb = p.eps_base;

    f32x4 qr[KQ], dr[KQ];
#pragma unroll
    for (int u = 0; u < KQ; ++u) {
        const int d = 8 * u + 4 * g;
        f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
        if (qi < T && d < D) {
            x = PurIO<IN>::load4(p.q, base + (size_t)qi * D + d);
            y = PurIO<IN>::load4(p.dout, base + (size_t)qi * D + d);
        }
        qr[u] = x;
        dr[u] = y;
    }
    const bool qok = qi < T;
    const float zinv = qok ? p.zinv[(size_t)bh * T + qi] : 0.f;
    const float nd = qok ? p.ndelta[(size_t)bh * T + qi] : 0.f;
    const int qdoc = (has_doc && qok) ? docb[qi] : -1;

    int kv_lo = 0;
    const int kv_hi = causal ? min(T, m0 + BM) : T;
    if (window > 0) kv_lo = max(0, m0 - window + 1) & ~(BN - 1);
    int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + BN - 1) / BN : 0;
    if (has_doc && ntiles > 0) {
        const int2 sp = doc_tile_span<BN>(docb, T, m0, min(T, m0 + BM), kv_lo / BN, kv_lo / BN + ntiles - 1,
                                          span_red);
        ntiles = sp.x <= sp.y ? sp.y - sp.x + 1 : 0;
        if (ntiles > 0) kv_lo = sp.x * BN;
    }

    Stage kst, vst;
    int dreg = -2;
    auto load_tile = [&](int key0) {
        kst.load(reinterpret_cast<const char*>(p.k) + base * PurIO<IN>::kBytes, key0, T, D, tid);
        vst.load(reinterpret_cast<const char*>(p.v) + base * PurIO<IN>::kBytes, key0, T, D, tid);
        if (has_doc && tid < BN) dreg = (key0 + tid < T) ? docb[key0 + tid] : -2;
    };
    auto store_tile = [&](int buf) {
        kst.template store<RS>(k_lds[buf], tid);
        vst.template store<RS>(v_lds[buf], tid);
        if (has_doc && tid < BN) doc_lds[buf][tid] = dreg;
    };

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = zero16();

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
        bool need_mask = (has_doc && !one_document(doc_lds[buf], BN, qdoc, qdoc)) || key0 + BN > T;
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
                    bool vis = true;
                    if (need_mask) {
                        const int kk = kbase + 8 * (r >> 2) + (r & 3);
                        const int kd = has_doc ? doc_lds[buf][kk - key0] : 0;
                        vis = kk < T && pur_visible(qi, kk, causal, window, has_doc, qdoc, kd);
                    }
                    const PurGrad gr = pur_grad(s[r], (tt[r] + nd) * zinv, gam, tau, eb, vis);
                    s[r] = PurIO<IN>::round(gr.dr);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int krow = nb * 32 + acc_row(r, g);
#pragma unroll
                    for (int db = 0; db < DB; ++db) acc[db] = mfma_f32(k_lds[buf][krow * RS + db * 32 + c], s[r], acc[db]);
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }
    if (qok) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = db * 32 + 8 * j + 4 * g;
                if (d < D) {
                    const f32x4 w = {acc[db][4 * j], acc[db][4 * j + 1], acc[db][4 * j + 2], acc[db][4 * j + 3]};
                    PurIO<IN>::store4(p.dq, base + (size_t)qi * D + d, w);
                }
            }
    }
}

// dgamma / dtau: output o sums, in a fixed order, the partials of the dK/dV
// workgroups whose head it covers (all of them for a shared parameter).
// (A template, so that several translation units can each hold it.)
template <int kUnused = 0>
__global__ __launch_bounds__(256) void purified_param_reduce_kernel(PurArgs p, int nwg, int n_scale) {
    __shared__ double red[256];
    const int out = blockIdx.x;
    const bool is_tau = out >= n_scale;
    const int o = is_tau ? out - n_scale : out;
    const bool per_head = is_tau ? (p.per_head_tau != 0) : (p.per_head_scale != 0);
    const float* part = p.part + (is_tau ? nwg : 0);
    const int BH = p.B * p.H;
    double acc = 0.0;
    for (int i = threadIdx.x; i < nwg; i += 256)
        if (!per_head || ((i % BH) % p.H) == o) acc += (double)part[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) (is_tau ? p.dtau : p.dscale)[o] = (float)red[0];
}

// Workgroups of the dK/dV kernel (the partial-sum count).
inline int purified_dkdv_groups(int B, int H, int T, int DP) {
    const int BK = (DP > 128 ? 1 : 4) * 32;
    return ((T + BK - 1) / BK) * B * H;
}

// Partial-sum slots the workspace holds for head dim DP: the most any dK/dV
// launch at that head dim writes (D = 128 with documents: 64-key blocks).
inline int purified_dkdv_groups_max(int B, int H, int T, int DP) {
    const int g = purified_dkdv_groups(B, H, T, DP);
    return DP == 128 ? max(g, ((T + 63) / 64) * B * H) : g;
}

template <class IN, int DP>
hipError_t launch_purified_fwd(const PurArgs& a, hipStream_t st) {
    using C = PurCfg<DP>;
    constexpr int BM = C::NW * 32;
    const dim3 grid((unsigned)((a.T + BM - 1) / BM) * (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((purified_fwd_kernel<IN, DP, C::NW, C::BN, C::FWD_WPE>), grid, dim3(C::NW * 64), 0, st, a);
    return hipGetLastError();
}

template <class IN, int DP>
hipError_t launch_purified_bwd(const PurArgs& a, hipStream_t st) {
    using C = PurCfg<DP>;
    const unsigned BH = (unsigned)(a.B * a.H);
    {
        int n = (a.D + 3) / 4, G = 1;
        while (G < n && G < 32) G <<= 1;
        const int64_t rows = (int64_t)a.B * a.H * a.T;
        const int per_block = 256 / G;
        hipLaunchKernelGGL((purified_delta_kernel<IN>), dim3((unsigned)((rows + per_block - 1) / per_block)), dim3(256),
                           0, st, a, G);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nwg = purified_dkdv_groups(a.B, a.H, a.T, DP);
    hipLaunchKernelGGL((purified_dkdv_kernel<IN, DP, C::KV_NW, C::BQ, C::KV_WPE, C::KV_LDS>), dim3((unsigned)nwg),
                       dim3(C::KV_NW * 64), 0, st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    constexpr int BM = C::NW * 32;
    hipLaunchKernelGGL((purified_dq_kernel<IN, DP, C::NW, C::BN, C::DQ_WPE>), dim3((unsigned)((a.T + BM - 1) / BM) * BH),
                       dim3(C::NW * 64), 0, st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int n_scale = a.per_head_scale ? a.H : 1, n_tau = a.per_head_tau ? a.H : 1;
    hipLaunchKernelGGL(purified_param_reduce_kernel<0>, dim3((unsigned)(n_scale + n_tau)), dim3(256), 0, st, a, nwg, n_scale);
    return hipGetLastError();
}

}  // namespace qdl
