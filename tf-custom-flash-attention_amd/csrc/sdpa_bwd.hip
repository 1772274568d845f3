// sdpa_bwd.hip -- backward kernels of the SdpaGrad op for gfx950.
//
// Replaces FlashAttnBwdKernel_KV, FlashAttnBwdKernel_Q and
// FlashAttnGradFunctor<GPUDevice,T> (sdpa/sdpa_bwd.cu.cc:13-453).  As in the
// reference the backward is split so that no atomics are needed:
//   1. dQ kernel   (one workgroup per query tile, loop over key blocks).  It
//      also computes delta_i = sum_d dO[i,d] * O[i,d] once per query row and
//      writes it to the caller's workspace.
//   2. dK/dV kernel (one workgroup per key tile, loop over query blocks),
//      reading delta from the workspace.
// Both recompute P = exp(score*scale - stats) from the forward's statistics.
//
// Per element (reference semantics, sdpa/sdpa_bwd.cu.cc:130-170 and :291-327):
//   P  = exp(scale * q.k - stats);      elements with P <= 1e-6 are skipped
//   kept    : P~ = P/(1-p), dS = scale * P~ * (dP - delta*(1-p))
//   dropped : P~ = 0,       dS = -scale * P * delta
//   dV += P~ dO,  dK += dS q,  dQ += dS k
// which is written here as dS = scale * P0 * (keep ? dP/(1-p) : 0 - delta)
// with P0 = (P > 1e-6 ? P : 0); the factors scale and 1/(1-p) are applied
// once when dK, dQ and dV are stored.
//
// MFMA formulation (fp16 kernels; the fp32 ones mirror it with k = 2):
//   dQ kernel, per wave of 32 queries (lane = query):
//     S^T  = K Q^T       A = K rows (LDS, b128)    B = Q   (registers)
//     dP^T = V dO^T      A = V rows (LDS, b128)    B = dO  (registers)
//     dQ^T += K^T dS^T   A = K^T (LDS transpose reads)  B = dS^T from the C layout
//   dK/dV kernel, per wave of 32 keys (lane = key):
//     S    = Q K^T       A = Q rows (LDS, b128)    B = K   (registers)
//     dP   = dO V^T      A = dO rows (LDS, b128)   B = V   (registers)
//     dV^T += dO^T P~    A = dO^T (LDS transpose)  B = P~ from the C layout
//     dK^T += Q^T dS     A = Q^T  (LDS transpose)  B = dS from the C layout
#include "sdpa_device.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"
#include "sdpa_tile.h"

namespace sdpa {

// dQ tiles: heaviest (last, under causal masking) first; see map_q_tile in
// the forward.  dK/dV tiles: under causal masking the first key tiles see the
// most queries, so the natural order is already heaviest first.
__device__ __forceinline__ void map_tile(int bid, int B, int tiles, bool reverse, int& b, int& t) {
    b = bid % B;
    const int level = bid / B;
    t = reverse ? (tiles - 1 - level) : level;
}

// ===========================================================================
// fp16
// ===========================================================================
template <int DQK, int DV>
struct BwdQF16Cfg {
    static constexpr int NT = 256, BM = 128, BN = 64;
    static constexpr int KT = BN * DQK, VT = BN * DV, STAGE = KT + VT;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE * sizeof(half_t);
    // waves per SIMD: at D_qk = 128 (with D_v >= 64) the kernel needs more
    // than 256 registers (two waves per SIMD spilled 44-148 bytes per lane in
    // the loop), so it runs one wave per SIMD with the whole register file:
    // 8-11% faster at D = 124 and 124 / 60
    static constexpr int WAVES = (DQK == 128 && DV >= 64) ? 1 : 2;
};

template <int DQK, int DV, bool VEC, bool DROP>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(BwdQF16Cfg<DQK, DV>::WAVES, BwdQF16Cfg<DQK, DV>::WAVES)))
void sdpa_bwd_dq_f16_kernel(const BwdParams p) {
    using Cfg = BwdQF16Cfg<DQK, DV>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, LK = DQK / 8, LV = DV / 8;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    half_t* lds = reinterpret_cast<half_t*>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const bool causal = p.c.causal != 0;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    map_tile(blockIdx.x, B, tiles, causal, b, qt);
    const int q0 = qt * BM, qw0 = q0 + wave * 32, my_q = qw0 + l32;
    const size_t row_q = (size_t)b * S_q + my_q;

    const half_t* Qb = static_cast<const half_t*>(p.q) + (size_t)b * S_q * D_qk;
    const half_t* Ob = static_cast<const half_t*>(p.o) + (size_t)b * S_q * D_v;
    const half_t* dOb = static_cast<const half_t*>(p.d_o) + (size_t)b * S_q * D_v;
    const half_t* Kb = static_cast<const half_t*>(p.k) + (size_t)b * S_kv * D_qk;
    const half_t* Vb = static_cast<const half_t*>(p.v) + (size_t)b * S_kv * D_v;

    half8 qreg[DQK / 16], doreg[DV / 16];
#pragma unroll
    for (int ks = 0; ks < DQK / 16; ++ks)
        qreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, VEC>(Qb, my_q, S_q, 16 * ks + 8 * hh, D_qk, D_qk));
    float dpart = 0.f;
#pragma unroll
    for (int ks = 0; ks < DV / 16; ++ks) {
        doreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, VEC>(dOb, my_q, S_q, 16 * ks + 8 * hh, D_v, D_v));
        const half8 o8 = __builtin_bit_cast(half8, load_row_chunk<half_t, VEC>(Ob, my_q, S_q, 16 * ks + 8 * hh, D_v, D_v));
#pragma unroll
        for (int e = 0; e < 8; ++e) dpart += (float)doreg[ks][e] * (float)o8[e];
    }
    const float delta = xhalf_sum(dpart);
    const bool row_ok = my_q < S_q;
    // P = exp2(fma(s, scale*log2e, -stats*log2e)); rows past S_q get P = 0.
    const float stats2 = row_ok ? p.stats[row_q] * kLog2e : INFINITY;
    if (row_ok && hh == 0) {
        p.delta[row_q] = delta;
        p.stats2[row_q] = stats2 + kGateShift;
    }
    const float sl2 = p.c.scale_log2;
    const float ksc = p.c.keep_scale;

    const int kv_end = causal ? min(S_kv, q0 + BM) : S_kv;
    const int nblk = (kv_end + BN - 1) / BN;
    const bool wave_live = qw0 < S_q;
    const int wave_last_q = min(qw0 + 31, S_q - 1);

    const uint64_t st_base = DROP ? lcg_state(p.c.seed_offset, row_q, (uint64_t)S_kv, 4 * hh) : 0;
    const uint32_t thr = p.c.drop_threshold;

    const int g16 = lane >> 4, i16 = lane & 15;
    const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
    const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);

    floatx16 dqacc[DQK / 32];
#pragma unroll
    for (int dt = 0; dt < DQK / 32; ++dt) dqacc[dt] = floatx16{};

    TileStage<half_t, BN, DQK, Cfg::NT, VEC> kst;
    TileStage<half_t, BN, DV, Cfg::NT, VEC> vst;
    if (nblk > 0) {
        kst.load(Kb, 0, S_kv, D_qk, D_qk, tid);
        vst.load(Vb, 0, S_kv, D_v, D_v, tid);
        kst.store_swz(lds, tid);
        vst.store_swz(lds + Cfg::KT, tid);
    }
    __syncthreads();

    for (int blk = 0; blk < nblk; ++blk) {
        const int kv0 = blk * BN;
        const half_t* Ks = lds + (blk & 1) * Cfg::STAGE;
        const half_t* Vs = Ks + Cfg::KT;
        const bool has_next = blk + 1 < nblk;
        if (has_next) {
            kst.load(Kb, kv0 + BN, S_kv - kv0 - BN, D_qk, D_qk, tid);
            vst.load(Vb, kv0 + BN, S_kv - kv0 - BN, D_v, D_v, tid);
        }

        if (wave_live && (!causal || kv0 <= wave_last_q)) {
            floatx16 sacc[BN / 32], dpacc[BN / 32];
#pragma unroll
            for (int t = 0; t < BN / 32; ++t) {
                sacc[t] = floatx16{};
                dpacc[t] = floatx16{};
            }
#pragma unroll
            for (int ks = 0; ks < DQK / 16; ++ks)
#pragma unroll
                for (int t = 0; t < BN / 32; ++t) {
                    const half8 a = *reinterpret_cast<const half8*>(Ks + swz_off<LK>(32 * t + l32, 16 * ks + 8 * hh));
                    sacc[t] = mfma_f16(a, qreg[ks], sacc[t]);
                }
#pragma unroll
            for (int ks = 0; ks < DV / 16; ++ks)
#pragma unroll
                for (int t = 0; t < BN / 32; ++t) {
                    const half8 a = *reinterpret_cast<const half8*>(Vs + swz_off<LV>(32 * t + l32, 16 * ks + 8 * hh));
                    dpacc[t] = mfma_f16(a, doreg[ks], dpacc[t]);
                }

            const bool need_mask = (kv0 + BN > S_kv) || (causal && kv0 + BN - 1 > qw0);
            const uint64_t st_blk = DROP ? st_base + (uint64_t)kv0 * kLcgMul : 0;
            half8 dsb[BN / 16];
#pragma unroll
            for (int t = 0; t < BN / 32; ++t) {
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    float ds2[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int rr = r + e;
                        float x = __builtin_fmaf(sacc[t][rr], sl2, -stats2);
                        if (need_mask) {
                            const int key = kv0 + 32 * t + 8 * (rr >> 2) + 4 * hh + (rr & 3);
                            if (key >= S_kv || (causal && key > my_q)) x = -INFINITY;
                        }
                        const float pr = fast_exp2(x);
                        const float p0 = pr > kEps ? pr : 0.f;
                        float dpk = DROP ? dpacc[t][rr] * ksc : dpacc[t][rr];
                        if constexpr (DROP) {
                            const uint64_t off = (uint64_t)(32 * t + 8 * (rr >> 2) + (rr & 3)) * kLcgMul;
                            dpk = lcg_keep(st_blk + off, thr) ? dpk : 0.f;
                        }
                        ds2[e] = p0 * (dpk - delta);
                    }
                    const half2v h = cvt_pk(ds2[0], ds2[1]);
                    const int s = 2 * t + (r >> 3), i = r & 7;
                    dsb[s][i] = h[0];
                    dsb[s][i + 1] = h[1];
                }
            }
#pragma unroll
            for (int s = 0; s < BN / 16; ++s)
#pragma unroll
                for (int dt = 0; dt < DQK / 32; ++dt) {
                    const half4 a0 = lds_read_tr(Ks + swz_off<LK>(16 * s + tr_row, 32 * dt + tr_col));
                    const half4 a1 = lds_read_tr(Ks + swz_off<LK>(16 * s + 8 + tr_row, 32 * dt + tr_col));
                    const half8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
                    dqacc[dt] = mfma_f16(a, dsb[s], dqacc[dt]);
                }
        }

        if (has_next) {
            half_t* Kn = lds + ((blk + 1) & 1) * Cfg::STAGE;
            kst.store_swz(Kn, tid);
            vst.store_swz(Kn + Cfg::KT, tid);
        }
        __syncthreads();
    }

    if (row_ok) {
        const float sc = p.c.scale;
        half_t* dQb = static_cast<half_t*>(p.dq) + row_q * D_qk;
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                half4 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[e] = (half_t)(dqacc[dt][4 * g4 + e] * sc);
                if constexpr (VEC) {
                    if (d0 < D_qk) *reinterpret_cast<half4*>(dQb + d0) = hv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_qk) dQb[d0 + e] = hv[e];
                }
            }
    }
}

template <int DQK, int DV>
struct BwdKVF16Cfg {
    static constexpr int NT = 256, BKV = 128, BQ = 32;
    static constexpr int QT = BQ * DQK, OT = BQ * DV;            // halves
    static constexpr int STAGE_BYTES = (QT + OT) * 2 + 2 * BQ * 4;  // + stats2[BQ], delta[BQ]
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE_BYTES;
    // one wave per SIMD at D_qk = D_v = 128, where K, V, dK and dV of a
    // 32-key group do not fit 256 registers (two waves spilled 148-184 bytes
    // per lane in the loop; one wave is 23% faster at D = 124).  At 128 / 64
    // two waves spill 20-44 bytes and are still 2.5% faster than one.
    static constexpr int WAVES = (DQK == 128 && DV == 128) ? 1 : 2;
};

template <int DQK, int DV, bool VEC, bool DROP>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(BwdKVF16Cfg<DQK, DV>::WAVES, BwdKVF16Cfg<DQK, DV>::WAVES)))
void sdpa_bwd_dkdv_f16_kernel(const BwdParams p) {
    using Cfg = BwdKVF16Cfg<DQK, DV>;
    constexpr int BKV = Cfg::BKV, BQ = Cfg::BQ, LQ = DQK / 8, LO = DV / 8;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const bool causal = p.c.causal != 0;
    const int tiles = (S_kv + BKV - 1) / BKV;
    int b, kt;
    map_tile(blockIdx.x, B, tiles, false, b, kt);
    const int k0 = kt * BKV, kw0 = k0 + wave * 32, my_k = kw0 + l32;
    const bool key_ok = my_k < S_kv;

    const half_t* Qb = static_cast<const half_t*>(p.q) + (size_t)b * S_q * D_qk;
    const half_t* dOb = static_cast<const half_t*>(p.d_o) + (size_t)b * S_q * D_v;
    const half_t* Kb = static_cast<const half_t*>(p.k) + (size_t)b * S_kv * D_qk;
    const half_t* Vb = static_cast<const half_t*>(p.v) + (size_t)b * S_kv * D_v;
    const float* statsb = p.stats + (size_t)b * S_q;
    const float* deltab = p.delta + (size_t)b * S_q;

    // K and V rows of this lane's key as B operands (lane = key, features in-lane).
    half8 kreg[DQK / 16], vreg[DV / 16];
#pragma unroll
    for (int ks = 0; ks < DQK / 16; ++ks)
        kreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, VEC>(Kb, my_k, S_kv, 16 * ks + 8 * hh, D_qk, D_qk));
#pragma unroll
    for (int ks = 0; ks < DV / 16; ++ks)
        vreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, VEC>(Vb, my_k, S_kv, 16 * ks + 8 * hh, D_v, D_v));
    prologue_loads_landed();

    // Queries below k0 see none of these keys under the causal mask.
    const int q_begin = causal ? (min(k0, S_q) / BQ) * BQ : 0;
    const int nblk = (S_q - q_begin + BQ - 1) / BQ;
    const bool wave_live = kw0 < S_kv;

    const float sl2 = p.c.scale_log2;
    const float ksc = p.c.keep_scale;
    // Dropout: st(q, key) = st(4*hh, key) + (q - 4*hh) * S_kv * A.  The row
    // step S_kv*A is wave-uniform.
    const uint64_t st_base = DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + 4 * hh, (uint64_t)S_kv, my_k) : 0;
    const uint64_t row_step = (uint64_t)S_kv * kLcgMul;
    const uint32_t thr = p.c.drop_threshold;

    const int g16 = lane >> 4, i16 = lane & 15;
    const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
    const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);

    floatx16 dkacc[DQK / 32], dvacc[DV / 32];
#pragma unroll
    for (int dt = 0; dt < DQK / 32; ++dt) dkacc[dt] = floatx16{};
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt) dvacc[dt] = floatx16{};

    auto stage_q = [&](int s) { return reinterpret_cast<half_t*>(smem + s * Cfg::STAGE_BYTES); };
    auto stage_o = [&](int s) { return reinterpret_cast<half_t*>(smem + s * Cfg::STAGE_BYTES) + Cfg::QT; };
    auto stage_f = [&](int s) {
        return reinterpret_cast<float*>(smem + s * Cfg::STAGE_BYTES + (Cfg::QT + Cfg::OT) * 2);
    };

    TileStage<half_t, BQ, DQK, Cfg::NT, VEC> qst;
    TileStage<half_t, BQ, DV, Cfg::NT, VEC> ost;
    float fpre = 0.f;  // threads 0..BQ-1: stats2 of row q0+tid; BQ..2BQ-1: delta of row q0+tid-BQ
    auto load_rows = [&](int q0) {
        qst.load(Qb, q0, S_q - q0, D_qk, D_qk, tid);
        ost.load(dOb, q0, S_q - q0, D_v, D_v, tid);
        if (tid < 2 * BQ) {
            const int r = q0 + (tid & (BQ - 1));
            if (tid < BQ) fpre = r < S_q ? statsb[r] * kLog2e : INFINITY;
            else fpre = r < S_q ? deltab[r] : 0.f;
        }
    };
    auto store_rows = [&](int s) {
        qst.store_swz(stage_q(s), tid);
        ost.store_swz(stage_o(s), tid);
        if (tid < 2 * BQ) stage_f(s)[tid] = fpre;
    };

    if (nblk > 0) {
        load_rows(q_begin);
        store_rows(0);
    }
    __syncthreads();

    for (int blk = 0; blk < nblk; ++blk) {
        const int q0 = q_begin + blk * BQ;
        const int cur = blk & 1;
        const half_t* Qs = stage_q(cur);
        const half_t* dOs = stage_o(cur);
        const float* Fs = stage_f(cur);
        const bool has_next = blk + 1 < nblk;
        if (has_next) load_rows(q0 + BQ);

        if (wave_live && (!causal || q0 + BQ - 1 >= kw0)) {
            floatx16 sacc[BQ / 32], dpacc[BQ / 32];
#pragma unroll
            for (int t = 0; t < BQ / 32; ++t) {
                sacc[t] = floatx16{};
                dpacc[t] = floatx16{};
            }
#pragma unroll
            for (int ks = 0; ks < DQK / 16; ++ks)
#pragma unroll
                for (int t = 0; t < BQ / 32; ++t) {
                    const half8 a = *reinterpret_cast<const half8*>(Qs + swz_off<LQ>(32 * t + l32, 16 * ks + 8 * hh));
                    sacc[t] = mfma_f16(a, kreg[ks], sacc[t]);
                }
#pragma unroll
            for (int ks = 0; ks < DV / 16; ++ks)
#pragma unroll
                for (int t = 0; t < BQ / 32; ++t) {
                    const half8 a = *reinterpret_cast<const half8*>(dOs + swz_off<LO>(32 * t + l32, 16 * ks + 8 * hh));
                    dpacc[t] = mfma_f16(a, vreg[ks], dpacc[t]);
                }

            const bool need_mask = !key_ok || (causal && q0 < kw0 + 31);
            const uint64_t st_blk = DROP ? st_base + (uint64_t)q0 * row_step : 0;
            half8 pkb[BQ / 16], dsb[BQ / 16];
#pragma unroll
            for (int t = 0; t < BQ / 32; ++t) {
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    // rows 32t + 8*g4 + 4*hh + 0..3 of the block: stats2 and delta as float4 broadcasts
                    const int rb = 32 * t + 8 * g4 + 4 * hh;
                    const floatx4 st4 = *reinterpret_cast<const floatx4*>(Fs + rb);
                    const floatx4 de4 = *reinterpret_cast<const floatx4*>(Fs + BQ + rb);
                    float pk4[4], ds4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int rr = 4 * g4 + e;
                        float x = __builtin_fmaf(sacc[t][rr], sl2, -st4[e]);
                        if (need_mask) {
                            const int q = q0 + rb + e;
                            if (!key_ok || (causal && my_k > q)) x = -INFINITY;
                        }
                        const float pr = fast_exp2(x);
                        const float p0 = pr > kEps ? pr : 0.f;
                        float dpk = DROP ? dpacc[t][rr] * ksc : dpacc[t][rr];
                        float pk = p0;
                        if constexpr (DROP) {
                            const uint64_t off = (uint64_t)(32 * t + 8 * g4 + e) * row_step;
                            const bool keep = lcg_keep(st_blk + off, thr);
                            dpk = keep ? dpk : 0.f;
                            pk = keep ? p0 : 0.f;
                        }
                        pk4[e] = pk;
                        ds4[e] = p0 * (dpk - de4[e]);
                    }
                    const int s = 2 * t + (g4 >> 1), i = 4 * (g4 & 1);
                    const half2v h0 = cvt_pk(pk4[0], pk4[1]), h1 = cvt_pk(pk4[2], pk4[3]);
                    const half2v d0 = cvt_pk(ds4[0], ds4[1]), d1 = cvt_pk(ds4[2], ds4[3]);
                    pkb[s][i] = h0[0];
                    pkb[s][i + 1] = h0[1];
                    pkb[s][i + 2] = h1[0];
                    pkb[s][i + 3] = h1[1];
                    dsb[s][i] = d0[0];
                    dsb[s][i + 1] = d0[1];
                    dsb[s][i + 2] = d1[0];
                    dsb[s][i + 3] = d1[1];
                }
            }
#pragma unroll
            for (int s = 0; s < BQ / 16; ++s) {
#pragma unroll
                for (int dt = 0; dt < DV / 32; ++dt) {
                    const half4 a0 = lds_read_tr(dOs + swz_off<LO>(16 * s + tr_row, 32 * dt + tr_col));
                    const half4 a1 = lds_read_tr(dOs + swz_off<LO>(16 * s + 8 + tr_row, 32 * dt + tr_col));
                    const half8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
                    dvacc[dt] = mfma_f16(a, pkb[s], dvacc[dt]);
                }
#pragma unroll
                for (int dt = 0; dt < DQK / 32; ++dt) {
                    const half4 a0 = lds_read_tr(Qs + swz_off<LQ>(16 * s + tr_row, 32 * dt + tr_col));
                    const half4 a1 = lds_read_tr(Qs + swz_off<LQ>(16 * s + 8 + tr_row, 32 * dt + tr_col));
                    const half8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
                    dkacc[dt] = mfma_f16(a, dsb[s], dkacc[dt]);
                }
            }
        }

        if (has_next) store_rows(cur ^ 1);
        __syncthreads();
    }

    if (key_ok) {
        const float sc = p.c.scale;
        half_t* dKb = static_cast<half_t*>(p.dk) + ((size_t)b * S_kv + my_k) * D_qk;
        half_t* dVb = static_cast<half_t*>(p.dv) + ((size_t)b * S_kv + my_k) * D_v;
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                half4 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[e] = (half_t)(dkacc[dt][4 * g4 + e] * sc);
                if constexpr (VEC) {
                    if (d0 < D_qk) *reinterpret_cast<half4*>(dKb + d0) = hv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_qk) dKb[d0 + e] = hv[e];
                }
            }
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                half4 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[e] = (half_t)(dvacc[dt][4 * g4 + e] * ksc);
                if constexpr (VEC) {
                    if (d0 < D_v) *reinterpret_cast<half4*>(dVb + d0) = hv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_v) dVb[d0 + e] = hv[e];
                }
            }
    }
}

// ===========================================================================
// fp32 (v_mfma_f32_32x32x2_f32).  Feature reductions are split between the
// half-waves (lane-half h covers features [h*D/2, (h+1)*D/2)) so operands are
// read as float4 runs; reductions over keys/queries pair k-step r of
// lane-half h with row 8*(r/4) + 4h + r%4 of the 32-row accumulator tile.
// ===========================================================================
template <int DQK, int DV>
struct BwdQF32Cfg {
    static constexpr int NT = 256, BM = 128, BN = 32;
    static constexpr int KS = DQK + 4, VS = DV + 4;
    static constexpr int KT = BN * KS, VT = BN * VS, STAGE = KT + VT;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE * sizeof(float);
    // one wave per SIMD where two spilled in the loop: D_qk = D_v = 128
    // (184-228 bytes per lane; one wave 19% faster), and D_qk = 128 / D_v =
    // 64 with the generic row loads (40-56 bytes; 3% faster).  Aligned 128 /
    // 64 with dropout keeps two waves: 20 bytes of spill, 4.6% faster than
    // one; c5's shape (aligned, no dropout) fits two waves.
    template <bool VEC, bool DROP>
    static constexpr int waves() { return (DQK == 128 && (DV == 128 || (DV == 64 && !VEC))) ? 1 : 2; }
};

template <int DQK, int DV, bool VEC, bool DROP>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(BwdQF32Cfg<DQK, DV>::template waves<VEC, DROP>(),
                                   BwdQF32Cfg<DQK, DV>::template waves<VEC, DROP>())))
void sdpa_bwd_dq_f32_kernel(const BwdParams p) {
    using Cfg = BwdQF32Cfg<DQK, DV>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, KS = Cfg::KS, VS = Cfg::VS;
    constexpr int HQ = DQK / 2, HV = DV / 2;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    float* lds = reinterpret_cast<float*>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const bool causal = p.c.causal != 0;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    map_tile(blockIdx.x, B, tiles, causal, b, qt);
    const int q0 = qt * BM, qw0 = q0 + wave * 32, my_q = qw0 + l32;
    const size_t row_q = (size_t)b * S_q + my_q;

    const float* Qb = static_cast<const float*>(p.q) + (size_t)b * S_q * D_qk;
    const float* Ob = static_cast<const float*>(p.o) + (size_t)b * S_q * D_v;
    const float* dOb = static_cast<const float*>(p.d_o) + (size_t)b * S_q * D_v;
    const float* Kb = static_cast<const float*>(p.k) + (size_t)b * S_kv * D_qk;
    const float* Vb = static_cast<const float*>(p.v) + (size_t)b * S_kv * D_v;

    float qf[HQ], dof[HV];
    float dpart = 0.f;
#pragma unroll
    for (int u = 0; u < HQ / 4; ++u) {
        const floatx4 f = __builtin_bit_cast(floatx4, load_row_chunk<float, VEC>(Qb, my_q, S_q, HQ * hh + 4 * u, D_qk, D_qk));
#pragma unroll
        for (int e = 0; e < 4; ++e) qf[4 * u + e] = f[e];
    }
#pragma unroll
    for (int u = 0; u < HV / 4; ++u) {
        const floatx4 f = __builtin_bit_cast(floatx4, load_row_chunk<float, VEC>(dOb, my_q, S_q, HV * hh + 4 * u, D_v, D_v));
        const floatx4 o = __builtin_bit_cast(floatx4, load_row_chunk<float, VEC>(Ob, my_q, S_q, HV * hh + 4 * u, D_v, D_v));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dof[4 * u + e] = f[e];
            dpart += f[e] * o[e];
        }
    }
    const float delta = xhalf_sum(dpart);
    const bool row_ok = my_q < S_q;
    const float stats2 = row_ok ? p.stats[row_q] * kLog2e : INFINITY;
    if (row_ok && hh == 0) {
        p.delta[row_q] = delta;
        p.stats2[row_q] = stats2 + kGateShift;
    }
    const float sl2 = p.c.scale_log2;
    const float ksc = p.c.keep_scale;

    const int kv_end = causal ? min(S_kv, q0 + BM) : S_kv;
    const int nblk = (kv_end + BN - 1) / BN;
    const bool wave_live = qw0 < S_q;
    const int wave_last_q = min(qw0 + 31, S_q - 1);
    const uint64_t st_base = DROP ? lcg_state(p.c.seed_offset, row_q, (uint64_t)S_kv, 4 * hh) : 0;
    const uint32_t thr = p.c.drop_threshold;

    floatx16 dqacc[DQK / 32];
#pragma unroll
    for (int dt = 0; dt < DQK / 32; ++dt) dqacc[dt] = floatx16{};

    TileStage<float, BN, DQK, Cfg::NT, VEC> kst;
    TileStage<float, BN, DV, Cfg::NT, VEC> vst;
    if (nblk > 0) {
        kst.load(Kb, 0, S_kv, D_qk, D_qk, tid);
        vst.load(Vb, 0, S_kv, D_v, D_v, tid);
        kst.template store<KS>(lds, tid);
        vst.template store<VS>(lds + Cfg::KT, tid);
    }
    __syncthreads();

    for (int blk = 0; blk < nblk; ++blk) {
        const int kv0 = blk * BN;
        const float* Ks = lds + (blk & 1) * Cfg::STAGE;
        const float* Vs = Ks + Cfg::KT;
        const bool has_next = blk + 1 < nblk;
        float* Kn = lds + ((blk + 1) & 1) * Cfg::STAGE;
        // The next block is staged in two halves (V, then K) so that only one
        // of them occupies registers at a time; the other buffer was released
        // by every wave at the previous iteration's barrier.
        if (has_next) vst.load(Vb, kv0 + BN, S_kv - kv0 - BN, D_v, D_v, tid);
        const bool live = wave_live && (!causal || kv0 <= wave_last_q);
        floatx16 sacc = floatx16{}, dpacc = floatx16{};
        if (live) {
#pragma unroll
            for (int u = 0; u < HQ / 4; ++u) {
                const floatx4 kk = *reinterpret_cast<const floatx4*>(Ks + l32 * KS + HQ * hh + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; ++e) sacc = mfma_f32(kk[e], qf[4 * u + e], sacc);
            }
#pragma unroll
            for (int u = 0; u < HV / 4; ++u) {
                const floatx4 vv = *reinterpret_cast<const floatx4*>(Vs + l32 * VS + HV * hh + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; ++e) dpacc = mfma_f32(vv[e], dof[4 * u + e], dpacc);
            }
        }
        if (has_next) {
            vst.template store<VS>(Kn + Cfg::KT, tid);
            kst.load(Kb, kv0 + BN, S_kv - kv0 - BN, D_qk, D_qk, tid);
        }
        if (live) {
            const bool need_mask = (kv0 + BN > S_kv) || (causal && kv0 + BN - 1 > qw0);
            const uint64_t st_blk = DROP ? st_base + (uint64_t)kv0 * kLcgMul : 0;
            float ds[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = __builtin_fmaf(sacc[r], sl2, -stats2);
                if (need_mask) {
                    const int key = kv0 + 8 * (r >> 2) + 4 * hh + (r & 3);
                    if (key >= S_kv || (causal && key > my_q)) x = -INFINITY;
                }
                const float pr = fast_exp2(x);
                const float p0 = pr > kEps ? pr : 0.f;
                float dpk = DROP ? dpacc[r] * ksc : dpacc[r];
                if constexpr (DROP) {
                    const uint64_t off = (uint64_t)(8 * (r >> 2) + (r & 3)) * kLcgMul;
                    dpk = lcg_keep(st_blk + off, thr) ? dpk : 0.f;
                }
                ds[r] = p0 * (dpk - delta);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r)
#pragma unroll
                for (int dt = 0; dt < DQK / 32; ++dt) {
                    const float a = Ks[(8 * (r >> 2) + 4 * hh + (r & 3)) * KS + 32 * dt + l32];
                    dqacc[dt] = mfma_f32(a, ds[r], dqacc[dt]);
                }
        }

        if (has_next) kst.template store<KS>(Kn, tid);
        __syncthreads();
    }

    if (row_ok) {
        const float sc = p.c.scale;
        float* dQb = static_cast<float*>(p.dq) + row_q * D_qk;
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                floatx4 fv;
#pragma unroll
                for (int e = 0; e < 4; ++e) fv[e] = dqacc[dt][4 * g4 + e] * sc;
                if constexpr (VEC) {
                    if (d0 < D_qk) *reinterpret_cast<floatx4*>(dQb + d0) = fv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_qk) dQb[d0 + e] = fv[e];
                }
            }
    }
}

template <int DQK, int DV>
struct BwdKVF32Cfg {
    static constexpr int NT = 256, BKV = 128, BQ = 32;
    static constexpr int QS = DQK + 4, OS = DV + 4;
    static constexpr int QT = BQ * QS, OT = BQ * OS;
    static constexpr int STAGE = QT + OT + 2 * BQ;  // floats: Q, dO, stats2, delta
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE * sizeof(float);
};

template <int DQK, int DV, bool VEC, bool DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_bwd_dkdv_f32_kernel(const BwdParams p) {
    using Cfg = BwdKVF32Cfg<DQK, DV>;
    constexpr int BKV = Cfg::BKV, BQ = Cfg::BQ, QS = Cfg::QS, OS = Cfg::OS;
    constexpr int HQ = DQK / 2, HV = DV / 2;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    float* lds = reinterpret_cast<float*>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const bool causal = p.c.causal != 0;
    const int tiles = (S_kv + BKV - 1) / BKV;
    int b, kt;
    map_tile(blockIdx.x, B, tiles, false, b, kt);
    const int k0 = kt * BKV, kw0 = k0 + wave * 32, my_k = kw0 + l32;
    const bool key_ok = my_k < S_kv;

    const float* Qb = static_cast<const float*>(p.q) + (size_t)b * S_q * D_qk;
    const float* dOb = static_cast<const float*>(p.d_o) + (size_t)b * S_q * D_v;
    const float* Kb = static_cast<const float*>(p.k) + (size_t)b * S_kv * D_qk;
    const float* Vb = static_cast<const float*>(p.v) + (size_t)b * S_kv * D_v;
    const float* statsb = p.stats + (size_t)b * S_q;
    const float* deltab = p.delta + (size_t)b * S_q;

    float kf[HQ], vf[HV];
#pragma unroll
    for (int u = 0; u < HQ / 4; ++u) {
        const floatx4 f = __builtin_bit_cast(floatx4, load_row_chunk<float, VEC>(Kb, my_k, S_kv, HQ * hh + 4 * u, D_qk, D_qk));
#pragma unroll
        for (int e = 0; e < 4; ++e) kf[4 * u + e] = f[e];
    }
#pragma unroll
    for (int u = 0; u < HV / 4; ++u) {
        const floatx4 f = __builtin_bit_cast(floatx4, load_row_chunk<float, VEC>(Vb, my_k, S_kv, HV * hh + 4 * u, D_v, D_v));
#pragma unroll
        for (int e = 0; e < 4; ++e) vf[4 * u + e] = f[e];
    }
    prologue_loads_landed();

    const int q_begin = causal ? (min(k0, S_q) / BQ) * BQ : 0;
    const int nblk = (S_q - q_begin + BQ - 1) / BQ;
    const bool wave_live = kw0 < S_kv;
    const float sl2 = p.c.scale_log2;
    const float ksc = p.c.keep_scale;
    const uint64_t st_base = DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + 4 * hh, (uint64_t)S_kv, my_k) : 0;
    const uint64_t row_step = (uint64_t)S_kv * kLcgMul;
    const uint32_t thr = p.c.drop_threshold;

    floatx16 dkacc[DQK / 32], dvacc[DV / 32];
#pragma unroll
    for (int dt = 0; dt < DQK / 32; ++dt) dkacc[dt] = floatx16{};
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt) dvacc[dt] = floatx16{};

    TileStage<float, BQ, DQK, Cfg::NT, VEC> qst;
    TileStage<float, BQ, DV, Cfg::NT, VEC> ost;
    float fpre = 0.f;
    auto load_rows = [&](int q0) {
        qst.template load<false>(Qb, q0, S_q - q0, D_qk, D_qk, tid);
        ost.template load<false>(dOb, q0, S_q - q0, D_v, D_v, tid);
        if (tid < 2 * BQ) {
            const int r = q0 + (tid & (BQ - 1));
            if (tid < BQ) fpre = r < S_q ? statsb[r] * kLog2e : INFINITY;
            else fpre = r < S_q ? deltab[r] : 0.f;
        }
    };
    auto store_rows = [&](int s) {
        float* base = lds + s * Cfg::STAGE;
        qst.template store<QS>(base, tid);
        ost.template store<OS>(base + Cfg::QT, tid);
        if (tid < 2 * BQ) base[Cfg::QT + Cfg::OT + tid] = fpre;
    };

    if (nblk > 0) {
        load_rows(q_begin);
        store_rows(0);
    }
    __syncthreads();

    for (int blk = 0; blk < nblk; ++blk) {
        const int q0 = q_begin + blk * BQ;
        const int cur = blk & 1;
        const float* Qs = lds + cur * Cfg::STAGE;
        const float* dOs = Qs + Cfg::QT;
        const float* Fs = dOs + Cfg::OT;
        const bool has_next = blk + 1 < nblk;
        if (has_next) load_rows(q0 + BQ);

        if (wave_live && (!causal || q0 + BQ - 1 >= kw0)) {
            floatx16 sacc = floatx16{}, dpacc = floatx16{};
#pragma unroll
            for (int u = 0; u < HQ / 4; ++u) {
                const floatx4 qq = *reinterpret_cast<const floatx4*>(Qs + l32 * QS + HQ * hh + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; ++e) sacc = mfma_f32(qq[e], kf[4 * u + e], sacc);
            }
#pragma unroll
            for (int u = 0; u < HV / 4; ++u) {
                const floatx4 oo = *reinterpret_cast<const floatx4*>(dOs + l32 * OS + HV * hh + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; ++e) dpacc = mfma_f32(oo[e], vf[4 * u + e], dpacc);
            }
            const bool need_mask = !key_ok || (causal && q0 < kw0 + 31);
            const uint64_t st_blk = DROP ? st_base + (uint64_t)q0 * row_step : 0;
            float pk[16], ds[16];
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int rb = 8 * g4 + 4 * hh;
                const floatx4 st4 = *reinterpret_cast<const floatx4*>(Fs + rb);
                const floatx4 de4 = *reinterpret_cast<const floatx4*>(Fs + BQ + rb);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * g4 + e;
                    float x = __builtin_fmaf(sacc[r], sl2, -st4[e]);
                    if (need_mask) {
                        const int q = q0 + rb + e;
                        if (!key_ok || (causal && my_k > q)) x = -INFINITY;
                    }
                    const float pr = fast_exp2(x);
                    const float p0 = pr > kEps ? pr : 0.f;
                    float dpk = DROP ? dpacc[r] * ksc : dpacc[r];
                    float pkk = p0;
                    if constexpr (DROP) {
                        const uint64_t off = (uint64_t)(8 * g4 + e) * row_step;
                        const bool keep = lcg_keep(st_blk + off, thr);
                        dpk = keep ? dpk : 0.f;
                        pkk = keep ? p0 : 0.f;
                    }
                    pk[r] = pkk;
                    ds[r] = p0 * (dpk - de4[e]);
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qrow = 8 * (r >> 2) + 4 * hh + (r & 3);
#pragma unroll
                for (int dt = 0; dt < DV / 32; ++dt)
                    dvacc[dt] = mfma_f32(dOs[qrow * OS + 32 * dt + l32], pk[r], dvacc[dt]);
#pragma unroll
                for (int dt = 0; dt < DQK / 32; ++dt)
                    dkacc[dt] = mfma_f32(Qs[qrow * QS + 32 * dt + l32], ds[r], dkacc[dt]);
            }
        }

        if (has_next) store_rows(cur ^ 1);
        __syncthreads();
    }

    if (key_ok) {
        const float sc = p.c.scale;
        float* dKb = static_cast<float*>(p.dk) + ((size_t)b * S_kv + my_k) * D_qk;
        float* dVb = static_cast<float*>(p.dv) + ((size_t)b * S_kv + my_k) * D_v;
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                floatx4 fv;
#pragma unroll
                for (int e = 0; e < 4; ++e) fv[e] = dkacc[dt][4 * g4 + e] * sc;
                if constexpr (VEC) {
                    if (d0 < D_qk) *reinterpret_cast<floatx4*>(dKb + d0) = fv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_qk) dKb[d0 + e] = fv[e];
                }
            }
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                floatx4 fv;
#pragma unroll
                for (int e = 0; e < 4; ++e) fv[e] = dvacc[dt][4 * g4 + e] * ksc;
                if constexpr (VEC) {
                    if (d0 < D_v) *reinterpret_cast<floatx4*>(dVb + d0) = fv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_v) dVb[d0 + e] = fv[e];
                }
            }
    }
}

// ---------------------------------------------------------------------------
// fp32 dK/dV with a 128-wide side: split roles.  One wave holding K, V, dK
// and dV of 32 keys (plus S, dP and the staged tiles) needs more than 256
// registers at D = 128, so each group of 32 keys gets two waves:
//   P role  (waves 0-3): S = Q K^T, P~, dV^T += dO^T P~; P goes to LDS with
//                        the dropout decision in its sign;
//   dS role (waves 4-7): dP = dO V^T, dS from the partner's P, dK^T += Q^T dS,
//                        one query block behind.
// Eight waves share one workgroup barrier per block of 32 queries.  Blocks
// pass through a ring of three LDS stages: in period n the P role reads
// block n, the dS role block n - 1, and all 512 threads stage block n + 1
// through registers into the third.  P of block m is exchanged through the
// buffer m & 1 (written in period m, read in period m + 1).
// ---------------------------------------------------------------------------
#ifndef SDPA_F32_SPLIT
#define SDPA_F32_SPLIT 1
#endif
template <int DQK, int DV>
struct BwdKVF32SplitCfg {
    static constexpr int NT = 512, BKV = 128, BQ = 32, NSTAGE = 3;
    static constexpr int QS = DQK + 4, OS = DV + 4;
    static constexpr int QT = BQ * QS, OT = BQ * OS;
    static constexpr int STAGE = QT + OT + 2 * BQ;  // floats: Q, dO, stats2, delta
    static constexpr int XB = 4 * 32 * 32;          // floats: P of 4 key groups x 32 queries
    static constexpr size_t LDS_BYTES = (NSTAGE * (size_t)STAGE + 2 * (size_t)XB) * sizeof(float);
    static_assert(LDS_BYTES <= 160 * 1024, "one workgroup per CU");
};

template <int DQK, int DV, bool VEC, bool DROP, bool DS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_bwd_dkdv_f32_split_kernel(const BwdParams p) {
    using Cfg = BwdKVF32SplitCfg<DQK, DV>;
    constexpr int BKV = Cfg::BKV, BQ = Cfg::BQ, QS = Cfg::QS, OS = Cfg::OS, NSTAGE = Cfg::NSTAGE;
    constexpr int HQ = DQK / 2, HV = DV / 2;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    float* lds = reinterpret_cast<float*>(smem);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), kw = wave & 3;
    const int l32 = lane & 31, hh = lane >> 5;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const bool causal = p.c.causal != 0;
    const int tiles = (S_kv + BKV - 1) / BKV;
    int b, kt;
    map_tile(blockIdx.x, B, tiles, false, b, kt);
    const int k0 = kt * BKV, kw0 = k0 + kw * 32, my_k = kw0 + l32;
    const bool key_ok = my_k < S_kv;

    const float* Qb = static_cast<const float*>(p.q) + (size_t)b * S_q * D_qk;
    const float* dOb = static_cast<const float*>(p.d_o) + (size_t)b * S_q * D_v;
    const float* statsb = p.stats + (size_t)b * S_q;
    const float* deltab = p.delta + (size_t)b * S_q;

    const int q_begin = causal ? (min(k0, S_q) / BQ) * BQ : 0;
    const int nblk = (S_q - q_begin + BQ - 1) / BQ;
    const bool wave_live = kw0 < S_kv;
    // Block m is skipped by both roles when the key group sees none of it.
    auto live = [&](int q0) { return wave_live && (!causal || q0 + BQ - 1 >= kw0); };
    const float sl2 = p.c.scale_log2;
    const float ksc = p.c.keep_scale;

    TileStage<float, BQ, DQK, Cfg::NT, VEC> qst;
    TileStage<float, BQ, DV, Cfg::NT, VEC> ost;
    float fpre = 0.f;
    auto load_rows = [&](int q0) {
        qst.load(Qb, q0, S_q - q0, D_qk, D_qk, tid);
        ost.load(dOb, q0, S_q - q0, D_v, D_v, tid);
        if (tid < 2 * BQ) {
            const int r = q0 + (tid & (BQ - 1));
            if (tid < BQ) fpre = r < S_q ? statsb[r] * kLog2e : INFINITY;
            else fpre = r < S_q ? deltab[r] : 0.f;
        }
    };
    auto store_rows = [&](int s) {
        float* base = lds + s * Cfg::STAGE;
        qst.template store<QS>(base, tid);
        ost.template store<OS>(base + Cfg::QT, tid);
        if (tid < 2 * BQ) base[Cfg::QT + Cfg::OT + tid] = fpre;
    };
    // P of block m for this key group: 16 floats per lane, lane-contiguous.
    auto xbuf = [&](int m) { return lds + NSTAGE * Cfg::STAGE + (m & 1) * Cfg::XB + kw * 1024; };

    if (nblk > 0) {
        load_rows(q_begin);
        store_rows(0);
    }

    if (wave < 4) {
        // ------------------------------------------------------------ P role
        const float* Kb = static_cast<const float*>(p.k) + (size_t)b * S_kv * D_qk;
        float kf[HQ];
#pragma unroll
        for (int u = 0; u < HQ / 4; ++u) {
            const floatx4 f = __builtin_bit_cast(floatx4, load_row_chunk<float, VEC>(Kb, my_k, S_kv, HQ * hh + 4 * u, D_qk, D_qk));
#pragma unroll
            for (int e = 0; e < 4; ++e) kf[4 * u + e] = f[e];
        }
        prologue_loads_landed();
        const uint64_t st_base = DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + 4 * hh, (uint64_t)S_kv, my_k) : 0;
        const uint64_t row_step = (uint64_t)S_kv * kLcgMul;
        const uint32_t thr = p.c.drop_threshold;
        floatx16 dvacc[DV / 32];
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt) dvacc[dt] = floatx16{};

        for (int n = 0; n <= nblk; ++n) {
            __syncthreads();
            const bool has_next = n + 1 < nblk;
            if (has_next) load_rows(q_begin + (n + 1) * BQ);
            const int q0 = q_begin + n * BQ;
            if (n < nblk && live(q0)) {
                const float* Qs = lds + (n % NSTAGE) * Cfg::STAGE;
                const float* dOs = Qs + Cfg::QT;
                const float* Fs = dOs + Cfg::OT;
                floatx16 sacc = floatx16{};
#pragma unroll
                for (int u = 0; u < HQ / 4; ++u) {
                    const floatx4 qq = *reinterpret_cast<const floatx4*>(Qs + l32 * QS + HQ * hh + 4 * u);
#pragma unroll
                    for (int e = 0; e < 4; ++e) sacc = mfma_f32(qq[e], kf[4 * u + e], sacc);
                }
                const bool need_mask = !key_ok || (causal && q0 < kw0 + 31);
                const uint64_t st_blk = DROP ? st_base + (uint64_t)q0 * row_step : 0;
                float* xs = xbuf(n);
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int rb = 8 * g4 + 4 * hh;
                    const floatx4 st4 = *reinterpret_cast<const floatx4*>(Fs + rb);
                    floatx4 xv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * g4 + e;
                        float x = __builtin_fmaf(sacc[r], sl2, -st4[e]);
                        if (need_mask) {
                            const int q = q0 + rb + e;
                            if (!key_ok || (causal && my_k > q)) x = -INFINITY;
                        }
                        const float pr = fast_exp2(x);
                        const float p0 = pr > kEps ? pr : 0.f;
                        float pkk = p0;
                        if constexpr (DROP) {
                            const bool keep = lcg_keep(st_blk + (uint64_t)(8 * g4 + e) * row_step, thr);
                            pkk = keep ? p0 : 0.f;
                            xv[e] = keep ? p0 : -p0;
                        } else {
                            xv[e] = p0;
                        }
                        sacc[r] = pkk;
                    }
                    *reinterpret_cast<floatx4*>(xs + (g4 * 64 + lane) * 4) = xv;
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int qrow = 8 * (r >> 2) + 4 * hh + (r & 3);
#pragma unroll
                    for (int dt = 0; dt < DV / 32; ++dt)
                        dvacc[dt] = mfma_f32(dOs[qrow * OS + 32 * dt + l32], sacc[r], dvacc[dt]);
                }
            }
            if (has_next) store_rows((n + 1) % NSTAGE);
        }
        if (key_ok) {
            float* dVb = static_cast<float*>(p.dv) + ((size_t)b * S_kv + my_k) * D_v;
#pragma unroll
            for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                    floatx4 fv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) fv[e] = dvacc[dt][4 * g4 + e] * ksc;
                    if constexpr (VEC) {
                        if (d0 < D_v) *reinterpret_cast<floatx4*>(dVb + d0) = fv;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (d0 + e < D_v) dVb[d0 + e] = fv[e];
                    }
                }
        }
    } else {
        // ----------------------------------------------------------- dS role
        const float* Vb = static_cast<const float*>(p.v) + (size_t)b * S_kv * D_v;
        float vf[HV];
#pragma unroll
        for (int u = 0; u < HV / 4; ++u) {
            const floatx4 f = __builtin_bit_cast(floatx4, load_row_chunk<float, VEC>(Vb, my_k, S_kv, HV * hh + 4 * u, D_v, D_v));
#pragma unroll
            for (int e = 0; e < 4; ++e) vf[4 * u + e] = f[e];
        }
        prologue_loads_landed();
        floatx16 dkacc[DQK / 32];
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt) dkacc[dt] = floatx16{};
        // dS path: this key group's dS of each visited block goes to its
        // chunk (DsLayout32): the lane's 16 values, query positions 16 hh + r,
        // as four 16-byte slots, one per store, each store 1 KB whole; zero
        // for keys past S_kv (the dQ kernel reads them unmasked)
        const DsLayout32 dsl(S_q, S_kv, causal);

        for (int n = 0; n <= nblk; ++n) {
            __syncthreads();
            const bool has_next = n + 1 < nblk;
            if (has_next) load_rows(q_begin + (n + 1) * BQ);
            const int m = n - 1;
            const int q0 = q_begin + m * BQ;
            if (m >= 0 && live(q0)) {
                const float* Qs = lds + (m % NSTAGE) * Cfg::STAGE;
                const float* dOs = Qs + Cfg::QT;
                const float* Fs = dOs + Cfg::OT;
                floatx16 dpacc = floatx16{};
#pragma unroll
                for (int u = 0; u < HV / 4; ++u) {
                    const floatx4 oo = *reinterpret_cast<const floatx4*>(dOs + l32 * OS + HV * hh + 4 * u);
#pragma unroll
                    for (int e = 0; e < 4; ++e) dpacc = mfma_f32(oo[e], vf[4 * u + e], dpacc);
                }
                // dS = P0 (keep ? dP / (1-p) : 0 - delta), P0 = |x|, keep = x > 0
                const float* xs = xbuf(m);
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const floatx4 xv = *reinterpret_cast<const floatx4*>(xs + (g4 * 64 + lane) * 4);
                    const floatx4 de4 = *reinterpret_cast<const floatx4*>(Fs + BQ + 8 * g4 + 4 * hh);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * g4 + e;
                        float dpk = DROP ? dpacc[r] * ksc : dpacc[r];
                        float p0 = xv[e];
                        if constexpr (DROP) {
                            dpk = xv[e] > 0.f ? dpk : 0.f;
                            p0 = __builtin_fabsf(xv[e]);
                        }
                        dpacc[r] = p0 * (dpk - de4[e]);
                    }
                }
                if constexpr (DS) {
                    unsigned char* grp = static_cast<unsigned char*>(p.ds) + dsl.offset(b, kt, q0 / BQ) + kw * 4096;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        floatx4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = key_ok ? dpacc[4 * u + e] : 0.f;
                        __builtin_nontemporal_store(
                            v, reinterpret_cast<floatx4*>(grp + DsLayout32::slot32(l32, 16 * hh + 4 * u)));
                    }
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int qrow = 8 * (r >> 2) + 4 * hh + (r & 3);
#pragma unroll
                    for (int dt = 0; dt < DQK / 32; ++dt)
                        dkacc[dt] = mfma_f32(Qs[qrow * QS + 32 * dt + l32], dpacc[r], dkacc[dt]);
                }
            }
            if (has_next) store_rows((n + 1) % NSTAGE);
        }
        if (key_ok) {
            const float sc = p.c.scale;
            float* dKb = static_cast<float*>(p.dk) + ((size_t)b * S_kv + my_k) * D_qk;
#pragma unroll
            for (int dt = 0; dt < DQK / 32; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                    floatx4 fv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) fv[e] = dkacc[dt][4 * g4 + e] * sc;
                    if constexpr (VEC) {
                        if (d0 < D_qk) *reinterpret_cast<floatx4*>(dKb + d0) = fv;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (d0 + e < D_qk) dKb[d0 + e] = fv[e];
                    }
                }
        }
    }
}

// ---------------------------------------------------------------------------
// Host launcher: dQ (+ delta) first, then dK/dV, on the caller's stream.
// ---------------------------------------------------------------------------
hipError_t launch_bwd(const BwdParams& p, DType dtype, bool vec, int phases, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv;
    if (B == 0) return hipSuccess;
    const bool drop = p.c.use_dropout != 0;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_dim(p.s.D_v, [&](auto dv) {
            return with_bool(vec, [&](auto v) {
                return with_bool(drop, [&](auto d) {
                    constexpr int DQK = decltype(dqk)::value, DV = decltype(dv)::value;
                    constexpr bool V = decltype(v)::value, D = decltype(d)::value;
                    hipError_t err = hipSuccess;
                    if (dtype == DType::F16) {
                        using CQ = BwdQF16Cfg<DQK, DV>;
                        using CK = BwdKVF16Cfg<DQK, DV>;
                        const unsigned gq = (unsigned)(((S_q + CQ::BM - 1) / CQ::BM) * B);
                        const unsigned gk = (unsigned)(((S_kv + CK::BKV - 1) / CK::BKV) * B);
                        if (phases & kBwdDq)
                            err = launch_kernel<sdpa_bwd_dq_f16_kernel<DQK, DV, V, D>>(gq, CQ::NT, CQ::LDS_BYTES, stream, p);
                        if (err == hipSuccess && (phases & kBwdDkDv))
                            err = launch_kernel<sdpa_bwd_dkdv_f16_kernel<DQK, DV, V, D>>(gk, CK::NT, CK::LDS_BYTES, stream, p);
                    } else {
                        using CQ = BwdQF32Cfg<DQK, DV>;
                        using CK = BwdKVF32Cfg<DQK, DV>;
                        using CS = BwdKVF32SplitCfg<DQK, DV>;
                        const unsigned gq = (unsigned)(((S_q + CQ::BM - 1) / CQ::BM) * B);
                        const unsigned gk = (unsigned)(((S_kv + CK::BKV - 1) / CK::BKV) * B);
                        if (phases & kBwdDq)
                            err = launch_kernel<sdpa_bwd_dq_f32_kernel<DQK, DV, V, D>>(gq, CQ::NT, CQ::LDS_BYTES, stream, p);
                        if (err == hipSuccess && (phases & kBwdDkDv)) {
                            if constexpr (SDPA_F32_SPLIT && (DQK == 128 || DV == 128)) {
                                static_assert(CS::BKV == DsLayout32::KT && CS::BQ == DsLayout32::QBK, "dS chunk geometry");
                                const unsigned gs = (unsigned)(((S_kv + CS::BKV - 1) / CS::BKV) * B);
                                if (p.ds)
                                    err = launch_kernel<sdpa_bwd_dkdv_f32_split_kernel<DQK, DV, V, D, true>>(
                                        gs, CS::NT, CS::LDS_BYTES, stream, p);
                                else
                                    err = launch_kernel<sdpa_bwd_dkdv_f32_split_kernel<DQK, DV, V, D, false>>(
                                        gs, CS::NT, CS::LDS_BYTES, stream, p);
                            } else if (p.ds) {
                                err = hipErrorInvalidValue;  // the dS path needs the split kernel
                            } else
                                err = launch_kernel<sdpa_bwd_dkdv_f32_kernel<DQK, DV, V, D>>(gk, CK::NT, CK::LDS_BYTES, stream, p);
                        }
                    }
                    return err;
                });
            });
        });
    });
}

}  // namespace sdpa
