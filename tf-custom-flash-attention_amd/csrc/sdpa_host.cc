// sdpa_host.cc -- CPU kernels of the Sdpa / SdpaGrad ops (the op's
// DEVICE_CPU registration), behind the C ABI of include/sdpa_cpu.h.
//
// Replaces functor::FlashAttnFunctor<CPUDevice, T> and
// FlashAttnGradFunctor<CPUDevice, T> (sdpa/sdpa_cpu.cc:213-457).  The
// reference computes one (query, key) element at a time, parallel over the
// batch only; these kernels are tiled for a CPU's vector units and cores:
//   forward   work item = (batch, 16 query rows); keys in blocks of 64,
//             S = Q K^T against a transposed K block (the inner loop runs
//             over 64 keys, so it vectorises without reassociating sums),
//             block-wise online softmax, O += P~ V.
//   backward  two passes, as the GPU kernels: pass 1 per (batch, 16 query
//             rows) computes delta and dQ; pass 2 per (batch, 64 keys)
//             recomputes P and dS and accumulates dK and dV.  No item writes
//             another item's output, so nothing is shared but read-only data.
// Work items are handed out by an atomic counter over a fixed set of threads.
//
// Element semantics are those of the reference CPU functors:
//   dropout active iff p > 0 (sdpa_cpu.cc:232-235), element (b,i,j) dropped
//   iff u(b,i,j) < p with the LCG hash of sdpa_cpu.cc:198-211;
//   l sums undropped probabilities; stats = m + log(l + 1e-6); o = acc / l if
//   l > 1e-6 else 0 (sdpa_cpu.cc:287-308);
//   the backward skips P < 1e-6; kept: dS = P/(1-p) (dP - delta (1-p)) scale,
//   dropped: dS = -P delta scale (sdpa_cpu.cc:376-428).
// Products and sums are fp32 (fp16 inputs are widened exactly with F16C and
// the outputs rounded to nearest even once).
#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "sdpa_checks.h"
#include "sdpa_cpu.h"
#include "sdpa_hip.h"  // sdpa_status_t codes (shared with the GPU library)

namespace {

constexpr int TQ = 16;     // query rows per work item
constexpr int TK = 64;     // keys per block (and per pass-2 work item)
constexpr int DMAX = 128;  // largest feature width (sdpa_cpu.cc:66-69)
constexpr float kEps = 1e-6f;
constexpr float kNegInf = -1e9f;
constexpr uint64_t kLcgMul = 6364136223846793005ULL;
constexpr uint64_t kLcgInc = 1442695040888963407ULL;

// ---- storage <-> fp32 ------------------------------------------------------
void widen(int dtype, const void* base, size_t off, int n, float* dst) {
    if (dtype == SDPA_CPU_DTYPE_F32) {
        std::memcpy(dst, static_cast<const float*>(base) + off, (size_t)n * sizeof(float));
        return;
    }
    const uint16_t* h = static_cast<const uint16_t*>(base) + off;
    int i = 0;
    for (; i + 8 <= n; i += 8)
        _mm256_storeu_ps(dst + i, _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(h + i))));
    for (; i < n; ++i) dst[i] = _cvtsh_ss(h[i]);
}

void narrow(int dtype, const float* src, int n, float f, void* base, size_t off) {
    if (dtype == SDPA_CPU_DTYPE_F32) {
        float* d = static_cast<float*>(base) + off;
        for (int i = 0; i < n; ++i) d[i] = src[i] * f;
        return;
    }
    uint16_t* h = static_cast<uint16_t*>(base) + off;
    const __m256 fv = _mm256_set1_ps(f);
    int i = 0;
    for (; i + 8 <= n; i += 8)
        _mm_storeu_si128(reinterpret_cast<__m128i*>(h + i),
                         _mm256_cvtps_ph(_mm256_mul_ps(_mm256_loadu_ps(src + i), fv), _MM_FROUND_TO_NEAREST_INT));
    for (; i < n; ++i) h[i] = _cvtss_sh(src[i] * f, _MM_FROUND_TO_NEAREST_INT);
}

// ---- dropout (sdpa_cpu.cc:198-211): dropped iff u < p --------------------
struct Dropout {
    bool on;
    float p, inv;        // p and 1 / (1 - p)
    uint64_t base;       // seed + offset
    uint64_t S_q, S_kv;  // counter strides
    bool dropped(uint64_t b, uint64_t i, uint64_t j) const {
        const uint64_t st = (base + (b * S_q + i) * S_kv + j) * kLcgMul + kLcgInc;
        return static_cast<float>(static_cast<uint32_t>(st >> 32)) / 4294967296.0f < p;
    }
};

struct Problem {
    int dtype, B, S_q, S_kv, D_qk, D_v;
    float scale;
    bool causal;
    Dropout drop;
};

// Threads used for n work items (nthreads <= 0: every hardware thread).
int thread_count(int nthreads, int n) {
    const int nt = nthreads > 0 ? nthreads : (int)std::max(1u, std::thread::hardware_concurrency());
    return std::max(1, std::min(nt, n));
}

// fn(worker, item) for item in [0, n) on thread_count(nthreads, n) threads;
// worker in [0, threads) identifies the calling thread (its scratch slot).
template <typename F>
void parallel_for(int n, int nthreads, F&& fn) {
    const int nt = thread_count(nthreads, n);
    std::atomic<int> next{0};
    auto worker = [&](int id) {
        for (int i = next.fetch_add(1); i < n; i = next.fetch_add(1)) fn(id, i);
    };
    std::vector<std::thread> pool;
    pool.reserve(nt - 1);
    for (int t = 1; t < nt; ++t) pool.emplace_back(worker, t);
    worker(0);
    for (auto& th : pool) th.join();
}

// A block of `n` (<= TK) rows of a [rows, D] matrix, widened, both row-major
// (rows[r * D + d]) and transposed (cols[d * TK + r], zero past n).
struct Block {
    float rows[TK * DMAX];
    float cols[DMAX * TK];
    void load(int dtype, const void* base, size_t row0, int n, int D, bool want_cols) {
        widen(dtype, base, row0 * (size_t)D, n * D, rows);
        if (!want_cols) return;
        for (int d = 0; d < D; ++d) {
            float* c = cols + d * TK;
            for (int r = 0; r < n; ++r) c[r] = rows[r * D + d];
            for (int r = n; r < TK; ++r) c[r] = 0.f;
        }
    }
};

// out[0..TK) = x . cols[d][0..TK) over D features (vectorised over keys).
inline void dot_cols(const float* x, const float* cols, int D, float* out) {
    for (int j = 0; j < TK; ++j) out[j] = 0.f;
    for (int d = 0; d < D; ++d) {
        const float xd = x[d];
        const float* c = cols + d * TK;
        for (int j = 0; j < TK; ++j) out[j] += xd * c[j];
    }
}

inline void axpy(float a, const float* x, float* y, int n) {
    for (int i = 0; i < n; ++i) y[i] += a * x[i];
}

// ---- forward ----------------------------------------------------------------
struct FwdScratch {
    float q[TQ * DMAX];
    float acc[TQ * DMAX];
    Block kb, vb;
    float s[TK];
};

void fwd_item(const Problem& P, const void* Q, const void* K, const void* V, void* O, float* stats,
              int item, FwdScratch& w) {
    const int tiles = (P.S_q + TQ - 1) / TQ;
    const int b = item / tiles, i0 = (item % tiles) * TQ, nq = std::min(TQ, P.S_q - i0);
    const int Dq = P.D_qk, Dv = P.D_v;
    widen(P.dtype, Q, ((size_t)b * P.S_q + i0) * Dq, nq * Dq, w.q);
    std::fill(w.acc, w.acc + nq * Dv, 0.f);
    float m[TQ], l[TQ];
    std::fill(m, m + TQ, kNegInf);
    std::fill(l, l + TQ, 0.f);
    const int kend = P.causal ? std::min(P.S_kv, i0 + nq) : P.S_kv;
    for (int j0 = 0; j0 < kend; j0 += TK) {
        const int nk = std::min(TK, kend - j0);
        w.kb.load(P.dtype, K, (size_t)b * P.S_kv + j0, nk, Dq, true);
        w.vb.load(P.dtype, V, (size_t)b * P.S_kv + j0, nk, Dv, false);
        for (int r = 0; r < nq; ++r) {
            const int i = i0 + r;
            const int lim = P.causal ? std::min(nk, i - j0 + 1) : nk;  // visible keys of this row
            if (lim <= 0) continue;
            dot_cols(w.q + r * Dq, w.kb.cols, Dq, w.s);
            float mx = -INFINITY;
            for (int j = 0; j < lim; ++j) {
                w.s[j] *= P.scale;
                mx = std::max(mx, w.s[j]);
            }
            const float m_new = std::max(m[r], mx);
            const float alpha = std::exp(m[r] - m_new);
            float* acc = w.acc + r * Dv;
            if (alpha != 1.f)
                for (int d = 0; d < Dv; ++d) acc[d] *= alpha;
            float lsum = 0.f;
            for (int j = 0; j < lim; ++j) {
                const float p = std::exp(w.s[j] - m_new);
                lsum += p;
                float pk = p;
                if (P.drop.on) pk = P.drop.dropped(b, i, j0 + j) ? 0.f : p * P.drop.inv;
                if (pk != 0.f) axpy(pk, w.vb.rows + j * Dv, acc, Dv);
            }
            l[r] = l[r] * alpha + lsum;
            m[r] = m_new;
        }
    }
    for (int r = 0; r < nq; ++r) {
        const size_t row = (size_t)b * P.S_q + i0 + r;
        stats[row] = m[r] + std::log(l[r] + kEps);
        const float inv = l[r] > kEps ? 1.f / l[r] : 0.f;
        narrow(P.dtype, w.acc + r * Dv, Dv, inv, O, row * Dv);
    }
}

// ---- backward -----------------------------------------------------------------
struct BwdScratch {
    float q[TQ * DMAX], dout[TQ * DMAX], o[TQ * DMAX];
    float g[TK * DMAX], g2[TK * DMAX];  // dQ rows (pass 1) / dK, dV rows (pass 2)
    Block kb, vb;
    float s[TK], dp[TK];
};

// dS of element (b, i, j) given the score s (unscaled), dP and delta; the
// kept probability P~ (0 if dropped or skipped) in *pk.  Returns false when
// the element is skipped (P < 1e-6).
inline bool element(const Problem& P, int b, int i, int j, float s, float dp, float st, float delta,
                    float* pk, float* ds) {
    const float prob = std::exp(s * P.scale - st);
    if (prob < kEps) return false;  // sdpa_cpu.cc:384-385
    if (P.drop.on && P.drop.dropped(b, i, j)) {
        *pk = 0.f;
        *ds = -prob * delta * P.scale;
        return true;
    }
    const float pinv = P.drop.on ? P.drop.inv : 1.f;
    const float pr = prob * pinv;
    *pk = pr;
    *ds = pr * (dp - delta / pinv) * P.scale;
    return true;
}

// Pass 1: delta and dQ of 16 query rows.
void bwd_dq_item(const Problem& P, const void* Q, const void* K, const void* V, const void* O,
                 const float* stats, const void* dO, void* dQ, float* delta_out, int item,
                 BwdScratch& w) {
    const int tiles = (P.S_q + TQ - 1) / TQ;
    const int b = item / tiles, i0 = (item % tiles) * TQ, nq = std::min(TQ, P.S_q - i0);
    const int Dq = P.D_qk, Dv = P.D_v;
    const size_t row0 = (size_t)b * P.S_q + i0;
    widen(P.dtype, Q, row0 * Dq, nq * Dq, w.q);
    widen(P.dtype, dO, row0 * Dv, nq * Dv, w.dout);
    widen(P.dtype, O, row0 * Dv, nq * Dv, w.o);
    float delta[TQ];
    for (int r = 0; r < nq; ++r) {
        float acc = 0.f;
        for (int d = 0; d < Dv; ++d) acc += w.dout[r * Dv + d] * w.o[r * Dv + d];
        delta[r] = acc;
        delta_out[row0 + r] = acc;
    }
    std::fill(w.g, w.g + nq * Dq, 0.f);
    const int kend = P.causal ? std::min(P.S_kv, i0 + nq) : P.S_kv;
    for (int j0 = 0; j0 < kend; j0 += TK) {
        const int nk = std::min(TK, kend - j0);
        w.kb.load(P.dtype, K, (size_t)b * P.S_kv + j0, nk, Dq, true);
        w.vb.load(P.dtype, V, (size_t)b * P.S_kv + j0, nk, Dv, true);
        for (int r = 0; r < nq; ++r) {
            const int i = i0 + r;
            const int lim = P.causal ? std::min(nk, i - j0 + 1) : nk;
            if (lim <= 0) continue;
            dot_cols(w.q + r * Dq, w.kb.cols, Dq, w.s);
            dot_cols(w.dout + r * Dv, w.vb.cols, Dv, w.dp);
            const float st = stats[row0 + r];
            for (int j = 0; j < lim; ++j) {
                float pk, ds;
                if (!element(P, b, i, j0 + j, w.s[j], w.dp[j], st, delta[r], &pk, &ds)) continue;
                axpy(ds, w.kb.rows + j * Dq, w.g + r * Dq, Dq);
            }
        }
    }
    for (int r = 0; r < nq; ++r) narrow(P.dtype, w.g + r * Dq, Dq, 1.f, dQ, (row0 + r) * Dq);
}

// Pass 2: dK and dV of 64 keys, over every query row that sees them.
void bwd_dkdv_item(const Problem& P, const void* Q, const void* K, const void* V, const float* stats,
                   const void* dO, void* dK, void* dV, const float* delta_in, int item,
                   BwdScratch& w) {
    const int tiles = (P.S_kv + TK - 1) / TK;
    const int b = item / tiles, j0 = (item % tiles) * TK, nk = std::min(TK, P.S_kv - j0);
    const int Dq = P.D_qk, Dv = P.D_v;
    w.kb.load(P.dtype, K, (size_t)b * P.S_kv + j0, nk, Dq, true);
    w.vb.load(P.dtype, V, (size_t)b * P.S_kv + j0, nk, Dv, true);
    float* dk = w.g;
    float* dv = w.g2;
    std::fill(dk, dk + nk * Dq, 0.f);
    std::fill(dv, dv + nk * Dv, 0.f);
    const int q_begin = P.causal ? j0 : 0;  // rows above j0 see none of these keys
    for (int i0 = q_begin; i0 < P.S_q; i0 += TQ) {
        const int nq = std::min(TQ, P.S_q - i0);
        const size_t row0 = (size_t)b * P.S_q + i0;
        widen(P.dtype, Q, row0 * Dq, nq * Dq, w.q);
        widen(P.dtype, dO, row0 * Dv, nq * Dv, w.dout);
        for (int r = 0; r < nq; ++r) {
            const int i = i0 + r;
            const int lim = P.causal ? std::min(nk, i - j0 + 1) : nk;
            if (lim <= 0) continue;
            dot_cols(w.q + r * Dq, w.kb.cols, Dq, w.s);
            dot_cols(w.dout + r * Dv, w.vb.cols, Dv, w.dp);
            const float st = stats[row0 + r], delta = delta_in[row0 + r];
            for (int j = 0; j < lim; ++j) {
                float pk, ds;
                if (!element(P, b, i, j0 + j, w.s[j], w.dp[j], st, delta, &pk, &ds)) continue;
                if (pk != 0.f) axpy(pk, w.dout + r * Dv, dv + j * Dv, Dv);
                axpy(ds, w.q + r * Dq, dk + j * Dq, Dq);
            }
        }
    }
    const size_t k0 = (size_t)b * P.S_kv + j0;
    for (int j = 0; j < nk; ++j) {
        narrow(P.dtype, dk + j * Dq, Dq, 1.f, dK, (k0 + j) * Dq);
        narrow(P.dtype, dv + j * Dv, Dv, 1.f, dV, (k0 + j) * Dv);
    }
}

int check(int dtype, int B, int S_q, int S_kv, int D_qk, int D_v, float dropout, int causal) {
    if (dtype != SDPA_CPU_DTYPE_F32 && dtype != SDPA_CPU_DTYPE_F16) return SDPA_ERR_DTYPE;
    if (B < 0 || S_q < 0 || S_kv < 0 || D_qk < 0 || D_v < 0) return SDPA_ERR_NEGATIVE_DIM;
    if (causal && S_q != S_kv) return SDPA_ERR_CAUSAL_SEQ;
    if (std::max(D_qk, D_v) > DMAX) return SDPA_ERR_FEATURE_TOO_LARGE;
    // dropout > 1 drops every element (u <= 1 < p), as in the reference; at
    // dropout == 1 the reference scales the rare u == 1 elements by 1 / 0
    if (dropout == 1.0f) return SDPA_ERR_DROPOUT_RANGE;
    return SDPA_OK;
}

Problem make_problem(int dtype, int B, int S_q, int S_kv, int D_qk, int D_v, float scale,
                     float dropout, int causal, uint64_t seed, uint64_t offset) {
    Problem P{dtype, B, S_q, S_kv, D_qk, D_v, scale, causal != 0, {}};
    P.drop.on = dropout > 0.0f;  // sdpa_cpu.cc:232
    P.drop.p = dropout;
    P.drop.inv = P.drop.on ? 1.0f / (1.0f - dropout) : 1.0f;
    P.drop.base = seed + offset;
    P.drop.S_q = (uint64_t)S_q;
    P.drop.S_kv = (uint64_t)S_kv;
    return P;
}

}  // namespace

extern "C" {

const char* sdpa_cpu_status_string(int status) { return sdpa::status_message(status); }

int sdpa_cpu_check_fwd(int q_rank, const int64_t* q_shape, int k_rank, const int64_t* k_shape, int v_rank,
                       const int64_t* v_shape, int seed_rank, int offset_rank, int causal_mask) {
    return sdpa::check_fwd_shapes(q_rank, q_shape, k_rank, k_shape, v_rank, v_shape, seed_rank, offset_rank,
                                  causal_mask);
}

int sdpa_cpu_check_bwd(int q_rank, const int64_t* q_shape, int k_rank, const int64_t* k_shape, int v_rank,
                       const int64_t* v_shape, int o_rank, const int64_t* o_shape, int stats_rank,
                       const int64_t* stats_shape, int do_rank, const int64_t* do_shape, int seed_rank,
                       int offset_rank, int causal_mask) {
    return sdpa::check_bwd_shapes(q_rank, q_shape, k_rank, k_shape, v_rank, v_shape, o_rank, o_shape, stats_rank,
                                  stats_shape, do_rank, do_shape, seed_rank, offset_rank, causal_mask);
}

int sdpa_cpu_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* stats,
                 int B, int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                 int causal_mask, uint64_t seed, uint64_t offset, int nthreads) {
    int st = check(dtype, B, S_q, S_kv, D_qk, D_v, dropout, causal_mask);
    if (st != SDPA_OK) return st;
    if ((size_t)B * S_q == 0) return SDPA_OK;
    if (!stats || (D_v > 0 && !o) || (D_qk > 0 && (!q || (S_kv > 0 && !k))) || (S_kv > 0 && D_v > 0 && !v))
        return SDPA_ERR_NULL_POINTER;
    const Problem P = make_problem(dtype, B, S_q, S_kv, D_qk, D_v, scale, dropout, causal_mask, seed, offset);
    const int items = B * ((S_q + TQ - 1) / TQ);
    std::vector<FwdScratch> scratch(thread_count(nthreads, items));
    parallel_for(items, nthreads, [&](int w, int item) { fwd_item(P, q, k, v, o, stats, item, scratch[w]); });
    return SDPA_OK;
}

int sdpa_cpu_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
                 const float* stats, const void* d_o, void* dq, void* dk, void* dv, int B, int S_q,
                 int S_kv, int D_qk, int D_v, float scale, float dropout, int causal_mask,
                 uint64_t seed, uint64_t offset, int nthreads) {
    int st = check(dtype, B, S_q, S_kv, D_qk, D_v, dropout, causal_mask);
    if (st != SDPA_OK) return st;
    if (B == 0) return SDPA_OK;
    const bool has_q = S_q > 0, has_kv = S_kv > 0;
    if ((has_q && !stats) || (has_q && D_qk > 0 && (!q || !dq)) || (has_q && D_v > 0 && (!d_o || !o)) ||
        (has_kv && D_qk > 0 && (!k || !dk)) || (has_kv && D_v > 0 && (!v || !dv)))
        return SDPA_ERR_NULL_POINTER;
    const Problem P = make_problem(dtype, B, S_q, S_kv, D_qk, D_v, scale, dropout, causal_mask, seed, offset);
    std::vector<float> delta((size_t)B * S_q);  // pass 1 -> pass 2
    const int q_items = B * ((S_q + TQ - 1) / TQ), k_items = B * ((S_kv + TK - 1) / TK);
    std::vector<BwdScratch> scratch(thread_count(nthreads, std::max(q_items, k_items)));
    if (q_items > 0)
        parallel_for(q_items, nthreads, [&](int w, int item) {
            bwd_dq_item(P, q, k, v, o, stats, d_o, dq, delta.data(), item, scratch[w]);
        });
    if (k_items > 0)
        parallel_for(k_items, nthreads, [&](int w, int item) {
            bwd_dkdv_item(P, q, k, v, stats, d_o, dk, dv, delta.data(), item, scratch[w]);
        });
    return SDPA_OK;
}

}  // extern "C"
