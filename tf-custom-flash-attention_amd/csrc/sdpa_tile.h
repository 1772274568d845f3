// sdpa_tile.h -- global -> register -> LDS tile staging used by the Sdpa
// kernels (the role of load_tile in sdpa/sdpa_utils.cuh:21-48: zero padding
// for rows >= S and columns >= D), done in 16-byte chunks by the whole
// workgroup so that each wave's loads are fully coalesced.
#pragma once

#include "sdpa_device.h"

namespace sdpa {

// One tile of ROWS x COLS elements of T (COLS = padded feature width), held
// in registers between the global load and the LDS store so that the loads
// of block n+1 overlap the MFMA work on block n.
//   VEC = true : every row starts 16-byte aligned and D is a multiple of the
//                chunk width, so a chunk is either entirely valid or entirely
//                past D (one dwordx4 load per chunk).
//   VEC = false: arbitrary D; elements are loaded one at a time.
template <typename T, int ROWS, int COLS, int NTHREADS, bool VEC>
struct TileStage {
    static constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
    static constexpr int CPR = COLS / EPC;           // chunks per row
    static constexpr int NCH = ROWS * CPR;
    static constexpr int PER_THREAD = (NCH + NTHREADS - 1) / NTHREADS;
    static_assert(COLS % EPC == 0, "padded width must be a whole number of chunks");

    uint4 r[PER_THREAD];

    // g: base of the [S, ld] matrix of this batch; rows row0.. are loaded,
    // rows >= nrows and columns >= ncols read as zero.  With VEC the chunks
    // are raw buffer loads over rows [row0, row0 + nrows): the descriptor's
    // record count zero-fills rows past the end and a column past ncols gets
    // an offset beyond every record, so the loads carry no branches (g and
    // row0 are wave-uniform).
    template <bool BUF = true>
    __device__ __forceinline__ void load(const T* __restrict__ g, int row0, int nrows, int ncols,
                                         int ld, int tid) {
        if constexpr (VEC && BUF) {
            const int row_bytes = ld * (int)sizeof(T);
            const int max_rows = row_bytes > 0 ? 0x7FFFFFFF / row_bytes : 0x7FFFFFFF;
            const int nrec = nrows <= 0 ? 0 : (nrows >= max_rows ? 0x7FFFFFFF : nrows * row_bytes);
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<T*>(g + (size_t)row0 * ld), (short)0, nrec, 0x00020000);
#pragma unroll
            for (int u = 0; u < PER_THREAD; ++u) {
                const int c = tid + u * NTHREADS;
                const int row = c / CPR;
                const int col = (c % CPR) * EPC;
                const bool ok = (NCH % NTHREADS == 0 || c < NCH) && col < ncols;
                const uint32_t off = ok ? (uint32_t)(row * row_bytes + col * (int)sizeof(T)) : 0x80000000u;
                r[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < PER_THREAD; ++u) {
            const int c = tid + u * NTHREADS;
            const int row = c / CPR;
            const int col = (c % CPR) * EPC;
            uint4 val = make_uint4(0, 0, 0, 0);
            if ((NCH % NTHREADS == 0 || c < NCH) && row < nrows) {
                const T* src = g + (size_t)(row0 + row) * ld + col;
                if constexpr (VEC) {
                    if (col < ncols) val = *reinterpret_cast<const uint4*>(src);
                } else {
                    T tmp[EPC];
#pragma unroll
                    for (int e = 0; e < EPC; ++e) tmp[e] = (col + e < ncols) ? src[e] : T(0);
                    __builtin_memcpy(&val, tmp, 16);
                }
            }
            r[u] = val;
        }
    }

    // Store into an unpadded, chunk-swizzled LDS tile (see swz_off).
    __device__ __forceinline__ void store_swz(T* lds, int tid) const;

    // Store into LDS with a row stride of STRIDE elements (STRIDE*sizeof(T) % 16 == 0).
    template <int STRIDE>
    __device__ __forceinline__ void store(T* lds, int tid) const {
        static_assert((STRIDE * (int)sizeof(T)) % 16 == 0, "LDS rows must stay 16-byte aligned");
#pragma unroll
        for (int u = 0; u < PER_THREAD; ++u) {
            const int c = tid + u * NTHREADS;
            if (NCH % NTHREADS == 0 || c < NCH) {
                const int row = c / CPR;
                const int col = (c % CPR) * EPC;
                *reinterpret_cast<uint4*>(lds + row * STRIDE + col) = r[u];
            }
        }
    }
};

// ---------------------------------------------------------------------------
// Swizzled fp16 tiles.  A tile of rows x (8*L) halves is stored without
// padding; the 16-byte chunk c of row r lives at chunk position c ^ swz<L>(r).
// LDS has 64 banks of 4 bytes, i.e. 16 "bank groups" of 16 bytes; the
// swizzle makes both access patterns of the kernels conflict-free:
//   (a) b128 row reads: 16 lanes read chunk c of 16 consecutive rows;
//   (b) ds_read_b64_tr_b16: per cycle 32 lanes read chunks c..c+3 (c % 4 == 0)
//       of 4 consecutive rows r0..r0+3 (r0 % 4 == 0).
// L = 16 (D = 128): one row per 64 banks; f(r) = 4*(r%4) + (r/4)%4 is a
//   bijection on 16 rows (a) and gives rows r0..r0+3 distinct high bits (b).
// L = 8 (D = 64): two rows per 64 banks (bank group 8*(r%2) + chunk);
//   f(r) = 4*((r/2)%2) + (r/4)%4.
// L = 4 (D = 32): four rows per 64 banks; f(r) = (r/4)%4.
// ---------------------------------------------------------------------------
template <int L>
__device__ __forceinline__ int swz(int r) {
    static_assert(L == 4 || L == 8 || L == 16, "swizzle defined for 32/64/128-wide fp16 rows");
    if constexpr (L == 16) return 4 * (r & 3) + ((r >> 2) & 3);
    else if constexpr (L == 8) return 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
    else return (r >> 2) & 3;
}

// Element offset of (row, col) in a swizzled tile of 8*L halves per row.
template <int L>
__device__ __forceinline__ int swz_off(int row, int col) {
    return row * (8 * L) + ((((col >> 3) ^ swz<L>(row))) << 3) + (col & 7);
}

template <typename T, int ROWS, int COLS, int NTHREADS, bool VEC>
__device__ __forceinline__ void TileStage<T, ROWS, COLS, NTHREADS, VEC>::store_swz(T* lds, int tid) const {
    static_assert(sizeof(T) == 2, "swizzled tiles hold fp16");
#pragma unroll
    for (int u = 0; u < PER_THREAD; ++u) {
        const int c = tid + u * NTHREADS;
        if (NCH % NTHREADS == 0 || c < NCH) {
            const int row = c / CPR;
            const int col = (c % CPR) * EPC;
            *reinterpret_cast<uint4*>(lds + swz_off<CPR>(row, col)) = r[u];
        }
    }
}

// Load 16 bytes of one row (elements col..col+EPC-1) straight into registers,
// zero-filled past nrows / ncols.
template <typename T, bool VEC>
__device__ __forceinline__ uint4 load_row_chunk(const T* __restrict__ g, int row, int nrows, int col,
                                                int ncols, int ld) {
    constexpr int EPC = 16 / (int)sizeof(T);
    uint4 val = make_uint4(0, 0, 0, 0);
    if (row < nrows) {
        const T* src = g + (size_t)row * ld + col;
        if constexpr (VEC) {
            if (col < ncols) val = *reinterpret_cast<const uint4*>(src);
        } else {
            T tmp[EPC];
#pragma unroll
            for (int e = 0; e < EPC; ++e) tmp[e] = (col + e < ncols) ? src[e] : T(0);
            __builtin_memcpy(&val, tmp, 16);
        }
    }
    return val;
}

}  // namespace sdpa
