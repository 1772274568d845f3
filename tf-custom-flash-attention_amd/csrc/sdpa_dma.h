// sdpa_dma.h -- building blocks of the fp16 kernels that stream their tiles
// from HBM straight into LDS (sdpa_f16_fwd/dq/dkdv.hip): buffer
// descriptors and the HBM -> LDS copy instructions, the chunk-swizzled tile
// layout and its MFMA operand reads, the XCD-aware work order and the fp16
// stores of accumulator rows.
//
// Data movement.  Tiles are copied by buffer_load_dwordx4 ... lds: lane L of
// a wave writes 16 bytes to LDS at (M0 + 16 L), and each lane picks the
// global chunk that belongs there, so the LDS image comes out in the
// chunk-swizzled layout of swz_off() (conflict-free row and transposed reads)
// without passing through VGPRs.  A descriptor's range ends at the end of
// its batch row, so rows past S and columns past D read as zero.
#pragma once

#include "sdpa_device.h"
#include "sdpa_tile.h"

namespace sdpa {
namespace {

extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

// Buffer descriptor (four SGPRs): base address, stride 0, num_records, and
// the word-3 configuration of a raw buffer on gfx950.
typedef int rsrc_t __attribute__((ext_vector_type(4)));

// MFMA operands read ahead from LDS (in MFMAs) by the fenced chains.
#ifndef SDPA_RD
#define SDPA_RD 4
#endif

// A voffset at or past num_records: the load returns zero and touches nothing.
constexpr uint32_t kOob = 0x80000000u;


// Raw buffer descriptor over [base, base + bytes); every field is wave-uniform.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, long long bytes) {
    const int n = bytes <= 0 ? 0 : (bytes >= 0x7FFFFFFFLL ? 0x7FFFFFFF : (int)bytes);
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return (rsrc_t){__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                    __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu)),
                    __builtin_amdgcn_readfirstlane(n), 0x00020000};
}

// A workgroup-uniform pointer held in scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// Descriptor over the rows [row0, rows) of a row-major matrix with row_bytes
// per row; rows past the end read as zero.  All arithmetic is wave-uniform
// 32-bit (max_rows = the largest row count whose byte size fits 31 bits).
__device__ __forceinline__ rsrc_t rsrc_rows(const unsigned char* base, int rows_left, int row_bytes, int max_rows) {
    const int n = rows_left <= 0 ? 0 : (rows_left >= max_rows ? 0x7FFFFFFF : rows_left * row_bytes);
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return (rsrc_t){__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                    __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu)),
                    __builtin_amdgcn_readfirstlane(n), 0x00020000};
}

// Source rows of a tile copy: rows [0, rows) of a row-major matrix starting
// at base (wave-uniform; rows past the end read as zero).  at(r0) is the
// descriptor of the rows from r0 on: a copy that starts r0 rows further down
// shifts the descriptor rather than its lane offsets (scalar work).
struct RowSrc {
    const unsigned char* base;
    int rows, row_bytes, max_rows;
    __device__ __forceinline__ rsrc_t at(int r0) const {
        return rsrc_rows(base + (size_t)r0 * row_bytes, rows - r0, row_bytes, max_rows);
    }
    // the same matrix seen from r0 rows further down
    __device__ __forceinline__ RowSrc shifted(int r0) const {
        return RowSrc{base + (size_t)r0 * row_bytes, rows - r0, row_bytes, max_rows};
    }
};

// nrows rows of row_bytes each, starting at row row0 of `matrix`.
__device__ __forceinline__ RowSrc row_src(const void* matrix, size_t row0, int nrows, int row_bytes) {
    const unsigned char* m = uniform_ptr(static_cast<const unsigned char*>(matrix) + row0 * (size_t)row_bytes);
    return RowSrc{m, nrows, row_bytes, row_bytes > 0 ? 0x7FFFFFFF / row_bytes : 0x7FFFFFFF};
}

// LDS byte address of a pointer into smem.
__device__ __forceinline__ uint32_t lds_addr(const unsigned char* p) {
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(base + (uint32_t)(p - smem)));
}

// 16 (or 4) bytes per lane from byte offset voff into LDS at wave_dst + 16 L
// (4 L).  The copies are issued from inline assembly: the compiler does not
// track them, so it adds no vmcnt waits of its own in front of later LDS
// reads (with the builtin it waits for every copy in flight before each
// ds_read_b64_tr_b16).  The kernels order copies and reads themselves: a
// stage is read only after wait_vm / wait_vm_n and a barrier, and a copy
// into a stage is issued only after a barrier that follows its last read.
// M0 holds the LDS base of the copy; the s_nop covers the M0 -> LDS-DMA hazard.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(rsrc_t r, unsigned char* wave_dst, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_addr(wave_dst)), "v"(voff), "s"(r)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(rsrc_t r, unsigned char* wave_dst, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(lds_addr(wave_dst)), "v"(voff), "s"(r)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
// s_waitcnt vmcnt(0): this wave's copies (and loads) have landed.
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Per-lane global offsets of one ROWS x (8 L) fp16 tile copied by NW waves.
// LDS chunk slot p (16 bytes) of the tile is row p / L, position p % L; it
// receives global chunk (p % L) ^ swz<L>(row) of that row.  Copy u of wave w
// fills slots (NW u + w) * 64 + lane, i.e. rows (NW u + w) * 64 / L + lane / L.
// The swizzle term depends on the row modulo 16, so it repeats every PERIOD
// copies (PERIOD = 1 when a round of NW copies spans a multiple of 16 rows):
// PERIOD offsets per lane plus whole rounds of rows cover all of the wave's
// copies.
template <int ROWS, int L, int NW>
struct TileDma {
    static constexpr int LOADS = ROWS * L / 64;  // wave-sized copies per tile
    static constexpr int PER_WAVE = (LOADS + NW - 1) / NW;
    static constexpr int MIN_PER_WAVE = LOADS / NW;  // copies issued by every wave
    static constexpr int RPR = NW * 64 / L;          // rows per round of NW copies
    static constexpr int PERIOD = RPR % 16 == 0 ? 1 : 16 / RPR;
    static_assert(RPR % 16 == 0 || 16 % RPR == 0, "round must divide or be a multiple of 16 rows");
    uint32_t voff0[PERIOD];  // offsets of copies 0 .. PERIOD-1 (kOob for chunks past D)
    uint32_t row_step;       // bytes between copies u and u + PERIOD

    // row_bytes: global row pitch; valid_chunks: 16-byte chunks inside D.
    __device__ __forceinline__ void init(int wave, int lane, int row_bytes, int valid_chunks) {
#pragma unroll
        for (int q = 0; q < PERIOD; ++q) {
            const int slot = (NW * q + wave) * 64 + lane;
            const int r = slot / L;
            const int c = (slot % L) ^ swz<L>(r);
            voff0[q] = c < valid_chunks ? (uint32_t)(r * row_bytes + c * 16) : kOob;
        }
        row_step = (uint32_t)(PERIOD * RPR * row_bytes);
    }
    __device__ __forceinline__ void issue(rsrc_t rs, unsigned char* tile, int wave) const {
#pragma unroll
        for (int u = 0; u < PER_WAVE; ++u)
            if (LOADS % NW == 0 || u * NW + wave < LOADS)
                dma16(rs, tile + (u * NW + wave) * 1024, voff0[u % PERIOD] + (u / PERIOD) * row_step);
    }
};

// s_waitcnt vmcnt(N): at most N of this wave's loads still in flight.
template <int N>
__device__ __forceinline__ void wait_vm_n() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 15] (n > 15 waits for 15).
__device__ __forceinline__ void wait_vm_upto(int n) {
    switch (n) {
        case 0: wait_vm_n<0>(); break;
        case 1: wait_vm_n<1>(); break;
        case 2: wait_vm_n<2>(); break;
        case 3: wait_vm_n<3>(); break;
        case 4: wait_vm_n<4>(); break;
        case 5: wait_vm_n<5>(); break;
        case 6: wait_vm_n<6>(); break;
        case 7: wait_vm_n<7>(); break;
        case 8: wait_vm_n<8>(); break;
        case 9: wait_vm_n<9>(); break;
        case 10: wait_vm_n<10>(); break;
        case 11: wait_vm_n<11>(); break;
        case 12: wait_vm_n<12>(); break;
        case 13: wait_vm_n<13>(); break;
        case 14: wait_vm_n<14>(); break;
        default: wait_vm_n<15>(); break;
    }
}

// Workgroup id -> (batch, tile), XCD-major: ids are dealt round-robin over
// the 8 XCDs (id % 8); XCD x owns a contiguous range of the batch-major tile
// list (B tiles-long rows), so the K/V (or Q/dO) rows a tile streams are
// shared in that XCD's L2 by the other tiles of its batch row.  The XCD
// splits its range into the fewest chunks of at most `wcap` rows' worth of
// tiles (equal sizes, +-1) and runs each chunk rank-major: rank 0 (the
// heaviest tile of a row when `reverse`, which runs a row's tiles last-first)
// of every row in the chunk, then rank 1, and so on.  The heavy tiles of a
// chunk's rows thus start together and the light ones fill the end of the
// launch; row by row, the last rows' heavy tiles started late and ran alone.
// A chunk may begin or end inside a row (when B is not a multiple of 8, or
// wcap does not divide B / 8): at each rank its rows are still a contiguous
// interval.  wcap = 1 with whole rows per XCD is plain row order;
// row_window() picks wcap.
__host__ __device__ __forceinline__ void xcd_map(int bid, int nblocks, int tiles, bool reverse, int wcap, int& b,
                                                  int& t) {
    const int xcd = bid & 7, local = bid >> 3;
    const int per = nblocks >> 3, rem = nblocks & 7;
    const int n_x = per + (xcd < rem ? 1 : 0);
    const int s_x = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
    // chunk of `local`: nch chunks, the first `extra` of them one longer (the
    // cap in 64 bits: a one-row side against a long other side makes
    // wcap * tiles exceed 2^31)
    const long long cap = (long long)wcap * tiles;
    const int nch = cap >= n_x ? 1 : (n_x + (int)cap - 1) / (int)cap;
    const int base = n_x / nch, extra = n_x - base * nch;
    int cs, size;
    if (local < extra * (base + 1)) {
        cs = (local / (base + 1)) * (base + 1);
        size = base + 1;
    } else {
        cs = extra * (base + 1) + ((local - extra * (base + 1)) / base) * base;
        size = base;
    }
    const int k = local - cs;  // position in the chunk's rank-major order
    cs += s_x;
    // rows r0 .. r1 of the chunk: r0 holds ranks p0 .. tiles-1, r1 ranks 0 .. p1
    const int r0 = cs / tiles, r1 = (cs + size - 1) / tiles;
    const int p0 = cs - r0 * tiles, p1 = cs + size - 1 - r1 * tiles;
    int q, row;
    if (r0 == r1) {
        q = p0 + k;
        row = r0;
    } else {
        // At rank q the rows are r0 + (q < p0) .. r1 - (q > p1), so the count
        // is d = r1 - r0 below a = min(p0, p1 + 1) and from c = max(p0, p1 + 1)
        // on, and d + 1 (p0 <= p1) or d - 1 (p0 > p1) in between.
        const int d = r1 - r0;
        const bool inner = p0 <= p1;
        const int a = inner ? p0 : p1 + 1, c = inner ? p1 + 1 : p0;
        const int dm = inner ? d + 1 : d - 1;
        const int n0 = a * d, n1 = (c - a) * dm;
        if (k < n0) {
            q = k / d;
            row = r0 + 1 + (k - q * d);
        } else if (k < n0 + n1) {
            const int kk = k - n0, j = kk / dm;
            q = a + j;
            row = (inner ? r0 : r0 + 1) + (kk - j * dm);
        } else {
            const int kk = k - n0 - n1, j = kk / d;
            q = c + j;
            row = r0 + (kk - j * d);
        }
    }
    b = row;
    t = reverse ? tiles - 1 - q : q;
}

// The xcd_map chunk cap for rows that each stream row_bytes: as many rows as
// stream at most 8 MiB (at least one), so a chunk's working set stays
// bounded.  c4 (2 MiB per row, 16 rows per XCD) gets 4; c3 (0.5 MiB, 32 rows
// per XCD) 16.
inline int row_window(size_t row_bytes) {
    const size_t w = row_bytes ? ((size_t)8 << 20) / row_bytes : 1;
    return w < 1 ? 1 : (w > (1 << 20) ? (1 << 20) : (int)w);
}

// Two fp32 values -> one dword of two RNE-rounded halves (v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, half2v));
}

__device__ __forceinline__ half8 half8_of(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(half8, (u4){w0, w1, w2, w3});
}

// Per-lane LDS byte offsets of the MFMA A-operand reads from a swizzled
// fp16 tile with L 16-byte chunks per row (see swz_off).  The swizzle only
// permutes chunks inside a 16 L-byte row and every tile base is a multiple of
// 256 bytes, so each read is (tile base + lane term) ^ constant, with the
// tile's row offset in the instruction's immediate field:
//   row read,  rows R0 + l32 (R0 % 16 == 0), features 16 ks + 8 hh .. +7:
//              ((base + row) ^ (32 ks)) + 16 L R0
//   transposed read of rows R0 + 16 s + {tr_row, tr_row + 8} (see
//   lds_read_tr), features 32 dt + tr_col:
//              ((base + tr[j]) ^ (64 dt)) + 16 L (R0 + 16 s)
template <int L>
struct SwzLane {
    uint32_t row, tr0, tr1;
    __device__ __forceinline__ void init(int lane) {
        const int l32 = lane & 31, hh = lane >> 5;
        row = (uint32_t)(l32 * 16 * L + 16 * (hh ^ swz<L>(l32)));
        const int g16 = lane >> 4, i16 = lane & 15;
        const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
        const int c = 2 * (g16 & 1) + ((i16 & 3) >> 1);  // chunk of column tr_col within 32 features
        const int sub = 8 * (i16 & 1);                   // byte of column tr_col within its chunk
        tr0 = (uint32_t)(tr_row * 16 * L + 16 * (c ^ swz<L>(tr_row)) + sub);
        tr1 = (uint32_t)((tr_row + 8) * 16 * L + 16 * (c ^ swz<L>(tr_row + 8)) + sub);
    }
};

// max(x, 0) of eight finite halves as a signed 16-bit max on their bit
// patterns (a set sign bit is a negative int16), one v_pk_max_i16 per pair.
__device__ __forceinline__ half8 relu_h8(half8 x) {
    typedef short short8 __attribute__((ext_vector_type(8)));
    return __builtin_bit_cast(half8, __builtin_elementwise_max(__builtin_bit_cast(short8, x), short8{}));
}

// Row-read A operand: rows R0 + l32 (R0 % 16 == 0), k-step ks.
// `a` = tile base + SwzLane::row.
template <int L>
__device__ __forceinline__ half8 lds_row(uint32_t a, int ks, int R0) {
    return *reinterpret_cast<const half8*>(smem + ((a ^ (uint32_t)(32 * ks)) + 16 * L * R0));
}

// Transposed A operand: tile rows R0 .. R0 + 15 (R0 % 16 == 0) in the order
// of the accumulator layout, features 32 dt + (0..31).
// a0 / a1 = tile base + SwzLane::tr0 / tr1.
template <int L>
__device__ __forceinline__ half8 lds_tr(uint32_t a0, uint32_t a1, int dt, int R0) {
    const half4 x0 = lds_read_tr(reinterpret_cast<const half_t*>(smem + ((a0 ^ (uint32_t)(64 * dt)) + 16 * L * R0)));
    const half4 x1 = lds_read_tr(reinterpret_cast<const half_t*>(smem + ((a1 ^ (uint32_t)(64 * dt)) + 16 * L * R0)));
    return __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Store 16 fp32 accumulator rows of a C^T tile (lane = output row, in-lane =
// features 32 dt + 8 g + 4 hh + e) as fp16 with a common factor.
template <int DN>
__device__ __forceinline__ void store_rows_f16(half_t* dst, const floatx16 (&acc)[DN / 32], float f, int hh) {
#pragma unroll
    for (int dt = 0; dt < DN / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            half4 hv;
#pragma unroll
            for (int e = 0; e < 4; ++e) hv[e] = (half_t)(acc[dt][4 * g + e] * f);
            *reinterpret_cast<half4*>(dst + 32 * dt + 8 * g + 4 * hh) = hv;
        }
}

// Same, columns >= ncols not written (D < padded width).
template <int DN>
__device__ __forceinline__ void store_rows_f16_n(half_t* dst, const floatx16 (&acc)[DN / 32], float f, int hh,
                                                 int ncols) {
#pragma unroll
    for (int dt = 0; dt < DN / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * dt + 8 * g + 4 * hh;
            if (d0 < ncols) {
                half4 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[e] = (half_t)(acc[dt][4 * g + e] * f);
                *reinterpret_cast<half4*>(dst + d0) = hv;
            }
        }
}

// ---------------------------------------------------------------------------
// Loop-invariant addressing.  Kernels whose LDS stages are unrolled keep each
// lane's read addresses in registers (absolute LDS byte addresses, the
// dynamic LDS base included) and add the stage / row offsets as instruction
// immediates, so a step issues no address arithmetic.
// ---------------------------------------------------------------------------

// Byte address of smem[0] in LDS (0 for a kernel without static LDS).
__device__ __forceinline__ uint32_t lds_base() {
    return (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem);
}

// 16 bytes from absolute LDS address a (ds_read_b128).
__device__ __forceinline__ half8 ld_b128(uint32_t a) {
    return *reinterpret_cast<const __attribute__((address_space(3))) half8*>((uintptr_t)a);
}

// ds_read_b64_tr_b16 from absolute LDS address a (lane layout: lds_read_tr).
__device__ __forceinline__ half4 ld_tr(uint32_t a) {
    return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                         reinterpret_cast<__attribute__((address_space(3))) fp16x4_tr*>((uintptr_t)a)));
}

// Transposed A operand from two lane addresses (SwzLane::tr0 / tr1 forms).
__device__ __forceinline__ half8 ld_tr8(uint32_t a0, uint32_t a1) {
    return __builtin_shufflevector(ld_tr(a0), ld_tr(a1), 0, 1, 2, 3, 4, 5, 6, 7);
}

// One 16-byte-per-lane copy to absolute LDS address m0 (wave-uniform) + 16 L.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_at(rsrc_t r, uint32_t m0, uint32_t voff) {
    // readfirstlane: the operands are wave-uniform; it only moves a value the
    // compiler happened to keep in a VGPR into an SGPR (a no-op otherwise)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane((int)m0)), "v"(voff), "s"(r)
                 : "memory", "m0");
}
// The same with the non-temporal hint, for data read once (the stored dS of
// the backward's dS path): L2 keeps the tiles that are read again.
__device__ __forceinline__ void dma16_at_nt(rsrc_t r, uint32_t m0, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane((int)m0)), "v"(voff), "s"(r)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Chunk swizzle of a tile that is only ever read transposed
// (ds_read_b64_tr_b16; pattern (b) of swz): it needs rows r0..r0+3 of a
// 4-row group to land on distinct bank groups, which 4 (r % 4) does for
// 256-byte rows (L = 16) and 4 ((r / 2) % 2) for 128-byte rows (L = 8);
// 64-byte rows (L = 4) need none.  Rows r and r + 8 then share a swizzle, so
// the two transposed reads of an MFMA operand differ by an immediate.
template <int L>
__device__ __forceinline__ int swz_tr(int r) {
    static_assert(L == 4 || L == 8 || L == 16, "swizzle defined for 32/64/128-wide fp16 rows");
    if constexpr (L == 16) return 4 * (r & 3);
    else if constexpr (L == 8) return 4 * ((r >> 1) & 1);
    else return 0;
}

// Lane offset of the transposed read of a swz_tr tile: rows R0 + tr_row
// (and + 8 at +128 L bytes), features 32 dt + tr_col; see SwzLane.
template <int L>
__device__ __forceinline__ uint32_t tr_lane_off(int lane) {
    const int g16 = lane >> 4, i16 = lane & 15;
    const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
    const int c = 2 * (g16 & 1) + ((i16 & 3) >> 1);
    const int sub = 8 * (i16 & 1);
    return (uint32_t)(tr_row * 16 * L + 16 * (c ^ swz_tr<L>(tr_row)) + sub);
}

// Copies of one ROWS x (8 L) fp16 tile by NW waves in the layout of TileDma
// (copy u of wave w fills LDS chunk slots (NW u + w) * 64 + lane, i.e. rows
// (NW u + w) * 64 / L + lane / L).  When a round of NW copies spans a
// multiple of 16 rows, every copy of a wave uses the lane offset of its first
// copy and a descriptor u whole rounds further down; a tile of fewer than NW
// copies is issued by waves 0 .. LOADS - 1, one each.  TR selects the swz_tr
// layout (tiles read only transposed).
template <int ROWS, int L, int NW, bool TR = false>
struct TileCopy {
    static constexpr int LOADS = ROWS * L / 64;
    static constexpr int PER_WAVE = LOADS >= NW ? LOADS / NW : 1;  // copies of an issuing wave
    static constexpr int RPR = NW * 64 / L;                          // rows per round of NW copies
    static_assert(LOADS >= NW ? (LOADS % NW == 0 && RPR % 16 == 0) : true,
                  "every wave issues the same number of copies; the swizzle repeats every round");
    uint32_t voff;  // lane offset of copy 0 (kOob for chunks past D)
    __device__ __forceinline__ void init(int wave, int lane, int row_bytes, int valid_chunks) {
        const int slot = wave * 64 + lane;
        const int r = slot / L;
        const int c = (slot % L) ^ (TR ? swz_tr<L>(r) : swz<L>(r));
        voff = c < valid_chunks ? (uint32_t)(r * row_bytes + c * 16) : kOob;
    }
    // copies this wave issues per tile
    __device__ __forceinline__ static int count(int wave) { return LOADS >= NW ? PER_WAVE : (wave < LOADS ? 1 : 0); }
    // m0wave = absolute LDS address of the tile + 1024 * wave; copy u reads
    // the rows from u * RPR on: one descriptor for the tile, the row offset
    // added to the lane offset (an out-of-range lane offset stays out of
    // range: kOob + PER_WAVE * RPR * row_bytes < 2^32).
    __device__ __forceinline__ void issue(const RowSrc& src, uint32_t m0wave, int wave) const {
        if (LOADS < NW && wave >= LOADS) return;
        const rsrc_t rs = src.at(0);
        const uint32_t step = (uint32_t)(RPR * src.row_bytes);
#pragma unroll
        for (int u = 0; u < PER_WAVE; ++u) dma16_at(rs, m0wave + (uint32_t)(u * NW * 1024), voff + (uint32_t)u * step);
    }
};
}  // namespace
}  // namespace sdpa
