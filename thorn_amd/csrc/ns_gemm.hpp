// Newton-Schulz GEMMs on gfx950: f16 MFMA (v_mfma_f32_32x32x16_f16), fp32 accumulation, operand
// tiles streamed global -> LDS by buffer DMA through a 4-stage ring, grouped launches over every
// matrix of a parameter group (ns_kernels.hip).
//
// One main loop (gemm_tile) serves every product of both Newton-Schulz schedules: Gram matrices
// X X^T / X^T X, products of s x s workspace matrices, and iterate updates Q X / X Q. Operands are
// read either K-major (ds_read_b128 fragments) or MN-major (two ds_read_tr16_b64 transposing
// reads), so no matrix is ever transposed in memory.
//
// A block is 512 threads, two waves per SIMD, and the two waves of a SIMD take turns: while the
// waves of one group issue nothing but MFMAs on fragments already in their registers, the waves
// of the other group read their next fragments from LDS, issue the direct loads of a later K
// tile and wait for them; a block barrier hands the MFMA pipes over. A wave's memory waits
// therefore never hold up the MFMA pipe of its SIMD. (With one wave per SIMD interleaving its
// loads between its MFMAs, measured on an MI355X: ~1400-1460 cycles per K tile of 32 at
// K = 1024 against 1200-1330 this way, and 1210 against 1050-1070 at K = 8192, 1024 being the
// MFMA time; the chip runs this load power-limited at 1.4-1.6 GHz either way.)
#pragma once

#include <type_traits>

#include "thorn_common.hpp"

namespace thorn {

// The start of a tile's main loop, for the per-block timestamps of a measurement build
// (-DTHORN_BLOCK_TIMESTAMPS; ns_kernels.hip); nothing otherwise.
__device__ __forceinline__ void ts_loop_start();

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Block tile 256 x 256, K step 32, 4 pipeline stages of LDS, 512 threads. SIMD s owns the
// 128 x 128 quadrant (s >> 1, s & 1) of a tile; its wave of group 0 (wave s) the left 64 columns
// of it, its wave of group 1 (wave s + 4) the right 64.
struct NsCfg {
    static constexpr int BM = 256, BN = 256, BK = 32, S = 4;
    static constexpr int NT = 512, NW = NT / 64;
    static constexpr int A_BYTES = BM * BK * 2;          // one stage of A, no padding
    static constexpr int B_BYTES = BN * BK * 2;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int LDS_BYTES = S * STAGE_BYTES;    // 128 KB
    static constexpr int A_LOADS = A_BYTES / 1024 / NW;  // 1 KB direct loads per wave per stage
    static constexpr int B_LOADS = B_BYTES / 1024 / NW;
    static constexpr int LOADS = A_LOADS + B_LOADS;      // 4
    static_assert(A_LOADS == B_LOADS && LOADS == 4, "per-wave load slots");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

// A GEMM operand in global memory (f16). Its layout is a compile-time property of the main loop
// (template flag KM):
//   K-major  (KM):  element (mn, k) at ptr[mn * ld + k]   (rows = number of valid mn rows)
//   MN-major (!KM): element (mn, k) at ptr[k * ld + mn]   (rows = number of valid k rows)
// ld is a multiple of 32 and the padding columns [logical width, ld) hold zeros, so a K tile of
// a K-major row is either entirely inside the row or entirely past its end; rows * ld * 2 bytes
// is below 2^30 (checked when a plan is created), so every byte offset of the loop, out-of-range
// ones included, fits 32 bits.
// packed: a symmetric s x s matrix (rows = s, ld = its padded width) stored as the panels of its
// upper block triangle (SqPanel): element (i, j), j >= 256 * (i / 256), of block row b = i / 256
// at ptr[panel_off(b) + (i - 256 b) * panel_ld(b) + j - 256 b]. Its operand rows start at a
// multiple of 256 (one block row), read K-major in its own panel from its diagonal block on, and
// MN-major before it, block by block from the mirror blocks in the panels above.
struct Operand {
    const _Float16* ptr;
    int64_t ld;
    int32_t rows;
    int32_t packed;
};

// The panels of a packed s x s matrix with padded width ld (a multiple of 32): panel b holds block
// row b, rows [256 b, min(256 b + 256, s)) and columns [256 b, ld), with row length ld - 256 b.
struct SqPanel {
    int64_t off;   // elements from the matrix's base
    int64_t ld;
    int32_t rows;
};
__host__ __device__ __forceinline__ int64_t panel_off(int64_t ld, int64_t b) { return 256 * (b * ld - 128 * b * (b - 1)); }
__host__ __device__ __forceinline__ SqPanel sq_panel(int s, int64_t ld, int b) {
    SqPanel p;
    p.off = panel_off(ld, b);
    p.ld = ld - 256 * b;
    p.rows = s - 256 * b < 256 ? s - 256 * b : 256;
    return p;
}
// Elements of a packed s x s matrix (all of its panels).
__host__ __device__ __forceinline__ int64_t packed_elems(int s, int64_t ld) {
    const int last = (s + 255) / 256 - 1;
    const SqPanel p = sq_panel(s, ld, last);
    return p.off + p.rows * p.ld;
}

// Byte offset past the end of every operand: the hardware range check of a buffer access turns it
// into a zero load or a dropped store.
constexpr uint32_t kOutOfRange = 0x80000000u;

// Raw buffer resource over [p, p + bytes), held in scalar registers (wave-uniform).
__device__ __forceinline__ u32x4 sgpr_rsrc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    u32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    r[1] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32)) & 0xFFFFu;
    r[2] = __builtin_amdgcn_readfirstlane(bytes);
    r[3] = 0x00020000u;
    return r;
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// Makes v opaque to the compiler: it is kept in registers as computed, and every later use reads
// those bits (the compiler may not recompute it another way).
__device__ __forceinline__ void opaque(half4& v) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    u32x2 b = __builtin_bit_cast(u32x2, v);
    asm volatile("" : "+v"(b));
    v = __builtin_bit_cast(half4, b);
}

// LDS layouts of one stage, 16-byte chunks, XOR-swizzled so that the fragment reads of a wave
// hit distinct banks:
//   K-major:  MN rows x 4 chunks (64 B); chunk c of row r sits at r*64 + (c ^ ((r >> 2) & 3))*16.
//             16 lanes reading rows r..r+15 at one chunk cover all 64 banks.
//   MN-major: 32 k-rows x MN/8 chunks; chunk c of k-row k at k*MN*2 + (c ^ ((k & 3) << 2))*16.
//             The 32 lanes of a ds_read_tr16_b64 pair read 4 k-rows x 4 chunks: 16 distinct
//             chunks mod 16, all 64 banks.
// A direct load writes 64 consecutive chunk slots (1 KB) at the address in M0, so each lane loads
// the global chunk whose swizzled position is its slot. Wave w owns slots [1024 (w P + q),
// 1024 (w P + q + 1)) of an operand's stage, q < P = PER_WAVE.
//
// OperandDma holds the buffer resource of one operand and, per lane, the byte offset of each of
// its chunk loads per stage for the next K tile to load (`cur`, advanced by `step` after each
// load). Loads of consecutive tiles are issued in order; begin_tile switches the offsets to the
// K-major layout at tile k0 (a symmetric matrix stored as its upper block triangle is read
// MN-major, from the transposed mirror block, before its diagonal block) and to out of range at
// tile kend, so the tiles that round K up to whole loop iterations, and the prefetches past the
// end, load zeros.
template <int MN>
struct OperandDma {
    static constexpr int PER_WAVE = MN * NsCfg::BK * 2 / 1024 / NsCfg::NW;
    static constexpr int KB = 256 / NsCfg::BK;   // K tiles per 256-block of a packed operand
    u32x4 rsrc;
    uint32_t cur[PER_WAVE];
    uint32_t kmaj[PER_WAVE];   // K-major offsets of tile 0 (a packed operand: as if its panel began at tile 0)
    uint32_t step;             // bytes per K tile in the current layout
    int k0, kend;
    // a packed operand: the matrix's padded width (its rows start at 32 k0); else 0. Held in a
    // vector register (the same in every lane): it is read once per 256 of K in the MN-major
    // part only, and the main loop has no scalar register to spare for it.
    int pwv;

    // K-major offsets of rows [mn0, mn0 + MN) in a layout with row stride ld from element base
    // (rows below `rows` valid), minus `back` bytes
    __device__ __forceinline__ static void km_offsets(int mn0, int rows, int64_t base, int64_t ld, int wave, int lane,
                                                      uint32_t back, uint32_t (&o)[PER_WAVE]) {
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const int slot = (wave * PER_WAVE + q) * 64 + lane;
            const int r = slot >> 2, pc = slot & 3;
            const int c = pc ^ ((r >> 2) & 3);
            o[q] = mn0 + r < rows ? static_cast<uint32_t>((base + int64_t(r) * ld + c * 8) * 2) - back : kOutOfRange;
        }
    }

    // MN-major offsets of columns [mn0, mn0 + MN) (those below cmax valid) of one K tile's 32 rows,
    // row stride ld, column c at element base + c - cshift
    __device__ __forceinline__ static void mn_offsets(int mn0, int cmax, int64_t base, int64_t ld, int cshift, int wave,
                                                      int lane, uint32_t (&o)[PER_WAVE]) {
        constexpr int CH = MN / 8;
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const int slot = (wave * PER_WAVE + q) * 64 + lane;
            const int k = slot / CH, pc = slot % CH;
            const int c = pc ^ ((k & 3) << 2);
            const int col = mn0 + c * 8;
            o[q] = col < cmax ? static_cast<uint32_t>((base + int64_t(k) * ld + col - cshift) * 2) : kOutOfRange;
        }
    }

    __device__ __forceinline__ void init(const Operand& op, int mn0, int wave, int lane, int k0_, int kend_) {
        k0 = k0_;
        kend = kend_;
        pwv = op.packed ? static_cast<int>(op.ld) : 0;
        asm volatile("" : "+v"(pwv));
        if (op.packed) {   // block row b = mn0 / 256 (k0 = KB b): K-major in panel b from tile k0 on
            const SqPanel last = sq_panel(op.rows, op.ld, (op.rows + 255) / 256 - 1);
            rsrc = sgpr_rsrc(op.ptr, static_cast<uint32_t>((last.off + last.rows * last.ld) * 2));
            const SqPanel pb = sq_panel(op.rows, op.ld, mn0 / 256);
            km_offsets(0, pb.rows, pb.off, pb.ld, wave, lane, static_cast<uint32_t>(64 * k0), kmaj);
        } else {
            rsrc = sgpr_rsrc(op.ptr, static_cast<uint32_t>(int64_t(op.rows) * op.ld * 2));
            km_offsets(mn0, op.rows, int64_t(mn0) * op.ld, op.ld, wave, lane, 0u, kmaj);
        }
        if (k0 <= 0) {
#pragma unroll
            for (int q = 0; q < PER_WAVE; ++q) cur[q] = kmaj[q];
            step = 64;
        } else {   // MN-major from tile 0: a packed operand's block 0 is in panel 0, row stride ld
            mn_offsets(mn0, static_cast<int>(op.ld), 0, op.ld, 0, wave, lane, cur);
            step = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(64 * op.ld));
        }
    }

    // Called before the first load of tile t, for t = 0, 1, 2, ... in order (t is wave-uniform: a
    // scalar branch).
    __device__ __forceinline__ void begin_tile(int t) {
        if (t == k0 && t > 0 && t < kend) {
#pragma unroll
            for (int q = 0; q < PER_WAVE; ++q) cur[q] = kmaj[q] + 64u * t;
            step = 64;
        }
        if (t == kend) {
#pragma unroll
            for (int q = 0; q < PER_WAVE; ++q) cur[q] = kOutOfRange;
        }
    }

    // Tile t (a multiple of KB, read MN-major: t < k0) starts block b = t / KB; a packed operand
    // holds it in panel b. The offsets move there by a constant: having walked the 256 rows of
    // block b - 1, a lane at k-row k of the tile and column j is at
    //   P(b-1) + (256 + k) ld(b-1) + j - 256 (b-1),
    // and P(b) = P(b-1) + 256 ld(b-1), ld(b) = ld(b-1) - 256 put element (256 b + k, j) at
    //   P(b) + k ld(b) + j - 256 b = that - 256 (k + 1);
    // the step (32 rows) shrinks by 32 * 256 elements. Lanes out of range stay out of range (they
    // have moved by at least 8 steps).
    __device__ __forceinline__ void next_panel() {
        if (__builtin_amdgcn_readfirstlane(pwv) == 0) return;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
        constexpr int CH = MN / 8;
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const int k = ((wave * PER_WAVE + q) * 64 + lane) / CH;
            cur[q] -= static_cast<uint32_t>(512 * (k + 1));
        }
        step -= 2 * 32 * 256;
    }

    // Direct load q of this wave for the current tile into LDS at m0 (wave-uniform byte address).
    // The compiler writes M0 right before the asm, whose s_nop gives the one wait state that an
    // M0 write needs before an LDS DMA reads it (a hazard the compiler does not see inside asm).
    // It is inline assembly so that the compiler does not track it as an LDS write: its
    // conservative aliasing would otherwise wait for every outstanding load before the next LDS
    // fragment read and serialize the pipeline. The main loop orders the loads explicitly
    // (waits and barriers); the "memory" clobber keeps LDS accesses from moving across them.
    __device__ __forceinline__ void issue(int q, uint32_t m0) {
        asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(cur[q]), "s"(rsrc), "{m0}"(m0) : "memory");
        cur[q] += step;
    }
};

// The C term of a tile's epilogue (out = f16(alpha * A B + beta * C)): the f16 tile of C at rows
// m0.., columns n0.. of a matrix with leading dimension ld and `rows` valid rows (ptr null: no C
// term, every load reads zeros). gemm_tile loads it into the epilogue's staging (EpiH) by direct
// loads: rows 192-255 in the prologue, into the 32 KB past the pipeline stages, and rows 0-63,
// 64-127 and 128-191 in the last three memory phases, into stages 0, 1 and 2 as the loop
// releases them (in place of the loads of tiles past the end, so every memory phase still issues
// one stage's share of loads per wave). Quarter q of the tile is 32 loads of two 512-byte
// staging rows each; wave w issues loads 4w .. 4w+3.
// r0, c0: the matrix row and column at ptr (a panel of a packed matrix; 0 otherwise), rows the
// valid rows from there.
struct TileC {
    const _Float16* ptr;
    int64_t ld;
    int32_t rows;
    int32_t r0, c0;
};

struct TileCDma {
    static constexpr int PER_WAVE = 32 / NsCfg::NW;
    u32x4 rsrc;
    uint32_t off[PER_WAVE];   // quarter 0 offsets of this lane's loads; quarter q adds q * qstep
    uint32_t qstep;           // bytes of 64 rows
    __device__ __forceinline__ void init(const TileC& c, int m0, int n0, int wave, int lane) {
        rsrc = sgpr_rsrc(c.ptr, c.ptr ? static_cast<uint32_t>(int64_t(c.rows) * c.ld * 2) : 0u);
        qstep = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(128 * c.ld));
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            const int row = 2 * (wave * PER_WAVE + j) + (lane >> 5);   // within quarter 0
            const int ch = (lane & 31) ^ (row & 31);                    // staging position lane & 31
            const int col = n0 + 8 * ch;
            off[j] = col < c.ld ? static_cast<uint32_t>((int64_t(m0 + row) * c.ld + col) * 2) : kOutOfRange;
        }
    }
    // load j of quarter q into LDS at m0 (wave-uniform)
    __device__ __forceinline__ void issue(int j, int q, uint32_t m0) {
        const uint32_t o = off[j] + q * qstep;
        asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(o), "s"(rsrc), "{m0}"(m0) : "memory");
    }
};

typedef __attribute__((address_space(3))) short4v lds_s4;
typedef __attribute__((address_space(3))) const half8 lds_h8;

// MFMA fragment (8 halves) for the 32-wide sub-tile at `t0` and k16 step `ks` of a stage, at a
// computed address (the small-matrix kernel's reads).
template <int MN, bool KM>
__device__ __forceinline__ half8 frag(const char* lds, int t0, int ks, int lane) {
    if (KM) {
        const int r = t0 + (lane & 31);
        const int c = 2 * ks + (lane >> 5);
        return *reinterpret_cast<const half8*>(lds + r * 64 + ((c ^ ((r >> 2) & 3)) << 4));
    }
    const int k = 16 * ks + 8 * (lane >> 5) + ((lane & 15) >> 2);
    const int mn = t0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int c = mn >> 3, off = (mn & 7) * 2;
    const char* p0 = lds + k * (MN * 2) + ((c ^ ((k & 3) << 2)) << 4) + off;
    const char* p1 = lds + (k + 4) * (MN * 2) + ((c ^ (((k + 4) & 3) << 2)) << 4) + off;
    short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0));
    short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p1));
    half4 l4 = __builtin_bit_cast(half4, lo), h4 = __builtin_bit_cast(half4, hi);
    return half8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
}

// Per-lane LDS fragment bases of one operand of the main loop (operand tiles of MN = 256): the
// 32-wide fragments I = 0 .. NI-1 at columns (or rows) w0 + 32 I. The four stages are two pairs
// 65536 bytes apart, so that every other part of an address fits the 16-bit immediate offset of
// the read:
//   K-major: b[pair][ks]; the wave's row offset is in the base, fragment I adds I * 2048 (32 rows
//            of 64 B) and the odd stage of a pair 32768.
//   MN-major: b[pair][I] per fragment (the XOR swizzle of chunk c = 4j + cl by 4x is 4(j ^ x) + cl
//            with j the fragment's 32-column block and x = k & 3 the lane's, so the fragment's part
//            is lane-dependent); ks adds 16 k-rows (8192 B) and the second read 4 k-rows (2048 B).
template <int NI>
struct FragBase {
    uint32_t b[2][NI > 2 ? NI : 2];
    __device__ __forceinline__ void init_kmajor(uint32_t lds0, int w0, int lane) {
#pragma unroll
        for (int pr = 0; pr < 2; ++pr)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int r = lane & 31, c = 2 * ks + (lane >> 5);
                b[pr][ks] = lds0 + pr * 65536 + w0 * 64 + r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
            }
    }
    __device__ __forceinline__ void init_mnmajor(uint32_t lds0, int w0, int lane) {
        const int x = (lane >> 2) & 3;
        const int k = 8 * (lane >> 5) + ((lane & 15) >> 2);
        const int cl = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
        const int off = 8 * (lane & 1);
#pragma unroll
        for (int pr = 0; pr < 2; ++pr)
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int j = w0 / 32 + i;
                b[pr][i] = lds0 + pr * 65536 + k * 512 + ((4 * (j ^ x) + cl) << 4) + off;
            }
    }
};

// Fragment I (k16 step KS) of an operand at byte offset OPOFF of stage ST.
template <bool KM, int ST, int KS, int OPOFF, int I, int NI>
__device__ __forceinline__ half8 frag_at(const FragBase<NI>& fb) {
    constexpr int SB = (ST & 1) * 32768;
    if constexpr (KM) {
        constexpr int imm = SB + OPOFF + I * 2048;
        static_assert(imm < 65536, "immediate offset");
        return *reinterpret_cast<lds_h8*>(fb.b[ST >> 1][KS] + imm);
    } else {
        static_assert(I < NI, "fragment base");
        constexpr int imm = SB + OPOFF + KS * 8192;
        static_assert(imm + 2048 < 65536, "immediate offset");
        const uint32_t a = fb.b[ST >> 1][I] + imm;
        short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(a));
        short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(a + 2048));
        half4 l4 = __builtin_bit_cast(half4, lo), h4 = __builtin_bit_cast(half4, hi);
        return half8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
    }
}

// Block barrier for LDS traffic only: this wave's LDS accesses are complete, then s_barrier.
// Unlike __syncthreads() it does not wait for outstanding global stores, so an epilogue's
// stores keep draining while the next staging pass runs.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A bare block barrier between the phases of the main loop. The scheduling barriers keep the
// compiler from moving MFMAs (which are not memory operations) across it.
__device__ __forceinline__ void phase_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// Work split of a tile between the 8 waves, as the 32 x 32 blocks each one computes. A wave's
// blocks are (A fragment a_idx(x), B fragment b_idx(y)) for its block list (x, y), where A
// fragment I covers tile rows abase + 32 I and B fragment J tile columns bbase + 32 J (abase and
// bbase per wave, TileWork). A diagonal tile of a symmetric result is only stored as its upper
// block triangle (the epilogue mirrors it), so of its 8 x 8 grid of blocks only the 36 with
// J >= I are computed:
//   full tile (kRoleFull): each wave its 128 x 64 (A 0-3, B 0-1);
//   diagonal quadrants (SIMDs 0 and 3, base 0 or 128): kRoleDiagA takes block rows {0, 3} of the
//     quadrant's upper triangle (5 blocks: (0,0) .. (0,3), (3,3)), kRoleDiagB rows {1, 2} (5:
//     (1,1) .. (1,3), (2,2), (2,3));
//   upper-right quadrant (SIMDs 1 and 2): kRoleHalf, 64 x 64 each (rows 0-63 or 64-127 of it,
//     columns 0-63 or 64-127 by group);
// nobody computes the lower-left quadrant. The waves of one group then issue at most 5 MFMAs
// per k16 step against 8 on a full tile.
enum TileRole : int { kRoleFull = 0, kRoleDiagA = 1, kRoleDiagB = 2, kRoleHalf = 3 };

template <int ROLE>
struct RoleMap {
    static constexpr int NA = ROLE == kRoleFull ? 4 : 2;                      // A fragments per k16 step
    static constexpr int NB = ROLE == kRoleFull ? 2 : ROLE == kRoleDiagA ? 4 : ROLE == kRoleDiagB ? 3 : 2;
    static constexpr int N = ROLE == kRoleFull ? 8 : ROLE == kRoleHalf ? 4 : 5;   // blocks
    static constexpr int AF = ROLE == kRoleHalf ? 2 : 4;                      // FragBase sizes
    static constexpr int BF = ROLE == kRoleFull || ROLE == kRoleHalf ? 2 : 4;
    // fragment index of A slot x / B slot y
    static constexpr int a_idx(int x) {
        return ROLE == kRoleDiagA ? (x == 0 ? 0 : 3) : ROLE == kRoleDiagB ? 1 + x : x;
    }
    static constexpr int b_idx(int y) { return ROLE == kRoleDiagB ? 1 + y : y; }
    // A slot and B slot of block q
    static constexpr int bx(int q) {
        return ROLE == kRoleFull ? q / 2 : ROLE == kRoleHalf ? q / 2 : ROLE == kRoleDiagA ? (q < 4 ? 0 : 1)
                                                                                          : (q < 3 ? 0 : 1);
    }
    static constexpr int by(int q) {
        return ROLE == kRoleFull ? q % 2 : ROLE == kRoleHalf ? q % 2 : ROLE == kRoleDiagA ? (q < 4 ? q : 3)
                                                                                          : (q < 3 ? q : q - 2);
    }
    // block q lies on the tile's diagonal (diagonal roles only; their A and B bases are equal)
    static constexpr bool on_diag(int q) {
        return (ROLE == kRoleDiagA || ROLE == kRoleDiagB) && a_idx(bx(q)) == b_idx(by(q));
    }
};

// The wave's role and fragment bases in a tile: waves s and s + 4 share SIMD s.
struct TileWork {
    int role, abase, bbase;
    __device__ __forceinline__ TileWork(bool diag, int wave) {
        const int simd = wave & 3, grp = wave >> 2;
        const bool dq = simd == 0 || simd == 3;   // a diagonal quadrant of a diagonal tile
        role = !diag ? kRoleFull : dq ? (grp == 0 ? kRoleDiagA : kRoleDiagB) : kRoleHalf;
        abase = !diag ? (simd >> 1) * 128 : dq ? (simd == 0 ? 0 : 128) : (simd == 1 ? 0 : 64);
        bbase = !diag ? (simd & 1) * 128 + grp * 64 : dq ? abase : 128 + grp * 64;
    }
};

// f(std::integral_constant<int, Q>) for Q = B .. E-1, as straight-line code with Q a constant.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// The fragments of one K tile (both k16 steps) of a role.
template <int ROLE>
struct Frags {
    using R = RoleMap<ROLE>;
    half8 a[2][R::NA];
    half8 b[2][R::NB];
};

// MFMA phase of a K tile: every block's two k16 steps, from registers only. The MFMA is issued as
// B^T A^T, so each 32 x 32 accumulator comes out transposed: lane l holds row (l & 31) and the
// four consecutive columns 8*(r/4) + 4*(l/32) + 0..3 in registers r..r+3.
template <int ROLE>
__device__ __forceinline__ void mfma_phase(const Frags<ROLE>& f, floatx16 (&acc)[RoleMap<ROLE>::N]) {
    using R = RoleMap<ROLE>;
    static_for<0, 2>([&](auto kc) {
        constexpr int ks = decltype(kc)::value;
        static_for<0, R::N>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.b[ks][R::by(q)], f.a[ks][R::bx(q)], acc[q], 0, 0, 0);
        });
    });
}

// Memory phase of K tile kt, held in stage ST = kt % 4: this wave's fragments of tile kt, then its
// share of the direct loads of tile kt+3 into stage (ST+3) % 4 (which both groups finished reading
// before the barrier that started this phase), then the wait for its own loads of tile kt+1 (all
// but the newest two tiles' loads) and for the fragments. CQ >= 0 (the last three memory phases of
// a tile): the loads fetch quarter CQ of the epilogue's C tile into stage CQ instead of a tile
// past the end of K.
template <class C, bool AK, bool BK, int ROLE, int ST, int CQ = -1>
__device__ __forceinline__ void mem_phase(int kt, Frags<ROLE>& f, const FragBase<RoleMap<ROLE>::AF>& ba,
                                          const FragBase<RoleMap<ROLE>::BF>& bb, OperandDma<C::BM>& da,
                                          OperandDma<C::BN>& db, TileCDma& dc, uint32_t m0w, uint32_t lds0) {
    using R = RoleMap<ROLE>;
    static_for<0, 2>([&](auto kc) {
        constexpr int ks = decltype(kc)::value;
        static_for<0, R::NA>([&](auto xc) {
            constexpr int x = decltype(xc)::value;
            f.a[ks][x] = frag_at<AK, ST, ks, 0, R::a_idx(x)>(ba);
        });
        static_for<0, R::NB>([&](auto yc) {
            constexpr int y = decltype(yc)::value;
            f.b[ks][y] = frag_at<BK, ST, ks, C::A_BYTES, R::b_idx(y)>(bb);
        });
    });
    constexpr int SL = (ST + 3) & 3;
    // The layouts switch at a few tiles only (and a packed operand read MN-major changes panel
    // every 256 of K): a scalar branch around the switch (left to itself, the compiler made both
    // switches selects in every memory phase).
    const int t = kt + 3;
    if (t == da.k0 || t == db.k0 || t == da.kend) {
        asm volatile("");
        da.begin_tile(t);
        db.begin_tile(t);
    }
    // Tiles that start a 256-block (t % 8 == 0) are loaded in the phases with ST == 1 only, and
    // an operand changes panel only where it is read MN-major.
    if constexpr (ST == 1 && CQ < 0 && (!AK || !BK)) {
        static_assert(OperandDma<C::BM>::KB == 8, "blocks of 8 K tiles");
        if (t % 8 == 0) {
            if constexpr (!AK) {
                if (t > 0 && t < da.k0) {
                    asm volatile("");
                    da.next_panel();
                }
            }
            if constexpr (!BK) {
                if (t > 0 && t < db.k0) {
                    asm volatile("");
                    db.next_panel();
                }
            }
        }
    }
    // M0 addresses recomputed from the wave's base in every phase (one scalar add each): hoisted
    // out of the loop, the 16 stage addresses took scalar registers that then spilled.
    uint32_t mw = m0w;
    asm volatile("" : "+s"(mw));
    if constexpr (CQ >= 0) {
        static_assert(SL == CQ, "quarter q of C goes to stage q");
        const uint32_t wq = mw - __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * C::A_LOADS * 1024 +
                            CQ * C::STAGE_BYTES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * TileCDma::PER_WAVE * 1024;
        static_for<0, TileCDma::PER_WAVE>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            dc.issue(j, CQ, wq + j * 1024);
        });
    } else {
        static_for<0, C::A_LOADS>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            da.issue(q, mw + SL * C::STAGE_BYTES + q * 1024);
        });
        static_for<0, C::B_LOADS>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            db.issue(q, mw + SL * C::STAGE_BYTES + C::A_BYTES + q * 1024);
        });
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * C::LOADS) : "memory");
    phase_barrier();
}

// The K tiles [lo, hi) of gemm_tile in one operand layout (AK / BK); lo and hi are multiples of 4,
// so tile lo is in stage 0 and each loop iteration is the four stages' memory and MFMA phases
// with no exit in between. `last`: this is the tile's last segment; the memory phases of its last
// three tiles load C quarters 0-2.
template <class C, bool AK, bool BK, int ROLE>
__device__ __forceinline__ void gemm_segment(int lo, int hi, bool last, const TileWork& tw, OperandDma<C::BM>& da,
                                             OperandDma<C::BN>& db, TileCDma& dc,
                                             floatx16 (&acc)[RoleMap<ROLE>::N], uint32_t lds0, uint32_t m0w) {
    if (lo >= hi) return;
    using R = RoleMap<ROLE>;
    const int lane = threadIdx.x & 63;
    FragBase<R::AF> ba;
    FragBase<R::BF> bb;
    if (AK) ba.init_kmajor(lds0, tw.abase, lane);
    else ba.init_mnmajor(lds0, tw.abase, lane);
    if (BK) bb.init_kmajor(lds0, tw.bbase, lane);
    else bb.init_mnmajor(lds0, tw.bbase, lane);
    Frags<ROLE> f;
    const int body_end = last ? hi - 4 : hi;
    for (int kt = lo; kt < body_end; kt += 4) {
        mem_phase<C, AK, BK, ROLE, 0>(kt, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
        mem_phase<C, AK, BK, ROLE, 1>(kt + 1, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
        mem_phase<C, AK, BK, ROLE, 2>(kt + 2, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
        mem_phase<C, AK, BK, ROLE, 3>(kt + 3, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
    }
    if (last) {
        const int kt = hi - 4;
        mem_phase<C, AK, BK, ROLE, 0>(kt, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
        mem_phase<C, AK, BK, ROLE, 1, 0>(kt + 1, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
        mem_phase<C, AK, BK, ROLE, 2, 1>(kt + 2, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
        mem_phase<C, AK, BK, ROLE, 3, 2>(kt + 3, f, ba, bb, da, db, dc, m0w, lds0);
        mfma_phase<ROLE>(f, acc);
        phase_barrier();
    }
}

// acc = A[rows of the wave's blocks, 0:K] * B[0:K, columns of its blocks] over KT K tiles of 32,
// A read MN-major for tiles t < a_k0 and K-major from there on, B likewise with b_k0 (a_k0 <=
// b_k0; each a multiple of 4 or >= KT): at most three segments, MN/MN, K/MN and K/K, in that
// order, through one 4-stage pipeline of direct loads. K runs to KT rounded up to a multiple of
// 4; the tiles past KT load zeros.
//
// Phases: every wave runs memory phase kt, barrier, MFMA phase kt, barrier for kt = 0, 1, ...;
// group 1 starts one phase late (an extra barrier before its first phase) and group 0 ends with
// an extra barrier, so in every phase one group multiplies and the other loads. Tile kt+3's loads
// are issued in memory phase kt (by each group, its share); a stage is refilled only after both
// groups have read it (phase 2 kt + 1 is the last to read tile kt, whose stage tile kt+4 receives
// in phase 2 kt + 2 at the earliest); each wave waits for its loads of tile kt+1 at the end of
// memory phase kt, before the barrier after which group 0 reads tile kt+1.
//
// `tw`: the wave's role and bases (a diagonal tile of a symmetric result computes only its upper
// blocks, TileWork). `ct`: the epilogue's C tile, loaded into the staging (TileC). Ends with
// every load and LDS read complete and a block barrier: the staging holds C and the rest of the
// stages is free.
template <class C, int ROLE>
__device__ __forceinline__ void gemm_tile(const Operand& A, const Operand& B, int m0, int n0, int KT, int a_k0,
                                          int b_k0, const TileC& ct, const TileWork& tw,
                                          floatx16 (&acc)[RoleMap<ROLE>::N], char* smem) {
    static_assert(C::S == 4 && C::BM == 256 && C::BN == 256, "the unrolled loop and the LDS bases assume these");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int q = 0; q < RoleMap<ROLE>::N; ++q) acc[q] = floatx16{};
    const int KT4 = (KT + 3) & ~3;
    OperandDma<C::BM> da;
    OperandDma<C::BN> db;
    da.init(A, m0, wave, lane, a_k0, KT);
    db.init(B, n0, wave, lane, b_k0, KT);
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
    const uint32_t m0w = lds0 + wave * C::A_LOADS * 1024;
    TileCDma dc;
    dc.init(ct, m0 - ct.r0, n0 - ct.c0, wave, lane);
    static_for<0, TileCDma::PER_WAVE>([&](auto jc) {   // C rows 192-255 into the 32 KB past the stages
        constexpr int j = decltype(jc)::value;
        dc.issue(j, 3, lds0 + C::LDS_BYTES + wave * TileCDma::PER_WAVE * 1024 + j * 1024);
    });
    static_for<0, C::S - 1>([&](auto tc) {
        constexpr int t = decltype(tc)::value;
        da.begin_tile(t);
        db.begin_tile(t);
        static_for<0, C::A_LOADS>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            da.issue(q, m0w + t * C::STAGE_BYTES + q * 1024);
        });
        static_for<0, C::B_LOADS>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            db.issue(q, m0w + t * C::STAGE_BYTES + C::A_BYTES + q * 1024);
        });
    });
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * C::LOADS) : "memory");   // tile 0 (and C rows 192-255)
    phase_barrier();
    ts_loop_start();
    if (wave >= 4) phase_barrier();   // group 1 starts one phase late
    const int k1 = a_k0 < KT ? a_k0 : KT4;
    const int k2 = b_k0 < k1 ? k1 : (b_k0 < KT ? b_k0 : KT4);
    const int lastseg = KT4 > k2 ? 2 : (k2 > k1 ? 1 : 0);   // segments are never all empty (KT >= 1)
    gemm_segment<C, false, false, ROLE>(0, k1, lastseg == 0, tw, da, db, dc, acc, lds0, m0w);
    gemm_segment<C, true, false, ROLE>(k1, k2, lastseg == 1, tw, da, db, dc, acc, lds0, m0w);
    gemm_segment<C, true, true, ROLE>(k2, KT4, lastseg == 2, tw, da, db, dc, acc, lds0, m0w);
    if (wave < 4) phase_barrier();    // group 0 waits out group 1's last MFMA phase
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Epilogue: every output of these GEMMs is f16, so the tile's final values are computed in
// registers from the accumulators and staged once, as f16, in LDS. The staging holds the 256 x 256
// tile in 512-byte rows: row r at byte rowbase(r) = r * 512 for r < 192 (pipeline stages 0-2)
// and 131072 + (r - 192) * 512 for r >= 192 (the 32 KB past the stages; stage 3 stays free), with
// 16-byte chunk c of row r at position c ^ (r & 31). The swizzle lets a direct load write two
// whole rows (TileC), spreads the 32 consecutive rows that the lanes of one accumulator block write
// (stage_f16) over the banks, and leaves each row's chunks a permutation for the row pass (32 lanes
// per row). All eight waves stage at once; diagonal tiles of symmetric results also stage the
// transposes of their upper values, which keeps them exactly symmetric.
template <class C>
struct EpiH {
    static constexpr int PITCH = 512;
    static constexpr int SPARE = C::LDS_BYTES;                     // rows 192..255 live here
    static constexpr int SMEM = C::LDS_BYTES + 64 * PITCH;         // 160 KB
    static constexpr int FREE = 3 * C::STAGE_BYTES;                // stage 3: unused by the staging
    static constexpr int ROWS = C::NT / 32;                        // rows per pass of the block
    static constexpr int ROW_ITERS = C::BM / ROWS;                 // row chunks per thread
    static_assert(FREE + 256 + 4 * C::NT <= SPARE, "scratch slots in the free stage");
    static_assert(C::BN / 8 == 32 && C::BM == 256 && C::STAGE_BYTES == 192 * PITCH / 3, "layout");
    static_assert(ROWS == 16 && 192 % ROWS == 0, "a pass of rows lies on one side of row 192");
    static_assert(SMEM <= 160 * 1024, "LDS");
    // byte offset of row r's start (r wave-uniform or compile-time above 192 or not)
    __device__ static __forceinline__ int rowbase(int r) { return r * PITCH + (r >= 192 ? SPARE - 192 * PITCH : 0); }
    // byte offset of (row r, column c); c % 4 == 0 for 8-byte accesses
    __device__ static __forceinline__ int off(int r, int c) {
        return rowbase(r) + ((((c >> 3) ^ (r & 31)) << 4) | ((c & 7) << 1));
    }
};

// Stages val(r, c, a) for the accumulators this wave owns: val gives the final f16 values of
// tile-local row r, columns c .. c+3 from their 4 accumulators a (computing the rounding to f16
// itself lets an fma with an f16 operand fuse into one instruction). The caller separates this
// from the previous use of smem and from the reads that follow with barriers.
// On a diagonal tile (symmetric results only) the blocks sit where TileWork put them and every
// value above the tile's diagonal is also written at its transposed position, so the staged tile
// is exactly symmetric: a block on the diagonal is written whole first, then the transposes of its
// upper elements replace the lower ones (a wave's LDS writes complete in program order, and each
// block on the diagonal belongs to one wave).
template <class C, int ROLE, class Val>
__device__ __forceinline__ void stage_f16(floatx16 (&acc)[RoleMap<ROLE>::N], char* smem, bool diag,
                                          const TileWork& tw, Val val) {
    using R = RoleMap<ROLE>;
    const int lane = threadIdx.x & 63;
    auto quad = [&](int q, int e) {
        return floatx4{acc[q][4 * e], acc[q][4 * e + 1], acc[q][4 * e + 2], acc[q][4 * e + 3]};
    };
    auto put = [&](int r, int c, const half4& h) { *reinterpret_cast<half4*>(smem + EpiH<C>::off(r, c)) = h; };
    // transposes of the 4 values; upper_only (a block on the tile's diagonal): only those above the
    // diagonal, the others go to a per-lane slot in the free stage (a lane-dependent branch per
    // element made the compiler reload the block's accumulators inside every branch)
    const int dump = EpiH<C>::FREE + 256 + 4 * static_cast<int>(threadIdx.x);
    auto put_t = [&](int r, int c, const half4& h, bool upper_only) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int a = EpiH<C>::off(c + e, r);
            *reinterpret_cast<_Float16*>(smem + (!upper_only || c + e > r ? a : dump)) = h[e];
        }
    };
    const int lr = lane & 31, lc = 4 * (lane >> 5);
    static_for<0, R::N>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        const int r = tw.abase + 32 * R::a_idx(R::bx(q)) + lr;
        const int cb = tw.bbase + 32 * R::b_idx(R::by(q)) + lc;
        half4 h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            h[e] = val(r, cb + 8 * e, quad(q, e));
            // one rounding for both copies: left visible, the compiler recomputed the value for the
            // transposed copy as a single-rounding fma_mix and the direct one as mul + convert,
            // which differ in rare elements and break the exact symmetry
            opaque(h[e]);
            put(r, cb + 8 * e, h[e]);
            if (!R::on_diag(q) && diag) put_t(r, cb + 8 * e, h[e], false);
        }
        if constexpr (R::on_diag(q)) {
            __builtin_amdgcn_sched_barrier(0);   // the whole block first
#pragma unroll
            for (int e = 0; e < 4; ++e) put_t(r, cb + 8 * e, h[e], true);
        }
    });
}

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

// fn(it, r, c8, h) over this thread's row chunks it = 0 .. ROW_ITERS-1 in row order: h = staged
// row r = 16 * it + tid / 32, columns c8 = 8 * (tid % 32) .. c8 + 7. The chunk's swizzled
// position is (tid % 32) ^ (r & 31) = ((tid % 32) ^ (tid / 32)) ^ (16 * (it % 2)), so two per-lane
// bases cover every chunk, the rest of each address being a constant. The bases are opaque to
// the compiler, which then adds the constants rather than keep 16 addresses live.
template <class C, class Fn>
__device__ __forceinline__ void each_row_chunk_h(const char* smem, Fn fn) {
    using E = EpiH<C>;
    const int tr = threadIdx.x >> 5, ck = threadIdx.x & 31, c8 = ck * 8;
    int base[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        base[a] = tr * E::PITCH + (((ck ^ tr) ^ (16 * a)) << 4);
        asm volatile("" : "+v"(base[a]));
    }
#pragma unroll
    for (int it = 0; it < E::ROW_ITERS; ++it) {
        const int r = E::ROWS * it + tr;
        const int rb = E::ROWS * it * E::PITCH + (E::ROWS * it >= 192 ? E::SPARE - 192 * E::PITCH : 0);
        fn(it, r, c8, *reinterpret_cast<const half8v*>(smem + base[it & 1] + rb));
    }
}

// Upper-triangle tile (ti <= tj) number q of a T x T tile grid, row by row.
__device__ __forceinline__ void tri_decode(int q, int T, int& ti, int& tj) {
    int row = 0, rem = q;
    while (rem >= T - row) {
        rem -= T - row;
        ++row;
    }
    ti = row;
    tj = row + rem;
}

}  // namespace thorn
