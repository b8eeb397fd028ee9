// Newton-Schulz GEMMs on gfx950: f16 MFMA (v_mfma_f32_32x32x16_f16), fp32 accumulation, operand
// tiles streamed global -> LDS by buffer DMA through a 4-stage ring, grouped launches over every
// matrix of a parameter group (ns_kernels.hip).
//
// One main loop (gemm_tile) serves every product of both Newton-Schulz schedules: Gram matrices
// X X^T / X^T X, products of s x s workspace matrices, and iterate updates Q X / X Q. Operands are
// read either K-major (ds_read_b128 fragments) or MN-major (two ds_read_tr16_b64 transposing
// reads), so no matrix is ever transposed in memory.
//
// The loop is shaped by how one wave per SIMD spends its cycles (measured on an MI355X with
// timing-only copies): the MFMAs alone take ~1070 cycles per K tile of 32 (1024 ideal), the LDS
// fragment reads add no cycles, and each direct load costs issue and wait time. So every direct
// load is one buffer instruction whose out-of-range lanes (rows or K past the operand) the
// hardware turns into zeros, with one vector add to advance it; the K loop is unrolled over the
// four stages so every LDS address is a per-lane base plus an immediate; and on full tiles the
// direct loads are spaced one per two MFMAs.
#pragma once

#include <type_traits>

#include "thorn_common.hpp"

namespace thorn {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Block tile BM x BN (256 x 256), K step 32, 256 threads as 2 x 2 waves, each wave owning
// (BM/2) x (BN/2) of the tile. S = 4 pipeline stages of LDS.
template <int BM_, int BN_, int S_ = 4>
struct GemmCfg {
    static constexpr int BM = BM_, BN = BN_, BK = 32, S = S_;
    static constexpr int WM = BM / 2, WN = BN / 2;
    static constexpr int TM = WM / 32, TN = WN / 32;
    static constexpr int A_BYTES = BM * BK * 2;          // one stage of A, no padding
    static constexpr int B_BYTES = BN * BK * 2;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int LDS_BYTES = S * STAGE_BYTES;
    static constexpr int A_LOADS = BM / 64;               // 1 KB direct loads per wave per stage
    static constexpr int B_LOADS = BN / 64;
    static constexpr int LOADS_PER_STAGE = A_LOADS + B_LOADS;
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
struct Operand {
    const _Float16* ptr;
    int64_t ld;
    int32_t rows;
};

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

// LDS layouts of one stage, 16-byte chunks, XOR-swizzled so that the fragment reads of a wave
// hit distinct banks:
//   K-major:  MN rows x 4 chunks (64 B); chunk c of row r sits at r*64 + (c ^ ((r >> 2) & 3))*16.
//             16 lanes reading rows r..r+15 at one chunk cover all 64 banks.
//   MN-major: 32 k-rows x MN/8 chunks; chunk c of k-row k at k*MN*2 + (c ^ ((k & 3) << 2))*16.
//             The 32 lanes of a ds_read_tr16_b64 pair read 4 k-rows x 4 chunks: 16 distinct
//             chunks mod 16, all 64 banks.
// A direct load writes 64 consecutive chunk slots (1 KB) at the address in M0, so each lane loads
// the global chunk whose swizzled position is its slot.
//
// OperandDma holds the buffer resource of one operand and, per lane, the byte offset of each of
// its MN/64 chunk loads per stage for the next K tile to load (`cur`, advanced by `step` after
// each load). Loads of consecutive tiles are issued in order; begin_tile switches the offsets to
// the K-major layout at tile k0 (a symmetric matrix stored as its upper block triangle is read
// MN-major, from the transposed mirror block, before its diagonal block) and to out of range at
// tile kend, so the tiles that round K up to whole loop iterations, and the prefetches past the
// end, load zeros.
template <int MN>
struct OperandDma {
    static constexpr int PER_WAVE = MN / 64;
    u32x4 rsrc;
    uint32_t cur[PER_WAVE];
    uint32_t kmaj[PER_WAVE];   // K-major offsets of tile 0
    uint32_t step;             // bytes per K tile in the current layout
    int k0, kend;

    __device__ __forceinline__ static void offsets(const Operand& op, int mn0, int wave, int lane, bool km,
                                                   uint32_t (&o)[PER_WAVE]) {
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const int slot = (wave * PER_WAVE + q) * 64 + lane;
            if (km) {
                const int r = slot >> 2, pc = slot & 3;
                const int c = pc ^ ((r >> 2) & 3);
                const int row = mn0 + r;
                o[q] = row < op.rows ? static_cast<uint32_t>((int64_t(row) * op.ld + c * 8) * 2) : kOutOfRange;
            } else {
                constexpr int CH = MN / 8;
                const int k = slot / CH, pc = slot % CH;
                const int c = pc ^ ((k & 3) << 2);
                const int col = mn0 + c * 8;
                o[q] = col < op.ld ? static_cast<uint32_t>((int64_t(k) * op.ld + col) * 2) : kOutOfRange;
            }
        }
    }

    __device__ __forceinline__ void init(const Operand& op, int mn0, int wave, int lane, int k0_, int kend_) {
        rsrc = sgpr_rsrc(op.ptr, static_cast<uint32_t>(int64_t(op.rows) * op.ld * 2));
        offsets(op, mn0, wave, lane, true, kmaj);
        k0 = k0_;
        kend = kend_;
        if (k0 <= 0) {
#pragma unroll
            for (int q = 0; q < PER_WAVE; ++q) cur[q] = kmaj[q];
            step = 64;
        } else {
            offsets(op, mn0, wave, lane, false, cur);
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

    // Direct load q of this wave for the current tile into LDS at m0 (wave-uniform byte address).
    // It is inline assembly so that the compiler does not track it as an LDS write: its
    // conservative aliasing would otherwise wait for every outstanding load before the next LDS
    // fragment read and serialize the pipeline. The main loop orders the loads explicitly
    // (lds_wait_barrier); the "memory" clobber keeps LDS accesses from moving across them.
    __device__ __forceinline__ void issue(int q, uint32_t m0) {
        asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(cur[q]), "s"(rsrc), "{m0}"(m0) : "memory");
        cur[q] += step;
    }
};

// The C term of a tile's epilogue (out = f16(alpha * A B + beta * C)): the f16 tile of C at rows
// m0.., columns n0.. of a matrix with leading dimension ld and `rows` valid rows (ptr null: no C
// term, every load reads zeros). gemm_tile loads it into the epilogue's staging (EpiH) by direct
// loads: rows 192-255 in the prologue, into the 32 KB past the pipeline stages, and rows 0-63,
// 64-127 and 128-191 in the last three K iterations, into stages 0, 1 and 2 as the loop releases
// them (in place of the loads of tiles past the end, so every iteration still issues one stage
// of loads per wave). Quarter q of the tile is 32 loads of two 512-byte staging rows each; wave w
// issues loads 8w .. 8w+7.
struct TileC {
    const _Float16* ptr;
    int64_t ld;
    int32_t rows;
};

struct TileCDma {
    u32x4 rsrc;
    uint32_t off[8];     // quarter 0 offsets of this lane's 8 loads; quarter q adds q * qstep
    uint32_t qstep;      // bytes of 64 rows
    __device__ __forceinline__ void init(const TileC& c, int m0, int n0, int wave, int lane) {
        rsrc = sgpr_rsrc(c.ptr, c.ptr ? static_cast<uint32_t>(int64_t(c.rows) * c.ld * 2) : 0u);
        qstep = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(128 * c.ld));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int row = 2 * (wave * 8 + j) + (lane >> 5);   // within quarter 0
            const int ch = (lane & 31) ^ (row & 31);             // staging position lane & 31
            const int col = n0 + 8 * ch;
            off[j] = col < c.ld ? static_cast<uint32_t>((int64_t(m0 + row) * c.ld + col) * 2) : kOutOfRange;
        }
    }
    // load j (0..7) of quarter q into LDS at m0 (wave-uniform)
    __device__ __forceinline__ void issue(int j, int q, uint32_t m0) {
        const uint32_t o = off[j] + q * qstep;
        asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(o), "s"(rsrc), "{m0}"(m0) : "memory");
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

// Per-lane LDS fragment bases of one operand of the main loop (operand tiles of MN = 256). The
// four stages are two pairs 65536 bytes apart, so that every other part of an address fits the
// 16-bit immediate offset of the read:
//   K-major: b[pair][ks]; the wave's row offset is in the base, fragment i adds i * 2048 (32 rows
//            of 64 B) and the odd stage of a pair 32768.
//   MN-major: b[pair][i] per fragment (the XOR swizzle of chunk c = 4j + cl by 4x is 4(j ^ x) + cl
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
        constexpr int imm = SB + OPOFF + KS * 8192;
        static_assert(imm + 2048 < 65536, "immediate offset");
        const uint32_t a = fb.b[ST >> 1][I] + imm;
        short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(a));
        short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(a + 2048));
        half4 l4 = __builtin_bit_cast(half4, lo), h4 = __builtin_bit_cast(half4, hi);
        return half8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
    }
}

// This wave's direct loads except the newest N are complete, then the block barrier: after it,
// every wave's loads up to that point are visible in LDS. The "memory" clobber keeps the
// compiler from moving LDS reads above it.
template <int N>
__device__ __forceinline__ void lds_wait_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Block barrier for LDS traffic only: this wave's LDS accesses are complete, then s_barrier.
// Unlike __syncthreads() it does not wait for outstanding global stores, so an epilogue's
// stores keep draining while the next staging pass runs.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Work split of a tile between its four waves. A diagonal tile of a symmetric result is only
// stored as its upper block triangle (the epilogue mirrors it), so of its 8 x 8 grid of 32 x 32
// blocks only the 36 with j >= i are computed: waves 0 and 3 take the blocks of their diagonal
// quadrants with j >= i (10 each), waves 1 and 2 split the upper-right quadrant (rows 0-63 and
// 64-127, 8 blocks each), and nobody computes the lower-left quadrant. The slowest wave then
// issues 10 MFMAs per k16 step instead of 16.
enum TileRole : int { kRoleFull = 0, kRoleTri = 1, kRoleHalf = 2 };

template <int ROLE, int TM, int TN>
struct RoleMap {
    static constexpr int N = ROLE == kRoleFull ? TM * TN : ROLE == kRoleTri ? TM * (TM + 1) / 2 : 2 * TN;
    // (i, j) of this wave's q-th MFMA block, rows before columns
    static constexpr int i(int q) {
        if (ROLE == kRoleFull || ROLE == kRoleHalf) return q / TN;
        int r = 0;
        while (q >= TN - r) {
            q -= TN - r;
            ++r;
        }
        return r;
    }
    static constexpr int j(int q) {
        if (ROLE != kRoleTri) return q % TN;
        int r = 0;
        while (q >= TN - r) {
            q -= TN - r;
            ++r;
        }
        return r + q;
    }
    static constexpr int NA = ROLE == kRoleHalf ? 2 : TM;   // A fragments per k16 step
    static constexpr int NF = NA + TN;                       // fragments per k16 step
};

// f(std::integral_constant<int, Q>) for Q = B .. E-1, as straight-line code with Q a constant.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Fragment Q of a k16 step of stage ST in the order the MFMAs use them: A0, B0 .. B(TN-1),
// A1 .. A(NA-1), in the layouts AK / BK (true = K-major).
template <class C, bool AK, bool BK, int ST, int KS, int Q>
__device__ __forceinline__ void read_frag(const FragBase<C::TM>& fa_base, const FragBase<C::TN>& fb_base,
                                          half8 (&ra)[C::TM], half8 (&rb)[C::TN]) {
    if constexpr (Q == 0) ra[0] = frag_at<AK, ST, KS, 0, 0>(fa_base);
    else if constexpr (Q <= C::TN) rb[Q - 1] = frag_at<BK, ST, KS, C::A_BYTES, Q - 1>(fb_base);
    else ra[Q - C::TN] = frag_at<AK, ST, KS, 0, Q - C::TN>(fa_base);
}

// K tile kt, held in stage ST = kt % 4, as one basic block of two k16 sub-steps of RoleMap::N
// MFMAs, the order of every instruction fixed explicitly. Sub-step 1 multiplies the ks 0
// fragments (fa[0], fb[0]) and reads the ks 1 fragments of stage ST after MFMA q. Then every
// wave waits for its own loads of tile kt+1 and meets the others at the block barrier: after it,
// tile kt+1 is visible and nobody reads stage (kt-1) % 4 any more, which then receives tile kt+3.
// Sub-step 2 multiplies the ks 1 fragments and, after MFMA q, reads fragment q of the next
// tile's ks 0 (stage ST+1) and issues the direct loads of tile kt+3: one per two MFMAs when the
// wave has twice as many MFMAs as loads (full tiles), else one per MFMA. (Loading tile kt+4 into
// stage ST instead, after a wait for this wave's LDS reads, gives the loads one more iteration
// but measured no faster.)
// CQ >= 0 (the last three iterations of a tile's K loop): the direct loads fetch quarter CQ of the
// epilogue's C tile into stage ST+3 instead of a tile past the end of K.
template <class C, bool AK, bool BK, int ROLE, int ST, int CQ = -1>
__device__ __forceinline__ void k_iter(int kt, OperandDma<C::BM>& da, OperandDma<C::BN>& db, TileCDma& dc,
                                       floatx16 (&acc)[C::TM][C::TN], half8 (&fa)[2][C::TM],
                                       half8 (&fb)[2][C::TN], const FragBase<C::TM>& ba, const FragBase<C::TN>& bb,
                                       uint32_t m0base, uint32_t lds0) {
    using R = RoleMap<ROLE, C::TM, C::TN>;
    constexpr int NM = R::N, NF = R::NF;
    constexpr int NA = OperandDma<C::BM>::PER_WAVE, NB = OperandDma<C::BN>::PER_WAVE;
    constexpr bool SPREAD = NM >= 2 * (NA + NB);
    constexpr int SN = (ST + 1) & 3, SL = (ST + 3) & 3;
    static_assert(NF <= NM && NA + NB <= NM, "one fragment and one direct load per MFMA at most");
    static_assert(NA + NB == 8, "a quarter of C is 8 loads per wave, one stage of operand loads");
    static_for<0, NM>([&](auto qc) {
        constexpr int q = decltype(qc)::value, i = R::i(q), j = R::j(q);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[0][j], fa[0][i], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (q < NF) read_frag<C, AK, BK, ST, 1, q>(ba, bb, fa[1], fb[1]);
        __builtin_amdgcn_sched_barrier(0);
    });
    lds_wait_barrier<(C::S - 3) * C::LOADS_PER_STAGE>();
    __builtin_amdgcn_sched_barrier(0);
    da.begin_tile(kt + C::S - 1);
    db.begin_tile(kt + C::S - 1);
    static_for<0, NM>([&](auto qc) {
        constexpr int q = decltype(qc)::value, i = R::i(q), j = R::j(q);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (q < NF) read_frag<C, AK, BK, SN, 0, q>(ba, bb, fa[0], fb[0]);
        constexpr int d = SPREAD ? (q % 2 == 0 ? q / 2 : NA + NB) : q;
        if constexpr (CQ >= 0) {
            static_assert(SL == CQ, "quarter q of C goes to stage q");
            const uint32_t wq = lds0 + CQ * C::STAGE_BYTES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 8192;
            if constexpr (d < NA + NB) dc.issue(d, CQ, wq + d * 1024);
        } else if constexpr (d < NA) {
            da.issue(d, m0base + SL * C::STAGE_BYTES + d * 1024);
        } else if constexpr (d < NA + NB) {
            db.issue(d - NA, m0base + SL * C::STAGE_BYTES + C::A_BYTES + (d - NA) * 1024);
        }
        __builtin_amdgcn_sched_barrier(0);
    });
}

// The K tiles [lo, hi) of gemm_tile in one operand layout (AK / BK); lo and hi are multiples of 4,
// so tile lo is in stage 0 and the loop body is the four stages' iterations with no exit in
// between (an exit per iteration made the compiler copy the accumulators at every one). On entry
// the stages hold tiles lo .. lo+2 (tile lo visible to every wave); the ks 0 fragments of tile lo
// are read first, in this segment's layouts.
// `last`: this is the tile's last segment; its last block of four iterations loads C quarters
// 0-2 in its last three.
template <class C, bool AK, bool BK, int ROLE>
__device__ __forceinline__ void gemm_segment(int lo, int hi, bool last, OperandDma<C::BM>& da, OperandDma<C::BN>& db,
                                             TileCDma& dc, floatx16 (&acc)[C::TM][C::TN], half8 (&fa)[2][C::TM],
                                             half8 (&fb)[2][C::TN], uint32_t lds0, uint32_t m0base) {
    if (lo >= hi) return;
    using R = RoleMap<ROLE, C::TM, C::TN>;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // kRoleHalf: wave 1 takes rows 0-63, wave 2 rows 64-127 of the upper-right quadrant
    const int wm = ROLE == kRoleHalf ? (wave >> 1) * (C::WM / 2) : (wave >> 1) * C::WM;
    const int wn = ROLE == kRoleHalf ? C::WN : (wave & 1) * C::WN;
    FragBase<C::TM> ba;
    FragBase<C::TN> bb;
    if (AK) ba.init_kmajor(lds0, wm, lane);
    else ba.init_mnmajor(lds0, wm, lane);
    if (BK) bb.init_kmajor(lds0, wn, lane);
    else bb.init_mnmajor(lds0, wn, lane);
    static_for<0, R::NF>([&](auto qc) { read_frag<C, AK, BK, 0, 0, decltype(qc)::value>(ba, bb, fa[0], fb[0]); });
    const int body_end = last ? hi - 4 : hi;
    for (int kt = lo; kt < body_end; kt += 4) {
        k_iter<C, AK, BK, ROLE, 0>(kt, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
        k_iter<C, AK, BK, ROLE, 1>(kt + 1, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
        k_iter<C, AK, BK, ROLE, 2>(kt + 2, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
        k_iter<C, AK, BK, ROLE, 3>(kt + 3, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
    }
    if (last) {
        const int kt = hi - 4;
        k_iter<C, AK, BK, ROLE, 0>(kt, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
        k_iter<C, AK, BK, ROLE, 1, 0>(kt + 1, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
        k_iter<C, AK, BK, ROLE, 2, 1>(kt + 2, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
        k_iter<C, AK, BK, ROLE, 3, 2>(kt + 3, da, db, dc, acc, fa, fb, ba, bb, m0base, lds0);
    }
}

// acc = A[m0 + wm + 32i .., 0:K] * B[0:K, n0 + wn + 32j ..] over KT K tiles of 32, A read
// MN-major for tiles t < a_k0 and K-major from there on, B likewise with b_k0 (a_k0 <= b_k0; each
// a multiple of 4 or >= KT): at most three segments, MN/MN, K/MN and K/K, in that order, through
// one 4-stage pipeline of direct loads. K runs to KT rounded up to a multiple of 4; the tiles
// past KT load zeros. The MFMA is issued as B^T A^T, so each 32 x 32 accumulator comes out
// transposed: lane l holds row (l & 31) and the four consecutive columns 8*(r/4) + 4*(l/32) + 0..3
// in registers r..r+3, which the epilogue writes to LDS as one 8-byte store. `diag`: the tile is a
// diagonal tile of a symmetric result (m0 == n0), split by TileRole; every role passes the same
// barriers (one per K tile, and the final one). `ct`: the epilogue's C tile, loaded into the
// staging (TileC). Ends with every load and LDS read complete and a block barrier: the staging
// holds C and the rest of the stages is free.
template <class C>
__device__ __forceinline__ void gemm_tile(const Operand& A, const Operand& B, int m0, int n0, int KT, int a_k0,
                                          int b_k0, const TileC& ct, floatx16 (&acc)[C::TM][C::TN], char* smem,
                                          bool diag = false) {
    static_assert(C::S == 4 && C::BM == 256 && C::BN == 256, "the unrolled loop and the LDS bases assume these");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = floatx16{};
    const int KT4 = (KT + 3) & ~3;
    OperandDma<C::BM> da;
    OperandDma<C::BN> db;
    da.init(A, m0, wave, lane, a_k0, KT);
    db.init(B, n0, wave, lane, b_k0, KT);
    constexpr int NA = OperandDma<C::BM>::PER_WAVE, NB = OperandDma<C::BN>::PER_WAVE;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
    const uint32_t m0base = lds0 + wave * NA * 1024;
    TileCDma dc;
    dc.init(ct, m0, n0, wave, lane);
    static_for<0, 8>([&](auto jc) {   // C rows 192-255 into the 32 KB past the stages
        constexpr int j = decltype(jc)::value;
        dc.issue(j, 3, lds0 + C::LDS_BYTES + wave * 8192 + j * 1024);
    });
    static_for<0, C::S - 1>([&](auto tc) {
        constexpr int t = decltype(tc)::value;
        da.begin_tile(t);
        db.begin_tile(t);
        static_for<0, NA>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            da.issue(q, m0base + t * C::STAGE_BYTES + q * 1024);
        });
        static_for<0, NB>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            db.issue(q, m0base + t * C::STAGE_BYTES + C::A_BYTES + q * 1024);
        });
    });
    lds_wait_barrier<(C::S - 2) * C::LOADS_PER_STAGE>();   // tile 0 visible
    const int k1 = a_k0 < KT ? a_k0 : KT4;
    const int k2 = b_k0 < k1 ? k1 : (b_k0 < KT ? b_k0 : KT4);
    const int lastseg = KT4 > k2 ? 2 : (k2 > k1 ? 1 : 0);   // segments are never all empty (KT >= 1)
    auto segments = [&](auto role) {
        constexpr int ROLE = decltype(role)::value;
        half8 fa[2][C::TM], fb[2][C::TN];
        gemm_segment<C, false, false, ROLE>(0, k1, lastseg == 0, da, db, dc, acc, fa, fb, lds0, m0base);
        gemm_segment<C, true, false, ROLE>(k1, k2, lastseg == 1, da, db, dc, acc, fa, fb, lds0, m0base);
        gemm_segment<C, true, true, ROLE>(k2, KT4, lastseg == 2, da, db, dc, acc, fa, fb, lds0, m0base);
    };
    if (!diag) segments(std::integral_constant<int, kRoleFull>{});
    else if (wave == 0 || wave == 3) segments(std::integral_constant<int, kRoleTri>{});
    else segments(std::integral_constant<int, kRoleHalf>{});
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Epilogue: every output of these GEMMs is f16, so the tile's final values are computed in
// registers from the accumulators and staged once, as f16, in LDS. The staging holds the 256 x 256
// tile in 512-byte rows: row r at byte rowbase(r) = r * 512 for r < 192 (pipeline stages 0-2)
// and 131072 + (r - 192) * 512 for r >= 192 (the 32 KB past the stages; stage 3 stays free), with
// 16-byte chunk c of row r at position c ^ (r & 31). The swizzle lets a direct load write two
// whole rows (TileC), spreads the 32 consecutive rows that the lanes of one accumulator block write
// (stage_f16) over the banks, and leaves each row's chunks a permutation for the row pass (32 lanes
// per row). All four waves stage at once; diagonal tiles of symmetric results also stage the
// transposes of their upper values, which keeps them exactly symmetric.
template <class C>
struct EpiH {
    static constexpr int PITCH = 512;
    static constexpr int SPARE = C::LDS_BYTES;                     // rows 192..255 live here
    static constexpr int SMEM = C::LDS_BYTES + 64 * PITCH;         // 160 KB
    static constexpr int FREE = 3 * C::STAGE_BYTES;                // stage 3: unused by the staging
    static_assert(FREE + 256 + 4 * 256 <= SPARE, "scratch slots in the free stage");
    static constexpr int ROW_ITERS = C::BM * (C::BN / 8) / 256;   // row chunks per thread
    static_assert(C::BN / 8 == 32 && C::BM == 256 && C::STAGE_BYTES == 192 * PITCH / 3, "layout");
    static_assert(SMEM <= 160 * 1024, "LDS");
    // byte offset of row r's start (r wave-uniform or compile-time above 192 or not)
    __device__ static __forceinline__ int rowbase(int r) { return r * PITCH + (r >= 192 ? SPARE - 192 * PITCH : 0); }
    // byte offset of (row r, column c); c % 4 == 0 for 8-byte accesses
    __device__ static __forceinline__ int off(int r, int c) {
        return rowbase(r) + ((((c >> 3) ^ (r & 31)) << 4) | ((c & 7) << 1));
    }
};

// Stages val(r, c, a, dblk) for the accumulators this wave owns: val gives the final f16 values
// of tile-local row r, columns c .. c+3 from their 4 accumulators a (computing the rounding to f16
// itself lets an fma with an f16 operand fuse into one instruction); dblk (wave-uniform) says that
// the 32 x 32 block holds elements of the tile's diagonal, r == c + e for some e, which only the
// diagonal blocks of waves 0 and 3 on a diagonal tile do. The caller separates this from the
// previous use of smem and from the reads that follow with barriers.
// On a diagonal tile (gemm_tile's `diag`, symmetric results only) the blocks sit where TileRole
// put them (waves 1 and 2: rows 0-63 and 64-127 of the upper-right quadrant; waves 0 and 3: the
// blocks on and above the diagonal of their quadrants) and every value above the tile's diagonal
// is also written at its transposed position, so the staged tile is exactly symmetric: the
// diagonal blocks of waves 0 and 3 are written whole first, then the transposes of their upper
// elements replace the lower ones (a wave's LDS writes complete in program order).
template <class C, class Val>
__device__ __forceinline__ void stage_f16(floatx16 (&acc)[C::TM][C::TN], char* smem, bool diag, Val val) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    auto quad = [&](int i, int j, int q) {
        return floatx4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
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
    auto final4 = [&](int r, int c, const floatx4& a, bool dblk) { return val(r, c, a, dblk); };
    const int lr = lane & 31, lc = 4 * (lane >> 5);
    if (diag && (wave == 1 || wave == 2)) {
        const int r0 = (wave >> 1) * (C::WM / 2);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < C::TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = r0 + 32 * i + lr, c = C::WN + 32 * j + 8 * q + lc;
                    const half4 h = final4(r, c, quad(i, j, q), false);
                    put(r, c, h);
                    put_t(r, c, h, false);
                }
    } else if (diag) {
        const int wm = (wave >> 1) * C::WM;
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
            for (int j = i; j < C::TN; ++j) {
                half4 h[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = wm + 32 * i + lr, c = wm + 32 * j + 8 * q + lc;
                    h[q] = final4(r, c, quad(i, j, q), i == j);
                    put(r, c, h[q]);
                    if (j > i) put_t(r, c, h[q], false);
                }
                if (j == i) {
                    __builtin_amdgcn_sched_barrier(0);   // the whole block first
#pragma unroll
                    for (int q = 0; q < 4; ++q) put_t(wm + 32 * i + lr, wm + 32 * j + 8 * q + lc, h[q], true);
                }
            }
    } else {
        const int wm = (wave >> 1) * C::WM, wn = (wave & 1) * C::WN;
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
            for (int j = 0; j < C::TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = wm + 32 * i + lr, c = wn + 32 * j + 8 * q + lc;
                    put(r, c, final4(r, c, quad(i, j, q), false));
                }
    }
}

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

// fn(it, r, c8, h) over this thread's row chunks it = 0 .. ROW_ITERS-1 in row order: h = staged
// row r = 8 * it + tid / 32, columns c8 = 8 * (tid % 32) .. c8 + 7. The chunk's swizzled
// position is (tid % 32) ^ (r & 31) = ((tid % 32) ^ (tid / 32)) ^ (8 * (it % 4)), so four per-lane
// bases cover every chunk, the rest of each address being a constant. The bases are opaque to
// the compiler, which then adds the constants rather than keep 32 addresses live.
template <class C, class Fn>
__device__ __forceinline__ void each_row_chunk_h(const char* smem, Fn fn) {
    using E = EpiH<C>;
    const int tr = threadIdx.x >> 5, ck = threadIdx.x & 31, c8 = ck * 8;
    int base[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        base[a] = tr * E::PITCH + (((ck ^ tr) ^ (8 * a)) << 4);
        asm volatile("" : "+v"(base[a]));
    }
#pragma unroll
    for (int it = 0; it < E::ROW_ITERS; ++it) {
        const int r = 8 * it + tr;
        const int rb = 8 * it * E::PITCH + (8 * it >= 192 ? E::SPARE - 192 * E::PITCH : 0);
        fn(it, r, c8, *reinterpret_cast<const half8v*>(smem + base[it & 3] + rb));
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
