// Newton-Schulz GEMMs on gfx950: f16 MFMA (v_mfma_f32_32x32x16_f16), fp32 accumulation, LDS
// double-buffered tiles and grouped launches over every matrix of a parameter group.
//
// One Newton-Schulz iteration X <- (a I + b A + c A^2) X with A the Gram matrix on the short side
// (reference: thorn.py:654-658, the plain quintic; a is folded into the polynomial's diagonal) is
// three grouped launches:
//   gram:   A = X X^T (wide) or X^T X (tall), s x s, upper-triangle tiles only, mirrored stores;
//   poly:   P = a I + b A + c A A, same symmetric tiling;
//   update: X' = P X (wide) or X P (tall), written back in the parameter's own row-major layout.
// Operands are read either K-major (ds_read_b128 fragments) or MN-major (two ds_read_tr16_b64
// transposing reads), so no matrix is ever transposed in memory.
#pragma once

#include <type_traits>

#include "thorn_common.hpp"

namespace thorn {

// Block tile BM x BN (128 or 256 each), K step 32, 256 threads as 2 x 2 waves, each wave owning
// (BM/2) x (BN/2) of the tile. S pipeline stages of LDS, filled by direct global->LDS loads.
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
// ld is a multiple of 8 and the padding columns [logical width, ld) hold zeros, so a 16-byte
// chunk is either entirely inside a row or entirely outside it; chunks outside are read from
// `zero`, a 16-byte block of zeros.
struct Operand {
    const _Float16* ptr;
    int64_t ld;
    int32_t rows;
};

// LDS layouts of one stage, 16-byte chunks, XOR-swizzled so that the fragment reads of a wave
// hit distinct banks:
//   K-major:  MN rows x 4 chunks (64 B); chunk c of row r sits at r*64 + (c ^ ((r >> 2) & 3))*16.
//             16 lanes reading rows r..r+15 at one chunk cover all 64 banks.
//   MN-major: 32 k-rows x MN/8 chunks; chunk c of k-row k at k*MN*2 + (c ^ ((k & 3) << 2))*16.
//             The 32 lanes of a ds_read_tr16_b64 pair read 4 k-rows x 4 chunks: 16 distinct
//             chunks mod 16, all 64 banks.
// The direct loads write 64 consecutive chunk slots per instruction, so each lane loads the
// global chunk whose swizzled position is its slot.
//
// DmaSrc holds, per lane, the global source of each of its MN/64 chunk loads for K tile 0 and
// the bound that decides, per tile t, whether the chunk exists (t * 32 < lim) or comes from
// `zero`; tile t's source is src + t * step bytes.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

template <int MN, bool KM>
struct DmaSrc {
    static constexpr int PER_WAVE = MN / 64;
    const char* src[PER_WAVE];
    int lim[PER_WAVE];
    int64_t step;

    __device__ __forceinline__ void init(const Operand& op, int mn0, int wave, int lane) {
        const char* base = reinterpret_cast<const char*>(op.ptr);
        step = KM ? int64_t(BKC * 2) : int64_t(BKC) * op.ld * 2;
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const int slot = (wave * PER_WAVE + q) * 64 + lane;
            if (KM) {
                const int r = slot >> 2, pc = slot & 3;
                const int c = pc ^ ((r >> 2) & 3);
                const int64_t row = mn0 + r;
                src[q] = base + (row * op.ld + c * 8) * 2;
                lim[q] = row < op.rows ? static_cast<int>(op.ld) - c * 8 : 0;
            } else {
                constexpr int CH = MN / 8;
                const int k = slot / CH, pc = slot % CH;
                const int c = pc ^ ((k & 3) << 2);
                const int64_t col = mn0 + c * 8;
                src[q] = base + (int64_t(k) * op.ld + col) * 2;
                lim[q] = col < op.ld ? op.rows - k : 0;
            }
        }
    }

    static constexpr int BKC = 32;   // K elements per tile
};

typedef __attribute__((address_space(3))) short4v lds_s4;

// MFMA fragment (8 halves) for the 32-wide sub-tile at `t0` and k16 step `ks` of a stage.
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

// The A and B operand sources of one tile: each is read MN-major for K tiles t < k0 and K-major
// from there on (k0 = 0: always K-major; k0 >= the tile count: always MN-major). A symmetric
// matrix stored as its upper block triangle is read MN-major, from the transposed mirror block,
// before its diagonal block and K-major from there on.
//
// The loads of consecutive K tiles are issued in order (t = 0, 1, 2, ...), so each lane keeps the
// source of its chunks of the next tile (`cur`) and advances it by the layout's tile stride after
// every load: a load costs a compare, a select and a 64-bit add of vector work, which the MFMA
// it follows in the loop body covers. begin_tile switches the sources to the K-major layout when
// the next tile is tile k0.
template <int MN>
struct DmaPair {
    static constexpr int PER_WAVE = MN / 64;
    DmaSrc<MN, true> kmaj;           // K-major sources of tile 0, for the switch at k0
    const char* cur[PER_WAVE];       // this lane's chunk q of the next tile to issue
    int lim[PER_WAVE];               // chunk q exists in tile t iff t * 32 < lim[q]
    int64_t step;                    // bytes between consecutive K tiles in the current layout
    int k0;

    __device__ __forceinline__ void init(const Operand& op, int mn0, int wave, int lane, int k0_) {
        kmaj.init(op, mn0, wave, lane);
        k0 = k0_;
        if (k0 <= 0) {
#pragma unroll
            for (int q = 0; q < PER_WAVE; ++q) {
                cur[q] = kmaj.src[q];
                lim[q] = kmaj.lim[q];
            }
            step = kmaj.step;
        } else {
            DmaSrc<MN, false> mnmaj;
            mnmaj.init(op, mn0, wave, lane);
#pragma unroll
            for (int q = 0; q < PER_WAVE; ++q) {
                cur[q] = mnmaj.src[q];
                lim[q] = mnmaj.lim[q];
            }
            step = mnmaj.step;
        }
    }

    // Called before the first load of tile t, for t = 0, 1, 2, ... in order (t is wave-uniform,
    // so this is a scalar branch taken at most once per tile).
    __device__ __forceinline__ void begin_tile(int t) {
        if (t == k0 && t > 0) {
#pragma unroll
            for (int q = 0; q < PER_WAVE; ++q) {
                cur[q] = kmaj.src[q] + t * kmaj.step;
                lim[q] = kmaj.lim[q];
            }
            step = kmaj.step;
        }
    }

    // Direct load q of this wave for K tile t (the tile of the last begin_tile) into the stage at
    // `lds` (a wave-uniform LDS byte address of this operand's part of the stage). Every address
    // is inside the operand (chunks past its end come from `zero`) for any t >= 0.
    // The load is inline assembly so that the compiler does not track it as an LDS write: its
    // conservative aliasing would otherwise wait for every outstanding load before the next LDS
    // fragment read and serialize the pipeline. The main loop orders the loads explicitly
    // (lds_wait_barrier); the "memory" clobber keeps LDS accesses from moving across them.
    __device__ __forceinline__ void issue_one(int t, int q, uint32_t lds, const void* zero) {
        const void* p = t * DmaSrc<MN, true>::BKC < lim[q] ? static_cast<const void*>(cur[q]) : zero;
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"((const THORN_GLOBAL void*)p), "{m0}"(lds + q * 1024)
                     : "memory");
        cur[q] += step;
    }
};

// Reads fragment q of this wave's k16 step `ks` from the stage at `st` (A at st, B at
// st + A_BYTES) in the layouts AK / BK (true = K-major), numbered in the order the MFMAs of a
// sub-step use them: A0, B0 .. B(TN-1), A1 .. A(TM-1).
template <class C, bool AK, bool BK>
__device__ __forceinline__ void read_frag(const char* st, int ks, int q, int wm, int wn, int lane, half8 (&ra)[C::TM],
                                          half8 (&rb)[C::TN]) {
    if (q == 0) ra[0] = frag<C::BM, AK>(st, wm, ks, lane);
    else if (q <= C::TN) rb[q - 1] = frag<C::BN, BK>(st + C::A_BYTES, wn + 32 * (q - 1), ks, lane);
    else ra[q - C::TN] = frag<C::BM, AK>(st, wm + 32 * (q - C::TN), ks, lane);
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
        if (ROLE == kRoleFull) return q / TN;
        if (ROLE == kRoleHalf) return q / TN;
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
    // fragments read per k16 step: A0, B0 .. B(TN-1), A1 .. A(rows-1)
    static constexpr int NF = (ROLE == kRoleHalf ? 2 : TM) + TN;
};

// f(std::integral_constant<int, Q>) for Q = B .. E-1, as straight-line code with Q a constant.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// The K tiles [lo, hi) of gemm_tile in one operand layout (AK / BK). On entry the stages hold
// tiles lo .. lo+S-2 (tile lo visible to every wave); on exit they hold hi .. hi+S-2 likewise.
// Each iteration is one basic block of two k16 sub-steps of TM * TN MFMAs, the order of every
// instruction fixed explicitly: after MFMA q of the first sub-step, fragment q of the second;
// after MFMA q of the second, fragment q of the next tile's first sub-step and then direct load
// q of tile kt+S-1 (fragments in the order the MFMAs use them, so each is read as early as
// possible before its use). Between the two sub-steps every wave waits for its own loads of tile
// kt+1 and meets the others at the block barrier: after it, tile kt+1 is visible and nobody
// reads stage (kt-1) % S any more, which then receives tile kt+S-1. Tiles past the end of K are
// loaded (zeros or in-bounds data) and read but never used, which keeps the loop body free of
// branches.
template <class C, bool AK, bool BK, int ROLE = kRoleFull>
__device__ __forceinline__ void gemm_segment(int lo, int hi, DmaPair<C::BM>& da, DmaPair<C::BN>& db,
                                             floatx16 (&acc)[C::TM][C::TN], half8 (&fa)[2][C::TM],
                                             half8 (&fb)[2][C::TN], char* smem, const void* zero) {
    if (lo >= hi) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // kRoleHalf: wave 1 takes rows 0-63, wave 2 rows 64-127 of the upper-right quadrant
    const int wm = ROLE == kRoleHalf ? (wave >> 1) * (C::WM / 2) : (wave >> 1) * C::WM;
    const int wn = ROLE == kRoleHalf ? C::WN : (wave & 1) * C::WN;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
    using R = RoleMap<ROLE, C::TM, C::TN>;
    constexpr int NM = R::N;    // MFMAs per sub-step
    constexpr int NF = R::NF;   // fragments per sub-step
    constexpr int NA = DmaPair<C::BM>::PER_WAVE, NB = DmaPair<C::BN>::PER_WAVE;
    static_assert(NF <= NM && NA + NB <= NM, "one fragment and one direct load per MFMA at most");
    {
        const char* s0 = smem + (lo % C::S) * C::STAGE_BYTES;
#pragma unroll
        for (int q = 0; q < NF; ++q) read_frag<C, AK, BK>(s0, 0, q, wm, wn, lane, fa[0], fb[0]);
    }
    for (int kt = lo; kt < hi; ++kt) {
        const char* sa = smem + (kt % C::S) * C::STAGE_BYTES;
        da.begin_tile(kt + C::S - 1);
        db.begin_tile(kt + C::S - 1);
        static_for<0, NM>([&](auto qc) {
            constexpr int q = decltype(qc)::value, i = R::i(q), j = R::j(q);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[0][j], fa[0][i], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (q < NF) read_frag<C, AK, BK>(sa, 1, q, wm, wn, lane, fa[1], fb[1]);
            __builtin_amdgcn_sched_barrier(0);
        });
        lds_wait_barrier<(C::S - 3) * C::LOADS_PER_STAGE>();
        __builtin_amdgcn_sched_barrier(0);
        const int tn = kt + C::S - 1;
        const uint32_t st_new = lds0 + (tn % C::S) * C::STAGE_BYTES;
        const char* na = smem + ((kt + 1) % C::S) * C::STAGE_BYTES;
        static_for<0, NM>([&](auto qc) {
            constexpr int q = decltype(qc)::value, i = R::i(q), j = R::j(q);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (q < NF) read_frag<C, AK, BK>(na, 0, q, wm, wn, lane, fa[0], fb[0]);
            if constexpr (q < NA) da.issue_one(tn, q, st_new + wave * NA * 1024, zero);
            else if constexpr (q < NA + NB) db.issue_one(tn, q - NA, st_new + C::A_BYTES + wave * NB * 1024, zero);
            __builtin_amdgcn_sched_barrier(0);
        });
    }
}

// acc = A[m0 + wm + 32i .., 0:K] * B[0:K, n0 + wn + 32j ..] over KT K tiles of 32, A read
// MN-major for tiles t < a_k0 and K-major from there on, B likewise with b_k0 (a_k0 <= b_k0):
// at most three segments, MN/MN, K/MN and K/K, in that order, through one S-stage pipeline of
// direct global->LDS loads. The MFMA is issued as B^T A^T, so each 32 x 32 accumulator comes out
// transposed: lane l holds row (l & 31) and the four consecutive columns 8*(r/4) + 4*(l/32) + 0..3
// in registers r..r+3, which the epilogue writes to LDS as one 16-byte store. Ends with every
// load and LDS read complete and a block barrier, so the stages are free for the epilogue.
template <class C, int ROLE>
__device__ __forceinline__ void gemm_segments(int KT, int k1, int k2, DmaPair<C::BM>& da,
                                              DmaPair<C::BN>& db, floatx16 (&acc)[C::TM][C::TN], char* smem,
                                              const void* zero) {
    half8 fa[2][C::TM], fb[2][C::TN];
    gemm_segment<C, false, false, ROLE>(0, k1, da, db, acc, fa, fb, smem, zero);
    gemm_segment<C, true, false, ROLE>(k1, k2, da, db, acc, fa, fb, smem, zero);
    gemm_segment<C, true, true, ROLE>(k2, KT, da, db, acc, fa, fb, smem, zero);
}

// `diag`: the tile is a diagonal tile of a symmetric result (m0 == n0), split by TileRole.
template <class C>
__device__ __forceinline__ void gemm_tile(const Operand& A, const Operand& B, int m0, int n0, int KT, int a_k0,
                                          int b_k0, floatx16 (&acc)[C::TM][C::TN], char* smem, const void* zero,
                                          bool diag = false) {
    static_assert(C::S >= 3 && C::S <= 5, "pipeline depth");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = floatx16{};
    DmaPair<C::BM> da;
    DmaPair<C::BN> db;
    da.init(A, m0, wave, lane, a_k0);
    db.init(B, n0, wave, lane, b_k0);
    constexpr int NA = DmaPair<C::BM>::PER_WAVE, NB = DmaPair<C::BN>::PER_WAVE;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
#pragma unroll
    for (int t = 0; t < C::S - 1; ++t) {
        const uint32_t st = lds0 + t * C::STAGE_BYTES;
        da.begin_tile(t);
        db.begin_tile(t);
#pragma unroll
        for (int q = 0; q < NA; ++q) da.issue_one(t, q, st + wave * NA * 1024, zero);
#pragma unroll
        for (int q = 0; q < NB; ++q) db.issue_one(t, q, st + C::A_BYTES + wave * NB * 1024, zero);
    }
    lds_wait_barrier<(C::S - 2) * C::LOADS_PER_STAGE>();   // tile 0 visible
    const int k1 = a_k0 < KT ? a_k0 : KT;
    const int k2 = b_k0 < k1 ? k1 : (b_k0 < KT ? b_k0 : KT);
    // every role passes the same barriers: one per K tile, and the final one below
    if (!diag) gemm_segments<C, kRoleFull>(KT, k1, k2, da, db, acc, smem, zero);
    else if (wave == 0 || wave == 3) gemm_segments<C, kRoleTri>(KT, k1, k2, da, db, acc, smem, zero);
    else gemm_segments<C, kRoleHalf>(KT, k1, k2, da, db, acc, smem, zero);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Epilogue: every output of these GEMMs is f16, so the tile's final values are computed in
// registers from the accumulators and staged once, as f16, in LDS (reusing the pipeline stages).
// Row r of the staging starts at half rowoff(r) = r * SH + (r / 8) * PAD: rows are BN + 8 halves
// (16-byte aligned) and every 8 rows add 8 more, so that the 64 lanes writing an accumulator
// block (stage_f16: 32 consecutive rows, 8 bytes each) spread over the banks. All four waves
// stage at once and one pass of 16-byte row chunks (32 lanes per row) reads the tile back: half
// the LDS traffic of fp32 staging. Diagonal tiles of symmetric results also stage the transposes
// of their upper values, which keeps them exactly symmetric.
template <class C>
struct EpiH {
    static constexpr int SH = C::BN + 8;
    static constexpr int PAD = 8;
    static constexpr int BYTES = (C::BM * SH + (C::BM / 8) * PAD) * 2;
    static constexpr int SMEM = BYTES > C::LDS_BYTES ? BYTES : C::LDS_BYTES;
    static constexpr int ROW_ITERS = C::BM * (C::BN / 8) / 256;   // row chunks per thread
    static constexpr int ROW_STEP = 8 * SH + PAD;                  // halves between chunks it, it+1
    static_assert(C::BN / 8 == 32 && C::BM == 256, "256 x 256 tiles: one row per 32 lanes");
    __device__ static __forceinline__ int rowoff(int r) { return r * SH + (r >> 3) * PAD; }
};

// Stages f16(val(r, c, a, dblk)) for the accumulators this wave owns: val gives the final values
// of tile-local row r, columns c .. c+3 from their 4 accumulators a; dblk (wave-uniform) says that
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
    _Float16* S = reinterpret_cast<_Float16*>(smem);
    auto quad = [&](int i, int j, int q) {
        return floatx4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    };
    auto put = [&](int r, int c, const half4& h) { *reinterpret_cast<half4*>(S + EpiH<C>::rowoff(r) + c) = h; };
    auto put_t = [&](int r, int c, const half4& h, bool upper_only) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (!upper_only || c + e > r) S[EpiH<C>::rowoff(c + e) + r] = h[e];
    };
    auto final4 = [&](int r, int c, const floatx4& a, bool dblk) {
        const floatx4 v = val(r, c, a, dblk);
        return half4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    };
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

// Chunk `it` (0 .. ROW_ITERS-1) of this thread in row order: tile-local row 8 * it + tid / 32,
// columns c8 = 8 * (tid % 32) .. c8 + 7; its staging address is one per-thread base plus
// it * ROW_STEP halves.
__device__ __forceinline__ int row_chunk_base() {
    return (threadIdx.x >> 5) * (256 + 8) + (threadIdx.x & 31) * 8;
}

// fn(it, r, c8, h): h = staged row r, columns c8 .. c8+7, over this thread's row chunks. The base
// is opaque to the compiler, which then recomputes each chunk's address rather than keep 32 live.
template <class C, class Fn>
__device__ __forceinline__ void each_row_chunk_h(const char* smem, Fn fn) {
    static_assert(EpiH<C>::SH == 256 + 8, "row_chunk_base");
    const int tr = threadIdx.x >> 5, c8 = (threadIdx.x & 31) * 8;
    int off = row_chunk_base();
    asm volatile("" : "+v"(off));
    const _Float16* base = reinterpret_cast<const _Float16*>(smem) + off;
#pragma unroll
    for (int it = 0; it < EpiH<C>::ROW_ITERS; ++it)
        fn(it, 8 * it + tr, c8, *reinterpret_cast<const half8v*>(base + it * EpiH<C>::ROW_STEP));
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
