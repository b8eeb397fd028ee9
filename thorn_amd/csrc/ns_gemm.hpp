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

    // The loads are written as inline assembly so that the compiler does not track them as LDS
    // writes: its conservative aliasing would otherwise wait for every outstanding load before
    // the next LDS fragment read and serialize the pipeline. The main loop orders them explicitly
    // (lds_wait_barrier); the "memory" clobber keeps LDS accesses from moving across them.
    __device__ __forceinline__ void issue(int t, char* lds, const void* zero, int wave) const {
        const uint32_t base = __builtin_amdgcn_readfirstlane(lds_address(lds) + wave * PER_WAVE * 1024);
        const int64_t off = t * step;
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const void* p = (t * BKC < lim[q]) ? static_cast<const void*>(src[q] + off) : zero;
            asm volatile("global_load_lds_dwordx4 %0, off" ::"v"((const THORN_GLOBAL void*)p), "{m0}"(base + q * 1024)
                         : "memory");
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

// Scheduling hint for one k16 sub-step: NM MFMAs spread evenly between NR LDS fragment reads.
template <int NM, int NR, int Q = 0>
__device__ __forceinline__ void interleave_mfma_ds() {
    if constexpr (Q < NR) {
        constexpr int m = (Q + 1) * NM / NR - Q * NM / NR;
        if constexpr (m > 0) __builtin_amdgcn_sched_group_barrier(0x008, m, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        interleave_mfma_ds<NM, NR, Q + 1>();
    }
}

// acc[i][j] += A[m0 + wm + 32i .., K tiles kt0 .. kt_end) * B[.., n0 + wn + 32j ..] with operand
// layouts AK / BK (true = K-major).
// The MFMA is issued as B^T A^T, so each 32 x 32 accumulator comes out transposed: lane l holds
// row (l & 31) and the four consecutive columns 8*(r/4) + 4*(l/32) + 0..3 in registers r..r+3,
// which the epilogue writes to LDS as one 16-byte store.
//
// Pipeline over K tiles of 32 (S LDS stages, one block barrier per tile):
//   tile t is loaded into stage (t - kt0) % S S-1 tiles ahead of its use, by direct global->LDS
//   loads; each tile is two k16 sub-steps; the LDS fragment reads of the next sub-step are in
//   flight while the MFMAs of the current one run. Between the two sub-steps of tile t every wave
//   waits for its own loads of tile t+1 and meets the others at the barrier: after it, tile t+1
//   is visible and nobody reads stage (t-1) % S any more, which then receives tile t+S-1. The
//   range ends with every load complete and a barrier, so the stages are free again.
template <class C, bool AK, bool BK>
__device__ __forceinline__ void mainloop_range(const Operand& A, const Operand& B, int m0, int n0, int kt0,
                                               int kt_end, floatx16 (&acc)[C::TM][C::TN], char* smem,
                                               const void* zero) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * C::WM, wn = (wave & 1) * C::WN;
    DmaSrc<C::BM, AK> da;
    DmaSrc<C::BN, BK> db;
    da.init(A, m0, wave, lane);
    db.init(B, n0, wave, lane);
    const int KT = kt_end;
    auto stage_a = [&](int t) { return smem + ((t - kt0) % C::S) * C::STAGE_BYTES; };
    auto issue = [&](int t) {
        char* st = stage_a(t);
        da.issue(t, st, zero, wave);
        db.issue(t, st + C::A_BYTES, zero, wave);
    };
#pragma unroll
    for (int t = 0; t < C::S - 1; ++t)
        if (kt0 + t < KT) issue(kt0 + t);
    // tile kt0 ready: loads of the next min(S-2, n-1) tiles may still be in flight
    static_assert(C::S >= 3 && C::S <= 5, "pipeline depth");
    const int n = KT - kt0;
    if (C::S >= 5 && n >= 4) lds_wait_barrier<3 * C::LOADS_PER_STAGE>();
    else if (C::S >= 4 && n >= 3) lds_wait_barrier<2 * C::LOADS_PER_STAGE>();
    else if (n >= 2) lds_wait_barrier<C::LOADS_PER_STAGE>();
    else lds_wait_barrier<0>();

    constexpr int NREAD = C::TM * (AK ? 1 : 2) + C::TN * (BK ? 1 : 2);   // LDS reads per sub-step
    half8 fa[2][C::TM], fb[2][C::TN];
    {
        const char* sa = stage_a(kt0);
#pragma unroll
        for (int i = 0; i < C::TM; ++i) fa[0][i] = frag<C::BM, AK>(sa, wm + 32 * i, 0, lane);
#pragma unroll
        for (int j = 0; j < C::TN; ++j) fb[0][j] = frag<C::BN, BK>(sa + C::A_BYTES, wn + 32 * j, 0, lane);
    }
    for (int kt = kt0; kt < KT; ++kt) {
        const char* sa = stage_a(kt);
        // sub-step 0: read sub-step 1's fragments while the MFMAs of sub-step 0 run
#pragma unroll
        for (int i = 0; i < C::TM; ++i) fa[1][i] = frag<C::BM, AK>(sa, wm + 32 * i, 1, lane);
#pragma unroll
        for (int j = 0; j < C::TN; ++j) fb[1][j] = frag<C::BN, BK>(sa + C::A_BYTES, wn + 32 * j, 1, lane);
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
            for (int j = 0; j < C::TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[0][j], fa[0][i], acc[i][j], 0, 0, 0);
        interleave_mfma_ds<C::TM * C::TN, NREAD>();
        __builtin_amdgcn_sched_barrier(0);
        // tile kt+1 ready (tiles kt+2 .. kt+S-2 may still be in flight), stage (kt-1) % S free
        {
            const int ahead = (KT - 1 < kt + C::S - 2 ? KT - 1 : kt + C::S - 2) - (kt + 1);
            if (C::S >= 5 && ahead >= 2) lds_wait_barrier<2 * C::LOADS_PER_STAGE>();
            else if (C::S >= 4 && ahead >= 1) lds_wait_barrier<C::LOADS_PER_STAGE>();
            else lds_wait_barrier<0>();
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kt + C::S - 1 < KT) issue(kt + C::S - 1);
        // sub-step 1: read the next tile's first fragments while the MFMAs of sub-step 1 run
        if (kt + 1 < KT) {
            const char* na = stage_a(kt + 1);
#pragma unroll
            for (int i = 0; i < C::TM; ++i) fa[0][i] = frag<C::BM, AK>(na, wm + 32 * i, 0, lane);
#pragma unroll
            for (int j = 0; j < C::TN; ++j) fb[0][j] = frag<C::BN, BK>(na + C::A_BYTES, wn + 32 * j, 0, lane);
        }
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
            for (int j = 0; j < C::TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
        interleave_mfma_ds<C::TM * C::TN, NREAD>();
        __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier();   // every wave is done with the stages
}

// acc = A[m0 .., 0:K] * B[0:K, n0 ..] where A is read MN-major for K tiles t < a_k0 and K-major
// from there on, B likewise with b_k0: a symmetric matrix stored as its upper block triangle is
// read K-major from its diagonal block on and MN-major, from the transposed mirror block, before
// it. One pipelined loop: the direct loads and the fragment reads of a tile branch on its layout
// (uniformly), the MFMAs do not, so the accumulators keep one register assignment.
template <class C>
__device__ __forceinline__ void gemm_mainloop_mixed(const Operand& A, const Operand& B, int m0, int n0, int K,
                                                    int a_k0, int b_k0, floatx16 (&acc)[C::TM][C::TN], char* smem,
                                                    const void* zero) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * C::WM, wn = (wave & 1) * C::WN;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = floatx16{};
    DmaSrc<C::BM, true> dak;
    DmaSrc<C::BM, false> dam;
    DmaSrc<C::BN, true> dbk;
    DmaSrc<C::BN, false> dbm;
    dak.init(A, m0, wave, lane);
    dam.init(A, m0, wave, lane);
    dbk.init(B, n0, wave, lane);
    dbm.init(B, n0, wave, lane);
    const int KT = (K + C::BK - 1) / C::BK;
    auto stage_a = [&](int t) { return smem + (t % C::S) * C::STAGE_BYTES; };
    auto issue = [&](int t) {
        char* st = stage_a(t);
        if (t >= a_k0) dak.issue(t, st, zero, wave);
        else dam.issue(t, st, zero, wave);
        if (t >= b_k0) dbk.issue(t, st + C::A_BYTES, zero, wave);
        else dbm.issue(t, st + C::A_BYTES, zero, wave);
    };
    auto read = [&](int t, int ks, half8 (&ra)[C::TM], half8 (&rb)[C::TN]) {
        const char* st = stage_a(t);
        if (t >= a_k0) {
#pragma unroll
            for (int i = 0; i < C::TM; ++i) ra[i] = frag<C::BM, true>(st, wm + 32 * i, ks, lane);
        } else {
#pragma unroll
            for (int i = 0; i < C::TM; ++i) ra[i] = frag<C::BM, false>(st, wm + 32 * i, ks, lane);
        }
        if (t >= b_k0) {
#pragma unroll
            for (int j = 0; j < C::TN; ++j) rb[j] = frag<C::BN, true>(st + C::A_BYTES, wn + 32 * j, ks, lane);
        } else {
#pragma unroll
            for (int j = 0; j < C::TN; ++j) rb[j] = frag<C::BN, false>(st + C::A_BYTES, wn + 32 * j, ks, lane);
        }
    };
    auto mfmas = [&](const half8 (&ra)[C::TM], const half8 (&rb)[C::TN]) {
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
            for (int j = 0; j < C::TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(rb[j], ra[i], acc[i][j], 0, 0, 0);
    };
#pragma unroll
    for (int t = 0; t < C::S - 1; ++t)
        if (t < KT) issue(t);
    static_assert(C::S >= 3 && C::S <= 5, "pipeline depth");
    if (C::S >= 5 && KT >= 4) lds_wait_barrier<3 * C::LOADS_PER_STAGE>();
    else if (C::S >= 4 && KT >= 3) lds_wait_barrier<2 * C::LOADS_PER_STAGE>();
    else if (KT >= 2) lds_wait_barrier<C::LOADS_PER_STAGE>();
    else lds_wait_barrier<0>();
    half8 fa[2][C::TM], fb[2][C::TN];
    if (KT > 0) read(0, 0, fa[0], fb[0]);
    for (int kt = 0; kt < KT; ++kt) {
        read(kt, 1, fa[1], fb[1]);   // sub-step 1's fragments, in flight during sub-step 0's MFMAs
        mfmas(fa[0], fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        {
            const int ahead = (KT - 1 < kt + C::S - 2 ? KT - 1 : kt + C::S - 2) - (kt + 1);
            if (C::S >= 5 && ahead >= 2) lds_wait_barrier<2 * C::LOADS_PER_STAGE>();
            else if (C::S >= 4 && ahead >= 1) lds_wait_barrier<C::LOADS_PER_STAGE>();
            else lds_wait_barrier<0>();
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kt + C::S - 1 < KT) issue(kt + C::S - 1);
        if (kt + 1 < KT) read(kt + 1, 0, fa[0], fb[0]);   // next tile's first fragments
        mfmas(fa[1], fb[1]);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Single-layout main loop: AK / BK = whether A / B are K-major.
template <class C, bool AK, bool BK>
__device__ __forceinline__ void gemm_mainloop(const Operand& A, const Operand& B, int m0, int n0,
                                              int K, floatx16 (&acc)[C::TM][C::TN], char* smem,
                                              const void* zero) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = floatx16{};
    mainloop_range<C, AK, BK>(A, B, m0, n0, 0, (K + C::BK - 1) / C::BK, acc, smem, zero);
}

// Epilogue: the tile is streamed through LDS (reusing the pipeline stages) in two halves of
// WM = BM/2 rows, the rows owned by one row of waves:
//   for_rows: N[row][col] staging (fp32); each thread then gets 8 consecutive columns of one row,
//             so global traffic is 16-byte chunks with 32 lanes on one row;
//   for_cols: transposed staging T[col][row]; each thread gets 8 consecutive rows of one column
//             (the mirrored tile of a symmetric product).
template <class C>
struct Epi {
    static constexpr int NS = C::BN + 4;    // N row stride (floats): 16 lanes x 16 B on distinct banks
    static constexpr int TS = C::WM + 4;    // T row stride (floats)
    static constexpr int N_BYTES = C::WM * NS * 4;
    static constexpr int T_BYTES = C::BN * TS * 4;
    static constexpr int BYTES = N_BYTES > T_BYTES ? N_BYTES : T_BYTES;
    static constexpr int SMEM = BYTES > C::LDS_BYTES ? BYTES : C::LDS_BYTES;
    static constexpr int ROW_CHUNKS = C::WM * (C::BN / 8) / 256;   // per thread per half
    static constexpr int COL_CHUNKS = C::BN * (C::WM / 8) / 256;
};

// Chunk `it` of this thread in a half: 32 lanes of a wave share one row (row passes) or 16 lanes
// one column (column passes), so every global access of a chunk pass is coalesced.
template <class C>
__device__ __forceinline__ void row_chunk(int it, int& r, int& c8) {
    const int idx = it * 256 + threadIdx.x;
    r = idx / (C::BN / 8);
    c8 = (idx % (C::BN / 8)) * 8;
}
template <class C>
__device__ __forceinline__ void col_chunk(int it, int& c, int& r8) {
    const int idx = it * 256 + threadIdx.x;
    c = idx / (C::WM / 8);
    r8 = (idx % (C::WM / 8)) * 8;
}

// fn(it, half, local_row, col8, float (&v)[8]): v = acc[row][col8 .. col8+7] (tile coordinates:
// row = half * WM + local_row); `it` numbers this thread's chunks 0 .. ROW_CHUNKS-1, in the order
// given by row_chunk().
template <class C, class Fn>
__device__ __forceinline__ void for_rows(floatx16 (&acc)[C::TM][C::TN], char* smem, int half, Fn fn) {
    using E = Epi<C>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* N = reinterpret_cast<float*>(smem);
    lds_barrier();   // the previous user of smem (main loop or another pass) is done
    if ((wave >> 1) == half) {
        const int wn = (wave & 1) * C::WN;
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
            for (int j = 0; j < C::TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 32 * i + (lane & 31);
                    const int c = wn + 32 * j + 8 * q + 4 * (lane >> 5);
                    *reinterpret_cast<floatx4*>(N + r * E::NS + c) =
                        floatx4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                }
    }
    lds_barrier();
#pragma unroll
    for (int it = 0; it < E::ROW_CHUNKS; ++it) {
        int r, c8;
        row_chunk<C>(it, r, c8);
        const floatx4 a = *reinterpret_cast<const floatx4*>(N + r * E::NS + c8);
        const floatx4 b = *reinterpret_cast<const floatx4*>(N + r * E::NS + c8 + 4);
        float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        fn(it, half, r, c8, v);
    }
}

// fn(it, half, col, local_row8, float (&v)[8]): v = acc[row8 .. row8+7][col] with
// row8 = half*WM + local_row8; chunk order given by col_chunk().
template <class C, class Fn>
__device__ __forceinline__ void for_cols(floatx16 (&acc)[C::TM][C::TN], char* smem, int half, Fn fn) {
    using E = Epi<C>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* T = reinterpret_cast<float*>(smem);
    lds_barrier();
    if ((wave >> 1) == half) {
        const int wn = (wave & 1) * C::WN;
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
            for (int j = 0; j < C::TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 32 * i + (lane & 31);
                        const int c = wn + 32 * j + 8 * q + 4 * (lane >> 5) + e;
                        T[c * E::TS + r] = acc[i][j][4 * q + e];
                    }
    }
    lds_barrier();
#pragma unroll
    for (int it = 0; it < E::COL_CHUNKS; ++it) {
        int c, r8;
        col_chunk<C>(it, c, r8);
        const floatx4 a = *reinterpret_cast<const floatx4*>(T + c * E::TS + r8);
        const floatx4 b = *reinterpret_cast<const floatx4*>(T + c * E::TS + r8 + 4);
        float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        fn(it, half, c, r8, v);
    }
}

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

__device__ __forceinline__ half8v to_half8(const float (&v)[8]) {
    return half8v{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3],
                  (_Float16)v[4], (_Float16)v[5], (_Float16)v[6], (_Float16)v[7]};
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
