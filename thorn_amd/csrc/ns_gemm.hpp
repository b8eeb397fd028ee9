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

// Block tile BM x BN, K step BK, 256 threads as 2 x 2 waves, each wave (BM/2) x (BN/2).
template <int BM_, int BN_, int BK_>
struct GemmCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr int WM = BM / 2, WN = BN / 2;
    static constexpr int TM = WM / 32, TN = WN / 32;
    static constexpr int PADK = 8;    // row padding (halves) of K-major tiles: 144-byte rows for BK=64
    static constexpr int PADM = 16;   // row padding (halves) of MN-major tiles
    static constexpr int LDK = BK + PADK;
    static constexpr int LDA_MN = BM + PADM;
    static constexpr int LDB_MN = BN + PADM;
    static constexpr int A_HALVES = (BM * LDK > BK * LDA_MN) ? BM * LDK : BK * LDA_MN;
    static constexpr int B_HALVES = (BN * LDK > BK * LDB_MN) ? BN * LDK : BK * LDB_MN;
    static constexpr int STAGE_HALVES = A_HALVES + B_HALVES;
    static constexpr int LDS_HALVES = 2 * STAGE_HALVES;
    static constexpr int A_CHUNKS = BM * BK / 8 / 256;   // 16-byte chunks per thread per K step
    static constexpr int B_CHUNKS = BN * BK / 8 / 256;
    static_assert(A_CHUNKS * 256 * 8 == BM * BK, "A tile must split evenly over 256 threads");
    static_assert(B_CHUNKS * 256 * 8 == BN * BK, "B tile must split evenly over 256 threads");
};

// A GEMM operand in global memory: element (mn, k) lives at
//   K-major:  ptr[mn * ld + k]     (rows = number of valid mn rows)
//   MN-major: ptr[k * ld + mn]     (rows = number of valid k rows)
// ld is a multiple of 8 and the padding columns [logical width, ld) hold zeros, so a 16-byte
// chunk is either entirely inside a row or entirely outside it.
// Sources are f16, or fp32 (the first iterate) converted to f16 after scaling by `scale` on its
// way into LDS; the element type is a template parameter of the loader (F32).
struct Operand {
    const void* ptr;
    int64_t ld;
    int32_t rows;
    int32_t kmajor;
    float scale;
};

// Loads this thread's 16-byte f16 chunks (or 32-byte fp32 chunks, two registers each) of a tile.
template <int MNROWS, int BK, bool F32, int NREG>
__device__ __forceinline__ void gload(const Operand& op, int mn0, int k0, uint4 (&r)[NREG]) {
    constexpr int NCH = F32 ? NREG / 2 : NREG;
    constexpr int ESZ = F32 ? 4 : 2;
    const char* base = static_cast<const char*>(op.ptr);
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
        const int id = threadIdx.x + 256 * q;
        int64_t row, col;
        if (op.kmajor) {
            row = mn0 + id / (BK / 8);
            col = k0 + (id % (BK / 8)) * 8;
        } else {
            row = k0 + id / (MNROWS / 8);
            col = mn0 + (id % (MNROWS / 8)) * 8;
        }
        const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
        if (row < op.rows && col < op.ld) {
            const uint4* src = reinterpret_cast<const uint4*>(base + (row * op.ld + col) * ESZ);
            if (F32) {
                r[2 * q] = src[0];
                r[2 * q + 1] = src[1];
            } else {
                r[q] = src[0];
            }
        } else if (F32) {
            r[2 * q] = zero;
            r[2 * q + 1] = zero;
        } else {
            r[q] = zero;
        }
    }
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
}

__device__ __forceinline__ uint4 f32x8_to_f16x8(uint4 a, uint4 b, float s) {
    uint4 o;
    o.x = pack_h2(__uint_as_float(a.x) * s, __uint_as_float(a.y) * s);
    o.y = pack_h2(__uint_as_float(a.z) * s, __uint_as_float(a.w) * s);
    o.z = pack_h2(__uint_as_float(b.x) * s, __uint_as_float(b.y) * s);
    o.w = pack_h2(__uint_as_float(b.z) * s, __uint_as_float(b.w) * s);
    return o;
}

template <int MNROWS, int BK, int LDK, int LDMN, bool F32, int NREG>
__device__ __forceinline__ void lstore(const Operand& op, _Float16* lds, uint4 (&r)[NREG]) {
    constexpr int NCH = F32 ? NREG / 2 : NREG;
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
        const int id = threadIdx.x + 256 * q;
        int off;
        if (op.kmajor) off = (id / (BK / 8)) * LDK + (id % (BK / 8)) * 8;
        else off = (id / (MNROWS / 8)) * LDMN + (id % (MNROWS / 8)) * 8;
        const uint4 v = F32 ? f32x8_to_f16x8(r[2 * q], r[2 * q + 1], op.scale) : r[q];
        *reinterpret_cast<uint4*>(lds + off) = v;
    }
}

typedef __attribute__((address_space(3))) short4v lds_s4;

// MFMA fragment (8 halves) for 32-row tile `t0` (offset inside the block tile) at k step `kk`.
template <int LDK, int LDMN>
__device__ __forceinline__ half8 frag(const _Float16* lds, bool kmajor, int t0, int kk, int lane) {
    if (kmajor) {
        return *reinterpret_cast<const half8*>(lds + (t0 + (lane & 31)) * LDK + kk + 8 * (lane >> 5));
    }
    const int k = kk + 8 * (lane >> 5) + ((lane & 15) >> 2);
    const int mn = t0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(lds + k * LDMN + mn));
    short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(lds + (k + 4) * LDMN + mn));
    half4 l4 = __builtin_bit_cast(half4, lo), h4 = __builtin_bit_cast(half4, hi);
    return half8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
}

// acc[i][j] += A[m0 + wm + 32i .., 0:K] * B[0:K, n0 + wn + 32j ..] over the whole K range.
template <class C, bool AF32, bool BF32>
__device__ __forceinline__ void gemm_mainloop(const Operand& A, const Operand& B, int m0, int n0,
                                              int K, floatx16 (&acc)[C::TM][C::TN], _Float16* smem) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * C::WM, wn = (wave & 1) * C::WN;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = floatx16{};

    uint4 ra[C::A_CHUNKS * (AF32 ? 2 : 1)], rb[C::B_CHUNKS * (BF32 ? 2 : 1)];
    const int KT = (K + C::BK - 1) / C::BK;
    gload<C::BM, C::BK, AF32>(A, m0, 0, ra);
    gload<C::BN, C::BK, BF32>(B, n0, 0, rb);
    lstore<C::BM, C::BK, C::LDK, C::LDA_MN, AF32>(A, smem, ra);
    lstore<C::BN, C::BK, C::LDK, C::LDB_MN, BF32>(B, smem + C::A_HALVES, rb);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        _Float16* sa = smem + (kt & 1) * C::STAGE_HALVES;
        _Float16* sb = sa + C::A_HALVES;
        const bool more = kt + 1 < KT;
        if (more) {
            gload<C::BM, C::BK, AF32>(A, m0, (kt + 1) * C::BK, ra);
            gload<C::BN, C::BK, BF32>(B, n0, (kt + 1) * C::BK, rb);
        }
#pragma unroll
        for (int kk = 0; kk < C::BK; kk += 16) {
            half8 fa[C::TM], fb[C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; ++i) fa[i] = frag<C::LDK, C::LDA_MN>(sa, A.kmajor, wm + 32 * i, kk, lane);
#pragma unroll
            for (int j = 0; j < C::TN; ++j) fb[j] = frag<C::LDK, C::LDB_MN>(sb, B.kmajor, wn + 32 * j, kk, lane);
#pragma unroll
            for (int i = 0; i < C::TM; ++i)
#pragma unroll
                for (int j = 0; j < C::TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            _Float16* na = smem + ((kt + 1) & 1) * C::STAGE_HALVES;
            lstore<C::BM, C::BK, C::LDK, C::LDA_MN, AF32>(A, na, ra);
            lstore<C::BN, C::BK, C::LDK, C::LDB_MN, BF32>(B, na + C::A_HALVES, rb);
        }
        __syncthreads();
    }
}

// Row index (inside the block tile) of accumulator register r of 32x32 tile i for this lane.
template <class C>
__device__ __forceinline__ int acc_row(int wave, int lane, int i, int r) {
    return (wave >> 1) * C::WM + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}
template <class C>
__device__ __forceinline__ int acc_col(int wave, int lane, int j) {
    return (wave & 1) * C::WN + 32 * j + (lane & 31);
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
