// thorn::sym_addmm as a standalone batched operation (gfx950): out = f16(beta * C + alpha * A B)
// for products A B (and C) that are symmetric, on the Newton-Schulz engine's 256 x 256 tiles.
//
// The Newton-Schulz launches run these products inside their own workspace layout; this entry
// point gives the same tiles to caller tensors of any strides. Three launches:
//   1. sym_pack_kernel copies A (rows of A, K contiguous) and B^T (columns of B, K contiguous), and
//      C, into the engine's layouts, rows padded with zeros to a multiple of 32 (K) or 8 (C);
//   2. sym_addmm_kernel computes the upper block triangle of every product, one tile per block
//      (gemm_tile, then sym_store: one rounding of beta * C + alpha * A B, diagonal tiles computed
//      above their diagonal and mirrored, as the reference's Triton kernel does, thorn.py:209-280);
//   3. sym_unpack_kernel writes the caller's contiguous (nn, m, m) output, a block below the
//      diagonal read as the transpose of its mirror.
#include "ns_kernels.hip"

namespace thorn {

constexpr int kSymPackThreads = 256;

// dst[row][c] = src[b * s0 + r * s1 + c * s2] for c < cols and 0 for cols <= c < ld (row = b * rows
// + r; ld a multiple of 8): one 16-byte chunk of dst per thread and grid-stride step.
__global__ __launch_bounds__(kSymPackThreads) void sym_pack_kernel(const _Float16* __restrict__ src, int64_t s0,
                                                                   int64_t s1, int64_t s2, _Float16* __restrict__ dst,
                                                                   int rows, int cols, int ld, int64_t chunks) {
    const int cpr = ld / 8;
    for (int64_t i = int64_t(blockIdx.x) * kSymPackThreads + threadIdx.x; i < chunks;
         i += int64_t(gridDim.x) * kSymPackThreads) {
        const int64_t row = i / cpr;
        const int c8 = static_cast<int>(i - row * cpr) * 8;
        const int64_t b = row / rows;
        const int r = static_cast<int>(row - b * rows);
        const _Float16* s = src + b * s0 + int64_t(r) * s1;
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = c8 + e < cols ? s[int64_t(c8 + e) * s2] : static_cast<_Float16>(0.f);
        stg<half8>(dst + row * ld + c8, h);
    }
}

struct SymAddmmArgs {
    const _Float16* a;    // [nn][m][kp]: rows of A, K contiguous, zeros past k
    const _Float16* bt;   // [nn][m][kp]: rows of B^T
    const _Float16* c;    // [nc][m][mp] (nc = 1: one C for every product) or null
    _Float16* out;        // [nn][m][mp]: the upper block triangle of each result
    int64_t ab_mat, c_mat, o_mat;   // elements per matrix of a / bt, c (0: one C), out
    int32_t m, kp, mp, tiles;       // tiles: upper-triangle tiles of one result
    float alpha, beta;
};

template <int ROLE>
__device__ __forceinline__ void sym_addmm_tile(const SymAddmmArgs& p, const Operand& A, const Operand& B,
                                               const TileC& ct, _Float16* out, int m0, int n0, const TileWork& tw,
                                               char* smem) {
    floatx16 acc[RoleMap<ROLE>::N];
    gemm_tile<NsCfg, ROLE>(A, B, m0, n0, p.kp / NsCfg::BK, 0, 0, ct, tw, acc, smem);
    const TileOut o{out + int64_t(m0) * p.mp, p.mp, p.m - m0, 0};
    if (ct.ptr) {
        if (p.alpha != 1.f) sym_store<NsCfg, ROLE, true, true>(acc, tw, smem, o, m0, n0, p.alpha, p.beta);
        else sym_store<NsCfg, ROLE, true, false>(acc, tw, smem, o, m0, n0, 1.f, p.beta);
    } else {
        if (p.alpha != 1.f) sym_store<NsCfg, ROLE, false, true>(acc, tw, smem, o, m0, n0, p.alpha, 0.f);
        else sym_store<NsCfg, ROLE, false, false>(acc, tw, smem, o, m0, n0, 1.f, 0.f);
    }
}

// One upper-triangle tile of one product per block: block = product * tiles + tile.
__global__ __launch_bounds__(NsCfg::NT) void sym_addmm_kernel(SymAddmmArgs p) {
    __shared__ __attribute__((aligned(16))) char smem[EpiH<NsCfg>::SMEM];
    const int b = blockIdx.x / p.tiles, local = blockIdx.x - b * p.tiles;
    int ti, tj;
    tri_decode(local, (p.m + NsCfg::BM - 1) / NsCfg::BM, ti, tj);
    Operand A, B;
    A.ptr = p.a + b * p.ab_mat;
    B.ptr = p.bt + b * p.ab_mat;
    A.ld = B.ld = p.kp;
    A.rows = B.rows = p.m;
    A.packed = B.packed = 0;
    const TileC ct{p.c ? p.c + b * p.c_mat : nullptr, p.mp, p.m, 0, 0};
    _Float16* const out = p.out + b * p.o_mat;
    const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const TileWork tw(ti == tj, wave);
    switch (tw.role) {
        case kRoleFull: sym_addmm_tile<kRoleFull>(p, A, B, ct, out, m0, n0, tw, smem); break;
        case kRoleDiagA: sym_addmm_tile<kRoleDiagA>(p, A, B, ct, out, m0, n0, tw, smem); break;
        case kRoleDiagB: sym_addmm_tile<kRoleDiagB>(p, A, B, ct, out, m0, n0, tw, smem); break;
        default: sym_addmm_tile<kRoleHalf>(p, A, B, ct, out, m0, n0, tw, smem); break;
    }
}

// out[b][i][j] (contiguous nn x m x m) from the upper block triangle in buf ([nn][m][mp]): element
// (i, j) with block row i / 256 above block column j / 256 is read as (j, i).
__global__ __launch_bounds__(kSymPackThreads) void sym_unpack_kernel(const _Float16* __restrict__ buf, int mp,
                                                                     _Float16* __restrict__ out, int m, int64_t total) {
    const int64_t mm = int64_t(m) * m;
    for (int64_t i = int64_t(blockIdx.x) * kSymPackThreads + threadIdx.x; i < total;
         i += int64_t(gridDim.x) * kSymPackThreads) {
        const int64_t b = i / mm;
        const int64_t e = i - b * mm;
        const int r = static_cast<int>(e / m), c = static_cast<int>(e - int64_t(r) * m);
        const bool upper = r / NsCfg::BM <= c / NsCfg::BN;
        const int64_t src = upper ? int64_t(r) * mp + c : int64_t(c) * mp + r;
        out[i] = buf[b * int64_t(m) * mp + src];
    }
}

}  // namespace thorn
