// Grouped Newton-Schulz phase kernels over an orthogonalized parameter group (gfx950).
//
// Reference semantics: thorn.py:626-662 (_polar_decomp_impl). The build runs the plain quintic for
// every shape, on the Gram matrix of the short side, in f16 with fp32 accumulation; the first
// iterate is the fp32 momentum update u, scaled by 1/(||u||_F + 1e-8) and rounded to f16 on its way
// into LDS (thorn.py:632-635).
#include "ns_gemm.hpp"
#include "thorn_kernels.hpp"

namespace thorn {

using NsCfg = GemmCfg<128, 128, 64>;

// Input iterate of iteration `it`: the fp32 momentum update for it == 0, then f16 ping-pong.
__device__ __forceinline__ Operand iterate_operand(const OrthoMat& M, int it, bool kmajor) {
    Operand op;
    op.ld = M.ldx;
    op.rows = M.rows;
    op.kmajor = kmajor;
    if (it == 0) {
        op.ptr = M.x0;
        op.scale = M.scal[kScalSigma];
    } else {
        op.ptr = (it & 1) ? M.xa : M.xb;
        op.scale = 1.f;
    }
    return op;
}

__device__ __forceinline__ Operand square_operand(const _Float16* p, const OrthoMat& M) {
    Operand op;
    op.ptr = p;
    op.ld = M.lds;
    op.rows = M.s;
    op.kmajor = 1;
    op.scale = 1.f;
    return op;
}

// out = alpha * acc + beta * Csym + gamma * I on an upper-triangle tile, mirrored below the diagonal.
template <class C>
__device__ __forceinline__ void sym_epilogue(floatx16 (&acc)[C::TM][C::TN], _Float16* out,
                                             const _Float16* csym, int64_t ld, int n, int m0, int n0,
                                             bool mirror, float alpha, float beta, float gamma) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r0 = m0 + acc_row<C>(wave, lane, i, 4 * q);
                const int c = n0 + acc_col<C>(wave, lane, j);
                if (c >= n || r0 >= n) continue;
                float v[4];
                const bool full = r0 + 3 < n;
                half4 cv = half4{0, 0, 0, 0};
                if (beta != 0.f) {
                    if (full) {
                        cv = *reinterpret_cast<const half4*>(csym + (int64_t)c * ld + r0);
                    } else {
                        for (int e = 0; e < 4 && r0 + e < n; ++e) cv[e] = csym[(int64_t)c * ld + r0 + e];
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float t = alpha * acc[i][j][4 * q + e];
                    if (beta != 0.f) t += beta * static_cast<float>(cv[e]);
                    if (r0 + e == c) t += gamma;
                    v[e] = t;
                }
                half4 hv = half4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (r0 + e < n) out[(int64_t)(r0 + e) * ld + c] = hv[e];
                if (mirror) {
                    if (full) {
                        *reinterpret_cast<half4*>(out + (int64_t)c * ld + r0) = hv;
                    } else {
                        for (int e = 0; e < 4 && r0 + e < n; ++e) out[(int64_t)c * ld + r0 + e] = hv[e];
                    }
                }
            }
}

// Phase 1: Gram matrix of the short side of iterate `it` (FIRST: it == 0, fp32 source).
template <bool FIRST>
__global__ __launch_bounds__(256) void ns_gram_kernel(const OrthoMat* __restrict__ mats, TaskList tl, int it) {
    __shared__ __attribute__((aligned(16))) _Float16 smem[NsCfg::LDS_HALVES];
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int T = (M.s + NsCfg::BM - 1) / NsCfg::BM;
    int ti, tj;
    tri_decode(b - tl.starts[k], T, ti, tj);
    // wide (rows <= cols): A = X X^T, contraction over columns (K-major rows of X);
    // tall: A = X^T X, contraction over rows (MN-major columns of X).
    const bool kmaj = !M.tall;
    Operand A = iterate_operand(M, it, kmaj);
    Operand B = A;
    floatx16 acc[NsCfg::TM][NsCfg::TN];
    gemm_mainloop<NsCfg, FIRST, FIRST>(A, B, ti * NsCfg::BM, tj * NsCfg::BN, M.l, acc, smem);
    sym_epilogue<NsCfg>(acc, M.gram, nullptr, M.lds, M.s, ti * NsCfg::BM, tj * NsCfg::BN, ti != tj,
                        1.f, 0.f, 0.f);
}

// Phase 2: P = a I + b A + c A A (A symmetric, so both operands are K-major rows of A).
__global__ __launch_bounds__(256) void ns_poly_kernel(const OrthoMat* __restrict__ mats, TaskList tl,
                                                      float ca, float cb, float cc) {
    __shared__ __attribute__((aligned(16))) _Float16 smem[NsCfg::LDS_HALVES];
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int T = (M.s + NsCfg::BM - 1) / NsCfg::BM;
    int ti, tj;
    tri_decode(b - tl.starts[k], T, ti, tj);
    Operand A = square_operand(M.gram, M);
    floatx16 acc[NsCfg::TM][NsCfg::TN];
    gemm_mainloop<NsCfg, false, false>(A, A, ti * NsCfg::BM, tj * NsCfg::BN, M.s, acc, smem);
    sym_epilogue<NsCfg>(acc, M.poly, M.gram, M.lds, M.s, ti * NsCfg::BM, tj * NsCfg::BN, ti != tj,
                        cc, cb, ca);
}

// Phase 3: X' = P X (wide) or X P (tall). Not final: store the f16 iterate. Final: either apply
// the update to p directly (cautious weight decay, thorn.py:669-702) or store u' in f16 with
// per-row sums of squares for the per-row normalization (thorn.py:758-762).
template <bool FIRST>
__global__ __launch_bounds__(256) void ns_update_kernel(const OrthoMat* __restrict__ mats, TaskList tl,
                                                        int it, int final_iter) {
    __shared__ __attribute__((aligned(16))) _Float16 smem[NsCfg::LDS_HALVES];
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];
    const int ti = local / M.g3_tiles_n, tj = local % M.g3_tiles_n;
    const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
    Operand A, B;
    if (M.tall) {
        A = iterate_operand(M, it, true);      // rows of X, contraction over columns
        B = square_operand(M.poly, M);         // P symmetric: column n of P is row n
    } else {
        A = square_operand(M.poly, M);
        B = iterate_operand(M, it, false);     // X[k][n], contraction over rows
    }
    floatx16 acc[NsCfg::TM][NsCfg::TN];
    if (M.tall) gemm_mainloop<NsCfg, FIRST, false>(A, B, m0, n0, M.s, acc, smem);
    else gemm_mainloop<NsCfg, false, FIRST>(A, B, m0, n0, M.s, acc, smem);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (!final_iter) {
        _Float16* dst = (it & 1) ? M.xb : M.xa;
#pragma unroll
        for (int i = 0; i < NsCfg::TM; ++i)
#pragma unroll
            for (int j = 0; j < NsCfg::TN; ++j) {
                const int c = n0 + acc_col<NsCfg>(wave, lane, j);
                if (c >= M.cols) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + acc_row<NsCfg>(wave, lane, i, r);
                    if (row < M.rows) dst[(int64_t)row * M.ldx + c] = (_Float16)acc[i][j][r];
                }
            }
        return;
    }

    float* red = reinterpret_cast<float*>(smem);
    __syncthreads();   // smem is reused below
    if (M.flags & kFlagPNN) {
        // u' in f16 (the reference's polar factor is f16 rounded, thorn.py:635, 662) and per-row
        // partial sums of u'^2 over this tile's columns.
        float rs[NsCfg::TM][16];
#pragma unroll
        for (int i = 0; i < NsCfg::TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) rs[i][r] = 0.f;
#pragma unroll
        for (int i = 0; i < NsCfg::TM; ++i)
#pragma unroll
            for (int j = 0; j < NsCfg::TN; ++j) {
                const int c = n0 + acc_col<NsCfg>(wave, lane, j);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + acc_row<NsCfg>(wave, lane, i, r);
                    const _Float16 h = (_Float16)acc[i][j][r];
                    if (c < M.cols && row < M.rows) {
                        M.uout[(int64_t)row * M.ldx + c] = h;
                        const float f = (float)h;
                        rs[i][r] += f * f;
                    }
                }
            }
        // reduce over the 32 columns of each half-wave, then over the two column-waves
#pragma unroll
        for (int i = 0; i < NsCfg::TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float v = halfwave_sum(rs[i][r]);
                if ((lane & 31) == 0) {
                    const int row = acc_row<NsCfg>(wave, lane, i, r);
                    red[(wave & 1) * NsCfg::BM + row] = v;
                }
            }
        __syncthreads();
        for (int row = threadIdx.x; row < NsCfg::BM; row += 256) {
            const int gr = m0 + row;
            if (gr < M.rows) M.rowsqpart[(int64_t)tj * M.rows + gr] = red[row] + red[NsCfg::BM + row];
        }
        return;
    }

    // Direct apply: p <- p - eta * (u + wd * p * [u * p >= 0]) (thorn.py:679-680, 702).
    const bool md = (M.flags & (kFlagMD | kFlagMDScalar)) != 0;
    const bool apply = (M.flags & kFlagApply) != 0;
    float psq = 0.f;
#pragma unroll
    for (int i = 0; i < NsCfg::TM; ++i)
#pragma unroll
        for (int j = 0; j < NsCfg::TN; ++j) {
            const int c = n0 + acc_col<NsCfg>(wave, lane, j);
            if (c >= M.cols) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + acc_row<NsCfg>(wave, lane, i, r);
                if (row >= M.rows) continue;
                float* pp = M.p + (int64_t)row * M.cols + c;
                float p = *pp;
                if (apply) {
                    const float u = (float)(_Float16)acc[i][j][r];
                    p = cautious_step(p, u, M.eta, M.wd);
                    *pp = p;
                }
                psq += p * p;
            }
        }
    if (md) {
        const float t = block_sum(psq, red);
        if (threadIdx.x == 0) M.psqpart[local] = t;
    }
}

}  // namespace thorn
