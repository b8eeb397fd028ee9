// Grouped Newton-Schulz phase kernels over an orthogonalized parameter group (gfx950).
//
// Reference semantics: thorn.py:626-662 (_polar_decomp_impl). The build runs the plain quintic for
// every shape, on the Gram matrix of the short side, in f16 with fp32 accumulation; the first
// iterate is the fp32 momentum update u scaled by 1/(||u||_F + 1e-8) and rounded to f16
// (thorn.py:632-635) by ortho_cast_kernel.
#include "ns_gemm.hpp"
#include "thorn_kernels.hpp"

namespace thorn {

using NsCfg = GemmCfg<256, 256>;

// Input iterate of iteration `it` (f16): iteration 0 reads xb (the scaled first iterate), then the
// iterates alternate xa, xb, ...
__device__ __forceinline__ Operand iterate_operand(const OrthoMat& M, int it) {
    Operand op;
    op.ptr = (it & 1) ? M.xa : M.xb;
    op.ld = M.ldx;
    op.rows = M.rows;
    return op;
}

__device__ __forceinline__ Operand square_operand(const _Float16* p, const OrthoMat& M) {
    Operand op;
    op.ptr = p;
    op.ld = M.lds;
    op.rows = M.s;
    return op;
}

// First iterate: xb = f16(u * sigma), sigma = 1 / (||u||_F + 1e-8), over 16 x 256 tiles.
__global__ __launch_bounds__(256) void ortho_cast_kernel(const OrthoMat* __restrict__ mats, TaskList tl) {
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];
    const int tr = local / M.mom_tiles_c, tc = local % M.mom_tiles_c;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (M.flags & kFlagPrescaled) return;   // ortho_pre_kernel wrote xb (ortho_repair_kernel checks it)
    const float sigma = M.scal[kScalSigma];
    const int r0 = tr * 16 + wave * 4;
    const int c = tc * 256 + 4 * lane;
    if (c >= M.ldx) return;
    // x0 and xb share the padded layout; the padding of x0 is zero, so whole 4-chunks are safe
    float4 u[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
        if (r0 + rr < M.rows) u[rr] = ldg<float4>(M.x0 + (int64_t)(r0 + rr) * M.ldx + c);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        if (r0 + rr >= M.rows) break;
        const half4 h = half4{(_Float16)(u[rr].x * sigma), (_Float16)(u[rr].y * sigma), (_Float16)(u[rr].z * sigma),
                              (_Float16)(u[rr].w * sigma)};
        stg<half4>(M.xb + (int64_t)(r0 + rr) * M.ldx + c, h);
    }
}

// Prescaled first iterates whose scale drifted too far (kScalRepair): rebuild xb = f16(sigma * u)
// exactly from the gradient and the updated moment, u = g + beta1 * m (such matrices have no
// decouple_md). One block per matrix; the common case is an immediate exit.
__global__ __launch_bounds__(256) void ortho_repair_kernel(const OrthoMat* __restrict__ mats) {
    const OrthoMat& M = mats[blockIdx.x];
    if (!(M.flags & kFlagPrescaled) || M.scal[kScalRepair] == 0.f) return;
    const float sigma = M.scal[kScalSigma];
    for (int r = 0; r < M.rows; ++r)
        for (int c = threadIdx.x; c < M.cols; c += 256) {
            const int64_t i = (int64_t)r * M.cols + c;
            const float u = fmaf(ldg<float>(M.m + i), M.beta1, ldg<float>(M.g + i));
            M.xb[(int64_t)r * M.ldx + c] = (_Float16)(u * sigma);
        }
}

// out = alpha * acc + beta * Csym + gamma * I (f16) on an upper-triangle tile, and the same values
// mirrored into the transposed tile below the diagonal. Csym is symmetric, so the term for
// (r, c) can be read from row r or row c alike.
template <class C>
__device__ __forceinline__ void sym_store(floatx16 (&acc)[C::TM][C::TN], char* smem, _Float16* out,
                                          const _Float16* csym, int64_t ld, int n, int m0, int n0,
                                          bool mirror, float alpha, float beta, float gamma) {
    using E = Epi<C>;
#pragma unroll 1
    for (int h = 0; h < 2; ++h) {
        // the beta * Csym chunks of a pass are all requested before any of them is needed (the
        // loads overlap the LDS staging)
        half8v cpre[E::ROW_CHUNKS];
        static_assert(E::ROW_CHUNKS == E::COL_CHUNKS, "one prefetch buffer serves both passes");
        if (beta != 0.f) {
#pragma unroll
            for (int it = 0; it < E::ROW_CHUNKS; ++it) {
                int lr, c8;
                row_chunk<C>(it, lr, c8);
                const int r = m0 + h * C::WM + lr, c = n0 + c8;
                cpre[it] = (r < n && c < ld) ? ldg<half8v>(csym + (int64_t)r * ld + c) : half8v{};
            }
        }
        for_rows<C>(acc, smem, h, [&](int it, int half, int lr, int c8, float (&v)[8]) {
            const int r = m0 + half * C::WM + lr, c = n0 + c8;
            if (r >= n || c >= ld) return;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float t = alpha * v[e];
                if (beta != 0.f) t += beta * static_cast<float>(cpre[it][e]);
                if (r == c + e) t += gamma;
                v[e] = t;
            }
            stg_nt<half8v>(out + (int64_t)r * ld + c, to_half8(v));
        });
        if (!mirror) continue;
        if (beta != 0.f) {
#pragma unroll
            for (int it = 0; it < E::COL_CHUNKS; ++it) {
                int cl, lr8;
                col_chunk<C>(it, cl, lr8);
                const int c = n0 + cl, r8 = m0 + h * C::WM + lr8;
                cpre[it] = (c < n && r8 < ld) ? ldg<half8v>(csym + (int64_t)c * ld + r8) : half8v{};
            }
        }
        for_cols<C>(acc, smem, h, [&](int it, int half, int cl, int lr8, float (&v)[8]) {
            const int c = n0 + cl, r8 = m0 + half * C::WM + lr8;   // v[e] is (r8 + e, c)
            if (c >= n || r8 >= ld) return;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float t = alpha * v[e];
                if (beta != 0.f) t += beta * static_cast<float>(cpre[it][e]);
                if (r8 + e == c) t += gamma;
                v[e] = t;
            }
            stg_nt<half8v>(out + (int64_t)c * ld + r8, to_half8(v));
        });
    }
}

// Phase 1: Gram matrix of the short side of iterate `it`.
__global__ __launch_bounds__(256) void ns_gram_kernel(const OrthoMat* __restrict__ mats, TaskList tl, int it) {
    __shared__ __attribute__((aligned(16))) char smem[Epi<NsCfg>::SMEM];
    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int T = (M.s + NsCfg::BM - 1) / NsCfg::BM;
    int ti, tj;
    tri_decode(b - tl.starts[k], T, ti, tj);
    // wide (rows <= cols): A = X X^T, contraction over columns (K-major rows of X);
    // tall: A = X^T X, contraction over rows (MN-major columns of X).
    const Operand A = iterate_operand(M, it);
    floatx16 acc[NsCfg::TM][NsCfg::TN];
    if (M.tall) gemm_mainloop<NsCfg, false, false>(A, A, ti * NsCfg::BM, tj * NsCfg::BN, M.l, acc, smem, M.zero);
    else gemm_mainloop<NsCfg, true, true>(A, A, ti * NsCfg::BM, tj * NsCfg::BN, M.l, acc, smem, M.zero);
    // iteration 0 reads the stored first iterate, which is sigma * u up to the factor x0scale
    const float osc = it == 0 ? M.scal[kScalX0Scale] : 1.f;
    sym_store<NsCfg>(acc, smem, M.gram, nullptr, M.lds, M.s, ti * NsCfg::BM, tj * NsCfg::BN, ti != tj,
                     osc * osc, 0.f, 0.f);
}

// Phase 2: P = a I + b A + c A A (A symmetric, so both operands are K-major rows of A).
__global__ __launch_bounds__(256) void ns_poly_kernel(const OrthoMat* __restrict__ mats, TaskList tl,
                                                      float ca, float cb, float cc) {
    __shared__ __attribute__((aligned(16))) char smem[Epi<NsCfg>::SMEM];
    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int T = (M.s + NsCfg::BM - 1) / NsCfg::BM;
    int ti, tj;
    tri_decode(b - tl.starts[k], T, ti, tj);
    const Operand A = square_operand(M.gram, M);
    floatx16 acc[NsCfg::TM][NsCfg::TN];
    gemm_mainloop<NsCfg, true, true>(A, A, ti * NsCfg::BM, tj * NsCfg::BN, M.s, acc, smem, M.zero);
    sym_store<NsCfg>(acc, smem, M.poly, M.gram, M.lds, M.s, ti * NsCfg::BM, tj * NsCfg::BN, ti != tj,
                     cc, cb, ca);
}

// Phase 3: X' = P X (wide) or X P (tall). Not final: store the f16 iterate. Final: either apply
// the update to p directly (cautious weight decay, thorn.py:669-702) or store u' in f16 with
// per-row sums of squares for the per-row normalization (thorn.py:758-762).
__global__ __launch_bounds__(256) void ns_update_kernel(const OrthoMat* __restrict__ mats, TaskList tl,
                                                        int it, int final_iter) {
    __shared__ __attribute__((aligned(16))) char smem[Epi<NsCfg>::SMEM];
    __shared__ float scratch[4];
    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];
    // column-major tile order: consecutive tiles share the column panel of X and, a few apart,
    // the row panels of P
    const int ti = local % M.g3_tiles_m, tj = local / M.g3_tiles_m;
    const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
    const Operand X = iterate_operand(M, it), P = square_operand(M.poly, M);
    floatx16 acc[NsCfg::TM][NsCfg::TN];
    if (M.tall)   // X P: rows of X (K-major); P symmetric, so column n of P is row n (K-major)
        gemm_mainloop<NsCfg, true, true>(X, P, m0, n0, M.s, acc, smem, M.zero);
    else          // P X: X[k][n] is MN-major
        gemm_mainloop<NsCfg, true, false>(P, X, m0, n0, M.s, acc, smem, M.zero);
    if (it == 0) {   // the stored first iterate is sigma * u up to the factor x0scale
        const float osc = M.scal[kScalX0Scale];
        if (osc != 1.f) {
#pragma unroll
            for (int i = 0; i < NsCfg::TM; ++i)
#pragma unroll
                for (int j = 0; j < NsCfg::TN; ++j) acc[i][j] *= osc;
        }
    }

    if (!final_iter) {
        _Float16* dst = (it & 1) ? M.xb : M.xa;
#pragma unroll 1
        for (int h = 0; h < 2; ++h)
            for_rows<NsCfg>(acc, smem, h, [&](int, int half, int lr, int c8, float (&v)[8]) {
                const int r = m0 + half * NsCfg::WM + lr, c = n0 + c8;
                if (r < M.rows && c < M.ldx) stg_nt<half8v>(dst + (int64_t)r * M.ldx + c, to_half8(v));
            });
        return;
    }

    if (M.flags & kFlagPNN) {
        // u' in f16 (the reference's polar factor is f16 rounded, thorn.py:635, 662) and per-row
        // partial sums of u'^2 over this tile's columns: the 32 lanes of a half-wave cover a row.
#pragma unroll 1
        for (int h = 0; h < 2; ++h)
            for_rows<NsCfg>(acc, smem, h, [&](int, int half, int lr, int c8, float (&v)[8]) {
                const int r = m0 + half * NsCfg::WM + lr, c = n0 + c8;
                const half8v hv = to_half8(v);
                float sq = 0.f;
                if (r < M.rows && c < M.ldx) {
                    stg_nt<half8v>(M.uout + (int64_t)r * M.ldx + c, hv);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float f = static_cast<float>(hv[e]);
                        sq += f * f;
                    }
                }
                sq = halfwave_sum(sq);
                if ((threadIdx.x & 31) == 0 && r < M.rows) stg<float>(M.rowsqpart + (int64_t)tj * M.rows + r, sq);
            });
        return;
    }

    // Direct apply: p <- p - eta * (u + wd * p * [u * p >= 0]) (thorn.py:679-680, 702).
    const bool md = (M.flags & (kFlagMD | kFlagMDScalar)) != 0;
    const bool apply = (M.flags & kFlagApply) != 0;
    const bool vec = (M.flags & kFlagVec4) != 0;
    float psq = 0.f;
#pragma unroll 1
    for (int h = 0; h < 2; ++h)
        for_rows<NsCfg>(acc, smem, h, [&](int, int half, int lr, int c8, float (&v)[8]) {
            const int r = m0 + half * NsCfg::WM + lr, c = n0 + c8;
            if (r >= M.rows || c >= M.cols) return;
            float* pp = M.p + (int64_t)r * M.cols + c;
            if (vec && c + 8 <= M.cols) {
                float4 p0 = ldg<float4>(pp), p1 = ldg<float4>(pp + 4);
                float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (apply) pv[e] = cautious_step(pv[e], (float)(_Float16)v[e], M.eta, M.wd);
                    psq += pv[e] * pv[e];
                }
                if (apply) {
                    stg_nt<float4>(pp, make_float4(pv[0], pv[1], pv[2], pv[3]));
                    stg_nt<float4>(pp + 4, make_float4(pv[4], pv[5], pv[6], pv[7]));
                }
            } else {
                for (int e = 0; e < 8 && c + e < M.cols; ++e) {
                    float p = ldg<float>(pp + e);
                    if (apply) {
                        p = cautious_step(p, (float)(_Float16)v[e], M.eta, M.wd);
                        stg_nt<float>(pp + e, p);
                    }
                    psq += p * p;
                }
            }
        });
    if (md) {
        const float t = block_sum(psq, scratch);
        if (threadIdx.x == 0) M.psqpart[local] = t;
    }
}

}  // namespace thorn
