// Grouped Newton-Schulz phase kernels over an orthogonalized parameter group (gfx950).
//
// Reference semantics: thorn.py:626-662 (_polar_decomp_impl), Gram Newton-Schulz with restarts,
// in f16 with fp32 accumulation. With R the Gram matrix of the short side and
// P_i = a_i I + b_i R + c_i R^2, iteration i multiplies Q by P_i and advances R to P_i R P_i;
// at a restart (and at the end) the iterate is updated, X <- Q X, and R is formed again from it.
// A restart before every iteration is the plain quintic X <- P_i X (thorn.py:655-658). The first
// iterate is u / (||u||_F + 1e-8) rounded to f16 (thorn.py:632-635).
#include "ns_gemm.hpp"
#include "thorn_kernels.hpp"

namespace thorn {

// One tile configuration for every Newton-Schulz GEMM: 256 x 256 tiles, one block per CU.
using NsCfg = GemmCfg<256, 256, 4>;

__device__ __forceinline__ Operand iterate_operand(const OrthoMat& M, int xsel) {
    Operand op;
    op.ptr = xsel == kXA ? M.xa : M.xb;
    op.ld = M.ldx;
    op.rows = M.rows;
    return op;
}

__device__ __forceinline__ _Float16* sym_buf(const OrthoMat& M, int sel) {
    switch (sel) {
        case kBufR: return M.gram;
        case kBufP: return M.poly;
        case kBufQA: return M.qa;
        case kBufQB: return M.qb;
        default: return M.tmp;
    }
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

// Buffer access to an s x ld f16 workspace matrix. Every load and store of the symmetric
// epilogue is a buffer instruction issued unconditionally: a chunk outside the matrix, or one the
// epilogue does not write, gets the offset kOutOfRange, past the resource's size, so the load
// returns zeros and the store is dropped. With no conditional memory operation, the compiler's
// waits count exactly the operations still needed (a conditional one made it wait for every
// outstanding store before each chunk). A null matrix gets a resource of size 0: all zeros.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOutOfRange = 0x80000000u;   // > the byte size of any matrix (s <= 32768)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sym_rsrc(const _Float16* m, int64_t ld, int n) {
    const uint32_t bytes = m ? static_cast<uint32_t>(int64_t(n) * ld * 2) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(m), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ uint32_t sym_off(bool ok, int r, int c, int64_t ld) {
    return ok ? static_cast<uint32_t>((int64_t(r) * ld + c) * 2) : kOutOfRange;
}
__device__ __forceinline__ half8v buf_load8(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_bit_cast(half8v, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0));
}
// aux 2: non-temporal
template <int AUX = 0>
__device__ __forceinline__ void buf_store8(__amdgpu_buffer_rsrc_t rs, uint32_t off, const half8v& v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, static_cast<int>(off), 0, AUX);
}

constexpr int kRowChunks = EpiH<NsCfg>::ROW_ITERS;   // row chunks of a tile per thread

// Csym row chunks first .. first + N - 1 of this thread (zeros outside the matrix).
template <int N>
__device__ __forceinline__ void sym_load(half8v (&cv)[N], __amdgpu_buffer_rsrc_t crs, int64_t ld, int n, int m0,
                                         int n0, int first) {
    const int tr = threadIdx.x >> 5, c8 = (threadIdx.x & 31) * 8;
#pragma unroll
    for (int it = 0; it < N; ++it) {
        const int r = m0 + 8 * (first + it) + tr, c = n0 + c8;
        cv[it] = buf_load8(crs, sym_off(r < n && c < ld, r, c, ld));
    }
}

// out = alpha * acc + beta * Csym + gamma * I (f16) on an upper-triangle tile of a symmetric s x s
// matrix (Csym optional: crs of size 0). Only the upper block triangle is stored: consumers read
// a block below the diagonal as the transpose of its mirror above it, and a diagonal block either
// way, so a diagonal tile must be exactly symmetric (an antisymmetric error in R grows through the
// Gram iteration): its upper triangle is computed and its lower triangle is the mirror.
// With Csym, its tile is first copied into the staging as is; each value is then replaced in
// place by the final value computed from it (the same lane reads and writes each position). On a
// diagonal tile the staging also receives the transposes of the values above the diagonal
// (stage_f16), so one pass of row chunks stores every tile. HAS_C: the Csym term is present (else crs and beta are
// unused); SCALE: alpha != 1 (else the product is stored unscaled, which x * 1 would leave as is).
template <class C, bool HAS_C, bool SCALE>
__device__ __forceinline__ void sym_store(floatx16 (&acc)[C::TM][C::TN], char* smem, _Float16* out,
                                          __amdgpu_buffer_rsrc_t crs, int64_t ld, int n, int m0, int n0,
                                          float alpha, float beta, float gamma) {
    using E = EpiH<C>;
    _Float16* const S = reinterpret_cast<_Float16*>(smem);
    const bool diag = m0 == n0;
    if constexpr (HAS_C) {
        // requested once the main loop is done: held through it, even a part of them would be
        // spilled to scratch memory by the register allocator
        half8v cv[kRowChunks];
        sym_load(cv, crs, ld, n, m0, n0, 0);
        _Float16* const base = S + row_chunk_base();
#pragma unroll
        for (int it = 0; it < kRowChunks; ++it) *reinterpret_cast<half8v*>(base + it * E::ROW_STEP) = cv[it];
        lds_barrier();
    }
    stage_f16<C>(acc, smem, diag, [&](int r, int c, const floatx4& a, bool dblk) {
        floatx4 t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = SCALE ? alpha * a[e] : a[e];
        if constexpr (HAS_C) {
            const half4 cv = *reinterpret_cast<const half4*>(S + E::rowoff(r) + c);
#pragma unroll
            for (int e = 0; e < 4; ++e) t[e] += beta * static_cast<float>(cv[e]);
        }
        if (dblk) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (r == c + e) t[e] += gamma;
        }
        return t;
    });
    lds_barrier();
    {
        // Row pass through a resource over the tile's rows below n: the row offset of a chunk is
        // an add to one per-lane offset, and a lane whose columns lie past ld stores nothing.
        const int rows = n - m0 < C::BM ? n - m0 : C::BM;
        const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
            out + int64_t(m0) * ld, 0, static_cast<int>(rows * ld * 2), 0x00020000);
        const int tr = threadIdx.x >> 5, ck = threadIdx.x & 31;
        const uint32_t vbase = n0 + 8 * ck < ld ? static_cast<uint32_t>((tr * ld + n0 + 8 * ck) * 2) : kOutOfRange;
        const uint32_t rstep = static_cast<uint32_t>(16 * ld);   // bytes of 8 rows
        each_row_chunk_h<C>(smem, [&](int it, int, int, const half8v& h) {
            buf_store8<2>(trs, vbase + it * rstep, h);
        });
    }
}

// One Newton-Schulz operation of a phase launch (see ns_phase_kernel).
enum NsOpKind : int32_t { kOpNone = 0, kOpGram = 1, kOpSym = 2, kOpUpdate = 3 };
struct NsOp {
    int32_t kind;
    int32_t xsel, first, final_iter;   // gram, update: iterate buffer, first-iterate scaling, last update
    int32_t asel, bsel, csel, osel;    // sym: out = alpha * A B + beta * C + gamma * I
    int32_t qsel;                      // update: X <- Q X
    float alpha, beta, gamma;
};

// Epilogue of an update tile (see ns_phase_kernel). Every field of the matrix table it needs is
// read once into a register first: stores through the matrix pointers could alias the table in
// global memory as far as the compiler knows, and it would reload fields after every store.
__device__ __forceinline__ void update_finish(const OrthoMat& M, floatx16 (&acc)[NsCfg::TM][NsCfg::TN], int local,
                                              int ti, int tj, const NsOp& op, char* smem, float* scratch) {
    const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
    const int rows = M.rows, cols = M.cols, ldx = M.ldx, flags = M.flags;
    // the stored first iterate is sigma * u up to the factor x0scale, applied as the first
    // update's tile is staged; every output of the update is the f16 rounding of acc * osc
    const float osc = op.first ? M.scal[kScalX0Scale] : 1.f;

    // The direct apply of a whole tile (every tile of a matrix with 256-multiple sides) streams p
    // through a ring of D row chunks: chunk L is row m0 + 8*L + tid/32, columns n0 + 8*(tid%32)
    // .. +7, requested into slot L % D as soon as chunk L - D has been used, the first D before
    // the tile is staged. Buffer instructions address it as one resource over the tile's rows
    // (scalar registers), a per-lane offset shared by every chunk and a wave-uniform row offset,
    // so no per-chunk address occupies vector registers.
    const bool apply_full = op.final_iter && !(flags & kFlagPNN) && (flags & kFlagVec4) &&
                            m0 + NsCfg::BM <= rows && n0 + NsCfg::BN <= cols;
    constexpr int D = 8;
    constexpr int NC = EpiH<NsCfg>::ROW_ITERS;
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        M.p + ((int64_t)m0 * cols + n0), 0, NsCfg::BM * cols * 4, 0x00020000);
    const int voff = ((threadIdx.x >> 5) * cols + (threadIdx.x & 31) * 8) * 4;
    auto soff = [&](int L) { return 8 * L * cols * 4; };
    float4 ring[D][2];
    auto fetch = [&](int L) {
        ring[L % D][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, voff, soff(L), 0));
        ring[L % D][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, voff + 16, soff(L), 0));
    };
    if (apply_full) {
#pragma unroll
        for (int L = 0; L < D; ++L) fetch(L);
    }

    if (op.first)
        stage_f16<NsCfg>(acc, smem, false, [&](int, int, const floatx4& a, bool) {
            return floatx4{a[0] * osc, a[1] * osc, a[2] * osc, a[3] * osc};
        });
    else
        stage_f16<NsCfg>(acc, smem, false, [](int, int, const floatx4& a, bool) { return a; });
    lds_barrier();

    // The f16 row passes (next iterate, u'): one buffer resource over the tile's rows below
    // `rows`, so a chunk's offset is one per-lane offset plus a uniform row step; a lane whose
    // columns lie past ldx stores nothing.
    const int tr = threadIdx.x >> 5, ck = threadIdx.x & 31;
    const bool col_ok = n0 + 8 * ck < ldx;
    const uint32_t vbase = col_ok ? static_cast<uint32_t>((tr * ldx + n0 + 8 * ck) * 2) : kOutOfRange;
    const uint32_t rstep = static_cast<uint32_t>(16 * ldx);   // bytes of 8 rows
    auto tile_rsrc = [&](_Float16* base) {
        const int trows = rows - m0 < NsCfg::BM ? rows - m0 : NsCfg::BM;
        return __builtin_amdgcn_make_buffer_rsrc(base + int64_t(m0) * ldx, 0, trows * ldx * 2, 0x00020000);
    };

    if (!op.final_iter) {
        const __amdgpu_buffer_rsrc_t drs = tile_rsrc(op.xsel == kXA ? M.xb : M.xa);
        each_row_chunk_h<NsCfg>(smem, [&](int it, int, int, const half8v& h) {
            buf_store8<2>(drs, vbase + it * rstep, h);
        });
        return;
    }

    if (flags & kFlagPNN) {
        // u' in f16 (the reference's polar factor is f16 rounded, thorn.py:635, 662) and per-row
        // partial sums of u'^2 over this tile's columns (consecutive lanes cover a row).
        const __amdgpu_buffer_rsrc_t urs = tile_rsrc(M.uout);
        float* const rowsq = M.rowsqpart + (int64_t)tj * rows;
        // The row sums go through a buffer resource with an out-of-range offset for every lane
        // but a row's last: a conditional store per chunk split the pass into a block per
        // chunk, each a dependent chain of adds and lane moves.
        const __amdgpu_buffer_rsrc_t qrs =
            __builtin_amdgcn_make_buffer_rsrc(rowsq + m0, 0, (rows - m0) * 4, 0x00020000);
        const uint32_t qoff = ck == 31 ? static_cast<uint32_t>(tr * 4) : kOutOfRange;
        each_row_chunk_h<NsCfg>(smem, [&](int it, int lr, int, const half8v& h) {
            buf_store8<2>(urs, vbase + it * rstep, h);
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = static_cast<float>(h[e]);
                t += f * f;
            }
            static_assert(NsCfg::BN / 8 == 32, "one row per 32 lanes (one 8-column chunk per lane)");
            t = sum32_upper(m0 + lr < rows && col_ok ? t : 0.f);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, t), qrs, qoff + it * 32, 0, 0);
        });
        return;
    }

    // Direct apply: p <- p - eta * (u + wd * p * [u * p >= 0]) (thorn.py:679-680, 702).
    const bool md = (flags & (kFlagMD | kFlagMDScalar)) != 0;
    const bool apply = (flags & kFlagApply) != 0;
    const bool vec = (flags & kFlagVec4) != 0;
    // Magma scales the step by the parameter's s, updated on the device by ortho_norm_kernel
    // (thorn.py:1405)
    const float eta = (flags & kFlagMagma) ? M.eta * ldg<float>(M.magma_s) : M.eta, wd = M.wd;
    float* const p = M.p;
    float psq = 0.f;
    auto step8 = [&](float (&pv)[8], const half8v& h) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float q = cautious_step(pv[e], static_cast<float>(h[e]), eta, wd);
            pv[e] = apply ? q : pv[e];
            psq += pv[e] * pv[e];
        }
    };
    if (apply_full) {
        // No memory operation in the pass is conditional, so each wait covers exactly the load
        // it needs.
        each_row_chunk_h<NsCfg>(smem, [&](int L, int, int, const half8v& h) {
            const float4 p0 = ring[L % D][0], p1 = ring[L % D][1];
            float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            step8(pv, h);
            // Stored whether or not the matrix is applied (the launch's task lists hold only
            // applied matrices; otherwise p is written back unchanged). Each of the two stores
            // covers every other 16 bytes: plain stores, which L2 merges into lines.
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, make_float4(pv[0], pv[1], pv[2], pv[3])),
                                                   prs, voff, soff(L), 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, make_float4(pv[4], pv[5], pv[6], pv[7])),
                                                   prs, voff + 16, soff(L), 0);
            if (L + D < NC) fetch(L + D);
            __builtin_amdgcn_sched_barrier(0);   // one chunk at a time: no hoisted LDS reads
        });
    } else {   // edge tiles: each chunk loaded where it is used
        each_row_chunk_h<NsCfg>(smem, [&](int, int lr, int c8, const half8v& h) {
            const int r = m0 + lr, c = n0 + c8;
            if (r >= rows || c >= cols) return;
            float* pp = p + (int64_t)r * cols + c;
            if (vec && c + 8 <= cols) {
                const float4 p0 = ldg<float4>(pp), p1 = ldg<float4>(pp + 4);
                float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                step8(pv, h);
                if (apply) {
                    stg<float4>(pp, make_float4(pv[0], pv[1], pv[2], pv[3]));
                    stg<float4>(pp + 4, make_float4(pv[4], pv[5], pv[6], pv[7]));
                }
            } else {
                for (int e = 0; e < 8 && c + e < cols; ++e) {
                    float x = ldg<float>(pp + e);
                    if (apply) {
                        x = cautious_step(x, static_cast<float>(h[e]), eta, wd);
                        stg<float>(pp + e, x);
                    }
                    psq += x * x;
                }
            }
        });
    }
    if (md) {
        const float t = block_sum(psq, scratch);
        if (threadIdx.x == 0) M.psqpart[local] = t;
    }
}

// A Newton-Schulz phase launch: t0.total blocks run op0 over the tiles of task list t0, the other
// t1.total blocks run op1 over t1, each XCD taking its eighth of the list with the longer tiles
// first (t1_first: t1's; see xcd_split). The two operations belong to disjoint sets of matrices
// (the square ones, on the plain quintic, and the others, on Gram Newton-Schulz), so one launch
// carries a step of each schedule. Each block computes one 256 x 256 tile:
//   Gram (kOpGram): R = X X^T (wide) or X^T X (tall) of the iterate in buffer `xsel`, rows of X
//     read K-major or its columns MN-major; upper-triangle tile number `local`. `first`: the
//     iterate is the stored first iterate, sigma * u up to the factor x0scale.
//   Symmetric product (kOpSym): out = alpha * A B + beta * C + gamma * I over s x s workspace
//     matrices that are symmetric and commute (all are polynomials in the same R), so the product
//     is symmetric: upper-triangle tiles. A's block row ti and B's block row tj (B symmetric: its
//     column is its row); a matrix stored as its upper block triangle is read MN-major (from the
//     transposed mirror block) before its diagonal block. C may be absent (csel < 0).
//   Update (kOpUpdate): X' = Q X (wide) or X Q (tall) with X in buffer `xsel` and Q the workspace
//     matrix `qsel`, output tile number `local` in column-major order (consecutive tiles share
//     the column panel of X and, a few apart, the row panels of Q); Q's blocks before the
//     diagonal block are read transposed from their mirror above it. See update_finish for the
//     epilogue.
// All three run the same main loop (gemm_tile) with per-operation operands and layouts.
__global__ __launch_bounds__(256) void ns_phase_kernel(const OrthoMat* __restrict__ mats, TaskList t0, NsOp op0,
                                                       TaskList t1, NsOp op1, int t1_first) {
    __shared__ __attribute__((aligned(16))) char smem[EpiH<NsCfg>::SMEM];
    __shared__ float scratch[4];
    int b;
    const bool later = t1_first ? xcd_split(blockIdx.x, t1.total, t0.total, b)
                                : xcd_split(blockIdx.x, t0.total, t1.total, b);
    const bool second = t1_first ? !later : later;
    const TaskList& tl = second ? t1 : t0;
    const NsOp& op = second ? op1 : op0;
    if (op.kind == kOpNone) return;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];

    constexpr int KB = NsCfg::BM / NsCfg::BK;   // K tiles per block
    const int KTs = (M.s + NsCfg::BK - 1) / NsCfg::BK;
    int ti, tj, KT, a_k0, b_k0;
    Operand A, B;
    if (op.kind == kOpUpdate) {
        ti = local % M.g3_tiles_m;
        tj = local / M.g3_tiles_m;
        const Operand X = iterate_operand(M, op.xsel), Q = square_operand(sym_buf(M, op.qsel), M);
        KT = KTs;
        if (M.tall) {   // X Q: rows of X (K-major); column n of Q is its row n
            A = X;
            B = Q;
            a_k0 = 0;
            b_k0 = tj * KB;
        } else {        // Q X: X[k][n] is MN-major
            A = Q;
            B = X;
            a_k0 = ti * KB;
            b_k0 = KT;
        }
    } else {
        tri_decode(local, (M.s + NsCfg::BM - 1) / NsCfg::BM, ti, tj);
        if (op.kind == kOpGram) {
            A = B = iterate_operand(M, op.xsel);
            KT = (M.l + NsCfg::BK - 1) / NsCfg::BK;
            a_k0 = b_k0 = M.tall ? KT : 0;   // tall: contraction over rows, MN-major columns of X
        } else {
            A = square_operand(sym_buf(M, op.asel), M);
            B = square_operand(sym_buf(M, op.bsel), M);
            KT = KTs;
            a_k0 = ti * KB;
            b_k0 = tj * KB;
        }
    }
    floatx16 acc[NsCfg::TM][NsCfg::TN];
    gemm_tile<NsCfg>(A, B, ti * NsCfg::BM, tj * NsCfg::BN, KT, a_k0, b_k0, acc, smem, M.zero,
                     op.kind != kOpUpdate && ti == tj);
    if (op.kind == kOpUpdate) {
        update_finish(M, acc, local, ti, tj, op, smem, scratch);
    } else if (op.kind == kOpGram) {
        const __amdgpu_buffer_rsrc_t none = sym_rsrc(nullptr, 0, 0);
        const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
        if (op.first) {
            const float osc = M.scal[kScalX0Scale];
            sym_store<NsCfg, false, true>(acc, smem, M.gram, none, M.lds, M.s, m0, n0, osc * osc, 0.f, 0.f);
        } else {
            sym_store<NsCfg, false, false>(acc, smem, M.gram, none, M.lds, M.s, m0, n0, 1.f, 0.f, 0.f);
        }
    } else {
        const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
        _Float16* const out = sym_buf(M, op.osel);
        if (op.csel >= 0 && op.beta != 0.f) {
            sym_store<NsCfg, true, true>(acc, smem, out, sym_rsrc(sym_buf(M, op.csel), M.lds, M.s), M.lds, M.s, m0,
                                         n0, op.alpha, op.beta, op.gamma);
        } else if (op.alpha != 1.f) {
            sym_store<NsCfg, false, true>(acc, smem, out, sym_rsrc(nullptr, 0, 0), M.lds, M.s, m0, n0, op.alpha, 0.f,
                                          op.gamma);
        } else {
            sym_store<NsCfg, false, false>(acc, smem, out, sym_rsrc(nullptr, 0, 0), M.lds, M.s, m0, n0, 1.f, 0.f,
                                           op.gamma);
        }
    }
}

}  // namespace thorn
