// Grouped Newton-Schulz phase kernels over an orthogonalized parameter group (gfx950).
//
// Reference semantics: thorn.py:626-662 (_polar_decomp_impl) in f16 with fp32 accumulation, with
// the reference's own recurrences and rounding points: every product is rounded to f16 once, as
// f16(beta * C + alpha * (A B)) (the eager baddbmm), and Q = Z + a I rounds Z first.
//   Gram Newton-Schulz (non-square matrices, thorn.py:637-653), R = X X^T of the short side:
//     for each iteration i: a restart (i in S, i != 0) sets X <- Q X and R <- X X^T;
//     Z = b R + c R R;  Q = Z + a I (i == 0 or a restart) or Q = a Q + Q Z;
//     unless the next iteration restarts or this is the last: RZ = a R + R Z, R = a RZ + Z RZ;
//     at the end X <- Q X.
//   Plain quintic (square matrices, thorn.py:654-658): A = X X^T, B = b A + c A A, X <- a X + B X.
// The first iterate is u / (||u||_F + 1e-8) rounded to f16 (thorn.py:632-635).
#pragma once
#include "ns_gemm.hpp"
#include "thorn_kernels.hpp"

namespace thorn {

// Per-block timestamps of ns_phase_kernel, in a measurement build only (-DTHORN_BLOCK_TIMESTAMPS,
// `python -m thorn_amd.blocksplit`): thread 0 of each block takes a slot and records, with
// s_memrealtime (100 MHz) and s_memtime (shader clock), the block's start [0], its main loop's
// start [1] (gemm_tile, after the prologue's loads are issued and tile 0 has landed), the loop's
// end [2] and the block's end [3] (clock values at 4 + k), its hardware and XCC ids [8] and the
// tile's kind, diagonal or final flag and K tiles [9]. thorn_block_timestamps copies them out.
#ifdef THORN_BLOCK_TIMESTAMPS
constexpr unsigned kTsSlots = 262144;
__device__ unsigned long long g_ts[12 * kTsSlots];
__device__ unsigned int g_ts_n;
__device__ unsigned long long g_ls[2 * 4096];   // per CU: the loop start of its running block
__device__ __forceinline__ unsigned ts_cu() {
    unsigned hw, xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    return ((xcc & 15) << 8) | ((hw >> 8) & 255);
}
__device__ __forceinline__ void ts_loop_start() {
    if (threadIdx.x == 0) {
        const unsigned c = ts_cu();
        g_ls[2 * c] = __builtin_amdgcn_s_memrealtime();
        g_ls[2 * c + 1] = __builtin_amdgcn_s_memtime();
    }
}
__device__ __forceinline__ void ts_mark(unsigned slot, int k) {
    if (threadIdx.x == 0) {
        g_ts[12 * slot + k] = __builtin_amdgcn_s_memrealtime();
        g_ts[12 * slot + 4 + k] = __builtin_amdgcn_s_memtime();
        if (k == 2) {
            const unsigned cu = ts_cu();
            g_ts[12 * slot + 1] = g_ls[2 * cu];
            g_ts[12 * slot + 5] = g_ls[2 * cu + 1];
        }
    }
}
__device__ __forceinline__ unsigned ts_begin() {
    unsigned slot = 0;
    if (threadIdx.x == 0) {
        slot = atomicAdd(&g_ts_n, 1u) % kTsSlots;
        unsigned hw, xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        g_ts[12 * slot + 8] = (unsigned long long)hw | ((unsigned long long)xcc << 32);
    }
    ts_mark(slot, 0);
    return slot;
}
__device__ __forceinline__ void ts_end(unsigned slot, unsigned long long meta) {
    __syncthreads();
    ts_mark(slot, 3);
    if (threadIdx.x == 0) g_ts[12 * slot + 9] = meta;
}
// ns_small_kernel's workgroups: [1] and [2] are the ends of its prologue and of its schedule
__device__ __forceinline__ void ts_point(unsigned slot, int k) {
    if (threadIdx.x == 0) {
        g_ts[12 * slot + k] = __builtin_amdgcn_s_memrealtime();
        g_ts[12 * slot + 4 + k] = __builtin_amdgcn_s_memtime();
    }
}
// ... and per operation q < 64 of its schedule (workgroup slots below kSopSlots): the operation's
// start [0], its products done [1], its stores issued [2] (the barrier follows), and inside the
// product's K loop the first chunk landed in every wave [3] and the loop's end [4]
constexpr unsigned kSopSlots = 4096;
constexpr int kSopWords = 5;
__device__ unsigned long long g_sop[kSopSlots * 64 * kSopWords];
__device__ __forceinline__ void ts_op(unsigned slot, int q, int k) {
    if (threadIdx.x == 0 && slot < kSopSlots && q < 64)
        g_sop[(slot * 64 + q) * kSopWords + k] = __builtin_amdgcn_s_memrealtime();
}
#else
__device__ __forceinline__ void ts_loop_start() {}
__device__ __forceinline__ void ts_mark(unsigned, int) {}
__device__ __forceinline__ unsigned ts_begin() { return 0; }
__device__ __forceinline__ void ts_end(unsigned, unsigned long long) {}
__device__ __forceinline__ void ts_point(unsigned, int) {}
__device__ __forceinline__ void ts_op(unsigned, int, int) {}
#endif

__device__ __forceinline__ Operand iterate_operand(const OrthoMat& M, int xsel) {
    Operand op;
    op.ptr = xsel == kXA ? M.xa : M.xb;
    op.ld = M.ldx;
    op.rows = M.rows;
    op.packed = 0;
    return op;
}

__device__ __forceinline__ _Float16* sym_buf(const OrthoMat& M, int sel) {
    switch (sel) {
        case kBufR: return M.gram;
        case kBufZ: return M.zbuf;
        case kBufQA: return M.qa;
        default: return M.qb;
    }
}

// An s x s workspace matrix (R, Z, QA, QB): its upper block triangle in panels (Operand::packed).
__device__ __forceinline__ Operand square_operand(const _Float16* p, const OrthoMat& M) {
    Operand op;
    op.ptr = p;
    op.ld = M.lds;
    op.rows = M.s;
    op.packed = 1;
    return op;
}

// Buffers of a matrix on the small-matrix path (kFlagSmall; ns_small.hip) inside OrthoMat: sq[i]
// (R, Z, QA, QB, s_p x s_p) at M.small + i * sqe, their transposes after them, then the iterate
// slots xw[2] (s_p x l_p, the wide orientation) and xwt[2] (their transposes); sizes in elements,
// every buffer padded to multiples of 32 with zeros that stay zero.
struct SmallView {
    _Float16* base;
    int sp, lp;          // s and l rounded up to 32
    int64_t sqe, xe;     // elements of an s_p x s_p and of an s_p x l_p buffer
    __device__ __forceinline__ _Float16* sq(int i) const { return base + i * sqe; }
    __device__ __forceinline__ _Float16* sqt(int i) const { return base + (4 + i) * sqe; }
    __device__ __forceinline__ _Float16* xw(int i) const { return base + 8 * sqe + i * xe; }
    __device__ __forceinline__ _Float16* xwt(int i) const { return base + 8 * sqe + (2 + i) * xe; }
};

__device__ __forceinline__ SmallView small_view(const OrthoMat& M) {
    SmallView v;
    v.base = M.small;
    v.sp = (M.s + 31) & ~31;
    v.lp = (M.l + 31) & ~31;
    v.sqe = int64_t(v.sp) * v.sp;
    v.xe = int64_t(v.sp) * v.lp;
    return v;
}

// The padding of a small matrix's first iterate (rows s .. s_p and columns l .. l_p of both
// orientations of slot 0) cleared by threads tid = 0 .. nt-1.
__device__ __forceinline__ void small_x0_padding(const OrthoMat& M, const SmallView& V, int tid, int nt) {
    for (int e = tid; e < (V.sp - M.s) * V.lp; e += nt) {   // rows s .. s_p
        const int i = M.s + e / V.lp, j = e % V.lp;
        V.xw(0)[int64_t(i) * V.lp + j] = _Float16(0.f);
        V.xwt(0)[int64_t(j) * V.sp + i] = _Float16(0.f);
    }
    for (int e = tid; e < M.s * (V.lp - M.l); e += nt) {     // columns l .. l_p
        const int i = e / (V.lp - M.l), j = M.l + e % (V.lp - M.l);
        V.xw(0)[int64_t(i) * V.lp + j] = _Float16(0.f);
        V.xwt(0)[int64_t(j) * V.sp + i] = _Float16(0.f);
    }
}

// Row r, columns c0 + lane + 64 e (e < 4), of a small matrix's first iterate f16(u / denom), u from
// the updated moment and the gradient, straight into both wide orientations of iterate slot 0.
__device__ __forceinline__ void small_x0_row(const OrthoMat& M, const SmallView& V, int r, int c0, int lane,
                                             float denom, float beta1) {
    const int64_t rb = (int64_t)r * M.cols;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int c = c0 + lane + 64 * e;
        if (c >= M.cols) continue;
        const _Float16 x = (_Float16)(fmaf(ldg<float>(M.m + rb + c), beta1, ldg<float>(M.g + rb + c)) / denom);
        const int i = M.tall ? c : r, j = M.tall ? r : c;   // wide (s x l) position
        V.xw(0)[int64_t(i) * V.lp + j] = x;
        V.xwt(0)[int64_t(j) * V.sp + i] = x;
    }
}

// First iterate, exact form (thorn.py:632-635): xb = f16(u / (||u||_F + 1e-8)) with
// u = g + beta1 * m recomputed from the gradient (times the decouple_md gains: ortho_pre_kernel
// writes g back for those matrices, as the reference's g.mul_ does) and the updated moment, the
// same fmaf as ortho_pre_kernel. It runs for the matrices applied this step on the exact path, and
// for prescaled ones whose stored iterate is out of range after a gradient-scale jump
// (kScalRepair). Grid: x strides
// over the 16 x 256 tiles of matrix blockIdx.y; a matrix that needs neither returns at once.
__global__ __launch_bounds__(256) void ortho_cast_kernel(const OrthoMat* __restrict__ mats) {
    const OrthoMat& M = mats[blockIdx.y];
    if ((M.flags & (kFlagAdam | kFlagApply)) != kFlagApply) return;   // no Newton-Schulz this step
    if ((M.flags & kFlagPrescaled) && M.scal[kScalRepair] == 0.f) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ntiles = M.mom_tiles_r * M.mom_tiles_c;
    const float denom = M.scal[kScalDenom], beta1 = M.beta1;
    const bool vec = M.flags & kFlagVec4;
    // The Newton-Schulz products read padding (columns past the matrix up to ld, and for the
    // small path rows and columns up to multiples of 32) and must find zeros there. Every later
    // iterate and product writes its padding from zero-padded inputs, so the first iterate's
    // padding is cleared here: the workspace may hold another plan's data (plans of one group
    // that run in turn on one workspace).
    if (blockIdx.x == 0) {
        if (M.flags & kFlagSmall) {
            small_x0_padding(M, small_view(M), threadIdx.x, 256);
        } else if (M.ldx > M.cols) {
            for (int e = threadIdx.x; e < M.rows * (M.ldx - M.cols); e += 256) {
                const int r = e / (M.ldx - M.cols), c = M.cols + e % (M.ldx - M.cols);
                M.xb[int64_t(r) * M.ldx + c] = _Float16(0.f);
            }
        }
    }
    for (int t = blockIdx.x; t < ntiles; t += gridDim.x) {
        const int tr = t / M.mom_tiles_c, tc = t % M.mom_tiles_c;
        const int r0 = tr * 16 + wave * 4, c0 = tc * 256;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int r = r0 + rr;
            if (r >= M.rows) break;
            const int64_t rb = (int64_t)r * M.cols;
            _Float16* xrow = M.xb + (int64_t)r * M.ldx;
            if (M.flags & kFlagSmall) {
                small_x0_row(M, small_view(M), r, c0, lane, denom, beta1);
            } else if (vec) {
                const int c = c0 + 4 * lane;
                if (c >= M.cols) continue;
                const float4 g4 = ldg<float4>(M.g + rb + c), m4 = ldg<float4>(M.m + rb + c);
                stg<half4>(xrow + c, half4{(_Float16)(fmaf(m4.x, beta1, g4.x) / denom),
                                           (_Float16)(fmaf(m4.y, beta1, g4.y) / denom),
                                           (_Float16)(fmaf(m4.z, beta1, g4.z) / denom),
                                           (_Float16)(fmaf(m4.w, beta1, g4.w) / denom)});
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int c = c0 + lane + 64 * e;
                    if (c < M.cols)
                        xrow[c] = (_Float16)(fmaf(ldg<float>(M.m + rb + c), beta1, ldg<float>(M.g + rb + c)) / denom);
                }
            }
        }
    }
}

// Epilogue stores are buffer instructions issued unconditionally: a chunk outside the matrix gets
// the offset kOutOfRange, past the resource's size, and the store is dropped. With no conditional
// memory operation, the compiler's waits count exactly the operations still needed (a conditional
// one made it wait for every outstanding store before each chunk).
// aux 2: non-temporal
template <int AUX = 0>
__device__ __forceinline__ void buf_store8(__amdgpu_buffer_rsrc_t rs, uint32_t off, const half8v& v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, static_cast<int>(off), 0, AUX);
}

// Row pass: stores the staged f16 tile (rows m0.. below n, columns n0..) into `out` through a
// resource over the tile's rows: the row offset of a chunk is an add to one per-lane offset, and a
// lane whose columns lie past ld stores nothing.
template <class C>
__device__ __forceinline__ void store_staged(const char* smem, _Float16* out, int64_t ld, int n, int m0, int n0) {
    const int rows = n - m0 < C::BM ? n - m0 : C::BM;
    const __amdgpu_buffer_rsrc_t trs =
        __builtin_amdgcn_make_buffer_rsrc(out + int64_t(m0) * ld, 0, static_cast<int>(rows * ld * 2), 0x00020000);
    const int tr = threadIdx.x >> 5, ck = threadIdx.x & 31;
    const uint32_t vbase = n0 + 8 * ck < ld ? static_cast<uint32_t>((tr * ld + n0 + 8 * ck) * 2) : kOutOfRange;
    const uint32_t rstep = static_cast<uint32_t>(EpiH<C>::ROWS * ld * 2);   // bytes of a pass of rows
    each_row_chunk_h<C>(smem, [&](int it, int, int, const half8v& h) { buf_store8<2>(trs, vbase + it * rstep, h); });
}

// out = f16(fma(beta, Csym, alpha * acc)) on an upper-triangle tile of a symmetric s x s matrix
// (Csym optional): one rounding to f16 of beta * C + alpha * (A B), where the reference's eager
// baddbmm rounds it (the fma with an f16 operand is one instruction on gfx950). Only the upper
// block triangle is stored: consumers read a block below the diagonal as the transpose of its
// mirror above it, and a diagonal block either way, so a diagonal tile must be exactly symmetric:
// its upper triangle is computed and its lower triangle is the mirror.
// With Csym, gemm_tile has loaded its tile into the staging (TileC); each value is replaced in
// place by the final value computed from it (the same lane reads and writes each position). On a
// diagonal tile the staging also receives the transposes of the values above the diagonal
// (stage_f16), so one pass of row chunks stores every tile. HAS_C: the Csym term is present (else
// beta is unused); SCALE: alpha != 1 (else the product is stored unscaled, which x * 1 would
// leave as is). DUAL: the tile is also stored to out2 as Q = Z + a I, the diagonal elements
// rounded from the f16 Z (thorn.py:648, `Z + a * I` in f16): f16(float(Z_ii) + dual_add) with
// dual_add = f16(a).
// Where the tile at (m0, n0) of a result goes: its rows [m0, m0 + rows) are rows [0, rows) at ptr,
// column c at ptr column c - c0, row stride ld (a panel of a packed matrix, or the matrix itself
// from row m0 with c0 = 0).
struct TileOut {
    _Float16* ptr;
    int64_t ld;
    int32_t rows, c0;
};

// The tile (ti, tj), tj >= ti, of a packed s x s workspace matrix at base.
__device__ __forceinline__ TileOut packed_out(_Float16* base, const OrthoMat& M, int ti) {
    const SqPanel p = sq_panel(M.s, M.lds, ti);
    return TileOut{base + p.off, p.ld, p.rows, 256 * ti};
}

template <class C, int ROLE, bool HAS_C, bool SCALE, bool DUAL = false>
__device__ __forceinline__ void sym_store(floatx16 (&acc)[RoleMap<ROLE>::N], const TileWork& tw, char* smem,
                                          const TileOut& o, int m0, int n0, float alpha, float beta,
                                          _Float16* out2 = nullptr, float dual_add = 0.f) {
    using E = EpiH<C>;
    const bool diag = m0 == n0;
    stage_f16<C, ROLE>(acc, smem, diag, tw, [&](int r, int c, const floatx4& a) {
        half4 h;
        if constexpr (HAS_C) {
            const half4 cv = *reinterpret_cast<const half4*>(smem + E::off(r, c));
#pragma unroll
            for (int e = 0; e < 4; ++e)
                h[e] = static_cast<_Float16>(fmaf(beta, static_cast<float>(cv[e]), SCALE ? alpha * a[e] : a[e]));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = static_cast<_Float16>(SCALE ? alpha * a[e] : a[e]);
        }
        return h;
    });
    lds_barrier();
    store_staged<C>(smem, o.ptr, o.ld, o.rows, 0, n0 - o.c0);
    if constexpr (DUAL) {
        if (diag) {
            lds_barrier();   // the row pass has read the staging
            const int r = threadIdx.x;   // the diagonal element of row r (threads past 256 have none)
            if (r < C::BM && r < o.rows) {
                _Float16& z = *reinterpret_cast<_Float16*>(smem + E::off(r, r));
                z = static_cast<_Float16>(static_cast<float>(z) + dual_add);
            }
            lds_barrier();
        }
        store_staged<C>(smem, out2, o.ld, o.rows, 0, n0 - o.c0);
    }
}

// One Newton-Schulz operation of a phase launch (see ns_phase_kernel).
enum NsOpKind : int32_t { kOpNone = 0, kOpGram = 1, kOpSym = 2, kOpUpdate = 3 };
struct NsOp {
    int32_t kind;
    int32_t xsel, first, final_iter;   // gram, update: iterate buffer, first-iterate scaling, last update
    int32_t asel, bsel, csel, osel;    // sym: out = f16(alpha * A B + beta * C) (C absent: csel < 0)
    int32_t osel2;                     // sym: >= 0: also Q = out + a I into this buffer (dual_add = f16(a))
    int32_t qsel;                      // update: X <- Q X, or X <- beta X + Q X when csel >= 0
    float alpha, beta, dual_add;
};

// Epilogue of an update tile (see ns_phase_kernel). Every field of the matrix table it needs is
// read once into a register first: stores through the matrix pointers could alias the table in
// global memory as far as the compiler knows, and it would reload fields after every store.
// HAS_C: the plain quintic's X <- a X + B X (thorn.py:658): gemm_tile has staged the tile of the
// input iterate X and each output is f16(fma(beta * osc, X, osc * acc)), one rounding of a X + B X
// as in the reference; otherwise f16(osc * acc).
template <bool HAS_C>
__device__ __forceinline__ void update_finish(const OrthoMat& M, floatx16 (&acc)[RoleMap<kRoleFull>::N],
                                              const TileWork& tw, int local, int ti, int tj, const NsOp& op,
                                              char* smem, float* scratch) {
    const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
    const int rows = M.rows, cols = M.cols, ldx = M.ldx, flags = M.flags;
    // the stored first iterate is sigma * u up to the factor x0scale, applied as the first
    // update's tile is staged; every output of the update is the f16 rounding of acc * osc
    // (plus the X term)
    const float osc = op.first ? M.scal[kScalX0Scale] : 1.f;
    _Float16* const xout = op.xsel == kXA ? M.xb : M.xa;   // the input iterate's tile is in the staging

    // The direct apply of a whole tile (every tile of a matrix with 256-multiple sides) streams p
    // through a ring of D row chunks: chunk L is row m0 + 16*L + tid/32, columns n0 + 8*(tid%32)
    // .. +7, requested into slot L % D as soon as chunk L - D has been used, the first D before
    // the tile is staged. Buffer instructions address it as one resource over the tile's rows
    // (scalar registers), a per-lane offset shared by every chunk and a wave-uniform row offset,
    // so no per-chunk address occupies vector registers.
    const bool apply_full = op.final_iter && !(flags & kFlagPNN) && (flags & kFlagVec4) &&
                            m0 + NsCfg::BM <= rows && n0 + NsCfg::BN <= cols;
    constexpr int NC = EpiH<NsCfg>::ROW_ITERS;
    constexpr int D = 8;
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        M.p + ((int64_t)m0 * cols + n0), 0, NsCfg::BM * cols * 4, 0x00020000);
    const int voff = ((threadIdx.x >> 5) * cols + (threadIdx.x & 31) * 8) * 4;
    auto soff = [&](int L) { return EpiH<NsCfg>::ROWS * L * cols * 4; };
    float4 ring[D][2];
    auto fetch = [&](int L) {
        ring[L % D][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, voff, soff(L), 0));
        ring[L % D][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, voff + 16, soff(L), 0));
    };
    if (apply_full) {
#pragma unroll
        for (int L = 0; L < D; ++L) fetch(L);
    }

    if constexpr (HAS_C) {
        // gemm_tile has loaded the tile of the input iterate X into the staging
        const float bx = op.beta * osc;
        stage_f16<NsCfg, kRoleFull>(acc, smem, false, tw, [&](int r, int c, const floatx4& a) {
            const half4 xv = *reinterpret_cast<const half4*>(smem + EpiH<NsCfg>::off(r, c));
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = static_cast<_Float16>(fmaf(bx, static_cast<float>(xv[e]), osc * a[e]));
            return h;
        });
    } else if (op.first) {
        stage_f16<NsCfg, kRoleFull>(acc, smem, false, tw, [&](int, int, const floatx4& a) {
            return half4{(_Float16)(a[0] * osc), (_Float16)(a[1] * osc), (_Float16)(a[2] * osc), (_Float16)(a[3] * osc)};
        });
    } else {
        stage_f16<NsCfg, kRoleFull>(acc, smem, false, tw, [](int, int, const floatx4& a) {
            return half4{(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3]};
        });
    }
    lds_barrier();

    // The f16 row passes (next iterate, u'): one buffer resource over the tile's rows below
    // `rows`, so a chunk's offset is one per-lane offset plus a uniform row step; a lane whose
    // columns lie past ldx stores nothing.
    const int tr = threadIdx.x >> 5, ck = threadIdx.x & 31;
    const bool col_ok = n0 + 8 * ck < ldx;
    const uint32_t vbase = col_ok ? static_cast<uint32_t>((tr * ldx + n0 + 8 * ck) * 2) : kOutOfRange;
    const uint32_t rstep = static_cast<uint32_t>(EpiH<NsCfg>::ROWS * ldx * 2);   // bytes of a pass of rows
    auto tile_rsrc = [&](_Float16* base) {
        const int trows = rows - m0 < NsCfg::BM ? rows - m0 : NsCfg::BM;
        return __builtin_amdgcn_make_buffer_rsrc(base + int64_t(m0) * ldx, 0, trows * ldx * 2, 0x00020000);
    };

    if (!op.final_iter) {
        const __amdgpu_buffer_rsrc_t drs = tile_rsrc(xout);
        each_row_chunk_h<NsCfg>(smem, [&](int it, int, int, const half8v& h) {
            buf_store8<2>(drs, vbase + it * rstep, h);
        });
        return;
    }

    if (flags & kFlagPNN) {
        // u' in f16 into the iterate buffer this update does not read (the reference's polar
        // factor is f16 rounded, thorn.py:635, 662) and per-row
        // partial sums of u'^2 over this tile's columns (consecutive lanes cover a row).
        const __amdgpu_buffer_rsrc_t urs = tile_rsrc(xout);
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
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, t), qrs, qoff + it * EpiH<NsCfg>::ROWS * 4,
                                                  0, 0);
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
            // Two wait states before any VALU writes the data registers of these 16-byte stores
            // (gfx950 needs them after a store of more than 8 bytes). The compiler inserts them
            // itself, but it counts the scheduling barrier below as one: measured, a VALU write
            // right after the second store corrupted its first element.
            asm volatile("s_nop 1");
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

// A Gram or symmetric-product tile (see ns_phase_kernel) in this wave's role: the main loop, then
// the store of the upper-triangle tile (with its mirror on a diagonal tile).
template <int ROLE>
__device__ __forceinline__ void sym_tile(const OrthoMat& M, const NsOp& op, const Operand& A, const Operand& B, int m0,
                                         int n0, int KT, int a_k0, int b_k0, const TileC& ct, const TileWork& tw,
                                         char* smem, unsigned tslot) {
    floatx16 acc[RoleMap<ROLE>::N];
    gemm_tile<NsCfg, ROLE>(A, B, m0, n0, KT, a_k0, b_k0, ct, tw, acc, smem);
    ts_mark(tslot, 2);
    const int ti = m0 / NsCfg::BM;
    if (op.kind == kOpGram) {
        const TileOut o = packed_out(M.gram, M, ti);
        if (op.first) {
            const float osc = M.scal[kScalX0Scale];
            sym_store<NsCfg, ROLE, false, true>(acc, tw, smem, o, m0, n0, osc * osc, 0.f);
        } else {
            sym_store<NsCfg, ROLE, false, false>(acc, tw, smem, o, m0, n0, 1.f, 0.f);
        }
        return;
    }
    const TileOut o = packed_out(sym_buf(M, op.osel), M, ti);
    if (op.csel >= 0) {
        if (op.osel2 >= 0)
            sym_store<NsCfg, ROLE, true, true, true>(acc, tw, smem, o, m0, n0, op.alpha, op.beta,
                                                     packed_out(sym_buf(M, op.osel2), M, ti).ptr, op.dual_add);
        else if (op.alpha != 1.f)
            sym_store<NsCfg, ROLE, true, true>(acc, tw, smem, o, m0, n0, op.alpha, op.beta);
        else
            sym_store<NsCfg, ROLE, true, false>(acc, tw, smem, o, m0, n0, 1.f, op.beta);
    } else if (op.alpha != 1.f) {
        sym_store<NsCfg, ROLE, false, true>(acc, tw, smem, o, m0, n0, op.alpha, 0.f);
    } else {
        sym_store<NsCfg, ROLE, false, false>(acc, tw, smem, o, m0, n0, 1.f, 0.f);
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
//   Symmetric product (kOpSym): out = f16(alpha * A B + beta * C) over s x s workspace matrices
//     that are symmetric and commute (all are polynomials in the same R), so the product is
//     symmetric: upper-triangle tiles. A's block row ti and B's block row tj (B symmetric: its
//     column is its row); a matrix stored as its upper block triangle is read MN-major (from the
//     transposed mirror block) before its diagonal block. C may be absent (csel < 0). With
//     osel2 >= 0 the tile is also stored as Q = out + a I (Gram Newton-Schulz after a restart).
//   Update (kOpUpdate): X' = Q X (wide) or X Q (tall) with X in buffer `xsel` and Q the workspace
//     matrix `qsel`, plus beta X when csel >= 0 (the plain quintic's a X + B X); output tile
//     number `local` in column-major order (consecutive tiles share the column panel of X and, a
//     few apart, the row panels of Q); Q's blocks before the diagonal block are read transposed
//     from their mirror above it. The output goes to the other iterate buffer. See update_finish
//     for the epilogue.
// All three run the same main loop (gemm_tile) with per-operation operands and layouts.
__global__ __launch_bounds__(NsCfg::NT) void ns_phase_kernel(const OrthoMat* __restrict__ mats, TaskList t0, NsOp op0,
                                                       TaskList t1, NsOp op1, int t1_first) {
    __shared__ __attribute__((aligned(16))) char smem[EpiH<NsCfg>::SMEM];
    float* const scratch = reinterpret_cast<float*>(smem + EpiH<NsCfg>::FREE);   // block sums after the row pass
    int b;
    const bool later = t1_first ? xcd_split(blockIdx.x, t1.total, t0.total, b)
                                : xcd_split(blockIdx.x, t0.total, t1.total, b);
    const bool second = t1_first ? !later : later;
    const TaskList& tl = second ? t1 : t0;
    const NsOp& op = second ? op1 : op0;
    if (op.kind == kOpNone) return;
    const unsigned slot = ts_begin();
    const int2 task = *reinterpret_cast<const int2*>(tl.map + 2 * b);   // matrix, tile within it
    const OrthoMat& M = mats[task.x];
    const int local = task.y;

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
    // the epilogue's C term, loaded by gemm_tile into the staging: the input iterate's tile for the
    // plain quintic's X <- a X + B X, Csym for a symmetric product
    TileC ct{nullptr, 0, 0, 0, 0};
    if (op.csel >= 0) {
        if (op.kind == kOpUpdate) {
            ct = TileC{op.xsel == kXA ? M.xa : M.xb, M.ldx, M.rows, 0, 0};
        } else if (op.kind == kOpSym) {   // tile (ti, tj) of a packed matrix: in panel ti
            const SqPanel p = sq_panel(M.s, M.lds, ti);
            ct = TileC{sym_buf(M, op.csel) + p.off, p.ld, p.rows, ti * NsCfg::BM, ti * NsCfg::BM};
        }
    }
    const int m0 = ti * NsCfg::BM, n0 = tj * NsCfg::BN;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    if (op.kind == kOpUpdate) {
        const TileWork tw(false, wave);
        floatx16 acc[RoleMap<kRoleFull>::N];
        gemm_tile<NsCfg, kRoleFull>(A, B, m0, n0, KT, a_k0, b_k0, ct, tw, acc, smem);
        ts_mark(slot, 2);
        if (op.csel >= 0) update_finish<true>(M, acc, tw, local, ti, tj, op, smem, scratch);
        else update_finish<false>(M, acc, tw, local, ti, tj, op, smem, scratch);
        ts_end(slot, (unsigned long long)(op.kind | (op.final_iter << 4) | (KT << 8)) |
                         ((unsigned long long)blockIdx.x << 32));
        return;
    }
    const TileWork tw(ti == tj, wave);
    switch (tw.role) {
        case kRoleFull: sym_tile<kRoleFull>(M, op, A, B, m0, n0, KT, a_k0, b_k0, ct, tw, smem, slot); break;
        case kRoleDiagA: sym_tile<kRoleDiagA>(M, op, A, B, m0, n0, KT, a_k0, b_k0, ct, tw, smem, slot); break;
        case kRoleDiagB: sym_tile<kRoleDiagB>(M, op, A, B, m0, n0, KT, a_k0, b_k0, ct, tw, smem, slot); break;
        default: sym_tile<kRoleHalf>(M, op, A, B, m0, n0, KT, a_k0, b_k0, ct, tw, smem, slot); break;
    }
    ts_end(slot, (unsigned long long)(op.kind | ((ti == tj) << 4) | (KT << 8)) | ((unsigned long long)blockIdx.x << 32));
}

}  // namespace thorn
