// Bandwidth-bound THORN kernels (gfx950): momentum + first Newton-Schulz iterate, per-matrix
// norms, decoupled-magnitude gains, per-row normalization apply, and the multi-tensor Adam.
//
// Elementwise kernels over a matrix use 16 x 256 tiles: 256 threads, wave w owns rows 4w..4w+3,
// lane l owns columns 4l..4l+3 (float4 path) or l, l+64, l+128, l+192 (scalar path). Partial sums
// are written per tile and reduced later in a fixed order, so every result is bitwise
// reproducible run to run (no float atomics).
#pragma once
#include "thorn_kernels.hpp"

namespace thorn {

constexpr int kTileR = 16, kTileC = 256;

__device__ __forceinline__ int tile_col(int c0, int lane, int e, bool vec) {
    return vec ? c0 + 4 * lane + e : c0 + lane + 64 * e;
}

// ---------------------------------------------------------------------------------------------
// Momentum, decoupled-magnitude pre-step and the first iterate (thorn.py:1376-1397, 890-908)
// ---------------------------------------------------------------------------------------------
//   md:   G = softplus(rg_i) * softplus(cg_j); p /= G; pg = p * g; g *= G
//         rowpart += pg * softplus(cg_j); colpart += pg * softplus(rg_i)
//   magma: magpart += (g*m, g*g, m*m) with the moment before the update (thorn.py:1390-1392)
//   m = m * beta1 + g;  u = g + beta1 * m;  normpart += u^2;  prescaled: xb = f16(u * 2^k)
// With decouple_md, g * G is written back into the gradient (the reference's in-place g.mul_,
// thorn.py:907), which ortho_cast_kernel then reads to rebuild u.
// kFlagAdam (a decouple_md tensor of an Adam group, thorn.py:1702-1711): the Magma statistics use
// the gradient before the gains (the mask comes first there), and the moments take the Adam step,
// m = lerp(m, g, 1 - beta1), v = beta2 v + (1 - beta2) g^2; ortho_adam_apply_kernel moves p.
__global__ __launch_bounds__(256) void ortho_pre_kernel(const OrthoMat* __restrict__ mats, TaskList tl) {
    __shared__ float colred[4][kTileC];
    __shared__ float scratch[12];
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];
    const int tr = local / M.mom_tiles_c, tc = local % M.mom_tiles_c;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = tr * kTileR + wave * 4, c0 = tc * kTileC;
    const bool md = M.flags & kFlagMD, mds = M.flags & kFlagMDScalar;
    const bool vec = M.flags & kFlagVec4;
    const bool presc = M.flags & kFlagPrescaled;   // never with kFlagAdam (no iterate)
    const bool magma = M.flags & kFlagMagma;
    const float prescale = presc ? M.scal[kScalPrescale] : 1.f;
    const float beta1 = M.beta1;
    const int nrows = M.rows - r0;   // rows of this wave's 4 that exist (may be <= 0)
    const bool adam = M.flags & kFlagAdam;
    const float a_w1 = M.adam_w1, a_beta2 = M.adam_beta2, a_w2 = M.adam_w2;

    float spc[4] = {1.f, 1.f, 1.f, 1.f};
    bool cok[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int c = tile_col(c0, lane, e, vec);
        cok[e] = c < M.cols;
        if (md && cok[e]) spc[e] = softplus_f(M.cg[c]);
    }
    const float sp_scalar = mds ? softplus_f(M.rg[0]) : 1.f;

    // all loads of the wave's 4 rows first, so they are in flight together
    float gv[4][4], mv[4][4], pv[4][4], vv[4][4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const int64_t rbase = (int64_t)(r0 + rr) * M.cols;
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[rr][e] = mv[rr][e] = pv[rr][e] = vv[rr][e] = 0.f;
        if (rr >= nrows) continue;
        if (vec) {
            if (cok[0]) {
                const int c = c0 + 4 * lane;
                const float4 g4 = ldg_nt<float4>(M.g + rbase + c), m4 = ldg_nt<float4>(M.m + rbase + c);
                gv[rr][0] = g4.x; gv[rr][1] = g4.y; gv[rr][2] = g4.z; gv[rr][3] = g4.w;
                mv[rr][0] = m4.x; mv[rr][1] = m4.y; mv[rr][2] = m4.z; mv[rr][3] = m4.w;
                if (md || mds) {
                    const float4 p4 = ldg_nt<float4>(M.p + rbase + c);
                    pv[rr][0] = p4.x; pv[rr][1] = p4.y; pv[rr][2] = p4.z; pv[rr][3] = p4.w;
                }
                if (adam) {
                    const float4 v4 = ldg_nt<float4>(M.v + rbase + c);
                    vv[rr][0] = v4.x; vv[rr][1] = v4.y; vv[rr][2] = v4.z; vv[rr][3] = v4.w;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (!cok[e]) continue;
                const int c = tile_col(c0, lane, e, false);
                gv[rr][e] = ldg<float>(M.g + rbase + c);
                mv[rr][e] = ldg<float>(M.m + rbase + c);
                if (md || mds) pv[rr][e] = ldg<float>(M.p + rbase + c);
                if (adam) vv[rr][e] = ldg<float>(M.v + rbase + c);
            }
        }
    }

    float colacc[4] = {0.f, 0.f, 0.f, 0.f};
    float nrm = 0.f;
    MagmaSums ms;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        if (rr >= nrows) break;   // uniform over the wave
        const int row = r0 + rr;
        const float spr = md ? softplus_f(M.rg[row]) : sp_scalar;
        const int64_t rbase = (int64_t)row * M.cols;
        float rowacc = 0.f;
        float xv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (!cok[e]) { xv[e] = 0.f; continue; }
            float g = gv[rr][e];
            if (adam && magma) ms.add(g, mv[rr][e]);   // thorn.py:1702, before the gains
            if (md || mds) {
                const float G = md ? spr * spc[e] : sp_scalar;
                const float p = pv[rr][e] / G;
                const float pg = p * g;
                g = g * G;
                pv[rr][e] = p;
                gv[rr][e] = g;
                rowacc += md ? pg * spc[e] : pg;
                colacc[e] += pg * spr;
            }
            if (adam) {   // thorn.py:876-877
                mv[rr][e] = lerp_torch(mv[rr][e], g, a_w1);
                vv[rr][e] = vv[rr][e] * a_beta2 + a_w2 * g * g;
                xv[e] = 0.f;
                continue;
            }
            if (magma) ms.add(g, mv[rr][e]);
            const float m = mv[rr][e] * beta1 + g;
            mv[rr][e] = m;
            const float u = fmaf(m, beta1, g);
            xv[e] = u;
            nrm += u * u;
        }
        if (md || mds) {
            rowacc = wave_sum(rowacc);
            if (lane == 0) M.rowpart[(int64_t)tc * M.rows + row] = rowacc;
        }
        // first iterate: directly f16(u * 2^k) with the previous step's power of two, or later
        // by ortho_cast_kernel (exact path) once ||u|| is known
        _Float16* hrow = M.xb + (int64_t)row * M.ldx;
        if (vec) {
            if (cok[0]) {
                const int c = c0 + 4 * lane;
                stg_nt<float4>(M.m + rbase + c, make_float4(mv[rr][0], mv[rr][1], mv[rr][2], mv[rr][3]));
                if (md || mds) {
                    stg_nt<float4>(M.p + rbase + c, make_float4(pv[rr][0], pv[rr][1], pv[rr][2], pv[rr][3]));
                    stg<float4>(M.g + rbase + c, make_float4(gv[rr][0], gv[rr][1], gv[rr][2], gv[rr][3]));
                }
                if (adam) stg_nt<float4>(M.v + rbase + c, make_float4(vv[rr][0], vv[rr][1], vv[rr][2], vv[rr][3]));
                if (presc)
                    stg<half4>(hrow + c, half4{(_Float16)(xv[0] * prescale), (_Float16)(xv[1] * prescale),
                                               (_Float16)(xv[2] * prescale), (_Float16)(xv[3] * prescale)});
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (!cok[e]) continue;
                const int c = tile_col(c0, lane, e, false);
                stg_nt<float>(M.m + rbase + c, mv[rr][e]);
                if (md || mds) {
                    stg_nt<float>(M.p + rbase + c, pv[rr][e]);
                    stg<float>(M.g + rbase + c, gv[rr][e]);
                }
                if (adam) stg_nt<float>(M.v + rbase + c, vv[rr][e]);
                if (presc) hrow[c] = (_Float16)(xv[e] * prescale);
            }
        }
    }

    if (md) {
#pragma unroll
        for (int e = 0; e < 4; ++e) colred[wave][tile_col(0, lane, e, vec)] = colacc[e];
        __syncthreads();
        const int c = c0 + threadIdx.x;
        if (c < M.cols) {
            const float t = colred[0][threadIdx.x] + colred[1][threadIdx.x] + colred[2][threadIdx.x] +
                            colred[3][threadIdx.x];
            M.colpart[(int64_t)tr * M.cols + c] = t;
        }
    }
    const float total = block_sum(nrm, scratch);
    if (threadIdx.x == 0) M.normpart[local] = total;
    if (magma) {
        const MagmaSums t = block_sum(ms, scratch);
        if (threadIdx.x == 0) stg<float4>(M.magpart + local, make_float4(t.gm, t.gg, t.mm, 0.f));
    }
}

// ---------------------------------------------------------------------------------------------
// Per matrix: sigma = 1 / (||u||_F + 1e-8) (thorn.py:633) and, with decouple_md, the Adam-atan2
// steps of the gains from d softplus (thorn.py:910-967). The gains' updates only read p*g from
// before the parameter update, so they run here, before Newton-Schulz.
// ---------------------------------------------------------------------------------------------
// Grid: one column of blocks per matrix, kNormSlices deep. Block (i, 0) takes sigma, Magma, the
// row gains and the scalar gain; block (i, g) takes slice g of the column gains (each column's sum
// runs over rows / 16 partials, the long part).
constexpr int kNormSlices = 8;

// ||u||_F^2 of one matrix from its tile partials, summed by threads 0..255 in turn and then across
// their waves; a larger block gets the same sum (its other waves add zeros). Every thread returns it.
__device__ __forceinline__ float norm_partials(const OrthoMat& M, float* scratch) {
    const int ntiles = M.mom_tiles_r * M.mom_tiles_c;
    float s = 0.f;
    if (threadIdx.x < 256)
        for (int t = threadIdx.x; t < ntiles; t += 256) s += M.normpart[t];
    return block_sum(s, scratch);
}

// ||u||_F + 1e-8 from ||u||_F^2 (thorn.py:633)
__device__ __forceinline__ float norm_denom(float s) { return sqrtf(s) + 1e-8f; }

// sigma = 1 / (||u||_F + 1e-8) and the first-iterate scales of one matrix from ||u||_F^2 (one
// thread writes them).
__device__ __forceinline__ void norm_write_scales(const OrthoMat& M, float s) {
    const float denom = norm_denom(s);
    const float sigma = 1.f / denom;
    float x0scale = 1.f, repair = 0.f;
    if (M.flags & kFlagPrescaled) {
        // the stored iterate is u * 2^k; it matches the exact f16(sigma * u) range while 2^k is
        // within a factor 16 of sigma, otherwise ortho_cast_kernel rebuilds it exactly
        const float ratio = M.scal[kScalPrescale] / sigma;
        if (ratio > 16.f || ratio < 0.0625f || !(ratio == ratio)) repair = 1.f;
        else x0scale = sigma / M.scal[kScalPrescale];
    }
    M.scal[kScalSigma] = sigma;
    M.scal[kScalDenom] = denom;
    M.scal[kScalX0Scale] = x0scale;
    M.scal[kScalRepair] = repair;
    // next step's prescale: the power of two nearest sigma (kept when sigma is not finite)
    if (sigma > 0.f && sigma < 3.0e38f) {
        const int e = (int)rintf(log2f(sigma));
        M.scal[kScalPrescale] = ldexpf(1.f, e < -120 ? -120 : (e > 120 ? 120 : e));
    } else if (!(M.scal[kScalPrescale] > 0.f)) {
        M.scal[kScalPrescale] = 1.f;
    }
}

// sigma = 1 / (||u||_F + 1e-8), the first-iterate scales and Magma's s of one matrix.
__device__ __forceinline__ void norm_sigma_magma(const OrthoMat* __restrict__ mats, int n_mats, const OrthoMat& M,
                                                 float* scratch) {
    const float s = norm_partials(M, scratch);
    if (threadIdx.x == 0) norm_write_scales(M, s);

    // Magma (thorn.py:822-830): the first matrix of a parameter reduces the tile sums of all of
    // the parameter's matrices and moves s, which the apply kernels read later in the stream
    if ((M.flags & kFlagMagma) && M.magma_n > 0) {
        MagmaSums t;
        for (int q = 0; q < M.magma_n && (int)blockIdx.x + q < n_mats; ++q) {
            const OrthoMat& Q = mats[blockIdx.x + q];
            const int nt = Q.mom_tiles_r * Q.mom_tiles_c;
            for (int i = threadIdx.x; i < nt; i += 256) t.add(ldg<float4>(Q.magpart + i));
        }
        t = block_sum(t, scratch);
        if (threadIdx.x == 0) magma_update(t, M.magma_s);
    }
}

__global__ __launch_bounds__(256) void ortho_norm_kernel(const OrthoMat* __restrict__ mats, int n_mats) {
    __shared__ float scratch[12];
    const OrthoMat& M = mats[blockIdx.x];
    const int slice = blockIdx.y;
    if (slice == 0) norm_sigma_magma(mats, n_mats, M, scratch);
    // the small-matrix launch's cluster barrier word starts with count 0 (its generation bits may
    // hold any value; this clears them too): the workspace may hold another plan's data
    if (slice == 0 && threadIdx.x == 0 && (M.flags & kFlagSmall)) M.small_bar[0] = 0;

    const bool md = M.flags & kFlagMD, mds = M.flags & kFlagMDScalar;
    if (!(md || mds) || !(M.flags & kFlagApply)) return;
    AdamScalars a;
    a.lr = M.gain_lr; a.wd = 0.f; a.beta2 = M.gain_beta2; a.w1 = M.gain_w1; a.w2 = M.gain_w2;
    a.bc1 = M.gain_bc1; a.bc2 = M.gain_bc2; a.eps = M.gain_eps;
    a.apply = true; a.degenerate = false; a.atan2_mode = M.gain_eps == 0.f;
    if (md) {
        for (int i = threadIdx.x; i < M.rows && slice == 0; i += 256) {
            float t = 0.f;
            for (int c = 0; c < M.mom_tiles_c; ++c) t += M.rowpart[(int64_t)c * M.rows + i];
            float gain = M.rg[i], mo = M.rgm[i], va = M.rgv[i];
            const float grad = t * sigmoid_f(gain);
            adam_elem(gain, grad, mo, va, a);
            M.rg[i] = gain; M.rgm[i] = mo; M.rgv[i] = va;
        }
        const int per = (M.cols + kNormSlices - 1) / kNormSlices;
        const int j1 = min(M.cols, (slice + 1) * per);
        for (int j = slice * per + threadIdx.x; j < j1; j += 256) {
            float t = 0.f;
            for (int r = 0; r < M.mom_tiles_r; ++r) t += M.colpart[(int64_t)r * M.cols + j];
            float gain = M.cg[j], mo = M.cgm[j], va = M.cgv[j];
            const float grad = t * sigmoid_f(gain);
            adam_elem(gain, grad, mo, va, a);
            M.cg[j] = gain; M.cgm[j] = mo; M.cgv[j] = va;
        }
    } else if (slice == 0 && M.gain_n > 0) {
        // one scalar gain per parameter: its first matrix sums the partials of all of them
        // (p_g.sum() over the whole tensor, thorn.py:920) and steps the gain once
        float t = 0.f;
        for (int q = 0; q < M.gain_n && (int)blockIdx.x + q < n_mats; ++q) {
            const OrthoMat& Q = mats[blockIdx.x + q];
            for (int i = threadIdx.x; i < Q.rows; i += 256)
                for (int c = 0; c < Q.mom_tiles_c; ++c) t += Q.rowpart[(int64_t)c * Q.rows + i];
        }
        t = block_sum(t, scratch);
        if (threadIdx.x == 0) {
            float gain = M.rg[0], mo = M.rgm[0], va = M.rgv[0];
            const float grad = t * sigmoid_f(gain);
            adam_elem(gain, grad, mo, va, a);
            M.rg[0] = gain; M.rgm[0] = mo; M.rgv[0] = va;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Per-row normalization (thorn.py:709-766): s_i = rsqrt(max(mean_j u'_ij^2, eps)),
// gamma = ||u'||_F / max(||s * u'||_F, eps); one block per matrix.
// ---------------------------------------------------------------------------------------------
// The last Newton-Schulz update leaves u' (f16) in one of the two iterate buffers, which one
// depending on the schedule: usel[0] for square matrices (plain quintic), usel[1] for the others.
struct UoutSel {
    int32_t sel[2];
};
__device__ __forceinline__ const _Float16* uout_of(const OrthoMat& M, const UoutSel& u) {
    return u.sel[M.s == M.l ? 0 : 1] == kXA ? M.xa : M.xb;
}

// sum_j u'_ij^2 of row i from its partial sums
__device__ __forceinline__ float pnn_row_sum(const OrthoMat& M, int i) {
    float rs = 0.f;
    for (int t = 0; t < M.rowsq_tiles; ++t) rs += M.rowsqpart[(int64_t)t * M.rows + i];
    return rs;
}

// s_i from the row's sum of squares (eps = torch.finfo(p.dtype).eps)
__device__ __forceinline__ float pnn_row_scale(const OrthoMat& M, float rs) {
    const float mean = rs / (float)M.cols;
    return 1.f / sqrtf(fmaxf(mean, M.pnn_eps));
}

// gamma of one matrix, rows taken by threads 0..255 in turn (a larger block gets the same value:
// its other waves add zeros); s_i into out[i] unless out is null (global or LDS memory). Every
// thread returns gamma.
__device__ __forceinline__ float pnn_gamma(const OrthoMat& M, float* scratch, float* out) {
    float tot = 0.f, nw = 0.f;
    if (threadIdx.x < 256)
        for (int i = threadIdx.x; i < M.rows; i += 256) {
            const float rs = pnn_row_sum(M, i);
            const float s = pnn_row_scale(M, rs);
            if (out) out[i] = s;
            tot += rs;
            nw += s * s * rs;
        }
    tot = block_sum(tot, scratch);
    nw = block_sum(nw, scratch);
    return sqrtf(tot) / fmaxf(sqrtf(nw), M.pnn_eps);
}

__global__ __launch_bounds__(256) void ortho_rowstats_kernel(const OrthoMat* __restrict__ mats,
                                                             const int32_t* __restrict__ idx) {
    __shared__ float scratch[4];
    const OrthoMat& M = mats[idx[blockIdx.x]];
    const float gamma = pnn_gamma(M, scratch, M.rowscale);
    if (threadIdx.x == 0) M.scal[kScalGamma] = gamma;
}

// p <- p - eta * cwd((u' * s_i) * gamma) on elementwise tile `local` of a matrix (per-row
// normalized) or p <- p - eta * cwd(u') (another small-path matrix), by 256 threads t256 = 0..255
// in the tile layout; returns this thread's sum of p^2 after the update. scale(row) gives s_i.
template <class RowScale>
__device__ __forceinline__ float pnn_apply_tile(const OrthoMat& M, int local, int t256, const _Float16* uout,
                                                float gamma, RowScale scale) {
    const int tr = local / M.mom_tiles_c, tc = local % M.mom_tiles_c;
    const int lane = t256 & 63, wave = t256 >> 6;
    const int r0 = tr * kTileR + wave * 4, c0 = tc * kTileC;
    const bool pnn = M.flags & kFlagPNN;
    const float eta = (M.flags & kFlagMagma) ? M.eta * ldg<float>(M.magma_s) : M.eta;   // thorn.py:1405
    const bool vec = M.flags & kFlagVec4;
    const int nrows = M.rows - r0;
    float psq = 0.f;
    if (vec) {
        // lane owns columns c .. c+3 of each of the wave's 4 rows; loads first
        const int c = c0 + 4 * lane;
        const bool ok = c < M.cols;
        float4 pv[4];
        half4 uv[4];
        float sv[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            pv[rr] = make_float4(0.f, 0.f, 0.f, 0.f);
            uv[rr] = half4{};
            sv[rr] = 0.f;
            if (rr >= nrows || !ok) continue;
            const int row = r0 + rr;
            pv[rr] = ldg_nt<float4>(M.p + (int64_t)row * M.cols + c);
            uv[rr] = ldg_nt<half4>(uout + (int64_t)row * M.ldx + c);
            sv[rr] = pnn ? scale(row) : 1.f;
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            if (rr >= nrows || !ok) continue;
            float p[4] = {pv[rr].x, pv[rr].y, pv[rr].z, pv[rr].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float u = ((float)uv[rr][e] * sv[rr]) * gamma;
                p[e] = cautious_step(p[e], u, eta, M.wd);
                psq += p[e] * p[e];
            }
            stg_nt<float4>(M.p + (int64_t)(r0 + rr) * M.cols + c, make_float4(p[0], p[1], p[2], p[3]));
        }
    } else {
        for (int rr = 0; rr < 4; ++rr) {
            const int row = r0 + rr;
            if (row >= M.rows) break;
            const float s = pnn ? scale(row) : 1.f;
            const int64_t rbase = (int64_t)row * M.cols;
            const _Float16* urow = uout + (int64_t)row * M.ldx;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = c0 + lane + 64 * e;
                if (c >= M.cols) continue;
                const float u = ((float)urow[c] * s) * gamma;
                const float p = cautious_step(M.p[rbase + c], u, eta, M.wd);
                M.p[rbase + c] = p;
                psq += p * p;
            }
        }
    }
    return psq;
}

// pnn_apply_tile over per-row-normalized matrices and the other small-path matrices (whose u'
// ns_small_kernel leaves in xa), s_i and gamma from ortho_rowstats_kernel, plus p^2 partials for
// md.
__global__ __launch_bounds__(256) void ortho_pnn_apply_kernel(const OrthoMat* __restrict__ mats, TaskList tl,
                                                              UoutSel usel) {
    __shared__ float scratch[4];
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];
    if (!(M.flags & kFlagApply)) return;   // not due this step: p is left as it is
    const float gamma = (M.flags & kFlagPNN) ? M.scal[kScalGamma] : 1.f;
    const _Float16* const uout = (M.flags & kFlagSmall) ? M.xa : uout_of(M, usel);
    const float psq = pnn_apply_tile(M, local, threadIdx.x, uout, gamma,
                                     [&](int row) { return ldg<float>(M.rowscale + row); });
    if (M.flags & (kFlagMD | kFlagMDScalar)) {
        const float t = block_sum(psq, scratch);
        if (threadIdx.x == 0) M.psqpart[local] = t;
    }
}

// ---------------------------------------------------------------------------------------------
// Adam step of the decouple_md tensors of an Adam group (thorn.py:1704-1714, 878-888), after
// ortho_pre_kernel moved m and v and ortho_norm_kernel moved Magma's s: p <- p - lr * cwd(u) with
// u = atan2(m bc1, sqrt(v bc2)) (eps = 0), m bc1 / (sqrt(v bc2) + eps), or m when degenerate;
// p^2 partials for the renormalization (per tile, or per row and column tile with kFlagNormRows).
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ortho_adam_apply_kernel(const OrthoMat* __restrict__ mats, TaskList tl) {
    __shared__ float scratch[4];
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];
    const int tr = local / M.mom_tiles_c, tc = local % M.mom_tiles_c;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = tr * kTileR + wave * 4, c0 = tc * kTileC;
    const bool rows_norm = M.flags & kFlagNormRows;
    AdamScalars a;
    a.lr = (M.flags & kFlagMagma) ? M.eta * ldg<float>(M.magma_s) : M.eta;   // thorn.py:1712
    a.wd = M.wd; a.beta2 = M.adam_beta2; a.w1 = M.adam_w1; a.w2 = M.adam_w2;
    a.bc1 = M.adam_bc1; a.bc2 = M.adam_bc2; a.eps = M.adam_eps;
    a.apply = true;
    a.degenerate = M.flags & kFlagAdamDegen;
    a.atan2_mode = M.adam_eps == 0.f;
    float psq = 0.f;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const int row = r0 + rr;
        if (row >= M.rows) break;   // uniform over the wave
        const int64_t rbase = (int64_t)row * M.cols;
        float rsq = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = c0 + lane + 64 * e;
            if (c >= M.cols) continue;
            float pe = ldg<float>(M.p + rbase + c);
            const float me = ldg<float>(M.m + rbase + c), ve = ldg<float>(M.v + rbase + c);
            float u;
            if (a.degenerate) u = me;
            else if (a.atan2_mode) u = atan2f(me * a.bc1, sqrtf(ve * a.bc2));
            else u = (me * a.bc1) / (sqrtf(ve * a.bc2) + a.eps);
            pe = cautious_step(pe, u, a.lr, a.wd);
            stg<float>(M.p + rbase + c, pe);
            rsq += pe * pe;
        }
        if (rows_norm) {
            const float t = wave_sum(rsq);
            if (lane == 0) M.rowpsq[(int64_t)tc * M.rows + row] = t;
        }
        psq += rsq;
    }
    const float t = block_sum(psq, scratch);
    if (threadIdx.x == 0) M.psqpart[local] = t;
}

// ---------------------------------------------------------------------------------------------
// decouple_md tail (thorn.py:1414-1421, 1716-1721, 969-977): p *= target / (||p|| + 1e-8), then
// p *= softplus(rg_i), p *= softplus(cg_j) with the gains already updated. The norm is the
// matrix's Frobenius norm, or each row's with kFlagNormRows (its factor in rowscale).
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ortho_md_factor_kernel(const OrthoMat* __restrict__ mats,
                                                              const int32_t* __restrict__ idx) {
    __shared__ float scratch[4];
    const OrthoMat& M = mats[idx[blockIdx.x]];
    if (M.flags & kFlagNormRows) {
        for (int r = threadIdx.x; r < M.rows; r += 256) {
            float t = 0.f;
            for (int c = 0; c < M.mom_tiles_c; ++c) t += M.rowpsq[(int64_t)c * M.rows + r];
            M.rowscale[r] = M.target[r] / (sqrtf(t) + 1e-8f);
        }
        return;
    }
    float s = 0.f;
    for (int t = threadIdx.x; t < M.n_psq; t += 256) s += M.psqpart[t];
    s = block_sum(s, scratch);
    if (threadIdx.x == 0) M.scal[kScalMDFactor] = M.target[0] / (sqrtf(s) + 1e-8f);
}

__global__ __launch_bounds__(256) void ortho_md_rescale_kernel(const OrthoMat* __restrict__ mats, TaskList tl) {
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const OrthoMat& M = mats[tl.order[k]];
    const int local = b - tl.starts[k];
    const int tr = local / M.mom_tiles_c, tc = local % M.mom_tiles_c;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = tr * kTileR + wave * 4, c0 = tc * kTileC;
    const bool md = M.flags & kFlagMD;
    const bool apply = M.flags & kFlagApply;
    const bool vec = M.flags & kFlagVec4;
    const bool rows_norm = M.flags & kFlagNormRows;
    const float f = M.scal[kScalMDFactor];
    float spc[4];
    bool cok[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int c = tile_col(c0, lane, e, vec);
        cok[e] = c < M.cols;
        spc[e] = (md && cok[e]) ? softplus_f(M.cg[c]) : 1.f;
    }
    const float sp_scalar = md ? 1.f : softplus_f(M.rg[0]);
    const int nrows = M.rows - r0;
    // the wave's 4 rows are loaded first, so their loads are in flight together
    float pv[4][4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
#pragma unroll
        for (int e = 0; e < 4; ++e) pv[rr][e] = 0.f;
        if (rr >= nrows) continue;
        const int64_t rbase = (int64_t)(r0 + rr) * M.cols;
        if (vec) {
            if (cok[0]) {
                const float4 p4 = ldg_nt<float4>(M.p + rbase + c0 + 4 * lane);
                pv[rr][0] = p4.x; pv[rr][1] = p4.y; pv[rr][2] = p4.z; pv[rr][3] = p4.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (cok[e]) pv[rr][e] = ldg<float>(M.p + rbase + tile_col(c0, lane, e, false));
        }
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        if (rr >= nrows) break;
        const int row = r0 + rr;
        const float spr = md ? softplus_f(M.rg[row]) : sp_scalar;
        const int64_t rbase = (int64_t)row * M.cols;
        const float fr = rows_norm ? M.rowscale[row] : f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float p = pv[rr][e];
            if (apply) p = p * fr;
            p = p * spr;
            if (md) p = p * spc[e];
            pv[rr][e] = p;
        }
        if (vec) {
            if (cok[0]) stg_nt<float4>(M.p + rbase + c0 + 4 * lane, make_float4(pv[rr][0], pv[rr][1], pv[rr][2], pv[rr][3]));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (cok[e]) M.p[rbase + tile_col(c0, lane, e, false)] = pv[rr][e];
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Multi-tensor Adam / Adam-atan2 with cautious weight decay (thorn.py:838-888), 4096 elements
// per block.
// ---------------------------------------------------------------------------------------------
constexpr int kAdamChunk = 4096;

__global__ __launch_bounds__(256) void adam_kernel(const AdamTensor* __restrict__ ts, TaskList tl) {
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const AdamTensor& T = ts[tl.order[k]];
    const int64_t base = (int64_t)(b - tl.starts[k]) * kAdamChunk;
    AdamScalars s;
    s.lr = T.lr; s.wd = T.wd; s.beta2 = T.beta2; s.w1 = T.w1; s.w2 = T.w2;
    s.bc1 = T.bc1; s.bc2 = T.bc2; s.eps = T.eps;
    s.apply = T.flags & kAdamApply;
    if (s.apply && (T.flags & kAdamMagma)) s.lr *= ldg<float>(T.magma_s);   // thorn.py:1712
    s.degenerate = T.flags & kAdamDegenerate;
    s.atan2_mode = T.flags & kAdamAtan2;
    constexpr int Q = kAdamChunk / 1024;
    if ((T.flags & kAdamVec4) && base + kAdamChunk <= T.n) {
        // whole chunk: every thread loads its 4 float4 groups of p, g, m, v before computing
        float4 p4[Q], g4[Q], m4[Q], v4[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int64_t i = base + (int64_t)(q * 256 + threadIdx.x) * 4;
            p4[q] = s.apply ? ldg_nt<float4>(T.p + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            g4[q] = ldg_nt<float4>(T.g + i);
            m4[q] = ldg_nt<float4>(T.m + i);
            v4[q] = ldg_nt<float4>(T.v + i);
        }
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int64_t i = base + (int64_t)(q * 256 + threadIdx.x) * 4;
            adam_elem(p4[q].x, g4[q].x, m4[q].x, v4[q].x, s);
            adam_elem(p4[q].y, g4[q].y, m4[q].y, v4[q].y, s);
            adam_elem(p4[q].z, g4[q].z, m4[q].z, v4[q].z, s);
            adam_elem(p4[q].w, g4[q].w, m4[q].w, v4[q].w, s);
            stg_nt<float4>(T.m + i, m4[q]);
            stg_nt<float4>(T.v + i, v4[q]);
            if (s.apply) stg_nt<float4>(T.p + i, p4[q]);
        }
    } else {
        for (int q = 0; q < kAdamChunk / 256; ++q) {
            const int64_t j = base + q * 256 + threadIdx.x;
            if (j >= T.n) break;
            float p = s.apply ? T.p[j] : 0.f, m = T.m[j], v = T.v[j];
            adam_elem(p, T.g[j], m, v, s);
            T.m[j] = m; T.v[j] = v;
            if (s.apply) T.p[j] = p;
        }
    }
}

// Magma statistics of the Adam tensors (thorn.py:1702): g and the moment before the update, per
// 4096-element chunk (the chunks of adam_kernel), over the tensors of the Magma task list.
__global__ __launch_bounds__(256) void adam_magma_stats_kernel(const AdamTensor* __restrict__ ts, TaskList tl) {
    __shared__ float scratch[12];
    const int b = blockIdx.x;
    const int k = find_task(tl.starts, tl.n, b);
    const AdamTensor& T = ts[tl.order[k]];
    const int local = b - tl.starts[k];
    const int64_t base = (int64_t)local * kAdamChunk;
    MagmaSums ms;
    if ((T.flags & kAdamVec4) && base + kAdamChunk <= T.n) {
#pragma unroll
        for (int q = 0; q < kAdamChunk / 1024; ++q) {
            const int64_t i = base + (int64_t)(q * 256 + threadIdx.x) * 4;
            const float4 g4 = ldg<float4>(T.g + i), m4 = ldg<float4>(T.m + i);
            ms.add(g4.x, m4.x);
            ms.add(g4.y, m4.y);
            ms.add(g4.z, m4.z);
            ms.add(g4.w, m4.w);
        }
    } else {
        for (int q = 0; q < kAdamChunk / 256; ++q) {
            const int64_t j = base + q * 256 + threadIdx.x;
            if (j >= T.n) break;
            ms.add(ldg<float>(T.g + j), ldg<float>(T.m + j));
        }
    }
    const MagmaSums t = block_sum(ms, scratch);
    if (threadIdx.x == 0) stg<float4>(T.magpart + local, make_float4(t.gm, t.gg, t.mm, 0.f));
}

// One block per Magma tensor (order[blockIdx.x]): its chunk sums in order, then s (thorn.py:822-830).
__global__ __launch_bounds__(256) void adam_magma_finalize_kernel(const AdamTensor* __restrict__ ts,
                                                                  const int32_t* __restrict__ order) {
    __shared__ float scratch[12];
    const AdamTensor& T = ts[order[blockIdx.x]];
    const int64_t chunks = (T.n + kAdamChunk - 1) / kAdamChunk;
    MagmaSums t;
    for (int64_t i = threadIdx.x; i < chunks; i += 256) t.add(ldg<float4>(T.magpart + i));
    t = block_sum(t, scratch);
    if (threadIdx.x == 0) magma_update(t, T.magma_s);
}

// Row-sparse Adam (thorn.py:1673-1700): block k updates row rows_idx[k] of p, m, v with gradient
// row k, the same per-element arithmetic as adam_kernel; rows outside [0, rows) are skipped.
struct SparseAdamArgs {
    float* p;
    float* m;
    float* v;
    const float* gv;
    const int64_t* rows_idx;
    int64_t rows, row_len;
    AdamScalars s;
    int32_t vec;   // row_len % 4 == 0 and p, m, v, gv 16-byte aligned
    float* magma_s;     // Magma: state['s'] (lr scaled by it), or null
    float4* magma_work; // Magma: one partial-sum slot per block of adam_sparse_magma_kernel
};

// Magma statistics of a row-sparse gradient (thorn.py:1676-1679): gradient rows against the
// gathered moment rows. Block b takes gradient rows b, b + gridDim.x, ... and writes one partial
// sum; adam_sparse_magma_finalize_kernel reduces the gridDim.x partials in order.
__global__ __launch_bounds__(256) void adam_sparse_magma_kernel(SparseAdamArgs a, int64_t nnz) {
    __shared__ float scratch[12];
    MagmaSums ms;
    for (int64_t k = blockIdx.x; k < nnz; k += gridDim.x) {
        const int64_t r = ldg<int64_t>(a.rows_idx + k);
        if (r < 0 || r >= a.rows) continue;
        const float* g = a.gv + k * a.row_len;
        const float* m = a.m + r * a.row_len;
        if (a.vec) {
            for (int64_t c = (int64_t)threadIdx.x * 4; c < a.row_len; c += 1024) {
                const float4 g4 = ldg<float4>(g + c), m4 = ldg<float4>(m + c);
                ms.add(g4.x, m4.x);
                ms.add(g4.y, m4.y);
                ms.add(g4.z, m4.z);
                ms.add(g4.w, m4.w);
            }
        } else {
            for (int64_t c = threadIdx.x; c < a.row_len; c += 256) ms.add(ldg<float>(g + c), ldg<float>(m + c));
        }
    }
    const MagmaSums t = block_sum(ms, scratch);
    if (threadIdx.x == 0) stg<float4>(a.magma_work + blockIdx.x, make_float4(t.gm, t.gg, t.mm, 0.f));
}

__global__ __launch_bounds__(256) void adam_sparse_magma_finalize_kernel(const float4* __restrict__ part, int n,
                                                                         float* s) {
    __shared__ float scratch[12];
    MagmaSums t;
    for (int i = threadIdx.x; i < n; i += 256) t.add(ldg<float4>(part + i));
    t = block_sum(t, scratch);
    if (threadIdx.x == 0) magma_update(t, s);
}

__global__ __launch_bounds__(256) void adam_sparse_kernel(SparseAdamArgs a) {
    const int64_t k = blockIdx.x;
    const int64_t r = ldg<int64_t>(a.rows_idx + k);
    if (r < 0 || r >= a.rows) return;
    AdamScalars s = a.s;
    if (s.apply && a.magma_s) s.lr *= ldg<float>(a.magma_s);   // thorn.py:1687
    const float* g = a.gv + k * a.row_len;
    float* p = a.p + r * a.row_len;
    float* m = a.m + r * a.row_len;
    float* v = a.v + r * a.row_len;
    if (a.vec) {
        for (int64_t c = (int64_t)threadIdx.x * 4; c < a.row_len; c += 1024) {
            float4 p4 = s.apply ? ldg<float4>(p + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 g4 = ldg<float4>(g + c);
            float4 m4 = ldg<float4>(m + c), v4 = ldg<float4>(v + c);
            adam_elem(p4.x, g4.x, m4.x, v4.x, s);
            adam_elem(p4.y, g4.y, m4.y, v4.y, s);
            adam_elem(p4.z, g4.z, m4.z, v4.z, s);
            adam_elem(p4.w, g4.w, m4.w, v4.w, s);
            stg<float4>(m + c, m4);
            stg<float4>(v + c, v4);
            if (s.apply) stg<float4>(p + c, p4);
        }
    } else {
        for (int64_t c = threadIdx.x; c < a.row_len; c += 256) {
            float pe = s.apply ? p[c] : 0.f, me = m[c], ve = v[c];
            adam_elem(pe, g[c], me, ve, s);
            m[c] = me;
            v[c] = ve;
            if (s.apply) p[c] = pe;
        }
    }
}

}  // namespace thorn
