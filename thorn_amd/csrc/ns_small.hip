// Newton-Schulz for small matrices (short side s <= 256): one launch runs the whole schedule of
// every small matrix of a group (gfx950).
//
// The grouped 256 x 256-tile launches of ns_kernels.hip give a small matrix one tile per phase, so
// its 18 phases cost 18 launch latencies. Here each small matrix gets a cluster of 1024-thread
// workgroups (one for s <= 128; above, enough for its s x s products in 64 x 64 super-tiles and
// its s x l updates in 128 x 128 ones to take one round each, at most 16), placed on one XCD
// (block map), that runs every operation of the schedule in turn, 32 x 32 output tiles
// dealt to its 16 * C waves, with a barrier between operations (SmallSync). The
// operands stay in the L2-resident workspace, each s x s result and each iterate also stored
// transposed, so that every MFMA fragment, of A or of B, is one 16-byte load of a K-contiguous row.
// Products are computed whole (no mirroring of a symmetric result), and every output is rounded to
// f16 once from f16(beta C + alpha A B), as the reference's eager baddbmm does (thorn.py:338-343),
// so on small matrices the iteration tracks the reference's f16 trajectory closely.
//
// Workspace of a small matrix (all f16, padded to multiples of 32 with zeros that stay zero):
//   xw[2], xwt[2]: the iterate in the wide orientation (s_p x l_p) and transposed (l_p x s_p),
//     two slots; the iterate of a tall parameter is the transpose of its rows (thorn.py:629-630);
//   sq[4], sqt[4]: R, Z, QA, QB (s_p x s_p) and their transposes.
// The first iterate is written into xw[0] and xwt[0] by ortho_cast_kernel;
// u' goes to xa in the parameter's orientation, with the per-row partial sums of u'^2 that the
// per-row normalization needs.
//
// A plan whose matrices all take this path (none with decouple_md, Magma or an Adam step, every
// one applied this step) runs its whole step as ns_small_kernel<true>: each cluster also does, for
// its own matrix, the work of ortho_pre_kernel (momentum, tile partials of ||u||^2),
// ortho_norm_kernel (the norm) and ortho_cast_kernel (the first iterate) before the schedule, and
// of ortho_rowstats_kernel and ortho_pnn_apply_kernel (the update of p) after it: one launch in
// place of six, two more cluster barriers. The elementwise parts keep those kernels' 16 x 256
// tiles, thread layouts and summation orders (each 256-thread quarter of a workgroup takes one
// tile at a time; the norm, the row statistics and the apply are the same device functions), so
// every value is bit for bit the one the separate launches give.
#include "ns_kernels.hip"
#include "update_kernels.hip"

namespace thorn {

constexpr int kSmallMaxS = 256;        // short side of the matrices this path takes
constexpr int kSmallMaxOps = 64;       // operations per schedule
constexpr int kSmallThreads = 1024;    // 16 waves per workgroup
constexpr int kSmallWaves = kSmallThreads / 64;

struct SmallOp {
    int8_t kind;     // kOpGram, kOpSym, kOpUpdate
    int8_t a, b, c;  // sym: A, B, C buffers (c < 0: none); update: a = Q buffer, c >= 0: + beta X
    int8_t o, o2;    // sym: output buffer, dual output (Q = out + dual I) or -1
    int8_t xsel;     // gram, update: iterate slot read (the update writes the other one)
    int8_t fin;      // update: the last one (writes u')
    float alpha, beta, dual;
};

struct SmallSchedule {
    SmallOp op[2][kSmallMaxOps];   // [0] square matrices (plain quintic), [1] the others (Gram)
    int32_t n[2];
};

// Barrier of the C workgroups of one matrix, on one word of the workspace: the arrival count in
// bits 0-15 and the generation in bits 16-31. A member arrives by adding 1 and learns the
// generation from the value it gets back; the last one to arrive (count C - 1 before its add) adds
// 2^16 - C, which clears the count and advances the generation in one atomic, and the others poll
// the word until the generation moves. Agent-scope release on arrival and acquire on departure.
// The wait is bounded: a cluster whose members are not all resident cannot hang the GPU; after
// `spin` polls (each a 64-cycle sleep) it sets *err and goes on. Should a member that gave up
// waiting arrive at the next barrier first, its arrival stays in the count (the last arrival
// subtracts C, it does not store 0), so every launch, whose members each arrive once at every
// barrier, leaves the count at 0.
__device__ __forceinline__ bool cluster_last(unsigned old, int C) { return (old & 0xFFFFu) == unsigned(C - 1); }
__device__ __forceinline__ void cluster_poll(unsigned* w, unsigned old, int* err, int spin) {
    int it = 0;
    while ((__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 16) == (old >> 16)) {
        if (it++ >= spin) {
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ void cluster_barrier(int* bar, int C, int* err, int spin) {
    __syncthreads();
    if (C > 1 && threadIdx.x == 0) {
        unsigned* w = reinterpret_cast<unsigned*>(bar);
        const unsigned old = __hip_atomic_fetch_add(w, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (cluster_last(old, C)) {
            __hip_atomic_fetch_add(w, (1u << 16) - unsigned(C), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            cluster_poll(w, old, err, spin);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
    }
    __syncthreads();
}

// The same barrier for a cluster whose workgroups all run on one XCD, so that they share its L2,
// which is then the point where their stores meet: each wave's stores are complete in the L2
// before the arrival (vmcnt(0)), and after the departure the caches between the CU and the L2
// are invalidated together with the L2's clean lines (buffer_inv sc1), so the loads that follow
// read what the other members stored. The L2 is not written back (buffer_wbl2 sc1), as the
// agent-scope barrier does it for other XCDs. (Invalidating the CU's L1 alone, buffer_inv sc0, as
// LLVM's gfx942 model does for a workgroup split over CUs, left stale operands in one sequence
// whose members shared the XCD but not a shader engine.) The word is accessed exactly as there
// (the same atomics and polling loads).
__device__ __forceinline__ void cluster_barrier_xcd(int* bar, int C, int* err, int spin) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (C > 1 && threadIdx.x == 0) {
        unsigned* w = reinterpret_cast<unsigned*>(bar);
        const unsigned old = __hip_atomic_fetch_add(w, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (cluster_last(old, C))
            __hip_atomic_fetch_add(w, (1u << 16) - unsigned(C), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            cluster_poll(w, old, err, spin);
        asm volatile("buffer_inv sc1\n\ts_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
}

// The XCD (XCC) this workgroup runs on.
__device__ __forceinline__ int xcc_id() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return static_cast<int>(x & 0xF);
}

// A cluster's barriers. At the start each member stores its XCC id in the barrier's words; the
// first barrier is agent scope, after which each member reads all the ids, and when they are equal
// (the launch placed the cluster on one XCD: block b runs on XCD b mod 8 up to a fixed offset, and
// the block map gives a cluster's members one residue) every later barrier is the XCD-local one.
// The placement is a dispatch order, not a guarantee, so the ids decide: with members on two XCDs
// every barrier stays agent scope. (The ids ride on the first barrier the kernel needs anyway; a
// barrier of their own at the start cost one more agent-scope round.)
struct SmallSync {
    int* bar;   // the barrier word, an unused word, then one XCC id per member
    int* err;
    int C, spin;
    bool local, ids;   // ids: the XCC ids are read after the next (agent-scope) barrier
    // xcd: XCD-local barriers allowed (thorn_ortho_set_small_xcd_barriers; with 0 every barrier is
    // agent scope)
    __device__ __forceinline__ SmallSync(int* bar_, int member, int C_, int* err_, int spin_, bool xcd)
        : bar(bar_), err(err_), C(C_), spin(spin_), local(false), ids(C_ > 1 && xcd) {
        if (ids && threadIdx.x == 0) bar[2 + member] = xcc_id();
    }
    __device__ __forceinline__ void wait() {
        if (local) {
            cluster_barrier_xcd(bar, C, err, spin);
            return;
        }
        cluster_barrier(bar, C, err, spin);
        if (ids) {
            bool same = true;
            for (int i = 1; i < C; ++i) same = same && bar[2 + i] == bar[2];
            local = __builtin_amdgcn_readfirstlane(same ? 1 : 0) != 0;
            ids = false;
        }
    }
};
constexpr int kSmallBarWords = 2 + 16;   // the largest cluster has 16 members

// Operand panels in LDS: a super-tile of up to 128 x 128 outputs (up to 16 tiles of 32 x 32, one
// per wave) is computed from K chunks of 32: rows [M0, M0+SM) of A and [N0, N0+SN) of BT, 64
// bytes each, in the K-major stage layout of the large-matrix GEMM (chunk c of row r at
// r * 64 + (c ^ ((r >> 2) & 3)) * 16: 16 lanes reading rows r..r+15 at one chunk cover all banks).
// A ring of kSmallStages stages is filled by direct global-to-LDS loads, one 1 KB load per wave
// per chunk (its 64 lanes fill 64 consecutive 16-byte slots: lane slot s holds the chunk whose
// swizzled position is s), kSmallStages - 1 chunks ahead of the MFMAs. Two chunks in flight are
// as fast as three (5.4 against 5.5 us per 256 x 256 x 256 product), and seven are slower (6.7 us):
// the loop's time per chunk follows the LDS traffic of its 16 waves' fragment reads (64 KB per
// chunk for a 128 x 128 super-tile) more than the loads' latency. Between products the ring holds
// the waves' epilogue staging tiles (and, in the fused step, the first iterate's transposes).
constexpr int kSmallStages = 3;
constexpr int kSmallStageBytes = 2 * 128 * 64;   // A rows [0, 128), then BT rows [0, 128)

// This wave's direct loads except the newest n (0 <= n <= kSmallStages - 2, wave-uniform) are
// complete, then the block barrier.
__device__ __forceinline__ void wait_loads_barrier(int n) {
    switch (n) {
        case 0: asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(1)\n\ts_barrier" ::: "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(2)\n\ts_barrier" ::: "memory"); break;
        case 3: asm volatile("s_waitcnt vmcnt(3)\n\ts_barrier" ::: "memory"); break;
        case 4: asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory"); break;
        case 5: asm volatile("s_waitcnt vmcnt(5)\n\ts_barrier" ::: "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory"); break;
    }
}
static_assert(kSmallStages - 2 <= 6, "wait_loads_barrier covers 0 .. kSmallStages - 2");

// The C term of a wave's tile in LDS (kCTileBytes per wave): its 32 rows of C^T (rows n0..,
// columns m0..m0+31), 64 bytes each, chunk c of row r at r * 64 + (c ^ ((r >> 2) & 3)) * 16,
// filled by two direct loads (the 64 lanes of each fill 64 consecutive 16-byte slots); `ok` false
// loads `zero` instead. Requested just before the product's first chunks (eight-byte loads of the
// C^T rows into registers, 32 rows per instruction, had taken ~0.7 us more than the chunk alone;
// these two cost the first chunk little, and issued after the chunks they were still in flight
// when a short K loop ended).
constexpr int kCTileBytes = 32 * 64;
__device__ __forceinline__ void small_issue_c(uint32_t lds, const _Float16* CT, int64_t ldc, int m0, int n0, bool ok,
                                              const void* zero, int lane) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r = 16 * h + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
        const void* p = ok ? static_cast<const void*>(CT + int64_t(n0 + r) * ldc + m0 + 8 * c) : zero;
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"((const THORN_GLOBAL void*)p),
                     "{m0}"(lds + h * 1024)
                     : "memory");
    }
}

// This lane's C values of its tile from the LDS copy, in the accumulator layout: cv[g][e] is
// C[m0 + 8g + 4(lane / 32) + e][n0 + lane % 32].
__device__ __forceinline__ void small_read_c(half4 (&cv)[4], const char* ctile, int lane) {
    const int j = lane & 31;
#pragma unroll
    for (int g = 0; g < 4; ++g)
        cv[g] = *reinterpret_cast<const half4*>(ctile + j * 64 + ((g ^ ((j >> 2) & 3)) << 4) + 8 * (lane >> 5));
}

// acc (this wave's tile of the super-tile, if it has one) = A[M0.., 0:K] * B[0:K, N0..] with A
// row-major (lda) and B given by its transpose BT row-major (ldb), K a multiple of 32, every
// operand row inside the padded buffers (rows past sm / sn read `zero`). With CT, the wave's C
// tile (CT at m0, n0) is also loaded into `ctile` (small_issue_c). The whole workgroup calls it
// (barriers inside; the first one orders it after every wave's use of the staging tiles in the
// ring); on return every load has landed and the stages are free.
__device__ __forceinline__ floatx16 small_block(char* stages, const void* zero, const _Float16* A, int64_t lda,
                                                const _Float16* BT, int64_t ldb, int M0, int N0, int sm, int sn,
                                                int K, int wave, int lane, bool has_tile, int ti, int tj,
                                                uint32_t ctile, const _Float16* CT, int64_t ldc, int m0, int n0,
                                                unsigned tslot = 0, int q = 0) {
    floatx16 acc = {};
    const int nk = K / 32;
    const int slot = wave * 64 + lane, part = slot >> 9, r = (slot >> 2) & 127;
    const int c = (slot & 3) ^ ((r >> 2) & 3);
    const bool ok = part == 0 ? r < sm : r < sn;
    // a wave whose 16 rows all lie past sm / sn (an edge super-tile) loads nothing: its waits then
    // pass at once
    const bool loads = 16 * (wave & 7) < (part == 0 ? sm : sn);
    const char* src = reinterpret_cast<const char*>(part == 0 ? A + int64_t(M0 + r) * lda : BT + int64_t(N0 + r) * ldb) +
                      16 * c;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(stages)) + wave * 1024;
    auto issue = [&](int t) {
        if (!loads) return;
        const void* p = ok ? static_cast<const void*>(src + int64_t(t) * 64) : zero;
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"((const THORN_GLOBAL void*)p),
                     "{m0}"(lds0 + (t % kSmallStages) * kSmallStageBytes)
                     : "memory");
    };
    __syncthreads();
    // the C loads first: they return before chunk 0 (loads return in order), so no wait covers
    // them alone
    if (CT) small_issue_c(ctile, CT, ldc, m0, n0, has_tile, zero, lane);
    const int pre = nk < kSmallStages - 1 ? nk : kSmallStages - 1;
    for (int t = 0; t < pre; ++t) issue(t);
    for (int kc = 0; kc < nk; ++kc) {
        // this wave's loads of chunk kc have landed (the ones issued after it may still be in
        // flight); after the barrier every wave's have, and nobody reads stage (kc - 1) % S any
        // more, which then receives chunk kc + S - 1
        const int ahead = nk - 1 - kc < kSmallStages - 2 ? nk - 1 - kc : kSmallStages - 2;
        wait_loads_barrier(ahead);
        if (kc == 0) ts_op(tslot, q, 3);
        if (kc + kSmallStages - 1 < nk) issue(kc + kSmallStages - 1);
        if (has_tile) {
            const char* st = stages + (kc % kSmallStages) * kSmallStageBytes;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8 a = frag<128, true>(st, 32 * ti, ks, lane);
                const half8 b = frag<128, true>(st + kSmallStageBytes / 2, 32 * tj, ks, lane);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
            }
        }
    }
    ts_op(tslot, q, 4);
    __syncthreads();   // every wave is done with the stages (the last wait was vmcnt(0): the C loads too)
    return acc;
}

// The wave's 32 x 32 f16 staging tile: row-major, rows of 34 halves.
constexpr int kStageLd = 34;

// Lanes of one wave hand values to each other through the staging tile: every LDS access before
// this point is complete, and (a compiler memory barrier) none is moved across it or served from
// a value loaded before it. Without it the compiler may reuse a value it already loaded, since a
// write by another lane is not visible to a single thread's program order.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Stages f16(alpha * acc + beta * C) of tile (m0, n0), C from small_read_c (HAS_C).
template <bool HAS_C>
__device__ __forceinline__ void small_stage(const floatx16& acc, _Float16* stage, float alpha, float beta,
                                            const half4 (&cv)[4], int lane) {
    const int j = lane & 31;
    wave_lds_sync();   // the previous tile's reads of the staging are done
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int i0 = 8 * g + 4 * (lane >> 5);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float t = alpha * acc[4 * g + e];
            if (HAS_C) t += beta * static_cast<float>(cv[g][e]);
            stage[(i0 + e) * kStageLd + j] = static_cast<_Float16>(t);
        }
    }
    wave_lds_sync();   // the whole tile is staged before any lane reads it
}

// Stores the staged tile to out (row-major, ld) at (m0, n0) and its transpose to outT (ldt) at
// (n0, m0): 16-byte chunks, 2 + 2 per lane. Tiles lie inside the padded buffers.
__device__ __forceinline__ void small_store(const _Float16* stage, _Float16* out, int64_t ld, _Float16* outT,
                                            int64_t ldt, int m0, int n0, int lane) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int ch = lane + 64 * q, r = ch >> 2, c8 = (ch & 3) * 8;
        half8 h, t;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h[e] = stage[r * kStageLd + c8 + e];
            t[e] = stage[(c8 + e) * kStageLd + r];
        }
        stg<half8>(out + int64_t(m0 + r) * ld + n0 + c8, h);
        stg<half8>(outT + int64_t(n0 + r) * ldt + m0 + c8, t);
    }
}

// u' (f16) in the parameter's orientation into xa, from the staged tile (m0, n0) of the wide
// iterate (s_p x l_p); per-row partial sums of u'^2 into rowsqpart[tile column][row] for
// per-row-normalized matrices. Element (i, j) of the wide iterate is parameter element (i, j)
// (wide or square) or (j, i) (tall).
__device__ __forceinline__ void small_store_final(const _Float16* stage, const OrthoMat& M, int m0, int n0, int lane) {
    const bool tall = M.tall;
    const int prow0 = tall ? n0 : m0, pcol0 = tall ? m0 : n0;   // the tile in the parameter's orientation
    auto at = [&](int pr, int pc) { return tall ? stage[pc * kStageLd + pr] : stage[pr * kStageLd + pc]; };
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int ch = lane + 64 * q, r = ch >> 2, c8 = (ch & 3) * 8;
        if (prow0 + r < M.rows && pcol0 + c8 < M.ldx) {
            half8 h;
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = at(r, c8 + e);
            stg<half8>(M.xa + int64_t(prow0 + r) * M.ldx + pcol0 + c8, h);
        }
    }
    if ((M.flags & kFlagPNN) && lane < 32 && prow0 + lane < M.rows) {
        float t = 0.f;
        for (int c = 0; c < 32; ++c) {
            const float f = static_cast<float>(at(lane, c));
            t += f * f;
        }
        M.rowsqpart[int64_t(pcol0 >> 5) * M.rows + prow0 + lane] = t;
    }
}

// The fused step's prologue and epilogue: a workgroup's four 256-thread quarters take elementwise
// tiles 4 member + q, then 4 (member + C) + q, ... of the matrix.
constexpr int kQuarter = 256;
static_assert(kSmallThreads == 4 * kQuarter, "four quarters of a workgroup");

// ortho_pre_kernel's momentum for a matrix without decouple_md, Magma or an Adam step, on
// elementwise tile t by one quarter (t256 = 0..255 in that kernel's thread layout): m <- beta1 m +
// g, stored; returns this thread's sum of u^2, u = g + beta1 m, in that kernel's order.
__device__ __forceinline__ float small_momentum_tile(const OrthoMat& M, int t, int t256) {
    const int lane = t256 & 63, wave = t256 >> 6;
    const int tr = t / M.mom_tiles_c, tc = t % M.mom_tiles_c;
    const int r0 = tr * kTileR + wave * 4, c0 = tc * kTileC;
    const int nrows = M.rows - r0;
    const float beta1 = M.beta1;
    float nrm = 0.f;
    if (M.flags & kFlagVec4) {
        const int c = c0 + 4 * lane;
        if (c >= M.cols) return 0.f;
        float4 gv[4], mv[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            gv[rr] = mv[rr] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (rr >= nrows) continue;
            const int64_t o = (int64_t)(r0 + rr) * M.cols + c;
            gv[rr] = ldg_nt<float4>(M.g + o);
            mv[rr] = ldg_nt<float4>(M.m + o);
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            if (rr >= nrows) break;
            const float g[4] = {gv[rr].x, gv[rr].y, gv[rr].z, gv[rr].w};
            float m[4] = {mv[rr].x, mv[rr].y, mv[rr].z, mv[rr].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                m[e] = m[e] * beta1 + g[e];
                const float u = fmaf(m[e], beta1, g[e]);
                nrm += u * u;
            }
            stg_nt<float4>(M.m + (int64_t)(r0 + rr) * M.cols + c, make_float4(m[0], m[1], m[2], m[3]));
        }
    } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            if (rr >= nrows) break;
            const int64_t rb = (int64_t)(r0 + rr) * M.cols;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = c0 + lane + 64 * e;
                if (c >= M.cols) continue;
                const float g = ldg<float>(M.g + rb + c);
                const float m = ldg<float>(M.m + rb + c) * beta1 + g;
                stg_nt<float>(M.m + rb + c, m);
                const float u = fmaf(m, beta1, g);
                nrm += u * u;
            }
        }
    }
    return nrm;
}

// First iterate of elementwise tile t by one quarter: the values of small_x0_row; the orientation
// in which the tile's columns are contiguous stored directly, the other through the quarter's LDS
// transpose `tt` (256 rows of kX0Pitch halves, row c - c0 holding rows r0 .. r0 + 15) as 16-byte
// chunks of 8 rows (rows past the matrix, inside the padded side, receive zeros). All quarters
// call it the same number of times (block barriers); `active`: t is a tile of the matrix.
constexpr int kX0Pitch = 24;   // halves: 16-byte aligned rows, spread over the banks
static_assert(4 * kQuarter * kX0Pitch * 2 <= kSmallStages * kSmallStageBytes, "four transposes in the ring");
__device__ __forceinline__ void small_x0_tile(const OrthoMat& M, const SmallView& V, int t, int t256, bool active,
                                              float denom, _Float16* tt) {
    const int lane = t256 & 63, wave = t256 >> 6;
    const int r0 = (t / M.mom_tiles_c) * kTileR, c0 = (t % M.mom_tiles_c) * kTileC;
    _Float16* const direct = M.tall ? V.xwt(0) : V.xw(0);   // row r of the parameter, contiguous
    const int ldd = M.tall ? V.sp : V.lp;
    _Float16* const tpose = M.tall ? V.xw(0) : V.xwt(0);    // column c of the parameter, contiguous
    const int ldt = M.tall ? V.lp : V.sp;
    if (active) {
        const float beta1 = M.beta1;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int rl = wave * 4 + rr, r = r0 + rl;
            const int64_t rb = (int64_t)r * M.cols;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int cl = lane + 64 * e, c = c0 + cl;
                _Float16 x = _Float16(0.f);
                if (r < M.rows && c < M.cols) {
                    x = (_Float16)(fmaf(ldg<float>(M.m + rb + c), beta1, ldg<float>(M.g + rb + c)) / denom);
                    direct[int64_t(r) * ldd + c] = x;
                }
                tt[cl * kX0Pitch + rl] = x;
            }
        }
    }
    __syncthreads();
    if (active) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int chunk = t256 + kQuarter * h2, cl = chunk >> 1, h = chunk & 1;
            if (c0 + cl < M.cols)
                stg<half8>(tpose + int64_t(c0 + cl) * ldt + r0 + 8 * h,
                           *reinterpret_cast<const half8*>(tt + cl * kX0Pitch + 8 * h));
        }
    }
    __syncthreads();   // the transpose is read before the next round writes it
}

// Before the schedule: the momentum and the tile partials of ||u||^2 (each tile's sum over its 256
// threads as block_sum adds them), a cluster barrier, the norm and, in member 0, the matrix's
// scalars, the first iterate f16(u / (||u|| + 1e-8)) and its padding, a cluster barrier.
__device__ __forceinline__ void small_fused_prologue(const OrthoMat& M, const SmallView& V, int member, int C,
                                                     float* red, char* stages, SmallSync& sync) {
    const int q = threadIdx.x / kQuarter, t256 = threadIdx.x % kQuarter;
    const int ntiles = M.mom_tiles_r * M.mom_tiles_c, per = 4 * C;
    for (int t0 = 0; t0 < ntiles; t0 += per) {   // the same trip count in every quarter (barriers)
        const int t = t0 + 4 * member + q;
        float nrm = t < ntiles ? small_momentum_tile(M, t, t256) : 0.f;
        nrm = wave_sum(nrm);
        __syncthreads();   // the previous round's reads of red are done
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = nrm;
        __syncthreads();
        if (t < ntiles && t256 == 0) {
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) sum += red[4 * q + i];
            M.normpart[t] = sum;
        }
    }
    sync.wait();
    const float s = norm_partials(M, red);
    if (member == 0 && threadIdx.x == 0) norm_write_scales(M, s);
    const float denom = norm_denom(s);
    if (member == 0) small_x0_padding(M, V, threadIdx.x, kSmallThreads);
    _Float16* const tt = reinterpret_cast<_Float16*>(stages) + q * kQuarter * kX0Pitch;
    for (int t0 = 0; t0 < ntiles; t0 += per) {
        const int t = t0 + 4 * member + q;
        small_x0_tile(M, V, t < ntiles ? t : 0, t256, t < ntiles, denom, tt);
    }
    sync.wait();
}

// After the schedule (its last barrier has made every member's u' and row sums visible): gamma and
// the row scales s_i of per-row-normalized matrices (every member computes them, into LDS while
// the rows fit; member 0 also stores gamma, as ortho_rowstats_kernel does), then p's update on
// this member's tiles.
constexpr int kFusedMaxScaleRows = kSmallStages * kSmallStageBytes / 4;
__device__ __forceinline__ void small_fused_apply(const OrthoMat& M, int member, int C, float* red, char* stages) {
    const int q = threadIdx.x / kQuarter, t256 = threadIdx.x % kQuarter;
    const bool pnn = M.flags & kFlagPNN;
    float* const sc = reinterpret_cast<float*>(stages);
    const bool staged = M.rows <= kFusedMaxScaleRows;
    const float gamma = pnn ? pnn_gamma(M, red, staged ? sc : nullptr) : 1.f;   // its block_sum syncs sc
    if (pnn && member == 0 && threadIdx.x == 0) M.scal[kScalGamma] = gamma;
    const int ntiles = M.mom_tiles_r * M.mom_tiles_c;
    for (int t = 4 * member + q; t < ntiles; t += 4 * C) {
        if (staged)
            (void)pnn_apply_tile(M, t, t256, M.xa, gamma, [&](int row) { return sc[row]; });
        else
            (void)pnn_apply_tile(M, t, t256, M.xa, gamma,
                                 [&](int row) { return pnn_row_scale(M, pnn_row_sum(M, row)); });
    }
}

// One launch: the schedule of every small matrix in the task list, whose block map gives each block
// its matrix and its place in the matrix's cluster (thorn_ortho_fill_table gives a cluster's blocks
// one residue mod 8, so that they run on one XCD). err: set when a cluster barrier times out.
// Each operation's output is cut into super-tiles of 64 x 64 or 128 x 128 (the size that takes
// fewer rounds over the cluster, 64 on a tie) dealt to the cluster's workgroups; within one, wave
// w takes the 32 x 32 tile (w % (SM/32), w / (SM/32)).
// FUSED: the plan's whole step (small_fused_prologue, the schedule, small_fused_apply).
template <bool FUSED>
__global__ __launch_bounds__(kSmallThreads) void ns_small_kernel(const OrthoMat* __restrict__ mats, TaskList tl,
                                                                 SmallSchedule sc, int* err, int spin,
                                                                 int xcd_barriers) {
    __shared__ __attribute__((aligned(1024))) char stages[kSmallStages * kSmallStageBytes];
    __shared__ float red[kSmallWaves];
    __shared__ __attribute__((aligned(1024))) char cbuf[kSmallWaves * kCTileBytes];   // C tiles (small_issue_c)
    static_assert(kSmallWaves * 32 * kStageLd * 2 <= kSmallStages * kSmallStageBytes, "staging tiles in the ring");
    // the block map: (matrix, member | C << 8), or matrix -1 for a block that has no work
    const int mat = tl.map[2 * blockIdx.x];
    if (mat < 0) return;
    const int mc = tl.map[2 * blockIdx.x + 1];
    const OrthoMat& M = mats[mat];
    const int member = mc & 255, C = mc >> 8;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    _Float16* const stage = reinterpret_cast<_Float16*>(stages) + wave * 32 * kStageLd;
    const char* const ctile = cbuf + wave * kCTileBytes;
    const uint32_t ctile_lds = __builtin_amdgcn_readfirstlane(lds_address(ctile));
    const SmallView V = small_view(M);
    SmallSync sync(M.small_bar, member, C, err, spin, xcd_barriers != 0);
    const int set = M.rows == M.cols ? 0 : 1;
    const unsigned tslot = ts_begin();
    if constexpr (FUSED) small_fused_prologue(M, V, member, C, red, stages, sync);
    ts_point(tslot, 1);

    const int nops = sc.n[set];
    for (int q = 0; q < nops; ++q) {
        const SmallOp op = sc.op[set][q];
        ts_op(tslot, q, 0);
        ts_op(tslot, q, 1);   // kept by a workgroup with no super-tile in this operation
        // output rows x cols and the operands of this operation
        const int orows = V.sp, ocols = op.kind == kOpUpdate ? V.lp : V.sp;
        const _Float16 *A, *BT, *CT = nullptr;
        int64_t lda, ldb;
        int K;
        if (op.kind == kOpGram) {          // R = X X^T, K = l
            A = BT = V.xw(op.xsel);
            lda = ldb = V.lp;
            K = V.lp;
        } else if (op.kind == kOpSym) {    // out = alpha A B + beta C
            A = V.sq(op.a);
            BT = V.sqt(op.b);
            lda = ldb = V.sp;
            K = V.sp;
            if (op.c >= 0) CT = V.sqt(op.c);
        } else {                           // X' = Q X (+ beta X), K = s
            A = V.sq(op.a);
            BT = V.xwt(op.xsel);
            lda = ldb = V.sp;
            K = V.sp;
            if (op.c >= 0) CT = V.xwt(op.xsel);
        }
        // super-tiles of 64 x 64 when they take no more rounds over the cluster than 128 x 128 ones
        // (a quarter of the K-loop work per workgroup), else 128 x 128
        const int r64 = (orows + 63) / 64 * ((ocols + 63) / 64), r128 = (orows + 127) / 128 * ((ocols + 127) / 128);
        const int TS = (r64 + C - 1) / C <= (r128 + C - 1) / C ? 64 : 128;
        const int SM = min(orows, TS), SN = min(ocols, TS);
        const int SR = (orows + TS - 1) / TS, SC = (ocols + TS - 1) / TS;
        const int tm = SM / 32;
        const bool has_tile = wave < tm * (SN / 32);
        const int ti = has_tile ? wave % tm : 0, tj = has_tile ? wave / tm : 0;
        for (int st = member; st < SR * SC; st += C) {
            const int M0 = TS * (st % SR), N0 = TS * (st / SR);
            const int sm = min(SM, orows - M0), sn = min(SN, ocols - N0);
            const bool mine = has_tile && 32 * ti < sm && 32 * tj < sn;
            const int m0 = M0 + 32 * ti, n0 = N0 + 32 * tj;
            // every C^T has s_p columns
            const floatx16 acc = small_block(stages, M.zero, A, lda, BT, ldb, M0, N0, sm, sn, K, wave, lane, mine,
                                             ti, tj, ctile_lds, CT, V.sp, m0, n0, tslot, q);
            ts_op(tslot, q, 1);
            if (!mine) continue;
            half4 cv[4] = {};
            if (CT) small_read_c(cv, ctile, lane);
            const float alpha = op.kind == kOpSym ? op.alpha : 1.f;
            if (CT) small_stage<true>(acc, stage, alpha, op.beta, cv, lane);
            else small_stage<false>(acc, stage, alpha, op.beta, cv, lane);
            if (op.kind == kOpGram) {
                small_store(stage, V.sq(kBufR), V.sp, V.sqt(kBufR), V.sp, m0, n0, lane);
            } else if (op.kind == kOpSym) {
                small_store(stage, V.sq(op.o), V.sp, V.sqt(op.o), V.sp, m0, n0, lane);
                if (op.o2 >= 0) {
                    wave_lds_sync();
                    if (m0 == n0 && lane < 32 && m0 + lane < M.s) {
                        _Float16& z = stage[lane * kStageLd + lane];
                        z = static_cast<_Float16>(static_cast<float>(z) + op.dual);
                    }
                    wave_lds_sync();
                    small_store(stage, V.sq(op.o2), V.sp, V.sqt(op.o2), V.sp, m0, n0, lane);
                }
            } else if (op.fin) {
                small_store_final(stage, M, m0, n0, lane);
            } else {
                const int xo = 1 - op.xsel;
                small_store(stage, V.xw(xo), V.lp, V.xwt(xo), V.sp, m0, n0, lane);
            }
        }
        ts_op(tslot, q, 2);
        sync.wait();
    }
    ts_point(tslot, 2);
    if constexpr (FUSED) small_fused_apply(M, member, C, red, stages);
    // kind 4 (small), fused flag, the member and the matrix's index in the plan
    ts_end(tslot, 4ull | (FUSED ? 16ull : 0ull) | (static_cast<unsigned long long>(member) << 8) |
                      (static_cast<unsigned long long>(mat) << 20));
}

}  // namespace thorn
