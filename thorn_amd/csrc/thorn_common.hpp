// Shared device helpers and table layouts for the THORN step on gfx950 (MI355X).
//
// Everything here is CDNA4-specific: 64-lane wavefronts, the f16 MFMA builtins and the
// ds_read_tr16_b64 LDS transpose read. Lane layouts used below were checked on an MI355X:
//   v_mfma_f32_32x32x16_f16: lane l feeds A[row l%32][k 8*(l/32)+e] and B[k 8*(l/32)+e][col l%32],
//     and holds D[8*(r/4) + 4*(l/32) + r%4][l%32] in accumulator register r.
//   ds_read_tr16_b64: in each 16-lane group, lane i (a=i/4, b=i%4) receives element b of the
//     8-byte chunks addressed by lanes a, a+4, a+8, a+12.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace thorn {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((vector_size(8)));

constexpr int kWave = 64;

// Global-memory views of generic pointers. Loads and stores through them compile to global_*
// instructions (vmcnt only) instead of flat_* (which also count in lgkmcnt and so force the LDS
// fragment reads of the GEMM pipeline to drain).
#define THORN_GLOBAL __attribute__((address_space(1)))

// (The host pass of the compiler type-checks device templates too but has no address space 1
// view of these types; it never runs this code.)
template <class T>
__device__ __forceinline__ T ldg(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *reinterpret_cast<const THORN_GLOBAL T*>(reinterpret_cast<uintptr_t>(p));
#else
    return *reinterpret_cast<const T*>(p);
#endif
}
template <class T>
__device__ __forceinline__ void stg(void* p, const T& v) {
#if defined(__HIP_DEVICE_COMPILE__)
    *reinterpret_cast<THORN_GLOBAL T*>(reinterpret_cast<uintptr_t>(p)) = v;
#else
    *reinterpret_cast<T*>(p) = v;
#endif
}
// Streaming load: marked non-temporal, for data read once per step (the elementwise kernels'
// inputs). On gfx950 the Adam access pattern reads 7% faster this way.
template <class T>
__device__ __forceinline__ T ldg_nt(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    if constexpr (sizeof(T) == 16)
        return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const THORN_GLOBAL u32x4*>(a)));
    else if constexpr (sizeof(T) == 8)
        return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const THORN_GLOBAL u32x2*>(a)));
    else if constexpr (sizeof(T) == 4)
        return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const THORN_GLOBAL unsigned*>(a)));
    else
        return ldg<T>(p);
#else
    return *reinterpret_cast<const T*>(p);
#endif
}

// Streaming store: marked non-temporal, so large outputs that the next kernel reads from HBM
// anyway do not displace the L2 lines the running GEMMs reuse.
template <class T>
__device__ __forceinline__ void stg_nt(void* p, const T& v) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    if constexpr (sizeof(T) == 16)
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<THORN_GLOBAL u32x4*>(a));
    else if constexpr (sizeof(T) == 8)
        __builtin_nontemporal_store(__builtin_bit_cast(u32x2, v), reinterpret_cast<THORN_GLOBAL u32x2*>(a));
    else if constexpr (sizeof(T) == 4)
        __builtin_nontemporal_store(__builtin_bit_cast(unsigned, v), reinterpret_cast<THORN_GLOBAL unsigned*>(a));
    else
        stg<T>(p, v);
#else
    *reinterpret_cast<T*>(p) = v;
#endif
}

// ---------------------------------------------------------------------------------------------
// Numeric helpers
// ---------------------------------------------------------------------------------------------

// log(1 + exp(x)) with PyTorch's default threshold: x > 20 returns x (F.softplus, beta=1).
__device__ __forceinline__ float softplus_f(float x) {
    return x > 20.f ? x : log1pf(expf(x));
}

__device__ __forceinline__ float sigmoid_f(float x) {
    return 1.f / (1.f + expf(-x));
}

// v from the lane selected by the DPP control CTRL; lanes of the 16-lane rows outside ROW_MASK
// (and lanes without a source) get 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF,
                                                                 false));
}

// Sum over each aligned group of 32 lanes with DPP moves (register to register, no LDS round
// trip): pairs and quads by quad permutes, 8 and 16 lanes by the half-row and row mirrors, then
// row_bcast15 adds row 0's sum into row 1 (and row 2's into row 3). The group sum is exact in
// lanes 16..31 and 48..63 (the upper row of each group); other lanes hold partial sums. All
// lanes must be active.
__device__ __forceinline__ float sum32_upper(float v) {
    v += dpp_mov<0xB1>(v);          // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);          // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);         // row_half_mirror
    v += dpp_mov<0x140>(v);         // row_mirror
    v += dpp_mov<0x142, 0xA>(v);    // row_bcast15 into rows 1 and 3 (rows 0 and 2 add 0)
    return v;
}

// Sum over the wave (all 64 lanes active), returned to every lane: the two 32-lane sums joined
// by row_bcast31 into rows 2 and 3, then read from lane 63.
__device__ __forceinline__ float wave_sum(float v) {
    v = sum32_upper(v);
    v += dpp_mov<0x143, 0xC>(v);    // row_bcast31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Deterministic block reduction over blockDim.x threads (a multiple of 64, at most 1024).
// Every thread returns the total. `scratch` holds at least blockDim.x / 64 floats.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wid] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += scratch[i];
    return t;
}

// Workgroups of a launch are dispatched to the 8 XCDs round-robin (block b runs on XCD b % 8),
// and each XCD has its own L2. A launch over two tile lists P and Q (np and nq tiles) makes XCD x
// run a contiguous eighth of P, then a contiguous eighth of Q: tiles that share operand panels
// share an L2, and every XCD gets the same mix of both lists. P's eighths go to XCDs 0..7 (the
// np % 8 larger ones first); Q's continue where P's remainder stopped, so each XCD's share of the
// two adds up to its share of the blocks, ceil((np + nq - x) / 8). Returns whether block b is a
// tile of Q, and its tile index in its list; a bijection from [0, np + nq).
__device__ __forceinline__ bool xcd_split(int b, int np, int nq, int& idx) {
    const int x = b & 7, i = b >> 3;
    const int pp = np >> 3, rp = np & 7;
    const int cp = pp + (x < rp ? 1 : 0);   // this XCD's tiles of P
    if (i < cp) {
        idx = x * pp + (x < rp ? x : rp) + i;
        return false;
    }
    const int pq = nq >> 3, rq = nq & 7, xq = (x - rp) & 7;
    idx = xq * pq + (xq < rq ? xq : rq) + (i - cp);
    return true;
}

// Finds the task k with starts[k] <= b < starts[k+1] (starts has n+1 entries, ascending).
__device__ __forceinline__ int find_task(const int32_t* starts, int n, int b) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (starts[mid] <= b) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// ---------------------------------------------------------------------------------------------
// Device tables (built on the host by the plan, copied to the device by the caller each step)
// ---------------------------------------------------------------------------------------------

enum OrthoFlags : int32_t {
    kFlagPNN = 1,        // per-row normalization of the update (tall, or forced)
    kFlagMD = 2,         // decoupled magnitude/direction with row and column gains
    kFlagMDScalar = 4,   // decoupled magnitude/direction with one scalar gain
    kFlagKeepGrad = 8,   // write g *= gain back into the user's gradient (none_grad=False)
    kFlagApply = 16,     // the parameter is updated this step
    kFlagVec4 = 32,      // p, g, m 16-byte aligned and cols % 4 == 0: float4 path
    kFlagPrescaled = 64, // first iterate written in f16 as u * 2^k, 2^k from the previous step
    kFlagMagma = 128,    // Magma: statistics into magpart, eta scaled by *magma_s
    kFlagAdam = 256,     // decouple_md tensor of an Adam group: Adam step instead of Newton-Schulz
    kFlagNormRows = 512, // kFlagAdam: renormalize per row (norm_axis = -1)
    kFlagAdamDegen = 1024, // kFlagAdam: rectification says rho <= 4, u = m
    kFlagSmall = 2048,   // Newton-Schulz in ns_small_kernel; u' in xa, applied by ortho_pnn_apply_kernel
};

// One matrix of an orthogonalized group. All user tensors are fp32, row-major rows x cols,
// contiguous; workspace buffers use padded leading dimensions (multiples of 8 elements).
struct OrthoMat {
    float* p;
    float* g;
    float* m;
    float* rg;   // row gains (rows) or the scalar gain
    float* cg;   // column gains (cols)
    float* rgm;
    float* rgv;
    float* cgm;
    float* cgv;
    const float* target;   // decoupled-magnitude target norm (0-d)
    const void* zero;      // 256 bytes of zeros in the workspace (source of out-of-range tile chunks)

    _Float16* xa;      // rows x ldx, Newton-Schulz iterate (ping)
    _Float16* xb;      // rows x ldx, Newton-Schulz iterate (pong); the final u' of per-row-normalized
                       // matrices goes to whichever of the two the last update does not read
    _Float16* gram;    // s x lds: R, the Gram matrix of the short side (plain quintic: A = X X^T)
    _Float16* zbuf;    // s x lds: Z = b R + c R^2 (plain quintic: B = b A + c A^2)
    _Float16* qa;      // s x lds: Q, the accumulated polynomial since the last restart, or R Z
    _Float16* qb;      // s x lds: (ping-pong with qa; non-square matrices only)
    float* normpart;   // [mom_tiles] partial sums of u^2
    float* rowpart;    // [mom_tiles_c][rows] partial row sums of p*g*softplus(cg)
    float* colpart;    // [mom_tiles_r][cols] partial column sums of p*g*softplus(rg)
    float* rowsqpart;  // [g3_tiles_n][rows] partial row sums of u'^2
    float* rowscale;   // [rows] per-row rsqrt(mean u'^2)
    float* scal;       // [8] per-matrix scalars (see kScal*)
    float* psqpart;    // [n_psq] partial sums of p^2 after the update
    float* magma_s;    // Magma: state['s'] of the parameter this matrix belongs to
    float4* magpart;   // [mom_tiles] Magma partial sums (g.m, g.g, m.m, 0) per elementwise tile

    int32_t rows, cols, s, l;
    int32_t ldx, lds;
    int32_t tall;
    int32_t flags;
    float eta;        // lr * scaling for this matrix
    float wd;
    float beta1;
    float gain_lr, gain_beta2, gain_w1, gain_w2, gain_eps;
    float gain_bc1, gain_bc2;   // Adam bias corrections for the gains at this matrix's step
    int32_t mom_tiles_r, mom_tiles_c;
    int32_t g3_tiles_m, g3_tiles_n;
    int32_t n_psq;
    int32_t apply_tiles;   // elementwise tiles of the per-row-normalized apply kernel
    int32_t magma_n;       // Magma: matrices of the parameter when this is its first one, else 0
    int32_t gain_n;        // scalar decouple_md gain: matrices of the parameter when this is its
                           // first one, else 0 (one gain for the whole parameter, thorn.py:1609-1612)
    // kFlagAdam: state['variance'] and the Adam scalars (lr is eta, wd is wd)
    float* v;
    float* rowpsq;    // kFlagNormRows: [mom_tiles_c][rows] partial row sums of p^2 after the update
    float adam_beta2, adam_w1, adam_w2, adam_bc1, adam_bc2, adam_eps;
    _Float16* small;     // kFlagSmall: the small-matrix iterates and s x s buffers (ns_small.hip)
    int* small_bar;      // kFlagSmall: the cluster barrier (count, generation)
    int32_t rowsq_tiles; // partial sums per row in rowsqpart (column tiles of the last update)
    float pnn_eps;       // per-row normalization's eps: torch.finfo(p.dtype).eps (thorn.py:720)
};

enum ScalSlot : int {
    kScalSigma = 0,    // 1 / (||u||_F + 1e-8)
    kScalDenom = 6,    // ||u||_F + 1e-8, the divisor of the exact first iterate (thorn.py:633)
    kScalGamma = 1,    // per-row-normalization Frobenius rescale
    kScalMDFactor = 2, // target / (||p||_F + 1e-8)
    kScalX0Scale = 3,  // factor from the stored f16 first iterate to sigma * u (1 when exact)
    kScalPrescale = 4, // 2^k nearest sigma: the next step's first-iterate prescale
    kScalRepair = 5,   // 1: the prescaled first iterate is out of range; ortho_cast_kernel rebuilds it
};

// Selectors of the s x s workspace matrices and of the two iterate buffers.
enum SymBuf : int { kBufR = 0, kBufZ = 1, kBufQA = 2, kBufQB = 3 };
enum XBuf : int { kXB = 0, kXA = 1 };   // the first iterate is written to xb

// A grouped launch: task k covers blocks [starts[k], starts[k+1]) and works on matrix order[k].
struct TaskList {
    const int32_t* order;
    const int32_t* starts;
    int32_t n;
    int32_t total;
    // optional (Newton-Schulz lists): per block b, map[2b] = the matrix (order[k] of its task k)
    // and map[2b + 1] = b - starts[k], so a block finds its tile with one load instead of a
    // search of dependent loads
    const int32_t* map = nullptr;
};

// One tensor of a non-orthogonalized (Adam) group, flattened.
struct AdamTensor {
    float* p;
    const float* g;
    float* m;
    float* v;
    int64_t n;
    float lr;       // group lr * rect * magma
    float wd;
    float beta2;
    float w1, w2;   // 1 - beta1, 1 - beta2 (rounded from double)
    float bc1, bc2;
    float eps;
    int32_t flags;  // kAdam*
    float* magma_s;    // Magma: state['s']
    float4* magpart;   // Magma: [chunks] partial sums (g.m, g.g, m.m, 0) per 4096-element chunk
};

enum AdamFlags : int32_t {
    kAdamApply = 1,       // write p (the reference skips p when it is not updated this step)
    kAdamDegenerate = 2,  // rectification says rho <= 4: u = m, lr*rect == 0
    kAdamAtan2 = 4,       // eps == 0: Adam-atan2
    kAdamVec4 = 8,        // all four pointers 16-byte aligned: float4 path
    kAdamMagma = 16,      // Magma statistics, lr scaled by *magma_s
};

}  // namespace thorn
