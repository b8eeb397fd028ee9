/*
 * thorn_amd.h - C ABI of the MI355X (gfx950) THORN optimizer step.
 *
 * The reference (pykeio/THORN, thorn/thorn.py) is a pure-Python PyTorch optimizer with no FFI.
 * Its drop-in boundary is the Python API `THORN(...).step()`; this library is what the build's
 * `thorn_amd.THORN` drives underneath, and each entry point below replaces a stretch of the
 * reference's step named in its comment.
 *
 * Conventions
 *   - All tensor pointers are device pointers to contiguous row-major fp32 data.
 *   - Streams are hipStream_t passed as void*; every launch is asynchronous on that stream.
 *   - Functions return 0 on success or a THORN_ERR_* code; thorn_last_error() describes the
 *     last failure on the calling thread.
 *   - The library allocates no device memory. Workspaces and tables come from the caller.
 *   - Tables: the caller gets their size from *_table_bytes, lets *_fill_table write the bytes
 *     into host memory (device addresses inside refer to `table_dev`), copies those bytes to
 *     `table_dev` on the same stream, then calls the *_step function.
 *   - Magma (momentum_align, thorn.py:800-836): a tensor whose step record carries `magma_s`
 *     (state['s'], a 0-d fp32 device tensor) has its Magma statistics computed on the device, with
 *     no host sync: cos = cosine similarity of the gradient and the moment before this step's
 *     update (eps 1e-8 on each norm), then *magma_s = 0.9 * s + 0.1 * sigmoid(cos / 2), and, if the
 *     tensor is applied this step, its learning rate is multiplied by the new *magma_s. The random
 *     mask (thorn.py:831-833) stays with the caller, who runs the PRNG on the host and clears the
 *     apply flag of a masked step; s moves on every step either way.
 */
#ifndef THORN_AMD_H
#define THORN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define THORN_ABI_VERSION 10

enum {
    THORN_OK = 0,
    THORN_ERR_INVALID = 1,     /* bad argument (shape, null pointer, alignment) */
    THORN_ERR_HIP = 2,         /* a HIP runtime call or kernel launch failed */
    THORN_ERR_UNSUPPORTED = 3, /* valid request this build does not implement */
};

/* Per-matrix option flags (ThornOrthoMatDesc.flags). */
#define THORN_MAT_PER_ROW_NORM 1   /* per-row normalization (thorn.py:704-707, 709-766) */
#define THORN_MAT_MD 2             /* decouple_md with row and column gains (thorn.py:1603-1608) */
#define THORN_MAT_MD_SCALAR 4      /* decouple_md with one scalar gain (thorn.py:1609-1612) */
#define THORN_MAT_ADAM 8           /* a decouple_md tensor of a non-orthogonalized group: the update
                                      is the Adam step (thorn.py:1702-1721), no Newton-Schulz; needs
                                      THORN_MAT_MD or THORN_MAT_MD_SCALAR. A 1-D tensor is 1 x n. */
#define THORN_MAT_NORM_ROWS 16     /* with THORN_MAT_ADAM: the renormalization runs per row
                                      (norm_axis = -1, thorn.py:594-595, 1717); target_norm then
                                      points at `rows` values */

/* Per-step flags (ThornOrthoMatStep.step_flags). */
#define THORN_STEP_KEEP_GRAD 8     /* none_grad=False. No effect since ABI 5: the gradient of a
                                      decouple_md matrix is always multiplied by its gains in
                                      place, as the reference's g.mul_ does (thorn.py:907) */
#define THORN_STEP_APPLY 16        /* update the parameter this step (thorn.py:1395-1396) */

int thorn_abi_version(void);
const char* thorn_last_error(void);
/* sizeof of the ABI structs, so bindings can verify their layout:
 * 0 = ThornOrthoMatDesc, 1 = ThornOrthoMatStep, 2 = ThornAdamTensorStep, 3 = ThornAdamSparseStep;
 * 0 for anything else. */
size_t thorn_abi_struct_size(int which);

/* ------------------------------------------------------------------------------------------
 * Orthogonalized group: momentum, Newton-Schulz, per-row normalization, cautious weight decay,
 * decouple_md. Replaces THORN._batched_ortho_step (thorn.py:1427-1457) with _ortho_pre
 * (thorn.py:1383-1397), _polar_decomp (thorn.py:626-667, including thorn::sym_addmm
 * thorn.py:298-377) and _ortho_post (thorn.py:1399-1425).
 * ------------------------------------------------------------------------------------------ */

typedef struct ThornOrthoMatDesc {
    int64_t rows, cols;   /* one matrix; a parameter with ndim > 2 is one desc per matrix */
    int32_t flags;        /* THORN_MAT_* */
    int32_t reserved;
} ThornOrthoMatDesc;

typedef struct ThornOrthoMatStep {
    float* p;             /* parameter (rows x cols) */
    float* g;             /* gradient */
    float* m;             /* state['moment'] */
    float* row_gain;      /* decouple_md: state['row_gain'] (rows) or state['gain'] (scalar; the
                             consecutive matrices of a parameter share it and it steps once) */
    float* col_gain;      /* state['col_gain'] (cols) */
    float* row_gain_moment;
    float* row_gain_variance;
    float* col_gain_moment;
    float* col_gain_variance;
    const float* target_norm;  /* state['target_norm'], 0-d */
    float eta;            /* group lr * _lr_scale_ortho (thorn.py:1405) */
    float weight_decay;
    float beta1;
    float gain_lr, gain_beta2, gain_w1, gain_w2, gain_eps;  /* w1 = 1 - beta1, w2 = 1 - beta2 */
    float gain_bc1, gain_bc2;  /* 1/(1 - beta1^step), 1/(1 - beta2^step) of the gain Adam */
    int32_t step_flags;   /* THORN_STEP_* */
    int32_t reserved;
    float* magma_s;       /* Magma: state['s'] (0-d) or null. Consecutive matrices with the same
                             magma_s are one parameter: the cosine similarity spans them all. */
    /* THORN_MAT_ADAM only (thorn.py:838-888 with lr = eta, the group lr * rect * magma): */
    float* v;             /* state['variance'] */
    float adam_beta2, adam_w1, adam_w2;    /* beta2, 1 - beta1, 1 - beta2 */
    float adam_bc1, adam_bc2, adam_eps;    /* bias corrections; eps 0 selects Adam-atan2 */
    int32_t adam_degenerate;               /* rect == 0: u = m (thorn.py:883-885) */
    float pnn_eps;        /* per-row normalization's eps, torch.finfo(p.dtype).eps (thorn.py:720);
                             0 selects float32's */
} ThornOrthoMatStep;

typedef struct thorn_ortho_plan* thorn_ortho_plan_t;

int thorn_ortho_plan_create(const ThornOrthoMatDesc* mats, int n, thorn_ortho_plan_t* out);
void thorn_ortho_plan_destroy(thorn_ortho_plan_t plan);
/* Device workspace; must be zero-filled once when allocated and kept for every later step.
 * Consecutive steps of a plan on the same workspace write the first Newton-Schulz iterate directly
 * in f16, prescaled by a power of two the previous step stored there (rebuilt exactly when the
 * gradient scale moved by more than 16x); the first step on a workspace takes the exact path. */
size_t thorn_ortho_workspace_bytes(thorn_ortho_plan_t plan);
/* The int32 at this byte offset of the workspace becomes nonzero in a step in which a cluster of
 * workgroups of the small-matrix Newton-Schulz launch did not all become resident (its bounded
 * barrier wait expired; that step's small-matrix updates are then not valid), and stays so until
 * the caller clears it (a zero-filled workspace starts clear; the library never clears it, so a
 * caller may read it every few steps). The thorn_amd package reads it every 16 steps that ran
 * the launch, and at THORN.check_status(), into pinned memory, raises RuntimeError when it is set
 * and clears it. */
#define THORN_WS_STATUS_OFFSET 256
/* Polls (a 64-cycle sleep each) of the small-matrix launch's bounded cluster barrier before it
 * gives up and sets the status word; default 2^24. No counterpart in the reference: a test hook
 * that makes the wait expire from the host (0: at the first wait that would block) while every
 * kernel still exits normally. */
int thorn_ortho_set_spin_limit(thorn_ortho_plan_t plan, int polls);
/* No counterpart in the reference (its eager step is one launch per operation): a step whose
 * matrices all take the small-matrix path (short side <= 256, fewer than 2^20 elements), none with
 * decouple_md or Magma, all with THORN_STEP_APPLY, on the workspace the plan last stepped on, runs
 * as one launch (momentum, norm, first iterate, Newton-Schulz, row statistics and the update of p,
 * each matrix by its cluster of workgroups) instead of six; its results are bit for bit those of
 * the separate launches. On by default; enable = 0 keeps the separate launches (for comparison). */
int thorn_ortho_set_small_fusion(thorn_ortho_plan_t plan, int enable);
/* No counterpart in the reference. The small-matrix launch places each matrix's cluster of
 * workgroups on one XCD and, when the workgroups find that they share one (their XCC ids agree),
 * synchronizes them through that XCD's L2: no L2 write-back at the barriers, which the agent-scope
 * barrier needs for other XCDs, and an invalidate of the caches up to the L2 after each; results
 * are bit for bit the same. On by default; enable = 0 keeps agent-scope barriers throughout (for
 * comparison). */
int thorn_ortho_set_small_xcd_barriers(thorn_ortho_plan_t plan, int enable);
size_t thorn_ortho_table_bytes(thorn_ortho_plan_t plan);
int thorn_ortho_fill_table(thorn_ortho_plan_t plan, const ThornOrthoMatStep* steps, void* workspace,
                           void* table_dev, void* table_host);
/* Runs the whole step for the group: coeffs holds iters (a, b, c) triples (thorn.py:425-480),
 * 1 <= iters <= 32. Non-square matrices run Gram Newton-Schulz (thorn.py:637-653) with a restart
 * before iteration i for every bit i (1 <= i < iters) set in restart_mask, the restart positions of
 * _gram_ns_restarts (thorn.py:483-514); square ones run the plain quintic (thorn.py:654-658). Both
 * follow the reference's recurrences and f16 rounding points (Z, Q, RZ, R; A, B, aX + BX).
 * With decouple_md, the gradient is multiplied by the gains in place (thorn.py:907).
 * A matrix without THORN_STEP_APPLY updates its momentum (and, with decouple_md, goes through the
 * gain round trip p / G * G) but not its parameter, as the reference does for a step that is not
 * due under update_rate (thorn.py:1395, 1403-1421). iters = 0 runs only that part, for a table in
 * which no matrix has THORN_STEP_APPLY (coeffs may then be null). */
int thorn_ortho_step(thorn_ortho_plan_t plan, const void* table_dev, const float* coeffs, int iters,
                     uint32_t restart_mask, void* stream);
/* No counterpart in the reference (its eager step runs on one stream): thorn_ortho_step, and
 * ns_begin_event (a hipEvent_t, or null) is recorded on the stream once the step's prologue
 * launches (momentum, norms, first iterate) are enqueued: before its first Newton-Schulz launch,
 * or at the end of a step without one. For callers that overlap independent work with the
 * Newton-Schulz launches: THORN runs a large orthogonalized group as two plans on two streams,
 * the second waiting for this event of the first, so that each fills the other's idle tails. */
int thorn_ortho_step_event(thorn_ortho_plan_t plan, const void* table_dev, const float* coeffs, int iters,
                           uint32_t restart_mask, void* stream, void* ns_begin_event);

/* No counterpart in the reference. For callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc; it copies its table from host memory, and is not made or
 * tested for HIP graph capture): thorn_ortho_fill_table
 * and thorn_ortho_step in one call, with the workspace and the device table in a file-scope
 * device array of THORN_NOALLOC_SCRATCH_BYTES per GPU instead of caller memory. It calls no
 * hipMalloc or hipFree; the plan (thorn_ortho_plan_create, made beforehand) holds the host side
 * of the table. Every call clears the workspace part of the array with a kernel and takes the
 * exact first iterate (nothing is carried between calls). Plans whose workspace and table exceed
 * the array are refused with THORN_ERR_INVALID. All calls on one GPU share the array: calls that
 * overlap in time on one GPU (other streams, other threads) race and must be serialized by the
 * caller. The results equal thorn_ortho_step's on a fresh workspace. */
#define THORN_NOALLOC_SCRATCH_BYTES (32u << 20)
int thorn_ortho_step_noalloc(thorn_ortho_plan_t plan, const ThornOrthoMatStep* steps, const float* coeffs,
                             int iters, uint32_t restart_mask, void* stream);

/* ------------------------------------------------------------------------------------------
 * Non-orthogonalized group: Adam / Adam-atan2 / rectified Adam with cautious weight decay, all
 * tensors of all such groups in one launch. Replaces the per-parameter loop of _step_params
 * (thorn.py:1659-1727) around _adam_update (thorn.py:838-888).
 * ------------------------------------------------------------------------------------------ */

typedef struct ThornAdamTensorStep {
    float* p;
    const float* g;
    float* m;             /* state['moment'] */
    float* v;             /* state['variance'] */
    float lr;             /* group lr * rect * magma (thorn.py:1712) */
    float weight_decay;
    float beta2;
    float w1, w2;         /* 1 - beta1, 1 - beta2 */
    float bc1, bc2;       /* 1/(1 - beta1^step), 1/(1 - beta2^step) */
    float eps;            /* 0 selects Adam-atan2 (thorn.py:879-880) */
    int32_t apply;        /* update p (thorn.py:1707) */
    int32_t degenerate;   /* rect == 0: u = m (thorn.py:883-885) */
    float* magma_s;       /* Magma: state['s'] (0-d) or null */
} ThornAdamTensorStep;

typedef struct thorn_adam_plan* thorn_adam_plan_t;

int thorn_adam_plan_create(const int64_t* numel, int n, thorn_adam_plan_t* out);
void thorn_adam_plan_destroy(thorn_adam_plan_t plan);
size_t thorn_adam_table_bytes(thorn_adam_plan_t plan);
/* Device workspace for the Magma statistics (16 bytes per 4096 elements), 256-byte aligned, kept
 * for the plan's lifetime; its contents need no initialization. Only needed when a step record
 * carries magma_s (fill_table accepts a null workspace otherwise). */
size_t thorn_adam_workspace_bytes(thorn_adam_plan_t plan);
int thorn_adam_fill_table(thorn_adam_plan_t plan, const ThornAdamTensorStep* steps, void* workspace,
                          void* table_dev, void* table_host);
int thorn_adam_step(thorn_adam_plan_t plan, const void* table_dev, void* stream);

/* One tensor with a row-sparse gradient (e.g. nn.Embedding(sparse=True)): the sparse branch of
 * _step_params (thorn.py:1667-1700). The gradient comes coalesced, its row indices distinct (as
 * torch's coalesce() leaves them); row g_rows[k] of p, m and v takes gradient row g_values[k]
 * with the arithmetic of thorn_adam_step, and every other row keeps its parameter and state.
 * Row indices outside [0, rows) are skipped. nnz = 0 launches nothing. */
typedef struct ThornAdamSparseStep {
    float* p;             /* rows x row_len, contiguous */
    float* m;             /* state['moment'], like p */
    float* v;             /* state['variance'], like p */
    const float* g_values;  /* nnz x row_len, contiguous */
    const int64_t* g_rows;  /* nnz row indices */
    int64_t rows, row_len, nnz;
    float lr, weight_decay, beta2, w1, w2, bc1, bc2, eps;   /* as in ThornAdamTensorStep */
    int32_t apply;
    int32_t degenerate;
    float* magma_s;       /* Magma: state['s'] (0-d) or null; the cosine similarity is over the
                             gradient rows and the gathered moment rows (thorn.py:1676-1679) */
    void* magma_work;     /* with magma_s: THORN_SPARSE_MAGMA_WORK_BYTES of device scratch,
                             16-byte aligned; calls that share it must not overlap */
} ThornAdamSparseStep;
#define THORN_SPARSE_MAGMA_WORK_BYTES 16384
int thorn_adam_sparse_step(const ThornAdamSparseStep* step, void* stream);

/* ------------------------------------------------------------------------------------------
 * thorn::sym_addmm (thorn.py:298-368, the custom op behind every Newton-Schulz product of the
 * reference): out = beta * C + alpha * (A @ B) for products A @ B and C that are symmetric, f16,
 * batched: A (nn, m, k), B (nn, k, m), C absent (c_mats = 0), one (m, m) matrix for every product
 * (c_mats = 1) or (nn, m, m) (c_mats = nn); element strides of each as {batch, row, column} (any
 * strides; a 2-D C's batch stride is unused). out is contiguous (nn, m, m). As the reference's
 * Triton kernel (thorn.py:209-280), only the upper block triangle of A @ B (and of C) is read
 * and computed, with fp32 accumulation and one rounding to f16; the rest is its mirror.
 * workspace: thorn_sym_addmm_workspace_bytes() bytes of device memory, 256-byte aligned; calls
 * that share it must not overlap. Limits: nn <= 65535 (thorn.py:332), m * round_up(k, 32) and
 * m * round_up(m, 8) below 2^30 elements.
 * ------------------------------------------------------------------------------------------ */
size_t thorn_sym_addmm_workspace_bytes(int64_t nn, int64_t m, int64_t k, int64_t c_mats);
int thorn_sym_addmm(const void* a, const int64_t* a_strides, const void* b, const int64_t* b_strides, const void* c,
                    const int64_t* c_strides, int64_t c_mats, void* out, int64_t nn, int64_t m, int64_t k,
                    float alpha, float beta, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Optional launch timing (measurement only; no counterpart in the reference). While enabled, the
 * *_step functions record a hipEvent pair around every launch, up to `max_launches` launches;
 * *_timing_read waits for them, writes the summed milliseconds and launch counts per kernel
 * kind (THORN_KIND_*) and starts a new window. max_launches = 0 disables timing.
 * ------------------------------------------------------------------------------------------ */
enum {
    THORN_KIND_PRE = 0,        /* momentum + first iterate (ortho_pre_kernel) */
    THORN_KIND_NORM = 1,       /* per-matrix norm, decouple_md gains */
    THORN_KIND_GRAM = 2,       /* Newton-Schulz Gram matrix R of the iterate */
    THORN_KIND_POLY = 3,       /* Newton-Schulz Z = b R + c R^2 (plain quintic: B = b A + c A^2) */
    THORN_KIND_UPDATE = 4,     /* Newton-Schulz update Q X / X Q (and the fused apply) */
    THORN_KIND_ROWSTATS = 5,   /* per-row normalization statistics */
    THORN_KIND_PNN_APPLY = 6,  /* per-row normalized apply */
    THORN_KIND_MD_FACTOR = 7,  /* decouple_md renormalization factor */
    THORN_KIND_MD_RESCALE = 8, /* decouple_md reassembly */
    THORN_KIND_ADAM = 9,       /* multi-tensor Adam */
    THORN_KIND_CAST = 10,      /* first iterate: u / ||u|| rounded to f16 */
    THORN_KIND_SYMPROD = 11,   /* Gram Newton-Schulz products a Q + Q Z, a R + R Z, a RZ + Z RZ */
    THORN_KIND_MAGMA = 12,     /* Magma statistics of the Adam tensors */
    THORN_KIND_SMALL = 13,     /* the whole Newton-Schulz of the small matrices (one launch) */
    THORN_KIND_COUNT = 14
};
int thorn_ortho_timing_enable(thorn_ortho_plan_t plan, int max_launches);
int thorn_ortho_timing_read(thorn_ortho_plan_t plan, double* ms, int* launches, int n_kinds);
/* The same window as start and end times: for each recorded launch (up to max), its kind and its
 * start and end in milliseconds after ref_event, a hipEvent (timing enabled) that the caller
 * recorded before the launches on any stream of the device; *n receives the number written. For
 * launches that overlap other streams' work, whose durations overlap too. Starts a new window. */
int thorn_ortho_timing_intervals(thorn_ortho_plan_t plan, void* ref_event, double* start_ms, double* end_ms,
                                 int* kinds, int max, int* n);
int thorn_adam_timing_enable(thorn_adam_plan_t plan, int max_launches);
int thorn_adam_timing_read(thorn_adam_plan_t plan, double* ms, int* launches, int n_kinds);

#ifdef __cplusplus
}
#endif

#endif /* THORN_AMD_H */
