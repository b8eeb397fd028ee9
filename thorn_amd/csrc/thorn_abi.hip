// C ABI of the THORN step (declared in include/thorn_amd.h): host-side plans, device tables and
// the launch sequence. One translation unit: the kernel sources are included below.
#include "../../include/thorn_amd.h"
#include "ns_small.hip"
#include "sym_addmm.hip"
#include "task_layout.hpp"
#include "update_kernels.hip"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <string>
#include <vector>

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(THORN_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return THORN_OK;
}

constexpr size_t kAlign = 256;
constexpr int64_t kPrescaleMinElems = int64_t(1) << 20;   // see thorn_ortho_fill_table
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Offsets of one matrix's workspace buffers (bytes from the workspace base; kNone = absent).
constexpr size_t kNone = ~size_t(0);
struct MatLayout {
    int32_t rows, cols, s, l, ldx, lds, tall, flags;
    int32_t mom_tiles_r, mom_tiles_c, g3_tiles_m, g3_tiles_n, sym_tiles, n_psq;
    size_t xa, xb, gram, zbuf, qa, qb, normpart, rowpart, colpart, rowsqpart, rowscale, scal, psqpart;
    size_t magpart, rowpsq, small, small_bar;
    bool adam, norm_rows;   // THORN_MAT_ADAM, THORN_MAT_NORM_ROWS
    bool is_small;          // Newton-Schulz in ns_small_kernel
    int32_t cluster;        // its workgroups
    int32_t rowsq_tiles;
};

struct TaskOffsets {
    size_t order, starts;
    int32_t n, total;
    size_t map = 0;   // the block map (TaskList::map), 0: none
};

// Optional per-launch timing: a pool of hipEvent pairs recorded around each launch while enabled.
struct LaunchTimer {
    std::vector<hipEvent_t> ev;   // 2 per record
    std::vector<int> kind;
    int used = 0;
    bool overflow = false;

    ~LaunchTimer() { release(); }
    void release() {
        for (hipEvent_t e : ev) (void)hipEventDestroy(e);
        ev.clear();
        kind.clear();
        used = 0;
    }
    bool enabled() const { return !ev.empty(); }
    int begin(int k, hipStream_t st) {
        if (!enabled()) return -1;
        if (used >= static_cast<int>(kind.size())) {
            overflow = true;
            return -1;
        }
        kind[used] = k;
        (void)hipEventRecord(ev[2 * used], st);
        return used++;
    }
    void end(int slot, hipStream_t st) {
        if (slot >= 0) (void)hipEventRecord(ev[2 * slot + 1], st);
    }
};

int timer_enable(LaunchTimer& t, int max_launches) {
    t.release();
    if (max_launches <= 0) return THORN_OK;
    t.ev.resize(2 * size_t(max_launches));
    t.kind.assign(max_launches, -1);
    for (auto& e : t.ev) {
        if (hipEventCreate(&e) != hipSuccess) {
            t.release();
            return THORN_ERR_HIP;
        }
    }
    t.used = 0;
    t.overflow = false;
    return THORN_OK;
}

int timer_read(LaunchTimer& t, double* ms, int* count, int n_kinds) {
    for (int k = 0; k < n_kinds; ++k) {
        ms[k] = 0.0;
        count[k] = 0;
    }
    for (int i = 0; i < t.used; ++i) {
        if (hipEventSynchronize(t.ev[2 * i + 1]) != hipSuccess) return THORN_ERR_HIP;
        float e = 0.f;
        if (hipEventElapsedTime(&e, t.ev[2 * i], t.ev[2 * i + 1]) != hipSuccess) return THORN_ERR_HIP;
        const int k = t.kind[i];
        if (k >= 0 && k < n_kinds) {
            ms[k] += e;
            count[k] += 1;
        }
    }
    const bool of = t.overflow;
    t.used = 0;
    t.overflow = false;
    return of ? THORN_ERR_INVALID : THORN_OK;
}

// Each recorded launch's kind and its start and end in ms after `ref` (an event recorded by the
// caller before the launches, timing enabled); starts a new window like timer_read.
int timer_intervals(LaunchTimer& t, hipEvent_t ref, double* s, double* e, int* kinds, int max, int* n) {
    *n = 0;
    const int k = t.used < max ? t.used : max;
    for (int i = 0; i < t.used; ++i) {
        if (hipEventSynchronize(t.ev[2 * i + 1]) != hipSuccess) return THORN_ERR_HIP;
        if (i >= k) continue;
        float a = 0.f, b = 0.f;
        if (hipEventElapsedTime(&a, ref, t.ev[2 * i]) != hipSuccess) return THORN_ERR_HIP;
        if (hipEventElapsedTime(&b, ref, t.ev[2 * i + 1]) != hipSuccess) return THORN_ERR_HIP;
        s[i] = a;
        e[i] = b;
        kinds[i] = t.kind[i];
    }
    *n = k;
    const bool of = t.overflow || t.used > max;
    t.used = 0;
    t.overflow = false;
    return of ? THORN_ERR_INVALID : THORN_OK;
}

}  // namespace

struct thorn_ortho_plan {
    std::vector<MatLayout> mats;
    size_t ws_bytes = 0;
    size_t table_bytes = 0;
    size_t mats_off = 0;
    // Newton-Schulz task lists per matrix set: [0] square matrices (plain quintic), [1] the others
    // (Gram Newton-Schulz); sym = upper-triangle tiles of s x s products, g3 = tiles of X updates.
    TaskOffsets pre{}, sym[2]{}, g3[2]{}, pnn{}, rs{}, md{}, adam{}, small{};
    // pnn: matrices applied by ortho_pnn_apply_kernel (per-row-normalized or small); rs: the
    // per-row-normalized ones (ortho_rowstats_kernel); small: ns_small_kernel's clusters
    std::vector<int32_t> pre_order, sym_order[2], g3_order[2], pnn_order, rs_order, md_order, adam_order, small_order;
    // The Newton-Schulz and per-row-normalization lists of the last filled table: only the
    // matrices applied this step (the reference skips the polar factor of the others,
    // thorn.py:1395-1396, 1436-1441). Same table offsets, fewer entries.
    TaskOffsets sym_live[2]{}, g3_live[2]{}, pnn_live{}, rs_live{}, adam_live{}, small_live{};
    // mean short and long side of each set's matrices: the contraction lengths of its GEMM tiles
    // (long side: Gram matrices; short side: the other products), to run longer tiles first
    double mean_s[2]{}, mean_l[2]{};
    int max_mom_tiles = 0;   // elementwise 16 x 256 tiles of the largest matrix
    // per-matrix block counts of the task lists, and room for one filtered list: fill_table runs
    // every step and allocates nothing
    std::vector<int64_t> mom_blocks, sym_blocks, g3_blocks, small_blocks, one_block;
    std::vector<int32_t> kept;
    // ns_small_kernel's block map (room for 8 blocks per cluster member) and its clusters sorted by
    // size (filled every step, capacity reserved at plan creation)
    size_t small_map = 0;
    std::vector<int32_t> small_sorted;
    std::vector<char> host_table;   // host side of the table for thorn_ortho_step_noalloc
    LaunchTimer timer;
    int spin_limit = 1 << 24;   // polls of the small-matrix cluster barrier before it gives up
    // The last filled table's step runs as one ns_small_kernel<true> launch (see ns_small.hip):
    // every matrix on the small path, none with decouple_md, Magma or an Adam step, all applied,
    // and the workspace the one this plan stepped on last, whose cluster barriers its previous
    // launch left at count 0. small_fusion: thorn_ortho_set_small_fusion.
    bool small_fusion = true;
    bool fused_small = false;
    bool small_xcd = true;   // XCD-local cluster barriers allowed: thorn_ortho_set_small_xcd_barriers
    // The first iterate of a step is written directly in f16, prescaled by the power of two the
    // previous step stored in the workspace, when the previous step ran on the same workspace.
    const void* filled_ws = nullptr;   // workspace of the last fill_table
    const void* stepped_ws = nullptr;  // workspace of the last completed thorn_ortho_step
    bool any_exact = true;             // the last filled table has matrices on the exact path
    bool any_apply = true;             // the last filled table has matrices flagged THORN_STEP_APPLY
    bool any_adam_apply = true;        // ... among its THORN_MAT_ADAM ones
};

struct thorn_adam_plan {
    std::vector<int64_t> numel;
    std::vector<int32_t> order;
    std::vector<int32_t> starts;
    std::vector<int64_t> chunk0;   // per tensor: its first 4096-element chunk in the launch
    size_t table_bytes = 0;
    size_t starts_off = 0, order_off = 0;
    size_t mg_starts_off = 0, mg_order_off = 0;   // task list of the Magma tensors (per step)
    size_t ws_bytes = 0;
    int32_t total = 0;
    int32_t mg_n = 0, mg_total = 0;   // Magma tensors and their chunks in the last filled table
    LaunchTimer timer;
};

namespace {

using thorn::NsCfg;

// Appends a task list (order + block starts, and with `map` the block map) to the table layout.
TaskOffsets add_tasks(size_t& off, const std::vector<int32_t>& order, const std::vector<int64_t>& blocks_of,
                      bool map = false) {
    TaskOffsets t;
    t.n = static_cast<int32_t>(order.size());
    int64_t total = 0;
    for (int32_t i : order) total += blocks_of[i];
    t.total = static_cast<int32_t>(total);
    t.order = off;
    off = align_up(off + sizeof(int32_t) * std::max<size_t>(1, order.size()), 16);
    t.starts = off;
    off = align_up(off + sizeof(int32_t) * (order.size() + 1), 16);
    if (map) {
        t.map = off;
        off = align_up(off + 2 * sizeof(int32_t) * std::max<int64_t>(1, total), 16);
    }
    return t;
}

// Writes a task list's order and block starts, and its block map if it has one (see
// task_layout.hpp: big matrices striped over the XCDs' chunks).
bool write_tasks(char* host, const TaskOffsets& t, const std::vector<int32_t>& order,
                 const std::vector<int64_t>& blocks_of) {
    int32_t* o = reinterpret_cast<int32_t*>(host + t.order);
    int32_t* s = reinterpret_cast<int32_t*>(host + t.starts);
    int32_t acc = 0;
    for (size_t k = 0; k < order.size(); ++k) {
        o[k] = order[k];
        s[k] = acc;
        acc += static_cast<int32_t>(blocks_of[order[k]]);
    }
    s[order.size()] = acc;
    if (!t.map) return true;
    return thorn_layout::write_block_map(reinterpret_cast<int32_t*>(host + t.map), order.data(),
                                         static_cast<int>(order.size()), blocks_of.data());
}

thorn::TaskList task_list(const char* dev, const TaskOffsets& t) {
    thorn::TaskList tl;
    tl.order = reinterpret_cast<const int32_t*>(dev + t.order);
    tl.starts = reinterpret_cast<const int32_t*>(dev + t.starts);
    tl.n = t.n;
    tl.total = t.total;
    tl.map = t.map ? reinterpret_cast<const int32_t*>(dev + t.map) : nullptr;
    return tl;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct ScheduledOp {
    thorn::NsOp op;
    int kind;   // THORN_KIND_* for launch timing
};

// A fixed-capacity list of operations (the schedules are built on every step, without touching
// the heap): iters <= 32 takes at most 6 per iteration and 2 more.
struct OpList {
    static constexpr int kCap = 200;
    ScheduledOp v[kCap];
    int n = 0;
    void push_back(const ScheduledOp& o) {
        if (n < kCap) v[n] = o;
        ++n;   // n > kCap marks an overflow, which the caller reports
    }
    size_t size() const { return static_cast<size_t>(n); }
    bool overflow() const { return n > kCap; }
    const ScheduledOp& operator[](size_t i) const { return v[i]; }
    const ScheduledOp* begin() const { return v; }
    const ScheduledOp* end() const { return v + (n < kCap ? n : kCap); }
};

// The Newton-Schulz launch sequence of one matrix set and the iterate buffer that holds u' after
// its last update (the per-row normalization reads it from there).
struct NsSchedule {
    OpList ops;
    int uout_sel;
};

thorn::NsOp make_op(int32_t kind) {
    thorn::NsOp o{};
    o.kind = kind;
    o.csel = -1;
    o.osel2 = -1;
    o.alpha = 1.f;
    return o;
}

inline int other_x(int xsel) { return xsel == thorn::kXB ? thorn::kXA : thorn::kXB; }

void push_gram(OpList& ops, int xsel, bool first) {
    thorn::NsOp o = make_op(thorn::kOpGram);
    o.xsel = xsel;
    o.first = first ? 1 : 0;
    ops.push_back({o, THORN_KIND_GRAM});
}

void push_update(OpList& ops, int xsel, int qsel, bool first, bool fin, bool plus_x, float beta) {
    thorn::NsOp o = make_op(thorn::kOpUpdate);
    o.xsel = xsel;
    o.qsel = qsel;
    o.first = first ? 1 : 0;
    o.final_iter = fin ? 1 : 0;
    if (plus_x) {
        o.csel = 0;
        o.beta = beta;
    }
    ops.push_back({o, THORN_KIND_UPDATE});
}

// out = f16(alpha * A B + beta * C); dual >= 0: also Q = out + f16(dual_a) I into buffer `dual`
void push_sym(OpList& ops, int a, int b, int c, int out, float alpha, float beta, int kind,
              int dual = -1, float dual_a = 0.f) {
    thorn::NsOp o = make_op(thorn::kOpSym);
    o.asel = a;
    o.bsel = b;
    o.csel = c;
    o.osel = out;
    o.alpha = alpha;
    o.beta = beta;
    o.osel2 = dual;
    o.dual_add = static_cast<float>(static_cast<_Float16>(dual_a));   // `a * I` in f16
    ops.push_back({o, kind});
}

// Gram Newton-Schulz with restarts, the reference's recurrences and rounding points
// (thorn.py:637-653); bit i of `mask`: restart before iteration i. RZ lives in whichever Q buffer
// does not hold Q.
NsSchedule gram_schedule(int iters, uint32_t mask, const float* coeffs) {
    using namespace thorn;
    auto restarts_at = [&](int i) { return i > 0 && i < 32 && ((mask >> i) & 1u); };
    NsSchedule sc;
    int xsel = kXB;    // the first iterate
    bool first = true; // xsel still holds it
    int qsel = -1;
    push_gram(sc.ops, xsel, true);
    for (int i = 0; i < iters; ++i) {
        const float a = coeffs[3 * i], b = coeffs[3 * i + 1], c = coeffs[3 * i + 2];
        const bool restart = restarts_at(i);
        if (restart) {   // X <- Q X, R <- X X^T (thorn.py:641-643)
            push_update(sc.ops, xsel, qsel, first, false, false, 0.f);
            xsel = other_x(xsel);
            first = false;
            push_gram(sc.ops, xsel, false);
        }
        if (i == 0 || restart) {   // Z = b R + c R R; Q = Z + a I (thorn.py:647-648)
            qsel = kBufQA;
            push_sym(sc.ops, kBufR, kBufR, kBufR, kBufZ, c, b, THORN_KIND_POLY, qsel, a);
        } else {                   // Z; Q = a Q + Q Z
            push_sym(sc.ops, kBufR, kBufR, kBufR, kBufZ, c, b, THORN_KIND_POLY);
            const int qn = qsel == kBufQA ? kBufQB : kBufQA;
            push_sym(sc.ops, qsel, kBufZ, qsel, qn, 1.f, a, THORN_KIND_SYMPROD);
            qsel = qn;
        }
        if (i < iters - 1 && !restarts_at(i + 1)) {   // RZ = a R + R Z; R = a RZ + Z RZ (thorn.py:649-651)
            const int rz = qsel == kBufQA ? kBufQB : kBufQA;
            push_sym(sc.ops, kBufR, kBufZ, kBufR, rz, 1.f, a, THORN_KIND_SYMPROD);
            push_sym(sc.ops, kBufZ, rz, rz, kBufR, 1.f, a, THORN_KIND_SYMPROD);
        }
    }
    push_update(sc.ops, xsel, qsel, first, true, false, 0.f);   // X <- Q X (thorn.py:653)
    sc.uout_sel = other_x(xsel);
    return sc;
}

// The plain quintic (thorn.py:654-658): A = X X^T; B = b A + c A A; X <- a X + B X.
NsSchedule plain_schedule(int iters, const float* coeffs) {
    using namespace thorn;
    NsSchedule sc;
    int xsel = kXB;
    for (int i = 0; i < iters; ++i) {
        const float a = coeffs[3 * i], b = coeffs[3 * i + 1], c = coeffs[3 * i + 2];
        push_gram(sc.ops, xsel, i == 0);
        push_sym(sc.ops, kBufR, kBufR, kBufR, kBufZ, c, b, THORN_KIND_POLY);
        push_update(sc.ops, xsel, kBufZ, i == 0, i == iters - 1, true, a);
        xsel = other_x(xsel);
    }
    sc.uout_sel = xsel;   // the buffer the last update wrote
    return sc;
}

// The compact form of a schedule for ns_small_kernel's kernel arguments; false if it is too long.
bool small_encode(const NsSchedule& sc, thorn::SmallOp* out, int32_t& n) {
    n = 0;
    if (sc.ops.size() > static_cast<size_t>(thorn::kSmallMaxOps)) return false;
    for (const ScheduledOp& so : sc.ops) {
        const thorn::NsOp& o = so.op;
        thorn::SmallOp s{};
        s.kind = static_cast<int8_t>(o.kind);
        s.xsel = static_cast<int8_t>(o.xsel);
        s.fin = static_cast<int8_t>(o.final_iter);
        s.alpha = o.alpha;
        s.beta = o.beta;
        s.dual = o.dual_add;
        s.o2 = -1;
        if (o.kind == thorn::kOpSym) {
            s.a = static_cast<int8_t>(o.asel);
            s.b = static_cast<int8_t>(o.bsel);
            s.c = static_cast<int8_t>(o.csel);
            s.o = static_cast<int8_t>(o.osel);
            s.o2 = static_cast<int8_t>(o.osel2);
        } else if (o.kind == thorn::kOpUpdate) {
            s.a = static_cast<int8_t>(o.qsel);
            s.c = static_cast<int8_t>(o.csel);
        }
        out[n++] = s;
    }
    return true;
}

// ---------------------------------------------------------------------------------------------
// Workspace of thorn_ortho_step_noalloc: a file-scope device array (one copy per GPU the library
// runs on, held until the process ends). Host code never uses the array's name as an address: its
// per-device address comes from hipGetSymbolAddress, taken once per device with that device
// current.
// ---------------------------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = size_t(THORN_NOALLOC_SCRATCH_BYTES);
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[THORN_NOALLOC_SCRATCH_BYTES];

namespace {

int scratch_of_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(THORN_ERR_HIP, std::string("thorn_ortho_step_noalloc: hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(THORN_ERR_UNSUPPORTED, "thorn_ortho_step_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(THORN_ERR_HIP, std::string("thorn_ortho_step_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return THORN_OK;
}

// Plans may share one workspace (the optimizer's batches of a group run in turn on one). The
// first iterate's prescale factors a step leaves in the workspace belong to the plan that ran it,
// so each workspace remembers the last plan that stepped on it.
std::mutex g_ws_mu;
std::unordered_map<const void*, const thorn_ortho_plan*> g_ws_last;

const thorn_ortho_plan* last_plan_on(const void* ws) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    const auto it = g_ws_last.find(ws);
    return it == g_ws_last.end() ? nullptr : it->second;
}

void note_step(const thorn_ortho_plan* plan) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    g_ws_last[plan->filled_ws] = plan;
}

void forget_plan(const thorn_ortho_plan* plan) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (auto it = g_ws_last.begin(); it != g_ws_last.end();)
        it = it->second == plan ? g_ws_last.erase(it) : std::next(it);
}

}  // namespace

namespace thorn {
// Clears n16 16-byte words (the no-alloc workspace must start at zero: its padding and the zero
// page are read by the Newton-Schulz kernels). A fill kernel rather than a memset, so that a
// caller may capture the step in a graph.
__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* __restrict__ p, int64_t n16) {
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n16; i += int64_t(gridDim.x) * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}
}  // namespace thorn

namespace {

// Workspace layout of thorn_sym_addmm: packed A, packed B^T, packed C, the upper block triangles.
struct SymAddmmLayout {
    int64_t kp, mp;
    size_t a, bt, c, out, bytes;
};

SymAddmmLayout sym_addmm_layout(int64_t nn, int64_t m, int64_t k, int64_t c_mats) {
    SymAddmmLayout L;
    L.kp = std::max<int64_t>(32, cdiv(k, 32) * 32);
    L.mp = cdiv(m, 8) * 8;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off = align_up(off + bytes, kAlign); return o; };
    L.a = take(size_t(nn) * m * L.kp * 2);
    L.bt = take(size_t(nn) * m * L.kp * 2);
    L.c = take(size_t(c_mats) * m * L.mp * 2);
    L.out = take(size_t(nn) * m * L.mp * 2);
    L.bytes = std::max<size_t>(off, kAlign);
    return L;
}

unsigned grid_for(int64_t items, int per_block) {
    return static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(cdiv(items, per_block), 1), 1 << 20));
}

}  // namespace

extern "C" {

#ifdef THORN_BLOCK_TIMESTAMPS
// Measurement build only (not in thorn_amd.h): copies the per-block timestamps (12 words per
// block, see ns_kernels.hip) and their count, and starts a new window.
int thorn_block_timestamps(unsigned long long* host, unsigned* n) {
    if (hipMemcpyFromSymbol(n, HIP_SYMBOL(thorn::g_ts_n), sizeof(unsigned)) != hipSuccess) return THORN_ERR_HIP;
    if (hipMemcpyFromSymbol(host, HIP_SYMBOL(thorn::g_ts), sizeof(thorn::g_ts)) != hipSuccess) return THORN_ERR_HIP;
    const unsigned z = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(thorn::g_ts_n), &z, sizeof(unsigned)) != hipSuccess) return THORN_ERR_HIP;
    return THORN_OK;
}
// ... and ns_small_kernel's per-operation timestamps (kSopSlots x 64 x kSopWords words, see
// ns_kernels.hip)
int thorn_small_op_timestamps(unsigned long long* host) {
    if (hipMemcpyFromSymbol(host, HIP_SYMBOL(thorn::g_sop), sizeof(thorn::g_sop)) != hipSuccess) return THORN_ERR_HIP;
    return THORN_OK;
}
#endif

int thorn_abi_version(void) { return THORN_ABI_VERSION; }

const char* thorn_last_error(void) { return g_last_error.c_str(); }

size_t thorn_abi_struct_size(int which) {
    switch (which) {
        case 0: return sizeof(ThornOrthoMatDesc);
        case 1: return sizeof(ThornOrthoMatStep);
        case 2: return sizeof(ThornAdamTensorStep);
        case 3: return sizeof(ThornAdamSparseStep);
        default: return 0;
    }
}

int thorn_ortho_plan_create(const ThornOrthoMatDesc* descs, int n, thorn_ortho_plan_t* out) {
    if (!out) return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: out is null");
    *out = nullptr;
    if (n < 0 || (n > 0 && !descs)) return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: bad matrix list");
    auto* plan = new thorn_ortho_plan();
    size_t ws = kAlign;   // [0, 256): zeros, never written (source of out-of-range GEMM tile chunks)
    ws += kAlign;         // [256, 512): status words (THORN_WS_STATUS_OFFSET)
    auto take = [&ws](size_t bytes) {
        if (bytes == 0) return kNone;
        const size_t o = ws;
        ws = align_up(ws + bytes, kAlign);
        return o;
    };
    for (int i = 0; i < n; ++i) {
        const ThornOrthoMatDesc& d = descs[i];
        // sides up to 2^20: the epilogues' 32-bit byte offsets from a tile's first row reach
        // 512 * ld < 2^31
        if (d.rows <= 0 || d.cols <= 0 || d.rows > (1 << 20) || d.cols > (1 << 20) ||
            d.rows * d.cols > (int64_t(1) << 30)) {
            delete plan;
            return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: matrix " + std::to_string(i) +
                                               " has unsupported shape " + std::to_string(d.rows) + "x" +
                                               std::to_string(d.cols));
        }
        if ((d.flags & THORN_MAT_MD) && (d.flags & THORN_MAT_MD_SCALAR)) {
            delete plan;
            return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: MD and MD_SCALAR are exclusive");
        }
        if ((d.flags & THORN_MAT_ADAM) &&
            (!(d.flags & (THORN_MAT_MD | THORN_MAT_MD_SCALAR)) || (d.flags & THORN_MAT_PER_ROW_NORM))) {
            delete plan;
            return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: ADAM needs MD or MD_SCALAR and no PER_ROW_NORM");
        }
        if ((d.flags & THORN_MAT_NORM_ROWS) && !(d.flags & THORN_MAT_ADAM)) {
            delete plan;
            return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: NORM_ROWS needs ADAM");
        }
        MatLayout L{};
        L.rows = static_cast<int32_t>(d.rows);
        L.cols = static_cast<int32_t>(d.cols);
        L.s = std::min(L.rows, L.cols);
        L.l = std::max(L.rows, L.cols);
        L.tall = L.rows > L.cols;
        // leading dimensions are multiples of 32 (one K tile of the GEMM loop): a K tile of a
        // K-major row is then inside the row or past its end, never across it
        L.ldx = static_cast<int32_t>(align_up(L.cols, 32));
        L.lds = static_cast<int32_t>(align_up(L.s, 32));
        L.flags = d.flags & (THORN_MAT_PER_ROW_NORM | THORN_MAT_MD | THORN_MAT_MD_SCALAR);
        L.adam = (d.flags & THORN_MAT_ADAM) != 0;
        // the GEMM loop addresses each f16 iterate with 32-bit byte offsets (out-of-range ones
        // included), which holds below 1 GiB
        if (!L.adam && int64_t(L.rows) * L.ldx * 2 >= (int64_t(1) << 30)) {
            delete plan;
            return fail(THORN_ERR_UNSUPPORTED, "thorn_ortho_plan_create: matrix " + std::to_string(i) +
                                                   " has more than 2^29 elements (its f16 Newton-Schulz iterate "
                                                   "would exceed 1 GiB)");
        }
        L.norm_rows = (d.flags & THORN_MAT_NORM_ROWS) != 0;
        L.mom_tiles_r = static_cast<int32_t>(cdiv(L.rows, thorn::kTileR));
        L.mom_tiles_c = static_cast<int32_t>(cdiv(L.cols, thorn::kTileC));
        L.g3_tiles_m = static_cast<int32_t>(cdiv(L.rows, NsCfg::BM));
        L.g3_tiles_n = static_cast<int32_t>(cdiv(L.cols, NsCfg::BN));
        const int32_t T = static_cast<int32_t>(cdiv(L.s, NsCfg::BM));
        L.sym_tiles = T * (T + 1) / 2;
        const bool pnn = L.flags & THORN_MAT_PER_ROW_NORM;
        const bool md = L.flags & (THORN_MAT_MD | THORN_MAT_MD_SCALAR);
        const int64_t mom_tiles = int64_t(L.mom_tiles_r) * L.mom_tiles_c;
        // small matrices run their whole Newton-Schulz in ns_small_kernel and are applied by
        // ortho_pnn_apply_kernel (u' in xa); they always take the exact first iterate
        L.is_small = !L.adam && L.s <= thorn::kSmallMaxS && int64_t(L.rows) * L.cols < kPrescaleMinElems;
        // workgroups of its small-matrix cluster: one for s <= 128 (its s x s products are one
        // 128 x 128 super-tile, so more would only add barriers); above, enough for the s x s
        // products in 64 x 64 super-tiles and the s x l updates in 128 x 128 ones to take one round
        // each (ns_small_kernel picks each operation's super-tile size from the cluster), at most 16
        L.cluster = L.s <= 128 ? 1
                               : static_cast<int32_t>(std::min<int64_t>(
                                     16, std::max<int64_t>(cdiv(L.s, 64) * cdiv(L.s, 64), cdiv(L.s, 128) * cdiv(L.l, 128))));
        L.rowsq_tiles = static_cast<int32_t>(L.is_small ? cdiv(L.cols, 32) : L.g3_tiles_n);
        L.n_psq = md ? static_cast<int32_t>(pnn || L.adam || L.is_small ? mom_tiles
                                                                         : int64_t(L.g3_tiles_m) * L.g3_tiles_n)
                     : 0;
        // an Adam-group tensor runs no Newton-Schulz: no iterate or s x s buffers
        const size_t xbytes = L.adam ? 0 : size_t(L.rows) * L.ldx * 2;
        // R, Z, QA, QB: the upper block triangle in panels (SqPanel)
        const size_t sbytes = L.adam || L.is_small ? 0 : size_t(thorn::packed_elems(L.s, L.lds)) * 2;
        const bool square = L.rows == L.cols;   // the plain quintic needs no Q (thorn.py:654-658)
        if (L.is_small) {
            const size_t sp = align_up(L.s, 32), lp = align_up(L.l, 32);
            L.small = take((8 * sp * sp + 4 * sp * lp) * 2);
            L.small_bar = take(thorn::kSmallBarWords * sizeof(int));
        } else {
            L.small = L.small_bar = kNone;
        }
        L.xa = take(xbytes);
        L.xb = take(xbytes);
        L.gram = take(sbytes);
        L.zbuf = take(sbytes);
        L.qa = square ? kNone : take(sbytes);
        L.qb = square ? kNone : take(sbytes);
        L.rowpsq = L.norm_rows ? take(sizeof(float) * size_t(L.mom_tiles_c) * L.rows) : kNone;
        L.normpart = take(sizeof(float) * mom_tiles);
        L.rowpart = md ? take(sizeof(float) * size_t(L.mom_tiles_c) * L.rows) : kNone;
        L.colpart = (L.flags & THORN_MAT_MD) ? take(sizeof(float) * size_t(L.mom_tiles_r) * L.cols) : kNone;
        L.rowsqpart = pnn ? take(sizeof(float) * size_t(L.rowsq_tiles) * L.rows) : kNone;
        L.rowscale = pnn || L.norm_rows ? take(sizeof(float) * L.rows) : kNone;
        L.scal = take(sizeof(float) * 8);
        L.psqpart = md ? take(sizeof(float) * L.n_psq) : kNone;
        L.magpart = take(sizeof(float4) * mom_tiles);
        plan->mats.push_back(L);
    }
    plan->ws_bytes = std::max<size_t>(ws, kAlign);

    // Task orders. The GEMM kernels remap blocks so that each XCD runs a contiguous eighth of
    // the tiles; to give every eighth the same mix of work, matrices are dealt to 8 bins in
    // snake order by cost (s^2 * l per tile row), and the bins are concatenated.
    std::vector<int32_t> all(n);
    for (int i = 0; i < n; ++i) all[i] = i;
    plan->pre_order = all;
    auto snake = [&](const std::vector<int32_t>& set, auto cost) {
        std::vector<int32_t> by = set;
        std::stable_sort(by.begin(), by.end(), [&](int a, int b) { return cost(a) > cost(b); });
        std::vector<std::vector<int32_t>> bins(8);
        for (size_t r = 0; r < by.size(); ++r) {
            const size_t round = r / 8, pos = r % 8;
            bins[(round & 1) ? 7 - pos : pos].push_back(by[r]);
        }
        std::vector<int32_t> out;
        for (auto& bin : bins) out.insert(out.end(), bin.begin(), bin.end());
        return out;
    };
    // Gram Newton-Schulz for every non-square matrix, the plain quintic for square ones
    // (thorn.py:628, 637-658).
    std::vector<int32_t> sets[2];
    for (int i = 0; i < n; ++i)
        if (!plan->mats[i].adam && !plan->mats[i].is_small)
            sets[plan->mats[i].rows != plan->mats[i].cols ? 1 : 0].push_back(i);
    for (int q = 0; q < 2; ++q) {
        for (int i : sets[q]) {
            plan->mean_s[q] += plan->mats[i].s;
            plan->mean_l[q] += plan->mats[i].l;
        }
        if (!sets[q].empty()) {
            plan->mean_s[q] /= double(sets[q].size());
            plan->mean_l[q] /= double(sets[q].size());
        }
    }
    for (int q = 0; q < 2; ++q) {
        plan->sym_order[q] = snake(sets[q], [&](int i) { return double(plan->mats[i].sym_tiles) * plan->mats[i].l; });
        plan->g3_order[q] = snake(sets[q], [&](int i) {
            return double(plan->mats[i].g3_tiles_m) * plan->mats[i].g3_tiles_n * plan->mats[i].s;
        });
    }
    for (int i = 0; i < n; ++i) {
        const MatLayout& L = plan->mats[i];
        if (L.flags & THORN_MAT_PER_ROW_NORM) plan->rs_order.push_back(i);
        if ((L.flags & THORN_MAT_PER_ROW_NORM) || L.is_small) plan->pnn_order.push_back(i);
        if (L.flags & (THORN_MAT_MD | THORN_MAT_MD_SCALAR)) plan->md_order.push_back(i);
        if (L.adam) plan->adam_order.push_back(i);
        if (L.is_small) plan->small_order.push_back(i);
    }
    plan->mom_blocks.assign(n, 0);
    plan->sym_blocks.assign(n, 0);
    plan->g3_blocks.assign(n, 0);
    plan->small_blocks.assign(n, 0);
    plan->one_block.assign(n, 1);
    plan->kept.reserve(n);
    std::vector<int64_t>& mom_blocks = plan->mom_blocks;
    std::vector<int64_t>& sym_blocks = plan->sym_blocks;
    std::vector<int64_t>& g3_blocks = plan->g3_blocks;
    std::vector<int64_t>& small_blocks = plan->small_blocks;
    std::vector<int64_t>& one_block = plan->one_block;
    for (int i = 0; i < n; ++i) {
        const MatLayout& L = plan->mats[i];
        mom_blocks[i] = int64_t(L.mom_tiles_r) * L.mom_tiles_c;
        sym_blocks[i] = L.sym_tiles;
        g3_blocks[i] = int64_t(L.g3_tiles_m) * L.g3_tiles_n;
        small_blocks[i] = L.cluster;
        plan->max_mom_tiles = std::max<int64_t>(plan->max_mom_tiles, mom_blocks[i]);
    }
    if (n > 65535) {
        delete plan;
        return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: more than 65535 matrices in one plan");
    }
    size_t off = 0;
    plan->mats_off = 0;
    off = align_up(sizeof(thorn::OrthoMat) * std::max(1, n), 64);
    plan->pre = add_tasks(off, plan->pre_order, mom_blocks);
    for (int q = 0; q < 2; ++q) {
        plan->sym[q] = add_tasks(off, plan->sym_order[q], sym_blocks, true);
        plan->g3[q] = add_tasks(off, plan->g3_order[q], g3_blocks, true);
    }
    plan->pnn = add_tasks(off, plan->pnn_order, mom_blocks);
    plan->rs = add_tasks(off, plan->rs_order, one_block);
    plan->md = add_tasks(off, plan->md_order, mom_blocks);
    plan->adam = add_tasks(off, plan->adam_order, mom_blocks);
    plan->small = add_tasks(off, plan->small_order, small_blocks);
    plan->small_map = off;
    off = align_up(off + 2 * sizeof(int32_t) * std::max<int64_t>(1, 8 * int64_t(plan->small.total)), 16);
    plan->small_sorted.reserve(plan->small_order.size());
    plan->table_bytes = off;
    plan->host_table.assign(plan->table_bytes, 0);
    if (int64_t(plan->sym[0].total) + plan->sym[1].total + plan->g3[0].total + plan->g3[1].total >=
        (int64_t(1) << 31) - 1) {
        delete plan;
        return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: grid too large");
    }
    for (const TaskOffsets* t : {&plan->pre}) {
        if (int64_t(t->total) >= (int64_t(1) << 31) - 1) {
            delete plan;
            return fail(THORN_ERR_INVALID, "thorn_ortho_plan_create: grid too large");
        }
    }
    *out = plan;
    return THORN_OK;
}

void thorn_ortho_plan_destroy(thorn_ortho_plan_t plan) {
    if (plan) forget_plan(plan);
    delete plan;
}

size_t thorn_ortho_workspace_bytes(thorn_ortho_plan_t plan) { return plan ? plan->ws_bytes : 0; }

size_t thorn_ortho_table_bytes(thorn_ortho_plan_t plan) { return plan ? plan->table_bytes : 0; }

int thorn_ortho_fill_table(thorn_ortho_plan_t plan, const ThornOrthoMatStep* steps, void* workspace,
                           void* table_dev, void* table_host) {
    if (!plan || !table_dev || !table_host) return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: null argument");
    // the prescale factors in the workspace are this plan's only if no other plan stepped on it since
    const bool own_workspace = last_plan_on(workspace) == plan;
    const int n = static_cast<int>(plan->mats.size());
    if (n > 0 && (!steps || !workspace)) return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: null steps/workspace");
    if ((reinterpret_cast<uintptr_t>(workspace) % kAlign) != 0)
        return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: workspace must be 256-byte aligned");
    if ((reinterpret_cast<uintptr_t>(table_dev) % 64) != 0)
        return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: table_dev must be 64-byte aligned");
    char* host = static_cast<char*>(table_host);
    std::memset(host, 0, plan->table_bytes);
    char* ws = static_cast<char*>(workspace);
    auto at = [ws](size_t o) -> void* { return o == kNone ? nullptr : ws + o; };
    bool any_exact = false, any_apply = false, any_adam_apply = false;
    bool fuse = plan->small_fusion && n > 0 && own_workspace && workspace == plan->stepped_ws;
    auto* mats = reinterpret_cast<thorn::OrthoMat*>(host + plan->mats_off);
    for (int i = 0; i < n; ++i) {
        const MatLayout& L = plan->mats[i];
        const ThornOrthoMatStep& S = steps[i];
        const bool md = L.flags & THORN_MAT_MD, mds = L.flags & THORN_MAT_MD_SCALAR;
        if (!S.p || !S.g || !S.m || (L.adam && !S.v))
            return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: matrix " + std::to_string(i) +
                                               " has a null p/g/m (or v)");
        if ((md && (!S.row_gain || !S.col_gain || !S.row_gain_moment || !S.row_gain_variance ||
                    !S.col_gain_moment || !S.col_gain_variance || !S.target_norm)) ||
            (mds && (!S.row_gain || !S.row_gain_moment || !S.row_gain_variance || !S.target_norm)))
            return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: matrix " + std::to_string(i) + " lacks gain state");
        if (((reinterpret_cast<uintptr_t>(S.p) | reinterpret_cast<uintptr_t>(S.g) |
              reinterpret_cast<uintptr_t>(S.m)) & 3u) != 0)
            return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: fp32 tensors must be 4-byte aligned");
        thorn::OrthoMat& M = mats[i];
        M.p = S.p; M.g = S.g; M.m = S.m;
        M.rg = S.row_gain; M.cg = S.col_gain;
        M.rgm = S.row_gain_moment; M.rgv = S.row_gain_variance;
        M.cgm = S.col_gain_moment; M.cgv = S.col_gain_variance;
        M.target = S.target_norm;
        M.zero = ws;
        M.xa = static_cast<_Float16*>(at(L.xa));
        M.xb = static_cast<_Float16*>(at(L.xb));
        M.gram = static_cast<_Float16*>(at(L.gram));
        M.zbuf = static_cast<_Float16*>(at(L.zbuf));
        M.qa = static_cast<_Float16*>(at(L.qa));
        M.qb = static_cast<_Float16*>(at(L.qb));
        M.normpart = static_cast<float*>(at(L.normpart));
        M.rowpart = static_cast<float*>(at(L.rowpart));
        M.colpart = static_cast<float*>(at(L.colpart));
        M.rowsqpart = static_cast<float*>(at(L.rowsqpart));
        M.rowscale = static_cast<float*>(at(L.rowscale));
        M.scal = static_cast<float*>(at(L.scal));
        M.psqpart = static_cast<float*>(at(L.psqpart));
        M.magpart = static_cast<float4*>(at(L.magpart));
        M.rowpsq = static_cast<float*>(at(L.rowpsq));
        M.small = static_cast<_Float16*>(at(L.small));
        M.small_bar = static_cast<int*>(at(L.small_bar));
        M.rowsq_tiles = L.rowsq_tiles;
        M.v = S.v;
        M.adam_beta2 = S.adam_beta2; M.adam_w1 = S.adam_w1; M.adam_w2 = S.adam_w2;
        M.adam_bc1 = S.adam_bc1; M.adam_bc2 = S.adam_bc2; M.adam_eps = S.adam_eps;
        M.pnn_eps = S.pnn_eps > 0.f ? S.pnn_eps : 1.1920928955078125e-07f;   // torch.finfo(torch.float32).eps
        M.magma_s = S.magma_s;
        M.magma_n = 0;
        if (S.magma_s && (i == 0 || steps[i - 1].magma_s != S.magma_s)) {   // first matrix of a parameter
            int cnt = 1;
            while (i + cnt < n && steps[i + cnt].magma_s == S.magma_s) ++cnt;
            M.magma_n = cnt;
        }
        M.gain_n = 0;
        if (mds && (i == 0 || steps[i - 1].row_gain != S.row_gain)) {   // first matrix of a parameter
            int cnt = 1;
            while (i + cnt < n && steps[i + cnt].row_gain == S.row_gain) ++cnt;
            M.gain_n = cnt;
        }
        M.rows = L.rows; M.cols = L.cols; M.s = L.s; M.l = L.l;
        M.ldx = L.ldx; M.lds = L.lds; M.tall = L.tall;
        int32_t flags = L.flags | (S.step_flags & (THORN_STEP_KEEP_GRAD | THORN_STEP_APPLY));
        if (L.adam) flags |= thorn::kFlagAdam | (S.adam_degenerate ? thorn::kFlagAdamDegen : 0);
        if (L.norm_rows) flags |= thorn::kFlagNormRows;
        if (L.is_small) flags |= thorn::kFlagSmall;
        if (L.cols % 4 == 0 && aligned16(S.p) && aligned16(S.g) && aligned16(S.m) && (!L.adam || aligned16(S.v)))
            flags |= thorn::kFlagVec4;
        // The first iterate of a large matrix is written directly in f16 with the previous step's
        // power-of-two scale (one pass less over u); small matrices, whose Newton-Schulz rounding
        // is not averaged out, take the exact form of thorn.py:632-635 (and Adam-step tensors
        // have no iterate).
        if (!L.adam && workspace == plan->stepped_ws && own_workspace &&
            int64_t(L.rows) * L.cols >= kPrescaleMinElems)
            flags |= thorn::kFlagPrescaled;
        else if (!L.adam) any_exact = true;
        if (S.magma_s) {
            if (reinterpret_cast<uintptr_t>(S.magma_s) & 3u)
                return fail(THORN_ERR_INVALID, "thorn_ortho_fill_table: magma_s must be 4-byte aligned");
            flags |= thorn::kFlagMagma;
        }
        M.flags = flags;
        fuse = fuse && L.is_small && !(flags & (thorn::kFlagMD | thorn::kFlagMDScalar | thorn::kFlagMagma)) &&
               (flags & thorn::kFlagApply);
        if (L.adam) any_adam_apply = any_adam_apply || (flags & thorn::kFlagApply);
        else any_apply = any_apply || (flags & thorn::kFlagApply);
        M.eta = S.eta; M.wd = S.weight_decay; M.beta1 = S.beta1;
        M.gain_lr = S.gain_lr; M.gain_beta2 = S.gain_beta2; M.gain_w1 = S.gain_w1; M.gain_w2 = S.gain_w2;
        M.gain_eps = S.gain_eps; M.gain_bc1 = S.gain_bc1; M.gain_bc2 = S.gain_bc2;
        M.mom_tiles_r = L.mom_tiles_r; M.mom_tiles_c = L.mom_tiles_c;
        M.g3_tiles_m = L.g3_tiles_m; M.g3_tiles_n = L.g3_tiles_n;
        M.n_psq = L.n_psq;
        M.apply_tiles = L.mom_tiles_r * L.mom_tiles_c;
    }
    const std::vector<int64_t>& mom_blocks = plan->mom_blocks;
    const std::vector<int64_t>& sym_blocks = plan->sym_blocks;
    const std::vector<int64_t>& g3_blocks = plan->g3_blocks;
    const std::vector<int64_t>& small_blocks = plan->small_blocks;
    const std::vector<int64_t>& one_block = plan->one_block;
    auto applied_only = [&](const std::vector<int32_t>& order, const TaskOffsets& full,
                            const std::vector<int64_t>& blocks_of, TaskOffsets& live) {
        std::vector<int32_t>& kept = plan->kept;   // capacity n since plan creation
        kept.clear();
        int64_t total = 0;
        for (int32_t i : order) {
            if (!(mats[i].flags & thorn::kFlagApply)) continue;
            kept.push_back(i);
            total += blocks_of[i];
        }
        write_tasks(host, full, kept, blocks_of);
        live = full;
        live.n = static_cast<int32_t>(kept.size());
        live.total = static_cast<int32_t>(total);
    };
    write_tasks(host, plan->pre, plan->pre_order, mom_blocks);
    for (int q = 0; q < 2; ++q) {
        applied_only(plan->sym_order[q], plan->sym[q], sym_blocks, plan->sym_live[q]);
        applied_only(plan->g3_order[q], plan->g3[q], g3_blocks, plan->g3_live[q]);
    }
    applied_only(plan->pnn_order, plan->pnn, mom_blocks, plan->pnn_live);
    applied_only(plan->rs_order, plan->rs, one_block, plan->rs_live);
    applied_only(plan->adam_order, plan->adam, mom_blocks, plan->adam_live);
    applied_only(plan->small_order, plan->small, small_blocks, plan->small_live);
    {
        // ns_small_kernel's block map: each cluster on one XCD, whose L2 its workgroups then share
        // (their barriers can skip the L2 maintenance, ns_small.hip)
        std::vector<int32_t>& live = plan->small_sorted;   // capacity n since plan creation
        live.clear();
        for (int32_t i : plan->small_order)
            if (mats[i].flags & thorn::kFlagApply) live.push_back(i);
        std::vector<int32_t>& srt = plan->kept;   // capacity n, free again after applied_only
        srt.resize(live.size());
        plan->small_live.total = static_cast<int32_t>(thorn_layout::write_cluster_map(
            reinterpret_cast<int32_t*>(host + plan->small_map), live.data(), static_cast<int>(live.size()),
            small_blocks.data(), srt.data()));
        plan->small_live.map = plan->small_map;
    }
    write_tasks(host, plan->md, plan->md_order, mom_blocks);
    plan->filled_ws = workspace;
    plan->fused_small = fuse;
    plan->any_exact = any_exact;
    plan->any_apply = any_apply;
    plan->any_adam_apply = any_adam_apply;
    return THORN_OK;
}

namespace {

// thorn_ortho_step, recording ns_begin (if not null) on the stream once the prologue launches are
// enqueued: before the first Newton-Schulz launch, or at the end of a step without one.
int ortho_step(thorn_ortho_plan_t plan, const void* table_dev, const float* coeffs, int iters,
               uint32_t restart_mask, void* stream, hipEvent_t ns_begin) {
    if (!plan || !table_dev) return fail(THORN_ERR_INVALID, "thorn_ortho_step: null argument");
    if (iters < 0 || iters > 32 || (iters > 0 && !coeffs))
        return fail(THORN_ERR_INVALID, "thorn_ortho_step: need 0 <= iters <= 32 and coefficients");
    if (iters == 0 && plan->any_apply)
        return fail(THORN_ERR_INVALID,
                    "thorn_ortho_step: iters = 0 (momentum only) with matrices flagged THORN_STEP_APPLY");
    const int n = static_cast<int>(plan->mats.size());
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto signal = [&]() -> int {
        if (ns_begin && hipEventRecord(ns_begin, st) != hipSuccess)
            return fail(THORN_ERR_HIP, "thorn_ortho_step_event: hipEventRecord failed");
        return THORN_OK;
    };
    if (n == 0) return signal();
    const char* dev = static_cast<const char*>(table_dev);
    const auto* mats = reinterpret_cast<const thorn::OrthoMat*>(dev + plan->mats_off);
    LaunchTimer& tm = plan->timer;
    int rc, slot;
    int* const status = reinterpret_cast<int*>(static_cast<char*>(const_cast<void*>(plan->filled_ws)) +
                                               THORN_WS_STATUS_OFFSET);
#define THORN_LAUNCH(kind, name, ...)                      \
    slot = tm.begin(kind, st);                             \
    hipLaunchKernelGGL(__VA_ARGS__);                       \
    tm.end(slot, st);                                      \
    if ((rc = check_launch(name))) return rc;

    // ns_small_kernel over small_live: the schedule of each small matrix (fused: the whole step)
    auto launch_small = [&](bool fused, const NsSchedule* sched) -> int {
        thorn::SmallSchedule ss{};
        for (int q = 0; q < 2; ++q) {
            if (!small_encode(sched[q], ss.op[q], ss.n[q]))
                return fail(THORN_ERR_UNSUPPORTED, "thorn_ortho_step: more than " +
                                                       std::to_string(thorn::kSmallMaxOps) +
                                                       " Newton-Schulz operations for the small-matrix path");
        }
        if (fused) {
            THORN_LAUNCH(THORN_KIND_SMALL, "ns_small_kernel", thorn::ns_small_kernel<true>,
                         dim3(plan->small_live.total), dim3(thorn::kSmallThreads), 0, st, mats,
                         task_list(dev, plan->small_live), ss, status, plan->spin_limit,
                         plan->small_xcd ? 1 : 0);
        } else {
            THORN_LAUNCH(THORN_KIND_SMALL, "ns_small_kernel", thorn::ns_small_kernel<false>,
                         dim3(plan->small_live.total), dim3(thorn::kSmallThreads), 0, st, mats,
                         task_list(dev, plan->small_live), ss, status, plan->spin_limit,
                         plan->small_xcd ? 1 : 0);
        }
        return THORN_OK;
    };
    if (plan->fused_small && iters > 0) {   // the whole step in one launch (ns_small.hip)
        const NsSchedule sched[2] = {plain_schedule(iters, coeffs), gram_schedule(iters, restart_mask, coeffs)};
        if (sched[0].ops.overflow() || sched[1].ops.overflow())
            return fail(THORN_ERR_INVALID, "thorn_ortho_step: too many Newton-Schulz operations");
        if ((rc = signal())) return rc;
        if ((rc = launch_small(true, sched))) return rc;
        plan->stepped_ws = plan->filled_ws;
        note_step(plan);
        return THORN_OK;
    }

    THORN_LAUNCH(THORN_KIND_PRE, "ortho_pre_kernel", thorn::ortho_pre_kernel, dim3(plan->pre.total), dim3(256), 0,
                 st, mats, task_list(dev, plan->pre));
    THORN_LAUNCH(THORN_KIND_NORM, "ortho_norm_kernel", thorn::ortho_norm_kernel,
                 dim3(n, plan->md.n > 0 ? thorn::kNormSlices : 1), dim3(256), 0, st, mats, n);
    if (plan->adam_live.n > 0) {   // the Adam step of the decouple_md tensors of an Adam group
        const thorn::TaskList ad = task_list(dev, plan->adam_live);
        THORN_LAUNCH(THORN_KIND_ADAM, "ortho_adam_apply_kernel", thorn::ortho_adam_apply_kernel, dim3(ad.total),
                     dim3(256), 0, st, mats, ad);
    }
    if (iters == 0) {   // no Newton-Schulz update is due: the decouple_md tail and done
        if (plan->md.n > 0) {   // p *= target / ||p|| where applied, then p *= softplus(gains)
            const thorn::TaskList md = task_list(dev, plan->md);
            if (plan->any_adam_apply) {
                THORN_LAUNCH(THORN_KIND_MD_FACTOR, "ortho_md_factor_kernel", thorn::ortho_md_factor_kernel,
                             dim3(md.n), dim3(256), 0, st, mats, md.order);
            }
            THORN_LAUNCH(THORN_KIND_MD_RESCALE, "ortho_md_rescale_kernel", thorn::ortho_md_rescale_kernel,
                         dim3(md.total), dim3(256), 0, st, mats, md);
        }
        plan->stepped_ws = plan->filled_ws;
        note_step(plan);
        return signal();
    }
    // The exact first iterate (and the rebuild of prescaled ones out of range): one row of blocks
    // per matrix, a tile per block when some matrix is on the exact path, else 64 blocks per
    // matrix that return at once unless a gradient scale jumped.
    {
        const int gx = plan->any_exact ? std::max(plan->max_mom_tiles, 1) : std::min(plan->max_mom_tiles, 64);
        THORN_LAUNCH(THORN_KIND_CAST, "ortho_cast_kernel", thorn::ortho_cast_kernel, dim3(std::max(gx, 1), n),
                     dim3(256), 0, st, mats);
    }
    if ((rc = signal())) return rc;
    // Newton-Schulz: square matrices on the plain quintic, the others on Gram Newton-Schulz with
    // the given restarts (thorn.py:628, 637-658); step k of both schedules shares launch k.
    const NsSchedule sched[2] = {plain_schedule(iters, coeffs), gram_schedule(iters, restart_mask, coeffs)};
    if (sched[0].ops.overflow() || sched[1].ops.overflow())
        return fail(THORN_ERR_INVALID, "thorn_ortho_step: too many Newton-Schulz operations");
    const thorn::TaskList sym[2] = {task_list(dev, plan->sym_live[0]), task_list(dev, plan->sym_live[1])};
    const thorn::TaskList g3[2] = {task_list(dev, plan->g3_live[0]), task_list(dev, plan->g3_live[1])};
    const size_t steps = std::max(sched[0].ops.size(), sched[1].ops.size());
    for (size_t k = 0; k < steps; ++k) {
        thorn::NsOp op[2]{};
        thorn::TaskList tl[2]{};
        int kind = -1;
        for (int q = 1; q >= 0; --q) {   // the Gram set first: it names the launch for timing
            if (k >= sched[q].ops.size() || sym[q].n == 0) continue;
            op[q] = sched[q].ops[k].op;
            tl[q] = op[q].kind == thorn::kOpUpdate ? g3[q] : sym[q];
            if (kind < 0) kind = sched[q].ops[k].kind;
        }
        const int total = tl[1].total + tl[0].total;
        if (total == 0) continue;
        auto klen = [&](int q) {
            return op[q].kind == thorn::kOpNone ? 0.0 : op[q].kind == thorn::kOpGram ? plan->mean_l[q] : plan->mean_s[q];
        };
        // longer tiles first; on equal contraction lengths the square set's list first (measured
        // slightly faster: NS 5.87 against 5.89 ms per step on config 2)
        const int square_first = klen(0) >= klen(1) ? 1 : 0;
        THORN_LAUNCH(kind, "ns_phase_kernel", thorn::ns_phase_kernel, dim3(total), dim3(thorn::NsCfg::NT), 0, st,
                     mats, tl[1], op[1], tl[0], op[0], square_first);
    }
    if (plan->small_live.n > 0) {   // every small matrix's whole schedule in one launch
        if ((rc = launch_small(false, sched))) return rc;
    }
    if (plan->rs_live.n > 0) {
        const thorn::TaskList rs = task_list(dev, plan->rs_live);
        THORN_LAUNCH(THORN_KIND_ROWSTATS, "ortho_rowstats_kernel", thorn::ortho_rowstats_kernel, dim3(rs.n),
                     dim3(256), 0, st, mats, rs.order);
    }
    if (plan->pnn_live.n > 0) {
        const thorn::TaskList pnn = task_list(dev, plan->pnn_live);
        thorn::UoutSel usel;
        usel.sel[0] = sched[0].uout_sel;
        usel.sel[1] = sched[1].uout_sel;
        THORN_LAUNCH(THORN_KIND_PNN_APPLY, "ortho_pnn_apply_kernel", thorn::ortho_pnn_apply_kernel, dim3(pnn.total),
                     dim3(256), 0, st, mats, pnn, usel);
    }
    if (plan->md.n > 0) {
        const thorn::TaskList md = task_list(dev, plan->md);
        THORN_LAUNCH(THORN_KIND_MD_FACTOR, "ortho_md_factor_kernel", thorn::ortho_md_factor_kernel, dim3(md.n),
                     dim3(256), 0, st, mats, md.order);
        THORN_LAUNCH(THORN_KIND_MD_RESCALE, "ortho_md_rescale_kernel", thorn::ortho_md_rescale_kernel,
                     dim3(md.total), dim3(256), 0, st, mats, md);
    }
#undef THORN_LAUNCH
    plan->stepped_ws = plan->filled_ws;
    note_step(plan);
    return THORN_OK;
}

}  // namespace

int thorn_ortho_step(thorn_ortho_plan_t plan, const void* table_dev, const float* coeffs, int iters,
                     uint32_t restart_mask, void* stream) {
    return ortho_step(plan, table_dev, coeffs, iters, restart_mask, stream, nullptr);
}

int thorn_ortho_step_event(thorn_ortho_plan_t plan, const void* table_dev, const float* coeffs, int iters,
                           uint32_t restart_mask, void* stream, void* ns_begin_event) {
    return ortho_step(plan, table_dev, coeffs, iters, restart_mask, stream, static_cast<hipEvent_t>(ns_begin_event));
}

int thorn_ortho_step_noalloc(thorn_ortho_plan_t plan, const ThornOrthoMatStep* steps, const float* coeffs,
                             int iters, uint32_t restart_mask, void* stream) {
    if (!plan) return fail(THORN_ERR_INVALID, "thorn_ortho_step_noalloc: null plan");
    const size_t ws_bytes = align_up(plan->ws_bytes, kAlign);
    const size_t need = ws_bytes + align_up(plan->table_bytes, kAlign);
    if (need > kNoAllocScratchBytes)
        return fail(THORN_ERR_INVALID, "thorn_ortho_step_noalloc: the plan needs " + std::to_string(need) +
                                           " bytes of workspace and table; the no-alloc limit is " +
                                           std::to_string(kNoAllocScratchBytes) + " bytes (THORN_NOALLOC_SCRATCH_BYTES)");
    void* base = nullptr;
    if (int rc = scratch_of_current_device(&base)) return rc;
    char* ws = static_cast<char*>(base);
    char* table_dev = ws + ws_bytes;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // the array is shared by every call on this GPU: start from zeros and the exact first iterate
    plan->stepped_ws = nullptr;
    if (int rc = thorn_ortho_fill_table(plan, steps, ws, table_dev, plan->host_table.data())) return rc;
    const int64_t n16 = static_cast<int64_t>(ws_bytes / 16);
    const int grid = static_cast<int>(std::min<int64_t>((n16 + 255) / 256, 2048));
    hipLaunchKernelGGL(thorn::zero_fill_kernel, dim3(std::max(grid, 1)), dim3(256), 0, st,
                       reinterpret_cast<uint4*>(ws), n16);
    if (int rc = check_launch("zero_fill_kernel")) return rc;
    if (plan->table_bytes > 0) {
        const hipError_t e = hipMemcpyAsync(table_dev, plan->host_table.data(), plan->table_bytes,
                                            hipMemcpyHostToDevice, st);
        if (e != hipSuccess)
            return fail(THORN_ERR_HIP, std::string("thorn_ortho_step_noalloc: table copy: ") + hipGetErrorString(e));
    }
    const int rc = thorn_ortho_step(plan, table_dev, coeffs, iters, restart_mask, stream);
    plan->stepped_ws = nullptr;   // the next call may find another plan's data in the array
    return rc;
}

int thorn_ortho_set_spin_limit(thorn_ortho_plan_t plan, int polls) {
    if (!plan || polls < 0) return fail(THORN_ERR_INVALID, "thorn_ortho_set_spin_limit: null plan or negative limit");
    plan->spin_limit = polls;
    return THORN_OK;
}

int thorn_ortho_set_small_fusion(thorn_ortho_plan_t plan, int enable) {
    if (!plan) return fail(THORN_ERR_INVALID, "thorn_ortho_set_small_fusion: null plan");
    plan->small_fusion = enable != 0;
    return THORN_OK;
}

int thorn_ortho_set_small_xcd_barriers(thorn_ortho_plan_t plan, int enable) {
    if (!plan) return fail(THORN_ERR_INVALID, "thorn_ortho_set_small_xcd_barriers: null plan");
    plan->small_xcd = enable != 0;
    return THORN_OK;
}

int thorn_ortho_timing_enable(thorn_ortho_plan_t plan, int max_launches) {
    if (!plan) return fail(THORN_ERR_INVALID, "thorn_ortho_timing_enable: null plan");
    if (timer_enable(plan->timer, max_launches)) return fail(THORN_ERR_HIP, "thorn_ortho_timing_enable: hipEventCreate failed");
    return THORN_OK;
}

int thorn_ortho_timing_intervals(thorn_ortho_plan_t plan, void* ref_event, double* start_ms, double* end_ms,
                                 int* kinds, int max, int* n) {
    if (!plan || !ref_event || !n || max < 0 || (max > 0 && (!start_ms || !end_ms || !kinds)))
        return fail(THORN_ERR_INVALID, "thorn_ortho_timing_intervals: bad argument");
    const int rc = timer_intervals(plan->timer, static_cast<hipEvent_t>(ref_event), start_ms, end_ms, kinds, max, n);
    if (rc == THORN_ERR_HIP) return fail(rc, "thorn_ortho_timing_intervals: event query failed");
    if (rc) return fail(rc, "thorn_ortho_timing_intervals: more launches than the enabled capacity or than max");
    return THORN_OK;
}

int thorn_ortho_timing_read(thorn_ortho_plan_t plan, double* ms, int* launches, int n_kinds) {
    if (!plan || !ms || !launches || n_kinds < 0) return fail(THORN_ERR_INVALID, "thorn_ortho_timing_read: bad argument");
    const int rc = timer_read(plan->timer, ms, launches, n_kinds);
    if (rc == THORN_ERR_HIP) return fail(rc, "thorn_ortho_timing_read: event query failed");
    if (rc) return fail(rc, "thorn_ortho_timing_read: more launches than the enabled capacity");
    return THORN_OK;
}

int thorn_adam_plan_create(const int64_t* numel, int n, thorn_adam_plan_t* out) {
    if (!out) return fail(THORN_ERR_INVALID, "thorn_adam_plan_create: out is null");
    *out = nullptr;
    if (n < 0 || (n > 0 && !numel)) return fail(THORN_ERR_INVALID, "thorn_adam_plan_create: bad tensor list");
    auto* plan = new thorn_adam_plan();
    plan->numel.assign(numel, numel + n);
    plan->chunk0.assign(n, 0);
    int64_t acc = 0;
    for (int i = 0; i < n; ++i) {
        if (numel[i] < 0) {
            delete plan;
            return fail(THORN_ERR_INVALID, "thorn_adam_plan_create: negative numel");
        }
        plan->chunk0[i] = acc;
        if (numel[i] == 0) continue;
        plan->order.push_back(i);
        plan->starts.push_back(static_cast<int32_t>(acc));
        acc += cdiv(numel[i], thorn::kAdamChunk);
        if (acc >= (int64_t(1) << 31) - 1) {
            delete plan;
            return fail(THORN_ERR_INVALID, "thorn_adam_plan_create: grid too large");
        }
    }
    plan->starts.push_back(static_cast<int32_t>(acc));
    plan->total = static_cast<int32_t>(acc);
    size_t off = align_up(sizeof(thorn::AdamTensor) * std::max(1, n), 64);
    plan->order_off = off;
    off = align_up(off + sizeof(int32_t) * std::max<size_t>(1, plan->order.size()), 16);
    plan->starts_off = off;
    off = align_up(off + sizeof(int32_t) * plan->starts.size(), 16);
    plan->mg_order_off = off;
    off = align_up(off + sizeof(int32_t) * std::max<size_t>(1, plan->order.size()), 16);
    plan->mg_starts_off = off;
    off = align_up(off + sizeof(int32_t) * (plan->order.size() + 1), 16);
    plan->table_bytes = off;
    plan->ws_bytes = align_up(sizeof(float4) * std::max<int64_t>(1, acc), kAlign);
    *out = plan;
    return THORN_OK;
}

void thorn_adam_plan_destroy(thorn_adam_plan_t plan) { delete plan; }

size_t thorn_adam_table_bytes(thorn_adam_plan_t plan) { return plan ? plan->table_bytes : 0; }

size_t thorn_adam_workspace_bytes(thorn_adam_plan_t plan) { return plan ? plan->ws_bytes : 0; }

int thorn_adam_fill_table(thorn_adam_plan_t plan, const ThornAdamTensorStep* steps, void* workspace,
                          void* table_dev, void* table_host) {
    if (!plan || !table_dev || !table_host) return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: null argument");
    const int n = static_cast<int>(plan->numel.size());
    if (n > 0 && !steps) return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: null steps");
    if ((reinterpret_cast<uintptr_t>(table_dev) % 64) != 0)
        return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: table_dev must be 64-byte aligned");
    if ((reinterpret_cast<uintptr_t>(workspace) % kAlign) != 0)
        return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: workspace must be 256-byte aligned");
    char* host = static_cast<char*>(table_host);
    std::memset(host, 0, plan->table_bytes);
    auto* ts = reinterpret_cast<thorn::AdamTensor*>(host);
    std::vector<int32_t> mg_order, mg_starts;
    int64_t mg_acc = 0;
    for (int i = 0; i < n; ++i) {
        const ThornAdamTensorStep& S = steps[i];
        if (plan->numel[i] > 0 && (!S.g || !S.m || !S.v || (S.apply && !S.p)))
            return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: tensor " + std::to_string(i) + " has a null pointer");
        if (((reinterpret_cast<uintptr_t>(S.p) | reinterpret_cast<uintptr_t>(S.g) |
              reinterpret_cast<uintptr_t>(S.m) | reinterpret_cast<uintptr_t>(S.v)) & 3u) != 0)
            return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: fp32 tensors must be 4-byte aligned");
        thorn::AdamTensor& T = ts[i];
        T.p = S.p; T.g = S.g; T.m = S.m; T.v = S.v;
        T.n = plan->numel[i];
        T.lr = S.lr; T.wd = S.weight_decay; T.beta2 = S.beta2; T.w1 = S.w1; T.w2 = S.w2;
        T.bc1 = S.bc1; T.bc2 = S.bc2; T.eps = S.eps;
        int32_t f = 0;
        if (S.apply) f |= thorn::kAdamApply;
        if (S.degenerate) f |= thorn::kAdamDegenerate;
        if (S.eps == 0.f) f |= thorn::kAdamAtan2;
        if ((!S.apply || aligned16(S.p)) && aligned16(S.g) && aligned16(S.m) && aligned16(S.v)) f |= thorn::kAdamVec4;
        if (S.magma_s && plan->numel[i] > 0) {
            if (!workspace)
                return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: Magma needs the workspace");
            if (reinterpret_cast<uintptr_t>(S.magma_s) & 3u)
                return fail(THORN_ERR_INVALID, "thorn_adam_fill_table: magma_s must be 4-byte aligned");
            f |= thorn::kAdamMagma;
            T.magma_s = S.magma_s;
            T.magpart = static_cast<float4*>(workspace) + plan->chunk0[i];
            mg_order.push_back(i);
            mg_starts.push_back(static_cast<int32_t>(mg_acc));
            mg_acc += cdiv(plan->numel[i], thorn::kAdamChunk);
        }
        T.flags = f;
    }
    mg_starts.push_back(static_cast<int32_t>(mg_acc));
    std::memcpy(host + plan->order_off, plan->order.data(), sizeof(int32_t) * plan->order.size());
    std::memcpy(host + plan->starts_off, plan->starts.data(), sizeof(int32_t) * plan->starts.size());
    std::memcpy(host + plan->mg_order_off, mg_order.data(), sizeof(int32_t) * mg_order.size());
    std::memcpy(host + plan->mg_starts_off, mg_starts.data(), sizeof(int32_t) * mg_starts.size());
    plan->mg_n = static_cast<int32_t>(mg_order.size());
    plan->mg_total = static_cast<int32_t>(mg_acc);
    return THORN_OK;
}

int thorn_adam_step(thorn_adam_plan_t plan, const void* table_dev, void* stream) {
    if (!plan || !table_dev) return fail(THORN_ERR_INVALID, "thorn_adam_step: null argument");
    if (plan->total == 0) return THORN_OK;
    const char* dev = static_cast<const char*>(table_dev);
    thorn::TaskList tl;
    tl.order = reinterpret_cast<const int32_t*>(dev + plan->order_off);
    tl.starts = reinterpret_cast<const int32_t*>(dev + plan->starts_off);
    tl.n = static_cast<int32_t>(plan->order.size());
    tl.total = plan->total;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* ts = reinterpret_cast<const thorn::AdamTensor*>(dev);
    int slot;
    if (plan->mg_n > 0) {   // Magma: the statistics of g and m must be complete before any p moves
        thorn::TaskList mg;
        mg.order = reinterpret_cast<const int32_t*>(dev + plan->mg_order_off);
        mg.starts = reinterpret_cast<const int32_t*>(dev + plan->mg_starts_off);
        mg.n = plan->mg_n;
        mg.total = plan->mg_total;
        slot = plan->timer.begin(THORN_KIND_MAGMA, st);
        hipLaunchKernelGGL(thorn::adam_magma_stats_kernel, dim3(mg.total), dim3(256), 0, st, ts, mg);
        if (int rc = check_launch("adam_magma_stats_kernel")) return rc;
        hipLaunchKernelGGL(thorn::adam_magma_finalize_kernel, dim3(mg.n), dim3(256), 0, st, ts, mg.order);
        plan->timer.end(slot, st);
        if (int rc = check_launch("adam_magma_finalize_kernel")) return rc;
    }
    slot = plan->timer.begin(THORN_KIND_ADAM, st);
    hipLaunchKernelGGL(thorn::adam_kernel, dim3(plan->total), dim3(256), 0, st, ts, tl);
    plan->timer.end(slot, st);
    return check_launch("adam_kernel");
}

int thorn_adam_sparse_step(const ThornAdamSparseStep* S, void* stream) {
    if (!S) return fail(THORN_ERR_INVALID, "thorn_adam_sparse_step: null argument");
    if (S->nnz < 0 || S->rows < 0 || S->row_len < 0)
        return fail(THORN_ERR_INVALID, "thorn_adam_sparse_step: negative size");
    if (S->nnz == 0 || S->row_len == 0) return THORN_OK;
    if (S->nnz > INT32_MAX) return fail(THORN_ERR_INVALID, "thorn_adam_sparse_step: more than 2^31 - 1 gradient rows");
    if (!S->p || !S->m || !S->v || !S->g_values || !S->g_rows)
        return fail(THORN_ERR_INVALID, "thorn_adam_sparse_step: null pointer");
    if (((reinterpret_cast<uintptr_t>(S->p) | reinterpret_cast<uintptr_t>(S->m) |
          reinterpret_cast<uintptr_t>(S->v) | reinterpret_cast<uintptr_t>(S->g_values)) & 3u) != 0 ||
        (reinterpret_cast<uintptr_t>(S->g_rows) & 7u) != 0)
        return fail(THORN_ERR_INVALID, "thorn_adam_sparse_step: misaligned tensor");
    thorn::SparseAdamArgs a;
    a.p = S->p; a.m = S->m; a.v = S->v;
    a.gv = S->g_values; a.rows_idx = S->g_rows;
    a.rows = S->rows; a.row_len = S->row_len;
    a.s.lr = S->lr; a.s.wd = S->weight_decay; a.s.beta2 = S->beta2; a.s.w1 = S->w1; a.s.w2 = S->w2;
    a.s.bc1 = S->bc1; a.s.bc2 = S->bc2; a.s.eps = S->eps;
    a.s.apply = S->apply != 0;
    a.s.degenerate = S->degenerate != 0;
    a.s.atan2_mode = S->eps == 0.f;
    a.vec = S->row_len % 4 == 0 && aligned16(S->p) && aligned16(S->m) && aligned16(S->v) && aligned16(S->g_values);
    a.magma_s = S->magma_s;
    a.magma_work = static_cast<float4*>(S->magma_work);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (S->magma_s) {
        if (!S->magma_work) return fail(THORN_ERR_INVALID, "thorn_adam_sparse_step: Magma needs magma_work");
        if ((reinterpret_cast<uintptr_t>(S->magma_s) & 3u) != 0 ||
            (reinterpret_cast<uintptr_t>(S->magma_work) & 15u) != 0)
            return fail(THORN_ERR_INVALID, "thorn_adam_sparse_step: misaligned Magma buffer");
        constexpr int64_t kSlots = THORN_SPARSE_MAGMA_WORK_BYTES / sizeof(float4);
        const int nb = static_cast<int>(std::min<int64_t>(S->nnz, kSlots));
        hipLaunchKernelGGL(thorn::adam_sparse_magma_kernel, dim3(nb), dim3(256), 0, st, a, S->nnz);
        if (int rc = check_launch("adam_sparse_magma_kernel")) return rc;
        hipLaunchKernelGGL(thorn::adam_sparse_magma_finalize_kernel, dim3(1), dim3(256), 0, st, a.magma_work, nb,
                           S->magma_s);
        if (int rc = check_launch("adam_sparse_magma_finalize_kernel")) return rc;
    }
    hipLaunchKernelGGL(thorn::adam_sparse_kernel, dim3(static_cast<unsigned>(S->nnz)), dim3(256), 0, st, a);
    return check_launch("adam_sparse_kernel");
}

size_t thorn_sym_addmm_workspace_bytes(int64_t nn, int64_t m, int64_t k, int64_t c_mats) {
    if (nn < 0 || m < 0 || k < 0 || c_mats < 0) return 0;
    return sym_addmm_layout(nn, m, k, c_mats).bytes;
}

int thorn_sym_addmm(const void* a, const int64_t* as, const void* b, const int64_t* bs, const void* c,
                    const int64_t* cs, int64_t c_mats, void* out, int64_t nn, int64_t m, int64_t k, float alpha,
                    float beta, void* workspace, size_t workspace_bytes, void* stream) {
    if (nn < 0 || m < 0 || k < 0) return fail(THORN_ERR_INVALID, "thorn_sym_addmm: negative size");
    if (nn > 65535) return fail(THORN_ERR_INVALID, "thorn_sym_addmm: more than 65535 products");
    if (c_mats != 0 && c_mats != 1 && c_mats != nn)
        return fail(THORN_ERR_INVALID, "thorn_sym_addmm: c_mats must be 0, 1 or nn");
    if (nn == 0 || m == 0) return THORN_OK;
    if (!a || !b || !as || !bs || !out || !workspace || (c_mats > 0 && (!c || !cs)))
        return fail(THORN_ERR_INVALID, "thorn_sym_addmm: null argument");
    const SymAddmmLayout L = sym_addmm_layout(nn, m, k, c_mats);
    if (m * L.kp >= (int64_t(1) << 30) || m * L.mp >= (int64_t(1) << 30))
        return fail(THORN_ERR_INVALID, "thorn_sym_addmm: a matrix of 2^30 elements or more");
    if (workspace_bytes < L.bytes || (reinterpret_cast<uintptr_t>(workspace) & (kAlign - 1)) != 0)
        return fail(THORN_ERR_INVALID, "thorn_sym_addmm: workspace too small or not 256-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    auto* pa = reinterpret_cast<_Float16*>(ws + L.a);
    auto* pb = reinterpret_cast<_Float16*>(ws + L.bt);
    auto* pc = reinterpret_cast<_Float16*>(ws + L.c);
    auto* po = reinterpret_cast<_Float16*>(ws + L.out);
    const auto* A = static_cast<const _Float16*>(a);
    const auto* B = static_cast<const _Float16*>(b);
    const int mi = static_cast<int>(m), kpi = static_cast<int>(L.kp), mpi = static_cast<int>(L.mp);
    const int ki = static_cast<int>(std::min<int64_t>(k, L.kp));
    // rows of A (K contiguous); rows of B^T: column n of B, element k at b[k * bs[1] + n * bs[2]]
    const int64_t ach = nn * m * (L.kp / 8);
    hipLaunchKernelGGL(thorn::sym_pack_kernel, dim3(grid_for(ach, thorn::kSymPackThreads)),
                       dim3(thorn::kSymPackThreads), 0, st, A, as[0], as[1], as[2], pa, mi, ki, kpi, ach);
    if (int rc = check_launch("sym_pack_kernel")) return rc;
    hipLaunchKernelGGL(thorn::sym_pack_kernel, dim3(grid_for(ach, thorn::kSymPackThreads)),
                       dim3(thorn::kSymPackThreads), 0, st, B, bs[0], bs[2], bs[1], pb, mi, ki, kpi, ach);
    if (int rc = check_launch("sym_pack_kernel")) return rc;
    if (c_mats > 0) {
        const int64_t cch = c_mats * m * (L.mp / 8);
        hipLaunchKernelGGL(thorn::sym_pack_kernel, dim3(grid_for(cch, thorn::kSymPackThreads)),
                           dim3(thorn::kSymPackThreads), 0, st, static_cast<const _Float16*>(c), cs[0], cs[1], cs[2],
                           pc, mi, mi, mpi, cch);
        if (int rc = check_launch("sym_pack_kernel")) return rc;
    }
    thorn::SymAddmmArgs p;
    p.a = pa;
    p.bt = pb;
    p.c = c_mats > 0 ? pc : nullptr;
    p.out = po;
    p.ab_mat = m * L.kp;
    p.c_mat = c_mats > 1 ? m * L.mp : 0;
    p.o_mat = m * L.mp;
    p.m = mi;
    p.kp = kpi;
    p.mp = mpi;
    const int64_t T = cdiv(m, thorn::NsCfg::BM);
    p.tiles = static_cast<int>(T * (T + 1) / 2);
    p.alpha = alpha;
    p.beta = beta;
    hipLaunchKernelGGL(thorn::sym_addmm_kernel, dim3(static_cast<unsigned>(nn * p.tiles)), dim3(thorn::NsCfg::NT), 0,
                       st, p);
    if (int rc = check_launch("sym_addmm_kernel")) return rc;
    const int64_t total = nn * m * m;
    hipLaunchKernelGGL(thorn::sym_unpack_kernel, dim3(grid_for(total, thorn::kSymPackThreads)),
                       dim3(thorn::kSymPackThreads), 0, st, po, mpi, static_cast<_Float16*>(out), mi, total);
    return check_launch("sym_unpack_kernel");
}

int thorn_adam_timing_enable(thorn_adam_plan_t plan, int max_launches) {
    if (!plan) return fail(THORN_ERR_INVALID, "thorn_adam_timing_enable: null plan");
    if (timer_enable(plan->timer, max_launches)) return fail(THORN_ERR_HIP, "thorn_adam_timing_enable: hipEventCreate failed");
    return THORN_OK;
}

int thorn_adam_timing_read(thorn_adam_plan_t plan, double* ms, int* launches, int n_kinds) {
    if (!plan || !ms || !launches || n_kinds < 0) return fail(THORN_ERR_INVALID, "thorn_adam_timing_read: bad argument");
    const int rc = timer_read(plan->timer, ms, launches, n_kinds);
    if (rc == THORN_ERR_HIP) return fail(rc, "thorn_adam_timing_read: event query failed");
    if (rc) return fail(rc, "thorn_adam_timing_read: more launches than the enabled capacity");
    return THORN_OK;
}

}  // extern "C"
