// executor.hip — the C ABI of liblbr_executor.so: device setup, memory,
// the dispatch table, plans (decoded launch lists, optional hipGraph) and
// timing.  Declarations and the contract are in include/lbr_executor.h.
//
// The dispatch table mirrors csrc/executor.c:409-452 (same op codes, same
// extras decoding); instead of calling a CPU kernel, each entry decodes its
// OpNode once into a Step (validated kernel arguments) and the Step's
// launcher enqueues the HIP kernel on the library stream.  Unknown ops return
// LBR_ERR_UNSUPPORTED where the reference prints and aborts
// (executor.c:461-464).
#include "lbr_device.h"
#include "lbr_fusion.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#define LBR_VERSION "lbr-executor 0.1 gfx950"

static_assert(sizeof(OpNode) == 312, "OpNode must match csrc/runtime.h:60-69 (312 bytes)");
static_assert(offsetof(OpNode, inputs) == 8, "OpNode.inputs offset");
static_assert(offsetof(OpNode, output) == 104, "OpNode.output offset");
static_assert(offsetof(OpNode, out_shape) == 112, "OpNode.out_shape offset");
static_assert(offsetof(OpNode, n_dims) == 208, "OpNode.n_dims offset");
static_assert(offsetof(OpNode, elem_size) == 212, "OpNode.elem_size offset");
static_assert(offsetof(OpNode, extra) == 216, "OpNode.extra offset");

// ------------------------------------------------------------------ errors
static thread_local char g_err[512] = "";

void lbr_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

#define HIP_TRY(expr)                                                                       \
    do {                                                                                    \
        hipError_t _e = (expr);                                                             \
        if (_e != hipSuccess) {                                                             \
            lbr_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__,  \
                          __LINE__);                                                        \
            return LBR_ERR_HIP;                                                             \
        }                                                                                   \
    } while (0)

// ------------------------------------------------------------------ device
static std::mutex g_mu;

// Dependent arithmetic only, `iters` steps of it: a GPU-side delay of known length
// for lbr_plan_profile (x stays a; the store never happens for a = 0, b = 1).
__device__ float g_busy_sink;
__global__ void lbr_busy(int iters, float a, float b) {
    float x = a;
    for (int i = 0; i < iters; ++i) x = fmaf(x, b, a);
    if (x == -1.f) g_busy_sink = x;
}
static int g_device = -1;
static hipStream_t g_stream = nullptr;
static int g_cus = 0;

int lbr_device_cus() { return g_cus; }

// One device workspace for a step list: sized to the largest step's need and
// shared by all of them (they run in order on one stream).
static int assign_workspace(std::vector<Step>& steps, void** out) {
    size_t need = 0;
    for (const Step& s : steps) need = s.ws_bytes > need ? s.ws_bytes : need;
    *out = nullptr;
    if (!need) return LBR_OK;
    HIP_TRY(hipMalloc(out, need));
    for (Step& s : steps) s.ws = *out;
    return LBR_OK;
}

static int ensure_init() {
    if (g_stream) return LBR_OK;
    return lbr_init(0);
}

// Workspace of the one-shot entry points (lbr_execute / execute): owned by
// the library, grown when a call needs more and never shrunk, so repeated
// calls allocate nothing.  Every one-shot call ends with a stream
// synchronisation, so when the next call grows it no kernel still uses the
// old block.  Guarded by g_exec_mu (the one-shot calls are serialised, as
// the reference's execute is single-caller).
static std::mutex g_exec_mu;
static void* g_exec_ws = nullptr;
static size_t g_exec_ws_bytes = 0;
static int g_exec_ws_device = -1;

static int exec_workspace(size_t need, void** out) {
    if (g_exec_ws && g_exec_ws_device != g_device) {
        // the library moved to another device: the old block belongs to that one
        int cur = g_device;
        HIP_TRY(hipSetDevice(g_exec_ws_device));
        (void)hipFree(g_exec_ws);
        HIP_TRY(hipSetDevice(cur));
        g_exec_ws = nullptr;
        g_exec_ws_bytes = 0;
    }
    if (need > g_exec_ws_bytes) {
        if (g_exec_ws) HIP_TRY(hipFree(g_exec_ws));
        g_exec_ws = nullptr;
        g_exec_ws_bytes = 0;
        const size_t grown = (need + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);   // whole MiB
        HIP_TRY(hipMalloc(&g_exec_ws, grown));
        g_exec_ws_bytes = grown;
        g_exec_ws_device = g_device;
    }
    *out = need ? g_exec_ws : nullptr;
    return LBR_OK;
}

// Workspace of lbr_execute_noalloc: a file-scope device array of a fixed
// size, one copy per GPU, held until the process ends.  Its host-side name
// is only a stand-in for the symbol, never a device address: lbr_init
// resolves the address once per device (hipGetSymbolAddress, that device
// current) into g_scratch_dev[device], and only that pointer is passed to
// kernels.  Nothing in it needs to start at zero: the GEMM split-K ranges
// and the attention key-range segments write every partial they later read.
// Size: the largest per-call workspace of the seven benchmark workloads'
// one-kernel-per-node arrays is 40 MiB (the Qwen3-4B body's down projection,
// 4 K ranges x 1024 x 2560 floats of partial sums; its attention runs on
// folded 64-row blocks with no workspace); the GPT-2 and 7B workloads need at
// most 25 MiB.
#define LBR_SCRATCH_BYTES ((size_t)48 << 20)
#define LBR_MAX_DEVICES 64
static __device__ __align__(256) unsigned char scratch[LBR_SCRATCH_BYTES];
static void* g_scratch_dev[LBR_MAX_DEVICES] = {};

// ------------------------------------------------------------------ host staging
// Uploads from ordinary (pageable) host memory go through a library-owned
// pinned ring of two chunks: the host copies chunk k into one half while
// the DMA engine moves chunk k−1 out of the other, so the input crosses
// PCIe at pinned-memory speed with the host copy hidden behind it.  The
// host copy itself is split over a small pool of persistent threads (one
// thread copies at a fraction of the socket's memory bandwidth).
#define LBR_RING_CHUNK ((size_t)8 << 20)

class CopyPool {
   public:
    explicit CopyPool(unsigned workers) {
        for (unsigned i = 0; i < workers; ++i) std::thread([this, i] { work(i + 1); }).detach();
        n_threads_ = workers + 1;
    }
    // dst[0, n) = src[0, n), split into n_threads_ slices; returns when all are done
    void copy(char* dst, const char* src, size_t n) {
        const size_t per = ((n + n_threads_ - 1) / n_threads_ + 63) & ~(size_t)63;
        if (n_threads_ == 1 || n < ((size_t)1 << 20)) {
            memcpy(dst, src, n);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(m_);
            dst_ = dst;
            src_ = src;
            n_ = n;
            per_ = per;
            pending_ = n_threads_ - 1;
            ++gen_;
        }
        cv_.notify_all();
        memcpy(dst, src, std::min(per, n));
        std::unique_lock<std::mutex> lk(m_);
        done_.wait(lk, [this] { return pending_ == 0; });
    }

   private:
    void work(unsigned id) {
        unsigned seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> lk(m_);
            cv_.wait(lk, [&] { return gen_ != seen; });
            seen = gen_;
            char* d = dst_;
            const char* s = src_;
            const size_t n = n_, per = per_, lo = id * per;
            lk.unlock();
            if (lo < n) memcpy(d + lo, s + lo, std::min(per, n - lo));
            lk.lock();
            if (--pending_ == 0) done_.notify_one();
        }
    }
    std::mutex m_;
    std::condition_variable cv_, done_;
    char* dst_ = nullptr;
    const char* src_ = nullptr;
    size_t n_ = 0, per_ = 0;
    unsigned gen_ = 0, n_threads_ = 1;
    int pending_ = 0;
};

static std::mutex g_up_mu;
static CopyPool* g_copy_pool = nullptr;   // never destroyed: its threads are detached and idle at exit
static char* g_ring = nullptr;
static hipEvent_t g_ring_ev[2] = {nullptr, nullptr};
static bool g_ring_busy[2] = {false, false};

// ------------------------------------------------------------------ dispatch table
typedef int (*decode_fn)(const OpNode*, Step*);

static decode_fn decoder_for(int op) {
    switch (op) {
        case OP_RELU: case OP_EXP: case OP_TANH: case OP_POW: case OP_GELU:
        case OP_RSQRT: case OP_SILU: case OP_NEG: case OP_COS: case OP_SIN:
            return decode_unary;
        case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV:
            return decode_binary;
        case OP_MAX: case OP_SUM:
            return decode_reduce;
        case OP_SOFTMAX:
            return decode_softmax;
        case OP_MATMUL: case OP_MATMUL_ADD:
            return decode_matmul;
        case OP_RESHAPE:
            return decode_reshape;
        case OP_TRANSPOSE:
            return decode_transpose;
        case OP_SLICE:
            return decode_slice;
        case OP_EMBEDDING:
            return decode_embedding;
        case OP_CAT:
            return decode_cat;
        case OP_LAYERNORM:
            return decode_layernorm;
        case OP_RMSNORM:
            return decode_rmsnorm;
        case OP_FUSED_BIAS_RELU:
            return decode_bias_relu;
        case OP_ATTENTION:
            return decode_attention;
        case OP_GATED_ACT:
            return decode_gated_act;
        default:
            return nullptr;  // OP_PERMUTE has no kernel, as in the reference
    }
}

int lbr_node_check(const OpNode* n, int index) {
    if (n->n_inputs < 0 || n->n_inputs > MAX_INPUTS || n->n_dims < 0 || n->n_dims > MAX_DIMS) {
        lbr_set_error("executor: node %d has n_inputs=%d n_dims=%d", index, n->n_inputs, n->n_dims);
        return LBR_ERR_INVALID;
    }
    if (n->elem_size != 1 && n->elem_size != 2 && n->elem_size != 4 && n->elem_size != 8) {
        lbr_set_error("executor: node %d has elem_size %d", index, n->elem_size);
        return LBR_ERR_INVALID;
    }
    long long total = 1;
    for (int i = 0; i < n->n_dims; ++i) {
        if (n->out_shape[i] < 0) {
            lbr_set_error("executor: node %d has a negative dim", index);
            return LBR_ERR_INVALID;
        }
        // 2^40 elements is more than any device holds; the bound (on the nonzero dims, so
        // that it holds for every subset of them) keeps every product of dims, and of dims
        // with one of the op's extras (each < 2^31), inside 64 bits
        if (n->out_shape[i] > 0 && total > LBR_MAX_ELEMENTS / n->out_shape[i]) {
            lbr_set_error("executor: node %d has more than 2^40 elements", index);
            return LBR_ERR_INVALID;
        }
        if (n->out_shape[i] > 0) total *= n->out_shape[i];
    }
    return LBR_OK;
}

static int decode_node(const OpNode* n, int index, Step* s) {
    memset(s, 0, sizeof(*s));
    s->node_index = index;
    s->n_nodes = 1;
    decode_fn d = decoder_for(n->op);
    if (!d) {
        lbr_set_error("executor: unknown op %d (node %d)", n->op, index);
        return LBR_ERR_UNSUPPORTED;
    }
    if (int rc = lbr_node_check(n, index)) return rc;
    s->n_in = n->n_inputs;
    int rc = d(n, s);
    if (rc != LBR_OK) {
        char tmp[512];
        snprintf(tmp, sizeof(tmp), "node %d (op %d): %s", index, n->op, g_err);
        lbr_set_error("%s", tmp);
    }
    return rc;
}

// ------------------------------------------------------------------ plan
struct lbr_plan {
    std::vector<Step> steps;
    int n_nodes = 0;
    std::vector<int> node_step;  // node → its step, −1 inside a fused run after its first node
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void* ws = nullptr;          // shared step workspace (split-K partial sums)
    void* relay = nullptr;       // attention outputs moved off their inputs (lbr_relay_ok)
    void* head_relay = nullptr;  // Q/K head outputs moved off a GEMM's input (relay_head_outputs)
    void* gated_relay = nullptr; // gated-pair outputs moved off their GEMM's input (relay_gated_outputs)
};

static void free_plan(lbr_plan* p) {
    if (p->exec) (void)hipGraphExecDestroy(p->exec);
    if (p->graph) (void)hipGraphDestroy(p->graph);
    if (p->ws) (void)hipFree(p->ws);
    if (p->relay) (void)hipFree(p->relay);
    if (p->head_relay) (void)hipFree(p->head_relay);
    if (p->gated_relay) (void)hipFree(p->gated_relay);
    delete p;
}

// Deferred attentions whose output only the next GEMM reads write into one
// plan-owned buffer instead (the steps run in order, and each GEMM consumes
// the buffer before the next attention writes it): a split attention's cut
// blocks alone then go through the merge kernel, a key-quartered one stores
// its rows directly.
static int relay_attention_outputs(lbr_plan* p, const OpNode* nodes, int n_nodes, const void* const* live_ptr,
                                   const size_t* live_bytes, int n_live) {
    std::vector<size_t> picks;
    size_t need = 0;
    for (size_t i = 0; i + 1 < p->steps.size(); ++i)
        if (lbr_relay_ok(nodes, n_nodes, p->steps[i], p->steps[i + 1], live_ptr, live_bytes, n_live)) {
            picks.push_back(i);
            const Step& a = p->steps[i];
            need = std::max(need, (size_t)(a.i[0] * a.i[1] * a.i[2]) * sizeof(float));
        }
    if (picks.empty()) return LBR_OK;
    HIP_TRY(hipMalloc(&p->relay, need));
    for (size_t i : picks) {
        p->steps[i].out = p->relay;
        p->steps[i].i[14] = 0;
        // the deferred names are "<kernel>[+v][+transpose]+defer"
        const char* nm = p->steps[i].name;
        const bool v = strstr(nm, "+v") != nullptr, t = strstr(nm, "+transpose") != nullptr;
        p->steps[i].name = lbr_attn_step_name(p->steps[i], v, t, 2);
        p->steps[i + 1].in[0] = p->relay;
    }
    return LBR_OK;
}

// Q/K head outputs that a GEMM's head-prologue epilogue would write over the
// GEMM's own input A (lbr_merge_gemm_head_prologue sets Step::i[27] to the
// ATTENTION node that alone reads them, + 1): one buffer of the plan's own takes
// them, and that attention's step reads Q and K there.  One buffer serves every
// layer: the steps run in order, and each attention has read its Q and K before
// the next such GEMM writes.
static int relay_head_outputs(lbr_plan* p) {
    auto bytes = [](const Step& g, int part) {
        return part < g.i[18] ? ((size_t)(g.i[0] * g.i[22 + part] * 128) * sizeof(float) + 255) / 256 * 256 : 0;
    };
    std::vector<std::pair<size_t, size_t>> picks;
    size_t need = 0;
    for (size_t gi = 0; gi < p->steps.size(); ++gi) {
        const Step& g = p->steps[gi];
        if (g.i[18] <= 0 || g.i[27] <= 0) continue;
        const int node = (int)g.i[27] - 1;
        size_t ai = gi + 1;
        while (ai < p->steps.size() &&
               !(p->steps[ai].node_index <= node && node < p->steps[ai].node_index + p->steps[ai].n_nodes))
            ++ai;
        if (ai >= p->steps.size() || p->steps[ai].in[0] != g.in[4] ||
            (g.i[18] == 2 && p->steps[ai].in[1] != g.in[5])) {
            lbr_set_error("lbr_plan_create: the attention that reads head outputs of GEMM node %d is not node %d's "
                          "step", g.node_index, node);
            return LBR_ERR_INVALID;
        }
        picks.push_back({gi, ai});
        need = std::max(need, bytes(g, 0) + bytes(g, 1));
    }
    if (picks.empty()) return LBR_OK;
    HIP_TRY(hipMalloc(&p->head_relay, need));
    for (const auto& pa : picks) {
        Step& g = p->steps[pa.first];
        Step& a = p->steps[pa.second];
        g.in[4] = a.in[0] = p->head_relay;
        if (g.i[18] == 2) g.in[5] = a.in[1] = (char*)p->head_relay + bytes(g, 0);
    }
    return LBR_OK;
}

// Gated-pair GEMM steps whose output the planner put over the GEMM's own input
// A (GEMM_GATED with FusedRun::relay_out, Step::i[28]): one buffer of the plan's
// own takes the output, and the GEMM right after, its only reader, reads A there
// (one buffer for every layer: the steps run in order).
static int relay_gated_outputs(lbr_plan* p) {
    std::vector<size_t> picks;
    size_t need = 0;
    for (size_t i = 0; i < p->steps.size(); ++i) {
        const Step& s = p->steps[i];
        if (s.fuse_kind != LBR_FUSE_GEMM_GATED || s.i[28] != 1) continue;
        if (i + 1 >= p->steps.size() || p->steps[i + 1].in[0] != s.out || !p->steps[i + 1].name ||
            strncmp(p->steps[i + 1].name, "gemm_", 5) != 0) {
            lbr_set_error("lbr_plan_create: the gated GEMM at node %d is not followed by the GEMM reading its "
                          "output as A", s.node_index);
            return LBR_ERR_INVALID;
        }
        picks.push_back(i);
        need = std::max(need, (size_t)(s.i[0] * s.i[32]) * sizeof(float));
    }
    if (picks.empty()) return LBR_OK;
    HIP_TRY(hipMalloc(&p->gated_relay, need));
    for (size_t i : picks) {
        p->steps[i].out = p->gated_relay;
        p->steps[i + 1].in[0] = p->gated_relay;
    }
    return LBR_OK;
}

// Keys in fragment-major order (lbr_frag_keys_ok): a key-quartered attention
// whose K only its own step reads gets it from the head-scattering GEMM that
// writes it in the order the attention's K loads take it, whole cache lines
// per load instead of half lines.
static void fragment_keys(lbr_plan* p, const OpNode* nodes, int n_nodes, const void* const* live_ptr,
                          const size_t* live_bytes, int n_live) {
    for (size_t a = 0; a < p->steps.size(); ++a) {
        Step& at = p->steps[a];
        if (!at.name || strncmp(at.name, "attn_fwd_kq", 11) != 0 || at.i[15] != 1) continue;
        for (size_t g = a; g-- > 0;) {
            Step& gm = p->steps[g];
            if (!gm.name || strncmp(gm.name, "gemm_", 5) != 0 || gm.i[19] <= 0) continue;
            int k = -1;
            for (int q = 0; q < gm.i[19] && q < 4; ++q)
                if (gm.in[4 + q] == at.in[1]) k = q;
            if (k < 0) continue;
            if (lbr_frag_keys_ok(nodes, n_nodes, gm, k, at, live_ptr, live_bytes, n_live)) {
                gm.i[5] |= 1LL << k;
                at.i[16] = 1;
            }
            break;
        }
    }
}

static void run_steps(const std::vector<Step>& steps, hipStream_t st) {
    for (const Step& s : steps) s.run(s, st);
}

static bool bad_live(const void* const* live_ptr, const size_t* live_bytes, int n_live) {
    return n_live < 0 || (n_live > 0 && (!live_ptr || !live_bytes));
}

// Measured tiles of the workloads' GEMM steps (MI355X): where timing each step
// in its plan (every tile, and K splits of 1 to 8 ranges) found a faster tile
// than the model's.  A listed step (same step name and M, N, K) takes its
// tile, and its number of K ranges when `ks` > 0, without timing, so plans
// come out the same run to run; the model's pick holds for every other step.
// Every tile sums each output's K terms in the same order: the tile never
// changes a result bit; another number of K ranges sums the ranges' partial
// sums instead (a step whose reduce carries a norm keeps its ranges).
struct TunedTile {
    const char* step;
    long long M, N, K;
    const char* tile;
    int ks;   // K ranges; 0: the step's own
};
static const TunedTile kTunedTiles[] = {
    // GPT-2-width block (512 rows; µs for the listed tile against the model's)
    {"gemm_dma_f32_nt+heads", 512, 2304, 768, "32x160", 0},      // QKV: 24.6 against 26.6 (32x48)
    {"gemm_dma_f32_nt+tin+resid+layernorm", 512, 768, 768, "32x96", 0},   // O proj + LN2 (2 ranges): 12.7 against 14.0 (64x64)
    {"gemm_dma_f32_nt+tin+resid", 512, 768, 768, "32x64", 1},    // O proj, LN apart: 12.2 against 14.1 (64x64, 2 ranges)
    {"gemm_dma_f32_nt+act", 512, 3072, 768, "32x64", 0},         // FFN1: 25.6 against 27.5 (32x48)
    {"gemm_dma_f32_nt+resid", 512, 768, 3072, "32x96", 2},       // FFN2: 28.2 against 30.4 (64x64, 8 ranges)
    // GPT-2 body and LM (1024 rows)
    {"gemm_dma_f32_nt+heads", 1024, 2304, 768, "32x96", 0},      // QKV: 34.9 against 43.3 (32x48s4)
    {"gemm_dma_f32_nt+resid+layernorm", 1024, 768, 768, "32x96", 0},   // O proj + LN: 19.6 against 22.2
    {"gemm_dma_f32_nt+resid", 1024, 768, 768, "32x96", 1},       // O proj (LM): 15.0 against 18.0 (64x64)
};

// The tiles (and K ranges) of kTunedTiles, before the plan's workspace is
// sized; marks the steps it set.  Skipped under LBR_GEMM_AUTOTUNE=0 or 2 and
// under a tile or K split forced by LBR_GEMM_TILE / LBR_GEMM_KSPLIT.
static void table_tiles(std::vector<Step>& steps, std::vector<char>* tabled) {
    tabled->assign(steps.size(), 0);
    const char* env = getenv("LBR_GEMM_AUTOTUNE");
    const int mode = env ? atoi(env) : -1;
    if (mode == 0 || mode == 2 || getenv("LBR_GEMM_TILE") || getenv("LBR_GEMM_KSPLIT")) return;
    for (size_t i = 0; i < steps.size(); ++i) {
        Step& s = steps[i];
        if (!s.name || strncmp(s.name, "gemm_dma_f32", 12) != 0 || !s.i[14] || s.i[3] != 1) continue;
        for (const TunedTile& t : kTunedTiles) {
            if (strcmp(s.name, t.step) != 0 || s.i[0] != t.M || s.i[1] != t.N || s.i[2] != t.K) continue;
            const int tile = gemm_dma_tile_by_name(t.tile);
            Step u = s;
            if (tile < 0 || !gemm_dma_retile(&u, tile) || (t.ks > 0 && !gemm_dma_set_ksplit(&u, t.ks))) continue;
            s = u;
            (*tabled)[i] = 1;
        }
    }
}

// Tile timing at plan creation (after table_tiles).  LBR_GEMM_AUTOTUNE=1 times
// every small one-batch, unsplit DMA GEMM step the table did not set
// (2^24 to 2^34 flops: larger ones run on the big tiles, which the model ranks
// well; smaller ones last a few µs, which launch gaps would swamp) over every
// tile its launcher family has — one warm-up launch, then three timed batches
// of three launches, the fastest batch counting — and a tile at least 3% faster
// than the model's choice replaces it; LBR_GEMM_AUTOTUNE=2 ignores the table
// (to regenerate it); unset or 0, or a tile forced by LBR_GEMM_TILE, times
// nothing.  The ranges a timed step writes are saved first and restored after,
// so plan creation leaves memory as it found it.
static int autotune_gemms(std::vector<Step>& steps, const std::vector<char>& tabled) {
    const char* env = getenv("LBR_GEMM_AUTOTUNE");
    const int mode = env ? atoi(env) : -1;
    if (getenv("LBR_GEMM_TILE")) return LBR_OK;
    if (mode < 1) return LBR_OK;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    void* save = nullptr;
    size_t save_cap = 0;
    hipError_t err = hipEventCreate(&e0);
    if (err == hipSuccess) err = hipEventCreate(&e1);
    for (size_t i = 0; i < steps.size() && err == hipSuccess; ++i) {
        Step& s = steps[i];
        if (!s.name || strncmp(s.name, "gemm_dma_f32", 12) != 0 || tabled[i] || s.i[10] > 1) continue;
        int cand[32];
        const int nc = gemm_dma_tune_candidates(s, cand, 32);
        // below 2^24 flops a launch lasts a few µs and the timing measures launch
        // gaps, not the tile: the model's choice stands
        const double flops = 2.0 * (double)s.i[0] * (double)s.i[1] * (double)s.i[2];
        if (nc < 2 || flops >= 17179869184.0 || flops < 16777216.0) continue;
        void* wp[4];
        size_t wb[4], total = 0;
        const int nw = gemm_dma_written(s, wp, wb, 4);
        for (int k = 0; k < nw; ++k) total += wb[k];
        if (total > save_cap) {
            if (save) (void)hipFree(save);
            save = nullptr;
            save_cap = 0;
            if ((err = hipMalloc(&save, total)) != hipSuccess) break;
            save_cap = total;
        }
        for (int k = 0, off = 0; k < nw && err == hipSuccess; off += (int)(wb[k] / sizeof(float)), ++k)
            err = hipMemcpyAsync((float*)save + off, wp[k], wb[k], hipMemcpyDeviceToDevice, g_stream);
        const int model_tile = (int)s.i[14] - 1;
        int best = model_tile;
        float best_ms = 0.f, model_ms = 0.f;
        for (int c = 0; c < nc && err == hipSuccess; ++c) {
            Step t = s;
            if (!gemm_dma_retile(&t, cand[c])) continue;
            t.run(t, g_stream);   // warm-up
            // the fastest of three timed batches of three launches
            float ms = 0.f;
            for (int rep = 0; rep < 3 && err == hipSuccess; ++rep) {
                err = hipEventRecord(e0, g_stream);
                for (int r = 0; r < 3 && err == hipSuccess; ++r) t.run(t, g_stream);
                if (err == hipSuccess) err = hipEventRecord(e1, g_stream);
                if (err == hipSuccess) err = hipEventSynchronize(e1);
                if (err == hipSuccess) err = hipGetLastError();
                float rms = 0.f;
                if (err == hipSuccess) err = hipEventElapsedTime(&rms, e0, e1);
                if (err == hipSuccess && (rep == 0 || rms < ms)) ms = rms;
            }
            if (err != hipSuccess) break;
            if (cand[c] == model_tile) model_ms = ms;
            if (best_ms == 0.f || ms < best_ms) {
                best_ms = ms;
                best = cand[c];
            }
        }
        if (err != hipSuccess) break;
        if (best != model_tile && model_ms > 0.f && best_ms < 0.97f * model_ms) gemm_dma_retile(&s, best);
        for (int k = 0, off = 0; k < nw && err == hipSuccess; off += (int)(wb[k] / sizeof(float)), ++k)
            err = hipMemcpyAsync(wp[k], (float*)save + off, wb[k], hipMemcpyDeviceToDevice, g_stream);
    }
    if (err == hipSuccess) err = hipStreamSynchronize(g_stream);
    if (save) (void)hipFree(save);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (err != hipSuccess) {
        lbr_set_error("lbr_plan_create: GEMM tile timing failed: %s", hipGetErrorString(err));
        return LBR_ERR_HIP;
    }
    return LBR_OK;
}

// Decode every node (so each is validated exactly as without fusion), then
// replace the fused runs by their steps; capture a hipGraph if asked.
// The host half of plan creation: decode every node, find the fused runs, build
// their steps and join steps (no device call).  The plan's steps and node map
// are filled; on an error they are left partial.
static int build_steps(lbr_plan* p, const OpNode* nodes, int n_nodes, bool fuse, const void* const* live_ptr,
                       const size_t* live_bytes, int n_live) {
    p->n_nodes = n_nodes;
    std::vector<Step> decoded((size_t)n_nodes);
    for (int i = 0; i < n_nodes; ++i) {
        int rc = decode_node(&nodes[i], i, &decoded[i]);
        if (rc) return rc;
    }
    std::vector<FusedRun> runs;
    if (fuse) {
        int rc = lbr_find_fusions(nodes, n_nodes, live_ptr, live_bytes, n_live, &runs);
        if (rc) return rc;
    }
    p->node_step.assign((size_t)n_nodes, -1);
    size_t r = 0;
    for (int i = 0; i < n_nodes;) {
        p->node_step[i] = (int)p->steps.size();
        if (r < runs.size() && runs[r].first == i) {
            Step s;
            int rc = lbr_fused_step(nodes, runs[r], &s);
            if (rc) return rc;
            s.fuse_kind = runs[r].kind;
            i += runs[r].count;
            ++r;
            // the K prologue right after the Q prologue of a layer joins its launch
            if (r < runs.size() && runs[r].first == i && runs[r].kind == LBR_FUSE_HEAD_PROLOGUE) {
                Step s2;
                rc = lbr_fused_step(nodes, runs[r], &s2);
                if (rc) return rc;
                s2.fuse_kind = runs[r].kind;
                if (lbr_merge_head_steps(&s, s2)) {
                    i += runs[r].count;
                    ++r;
                }
            }
            // an attention output projection whose output only feeds the MLP
            // right after it runs inside the MLP's kernel
            if (r < runs.size() && runs[r].first == i && runs[r].kind == LBR_FUSE_MLP &&
                s.fuse_kind == LBR_FUSE_TRANSPOSE_GEMM) {
                Step s2;
                rc = lbr_fused_step(nodes, runs[r], &s2);
                if (rc) return rc;
                s2.fuse_kind = runs[r].kind;
                if (lbr_merge_proj_mlp(&s2, s)) {
                    s = s2;
                    i += runs[r].count;
                    ++r;
                }
            }
            // a norm of this GEMM's split-K output runs in its reduce kernel
            if (i < n_nodes && (r >= runs.size() || runs[r].first != i) && lbr_merge_reduce_norm(&s, decoded[i])) ++i;
            // the Q/K head prologues of a plain GEMM's output run in its epilogue
            if (s.fuse_kind == LBR_FUSE_HEAD_PROLOGUE && !p->steps.empty() &&
                lbr_merge_gemm_head_prologue(&p->steps.back(), s, nodes, n_nodes, live_ptr, live_bytes, n_live)) {
                for (int k = s.node_index; k < s.node_index + s.n_nodes; ++k) p->node_step[k] = -1;
                continue;
            }
            p->steps.push_back(s);
        } else {
            // an ADD whose sum only a norm right after it reads first (a position
            // table, say): the norm kernel adds
            Step nstep;
            if (fuse && i + 1 < n_nodes && (r >= runs.size() || runs[r].first != i + 1)) {
                nstep = decoded[i + 1];
                if (lbr_merge_add_norm(&nstep, decoded[i], &nodes[i])) {
                    p->steps.push_back(nstep);
                    i += 2;
                    continue;
                }
            }
            p->steps.push_back(decoded[i]);
            ++i;
        }
    }
    return LBR_OK;
}

static int check_kernels(const lbr_plan& p) {
    for (size_t i = 0; i < p.steps.size(); ++i)
        if (!p.steps[i].run) {
            lbr_set_error("lbr_plan_create: step %zu (node %d) has no kernel", i, p.steps[i].node_index);
            return LBR_ERR_INVALID;
        }
    return LBR_OK;
}

static int create_plan(const OpNode* nodes, int n_nodes, int use_graph, bool fuse, const void* const* live_ptr,
                       const size_t* live_bytes, int n_live, lbr_plan** out_plan) {
    lbr_plan* p = new lbr_plan();
    int rc = build_steps(p, nodes, n_nodes, fuse, live_ptr, live_bytes, n_live);
    if (rc) {
        delete p;
        return rc;
    }
    rc = !fuse ? LBR_OK : relay_attention_outputs(p, nodes, n_nodes, live_ptr, live_bytes, n_live);
    if (!rc && fuse) rc = relay_head_outputs(p);
    if (!rc && fuse) rc = relay_gated_outputs(p);
    if (!rc && fuse) fragment_keys(p, nodes, n_nodes, live_ptr, live_bytes, n_live);
    if (!rc) rc = check_kernels(*p);
    std::vector<char> tabled;
    if (!rc) table_tiles(p->steps, &tabled);
    if (!rc) rc = assign_workspace(p->steps, &p->ws);
    if (!rc) rc = autotune_gemms(p->steps, tabled);
    if (rc) {
        free_plan(p);
        return rc;
    }
    if (use_graph && !p->steps.empty()) {
        hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            run_steps(p->steps, g_stream);
            e = hipStreamEndCapture(g_stream, &p->graph);
        }
        if (e == hipSuccess) e = hipGraphInstantiate(&p->exec, p->graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            lbr_set_error("lbr_plan_create: graph capture failed: %s", hipGetErrorString(e));
            free_plan(p);
            return LBR_ERR_HIP;
        }
    }
    *out_plan = p;
    return LBR_OK;
}

extern "C" {

const char* lbr_last_error(void) { return g_err; }

const char* lbr_version(void) { return LBR_VERSION; }

int lbr_opnode_size(void) { return (int)sizeof(OpNode); }

int lbr_init(int device) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_stream && g_device == device) return LBR_OK;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= device || device < 0) {
        lbr_set_error("lbr_init: no HIP device %d (found %d)", device, count);
        return LBR_ERR_NO_DEVICE;
    }
    HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        lbr_set_error("lbr_init: device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
        return LBR_ERR_NO_DEVICE;
    }
    HIP_TRY(mlp_prepare_device());
    // this device's copy of the no-allocation scratch array (see lbr_execute_noalloc)
    if (device < LBR_MAX_DEVICES && !g_scratch_dev[device]) {
        void* ptr = nullptr;
        HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) {
            lbr_set_error("lbr_init: no device address for the scratch array on device %d", device);
            return LBR_ERR_HIP;
        }
        g_scratch_dev[device] = ptr;
    }
    if (g_stream) {
        (void)hipStreamDestroy(g_stream);
        g_stream = nullptr;
    }
    HIP_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    g_device = device;
    g_cus = prop.multiProcessorCount;
    return LBR_OK;
}

int lbr_op_supported(int op) { return decoder_for(op) != nullptr; }

int lbr_device_alloc(size_t bytes, void** out_ptr) {
    if (!out_ptr) {
        lbr_set_error("lbr_device_alloc: null out_ptr");
        return LBR_ERR_INVALID;
    }
    int rc = ensure_init();
    if (rc) return rc;
    *out_ptr = nullptr;
    HIP_TRY(hipMalloc(out_ptr, bytes ? bytes : 256));
    return LBR_OK;
}

int lbr_device_free(void* ptr) {
    if (!ptr) return LBR_OK;
    HIP_TRY(hipFree(ptr));
    return LBR_OK;
}

int lbr_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return LBR_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return LBR_OK;
}

int lbr_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return LBR_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return LBR_OK;
}

int lbr_host_alloc(size_t bytes, void** out_ptr) {
    if (!out_ptr) {
        lbr_set_error("lbr_host_alloc: null out_ptr");
        return LBR_ERR_INVALID;
    }
    int rc = ensure_init();
    if (rc) return rc;
    *out_ptr = nullptr;
    HIP_TRY(hipHostMalloc(out_ptr, bytes ? bytes : 256, hipHostMallocDefault));
    return LBR_OK;
}

int lbr_host_free(void* ptr) {
    if (!ptr) return LBR_OK;
    HIP_TRY(hipHostFree(ptr));
    return LBR_OK;
}

int lbr_upload_async(void* dst, const void* src, size_t bytes) {
    if (bytes && (!dst || !src)) {
        lbr_set_error("lbr_upload_async: null pointer");
        return LBR_ERR_INVALID;
    }
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return LBR_OK;
    std::lock_guard<std::mutex> lock(g_up_mu);
    if (!g_ring) {
        void* ring = nullptr;
        HIP_TRY(hipHostMalloc(&ring, 2 * LBR_RING_CHUNK, hipHostMallocDefault));
        for (hipEvent_t& e : g_ring_ev) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        const unsigned hw = std::thread::hardware_concurrency();
        g_copy_pool = new CopyPool(std::min(7u, hw > 1 ? hw - 1 : 0u));
        g_ring = (char*)ring;
    }
    size_t off = 0;
    for (int k = 0; off < bytes; ++k) {
        const int slot = k & 1;
        const size_t n = std::min(LBR_RING_CHUNK, bytes - off);
        if (g_ring_busy[slot]) HIP_TRY(hipEventSynchronize(g_ring_ev[slot]));   // its last DMA is done
        char* stage = g_ring + slot * LBR_RING_CHUNK;
        g_copy_pool->copy(stage, (const char*)src + off, n);
        HIP_TRY(hipMemcpyAsync((char*)dst + off, stage, n, hipMemcpyHostToDevice, g_stream));
        HIP_TRY(hipEventRecord(g_ring_ev[slot], g_stream));
        g_ring_busy[slot] = true;
        off += n;
    }
    return LBR_OK;
}

int lbr_download_async(void* dst, const void* src, size_t bytes) {
    if (bytes && (!dst || !src)) {
        lbr_set_error("lbr_download_async: null pointer");
        return LBR_ERR_INVALID;
    }
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return LBR_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    return LBR_OK;
}

int lbr_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return LBR_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return LBR_OK;
}

int lbr_memset(void* dst, int value, size_t bytes) {
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return LBR_OK;
    HIP_TRY(hipMemsetAsync(dst, value, bytes, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return LBR_OK;
}

int lbr_execute(const OpNode* nodes, int n_nodes) {
    if (n_nodes < 0 || (n_nodes > 0 && !nodes)) {
        lbr_set_error("lbr_execute: bad node array");
        return LBR_ERR_INVALID;
    }
    int rc = ensure_init();
    if (rc) return rc;
    std::vector<Step> steps((size_t)n_nodes);
    size_t need = 0;
    for (int i = 0; i < n_nodes; ++i) {
        rc = decode_node(&nodes[i], i, &steps[i]);
        if (rc) return rc;
        need = steps[i].ws_bytes > need ? steps[i].ws_bytes : need;
    }
    std::lock_guard<std::mutex> lock(g_exec_mu);
    void* ws = nullptr;
    rc = exec_workspace(need, &ws);
    if (rc) return rc;
    for (Step& s : steps) s.ws = ws;
    run_steps(steps, g_stream);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        lbr_set_error("lbr_execute: %s", hipGetErrorString(e));
        return LBR_ERR_HIP;
    }
    return LBR_OK;
}

// lbr_execute without any allocation: the workspace is this device's copy
// of `scratch` (address resolved by lbr_init), the node array is decoded
// twice into one Step on the stack (every node checked, and the workspace
// need summed up, before the first launch), and the call needs lbr_init to
// have run on this device.  Every call on the device shares the array; the
// library serialises the calls (g_exec_mu) and each ends with a stream
// synchronisation.
int lbr_execute_noalloc(const OpNode* nodes, int n_nodes) {
    if (n_nodes < 0 || (n_nodes > 0 && !nodes)) {
        lbr_set_error("lbr_execute_noalloc: bad node array");
        return LBR_ERR_INVALID;
    }
    if (!g_stream || g_device < 0 || g_device >= LBR_MAX_DEVICES || !g_scratch_dev[g_device]) {
        lbr_set_error("lbr_execute_noalloc: call lbr_init(device) first (this entry point does no set-up)");
        return LBR_ERR_INVALID;
    }
    Step s;
    size_t need = 0;
    for (int i = 0; i < n_nodes; ++i) {
        const int rc = decode_node(&nodes[i], i, &s);
        if (rc) return rc;
        need = s.ws_bytes > need ? s.ws_bytes : need;
    }
    if (need > LBR_SCRATCH_BYTES) {
        lbr_set_error("lbr_execute_noalloc: the nodes need %zu bytes of workspace; the no-allocation scratch "
                      "holds %zu (use lbr_execute or a plan)", need, (size_t)LBR_SCRATCH_BYTES);
        return LBR_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lock(g_exec_mu);
    void* ws = g_scratch_dev[g_device];
    for (int i = 0; i < n_nodes; ++i) {
        const int rc = decode_node(&nodes[i], i, &s);
        if (rc) return rc;
        if (s.ws_bytes > LBR_SCRATCH_BYTES) {   // the same nodes: cannot differ from the first pass
            lbr_set_error("lbr_execute_noalloc: node %d needs %zu bytes of workspace", i, s.ws_bytes);
            return LBR_ERR_INVALID;
        }
        s.ws = s.ws_bytes ? ws : nullptr;
        s.run(s, g_stream);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        lbr_set_error("lbr_execute_noalloc: %s", hipGetErrorString(e));
        return LBR_ERR_HIP;
    }
    return LBR_OK;
}

// The reference's entry point by its own name (csrc/executor.c:458), so its
// ctypes binding (runtime/executor/common.py:157-159: argtypes
// [POINTER(COpNode), c_int], restype None) resolves unchanged.  Same work as
// lbr_execute; the int status is there for callers that read it.
int execute(const OpNode* nodes, int n_nodes) { return lbr_execute(nodes, n_nodes); }

int lbr_execute_workspace_bytes(size_t* out_bytes) {
    if (!out_bytes) {
        lbr_set_error("lbr_execute_workspace_bytes: null out_bytes");
        return LBR_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lock(g_exec_mu);
    *out_bytes = g_exec_ws_bytes;
    return LBR_OK;
}

int lbr_plan_create(const OpNode* nodes, int n_nodes, int use_graph, lbr_plan** out_plan) {
    if (!out_plan || n_nodes < 0 || (n_nodes > 0 && !nodes)) {
        lbr_set_error("lbr_plan_create: bad arguments");
        return LBR_ERR_INVALID;
    }
    *out_plan = nullptr;
    int rc = ensure_init();
    if (rc) return rc;
    return create_plan(nodes, n_nodes, use_graph, false, nullptr, nullptr, 0, out_plan);
}

int lbr_plan_create_fused(const OpNode* nodes, int n_nodes, int use_graph, const void* const* live_ptr,
                          const size_t* live_bytes, int n_live, lbr_plan** out_plan) {
    if (!out_plan || n_nodes < 0 || (n_nodes > 0 && !nodes) || bad_live(live_ptr, live_bytes, n_live)) {
        lbr_set_error("lbr_plan_create_fused: bad arguments");
        return LBR_ERR_INVALID;
    }
    *out_plan = nullptr;
    int rc = ensure_init();
    if (rc) return rc;
    return create_plan(nodes, n_nodes, use_graph, true, live_ptr, live_bytes, n_live, out_plan);
}

int lbr_fusion_windows(const OpNode* nodes, int n_nodes, const void* const* live_ptr, const size_t* live_bytes,
                       int n_live, lbr_window* out, int cap, int* n_out) {
    if (!n_out || n_nodes < 0 || (n_nodes > 0 && !nodes) || cap < 0 || (cap > 0 && !out) ||
        bad_live(live_ptr, live_bytes, n_live)) {
        lbr_set_error("lbr_fusion_windows: bad arguments");
        return LBR_ERR_INVALID;
    }
    std::vector<FusedRun> runs;
    int rc = lbr_find_fusions(nodes, n_nodes, live_ptr, live_bytes, n_live, &runs);
    if (rc) return rc;
    for (size_t k = 0; k < runs.size() && (int)k < cap; ++k) {
        out[k].first = runs[k].first;
        out[k].count = runs[k].count;
        out[k].kind = runs[k].kind;
    }
    *n_out = (int)runs.size();
    return LBR_OK;
}

int lbr_check_nodes(const OpNode* nodes, int n_nodes, int fuse, const void* const* live_ptr,
                    const size_t* live_bytes, int n_live, int* n_steps) {
    if (n_nodes < 0 || (n_nodes > 0 && !nodes) || bad_live(live_ptr, live_bytes, n_live)) {
        lbr_set_error("lbr_check_nodes: bad arguments");
        return LBR_ERR_INVALID;
    }
    lbr_plan p;
    int rc = build_steps(&p, nodes, n_nodes, fuse != 0, live_ptr, live_bytes, n_live);
    // the plan's other host passes that need no device (the relays allocate their
    // buffers, so they are left out: they change pointers, not the steps)
    if (!rc && fuse) fragment_keys(&p, nodes, n_nodes, live_ptr, live_bytes, n_live);
    if (!rc) rc = check_kernels(p);
    if (!rc) {
        std::vector<char> tabled;
        table_tiles(p.steps, &tabled);
    }
    if (!rc && n_steps) *n_steps = (int)p.steps.size();
    return rc;
}

int lbr_plan_num_steps(const lbr_plan* p) { return p ? (int)p->steps.size() : 0; }

int lbr_plan_step_info(const lbr_plan* p, int step, int* first_node, int* n_nodes, int* kind) {
    if (!p || step < 0 || step >= (int)p->steps.size()) {
        lbr_set_error("lbr_plan_step_info: bad arguments");
        return LBR_ERR_INVALID;
    }
    if (first_node) *first_node = p->steps[step].node_index;
    if (n_nodes) *n_nodes = p->steps[step].n_nodes;
    if (kind) *kind = p->steps[step].fuse_kind;
    return LBR_OK;
}

int lbr_plan_step_args(const lbr_plan* p, int step, long long* ints_out, int cap) {
    const int n = (int)(sizeof(Step::i) / sizeof(Step::i[0]));
    if (!p || step < 0 || step >= (int)p->steps.size() || cap < 0 || (cap > 0 && !ints_out)) {
        lbr_set_error("lbr_plan_step_args: bad arguments");
        return LBR_ERR_INVALID;
    }
    for (int k = 0; k < cap && k < n; ++k) ints_out[k] = p->steps[step].i[k];
    return LBR_OK;
}

int lbr_plan_destroy(lbr_plan* p) {
    if (!p) return LBR_OK;
    free_plan(p);
    return LBR_OK;
}

int lbr_plan_num_nodes(const lbr_plan* p) { return p ? p->n_nodes : 0; }

int lbr_plan_launch(lbr_plan* p) {
    if (!p) {
        lbr_set_error("lbr_plan_launch: null plan");
        return LBR_ERR_INVALID;
    }
    if (p->exec) {
        HIP_TRY(hipGraphLaunch(p->exec, g_stream));
    } else {
        run_steps(p->steps, g_stream);
        HIP_TRY(hipGetLastError());
    }
    return LBR_OK;
}

int lbr_synchronize(void) {
    int rc = ensure_init();
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(g_stream));
    return LBR_OK;
}

int lbr_plan_time(lbr_plan* p, int iters, float* out_ms) {
    if (!p || !out_ms || iters <= 0) {
        lbr_set_error("lbr_plan_time: bad arguments");
        return LBR_ERR_INVALID;
    }
    hipEvent_t a, b;
    HIP_TRY(hipEventCreate(&a));
    HIP_TRY(hipEventCreate(&b));
    HIP_TRY(hipEventRecord(a, g_stream));
    for (int i = 0; i < iters; ++i) {
        int rc = lbr_plan_launch(p);
        if (rc) {
            (void)hipEventDestroy(a);
            (void)hipEventDestroy(b);
            return rc;
        }
    }
    HIP_TRY(hipEventRecord(b, g_stream));
    HIP_TRY(hipEventSynchronize(b));
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *out_ms = ms;
    return LBR_OK;
}

int lbr_plan_profile(lbr_plan* p, int iters, float* out_ms, int n_out) {
    if (!p || !out_ms || iters <= 0 || n_out < p->n_nodes) {
        lbr_set_error("lbr_plan_profile: bad arguments");
        return LBR_ERR_INVALID;
    }
    const size_t n = p->steps.size();
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    // Each step runs `iters` times back to back between one event pair, so the
    // events' own cost (a completion signal and a fresh dispatch per event) is
    // spread over `iters` launches. Eager launches would still leave the GPU idle
    // while the host enqueues the next one; a busy kernel queued first keeps it
    // occupied until they are all enqueued: 40 us of GPU time per launch covers the
    // host's enqueue cost, profilers included. Its length is calibrated once.
    HIP_TRY(hipEventRecord(e0, g_stream));
    hipLaunchKernelGGL(lbr_busy, dim3(1), dim3(64), 0, g_stream, 1 << 16, 0.f, 1.f);
    HIP_TRY(hipEventRecord(e1, g_stream));
    HIP_TRY(hipEventSynchronize(e1));
    HIP_TRY(hipGetLastError());
    float cal_ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&cal_ms, e0, e1));
    const double want_ms = std::max(0.2, 0.04 * (double)iters);
    const double busy = cal_ms > 0.f ? want_ms / cal_ms * (double)(1 << 16) : (double)(1 << 20);
    const int busy_iters = (int)std::min(busy, (double)(1 << 28));
    // A repeated step may read what its own previous launch wrote (an in-place
    // epilogue, an output stored over its input): the values change, the work does
    // not (grids, loop trips and addresses follow shapes; the only data-indexed
    // reads, embedding rows, index graph inputs, which no step writes). One plain
    // pass at the end leaves every buffer as a forward pass leaves it.
    std::vector<double> acc(n, 0.0);
    for (size_t i = 0; i < n; ++i) {
        hipLaunchKernelGGL(lbr_busy, dim3(1), dim3(64), 0, g_stream, busy_iters, 0.f, 1.f);
        HIP_TRY(hipEventRecord(e0, g_stream));
        for (int it = 0; it < iters; ++it) p->steps[i].run(p->steps[i], g_stream);
        HIP_TRY(hipEventRecord(e1, g_stream));
        HIP_TRY(hipEventSynchronize(e1));
        HIP_TRY(hipGetLastError());
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
        acc[i] = ms;
    }
    run_steps(p->steps, g_stream);
    HIP_TRY(hipStreamSynchronize(g_stream));
    HIP_TRY(hipGetLastError());
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    // a step's time goes to its first node; the other nodes of a fused run get 0
    for (int i = 0; i < p->n_nodes; ++i) out_ms[i] = 0.f;
    for (size_t i = 0; i < n; ++i) out_ms[p->steps[i].node_index] = (float)(acc[i] / iters);
    return LBR_OK;
}

int lbr_plan_node_kernel(const lbr_plan* p, int index, char* name_out, int name_cap) {
    if (!p || index < 0 || index >= p->n_nodes || !name_out || name_cap <= 0) {
        lbr_set_error("lbr_plan_node_kernel: bad arguments");
        return LBR_ERR_INVALID;
    }
    const int st = p->node_step[index];
    const char* name = st < 0 ? "fused" : (p->steps[st].name ? p->steps[st].name : "?");
    snprintf(name_out, (size_t)name_cap, "%s", name);
    return LBR_OK;
}

}  // extern "C"
