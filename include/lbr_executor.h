/*
 * lbr_executor.h — C ABI of the MI355X (gfx950) compiled-executor library
 * `liblbr_executor.so`.
 *
 * The library replaces the reference's CPU dispatch loop
 *   void execute(OpNode* nodes, int n_nodes)          csrc/executor.c:458-467
 * loaded by ctypes in runtime/executor/common.py:148-163 and called from
 * runtime/executor/compiled.py:87/91.  The node record and the op codes are
 * byte-identical to csrc/runtime.h:11-69 (mirrored by COpNode,
 * runtime/executor/common.py:125-141), so the Python host layer builds the
 * same node array it builds for the CPU executor; the only difference is
 * that every pointer in inputs[] / output is a device address (arena base +
 * planner offset, a device-resident weight, or a fixed device staging
 * buffer for a graph input).
 *
 * Differences from the reference boundary, all deliberate:
 *   - every call returns an int status (LBR_OK = 0) instead of abort();
 *     lbr_last_error() returns the message of the most recent failure on
 *     the calling thread;
 *   - device memory is owned by the library (lbr_device_alloc/free), since
 *     the caller's numpy arena cannot be read by the GPU;
 *   - a node array can be turned into a plan once (validated, decoded into
 *     kernel launches, optionally captured into a hipGraph) and replayed.
 *
 * Threading contract (same as the reference): one caller at a time per
 * plan; all work is issued on the library's single stream.
 */
#ifndef LBR_EXECUTOR_H
#define LBR_EXECUTOR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Op codes — identical values to csrc/runtime.h:11-55 and runtime/ir.py:36-90. */
enum OpType {
    OP_RELU = 100, OP_EXP = 101, OP_TANH = 102, OP_POW = 103, OP_GELU = 104,
    OP_RSQRT = 105, OP_SILU = 106, OP_NEG = 107, OP_COS = 108, OP_SIN = 109,

    OP_ADD = 200, OP_SUB = 201, OP_MUL = 202, OP_DIV = 203,

    OP_MAX = 300, OP_SUM = 301, OP_SOFTMAX = 302,

    OP_MATMUL = 400,

    OP_RESHAPE = 500, OP_TRANSPOSE = 501, OP_PERMUTE = 502, OP_SLICE = 503,
    OP_EMBEDDING = 504, OP_CAT = 505,

    OP_LAYERNORM = 600, OP_RMSNORM = 601,

    OP_MATMUL_ADD = 1000, OP_FUSED_BIAS_RELU = 1001, OP_ATTENTION = 1002,
    OP_GATED_ACT = 1003
};

#define MAX_INPUTS 12
#define MAX_DIMS   24

/* Node record — layout identical to csrc/runtime.h:60-69 (312 bytes on
 * x86-64).  `extra` holds the op-specific integers packed by the host
 * layer's extras packers (runtime/ops.py:137-329); floats are bit-cast. */
typedef struct {
    int   op;
    int   n_inputs;
    void* inputs[MAX_INPUTS];
    void* output;
    int   out_shape[MAX_DIMS];
    int   n_dims;
    int   elem_size;
    int   extra[MAX_DIMS];
} OpNode;

/* Status codes. */
#define LBR_OK              0
#define LBR_ERR_INVALID     1   /* malformed node / argument             */
#define LBR_ERR_UNSUPPORTED 2   /* op code with no device kernel          */
#define LBR_ERR_HIP         3   /* a HIP runtime call failed              */
#define LBR_ERR_NO_DEVICE   4   /* no usable gfx950 device                */

/* Message of the most recent failure on this thread ("" if none). */
const char* lbr_last_error(void);

/* Library version string. */
const char* lbr_version(void);

/* sizeof(OpNode) as compiled into the library (312), so the ctypes mirror
 * can be checked at load time. */
int lbr_opnode_size(void);

/* Select `device`, check it is a gfx950 part and create the library stream.
 * Idempotent for the same device.  Every other entry point that touches the
 * GPU calls it with device 0 if it has not been called. */
int lbr_init(int device);

/* 1 if op code `op` has a device kernel (the dispatch-table coverage the
 * host layer's compiled-dispatch validator checks; runtime/validation/
 * execution.py:16-34 keeps the CPU executor's set). */
int lbr_op_supported(int op);

/* Device memory owned by the library.  lbr_device_alloc returns memory
 * aligned to 256 bytes. */
int lbr_device_alloc(size_t bytes, void** out_ptr);
int lbr_device_free(void* ptr);
int lbr_memcpy_h2d(void* dst_device, const void* src_host, size_t bytes);
int lbr_memcpy_d2h(void* dst_host, const void* src_device, size_t bytes);
int lbr_memcpy_d2d(void* dst_device, const void* src_device, size_t bytes);
int lbr_memset(void* dst_device, int value, size_t bytes);

/* Pinned (page-locked) host memory, which the DMA engines read and write
 * directly: the destination of choice for lbr_download_async. */
int lbr_host_alloc(size_t bytes, void** out_ptr);
int lbr_host_free(void* ptr);

/* Enqueue a host→device copy on the library stream from ordinary host
 * memory.  The bytes go through a library-owned pinned ring of two 8 MiB
 * chunks: the host copies one chunk (split over a few threads) while the
 * previous one is in flight.  When the call returns `src` may be reused;
 * the device copy completes in stream order (before a later plan launch). */
int lbr_upload_async(void* dst_device, const void* src_host, size_t bytes);

/* Enqueue a device→host copy on the library stream (asynchronous when
 * dst_host is pinned memory from lbr_host_alloc); lbr_synchronize waits. */
int lbr_download_async(void* dst_host, const void* src_device, size_t bytes);

/* Drop-in for execute(OpNode*, int) (csrc/executor.c:458-467): launch every
 * node in order on the library stream and wait for completion.  Returns
 * LBR_ERR_UNSUPPORTED for an op without a kernel (where the reference
 * aborts), LBR_ERR_INVALID for a node whose fields do not fit its op.
 * Every node is decoded and checked before the first launch.  Kernels that
 * need a workspace (GEMM split-K partial sums, attention key-range
 * partials) share one library-owned device block that grows to the largest
 * need seen and is kept for later calls; calls are serialised. */
int lbr_execute(const OpNode* nodes, int n_nodes);

/* The reference's symbol itself, `void execute(OpNode* nodes, int n_nodes)`
 * (csrc/executor.c:458), bound by name in runtime/executor/common.py:157-159
 * with restype None.  Same behaviour as lbr_execute; the returned status is
 * ignored by that binding and can be read by callers that declare c_int. */
int execute(const OpNode* nodes, int n_nodes);

/* Bytes of the one-shot workspace currently held (0 before any call that
 * needed one). */
int lbr_execute_workspace_bytes(size_t* out_bytes);

/* lbr_execute without any allocation.  No counterpart in the reference
 * (its execute never allocates, because its kernels need no device
 * workspace); it is for callers that cannot allocate device memory: code
 * that must not call hipMalloc/hipFree (serving loops, harnesses that forbid
 * it).  The workspace is a fixed 48 MiB device array inside the library,
 * one copy per GPU, held until the process ends; its address is resolved by
 * lbr_init, which must have run on the current device first (this call does
 * no set-up).  Node arrays whose kernels need more workspace than that (GEMM
 * split-K partial sums, attention key-range partials) are rejected with
 * LBR_ERR_INVALID before anything is launched (48 MiB holds the 40 MiB the
 * largest benchmark workload, the Qwen3-4B body at S=1024, needs).  All calls on one GPU share
 * that array and keep the last call's contents (nothing relies on them);
 * calls overlapping on one GPU would race on it, so the library serialises
 * them, and each call waits for its work like lbr_execute. */
int lbr_execute_noalloc(const OpNode* nodes, int n_nodes);

/* Plans: validate and decode the node array once; launches reuse the
 * decoded kernel arguments.  With use_graph != 0 the launch sequence is
 * captured into a hipGraph at creation and every lbr_plan_launch replays it
 * (the device pointers in the nodes must stay valid and unchanged). */
typedef struct lbr_plan lbr_plan;
int lbr_plan_create(const OpNode* nodes, int n_nodes, int use_graph,
                    lbr_plan** out_plan);
int lbr_plan_destroy(lbr_plan* plan);
int lbr_plan_num_nodes(const lbr_plan* plan);

/* Enqueue one forward pass on the library stream (asynchronous). */
int lbr_plan_launch(lbr_plan* plan);

/* Wait for all work on the library stream. */
int lbr_synchronize(void);

/* Time `iters` back-to-back lbr_plan_launch calls with hipEvents recorded
 * on the library stream; *out_ms = total elapsed milliseconds. */
int lbr_plan_time(lbr_plan* plan, int iters, float* out_ms);

/* Per-node device time: runs each step of the plan `iters` times back to back
 * between one hipEvent pair (on the library stream, behind a short arithmetic-only
 * kernel that keeps the GPU busy while the host enqueues them), then one plain
 * pass, and writes the mean milliseconds per launch of node i's step to out_ms[i]
 * (0 for the later nodes of a fused run; n_out >= number of nodes). */
int lbr_plan_profile(lbr_plan* plan, int iters, float* out_ms, int n_out);

/* Short name of the kernel that executes node `index` (for reports); nodes
 * inside a fused run after its first report "fused". */
int lbr_plan_node_kernel(const lbr_plan* plan, int index, char* name_out,
                         int name_cap);

/* ---------------------------------------------------------------------
 * Peephole fusion.  No counterpart in the reference (its executor runs one
 * kernel per node, csrc/executor.c:458-467); the node array stays exactly
 * as the host layer builds it.  At plan creation runs of consecutive nodes
 * that one kernel can execute are replaced by that kernel when every value
 * the run produces, other than its final outputs, is dead afterwards (not
 * read by a later node before being overwritten, not inside a live-out
 * range) and no final output overlaps memory the fused kernel reads.
 * Live-out ranges are the byte ranges the caller reads after a launch (the
 * graph outputs); final outputs hold what the unfused nodes would write.
 * ------------------------------------------------------------------- */
#define LBR_FUSE_NONE          0
#define LBR_FUSE_GEMM_RESID    1  /* MATMUL[_ADD] → ADD(C, R): R added in the GEMM epilogue     */
#define LBR_FUSE_GEMM_HEADS    2  /* MATMUL[_ADD] → k × (SLICE → [ADD bias] → TRANSPOSE(S,H)):
                                     the epilogue writes each column range as [B, H, S, hd]     */
#define LBR_FUSE_HEAD_PROLOGUE 3  /* SLICE → [ADD bias] → [RMSNORM] → TRANSPOSE(S,H) → [RoPE]
                                     (7-node rotate-half window) as one kernel                  */
#define LBR_FUSE_ATTN_TRANSPOSE 4 /* ATTENTION → TRANSPOSE(H,S): the attention kernel writes
                                     its output as [B, S, H, hd]                                */
#define LBR_FUSE_GEMM_ACT      5  /* MATMUL[_ADD] → RELU | GELU | SILU: the activation is
                                     applied in the GEMM epilogue                               */
#define LBR_FUSE_GEMM_GATED    6  /* MATMUL[_ADD] (N = 2F) → SLICE [0,F) → SLICE [F,2F) →
                                     GATED_ACT: the GEMM pairs gate and up columns in each tile
                                     and writes act(gate)·up as [M, F]                           */
#define LBR_FUSE_TRANSPOSE_GEMM 7 /* TRANSPOSE(H,S) of [B,H,S,hd] → MATMUL[_ADD] → [ADD(C, R)]:
                                     the GEMM reads its A operand in the untransposed layout
                                     (and adds R in its epilogue)                               */
#define LBR_FUSE_ATTN_SLICED_V  8 /* SLICE(C, last dim) → TRANSPOSE(S,H) → ATTENTION with it as
                                     V → [TRANSPOSE(H,S)]: the attention kernel reads V rows
                                     straight from C's columns (and writes [B, S, H, hd])        */
#define LBR_FUSE_NORM_GEMM     10 /* RMSNORM | LAYERNORM → GEMM: the GEMM reads the norm's input
                                     and applies the norm on the fly (DMA kernel, one batch,
                                     no K split, K ≤ 4096); the other GEMM kinds take the same
                                     prologue when a norm precedes them (their run then starts
                                     at the norm)                                               */
#define LBR_FUSE_MLP           11 /* [RMSNORM | LAYERNORM →] MATMUL[_ADD] → RELU | GELU | SILU →
                                     MATMUL[_ADD] [→ ADD(y, R)], small: one kernel per 16 rows
                                     with both weights staged in LDS (each ≤ 64 KiB) and the
                                     hidden activations in LDS (D, H and the output width
                                     multiples of 16, each wavefront's share of a weight ≤ 16
                                     float4 a lane, 2·M·(H·D + D2·H) ≤ 2^25 flops)              */
#define LBR_FUSE_ADD_NORM      12 /* ADD (same shape, or a [P, N] row block broadcast over the
                                      leading dims) → RMSNORM | LAYERNORM: the norm kernel adds,
                                      writes the sum and normalises it (a plan step join; not
                                      reported by lbr_fusion_windows)                      */
#define LBR_FUSE_GEMM_HEAD_PROLOGUE 13 /* MATMUL[_ADD] → the HEAD_PROLOGUE run(s) of its output
                                      (the Q and K of a layer, head dim 128): the GEMM runs
                                      64×128 tiles, one head each, and normalises, rotates
                                      and stores each head in its epilogue (a plan step join;
                                      not reported by lbr_fusion_windows)                  */

typedef struct {
    int first;   /* index of the run's first node */
    int count;   /* nodes in the run              */
    int kind;    /* LBR_FUSE_*                    */
} lbr_window;

/* The runs lbr_plan_create_fused would fuse, without touching a device (the
 * node pointers are only compared, never dereferenced).  Writes up to `cap`
 * windows and their total count to *n_out. */
int lbr_fusion_windows(const OpNode* nodes, int n_nodes,
                       const void* const* live_ptr, const size_t* live_bytes,
                       int n_live, lbr_window* out, int cap, int* n_out);

/* The host half of lbr_plan_create (fuse = 0) or lbr_plan_create_fused
 * (fuse = 1) without touching a device: every record checked (counts within
 * its arrays, elem_size 1, 2, 4 or 8, no negative dim, at most 2^40
 * elements), every node decoded and its extras checked against its shape,
 * the fused runs found and their steps and step joins built, the key layout
 * and the tile table applied (not the relay buffers, which are allocated).
 * Returns the
 * status and error those calls would report for a malformed or unsupported
 * node array, and the number of kernel steps in *n_steps (may be NULL).
 * Choices that depend on the device take 256 CUs before lbr_init.  No
 * counterpart in the reference (its execute(), csrc/executor.c:409-452, trusts
 * the host layer's records): for callers that build node arrays themselves
 * and want them checked before a device is touched. */
int lbr_check_nodes(const OpNode* nodes, int n_nodes, int fuse,
                    const void* const* live_ptr, const size_t* live_bytes,
                    int n_live, int* n_steps);

/* lbr_plan_create with peephole fusion (live-out ranges as above). */
int lbr_plan_create_fused(const OpNode* nodes, int n_nodes, int use_graph,
                          const void* const* live_ptr,
                          const size_t* live_bytes, int n_live,
                          lbr_plan** out_plan);

/* Kernel steps of a plan (≤ nodes) and the nodes step `step` covers. */
int lbr_plan_num_steps(const lbr_plan* plan);
int lbr_plan_step_info(const lbr_plan* plan, int step, int* first_node,
                       int* n_nodes, int* kind);

/* x / d by the multiply-shift divisor the attention key-range split and the
 * head prologue index with (lbr_fast_divisor, lbr_fdiv), computed on the host
 * exactly as the kernels do (x < 2^31, d >= 1): test support, no counterpart
 * in the reference. */
unsigned lbr_fast_div(unsigned x, unsigned d);

/* The (head, 16-row query block) each workgroup of the key-quartered
 * attention kernel runs, for `bh` heads of `seq` rows (causal or not) on
 * `cus` CUs: workgroup w gets heads_out[w], blocks_out[w] (w < cap).  The
 * same assignment and index arithmetic as the launch, run on the host: test
 * support, no counterpart in the reference.  Returns the grid size. */
int lbr_attn_kq_grid(long long bh, int seq, int causal, int cus,
                     int* heads_out, int* blocks_out, int cap);

/* Name ("64x64", "32x48s4" ...) of DMA GEMM tile index `tile` (the value
 * lbr_plan_step_args reports in [14], less one), "" for other indices: for
 * reports, no counterpart in the reference. */
const char* lbr_gemm_tile_name(int tile);

/* The decoded integer launch arguments of step `step` (up to `cap` of them,
 * 40 at most), for tests and reports.  Their meaning is the kernel's: for
 * the attention kernel [6] = causal blocks folded in pairs, [7] = key-range
 * split workgroups (0: no split), [14] = deferred output, [15] = the
 * key-quartered 16-row kernel; for the GEMM
 * kernels [10] = K ranges, [14] = DMA tile index + 1 (0: register-staged
 * kernel). */
int lbr_plan_step_args(const lbr_plan* plan, int step, long long* ints_out,
                       int cap);

#ifdef __cplusplus
}
#endif

#endif /* LBR_EXECUTOR_H */
