// lbr_fusion.h — fused runs of consecutive OpNodes found at plan creation
// (fusion.hip) and the decoded launch record that replaces each run.
#pragma once

#include <vector>

#include "lbr_device.h"

struct FusedRun {
    int first = 0, count = 0, kind = LBR_FUSE_NONE;
    // GEMM_HEADS: split k takes C columns [col_begin[k], col_begin[k] + width[k])
    int n_split = 0;
    int col_begin[5] = {0, 0, 0, 0, 0};
    int width[4] = {0, 0, 0, 0};
    const void* dst[4] = {nullptr, nullptr, nullptr, nullptr};
    const void* sbias[4] = {nullptr, nullptr, nullptr, nullptr};   // [0] = HEAD_PROLOGUE bias
    int Hs[4] = {0, 0, 0, 0};                                       // [0] = HEAD_PROLOGUE heads
    int B = 0, S = 0, hd = 0;
    // GEMM_RESID
    const void* resid = nullptr;
    const void* out = nullptr;
    // HEAD_PROLOGUE
    const void* src = nullptr;
    long long ld = 0;
    const void* norm_w = nullptr;
    float eps = 0.f;
    bool rope = false;
    const void* cos = nullptr;
    const void* sin = nullptr;
    long long cst[3] = {0, 0, 0}, sst[3] = {0, 0, 0};
    // GEMM_ACT: LBR_ACT_* applied to C
    int act = 0;
    // GEMM_GATED: F output columns, gate half at columns [gate_base, gate_base + F),
    // GATED_ACT's act code and bias (`out` is the GATED_ACT output)
    int gF = 0, gate_base = 0, gact = 0;
    const void* gbias = nullptr;
    // GEMM_GATED: the output lies over the GEMM's A (the planner's reuse of a dead
    // input), and only the A of the GEMM right after reads it: the plan writes it into a
    // buffer of its own and points that GEMM there (relay_gated_outputs)
    bool relay_out = false;
    // TRANSPOSE_GEMM: the GEMM's A in head layout [B, H, S, hd] at `src`; `resid` /
    // `out` set when the residual ADD is fused as well (B, S, hd and Hs[0] = H)
    // ATTN_SLICED_V: the ATTENTION is node first + attn_at; V rows come from `src`
    // ([B·S, ld] row-major) at column col_begin[0], Hs[1] K/V heads; Hs[0] query
    // heads; `out` is the attention output or, when the run ends with its
    // TRANSPOSE(H,S), that transpose's output
    int attn_at = 0;
    // ATTN_TRANSPOSE / ATTN_SLICED_V: the final output lies over memory the attention
    // reads; taken only under the key-range split, whose merge kernel then writes every
    // row (after the split kernel has finished reading)
    bool defer = false;
    // MLP: the run's GEMM1 is node first (+1 with a norm), its activation `act`,
    // GEMM2 after it, `resid` / `out` the fused residual ADD's other input and output
    // (`out` is GEMM2's output without it)
    // Norm prologue (any GEMM kind, and NORM_GEMM alone): node `first` is a RMSNORM /
    // LAYERNORM over the K columns of `norm_src` whose output was the GEMM's A; the
    // GEMM is node first + 1 and reads norm_src instead (LBR_NORM_*, 0: none)
    int norm = 0;
    const void* norm_src = nullptr;
    const void* norm_g = nullptr;
    const void* norm_b = nullptr;
    float norm_eps = 0.f;
};

// Fusable runs of nodes[0..n) in stream order; live-out ranges are the
// graph outputs the caller reads after the plan runs.
int lbr_find_fusions(const OpNode* nodes, int n, const void* const* live_ptr, const size_t* live_bytes, int n_live,
                     std::vector<FusedRun>* out);

// Launch record of one fused run.
int lbr_fused_step(const OpNode* nodes, const FusedRun& f, Step* s);

// Joins the HEAD_PROLOGUE step b (the run right after a's) into a as the
// second part of one float4 launch, when both are the same kernel over the
// same source rows and tables and neither output overlaps what the other
// reads; false leaves a unchanged.
bool lbr_merge_head_steps(Step* a, const Step& b);

// Joins the HEAD_PROLOGUE step h into the plain DMA GEMM step g right before it
// that writes h's source (head dim 128): g's 64×128 tiles apply the prologue in
// their epilogue; false leaves g unchanged.
bool lbr_merge_gemm_head_prologue(Step* g, const Step& h, const OpNode* nodes, int n, const void* const* live_ptr,
                                  const size_t* live_bytes, int n_live);

// Joins the TRANSPOSE_GEMM step t (the run right before u's) into the MLP
// step u when u's input is t's output: u's kernel then computes that input
// (and still writes it); false leaves u unchanged.
bool lbr_merge_proj_mlp(Step* u, const Step& t);

// Joins the decoded RMSNORM / LAYERNORM step n right after the split-K
// residual GEMM step g that produces its input: g's reduce kernel then also
// writes the normalised rows; false leaves g unchanged.
bool lbr_merge_reduce_norm(Step* g, const Step& n);

// Joins the decoded ADD step a (node add) into the decoded RMSNORM /
// LAYERNORM step n right after it that normalises the sum (same-shape or
// row-block broadcast ADD): n's kernel then adds, writes the sum and
// normalises it; false leaves n unchanged.
bool lbr_merge_add_norm(Step* n, const Step& a, const OpNode* add);

// Whether the deferred split attention step `at` can write into a buffer of
// the plan's own that the DMA GEMM step `gm` right after it reads as A (its
// only reader): the attention's store is then not deferred.
bool lbr_relay_ok(const OpNode* nodes, int n, const Step& at, const Step& gm, const void* const* live_ptr,
                  const size_t* live_bytes, int n_live);

// GEMM step `gm` may write head split k fragment-major for the key-quartered
// attention step `at` that reads it as K (and nothing else reads it).
bool lbr_frag_keys_ok(const OpNode* nodes, int n, const Step& gm, int k, const Step& at, const void* const* live_ptr,
                      const size_t* live_bytes, int n_live);

// Byte range [*lo, *hi) input k of node nd reads (per op, from its shape and
// extras); *hi = UINTPTR_MAX when the node does not fix it.
void lbr_input_extent(const OpNode* nd, int k, unsigned long long* lo, unsigned long long* hi);


