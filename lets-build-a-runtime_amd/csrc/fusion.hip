// fusion.hip — peephole fusion over the unchanged OpNode array.
//
// The node stream the host layer builds (runtime/executor/nodes.py, the
// reference's compiled.py:50-157) is kept exactly; at plan creation the
// library looks for short runs of consecutive nodes that one kernel can do
// and launches that kernel in their place.  A run is fused only when
//   * its nodes match one of the patterns below exactly (ops, extras,
//     pointer chaining, shapes), and
//   * every value the run produces except its final outputs is dead: no
//     later node reads it before the memory is overwritten, and it does not
//     overlap a caller-declared live-out range (the graph outputs), and
//   * no final output overlaps memory the fused kernel reads (the planner
//     may place a node's output over its dead input; one fused kernel reads
//     and writes with a different index map, so that reuse is refused).
// Final outputs land at the planner's offsets with the values the unfused
// nodes would write (same operation order for every rounding step; the only
// reassociation is the sum of squares inside RMSNorm).
//
// Patterns:
//   GEMM_RESID  MATMUL[_ADD] → ADD(same shape, C, R): R is added in the GEMM
//               epilogue (the residual adds of every pre-norm block).
//   GEMM_HEADS  MATMUL[_ADD] → k × (SLICE last dim → [ADD bias row] →
//               TRANSPOSE(S,H)): the GEMM epilogue writes each column range
//               straight into its [B, H, S, hd] output (merged QKV
//               projections, passes.py merge_parallel_matmuls).
//   HEAD_PROLOGUE  SLICE last dim → [ADD bias row] → [RMSNORM over hd] →
//               TRANSPOSE(S,H) → [RoPE: MUL cos, SLICE, SLICE, NEG, CAT,
//               MUL sin, ADD]: hd/4 lanes per (token, head) row, one float4
//               each (a whole wavefront per row when rows are not 16-byte
//               aligned).
//   ATTN_TRANSPOSE  ATTENTION → TRANSPOSE(H,S): the attention kernel stores
//               its rows straight into [B, S, H, hd].
//   ATTN_SLICED_V  SLICE(C, last dim) → TRANSPOSE(S,H) → ATTENTION taking it
//               as V → [TRANSPOSE(H,S)]: the attention kernel reads the V
//               rows from C's column range with C's row stride (the V of a
//               merged QKV projection whose Q and K went through norm/RoPE).
//   GEMM_ACT    MATMUL[_ADD] → RELU | GELU | SILU: the activation runs in the
//               GEMM epilogue (the FFN's first projection).
//   GEMM_GATED  MATMUL[_ADD] with 2F columns → SLICE [0,F) and SLICE [F,2F)
//               → GATED_ACT(gate, [bias], up): the GEMM fetches gate and up
//               weight rows interleaved in blocks of 16 columns, so each lane
//               holds both values of an output element, and writes
//               act(gate)·up as [M, F] (the merged gate/up projection of a
//               SiLU-gated FFN).
//   TRANSPOSE_GEMM  TRANSPOSE(H,S) of the attention output [B,H,S,hd] →
//               MATMUL[_ADD] → [ADD(C, R)]: the GEMM reads its A operand in
//               the [B,H,S,hd] layout (a 32-wide K step stays inside one head
//               when hd is a multiple of 32, or covers 32/hd whole heads when hd
//               divides 32) and adds R in its epilogue —
//               the O projection and its residual without the transpose.
#include "lbr_device.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

#include "lbr_fusion.h"

namespace {

// ------------------------------------------------------------ device kernel

struct HeadArgs {
    const float* src;         // sliced tensor (rows × ld), columns col0 ..
    long long ld;
    int col0;
    int B, S, H, hd;
    const float* bias;        // [H·hd] or null
    const float* w;           // RMSNorm weight [hd] or null
    float eps;
    const float* cos;         // RoPE tables, element (b,h,s,d) at b·c[0]+h·c[1]+s·c[2]+d
    const float* sin;
    long long cst[3], sst[3];
    float* out;               // [B, H, S, hd]
    long long rows;           // B·S·H
};

template <int VPL, bool BIAS, bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void head_prologue(HeadArgs a) {
    const int lane = threadIdx.x & 63;
    const long long row = blockIdx.x * 4LL + (threadIdx.x >> 6);   // (b·S + s)·H + h
    if (row >= a.rows) return;
    const int h = (int)(row % a.H);
    const long long bs = row / a.H;
    const int s = (int)(bs % a.S), b = (int)(bs / a.S);
    const float* __restrict__ x = a.src + bs * a.ld + a.col0 + (long long)h * a.hd;
    const long long cb = ROPE ? b * a.cst[0] + h * a.cst[1] + s * a.cst[2] : 0;
    const long long sb = ROPE ? b * a.sst[0] + h * a.sst[1] + s * a.sst[2] : 0;
    // every load (row, bias, norm weight, RoPE tables) issues before the
    // reduction, so the row's memory latencies overlap
    float v[VPL], wv[VPL], cv[VPL], sv[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int d = lane + 64 * j;
        v[j] = x[d];
        if (NORM) wv[j] = a.w[d];
        if (ROPE) {
            cv[j] = a.cos[cb + d];
            sv[j] = a.sin[sb + d];
        }
        if (BIAS) v[j] = v[j] + a.bias[h * a.hd + d];
    }
    if (NORM) {   // norm.c:100-107 order: x · (1/sqrt(Σx²/n + eps)) · w
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < VPL; ++j) ss += v[j] * v[j];
        ss = wave_sum(ss);
        const float scale = 1.0f / sqrtf(ss / a.hd + a.eps);
#pragma unroll
        for (int j = 0; j < VPL; ++j) v[j] = v[j] * scale * wv[j];
    }
    float* __restrict__ o = a.out + (((long long)b * a.H + h) * a.S + s) * a.hd;
    if (ROPE) {   // y = x·cos + rotate_half(x)·sin, rotate_half = cat(−x[half:], x[:half])
        const int half = a.hd / 2;
        float p[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if (VPL >= 2) p[j] = v[j ^ (VPL / 2)];      // half = 64·VPL/2: partner in this lane
            else p[j] = __shfl_xor(v[j], 32, 64);         // hd = 64: partner 32 lanes away
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int d = lane + 64 * j;
            const float rot = d < half ? -p[j] : p[j];
            o[d] = __fadd_rn(__fmul_rn(v[j], cv[j]), __fmul_rn(rot, sv[j]));
        }
    } else {
#pragma unroll
        for (int j = 0; j < VPL; ++j) o[lane + 64 * j] = v[j];
    }
}

// float4 form for 16-byte aligned rows.  A row of HD floats is LPR = HD/4
// lanes holding one float4 each, so one float4 slot of a wavefront covers
// HPS = 64/LPR rows (2 at HD = 128), and each lane holds R slots: a
// wavefront task is R·HPS heads of one token.  Every load of the task (R
// rows, their biases, the norm weight, the RoPE rows) issues before any
// arithmetic; RoPE tables that do not vary over heads are loaded once.  The
// RMSNorm sum over the row's LPR lanes and the rotate-half partner LPR/2
// lanes away (d ± HD/2) move through DPP and row swaps, not LDS.
//
// Up to two parts share a launch: the Q and K prologues of one attention
// layer, sliced from the same projection output with the same RoPE tables.
// Tasks run head group by head group (G0 groups of part 0, then G1 of part
// 1), each over all tokens, so neighbouring wavefronts write neighbouring
// rows of the same heads.
struct HeadPart {
    int col0, H, G;           // first column in the source, heads, tasks per token
    const float* bias;        // [H·hd] or null
    const float* w;           // RMSNorm weight [hd] or null
    float* out;               // [B, H, S, hd]
    float eps;
};

struct HeadArgs4 {
    const float* src;
    long long ld;
    int S, T;                 // tokens per batch, tasks per token (G0 + G1)
    int N_m, N_s, S_m, S_s;   // divisors by the token count and S (lbr_fdiv)
    unsigned tokens, tasks;   // B·S, B·S·T
    const float* cos;
    const float* sin;
    long long cst[3], sst[3];
    bool shared_tables;       // cst[1] == sst[1] == 0: one RoPE row per token
    HeadPart p[2];
};

template <int HD, bool BIAS, bool NORM, bool ROPE, int R>
__global__ __launch_bounds__(256) void head_rows4(HeadArgs4 a) {
    constexpr int LPR = HD / 4;
    constexpr int HPS = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const unsigned task = blockIdx.x * 4u + (unsigned)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (task >= a.tasks) return;   // whole wavefronts leave: shuffles stay inside live ones
    const unsigned rg = lbr_fdiv(task, a.N_m, a.N_s);              // head group of the parts
    const unsigned bs = task - rg * a.tokens;                       // token b·S + s
    const int r = (int)rg;
    const unsigned b = lbr_fdiv(bs, a.S_m, a.S_s);
    const int s = (int)(bs - b * (unsigned)a.S);
    const bool second = r >= a.p[0].G;
    const int col0 = second ? a.p[1].col0 : a.p[0].col0;
    const int H = second ? a.p[1].H : a.p[0].H;
    const float* __restrict__ bias = second ? a.p[1].bias : a.p[0].bias;
    const float* __restrict__ w = second ? a.p[1].w : a.p[0].w;
    float* __restrict__ out = second ? a.p[1].out : a.p[0].out;
    const float eps = second ? a.p[1].eps : a.p[0].eps;
    const int grp = second ? r - a.p[0].G : r;
    const int l = lane % LPR;
    const int d = 4 * l;
    const int h0 = grp * (R * HPS) + lane / LPR;                   // slot k holds head h0 + k·HPS
    const float* __restrict__ x = a.src + (long long)bs * a.ld + col0 + d;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 xv[R], cv[R], sv[R], wv = zero;
#pragma unroll
    for (int k = 0; k < R; ++k) cv[k] = sv[k] = zero;   // read only with ROPE
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int h = h0 + k * HPS;
        xv[k] = h < H ? *reinterpret_cast<const float4*>(x + (long long)h * HD) : zero;
    }
    if (NORM) wv = *reinterpret_cast<const float4*>(w + d);
    if (ROPE) {
        if (a.shared_tables) {
            const float4 c = *reinterpret_cast<const float4*>(a.cos + b * a.cst[0] + s * a.cst[2] + d);
            const float4 sn = *reinterpret_cast<const float4*>(a.sin + b * a.sst[0] + s * a.sst[2] + d);
#pragma unroll
            for (int k = 0; k < R; ++k) {
                cv[k] = c;
                sv[k] = sn;
            }
        } else {
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const int h = min(h0 + k * HPS, H - 1);
                cv[k] = *reinterpret_cast<const float4*>(a.cos + b * a.cst[0] + h * a.cst[1] + s * a.cst[2] + d);
                sv[k] = *reinterpret_cast<const float4*>(a.sin + b * a.sst[0] + h * a.sst[1] + s * a.sst[2] + d);
            }
        }
    }
    if (BIAS) {
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int h = min(h0 + k * HPS, H - 1);
            const float4 bv = *reinterpret_cast<const float4*>(bias + h * HD + d);
            xv[k].x = xv[k].x + bv.x;
            xv[k].y = xv[k].y + bv.y;
            xv[k].z = xv[k].z + bv.z;
            xv[k].w = xv[k].w + bv.w;
        }
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const float4 y = lbr_head_row<LPR, HD>(xv[k], NORM, wv, eps, ROPE, cv[k], sv[k], lane);
        const int h = h0 + k * HPS;
        if (h < H) *reinterpret_cast<float4*>(out + (((long long)b * H + h) * a.S + s) * HD + d) = y;
    }
}

// Step::in[0]=src [1]=bias [2]=w [3]=cos [4]=sin; i[0]=ld [1]=col0 [2]=B
// [3]=S [4]=H [5]=hd [6..8]=cos strides [9..11]=sin strides [12]=rows
// [13]=float4 kernel; f[0]=eps
HeadArgs head_args(const Step& s) {
    HeadArgs a;
    a.src = (const float*)s.in[0];
    a.bias = (const float*)s.in[1];
    a.w = (const float*)s.in[2];
    a.cos = (const float*)s.in[3];
    a.sin = (const float*)s.in[4];
    a.out = (float*)s.out;
    a.ld = s.i[0];
    a.col0 = (int)s.i[1];
    a.B = (int)s.i[2];
    a.S = (int)s.i[3];
    a.H = (int)s.i[4];
    a.hd = (int)s.i[5];
    for (int k = 0; k < 3; ++k) {
        a.cst[k] = s.i[6 + k];
        a.sst[k] = s.i[9 + k];
    }
    a.rows = s.i[12];
    a.eps = s.f[0];
    return a;
}

template <int VPL, bool BIAS, bool NORM, bool ROPE>
void launch_head_prologue(const Step& s, hipStream_t st) {
    const HeadArgs a = head_args(s);
    if (a.rows <= 0) return;
    hipLaunchKernelGGL((head_prologue<VPL, BIAS, NORM, ROPE>), dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, st,
                       a);
}

constexpr int kHeadSlots = 2;   // R: row slots per lane of the float4 kernel

// The float4 kernel's step: the scalar step's fields for part 0, and
// i[14] = parts (1 or 2), i[15] = H, i[16] = col0 of part 1, in[5..7] = its
// bias, weight and output, f[1] = its eps (set by lbr_merge_head_steps).
template <int HD, bool BIAS, bool NORM, bool ROPE>
void launch_head_rows4(const Step& s, hipStream_t st) {
    constexpr int HPT = kHeadSlots * (256 / HD);   // heads per wavefront task
    const long long tokens = s.i[2] * s.i[3];
    if (tokens <= 0 || s.i[4] <= 0) return;
    HeadArgs4 a;
    a.src = (const float*)s.in[0];
    a.ld = s.i[0];
    a.S = (int)s.i[3];
    a.cos = (const float*)s.in[3];
    a.sin = (const float*)s.in[4];
    for (int k = 0; k < 3; ++k) {
        a.cst[k] = s.i[6 + k];
        a.sst[k] = s.i[9 + k];
    }
    a.shared_tables = a.cst[1] == 0 && a.sst[1] == 0;
    const int parts = s.i[14] == 2 ? 2 : 1;
    for (int p = 0; p < 2; ++p) {
        const bool on = p < parts;
        HeadPart& q = a.p[p];
        q.col0 = (int)(p ? s.i[16] : s.i[1]);
        q.H = on ? (int)(p ? s.i[15] : s.i[4]) : 0;
        q.G = (q.H + HPT - 1) / HPT;
        q.bias = (const float*)(p ? s.in[5] : s.in[1]);
        q.w = (const float*)(p ? s.in[6] : s.in[2]);
        q.out = (float*)(p ? (void*)s.in[7] : s.out);
        q.eps = p ? s.f[1] : s.f[0];
    }
    a.T = a.p[0].G + a.p[1].G;
    a.tokens = (unsigned)tokens;
    a.tasks = (unsigned)(tokens * a.T);
    lbr_fast_divisor(a.tokens, &a.N_m, &a.N_s);
    lbr_fast_divisor((unsigned)a.S, &a.S_m, &a.S_s);
    hipLaunchKernelGGL((head_rows4<HD, BIAS, NORM, ROPE, kHeadSlots>), dim3((a.tasks + 3) / 4), dim3(256), 0, st, a);
}

// W = VPL (scalar kernel, 64·VPL = hd) or HD (float4 kernel)
template <int W, bool BIAS, bool VEC>
step_fn pick_hp2(bool norm, bool rope) {
    if constexpr (VEC) {
        if (norm) return rope ? launch_head_rows4<W, BIAS, true, true> : launch_head_rows4<W, BIAS, true, false>;
        return rope ? launch_head_rows4<W, BIAS, false, true> : launch_head_rows4<W, BIAS, false, false>;
    } else {
        if (norm) return rope ? launch_head_prologue<W, BIAS, true, true> : launch_head_prologue<W, BIAS, true, false>;
        return rope ? launch_head_prologue<W, BIAS, false, true> : launch_head_prologue<W, BIAS, false, false>;
    }
}

template <int W, bool VEC>
step_fn pick_hp(bool bias, bool norm, bool rope) {
    return bias ? pick_hp2<W, true, VEC>(norm, rope) : pick_hp2<W, false, VEC>(norm, rope);
}

// ------------------------------------------------------------ matching

struct Rng {
    uintptr_t lo, hi;
};

bool overlap(Rng a, Rng b) { return a.lo < b.hi && b.lo < a.hi; }

Rng out_rng(const OpNode* n) {
    const uintptr_t p = (uintptr_t)n->output;
    return {p, p + (uintptr_t)(node_total(n) * (n->elem_size > 0 ? n->elem_size : 4))};
}

long long prod_dims(const OpNode* n, int lo, int hi) {
    long long r = 1;
    for (int d = lo; d < hi && d < n->n_dims; ++d) r *= n->out_shape[d];
    return r;
}

// Bytes input k of node nd reads: the per-op rule the host layer checks
// before launch (elements from the output shape and the extras, times the
// element size; token ids are int64).  An extent the node does not fix (an
// EMBEDDING table with no row count, an op outside the table) reaches to the
// top of the address space, which can only make the liveness walk refuse
// more.
Rng input_rng(const OpNode* nd, int k) {
    const uintptr_t p = (uintptr_t)nd->inputs[k];
    const long long es = nd->elem_size > 0 ? nd->elem_size : 4;
    const long long total = node_total(nd), last = node_last_dim(nd);
    const long long lead = last ? total / last : 0;
    const int* x = nd->extra;
    long long e = -1;   // elements read; −1: not fixed by the node
    // products of extents, −1 when a factor is negative or the product passes
    // 2^40 elements (no node's operand is that large: the extent is then not fixed)
    auto mul = [](std::initializer_list<long long> f) {
        long long r = 1;
        for (long long v : f) {
            if (v < 0 || (v > 0 && r > LBR_MAX_ELEMENTS / v)) return -1LL;
            r *= v;
        }
        return r;
    };
    auto bcast = [&](int base) {   // [ndim, a strides, b strides, out shape] at extra[base]
        const int nd_ = x[base];
        if (nd_ < 0 || nd_ > (MAX_DIMS - 1 - base) / 3 || k > 1) return -1LL;
        long long span = 1;
        for (int d = 0; d < nd_; ++d) {
            const long long s = x[base + 1 + 2 * nd_ + d];
            if (s == 0) return 0LL;
            const long long t = mul({s - 1, x[base + 1 + k * nd_ + d]});
            if (t < 0 || span > LBR_MAX_ELEMENTS - t) return -1LL;
            span += t;
        }
        return span;
    };
    switch (nd->op) {
        case OP_RELU: case OP_EXP: case OP_TANH: case OP_POW: case OP_GELU: case OP_RSQRT: case OP_SILU:
        case OP_NEG: case OP_COS: case OP_SIN: case OP_SOFTMAX: case OP_RESHAPE:
            e = k == 0 ? total : -1;
            break;
        case OP_ADD:   // modes: 0 bias row, 1 same shape, 2 scalar, 3 broadcast
            e = x[0] == 3 ? bcast(1) : (k == 0 || x[0] == 1) ? total : x[0] == 0 ? last : -1;
            break;
        case OP_SUB: case OP_MUL: case OP_DIV:   // modes: 0 same shape, 1 scalar, 2 broadcast
            e = x[0] == 2 ? bcast(1) : (k == 0 || x[0] == 0) ? total : -1;
            break;
        case OP_MAX: case OP_SUM:
            e = x[0] >= 0 ? mul({prod_dims(nd, 0, x[0]), x[1], prod_dims(nd, x[0], nd->n_dims)}) : mul({x[1], total});
            break;
        case OP_MATMUL: case OP_MATMUL_ADD: {
            const long long K = x[0], N = last;
            const bool b2d = x[2] != 0;
            const long long M = b2d ? lead : (nd->n_dims >= 2 ? nd->out_shape[nd->n_dims - 2] : 1);
            const long long batches = b2d ? 1 : prod_dims(nd, 0, nd->n_dims - 2);
            e = k == 0 ? mul({batches, M, K}) : k == 1 ? mul({batches, N, K}) : k == 2 ? N : -1;
            break;
        }
        case OP_TRANSPOSE:
            e = nd->n_dims == 2 ? mul({x[0], x[1]}) : mul({x[0], x[1], x[2], x[3], x[4]});
            break;
        case OP_SLICE:
            e = mul({x[0], x[1], x[4]});
            break;
        case OP_CAT:
            e = (x[0] >= 0 && k < MAX_DIMS - 1)
                    ? mul({prod_dims(nd, 0, x[0]), x[1 + k], prod_dims(nd, x[0] + 1, nd->n_dims)}) : -1;
            break;
        case OP_EMBEDDING:
            if (k == 0) return {p, p + (uintptr_t)(lead * 8)};
            e = x[1] > 0 ? mul({x[1], last}) : -1;
            break;
        case OP_LAYERNORM: case OP_RMSNORM: case OP_FUSED_BIAS_RELU:
            e = k == 0 ? total : last;
            break;
        case OP_GATED_ACT:
            e = (x[0] != 0 && k == 1) ? last : total;
            break;
        case OP_ATTENTION: {
            const long long S = x[0], hd = x[1], group = x[4] > 0 ? x[4] : 1;
            const long long bh = prod_dims(nd, 0, nd->n_dims - 2), kvh = bh ? (bh - 1) / group + 1 : 0;
            e = k == 0 ? mul({bh, S, hd}) : k <= 2 ? mul({kvh, S, hd}) : (k == 3 && x[3]) ? mul({bh, S, S}) : -1;
            break;
        }
        default:
            break;
    }
    if (e < 0) return {p, UINTPTR_MAX};
    return {p, p + (uintptr_t)(e * es)};
}

Rng rng(const void* p, long long bytes) { return {(uintptr_t)p, (uintptr_t)p + (uintptr_t)bytes}; }

bool is_f32(const OpNode* n) { return n->elem_size == 4; }

// inter minus w.
void subtract(std::vector<Rng>* inter, Rng w) {
    std::vector<Rng> rest;
    for (const Rng& r : *inter) {
        if (!overlap(r, w)) {
            rest.push_back(r);
            continue;
        }
        if (r.lo < w.lo) rest.push_back({r.lo, w.lo});
        if (w.hi < r.hi) rest.push_back({w.hi, r.hi});
    }
    inter->swap(rest);
}

// Values the run [first, end) writes to `inter` are dead once the run is
// over: the parts its own final outputs `outs` overwrite do not count;
// walking the later nodes in order, no input's read extent (input_rng)
// overlaps a part not yet overwritten, and what is left at the end overlaps
// no live-out range.
bool dead_after(const OpNode* nodes, int n, int end, std::vector<Rng> inter, const std::vector<Rng>& outs,
                const std::vector<Rng>& live) {
    for (const Rng& o : outs) subtract(&inter, o);
    for (int j = end; j < n && !inter.empty(); ++j) {
        const OpNode* nd = &nodes[j];
        // ATTENTION's trailing input is the planner's scratch slot (ops.py:437-459):
        // written before it is read, so it is not a read of older values
        const int reads = nd->op == OP_ATTENTION ? 3 + (nd->extra[3] != 0) : nd->n_inputs;
        for (int k = 0; k < reads && k < nd->n_inputs && k < MAX_INPUTS; ++k) {
            const Rng in = input_rng(nd, k);
            for (const Rng& r : inter)
                if (overlap(r, in)) return false;
        }
        subtract(&inter, out_rng(nd));
    }
    for (const Rng& r : inter)
        for (const Rng& l : live)
            if (overlap(r, l)) return false;
    return true;
}

float extra_f(const OpNode* n, int i) { return node_extra_float(n, i); }

struct Rope {
    const void* cos;
    const void* sin;
    long long cst[3], sst[3];
    const void* out;
};

// The 7-node rotate_half RoPE window (HF apply_rotary_pos_emb as exported:
// q·cos, q[..., :half], q[..., half:], −, cat, ·sin, +) on x = [B, H, S, hd].
bool match_rope(const OpNode* nodes, int n, int q, const void* x, int B, int H, int S, int hd, Rope* r,
                std::vector<Rng>* inter) {
    if (q + 7 > n || hd % 2) return false;
    const int half = hd / 2;
    const long long rows = (long long)B * H * S;
    const OpNode* mc = &nodes[q];
    const OpNode* s1 = &nodes[q + 1];
    const OpNode* s2 = &nodes[q + 2];
    const OpNode* ng = &nodes[q + 3];
    const OpNode* ct = &nodes[q + 4];
    const OpNode* ms = &nodes[q + 5];
    const OpNode* ad = &nodes[q + 6];
    for (int k = 0; k < 7; ++k)
        if (!is_f32(&nodes[q + k])) return false;
    const int shape[4] = {B, H, S, hd};
    auto bcast_mul = [&](const OpNode* m, const void* a, long long* st) {
        // SUB/MUL/DIV extras: [2 = broadcast, ndim, a strides, b strides, out shape]
        if (m->op != OP_MUL || m->n_inputs < 2 || m->inputs[0] != a || m->n_dims != 4) return false;
        if (m->extra[0] != 2 || m->extra[1] != 4) return false;
        const long long full[4] = {(long long)H * S * hd, (long long)S * hd, hd, 1};
        for (int d = 0; d < 4; ++d) {
            if (m->out_shape[d] != shape[d] || m->extra[10 + d] != shape[d]) return false;
            const long long as = m->extra[2 + d];
            if (!(as == full[d] || (as == 0 && shape[d] == 1))) return false;
        }
        if (m->extra[6 + 3] != 1) return false;
        for (int d = 0; d < 3; ++d) st[d] = shape[d] == 1 ? 0 : m->extra[6 + d];
        return true;
    };
    if (!bcast_mul(mc, x, r->cst)) return false;
    // SLICE extras [outer, orig, start, len, inner] along the last dim
    if (s1->op != OP_SLICE || s1->inputs[0] != x || s1->extra[0] != rows || s1->extra[1] != hd ||
        s1->extra[2] != 0 || s1->extra[3] != half || s1->extra[4] != 1)
        return false;
    if (s2->op != OP_SLICE || s2->inputs[0] != x || s2->extra[0] != rows || s2->extra[1] != hd ||
        s2->extra[2] != half || s2->extra[3] != half || s2->extra[4] != 1)
        return false;
    if (ng->op != OP_NEG || ng->inputs[0] != s2->output || node_total(ng) != rows * half) return false;
    // CAT extras [dim, sizes...]: cat(−x2, x1) on the last dim
    if (ct->op != OP_CAT || ct->n_inputs != 2 || ct->inputs[0] != ng->output || ct->inputs[1] != s1->output ||
        ct->n_dims != 4 || ct->extra[0] != 3 || ct->extra[1] != half || ct->extra[2] != half)
        return false;
    if (!bcast_mul(ms, ct->output, r->sst)) return false;
    // ADD extras [1] = same shape
    if (ad->op != OP_ADD || ad->n_inputs < 2 || ad->extra[0] != 1 || node_total(ad) != rows * hd) return false;
    const bool ab = ad->inputs[0] == mc->output && ad->inputs[1] == ms->output;
    const bool ba = ad->inputs[0] == ms->output && ad->inputs[1] == mc->output;
    if (!ab && !ba) return false;
    r->cos = mc->inputs[1];
    r->sin = ms->inputs[1];
    r->out = ad->output;
    for (int k = 0; k < 6; ++k) inter->push_back(out_rng(&nodes[q + k]));
    return true;
}

// SLICE(C, last dim) → [ADD bias row] → [RMSNORM] → TRANSPOSE(S,H) → [RoPE]
// starting at node p.  C has `rows` rows of `ld` floats.
struct HeadChain {
    int first = 0, count = 0;
    int col0 = 0, width = 0;
    int B = 0, S = 0, H = 0, hd = 0;
    const void* bias = nullptr;
    const void* norm_w = nullptr;
    float eps = 0.f;
    bool rope = false;
    Rope rp{};
    const void* out = nullptr;
    Rng out_r{};
    std::vector<Rng> inter;   // values written by the chain other than `out`
};

bool match_head_chain(const OpNode* nodes, int n, int p, const void* C, long long rows, int ld, bool norm_rope,
                      HeadChain* hc) {
    const OpNode* sl = &nodes[p];
    if (sl->op != OP_SLICE || sl->n_inputs < 1 || sl->inputs[0] != C || !is_f32(sl)) return false;
    if (sl->extra[0] != rows || sl->extra[1] != ld || sl->extra[4] != 1) return false;
    hc->first = p;
    hc->col0 = sl->extra[2];
    hc->width = sl->extra[3];
    hc->inter.clear();
    hc->inter.push_back(out_rng(sl));
    const void* cur = sl->output;
    int q = p + 1;
    if (q < n && nodes[q].op == OP_ADD && nodes[q].n_inputs >= 2 && nodes[q].inputs[0] == cur &&
        nodes[q].extra[0] == 0 && is_f32(&nodes[q]) && node_last_dim(&nodes[q]) == hc->width) {
        hc->bias = nodes[q].inputs[1];
        cur = nodes[q].output;
        hc->inter.push_back(out_rng(&nodes[q]));
        ++q;
    }
    int norm_hd = 0;
    if (norm_rope && q < n && nodes[q].op == OP_RMSNORM && nodes[q].n_inputs >= 2 && nodes[q].inputs[0] == cur &&
        is_f32(&nodes[q]) && nodes[q].n_dims >= 2) {
        norm_hd = node_last_dim(&nodes[q]);
        if (norm_hd <= 0 || hc->width % norm_hd) return false;
        hc->norm_w = nodes[q].inputs[1];
        hc->eps = extra_f(&nodes[q], 0);
        cur = nodes[q].output;
        hc->inter.push_back(out_rng(&nodes[q]));
        ++q;
    }
    // N-D TRANSPOSE extras [outer, A, middle, B, inner]: [B, S, 1, H, hd]
    if (q >= n) return false;
    const OpNode* tr = &nodes[q];
    if (tr->op != OP_TRANSPOSE || tr->n_inputs < 1 || tr->inputs[0] != cur || tr->n_dims != 4 || !is_f32(tr))
        return false;
    const int B = tr->extra[0], S = tr->extra[1], H = tr->extra[3], hd = tr->extra[4];
    if (tr->extra[2] != 1 || (long long)B * S != rows || (long long)H * hd != hc->width) return false;
    if (norm_hd && norm_hd != hd) return false;
    if (tr->out_shape[0] != B || tr->out_shape[1] != H || tr->out_shape[2] != S || tr->out_shape[3] != hd)
        return false;
    hc->B = B;
    hc->S = S;
    hc->H = H;
    hc->hd = hd;
    cur = tr->output;
    ++q;
    hc->rope = false;
    if (norm_rope) {
        std::vector<Rng> ri;
        Rope r{};
        if (match_rope(nodes, n, q, cur, B, H, S, hd, &r, &ri)) {
            hc->inter.push_back(out_rng(tr));
            hc->inter.insert(hc->inter.end(), ri.begin(), ri.end());
            hc->rope = true;
            hc->rp = r;
            cur = r.out;
            q += 7;
        }
    }
    hc->out = cur;
    hc->out_r = out_rng(&nodes[q - 1]);
    hc->count = q - p;
    return true;
}

// Extent of a GEMM's inputs (A, B, bias) for the overlap test.
// GEMM_GATED over its own A: the gated output y (at ptr) can move to a buffer of
// the plan's own when node `next` is a GEMM that reads it as A, no other read sees
// y's bytes before they are overwritten, and y is not live-out.
bool gated_relay_ok(const OpNode* nodes, int n, int next, const void* ptr, Rng y, const std::vector<Rng>& live) {
    const char* e = getenv("LBR_GATED_RELAY");
    if (e && atoi(e) == 0) return false;
    if (next >= n || (nodes[next].op != OP_MATMUL && nodes[next].op != OP_MATMUL_ADD) || nodes[next].inputs[0] != ptr)
        return false;
    std::vector<Rng> rest{y};
    for (int j = next; j < n && !rest.empty(); ++j) {
        const OpNode* nd = &nodes[j];
        const int reads = nd->op == OP_ATTENTION ? 3 + (nd->extra[3] != 0) : nd->n_inputs;
        for (int k = 0; k < reads && k < nd->n_inputs && k < MAX_INPUTS; ++k) {
            if (j == next && k == 0) continue;   // the read that moves to the buffer
            const Rng in = input_rng(nd, k);
            for (const Rng& r : rest)
                if (overlap(r, in)) return false;
        }
        subtract(&rest, out_rng(nd));
    }
    for (const Rng& r : rest)
        for (const Rng& l : live)
            if (overlap(r, l)) return false;
    return true;
}

void gemm_input_rngs(const OpNode* g, const Step& st, std::vector<Rng>* r) {
    const long long M = st.i[0], N = st.i[1], K = st.i[2], batches = st.i[3];
    const bool b2d = g->extra[2] != 0;
    r->push_back(rng(g->inputs[0], M * K * batches * 4));
    r->push_back(rng(g->inputs[1], N * K * (b2d ? 1 : batches) * 4));
    if (g->op == OP_MATMUL_ADD) r->push_back(rng(g->inputs[2], N * 4));
}

bool any_overlap(Rng a, const std::vector<Rng>& v) {
    for (const Rng& b : v)
        if (overlap(a, b)) return true;
    return false;
}

// ATTN_SLICED_V: the ATTENTION at node at_i takes as its V the [B, H, S, hd]
// head layout `v` of H column groups of hd starting at column col0 of the
// row-major [B·S, ld] tensor `src`; nodes [first, at_i) made `v` (their
// outputs `inter`) and are dropped, the kernel reading src instead.  The
// attention's output TRANSPOSE(H,S) at at_i + 1 joins the run when it can.
bool match_attn_sliced_v(const OpNode* nodes, int n, int first, int at_i, const void* src, int ld, int col0, int B,
                         int S, int H, int hd, const void* v, std::vector<Rng> inter, const std::vector<Rng>& live,
                         FusedRun* f) {
    if (at_i >= n) return false;
    const OpNode* at = &nodes[at_i];
    if (at->op != OP_ATTENTION || at->n_inputs < 3 || at->inputs[2] != v || at->inputs[0] == v ||
        at->inputs[1] == v || !is_f32(at) || at->n_dims != 4 || at->out_shape[0] != B || at->out_shape[2] != S ||
        at->out_shape[3] != hd || at->extra[0] != S || at->extra[1] != hd || ld % 4 || col0 % 4 ||
        !lbr_aligned(src, 16))
        return false;
    Step as = Step();
    if (decode_attention(at, &as) != LBR_OK) {
        lbr_set_error("");
        return false;
    }
    const int Hq = at->out_shape[1], group = at->extra[4] > 0 ? at->extra[4] : 1;
    if (as.i[10] != 1 || Hq != H * group) return false;   // the 16x16 kernel reads a strided V
    // the key-quartered kernel addresses one head's V rows with 32-bit byte offsets
    if (as.i[15] == 1 && ((long long)(S - 1) * ld + hd) * 4 >= (1LL << 31)) return false;
    const long long q_bytes = (long long)B * Hq * S * hd * 4;
    std::vector<Rng> reads{rng(at->inputs[0], q_bytes), rng(at->inputs[1], q_bytes / group),
                           rng(src, (long long)B * S * ld * 4)};
    if (at->extra[3] != 0) reads.push_back(rng(at->inputs[3], (long long)B * Hq * S * S * 4));
    // a schedule with a deferred store (key-range split, key-quartered kernel) lets the output
    // lie over what the kernel reads
    const bool split = lbr_attn_can_defer(as);
    const OpNode* tr = at_i + 1 < n ? &nodes[at_i + 1] : nullptr;
    int end = at_i + 1;
    Rng y = out_rng(at);
    // the kernel stores the transposed rows as float4s: the transpose output must be 16-byte aligned
    if (tr && tr->op == OP_TRANSPOSE && tr->n_inputs >= 1 && tr->inputs[0] == at->output && is_f32(tr) &&
        tr->n_dims == 4 && tr->extra[0] == B && tr->extra[1] == Hq && tr->extra[2] == 1 && tr->extra[3] == S &&
        tr->extra[4] == hd && lbr_aligned(tr->output, 16)) {
        std::vector<Rng> inter2 = inter;
        inter2.push_back(out_rng(at));
        if ((split || !any_overlap(out_rng(tr), reads)) && dead_after(nodes, n, at_i + 2, inter2, {out_rng(tr)}, live)) {
            inter = inter2;
            y = out_rng(tr);
            end = at_i + 2;
        }
    }
    const bool over = any_overlap(y, reads);
    if ((over && !split) || !dead_after(nodes, n, end, inter, {y}, live)) return false;
    f->defer = over;
    f->first = first;
    f->count = end - first;
    f->kind = LBR_FUSE_ATTN_SLICED_V;
    f->attn_at = at_i - first;
    f->src = src;
    f->ld = ld;
    f->col_begin[0] = col0;
    f->Hs[0] = Hq;
    f->Hs[1] = H;
    f->out = end == at_i + 2 ? tr->output : at->output;
    return true;
}

bool gemm_step(const OpNode* g, Step* st) {
    if (g->op != OP_MATMUL && g->op != OP_MATMUL_ADD) return false;
    *st = Step();
    if (decode_matmul(g, st) != LBR_OK) {
        lbr_set_error("");
        return false;
    }
    return st->i[13] == 1;
}

// TRANSPOSE_GEMM at node i: T = TRANSPOSE(O [B, H, S, hd] → [B, S, H, hd]) is the A
// operand of the next GEMM (DMA kernel, one batch, hd a multiple of its 32-wide K
// step or a divisor of it, so every step starts a head): the GEMM reads O directly; a
// residual ADD right after it is taken into the epilogue as well.
bool match_transpose_gemm(const OpNode* nodes, int n, int i, const std::vector<Rng>& live, FusedRun* f) {
    const OpNode* nd = &nodes[i];
    if (!(nd->op == OP_TRANSPOSE && i + 1 < n && is_f32(nd) && nd->n_dims == 4 && nd->n_inputs >= 1 &&
          nd->extra[2] == 1))
        return false;
    const int B = nd->extra[0], H = nd->extra[1], S = nd->extra[3], hd = nd->extra[4];
    const OpNode* mm = &nodes[i + 1];
    Step ms;
    if (!(nd->out_shape[0] == B && nd->out_shape[1] == S && nd->out_shape[2] == H && nd->out_shape[3] == hd &&
          (hd % 32 == 0 || (32 % hd == 0 && hd % 4 == 0)) && mm->n_inputs >= 2 && mm->inputs[0] == nd->output && is_f32(mm) && gemm_step(mm, &ms) &&
          ms.i[14] && ms.i[3] == 1 && ms.i[0] == (long long)B * S && ms.i[2] == (long long)H * hd &&
          lbr_aligned(nd->inputs[0], 16) && gemm_dma_heads_launcher((int)ms.i[14] - 1, ms.i[6] != 0)))
        return false;   // (the 64-wide-K-step tiles have no head-layout form)
    std::vector<Rng> reads;
    gemm_input_rngs(mm, ms, &reads);
    reads[0] = rng(nd->inputs[0], (long long)B * H * S * hd * 4);   // A is read as O
    const Rng t_r = out_rng(nd), c_r = out_rng(mm);
    *f = FusedRun();
    f->first = i;
    f->kind = LBR_FUSE_TRANSPOSE_GEMM;
    f->src = nd->inputs[0];
    f->B = B;
    f->S = S;
    f->hd = hd;
    f->Hs[0] = H;
    // with the residual ADD: y = C + R
    if (i + 2 < n) {
        const OpNode* ad = &nodes[i + 2];
        if (ad->op == OP_ADD && ad->n_inputs >= 2 && ad->extra[0] == 1 && is_f32(ad) &&
            node_total(ad) == node_total(mm) && (ad->inputs[0] == mm->output) != (ad->inputs[1] == mm->output)) {
            const void* R = ad->inputs[0] == mm->output ? ad->inputs[1] : ad->inputs[0];
            const Rng y = out_rng(ad), r_r = rng(R, node_total(mm) * 4);
            if (!any_overlap(y, reads) && (y.lo == r_r.lo || !overlap(y, r_r)) &&
                dead_after(nodes, n, i + 3, {t_r, c_r}, {y}, live)) {
                f->count = 3;
                f->resid = R;
                f->out = ad->output;
                return true;
            }
        }
    }
    if (!any_overlap(c_r, reads) && dead_after(nodes, n, i + 2, {t_r}, {c_r}, live)) {
        f->count = 2;
        f->out = mm->output;
        return true;
    }
    return false;
}

// Norm prologue: node p is a RMSNORM / LAYERNORM whose output is the A operand
// of GEMM node p + 1 and nothing else reads — the GEMM can read the norm's
// input and apply the norm itself (DMA kernel, one batch, no K split, 16-byte
// aligned x and weights, K = the norm's columns).  `end` is the end of the
// run the GEMM heads (p + 2 when it is alone): no output inside it may land
// on the norm's input or weights, which the GEMM reads to the end.
bool match_norm_prologue(const OpNode* nodes, int n, int p, int end, const std::vector<Rng>& live, FusedRun* f) {
    if (p + 1 >= n) return false;
    const OpNode* nm = &nodes[p];
    const OpNode* g = &nodes[p + 1];
    const bool rms = nm->op == OP_RMSNORM;
    if ((nm->op != OP_LAYERNORM && !rms) || !is_f32(nm) || nm->n_inputs < (rms ? 2 : 3)) return false;
    Step gs;
    // DMA path only, and a tile with a prologue variant (not the 256×256 tile,
    // nor the deeper-pipelined ones)
    if (!gemm_step(g, &gs) || !gs.i[14] || gs.i[3] != 1 || gs.i[10] > 1 || g->inputs[0] != nm->output) return false;
    if (!gemm_dma_norm_launcher((int)gs.i[14] - 1, gs.i[6] != 0, rms ? LBR_NORM_RMS : LBR_NORM_LAYER)) return false;
    const long long cols = node_last_dim(nm);
    if (cols <= 0 || gs.i[2] != cols || gs.i[0] * cols != node_total(nm)) return false;
    // Small GEMMs only: there the norm's own launch is most of its cost.  The
    // prologue's VALU work and γ/β loads slow a large GEMM by more than the norm
    // kernel costs (measured, GPT-2 S=1024 body 0.412 → 0.453 ms, Qwen3-4B body
    // 3.22 → 3.43 ms; the toy block 43.9 → 39.9 µs).  LBR_NORM_PROLOGUE=always
    // takes it at any size, =0 never.
    const char* mode = getenv("LBR_NORM_PROLOGUE");
    if (mode && strcmp(mode, "0") == 0) return false;
    const bool always = mode && strcmp(mode, "always") == 0;
    if (!always && gs.i[0] * gs.i[1] * gs.i[2] > (1LL << 26)) return false;
    const void* x = nm->inputs[0];
    const void* w = nm->inputs[1];
    const void* b = rms ? nullptr : nm->inputs[2];
    if (!lbr_aligned(x, 16) || !lbr_aligned(w, 16) || (b && !lbr_aligned(b, 16))) return false;
    const std::vector<Rng> reads{rng(x, node_total(nm) * 4), rng(w, cols * 4), rng(b, b ? cols * 4 : 0)};
    for (int j = p + 1; j < end; ++j)
        if (any_overlap(out_rng(&nodes[j]), reads)) return false;
    if (!dead_after(nodes, n, p + 2, {out_rng(nm)}, {}, live)) return false;
    f->norm = rms ? LBR_NORM_RMS : LBR_NORM_LAYER;
    f->norm_src = x;
    f->norm_g = w;
    f->norm_b = b;
    f->norm_eps = node_extra_float(nm, 0);
    return true;
}

int act_code(const OpNode* ac) {
    return ac->op == OP_RELU ? LBR_ACT_RELU : ac->op == OP_GELU ? LBR_ACT_GELU : ac->op == OP_SILU ? LBR_ACT_SILU
                                                                                                 : LBR_ACT_NONE;
}

// MLP at node i: GEMM1 → activation → GEMM2 [→ ADD(y, R)], one batch, B [N, K],
// small enough for mlp_rows (the hidden rows of 16 tokens in LDS, at most 2^25
// flops: a launch-bound chain).  A RMSNORM / LAYERNORM at node i−1 (`free`:
// no earlier run took it) whose output is only GEMM1's A joins the run: the
// kernel then reads the norm's input x and normalises its rows itself.  The
// kernel writes only y and reads x (or GEMM1's A), the weights, the biases
// and R: x and R may coincide with y row for row (each workgroup reads its
// rows before it writes them), nothing it reads may overlap y otherwise; the
// norm's output, GEMM1's, the activation's and (with the ADD) GEMM2's must be
// dead after the run.  LBR_MLP_FUSE=0 disables.
bool match_mlp(const OpNode* nodes, int n, int i, bool free, const std::vector<Rng>& live, FusedRun* f) {
    if (i + 2 >= n) return false;
    const char* mode = getenv("LBR_MLP_FUSE");
    if (mode && strcmp(mode, "0") == 0) return false;
    const OpNode* g1 = &nodes[i];
    const OpNode* ac = &nodes[i + 1];
    const OpNode* g2 = &nodes[i + 2];
    const int act = act_code(ac);
    if (act == LBR_ACT_NONE || ac->n_inputs < 1 || ac->inputs[0] != g1->output || !is_f32(ac) || !is_f32(g1) ||
        !is_f32(g2) || node_total(ac) != node_total(g1) || g2->n_inputs < 2 || g2->inputs[0] != ac->output)
        return false;
    Step s1, s2;
    if (!gemm_step(g1, &s1) || !gemm_step(g2, &s2)) return false;
    const long long M = s1.i[0], D = s1.i[2], H = s1.i[1], D2 = s2.i[1];
    if (s1.i[3] != 1 || s2.i[3] != 1 || !s1.i[4] || !s2.i[4] || s2.i[0] != M || s2.i[2] != H) return false;
    if (!mlp_shape_ok(M, D, H, D2) || 2.0 * (double)M * (double)(H * D + D2 * H) > 33554432.0) return false;
    const OpNode* ad = nullptr;
    const void* R = nullptr;
    if (i + 3 < n) {
        const OpNode* a = &nodes[i + 3];
        if (a->op == OP_ADD && a->n_inputs >= 2 && a->extra[0] == 1 && is_f32(a) && node_total(a) == node_total(g2) &&
            (a->inputs[0] == g2->output) != (a->inputs[1] == g2->output)) {
            ad = a;
            R = a->inputs[0] == g2->output ? a->inputs[1] : a->inputs[0];
        }
    }
    const int count = ad ? 4 : 3;
    const void* y = ad ? ad->output : g2->output;
    const Rng y_r = rng(y, M * D2 * 4);
    const void* b1 = g1->op == OP_MATMUL_ADD ? g1->inputs[2] : nullptr;
    const void* b2 = g2->op == OP_MATMUL_ADD ? g2->inputs[2] : nullptr;
    const void* ptrs[] = {g1->inputs[1], b1, g2->inputs[1], b2, R, y};
    for (const void* q : ptrs)
        if (q && !lbr_aligned(q, 16)) return false;
    const std::vector<Rng> consts{rng(g1->inputs[1], H * D * 4), rng(b1, b1 ? H * 4 : 0),
                                  rng(g2->inputs[1], D2 * H * 4), rng(b2, b2 ? D2 * 4 : 0)};
    if (any_overlap(y_r, consts)) return false;
    if (R && overlap(y_r, rng(R, M * D2 * 4)) && y != R) return false;
    // what the kernel reads as its rows: x (rows read, then overwritten only row for row)
    auto rows_ok = [&](const void* x) {
        return lbr_aligned(x, 16) && (!overlap(y_r, rng(x, M * D * 4)) || (y == x && D2 == D));
    };
    std::vector<Rng> inter{out_rng(g1), out_rng(ac)};
    if (ad) inter.push_back(out_rng(g2));
    // the norm before GEMM1
    const OpNode* nm = i > 0 && free ? &nodes[i - 1] : nullptr;
    if (nm && (nm->op == OP_LAYERNORM || nm->op == OP_RMSNORM)) {
        const bool rms = nm->op == OP_RMSNORM;
        const void* x = nm->inputs[0];
        const void* w = nm->inputs[1];
        const void* b = rms ? nullptr : nm->inputs[2];
        std::vector<Rng> inter_n = inter;
        inter_n.push_back(out_rng(nm));
        if (is_f32(nm) && nm->n_inputs >= (rms ? 2 : 3) && g1->inputs[0] == nm->output &&
            node_last_dim(nm) == D && node_total(nm) == M * D && rows_ok(x) && lbr_aligned(w, 16) &&
            (!b || lbr_aligned(b, 16)) && !overlap(y_r, rng(w, D * 4)) && !(b && overlap(y_r, rng(b, D * 4))) &&
            dead_after(nodes, n, i + count, inter_n, {y_r}, live)) {
            f->first = i - 1;
            f->count = count + 1;
            f->kind = LBR_FUSE_MLP;
            f->act = act;
            f->resid = R;
            f->out = y;
            f->norm = rms ? LBR_NORM_RMS : LBR_NORM_LAYER;
            f->norm_src = x;
            f->norm_g = w;
            f->norm_b = b;
            f->norm_eps = node_extra_float(nm, 0);
            return true;
        }
    }
    if (!rows_ok(g1->inputs[0]) || !dead_after(nodes, n, i + count, inter, {y_r}, live)) return false;
    f->first = i;
    f->count = count;
    f->kind = LBR_FUSE_MLP;
    f->act = act;
    f->resid = R;
    f->out = y;
    return true;
}

bool gemm_first_kind(int kind) {
    return kind == LBR_FUSE_GEMM_HEADS || kind == LBR_FUSE_GEMM_GATED || kind == LBR_FUSE_GEMM_ACT ||
           kind == LBR_FUSE_GEMM_RESID;
}

}  // namespace

void lbr_input_extent(const OpNode* nd, int k, unsigned long long* lo, unsigned long long* hi) {
    const Rng r = input_rng(nd, k);
    *lo = r.lo;
    *hi = r.hi;
}

// An attention step whose output lies over its inputs stores every row
// through a second kernel (deferred output: the key-range split's merge, or
// attn_kq_flush).  When the step right
// after it is a one-batch DMA GEMM whose A operand is exactly that output,
// and no other read sees the output's bytes before they are overwritten or
// at the end (live-out), the plan can give the attention a buffer of its
// own and point the GEMM's A there: the store is then no longer deferred.
bool lbr_relay_ok(const OpNode* nodes, int n, const Step& at, const Step& gm, const void* const* live_ptr,
                  const size_t* live_bytes, int n_live) {
    const char* e = getenv("LBR_ATTN_RELAY");
    if (e && atoi(e) == 0) return false;
    if (!at.name || strncmp(at.name, "attn_fwd_", 9) != 0 || !lbr_attn_can_defer(at) || !at.i[14]) return false;
    if (!gm.name || strncmp(gm.name, "gemm_dma_f32_nt", 15) != 0 || gm.in[0] != at.out || gm.i[3] != 1 || gm.i[35])
        return false;
    const long long yb = at.i[0] * at.i[1] * at.i[2] * 4;
    if (gm.i[0] * gm.i[2] * 4 != yb) return false;
    const int g0 = gm.node_index;
    const int end = at.node_index + at.n_nodes;
    if (g0 < end || g0 >= n) return false;
    std::vector<Rng> inter{rng(at.out, yb)};
    for (int j = end; j < n && !inter.empty(); ++j) {
        const OpNode* nd = &nodes[j];
        const int reads = nd->op == OP_ATTENTION ? 3 + (nd->extra[3] != 0) : nd->n_inputs;
        for (int k = 0; k < reads && k < nd->n_inputs && k < MAX_INPUTS; ++k) {
            if (j == g0 && k == 0) continue;   // the GEMM's A: the read that moves to the buffer
            const Rng in = input_rng(nd, k);
            for (const Rng& r : inter)
                if (overlap(r, in)) return false;
        }
        subtract(&inter, out_rng(nd));
    }
    for (const Rng& r : inter)
        for (int k = 0; k < n_live; ++k)
            if (overlap(r, rng(live_ptr[k], (long long)live_bytes[k]))) return false;
    return true;
}

// A head-scattering GEMM step can store split k fragment-major
// (lbr_frag_offset) for the key-quartered attention step that reads it as K,
// when the split is exactly that attention's K ([B, Hkv, S, hd] with S a
// multiple of 16 and hd the kernel's head dim) and no other read sees its
// bytes before they are overwritten or at the end (live-out): the Q and V
// reads of the attention itself included, so a K that is also its Q or V
// keeps the row-major layout.
bool lbr_frag_keys_ok(const OpNode* nodes, int n, const Step& gm, int k, const Step& at, const void* const* live_ptr,
                      const size_t* live_bytes, int n_live) {
    const char* e = getenv("LBR_KQ_FRAG");
    if (e && atoi(e) == 0) return false;
    if (!at.name || strncmp(at.name, "attn_fwd_kq", 11) != 0 || at.i[15] != 1) return false;
    if (!gm.name || strncmp(gm.name, "gemm_", 5) != 0 || k < 0 || k >= gm.i[19] || k >= 4 || gm.in[4 + k] != at.in[1])
        return false;
    const long long S = at.i[1], hd = at.i[2];
    if (S <= 0 || S % 16 != 0 || gm.i[30] != S || gm.i[29] != hd || at.i[5] != hd || at.i[4] <= 0) return false;
    const long long rows = gm.i[0];
    if (gm.i[3] != 1 || rows % S != 0 || (rows / S) * gm.i[25 + k] * at.i[4] != at.i[0]) return false;
    int an = -1;
    for (int j = at.node_index; j < at.node_index + at.n_nodes && j < n; ++j)
        if (nodes[j].op == OP_ATTENTION) {
            an = j;
            break;
        }
    const int end = gm.node_index + gm.n_nodes;
    if (an < end || nodes[an].inputs[1] != at.in[1]) return false;
    std::vector<Rng> inter{rng(at.in[1], at.i[0] / at.i[4] * S * hd * 4)};
    for (int j = end; j < n && !inter.empty(); ++j) {
        const OpNode* nd = &nodes[j];
        const int reads = nd->op == OP_ATTENTION ? 3 + (nd->extra[3] != 0) : nd->n_inputs;
        for (int q = 0; q < reads && q < nd->n_inputs && q < MAX_INPUTS; ++q) {
            if (j == an && q == 1) continue;   // the attention's K: the read that follows the layout
            const Rng in = input_rng(nd, q);
            for (const Rng& r : inter)
                if (overlap(r, in)) return false;
        }
        subtract(&inter, out_rng(nd));
    }
    for (const Rng& r : inter)
        for (int q = 0; q < n_live; ++q)
            if (overlap(r, rng(live_ptr[q], (long long)live_bytes[q]))) return false;
    return true;
}

// Find the fusable runs of `nodes` (in order, non-overlapping).
int lbr_find_fusions(const OpNode* nodes, int n, const void* const* live_ptr, const size_t* live_bytes, int n_live,
                     std::vector<FusedRun>* out) {
    out->clear();
    // every record within its arrays and sizes before any matcher reads one
    for (int k = 0; k < n; ++k)
        if (int rc = lbr_node_check(&nodes[k], k)) return rc;
    std::vector<Rng> live;
    for (int k = 0; k < n_live; ++k) live.push_back(rng(live_ptr[k], (long long)live_bytes[k]));
    int i = 0;
    while (i < n) {
        const OpNode* nd = &nodes[i];
        Step gs;
        if (gemm_step(nd, &gs)) {
            {
                FusedRun f;
                const bool free = out->empty() || out->back().first + out->back().count < i;
                if (match_mlp(nodes, n, i, free, live, &f)) {
                    out->push_back(f);
                    i = f.first + f.count;
                    continue;
                }
            }
            std::vector<Rng> gin;
            gemm_input_rngs(nd, gs, &gin);
            const Rng c_r = out_rng(nd);
            // GEMM_HEADS
            if (gs.i[3] == 1 && i + 1 < n) {
                const long long rows = gs.i[0];
                const int N = (int)gs.i[1];
                std::vector<HeadChain> chains;
                int q = i + 1;
                while (q < n && chains.size() < 4) {
                    HeadChain hc;
                    if (!match_head_chain(nodes, n, q, nd->output, rows, N, false, &hc)) break;
                    q += hc.count;
                    chains.push_back(hc);
                }
                bool ok = !chains.empty();
                std::vector<Rng> inter{c_r}, outs, reads = gin;
                for (const HeadChain& hc : chains) {
                    inter.insert(inter.end(), hc.inter.begin(), hc.inter.end());
                    if (hc.bias) reads.push_back(rng(hc.bias, (long long)hc.width * 4));
                }
                for (const HeadChain& hc : chains) {
                    if (any_overlap(hc.out_r, reads) || any_overlap(hc.out_r, outs)) ok = false;
                    outs.push_back(hc.out_r);
                }
                if (ok) ok = dead_after(nodes, n, q, inter, outs, live);
                // splits must tile the columns they cover in order, with one head dim and S
                for (size_t k = 1; ok && k < chains.size(); ++k)
                    ok = chains[k].col0 == chains[k - 1].col0 + chains[k - 1].width &&
                         chains[k].hd == chains[0].hd && chains[k].S == chains[0].S && chains[k].B == chains[0].B;
                if (ok) {
                    FusedRun f;
                    f.first = i;
                    f.count = q - i;
                    f.kind = LBR_FUSE_GEMM_HEADS;
                    f.n_split = (int)chains.size();
                    for (size_t k = 0; k < chains.size(); ++k) {
                        f.col_begin[k] = chains[k].col0;
                        f.width[k] = chains[k].width;
                        f.dst[k] = chains[k].out;
                        f.sbias[k] = chains[k].bias;
                        f.Hs[k] = chains[k].H;
                    }
                    f.hd = chains[0].hd;
                    f.S = chains[0].S;
                    f.B = chains[0].B;
                    out->push_back(f);
                    i = q;
                    continue;
                }
            }
            // GEMM_GATED: C [rows, 2F] → SLICE(C, last dim) × 2 → GATED_ACT(gate, [bias], up), one
            // slice the column half [0, F) and the other [F, 2F); DMA kernel, one batch, no K split
            if (gs.i[14] && gemm_dma_tile_pairs((int)gs.i[14] - 1) && gs.i[3] == 1 && gs.i[10] <= 1 &&
                gs.i[1] % 2 == 0 && i + 3 < n && is_f32(nd)) {
                const long long rows = gs.i[0];
                const int N = (int)gs.i[1], F = N / 2;
                const OpNode* s1 = &nodes[i + 1];
                const OpNode* s2 = &nodes[i + 2];
                const OpNode* ga = &nodes[i + 3];
                auto half = [&](const OpNode* sl) {   // column offset of a half slice of C, or -1
                    if (sl->op != OP_SLICE || sl->n_inputs < 1 || sl->inputs[0] != nd->output || !is_f32(sl) ||
                        sl->extra[0] != rows || sl->extra[1] != N || sl->extra[3] != F || sl->extra[4] != 1)
                        return -1;
                    return (sl->extra[2] == 0 || sl->extra[2] == F) ? sl->extra[2] : -1;
                };
                const int h1 = half(s1), h2 = half(s2);
                if (h1 >= 0 && h2 >= 0 && h1 != h2 && ga->op == OP_GATED_ACT && is_f32(ga) && ga->n_inputs >= 2 &&
                    node_total(ga) == rows * F && (ga->extra[1] == 0 || ga->extra[1] == 1)) {
                    const bool hb = ga->extra[0] != 0;
                    const void* x = ga->inputs[0];
                    const void* up = hb ? ga->inputs[2] : ga->inputs[1];
                    const void* gb = hb ? ga->inputs[1] : nullptr;
                    int gate_base = -1;
                    if (x == s1->output && up == s2->output) gate_base = h1;
                    if (x == s2->output && up == s1->output) gate_base = h2;
                    if (gate_base >= 0 && !(hb && ga->n_inputs < 3)) {
                        const Rng y = out_rng(ga);
                        std::vector<Rng> reads = gin;
                        if (gb) reads.push_back(rng(gb, (long long)F * 4));
                        bool ok = !any_overlap(y, reads), relay = false;
                        if (!ok && overlap(y, reads[0]) &&
                            !any_overlap(y, std::vector<Rng>(reads.begin() + 1, reads.end())) &&
                            gated_relay_ok(nodes, n, i + 4, ga->output, y, live))
                            ok = relay = true;
                        if (ok) ok = dead_after(nodes, n, i + 4, {c_r, out_rng(s1), out_rng(s2)}, {y}, live);
                        if (ok) {
                            FusedRun f;
                            f.first = i;
                            f.count = 4;
                            f.kind = LBR_FUSE_GEMM_GATED;
                            f.gF = F;
                            f.gate_base = gate_base;
                            f.gact = ga->extra[1];
                            f.gbias = gb;
                            f.out = ga->output;
                            f.relay_out = relay;
                            out->push_back(f);
                            i += 4;
                            continue;
                        }
                    }
                }
            }
            // GEMM_ACT: C → RELU | GELU | SILU (DMA kernel)
            if (gs.i[14] && i + 1 < n) {
                const OpNode* ac = &nodes[i + 1];
                const int act = ac->op == OP_RELU ? LBR_ACT_RELU
                              : ac->op == OP_GELU ? LBR_ACT_GELU
                              : ac->op == OP_SILU ? LBR_ACT_SILU : LBR_ACT_NONE;
                if (act != LBR_ACT_NONE && ac->n_inputs >= 1 && ac->inputs[0] == nd->output && is_f32(ac) &&
                    is_f32(nd) && node_total(ac) == node_total(nd)) {
                    const Rng y = out_rng(ac);
                    if (!any_overlap(y, gin) && dead_after(nodes, n, i + 2, {c_r}, {y}, live)) {
                        FusedRun f;
                        f.first = i;
                        f.count = 2;
                        f.kind = LBR_FUSE_GEMM_ACT;
                        f.act = act;
                        f.out = ac->output;
                        out->push_back(f);
                        i += 2;
                        continue;
                    }
                }
            }
            // GEMM_RESID
            if (i + 1 < n) {
                const OpNode* ad = &nodes[i + 1];
                if (ad->op == OP_ADD && ad->n_inputs >= 2 && ad->extra[0] == 1 && is_f32(ad) && is_f32(nd) &&
                    node_total(ad) == node_total(nd) && (ad->inputs[0] == nd->output) != (ad->inputs[1] == nd->output)) {
                    const void* R = ad->inputs[0] == nd->output ? ad->inputs[1] : ad->inputs[0];
                    const Rng y = out_rng(ad);
                    const Rng r_r = rng(R, node_total(nd) * 4);
                    bool ok = !any_overlap(y, gin) && (y.lo == r_r.lo || !overlap(y, r_r));
                    if (ok) ok = dead_after(nodes, n, i + 2, {c_r}, {y}, live);
                    if (ok) {
                        FusedRun f;
                        f.first = i;
                        f.count = 2;
                        f.kind = LBR_FUSE_GEMM_RESID;
                        f.resid = R;
                        f.out = ad->output;
                        out->push_back(f);
                        i += 2;
                        continue;
                    }
                }
            }
            ++i;
            continue;
        }
        // TRANSPOSE_GEMM: the GEMM after a head-layout transpose reads O directly
        {
            FusedRun f;
            if (match_transpose_gemm(nodes, n, i, live, &f)) {
                out->push_back(f);
                i += f.count;
                continue;
            }
        }
        // ATTN_TRANSPOSE: attention output [B, H, S, hd] transposed to [B, S, H, hd]
        if (nd->op == OP_ATTENTION && i + 1 < n && is_f32(nd) && nd->n_dims == 4) {
            const OpNode* tr = &nodes[i + 1];
            Step as = Step();
            const int B = nd->out_shape[0], H = nd->out_shape[1], S = nd->out_shape[2], hd = nd->out_shape[3];
            // (the kernel stores the transposed rows as float4s: 16-byte aligned output only)
            if (tr->op == OP_TRANSPOSE && tr->n_inputs >= 1 && tr->inputs[0] == nd->output && is_f32(tr) &&
                tr->n_dims == 4 && tr->extra[0] == B && tr->extra[1] == H && tr->extra[2] == 1 &&
                tr->extra[3] == S && tr->extra[4] == hd && lbr_aligned(tr->output, 16) &&
                decode_attention(nd, &as) == LBR_OK && as.i[10] == 1) {
                // the kernel reads Q, K, V (and the mask) while it writes the transposed output
                const bool mask = nd->extra[3] != 0;
                const long long qkv = (long long)B * H * S * hd * 4;
                const int group = nd->extra[4] > 0 ? nd->extra[4] : 1;
                std::vector<Rng> reads{rng(nd->inputs[0], qkv), rng(nd->inputs[1], qkv / group),
                                       rng(nd->inputs[2], qkv / group)};
                if (mask) reads.push_back(rng(nd->inputs[3], (long long)B * H * S * S * 4));
                // with a deferred store (key-range split, key-quartered kernel) the output may
                // lie over them, unless the transpose can go into the next GEMM instead, which
                // costs nothing
                const Rng y = out_rng(tr);
                const bool over = any_overlap(y, reads);
                FusedRun tg;
                const bool ok = !over || (lbr_attn_can_defer(as) && !match_transpose_gemm(nodes, n, i + 1, live, &tg));
                if (ok && dead_after(nodes, n, i + 2, {out_rng(nd)}, {y}, live)) {
                    FusedRun f;
                    f.first = i;
                    f.count = 2;
                    f.kind = LBR_FUSE_ATTN_TRANSPOSE;
                    f.out = tr->output;
                    f.Hs[0] = H;
                    f.defer = over;
                    out->push_back(f);
                    i += 2;
                    continue;
                }
            }
            lbr_set_error("");
        }
        // ATTN_SLICED_V: V of the attention two nodes on is SLICE(C, last dim) →
        // TRANSPOSE(S,H), read from C's columns ...
        if (nd->op == OP_SLICE && nd->n_inputs >= 1 && nd->extra[4] == 1 && is_f32(nd)) {
            HeadChain hc;
            const long long rows = nd->extra[0];
            const int ld = nd->extra[1];
            FusedRun f;
            if (match_head_chain(nodes, n, i, nd->inputs[0], rows, ld, false, &hc) && !hc.bias && hc.count == 2) {
                std::vector<Rng> inter = hc.inter;
                inter.push_back(hc.out_r);
                if (match_attn_sliced_v(nodes, n, i, i + 2, nd->inputs[0], ld, hc.col0, hc.B, hc.S, hc.H, hc.hd,
                                        hc.out, inter, live, &f)) {
                    out->push_back(f);
                    i += f.count;
                    continue;
                }
            }
        }
        // ... or V of the next attention is TRANSPOSE(S,H) of a [B, S, H, hd] tensor, read
        // in place
        if (nd->op == OP_TRANSPOSE && nd->n_inputs >= 1 && is_f32(nd) && nd->n_dims == 4 && nd->extra[2] == 1) {
            const int B = nd->extra[0], S = nd->extra[1], H = nd->extra[3], hd = nd->extra[4];
            FusedRun f;
            if (nd->out_shape[0] == B && nd->out_shape[1] == H && nd->out_shape[2] == S && nd->out_shape[3] == hd &&
                match_attn_sliced_v(nodes, n, i, i + 1, nd->inputs[0], H * hd, 0, B, S, H, hd, nd->output,
                                    {out_rng(nd)}, live, &f)) {
                out->push_back(f);
                i += f.count;
                continue;
            }
        }
        // HEAD_PROLOGUE: a SLICE of a row-major [rows, ld] tensor
        if (nd->op == OP_SLICE && nd->n_inputs >= 1 && nd->extra[4] == 1 && is_f32(nd)) {
            HeadChain hc;
            const long long rows = nd->extra[0];
            const int ld = nd->extra[1];
            if (match_head_chain(nodes, n, i, nd->inputs[0], rows, ld, true, &hc) &&
                (hc.hd == 64 || hc.hd == 128 || hc.hd == 256)) {
                std::vector<Rng> reads{rng(nd->inputs[0], rows * ld * 4)};
                if (hc.bias) reads.push_back(rng(hc.bias, (long long)hc.width * 4));
                if (hc.norm_w) reads.push_back(rng(hc.norm_w, (long long)hc.hd * 4));
                bool ok = !any_overlap(hc.out_r, reads);
                if (ok && hc.rope) {
                    // the tables' extents follow from their strides
                    auto ext = [&](const long long* st) {
                        return ((long long)(hc.B - 1) * st[0] + (long long)(hc.H - 1) * st[1] +
                                (long long)(hc.S - 1) * st[2] + hc.hd) * 4;
                    };
                    ok = !overlap(hc.out_r, rng(hc.rp.cos, ext(hc.rp.cst))) &&
                         !overlap(hc.out_r, rng(hc.rp.sin, ext(hc.rp.sst)));
                }
                if (ok) ok = dead_after(nodes, n, i + hc.count, hc.inter, {hc.out_r}, live);
                if (ok) {
                    FusedRun f;
                    f.first = i;
                    f.count = hc.count;
                    f.kind = LBR_FUSE_HEAD_PROLOGUE;
                    f.src = nd->inputs[0];
                    f.ld = ld;
                    f.col_begin[0] = hc.col0;
                    f.B = hc.B;
                    f.S = hc.S;
                    f.Hs[0] = hc.H;
                    f.hd = hc.hd;
                    f.sbias[0] = hc.bias;
                    f.norm_w = hc.norm_w;
                    f.eps = hc.eps;
                    f.rope = hc.rope;
                    if (hc.rope) {
                        f.cos = hc.rp.cos;
                        f.sin = hc.rp.sin;
                        for (int k = 0; k < 3; ++k) {
                            f.cst[k] = hc.rp.cst[k];
                            f.sst[k] = hc.rp.sst[k];
                        }
                    }
                    f.out = hc.out;
                    out->push_back(f);
                    i += hc.count;
                    continue;
                }
            }
        }
        ++i;
    }
    // Norm prologues: a norm just before a run that starts with its GEMM joins
    // the run; one before a GEMM no run took becomes a NORM_GEMM pair.
    std::vector<FusedRun> runs;
    size_t r = 0;
    for (int p = 0; p < n; ++p) {
        while (r < out->size() && (*out)[r].first < p) runs.push_back((*out)[r++]);
        if (r < out->size() && (*out)[r].first == p) continue;   // p heads a run: the loop above pushes it
        const bool in_run = !runs.empty() && runs.back().first + runs.back().count > p;
        if (in_run || (nodes[p].op != OP_LAYERNORM && nodes[p].op != OP_RMSNORM)) continue;
        FusedRun f;
        if (r < out->size() && (*out)[r].first == p + 1 && gemm_first_kind((*out)[r].kind)) {
            f = (*out)[r];
            if (match_norm_prologue(nodes, n, p, p + 1 + f.count, live, &f)) {
                f.first = p;
                f.count += 1;
                runs.push_back(f);
                ++r;
                ++p;   // the run's GEMM
            }
        } else if (r >= out->size() || (*out)[r].first > p + 1) {
            if (match_norm_prologue(nodes, n, p, p + 2, live, &f)) {
                f.first = p;
                f.count = 2;
                f.kind = LBR_FUSE_NORM_GEMM;
                runs.push_back(f);
                ++p;
            }
        }
    }
    while (r < out->size()) runs.push_back((*out)[r++]);
    *out = runs;
    return LBR_OK;
}

// Decoded launch record of a fused run.
int lbr_fused_step(const OpNode* nodes, const FusedRun& f, Step* s) {
    *s = Step();
    if (f.kind == LBR_FUSE_ATTN_TRANSPOSE) {
        int rc = decode_attention(&nodes[f.first], s);
        if (rc) return rc;
        if (s->i[10] != 1) {
            lbr_set_error("fusion: attention node %d cannot write a transposed output", f.first);
            return LBR_ERR_INVALID;
        }
        s->out = (void*)f.out;
        s->i[9] = f.Hs[0];
        s->name = lbr_attn_step_name(*s, false, true, 0);
        if (f.defer) {
            if (!lbr_attn_can_defer(*s)) {
                lbr_set_error("fusion: attention node %d writes over its inputs without a deferred store", f.first);
                return LBR_ERR_INVALID;
            }
            lbr_attn_defer(s);
            s->name = lbr_attn_step_name(*s, false, true, 1);
        }
    } else if (f.kind == LBR_FUSE_ATTN_SLICED_V) {
        const int at = f.first + f.attn_at;
        int rc = decode_attention(&nodes[at], s);
        if (rc) return rc;
        if (s->i[10] != 1) {
            lbr_set_error("fusion: attention node %d cannot read a strided V", at);
            return LBR_ERR_INVALID;
        }
        s->in[2] = (const float*)f.src + f.col_begin[0];
        s->i[12] = f.ld;
        s->i[13] = f.Hs[1];
        s->out = (void*)f.out;
        const bool tout = f.count == f.attn_at + 2;   // the output TRANSPOSE(H,S) joined the run
        if (tout) s->i[9] = f.Hs[0];
        s->name = lbr_attn_step_name(*s, true, tout, 0);
        if (f.defer) {
            if (!lbr_attn_can_defer(*s)) {
                lbr_set_error("fusion: attention node %d writes over its inputs without a deferred store", at);
                return LBR_ERR_INVALID;
            }
            lbr_attn_defer(s);
            s->name = lbr_attn_step_name(*s, true, tout, 1);
        }
    } else if (f.kind == LBR_FUSE_TRANSPOSE_GEMM) {
        int rc = decode_matmul(&nodes[f.first + 1], s);
        if (rc) return rc;
        if (!s->i[14] || s->i[3] != 1) {
            lbr_set_error("fusion: GEMM node %d is not on the single-batch DMA path", f.first + 1);
            return LBR_ERR_INVALID;
        }
        s->in[0] = f.src;
        s->run = gemm_dma_heads_launcher((int)s->i[14] - 1, s->i[6] != 0);
        if (!s->run) {
            lbr_set_error("fusion: GEMM node %d's tile has no head-layout form", f.first + 1);
            return LBR_ERR_INVALID;
        }
        s->i[35] = f.Hs[0];
        s->i[36] = f.S;
        s->i[37] = f.hd;
        s->out = (void*)f.out;
        if (f.resid) {
            s->in[3] = f.resid;
            s->i[12] = s->i[12] && lbr_aligned(f.out, 16);
            s->name = "gemm_dma_f32_nt+tin+resid";
        } else {
            s->name = "gemm_dma_f32_nt+tin";
        }
    } else if (f.kind == LBR_FUSE_MLP) {
        const int g1 = f.first + (f.norm ? 1 : 0);
        Step s1, s2;
        int rc = decode_matmul(&nodes[g1], &s1);
        if (!rc) rc = decode_matmul(&nodes[g1 + 2], &s2);
        if (rc) return rc;
        if (!mlp_shape_ok(s1.i[0], s1.i[2], s1.i[1], s2.i[1])) {
            lbr_set_error("fusion: MLP at node %d does not fit the one-kernel form", g1);
            return LBR_ERR_INVALID;
        }
        s->in[0] = f.norm ? f.norm_src : nodes[g1].inputs[0];
        s->in[1] = nodes[g1].inputs[1];
        s->in[2] = s1.i[6] ? nodes[g1].inputs[2] : nullptr;
        s->in[3] = nodes[g1 + 2].inputs[1];
        s->in[4] = s2.i[6] ? nodes[g1 + 2].inputs[2] : nullptr;
        s->in[5] = f.resid;
        s->in[6] = f.norm_g;
        s->in[7] = f.norm_b;
        s->out = (void*)f.out;
        s->i[0] = s1.i[0];
        s->i[1] = s1.i[2];
        s->i[2] = s1.i[1];
        s->i[3] = s2.i[1];
        s->i[4] = f.act;
        s->i[5] = f.norm;
        s->f[0] = s1.f[0];
        s->f[1] = s2.f[0];
        s->f[2] = f.norm_eps;
        s->run = mlp_launcher(s1.i[2], f.act);
        if (!s->run) {
            lbr_set_error("fusion: no MLP kernel for D=%lld (node %d)", s1.i[2], f.first + 1);
            return LBR_ERR_INVALID;
        }
        s->name = f.norm ? "mlp_rows+norm" : "mlp_rows";
    } else if (f.kind == LBR_FUSE_NORM_GEMM) {
        int rc = decode_matmul(&nodes[f.first + 1], s);
        if (rc) return rc;
        s->name = "gemm_dma_f32_nt";
    } else if (f.kind == LBR_FUSE_GEMM_ACT || f.kind == LBR_FUSE_GEMM_GATED) {
        int rc = decode_matmul(&nodes[f.first + (f.norm ? 1 : 0)], s);
        if (rc) return rc;
        if (!s->i[14] || (f.kind == LBR_FUSE_GEMM_GATED &&
                          (s->i[10] > 1 || s->i[3] != 1 || !gemm_dma_tile_pairs((int)s->i[14] - 1)))) {
            lbr_set_error("fusion: GEMM node %d is not on the DMA path without a K split", f.first);
            return LBR_ERR_INVALID;
        }
        s->out = (void*)f.out;
        if (f.kind == LBR_FUSE_GEMM_ACT) {
            s->i[31] = f.act;
            s->i[12] = s->i[12] && lbr_aligned(f.out, 16);
            s->name = "gemm_dma_f32_nt+act";
        } else {
            s->i[32] = f.gF;
            s->i[33] = f.gact;
            s->i[34] = f.gate_base;
            s->in[3] = f.gbias;
            s->i[28] = f.relay_out ? 1 : 0;   // relay_gated_outputs moves the output
            s->name = "gemm_dma_f32_nt+gated";
        }
    } else if (f.kind == LBR_FUSE_GEMM_RESID || f.kind == LBR_FUSE_GEMM_HEADS) {
        int rc = decode_matmul(&nodes[f.first + (f.norm ? 1 : 0)], s);
        if (rc) return rc;
        if (s->i[13] != 1) {
            lbr_set_error("fusion: GEMM node %d is not on the MFMA path", f.first);
            return LBR_ERR_INVALID;
        }
        if (f.kind == LBR_FUSE_GEMM_RESID) {
            s->in[3] = f.resid;
            s->out = (void*)f.out;
            s->i[12] = s->i[12] && lbr_aligned(f.out, 16);
            s->name = s->i[14] ? "gemm_dma_f32_nt+resid" : s->i[4] ? "gemm_mfma_f32_nt+resid" : "gemm_mfma_f32_nn+resid";
        } else {
            if (f.n_split < 1 || f.n_split > 4) {
                lbr_set_error("fusion: %d head splits", f.n_split);
                return LBR_ERR_INVALID;
            }
            s->i[19] = f.n_split;
            for (int k = 0; k < f.n_split; ++k) {
                s->i[20 + k] = f.col_begin[k];
                s->in[4 + k] = (void*)f.dst[k];
                s->in[8 + k] = f.sbias[k];
                s->i[25 + k] = f.Hs[k];
            }
            s->i[20 + f.n_split] = f.col_begin[f.n_split - 1] + f.width[f.n_split - 1];
            s->i[29] = f.hd;
            s->i[30] = f.S;
            s->name = s->i[14] ? "gemm_dma_f32_nt+heads" : s->i[4] ? "gemm_mfma_f32_nt+heads" : "gemm_mfma_f32_nn+heads";
        }
    } else {
        s->in[0] = f.src;
        s->in[1] = f.sbias[0];
        s->in[2] = f.norm_w;
        s->in[3] = f.cos;
        s->in[4] = f.sin;
        s->out = (void*)f.out;
        s->i[0] = f.ld;
        s->i[1] = f.col_begin[0];
        s->i[2] = f.B;
        s->i[3] = f.S;
        s->i[4] = f.Hs[0];
        s->i[5] = f.hd;
        for (int k = 0; k < 3; ++k) {
            s->i[6 + k] = f.cst[k];
            s->i[9 + k] = f.sst[k];
        }
        s->i[12] = (long long)f.B * f.S * f.Hs[0];
        s->f[0] = f.eps;
        const bool bias = f.sbias[0] != nullptr, norm = f.norm_w != nullptr;
        // 16-byte rows everywhere (source, output, bias, weight, RoPE rows) → float4 kernel
        bool vec = (long long)f.B * f.S < (1LL << 31) &&   // one x-block per token
                   lbr_aligned(f.src, 16) && f.ld % 4 == 0 && f.col_begin[0] % 4 == 0 && lbr_aligned(f.out, 16) &&
                   (!bias || lbr_aligned(f.sbias[0], 16)) && (!norm || lbr_aligned(f.norm_w, 16));
        if (f.rope) {
            vec = vec && lbr_aligned(f.cos, 16) && lbr_aligned(f.sin, 16);
            for (int k = 0; k < 3; ++k) vec = vec && f.cst[k] % 4 == 0 && f.sst[k] % 4 == 0;
        }
        // the float4 kernel's task index (token, heads group) stays below 2³¹
        const long long hpt = kHeadSlots * (256 / f.hd);
        vec = vec && (long long)f.B * f.S * 2 * ((f.Hs[0] + hpt - 1) / hpt) < (1LL << 31);
        const char* force = getenv("LBR_HEAD_PROLOGUE");   // "scalar" keeps the one-row-per-wave kernel
        if (force && strcmp(force, "scalar") == 0) vec = false;
        s->i[13] = vec;
        s->i[14] = 1;   // parts (lbr_merge_head_steps joins a second)
        switch (f.hd / 64) {
            case 1: s->run = vec ? pick_hp<64, true>(bias, norm, f.rope) : pick_hp<1, false>(bias, norm, f.rope); break;
            case 2: s->run = vec ? pick_hp<128, true>(bias, norm, f.rope) : pick_hp<2, false>(bias, norm, f.rope); break;
            default: s->run = vec ? pick_hp<256, true>(bias, norm, f.rope) : pick_hp<4, false>(bias, norm, f.rope); break;
        }
        s->name = f.rope ? (norm ? "head_norm_rope" : "head_rope") : (norm ? "head_norm" : "head_transpose");
    }
    if (f.norm && f.kind != LBR_FUSE_MLP) {   // the GEMM reads the norm's input and applies it (see match_norm_prologue)
        if (!s->i[14] || s->i[3] != 1 || s->i[10] > 1) {
            lbr_set_error("fusion: GEMM node %d is not on the single-batch DMA path without a K split", f.first + 1);
            return LBR_ERR_INVALID;
        }
        s->in[0] = f.norm_src;
        s->i[15] = f.norm;
        s->i[38] = (long long)(uintptr_t)f.norm_g;
        s->i[39] = (long long)(uintptr_t)f.norm_b;
        s->f[1] = f.norm_eps;
        s->run = gemm_dma_norm_launcher((int)s->i[14] - 1, s->i[6] != 0, f.norm);
        if (!s->run) {
            lbr_set_error("fusion: GEMM node %d's tile has no norm prologue", f.first + 1);
            return LBR_ERR_INVALID;
        }
        switch (f.kind) {
            case LBR_FUSE_GEMM_HEADS: s->name = "gemm_dma_f32_nt+norm+heads"; break;
            case LBR_FUSE_GEMM_RESID: s->name = "gemm_dma_f32_nt+norm+resid"; break;
            case LBR_FUSE_GEMM_ACT: s->name = "gemm_dma_f32_nt+norm+act"; break;
            case LBR_FUSE_GEMM_GATED: s->name = "gemm_dma_f32_nt+norm+gated"; break;
            default: s->name = "gemm_dma_f32_nt+norm"; break;
        }
    }
    s->node_index = f.first;
    s->n_nodes = f.count;
    return LBR_OK;
}

// Joins step b, the HEAD_PROLOGUE run right after a's in the stream, into a
// (both float4 kernels of the same form, the same source rows and RoPE
// tables): one launch then covers both parts.  Taken only when neither
// output overlaps anything either part reads, or the other output, so the
// joined launch computes what the two did in order.
bool lbr_merge_head_steps(Step* a, const Step& b) {
    if (a->fuse_kind != LBR_FUSE_HEAD_PROLOGUE || b.fuse_kind != LBR_FUSE_HEAD_PROLOGUE) return false;
    if (!a->i[13] || !b.i[13] || a->i[14] != 1 || b.i[14] != 1 || a->run != b.run) return false;
    if (getenv("LBR_HEAD_MERGE") && strcmp(getenv("LBR_HEAD_MERGE"), "0") == 0) return false;
    if (a->node_index + a->n_nodes != b.node_index) return false;
    if (a->in[0] != b.in[0] || a->in[3] != b.in[3] || a->in[4] != b.in[4]) return false;
    for (int k = 0; k <= 11; ++k)   // ld, B, S, hd and the table strides; k = 1, 4 are col0 and H
        if (k != 1 && k != 4 && a->i[k] != b.i[k]) return false;
    const long long B = a->i[2], S = a->i[3], hd = a->i[5];
    const long long hpt = kHeadSlots * (256 / hd);
    if (B * S * ((a->i[4] + hpt - 1) / hpt + (b.i[4] + hpt - 1) / hpt) >= (1LL << 31)) return false;
    auto out_rng = [&](const Step& t) { return Rng{(uintptr_t)t.out, (uintptr_t)t.out + (uintptr_t)(B * t.i[4] * S * hd * 4)}; };
    auto reads = [&](const Step& t) {
        std::vector<Rng> r{Rng{(uintptr_t)t.in[0], (uintptr_t)t.in[0] + (uintptr_t)(B * S * t.i[0] * 4)}};
        if (t.in[1]) r.push_back(Rng{(uintptr_t)t.in[1], (uintptr_t)t.in[1] + (uintptr_t)(t.i[4] * hd * 4)});
        if (t.in[2]) r.push_back(Rng{(uintptr_t)t.in[2], (uintptr_t)t.in[2] + (uintptr_t)(hd * 4)});
        for (int k = 0; k < 2; ++k) {
            const void* tab = t.in[3 + k];
            if (!tab) continue;
            const long long* st = &t.i[6 + 3 * k];
            const long long ext = ((B - 1) * st[0] + (t.i[4] - 1) * st[1] + (S - 1) * st[2] + hd) * 4;
            r.push_back(Rng{(uintptr_t)tab, (uintptr_t)tab + (uintptr_t)ext});
        }
        return r;
    };
    const Rng oa = out_rng(*a), ob = out_rng(b);
    if (overlap(oa, ob)) return false;
    for (const Rng& r : reads(*a))
        if (overlap(ob, r)) return false;
    for (const Rng& r : reads(b))
        if (overlap(oa, r)) return false;
    a->i[14] = 2;
    a->i[15] = b.i[4];
    a->i[16] = b.i[1];
    a->in[5] = b.in[1];
    a->in[6] = b.in[2];
    a->in[7] = b.out;
    a->f[1] = b.f[0];
    a->n_nodes += b.n_nodes;
    return true;
}

// Joins the HEAD_PROLOGUE step h (one part, or the Q and K parts of a layer
// joined by lbr_merge_head_steps; head dim 128) into the plain one-batch DMA GEMM
// step g right before it, whose output C is h's source: g then runs 64×128 tiles,
// and a tile that holds a head of a part normalises, rotates and stores it in
// its epilogue with the float4 prologue kernel's lanes and sums (the same bits).
// C's columns of the parts are not written, so no read of C other than a SLICE
// of columns outside them may follow the prologue, and C may not be live-out.
// The parts' outputs are written while the GEMM still reads A: where the planner
// put them over A (dead once the GEMM alone has run), the step gets Step::i[27] =
// the ATTENTION node that alone reads them (as Q and K) + 1, and the plan moves
// them to a buffer of its own (relay_head_outputs).
bool lbr_merge_gemm_head_prologue(Step* g, const Step& h, const OpNode* nodes, int n, const void* const* live_ptr,
                                  const size_t* live_bytes, int n_live) {
    const char* e = getenv("LBR_QKV_EPILOGUE");
    if (e && atoi(e) == 0) return false;
    if (h.fuse_kind != LBR_FUSE_HEAD_PROLOGUE || !h.i[13] || h.i[5] != 128) return false;
    if (!g->name || strcmp(g->name, "gemm_dma_f32_nt") != 0 || g->fuse_kind != LBR_FUSE_NONE || g->n_nodes != 1)
        return false;
    // no other epilogue, no K split, no norm prologue or reduce norm, row-major A, one batch
    if (g->i[3] != 1 || g->i[10] > 1 || g->i[19] || g->i[31] || g->i[32] || g->in[3] || g->i[15] || g->i[16] ||
        g->i[35] || g->i[18] || g->i[5])
        return false;
    const long long M = g->i[0], N = g->i[1];
    if (h.in[0] != g->out || h.i[0] != N || h.i[2] * h.i[3] != M || g->node_index + g->n_nodes != h.node_index)
        return false;
    if (N % 4 != 0 || !lbr_aligned(g->out, 16) || M * N >= (1LL << 31)) return false;
    const int parts = h.i[14] == 2 ? 2 : 1;
    const long long col[2] = {h.i[1], h.i[16]}, H[2] = {h.i[4], parts == 2 ? h.i[15] : 0};
    for (int p = 0; p < parts; ++p)
        if (col[p] % 128 != 0 || H[p] <= 0 || col[p] + H[p] * 128 > N) return false;
    const bool rope = h.in[3] != nullptr, norm = h.in[2] != nullptr;
    bool relay = false;
    // RoPE rows shared by the heads, the same strides for cos and sin
    if (rope && (h.i[7] != 0 || h.i[10] != 0 || h.i[6] != h.i[9] || h.i[8] != h.i[11])) return false;
    // the parts' outputs are written while other workgroups still read A, B, the bias, the
    // norm weights, the RoPE rows and the parts' biases (the planner may have put a prologue
    // output over A, dead once the GEMM alone has run), and while other tiles write C
    {
        const long long K = g->i[2];
        std::vector<Rng> reads{rng(g->in[0], M * K * 4), rng(g->in[1], N * K * 4), rng(g->out, M * N * 4)};
        if (g->in[2]) reads.push_back(rng(g->in[2], N * 4));
        for (int p = 0; p < parts; ++p) {
            const void* w = p ? h.in[6] : h.in[2];
            const void* pb = p ? h.in[5] : h.in[1];
            if (w) reads.push_back(rng(w, 128 * 4));
            if (pb) reads.push_back(rng(pb, H[p] * 128 * 4));
        }
        if (rope) {
            const long long B = h.i[2], S = h.i[3];
            const long long ext = ((B - 1) * h.i[6] + (S - 1) * h.i[8] + 128) * 4;
            reads.push_back(rng(h.in[3], ext));
            reads.push_back(rng(h.in[4], ext));
        }
        for (int p = 0; p < parts; ++p) {
            const Rng o = rng(p ? h.in[7] : h.out, M * H[p] * 128 * 4);
            for (size_t k = 0; k < reads.size(); ++k)
                if (overlap(o, reads[k])) {
                    if (k != 0) return false;
                    relay = true;   // over A only: the outputs can move to a buffer of the plan's own
                }
        }
        if (parts == 2 && overlap(rng(h.out, M * H[0] * 128 * 4), rng(h.in[7], M * H[1] * 128 * 4))) return false;
    }
    // moved outputs: after the run only one ATTENTION node reads them, as its Q (part 0) and K
    // (part 1), and they are not live-out; its step then reads the plan's buffer
    int relay_at = -1;
    if (relay) {
        for (int p = 0; p < parts; ++p) {
            const void* op = p ? h.in[7] : h.out;
            std::vector<Rng> rest{rng(op, M * H[p] * 128 * 4)};
            for (int j = h.node_index + h.n_nodes; j < n && !rest.empty(); ++j) {
                const OpNode* nd = &nodes[j];
                const int reads = nd->op == OP_ATTENTION ? 3 + (nd->extra[3] != 0) : nd->n_inputs;
                for (int q = 0; q < reads && q < nd->n_inputs && q < MAX_INPUTS; ++q) {
                    const Rng in = input_rng(nd, q);
                    bool hit = false;
                    for (const Rng& r : rest) hit = hit || overlap(r, in);
                    if (!hit) continue;
                    if (nd->op != OP_ATTENTION || q != p || nd->inputs[q] != op || (relay_at >= 0 && relay_at != j))
                        return false;
                    relay_at = j;
                }
                subtract(&rest, out_rng(nd));
            }
            for (const Rng& r : rest)
                for (int q = 0; q < n_live; ++q)
                    if (overlap(r, rng(live_ptr[q], (long long)live_bytes[q]))) return false;
        }
        if (relay_at < 0) return false;
    }
    // C's columns of the parts are never written: after the prologue only SLICEs of other
    // columns may read C (the V rows an attention takes), and C may not be live-out
    {
        const uintptr_t c0 = (uintptr_t)g->out, c1 = c0 + (uintptr_t)(M * N * 4);
        std::vector<Rng> rest{Rng{c0, c1}};
        for (int j = h.node_index + h.n_nodes; j < n && !rest.empty(); ++j) {
            const OpNode* nd = &nodes[j];
            const int reads = nd->op == OP_ATTENTION ? 3 + (nd->extra[3] != 0) : nd->n_inputs;
            for (int q = 0; q < reads && q < nd->n_inputs && q < MAX_INPUTS; ++q) {
                const Rng in = input_rng(nd, q);
                bool hit = false;
                for (const Rng& r : rest) hit = hit || overlap(r, in);
                if (!hit) continue;
                // a SLICE of C over its last dim: [outer, orig_dim, start, len, inner]
                if (nd->op != OP_SLICE || q != 0 || nd->inputs[0] != g->out || nd->extra[0] != M ||
                    nd->extra[1] != N || nd->extra[4] != 1)
                    return false;
                const long long a = nd->extra[2], b = a + nd->extra[3];
                for (int p = 0; p < parts; ++p)
                    if (a < col[p] + H[p] * 128 && col[p] < b) return false;
            }
            subtract(&rest, out_rng(nd));
        }
        for (const Rng& r : rest)
            for (int q = 0; q < n_live; ++q)
                if (overlap(r, rng(live_ptr[q], (long long)live_bytes[q]))) return false;
    }
    Step t = *g;
    if (!gemm_dma_retile(&t, gemm_dma_tile_by_name("64x128"))) return false;
    t.i[18] = parts;
    for (int p = 0; p < 2; ++p) {
        t.i[20 + p] = col[p];
        t.i[22 + p] = H[p];
    }
    t.i[24] = (norm ? 1 : 0) | (rope ? 2 : 0);
    t.i[27] = relay ? relay_at + 1 : 0;   // lbr_plan's relay_head_outputs moves the outputs
    t.i[25] = rope ? h.i[6] : 0;
    t.i[26] = rope ? h.i[8] : 0;
    t.i[30] = h.i[3];
    t.in[4] = h.out;
    t.in[5] = parts == 2 ? h.in[7] : nullptr;
    t.in[6] = h.in[2];
    t.in[7] = parts == 2 ? h.in[6] : nullptr;
    t.in[8] = h.in[3];
    t.in[9] = h.in[4];
    t.in[10] = h.in[1];
    t.in[11] = parts == 2 ? h.in[5] : nullptr;
    t.f[2] = h.f[0];
    t.f[3] = parts == 2 ? h.f[1] : 0.f;
    t.n_nodes += h.n_nodes;
    t.fuse_kind = LBR_FUSE_GEMM_HEAD_PROLOGUE;
    t.name = rope ? (norm ? "gemm_dma_f32_nt+head_norm_rope" : "gemm_dma_f32_nt+head_rope")
                  : (norm ? "gemm_dma_f32_nt+head_norm" : "gemm_dma_f32_nt+head_transpose");
    *g = t;
    return true;
}

// Joins the TRANSPOSE_GEMM step t (attention output projection, O in head
// layout, with its bias and residual) into the MLP step u right after it
// whose input x is t's output: the MLP kernel computes x itself (and still
// writes it), which saves a launch.  Every workgroup reads all of O and only
// its own rows of R0, x and R, so the written ranges (x, y) may meet R0, x and
// R only at the same base (row for row) and never O or a weight.
bool lbr_merge_proj_mlp(Step* u, const Step& t) {
    if (t.fuse_kind != LBR_FUSE_TRANSPOSE_GEMM || u->fuse_kind != LBR_FUSE_MLP) return false;
    if (getenv("LBR_PROJ_MLP") && strcmp(getenv("LBR_PROJ_MLP"), "0") == 0) return false;
    if (t.node_index + t.n_nodes != u->node_index) return false;
    const long long M = u->i[0], D = u->i[1], H = u->i[2], D2 = u->i[3], K0 = t.i[2];
    const long long oH = t.i[35], oS = t.i[36], ohd = t.i[37];
    if (t.i[10] > 1 || t.i[3] != 1 || t.i[0] != M || t.i[1] != D || u->in[0] != t.out || oH * ohd != K0 ||
        oS <= 0 || M % oS != 0 || !mlp_proj_ok(D, H, K0, ohd))
        return false;
    auto rg = [](const void* p, long long bytes) { return Rng{(uintptr_t)p, (uintptr_t)p + (uintptr_t)bytes}; };
    const Rng x = rg(t.out, M * D * 4), y = rg(u->out, M * D2 * 4);
    std::vector<Rng> fixed{rg(t.in[0], M * K0 * 4), rg(t.in[1], D * K0 * 4), rg(u->in[1], H * D * 4),
                           rg(u->in[3], D2 * H * 4)};
    if (t.in[2]) fixed.push_back(rg(t.in[2], D * 4));
    if (u->in[2]) fixed.push_back(rg(u->in[2], H * 4));
    if (u->in[4]) fixed.push_back(rg(u->in[4], D2 * 4));
    if (u->in[6]) fixed.push_back(rg(u->in[6], D * 4));
    if (u->in[7]) fixed.push_back(rg(u->in[7], D * 4));
    if (any_overlap(x, fixed) || any_overlap(y, fixed)) return false;
    // row-for-row: the same base and the same row width, else no overlap
    auto rows_ok = [&](const Rng& a, long long wa, const void* b, long long wb) {
        const Rng rb = rg(b, M * wb * 4);
        return a.lo == rb.lo ? wa == wb : !overlap(a, rb);
    };
    const bool res_x = u->in[5] == t.out;
    if (res_x && D2 != D) return false;
    if (t.in[3] && (!rows_ok(x, D, t.in[3], D) || !rows_ok(y, D2, t.in[3], D))) return false;
    if (!rows_ok(y, D2, t.out, D)) return false;
    if (u->in[5] && !res_x && (!rows_ok(x, D, u->in[5], D2) || !rows_ok(y, D2, u->in[5], D2))) return false;
    const step_fn run = mlp_launcher(D, (int)u->i[4], true);
    if (!run) return false;
    u->run = run;
    u->i[6] = 1;
    u->i[7] = K0;
    u->i[8] = oH;
    u->i[9] = oS;
    u->i[10] = ohd;
    u->i[11] = (t.i[6] ? 1 : 0) | (t.in[3] ? 4 : 0) | (res_x ? 8 : 0);   // MLP_HAS_B1, MLP_HAS_RESID, MLP_RES_X
    u->f[3] = t.f[0];
    u->in[8] = t.in[0];
    u->in[9] = t.in[1];
    u->in[10] = t.i[6] ? t.in[2] : nullptr;
    u->in[11] = t.in[3];
    u->node_index = t.node_index;
    u->n_nodes += t.n_nodes;
    u->name = u->i[5] ? "mlp_rows+proj+norm" : "mlp_rows+proj";
    return true;
}

// Joins the decoded RMSNORM / LAYERNORM step n right after the split-K GEMM
// step g (one batch, float4 reduce, no head split, gated pair or activation)
// whose output C it normalises over C's rows: g's reduce kernel then writes
// the normalised rows too.  The reduce handles whole rows, one workgroup
// (or wavefront) each, reading the partial sums, the bias and the residual
// row and writing C's row and the norm's row; so the norm's output may
// meet the residual only row for row and touch neither C, the bias nor the
// norm's weights.
bool lbr_merge_reduce_norm(Step* g, const Step& n) {
    if (getenv("LBR_REDUCE_NORM") && strcmp(getenv("LBR_REDUCE_NORM"), "0") == 0) return false;
    // an unsplit GEMM of at most 2^32 flops takes two K ranges to carry the norm
    // (GPT-2's attention projection + LayerNorm: 21.4 + 7.4 → 23.9 µs); the K sum
    // is then split in two, other roundings than the unsplit GEMM's.
    // LBR_REDUCE_NORM_SPLIT=0 keeps such GEMMs unsplit and their norms apart.
    const char* sp = getenv("LBR_REDUCE_NORM_SPLIT");
    const bool split2 = !(sp && strcmp(sp, "0") == 0) && g->i[10] <= 1 &&
                        2.0 * g->i[0] * g->i[1] * g->i[2] <= 4294967296.0;
    // a GEMM + residual ADD, with A row-major or read in head layout (TRANSPOSE_GEMM: the
    // reduce never reads A)
    const bool tin = g->fuse_kind == LBR_FUSE_TRANSPOSE_GEMM;
    if ((g->fuse_kind != LBR_FUSE_GEMM_RESID && !tin) || !g->in[3] || (g->i[10] <= 1 && !split2) || g->i[3] != 1 ||
        !g->i[12] || g->i[19] || g->i[32] || g->i[31] || g->i[16] || g->i[18] || !n.name)
        return false;
    const bool rms = strcmp(n.name, "rmsnorm") == 0;
    if (!rms && strcmp(n.name, "layernorm") != 0) return false;
    const long long M = g->i[0], N = g->i[1];
    if (g->node_index + g->n_nodes != n.node_index || n.in[0] != g->out || n.i[0] != M || n.i[1] != N ||
        (n.i[2] != 1 && n.i[2] != 2) || n.i[3] < 2 || n.i[3] > 4 || N % 4 || !lbr_aligned(g->out, 16) ||
        (g->in[3] && !lbr_aligned(g->in[3], 16)))   // 2 to 4 float4 a lane: rows of 257 to 4096 columns
        return false;
    auto rg = [](const void* q, long long bytes) { return Rng{(uintptr_t)q, (uintptr_t)q + (uintptr_t)bytes}; };
    const Rng y = rg(n.out, M * N * 4);
    std::vector<Rng> fixed{rg(g->out, M * N * 4), rg(n.in[1], N * 4)};
    if (n.in[2]) fixed.push_back(rg(n.in[2], N * 4));
    if (g->i[6]) fixed.push_back(rg(g->in[2], N * 4));
    if (any_overlap(y, fixed)) return false;
    if (g->in[3]) {
        const Rng r = rg(g->in[3], M * N * 4);
        if (overlap(y, r) && y.lo != r.lo) return false;
    }
    const bool forced = g->i[10] <= 1;
    if (forced && !gemm_dma_split2(g)) return false;
    g->i[16] = rms ? LBR_NORM_RMS : LBR_NORM_LAYER;
    g->i[17] = n.i[2] * 16 + n.i[3] + (forced ? 256 : 0);   // 256: the split was made for the norm
    g->in[4] = n.out;
    g->in[5] = n.in[1];
    g->in[6] = n.in[2];
    g->f[2] = n.f[0];
    g->n_nodes += 1;
    const bool dma = g->i[14] != 0;
    if (tin) g->name = rms ? "gemm_dma_f32_nt+tin+resid+rmsnorm" : "gemm_dma_f32_nt+tin+resid+layernorm";
    else
        g->name = dma ? (rms ? "gemm_dma_f32_nt+resid+rmsnorm" : "gemm_dma_f32_nt+resid+layernorm")
                      : (rms ? "gemm_mfma_f32+resid+rmsnorm" : "gemm_mfma_f32+resid+layernorm");
    return true;
}

// Joins the decoded ADD step a (node add) into the decoded RMSNORM /
// LAYERNORM step n right after it whose input is the sum: n's kernel then
// adds, writes the sum (the ADD's output) and normalises it.  The ADD must be
// one contiguous [M, N] operand plus either one of the same shape or a [P, N]
// block broadcast over the leading dims (row r adds row r mod P): a position
// table.  Each wavefront / workgroup owns whole rows: the sum may overlap the
// full operand only row for row (the same base), and nothing else either
// output touches may be read.
bool lbr_merge_add_norm(Step* n, const Step& a, const OpNode* add) {
    if (getenv("LBR_ADD_NORM") && strcmp(getenv("LBR_ADD_NORM"), "0") == 0) return false;
    if (!a.name || !n->name || add->op != OP_ADD || add->n_inputs < 2 || !is_f32(add)) return false;
    const bool rms = strcmp(n->name, "rmsnorm") == 0;
    if ((!rms && strcmp(n->name, "layernorm") != 0) || (n->i[2] != 1 && n->i[2] != 2) || n->in[3]) return false;
    if (a.node_index + a.n_nodes != n->node_index || n->in[0] != a.out) return false;
    const long long M = n->i[0], N = n->i[1];
    if (M <= 0 || N <= 0 || N % 4 || node_total(add) != M * N) return false;
    const void* full = nullptr;
    const void* part = nullptr;
    long long P = 0;
    if (add->extra[0] == 1) {   // same shape
        full = add->inputs[0];
        part = add->inputs[1];
        P = M;
    } else if (add->extra[0] == 3) {   // broadcast: [3, nd, a strides, b strides, out shape]
        const int nd = (int)add->extra[1];
        if (nd < 2 || 1 + 3 * nd > MAX_DIMS - 1) return false;
        const int* as = &add->extra[2];
        const int* bs = &add->extra[2 + nd];
        const int* sh = &add->extra[2 + 2 * nd];
        if (sh[nd - 1] != N) return false;
        auto contiguous = [&](const int* st) {
            long long want = 1;
            for (int d = nd - 1; d >= 0; --d) {
                if (sh[d] > 1 && st[d] != want) return false;
                want *= sh[d];
            }
            return true;
        };
        auto rows_of = [&](const int* st) {   // (row mod P)·N + col, P = sh[nd − 2]
            if (st[nd - 1] != 1 || (sh[nd - 2] > 1 && st[nd - 2] != N)) return false;
            for (int d = 0; d < nd - 2; ++d)
                if (sh[d] > 1 && st[d] != 0) return false;
            return true;
        };
        if (contiguous(as) && rows_of(bs)) {
            full = add->inputs[0];
            part = add->inputs[1];
        } else if (contiguous(bs) && rows_of(as)) {
            full = add->inputs[1];
            part = add->inputs[0];
        } else {
            return false;
        }
        P = sh[nd - 2];
    } else {
        return false;
    }
    if (P <= 0 || M % P || P > (1LL << 30) || !lbr_aligned(full, 16) || !lbr_aligned(part, 16) ||
        !lbr_aligned(a.out, 16))
        return false;
    auto rg = [](const void* q, long long bytes) { return Rng{(uintptr_t)q, (uintptr_t)q + (uintptr_t)bytes}; };
    const Rng h = rg(a.out, M * N * 4), y = rg(n->out, M * N * 4), f = rg(full, M * N * 4);
    std::vector<Rng> fixed{rg(part, P * N * 4), rg(n->in[1], N * 4)};
    if (n->in[2]) fixed.push_back(rg(n->in[2], N * 4));
    if (any_overlap(h, fixed) || any_overlap(y, fixed) || overlap(h, y)) return false;
    if ((overlap(h, f) && h.lo != f.lo) || (overlap(y, f) && y.lo != f.lo)) return false;
    n->in[0] = full;
    n->in[3] = part;
    n->i[4] = P;
    n->in[4] = a.out;
    n->node_index = a.node_index;
    n->n_nodes += a.n_nodes;
    n->fuse_kind = LBR_FUSE_ADD_NORM;
    n->name = rms ? "rmsnorm+add" : "layernorm+add";
    return true;
}

