// tiny.hip — the whole plan in one workgroup, for launch-bound graphs.
//
// A graph as small as the toy block (S = 32, D = 64) spends nearly all of
// its time in per-kernel latency: each launch pays dispatch, a first memory
// round trip and a drain of a few microseconds whatever its work, so seven
// fused kernels cost ~40 µs for 3.3 MFLOP.  When every intermediate fits in
// one CU's LDS, one 1024-thread workgroup runs the node array itself, node
// after node with a workgroup barrier between them.
//
// One CU is a narrow machine: its 4 SIMDs issue a 64-lane VALU instruction
// in 4 cycles each, so an instruction that all 16 wavefronts execute costs
// ~16 cycles of wall time.  The design follows from that:
//   * the host decodes every node into a TyOp record of ready values —
//     element counts, strides, multiply-shift divisors, operand addresses
//     already resolved to an LDS offset or a global address, GEMM staging and
//     K-split choices — which the kernel reads with scalar loads, so the
//     per-node cost is a few scalar instructions, not a per-lane decode;
//   * index arithmetic divides by multiplying (one v_mul_hi and a shift);
//   * row operations give each row as many lanes as keep the workgroup busy,
//     with the row held in registers.
// The CU's 160 KiB of LDS holds the arena window — the byte range spanning
// every node's output — at the same relative offsets, so intermediates never
// reach HBM, and after it a staging area: a GEMM copies its B operand (and A,
// with padded rows, so that the 16 rows an MFMA reads hit different LDS
// banks) there with all wavefronts' loads in flight at once, in K chunks when
// it does not fit; attention keeps one head group's scores there.  Graph
// inputs and weights stay in global memory.  At the end the caller-visible
// ranges (the declared live-out ranges, or every node's output when none are
// declared) are copied back.
// Semantics follow the device kernels of the other files (and so the
// reference's kernels, csrc/ops/*.c): the same extras decoding, the same
// activation functions; GEMM and reduction sums are reassociated, so results
// match the multi-kernel plan within fp32 rounding, not bit for bit.
//
// Status: opt-in (LBR_TINY=1).  Measured on the toy block it loses to the
// peephole-fused multi-kernel plan (kernel 54 µs against 43.5 µs per
// replay): a node costs ~0.8 µs however small (one wavefront's chain of
// record reads, dependent LDS round trips and branches, times the barrier),
// and one CU's fp32 matrix rate (256 FLOP/cycle) caps each GEMM.
#include "lbr_device.h"
#include "lbr_fusion.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <type_traits>
#include <vector>

namespace {

constexpr int TY_NT = 1024;                  // 16 wavefronts
constexpr int TY_WAVES = TY_NT / 64;
constexpr int TY_LDS = 160 * 1024;           // the CU's LDS: window + staging
constexpr long long TY_MAX_FLOP = 32LL << 20;   // beyond this the multi-kernel plan wins
constexpr int TY_MAX_ATTN_S = 256;
constexpr int TY_MAX_HD = 128;
constexpr int TY_BPW = 2;                    // GEMM work items per wavefront per pass (more spill)
constexpr int TY_CPL = 8;                    // row elements per lane held in registers

enum TyKind : int {
    TY_UNARY = 1, TY_BIN_SAME, TY_BIN_SCALAR, TY_BIN_ROW, TY_BIN_BCAST, TY_BIAS_RELU, TY_GATED, TY_NORM,
    TY_SOFTMAX, TY_GEMM, TY_ATTN, TY_COPY, TY_SLICE, TY_TRANS2D, TY_SWAP, TY_CAT
};

// A node as the kernel runs it.  Operand k (p[5] is the output) is an LDS
// byte offset when bit k of `lds` is set, else a global address.  n[] and
// f[] are per kind (see the kernels below and build_op).  Divisors appear as
// (m, s) pairs: x / d is __umulhi(x, m) >> s, or x itself when m is 0 (d = 1).
struct TyOp {
    int kind, sub, lds, total;
    int n[24];
    float f[4];
    unsigned long long p[6];
};
static_assert(sizeof(TyOp) == 176, "TyOp layout");

// GEMM flags (TyOp::n[4])
constexpr int G_TRANS_B = 1, G_B2D = 2, G_BIAS = 4, G_STAGE_B = 8, G_STAGE_A = 16, G_B_VEC = 32, G_A_VEC = 64;

// The records live in LDS (copied there at the start): a field read gives a
// VGPR, and readfirstlane makes it the scalar it is (it is the same in every
// lane), so the arithmetic on it stays on the scalar unit.
__device__ __forceinline__ int rf(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ unsigned long long rf64(unsigned long long v) {
    const unsigned lo = __builtin_amdgcn_readfirstlane((int)(unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((int)(unsigned)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

// The fields every node uses — kind, operands, n[0..7], f[] — read from the
// LDS record in one batch of 16-byte loads (one wait), as scalars.  The rest
// of n[] is read where a kind needs it.
struct Node {
    int kind, sub, lds, total;
    int n[8];
    float f[4];
    unsigned long long p[6];
};

__device__ __forceinline__ Node read_node(const TyOp* op) {
    const int4* q = reinterpret_cast<const int4*>(op);
    const int4 h = q[0], a = q[1], b = q[2], f = q[7];
    const int4 p01 = q[8], p23 = q[9], p45 = q[10];
    Node d;
    d.kind = rf(h.x), d.sub = rf(h.y), d.lds = rf(h.z), d.total = rf(h.w);
    d.n[0] = rf(a.x), d.n[1] = rf(a.y), d.n[2] = rf(a.z), d.n[3] = rf(a.w);
    d.n[4] = rf(b.x), d.n[5] = rf(b.y), d.n[6] = rf(b.z), d.n[7] = rf(b.w);
    d.f[0] = __int_as_float(rf(f.x)), d.f[1] = __int_as_float(rf(f.y));
    d.f[2] = __int_as_float(rf(f.z)), d.f[3] = __int_as_float(rf(f.w));
    auto u64 = [](int lo, int hi) { return ((unsigned long long)(unsigned)rf(hi) << 32) | (unsigned)rf(lo); };
    d.p[0] = u64(p01.x, p01.y), d.p[1] = u64(p01.z, p01.w);
    d.p[2] = u64(p23.x, p23.y), d.p[3] = u64(p23.z, p23.w);
    d.p[4] = u64(p45.x, p45.y), d.p[5] = u64(p45.z, p45.w);
    return d;
}

__device__ __forceinline__ float* opnd(const Node& d, char* lds, int k) {
    return ((d.lds >> k) & 1) ? reinterpret_cast<float*>(lds + d.p[k]) : reinterpret_cast<float*>(d.p[k]);
}

__device__ __forceinline__ unsigned* opnd_u(const Node& d, char* lds, int k) {
    return reinterpret_cast<unsigned*>(opnd(d, lds, k));
}

// i over [0, total) with U elements per thread per round: every load of a
// round is issued before its first store (ld computes the value, st writes
// it), so a thread's memory latencies overlap instead of adding up.
template <int U, class Ld, class St>
__device__ __forceinline__ void each(int total, Ld ld, St st) {
    for (int base = threadIdx.x; base < total; base += U * TY_NT) {
        decltype(ld(0)) v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (base + u * TY_NT < total) v[u] = ld(base + u * TY_NT);
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (base + u * TY_NT < total) st(base + u * TY_NT, v[u]);
    }
}

template <int OP>
__device__ __forceinline__ float unary_f(float x, float s) {
    if constexpr (OP == OP_RELU) return x > 0.0f ? x : 0.0f;
    else if constexpr (OP == OP_EXP) return expf(x);
    else if constexpr (OP == OP_TANH) return tanhf(x);
    else if constexpr (OP == OP_POW) return powf(x, s);
    else if constexpr (OP == OP_GELU) return lbr_gelu_tanh(x);
    else if constexpr (OP == OP_RSQRT) return 1.0f / sqrtf(x);
    else if constexpr (OP == OP_SILU) return lbr_silu(x);
    else if constexpr (OP == OP_NEG) return -x;
    else if constexpr (OP == OP_COS) return cosf(x);
    else return sinf(x);   // OP_SIN
}

// unary ops: sub = op code, f[0] = POW's exponent
template <int OP>
__device__ __forceinline__ void t_unary(const TyOp& o, const Node& d, char* lds) {
    const float* x = opnd(d, lds, 0);
    float* y = opnd(d, lds, 5);
    const float s = d.f[0];
    each<4>(d.total, [&](int i) { return unary_f<OP>(x[i], s); }, [&](int i, float v) { y[i] = v; });
}

template <int B>   // 0 add, 1 sub, 2 mul, 3 div
__device__ __forceinline__ float binop_f(float a, float b) {
    if constexpr (B == 0) return a + b;
    else if constexpr (B == 1) return a - b;
    else if constexpr (B == 2) return a * b;
    else return a / b;
}

// SAME: a[i] ∘ b[i]; SCALAR: a[i] ∘ f[0]; ROW: a[i] ∘ b[i mod N], N = n[0]
// (divisor n[1], n[2]); BCAST: up to 4 merged dims, n[0] = nd, dim d at
// n[1 + 5d ..]: size, a stride, b stride, divisor (runtime/ops.py:174-235).
template <int B>
__device__ __forceinline__ void t_binary(const TyOp& o, const Node& d, char* lds) {
    const float* a = opnd(d, lds, 0);
    const float* b = opnd(d, lds, 1);
    float* y = opnd(d, lds, 5);
    auto st = [&](int i, float v) { y[i] = v; };
    switch (d.kind) {
        case TY_BIN_SAME:
            each<4>(d.total, [&](int i) { return binop_f<B>(a[i], b[i]); }, st);
            break;
        case TY_BIN_SCALAR: {
            const float s = d.f[0];
            each<4>(d.total, [&](int i) { return binop_f<B>(a[i], s); }, st);
            break;
        }
        case TY_BIN_ROW: {
            const unsigned N = d.n[0];
            const int m = d.n[1], sh = d.n[2];
            each<4>(d.total, [&](int i) { return binop_f<B>(a[i], b[i - lbr_fdiv(i, m, sh) * N]); }, st);
            break;
        }
        default: {   // TY_BIN_BCAST
            const int nd = d.n[0];
            each<2>(d.total, [&](int i) {
                unsigned r = (unsigned)i;
                int ai = 0, bi = 0;
#pragma unroll
                for (int d = 3; d >= 0; --d) {
                    if (d >= nd) continue;
                    const int* e = o.n + 1 + 5 * d;   // LDS record
                    const unsigned q = lbr_fdiv(r, rf(e[3]), rf(e[4]));
                    const int c = (int)(r - q * (unsigned)rf(e[0]));
                    r = q;
                    ai += c * rf(e[1]);
                    bi += c * rf(e[2]);
                }
                return binop_f<B>(a[ai], b[bi]);
            }, st);
        }
    }
}

// FUSED_BIAS_RELU relu(x + bias[col]) (elementwise.c:82-90); column =
// i mod n[0] (divisor n[1], n[2]).
__device__ __forceinline__ void t_bias_relu(const TyOp& o, const Node& d, char* lds) {
    const float* x = opnd(d, lds, 0);
    const float* bias = opnd(d, lds, 1);
    float* y = opnd(d, lds, 5);
    const unsigned N = d.n[0];
    const int m = d.n[1], sh = d.n[2];
    each<4>(d.total, [&](int i) {
        const float v = x[i] + bias[i - lbr_fdiv(i, m, sh) * N];
        return v > 0.f ? v : 0.f;
    }, [&](int i, float v) { y[i] = v; });
}

// GATED_ACT act(x [+ bias[col]]) · up (executor.c:354-369): sub = 0 SiLU,
// 1 GELU; operands x, up, bias; column as in t_bias_relu.
template <bool SILU, bool BIAS>
__device__ __forceinline__ void t_gated(const TyOp& o, const Node& d, char* lds) {
    const float* x = opnd(d, lds, 0);
    const float* up = opnd(d, lds, 1);
    const float* bias = opnd(d, lds, 2);
    float* y = opnd(d, lds, 5);
    const unsigned N = d.n[0];
    const int m = d.n[1], sh = d.n[2];
    each<4>(d.total, [&](int i) {
        const float v = BIAS ? x[i] + bias[i - lbr_fdiv(i, m, sh) * N] : x[i];
        return (SILU ? lbr_silu(v) : lbr_gelu_tanh(v)) * up[i];
    }, [&](int i, float v) { y[i] = v; });
}

// Reductions over the `lpr` lanes of a row group (aligned, a power of two).
__device__ __forceinline__ float group_sum(float v, int lpr) {
    for (int off = lpr >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float group_max(float v, int lpr) {
    for (int off = lpr >> 1; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// LAYERNORM (norm.c:47-64, two-pass) / RMSNORM (norm.c:100-107), sub = rms;
// n[0] rows, n[1] cols, n[2] lanes per row (lpr), n[3] log2 lpr, n[4] cols
// per lane (≤ TY_CPL; 0: a wavefront per row, for wide rows); f[0] eps,
// f[1] 1/cols.
template <bool RMS>
__device__ __forceinline__ void t_norm(const TyOp& o, const Node& d, char* lds) {
    const float* x = opnd(d, lds, 0);
    const float* g = opnd(d, lds, 1);
    const float* b = opnd(d, lds, 2);
    float* y = opnd(d, lds, 5);
    const int rows = d.n[0], cols = d.n[1], lpr = d.n[2], cpl = d.n[4];
    const float eps = d.f[0], inv_cols = d.f[1];
    if (cpl > 0) {
        const int j = threadIdx.x & (lpr - 1);
        float gv[TY_CPL], bv[TY_CPL];
#pragma unroll
        for (int t = 0; t < TY_CPL; ++t) {
            const int c = j + t * lpr;
            gv[t] = (t < cpl && c < cols) ? g[c] : 0.f;
            bv[t] = (!RMS && t < cpl && c < cols) ? b[c] : 0.f;
        }
        for (int r = threadIdx.x >> d.n[3]; r < rows; r += TY_NT >> d.n[3]) {
            const float* xr = x + r * cols;
            float xv[TY_CPL], s = 0.f;
#pragma unroll
            for (int t = 0; t < TY_CPL; ++t) {
                const int c = j + t * lpr;
                xv[t] = (t < cpl && c < cols) ? xr[c] : 0.f;
                s += RMS ? xv[t] * xv[t] : xv[t];
            }
            s = group_sum(s, lpr);
            float* yr = y + r * cols;
            if (RMS) {
                const float scale = 1.0f / sqrtf(s * inv_cols + eps);
#pragma unroll
                for (int t = 0; t < TY_CPL; ++t)
                    if (t < cpl && j + t * lpr < cols) yr[j + t * lpr] = xv[t] * scale * gv[t];
                continue;
            }
            const float mean = s * inv_cols;
            float var = 0.f;
#pragma unroll
            for (int t = 0; t < TY_CPL; ++t) {
                const float d = (t < cpl && j + t * lpr < cols) ? xv[t] - mean : 0.f;
                var += d * d;
            }
            var = group_sum(var, lpr);
            const float inv_std = 1.0f / sqrtf(var * inv_cols + eps);
#pragma unroll
            for (int t = 0; t < TY_CPL; ++t)
                if (t < cpl && j + t * lpr < cols) yr[j + t * lpr] = (xv[t] - mean) * inv_std * gv[t] + bv[t];
        }
        return;
    }
    const int lane = threadIdx.x & 63;
    for (int r = threadIdx.x >> 6; r < rows; r += TY_WAVES) {
        const float* xr = x + r * cols;
        float* yr = y + r * cols;
        float s = 0.f;
        for (int c = lane; c < cols; c += 64) s += RMS ? xr[c] * xr[c] : xr[c];
        s = wave_sum(s);
        if (RMS) {
            const float scale = 1.0f / sqrtf(s * inv_cols + eps);
            for (int c = lane; c < cols; c += 64) yr[c] = xr[c] * scale * g[c];
            continue;
        }
        const float mean = s * inv_cols;
        float var = 0.f;
        for (int c = lane; c < cols; c += 64) {
            const float d = xr[c] - mean;
            var += d * d;
        }
        var = wave_sum(var);
        const float inv_std = 1.0f / sqrtf(var * inv_cols + eps);
        for (int c = lane; c < cols; c += 64) yr[c] = (xr[c] - mean) * inv_std * g[c] + b[c];
    }
}

// Row softmax y = softmax(x) over `cols` of rows `ld` floats apart (x and y
// may be the same rows), lpr lanes per row (2^lg), cpl ≤ TY_CPL elements per
// lane.  With ATTN, scores above the causal diagonal are −∞ and the additive
// mask row (mask_row0 + r of mask, cols wide) is added: row r of the head
// group is query r mod S (divisor qm, qs; S = cols).
template <bool ATTN>
__device__ __forceinline__ void row_softmax(const float* x, float* y, int rows, int cols, int ld, int lpr, int lg,
                                            int cpl, bool causal, const float* mask, int mask_row0, int qm, int qs) {
    const int j = threadIdx.x & (lpr - 1);
    for (int r = threadIdx.x >> lg; r < rows; r += TY_NT >> lg) {
        const float* xr = x + r * ld;
        const int q = ATTN ? r - (int)lbr_fdiv(r, qm, qs) * cols : 0;
        float v[TY_CPL];
        float m = -INFINITY;
#pragma unroll
        for (int t = 0; t < TY_CPL; ++t) {
            const int c = j + t * lpr;
            float sv = -INFINITY;
            if (t < cpl && c < cols && !(ATTN && causal && c > q)) {
                sv = xr[c];
                if (ATTN && mask) sv += mask[(mask_row0 + r) * cols + c];
            }
            v[t] = sv;
            m = fmaxf(m, sv);
        }
        m = group_max(m, lpr);
        float l = 0.f;
#pragma unroll
        for (int t = 0; t < TY_CPL; ++t) {
            v[t] = v[t] == -INFINITY ? 0.f : expf(v[t] - m);
            l += v[t];
        }
        l = group_sum(l, lpr);
        const float inv_l = 1.0f / l;
        float* yr = y + r * ld;
#pragma unroll
        for (int t = 0; t < TY_CPL; ++t)
            if (t < cpl && j + t * lpr < cols) yr[j + t * lpr] = v[t] * inv_l;
    }
}

// SOFTMAX over the last dim (reduce.c:78-97): n[0] rows, n[1] cols, n[2] lpr,
// n[3] log2 lpr, n[4] cols per lane (0: a wavefront per row, wide rows).
__device__ __forceinline__ void t_softmax(const TyOp& o, const Node& d, char* lds) {
    const float* x = opnd(d, lds, 0);
    float* y = opnd(d, lds, 5);
    const int rows = d.n[0], cols = d.n[1];
    if (d.n[4] > 0) {
        row_softmax<false>(x, y, rows, cols, cols, d.n[2], d.n[3], d.n[4], false, nullptr, 0, 0, 0);
        return;
    }
    const int lane = threadIdx.x & 63;
    for (int r = threadIdx.x >> 6; r < rows; r += TY_WAVES) {
        const float* xr = x + r * cols;
        float* yr = y + r * cols;
        float m = -FLT_MAX;
        for (int c = lane; c < cols; c += 64) m = fmaxf(m, xr[c]);
        m = wave_max(m);
        float s = 0.f;
        for (int c = lane; c < cols; c += 64) {
            const float e = expf(xr[c] - m);
            yr[c] = e;
            s += e;
        }
        s = wave_sum(s);
        for (int c = lane; c < cols; c += 64) yr[c] = yr[c] / s;
    }
}

// Lane (kq, i) of a 16×16 MFMA block holds 4 consecutive k of row i of A and
// of column i of op(B), so MFMA q of a 16-wide K step reduces k = 4·kq + q;
// register r of lane (g, j) holds row 4·g + r, column j of the block.
__device__ __forceinline__ void load4(const float* r, int kk, int kn, bool vec, float v[4]) {
    if (vec && kk + 4 <= kn) {
        const float4 t = *reinterpret_cast<const float4*>(r + kk);
        v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = kk + q < kn ? r[kk + q] : 0.f;
    }
}

// 4 consecutive k of staged row r (see stage_rows; kk is a multiple of 4).
__device__ __forceinline__ void load4_staged(const float* row, int kk, int kn, int sw, int r, float v[4]) {
    if (kk + 4 <= kn) {
        const float4 t = *reinterpret_cast<const float4*>(row + 4 * ((kk >> 2) ^ (r & sw)));
        v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
    } else {   // the ragged end of an unswizzled row
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = kk + q < kn ? row[kk + q] : 0.f;
    }
}

// C[z] = alpha · A[z] · op(B[(zoff + z) / zdiv]) for z < Z: A rows lda apart;
// op(B) = Bᵀ of B stored [N][ldb] when BT, else B stored [K][ldb]; blocks of
// 16×16 over the wavefronts (block b → z = b / (bm·bn), divisor zm, zs; row
// block = rem / bn, divisor nm, ns), operands read where they are.
__device__ __forceinline__ void mm_direct(int Z, int M, int N, int K, const float* A, int sA, int lda, const float* B,
                                          int sB, int ldb, int zoff, int zdiv, bool BT, float* C, int sC, int ldc,
                                          float alpha, int bm, int bn, int zm, int zs, int nm, int ns) {
    const int lane = threadIdx.x & 63, kq = lane >> 4, li = lane & 15;
    const int nblk = Z * bm * bn;
    const bool avec = ((unsigned long long)A & 15) == 0 && lda % 4 == 0 && sA % 4 == 0;
    const bool bvec = BT && ((unsigned long long)B & 15) == 0 && ldb % 4 == 0 && sB % 4 == 0;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int blk = wave; blk < nblk; blk += TY_WAVES) {
        const int z = (int)lbr_fdiv(blk, zm, zs), rem = blk - z * bm * bn;
        const int mb = (int)lbr_fdiv(rem, nm, ns);
        const int m0 = mb * 16, n0 = (rem - mb * bn) * 16;
        const float* Ar = A + z * sA + min(m0 + li, M - 1) * lda;
        const float* Bb = B + ((zoff + z) / zdiv) * sB;
        const int nb = min(n0 + li, N - 1);
        floatx4 c = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < K; k0 += 16) {
            const int kk = k0 + 4 * kq;
            float av[4], bv[4];
            load4(Ar, kk, K, avec, av);
            if (BT) {
                load4(Bb + nb * ldb, kk, K, bvec, bv);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) bv[q] = kk + q < K ? Bb[(kk + q) * ldb + nb] : 0.f;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[q], bv[q], c, 0, 0, 0);
        }
        if (n0 + li < N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 4 * kq + r;
                if (m < M) C[z * sC + m * ldc + n0 + li] = alpha * c[r];
            }
        }
    }
}

// Copy rows [0, rows) × columns [k0, k0 + kn) of a row-major matrix (rows ld
// floats apart) into the staging area with rows `st` floats apart.  With
// vec, 4-float chunk c of row r lands at chunk c ^ (r & sw): the 16 rows an
// MFMA step reads at one chunk then sit in different LDS banks without
// padding the rows (sw + 1 divides the chunks per row).
template <int U>
__device__ __forceinline__ void stage_rows(const float* src, int rows, int ld, int k0, int kn, float* dst, int st,
                                           bool vec, int sw) {
    if (vec) {   // ld, k0, kn and st multiples of 4, src 16-byte aligned
        const unsigned q4 = kn >> 2;
        each<U>(rows * (int)q4, [&](int i) {
            const unsigned r = (unsigned)i / q4, c = (unsigned)i - r * q4;
            return *reinterpret_cast<const float4*>(src + r * ld + k0 + 4 * c);
        }, [&](int i, float4 v) {
            const unsigned r = (unsigned)i / q4, c = (unsigned)i - r * q4;
            *reinterpret_cast<float4*>(dst + r * st + 4 * (c ^ (r & sw))) = v;
        });
    } else {
        each<U>(rows * kn, [&](int i) {
            const unsigned r = (unsigned)i / (unsigned)kn, c = (unsigned)i - r * kn;
            return src[r * ld + k0 + c];
        }, [&](int i, float v) {
            const unsigned r = (unsigned)i / (unsigned)kn, c = (unsigned)i - r * kn;
            dst[r * st + c] = v;
        });
    }
}

// MATMUL / MATMUL_ADD (executor.c:197-224, 312-346): MATMUL_ADD adds bias[n]
// with alpha fixed to 1 (f[0] = alpha).  n[0] M, n[1] N, n[2] K, n[3]
// batches, n[4] G_* flags, n[5] K chunk kc, n[6] staged B row stride, n[7]
// staged A row stride, n[8] bm, n[9] bn, n[10] output blocks, n[11] K split
// ks, n[12] staged B offset, n[13] staged A offset, n[14] split partials
// offset (LDS bytes), n[15..16] divisor bm·bn, n[17..18] divisor bn,
// n[19..20] divisor of the block count, n[21] / n[22] chunk swizzle of the
// staged B / A rows (0: rows padded instead).
// Work items (block, K split) go to the wavefronts, TY_BPW per wavefront per
// pass; split s takes the 16-wide K steps s, s + ks, ..; with ks > 1 (one
// pass, one chunk) splits 1.. leave partial sums in LDS for split 0.
__device__ __forceinline__ void t_gemm(const TyOp& o, const Node& d, char* lds) {
    const float* A = opnd(d, lds, 0);
    const float* B = opnd(d, lds, 1);
    const float* bias = opnd(d, lds, 2);
    float* C = opnd(d, lds, 5);
    const int M = d.n[0], N = d.n[1], K = d.n[2], fl = d.n[4], kc = d.n[5];
    const int kbs = d.n[6], kas = d.n[7], swb = rf(o.n[21]), swa = rf(o.n[22]);
    const int bm = rf(o.n[8]), bn = rf(o.n[9]), nblk = rf(o.n[10]), ks = rf(o.n[11]);
    const int zm = rf(o.n[15]), zs = rf(o.n[16]), bnm = rf(o.n[17]), bns = rf(o.n[18]);
    const int sm = rf(o.n[19]), ss = rf(o.n[20]);
    const bool trans_b = fl & G_TRANS_B, b2d = fl & G_B2D, has_bias = fl & G_BIAS;
    const bool sb = fl & G_STAGE_B, sa = fl & G_STAGE_A, bvec = fl & G_B_VEC, avec = fl & G_A_VEC;
    float* SB = reinterpret_cast<float*>(lds + rf(o.n[12]));
    float* SA = reinterpret_cast<float*>(lds + rf(o.n[13]));
    float* RED = reinterpret_cast<float*>(lds + rf(o.n[14]));
    const float alpha = d.f[0];
    const int lane = threadIdx.x & 63, kq = lane >> 4, li = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int items = nblk * ks;
    const bool once = kc == K;
    // U loads in flight per thread: 4 for the one-off copy, 2 inside the pass
    // loop, where the accumulators hold registers
    auto stage = [&](int k0, int kn, auto u) {
        constexpr int U = decltype(u)::value;
        if (sb) {
            if (trans_b) stage_rows<U>(B, N, K, k0, kn, SB, kbs, bvec, swb);
            else stage_rows<U>(B + k0 * N, kn, N, 0, N, SB, N, bvec, 0);
        }
        if (sa) stage_rows<U>(A, M, K, k0, kn, SA, kas, avec, swa);
    };
    if (once && (sa || sb)) {
        stage(0, K, std::integral_constant<int, 4>());
        __syncthreads();
    }
    for (int pass = 0; pass < items; pass += TY_WAVES * TY_BPW) {
        floatx4 acc[TY_BPW];
#pragma unroll
        for (int b = 0; b < TY_BPW; ++b) acc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < K; k0 += kc) {
            const int kn = min(kc, K - k0);
            if (!once && (sa || sb)) {
                __syncthreads();   // the previous chunk's readers are done
                stage(k0, kn, std::integral_constant<int, 2>());
                __syncthreads();
            }
#pragma unroll
            for (int b = 0; b < TY_BPW; ++b) {
                const int item = pass + wave + b * TY_WAVES;
                if (item >= items) continue;   // uniform per wavefront
                const int split = (int)lbr_fdiv(item, sm, ss), blk = item - split * nblk;
                const int bz = (int)lbr_fdiv(blk, zm, zs), rem = blk - bz * bm * bn;
                const int mb = (int)lbr_fdiv(rem, bnm, bns);
                const int m0 = mb * 16, n0 = (rem - mb * bn) * 16;
                const int ma = min(m0 + li, M - 1), nb = min(n0 + li, N - 1);
                const float* Bz = B + (b2d ? 0 : bz * N * K);
                const float* Ar = sa ? SA + ma * kas : A + (bz * M + ma) * K + k0;
                const float* Br = sb ? (trans_b ? SB + nb * kbs : SB + nb)
                                     : (trans_b ? Bz + nb * K + k0 : Bz + k0 * N + nb);
                floatx4 c = acc[b];
                for (int kl = split * 16; kl < kn; kl += 16 * ks) {
                    const int kk = kl + 4 * kq;
                    float av[4], bv[4];
                    if (sa) load4_staged(Ar, kk, kn, swa, ma, av);
                    else load4(Ar, kk, kn, avec, av);
                    if (trans_b) {
                        if (sb) load4_staged(Br, kk, kn, swb, nb, bv);
                        else load4(Br, kk, kn, bvec, bv);
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q) bv[q] = kk + q < kn ? Br[(kk + q) * N] : 0.f;
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[q], bv[q], c, 0, 0, 0);
                }
                acc[b] = c;
            }
        }
        if (ks > 1) {   // one pass: splits 1.. hand their partial sums to split 0
#pragma unroll
            for (int b = 0; b < TY_BPW; ++b) {
                const int item = pass + wave + b * TY_WAVES;
                if (item >= items || item < nblk) continue;
                float* dst = RED + ((item - nblk) * 64 + lane) * 4;
                *reinterpret_cast<float4*>(dst) = float4{acc[b][0], acc[b][1], acc[b][2], acc[b][3]};
            }
            __syncthreads();
#pragma unroll
            for (int b = 0; b < TY_BPW; ++b) {
                const int item = pass + wave + b * TY_WAVES;
                if (item >= nblk) continue;
                for (int s = 1; s < ks; ++s) {
                    const float4 t = *reinterpret_cast<const float4*>(RED + (((s - 1) * nblk + item) * 64 + lane) * 4);
                    acc[b][0] += t.x, acc[b][1] += t.y, acc[b][2] += t.z, acc[b][3] += t.w;
                }
            }
        }
#pragma unroll
        for (int b = 0; b < TY_BPW; ++b) {
            const int item = pass + wave + b * TY_WAVES;
            if (item >= items || item >= nblk) continue;   // split 0 writes
            const int bz = (int)lbr_fdiv(item, zm, zs), rem = item - bz * bm * bn;
            const int mb = (int)lbr_fdiv(rem, bnm, bns);
            const int m0 = mb * 16, nn = (rem - mb * bn) * 16 + li;
            if (nn >= N) continue;
            const float bi = has_bias ? bias[nn] : 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 4 * kq + r;
                if (m < M) C[(bz * M + m) * N + nn] = has_bias ? acc[b][r] + bi : alpha * acc[b][r];
            }
        }
    }
}

// ATTENTION (attn.c:26-80, 121-253): scores q·k/√hd (+ mask), causal −∞
// above the diagonal, softmax, ·V; kv head = head / group.  Per group of hg
// heads, three steps a barrier apart: the scores as a batched GEMM on the
// matrix cores into the staging area (rows ld floats apart), the masked row
// softmax in place, and P·V as a second GEMM.  n[0] bh, n[1] S, n[2] hd,
// n[3] group, n[4] causal, n[5] has mask, n[6] hg, n[7] score row stride,
// n[8] lpr, n[9] log2 lpr, n[10] cols per lane, n[11] staging offset,
// n[12] bm = bn of the scores, n[13] bn of P·V, n[14..15] divisor S,
// n[16..17] divisor bm², n[18..19] divisor bm, n[20..21] divisor bm·bn2,
// n[22..23] divisor bn2; f[0] = 1/√hd.
__device__ __forceinline__ void t_attention(const TyOp& o, const Node& d, char* lds) {
    const float* Q = opnd(d, lds, 0);
    const float* Kt = opnd(d, lds, 1);
    const float* V = opnd(d, lds, 2);
    const float* mask = d.n[5] ? opnd(d, lds, 3) : nullptr;
    float* O = opnd(d, lds, 5);
    const int bh = d.n[0], S = d.n[1], hd = d.n[2], group = d.n[3], hg = d.n[6], ld = d.n[7];
    const bool causal = d.n[4] != 0;
    float* sc = reinterpret_cast<float*>(lds + rf(o.n[11]));
    const int bm = rf(o.n[12]), bn2 = rf(o.n[13]);
    for (int h0 = 0; h0 < bh; h0 += hg) {
        const int nh = min(hg, bh - h0);
        mm_direct(nh, S, S, hd, Q + h0 * S * hd, S * hd, hd, Kt, S * hd, hd, h0, group, true, sc, S * ld, ld, d.f[0],
                  bm, bm, rf(o.n[16]), rf(o.n[17]), rf(o.n[18]), rf(o.n[19]));
        __syncthreads();
        row_softmax<true>(sc, sc, nh * S, S, ld, rf(o.n[8]), rf(o.n[9]), rf(o.n[10]), causal, mask, h0 * S,
                          rf(o.n[14]), rf(o.n[15]));
        __syncthreads();
        mm_direct(nh, S, hd, S, sc, S * ld, ld, V, S * hd, hd, h0, group, false, O + h0 * S * hd, S * hd, hd, 1.0f,
                  bm, bn2, rf(o.n[20]), rf(o.n[21]), rf(o.n[22]), rf(o.n[23]));
        if (h0 + hg < bh) __syncthreads();   // the scores area is free for the next head group
    }
}

// Copies in 4-byte words (elem_size 4 or 8): RESHAPE, SLICE, TRANSPOSE, CAT
// (shape.c:92-138, executor.c:228-282).  SLICE: n[0] inner words, n[1] len,
// n[2] orig, n[3] start, n[4..5] divisor inner, n[6..7] divisor len.
// TRANS2D: n[0] rows, n[1] cols, n[2] log2 words per element, n[3..4]
// divisor rows.  SWAP [outer, A, mid, B, inner] → [outer, B, mid, A, inner]:
// n[0] A, n[1] mid, n[2] B, n[3] inner words, then divisors of inner, A,
// mid, B at n[4..11].  CAT: n[0] inputs (≤ 4), n[1] output row words, input
// k at n[2 + 4k ..]: segment words, its divisor, offset in the row.
__device__ __forceinline__ void t_copy(const TyOp& o, const Node& d, char* lds) {
    const unsigned* in = opnd_u(d, lds, 0);
    unsigned* out = opnd_u(d, lds, 5);
    auto st = [&](int i, unsigned v) { out[i] = v; };
    switch (d.kind) {
        case TY_COPY:
            each<4>(d.total, [&](int i) { return in[i]; }, st);
            break;
        case TY_SLICE: {   // index arithmetic per element: 2 per thread per round
            const unsigned inner = d.n[0], len = d.n[1], orig = d.n[2], start = d.n[3];
            each<2>(d.total, [&](int i) {
                const unsigned r = lbr_fdiv(i, d.n[4], d.n[5]), x = (unsigned)i - r * inner;
                const unsigned ob = lbr_fdiv(r, d.n[6], d.n[7]), l = r - ob * len;
                return in[(ob * orig + start + l) * inner + x];
            }, st);
            break;
        }
        case TY_TRANS2D: {   // in [rows, cols] → out [cols, rows]
            const unsigned rows = d.n[0], cols = d.n[1], lw = d.n[2];
            each<2>(d.total, [&](int i) {
                const unsigned e = (unsigned)i >> lw, x = (unsigned)i & ((1u << lw) - 1);
                const unsigned c = lbr_fdiv(e, d.n[3], d.n[4]), r = e - c * rows;
                return in[((r * cols + c) << lw) + x];
            }, st);
            break;
        }
        case TY_SWAP: {
            const unsigned A = d.n[0], mid = d.n[1], B = d.n[2], inner = d.n[3];
            const int m8 = rf(o.n[8]), s9 = rf(o.n[9]), m10 = rf(o.n[10]), s11 = rf(o.n[11]);
            each<2>(d.total, [&](int i) {
                unsigned r = (unsigned)i, q;
                q = lbr_fdiv(r, d.n[4], d.n[5]);
                const unsigned x = r - q * inner;
                r = q;
                q = lbr_fdiv(r, d.n[6], d.n[7]);
                const unsigned a = r - q * A;
                r = q;
                q = lbr_fdiv(r, m8, s9);
                const unsigned m = r - q * mid;
                r = q;
                q = lbr_fdiv(r, m10, s11);
                const unsigned b = r - q * B;
                return in[(((q * A + a) * mid + m) * B + b) * inner + x];
            }, st);
            break;
        }
        default: {   // TY_CAT
            const unsigned row = d.n[1];
            const int outer = d.total / (int)row;
            for (int k = 0; k < d.n[0]; ++k) {
                // input k of a runtime loop: from the record (a Node field at a runtime index would go to scratch)
                const unsigned long long pk = rf64(o.p[k]);
                const unsigned* src = ((d.lds >> k) & 1) ? reinterpret_cast<const unsigned*>(lds + pk)
                                                         : reinterpret_cast<const unsigned*>(pk);
                const int* e = o.n + 2 + 4 * k;
                const unsigned seg = rf(e[0]), off = rf(e[3]);
                each<2>(outer * (int)seg, [&](int i) { return src[i]; }, [&](int i, unsigned v) {
                    const unsigned ob = lbr_fdiv(i, rf(e[1]), rf(e[2]));
                    out[ob * row + off + ((unsigned)i - ob * seg)] = v;
                });
            }
        }
    }
}

// recs: the n records then the n_pf prefetch ranges (address, lines before
// it, lines), copied to LDS at rec_off; wb: the write-back ranges.
__global__ __launch_bounds__(TY_NT) void tiny_graph(const float4* __restrict__ recs, int n, int n_pf, int rec_off,
                                                    const long long* __restrict__ wb, int n_wb,
                                                    unsigned long long lo) {
    __shared__ __attribute__((aligned(16))) float4 lds4[TY_LDS / 16];
    char* lds = reinterpret_cast<char*>(lds4);
    // the records into LDS: one round trip for all of them
    {
        float4* dst = reinterpret_cast<float4*>(lds + rec_off);
        const int n4 = (n * (int)sizeof(TyOp) + n_pf * 24 + 15) / 16;
        each<2>(n4, [&](int i) { return recs[i]; }, [&](int i, float4 v) { dst[i] = v; });
    }
    __syncthreads();
    const TyOp* ops = reinterpret_cast<const TyOp*>(lds + rec_off);
    // Touch every 128-byte line of the global operands (weights, biases,
    // inputs) once, all lines in flight together: the nodes' own reads of
    // them then hit L2 instead of paying a trip to HBM each.
    if (n_pf > 0) {
        const long long* pf = reinterpret_cast<const long long*>(lds + rec_off + n * sizeof(TyOp));
        const int lines = (int)(pf[3 * (n_pf - 1) + 1] + pf[3 * (n_pf - 1) + 2]);
        unsigned acc = 0;
        for (int base = threadIdx.x; base < lines; base += 4 * TY_NT) {
            unsigned v[4] = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int l = base + u * TY_NT;
                if (l >= lines) continue;
                int r = 0;
                while (r + 1 < n_pf && pf[3 * (r + 1) + 1] <= l) ++r;
                v[u] = *reinterpret_cast<const unsigned*>(
                    static_cast<uintptr_t>(pf[3 * r] + (unsigned long long)(l - pf[3 * r + 1]) * 128));
            }
            acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
        }
        if (acc == 0x9e3779b9u && n_wb < 0) lds4[0].x = 0.f;   // keeps the loads; n_wb is never negative
    }
    for (int i = 0; i < n; ++i) {
        const TyOp& o = ops[i];
        const Node d = read_node(&o);
        switch (d.kind) {
            case TY_UNARY:
                switch (d.sub) {
                    case OP_RELU: t_unary<OP_RELU>(o, d, lds); break;
                    case OP_EXP: t_unary<OP_EXP>(o, d, lds); break;
                    case OP_TANH: t_unary<OP_TANH>(o, d, lds); break;
                    case OP_POW: t_unary<OP_POW>(o, d, lds); break;
                    case OP_GELU: t_unary<OP_GELU>(o, d, lds); break;
                    case OP_RSQRT: t_unary<OP_RSQRT>(o, d, lds); break;
                    case OP_SILU: t_unary<OP_SILU>(o, d, lds); break;
                    case OP_NEG: t_unary<OP_NEG>(o, d, lds); break;
                    case OP_COS: t_unary<OP_COS>(o, d, lds); break;
                    default: t_unary<OP_SIN>(o, d, lds); break;
                }
                break;
            case TY_BIN_SAME: case TY_BIN_SCALAR: case TY_BIN_ROW: case TY_BIN_BCAST:
                switch (d.sub) {
                    case 0: t_binary<0>(o, d, lds); break;
                    case 1: t_binary<1>(o, d, lds); break;
                    case 2: t_binary<2>(o, d, lds); break;
                    default: t_binary<3>(o, d, lds); break;
                }
                break;
            case TY_BIAS_RELU: t_bias_relu(o, d, lds); break;
            case TY_GATED:
                if (d.sub == 0) {
                    if (d.n[3]) t_gated<true, true>(o, d, lds);
                    else t_gated<true, false>(o, d, lds);
                } else {
                    if (d.n[3]) t_gated<false, true>(o, d, lds);
                    else t_gated<false, false>(o, d, lds);
                }
                break;
            case TY_NORM:
                if (d.sub) t_norm<true>(o, d, lds);
                else t_norm<false>(o, d, lds);
                break;
            case TY_SOFTMAX: t_softmax(o, d, lds); break;
            case TY_GEMM: t_gemm(o, d, lds); break;
            case TY_ATTN: t_attention(o, d, lds); break;
            default: t_copy(o, d, lds); break;
        }
        __syncthreads();   // the node's writes are visible to every wavefront of the next
    }
    // the caller-visible ranges back to global memory
    for (int r = 0; r < n_wb; ++r) {
        const long long off = wb[2 * r], bytes = wb[2 * r + 1];
        const unsigned* src = reinterpret_cast<const unsigned*>(lds + off);
        unsigned* dst = reinterpret_cast<unsigned*>(static_cast<uintptr_t>(lo + off));
        each<4>((int)(bytes / 4), [&](int i) { return src[i]; }, [&](int i, unsigned v) { dst[i] = v; });
    }
}

void launch_tiny(const Step& s, hipStream_t st) {
    hipLaunchKernelGGL(tiny_graph, dim3(1), dim3(TY_NT), 0, st, (const float4*)s.in[0], (int)s.i[0], (int)s.i[3],
                       (int)s.i[4], (const long long*)s.in[1], (int)s.i[1], (unsigned long long)s.i[2]);
}

// ---------------------------------------------------------------------------
// Host side: eligibility, LDS layout, node decoding
// ---------------------------------------------------------------------------

struct Range {
    unsigned long long lo, hi;
};

std::vector<Range> merged(std::vector<Range> v) {
    std::sort(v.begin(), v.end(), [](const Range& a, const Range& b) { return a.lo < b.lo; });
    std::vector<Range> out;
    for (const Range& r : v) {
        if (r.hi <= r.lo) continue;
        if (!out.empty() && r.lo <= out.back().hi) out.back().hi = std::max(out.back().hi, r.hi);
        else out.push_back(r);
    }
    return out;
}

bool f32_op(int op) {
    switch (op) {
        case OP_RELU: case OP_EXP: case OP_TANH: case OP_POW: case OP_GELU: case OP_RSQRT: case OP_SILU:
        case OP_NEG: case OP_COS: case OP_SIN: case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV:
        case OP_FUSED_BIAS_RELU: case OP_GATED_ACT: case OP_LAYERNORM: case OP_RMSNORM: case OP_SOFTMAX:
        case OP_MATMUL: case OP_MATMUL_ADD: case OP_ATTENTION:
            return true;
        default:
            return false;
    }
}

bool copy_op(int op) { return op == OP_RESHAPE || op == OP_SLICE || op == OP_TRANSPOSE || op == OP_CAT; }

// Inputs the interpreter reads (scalar-mode binaries ignore a second input;
// attention's planner scratch slot is not read).
int reads_of(const OpNode* nd) {
    switch (nd->op) {
        case OP_ADD: return nd->extra[0] == 2 ? 1 : 2;
        case OP_SUB: case OP_MUL: case OP_DIV: return nd->extra[0] == 1 ? 1 : 2;
        case OP_FUSED_BIAS_RELU: return 2;
        case OP_GATED_ACT: return nd->extra[0] != 0 ? 3 : 2;
        case OP_LAYERNORM: return 3;
        case OP_RMSNORM: return 2;
        case OP_MATMUL: return 2;
        case OP_MATMUL_ADD: return 3;
        case OP_ATTENTION: return 3 + (nd->extra[3] != 0);
        case OP_CAT: return nd->n_inputs;
        default: return 1;   // unary, SOFTMAX, RESHAPE, SLICE, TRANSPOSE
    }
}

int log2_of(int x) {
    int l = 0;
    while ((1 << l) < x) ++l;
    return l;
}

// Lanes per row for a row operation over `rows` rows of `cols`: enough that
// cols / lpr ≤ TY_CPL (registers), then more while that still leaves half
// the workgroup's lanes idle (each extra lane adds a shuffle step per row).
// cpl = 0: the row does not fit the registers (a wavefront per row).
void row_lanes(long long rows, int cols, int* lpr, int* cpl) {
    int l = 1;
    while (l < 64 && (cols + l - 1) / l > TY_CPL) l <<= 1;
    while (l < 64 && l < cols && rows * l * 2 <= TY_NT / 2) l <<= 1;
    *lpr = l;
    *cpl = (cols + l - 1) / l > TY_CPL ? 0 : (cols + l - 1) / l;
}

struct Ctx {
    unsigned long long lo, hi;   // the window
    int stage_off, stage_bytes;  // LDS staging area
};

void set_opnd(TyOp* o, int k, const void* p, const Ctx& c) {
    const unsigned long long a = (unsigned long long)p;
    if (a >= c.lo && a < c.hi) {
        o->lds |= 1 << k;
        o->p[k] = a - c.lo;
    } else {
        o->p[k] = a;
    }
}

// Broadcast extras [mode, nd, a strides, b strides, out shape] merged to at
// most 4 dims: size-1 dims dropped, neighbours that stay linear for both
// operands joined.
bool pack_bcast(const OpNode* nd_, TyOp* o) {
    const int* x = nd_->extra;
    const int nd = x[1];
    if (nd < 1 || 2 + 3 * nd > MAX_DIMS) return false;
    long long cs[MAX_DIMS], ca[MAX_DIMS], cb[MAX_DIMS];
    int cn = 0;
    for (int d = 0; d < nd; ++d) {
        const long long size = x[2 + 2 * nd + d], as = x[2 + d], bs = x[2 + nd + d];
        if (size == 1) continue;
        if (cn > 0 && ca[cn - 1] == as * size && cb[cn - 1] == bs * size) {
            cs[cn - 1] *= size;
            ca[cn - 1] = as;
            cb[cn - 1] = bs;
            continue;
        }
        cs[cn] = size, ca[cn] = as, cb[cn] = bs;
        ++cn;
    }
    if (cn > 4) return false;
    o->n[0] = cn;
    for (int d = 0; d < cn; ++d) {
        int* e = o->n + 1 + 5 * d;
        e[0] = (int)cs[d], e[1] = (int)ca[d], e[2] = (int)cb[d];
        lbr_fast_divisor((unsigned)cs[d], &e[3], &e[4]);
    }
    return true;
}

long long round4(long long x) { return (x + 3) & ~3LL; }

// XOR mask over the 4-float chunks of a staged row of kc floats: the largest
// power of two (at most 16) dividing the chunk count, minus one; 0 when kc is
// not a multiple of 4 or a row is one chunk (the rows are padded then).
int chunk_swizzle(int kc) {
    if (kc <= 0 || kc % 4) return 0;
    const int chunks = kc / 4;
    int p = 1;
    while (p < 16 && chunks % (p * 2) == 0) p *= 2;
    return p - 1;
}

// GEMM staging, chunking and K split (see t_gemm).  Staging needs one batch
// (a shared B, an A of M rows): B and A with padded rows when both fit with
// the whole K, else the largest 16-multiple K chunk with both, else with B
// alone; none of it, and the operands are read where they are.
bool plan_gemm(const OpNode* nd, const Ctx& c, TyOp* o) {
    const long long total = node_total(nd);
    const int N = node_last_dim(nd);
    const int K = nd->extra[0];
    const bool trans_b = nd->extra[1] != 0, b2d = nd->extra[2] != 0;
    if (N <= 0 || total == 0 || K < 0) return false;
    const long long M = b2d ? total / N : nd->out_shape[nd->n_dims - 2];
    if (M <= 0) return false;
    const long long batches = b2d ? 1 : total / (M * N);
    const long long bm = (M + 15) / 16, bn = (N + 15) / 16, nblk = batches * bm * bn;
    if (M * K >= (1LL << 31) || (long long)N * K >= (1LL << 31) || nblk * 16 >= (1LL << 31)) return false;
    int fl = (trans_b ? G_TRANS_B : 0) | (b2d ? G_B2D : 0) | (nd->op == OP_MATMUL_ADD ? G_BIAS : 0);
    const bool bv = lbr_aligned(nd->inputs[1], 16) && (trans_b ? K % 4 == 0 : N % 4 == 0);
    const bool av = lbr_aligned(nd->inputs[0], 16) && K % 4 == 0;
    if (bv) fl |= G_B_VEC;
    if (av) fl |= G_A_VEC;
    const long long avail = c.stage_bytes / 4;   // floats
    // rows of kc floats when the chunk swizzle applies, else padded by 4
    auto row_floats = [&](long long kc, bool vec) { return vec && chunk_swizzle((int)kc) ? kc : round4(kc) + 4; };
    auto b_floats = [&](long long kc) { return round4(trans_b ? N * row_floats(kc, bv) : kc * N); };
    auto a_floats = [&](long long kc) { return M * row_floats(kc, av); };
    int kc = K;
    bool sb = false, sa = false;
    if (batches == 1 && K > 0) {
        if (b_floats(K) + a_floats(K) <= avail) {
            sb = sa = true;
        } else {
            for (int with_a = 1; with_a >= 0 && !sb; --with_a) {
                long long k = K;
                while (k > 0 && b_floats(k) + (with_a ? a_floats(k) : 0) > avail) k = (k - 1) & ~15LL;
                if (k >= 16 || k == K) {
                    kc = (int)k, sb = true, sa = with_a;
                }
            }
        }
    }
    if (!sb) kc = K;
    // K split over the wavefronts for small block counts (one pass, one chunk)
    int ks = 1;
    const long long used = (sb ? b_floats(kc) : 0) + (sa ? a_floats(kc) : 0);
    if (kc == K) {
        while (ks * 2 * nblk <= TY_WAVES && ks * 2 * 16 <= K && used + (long long)(ks * 2 - 1) * nblk * 256 <= avail)
            ks *= 2;
    }
    if (sb) fl |= G_STAGE_B;
    if (sa) fl |= G_STAGE_A;
    const int swb = sb && trans_b && bv ? chunk_swizzle(kc) : 0, swa = sa && av ? chunk_swizzle(kc) : 0;
    const int kbs = !trans_b ? N : swb ? kc : (int)round4(kc) + 4, kas = swa ? kc : (int)round4(kc) + 4;
    o->kind = TY_GEMM;
    o->total = (int)total;
    o->n[0] = (int)M, o->n[1] = N, o->n[2] = K, o->n[3] = (int)batches, o->n[4] = fl;
    o->n[5] = kc, o->n[6] = kbs, o->n[7] = kas, o->n[21] = swb, o->n[22] = swa;
    o->n[8] = (int)bm, o->n[9] = (int)bn, o->n[10] = (int)nblk, o->n[11] = ks;
    o->n[12] = c.stage_off;
    o->n[13] = c.stage_off + (int)((sb ? b_floats(kc) : 0) * 4);
    o->n[14] = o->n[13] + (int)((sa ? a_floats(kc) : 0) * 4);
    lbr_fast_divisor((unsigned)(bm * bn), &o->n[15], &o->n[16]);
    lbr_fast_divisor((unsigned)bn, &o->n[17], &o->n[18]);
    lbr_fast_divisor((unsigned)nblk, &o->n[19], &o->n[20]);
    o->f[0] = nd->op == OP_MATMUL_ADD ? 1.0f : (nd->extra[3] ? __builtin_bit_cast(float, nd->extra[3]) : 1.0f);
    set_opnd(o, 0, nd->inputs[0], c);
    set_opnd(o, 1, nd->inputs[1], c);
    if (nd->op == OP_MATMUL_ADD) set_opnd(o, 2, nd->inputs[2], c);
    return true;
}

bool plan_attention(const OpNode* nd, const Ctx& c, TyOp* o) {
    const int S = nd->extra[0], hd = nd->extra[1], group = nd->extra[4] > 0 ? nd->extra[4] : 1;
    long long bh = 1;
    for (int i = 0; i < nd->n_dims - 2; ++i) bh *= nd->out_shape[i];
    if (S <= 0 || hd <= 0 || bh <= 0 || bh % group != 0) return false;
    const int ld = (int)round4(S) + 4;   // padded score rows: the 16 rows an MFMA reads hit different banks
    const long long per_head = (long long)S * ld;
    const long long hg = std::min<long long>(bh, (c.stage_bytes / 4) / per_head);
    if (hg < 1) return false;
    int lpr, cpl;
    row_lanes(hg * S, S, &lpr, &cpl);
    if (cpl == 0) return false;
    const int bm = (S + 15) / 16, bn2 = (hd + 15) / 16;
    o->kind = TY_ATTN;
    o->total = (int)(bh * S * hd);
    o->n[0] = (int)bh, o->n[1] = S, o->n[2] = hd, o->n[3] = group, o->n[4] = nd->extra[2] != 0;
    o->n[5] = nd->extra[3] != 0, o->n[6] = (int)hg, o->n[7] = ld, o->n[8] = lpr, o->n[9] = log2_of(lpr);
    o->n[10] = cpl, o->n[11] = c.stage_off, o->n[12] = bm, o->n[13] = bn2;
    lbr_fast_divisor((unsigned)S, &o->n[14], &o->n[15]);
    lbr_fast_divisor((unsigned)(bm * bm), &o->n[16], &o->n[17]);
    lbr_fast_divisor((unsigned)bm, &o->n[18], &o->n[19]);
    lbr_fast_divisor((unsigned)(bm * bn2), &o->n[20], &o->n[21]);
    lbr_fast_divisor((unsigned)bn2, &o->n[22], &o->n[23]);
    o->f[0] = 1.0f / sqrtf((float)hd);   // attn.c:68/242
    for (int k = 0; k < 3 + (nd->extra[3] != 0); ++k) set_opnd(o, k, nd->inputs[k], c);
    return true;
}

// The TyOp of one node, or false when the interpreter cannot take it.
bool build_op(const OpNode* nd, const Ctx& c, TyOp* o) {
    memset(o, 0, sizeof(*o));
    const long long total = node_total(nd);
    if (total * (nd->elem_size / 4) >= (1LL << 31) / 2) return false;
    o->total = (int)total;
    const int N = node_last_dim(nd) > 0 ? node_last_dim(nd) : 1;
    bool ok = true;
    switch (nd->op) {
        case OP_RELU: case OP_EXP: case OP_TANH: case OP_POW: case OP_GELU:
        case OP_RSQRT: case OP_SILU: case OP_NEG: case OP_COS: case OP_SIN:
            o->kind = TY_UNARY;
            o->sub = nd->op;
            o->f[0] = nd->op == OP_POW ? __builtin_bit_cast(float, nd->extra[0]) : 0.f;
            set_opnd(o, 0, nd->inputs[0], c);
            break;
        case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV: {
            o->sub = nd->op == OP_ADD ? 0 : nd->op == OP_SUB ? 1 : nd->op == OP_MUL ? 2 : 3;
            const int mode = nd->extra[0];
            o->kind = nd->op == OP_ADD ? (mode == 2 ? TY_BIN_SCALAR : mode == 1 ? TY_BIN_SAME
                                          : mode == 3 ? TY_BIN_BCAST : TY_BIN_ROW)
                                       : (mode == 1 ? TY_BIN_SCALAR : mode == 2 ? TY_BIN_BCAST : TY_BIN_SAME);
            set_opnd(o, 0, nd->inputs[0], c);
            if (o->kind == TY_BIN_SCALAR) {
                o->f[0] = __builtin_bit_cast(float, nd->extra[1]);
                break;
            }
            set_opnd(o, 1, nd->inputs[1], c);
            if (o->kind == TY_BIN_ROW) {
                o->n[0] = N;
                lbr_fast_divisor((unsigned)N, &o->n[1], &o->n[2]);
            } else if (o->kind == TY_BIN_BCAST) {
                ok = pack_bcast(nd, o);
            }
            break;
        }
        case OP_FUSED_BIAS_RELU:
            o->kind = TY_BIAS_RELU;
            o->n[0] = N;
            lbr_fast_divisor((unsigned)N, &o->n[1], &o->n[2]);
            set_opnd(o, 0, nd->inputs[0], c);
            set_opnd(o, 1, nd->inputs[1], c);
            break;
        case OP_GATED_ACT: {   // inputs [x, up] or [x, bias, up]
            const bool hb = nd->extra[0] != 0;
            o->kind = TY_GATED;
            o->sub = nd->extra[1] == 0 ? 0 : 1;
            o->n[0] = N;
            lbr_fast_divisor((unsigned)N, &o->n[1], &o->n[2]);
            o->n[3] = hb;
            set_opnd(o, 0, nd->inputs[0], c);
            set_opnd(o, 1, hb ? nd->inputs[2] : nd->inputs[1], c);
            if (hb) set_opnd(o, 2, nd->inputs[1], c);
            break;
        }
        case OP_LAYERNORM: case OP_RMSNORM: case OP_SOFTMAX: {
            const int cols = node_last_dim(nd);
            if (cols <= 0) return false;
            const long long rows = total / cols;
            int lpr, cpl;
            row_lanes(rows, cols, &lpr, &cpl);
            o->kind = nd->op == OP_SOFTMAX ? TY_SOFTMAX : TY_NORM;
            o->sub = nd->op == OP_RMSNORM;
            o->n[0] = (int)rows, o->n[1] = cols, o->n[2] = lpr, o->n[3] = log2_of(lpr), o->n[4] = cpl;
            o->f[0] = nd->op == OP_SOFTMAX ? 0.f : __builtin_bit_cast(float, nd->extra[0]);
            o->f[1] = 1.0f / cols;
            set_opnd(o, 0, nd->inputs[0], c);
            if (nd->op != OP_SOFTMAX) set_opnd(o, 1, nd->inputs[1], c);
            if (nd->op == OP_LAYERNORM) set_opnd(o, 2, nd->inputs[2], c);
            break;
        }
        case OP_MATMUL: case OP_MATMUL_ADD: ok = plan_gemm(nd, c, o); break;
        case OP_ATTENTION: ok = plan_attention(nd, c, o); break;
        default: ok = false; break;   // copies, below
    }
    if (f32_op(nd->op)) {
        set_opnd(o, 5, nd->output, c);
        return ok;
    }
    // copies, in 4-byte words
    const int ew = nd->elem_size / 4;
    set_opnd(o, 0, nd->inputs[0], c);
    set_opnd(o, 5, nd->output, c);
    o->total = (int)(total * ew);
    if (nd->op == OP_RESHAPE || total == 0) {
        o->kind = TY_COPY;
        return true;
    }
    if (nd->op == OP_SLICE) {
        const long long inner = (long long)nd->extra[4] * ew;
        if (inner <= 0 || nd->extra[3] <= 0) return false;
        o->kind = TY_SLICE;
        o->n[0] = (int)inner, o->n[1] = nd->extra[3], o->n[2] = nd->extra[1], o->n[3] = nd->extra[2];
        lbr_fast_divisor((unsigned)inner, &o->n[4], &o->n[5]);
        lbr_fast_divisor((unsigned)nd->extra[3], &o->n[6], &o->n[7]);
        o->total = (int)((long long)nd->extra[0] * nd->extra[3] * inner);
        return true;
    }
    if (nd->op == OP_TRANSPOSE) {
        if (nd->n_dims == 2) {
            if (nd->extra[0] <= 0 || nd->extra[1] <= 0) return false;
            o->kind = TY_TRANS2D;
            o->n[0] = nd->extra[0], o->n[1] = nd->extra[1], o->n[2] = ew == 2 ? 1 : 0;
            lbr_fast_divisor((unsigned)nd->extra[0], &o->n[3], &o->n[4]);
            return true;
        }
        const long long A = nd->extra[1], mid = nd->extra[2], B = nd->extra[3], inner = (long long)nd->extra[4] * ew;
        if (A <= 0 || mid <= 0 || B <= 0 || inner <= 0) return false;
        o->kind = TY_SWAP;
        o->n[0] = (int)A, o->n[1] = (int)mid, o->n[2] = (int)B, o->n[3] = (int)inner;
        lbr_fast_divisor((unsigned)inner, &o->n[4], &o->n[5]);
        lbr_fast_divisor((unsigned)A, &o->n[6], &o->n[7]);
        lbr_fast_divisor((unsigned)mid, &o->n[8], &o->n[9]);
        lbr_fast_divisor((unsigned)B, &o->n[10], &o->n[11]);
        return true;
    }
    // CAT
    const int nin = nd->n_inputs, dim = nd->extra[0];
    if (nin < 1 || nin > 4 || dim < 0 || dim >= nd->n_dims) return false;
    long long inner = ew, total_dim = 0;
    for (int i = dim + 1; i < nd->n_dims; ++i) inner *= nd->out_shape[i];
    for (int k = 0; k < nin; ++k) total_dim += nd->extra[1 + k];
    if (total_dim <= 0 || inner <= 0) return false;
    o->kind = TY_CAT;
    o->n[0] = nin, o->n[1] = (int)(total_dim * inner);
    long long off = 0;
    for (int k = 0; k < nin; ++k) {
        int* e = o->n + 2 + 4 * k;
        e[0] = (int)(nd->extra[1 + k] * inner);
        lbr_fast_divisor((unsigned)std::max(1, e[0]), &e[1], &e[2]);
        e[3] = (int)off;
        off += e[0];
        set_opnd(o, k, nd->inputs[k], c);
    }
    return true;
}

constexpr long long TY_MAX_PREFETCH_LINES = 8192;   // 1 MiB of global operands touched at the start

struct TinyLayout {
    unsigned long long lo = 0, hi = 0;
    std::vector<long long> wb;   // (window offset, bytes) pairs
    std::vector<TyOp> ops;
    std::vector<long long> pf;   // prefetch ranges: (128-byte aligned address, lines before, lines)
    int rec_off = 0;             // LDS offset of the records and the prefetch ranges
};

// Whether the whole node array can run as one workgroup, and its LDS window,
// write-back list and decoded nodes if so.  Every node must be one the
// interpreter executes with shapes it handles; the span of all node outputs
// must fit the CU's LDS; an input must lie wholly inside or wholly outside
// that window, and inside only where an earlier node wrote it; and the
// graph's GEMM + attention work must be small.  What the window leaves of
// the LDS stages GEMM operands and attention scores.  Write-back: the
// live-out ranges when the caller declared them, else every node's output.
bool tiny_layout(const OpNode* nodes, int n, const void* const* live_ptr, const size_t* live_bytes, int n_live,
                 bool have_live, TinyLayout* L) {
    // opt-in (LBR_TINY=1): on the graphs measured so far the multi-kernel
    // plan is faster (the toy block: 54 µs one workgroup, 43.5 µs seven
    // fused kernels); one node is one launch either way
    const char* env = getenv("LBR_TINY");
    if (!(env && atoi(env) != 0) || n < 2 || n > 256) return false;
    std::vector<Range> outs;
    long long flops = 0;
    for (int i = 0; i < n; ++i) {
        const OpNode* nd = &nodes[i];
        const bool f32 = f32_op(nd->op);
        if (!f32 && !copy_op(nd->op)) return false;
        if (f32 && nd->elem_size != 4) return false;
        if (!f32 && nd->elem_size != 4 && nd->elem_size != 8) return false;
        if (nd->n_dims < 1 || nd->n_dims > MAX_DIMS || !nd->output) return false;
        const int reads = reads_of(nd);
        if (reads < 1 || reads > MAX_INPUTS || nd->n_inputs < reads) return false;
        for (int k = 0; k < reads; ++k)
            if (!nd->inputs[k]) return false;
        if (nd->op == OP_SLICE && (nd->extra[2] < 0 || nd->extra[3] < 0 || nd->extra[2] + nd->extra[3] > nd->extra[1]))
            return false;
        const long long total = node_total(nd);
        if (nd->op == OP_MATMUL || nd->op == OP_MATMUL_ADD) {
            if (nd->extra[0] < 0 || (nd->extra[2] == 0 && nd->n_dims < 2)) return false;
            flops += 2 * total * (long long)nd->extra[0];
        }
        if (nd->op == OP_ATTENTION) {
            const int S = nd->extra[0], hd = nd->extra[1];
            if (S <= 0 || S > TY_MAX_ATTN_S || hd <= 0 || hd > TY_MAX_HD || nd->n_dims < 2) return false;
            flops += 4 * (total / hd) * S * (long long)hd;
        }
        const unsigned long long p = (unsigned long long)nd->output;
        outs.push_back({p, p + (unsigned long long)(total * nd->elem_size)});
    }
    if (flops > TY_MAX_FLOP) return false;
    unsigned long long lo = ~0ULL, hi = 0;
    for (const Range& r : outs)
        if (r.hi > r.lo) {
            lo = std::min(lo, r.lo);
            hi = std::max(hi, r.hi);
        }
    if (hi <= lo) return false;
    lo &= ~15ULL;   // the LDS window starts 16-byte aligned, like the arena offsets it mirrors
    const unsigned long long win = (hi - lo + 15) & ~15ULL;
    if (win > (unsigned long long)TY_LDS) return false;
    // inputs: wholly outside the window, or wholly inside and written before
    std::vector<Range> written;
    for (int i = 0; i < n; ++i) {
        const OpNode* nd = &nodes[i];
        const int reads = reads_of(nd);
        for (int k = 0; k < reads; ++k) {
            unsigned long long a = 0, b = 0;
            lbr_input_extent(nd, k, &a, &b);
            if (b <= a) continue;
            if (b - a >= (1ULL << 31)) return false;   // the interpreter indexes in 32 bits (and bounded reads)
            if (b <= lo || a >= hi) continue;     // outside
            if (a < lo || b > hi) return false;   // straddles the window (or unbounded)
            bool covered = false;
            for (const Range& r : written)
                if (r.lo <= a && b <= r.hi) covered = true;
            if (!covered) return false;
        }
        written.push_back(outs[i]);
        written = merged(written);
    }
    // global operands to touch at the start: every read outside the window
    std::vector<Range> glob;
    for (int i = 0; i < n; ++i)
        for (int k = 0; k < reads_of(&nodes[i]); ++k) {
            unsigned long long a = 0, b = 0;
            lbr_input_extent(&nodes[i], k, &a, &b);
            if (b > a && (b <= lo || a >= hi)) glob.push_back({a & ~127ULL, (b + 127) & ~127ULL});
        }
    glob = merged(glob);
    L->pf.clear();
    long long lines = 0;
    for (const Range& r : glob) {
        const long long nl = std::min<long long>((long long)((r.hi - r.lo) / 128), TY_MAX_PREFETCH_LINES - lines);
        if (nl <= 0) break;
        L->pf.push_back((long long)r.lo);
        L->pf.push_back(lines);
        L->pf.push_back(nl);
        lines += nl;
    }
    // LDS: the window, the staging area, then the records and prefetch ranges
    const long long rec_bytes = ((long long)n * (long long)sizeof(TyOp) + (long long)L->pf.size() * 8 + 15) & ~15LL;
    if ((long long)win + rec_bytes > TY_LDS) return false;
    L->rec_off = (int)(TY_LDS - rec_bytes);
    // the nodes as the kernel runs them
    Ctx c;
    c.lo = lo;
    c.hi = hi;
    c.stage_off = (int)win;
    c.stage_bytes = L->rec_off - (int)win;
    L->ops.assign((size_t)n, TyOp());
    for (int i = 0; i < n; ++i)
        if (!build_op(&nodes[i], c, &L->ops[(size_t)i])) return false;
    const char* dump = getenv("LBR_TINY_DUMP");
    if (dump && atoi(dump) != 0) {   // the decoded records, one line each, for diagnostics
        fprintf(stderr, "tiny window %llu bytes, staging %d bytes at %d\n", hi - lo, c.stage_bytes, c.stage_off);
        for (int i = 0; i < n; ++i) {
            const TyOp& o = L->ops[(size_t)i];
            fprintf(stderr, "tiny op %d kind %d sub %d lds %d total %d n", i, o.kind, o.sub, o.lds, o.total);
            for (int k = 0; k < 24; ++k) fprintf(stderr, " %d", o.n[k]);
            fprintf(stderr, "\n");
        }
    }
    // write-back ranges, relative to the window
    std::vector<Range> wb;
    if (have_live) {
        for (int k = 0; k < n_live; ++k) {
            const unsigned long long a = (unsigned long long)live_ptr[k], b = a + live_bytes[k];
            const unsigned long long ca = std::max(a, lo), cb = std::min(b, hi);
            if (cb > ca) wb.push_back({ca, cb});
        }
    } else {
        wb = outs;
    }
    wb = merged(wb);
    L->lo = lo;
    L->hi = hi;
    L->wb.clear();
    for (const Range& r : wb) {
        // whole 4-byte words (outputs are 4- or 8-byte elements at planner offsets)
        if ((r.lo - lo) % 4 || (r.hi - r.lo) % 4) return false;
        L->wb.push_back((long long)(r.lo - lo));
        L->wb.push_back((long long)(r.hi - r.lo));
    }
    return true;
}

}  // namespace

bool lbr_tiny_eligible(const OpNode* nodes, int n, const void* const* live_ptr, const size_t* live_bytes,
                       int n_live, bool have_live) {
    TinyLayout L;
    return tiny_layout(nodes, n, live_ptr, live_bytes, n_live, have_live, &L);
}

// The launch record of a one-workgroup plan, when tiny_layout admits the
// graph.  The decoded nodes and the write-back list go to device memory at
// *dev_buf (the plan owns it).
int lbr_tiny_step(const OpNode* nodes, int n, const void* const* live_ptr, const size_t* live_bytes, int n_live,
                  bool have_live, Step* s, void** dev_buf, bool* taken) {
    *taken = false;
    *dev_buf = nullptr;
    TinyLayout L;
    if (!tiny_layout(nodes, n, live_ptr, live_bytes, n_live, have_live, &L)) return LBR_OK;
    const size_t op_bytes = sizeof(TyOp) * (size_t)n;
    const size_t rec_bytes = op_bytes + L.pf.size() * sizeof(long long);
    const size_t wb_off = (rec_bytes + 15) & ~(size_t)15;
    const size_t bytes = wb_off + L.wb.size() * sizeof(long long) + 16;
    void* buf = nullptr;
    if (hipMalloc(&buf, bytes) != hipSuccess) {
        lbr_set_error("tiny plan: hipMalloc of %zu bytes failed", bytes);
        return LBR_ERR_HIP;
    }
    hipError_t e = hipMemcpy(buf, L.ops.data(), op_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess && !L.pf.empty())
        e = hipMemcpy((char*)buf + op_bytes, L.pf.data(), L.pf.size() * sizeof(long long), hipMemcpyHostToDevice);
    if (e == hipSuccess && !L.wb.empty())
        e = hipMemcpy((char*)buf + wb_off, L.wb.data(), L.wb.size() * sizeof(long long), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(buf);
        lbr_set_error("tiny plan: upload failed: %s", hipGetErrorString(e));
        return LBR_ERR_HIP;
    }
    *s = Step();
    s->run = launch_tiny;
    s->name = "tiny_graph";
    s->node_index = 0;
    s->n_nodes = n;
    s->fuse_kind = LBR_FUSE_TINY;
    s->in[0] = buf;
    s->in[1] = (char*)buf + wb_off;
    s->i[0] = n;
    s->i[1] = (long long)L.wb.size() / 2;
    s->i[2] = (long long)L.lo;
    s->i[3] = (long long)L.pf.size() / 3;
    s->i[4] = L.rec_off;
    *dev_buf = buf;
    *taken = true;
    return LBR_OK;
}

extern "C" unsigned lbr_tiny_fast_div(unsigned x, unsigned d) {
    int m = 0, sh = 0;
    lbr_fast_divisor(d, &m, &sh);
    if (m == 0) return x;
    return (unsigned)(((unsigned long long)x * (unsigned)m) >> 32) >> sh;
}
