// elementwise.hip — memory-bound element-wise kernels for gfx950.
//
// Covers the unary ops (csrc/executor.c:58-77 → csrc/ops/elementwise.c),
// the binary ops with their extras modes (executor.c:96-168, modes packed by
// runtime/ops.py:203-235), general broadcasting (csrc/ops/shape.c:32-62),
// FUSED_BIAS_RELU (elementwise.c:82-90) and GATED_ACT (elementwise.c:96-136).
//
// Design: grid-stride loops, 16-byte vector loads/stores when every pointer is
// 16-byte aligned and the element count allows it (checked per node at decode
// time, since planner offsets are arbitrary byte offsets), scalar otherwise.
// Every kernel is safe when `out` aliases its first input (the planner's
// in-place sharing): each element is read before the same element is written.
#include "lbr_device.h"

#include <math.h>

namespace {

enum UnaryKind { U_RELU, U_EXP, U_TANH, U_POW, U_GELU, U_RSQRT, U_SILU, U_NEG, U_COS, U_SIN };

__device__ __forceinline__ float gelu_tanh(float x) { return lbr_gelu_tanh(x); }

__device__ __forceinline__ float silu(float x) { return lbr_silu(x); }

template <int K>
__device__ __forceinline__ float unary_apply(float x, float s) {
    if constexpr (K == U_RELU) return x > 0.0f ? x : 0.0f;
    if constexpr (K == U_EXP) return expf(x);
    if constexpr (K == U_TANH) return tanhf(x);
    if constexpr (K == U_POW) return powf(x, s);
    if constexpr (K == U_GELU) return gelu_tanh(x);
    if constexpr (K == U_RSQRT) return 1.0f / sqrtf(x);
    if constexpr (K == U_SILU) return silu(x);
    if constexpr (K == U_NEG) return -x;
    if constexpr (K == U_COS) return cosf(x);
    if constexpr (K == U_SIN) return sinf(x);
    return x;
}

template <int K>
__global__ void unary_vec4(const float4* __restrict__ x, float4* __restrict__ out, long long n4, float s) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4;
         i += (long long)gridDim.x * blockDim.x) {
        float4 v = x[i];
        v.x = unary_apply<K>(v.x, s);
        v.y = unary_apply<K>(v.y, s);
        v.z = unary_apply<K>(v.z, s);
        v.w = unary_apply<K>(v.w, s);
        out[i] = v;
    }
}

template <int K>
__global__ void unary_scalar(const float* __restrict__ x, float* __restrict__ out, long long n, float s) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        out[i] = unary_apply<K>(x[i], s);
}

// Binary ops: 0 add, 1 sub, 2 mul, 3 div (operator codes of shape.c:32-62).
template <int OPC>
__device__ __forceinline__ float binop(float a, float b) {
    if constexpr (OPC == 0) return a + b;
    if constexpr (OPC == 1) return a - b;
    if constexpr (OPC == 2) return a * b;
    return a / b;
}

// Same-shape: out[i] = a[i] op b[i]
template <int OPC>
__global__ void binary_same_vec4(const float4* __restrict__ a, const float4* __restrict__ b,
                                 float4* __restrict__ out, long long n4) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4;
         i += (long long)gridDim.x * blockDim.x) {
        float4 x = a[i], y = b[i];
        x.x = binop<OPC>(x.x, y.x);
        x.y = binop<OPC>(x.y, y.y);
        x.z = binop<OPC>(x.z, y.z);
        x.w = binop<OPC>(x.w, y.w);
        out[i] = x;
    }
}

template <int OPC>
__global__ void binary_same_scalar(const float* __restrict__ a, const float* __restrict__ b,
                                   float* __restrict__ out, long long n) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        out[i] = binop<OPC>(a[i], b[i]);
}

// Tensor-scalar: out[i] = a[i] op s
template <int OPC>
__global__ void binary_scalar_vec4(const float4* __restrict__ a, float4* __restrict__ out, long long n4, float s) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4;
         i += (long long)gridDim.x * blockDim.x) {
        float4 x = a[i];
        x.x = binop<OPC>(x.x, s);
        x.y = binop<OPC>(x.y, s);
        x.z = binop<OPC>(x.z, s);
        x.w = binop<OPC>(x.w, s);
        out[i] = x;
    }
}

template <int OPC>
__global__ void binary_scalar_scalar(const float* __restrict__ a, float* __restrict__ out, long long n, float s) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        out[i] = binop<OPC>(a[i], s);
}

// Row bias: out[r, c] = a[r, c] + bias[c]  (ADD mode 0, kernel_add with M rows)
// RELU variant = FUSED_BIAS_RELU.
template <bool RELU>
__global__ void bias_rows_vec4(const float4* __restrict__ a, const float4* __restrict__ bias,
                               float4* __restrict__ out, long long n4, int N4) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4;
         i += (long long)gridDim.x * blockDim.x) {
        float4 x = a[i];
        const float4 b = bias[i % N4];
        x.x += b.x; x.y += b.y; x.z += b.z; x.w += b.w;
        if (RELU) {
            x.x = x.x > 0.f ? x.x : 0.f;
            x.y = x.y > 0.f ? x.y : 0.f;
            x.z = x.z > 0.f ? x.z : 0.f;
            x.w = x.w > 0.f ? x.w : 0.f;
        }
        out[i] = x;
    }
}

template <bool RELU>
__global__ void bias_rows_scalar(const float* __restrict__ a, const float* __restrict__ bias,
                                 float* __restrict__ out, long long n, int N) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        float v = a[i] + bias[i % N];
        if (RELU) v = v > 0.f ? v : 0.f;
        out[i] = v;
    }
}

// General broadcast: per output element decompose the row-major index over
// `shape` (collapsed to at most 8 dims) and gather with per-operand strides
// (stride 0 on broadcast dims), matching kernel_broadcast_binop's odometer.
struct BcastParams {
    int ndim;
    int shape[8];
    long long as[8];
    long long bs[8];
};

template <int OPC>
__global__ void broadcast_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                 float* __restrict__ out, long long n, BcastParams p) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        long long rem = i, ao = 0, bo = 0;
        for (int d = p.ndim - 1; d >= 0; --d) {
            const long long c = rem % p.shape[d];
            rem /= p.shape[d];
            ao += c * p.as[d];
            bo += c * p.bs[d];
        }
        out[i] = binop<OPC>(a[ao], b[bo]);
    }
}

// Broadcast where b repeats with period `period` over the flat index and a is
// same-shape (e.g. RoPE: q[1,H,S,D] * cos[1,1,S,D]); vectorised.
template <int OPC>
__global__ void broadcast_period_vec4(const float4* __restrict__ a, const float4* __restrict__ b,
                                      float4* __restrict__ out, long long n4, long long period4) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4;
         i += (long long)gridDim.x * blockDim.x) {
        float4 x = a[i];
        const float4 y = b[i % period4];
        x.x = binop<OPC>(x.x, y.x);
        x.y = binop<OPC>(x.y, y.y);
        x.z = binop<OPC>(x.z, y.z);
        x.w = binop<OPC>(x.w, y.w);
        out[i] = x;
    }
}

// GATED_ACT: out = act(x [+ bias]) * up   (elementwise.c:96-136)
template <int ACT, bool HAS_BIAS>
__device__ __forceinline__ float gated(float x, float b, float u) {
    float v = HAS_BIAS ? x + b : x;
    float g = (ACT == 0) ? silu(v) : gelu_tanh(v);
    return g * u;
}

template <int ACT, bool HAS_BIAS>
__global__ void gated_vec4(const float4* __restrict__ x, const float4* __restrict__ up,
                           const float4* __restrict__ bias, float4* __restrict__ out, long long n4, int N4) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4;
         i += (long long)gridDim.x * blockDim.x) {
        const float4 xv = x[i];
        const float4 uv = up[i];
        float4 bv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (HAS_BIAS) bv = bias[i % N4];
        float4 r;
        r.x = gated<ACT, HAS_BIAS>(xv.x, bv.x, uv.x);
        r.y = gated<ACT, HAS_BIAS>(xv.y, bv.y, uv.y);
        r.z = gated<ACT, HAS_BIAS>(xv.z, bv.z, uv.z);
        r.w = gated<ACT, HAS_BIAS>(xv.w, bv.w, uv.w);
        out[i] = r;
    }
}

template <int ACT, bool HAS_BIAS>
__global__ void gated_scalar(const float* __restrict__ x, const float* __restrict__ up,
                             const float* __restrict__ bias, float* __restrict__ out, long long n, int N) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const float b = HAS_BIAS ? bias[i % N] : 0.f;
        out[i] = gated<ACT, HAS_BIAS>(x[i], b, up[i]);
    }
}

constexpr int EW_BLOCK = 256;
constexpr unsigned EW_GRID_CAP = 256 * 16;

// ---------------------------------------------------------------------------
// Host launchers.  Step::i[0] = element count; i[1] = vectorised flag; other
// slots documented per launcher.
// ---------------------------------------------------------------------------

template <int K>
void launch_unary(const Step& s, hipStream_t st) {
    const long long n = s.i[0];
    if (s.i[1]) {
        const long long n4 = n / 4;
        hipLaunchKernelGGL(unary_vec4<K>, dim3(lbr_grid(n4, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0, st,
                           (const float4*)s.in[0], (float4*)s.out, n4, s.f[0]);
    } else {
        hipLaunchKernelGGL(unary_scalar<K>, dim3(lbr_grid(n, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0, st,
                           (const float*)s.in[0], (float*)s.out, n, s.f[0]);
    }
}

template <int OPC>
void launch_same(const Step& s, hipStream_t st) {
    const long long n = s.i[0];
    if (s.i[1]) {
        hipLaunchKernelGGL(binary_same_vec4<OPC>, dim3(lbr_grid(n / 4, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0,
                           st, (const float4*)s.in[0], (const float4*)s.in[1], (float4*)s.out, n / 4);
    } else {
        hipLaunchKernelGGL(binary_same_scalar<OPC>, dim3(lbr_grid(n, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0,
                           st, (const float*)s.in[0], (const float*)s.in[1], (float*)s.out, n);
    }
}

template <int OPC>
void launch_scalar(const Step& s, hipStream_t st) {
    const long long n = s.i[0];
    if (s.i[1]) {
        hipLaunchKernelGGL(binary_scalar_vec4<OPC>, dim3(lbr_grid(n / 4, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0,
                           st, (const float4*)s.in[0], (float4*)s.out, n / 4, s.f[0]);
    } else {
        hipLaunchKernelGGL(binary_scalar_scalar<OPC>, dim3(lbr_grid(n, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0,
                           st, (const float*)s.in[0], (float*)s.out, n, s.f[0]);
    }
}

// i[2] = N (row length of the bias)
template <bool RELU>
void launch_bias_rows(const Step& s, hipStream_t st) {
    const long long n = s.i[0];
    const int N = (int)s.i[2];
    if (s.i[1]) {
        hipLaunchKernelGGL(bias_rows_vec4<RELU>, dim3(lbr_grid(n / 4, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0,
                           st, (const float4*)s.in[0], (const float4*)s.in[1], (float4*)s.out, n / 4, N / 4);
    } else {
        hipLaunchKernelGGL(bias_rows_scalar<RELU>, dim3(lbr_grid(n, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0,
                           st, (const float*)s.in[0], (const float*)s.in[1], (float*)s.out, n, N);
    }
}

// i[2] = ndim, i[3..10] shape, i[11..18] a strides, i[19..26] b strides,
// i[27] = period (0 = general path)
template <int OPC>
void launch_broadcast(const Step& s, hipStream_t st) {
    const long long n = s.i[0];
    if (s.i[27] > 0) {
        hipLaunchKernelGGL(broadcast_period_vec4<OPC>, dim3(lbr_grid(n / 4, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK),
                           0, st, (const float4*)s.in[0], (const float4*)s.in[1], (float4*)s.out, n / 4,
                           s.i[27] / 4);
        return;
    }
    BcastParams p;
    p.ndim = (int)s.i[2];
    for (int d = 0; d < 8; ++d) {
        p.shape[d] = (int)s.i[3 + d];
        p.as[d] = s.i[11 + d];
        p.bs[d] = s.i[19 + d];
    }
    hipLaunchKernelGGL(broadcast_kernel<OPC>, dim3(lbr_grid(n, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK), 0, st,
                       (const float*)s.in[0], (const float*)s.in[1], (float*)s.out, n, p);
}

// in[0] = x, in[1] = up, in[2] = bias (or null); i[2] = N
template <int ACT, bool HAS_BIAS>
void launch_gated(const Step& s, hipStream_t st) {
    const long long n = s.i[0];
    const int N = (int)s.i[2];
    if (s.i[1]) {
        hipLaunchKernelGGL((gated_vec4<ACT, HAS_BIAS>), dim3(lbr_grid(n / 4, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK),
                           0, st, (const float4*)s.in[0], (const float4*)s.in[1], (const float4*)s.in[2],
                           (float4*)s.out, n / 4, N / 4);
    } else {
        hipLaunchKernelGGL((gated_scalar<ACT, HAS_BIAS>), dim3(lbr_grid(n, EW_BLOCK, EW_GRID_CAP)), dim3(EW_BLOCK),
                           0, st, (const float*)s.in[0], (const float*)s.in[1], (const float*)s.in[2],
                           (float*)s.out, n, N);
    }
}

bool vec_ok(long long n, const void* a, const void* b, const void* c) {
    return (n % 4 == 0) && lbr_aligned(a, 16) && (!b || lbr_aligned(b, 16)) && (!c || lbr_aligned(c, 16));
}

int check_ptrs(const OpNode* n, int need_inputs) {
    if (n->n_inputs < need_inputs) {
        lbr_set_error("op %d: expected %d inputs, got %d", n->op, need_inputs, n->n_inputs);
        return LBR_ERR_INVALID;
    }
    for (int i = 0; i < need_inputs; ++i)
        if (!n->inputs[i]) {
            lbr_set_error("op %d: input %d is null", n->op, i);
            return LBR_ERR_INVALID;
        }
    if (!n->output) {
        lbr_set_error("op %d: output is null", n->op);
        return LBR_ERR_INVALID;
    }
    if (n->n_dims < 0 || n->n_dims > MAX_DIMS) {
        lbr_set_error("op %d: n_dims %d out of range", n->op, n->n_dims);
        return LBR_ERR_INVALID;
    }
    return LBR_OK;
}

template <int OPC>
step_fn same_fn() { return launch_same<OPC>; }

step_fn same_for(int opc) {
    switch (opc) {
        case 0: return launch_same<0>;
        case 1: return launch_same<1>;
        case 2: return launch_same<2>;
        default: return launch_same<3>;
    }
}
step_fn scalar_for(int opc) {
    switch (opc) {
        case 0: return launch_scalar<0>;
        case 1: return launch_scalar<1>;
        case 2: return launch_scalar<2>;
        default: return launch_scalar<3>;
    }
}
step_fn bcast_for(int opc) {
    switch (opc) {
        case 0: return launch_broadcast<0>;
        case 1: return launch_broadcast<1>;
        case 2: return launch_broadcast<2>;
        default: return launch_broadcast<3>;
    }
}

// Fill a broadcast step from extras [ndim, a_strides, b_strides, out_shape]
// starting at extra[base] (ops.py:174-200).  Adjacent dims are merged where
// both operands stay linear across them, and the "b repeats with a period,
// a is dense" layout gets a vectorised kernel.
int fill_broadcast(const OpNode* n, int base, Step* s) {
    const int nd = n->extra[base];
    if (nd < 1 || nd > (MAX_DIMS - base - 1) / 3) {
        lbr_set_error("broadcast: ndim %d does not fit the extras", nd);
        return LBR_ERR_INVALID;
    }
    long long shape[MAX_DIMS], as[MAX_DIMS], bs[MAX_DIMS];
    long long total = 1;
    for (int d = 0; d < nd; ++d) {
        as[d] = n->extra[base + 1 + d];
        bs[d] = n->extra[base + 1 + nd + d];
        shape[d] = n->extra[base + 1 + 2 * nd + d];
        if (shape[d] < 0 || as[d] < 0 || bs[d] < 0) {
            lbr_set_error("broadcast: negative dim or stride");
            return LBR_ERR_INVALID;
        }
        if (shape[d] > 0 && total > LBR_MAX_ELEMENTS / shape[d]) {
            lbr_set_error("broadcast: more than 2^40 elements");
            return LBR_ERR_INVALID;
        }
        total *= shape[d];
    }
    if (total != node_total(n)) {
        lbr_set_error("broadcast: %lld elements, the output has %lld", total, node_total(n));
        return LBR_ERR_INVALID;
    }
    // drop size-1 dims, then merge neighbours that stay linear for both operands
    long long cs[MAX_DIMS], ca[MAX_DIMS], cb[MAX_DIMS];
    int cn = 0;
    for (int d = 0; d < nd; ++d) {
        if (shape[d] == 1) continue;
        if (cn > 0 && ca[cn - 1] == as[d] * shape[d] && cb[cn - 1] == bs[d] * shape[d]) {
            cs[cn - 1] *= shape[d];
            ca[cn - 1] = as[d];
            cb[cn - 1] = bs[d];
            continue;
        }
        cs[cn] = shape[d];
        ca[cn] = as[d];
        cb[cn] = bs[d];
        ++cn;
    }
    if (cn == 0) {
        cs[0] = 1;
        ca[0] = 0;
        cb[0] = 0;
        cn = 1;
    }
    if (cn > 8) {
        lbr_set_error("broadcast: %d non-mergeable dims (max 8)", cn);
        return LBR_ERR_UNSUPPORTED;
    }
    s->i[0] = total;
    s->i[2] = cn;
    for (int d = 0; d < 8; ++d) {
        s->i[3 + d] = d < cn ? cs[d] : 1;
        s->i[11 + d] = d < cn ? ca[d] : 0;
        s->i[19 + d] = d < cn ? cb[d] : 0;
    }
    // period detection: a dense row-major, b dense over the trailing dims and
    // zero-stride over the leading ones
    s->i[27] = 0;
    {
        bool a_dense = true;
        long long st = 1;
        for (int d = cn - 1; d >= 0; --d) {
            if (ca[d] != st) a_dense = false;
            st *= cs[d];
        }
        int split = cn;  // dims [split, cn) are dense in b, [0, split) are zero-stride
        long long bst = 1;
        for (int d = cn - 1; d >= 0; --d) {
            if (cb[d] == bst) {
                bst *= cs[d];
                split = d;
            } else {
                break;
            }
        }
        bool lead_zero = true;
        for (int d = 0; d < split; ++d)
            if (cb[d] != 0) lead_zero = false;
        if (a_dense && lead_zero && split > 0 && bst % 4 == 0 && total % 4 == 0 && lbr_aligned(n->inputs[0], 16) &&
            lbr_aligned(n->inputs[1], 16) && lbr_aligned(n->output, 16))
            s->i[27] = bst;
    }
    return LBR_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Decoders
// ---------------------------------------------------------------------------

int decode_unary(const OpNode* n, Step* s) {
    int rc = check_ptrs(n, 1);
    if (rc) return rc;
    const long long total = node_total(n);
    s->in[0] = n->inputs[0];
    s->out = n->output;
    s->i[0] = total;
    s->i[1] = vec_ok(total, n->inputs[0], n->output, nullptr);
    s->f[0] = 0.f;
    switch (n->op) {
        case OP_RELU: s->run = launch_unary<U_RELU>; s->name = "relu"; break;
        case OP_EXP: s->run = launch_unary<U_EXP>; s->name = "exp"; break;
        case OP_TANH: s->run = launch_unary<U_TANH>; s->name = "tanh"; break;
        case OP_POW:
            s->run = launch_unary<U_POW>;
            s->name = "pow";
            s->f[0] = node_extra_float(n, 0);
            break;
        case OP_GELU: s->run = launch_unary<U_GELU>; s->name = "gelu_tanh"; break;
        case OP_RSQRT: s->run = launch_unary<U_RSQRT>; s->name = "rsqrt"; break;
        case OP_SILU: s->run = launch_unary<U_SILU>; s->name = "silu"; break;
        case OP_NEG: s->run = launch_unary<U_NEG>; s->name = "neg"; break;
        case OP_COS: s->run = launch_unary<U_COS>; s->name = "cos"; break;
        case OP_SIN: s->run = launch_unary<U_SIN>; s->name = "sin"; break;
        default: lbr_set_error("decode_unary: op %d", n->op); return LBR_ERR_UNSUPPORTED;
    }
    return LBR_OK;
}

// ADD extras[0]: 0 bias, 1 same, 2 scalar, 3 broadcast (executor.c:96-117)
// SUB/MUL/DIV extras[0]: 0 same, 1 scalar, 2 broadcast (executor.c:119-168)
int decode_binary(const OpNode* n, Step* s) {
    const int opc = n->op == OP_ADD ? 0 : n->op == OP_SUB ? 1 : n->op == OP_MUL ? 2 : 3;
    const int mode = n->extra[0];
    enum { M_BIAS, M_SAME, M_SCALAR, M_BCAST } kind;
    if (n->op == OP_ADD) {
        kind = mode == 2 ? M_SCALAR : mode == 1 ? M_SAME : mode == 3 ? M_BCAST : M_BIAS;
    } else {
        kind = mode == 1 ? M_SCALAR : mode == 2 ? M_BCAST : M_SAME;
    }
    int rc = check_ptrs(n, kind == M_SCALAR ? 1 : 2);
    if (rc) return rc;
    const long long total = node_total(n);
    s->in[0] = n->inputs[0];
    s->in[1] = kind == M_SCALAR ? nullptr : n->inputs[1];
    s->out = n->output;
    s->i[0] = total;
    static const char* names[4][4] = {{"add_bias", "add", "add_scalar", "add_broadcast"},
                                      {"sub_bias", "sub", "sub_scalar", "sub_broadcast"},
                                      {"mul_bias", "mul", "mul_scalar", "mul_broadcast"},
                                      {"div_bias", "div", "div_scalar", "div_broadcast"}};
    s->name = names[opc][kind];
    switch (kind) {
        case M_SCALAR:
            s->i[1] = vec_ok(total, n->inputs[0], n->output, nullptr);
            s->f[0] = node_extra_float(n, 1);
            s->run = scalar_for(opc);
            return LBR_OK;
        case M_SAME:
            s->i[1] = vec_ok(total, n->inputs[0], n->inputs[1], n->output);
            s->run = same_for(opc);
            return LBR_OK;
        case M_BIAS: {
            const int N = node_last_dim(n);
            if (N <= 0) {
                lbr_set_error("add_bias: zero-width rows");
                return total == 0 ? LBR_OK : LBR_ERR_INVALID;
            }
            s->i[2] = N;
            s->i[1] = vec_ok(total, n->inputs[0], n->inputs[1], n->output) && (N % 4 == 0);
            s->run = launch_bias_rows<false>;
            return LBR_OK;
        }
        case M_BCAST:
            rc = fill_broadcast(n, 1, s);
            if (rc) return rc;
            s->run = bcast_for(opc);
            return LBR_OK;
    }
    return LBR_ERR_INVALID;
}

int decode_bias_relu(const OpNode* n, Step* s) {
    int rc = check_ptrs(n, 2);
    if (rc) return rc;
    const long long total = node_total(n);
    const int N = node_last_dim(n);
    s->in[0] = n->inputs[0];
    s->in[1] = n->inputs[1];
    s->out = n->output;
    s->i[0] = total;
    s->i[2] = N > 0 ? N : 1;
    s->i[1] = vec_ok(total, n->inputs[0], n->inputs[1], n->output) && (N % 4 == 0);
    s->run = launch_bias_rows<true>;
    s->name = "bias_relu";
    return LBR_OK;
}

// extras [has_bias, act]; inputs [x, up] or [x, bias, up] (executor.c:354-369)
int decode_gated_act(const OpNode* n, Step* s) {
    const int has_bias = n->extra[0];
    const int act = n->extra[1];
    int rc = check_ptrs(n, has_bias ? 3 : 2);
    if (rc) return rc;
    const long long total = node_total(n);
    const int N = node_last_dim(n);
    s->in[0] = n->inputs[0];
    s->in[1] = has_bias ? n->inputs[2] : n->inputs[1];
    s->in[2] = has_bias ? n->inputs[1] : nullptr;
    s->out = n->output;
    s->i[0] = total;
    s->i[2] = N > 0 ? N : 1;
    s->i[1] = vec_ok(total, s->in[0], s->in[1], n->output) && (!has_bias || (lbr_aligned(s->in[2], 16) && N % 4 == 0));
    if (act == 0) {
        s->run = has_bias ? launch_gated<0, true> : launch_gated<0, false>;
        s->name = "gated_silu";
    } else {
        s->run = has_bias ? launch_gated<1, true> : launch_gated<1, false>;
        s->name = "gated_gelu";
    }
    return LBR_OK;
}
