// norm.hip — row-wise kernels for gfx950: LayerNorm, RMSNorm, softmax and
// the MAX/SUM reductions.
//
// LayerNorm follows csrc/ops/norm.c:47-64 (two-pass, variance from centered
// values, inv_std = 1/sqrtf(var/cols + eps), out = d·inv_std·γ + β); RMSNorm
// follows norm.c:100-107 (scale = 1/sqrtf(Σx²/cols + eps), out = x·scale·w);
// softmax follows csrc/ops/reduce.c:78-97 (max-shift, expf, divide by sum);
// MAX/SUM reduce the middle axis of [outer, axis, inner] (reduce.c:8-36).
//
// Mapping: rows of <= 1024 columns get one 64-lane wavefront each (4 rows per
// 256-thread block) with the row held in registers; wider rows get a whole
// block, holding up to 16 values per thread in registers, else re-reading the
// row (L2-resident) in a strided loop.  HBM traffic is one read and one write
// of the row either way.
#include "lbr_device.h"

#include <float.h>
#include <math.h>

namespace {

constexpr int NB = 256;  // block size for row kernels

// ----------------------------- LayerNorm / RMSNorm -------------------------

// One wave per row, cols <= 64 * 4 * VPL, float4 path (cols % 4 == 0).
// With a pre-add (lbr_merge_add_norm): the normalised row is x + p, p = row
// (row mod period) of addb, and that sum is also written to hout (the ADD's
// output) — the same single addition the ADD kernel makes.
__device__ __forceinline__ void norm_pre_add(float4& v, const float* __restrict__ addb, long long row, int period,
                                             int cols, int idx, float* __restrict__ hout) {
    const float4 p = reinterpret_cast<const float4*>(addb + (row % period) * cols)[idx];
    v.x = v.x + p.x;
    v.y = v.y + p.y;
    v.z = v.z + p.z;
    v.w = v.w + p.w;
    reinterpret_cast<float4*>(hout + row * cols)[idx] = v;
}

template <bool RMS, int VPL>
__global__ __launch_bounds__(NB) void norm_wave_rows(const float* __restrict__ x, const float* __restrict__ g,
                                                     const float* __restrict__ b, float* __restrict__ out,
                                                     long long rows, int cols, float eps, const float* __restrict__ addb,
                                                     int period, float* __restrict__ hout) {
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * (NB / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    const int c4 = cols / 4;
    const float4* xr = reinterpret_cast<const float4*>(x + row * cols);
    const float4* g4 = reinterpret_cast<const float4*>(g);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    // row, weight and (LayerNorm) bias loads all issue before the reduction
    float4 v[VPL], wv[VPL], bv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = lane + k * 64;
        const bool in = idx < c4;
        v[k] = in ? xr[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[k] = in ? g4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
        bv[k] = in && !RMS ? b4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (addb) {
#pragma unroll
        for (int k = 0; k < VPL; ++k)
            if (lane + k * 64 < c4) norm_pre_add(v[k], addb, row, period, cols, lane + k * 64, hout);
    }
    lbr_norm_row_wave<RMS, VPL>(v, wv, bv, reinterpret_cast<float4*>(out + row * cols), c4, cols, eps);
}

// One block per row, float4 path, cols <= NB * 4 * VPL.
template <bool RMS, int VPL>
__global__ __launch_bounds__(NB) void norm_block_rows(const float* __restrict__ x, const float* __restrict__ g,
                                                      const float* __restrict__ b, float* __restrict__ out,
                                                      long long rows, int cols, float eps,
                                                      const float* __restrict__ addb, int period,
                                                      float* __restrict__ hout) {
    __shared__ float red[NB / 64];
    const long long row = blockIdx.x;
    const int c4 = cols / 4;
    const float4* xr = reinterpret_cast<const float4*>(x + row * cols);
    const float4* g4 = reinterpret_cast<const float4*>(g);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    // the row, the weight and (LayerNorm) the bias are all loaded before the
    // first reduction, so their latencies overlap
    float4 v[VPL], wv[VPL], bv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = threadIdx.x + k * NB;
        const bool in = idx < c4;
        v[k] = in ? xr[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[k] = in ? g4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
        bv[k] = in && !RMS ? b4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (addb) {
#pragma unroll
        for (int k = 0; k < VPL; ++k)
            if ((int)threadIdx.x + k * NB < c4) norm_pre_add(v[k], addb, row, period, cols, threadIdx.x + k * NB, hout);
    }
    lbr_norm_row_block<RMS, VPL>(v, wv, bv, reinterpret_cast<float4*>(out + row * cols), c4, cols, eps, red);
}

// Generic: one block per row, scalar loads, any cols / alignment.  The row is
// re-read (from L2) for each pass.  Safe in place: the last pass reads x[j]
// before writing out[j] for the same j, and earlier passes only read.
template <bool RMS>
__global__ __launch_bounds__(NB) void norm_generic(const float* __restrict__ x, const float* __restrict__ g,
                                                   const float* __restrict__ b, float* out, long long rows,
                                                   int cols, float eps) {
    __shared__ float red[NB / 64];
    const long long row = blockIdx.x;
    const float* xr = x + row * cols;
    float* orow = out + row * cols;
    float s = 0.f;
    for (int j = threadIdx.x; j < cols; j += NB) s += RMS ? xr[j] * xr[j] : xr[j];
    s = block_sum(s, red);
    if (RMS) {
        const float scale = 1.0f / sqrtf(s / cols + eps);
        for (int j = threadIdx.x; j < cols; j += NB) orow[j] = xr[j] * scale * g[j];
        return;
    }
    const float mean = s / cols;
    float var = 0.f;
    for (int j = threadIdx.x; j < cols; j += NB) {
        const float d = xr[j] - mean;
        var += d * d;
    }
    var = block_sum(var, red);
    const float inv_std = 1.0f / sqrtf(var / cols + eps);
    for (int j = threadIdx.x; j < cols; j += NB) orow[j] = (xr[j] - mean) * inv_std * g[j] + b[j];
}

// i[0] rows, i[1] cols, i[2] variant (0 generic, 1 wave, 2 block); i[3] = VPL
template <bool RMS>
void launch_norm(const Step& s, hipStream_t st) {
    const long long rows = s.i[0];
    const int cols = (int)s.i[1];
    const float eps = s.f[0];
    const float* x = (const float*)s.in[0];
    const float* g = (const float*)s.in[1];
    const float* b = RMS ? nullptr : (const float*)s.in[2];
    float* out = (float*)s.out;
    // pre-add (lbr_merge_add_norm): in[3] the broadcast operand, i[4] its period
    // in rows, in[4] the sum's output
    const float* addb = (const float*)s.in[3];
    const int period = s.in[3] ? (int)s.i[4] : 1;
    float* hout = (float*)s.in[4];
    if (rows <= 0) return;
    switch (s.i[2]) {
        case 1: {
            const unsigned grid = (unsigned)((rows + (NB / 64) - 1) / (NB / 64));
            switch (s.i[3]) {
                case 1: hipLaunchKernelGGL((norm_wave_rows<RMS, 1>), dim3(grid), dim3(NB), 0, st, x, g, b, out, rows, cols, eps, addb, period, hout); break;
                case 2: hipLaunchKernelGGL((norm_wave_rows<RMS, 2>), dim3(grid), dim3(NB), 0, st, x, g, b, out, rows, cols, eps, addb, period, hout); break;
                default: hipLaunchKernelGGL((norm_wave_rows<RMS, 4>), dim3(grid), dim3(NB), 0, st, x, g, b, out, rows, cols, eps, addb, period, hout); break;
            }
            break;
        }
        case 2:
            switch (s.i[3]) {
                case 2: hipLaunchKernelGGL((norm_block_rows<RMS, 2>), dim3((unsigned)rows), dim3(NB), 0, st, x, g, b, out, rows, cols, eps, addb, period, hout); break;
                case 4: hipLaunchKernelGGL((norm_block_rows<RMS, 4>), dim3((unsigned)rows), dim3(NB), 0, st, x, g, b, out, rows, cols, eps, addb, period, hout); break;
                case 8: hipLaunchKernelGGL((norm_block_rows<RMS, 8>), dim3((unsigned)rows), dim3(NB), 0, st, x, g, b, out, rows, cols, eps, addb, period, hout); break;
                default: hipLaunchKernelGGL((norm_block_rows<RMS, 16>), dim3((unsigned)rows), dim3(NB), 0, st, x, g, b, out, rows, cols, eps, addb, period, hout); break;
            }
            break;
        default:
            hipLaunchKernelGGL((norm_generic<RMS>), dim3((unsigned)rows), dim3(NB), 0, st, x, g, b, out, rows, cols, eps);
            break;
    }
}

int choose_norm_variant(long long cols, const void* x, const void* g, const void* b, const void* out, Step* s) {
    const bool vec = cols % 4 == 0 && lbr_aligned(x, 16) && lbr_aligned(g, 16) && (!b || lbr_aligned(b, 16)) &&
                     lbr_aligned(out, 16);
    s->i[2] = 0;
    s->i[3] = 0;
    if (!vec) return LBR_OK;
    if (cols <= 256) { s->i[2] = 1; s->i[3] = 1; }
    else if (cols <= 512) { s->i[2] = 1; s->i[3] = 2; }
    else if (cols <= 1024) { s->i[2] = 1; s->i[3] = 4; }
    else if (cols <= 2048) { s->i[2] = 2; s->i[3] = 2; }
    else if (cols <= 4096) { s->i[2] = 2; s->i[3] = 4; }
    else if (cols <= 8192) { s->i[2] = 2; s->i[3] = 8; }
    else if (cols <= 16384) { s->i[2] = 2; s->i[3] = 16; }
    return LBR_OK;
}

// ----------------------------- Softmax -------------------------------------

// One block per row: max, exp + sum (written to out), divide.  In-place safe.
__global__ __launch_bounds__(NB) void softmax_rows(const float* x, float* out, int cols) {
    __shared__ float red[NB / 64];
    const long long row = blockIdx.x;
    const float* xr = x + row * cols;
    float* orow = out + row * cols;
    float m = -FLT_MAX;
    for (int j = threadIdx.x; j < cols; j += NB) m = fmaxf(m, xr[j]);
    m = block_max(m, red);
    float s = 0.f;
    for (int j = threadIdx.x; j < cols; j += NB) {
        const float e = expf(xr[j] - m);
        orow[j] = e;
        s += e;
    }
    s = block_sum(s, red);
    for (int j = threadIdx.x; j < cols; j += NB) orow[j] = orow[j] / s;
}

void launch_softmax(const Step& s, hipStream_t st) {
    if (s.i[0] <= 0 || s.i[1] <= 0) return;
    hipLaunchKernelGGL(softmax_rows, dim3((unsigned)s.i[0]), dim3(NB), 0, st, (const float*)s.in[0], (float*)s.out,
                       (int)s.i[1]);
}

// ----------------------------- MAX / SUM -----------------------------------

// inner > 1: one thread per (outer, j), loop over the axis (coalesced over j).
template <bool IS_MAX>
__global__ void reduce_mid(const float* __restrict__ x, float* __restrict__ out, int outer, int axis, int inner) {
    const long long n = (long long)outer * inner;
    for (long long t = blockIdx.x * (long long)blockDim.x + threadIdx.x; t < n;
         t += (long long)gridDim.x * blockDim.x) {
        const long long o = t / inner, j = t % inner;
        float acc = IS_MAX ? -FLT_MAX : 0.f;
        for (int a = 0; a < axis; ++a) {
            const float v = x[(o * axis + a) * inner + j];
            acc = IS_MAX ? (v > acc ? v : acc) : acc + v;
        }
        out[t] = acc;
    }
}

// inner == 1: one wave per row.
template <bool IS_MAX>
__global__ __launch_bounds__(NB) void reduce_last(const float* __restrict__ x, float* __restrict__ out, int outer,
                                                  int axis) {
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * (NB / 64) + threadIdx.x / 64;
    if (row >= outer) return;
    float acc = IS_MAX ? -FLT_MAX : 0.f;
    for (int a = lane; a < axis; a += 64) {
        const float v = x[row * axis + a];
        acc = IS_MAX ? (v > acc ? v : acc) : acc + v;
    }
    acc = IS_MAX ? wave_max(acc) : wave_sum(acc);
    if (lane == 0) out[row] = acc;
}

template <bool IS_MAX>
void launch_reduce(const Step& s, hipStream_t st) {
    const int outer = (int)s.i[0], axis = (int)s.i[1], inner = (int)s.i[2];
    if ((long long)outer * inner <= 0) return;
    if (inner == 1) {
        hipLaunchKernelGGL(reduce_last<IS_MAX>, dim3((outer + 3) / 4), dim3(NB), 0, st, (const float*)s.in[0],
                           (float*)s.out, outer, axis);
    } else {
        hipLaunchKernelGGL(reduce_mid<IS_MAX>, dim3(lbr_grid((long long)outer * inner, NB, 8192)), dim3(NB), 0, st,
                           (const float*)s.in[0], (float*)s.out, outer, axis, inner);
    }
}

int need(const OpNode* n, int k) {
    if (n->n_inputs < k || !n->output) {
        lbr_set_error("op %d: expected %d inputs and an output", n->op, k);
        return LBR_ERR_INVALID;
    }
    for (int i = 0; i < k; ++i)
        if (!n->inputs[i]) {
            lbr_set_error("op %d: input %d is null", n->op, i);
            return LBR_ERR_INVALID;
        }
    return LBR_OK;
}

}  // namespace

// LAYERNORM: inputs [x, gamma, beta], extra[0] = eps bits (executor.c:296-301)
int decode_layernorm(const OpNode* n, Step* s) {
    int rc = need(n, 3);
    if (rc) return rc;
    const long long rows = node_leading(n);
    const int cols = node_last_dim(n);
    s->in[0] = n->inputs[0];
    s->in[1] = n->inputs[1];
    s->in[2] = n->inputs[2];
    s->out = n->output;
    s->i[0] = cols > 0 ? rows : 0;
    s->i[1] = cols;
    s->f[0] = node_extra_float(n, 0);
    s->run = launch_norm<false>;
    s->name = "layernorm";
    return choose_norm_variant(cols, n->inputs[0], n->inputs[1], n->inputs[2], n->output, s);
}

// RMSNORM: inputs [x, weight], extra[0] = eps bits (executor.c:303-308)
int decode_rmsnorm(const OpNode* n, Step* s) {
    int rc = need(n, 2);
    if (rc) return rc;
    const long long rows = node_leading(n);
    const int cols = node_last_dim(n);
    s->in[0] = n->inputs[0];
    s->in[1] = n->inputs[1];
    s->in[2] = nullptr;
    s->out = n->output;
    s->i[0] = cols > 0 ? rows : 0;
    s->i[1] = cols;
    s->f[0] = node_extra_float(n, 0);
    s->run = launch_norm<true>;
    s->name = "rmsnorm";
    return choose_norm_variant(cols, n->inputs[0], n->inputs[1], nullptr, n->output, s);
}

// SOFTMAX over the last dim (executor.c:188-193)
int decode_softmax(const OpNode* n, Step* s) {
    int rc = need(n, 1);
    if (rc) return rc;
    s->in[0] = n->inputs[0];
    s->out = n->output;
    s->i[0] = node_leading(n);
    s->i[1] = node_last_dim(n);
    s->run = launch_softmax;
    s->name = "softmax";
    return LBR_OK;
}

// MAX / SUM: extras [axis, axis_size]; outer = Π out_shape[0:axis],
// inner = Π out_shape[axis:] (executor.c:172-186).
int decode_reduce(const OpNode* n, Step* s) {
    int rc = need(n, 1);
    if (rc) return rc;
    const int axis = n->extra[0];
    const int axis_size = n->extra[1];
    long long outer = 1, inner = 1;
    for (int i = 0; i < axis && i < n->n_dims; ++i) outer *= n->out_shape[i];
    for (int i = axis < 0 ? 0 : axis; i < n->n_dims; ++i) inner *= n->out_shape[i];
    if (axis_size < 0 || outer > INT32_MAX || inner > INT32_MAX) {
        lbr_set_error("reduce: unsupported sizes");
        return LBR_ERR_INVALID;
    }
    s->in[0] = n->inputs[0];
    s->out = n->output;
    s->i[0] = outer;
    s->i[1] = axis_size;
    s->i[2] = inner;
    if (n->op == OP_MAX) {
        s->run = launch_reduce<true>;
        s->name = "reduce_max";
    } else {
        s->run = launch_reduce<false>;
        s->name = "reduce_sum";
    }
    return LBR_OK;
}
