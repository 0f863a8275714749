// lbr_device.h — device-side helpers shared by the gfx950 kernels, and the
// decoded-launch record (`Step`) the executor builds from each OpNode.
//
// Wavefronts are 64 lanes wide on CDNA4; every reduction here is written for
// that width (no 32-lane warp assumptions).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/lbr_executor.h"

#define LBR_WAVE 64

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Activations, shared by the element-wise kernels and the GEMM epilogues so
// a fused epilogue rounds exactly like the separate node would.
// ---------------------------------------------------------------------------

// 0.5·x·(1 + tanh(z)), z = √(2/π)·(x + 0.044715·x³)  (elementwise.c:185-190),
// evaluated in its sigmoid form: 0.5·(1 + tanh(z)) = 1/(1 + e^(−2z)), so
// GELU(x) = x / (1 + e^(−2z)) — the hardware exp2 and reciprocal (about 1
// ulp each) instead of a tanh; e^(−2z) overflowing to inf gives ∓0,
// underflowing to 0 gives x.
__device__ __forceinline__ float lbr_gelu_tanh(float x) {
    const float z = 0.7978845608f * (x + 0.044715f * x * x * x);
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * z));
}

// x·σ(x) = x / (1 + e^(−x)), same evaluation
__device__ __forceinline__ float lbr_silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Row-norm arithmetic shared by norm_wave_rows and the fused MLP's prologue,
// with contraction off (the compiler may otherwise form a different fused
// multiply-add in each kernel: fma(y, y, x·x) in one, fma(x, x, y·y) in the
// other), so both kernels normalise a row to the same bits: the float4
// partial sum of x or x², and (x − μ)·r·γ + β / x·s·w.
__device__ __forceinline__ float lbr_sum4(float4 v) {
#pragma clang fp contract(off)
    return (v.x + v.y) + (v.z + v.w);
}
__device__ __forceinline__ float lbr_sumsq4(float4 v) {
#pragma clang fp contract(off)
    return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
}
__device__ __forceinline__ float4 lbr_norm_affine(float4 d, float r, float4 w, float4 b) {
#pragma clang fp contract(off)
    return make_float4(d.x * r * w.x + b.x, d.y * r * w.y + b.y, d.z * r * w.z + b.z, d.w * r * w.w + b.w);
}
__device__ __forceinline__ float4 lbr_norm_scale(float4 x, float s, float4 w) {
#pragma clang fp contract(off)
    return make_float4(x.x * s * w.x, x.y * s * w.y, x.z * s * w.z, x.w * s * w.w);
}

// GEMM epilogue activation codes (fused MATMUL → RELU / GELU / SILU)
#define LBR_ACT_NONE 0
#define LBR_ACT_RELU 1
#define LBR_ACT_GELU 2
#define LBR_ACT_SILU 3

__device__ __forceinline__ float lbr_act(int act, float v) {
    switch (act) {
        case LBR_ACT_RELU: return v > 0.0f ? v : 0.0f;
        case LBR_ACT_GELU: return lbr_gelu_tanh(v);
        case LBR_ACT_SILU: return lbr_silu(v);
        default: return v;
    }
}

// ---------------------------------------------------------------------------
// Wave / block reductions (64-lane wavefronts)
// ---------------------------------------------------------------------------

// s_waitcnt immediate that waits until at most n vector-memory operations of
// the wave are outstanding (gfx9 encoding: vmcnt bits [3:0] and [15:14]; the
// other counters at their maximum, as in 0x3F70 = vmcnt(0)).
constexpr int lbr_waitcnt_vm(int n) { return 0x3F70 | (n & 15) | (((n >> 4) & 3) << 14); }

// Direct-to-LDS load of 16 bytes a lane: lane l's bytes at voff + soff of the
// buffer land at lds + 16·l (lds wave-uniform), so one instruction fills a
// contiguous 1 KB of LDS.  Counts in vmcnt like any vector load.
__device__ __forceinline__ void lbr_dma16(__amdgpu_buffer_rsrc_t r, float* lds, unsigned voff, unsigned soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
}

// DPP / row-swap lane exchanges (VALU; no LDS round trip).  lbr_dpp<CTRL>
// returns v of the lane that the DPP control selects: 0xB1 quad_perm
// [1,0,3,2] (lane ^ 1), 0x4E quad_perm [2,3,0,1] (lane ^ 2), 0x141
// row_half_mirror (7 − i within 8 lanes), 0x140 row_mirror (15 − i within
// 16), 0x128 row_ror:8 (lane ^ 8 within 16).
template <int CTRL>
__device__ __forceinline__ float lbr_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G lanes (G = 16, 32 or 64); every lane of a
// group gets the same value.  Pairs are combined as x + y = y + x, so the
// lanes agree bit for bit.  v_permlane16_swap(u, u) returns {u of the even
// 16-lane row, u of the odd row} of each row pair (v_permlane32_swap: of
// each 32-lane half).
template <int G>
__device__ __forceinline__ float lbr_group_sum(float s) {
    static_assert(G == 16 || G == 32 || G == 64, "group of 16, 32 or 64 lanes");
    s += lbr_dpp<0xB1>(s);
    s += lbr_dpp<0x4E>(s);
    s += lbr_dpp<0x141>(s);
    s += lbr_dpp<0x140>(s);
    if (G >= 32) {
        const unsigned u = __float_as_uint(s);
        auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    }
    if (G == 64) {
        const unsigned u = __float_as_uint(s);
        auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        s = __uint_as_float(b[0]) + __uint_as_float(b[1]);
    }
    return s;
}

// v of lane ^ (G/2) for G = 16, 32 or 64.
template <int G>
__device__ __forceinline__ float lbr_half_partner(float v, int lane) {
    static_assert(G == 16 || G == 32 || G == 64, "group of 16, 32 or 64 lanes");
    if constexpr (G == 16) {
        return lbr_dpp<0x128>(v);
    } else if constexpr (G == 32) {
        const unsigned u = __float_as_uint(v);
        auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __uint_as_float((lane & 16) ? a[0] : a[1]);
    } else {
        const unsigned u = __float_as_uint(v);
        auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __uint_as_float((lane & 32) ? b[0] : b[1]);
    }
}

template <int LPR, int HD>
__device__ __forceinline__ float4 lbr_head_row(float4 x, bool norm, float4 w, float eps, bool rope, float4 c4, float4 s4,
                                               int lane) {
#pragma clang fp contract(off)
    float v[4] = {x.x, x.y, x.z, x.w};
    if (norm) {
        const float ss = lbr_group_sum<LPR>((v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]));
        const float scale = 1.0f / sqrtf(ss / HD + eps);
        v[0] = v[0] * scale * w.x;
        v[1] = v[1] * scale * w.y;
        v[2] = v[2] * scale * w.z;
        v[3] = v[3] * scale * w.w;
    }
    if (!rope) return make_float4(v[0], v[1], v[2], v[3]);
    const float sign = (lane % LPR) < LPR / 2 ? -1.0f : 1.0f;
    const float c[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
    float o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float rot = sign * lbr_half_partner<LPR>(v[q], lane);
        o[q] = v[q] * c[q] + rot * sn[q];
    }
    return make_float4(o[0], o[1], o[2], o[3]);
}

// One head row of the float4 head prologue: LPR lanes hold the row's HD values,
// 4 consecutive a lane (x, already biased).  RMSNorm (norm.c:100-107 order:
// x · (1/sqrt(Σx²/HD + eps)) · w) and rotate-half RoPE (y = x·cos +
// rotate_half(x)·sin, rotate_half = cat(−x[HD/2:], x[:HD/2]); the partner is LPR/2
// lanes away).  Shared by the prologue kernel and the QKV GEMM's head epilogue,
// with contraction off, so both round every multiply and add on its own and give
// the same bits.  Every lane of the wavefront must take part (cross-lane sums).
template <int LPR, int HD>
__device__ __forceinline__ float4 lbr_head_row(float4 x, bool norm, float4 w, float eps, bool rope, float4 c4, float4 s4,
                                               int lane);

// Max over aligned groups of G lanes, as lbr_group_sum.
template <int G>
__device__ __forceinline__ float lbr_group_max(float s) {
    static_assert(G == 16 || G == 32 || G == 64, "group of 16, 32 or 64 lanes");
    s = fmaxf(s, lbr_dpp<0xB1>(s));
    s = fmaxf(s, lbr_dpp<0x4E>(s));
    s = fmaxf(s, lbr_dpp<0x141>(s));
    s = fmaxf(s, lbr_dpp<0x140>(s));
    if (G >= 32) {
        const unsigned u = __float_as_uint(s);
        auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        s = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    }
    if (G == 64) {
        const unsigned u = __float_as_uint(s);
        auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        s = fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
    }
    return s;
}

// Whole-wavefront sum / max (every lane active); every lane gets the result.
__device__ __forceinline__ float wave_sum(float v) { return lbr_group_sum<LBR_WAVE>(v); }

__device__ __forceinline__ float wave_max(float v) { return lbr_group_max<LBR_WAVE>(v); }

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024).  `red` must hold
// at least blockDim.x/64 floats.  All threads get the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & (LBR_WAVE - 1);
    const int wid = threadIdx.x / LBR_WAVE;
    const int nw = blockDim.x / LBR_WAVE;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
    const int lane = threadIdx.x & (LBR_WAVE - 1);
    const int wid = threadIdx.x / LBR_WAVE;
    const int nw = blockDim.x / LBR_WAVE;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < nw; ++i) t = fmaxf(t, red[i]);
    return t;
}

// Row norms, shared by the norm kernels and the split-K reduce that ends in a
// norm (so the two give the same bits).  The row is held as float4s, lane /
// thread t holding float4 idx = t + stride·k for k < VPL (0 past the row's
// c4 = cols/4 float4s); wv / bv are the weight (γ) and LayerNorm bias (β) at
// the same positions.  RMSNorm follows csrc/ops/norm.c:100-107 (x · 1/√(Σx²/n
// + eps) · w), LayerNorm norm.c:47-64 (two passes, centred variance).
// Wave form: one wavefront per row (stride 64, wave_sum).
template <bool RMS, int VPL>
__device__ __forceinline__ void lbr_norm_row_wave(float4 (&v)[VPL], const float4 (&wv)[VPL],
                                                  const float4 (&bv)[VPL], float4* __restrict__ o4, int c4,
                                                  int cols, float eps) {
    const int lane = threadIdx.x & 63;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) s += RMS ? lbr_sumsq4(v[k]) : lbr_sum4(v[k]);
    s = wave_sum(s);
    if (RMS) {
        const float scale = 1.0f / sqrtf(s / cols + eps);
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int idx = lane + k * 64;
            if (idx < c4) o4[idx] = lbr_norm_scale(v[k], scale, wv[k]);
        }
        return;
    }
    const float mean = s / cols;
    float var = 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = lane + k * 64;
        if (idx < c4) {
            v[k].x -= mean; v[k].y -= mean; v[k].z -= mean; v[k].w -= mean;
            var += lbr_sumsq4(v[k]);
        }
    }
    var = wave_sum(var);
    const float inv_std = 1.0f / sqrtf(var / cols + eps);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = lane + k * 64;
        if (idx < c4) o4[idx] = lbr_norm_affine(v[k], inv_std, wv[k], bv[k]);
    }
}

// Block form: one 256-thread workgroup per row (stride 256, block_sum through
// red[4]).
template <bool RMS, int VPL>
__device__ __forceinline__ void lbr_norm_row_block(float4 (&v)[VPL], const float4 (&wv)[VPL],
                                                   const float4 (&bv)[VPL], float4* __restrict__ o4, int c4,
                                                   int cols, float eps, float* red) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) s += RMS ? lbr_sumsq4(v[k]) : lbr_sum4(v[k]);
    s = block_sum(s, red);
    if (RMS) {
        const float scale = 1.0f / sqrtf(s / cols + eps);
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int idx = threadIdx.x + k * 256;
            if (idx < c4) o4[idx] = lbr_norm_scale(v[k], scale, wv[k]);
        }
        return;
    }
    const float mean = s / cols;
    float var = 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = threadIdx.x + k * 256;
        if (idx < c4) {
            v[k].x -= mean; v[k].y -= mean; v[k].z -= mean; v[k].w -= mean;
            var += lbr_sumsq4(v[k]);
        }
    }
    var = block_sum(var, red);
    const float inv_std = 1.0f / sqrtf(var / cols + eps);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = threadIdx.x + k * 256;
        if (idx < c4) o4[idx] = lbr_norm_affine(v[k], inv_std, wv[k], bv[k]);
    }
}

// ---------------------------------------------------------------------------
// Decoded launch record
// ---------------------------------------------------------------------------
//
// Each OpNode decodes (once, at plan creation) into one Step: the host
// launcher to call plus every argument it needs, already validated.
struct Step;
typedef void (*step_fn)(const Step&, hipStream_t);

struct Step {
    step_fn run;
    const char* name;         // kernel name for reports
    int node_index;           // first node this step executes
    int n_nodes;              // nodes it covers (1, or the length of a fused run)
    int fuse_kind;            // LBR_FUSE_* of a fused run
    const void* in[MAX_INPUTS];
    void* out;
    int n_in;
    long long i[40];          // integer parameters (meaning per launcher)
    float f[4];               // float parameters
    size_t ws_bytes;          // device workspace this step needs (0 = none)
    void* ws;                 // workspace assigned by the plan (shared by all steps)
};

// Number of compute units of the initialised device (0 before lbr_init).
int lbr_device_cus();

// x / d as ((x · m) >> 32) >> s for 0 ≤ x < 2³¹ (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994, with 31-bit
// dividends: for 2^(l−1) < d ≤ 2^l, m = ⌈2^(31+l) / d⌉ < 2³² and s = l − 1).
// d = 1 is m = 0 (lbr_fdiv passes x through).  The host computes (m, s) once;
// a kernel divides by a uniform d with one multiply-high and a shift.
static inline void lbr_fast_divisor(unsigned d, int* m, int* s) {
    if (d <= 1) {
        *m = 0;
        *s = 0;
        return;
    }
    int l = 0;
    while ((1ULL << l) < d) ++l;
    const unsigned long long mm = ((1ULL << (31 + l)) + d - 1) / d;
    *m = (int)(unsigned)mm;
    *s = l - 1;
}

__device__ __forceinline__ unsigned lbr_fdiv(unsigned x, int m, int s) {
    return m == 0 ? x : __umulhi(x, (unsigned)m) >> s;
}

// Fragment-major layout of one head's [S, hd] rows (the keys the key-quartered
// attention reads, written so by the QKV GEMM's head scatter): rows go in groups
// of 16, and each group's 16 × hd values as hd/16 chunks of [16 rows][16 columns],
// so that the 16-row × 16-column operand fragment one load instruction fetches is
// 1 KiB of contiguous memory. S must be a multiple of 16. The offset of element
// (s, d) is the sum of a row part and a column part.
__host__ __device__ __forceinline__ long long lbr_frag_offset(int s, int d, int hd) {
    return (long long)(s & ~15) * hd + ((d >> 4) << 8) + ((s & 15) << 4) + (d & 15);
}

static inline bool lbr_aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

static inline unsigned lbr_grid(long long work, int per_block, unsigned cap) {
    long long g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > (long long)cap) g = cap;
    return (unsigned)g;
}

// Decoders, one per op family (each returns LBR_OK or an error code after
// setting the thread's error message through lbr_set_error()).
void lbr_set_error(const char* fmt, ...);

int decode_unary(const OpNode* n, Step* s);
int decode_binary(const OpNode* n, Step* s);
int decode_bias_relu(const OpNode* n, Step* s);
int decode_gated_act(const OpNode* n, Step* s);
int decode_reduce(const OpNode* n, Step* s);
int decode_softmax(const OpNode* n, Step* s);
int decode_layernorm(const OpNode* n, Step* s);
int decode_rmsnorm(const OpNode* n, Step* s);
int decode_reshape(const OpNode* n, Step* s);
int decode_transpose(const OpNode* n, Step* s);
int decode_slice(const OpNode* n, Step* s);
int decode_cat(const OpNode* n, Step* s);
int decode_embedding(const OpNode* n, Step* s);
int decode_matmul(const OpNode* n, Step* s);
// DMA GEMM launcher reading A in head layout (fused TRANSPOSE → GEMM); tile = Step::i[14] − 1
step_fn gemm_dma_heads_launcher(int tile, bool has_bias);
// Norm prologue of a DMA GEMM (fused RMSNORM / LAYERNORM → GEMM): Step::i[15]
#define LBR_NORM_RMS 1
#define LBR_NORM_LAYER 2
step_fn gemm_dma_norm_launcher(int tile, bool has_bias, int norm);

// Measured tile choice (plan creation): the DMA tiles a one-batch, unsplit
// GEMM step can run with (its family: plain, norm prologue, head-layout A,
// gated pair); switch the step to one of them; the byte ranges it writes.
int gemm_dma_tune_candidates(const Step& s, int* tiles, int cap);
// Whether a DMA tile (Step::i[14] − 1) holds gated pairs (GEMM_GATED fusion).
bool gemm_dma_tile_pairs(int tile);
// Two K ranges for an unsplit one-batch DMA GEMM (its reduce can then take a
// norm); false leaves the step unchanged.
bool gemm_dma_split2(Step* s);
bool gemm_dma_retile(Step* s, int tile);
bool gemm_dma_set_ksplit(Step* s, int ks);
// Index of the DMA tile called `name` ("32x48", "64x64" ...), or -1.
int gemm_dma_tile_by_name(const char* name);
int gemm_dma_written(const Step& s, void** ptr, size_t* bytes, int cap);
int decode_attention(const OpNode* n, Step* s);
// Whether a decoded attention step can defer its store (its rows staged, then
// written by a second kernel after every read of Q, K and V, so that O may lie
// over them): the key-range split (merge kernel), the key-quartered kernel and
// the 16x16 kernel on folded 64-row blocks (attn_kq_flush).
inline bool lbr_attn_can_defer(const Step& s) { return s.i[7] > 0 || s.i[15] == 1 || s.i[18] == 1; }
// Marks a decoded attention step (lbr_attn_can_defer) as deferring its store,
// with the workspace that needs.
void lbr_attn_defer(Step* s);
// Step name of an attention: its kernel, then "+v" (V read from a row-major
// source), "+transpose" (O stored as [B, S, H, D]) and, for store 1 / 2,
// "+defer" / "+relay".
const char* lbr_attn_step_name(const Step& s, bool v, bool t, int store);
// Fused MLP (mlp.hip): whether rows of width D, hidden H and output D2 fit
// the one-kernel form; its launcher (Step layout in mlp.hip).
bool mlp_shape_ok(long long M, long long D, long long H, long long D2);
step_fn mlp_launcher(long long D, int act, bool oproj = false);
// Raises the MLP kernels' dynamic LDS limit on the current device (lbr_init).
hipError_t mlp_prepare_device();
// Whether the MLP kernel can also compute its input rows x = O·Woᵀ (+ bo)
// (+ R0) from O in head layout (head dim hd, K0 = O's row width).
bool mlp_proj_ok(long long D, long long H, long long K0, long long hd);

// A node record's counts within its arrays (n_inputs ≤ MAX_INPUTS, n_dims ≤
// MAX_DIMS), elem_size 1, 2, 4 or 8, no negative dim and at most
// LBR_MAX_ELEMENTS as the product of its nonzero dims; else an error naming
// node `index`.
#define LBR_MAX_ELEMENTS (1LL << 40)
int lbr_node_check(const OpNode* n, int index);

// Helpers over the node record (same meaning as csrc/executor.c:30-48).
static inline long long node_total(const OpNode* n) {
    long long t = 1;
    for (int i = 0; i < n->n_dims; ++i) t *= n->out_shape[i];
    return t;
}
static inline long long node_leading(const OpNode* n) {
    long long r = 1;
    for (int i = 0; i < n->n_dims - 1; ++i) r *= n->out_shape[i];
    return r;
}
static inline int node_last_dim(const OpNode* n) {
    return n->n_dims > 0 ? n->out_shape[n->n_dims - 1] : 1;
}
// Whether extents an op's extras give (each ≥ 0) multiply to the node's
// element count, without overflow.
static inline bool lbr_sizes_match(const OpNode* n, std::initializer_list<long long> ext) {
    long long t = 1;
    for (long long e : ext) {
        if (e < 0 || (e > 0 && t > LBR_MAX_ELEMENTS / e)) return false;
        t *= e;
    }
    return t == node_total(n);
}
static inline float node_extra_float(const OpNode* n, int idx) {
    union { int i; float f; } u;
    u.i = n->extra[idx];
    return u.f;
}
