// mlp.hip — the feed-forward block of a small-M graph as one kernel.
//
// Replaces the chain [LAYERNORM | RMSNORM →] MATMUL[_ADD] → RELU | GELU |
// SILU → MATMUL[_ADD] [→ ADD(residual)] (the MLP of the reference's
// transformer blocks, each node dispatched by csrc/executor.c:197-224,
// 296-308 and the element-wise cases) when its hidden activations fit in
// LDS: one 4-wavefront workgroup per 16 rows normalises its rows into LDS,
// computes h = act(x·W1ᵀ + b1) into LDS, then y = h·W2ᵀ + b2 (+ R) to HBM.
// For the launch-bound sizes it serves, each wavefront's share of both
// weight matrices (at most 16 float4 fragments per lane per GEMM, 4 column
// blocks) is loaded into registers at the start.
// The hidden activations never leave the CU and the chain is one launch;
// for the toy block's 32 rows the two GEMMs and the norm otherwise cost
// three launches and two HBM round trips of h.
//
// The results equal the unfused kernels' bit for bit:
// * the norm uses norm_wave_rows' per-lane arithmetic (one wavefront per
//   row, float4 idx = lane + 64·k, the same sums and affine terms with
//   contraction off, lbr_sum4 / lbr_sumsq4 / lbr_norm_*, and wave_sum);
// * each GEMM sums an output's K terms in the DMA GEMM's order: 16-wide
//   chunks in order, and within a chunk v_mfma_f32_16x16x4_f32 number q
//   reduces k = 16c + 4·kq + q over the four lane groups kq;
// * the epilogues add the bias, apply the activation, and add the residual
//   in the unfused order (the residual ADD is commutative in IEEE).
#include "lbr_device.h"

#include <math.h>

namespace {

constexpr int MLP_NT = 256;     // 4 wavefronts
constexpr int MLP_RB = 16;      // rows per workgroup (one MFMA row block)
constexpr int MLP_FR = 16;      // B fragments (float4) per wave per GEMM: all loaded up front
constexpr int MLP_NBW = 4;      // column blocks per wave per GEMM (its biases, loaded up front)
constexpr size_t MLP_LDS_MAX = 64 * 1024;   // dynamic LDS without a launch attribute

struct MlpArgs {
    const float* x;     // [M, D]: the norm's input, or GEMM1's A
    const float* w1;    // [H, D]
    const float* b1;    // [H] or null
    const float* w2;    // [D2, H]
    const float* b2;    // [D2] or null
    const float* r;     // [M, D2] residual or null
    const float* g;     // norm weight [D] (norm != 0)
    const float* be;    // LayerNorm bias [D]
    float* y;           // [M, D2]
    int M, D, H, D2, act, norm;
    float alpha1, alpha2, eps;
};

// This wave's B fragments of C = A·Wᵀ, W [cols, K] row-major: the wave takes
// column blocks wave, wave + 4, …; fragment p = (block j, 16-wide K chunk c),
// block-major; lane (kq, lr) holds W[16·(wave + 4j) + lr][16c + 4kq .. +3].
// All P ≤ MLP_FR of them are issued together (P is wave-uniform).
__device__ __forceinline__ void mlp_load_frags(const float* __restrict__ W, int K, int P, float4 (&f)[MLP_FR]) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const float* __restrict__ wl = W + (long long)(16 * wave + (lane & 15)) * K + 4 * (lane >> 4);
    const int nch = K / 16;
    int j = 0, c = 0;
#pragma unroll
    for (int p = 0; p < MLP_FR; ++p) {
        if (p < P) {
            f[p] = *reinterpret_cast<const float4*>(wl + (long long)j * 64 * K + 16 * c);
            if (++c == nch) {
                c = 0;
                ++j;
            }
        }
    }
}

// C[16 rows, this wave's blocks] = A[16, K] (LDS rows of stride lda) · Wᵀ from
// the P fragments; each block's result goes to epi(local block j, acc) with
// D[4·kq + r][lr] in acc[r].
template <typename Epi>
__device__ __forceinline__ void mlp_gemm(const float* __restrict__ A, int lda, int K, int P, const float4 (&f)[MLP_FR],
                                         Epi epi) {
    const int lane = threadIdx.x & 63;
    const float* a_row = A + (lane & 15) * lda + 4 * (lane >> 4);
    const int nch = K / 16;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    int j = 0, c = 0;
#pragma unroll
    for (int p = 0; p < MLP_FR; ++p) {
        if (p < P) {
            const float4 a = *reinterpret_cast<const float4*>(a_row + 16 * c);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, f[p].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, f[p].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, f[p].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, f[p].w, acc, 0, 0, 0);
            if (++c == nch) {
                epi(j, acc);
                acc = floatx4{0.f, 0.f, 0.f, 0.f};
                c = 0;
                ++j;
            }
        }
    }
}

// A loaded row normalised into LDS (one wavefront; w / b the norm's weight and
// bias float4s of the lane), or copied when norm == 0.
template <int VPL>
__device__ __forceinline__ void mlp_norm_row(const MlpArgs& g, float4 (&v)[VPL], const float4 (&w)[VPL],
                                             const float4 (&b)[VPL], float* dst) {
    const int lane = threadIdx.x & 63;
    const int c4 = g.D / 4;
    float4* d4 = reinterpret_cast<float4*>(dst);
    if (g.norm == 0) {
#pragma unroll
        for (int k = 0; k < VPL; ++k)
            if (lane + k * 64 < c4) d4[lane + k * 64] = v[k];
        return;
    }
    const bool rms = g.norm == LBR_NORM_RMS;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) s += rms ? lbr_sumsq4(v[k]) : lbr_sum4(v[k]);
    s = wave_sum(s);
    if (rms) {
        const float scale = 1.0f / sqrtf(s / g.D + g.eps);
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int idx = lane + k * 64;
            if (idx < c4) d4[idx] = lbr_norm_scale(v[k], scale, w[k]);
        }
        return;
    }
    const float mean = s / g.D;
    float var = 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        if (lane + k * 64 < c4) {
            v[k].x -= mean;
            v[k].y -= mean;
            v[k].z -= mean;
            v[k].w -= mean;
            var += lbr_sumsq4(v[k]);
        }
    }
    var = wave_sum(var);
    const float inv_std = 1.0f / sqrtf(var / g.D + g.eps);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = lane + k * 64;
        if (idx < c4) d4[idx] = lbr_norm_affine(v[k], inv_std, w[k], b[k]);
    }
}

// LDS: xs [16][D + 4] (normalised rows), hs [16][H + 4] (hidden rows); the
// 4-float row padding puts the 16 rows of a fragment read in distinct banks.
// Every global load (the wave's 4 rows, the norm's weight and bias, both
// weights' fragments, both biases, the residual) is issued before the rows
// are normalised, so the kernel waits for one memory round trip.  The output
// is written only after the workgroup has read all of its residual rows (the
// residual may lie under the output, row for row).
template <int ACT, int VPL>
__global__ __launch_bounds__(MLP_NT) void mlp_rows(MlpArgs g) {
    extern __shared__ float smem[];
    const int ldx = g.D + 4, ldh = g.H + 4;
    float* xs = smem;
    float* hs = smem + MLP_RB * ldx;
    const long long r0 = (long long)blockIdx.x * MLP_RB;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, kq = lane >> 4;
    const int nb1 = g.H / 16 > wave ? (g.H / 16 - wave + 3) / 4 : 0;
    const int nb2 = g.D2 / 16 > wave ? (g.D2 / 16 - wave + 3) / 4 : 0;
    // the wave's 4 rows and the norm's weight and bias first (needed first), then
    // both weights' fragments, the biases and the residual; a lane past the row's
    // D/4 float4s holds 0, as in norm_wave_rows, so the row sums see exactly the row
    const int c4 = g.D / 4;
    float4 xv[MLP_RB / 4][VPL], nw[VPL], nbv[VPL];
#pragma unroll
    for (int i = 0; i < MLP_RB / 4; ++i) {
        const long long row = r0 + wave + 4 * i;
        const float4* xr = reinterpret_cast<const float4*>(g.x + row * g.D);
#pragma unroll
        for (int k = 0; k < VPL; ++k)
            xv[i][k] = row < g.M && lane + 64 * k < c4 ? xr[lane + 64 * k] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const bool in = g.norm && lane + 64 * k < c4;
        nw[k] = in ? reinterpret_cast<const float4*>(g.g)[lane + 64 * k] : make_float4(0.f, 0.f, 0.f, 0.f);
        nbv[k] = in && g.norm == LBR_NORM_LAYER ? reinterpret_cast<const float4*>(g.be)[lane + 64 * k]
                                                : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float4 f1[MLP_FR], f2[MLP_FR];
    mlp_load_frags(g.w1, g.D, nb1 * (g.D / 16), f1);
    mlp_load_frags(g.w2, g.H, nb2 * (g.H / 16), f2);
    float bias1[MLP_NBW], bias2[MLP_NBW], res[MLP_NBW][4];
#pragma unroll
    for (int j = 0; j < MLP_NBW; ++j) {
        const int col = 16 * (wave + 4 * j) + lr;
        bias1[j] = g.b1 && j < nb1 ? g.b1[col] : 0.f;
        bias2[j] = g.b2 && j < nb2 ? g.b2[col] : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const long long row = r0 + 4 * kq + r;
            res[j][r] = g.r && j < nb2 && row < g.M ? g.r[row * g.D2 + col] : 0.f;
        }
    }
#pragma unroll
    for (int i = 0; i < MLP_RB / 4; ++i) {
        if (r0 + wave + 4 * i < g.M) {
            mlp_norm_row<VPL>(g, xv[i], nw, nbv, xs + (wave + 4 * i) * ldx);
        } else {   // rows past M: zeros (their results are never stored)
            float4* d4 = reinterpret_cast<float4*>(xs + (wave + 4 * i) * ldx);
#pragma unroll
            for (int k = 0; k < VPL; ++k)
                if (lane + 64 * k < g.D / 4) d4[lane + 64 * k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    __syncthreads();
    // h = act(xs·W1ᵀ + b1): D[4·kq + r][lr] of block j is h[4·kq + r][16·(wave + 4j) + lr]
    mlp_gemm(xs, ldx, g.D, nb1 * (g.D / 16), f1, [&](int j, const floatx4& acc) {
        const int col = 16 * (wave + 4 * j) + lr;
        float bv = 0.f;
#pragma unroll
        for (int t = 0; t < MLP_NBW; ++t) bv = t == j ? bias1[t] : bv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float v = g.b1 ? acc[r] + bv : g.alpha1 * acc[r];
            hs[(4 * kq + r) * ldh + col] = lbr_act(ACT, v);
        }
    });
    __syncthreads();
    // y = hs·W2ᵀ + b2 (+ R)
    mlp_gemm(hs, ldh, g.H, nb2 * (g.H / 16), f2, [&](int j, const floatx4& acc) {
        const int col = 16 * (wave + 4 * j) + lr;
        float bv = 0.f, rv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < MLP_NBW; ++t) {
            bv = t == j ? bias2[t] : bv;
#pragma unroll
            for (int r = 0; r < 4; ++r) rv[r] = t == j ? res[t][r] : rv[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const long long row = r0 + 4 * kq + r;
            if (row >= g.M) continue;
            float v = g.b2 ? acc[r] + bv : g.alpha2 * acc[r];
            if (g.r) v = v + rv[r];
            g.y[row * g.D2 + col] = v;
        }
    });
}

// Step: in[0] x, in[1] W1, in[2] b1, in[3] W2, in[4] b2, in[5] R, in[6] norm
// weight, in[7] LayerNorm bias; i[0] M, i[1] D, i[2] H, i[3] D2, i[4] act
// (LBR_ACT_*), i[5] norm (LBR_NORM_*, 0 none); f[0] alpha1, f[1] alpha2,
// f[2] eps.
template <int ACT, int VPL>
void launch_mlp(const Step& s, hipStream_t st) {
    MlpArgs g;
    g.x = (const float*)s.in[0];
    g.w1 = (const float*)s.in[1];
    g.b1 = (const float*)s.in[2];
    g.w2 = (const float*)s.in[3];
    g.b2 = (const float*)s.in[4];
    g.r = (const float*)s.in[5];
    g.g = (const float*)s.in[6];
    g.be = (const float*)s.in[7];
    g.y = (float*)s.out;
    g.M = (int)s.i[0];
    g.D = (int)s.i[1];
    g.H = (int)s.i[2];
    g.D2 = (int)s.i[3];
    g.act = (int)s.i[4];
    g.norm = (int)s.i[5];
    g.alpha1 = s.f[0];
    g.alpha2 = s.f[1];
    g.eps = s.f[2];
    if (g.M <= 0) return;
    const size_t lds = (size_t)MLP_RB * (g.D + 4 + g.H + 4) * sizeof(float);
    hipLaunchKernelGGL((mlp_rows<ACT, VPL>), dim3((unsigned)((g.M + MLP_RB - 1) / MLP_RB)), dim3(MLP_NT), lds, st, g);
}

}  // namespace

// Fragments per wave of a GEMM with `cols` output columns and depth K.
static long long mlp_frags(long long cols, long long K) { return (cols / 16 + 3) / 4 * (K / 16); }

bool mlp_shape_ok(long long M, long long D, long long H, long long D2) {
    return M > 0 && D > 0 && H > 0 && D2 > 0 && D % 16 == 0 && H % 16 == 0 && D2 % 16 == 0 && D <= 1024 &&
           (H / 16 + 3) / 4 <= MLP_NBW && (D2 / 16 + 3) / 4 <= MLP_NBW && mlp_frags(H, D) <= MLP_FR &&
           mlp_frags(D2, H) <= MLP_FR && (size_t)MLP_RB * (D + 4 + H + 4) * sizeof(float) <= MLP_LDS_MAX;
}

template <int ACT>
static step_fn mlp_launcher_act(long long D) {
    return D <= 256 ? launch_mlp<ACT, 1> : D <= 512 ? launch_mlp<ACT, 2> : launch_mlp<ACT, 4>;
}

step_fn mlp_launcher(long long D, int act) {
    switch (act) {
        case LBR_ACT_RELU: return mlp_launcher_act<LBR_ACT_RELU>(D);
        case LBR_ACT_GELU: return mlp_launcher_act<LBR_ACT_GELU>(D);
        default: return mlp_launcher_act<LBR_ACT_SILU>(D);
    }
}
