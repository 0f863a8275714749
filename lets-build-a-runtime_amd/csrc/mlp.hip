// mlp.hip — the feed-forward block of a small-M graph as one kernel.
//
// Replaces the chain [LAYERNORM | RMSNORM →] MATMUL[_ADD] → RELU | GELU |
// SILU → MATMUL[_ADD] [→ ADD(residual)] (the MLP of the reference's
// transformer blocks, each node dispatched by csrc/executor.c:197-224,
// 296-308 and the element-wise cases) when its hidden activations fit in
// LDS: one 4-wavefront workgroup per 16 rows normalises its rows into LDS,
// computes h = act(x·W1ᵀ + b1) into LDS, then y = h·W2ᵀ + b2 (+ R) to HBM.
// For the launch-bound sizes it serves, both weight matrices (at most 64 KB
// each) are staged whole in LDS by direct-to-LDS DMA issued at the start,
// and each wavefront reads its fragments (at most 16 float4 per lane per GEMM,
// 4 column blocks) from there.
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
constexpr int MLP_FR = 16;      // B fragments (float4) per wave per GEMM: all read from LDS up front
constexpr int MLP_DMA = 16;     // weight DMA instructions per wave per GEMM (≤ 64 KB of weight)
constexpr int MLP_WMAX = 4 * MLP_DMA * 256;   // floats of one staged weight (64 KB)
constexpr int MLP_NBW = 4;      // column blocks per wave per GEMM (its biases, loaded up front)
constexpr size_t MLP_LDS_MAX = 160 * 1024;  // gfx950's LDS per workgroup (the launcher raises the dynamic limit)
constexpr int MLP_HAS_B1 = 1, MLP_HAS_B2 = 2, MLP_HAS_RESID = 4, MLP_RES_X = 8;
constexpr int MLP_OC = 8;       // projection prologue: K0/16 chunks a lane holds (K0 ≤ 128)
constexpr int MLP_OB = 2;       // projection prologue: column blocks per wave (D ≤ 128)

// W [R, K] as staged in LDS (mlp_stage_weight): its shape, the chunk swizzle
// mask and the divisor by K/4.
struct MlpWeight {
    int R, K, mask;
    int kc_m, kc_s;   // divisor by K/4 (lbr_fdiv)
};

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
    int has;            // MLP_HAS_*: which of b1, b2, r are present (absent ones, and g / be, point at x)
    int M, D, H, D2, act, norm;
    float alpha1, alpha2, eps;
    MlpWeight w1s, w2s;   // W1 [H, D] and W2 [D2, H] as staged in LDS
    // projection prologue (OPROJ): x = O·Woᵀ (+ bo) (+ R0) computed here and
    // written to x, O in head layout [B, oH, oS, ohd] (columns h·ohd + d)
    const float* oa;      // O
    const float* ow;      // Wo [D, K0]
    const float* ob;      // bo [D] (or x)
    const float* orr;     // R0 [M, D] (or x)
    float* ox;            // x, written
    int K0, oH, oS, ohd, ohas;   // ohas: MLP_HAS_B1 (bo), MLP_HAS_RESID (R0), MLP_RES_X (r is x)
    float oalpha;
};

// A weight W [R, K] (row-major) staged in LDS by direct-to-LDS DMA.  In LDS
// the rows keep their order and length, and 16-byte chunk q of row r holds
// W's chunk q ^ (r & mask) of that row (mask + 1 = the largest power of two
// ≤ 16 dividing K/4), so the 16 rows of a fragment read fall in distinct bank
// groups.  One DMA instruction fills 64 consecutive LDS chunks from 64
// global chunks of the same rows, permuted within each row: a coalesced 1 KB
// read, where loading fragments straight from HBM gathers 16 rows × 64 B per
// instruction (2.2× slower measured at the toy block's 128 KB).  Each wave
// issues MLP_DMA instructions (R·K/256 in all, at most 4·MLP_DMA; a wave
// past the end repeats the last one, writing the same bytes again), so every
// wave has the same count in flight.

__device__ __forceinline__ void mlp_stage_weight(const float* __restrict__ W, const MlpWeight& w, float* lds) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kc = w.K / 4, n = w.R * kc / 64;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, w.R * w.K * 4, 0x00020000);
#pragma unroll
    for (int t = 0; t < MLP_DMA; ++t) {
        const int ins = min(wave + 4 * t, n - 1);
        const int L = ins * 64 + lane;                        // LDS chunk: row r, position q
        const int r = (int)lbr_fdiv((unsigned)L, w.kc_m, w.kc_s);
        const int q = L - r * kc;
        lbr_dma16(rs, lds + ins * 256, (unsigned)(r * w.K + 4 * (q ^ (r & w.mask))) * 4u, 0u);
    }
}

// This wave's B fragments of C = A·Wᵀ from the staged W: the wave takes
// column blocks wave, wave + 4, …; fragment p = (block j, 16-wide K chunk c),
// block-major; lane (kq, lr) holds W[16·(wave + 4j) + lr][16c + 4kq .. +3].
// All MLP_FR reads issue (past P the last fragment repeats; a wave with no
// block reads row R − 1), with no branch around them.
__device__ __forceinline__ void mlp_read_frags(const float* __restrict__ lds, const MlpWeight& w, int P,
                                               float4 (&f)[MLP_FR]) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nch = w.K / 16;
    int j = 0, c = 0;
#pragma unroll
    for (int p = 0; p < MLP_FR; ++p) {
        const int r = min(16 * (wave + 4 * j) + (lane & 15), w.R - 1);
        f[p] = *reinterpret_cast<const float4*>(lds + r * w.K + 4 * ((4 * c + (lane >> 4)) ^ (r & w.mask)));
        const bool step = p + 1 < P;   // wave-uniform: stay on the last fragment past P
        c = step ? (c + 1 == nch ? 0 : c + 1) : c;
        j = step && c == 0 ? j + 1 : j;
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
    for (int k = 0; k < VPL; ++k) {   // a lane past the row adds 0, as norm_wave_rows' zeroed values do
        const float t = rms ? lbr_sumsq4(v[k]) : lbr_sum4(v[k]);
        s += lane + k * 64 < c4 ? t : 0.f;
    }
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

// LDS: W1 [H][D] and W2 [D2][H] (staged, chunk-swizzled; static), xs [16][D + 4]
// (normalised rows), hs [16][H + 4] (hidden rows); the 4-float row padding
// puts the 16 rows of an A fragment read in distinct banks.  Every global
// load (the wave's 4 rows, the norm's weight and bias, both biases, the
// residual, then both weights' DMAs) is issued before the rows are
// normalised, so the kernel waits for one memory round trip.  The output is
// written only after the workgroup has read all of its residual rows (the
// residual may lie under the output, row for row).
template <int ACT, int VPL, bool OPROJ>
__global__ __launch_bounds__(MLP_NT) void mlp_rows(MlpArgs g) {
    // the staged weights in LDS variables of their own: the compiler then
    // knows the norm's and GEMM1's LDS stores do not touch what the weight
    // DMAs still in flight write, and does not wait for them
    __shared__ __attribute__((aligned(1024))) float w1l[MLP_WMAX];
    __shared__ __attribute__((aligned(1024))) float w2l[MLP_WMAX];
    extern __shared__ float smem[];
    const int ldx = g.D + 4, ldh = g.H + 4;
    float* xs = smem;
    float* hs = xs + MLP_RB * ldx;
    float* xin = hs + MLP_RB * ldh;   // OPROJ: the projected rows x
    const long long r0 = (long long)blockIdx.x * MLP_RB;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, kq = lane >> 4;
    const int nb1 = g.H / 16 > wave ? (g.H / 16 - wave + 3) / 4 : 0;
    const int nb2 = g.D2 / 16 > wave ? (g.D2 / 16 - wave + 3) / 4 : 0;
    // Every load issues unconditionally from a clamped address (the host
    // replaces an absent input by x and says so in g.has), so no branch hides
    // a load from the compiler's count: the norm waits only for the rows,
    // GEMM1 for W1's fragments.  Values loaded from outside the data are never
    // used: the norm counts only lanes inside the row, and the epilogues use
    // a bias or residual value only for a present input, a block of the wave
    // and a row below M.  The rows come first (needed first), the weights' DMAs
    // last.
    const int c4 = g.D / 4;
    float4 xv[MLP_RB / 4][VPL], nw[VPL], nbv[VPL];
    // OPROJ: lane (kq, lr) holds O's row r0 + lr, columns 16c + 4kq .. +3 (one
    // head's run of 4: ohd % 4 == 0), chunk-major Wo fragments of the wave's
    // blocks wave, wave + 4 (f0[c·MLP_OB + j]), the bias and R0 in the
    // accumulator layout (rows 4kq + r, column 16·(wave + 4j) + lr)
    float4 a0[OPROJ ? MLP_OC : 1], f0[OPROJ ? MLP_OC * MLP_OB : 1];
    float bias0[MLP_OB], r0v[MLP_OB][4];
    const int nch0 = g.K0 / 16;
    const int nb0 = g.D / 16 > wave ? (g.D / 16 - wave + 3) / 4 : 0;
    if constexpr (OPROJ) {
        const int row = (int)min(r0 + lr, (long long)g.M - 1);
        const int b = row / g.oS, sq = row - b * g.oS;
#pragma unroll
        for (int c = 0; c < MLP_OC; ++c) {
            const int k = 16 * min(c, nch0 - 1) + 4 * kq, h = k / g.ohd;
            a0[c] = *reinterpret_cast<const float4*>(
                g.oa + ((long long)(b * g.oH + h) * g.oS + sq) * g.ohd + (k - h * g.ohd));
#pragma unroll
            for (int j = 0; j < MLP_OB; ++j) {
                const int wr = min(16 * (wave + 4 * j) + lr, g.D - 1);
                f0[c * MLP_OB + j] = *reinterpret_cast<const float4*>(g.ow + (long long)wr * g.K0 + k);
            }
        }
#pragma unroll
        for (int j = 0; j < MLP_OB; ++j) {
            const int col = min(16 * (wave + 4 * j) + lr, g.D - 1);
            bias0[j] = g.ob[(g.ohas & MLP_HAS_B1) ? col : 0];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const long long rr = min(r0 + 4 * kq + r, (long long)g.M - 1);
                r0v[j][r] = g.orr[(g.ohas & MLP_HAS_RESID) ? rr * g.D + col : 0];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < MLP_RB / 4; ++i) {
            const long long row = min(r0 + wave + 4 * i, (long long)g.M - 1);
            const float4* xr = reinterpret_cast<const float4*>(g.x + row * g.D);
#pragma unroll
            for (int k = 0; k < VPL; ++k) xv[i][k] = xr[min(lane + 64 * k, c4 - 1)];
        }
    }
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = min(lane + 64 * k, c4 - 1);
        nw[k] = reinterpret_cast<const float4*>(g.g)[idx];
        nbv[k] = reinterpret_cast<const float4*>(g.be)[idx];
    }
    float bias1[MLP_NBW], bias2[MLP_NBW], res[MLP_NBW][4];
#pragma unroll
    for (int j = 0; j < MLP_NBW; ++j) {
        const int col = 16 * (wave + 4 * j) + lr;
        // an absent bias or residual reads element 0 of x
        bias1[j] = g.b1[(g.has & MLP_HAS_B1) ? min(col, g.H - 1) : 0];
        bias2[j] = g.b2[(g.has & MLP_HAS_B2) ? min(col, g.D2 - 1) : 0];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const long long row = min(r0 + 4 * kq + r, (long long)g.M - 1);
            res[j][r] = g.r[(g.has & MLP_HAS_RESID) && !(g.ohas & MLP_RES_X) ? row * g.D2 + min(col, g.D2 - 1) : 0];
        }
    }
    // the weights last: W1's MLP_DMA instructions, then W2's (their order fixes
    // the vmcnt thresholds below)
    __builtin_amdgcn_sched_barrier(0);
    mlp_stage_weight(g.w1, g.w1s, w1l);
    __builtin_amdgcn_sched_barrier(0);
    mlp_stage_weight(g.w2, g.w2s, w2l);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (OPROJ) {
        // x = O·Woᵀ (+ bo) (+ R0) in the transposed-A GEMM's order: 16-wide
        // chunks in order, MFMA q over k = 16c + 4kq + q; bias, then residual
        floatx4 acc0[MLP_OB];
#pragma unroll
        for (int j = 0; j < MLP_OB; ++j) acc0[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < MLP_OC; ++c) {
            if (c < nch0) {
#pragma unroll
                for (int j = 0; j < MLP_OB; ++j) {
                    if (j < nb0) {
                        const float4 fb = f0[c * MLP_OB + j];
                        acc0[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[c].x, fb.x, acc0[j], 0, 0, 0);
                        acc0[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[c].y, fb.y, acc0[j], 0, 0, 0);
                        acc0[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[c].z, fb.z, acc0[j], 0, 0, 0);
                        acc0[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[c].w, fb.w, acc0[j], 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < MLP_OB; ++j) {
            if (j >= nb0) continue;
            const int col = 16 * (wave + 4 * j) + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = (g.ohas & MLP_HAS_B1) ? acc0[j][r] + bias0[j] : g.oalpha * acc0[j][r];
                if (g.ohas & MLP_HAS_RESID) v = v + r0v[j][r];
                const long long row = r0 + 4 * kq + r;
                xin[(4 * kq + r) * ldx + col] = v;
                if (row < g.M) g.ox[row * g.D + col] = v;
                if (g.ohas & MLP_RES_X) res[j][r] = v;   // the MLP's residual is x (D2 == D)
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < MLP_RB / 4; ++i) {
            const float4* xr = reinterpret_cast<const float4*>(xin + (wave + 4 * i) * ldx);
#pragma unroll
            for (int k = 0; k < VPL; ++k) xv[i][k] = xr[min(lane + 64 * k, c4 - 1)];
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
    // this wave's W1 DMAs have landed (at most W2's are still out), then every wave's
    __builtin_amdgcn_s_waitcnt(lbr_waitcnt_vm(MLP_DMA));
    __syncthreads();
    float4 f[MLP_FR];
    mlp_read_frags(w1l, g.w1s, nb1 * (g.D / 16), f);
    // h = act(xs·W1ᵀ + b1): D[4·kq + r][lr] of block j is h[4·kq + r][16·(wave + 4j) + lr]
    mlp_gemm(xs, ldx, g.D, nb1 * (g.D / 16), f, [&](int j, const floatx4& acc) {
        const int col = 16 * (wave + 4 * j) + lr;
        float bv = 0.f;
#pragma unroll
        for (int t = 0; t < MLP_NBW; ++t) bv = t == j ? bias1[t] : bv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float v = (g.has & MLP_HAS_B1) ? acc[r] + bv : g.alpha1 * acc[r];
            hs[(4 * kq + r) * ldh + col] = lbr_act(ACT, v);
        }
    });
    __builtin_amdgcn_s_waitcnt(lbr_waitcnt_vm(0));   // W2's DMAs too
    __syncthreads();
    mlp_read_frags(w2l, g.w2s, nb2 * (g.H / 16), f);
    // y = hs·W2ᵀ + b2 (+ R)
    mlp_gemm(hs, ldh, g.H, nb2 * (g.H / 16), f, [&](int j, const floatx4& acc) {
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
            float v = (g.has & MLP_HAS_B2) ? acc[r] + bv : g.alpha2 * acc[r];
            if (g.has & MLP_HAS_RESID) v = v + rv[r];
            g.y[row * g.D2 + col] = v;
        }
    });
}

MlpWeight mlp_weight(int R, int K) {
    MlpWeight w;
    w.R = R;
    w.K = K;
    const int kc = K / 4;
    w.mask = (kc & -kc) >= 16 ? 15 : (kc & -kc) - 1;
    lbr_fast_divisor((unsigned)kc, &w.kc_m, &w.kc_s);
    return w;
}

// Dynamic LDS (xs, hs, and with the projection prologue xin); the two
// staged weights take 2·MLP_WMAX floats more.
size_t mlp_lds_bytes(long long D, long long H, bool oproj) {
    return (size_t)(MLP_RB * (D + 4 + H + 4 + (oproj ? D + 4 : 0))) * sizeof(float);
}

// Step: in[0] x, in[1] W1, in[2] b1, in[3] W2, in[4] b2, in[5] R, in[6] norm
// weight, in[7] LayerNorm bias; i[0] M, i[1] D, i[2] H, i[3] D2, i[4] act
// (LBR_ACT_*), i[5] norm (LBR_NORM_*, 0 none); f[0] alpha1, f[1] alpha2,
// f[2] eps.  Projection prologue (lbr_merge_proj_mlp): i[6] = 1, i[7] K0,
// i[8..10] O's heads, tokens per batch and head dim, i[11] MLP_HAS_B1 /
// MLP_HAS_RESID / MLP_RES_X, f[3] alpha; in[8] O, in[9] Wo, in[10] bo,
// in[11] R0 (x = in[0] is then written).
template <int ACT, int VPL, bool OPROJ>
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
    // absent inputs: a flag, and a read-only input with at least D floats in
    // place of the pointer (x, or Wo when x is written here): every lane loads
    // from a valid address and the kernel discards the value
    const float* stand_in = OPROJ ? (const float*)s.in[9] : g.x;
    g.has = (g.b1 ? MLP_HAS_B1 : 0) | (g.b2 ? MLP_HAS_B2 : 0) | (g.r ? MLP_HAS_RESID : 0);
    g.ohas = OPROJ ? (int)s.i[11] : 0;
    if (!g.b1) g.b1 = stand_in;
    if (!g.b2) g.b2 = stand_in;
    if (!g.r || (g.ohas & MLP_RES_X)) g.r = stand_in;   // MLP_RES_X: the residual comes from registers
    if (!g.g) g.g = stand_in;
    if (!g.be) g.be = stand_in;
    g.w1s = mlp_weight(g.H, g.D);
    g.w2s = mlp_weight(g.D2, g.H);
    g.oa = g.ow = g.ob = g.orr = stand_in;
    g.ox = nullptr;
    g.K0 = 16;
    g.oH = g.oS = g.ohd = 1;
    g.oalpha = 1.f;
    if (OPROJ) {
        g.K0 = (int)s.i[7];
        g.oH = (int)s.i[8];
        g.oS = (int)s.i[9];
        g.ohd = (int)s.i[10];
        g.oalpha = s.f[3];
        g.oa = (const float*)s.in[8];
        g.ow = (const float*)s.in[9];
        g.ob = s.in[10] ? (const float*)s.in[10] : stand_in;
        g.orr = s.in[11] ? (const float*)s.in[11] : stand_in;
        g.ox = (float*)s.in[0];
    }
    hipLaunchKernelGGL((mlp_rows<ACT, VPL, OPROJ>), dim3((unsigned)((g.M + MLP_RB - 1) / MLP_RB)), dim3(MLP_NT),
                       mlp_lds_bytes(g.D, g.H, OPROJ), st, g);
}

}  // namespace

// Fragments per wave of a GEMM with `cols` output columns and depth K.
static long long mlp_frags(long long cols, long long K) { return (cols / 16 + 3) / 4 * (K / 16); }

bool mlp_shape_ok(long long M, long long D, long long H, long long D2) {
    return M > 0 && D > 0 && H > 0 && D2 > 0 && D % 16 == 0 && H % 16 == 0 && D2 % 16 == 0 && D <= 1024 &&
           (H / 16 + 3) / 4 <= MLP_NBW && (D2 / 16 + 3) / 4 <= MLP_NBW && mlp_frags(H, D) <= MLP_FR &&
           mlp_frags(D2, H) <= MLP_FR && H * D <= MLP_WMAX && D2 * H <= MLP_WMAX &&
           mlp_lds_bytes(D, H, false) + 2 * MLP_WMAX * sizeof(float) <= MLP_LDS_MAX;
}

template <int ACT, bool OPROJ>
static hipError_t mlp_raise_lds() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&mlp_rows<ACT, 1, OPROJ>),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)(MLP_LDS_MAX - 2 * MLP_WMAX * sizeof(float)));
}

// The kernel's LDS (128 KB static + xs, hs) exceeds the default: lbr_init
// raises the dynamic limit of every instantiation the launcher hands out, on
// the device it initialises (outside any graph capture), so choosing the
// kernel at plan creation makes no device call.
hipError_t mlp_prepare_device() {
    hipError_t e = mlp_raise_lds<LBR_ACT_RELU, false>();
    if (e == hipSuccess) e = mlp_raise_lds<LBR_ACT_RELU, true>();
    if (e == hipSuccess) e = mlp_raise_lds<LBR_ACT_GELU, false>();
    if (e == hipSuccess) e = mlp_raise_lds<LBR_ACT_GELU, true>();
    if (e == hipSuccess) e = mlp_raise_lds<LBR_ACT_SILU, false>();
    if (e == hipSuccess) e = mlp_raise_lds<LBR_ACT_SILU, true>();
    return e;
}

// D ≤ 256 always holds (each wave's W1 fragments, ceil(H/64)·D/16, are at
// most 16), so the rows take one float4 a lane.
template <int ACT>
static step_fn mlp_launcher_act(bool oproj) {
    return oproj ? launch_mlp<ACT, 1, true> : launch_mlp<ACT, 1, false>;
}

step_fn mlp_launcher(long long D, int act, bool oproj) {
    if (D > 256) return nullptr;
    switch (act) {
        case LBR_ACT_RELU: return mlp_launcher_act<LBR_ACT_RELU>(oproj);
        case LBR_ACT_GELU: return mlp_launcher_act<LBR_ACT_GELU>(oproj);
        default: return mlp_launcher_act<LBR_ACT_SILU>(oproj);
    }
}

bool mlp_proj_ok(long long D, long long H, long long K0, long long hd) {
    return D <= 16 * 4 * MLP_OB && K0 % 16 == 0 && K0 / 16 <= MLP_OC && hd % 4 == 0 && K0 % hd == 0 &&
           mlp_lds_bytes(D, H, true) + 2 * MLP_WMAX * sizeof(float) <= MLP_LDS_MAX;
}
