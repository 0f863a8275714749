// attention.hip — fused attention on the gfx950 matrix cores.
//
// Replaces kernel_attention / kernel_attention_flash (csrc/ops/attn.c:26-253)
// behind ATTENTION (csrc/executor.c:371-397):
//   O[bh] = softmax(Q[bh]·K[kv]ᵀ · 1/√hd  (+ mask[bh])  (causal: −∞ above the
//           diagonal)) · V[kv],      kv = bh / group_size   (attn.c:73, 247)
// Q, K, V, O are [batch·heads, S, hd] contiguous.  extras
// [seq_len, head_dim, causal, has_mask, group_size] (runtime/ops.py:257-262);
// inputs [Q, K, V, scratch] or [Q, K, V, mask, scratch].  The planner's
// scratch slot is not needed: the online-softmax state lives in registers.
//
// Single-pass online-softmax kernels serve every sequence length (the
// reference's S ≤ 256 / mask path and its flash path compute the same
// function).  Layout choice: they compute Sᵀ = K·Qᵀ and Oᵀ = Vᵀ·Pᵀ, so in both
// accumulators a lane owns one query row: the running max / sum and the
// rescale of O are per-lane scalars, and the exponentiated scores are fed
// straight back as the B operand of the P·V product without leaving
// registers.
//
// * attn_fwd_mfma16 (hd ≤ 128, the main path): v_mfma_f32_16x16x4_f32,
//   8 wavefronts × 16 query rows = 128 rows per workgroup; a row's scores are
//   spread over 4 lanes (exchanged with permlane swaps).  Interior key tiles
//   run without mask code, the softmax reference max moves only in steps of
//   more than 2^8, and the row sum is reduced once at the end.  Causal grids
//   fold query blocks in pairs; small grids split the key range
//   (attn_fwd_mfma16_split + attn_split_merge).
// * attn_fwd_mfma (128 < hd ≤ 256): v_mfma_f32_32x32x2_f32, 4 wavefronts × 32
//   query rows, a row's scores in 2 lanes (lane l ↔ l^32).
// * attn_fwd_rows (hd % 8 != 0): one workgroup per query row, scores in LDS.
//
// K/V tiles of 32 keys are staged in LDS (zero-filled past S and past hd);
// the next tile is fetched into registers while the current one is consumed
// from LDS, so global-load latency hides behind the MFMAs.  Exponentials use
// the hardware v_exp_f32 (exp2; a denormal result flushes to zero, which
// cannot change a softmax row that always contains a term equal to 1).
// Causal: tiles entirely above a wavefront's rows are skipped; workgroups are
// issued heaviest-first (last query block first) to balance the triangle.
#include "lbr_device.h"

#include <float.h>
#include <math.h>

#include <algorithm>
#include <array>
#include <map>
#include <mutex>
#include <string>
#include <vector>

// attn_fwd_kq's workgroup assignment (defined with the host code below) and how
// many of its workgroups one CU holds at once.
const std::vector<unsigned short>& kq_plan(long long bh, int S, bool causal, int C, int per_cu);
int kq_per_cu(int dp);

namespace {

constexpr int AT_NT = 256;       // 4 waves
constexpr int AT_QB = 128;       // query rows per workgroup
constexpr int AT_KB = 32;        // keys per LDS tile (one 32-row MFMA block)
constexpr float LOG2E = 1.4426950408889634f;

struct AttnArgs {
    const float* Q;
    const float* K;
    const float* V;
    float* O;
    const float* mask;
    int S, D, group_size, n_qblocks;
    float scale_log2;            // (1/√hd)·log2(e)
    int fold;                    // causal: workgroup j also runs query block j (16x16 kernel)
    // Key-range split (16x16 kernel, small grids): the key tiles of all
    // (head, query block) pairs, numbered head-major then block then tile,
    // are cut into sk_wg contiguous equal shares, one per workgroup.
    int sk_wg;                   // workgroups of the split grid (0: no split)
    int sk_maxseg;               // partial slots per (head, query block)
    int sk_tiles;                // key tiles of all heads (sk_wg · sk_tiles < 2³¹)
    int sk_head_tiles;           // key tiles of one head
    // divisions by sk_wg, sk_tiles and sk_head_tiles as multiply-high and
    // shift (lbr_fdiv): the share and segment arithmetic stays in a few
    // scalar instructions instead of 64-bit division routines
    int sk_wg_m, sk_wg_s, sk_tiles_m, sk_tiles_s, sk_ht_m, sk_ht_s;
    float* part;                 // split partials Σ p·V: [bh][query block][sk_maxseg][128 rows][D]
    float* ml;                   // split running max and Σ p, same slots: [..][128 rows][2]
    int sk_defer;                // 1: every block's rows go through the workspace and
                                 // attn_split_merge writes all of O, after the split kernel
                                 // has read Q, K and V (O may then lie over them)
    int o_heads;                 // 0: O is [bh, S, D]; H > 0: O is [B, S, H, D] (fused transpose)
    // V read from the columns of a row-major [B·S, v_ld] tensor (16x16 kernel, fused
    // SLICE → TRANSPOSE): row s of K/V head b·v_heads + h at V + (b·S + s)·v_ld + h·D.
    // v_ld = 0: V is [kv heads, S, D] like K.
    long long v_ld;
    int v_heads;
    // 16-row key-quartered kernel (attn_fwd_kq): query blocks of 16 rows, kq_nq per head;
    // k_frag: K is stored fragment-major (lbr_frag_offset) by the GEMM that wrote it
    int kq_nq, kq_bh;
    int k_frag;
};

// Row q of head bh in the output: [bh][S][D], or [B][S][H][D] when the
// following TRANSPOSE(1, 2) is fused (16x16 kernel only).
__device__ __forceinline__ float* attn_out_row(const AttnArgs& g, long long bh, long long q) {
    if (g.o_heads) {
        const long long b = bh / g.o_heads, h = bh - b * g.o_heads;
        return g.O + ((b * g.S + q) * g.o_heads + h) * (long long)g.D;
    }
    return g.O + (bh * g.S + q) * (long long)g.D;
}

// One K/V tile (AT_KB keys × DP) staged through registers: thread t holds the
// float4 granules idx = t + i·AT_NT of each tile in row-major order.  Keys
// past S and columns past D read as zero.
template <int DP>
struct AttnStage {
    static constexpr int PER = AT_KB * DP / 4 / AT_NT;
    float4 k[PER];
    float4 v[PER];
};

template <int DP>
__device__ __forceinline__ void attn_load_tile(const float* __restrict__ Kb, const float* __restrict__ Vb, int k0,
                                               int S, int D, AttnStage<DP>& st) {
#pragma unroll
    for (int i = 0; i < AttnStage<DP>::PER; ++i) {
        const int idx = threadIdx.x + i * AT_NT;
        const int r = idx / (DP / 4), d = (idx % (DP / 4)) * 4;
        const bool ok = k0 + r < S && d < D;
        const long long off = (long long)(k0 + r) * D + d;
        st.k[i] = ok ? *reinterpret_cast<const float4*>(Kb + off) : make_float4(0.f, 0.f, 0.f, 0.f);
        st.v[i] = ok ? *reinterpret_cast<const float4*>(Vb + off) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int DP>
__device__ __forceinline__ void attn_store_tile(float (*Ks)[DP + 4], float (*Vs)[DP + 4], const AttnStage<DP>& st) {
#pragma unroll
    for (int i = 0; i < AttnStage<DP>::PER; ++i) {
        const int idx = threadIdx.x + i * AT_NT;
        const int r = idx / (DP / 4), d = (idx % (DP / 4)) * 4;
        *reinterpret_cast<float4*>(&Ks[r][d]) = st.k[i];
        *reinterpret_cast<float4*>(&Vs[r][d]) = st.v[i];
    }
}

template <int DP, bool CAUSAL, bool HAS_MASK>
__global__ __launch_bounds__(AT_NT, DP >= 256 ? 1 : 2) void attn_fwd_mfma(AttnArgs g) {
    constexpr int NCH = DP / 8;      // 8-wide d chunks
    constexpr int NDB = DP / 32;     // 32-wide d blocks of Oᵀ
    __shared__ float Ks[AT_KB][DP + 4];
    __shared__ float Vs[AT_KB][DP + 4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane & 31, lh = lane >> 5;
    const int qblk = CAUSAL ? (g.n_qblocks - 1 - (int)blockIdx.x) : (int)blockIdx.x;
    const long long bh = blockIdx.y;
    const long long kvh = bh / g.group_size;
    const int S = g.S, D = g.D;
    const float* __restrict__ Qb = g.Q + bh * (long long)S * D;
    const float* __restrict__ Kb = g.K + kvh * (long long)S * D;
    const float* __restrict__ Vb = g.V + kvh * (long long)S * D;
    const int q_wave0 = qblk * AT_QB + wave * 32;
    const int q = q_wave0 + lq;            // this lane's query row

    // Q fragment, pre-scaled by log2(e)/√hd: lane holds Q[q][8c + 4h + 0..3]
    floatx4 qf[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int d = c * 8 + lh * 4;
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (q < S && d < D) {
            const float4 t = *reinterpret_cast<const float4*>(Qb + (long long)q * D + d);
            v[0] = t.x * g.scale_log2;
            v[1] = t.y * g.scale_log2;
            v[2] = t.z * g.scale_log2;
            v[3] = t.w * g.scale_log2;
        }
        qf[c] = v;
    }

    floatx16 oacc[NDB];
#pragma unroll
    for (int b = 0; b < NDB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[b][r] = 0.f;
    float m_run = -FLT_MAX, l_run = 0.f;

    int n_tiles = (S + AT_KB - 1) / AT_KB;
    if (CAUSAL) n_tiles = min(n_tiles, min(S - 1, qblk * AT_QB + AT_QB - 1) / AT_KB + 1);

    AttnStage<DP> st;
    attn_load_tile<DP>(Kb, Vb, 0, S, D, st);
    attn_store_tile<DP>(Ks, Vs, st);
    __syncthreads();

    for (int kt = 0; kt < n_tiles; ++kt) {
        const int k0 = kt * AT_KB;
        // next tile's global loads are in flight while this one is consumed from LDS
        if (kt + 1 < n_tiles) attn_load_tile<DP>(Kb, Vb, k0 + AT_KB, S, D, st);

        // Causal: a tile whose first key is past this wave's last row contributes nothing.
        if (!CAUSAL || k0 <= q_wave0 + 31) {
            // Sᵀ[kv][q] for the tile's 32 keys (already scaled by log2 e / √hd)
            floatx16 sacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const floatx4 kf = *reinterpret_cast<const floatx4*>(&Ks[lq][c * 8 + lh * 4]);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[i], qf[c][i], sacc, 0, 0, 0);
            }

            // mask / causal / tail, then the tile's row max
            float tmax = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kv = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
                float sv = sacc[r];
                if (HAS_MASK && kv < S && q < S) sv += g.mask[(bh * S + q) * (long long)S + kv] * LOG2E;
                if (kv >= S || (CAUSAL && kv > q)) sv = -INFINITY;
                sacc[r] = sv;
                tmax = fmaxf(tmax, sv);
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float m_new = fmaxf(m_run, tmax);
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
            float psum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(sacc[r] - m_new);
                sacc[r] = p;
                psum += p;
            }
            psum += __shfl_xor(psum, 32, 64);
            l_run = l_run * corr + psum;
            m_run = m_new;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[db][r] *= corr;

            // Oᵀ[d][q] += Σ_kv V[kv][d] · P[q][kv]
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kvl = 8 * (r >> 2) + 4 * lh + (r & 3);
#pragma unroll
                for (int db = 0; db < NDB; ++db)
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[kvl][db * 32 + lq], sacc[r], oacc[db], 0,
                                                                   0, 0);
            }
        }
        __syncthreads();
        if (kt + 1 < n_tiles) {
            attn_store_tile<DP>(Ks, Vs, st);
            __syncthreads();
        }
    }

    // O[q][d] = Oᵀ[d][q] / l ; lane holds d = 32·db + 8·j + 4·h + (0..3)
    if (q < S) {
        const float inv_l = 1.0f / l_run;
        float* __restrict__ Ob = g.O + bh * (long long)S * D + (long long)q * D;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = db * 32 + 8 * j + 4 * lh;
                if (d < D) {
                    float4 o;
                    o.x = oacc[db][4 * j + 0] * inv_l;
                    o.y = oacc[db][4 * j + 1] * inv_l;
                    o.z = oacc[db][4 * j + 2] * inv_l;
                    o.w = oacc[db][4 * j + 3] * inv_l;
                    *reinterpret_cast<float4*>(Ob + d) = o;
                }
            }
    }
}

// ---------------------------------------------------------------------------
// Head dims ≤ 128: v_mfma_f32_16x16x4_f32 with 16 query rows per wavefront.
//
// Same transposed formulation (Sᵀ = K·Qᵀ, Oᵀ = Vᵀ·Pᵀ, lane owns query row
// l%16), but the 16-row wavefront tile halves the per-wave register state
// (Q: hd/4, O: hd/4, scores: 8 VGPRs), so an 8-wavefront workgroup of 128
// query rows runs at 4 wavefronts per SIMD and the matrix core has twice as
// many independent instruction streams to hide LDS and softmax latency.
// Operand layout of the 16x16x4 MFMA: A[i][k] from lane 16k+i, B[k][j] from
// lane 16k+j, D[4g+r][j] in register r of lane 16g+j.  K-chunks of 16 d:
// lane group g reads K/Q[.][16c+4g .. +3] as one float4; MFMA i of the chunk
// reduces d = 16c+4g+i over the four groups.
// In Oᵀ = Vᵀ·Pᵀ the row index i of d-block db stands for head dim
//   d(db, i) = W·i + db%W + 16W·(db/W),   W = min(4, hd/16),
// so one lane's V operands for the W blocks db = W·h .. W·h+W-1 are the W
// consecutive floats V[key][16W·h + W·i ..] — one LDS vector read feeds W
// MFMAs — and one lane's outputs O[q][..] are runs of 4W consecutive floats.
// LDS rows are padded to hd+4 floats: the K reads (16 rows × 4 groups of
// 16 B) and the V reads (4 rows × 16 lanes × W consecutive floats) hit
// distinct banks.
// Cross-row all-reduce of lanes l, l^16 and l^32 through the gfx950 row
// swaps (v_permlane16_swap / v_permlane32_swap: VALU, no LDS round trip).
// swap(x, x) returns the pair {x[l], x[l^16]} (resp. l^32) in some order;
// max and + are commutative, so the result equals the shuffle reduction.
__device__ __forceinline__ float rows4_max(float x) {
    const unsigned u = __float_as_uint(x);
    auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const unsigned v = __float_as_uint(x);
    auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows4_sum(float x) {
    const unsigned u = __float_as_uint(x);
    auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const unsigned v = __float_as_uint(x);
    auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

constexpr int A16_NT = 512;      // 8 waves
constexpr int A16_QB = 128;      // query rows per workgroup (16 per wave)
constexpr int A16_KB = 32;       // keys per tile
// The softmax reference max moves only when a score exceeds it by more than
// this (log2 units), so every exponentiated score stays ≤ 2^8.
constexpr float ATTN_LAZY = 8.0f;

template <bool B>
struct BoolTag {
    static constexpr bool value = B;
};

// Key tiles query block `qblk` needs: all of them, or (causal) up to the one
// holding its last row's diagonal.
__device__ __forceinline__ int attn16_tiles(const AttnArgs& g, int qblk, bool causal, int qb = A16_QB) {
    const int nt = (g.S + A16_KB - 1) / A16_KB;
    return causal ? min(nt, min(g.S - 1, qblk * qb + qb - 1) / A16_KB + 1) : nt;
}

// One query block (16·NWQ rows, NWQ wavefronts of 16) of one head over key
// tiles [t0, t1): streams them through Ks/Vs.  slot < 0: the range is the
// whole row, write O (or, deferred, stage the row in the workspace for
// attn_kq_flush).  slot >= 0: write the unnormalised partial (Σ p·V, running
// max m, Σ p) of this key range to the split workspace for attn_split_merge.
template <int DP, bool CAUSAL, bool HAS_MASK, bool SPLIT, bool DB = SPLIT, int NWQ = 8>
__device__ __forceinline__ void attn16_qblock(const AttnArgs& g, int bhi, int qblk, int t0_, int t1, long long slot,
                                              float (*Ks)[DP + 4], float (*Vs)[DP + 4]) {
    constexpr int NCH = DP / 16;     // 16-wide d chunks (S reduction) and d blocks (O)
    constexpr int W = NCH < 4 ? NCH : 4;
    typedef float VW __attribute__((ext_vector_type(W)));
    constexpr int NT = 64 * NWQ, QB = 16 * NWQ;                  // threads, query rows
    static_assert(!SPLIT || NWQ == 8, "the split's partial slots hold 128 rows");
    constexpr int TILE4 = A16_KB * DP / 4;                       // float4 granules per K (or V) tile
    constexpr int PER = (TILE4 + NT - 1) / NT;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    // the caller passes the head; without a split the range starts at tile 0
    const long long bh = bhi;
    const int t0 = SPLIT ? t0_ : 0;
    const long long kvh = bh / g.group_size;
    const int S = g.S, D = g.D;
    const float* __restrict__ Qb = g.Q + bh * (long long)S * D;
    const float* __restrict__ Kb = g.K + kvh * (long long)S * D;
    const float* __restrict__ Vb = g.V + kvh * (long long)S * D;
    long long vst = D;                                           // V row stride
    if (g.v_ld) {
        const long long b = kvh / g.v_heads;
        Vb = g.V + b * S * g.v_ld + (kvh - b * g.v_heads) * D;
        vst = g.v_ld;
    }
    const int q_wave0 = qblk * QB + wave * 16;
    const int q = q_wave0 + lr;

    floatx4 qf[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int d = 16 * c + 4 * lg;
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (q < S && d < D) {
            const float4 t = *reinterpret_cast<const float4*>(Qb + (long long)q * D + d);
            v[0] = t.x * g.scale_log2;
            v[1] = t.y * g.scale_log2;
            v[2] = t.z * g.scale_log2;
            v[3] = t.w * g.scale_log2;
        }
        qf[c] = v;
    }

    floatx4 oacc[NCH];
#pragma unroll
    for (int b = 0; b < NCH; ++b) oacc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
    // m_run: the reference max of this lane's row (the same in the row's 4 lanes);
    // l_part: Σ 2^(s − m_run) over the keys this lane holds (4g + r, 16 + 4g + r of
    // each tile) — the row sum is the total over the 4 lanes, taken once at the end
    float m_run = -FLT_MAX, l_part = 0.f;

    // Tiles [t0, t_fast) lie wholly inside S and, causal, at or below the block's
    // first row, and the head dim fills DP: no bounds, causal or padding test.
    int t_fast = t0;
    if (!HAS_MASK && D == DP) {
        int e = S / A16_KB;
        if (CAUSAL) e = min(e, (qblk * QB + 1) / A16_KB);
        t_fast = max(t0, min(t1, e));
    }

    float4 kr[PER], vr[PER];
    auto load = [&](int k0, auto checked_tag) {
        constexpr bool CHECKED = decltype(checked_tag)::value;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + i * NT;
            const int r = idx / (DP / 4), d = (idx % (DP / 4)) * 4;
            const long long voff = (long long)(k0 + r) * vst + d;
            if (CHECKED) {
                const bool ok = idx < TILE4 && k0 + r < S && d < D;
                const long long off = (long long)(k0 + r) * D + d;
                kr[i] = ok ? *reinterpret_cast<const float4*>(Kb + off) : make_float4(0.f, 0.f, 0.f, 0.f);
                vr[i] = ok ? *reinterpret_cast<const float4*>(Vb + voff) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else if (TILE4 % NT == 0 || idx < TILE4) {
                // D == DP: granule idx of the K tile is float offset 4·idx from row k0
                const long long off = (long long)k0 * DP + 4 * idx;
                kr[i] = *reinterpret_cast<const float4*>(Kb + off);
                vr[i] = *reinterpret_cast<const float4*>(Vb + voff);
            }
        }
    };
    // DB (the split kernel): Ks and Vs hold two tiles, the one being read and
    // the next one being stored, so a tile ends with one barrier, not two
    int cur = 0;
    auto store = [&](int buf) {
        float (*Kd)[DP + 4] = Ks + buf * A16_KB;
        float (*Vd)[DP + 4] = Vs + buf * A16_KB;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + i * NT;
            if (idx < TILE4) {
                const int r = idx / (DP / 4), d = (idx % (DP / 4)) * 4;
                *reinterpret_cast<float4*>(&Kd[r][d]) = kr[i];
                *reinterpret_cast<float4*>(&Vd[r][d]) = vr[i];
            }
        }
    };

    if (t0 < t_fast) load(t0 * A16_KB, BoolTag<false>());
    else load(t0 * A16_KB, BoolTag<true>());
    store(0);
    __syncthreads();

    // One key tile.  The scores are exponentiated against m_run, which moves only
    // when some lane's tile max exceeds it by more than ATTN_LAZY (log2 units):
    // then the row max is taken across the row's 4 lanes, and O and l_part are
    // rescaled.  Otherwise every p = 2^(s − m_run) ≤ 2^ATTN_LAZY and the
    // softmax step is 8 exponentials and 8 adds, with no cross-lane work.
    // MASKED tiles apply the bounds, causal and additive-mask terms per score.
    // PCHECK: the prefetched next tile needs the bounds-checked load.
    auto tile = [&](int kt, auto masked_tag, auto pcheck_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        const int k0 = kt * A16_KB;
        if (kt + 1 < t1) load(k0 + A16_KB, pcheck_tag);
        const float (*Kc)[DP + 4] = Ks + cur * A16_KB;
        const float (*Vc)[DP + 4] = Vs + cur * A16_KB;

        if (!MASKED || !CAUSAL || k0 <= q_wave0 + 15) {
            // Sᵀ for two 16-key blocks; register r of block b = key k0 + 16b + 4g + r
            floatx4 sacc[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                sacc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    const floatx4 kf = *reinterpret_cast<const floatx4*>(&Kc[16 * b + lr][16 * c + 4 * lg]);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        sacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[i], qf[c][i], sacc[b], 0, 0, 0);
                }
            }

            float tmax = -INFINITY;
            if (MASKED) {
                // a tile wholly inside S and (causal) at or below this wave's first row
                // needs no per-score bounds or causal test (wave-uniform)
                const bool inner = k0 + A16_KB <= S && (!CAUSAL || k0 + A16_KB - 1 <= q_wave0);
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int kv = k0 + 16 * b + 4 * lg + r;
                        float sv = sacc[b][r];
                        if (HAS_MASK && kv < S && q < S) sv += g.mask[(bh * S + q) * (long long)S + kv] * LOG2E;
                        if (!inner && (kv >= S || (CAUSAL && kv > q))) sv = -INFINITY;
                        sacc[b][r] = sv;
                        tmax = fmaxf(tmax, sv);
                    }
            } else {
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sacc[b][r]);
            }
            if (__any(tmax > m_run + ATTN_LAZY)) {
                const float m_new = fmaxf(m_run, rows4_max(tmax));
                const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
                for (int db = 0; db < NCH; ++db) oacc[db] *= corr;
                l_part *= corr;
                m_run = m_new;
            }
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = __builtin_amdgcn_exp2f(sacc[b][r] - m_run);
                    sacc[b][r] = p;
                    l_part += p;
                }

            // Oᵀ[d][q] += Σ_kv V[kv][d]·P[q][kv]; MFMA (b, r) takes key 16b + 4g + r from group g
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kvl = 16 * b + 4 * lg + r;
#pragma unroll
                    for (int h = 0; h < NCH / W; ++h) {
                        const VW vv = *reinterpret_cast<const VW*>(&Vc[kvl][16 * W * h + W * lr]);
#pragma unroll
                        for (int w = 0; w < W; ++w)
                            oacc[W * h + w] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[w], sacc[b][r], oacc[W * h + w],
                                                                                  0, 0, 0);
                    }
                }
        }
        if (DB) {
            if (kt + 1 < t1) store(cur ^ 1);
            __syncthreads();   // the next tile is stored, and no wave still reads this one
            cur ^= 1;
        } else {
            __syncthreads();
            if (kt + 1 < t1) {
                store(0);
                __syncthreads();
            }
        }
    };
    int kt = t0;
    for (; kt + 1 < t_fast; ++kt) tile(kt, BoolTag<false>(), BoolTag<false>());
    if (kt < t_fast) tile(kt++, BoolTag<false>(), BoolTag<true>());
    for (; kt < t1; ++kt) tile(kt, BoolTag<true>(), BoolTag<true>());
    const float l_run = rows4_sum(l_part);

    // O[q][d] = Oᵀ[d][q] / l; register r of block W·h + w holds row i = 4g + r,
    // i.e. d = 16W·h + W·(4g + r) + w: W consecutive floats per (h, r)
    if (q < S) {
        const bool part = SPLIT && slot >= 0;
        const long long prow = slot * A16_QB + (q - qblk * A16_QB);   // partial row in the workspace
        const float inv_l = part ? 1.0f : 1.0f / l_run;
        // a deferred unsplit block stages its rows as [bh, S, D] for attn_kq_flush
        float* __restrict__ Ob = part ? g.part + prow * D
                                      : (!SPLIT && g.sk_defer) ? g.part + (bh * S + q) * (long long)D
                                                               : attn_out_row(g, bh, q);
        if (part && lg == 0) {
            g.ml[2 * prow] = m_run;
            g.ml[2 * prow + 1] = l_run;
        }
#pragma unroll
        for (int h = 0; h < NCH / W; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 16 * W * h + W * (4 * lg + r);
                if (d < D) {
                    VW o;
#pragma unroll
                    for (int w = 0; w < W; ++w) o[w] = oacc[W * h + w][r] * inv_l;
                    *reinterpret_cast<VW*>(Ob + d) = o;
                }
            }
    }
}

// Causal work per query block grows linearly with its index, and the
// hardware places consecutive workgroups round-robin over the CUs, so a
// one-block-per-workgroup grid leaves some CUs with only the longest blocks.
// With g.fold set, workgroup j runs block n-1-j and then block j: every
// workgroup carries the same number of key tiles.
//
// Key-range split (g.sk_wg > 0, small grids): the key tiles of every (head,
// query block) pair in order — head, then block 0 .. n-1, then tile — form
// one sequence of sk_tiles tiles; workgroup w takes tiles
// [sk_bound(w), sk_bound(w+1)), an equal share, so every CU carries the same
// number of tiles whatever the causal block lengths.  A query block inside
// one share writes O; a block cut by share boundaries is computed in
// segments, segment j by the j-th workgroup that touches it, each writing
// its partial to slot (head, block, j) for attn_split_merge.

// First tile of workgroup w's share (sk_bound(sk_wg) = sk_tiles).
__device__ __forceinline__ int sk_bound(const AttnArgs& g, int w) {
    return (int)lbr_fdiv((unsigned)(w * g.sk_tiles), g.sk_wg_m, g.sk_wg_s);
}

// Workgroup whose share holds tile G.
__device__ __forceinline__ int sk_owner(const AttnArgs& g, int G) {
    int w = (int)lbr_fdiv((unsigned)(G * g.sk_wg), g.sk_tiles_m, g.sk_tiles_s);
    while (w + 1 < g.sk_wg && sk_bound(g, w + 1) <= G) ++w;
    while (w > 0 && sk_bound(g, w) > G) --w;
    return w;
}

// First tile of query block qb within its head.
__device__ __forceinline__ int sk_block_start(const AttnArgs& g, int qb, bool causal) {
    int t = 0;
    for (int b = 0; b < qb; ++b) t += attn16_tiles(g, b, causal);
    return t;
}

// NWQ = 8: 128-row blocks, a few workgroups a CU.  NWQ = 4: 64-row blocks,
// folded, for causal grids the 128-row fold leaves short of one workgroup a CU
// (Qwen3-4B S1024: 32 heads × 8 pairs of 64-row blocks = 256 workgroups, one a
// CU with equal work, where 128-row blocks give 128 pairs or a key-range
// split and its merge); one workgroup a CU holds two K/V tiles in LDS, so a
// tile ends with one barrier.
// NWQ = 4 runs a one-dimensional grid of (head, block) pairs numbered head-major,
// remapped so that XCD x (workgroups w ≡ x mod 8) takes the contiguous x-th eighth:
// whole heads, so a GQA group's K/V rows stay in that XCD's L2 (Qwen3-4B: 4 query
// heads, one K/V head of 1 MB, per XCD) instead of every XCD streaming all of them.
template <int DP, bool CAUSAL, bool HAS_MASK, int NWQ = 8>
__global__ __launch_bounds__(64 * NWQ, NWQ == 8 ? 4 : 1) void attn_fwd_mfma16(AttnArgs g) {
    constexpr bool DB = NWQ == 4;
    constexpr int QB = 16 * NWQ;
    __shared__ float Ks[(DB ? 2 : 1) * A16_KB][DP + 4];
    __shared__ float Vs[(DB ? 2 : 1) * A16_KB][DP + 4];
    int j = blockIdx.x, bh = blockIdx.y;
    if (NWQ == 4) {
        const int per_head = g.fold ? (g.n_qblocks + 1) / 2 : g.n_qblocks;
        const int total = gridDim.x, w = blockIdx.x;
        const int t = total % 8 == 0 ? (w % 8) * (total / 8) + w / 8 : w;
        bh = t / per_head;
        j = t - bh * per_head;
    }
    const int last = g.n_qblocks - 1 - j;
    if (!CAUSAL) {
        attn16_qblock<DP, CAUSAL, HAS_MASK, false, DB, NWQ>(g, bh, j, 0, attn16_tiles(g, j, false, QB), -1, Ks, Vs);
        return;
    }
    attn16_qblock<DP, CAUSAL, HAS_MASK, false, DB, NWQ>(g, bh, last, 0, attn16_tiles(g, last, true, QB), -1, Ks, Vs);
    if (g.fold && j < last) {   // folded second block: query block j
        __syncthreads();
        attn16_qblock<DP, CAUSAL, HAS_MASK, false, DB, NWQ>(g, bh, j, 0, attn16_tiles(g, j, true, QB), -1, Ks, Vs);
    }
}

template <int DP, bool CAUSAL, bool HAS_MASK>
__global__ __launch_bounds__(A16_NT, 4) void attn_fwd_mfma16_split(AttnArgs g) {
    __shared__ float Ks[2 * A16_KB][DP + 4];
    __shared__ float Vs[2 * A16_KB][DP + 4];
    const int w = blockIdx.x;
    const int end = sk_bound(g, w + 1);
    int G = sk_bound(g, w);
    while (G < end) {
        const int bh = (int)lbr_fdiv((unsigned)G, g.sk_ht_m, g.sk_ht_s);
        int t0 = G - bh * g.sk_head_tiles;
        int qb = 0, nt = attn16_tiles(g, 0, CAUSAL);
        while (t0 >= nt) {
            t0 -= nt;
            nt = attn16_tiles(g, ++qb, CAUSAL);
        }
        const int t1 = min(nt, t0 + (end - G));
        // a block cut by a share boundary (or any block, deferred): segment index = this
        // workgroup − the owner of its first tile
        const long long slot = (g.sk_defer || t0 > 0 || t1 < nt)
                                   ? ((long long)bh * g.n_qblocks + qb) * g.sk_maxseg + (w - sk_owner(g, G - t0))
                                   : -1;
        attn16_qblock<DP, CAUSAL, HAS_MASK, true>(g, bh, qb, t0, t1, slot, Ks, Vs);
        G += t1 - t0;
    }
}

// ---------------------------------------------------------------------------
// Small grids: 16 query rows per workgroup, the key tiles dealt four ways.
//
// With one 16-row wavefront per query block, the last rows of a causal head
// are a serial chain of S/32 key tiles on one SIMD (S = 1024, hd = 64: 32
// tiles × 64 MFMAs × 32 cycles ≈ 30 µs) however the grid is cut.  Here the
// four wavefronts of a workgroup hold the same 16 query rows and take every
// fourth key tile (tile t → wavefront t mod 4, which also spreads the causal
// diagonal), each with its own running max, sum and O.  At the end the four
// partial rows meet in LDS and are combined in wavefront order:
//   O = Σ_w 2^(m_w − M)·O_w / Σ_w 2^(m_w − M)·l_w,   M = max_w m_w.
// No partial leaves the workgroup and no merge kernel runs.  Nothing is
// shared between the wavefronts, so K and V go from global memory (L2)
// straight into registers, in the MFMA operand layouts of attn16_qblock; the
// next tile's K is requested as soon as the current scores are formed and its
// V as soon as P·V has been issued.  Rows past S read as zero through the
// buffer views' range check (their scores are masked and their p is 0).
// Head dims 32, 64 and 128 only (D == DP: no padded columns).
//
// Grid: one workgroup per (head, 16-row block), all resident at once (a few
// per CU).  The hardware hands workgroup w to CU w mod C (C CUs; XCD w mod 8),
// so workgroups w, w + C, w + 2C ... share a CU and its SIMDs, and a CU's time
// is the sum of its blocks' key tiles.  The host assigns the blocks (kq_plan):
// heaviest first, each to the least-loaded CU of the XCD that holds its head
// (whole heads, or alternate blocks of them, per XCD, so that the K/V rows a
// workgroup streams stay in that XCD's L2), and passes the assignment in the
// kernel arguments.  Without one (more blocks than fit at once) workgroup w
// runs block levels from the heaviest down.
constexpr int KQ_WAVES = 4;
constexpr int KQ_NT = 64 * KQ_WAVES;
constexpr int KQ_QB = 16;        // query rows per workgroup
constexpr int KQ_MAP_MAX = 1536; // blocks a kernel-argument assignment holds (3 KiB)

struct KqArgs {
    AttnArgs g;
    int n_map;                           // 0: no assignment (heaviest block level first)
    unsigned short map[KQ_MAP_MAX];      // workgroup → block index head·kq_nq + block
};

__host__ __device__ __forceinline__ void kq_item(const KqArgs& k, int w, int* bh, int* qblk) {
    const int nq = k.g.kq_nq;
    int it;
    if (k.n_map) {
        it = k.map[w];
    } else {
        const int level = w / k.g.kq_bh;
        it = (w - level * k.g.kq_bh) * nq + (nq - 1 - level);
    }
    *bh = it / nq;
    *qblk = it - *bh * nq;
}

template <int DP, bool CAUSAL, bool HAS_MASK>
__global__ __launch_bounds__(KQ_NT, 2) void attn_fwd_kq(KqArgs k) {
    const AttnArgs& g = k.g;
    constexpr int NCH = DP / 16;     // 16-wide d chunks (S reduction) and d blocks (O)
    constexpr int W = NCH < 4 ? NCH : 4;
    constexpr int NH = NCH / W;
    typedef float VW __attribute__((ext_vector_type(W)));
    __shared__ float o_sh[KQ_WAVES][KQ_QB][DP + 4];
    __shared__ float m_sh[KQ_WAVES][KQ_QB];
    __shared__ float l_sh[KQ_WAVES][KQ_QB];

    // the wavefront index as a scalar: the key tiles, their offsets and the loop are uniform
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    int bhi, qblk;
    kq_item(k, blockIdx.x, &bhi, &qblk);
    const long long bh = bhi, kvh = bh / g.group_size;
    const int S = g.S, D = g.D;
    const float* Qb = g.Q + bh * (long long)S * DP;
    const float* Kb = g.K + kvh * (long long)S * DP;
    const float* Vb = g.V + kvh * (long long)S * DP;
    unsigned vst = DP;                                           // V row stride (floats)
    if (g.v_ld) {
        const long long b = kvh / g.v_heads;
        Vb = g.V + b * S * g.v_ld + (kvh - b * g.v_heads) * DP;
        vst = (unsigned)g.v_ld;
    }
    // Buffer views of this head's Q, K and V rows (byte offsets < 2^32, checked by the
    // host): every load below is a fixed per-lane offset plus a uniform one, and rows past
    // S fall outside the view and read as zero.
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)Qb, (short)0, S * DP * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)Kb, (short)0, S * DP * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)Vb, (short)0, (int)(((S - 1) * vst + DP) * 4u), 0x00020000);
    const int q0 = qblk * KQ_QB, q = q0 + lr;

    // Q rows, pre-scaled (rows past S read zero; their lanes are never stored, and a lane's
    // scores, max and sum never mix with another row's): all loads, then one wait
    floatx4 qf[NCH];

    const int nt = (S + A16_KB - 1) / A16_KB;
    const int T = CAUSAL ? min(nt, min(S - 1, q0 + KQ_QB - 1) / A16_KB + 1) : nt;
    // tiles [0, t_fast) lie wholly inside S and (causal) at or below the block's first row:
    // no per-score test; with 16-row blocks only the last tile can need one
    int t_fast = HAS_MASK ? 0 : S / A16_KB;
    if (CAUSAL) t_fast = min(t_fast, (q0 + 1) / A16_KB);

    floatx4 kf[2][NCH];
    VW vf[2][4][NH];
    // K rows 32t + 16b + lr, d 16c + 4lg .. +3 (A operand of Sᵀ = K·Qᵀ). Row-major, one
    // load instruction reads 64 of the 128 bytes of 16 lines; fragment-major
    // (lbr_frag_offset), 1 KiB of 8 whole lines, which halves the L2 requests for K.
    const unsigned ko = g.k_frag ? (unsigned)(lr * 16 + 4 * lg) * 4u : (unsigned)(lr * DP + 4 * lg) * 4u;
    const unsigned kcs = g.k_frag ? 1024u : 64u;
    auto load_k = [&](int t) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const unsigned so = (unsigned)((t * A16_KB + 16 * b) * DP) * 4u;
#pragma unroll
            for (int c = 0; c < NCH; ++c)
                kf[b][c] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rk, ko + kcs * c, so, 0));
        }
    };
    // V rows 32t + 16b + 4lg + rr, d 16W·h + W·lr .. +W−1 (A operand of Oᵀ = Vᵀ·Pᵀ)
    const unsigned vo = (4 * lg * vst + W * lr) * 4u;
    auto load_v = [&](int t) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const unsigned so = (unsigned)(t * A16_KB + 16 * b + rr) * vst * 4u;
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    if constexpr (W == 4)
                        vf[b][rr][h] = __builtin_bit_cast(
                            VW, __builtin_amdgcn_raw_buffer_load_b128(rv, vo + 64 * W * h, so, 0));
                    else
                        vf[b][rr][h] = __builtin_bit_cast(
                            VW, __builtin_amdgcn_raw_buffer_load_b64(rv, vo + 64 * W * h, so, 0));
                }
            }
    };

    floatx4 oacc[NCH];
#pragma unroll
    for (int b = 0; b < NCH; ++b) oacc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
    // m_run: reference max of this lane's row (the same in the row's 4 lanes); l_part: Σ p
    // over the keys this lane holds — the row sum is the total over the 4 lanes
    float m_run = -FLT_MAX, l_part = 0.f;

    // This wavefront's tiles t = wave, wave + 4, ...: K of the next tile is fetched once the
    // current scores are formed, V once the current P·V is issued.  (Issuing the next
    // tile's scores before the current P·V, to run the softmax under the P·V MFMAs,
    // measured slower: GPT-2 S1024 25.3 → 27.5 µs.)
    int t = wave;
    {
        // Q rows, pre-scaled (rows past S read zero; their lanes are never stored, and a
        // lane's scores, max and sum never mix with another row's). The four wavefronts
        // share the block's rows: each fetches the 16-column chunks c = wave mod 4, issues
        // its first K/V tile, and the chunks meet in LDS (the combine area, free until
        // the end). One request per Q line instead of four matters at launch, when every
        // workgroup asks the L2 for its Q and first tile at once.
        constexpr int QPW = (NCH + KQ_WAVES - 1) / KQ_WAVES;
        floatx4 qpart[QPW];
        const unsigned qo = (unsigned)(q * DP + 4 * lg) * 4u;
#pragma unroll
        for (int c = 0; c < QPW; ++c)
            if (wave + KQ_WAVES * c < NCH)
                qpart[c] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo + 64 * (wave + KQ_WAVES * c), 0, 0));
        if (t < T) {
            load_k(t);
            load_v(t);
        }
#pragma unroll
        for (int c = 0; c < QPW; ++c)
            if (wave + KQ_WAVES * c < NCH)
                *reinterpret_cast<floatx4*>(&o_sh[0][lr][16 * (wave + KQ_WAVES * c) + 4 * lg]) = qpart[c];
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NCH; ++c) qf[c] = *reinterpret_cast<const floatx4*>(&o_sh[0][lr][16 * c + 4 * lg]);
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NCH; ++c) qf[c] *= g.scale_log2;
    }
    for (; t < T; t += KQ_WAVES) {
        const int k0 = t * A16_KB;
        // the prefetched tile; the last iteration loads its own tile again, so that every
        // path has the same loads in flight and each wait counts exactly
        const int tn = t + KQ_WAVES < T ? t + KQ_WAVES : t;
        // Sᵀ for two 16-key blocks; register r of block b = key k0 + 16b + 4g + r
        floatx4 sacc[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            sacc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    sacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[b][c][i], qf[c][i], sacc[b], 0, 0, 0);
        }
        load_k(tn);

        // p = 2^(s − m_run); m_run moves only when some lane's tile max exceeds it by more
        // than ATTN_LAZY (log2 units): then the row max is taken across the row's 4 lanes
        // and O and l_part are rescaled.  Tiles from t_fast apply the bounds, causal and
        // additive-mask terms per score.
        float tmax = -INFINITY;
        if (t >= t_fast) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kv = k0 + 16 * b + 4 * lg + r;
                    float sv = sacc[b][r];
                    if (HAS_MASK && kv < S && q < S) sv += g.mask[(bh * S + q) * (long long)S + kv] * LOG2E;
                    if (kv >= S || (CAUSAL && kv > q)) sv = -INFINITY;
                    sacc[b][r] = sv;
                    tmax = fmaxf(tmax, sv);
                }
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sacc[b][r]);
        }
        if (__any(tmax > m_run + ATTN_LAZY)) {
            const float m_new = fmaxf(m_run, rows4_max(tmax));
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
            for (int db = 0; db < NCH; ++db) oacc[db] *= corr;
            l_part *= corr;
            m_run = m_new;
        }
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = __builtin_amdgcn_exp2f(sacc[b][r] - m_run);
                sacc[b][r] = p;
                l_part += p;
            }
        // Oᵀ[d][q] += Σ_kv V[kv][d]·P[q][kv]; MFMA (b, r) takes key 16b + 4g + r from group g
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int h = 0; h < NH; ++h)
#pragma unroll
                    for (int w = 0; w < W; ++w)
                        oacc[W * h + w] =
                            __builtin_amdgcn_mfma_f32_16x16x4f32(vf[b][r][h][w], sacc[b][r], oacc[W * h + w], 0, 0, 0);
        load_v(tn);
        // keeps the V prefetch at the end of this iteration: otherwise the compiler merges it
        // with the load before the loop into one load at the top of the next iteration, after
        // which P·V waits for it
        __builtin_amdgcn_sched_barrier(0);
    }
    const float l_row = rows4_sum(l_part);

    // this wavefront's rows, relative to its own m_run, into LDS: register r of d block
    // W·h + w holds d = 16W·h + W·(4g + r) + w
    if (lg == 0) {
        m_sh[wave][lr] = m_run;
        l_sh[wave][lr] = l_row;
    }
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            VW o;
#pragma unroll
            for (int w = 0; w < W; ++w) o[w] = oacc[W * h + w][r];
            *reinterpret_cast<VW*>(&o_sh[wave][lr][16 * W * h + W * (4 * lg + r)]) = o;
        }
    __syncthreads();

    // combine: thread → (row, 4 columns); the four partials in wavefront order
    constexpr int TPR = DP / 4;
#pragma unroll
    for (int e0 = 0; e0 < KQ_QB * TPR; e0 += KQ_NT) {
        const int e = e0 + tid;
        const int row = e / TPR, d = (e % TPR) * 4;
        const int qq = q0 + row;
        if ((KQ_QB * TPR) % KQ_NT != 0 && e >= KQ_QB * TPR) break;
        if (qq >= S || d >= D) continue;
        float M = m_sh[0][row];
#pragma unroll
        for (int w = 1; w < KQ_WAVES; ++w) M = fmaxf(M, m_sh[w][row]);
        float L = 0.f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < KQ_WAVES; ++w) {
            const float s = __builtin_amdgcn_exp2f(m_sh[w][row] - M);
            L += s * l_sh[w][row];
            const float4 p = *reinterpret_cast<const float4*>(&o_sh[w][row][d]);
            acc.x += s * p.x;
            acc.y += s * p.y;
            acc.z += s * p.z;
            acc.w += s * p.w;
        }
        const float inv_l = 1.0f / L;
        acc.x *= inv_l;
        acc.y *= inv_l;
        acc.z *= inv_l;
        acc.w *= inv_l;
        float* dst = g.sk_defer ? g.part + (bh * S + qq) * (long long)D : attn_out_row(g, bh, qq);
        *reinterpret_cast<float4*>(dst + d) = acc;
    }
}

// Deferred output of attn_fwd_kq: rows staged in [bh, S, D] are stored to O
// (or its fused [B, S, H, D] transpose) once every read of Q, K and V is done.
__global__ __launch_bounds__(256) void attn_kq_flush(AttnArgs g) {
    const int tpr = g.D / 4;
    const long long t = blockIdx.x * 256LL + threadIdx.x;
    const long long row = t / tpr;
    const int d = (int)(t - row * tpr) * 4;
    const long long bh = blockIdx.y;
    if (row >= g.S) return;
    *reinterpret_cast<float4*>(attn_out_row(g, bh, row) + d) =
        *reinterpret_cast<const float4*>(g.part + (bh * g.S + row) * (long long)g.D + d);
}

// Combine the key-range partials of every query row whose block was split:
// O = Σ_c 2^(m_c − M)·acc_c / Σ_c 2^(m_c − M)·l_c, M = max_c m_c, segments
// summed in key order.  Rows of unsplit blocks return, unless g.sk_defer:
// then their single partial is normalised here (weight 2^0 = 1, so the
// result is bit-identical to the direct store).  Thread t of a row
// handles d = 4t .. 4t+3 (D % 4 == 0 on this path), so a row of hd = 128
// takes 32 threads and every load and store is a float4.
__global__ __launch_bounds__(256) void attn_split_merge(AttnArgs g, int causal) {
    const int tpr = g.D / 4;                                    // threads per row
    const long long t = blockIdx.x * 256LL + threadIdx.x;
    const long long row = t / tpr;
    const int d = (int)(t - row * tpr) * 4;
    const long long bh = blockIdx.y;
    if (row >= g.S) return;
    const int qb = (int)(row / A16_QB);
    const int G0 = (int)bh * g.sk_head_tiles + sk_block_start(g, qb, causal != 0);
    const int G1 = G0 + attn16_tiles(g, qb, causal != 0);
    const int nc = sk_owner(g, G1 - 1) - sk_owner(g, G0) + 1;
    if (nc <= 1 && !g.sk_defer) return;
    const long long r0 = (bh * g.n_qblocks + qb) * g.sk_maxseg * A16_QB + (row - (long long)qb * A16_QB);
    float M = -FLT_MAX;
    float L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    constexpr int NC_REG = 8;
    if (nc <= NC_REG) {
        // every segment's loads issued at once (one memory latency, not two
        // dependent rounds); the same sums in the same order as below
        float2 ml[NC_REG];
        float4 p[NC_REG];
#pragma unroll
        for (int c = 0; c < NC_REG; ++c)
            if (c < nc) {
                const long long pr = r0 + (long long)c * A16_QB;
                ml[c] = *reinterpret_cast<const float2*>(g.ml + 2 * pr);
                p[c] = *reinterpret_cast<const float4*>(g.part + pr * g.D + d);
            }
#pragma unroll
        for (int c = 0; c < NC_REG; ++c)
            if (c < nc) M = fmaxf(M, ml[c].x);
#pragma unroll
        for (int c = 0; c < NC_REG; ++c)
            if (c < nc) {
                const float w = __builtin_amdgcn_exp2f(ml[c].x - M);
                L += w * ml[c].y;
                acc.x += w * p[c].x;
                acc.y += w * p[c].y;
                acc.z += w * p[c].z;
                acc.w += w * p[c].w;
            }
    } else {
        for (int c = 0; c < nc; ++c) M = fmaxf(M, g.ml[2 * (r0 + (long long)c * A16_QB)]);
        for (int c = 0; c < nc; ++c) {
            const long long pr = r0 + (long long)c * A16_QB;
            const float w = __builtin_amdgcn_exp2f(g.ml[2 * pr] - M);
            L += w * g.ml[2 * pr + 1];
            const float4 p = *reinterpret_cast<const float4*>(g.part + pr * g.D + d);
            acc.x += w * p.x;
            acc.y += w * p.y;
            acc.z += w * p.z;
            acc.w += w * p.w;
        }
    }
    const float inv_l = 1.0f / L;
    acc.x *= inv_l;
    acc.y *= inv_l;
    acc.z *= inv_l;
    acc.w *= inv_l;
    *reinterpret_cast<float4*>(attn_out_row(g, bh, row) + d) = acc;
}

// Fallback for head dims the MFMA kernel does not take (hd % 8 != 0 or
// hd > 256): one workgroup per (bh, query row), scores held in LDS.
__global__ __launch_bounds__(256) void attn_fwd_rows(AttnArgs g, int causal) {
    extern __shared__ float sc[];
    __shared__ float red[4];
    const long long bh = blockIdx.y;
    const int q = blockIdx.x;
    const int S = g.S, D = g.D;
    const long long kvh = bh / g.group_size;
    const float* Qr = g.Q + (bh * S + q) * (long long)D;
    const float* Kb = g.K + kvh * (long long)S * D;
    const float* Vb = g.V + kvh * (long long)S * D;
    const float scale = g.scale_log2 / LOG2E;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < S; j += blockDim.x) {
        float acc = 0.f;
        for (int d = 0; d < D; ++d) acc += Qr[d] * Kb[(long long)j * D + d];
        float sv = acc * scale;
        if (g.mask) sv += g.mask[(bh * S + q) * (long long)S + j];
        if (causal && j > q) sv = -INFINITY;
        sc[j] = sv;
        mx = fmaxf(mx, sv);
    }
    mx = block_max(mx, red);
    float sum = 0.f;
    for (int j = threadIdx.x; j < S; j += blockDim.x) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    __syncthreads();
    float* Or = g.O + (bh * S + q) * (long long)D;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float acc = 0.f;
        for (int j = 0; j < S; ++j) acc += sc[j] * Vb[(long long)j * D + d];
        Or[d] = acc / sum;
    }
}

// Step::i: [0]=bh [1]=S [2]=D [3]=causal [4]=group [5]=DP (0 = row fallback)
//          [6]=fold [7]=split workgroups (0 = none) [8]=split partial slots per (head, block)
//          [9]=heads of a fused output transpose (0 = none) [10]=16x16 kernel (transpose fusable)
//          [11]=key tiles per head (split) [12]=V row stride when V is read from the columns
//          of a row-major tensor (0 = contiguous) [13]=K/V heads of that layout
//          [14]=deferred output (the merge kernel, or attn_kq_flush, writes every row of O)
//          [15]=key-quartered kernel (attn_fwd_kq) [16]=K stored fragment-major (key-quartered
//          kernel only; set by the plan with the QKV GEMM's head scatter, lbr_frag_keys_ok)
//          [18]=16x16 kernel on folded 64-row query blocks (4 wavefronts)
AttnArgs make_args(const Step& s) {
    AttnArgs g;
    g.Q = (const float*)s.in[0];
    g.K = (const float*)s.in[1];
    g.V = (const float*)s.in[2];
    g.mask = (const float*)s.in[3];
    g.O = (float*)s.out;
    g.S = (int)s.i[1];
    g.D = (int)s.i[2];
    g.group_size = (int)s.i[4];
    g.n_qblocks = (g.S + AT_QB - 1) / AT_QB;
    g.scale_log2 = s.f[0] * LOG2E;
    g.fold = 0;
    g.o_heads = 0;
    g.sk_defer = 0;
    g.v_ld = 0;
    g.v_heads = 1;
    g.k_frag = 0;
    return g;
}

template <int DP, bool CAUSAL, bool HAS_MASK>
void launch_attn(const Step& s, hipStream_t st) {
    AttnArgs g = make_args(s);
    if (g.S <= 0 || s.i[0] <= 0) return;
    hipLaunchKernelGGL((attn_fwd_mfma<DP, CAUSAL, HAS_MASK>), dim3(g.n_qblocks, (unsigned)s.i[0]), dim3(AT_NT), 0, st,
                       g);
}

void launch_attn_rows(const Step& s, hipStream_t st) {
    AttnArgs g = make_args(s);
    if (g.S <= 0 || s.i[0] <= 0) return;
    hipLaunchKernelGGL(attn_fwd_rows, dim3(g.S, (unsigned)s.i[0]), dim3(256), (size_t)g.S * sizeof(float), st, g,
                       (int)s.i[3]);
}

template <int DP, bool CAUSAL, bool HAS_MASK>
void launch_attn16(const Step& s, hipStream_t st) {
    AttnArgs g = make_args(s);
    if (g.S <= 0 || s.i[0] <= 0) return;
    g.n_qblocks = (g.S + A16_QB - 1) / A16_QB;
    g.fold = CAUSAL && s.i[6] != 0;
    g.o_heads = (int)s.i[9];
    if (s.i[12]) {
        g.v_ld = s.i[12];
        g.v_heads = (int)s.i[13];
    }
    g.sk_wg = (int)s.i[7];
    g.sk_maxseg = (int)s.i[8];
    g.sk_head_tiles = (int)s.i[11];
    g.sk_tiles = (int)(s.i[11] * s.i[0]);
    lbr_fast_divisor((unsigned)g.sk_wg, &g.sk_wg_m, &g.sk_wg_s);
    lbr_fast_divisor((unsigned)g.sk_tiles, &g.sk_tiles_m, &g.sk_tiles_s);
    lbr_fast_divisor((unsigned)g.sk_head_tiles, &g.sk_ht_m, &g.sk_ht_s);
    if (g.sk_wg > 0) {
        // workspace: partials, then (m, l) pairs
        const long long rows = s.i[0] * g.n_qblocks * (long long)g.sk_maxseg * A16_QB;
        g.part = (float*)s.ws;
        g.ml = g.part + rows * g.D;
        g.sk_defer = s.i[14] != 0;
        hipLaunchKernelGGL((attn_fwd_mfma16_split<DP, CAUSAL, HAS_MASK>), dim3((unsigned)g.sk_wg), dim3(A16_NT), 0, st,
                           g);
        hipLaunchKernelGGL(attn_split_merge, dim3((unsigned)(((long long)g.S * (g.D / 4) + 255) / 256), (unsigned)s.i[0]),
                           dim3(256), 0, st, g, (int)CAUSAL);
        return;
    }
    g.part = g.ml = nullptr;
    if (s.i[18]) {
        // 64-row folded blocks; a deferred store stages the rows for attn_kq_flush
        g.n_qblocks = (g.S + 63) / 64;
        g.sk_defer = s.i[14] != 0;
        if (g.sk_defer) g.part = (float*)s.ws;
        const unsigned gx = g.fold ? (unsigned)(g.n_qblocks + 1) / 2 : (unsigned)g.n_qblocks;
        hipLaunchKernelGGL((attn_fwd_mfma16<DP, CAUSAL, HAS_MASK, 4>), dim3(gx * (unsigned)s.i[0]), dim3(256), 0, st,
                           g);
        if (g.sk_defer)
            hipLaunchKernelGGL(attn_kq_flush, dim3((unsigned)(((long long)g.S * (g.D / 4) + 255) / 256),
                                                   (unsigned)s.i[0]),
                               dim3(256), 0, st, g);
        return;
    }
    const unsigned gx = g.fold ? (unsigned)(g.n_qblocks + 1) / 2 : (unsigned)g.n_qblocks;
    hipLaunchKernelGGL((attn_fwd_mfma16<DP, CAUSAL, HAS_MASK>), dim3(gx, (unsigned)s.i[0]), dim3(A16_NT), 0, st, g);
}

// kq_plan's cache: one assignment per (heads, S, causal, CUs, workgroups per CU).
std::mutex g_kq_mu;
std::map<std::array<long long, 5>, std::vector<unsigned short>> g_kq_plans;

template <int DP, bool CAUSAL, bool HAS_MASK>
void launch_attn_kq(const Step& s, hipStream_t st) {
    AttnArgs g = make_args(s);
    if (g.S <= 0 || s.i[0] <= 0) return;
    const int bh = (int)s.i[0];
    g.o_heads = (int)s.i[9];
    if (s.i[12]) {
        g.v_ld = s.i[12];
        g.v_heads = (int)s.i[13];
    }
    g.kq_nq = (g.S + KQ_QB - 1) / KQ_QB;
    g.kq_bh = bh;
    g.k_frag = s.i[16] != 0;
    g.sk_defer = s.i[14] != 0;
    g.part = g.sk_defer ? (float*)s.ws : nullptr;
    g.ml = nullptr;
    KqArgs k;
    k.g = g;
    const std::vector<unsigned short>& map = kq_plan(bh, g.S, CAUSAL, lbr_device_cus(), kq_per_cu(DP));
    k.n_map = (int)map.size();
    std::copy(map.begin(), map.end(), k.map);
    hipLaunchKernelGGL((attn_fwd_kq<DP, CAUSAL, HAS_MASK>), dim3((unsigned)(g.kq_nq * bh)), dim3(KQ_NT), 0, st, k);
    if (g.sk_defer)
        hipLaunchKernelGGL(attn_kq_flush, dim3((unsigned)(((long long)g.S * (g.D / 4) + 255) / 256), (unsigned)bh),
                           dim3(256), 0, st, g);
}

// Key tiles of query block q (host mirror of attn16_tiles).
int attn16_block_tiles(int S, bool causal, int q) {
    const int nt = (S + A16_KB - 1) / A16_KB;
    return causal ? std::min(nt, std::min(S - 1, q * A16_QB + A16_QB - 1) / A16_KB + 1) : nt;
}

// Key-range split of `bh` heads over `wg` workgroups (host mirror of
// sk_bound / sk_owner): the largest number of segments any (head, query
// block) is cut into, i.e. the partial slots each pair needs.
int attn16_max_segments(int S, bool causal, long long bh, long long wg) {
    const int nq = (S + A16_QB - 1) / A16_QB;
    long long head = 0;
    for (int q = 0; q < nq; ++q) head += attn16_block_tiles(S, causal, q);
    const long long total = head * bh;
    auto owner = [&](long long G) {
        long long w = G * wg / total;
        while (w + 1 < wg && (w + 1) * total / wg <= G) ++w;
        while (w > 0 && w * total / wg > G) --w;
        return w;
    };
    long long best = 1;
    for (long long h = 0; h < bh; ++h) {
        long long G = h * head;
        for (int q = 0; q < nq; ++q) {
            const int t = attn16_block_tiles(S, causal, q);
            best = std::max(best, owner(G + t - 1) - owner(G) + 1);
            G += t;
        }
    }
    return (int)best;
}

template <int DP>
step_fn pick(bool causal, bool mask) {
    if (causal) return mask ? launch_attn<DP, true, true> : launch_attn<DP, true, false>;
    return mask ? launch_attn<DP, false, true> : launch_attn<DP, false, false>;
}

template <int DP>
step_fn pick16(bool causal, bool mask) {
    if (causal) return mask ? launch_attn16<DP, true, true> : launch_attn16<DP, true, false>;
    return mask ? launch_attn16<DP, false, true> : launch_attn16<DP, false, false>;
}

template <int DP>
step_fn pick_kq(bool causal, bool mask) {
    if (causal) return mask ? launch_attn_kq<DP, true, true> : launch_attn_kq<DP, true, false>;
    return mask ? launch_attn_kq<DP, false, true> : launch_attn_kq<DP, false, false>;
}

}  // namespace

void lbr_attn_defer(Step* s) {
    s->i[14] = 1;
    // the key-quartered kernel and the 64-row fold stage every row of O ([bh, S, D]) for
    // attn_kq_flush; the split's workspace (its partials) already covers every block
    if (s->i[15] == 1 || s->i[18] == 1)
        s->ws_bytes = (size_t)s->i[0] * (size_t)s->i[1] * (size_t)s->i[2] * sizeof(float) + 256;
}

const char* lbr_attn_step_name(const Step& s, bool v, bool t, int store) {
    static const std::vector<std::string> table = [] {
        std::vector<std::string> n;
        for (int k = 0; k < 2; ++k)
            for (int a = 0; a < 2; ++a)
                for (int b = 0; b < 2; ++b)
                    for (int c = 0; c < 3; ++c)
                        n.push_back(std::string(k ? "attn_fwd_kq_f32" : "attn_fwd_mfma16_f32") + (a ? "+v" : "") +
                                    (b ? "+transpose" : "") + (c == 1 ? "+defer" : c == 2 ? "+relay" : ""));
        return n;
    }();
    const int kq = s.i[15] == 1;
    return table[(((kq * 2 + (v ? 1 : 0)) * 2 + (t ? 1 : 0)) * 3) + (store < 0 || store > 2 ? 0 : store)].c_str();
}

// Whole heads, or alternate blocks of them, per XCD: the smallest P in
// {1, 2, 4, 8} that divides the 16-row blocks and makes bh·P units (head h,
// blocks b ≡ p mod P) a multiple of the 8 XCDs; *upx = units per XCD, 0 when
// no P fits.
void attn_kq_layout(long long bh, int S, int* P, int* upx) {
    const int nq = (S + KQ_QB - 1) / KQ_QB;
    *P = 1;
    *upx = 0;
    for (int p = 1; p <= 8; p *= 2)
        if (p <= nq && nq % p == 0 && (bh * p) % 8 == 0) {
            *P = p;
            *upx = (int)(bh * p / 8);
            return;
        }
}

// Workgroups of attn_fwd_kq one CU holds at once (4 wavefronts each): the
// register budget of 128 (hd ≤ 64) or 256 (hd 128) VGPRs leaves 4 or 2
// wavefronts per SIMD.
int kq_per_cu(int dp) { return dp <= 64 ? 4 : 2; }

// The block each workgroup runs (LPT: longest processing time first).  With C
// CUs, workgroup w = r·C + g is the r-th on CU g (XCD g mod 8).  Blocks are
// taken heaviest first (causal: most key tiles) and each goes to the CU of its
// head's XCD with the least load so far, ties to the CU with fewer slots left
// (so the heaviest blocks get CUs of their own when some CUs hold fewer
// workgroups), then the lowest index.  Empty (the kernel's own order) when the
// grid does not fit on the CUs at once, or C is not a multiple of 8, or the
// grid exceeds the kernel-argument table.
const std::vector<unsigned short>& kq_plan(long long bh, int S, bool causal, int C, int per_cu) {
    std::lock_guard<std::mutex> lock(g_kq_mu);
    std::vector<unsigned short>& map = g_kq_plans[{bh, S, causal ? 1 : 0, C, per_cu}];
    const int nq = (S + KQ_QB - 1) / KQ_QB;
    const long long n = bh * nq;
    if (!map.empty() || C <= 0 || C % 8 || n > (long long)per_cu * C || n > KQ_MAP_MAX) return map;
    const int nt = (S + A16_KB - 1) / A16_KB;
    auto weight = [&](int b) { return causal ? std::min(nt, std::min(S - 1, b * KQ_QB + KQ_QB - 1) / A16_KB + 1) : nt; };
    int P, upx;
    attn_kq_layout(bh, S, &P, &upx);
    std::vector<int> items((size_t)n);
    for (int i = 0; i < (int)n; ++i) items[i] = i;
    std::stable_sort(items.begin(), items.end(), [&](int a, int b) { return weight(a % nq) > weight(b % nq); });
    std::vector<long long> load(C, 0);
    std::vector<int> used(C, 0), cap(C, 0);
    for (int g = 0; g < C; ++g) cap[g] = g < n ? (int)((n - g + C - 1) / C) : 0;
    std::vector<unsigned short> out((size_t)n);
    for (int it : items) {
        const int h = it / nq, b = it % nq;
        const int x = upx > 0 ? (h * P + b % P) / upx : -1;
        int best = -1;
        for (int g = x < 0 ? 0 : x; g < C; g += x < 0 ? 1 : 8) {
            if (used[g] >= cap[g]) continue;
            if (best < 0 || load[g] < load[best] ||
                (load[g] == load[best] && cap[g] - used[g] < cap[best] - used[best]))
                best = g;
        }
        if (best < 0) return map;   // capacities do not match the XCD layout: keep the kernel's order
        out[(size_t)used[best] * C + best] = (unsigned short)it;
        ++used[best];
        load[best] += weight(b);
    }
    map = out;
    return map;
}

extern "C" unsigned lbr_fast_div(unsigned x, unsigned d) {
    int m = 0, sh = 0;
    lbr_fast_divisor(d, &m, &sh);
    if (m == 0) return x;
    return (unsigned)(((unsigned long long)x * (unsigned)m) >> 32) >> sh;
}

extern "C" int lbr_attn_kq_grid(long long bh, int seq, int causal, int cus, int* heads_out, int* blocks_out,
                                int cap) {
    if (bh <= 0 || seq <= 0) return 0;
    KqArgs k;
    k.g = AttnArgs();
    k.g.kq_nq = (seq + KQ_QB - 1) / KQ_QB;
    k.g.kq_bh = (int)bh;
    const std::vector<unsigned short>& map = kq_plan(bh, seq, causal != 0, cus, kq_per_cu(64));
    k.n_map = (int)map.size();
    std::copy(map.begin(), map.end(), k.map);
    const long long n = k.g.kq_nq * bh;
    for (long long w = 0; w < n && w < cap; ++w) kq_item(k, (int)w, &heads_out[w], &blocks_out[w]);
    return (int)n;
}

int decode_attention(const OpNode* n, Step* s) {
    // an additive mask replaces the causal pattern: the reference applies one or the other,
    // never both (attn.c:40-48; its flash path, the only other, takes no mask, executor.c:389)
    const int has_mask = n->extra[3] != 0;
    const int seq = n->extra[0], hd = n->extra[1], causal = n->extra[2] != 0 && !has_mask;
    const int group = n->extra[4] > 0 ? n->extra[4] : 1;
    if (n->n_inputs < (has_mask ? 4 : 3) || !n->output || n->n_dims < 2) {
        lbr_set_error("attention: malformed node");
        return LBR_ERR_INVALID;
    }
    for (int i = 0; i < (has_mask ? 4 : 3); ++i)
        if (!n->inputs[i]) {
            lbr_set_error("attention: input %d is null", i);
            return LBR_ERR_INVALID;
        }
    if (n->out_shape[n->n_dims - 2] != seq || n->out_shape[n->n_dims - 1] != hd) {
        lbr_set_error("attention: seq_len %d / head_dim %d are not the output's last dims %d x %d", seq, hd,
                      n->out_shape[n->n_dims - 2], n->out_shape[n->n_dims - 1]);
        return LBR_ERR_INVALID;
    }
    long long bh = 1;
    for (int i = 0; i < n->n_dims - 2; ++i) bh *= n->out_shape[i];
    if (seq <= 0 || hd <= 0 || bh > 65535 || (group > 1 && bh % group != 0)) {
        if (seq == 0 || bh == 0) {
            s->run = [](const Step&, hipStream_t) {};
            s->name = "attention_empty";
            return LBR_OK;
        }
        lbr_set_error("attention: unsupported sizes bh=%lld S=%d hd=%d group=%d", bh, seq, hd, group);
        return LBR_ERR_UNSUPPORTED;
    }
    s->in[0] = n->inputs[0];
    s->in[1] = n->inputs[1];
    s->in[2] = n->inputs[2];
    s->in[3] = has_mask ? n->inputs[3] : nullptr;
    s->out = n->output;
    s->i[0] = bh;
    s->i[1] = seq;
    s->i[2] = hd;
    s->i[3] = causal;
    s->i[4] = group;
    s->f[0] = 1.0f / sqrtf((float)hd);   // attn.c:68/242
    const bool aligned = lbr_aligned(n->inputs[0], 16) && lbr_aligned(n->inputs[1], 16) &&
                         lbr_aligned(n->inputs[2], 16) && lbr_aligned(n->output, 16);
    if (hd % 8 == 0 && hd <= 256 && aligned) {
        const int dp = hd <= 32 ? 32 : hd <= 64 ? 64 : hd <= 128 ? 128 : 256;
        s->i[5] = dp;
        // LBR_ATTN_TILE=32 keeps the 32x32 kernel for every head dim (A/B timing).
        const char* tile = getenv("LBR_ATTN_TILE");
        if (dp <= 128 && !(tile && atoi(tile) == 32)) {
            // Fold causal query blocks in pairs while that still leaves one
            // 8-wavefront workgroup per CU (LBR_ATTN_FOLD=0/1 overrides).
            const long long nq = (seq + A16_QB - 1) / A16_QB;
            const int cus = lbr_device_cus() > 0 ? lbr_device_cus() : 256;
            s->i[6] = causal && (nq + 1) / 2 * bh >= cus;
            const char* fold = getenv("LBR_ATTN_FOLD");
            if (fold) s->i[6] = causal && atoi(fold) != 0;
            // Grids that leave CUs idle (fewer than two 8-wavefront workgroups per
            // CU, not folded) take the key-range split: equal shares of all key
            // tiles, of at least 8 tiles (4 for hd <= 64) since every segment pays
            // a Q load, the first tile's latency and, when cut, a partial.  The
            // workgroup count is a whole number of rounds over the CUs (two
            // workgroups per CU, or one) when the shares allow it — a partial
            // round leaves some CUs with twice the work (measured: Qwen3 shares
            // of 8 tiles, 576 workgroups, 134 µs against 110 µs for 9-tile shares
            // on 512; GPT-2 256 workgroups 36 µs against 38 µs on 432) — else
            // one workgroup per minimum share.  No split when that gives no more
            // workgroups than the plain grid.  LBR_ATTN_SPLIT=<n> forces shares
            // of n tiles (0: no split), LBR_ATTN_SPLIT_WG=<n> n workgroups.
            // Grids that leave CUs idle (fewer than two 8-wavefront workgroups per CU,
            // not folded), head dim 32 or 64 (no padded columns): 16-row workgroups
            // with the key tiles dealt over four wavefronts (attn_fwd_kq), no merge.
            // GPT-2 S=1024: 33.1 µs + a 5.3 µs merge with the key-range split.
            // LBR_ATTN_KQ=1 forces it for any unpadded head dim ≤ 128, 0 turns it off;
            // a forced schedule (LBR_ATTN_FOLD / _TILE / _SPLIT / _SPLIT_WG) keeps it off.
            {
                const bool forced = getenv("LBR_ATTN_FOLD") || getenv("LBR_ATTN_SPLIT") || getenv("LBR_ATTN_SPLIT_WG");
                bool kq = hd == dp && hd <= 64 && !s->i[6] && nq * bh < 2LL * cus && !forced;
                const char* kqe = getenv("LBR_ATTN_KQ");
                if (kqe) kq = atoi(kqe) != 0 && hd == dp;
                const long long n16 = (seq + KQ_QB - 1) / KQ_QB;
                // the kernel's buffer views address one head's rows with 32-bit byte offsets
                if (kq && n16 * bh < (1LL << 31) && (long long)seq * hd * 4 < (1LL << 31)) {
                    s->i[6] = 0;
                    s->i[15] = 1;   // a deferred store stages its rows in the workspace (lbr_attn_defer)
                    switch (dp) {
                        case 32: s->run = pick_kq<32>(causal, has_mask); break;
                        case 64: s->run = pick_kq<64>(causal, has_mask); break;
                        default: s->run = pick_kq<128>(causal, has_mask); break;
                    }
                    s->name = "attn_fwd_kq_f32";
                    s->i[10] = 1;   // can write O as [B, S, H, D] and read a strided V, like the 16x16 kernel
                    return LBR_OK;
                }
            }
            // Causal grids the 128-row fold leaves short of one workgroup a CU, head dim
            // > 64: folded 64-row blocks (4 wavefronts) when their pairs give every CU one
            // workgroup of equal work, no split and no merge.  Qwen3-4B S1024 (32 heads):
            // 256 workgroups.  LBR_ATTN_FOLD64=1 forces it for any causal grid, 0 turns it
            // off; a forced schedule (LBR_ATTN_FOLD / _SPLIT / _SPLIT_WG) keeps it off.
            {
                const long long n64 = (seq + 63) / 64;
                const bool forced = getenv("LBR_ATTN_FOLD") || getenv("LBR_ATTN_SPLIT") || getenv("LBR_ATTN_SPLIT_WG");
                bool fold64 = causal && !s->i[6] && !forced && (n64 + 1) / 2 * bh >= cus;
                if (const char* f64 = getenv("LBR_ATTN_FOLD64")) fold64 = atoi(f64) != 0 && causal && !forced;
                if (fold64) {
                    s->i[6] = 1;
                    s->i[18] = 1;
                }
            }
            long long head_tiles = 0;
            for (int q = 0; q < nq; ++q) head_tiles += attn16_block_tiles(seq, causal != 0, q);
            const long long total = head_tiles * bh;
            long long wg = 0;
            // The key-range split described above, except when the heaviest block holds at
            // most 4 key tiles (S <= 128): the merge launch then costs more than the shorter
            // chain saves (one attention node,
            // back-to-back replays: H4 S128 hd 48 21.7 us split against 18.4 us whole, hd 16
            // 18.5 against 16.1; H8 S256 hd 48 22.1 against 27.8, H4 S512 23.0 against 46.8)
            if (!s->i[6] && nq * bh < 2LL * cus && attn16_block_tiles(seq, causal != 0, (int)nq - 1) > 4) {
                const int min_share = hd <= 64 ? 4 : 8;
                const long long rounds = std::min(2LL, total / ((long long)min_share * cus));
                // too few tiles for a whole round: shares of 2 tiles (hd <= 64), which
                // divide every block's 4k tiles (GPT-2-width S512: 240 workgroups,
                // 21.1 µs, against 22.9 µs for 4-tile shares and 25.0 for 3)
                wg = rounds > 0 ? rounds * cus : total / (hd <= 64 ? 2 : min_share);
                if (wg <= nq * bh) wg = 0;
            }
            const char* split = getenv("LBR_ATTN_SPLIT");
            if (split) {
                const long long n = atoi(split);
                wg = n > 0 ? (total + n - 1) / n : 0;
            }
            const char* split_wg = getenv("LBR_ATTN_SPLIT_WG");   // forces the workgroup count
            if (split_wg) wg = std::max(0, atoi(split_wg));
            wg = std::min(wg, total);   // every share holds at least one tile
            // the kernels' share arithmetic is 32-bit: wg · total < 2³¹
            if (wg > 0 && wg * total >= (1LL << 31)) wg = 0;
            if (wg > 0 && !s->i[6]) {
                const int maxseg = attn16_max_segments(seq, causal != 0, bh, wg);
                s->i[7] = wg;
                s->i[8] = maxseg;
                s->i[11] = head_tiles;
                s->ws_bytes = (size_t)(bh * nq * maxseg * A16_QB) * (size_t)(hd + 2) * sizeof(float) + 256;
            }
            switch (dp) {
                case 32: s->run = pick16<32>(causal, has_mask); break;
                case 64: s->run = pick16<64>(causal, has_mask); break;
                default: s->run = pick16<128>(causal, has_mask); break;
            }
            s->name = "attn_fwd_mfma16_f32";
            s->i[10] = 1;   // can write O as [B, S, H, D] (i[9] = H) for a fused transpose
            return LBR_OK;
        }
        switch (dp) {
            case 32: s->run = pick<32>(causal, has_mask); break;
            case 64: s->run = pick<64>(causal, has_mask); break;
            case 128: s->run = pick<128>(causal, has_mask); break;
            default: s->run = pick<256>(causal, has_mask); break;
        }
        s->name = "attn_fwd_mfma_f32";
        return LBR_OK;
    }
    if ((long long)seq * 4 > 60 * 1024) {
        lbr_set_error("attention: fallback path holds S scores in LDS; S=%d too long for hd=%d", seq, hd);
        return LBR_ERR_UNSUPPORTED;
    }
    s->i[5] = 0;
    s->run = launch_attn_rows;
    s->name = "attn_fwd_rows";
    return LBR_OK;
}
