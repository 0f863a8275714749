// gemm.hip — fp32 GEMM on the gfx950 matrix cores.
//
// Replaces kernel_matmul_ab / kernel_matmul_gemv (csrc/ops/matmul.c:19-79,
// cblas_sgemm / cblas_sgemv) behind MATMUL and MATMUL_ADD
// (csrc/executor.c:197-224, 312-346):
//   MATMUL      C = alpha · A · op(B)
//   MATMUL_ADD  C = bias[n] + A · op(B)   (alpha is not applied: the
//               reference hard-codes alpha = 1 on this path, executor.c:341/344)
// op(B) = Bᵀ when trans_b (B stored [N, K], nn.Linear layout) else B ([K, N]).
//
// Two kernels: gemm_dma_f32 (below the register-staged one) takes every
// trans_b GEMM with K a multiple of 32 — all the Linear layers of the
// workloads — with v_mfma_f32_16x16x4_f32, direct-to-LDS loads and a tile
// shape chosen per GEMM; gemm_mfma_f32 (v_mfma_f32_32x32x2_f32) takes the
// rest (B stored [K, N], ragged K, unaligned operands).
//
// gemm_mfma_f32 tiling: a 256-thread workgroup (4 wavefronts, 2×2) owns a 128×128 tile of
// C; each wavefront owns 64×64 = 2×2 MFMA blocks of 32×32 (64 accumulator
// registers per lane).  K advances in steps of 32: the next A/B tiles are
// fetched from global memory into registers while the current ones are
// consumed from LDS (rows padded to 36 floats so 16-byte LDS reads are
// conflict-free).  Each lane reads a float4 of 4 consecutive k for its row;
// the four components feed four MFMAs, so one MFMA reduces over k and k+4
// (the half-wave split of the 32x32x2 operand layout) — a reordering of the
// K sum, exact in real arithmetic.
//
// Workgroups are numbered so that consecutive ids share an A row panel and
// are mapped round-robin over the 8 XCDs by the hardware; the remap below
// gives each XCD a contiguous range of tiles so neighbouring tiles (which
// reuse the same A and B panels) hit the same L2.
#include "lbr_device.h"

#include <cstdlib>
#include <cstring>

namespace {

constexpr int BM = 128, BN = 128, BK = 32, LDK = BK + 4;
constexpr int NT = 256;
constexpr int N_XCD = 8;
constexpr int GROUP_M = 8;   // tile rows per L2 group

struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    int M, N, K;
    long long sA, sB, sC;     // batch strides (elements)
    float alpha;
    int tiles_m, tiles_n;
    float* W;                 // split-K partial sums [ksplit][batches][M][N] (ksplit > 1)
    int ksplit, kchunk;       // number of K ranges, K per range (multiple of BK)
    // Fused epilogues (set only by the plan's peephole fusion; all null/0 otherwise).
    const float* resid;       // C += resid (same layout as C): a following same-shape ADD
    int n_split;              // >0: C columns are scattered as attention heads, see epi_store
    int col_begin[5];         // split k owns columns [col_begin[k], col_begin[k+1])
    float* dst[4];            // split k's output, laid out [B, H, S, hd]
    const float* sbias[4];    // split k's bias row (indexed by column - col_begin[k]) or null
    int Hs[4], hd, S;         // heads of each split, head dim, rows per batch (M = B·S)
    int frag;                 // bit k: split k is stored fragment-major (lbr_frag_offset)
    // Head prologue in the epilogue (lbr_merge_gemm_head_prologue; 64×128 DMA tile, hd =
    // 128 = TN): C columns [hp_col[p], hp_col[p] + hp_H[p]·128) of part p hold heads of
    // 128; each tile's C values (+ bias) go round through LDS, get the part's bias,
    // per-head RMSNorm (weight hp_w[p], eps hp_eps[p]) and rotate-half RoPE (cos/sin row
    // of token (b, s) at b·hp_tst[0] + s·hp_tst[1]) and are stored as [B, H, S, 128] at
    // hp_out[p] (C's columns of the parts are not written); hp_flags: 1 norm, 2 RoPE
    int hp_parts, hp_flags, hp_S;
    int hp_col[2], hp_H[2];
    float* hp_out[2];
    const float* hp_w[2];
    const float* hp_b[2];
    float hp_eps[2];
    const float* hp_cos;
    const float* hp_sin;
    long long hp_tst[2];
    int act;                  // LBR_ACT_*: a following RELU / GELU / SILU applied to C (DMA kernel)
    // Gated pair (DMA kernel): the GEMM's columns hold a gate half and an up half
    // of gF columns each; the kernel writes out[m][j] = act(gate[m][j] (+ gbias[j]))·up[m][j]
    // to C as [M, gF]
    int gF;                   // 0: off
    int gbase;                // first column of the gate half (0 or gF; up is the other half)
    int gact;                 // 0: SiLU, 1: GELU (GATED_ACT extras[1])
    const float* gbias;       // GATED_ACT bias (applied to gate) or null
    // A in head layout (DMA kernel): A is stored [B, aH, aS, ahd] and read as the
    // [B·aS, aH·ahd] matrix its TRANSPOSE(1, 2) would give (aH = 0: A is row-major)
    int aH, aS, ahd;
    // Norm prologue (DMA kernel, NORM template argument): A is the input of a
    // RMSNORM / LAYERNORM over its K columns whose output was this GEMM's A;
    // nw = weight (γ), nb = LayerNorm bias (β), neps = eps
    const float* nw;
    const float* nb;
    float neps;
    // Norm after the split-K reduce (lbr_merge_reduce_norm): the reduce, one row
    // at a time, also normalises C's row into nt_out (RMSNORM / LAYERNORM over
    // the N columns, weight nt_w, LayerNorm bias nt_b)
    float* nt_out;
    const float* nt_w;
    const float* nt_b;
    float nt_eps;
};

// Final store of one C element (row m, column n of batch bz) with the fused
// epilogues applied in the order the unfused nodes would: v (already
// alpha-scaled or bias-added) + resid, then the scattered split's bias.
__device__ __forceinline__ void epi_store(const GemmArgs& g, long long bz, int m, int n, float v) {
    if (g.resid) v = v + g.resid[bz * g.sC + (long long)m * g.N + n];
    if (g.n_split == 0) {
        g.C[bz * g.sC + (long long)m * g.N + n] = v;
        return;
    }
    if (n < g.col_begin[0] || n >= g.col_begin[g.n_split]) return;   // columns no split reads
    int k = 0;
    while (k + 1 < g.n_split && n >= g.col_begin[k + 1]) ++k;
    const int c = n - g.col_begin[k];
    if (g.sbias[k]) v = v + g.sbias[k][c];
    const int h = c / g.hd, d = c - h * g.hd;
    const int b = m / g.S, s = m - b * g.S;
    const long long head = ((long long)b * g.Hs[k] + h) * g.S * g.hd;
    g.dst[k][head + (((g.frag >> k) & 1) ? lbr_frag_offset(s, d, g.hd) : (long long)s * g.hd + d)] = v;
}

__device__ __forceinline__ void tile_coords(const GemmArgs& g, int& tm, int& tn) {
    // XCD-aware remap: hardware places workgroup id w on XCD w % 8.
    const int tiles = g.tiles_m * g.tiles_n;
    int w = blockIdx.x;
    if (tiles % N_XCD == 0) {
        const int per = tiles / N_XCD;
        w = (w % N_XCD) * per + (w / N_XCD);
    }
    // grouped ordering: GROUP_M tile-rows advance together along N
    const int group_size = GROUP_M * g.tiles_n;
    const int gid = w / group_size;
    const int first_m = gid * GROUP_M;
    const int gm = min(g.tiles_m - first_m, GROUP_M);
    const int in_group = w % group_size;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

template <bool TRANS_B, bool VEC>
__device__ __forceinline__ void load_tiles(const GemmArgs& g, const float* __restrict__ A, const float* __restrict__ B,
                                           int m0, int n0, int k0, float4 (&ra)[4], float4 (&rb)[4]) {
    const int tid = threadIdx.x;
    if (VEC) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int idx = tid + p * NT;       // 0..1023
            const int row = idx >> 3;           // 0..127
            const int kc = (idx & 7) * 4;       // 0..28
            const int gm = m0 + row, gk = k0 + kc;
            ra[p] = (gm < g.M && gk < g.K) ? *reinterpret_cast<const float4*>(A + (long long)gm * g.K + gk)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (TRANS_B) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int idx = tid + p * NT;
                const int row = idx >> 3;
                const int kc = (idx & 7) * 4;
                const int gn = n0 + row, gk = k0 + kc;
                rb[p] = (gn < g.N && gk < g.K) ? *reinterpret_cast<const float4*>(B + (long long)gn * g.K + gk)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        } else {
            // B is [K, N]: read 4 consecutive n of one k row
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int idx = tid + p * NT;   // 0..1023
                const int kk = idx >> 5;        // 0..31
                const int nc = (idx & 31) * 4;  // 0..124
                const int gn = n0 + nc, gk = k0 + kk;
                rb[p] = (gn < g.N && gk < g.K) ? *reinterpret_cast<const float4*>(B + (long long)gk * g.N + gn)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    } else {
        // scalar fallback: 16 elements of each tile per thread, packed into float4 slots
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float v[4], w[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int idx = tid + (p * 4 + q) * NT;  // 0..4095
                const int row = idx >> 5, kk = idx & 31;
                const int gm = m0 + row, gk = k0 + kk;
                v[q] = (gm < g.M && gk < g.K) ? A[(long long)gm * g.K + gk] : 0.f;
                const int gn = n0 + row;
                if (TRANS_B) w[q] = (gn < g.N && gk < g.K) ? B[(long long)gn * g.K + gk] : 0.f;
                else w[q] = (gn < g.N && gk < g.K) ? B[(long long)gk * g.N + gn] : 0.f;
            }
            ra[p] = make_float4(v[0], v[1], v[2], v[3]);
            rb[p] = make_float4(w[0], w[1], w[2], w[3]);
        }
    }
}

template <bool TRANS_B, bool VEC>
__device__ __forceinline__ void store_tiles(float (*As)[LDK], float (*Bs)[LDK], const float4 (&ra)[4],
                                            const float4 (&rb)[4]) {
    const int tid = threadIdx.x;
    if (VEC) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int idx = tid + p * NT;
            const int row = idx >> 3, kc = (idx & 7) * 4;
            *reinterpret_cast<float4*>(&As[row][kc]) = ra[p];
        }
        if (TRANS_B) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int idx = tid + p * NT;
                const int row = idx >> 3, kc = (idx & 7) * 4;
                *reinterpret_cast<float4*>(&Bs[row][kc]) = rb[p];
            }
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int idx = tid + p * NT;
                const int kk = idx >> 5, nc = (idx & 31) * 4;
                Bs[nc + 0][kk] = rb[p].x;
                Bs[nc + 1][kk] = rb[p].y;
                Bs[nc + 2][kk] = rb[p].z;
                Bs[nc + 3][kk] = rb[p].w;
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float v[4] = {ra[p].x, ra[p].y, ra[p].z, ra[p].w};
            const float w[4] = {rb[p].x, rb[p].y, rb[p].z, rb[p].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int idx = tid + (p * 4 + q) * NT;
                const int row = idx >> 5, kk = idx & 31;
                As[row][kk] = v[q];
                Bs[row][kk] = w[q];
            }
        }
    }
}

template <bool TRANS_B, bool VEC, bool HAS_BIAS>
__global__ __launch_bounds__(NT, 2) void gemm_mfma_f32(GemmArgs g) {
    __shared__ float As[BM][LDK];
    __shared__ float Bs[BN][LDK];

    int tm, tn;
    tile_coords(g, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const long long bz = blockIdx.z;
    const float* __restrict__ A = g.A + bz * g.sA;
    const float* __restrict__ B = g.B + bz * g.sB;
    float* __restrict__ C = g.C + bz * g.sC;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lrow = lane & 31, lhalf = lane >> 5;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // K range of this workgroup: all of K, or split ks of ksplit (kchunk is a
    // multiple of BK, so only the last range can end inside a K step).
    const int ks = blockIdx.y;
    const int kbeg = ks * g.kchunk;
    const int kend = min(g.K, kbeg + g.kchunk);
    float4 ra[4], rb[4];
    const int nk = (kend - kbeg + BK - 1) / BK;
    load_tiles<TRANS_B, VEC>(g, A, B, m0, n0, kbeg, ra, rb);
    store_tiles<TRANS_B, VEC>(As, Bs, ra, rb);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) load_tiles<TRANS_B, VEC>(g, A, B, m0, n0, kbeg + (kt + 1) * BK, ra, rb);
#pragma unroll
        for (int c = 0; c < BK / 8; ++c) {
            const int kc = c * 8 + lhalf * 4;
            floatx4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const floatx4*>(&As[wm * 64 + i * 32 + lrow][kc]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const floatx4*>(&Bs[wn * 64 + j * 32 + lrow][kc]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][q], b[j][q], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
        if (kt + 1 < nk) {
            store_tiles<TRANS_B, VEC>(As, Bs, ra, rb);
            __syncthreads();
        }
    }

    // Epilogue.  Accumulator layout of the 32x32 block: lane l, register r
    // holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
    if (g.ksplit > 1) {
        // raw partial sums; splitk_reduce applies alpha / bias in a fixed order
        float* __restrict__ Wp = g.W + ((long long)ks * gridDim.z + bz) * (long long)g.M * g.N;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 64 + j * 32 + lrow;
                if (n >= g.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                    if (m < g.M) Wp[(long long)m * g.N + n] = acc[i][j][r];
                }
            }
        return;
    }
    if (g.n_split) {
        // Head scatter: the column fixes split, head, d and split bias; the
        // row fixes (b, s) = divmod(m, S), stepped from the block's first row.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + lrow;
            if (n >= g.N || n < g.col_begin[0] || n >= g.col_begin[g.n_split]) continue;
            int k = 0;
            while (k + 1 < g.n_split && n >= g.col_begin[k + 1]) ++k;
            const int c = n - g.col_begin[k];
            const int h = c / g.hd, d = c - h * g.hd;
            const float bv = HAS_BIAS ? g.bias[n] : 0.f;
            const float sb = g.sbias[k] ? g.sbias[k][c] : 0.f;
            const bool has_sb = g.sbias[k] != nullptr;
            const bool fr = (g.frag >> k) & 1;
            float* __restrict__ col = g.dst[k] + ((long long)h * g.S) * g.hd + (fr ? lbr_frag_offset(0, d, g.hd) : d);
            const long long bstride = (long long)g.Hs[k] * g.S * g.hd;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int mb = m0 + wm * 64 + i * 32 + 4 * lhalf;
                const int b0 = mb / g.S, s0 = mb - b0 * g.S;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int o = 8 * (r >> 2) + (r & 3);
                    if (mb + o >= g.M) continue;
                    int b = b0, s = s0 + o;
                    while (s >= g.S) {   // o < 32: at most one step unless S < 32
                        s -= g.S;
                        ++b;
                    }
                    float v = HAS_BIAS ? (acc[i][j][r] + bv) : g.alpha * acc[i][j][r];
                    if (has_sb) v = v + sb;
                    col[b * bstride + (fr ? lbr_frag_offset(s, 0, g.hd) : (long long)s * g.hd)] = v;
                }
            }
        }
        return;
    }
    if (g.resid) {
        const float* __restrict__ R = g.resid + bz * g.sC;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 64 + j * 32 + lrow;
                if (n >= g.N) continue;
                const float bv = HAS_BIAS ? g.bias[n] : 0.f;
                float rv[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) {   // all loads first, then the adds and stores
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                    rv[r] = m < g.M ? R[(long long)m * g.N + n] : 0.f;
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                    if (m < g.M) {
                        const float v = HAS_BIAS ? (acc[i][j][r] + bv) : g.alpha * acc[i][j][r];
                        C[(long long)m * g.N + n] = v + rv[r];
                    }
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + lrow;
            if (n >= g.N) continue;
            const float bv = HAS_BIAS ? g.bias[n] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                if (m < g.M) C[(long long)m * g.N + n] = HAS_BIAS ? (acc[i][j][r] + bv) : g.alpha * acc[i][j][r];
            }
        }
}

// ---------------------------------------------------------------- DMA GEMM (trans_b)
// C = A · Bᵀ with A [M, K] and B [N, K] both K-contiguous, K a multiple of
// the tile's K step (DBK = 32 floats; a few tiles take 64, see KB below, with
// 16 chunks a row, swizzled by r & 15, and 4 rows a DMA instruction): the
// 16-byte direct-to-LDS form of buffer loads streams each K step
// of the A and B tiles into LDS without passing through registers, into a
// second LDS stage while the first is consumed (one barrier per K step).
//
// LDS layout of a stage: the A tile's TM rows, then the B tile's TN rows,
// DBK floats (8 chunks of 16 bytes) per row, chunk c of row r stored at
// position c ^ (r & 7) so the 16-byte fragment reads of 8 consecutive rows
// hit 8 different bank groups.  One DMA instruction fills 1 KB = 8 rows:
// lane l lands at byte 16·l, i.e. row l/8, position l%8, so it fetches the
// logical chunk (l%8) ^ row.
//
// Math: v_mfma_f32_16x16x4_f32, a WGM×WGN grid of wavefronts each owning a
// (TM/WGM)×(TN/WGN) block of C.  Lane (kq, i) = (l/16, l%16) reads 4
// consecutive k of row i of a 16-row block; component q feeds MFMA q, which
// reduces over k = 4·kq + q of the 16-wide chunk — the four MFMAs cover the
// chunk exactly once (a reordering of the K sum).  Accumulator register r of
// lane l holds row 4·(l/16) + r, column l%16 of the 16×16 block.
//
// Software pipeline: the fragments of the next 16-wide K chunk are read
// while the MFMAs of the current one issue; at the last chunk of a K step
// the workgroup synchronises once (the next stage has landed and the
// current one is free), starts the DMA two steps ahead into the freed stage
// and reads the next step's first fragments.  sched_group_barrier pairs
// every DMA issue and fragment read with one MFMA so the matrix pipe keeps
// issuing.
constexpr int DBK = 32;

// 16-byte DMA into LDS: lane l's dword4 at r + voff + soff lands at lds + 16·l.
// (A plain device function: the builtin has no host-side form inside kernel templates.)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, float* lds, unsigned voff, unsigned soff) {
    lbr_dma16(r, lds, voff, soff);
}

template <int NV, int ND, int NM>
__device__ __forceinline__ void chunk_schedule() {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // one VMEM read (DMA)
    }
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NM - NV - ND, 0);
}

// NORM (norm prologue): 0 none; 1 RMSNORM — the A fragments are multiplied by
// w[k] and Σx² of each row is accumulated from them, the result is scaled by
// the row's 1/√(Σx²/K + eps) in the epilogue (= GEMM(x·scale·w)); 2
// LAYERNORM — with c the row's first element, the fragments become (x − c)·γ
// and Σ(x − c), Σ(x − c)² accumulate per row, u = Σ γ·B and v = Σ β·B per
// column, and the epilogue forms r·(acc − ((μ − c)·u) + v with r the row's
// 1/√(var + eps) (= GEMM((x − μ)·r·γ + β)).  The shift keeps the one-pass
// variance and the subtraction well conditioned when |μ| ≫ σ.  γ (and β) for
// each K step ride in the stage behind B, loaded by DMA with it.
constexpr int waitcnt_vm(int n) { return lbr_waitcnt_vm(n); }

// NS: LDS stages of the K pipeline.  Step kt+NS−1 is in flight while step kt
// is consumed, so a grid that leaves one or two workgroups on a CU (nothing
// else to hide a load round trip) can take more stages.
// KB: the K step, 32 (DBK) or 64 floats: a row of a stage is KB/4 chunks of 16
// bytes, chunk c of row r stored at c ^ (r mod KB/4), and one DMA instruction
// fills 64/(KB/4) rows.  A 64-wide step halves the barriers and waits per K.
template <int TM, int TN, int WGM, int WGN, int OCC, bool HAS_BIAS, bool AHEADS, int NORM = 0, int NS = 2,
          int KB = DBK>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void gemm_dma_f32(GemmArgs g) {
    constexpr int NW = WGM * WGN;
    constexpr int CH = KB / 4;                  // 16-byte chunks per tile row
    constexpr int RPI = 64 / CH;                // tile rows per DMA instruction
    constexpr int FM = TM / WGM / 16, FN = TN / WGN / 16;
    constexpr int IA = TM / NW / RPI, IB = TN / NW / RPI;
    static_assert(IA * NW * RPI == TM && IB * NW * RPI == TN, "tile rows must split evenly over the waves");
    static_assert((CH == 8 || CH == 16) && FM * 16 * WGM == TM && FN * 16 * WGN == TN, "tile shape");
    static_assert((TM / NW) % 8 == 0 && (TN / NW) % 8 == 0, "each wave's DMA rows start at a multiple of 8");
    static_assert(!AHEADS || KB == DBK, "A in head layout takes the 32-wide K step");
    constexpr int GOFF = (TM + TN) * KB;        // γ, then β, of the step (norm prologue)
    constexpr int STAGE = GOFF + (NORM ? 2 * KB : 0);
    constexpr int NCC = CH / 4;                 // 16-wide K chunks per step
    static_assert(NS >= 2, "pipeline stages");
    // DMA instructions per wave per step: the A and B rows, plus the norm's γ
    // (and β) in wave 0
    constexpr int PER_STEP = IA + IB;
    constexpr int PER_STEP0 = IA + IB + (NORM == 1 ? 1 : NORM == 2 ? 2 : 0);
    static_assert((NS - 1) * PER_STEP0 <= 63, "vmcnt holds at most 63");
    __shared__ __attribute__((aligned(1024))) float lds[NS * STAGE];

    int tm, tn;
    tile_coords(g, tm, tn);
    const int m0 = tm * TM, n0 = tn * TN;
    const long long bz = blockIdx.z;
    const int M = g.M, N = g.N, K = g.K;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    // DMA sources: row clamped to the matrix (rows past the edge are never stored);
    // lane (dr, dp) lands at position dp of row `row` and fetches its logical chunk
    // dp ^ (row mod CH)
    const int dr = lane / CH, dp = lane % CH;
    unsigned offA[IA], offB[IB];
#pragma unroll
    for (int t = 0; t < IA; ++t) {
        const int row = wave * (TM / NW) + t * RPI + dr;
        const int sw = dp ^ (row & (CH - 1));
        const int m = min(m0 + row, M - 1);
        if (AHEADS) {
            // head layout: row m = (b, s) starts at ((b·aH)·aS + s)·ahd.  The lane's 4 columns
            // c = 4·(dp ^ dr) of the 32-wide K step lie in head c / ahd of the step (0 when ahd
            // is a multiple of 32; 0 or 1 for ahd = 16) at offset c % ahd; the step's first head
            // goes in the scalar offset (soffA below)
            const int b = m / g.aS, s = m - b * g.aS;
            const int c = sw * 4;
            offA[t] = (unsigned)(((b * g.aH) * g.aS + s) * g.ahd + (c / g.ahd) * g.aS * g.ahd + c % g.ahd) * 4u;
        } else {
            offA[t] = (unsigned)(m * K + sw * 4) * 4u;
        }
    }
#pragma unroll
    for (int t = 0; t < IB; ++t) {
        const int row = wave * (TN / NW) + t * RPI + dr;
        const int sw = dp ^ (row & (CH - 1));
        int brow = min(n0 + row, N - 1);
        if (g.gF) {
            // gated pair: tile column blocks of 16 alternate gate, up for the same
            // TN/2 output columns starting at tn·TN/2 (clamped to the last one)
            const int jb = row >> 4;
            const int o = min(tn * (TN / 2) + (jb >> 1) * 16 + (row & 15), g.gF - 1);
            brow = (jb & 1) ? (g.gbase ? 0 : g.gF) + o : g.gbase + o;
        }
        offB[t] = (unsigned)(brow * K + sw * 4) * 4u;
    }
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.A + bz * g.sA), (short)0, M * K * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.B + bz * g.sB), (short)0, N * K * 4, 0x00020000);
    __amdgpu_buffer_rsrc_t rg = rb, rbe = rb;
    if (NORM) {
        rg = __builtin_amdgcn_make_buffer_rsrc((void*)g.nw, (short)0, K * 4, 0x00020000);
        if (NORM == 2) rbe = __builtin_amdgcn_make_buffer_rsrc((void*)g.nb, (short)0, K * 4, 0x00020000);
    }
    auto issue = [&](int k0, float* st) {
        float* la = st + wave * (TM / NW) * KB;
        float* lb = st + TM * KB + wave * (TN / NW) * KB;
        // K step k0 of A: column k0 (row-major), or head k0 / ahd at offset k0 % ahd (head
        // layout; ahd is a multiple of the step, or divides it so the step starts a head)
        const unsigned soffA =
            AHEADS ? (unsigned)((k0 / g.ahd) * g.aS * g.ahd + k0 % g.ahd) * 4u : (unsigned)k0 * 4u;
#pragma unroll
        for (int t = 0; t < IA; ++t) dma16(ra, la + t * RPI * KB, offA[t], soffA);
#pragma unroll
        for (int t = 0; t < IB; ++t) dma16(rb, lb + t * RPI * KB, offB[t], (unsigned)k0 * 4u);
        if (NORM && wave == 0) {   // the step's KB γ (lanes 0 .. CH−1) and β (lanes CH .. 2CH−1, landing
                                   // KB floats after γ), 16 bytes a lane
            if (lane < CH) dma16(rg, st + GOFF, (unsigned)lane * 16u, (unsigned)k0 * 4u);
            if (NORM == 2 && lane >= CH && lane < 2 * CH)
                dma16(rbe, st + GOFF, (unsigned)(lane - CH) * 16u, (unsigned)k0 * 4u);
        }
    };

    floatx4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // fragment reads: the swizzle depends on the row only through fi (blocks start at multiples of 16)
    const int fi = lane & 15, kq = lane >> 4;
    int rdA[NCC], rdB[NCC];
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
        const int o = fi * KB + (((cc * 4 + kq) ^ (fi & (CH - 1))) * 4);
        rdA[cc] = wm * (TM / WGM) * KB + o;
        rdB[cc] = TM * KB + wn * (TN / WGN) * KB + o;
    }
    floatx4 fa[2][FM], fb[2][FN];
    // norm prologue state: per fragment row (lane row fi of block i) the shift
    // c and Σ over the lane's k, per fragment column (fi of block j) u and v
    float nc[FM], ns1[FM], ns2[FM], nu[FN], nv[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) nc[i] = ns1[i] = ns2[i] = 0.f;
#pragma unroll
    for (int j = 0; j < FN; ++j) nu[j] = nv[j] = 0.f;
    auto frags = [&](const float* st, int cc, floatx4* a, floatx4* b) {
#pragma unroll
        for (int i = 0; i < FM; ++i) a[i] = *reinterpret_cast<const floatx4*>(st + rdA[cc] + i * 16 * KB);
#pragma unroll
        for (int j = 0; j < FN; ++j) b[j] = *reinterpret_cast<const floatx4*>(st + rdB[cc] + j * 16 * KB);
        if (NORM) {   // k = step start + 16·cc + 4·kq + q for every fragment of the lane
            const floatx4 w = *reinterpret_cast<const floatx4*>(st + GOFF + cc * 16 + (lane >> 4) * 4);
            if (NORM == 1) {
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    ns2[i] += (a[i][0] * a[i][0] + a[i][1] * a[i][1]) + (a[i][2] * a[i][2] + a[i][3] * a[i][3]);
                    a[i] = a[i] * w;
                }
            } else {
                const floatx4 be = *reinterpret_cast<const floatx4*>(st + GOFF + KB + cc * 16 + (lane >> 4) * 4);
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const floatx4 d = a[i] - nc[i];
                    ns1[i] += (d[0] + d[1]) + (d[2] + d[3]);
                    ns2[i] += (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]);
                    a[i] = d * w;
                }
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    nu[j] += (w[0] * b[j][0] + w[1] * b[j][1]) + (w[2] * b[j][2] + w[3] * b[j][3]);
                    nv[j] += (be[0] * b[j][0] + be[1] * b[j][1]) + (be[2] * b[j][2] + be[3] * b[j][3]);
                }
            }
        }
    };
    auto mma = [&](const floatx4* a, const floatx4* b) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][q], b[j][q], acc[i][j], 0, 0, 0);
    };

    // K range of this workgroup (split ks of ksplit; kchunk is a multiple of KB)
    const int ks = blockIdx.y;
    const int kbeg = ks * g.kchunk;
    const int nk = (min(K, kbeg + g.kchunk) - kbeg) / KB;
    if (nk > 0) {
        // NS stages: steps 0 .. NS−1 issued up front; at the end of step kt, step
        // kt+1 must have landed while kt+2 .. kt+NS−1 may still be in flight, then
        // step kt+NS goes into the stage step kt leaves.  Steps past the last are
        // re-fetches of the last step into stages no later step reads, so a wave
        // always has the same number of DMA instructions per step outstanding and
        // fixed vmcnt thresholds hold (wave 0 issues the norm's γ/β DMAs too).
        if (NORM == 2) {   // each fragment row's shift, its first element: issued first, so it
                           // has landed whenever step 0 has (loads complete in order)
#pragma unroll
            for (int i = 0; i < FM; ++i)
                nc[i] = g.A[(long long)min(m0 + wm * (TM / WGM) + i * 16 + fi, M - 1) * K];
        }
#pragma unroll
        for (int st = 0; st < NS; ++st) issue(kbeg + min(st, nk - 1) * KB, lds + st * STAGE);
        if (wave == 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 1) * PER_STEP0));   // step 0 landed
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 1) * PER_STEP));
        __syncthreads();
        frags(lds, 0, fa[0], fb[0]);
        int cur = 0;
        for (int kt = 0; kt < nk - 1; ++kt) {
            const int nxt = cur + STAGE == NS * STAGE ? 0 : cur + STAGE;
#pragma unroll
            for (int cc = 0; cc < NCC; ++cc) {
                if (cc + 1 < NCC) {
                    frags(lds + cur, cc + 1, fa[(cc + 1) & 1], fb[(cc + 1) & 1]);
                } else {
                    __builtin_amdgcn_sched_barrier(0);
                    // step kt+1 landed (this wave's DMA) ...
                    if (wave == 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * PER_STEP0));
                    else __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * PER_STEP));
                    __syncthreads();   // ... and every wave's; stage cur fully read
                    issue(kbeg + min(kt + NS, nk - 1) * KB, lds + cur);
                    frags(lds + nxt, 0, fa[0], fb[0]);
                }
                mma(fa[cc & 1], fb[cc & 1]);
                if (cc + 1 < NCC) chunk_schedule<0, FM + FN, 4 * FM * FN>();
                else chunk_schedule<IA + IB, FM + FN, 4 * FM * FN>();
            }
            cur = nxt;
        }
#pragma unroll
        for (int cc = 0; cc < NCC; ++cc) {
            if (cc + 1 < NCC) frags(lds + cur, cc + 1, fa[(cc + 1) & 1], fb[(cc + 1) & 1]);
            mma(fa[cc & 1], fb[cc & 1]);
            if (cc + 1 < NCC) chunk_schedule<0, FM + FN, 4 * FM * FN>();
        }
        __builtin_amdgcn_s_waitcnt(0x3F70);   // no DMA may still target this workgroup's LDS at exit
    }

    const int rq = (lane >> 4) * 4, cl = lane & 15;
    const int mw = m0 + wm * (TM / WGM), nw = n0 + wn * (TN / WGN);
    if (NORM) {
        // whole rows: sum the four kq lanes of each row and column, then take
        // each accumulator row's factors from the lane that holds that row
        const float invK = 1.0f / K;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            ns2[i] += __shfl_xor(ns2[i], 16, 64);
            ns2[i] += __shfl_xor(ns2[i], 32, 64);
            if (NORM == 2) {
                ns1[i] += __shfl_xor(ns1[i], 16, 64);
                ns1[i] += __shfl_xor(ns1[i], 32, 64);
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j)
            if (NORM == 2) {
                nu[j] += __shfl_xor(nu[j], 16, 64);
                nu[j] += __shfl_xor(nu[j], 32, 64);
                nv[j] += __shfl_xor(nv[j], 16, 64);
                nv[j] += __shfl_xor(nv[j], 32, 64);
            }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            // per fragment row fi: RMS scale, or LayerNorm r and μ − c
            float f0, f1 = 0.f;
            if (NORM == 1) {
                f0 = 1.0f / sqrtf(ns2[i] * invK + g.neps);
            } else {
                const float dm = ns1[i] * invK;
                const float var = fmaxf(ns2[i] * invK - dm * dm, 0.f);
                f0 = 1.0f / sqrtf(var + g.neps);
                f1 = dm;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float sr = __shfl(f0, rq + r, 64);
                const float dr = NORM == 2 ? __shfl(f1, rq + r, 64) : 0.f;
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j][r] = NORM == 1 ? acc[i][j][r] * sr : sr * (acc[i][j][r] - dr * nu[j]) + nv[j];
            }
        }
    }
    if constexpr (TM == 64 && TN == 128 && WGM == 2 && WGN == 2 && !AHEADS && NORM == 0) {
        int p = -1;
        for (int q = 0; q < g.hp_parts; ++q)
            if (n0 >= g.hp_col[q] && n0 < g.hp_col[q] + g.hp_H[q] * TN) p = q;
        if (p >= 0) {
            // one head per tile: C (+ bias) through LDS, then each wavefront takes 16 rows,
            // two a pass, a row over 32 lanes of 4 columns each — the lanes, sums and
            // partner swaps of head_rows4 at HD = 128, so the values are the same bits
            constexpr int TS = TN + 4;
            static_assert(TM * TS <= NS * STAGE, "the tile fits in the stages");
            __syncthreads();   // every wavefront's last fragment reads are done
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int c = wn * (TN / WGN) + j * 16 + cl;
                const float bv = HAS_BIAS ? g.bias[n0 + c] : 0.f;
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        lds[(wm * (TM / WGM) + i * 16 + rq + r) * TS + c] =
                            HAS_BIAS ? (acc[i][j][r] + bv) : g.alpha * acc[i][j][r];
            }
            __syncthreads();
            const int H = g.hp_H[p], h = (n0 - g.hp_col[p]) / TN, S = g.hp_S;
            const int l = lane & 31, d = 4 * l;
            const bool norm = g.hp_flags & 1, rope = g.hp_flags & 2;
            const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 wv = norm ? *reinterpret_cast<const float4*>(g.hp_w[p] + d) : zero;
            const float* __restrict__ pbias = g.hp_b[p];
            const float4 pb = pbias ? *reinterpret_cast<const float4*>(pbias + h * TN + d) : zero;
            const float eps = g.hp_eps[p];
#pragma unroll 2
            for (int pass = 0; pass < TM / NW / 2; ++pass) {
                const int row = wave * (TM / NW) + 2 * pass + (lane >> 5);
                const int m = m0 + row, mc = min(m, M - 1);
                const int b = mc / S, s = mc - b * S;
                const float4 x = *reinterpret_cast<const float4*>(&lds[row * TS + d]);
                float4 v = x;
                if (pbias) {
                    v.x = v.x + pb.x;
                    v.y = v.y + pb.y;
                    v.z = v.z + pb.z;
                    v.w = v.w + pb.w;
                }
                float4 c4 = zero, s4 = zero;
                if (rope) {
                    const long long t = b * g.hp_tst[0] + s * g.hp_tst[1] + d;
                    c4 = *reinterpret_cast<const float4*>(g.hp_cos + t);
                    s4 = *reinterpret_cast<const float4*>(g.hp_sin + t);
                }
                const float4 y = lbr_head_row<32, TN>(v, norm, wv, eps, rope, c4, s4, lane);
                if (m < M)
                    *reinterpret_cast<float4*>(g.hp_out[p] + (((long long)b * H + h) * S + s) * TN + d) = y;
            }
            return;
        }
    }
    if (g.ksplit > 1) {
        float* __restrict__ Wp = g.W + ((long long)ks * gridDim.z + bz) * (long long)M * N;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = nw + j * 16 + cl;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = mw + i * 16 + rq + r;
                    if (m < M) Wp[(long long)m * N + n] = acc[i][j][r];
                }
        }
        return;
    }
    if (g.n_split) {
        // head scatter: the column fixes split, head, d and split bias; the
        // row fixes (b, s) = divmod(m, S), stepped from each 4-row group's first row
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = nw + j * 16 + cl;
            if (n >= N || n < g.col_begin[0] || n >= g.col_begin[g.n_split]) continue;
            int k = 0;
            while (k + 1 < g.n_split && n >= g.col_begin[k + 1]) ++k;
            const int c = n - g.col_begin[k];
            const int h = c / g.hd, d = c - h * g.hd;
            const float bv = HAS_BIAS ? g.bias[n] : 0.f;
            const bool has_sb = g.sbias[k] != nullptr;
            const float sb = has_sb ? g.sbias[k][c] : 0.f;
            const bool fr = (g.frag >> k) & 1;
            float* __restrict__ col = g.dst[k] + ((long long)h * g.S) * g.hd + (fr ? lbr_frag_offset(0, d, g.hd) : d);
            const long long bstride = (long long)g.Hs[k] * g.S * g.hd;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int mb = mw + i * 16 + rq;
                const int b0 = mb / g.S, s0 = mb - b0 * g.S;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (mb + r >= M) continue;
                    int b = b0, s = s0 + r;
                    while (s >= g.S) {   // r < 4: at most one step unless S < 4
                        s -= g.S;
                        ++b;
                    }
                    float v = HAS_BIAS ? (acc[i][j][r] + bv) : g.alpha * acc[i][j][r];
                    if (has_sb) v = v + sb;
                    col[b * bstride + (fr ? lbr_frag_offset(s, 0, g.hd) : (long long)s * g.hd)] = v;
                }
            }
        }
        return;
    }
    if (FN % 2 == 0 && g.gF) {   // tiles with an odd block count never take a gated pair
        // gated pair: blocks j (gate) and j+1 (up) of this wave hold the same 16
        // output columns; out = act(gate (+ gated bias))·up, rounded like the
        // unfused GEMM → SLICE → GATED_ACT chain
        const int F = g.gF;
        float* __restrict__ C = g.C + bz * (long long)M * F;
#pragma unroll
        for (int j = 0; j + 1 < FN; j += 2) {
            const int o = tn * (TN / 2) + ((wn * FN + j) >> 1) * 16 + cl;
            if (o >= F) continue;
            const float bg = HAS_BIAS ? g.bias[g.gbase + o] : 0.f;
            const float bu = HAS_BIAS ? g.bias[(g.gbase ? 0 : F) + o] : 0.f;
            const float gb = g.gbias ? g.gbias[o] : 0.f;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = mw + i * 16 + rq + r;
                    if (m >= M) continue;
                    float x = HAS_BIAS ? (acc[i][j][r] + bg) : g.alpha * acc[i][j][r];
                    const float u = HAS_BIAS ? (acc[i][j + 1][r] + bu) : g.alpha * acc[i][j + 1][r];
                    if (g.gbias) x = x + gb;
                    const float a = g.gact == 0 ? lbr_silu(x) : lbr_gelu_tanh(x);
                    C[(long long)m * F + o] = a * u;
                }
        }
        return;
    }
    float* __restrict__ C = g.C + bz * g.sC;
    const float* __restrict__ R = g.resid ? g.resid + bz * g.sC : nullptr;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = nw + j * 16 + cl;
        if (n >= N) continue;
        const float bv = HAS_BIAS ? g.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            float rv[4] = {0.f, 0.f, 0.f, 0.f};
            if (R) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = mw + i * 16 + rq + r;
                    if (m < M) rv[r] = R[(long long)m * N + n];
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = mw + i * 16 + rq + r;
                if (m >= M) continue;
                float v = HAS_BIAS ? (acc[i][j][r] + bv) : g.alpha * acc[i][j][r];
                if (R) v = v + rv[r];
                C[(long long)m * N + n] = lbr_act(g.act, v);   // a fused activation never comes with resid
            }
        }
    }
}

// ---------------------------------------------------------------- GEMV
// M == 1 (decode): the reference switches to sgemv here (executor.c:217).
// trans_b: one wavefront per output column, lanes stride over K.
template <bool VEC, bool HAS_BIAS>
__global__ __launch_bounds__(256) void gemv_t(GemmArgs g) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= g.N) return;
    const long long bz = blockIdx.y;
    const float* __restrict__ a = g.A + bz * g.sA;
    const float* __restrict__ b = g.B + bz * g.sB + (long long)n * g.K;
    float acc = 0.f;
    if (VEC) {
        const int k4 = g.K / 4;
        const float4* a4 = reinterpret_cast<const float4*>(a);
        const float4* b4 = reinterpret_cast<const float4*>(b);
        for (int k = lane; k < k4; k += 64) {
            const float4 x = a4[k], y = b4[k];
            acc += (x.x * y.x + x.y * y.y) + (x.z * y.z + x.w * y.w);
        }
    } else {
        for (int k = lane; k < g.K; k += 64) acc += a[k] * b[k];
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        float* c = g.C + bz * g.sC;
        c[n] = HAS_BIAS ? acc + g.bias[n] : g.alpha * acc;
    }
}

// B is [K, N]: one thread per output column, loop over K (coalesced over n).
template <bool HAS_BIAS>
__global__ __launch_bounds__(256) void gemv_n(GemmArgs g) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= g.N) return;
    const long long bz = blockIdx.y;
    const float* __restrict__ a = g.A + bz * g.sA;
    const float* __restrict__ b = g.B + bz * g.sB;
    float acc = 0.f;
    for (int k = 0; k < g.K; ++k) acc += a[k] * b[(long long)k * g.N + n];
    float* c = g.C + bz * g.sC;
    c[n] = HAS_BIAS ? acc + g.bias[n] : g.alpha * acc;
}

// Step::i: [0]=M [1]=N [2]=K [3]=batches [4]=trans_b [5]=fragment-major head splits [6]=has_bias
//          [7]=sA [8]=sB [9]=sC [10]=ksplit [11]=kchunk [12]=float4 reduce
//          [13]=1 (takes fused epilogues) [14]=DMA tile + 1 (0: gemm_mfma_f32)
//          [19..30] head scatter, [31] activation, [32..34] gated pair, [35..37] A in
//          head layout (see below) ; f[0] = alpha
GemmArgs make_args(const Step& s) {
    GemmArgs g;
    g.A = (const float*)s.in[0];
    g.B = (const float*)s.in[1];
    g.bias = (const float*)s.in[2];
    g.C = (float*)s.out;
    g.M = (int)s.i[0];
    g.N = (int)s.i[1];
    g.K = (int)s.i[2];
    g.sA = s.i[7];
    g.sB = s.i[8];
    g.sC = s.i[9];
    g.alpha = s.f[0];
    g.tiles_m = (g.M + BM - 1) / BM;
    g.tiles_n = (g.N + BN - 1) / BN;
    g.ksplit = s.i[10] > 1 ? (int)s.i[10] : 1;
    g.kchunk = g.ksplit > 1 ? (int)s.i[11] : g.K;
    g.W = (float*)s.ws;
    // fused epilogue: in[3] = resid (gated pair: the GATED_ACT bias);
    // i[19] = n_split, i[20..24] = col_begin, in[4..7] = dst, in[8..11] =
    // split biases, i[25..28] = heads per split, i[29] = hd, i[30] = S,
    // i[5] = splits stored fragment-major (bit k, set by the plan);
    // i[31] = act; i[32] = gated F, i[33] = gated act, i[34] = gate half's first column
    g.gF = (int)s.i[32];
    g.gact = (int)s.i[33];
    g.gbase = (int)s.i[34];
    g.resid = g.gF ? nullptr : (const float*)s.in[3];
    g.gbias = g.gF ? (const float*)s.in[3] : nullptr;
    g.n_split = (int)s.i[19];
    for (int k = 0; k < 5; ++k) g.col_begin[k] = (int)s.i[20 + k];
    for (int k = 0; k < 4; ++k) {
        g.dst[k] = (float*)s.in[4 + k];
        g.sbias[k] = (const float*)s.in[8 + k];
        g.Hs[k] = (int)s.i[25 + k];
    }
    g.hd = (int)s.i[29];
    g.S = (int)s.i[30];
    g.frag = (int)s.i[5];
    // i[18] = head prologue parts (0: none; see lbr_merge_gemm_head_prologue), i[20..23]
    // = their first columns and heads, i[24] = flags, i[25..26] = RoPE row strides over
    // b and s, i[30] = S; in[4..5] outputs, in[6..7] norm weights, in[8..9] cos / sin,
    // in[10..11] biases; f[2..3] eps
    g.hp_parts = (int)s.i[18];
    g.hp_flags = (int)s.i[24];
    g.hp_S = (int)s.i[30];
    for (int p = 0; p < 2; ++p) {
        g.hp_col[p] = (int)s.i[20 + p];
        g.hp_H[p] = (int)s.i[22 + p];
        g.hp_out[p] = (float*)s.in[4 + p];
        g.hp_w[p] = (const float*)s.in[6 + p];
        g.hp_b[p] = (const float*)s.in[10 + p];
        g.hp_eps[p] = s.f[2 + p];
    }
    g.hp_cos = (const float*)s.in[8];
    g.hp_sin = (const float*)s.in[9];
    g.hp_tst[0] = s.i[25];
    g.hp_tst[1] = s.i[26];
    g.act = (int)s.i[31];
    // i[35..37] = A in head layout [B, H, S, hd]: H, S, hd (0: row-major A)
    g.aH = (int)s.i[35];
    g.aS = (int)s.i[36];
    g.ahd = (int)s.i[37];
    // i[15] = norm prologue (LBR_NORM_*), i[38] / i[39] = its weight / bias, f[1] = eps
    g.nw = (const float*)(uintptr_t)s.i[38];
    g.nb = (const float*)(uintptr_t)s.i[39];
    g.neps = s.f[1];
    // i[16] = norm after the split-K reduce (LBR_NORM_*), i[17] = its form
    // (16·(1 wave / 2 block per row) + float4 per lane, + 256 when the K split
    // was made for the norm); in[4] output, in[5]
    // weight, in[6] LayerNorm bias, f[2] eps (the head-split fields are unused
    // then: i[19] = 0)
    g.nt_out = s.i[16] ? (float*)s.in[4] : nullptr;
    g.nt_w = s.i[16] ? (const float*)s.in[5] : nullptr;
    g.nt_b = s.i[16] ? (const float*)s.in[6] : nullptr;
    g.nt_eps = s.f[2];
    return g;
}

// C[i] = alpha·Σ_ks W[ks][i] (MATMUL) or Σ_ks W[ks][i] + bias[i % N]
// (MATMUL_ADD), summing the K ranges in increasing order; then the fused
// epilogue, if any (VEC only with no head scatter).
template <bool HAS_BIAS, bool VEC>
__global__ void splitk_reduce(GemmArgs g, long long total) {
#pragma clang fp contract(off)   // the same roundings as splitk_reduce_norm (no a·alpha + r fused)
    const float* __restrict__ W = g.W;
    const int N = g.N, ksplit = g.ksplit;
    if (VEC) {
        const long long t4 = total / 4;
        for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < t4;
             i += (long long)gridDim.x * blockDim.x) {
            float4 s = reinterpret_cast<const float4*>(W)[i];
            for (int k = 1; k < ksplit; ++k) {
                const float4 w = reinterpret_cast<const float4*>(W + (long long)k * total)[i];
                s.x += w.x; s.y += w.y; s.z += w.z; s.w += w.w;
            }
            if (HAS_BIAS) {
                const float4 b = reinterpret_cast<const float4*>(g.bias)[(i * 4 % N) / 4];
                s.x += b.x; s.y += b.y; s.z += b.z; s.w += b.w;
            } else {
                s.x *= g.alpha; s.y *= g.alpha; s.z *= g.alpha; s.w *= g.alpha;
            }
            if (g.act) {
                s.x = lbr_act(g.act, s.x); s.y = lbr_act(g.act, s.y);
                s.z = lbr_act(g.act, s.z); s.w = lbr_act(g.act, s.w);
            }
            if (g.resid) {
                const float4 r = reinterpret_cast<const float4*>(g.resid)[i];
                s.x = s.x + r.x; s.y = s.y + r.y; s.z = s.z + r.z; s.w = s.w + r.w;
            }
            reinterpret_cast<float4*>(g.C)[i] = s;
        }
    } else {
        const long long MN = (long long)g.M * N;
        for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
             i += (long long)gridDim.x * blockDim.x) {
            float s = W[i];
            for (int k = 1; k < ksplit; ++k) s += W[(long long)k * total + i];
            s = lbr_act(g.act, HAS_BIAS ? s + g.bias[i % N] : g.alpha * s);
            const long long bz = i / MN, r = i - bz * MN;
            epi_store(g, bz, (int)(r / N), (int)(r % N), s);
        }
    }
}

// The split-K reduce of a one-batch GEMM whose output row feeds a norm: one
// wavefront (WAVE, N ≤ 1024) or one 256-thread workgroup per row sums the K
// ranges, adds the bias (or scales by alpha) and the residual exactly as
// splitk_reduce does, writes C's row, and normalises it into nt_out with the
// norm kernels' own per-lane layout and sums (lbr_norm_row_wave / _block), so
// both outputs equal the unfused reduce + norm bit for bit.
template <bool HAS_BIAS, bool RMS, int VPL, bool WAVE>
__global__ __launch_bounds__(256) void splitk_reduce_norm(GemmArgs g) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    constexpr int STRIDE = WAVE ? 64 : 256;
    const int N = g.N, c4 = N / 4;
    const long long total = (long long)g.M * N;
    const long long row = WAVE ? (long long)blockIdx.x * 4 + (threadIdx.x >> 6) : (long long)blockIdx.x;
    if (row >= g.M) return;   // whole wavefronts (WAVE) or the whole workgroup leave
    const int t = WAVE ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
    const float4* __restrict__ W4 = reinterpret_cast<const float4*>(g.W);
    const float4* __restrict__ w4 = reinterpret_cast<const float4*>(g.nt_w);
    const float4* __restrict__ b4 = reinterpret_cast<const float4*>(g.nt_b);
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    const long long t4 = total / 4;
    // every load of the row's slots issues before the sums: the weight, bias and
    // residual, then the partials CH ranges at a time (clamped indices, so no
    // branch hides a load; values past the row or past ksplit are never added)
    constexpr int CH = 4;
    float4 v[VPL], wv[VPL], bv[VPL], bias[VPL], res[VPL];
    long long i4[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int idx = t + k * STRIDE;
        const int ic = min(idx, c4 - 1);
        i4[k] = row * c4 + ic;
        wv[k] = w4[ic];
        bv[k] = RMS ? zero : b4[ic];
        bias[k] = HAS_BIAS ? reinterpret_cast<const float4*>(g.bias)[ic] : zero;
        res[k] = g.resid ? reinterpret_cast<const float4*>(g.resid)[i4[k]] : zero;
    }
    for (int k0 = 0; k0 < g.ksplit; k0 += CH) {
        float4 w[VPL][CH];
#pragma unroll
        for (int k = 0; k < VPL; ++k)
#pragma unroll
            for (int q = 0; q < CH; ++q) w[k][q] = W4[min(k0 + q, g.ksplit - 1) * t4 + i4[k]];
#pragma unroll
        for (int k = 0; k < VPL; ++k)
#pragma unroll
            for (int q = 0; q < CH; ++q) {
                if (k0 + q >= g.ksplit) continue;
                if (k0 + q == 0) {
                    v[k] = w[k][q];
                } else {
                    v[k].x += w[k][q].x; v[k].y += w[k][q].y; v[k].z += w[k][q].z; v[k].w += w[k][q].w;
                }
            }
    }
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        float4 s = v[k];
        if (HAS_BIAS) {
            s.x += bias[k].x; s.y += bias[k].y; s.z += bias[k].z; s.w += bias[k].w;
        } else {
            s.x *= g.alpha; s.y *= g.alpha; s.z *= g.alpha; s.w *= g.alpha;
        }
        if (g.resid) {
            s.x = s.x + res[k].x; s.y = s.y + res[k].y; s.z = s.z + res[k].z; s.w = s.w + res[k].w;
        }
        const bool in = t + k * STRIDE < c4;
        if (in) reinterpret_cast<float4*>(g.C)[i4[k]] = s;
        v[k] = in ? s : zero;
        if (!in) wv[k] = bv[k] = zero;
    }
    float4* o4 = reinterpret_cast<float4*>(g.nt_out + row * N);
    if constexpr (WAVE) lbr_norm_row_wave<RMS, VPL>(v, wv, bv, o4, c4, N, g.nt_eps);
    else lbr_norm_row_block<RMS, VPL>(v, wv, bv, o4, c4, N, g.nt_eps, red);
}

template <bool HAS_BIAS, bool RMS>
void launch_splitk_reduce_norm(const Step& s, const GemmArgs& g, hipStream_t st) {
    const int form = ((int)s.i[17] >> 4) & 15, vpl = (int)s.i[17] & 15;
    if (form == 1) {
        const dim3 grid((unsigned)((g.M + 3) / 4));
        // lbr_merge_reduce_norm takes rows of more than 256 columns (2 or 4 float4 a lane)
        if (vpl == 2) hipLaunchKernelGGL((splitk_reduce_norm<HAS_BIAS, RMS, 2, true>), grid, dim3(256), 0, st, g);
        else hipLaunchKernelGGL((splitk_reduce_norm<HAS_BIAS, RMS, 4, true>), grid, dim3(256), 0, st, g);
    } else {
        const dim3 grid((unsigned)g.M);   // lbr_merge_reduce_norm takes rows of at most 4096 columns
        if (vpl == 2) hipLaunchKernelGGL((splitk_reduce_norm<HAS_BIAS, RMS, 2, false>), grid, dim3(256), 0, st, g);
        else hipLaunchKernelGGL((splitk_reduce_norm<HAS_BIAS, RMS, 4, false>), grid, dim3(256), 0, st, g);
    }
}

template <bool HAS_BIAS>
void launch_splitk_reduce(const Step& s, const GemmArgs& g, hipStream_t st) {
    if (s.i[16]) {
        if (s.i[16] == LBR_NORM_RMS) launch_splitk_reduce_norm<HAS_BIAS, true>(s, g, st);
        else launch_splitk_reduce_norm<HAS_BIAS, false>(s, g, st);
        return;
    }
    const long long total = (long long)g.M * g.N * s.i[3];
    const bool v4 = s.i[12] != 0 && g.n_split == 0 && (!g.resid || lbr_aligned(g.resid, 16));
    const unsigned blocks = lbr_grid(v4 ? total / 4 : total, 256, 4096);
    if (v4)
        hipLaunchKernelGGL((splitk_reduce<HAS_BIAS, true>), dim3(blocks), dim3(256), 0, st, g, total);
    else
        hipLaunchKernelGGL((splitk_reduce<HAS_BIAS, false>), dim3(blocks), dim3(256), 0, st, g, total);
}

template <bool TRANS_B, bool VEC, bool HAS_BIAS>
void launch_gemm_t(const Step& s, hipStream_t st) {
    GemmArgs g = make_args(s);
    if (g.M <= 0 || g.N <= 0) return;
    dim3 grid(g.tiles_m * g.tiles_n, g.ksplit, (unsigned)s.i[3]);
    hipLaunchKernelGGL((gemm_mfma_f32<TRANS_B, VEC, HAS_BIAS>), grid, dim3(NT), 0, st, g);
    if (g.ksplit > 1) launch_splitk_reduce<HAS_BIAS>(s, g, st);
}

template <int TM, int TN, int WGM, int WGN, int OCC, bool HAS_BIAS, bool AHEADS, int NORM = 0, int NS = 2,
          int KB = DBK>
void launch_gemm_dma(const Step& s, hipStream_t st) {
    GemmArgs g = make_args(s);
    if (g.M <= 0 || g.N <= 0) return;
    g.tiles_m = (g.M + TM - 1) / TM;
    // a gated pair's tile covers TN/2 output columns (TN/2 gate + TN/2 up columns of C)
    g.tiles_n = g.gF ? (g.gF + TN / 2 - 1) / (TN / 2) : (g.N + TN - 1) / TN;
    dim3 grid(g.tiles_m * g.tiles_n, g.ksplit, (unsigned)s.i[3]);
    hipLaunchKernelGGL((gemm_dma_f32<TM, TN, WGM, WGN, OCC, HAS_BIAS, AHEADS, NORM, NS, KB>), grid,
                       dim3(64 * WGM * WGN), 0, st, g);
    if (g.ksplit > 1) launch_splitk_reduce<HAS_BIAS>(s, g, st);
}

// Tile shapes of the DMA GEMM: (TM, TN), workgroups resident per CU (LDS
// and registers), and measured steady-state fraction of the fp32 MFMA peak.
struct DmaTile {
    int tm, tn, occ, waves, kb;   // kb: K step (32 or 64 floats)
    double eff;
    const char* name;
    bool model;    // chosen by choose_dma's model; the others only by measurement
                   // (gemm_dma_tune_candidates) or by name (LBR_GEMM_TILE)
    bool pairs;    // an even number of 16-column blocks per wavefront (gated pairs)
};
constexpr DmaTile kDmaTiles[] = {
    {256, 256, 1, 8, 32, 0.94, "256x256", true, true},   // 8 wavefronts (4×2), 128 KB LDS
    {128, 128, 2, 4, 32, 0.92, "128x128", true, true},   // 4 wavefronts (2×2), 64 KB LDS
    {128, 64, 3, 4, 32, 0.9225, "128x64", true, true},   // 4 wavefronts (2×2), 48 KB LDS
    {64, 128, 3, 4, 32, 0.9225, "64x128", true, true},
    {64, 64, 4, 4, 32, 0.90, "64x64", true, true},       // 4 wavefronts (2×2) of 32×32, 32 KB LDS
    // Small-grid tiles.  The model cannot rank them against 64×64 (its error on
    // GPT-2-width GEMMs, ~18%, exceeds their differences, 5–20%): a 32×48 grid
    // wins where 64×64 leaves a fractional last round (1024×2304×768: 40.6 µs
    // with 4 stages vs 43.8; 512×2304×768: 24.9 vs 31.0; 512×3072×768: 26.8 vs
    // 31.3) and loses where it leaves two 2-wavefront workgroups per CU
    // (1024×768×768: 24.8 vs 20.0), so they are picked by timing.
    {32, 48, 8, 2, 32, 0.80, "32x48", false, false},     // 2 wavefronts (2×1) of 16×48, 20 KB LDS
    {32, 48, 5, 2, 32, 0.80, "32x48s4", false, false},   // the same with 4 LDS stages, 40 KB
    {64, 96, 4, 4, 32, 0.85, "64x96", false, true},      // 4 wavefronts (4×1) of 16×96, 40 KB LDS
    // Narrow 4-wavefront tiles for GEMMs of 512-1024 rows and K = 768-3072 (MI355X,
    // GEMM steps of the GPT-2-shaped workloads): one or two rounds of small
    // workgroups, each wavefront with few MFMA blocks, beat the 2-wavefront 32×48 and
    // the 64×64 tiles there by 5-20% (e.g. 1024×2304×768: 35.0 µs for 32×96 against
    // 43.3 for 32×48s4).
    {32, 160, 3, 4, 32, 0.85, "32x160", false, false},   // 4 wavefronts (2×2) of 16×80, 48 KB LDS
    {64, 32, 6, 4, 32, 0.80, "64x32", false, false},     // 4 wavefronts (2×2) of 32×16, 24 KB LDS
    {32, 64, 6, 4, 32, 0.80, "32x64", false, true},      // 4 wavefronts (2×2) of 16×32, 24 KB LDS
    {32, 96, 5, 4, 32, 0.80, "32x96", false, false},     // 4 wavefronts (2×2) of 16×48, 32 KB LDS
    // 64-wide K steps (K a multiple of 64; not with A in head layout), for the
    // timing at plan creation: on the GPT-2-shaped GEMMs they run within ±4% of the
    // same tiles with 32-wide steps (1024×768×3072 unsplit: 47.7 µs for 32×96k64
    // against 51.5), so halving the barriers per K is not what those GEMMs lack
    {32, 96, 2, 4, 64, 0.80, "32x96k64", false, false},     // 64 KB LDS
    {64, 64, 2, 4, 64, 0.90, "64x64k64", false, true},      // 64 KB LDS
};
constexpr int kNumDmaTiles = sizeof(kDmaTiles) / sizeof(kDmaTiles[0]);

// Tile shape and number of K ranges for the DMA GEMM.  Time model: the
// busiest CU runs ceil(items / CUs) workgroups of TM·TN·kchunk MACs each
// at the tile's efficiency, in rounds of `occ` resident workgroups that
// each pay ~3 µs of first-load latency and epilogue; a K split adds writing
// and re-reading the partial sums at ~5 TB/s plus a reduction launch.  A CU
// left with fewer than 8 resident wavefronts (one 4-wavefront workgroup)
// runs its tile at 0.9 of the efficiency: measured on GPT-2's FFN2 (1024 ×
// 768 × 3072, 192 tiles of 64×64), one workgroup per CU took 55.8 µs, and
// four K ranges, three workgroups per CU, took 46.3 µs.
// LBR_GEMM_TILE (a tile name) and LBR_GEMM_KSPLIT override the choice.
void choose_dma(long long M, long long N, int K, long long batches, int cus, int* tile, int* ksplit, int* kchunk) {
    const double peak_cu = 157.3e12 / 256.0;
    const char* force_tile = getenv("LBR_GEMM_TILE");
    const char* force_ks = getenv("LBR_GEMM_KSPLIT");
    double best = 1e30;
    *tile = 1;
    *ksplit = 1;
    *kchunk = K;
    if (cus <= 0) cus = 256;
    for (int t = 0; t < kNumDmaTiles; ++t) {
        const DmaTile& d = kDmaTiles[t];
        if (force_tile ? strcmp(force_tile, d.name) != 0 : !d.model) continue;
        if (K % d.kb) continue;
        const long long tiles = ((M + d.tm - 1) / d.tm) * ((N + d.tn - 1) / d.tn) * batches;
        for (int s = 1; s <= 16; ++s) {
            const int chunk = ((K + s - 1) / s + d.kb - 1) / d.kb * d.kb;
            const int s_eff = (K + chunk - 1) / chunk;
            if (force_ks) {
                if (s != atoi(force_ks) || s_eff != s) continue;
            } else if (s > 1 && (chunk < 256 || s_eff != s)) {
                continue;
            }
            const long long per_cu = (tiles * s_eff + cus - 1) / cus;
            const double eff = std::min<long long>(per_cu, d.occ) * d.waves < 8 ? 0.9 * d.eff : d.eff;
            double t_s = (double)per_cu * 2.0 * d.tm * d.tn * chunk / (eff * peak_cu);
            t_s += (double)((per_cu + d.occ - 1) / d.occ) * 3e-6;   // per round: first DMA, epilogue
            if (s_eff > 1) t_s += (2.0 * s_eff + 1.0) * M * N * batches * 4.0 / 5e12 + 4e-6;
            if (s_eff > 1 && !force_ks) t_s *= 1.05;   // split only for a clear gain
            if (t_s < best) {
                best = t_s;
                *tile = t;
                *ksplit = s_eff;
                *kchunk = s_eff > 1 ? chunk : K;
            }
        }
    }
}

template <bool HAS_BIAS, bool AHEADS = false, int NORM = 0>
step_fn dma_launcher(int tile) {
    switch (tile) {
        case 0:   // the norm prologue's registers do not fit beside the 256×256 accumulators
            if constexpr (NORM != 0) return nullptr;
            else return launch_gemm_dma<256, 256, 4, 2, 1, HAS_BIAS, AHEADS, NORM>;
        case 1: return launch_gemm_dma<128, 128, 2, 2, 2, HAS_BIAS, AHEADS, NORM>;
        case 2: return launch_gemm_dma<128, 64, 2, 2, 3, HAS_BIAS, AHEADS, NORM>;
        case 3: return launch_gemm_dma<64, 128, 2, 2, 3, HAS_BIAS, AHEADS, NORM>;
        // the 5th argument is the waves per SIMD the registers must allow: the
        // LDS-bound workgroups per CU × wavefronts per workgroup / 4, rounded up
        case 5: return launch_gemm_dma<32, 48, 2, 1, 4, HAS_BIAS, AHEADS, NORM>;
        case 6: return launch_gemm_dma<32, 48, 2, 1, 2, HAS_BIAS, AHEADS, NORM, 4>;
        case 7: return launch_gemm_dma<64, 96, 4, 1, 3, HAS_BIAS, AHEADS, NORM>;
        case 8: return launch_gemm_dma<32, 160, 2, 2, 3, HAS_BIAS, AHEADS, NORM>;
        case 9: return launch_gemm_dma<64, 32, 2, 2, 4, HAS_BIAS, AHEADS, NORM>;
        case 10: return launch_gemm_dma<32, 64, 2, 2, 4, HAS_BIAS, AHEADS, NORM>;
        case 11: return launch_gemm_dma<32, 96, 2, 2, 4, HAS_BIAS, AHEADS, NORM>;
        // 64-wide K steps: no A-in-head-layout form
        case 12: if constexpr (AHEADS) return nullptr; else return launch_gemm_dma<32, 96, 2, 2, 2, HAS_BIAS, AHEADS, NORM, 2, 64>;
        case 13: if constexpr (AHEADS) return nullptr; else return launch_gemm_dma<64, 64, 2, 2, 2, HAS_BIAS, AHEADS, NORM, 2, 64>;
        default: return launch_gemm_dma<64, 64, 2, 2, 4, HAS_BIAS, AHEADS, NORM>;
    }
}

// Number of K ranges for a GEMM of `tiles` 128×128 output tiles: the tile
// grid alone leaves CUs idle or unevenly loaded when it is small (e.g.
// M=1024, N=2560 → 160 tiles on 256 CUs).  Model: a CU's time ∝ the work of
// the workgroups it receives ÷ its efficiency with that many resident
// workgroups (0.75 for one, 0.95 for two, 1 for three or more), plus the
// extra HBM traffic of writing and re-reading the partial sums.  Split only
// when that predicts at least a 5% gain.
int choose_ksplit(long long tiles, int K, long long MN, int cus, int* kchunk) {
    *kchunk = K;
    if (cus <= 0 || K < 1024) return 1;
    auto eff = [](long long n) { return n <= 1 ? 0.75 : n == 2 ? 0.95 : 1.0; };
    const double gemm_s = 2.0 * MN * (double)K / 130e12;           // per batch, at ~83% of peak
    auto cost = [&](int s, int chunk) {
        const long long n = (tiles * s + cus - 1) / cus;             // workgroups on the busiest CU
        const double t = (double)n * chunk / K / eff(n);
        const double extra = s > 1 ? (2.0 * s + 1.0) * MN * 4.0 / 8e12 / gemm_s : 0.0;
        return t * (1.0 + extra);
    };
    double best = cost(1, K);
    int best_s = 1, best_chunk = K;
    for (int s = 2; s <= 16; ++s) {
        const int chunk = ((K + s - 1) / s + BK - 1) / BK * BK;
        if (chunk < 256) break;
        const int s_eff = (K + chunk - 1) / chunk;
        const double c = cost(s_eff, chunk);
        if (c < best * 0.95 && c < best) {
            best = c;
            best_s = s_eff;
            best_chunk = chunk;
        }
    }
    *kchunk = best_chunk;
    return best_s;
}

template <bool VEC, bool HAS_BIAS>
void launch_gemv_t(const Step& s, hipStream_t st) {
    GemmArgs g = make_args(s);
    if (g.N <= 0) return;
    hipLaunchKernelGGL((gemv_t<VEC, HAS_BIAS>), dim3((g.N + 3) / 4, (unsigned)s.i[3]), dim3(256), 0, st, g);
}

template <bool HAS_BIAS>
void launch_gemv_n(const Step& s, hipStream_t st) {
    GemmArgs g = make_args(s);
    if (g.N <= 0) return;
    hipLaunchKernelGGL((gemv_n<HAS_BIAS>), dim3((g.N + 255) / 256, (unsigned)s.i[3]), dim3(256), 0, st, g);
}

void zero_k_fill(const Step& s, hipStream_t st);

// K == 0: C = bias (MATMUL_ADD) or 0.
__global__ void fill_rows(float* C, const float* bias, long long rows, int N) {
    const long long n = rows * N;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        C[i] = bias ? bias[i % N] : 0.f;
}

void zero_k_fill(const Step& s, hipStream_t st) {
    const long long rows = s.i[0] * s.i[3];
    const int N = (int)s.i[1];
    if (rows * N <= 0) return;
    hipLaunchKernelGGL(fill_rows, dim3(lbr_grid(rows * N, 256, 4096)), dim3(256), 0, st, (float*)s.out,
                       s.i[6] ? (const float*)s.in[2] : nullptr, rows, N);
}

}  // namespace

// Launcher of the DMA GEMM with its A operand in head layout (TRANSPOSE_GEMM
// fusion): `tile` = Step::i[14] − 1 of the decoded GEMM.
step_fn gemm_dma_heads_launcher(int tile, bool has_bias) {
    return has_bias ? dma_launcher<true, true>(tile) : dma_launcher<false, true>(tile);
}

// Launcher of the DMA GEMM with a norm prologue (NORM = LBR_NORM_RMS or
// LBR_NORM_LAYER), `tile` = Step::i[14] − 1 of the decoded GEMM; null for
// the 256×256 tile, which has no such variant.
step_fn gemm_dma_norm_launcher(int tile, bool has_bias, int norm) {
    if (norm == LBR_NORM_RMS) return has_bias ? dma_launcher<true, false, 1>(tile) : dma_launcher<false, false, 1>(tile);
    return has_bias ? dma_launcher<true, false, 2>(tile) : dma_launcher<false, false, 2>(tile);
}

// Launcher of a decoded or fused DMA GEMM step for another tile: the same
// family (norm prologue i[15], A in head layout i[35], or plain) and bias;
// null when the tile has no such variant or cannot hold a gated pair
// (i[32]: two 16-column blocks per wavefront).
static step_fn dma_family_launcher(const Step& s, int tile) {
    if (tile < 0 || tile >= kNumDmaTiles || (s.i[32] && !kDmaTiles[tile].pairs)) return nullptr;
    const bool bias = s.i[6] != 0;
    if (s.i[15]) return gemm_dma_norm_launcher(tile, bias, (int)s.i[15]);
    if (s.i[35]) return gemm_dma_heads_launcher(tile, bias);
    return bias ? dma_launcher<true>(tile) : dma_launcher<false>(tile);
}

// Two K ranges for an unsplit one-batch DMA GEMM step (K ≥ 512, ranges a
// multiple of its tile's K step): its reduce kernel can then take a norm of
// its output.  False leaves the step unchanged.
bool gemm_dma_split2(Step* s) {
    const long long M = s->i[0], N = s->i[1], K = s->i[2];
    if (!s->i[14] || s->i[10] > 1 || s->i[3] != 1 || K < 512 || s->i[19] || s->i[32] || s->i[15] || s->i[18])
        return false;
    const int kb = kDmaTiles[s->i[14] - 1].kb;
    const long long chunk = (K / 2 + kb - 1) / kb * kb;
    if ((K + chunk - 1) / chunk != 2) return false;
    s->i[10] = 2;
    s->i[11] = chunk;
    s->ws_bytes = (size_t)2 * M * N * sizeof(float);
    return true;
}

// Sets the number of K ranges of a one-batch DMA GEMM step to ks (ranges of
// whole K steps of its tile; the split-K reduce then carries the step's bias,
// activation, residual or head scatter).  False, leaving the step unchanged,
// for epilogues the reduce does not carry (gated pair, head prologue, norm
// prologue), for a reduce that already normalises, or when K does not split
// into ks such ranges.
bool gemm_dma_set_ksplit(Step* s, int ks) {
    const long long M = s->i[0], N = s->i[1], K = s->i[2];
    if (!s->i[14] || s->i[3] != 1 || ks < 1 || s->i[16] || s->i[32] || s->i[18] || s->i[15]) return false;
    if (ks == 1) {
        s->i[10] = 1;
        s->i[11] = K;
        s->ws_bytes = 0;
        return true;
    }
    const int kb = kDmaTiles[s->i[14] - 1].kb;
    const long long chunk = ((K + ks - 1) / ks + kb - 1) / kb * kb;
    if ((K + chunk - 1) / chunk != ks) return false;
    s->i[10] = ks;
    s->i[11] = chunk;
    s->ws_bytes = (size_t)ks * M * N * sizeof(float);
    return true;
}

bool gemm_dma_tile_pairs(int tile) {
    return tile >= 0 && tile < kNumDmaTiles && kDmaTiles[tile].pairs;
}

// The model's time for one K range on tile t (choose_dma's terms).
static double dma_model_time(long long M, long long N, int K, int cus, int t) {
    const DmaTile& d = kDmaTiles[t];
    const double peak_cu = 157.3e12 / 256.0;
    if (cus <= 0) cus = 256;
    const long long tiles = ((M + d.tm - 1) / d.tm) * ((N + d.tn - 1) / d.tn);
    const long long per_cu = (tiles + cus - 1) / cus;
    const double eff = std::min<long long>(per_cu, d.occ) * d.waves < 8 ? 0.9 * d.eff : d.eff;
    return (double)per_cu * 2.0 * d.tm * d.tn * K / (eff * peak_cu) + (double)((per_cu + d.occ - 1) / d.occ) * 3e-6;
}

int gemm_dma_tune_candidates(const Step& s, int* tiles, int cap) {
    int n = 0;
    if (!s.i[14] || s.i[10] > 1 || s.i[3] != 1) return 0;   // one batch, no K split
    // tiles the model prices at more than twice its best are not timed (the
    // 256×256 tile on a 1024-row GEMM, say): only near-ties need measuring
    auto usable = [&](int t) { return dma_family_launcher(s, t) && s.i[2] % kDmaTiles[t].kb == 0; };
    double best = 1e30;
    for (int t = 0; t < kNumDmaTiles; ++t)
        if (usable(t)) best = std::min(best, dma_model_time(s.i[0], s.i[1], (int)s.i[2], lbr_device_cus(), t));
    for (int t = 0; t < kNumDmaTiles && n < cap; ++t)
        if (usable(t) && dma_model_time(s.i[0], s.i[1], (int)s.i[2], lbr_device_cus(), t) <= 2.0 * best)
            tiles[n++] = t;
    return n;
}

extern "C" const char* lbr_gemm_tile_name(int tile) {
    return tile >= 0 && tile < kNumDmaTiles ? kDmaTiles[tile].name : "";
}

int gemm_dma_tile_by_name(const char* name) {
    for (int t = 0; t < kNumDmaTiles; ++t)
        if (name && strcmp(name, kDmaTiles[t].name) == 0) return t;
    return -1;
}

bool gemm_dma_retile(Step* s, int tile) {
    const step_fn run = dma_family_launcher(*s, tile);
    // the K ranges must stay whole steps of the new tile
    if (!run || s->i[2] % kDmaTiles[tile].kb || s->i[11] % kDmaTiles[tile].kb) return false;
    s->run = run;
    s->i[14] = tile + 1;
    return true;
}

// Byte ranges a one-batch DMA GEMM step writes: the head-split outputs, or C
// (M × gated F columns, or M × N).
int gemm_dma_written(const Step& s, void** ptr, size_t* bytes, int cap) {
    const long long M = s.i[0], N = s.i[1];
    int n = 0;
    if (s.i[18] > 0) {   // head-prologue epilogue: the parts' outputs, and C's other columns
        for (int p = 0; p < s.i[18] && p < 2 && n < cap; ++p) {
            ptr[n] = (void*)s.in[4 + p];
            bytes[n++] = (size_t)(M * s.i[22 + p] * 128) * sizeof(float);
        }
        if (n < cap) {
            ptr[n] = s.out;
            bytes[n++] = (size_t)(M * N) * sizeof(float);
        }
        return n;
    }
    if (s.i[19] > 0) {
        for (int k = 0; k < s.i[19] && k < 4 && n < cap; ++k) {
            ptr[n] = (void*)s.in[4 + k];
            bytes[n++] = (size_t)(M * s.i[25 + k] * s.i[29]) * sizeof(float);
        }
        return n;
    }
    if (cap < 1) return 0;
    ptr[0] = s.out;
    bytes[0] = (size_t)(M * (s.i[32] ? s.i[32] : N)) * sizeof(float);
    return 1;
}

// MATMUL extras [K, trans_b, b_is_2d, alpha_bits] (alpha_bits 0 ⇒ 1.0);
// MATMUL_ADD inputs [A, B, bias] with the same extras (executor.c:197-224,
// 312-346).  M == 1 goes to the GEMV kernels as in the reference.
int decode_matmul(const OpNode* n, Step* s) {
    const bool has_bias = n->op == OP_MATMUL_ADD;
    const int need = has_bias ? 3 : 2;
    if (n->n_inputs < need || !n->output || n->n_dims < 1) {
        lbr_set_error("matmul: expected %d inputs, an output and n_dims >= 1", need);
        return LBR_ERR_INVALID;
    }
    for (int i = 0; i < need; ++i)
        if (!n->inputs[i]) {
            lbr_set_error("matmul: input %d is null", i);
            return LBR_ERR_INVALID;
        }
    const int N = n->out_shape[n->n_dims - 1];
    const int K = n->extra[0];
    const int trans_b = n->extra[1] != 0;
    const int b_is_2d = n->extra[2] != 0;
    const float alpha = n->extra[3] ? node_extra_float(n, 3) : 1.0f;
    long long M, batches;
    if (b_is_2d) {
        M = node_leading(n);
        batches = 1;
    } else {
        if (n->n_dims < 2) {
            lbr_set_error("matmul: batched form needs n_dims >= 2");
            return LBR_ERR_INVALID;
        }
        M = n->out_shape[n->n_dims - 2];
        batches = 1;
        for (int i = 0; i < n->n_dims - 2; ++i) batches *= n->out_shape[i];
    }
    if (M > INT32_MAX || N < 0 || K < 0 || N > (1 << 30) || K > (1 << 30) || batches > 65535) {
        lbr_set_error("matmul: unsupported sizes M=%lld N=%d K=%d batches=%lld", M, N, K, batches);
        return LBR_ERR_UNSUPPORTED;
    }
    s->in[0] = n->inputs[0];
    s->in[1] = n->inputs[1];
    s->in[2] = has_bias ? n->inputs[2] : nullptr;
    s->out = n->output;
    s->i[0] = M;
    s->i[1] = N;
    s->i[2] = K;
    s->i[3] = batches;
    s->i[4] = trans_b;
    s->i[6] = has_bias;
    s->i[7] = M * (long long)K;
    s->i[8] = (long long)N * K;
    s->i[9] = M * (long long)N;
    s->f[0] = has_bias ? 1.0f : alpha;
    if (K == 0) {
        s->run = zero_k_fill;
        s->name = "matmul_k0";
        return LBR_OK;
    }
    if (M == 1) {
        if (trans_b) {
            const bool vec = K % 4 == 0 && lbr_aligned(n->inputs[0], 16) && lbr_aligned(n->inputs[1], 16);
            s->run = vec ? (has_bias ? launch_gemv_t<true, true> : launch_gemv_t<true, false>)
                         : (has_bias ? launch_gemv_t<false, true> : launch_gemv_t<false, false>);
            s->name = "gemv_t";
        } else {
            s->run = has_bias ? launch_gemv_n<true> : launch_gemv_n<false>;
            s->name = "gemv_n";
        }
        return LBR_OK;
    }
    const bool vec = lbr_aligned(n->inputs[0], 16) && lbr_aligned(n->inputs[1], 16) && K % 4 == 0 &&
                     (trans_b || N % 4 == 0);
    s->i[12] = (N % 4 == 0) && lbr_aligned(n->output, 16) && (!has_bias || lbr_aligned(n->inputs[2], 16));
    s->i[13] = 1;   // MFMA path: takes the fused epilogues of Step::in[3..11], i[19..27]
    // DMA kernel: B [N, K], K a multiple of its K step, 16-byte aligned rows, and
    // each batch's A and B addressable with 31-bit byte offsets.
    const char* force_tile = getenv("LBR_GEMM_TILE");
    const bool legacy = force_tile && strcmp(force_tile, "legacy") == 0;
    if (!legacy && trans_b && vec && K % DBK == 0 && M * K * 4 < (1LL << 31) && (long long)N * K * 4 < (1LL << 31)) {
        int tile = 1, ks = 1, kchunk = K;
        choose_dma(M, N, K, batches, lbr_device_cus(), &tile, &ks, &kchunk);
        s->i[10] = ks;
        s->i[11] = kchunk;
        s->i[14] = tile + 1;
        s->ws_bytes = ks > 1 ? (size_t)ks * batches * M * N * sizeof(float) : 0;
        s->run = has_bias ? dma_launcher<true>(tile) : dma_launcher<false>(tile);
        s->name = "gemm_dma_f32_nt";
        return LBR_OK;
    }
    {
        const long long tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN) * batches;
        int kchunk = K;
        const int ks = choose_ksplit(tiles, K, M * (long long)N, lbr_device_cus(), &kchunk);
        s->i[10] = ks;
        s->i[11] = kchunk;
        s->ws_bytes = ks > 1 ? (size_t)ks * batches * M * N * sizeof(float) : 0;
    }
    if (trans_b) {
        if (vec) s->run = has_bias ? launch_gemm_t<true, true, true> : launch_gemm_t<true, true, false>;
        else s->run = has_bias ? launch_gemm_t<true, false, true> : launch_gemm_t<true, false, false>;
        s->name = "gemm_mfma_f32_nt";
    } else {
        if (vec) s->run = has_bias ? launch_gemm_t<false, true, true> : launch_gemm_t<false, true, false>;
        else s->run = has_bias ? launch_gemm_t<false, false, true> : launch_gemm_t<false, false, false>;
        s->name = "gemm_mfma_f32_nn";
    }
    return LBR_OK;
}
