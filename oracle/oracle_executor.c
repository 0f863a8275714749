/*
 * oracle_executor.c — TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of the reference compiled executor (csrc/executor.c and
 * the non-Apple branches of csrc/ops/{matmul,attn,norm,elementwise,reduce,
 * shape}.c), over the same OpNode ABI
 * (include/lbr_executor.h ≙ csrc/runtime.h).  It is the checker the GPU
 * library is compared against, and the CPU baseline bench.py reports.  It is
 * never linked into, loaded by, or called from the product path.
 *
 * The reference links cblas_sgemm / cblas_sgemv (OpenBLAS on Linux,
 * csrc/Makefile:10-13); neither the library nor a cblas.h exists in this
 * image, so the reference cannot be built here.  The BLAS contract
 * (row-major C = alpha·A·op(B) + beta·C, csrc/ops/matmul.c:19-79) is restated
 * by oracle_sgemm below: a cache-blocked, OpenMP-threaded loop nest with fp32
 * accumulation.  Like any BLAS its summation order is its own, so parity with
 * the reference at this boundary is tolerance-based, as in the reference's own
 * tests (tests/test_backends.py:20-48, atol 1e-4).
 *
 * Each function cites the reference lines it restates.  Differences from the
 * reference, all confined to undefined or unbuildable corners:
 *   - the batch·head loops of attention run in parallel (the reference's
 *     PARALLEL_FOR is serial on Linux, csrc/ops.h:56-57); each slice owns
 *     its own scratch slice exactly as in the reference, so results do not
 *     depend on the thread count;
 *   - 2-D TRANSPOSE honours elem_size 8 (the reference kernel is fp32-only,
 *     csrc/ops/shape.c:8-14).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "../include/lbr_executor.h"

#define FLASH_SEQ_THRESHOLD 256  /* executor.c:23, attn.c:111, ops.py:429 */
#define FLASH_BR 128             /* attn.c:106 */
#define FLASH_BC 256             /* attn.c:107 */

static char g_oracle_err[256];
const char* oracle_last_error(void) { return g_oracle_err; }

/* ------------------------------------------------------------------ helpers
 * executor.c:30-48 */
static long node_total(const OpNode* n) {
    long t = 1;
    for (int i = 0; i < n->n_dims; i++) t *= n->out_shape[i];
    return t;
}
static long node_leading(const OpNode* n) {
    long r = 1;
    for (int i = 0; i < n->n_dims - 1; i++) r *= n->out_shape[i];
    return r;
}
static float extra_f(const OpNode* n, int idx) {
    union { int i; float f; } u;
    u.i = n->extra[idx];
    return u.f;
}

/* ------------------------------------------------------------------ sgemm
 * Restates the cblas_sgemm contract used by matmul.c:19-40 and attn.c:32-61,
 * 153-222: row-major, A [M,K] (lda), op(B) = B [K,N] (ldb) or Bᵀ with B
 * [N,K] (ldb), C [M,N] (ldc); C = alpha·A·op(B) + beta·C. */
#define GB_M 64
#define GB_N 64
#define GB_K 256

static void sgemm_block(int trans_b, int i0, int i1, int j0, int j1, int K, float alpha,
                        const float* A, int lda, const float* B, int ldb, float beta, float* C, int ldc) {
    /* beta pass first (as BLAS: C = beta·C, then += alpha·A·op(B)) */
    for (int i = i0; i < i1; i++)
        for (int j = j0; j < j1; j++) C[(long)i * ldc + j] = beta == 0.0f ? 0.0f : beta * C[(long)i * ldc + j];
    float acc[GB_M][GB_N];
    for (int k0 = 0; k0 < K; k0 += GB_K) {
        const int k1 = k0 + GB_K < K ? k0 + GB_K : K;
        for (int i = i0; i < i1; i++)
            for (int j = j0; j < j1; j++) acc[i - i0][j - j0] = 0.0f;
        if (trans_b) {
            for (int i = i0; i < i1; i++) {
                const float* a = A + (long)i * lda;
                for (int j = j0; j < j1; j++) {
                    const float* b = B + (long)j * ldb;
                    float s = 0.0f;
#pragma omp simd reduction(+ : s)
                    for (int k = k0; k < k1; k++) s += a[k] * b[k];
                    acc[i - i0][j - j0] = s;
                }
            }
        } else {
            for (int i = i0; i < i1; i++) {
                const float* a = A + (long)i * lda;
                float* row = acc[i - i0];
                for (int k = k0; k < k1; k++) {
                    const float av = a[k];
                    const float* b = B + (long)k * ldb;
#pragma omp simd
                    for (int j = j0; j < j1; j++) row[j - j0] += av * b[j];
                }
            }
        }
        for (int i = i0; i < i1; i++)
            for (int j = j0; j < j1; j++) C[(long)i * ldc + j] += alpha * acc[i - i0][j - j0];
    }
}

static void oracle_sgemm(int threaded, int trans_b, int M, int N, int K, float alpha, const float* A, int lda,
                         const float* B, int ldb, float beta, float* C, int ldc) {
    const int bm = (M + GB_M - 1) / GB_M, bn = (N + GB_N - 1) / GB_N;
    const long nblk = (long)bm * bn;
    if (threaded) {
#pragma omp parallel for schedule(dynamic, 1)
        for (long t = 0; t < nblk; t++) {
            const int i0 = (int)(t / bn) * GB_M, j0 = (int)(t % bn) * GB_N;
            sgemm_block(trans_b, i0, i0 + GB_M < M ? i0 + GB_M : M, j0, j0 + GB_N < N ? j0 + GB_N : N, K, alpha,
                        A, lda, B, ldb, beta, C, ldc);
        }
    } else {
        for (long t = 0; t < nblk; t++) {
            const int i0 = (int)(t / bn) * GB_M, j0 = (int)(t % bn) * GB_N;
            sgemm_block(trans_b, i0, i0 + GB_M < M ? i0 + GB_M : M, j0, j0 + GB_N < N ? j0 + GB_N : N, K, alpha,
                        A, lda, B, ldb, beta, C, ldc);
        }
    }
}

/* kernel_matmul_ab (matmul.c:19-40): batched loop over sgemm */
static void k_matmul_ab(const float* a, const float* b, float* out, int M, int N, int K, int batches, int trans_b,
                        float alpha, float beta) {
    const int ldb = trans_b ? K : N;
    const long as = (long)M * K, bs = (long)N * K, cs = (long)M * N;
    for (int i = 0; i < batches; i++)
        oracle_sgemm(1, trans_b, M, N, K, alpha, a + i * as, K, b + i * bs, ldb, beta, out + i * cs, N);
}

/* kernel_matmul_gemv (matmul.c:64-79): y = alpha·op(B)·a + beta·y per batch.
 * trans_b: B [N,K] → y[n] = Σ_k B[n][k]·a[k]; else B [K,N] → y[n] = Σ_k B[k][n]·a[k] */
static void k_matmul_gemv(const float* a, const float* b, float* out, int N, int K, int batches, int trans_b,
                          float alpha, float beta) {
    for (int bi = 0; bi < batches; bi++) {
        const float* B = b + (long)bi * K * N;
        const float* x = a + (long)bi * K;
        float* y = out + (long)bi * N;
#pragma omp parallel for schedule(static)
        for (int n = 0; n < N; n++) {
            float s = 0.0f;
            if (trans_b)
                for (int k = 0; k < K; k++) s += B[(long)n * K + k] * x[k];
            else
                for (int k = 0; k < K; k++) s += B[(long)k * N + n] * x[k];
            y[n] = alpha * s + (beta == 0.0f ? 0.0f : beta * y[n]);
        }
    }
}

/* ------------------------------------------------------------------ elementwise
 * csrc/ops/elementwise.c (non-Apple paths) */
static float gelu_tanh(float x) { /* elementwise.c:185-190 */
    return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}
static float silu(float x) { return x / (1.0f + expf(-x)); } /* elementwise.c:211 */

static void unary(int op, const float* x, float* out, long n, float s) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (long i = 0; i < n; i++) {
        const float v = x[i];
        float r = v;
        switch (op) {
            case OP_RELU: r = v > 0.0f ? v : 0.0f; break;       /* 23-27 */
            case OP_EXP: r = expf(v); break;                    /* 66-70 */
            case OP_TANH: r = tanhf(v); break;                  /* 154-158 */
            case OP_POW: r = powf(v, s); break;                 /* 143-147 */
            case OP_GELU: r = gelu_tanh(v); break;              /* 167-191 */
            case OP_RSQRT: r = 1.0f / sqrtf(v); break;          /* 196-198 */
            case OP_SILU: r = silu(v); break;                   /* 203-205 */
            case OP_NEG: r = -v; break;                         /* 210-212 */
            case OP_COS: r = cosf(v); break;                    /* 217-219 */
            case OP_SIN: r = sinf(v); break;                    /* 224-226 */
        }
        out[i] = r;
    }
}

static float binop(int op, float a, float b) { /* shape.c:42-47 operator codes */
    switch (op) {
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        default: return a / b;
    }
}

/* kernel_broadcast_binop (shape.c:32-62): odometer over the output shape */
static void k_broadcast(const float* a, const float* b, float* out, const int* as, const int* bs, const int* shape,
                        int ndim, int op) {
    long total = 1;
    for (int d = 0; d < ndim; d++) total *= shape[d];
    int coords[MAX_DIMS] = {0};
    long ao = 0, bo = 0;
    for (long i = 0; i < total; i++) {
        out[i] = binop(op, a[ao], b[bo]);
        for (int d = ndim - 1; d >= 0; d--) {
            coords[d]++;
            ao += as[d];
            bo += bs[d];
            if (coords[d] < shape[d]) break;
            ao -= (long)coords[d] * as[d];
            bo -= (long)coords[d] * bs[d];
            coords[d] = 0;
        }
    }
}

static void dispatch_broadcast(const OpNode* n, int base, int op) { /* executor.c:86-94 */
    const int nd = n->extra[base];
    k_broadcast(n->inputs[0], n->inputs[1], n->output, &n->extra[base + 1], &n->extra[base + 1 + nd],
                &n->extra[base + 1 + 2 * nd], nd, op);
}

static void d_add(const OpNode* n) { /* executor.c:96-117 */
    const long t = node_total(n);
    const float* a = n->inputs[0];
    float* o = n->output;
    switch (n->extra[0]) {
        case 2: {
            const float s = extra_f(n, 1);
            for (long i = 0; i < t; i++) o[i] = a[i] + s;
            break;
        }
        case 1: {
            const float* b = n->inputs[1];
            for (long i = 0; i < t; i++) o[i] = a[i] + b[i];
            break;
        }
        case 3: dispatch_broadcast(n, 1, 0); break;
        default: { /* kernel_add (elementwise.c:9-16): M rows × N bias */
            const int N = n->out_shape[n->n_dims - 1];
            const float* b = n->inputs[1];
            const long M = t / N;
            for (long i = 0; i < M; i++)
                for (int j = 0; j < N; j++) o[i * N + j] = a[i * N + j] + b[j];
        }
    }
}

static void d_sub_mul_div(const OpNode* n, int op) { /* executor.c:119-168 */
    const long t = node_total(n);
    const float* a = n->inputs[0];
    float* o = n->output;
    switch (n->extra[0]) {
        case 1: {
            const float s = extra_f(n, 1);
            for (long i = 0; i < t; i++) o[i] = binop(op, a[i], s);
            break;
        }
        case 2: dispatch_broadcast(n, 1, op); break;
        default: {
            const float* b = n->inputs[1];
            for (long i = 0; i < t; i++) o[i] = binop(op, a[i], b[i]);
        }
    }
}

/* ------------------------------------------------------------------ reductions
 * reduce.c:8-36, 78-97 */
static void d_reduce(const OpNode* n, int is_max) { /* executor.c:172-186 */
    const int axis = n->extra[0], axis_size = n->extra[1];
    int outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= n->out_shape[i];
    for (int i = axis; i < n->n_dims; i++) inner *= n->out_shape[i];
    const float* x = n->inputs[0];
    float* out = n->output;
    for (int o = 0; o < outer; o++)
        for (int j = 0; j < inner; j++) {
            float acc = is_max ? -FLT_MAX : 0.0f;
            for (int a = 0; a < axis_size; a++) {
                const float v = x[((long)o * axis_size + a) * inner + j];
                if (is_max) { if (v > acc) acc = v; }
                else acc += v;
            }
            out[(long)o * inner + j] = acc;
        }
}

static void k_softmax(const float* x, float* out, long rows, int cols) { /* reduce.c:78-97 */
    for (long i = 0; i < rows; i++) {
        const float* r = x + i * cols;
        float* o = out + i * cols;
        float mx = r[0];
        for (int j = 1; j < cols; j++) if (r[j] > mx) mx = r[j];
        float sum = 0.0f;
        for (int j = 0; j < cols; j++) { o[j] = expf(r[j] - mx); sum += o[j]; }
        for (int j = 0; j < cols; j++) o[j] /= sum;
    }
}

/* ------------------------------------------------------------------ norms
 * norm.c:47-64 (LayerNorm), 100-107 (RMSNorm) */
static void k_layernorm(const float* x, const float* g, const float* b, float* out, long rows, int cols, float eps) {
#pragma omp parallel for schedule(static) if (rows > 64)
    for (long i = 0; i < rows; i++) {
        const float* r = x + i * cols;
        float* o = out + i * cols;
        float sum = 0.0f;
        for (int j = 0; j < cols; j++) sum += r[j];
        const float mean = sum / cols;
        float var = 0.0f;
        for (int j = 0; j < cols; j++) { const float d = r[j] - mean; o[j] = d; var += d * d; }
        const float inv_std = 1.0f / sqrtf(var / cols + eps);
        for (int j = 0; j < cols; j++) o[j] = o[j] * inv_std * g[j] + b[j];
    }
}

static void k_rmsnorm(const float* x, const float* w, float* out, long rows, int cols, float eps) {
#pragma omp parallel for schedule(static) if (rows > 64)
    for (long i = 0; i < rows; i++) {
        const float* r = x + i * cols;
        float* o = out + i * cols;
        float ss = 0.0f;
        for (int j = 0; j < cols; j++) ss += r[j] * r[j];
        const float scale = 1.0f / sqrtf(ss / cols + eps);
        for (int j = 0; j < cols; j++) o[j] = r[j] * scale * w[j];
    }
}

/* ------------------------------------------------------------------ attention
 * attn.c:26-80 (standard) and 121-253 (flash, non-Apple branches) */
static void attention_slice(const float* Q, const float* K, const float* V, float* O, float* S_, const float* mask,
                            int S, int D, float scale, int causal) {
    oracle_sgemm(0, 1, S, S, D, scale, Q, D, K, D, 0.0f, S_, S);
    if (mask) {
        const long ss = (long)S * S;
        for (long i = 0; i < ss; i++) S_[i] += mask[i];
    } else if (causal) {
        for (int i = 0; i < S; i++)
            for (int j = i + 1; j < S; j++) S_[(long)i * S + j] = -INFINITY;
    }
    k_softmax(S_, S_, S, S);
    oracle_sgemm(0, 0, S, D, S, 1.0f, S_, S, V, D, 0.0f, O, D);
}

static void attention_flash_slice(const float* Q, const float* K, const float* V, float* O, float* scratch, int S,
                                  int D, float scale, int causal) {
    for (int qi = 0; qi < S; qi += FLASH_BR) {
        const int br = qi + FLASH_BR <= S ? FLASH_BR : S - qi;
        const float* Qb = Q + (long)qi * D;
        float* Ob = O + (long)qi * D;
        float m[FLASH_BR], l[FLASH_BR];
        for (int r = 0; r < br; r++) { m[r] = -FLT_MAX; l[r] = 0.0f; }
        for (int r = 0; r < br; r++)
            for (int d = 0; d < D; d++) Ob[(long)r * D + d] = 0.0f;
        for (int kj = 0; kj < S; kj += FLASH_BC) {
            const int bc = kj + FLASH_BC <= S ? FLASH_BC : S - kj;
            if (causal && kj > qi + br - 1) break;                 /* attn.c:147-148 */
            oracle_sgemm(0, 1, br, bc, D, scale, Qb, D, K + (long)kj * D, D, 0.0f, scratch, bc);
            if (causal && kj + bc > qi) {                          /* attn.c:161-171 */
                for (int r = 0; r < br; r++) {
                    const int last_valid = qi + r - kj;
                    if (last_valid < bc - 1) {
                        const int start = last_valid < 0 ? 0 : last_valid + 1;
                        for (int c = start; c < bc; c++) scratch[(long)r * bc + c] = -INFINITY;
                    }
                }
            }
            for (int r = 0; r < br; r++) {                         /* attn.c:194-213 */
                float* Sr = scratch + (long)r * bc;
                float* Or = Ob + (long)r * D;
                float mt = Sr[0];
                for (int c = 1; c < bc; c++) if (Sr[c] > mt) mt = Sr[c];
                const float m_new = m[r] > mt ? m[r] : mt;
                const float corr = expf(m[r] - m_new);
                l[r] *= corr;
                for (int d = 0; d < D; d++) Or[d] *= corr;
                float ln = 0.0f;
                for (int c = 0; c < bc; c++) { const float p = expf(Sr[c] - m_new); Sr[c] = p; ln += p; }
                l[r] += ln;
                m[r] = m_new;
            }
            oracle_sgemm(0, 0, br, D, bc, 1.0f, scratch, bc, V + (long)kj * D, D, 1.0f, Ob, D);
        }
        for (int r = 0; r < br; r++) {                             /* attn.c:229-233 */
            const float inv_l = 1.0f / l[r];
            for (int d = 0; d < D; d++) Ob[(long)r * D + d] *= inv_l;
        }
    }
}

static void d_attention(const OpNode* n) { /* executor.c:371-397 */
    const int S = n->extra[0], D = n->extra[1], causal = n->extra[2], has_mask = n->extra[3];
    const int group = n->extra[4] > 0 ? n->extra[4] : 1;
    int bh_n = 1;
    for (int i = 0; i < n->n_dims - 2; i++) bh_n *= n->out_shape[i];
    const float* mask = has_mask ? n->inputs[3] : NULL;
    float* scratch = has_mask ? n->inputs[4] : n->inputs[3];
    const float scale = 1.0f / sqrtf((float)D);
    const long slice = (long)S * D;
    const float *Q = n->inputs[0], *K = n->inputs[1], *V = n->inputs[2];
    float* O = n->output;
    if (S > FLASH_SEQ_THRESHOLD && !has_mask) {
#pragma omp parallel for schedule(dynamic, 1)
        for (int bh = 0; bh < bh_n; bh++) {
            const int kv = bh / group;
            attention_flash_slice(Q + bh * slice, K + kv * slice, V + kv * slice, O + bh * slice,
                                  scratch + (long)bh * FLASH_BR * FLASH_BC, S, D, scale, causal);
        }
    } else {
        /* The planner sizes scratch for the flash kernel whenever S > 256
         * (ops.py:437-459) but a mask forces the standard kernel, which needs
         * S·S floats per slice: the reference overruns its scratch there.
         * The oracle takes its own buffer in that case. */
        const long sps = (long)S * S;
        float* own = NULL;
        if (S > FLASH_SEQ_THRESHOLD) {
            own = malloc((size_t)bh_n * sps * sizeof(float));
            if (!own) {
                snprintf(g_oracle_err, sizeof g_oracle_err, "oracle: out of memory for attention scratch");
                return;
            }
            scratch = own;
        }
#pragma omp parallel for schedule(dynamic, 1)
        for (int bh = 0; bh < bh_n; bh++) {
            const int kv = bh / group;
            attention_slice(Q + bh * slice, K + kv * slice, V + kv * slice, O + bh * slice, scratch + bh * sps,
                            mask ? mask + bh * sps : NULL, S, D, scale, causal);
        }
        free(own);
    }
}

/* ------------------------------------------------------------------ matmul dispatch
 * executor.c:197-224 (MATMUL), 312-346 (MATMUL_ADD: bias prefill, beta = 1,
 * alpha fixed to 1) */
static void d_matmul(const OpNode* n, int with_bias) {
    const int N = n->out_shape[n->n_dims - 1];
    const int K = n->extra[0], trans_b = n->extra[1], b_is_2d = n->extra[2];
    const float alpha = with_bias ? 1.0f : (n->extra[3] ? extra_f(n, 3) : 1.0f);
    int M, batches;
    if (b_is_2d) {
        M = (int)node_leading(n);
        batches = 1;
    } else {
        M = n->out_shape[n->n_dims - 2];
        batches = 1;
        for (int i = 0; i < n->n_dims - 2; i++) batches *= n->out_shape[i];
    }
    float beta = 0.0f;
    if (with_bias) {
        const float* bias = n->inputs[2];
        float* out = n->output;
        const long rows = (long)M * batches;
        for (long r = 0; r < rows; r++)
            for (int c = 0; c < N; c++) out[r * N + c] = bias[c];
        beta = 1.0f;
    }
    if (M == 1)
        k_matmul_gemv(n->inputs[0], n->inputs[1], n->output, N, K, batches, trans_b, alpha, beta);
    else
        k_matmul_ab(n->inputs[0], n->inputs[1], n->output, M, N, K, batches, trans_b, alpha, beta);
}

/* ------------------------------------------------------------------ shape ops
 * executor.c:228-292, shape.c */
static void d_transpose(const OpNode* n) {
    const int es = n->elem_size;
    if (n->n_dims == 2) { /* shape.c:8-14 */
        const int rows = n->extra[0], cols = n->extra[1];
        const char* a = n->inputs[0];
        char* o = n->output;
        for (int i = 0; i < rows; i++)
            for (int j = 0; j < cols; j++) memcpy(o + ((long)j * rows + i) * es, a + ((long)i * cols + j) * es, es);
        return;
    }
    const int outer = n->extra[0], A = n->extra[1], mid = n->extra[2], B = n->extra[3], inner = n->extra[4];
    const char* x = n->inputs[0];
    char* out = n->output;
    const long chunk = (long)inner * es;
    for (int o = 0; o < outer; o++)
        for (int b = 0; b < B; b++)
            for (int m = 0; m < mid; m++)
                for (int a = 0; a < A; a++) {
                    const long in_off = ((((long)o * A + a) * mid + m) * B + b) * inner;
                    const long out_off = ((((long)o * B + b) * mid + m) * A + a) * inner;
                    memcpy(out + out_off * es, x + in_off * es, chunk);
                }
}

static void d_slice(const OpNode* n) { /* shape.c:92-106 */
    const int outer = n->extra[0], orig = n->extra[1], start = n->extra[2], len = n->extra[3], inner = n->extra[4];
    const long es = n->elem_size;
    const long ss = (long)orig * inner * es, ds = (long)len * inner * es, cb = ds, so = (long)start * inner * es;
    const char* src = n->inputs[0];
    char* dst = n->output;
    for (int o = 0; o < outer; o++) memcpy(dst + o * ds, src + o * ss + so, cb);
}

static void d_cat(const OpNode* n) { /* executor.c:272-282, shape.c:121-138 */
    const int dim = n->extra[0];
    long outer = 1, inner = 1;
    for (int i = 0; i < dim; i++) outer *= n->out_shape[i];
    for (int i = dim + 1; i < n->n_dims; i++) inner *= n->out_shape[i];
    const long es = n->elem_size;
    long total = 0;
    for (int k = 0; k < n->n_inputs; k++) total += n->extra[1 + k];
    for (long o = 0; o < outer; o++) {
        long dst = o * total * inner;
        for (int k = 0; k < n->n_inputs; k++) {
            const long chunk = (long)n->extra[1 + k] * inner;
            const long src = o * n->extra[1 + k] * inner;
            memcpy((char*)n->output + dst * es, (const char*)n->inputs[k] + src * es, chunk * es);
            dst += chunk;
        }
    }
}

static void d_embedding(const OpNode* n) { /* shape.c:72-79 */
    const int dim = n->extra[0];
    const long rows = node_leading(n);
    const int64_t* ids = n->inputs[0];
    const float* table = n->inputs[1];
    float* out = n->output;
    for (long i = 0; i < rows; i++) memcpy(out + i * dim, table + ids[i] * dim, (size_t)dim * sizeof(float));
}

/* ------------------------------------------------------------------ execute
 * executor.c:458-467; returns nonzero instead of abort() on an unknown op */
int oracle_execute(OpNode* nodes, int n_nodes) {
    for (int i = 0; i < n_nodes; i++) {
        OpNode* n = &nodes[i];
        switch (n->op) {
            case OP_RELU: case OP_EXP: case OP_TANH: case OP_GELU: case OP_RSQRT:
            case OP_SILU: case OP_NEG: case OP_COS: case OP_SIN:
                unary(n->op, n->inputs[0], n->output, node_total(n), 0.0f);
                break;
            case OP_POW: unary(OP_POW, n->inputs[0], n->output, node_total(n), extra_f(n, 0)); break;
            case OP_ADD: d_add(n); break;
            case OP_SUB: d_sub_mul_div(n, 1); break;
            case OP_MUL: d_sub_mul_div(n, 2); break;
            case OP_DIV: d_sub_mul_div(n, 3); break;
            case OP_MAX: d_reduce(n, 1); break;
            case OP_SUM: d_reduce(n, 0); break;
            case OP_SOFTMAX: k_softmax(n->inputs[0], n->output, node_leading(n), n->out_shape[n->n_dims - 1]); break;
            case OP_MATMUL: d_matmul(n, 0); break;
            case OP_MATMUL_ADD: d_matmul(n, 1); break;
            case OP_RESHAPE:
                if (n->inputs[0] != n->output) memcpy(n->output, n->inputs[0], (size_t)node_total(n) * n->elem_size);
                break;
            case OP_TRANSPOSE: d_transpose(n); break;
            case OP_SLICE: d_slice(n); break;
            case OP_CAT: d_cat(n); break;
            case OP_EMBEDDING: d_embedding(n); break;
            case OP_LAYERNORM:
                k_layernorm(n->inputs[0], n->inputs[1], n->inputs[2], n->output, node_leading(n),
                            n->out_shape[n->n_dims - 1], extra_f(n, 0));
                break;
            case OP_RMSNORM:
                k_rmsnorm(n->inputs[0], n->inputs[1], n->output, node_leading(n), n->out_shape[n->n_dims - 1],
                          extra_f(n, 0));
                break;
            case OP_FUSED_BIAS_RELU: { /* elementwise.c:82-90 */
                const int N = n->out_shape[n->n_dims - 1];
                const long M = node_leading(n);
                const float *a = n->inputs[0], *b = n->inputs[1];
                float* o = n->output;
                for (long r = 0; r < M; r++)
                    for (int c = 0; c < N; c++) {
                        const float v = a[r * N + c] + b[c];
                        o[r * N + c] = v > 0.0f ? v : 0.0f;
                    }
                break;
            }
            case OP_GATED_ACT: { /* executor.c:354-369, elementwise.c:96-136 */
                const int has_bias = n->extra[0], act = n->extra[1];
                const int N = n->out_shape[n->n_dims - 1];
                const long M = node_leading(n);
                const float* x = n->inputs[0];
                const float* up = has_bias ? n->inputs[2] : n->inputs[1];
                const float* bias = has_bias ? n->inputs[1] : NULL;
                float* o = n->output;
#pragma omp parallel for schedule(static) if (M * N > 65536)
                for (long r = 0; r < M; r++)
                    for (int c = 0; c < N; c++) {
                        const float v = x[r * N + c] + (has_bias ? bias[c] : 0.0f);
                        const float g = act == 0 ? silu(v) : gelu_tanh(v);
                        o[r * N + c] = g * up[r * N + c];
                    }
                break;
            }
            case OP_ATTENTION: d_attention(n); break;
            default:
                snprintf(g_oracle_err, sizeof g_oracle_err, "oracle: unknown op %d (node %d)", n->op, i);
                return 1;
        }
    }
    return 0;
}

/* Number of OpenMP threads the oracle runs with. */
int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
