// shape.hip — data-movement kernels for gfx950: RESHAPE copy, TRANSPOSE
// (2-D and N-D swapaxes), SLICE, CAT and EMBEDDING.
//
// Semantics follow csrc/executor.c:228-292 and csrc/ops/shape.c:8-138:
//   RESHAPE   memcpy when input != output (only dispatched for an external
//             input, runtime/executor/compiled.py:52-54)
//   TRANSPOSE 2-D [rows, cols] → [cols, rows]; N-D swapaxes described by
//             extras [outer, A, middle, B, inner] (ops.py:149-171)
//   SLICE     extras [outer, orig_dim, start, len, inner] (ops.py:310-329)
//   CAT       extras [dim, size_0, size_1, ...] (ops.py:275-279)
//   EMBEDDING ids int64 [rows], table [vocab, dim] (shape.c:72-79)
//
// All of them are byte copies; the kernels pick the widest word (16, 8, 4 or
// 1 bytes) that every chunk size and base address allows, so the common
// fp32 cases move 16 bytes per lane with contiguous runs per wavefront.
#include "lbr_device.h"

namespace {

constexpr int CB = 256;
constexpr unsigned COPY_GRID_CAP = 256 * 16;

template <typename W>
__global__ void copy_words(const W* __restrict__ src, W* __restrict__ dst, long long n) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// Strided row copy: for o in [0, rows): dst[o*dst_stride + w] = src[o*src_stride + w],
// w in [0, row_words).  All quantities in words of type W.
template <typename W>
__global__ void copy_rows(const W* __restrict__ src, W* __restrict__ dst, long long rows, long long row_words,
                          long long src_stride, long long dst_stride) {
    const long long n = rows * row_words;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const long long o = i / row_words, w = i % row_words;
        dst[o * dst_stride + w] = src[o * src_stride + w];
    }
}

// N-D swapaxes: out[o][b][m][a][w] = in[o][a][m][b][w]; w counts words of a
// chunk of `inner` elements.
template <typename W>
__global__ void swapaxes_kernel(const W* __restrict__ src, W* __restrict__ dst, long long outer, long long A,
                                long long mid, long long B, long long chunk_words) {
    const long long n = outer * A * mid * B * chunk_words;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        long long r = i;
        const long long w = r % chunk_words; r /= chunk_words;
        const long long a = r % A; r /= A;
        const long long m = r % mid; r /= mid;
        const long long b = r % B; r /= B;
        const long long o = r;
        const long long src_idx = ((((o * A + a) * mid + m) * B + b) * chunk_words) + w;
        dst[i] = src[src_idx];
    }
}

// 2-D transpose through a 32x33 LDS tile (element type T of 4 or 8 bytes).
template <typename T>
__global__ __launch_bounds__(256) void transpose2d(const T* __restrict__ a, T* __restrict__ out, int rows, int cols) {
    __shared__ T tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int k = ty; k < 32; k += 8) {
        const int r = by + k, c = bx + tx;
        if (r < rows && c < cols) tile[k][tx] = a[(long long)r * cols + c];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int c = bx + k, r = by + tx;  // out[c][r]
        if (r < rows && c < cols) out[(long long)c * rows + r] = tile[tx][k];
    }
}

// CAT: one launch, blockIdx.y selects the input.
struct CatParams {
    const void* src[MAX_INPUTS];
    long long row_words[MAX_INPUTS];   // words per outer row of input k
    long long dst_off[MAX_INPUTS];     // word offset of input k inside an output row
    long long dst_row_words;           // words per outer row of the output
    long long outer;
};

template <typename W>
__global__ void cat_kernel(W* __restrict__ dst, CatParams p) {
    const int k = blockIdx.y;
    const W* __restrict__ src = reinterpret_cast<const W*>(p.src[k]);
    const long long rw = p.row_words[k];
    const long long n = p.outer * rw;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const long long o = i / rw, w = i % rw;
        dst[o * p.dst_row_words + p.dst_off[k] + w] = src[i];
    }
}

// EMBEDDING: out[r][:] = table[ids[r]][:].  Ids outside [0, vocab) would read
// outside the table; they produce a zero row instead.
__global__ void embedding_kernel(const long long* __restrict__ ids, const float* __restrict__ table,
                                 float* __restrict__ out, long long rows, int dim, long long vocab) {
    const long long r = blockIdx.x;
    if (r >= rows) return;
    const long long id = ids[r];
    const bool ok = id >= 0 && id < vocab;
    for (int j = threadIdx.x; j < dim; j += blockDim.x) out[r * dim + j] = ok ? table[id * dim + j] : 0.0f;
}

int word_size(long long bytes_a, long long bytes_b, const void* p, const void* q, long long extra_bytes = 16) {
    const int cands[4] = {16, 8, 4, 1};
    for (int w : cands) {
        if (bytes_a % w == 0 && bytes_b % w == 0 && extra_bytes % w == 0 && lbr_aligned(p, w) && lbr_aligned(q, w))
            return w;
    }
    return 1;
}

// ---- launchers ----
// copy: i[0] = words, i[1] = word size
void launch_copy(const Step& s, hipStream_t st) {
    const long long n = s.i[0];
    if (n <= 0) return;
    const unsigned g = lbr_grid(n, CB, COPY_GRID_CAP);
    switch (s.i[1]) {
        case 16: hipLaunchKernelGGL(copy_words<uint4>, dim3(g), dim3(CB), 0, st, (const uint4*)s.in[0], (uint4*)s.out, n); break;
        case 8: hipLaunchKernelGGL(copy_words<uint2>, dim3(g), dim3(CB), 0, st, (const uint2*)s.in[0], (uint2*)s.out, n); break;
        case 4: hipLaunchKernelGGL(copy_words<uint32_t>, dim3(g), dim3(CB), 0, st, (const uint32_t*)s.in[0], (uint32_t*)s.out, n); break;
        default: hipLaunchKernelGGL(copy_words<uint8_t>, dim3(g), dim3(CB), 0, st, (const uint8_t*)s.in[0], (uint8_t*)s.out, n); break;
    }
}

// rows: i[0] rows, i[1] row_words, i[2] src_stride, i[3] dst_stride (words), i[4] word size
void launch_rows(const Step& s, hipStream_t st) {
    const long long rows = s.i[0], rw = s.i[1];
    if (rows * rw <= 0) return;
    const unsigned g = lbr_grid(rows * rw, CB, COPY_GRID_CAP);
    switch (s.i[4]) {
        case 16: hipLaunchKernelGGL(copy_rows<uint4>, dim3(g), dim3(CB), 0, st, (const uint4*)s.in[0], (uint4*)s.out, rows, rw, s.i[2], s.i[3]); break;
        case 8: hipLaunchKernelGGL(copy_rows<uint2>, dim3(g), dim3(CB), 0, st, (const uint2*)s.in[0], (uint2*)s.out, rows, rw, s.i[2], s.i[3]); break;
        case 4: hipLaunchKernelGGL(copy_rows<uint32_t>, dim3(g), dim3(CB), 0, st, (const uint32_t*)s.in[0], (uint32_t*)s.out, rows, rw, s.i[2], s.i[3]); break;
        default: hipLaunchKernelGGL(copy_rows<uint8_t>, dim3(g), dim3(CB), 0, st, (const uint8_t*)s.in[0], (uint8_t*)s.out, rows, rw, s.i[2], s.i[3]); break;
    }
}

// swapaxes: i[0..3] outer, A, mid, B; i[4] chunk words; i[5] word size
void launch_swapaxes(const Step& s, hipStream_t st) {
    const long long n = s.i[0] * s.i[1] * s.i[2] * s.i[3] * s.i[4];
    if (n <= 0) return;
    const unsigned g = lbr_grid(n, CB, COPY_GRID_CAP);
    switch (s.i[5]) {
        case 16: hipLaunchKernelGGL(swapaxes_kernel<uint4>, dim3(g), dim3(CB), 0, st, (const uint4*)s.in[0], (uint4*)s.out, s.i[0], s.i[1], s.i[2], s.i[3], s.i[4]); break;
        case 8: hipLaunchKernelGGL(swapaxes_kernel<uint2>, dim3(g), dim3(CB), 0, st, (const uint2*)s.in[0], (uint2*)s.out, s.i[0], s.i[1], s.i[2], s.i[3], s.i[4]); break;
        case 4: hipLaunchKernelGGL(swapaxes_kernel<uint32_t>, dim3(g), dim3(CB), 0, st, (const uint32_t*)s.in[0], (uint32_t*)s.out, s.i[0], s.i[1], s.i[2], s.i[3], s.i[4]); break;
        default: hipLaunchKernelGGL(swapaxes_kernel<uint8_t>, dim3(g), dim3(CB), 0, st, (const uint8_t*)s.in[0], (uint8_t*)s.out, s.i[0], s.i[1], s.i[2], s.i[3], s.i[4]); break;
    }
}

// 2-D: i[0] rows, i[1] cols, i[2] elem size (4 or 8)
void launch_transpose2d(const Step& s, hipStream_t st) {
    const int rows = (int)s.i[0], cols = (int)s.i[1];
    if (rows <= 0 || cols <= 0) return;
    dim3 grid((cols + 31) / 32, (rows + 31) / 32);
    if (s.i[2] == 8)
        hipLaunchKernelGGL(transpose2d<uint2>, grid, dim3(256), 0, st, (const uint2*)s.in[0], (uint2*)s.out, rows, cols);
    else
        hipLaunchKernelGGL(transpose2d<uint32_t>, grid, dim3(256), 0, st, (const uint32_t*)s.in[0], (uint32_t*)s.out, rows, cols);
}

// cat: Step::i[0] = word size, i[1] = n_inputs, i[2] outer, i[3] dst_row_words,
// i[4+k] row_words[k], i[16+k] dst_off[k]
void launch_cat(const Step& s, hipStream_t st) {
    CatParams p;
    const int nin = (int)s.i[1];
    long long maxw = 0;
    for (int k = 0; k < MAX_INPUTS; ++k) {
        p.src[k] = k < nin ? s.in[k] : nullptr;
        p.row_words[k] = k < nin ? s.i[4 + k] : 0;
        p.dst_off[k] = k < nin ? s.i[16 + k] : 0;
        if (k < nin && p.row_words[k] > maxw) maxw = p.row_words[k];
    }
    p.outer = s.i[2];
    p.dst_row_words = s.i[3];
    if (p.outer * maxw <= 0 || nin <= 0) return;
    dim3 grid(lbr_grid(p.outer * maxw, CB, 2048), nin);
    switch (s.i[0]) {
        case 16: hipLaunchKernelGGL(cat_kernel<uint4>, grid, dim3(CB), 0, st, (uint4*)s.out, p); break;
        case 8: hipLaunchKernelGGL(cat_kernel<uint2>, grid, dim3(CB), 0, st, (uint2*)s.out, p); break;
        case 4: hipLaunchKernelGGL(cat_kernel<uint32_t>, grid, dim3(CB), 0, st, (uint32_t*)s.out, p); break;
        default: hipLaunchKernelGGL(cat_kernel<uint8_t>, grid, dim3(CB), 0, st, (uint8_t*)s.out, p); break;
    }
}

void launch_embedding(const Step& s, hipStream_t st) {
    if (s.i[0] <= 0) return;
    hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)s.i[0]), dim3(256), 0, st, (const long long*)s.in[0],
                       (const float*)s.in[1], (float*)s.out, s.i[0], (int)s.i[1], s.i[2]);
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
    if (n->elem_size <= 0) {
        lbr_set_error("op %d: elem_size %d", n->op, n->elem_size);
        return LBR_ERR_INVALID;
    }
    return LBR_OK;
}

void noop(const Step&, hipStream_t) {}

}  // namespace

int decode_reshape(const OpNode* n, Step* s) {
    int rc = need(n, 1);
    if (rc) return rc;
    s->in[0] = n->inputs[0];
    s->out = n->output;
    if (n->inputs[0] == n->output) {  // alias: nothing to do
        s->run = noop;
        s->name = "reshape_alias";
        return LBR_OK;
    }
    const long long bytes = node_total(n) * n->elem_size;
    const int w = word_size(bytes, bytes, n->inputs[0], n->output);
    s->i[0] = bytes / w;
    s->i[1] = w;
    s->run = launch_copy;
    s->name = "reshape_copy";
    return LBR_OK;
}

int decode_transpose(const OpNode* n, Step* s) {
    int rc = need(n, 1);
    if (rc) return rc;
    s->in[0] = n->inputs[0];
    s->out = n->output;
    if (n->n_dims == 2) {
        if (n->elem_size != 4 && n->elem_size != 8) {
            lbr_set_error("transpose2d: elem_size %d", n->elem_size);
            return LBR_ERR_UNSUPPORTED;
        }
        if (n->extra[0] < 0 || n->extra[1] < 0 || (long long)n->extra[0] * n->extra[1] != node_total(n)) {
            lbr_set_error("transpose2d: %d x %d does not match the output's %lld elements", n->extra[0],
                          n->extra[1], node_total(n));
            return LBR_ERR_INVALID;
        }
        s->i[0] = n->extra[0];
        s->i[1] = n->extra[1];
        s->i[2] = n->elem_size;
        s->run = launch_transpose2d;
        s->name = "transpose2d";
        return LBR_OK;
    }
    const long long outer = n->extra[0], A = n->extra[1], mid = n->extra[2], B = n->extra[3], inner = n->extra[4];
    if (!lbr_sizes_match(n, {outer, A, mid, B, inner})) {
        lbr_set_error("transpose: extents %lld x %lld x %lld x %lld x %lld do not match the output's %lld elements",
                      outer, A, mid, B, inner, node_total(n));
        return LBR_ERR_INVALID;
    }
    const long long chunk = inner * n->elem_size;
    const int w = word_size(chunk, chunk, n->inputs[0], n->output);
    s->i[0] = outer;
    s->i[1] = A;
    s->i[2] = mid;
    s->i[3] = B;
    s->i[4] = chunk / w;
    s->i[5] = w;
    s->run = launch_swapaxes;
    s->name = "transpose_swapaxes";
    return LBR_OK;
}

int decode_slice(const OpNode* n, Step* s) {
    int rc = need(n, 1);
    if (rc) return rc;
    const long long outer = n->extra[0], orig = n->extra[1], start = n->extra[2], len = n->extra[3],
                    inner = n->extra[4];
    const long long es = n->elem_size;
    if (start < 0 || len < 0 || start + len > orig) {
        lbr_set_error("slice: start %lld len %lld outside dim %lld", start, len, orig);
        return LBR_ERR_INVALID;
    }
    if (!lbr_sizes_match(n, {outer, len, inner})) {
        lbr_set_error("slice: %lld x %lld x %lld does not match the output's %lld elements", outer, len, inner,
                      node_total(n));
        return LBR_ERR_INVALID;
    }
    const long long src_stride = orig * inner * es, dst_stride = len * inner * es, copy = len * inner * es;
    const char* src = (const char*)n->inputs[0] + start * inner * es;
    const int w = word_size(src_stride, dst_stride, src, n->output, copy);
    s->in[0] = src;
    s->out = n->output;
    s->i[0] = outer;
    s->i[1] = copy / w;
    s->i[2] = src_stride / w;
    s->i[3] = dst_stride / w;
    s->i[4] = w;
    s->run = launch_rows;
    s->name = "slice";
    return LBR_OK;
}

int decode_cat(const OpNode* n, Step* s) {
    int rc = need(n, n->n_inputs);
    if (rc) return rc;
    const int nin = n->n_inputs;
    if (nin < 1 || nin > MAX_INPUTS || nin + 1 > MAX_DIMS) {
        lbr_set_error("cat: %d inputs", nin);
        return LBR_ERR_INVALID;
    }
    const int dim = n->extra[0];
    if (dim < 0 || dim >= n->n_dims) {
        lbr_set_error("cat: dim %d outside the output's %d dims", dim, n->n_dims);
        return LBR_ERR_INVALID;
    }
    long long outer = 1, inner = 1;
    for (int i = 0; i < dim; ++i) outer *= n->out_shape[i];
    for (int i = dim + 1; i < n->n_dims; ++i) inner *= n->out_shape[i];
    const long long es = n->elem_size;
    long long total_dim = 0;
    for (int k = 0; k < nin; ++k) {
        if (n->extra[1 + k] < 0) {
            lbr_set_error("cat: input %d has a negative extent", k);
            return LBR_ERR_INVALID;
        }
        total_dim += n->extra[1 + k];
    }
    if (total_dim != n->out_shape[dim]) {
        lbr_set_error("cat: the inputs' extents sum to %lld, the output's dim %d is %d", total_dim, dim,
                      n->out_shape[dim]);
        return LBR_ERR_INVALID;
    }
    // widest word every segment allows
    int w = 16;
    for (;;) {
        bool ok = lbr_aligned(n->output, w) && (total_dim * inner * es) % w == 0;
        for (int k = 0; k < nin && ok; ++k)
            ok = lbr_aligned(n->inputs[k], w) && (n->extra[1 + k] * inner * es) % w == 0;
        if (ok || w == 1) break;
        w /= 2;
    }
    s->out = n->output;
    s->i[0] = w;
    s->i[1] = nin;
    s->i[2] = outer;
    s->i[3] = total_dim * inner * es / w;
    long long off = 0;
    for (int k = 0; k < nin; ++k) {
        s->in[k] = n->inputs[k];
        s->i[4 + k] = n->extra[1 + k] * inner * es / w;
        s->i[16 + k] = off;
        off += s->i[4 + k];
    }
    s->n_in = nin;
    s->run = launch_cat;
    s->name = "cat";
    return LBR_OK;
}

// EMBEDDING: inputs [ids (int64), table], extra[0] = embed_dim (executor.c:284-292).
// extra[1] must carry the table's row count (the host layer writes it; the
// reference packer leaves it 0) so ids can be bounds-checked on the device.
int decode_embedding(const OpNode* n, Step* s) {
    int rc = need(n, 2);
    if (rc) return rc;
    if (n->extra[1] <= 0) {
        lbr_set_error("embedding: extra[1] must hold the table row count");
        return LBR_ERR_INVALID;
    }
    if (n->extra[0] < 0 || n->extra[0] != node_last_dim(n)) {
        lbr_set_error("embedding: embed_dim %d is not the output's last dim %d", n->extra[0], node_last_dim(n));
        return LBR_ERR_INVALID;
    }
    s->i[2] = n->extra[1];
    s->in[0] = n->inputs[0];
    s->in[1] = n->inputs[1];
    s->out = n->output;
    s->i[0] = node_leading(n);
    s->i[1] = n->extra[0];
    s->run = launch_embedding;
    s->name = "embedding";
    return LBR_OK;
}
