// Query x centroid tables, score gather and block-VQ reconstruction.
//
//   ss_build_lut      LUT[r][b][c] = q'[r][b-block] . C[b][c]   (codec.py:553-573)
//   ss_score_gather   S[r][t] = sum_b LUT[r][b][idx[t][b]]      (kernels.py:59-77)
//   ss_dequantize_blockvq  k_hat from indices, inverse-permuted (codec.py:516-543)
// These back the score-only API (attention_scores / the two-pass SDPA
// fallback) and the dequantised-key views; the decode hot path builds its
// LUT inside the fused kernel instead.
#include "ss_common.hpp"

namespace ss {

// grid (n_rows, n_blocks), block 256: thread c computes LUT[row][b][c].
__global__ void __launch_bounds__(256)
    build_lut_kernel(const void *q, int q_dtype, int64_t q_row_stride, const int32_t *perm,
                     float scale, const float *centroids, int n_blocks, int n_centroids,
                     int block_dim, float *lut) {
    extern __shared__ float qb[];  // [block_dim]
    const int64_t row = blockIdx.x;
    const int b = blockIdx.y;
    for (int k = threadIdx.x; k < block_dim; k += blockDim.x) {
        const int j = b * block_dim + k;
        const int src = perm ? perm[j] : j;
        qb[k] = round_to(q_dtype, load_as_f32(q, q_dtype, row * q_row_stride + src) * scale);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < n_centroids; c += blockDim.x) {
        const float *cv = centroids + ((int64_t)b * n_centroids + c) * block_dim;
        float dot = qb[0] * cv[0];
        for (int k = 1; k < block_dim; ++k) dot = fmaf(qb[k], cv[k], dot);
        lut[(row * n_blocks + b) * n_centroids + c] = dot;
    }
}

// grid (ceil(T/256), ceil(n_rows/rows_per_wg)); the WG's LUT rows live in LDS.
__global__ void __launch_bounds__(256)
    score_gather_kernel(const float *lut, int64_t n_rows, int rows_per_wg, int n_blocks,
                        int n_centroids, const uint8_t *idx, int64_t n_tok,
                        int64_t idx_row_stride, float *scores, int64_t out_row_stride) {
    extern __shared__ float tab[];  // [rows_per_wg][n_blocks][n_centroids]
    const int64_t r0 = (int64_t)blockIdx.y * rows_per_wg;
    const int nr = (int)min((int64_t)rows_per_wg, n_rows - r0);
    const int per_row = n_blocks * n_centroids;
    for (int i = threadIdx.x; i < nr * per_row; i += blockDim.x)
        tab[i] = lut[r0 * per_row + i];
    __syncthreads();
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_tok) return;
    const uint8_t *ip = idx + t * idx_row_stride;
    for (int r = 0; r < nr; ++r) {
        const float *tr = tab + r * per_row;
        float s = 0.f;
        for (int b = 0; b < n_blocks; ++b)
            s += tr[b * n_centroids + min((int)ip[b], n_centroids - 1)];
        scores[(r0 + r) * out_row_stride + t] = s;
    }
}

// one thread per output element (t, i): out[t][i] = k_hat_codec[t][inv_perm[i]]
__global__ void __launch_bounds__(256)
    dequant_blockvq_kernel(const uint8_t *idx, int64_t n_tok, int64_t idx_row_stride,
                           const float *centroids, int n_blocks, int n_centroids,
                           int block_dim, const int32_t *inv_perm, void *out, int out_dtype) {
    const int head_dim = n_blocks * block_dim;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_tok * head_dim) return;
    const int64_t t = e / head_dim;
    const int i = (int)(e - t * head_dim);
    const int j = inv_perm ? inv_perm[i] : i;
    const int b = j / block_dim, d = j - b * block_dim;
    const int c = min((int)idx[t * idx_row_stride + b], n_centroids - 1);
    store_from_f32(out, out_dtype, e,
                   centroids[((int64_t)b * n_centroids + c) * block_dim + d]);
}

}  // namespace ss

using namespace ss;

extern "C" int ss_build_lut(const void *q, int q_dtype, int64_t n_rows, int64_t q_row_stride,
                            int head_dim, const int32_t *perm, float scale,
                            const float *centroids, int n_blocks, int n_centroids,
                            int block_dim, float *lut, void *stream) {
    SS_REQUIRE(valid_dtype(q_dtype), "bad query dtype");
    SS_REQUIRE(n_rows >= 0, "negative n_rows");
    SS_REQUIRE(n_blocks * block_dim == head_dim && block_dim > 0,
               "n_blocks * block_dim != head_dim");
    SS_REQUIRE(n_centroids >= 1, "n_centroids must be >= 1");
    if (n_rows == 0) return SS_OK;
    SS_REQUIRE(q && centroids && lut, "null pointer argument");
    SS_REQUIRE(n_rows <= 0x7fffffff && n_blocks <= 65535, "grid too large");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(build_lut_kernel, dim3((unsigned)n_rows, n_blocks), dim3(256),
                       sizeof(float) * block_dim, st, q, q_dtype, q_row_stride, perm, scale,
                       centroids, n_blocks, n_centroids, block_dim, lut);
    SS_LAUNCH_CHECK("build_lut_kernel launch");
    return SS_OK;
}

extern "C" int ss_score_gather(const float *lut, int64_t n_rows, int n_blocks, int n_centroids,
                               const uint8_t *idx, int64_t n_tok, int64_t idx_row_stride,
                               float *scores, int64_t out_row_stride, void *stream) {
    SS_REQUIRE(n_rows >= 0 && n_tok >= 0, "negative sizes");
    SS_REQUIRE(n_blocks >= 1 && n_centroids >= 1 && n_centroids <= 256,
               "n_centroids must be 1..256 for uint8 indices");
    if (n_rows == 0 || n_tok == 0) return SS_OK;
    SS_REQUIRE(lut && idx && scores, "null pointer argument");
    const int per_row = n_blocks * n_centroids;
    SS_UNSUPPORTED(per_row <= 16384, "n_blocks * n_centroids %d > 16384", per_row);
    int rpw = 16384 / per_row;
    if (rpw > 4) rpw = 4;
    const int64_t ry = (n_rows + rpw - 1) / rpw;
    SS_REQUIRE(ry <= 65535, "too many rows for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    dim3 grid((unsigned)((n_tok + 255) / 256), (unsigned)ry);
    const size_t lds = sizeof(float) * rpw * per_row;
    hipLaunchKernelGGL(score_gather_kernel, grid, dim3(256), lds, st, lut, n_rows, rpw, n_blocks,
                       n_centroids, idx, n_tok, idx_row_stride, scores, out_row_stride);
    SS_LAUNCH_CHECK("score_gather_kernel launch");
    return SS_OK;
}

extern "C" int ss_dequantize_blockvq(const uint8_t *idx, int64_t n_tok, int64_t idx_row_stride,
                                     const float *centroids, int n_blocks, int n_centroids,
                                     int block_dim, const int32_t *inv_perm, void *out,
                                     int out_dtype, void *stream) {
    SS_REQUIRE(valid_dtype(out_dtype), "bad output dtype");
    SS_REQUIRE(n_tok >= 0 && n_blocks >= 1 && block_dim >= 1, "bad sizes");
    SS_REQUIRE(n_centroids >= 1 && n_centroids <= 256, "n_centroids must be 1..256");
    if (n_tok == 0) return SS_OK;
    SS_REQUIRE(idx && centroids && out, "null pointer argument");
    const int64_t total = n_tok * n_blocks * block_dim;
    SS_UNSUPPORTED(total < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(dequant_blockvq_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       st, idx, n_tok, idx_row_stride, centroids, n_blocks, n_centroids,
                       block_dim, inv_perm, out, out_dtype);
    SS_LAUNCH_CHECK("dequant_blockvq_kernel launch");
    return SS_OK;
}
