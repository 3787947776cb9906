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

// grid (ceil(T/256), n_heads * n_rgrp): workgroup (x, y) scores tokens
// 256x .. 256x + 255 of head y / n_rgrp (a (batch, KV head) pair) for its
// query rows (y % n_rgrp) * rows_per_wg ..; those rows' LUTs live in LDS.  A
// token's 16-block index row is one 16-byte load when rows are 16-byte
// aligned, else one byte per block.
__global__ void __launch_bounds__(256)
    score_gather_kernel(const float *lut, int64_t lut_head_stride, int64_t n_rows,
                        int rows_per_wg, int n_rgrp, int n_blocks, int n_centroids,
                        const uint8_t *idx, int64_t n_h, int64_t idx_sb, int64_t idx_sh,
                        int64_t idx_st, int64_t n_tok, float *scores, int64_t out_head_stride,
                        int64_t out_row_stride, int rows16) {
    extern __shared__ float tab[];  // [rows_per_wg][n_blocks][n_centroids]
    const int64_t head = blockIdx.y / n_rgrp;
    const int64_t r0 = (int64_t)(blockIdx.y % n_rgrp) * rows_per_wg;
    const int nr = (int)min((int64_t)rows_per_wg, n_rows - r0);
    const int per_row = n_blocks * n_centroids;
    const float *lh = lut + head * lut_head_stride + r0 * per_row;
    for (int i = threadIdx.x; i < nr * per_row; i += blockDim.x) tab[i] = lh[i];
    __syncthreads();
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_tok) return;
    const int64_t b = head / n_h, h = head - b * n_h;
    const uint8_t *ip = idx + b * idx_sb + h * idx_sh + t * idx_st;
    uint32_t code[16];
    if (rows16) {
        const uint4 w = *reinterpret_cast<const uint4 *>(ip);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int b2 = 0; b2 < 16; ++b2) code[b2] = (ws[b2 >> 2] >> (8 * (b2 & 3))) & 0xffu;
    }
    float *out = scores + head * out_head_stride + t;
    for (int r = 0; r < nr; ++r) {
        const float *tr = tab + r * per_row;
        float s = 0.f;
        if (rows16) {
#pragma unroll
            for (int b2 = 0; b2 < 16; ++b2) s += tr[b2 * n_centroids + min((int)code[b2], n_centroids - 1)];
        } else {
            for (int b2 = 0; b2 < n_blocks; ++b2)
                s += tr[b2 * n_centroids + min((int)ip[b2], n_centroids - 1)];
        }
        out[(r0 + r) * out_row_stride] = s;
    }
}

// The same for codecs of at most 16 blocks, four query rows per row group:
// the group's LUT sits in LDS as a float4 (its four rows) per (block,
// centroid), so a token's scores for all four rows take one 16-byte LDS
// gather per block; a workgroup scores kGatherTokens tokens so its 64 KB
// LUT copy is amortised over them.  Workgroups are handed to the 8 XCDs in
// turn by their linear id L, so work item w = (L % 8) * per_xcd + L / 8
// keeps a row group's token chunks on one XCD: its LUT is fetched from HBM
// into that XCD's L2 once, not once per XCD.
constexpr int kGatherTokens = 4096;
constexpr int kGatherThreads = 512;

template <bool kRows16>
__global__ void __launch_bounds__(kGatherThreads)
    score_gather4_kernel(const float *lut, int64_t lut_head_stride, int64_t n_rows, int n_rgrp,
                         int n_blocks, int n_centroids, const uint8_t *idx, int64_t n_h,
                         int64_t idx_sb, int64_t idx_sh, int64_t idx_st, int64_t n_tok,
                         float *scores, int64_t out_head_stride, int64_t out_row_stride,
                         int64_t n_chunk, int64_t n_work, int64_t per_xcd) {
    extern __shared__ float4 tab4[];  // [n_blocks][256] float4
    const int64_t w = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (w >= n_work) return;  // the grid is padded to a multiple of 8
    const int64_t grp = w / n_chunk, chunk = w - grp * n_chunk;
    const int64_t head = grp / n_rgrp;
    const int64_t r0 = (grp % n_rgrp) * 4;
    const int nr = (int)min((int64_t)4, n_rows - r0);
    const int per_row = n_blocks * n_centroids;
    const float *lh = lut + head * lut_head_stride + r0 * per_row;
    const int64_t b0 = head / n_h, h0 = head - b0 * n_h;
    const uint8_t *ih = idx + b0 * idx_sb + h0 * idx_sh;
    const int64_t t0 = chunk * kGatherTokens;
    const int64_t t_end = min(n_tok, t0 + kGatherTokens);
    // 16-byte index rows: the thread's kTokPer rows are requested right
    // after the LUT loads, so they stream while the LUT reaches LDS
    constexpr int kTokPer = kGatherTokens / kGatherThreads;
    uint4 rq[kTokPer];
    const auto load_rows = [&]() {
        if (!kRows16) return;
#pragma unroll
        for (int k = 0; k < kTokPer; ++k) {
            // rows past t_end read the last row again (their scores are not stored)
            const int64_t t = min(t0 + threadIdx.x + k * kGatherThreads, t_end - 1);
            rq[k] = *reinterpret_cast<const uint4 *>(ih + t * idx_st);
        }
    };
    if (n_centroids == 256 && n_blocks == 16) {
        // entry i = block * 256 + centroid: consecutive threads take
        // consecutive entries, so each row's loads are coalesced and the
        // float4 stores fall in distinct LDS banks
        constexpr int kPer = 16 * 256 / kGatherThreads;
        float v[kPer][4];
#pragma unroll
        for (int k = 0; k < kPer; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                v[k][r] = lh[min(r, nr - 1) * per_row + threadIdx.x + k * kGatherThreads];
        __builtin_amdgcn_sched_barrier(0);  // LUT loads issue before the index rows
        load_rows();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < kPer; ++k)
#pragma unroll
            for (int r = 1; r < 4; ++r)
                if (r >= nr) v[k][r] = 0.f;  // rows past the last read row nr - 1 again
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            tab4[threadIdx.x + k * kGatherThreads] = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
    } else {
        for (int i = threadIdx.x; i < n_blocks * 256; i += blockDim.x) {
            const int b = i >> 8, c = i & 255;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (c < n_centroids)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r < nr) v[r] = lh[r * per_row + b * n_centroids + c];
            tab4[i] = make_float4(v[0], v[1], v[2], v[3]);
        }
        load_rows();
    }
    __syncthreads();
    float *out = scores + head * out_head_stride + r0 * out_row_stride;
    const auto emit = [&](int64_t t, float4 acc) {
        const float a4[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (r < nr) out[r * out_row_stride + t] = a4[r];
    };
    if (kRows16) {
#pragma unroll
        for (int k = 0; k < kTokPer; ++k) {
            const int64_t t = t0 + threadIdx.x + k * kGatherThreads;
            if (t >= t_end) break;
            const uint32_t ws[4] = {rq[k].x, rq[k].y, rq[k].z, rq[k].w};
            typedef float f4v __attribute__((ext_vector_type(4)));
            const f4v *tv = reinterpret_cast<const f4v *>(tab4);
            f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int b = 0; b < 16; ++b) {
                const int c = min((int)((ws[b >> 2] >> (8 * (b & 3))) & 0xffu), n_centroids - 1);
                acc += tv[b * 256 + c];
            }
            emit(t, make_float4(acc.x, acc.y, acc.z, acc.w));
        }
        return;
    }
    for (int64_t t = t0 + threadIdx.x; t < t_end; t += blockDim.x) {
        const uint8_t *ip = ih + t * idx_st;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int b = 0; b < n_blocks; ++b) {
            const float4 e = tab4[b * 256 + min((int)ip[b], n_centroids - 1)];
            acc.x += e.x;
            acc.y += e.y;
            acc.z += e.z;
            acc.w += e.w;
        }
        emit(t, acc);
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

static int score_gather_impl(const float *lut, int64_t lut_head_stride, int64_t n_rows,
                             int n_blocks, int n_centroids, const uint8_t *idx, int64_t n_b,
                             int64_t n_h, int64_t idx_sb, int64_t idx_sh, int64_t idx_st,
                             int64_t n_tok, float *scores, int64_t out_head_stride,
                             int64_t out_row_stride, void *stream) {
    SS_REQUIRE(n_rows >= 0 && n_tok >= 0 && n_b >= 0 && n_h >= 0, "negative sizes");
    SS_REQUIRE(n_blocks >= 1 && n_centroids >= 1 && n_centroids <= 256,
               "n_centroids must be 1..256 for uint8 indices");
    if (n_rows == 0 || n_tok == 0 || n_b * n_h == 0) return SS_OK;
    SS_REQUIRE(lut && idx && scores, "null pointer argument");
    const int per_row = n_blocks * n_centroids;
    SS_UNSUPPORTED(per_row <= 16384, "n_blocks * n_centroids %d > 16384", per_row);
    int rpw = 16384 / per_row;
    if (rpw > 4) rpw = 4;
    const int64_t n_rgrp = (n_rows + rpw - 1) / rpw;
    const int64_t ry = n_b * n_h * n_rgrp;
    SS_UNSUPPORTED(ry <= 65535, "too many (head, row group) pairs for one launch");
    const int rows16 = n_blocks == 16 && ((uintptr_t)idx % 16) == 0 && idx_sb % 16 == 0 &&
                       idx_sh % 16 == 0 && idx_st % 16 == 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (n_blocks <= 16) {  // float4 LUT of four rows, many tokens per workgroup
        const int64_t n_rg4 = (n_rows + 3) / 4;
        const int64_t ry4 = n_b * n_h * n_rg4;
        const int64_t n_chunk = (n_tok + kGatherTokens - 1) / kGatherTokens;
        const int64_t n_work = ry4 * n_chunk, per_xcd = (n_work + 7) / 8;
        SS_UNSUPPORTED(per_xcd * 8 <= 0x7fffffff, "too many workgroups for one launch");
        const dim3 grid4((unsigned)(per_xcd * 8));
        const size_t lds4 = sizeof(float4) * n_blocks * 256;
        const auto kern = rows16 ? score_gather4_kernel<true> : score_gather4_kernel<false>;
        if (lds4 > 65536) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)lds4);
            if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(score gather)");
        }
        hipLaunchKernelGGL(kern, grid4, dim3(kGatherThreads), lds4, st, lut, lut_head_stride,
                           n_rows, (int)n_rg4, n_blocks, n_centroids, idx, n_h, idx_sb, idx_sh,
                           idx_st, n_tok, scores, out_head_stride, out_row_stride, n_chunk,
                           n_work, per_xcd);
        SS_LAUNCH_CHECK("score_gather4_kernel launch");
        return SS_OK;
    }
    dim3 grid((unsigned)((n_tok + 255) / 256), (unsigned)ry);
    const size_t lds = sizeof(float) * rpw * per_row;
    hipLaunchKernelGGL(score_gather_kernel, grid, dim3(256), lds, st, lut, lut_head_stride, n_rows,
                       rpw, (int)n_rgrp, n_blocks, n_centroids, idx, n_h, idx_sb, idx_sh, idx_st,
                       n_tok, scores, out_head_stride, out_row_stride, rows16);
    SS_LAUNCH_CHECK("score_gather_kernel launch");
    return SS_OK;
}

extern "C" int ss_score_gather(const float *lut, int64_t n_rows, int n_blocks, int n_centroids,
                               const uint8_t *idx, int64_t n_tok, int64_t idx_row_stride,
                               float *scores, int64_t out_row_stride, void *stream) {
    return score_gather_impl(lut, 0, n_rows, n_blocks, n_centroids, idx, 1, 1, 0, 0,
                             idx_row_stride, n_tok, scores, 0, out_row_stride, stream);
}

extern "C" int ss_score_gather_heads(const float *lut, int64_t n_rows, int n_blocks,
                                     int n_centroids, const uint8_t *idx, int64_t n_b,
                                     int64_t n_h, int64_t idx_sb, int64_t idx_sh, int64_t idx_st,
                                     int64_t n_tok, float *scores, void *stream) {
    const int64_t per_row = (int64_t)n_blocks * n_centroids;
    return score_gather_impl(lut, n_rows * per_row, n_rows, n_blocks, n_centroids, idx, n_b, n_h,
                             idx_sb, idx_sh, idx_st, n_tok, scores, n_rows * n_tok, n_tok, stream);
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
