// Block-VQ encoder: nearest of n_centroids codewords per block_dim-dim block.
//
// Semantics of the reference encode kernel (kernels.py:995-1027): squared L2
// distance, strict '<' so ties keep the lowest index, uint8 out; the key is
// first gathered through the ProfilePerm permutation (codec.py:435-436).
// The reference's float32 sum is not bit-pinned (Metal fast-math), so the
// index is defined by exact arithmetic: every (token, block) is first ranked
// in float32 (direct form, fused multiply-add accumulation), and when the
// runner-up is within kSuspectRel of the best -- wider than the float32
// error of an 8-term sum of squares -- the block is re-ranked in float64.
//
// Two launch shapes:
//   * bulk (prefill / flush): one token per lane, a workgroup owns 256
//     tokens x kBlocksPerWG blocks; those blocks' codebooks sit in LDS and
//     every lane of a wave reads the same codeword (LDS broadcast);
//   * small (decode-step append, few tokens): one wave per (token, block),
//     lanes split the codebook and reduce (distance, index) across the wave.
#include "ss_common.hpp"

namespace ss {

constexpr float kSuspectRel = 4e-6f;
constexpr int kEncThreads = 256;
constexpr int kBlocksPerWG = 4;

struct EncodeArgs {
    const void *keys;
    int keys_dtype;
    int64_t n_h, n_t, n_tok;
    int64_t k_sb, k_sh, k_st;
    const int32_t *perm;
    const float *centroids;
    int n_blocks, n_centroids;
    uint8_t *out;
    int64_t o_sb, o_sh, o_st;
};

struct TokAddr {
    int64_t key, out;
};

__device__ __forceinline__ TokAddr token_addr(const EncodeArgs &a, int64_t n) {
    const int64_t b = n / (a.n_h * a.n_t);
    const int64_t rem = n - b * a.n_h * a.n_t;
    const int64_t h = rem / a.n_t;
    const int64_t t = rem - h * a.n_t;
    return {b * a.k_sb + h * a.k_sh + t * a.k_st, b * a.o_sb + h * a.o_sh + t * a.o_st};
}

template <int BD>
__device__ __forceinline__ int refine_f64(const float (&kv)[BD], const float *cb, int nc) {
    double best = 0.0;
    int bi = 0;
    for (int c = 0; c < nc; ++c) {
        double d = 0.0;
#pragma unroll
        for (int k = 0; k < BD; ++k) {
            const double df = (double)kv[k] - (double)cb[c * BD + k];
            d = fma(df, df, d);
        }
        if (c == 0 || d < best) {
            best = d;
            bi = c;
        }
    }
    return bi;
}

// ---- bulk: token per lane ----
template <int BD>
__global__ void __launch_bounds__(kEncThreads) encode_bulk_kernel(EncodeArgs a) {
    extern __shared__ __align__(16) float cbuf[];  // [kBlocksPerWG][nc][BD]
    const int nc = a.n_centroids;
    const int blk0 = blockIdx.y * kBlocksPerWG;
    const int nblk = min(kBlocksPerWG, a.n_blocks - blk0);
    const int total = nblk * nc * BD;
    const float *src = a.centroids + (int64_t)blk0 * nc * BD;
    for (int i = threadIdx.x; i < total; i += kEncThreads) cbuf[i] = src[i];
    __syncthreads();

    const int64_t n = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
    if (n >= a.n_tok) return;
    const TokAddr ad = token_addr(a, n);
    for (int bl = 0; bl < nblk; ++bl) {
        const int blk = blk0 + bl;
        float kv[BD];
#pragma unroll
        for (int k = 0; k < BD; ++k) {
            const int j = blk * BD + k;
            kv[k] = load_as_f32(a.keys, a.keys_dtype, ad.key + (a.perm ? a.perm[j] : j));
        }
        const float *cb = cbuf + bl * nc * BD;
        float best = INFINITY, second = INFINITY;
        int bi = 0;
        for (int c = 0; c < nc; ++c) {
            const float *cv = cb + c * BD;
            float df = kv[0] - cv[0];
            float d = df * df;
#pragma unroll
            for (int k = 1; k < BD; ++k) {
                df = kv[k] - cv[k];
                d = fmaf(df, df, d);
            }
            const bool lt = d < best;
            second = lt ? best : fminf(second, d);
            bi = lt ? c : bi;
            best = lt ? d : best;
        }
        if (!(second > best * (1.0f + kSuspectRel))) bi = refine_f64<BD>(kv, cb, nc);
        a.out[ad.out + blk] = (uint8_t)bi;
    }
}

// ---- small: wave per (token, block) ----
template <int BD>
__global__ void __launch_bounds__(kEncThreads) encode_small_kernel(EncodeArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t job = (int64_t)blockIdx.x * (kEncThreads / kWave) + (threadIdx.x >> 6);
    if (job >= a.n_tok * a.n_blocks) return;  // wave-uniform
    const int64_t n = job / a.n_blocks;
    const int blk = (int)(job - n * a.n_blocks);
    const TokAddr ad = token_addr(a, n);
    float kv[BD];
#pragma unroll
    for (int k = 0; k < BD; ++k) {
        const int j = blk * BD + k;
        kv[k] = load_as_f32(a.keys, a.keys_dtype, ad.key + (a.perm ? a.perm[j] : j));
    }
    const int nc = a.n_centroids;
    const float *cb = a.centroids + (int64_t)blk * nc * BD;
    float best = INFINITY, second = INFINITY;
    int bi = 0x7fffffff;
    for (int c = lane; c < nc; c += kWave) {
        const float *cv = cb + c * BD;
        float df = kv[0] - cv[0];
        float d = df * df;
#pragma unroll
        for (int k = 1; k < BD; ++k) {
            df = kv[k] - cv[k];
            d = fmaf(df, df, d);
        }
        const bool lt = d < best;
        second = lt ? best : fminf(second, d);
        bi = lt ? c : bi;
        best = lt ? d : best;
    }
    // wave reduction of (best, index) with lowest-index ties, keeping the
    // runner-up distance
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o);
        const float os = __shfl_xor(second, o);
        const int oi = __shfl_xor(bi, o);
        const bool mine = best < ob || (best == ob && bi < oi);
        second = mine ? fminf(second, ob) : fminf(os, best);
        best = mine ? best : ob;
        bi = mine ? bi : oi;
    }
    if (!(second > best * (1.0f + kSuspectRel))) {
        double b64 = INFINITY;
        int i64 = 0x7fffffff;
        for (int c = lane; c < nc; c += kWave) {
            double d = 0.0;
#pragma unroll
            for (int k = 0; k < BD; ++k) {
                const double df = (double)kv[k] - (double)cb[c * BD + k];
                d = fma(df, df, d);
            }
            if (d < b64) {
                b64 = d;
                i64 = c;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const double ob = __shfl_xor(b64, o);
            const int oi = __shfl_xor(i64, o);
            const bool mine = b64 < ob || (b64 == ob && i64 < oi);
            b64 = mine ? b64 : ob;
            i64 = mine ? i64 : oi;
        }
        bi = i64;
    }
    if (bi == 0x7fffffff) bi = 0;  // every distance NaN: the reference keeps index 0
    if (lane == 0) a.out[ad.out + blk] = (uint8_t)bi;
}

template <int BD>
static int launch_encode(const EncodeArgs &a, hipStream_t st) {
    const int64_t jobs = a.n_tok * a.n_blocks;
    // few tokens (decode-step append): parallelise each block over the codebook
    if (jobs <= 4096) {
        const int per = kEncThreads / kWave;
        dim3 grid((unsigned)((jobs + per - 1) / per));
        hipLaunchKernelGGL(encode_small_kernel<BD>, grid, dim3(kEncThreads), 0, st, a);
        SS_LAUNCH_CHECK("encode_small_kernel launch");
        return SS_OK;
    }
    const size_t lds = sizeof(float) * kBlocksPerWG * a.n_centroids * BD;
    dim3 grid((unsigned)((a.n_tok + kEncThreads - 1) / kEncThreads),
              (unsigned)((a.n_blocks + kBlocksPerWG - 1) / kBlocksPerWG));
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void *>(encode_bulk_kernel<BD>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(encode)");
    }
    hipLaunchKernelGGL(encode_bulk_kernel<BD>, grid, dim3(kEncThreads), lds, st, a);
    SS_LAUNCH_CHECK("encode_bulk_kernel launch");
    return SS_OK;
}

}  // namespace ss

using namespace ss;

extern "C" int ss_encode_blockvq(const void *keys, int keys_dtype, int64_t n_b, int64_t n_h,
                                 int64_t n_t, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                 int head_dim, const int32_t *perm, const float *centroids,
                                 int n_blocks, int n_centroids, int block_dim, uint8_t *out,
                                 int64_t o_sb, int64_t o_sh, int64_t o_st, void *stream) {
    SS_REQUIRE(valid_dtype(keys_dtype), "bad key dtype");
    SS_REQUIRE(n_b >= 0 && n_h >= 0 && n_t >= 0, "negative token counts");
    SS_REQUIRE(head_dim > 0 && block_dim > 0 && n_blocks * block_dim == head_dim,
               "n_blocks (%d) * block_dim (%d) != head_dim (%d)", n_blocks, block_dim, head_dim);
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256,
                   "n_centroids %d unsupported for uint8 indices (1..256)", n_centroids);
    SS_UNSUPPORTED(block_dim == 4 || block_dim == 8 || block_dim == 16,
                   "block_dim %d unsupported (4, 8, 16)", block_dim);
    const int64_t n_tok = n_b * n_h * n_t;
    if (n_tok == 0) return SS_OK;
    SS_REQUIRE(keys && centroids && out, "null pointer argument");
    EncodeArgs a{keys, keys_dtype, n_h,  n_t,        n_tok,     k_sb, k_sh, k_st,
                 perm, centroids,  n_blocks, n_centroids, out, o_sb, o_sh, o_st};
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (block_dim == 8) return launch_encode<8>(a, st);
    if (block_dim == 4) return launch_encode<4>(a, st);
    return launch_encode<16>(a, st);
}
