// Codec fitting on the GPU: Lloyd k-means of every codec block at once.
//
// Restates the reference's per-block k-means (codec.py:53-103), one
// workgroup per block: expanded-form float32 distances x_sq + c_sq - 2 x.c
// with first-index argmin, then per-centroid sums accumulated in point order
// in float32 (numpy's np.add.at order), divided in double and rounded to
// float32 (numpy's in-place float32 / float64 division); empty clusters keep
// their centroid.  Squared norms follow numpy's float32 reduction of a short
// row: sequential below 8 elements, the 8-way pairwise tree at 8.  The dot
// products x.c are the one step whose rounding the reference leaves to its
// BLAS: here they are sequential fused multiply-adds, so assignments can
// differ from the reference's at near-ties only.
#include "ss_common.hpp"

namespace ss {

template <int BD>
__device__ __forceinline__ float row_sq(const float *v) {
    float s[BD];
#pragma unroll
    for (int j = 0; j < BD; ++j) s[j] = __fmul_rn(v[j], v[j]);
    if constexpr (BD == 8) {
        return __fadd_rn(__fadd_rn(__fadd_rn(s[0], s[1]), __fadd_rn(s[2], s[3])),
                         __fadd_rn(__fadd_rn(s[4], s[5]), __fadd_rn(s[6], s[7])));
    } else {
        float r = s[0];
#pragma unroll
        for (int j = 1; j < BD; ++j) r = __fadd_rn(r, s[j]);
        return r;
    }
}

constexpr int kFitThreads = 256;
constexpr int64_t kFitMaxPoints = 131072;  // uint8 assignments of one block in LDS

template <int BD>
__global__ void __launch_bounds__(kFitThreads)
    kmeans_block_kernel(const float *data, int64_t n, int k, int iters, float *cents,
                        uint8_t *assign_out) {
    extern __shared__ __align__(16) float fsm[];
    float *cs = fsm;                                         // [256][BD] centroids
    float *csq = cs + 256 * BD;                              // [256] squared norms
    uint8_t *asg = reinterpret_cast<uint8_t *>(csq + 256);  // [n] assignments
    const int b = blockIdx.x, tid = threadIdx.x;
    const float *x = data + (int64_t)b * n * BD;
    float *c = cents + (int64_t)b * k * BD;
    for (int i = tid; i < k * BD; i += kFitThreads) cs[i] = c[i];
    __syncthreads();
    for (int it = 0; it < iters; ++it) {
        if (tid < k) csq[tid] = row_sq<BD>(cs + tid * BD);
        __syncthreads();
        // assignment: every point against every centroid, first minimum
        for (int64_t i = tid; i < n; i += kFitThreads) {
            float xv[BD];
#pragma unroll
            for (int j = 0; j < BD; ++j) xv[j] = x[i * BD + j];
            const float xsq = row_sq<BD>(xv);
            float best = INFINITY;
            int bi = 0;
            for (int kk = 0; kk < k; ++kk) {
                const float *ck = cs + kk * BD;
                float dot = __fmul_rn(xv[0], ck[0]);
#pragma unroll
                for (int j = 1; j < BD; ++j) dot = fmaf(xv[j], ck[j], dot);
                const float dist = __fsub_rn(__fadd_rn(xsq, csq[kk]), __fmul_rn(2.f, dot));
                if (dist < best) {
                    best = dist;
                    bi = kk;
                }
            }
            asg[i] = (uint8_t)bi;
        }
        __syncthreads();
        // update: thread kk sums its points in point order
        if (tid < k) {
            float s[BD];
#pragma unroll
            for (int j = 0; j < BD; ++j) s[j] = 0.f;
            int64_t cnt = 0;
            auto take = [&](int64_t i) {
                ++cnt;
#pragma unroll
                for (int j = 0; j < BD; ++j) s[j] = __fadd_rn(s[j], x[i * BD + j]);
            };
            // four assignments per LDS read, still in point order
            const uint32_t *asg4 = reinterpret_cast<const uint32_t *>(asg);
            const int64_t n4 = n / 4;
            for (int64_t w = 0; w < n4; ++w) {
                const uint32_t v = asg4[w];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (((v >> (8 * q)) & 0xffu) == (uint32_t)tid) take(w * 4 + q);
            }
            for (int64_t i = n4 * 4; i < n; ++i)
                if (asg[i] == tid) take(i);
            if (cnt > 0) {
#pragma unroll
                for (int j = 0; j < BD; ++j)
                    cs[tid * BD + j] = (float)((double)s[j] / (double)cnt);
            }
        }
        __syncthreads();
    }
    for (int i = tid; i < k * BD; i += kFitThreads) c[i] = cs[i];
    if (assign_out)
        for (int64_t i = tid; i < n; i += kFitThreads) assign_out[(int64_t)b * n + i] = asg[i];
}

}  // namespace ss

using namespace ss;

extern "C" int ss_kmeans_blocks(const float *data, int n_blocks, int64_t n_points, int block_dim,
                                int n_centroids, int iters, float *centroids, uint8_t *assign,
                                void *stream) {
    SS_REQUIRE(data && centroids, "null data/centroids");
    SS_REQUIRE(n_blocks >= 1, "n_blocks must be positive");
    SS_UNSUPPORTED(block_dim == 4 || block_dim == 8, "block_dim %d unsupported (4 or 8)",
                   block_dim);
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256,
                   "n_centroids %d unsupported (1..256)", n_centroids);
    SS_REQUIRE(n_points > n_centroids,
               "k-means needs more points (%lld) than centroids (%d); the caller zero-pads",
               (long long)n_points, n_centroids);
    SS_UNSUPPORTED(n_points <= kFitMaxPoints, "at most %lld points per block (got %lld)",
                   (long long)kFitMaxPoints, (long long)n_points);
    SS_REQUIRE(iters >= 0, "negative iteration count");
    SS_REQUIRE(((uintptr_t)data % 4) == 0 && ((uintptr_t)centroids % 4) == 0,
               "data/centroids must be 4-byte aligned");
    const size_t lds = (size_t)(256 * block_dim + 256) * sizeof(float) + (size_t)n_points;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    auto run = [&](auto kern) -> int {
        static int attr_lds = 0;
        if ((int)lds > attr_lds) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds);
            if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(kmeans)");
            attr_lds = (int)lds;
        }
        hipLaunchKernelGGL(kern, dim3(n_blocks), dim3(kFitThreads), lds, st, data, n_points,
                           n_centroids, iters, centroids, assign);
        SS_LAUNCH_CHECK("kmeans_block_kernel launch");
        return SS_OK;
    };
    return block_dim == 8 ? run(kmeans_block_kernel<8>) : run(kmeans_block_kernel<4>);
}
