// KV-cache value layout: append tokens into the 8-token interleaved fp16 layout.
//
// The decode kernel's MFMA path reads values as [cap/8][head_dim][8] per
// (batch, KV head): the 8 consecutive tokens of one dim are 16 contiguous
// bytes, the K-major operand of v_mfma_f32_16x16x32_f16.  Appending T new
// tokens at position `offset` scatters each token's head_dim values with a
// 16-byte stride; the index cache keeps the token-major [cap][n_blocks]
// layout of the reference (cache.py:102-150).
#include "ss_common.hpp"

namespace ss {

__global__ void __launch_bounds__(256)
    append_il8_kernel(const void *v, int v_dtype, int64_t n_h, int64_t n_t, int64_t n_tok,
                      int64_t v_sb, int64_t v_sh, int64_t v_st, int d, __half *out, int64_t cap,
                      int64_t offset) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_tok * d) return;
    const int64_t n = e / d;
    const int j = (int)(e - n * d);
    const int64_t b = n / (n_h * n_t);
    const int64_t rem = n - b * n_h * n_t;
    const int64_t h = rem / n_t;
    const int64_t t = rem - h * n_t;
    const float x = load_as_f32(v, v_dtype, b * v_sb + h * v_sh + t * v_st + j);
    store_value_il8(out, b * n_h + h, cap, d, offset + t, j, x);
}

// Whole keys for the hybrid prompt kernel: one wave per token.  Dim j of the
// output is dim perm[j] of the key (the codec's basis; perm null = identity).
// With s = row_exp_shift(max |key|), row 0 = fp16(key * 2^-s) and row 1 =
// fp16(key * 2^-s - row 0); factor = 2^s.  Multiplying by a power of two is
// exact, so row 0 + row 1 is the key times 2^-s to 22 significant bits, and
// exactly for fp16 and bf16 keys (row 1 = 0); a remainder below fp16's
// normal range is rounded there, under 2^-38 of the row's largest element.
__global__ void __launch_bounds__(256)
    raw_key_rows_kernel(const void *k, int k_dtype, int64_t n_h, int64_t n_t, int64_t n_tok,
                        int64_t k_sb, int64_t k_sh, int64_t k_st, int d, const int32_t *perm,
                        __half *rows, float *fac) {
    const int64_t n = (int64_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (n >= n_tok) return;  // whole waves leave together
    const int64_t b = n / (n_h * n_t);
    const int64_t rem = n - b * n_h * n_t;
    const int64_t h = rem / n_t;
    const int64_t t = rem - h * n_t;
    const int64_t base = b * k_sb + h * k_sh + t * k_st;
    float m = 0.f;
    for (int j = lane; j < d; j += 64)
        m = fmaxf(m, fabsf(load_as_f32(k, k_dtype, base + (perm ? perm[j] : j))));
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const int s = row_exp_shift(m);
    const float down = exp2i(-s);
    __half *r0 = rows + n * 2 * d;
    for (int j = lane; j < d; j += 64) {
        const float x = load_as_f32(k, k_dtype, base + (perm ? perm[j] : j)) * down;
        const __half hi = __float2half(x);
        r0[j] = hi;
        r0[d + j] = __float2half(x - __half2float(hi));
    }
    if (lane == 0) fac[n] = exp2i(s);
}

}  // namespace ss

using namespace ss;

extern "C" int ss_append_values_il8(const void *values, int v_dtype, int64_t n_b, int64_t n_h,
                                    int64_t n_t, int64_t v_sb, int64_t v_sh, int64_t v_st,
                                    int head_dim, void *out_il8, int64_t cap, int64_t offset,
                                    void *stream) {
    SS_REQUIRE(valid_dtype(v_dtype), "bad value dtype");
    SS_REQUIRE(n_b >= 0 && n_h >= 0 && n_t >= 0 && head_dim >= 1, "bad sizes");
    SS_REQUIRE(cap % 8 == 0, "cap must be a multiple of 8");
    SS_REQUIRE(offset >= 0 && offset + n_t <= cap, "tokens [%lld, %lld) exceed cap %lld",
               (long long)offset, (long long)(offset + n_t), (long long)cap);
    const int64_t n_tok = n_b * n_h * n_t;
    if (n_tok == 0) return SS_OK;
    SS_REQUIRE(values && out_il8, "null pointer argument");
    const int64_t total = n_tok * head_dim;
    SS_UNSUPPORTED(total < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(append_il8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                       values, v_dtype, n_h, n_t, n_tok, v_sb, v_sh, v_st, head_dim,
                       reinterpret_cast<__half *>(out_il8), cap, offset);
    SS_LAUNCH_CHECK("append_il8_kernel launch");
    return SS_OK;
}

extern "C" int ss_raw_key_rows(const void *keys, int k_dtype, int64_t n_b, int64_t n_h,
                               int64_t n_t, int64_t k_sb, int64_t k_sh, int64_t k_st,
                               int head_dim, const int32_t *perm, void *rows, float *factors,
                               void *stream) {
    SS_REQUIRE(valid_dtype(k_dtype), "bad key dtype");
    SS_REQUIRE(n_b >= 0 && n_h >= 0 && n_t >= 0 && head_dim >= 1, "bad sizes");
    const int64_t n_tok = n_b * n_h * n_t;
    if (n_tok == 0) return SS_OK;
    SS_REQUIRE(keys && rows && factors, "null pointer argument");
    SS_UNSUPPORTED(n_tok < (1LL << 31), "too many tokens for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(raw_key_rows_kernel, dim3((unsigned)((n_tok + 3) / 4)), dim3(256), 0, st,
                       keys, k_dtype, n_h, n_t, n_tok, k_sb, k_sh, k_st, head_dim, perm,
                       reinterpret_cast<__half *>(rows), factors);
    SS_LAUNCH_CHECK("raw_key_rows_kernel launch");
    return SS_OK;
}
