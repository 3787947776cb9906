// Value codecs: grouped asymmetric quantisation, bit packing, scalar quantise.
//
// Integer outputs (codes, packed words, scalar indices) are bit-exact with the
// reference's arithmetic: every float32 step is an IEEE operation with no
// contraction (__fsub_rn / __fdiv_rn / rintf), mirroring kernels.py:1173-1228.
#include "ss_common.hpp"

namespace ss {

__host__ __device__ constexpr int vals_per_word(int bits) { return 32 / bits; }

__host__ __device__ inline int packed_words(int d, int bits) {
    const int vpw = vals_per_word(bits);
    return (d + vpw - 1) / vpw;
}

// One thread per token: groups' min/max -> scale/zero -> codes -> packed words.
__global__ void __launch_bounds__(256)
    quantize_grouped_kernel(const void *values, int v_dtype, int64_t n_h, int64_t n_t,
                            int64_t n_tok, int64_t v_sb, int64_t v_sh, int64_t v_st, int d,
                            int bits, int group, uint32_t *packed, void *scales, void *zeros,
                            int sz_dtype, int64_t o_sb, int64_t o_sh, int64_t o_st) {
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= n_tok) return;
    const int64_t b = n / (n_h * n_t);
    const int64_t rem = n - b * n_h * n_t;
    const int64_t h = rem / n_t;
    const int64_t t = rem - h * n_t;
    const int64_t vin = b * v_sb + h * v_sh + t * v_st;
    const int64_t orow = b * o_sb + h * o_sh + t * o_st;
    const int n_groups = d / group;
    const int vpw = vals_per_word(bits);
    const int nw = packed_words(d, bits);
    const float maxv = (float)((1 << bits) - 1);
    const uint32_t mask = (1u << bits) - 1u;

    uint32_t word = 0u;
    int word_i = 0, slot = 0;
    for (int g = 0; g < n_groups; ++g) {
        float mn = INFINITY, mx = -INFINITY;
        for (int k = 0; k < group; ++k) {
            const float v = load_as_f32(values, v_dtype, vin + g * group + k);
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        float sc = __fdiv_rn(__fsub_rn(mx, mn), maxv);
        if (sc < 1e-8f) sc = 1e-8f;
        store_from_f32(scales, sz_dtype, orow * n_groups + g, sc);
        store_from_f32(zeros, sz_dtype, orow * n_groups + g, mn);
        for (int k = 0; k < group; ++k) {
            const float v = load_as_f32(values, v_dtype, vin + g * group + k);
            float qf = rintf(__fdiv_rn(__fsub_rn(v, mn), sc));
            qf = fminf(fmaxf(qf, 0.f), maxv);
            word |= ((uint32_t)qf & mask) << (slot * bits);
            if (++slot == vpw) {
                packed[orow * nw + word_i++] = word;
                word = 0u;
                slot = 0;
            }
        }
    }
    if (slot) packed[orow * nw + word_i] = word;  // zero-padded tail word
}

// One thread per output value.
__global__ void __launch_bounds__(256)
    dequantize_grouped_kernel(const uint32_t *packed, const void *scales, const void *zeros,
                              int sz_dtype, int64_t n_tok, int d, int bits, int group, void *out,
                              int out_dtype) {
    // separate multiply and add, as the reference's elementwise ops round
    // (device code is otherwise compiled with fp-contract=fast)
#pragma clang fp contract(off)
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_tok * d) return;
    const int64_t t = e / d;
    const int i = (int)(e - t * d);
    const int vpw = vals_per_word(bits);
    const int nw = packed_words(d, bits);
    const int n_groups = d / group;
    const uint32_t w = packed[t * nw + i / vpw];
    const float q = (float)((w >> ((i % vpw) * bits)) & ((1u << bits) - 1u));
    const int64_t gi = t * n_groups + i / group;
    const float sc = load_as_f32(scales, sz_dtype, gi);
    const float zr = load_as_f32(zeros, sz_dtype, gi);
    const float prod = q * sc;
    store_from_f32(out, out_dtype, e, prod + zr);
}

__global__ void __launch_bounds__(256)
    pack_kernel(const uint8_t *in, int64_t n_rows, int d, int bits, uint32_t *out) {
    const int nw = packed_words(d, bits);
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_rows * nw) return;
    const int64_t r = e / nw;
    const int w = (int)(e - r * nw);
    const int vpw = vals_per_word(bits);
    const uint32_t mask = (1u << bits) - 1u;
    uint32_t word = 0u;
    for (int k = 0; k < vpw; ++k) {
        const int col = w * vpw + k;
        if (col < d) word |= ((uint32_t)in[r * d + col] & mask) << (k * bits);
    }
    out[e] = word;
}

__global__ void __launch_bounds__(256)
    unpack_kernel(const uint32_t *in, int64_t n_rows, int d, int bits, uint32_t *out) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_rows * d) return;
    const int64_t r = e / d;
    const int i = (int)(e - r * d);
    const int vpw = vals_per_word(bits);
    const uint32_t w = in[r * packed_words(d, bits) + i / vpw];
    out[e] = (w >> ((i % vpw) * bits)) & ((1u << bits) - 1u);
}

__global__ void __launch_bounds__(256)
    scalar_quantize_kernel(const float *v, int64_t n, const float *bnd, int nb, uint8_t *out) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const float x = v[e];
    unsigned cnt = 0;
    for (int b = 0; b < nb; ++b) cnt += x > bnd[b] ? 1u : 0u;
    out[e] = (uint8_t)cnt;
}

// Bit offset of token i inside an interleaved word: bits*(i/2) in the low
// half for even i, +16 for odd i.
__device__ __forceinline__ int il_pos(int bits, int i) { return bits * (i >> 1) + 16 * (i & 1); }

// Interleaved code layout of the fused grouped-value decode: per (b, h), word
// (blk, d) of [cap / vpw][D] holds dim d of tokens blk*vpw .. blk*vpw + vpw - 1,
// token i of the block at bit bits*(i/2) + 16*(i%2).  One thread per (block,
// dim) of the appended range; bits of tokens outside [offset, offset + n_t)
// are kept.
__global__ void __launch_bounds__(256)
    pack_grouped_il_kernel(const uint32_t *packed, int64_t n_h, int64_t n_t, int64_t p_sb,
                           int64_t p_sh, int64_t p_st, int d, int bits, uint32_t *out_il,
                           int64_t cap, int64_t offset, int64_t b0, int64_t n_blk) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t bh = blockIdx.y;  // b * n_h + h
    if (e >= n_blk * d) return;
    const int64_t blk = b0 + e / d;
    const int dd = (int)(e % d);
    const int vpw = vals_per_word(bits);
    const int nw = packed_words(d, bits);
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t b = bh / n_h, h = bh - b * n_h;
    uint32_t *wp = out_il + (bh * (cap / vpw) + blk) * d + dd;
    uint32_t word = *wp;
    for (int i = 0; i < vpw; ++i) {
        const int64_t t = blk * vpw + i - offset;  // row of the appended chunk
        if (t < 0 || t >= n_t) continue;
        const uint32_t w = packed[(b * p_sb + h * p_sh + t * p_st) * nw + dd / vpw];
        const uint32_t code = (w >> ((dd % vpw) * bits)) & mask;
        const int pos = il_pos(bits, i);
        word = (word & ~(mask << pos)) | (code << pos);
    }
    *wp = word;
}

// The inverse of pack_grouped_il_kernel: one thread per output packed word
// (row t of (B, H) row bh, word w) gathers its vpw dims' codes of token t.
__global__ void __launch_bounds__(256)
    grouped_il_unpack_kernel(const uint32_t *codes_il, int64_t n_t, int64_t cap, int d, int bits,
                             uint32_t *out) {
    const int nw = d / vals_per_word(bits);
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t bh = blockIdx.y;
    if (e >= n_t * nw) return;
    const int64_t t = e / nw;
    const int w = (int)(e - t * nw);
    const int vpw = vals_per_word(bits);
    const uint32_t mask = (1u << bits) - 1u;
    const int pos = il_pos(bits, (int)(t % vpw));
    const uint32_t *src = codes_il + (bh * (cap / vpw) + t / vpw) * d + w * vpw;
    uint32_t word = 0u;
    for (int k = 0; k < vpw; ++k) word |= ((src[k] >> pos) & mask) << (k * bits);
    out[bh * n_t * nw + e] = word;
}

// Interleaved codes -> values in the 8-token interleaved fp16 layout
// [cap_out/8][d][8] per (B, H) row: one thread per (row, code word, dim)
// decodes the word's vpw tokens, v = fp16(q * scale + zero) (multiply and add
// rounded separately in float32, as dequantize_grouped_kernel), and writes
// each 8-token group it covers as one 16-byte store.  Tokens at or past n_t
// inside the last group are written as zero; groups starting at or past n_t
// are not written.
__global__ void __launch_bounds__(256)
    grouped_il_to_il8_kernel(const uint32_t *codes_il, int64_t cap, int d, int bits, int group,
                             const void *scales, const void *zeros, int sz_dtype, int64_t sz_cap,
                             int64_t n_t, int64_t n_blk, __half *out, int64_t cap_out) {
#pragma clang fp contract(off)
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t bh = blockIdx.y;
    if (e >= n_blk * d) return;
    const int64_t blk = e / d;
    const int dd = (int)(e - blk * d);
    const int vpw = vals_per_word(bits);
    const uint32_t mask = (1u << bits) - 1u;
    const int n_groups = d / group;
    const uint32_t word = codes_il[(bh * (cap / vpw) + blk) * d + dd];
    for (int h8 = 0; h8 < vpw / 8; ++h8) {
        const int64_t t0 = blk * vpw + h8 * 8;
        if (t0 >= n_t) break;
        __half v8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t t = t0 + i;
            float x = 0.f;
            if (t < n_t) {
                const float q = (float)((word >> il_pos(bits, h8 * 8 + i)) & mask);
                const int64_t gi = (bh * sz_cap + t) * n_groups + dd / group;
                const float prod = q * load_as_f32(scales, sz_dtype, gi);
                x = prod + load_as_f32(zeros, sz_dtype, gi);
            }
            v8[i] = __float2half(x);
        }
        *reinterpret_cast<uint4 *>(out + ((bh * (cap_out / 8) + t0 / 8) * d + dd) * 8) =
            *reinterpret_cast<const uint4 *>(v8);
    }
}

static inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace ss

using namespace ss;

extern "C" int ss_quantize_values_grouped(const void *values, int v_dtype, int64_t n_b,
                                          int64_t n_h, int64_t n_t, int64_t v_sb, int64_t v_sh,
                                          int64_t v_st, int head_dim, int bits, int group_size,
                                          uint32_t *packed, void *scales, void *zeros,
                                          int sz_dtype, int64_t o_sb, int64_t o_sh, int64_t o_st,
                                          void *stream) {
    SS_REQUIRE(valid_dtype(v_dtype), "bad value dtype");
    SS_REQUIRE(sz_dtype == SS_F32 || sz_dtype == SS_F16, "scale/zero dtype must be f32 or f16");
    SS_REQUIRE(bits == 2 || bits == 3 || bits == 4, "bits must be 2, 3 or 4");
    SS_REQUIRE(group_size >= 1 && head_dim >= 1 && head_dim % group_size == 0,
               "head_dim %d not divisible by group_size %d", head_dim, group_size);
    SS_REQUIRE(!(bits == 2 && head_dim % 16) && !(bits == 4 && head_dim % 8),
               "head_dim %d cannot be packed at %d bits", head_dim, bits);
    SS_REQUIRE(n_b >= 0 && n_h >= 0 && n_t >= 0, "negative sizes");
    const int64_t n_tok = n_b * n_h * n_t;
    if (n_tok == 0) return SS_OK;
    SS_REQUIRE(values && packed && scales && zeros, "null pointer argument");
    SS_UNSUPPORTED(n_tok < (1LL << 32), "too many tokens for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(quantize_grouped_kernel, dim3(blocks_for(n_tok)), dim3(256), 0, st, values,
                       v_dtype, n_h, n_t, n_tok, v_sb, v_sh, v_st, head_dim, bits, group_size,
                       packed, scales, zeros, sz_dtype, o_sb, o_sh, o_st);
    SS_LAUNCH_CHECK("quantize_grouped_kernel launch");
    return SS_OK;
}

extern "C" int ss_dequantize_values_grouped(const uint32_t *packed, const void *scales,
                                            const void *zeros, int sz_dtype, int64_t n_tok,
                                            int head_dim, int bits, int group_size, void *out,
                                            int out_dtype, void *stream) {
    SS_REQUIRE(valid_dtype(out_dtype), "bad output dtype");
    SS_REQUIRE(sz_dtype == SS_F32 || sz_dtype == SS_F16, "scale/zero dtype must be f32 or f16");
    SS_REQUIRE(bits == 2 || bits == 3 || bits == 4, "bits must be 2, 3 or 4");
    SS_REQUIRE(group_size >= 1 && head_dim % group_size == 0, "bad group size");
    SS_REQUIRE(n_tok >= 0, "negative sizes");
    if (n_tok == 0) return SS_OK;
    SS_REQUIRE(packed && scales && zeros && out, "null pointer argument");
    const int64_t total = n_tok * head_dim;
    SS_UNSUPPORTED(total < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(dequantize_grouped_kernel, dim3(blocks_for(total)), dim3(256), 0, st,
                       packed, scales, zeros, sz_dtype, n_tok, head_dim, bits, group_size, out,
                       out_dtype);
    SS_LAUNCH_CHECK("dequantize_grouped_kernel launch");
    return SS_OK;
}

extern "C" int ss_pack_indices(const uint8_t *in, int64_t n_rows, int d, int bits, uint32_t *out,
                               void *stream) {
    SS_REQUIRE(bits == 2 || bits == 3 || bits == 4, "bits must be 2, 3 or 4");
    SS_REQUIRE(!(bits == 2 && d % 16), "last dim must be divisible by 16 for 2-bit, got %d", d);
    SS_REQUIRE(!(bits == 4 && d % 8), "last dim must be divisible by 8 for 4-bit, got %d", d);
    SS_REQUIRE(n_rows >= 0 && d >= 1, "bad sizes");
    if (n_rows == 0) return SS_OK;
    SS_REQUIRE(in && out, "null pointer argument");
    const int64_t total = n_rows * packed_words(d, bits);
    SS_UNSUPPORTED(total < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(pack_kernel, dim3(blocks_for(total)), dim3(256), 0, st, in, n_rows, d, bits,
                       out);
    SS_LAUNCH_CHECK("pack_kernel launch");
    return SS_OK;
}

extern "C" int ss_unpack_indices(const uint32_t *in, int64_t n_rows, int d, int bits,
                                 uint32_t *out, void *stream) {
    SS_REQUIRE(bits == 2 || bits == 3 || bits == 4, "bits must be 2, 3 or 4");
    SS_REQUIRE(n_rows >= 0 && d >= 1, "bad sizes");
    if (n_rows == 0) return SS_OK;
    SS_REQUIRE(in && out, "null pointer argument");
    const int64_t total = n_rows * d;
    SS_UNSUPPORTED(total < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(unpack_kernel, dim3(blocks_for(total)), dim3(256), 0, st, in, n_rows, d,
                       bits, out);
    SS_LAUNCH_CHECK("unpack_kernel launch");
    return SS_OK;
}

extern "C" int ss_scalar_quantize(const float *values, int64_t n, const float *boundaries,
                                  int n_boundaries, uint8_t *out, void *stream) {
    SS_REQUIRE(n >= 0 && n_boundaries >= 0 && n_boundaries <= 255, "bad sizes");
    if (n == 0) return SS_OK;
    SS_REQUIRE(values && out && (boundaries || n_boundaries == 0), "null pointer argument");
    SS_UNSUPPORTED(n < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(scalar_quantize_kernel, dim3(blocks_for(n)), dim3(256), 0, st, values, n,
                       boundaries, n_boundaries, out);
    SS_LAUNCH_CHECK("scalar_quantize_kernel launch");
    return SS_OK;
}

extern "C" int ss_pack_grouped_il(const uint32_t *packed, int64_t n_b, int64_t n_h, int64_t n_t,
                                  int64_t p_sb, int64_t p_sh, int64_t p_st, int head_dim, int bits,
                                  uint32_t *out_il, int64_t cap, int64_t offset, void *stream) {
    SS_REQUIRE(bits == 2 || bits == 4, "interleaved codes need bits 2 or 4 (got %d)", bits);
    SS_REQUIRE(head_dim >= 1 && head_dim % (32 / bits) == 0, "head_dim %d cannot be packed at %d bits",
               head_dim, bits);
    SS_REQUIRE(n_b >= 0 && n_h >= 0 && n_t >= 0 && offset >= 0, "negative sizes");
    SS_REQUIRE(cap % (32 / bits) == 0, "cap must be a multiple of %d", 32 / bits);
    SS_REQUIRE(offset + n_t <= cap, "append range [%lld, %lld) past cap %lld", (long long)offset,
               (long long)(offset + n_t), (long long)cap);
    if (n_b * n_h * n_t == 0) return SS_OK;
    SS_REQUIRE(packed && out_il, "null pointer argument");
    SS_UNSUPPORTED(n_b * n_h < 65536, "too many (batch, head) rows for one launch");
    const int vpw = 32 / bits;
    const int64_t b0 = offset / vpw, b1 = (offset + n_t - 1) / vpw;
    const int64_t n_blk = b1 - b0 + 1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(pack_grouped_il_kernel, dim3(blocks_for(n_blk * head_dim), (unsigned)(n_b * n_h)),
                       dim3(256), 0, st, packed, n_h, n_t, p_sb, p_sh, p_st, head_dim, bits, out_il,
                       cap, offset, b0, n_blk);
    SS_LAUNCH_CHECK("pack_grouped_il_kernel launch");
    return SS_OK;
}

extern "C" int ss_grouped_il_to_packed(const uint32_t *codes_il, int64_t n_bh, int64_t cap,
                                       int head_dim, int bits, int64_t n_t, uint32_t *out,
                                       void *stream) {
    SS_REQUIRE(bits == 2 || bits == 4, "interleaved codes need bits 2 or 4 (got %d)", bits);
    SS_REQUIRE(head_dim >= 1 && head_dim % (32 / bits) == 0, "head_dim %d cannot be packed at %d bits",
               head_dim, bits);
    SS_REQUIRE(n_bh >= 0 && n_t >= 0, "negative sizes");
    SS_REQUIRE(cap % (32 / bits) == 0 && n_t <= cap, "n_t %lld past cap %lld (a multiple of %d)",
               (long long)n_t, (long long)cap, 32 / bits);
    if (n_bh * n_t == 0) return SS_OK;
    SS_REQUIRE(codes_il && out, "null pointer argument");
    SS_UNSUPPORTED(n_bh < 65536, "too many (batch, head) rows for one launch");
    const int64_t total = n_t * (head_dim / (32 / bits));
    SS_UNSUPPORTED(total < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(grouped_il_unpack_kernel, dim3(blocks_for(total), (unsigned)n_bh), dim3(256),
                       0, st, codes_il, n_t, cap, head_dim, bits, out);
    SS_LAUNCH_CHECK("grouped_il_unpack_kernel launch");
    return SS_OK;
}

extern "C" int ss_grouped_il_to_il8(const uint32_t *codes_il, int64_t n_bh, int64_t cap,
                                    int head_dim, int bits, int group_size, const void *scales,
                                    const void *zeros, int sz_dtype, int64_t sz_cap, int64_t n_t,
                                    void *out_il8, int64_t cap_out, void *stream) {
    SS_REQUIRE(bits == 2 || bits == 4, "interleaved codes need bits 2 or 4 (got %d)", bits);
    SS_REQUIRE(sz_dtype == SS_F32 || sz_dtype == SS_F16, "scale/zero dtype must be f32 or f16");
    SS_REQUIRE(head_dim >= 1 && head_dim % (32 / bits) == 0, "head_dim %d cannot be packed at %d bits",
               head_dim, bits);
    SS_REQUIRE(group_size >= 1 && head_dim % group_size == 0,
               "group_size %d does not divide head_dim %d", group_size, head_dim);
    SS_REQUIRE(n_bh >= 0 && n_t >= 0, "negative sizes");
    SS_REQUIRE(cap % (32 / bits) == 0 && n_t <= cap, "n_t %lld past the codes' cap %lld",
               (long long)n_t, (long long)cap);
    SS_REQUIRE(n_t <= sz_cap, "n_t %lld past the scales' cap %lld", (long long)n_t,
               (long long)sz_cap);
    SS_REQUIRE(cap_out % 8 == 0 && n_t <= cap_out, "n_t %lld past cap_out %lld (a multiple of 8)",
               (long long)n_t, (long long)cap_out);
    if (n_bh * n_t == 0) return SS_OK;
    SS_REQUIRE(codes_il && scales && zeros && out_il8, "null pointer argument");
    SS_UNSUPPORTED(n_bh < 65536, "too many (batch, head) rows for one launch");
    const int vpw = 32 / bits;
    const int64_t n_blk = (n_t + vpw - 1) / vpw;
    const int64_t total = n_blk * head_dim;
    SS_UNSUPPORTED(total < (1LL << 32), "too many elements for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(grouped_il_to_il8_kernel, dim3(blocks_for(total), (unsigned)n_bh), dim3(256),
                       0, st, codes_il, cap, head_dim, bits, group_size, scales, zeros, sz_dtype,
                       sz_cap, n_t, n_blk, reinterpret_cast<__half *>(out_il8), cap_out);
    SS_LAUNCH_CHECK("grouped_il_to_il8_kernel launch");
    return SS_OK;
}
