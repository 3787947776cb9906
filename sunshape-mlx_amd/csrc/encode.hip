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
#include "encode_wave.hpp"

namespace ss {

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



// Index of block blk of token n (a wave per (token, block); lane 0 stores
// it).  8-dim blocks of at most 256 centroids take one memory round trip:
// the lane's centroids, the whole key row (dims lane + 64u, coalesced) and
// the block's permutation entries are loaded together, and the permuted
// dims come from their lanes by a shuffle; other shapes load the block's
// dims through the permutation (exact_block_wave).
template <int BD>
__device__ __forceinline__ void encode_block_wave(const EncodeArgs &a, int64_t n, int blk, int lane) {
    const TokAddr ad = token_addr(a, n);
    const int d = a.n_blocks * BD;
    if constexpr (BD == 8) {
        if (a.n_centroids <= 4 * kWave && d <= 4 * kWave) {
            const float *cbb = a.centroids + (int64_t)blk * a.n_centroids * 8;
            float4 cv[4][2];
            load_centroids8(cbb, a.n_centroids, lane, cv);
            float kr[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                kr[u] = lane + kWave * u < d ? load_as_f32(a.keys, a.keys_dtype, ad.key + lane + kWave * u)
                                             : 0.f;
            float kv[8];
            block_dims8(kr, a.perm, blk, kv);
            const int bi = exact_block_wave_regs8(kv, cv, cbb, a.n_centroids, lane);
            if (lane == 0) a.out[ad.out + blk] = (uint8_t)bi;
            return;
        }
    }
    float kv[BD];
#pragma unroll
    for (int k = 0; k < BD; ++k) {
        const int j = blk * BD + k;
        kv[k] = load_as_f32(a.keys, a.keys_dtype, ad.key + (a.perm ? a.perm[j] : j));
    }
    const int bi = exact_block_wave<BD>(kv, a.centroids + (int64_t)blk * a.n_centroids * BD,
                                        a.n_centroids, lane);
    if (lane == 0) a.out[ad.out + blk] = (uint8_t)bi;
}

// ---- small: wave per (token, block) ----
template <int BD>
__global__ void __launch_bounds__(kEncThreads) encode_small_kernel(EncodeArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t job = (int64_t)blockIdx.x * (kEncThreads / kWave) + (threadIdx.x >> 6);
    if (job >= a.n_tok * a.n_blocks) return;  // wave-uniform
    const int64_t n = job / a.n_blocks;
    const int blk = (int)(job - n * a.n_blocks);
    encode_block_wave<BD>(a, n, blk, lane);
}

// ---- decode-step KV append: keys encoded and values stored in one launch ----
//
// Workgroups [0, n_enc) run encode_small_kernel's waves (one per (token,
// block)); the rest store the tokens' values into the 8-token interleaved
// fp16 cache (cache_ops.hip's append_il8_kernel), one element per thread.
struct ValueAppend {
    const void *values;
    int v_dtype;
    int64_t v_sb, v_sh, v_st;
    int d;
    __half *out_il8;
    int64_t cap, offset;
};

template <int BD>
__global__ void __launch_bounds__(kEncThreads) append_kv_small_kernel(EncodeArgs a, ValueAppend v,
                                                                      int n_enc) {
    if ((int)blockIdx.x < n_enc) {
        const int lane = threadIdx.x & (kWave - 1);
        const int64_t job = (int64_t)blockIdx.x * (kEncThreads / kWave) + (threadIdx.x >> 6);
        if (job >= a.n_tok * a.n_blocks) return;  // wave-uniform
        const int64_t n = job / a.n_blocks;
        const int blk = (int)(job - n * a.n_blocks);
        encode_block_wave<BD>(a, n, blk, lane);
        return;
    }
    const int64_t e = (int64_t)(blockIdx.x - n_enc) * kEncThreads + threadIdx.x;
    if (e >= a.n_tok * v.d) return;
    const int64_t n = e / v.d;
    const int j = (int)(e - n * v.d);
    const int64_t b = n / (a.n_h * a.n_t);
    const int64_t rem = n - b * a.n_h * a.n_t;
    const int64_t h = rem / a.n_t;
    const int64_t t = rem - h * a.n_t;
    const float x = load_as_f32(v.values, v.v_dtype, b * v.v_sb + h * v.v_sh + t * v.v_st + j);
    store_value_il8(v.out_il8, b * a.n_h + h, v.cap, v.d, v.offset + t, j, x);
}

// ---- one decode step of a hybrid cache with grouped values (interleaved codes) ----
//
// Three kinds of workgroups in one launch:
//   [0, n_put):            the step's new keys and values stored into the
//                          full-precision buffer at buffer position put_pos;
//   [n_put, n_put + n_enc): a wave per (flushed token, block) encodes the
//                          oldest buffered keys (exact_block_wave);
//   the rest:              a wave per (head, interleaved code-word row) of
//                          the flushed range quantises its tokens' values with
//                          the grouped min/max rule of quantize_grouped_kernel
//                          (values.hip; the same IEEE steps, so codes and
//                          scale/zero are identical), lane l owning dims
//                          l*d/64 .., and rewrites its words, keeping the bits
//                          of tokens outside the range; a group's first lane
//                          stores that token's scale and zero.
// The flushed buffer range and the stored range are disjoint (checked on
// the host), so no workgroup reads what another writes.
struct HybridGroupedStep {
    // new tokens (n_b x n_h x n_new) and the buffer [n_b][n_h][buf_cap][d]
    const void *keys, *values;
    int kv_dtype;
    int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
    int64_t n_new;
    void *buf_keys, *buf_values;
    int buf_dtype;
    int64_t buf_cap, put_pos;
    // flushed buffer tokens [flush_pos, flush_pos + n_flush) -> compressed
    // positions [offset, offset + n_flush) of a cache of capacity cap
    int64_t flush_pos, n_flush, offset, cap;
    int d, bits, group;
    uint32_t *codes_il;  // [n_b][n_h][cap / (32 / bits)][d]
    void *scales, *zeros;
    int sz_dtype;
    int64_t blk0, n_blk;  // code words touched: word rows blk0 .. blk0 + n_blk - 1
    int64_t n_bh;         // batch x heads
};

template <int BD>
__global__ void __launch_bounds__(kEncThreads)
    hybrid_grouped_step_kernel(EncodeArgs a, HybridGroupedStep s, int n_put, int n_enc) {
    const int64_t n_bh = s.n_bh;
    if ((int)blockIdx.x < n_put) {
        const int64_t e = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
        const int64_t per = s.n_new * s.d;
        if (e >= 2 * n_bh * per) return;
        const bool is_v = e >= n_bh * per;
        const int64_t r = is_v ? e - n_bh * per : e;
        const int64_t bh = r / per, rem = r - bh * per;
        const int64_t t = rem / s.d;
        const int j = (int)(rem - t * s.d);
        const int64_t b = bh / a.n_h, h = bh - b * a.n_h;
        const float x = is_v ? load_as_f32(s.values, s.kv_dtype, b * s.v_sb + h * s.v_sh + t * s.v_st + j)
                             : load_as_f32(s.keys, s.kv_dtype, b * s.k_sb + h * s.k_sh + t * s.k_st + j);
        store_from_f32(is_v ? s.buf_values : s.buf_keys, s.buf_dtype,
                       (bh * s.buf_cap + s.put_pos + t) * s.d + j, x);
        return;
    }
    if ((int)blockIdx.x < n_put + n_enc) {
        const int lane = threadIdx.x & (kWave - 1);
        const int64_t job = (int64_t)(blockIdx.x - n_put) * (kEncThreads / kWave) + (threadIdx.x >> 6);
        if (job >= a.n_tok * a.n_blocks) return;  // wave-uniform
        const int64_t n = job / a.n_blocks;
        const int blk = (int)(job - n * a.n_blocks);
        encode_block_wave<BD>(a, n, blk, lane);
        return;
    }
    // values: a wave per (bh, code-word row) of the flushed range; lane l
    // owns dims l * dpl .. + dpl - 1 (dpl = d / 64), so a token's group
    // min / max is a reduction over the group's aligned lanes and each
    // token costs one load per lane
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t job = (int64_t)(blockIdx.x - n_put - n_enc) * (kEncThreads / kWave) +
                        (threadIdx.x >> 6);
    if (job >= n_bh * s.n_blk) return;  // wave-uniform
    const int64_t bh = job / s.n_blk;
    const int64_t blk = s.blk0 + (job - bh * s.n_blk);
    const int dpl = s.d / kWave;         // 1 or 2 (checked on the host)
    const int glanes = s.group / dpl;    // lanes of one group: 32 or 64
    const int vpw = 32 / s.bits;
    const uint32_t mask = (1u << s.bits) - 1u;
    const float maxv = (float)((1 << s.bits) - 1);
    const int n_groups = s.d / s.group;
    uint32_t *wp = s.codes_il + (bh * (s.cap / vpw) + blk) * s.d + lane * dpl;
    uint32_t word[2] = {wp[0], dpl > 1 ? wp[1] : 0u};
    for (int i = 0; i < vpw; ++i) {
        const int64_t t = blk * vpw + i - s.offset;  // flushed token of this slot
        if (t < 0 || t >= s.n_flush) continue;       // wave-uniform
        const int64_t vin = (bh * s.buf_cap + s.flush_pos + t) * s.d + lane * dpl;
        float x[2];
        x[0] = load_as_f32(s.buf_values, s.buf_dtype, vin);
        x[1] = dpl > 1 ? load_as_f32(s.buf_values, s.buf_dtype, vin + 1) : x[0];
        float mn = fminf(x[0], x[1]), mx = fmaxf(x[0], x[1]);
        for (int o = glanes / 2; o > 0; o >>= 1) {
            mn = fminf(mn, __shfl_xor(mn, o));
            mx = fmaxf(mx, __shfl_xor(mx, o));
        }
        float sc = __fdiv_rn(__fsub_rn(mx, mn), maxv);
        if (sc < 1e-8f) sc = 1e-8f;
        // token i of the word: bits*(i/2) in the low half for even i, +16 for odd i
        const int pos = s.bits * (i >> 1) + 16 * (i & 1);
        for (int k = 0; k < dpl; ++k) {
            float qf = rintf(__fdiv_rn(__fsub_rn(x[k], mn), sc));
            qf = fminf(fmaxf(qf, 0.f), maxv);
            word[k] = (word[k] & ~(mask << pos)) | (((uint32_t)qf & mask) << pos);
        }
        if (lane % glanes == 0) {
            const int64_t srow = (bh * s.cap + s.offset + t) * n_groups + lane / glanes;
            store_from_f32(s.scales, s.sz_dtype, srow, sc);
            store_from_f32(s.zeros, s.sz_dtype, srow, mn);
        }
    }
    wp[0] = word[0];
    if (dpl > 1) wp[1] = word[1];
}

// ---- bulk on the matrix cores (block_dim 8): a bounded filter, then exact ties ----
//
// Per block b the codebook and the keys are scaled by s_b, a power of two
// that brings the block's largest centroid element into [8, 16) (exact),
// and split into fp16 parts x = x_hi + x_lo (x_lo = fp16(x - x_hi)).  Two
// v_mfma_f32_32x32x16_f16 (32 centroids x 32 tokens, the second
// accumulating onto the first) give
//
//   D(c) = (1-e)|y_c|^2 - 2 x.y_c + (1+e)|x|^2 + 2e max_c|y_c|^2 + 3 a0
//
// (K slots: -2x_hi.y_hi, -2x_hi.y_lo, -2x_lo.y_hi, the split (1-e)|y_c|^2
// and the split constant), fp16 products exact, fp32 sums.  Its float error
// e'(c) is below e_acc (2|x|^2 + 2|y_c|^2) + a_abs, e_acc < 2^-16.9 (33 fp32
// additions rounded either way; the 2^-22 relative / 2^-25 absolute split
// error of each operand), a_abs < 2^-21; with e = 2^-15 and a0 = 2^-19:
//   * D(c) >= 0, so D's bits order as unsigned integers (no float min/max
//     canonicalisation, no denormal flushing);
//   * for any two centroids, d(c) - d(c1) >= D(c) - D(c1)
//     - 2e (|x|^2 + |y_c1|^2) - 2 a0 (d the exact squared distance).
// Each lane keeps the two smallest D of its 128 centroids (16 per product,
// 8 tiles), with (tile, register) in the low 7 mantissa bits (at most 127
// ulps, 2^-16 relative); the two lane halves of a token are merged into the
// smallest D1 (centroid c1) and the runner-up D2.  If D2 - D1 exceeds
// 2e (|x|^2 + |y_c1|^2) + 2 a0 + 2^-15 D2, every other centroid's exact
// distance exceeds c1's, and c1 is the exact nearest codeword.  Otherwise
// the (token, block) joins a per-wave queue ranked exactly by the whole
// wave (exact_block_wave: direct-form float32, float64 on near-ties), as do
// keys outside the scaled fp16 range and blocks with non-finite centroids.
// The index is therefore the exact-arithmetic argmin with lowest-index
// ties, the same as encode_bulk_kernel's.
//
// Persistent workgroups of 16 waves, one per CU: wave b owns block b and
// keeps its 256 centroids' operands in registers for the whole launch;
// each tile of 128 tokens is gathered (permuted, scaled, split) into LDS by
// all threads, with the next tile's loads in flight during the products.
constexpr int kEmTokens = 128;   // tokens per tile (4 groups of 32)
constexpr int kEmWaves = 16;     // wave b ranks block b
constexpr int kEmQueue = 64;     // per-wave queue of (token, block) to rank exactly
constexpr float kEmEps = 1.0f / 32768.f;
constexpr float kEmAbs = 1.0f / 524288.f;
constexpr int kEmTiles = 8;      // 8 centroid tiles of 32
constexpr float kEmMaxQ = 60000.f;  // |x|^2 bound: the split constant stays in fp16

template <class T>
using lds_ptr = __attribute__((address_space(3))) T *;
typedef _Float16 em_f16x8 __attribute__((ext_vector_type(8)));
typedef float em_f32x16 __attribute__((ext_vector_type(16)));

// median of three unsigned words in one v_med3_u32 (the compiler expands the
// min/max form into two instructions)
__device__ __forceinline__ uint32_t umed3(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

struct EncOps {  // the prepared codebook (ss_encode_codebook)
    static size_t ops_bytes(int nb) { return (size_t)nb * kEmTiles * kWave * 16; }  // A operands
    static size_t qpk_bytes(int nb) { return (size_t)nb * 256 * 4; }                // split (1-e)|y|^2
    static size_t n2_bytes(int nb) { return (size_t)nb * 256 * 4; }                 // |y|^2
    // then [nb] scales s_b and [nb] max |y|^2
    static size_t bytes(int nb) {
        return ops_bytes(nb) + qpk_bytes(nb) + n2_bytes(nb) + (((size_t)nb * 8 + 15) & ~size_t(15));
    }
};

// One workgroup per block: the scale s_b, then for centroid c of tile
// t = c/32 its A operand (lane c%32: y_hi, lane 32 + c%32: y_lo), the split
// (1-e)|y_c|^2 (fp16 hi, lo packed in a word), |y_c|^2 and the block's max
// |y|^2.  A codebook with a non-finite entry gets s_b = 0 (every token of
// the block ranked exactly).
__global__ void __launch_bounds__(256) encode_codebook_kernel(const float *cents, int nb, int nc,
                                                              uint4 *ops, uint32_t *qpk, float *n2t,
                                                              float *sig) {
    __shared__ float red[256];
    const int b = blockIdx.x, c = threadIdx.x;
    float y[8];
    float ma = 0.f;
    bool fin = true;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        y[d] = c < nc ? cents[((int64_t)b * nc + c) * 8 + d] : 0.f;
        fin = fin && fabsf(y[d]) <= 3.0e38f;
        ma = fmaxf(ma, fabsf(y[d]));
    }
    const int bad = __syncthreads_or(!fin);
    red[c] = fin ? ma : 0.f;
    __syncthreads();
    for (int s2 = 128; s2 > 0; s2 >>= 1) {
        if (c < s2) red[c] = fmaxf(red[c], red[c + s2]);
        __syncthreads();
    }
    float sg = 1.f;
    if (red[0] > 0.f) {
        int e;
        frexpf(red[0], &e);
        sg = ldexpf(1.f, min(max(4 - e, -120), 120));
    }
    if (bad) sg = 0.f;
    if (c == 0) sig[b] = sg;
    em_f16x8 hi, lo;
    float q = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        const float x = bad ? 0.f : y[d] * sg;
        hi[d] = (_Float16)x;
        lo[d] = (_Float16)(x - (float)hi[d]);
        q = fmaf(x, x, q);
    }
    const float qs = q * (1.f - kEmEps);
    const _Float16 qh = (_Float16)qs, ql = (_Float16)(qs - (float)qh);
    uint4 *o = ops + ((int64_t)b * kEmTiles + (c >> 5)) * kWave + (c & 31);
    o[0] = __builtin_bit_cast(uint4, hi);
    o[32] = __builtin_bit_cast(uint4, lo);
    qpk[b * 256 + c] = (uint32_t)__builtin_bit_cast(uint16_t, qh) | ((uint32_t)__builtin_bit_cast(uint16_t, ql) << 16);
    n2t[b * 256 + c] = q;
    __syncthreads();
    red[c] = q;
    __syncthreads();
    for (int s2 = 128; s2 > 0; s2 >>= 1) {
        if (c < s2) red[c] = fmaxf(red[c], red[c + s2]);
        __syncthreads();
    }
    if (c == 0) sig[nb + b] = red[0];
}

// a key element from its LDS-DMA dword slot (2-byte types in the low half)
template <class KT>
__device__ __forceinline__ float slot_f32(uint32_t w) {
    if constexpr (std::is_same<KT, float>::value) return __uint_as_float(w);
    else if constexpr (std::is_same<KT, __half>::value) return __half2float(__ushort_as_half((unsigned short)w));
    else return __uint_as_float(w << 16);
}

// LDS of encode_mfma_kernel (one workgroup per CU)
template <class KT>
struct EmLds {
    static constexpr bool KLO = !std::is_same<KT, __half>::value;  // keys carry an fp16 lo part
    static constexpr int T = KLO ? 64 : 128;                      // tokens per tile
    static constexpr int KW = KLO ? 32 : 16;                      // key operand bytes per (token, block)
    static size_t bytes(int nb) {
        return (size_t)T * (nb * KW + 16)          // operands
               + (size_t)T * nb * 9                // split constant, |x|^2, indices
               + (size_t)nb * 8 * 4                // permutation
               + (size_t)kEmWaves * kEmQueue * 4   // queues
               + (size_t)kEmWaves * 4              // queue lengths
               + (size_t)kEmWaves * 256 * 4        // split (1-e)|y_c|^2 of each wave's block
               + (size_t)T * nb * 8 * sizeof(KT);  // the next tile's key rows
    }
};

template <class KT, bool FULL>  // key element type; FULL: 256 centroids (no partial tile)
__global__ void __launch_bounds__(kEmWaves * kWave)
    encode_mfma_kernel(EncodeArgs a, const uint4 *ops, const uint32_t *qpk, const float *n2t, const float *sig) {
    using L = EmLds<KT>;
    constexpr bool KLO = L::KLO;
    constexpr int T = L::T, KW = L::KW;
    constexpr int TH = kEmWaves * kWave;
    const int NB = a.n_blocks, nc = a.n_centroids, nt = FULL ? kEmTiles : (nc + 31) >> 5;
    // token rows padded by 16 bytes: consecutive tokens' 16-byte reads hit
    // distinct bank groups
    const int tstr = NB * KW + 16;
    extern __shared__ __align__(16) char sm[];
    char *kop = sm;                                                // [T][tstr]: -2 x_hi (, -2 x_lo)
    uint32_t *kck = reinterpret_cast<uint32_t *>(sm + T * tstr);   // [T][NB] split constant (fp16 hi, lo)
    float *kn2 = reinterpret_cast<float *>(kck + T * NB);          // [T][NB] |x|^2 (-1: rank exactly)
    uint32_t *qw = reinterpret_cast<uint32_t *>(kn2 + T * NB);     // [kEmWaves][256] split (1-e)|y_c|^2
    int *perm_l = reinterpret_cast<int *>(qw + kEmWaves * 256);    // [NB * 8]
    int *queue = perm_l + NB * 8;                                  // [kEmWaves][kEmQueue]
    int *qlen = queue + kEmWaves * kEmQueue;                       // [kEmWaves]
    KT *raw = reinterpret_cast<KT *>(qlen + kEmWaves);             // [T][D] key rows of the tile
    uint8_t *oix = reinterpret_cast<uint8_t *>(raw + T * NB * 8);  // [T][NB] indices
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int D = NB * 8;
    const int64_t n_tiles = (a.n_tok + T - 1) / T;
    const bool owner = wv < NB;  // this wave ranks block wv
    // 16 blocks and 16-byte aligned output rows: whole rows are stored at once
    const bool out16 = NB == 16 && ((uintptr_t)a.out % 16) == 0 && a.o_sb % 16 == 0 && a.o_sh % 16 == 0 &&
                       a.o_st % 16 == 0;

    for (int j = tid; j < D; j += TH) perm_l[j] = a.perm ? min(max(a.perm[j], 0), D - 1) : j;
    for (int j = tid; j < kEmWaves * 256; j += TH) qw[j] = (j >> 8) < NB ? qpk[j] : 0u;
    // this wave's codebook operand (block wv), kept for the whole launch:
    // Y[t] (lanes 0-31 y_hi, 32-63 y_lo of centroid 32t + lane%32)
    em_f16x8 Y[kEmTiles];
    if (owner) {
#pragma unroll
        for (int t = 0; t < kEmTiles; ++t)
            if (t < nt) Y[t] = __builtin_bit_cast(em_f16x8, ops[((int64_t)wv * kEmTiles + t) * kWave + lane]);
    }
    const uint32_t *qb = qw + (owner ? wv : 0) * 256;
    __syncthreads();

    // The tile's key rows are copied whole into LDS (global_load_lds of 16
    // bytes per lane: 64 lanes move 1 KB of consecutive rows), issued one
    // tile ahead; the permutation is applied from LDS.  Rows are 16-byte
    // aligned (checked by the host).
    constexpr int RC = 16 / (int)sizeof(KT);     // elements per 16-byte chunk
    const int row_chunks = D / RC;               // chunks per key row
    const int n_chunks = T * row_chunks;         // chunks per tile
    const uint32_t raw_l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(raw));
    auto gather = [&](int64_t tile) {
        if (tile >= n_tiles) return;
        for (int c0 = wv * kWave; c0 < n_chunks; c0 += TH) {  // wave-uniform
            const int c = c0 + lane;
            const int row = c / row_chunks, ch = c - row * row_chunks;
            const int64_t n = min(tile * T + row, a.n_tok - 1);  // clamped: stays in bounds
            const KT *src = static_cast<const KT *>(a.keys) + token_addr(a, n).key + ch * RC;
            if (c < n_chunks)
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const char *>(src),
                                                 reinterpret_cast<lds_ptr<void>>(raw_l + (uint32_t)c0 * 16u), 16, 0, 0);
        }
    };
    // permute, scale, range-check and split the tile's keys into the LDS
    // operands: item i = (token i / NB, block i % NB)
    auto stage = [&](int64_t tile) {
        for (int i = tid; i < T * NB; i += TH) {
            const int tl = i / NB, b = i - tl * NB;
            const bool live = tile * T + tl < a.n_tok;
            const float sg = sig[b];
            const KT *xr = raw + tl * D;
            float q = 0.f;
            em_f16x8 h, l;
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const float xs = to_f32(xr[perm_l[b * 8 + d]]) * sg;
                q = fmaf(xs, xs, q);
                h[d] = (_Float16)xs;
                l[d] = (_Float16)(xs - (float)h[d]);
            }
            // NaN, inf and keys too far out for the fp16 operands fail
            const bool ok = live && sg > 0.f && q < kEmMaxQ;
            if (!ok) h = l = em_f16x8{};
            *reinterpret_cast<em_f16x8 *>(kop + tl * tstr + b * KW) = h * (_Float16)(-2.0f);
            if constexpr (KLO) *reinterpret_cast<em_f16x8 *>(kop + tl * tstr + b * KW + 16) = l * (_Float16)(-2.0f);
            const float ck = ok ? fmaf(q, 1.f + kEmEps, fmaf(2.f * kEmEps, sig[NB + b], 3.f * kEmAbs)) : 0.f;
            const _Float16 ch = (_Float16)ck, cl = (_Float16)(ck - (float)ch);
            kck[i] = (uint32_t)__builtin_bit_cast(uint16_t, ch) | ((uint32_t)__builtin_bit_cast(uint16_t, cl) << 16);
            kn2[i] = ok ? q : -1.f;
        }
    };

    const int h = lane >> 5, j32 = lane & 31;
    int *wq = queue + wv * kEmQueue;
    int qn = 0;  // entries in this wave's queue (wave-uniform)
    // Rank the queued (iteration, token, block) entries exactly, the whole
    // wave per entry.  Each lane first loads the key elements of entry
    // lane (one memory round trip for the batch).  Entries of the tile in
    // progress (iteration cur) go to its LDS indices; earlier tiles' rows
    // have been stored already, so theirs go straight to the output.
    // Rank n_ent entries exactly, the whole wave per entry; entry j is
    // ent_of(j) = (iteration << 15) | (token << 8) | block.  Each lane first
    // loads the key elements of entry lane (one memory round trip per 64
    // entries).  Entries of the tile in progress (iteration cur) go to its
    // LDS indices; earlier tiles' rows are stored already, so theirs go
    // straight to the output.
    auto rank_entries = [&](int n_ent, auto ent_of, int cur) {
        for (int j0 = 0; j0 < n_ent; j0 += kWave) {
            const int ent_l = j0 + lane < n_ent ? ent_of(j0 + lane) : 0;
            const int it_l = ent_l >> 15, tl_l = (ent_l >> 8) & 127, b_l = ent_l & 255;
            const int64_t n_l = min(((int64_t)blockIdx.x + (int64_t)it_l * gridDim.x) * T + tl_l, a.n_tok - 1);
            const TokAddr ad_l = token_addr(a, n_l);
            float kvl[8];
#pragma unroll
            for (int d = 0; d < 8; ++d)
                kvl[d] = to_f32(static_cast<const KT *>(a.keys)[ad_l.key + perm_l[min(b_l, NB - 1) * 8 + d]]);
            const int ne = min(n_ent - j0, kWave);
            for (int e = 0; e < ne; ++e) {
                float kv[8];
#pragma unroll
                for (int d = 0; d < 8; ++d) kv[d] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kvl[d]), e));
                const int ent = __builtin_amdgcn_readlane(ent_l, e);
                const int it = ent >> 15, tl = (ent >> 8) & 127, b = ent & 255;
                const int bi = exact_block_wave<8>(kv, a.centroids + (int64_t)b * nc * 8, nc, lane);
                if (lane == 0) {
                    if (it == cur)
                        oix[tl * NB + b] = (uint8_t)bi;
                    else
                        a.out[token_addr(a, ((int64_t)blockIdx.x + (int64_t)it * gridDim.x) * T + tl).out + b] =
                            (uint8_t)bi;
                }
            }
        }
    };
    // this wave's queue, when full
    auto flush = [&](int cur) {
        wave_lds_sync();
        rank_entries(qn, [&](int j) { return wq[j]; }, cur);
        wave_lds_sync();
        qn = 0;
    };

    int64_t tile = blockIdx.x;
    gather(tile);
    for (int it = 0; tile < n_tiles; tile += gridDim.x, ++it) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's row copies have landed
        __syncthreads();                                     // ... and every other wave's
        stage(tile);
        __syncthreads();
        gather(tile + gridDim.x);  // the next tile's keys stream in during the products
        if (owner) {
            const int b = wv;
            for (int q0 = 0; q0 < T; q0 += 32) {
                const int tl = q0 + j32;
                // products per centroid tile (32 centroids x 32 tokens):
                //   Y . [-2x_hi; -2x_hi]       y_hi.x_hi (lanes 0-31), y_lo.x_hi (32-63)
                //   Y . [-2x_lo; -2x_lo]       (float32 / bfloat16 keys)
                //   [q_hi, q_lo, 1, 1, 0..] . [1, 1, c_hi, c_lo, 0..; 0]   (1-e)|y|^2 + constant
                const em_f16x8 B0 = *reinterpret_cast<const em_f16x8 *>(kop + tl * tstr + b * KW);
                em_f16x8 B1 = {};
                if constexpr (KLO) B1 = *reinterpret_cast<const em_f16x8 *>(kop + tl * tstr + b * KW + 16);
                em_f16x8 B3 = {};
                if (h == 0) {
                    const uint32_t ck = kck[tl * NB + b];
                    B3[0] = (_Float16)1.0f;
                    B3[1] = (_Float16)1.0f;
                    B3[2] = __builtin_bit_cast(_Float16, (uint16_t)(ck & 0xffffu));
                    B3[3] = __builtin_bit_cast(_Float16, (uint16_t)(ck >> 16));
                }
                // two trackers (tiles 0-3 and 4-7), so the (tile, register)
                // code stays an inline constant (0..63) of v_and_or_b32
                uint32_t m1[2] = {0xffffffffu, 0xffffffffu}, m2[2] = {0xffffffffu, 0xffffffffu};
#pragma unroll
                for (int t = 0; t < kEmTiles; ++t) {
                    if (FULL || t < nt) {
                        em_f32x16 Dv = __builtin_amdgcn_mfma_f32_32x32x16_f16(Y[t], B0, em_f32x16{}, 0, 0, 0);
                        if constexpr (KLO) Dv = __builtin_amdgcn_mfma_f32_32x32x16_f16(Y[t], B1, Dv, 0, 0, 0);
                        const em_f16x8 A3 =
                            __builtin_bit_cast(em_f16x8, uint4{qb[32 * t + (lane & 31)], 0x3c003c00u, 0u, 0u});
                        Dv = __builtin_amdgcn_mfma_f32_32x32x16_f16(A3, B3, Dv, 0, 0, 0);
                        const int hk = t >> 2;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            uint32_t p = (__float_as_uint(Dv[r]) & 0xffffff80u) | (uint32_t)((t & 3) * 16 + r);
                            // centroid row of register r: 8*(r/4) + 4*h + r%4
                            if (!FULL && t == nt - 1)
                                p = (32 * t + 8 * (r >> 2) + 4 * h + (r & 3) < nc) ? p : 0xffffffffu;
                            m2[hk] = umed3(m1[hk], m2[hk], p);
                            m1[hk] = min(m1[hk], p);
                        }
                    }
                }
                // the two trackers (codes of tiles 4-7 get 64 added) ...
                const bool lo_win = m1[0] < m1[1];
                const uint32_t t2 = umed3(m1[0], m1[1], min(m2[0], m2[1]));
                const uint32_t t1 = lo_win ? m1[0] : m1[1];
                const int tcode = (int)(t1 & 63u) + (lo_win ? 0 : 64);
                // ... then the token's other lane half (centroid rows 4..7 of each 8)
                const uint32_t o1 = __shfl_xor(t1, 32), o2 = __shfl_xor(t2, 32);
                const int ocode = __shfl_xor(tcode, 32);
                const uint32_t M2 = umed3(t1, o1, min(t2, o2));
                const bool mine = t1 < o1;
                const uint32_t M1 = mine ? t1 : o1;
                const int hw = mine ? h : 1 - h;
                const int code = mine ? tcode : ocode, rr = code & 15;
                const int C1 = 32 * (code >> 4) + 8 * (rr >> 2) + 4 * hw + (rr & 3);
                const bool tok = h == 0 && tile * T + tl < a.n_tok;
                const float qk = kn2[tl * NB + b];
                bool accept = false;
                if (tok && qk >= 0.f && C1 < nc && t1 != o1) {
                    // |y_c1|^2 from its split (1-e)|y|^2, rounded up
                    const uint32_t qv = qb[C1];
                    const float qc = ((float)__builtin_bit_cast(_Float16, (uint16_t)(qv & 0xffffu)) +
                                      (float)__builtin_bit_cast(_Float16, (uint16_t)(qv >> 16))) *
                                     (1.f + 2.f * kEmEps);
                    const float f1 = __uint_as_float(M1), f2 = __uint_as_float(M2);
                    const float win = fmaf(2.01f * kEmEps, qk + qc, 2.f * kEmAbs) + f2 * (1.f / 32768.f);
                    // M2 = 0xffffffff (NaN): a single centroid, nothing to beat
                    accept = f2 - f1 > win || M2 == 0xffffffffu;
                }
                if (tok && accept) oix[tl * NB + b] = (uint8_t)C1;
                const bool need = tok && !accept;
                const uint64_t bal = __ballot(need);
                if (need) {
                    const int pos = qn + (int)__builtin_amdgcn_mbcnt_hi(
                                             (uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
                    wq[pos] = (it << 15) | (tl << 8) | b;
                }
                qn += __popcll(bal);
                if (qn > kEmQueue - 32) flush(it);
            }
            // entries wait for a full queue or the end of the launch (the
            // iteration field holds 16 bits)
            if (it >= 0xfffe && qn > 0) flush(it);
        }
        __syncthreads();
        if (out16) {  // one 16-byte store per token row
            if (tid < T && tile * T + tid < a.n_tok)
                *reinterpret_cast<uint4 *>(a.out + token_addr(a, tile * T + tid).out) =
                    *reinterpret_cast<const uint4 *>(oix + tid * 16);
        } else {
            for (int i = tid; i < T * NB; i += TH) {
                const int tl = i / NB, b = i - tl * NB;
                const int64_t n = tile * T + tl;
                if (n < a.n_tok) a.out[token_addr(a, n).out + b] = oix[i];
            }
        }
    }
    // What is left in the queues is ranked by all 16 waves together (entry
    // k of the concatenated queues by wave k % 16); the last tile's rows are
    // stored, ordered before these stores by the barrier.
    if (lane == 0) qlen[wv] = owner ? qn : 0;
    __syncthreads();
    int tot = 0;
#pragma unroll
    for (int q = 0; q < kEmWaves; ++q) tot += qlen[q];
    const int mine = tot > wv ? (tot - wv + kEmWaves - 1) / kEmWaves : 0;
    rank_entries(mine, [&](int j) {
        int k = wv + j * kEmWaves;  // index into the concatenated queues
        int q = 0;
        while (k >= qlen[q]) k -= qlen[q++];
        return queue[q * kEmQueue + k];
    }, -1);
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

static int encode_impl(const void *keys, int keys_dtype, int64_t n_b, int64_t n_h, int64_t n_t,
                       int64_t k_sb, int64_t k_sh, int64_t k_st, int head_dim, const int32_t *perm,
                       const float *centroids, int n_blocks, int n_centroids, int block_dim,
                       uint8_t *out, int64_t o_sb, int64_t o_sh, int64_t o_st, const void *prepared,
                       void *stream) {
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
    // the matrix-core encoder copies whole key rows in 16-byte pieces
    const int ksz = dtype_bytes(keys_dtype);
    const bool rows16 = ((uintptr_t)keys % 16) == 0 && (k_sb * ksz) % 16 == 0 && (k_sh * ksz) % 16 == 0 &&
                        (k_st * ksz) % 16 == 0;
    if (prepared && rows16 && block_dim == 8 && n_blocks <= 16 && n_tok * n_blocks > 4096) {
        SS_REQUIRE(((uintptr_t)prepared % 16) == 0, "prepared codebook must be 16-byte aligned");
        const char *p = static_cast<const char *>(prepared);
        const uint4 *ops = reinterpret_cast<const uint4 *>(p);
        const uint32_t *qpk = reinterpret_cast<const uint32_t *>(p + EncOps::ops_bytes(n_blocks));
        const float *n2t =
            reinterpret_cast<const float *>(p + EncOps::ops_bytes(n_blocks) + EncOps::qpk_bytes(n_blocks));
        const float *sig = n2t + (size_t)n_blocks * 256;
        auto go = [&](auto kt, auto full) -> int {
            using KT = decltype(kt);
            constexpr bool FULL = decltype(full)::value;
            const size_t lds = EmLds<KT>::bytes(n_blocks);
            const void *fn = reinterpret_cast<const void *>(encode_mfma_kernel<KT, FULL>);
            if (lds > 65536) {
                hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(encode_mfma)");
            }
            const int64_t n_tiles = (n_tok + EmLds<KT>::T - 1) / EmLds<KT>::T;
            dim3 grid((unsigned)std::min<int64_t>(n_tiles, device_cu_count()));
            hipLaunchKernelGGL((encode_mfma_kernel<KT, FULL>), grid, dim3(kEmWaves * kWave), lds, st, a, ops,
                               qpk, n2t, sig);
            return SS_OK;
        };
        auto go2 = [&](auto kt) -> int {
            return n_centroids == 256 ? go(kt, std::true_type{}) : go(kt, std::false_type{});
        };
        const int rc = keys_dtype == SS_F16 ? go2(__half{}) : keys_dtype == SS_BF16 ? go2(__hip_bfloat16{}) : go2(float{});
        if (rc != SS_OK) return rc;
        SS_LAUNCH_CHECK("encode_mfma_kernel launch");
        return SS_OK;
    }
    if (block_dim == 8) return launch_encode<8>(a, st);
    if (block_dim == 4) return launch_encode<4>(a, st);
    return launch_encode<16>(a, st);
}

extern "C" int ss_encode_blockvq(const void *keys, int keys_dtype, int64_t n_b, int64_t n_h,
                                 int64_t n_t, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                 int head_dim, const int32_t *perm, const float *centroids,
                                 int n_blocks, int n_centroids, int block_dim, uint8_t *out,
                                 int64_t o_sb, int64_t o_sh, int64_t o_st, void *stream) {
    return encode_impl(keys, keys_dtype, n_b, n_h, n_t, k_sb, k_sh, k_st, head_dim, perm, centroids,
                       n_blocks, n_centroids, block_dim, out, o_sb, o_sh, o_st, nullptr, stream);
}

extern "C" size_t ss_encode_codebook_bytes(int n_blocks) {
    return n_blocks > 0 ? EncOps::bytes(n_blocks) : 0;
}

extern "C" int ss_encode_codebook(const float *centroids, int n_blocks, int n_centroids,
                                  int block_dim, void *prepared, void *stream) {
    SS_REQUIRE(centroids && prepared, "null pointer argument");
    SS_UNSUPPORTED(block_dim == 8, "block_dim %d unsupported for the prepared codebook (8)", block_dim);
    SS_UNSUPPORTED(n_blocks >= 1 && n_blocks <= 16, "n_blocks %d unsupported (1..16)", n_blocks);
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256, "n_centroids %d unsupported (1..256)",
                   n_centroids);
    SS_REQUIRE(((uintptr_t)prepared % 16) == 0, "prepared codebook must be 16-byte aligned");
    char *p = static_cast<char *>(prepared);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint32_t *qpk = reinterpret_cast<uint32_t *>(p + EncOps::ops_bytes(n_blocks));
    float *n2t = reinterpret_cast<float *>(p + EncOps::ops_bytes(n_blocks) + EncOps::qpk_bytes(n_blocks));
    hipLaunchKernelGGL(encode_codebook_kernel, dim3(n_blocks), dim3(256), 0, st, centroids, n_blocks,
                       n_centroids, reinterpret_cast<uint4 *>(p), qpk, n2t, n2t + (size_t)n_blocks * 256);
    SS_LAUNCH_CHECK("encode_codebook_kernel launch");
    return SS_OK;
}

extern "C" int ss_encode_blockvq_prepared(const void *keys, int keys_dtype, int64_t n_b, int64_t n_h,
                                          int64_t n_t, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                          int head_dim, const int32_t *perm, const float *centroids,
                                          int n_blocks, int n_centroids, int block_dim, uint8_t *out,
                                          int64_t o_sb, int64_t o_sh, int64_t o_st,
                                          const void *prepared, void *stream) {
    return encode_impl(keys, keys_dtype, n_b, n_h, n_t, k_sb, k_sh, k_st, head_dim, perm, centroids,
                       n_blocks, n_centroids, block_dim, out, o_sb, o_sh, o_st, prepared, stream);
}

extern "C" int ss_append_kv_il8(const void *keys, int keys_dtype, const void *values, int v_dtype,
                                int64_t n_b, int64_t n_h, int64_t n_t, int64_t k_sb, int64_t k_sh,
                                int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int head_dim,
                                const int32_t *perm, const float *centroids, int n_blocks,
                                int n_centroids, int block_dim, const void *prepared,
                                uint8_t *idx_cache, void *values_il8, int64_t cap, int64_t offset,
                                void *stream) {
    SS_REQUIRE(valid_dtype(keys_dtype) && valid_dtype(v_dtype), "bad key or value dtype");
    SS_REQUIRE(n_b >= 0 && n_h >= 0 && n_t >= 0, "negative token counts");
    SS_REQUIRE(head_dim > 0 && block_dim > 0 && n_blocks * block_dim == head_dim,
               "n_blocks (%d) * block_dim (%d) != head_dim (%d)", n_blocks, block_dim, head_dim);
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256,
                   "n_centroids %d unsupported for uint8 indices (1..256)", n_centroids);
    SS_UNSUPPORTED(block_dim == 4 || block_dim == 8 || block_dim == 16,
                   "block_dim %d unsupported (4, 8, 16)", block_dim);
    SS_REQUIRE(cap % 8 == 0, "cap must be a multiple of 8");
    SS_REQUIRE(offset >= 0 && offset + n_t <= cap, "tokens [%lld, %lld) exceed cap %lld",
               (long long)offset, (long long)(offset + n_t), (long long)cap);
    const int64_t n_tok = n_b * n_h * n_t;
    if (n_tok == 0) return SS_OK;
    SS_REQUIRE(keys && values && centroids && idx_cache && values_il8, "null pointer argument");
    SS_UNSUPPORTED(n_tok * head_dim < (1LL << 31), "too many elements for one launch");
    // the index cache [n_b][n_h][cap][n_blocks], rows from `offset` on
    uint8_t *out = idx_cache + offset * n_blocks;
    const int64_t o_st = n_blocks, o_sh = cap * n_blocks, o_sb = n_h * o_sh;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (n_tok * n_blocks > 4096) {  // a prompt: the bulk encoders, then the values
        const int rc = encode_impl(keys, keys_dtype, n_b, n_h, n_t, k_sb, k_sh, k_st, head_dim, perm,
                                   centroids, n_blocks, n_centroids, block_dim, out, o_sb, o_sh, o_st,
                                   prepared, stream);
        if (rc != SS_OK) return rc;
        return ss_append_values_il8(values, v_dtype, n_b, n_h, n_t, v_sb, v_sh, v_st, head_dim,
                                    values_il8, cap, offset, stream);
    }
    EncodeArgs a{keys, keys_dtype, n_h,  n_t,        n_tok,     k_sb, k_sh, k_st,
                 perm, centroids,  n_blocks, n_centroids, out, o_sb, o_sh, o_st};
    const ValueAppend v{values, v_dtype, v_sb, v_sh, v_st, head_dim,
                        static_cast<__half *>(values_il8), cap, offset};
    const int per = kEncThreads / kWave;
    const int n_enc = (int)((n_tok * n_blocks + per - 1) / per);
    const int n_val = (int)((n_tok * head_dim + kEncThreads - 1) / kEncThreads);
    const dim3 grid((unsigned)(n_enc + n_val));
    if (block_dim == 8)
        hipLaunchKernelGGL(append_kv_small_kernel<8>, grid, dim3(kEncThreads), 0, st, a, v, n_enc);
    else if (block_dim == 4)
        hipLaunchKernelGGL(append_kv_small_kernel<4>, grid, dim3(kEncThreads), 0, st, a, v, n_enc);
    else
        hipLaunchKernelGGL(append_kv_small_kernel<16>, grid, dim3(kEncThreads), 0, st, a, v, n_enc);
    SS_LAUNCH_CHECK("append_kv_small_kernel launch");
    return SS_OK;
}

extern "C" int ss_hybrid_append_grouped_il(
    const void *keys, const void *values, int kv_dtype, int64_t n_b, int64_t n_h, int64_t n_new,
    int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st,
    void *buf_keys, void *buf_values, int buf_dtype, int64_t buf_cap, int64_t put_pos,
    int64_t flush_pos, int64_t n_flush, int head_dim, const int32_t *perm, const float *centroids,
    int n_blocks, int n_centroids, int block_dim, uint8_t *idx_cache, int bits, int group_size,
    uint32_t *codes_il, void *scales, void *zeros, int sz_dtype, int64_t cap, int64_t offset,
    void *stream) {
    SS_REQUIRE(valid_dtype(kv_dtype) && valid_dtype(buf_dtype), "bad key/value or buffer dtype");
    SS_REQUIRE(sz_dtype == SS_F32 || sz_dtype == SS_F16, "scale/zero dtype must be f32 or f16");
    SS_UNSUPPORTED(block_dim == 8 && n_blocks * 8 == head_dim, "block_dim 8 codecs only");
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256, "n_centroids %d unsupported (1..256)",
                   n_centroids);
    SS_UNSUPPORTED(bits == 2 || bits == 4, "interleaved codes are 2- or 4-bit");
    SS_UNSUPPORTED((head_dim == 64 || head_dim == 128) &&
                       (group_size == head_dim || 2 * group_size == head_dim),
                   "head_dim %d with group_size %d unsupported (64 or 128, group head_dim or "
                   "half of it)", head_dim, group_size);
    SS_REQUIRE(n_b >= 0 && n_h >= 0 && n_new >= 0 && n_flush >= 0, "negative sizes");
    SS_REQUIRE(put_pos >= 0 && put_pos + n_new <= buf_cap && flush_pos >= 0 &&
                   flush_pos + n_flush <= buf_cap,
               "buffer ranges exceed its capacity %lld", (long long)buf_cap);
    SS_REQUIRE(n_new == 0 || n_flush == 0 || put_pos >= flush_pos + n_flush ||
                   put_pos + n_new <= flush_pos,
               "the stored and flushed buffer ranges overlap");
    const int vpw = 32 / bits;
    SS_REQUIRE(cap % vpw == 0 && offset >= 0 && offset + n_flush <= cap,
               "compressed range [%lld, %lld) exceeds cap %lld", (long long)offset,
               (long long)(offset + n_flush), (long long)cap);
    const int64_t n_bh = n_b * n_h;
    if (n_bh == 0 || (n_new == 0 && n_flush == 0)) return SS_OK;
    SS_REQUIRE(buf_keys && buf_values && (n_new == 0 || (keys && values)), "null pointer argument");
    SS_REQUIRE(n_flush == 0 || (centroids && idx_cache && codes_il && scales && zeros),
               "null pointer argument");
    SS_UNSUPPORTED(n_flush * n_blocks <= 65536 && n_new * head_dim <= (1 << 20),
                   "step too large for one launch (take the separate appends)");
    // keys to encode: the flushed buffer rows; indices at compressed rows offset ..
    EncodeArgs a{reinterpret_cast<const char *>(buf_keys) +
                     flush_pos * head_dim * dtype_bytes(buf_dtype),
                 buf_dtype, n_h, n_flush, n_bh * n_flush, n_h * buf_cap * head_dim,
                 buf_cap * head_dim, head_dim, perm, centroids, n_blocks, n_centroids,
                 idx_cache + offset * n_blocks, n_h * cap * n_blocks, cap * n_blocks, n_blocks};
    HybridGroupedStep hs{keys, values, kv_dtype, k_sb, k_sh, k_st, v_sb, v_sh, v_st, n_new,
                         buf_keys, buf_values, buf_dtype, buf_cap, put_pos, flush_pos, n_flush,
                         offset, cap, head_dim, bits, group_size, codes_il, scales, zeros, sz_dtype,
                         offset / vpw, n_flush ? (offset + n_flush - 1) / vpw - offset / vpw + 1 : 0,
                         n_bh};
    const int n_put = (int)((2 * n_bh * n_new * head_dim + kEncThreads - 1) / kEncThreads);
    const int per = kEncThreads / kWave;
    const int n_enc = (int)((n_bh * n_flush * n_blocks + per - 1) / per);
    const int64_t n_val = (n_bh * hs.n_blk + per - 1) / per;  // a wave per (bh, word row)
    SS_UNSUPPORTED(n_put + n_enc + n_val < (1LL << 31), "step too large for one launch");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(hybrid_grouped_step_kernel<8>, dim3((unsigned)(n_put + n_enc + n_val)),
                       dim3(kEncThreads), 0, st, a, hs, n_put, n_enc);
    SS_LAUNCH_CHECK("hybrid_grouped_step_kernel launch");
    return SS_OK;
}
